// Device ingest: a .lithe index stream (uploaded as uint16) reordered into the residency order and
// packed 7 x 9 bits per word straight into a bank slot, one thread per word.
//
// Residency position p = block * L + level (blocks of module m: A then B, modules in order); stream
// position of (segment s, block j of the segment, level l) = table[3s + 2] + l * table[3s + 1] + j.
// Neighbouring threads read neighbouring blocks of one level row, so each level's reads coalesce;
// the 16 KB segment table of a 342-module layout stays in the caches.
#include <stdint.h>

#include "lithe_common.h"

namespace lithe {
namespace {

constexpr int kThreads = 256;

__global__ void __launch_bounds__(kThreads) ingest_kernel(const uint16_t *__restrict__ stream, int64_t n_stream,
                                                         int32_t L, int32_t n_seg, const int64_t *__restrict__ table,
                                                         uint64_t *__restrict__ words, int64_t n_words,
                                                         int32_t *__restrict__ err) {
    const int64_t w = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (w >= n_words) return;
    const int64_t p0 = w * 7;
    uint64_t v = 0;
    int32_t bits = 0;
    if (p0 < n_stream) {
        // last segment whose first block is <= the block of p0
        const int64_t blk0 = p0 / L;
        int32_t lo = 0, hi = n_seg;
        while (hi - lo > 1) {
            const int32_t mid = (lo + hi) >> 1;
            if (table[3 * (int64_t)mid] <= blk0) lo = mid;
            else hi = mid;
        }
        int32_t seg = lo;
#pragma unroll
        for (int k = 0; k < 7; ++k) {
            const int64_t p = p0 + k;
            if (p >= n_stream) break;
            const int64_t blk = p / L, lvl = p - blk * L;
            while (seg + 1 < n_seg && blk >= table[3 * (int64_t)seg] + table[3 * (int64_t)seg + 1]) ++seg;
            const int64_t *r = table + 3 * (int64_t)seg;
            int64_t q = r[2] + lvl * r[1] + (blk - r[0]);
            if (q < 0 || q >= n_stream) {    // a table that does not describe this stream: never read past it
                bits |= 2;
                q = 0;
            }
            uint32_t x = stream[q];
            if (x > kIndexMask) {
                bits |= 1;
                x = 0;
            }
            v |= (uint64_t)x << (9 * k);
        }
    }
    words[w] = v;
    if (bits && err) __hip_atomic_fetch_or(err, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace
}  // namespace lithe

using namespace lithe;

extern "C" int32_t lithe_ingest(const uint16_t *stream, int64_t n_stream, int32_t num_levels, int32_t n_segments,
                                const int64_t *table, uint64_t *words, int64_t n_words, int32_t *err_flag,
                                void *hip_stream) {
    if (n_stream < 0 || n_segments < 1 || n_words < 0) return LITHE_ERR_SHAPE;
    if (num_levels < 1 || num_levels > kMaxLevels) return LITHE_ERR_LEVELS;
    if (n_words < (n_stream + 6) / 7) return LITHE_ERR_SHAPE;
    if (n_words == 0) return LITHE_OK;
    if (!stream || !table || !words) return LITHE_ERR_NULL;
    const int64_t grid = (n_words + kThreads - 1) / kThreads;
    if (grid > kMaxGridX) return LITHE_ERR_SHAPE;
    hipLaunchKernelGGL(ingest_kernel, dim3((unsigned)grid), dim3(kThreads), 0, (hipStream_t)hip_stream, stream,
                       n_stream, num_levels, n_segments, table, words, n_words, err_flag);
    return hipGetLastError() == hipSuccess ? LITHE_OK : LITHE_ERR_HIP;
}
