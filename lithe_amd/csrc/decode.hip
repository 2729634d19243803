// 9-bit pack / unpack and the bulk decode of packed (or unpacked) index streams.
//
// Bulk decode is write-bound: one adapter of the 342-linear FLUX layout reads 2.4 MB of
// packed words and writes 89.7 MB of bf16. Each thread owns one half of a 64-value
// block: it decodes the 8 distinct values of its half period (the codeword period is
// 16, see lithe_common.h) once and stores them to the 4 places they occur, so the
// per-element cost is a quarter of a direct decode.
#include <stdint.h>

#include <algorithm>

#include "lithe_common.h"

namespace lithe {
namespace {

constexpr int kThreads = 256;

__global__ void __launch_bounds__(kThreads) unpack9_kernel(const uint64_t *__restrict__ words, int64_t n,
                                                          void *__restrict__ out, int32_t out_dtype) {
    const int64_t w = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t n_words = (n + 6) / 7;
    if (w >= n_words) return;
    const uint64_t word = words[w];
#pragma unroll
    for (int j = 0; j < 7; ++j) {
        const int64_t p = w * 7 + j;
        if (p >= n) break;
        const uint32_t v = (uint32_t)(word >> (9 * j)) & kIndexMask;
        if (out_dtype == LITHE_DT_I64) static_cast<int64_t *>(out)[p] = v;
        else if (out_dtype == LITHE_DT_I32) static_cast<int32_t *>(out)[p] = (int32_t)v;
        else static_cast<int16_t *>(out)[p] = (int16_t)v;
    }
}

__global__ void __launch_bounds__(kThreads) pack9_kernel(const void *__restrict__ idx, int32_t idx_dtype,
                                                        int64_t n, uint64_t *__restrict__ words,
                                                        int32_t *__restrict__ err) {
    const int64_t w = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t n_words = (n + 6) / 7;
    if (w >= n_words) return;
    uint64_t word = 0;
    bool bad = false;
#pragma unroll
    for (int j = 0; j < 7; ++j) {
        const int64_t p = w * 7 + j;
        if (p >= n) break;
        int64_t v;
        if (idx_dtype == LITHE_DT_U16) v = static_cast<const uint16_t *>(idx)[p];
        else if (idx_dtype == LITHE_DT_I16) v = static_cast<const int16_t *>(idx)[p];
        else if (idx_dtype == LITHE_DT_I32) v = static_cast<const int32_t *>(idx)[p];
        else v = static_cast<const int64_t *>(idx)[p];
        if (v < 0 || v > (int64_t)kIndexMask) {
            bad = true;
            v = 0;
        }
        word |= (uint64_t)v << (9 * j);
    }
    words[w] = word;
    if (bad && err) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct DecodeArgs {
    IdxSrc src;
    Luts luts;
    const int32_t *slots;
    const int8_t *sides;
    void *out;
    int64_t n_blocks;
    int64_t out_sel_stride;
    int32_t *err;
    // stacked output (decoded-mode serving): factor segments of the layout, rows of three int64
    // (first block, block count, -); block blk of segment s and selection sel lands at block
    // n_sel * first_s + sel * count_s + (blk - first_s) of the output. NULL: slot-major output.
    const int64_t *seg;
    int32_t n_seg;
    int32_t n_sel;
};

// Output block of (selection sel, block blk) in the stacked layout; *s is the segment of a block
// at or before blk on entry (0 works) and blk's segment on return.
__device__ __forceinline__ int64_t stacked_block(const DecodeArgs &a, int32_t &s, int64_t blk, int sel) {
    while (s + 1 < a.n_seg && blk >= a.seg[3 * (int64_t)s] + a.seg[3 * (int64_t)s + 1]) ++s;
    const int64_t first = a.seg[3 * (int64_t)s], count = a.seg[3 * (int64_t)s + 1];
    return (int64_t)a.n_sel * first + (int64_t)sel * count + (blk - first);
}

// Segment holding block blk (binary search over the first blocks).
__device__ __forceinline__ int32_t find_seg(const DecodeArgs &a, int64_t blk) {
    int32_t lo = 0, hi = a.n_seg;
    while (hi - lo > 1) {
        const int32_t mid = (lo + hi) >> 1;
        if (a.seg[3 * (int64_t)mid] <= blk) lo = mid;
        else hi = mid;
    }
    return lo;
}

template <typename OutT>
__global__ void __launch_bounds__(kThreads) decode_kernel(DecodeArgs a) {
    __shared__ float lut[2 * kMaxLevels * 10];
    if (threadIdx.x < 2 * kMaxLevels * 10) lut[threadIdx.x] = (&a.luts.v[0][0][0])[threadIdx.x];
    __syncthreads();

    const int64_t half = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t block = half >> 1;
    if (block >= a.n_blocks) return;
    const int h = (int)(half & 1);
    const int sel = blockIdx.y;
    int64_t slot = a.slots ? a.slots[sel] : 0;
    int64_t ob = (int64_t)sel * (a.out_sel_stride / kBlock) + block;
    if (a.seg) {
        int32_t sg = find_seg(a, block);
        ob = stacked_block(a, sg, block, sel);
        if (ob < 0 || ob >= (int64_t)a.n_sel * a.n_blocks) {    // table inconsistent with n_blocks
            record_error(a.err, kErrTable);
            return;
        }
    }
    OutT *out = static_cast<OutT *>(a.out) + ob * kBlock + 8 * h;

    float v[8];
    if (slot < 0 || slot >= a.src.n_slots) {
        if (threadIdx.x == 0 && (block & 127) == 0) record_error(a.err, kErrSlot);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.0f;
    } else {
        uint32_t k[kMaxLevels];
        if (!fetch_indices(a.src, slot, block, k)) record_error(a.err, kErrIndex);
        const int side = a.sides ? (int)a.sides[block] : 0;
        const float *tab = lut + side * kMaxLevels * 10;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t m = h ? sign_mask(8 + e) : sign_mask(e);
            v[e] = decode_value(tab, a.src.levels, k, m);
        }
    }
    if constexpr (sizeof(OutT) == 2) {
        bf16x8 pk;
#pragma unroll
        for (int e = 0; e < 8; ++e) pk[e] = (__bf16)v[e];
#pragma unroll
        for (int j = 0; j < 4; ++j) *reinterpret_cast<bf16x8 *>(out + 16 * j) = pk;
    } else {
        f32x4 lo = {v[0], v[1], v[2], v[3]};
        f32x4 hi = {v[4], v[5], v[6], v[7]};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            *reinterpret_cast<f32x4 *>(out + 16 * j) = lo;
            *reinterpret_cast<f32x4 *>(out + 16 * j + 4) = hi;
        }
    }
}

// Packed 3-level fast path of the bulk decode (the resident bank of the twin codebook). Each
// thread owns kDecodeIter half-blocks of one selected slot, spaced kThreads apart, and issues
// the index loads of all of them before decoding the first, so a wave keeps kDecodeIter round
// trips in flight instead of one. Output order and values are those of decode_kernel.
// Side bytes: a workgroup (SPAN consecutive blocks from blockIdx.x * SPAN) reads its sides with
// coalesced 4-byte loads issued after the index loads and takes them from LDS; each thread owns
// 24 half-blocks (240 VGPRs, 2 waves per SIMD, no scratch). Measured against one byte load per
// half-block and 8 half-blocks per thread: rank 16 (0.7 MB of sides) 4.57 -> 4.70 TB/s with 16
// half-blocks, -> 4.81 with 24; rank 64 (2.8 MB) 3.95 -> 4.45 -> 4.66 TB/s; 32 half-blocks per
// thread drop to 3.6 TB/s. The staging alone at 8 half-blocks lost 3 % at rank 16. Every wave finishes its loads before its first
// store (stores that start while a workgroup's index loads are landing cost 6 % at rank 16). The
// last workgroup of a selection, or a side table not 4-byte aligned, reads the bytes one by one.
constexpr int kDecodeIter = 24;
template <typename OutT>
__global__ void __launch_bounds__(kThreads) decode_packed3_kernel(DecodeArgs a) {
    constexpr int SPAN = kThreads * kDecodeIter / 2;
    static_assert(SPAN % (4 * kThreads) == 0, "whole 4-byte side loads per thread");
    __shared__ float lut[2 * kMaxLevels * 10];
    __shared__ int8_t wg_side[SPAN];
    if (threadIdx.x < 2 * kMaxLevels * 10) lut[threadIdx.x] = (&a.luts.v[0][0][0])[threadIdx.x];
    const int64_t b0 = (int64_t)blockIdx.x * SPAN;
    const bool whole = a.sides && b0 + SPAN <= a.n_blocks &&
                       (reinterpret_cast<uintptr_t>(a.sides) & 3u) == 0;

    const int sel = blockIdx.y;
    const int64_t slot = a.slots ? a.slots[sel] : 0;
    const bool bad = slot < 0 || slot >= a.src.n_slots;
    const int64_t halves = a.n_blocks * 2;
    const int64_t h0 = (int64_t)blockIdx.x * (kThreads * kDecodeIter) + threadIdx.x;
    OutT *out = static_cast<OutT *>(a.out) + (a.seg ? 0 : (int64_t)sel * a.out_sel_stride);
    int32_t sg = a.seg ? find_seg(a, std::min(h0, halves - 1) >> 1) : 0;

    int64_t blk[kDecodeIter], sl[kDecodeIter];
    RawIdx raw[kDecodeIter];
    int8_t side[kDecodeIter];
#pragma unroll
    for (int i = 0; i < kDecodeIter; ++i) {
        const int64_t hf = std::min(h0 + (int64_t)i * kThreads, halves - 1);   // clamped: loads stay in range
        blk[i] = hf >> 1;
        sl[i] = bad ? 0 : slot;
    }
    load_raw<kDecodeIter, true, 3>(a.src, sl, blk, raw);
    if (whole) {
        uint32_t sw[SPAN / (4 * kThreads)];
#pragma unroll
        for (int q = 0; q < SPAN / (4 * kThreads); ++q)
            sw[q] = *reinterpret_cast<const uint32_t *>(a.sides + b0 + 4 * (int64_t)(threadIdx.x + q * kThreads));
#pragma unroll
        for (int q = 0; q < SPAN / (4 * kThreads); ++q)
            *reinterpret_cast<uint32_t *>(wg_side + 4 * (threadIdx.x + q * kThreads)) = sw[q];
    } else {
#pragma unroll
        for (int i = 0; i < kDecodeIter; ++i) side[i] = a.sides ? a.sides[blk[i]] : 0;
    }
    __syncthreads();    // value tables (and staged sides) visible
    if (bad && threadIdx.x == 0 && blockIdx.x == 0) record_error(a.err, kErrSlot);

#pragma unroll
    for (int i = 0; i < kDecodeIter; ++i) {
        const int64_t hf = h0 + (int64_t)i * kThreads;
        if (hf >= halves) break;
        const int h = (int)(hf & 1);
        uint32_t k[kMaxLevels];
        extract_indices<true, 3>(a.src, blk[i], raw[i], k);
        const int sd = whole ? wg_side[blk[i] - b0] : side[i];
        const float *tab = lut + sd * kMaxLevels * 10;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t m = h ? sign_mask(8 + e) : sign_mask(e);
            v[e] = bad ? 0.0f : decode_value<3>(tab, 3, k, m);
        }
        const int64_t ob = a.seg ? stacked_block(a, sg, blk[i], sel) : blk[i];
        if (a.seg && (ob < 0 || ob >= (int64_t)a.n_sel * a.n_blocks)) {    // table inconsistent with n_blocks
            record_error(a.err, kErrTable);
            continue;
        }
        OutT *o = out + ob * kBlock + 8 * h;
        if constexpr (sizeof(OutT) == 2) {
            bf16x8 pk;
#pragma unroll
            for (int e = 0; e < 8; ++e) pk[e] = (__bf16)v[e];
#pragma unroll
            for (int j = 0; j < 4; ++j) *reinterpret_cast<bf16x8 *>(o + 16 * j) = pk;
        } else {
            f32x4 lo = {v[0], v[1], v[2], v[3]};
            f32x4 hi = {v[4], v[5], v[6], v[7]};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                *reinterpret_cast<f32x4 *>(o + 16 * j) = lo;
                *reinterpret_cast<f32x4 *>(o + 16 * j + 4) = hi;
            }
        }
    }
}

// Packed 3-level bulk decode to bf16, software-pipelined, whole-line stores. Each thread runs
// kLineBatches batches of kLineBatch half-blocks (spaced kThreads apart, consecutive threads on
// consecutive half-blocks); the index loads of batch i + 1 are in flight while batch i is decoded
// and stored. Per half-block a lane decodes its 8 distinct values once; the wave's 64 halves
// (32 blocks) go through a 1 KB LDS exchange and every store instruction writes 8 whole 128-byte
// lines: lane L stores chunk L % 8 (half (L % 8) & 1 of the period) of block 8 s + L / 8.
// Measured on MI355X (FLUX 342-linear layout, 2,000-slot bank): 5.48 TB/s at rank 16 and 5.43 at
// rank 64, against 4.83 / 4.62 for decode_packed3_kernel (24 half-blocks per thread, all loads
// before the first store, each lane storing its 8 values 4 times at a 32-byte stride). The same
// pipeline with that store shape ran 3.99 / 3.94; non-temporal line stores 5.36 / 5.37; 4 or 16
// half-blocks per batch, 1, 4 or 8 batches per workgroup 5.05-5.40 (8 x 4 and wider spill or drop
// to 3 waves per SIMD). Stacked output (decoded-mode serving): a lane finds the output block of
// the block it stores, walking the segment table forward.
constexpr int kLineBatch = 8;
constexpr int kLineBatches = 2;
__global__ void __launch_bounds__(kThreads) decode_packed3_lines_kernel(DecodeArgs a) {
    constexpr int B = kLineBatch;
    constexpr int PER_WG = kThreads * B * kLineBatches;    // half-blocks per workgroup
    constexpr int SPAN = PER_WG / 2;                       // blocks per workgroup
    static_assert(SPAN % (4 * kThreads) == 0, "whole 4-byte side loads per thread");
    __shared__ float lut[2 * kMaxLevels * 10];
    __shared__ int8_t wg_side[SPAN];
    __shared__ bf16x8 xch[kThreads];                       // 1 KB per wave
    if (threadIdx.x < 2 * kMaxLevels * 10) lut[threadIdx.x] = (&a.luts.v[0][0][0])[threadIdx.x];
    const int64_t b0 = (int64_t)blockIdx.x * SPAN;
    const bool whole = a.sides && b0 + SPAN <= a.n_blocks && (reinterpret_cast<uintptr_t>(a.sides) & 3u) == 0;
    const int sel = blockIdx.y;
    const int64_t slot = a.slots ? a.slots[sel] : 0;
    const bool bad = slot < 0 || slot >= a.src.n_slots;
    const int64_t halves = a.n_blocks * 2;
    const int lane = threadIdx.x & 63;
    const int64_t h0 = (int64_t)blockIdx.x * PER_WG + threadIdx.x;
    __bf16 *out = static_cast<__bf16 *>(a.out) + (a.seg ? 0 : (int64_t)sel * a.out_sel_stride);
    int32_t sg = a.seg ? find_seg(a, std::min(b0, a.n_blocks - 1)) : 0;

    RawIdx raw[2][B];
    auto loads = [&](int i, RawIdx *r) __attribute__((always_inline)) {
        int64_t sl[B], blk[B];
#pragma unroll
        for (int q = 0; q < B; ++q) {
            blk[q] = std::min(h0 + (int64_t)(i * B + q) * kThreads, halves - 1) >> 1;   // clamped: in range
            sl[q] = bad ? 0 : slot;
        }
        load_raw<B, true, 3>(a.src, sl, blk, r);
    };
    loads(0, raw[0]);
    if (whole) {
        uint32_t sw[SPAN / (4 * kThreads)];
#pragma unroll
        for (int q = 0; q < SPAN / (4 * kThreads); ++q)
            sw[q] = *reinterpret_cast<const uint32_t *>(a.sides + b0 + 4 * (int64_t)(threadIdx.x + q * kThreads));
#pragma unroll
        for (int q = 0; q < SPAN / (4 * kThreads); ++q)
            *reinterpret_cast<uint32_t *>(wg_side + 4 * (threadIdx.x + q * kThreads)) = sw[q];
    }
    __syncthreads();    // value tables (and staged sides) visible
    if (bad && threadIdx.x == 0 && blockIdx.x == 0) record_error(a.err, kErrSlot);

    bf16x8 *wx = xch + (threadIdx.x & ~63);
#pragma unroll
    for (int i = 0; i < kLineBatches; ++i) {
        if (i + 1 < kLineBatches) loads(i + 1, raw[(i + 1) & 1]);
#pragma unroll
        for (int q = 0; q < B; ++q) {
            const int64_t hf = h0 + (int64_t)(i * B + q) * kThreads;
            const int64_t blk = std::min(hf, halves - 1) >> 1;
            const int h = (int)(hf & 1);
            uint32_t k[kMaxLevels];
            extract_indices<true, 3>(a.src, blk, raw[i & 1][q], k);
            const int sd = whole ? wg_side[blk - b0] : (a.sides ? a.sides[blk] : 0);
            const float *tab = lut + sd * kMaxLevels * 10;
            bf16x8 pk;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t m = h ? sign_mask(8 + e) : sign_mask(e);
                pk[e] = (__bf16)(bad ? 0.0f : decode_value<3>(tab, 3, k, m));
            }
            // the wave's lanes hold halves hw .. hw + 63 (hw even) = blocks hw / 2 .. hw / 2 + 31
            wave_lds_sync();     // the other lanes have read the previous halves
            xch[threadIdx.x] = pk;
            wave_lds_sync();     // every lane's half is in the exchange
            const int64_t bw = (hf - lane) >> 1;
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const int mb = 8 * st + (lane >> 3), c = lane & 7;
                const bf16x8 v = wx[2 * mb + (c & 1)];
                const int64_t b = bw + mb;
                if (b >= a.n_blocks) continue;
                const int64_t ob = a.seg ? stacked_block(a, sg, b, sel) : b;
                if (a.seg && (ob < 0 || ob >= (int64_t)a.n_sel * a.n_blocks)) {    // table inconsistent with n_blocks
                    record_error(a.err, kErrTable);
                    continue;
                }
                *reinterpret_cast<bf16x8 *>(out + ob * kBlock + 8 * c) = v;
            }
        }
    }
}

}  // namespace

// True when blocks [block_off, block_off + n_blocks) of every slot lie inside the slot's
// extent as described by the strides (guards the kernels against out-of-bounds reads).
bool src_covers(const lithe_index_src &s, int64_t n_blocks) {
    const int64_t end = s.block_off + n_blocks;
    switch (s.kind) {
        case LITHE_IDX_PACKED9: return end * s.num_levels <= s.slot_stride * 7;
        case LITHE_IDX_LEVEL_I32:
        case LITHE_IDX_LEVEL_I16:
            return end <= s.level_stride && (int64_t)s.num_levels * s.level_stride <= s.slot_stride;
        case LITHE_IDX_BLOCK_I16: return end * s.num_levels <= s.slot_stride;
        default: return false;
    }
}

namespace {

int32_t check_src(const lithe_index_src *s) {
    if (!s || !s->base) return LITHE_ERR_NULL;
    if (s->num_levels < 1 || s->num_levels > kMaxLevels) return LITHE_ERR_LEVELS;
    if (s->kind < LITHE_IDX_PACKED9 || s->kind > LITHE_IDX_BLOCK_I16) return LITHE_ERR_DTYPE;
    if (s->slot_stride < 0 || s->level_stride < 0 || s->block_off < 0 || s->n_slots < 1)
        return LITHE_ERR_SHAPE;
    // packed positions inside one slot are 32-bit in the kernels
    if (s->kind == LITHE_IDX_PACKED9 && s->slot_stride >= ((int64_t)1 << 32) / 7) return LITHE_ERR_SHAPE;
    return LITHE_OK;
}

}  // namespace

IdxSrc make_src(const lithe_index_src &s) {
    IdxSrc r;
    r.base = s.base;
    r.slot_stride = s.slot_stride;
    r.level_stride = s.level_stride;
    r.block_off = s.block_off;
    r.n_slots = s.n_slots;
    r.kind = s.kind;
    r.levels = s.num_levels;
    return r;
}

int32_t validate_src(const lithe_index_src *s) { return check_src(s); }

}  // namespace lithe

using namespace lithe;

extern "C" int32_t lithe_unpack9(const uint64_t *words, int64_t n, void *out, int32_t out_dtype, void *stream) {
    if (n < 0) return LITHE_ERR_SHAPE;
    if (out_dtype != LITHE_DT_I16 && out_dtype != LITHE_DT_I32 && out_dtype != LITHE_DT_I64)
        return LITHE_ERR_DTYPE;
    if (n == 0) return LITHE_OK;
    if (!words || !out) return LITHE_ERR_NULL;
    const int64_t n_words = (n + 6) / 7;
    const int64_t grid = (n_words + kThreads - 1) / kThreads;
    if (grid > kMaxGridX) return LITHE_ERR_SHAPE;
    hipLaunchKernelGGL(unpack9_kernel, dim3((unsigned)grid), dim3(kThreads), 0, (hipStream_t)stream, words, n,
                       out, out_dtype);
    return hipGetLastError() == hipSuccess ? LITHE_OK : LITHE_ERR_HIP;
}

extern "C" int32_t lithe_pack9(const void *idx, int32_t idx_dtype, int64_t n, uint64_t *words, int32_t *err_flag,
                               void *stream) {
    if (n < 0) return LITHE_ERR_SHAPE;
    if (idx_dtype != LITHE_DT_U16 && idx_dtype != LITHE_DT_I16 && idx_dtype != LITHE_DT_I32 &&
        idx_dtype != LITHE_DT_I64)
        return LITHE_ERR_DTYPE;
    if (n == 0) return LITHE_OK;
    if (!idx || !words) return LITHE_ERR_NULL;
    const int64_t n_words = (n + 6) / 7;
    const int64_t grid = (n_words + kThreads - 1) / kThreads;
    if (grid > kMaxGridX) return LITHE_ERR_SHAPE;
    hipLaunchKernelGGL(pack9_kernel, dim3((unsigned)grid), dim3(kThreads), 0, (hipStream_t)stream, idx, idx_dtype,
                       n, words, err_flag);
    return hipGetLastError() == hipSuccess ? LITHE_OK : LITHE_ERR_HIP;
}

static int32_t decode_impl(const lithe_index_src *src, const int32_t *slots, int32_t n_sel, int64_t n_blocks,
                           const int8_t *sides, const lithe_lut *lut_a, const lithe_lut *lut_b, void *out,
                           int32_t out_dtype, int64_t out_sel_stride, int32_t *err_flag, const int64_t *seg,
                           int32_t n_seg, void *stream) {
    int32_t rc = check_src(src);
    if (rc) return rc;
    if (!src_covers(*src, n_blocks)) return LITHE_ERR_SHAPE;
    if (!lut_a || !out) return LITHE_ERR_NULL;
    if (sides && !lut_b) return LITHE_ERR_NULL;
    if (n_sel < 1 || n_blocks < 0 || n_sel > 65535) return LITHE_ERR_SHAPE;
    if (!slots && n_sel != 1) return LITHE_ERR_NULL;
    if (lut_a->num_levels != src->num_levels || (lut_b && lut_b->num_levels != src->num_levels))
        return LITHE_ERR_LEVELS;
    if (out_dtype != LITHE_DT_BF16 && out_dtype != LITHE_DT_F32) return LITHE_ERR_DTYPE;
    if (n_sel > 1 && out_sel_stride < n_blocks * kBlock) return LITHE_ERR_SHAPE;
    const int esz = out_dtype == LITHE_DT_BF16 ? 2 : 4;
    if (((uintptr_t)out & 15u) || ((out_sel_stride * esz) & 15)) return LITHE_ERR_ALIGN;
    if (n_blocks == 0) return LITHE_OK;

    DecodeArgs a;
    a.src = make_src(*src);
    for (int s = 0; s < 2; ++s) {
        const lithe_lut *t = (s == 0 || !lut_b) ? lut_a : lut_b;
        for (int l = 0; l < kMaxLevels; ++l)
            for (int p = 0; p < 10; ++p) a.luts.v[s][l][p] = t->value[l][p];
    }
    a.slots = slots;
    a.sides = sides;
    a.out = out;
    a.n_blocks = n_blocks;
    a.out_sel_stride = out_sel_stride;
    a.err = err_flag;
    a.seg = seg;
    a.n_seg = n_seg;
    a.n_sel = n_sel;
    const int64_t halves = n_blocks * 2;
    // the widest grid is the one-half-block-per-thread kernel's
    if ((halves + kThreads - 1) / kThreads > kMaxGridX || n_sel > kMaxGridY) return LITHE_ERR_SHAPE;
    if (src->kind == LITHE_IDX_PACKED9 && src->num_levels == 3 && out_dtype == LITHE_DT_BF16) {
        constexpr int64_t per_wg = (int64_t)kThreads * kLineBatch * kLineBatches;
        dim3 grid((unsigned)((halves + per_wg - 1) / per_wg), (unsigned)n_sel);
        hipLaunchKernelGGL(decode_packed3_lines_kernel, grid, dim3(kThreads), 0, (hipStream_t)stream, a);
        return hipGetLastError() == hipSuccess ? LITHE_OK : LITHE_ERR_HIP;
    }
    if (src->kind == LITHE_IDX_PACKED9 && src->num_levels == 3) {
        const int64_t per_wg = (int64_t)kThreads * kDecodeIter;
        dim3 grid((unsigned)((halves + per_wg - 1) / per_wg), (unsigned)n_sel);
        if (out_dtype == LITHE_DT_BF16)
            hipLaunchKernelGGL(decode_packed3_kernel<__bf16>, grid, dim3(kThreads), 0, (hipStream_t)stream, a);
        else
            hipLaunchKernelGGL(decode_packed3_kernel<float>, grid, dim3(kThreads), 0, (hipStream_t)stream, a);
        return hipGetLastError() == hipSuccess ? LITHE_OK : LITHE_ERR_HIP;
    }
    dim3 grid((unsigned)((halves + kThreads - 1) / kThreads), (unsigned)n_sel);
    if (out_dtype == LITHE_DT_BF16)
        hipLaunchKernelGGL(decode_kernel<__bf16>, grid, dim3(kThreads), 0, (hipStream_t)stream, a);
    else
        hipLaunchKernelGGL(decode_kernel<float>, grid, dim3(kThreads), 0, (hipStream_t)stream, a);
    return hipGetLastError() == hipSuccess ? LITHE_OK : LITHE_ERR_HIP;
}

extern "C" int32_t lithe_decode(const lithe_index_src *src, const int32_t *slots, int32_t n_sel, int64_t n_blocks,
                                const int8_t *sides, const lithe_lut *lut_a, const lithe_lut *lut_b, void *out,
                                int32_t out_dtype, int64_t out_sel_stride, int32_t *err_flag, void *stream) {
    return decode_impl(src, slots, n_sel, n_blocks, sides, lut_a, lut_b, out, out_dtype, out_sel_stride, err_flag,
                       nullptr, 0, stream);
}

extern "C" int32_t lithe_decode_stacked(const lithe_index_src *src, const int32_t *slots, int32_t n_sel,
                                        int64_t n_blocks, int32_t n_segments, const int64_t *table,
                                        const int8_t *sides, const lithe_lut *lut_a, const lithe_lut *lut_b,
                                        void *out, int32_t out_dtype, int32_t *err_flag, void *stream) {
    if (!table) return LITHE_ERR_NULL;
    if (n_segments < 1) return LITHE_ERR_SHAPE;
    return decode_impl(src, slots, n_sel, n_blocks, sides, lut_a, lut_b, out, out_dtype, n_blocks * kBlock,
                       err_flag, table, n_segments, stream);
}
