// Greedy residual encode of 64-value blocks against the twin codebook (closed-form search).
//
// Every codeword of a level has the same norm, so the nearest codeword to a block r has bit q of
// its index set exactly when <r, U[:, q]> > 0, with U[t, q] = (-1)^popcount(t & q) the first nine
// Sylvester-Hadamard columns (lithe/quant.py:46-50, lithe/codebook.py:45-49). Level l picks
// k_l from the residual, adds pool[l][k_l] to the reconstruction and subtracts it from the
// residual, in fp32 and in that order (lithe/quant.py:54-71).
//
// Layout: a block is handled by one 16-lane DPP row; lane j holds values 4j .. 4j + 3 (one 16-byte
// load, so a wave's load instruction covers four whole blocks = 1 KB of whole lines). Per level each
// lane forms the nine signed partial sums of its four values, and four DPP steps (swap within
// pairs, swap pairs of a quad, half-row mirror, row mirror) reduce them over the row: every lane
// ends with the same nine sums (fp32 addition is commutative, so both partners of a step compute
// the same value). The codeword value at position t is the value-table lookup
// lut[l][popcount((k ^ m_t) & 511)] of the bulk decode.
#include <stdint.h>

#include "lithe_common.h"

namespace lithe {
namespace {

constexpr int kThreads = 256;
constexpr int kBlocksPerWave = 4;              // 64 lanes / 16 lanes per block

__device__ __forceinline__ float dpp_sum16(float v) {
    // quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
    return v;
}

template <typename IdxT>
__global__ void __launch_bounds__(kThreads) encode_kernel(const float *__restrict__ blocks, int64_t n,
                                                         const int8_t *__restrict__ sides, Luts luts, int32_t levels,
                                                         IdxT *__restrict__ idx, int64_t level_stride,
                                                         int64_t block_stride, float *__restrict__ recon) {
    __shared__ float lut[2 * kMaxLevels * 10];
    if (threadIdx.x < 2 * kMaxLevels * 10) lut[threadIdx.x] = (&luts.v[0][0][0])[threadIdx.x];
    __syncthreads();

    const int lane = threadIdx.x & 63, j = lane & 15;
    const int64_t blk = ((int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6)) * kBlocksPerWave + (lane >> 4);
    const bool valid = blk < n;
    const int64_t b = valid ? blk : n - 1;           // clamped: every lane of a row loads and reduces
    f32x4 r = *reinterpret_cast<const f32x4 *>(blocks + b * kBlock + 4 * j);
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};

    // sign bits of this lane's four positions for the nine hyperplanes; codeword masks m_t
    uint32_t neg[4], mt[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t t = (uint32_t)(4 * j + e);
        uint32_t s = 0;
#pragma unroll
        for (int q = 0; q < 9; ++q) s |= (uint32_t)(__builtin_popcount(t & (uint32_t)q) & 1) << q;
        neg[e] = s;
        mt[e] = sign_mask(t & 15u);
    }
    for (int l = 0; l < levels; ++l) {
        uint32_t k = 0;
#pragma unroll
        for (int q = 0; q < 9; ++q) {
            float p = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) p += ((neg[e] >> q) & 1u) ? -r[e] : r[e];
            p = dpp_sum16(p);
            k |= (p > 0.0f ? 1u : 0u) << q;
        }
        const float *tab = lut + (sides && sides[b] ? kMaxLevels * 10 : 0) + l * 10;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float c = tab[__builtin_popcount((k ^ mt[e]) & kIndexMask)];
            acc[e] += c;
            r[e] -= c;
        }
        if (valid && j == 0) idx[(int64_t)l * level_stride + blk * block_stride] = (IdxT)k;
    }
    if (recon && valid) *reinterpret_cast<f32x4 *>(recon + blk * kBlock + 4 * j) = acc;
}

}  // namespace
}  // namespace lithe

using namespace lithe;

extern "C" int32_t lithe_encode(const float *blocks, int64_t n, const int8_t *sides, const lithe_lut *lut_a,
                                const lithe_lut *lut_b, void *idx, int32_t idx_dtype, int64_t idx_level_stride,
                                int64_t idx_block_stride, float *recon, void *stream) {
    if (n < 0) return LITHE_ERR_SHAPE;
    if (!lut_a || (sides && !lut_b)) return LITHE_ERR_NULL;
    const int L = lut_a->num_levels;
    if (L < 1 || L > kMaxLevels || (sides && lut_b->num_levels != L)) return LITHE_ERR_LEVELS;
    if (idx_dtype != LITHE_DT_I16 && idx_dtype != LITHE_DT_I32 && idx_dtype != LITHE_DT_I64) return LITHE_ERR_DTYPE;
    if (n == 0) return LITHE_OK;
    if (!blocks || !idx) return LITHE_ERR_NULL;
    // the L x n index positions must be distinct: (L, n) level-major or (n, L) block-major
    const bool level_major = idx_block_stride == 1 && idx_level_stride >= n;
    const bool block_major = idx_level_stride == 1 && idx_block_stride >= L;
    if (!level_major && !block_major) return LITHE_ERR_SHAPE;
    if (((uintptr_t)blocks & 15u) || ((uintptr_t)recon & 15u)) return LITHE_ERR_ALIGN;
    Luts luts{};
    for (int s = 0; s < 2; ++s) {
        const lithe_lut *t = (s == 0 || !lut_b) ? lut_a : lut_b;
        for (int l = 0; l < kMaxLevels; ++l)
            for (int p = 0; p < 10; ++p) luts.v[s][l][p] = t->value[l][p];
    }
    const int64_t per_wg = (kThreads / 64) * kBlocksPerWave;
    const dim3 grid((unsigned)((n + per_wg - 1) / per_wg));
    hipStream_t st = (hipStream_t)stream;
    if (idx_dtype == LITHE_DT_I16)
        hipLaunchKernelGGL(encode_kernel<int16_t>, grid, dim3(kThreads), 0, st, blocks, n, sides, luts, L,
                           static_cast<int16_t *>(idx), idx_level_stride, idx_block_stride, recon);
    else if (idx_dtype == LITHE_DT_I32)
        hipLaunchKernelGGL(encode_kernel<int32_t>, grid, dim3(kThreads), 0, st, blocks, n, sides, luts, L,
                           static_cast<int32_t *>(idx), idx_level_stride, idx_block_stride, recon);
    else
        hipLaunchKernelGGL(encode_kernel<int64_t>, grid, dim3(kThreads), 0, st, blocks, n, sides, luts, L,
                           static_cast<int64_t *>(idx), idx_level_stride, idx_block_stride, recon);
    return hipGetLastError() == hipSuccess ? LITHE_OK : LITHE_ERR_HIP;
}
