// Greedy residual encode of 64-value blocks against the twin codebook (closed-form search).
//
// Every codeword of a level has the same norm, so the nearest codeword to a block r has bit q of
// its index set exactly when <r, U[:, q]> > 0, with U[t, q] = (-1)^popcount(t & q) the first nine
// Sylvester-Hadamard columns (lithe/quant.py:46-50, lithe/codebook.py:45-49). Level l picks
// k_l from the residual, adds pool[l][k_l] to the reconstruction and subtracts it from the
// residual, in fp32 and in that order (lithe/quant.py:54-71).
//
// Layout: a block is handled by one 16-lane DPP row. Lane (quad c, position i) holds the four values
// t = 16 i + 4 c + e, e < 4 (one 16-byte load; a wave's load instruction covers four whole blocks),
// so quad c owns the residues t mod 16 = 4 c + e. Since q < 16, (-1)^popcount(t & q) factorises as
// (-1)^popcount(e & (q & 3)) (-1)^popcount(c & (q >> 2)), and the nine projections are
//   p_q = sum_c (-1)^popcount(c & (q >> 2)) H_c[q & 3],  H_c[g] = sum over the quad of W[g],
// with W the 4-point Walsh transform of a lane's four values. Per level: W in the lane, H by two
// DPP steps inside the quad (swap pairs, swap halves), then each p_q by two DPP steps across the
// quads (half-row mirror, row mirror). Both partners of every step add the same two values, so all
// sixteen lanes end with bit-identical projections and the same index. The codeword value at
// position t is the value-table lookup lut[l][popcount((k ^ m_t) & 511)] of the bulk decode.
#include <stdint.h>

#include "lithe_common.h"

namespace lithe {
namespace {

constexpr int kThreads = 256;
constexpr int kBlocksPerWave = 4;              // 64 lanes / 16 lanes per block

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int kQuadSwapPairs = 0xB1;    // quad_perm [1, 0, 3, 2]
constexpr int kQuadSwapHalves = 0x4E;   // quad_perm [2, 3, 0, 1]
constexpr int kRowHalfMirror = 0x141;   // lane i <-> 7 - i within each half row
constexpr int kRowMirror = 0x140;       // lane i <-> 15 - i

template <typename IdxT>
__global__ void __launch_bounds__(kThreads) encode_kernel(const float *__restrict__ blocks, int64_t n,
                                                         const int8_t *__restrict__ sides, Luts luts, int32_t levels,
                                                         IdxT *__restrict__ idx, int64_t level_stride,
                                                         int64_t block_stride, float *__restrict__ recon) {
    __shared__ float lut[2 * kMaxLevels * 10];
    if (threadIdx.x < 2 * kMaxLevels * 10) lut[threadIdx.x] = (&luts.v[0][0][0])[threadIdx.x];
    __syncthreads();

    const int lane = threadIdx.x & 63, j = lane & 15, c = j >> 2, i = j & 3;
    const int64_t blk = ((int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6)) * kBlocksPerWave + (lane >> 4);
    const bool valid = blk < n;
    const int64_t b = valid ? blk : n - 1;           // clamped: every lane of a row loads and reduces
    const int t0 = 16 * i + 4 * c;
    f32x4 r = *reinterpret_cast<const f32x4 *>(blocks + b * kBlock + t0);
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};

    uint32_t mt[4];                                  // codeword masks of this lane's positions
#pragma unroll
    for (int e = 0; e < 4; ++e) mt[e] = sign_mask((uint32_t)(4 * c + e));
    const bool neg1 = c & 1, neg2 = c & 2;           // quad signs of q >> 2 = 1 and 2
    for (int l = 0; l < levels; ++l) {
        // 4-point Walsh transform of the lane's values, then the sum over the quad
        const float a0 = r[0] + r[1], a1 = r[0] - r[1], a2 = r[2] + r[3], a3 = r[2] - r[3];
        float h[4] = {a0 + a2, a1 + a3, a0 - a2, a1 - a3};
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            h[g] += dpp<kQuadSwapPairs>(h[g]);
            h[g] += dpp<kQuadSwapHalves>(h[g]);
        }
        uint32_t k = 0;
#pragma unroll
        for (int q = 0; q < 9; ++q) {
            const float hv = h[q & 3];
            float p = (q >> 2) == 0 ? hv : (q >> 2) == 1 ? (neg1 ? -hv : hv) : (neg2 ? -hv : hv);
            p += dpp<kRowHalfMirror>(p);
            p += dpp<kRowMirror>(p);
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
    if (recon && valid) *reinterpret_cast<f32x4 *>(recon + blk * kBlock + t0) = acc;
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
