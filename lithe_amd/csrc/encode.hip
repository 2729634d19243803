// Greedy residual encode of 64-value blocks against the twin codebook (closed-form search).
//
// Every codeword of a level has the same norm, so the nearest codeword to a block r has bit q of
// its index set exactly when <r, U[:, q]> > 0, with U[t, q] = (-1)^popcount(t & q) the first nine
// Sylvester-Hadamard columns (lithe/quant.py:46-50, lithe/codebook.py:45-49). Level l picks
// k_l from the residual, adds pool[l][k_l] to the reconstruction and subtracts it from the
// residual, in fp32 and in that order (lithe/quant.py:54-71).
//
// Layout: a block is handled by one quad. Lane c of the quad holds the sixteen values
// t = 16 i + 4 c + e (i, e < 4; four 16-byte loads at 64-byte steps), so it owns the residues
// t mod 16 = 4 c + e. Because q < 16, the projection on column q depends on t mod 16 only, and
// with q = 4 h + g, (-1)^popcount(t & q) = (-1)^popcount(c & h) (-1)^popcount(e & g):
//   fold      s[e] = sum_i r[16 i + 4 c + e]                       (in the lane)
//   Walsh     w_c[g] = sum_e (-1)^popcount(e & g) s[e]             (in the lane)
//   butterfly p[4 h + g] = sum_c (-1)^popcount(c & h) w_c[g]       (two DPP steps over the quad)
// after which lane h holds p[4 h .. 4 h + 3]; each lane sets the index bits of its own
// projections and two DPP ORs give every lane of the quad the whole index. The codeword of
// level l is periodic in t with period 16, so the residual stays folded: s[e] -= 4 c_l[4 c + e]
// (exact: the fold of a 16-periodic block is 4 times its period). The reconstruction is the
// level-order fp32 sum of the codewords, written as four copies of the lane's four values.
// The codeword value at position t is lut[l][popcount((k ^ m_t) & 511)], as in the bulk decode.
#include <stdint.h>

#include "lithe_common.h"

namespace lithe {
namespace {

constexpr int kThreads = 256;
constexpr int kBlocksPerWave = 16;             // 64 lanes / 4 lanes per block

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}
constexpr int kQuadSwapPairs = 0xB1;    // quad_perm [1, 0, 3, 2]: lane c <-> c ^ 1
constexpr int kQuadSwapHalves = 0x4E;   // quad_perm [2, 3, 0, 1]: lane c <-> c ^ 2

__device__ __forceinline__ float flip_sign(float v, uint32_t sign) {
    return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v) ^ sign);
}

template <typename IdxT>
__global__ void __launch_bounds__(kThreads) encode_kernel(const float *__restrict__ blocks, int64_t n,
                                                         const int8_t *__restrict__ sides, Luts luts, int32_t levels,
                                                         IdxT *__restrict__ idx, int64_t level_stride,
                                                         int64_t block_stride, float *__restrict__ recon) {
    __shared__ float lut[2 * kMaxLevels * 10];
    if (threadIdx.x < 2 * kMaxLevels * 10) lut[threadIdx.x] = (&luts.v[0][0][0])[threadIdx.x];
    __syncthreads();

    const int lane = threadIdx.x & 63, c = lane & 3;
    const int64_t blk = ((int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6)) * kBlocksPerWave + (lane >> 2);
    const bool valid = blk < n;
    const int64_t b = valid ? blk : n - 1;           // clamped: every lane of a quad loads and exchanges
    const float *src = blocks + b * kBlock + 4 * c;
    f32x4 r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = *reinterpret_cast<const f32x4 *>(src + 16 * i);
    float s[4], acc[4];
    uint32_t mt[4];                                  // codeword masks of this lane's residues
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        s[e] = (r[0][e] + r[1][e]) + (r[2][e] + r[3][e]);
        acc[e] = 0.0f;
        mt[e] = sign_mask((uint32_t)(4 * c + e)) & kIndexMask;
    }
    const uint32_t sign1 = (c & 1) ? 0x80000000u : 0u, sign2 = (c & 2) ? 0x80000000u : 0u;
    const float *tab = lut + (sides && sides[b] ? kMaxLevels * 10 : 0);
    uint32_t own = 0;                                // the index of level c, stored by lane c
    for (int l = 0; l < levels; ++l) {
        const float a0 = s[0] + s[1], a1 = s[0] - s[1], a2 = s[2] + s[3], a3 = s[2] - s[3];
        const float w[4] = {a0 + a2, a1 + a3, a0 - a2, a1 - a3};
        uint32_t bits = 0;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            float p = dpp<kQuadSwapPairs>(w[g]) + flip_sign(w[g], sign1);
            p = dpp<kQuadSwapHalves>(p) + flip_sign(p, sign2);
            bits |= (p > 0.0f ? 1u : 0u) << g;
        }
        uint32_t k = (bits << (4 * c)) & kIndexMask;
        k |= dpp<kQuadSwapPairs>(k);
        k |= dpp<kQuadSwapHalves>(k);
        own = c == l ? k : own;
        const float *tl = tab + l * 10;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float v = tl[__builtin_popcount(k ^ mt[e])];
            acc[e] += v;
            s[e] = fmaf(-4.0f, v, s[e]);
        }
    }
    if (valid && c < levels) idx[(int64_t)c * level_stride + blk * block_stride] = (IdxT)own;
    if (recon && valid) {
        float *dst = recon + blk * kBlock + 4 * c;
        const f32x4 v = {acc[0], acc[1], acc[2], acc[3]};
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<f32x4 *>(dst + 16 * i) = v;
    }
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
    if ((n + per_wg - 1) / per_wg > kMaxGridX) return LITHE_ERR_SHAPE;
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
