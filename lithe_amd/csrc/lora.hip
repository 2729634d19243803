// Per-sample LoRA delta with the factors decoded on the fly (or read dense):
//
//   shrink:  mid[row, g*16 + r] = round_x( sum_k x[row, k] * A_g[r, k] * mid_scale[b] )
//   expand:  y[row, o]          = round_y( y + round_y( round_y( sum_{g,r} mid * B_g[o, r] ) * s_b ) )
//
// g runs over "rank groups": route entry j of a sample contributes ceil(rank/16) groups of
// 16 ranks each (rank-stacked mixtures, lithe/serve.py:89-96). Both kernels use gfx950
// MFMA tiles with 16 tokens per wave:
//
// shrink  v_mfma_f32_16x16x32_bf16 (fp32: 16x16x4 f32). A-operand = decoded factor rows
//         (lane%16 = rank), B-operand = x^T (lane%16 = token); lane group q = lane/16 owns
//         k = 8q..8q+7 of each 32-wide step, so a row of x is read 64 contiguous bytes per
//         instruction. The decoded A chunk lives in LDS as one 16-value period per
//         (rank, block): the period-16 structure of the codebook makes it 4x smaller than
//         the dense chunk. Long reductions split over K; the last workgroup of a token tile
//         to finish (atomic ticket) sums the fp32 partials in chunk order, so the result
//         does not depend on scheduling.
// expand  v_mfma_f32_16x16x16_bf16 (fp32: 16x16x4 f32) with the decoded B tile as the
//         A-operand (lane%16 = output row) and mid^T as the B-operand (lane%16 = token).
//         Output rows are assigned so that each lane ends with 8 consecutive outputs of its
//         token: y is read-modified-written 16 bytes per lane, 64 contiguous bytes per row
//         per instruction, with the reference's rounding chain applied in registers.
#include <stdint.h>
#include <stdlib.h>

#include <algorithm>
#include <type_traits>

#include "lithe_common.h"

namespace lithe {

bool src_covers(const lithe_index_src &s, int64_t n_blocks);
int32_t validate_src(const lithe_index_src *s);
IdxSrc make_src(const lithe_index_src &s);

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kMaxGroups = 8;
constexpr int kLdsBudget = 60 * 1024;

enum { SRC_INDEXED = 1, SRC_DENSE = 2 };

struct LoraArgs {
    const void *x;
    void *y;
    void *mid;
    float *part;
    uint32_t *counters;
    int32_t *err;
    int64_t n_batch, seq, d_in, d_out, rows;
    int32_t rank, G, n_rg, n_route, MR;
    int32_t tiles_s, subs_s, S, Kc, pat_rs;
    int32_t tiles_e, subs_e, BO, brs, vec_y;
    int32_t accumulate;
    float out_scale;
    const int32_t *r_slot;
    const float *r_w;
    const float *s_scale;
    const float *mid_scale;
    const float *out_scale_vec;
    IdxSrc a_src, b_src;
    Luts luts;
    const void *dense_a, *dense_b;
    int64_t n_slots;
};

template <typename T> struct Vec8;
template <> struct Vec8<__bf16> { typedef bf16x8 type; };

// Route of sample b: slot and sqrt-weight of every rank group, staged in LDS by the
// first G threads. Returns (uniformly) whether any group is active.
__device__ __forceinline__ bool load_route(const LoraArgs &a, int64_t b, int64_t *s_slot, float *s_w,
                                           int *s_any) {
    const int tid = threadIdx.x;
    if (tid == 0) *s_any = 0;
    __syncthreads();
    if (tid < a.G) {
        const int j = tid / a.n_rg;
        const int32_t s = a.r_slot[b * a.n_route + j];
        int64_t slot = -1;
        if (s >= 0 && (int64_t)s < a.n_slots) slot = s;
        else if (s != -1) record_error(a.err, kErrSlot);
        s_slot[tid] = slot;
        s_w[tid] = a.r_w ? a.r_w[b * a.n_route + j] : 1.0f;
        if (slot >= 0) atomicOr(s_any, 1);
    }
    __syncthreads();
    return *s_any != 0;
}

// ============================================================================ shrink
template <typename XT, int SRC, int GM>
__global__ void __launch_bounds__(kThreads) shrink_kernel(LoraArgs a) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    __shared__ float lut[kMaxLevels * 10];
    __shared__ int64_t s_slot[kMaxGroups];
    __shared__ float s_w[kMaxGroups];
    __shared__ int s_any, s_last;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, r16 = lane & 15, gq = lane >> 4;
    const int tile = blockIdx.x;
    const int64_t b = tile / a.tiles_s;
    const int mt = tile % a.tiles_s;
    const int kc = blockIdx.y;
    const int64_t k0 = (int64_t)kc * a.Kc;
    const int kn = (int)std::min<int64_t>(a.Kc, a.d_in - k0);
    const int nbk = kn / kBlock;

    if (!load_route(a, b, s_slot, s_w, &s_any)) return;

    XT *pat = reinterpret_cast<XT *>(smem);
    if constexpr (SRC == SRC_INDEXED) {
        if (tid < kMaxLevels * 10) lut[tid] = (&a.luts.v[0][0][0])[tid];
        __syncthreads();
        const int L = a.a_src.levels;
        const int64_t row_blocks = a.d_in / kBlock;
        const int items = a.G * 16 * nbk;
        for (int it = tid; it < items; it += kThreads) {
            const int cb = it % nbk;
            const int gr = it / nbk;
            const int g = gr >> 4, r = gr & 15;
            const int rr = (g % a.n_rg) * 16 + r;
            float v[16];
            const int64_t slot = s_slot[g];
            if (slot < 0 || rr >= a.rank) {
#pragma unroll
                for (int t = 0; t < 16; ++t) v[t] = 0.0f;
            } else {
                uint32_t k[kMaxLevels];
                const int64_t blk = rr * row_blocks + k0 / kBlock + cb;
                if (!fetch_indices(a.a_src, slot, blk, k)) record_error(a.err, kErrIndex);
                const float w = s_w[g];
#pragma unroll
                for (int t = 0; t < 16; ++t) v[t] = decode_value(lut, L, k, sign_mask(t)) * w;
            }
            XT *dst = pat + gr * a.pat_rs + cb * 16;
            if constexpr (sizeof(XT) == 2) {
                bf16x8 p0, p1;
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    p0[t] = (__bf16)v[t];
                    p1[t] = (__bf16)v[8 + t];
                }
                reinterpret_cast<bf16x8 *>(dst)[0] = p0;
                reinterpret_cast<bf16x8 *>(dst)[1] = p1;
            } else {
#pragma unroll
                for (int t = 0; t < 16; t += 4) *reinterpret_cast<f32x4 *>(dst + t) = {v[t], v[t + 1], v[t + 2], v[t + 3]};
            }
        }
        __syncthreads();
    }

    const float ms_b = a.mid_scale ? a.mid_scale[b] : 1.0f;
    for (int sub = 0; sub < a.subs_s; ++sub) {
        const int64_t m = ((int64_t)mt * a.subs_s + sub) * (kWaves * 16) + wave * 16 + r16;
        const bool valid = m < a.seq;
        const int64_t row = b * a.seq + (valid ? m : 0);
        const XT *xr = static_cast<const XT *>(a.x) + row * a.d_in + k0;
        f32x4 acc[GM];
#pragma unroll
        for (int g = 0; g < GM; ++g) acc[g] = {0.0f, 0.0f, 0.0f, 0.0f};

        if constexpr (sizeof(XT) == 2) {
            constexpr int U = 8;
            const int steps = kn / 32;
            const XT *xl = xr + 8 * gq;
            for (int s0 = 0; s0 < steps; s0 += U) {
                bf16x8 xv[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    if (s0 + u < steps && valid) xv[u] = *reinterpret_cast<const bf16x8 *>(xl + 32 * (s0 + u));
                    else xv[u] = bf16x8{};
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int s = s0 + u;
                    if (s >= steps) break;
#pragma unroll
                    for (int g = 0; g < GM; ++g) {
                        if (g >= a.G) break;
                        bf16x8 av;
                        if constexpr (SRC == SRC_INDEXED) {
                            av = *reinterpret_cast<const bf16x8 *>(pat + (g * 16 + r16) * a.pat_rs + (s >> 1) * 16 +
                                                                   8 * (gq & 1));
                        } else {
                            const int rr = (g % a.n_rg) * 16 + r16;
                            const int64_t slot = s_slot[g];
                            if (slot >= 0 && rr < a.rank)
                                av = *reinterpret_cast<const bf16x8 *>(static_cast<const XT *>(a.dense_a) +
                                                                       (slot * a.rank + rr) * a.d_in + k0 + 32 * s +
                                                                       8 * gq);
                            else
                                av = bf16x8{};
                        }
                        acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, xv[u], acc[g], 0, 0, 0);
                    }
                }
            }
        } else {
            constexpr int U = 8;
            const int steps = kn / 16;
            const XT *xl = xr + 4 * gq;
            for (int s0 = 0; s0 < steps; s0 += U) {
                f32x4 xv[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    if (s0 + u < steps && valid) xv[u] = *reinterpret_cast<const f32x4 *>(xl + 16 * (s0 + u));
                    else xv[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int s = s0 + u;
                    if (s >= steps) break;
#pragma unroll
                    for (int g = 0; g < GM; ++g) {
                        if (g >= a.G) break;
                        f32x4 av;
                        if constexpr (SRC == SRC_INDEXED) {
                            av = *reinterpret_cast<const f32x4 *>(pat + (g * 16 + r16) * a.pat_rs + (s >> 2) * 16 +
                                                                  4 * gq);
                        } else {
                            const int rr = (g % a.n_rg) * 16 + r16;
                            const int64_t slot = s_slot[g];
                            if (slot >= 0 && rr < a.rank)
                                av = *reinterpret_cast<const f32x4 *>(static_cast<const XT *>(a.dense_a) +
                                                                      (slot * a.rank + rr) * a.d_in + k0 + 16 * s +
                                                                      4 * gq);
                            else
                                av = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                        }
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            acc[g] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[e], xv[u][e], acc[g], 0, 0, 0);
                    }
                }
            }
        }

        // acc[g][e] = sum over this chunk for token r16, rank 4*gq + e of group g.
        if (!valid) continue;
        if (a.S == 1) {
#pragma unroll
            for (int g = 0; g < GM; ++g) {
                if (g >= a.G) break;
                if (s_slot[g] < 0) continue;
                XT *dst = static_cast<XT *>(a.mid) + row * a.MR + g * 16 + 4 * gq;
#pragma unroll
                for (int e = 0; e < 4; ++e) dst[e] = DT<XT>::from_f32(acc[g][e] * ms_b);
            }
        } else {
#pragma unroll
            for (int g = 0; g < GM; ++g) {
                if (g >= a.G) break;
                *reinterpret_cast<f32x4 *>(a.part + ((int64_t)kc * a.rows + row) * a.MR + g * 16 + 4 * gq) = acc[g];
            }
        }
    }
    if (a.S == 1) return;

    // Split-K: the last of the S workgroups of this token tile reduces the partials.
    __syncthreads();
    if (tid == 0) {
        __threadfence();
        const uint32_t old =
            __hip_atomic_fetch_add(&a.counters[tile], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (old == (uint32_t)(a.S - 1));
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (int sub = 0; sub < a.subs_s; ++sub) {
        const int64_t m = ((int64_t)mt * a.subs_s + sub) * (kWaves * 16) + wave * 16 + r16;
        if (m >= a.seq) continue;
        const int64_t row = b * a.seq + m;
#pragma unroll
        for (int g = 0; g < GM; ++g) {
            if (g >= a.G) break;
            if (s_slot[g] < 0) continue;
            const float *src = a.part + row * a.MR + g * 16 + 4 * gq;
            f32x4 sum = *reinterpret_cast<const f32x4 *>(src);
            for (int c = 1; c < a.S; ++c) sum += *reinterpret_cast<const f32x4 *>(src + (int64_t)c * a.rows * a.MR);
            XT *dst = static_cast<XT *>(a.mid) + row * a.MR + g * 16 + 4 * gq;
#pragma unroll
            for (int e = 0; e < 4; ++e) dst[e] = DT<XT>::from_f32(sum[e] * ms_b);
        }
    }
    if (tid == 0) __hip_atomic_store(&a.counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ============================================================================ expand
template <typename YT>
__device__ __forceinline__ float finish(float acc, float s, float yold, int accumulate) {
    const float d = DT<YT>::round(DT<YT>::round(acc) * s);
    return accumulate ? DT<YT>::round(yold + d) : d;
}

template <typename XT, typename YT, int SRC, int GM, int BOM>
__global__ void __launch_bounds__(kThreads) expand_kernel(LoraArgs a) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    __shared__ float lut[kMaxLevels * 10];
    __shared__ int64_t s_slot[kMaxGroups];
    __shared__ float s_w[kMaxGroups];
    __shared__ int s_any;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63, r16 = lane & 15, gq = lane >> 4;
    const int o_tiles = (int)((a.d_out + a.BO - 1) / a.BO);
    const int64_t obase = (int64_t)(blockIdx.x % o_tiles) * a.BO;
    const int tile = blockIdx.x / o_tiles;
    const int64_t b = tile / a.tiles_e;
    const int mt = tile % a.tiles_e;
    const float s_b = a.out_scale_vec ? a.out_scale_vec[b] : a.out_scale;

    const bool any = load_route(a, b, s_slot, s_w, &s_any);
    if (!any) {
        if (a.accumulate) return;
        // Empty route in write mode: the delta is zero.
        for (int sub = 0; sub < a.subs_e; ++sub) {
            const int64_t m = ((int64_t)mt * a.subs_e + sub) * (kWaves * 16) + wave * 16 + r16;
            if (m >= a.seq) continue;
            YT *yr = static_cast<YT *>(a.y) + (b * a.seq + m) * a.d_out;
            for (int o = gq; o < a.BO; o += 4)
                if (obase + o < a.d_out) yr[obase + o] = DT<YT>::from_f32(0.0f);
        }
        return;
    }

    // ---- B tile (BO outputs x 16 ranks per group) into LDS, in the activation dtype.
    XT *bt = reinterpret_cast<XT *>(smem);
    if constexpr (SRC == SRC_INDEXED) {
        if (tid < kMaxLevels * 10) lut[tid] = (&a.luts.v[1][0][0])[tid];
        __syncthreads();
    }
    {
        const int L = a.b_src.levels;
        const int items = a.G * a.BO;
        for (int it = tid; it < items; it += kThreads) {
            const int g = it / a.BO, ol = it % a.BO;
            const int64_t o = obase + ol;
            const int rr0 = (g % a.n_rg) * 16;
            const int64_t slot = s_slot[g];
            float v[16];
            if (slot < 0 || o >= a.d_out) {
#pragma unroll
                for (int t = 0; t < 16; ++t) v[t] = 0.0f;
            } else if constexpr (SRC == SRC_INDEXED) {
                const float sc = a.s_scale ? a.s_scale[slot] : 1.0f;
                const float w = s_w[g];
                int64_t cached = -1;
                uint32_t k[kMaxLevels] = {0, 0, 0, 0};
#pragma unroll
                for (int t = 0; t < 16; ++t) {
                    v[t] = 0.0f;
                    if (rr0 + t < a.rank) {
                        const int64_t f = o * a.rank + rr0 + t;
                        const int64_t blk = f >> 6;
                        if (blk != cached) {
                            if (!fetch_indices(a.b_src, slot, blk, k)) record_error(a.err, kErrIndex);
                            cached = blk;
                        }
                        v[t] = (decode_value(lut, L, k, sign_mask((uint32_t)(f & 15))) * sc) * w;
                    }
                }
            } else {
                const XT *src = static_cast<const XT *>(a.dense_b) + (slot * a.d_out + o) * a.rank;
#pragma unroll
                for (int t = 0; t < 16; ++t) v[t] = (rr0 + t < a.rank) ? DT<XT>::to_f32(src[rr0 + t]) : 0.0f;
            }
            XT *dst = bt + (g * a.BO + ol) * a.brs;
#pragma unroll
            for (int t = 0; t < 16; ++t) dst[t] = DT<XT>::from_f32(v[t]);
        }
    }
    __syncthreads();

    // ---- B fragments into registers. MFMA (p, h) row i <-> output 32p + 8(i/4) + 4h + (i%4).
    constexpr int NP = BOM / 32;
    const int np = a.BO / 32;
    typedef typename std::conditional<sizeof(XT) == 2, i16x4, f32x4>::type Frag;
    Frag bfr[NP][2][GM];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int ol = 32 * p + 8 * (r16 >> 2) + 4 * h + (r16 & 3);
#pragma unroll
            for (int g = 0; g < GM; ++g) {
                if (p < np && g < a.G) {
                    const XT *src = bt + (g * a.BO + ol) * a.brs + 4 * gq;
                    if constexpr (sizeof(XT) == 2) bfr[p][h][g] = *reinterpret_cast<const i16x4 *>(src);
                    else bfr[p][h][g] = *reinterpret_cast<const f32x4 *>(src);
                } else {
                    bfr[p][h][g] = Frag{};
                }
            }
        }
    }

    for (int sub = 0; sub < a.subs_e; ++sub) {
        const int64_t m = ((int64_t)mt * a.subs_e + sub) * (kWaves * 16) + wave * 16 + r16;
        const bool valid = m < a.seq;
        const int64_t row = b * a.seq + (valid ? m : 0);
        Frag mf[GM];
#pragma unroll
        for (int g = 0; g < GM; ++g) {
            if (g < a.G && valid && s_slot[g] >= 0) {
                const XT *src = static_cast<const XT *>(a.mid) + row * a.MR + g * 16 + 4 * gq;
                if constexpr (sizeof(XT) == 2) mf[g] = *reinterpret_cast<const i16x4 *>(src);
                else mf[g] = *reinterpret_cast<const f32x4 *>(src);
            } else {
                mf[g] = Frag{};
            }
        }
        YT *yr = static_cast<YT *>(a.y) + row * a.d_out;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            if (p >= np) break;
            f32x4 acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int g = 0; g < GM; ++g) {
                    if (g >= a.G) break;
                    if constexpr (sizeof(XT) == 2) {
                        acc[h] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bfr[p][h][g], mf[g], acc[h], 0, 0, 0);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            acc[h] = __builtin_amdgcn_mfma_f32_16x16x4f32(bfr[p][h][g][e], mf[g][e], acc[h], 0, 0, 0);
                    }
                }
            }
            if (!valid) continue;
            const int64_t o8 = obase + 32 * p + 8 * gq;
            if (o8 >= a.d_out) continue;
            float vals[8] = {acc[0][0], acc[0][1], acc[0][2], acc[0][3], acc[1][0], acc[1][1], acc[1][2], acc[1][3]};
            YT *yp = yr + o8;
            if (a.vec_y && o8 + 8 <= a.d_out) {
                if constexpr (sizeof(YT) == 2) {
                    bf16x8 yo = a.accumulate ? *reinterpret_cast<const bf16x8 *>(yp) : bf16x8{};
                    bf16x8 yn;
#pragma unroll
                    for (int e = 0; e < 8; ++e) yn[e] = (__bf16)finish<YT>(vals[e], s_b, (float)yo[e], a.accumulate);
                    *reinterpret_cast<bf16x8 *>(yp) = yn;
                } else {
                    f32x4 y0 = {0.0f, 0.0f, 0.0f, 0.0f}, y1 = {0.0f, 0.0f, 0.0f, 0.0f};
                    if (a.accumulate) {
                        y0 = *reinterpret_cast<const f32x4 *>(yp);
                        y1 = *reinterpret_cast<const f32x4 *>(yp + 4);
                    }
                    f32x4 n0, n1;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        n0[e] = finish<YT>(vals[e], s_b, y0[e], a.accumulate);
                        n1[e] = finish<YT>(vals[4 + e], s_b, y1[e], a.accumulate);
                    }
                    *reinterpret_cast<f32x4 *>(yp) = n0;
                    *reinterpret_cast<f32x4 *>(yp + 4) = n1;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    if (o8 + e >= a.d_out) break;
                    const float yo = a.accumulate ? DT<YT>::to_f32(yp[e]) : 0.0f;
                    yp[e] = DT<YT>::from_f32(finish<YT>(vals[e], s_b, yo, a.accumulate));
                }
            }
        }
    }
}

// ============================================================================ host plan
int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    if (!v || !*v) return dflt;
    const int x = atoi(v);
    return x > 0 ? x : dflt;
}

struct Plan {
    int G, n_rg, GM, MR;
    int tiles_s, subs_s, S, Kc, pat_rs;
    size_t lds_s;
    int tiles_e, subs_e, BO, BOM, brs;
    size_t lds_e;
    int64_t off_counters, off_mid, off_part, total;
};

int64_t align256(int64_t v) { return (v + 255) & ~int64_t(255); }

Plan make_plan(int64_t n_batch, int64_t seq, int64_t d_in, int64_t d_out, int rank, int n_route, int xbytes,
               bool dense) {
    Plan p{};
    p.n_rg = (rank + 15) / 16;
    p.G = p.n_rg * n_route;
    p.GM = p.G <= 1 ? 1 : p.G <= 2 ? 2 : p.G <= 4 ? 4 : 8;
    p.MR = p.G * 16;
    const int64_t rows = n_batch * seq;
    const int target = env_int("LITHE_TARGET_WGS", 1536);

    // shrink: 64 tokens per workgroup sub-tile, K split for LDS capacity and parallelism.
    p.subs_s = env_int("LITHE_SHRINK_SUBS", 1);
    const int64_t tm_s = 64 * (int64_t)p.subs_s;
    p.tiles_s = (int)std::max<int64_t>(1, (seq + tm_s - 1) / tm_s);
    const int64_t items = n_batch * p.tiles_s;
    const int nb_total = (int)(d_in / kBlock);
    const int pad = 16 / xbytes;
    int s_lds = 1;
    if (!dense) {
        const int nb_max = (int)((kLdsBudget / (p.G * 16 * xbytes) - pad) / 16);
        s_lds = (nb_total + nb_max - 1) / std::max(1, nb_max);
    }
    const int s_par = (int)std::min<int64_t>((target + items - 1) / items, std::max(1, nb_total / 4));
    int S = std::max(s_lds, std::max(1, s_par));
    S = std::min(S, std::max(1, nb_total));
    if (getenv("LITHE_SHRINK_SPLIT")) S = std::min(nb_total, std::max(s_lds, env_int("LITHE_SHRINK_SPLIT", S)));
    const int nb = (nb_total + S - 1) / S;
    p.S = (nb_total + nb - 1) / nb;
    p.Kc = nb * kBlock;
    p.pat_rs = nb * 16 + pad;
    p.lds_s = dense ? 0 : (size_t)p.G * 16 * p.pat_rs * xbytes;

    // expand: BO outputs x 64*subs tokens per workgroup.
    int bo_max = xbytes == 2 ? std::min(256, 512 / p.GM) : std::min(128, 256 / p.GM);
    bo_max = std::max(32, bo_max);
    p.BOM = bo_max;
    p.BO = (int)std::min<int64_t>(bo_max, ((d_out + 31) / 32) * 32);
    p.brs = 16 + (xbytes == 2 ? 4 : 4);
    p.lds_e = (size_t)p.G * p.BO * p.brs * xbytes;
    const int64_t o_tiles = (d_out + p.BO - 1) / p.BO;
    const int64_t base_items = n_batch * ((seq + 63) / 64) * o_tiles;
    int subs = (int)std::max<int64_t>(1, std::min<int64_t>(4, base_items / target));
    if (getenv("LITHE_EXPAND_SUBS")) subs = env_int("LITHE_EXPAND_SUBS", subs);
    p.subs_e = subs;
    p.tiles_e = (int)std::max<int64_t>(1, (seq + 64 * (int64_t)subs - 1) / (64 * (int64_t)subs));

    // workspace
    p.off_counters = 256;
    p.off_mid = align256(p.off_counters + 4 * n_batch * p.tiles_s);
    p.off_part = align256(p.off_mid + rows * p.MR * xbytes);
    p.total = align256(p.off_part + (p.S > 1 ? (int64_t)p.S * rows * p.MR * 4 : 0));
    return p;
}

template <typename XT, typename YT, int SRC, int GM, int BOM>
void launch(const Plan &p, LoraArgs &a, hipStream_t st) {
    dim3 gs((unsigned)(a.n_batch * p.tiles_s), (unsigned)p.S);
    hipLaunchKernelGGL((shrink_kernel<XT, SRC, GM>), gs, dim3(kThreads), p.lds_s, st, a);
    dim3 ge((unsigned)(((a.d_out + p.BO - 1) / p.BO) * a.n_batch * p.tiles_e));
    hipLaunchKernelGGL((expand_kernel<XT, YT, SRC, GM, BOM>), ge, dim3(kThreads), p.lds_e, st, a);
}

template <typename XT, typename YT, int SRC>
int32_t dispatch_gm(const Plan &p, LoraArgs &a, hipStream_t st) {
    constexpr bool bf = sizeof(XT) == 2;
    switch (p.GM) {
        case 1: launch<XT, YT, SRC, 1, bf ? 256 : 128>(p, a, st); break;
        case 2: launch<XT, YT, SRC, 2, bf ? 256 : 128>(p, a, st); break;
        case 4: launch<XT, YT, SRC, 4, bf ? 128 : 64>(p, a, st); break;
        default: launch<XT, YT, SRC, 8, bf ? 64 : 32>(p, a, st); break;
    }
    return hipGetLastError() == hipSuccess ? LITHE_OK : LITHE_ERR_HIP;
}

template <typename XT, typename YT>
int32_t dispatch_src(const Plan &p, LoraArgs &a, int kind, hipStream_t st) {
    return kind == LITHE_FACTOR_DENSE ? dispatch_gm<XT, YT, SRC_DENSE>(p, a, st)
                                      : dispatch_gm<XT, YT, SRC_INDEXED>(p, a, st);
}

}  // namespace
}  // namespace lithe

using namespace lithe;

extern "C" int64_t lithe_lora_workspace_bytes(int64_t n_batch, int64_t seq, int64_t d_in, int64_t d_out,
                                              int32_t rank, int32_t n_route, int32_t x_dtype) {
    if (n_batch < 0 || seq < 0 || d_in < kBlock || d_out < 1 || rank < 1 || n_route < 1) return LITHE_ERR_SHAPE;
    if (x_dtype != LITHE_DT_BF16 && x_dtype != LITHE_DT_F32) return LITHE_ERR_DTYPE;
    const int n_rg = (rank + 15) / 16;
    if (n_rg * n_route > kMaxGroups) return LITHE_ERR_SHAPE;
    // The plan depends on the factor kind only through the LDS capacity; size for the larger.
    const Plan a = make_plan(n_batch, seq, d_in, d_out, rank, n_route, x_dtype == LITHE_DT_BF16 ? 2 : 4, false);
    const Plan b = make_plan(n_batch, seq, d_in, d_out, rank, n_route, x_dtype == LITHE_DT_BF16 ? 2 : 4, true);
    return std::max(a.total, b.total);
}

extern "C" int32_t lithe_lora_delta(const void *x, int32_t x_dtype, int64_t n_batch, int64_t seq, int64_t d_in,
                                    void *y, int32_t y_dtype, int64_t d_out, int32_t accumulate, int32_t rank,
                                    const lithe_factors *f, const lithe_routes *routes, const float *mid_scale,
                                    float out_scale, const float *out_scale_vec, void *workspace,
                                    int64_t workspace_bytes, void *stream) {
    if (!f || !routes) return LITHE_ERR_NULL;
    if (x_dtype != LITHE_DT_BF16 && x_dtype != LITHE_DT_F32) return LITHE_ERR_DTYPE;
    if (y_dtype != LITHE_DT_BF16 && y_dtype != LITHE_DT_F32) return LITHE_ERR_DTYPE;
    if (n_batch < 0 || seq < 0 || d_in < 1 || d_out < 1 || rank < 1 || routes->n_route < 1) return LITHE_ERR_SHAPE;
    if (n_batch > 65535 || seq > (int64_t)1 << 30) return LITHE_ERR_SHAPE;
    if (d_in % kBlock || (d_out * rank) % kBlock) return LITHE_ERR_ALIGN;
    const int n_rg = (rank + 15) / 16;
    if (n_rg * routes->n_route > kMaxGroups) return LITHE_ERR_SHAPE;
    if (n_batch == 0 || seq == 0) return LITHE_OK;
    if (!x || !y || !routes->slot || !workspace) return workspace ? LITHE_ERR_NULL : LITHE_ERR_WORKSPACE;
    const int xbytes = x_dtype == LITHE_DT_BF16 ? 2 : 4;
    const int ybytes = y_dtype == LITHE_DT_BF16 ? 2 : 4;
    if (((uintptr_t)x & 15u) || ((uintptr_t)workspace & 255u)) return LITHE_ERR_ALIGN;
    if ((uintptr_t)y & (uintptr_t)(ybytes - 1)) return LITHE_ERR_ALIGN;

    LoraArgs a{};
    if (f->kind == LITHE_FACTOR_INDEXED) {
        int32_t rc = validate_src(&f->a_idx);
        if (rc) return rc;
        rc = validate_src(&f->b_idx);
        if (rc) return rc;
        if (f->a_idx.num_levels != f->b_idx.num_levels || f->lut_a.num_levels != f->a_idx.num_levels ||
            f->lut_b.num_levels != f->a_idx.num_levels)
            return LITHE_ERR_LEVELS;
        if (!src_covers(f->a_idx, rank * d_in / kBlock) || !src_covers(f->b_idx, d_out * rank / kBlock))
            return LITHE_ERR_SHAPE;
        a.a_src = make_src(f->a_idx);
        a.b_src = make_src(f->b_idx);
        a.n_slots = std::min(f->a_idx.n_slots, f->b_idx.n_slots);
        for (int l = 0; l < kMaxLevels; ++l)
            for (int q = 0; q < 10; ++q) {
                a.luts.v[0][l][q] = f->lut_a.value[l][q];
                a.luts.v[1][l][q] = f->lut_b.value[l][q];
            }
    } else if (f->kind == LITHE_FACTOR_DENSE) {
        if (!f->dense_a || !f->dense_b) return LITHE_ERR_NULL;
        if (f->dense_dtype != x_dtype) return LITHE_ERR_DTYPE;
        if (f->n_dense < 1) return LITHE_ERR_SHAPE;
        if ((uintptr_t)f->dense_a & 15u) return LITHE_ERR_ALIGN;
        a.dense_a = f->dense_a;
        a.dense_b = f->dense_b;
        a.n_slots = f->n_dense;
    } else {
        return LITHE_ERR_DTYPE;
    }

    const Plan p = make_plan(n_batch, seq, d_in, d_out, rank, routes->n_route, xbytes, f->kind == LITHE_FACTOR_DENSE);
    if (workspace_bytes < p.total) return LITHE_ERR_WORKSPACE;

    char *ws = static_cast<char *>(workspace);
    a.x = x;
    a.y = y;
    a.err = reinterpret_cast<int32_t *>(ws);
    a.counters = reinterpret_cast<uint32_t *>(ws + p.off_counters);
    a.mid = ws + p.off_mid;
    a.part = reinterpret_cast<float *>(ws + p.off_part);
    a.n_batch = n_batch;
    a.seq = seq;
    a.d_in = d_in;
    a.d_out = d_out;
    a.rows = n_batch * seq;
    a.rank = rank;
    a.G = p.G;
    a.n_rg = p.n_rg;
    a.n_route = routes->n_route;
    a.MR = p.MR;
    a.tiles_s = p.tiles_s;
    a.subs_s = p.subs_s;
    a.S = p.S;
    a.Kc = p.Kc;
    a.pat_rs = p.pat_rs;
    a.tiles_e = p.tiles_e;
    a.subs_e = p.subs_e;
    a.BO = p.BO;
    a.brs = p.brs;
    a.vec_y = (d_out % 8 == 0) && (((uintptr_t)y & 15u) == 0);
    a.accumulate = accumulate ? 1 : 0;
    a.out_scale = out_scale;
    a.r_slot = routes->slot;
    a.r_w = routes->weight_sqrt;
    a.s_scale = routes->slot_scale;
    a.mid_scale = mid_scale;
    a.out_scale_vec = out_scale_vec;

    hipStream_t st = (hipStream_t)stream;
    if (x_dtype == LITHE_DT_BF16) {
        return y_dtype == LITHE_DT_BF16 ? dispatch_src<__bf16, __bf16>(p, a, f->kind, st)
                                        : dispatch_src<__bf16, float>(p, a, f->kind, st);
    }
    return y_dtype == LITHE_DT_BF16 ? dispatch_src<float, __bf16>(p, a, f->kind, st)
                                    : dispatch_src<float, float>(p, a, f->kind, st);
}

extern "C" int32_t lithe_workspace_errors(const void *workspace, int32_t *flags, int32_t clear, void *stream) {
    if (!workspace || !flags) return LITHE_ERR_NULL;
    hipStream_t st = (hipStream_t)stream;
    if (hipMemcpyAsync(flags, workspace, sizeof(int32_t), hipMemcpyDeviceToHost, st) != hipSuccess) return LITHE_ERR_HIP;
    if (hipStreamSynchronize(st) != hipSuccess) return LITHE_ERR_HIP;
    if (clear && *flags) {
        if (hipMemsetAsync(const_cast<void *>(workspace), 0, sizeof(int32_t), st) != hipSuccess) return LITHE_ERR_HIP;
        if (hipStreamSynchronize(st) != hipSuccess) return LITHE_ERR_HIP;
    }
    return LITHE_OK;
}
