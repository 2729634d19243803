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

enum { SRC_INDEXED = 1, SRC_DENSE = 2 };

struct LoraArgs {
    const void *x;
    void *y;
    void *mid;
    int32_t *err;
    int64_t n_batch, seq, d_in, d_out, rows;
    int32_t rank, G, n_rg, n_route, MR;
    int32_t tiles_s, tg, Kc, arow, red_off;
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

// Route of sample b: slot and sqrt-weight of every rank group, staged in LDS by the
// first G threads. Returns (uniformly) whether any group is active.
__device__ __forceinline__ bool load_route(const LoraArgs &a, int64_t b, int64_t *s_slot, float *s_w,
                                           int *s_any) {
    const int tid = threadIdx.x;
    if (tid == 0) *s_any = 0;
    if (tid >= a.G && tid < kMaxGroups) {
        s_slot[tid] = -1;
        s_w[tid] = 0.0f;
    }
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
// Workgroup = 4 waves over a tile of 16*TG tokens; the KS = 4/TG waves that share a
// 16-token group split the K range and reduce their fp32 partials through LDS in a
// fixed order (deterministic, no global synchronisation). The decoded A factor is
// staged through LDS in chunks of Kc; each chunk holds one 16-value period per
// (rank, block) for decoded factors, or the dense rows for dense factors.
template <typename XT, int SRC, int GM>
__global__ void __launch_bounds__(kThreads) shrink_kernel(LoraArgs a) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    __shared__ float lut[kMaxLevels * 10];
    __shared__ int64_t s_slot[kMaxGroups];
    __shared__ float s_w[kMaxGroups];
    __shared__ int s_any;

    constexpr bool kBf16 = sizeof(XT) == 2;
    constexpr int KSTEP = kBf16 ? 32 : 16;        // k covered by one lane-group load of 16 bytes x 4 groups
    const int tid = threadIdx.x;
    // wave index as a scalar: loop bounds derived from it stay uniform (SGPR) branches
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, r16 = lane & 15, gq = lane >> 4;
    const int TG = a.tg, KS = kWaves / a.tg;
    const int tgi = wave % TG, ksi = wave / TG;
    const int tile = blockIdx.x;
    const int64_t b = tile / a.tiles_s;
    const int mt = tile % a.tiles_s;
    const int64_t m = (int64_t)mt * 16 * TG + tgi * 16 + r16;
    const bool valid = m < a.seq;
    const int64_t row = b * a.seq + (valid ? m : a.seq - 1);

    if (!load_route(a, b, s_slot, s_w, &s_any)) return;
    if constexpr (SRC == SRC_INDEXED) {
        if (tid < kMaxLevels * 10) lut[tid] = (&a.luts.v[0][0][0])[tid];
    }

    XT *chunk = reinterpret_cast<XT *>(smem);
    f32x4 acc[GM];
#pragma unroll
    for (int g = 0; g < GM; ++g) acc[g] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int64_t row_blocks = a.d_in / kBlock;
    const XT *xrow = static_cast<const XT *>(a.x) + row * a.d_in;
    for (int64_t k0 = 0; k0 < a.d_in; k0 += a.Kc) {
        const int kn = (int)std::min<int64_t>(a.Kc, a.d_in - k0);
        __syncthreads();   // LDS free (previous chunk consumed; lut visible)
        if constexpr (SRC == SRC_INDEXED) {
            const int L = a.a_src.levels;
            const int nbk = kn / kBlock;
            const int items = GM * 16 * nbk;
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
                XT *dst = chunk + gr * a.arow + cb * 16;
                if constexpr (kBf16) {
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
                    for (int t = 0; t < 16; t += 4)
                        *reinterpret_cast<f32x4 *>(dst + t) = f32x4{v[t], v[t + 1], v[t + 2], v[t + 3]};
                }
            }
        } else {
            constexpr int EV = 16 / sizeof(XT);     // elements per 16-byte vector
            const int per_row = kn / EV;
            const int items = GM * 16 * per_row;
            for (int it = tid; it < items; it += kThreads) {
                const int c = it % per_row;
                const int gr = it / per_row;
                const int g = gr >> 4, r = gr & 15;
                const int rr = (g % a.n_rg) * 16 + r;
                const int64_t slot = s_slot[g];
                f32x4 v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                if (slot >= 0 && rr < a.rank)
                    v = *reinterpret_cast<const f32x4 *>(static_cast<const XT *>(a.dense_a) +
                                                         (slot * a.rank + rr) * a.d_in + k0 + c * EV);
                *reinterpret_cast<f32x4 *>(chunk + gr * a.arow + c * EV) = v;
            }
        }
        __syncthreads();

        // this wave's share of the chunk's k-steps
        const int steps = kn / KSTEP;
        const int s_lo = ksi * steps / KS, s_hi = (ksi + 1) * steps / KS;
        const XT *xl = xrow + k0 + (kBf16 ? 8 : 4) * gq;
        // A-fragment: rank row r16 of group g; position of k-step s inside the chunk
        auto a_off = [&](int s) -> int {
            if constexpr (SRC == SRC_INDEXED) {
                return kBf16 ? (s >> 1) * 16 + 8 * (gq & 1) : (s >> 2) * 16 + 4 * gq;
            } else {
                return s * KSTEP + (kBf16 ? 8 : 4) * gq;
            }
        };
        typedef typename std::conditional<kBf16, bf16x8, f32x4>::type XV;
        constexpr int U = 8;
        // One batch = U k-steps. A fragments of the batch are read from LDS up front, then
        // the MFMAs; the next batch's x loads are always in flight (when there is no next
        // batch every lane reads the same dummy address), so the loop has no branches
        // between a load and its use.
        auto compute_batch = [&](const XV *xv, int s0, int nsteps) {
            XV av[U][GM];
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int g = 0; g < GM; ++g)
                    if (u < nsteps)
                        av[u][g] = *reinterpret_cast<const XV *>(chunk + (g * 16 + r16) * a.arow + a_off(s0 + u));
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (u >= nsteps) break;
#pragma unroll
                for (int g = 0; g < GM; ++g) {
                    if constexpr (kBf16) {
                        acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[u][g], xv[u], acc[g], 0, 0, 0);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            acc[g] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u][g][e], xv[u][e], acc[g], 0, 0, 0);
                    }
                }
            }
        };
        const XT *dummy = static_cast<const XT *>(a.x);
        auto load_batch = [&](XV *buf, int s0, bool real) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const XT *ptr = real ? xl + KSTEP * (s0 + u) : dummy;
                buf[u] = *reinterpret_cast<const XV *>(ptr);
            }
        };
        const int nfull = (s_hi - s_lo) / U;
        int s = s_lo;
        XV xa[U], xb[U];
        if (nfull > 0) load_batch(xa, s, true);
        for (int i = 0; i < nfull; i += 2) {
            load_batch(xb, s + U, i + 1 < nfull);
            __builtin_amdgcn_sched_barrier(0);    // keep the prefetch ahead of this batch's MFMAs
            compute_batch(xa, s, U);
            s += U;
            if (i + 1 >= nfull) break;
            load_batch(xa, s + U, i + 2 < nfull);
            __builtin_amdgcn_sched_barrier(0);
            compute_batch(xb, s, U);
            s += U;
        }
        const int rem = s_hi - s;
        if (rem > 0) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const XT *ptr = u < rem ? xl + KSTEP * (s + u) : dummy;
                xa[u] = *reinterpret_cast<const XV *>(ptr);
            }
            compute_batch(xa, s, rem);
        }
    }

    // acc[g][e] = partial sum for token r16, rank 4*gq + e of group g over this wave's k-slices
    const float ms_b = a.mid_scale ? a.mid_scale[b] : 1.0f;
    if (KS > 1) {
        float *red = reinterpret_cast<float *>(smem + a.red_off);
#pragma unroll
        for (int g = 0; g < GM; ++g) *reinterpret_cast<f32x4 *>(red + ((wave * GM + g) * 64 + lane) * 4) = acc[g];
        __syncthreads();
        if (ksi != 0) return;
#pragma unroll
        for (int g = 0; g < GM; ++g) {
            f32x4 sum = *reinterpret_cast<const f32x4 *>(red + ((tgi * GM + g) * 64 + lane) * 4);
            for (int k2 = 1; k2 < KS; ++k2)
                sum += *reinterpret_cast<const f32x4 *>(red + (((k2 * TG + tgi) * GM + g) * 64 + lane) * 4);
            acc[g] = sum;
        }
    }
    if (!valid) return;
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        if (s_slot[g] < 0) continue;
        XT *dst = static_cast<XT *>(a.mid) + row * a.MR + g * 16 + 4 * gq;
        if constexpr (kBf16) {
            bf16x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = (__bf16)(acc[g][e] * ms_b);
            *reinterpret_cast<bf16x4 *>(dst) = o;
        } else {
            *reinterpret_cast<f32x4 *>(dst) = acc[g] * ms_b;
        }
    }
}

// ============================================================================ expand
template <typename YT>
__device__ __forceinline__ float finish(float acc, float s, float yold, int accumulate) {
    const float d = DT<YT>::round(DT<YT>::round(acc) * s);
    return accumulate ? DT<YT>::round(yold + d) : d;
}

// y vector of 8 consecutive outputs (16 B for bf16, 32 B for fp32).
template <typename YT> struct Y8;
template <> struct Y8<__bf16> {
    bf16x8 v;
    __device__ __forceinline__ void load(const __bf16 *p) { v = *reinterpret_cast<const bf16x8 *>(p); }
    __device__ __forceinline__ void store(__bf16 *p) const { *reinterpret_cast<bf16x8 *>(p) = v; }
    __device__ __forceinline__ float get(int e) const { return (float)v[e]; }
    __device__ __forceinline__ void set(int e, float f) { v[e] = (__bf16)f; }
};
template <> struct Y8<float> {
    f32x4 lo, hi;
    __device__ __forceinline__ void load(const float *p) {
        lo = *reinterpret_cast<const f32x4 *>(p);
        hi = *reinterpret_cast<const f32x4 *>(p + 4);
    }
    __device__ __forceinline__ void store(float *p) const {
        *reinterpret_cast<f32x4 *>(p) = lo;
        *reinterpret_cast<f32x4 *>(p + 4) = hi;
    }
    __device__ __forceinline__ float get(int e) const { return e < 4 ? lo[e] : hi[e - 4]; }
    __device__ __forceinline__ void set(int e, float f) {
        if (e < 4) lo[e] = f;
        else hi[e - 4] = f;
    }
};

template <typename XT, typename YT, int SRC, int GM, int BOM, bool ACC>
__global__ void __launch_bounds__(kThreads) expand_kernel(LoraArgs a) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    __shared__ float lut[kMaxLevels * 10];
    __shared__ int64_t s_slot[kMaxGroups];
    __shared__ float s_w[kMaxGroups];
    __shared__ int s_any;

    const int tid = threadIdx.x;
    // wave index as a scalar: loop bounds derived from it stay uniform (SGPR) branches
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, r16 = lane & 15, gq = lane >> 4;
    const int o_tiles = (int)((a.d_out + a.BO - 1) / a.BO);
    const int64_t obase = (int64_t)(blockIdx.x % o_tiles) * a.BO;
    const int tile = blockIdx.x / o_tiles;
    const int64_t b = tile / a.tiles_e;
    const int mt = tile % a.tiles_e;
    const float s_b = a.out_scale_vec ? a.out_scale_vec[b] : a.out_scale;

    const bool any = load_route(a, b, s_slot, s_w, &s_any);
    if (!any) {
        if (ACC) return;
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
        const int items = GM * a.BO;
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

    // ---- B fragments into registers. MFMA (p, h) row i <-> output 32p + 8(i/4) + 4h + (i%4),
    // so lane (token r16, group gq) ends with outputs 32p + 8gq .. +7 of its token.
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
                if (p < np) {
                    const XT *src = bt + (g * a.BO + ol) * a.brs + 4 * gq;
                    if constexpr (sizeof(XT) == 2) bfr[p][h][g] = *reinterpret_cast<const i16x4 *>(src);
                    else bfr[p][h][g] = *reinterpret_cast<const f32x4 *>(src);
                } else {
                    bfr[p][h][g] = Frag{};
                }
            }
        }
    }

    auto compute = [&](const Frag *mf, int p, float vals[8]) {
        f32x4 acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int g = 0; g < GM; ++g) {
                if constexpr (sizeof(XT) == 2) {
                    acc[h] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bfr[p][h][g], mf[g], acc[h], 0, 0, 0);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        acc[h] = __builtin_amdgcn_mfma_f32_16x16x4f32(bfr[p][h][g][e], mf[g][e], acc[h], 0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            vals[e] = acc[0][e];
            vals[4 + e] = acc[1][e];
        }
    };
    // mid fragments; groups without an adapter point at group 0 of the same row (their B
    // tile is zero), so every lane issues the same unconditional loads.
    int gsrc[GM];
#pragma unroll
    for (int g = 0; g < GM; ++g) gsrc[g] = (g < a.G && s_slot[g] >= 0) ? g : 0;
    auto load_mid = [&](int64_t row, Frag *mf) {
#pragma unroll
        for (int g = 0; g < GM; ++g) {
            const XT *src = static_cast<const XT *>(a.mid) + row * a.MR + gsrc[g] * 16 + 4 * gq;
            if constexpr (sizeof(XT) == 2) mf[g] = *reinterpret_cast<const i16x4 *>(src);
            else mf[g] = *reinterpret_cast<const f32x4 *>(src);
        }
    };
    auto sub_row = [&](int sub, bool &valid) -> int64_t {
        const int64_t m = ((int64_t)mt * a.subs_e + sub) * (kWaves * 16) + wave * 16 + r16;
        valid = m < a.seq;
        return b * a.seq + (valid ? m : a.seq - 1);
    };

    if (a.vec_y) {
        // Vector path: every load is unconditional (rows and columns clamped in range).
        // Two sub-tile buffers ping-pong: the next sub-tile's mid and y loads are in
        // flight while the current one computes and stores; with no next sub-tile they
        // read one dummy address, so no branch separates a load from its use.
        const int64_t omax = a.d_out - 8;
        const YT *ydummy = static_cast<const YT *>(a.y);
        struct Sub {
            int64_t row;
            bool valid;
            Frag mf[GM];
            Y8<YT> yv[NP];
        };
        auto load_sub = [&](Sub &t, int sub, bool real) {
            t.row = sub_row(real ? sub : 0, t.valid);
            t.valid = t.valid && real;
            load_mid(t.row, t.mf);
            if constexpr (ACC) {
#pragma unroll
                for (int p = 0; p < NP; ++p)
                    if (p < np)
                        t.yv[p].load(real ? static_cast<const YT *>(a.y) + t.row * a.d_out +
                                                std::min<int64_t>(obase + 32 * p + 8 * gq, omax)
                                          : ydummy);
            }
        };
        auto process = [&](const Sub &t) {
            YT *yr = static_cast<YT *>(a.y) + t.row * a.d_out;
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                if (p >= np) break;
                float vals[8];
                compute(t.mf, p, vals);
                const int64_t o8 = obase + 32 * p + 8 * gq;
                Y8<YT> out;
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    out.set(e, finish<YT>(vals[e], s_b, ACC ? t.yv[p].get(e) : 0.0f, ACC));
                if (t.valid && o8 < a.d_out) out.store(yr + o8);
            }
        };
        Sub ta, tb;
        load_sub(ta, 0, true);
        for (int sub = 0; sub < a.subs_e; sub += 2) {
            load_sub(tb, sub + 1, sub + 1 < a.subs_e);
            __builtin_amdgcn_sched_barrier(0);
            process(ta);
            if (sub + 1 >= a.subs_e) break;
            load_sub(ta, sub + 2, sub + 2 < a.subs_e);
            __builtin_amdgcn_sched_barrier(0);
            process(tb);
        }
    } else {
        // Element path for d_out not a multiple of 8 (rows not 16-byte aligned).
        for (int sub = 0; sub < a.subs_e; ++sub) {
            bool valid;
            const int64_t row = sub_row(sub, valid);
            Frag mf[GM];
            load_mid(row, mf);
            YT *yr = static_cast<YT *>(a.y) + row * a.d_out;
            for (int p = 0; p < np; ++p) {
                float vals[8];
                compute(mf, p, vals);
                const int64_t o8 = obase + 32 * p + 8 * gq;
                if (!valid) continue;
                for (int e = 0; e < 8; ++e) {
                    if (o8 + e >= a.d_out) break;
                    const float yo = ACC ? DT<YT>::to_f32(yr[o8 + e]) : 0.0f;
                    yr[o8 + e] = DT<YT>::from_f32(finish<YT>(vals[e], s_b, yo, ACC));
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
    int tiles_s, tg, Kc, arow, red_off;
    size_t lds_s;
    int tiles_e, subs_e, BO, BOM, brs;
    size_t lds_e;
    int64_t off_mid, total;
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
    const int target = env_int("LITHE_TARGET_WGS", 1024);

    // shrink: 16*tg tokens per workgroup, the K range split over 4/tg waves per token group.
    int tg = 4;
    while (tg > 1 && n_batch * ((seq + 16 * tg - 1) / (16 * tg)) < target) tg /= 2;
    if (getenv("LITHE_SHRINK_TG")) {
        const int v = env_int("LITHE_SHRINK_TG", tg);
        tg = v >= 4 ? 4 : v >= 2 ? 2 : 1;
    }
    p.tg = tg;
    p.tiles_s = (int)std::max<int64_t>(1, (seq + 16 * tg - 1) / (16 * tg));
    const int pad = 16 / xbytes;
    const int budget = env_int("LITHE_CHUNK_LDS", 26 * 1024);
    const int64_t rowbytes_per_k = dense ? xbytes : 0;      // dense rows: 1 element per k
    int64_t kc;
    if (dense) {
        kc = ((budget / (p.GM * 16 * xbytes) - pad) / 64) * 64;
    } else {
        kc = ((budget / (p.GM * 16 * xbytes) - pad) / 16) * 64;    // one 16-value period per 64 k
    }
    (void)rowbytes_per_k;
    kc = std::max<int64_t>(64, kc);
    const int64_t nb_total = d_in / kBlock;
    const int64_t nchunk = (d_in + kc - 1) / kc;
    const int64_t nb = (nb_total + nchunk - 1) / nchunk;     // balanced chunks
    p.Kc = (int)(nb * kBlock);
    p.arow = dense ? (int)(p.Kc + pad) : (int)(nb * 16 + pad);
    const size_t chunk_bytes = (size_t)p.GM * 16 * p.arow * xbytes;
    p.red_off = (int)((chunk_bytes + 15) & ~size_t(15));
    p.lds_s = p.red_off + (tg < 4 ? (size_t)kWaves * p.GM * 64 * 16 : 0);

    // expand: BO outputs x 64*subs tokens per workgroup.
    int bo_max = xbytes == 2 ? std::min(256, 512 / p.GM) : std::min(128, 256 / p.GM);
    bo_max = std::max(32, bo_max);
    p.BOM = bo_max;
    p.BO = (int)std::min<int64_t>(bo_max, ((d_out + 31) / 32) * 32);
    p.brs = 16 + 4;
    p.lds_e = (size_t)p.GM * p.BO * p.brs * xbytes;
    const int64_t o_tiles = (d_out + p.BO - 1) / p.BO;
    const int64_t base_items = n_batch * ((seq + 63) / 64) * o_tiles;
    int subs = (int)std::max<int64_t>(1, std::min<int64_t>(4, base_items / (2 * target)));
    if (getenv("LITHE_EXPAND_SUBS")) subs = env_int("LITHE_EXPAND_SUBS", subs);
    p.subs_e = subs;
    p.tiles_e = (int)std::max<int64_t>(1, (seq + 64 * (int64_t)subs - 1) / (64 * (int64_t)subs));

    // workspace: [error word | mid]
    p.off_mid = 256;
    p.total = align256(p.off_mid + rows * p.MR * xbytes);
    return p;
}

template <typename XT, typename YT, int SRC, int GM, int BOM>
void launch(const Plan &p, LoraArgs &a, hipStream_t st) {
    dim3 gs((unsigned)(a.n_batch * p.tiles_s));
    hipLaunchKernelGGL((shrink_kernel<XT, SRC, GM>), gs, dim3(kThreads), p.lds_s, st, a);
    dim3 ge((unsigned)(((a.d_out + p.BO - 1) / p.BO) * a.n_batch * p.tiles_e));
    if (a.accumulate)
        hipLaunchKernelGGL((expand_kernel<XT, YT, SRC, GM, BOM, true>), ge, dim3(kThreads), p.lds_e, st, a);
    else
        hipLaunchKernelGGL((expand_kernel<XT, YT, SRC, GM, BOM, false>), ge, dim3(kThreads), p.lds_e, st, a);
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
    a.mid = ws + p.off_mid;
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
    a.tg = p.tg;
    a.Kc = p.Kc;
    a.arow = p.arow;
    a.red_off = p.red_off;
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
