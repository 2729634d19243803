// Per-sample LoRA delta with the factors decoded from index streams (or read dense):
//
//   decode:  period[b, j, blk, 0..15] = round_x( w * sum_l lut[l][popc((k_l ^ m_t) & 511)] )
//   shrink:  mid[row, g*16 + r]      = round_x( sum_k x[row, k] * A_g[r, k] * mid_scale[b] )
//   expand:  y[row, o]               = round_y( y + round_y( round_y( sum_{g,r} mid * B_g[o, r] ) * s_b ) )
//
// The codewords repeat with period 16 (lithe_common.h), so a decoded 64-value block is
// fully described by 16 values. One small decode launch writes those periods for the
// routed adapters of the batch into the workspace, 4x smaller than the dense factors
// and far smaller than a tile of x; the shrink and expand kernels then stream x and y
// and read factor fragments from the cache-resident periods. Nothing is decoded twice.
//
// g runs over "rank groups": route entry j of a sample contributes ceil(rank/16) groups of
// 16 ranks (rank-stacked mixtures, lithe/serve.py:89-96).
//
// shrink  v_mfma_f32_16x16x32_bf16 (fp32: 16x16x4 f32), one wave per 16 tokens x K slice.
//         A-operand = factor rows (lane%16 = rank), B-operand = x^T (lane%16 = token); lane
//         group q = lane/16 owns k = 8q..8q+7 of each 32-wide step, so every row of x is read
//         in 64-byte pieces. Loads are software-pipelined two batches deep with no branch
//         between a load and its use. Waves that split one token group's K range reduce
//         their fp32 partials through LDS in a fixed order (deterministic).
// expand  v_mfma_f32_16x16x16_bf16 (fp32: 16x16x4 f32) with the factor B tile as the
//         A-operand (lane%16 = output row) and mid^T as the B-operand (lane%16 = token).
//         Output rows are assigned so that each lane ends with 8 consecutive outputs of its
//         token: y is read-modified-written 16 bytes per lane with the reference's rounding
//         chain applied in registers, the next sub-tile's loads in flight.
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
    void *pat_a;        // (n_batch * n_route, n_rg * 16, d_in / 64, 16) periods of A, rows padded to 16
    void *pat_b;        // (n_batch * n_route, d_out * rank / 64, 16) periods of B
    int32_t *err;
    int64_t n_batch, seq, d_in, d_out, rows;
    int64_t nb_a_route, nb_b_route;   // blocks per route entry in pat_a / pat_b
    int32_t rank, G, n_rg, n_route, MR;
    int32_t tiles_s, ks, Kc, arow, red_off;
    int32_t tiles_e, subs_e, BO, vec_y;
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

// Slot of route entry j of sample b, or -1 (empty entry or out of range; the latter is recorded).
__device__ __forceinline__ int64_t route_slot(const LoraArgs &a, int64_t b, int j, bool record) {
    const int32_t s = a.r_slot[b * a.n_route + j];
    if (s >= 0 && (int64_t)s < a.n_slots) return s;
    if (record && s != -1) record_error(a.err, kErrSlot);
    return -1;
}

// ============================================================================ decode
// One thread per (route entry, block) of A or B: the 16-value period of the block, with the
// route's multipliers (sqrt mixture weight; alpha / r for B) applied before the cast to the
// activation dtype. Empty entries and the padding rows of A (rank not a multiple of 16)
// are written as zeros.
template <typename XT>
__global__ void __launch_bounds__(kThreads) decode_periods_kernel(LoraArgs a, int64_t n_a_items,
                                                                  int64_t n_items) {
    __shared__ float lut[2 * kMaxLevels * 10];
    if (threadIdx.x < 2 * kMaxLevels * 10) lut[threadIdx.x] = (&a.luts.v[0][0][0])[threadIdx.x];
    __syncthreads();
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= n_items) return;
    const bool is_a = i < n_a_items;
    const int64_t li = is_a ? i : i - n_a_items;
    const int64_t per = is_a ? a.nb_a_route : a.nb_b_route;
    const int64_t bj = li / per, blk = li % per;
    const int64_t b = bj / a.n_route;
    const int j = (int)(bj % a.n_route);
    const int64_t slot = route_slot(a, b, j, is_a && blk == 0);
    float v[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) v[t] = 0.0f;
    int64_t src_blk = blk;
    bool live = slot >= 0;
    if (is_a) {
        // pat_a rows are padded to 16 per rank group: row = blk / row_blocks
        const int64_t row_blocks = a.d_in / kBlock;
        const int64_t r = blk / row_blocks;
        live = live && r < a.rank;
        src_blk = r * row_blocks + blk % row_blocks;
    }
    if (live) {
        uint32_t k[kMaxLevels];
        const IdxSrc &src = is_a ? a.a_src : a.b_src;
        if (!fetch_indices(src, slot, src_blk, k)) record_error(a.err, kErrIndex);
        const float *tab = lut + (is_a ? 0 : kMaxLevels * 10);
        const float w = a.r_w ? a.r_w[b * a.n_route + j] : 1.0f;
        const float sc = (!is_a && a.s_scale) ? a.s_scale[slot] : 1.0f;
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const float d = decode_value(tab, src.levels, k, sign_mask(t));
            v[t] = is_a ? d * w : (d * sc) * w;
        }
    }
    XT *dst = static_cast<XT *>(is_a ? a.pat_a : a.pat_b) + li * 16;
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
        for (int t = 0; t < 16; t += 4) *reinterpret_cast<f32x4 *>(dst + t) = f32x4{v[t], v[t + 1], v[t + 2], v[t + 3]};
    }
}

// ============================================================================ shrink
// Workgroup = 4 waves of one sample; each wave owns 16 tokens and 1/ks of every K chunk
// (ks waves share a token group). The sample's decoded A periods of a K chunk are copied
// into LDS once per workgroup, so A fragments come from LDS (ds_read) while x streams
// through the vector memory path. Waves that split a token group's K range reduce their
// fp32 partials through LDS in a fixed order (deterministic).
template <typename XT, int SRC, int GM, int U>
__global__ void __launch_bounds__(kThreads) shrink_kernel(LoraArgs a) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    constexpr bool kBf16 = sizeof(XT) == 2;
    constexpr int KSTEP = kBf16 ? 32 : 16;
    constexpr int EV = 16 / sizeof(XT);      // elements per 16-byte vector
    typedef typename std::conditional<kBf16, bf16x8, f32x4>::type XV;

    const int tid = threadIdx.x;
    // wave index as a scalar: loop bounds derived from it stay uniform (SGPR) branches
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, r16 = lane & 15, gq = lane >> 4;
    const int ks = a.ks, tgw = kWaves / a.ks;
    const int tgi = wave % tgw, ksi = wave / tgw;
    const int tile = blockIdx.x;
    const int64_t b = tile / a.tiles_s;
    const int mt = tile % a.tiles_s;
    const int64_t m = ((int64_t)mt * tgw + tgi) * 16 + r16;
    const bool valid = m < a.seq;
    const int64_t row = b * a.seq + (valid ? m : a.seq - 1);

    int64_t gslot[GM];
#pragma unroll
    for (int g = 0; g < GM; ++g) gslot[g] = g < a.G ? route_slot(a, b, (g < a.G ? g : 0) / a.n_rg, false) : -1;

    XT *chunk = reinterpret_cast<XT *>(smem);
    float *red = reinterpret_cast<float *>(smem + a.red_off);
    const int64_t row_blocks = a.d_in / kBlock;
    f32x4 acc[GM];
#pragma unroll
    for (int g = 0; g < GM; ++g) acc[g] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const XT *xrow = static_cast<const XT *>(a.x) + row * a.d_in + (kBf16 ? 8 : 4) * gq;
    const XT *dummy = static_cast<const XT *>(a.x);

    for (int64_t k0 = 0; k0 < a.d_in; k0 += a.Kc) {
        const int kn = (int)std::min<int64_t>(a.Kc, a.d_in - k0);
        const int nbk = kn / kBlock;
        __syncthreads();   // previous chunk consumed
        // ---- fill: rows (g, r) of the chunk, 16 B per thread per step
        if constexpr (SRC == SRC_INDEXED) {
            const int per_row = nbk * 16 / EV;
            const int items = GM * 16 * per_row;
            for (int it = tid; it < items; it += kThreads) {
                const int c = it % per_row, gr = it / per_row;
                const int g = gr >> 4, r = gr & 15;
                const int gg = g < a.G ? g : 0;
                const int j = gg / a.n_rg, rr = (gg % a.n_rg) * 16 + r;
                f32x4 v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                if (g < a.G)
                    v = *reinterpret_cast<const f32x4 *>(static_cast<const XT *>(a.pat_a) +
                                                         (((b * a.n_route + j) * a.n_rg * 16 + rr) * row_blocks +
                                                          k0 / kBlock) * 16 + c * EV);
                *reinterpret_cast<f32x4 *>(chunk + gr * a.arow + c * EV) = v;
            }
        } else {
            const int per_row = kn / EV;
            const int items = GM * 16 * per_row;
            for (int it = tid; it < items; it += kThreads) {
                const int c = it % per_row, gr = it / per_row;
                const int g = gr >> 4, r = gr & 15;
                const int rr = ((g < a.G ? g : 0) % a.n_rg) * 16 + r;
                f32x4 v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                if (g < a.G && gslot[g] >= 0 && rr < a.rank)
                    v = *reinterpret_cast<const f32x4 *>(static_cast<const XT *>(a.dense_a) +
                                                         (gslot[g] * a.rank + rr) * a.d_in + k0 + c * EV);
                *reinterpret_cast<f32x4 *>(chunk + gr * a.arow + c * EV) = v;
            }
        }
        __syncthreads();

        // ---- stream this wave's share of the chunk's k-steps
        const int steps = kn / KSTEP;
        const int s_lo = ksi * steps / ks, s_hi = (ksi + 1) * steps / ks;
        const XT *xl = xrow + k0;
        auto a_ptr = [&](int g, int s) -> const XT * {
            if constexpr (SRC == SRC_INDEXED) {
                return chunk + (g * 16 + r16) * a.arow +
                       (kBf16 ? (s >> 1) * 16 + 8 * (gq & 1) : (s >> 2) * 16 + 4 * gq);
            } else {
                return chunk + (g * 16 + r16) * a.arow + s * KSTEP + (kBf16 ? 8 : 4) * gq;
            }
        };
        struct Batch {
            XV x[U];
        };
        auto load_batch = [&](Batch &bt, int s0, bool real) {
#pragma unroll
            for (int u = 0; u < U; ++u)
                bt.x[u] = *reinterpret_cast<const XV *>(real ? xl + (int64_t)KSTEP * (s0 + u) : dummy);
        };
        auto compute_batch = [&](const Batch &bt, int s0, int nsteps) {
            XV av[U][GM];
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int g = 0; g < GM; ++g)
                    if (u < nsteps) av[u][g] = *reinterpret_cast<const XV *>(a_ptr(g, s0 + u));
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (u >= nsteps) break;
#pragma unroll
                for (int g = 0; g < GM; ++g) {
                    if constexpr (kBf16) {
                        acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[u][g], bt.x[u], acc[g], 0, 0, 0);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            acc[g] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u][g][e], bt.x[u][e], acc[g], 0, 0, 0);
                    }
                }
            }
        };
        const int nfull = (s_hi - s_lo) / U;
        int s = s_lo;
        Batch ba, bb;
        if (nfull > 0) load_batch(ba, s, true);
        for (int i = 0; i < nfull; i += 2) {
            load_batch(bb, s + U, i + 1 < nfull);
            __builtin_amdgcn_sched_barrier(0);    // keep the prefetch ahead of this batch's MFMAs
            compute_batch(ba, s, U);
            s += U;
            if (i + 1 >= nfull) break;
            load_batch(ba, s + U, i + 2 < nfull);
            __builtin_amdgcn_sched_barrier(0);
            compute_batch(bb, s, U);
            s += U;
        }
        const int rem = s_hi - s;
        if (rem > 0) {
#pragma unroll
            for (int u = 0; u < U; ++u)
                ba.x[u] = *reinterpret_cast<const XV *>(u < rem ? xl + (int64_t)KSTEP * (s + u) : dummy);
            compute_batch(ba, s, rem);
        }
    }

    // acc[g][e]: token r16, rank 4*gq + e of group g, summed over this wave's k range
    if (ks > 1) {
#pragma unroll
        for (int g = 0; g < GM; ++g) *reinterpret_cast<f32x4 *>(red + ((wave * GM + g) * 64 + lane) * 4) = acc[g];
        __syncthreads();
        if (ksi != 0) return;
#pragma unroll
        for (int g = 0; g < GM; ++g) {
            f32x4 sum = *reinterpret_cast<const f32x4 *>(red + ((tgi * GM + g) * 64 + lane) * 4);
            for (int k2 = 1; k2 < ks; ++k2)
                sum += *reinterpret_cast<const f32x4 *>(red + (((k2 * tgw + tgi) * GM + g) * 64 + lane) * 4);
            acc[g] = sum;
        }
    }
    if (!valid) return;
    const float ms_b = a.mid_scale ? a.mid_scale[b] : 1.0f;
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        if (g >= a.G || gslot[g] < 0) continue;
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
__device__ __forceinline__ float finish(float acc, float s, float yold, bool accumulate) {
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
    typedef typename std::conditional<sizeof(XT) == 2, i16x4, f32x4>::type Frag;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, r16 = lane & 15, gq = lane >> 4;
    const int o_tiles = (int)((a.d_out + a.BO - 1) / a.BO);
    const int64_t obase = (int64_t)(blockIdx.x % o_tiles) * a.BO;
    const int tile = blockIdx.x / o_tiles;
    const int64_t b = tile / a.tiles_e;
    const int mt = tile % a.tiles_e;
    const float s_b = a.out_scale_vec ? a.out_scale_vec[b] : a.out_scale;

    int64_t gslot[GM];
    bool any = false;
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        gslot[g] = g < a.G ? route_slot(a, b, g / a.n_rg, false) : -1;
        any = any || gslot[g] >= 0;
    }
    auto sub_row = [&](int sub, bool &valid) -> int64_t {
        const int64_t m = ((int64_t)mt * a.subs_e + sub) * (kWaves * 16) + wave * 16 + r16;
        valid = m < a.seq;
        return b * a.seq + (valid ? m : a.seq - 1);
    };
    if (!any) {
        if (ACC) return;
        // Empty route in write mode: the delta is zero.
        for (int sub = 0; sub < a.subs_e; ++sub) {
            bool valid;
            const int64_t row = sub_row(sub, valid);
            if (!valid) continue;
            YT *yr = static_cast<YT *>(a.y) + row * a.d_out;
            for (int o = gq; o < a.BO; o += 4)
                if (obase + o < a.d_out) yr[obase + o] = DT<YT>::from_f32(0.0f);
        }
        return;
    }

    // ---- B fragments into registers. MFMA (p, h) row i <-> output 32p + 8(i/4) + 4h + (i%4),
    // so lane (token r16, group gq) ends with outputs 32p + 8gq .. +7 of its token.
    constexpr int NP = BOM / 32;
    const int np = a.BO / 32;
    Frag bfr[NP][2][GM];
    // With rank % 4 == 0 the 4 ranks of a fragment are 4 consecutive values of one period
    // (f = o * rank + rr is a multiple of 4), so each fragment is one 8-byte (fp32: 16-byte) load.
    const bool quad = (a.rank & 3) == 0;
#pragma unroll
    for (int p = 0; p < NP; ++p) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t o = obase + 32 * p + 8 * (r16 >> 2) + 4 * h + (r16 & 3);
#pragma unroll
            for (int g = 0; g < GM; ++g) {
                const int gg = g < a.G ? g : 0;
                const int j = gg / a.n_rg;
                const int rr = (gg % a.n_rg) * 16 + 4 * gq;
                const bool live = p < np && gslot[g] >= 0 && o < a.d_out && rr < a.rank;
                Frag fr = Frag{};
                if (live) {
                    if (SRC == SRC_INDEXED && quad) {
                        const int64_t f = o * a.rank + rr;
                        const XT *src = static_cast<const XT *>(a.pat_b) + (b * a.n_route + j) * a.nb_b_route * 16 +
                                        (f >> 6) * 16 + (f & 15);
                        if constexpr (sizeof(XT) == 2) fr = *reinterpret_cast<const i16x4 *>(src);
                        else fr = *reinterpret_cast<const f32x4 *>(src);
                    } else {
                        float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            if (rr + e >= a.rank) break;
                            if constexpr (SRC == SRC_INDEXED) {
                                const int64_t f = o * a.rank + rr + e;
                                v[e] = DT<XT>::to_f32(static_cast<const XT *>(a.pat_b)[
                                    (b * a.n_route + j) * a.nb_b_route * 16 + (f >> 6) * 16 + (f & 15)]);
                            } else {
                                v[e] = DT<XT>::to_f32(static_cast<const XT *>(a.dense_b)[
                                    (gslot[g] * a.d_out + o) * a.rank + rr + e]);
                            }
                        }
                        if constexpr (sizeof(XT) == 2) {
#pragma unroll
                            for (int e = 0; e < 4; ++e) fr[e] = __builtin_bit_cast(short, (__bf16)v[e]);
                        } else {
                            fr = f32x4{v[0], v[1], v[2], v[3]};
                        }
                    }
                }
                bfr[p][h][g] = fr;
            }
        }
    }

    auto compute = [&](const Frag *mf, int p, float vals[8]) {
        f32x4 acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int g = 0; g < GM; ++g) {
                // a group without an adapter contributes exact zeros (its mid slot is not written)
                const Frag m = gslot[g] >= 0 ? mf[g] : Frag{};
                if constexpr (sizeof(XT) == 2) {
                    acc[h] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bfr[p][h][g], m, acc[h], 0, 0, 0);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        acc[h] = __builtin_amdgcn_mfma_f32_16x16x4f32(bfr[p][h][g][e], m[e], acc[h], 0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            vals[e] = acc[0][e];
            vals[4 + e] = acc[1][e];
        }
    };
    // mid fragments; groups without an adapter read group 0 of the same row (their B
    // fragments are zero), so every lane issues the same unconditional loads.
    int gsrc[GM];
#pragma unroll
    for (int g = 0; g < GM; ++g) gsrc[g] = gslot[g] >= 0 ? g : 0;
    auto load_mid = [&](int64_t row, Frag *mf) {
#pragma unroll
        for (int g = 0; g < GM; ++g) {
            const XT *src = static_cast<const XT *>(a.mid) + row * a.MR + gsrc[g] * 16 + 4 * gq;
            if constexpr (sizeof(XT) == 2) mf[g] = *reinterpret_cast<const i16x4 *>(src);
            else mf[g] = *reinterpret_cast<const f32x4 *>(src);
        }
    };

    if (a.vec_y) {
        // Vector path: every load is unconditional (rows and columns clamped in range).
        // Two sub-tile buffers ping-pong: the next sub-tile's mid and y loads are in
        // flight while the current one computes and stores; with no next sub-tile they
        // read one dummy address, so no branch separates a load from its use.
        const int64_t omax = a.d_out - 8;
        const YT *ydummy = static_cast<const YT *>(a.y);
        const XT *mdummy = static_cast<const XT *>(a.mid);
        struct Sub {
            int64_t row;
            bool valid;
            Frag mf[GM];
            Y8<YT> yv[NP];
        };
        auto load_sub = [&](Sub &t, int sub, bool real) {
            t.row = sub_row(real ? sub : 0, t.valid);
            t.valid = t.valid && real;
#pragma unroll
            for (int g = 0; g < GM; ++g) {
                const XT *src = real ? static_cast<const XT *>(a.mid) + t.row * a.MR + gsrc[g] * 16 + 4 * gq : mdummy;
                if constexpr (sizeof(XT) == 2) t.mf[g] = *reinterpret_cast<const i16x4 *>(src);
                else t.mf[g] = *reinterpret_cast<const f32x4 *>(src);
            }
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
    int tiles_s, ks, Kc, arow, red_off;
    size_t lds_s;
    int tiles_e, subs_e, BO, BOM, U;
    int64_t nb_a_route, nb_b_route;
    int64_t off_mid, off_pa, off_pb, total;
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
    const int target = env_int("LITHE_TARGET_WAVES", 2048);

    // shrink: one wave per 16 tokens x (K / ks); ks grows until there are enough waves.
    const int64_t groups = n_batch * ((seq + 15) / 16);
    int ks = 1;
    while (ks < 4 && groups * ks < target) ks *= 2;
    if (getenv("LITHE_SHRINK_KS")) {
        const int v = env_int("LITHE_SHRINK_KS", ks);
        ks = v >= 4 ? 4 : v >= 2 ? 2 : 1;
    }
    p.ks = ks;
    const int tgw = kWaves / ks;
    p.tiles_s = (int)std::max<int64_t>(1, (seq + 16 * tgw - 1) / (16 * tgw));
    // LDS chunk of A: GM*16 rows; periods (16 values per 64 k) or dense rows (one value per k)
    const int pad = 16 / xbytes;
    const int budget = env_int("LITHE_CHUNK_LDS", 26 * 1024);
    int64_t kc = dense ? ((budget / (p.GM * 16 * xbytes) - pad) / 64) * 64
                       : ((budget / (p.GM * 16 * xbytes) - pad) / 16) * 64;
    kc = std::max<int64_t>(64, kc);
    const int64_t nb_total = d_in / kBlock;
    const int64_t nchunk = (d_in + kc - 1) / kc;
    const int64_t nbc = (nb_total + nchunk - 1) / nchunk;     // balanced chunks
    p.Kc = (int)(nbc * kBlock);
    p.arow = dense ? (int)(p.Kc + pad) : (int)(nbc * 16 + pad);
    const size_t chunk_bytes = (size_t)p.GM * 16 * p.arow * xbytes;
    p.red_off = (int)((chunk_bytes + 15) & ~size_t(15));
    p.lds_s = p.red_off + (ks > 1 ? (size_t)kWaves * p.GM * 64 * 16 : 0);

    // expand: BO outputs x 64*subs tokens per workgroup.
    int bo_max = xbytes == 2 ? std::min(256, 512 / p.GM) : std::min(128, 256 / p.GM);
    bo_max = std::max(32, bo_max);
    if (p.GM == 1 && env_int("LITHE_EXPAND_BO", 0) == 128) bo_max = 128;
    p.U = (p.GM == 1 && env_int("LITHE_SHRINK_U", 4) == 8) ? 8 : 4;
    p.BOM = bo_max;
    p.BO = (int)std::min<int64_t>(bo_max, ((d_out + 31) / 32) * 32);
    const int64_t o_tiles = (d_out + p.BO - 1) / p.BO;
    const int64_t base_wgs = n_batch * ((seq + 63) / 64) * o_tiles;
    int subs = (int)std::max<int64_t>(1, std::min<int64_t>(4, base_wgs / (2 * target)));
    if (getenv("LITHE_EXPAND_SUBS")) subs = env_int("LITHE_EXPAND_SUBS", subs);
    p.subs_e = subs;
    p.tiles_e = (int)std::max<int64_t>(1, (seq + 64 * (int64_t)subs - 1) / (64 * (int64_t)subs));

    // workspace: [error word | mid | A periods | B periods]
    p.nb_a_route = (int64_t)p.n_rg * 16 * (d_in / kBlock);
    p.nb_b_route = (d_out * rank) / kBlock;
    p.off_mid = 256;
    p.off_pa = align256(p.off_mid + rows * p.MR * xbytes);
    const int64_t pa_bytes = dense ? 0 : n_batch * n_route * p.nb_a_route * 16 * xbytes;
    const int64_t pb_bytes = dense ? 0 : n_batch * n_route * p.nb_b_route * 16 * xbytes;
    p.off_pb = align256(p.off_pa + pa_bytes);
    p.total = align256(p.off_pb + pb_bytes);
    return p;
}

template <typename XT, typename YT, int SRC, int GM, int BOM, int U>
void launch(const Plan &p, LoraArgs &a, hipStream_t st) {
    if constexpr (SRC == SRC_INDEXED) {
        const int64_t na = a.n_batch * a.n_route * a.nb_a_route;
        const int64_t nitems = na + a.n_batch * a.n_route * a.nb_b_route;
        hipLaunchKernelGGL((decode_periods_kernel<XT>), dim3((unsigned)((nitems + kThreads - 1) / kThreads)),
                           dim3(kThreads), 0, st, a, na, nitems);
    }
    hipLaunchKernelGGL((shrink_kernel<XT, SRC, GM, U>), dim3((unsigned)(a.n_batch * p.tiles_s)), dim3(kThreads),
                       p.lds_s, st, a);
    dim3 ge((unsigned)(((a.d_out + p.BO - 1) / p.BO) * a.n_batch * p.tiles_e));
    if (a.accumulate)
        hipLaunchKernelGGL((expand_kernel<XT, YT, SRC, GM, BOM, true>), ge, dim3(kThreads), 0, st, a);
    else
        hipLaunchKernelGGL((expand_kernel<XT, YT, SRC, GM, BOM, false>), ge, dim3(kThreads), 0, st, a);
}

template <typename XT, typename YT, int SRC>
int32_t dispatch_gm(const Plan &p, LoraArgs &a, hipStream_t st) {
    constexpr bool bf = sizeof(XT) == 2;
    switch (p.GM) {
        case 1:
            if (p.U == 8) {
                if (p.BOM == 128) launch<XT, YT, SRC, 1, 128, 8>(p, a, st);
                else launch<XT, YT, SRC, 1, bf ? 256 : 128, 8>(p, a, st);
            } else {
                if (p.BOM == 128) launch<XT, YT, SRC, 1, 128, 4>(p, a, st);
                else launch<XT, YT, SRC, 1, bf ? 256 : 128, 4>(p, a, st);
            }
            break;
        case 2: launch<XT, YT, SRC, 2, bf ? 256 : 128, 4>(p, a, st); break;
        case 4: launch<XT, YT, SRC, 4, bf ? 128 : 64, 4>(p, a, st); break;
        default: launch<XT, YT, SRC, 8, bf ? 64 : 32, 4>(p, a, st); break;
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
    // The indexed plan needs the period buffers, so it bounds the dense one.
    return make_plan(n_batch, seq, d_in, d_out, rank, n_route, x_dtype == LITHE_DT_BF16 ? 2 : 4, false).total;
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
    if (!x || !y || !routes->slot) return LITHE_ERR_NULL;
    if (!workspace) return LITHE_ERR_WORKSPACE;
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
    a.pat_a = ws + p.off_pa;
    a.pat_b = ws + p.off_pb;
    a.n_batch = n_batch;
    a.seq = seq;
    a.d_in = d_in;
    a.d_out = d_out;
    a.rows = n_batch * seq;
    a.nb_a_route = p.nb_a_route;
    a.nb_b_route = p.nb_b_route;
    a.rank = rank;
    a.G = p.G;
    a.n_rg = p.n_rg;
    a.n_route = routes->n_route;
    a.MR = p.MR;
    a.tiles_s = p.tiles_s;
    a.ks = p.ks;
    a.Kc = p.Kc;
    a.arow = p.arow;
    a.red_off = p.red_off;
    a.tiles_e = p.tiles_e;
    a.subs_e = p.subs_e;
    a.BO = p.BO;
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
