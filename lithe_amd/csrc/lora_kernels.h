// Kernels of the per-sample LoRA delta with the factors decoded on the fly from index streams (or read dense):
//
//   shrink:  mid[row, g*16 + r] = round_x( sum_k x[row, k] * A_g[r, k] * mid_scale[b] )
//   expand:  y[row, o]          = round_y( y + round_y( round_y( sum_{g,r} mid * B_g[o, r] ) * s_b ) )
//
// with A_g / B_g decoded in-kernel: value = round_x( w * sum_l lut[l][popc((k_l ^ m_t) & 511)] )
// (B: ((d * slot_scale) * w), the reference's fold of alpha / r into B followed by the sqrt
// mixture weight, lithe/serve.py:69-73, 89-96).
//
// The codewords repeat with period 16 (lithe_common.h), so a decoded 64-value block is
// fully described by 16 values. Each shrink workgroup decodes the periods of its sample's
// A rows for one K chunk straight from the index stream into LDS (a few KB of index words,
// cache-resident after the first workgroup of the sample touches them); each expand
// workgroup decodes the B periods of its output range the same way. Both issue the index
// loads of a fill together and ahead of the tile's first activation loads (route slots and
// weights come through scalar loads), so the decode waits for one memory round trip per K
// chunk while the activation stream is already in flight, and needs no extra launch.
//
// g runs over "rank groups": route entry j of a sample contributes ceil(rank/16) groups of
// 16 ranks (rank-stacked mixtures, lithe/serve.py:89-96).
//
// shrink  v_mfma_f32_16x16x32_bf16 (fp32: 16x16x4 f32), one wave per 16 tokens x K slice (two
//         16-token groups per wave with two or more rank groups). A-operand = factor rows
//         (lane%16 = rank), B-operand = x^T (lane%16 = token); lane group q = lane/16 owns
//         k = 8q..8q+7 of each 32-wide step. x arrives in whole 128-byte-line non-temporal loads,
//         software-pipelined two batches deep, and is reshuffled into that layout through a
//         per-wave LDS stage. Waves that split one token group's K range reduce their fp32
//         partials through LDS in a fixed order (deterministic).
// expand  v_mfma_f32_16x16x16_bf16 (fp32: 16x16x4 f32; 16x16x32 on summed rank groups at ranks
//         that are multiples of 32) with the factor B tile as the A-operand (lane%16 = output
//         row) and mid^T as the B-operand (lane%16 = token). Each lane ends with 8 consecutive
//         outputs of its token; the reference's rounding chain is applied in registers and the
//         deltas pass through LDS so that y is read-modified-written in whole-line non-temporal
//         accesses (whole 1 KB rows per wave with one rank group).
#pragma once

#include <stdint.h>
#include <stdlib.h>

#include <algorithm>
#include <type_traits>

#include "lithe_common.h"

namespace lithe {

bool src_covers(const lithe_index_src &s, int64_t n_blocks);
int32_t validate_src(const lithe_index_src *s);
IdxSrc make_src(const lithe_index_src &s);


constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kMaxGroups = 8;
// Dynamic LDS head of both kernels: the value table of one side. The tile data (A chunk or
// B periods) starts at kHead.
constexpr int kLutFloats = kMaxLevels * 10;
constexpr int kHead = 256;
static_assert(kLutFloats * 4 <= kHead, "LDS head overflow");
// Fill items per thread whose index loads are issued together (the plan keeps a piece's items
// within one batch). One rank group: one item (pieces of at most 16 blocks); the two items more
// cost 30 VGPRs, 4 waves per SIMD instead of 5 (measured: the FLUX sweeps 0.35-0.45 % slower).
// More groups: three.
__host__ __device__ constexpr int fill_batch(int gm) { return gm == 1 ? 1 : 3; }
#ifndef LITHE_SHRINK_U
#define LITHE_SHRINK_U 4
#endif
#ifndef LITHE_STAGE_LOADS
#define LITHE_STAGE_LOADS 2    // one step pair at a time: a 2 KB stage per wave (measured 0.2 % faster than 4 KB)
#endif
constexpr int kShrinkU = LITHE_SHRINK_U;         // k-steps per shrink load batch (even: loads move step pairs)
constexpr int kStageLoads = LITHE_STAGE_LOADS;   // loads of a batch that pass through the LDS stage at once
static_assert(kShrinkU % kStageLoads == 0 && kStageLoads % 2 == 0, "the stage takes whole step pairs");
#ifndef LITHE_EXCHANGE_OUTPUTS
#define LITHE_EXCHANGE_OUTPUTS 128
#endif
#ifndef LITHE_LINE_UNITS
#define LITHE_LINE_UNITS 8     // 16-byte units of one token row per whole-line y access (8, 16, 32)
#endif
#ifndef LITHE_EXPAND_XWAVE
#define LITHE_EXPAND_XWAVE 1   // whole-row y accesses with the delta exchanged across the workgroup's waves
#endif
constexpr int kExchangeOutputs = LITHE_EXCHANGE_OUTPUTS;   // outputs per expand LDS exchange (whole-line y)
constexpr int kLineUnits = LITHE_LINE_UNITS;
constexpr bool kXWave = LITHE_EXPAND_XWAVE != 0;
constexpr int kXWaveBytes = 32 * 512 * 2;                  // the workgroup's delta tile: 32 rows x 512 bf16
static_assert(kLineUnits == 8 || kLineUnits == 16 || kLineUnits == 32, "a y access covers 8, 4 or 2 token rows");

// Factor sources: SRC_PACKED is SRC_INDEXED with both index streams PACKED9 with 3 levels (the
// resident bank of the twin codebook), compiled without the kind dispatch of the other index
// layouts and with the level count fixed.
enum { SRC_INDEXED = 1, SRC_DENSE = 2, SRC_PACKED = 3 };
constexpr int kPackedLevels = 3;
template <int SRC> constexpr int fixed_levels() { return SRC == SRC_PACKED ? kPackedLevels : 0; }
// Expand variants with the cross-wave y path: one rank group, 256-output waves, indexed factors
// (with more groups or the rank collapse the path costs registers: 128 VGPRs and 68 bytes of
// scratch per lane in the 4-waves-per-SIMD variant, 2 waves per SIMD in the others; dense factors'
// 16 KB B tile plus the 32 KB delta tile leave 3 workgroups per CU: decoded-mode sweep 60.7 ->
// 66.9 ms).
template <int SRC, int GM, int BOM, int NS>
constexpr bool kXWaveKernel = kXWave && SRC != SRC_DENSE && GM == 1 && BOM == 256 && NS == 1;

struct LoraArgs {
    const void *x;
    void *y;
    void *mid;
    int32_t *err;
    int64_t n_batch, seq, d_in, d_out, rows;
    int32_t rank, G, n_rg, n_route, MR;
    int32_t tiles_s, ks, pb, arow, region, red_off, stage_off;
    int32_t tiles_e, subs_e, BO, vec_y, nblk_max, estage_off;
    int32_t wo_sh;      // expand: 2^wo_sh waves along the outputs of a workgroup (BO outputs each)
    int32_t accumulate;
    float out_scale;
    const int32_t *r_slot;
    const float *r_w;
    const float *s_scale;
    const float *mid_scale;
    const float *out_scale_vec;
    IdxSrc a_src, b_src;
    // Shared-input calls: the shrink's G groups are (module, route entry, rank group), module
    // m = g / G1; group g's A blocks start at a_goff[g] (a_src.block_off is 0 in the kernels).
    // The expand of one module reads mid groups [mid_goff, mid_goff + G).
    int64_t a_goff[kMaxGroups];
    int32_t G1, mid_goff;
    // Replicated shared-input shrink: n_mod_wg > 1 launches one workgroup per (token tile, module),
    // the modules of a tile on consecutive workgroup ids, so x is fetched from HBM once and the
    // other modules' reads hit the Infinity Cache. Module mod's groups start at a_goff[mod]
    // and write mid groups [mod * G, (mod + 1) * G).
    int32_t n_mod_wg;
    Luts luts;
    const void *dense_a, *dense_b;
    int64_t n_slots;
};

// Launch plan of one call (host side; the kernels read the fields copied into LoraArgs).
struct Plan {
    int G, n_rg, GM, MR;
    int GMs;    // rank groups the shrink is compiled for (GM, or exactly 3 for three groups)
    int tw;     // shrink: token groups per wave (1 or 2)
    int tiles_s, ks, pb, arow, region, red_off, stage_off;
    size_t lds_s, lds_e;
    int tiles_e, subs_e, BO, BOM, U, nblk_max, estage_off, wo_sh;
    int NS, GE;    // expand: rank groups summed per effective group (rank collapse), effective groups (power of two)
    int64_t off_mid, total;
};

// Grouped launch: one shrink grid (or one expand grid) over several jobs of one call. Workgroups
// [begin[j], begin[j + 1]) run job j; a job's fields replace those of the common LoraArgs.
// Shrink job: one x (one module, or the modules of a shared input in replicated form). Expand job:
// one module. Every job shares the routes, rank, dtypes and the index sources' bases and tables.
constexpr int kMaxJobs = 8;
struct GroupJob {
    const void *x;
    void *y;
    void *mid;
    int64_t seq, d_in, d_out, rows;
    int64_t a_goff[kMaxGroups];
    int64_t b_off;
    int32_t MR, mid_goff, n_mod_wg, xnt;
    int32_t tiles_s, ks, pb, arow, region, red_off, stage_off;
    int32_t tiles_e, subs_e, BO, vec_y, nblk_max, estage_off, wo_sh;
    float out_scale;
};
struct GroupArgs {
    LoraArgs a;                 // common fields
    GroupJob job[kMaxJobs];
    int32_t begin[kMaxJobs];    // first workgroup of each job (multiples of 8: XCD rounds stay aligned)
    int32_t n_jobs;
};

namespace {

// Slot of route entry j of sample b, or -1 (empty entry or out of range; the latter is recorded).
__device__ __forceinline__ int64_t route_slot(const LoraArgs &a, int64_t b, int j, bool record) {
    const int32_t s = a.r_slot[b * a.n_route + j];
    if (s >= 0 && (int64_t)s < a.n_slots) return s;
    if (record && s != -1) record_error(a.err, kErrSlot);
    return -1;
}

// m_t of lithe_common.h for a run-time t < 16: bit q of m_t is 1 ^ parity(t & q), and
// parity(t & q) is linear in the bits of t (bit i of t flips the q that have bit i set).
__host__ __device__ constexpr uint32_t sign_mask_rt(uint32_t t) {
    return 0x1FFu ^ (((t & 1u) ? 0xAAu : 0u) ^ ((t & 2u) ? 0xCCu : 0u) ^ ((t & 4u) ? 0xF0u : 0u) ^
                     ((t & 8u) ? 0x100u : 0u));
}
static_assert(sign_mask_rt(0) == sign_mask(0) && sign_mask_rt(5) == sign_mask(5) &&
                  sign_mask_rt(10) == sign_mask(10) && sign_mask_rt(15) == sign_mask(15),
              "linear form of the sign masks");

// Activations and outputs are touched once per call: their loads and stores carry the
// non-temporal hint, which keeps the streams from displacing the index words, the value
// tables and the rank-r intermediate in L2 and the Infinity Cache (measured on MI355X:
// +13 % read and +8 % read-modify-write bandwidth against plain accesses).
#ifndef LITHE_STREAM_NT
#define LITHE_STREAM_NT 0
#endif
template <typename V, bool FORCE_NT = false>
__device__ __forceinline__ V stream_load(const V *p) {
    if constexpr (FORCE_NT || LITHE_STREAM_NT) return __builtin_nontemporal_load(p);
    else return *p;
}
template <typename V, bool FORCE_NT = false>
__device__ __forceinline__ void stream_store(V *p, const V &v) {
    if constexpr (FORCE_NT || LITHE_STREAM_NT) __builtin_nontemporal_store(v, p);
    else *p = v;
}

// 8 values as one 16-byte bf16 vector.
template <typename XT>
__device__ __forceinline__ void store8(XT *dst, const float *v) {
    static_assert(sizeof(XT) == 2, "bf16 halves");
    bf16x8 p;
#pragma unroll
    for (int t = 0; t < 8; ++t) p[t] = (__bf16)v[t];
    *reinterpret_cast<bf16x8 *>(dst) = p;
}

template <typename XT>
__device__ __forceinline__ void store16(XT *dst, const float v[16]) {
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

// One side's value table into LDS. The table sits in the kernel arguments, so lane 0
// writes it from scalar registers: no vector load, nothing for later loads to wait behind.
__device__ __forceinline__ void stage_lut(float *lut, const float *v, int tid) {
    if (tid == 0) {
#pragma unroll
        for (int i = 0; i < kLutFloats; ++i) lut[i] = v[i];
    }
}

// ============================================================================ shrink
// Workgroup = 4 waves of one sample; each wave owns 16 tokens and 1/ks of every K piece
// (ks waves share a token group). K is cut into pieces of pb blocks, and the sample's A
// rows of a piece are decoded (dense factors: copied) into one of two LDS regions. The
// piece after next is decoded while the current one streams, so the decode's ALU work
// runs in the shadow of the activation loads and only piece 0 (and 1) sit in front of
// the stream. A fragments come from LDS (ds_read) while x streams through the vector
// memory path. Waves that split a token group's K range reduce their fp32 partials
// through LDS in a fixed order (deterministic).
// XNT: x loads carry the non-temporal hint (x is read once). The replicated shared-input form
// reads each x line from several workgroups of one XCD and keeps it in L2 instead.
// bid: the workgroup's index within this call's grid (a grouped launch passes it relative to the
// call's first workgroup); ids past the call's tiles (padding) return at once. goff: the first A
// block of each group (kMaxGroups entries in kernel-argument memory; a grouped launch passes its
// job's table, so its local copy of the arguments is only read at constant offsets and stays in
// registers).
// TW token groups per wave (16 tokens each, consecutive): every A fragment read from LDS and
// every A piece a workgroup decodes serve TW MFMAs / token groups (used with several rank groups).
template <typename XT, int SRC, int GM, int U, bool XNT, int TW = 1>
__device__ __forceinline__ void shrink_body(const LoraArgs &a, int bid, const int64_t *goff) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    constexpr bool kBf16 = sizeof(XT) == 2;
    constexpr int KSTEP = kBf16 ? 32 : 16;
    constexpr int SPB = kBlock / KSTEP;      // k-steps per 64-value block
    constexpr int EV = 16 / sizeof(XT);      // elements per 16-byte vector
    typedef typename std::conditional<kBf16, bf16x8, f32x4>::type XV;
    // Indexed bf16 factors: row r of a piece holds the first halves of its pb periods, then the
    // second halves (16-byte units), then one unit of padding. An MFMA's A fragment (lane: row r16,
    // half gq & 1 of one block) then reads without LDS bank conflicts at pieces of 16 or 48 blocks;
    // periods stored whole (half h at unit 2 c + h) conflicted 2-way on every read (measured:
    // SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE 0.5 in probes, 0.16 over the grouped FLUX sweep's
    // shrinks, 0 after; the sweep time did not change).
    constexpr bool kSplitHalves = kBf16 && SRC != SRC_DENSE;
    constexpr int FB = SRC == SRC_DENSE ? 3 : fill_batch(GM);    // dense rows: 16-byte pieces, three per thread

    const int tid = threadIdx.x;
    // wave index as a scalar: loop bounds derived from it stay uniform (SGPR) branches
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, r16 = lane & 15, gq = lane >> 4;
    const int ks = a.ks, tgw = kWaves / a.ks;
    const int tgi = wave % tgw, ksi = wave / tgw;
    // Replicated mode: workgroups are dealt round-robin to the 8 XCDs, so id w runs on XCD w % 8.
    // The modules of tile t sit at ids 8 (M (t / 8) + m) + t % 8: one XCD, consecutive in its
    // queue, sharing that XCD's L2 for x.
    int mod = 0, tile = bid;
    if (a.n_mod_wg > 1) {
        const int q = bid >> 3;
        mod = q % a.n_mod_wg;
        tile = (q / a.n_mod_wg) * 8 + (bid & 7);
    }
    if (tile >= (int)a.n_batch * a.tiles_s) return;    // padding (an XCD round, a grouped call): before any barrier
    const int64_t b = tile / a.tiles_s;
    const int mt = tile % a.tiles_s;
    const int64_t tg0 = ((int64_t)mt * tgw + tgi) * TW;    // first token group of this wave

    float *lut = reinterpret_cast<float *>(smem);
    XT *ring = reinterpret_cast<XT *>(smem + kHead);
    float *red = reinterpret_cast<float *>(smem + a.red_off);

    // Per-group slot and mixture weight. b and g are uniform, so these are scalar loads
    // (their own counter): nothing below waits behind them.
    int32_t gs[GM];
    float gw[GM];
    bool any = false;
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        const int j = ((g < a.G ? g : 0) % a.G1) / a.n_rg;
        gs[g] = g < a.G ? (int32_t)route_slot(a, b, j, false) : -1;
        gw[g] = a.r_w ? a.r_w[b * a.n_route + j] : 1.0f;
        any = any || gs[g] >= 0;
    }
    if (tid < GM && tid < a.G) route_slot(a, b, (tid % a.G1) / a.n_rg, true);   // records bad slot ids
    if (!any) return;    // no adapter on this sample: no mid row is read for it
    // gs[g] / gw[g] for a per-lane g < GM: a select chain over the (uniform) values. Passing them
    // through readfirstlane keeps the compiler from folding the chain back into an indexed load of
    // the local array, which would put the array in scratch (28-80 bytes per lane at 3-8 groups).
    auto group_slot = [&](int g) __attribute__((always_inline)) -> int32_t {
        int32_t r = gs[0];
#pragma unroll
        for (int q = 1; q < GM; ++q) r = g == q ? __builtin_amdgcn_readfirstlane(gs[q]) : r;
        return r;
    };
    auto group_weight = [&](int g) __attribute__((always_inline)) -> float {
        float r = gw[0];
#pragma unroll
        for (int q = 1; q < GM; ++q)
            r = g == q ? __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, gw[q]))) : r;
        return r;
    };
    auto group_rank0 = [&](int g) __attribute__((always_inline)) -> int {   // (g % n_rg) * 16
        int r = 0;
#pragma unroll
        for (int q = 1; q < GM; ++q) r = g == q ? (q % a.n_rg) * 16 : r;
        return r;
    };
    // module of this workgroup's A in replicated mode (uniform), a_goff[mod]
    int64_t mod_aoff = goff[0];
#pragma unroll
    for (int q = 1; q < kMaxGroups; ++q) mod_aoff = mod == q ? goff[q] : mod_aoff;
    auto group_aoff = [&](int g) __attribute__((always_inline)) -> int64_t {   // a_goff[g], branch-free
        if (a.n_mod_wg > 1) return mod_aoff;
        int64_t r = goff[0];
#pragma unroll
        for (int q = 1; q < GM; ++q) r = g == q ? goff[q] : r;
        return r;
    };
    if constexpr (SRC != SRC_DENSE) stage_lut(lut, a.luts.v[0][0], tid);

    const int nb = (int)(a.d_in / kBlock);
    const int pb = a.pb;
    const int npiece = (nb + pb - 1) / pb;
    auto piece_blocks = [&](int g) __attribute__((always_inline)) { return std::min(pb, nb - g * pb); };

    // ---- fills. Indexed: item = the 16-value period of (row gr, block c) of piece g, at
    // most FB items per thread (the plan keeps GM * 16 * pb <= FB * kThreads);
    // the index loads of a piece are issued one piece ahead of its decode.
    // item it of a piece: row gr = it % (GM*16), block c = it / (GM*16) (block-major: a shift)
    auto idx_item = [&](int g, int it, int &gr, int &c, bool &live) __attribute__((always_inline)) -> int64_t {
        gr = it % (GM * 16);     // constant divisor: a mask and a shift for power-of-two GM
        c = it / (GM * 16);
        const int grp = gr >> 4;
        const int rr = group_rank0(grp) + (gr & 15);
        live = group_slot(grp) >= 0 && rr < a.rank;
        return live ? group_aoff(grp) + (int64_t)rr * nb + (int64_t)g * pb + c : 0;
    };
    auto idx_load = [&](int g, RawIdx *dst) __attribute__((always_inline)) {
        if (g >= npiece) return;
        const int items = GM * 16 * piece_blocks(g);
        int64_t slot[FB], blk[FB];
#pragma unroll
        for (int q = 0; q < FB; ++q) {
            int gr, c;
            bool live;
            blk[q] = idx_item(g, std::min(q * kThreads + tid, items - 1), gr, c, live);
            slot[q] = live ? group_slot(gr >> 4) : 0;
        }
        load_raw<FB, SRC == SRC_PACKED, fixed_levels<SRC>()>(a.a_src, slot, blk, dst);
    };
    auto idx_store = [&](int g, const RawIdx *src) __attribute__((always_inline)) {
        if (g >= npiece) return;
        const int items = GM * 16 * piece_blocks(g);
        XT *reg = ring + (g & 1) * a.region;
#pragma unroll
        for (int q = 0; q < FB; ++q) {
            const int it = q * kThreads + tid;
            if (it >= items) break;
            int gr, c;
            bool live;
            const int64_t blk = idx_item(g, it, gr, c, live);
            uint32_t k[kMaxLevels];
            const bool ok = extract_indices<SRC == SRC_PACKED, fixed_levels<SRC>()>(a.a_src, blk, src[q], k);
            if (live && !ok) record_error(a.err, kErrIndex);
            const float w = group_weight(gr >> 4);
            float v[16];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                // unconditional lookups, then a select: no branch between the table reads
                float lo, hi;
                decode_value_pair<fixed_levels<SRC>()>(lut, a.a_src.levels, k, sign_mask(t), lo, hi);
                v[t] = live ? lo * w : 0.0f;
                v[t + 8] = live ? hi * w : 0.0f;
            }
            if constexpr (kSplitHalves) {
                // bf16: the two 8-value halves of a period sit pb units apart in the row
                store8<XT>(reg + gr * a.arow + c * 8, v);
                store8<XT>(reg + gr * a.arow + (pb + c) * 8, v + 8);
            } else {
                store16<XT>(reg + gr * a.arow + c * 16, v);
            }
            __builtin_amdgcn_sched_barrier(0);    // one item's values live at a time
        }
    };
    // Dense: 16-byte pieces of the factor rows, loaded and stored batch by batch.
    auto dense_fill = [&](int g) __attribute__((always_inline)) {
        if (g >= npiece) return;
        const int per_row = piece_blocks(g) * (kBlock / EV);
        const int items = GM * 16 * per_row;
        XT *reg = ring + (g & 1) * a.region;
        for (int base = 0; base < items; base += FB * kThreads) {
            f32x4 v[FB];
#pragma unroll
            for (int q = 0; q < FB; ++q) {
                const int it = std::min(base + q * kThreads + tid, items - 1);
                const int gr = it / per_row, c = it - gr * per_row;
                const int grp = gr >> 4, rr = (grp % a.n_rg) * 16 + (gr & 15);
                const bool live = group_slot(grp) >= 0 && rr < a.rank;
                // group_aoff: the module's A in a stacked buffer of several modules' factors
                // (grouped calls), n_slots (= n_dense) selections per factor; 0 for one module
                const int64_t off = live ? group_aoff(grp) * kBlock * a.n_slots +
                                               ((int64_t)group_slot(grp) * a.rank + rr) * a.d_in +
                                               (int64_t)g * pb * kBlock + c * EV
                                         : 0;
                v[q] = *reinterpret_cast<const f32x4 *>(static_cast<const XT *>(a.dense_a) + off);
            }
#pragma unroll
            for (int q = 0; q < FB; ++q) {
                const int it = base + q * kThreads + tid;
                if (it >= items) break;
                const int gr = it / per_row, c = it - gr * per_row;
                const int grp = gr >> 4, rr = (grp % a.n_rg) * 16 + (gr & 15);
                const bool live = group_slot(grp) >= 0 && rr < a.rank;
                *reinterpret_cast<f32x4 *>(reg + gr * a.arow + c * EV) = live ? v[q] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
    };

    // ---- this wave's k-steps: piece g contributes [g*pb*SPB + lo, g*pb*SPB + hi), cut into
    // batches of at most U steps that never straddle two pieces.
    struct Cur {
        int g, s, hi;
    };
    struct Desc {
        int g, s0, n;
    };
    auto share = [&](Cur &c) __attribute__((always_inline)) {
        const int n = piece_blocks(c.g) * SPB;
        c.s = c.g * pb * SPB + ksi * n / ks;
        c.hi = c.g * pb * SPB + (ksi + 1) * n / ks;
    };
    auto skip_empty = [&](Cur &c) __attribute__((always_inline)) {
        while (c.g < npiece && c.s >= c.hi) {
            ++c.g;
            if (c.g < npiece) share(c);
        }
    };
    auto next = [&](Cur &c) __attribute__((always_inline)) -> Desc {
        Desc d{npiece, 0, 0};
        if (c.g >= npiece) return d;
        d.g = c.g;
        d.s0 = c.s;
        d.n = std::min(U, c.hi - c.s);
        c.s += d.n;
        skip_empty(c);
        return d;
    };

    // ---- x stream. A k-step is 64 bytes of a token row (32 bf16 or 16 fp32), so a pair of
    // steps is one 128-byte line. Each load instruction covers whole lines: load (pair pi,
    // half eta) gives lane L token 8 eta + L / 8 and 16-byte chunk c = L % 8 of the pair
    // (chunk c = step 2 pi + c / 4, bytes 16 (c % 4) of it). Whole-line loads take the
    // non-temporal hint (measured: +15 % read bandwidth; split-line loads lose with it).
    // The MFMA wants lane (token r16, group gq) to hold chunk 4 sigma + gq of step 2 pi + sigma,
    // so every batch goes through a per-wave LDS staging area, one step pair (two loads, 2 KB)
    // at a time by default: 16-byte unit (pi, t, c) at pi * 128 + 8 t + (c ^ (t >> 1)), pi
    // counted inside the staged part (the XOR keeps both the writes and the reads free of bank
    // conflicts). A wave reuses its stage for the next pair after reading it (LDS accesses of
    // one wave complete in order).
    static_assert(U % 2 == 0, "x loads move pairs of k-steps");
    const int lr = lane >> 3, lc = lane & 7;
    const XT *lrow[TW][2];
#pragma unroll
    for (int tw = 0; tw < TW; ++tw)
#pragma unroll
        for (int eta = 0; eta < 2; ++eta) {
            const int64_t lm = (tg0 + tw) * 16 + 8 * eta + lr;
            lrow[tw][eta] = static_cast<const XT *>(a.x) + (b * a.seq + (lm < a.seq ? lm : a.seq - 1)) * a.d_in +
                            (lc & 3) * EV;
        }
    const XT *dummy = static_cast<const XT *>(a.x);
    constexpr int SL = kStageLoads < U ? kStageLoads : U;   // loads staged at a time
    char *stage = smem + a.stage_off + wave * (SL * 1024);
    struct Batch {
        XV x[TW][U];
    };
    auto load_batch = [&](Batch &bt, const Desc &d) __attribute__((always_inline)) {
#pragma unroll
        for (int tw = 0; tw < TW; ++tw)
#pragma unroll
            for (int j = 0; j < U; ++j) {
                const int st = 2 * (j >> 1) + (lc >> 2);    // step of this lane's chunk inside the batch
                bt.x[tw][j] = stream_load<XV, XNT>(
                    reinterpret_cast<const XV *>(st < d.n ? lrow[tw][j & 1] + (int64_t)KSTEP * (d.s0 + st) : dummy));
            }
    };
    // loads [m SL, (m + 1) SL) of token group tw of a batch (steps of the same range) pass through
    // the stage together
    auto stage_batch = [&](const Batch &bt, int tw, int m) __attribute__((always_inline)) {
        wave_lds_sync();    // the other lanes have read the stage's previous contents
#pragma unroll
        for (int j = m * SL; j < (m + 1) * SL; ++j) {
            const int t = 8 * (j & 1) + lr;
            *reinterpret_cast<XV *>(stage + (((j - m * SL) >> 1) * 128 + 8 * t + (lc ^ (t >> 1))) * 16) = bt.x[tw][j];
        }
        wave_lds_sync();    // every lane's chunks are in the stage before any lane reads them
    };
    auto staged = [&](int u, int m) __attribute__((always_inline)) -> XV {
        const int c = 4 * (u & 1) + gq;
        return *reinterpret_cast<const XV *>(stage + (((u - m * SL) >> 1) * 128 + 8 * r16 + (c ^ (r16 >> 1))) * 16);
    };
    f32x4 acc[TW][GM];
#pragma unroll
    for (int tw = 0; tw < TW; ++tw)
#pragma unroll
        for (int g = 0; g < GM; ++g) acc[tw][g] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    auto compute_chunk = [&](const Batch &bt, const Desc &d, const XT *reg, int sp, int m) __attribute__((always_inline)) {
        XV xv[TW][SL];
#pragma unroll
        for (int tw = 0; tw < TW; ++tw) {
            stage_batch(bt, tw, m);
#pragma unroll
            for (int v = 0; v < SL; ++v)
                if (m * SL + v < d.n) xv[tw][v] = staged(m * SL + v, m);
        }
        XV av[SL][GM];
#pragma unroll
        for (int v = 0; v < SL; ++v)
#pragma unroll
            for (int g = 0; g < GM; ++g) {
                const int u = m * SL + v;
                const XT *ap;
                if constexpr (SRC != SRC_DENSE)
                    ap = reg + g * 16 * a.arow + (kSplitHalves ? (((sp + u) >> 1) + (gq & 1) * pb) * 8
                                                  : kBf16 ? ((sp + u) >> 1) * 16 + 8 * (gq & 1) : ((sp + u) >> 2) * 16 + 4 * gq);
                else
                    ap = reg + g * 16 * a.arow + (sp + u) * KSTEP + (kBf16 ? 8 : 4) * gq;
                if (u < d.n) av[v][g] = *reinterpret_cast<const XV *>(ap);
            }
#pragma unroll
        for (int v = 0; v < SL; ++v) {
            if (m * SL + v >= d.n) break;
#pragma unroll
            for (int g = 0; g < GM; ++g)
#pragma unroll
                for (int tw = 0; tw < TW; ++tw) {
                    if constexpr (kBf16) {
                        acc[tw][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[v][g], xv[tw][v], acc[tw][g], 0, 0, 0);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            acc[tw][g] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[v][g][e], xv[tw][v][e], acc[tw][g], 0, 0, 0);
                    }
                }
        }
    };

    auto compute_batch = [&](const Batch &bt, const Desc &d) __attribute__((always_inline)) {
        const XT *reg = ring + (d.g & 1) * a.region + r16 * a.arow;
        const int sp = d.s0 - d.g * pb * SPB;    // step inside the piece
#pragma unroll
        for (int m = 0; m < U / SL; ++m) {
            if (m * SL >= d.n) break;
            compute_chunk(bt, d, reg, sp, m);
        }
    };

    // ---- prologue: index loads of pieces 0 and 1, then x of the first two batches; the
    // decode below waits for its own loads only (loads complete in order).
    RawIdx raw[FB];
    {
        RawIdx raw1[FB];
        if constexpr (SRC != SRC_DENSE) {
            idx_load(0, raw);
            idx_load(1, raw1);
        }
        __builtin_amdgcn_sched_barrier(0);
        Cur cur{0, 0, 0};
        share(cur);
        skip_empty(cur);
        Desc da = next(cur), db = next(cur);
        Batch ba, bb;
        load_batch(ba, da);
        load_batch(bb, db);
        if constexpr (SRC != SRC_DENSE) {
            __syncthreads();    // the value table staged by lane 0 is visible to every wave
            idx_store(0, raw);
            idx_store(1, raw1);
            idx_load(2, raw);
        } else {
            dense_fill(0);
            dense_fill(1);
        }
        __syncthreads();

        // ---- main loop. Entering piece g + 1 from g: barrier (all waves are done with piece
        // g, and piece g + 1 is complete), then piece g + 2 is filled into piece g's region.
        int pg = 0;
        auto enter = [&](int g) __attribute__((always_inline)) {
            while (pg < g) {
                __syncthreads();
                if constexpr (SRC != SRC_DENSE) {
                    idx_store(pg + 2, raw);
                    idx_load(pg + 3, raw);
                } else {
                    dense_fill(pg + 2);
                }
                ++pg;
            }
        };
        // batch i sits in ba (i even) or bb (i odd); batch i + 1 is in flight in the other (a third
        // batch in flight measured no faster on the FLUX sweeps)
        while (da.n > 0) {
            enter(da.g);
            compute_batch(ba, da);
            da = next(cur);
            load_batch(ba, da);
            __builtin_amdgcn_sched_barrier(0);    // keep the refill ahead of the next MFMAs
            if (db.n == 0) break;
            enter(db.g);
            compute_batch(bb, db);
            db = next(cur);
            load_batch(bb, db);
            __builtin_amdgcn_sched_barrier(0);
        }
        enter(npiece - 1);    // every wave passes the same npiece - 1 boundaries
    }

    // acc[tw][g][e]: token r16 of group tw, rank 4*gq + e of group g, summed over this wave's k range
    if (ks > 1) {
#pragma unroll
        for (int tw = 0; tw < TW; ++tw)
#pragma unroll
            for (int g = 0; g < GM; ++g)
                *reinterpret_cast<f32x4 *>(red + (((tw * kWaves + wave) * GM + g) * 64 + lane) * 4) = acc[tw][g];
        __syncthreads();
        if (ksi != 0) return;
#pragma unroll
        for (int tw = 0; tw < TW; ++tw)
#pragma unroll
            for (int g = 0; g < GM; ++g) {
                f32x4 sum = *reinterpret_cast<const f32x4 *>(red + (((tw * kWaves + tgi) * GM + g) * 64 + lane) * 4);
                for (int k2 = 1; k2 < ks; ++k2)
                    sum += *reinterpret_cast<const f32x4 *>(red + (((tw * kWaves + k2 * tgw + tgi) * GM + g) * 64 + lane) * 4);
                acc[tw][g] = sum;
            }
    }
    const float ms_b = a.mid_scale ? a.mid_scale[b] : 1.0f;
#pragma unroll
    for (int tw = 0; tw < TW; ++tw) {
        const int64_t m = (tg0 + tw) * 16 + r16;
        if (m >= a.seq) break;    // later groups are further out
        const int64_t row = b * a.seq + m;
#pragma unroll
        for (int g = 0; g < GM; ++g) {
            if (gs[g] < 0) continue;
            XT *dst = static_cast<XT *>(a.mid) + row * a.MR + (mod * a.G + g) * 16 + 4 * gq;
            if constexpr (kBf16) {
                bf16x4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = (__bf16)(acc[tw][g][e] * ms_b);
                *reinterpret_cast<bf16x4 *>(dst) = o;
            } else {
                *reinterpret_cast<f32x4 *>(dst) = acc[tw][g] * ms_b;
            }
        }
    }
}

template <typename XT, int SRC, int GM, int U, bool XNT, int TW = 1>
__global__ void __launch_bounds__(kThreads) shrink_kernel(LoraArgs a) {
    shrink_body<XT, SRC, GM, U, XNT, TW>(a, (int)blockIdx.x, a.a_goff);
}

// ============================================================================ expand
template <typename YT>
__device__ __forceinline__ float finish(float acc, float s, float yold, bool accumulate) {
    // `delta * scaling` and `out + delta` are two rounded operations in the reference; with fp32 y
    // nothing rounds between them, so the multiply-add must not be contracted into one fma
#pragma clang fp contract(off)
    const float d = DT<YT>::round(DT<YT>::round(acc) * s);
    return accumulate ? DT<YT>::round(yold + d) : d;
}

// y vector of 8 consecutive outputs (16 B for bf16, 32 B for fp32).
template <typename YT> struct Y8;
template <> struct Y8<__bf16> {
    bf16x8 v;
    __device__ __forceinline__ void load(const __bf16 *p) { v = stream_load(reinterpret_cast<const bf16x8 *>(p)); }
    __device__ __forceinline__ void store(__bf16 *p) const { stream_store(reinterpret_cast<bf16x8 *>(p), v); }
    __device__ __forceinline__ float get(int e) const { return (float)v[e]; }
    __device__ __forceinline__ void set(int e, float f) { v[e] = (__bf16)f; }
};
template <> struct Y8<float> {
    f32x4 lo, hi;
    __device__ __forceinline__ void load(const float *p) {
        lo = stream_load(reinterpret_cast<const f32x4 *>(p));
        hi = stream_load(reinterpret_cast<const f32x4 *>(p + 4));
    }
    __device__ __forceinline__ void store(float *p) const {
        stream_store(reinterpret_cast<f32x4 *>(p), lo);
        stream_store(reinterpret_cast<f32x4 *>(p + 4), hi);
    }
    __device__ __forceinline__ float get(int e) const { return e < 4 ? lo[e] : hi[e - 4]; }
    __device__ __forceinline__ void set(int e, float f) {
        if (e < 4) lo[e] = f;
        else hi[e - 4] = f;
    }
};

// Rank collapse (NS > 1, bf16 activations, packed or indexed factors). Every decoded 64-value
// block is four copies of one 16-value period: value p of a codebook entry is a sum over the
// generator columns q = 0..8 of H64[p][q] = (-1)^popcount(p & q), which depends on p only
// through p & 15. B row o holds ranks o * rank + r of the flat factor, so when rank is a multiple
// of 16 NS, the NS rank groups 16 (NS e) .. 16 (NS e + NS) - 1 of output o lie in one block and
// have equal B fragments: sum_g mid[g] . P = (sum_g mid[g]) . P. The expand then sums the NS mid
// fragments of each such set in fp32, splits the sum s into bf16 hi = bf16(s) and lo = bf16(s - hi)
// (|s - hi - lo| <= 2^-17 |s|) and runs one 16x16x32 MFMA on K = (hi, lo) against (P, P): GM
// counts these sets ("effective groups", each NS groups of one route), not the rank groups.
template <typename XT, typename YT, int SRC, int GM, int BOM, bool ACC, bool QUAD, int NS = 1>
__device__ __forceinline__ void expand_body(const LoraArgs &a, int bid) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    static_assert(NS == 1 || (sizeof(XT) == 2 && SRC != SRC_DENSE && QUAD), "rank collapse: bf16, indexed factors");
    // bf16 y with output tiles of whole lines: the whole-line y path (line_subtile below)
    constexpr bool LINE = sizeof(YT) == 2 && BOM % 64 == 0;
    typedef typename std::conditional<NS != 1, bf16x8, typename std::conditional<sizeof(XT) == 2, i16x4, f32x4>::type>::type Frag;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, r16 = lane & 15, gq = lane >> 4;
    // Workgroup tile: 2^wo_sh waves along the outputs (BO each) x 4 / 2^wo_sh waves along the
    // tokens (16 each per sub-tile); wave (wt, wq) takes tokens wt * 16 .. and outputs obase ..
    const int wt = wave >> a.wo_sh, wq = wave & ((1 << a.wo_sh) - 1);
    const int BOW = a.BO << a.wo_sh;                   // outputs per workgroup
    const int TPS = (kWaves >> a.wo_sh) * 16;          // tokens per sub-tile
    const int o_tiles = (int)((a.d_out + BOW - 1) / BOW);
    const int64_t obase_wg = (int64_t)(bid % o_tiles) * BOW;
    const int64_t obase = obase_wg + (int64_t)wq * a.BO;
    const int tile = bid / o_tiles;
    if (tile >= (int)a.n_batch * a.tiles_e) return;    // padding of a grouped call (before any barrier)
    const int64_t b = tile / a.tiles_e;
    const int mt = tile % a.tiles_e;
    const float s_b = a.out_scale_vec ? a.out_scale_vec[b] : a.out_scale;

    int64_t gslot[GM];
    bool any = false;
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        gslot[g] = g * NS < a.G ? route_slot(a, b, g * NS / a.n_rg, false) : -1;
        any = any || gslot[g] >= 0;
    }
    auto sub_row = [&](int sub, bool &valid) __attribute__((always_inline)) -> int64_t {
        const int64_t m = ((int64_t)mt * a.subs_e + sub) * TPS + wt * 16 + r16;
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

    constexpr int NP = BOM / 32;
    const int np = a.BO / 32;

    // Whole-line y path (bf16 y): access j of a wave's 16 x BOM tile covers token rows
    // IR (j % RB) + lane / IC and 16-byte units IC (j / RB) + lane % IC (IC units of IR rows, whole
    // 128-byte lines); lrow holds the rows of the RB row blocks of sub-tile `sub`.
    // They are issued per sub-tile, after the B tile is built. Issued earlier they cost the
    // sweep 1.8 % ahead of the B index loads (the decode waits behind them: loads complete in
    // order) and 2.6 % right behind them (the decode does not wait, but the tile's y registers
    // stay live through the decode and the barrier).
    constexpr int NJ = BOM / 32;
    constexpr int HB = kExchangeOutputs < BOM ? kExchangeOutputs : BOM;   // outputs per exchange
    constexpr int IC = kLineUnits < HB / 8 ? kLineUnits : HB / 8;
    constexpr int IR = 64 / IC, RB = 16 / IR;
    const int64_t omax = a.d_out - 8;
    auto line_rows = [&](int sub, int64_t *lrow, bool *lval) __attribute__((always_inline)) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int64_t m = ((int64_t)mt * a.subs_e + sub) * TPS + wt * 16 + IR * rb + lane / IC;
            lval[rb] = m < a.seq;
            lrow[rb] = (b * a.seq + (lval[rb] ? m : a.seq - 1)) * a.d_out;
        }
    };
    auto line_load = [&](int sub, bf16x8 *yv) __attribute__((always_inline)) {
        int64_t lrow[RB];
        bool lval[RB];
        line_rows(sub, lrow, lval);
        const __bf16 *yb = static_cast<const __bf16 *>(a.y);
#pragma unroll
        for (int j = 0; j < NJ; ++j)
            yv[j] = stream_load<bf16x8, true>(reinterpret_cast<const bf16x8 *>(
                yb + lrow[j % RB] + std::min<int64_t>(obase + 8 * (IC * (j / RB) + lane % IC), omax)));
    };

    // mid fragments; groups without an adapter read group 0 of the same row (their B
    // fragments are zero), so every lane issues the same unconditional loads.
    int gsrc[GM];
#pragma unroll
    for (int g = 0; g < GM; ++g) gsrc[g] = gslot[g] >= 0 ? g : 0;

    // Per-route B multipliers (scalar loads: b and the route are uniform). Route j's first
    // rank group is j * n_rg (effective group j * n_rg / NS).
    float gw[GM], gsc[GM];
#pragma unroll
    for (int g = 0; g < GM; ++g) {
        const int j = (g * NS < a.G ? g * NS : 0) / a.n_rg;
        gw[g] = a.r_w ? a.r_w[b * a.n_route + j] : 1.0f;
        gsc[g] = (gslot[g] >= 0 && a.s_scale) ? a.s_scale[gslot[g]] : 1.0f;
    }
    auto route_pick = [&](int j, int64_t &slot, float &w, float &sc) __attribute__((always_inline)) {
        const int g0 = j * a.n_rg;
        slot = gslot[0];
        w = gw[0];
        sc = gsc[0];
#pragma unroll
        for (int q = 1; q < GM; ++q) {
            slot = g0 == q * NS ? gslot[q] : slot;
            w = g0 == q * NS ? gw[q] : w;
            sc = g0 == q * NS ? gsc[q] : sc;
        }
    };

    // ---- B tile of this output range into LDS (bp), read from there by every MFMA.
    // Indexed: the 16-value periods of blocks [blk_lo, blk_lo + nblk) of every route entry,
    // one item per pair of quarter periods (positions 4 q .. 4 q + 3 and 4 q + 8 .. 4 q + 11, decoded
    // together: decode_value_pair), 2 items per thread per batch.
    // Dense: rows o in [obase_wg, o_end_wg) of every route entry's B, (route, o - obase_wg, rank).
    float *lut = reinterpret_cast<float *>(smem);
    XT *bp = reinterpret_cast<XT *>(smem + kHead);
    // the tile covers the workgroup's outputs [obase_wg, o_end_wg); o_end bounds this wave's
    const int64_t blk_lo = (obase_wg * a.rank) >> 6;
    const int64_t o_end_wg = std::min<int64_t>(obase_wg + BOW, a.d_out);
    const int64_t o_end = std::min<int64_t>(obase + a.BO, a.d_out);
    if constexpr (SRC != SRC_DENSE) {
        const int per_route = (int)(((o_end_wg * a.rank + kBlock - 1) >> 6) - blk_lo) * 2;
        const int items = a.n_route * per_route;
        RawIdx raw[2];
        // block of item `it` inside the factor; 0 if its route entry is empty
        auto dec_block = [&](int it, int64_t &slot, float &w, float &sc) __attribute__((always_inline)) -> int64_t {
            const int j = a.n_route == 1 ? 0 : it / per_route;
            route_pick(j, slot, w, sc);
            const int64_t blk = blk_lo + ((it - j * per_route) >> 1);
            return slot >= 0 ? blk : 0;
        };
        auto dec_load = [&](int base) __attribute__((always_inline)) {
            int64_t slot[2], blk[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                float w, sc;
                blk[q] = dec_block(std::min(base + q * kThreads + tid, items - 1), slot[q], w, sc);
                slot[q] = slot[q] >= 0 ? slot[q] : 0;
            }
            load_raw<2, SRC == SRC_PACKED, fixed_levels<SRC>()>(a.b_src, slot, blk, raw);
        };
        auto dec_store = [&](int base) __attribute__((always_inline)) {
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int it = base + q * kThreads + tid;
                if (it >= items) break;
                const int j = a.n_route == 1 ? 0 : it / per_route;
                const int rem = it - j * per_route;
                const int blk = rem >> 1, qp = rem & 1;
                int64_t slot;
                float w, sc;
                uint32_t k[kMaxLevels];
                const bool ok = extract_indices<SRC == SRC_PACKED, fixed_levels<SRC>()>(a.b_src, dec_block(it, slot, w, sc), raw[q], k);
                const bool live = slot >= 0;
                if (live && !ok) record_error(a.err, kErrIndex);
                XT *dst = bp + ((int64_t)j * a.nblk_max + blk) * 16 + 4 * qp;
                float v[8];    // positions 4 qp + e and 4 qp + 8 + e
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float lo, hi;
                    decode_value_pair<fixed_levels<SRC>()>(lut, a.b_src.levels, k, sign_mask_rt(4 * qp + e), lo, hi);
                    v[e] = live ? (lo * sc) * w : 0.0f;
                    v[4 + e] = live ? (hi * sc) * w : 0.0f;
                }
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    if constexpr (sizeof(XT) == 2) {
                        bf16x4 pk;
#pragma unroll
                        for (int e = 0; e < 4; ++e) pk[e] = (__bf16)v[4 * h + e];
                        *reinterpret_cast<bf16x4 *>(dst + 8 * h) = pk;
                    } else {
                        *reinterpret_cast<f32x4 *>(dst + 8 * h) = f32x4{v[4 * h], v[4 * h + 1], v[4 * h + 2], v[4 * h + 3]};
                    }
                }
            }
        };
        dec_load(0);
        stage_lut(lut, a.luts.v[1][0], tid);
        __syncthreads();
        dec_store(0);
        for (int base = 2 * kThreads; base < items; base += 2 * kThreads) {
            dec_load(base);
            dec_store(base);
        }
    } else {
        // 16-byte vectors of (o_end_wg - obase_wg) * rank consecutive values per route entry
        constexpr int EV = 16 / sizeof(XT);
        const int per_route = (int)((o_end_wg - obase_wg) * a.rank / EV);
        const int items = a.n_route * per_route;
        for (int it = tid; it < items; it += kThreads) {
            const int j = it / per_route, c = it - j * per_route;
            int64_t slot;
            float w, sc;
            route_pick(j, slot, w, sc);
            f32x4 v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            // b_src.block_off: the module's B in a stacked buffer (grouped calls), else 0
            if (slot >= 0)
                v = *reinterpret_cast<const f32x4 *>(static_cast<const XT *>(a.dense_b) +
                                                     a.b_src.block_off * kBlock * a.n_slots +
                                                     (slot * a.d_out + obase_wg) * a.rank + (int64_t)c * EV);
            *reinterpret_cast<f32x4 *>(bp + (int64_t)j * BOW * a.rank + (int64_t)c * EV) = v;
        }
    }
    __syncthreads();

    // ---- B fragment (p, h, g) from LDS. MFMA (p, h) row i <-> output 32p + 8(i/4) + 4h + (i%4),
    // so lane (token r16, group gq) ends with outputs 32p + 8gq .. +7 of its token. QUAD
    // (rank % 4 == 0): the 4 ranks of a fragment are 4 consecutive LDS values, one 8-byte read
    // (fp32: 16 bytes); dead fragments read a valid address and are zeroed, without branches.
    auto b_index = [&](int j, int64_t o, int r) __attribute__((always_inline)) -> int64_t {
        if constexpr (SRC != SRC_DENSE) {
            const int64_t f = o * a.rank + r;
            return ((int64_t)j * a.nblk_max + (f >> 6) - blk_lo) * 16 + (f & 15);
        } else {
            return ((int64_t)j * BOW + (o - obase_wg)) * a.rank + r;
        }
    };
    auto bfrag = [&](int p, int h, int g) __attribute__((always_inline)) -> Frag {
        const int64_t o = obase + 32 * p + 8 * (r16 >> 2) + 4 * h + (r16 & 3);
        if constexpr (NS != 1) {
            // half gq & 1 of the period of output o and effective group g (K = (P, P))
            const int gg = g * NS < a.G ? g * NS : 0;
            const bool live = p < np && gslot[g] >= 0 && o < o_end;
            const i16x8 fr = *reinterpret_cast<const i16x8 *>(
                bp + b_index(gg / a.n_rg, live ? o : obase, (gg % a.n_rg) * 16) + 8 * (gq & 1));
            return __builtin_bit_cast(Frag, live ? fr : i16x8{});
        }
        const int gg = g < a.G ? g : 0;
        const int j = gg / a.n_rg;
        const int rr = (gg % a.n_rg) * 16 + 4 * gq;
        const bool live = p < np && gslot[g] >= 0 && o < o_end && rr < a.rank;
        Frag fr;
        if constexpr (QUAD) {
            fr = *reinterpret_cast<const Frag *>(bp + b_index(j, live ? o : obase, live ? rr : 0));
            fr = live ? fr : Frag{};
        } else {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const bool le = live && rr + e < a.rank;
                const float t = DT<XT>::to_f32(bp[b_index(j, le ? o : obase, le ? rr + e : 0)]);
                v[e] = le ? t : 0.0f;
            }
            if constexpr (sizeof(XT) == 2) {
#pragma unroll
                for (int e = 0; e < 4; ++e) fr[e] = __builtin_bit_cast(short, (__bf16)v[e]);
            } else {
                fr = f32x4{v[0], v[1], v[2], v[3]};
            }
        }
        return fr;
    };
    auto compute = [&](const Frag *mf, int p, float vals[8]) __attribute__((always_inline)) {
        f32x4 acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int g = 0; g < GM; ++g) {
                // a group without an adapter contributes exact zeros (its mid slot is not written)
                const Frag bf = bfrag(p, h, g);
                if constexpr (NS != 1) {
                    const Frag m = __builtin_bit_cast(
                        Frag, gslot[g] >= 0 ? __builtin_bit_cast(i16x8, mf[g]) : i16x8{});
                    acc[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf, m, acc[h], 0, 0, 0);
                } else if constexpr (sizeof(XT) == 2) {
                    const Frag m = gslot[g] >= 0 ? mf[g] : Frag{};
                    acc[h] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bf, m, acc[h], 0, 0, 0);
                } else {
                    const Frag m = gslot[g] >= 0 ? mf[g] : Frag{};
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        acc[h] = __builtin_amdgcn_mfma_f32_16x16x4f32(bf[e], m[e], acc[h], 0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            vals[e] = acc[0][e];
            vals[4 + e] = acc[1][e];
        }
    };

    // ---- sub-tiles: 16 tokens per wave each. Every load of a sub-tile is issued up front
    // (rows and columns clamped in range); waves of other workgroups hide the latency.

    // Whole-line y path (bf16 y). The y tile of a wave (16 tokens x BOM outputs) moves in
    // loads and stores that each cover whole 128-byte lines (default: 8 token rows x 128 B per
    // access; 4 x 256 B and 2 x 512 B measured 0.3-0.5 % slower on the grouped FLUX sweep), with
    // the non-temporal hint (measured: +5 % read-modify-write bandwidth; split-line accesses lose
    // with it). The
    // delta d = round_y(round_y(acc) * s) is finished in the MFMA layout (lane: token r16,
    // outputs 32 p + 8 gq ..) and exchanged through a per-wave LDS tile, HB outputs at a time
    // (a 4 KB tile: the workgroup's LDS stays small enough for 8 workgroups per CU): 16-byte
    // unit (token t, chunk q) at (HB / 8) t + (q ^ swz(t)), conflict-free for both sides at
    // HB >= 128. A wave reuses its tile for the next half after reading it back (LDS accesses
    // of one wave complete in order).
    auto line_subtile = [&](int sub, const Frag *mf, const bf16x8 *yv) __attribute__((always_inline)) {
        __bf16 *stg = reinterpret_cast<__bf16 *>(smem + a.estage_off) + wave * 16 * HB;
        constexpr int RU = HB / 8;     // 16-byte units per token row of the tile
        auto unit = [&](int t, int q) __attribute__((always_inline)) {
            const int swz = ((t & 7) | ((((t >> 3) ^ t) & 1) << 3)) & (RU - 1);
            return stg + (RU * t + (q ^ swz)) * 8;
        };
        int64_t lrow[RB];
        bool lval[RB];
        line_rows(sub, lrow, lval);
        __bf16 *yb = static_cast<__bf16 *>(a.y);
        constexpr int PH = HB / 32;    // MFMA column groups (and y accesses) per exchange
#pragma unroll
        for (int h = 0; h < BOM / HB; ++h) {
            wave_lds_sync();    // the other lanes have read the tile's previous contents
#pragma unroll
            for (int p = h * PH; p < (h + 1) * PH; ++p) {
                if (p >= np) break;
                float vals[8];
                compute(mf, p, vals);
                bf16x8 d;
#pragma unroll
                for (int e = 0; e < 8; ++e) d[e] = (__bf16)(DT<YT>::round(vals[e]) * s_b);
                *reinterpret_cast<bf16x8 *>(unit(r16, 4 * (p - h * PH) + gq)) = d;
            }
            wave_lds_sync();    // every lane's deltas are in the tile before any lane reads them
#pragma unroll
            for (int j = h * PH; j < (h + 1) * PH; ++j) {
                const int t = IR * (j % RB) + lane / IC, q = IC * (j / RB) + lane % IC;
                const bf16x8 d = *reinterpret_cast<const bf16x8 *>(unit(t, q - h * RU));
                const int64_t o8 = obase + 8 * q;
                bf16x8 out;
                if constexpr (ACC) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) out[e] = (__bf16)((float)yv[j][e] + (float)d[e]);
                } else {
                    out = d;
                }
                if (lval[j % RB] && 8 * q < a.BO && o8 < a.d_out)
                    stream_store<bf16x8, true>(reinterpret_cast<bf16x8 *>(yb + lrow[j % RB] + o8), out);
            }
        }
    };
    // Cross-wave y path (kXWaveKernel; bf16 y, 2 waves of 256 outputs along the outputs, 32-token
    // sub-tiles): wave w reads and writes rows 8 w .. 8 w + 7 of the workgroup's 32 x 512 y tile,
    // one whole 1 KB row per access; the deltas, computed in the MFMA layout by wave (wt, wq) for
    // rows 16 wt .. and outputs 256 wq .., pass through a 32 KB LDS tile between two workgroup
    // barriers. 16-byte unit u of tile row t sits at 64 t + (u ^ (t & 15)): the MFMA-layout writes
    // (16 rows x 4 units per instruction) and the row reads are free of bank conflicts.
    // Read-modify-write probes (1 GB of 6 KB / 24 KB rows, 32 x 1 KB workgroup tiles): 6.25 / 6.47
    // TB/s with 8 whole rows per wave against 5.95-6.11 / 6.24-6.42 with 16 rows x 512 B per wave.
    // FLUX sweeps (alternating builds, one box): grouped 54.69-54.80 -> 53.94-54.01 ms, per module
    // 57.55 -> 56.41, hb 62.89 -> 62.05.
    auto xwave_subtile = [&](int sub, const Frag *mf) __attribute__((always_inline)) {
        __bf16 *tile = reinterpret_cast<__bf16 *>(smem + a.estage_off);
        auto tunit = [&](int t, int u) __attribute__((always_inline)) { return tile + (64 * t + (u ^ (t & 15))) * 8; };
        __bf16 *yb = static_cast<__bf16 *>(a.y);
        const int64_t m0 = ((int64_t)mt * a.subs_e + sub) * TPS + 8 * wave;
        const int64_t o8 = obase_wg + 8 * lane;
        const int64_t oc = std::min<int64_t>(o8, omax);
        bf16x8 yv[8];
        if constexpr (ACC) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int64_t m = m0 + i;
                yv[i] = stream_load<bf16x8, true>(reinterpret_cast<const bf16x8 *>(
                    yb + (b * a.seq + (m < a.seq ? m : a.seq - 1)) * a.d_out + oc));
            }
        }
        if (sub > 0) __syncthreads();    // every wave has read the previous sub-tile's deltas
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            float vals[8];
            compute(mf, p, vals);
            bf16x8 d;
#pragma unroll
            for (int e = 0; e < 8; ++e) d[e] = (__bf16)(DT<YT>::round(vals[e]) * s_b);
            *reinterpret_cast<bf16x8 *>(tunit(16 * wt + r16, 32 * wq + 4 * p + gq)) = d;
        }
        __syncthreads();                 // the whole tile is written
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const bf16x8 d = *reinterpret_cast<const bf16x8 *>(tunit(8 * wave + i, lane));
            bf16x8 out;
            if constexpr (ACC) {
#pragma unroll
                for (int e = 0; e < 8; ++e) out[e] = (__bf16)((float)yv[i][e] + (float)d[e]);
            } else {
                out = d;
            }
            const int64_t m = m0 + i;
            if (m < a.seq && o8 < a.d_out)
                stream_store<bf16x8, true>(reinterpret_cast<bf16x8 *>(yb + (b * a.seq + m) * a.d_out + o8), out);
        }
    };
    for (int sub = 0; sub < a.subs_e; ++sub) {
        // keeps the B fragment reads inside the loop (read from LDS per use, not held in registers)
        asm volatile("" ::: "memory");
        bool valid;
        const int64_t row = sub_row(sub, valid);
        Frag mf[GM];
#pragma unroll
        for (int g = 0; g < GM; ++g) {
            if constexpr (NS != 1) {
                // lane (token r16, gq): values 8 (gq & 1) .. + 7 of the sum of the NS groups' mid
                // fragments, its bf16 hi part (gq < 2) or lo part (gq >= 2)
                const XT *src = static_cast<const XT *>(a.mid) + row * a.MR + (a.mid_goff + gsrc[g] * NS) * 16 + 8 * (gq & 1);
                float s[8];
#pragma unroll
                for (int q = 0; q < NS; ++q) {
                    const bf16x8 v = *reinterpret_cast<const bf16x8 *>(src + q * 16);
#pragma unroll
                    for (int e = 0; e < 8; ++e) s[e] = q == 0 ? (float)v[e] : s[e] + (float)v[e];
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const __bf16 hi = (__bf16)s[e];
                    mf[g][e] = gq < 2 ? hi : (__bf16)(s[e] - (float)hi);
                }
            } else if constexpr (sizeof(XT) == 2) {
                const XT *src = static_cast<const XT *>(a.mid) + row * a.MR + (a.mid_goff + gsrc[g]) * 16 + 4 * gq;
                mf[g] = *reinterpret_cast<const i16x4 *>(src);
            } else {
                const XT *src = static_cast<const XT *>(a.mid) + row * a.MR + (a.mid_goff + gsrc[g]) * 16 + 4 * gq;
                mf[g] = *reinterpret_cast<const f32x4 *>(src);
            }
        }
        YT *yr = static_cast<YT *>(a.y) + row * a.d_out;
        if constexpr (kXWaveKernel<SRC, GM, BOM, NS> && LINE) {
            if (a.vec_y && a.wo_sh == 1 && a.BO == 256) {
                xwave_subtile(sub, mf);
                continue;
            }
        }
        if constexpr (LINE) {
            if (a.vec_y) {
                bf16x8 yv[NJ];
                if (ACC) line_load(sub, yv);
                line_subtile(sub, mf, yv);
                continue;
            }
        }
        if (a.vec_y) {
            Y8<YT> yv[NP];
            if constexpr (ACC) {
#pragma unroll
                for (int p = 0; p < NP; ++p)
                    if (p < np) yv[p].load(yr + std::min<int64_t>(obase + 32 * p + 8 * gq, omax));
            }
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                if (p >= np) break;
                float vals[8];
                compute(mf, p, vals);
                const int64_t o8 = obase + 32 * p + 8 * gq;
                Y8<YT> out;
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    out.set(e, finish<YT>(vals[e], s_b, ACC ? yv[p].get(e) : 0.0f, ACC));
                if (valid && o8 < a.d_out) out.store(yr + o8);
            }
        } else {
            // element path for d_out not a multiple of 8 (rows not 16-byte aligned)
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

// Two entry points of one body: the second asks the compiler for 4 waves per SIMD (at most
// 128 VGPRs); it is used where the body fits that budget without spilling (one rank group,
// bf16 output).
template <typename XT, typename YT, int SRC, int GM, int BOM, bool ACC, bool QUAD, int NS = 1>
__global__ void __launch_bounds__(kThreads) expand_kernel(LoraArgs a) {
    expand_body<XT, YT, SRC, GM, BOM, ACC, QUAD, NS>(a, (int)blockIdx.x);
}
template <typename XT, typename YT, int SRC, int GM, int BOM, bool ACC, bool QUAD, int NS = 1>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) expand_kernel_w4(LoraArgs a) {
    expand_body<XT, YT, SRC, GM, BOM, ACC, QUAD, NS>(a, (int)blockIdx.x);
}

#ifndef LITHE_SHARED_X_NT
#define LITHE_SHARED_X_NT 0
#endif

// U of a shrink with TW token groups per wave: the x registers of a batch stay at kShrinkU loads
template <int TW> constexpr int shrink_u() { return kShrinkU / TW >= 2 ? kShrinkU / TW : 2; }

template <typename XT, int SRC, int GM, int TW = 1>
void launch_shrink(const Plan &p, const LoraArgs &a, hipStream_t st) {
    if constexpr (SRC != SRC_DENSE && !LITHE_SHARED_X_NT) {
        if (a.n_mod_wg > 1) {    // replicated shared-input shrink: x stays in L2 for the other modules
            hipLaunchKernelGGL((shrink_kernel<XT, SRC, GM, shrink_u<TW>(), false, TW>),
                               dim3((unsigned)((a.n_batch * p.tiles_s + 7) / 8 * 8 * a.n_mod_wg)), dim3(kThreads),
                               p.lds_s, st, a);
            return;
        }
    }
    hipLaunchKernelGGL((shrink_kernel<XT, SRC, GM, shrink_u<TW>(), true, TW>),
                       dim3((unsigned)(a.n_mod_wg > 1 ? (a.n_batch * p.tiles_s + 7) / 8 * 8 * a.n_mod_wg
                                                      : a.n_batch * p.tiles_s)),
                       dim3(kThreads), p.lds_s, st, a);
}

template <typename XT, typename YT, int SRC, int GM, int BOM, int NS = 1>
void launch_expand(const Plan &p, const LoraArgs &a, hipStream_t st) {
    const int64_t bow = (int64_t)p.BO << p.wo_sh;
    dim3 ge((unsigned)(((a.d_out + bow - 1) / bow) * a.n_batch * p.tiles_e));
    if constexpr (NS != 1) {    // rank % 32 == 0: whole 4-rank fragments
        if constexpr (GM == 1 && sizeof(YT) == 2) {
            if (a.accumulate) hipLaunchKernelGGL((expand_kernel_w4<XT, YT, SRC, GM, BOM, true, true, NS>), ge, dim3(kThreads), p.lds_e, st, a);
            else hipLaunchKernelGGL((expand_kernel_w4<XT, YT, SRC, GM, BOM, false, true, NS>), ge, dim3(kThreads), p.lds_e, st, a);
        } else {
            if (a.accumulate) hipLaunchKernelGGL((expand_kernel<XT, YT, SRC, GM, BOM, true, true, NS>), ge, dim3(kThreads), p.lds_e, st, a);
            else hipLaunchKernelGGL((expand_kernel<XT, YT, SRC, GM, BOM, false, true, NS>), ge, dim3(kThreads), p.lds_e, st, a);
        }
        return;
    }
    const bool quad = (a.rank & 3) == 0;
    if constexpr (GM == 1 && sizeof(YT) == 2) {
        if (quad) {
            if (a.accumulate)
                hipLaunchKernelGGL((expand_kernel_w4<XT, YT, SRC, GM, BOM, true, true>), ge, dim3(kThreads), p.lds_e, st, a);
            else
                hipLaunchKernelGGL((expand_kernel_w4<XT, YT, SRC, GM, BOM, false, true>), ge, dim3(kThreads), p.lds_e, st, a);
            return;
        }
    }
    if (a.accumulate) {
        if (quad) hipLaunchKernelGGL((expand_kernel<XT, YT, SRC, GM, BOM, true, true>), ge, dim3(kThreads), p.lds_e, st, a);
        else hipLaunchKernelGGL((expand_kernel<XT, YT, SRC, GM, BOM, true, false>), ge, dim3(kThreads), p.lds_e, st, a);
    } else {
        if (quad) hipLaunchKernelGGL((expand_kernel<XT, YT, SRC, GM, BOM, false, true>), ge, dim3(kThreads), p.lds_e, st, a);
        else hipLaunchKernelGGL((expand_kernel<XT, YT, SRC, GM, BOM, false, false>), ge, dim3(kThreads), p.lds_e, st, a);
    }
}

// Job of workgroup `bid` of a grouped launch (scalar compares over the job table).
__device__ __forceinline__ int group_job(const GroupArgs &g, int bid) {
    int j = 0;
#pragma unroll
    for (int q = 1; q < kMaxJobs; ++q) j += (q < g.n_jobs && bid >= g.begin[q]) ? 1 : 0;
    return j;
}

__host__ __device__ __forceinline__ void apply_job(LoraArgs &a, const GroupJob &j) {
    a.x = j.x;
    a.y = j.y;
    a.mid = j.mid;
    a.seq = j.seq;
    a.d_in = j.d_in;
    a.d_out = j.d_out;
    a.rows = j.rows;
    a.b_src.block_off = j.b_off;
    a.MR = j.MR;
    a.mid_goff = j.mid_goff;
    a.n_mod_wg = j.n_mod_wg;
    a.tiles_s = j.tiles_s;
    a.ks = j.ks;
    a.pb = j.pb;
    a.arow = j.arow;
    a.region = j.region;
    a.red_off = j.red_off;
    a.stage_off = j.stage_off;
    a.tiles_e = j.tiles_e;
    a.subs_e = j.subs_e;
    a.BO = j.BO;
    a.vec_y = j.vec_y;
    a.nblk_max = j.nblk_max;
    a.estage_off = j.estage_off;
    a.wo_sh = j.wo_sh;
    a.out_scale = j.out_scale;
}

// The x loads of a job take the non-temporal hint unless the job is a replicated shared input
// (its modules' workgroups read each x line from L2); the choice is uniform per workgroup.
template <typename XT, int SRC, int GM, int U, int TW = 1>
__global__ void __launch_bounds__(kThreads) shrink_group_kernel(GroupArgs g) {
    const int bid = (int)blockIdx.x;
    const int j = group_job(g, bid);
    LoraArgs a = g.a;
    apply_job(a, g.job[j]);
    if (g.job[j].xnt) shrink_body<XT, SRC, GM, U, true, TW>(a, bid - g.begin[j], g.job[j].a_goff);
    else shrink_body<XT, SRC, GM, U, false, TW>(a, bid - g.begin[j], g.job[j].a_goff);
}

template <typename XT, typename YT, int SRC, int GM, int BOM, bool ACC, bool QUAD, int NS>
__device__ __forceinline__ void expand_group_body(const GroupArgs &g) {
    const int bid = (int)blockIdx.x;
    const int j = group_job(g, bid);
    LoraArgs a = g.a;
    apply_job(a, g.job[j]);
    expand_body<XT, YT, SRC, GM, BOM, ACC, QUAD, NS>(a, bid - g.begin[j]);
}
template <typename XT, typename YT, int SRC, int GM, int BOM, bool ACC, bool QUAD, int NS = 1>
__global__ void __launch_bounds__(kThreads) expand_group_kernel(GroupArgs g) {
    expand_group_body<XT, YT, SRC, GM, BOM, ACC, QUAD, NS>(g);
}
template <typename XT, typename YT, int SRC, int GM, int BOM, bool ACC, bool QUAD, int NS = 1>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) expand_group_kernel_w4(GroupArgs g) {
    expand_group_body<XT, YT, SRC, GM, BOM, ACC, QUAD, NS>(g);
}

template <typename XT, int SRC, int GM, int TW = 1>
void launch_shrink_group(const GroupArgs &g, unsigned grid, size_t lds, hipStream_t st) {
    hipLaunchKernelGGL((shrink_group_kernel<XT, SRC, GM, shrink_u<TW>(), TW>), dim3(grid), dim3(kThreads), lds, st, g);
}

template <typename XT, typename YT, int SRC, int GM, int BOM, int NS = 1>
void launch_expand_group(const GroupArgs &g, unsigned grid, size_t lds, hipStream_t st) {
    const dim3 ge(grid);
    if constexpr (NS != 1) {    // rank % 32 == 0: whole 4-rank fragments
        if constexpr (GM == 1 && sizeof(YT) == 2) {
            if (g.a.accumulate) hipLaunchKernelGGL((expand_group_kernel_w4<XT, YT, SRC, GM, BOM, true, true, NS>), ge, dim3(kThreads), lds, st, g);
            else hipLaunchKernelGGL((expand_group_kernel_w4<XT, YT, SRC, GM, BOM, false, true, NS>), ge, dim3(kThreads), lds, st, g);
        } else {
            if (g.a.accumulate) hipLaunchKernelGGL((expand_group_kernel<XT, YT, SRC, GM, BOM, true, true, NS>), ge, dim3(kThreads), lds, st, g);
            else hipLaunchKernelGGL((expand_group_kernel<XT, YT, SRC, GM, BOM, false, true, NS>), ge, dim3(kThreads), lds, st, g);
        }
        return;
    }
    const bool quad = (g.a.rank & 3) == 0;
    if constexpr (GM == 1 && sizeof(YT) == 2) {
        if (quad) {
            if (g.a.accumulate)
                hipLaunchKernelGGL((expand_group_kernel_w4<XT, YT, SRC, GM, BOM, true, true>), ge, dim3(kThreads), lds, st, g);
            else
                hipLaunchKernelGGL((expand_group_kernel_w4<XT, YT, SRC, GM, BOM, false, true>), ge, dim3(kThreads), lds, st, g);
            return;
        }
    }
    if (g.a.accumulate) {
        if (quad) hipLaunchKernelGGL((expand_group_kernel<XT, YT, SRC, GM, BOM, true, true>), ge, dim3(kThreads), lds, st, g);
        else hipLaunchKernelGGL((expand_group_kernel<XT, YT, SRC, GM, BOM, true, false>), ge, dim3(kThreads), lds, st, g);
    } else {
        if (quad) hipLaunchKernelGGL((expand_group_kernel<XT, YT, SRC, GM, BOM, false, true>), ge, dim3(kThreads), lds, st, g);
        else hipLaunchKernelGGL((expand_group_kernel<XT, YT, SRC, GM, BOM, false, false>), ge, dim3(kThreads), lds, st, g);
    }
}

// TW: token groups per wave (2 only with several rank groups).
template <typename XT, int SRC>
void dispatch_shrink_group(int GM, int TW, const GroupArgs &g, unsigned grid, size_t lds, hipStream_t st) {
    if constexpr (SRC == SRC_DENSE) {    // dense factors: one token group per wave, no 3-group kernel
        switch (GM) {
            case 1: launch_shrink_group<XT, SRC, 1>(g, grid, lds, st); break;
            case 2: launch_shrink_group<XT, SRC, 2>(g, grid, lds, st); break;
            case 4: launch_shrink_group<XT, SRC, 4>(g, grid, lds, st); break;
            default: launch_shrink_group<XT, SRC, 8>(g, grid, lds, st); break;
        }
    } else {
        if (TW == 2) {
            switch (GM) {
                case 2: launch_shrink_group<XT, SRC, 2, 2>(g, grid, lds, st); break;
                case 3: launch_shrink_group<XT, SRC, 3, 2>(g, grid, lds, st); break;
                case 4: launch_shrink_group<XT, SRC, 4, 2>(g, grid, lds, st); break;
                default: launch_shrink_group<XT, SRC, 8, 2>(g, grid, lds, st); break;
            }
            return;
        }
        switch (GM) {
            case 1: launch_shrink_group<XT, SRC, 1>(g, grid, lds, st); break;
            case 2: launch_shrink_group<XT, SRC, 2>(g, grid, lds, st); break;
            case 3: launch_shrink_group<XT, SRC, 3>(g, grid, lds, st); break;
            case 4: launch_shrink_group<XT, SRC, 4>(g, grid, lds, st); break;
            default: launch_shrink_group<XT, SRC, 8>(g, grid, lds, st); break;
        }
    }
}

// BOM as in dispatch_expand (bf16 activations); GM counts effective groups of NS rank groups.
template <typename XT, typename YT, int SRC>
void dispatch_expand_group(int GM, int BOM, int NS, const GroupArgs &g, unsigned grid, size_t lds, hipStream_t st) {
    if constexpr (SRC == SRC_DENSE) {    // dense factors: no rank collapse, 256 outputs per wave at one group
        switch (GM) {
            case 1: launch_expand_group<XT, YT, SRC, 1, 256>(g, grid, lds, st); break;
            case 2: launch_expand_group<XT, YT, SRC, 2, 256>(g, grid, lds, st); break;
            case 4: launch_expand_group<XT, YT, SRC, 4, 128>(g, grid, lds, st); break;
            default: launch_expand_group<XT, YT, SRC, 8, 64>(g, grid, lds, st); break;
        }
    } else {
        if (NS == 4) {
            if (GM == 1) launch_expand_group<XT, YT, SRC, 1, 256, 4>(g, grid, lds, st);
            else launch_expand_group<XT, YT, SRC, 2, 256, 4>(g, grid, lds, st);
            return;
        }
        if (NS == 2) {
            if (GM == 1) launch_expand_group<XT, YT, SRC, 1, 256, 2>(g, grid, lds, st);
            else if (GM == 2) launch_expand_group<XT, YT, SRC, 2, 256, 2>(g, grid, lds, st);
            else launch_expand_group<XT, YT, SRC, 4, 128, 2>(g, grid, lds, st);
            return;
        }
        switch (GM) {
            case 1:
                if (BOM == 256) launch_expand_group<XT, YT, SRC, 1, 256>(g, grid, lds, st);
                else launch_expand_group<XT, YT, SRC, 1, 128>(g, grid, lds, st);
                break;
            case 2: launch_expand_group<XT, YT, SRC, 2, 256>(g, grid, lds, st); break;
            case 4: launch_expand_group<XT, YT, SRC, 4, 128>(g, grid, lds, st); break;
            default: launch_expand_group<XT, YT, SRC, 8, 64>(g, grid, lds, st); break;
        }
    }
}

template <typename XT, int SRC>
void dispatch_shrink(const Plan &p, const LoraArgs &a, hipStream_t st) {
    if constexpr (SRC != SRC_DENSE && sizeof(XT) == 2) {
        if (p.tw == 2) {
            switch (p.GMs) {
                case 2: launch_shrink<XT, SRC, 2, 2>(p, a, st); break;
                case 3: launch_shrink<XT, SRC, 3, 2>(p, a, st); break;
                case 4: launch_shrink<XT, SRC, 4, 2>(p, a, st); break;
                default: launch_shrink<XT, SRC, 8, 2>(p, a, st); break;
            }
            return;
        }
    }
    switch (p.GMs) {
        case 1: launch_shrink<XT, SRC, 1>(p, a, st); break;
        case 2: launch_shrink<XT, SRC, 2>(p, a, st); break;
        case 3: launch_shrink<XT, SRC, 3>(p, a, st); break;
        case 4: launch_shrink<XT, SRC, 4>(p, a, st); break;
        default: launch_shrink<XT, SRC, 8>(p, a, st); break;
    }
}

// expand output tiles: BOM outputs per workgroup (make_plan's bo_max for the same GM)
template <typename XT, typename YT, int SRC>
void dispatch_expand(const Plan &p, const LoraArgs &a, hipStream_t st) {
    constexpr bool bf = sizeof(XT) == 2;
    if constexpr (bf && SRC != SRC_DENSE) {
        if (p.NS == 4) {
            if (p.GE == 1) launch_expand<XT, YT, SRC, 1, 256, 4>(p, a, st);
            else launch_expand<XT, YT, SRC, 2, 256, 4>(p, a, st);
            return;
        }
        if (p.NS == 2) {
            if (p.GE == 1) launch_expand<XT, YT, SRC, 1, 256, 2>(p, a, st);
            else if (p.GE == 2) launch_expand<XT, YT, SRC, 2, 256, 2>(p, a, st);
            else launch_expand<XT, YT, SRC, 4, 128, 2>(p, a, st);
            return;
        }
    }
    switch (p.GE) {
        case 1:
            if (bf && p.BOM == 256) launch_expand<XT, YT, SRC, 1, 256>(p, a, st);
            else launch_expand<XT, YT, SRC, 1, 128>(p, a, st);
            break;
        case 2: launch_expand<XT, YT, SRC, 2, bf ? 256 : 128>(p, a, st); break;
        case 4: launch_expand<XT, YT, SRC, 4, bf ? 128 : 64>(p, a, st); break;
        default: launch_expand<XT, YT, SRC, 8, bf ? 64 : 32>(p, a, st); break;
    }
}

}  // namespace

// Launchers of one activation / output dtype pair, each compiled in a translation unit of its own
// (lora_shrink_*.hip, lora_expand_*.hip) so the kernel variants build in parallel.
void launch_shrink_bf16(const Plan &p, const LoraArgs &a, int src, hipStream_t st);
void launch_shrink_f32(const Plan &p, const LoraArgs &a, int src, hipStream_t st);
void launch_expand_bf16_bf16(const Plan &p, const LoraArgs &a, int src, hipStream_t st);
void launch_expand_bf16_f32(const Plan &p, const LoraArgs &a, int src, hipStream_t st);
void launch_expand_f32_bf16(const Plan &p, const LoraArgs &a, int src, hipStream_t st);
void launch_expand_f32_f32(const Plan &p, const LoraArgs &a, int src, hipStream_t st);
// Grouped launches (bf16 activations and outputs, packed 3-level factors); false if the call has
// no grouped kernel (the caller then launches job by job).
bool launch_shrink_group_bf16(int GM, int TW, const GroupArgs &g, unsigned grid, size_t lds, int src, hipStream_t st);
bool launch_expand_group_bf16_bf16(int GM, int BOM, int NS, const GroupArgs &g, unsigned grid, size_t lds, int src,
                                   hipStream_t st);

}  // namespace lithe
