// Host side of the per-sample LoRA delta: plans, argument checks and the C entry points
// (lithe_lora_workspace_bytes, lithe_lora_delta, lithe_lora_delta_noalloc, lithe_lora_delta_shared_x,
// lithe_workspace_errors). The kernels are in lora_kernels.h.
#include <atomic>
#include <mutex>

#include "lora_kernels.h"

// Static scratch of lithe_lora_delta_noalloc: the rank-r intermediate of one call. Every GPU the
// library runs on holds its own copy until the process ends. In host code `scratch` only names the
// symbol; its device address comes from hipGetSymbolAddress (static_scratch() below).
static __device__ __align__(256) char scratch[LITHE_STATIC_SCRATCH_BYTES];

namespace lithe {
namespace {

// ============================================================================ host plan
int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    if (!v || !*v) return dflt;
    const int x = atoi(v);
    return x > 0 ? x : dflt;
}


int64_t align256(int64_t v) { return (v + 255) & ~int64_t(255); }

// Shrink form of modules that read one input (n_mod modules of G1 rank groups each, `groups`
// 16-token groups over the launch). Stacked: one workgroup per token tile carries every module's
// rank groups, so x is staged once and each x fragment meets every module's A fragments.
// Replicated: one single-module workgroup per (tile, module), x shared through L2. With two token
// groups per wave the stacked form wins where its grid needs no K split (q / k / v sweep, one call
// per module: 51.50 -> 50.43 ms; the 4,096-token calls 5.41 -> 5.70 TB/s) and loses on small grids
// (512 tokens: 112 workgroups, 3.29 -> 2.72 TB/s). The caller checks n_mod * G1 <= kMaxGroups.
// LITHE_SHARED_X_STACKED=1 / 0 forces either form.
bool stack_shared(int64_t groups, int n_mod, int G1, int xbytes) {
    if (const char *v = getenv("LITHE_SHARED_X_STACKED")) return atoi(v) != 0;
    return xbytes == 2 && n_mod > 1 && n_mod * G1 <= kMaxGroups && groups >= 2048;
}

// Launch context of a grouped call: the plan rules that depend on the grid's size (the shrink's K
// split, the expand's sub-tiles) see the whole grid of the launch, not one job.
struct PlanCtx {
    int64_t groups;     // 16-token groups of every shrink job of the launch
};

Plan make_plan(int64_t n_batch, int64_t seq, int64_t d_in, int64_t d_out, int rank, int n_route, int xbytes,
               bool dense, int ybytes = 2, const PlanCtx *ctx = nullptr) {
    Plan p{};
    p.n_rg = (rank + 15) / 16;
    p.G = p.n_rg * n_route;
    p.GM = p.G <= 1 ? 1 : p.G <= 2 ? 2 : p.G <= 4 ? 4 : 8;
    // the shrink is also compiled for exactly three groups (a 3-entry mixture, q / k / v stacked):
    // a quarter less MFMA and A-fragment work than padding to four
    p.GMs = p.G == 3 && !dense ? 3 : p.GM;
    p.MR = p.G * 16;
    const int64_t rows = n_batch * seq;
    const int target = env_int("LITHE_TARGET_WAVES", 2048);

    // shrink token groups per wave: with several rank groups (bf16, packed or indexed factors)
    // each wave takes two 16-token groups, which share its A fragment reads and the workgroup's
    // A decode. LITHE_SHRINK_TW=1 / 2 overrides.
    p.tw = (xbytes == 2 && !dense && p.GMs >= 2) ? 2 : 1;
    if (const char *v = getenv("LITHE_SHRINK_TW")) p.tw = (atoi(v) == 2 && xbytes == 2 && !dense && p.GMs >= 2) ? 2 : 1;

    // shrink: one wave per 16 tw tokens x (K / ks); ks grows until there are enough waves.
    const int64_t groups = ctx ? ctx->groups : n_batch * ((seq + 15) / 16);
    int ks = 1;
    // long K: shorter per-wave streams; with 4 or 8 rank groups a 4-way split costs more in
    // LDS reads than it gains (measured on the q/k/v shared-input shapes)
    const int ks_max = p.GM >= 4 ? 2 : 4;
    if (p.tw == 1) {
        while (ks < ks_max && (groups * ks < target || d_in / ks > 6144)) ks *= 2;
    } else {
        // Two token groups per wave: a K split halves the tokens that share each A piece; grouped
        // FLUX sweeps at ranks 32 / 48 / 64 / 96 / 128 ran 58.7 / 79.1 / 64.0 / 114.6 / 86.0 ms
        // with no split (the 12,288-input projections included) against 60.2 / 82.4 / 72.0 /
        // 135.2 / 107.4 with the one-group rule. Split only below 1,024 waves.
        while (ks < ks_max && groups * ks / 2 < target / 2) ks *= 2;
    }
    if (getenv("LITHE_SHRINK_KS")) {
        const int v = env_int("LITHE_SHRINK_KS", ks);
        ks = v >= 4 ? 4 : v >= 2 ? 2 : 1;
    }
    p.ks = ks;
    const int tgw = kWaves / ks;
    p.tiles_s = (int)std::max<int64_t>(1, (seq + 16 * tgw * p.tw - 1) / (16 * tgw * p.tw));
    // Ring of two LDS regions, each holding the GM*16 factor rows of one K piece of pb blocks:
    // periods (16 values per block; the plan keeps a piece's items within one fill batch) or
    // dense rows (64 values per block). Every piece boundary is a workgroup barrier, so pieces
    // are as long as the fill batch allows; a factor that fits one piece gets one region.
    const int pad = 16 / xbytes;
    if (dense) {
        // dense rows are 4x the LDS of periods: 4-block pieces with whole-K waves, 12 when K is
        // split over 4 waves (measured over the FLUX shapes)
        p.pb = std::max(1, (ks >= 4 ? 12 : 4) / p.GM);
        p.arow = p.pb * kBlock + pad;
    } else {
        // Pieces as long as one fill batch allows: 16 blocks for one rank group (one item per
        // thread; its registers matter more than the barriers of shorter pieces), up to 48 with
        // K split over 4 waves and more groups (fewer barriers), 16 with whole-K waves (the LDS of
        // a longer piece costs a workgroup of occupancy; measured over the FLUX shapes).
        // Three groups: 8-block pieces keep the ring at 26 KB (4 workgroups per CU). Whole-K waves
        // with two token groups each (half the workgroups) take 16-block pieces: the stacked
        // q / k / v shrink at 4,096 tokens 5.69 -> 5.72 TB/s. (A K split keeps 8: its partition of K
        // follows the piece size, and both token-group forms then give the same sums.)
        p.pb = std::max(1, std::min(ks >= 4 ? 48 : 16, fill_batch(p.GMs) * kThreads / (p.GMs * 16)));
        if (p.GMs == 3 && (p.tw == 1 || ks > 1)) p.pb = std::min(8, fill_batch(3) * kThreads / (3 * 16));
        p.arow = p.pb * 16 + pad;
    }
    if (getenv("LITHE_SHRINK_PB")) {
        p.pb = std::max(1, std::min(env_int("LITHE_SHRINK_PB", p.pb), fill_batch(p.GMs) * kThreads / (p.GMs * 16)));
        p.arow = p.pb * (dense ? kBlock : 16) + pad;
    }
    p.region = p.GMs * 16 * p.arow;
    const int64_t npiece = (d_in / kBlock + p.pb - 1) / p.pb;
    p.red_off = kHead + (npiece > 1 ? 2 : 1) * p.region * xbytes;
    p.stage_off = p.red_off + (ks > 1 ? kWaves * p.GMs * 64 * 16 * p.tw : 0);
    p.lds_s = p.stage_off + (size_t)kWaves * std::min(kStageLoads, kShrinkU) * 1024;

    // expand rank collapse (bf16 activations, packed or indexed factors): the NS rank groups of an
    // output that share one 64-value factor block are summed before the MFMA (expand_body);
    // rank 64 / 128: sets of 4, rank 32 / 96: pairs. LITHE_EXPAND_NS=1 turns it off.
    p.NS = 1;
    if (xbytes == 2 && !dense && rank % 32 == 0) p.NS = rank % 64 == 0 ? 4 : 2;
    if (const char *v = getenv("LITHE_EXPAND_NS"))
        if (atoi(v) == 1) p.NS = 1;
    const int ge = p.G / p.NS;
    p.GE = ge <= 1 ? 1 : ge <= 2 ? 2 : ge <= 4 ? 4 : 8;

    // expand: a wave computes BO outputs x 16 tokens per sub-tile (the workgroup's layout below).
    int bo_max = xbytes == 2 ? std::min(256, 512 / p.GE) : std::min(128, 256 / p.GE);
    bo_max = std::max(32, bo_max);
    if (getenv("LITHE_EXPAND_BO") && xbytes == 2 && p.GE == 1 && p.NS == 1 && !dense)
        bo_max = env_int("LITHE_EXPAND_BO", bo_max) == 128 ? 128 : 256;
    p.U = 4;
    p.BOM = bo_max;
    p.BO = (int)std::min<int64_t>(bo_max, ((d_out + 31) / 32) * 32);
    const int64_t o_tiles = (d_out + p.BO - 1) / p.BO;
    const int64_t base_wgs = n_batch * ((seq + 63) / 64) * o_tiles;
    // Waves along the outputs of a workgroup (2^wo_sh of them, BO outputs each; the others along
    // the tokens): a workgroup's y tile is 64 / 2^wo_sh token rows x 2^wo_sh * BO outputs. bf16 y
    // takes two: read-modify-write probes (1 GB of 6 KB / 24 KB rows) moved 64-row x 256 B tiles
    // at 5.53 / 5.60 TB/s, 64 x 512 B at 5.78 / 5.82, 32 x 512 B at 5.79-6.05 / 6.07-6.19, 32 x 1 KB
    // at 5.95-6.09 / 6.26-6.42, 2 KB-wide tiles at 5.5-5.8. On the FLUX sweeps (one box): grouped
    // 57.7 -> 54.9 ms, per module 59.7 -> 58.1 ms with 256-output waves two along the outputs
    // (32 x 1 KB tiles); 128-output waves two along the outputs (the former rule for grids under
    // 14,336 workgroups) 0.1-0.4 % slower, four along the outputs 1-2 % slower.
    // Dense factors too (decoded-mode sweep 62.5 -> 60.6 ms; their B tile is 16 KB at rank 16).
    int wo = ybytes == 2 ? 2 : 1;
    if (getenv("LITHE_EXPAND_WO")) {
        const int v = env_int("LITHE_EXPAND_WO", 1);
        wo = v >= 4 ? 4 : v >= 2 ? 2 : 1;
    }
    while (wo > 1 && (int64_t)wo * p.BO > ((d_out + 31) / 32) * 32) wo >>= 1;
    p.wo_sh = wo == 4 ? 2 : wo == 2 ? 1 : 0;
    // One rank group: 2 sub-tiles per workgroup only for mid-sized grids with one wave along the
    // outputs (fp32 y); everywhere else one sub-tile (more, shorter workgroups) measured faster,
    // and with two waves along the outputs one sub-tile was faster on every FLUX sweep.
    int subs = (base_wgs >= 4 * 256 && base_wgs < 16 * 256 && !ctx && wo == 1) ? 2 : 1;
    // Several rank groups: the B tile a workgroup builds (n_route * rank / 2 bytes of periods per
    // output) grows with the groups, its y tile (64 bytes per output and sub-tile) does not, so
    // more tokens per workgroup amortize it: the tile ratio is G / 8. Grouped FLUX sweeps (bf16,
    // packed, rank collapse): rank 32 63.3 -> 60.6 ms and rank 64 83.0 -> 73.9 ms with 2 sub-tiles
    // (4: slower), rank 128 142.1 -> 127.5 ms with 4 and (with the two-token-group shrink)
    // 86.2 -> 81.8 ms with 8 rather than 4. Without the collapse (one MFMA per rank group) rank 32
    // was best at 2 (72.2 -> 60.8 ms), rank 64 at 4 to 8 (130.6 -> 83.3 / 80.7 ms).
    // A grouped launch's grid is the sum of its jobs: its short (512-token) jobs take the rule too.
    if (p.G >= 2) {
        const int sg = p.G >= 8 ? 8 : (p.G >= 4 && p.NS == 1) ? 4 : 2;
        if (ctx || base_wgs >= (int64_t)sg * 1024) subs = std::max(subs, sg);
    }
    if (getenv("LITHE_EXPAND_SUBS")) subs = env_int("LITHE_EXPAND_SUBS", subs);
    p.subs_e = subs;
    const int64_t tps = 64 / wo;     // tokens per sub-tile
    p.tiles_e = (int)std::max<int64_t>(1, (seq + tps * subs - 1) / (tps * subs));
    // B periods of one workgroup's outputs: the blocks covering [obase, obase + wo * BO) of a route
    p.nblk_max = (int)(((int64_t)wo * p.BO * rank + kBlock - 1) / kBlock + 1);
    p.lds_e = kHead + (dense ? (size_t)n_route * wo * p.BO * rank * xbytes : (size_t)n_route * p.nblk_max * 16 * xbytes);
    // whole-line y path (bf16 y, output tiles of whole lines): a 16 x BOM bf16 tile per wave
    p.estage_off = (int)((p.lds_e + 15) & ~size_t(15));
    if (ybytes == 2 && p.BOM % 64 == 0)
        p.lds_e = p.estage_off + (size_t)kWaves * 16 * std::min(p.BOM, kExchangeOutputs) * 2;
    if (kXWave && !dense && ybytes == 2 && p.GE == 1 && p.NS == 1 && p.BOM == 256 && p.BO == 256 && p.wo_sh == 1)    // the cross-wave delta tile
        p.lds_e = p.estage_off + (size_t)std::max(kXWaveBytes, kWaves * 16 * kExchangeOutputs * 2);

    // workspace: [error word | mid]
    p.off_mid = 256;
    p.total = align256(p.off_mid + rows * p.MR * xbytes);
    return p;
}

// The grouped kernels are compiled for bf16 activations and outputs with packed 3-level factors.
bool launch_shrink_group_bf16_ok(int x_dtype, int y_dtype, int src) {
    return x_dtype == LITHE_DT_BF16 && y_dtype == LITHE_DT_BF16 && (src == SRC_PACKED || src == SRC_DENSE);
}

int src_of(const LoraArgs &a, int kind) {
    if (kind == LITHE_FACTOR_DENSE) return SRC_DENSE;
    if (a.a_src.kind == LITHE_IDX_PACKED9 && a.b_src.kind == LITHE_IDX_PACKED9 && a.a_src.levels == kPackedLevels)
        return SRC_PACKED;
    return SRC_INDEXED;
}

void launch_typed(bool shrink, int x_dtype, int y_dtype, const Plan &p, const LoraArgs &a, int src, hipStream_t st) {
    const bool xb = x_dtype == LITHE_DT_BF16, yb = y_dtype == LITHE_DT_BF16;
    if (shrink) {
        if (xb) launch_shrink_bf16(p, a, src, st);
        else launch_shrink_f32(p, a, src, st);
    } else if (xb) {
        if (yb) launch_expand_bf16_bf16(p, a, src, st);
        else launch_expand_bf16_f32(p, a, src, st);
    } else {
        if (yb) launch_expand_f32_bf16(p, a, src, st);
        else launch_expand_f32_f32(p, a, src, st);
    }
}

// Copies a plan's shrink fields into the kernel arguments.
void set_shrink_fields(LoraArgs &a, const Plan &p) {
    a.G = p.G;
    a.n_rg = p.n_rg;
    a.MR = p.MR;
    a.tiles_s = p.tiles_s;
    a.ks = p.ks;
    a.pb = p.pb;
    a.arow = p.arow;
    a.region = p.region;
    a.red_off = p.red_off;
    a.stage_off = p.stage_off;
}

// Copies a plan's expand fields into the kernel arguments.
void set_expand_fields(LoraArgs &a, const Plan &p) {
    a.tiles_e = p.tiles_e;
    a.subs_e = p.subs_e;
    a.BO = p.BO;
    a.nblk_max = p.nblk_max;
    a.estage_off = p.estage_off;
    a.wo_sh = p.wo_sh;
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
    return make_plan(n_batch, seq, d_in, d_out, rank, n_route, x_dtype == LITHE_DT_BF16 ? 2 : 4, false).total;
}

namespace lithe {
namespace {

// Checks shared by the delta entry points (sizes, dtypes, alignment of x and of the workspace; a call
// on the static scratch has no workspace to check).
int32_t check_call(const void *x, int32_t x_dtype, int64_t n_batch, int64_t seq, int64_t d_in, int32_t y_dtype,
                   int32_t rank, const lithe_routes *routes, int groups_per_module, int n_mod, const void *workspace,
                   bool static_scratch = false) {
    if (!routes) return LITHE_ERR_NULL;
    if (x_dtype != LITHE_DT_BF16 && x_dtype != LITHE_DT_F32) return LITHE_ERR_DTYPE;
    if (y_dtype != LITHE_DT_BF16 && y_dtype != LITHE_DT_F32) return LITHE_ERR_DTYPE;
    if (n_batch < 0 || seq < 0 || d_in < 1 || rank < 1 || routes->n_route < 1) return LITHE_ERR_SHAPE;
    if (n_batch > 65535 || seq > (int64_t)1 << 30) return LITHE_ERR_SHAPE;
    if (d_in % kBlock) return LITHE_ERR_ALIGN;
    if ((int64_t)groups_per_module * routes->n_route * n_mod > kMaxGroups) return LITHE_ERR_SHAPE;
    if (n_batch == 0 || seq == 0) return LITHE_OK;
    if (!x || !routes->slot) return LITHE_ERR_NULL;
    if (static_scratch) return ((uintptr_t)x & 15u) ? LITHE_ERR_ALIGN : LITHE_OK;
    if (!workspace) return LITHE_ERR_WORKSPACE;
    if (((uintptr_t)x & 15u) || ((uintptr_t)workspace & 255u)) return LITHE_ERR_ALIGN;
    return LITHE_OK;
}

// Validates indexed factors of one module (A over rank x d_in, B over d_out x rank).
int32_t check_indexed(const lithe_factors *f, int32_t rank, int64_t d_in, int64_t d_out) {
    int32_t rc = validate_src(&f->a_idx);
    if (rc) return rc;
    rc = validate_src(&f->b_idx);
    if (rc) return rc;
    if (f->a_idx.num_levels != f->b_idx.num_levels || f->lut_a.num_levels != f->a_idx.num_levels ||
        f->lut_b.num_levels != f->a_idx.num_levels)
        return LITHE_ERR_LEVELS;
    if (!src_covers(f->a_idx, rank * d_in / kBlock) || !src_covers(f->b_idx, d_out * rank / kBlock))
        return LITHE_ERR_SHAPE;
    return LITHE_OK;
}

// Workgroup counts of the shrink (n_mod_wg > 1: replicated shared-input layout, padded to whole
// XCD rounds) and of the expand (bounded over its sub-tile choices) fit a launch.
bool grids_fit(const Plan &p, int64_t n_batch, int64_t d_out, int n_mod_wg) {
    const int64_t shrink = n_mod_wg > 1 ? (n_batch * p.tiles_s + 7) / 8 * 8 * n_mod_wg : n_batch * p.tiles_s;
    const int64_t bow = (int64_t)p.BO << p.wo_sh;
    const int64_t expand = ((d_out + bow - 1) / bow) * n_batch * p.tiles_e * p.subs_e;
    return shrink <= kMaxGridX && expand <= kMaxGridX;
}

void copy_lut(float dst[kMaxLevels][10], const lithe_lut &l) {
    for (int v = 0; v < kMaxLevels; ++v)
        for (int q = 0; q < 10; ++q) dst[v][q] = l.value[v][q];
}

// Fields common to the shrink and the expand of a call: the error word (nullable) and the base of
// the rank-r intermediate.
void set_call_fields(LoraArgs &a, const void *x, int32_t *err, void *mid, int64_t n_batch, int64_t seq, int64_t d_in,
                     int32_t rank, const lithe_routes *routes, const float *mid_scale) {
    a.x = x;
    a.err = err;
    a.mid = mid;
    a.n_batch = n_batch;
    a.seq = seq;
    a.d_in = d_in;
    a.rows = n_batch * seq;
    a.rank = rank;
    a.n_route = routes->n_route;
    a.r_slot = routes->slot;
    a.r_w = routes->weight_sqrt;
    a.s_scale = routes->slot_scale;
    a.mid_scale = mid_scale;
}

// Fields of one module's expand.
void set_module_fields(LoraArgs &a, void *y, int64_t d_out, int32_t accumulate, float out_scale,
                       const float *out_scale_vec) {
    a.y = y;
    a.d_out = d_out;
    a.vec_y = (d_out % 8 == 0) && (((uintptr_t)y & 15u) == 0);
    a.accumulate = accumulate ? 1 : 0;
    a.out_scale = out_scale;
    a.out_scale_vec = out_scale_vec;
}

}  // namespace
}  // namespace lithe

namespace lithe {
namespace {

void *static_scratch();

// Body of lithe_lora_delta and lithe_lora_delta_noalloc. Workspace calls: the error word at
// `workspace`, the rank-r intermediate 256 bytes further, workspace_bytes in all. Static-scratch
// calls (workspace NULL, use_static): the intermediate in the current device's static scratch of
// LITHE_STATIC_SCRATCH_BYTES, the error word at err_flag (nullable).
int32_t lora_delta(const void *x, int32_t x_dtype, int64_t n_batch, int64_t seq, int64_t d_in, void *y,
                   int32_t y_dtype, int64_t d_out, int32_t accumulate, int32_t rank, const lithe_factors *f,
                   const lithe_routes *routes, const float *mid_scale, float out_scale, const float *out_scale_vec,
                   void *workspace, int64_t workspace_bytes, bool use_static, int32_t *err_flag, void *stream) {
    if (!f) return LITHE_ERR_NULL;
    const int n_rg = rank > 0 ? (rank + 15) / 16 : 1;
    int32_t rc = check_call(x, x_dtype, n_batch, seq, d_in, y_dtype, rank, routes, n_rg, 1, workspace, use_static);
    if (rc || n_batch == 0 || seq == 0) return rc;
    if (d_out < 1) return LITHE_ERR_SHAPE;
    if ((d_out * rank) % kBlock) return LITHE_ERR_ALIGN;
    if (!y) return LITHE_ERR_NULL;
    const int xbytes = x_dtype == LITHE_DT_BF16 ? 2 : 4;
    const int ybytes = y_dtype == LITHE_DT_BF16 ? 2 : 4;
    if ((uintptr_t)y & (uintptr_t)(ybytes - 1)) return LITHE_ERR_ALIGN;

    LoraArgs a{};
    if (f->kind == LITHE_FACTOR_INDEXED) {
        rc = check_indexed(f, rank, d_in, d_out);
        if (rc) return rc;
        a.a_src = make_src(f->a_idx);
        a.b_src = make_src(f->b_idx);
        for (int g = 0; g < kMaxGroups; ++g) a.a_goff[g] = a.a_src.block_off;
        a.a_src.block_off = 0;
        a.n_slots = std::min(f->a_idx.n_slots, f->b_idx.n_slots);
        copy_lut(a.luts.v[0], f->lut_a);
        copy_lut(a.luts.v[1], f->lut_b);
    } else if (f->kind == LITHE_FACTOR_DENSE) {
        if (!f->dense_a || !f->dense_b) return LITHE_ERR_NULL;
        if (f->dense_dtype != x_dtype) return LITHE_ERR_DTYPE;
        if (f->n_dense < 1) return LITHE_ERR_SHAPE;
        if (((uintptr_t)f->dense_a & 15u) || ((uintptr_t)f->dense_b & 15u)) return LITHE_ERR_ALIGN;
        if (routes->weight_sqrt || routes->slot_scale) return LITHE_ERR_UNSUPPORTED;
        a.dense_a = f->dense_a;
        a.dense_b = f->dense_b;
        a.n_slots = f->n_dense;
    } else {
        return LITHE_ERR_DTYPE;
    }

    const Plan p = make_plan(n_batch, seq, d_in, d_out, rank, routes->n_route, xbytes, f->kind == LITHE_FACTOR_DENSE,
                             ybytes);
    if (!grids_fit(p, n_batch, d_out, 1)) return LITHE_ERR_SHAPE;
    int32_t *err = err_flag;
    void *mid = nullptr;
    if (use_static) {
        if (p.total - p.off_mid > LITHE_STATIC_SCRATCH_BYTES) return LITHE_ERR_WORKSPACE;
        if (!(mid = static_scratch())) return LITHE_ERR_HIP;
    } else {
        if (workspace_bytes < p.total) return LITHE_ERR_WORKSPACE;
        err = static_cast<int32_t *>(workspace);
        mid = static_cast<char *>(workspace) + p.off_mid;
    }
    set_call_fields(a, x, err, mid, n_batch, seq, d_in, rank, routes, mid_scale);
    set_module_fields(a, y, d_out, accumulate, out_scale, out_scale_vec);
    set_shrink_fields(a, p);
    set_expand_fields(a, p);
    a.G1 = p.G;
    a.mid_goff = 0;
    const int src = src_of(a, f->kind);
    hipStream_t st = (hipStream_t)stream;
    launch_typed(true, x_dtype, y_dtype, p, a, src, st);
    launch_typed(false, x_dtype, y_dtype, p, a, src, st);
    return hipGetLastError() == hipSuccess ? LITHE_OK : LITHE_ERR_HIP;
}

}  // namespace
}  // namespace lithe

extern "C" int32_t lithe_lora_delta(const void *x, int32_t x_dtype, int64_t n_batch, int64_t seq, int64_t d_in,
                                    void *y, int32_t y_dtype, int64_t d_out, int32_t accumulate, int32_t rank,
                                    const lithe_factors *f, const lithe_routes *routes, const float *mid_scale,
                                    float out_scale, const float *out_scale_vec, void *workspace,
                                    int64_t workspace_bytes, void *stream) {
    return lithe::lora_delta(x, x_dtype, n_batch, seq, d_in, y, y_dtype, d_out, accumulate, rank, f, routes, mid_scale,
                             out_scale, out_scale_vec, workspace, workspace_bytes, false, nullptr, stream);
}

extern "C" int32_t lithe_lora_delta_shared_x(const void *x, int32_t x_dtype, int64_t n_batch, int64_t seq,
                                             int64_t d_in, int32_t n_mod, void *const *y, int32_t y_dtype,
                                             const int64_t *d_out, int32_t accumulate, int32_t rank,
                                             const lithe_factors *f, const lithe_routes *routes,
                                             const float *mid_scale, const float *out_scale, void *workspace,
                                             int64_t workspace_bytes, void *stream) {
    if (!f || !y || !d_out || !out_scale) return LITHE_ERR_NULL;
    if (n_mod < 1 || n_mod > kMaxGroups) return LITHE_ERR_SHAPE;
    const int n_rg = rank > 0 ? (rank + 15) / 16 : 1;
    int32_t rc = check_call(x, x_dtype, n_batch, seq, d_in, y_dtype, rank, routes, n_rg, 1, workspace);
    if (rc || n_batch == 0 || seq == 0) return rc;
    const int xbytes = x_dtype == LITHE_DT_BF16 ? 2 : 4;
    const int G1 = n_rg * routes->n_route;
    // replicated form: a workgroup carries one module's rank groups; the stacked form carries all
    const bool stacked = stack_shared(n_batch * ((seq + 15) / 16), n_mod, G1, xbytes);
    if (stacked && n_mod * G1 > kMaxGroups) return LITHE_ERR_SHAPE;
    const int ybytes = y_dtype == LITHE_DT_BF16 ? 2 : 4;
    int64_t d_out_max = 1;
    for (int m = 0; m < n_mod; ++m) {
        if (f[m].kind != LITHE_FACTOR_INDEXED) return LITHE_ERR_UNSUPPORTED;
        if (d_out[m] < 1) return LITHE_ERR_SHAPE;
        if ((d_out[m] * rank) % kBlock) return LITHE_ERR_ALIGN;
        if (!y[m]) return LITHE_ERR_NULL;
        if ((uintptr_t)y[m] & (uintptr_t)(ybytes - 1)) return LITHE_ERR_ALIGN;
        rc = check_indexed(&f[m], rank, d_in, d_out[m]);
        if (rc) return rc;
        // one shrink reads every module's A: one index source and one A value table
        const lithe_index_src &s0 = f[0].a_idx, &sm = f[m].a_idx;
        if (sm.base != s0.base || sm.kind != s0.kind || sm.num_levels != s0.num_levels ||
            sm.slot_stride != s0.slot_stride || sm.level_stride != s0.level_stride || sm.n_slots != s0.n_slots)
            return LITHE_ERR_UNSUPPORTED;
        for (int l = 0; l < kMaxLevels; ++l)
            for (int q = 0; q < 10; ++q)
                if (f[m].lut_a.value[l][q] != f[0].lut_a.value[l][q]) return LITHE_ERR_UNSUPPORTED;
        d_out_max = std::max(d_out_max, d_out[m]);
    }
    const Plan ps = make_plan(n_batch, seq, d_in, d_out_max, rank, routes->n_route * n_mod, xbytes, false, ybytes);
    if (!grids_fit(ps, n_batch, d_out_max, n_mod)) return LITHE_ERR_SHAPE;
    if (workspace_bytes < ps.total) return LITHE_ERR_WORKSPACE;

    LoraArgs a{};
    a.a_src = make_src(f[0].a_idx);
    a.a_src.block_off = 0;
    a.n_slots = f[0].a_idx.n_slots;
    copy_lut(a.luts.v[0], f[0].lut_a);
    set_call_fields(a, x, static_cast<int32_t *>(workspace), static_cast<char *>(workspace) + ps.off_mid, n_batch, seq,
                    d_in, rank, routes, mid_scale);
    // Shrink: module-stacked (all modules' A rows as rank groups of one workgroup) or replicated
    // (one single-module workgroup per tile and module, x shared through L2).
    Plan pshrink = ps;
    if (stacked) {
        for (int g = 0; g < kMaxGroups; ++g) a.a_goff[g] = f[std::min(g / G1, n_mod - 1)].a_idx.block_off;
        a.n_mod_wg = 1;
    } else {
        pshrink = make_plan(n_batch, seq, d_in, d_out_max, rank, routes->n_route, xbytes, false, ybytes);
        for (int g = 0; g < kMaxGroups; ++g) a.a_goff[g] = f[std::min(g, n_mod - 1)].a_idx.block_off;
        a.n_mod_wg = n_mod;
    }
    set_shrink_fields(a, pshrink);
    a.MR = ps.MR;          // mid rows hold every module's groups
    a.G1 = G1;
    a.b_src = make_src(f[0].b_idx);
    set_module_fields(a, y[0], d_out[0], accumulate, out_scale[0], nullptr);
    hipStream_t st = (hipStream_t)stream;
    const int src = src_of(a, LITHE_FACTOR_INDEXED);
    launch_typed(true, x_dtype, y_dtype, pshrink, a, src, st);

    // Expands: one grouped launch for every module when they read one B index source and one B
    // value table (one bank; bf16, packed indices), else one launch per module. The outputs are
    // the same either way (a module's expand sums do not depend on its tiling).
    bool one_b = x_dtype == LITHE_DT_BF16 && y_dtype == LITHE_DT_BF16 && src == SRC_PACKED &&
                 getenv("LITHE_GROUPED_SERIAL") == nullptr;
    for (int m = 1; m < n_mod && one_b; ++m) {
        const lithe_index_src &b0 = f[0].b_idx, &bm = f[m].b_idx;
        one_b = bm.base == b0.base && bm.kind == b0.kind && bm.num_levels == b0.num_levels &&
                bm.slot_stride == b0.slot_stride && bm.level_stride == b0.level_stride && bm.n_slots == b0.n_slots;
        for (int l = 0; l < kMaxLevels; ++l)
            for (int q = 0; q < 10; ++q) one_b = one_b && f[m].lut_b.value[l][q] == f[0].lut_b.value[l][q];
    }
    if (one_b) {
        const PlanCtx ctx{n_batch * ((seq + 15) / 16)};
        GroupArgs ge{};
        ge.a = a;
        ge.a.n_slots = std::min(f[0].a_idx.n_slots, f[0].b_idx.n_slots);
        copy_lut(ge.a.luts.v[1], f[0].lut_b);
        Plan pe[kMaxJobs];
        int64_t wg = 0;
        size_t lds_e = 0;
        for (int m = 0; m < n_mod; ++m) {
            const Plan p = make_plan(n_batch, seq, d_in, d_out[m], rank, routes->n_route, xbytes, false, ybytes, &ctx);
            pe[m] = p;
            set_shrink_fields(ge.a, p);    // G, n_rg of one module (the same for every job)
            GroupJob &j = ge.job[m];
            j.x = x;
            j.y = y[m];
            j.mid = a.mid;
            j.seq = seq;
            j.d_in = d_in;
            j.d_out = d_out[m];
            j.rows = n_batch * seq;
            for (int g = 0; g < kMaxGroups; ++g) j.a_goff[g] = a.a_goff[g];
            j.b_off = f[m].b_idx.block_off;
            j.MR = ps.MR;
            j.mid_goff = m * G1;
            j.n_mod_wg = 1;
            j.xnt = 1;
            j.tiles_s = p.tiles_s;
            j.ks = p.ks;
            j.pb = p.pb;
            j.arow = p.arow;
            j.region = p.region;
            j.red_off = p.red_off;
            j.stage_off = p.stage_off;
            j.tiles_e = p.tiles_e;
            j.subs_e = p.subs_e;
            j.BO = p.BO;
            j.vec_y = (d_out[m] % 8 == 0) && (((uintptr_t)y[m] & 15u) == 0);
            j.nblk_max = p.nblk_max;
            j.estage_off = p.estage_off;
            j.wo_sh = p.wo_sh;
            j.out_scale = out_scale[m];
            ge.begin[m] = (int32_t)wg;
            const int64_t bow = (int64_t)p.BO << p.wo_sh;
            wg += (((d_out[m] + bow - 1) / bow) * n_batch * p.tiles_e + 7) / 8 * 8;
            lds_e = std::max(lds_e, p.lds_e);
        }
        ge.n_jobs = n_mod;
        if (wg > kMaxGridX) return LITHE_ERR_SHAPE;
        launch_expand_group_bf16_bf16(pe[0].GE, pe[0].BOM, pe[0].NS, ge, (unsigned)wg, lds_e, src, st);
        return hipGetLastError() == hipSuccess ? LITHE_OK : LITHE_ERR_HIP;
    }
    for (int m = 0; m < n_mod; ++m) {
        const Plan pe = make_plan(n_batch, seq, d_in, d_out[m], rank, routes->n_route, xbytes, false, ybytes);
        LoraArgs e = a;
        e.b_src = make_src(f[m].b_idx);
        e.n_slots = std::min(f[m].a_idx.n_slots, f[m].b_idx.n_slots);
        copy_lut(e.luts.v[1], f[m].lut_b);
        set_module_fields(e, y[m], d_out[m], accumulate, out_scale[m], nullptr);
        e.G = pe.G;            // this module's groups; mid rows keep the shrink's width
        e.mid_goff = m * G1;
        set_expand_fields(e, pe);
        launch_typed(false, x_dtype, y_dtype, pe, e, src_of(e, LITHE_FACTOR_INDEXED), st);
    }
    return hipGetLastError() == hipSuccess ? LITHE_OK : LITHE_ERR_HIP;
}

namespace lithe {
namespace {

// Shrink jobs of a grouped call: the modules that read one input (same x, seq and d_in; at most
// kMaxGroups per job) share a job, each job owns one intermediate region of the workspace.
struct GroupLayout {
    int n_sj;
    int sj_of_mod[kMaxJobs];      // shrink job of module m
    int pos_in_sj[kMaxJobs];      // module m's place in its job (its rank groups in the job's rows)
    int n_in_sj[kMaxJobs];        // modules of each job
    int mods_of_sj[kMaxJobs][kMaxGroups];
    int64_t mid_off[kMaxJobs];    // byte offset of each job's intermediate
    int64_t total;                // workspace bytes
};

void group_layout(int64_t n_batch, int n_mod, const lithe_module *mods, int G, int xbytes, GroupLayout &L) {
    L = GroupLayout{};
    for (int m = 0; m < n_mod; ++m) {
        int j = -1;
        for (int q = 0; q < L.n_sj && j < 0; ++q) {
            const lithe_module &f = mods[L.mods_of_sj[q][0]];
            if (f.x == mods[m].x && f.seq == mods[m].seq && f.d_in == mods[m].d_in && L.n_in_sj[q] < kMaxGroups) j = q;
        }
        if (j < 0) j = L.n_sj++;
        L.sj_of_mod[m] = j;
        L.pos_in_sj[m] = L.n_in_sj[j];
        L.mods_of_sj[j][L.n_in_sj[j]++] = m;
    }
    int64_t off = 256;
    for (int q = 0; q < L.n_sj; ++q) {
        L.mid_off[q] = off;
        off = align256(off + n_batch * mods[L.mods_of_sj[q][0]].seq * (int64_t)L.n_in_sj[q] * G * 16 * xbytes);
    }
    L.total = off;
}

int64_t round8(int64_t v) { return (v + 7) / 8 * 8; }

}  // namespace
}  // namespace lithe

extern "C" int64_t lithe_lora_grouped_workspace_bytes(int64_t n_batch, int32_t n_mod, const lithe_module *mods,
                                                      int32_t rank, int32_t n_route, int32_t x_dtype) {
    if (!mods) return LITHE_ERR_NULL;
    if (n_mod < 1 || n_mod > kMaxJobs || n_batch < 0 || rank < 1 || n_route < 1) return LITHE_ERR_SHAPE;
    if (x_dtype != LITHE_DT_BF16 && x_dtype != LITHE_DT_F32) return LITHE_ERR_DTYPE;
    const int G = ((rank + 15) / 16) * n_route;
    if (G > kMaxGroups) return LITHE_ERR_SHAPE;
    for (int m = 0; m < n_mod; ++m)
        if (mods[m].seq < 0) return LITHE_ERR_SHAPE;
    GroupLayout L;
    group_layout(n_batch, n_mod, mods, G, x_dtype == LITHE_DT_BF16 ? 2 : 4, L);
    return L.total;
}

extern "C" int32_t lithe_lora_delta_grouped(int32_t n_mod, const lithe_module *mods_in, int32_t x_dtype,
                                            int32_t y_dtype, int64_t n_batch, int32_t accumulate, int32_t rank,
                                            const lithe_factors *f, const lithe_routes *routes, void *workspace,
                                            int64_t workspace_bytes, void *stream) {
    if (!mods_in || !f) return LITHE_ERR_NULL;
    if (n_mod < 1 || n_mod > kMaxJobs) return LITHE_ERR_SHAPE;
    const bool dense = f->kind == LITHE_FACTOR_DENSE;
    if (f->kind != LITHE_FACTOR_INDEXED && !dense) return LITHE_ERR_UNSUPPORTED;
    const int n_rg = rank > 0 ? (rank + 15) / 16 : 1;
    const int xbytes = x_dtype == LITHE_DT_BF16 ? 2 : 4;
    const int ybytes = y_dtype == LITHE_DT_BF16 ? 2 : 4;
    // validate every module as lithe_lora_delta would; keep those with tokens
    lithe_module mods[kMaxJobs];
    int n_act = 0;
    for (int m = 0; m < n_mod; ++m) {
        const lithe_module &md = mods_in[m];
        int32_t rc = check_call(md.x, x_dtype, n_batch, md.seq, md.d_in, y_dtype, rank, routes, n_rg, 1, workspace);
        if (rc) return rc;
        if (n_batch == 0 || md.seq == 0) continue;
        if (md.d_out < 1) return LITHE_ERR_SHAPE;
        if ((md.d_out * rank) % kBlock) return LITHE_ERR_ALIGN;
        if (!md.y) return LITHE_ERR_NULL;
        if ((uintptr_t)md.y & (uintptr_t)(ybytes - 1)) return LITHE_ERR_ALIGN;
        if (dense) {
            if (md.a_block_off < 0 || md.b_block_off < 0) return LITHE_ERR_SHAPE;
        } else {
            lithe_factors fm = *f;
            fm.a_idx.block_off = md.a_block_off;
            fm.b_idx.block_off = md.b_block_off;
            rc = check_indexed(&fm, rank, md.d_in, md.d_out);
            if (rc) return rc;
        }
        mods[n_act++] = md;
    }
    if (n_act == 0) return LITHE_OK;
    for (int m = 0; m < n_act; ++m)
        for (int q = m + 1; q < n_act; ++q) {
            const uintptr_t lo0 = (uintptr_t)mods[m].y, lo1 = (uintptr_t)mods[q].y;
            const uintptr_t hi0 = lo0 + (uintptr_t)(n_batch * mods[m].seq * mods[m].d_out * ybytes);
            const uintptr_t hi1 = lo1 + (uintptr_t)(n_batch * mods[q].seq * mods[q].d_out * ybytes);
            if (lo0 < hi1 && lo1 < hi0) return LITHE_ERR_OVERLAP;
        }
    const int G = n_rg * routes->n_route;
    GroupLayout L;
    group_layout(n_batch, n_act, mods, G, xbytes, L);
    if (workspace_bytes < L.total) return LITHE_ERR_WORKSPACE;

    PlanCtx ctx{0};
    for (int q = 0; q < L.n_sj; ++q) ctx.groups += n_batch * ((mods[L.mods_of_sj[q][0]].seq + 15) / 16);

    // common fields; each job's fields are applied over them
    char *ws = static_cast<char *>(workspace);
    LoraArgs a{};
    if (dense) {
        // module m's A / B: the (n_dense, rank, d_in) / (n_dense, d_out, rank) stacks at elements
        // n_dense * 64 * a_block_off / b_block_off of dense_a / dense_b (lithe_decode_stacked's layout)
        if (!f->dense_a || !f->dense_b) return LITHE_ERR_NULL;
        if (f->dense_dtype != x_dtype) return LITHE_ERR_DTYPE;
        if (f->n_dense < 1) return LITHE_ERR_SHAPE;
        if (((uintptr_t)f->dense_a & 15u) || ((uintptr_t)f->dense_b & 15u)) return LITHE_ERR_ALIGN;
        if (routes->weight_sqrt || routes->slot_scale) return LITHE_ERR_UNSUPPORTED;
        a.dense_a = f->dense_a;
        a.dense_b = f->dense_b;
        a.n_slots = f->n_dense;
    } else {
        a.a_src = make_src(f->a_idx);
        a.a_src.block_off = 0;
        a.b_src = make_src(f->b_idx);
        a.n_slots = std::min(f->a_idx.n_slots, f->b_idx.n_slots);
        copy_lut(a.luts.v[0], f->lut_a);
        copy_lut(a.luts.v[1], f->lut_b);
    }
    set_call_fields(a, mods[0].x, reinterpret_cast<int32_t *>(ws), ws + L.mid_off[0], n_batch, mods[0].seq,
                    mods[0].d_in, rank, routes, nullptr);
    set_module_fields(a, mods[0].y, mods[0].d_out, accumulate, 1.0f, nullptr);
    a.G1 = G;
    const int src = src_of(a, f->kind);

    // Modules that share an input: stacked (every job's modules as rank groups of one workgroup;
    // one kernel serves the launch, so only when every job has the same module count) or
    // replicated (one workgroup per tile and module, x shared through L2).
    const int nm0 = L.n_in_sj[0];
    bool stack = !dense && nm0 > 1 && nm0 * G <= kMaxGroups;
    for (int q = 1; q < L.n_sj; ++q) stack = stack && L.n_in_sj[q] == nm0;
    stack = stack && stack_shared(ctx.groups, nm0, G, xbytes);
    // shrink jobs, largest first (the short ones fill the tail of the grid)
    GroupArgs gs{};
    gs.a = a;
    Plan ps[kMaxJobs];
    int order[kMaxJobs];
    for (int q = 0; q < L.n_sj; ++q) order[q] = q;
    auto sj_work = [&](int q) { const lithe_module &md = mods[L.mods_of_sj[q][0]]; return md.seq * md.d_in * L.n_in_sj[q]; };
    std::stable_sort(order, order + L.n_sj, [&](int u, int v) { return sj_work(u) > sj_work(v); });
    int64_t wg = 0;
    size_t lds_s = 0;
    for (int k = 0; k < L.n_sj; ++k) {
        const int q = order[k];
        const lithe_module &md = mods[L.mods_of_sj[q][0]];
        const int nm = L.n_in_sj[q];
        const Plan p = make_plan(n_batch, md.seq, md.d_in, md.d_out, rank, routes->n_route * (stack ? nm : 1), xbytes,
                                 dense, ybytes, &ctx);
        ps[k] = p;
        set_shrink_fields(gs.a, p);       // G, n_rg (the same for every job)
        GroupJob &j = gs.job[k];
        j.x = md.x;
        j.y = md.y;
        j.mid = ws + L.mid_off[q];
        j.seq = md.seq;
        j.d_in = md.d_in;
        j.d_out = md.d_out;
        j.rows = n_batch * md.seq;
        // stacked: group g belongs to module g / G; replicated: the workgroups of module m use a_goff[m]
        for (int g = 0; g < kMaxGroups; ++g)
            j.a_goff[g] = mods[L.mods_of_sj[q][std::min(stack ? g / G : g, nm - 1)]].a_block_off;
        j.MR = nm * G * 16;
        j.n_mod_wg = stack ? 1 : nm;
        j.xnt = j.n_mod_wg > 1 ? 0 : 1;
        j.tiles_s = p.tiles_s;
        j.ks = p.ks;
        j.pb = p.pb;
        j.arow = p.arow;
        j.region = p.region;
        j.red_off = p.red_off;
        j.stage_off = p.stage_off;
        gs.begin[k] = (int32_t)wg;
        const int64_t tiles = n_batch * p.tiles_s;
        wg += round8(j.n_mod_wg > 1 ? round8(tiles) * nm : tiles);
        lds_s = std::max(lds_s, p.lds_s);
    }
    gs.n_jobs = L.n_sj;
    const int64_t grid_s = wg;

    // expand jobs (one per module), largest first
    GroupArgs ge{};
    ge.a = a;
    Plan pe[kMaxJobs];
    for (int m = 0; m < n_act; ++m) order[m] = m;
    std::stable_sort(order, order + n_act,
                     [&](int u, int v) { return mods[u].seq * mods[u].d_out > mods[v].seq * mods[v].d_out; });
    wg = 0;
    size_t lds_e = 0;
    for (int k = 0; k < n_act; ++k) {
        const int m = order[k];
        const lithe_module &md = mods[m];
        const Plan p = make_plan(n_batch, md.seq, md.d_in, md.d_out, rank, routes->n_route, xbytes, dense, ybytes, &ctx);
        pe[k] = p;
        set_shrink_fields(ge.a, p);
        GroupJob &j = ge.job[k];
        const int q = L.sj_of_mod[m];
        j.x = md.x;
        j.y = md.y;
        j.mid = ws + L.mid_off[q];
        j.seq = md.seq;
        j.d_in = md.d_in;
        j.d_out = md.d_out;
        j.rows = n_batch * md.seq;
        for (int g = 0; g < kMaxGroups; ++g) j.a_goff[g] = md.a_block_off;
        j.b_off = md.b_block_off;
        j.MR = L.n_in_sj[q] * G * 16;
        j.mid_goff = L.pos_in_sj[m] * G;
        j.n_mod_wg = 1;
        j.tiles_e = p.tiles_e;
        j.subs_e = p.subs_e;
        j.BO = p.BO;
        j.vec_y = (md.d_out % 8 == 0) && (((uintptr_t)md.y & 15u) == 0);
        j.nblk_max = p.nblk_max;
        j.estage_off = p.estage_off;
        j.wo_sh = p.wo_sh;
        j.out_scale = md.out_scale;
        ge.begin[k] = (int32_t)wg;
        const int64_t bow = (int64_t)p.BO << p.wo_sh;
        wg += round8(((md.d_out + bow - 1) / bow) * n_batch * p.tiles_e);
        lds_e = std::max(lds_e, p.lds_e);
    }
    ge.n_jobs = n_act;
    const int64_t grid_e = wg;
    if (grid_s > kMaxGridX || grid_e > kMaxGridX) return LITHE_ERR_SHAPE;

    hipStream_t st = (hipStream_t)stream;
    const bool grouped = getenv("LITHE_GROUPED_SERIAL") == nullptr;
    if (grouped && launch_shrink_group_bf16_ok(x_dtype, y_dtype, src)) {
        launch_shrink_group_bf16(ps[0].GMs, ps[0].tw, gs, (unsigned)grid_s, lds_s, src, st);
        launch_expand_group_bf16_bf16(pe[0].GE, pe[0].BOM, pe[0].NS, ge, (unsigned)grid_e, lds_e, src, st);
    } else {
        // job by job through the per-call kernels (other dtypes and factor kinds)
        for (int k = 0; k < gs.n_jobs; ++k) {
            LoraArgs aj = gs.a;
            apply_job(aj, gs.job[k]);
            for (int g = 0; g < kMaxGroups; ++g) aj.a_goff[g] = gs.job[k].a_goff[g];
            launch_typed(true, x_dtype, y_dtype, ps[k], aj, src, st);
        }
        for (int k = 0; k < ge.n_jobs; ++k) {
            LoraArgs aj = ge.a;
            apply_job(aj, ge.job[k]);
            launch_typed(false, x_dtype, y_dtype, pe[k], aj, src, st);
        }
    }
    return hipGetLastError() == hipSuccess ? LITHE_OK : LITHE_ERR_HIP;
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

namespace lithe {
namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
std::atomic<void *> g_scratch_addr[kScratchDevices];

// Device address of the current device's static scratch, looked up once per device (with that
// device current) and kept; nullptr if the lookup fails.
void *static_scratch() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices) return nullptr;
    void *p = g_scratch_addr[dev].load(std::memory_order_acquire);
    if (p) return p;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (!p) {
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
        g_scratch_addr[dev].store(p, std::memory_order_release);
    }
    return p;
}

}  // namespace
}  // namespace lithe

extern "C" int32_t lithe_lora_delta_noalloc(const void *x, int32_t x_dtype, int64_t n_batch, int64_t seq,
                                            int64_t d_in, void *y, int32_t y_dtype, int64_t d_out, int32_t accumulate,
                                            int32_t rank, const lithe_factors *f, const lithe_routes *routes,
                                            const float *mid_scale, float out_scale, const float *out_scale_vec,
                                            int32_t *err_flag, void *stream) {
    return lithe::lora_delta(x, x_dtype, n_batch, seq, d_in, y, y_dtype, d_out, accumulate, rank, f, routes, mid_scale,
                             out_scale, out_scale_vec, nullptr, 0, true, err_flag, stream);
}
