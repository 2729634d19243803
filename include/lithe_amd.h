/*
 * lithe_amd: C ABI of the MI355X (gfx950) index-resident multi-adapter LoRA path.
 *
 * Every entry point takes device pointers and sizes (no framework types),
 * validates its arguments before touching the GPU, enqueues its kernels on
 * the given HIP stream (NULL = the null stream) and returns without
 * synchronising. Return value: LITHE_OK (0) or a negative LITHE_ERR_* code;
 * lithe_status_string() names it. The library never allocates device memory:
 * scratch space is a caller-provided workspace.
 *
 * Citations name the reference function each entry point replaces
 * (paths relative to the reference repository root).
 */
#ifndef LITHE_AMD_H
#define LITHE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status codes */
#define LITHE_OK             0
#define LITHE_ERR_NULL      -1   /* a required pointer is NULL */
#define LITHE_ERR_SHAPE     -2   /* a size is negative, zero where it must not be, or inconsistent */
#define LITHE_ERR_ALIGN     -3   /* d_in or d_out * rank not a multiple of the 64-value block */
#define LITHE_ERR_DTYPE     -4   /* unsupported dtype / kind code */
#define LITHE_ERR_RANGE     -5   /* an index value above 511 (host packing) */
#define LITHE_ERR_WORKSPACE -6   /* workspace NULL or smaller than lithe_lora_workspace_bytes() */
#define LITHE_ERR_HIP       -7   /* a HIP launch or query failed */
#define LITHE_ERR_LEVELS    -8   /* num_levels outside [1, 4] */
#define LITHE_ERR_UNSUPPORTED -9 /* weight_sqrt / slot_scale given with dense factors */
#define LITHE_ERR_OVERLAP  -10   /* two modules of a grouped call write overlapping outputs */

/* ---------------------------------------------------------------- dtype codes */
#define LITHE_DT_BF16  1
#define LITHE_DT_F32   2
#define LITHE_DT_F16   3
#define LITHE_DT_I16   4
#define LITHE_DT_I32   5
#define LITHE_DT_I64   6
#define LITHE_DT_U16   7

/* ---------------------------------------------------------------- index sources */
/* Packed residency stream: uint64 words, index p of a slot at bits [9(p%7), 9(p%7)+9)
 * of word p/7, p = block * num_levels + level (lithe/kernels/packed.py:1-9, 38-52). */
#define LITHE_IDX_PACKED9    1
/* Level-major integer indices (n_slots, num_levels, n_blocks), as idx_A / idx_B of
 * lithe/kernels/shared.py:203-204 (int32) and lithe/serve.py:58-60 (int16). */
#define LITHE_IDX_LEVEL_I32  2
#define LITHE_IDX_LEVEL_I16  3
/* Block-major int16 indices (n_blocks, num_levels) per slot (lithe/kernels/packed.py:225-238). */
#define LITHE_IDX_BLOCK_I16  4

typedef struct lithe_index_src {
    const void *base;       /* device pointer */
    int32_t kind;           /* LITHE_IDX_* */
    int32_t num_levels;     /* 1..4 */
    int64_t slot_stride;    /* elements (uint64 words for PACKED9, < 2^32 / 7) from one slot to the next */
    int64_t level_stride;   /* elements from one level to the next (LEVEL_* kinds only) */
    int64_t block_off;      /* first block of the factor inside a slot (a_off / b_off of the layout) */
    int64_t n_slots;        /* number of addressable slots; larger slot ids are rejected in-kernel */
} lithe_index_src;

/* Value table of one side: value[l][p] is the pool value at level l of a codeword
 * coordinate whose 9-bit sign mismatch count popcount((k ^ m_t) & 511) is p, i.e.
 * sigma_l * (9 - 2p) / 3 in the pool's precision (lithe/codebook.py:59-77). */
typedef struct lithe_lut {
    int32_t num_levels;     /* 1..4 */
    float value[4][10];
} lithe_lut;

/* ---------------------------------------------------------------- misc */
int32_t lithe_abi_version(void);                 /* 1 */
const char *lithe_status_string(int32_t code);

/* ---------------------------------------------------------------- pack / unpack */
/* Host packing of n uint16 indices into ceil(n/7) words; LITHE_ERR_RANGE if any > 511.
 * Replaces pack_indices, lithe/kernels/packed.py:38-52. */
int32_t lithe_pack9_host(const uint16_t *idx, int64_t n, uint64_t *words);

/* Device packing. idx_dtype in {U16, I16, I32, I64}. A value outside [0, 511] writes
 * 1 to *err_flag (device int32, may be NULL) and its field is packed as 0.
 * Replaces pack_indices for device-resident indices (lithe/kernels/packed.py:38-52). */
int32_t lithe_pack9(const void *idx, int32_t idx_dtype, int64_t n, uint64_t *words,
                    int32_t *err_flag, void *stream);

/* Device unpacking of n indices; out_dtype in {I16, I32, I64}.
 * Replaces unpack_indices, lithe/kernels/packed.py:55-60. */
int32_t lithe_unpack9(const uint64_t *words, int64_t n, void *out, int32_t out_dtype, void *stream);

/* ---------------------------------------------------------------- ingest (.lithe stream -> bank slot) */
/* The .lithe index stream (lithe/fileio.py:1-13) holds the A matrices of every module in header
 * order, then the B matrices, each as its (L, n_blocks) matrix in row-major order. The residency
 * order of a bank slot is (block, level)-major with each module's A blocks followed by its B
 * blocks (lithe/kernels/packed.py:125-133). A layout's segment table has one row of three int64
 * per factor, in residency order (module m: A = row 2m, B = row 2m + 1): first residency block,
 * block count, first element of the factor in the stream.
 * Replaces the module bookkeeping of load_lithe (lithe/fileio.py:136-150) and PackedLayout
 * (lithe/kernels/packed.py:100-117). */
int32_t lithe_ingest_table(int32_t n_modules, const int64_t *blocks_a, const int64_t *blocks_b,
                           int32_t num_levels, int64_t *table);

/* Host: reorder n_stream uint16 stream indices into the residency order and pack them 7 per word
 * (words[n_words], zero-padded). LITHE_ERR_RANGE (nothing written) if any index > 511,
 * LITHE_ERR_SHAPE if the table does not describe exactly n_stream indices.
 * Replaces flat_indices + pack_indices over a loaded adapter (lithe/kernels/packed.py:38-52, 125-143). */
int32_t lithe_ingest_host(const uint16_t *stream, int64_t n_stream, int32_t num_levels, int32_t n_segments,
                          const int64_t *table, uint64_t *words, int64_t n_words);

/* Device: the same from a device stream and a device copy of the table, written straight into
 * `words` (e.g. a bank slot). *err_flag (device int32, nullable) gets bit 1 for an index > 511
 * (packed as 0) and bit 2 for a table position outside the stream (read as index 0). */
int32_t lithe_ingest(const uint16_t *stream, int64_t n_stream, int32_t num_levels, int32_t n_segments,
                     const int64_t *table, uint64_t *words, int64_t n_words, int32_t *err_flag,
                     void *stream_hip);

/* ---------------------------------------------------------------- bulk decode */
/* Decode n_blocks 64-value blocks of each selected slot to dense values:
 *   out[s][blk][t] = sum_l lut_side(blk).value[l][popcount((k_l ^ m_t) & 511)]   (fp32, l in order)
 * cast once to out_dtype (BF16: round to nearest even, or F32). sides[blk] = 0 picks lut_a,
 * 1 picks lut_b (sides NULL: all lut_a). slots: device int32 (n_sel,), NULL = slot 0 for n_sel == 1.
 * out_sel_stride: elements between the outputs of consecutive selected slots.
 * err_flag (device int32, nullable) gets bit 1 for a slot id outside [0, n_slots) (its output
 * is zero-filled) and bit 2 for an unpacked index above 511 (decoded as index 0).
 * Replaces _decode_packed_kernel / decode_packed (lithe/kernels/packed.py:151-177, 205-222),
 * _decode_int16_kernel / decode_int16 (:179-195, :225-238) and quant.rvq_decode_blocks
 * (lithe/quant.py:74-81). */
int32_t lithe_decode(const lithe_index_src *src, const int32_t *slots, int32_t n_sel,
                     int64_t n_blocks, const int8_t *sides, const lithe_lut *lut_a,
                     const lithe_lut *lut_b, void *out, int32_t out_dtype,
                     int64_t out_sel_stride, int32_t *err_flag, void *stream);

/* Bulk decode into the stacked layout of decoded-mode serving: every factor of the layout gets
 * its selections side by side, so module m's A is an (n_sel, rank, d_in) array and its B an
 * (n_sel, d_out, rank) array, ready for LITHE_FACTOR_DENSE. table: device copy of the layout's
 * segment table (lithe_ingest_table; rows in residency order, only the first two columns are
 * read). Block blk of segment s (first block f, count n) of selection i is written at output
 * block n_sel * f + i * n + (blk - f). err_flag bit 4: a table row maps a block outside the
 * n_sel * n_blocks output blocks (nothing is written there). Otherwise as lithe_decode.
 * Replaces decode_packed + split_decoded + the per-module torch.stack of
 * PerSampleLoRALinear._build_stacked (lithe/kernels/packed.py:205-222, 260-269;
 * lithe/kernels/layers.py:58-64). */
int32_t lithe_decode_stacked(const lithe_index_src *src, const int32_t *slots, int32_t n_sel,
                             int64_t n_blocks, int32_t n_segments, const int64_t *table,
                             const int8_t *sides, const lithe_lut *lut_a, const lithe_lut *lut_b,
                             void *out, int32_t out_dtype, int32_t *err_flag, void *stream);

/* ---------------------------------------------------------------- encode (nearest-codeword search) */
/* Greedy L-level encode of n 64-value fp32 blocks against the twin codebook, L = lut_a->num_levels:
 * at level l, bit q of the index is [<r, U[:, q]> > 0] for the residual r and the nine
 * Sylvester-Hadamard columns U[t, q] = (-1)^popcount(t & q) (all codewords of a level have one
 * norm, so this is the nearest codeword); the codeword value[l][popcount((k ^ m_t) & 511)] is
 * added to the reconstruction and subtracted from the residual in fp32. sides[i] = 1 (sides
 * nullable) encodes block i with lut_b, else lut_a. Index l of block i is written to
 * idx[l * idx_level_stride + i * idx_block_stride] (dtype I16, I32 or I64): (L, n) level-major
 * (block stride 1, level stride >= n: a .lithe factor matrix) or (n, L) block-major (level
 * stride 1, block stride >= L: the residency order of a slot). recon (nullable, 16-byte
 * aligned) receives the (n, 64) fp32 reconstruction. The fp32 projections are summed in a fixed
 * order that differs from a BLAS matmul, so a projection within rounding of zero may take the
 * other sign.
 * Replaces _lattice_search_kernel / lattice_search / rvq_encode_blocks_fast
 * (lithe/kernels/search.py:27-99) and quant.rvq_encode_blocks (lithe/quant.py:46-71). */
int32_t lithe_encode(const float *blocks, int64_t n, const int8_t *sides, const lithe_lut *lut_a,
                     const lithe_lut *lut_b, void *idx, int32_t idx_dtype, int64_t idx_level_stride,
                     int64_t idx_block_stride, float *recon, void *stream);

/* ---------------------------------------------------------------- per-sample LoRA delta */
/* Where the factors of the delta come from. */
#define LITHE_FACTOR_INDEXED 1   /* decoded in-kernel from index sources + value tables */
#define LITHE_FACTOR_DENSE   2   /* dense A (n, rank, d_in) and B (n, d_out, rank) */

typedef struct lithe_factors {
    int32_t kind;               /* LITHE_FACTOR_* */
    int32_t dense_dtype;        /* DENSE: BF16 or F32 */
    lithe_index_src a_idx;      /* INDEXED: A (rank, d_in) blocks, row-major flattening */
    lithe_index_src b_idx;      /* INDEXED: B (d_out, rank) blocks, row-major flattening */
    lithe_lut lut_a, lut_b;     /* INDEXED */
    const void *dense_a;        /* DENSE: (n_dense, rank, d_in) */
    const void *dense_b;        /* DENSE: (n_dense, d_out, rank) */
    int64_t n_dense;            /* DENSE: number of factor pairs */
} lithe_factors;

/* Per-sample routing: sample b uses route entries slot[b * n_route + j], j < n_route
 * (-1 = empty entry). Entry j contributes its adapter at rank offset j * rank of the
 * rank-stacked factors (lithe/serve.py:85-96). weight_sqrt (nullable) multiplies both
 * decoded factors of the entry; slot_scale[slot] (nullable) multiplies B first
 * (alpha / r folded into B, lithe/serve.py:69-73). Both apply to INDEXED factors only:
 * with DENSE factors they must be NULL (LITHE_ERR_UNSUPPORTED). */
typedef struct lithe_routes {
    const int32_t *slot;        /* device (n_batch, n_route) */
    const float *weight_sqrt;   /* device (n_batch, n_route) or NULL */
    const float *slot_scale;    /* device (n_slots,) or NULL */
    int32_t n_route;            /* >= 1 */
} lithe_routes;

/* Bytes of workspace lithe_lora_delta needs for these sizes: a 256-byte head whose first
 * int32 is the in-kernel error word (zero it before the first use; lithe_workspace_errors
 * reads and clears it), then the rank-r intermediate x A^T of every token. Calls that
 * overlap in time must not share a workspace. */
int64_t lithe_lora_workspace_bytes(int64_t n_batch, int64_t seq, int64_t d_in, int64_t d_out,
                                   int32_t rank, int32_t n_route, int32_t x_dtype);

/* y (n_batch, seq, d_out) receives the per-sample LoRA delta of x (n_batch, seq, d_in):
 *   mid   = round_x( (x A^T) * mid_scale[b] )          fp32 accumulation, A rows stacked per route
 *   d     = round_y( round_y(mid B^T) * s_b )           s_b = out_scale_vec ? out_scale_vec[b] : out_scale
 *   y     = accumulate ? round_y(y + d) : d
 * round_x / round_y round to the activation / output dtype (BF16: nearest even). The rounding
 * chain is the reference's: y_lo in x.dtype, delta in out_dtype, `delta * scaling`, `out + delta`.
 * x_dtype in {BF16, F32}; y_dtype in {BF16, F32}. d_in % 64 == 0 and d_out * rank % 64 == 0.
 * Samples whose route entries are all empty leave y untouched (accumulate) or zero it.
 * Replaces _shared_decode_A_matmul_kernel + _shared_decode_B_matmul_kernel and the host
 * wrapper shared_codebook_lora_delta (lithe/kernels/shared.py:36-157, 197-263), the SGMV pair
 * _lora_shrink_kernel + _lora_expand_kernel (lithe/kernels/sgmv.py:29-100, 112-160), and the
 * delta of IndexLoRALinear.forward (lithe/kernels/layers.py:120-131), MultiAdapterLinear.forward
 * (lithe/serve.py:75-97) and LitheLinear.forward (lithe/module.py:145-156). */
int32_t lithe_lora_delta(const void *x, int32_t x_dtype, int64_t n_batch, int64_t seq, int64_t d_in,
                         void *y, int32_t y_dtype, int64_t d_out, int32_t accumulate, int32_t rank,
                         const lithe_factors *factors, const lithe_routes *routes,
                         const float *mid_scale, float out_scale, const float *out_scale_vec,
                         void *workspace, int64_t workspace_bytes, void *stream);

/* Bytes of the static scratch lithe_lora_delta_noalloc uses on each GPU (held until the process
 * ends): the rank-r intermediate of up to 524,288 tokens at rank 16 with bf16 activations. */
#define LITHE_STATIC_SCRATCH_BYTES 16777216

/* No counterpart in the reference. For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): lithe_lora_delta with the
 * rank-r intermediate in a static device array of LITHE_STATIC_SCRATCH_BYTES per GPU instead of a
 * workspace. It calls no hipMalloc or hipFree. A call whose intermediate
 * (lithe_lora_workspace_bytes() - 256 bytes) exceeds the array returns LITHE_ERR_WORKSPACE before any
 * launch. err_flag (device int32, nullable) receives the in-kernel error bits of lithe_lora_delta's
 * error word (OR-ed in, never cleared). The array of the current device is shared by every call on
 * that device and keeps the last call's contents (nothing in it needs to start at zero): calls that
 * overlap in time on one GPU (other streams, other threads) race and must not be issued. */
int32_t lithe_lora_delta_noalloc(const void *x, int32_t x_dtype, int64_t n_batch, int64_t seq, int64_t d_in,
                                 void *y, int32_t y_dtype, int64_t d_out, int32_t accumulate, int32_t rank,
                                 const lithe_factors *factors, const lithe_routes *routes,
                                 const float *mid_scale, float out_scale, const float *out_scale_vec,
                                 int32_t *err_flag, void *stream);

/* Shared-input group: n_mod modules whose linears read the same x (the to_q / to_k / to_v
 * projections of a FLUX attention block, or add_q / add_k / add_v_proj). One shrink reads x once
 * and produces the rank-r intermediate of every module (mid = x [A_0; A_1; ...]^T, stacked as
 * rank groups), then the expand of every module updates y[m] (n_batch, seq, d_out[m]) exactly as
 * lithe_lora_delta would with out_scale[m] (no out_scale_vec): one launch for all of them when
 * the modules share one B index source and B table (bf16, packed indices), else one per module. Factors: n_mod INDEXED entries
 * that share one A index source (base, kind, levels, strides, n_slots; each module's A at its
 * own block_off) and one A value table; each module has its own B source and B table.
 * y, d_out, out_scale and factors are host arrays of n_mod entries (y[m] a device pointer).
 * ceil(rank / 16) * n_route <= 8. The shrink carries all modules in one workgroup per token tile
 * when n_mod * ceil(rank / 16) * n_route <= 8 and the call is large (bf16 x, >= 2,048 16-token
 * groups), else one workgroup per tile and module. Workspace: lithe_lora_workspace_bytes(n_batch, seq,
 * d_in, max d_out, rank, n_route * n_mod, x_dtype). LITHE_ERR_UNSUPPORTED if the A sources or
 * A tables differ, or a factor is DENSE.
 * Replaces three shared_codebook_lora_delta calls over one input (lithe/kernels/shared.py:197-263
 * via IndexLoRALinear.forward, lithe/kernels/layers.py:120-131), the q/k/v fusion of
 * wrap_index (serving/_common.py:294-311). */
int32_t lithe_lora_delta_shared_x(const void *x, int32_t x_dtype, int64_t n_batch, int64_t seq, int64_t d_in,
                                  int32_t n_mod, void *const *y, int32_t y_dtype, const int64_t *d_out,
                                  int32_t accumulate, int32_t rank, const lithe_factors *factors,
                                  const lithe_routes *routes, const float *mid_scale, const float *out_scale,
                                  void *workspace, int64_t workspace_bytes, void *stream);

/* One module of a grouped call: its input, its base output and where its factors sit in a slot. */
typedef struct lithe_module {
    const void *x;          /* device (n_batch, seq, d_in), 16-byte aligned */
    void *y;                /* device (n_batch, seq, d_out) */
    int64_t seq, d_in, d_out;
    int64_t a_block_off;    /* first block of the module's A (rank x d_in) in a slot of factors->a_idx */
    int64_t b_block_off;    /* first block of the module's B (d_out x rank) in a slot of factors->b_idx */
    float out_scale;        /* alpha / r of the module */
} lithe_module;

#define LITHE_MAX_GROUP_MODULES 8

/* Bytes of workspace lithe_lora_delta_grouped needs for these modules: a 256-byte head (the error
 * word, as for lithe_lora_workspace_bytes) and the rank-r intermediate of every distinct input. */
int64_t lithe_lora_grouped_workspace_bytes(int64_t n_batch, int32_t n_mod, const lithe_module *mods, int32_t rank,
                                           int32_t n_route, int32_t x_dtype);

/* The deltas of n_mod <= LITHE_MAX_GROUP_MODULES independent modules of one batch in one shrink launch
 * and one expand launch: module m updates mods[m].y exactly as lithe_lora_delta(mods[m].x, ...,
 * mods[m].y, ..., out_scale = mods[m].out_scale) would (no mid_scale, no out_scale_vec). Modules with
 * the same x, seq and d_in share one shrink over x (x read once, as lithe_lora_delta_shared_x).
 * Every module uses the same routes, rank and dtypes, and the same index sources and value tables
 * (factors: one INDEXED entry whose a_idx / b_idx block_off are ignored: each module's offsets come
 * from a_block_off / b_block_off). Decoded mode: one DENSE entry over stacked factors in the layout
 * lithe_decode_stacked writes (module m's A (n_dense, rank, d_in) at element n_dense * 64 *
 * a_block_off of dense_a, its B (n_dense, d_out, rank) at n_dense * 64 * b_block_off of dense_b; the
 * caller keeps them inside its buffers; no weight_sqrt / slot_scale). The launch plan is made for the whole grid, so the K split of a
 * module's shrink can differ from its lithe_lora_delta plan (the fp32 sums are then grouped
 * differently). Modules with seq == 0 are skipped. Outputs of two modules must not overlap
 * (LITHE_ERR_OVERLAP); an output may alias another module's input (every shrink ends before the
 * first expand starts).
 * Replaces the calls of independent IndexLoRALinear layers of one transformer block that a serving
 * step issues back to back (the image and text projections of a FLUX double block,
 * lithe/kernels/layers.py:120-131 via serving/_common.py:294-311), each of which launches its own
 * shrink and expand (lithe/kernels/shared.py:197-263). */
int32_t lithe_lora_delta_grouped(int32_t n_mod, const lithe_module *mods, int32_t x_dtype, int32_t y_dtype,
                                 int64_t n_batch, int32_t accumulate, int32_t rank, const lithe_factors *factors,
                                 const lithe_routes *routes, void *workspace, int64_t workspace_bytes, void *stream);

/* Reads the in-kernel error word of a workspace (slot id out of range, index > 511) into
 * *flags on the host; synchronises the stream. 0 = no error since the last clear. */
int32_t lithe_workspace_errors(const void *workspace, int32_t *flags, int32_t clear, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* LITHE_AMD_H */
