/*
 * CPU oracle, C restatement (test infrastructure only; never linked into the
 * product library). Independent of the numpy restatement in oracle/*.py so
 * the two check each other bit for bit.
 *
 *   lo_pack9      lithe/kernels/packed.py:38-52   seven 9-bit fields per uint64
 *   lo_unpack9    lithe/kernels/packed.py:55-60
 *   lo_decode     lithe/kernels/packed.py:241-250 gather rows of the fp32 pool of the
 *                                                 block's side, sum levels in order
 *   lo_bf16       torch's fp32 -> bf16 cast (round to nearest even)
 *
 * Paths are relative to the reference repository root.
 */
#include <stdint.h>
#include <string.h>

int lo_pack9(const uint16_t *idx, int64_t n, uint64_t *words) {
    int64_t n_words = (n + 6) / 7;
    for (int64_t i = 0; i < n; ++i)
        if (idx[i] > 511) return -1;
    for (int64_t w = 0; w < n_words; ++w) {
        uint64_t v = 0;
        for (int j = 0; j < 7; ++j) {
            int64_t p = w * 7 + j;
            if (p < n) v |= (uint64_t)idx[p] << (9 * j);
        }
        words[w] = v;
    }
    return 0;
}

void lo_unpack9(const uint64_t *words, int64_t n, int64_t *out) {
    for (int64_t p = 0; p < n; ++p)
        out[p] = (int64_t)((words[p / 7] >> (9 * (p % 7))) & 0x1FFu);
}

static uint16_t bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

void lo_bf16(const float *in, uint16_t *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = bf16_rne(in[i]);
}

/* words: packed stream of one adapter; sides: 0 = A, 1 = B per block (NULL = all A);
 * pools (L, 512, 64) fp32 row-major; out_f32 (n_blocks, 64) or out_bf16 (either may be NULL). */
void lo_decode(const uint64_t *words, int64_t n_blocks, int levels, const int8_t *sides,
               const float *pool_a, const float *pool_b, float *out_f32, uint16_t *out_bf16) {
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < n_blocks; ++b) {
        const float *pool = (sides && sides[b]) ? pool_b : pool_a;
        float acc[64];
        for (int l = 0; l < levels; ++l) {
            int64_t p = b * levels + l;
            uint32_t k = (uint32_t)((words[p / 7] >> (9 * (p % 7))) & 0x1FFu);
            const float *row = pool + ((int64_t)l * 512 + k) * 64;
            for (int t = 0; t < 64; ++t) acc[t] = (l == 0) ? row[t] : acc[t] + row[t];
        }
        for (int t = 0; t < 64; ++t) {
            if (out_f32) out_f32[b * 64 + t] = acc[t];
            if (out_bf16) out_bf16[b * 64 + t] = bf16_rne(acc[t]);
        }
    }
}
