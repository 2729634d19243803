// Host-side entry points of liblithe_amd: version, status strings, host packing.
#include <stdint.h>

#include <algorithm>
#include <thread>
#include <vector>

#include "lithe_amd.h"

extern "C" int32_t lithe_abi_version(void) { return 1; }

extern "C" const char *lithe_status_string(int32_t code) {
    switch (code) {
        case LITHE_OK: return "ok";
        case LITHE_ERR_NULL: return "a required pointer is NULL";
        case LITHE_ERR_SHAPE: return "sizes are out of range or inconsistent";
        case LITHE_ERR_ALIGN: return "d_in and d_out * rank must be multiples of 64 and buffers 16-byte aligned";
        case LITHE_ERR_DTYPE: return "unsupported dtype or kind";
        case LITHE_ERR_RANGE: return "indices must be < 512 for 9-bit packing";
        case LITHE_ERR_WORKSPACE: return "workspace missing or too small";
        case LITHE_ERR_HIP: return "HIP launch failed";
        case LITHE_ERR_LEVELS: return "num_levels must be in [1, 4] and agree across sources";
        case LITHE_ERR_UNSUPPORTED: return "route weights and slot scales apply to indexed factors only";
        case LITHE_ERR_OVERLAP: return "two modules of a grouped call write overlapping outputs";
        default: return "unknown status";
    }
}

// Seven 9-bit fields per word, field j at bits [9j, 9j + 9); the last word is
// zero-padded. Range check first so a failing call writes nothing.
extern "C" int32_t lithe_pack9_host(const uint16_t *idx, int64_t n, uint64_t *words) {
    if (n < 0) return LITHE_ERR_SHAPE;
    if (n == 0) return LITHE_OK;
    if (!idx || !words) return LITHE_ERR_NULL;
    for (int64_t i = 0; i < n; ++i)
        if (idx[i] > 511) return LITHE_ERR_RANGE;
    const int64_t n_words = (n + 6) / 7;
    auto work = [&](int64_t w0, int64_t w1) {
        for (int64_t w = w0; w < w1; ++w) {
            uint64_t v = 0;
            const int64_t p0 = w * 7;
            const int m = (int)((n - p0) < 7 ? (n - p0) : 7);
            for (int j = 0; j < m; ++j) v |= (uint64_t)idx[p0 + j] << (9 * j);
            words[w] = v;
        }
    };
    const int64_t per = int64_t(1) << 20;
    unsigned hw = std::thread::hardware_concurrency();
    const int64_t nt = n_words < 2 * per ? 1 : std::min<int64_t>(hw ? hw : 1, (n_words + per - 1) / per);
    if (nt <= 1) {
        work(0, n_words);
        return LITHE_OK;
    }
    std::vector<std::thread> th;
    const int64_t chunk = (n_words + nt - 1) / nt;
    for (int64_t t = 0; t < nt; ++t) {
        const int64_t w0 = t * chunk, w1 = std::min(n_words, w0 + chunk);
        if (w0 < w1) th.emplace_back(work, w0, w1);
    }
    for (auto &t : th) t.join();
    return LITHE_OK;
}

// ---------------------------------------------------------------- ingest (.lithe stream -> residency words)
// Segment s of a layout is one factor of one module in residency order (module m: A = 2m, B = 2m + 1):
// table[3s] = first residency block, table[3s + 1] = its block count, table[3s + 2] = the factor's first
// element in the .lithe index stream (the A matrices of all modules, then the B matrices, each (L, n)
// row-major).
extern "C" int32_t lithe_ingest_table(int32_t n_modules, const int64_t *blocks_a, const int64_t *blocks_b,
                                      int32_t num_levels, int64_t *table) {
    if (n_modules < 0 || num_levels < 1 || num_levels > 4) return n_modules < 0 ? LITHE_ERR_SHAPE : LITHE_ERR_LEVELS;
    if (n_modules == 0) return LITHE_OK;
    if (!blocks_a || !blocks_b || !table) return LITHE_ERR_NULL;
    int64_t total_a = 0;
    for (int32_t m = 0; m < n_modules; ++m) {
        if (blocks_a[m] < 0 || blocks_b[m] < 0) return LITHE_ERR_SHAPE;
        total_a += blocks_a[m];
    }
    int64_t block = 0, off_a = 0, off_b = total_a * num_levels;
    for (int32_t m = 0; m < n_modules; ++m) {
        int64_t *ra = table + 6 * (int64_t)m, *rb = ra + 3;
        ra[0] = block;
        ra[1] = blocks_a[m];
        ra[2] = off_a;
        rb[0] = block + blocks_a[m];
        rb[1] = blocks_b[m];
        rb[2] = off_b;
        block += blocks_a[m] + blocks_b[m];
        off_a += blocks_a[m] * num_levels;
        off_b += blocks_b[m] * num_levels;
    }
    return LITHE_OK;
}

namespace {

// Index of the last segment whose first block is <= blk (segments sorted by first block).
int64_t find_segment(const int64_t *table, int32_t n_seg, int64_t blk) {
    int64_t lo = 0, hi = n_seg;    // invariant: table[3 lo] <= blk < table[3 hi]
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) / 2;
        if (table[3 * mid] <= blk) lo = mid;
        else hi = mid;
    }
    return lo;
}

// Checks that the table describes n_stream indices in contiguous residency order.
int32_t check_table(const int64_t *table, int32_t n_seg, int32_t num_levels, int64_t n_stream) {
    int64_t block = 0, total = 0;
    for (int32_t s = 0; s < n_seg; ++s) {
        const int64_t *r = table + 3 * (int64_t)s;
        if (r[0] != block || r[1] < 0 || r[2] < 0 || r[2] + r[1] * num_levels > n_stream) return LITHE_ERR_SHAPE;
        block += r[1];
        total += r[1] * num_levels;
    }
    return total == n_stream ? LITHE_OK : LITHE_ERR_SHAPE;
}

}  // namespace

extern "C" int32_t lithe_ingest_host(const uint16_t *stream, int64_t n_stream, int32_t num_levels, int32_t n_segments,
                                     const int64_t *table, uint64_t *words, int64_t n_words) {
    if (n_stream < 0 || n_segments < 1 || n_words < 0) return LITHE_ERR_SHAPE;
    if (num_levels < 1 || num_levels > 4) return LITHE_ERR_LEVELS;
    if (!stream || !table || !words) return n_stream == 0 ? LITHE_OK : LITHE_ERR_NULL;
    int32_t rc = check_table(table, n_segments, num_levels, n_stream);
    if (rc) return rc;
    if (n_words < (n_stream + 6) / 7) return LITHE_ERR_SHAPE;
    for (int64_t i = 0; i < n_stream; ++i)
        if (stream[i] > 511) return LITHE_ERR_RANGE;
    const int64_t need = (n_stream + 6) / 7;
    auto work = [&](int64_t w0, int64_t w1) {
        if (w0 >= w1) return;
        int64_t seg = find_segment(table, n_segments, (w0 * 7) / num_levels);
        for (int64_t w = w0; w < w1; ++w) {
            uint64_t v = 0;
            for (int k = 0; k < 7; ++k) {
                const int64_t p = w * 7 + k;
                if (p >= n_stream) break;
                const int64_t blk = p / num_levels, lvl = p - blk * num_levels;
                while (blk >= table[3 * seg] + table[3 * seg + 1]) ++seg;
                const int64_t *r = table + 3 * seg;
                v |= (uint64_t)stream[r[2] + lvl * r[1] + (blk - r[0])] << (9 * k);
            }
            words[w] = v;
        }
    };
    const int64_t per = int64_t(1) << 18;
    unsigned hw = std::thread::hardware_concurrency();
    const int64_t nt = need < 2 * per ? 1 : std::min<int64_t>(hw ? hw : 1, (need + per - 1) / per);
    if (nt <= 1) {
        work(0, need);
    } else {
        std::vector<std::thread> th;
        const int64_t chunk = (need + nt - 1) / nt;
        for (int64_t t = 0; t < nt; ++t) th.emplace_back(work, t * chunk, std::min(need, (t + 1) * chunk));
        for (auto &t : th) t.join();
    }
    for (int64_t w = need; w < n_words; ++w) words[w] = 0;
    return LITHE_OK;
}
