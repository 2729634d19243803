// Host-side entry points of liblithe_amd: version, status strings, host packing.
#include <stdint.h>

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
