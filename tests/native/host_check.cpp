// Sanitizer driver for the host half of liblithe_amd (lithe_amd/csrc/host.cpp): the 9-bit host
// packer and the .lithe-stream ingest, checked against direct restatements below on edge sizes,
// on sizes large enough for the threaded paths, and on their error paths. Built by
// tests/test_host_sanitized.py with AddressSanitizer + UndefinedBehaviorSanitizer and with
// ThreadSanitizer; exits non-zero on the first mismatch.
#include <stdint.h>
#include <stdio.h>

#include <random>
#include <vector>

#include "lithe_amd.h"

static int failures = 0;
#define CHECK(cond, ...)                                  \
    do {                                                  \
        if (!(cond)) {                                    \
            fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            fprintf(stderr, __VA_ARGS__);                 \
            fprintf(stderr, "\n");                        \
            ++failures;                                   \
        }                                                 \
    } while (0)

// index p of a stream at bits [9 (p % 7), +9) of word p / 7 (lithe/kernels/packed.py:38-52)
static std::vector<uint64_t> pack_direct(const std::vector<uint16_t> &v) {
    std::vector<uint64_t> w((v.size() + 6) / 7, 0);
    for (size_t p = 0; p < v.size(); ++p) w[p / 7] |= (uint64_t)v[p] << (9 * (p % 7));
    return w;
}

static void check_pack(std::mt19937_64 &rng) {
    for (int64_t n : {0L, 1L, 6L, 7L, 8L, 700L, 1001L, 14680071L}) {    // the last: 2,097,153 words, threaded
        std::vector<uint16_t> v(n);
        for (auto &x : v) x = (uint16_t)(rng() % 512);
        std::vector<uint64_t> got((n + 6) / 7 + 1, 0xABCDu);             // one guard word past the end
        CHECK(lithe_pack9_host(v.data(), n, got.data()) == LITHE_OK, "pack n=%ld", (long)n);
        const std::vector<uint64_t> want = pack_direct(v);
        for (size_t i = 0; i < want.size(); ++i) CHECK(got[i] == want[i], "pack n=%ld word %zu", (long)n, i);
        CHECK(got.back() == 0xABCDu, "pack n=%ld wrote past its words", (long)n);
    }
    std::vector<uint16_t> bad = {1, 2, 512, 3};
    std::vector<uint64_t> w(1, 77);
    CHECK(lithe_pack9_host(bad.data(), 4, w.data()) == LITHE_ERR_RANGE && w[0] == 77, "range error writes nothing");
    CHECK(lithe_pack9_host(nullptr, 4, w.data()) == LITHE_ERR_NULL, "null input");
    CHECK(lithe_pack9_host(bad.data(), -1, w.data()) == LITHE_ERR_SHAPE, "negative size");
}

// Residency order of one adapter: module m's A blocks then its B blocks, (block, level)-major;
// the .lithe stream holds every module's A matrix, then every B matrix, each (L, n) row-major
// (lithe/fileio.py:1-13, lithe/kernels/packed.py:125-133).
static std::vector<uint16_t> residency_direct(const std::vector<uint16_t> &stream, const std::vector<int64_t> &na,
                                              const std::vector<int64_t> &nb, int L) {
    std::vector<uint16_t> out;
    int64_t total_a = 0;
    for (int64_t a : na) total_a += a;
    int64_t off_a = 0, off_b = total_a * L;
    for (size_t m = 0; m < na.size(); ++m) {
        for (int64_t blk = 0; blk < na[m]; ++blk)
            for (int l = 0; l < L; ++l) out.push_back(stream[off_a + l * na[m] + blk]);
        for (int64_t blk = 0; blk < nb[m]; ++blk)
            for (int l = 0; l < L; ++l) out.push_back(stream[off_b + l * nb[m] + blk]);
        off_a += na[m] * L;
        off_b += nb[m] * L;
    }
    return out;
}

static void check_ingest(std::mt19937_64 &rng) {
    struct Case { int n_mod, L; int64_t max_blocks; };
    for (Case c : {Case{1, 3, 5}, Case{4, 1, 40}, Case{7, 4, 300}, Case{342, 3, 3840}}) {   // the last: FLUX-sized, threaded
        std::vector<int64_t> na(c.n_mod), nb(c.n_mod);
        int64_t n_idx = 0;
        for (int m = 0; m < c.n_mod; ++m) {
            na[m] = 1 + (int64_t)(rng() % c.max_blocks);
            nb[m] = (int64_t)(rng() % c.max_blocks);                       // a factor may be empty
            n_idx += (na[m] + nb[m]) * c.L;
        }
        std::vector<uint16_t> stream(n_idx);
        for (auto &x : stream) x = (uint16_t)(rng() % 512);
        std::vector<int64_t> table(3 * 2 * c.n_mod);
        CHECK(lithe_ingest_table(c.n_mod, na.data(), nb.data(), c.L, table.data()) == LITHE_OK, "table");
        const std::vector<uint64_t> want = pack_direct(residency_direct(stream, na, nb, c.L));
        std::vector<uint64_t> got(want.size() + 1, 0x5555u);
        CHECK(lithe_ingest_host(stream.data(), n_idx, c.L, 2 * c.n_mod, table.data(), got.data(),
                                (int64_t)want.size()) == LITHE_OK, "ingest %d modules", c.n_mod);
        for (size_t i = 0; i < want.size(); ++i) CHECK(got[i] == want[i], "ingest %d modules word %zu", c.n_mod, i);
        CHECK(got.back() == 0x5555u, "ingest wrote past its words");
        if (n_idx > 1) {
            stream[n_idx / 2] = 600;                                           // out of the 9-bit range
            std::vector<uint64_t> keep(want.size(), 9);
            CHECK(lithe_ingest_host(stream.data(), n_idx, c.L, 2 * c.n_mod, table.data(), keep.data(),
                                    (int64_t)keep.size()) == LITHE_ERR_RANGE && keep[0] == 9, "range error");
            CHECK(lithe_ingest_host(stream.data(), n_idx - 1, c.L, 2 * c.n_mod, table.data(), keep.data(),
                                    (int64_t)keep.size()) == LITHE_ERR_SHAPE, "short stream");
        }
    }
    std::vector<int64_t> neg = {-1}, one = {1}, table(6);
    CHECK(lithe_ingest_table(1, neg.data(), one.data(), 3, table.data()) == LITHE_ERR_SHAPE, "negative blocks");
    CHECK(lithe_ingest_table(1, one.data(), one.data(), 5, table.data()) == LITHE_ERR_LEVELS, "levels");
}

int main() {
    std::mt19937_64 rng(2024);
    check_pack(rng);
    check_ingest(rng);
    for (int32_t code = 0; code >= -10; --code) CHECK(lithe_status_string(code) != nullptr, "status %d", code);
    if (failures) {
        fprintf(stderr, "%d failure(s)\n", failures);
        return 1;
    }
    printf("host checks passed\n");
    return 0;
}
