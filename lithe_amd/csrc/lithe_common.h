// Device-side building blocks shared by the gfx950 kernels of liblithe_amd.
//
// Codeword arithmetic. The codebook of the reference (lithe/codebook.py:1-17, 59-63)
// is 3 c_k[t] = sum_{q<9} H[t, q] s_k[q] with H[t, q] = (-1)^popcount(t & q) and
// s_k[q] = +1 iff bit q of k is set. Writing m_t for the 9-bit mask whose bit q is
// [popcount(t & q) is even], each term is +1 exactly where bit q of k equals bit q
// of m_t, so 3 c_k[t] = 9 - 2 popcount((k ^ m_t) & 511). Because q < 16, m_t only
// depends on t mod 16: every codeword (and every decoded 64-value block) repeats
// with period 16. A pool value is then a 10-entry table lookup per level,
// value[l][popcount], which the host derives from the pool tensors it is given.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lithe_amd.h"

namespace lithe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBlock = 64;
// Launch limits: workgroups along x (and along y, where a launch uses it); larger problems are
// rejected with LITHE_ERR_SHAPE before any launch.
constexpr int64_t kMaxGridX = 0x7fffffff;
constexpr int64_t kMaxGridY = 65535;
constexpr int kMaxLevels = 4;
constexpr uint32_t kIndexMask = 0x1FFu;

// Error bits written to the workspace error word.
constexpr int32_t kErrSlot = 1;    // slot id outside [0, n_slots)
constexpr int32_t kErrIndex = 2;   // level-major index outside [0, 511]
constexpr int32_t kErrTable = 4;   // a segment table that maps a block outside the output

// m_t for t in [0, 16): bit q set iff popcount(t & q) is even (q in [0, 9)).
__host__ __device__ constexpr uint32_t sign_mask(uint32_t t) {
    uint32_t m = 0;
    for (uint32_t q = 0; q < 9; ++q) m |= ((__builtin_popcount(t & q) & 1u) ^ 1u) << q;
    return m;
}

// Flat, trivially copyable description of an index source (kernel argument).
struct IdxSrc {
    const void *base;
    int64_t slot_stride;
    int64_t level_stride;
    int64_t block_off;
    int64_t n_slots;
    int32_t kind;
    int32_t levels;
};

// Value tables of both sides (kernel argument, staged into LDS by each kernel).
struct Luts {
    float v[2][kMaxLevels][10];
};

// Raw index data of one block, loaded but not yet decoded: for PACKED9 the two uint64
// words that hold its L fields (possibly the same word twice), for the unpacked kinds
// the L integers (levels past L repeat level L - 1).
struct RawIdx {
    uint32_t v[4];
};

// Loads the raw index data of NQ blocks. The kind switch sits outside the block loop and
// every load is unconditional, so all NQ blocks' loads issue back to back and nothing
// waits for them until extract_indices() reads the registers.
// PK: the source is known to be PACKED9 (the kernels' fast path); no kind dispatch is emitted.
template <int NQ, bool PK = false, int LV = 0>
__device__ __forceinline__ void load_raw(const IdxSrc &s, const int64_t slot[NQ], const int64_t block[NQ],
                                         RawIdx r[NQ]) {
    const int L = LV > 0 ? LV : s.levels;
    switch (PK ? LITHE_IDX_PACKED9 : s.kind) {
        case LITHE_IDX_PACKED9:
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                // positions inside a slot fit 32 bits (the host checks slot_stride * 7 < 2^32),
                // so / 7 is a multiply-high, not a 64-bit division routine
                const uint64_t *w = static_cast<const uint64_t *>(s.base) + slot[q] * s.slot_stride;
                const uint32_t p0 = (uint32_t)(s.block_off + block[q]) * (uint32_t)L;
                const uint64_t lo = w[p0 / 7u];
                const uint64_t hi = w[(p0 + (uint32_t)L - 1u) / 7u];
                r[q].v[0] = (uint32_t)lo;
                r[q].v[1] = (uint32_t)(lo >> 32);
                r[q].v[2] = (uint32_t)hi;
                r[q].v[3] = (uint32_t)(hi >> 32);
            }
            break;
        case LITHE_IDX_LEVEL_I32:
#pragma unroll
            for (int q = 0; q < NQ; ++q)
#pragma unroll
                for (int l = 0; l < kMaxLevels; ++l)
                    r[q].v[l] = (uint32_t) static_cast<const int32_t *>(s.base)[
                        slot[q] * s.slot_stride + (l < L ? l : L - 1) * s.level_stride + s.block_off + block[q]];
            break;
        case LITHE_IDX_LEVEL_I16:
#pragma unroll
            for (int q = 0; q < NQ; ++q)
#pragma unroll
                for (int l = 0; l < kMaxLevels; ++l)
                    r[q].v[l] = (uint32_t)(int32_t) static_cast<const int16_t *>(s.base)[
                        slot[q] * s.slot_stride + (l < L ? l : L - 1) * s.level_stride + s.block_off + block[q]];
            break;
        default:  // LITHE_IDX_BLOCK_I16
#pragma unroll
            for (int q = 0; q < NQ; ++q)
#pragma unroll
                for (int l = 0; l < kMaxLevels; ++l)
                    r[q].v[l] = (uint32_t)(int32_t) static_cast<const int16_t *>(s.base)[
                        slot[q] * s.slot_stride + (s.block_off + block[q]) * L + (l < L ? l : L - 1)];
            break;
    }
}

// The L indices of block `block` from its raw data. Returns false when an index read from
// an unpacked source is out of range (it is then replaced by 0).
template <bool PK = false, int LV = 0>
__device__ __forceinline__ bool extract_indices(const IdxSrc &s, int64_t block, const RawIdx &r,
                                                uint32_t k[kMaxLevels]) {
    const int L = LV > 0 ? LV : s.levels;
    if (PK || s.kind == LITHE_IDX_PACKED9) {
        const uint32_t p0 = (uint32_t)(s.block_off + block) * (uint32_t)L;
        const uint32_t w0 = p0 / 7u;
        const uint64_t lo = (uint64_t)r.v[0] | ((uint64_t)r.v[1] << 32);
        const uint64_t hi = (uint64_t)r.v[2] | ((uint64_t)r.v[3] << 32);
#pragma unroll
        for (int l = 0; l < kMaxLevels; ++l) {
            const uint32_t p = p0 + (uint32_t)l;
            const uint32_t wq = p / 7u;
            const uint64_t word = (wq == w0) ? lo : hi;
            k[l] = l < L ? (uint32_t)(word >> (9u * (p - 7u * wq))) & kIndexMask : 0u;
        }
        return true;
    }
    bool ok = true;
#pragma unroll
    for (int l = 0; l < kMaxLevels; ++l) {
        uint32_t v = r.v[l];
        if (l < L && v > kIndexMask) {   // negative values wrap above 511 as well
            ok = false;
            v = 0;
        }
        k[l] = l < L ? v : 0u;
    }
    return ok;
}

// The L indices of block `block` of slot `slot` (load_raw + extract_indices for one block).
__device__ __forceinline__ bool fetch_indices(const IdxSrc &s, int64_t slot, int64_t block,
                                              uint32_t k[kMaxLevels]) {
    RawIdx r[1];
    const int64_t sl[1] = {slot}, bl[1] = {block};
    load_raw<1>(s, sl, bl, r);
    return extract_indices(s, block, r[0], k);
}

// Decoded value at period position t (mask m = sign_mask(t)) from the L indices,
// summed in level order in fp32: (v0 + v1) + v2 (+ v3). LV > 0 fixes L = LV at compile
// time (branch-free: every table lookup of a block can be in flight at once); LV = 0 reads L.
template <int LV = 0>
__device__ __forceinline__ float decode_value(const float *lut /* [levels][10] in LDS */, int L,
                                              const uint32_t k[kMaxLevels], uint32_t m) {
    float v = lut[__builtin_popcount((k[0] ^ m) & kIndexMask)];
#pragma unroll
    for (int l = 1; l < kMaxLevels; ++l)
        if (LV > 0 ? l < LV : l < L) v += lut[l * 10 + __builtin_popcount((k[l] ^ m) & kIndexMask)];
    return v;
}

// The values at period positions t and t + 8 (t < 8). sign_mask(t + 8) = sign_mask(t) ^ 0x100 and
// bit 8 of sign_mask(t) is set, so per level popcount((k ^ m_{t+8}) & 511) is the position-t count
// plus 1 when bit 8 of k is set and minus 1 when it is clear (the count stays in [0, 9]): one table
// offset per level and index replaces the second xor and popcount. Same table entries, same fp32
// order as two decode_value calls.
template <int LV = 0>
__device__ __forceinline__ void decode_value_pair(const float *lut, int L, const uint32_t k[kMaxLevels], uint32_t m,
                                                  float &lo, float &hi) {
    int pc = __builtin_popcount((k[0] ^ m) & kIndexMask);
    int d = (int)((k[0] >> 8) & 1u) * 2 - 1;
    lo = lut[pc];
    hi = lut[pc + d];
#pragma unroll
    for (int l = 1; l < kMaxLevels; ++l)
        if (LV > 0 ? l < LV : l < L) {
            pc = __builtin_popcount((k[l] ^ m) & kIndexMask);
            d = (int)((k[l] >> 8) & 1u) * 2 - 1;
            lo += lut[l * 10 + pc];
            hi += lut[l * 10 + d + pc];
        }
}
static_assert((sign_mask(0) ^ 0x100u) == sign_mask(8) && (sign_mask(3) ^ 0x100u) == sign_mask(11) &&
                  (sign_mask(7) ^ 0x100u) == sign_mask(15) && (sign_mask(5) & 0x100u) != 0,
              "positions t and t + 8 differ in bit 8 of the sign mask only");

// ---------------------------------------------------------------- dtype helpers
template <typename T> struct DT;
template <> struct DT<__bf16> {
    static constexpr int bytes = 2;
    __device__ static __forceinline__ __bf16 from_f32(float f) { return (__bf16)f; }
    __device__ static __forceinline__ float to_f32(__bf16 v) { return (float)v; }
    __device__ static __forceinline__ float round(float f) { return (float)(__bf16)f; }
};
template <> struct DT<float> {
    static constexpr int bytes = 4;
    __device__ static __forceinline__ float from_f32(float f) { return f; }
    __device__ static __forceinline__ float to_f32(float v) { return v; }
    __device__ static __forceinline__ float round(float f) { return f; }
};

// Orders the LDS accesses of one wave around a cross-lane exchange: every access before it (in
// program order) is complete and visible to the other lanes of the wave before any access after
// it. The LDS executes one wave's accesses in order, so this costs no wait; it keeps the compiler
// from moving a lane's accesses across the exchange point.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ void record_error(int32_t *err, int32_t bits) {
    if (err) __hip_atomic_fetch_or(err, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace lithe
