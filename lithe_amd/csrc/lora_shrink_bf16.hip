// Shrink kernels for bf16 activations (one translation unit per dtype: parallel builds).
#include "lora_kernels.h"

namespace lithe {

void launch_shrink_bf16(const Plan &p, const LoraArgs &a, int src, hipStream_t st) {
    if (src == SRC_DENSE) dispatch_shrink<__bf16, SRC_DENSE>(p, a, st);
    else if (src == SRC_PACKED) dispatch_shrink<__bf16, SRC_PACKED>(p, a, st);
    else dispatch_shrink<__bf16, SRC_INDEXED>(p, a, st);
}

bool launch_shrink_group_bf16(int GM, int TW, const GroupArgs &g, unsigned grid, size_t lds, int src, hipStream_t st) {
    if (src == SRC_PACKED) dispatch_shrink_group<__bf16, SRC_PACKED>(GM, TW, g, grid, lds, st);
    else if (src == SRC_DENSE) dispatch_shrink_group<__bf16, SRC_DENSE>(GM, TW, g, grid, lds, st);
    else return false;
    return true;
}

}  // namespace lithe
