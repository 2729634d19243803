// Expand kernels for bf16 activations and bf16 outputs (one translation unit per dtype pair:
// parallel builds).
#include "lora_kernels.h"

namespace lithe {

void launch_expand_bf16_bf16(const Plan &p, const LoraArgs &a, int src, hipStream_t st) {
    if (src == SRC_DENSE) dispatch_expand<__bf16, __bf16, SRC_DENSE>(p, a, st);
    else if (src == SRC_PACKED) dispatch_expand<__bf16, __bf16, SRC_PACKED>(p, a, st);
    else dispatch_expand<__bf16, __bf16, SRC_INDEXED>(p, a, st);
}

bool launch_expand_group_bf16_bf16(int GM, int BOM, int NS, const GroupArgs &g, unsigned grid, size_t lds, int src,
                                   hipStream_t st) {
    if (src == SRC_PACKED) dispatch_expand_group<__bf16, __bf16, SRC_PACKED>(GM, BOM, NS, g, grid, lds, st);
    else if (src == SRC_DENSE) dispatch_expand_group<__bf16, __bf16, SRC_DENSE>(GM, BOM, NS, g, grid, lds, st);
    else return false;
    return true;
}

}  // namespace lithe
