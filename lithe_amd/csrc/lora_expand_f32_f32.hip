// Expand kernels for fp32 activations and fp32 outputs (one translation unit per dtype pair:
// parallel builds).
#include "lora_kernels.h"

namespace lithe {

void launch_expand_f32_f32(const Plan &p, const LoraArgs &a, int src, hipStream_t st) {
    if (src == SRC_DENSE) dispatch_expand<float, float, SRC_DENSE>(p, a, st);
    else if (src == SRC_PACKED) dispatch_expand<float, float, SRC_PACKED>(p, a, st);
    else dispatch_expand<float, float, SRC_INDEXED>(p, a, st);
}

}  // namespace lithe
