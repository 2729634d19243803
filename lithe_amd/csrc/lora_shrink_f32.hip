// Shrink kernels for fp32 activations (one translation unit per dtype: parallel builds).
#include "lora_kernels.h"

namespace lithe {

void launch_shrink_f32(const Plan &p, const LoraArgs &a, int src, hipStream_t st) {
    if (src == SRC_DENSE) dispatch_shrink<float, SRC_DENSE>(p, a, st);
    else if (src == SRC_PACKED) dispatch_shrink<float, SRC_PACKED>(p, a, st);
    else dispatch_shrink<float, SRC_INDEXED>(p, a, st);
}

}  // namespace lithe
