// BF16 instantiations of the MFMA sparse-convolution kernel
// (v_mfma_f32_32x32x16_bf16, FP32 accumulation).
#include "conv_kernels.hpp"

namespace s3dx {

KernelFn pick_mfma_bf16(int id, int kc, bool xf) {
    switch (kc) {
    case 128: return pick_kc<uint16_t, 128>(id, xf);
    case 64: return pick_kc<uint16_t, 64>(id, xf);
    case 32: return pick_kc<uint16_t, 32>(id, xf);
    default: return nullptr;
    }
}

KernelFn pick_linear_bf16(int nbt) { return pick_linear<uint16_t>(nbt); }

}  // namespace s3dx
