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

KernelFn pick_linear_pipe_bf16(int nbt, int ks) {
    switch (nbt) {
    case 1: return pick_linear_pipe_ks<1>(ks);
    case 2: return pick_linear_pipe_ks<2>(ks);
    case 3: return pick_linear_pipe_ks<3>(ks);
    case 4: return pick_linear_pipe_ks<4>(ks);
    default: return nullptr;
    }
}

}  // namespace s3dx
