// FP32 instantiations of the MFMA sparse-convolution kernel
// (v_mfma_f32_32x32x2f32).
#include "conv_kernels.hpp"

namespace s3dx {

KernelFn pick_mfma_f32(int id, int kc, bool xf) {
    switch (kc) {
    case 64: return pick_kc<float, 64>(id, xf);
    case 32: return pick_kc<float, 32>(id, xf);
    default: return nullptr;
    }
}

KernelFn pick_splitk_stream_k_f32() { return conv_splitk_sk_kernel<float, 4, 32, 0, 1, 2>; }

void launch_splitk_combine_f32(const ConvArgs &a, int64_t tiles, int groups, hipStream_t stream) {
    hipLaunchKernelGGL(HIP_KERNEL_NAME(splitk_combine_kernel<float, 4, 32, 2>),
                       dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(groups)), dim3(256), 0, stream, a);
}

KernelFn pick_linear_f32(int nbt) { return pick_linear<float>(nbt); }

KernelFn pick_linear_f32_bf16_rows(int nbt) { return pick_linear<float, true>(nbt); }

KernelFn pick_linear_split(int nbt, int ksx, bool residual) {
    switch (nbt) {
    case 1: return residual ? pick_linear_split_ks<1, true>(ksx) : pick_linear_split_ks<1, false>(ksx);
    case 2: return residual ? pick_linear_split_ks<2, true>(ksx) : pick_linear_split_ks<2, false>(ksx);
    case 3: return residual ? pick_linear_split_ks<3, true>(ksx) : pick_linear_split_ks<3, false>(ksx);
    case 4: return residual ? pick_linear_split_ks<4, true>(ksx) : pick_linear_split_ks<4, false>(ksx);
    default: return nullptr;
    }
}

}  // namespace s3dx
