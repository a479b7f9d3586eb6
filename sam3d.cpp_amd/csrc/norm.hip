// Row ops around the sparse convolutions: LayerNorm (+affine, modulate,
// SiLU), SparseGroupNorm statistics, per-channel affine + SiLU, the SLat
// mean-pool downsample and nearest upsample, and dtype conversion.
//
// Reference: gb_layer_norm graph_builder.cpp:56-62 (ggml_norm, eps 1e-6 at
// slat_flow_graph.cpp:245-256), modulate slat_flow_graph.cpp:55-59,
// sparse_group_norm mesh_decoder_graph.cpp:16-30 (32 groups, eps 1e-5),
// downsample/upsample slat_flow_graph.cpp:157-190.
#include "common.hpp"

namespace s3dx {
namespace {

template <class T>
__device__ __forceinline__ float ld(const void *p, int64_t i) {
    return load_as_f32<T>(static_cast<const T *>(p) + i);
}
template <class T>
__device__ __forceinline__ void st(void *p, int64_t i, float v) {
    store_from_f32<T>(static_cast<T *>(p) + i, v);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) v += __shfl_xor(v, d, 64);
    return v;
}

// One wave per row; two passes over the row (mean, then centred variance).
template <class TI, class TO>
__global__ void __launch_bounds__(256)
layernorm_kernel(const void *x, int64_t n, int32_t c, float eps, const float *w, const float *b,
                 const float *ms, const float *mh, int32_t do_silu, void *y) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= n) return;
    const int64_t base = row * c;
    float s = 0.0f;
    for (int k = lane; k < c; k += 64) s += ld<TI>(x, base + k);
    const float mean = wave_sum(s) / static_cast<float>(c);
    float q = 0.0f;
    for (int k = lane; k < c; k += 64) {
        const float t = ld<TI>(x, base + k) - mean;
        q += t * t;
    }
    const float rstd = rsqrtf(wave_sum(q) / static_cast<float>(c) + eps);
    for (int k = lane; k < c; k += 64) {
        float t = (ld<TI>(x, base + k) - mean) * rstd;
        if (w) t *= w[k];
        if (b) t += b[k];
        if (ms) t = (t * ms[k] + t) + mh[k];
        if (do_silu) t = silu(t);
        st<TO>(y, base + k, t);
    }
}

template <class T>
__global__ void __launch_bounds__(256)
add_kernel(const void *a, const void *b, int64_t count, void *y) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride)
        st<T>(y, i, ld<T>(a, i) + ld<T>(b, i));
}

// GroupNorm statistics, pass 1 (centre == nullptr: plain sums) or pass 2
// (sums of squared deviations from the group mean).  Block (64 x 4): x over
// channels, y over rows; writes per-block per-channel partials.
constexpr int kStatBlocks = 512;
constexpr int kMaxChanPerThread = 16;  // c <= 1024

template <class T>
__global__ void __launch_bounds__(256)
gn_partial_kernel(const void *x, int64_t n, int32_t c, int32_t cg, const double *group_mean,
                  float *partials) {
    __shared__ float red[4][1024];
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const int64_t rows_per = (n + gridDim.x - 1) / gridDim.x;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * rows_per;
    const int64_t r1 = min(n, r0 + rows_per);
    float acc[kMaxChanPerThread];
    float centre[kMaxChanPerThread];
#pragma unroll
    for (int q = 0; q < kMaxChanPerThread; ++q) {
        acc[q] = 0.0f;
        const int ch = tx + q * 64;
        centre[q] = (group_mean && ch < c) ? static_cast<float>(group_mean[ch / cg]) : 0.0f;
    }
    for (int64_t r = r0 + ty; r < r1; r += 4) {
#pragma unroll
        for (int q = 0; q < kMaxChanPerThread; ++q) {
            const int ch = tx + q * 64;
            if (ch < c) {
                const float v = ld<T>(x, r * c + ch);
                if (group_mean) {
                    const float d = v - centre[q];
                    acc[q] += d * d;
                } else {
                    acc[q] += v;
                }
            }
        }
    }
#pragma unroll
    for (int q = 0; q < kMaxChanPerThread; ++q) {
        const int ch = tx + q * 64;
        if (ch < c) red[ty][ch] = acc[q];
    }
    __syncthreads();
    for (int ch = threadIdx.x; ch < c; ch += 256)
        partials[static_cast<int64_t>(blockIdx.x) * c + ch] =
            (red[0][ch] + red[1][ch]) + (red[2][ch] + red[3][ch]);
}

// Reduce partials over blocks per group (double), in a fixed order.
__global__ void __launch_bounds__(256)
gn_reduce_kernel(const float *partials, int nblocks, int32_t c, int32_t cg, int32_t groups,
                 double denom, double *group_out) {
    // one block per group
    const int g = blockIdx.x;
    if (g >= groups) return;
    __shared__ double red[256];
    double s = 0.0;
    const int items = nblocks * cg;
    for (int i = threadIdx.x; i < items; i += 256) {
        const int blk = i / cg, ch = g * cg + (i - (i / cg) * cg);
        s += static_cast<double>(partials[static_cast<int64_t>(blk) * c + ch]);
    }
    red[threadIdx.x] = s;
    __syncthreads();
    for (int d = 128; d > 0; d >>= 1) {
        if (threadIdx.x < d) red[threadIdx.x] += red[threadIdx.x + d];
        __syncthreads();
    }
    if (threadIdx.x == 0) group_out[g] = red[0] / denom;
}

__global__ void gn_finalize_kernel(const double *mean, const double *var, int32_t c, int32_t cg,
                                   float eps, const float *gamma, const float *beta, float *scale,
                                   float *shift) {
    const int ch = blockIdx.x * blockDim.x + threadIdx.x;
    if (ch >= c) return;
    const int g = ch / cg;
    const double rstd = 1.0 / sqrt(var[g] + static_cast<double>(eps));
    const double ga = gamma ? gamma[ch] : 1.0;
    const double be = beta ? beta[ch] : 0.0;
    scale[ch] = static_cast<float>(ga * rstd);
    shift[ch] = static_cast<float>(be - mean[g] * ga * rstd);
}

template <class TI, class TO>
__global__ void __launch_bounds__(256)
affine_kernel(const void *x, int64_t n, int32_t c, const float *scale, const float *shift,
              int32_t do_silu, void *y) {
    const int64_t count = n * c;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride) {
        const int ch = static_cast<int>(i % c);
        float t = ld<TI>(x, i) * scale[ch] + shift[ch];
        if (do_silu) t = silu(t);
        st<TO>(y, i, t);
    }
}

template <class T>
__global__ void __launch_bounds__(256)
downsample_kernel(const void *x, int64_t nf, int32_t c, const int32_t *children,
                  const float *inv_count, int64_t nc, void *y) {
    const int64_t count = nc * c;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride) {
        const int64_t r = i / c;
        const int ch = static_cast<int>(i - r * c);
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int32_t f = children[r * 8 + j];
            if (f >= 0 && f < nf) s += ld<T>(x, static_cast<int64_t>(f) * c + ch);
        }
        st<T>(y, i, s * inv_count[r]);
    }
}

template <class T>
__global__ void __launch_bounds__(256)
upsample_kernel(const void *coarse, int64_t nc, int32_t c, const int32_t *f2c, int64_t nf,
                void *y) {
    const int64_t count = nf * c;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride) {
        const int64_t r = i / c;
        const int ch = static_cast<int>(i - r * c);
        const int32_t src = f2c[r];
        st<T>(y, i, (src >= 0 && src < nc) ? ld<T>(coarse, static_cast<int64_t>(src) * c + ch) : 0.0f);
    }
}

template <class TI, class TO>
__global__ void __launch_bounds__(256) convert_kernel(const void *x, int64_t count, void *y) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride)
        st<TO>(y, i, ld<TI>(x, i));
}

unsigned grid_for(int64_t count) {
    const int64_t b = (count + 255) / 256;
    return static_cast<unsigned>(b < 1 ? 1 : (b > 16384 ? 16384 : b));
}

#define S3DX_DISPATCH2(XD, YD, KERNEL, ...)                                                  \
    do {                                                                                     \
        if ((XD) == S3DX_BF16 && (YD) == S3DX_BF16) KERNEL<uint16_t, uint16_t> __VA_ARGS__;  \
        else if ((XD) == S3DX_BF16) KERNEL<uint16_t, float> __VA_ARGS__;                     \
        else if ((YD) == S3DX_BF16) KERNEL<float, uint16_t> __VA_ARGS__;                     \
        else KERNEL<float, float> __VA_ARGS__;                                               \
    } while (0)

struct GnLayout {
    float *partials;
    double *mean, *var;
};
template <class W>
void gn_layout(W &w, int32_t c, int32_t groups, GnLayout *l) {
    if constexpr (std::is_same_v<W, Carver>) {
        l->partials = w.template take<float>(static_cast<uint64_t>(kStatBlocks) * c);
        l->mean = w.template take<double>(groups);
        l->var = w.template take<double>(groups);
    } else {
        w.template take<float>(static_cast<uint64_t>(kStatBlocks) * c);
        w.template take<double>(groups);
        w.template take<double>(groups);
    }
}

}  // namespace

void layernorm_rows_launch(const void *x, int32_t x_dtype, int64_t n, int32_t c, float eps,
                           const float *w, const float *b, const float *mod_scale,
                           const float *mod_shift, int32_t do_silu, void *y, int32_t y_dtype,
                           hipStream_t stream) {
    const unsigned blocks = static_cast<unsigned>((n + 3) / 4);
    S3DX_DISPATCH2(x_dtype, y_dtype, layernorm_kernel,
                   <<<blocks, 256, 0, stream>>>(x, n, c, eps, w, b, mod_scale, mod_shift, do_silu, y));
    launch_check("layernorm");
}

void add_rows_launch(const void *a, const void *b, int32_t dtype, int64_t count, void *y,
                     hipStream_t stream) {
    if (dtype == S3DX_BF16) add_kernel<uint16_t><<<grid_for(count), 256, 0, stream>>>(a, b, count, y);
    else add_kernel<float><<<grid_for(count), 256, 0, stream>>>(a, b, count, y);
    launch_check("add");
}

}  // namespace s3dx

using namespace s3dx;

extern "C" {

S3DX_API s3dx_status s3dx_layernorm_rows(const void *x, int32_t x_dtype, int64_t n, int32_t c,
                                         float eps, const float *w, const float *b,
                                         const float *mod_scale, const float *mod_shift,
                                         int32_t silu, void *y, int32_t y_dtype,
                                         s3dx_stream stream, char *error,
                                         uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(x && y, "NULL feature pointer");
        require(n > 0 && c > 0, "sizes must be positive");
        require_dtype(x_dtype);
        require_dtype(y_dtype);
        require((mod_scale == nullptr) == (mod_shift == nullptr),
                "modulate scale and shift must both be set");
        require(x != y || x_dtype == y_dtype, "in-place LayerNorm needs equal dtypes");
        layernorm_rows_launch(x, x_dtype, n, c, eps, w, b, mod_scale, mod_shift, silu, y, y_dtype,
                              as_stream(stream));
    });
}

S3DX_API s3dx_status s3dx_groupnorm_workspace_size(int64_t n, int32_t c, int32_t groups,
                                                   uint64_t *bytes, char *error,
                                                   uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(bytes != nullptr, "bytes is NULL");
        require(n > 0 && c > 0 && groups > 0 && c % groups == 0, "invalid GroupNorm shape");
        require(c <= 64 * kMaxChanPerThread, "GroupNorm supports at most 1024 channels");
        Sizer s;
        gn_layout(s, c, groups, nullptr);
        *bytes = s.used;
    });
}

S3DX_API s3dx_status s3dx_groupnorm_stats(const void *x, int32_t x_dtype, int64_t n, int32_t c,
                                          int32_t groups, float eps, const float *gamma,
                                          const float *beta, float *scale, float *shift,
                                          void *workspace, uint64_t workspace_bytes,
                                          s3dx_stream stream, char *error,
                                          uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(x && scale && shift && workspace, "NULL argument");
        require(n > 0 && c > 0 && groups > 0 && c % groups == 0, "invalid GroupNorm shape");
        require(c <= 64 * kMaxChanPerThread, "GroupNorm supports at most 1024 channels");
        require_dtype(x_dtype);
        const hipStream_t s = as_stream(stream);
        Carver w(workspace, workspace_bytes);
        GnLayout l;
        gn_layout(w, c, groups, &l);
        const int cg = c / groups;
        const double denom = static_cast<double>(n) * cg;
        const bool bf = x_dtype == S3DX_BF16;
        // pass 1: means
        if (bf) gn_partial_kernel<uint16_t><<<kStatBlocks, 256, 0, s>>>(x, n, c, cg, nullptr, l.partials);
        else gn_partial_kernel<float><<<kStatBlocks, 256, 0, s>>>(x, n, c, cg, nullptr, l.partials);
        launch_check("gn_partial");
        gn_reduce_kernel<<<groups, 256, 0, s>>>(l.partials, kStatBlocks, c, cg, groups, denom, l.mean);
        launch_check("gn_reduce");
        // pass 2: centred variance
        if (bf) gn_partial_kernel<uint16_t><<<kStatBlocks, 256, 0, s>>>(x, n, c, cg, l.mean, l.partials);
        else gn_partial_kernel<float><<<kStatBlocks, 256, 0, s>>>(x, n, c, cg, l.mean, l.partials);
        launch_check("gn_partial");
        gn_reduce_kernel<<<groups, 256, 0, s>>>(l.partials, kStatBlocks, c, cg, groups, denom, l.var);
        launch_check("gn_reduce");
        gn_finalize_kernel<<<(c + 255) / 256, 256, 0, s>>>(l.mean, l.var, c, cg, eps, gamma, beta,
                                                           scale, shift);
        launch_check("gn_finalize");
    });
}

S3DX_API s3dx_status s3dx_affine_rows(const void *x, int32_t x_dtype, int64_t n, int32_t c,
                                      const float *scale, const float *shift, int32_t silu,
                                      void *y, int32_t y_dtype, s3dx_stream stream, char *error,
                                      uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(x && y && scale && shift, "NULL argument");
        require(n > 0 && c > 0, "sizes must be positive");
        require_dtype(x_dtype);
        require_dtype(y_dtype);
        require(x != y || x_dtype == y_dtype, "in-place affine needs equal dtypes");
        S3DX_DISPATCH2(x_dtype, y_dtype, affine_kernel,
                       <<<grid_for(n * c), 256, 0, as_stream(stream)>>>(x, n, c, scale, shift, silu, y));
        launch_check("affine");
    });
}

S3DX_API s3dx_status s3dx_downsample_mean(const void *x, int32_t dtype, int64_t nf, int32_t c,
                                          const int32_t *children, const float *inv_count,
                                          int64_t nc, void *y, s3dx_stream stream, char *error,
                                          uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(x && y && children && inv_count, "NULL argument");
        require(nf > 0 && nc > 0 && c > 0, "sizes must be positive");
        require_dtype(dtype);
        const hipStream_t s = as_stream(stream);
        if (dtype == S3DX_BF16)
            downsample_kernel<uint16_t><<<grid_for(nc * c), 256, 0, s>>>(x, nf, c, children, inv_count, nc, y);
        else
            downsample_kernel<float><<<grid_for(nc * c), 256, 0, s>>>(x, nf, c, children, inv_count, nc, y);
        launch_check("downsample");
    });
}

S3DX_API s3dx_status s3dx_upsample_nearest(const void *coarse, int32_t dtype, int64_t nc,
                                           int32_t c, const int32_t *fine_to_coarse, int64_t nf,
                                           void *y, s3dx_stream stream, char *error,
                                           uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(coarse && y && fine_to_coarse, "NULL argument");
        require(nf > 0 && nc > 0 && c > 0, "sizes must be positive");
        require_dtype(dtype);
        const hipStream_t s = as_stream(stream);
        if (dtype == S3DX_BF16)
            upsample_kernel<uint16_t><<<grid_for(nf * c), 256, 0, s>>>(coarse, nc, c, fine_to_coarse, nf, y);
        else
            upsample_kernel<float><<<grid_for(nf * c), 256, 0, s>>>(coarse, nc, c, fine_to_coarse, nf, y);
        launch_check("upsample");
    });
}

S3DX_API s3dx_status s3dx_convert(const void *x, int32_t x_dtype, int64_t count, void *y,
                                  int32_t y_dtype, s3dx_stream stream, char *error,
                                  uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(x && y, "NULL argument");
        require(count > 0, "count must be positive");
        require_dtype(x_dtype);
        require_dtype(y_dtype);
        require(x != y || x_dtype == y_dtype, "in-place conversion needs equal dtypes");
        S3DX_DISPATCH2(x_dtype, y_dtype, convert_kernel,
                       <<<grid_for(count), 256, 0, as_stream(stream)>>>(x, count, y));
        launch_check("convert");
    });
}

}  // extern "C"
