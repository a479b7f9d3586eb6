// Submanifold sparse convolution: gather-GEMM with fused prologue/epilogue.
//
// Replaces the SLat conv lambda (slat_flow_graph.cpp:105-155: concat zero
// row -> get_rows im2col -> mul_mat -> + bias) and the mesh convolution lambda
// (mesh_decoder_graph.cpp:81-103: 27 x get_rows/mask/mul_mat/add, + bias).
// Both compute y[i] = b + sum_o W_o x[kmap[i][o]] with missing neighbours
// contributing zero; here it is one output-stationary implicit GEMM:
//
//   M = output rows (128 per workgroup, 32 per wave), N = Cout tile (32*NB),
//   K = sum over present offsets o of Cin.
//
// Per (offset, Cin chunk) the workgroup stages the weight chunk in LDS in the
// exact MFMA B-operand lane order (packed once at load time), each wave
// gathers its 32 rows' neighbour features straight into VGPRs as 16-byte
// loads (a missing neighbour is a zero fragment, no im2col buffer), and issues
// 32x32 MFMAs with FP32 accumulation.  Offsets that no row of the tile has
// are skipped.  The epilogue applies bias, optional LayerNorm (full row in
// the tile), modulate, SiLU and residual, and stores FP32 or BF16.
//
// Operand layouts of the 32x32 MFMAs (wave64, one block):
//   A (32 x K): lane l holds row l%32, k-group l/32;  B (K x 32): lane l holds
//   column l%32, k-group l/32;  D: lane l holds column l%32, register r holds
//   row 8*(r/4) + 4*(l/32) + r%4.
//   bf16 32x32x16: each lane carries 8 consecutive k (16 bytes).
//   f32  32x32x2 : each lane carries 1 k; four MFMAs consume one 16-byte
//                  fragment (channels s*8 + (l/32)*4 + j, j = 0..3), with the
//                  weight packed in the same permuted order.
#include "conv_kernels.hpp"

#include <algorithm>
#include <cstdio>

#include <cstdlib>
#include <memory>
#include <vector>

namespace s3dx {
namespace {

// ---------------------------------------------------------------------------
// Generic VALU path: any Cin/Cout.  64 x 64 output tile, 16-channel chunks
// staged in LDS, 4 x 4 outputs per thread.  Weights fp32 [kvol][cin][cout].
// LayerNorm is not fused here; the host runs it as a separate pass.
// ---------------------------------------------------------------------------
constexpr int kGM = 64, kGN = 64, kGK = 16;

template <class T>
__device__ __forceinline__ float load_input(const ConvArgs &a, int32_t j, int32_t c) {
    return load_as_f32<T>(static_cast<const T *>(a.x) + static_cast<int64_t>(j) * a.cin + c);
}

// ---------------------------------------------------------------------------
// Input transforms of the mesh upsample block (mesh_decoder_graph.cpp:16-38,
// 109-134), applied once per source element before the conv gathers it 27
// times: out[r] = SiLU((x[src(r)] + slot_offset[r & 7]) * scale + shift),
// src(r) = r >> 3 when the rows are the parents' children (slot offsets
// set), else r.  Each step is optional; rounded once to T, as storing the
// transformed tensor would round it.
// ---------------------------------------------------------------------------
struct XformArgs {
    const void *x;
    void *out;
    int64_t rows;  // output rows
    int32_t cin;
    int32_t children;  // output row r reads x row r >> 3 and adds slot_offset[r & 7]
    const float *slot_offset;
    const float *scale, *shift;
};

template <class T>
__device__ __forceinline__ float xform_one(const XformArgs &a, float v, int64_t r, int32_t c) {
    if (a.children) v += a.slot_offset[(r & 7) * a.cin + c];
    if (a.scale) v = silu(v * a.scale[c] + a.shift[c]);
    return v;
}

// 16-byte pieces (cin a multiple of the piece's element count): each
// thread takes pieces of a grid-stride sequence (32-bit indices: rows*cin
// pieces < 2^32 is checked by the host), reading the piece's per-channel
// scale / shift / slot offsets as float4 vectors.
template <class T>
__global__ void __launch_bounds__(256) xform_rows_kernel(XformArgs a) {
    constexpr int E = 16 / sizeof(T);
    const uint32_t ppr = static_cast<uint32_t>(a.cin) / E;
    const uint32_t total = static_cast<uint32_t>(a.rows) * ppr;
    for (uint32_t u = blockIdx.x * 256u + threadIdx.x; u < total; u += gridDim.x * 256u) {
        const uint32_t r = u / ppr;
        const int32_t c0 = static_cast<int32_t>(u - r * ppr) * E;
        const int64_t src = a.children ? (r >> 3) : r;
        const uint4 raw = *reinterpret_cast<const uint4 *>(static_cast<const T *>(a.x) + src * a.cin + c0);
        float v[E];
        if constexpr (E == 8) {
            const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                v[2 * k] = bf16_to_f32(static_cast<uint16_t>(w4[k] & 0xffffu));
                v[2 * k + 1] = bf16_to_f32(static_cast<uint16_t>(w4[k] >> 16));
            }
        } else {
            v[0] = __builtin_bit_cast(float, raw.x);
            v[1] = __builtin_bit_cast(float, raw.y);
            v[2] = __builtin_bit_cast(float, raw.z);
            v[3] = __builtin_bit_cast(float, raw.w);
        }
        auto load = [&](const float *p, float (&out)[E]) __attribute__((always_inline)) {
#pragma unroll
            for (int k = 0; k < E; k += 4) {
                const float4 q = *reinterpret_cast<const float4 *>(p + k);
                out[k] = q.x;
                out[k + 1] = q.y;
                out[k + 2] = q.z;
                out[k + 3] = q.w;
            }
        };
        if (a.children) {
            float so[E];
            load(a.slot_offset + (r & 7) * a.cin + c0, so);
#pragma unroll
            for (int k = 0; k < E; ++k) v[k] += so[k];
        }
        if (a.scale) {
            float sc[E], sh[E];
            load(a.scale + c0, sc);
            load(a.shift + c0, sh);
#pragma unroll
            for (int k = 0; k < E; ++k) v[k] = silu(v[k] * sc[k] + sh[k]);
        }
        uint4 o;
        if constexpr (E == 8) {
            uint32_t w4[4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                w4[k] = static_cast<uint32_t>(f32_to_bf16(v[2 * k])) | (static_cast<uint32_t>(f32_to_bf16(v[2 * k + 1])) << 16);
            o = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        } else {
            o = make_uint4(__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[1]),
                           __builtin_bit_cast(uint32_t, v[2]), __builtin_bit_cast(uint32_t, v[3]));
        }
        *reinterpret_cast<uint4 *>(static_cast<T *>(a.out) + static_cast<int64_t>(r) * a.cin + c0) = o;
    }
}

// Any cin: one element per thread.
template <class T>
__global__ void __launch_bounds__(256) xform_elems_kernel(XformArgs a) {
    const int64_t total = a.rows * a.cin;
    for (int64_t u = blockIdx.x * 256ll + threadIdx.x; u < total; u += gridDim.x * 256ll) {
        const int64_t r = u / a.cin;
        const int32_t c = static_cast<int32_t>(u - r * a.cin);
        const int64_t src = a.children ? (r >> 3) : r;
        const float v = xform_one<T>(a, load_as_f32<T>(static_cast<const T *>(a.x) + src * a.cin + c), r, c);
        if constexpr (sizeof(T) == 2) static_cast<uint16_t *>(a.out)[u] = f32_to_bf16(v);
        else static_cast<float *>(a.out)[u] = v;
    }
}

template <class T>
__global__ void __launch_bounds__(256) conv_generic_kernel(ConvArgs a) {
    __shared__ float As[kGK][kGM + 4];
    __shared__ float Bs[kGK][kGN + 4];
    __shared__ int32_t rows[kGM * kMaxKvol];
    __shared__ uint32_t omask;
    const int tid = threadIdx.x;
    const int tile = xcd_tile(blockIdx.x, gridDim.x);
    const int64_t m0 = static_cast<int64_t>(tile) * kGM;
    const int n0 = blockIdx.y * kGN;
    const int kvol = a.kvol;
    if (tid == 0) omask = 0;
    __syncthreads();
    uint32_t my_mask = 0;
    for (int idx = tid; idx < kGM * kvol; idx += 256) {
        const int r = idx / kvol, o = idx - r * kvol;
        const int64_t row = m0 + r;
        int64_t j = -1;
        if (row < a.n_out) j = a.kmap ? a.kmap[row * kvol + o] : row;
        const bool valid = j >= 0 && j < a.n_src;
        rows[idx] = valid ? static_cast<int32_t>(j >> a.row_shift) : -1;
        if (valid) my_mask |= 1u << o;
    }
    if (my_mask) atomicOr(&omask, my_mask);
    __syncthreads();
    const uint32_t mask = omask;

    const int ty = tid >> 4, tx = tid & 15;
    float acc[4][4] = {};
    const float *w = static_cast<const float *>(a.w);
    for (int o = 0; o < kvol; ++o) {
        if (!((mask >> o) & 1u)) continue;
        for (int c0 = 0; c0 < a.cin; c0 += kGK) {
            __syncthreads();
            {   // A: 64 rows x 16 channels, thread -> (row, 4 channels)
                const int r = tid >> 2, kq = (tid & 3) * 4;
                const int32_t j = rows[r * kvol + o];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int c = c0 + kq + e;
                    As[kq + e][r] = (j >= 0 && c < a.cin) ? load_input<T>(a, j, c) : 0.0f;
                }
            }
            {   // B: 16 channels x 64 columns
                const int k = tid >> 4, nq = (tid & 15) * 4;
                const int c = c0 + k;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int col = n0 + nq + e;
                    Bs[k][nq + e] = (c < a.cin && col < a.cout)
                                        ? w[(static_cast<int64_t>(o) * a.cin + c) * a.cout + col]
                                        : 0.0f;
                }
            }
            __syncthreads();
#pragma unroll
            for (int k = 0; k < kGK; ++k) {
                float av[4], bv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) av[i] = As[k][ty * 4 + i];
#pragma unroll
                for (int i = 0; i < 4; ++i) bv[i] = Bs[k][tx * 4 + i];
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) acc[i][jj] += av[i] * bv[jj];
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t row = m0 + ty * 4 + i;
        if (row >= a.n_out) continue;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int col = n0 + tx * 4 + jj;
            if (col >= a.cout) continue;
            float t = acc[i][jj] + (a.bias ? a.bias[col] : 0.0f);
            if (a.silu) t = silu(t);
            const int64_t off = row * a.cout + col;
            const int64_t roff = (row >> a.residual_shift) * a.cout + col;
            if (a.y_bf16) {
                if (a.residual) t += bf16_to_f32(static_cast<const uint16_t *>(a.residual)[roff]);
                static_cast<uint16_t *>(a.y)[off] = f32_to_bf16(t);
            } else {
                if (a.residual) t += static_cast<const float *>(a.residual)[roff];
                static_cast<float *>(a.y)[off] = t;
            }
        }
    }
}

}  // namespace

// LayerNorm / residual helpers for the generic path live in norm.hip.
void layernorm_rows_launch(const void *x, int32_t x_dtype, int64_t n, int32_t c, float eps,
                           const float *w, const float *b, const float *mod_scale,
                           const float *mod_shift, int32_t silu, void *y, int32_t y_dtype,
                           hipStream_t stream, const void *residual = nullptr, int32_t residual_shift = 0);
void convert_launch(const void *x, int32_t x_dtype, int64_t count, void *y, int32_t y_dtype,
                    hipStream_t stream);

}  // namespace s3dx

// ---------------------------------------------------------------------------
// Host side: the prepared layer object.
// ---------------------------------------------------------------------------
struct s3dx_conv {
    int32_t cin = 0, cout = 0, kvol = 0, dtype = 0;
    int32_t in_dtype = 0;  // dtype of x: the layer's, or BF16 rows into an FP32 layer
    int32_t cout_pad = 0;  // packed MFMA weight columns (whole 32-column blocks)
    bool mfma = false;
    int nb = 0, kc = 0;  // MFMA tiling
    void *w = nullptr;   // packed weights (device)
    // FP32 1x1 layers: the weights again as three BF16 terms, for BF16 input
    // rows on BF16 MFMAs (linear_split_kernel); nullptr for other shapes.
    void *w_split = nullptr;
    float *bias = nullptr;
    float *slot_offset = nullptr;
    bool gather_parent = false;
    const float *pre_scale = nullptr, *pre_shift = nullptr;  // caller-owned device
    bool ln = false, silu = false;
    bool residual_parent = false;  // residual has one row per 8 output rows
    float eps = 1e-6f;
    float *ln_w = nullptr, *ln_b = nullptr, *mod_scale = nullptr, *mod_shift = nullptr;
    // Per-run modulate (caller-owned device [cout]); replaces mod_scale/shift.
    const float *dmod_scale = nullptr, *dmod_shift = nullptr;
    bool weights_set = false;
    // Transformed input rows (slot offsets / affine + SiLU applied), grown on
    // demand by s3dx_conv_run; one buffer per layer object.
    mutable void *xin = nullptr;
    mutable int64_t xin_bytes = 0;
    // FP32 conv output ahead of a LayerNorm that runs as its own pass (the
    // output tile does not span the row), grown on demand like xin.
    mutable void *pre_ln = nullptr;
    mutable int64_t pre_ln_bytes = 0;
    // Stream-K launches: two FP32 128 x 128 tiles per run for the pieces
    // that are part of a tile, grown on demand like xin.
    mutable void *sk_part = nullptr;
    mutable int64_t sk_part_bytes = 0;

    bool transforms() const { return slot_offset != nullptr || pre_scale != nullptr; }

    ~s3dx_conv() {
        for (void *p : {w, w_split, static_cast<void *>(bias), static_cast<void *>(slot_offset),
                        static_cast<void *>(ln_w), static_cast<void *>(ln_b),
                        static_cast<void *>(mod_scale), static_cast<void *>(mod_shift), xin, pre_ln, sk_part})
            if (p) (void)hipFree(p);
    }
};

// A kernel map's gather plan (per 64-row tile: the distinct source rows and
// the slot table the halo kernel stages them by), for the source rows of one
// layer setup.
struct s3dx_gather_plan {
    void *d = nullptr;
    int rows = 64;         // tile height of the records (64 or 128)
    int64_t capacity = 0;  // output rows the allocation covers
    int64_t n_out = 0, n_src = 0;
    int32_t shift = 0;
    ~s3dx_gather_plan() {
        if (d) (void)hipFree(d);
    }
};

namespace s3dx {
namespace {

KernelFn tiling_kernel(int id, bool bf, int kc, bool xf) {
    if (id == 20 || id == 21) return bf && kc == 64 && !xf ? pick_halo_bf16(id == 20 ? 128 : 64) : nullptr;
    return bf ? pick_mfma_bf16(id, kc, xf) : pick_mfma_f32(id, kc, xf);
}

// Picks the workgroup tiling for nb 32-column blocks per workgroup.  The
// split-K kernel (each weight fragment loaded once per workgroup, straight
// into the one wave that uses it) is preferred whenever it is compiled for
// the shape, with 128-channel tasks (32- or 64-channel chunks joined) ahead
// of 64-channel ones; otherwise waves that own all 128 columns of a row (tiling 10)
// gather each row once and stream two tasks per stage, and two 32-row blocks
// per wave halve the LDS traffic per MFMA when that still leaves one
// workgroup per CU.  S3DX_CONV_TILING=<id> overrides (tuning).
// splitk_ok: the packed weights fit the split-K kernel's 32-bit buffer
// offsets (< 2 GiB).
// Task channels tiling `id` runs at for kc: tiling 11 takes at most 64
// (BF16) or 32 (FP32) channels, where its 128 x 128 tiles do not spill.
int tiling_kc(int id, bool bf, int kc, int cin) {
    const int cap = bf ? 64 : 32;
    return id == 11 && kc > cap && cin % cap == 0 ? cap : kc;
}

const Tiling *choose_tiling(int64_t n_out, int nb, int ntiles, bool bf, int kc, bool xf, bool splitk_ok, int cin) {
    auto usable = [&](const Tiling &t) {
        return t.cols() == nb * 32 && (splitk_ok || !t.splitk) && tiling_kernel(t.id, bf, tiling_kc(t.id, bf, kc, cin), xf);
    };
    if (const char *e = std::getenv("S3DX_CONV_TILING")) {
        const int id = std::atoi(e);
        for (const Tiling &t : kTilings)
            if (t.id == id && usable(t)) return &t;
    }
    auto blocks = [&](const Tiling &t) { return (n_out + t.rows() - 1) / t.rows() * ntiles; };
    const Tiling *best = nullptr;
    int best_rank = 1 << 30;
    for (const Tiling &t : kTilings) {
        if (!usable(t)) continue;
        int rank;
        if (t.id >= 17) continue;                 // 64-row tiles: chosen by plan_launch
        if (t.splitk) rank = t.id >= 15 ? 0 : 1;  // 128-channel tasks (chunks joined) first
        else if (t.wn == 1 && t.nbw == 4) rank = blocks(t) >= 192 ? 2 : 10;  // 32x128 wave tiles
        else if (t.mbw == 2) rank = blocks(t) >= 256 ? 3 : 20;
        else rank = 5;
        if (rank < best_rank) {
            best_rank = rank;
            best = &t;
        }
    }
    return best;
}

// Kernel choice of one launch, shared by s3dx_conv_run and s3dx_conv_plan.
struct LaunchPlan {
    bool mfma = false;      // MFMA kernel (else the generic VALU kernel)
    bool xf = false;        // 64-bit addressed gathers (source above 2 GiB)
    bool fused_ln = false;  // LayerNorm in the MFMA epilogue
    int nb = 0, kc = 0;     // 32-column blocks per workgroup, channels per task
    bool linear = false;    // the 1x1-layer kernel (weights resident in LDS)
    bool split = false;     // linear_split_kernel: BF16 rows, three-term BF16 weights
    bool pipe = false;      // linear_pipe_kernel: BF16 layer, BF16 output, no residual
    bool half_chunk = false;  // halo kernel with a last chunk of 32 channels (64-row tiles only)
    bool stream_k = false;    // the 8-wave kernel over equal runs of (group, tile, chunk) units
    int64_t sk_units = 0;     // (column group, tile, chunk) units of a stream-K launch
    int sk_groups = 0;        // its 128-column groups
    bool sk_splitk = false;   // the stream-K runs are the FP32 split-K kernel's (64-row tiles)
    unsigned smem = 0;      // dynamic LDS bytes
    unsigned threads = 256; // workgroup size
    const Tiling *tl = nullptr;
    KernelFn fn = nullptr;
    dim3 grid;
};

// Compute units of the current device (256 without one: a host-only query).
int64_t device_cus() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
        (void)hipGetLastError();
        return 256;
    }
    return cus;
}

// Workgroups of `threads` threads of `fn` with `smem` dynamic LDS that the device
// holds at once (at least one per CU).  Without a device (a host-only plan
// query) it assumes 256 CUs holding two each.
int64_t resident_blocks(KernelFn fn, unsigned smem, int threads = 256) {
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(fn), threads, smem) !=
            hipSuccess) {
        (void)hipGetLastError();
        return 512;
    }
    return static_cast<int64_t>(std::max(cus, 1)) * std::max(per_cu, 1);
}

// Channels per task for nb column blocks: the largest of 128 / 64 / 32 that
// divides cin and keeps one weight stage (kc x nb*32) within 32 KiB (FP32:
// at most 64); 0 if none.
int task_channels(int cin, int nb, bool bf) {
    for (int cand : {128, 64, 32})
        if (cin % cand == 0 && (bf || cand <= 64) && cand * nb * 32 * (bf ? 2 : 4) <= 32768) return cand;
    return cin % 32 == 0 ? 32 : 0;
}

// What the conv gathers from: the caller's rows, or the transformed rows the
// pre-pass writes (children when slot offsets are set), and the shift that
// turns a kmap entry into a row of it.
struct Source {
    int64_t rows = 0;   // rows of the gathered tensor
    int64_t n_src = 0;  // bound on kmap entries
    int32_t shift = 0;
    bool children = false, pre = false;
};

Source source_of(const s3dx_conv *conv, int64_t n_in) {
    Source src;
    src.children = conv->gather_parent && conv->slot_offset != nullptr;
    src.pre = conv->transforms();
    src.rows = src.children ? 8 * n_in : n_in;
    src.shift = conv->gather_parent && !src.children ? 3 : 0;
    src.n_src = conv->gather_parent ? 8 * n_in : n_in;
    return src;
}

// FP32 1x1 layers with Cin = 32, 64, 96 or 128 and at most 128 output
// columns keep their weights also as three BF16 terms (w_split): BF16 rows
// then run on BF16 MFMAs (linear_split_kernel).
bool has_split_terms(const s3dx_conv *conv) {
    return conv->dtype == S3DX_F32 && conv->mfma && conv->kvol == 1 && conv->cin % 16 == 0 &&
           pick_linear_split(conv->cout_pad / 32, conv->cin / 16) != nullptr;
}

// bf16_rows: x holds BF16 rows for an FP32 layer; only the linear kernels
// read them as they are (the caller converts them for any other plan).
// allow_pipe: the output is BF16 and there is no residual (the pipelined
// 1x1 kernel writes only that).
LaunchPlan plan_launch(const s3dx_conv *conv, int64_t x_bytes, int64_t n_out, bool aligned16,
                       bool bf16_rows = false, bool allow_pipe = true) {
    LaunchPlan p;
    const bool bf = conv->dtype == S3DX_BF16;
    p.mfma = conv->mfma && aligned16;
    if (p.mfma && conv->kvol == 1 && x_bytes < (int64_t(1) << 31)) {
        // 1x1 layer: every weight fragment fits in LDS -> the linear kernel.
        const int nbt = conv->cout_pad / 32;
        const int frags = conv->cin / (bf ? 16 : 8) * nbt * 64;
        KernelFn fn = bf ? pick_linear_bf16(nbt) : bf16_rows ? pick_linear_f32_bf16_rows(nbt) : pick_linear_f32(nbt);
        // BF16 rows into an FP32 layer whose weights have BF16 terms: one
        // wave per column block, a persistent grid over 32-row blocks.
        KernelFn split = bf16_rows && has_split_terms(conv) ? pick_linear_split(nbt, conv->cin / 16) : nullptr;
        if (split && !std::getenv("S3DX_CONV_TILING")) {
            p.linear = p.split = true;
            p.fn = split;
            p.nb = nbt;
            p.threads = 64 * nbt;
            p.grid = dim3(static_cast<unsigned>(std::min<int64_t>((n_out + 31) / 32, resident_blocks(split, 0, p.threads))));
            return p;
        }
        // BF16 layers with Cin = 64, 128, 192 or 256: the pipelined kernel,
        // persistent workgroups over the 32-row blocks.
        // Wider layers (a multiple of four column blocks): 128-column groups.
        const int pnb = nbt <= 4 ? nbt : nbt % 4 == 0 ? 4 : 0;
        KernelFn pipe = bf && allow_pipe && pnb && !conv->ln && conv->cin % 16 == 0 && conv->cout % 8 == 0 &&
                                n_out * conv->cout * 2 < (int64_t(1) << 31)
                            ? pick_linear_pipe_bf16(pnb, conv->cin / 16)
                            : nullptr;
        const int pfrags = conv->cin / 16 * pnb * 64;
        if (pipe && pfrags <= kLinearMaxFrags && !std::getenv("S3DX_CONV_TILING")) {
            p.linear = p.pipe = true;
            p.fn = pipe;
            p.nb = pnb;
            p.smem = static_cast<unsigned>(pfrags) * 16 + 4 * 8 * (pnb * 32 + 4) * 4;
            const int64_t groups = nbt / pnb;
            const int64_t per_group = std::max<int64_t>(1, resident_blocks(pipe, p.smem) / groups);
            p.grid = dim3(static_cast<unsigned>(std::min<int64_t>((n_out + 127) / 128, per_group)),
                          static_cast<unsigned>(groups));
            return p;
        }
        if (fn && frags <= kLinearMaxFrags && !std::getenv("S3DX_CONV_TILING")) {
            p.linear = true;
            p.fn = fn;
            p.nb = nbt;
            // weights, then 8 staged output rows of (nbt*32 + 4) floats per wave
            p.smem = static_cast<unsigned>(frags) * 16 + 4 * 8 * (nbt * 32 + 4) * 4;
            // One pass of resident workgroups: a second, partial pass would
            // cost a whole workgroup's time for a fraction of the rows.
            const int64_t wave_blocks = (n_out + 127) / 128;  // four 32-row blocks per workgroup pass
            p.grid = dim3(static_cast<unsigned>(std::min<int64_t>(wave_blocks, resident_blocks(fn, p.smem))));
            return p;
        }
    }
    if (p.mfma) {
        // Buffer-resource gathers address at most 2 GiB; larger inputs take
        // the XF=1 (64-bit addressed) variant.
        p.xf = x_bytes >= (int64_t(1) << 31);
        const int64_t w_bytes = static_cast<int64_t>(conv->kvol) * conv->cin * conv->cout_pad * (bf ? 2 : 4);
        const bool splitk_ok = w_bytes < (int64_t(1) << 31);
        // The whole row per workgroup (conv->nb) unless a narrower column
        // tile has a split-K kernel and no LayerNorm needs the full row:
        // then each column tile re-gathers A (from L2), but every weight
        // fragment is loaded once, straight into the wave that uses it.
        // S3DX_CONV_NB=<blocks> overrides (tuning).
        const int blocks = conv->cout_pad / 32;
        int forced = 0;
        if (const char *e = std::getenv("S3DX_CONV_NB")) forced = std::atoi(e);
        // S3DX_CONV_KC=<channels> overrides the task width where the layer
        // allows it (tuning).
        int forced_kc = 0;
        if (const char *e = std::getenv("S3DX_CONV_KC")) forced_kc = std::atoi(e);
        auto try_nb = [&](int nb) {
            int kc = task_channels(conv->cin, nb, bf);
            if (kc == 0) return false;
            if ((forced_kc == 32 || forced_kc == 64 || forced_kc == 128) && forced_kc <= kc &&
                conv->cin % forced_kc == 0)
                kc = forced_kc;
            const Tiling *t = choose_tiling(n_out, nb, blocks / nb, bf, kc, p.xf, splitk_ok, conv->cin);
            if (!t) return false;
            p.nb = nb;
            p.kc = tiling_kc(t->id, bf, kc, conv->cin);
            p.tl = t;
            return true;
        };
        const bool use_forced =
            forced > 0 && blocks % forced == 0 && (!conv->ln || forced * 32 == conv->cout) && try_nb(forced);
        if (!use_forced) {
            require(try_nb(conv->nb), "no MFMA kernel for this shape");
            // S3DX_CONV_TILING=18 (tuning, tests): its tasks are 64 channels.
            if (const char *e = std::getenv("S3DX_CONV_TILING"))
                if (std::atoi(e) == 18 && conv->cin % (bf ? 64 : 32) == 0 &&
                    tiling_kernel(18, bf, bf ? 64 : 32, p.xf) && p.nb == 4)
                    for (const Tiling &t : kTilings)
                        if (t.id == 18) {
                            p.tl = &t;
                            p.kc = bf ? 64 : 32;
                        }
            if (!p.tl->splitk && !conv->ln && conv->kvol == kMaxKvol) {
                const LaunchPlan whole = p;
                bool found = false;
                for (int nb : {4, 3, 2})
                    if (!found && nb < conv->nb && blocks % nb == 0 && try_nb(nb)) found = p.tl->splitk;
                if (!found) p = whole;
            }
            // 128-column tiles: 64-row tiles with two workgroups per CU
            // (tiling 18, half-width tasks) overlap one workgroup's gathers,
            // barriers and epilogue with the other's MFMAs, once there are at
            // least half as many 128-row tiles as CUs (config 2 ~5%).  (A
            // 128-channel-task variant spilled 16 VGPRs and ran the 128 ->
            // 1024 skip on 5,086 rows in 13.1 us against 11.1 us here.)
            if (p.tl->id == 11 && forced == 0 && !std::getenv("S3DX_CONV_TILING")) {
                const int64_t rt = (n_out + 127) / 128;
                const int64_t cus = device_cus(), tiles = rt * (blocks / p.nb);
                const int kc18 = bf ? 64 : 32;  // half-width tasks
                if (2 * tiles >= cus && conv->cin % kc18 == 0 && tiling_kernel(18, bf, kc18, p.xf)) {
                    for (const Tiling &t : kTilings)
                        if (t.id == 18) p.tl = &t;
                    p.kc = kc18;
                }
            }
            // (Tiling 11 runs 64-channel BF16 or 32-channel FP32 tasks, see
            // tiling_kc: the wider ones spilled 8-12 bytes a lane and ran no
            // faster -- FP32 1024 -> 1024 on 5,086 rows: 3,300 us either way.)
            // Joined-chunk 96-column tasks (15) over more 128-row tiles than
            // one pass over the CUs: the same kernel with 64-row tiles, two
            // workgroups per CU (19).
            if (p.tl->id == 15 && forced == 0 && !std::getenv("S3DX_CONV_TILING")) {
                const int64_t tiles = (n_out + 127) / 128 * (blocks / p.nb);
                if (tiles > device_cus() && tiling_kernel(19, bf, p.kc, p.xf))
                    for (const Tiling &t : kTilings)
                        if (t.id == 19) p.tl = &t;
            }
            // Few row tiles (small voxel sets): split-K runs one workgroup
            // per CU, so narrower column tiles that still fit in one pass
            // over the CUs finish sooner (each re-gathers A from L2).
            if (p.tl->splitk && !conv->ln && !std::getenv("S3DX_CONV_TILING")) {
                const int64_t rt = (n_out + 127) / 128;
                const int64_t cus = device_cus();
                if (rt * (blocks / p.nb) < cus) {
                    const LaunchPlan wide = p;
                    LaunchPlan best = p;
                    for (int nb : {3, 2, 1}) {
                        if (nb >= wide.nb || blocks % nb != 0 || rt * (blocks / nb) > cus) continue;
                        if (try_nb(nb) && p.tl->splitk) best = p;
                        p = wide;
                    }
                    p = best;
                    // FP32 32-column tiles: 32-row tiles (tiling 24) put several
                    // waves on each SIMD instead of one wave running every
                    // MFMA of a 128-row tile alone (the 64-channel sphere
                    // shell: 33.9 -> 24.7 us).
                    if (!bf && p.nb == 1 && tiling_kernel(24, bf, p.kc, p.xf))
                        for (const Tiling &t : kTilings)
                            if (t.id == 24) p.tl = &t;
                }
            }
        }
        // The halo-staged kernels for BF16 3x3x3 layers whose channels come
        // in 64-channel chunks and 128-column tiles: a tile stages each
        // distinct source row once per chunk into LDS and reads every weight
        // fragment once.  64-row tiles (tiling 21) by default, 128-row tiles
        // (tiling 20) with S3DX_CONV_HALO=128; S3DX_CONV_TILING=<other id> or
        // S3DX_CONV_HALO=0 keeps the kernels above (tuning, tests).  Layers
        // whose columns come in 96 but not 128 (the mesh decoder's 192 and
        // 96) take 64-row, 96-column tiles when no LayerNorm spans the row.
        // Cin 32 above a multiple of 64 (the mesh decoder's 96) can run the
        // 64-row kernel with a half-width last chunk, but only when tiling
        // 21 is forced: a 64-row tile of Cin 96 holds too little MFMA work
        // for its staging and four-way reduction, and the split-K kernel is
        // faster (96 -> 96 on 1.81M rows: 1,247 us against 1,443 us).
        {
            const char *te = std::getenv("S3DX_CONV_TILING");
            const char *he = std::getenv("S3DX_CONV_HALO");
            const int tid = te ? std::atoi(te) : 0;
            const bool allowed = te ? (tid == 20 || tid == 21) : !(he && std::atoi(he) == 0);
            // A LayerNorm the split-K tile could not fuse either (its tile
            // narrower than the row) runs as its own pass after the halo kernel.
            const bool ln_ok = !conv->ln || conv->cout == 128 || p.nb * 32 != conv->cout;
            const bool nb4 = blocks % 4 == 0 && ln_ok;
            const bool nb3 = !nb4 && blocks % 3 == 0 && !conv->ln && tid != 20 && !(he && std::atoi(he) == 128);
            const int want = tid == 20 || tid == 21 ? tid : (he && std::atoi(he) == 128 ? 20 : 21);
            const bool chunks_ok = conv->cin % 64 == 0 || (conv->cin % 32 == 0 && tid == 21);
            // (the halo kernels read the map through a buffer resource: under 2 GiB)
            const bool map_ok = n_out * kMaxKvol * 4 < (int64_t(1) << 31);
            if (allowed && bf && conv->kvol == kMaxKvol && chunks_ok && (nb4 || nb3) && !p.xf && splitk_ok && map_ok) {
                for (const Tiling &t : kTilings)
                    if (t.id == want) p.tl = &t;
                p.nb = nb3 ? 3 : 4;
                p.kc = 64;
                p.half_chunk = conv->cin % 64 != 0;
            }
        }
        p.fused_ln = conv->ln && p.nb * 32 == conv->cout;
        p.fn = p.tl->id == 21 && p.nb == 3 ? pick_halo_bf16(64, 3) : tiling_kernel(p.tl->id, bf, p.kc, p.xf);
        require(p.fn != nullptr, "no MFMA kernel for this shape");
        const int64_t mt = (n_out + p.tl->rows() - 1) / p.tl->rows();
        p.grid = dim3(static_cast<unsigned>(mt), static_cast<unsigned>(blocks / p.nb));
        // FP32 tiling 18 whose tiles do not fill whole passes at two
        // workgroups per CU: stream-K runs, two per CU.  The workgroups are
        // latency-bound, so a pass costs about the same however full it is
        // (1024 -> 1024 on 5,086 rows, 640 workgroups, ran 1.52x the time of
        // the 512 of 4,096 rows), and equal runs shorten even one pass
        // (2048 -> 128 on 442 tiles: 3,143 -> 2,824 us; no L2 penalty at
        // FP32's MFMA rate).  Tiles of at least 200 tasks (Cin 256 and up:
        // at 128 -> 128, 108 tasks a tile, the combine pass takes what the
        // balance gives) and half a pass of them at least, so that pieces
        // stay long.  S3DX_STREAM_K=0 turns it off.
        if (p.tl->id == 18 && !bf && p.kc == 32 && p.nb == 4 && !p.xf && conv->kvol == kMaxKvol) {
            const char *off = std::getenv("S3DX_STREAM_K");
            const int64_t wgs = mt * p.grid.y, ntf = int64_t(kMaxKvol) * (conv->cin / 32);
            int64_t runs = 2 * device_cus();
            bool forced = false;
            if (const char *e = std::getenv("S3DX_STREAM_K_RUNS")) {
                runs = std::atoi(e);
                forced = true;
            }
            const bool want = forced ? true : wgs % runs != 0 && 2 * wgs >= runs && ntf >= 200;
            if (!(off && std::atoi(off) == 0) && want && runs >= 1 && runs <= 65535 && wgs * ntf >= 2 * runs) {
                p.stream_k = true;
                p.sk_splitk = true;
                p.sk_groups = static_cast<int>(p.grid.y);
                p.sk_units = wgs * ntf;
                p.fn = pick_splitk_stream_k_f32();
                p.grid = dim3(static_cast<unsigned>(runs), 1);
            }
        }
    } else {
        p.grid = dim3(static_cast<unsigned>((n_out + kGM - 1) / kGM),
                      static_cast<unsigned>((conv->cout + kGN - 1) / kGN));
    }
    return p;
}

// Runs of a stream-K launch of the 8-wave kernel (one workgroup per CU)
// for a layer of Cin `cin` over `groups` 128-column groups, or 0 when whole
// tiles suit it: fewer than 8 chunks of 64 channels (a piece would carry a
// tile's fixed costs for little work), or no more tiles than CUs, or a tile
// count the CUs divide.  With every tile in one pass over the CUs, whole
// tiles walk the chunks in step, so an XCD's L2 holds one chunk's weights
// at a time; runs starting at scattered chunks make it hold them all
// (2048 -> 128 on 221 tiles: 289 us whole, 373 us in runs), which the
// CUs left idle do not repay.  S3DX_STREAM_K=0 turns it off;
// S3DX_STREAM_K_RUNS=<n> sets the run count (tests).
int stream_k_runs(int cin, int64_t n_out, int64_t groups) {
    if (const char *e = std::getenv("S3DX_STREAM_K"))
        if (std::atoi(e) == 0) return 0;
    const int64_t chunks = cin / 64;
    if (cin % 64 != 0 || chunks < 8) return 0;
    const int64_t tiles = (n_out + 127) / 128 * groups;
    int64_t runs = device_cus();
    bool forced = false;
    if (const char *e = std::getenv("S3DX_STREAM_K_RUNS")) {
        runs = std::atoi(e);
        forced = true;
    }
    if (runs < 1 || runs > 65535 || tiles * chunks < 2 * runs) return 0;
    if (!forced && (tiles <= runs || tiles % runs == 0)) return 0;
    return static_cast<int>(runs);
}

// A planned launch: the halo kernel of the plan's tile height in place of
// the unplanned halo kernel (64-row records: tiling 21 only; 128-row records:
// tilings 20 and 21, on the 8-wave kernel, in stream-K runs where those pay).
// Other launches are unchanged.
void apply_gather_plan(LaunchPlan &p, const s3dx_gather_plan *g, int64_t n_out, bool bf16_rows, int cin) {
    if (bf16_rows || !p.mfma || !p.tl || (p.tl->id != 20 && p.tl->id != 21)) return;
    if (g->rows == 64 && p.tl->id == 21) {
        p.fn = pick_halo_bf16_planned(64, p.nb);
    } else if (g->rows == 128 && p.nb == 4 && !p.half_chunk) {
        for (const Tiling &t : kTilings)
            if (t.id == 22) p.tl = &t;
        p.fn = pick_halo_bf16_planned(128);
        p.threads = kHalo8Threads;
        const int64_t tiles = (n_out + 127) / 128;
        p.grid = dim3(static_cast<unsigned>(tiles), p.grid.y);
        if (const int runs = stream_k_runs(cin, n_out, p.grid.y)) {
            p.fn = pick_halo8_stream_k();
            p.stream_k = true;
            p.sk_groups = static_cast<int>(p.grid.y);
            p.sk_units = tiles * p.grid.y * (cin / 64);
            p.grid = dim3(static_cast<unsigned>(runs), 1);
        }
    }
}

// Tile height of the gather plan for `conv`: 128-row records when the
// layer runs a halo kernel and 128-row tiles fill the CUs in one pass (one
// 8-wave workgroup per CU), else 64.  S3DX_PLAN_ROWS=64|128 forces it.
int gather_plan_rows(const s3dx_conv *conv, int64_t x_bytes, int64_t n_out) {
    if (const char *e = std::getenv("S3DX_PLAN_ROWS")) {
        const int r = std::atoi(e);
        if (r == 64 || r == 128) return r;
    }
    const LaunchPlan p = plan_launch(conv, x_bytes, n_out, true);
    if (!p.mfma || !p.tl || (p.tl->id != 20 && p.tl->id != 21) || p.nb != 4 || p.half_chunk) return 64;
    const int64_t tiles = (n_out + 127) / 128 * static_cast<int64_t>(p.grid.y);
    return tiles <= device_cus() || stream_k_runs(conv->cin, n_out, p.grid.y) ? 128 : 64;
}

float *upload_f32(const float *host, size_t count) {
    if (!host) return nullptr;
    void *d = nullptr;
    hip_check(hipMalloc(&d, count * sizeof(float)), "hipMalloc");
    const hipError_t e = hipMemcpy(d, host, count * sizeof(float), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(d);
        hip_check(e, "hipMemcpy");
    }
    return static_cast<float *>(d);
}

// A buffer the layer owns, at least `bytes` long.  Growing it waits for the
// stream's earlier work, which may still read the old one.
void *layer_buffer(void *&buf, int64_t &have, int64_t bytes, hipStream_t s) {
    if (bytes > have) {
        if (buf) {
            hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
            hip_check(hipFree(buf), "hipFree");
            buf = nullptr;
            have = 0;
        }
        hip_check(hipMalloc(&buf, static_cast<size_t>(bytes)), "hipMalloc");
        have = bytes;
    }
    return buf;
}

// The layer's transformed-input buffer.
void *transform_buffer(const s3dx_conv *conv, int64_t bytes, hipStream_t s) {
    return layer_buffer(conv->xin, conv->xin_bytes, bytes, s);
}

void replace(float *&slot, float *fresh) {
    if (slot) (void)hipFree(slot);
    slot = fresh;
}

inline float weight_at(const float *w, int32_t layout, int kvol, int cin, int cout, int o, int co,
                       int ci) {
    return layout == S3DX_WEIGHT_SLAT
               ? w[(static_cast<int64_t>(co) * kvol + o) * cin + ci]
               : w[(static_cast<int64_t>(o) * cout + co) * cin + ci];
}

inline float round_bf16(float v) { return bf16_to_f32(f32_to_bf16(v)); }

}  // namespace
}  // namespace s3dx

using namespace s3dx;

extern "C" {

S3DX_API s3dx_status s3dx_conv_create(int32_t cin, int32_t cout, int32_t kvol, int32_t dtype,
                                      s3dx_conv **out, char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(out != nullptr, "out is NULL");
        *out = nullptr;
        require(cin > 0 && cout > 0, "channel counts must be positive");
        require(cin <= 65536 && cout <= 65536, "channel counts above 65536");
        require(kvol == 27 || kvol == 1, "kvol must be 27 or 1");
        require_dtype(dtype);
        auto c = std::make_unique<s3dx_conv>();
        c->cin = cin;
        c->cout = cout;
        c->kvol = kvol;
        c->dtype = dtype;
        c->in_dtype = dtype;
        const bool bf = dtype == S3DX_BF16;
        // Column blocks per workgroup: the whole row when Cout <= 256 (so a
        // LayerNorm epilogue sees it), else 128-column tiles.  A Cout that
        // is not a multiple of 32 is padded to whole blocks with zero
        // weights; the epilogue stores only the real columns.
        int nb = 0;
        const int blocks = (cout + 31) / 32;
        if (blocks <= 8) {
            for (int cand : {8, 6, 4, 3, 2, 1})
                if (cand == blocks) nb = cand;
            if (nb == 0) nb = 1;  // 5 or 7 blocks: 32-column tiles
        } else {
            for (int cand : {4, 2, 1})
                if (nb == 0 && blocks % cand == 0) nb = cand;
        }
        c->cout_pad = blocks * 32;
        const int kc = nb != 0 ? task_channels(cin, nb, bf) : 0;
        c->mfma = kc != 0 && nb != 0;
        c->kc = kc;
        c->nb = nb;
        *out = c.release();
    });
}

S3DX_API void s3dx_conv_free(s3dx_conv *conv) { delete conv; }

S3DX_API s3dx_status s3dx_conv_set_weights(s3dx_conv *conv, const float *host_weight,
                                           int32_t layout, const float *host_bias, char *error,
                                           uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(conv && host_weight, "NULL argument");
        require(layout == S3DX_WEIGHT_SLAT || layout == S3DX_WEIGHT_MESH, "unknown weight layout");
        const int cin = conv->cin, cout = conv->cout, kvol = conv->kvol;
        const bool bf = conv->dtype == S3DX_BF16;
        std::vector<uint8_t> packed;
        if (conv->mfma) {
            // [o][k-step][col block][lane][16 bytes], the B-operand lane order.
            const int E = bf ? 8 : 4, CPK = 2 * E;
            const int ksteps = cin / CPK, nbtot = conv->cout_pad / 32;
            const size_t frags = static_cast<size_t>(kvol) * ksteps * nbtot * 64;
            packed.resize(frags * 16);
            size_t f = 0;
            for (int o = 0; o < kvol; ++o)
                for (int s = 0; s < ksteps; ++s)
                    for (int nbk = 0; nbk < nbtot; ++nbk)
                        for (int l = 0; l < 64; ++l, ++f) {
                            const int co = nbk * 32 + (l & 31);
                            uint8_t *dst = packed.data() + f * 16;
                            for (int e = 0; e < E; ++e) {
                                const int ci = s * CPK + (l >> 5) * E + e;
                                const float v = co < cout ? weight_at(host_weight, layout, kvol, cin, cout, o, co, ci)
                                                          : 0.0f;
                                if (bf) {
                                    const uint16_t h = f32_to_bf16(v);
                                    std::memcpy(dst + e * 2, &h, 2);
                                } else {
                                    std::memcpy(dst + e * 4, &v, 4);
                                }
                            }
                        }
        } else {
            // fp32 [o][cin][cout]; bf16 layers keep bf16-rounded values.
            packed.resize(static_cast<size_t>(kvol) * cin * cout * sizeof(float));
            float *dst = reinterpret_cast<float *>(packed.data());
            for (int o = 0; o < kvol; ++o)
                for (int ci = 0; ci < cin; ++ci)
                    for (int co = 0; co < cout; ++co) {
                        float v = weight_at(host_weight, layout, kvol, cin, cout, o, co, ci);
                        dst[(static_cast<size_t>(o) * cin + ci) * cout + co] = bf ? round_bf16(v) : v;
                    }
        }
        void *d = nullptr;
        hip_check(hipMalloc(&d, packed.size()), "hipMalloc weights");
        const hipError_t e = hipMemcpy(d, packed.data(), packed.size(), hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            (void)hipFree(d);
            hip_check(e, "hipMemcpy weights");
        }
        if (conv->w) (void)hipFree(conv->w);
        conv->w = d;
        if (conv->w_split) (void)hipFree(conv->w_split);
        conv->w_split = nullptr;
        const int nbtot = conv->cout_pad / 32;
        if (has_split_terms(conv)) {
            // [k-step of 16][col block][term][lane][8 BF16], the BF16 B-operand
            // lane order; term t+1 is the BF16 rounding of what terms 0..t
            // leave of the FP32 weight (each remainder is exact in FP32).
            std::vector<uint16_t> terms(static_cast<size_t>(cin) * nbtot * 32 * 3);
            size_t f = 0;
            for (int s16 = 0; s16 < cin / 16; ++s16)
                for (int nbk = 0; nbk < nbtot; ++nbk)
                    for (int t = 0; t < 3; ++t)
                        for (int l = 0; l < 64; ++l)
                            for (int e = 0; e < 8; ++e, ++f) {
                                const int co = nbk * 32 + (l & 31), ci = s16 * 16 + (l >> 5) * 8 + e;
                                float v = co < cout ? weight_at(host_weight, layout, 1, cin, cout, 0, co, ci) : 0.0f;
                                uint16_t h = f32_to_bf16(v);
                                for (int k = 0; k < t; ++k) {
                                    v -= bf16_to_f32(h);
                                    h = f32_to_bf16(v);
                                }
                                terms[f] = h;
                            }
            void *ds = nullptr;
            hip_check(hipMalloc(&ds, terms.size() * 2), "hipMalloc weight terms");
            const hipError_t es = hipMemcpy(ds, terms.data(), terms.size() * 2, hipMemcpyHostToDevice);
            if (es != hipSuccess) {
                (void)hipFree(ds);
                hip_check(es, "hipMemcpy weight terms");
            }
            conv->w_split = ds;
        }
        replace(conv->bias, upload_f32(host_bias, static_cast<size_t>(cout)));
        conv->weights_set = true;
    });
}

S3DX_API s3dx_status s3dx_conv_set_gather_parent(s3dx_conv *conv, int32_t enable,
                                                 const float *host_slot_offset, char *error,
                                                 uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(conv != nullptr, "conv is NULL");
        conv->gather_parent = enable != 0;
        replace(conv->slot_offset,
                enable ? upload_f32(host_slot_offset, static_cast<size_t>(8) * conv->cin) : nullptr);
    });
}

S3DX_API s3dx_status s3dx_conv_set_input_affine_silu(s3dx_conv *conv, const float *scale,
                                                     const float *shift, char *error,
                                                     uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(conv != nullptr, "conv is NULL");
        require((scale == nullptr) == (shift == nullptr), "scale and shift must both be set");
        conv->pre_scale = scale;
        conv->pre_shift = shift;
    });
}

S3DX_API s3dx_status s3dx_conv_set_layernorm(s3dx_conv *conv, int32_t enable, float eps,
                                             const float *host_weight, const float *host_bias,
                                             const float *host_mod_scale,
                                             const float *host_mod_shift, char *error,
                                             uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(conv != nullptr, "conv is NULL");
        require(eps >= 0.0f, "eps must be non-negative");
        require((host_mod_scale == nullptr) == (host_mod_shift == nullptr),
                "modulate scale and shift must both be set");
        const size_t c = static_cast<size_t>(conv->cout);
        conv->ln = enable != 0;
        conv->eps = eps;
        replace(conv->ln_w, enable ? upload_f32(host_weight, c) : nullptr);
        replace(conv->ln_b, enable ? upload_f32(host_bias, c) : nullptr);
        replace(conv->mod_scale, enable ? upload_f32(host_mod_scale, c) : nullptr);
        replace(conv->mod_shift, enable ? upload_f32(host_mod_shift, c) : nullptr);
        if (!enable) conv->dmod_scale = conv->dmod_shift = nullptr;
    });
}

S3DX_API s3dx_status s3dx_conv_set_modulate(s3dx_conv *conv, const float *scale, const float *shift,
                                            char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(conv != nullptr, "conv is NULL");
        require((scale == nullptr) == (shift == nullptr), "modulate scale and shift must both be set");
        require(scale == nullptr || conv->ln, "modulate needs the LayerNorm epilogue (s3dx_conv_set_layernorm)");
        conv->dmod_scale = scale;
        conv->dmod_shift = shift;
    });
}

S3DX_API s3dx_status s3dx_conv_set_silu(s3dx_conv *conv, int32_t enable, char *error,
                                        uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(conv != nullptr, "conv is NULL");
        conv->silu = enable != 0;
    });
}

S3DX_API s3dx_status s3dx_conv_set_residual_parent(s3dx_conv *conv, int32_t enable, char *error,
                                                   uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(conv != nullptr, "conv is NULL");
        conv->residual_parent = enable != 0;
    });
}

S3DX_API s3dx_status s3dx_conv_set_input_dtype(s3dx_conv *conv, int32_t dtype, char *error,
                                              uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(conv != nullptr, "conv is NULL");
        require_dtype(dtype);
        require(dtype == conv->dtype || (dtype == S3DX_BF16 && conv->dtype == S3DX_F32),
                "input dtype must be the layer's, or BF16 for an FP32 layer");
        conv->in_dtype = dtype;
    });
}

}  // extern "C"

namespace {

// The launch description behind s3dx_conv_plan and s3dx_conv_plan_planned.
void describe_launch(const s3dx_conv *conv, const s3dx_gather_plan *gplan, int64_t n_in, int64_t n_out, char *plan,
                     uint64_t plan_capacity) {
    {
        require(conv != nullptr, "conv is NULL");
        require(plan != nullptr && plan_capacity > 0, "plan buffer is empty");
        require(n_in > 0 && n_out > 0, "row counts must be positive");
        const Source src = source_of(conv, n_in);
        require(conv->kvol != 1 || n_out <= src.n_src,
                "n_out exceeds the input rows (kvol 1 without a map reads row i of x)");
        const bool bf16_rows = conv->in_dtype != conv->dtype;
        const int64_t x_bytes = src.rows * conv->cin * static_cast<int64_t>(dtype_size(conv->in_dtype));
        LaunchPlan p = plan_launch(conv, x_bytes, n_out, true, bf16_rows);
        const bool widen = bf16_rows && !p.linear;
        if (widen) p = plan_launch(conv, src.rows * conv->cin * 4, n_out, true);
        if (gplan) {
            require(gplan->n_out == n_out && gplan->n_src == src.n_src && gplan->shift == src.shift,
                    "gather plan was built for another map size or source rows");
            apply_gather_plan(p, gplan, n_out, bf16_rows, conv->cin);
        }
        const bool planned = gplan && (p.fn == pick_halo_bf16_planned(64) || p.fn == pick_halo_bf16_planned(128) ||
                                       p.fn == pick_halo_bf16_planned(64, 3) || p.stream_k);
        char text[256];
        const bool halo = p.mfma && !p.linear && p.tl->id >= 20 && p.tl->id <= 22;  // the halo-staged kernels
        char groups[16] = "";
        if (p.grid.y > 1) std::snprintf(groups, sizeof(groups), "x%u", p.grid.y);
        if (p.linear)
            std::snprintf(text, sizeof(text), "linear%s cols=%d ksteps=%d%s ln=%s grid=%u%s", p.pipe ? " pipe" : "",
                          p.nb * 32,
                          conv->cin / (conv->dtype == S3DX_BF16 || p.split ? 16 : 8),
                          p.split ? " terms=3" : "", conv->ln ? "separate" : "none", p.grid.x, groups);
        else if (p.mfma)
            std::snprintf(text, sizeof(text), "mfma tiling=%d%s%s%s rows=%d cols=%d kc=%d%s xf=%d ln=%s grid=%ux%u",
                          p.tl->id, p.tl->splitk ? " split-k" : "", halo ? " halo" : "",
                          p.stream_k ? " stream-k" : "", p.tl->rows(),
                          halo ? p.nb * 32 : p.tl->cols(), p.kc, p.half_chunk ? "+32" : "",
                          p.xf ? 1 : 0, conv->ln ? (p.fused_ln ? "fused" : "separate") : "none", p.grid.x,
                          p.grid.y);
        else
            std::snprintf(text, sizeof(text), "generic rows=%d cols=%d ln=%s grid=%ux%u", kGM, kGN,
                          conv->ln ? "separate" : "none", p.grid.x, p.grid.y);
        std::snprintf(plan, plan_capacity, "%s%s%s%s%s", bf16_rows ? (widen ? "in=bf16 pre=widen " : "in=bf16 ") : "",
                      src.pre ? (src.children ? "pre=children " : "pre=rows ") : "", src.shift ? "parent-rows " : "",
                      text, planned ? (gplan->rows == 128 ? " plan=128" : " plan=64") : "");
    }
}

}  // namespace

extern "C" {

S3DX_API s3dx_status s3dx_conv_plan(const s3dx_conv *conv, int64_t n_in, int64_t n_out, char *plan,
                                    uint64_t plan_capacity, char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] { describe_launch(conv, nullptr, n_in, n_out, plan, plan_capacity); });
}

S3DX_API s3dx_status s3dx_conv_plan_planned(const s3dx_conv *conv, const s3dx_gather_plan *gather_plan,
                                            int64_t n_in, int64_t n_out, char *plan, uint64_t plan_capacity,
                                            char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(gather_plan != nullptr, "gather plan is NULL");
        describe_launch(conv, gather_plan, n_in, n_out, plan, plan_capacity);
    });
}

}  // extern "C"

namespace {

void conv_run_impl(const s3dx_conv *conv, const s3dx_gather_plan *gplan, const void *x, int64_t n_in,
                   const int32_t *kmap, int64_t n_out, const void *residual, void *y, int32_t y_dtype,
                   s3dx_stream stream) {
    {
        require(conv != nullptr, "conv is NULL");
        require(conv->weights_set, "weights not set");
        require(x && y, "NULL feature pointer");
        require(kmap != nullptr || conv->kvol == 1, "kmap is NULL for kvol 27");
        require(n_in > 0 && n_out > 0, "row counts must be positive");
        require(n_out <= INT32_MAX, "n_out exceeds INT32_MAX");
        require_dtype(y_dtype);
        require(aligned(x, 16) && aligned(y, 4) && aligned(residual, 4), "misaligned buffer");
        const Source src = source_of(conv, n_in);
        require(src.n_src <= INT32_MAX, "input rows exceed INT32_MAX");
        require(kmap != nullptr || n_out <= src.n_src,
                "n_out exceeds the input rows (kvol 1 without a map reads row i of x)");
        const hipStream_t s = as_stream(stream);
        const bool bf = conv->dtype == S3DX_BF16;
        const bool bf16_rows = conv->in_dtype != conv->dtype;  // BF16 rows into an FP32 layer
        require(!(bf16_rows && src.pre), "BF16 input rows do not combine with input transforms");
        const int64_t x_bytes = src.rows * conv->cin * static_cast<int64_t>(dtype_size(conv->in_dtype));
        if (src.pre) {
            XformArgs xa{};
            xa.x = x;
            xa.out = transform_buffer(conv, x_bytes, s);
            xa.rows = src.rows;
            xa.cin = conv->cin;
            xa.children = src.children;
            xa.slot_offset = conv->slot_offset;
            xa.scale = conv->pre_scale;
            xa.shift = conv->pre_shift;
            // 16-byte pieces with 32-bit piece indices; else one element per thread.
            const bool vec = conv->cin % (bf ? 8 : 4) == 0 &&
                             src.rows * (conv->cin / (bf ? 8 : 4)) < (int64_t(1) << 32) &&
                             aligned(conv->pre_scale, 16) && aligned(conv->pre_shift, 16);
            const int64_t items = src.rows * (vec ? conv->cin / (bf ? 8 : 4) : conv->cin);
            const dim3 grid(static_cast<unsigned>(std::min<int64_t>((items + 255) / 256, 16384)));
            if (vec) {
                if (bf) hipLaunchKernelGGL(xform_rows_kernel<uint16_t>, grid, dim3(256), 0, s, xa);
                else hipLaunchKernelGGL(xform_rows_kernel<float>, grid, dim3(256), 0, s, xa);
            } else {
                if (bf) hipLaunchKernelGGL(xform_elems_kernel<uint16_t>, grid, dim3(256), 0, s, xa);
                else hipLaunchKernelGGL(xform_elems_kernel<float>, grid, dim3(256), 0, s, xa);
            }
            launch_check("conv_xform");
            x = xa.out;
        }
        ConvArgs a{};
        a.x = x;
        a.x_bytes = x_bytes;
        a.n_src = src.n_src;
        a.row_shift = src.shift;
        a.cin = conv->cin;
        a.kmap = kmap;
        a.n_out = n_out;
        a.kvol = conv->kvol;
        a.w = conv->w;  // linear_split_kernel: w_split, set below
        a.bias = conv->bias;
        a.cout = conv->cout;
        a.cout_pad = conv->cout_pad;
        a.residual = residual;
        a.residual_shift = conv->residual_parent ? 3 : 0;
        a.y = y;
        a.y_bf16 = y_dtype == S3DX_BF16;
        a.silu = conv->silu;
        a.eps = conv->eps;
        a.ln_w = conv->ln_w;
        a.ln_b = conv->ln_b;
        a.mod_scale = conv->dmod_scale ? conv->dmod_scale : conv->mod_scale;
        a.mod_shift = conv->dmod_scale ? conv->dmod_shift : conv->mod_shift;
        // The MFMA kernel reads the map and writes rows with 16-byte accesses.
        const bool aligned16 = aligned(kmap, 16) && aligned(y, 16) && aligned(residual, 16);
        LaunchPlan plan = plan_launch(conv, a.x_bytes, n_out, aligned16, bf16_rows,
                                      residual == nullptr && y_dtype == S3DX_BF16);
        if (bf16_rows && !plan.linear) {
            // Other kernels read the layer's dtype: the rows are widened
            // (exactly) once, into the layer's buffer.
            const int64_t count = src.rows * conv->cin;
            void *xw = transform_buffer(conv, count * 4, s);
            convert_launch(x, S3DX_BF16, count, xw, S3DX_F32, s);
            a.x = xw;
            a.x_bytes = count * 4;
            plan = plan_launch(conv, a.x_bytes, n_out, aligned16);
        }
        if (plan.split) a.w = conv->w_split;
        if (gplan) {
            require(gplan->n_out == n_out && gplan->n_src == src.n_src && gplan->shift == src.shift,
                    "gather plan was built for another map size or source rows");
            // Only the halo kernels read plans; other launches ignore it.
            apply_gather_plan(plan, gplan, n_out, bf16_rows, conv->cin);
            if (plan.fn == pick_halo_bf16_planned(64) || plan.fn == pick_halo_bf16_planned(128) ||
                plan.fn == pick_halo_bf16_planned(64, 3) || plan.stream_k)
                a.plan = gplan->d;
        }
        // A LayerNorm the epilogue cannot fuse runs as its own pass over the
        // conv's FP32 output (the layer's buffer), then modulate, SiLU and
        // the residual, rounded once to y_dtype as the fused epilogue does.
        const bool separate_ln = conv->ln && !(plan.mfma && plan.fused_ln);
        if (separate_ln) {
            a.y = layer_buffer(conv->pre_ln, conv->pre_ln_bytes, n_out * conv->cout * 4, s);
            a.y_bf16 = 0;
            a.silu = 0;
            a.residual = nullptr;
            a.ln = 0;
        }
        if (plan.mfma) {
            a.ln = plan.fused_ln;
            // The three-term kernel has an instantiation that reads a residual
            // (grid-stride over the same blocks, so the grid stands).
            if (plan.split && a.residual) plan.fn = pick_linear_split(plan.nb, conv->cin / 16, true);
            if (plan.stream_k) {
                a.sk_wgs = static_cast<int32_t>(plan.grid.x);
                a.sk_units = plan.sk_units;
                a.sk_partial = static_cast<float *>(layer_buffer(
                    conv->sk_part, conv->sk_part_bytes, static_cast<int64_t>(plan.grid.x) * 2 * 128 * 128 * 4, s));
            }
            hipLaunchKernelGGL(plan.fn, plan.grid, dim3(plan.threads), plan.smem, s, a);
            launch_check(plan.linear ? "conv_linear" : "conv_mfma");
            if (plan.stream_k && plan.sk_splitk) {
                launch_splitk_combine_f32(a, (n_out + 63) / 64, plan.sk_groups, s);
                launch_check("conv_splitk_combine");
            } else if (plan.stream_k) {
                launch_halo8_combine(a, (n_out + 127) / 128, plan.sk_groups, s);
                launch_check("conv_halo8_combine");
            }
        } else {
            a.ln = 0;
            if (bf) hipLaunchKernelGGL(conv_generic_kernel<uint16_t>, plan.grid, dim3(256), 0, s, a);
            else hipLaunchKernelGGL(conv_generic_kernel<float>, plan.grid, dim3(256), 0, s, a);
            launch_check("conv_generic");
        }
        if (separate_ln)
            layernorm_rows_launch(conv->pre_ln, S3DX_F32, n_out, conv->cout, conv->eps, conv->ln_w, conv->ln_b,
                                  a.mod_scale, a.mod_shift, conv->silu ? 1 : 0, y, y_dtype, s, residual,
                                  conv->residual_parent ? 3 : 0);
    }
}

}  // namespace

extern "C" {

S3DX_API s3dx_status s3dx_conv_run(const s3dx_conv *conv, const void *x, int64_t n_in,
                                   const int32_t *kmap, int64_t n_out, const void *residual,
                                   void *y, int32_t y_dtype, s3dx_stream stream, char *error,
                                   uint64_t error_capacity) {
    return boundary(error, error_capacity,
                    [&] { conv_run_impl(conv, nullptr, x, n_in, kmap, n_out, residual, y, y_dtype, stream); });
}

}  // extern "C"

namespace {

// Checks the arguments and enqueues the build of `p` (allocated for at least
// n_out rows) over `kmap`.
void gather_plan_build(s3dx_gather_plan *p, const s3dx_conv *conv, int64_t n_in, const int32_t *kmap,
                       int64_t n_out, s3dx_stream stream) {
    const Source src = source_of(conv, n_in);
    require(src.n_src <= INT32_MAX, "input rows exceed INT32_MAX");
    // (the build reads the map through a buffer resource: under 2 GiB)
    require(n_out * kMaxKvol * 4 < (int64_t(1) << 31), "kernel maps of 2 GiB or more have no gather plan");
    launch_gather_plan_build(p->rows, kmap, n_out, src.n_src, src.shift, p->d, as_stream(stream));
    launch_check("gather_plan_build");
    p->n_out = n_out;
    p->n_src = src.n_src;
    p->shift = src.shift;
}

void gather_plan_check(const s3dx_conv *conv, int64_t n_in, const int32_t *kmap, int64_t n_out) {
    require(conv != nullptr && kmap != nullptr, "NULL argument");
    require(conv->kvol == kMaxKvol, "gather plans are for 3x3x3 layers");
    require(n_in > 0 && n_out > 0 && n_out <= INT32_MAX, "row counts out of range");
    require(aligned(kmap, 16), "kmap must be 16-byte aligned");
}

}  // namespace

extern "C" {

S3DX_API s3dx_status s3dx_gather_plan_create(const s3dx_conv *conv, int64_t n_in, const int32_t *kmap,
                                             int64_t n_out, s3dx_stream stream, s3dx_gather_plan **out,
                                             char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(out != nullptr, "out is NULL");
        *out = nullptr;
        gather_plan_check(conv, n_in, kmap, n_out);
        const Source src = source_of(conv, n_in);
        auto p = std::make_unique<s3dx_gather_plan>();
        p->rows = gather_plan_rows(conv, src.rows * conv->cin * static_cast<int64_t>(dtype_size(conv->in_dtype)),
                                   n_out);
        const int64_t bytes =
            (n_out + p->rows - 1) / p->rows * (p->rows == 128 ? kGatherPlanRecord128 : kGatherPlanRecord);
        require(bytes < (int64_t(1) << 31), "map too large for a gather plan");
        hip_check(hipMalloc(&p->d, static_cast<size_t>(bytes)), "hipMalloc gather plan");
        p->capacity = n_out;
        gather_plan_build(p.get(), conv, n_in, kmap, n_out, stream);
        *out = p.release();
    });
}

S3DX_API void s3dx_gather_plan_free(s3dx_gather_plan *plan) { delete plan; }

S3DX_API s3dx_status s3dx_gather_plan_rebuild(s3dx_gather_plan *plan, const s3dx_conv *conv, int64_t n_in,
                                              const int32_t *kmap, int64_t n_out, s3dx_stream stream,
                                              char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(plan != nullptr, "plan is NULL");
        gather_plan_check(conv, n_in, kmap, n_out);
        require(n_out <= plan->capacity, "n_out exceeds the rows the plan was created for");
        gather_plan_build(plan, conv, n_in, kmap, n_out, stream);
    });
}

S3DX_API s3dx_status s3dx_kmap_subm3_planned(const int32_t *coords, int64_t n, int32_t missing_value,
                                             int32_t *kmap, s3dx_gather_plan *plan, const s3dx_conv *conv,
                                             void *workspace, uint64_t workspace_bytes, s3dx_stream stream,
                                             char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(coords != nullptr && aligned(coords, 16), "coords must be non-NULL and 16-byte aligned");
        require(n > 0 && n <= INT32_MAX / 27, "voxel count out of range");
        require(plan != nullptr && workspace != nullptr, "NULL argument");
        gather_plan_check(conv, n, kmap, n);
        require(!conv->gather_parent, "the layer gathers parent rows: its plan does not name the map's own rows");
        require(n <= plan->capacity, "n exceeds the rows the plan was created for");
        launch_kmap_plan(plan->rows, coords, n, missing_value, kmap, workspace, workspace_bytes, plan->d,
                         as_stream(stream));
        launch_check("kmap_plan");
        plan->n_out = n;
        plan->n_src = n;
        plan->shift = 0;
    });
}

S3DX_API s3dx_status s3dx_conv_run_planned(const s3dx_conv *conv, const s3dx_gather_plan *plan, const void *x,
                                           int64_t n_in, const int32_t *kmap, int64_t n_out, const void *residual,
                                           void *y, int32_t y_dtype, s3dx_stream stream, char *error,
                                           uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(plan != nullptr, "plan is NULL");
        conv_run_impl(conv, plan, x, n_in, kmap, n_out, residual, y, y_dtype, stream);
    });
}

}  // extern "C"
