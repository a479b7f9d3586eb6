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
#include "common.hpp"

#include <memory>
#include <vector>

namespace s3dx {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct ConvArgs {
    const void *x;
    int64_t n_src;  // rows addressable through the kmap (8 * parents when gathering parents)
    int32_t cin;
    const int32_t *kmap;
    int64_t n_out;
    int32_t kvol;
    const void *w;
    const float *bias;
    int32_t cout;
    const void *residual;
    void *y;
    int32_t y_bf16;
    int32_t gather_parent;
    const float *slot_offset;
    const float *pre_scale;
    const float *pre_shift;
    int32_t ln;
    float eps;
    const float *ln_w;
    const float *ln_b;
    const float *mod_scale;
    const float *mod_shift;
    int32_t silu;
};

constexpr int kBM = 128;      // rows per workgroup (4 waves x 32)
constexpr int kMaxKvol = 27;

// Workgroups are dealt round-robin over the 8 XCDs; give each XCD a
// contiguous run of row tiles so neighbouring gathers share its L2.
__device__ __forceinline__ int xcd_tile(int bid, int nblocks) {
    const int q = nblocks / 8, r = nblocks % 8;
    const int xcd = bid % 8, local = bid / 8;
    return xcd * q + min(xcd, r) + local;
}

template <class T>
struct Frag;
template <>
struct Frag<uint16_t> {
    static constexpr int E = 8;  // elements per 16-byte fragment
};
template <>
struct Frag<float> {
    static constexpr int E = 4;
};

// Applies the optional input transforms to one 16-byte fragment of row j,
// channels c0 .. c0+E.  Returns the fragment in T.
template <class T>
__device__ __forceinline__ uint4 load_fragment(const ConvArgs &a, int32_t j, int32_t c0) {
    constexpr int E = Frag<T>::E;
    if (j < 0) return make_uint4(0, 0, 0, 0);
    const int64_t src = a.gather_parent ? (j >> 3) : j;
    const T *xp = static_cast<const T *>(a.x) + src * a.cin + c0;
    uint4 raw = *reinterpret_cast<const uint4 *>(xp);
    const bool slot = a.gather_parent && a.slot_offset;
    const bool affine = a.pre_scale != nullptr;
    if (!slot && !affine) return raw;
    float v[E];
    if constexpr (E == 8) {
        const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = bf16_to_f32(static_cast<uint16_t>(w4[e] & 0xffffu));
            v[2 * e + 1] = bf16_to_f32(static_cast<uint16_t>(w4[e] >> 16));
        }
    } else {
        v[0] = __builtin_bit_cast(float, raw.x);
        v[1] = __builtin_bit_cast(float, raw.y);
        v[2] = __builtin_bit_cast(float, raw.z);
        v[3] = __builtin_bit_cast(float, raw.w);
    }
    if (slot) {
        const float *so = a.slot_offset + (j & 7) * a.cin + c0;
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] += so[e];
    }
    if (affine) {
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = silu(v[e] * a.pre_scale[c0 + e] + a.pre_shift[c0 + e]);
    }
    if constexpr (E == 8) {
        uint32_t w4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            w4[e] = static_cast<uint32_t>(f32_to_bf16(v[2 * e])) |
                    (static_cast<uint32_t>(f32_to_bf16(v[2 * e + 1])) << 16);
        return make_uint4(w4[0], w4[1], w4[2], w4[3]);
    } else {
        return make_uint4(__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[1]),
                          __builtin_bit_cast(uint32_t, v[2]), __builtin_bit_cast(uint32_t, v[3]));
    }
}

template <class T>
__device__ __forceinline__ f32x16 mfma_step(uint4 af, uint4 bf, f32x16 acc) {
    if constexpr (sizeof(T) == 2) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, af),
                                                       __builtin_bit_cast(bf16x8, bf), acc, 0, 0,
                                                       0);
    } else {
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__builtin_bit_cast(float, af.x),
                                                   __builtin_bit_cast(float, bf.x), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__builtin_bit_cast(float, af.y),
                                                   __builtin_bit_cast(float, bf.y), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__builtin_bit_cast(float, af.z),
                                                   __builtin_bit_cast(float, bf.z), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__builtin_bit_cast(float, af.w),
                                                   __builtin_bit_cast(float, bf.w), acc, 0, 0, 0);
        return acc;
    }
}

// T: uint16_t (bf16) or float.  NB: 32-column blocks per tile.  KC: Cin
// channels per staged chunk.
template <class T, int NB, int KC>
__global__ void __launch_bounds__(256) conv_mfma_kernel(ConvArgs a) {
    constexpr int E = Frag<T>::E;
    constexpr int CPK = 2 * E;       // channels per k-step (both lane halves)
    constexpr int KS = KC / CPK;     // k-steps per chunk
    __shared__ uint4 wlds[KS * NB * 64];
    __shared__ int32_t rows[kBM * kMaxKvol];
    __shared__ uint32_t omask;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tile = xcd_tile(blockIdx.x, gridDim.x);
    const int64_t m0 = static_cast<int64_t>(tile) * kBM;
    const int nb0 = blockIdx.y * NB;  // first 32-column block of this tile
    const int nbtot = a.cout / 32;
    const int kvol = a.kvol;
    const int ksteps_total = a.cin / CPK;

    if (tid == 0) omask = 0;
    __syncthreads();
    // Stage this tile's neighbour rows; -1 marks a missing neighbour.
    uint32_t my_mask = 0;
    for (int idx = tid; idx < kBM * kvol; idx += 256) {
        const int r = idx / kvol, o = idx - r * kvol;
        const int64_t row = m0 + r;
        int64_t j = -1;
        if (row < a.n_out) j = a.kmap ? a.kmap[row * kvol + o] : row;
        const bool valid = j >= 0 && j < a.n_src;
        rows[idx] = valid ? static_cast<int32_t>(j) : -1;
        if (valid) my_mask |= 1u << o;
    }
    if (my_mask) atomicOr(&omask, my_mask);
    __syncthreads();
    const uint32_t mask = omask;

    f32x16 acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x16{};

    const uint4 *wg = static_cast<const uint4 *>(a.w);
    const int my_row = wave * 32 + (lane & 31);
    const int half = lane >> 5;

    for (int o = 0; o < kvol; ++o) {
        if (!((mask >> o) & 1u)) continue;
        const int32_t j = rows[my_row * kvol + o];
        for (int kc = 0; kc < a.cin; kc += KC) {
            // Gather this wave's A fragments for the chunk.
            uint4 af[KS];
#pragma unroll
            for (int s = 0; s < KS; ++s) af[s] = load_fragment<T>(a, j, kc + s * CPK + half * E);
            __syncthreads();  // previous chunk's LDS reads are done
            // Stage the weight chunk: KS k-steps x NB column blocks x 64 lanes.
            const int64_t kstep0 = static_cast<int64_t>(o) * ksteps_total + kc / CPK;
            for (int q = tid; q < KS * NB * 64; q += 256) {
                const int s = q / (NB * 64);
                const int rem = q - s * (NB * 64);
                const int nbl = rem >> 6;
                wlds[q] = wg[((kstep0 + s) * nbtot + nb0 + nbl) * 64 + (rem & 63)];
            }
            __syncthreads();
#pragma unroll
            for (int s = 0; s < KS; ++s) {
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    acc[nb] = mfma_step<T>(af[s], wlds[(s * NB + nb) * 64 + lane], acc[nb]);
            }
        }
    }

    // ---- epilogue ----
    const int col_in_blk = lane & 31;
    float v[NB][16];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int col = (nb0 + nb) * 32 + col_in_blk;
        const float b = a.bias ? a.bias[col] : 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) v[nb][r] = acc[nb][r] + b;
    }
    if (a.ln) {
        // The tile holds whole rows (NT == cout): row statistics reduce over
        // the NB registers and the 32 lanes of this lane half.
        const float inv_c = 1.0f / static_cast<float>(a.cout);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float s = 0.0f;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) s += v[nb][r];
#pragma unroll
            for (int d = 1; d < 32; d <<= 1) s += __shfl_xor(s, d, 64);
            const float mean = s * inv_c;
            float q = 0.0f;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const float t = v[nb][r] - mean;
                q += t * t;
            }
#pragma unroll
            for (int d = 1; d < 32; d <<= 1) q += __shfl_xor(q, d, 64);
            const float rstd = rsqrtf(q * inv_c + a.eps);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) v[nb][r] = (v[nb][r] - mean) * rstd;
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const int col = (nb0 + nb) * 32 + col_in_blk;
            const float w = a.ln_w ? a.ln_w[col] : 1.0f;
            const float b = a.ln_b ? a.ln_b[col] : 0.0f;
            const float ms = a.mod_scale ? a.mod_scale[col] : 0.0f;
            const float mh = a.mod_shift ? a.mod_shift[col] : 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float t = v[nb][r] * w + b;
                if (a.mod_scale) t = (t * ms + t) + mh;
                v[nb][r] = t;
            }
        }
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int col = (nb0 + nb) * 32 + col_in_blk;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t row = m0 + wave * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
            if (row >= a.n_out) continue;
            float t = v[nb][r];
            if (a.silu) t = silu(t);
            const int64_t off = row * a.cout + col;
            if (a.y_bf16) {
                if (a.residual) t += bf16_to_f32(static_cast<const uint16_t *>(a.residual)[off]);
                static_cast<uint16_t *>(a.y)[off] = f32_to_bf16(t);
            } else {
                if (a.residual) t += static_cast<const float *>(a.residual)[off];
                static_cast<float *>(a.y)[off] = t;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Generic VALU path: any Cin/Cout.  64 x 64 output tile, 16-channel chunks
// staged in LDS, 4 x 4 outputs per thread.  Weights fp32 [kvol][cin][cout].
// LayerNorm is not fused here; the host runs it as a separate pass.
// ---------------------------------------------------------------------------
constexpr int kGM = 64, kGN = 64, kGK = 16;

template <class T>
__device__ __forceinline__ float load_input(const ConvArgs &a, int32_t j, int32_t c) {
    const int64_t src = a.gather_parent ? (j >> 3) : j;
    float v = load_as_f32<T>(static_cast<const T *>(a.x) + src * a.cin + c);
    if (a.gather_parent && a.slot_offset) v += a.slot_offset[(j & 7) * a.cin + c];
    if (a.pre_scale) v = silu(v * a.pre_scale[c] + a.pre_shift[c]);
    if constexpr (sizeof(T) == 2) v = bf16_to_f32(f32_to_bf16(v));
    return v;
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
        rows[idx] = valid ? static_cast<int32_t>(j) : -1;
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
            if (a.y_bf16) {
                if (a.residual) t += bf16_to_f32(static_cast<const uint16_t *>(a.residual)[off]);
                static_cast<uint16_t *>(a.y)[off] = f32_to_bf16(t);
            } else {
                if (a.residual) t += static_cast<const float *>(a.residual)[off];
                static_cast<float *>(a.y)[off] = t;
            }
        }
    }
}

using KernelFn = void (*)(ConvArgs);

template <class T>
KernelFn pick_mfma(int nb, int kc) {
#define S3DX_NB_CASES(KCV)                              \
    switch (nb) {                                       \
    case 1: return conv_mfma_kernel<T, 1, KCV>;         \
    case 2: return conv_mfma_kernel<T, 2, KCV>;         \
    case 3: return conv_mfma_kernel<T, 3, KCV>;         \
    case 4: return conv_mfma_kernel<T, 4, KCV>;         \
    case 6: return conv_mfma_kernel<T, 6, KCV>;         \
    case 8: return conv_mfma_kernel<T, 8, KCV>;         \
    default: return nullptr;                            \
    }
    if constexpr (sizeof(T) == 2) {
        if (kc == 128) { S3DX_NB_CASES(128) }
        if (kc == 64) { S3DX_NB_CASES(64) }
        if (kc == 32) { S3DX_NB_CASES(32) }
    } else {
        if (kc == 64) { S3DX_NB_CASES(64) }
        if (kc == 32) { S3DX_NB_CASES(32) }
    }
#undef S3DX_NB_CASES
    return nullptr;
}

}  // namespace

// LayerNorm / residual helpers for the generic path live in norm.hip.
void layernorm_rows_launch(const void *x, int32_t x_dtype, int64_t n, int32_t c, float eps,
                           const float *w, const float *b, const float *mod_scale,
                           const float *mod_shift, int32_t silu, void *y, int32_t y_dtype,
                           hipStream_t stream);
void add_rows_launch(const void *a, const void *b, int32_t dtype, int64_t count, void *y,
                     hipStream_t stream);

}  // namespace s3dx

// ---------------------------------------------------------------------------
// Host side: the prepared layer object.
// ---------------------------------------------------------------------------
struct s3dx_conv {
    int32_t cin = 0, cout = 0, kvol = 0, dtype = 0;
    bool mfma = false;
    int nb = 0, kc = 0;  // MFMA tiling
    void *w = nullptr;   // packed weights (device)
    float *bias = nullptr;
    float *slot_offset = nullptr;
    bool gather_parent = false;
    const float *pre_scale = nullptr, *pre_shift = nullptr;  // caller-owned device
    bool ln = false, silu = false;
    float eps = 1e-6f;
    float *ln_w = nullptr, *ln_b = nullptr, *mod_scale = nullptr, *mod_shift = nullptr;
    bool weights_set = false;

    ~s3dx_conv() {
        for (void *p : {w, static_cast<void *>(bias), static_cast<void *>(slot_offset),
                        static_cast<void *>(ln_w), static_cast<void *>(ln_b),
                        static_cast<void *>(mod_scale), static_cast<void *>(mod_shift)})
            if (p) (void)hipFree(p);
    }
};

namespace s3dx {
namespace {

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
        const bool bf = dtype == S3DX_BF16;
        int kc = 0;
        if (bf) kc = cin % 128 == 0 ? 128 : cin % 64 == 0 ? 64 : cin % 32 == 0 ? 32 : 0;
        else kc = cin % 64 == 0 ? 64 : cin % 32 == 0 ? 32 : 0;
        int nb = 0;
        if (cout % 32 == 0) {
            const int blocks = cout / 32;
            for (int cand : {8, 6, 4, 3, 2, 1})
                if (blocks % cand == 0) {
                    nb = cand;
                    break;
                }
        }
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
            const int ksteps = cin / CPK, nbtot = cout / 32;
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
                                const float v = weight_at(host_weight, layout, kvol, cin, cout, o, co, ci);
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
    });
}

S3DX_API s3dx_status s3dx_conv_set_silu(s3dx_conv *conv, int32_t enable, char *error,
                                        uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(conv != nullptr, "conv is NULL");
        conv->silu = enable != 0;
    });
}

S3DX_API s3dx_status s3dx_conv_run(const s3dx_conv *conv, const void *x, int64_t n_in,
                                   const int32_t *kmap, int64_t n_out, const void *residual,
                                   void *y, int32_t y_dtype, s3dx_stream stream, char *error,
                                   uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(conv != nullptr, "conv is NULL");
        require(conv->weights_set, "weights not set");
        require(x && y, "NULL feature pointer");
        require(kmap != nullptr || conv->kvol == 1, "kmap is NULL for kvol 27");
        require(n_in > 0 && n_out > 0, "row counts must be positive");
        require(n_out <= INT32_MAX, "n_out exceeds INT32_MAX");
        require_dtype(y_dtype);
        require(aligned(x, 16) && aligned(y, 4) && aligned(residual, 4), "misaligned buffer");
        const int64_t n_src = conv->gather_parent ? n_in * 8 : n_in;
        require(n_src <= INT32_MAX, "input rows exceed INT32_MAX");
        const hipStream_t s = as_stream(stream);
        ConvArgs a{};
        a.x = x;
        a.n_src = n_src;
        a.cin = conv->cin;
        a.kmap = kmap;
        a.n_out = n_out;
        a.kvol = conv->kvol;
        a.w = conv->w;
        a.bias = conv->bias;
        a.cout = conv->cout;
        a.residual = residual;
        a.y = y;
        a.y_bf16 = y_dtype == S3DX_BF16;
        a.gather_parent = conv->gather_parent;
        a.slot_offset = conv->slot_offset;
        a.pre_scale = conv->pre_scale;
        a.pre_shift = conv->pre_shift;
        a.silu = conv->silu;
        a.eps = conv->eps;
        a.ln_w = conv->ln_w;
        a.ln_b = conv->ln_b;
        a.mod_scale = conv->mod_scale;
        a.mod_shift = conv->mod_shift;
        const bool bf = conv->dtype == S3DX_BF16;
        const bool fused_ln = conv->ln && conv->mfma && conv->nb * 32 == conv->cout;
        if (conv->mfma) {
            a.ln = fused_ln;
            if (conv->ln && !fused_ln) {  // LayerNorm as a separate pass
                a.silu = 0;
                a.residual = nullptr;
            }
            const KernelFn fn = bf ? pick_mfma<uint16_t>(conv->nb, conv->kc)
                                   : pick_mfma<float>(conv->nb, conv->kc);
            require(fn != nullptr, "no MFMA kernel for this shape");
            const int64_t mt = (n_out + kBM - 1) / kBM;
            const dim3 grid(static_cast<unsigned>(mt), static_cast<unsigned>(conv->cout / (32 * conv->nb)));
            hipLaunchKernelGGL(fn, grid, dim3(256), 0, s, a);
            launch_check("conv_mfma");
        } else {
            a.ln = 0;
            if (conv->ln) {
                a.silu = 0;
                a.residual = nullptr;
            }
            const int64_t mt = (n_out + kGM - 1) / kGM;
            const dim3 grid(static_cast<unsigned>(mt), static_cast<unsigned>((conv->cout + kGN - 1) / kGN));
            if (bf) hipLaunchKernelGGL(conv_generic_kernel<uint16_t>, grid, dim3(256), 0, s, a);
            else hipLaunchKernelGGL(conv_generic_kernel<float>, grid, dim3(256), 0, s, a);
            launch_check("conv_generic");
        }
        if (conv->ln && !a.ln) {
            layernorm_rows_launch(y, y_dtype, n_out, conv->cout, conv->eps, conv->ln_w, conv->ln_b,
                                  conv->mod_scale, conv->mod_shift, conv->silu ? 1 : 0, y, y_dtype, s);
            if (residual) add_rows_launch(y, residual, y_dtype, n_out * conv->cout, y, s);
        }
    });
}

}  // extern "C"
