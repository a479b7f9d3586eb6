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
// res (in TO, may be NULL): added after the SiLU, row (row >> res_shift).
template <class TI, class TO>
__global__ void __launch_bounds__(256)
layernorm_kernel(const void *x, int64_t n, int32_t c, float eps, const float *w, const float *b,
                 const float *ms, const float *mh, int32_t do_silu, void *y, const void *res,
                 int32_t res_shift) {
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
        if (res) t += ld<TO>(res, (row >> res_shift) * c + k);
        st<TO>(y, base + k, t);
    }
}

// VE elements of T at element offset `elem` as floats (one 8- or 16-byte
// access, or two 16-byte ones), and back.
template <class T, int VE>
__device__ __forceinline__ void vload(const void *base, int64_t elem, float (&v)[VE]) {
    constexpr int BYTES = VE * static_cast<int>(sizeof(T));
    const char *p = static_cast<const char *>(base) + elem * static_cast<int64_t>(sizeof(T));
    uint32_t wd[BYTES / 4];
    if constexpr (BYTES == 8) {
        const uint2 t = *reinterpret_cast<const uint2 *>(p);
        wd[0] = t.x;
        wd[1] = t.y;
    } else {
#pragma unroll
        for (int q = 0; q < BYTES / 16; ++q) {
            const uint4 t = reinterpret_cast<const uint4 *>(p)[q];
            wd[4 * q] = t.x;
            wd[4 * q + 1] = t.y;
            wd[4 * q + 2] = t.z;
            wd[4 * q + 3] = t.w;
        }
    }
#pragma unroll
    for (int e = 0; e < VE; ++e) {
        if constexpr (sizeof(T) == 2)
            v[e] = bf16_to_f32(static_cast<uint16_t>(e & 1 ? wd[e >> 1] >> 16 : wd[e >> 1] & 0xffffu));
        else
            v[e] = __builtin_bit_cast(float, wd[e]);
    }
}
template <class T, int VE>
__device__ __forceinline__ void vstore(void *base, int64_t elem, const float (&v)[VE]) {
    constexpr int BYTES = VE * static_cast<int>(sizeof(T));
    char *p = static_cast<char *>(base) + elem * static_cast<int64_t>(sizeof(T));
    uint32_t wd[BYTES / 4];
#pragma unroll
    for (int e = 0; e < VE; ++e) {
        if constexpr (sizeof(T) == 2) {
            const uint32_t h = f32_to_bf16(v[e]);
            if (e & 1) wd[e >> 1] |= h << 16;
            else wd[e >> 1] = h;
        } else {
            wd[e] = __builtin_bit_cast(uint32_t, v[e]);
        }
    }
    if constexpr (BYTES == 8) {
        *reinterpret_cast<uint2 *>(p) = make_uint2(wd[0], wd[1]);
    } else {
#pragma unroll
        for (int q = 0; q < BYTES / 16; ++q)
            reinterpret_cast<uint4 *>(p)[q] = make_uint4(wd[4 * q], wd[4 * q + 1], wd[4 * q + 2], wd[4 * q + 3]);
    }
}

// LayerNorm with the row held in registers: 2^lpr_log2 lanes per row (64 /
// lanes rows per wave), each lane PPL pieces of VE = 16 / sizeof(TI)
// elements (piece p*lanes + lane: consecutive lanes read consecutive 16-byte
// pieces), so the row is read once and written once.  Mean, then the
// centred variance of the held values, both reduced over the row's lanes
// by xor shuffles.  Requires rows of whole pieces and 16-byte aligned
// buffers and parameter vectors.
template <class TI, class TO, int PPL>
__global__ void __launch_bounds__(256)
layernorm_vec_kernel(const void *x, int64_t n, int32_t c, int32_t lpr_log2, float eps, const float *w,
                     const float *b, const float *ms, const float *mh, int32_t do_silu, void *y, const void *res,
                     int32_t res_shift) {
    constexpr int VE = 16 / static_cast<int>(sizeof(TI));
    const int lane = threadIdx.x & 63;
    const int lpr = 1 << lpr_log2;
    const int64_t row = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * (64 >> lpr_log2) +
                        (lane >> lpr_log2);
    const int sl = lane & (lpr - 1);
    const int ppr = c / VE;
    const bool active = row < n;
    float v[PPL][VE];
    float sum = 0.0f;
    // The row's PPL pieces are loaded unconditionally (a piece or row past
    // the end rereads the last one and is zeroed after) and widened only once
    // all are issued: a load under a condition, or widened next to it, makes
    // the compiler wait for each piece in turn.
    {
        const int64_t lrow = active ? row : n - 1;
        uint4 raw[PPL];
#pragma unroll
        for (int p = 0; p < PPL; ++p) {
            const int pi = min(p * lpr + sl, ppr - 1);
            raw[p] = *reinterpret_cast<const uint4 *>(static_cast<const TI *>(x) + lrow * c +
                                                      static_cast<int64_t>(pi) * VE);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int p = 0; p < PPL; ++p) {
            const bool in = active && p * lpr + sl < ppr;
            const uint32_t w4[4] = {raw[p].x, raw[p].y, raw[p].z, raw[p].w};
#pragma unroll
            for (int e = 0; e < VE; ++e) {
                float f;
                if constexpr (sizeof(TI) == 2)
                    f = bf16_to_f32(static_cast<uint16_t>(e & 1 ? w4[e >> 1] >> 16 : w4[e >> 1] & 0xffffu));
                else
                    f = __builtin_bit_cast(float, w4[e]);
                v[p][e] = in ? f : 0.0f;
                sum += v[p][e];
            }
        }
    }
    for (int d = 1; d < lpr; d <<= 1) sum += __shfl_xor(sum, d, 64);
    const float mean = sum / static_cast<float>(c);
    float q = 0.0f;
#pragma unroll
    for (int p = 0; p < PPL; ++p) {
        if (p * lpr + sl >= ppr) continue;
#pragma unroll
        for (int e = 0; e < VE; ++e) {
            const float t = v[p][e] - mean;
            q += t * t;
        }
    }
    for (int d = 1; d < lpr; d <<= 1) q += __shfl_xor(q, d, 64);
    const float rstd = rsqrtf(q / static_cast<float>(c) + eps);
    if (!active) return;
#pragma unroll
    for (int p = 0; p < PPL; ++p) {
        const int pi = p * lpr + sl;
        if (pi >= ppr) continue;
        const int64_t ch = static_cast<int64_t>(pi) * VE;
        float t[VE], pw[VE], pb[VE], r[VE];
#pragma unroll
        for (int e = 0; e < VE; ++e) t[e] = (v[p][e] - mean) * rstd;
        if (w) {
            vload<float, VE>(w, ch, pw);
#pragma unroll
            for (int e = 0; e < VE; ++e) t[e] *= pw[e];
        }
        if (b) {
            vload<float, VE>(b, ch, pb);
#pragma unroll
            for (int e = 0; e < VE; ++e) t[e] += pb[e];
        }
        if (ms) {
            vload<float, VE>(ms, ch, pw);
            vload<float, VE>(mh, ch, pb);
#pragma unroll
            for (int e = 0; e < VE; ++e) t[e] = (t[e] * pw[e] + t[e]) + pb[e];
        }
        if (do_silu) {
#pragma unroll
            for (int e = 0; e < VE; ++e) t[e] = silu(t[e]);
        }
        if (res) {
            vload<TO, VE>(res, (row >> res_shift) * c + ch, r);
#pragma unroll
            for (int e = 0; e < VE; ++e) t[e] += r[e];
        }
        vstore<TO, VE>(y, row * c + ch, t);
    }
}

// GroupNorm statistics in one pass over x.  Each channel's values are
// shifted by its row-0 value K (the shifted-data variance method), so
// sum (x - K) and sum (x - K)^2 stay well conditioned when |mean| >> std.
// Block b owns a contiguous run of rows; a thread owns VE*MP channels of one
// row slot (pieces of VE channels, 16-byte loads when VE > 1) and walks the
// run `rstep` rows at a time.  Writes per-block per-channel partial sums
// partials[b][0][ch] and partials[b][1][ch]; gn_finalize_kernel combines
// them per group in double, in a fixed order.
constexpr int kStatBlocks = 1024;
constexpr int kMaxGnChannels = 1024;

// A piece as loaded (16 bytes, or one element when VE == 1) and its
// widening to float, kept apart so several pieces' loads can be issued
// before the first is widened.
// (A single element is held zero-extended in 32 bits, so pieces never share
// a register.)
template <class T, int VE>
using RawPiece = std::conditional_t<(VE > 1), uint4, uint32_t>;

template <class T, int VE>
__device__ __forceinline__ RawPiece<T, VE> load_raw_piece(const void *x, int64_t off) {
    if constexpr (VE == 1) {
        if constexpr (sizeof(T) == 2) return static_cast<const uint16_t *>(x)[off];
        else return static_cast<const uint32_t *>(x)[off];
    } else {
        return *reinterpret_cast<const uint4 *>(static_cast<const T *>(x) + off);
    }
}

template <class T, int VE>
__device__ __forceinline__ void widen_piece(const RawPiece<T, VE> &raw, float (&v)[VE]) {
    if constexpr (VE == 1) {
        if constexpr (sizeof(T) == 2) v[0] = bf16_to_f32(static_cast<uint16_t>(raw));
        else v[0] = __builtin_bit_cast(float, raw);
    } else {
        const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
        if constexpr (sizeof(T) == 2) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                v[2 * k] = bf16_to_f32(static_cast<uint16_t>(w4[k] & 0xffffu));
                v[2 * k + 1] = bf16_to_f32(static_cast<uint16_t>(w4[k] >> 16));
            }
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) v[k] = __builtin_bit_cast(float, w4[k]);
        }
    }
}

template <class T, int VE, int MP>
__global__ void __launch_bounds__(256)
gn_sums_kernel(const void *x, int64_t n, int32_t c, float *partials) {
    __shared__ float red[2][2048];
    const int ppr = c / VE;                 // pieces per row
    const int tpr = ppr < 256 ? ppr : 256;  // threads per row slot
    const int rstep = 256 / tpr;
    const int tid = threadIdx.x;
    const int roff = tid / tpr, p0 = tid - roff * tpr;
    const bool active = roff < rstep;
    const int64_t rows_per = (n + gridDim.x - 1) / gridDim.x;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * rows_per;
    const int64_t r1 = min(n, r0 + rows_per);
    float k[MP][VE], s[MP][VE], q[MP][VE];
#pragma unroll
    for (int i = 0; i < MP; ++i) {
        const int p = p0 + i * tpr;
        if (active && p < ppr) widen_piece<T, VE>(load_raw_piece<T, VE>(x, static_cast<int64_t>(p) * VE), k[i]);
#pragma unroll
        for (int e = 0; e < VE; ++e) {
            s[i][e] = 0.0f;
            q[i][e] = 0.0f;
        }
    }
    if (active) {
        // kRowsInFlight rows' loads are issued before the first is summed (the
        // barrier stops the scheduler from pairing each load with its use);
        // each accumulator still takes the rows in increasing order.  Rows
        // past the run's end reread its last row and are not added.
        constexpr int kRowsInFlight = 8;
        using Raw = RawPiece<T, VE>;
        auto add_row = [&](const Raw (&raw)[MP]) {
#pragma unroll
            for (int i = 0; i < MP; ++i) {
                if (MP > 1 && p0 + i * tpr >= ppr) continue;
                float v[VE];
                widen_piece<T, VE>(raw[i], v);
#pragma unroll
                for (int e = 0; e < VE; ++e) {
                    const float d = v[e] - k[i][e];
                    s[i][e] += d;
                    q[i][e] += d * d;
                }
            }
        };
        auto load_row = [&](int64_t r, Raw (&raw)[MP]) {
#pragma unroll
            for (int i = 0; i < MP; ++i) {
                const int p = p0 + i * tpr;
                if (MP > 1 && p >= ppr) continue;
                raw[i] = load_raw_piece<T, VE>(x, r * c + static_cast<int64_t>(p) * VE);
            }
        };
        for (int64_t r = r0 + roff; r < r1; r += kRowsInFlight * rstep) {
            Raw raw[kRowsInFlight][MP];
#pragma unroll
            for (int u = 0; u < kRowsInFlight; ++u) load_row(min(r + u * rstep, r1 - 1), raw[u]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < kRowsInFlight; ++u)
                if (r + u * rstep < r1) add_row(raw[u]);
        }
#pragma unroll
        for (int i = 0; i < MP; ++i) {
            const int p = p0 + i * tpr;
            if (MP > 1 && p >= ppr) continue;
#pragma unroll
            for (int e = 0; e < VE; ++e) {
                red[0][roff * c + p * VE + e] = s[i][e];
                red[1][roff * c + p * VE + e] = q[i][e];
            }
        }
    }
    __syncthreads();
    for (int ch = tid; ch < c; ch += 256) {
        float ts = 0.0f, tq = 0.0f;
        for (int j = 0; j < rstep; ++j) {
            ts += red[0][j * c + ch];
            tq += red[1][j * c + ch];
        }
        float *out = partials + static_cast<int64_t>(blockIdx.x) * 2 * c;
        out[ch] = ts;
        out[c + ch] = tq;
    }
}

// One block per group: per-channel totals over the stat blocks, then the
// group mean and centred variance from the shifted sums
//   sum_r (x - m)^2 = sum_r (x - K)^2 - 2 (m - K) sum_r (x - K) + n (m - K)^2,
// then scale = gamma * rstd, shift = beta - m * gamma * rstd per channel.
// The group's partials are 2 cg items a stat block (item j < cg: sum (x - K)
// of channel j; item cg + j: sum (x - K)^2 of channel j), two runs of cg
// floats.  A pass takes up to kFinalizeThreads items; thread t adds item
// t mod w over stat blocks s, s + slots, ... (s = t / w, slots =
// kFinalizeThreads / w), so one wave load covers consecutive channels of a
// few stat blocks instead of 64 cache lines.  Loads go kFinalizeBatch at a
// time (past the last stat block they reread it and add 0).  Slot totals meet
// in LDS and are added in slot order: a fixed order whatever the timing.
constexpr int kFinalizeThreads = 1024;
constexpr int kFinalizeBatch = 16;
static_assert(kMaxGnChannels <= kFinalizeThreads, "a thread per channel of a group");
template <class T>
__global__ void __launch_bounds__(kFinalizeThreads)
gn_finalize_kernel(const void *x, const float *partials, int64_t n, int32_t c, int32_t cg, float eps,
                   const float *gamma, const float *beta, float *scale, float *shift) {
    __shared__ double slot_sum[kFinalizeThreads];
    __shared__ double tot[2 * kMaxGnChannels];
    __shared__ double kx[kMaxGnChannels];
    __shared__ double stats[2];
    const int g = blockIdx.x, tid = threadIdx.x;
    // Thread cl < cg owns channel g cg + cl.  Its shift and affine values
    // are loaded first, unconditionally (other threads reread the group's
    // last channel; a NULL gamma or beta reads partials instead and is
    // replaced by 1 or 0 at the use), so they land while the partials are
    // added.
    const bool own = tid < cg;
    const int och = g * cg + min(tid, cg - 1);
    const T kraw = static_cast<const T *>(x)[och];
    const float graw = (gamma ? gamma : partials)[och];
    const float braw = (beta ? beta : partials)[och];
    const int items = 2 * cg;
    for (int j0 = 0; j0 < items; j0 += kFinalizeThreads) {
        const int w = min(items - j0, kFinalizeThreads);
        const int slots = kFinalizeThreads / w;
        const int slot = tid / w, jl = tid - slot * w, j = j0 + jl;
        if (slot < slots) {
            const float *p = partials + (j < cg ? g * cg + j : c + g * cg + (j - cg));
            double a = 0.0;
            for (int b = slot; b < kStatBlocks; b += kFinalizeBatch * slots) {
                float v[kFinalizeBatch];
#pragma unroll
                for (int u = 0; u < kFinalizeBatch; ++u)
                    v[u] = p[static_cast<int64_t>(min(b + u * slots, kStatBlocks - 1)) * 2 * c];
                // Keeps the scheduler from pairing each load with its add.
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int u = 0; u < kFinalizeBatch; ++u)
                    a += b + u * slots < kStatBlocks ? static_cast<double>(v[u]) : 0.0;
            }
            slot_sum[slot * w + jl] = a;
        }
        __syncthreads();
        if (tid < w) {
            double a = 0.0;
            for (int s = 0; s < slots; ++s) a += slot_sum[s * w + tid];
            tot[j] = a;
        }
        __syncthreads();
    }
    if (own) kx[tid] = static_cast<double>(load_as_f32<T>(&kraw));
    __syncthreads();
    if (tid == 0) {
        const double *t1 = tot, *t2 = tot + cg;
        const double dn = static_cast<double>(n);
        double sum = 0.0;
        for (int cl = 0; cl < cg; ++cl) sum += kx[cl] * dn + t1[cl];
        const double m = sum / (dn * cg);
        double ss = 0.0;
        for (int cl = 0; cl < cg; ++cl) {
            const double dk = m - kx[cl];
            ss += t2[cl] - 2.0 * dk * t1[cl] + dn * dk * dk;
        }
        const double var = ss / (dn * cg);
        stats[0] = m;
        stats[1] = 1.0 / sqrt((var > 0.0 ? var : 0.0) + static_cast<double>(eps));
    }
    __syncthreads();
    if (own) {
        const double ga = gamma ? static_cast<double>(graw) : 1.0;
        const double be = beta ? static_cast<double>(braw) : 0.0;
        scale[och] = static_cast<float>(ga * stats[1]);
        shift[och] = static_cast<float>(be - stats[0] * ga * stats[1]);
    }
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

// Row-piece variants: rows of whole 16-byte pieces (E = 8 BF16 or 4 FP32
// values), both buffers 16-byte aligned, fewer than 2^30 pieces.  Each
// element sums its children in the same order as the kernels above.
template <class T>
__global__ void __launch_bounds__(256)
downsample16_kernel(const uint4 *x, int64_t nf, int32_t ppr, const int32_t *children,
                    const float *inv_count, int32_t count, uint4 *y) {
    constexpr int E = 16 / static_cast<int>(sizeof(T));
    for (int32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += gridDim.x * blockDim.x) {
        const int32_t r = i / ppr, pc = i - r * ppr;
        float acc[E];
#pragma unroll
        for (int e = 0; e < E; ++e) acc[e] = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int32_t f = children[static_cast<int64_t>(r) * 8 + j];
            if (f < 0 || f >= nf) continue;
            const uint4 v = x[static_cast<int64_t>(f) * ppr + pc];
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < E; ++e) {
                if constexpr (sizeof(T) == 2)
                    acc[e] += bf16_to_f32(static_cast<uint16_t>(e & 1 ? w[e >> 1] >> 16 : w[e >> 1] & 0xffffu));
                else
                    acc[e] += __builtin_bit_cast(float, w[e]);
            }
        }
        const float k = inv_count[r];
        uint32_t o[4];
        if constexpr (sizeof(T) == 2) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                o[q] = static_cast<uint32_t>(f32_to_bf16(acc[2 * q] * k)) |
                       (static_cast<uint32_t>(f32_to_bf16(acc[2 * q + 1] * k)) << 16);
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) o[q] = __builtin_bit_cast(uint32_t, acc[q] * k);
        }
        y[i] = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

// Nearest upsample as a row gather of 16-byte pieces (a copy: any dtype).
__global__ void __launch_bounds__(256)
upsample16_kernel(const uint4 *coarse, int64_t nc, int32_t ppr, const int32_t *f2c, int32_t count,
                  uint4 *y) {
    for (int32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += gridDim.x * blockDim.x) {
        const int32_t r = i / ppr, pc = i - r * ppr;
        const int32_t src = f2c[r];
        y[i] = src >= 0 && src < nc ? coarse[static_cast<int64_t>(src) * ppr + pc] : make_uint4(0u, 0u, 0u, 0u);
    }
}

// Row concatenation through an optional row index: y[i] = [a[r], b[r]],
// r = rows ? rows[i] : i, zero rows for r outside [0, n_src).  The piece
// variant moves 16-byte pieces (both halves whole pieces, buffers aligned);
// the element variant any widths.  A copy: bit-exact in either dtype.
__global__ void __launch_bounds__(256)
concat16_kernel(const uint4 *a, int32_t ppa, const uint4 *b, int32_t ppb, int64_t n_src, const int32_t *rows,
                int32_t count, uint4 *y) {
    const int32_t ppr = ppa + ppb;
    for (int32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += gridDim.x * blockDim.x) {
        const int32_t r = i / ppr, pc = i - r * ppr;
        const int64_t src = rows ? rows[r] : r;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (src >= 0 && src < n_src) v = pc < ppa ? a[src * ppa + pc] : b[src * ppb + (pc - ppa)];
        y[i] = v;
    }
}

template <class T>
__global__ void __launch_bounds__(256)
concat_kernel(const T *a, int32_t ca, const T *b, int32_t cb, int64_t n_src, const int32_t *rows, int64_t n, T *y) {
    const int32_t c = ca + cb;
    const int64_t count = n * c;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) {
        const int64_t r = i / c;
        const int32_t ch = static_cast<int32_t>(i - r * c);
        const int64_t src = rows ? rows[r] : r;
        T v = T(0);
        if (src >= 0 && src < n_src) v = ch < ca ? a[src * ca + ch] : b[src * cb + (ch - ca)];
        y[i] = v;
    }
}

template <class TI, class TO>
__global__ void __launch_bounds__(256) convert_kernel(const void *x, int64_t count, void *y) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride)
        st<TO>(y, i, ld<TI>(x, i));
}

// 8 elements per thread step (16-byte accesses; both buffers 16-byte
// aligned), the last count % 8 elements one per thread.
template <class TI, class TO>
__global__ void __launch_bounds__(256) convert8_kernel(const void *x, int64_t count, void *y) {
    const int64_t groups = count / 8;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    for (int64_t g = tid; g < groups; g += stride) {
        float v[8];
        if constexpr (sizeof(TI) == 2) {
            const uint4 r = reinterpret_cast<const uint4 *>(x)[g];
            const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                v[2 * k] = bf16_to_f32(static_cast<uint16_t>(w[k] & 0xffffu));
                v[2 * k + 1] = bf16_to_f32(static_cast<uint16_t>(w[k] >> 16));
            }
        } else {
            const float4 a = reinterpret_cast<const float4 *>(x)[2 * g], b = reinterpret_cast<const float4 *>(x)[2 * g + 1];
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        }
        if constexpr (sizeof(TO) == 2) {
            uint32_t w[4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                w[k] = static_cast<uint32_t>(f32_to_bf16(v[2 * k])) | (static_cast<uint32_t>(f32_to_bf16(v[2 * k + 1])) << 16);
            reinterpret_cast<uint4 *>(y)[g] = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
            reinterpret_cast<float4 *>(y)[2 * g] = make_float4(v[0], v[1], v[2], v[3]);
            reinterpret_cast<float4 *>(y)[2 * g + 1] = make_float4(v[4], v[5], v[6], v[7]);
        }
    }
    if (tid < count - groups * 8) st<TO>(y, groups * 8 + tid, ld<TI>(x, groups * 8 + tid));
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

struct LnVecArgs {
    const void *x;
    int64_t n;
    int32_t c, lg;
    float eps;
    const float *w, *b, *ms, *mh;
    int32_t silu;
    void *y;
    const void *res;
    int32_t res_shift;
};
template <int PPL>
void ln_vec_launch(const LnVecArgs &a, int32_t xd, int32_t yd, unsigned blocks, hipStream_t stream) {
#define S3DX_LN_VEC(TI, TO)                                                                                   \
    layernorm_vec_kernel<TI, TO, PPL><<<blocks, 256, 0, stream>>>(a.x, a.n, a.c, a.lg, a.eps, a.w, a.b, a.ms, \
                                                                  a.mh, a.silu, a.y, a.res, a.res_shift)
    if (xd == S3DX_BF16 && yd == S3DX_BF16) S3DX_LN_VEC(uint16_t, uint16_t);
    else if (xd == S3DX_BF16) S3DX_LN_VEC(uint16_t, float);
    else if (yd == S3DX_BF16) S3DX_LN_VEC(float, uint16_t);
    else S3DX_LN_VEC(float, float);
#undef S3DX_LN_VEC
}

struct GnLayout {
    float *partials;  // [kStatBlocks][2][c]
};
template <class W>
void gn_layout(W &w, int32_t c, GnLayout *l) {
    if constexpr (std::is_same_v<W, Carver>) l->partials = w.template take<float>(static_cast<uint64_t>(kStatBlocks) * 2 * c);
    else w.template take<float>(static_cast<uint64_t>(kStatBlocks) * 2 * c);
}

}  // namespace

void layernorm_rows_launch(const void *x, int32_t x_dtype, int64_t n, int32_t c, float eps,
                           const float *w, const float *b, const float *mod_scale,
                           const float *mod_shift, int32_t do_silu, void *y, int32_t y_dtype,
                           hipStream_t stream, const void *residual, int32_t residual_shift) {
    const int64_t ve = 16 / dtype_size(x_dtype);
    const int64_t ppr = c % ve == 0 ? c / ve : 0;
    const bool vec = ppr > 0 && ppr <= 512 && x != y && aligned(x, 16) && aligned(y, 16) &&
                     (!residual || aligned(residual, 16)) && (!w || aligned(w, 16)) && (!b || aligned(b, 16)) &&
                     (!mod_scale || (aligned(mod_scale, 16) && aligned(mod_shift, 16)));
    if (vec) {
        int lg = 0;
        while ((1 << lg) < ppr && lg < 6) ++lg;  // lanes per row: 2^lg, at most 64
        const int64_t ppl = (ppr + (1 << lg) - 1) >> lg;
        const int64_t rows_per_block = 4 * (64 >> lg);
        const unsigned blocks = static_cast<unsigned>((n + rows_per_block - 1) / rows_per_block);
        const LnVecArgs la{x, n, c, lg, eps, w, b, mod_scale, mod_shift, do_silu, y, residual, residual_shift};
        if (ppl <= 1) ln_vec_launch<1>(la, x_dtype, y_dtype, blocks, stream);
        else if (ppl <= 2) ln_vec_launch<2>(la, x_dtype, y_dtype, blocks, stream);
        else if (ppl <= 4) ln_vec_launch<4>(la, x_dtype, y_dtype, blocks, stream);
        else ln_vec_launch<8>(la, x_dtype, y_dtype, blocks, stream);
    } else {
        const unsigned blocks = static_cast<unsigned>((n + 3) / 4);
        S3DX_DISPATCH2(x_dtype, y_dtype, layernorm_kernel,
                       <<<blocks, 256, 0, stream>>>(x, n, c, eps, w, b, mod_scale, mod_shift, do_silu, y,
                                                    residual, residual_shift));
    }
    launch_check("layernorm");
}

void convert_launch(const void *x, int32_t x_dtype, int64_t count, void *y, int32_t y_dtype,
                    hipStream_t stream) {
    if (x != y && aligned(x, 16) && aligned(y, 16))
        S3DX_DISPATCH2(x_dtype, y_dtype, convert8_kernel, <<<grid_for((count + 7) / 8), 256, 0, stream>>>(x, count, y));
    else
        S3DX_DISPATCH2(x_dtype, y_dtype, convert_kernel, <<<grid_for(count), 256, 0, stream>>>(x, count, y));
    launch_check("convert");
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
                              as_stream(stream), nullptr, 0);
    });
}

S3DX_API s3dx_status s3dx_groupnorm_workspace_size(int64_t n, int32_t c, int32_t groups,
                                                   uint64_t *bytes, char *error,
                                                   uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(bytes != nullptr, "bytes is NULL");
        require(n > 0 && c > 0 && groups > 0 && c % groups == 0, "invalid GroupNorm shape");
        require(c <= kMaxGnChannels, "GroupNorm supports at most 1024 channels");
        Sizer s;
        gn_layout(s, c, nullptr);
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
        require(c <= kMaxGnChannels, "GroupNorm supports at most 1024 channels");
        require_dtype(x_dtype);
        const hipStream_t s = as_stream(stream);
        Carver w(workspace, workspace_bytes);
        GnLayout l;
        gn_layout(w, c, &l);
        const int cg = c / groups;
        const bool bf = x_dtype == S3DX_BF16;
        // 16-byte pieces when rows are whole pieces and x is 16-byte aligned.
        const bool vec = c % (bf ? 8 : 4) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
        if (bf) {
            if (vec) gn_sums_kernel<uint16_t, 8, 1><<<kStatBlocks, 256, 0, s>>>(x, n, c, l.partials);
            else gn_sums_kernel<uint16_t, 1, 4><<<kStatBlocks, 256, 0, s>>>(x, n, c, l.partials);
        } else {
            if (vec) gn_sums_kernel<float, 4, 1><<<kStatBlocks, 256, 0, s>>>(x, n, c, l.partials);
            else gn_sums_kernel<float, 1, 4><<<kStatBlocks, 256, 0, s>>>(x, n, c, l.partials);
        }
        launch_check("gn_sums");
        if (bf) gn_finalize_kernel<uint16_t><<<groups, kFinalizeThreads, 0, s>>>(x, l.partials, n, c, cg, eps,
                                                                                     gamma, beta, scale, shift);
        else gn_finalize_kernel<float><<<groups, kFinalizeThreads, 0, s>>>(x, l.partials, n, c, cg, eps, gamma,
                                                                                beta, scale, shift);
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
        const int64_t rowb = static_cast<int64_t>(c) * dtype_size(dtype);
        if (rowb % 16 == 0 && aligned(x, 16) && aligned(y, 16) && nc * (rowb / 16) < (int64_t(1) << 30)) {
            const int32_t ppr = static_cast<int32_t>(rowb / 16), count = static_cast<int32_t>(nc * ppr);
            const uint4 *xv = static_cast<const uint4 *>(x);
            if (dtype == S3DX_BF16)
                downsample16_kernel<uint16_t><<<grid_for(count), 256, 0, s>>>(xv, nf, ppr, children, inv_count, count,
                                                                             static_cast<uint4 *>(y));
            else
                downsample16_kernel<float><<<grid_for(count), 256, 0, s>>>(xv, nf, ppr, children, inv_count, count,
                                                                          static_cast<uint4 *>(y));
        } else if (dtype == S3DX_BF16) {
            downsample_kernel<uint16_t><<<grid_for(nc * c), 256, 0, s>>>(x, nf, c, children, inv_count, nc, y);
        } else {
            downsample_kernel<float><<<grid_for(nc * c), 256, 0, s>>>(x, nf, c, children, inv_count, nc, y);
        }
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
        const int64_t rowb = static_cast<int64_t>(c) * dtype_size(dtype);
        if (rowb % 16 == 0 && aligned(coarse, 16) && aligned(y, 16) && nf * (rowb / 16) < (int64_t(1) << 30)) {
            const int32_t ppr = static_cast<int32_t>(rowb / 16), count = static_cast<int32_t>(nf * ppr);
            upsample16_kernel<<<grid_for(count), 256, 0, s>>>(static_cast<const uint4 *>(coarse), nc, ppr,
                                                             fine_to_coarse, count, static_cast<uint4 *>(y));
        } else if (dtype == S3DX_BF16) {
            upsample_kernel<uint16_t><<<grid_for(nf * c), 256, 0, s>>>(coarse, nc, c, fine_to_coarse, nf, y);
        } else {
            upsample_kernel<float><<<grid_for(nf * c), 256, 0, s>>>(coarse, nc, c, fine_to_coarse, nf, y);
        }
        launch_check("upsample");
    });
}

S3DX_API s3dx_status s3dx_concat_rows(const void *a, int32_t ca, const void *b, int32_t cb, int32_t dtype,
                                      int64_t n_src, const int32_t *rows, int64_t n, void *y, s3dx_stream stream,
                                      char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(a && b && y, "NULL argument");
        require(ca > 0 && cb > 0 && n > 0 && n_src > 0, "sizes must be positive");
        require(rows != nullptr || n <= n_src, "without a row index n must not exceed n_src");
        require_dtype(dtype);
        const hipStream_t s = as_stream(stream);
        const int64_t es = dtype_size(dtype), ab = ca * es, bb = cb * es;
        if (ab % 16 == 0 && bb % 16 == 0 && aligned(a, 16) && aligned(b, 16) && aligned(y, 16) &&
            n * ((ab + bb) / 16) < (int64_t(1) << 30)) {
            const int32_t ppa = static_cast<int32_t>(ab / 16), ppb = static_cast<int32_t>(bb / 16);
            const int32_t count = static_cast<int32_t>(n * (ppa + ppb));
            concat16_kernel<<<grid_for(count), 256, 0, s>>>(static_cast<const uint4 *>(a), ppa,
                                                           static_cast<const uint4 *>(b), ppb, n_src, rows, count,
                                                           static_cast<uint4 *>(y));
        } else if (dtype == S3DX_BF16) {
            concat_kernel<uint16_t><<<grid_for(n * (ca + cb)), 256, 0, s>>>(
                static_cast<const uint16_t *>(a), ca, static_cast<const uint16_t *>(b), cb, n_src, rows, n,
                static_cast<uint16_t *>(y));
        } else {
            concat_kernel<float><<<grid_for(n * (ca + cb)), 256, 0, s>>>(
                static_cast<const float *>(a), ca, static_cast<const float *>(b), cb, n_src, rows, n,
                static_cast<float *>(y));
        }
        launch_check("concat_rows");
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
        convert_launch(x, x_dtype, count, y, y_dtype, as_stream(stream));
    });
}

}  // extern "C"
