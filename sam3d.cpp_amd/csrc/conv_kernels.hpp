// Device side of the MFMA gather-GEMM sparse convolution (see conv.hip for
// the operator it implements).  Instantiated per element type in
// conv_bf16.hip and conv_f32.hip.
#pragma once

#include "common.hpp"

#include <type_traits>

namespace s3dx {

struct ConvArgs {
    const void *x;
    int64_t x_bytes;  // bytes addressable at x
    int64_t n_src;    // rows addressable through the kmap (8 * parents when gathering parents)
    int32_t cin;
    const int32_t *kmap;
    int64_t n_out;
    int32_t kvol;
    const void *w;
    const float *bias;
    int32_t cout;      // output columns (row stride of y and residual)
    int32_t cout_pad;  // packed weight columns: cout rounded up to 32
    const void *residual;
    int32_t residual_shift;  // output row i adds residual row i >> residual_shift
    void *y;
    int32_t y_bf16;
    int32_t row_shift;  // kmap entry j reads source row j >> row_shift (3: parent of child j)
    int32_t ln;
    float eps;
    const float *ln_w;
    const float *ln_b;
    const float *mod_scale;
    const float *mod_shift;
    int32_t silu;
    const void *plan;  // per-tile gather plan records (halo kernel), or nullptr
    // Stream-K launches of the 8-wave halo kernel: sk_wgs equal runs over the
    // sk_units (column group, tile, chunk) units, and two FP32 128 x 128 tile
    // slots per run for the pieces that are part of a tile.
    int32_t sk_wgs;
    int64_t sk_units;
    float *sk_partial;
};

using KernelFn = void (*)(ConvArgs);

// Workgroup tilings of the MFMA kernel: 4 waves in WM x WN (WM = 4/WN), each
// wave MBW x NBW blocks of 32x32 outputs.
// Tilings 20, 21: the halo-staged kernel (conv_halo.hip), 128- and 64-row split-K tiles;
// 22: its 8-wave 128-row variant, launched only with a 128-row gather plan.
// Split-K tilings (splitk = 1): 128 rows x 32*nbw columns, each wave owning
// the whole tile for a quarter of the k-steps.  Ids 15 and 16 (BF16, 32- or
// 64-channel chunks) build each 128-channel task from 4 or 2 chunks.  Ids 17
// and 18 (BF16, 128 columns) use 64-row tiles, two workgroups per CU, with
// 128- and 64-channel tasks.
struct Tiling {
    int id, mbw, nbw, wn, splitk;
    int rows() const { return splitk ? 32 * mbw : 32 * mbw * (4 / wn); }
    int cols() const { return 32 * nbw * wn; }
};
inline constexpr Tiling kTilings[] = {
    {0, 1, 1, 1, 0}, {1, 1, 1, 2, 0}, {2, 1, 3, 1, 0}, {3, 1, 2, 2, 0}, {4, 1, 3, 2, 0},
    {5, 1, 4, 2, 0}, {6, 2, 1, 2, 0}, {7, 2, 3, 1, 0}, {8, 2, 2, 2, 0}, {9, 2, 3, 2, 0},
    {10, 1, 4, 1, 0}, {11, 4, 4, 1, 1}, {12, 4, 2, 1, 1}, {13, 4, 3, 1, 1}, {14, 4, 1, 1, 1},
    {15, 4, 3, 1, 1}, {16, 4, 4, 1, 1}, {18, 2, 4, 1, 1},
    {19, 2, 3, 1, 1}, {20, 4, 4, 1, 1}, {21, 2, 4, 1, 1}, {22, 4, 4, 1, 1},
    {23, 2, 1, 1, 1}, {24, 1, 1, 1, 1},
};

// MFMA kernel for tiling `id`, kc channels per task, xf 64-bit gathers;
// nullptr if that combination is not compiled.
KernelFn pick_mfma_bf16(int id, int kc, bool xf);
KernelFn pick_mfma_f32(int id, int kc, bool xf);
// 1x1-layer kernel for nbt 32-column blocks (1, 2, 3, 4, 6, 8), else nullptr.
KernelFn pick_linear_bf16(int nbt);
// linear_pipe_kernel for nbt column blocks and Cin = 16 * ks; nullptr for
// other shapes.
KernelFn pick_linear_pipe_bf16(int nbt, int ks);
KernelFn pick_linear_f32(int nbt);
// The halo-staged BF16 kernel for `rows`-row x (nb * 32)-column tiles
// (tiling 20: 128 rows, 21: 64 rows; nb 4, or 3 for 64-row tiles; 64-channel
// halo chunks; Cin a multiple of 64, Cout padded to whole tiles, kvol 27,
// inputs and weights below 2 GiB), else nullptr.
KernelFn pick_halo_bf16(int rows, int nb = 4);
// The halo kernels reading a precomputed gather plan (a.plan): 64-row tiles
// (4 waves, two workgroups per CU; 128 or 96 columns) or 128-row tiles (8
// waves, one workgroup per CU, launched with kHalo8Threads threads, 128
// columns); the plan builder (one workgroup per tile of `rows` rows); a plan
// record's bytes.
KernelFn pick_halo_bf16_planned(int rows, int nb = 4);
constexpr int kHalo8Threads = 512;
// The 8-wave kernel's stream-K variant (grid: a.sk_wgs runs of one
// workgroup, kHalo8Threads threads), and the pass that finishes the tiles its
// runs left in parts (after it, on the same stream).
KernelFn pick_halo8_stream_k();
void launch_halo8_combine(const ConvArgs &a, int64_t tiles, int groups, hipStream_t stream);
// The same for the FP32 split-K kernel of tiling 18 (64-row x 128-column
// tiles, 32-channel tasks, two workgroups per CU): its stream-K variant and
// the pass over its split tiles (tiles of 64 rows).
KernelFn pick_splitk_stream_k_f32();
void launch_splitk_combine_f32(const ConvArgs &a, int64_t tiles, int groups, hipStream_t stream);
void launch_gather_plan_build(int rows, const int32_t *kmap, int64_t n_out, int64_t n_src, int32_t row_shift,
                              void *plan, hipStream_t stream);
// Kernel map of coords (insert, then one workgroup per plan tile computing
// its 27 * rows entries) and the map's gather plan from the same lookups.
void launch_kmap_plan(int rows, const int32_t *coords, int64_t n, int32_t missing, int32_t *kmap, void *workspace,
                      uint64_t workspace_bytes, void *plan, hipStream_t stream);
constexpr int kGatherPlanRecord = 7168;      // 64-row tiles
constexpr int kGatherPlanRecord128 = 18432;  // 128-row tiles
// The FP32 1x1-layer kernel reading BF16 rows, else nullptr.
KernelFn pick_linear_f32_bf16_rows(int nbt);
// The same on BF16 MFMAs with three-term split weights (Cin = 16 * ksx,
// ksx in {2, 4, 6, 8}; nbt in 1..4), else nullptr.
KernelFn pick_linear_split(int nbt, int ksx, bool residual = false);

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kMaxKvol = 27;

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

// One 16-byte fragment of source row j (already shifted), channels c0 ..
// c0+E, with 64-bit addressing; a zero fragment when j < 0.
template <class T>
__device__ __forceinline__ uint4 load_fragment(const ConvArgs &a, int32_t j, int32_t c0) {
    if (j < 0) return make_uint4(0, 0, 0, 0);
    const T *xp = static_cast<const T *>(a.x) + static_cast<int64_t>(j) * a.cin + c0;
    return *reinterpret_cast<const uint4 *>(xp);
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

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Plain gather of one 16-byte fragment through a raw buffer resource: a
// missing neighbour (j < 0) gets an offset past the buffer end, which the
// hardware answers with zeros -- no branch, no wasted bandwidth.
template <class T>
__device__ __forceinline__ uint4 gather_plain(const void *base, int32_t bytes, int32_t j, int32_t cin,
                                              int32_t c0) {
    const uint32_t off = j >= 0 ? (static_cast<uint32_t>(j) * static_cast<uint32_t>(cin) +
                                   static_cast<uint32_t>(c0)) * static_cast<uint32_t>(sizeof(T))
                                : 0x80000000u;
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0), bytes,
                                          0x00020000),
        off, 0, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Weight chunk of one task: WFR 16-byte fragments, laid out as k-steps of
// ROW fragments (NBB column blocks x 64 lanes) that sit `stride` fragments
// apart in the packed global array.
template <int WPT, int WFR, int ROW>
__device__ __forceinline__ void load_weights(u32x4 (&wr)[WPT], const uint4 *src, int stride,
                                             int tid) {
    const u32x4 *v = reinterpret_cast<const u32x4 *>(src);
#pragma unroll
    for (int q = 0; q < WPT; ++q) {
        const int idx = tid + q * 256;
        if (WFR % 256 != 0 && idx >= WFR) continue;
        const int s = idx / ROW;
        wr[q] = v[static_cast<int64_t>(s) * stride + (idx - s * ROW)];
    }
}

template <int WPT, int WFR>
__device__ __forceinline__ void store_weights(uint4 *buf, const u32x4 (&wr)[WPT], int tid) {
    u32x4 *v = reinterpret_cast<u32x4 *>(buf);
#pragma unroll
    for (int q = 0; q < WPT; ++q) {
        const int idx = tid + q * 256;
        if (WFR % 256 != 0 && idx >= WFR) continue;
        v[idx] = wr[q];
    }
}

// Keeps the compiler from moving memory operations across this point.
__device__ __forceinline__ void mem_order() { asm volatile("" ::: "memory"); }

// Keeps the instruction scheduler from moving anything across this point
// (the prefetch loads stay ahead of the MFMAs that hide their latency).
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// Waits for this wave's LDS traffic, then joins the workgroup barrier.  Unlike
// __syncthreads() it leaves global loads in flight, so the next task's
// gathers and weight loads overlap the barrier and the MFMAs.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Row-major finish of a workgroup's FP32 output tile: TPR threads per row,
// 8 consecutive columns each, RPP rows per pass over BM rows (NTH threads).
template <int TPR, int BM, int NTH = 256>
struct RowMap {
    static constexpr int RPP = NTH / TPR;
    static constexpr int PASSES = (BM + RPP - 1) / RPP;
    static constexpr bool POW2 = (TPR & (TPR - 1)) == 0;  // row groups are aligned lane segments
};

// Loads the residual values a thread will finish (8 bf16 in [p][0], or 8
// floats in [p][0..1]); issued early so the latency overlaps other work.
template <int TPR, int BM, int NTH = 256>
__device__ __forceinline__ void load_residual(const ConvArgs &a, int64_t m0, int nb0, int tile_rows, int tid,
                                              uint4 (&res)[RowMap<TPR, BM, NTH>::PASSES][2]) {
    using RM = RowMap<TPR, BM, NTH>;
    const int cg = tid % TPR, rsub = tid / TPR;
    const int col0 = nb0 * 32 + cg * 8;
    // Whole 16-byte pieces (cout % 8 == 0), a residual under 2 GiB and at
    // most four passes (eight would spill in the 128-row split-K tiles): every
    // pass issues the same two buffer loads whatever it finds (no residual:
    // an empty resource; rows or columns outside the tile, and the second
    // piece of BF16 rows: an offset the resource drops, reading zeros), so
    // the passes' loads are in flight together -- with a load under a
    // condition the compiler waits for each pass's at its join.
    const int esz = a.y_bf16 ? 2 : 4;
    const int64_t res_rows = (a.n_out + (int64_t(1) << a.residual_shift) - 1) >> a.residual_shift;
    const int64_t res_bytes = a.residual ? res_rows * a.cout * esz : 0;
    if (RM::PASSES <= 4 && a.cout % 8 == 0 && res_bytes < (int64_t(1) << 31)) {
        const auto r_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(a.residual ? a.residual : a.y),
                                                              static_cast<short>(0), static_cast<int32_t>(res_bytes),
                                                              0x00020000);
        constexpr int32_t kOut = int32_t(0x80000000);
#pragma unroll
        for (int p = 0; p < RM::PASSES; ++p) {
            const int rl = p * RM::RPP + rsub;
            const bool in = rsub < RM::RPP && rl < tile_rows && col0 < a.cout;
            const int32_t off =
                in ? static_cast<int32_t>((((m0 + rl) >> a.residual_shift) * a.cout + col0) * esz) : kOut;
            const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(r_rsrc, off, 0, 0);
            const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(r_rsrc, in && esz == 4 ? off + 16 : kOut, 0, 0);
            res[p][0] = make_uint4(v0.x, v0.y, v0.z, v0.w);
            res[p][1] = make_uint4(v1.x, v1.y, v1.z, v1.w);
        }
        return;
    }
#pragma unroll
    for (int p = 0; p < RM::PASSES; ++p) {
        res[p][0] = res[p][1] = make_uint4(0, 0, 0, 0);
        const int rl = p * RM::RPP + rsub;
        if (!a.residual || rsub >= RM::RPP || rl >= tile_rows || col0 >= a.cout) continue;
        const int64_t off = ((m0 + rl) >> a.residual_shift) * a.cout + col0;
        if (a.cout % 8 != 0) {  // rows not 16-byte aligned: element loads of the real columns
            uint32_t w[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                w[k] = 0u;
                if (col0 + k < a.cout)
                    w[k] = a.y_bf16 ? static_cast<const uint16_t *>(a.residual)[off + k]
                                    : static_cast<const uint32_t *>(a.residual)[off + k];
            }
            if (a.y_bf16) {
                res[p][0] = make_uint4(w[0] | (w[1] << 16), w[2] | (w[3] << 16), w[4] | (w[5] << 16),
                                       w[6] | (w[7] << 16));
            } else {
                res[p][0] = make_uint4(w[0], w[1], w[2], w[3]);
                res[p][1] = make_uint4(w[4], w[5], w[6], w[7]);
            }
            continue;
        }
        if (a.y_bf16) {
            res[p][0] = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(a.residual) + off);
        } else {
            const uint4 *rp = reinterpret_cast<const uint4 *>(static_cast<const float *>(a.residual) + off);
            res[p][0] = rp[0];
            res[p][1] = rp[1];
        }
    }
}

// Finishes the tile staged in LDS (stg, BM rows x STG_LD floats): bias,
// LayerNorm over the row (the tile spans cout), modulate, SiLU, residual
// (prefetched by load_residual), 16-byte stores.  Row statistics are summed
// across the row's TPR lanes with shuffles when TPR is a power of two, else
// through `part` (2*BM*TPR floats of LDS).
// The per-column parameters of a thread's 8 columns from col0: bias,
// LayerNorm affine, modulation.  Padded columns (col >= cout, zero weights)
// read none.  Kernels with latency to hide load them early.
struct RowParams {
    float bias[8], lw[8], lb[8], ms[8], mh[8];
};
// Columns col0..col0+7 of a per-column float array (dflt for a null array
// and past cout): two 16-byte loads when the eight are real and the array
// is 16-byte aligned (col0 is a multiple of 8), else element loads.
__device__ __forceinline__ void load_cols8(const float *p, int col0, int cout, float dflt, float (&o)[8]) {
    if (p == nullptr) {
#pragma unroll
        for (int k = 0; k < 8; ++k) o[k] = dflt;
        return;
    }
    if (col0 + 8 <= cout && (reinterpret_cast<uintptr_t>(p) & 15u) == 0) {
        const float4 x0 = *reinterpret_cast<const float4 *>(p + col0);
        const float4 x1 = *reinterpret_cast<const float4 *>(p + col0 + 4);
        o[0] = x0.x; o[1] = x0.y; o[2] = x0.z; o[3] = x0.w;
        o[4] = x1.x; o[5] = x1.y; o[6] = x1.z; o[7] = x1.w;
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) o[k] = col0 + k < cout ? p[col0 + k] : dflt;
    }
}
// Bias and LayerNorm affine; the modulation separately (load_row_mod).
__device__ __forceinline__ void load_row_params(const ConvArgs &a, int col0, RowParams &q) {
    load_cols8(a.bias, col0, a.cout, 0.0f, q.bias);
    load_cols8(a.ln_w, col0, a.cout, 1.0f, q.lw);
    load_cols8(a.ln_b, col0, a.cout, 0.0f, q.lb);
}
__device__ __forceinline__ void load_row_mod(const ConvArgs &a, int col0, RowParams &q) {
    load_cols8(a.mod_scale, col0, a.cout, 0.0f, q.ms);
    load_cols8(a.mod_shift, col0, a.cout, 0.0f, q.mh);
}

// v, through an empty asm when ON: a value the compiler cannot hoist out of
// a loop around the caller.
template <bool ON>
__device__ __forceinline__ int opaque_scalar(int v) {
    if constexpr (ON) asm volatile("" : "+s"(v));
    return v;
}

// SWZ: the tile's 16-byte group q of row r sits at q ^ 8 when r & 4.
template <int TPR, int BM, int STG_LD, int NTH = 256, bool SWZ = false>
__device__ __forceinline__ void finish_rows(const ConvArgs &a, const float *stg, float *part, int64_t m0,
                                            int nb0, int tile_rows, int tid,
                                            const uint4 (&res)[RowMap<TPR, BM, NTH>::PASSES][2],
                                            const RowParams &q, float inv_cout = 0.0f) {
    using RM = RowMap<TPR, BM, NTH>;
    constexpr int RPP = RM::RPP;
    constexpr int PASSES = RM::PASSES;
    const int cg = tid % TPR, rsub = tid / TPR;
    const bool active = rsub < RPP;
    const int col0 = nb0 * 32 + cg * 8;  // global column of this thread's 8 values
    // (inv_cout: 1/cout formed by the caller, or 0 to form it here)
    const float inv_c = inv_cout != 0.0f ? inv_cout : 1.0f / static_cast<float>(a.cout);
    // Padded columns are not stored.  Rows of a cout that is not a multiple
    // of 8 are not 16-byte aligned: element stores.
    const bool ragged = a.cout % 8 != 0;
    const float(&bias8)[8] = q.bias;

    auto tile_vals = [&](int rl, float (&v)[8]) __attribute__((always_inline)) {
        const int c8 = SWZ ? (cg * 8) ^ (((rl >> 2) & 1) << 5) : cg * 8;
        const float4 *p = reinterpret_cast<const float4 *>(stg + rl * STG_LD + c8);
        const float4 x0 = p[0], x1 = p[1];
        v[0] = x0.x + bias8[0]; v[1] = x0.y + bias8[1]; v[2] = x0.z + bias8[2]; v[3] = x0.w + bias8[3];
        v[4] = x1.x + bias8[4]; v[5] = x1.y + bias8[5]; v[6] = x1.z + bias8[6]; v[7] = x1.w + bias8[7];
    };
    // Sum over the row's TPR lanes, every lane receiving the total.  A
    // 16-lane group is one DPP row: rotations by 8, 4, 2, 1 (VALU, no LDS).
    auto row_sum = [&](float x) __attribute__((always_inline)) {
        if constexpr (TPR == 16) {
            x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128, 0xf, 0xf, false));
            x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x124, 0xf, 0xf, false));
            x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x122, 0xf, 0xf, false));
            x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x121, 0xf, 0xf, false));
        } else {
#pragma unroll
            for (int d = TPR / 2; d >= 1; d >>= 1) x += __shfl_xor(x, d, TPR);
        }
        return x;
    };

    if constexpr (!RM::POW2) {
        if (a.ln) {
            // Row statistics through LDS partials.
            float *psum = part, *psq = part + BM * TPR;
#pragma unroll
            for (int p = 0; p < PASSES; ++p) {
                const int rl = p * RPP + rsub;
                if (!active || rl >= BM) continue;
                float v[8];
                tile_vals(rl, v);
                psum[rl * TPR + cg] = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
            }
            __syncthreads();
#pragma unroll
            for (int p = 0; p < PASSES; ++p) {
                const int rl = p * RPP + rsub;
                if (!active || rl >= BM) continue;
                float m = 0.0f;
                for (int g = 0; g < TPR; ++g) m += psum[rl * TPR + g];
                m *= inv_c;
                float v[8];
                tile_vals(rl, v);
                float q = 0.0f;
#pragma unroll
                for (int k = 0; k < 8; ++k) q += (v[k] - m) * (v[k] - m);
                psq[rl * TPR + cg] = q;
            }
            __syncthreads();
        }
    }

    // LayerNorm affine and modulate as one affine per column: the row's
    // t = (v - mean) * rstd becomes t * la + lc, la = lw (1 + ms) and
    // lc = lb (1 + ms) + mh (the modulate h * ms + h + mh of h = t * lw + lb).
    float la[8], lc[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        la[k] = q.lw[k];
        lc[k] = q.lb[k];
    }
    if (a.ln && a.mod_scale) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float s1 = 1.0f + q.ms[k];
            la[k] = q.lw[k] * s1;
            lc[k] = fmaf(q.lb[k], s1, q.mh[k]);
        }
    }
    // Power-of-two groups: LayerNorm statistics of every pass first, all
    // passes in lockstep so the cross-lane sums overlap (two-pass mean /
    // variance; every lane of a group takes part, whatever its row).
    float mean_p[PASSES], var_p[PASSES];
    float vs[RM::POW2 ? PASSES : 1][8];  // the thread's tile values, read once
    if constexpr (RM::POW2) {
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int rl = p * RPP + rsub;
            tile_vals(rl < BM ? rl : BM - 1, vs[p]);
        }
        if (a.ln) {
#pragma unroll
            for (int p = 0; p < PASSES; ++p)
                mean_p[p] = ((vs[p][0] + vs[p][1]) + (vs[p][2] + vs[p][3])) +
                            ((vs[p][4] + vs[p][5]) + (vs[p][6] + vs[p][7]));
#pragma unroll
            for (int p = 0; p < PASSES; ++p) mean_p[p] = row_sum(mean_p[p]) * inv_c;
            // vs becomes v - mean (used again to normalize)
#pragma unroll
            for (int p = 0; p < PASSES; ++p) {
                float d2 = 0.0f;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    vs[p][k] -= mean_p[p];
                    d2 += vs[p][k] * vs[p][k];
                }
                var_p[p] = d2;
            }
#pragma unroll
            for (int p = 0; p < PASSES; ++p) var_p[p] = row_sum(var_p[p]);
        }
    }
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        const int rl = p * RPP + rsub;
        if constexpr (!RM::POW2) {
            if (!active || rl >= tile_rows) continue;
        }
        float v[8];
        if constexpr (RM::POW2) {
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = vs[p][k];
        } else {
            tile_vals(rl, v);
        }
        if (a.ln) {
            float m, q;
            if constexpr (RM::POW2) {
                m = 0.0f;  // v already holds v - mean
                q = var_p[p];
            } else {
                m = 0.0f;
                q = 0.0f;
                for (int g = 0; g < TPR; ++g) {
                    m += part[rl * TPR + g];
                    q += part[BM * TPR + rl * TPR + g];
                }
                m *= inv_c;
            }
            const float rstd = rsqrtf(q * inv_c + a.eps);
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = fmaf((v[k] - m) * rstd, la[k], lc[k]);
        }
        if (a.silu) {
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = silu(v[k]);
        }
        if (rl >= tile_rows || col0 >= a.cout) continue;
        const int64_t off = (m0 + rl) * a.cout + col0;
        if (ragged) {
            if (a.residual) {
                const uint32_t rw[8] = {res[p][0].x, res[p][0].y, res[p][0].z, res[p][0].w,
                                        res[p][1].x, res[p][1].y, res[p][1].z, res[p][1].w};
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    v[k] += a.y_bf16 ? bf16_to_f32(static_cast<uint16_t>(k & 1 ? rw[k >> 1] >> 16 : rw[k >> 1] & 0xffffu))
                                     : __builtin_bit_cast(float, rw[k]);
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (col0 + k >= a.cout) continue;
                if (a.y_bf16) static_cast<uint16_t *>(a.y)[off + k] = f32_to_bf16(v[k]);
                else static_cast<float *>(a.y)[off + k] = v[k];
            }
            continue;
        }
        if (a.y_bf16) {
            if (a.residual) {
                const uint32_t rw[4] = {res[p][0].x, res[p][0].y, res[p][0].z, res[p][0].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    v[2 * k] += bf16_to_f32(static_cast<uint16_t>(rw[k] & 0xffffu));
                    v[2 * k + 1] += bf16_to_f32(static_cast<uint16_t>(rw[k] >> 16));
                }
            }
            uint32_t o4[4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                o4[k] = pack_bf16x2(v[2 * k], v[2 * k + 1]);
            // Streaming stores: the rows are read by the next kernel, likely
            // on another XCD, so they need not sit dirty in this XCD's L2
            // (whose write-back at kernel end is on the critical path).
            __builtin_nontemporal_store(u32x4{o4[0], o4[1], o4[2], o4[3]},
                                        reinterpret_cast<u32x4 *>(static_cast<uint16_t *>(a.y) + off));
        } else {
            float4 *yp = reinterpret_cast<float4 *>(static_cast<float *>(a.y) + off);
            if (a.residual) {
                const uint4 r0 = res[p][0], r1 = res[p][1];
                v[0] += __builtin_bit_cast(float, r0.x); v[1] += __builtin_bit_cast(float, r0.y);
                v[2] += __builtin_bit_cast(float, r0.z); v[3] += __builtin_bit_cast(float, r0.w);
                v[4] += __builtin_bit_cast(float, r1.x); v[5] += __builtin_bit_cast(float, r1.y);
                v[6] += __builtin_bit_cast(float, r1.z); v[7] += __builtin_bit_cast(float, r1.w);
            }
            __builtin_nontemporal_store(
                u32x4{__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[1]),
                      __builtin_bit_cast(uint32_t, v[2]), __builtin_bit_cast(uint32_t, v[3])},
                reinterpret_cast<u32x4 *>(yp));
            __builtin_nontemporal_store(
                u32x4{__builtin_bit_cast(uint32_t, v[4]), __builtin_bit_cast(uint32_t, v[5]),
                      __builtin_bit_cast(uint32_t, v[6]), __builtin_bit_cast(uint32_t, v[7])},
                reinterpret_cast<u32x4 *>(yp) + 1);
        }
    }
}

template <int TPR, int BM, int STG_LD, int NTH = 256>
__device__ __forceinline__ void finish_rows(const ConvArgs &a, const float *stg, float *part, int64_t m0,
                                            int nb0, int tile_rows, int tid,
                                            const uint4 (&res)[RowMap<TPR, BM, NTH>::PASSES][2]) {
    RowParams q;
    load_row_params(a, nb0 * 32 + (tid % TPR) * 8, q);
    load_row_mod(a, nb0 * 32 + (tid % TPR) * 8, q);
    finish_rows<TPR, BM, STG_LD, NTH>(a, stg, part, m0, nb0, tile_rows, tid, res, q);
}

// LDS budget of a tiling: two weight buffers, or (after the main loop) the
// FP32 output tile plus LayerNorm partials, then the neighbour-row table.
template <class T, int MBW, int NBW, int WN, int KC, int S>
struct ConvSmem {
    static constexpr int E = Frag<T>::E;
    static constexpr int KS = KC / (2 * E);
    static constexpr int BM = 32 * MBW * (4 / WN);
    static constexpr int NT = 32 * NBW * WN;
    static constexpr int WFR = KS * (NBW * WN) * 64;  // 16-byte weight fragments per task
    static constexpr int STG_LD = NT + 8;             // padded FP32 row of the output tile
    static constexpr int TPR = NT / 8;                // epilogue threads per row
    static constexpr int W_BYTES = 2 * S * WFR * 16;
    static constexpr int STG_BYTES = BM * STG_LD * 4;
    static constexpr int PART_BYTES = 2 * BM * TPR * 4;
    static constexpr int REGION0 = W_BYTES > STG_BYTES + PART_BYTES ? W_BYTES : STG_BYTES + PART_BYTES;
    static constexpr int ROWS_BYTES = BM * kMaxKvol * 4;
    static constexpr int TOTAL = REGION0 + ROWS_BYTES + 128;
    static constexpr int OCC = (TOTAL <= 80 * 1024 && MBW == 1) ? 2 : 1;
};

// T: uint16_t (bf16) or float.  XF: 0 = buffer-resource gathers (inputs
// below 2 GiB), 1 = 64-bit addressed gathers.
//
// Workgroup = 4 waves arranged WM x WN (WM = 4 / WN).  A wave owns MBW 32-row
// blocks x NBW 32-column blocks of the output (BM = WM*MBW*32 rows and
// NT = WN*NBW*32 columns per workgroup).  KC: Cin channels per task; a task is
// one (present offset, Cin chunk).
//
// Pipeline: S consecutive tasks form a stage.  While the MFMAs consume stage
// g (B fragments from LDS buffer g%2, A fragments in registers), the weight
// chunks and gathers of stage g+1 land in registers; the weights then go to
// buffer (g+1)%2.  A stage's weight loads precede its gathers, so the wait
// before the weights' LDS store leaves the gathers in flight.
//
// Epilogue: the FP32 tile goes through LDS and is finished row-major (bias,
// LayerNorm over the row, modulate, SiLU, residual) with 16-byte stores.
template <class T, int MBW, int NBW, int WN, int KC, int XF, int S>
__global__ void __launch_bounds__(256, (ConvSmem<T, MBW, NBW, WN, KC, S>::OCC))
conv_mfma_kernel(ConvArgs a) {
    using SM = ConvSmem<T, MBW, NBW, WN, KC, S>;
    constexpr int E = Frag<T>::E;
    constexpr int CPK = 2 * E;             // channels per k-step (both lane halves)
    constexpr int KS = SM::KS;             // k-steps per task
    constexpr int BM = SM::BM;
    constexpr int NBB = NBW * WN;          // 32-column blocks per workgroup
    constexpr int WFR = SM::WFR;
    constexpr int WPT = (WFR + 255) / 256; // weight fragments per thread per task
    __shared__ __align__(16) char smem[SM::TOTAL];
    uint4 *wlds0 = reinterpret_cast<uint4 *>(smem);
    uint4 *wlds1 = wlds0 + S * WFR;
    float *stg = reinterpret_cast<float *>(smem);
    float *part = reinterpret_cast<float *>(smem + SM::STG_BYTES);
    int32_t *rows = reinterpret_cast<int32_t *>(smem + SM::REGION0);
    int32_t *olist = rows + BM * kMaxKvol;
    uint32_t *omask = reinterpret_cast<uint32_t *>(olist + kMaxKvol);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int wm = wave / WN, wn = wave - (wave / WN) * WN;
    const int tile = xcd_tile(blockIdx.x, gridDim.x);
    const int64_t m0 = static_cast<int64_t>(tile) * BM;
    const int nb0 = blockIdx.y * NBB;  // first 32-column block of this workgroup
    const int nbtot = a.cout_pad / 32;
    const int kvol = a.kvol;
    const int ksteps_total = a.cin / CPK;
    const int chunks = a.cin / KC;
    const int tile_rows = static_cast<int>(min(static_cast<int64_t>(BM), a.n_out - m0));

    // ---- prologue: this tile's neighbour rows (-1 = missing) and offset mask
    if (tid == 0) *omask = 0;
    uint32_t my_mask = 0;
    if (a.kmap) {
        // The slice kmap[m0*kvol ..) is contiguous; stage it with independent
        // 16-byte loads (kvol is 27 or 1, divisions by constants).
        const int count = tile_rows * kvol;
        const int4 *src = reinterpret_cast<const int4 *>(a.kmap + m0 * kvol);
        constexpr int Q = (BM * kMaxKvol / 4 + 255) / 256;
        int4 v[Q];
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int e = (tid + q * 256) * 4;
            if (e + 3 < count) {
                v[q] = src[tid + q * 256];
            } else {
                v[q] = make_int4(-1, -1, -1, -1);
                if (e < count) v[q].x = a.kmap[m0 * kvol + e];
                if (e + 1 < count) v[q].y = a.kmap[m0 * kvol + e + 1];
                if (e + 2 < count) v[q].z = a.kmap[m0 * kvol + e + 2];
            }
        }
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int e0 = (tid + q * 256) * 4;
            const int jv[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int e = e0 + k;
                if (e >= BM * kvol) continue;
                const bool valid = e < count && jv[k] >= 0 && jv[k] < a.n_src;
                rows[e] = valid ? jv[k] >> a.row_shift : -1;
                const int o = kvol == 27 ? e % 27 : 0;
                if (valid) my_mask |= 1u << o;
            }
        }
    } else {
        for (int r = tid; r < BM; r += 256) {
            const int64_t j = m0 + r;
            const bool valid = r < tile_rows && j < a.n_src;
            rows[r] = valid ? static_cast<int32_t>(j >> a.row_shift) : -1;
            if (valid) my_mask = 1u;
        }
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) my_mask |= __shfl_xor(my_mask, d, 64);
    __syncthreads();
    if (lane == 0 && my_mask) atomicOr(omask, my_mask);
    __syncthreads();
    const uint32_t mask = *omask;
    if (tid == 0) {
        int k = 0;
        for (int o = 0; o < kvol; ++o)
            if ((mask >> o) & 1u) olist[k++] = o;
    }
    __syncthreads();
    const int ntasks = __popc(mask) * chunks;

    f32x16 acc[MBW][NBW];
#pragma unroll
    for (int mb = 0; mb < MBW; ++mb)
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb) acc[mb][nb] = f32x16{};

    const uint4 *wg = static_cast<const uint4 *>(a.w);
    const int half = lane >> 5;
    const int row_base = wm * MBW * 32 + (lane & 31);  // + mb*32
    const int32_t xbytes = static_cast<int32_t>(a.x_bytes < INT32_MAX ? a.x_bytes : INT32_MAX);

    auto load_w = [&](int t, u32x4 (&wr)[WPT]) __attribute__((always_inline)) {
        const int tq = t / chunks;
        const int kcv = (t - tq * chunks) * KC;
        load_weights<WPT, WFR, NBB * 64>(
            wr, wg + ((static_cast<int64_t>(olist[tq]) * ksteps_total + kcv / CPK) * nbtot + nb0) * 64,
            nbtot * 64, tid);
    };
    auto load_a = [&](int t, uint4 (&af)[MBW][KS]) __attribute__((always_inline)) {
        const int tq = t / chunks;
        const int kcv = (t - tq * chunks) * KC;
        const int o = olist[tq];
#pragma unroll
        for (int mb = 0; mb < MBW; ++mb) {
            const int32_t j = rows[(row_base + mb * 32) * kvol + o];
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                if constexpr (XF == 0)
                    af[mb][s] = gather_plain<T>(a.x, xbytes, j, a.cin, kcv + s * CPK + half * E);
                else
                    af[mb][s] = load_fragment<T>(a, j, kcv + s * CPK + half * E);
            }
        }
    };
    // B fragments are read from LDS one k-step ahead of the MFMAs that use
    // them (two register sets), so LDS latency hides behind MFMA issue.
    auto compute = [&](const uint4 (&af)[MBW][KS], const uint4 *buf) __attribute__((always_inline)) {
        uint4 bw[2][NBW];
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb) bw[0][nb] = buf[(wn * NBW + nb) * 64 + lane];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            if (s + 1 < KS) {
#pragma unroll
                for (int nb = 0; nb < NBW; ++nb)
                    bw[(s + 1) & 1][nb] = buf[((s + 1) * NBB + wn * NBW + nb) * 64 + lane];
            }
            sched_fence();
#pragma unroll
            for (int mb = 0; mb < MBW; ++mb)
#pragma unroll
                for (int nb = 0; nb < NBW; ++nb)
                    acc[mb][nb] = mfma_step<T>(af[mb][s], bw[s & 1][nb], acc[mb][nb]);
            sched_fence();
        }
    };
    // Stage g = tasks g*S .. g*S+S-1 (indices clamped so every stage issues
    // the same loads, which keeps the compiler's vmcnt waits exact).
    auto load_stage = [&](int g, uint4 (&af)[S][MBW][KS], u32x4 (&wr)[S][WPT]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < S; ++i) load_w(min(g * S + i, ntasks - 1), wr[i]);
        mem_order();
#pragma unroll
        for (int i = 0; i < S; ++i) load_a(min(g * S + i, ntasks - 1), af[i]);
    };
    auto store_stage = [&](uint4 *buf, const u32x4 (&wr)[S][WPT]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < S; ++i) store_weights<WPT, WFR>(buf + i * WFR, wr[i], tid);
    };
    auto compute_stage = [&](int g, const uint4 (&af)[S][MBW][KS], const uint4 *buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < S; ++i)
            if (S == 1 || g * S + i < ntasks) compute(af[i], buf + i * WFR);
    };

    if (ntasks > 0) {
        const int nstages = (ntasks + S - 1) / S;
        uint4 a0[S][MBW][KS], a1[S][MBW][KS];
        u32x4 wr[S][WPT];
        load_stage(0, a0, wr);
        store_stage(wlds0, wr);
        lds_barrier();
        for (int g = 0; g < nstages; g += 2) {
            load_stage(min(g + 1, nstages - 1), a1, wr);
            sched_fence();
            compute_stage(g, a0, wlds0);
            sched_fence();
            store_stage(wlds1, wr);
            lds_barrier();
            if (g + 1 >= nstages) break;
            load_stage(min(g + 2, nstages - 1), a0, wr);
            sched_fence();
            compute_stage(g + 1, a1, wlds1);
            sched_fence();
            store_stage(wlds0, wr);
            lds_barrier();
        }
    }
    uint4 res[RowMap<SM::TPR, BM>::PASSES][2];
    load_residual<SM::TPR, BM>(a, m0, nb0, tile_rows, tid, res);
    // Every wave is done with the weight buffers before the tile reuses them.
    __syncthreads();

    // ---- epilogue: FP32 tile through LDS, then row-major finish ----
#pragma unroll
    for (int mb = 0; mb < MBW; ++mb)
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb) {
            const int col = (wn * NBW + nb) * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int rl = (wm * MBW + mb) * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                stg[rl * SM::STG_LD + col] = acc[mb][nb][r];
            }
        }
    __syncthreads();

    finish_rows<SM::TPR, BM, SM::STG_LD>(a, stg, part, m0, nb0, tile_rows, tid, res);
}

// ---------------------------------------------------------------------------
// Split-K variant: each of the 4 waves owns the whole 128 x (32*NB) output
// tile (4 x NB accumulator blocks) but only k-steps s = wave (mod 4) of every
// task, so each B fragment is used by one wave only and is loaded straight
// from the packed weights (1 KiB contiguous per instruction).
//
// A (the gathered neighbour rows) is staged through LDS: the workgroup loads
// a task's 128 rows x KC channels with consecutive lanes on consecutive
// 16-byte pieces of one row, so every quarter-wave reads whole 128-byte
// lines.  (Loading MFMA fragments straight from global memory puts 16
// different rows in each quarter-wave and runs at about a quarter of the L1
// rate.)  Rows sit at a padded stride, which keeps both the row-major stores
// and the fragment reads free of bank conflicts.  Tasks run over all kvol
// offsets (weights of the first task are requested before the kernel map is
// staged); offsets absent from the tile skip their MFMAs.  The four partial
// tiles are summed through LDS in a fixed order (deterministic), then
// finished by the same row-major epilogue.
// ---------------------------------------------------------------------------
template <class T, int NB, int KC, int MB>
struct SplitSmem {
    static constexpr int BM = 32 * MB;
    static constexpr int RPH = MB == 4 ? 2 : 1;  // 32-row blocks reduced per phase
    static constexpr int NT = 32 * NB;
    static constexpr int ROWB = KC * static_cast<int>(sizeof(T));  // A bytes per row per task
    static constexpr int A_LD = ROWB + 16;                          // padded LDS row
    static constexpr int A_BYTES = 2 * BM * A_LD;                   // double buffer
    static constexpr int STG_LD = NT + 8;
    static constexpr int TPR = NT / 8;
    static constexpr int RED_BYTES = RPH * NB * 4 * 4096;  // per phase: RPH x NB blocks x 4 writers, 4 KiB each
    static constexpr int STG_BYTES = BM * STG_LD * 4;
    static constexpr int PART_BYTES = 2 * BM * TPR * 4;
    static constexpr int R0A = RED_BYTES > A_BYTES ? RED_BYTES : A_BYTES;
    static constexpr int REGION0 = R0A > STG_BYTES + PART_BYTES ? R0A : STG_BYTES + PART_BYTES;
    static constexpr int ROWS_BYTES = BM * kMaxKvol * 4;
    static constexpr int TOTAL = REGION0 + ROWS_BYTES + 128;
};

// Stream-K runs: run g takes units [sk_run_begin(g), sk_run_begin(g + 1)).
__device__ __forceinline__ int64_t sk_run_begin(int64_t g, int64_t units, int32_t runs) { return g * units / runs; }
// The run holding unit u (runs are non-empty when units >= runs).
__device__ __forceinline__ int sk_run_of(int64_t u, int64_t units, int32_t runs) {
    int g = static_cast<int>(min(static_cast<int64_t>(runs - 1), u * runs / units));
    while (g + 1 < runs && sk_run_begin(g + 1, units, runs) <= u) ++g;
    while (g > 0 && sk_run_begin(g, units, runs) > u) --g;
    return g;
}

// SUB > 1: a task is SUB consecutive sub-tasks (offset, KC/SUB-channel
// chunk), so that Cin of 96 (32-channel chunks) or 192 (64) still gives each
// wave whole k-steps of a 128-channel task.
//
// SK (conv_splitk_sk_kernel, SUB 1): stream-K runs over the (column group,
// tile, task) units, tasks counted over all kvol offsets of a tile, as the
// 8-wave halo kernel's (equal runs, whole tiles finished here, parts of a
// tile left as FP32 tiles in the run's two slots for splitk_combine_kernel).
template <class T, int NB, int KC, int XF, int SUB, int MB, bool SK>
__device__ __forceinline__ void splitk_body(const ConvArgs &a) {
    static_assert(!SK || SUB == 1, "stream-K runs walk single-chunk tasks");
    using SM = SplitSmem<T, NB, KC, MB>;
    constexpr int RPH = SM::RPH;
    constexpr int E = Frag<T>::E;
    constexpr int CPK = 2 * E;
    constexpr int KS = KC / CPK;  // k-steps per task
    static_assert(KS % 4 == 0, "k-steps per task must split over 4 waves");
    static_assert(SM::ROWB % 128 == 0, "A rows must cover whole 128-byte lines");
    constexpr int KSW = KS / 4;   // k-steps per wave per task
    constexpr int BM = SM::BM;
    constexpr int PPR = SM::ROWB / 16;       // 16-byte pieces per row
    constexpr int APT = BM * PPR / 256;      // pieces per thread per task
    constexpr int KCS = KC / SUB;            // channels per sub-task
    constexpr int KSS = KS / SUB;            // k-steps per sub-task
    constexpr int PPS = PPR / SUB;           // pieces per sub-task row
    static_assert(KC % SUB == 0 && KS % SUB == 0 && PPR % SUB == 0 && 256 % PPR == 0,
                  "sub-tasks must be whole k-steps and whole pieces");
    __shared__ __align__(16) char smem[SM::TOTAL];
    float *stg = reinterpret_cast<float *>(smem);
    float *part = reinterpret_cast<float *>(smem + SM::STG_BYTES);
    float4 *red = reinterpret_cast<float4 *>(smem);
    char *abuf = smem;
    int32_t *rows = reinterpret_cast<int32_t *>(smem + SM::REGION0);
    uint32_t *omask = reinterpret_cast<uint32_t *>(rows + BM * kMaxKvol);
    const int chunks_all = a.cin / (KC / SUB);  // sub-task chunks per offset

    // One tile's tasks [tb0, tb1) (all of them: 0, INT32_MAX), finished into
    // y, or with part_out its FP32 tile left there.
    auto piece = [&](const int tile, const int nb0, const int tb0, const int tb1, float *const part_out)
        __attribute__((always_inline)) {
    // (stream-K: the thread index passes an empty asm in each piece, so that
    // what derives from it is computed per piece, not hoisted out of the
    // run's loop and held -- spilled -- across every piece)
    int tid_v = static_cast<int>(threadIdx.x);
    if constexpr (SK) asm volatile("" : "+v"(tid_v));
    const int tid = tid_v, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int half = lane >> 5;
    const int64_t m0 = static_cast<int64_t>(tile) * BM;
    const int nbtot = a.cout_pad / 32;
    const int kvol = a.kvol;
    const int ksteps_total = a.cin / CPK;
    const int chunks = a.cin / KCS;  // sub-task chunks per offset
    const int tile_rows = static_cast<int>(min(static_cast<int64_t>(BM), a.n_out - m0));
    const int32_t xbytes = static_cast<int32_t>(a.x_bytes < INT32_MAX ? a.x_bytes : INT32_MAX);
    constexpr int ES = static_cast<int>(sizeof(T));
    // Packed weights through a buffer resource (the host keeps them < 2 GiB):
    // per task a scalar byte offset, per column block an immediate.
    const int64_t w_bytes = static_cast<int64_t>(kvol) * a.cin * a.cout_pad * ES;
    const auto w_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(a.w), static_cast<short>(0),
                                                          static_cast<int32_t>(w_bytes), 0x00020000);
    const auto x_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(a.x), static_cast<short>(0),
                                                          xbytes, 0x00020000);

    // Sub-tasks are the (present offset, Cin chunk) pairs in ascending
    // order.  A cursor walks them in scalar registers: the offsets not yet
    // visited as a bit mask, the current offset and chunk.  Past the last
    // sub-task it stays on the last one (prefetches beyond the end reload it
    // harmlessly).  A task takes the next SUB sub-tasks, packed as 16-bit
    // fields (offset | chunk << 5; chunks < 2048 as Cin <= 65536) of one
    // scalar, not an array the compiler would move to memory; `left` counts
    // the sub-tasks from its first one on, so those past the end
    // (left <= k) gather and multiply zeros.
    struct Cursor {
        uint32_t rest;
        int o, kc;
    };
    // Offsets are below 27, so bit 31 of the mask is never set: `more` comes
    // from the ctz (testing rest itself next to rest - 1 makes the compiler
    // use a vector subtract and a readfirstlane, ~20 cycles per task).
    auto advance = [&](Cursor &c) __attribute__((always_inline)) {
        const bool wrap = c.kc + 1 == chunks;
        const int next_o = __builtin_ctz(c.rest | 0x80000000u);
        const bool more = next_o != 31;
        const uint32_t cleared = c.rest & (c.rest - 1u);
        c.o = wrap && more ? next_o : c.o;
        c.kc = wrap ? (more ? 0 : c.kc) : c.kc + 1;
        c.rest = wrap && more ? cleared : c.rest;
    };
    static_assert(SUB <= 4, "four 16-bit sub-task fields");
    struct Task {
        int o, kc;    // SUB == 1
        uint64_t pk;  // SUB > 1
        int left;
    };
    auto next_task = [&](Cursor &cur, int &left, Task &t) __attribute__((always_inline)) {
        if constexpr (SUB == 1) {
            advance(cur);
            t.o = cur.o;
            t.kc = cur.kc;
        } else {
            uint64_t pk = 0;
#pragma unroll
            for (int k = 0; k < SUB; ++k) {
                advance(cur);
                pk |= static_cast<uint64_t>(static_cast<uint32_t>(cur.o | (cur.kc << 5))) << (16 * k);
            }
            t.pk = pk;
            t.left = left;
            left -= SUB;
        }
    };
    // (offset, chunk) of sub-task s (s may be per lane)
    auto sub_o = [&](const Task &t, int s) __attribute__((always_inline)) {
        return SUB == 1 ? t.o : static_cast<int>(static_cast<uint32_t>(t.pk >> (16 * s)) & 31u);
    };
    auto sub_kc = [&](const Task &t, int s) __attribute__((always_inline)) {
        return SUB == 1 ? t.kc : static_cast<int>((static_cast<uint32_t>(t.pk >> (16 * s)) & 0xffffu) >> 5);
    };
    const int my_sub = (tid % PPR) / PPS;  // this thread's pieces all lie in one sub-task
    // Fragment (k-step ks, column block cb) of the packed weights sits at
    // byte ((ks * nbtot + cb) * 64 + lane) * 16.  With ROT (NB = 4) wave w
    // keeps column block (k + w) mod 4 in accumulator k, so the block it owns
    // in the final reduction is always accumulator 0.
    constexpr bool ROT = NB == 4;
    // With one k-step per wave per task, the column block (rotated for ROT)
    // goes into a per-lane offset computed once: no scalar work per load.
    // With more, those registers would add spills: it goes into the scalar
    // offset (rotated) or the immediate.
    constexpr bool BVO = KSW == 1;
    int32_t bvo[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) bvo[nb] = lane * 16 + (ROT ? ((nb + wave) & 3) : nb) * 1024;
    auto load_b = [&](const Task &t, uint4 (&bf)[KSW][NB]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < KSW; ++i) {
            // k-step wave + 4 i of the task: step (wave + 4 i) % KSS of
            // sub-task (wave + 4 i) / KSS (wave-uniform, scalar)
            const int s = wave + 4 * i, sub = s / KSS;
            const int ks = sub_o(t, sub) * ksteps_total + sub_kc(t, sub) * KSS + (s - sub * KSS);
            int32_t sbase = (ks * nbtot + nb0) * 1024;
            if constexpr (SUB > 1) sbase = sub < t.left ? sbase : static_cast<int32_t>(0xC0000000u);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const u32x4 v =
                    BVO ? __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, bvo[nb], sbase, 0)
                    : ROT ? __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, lane * 16, sbase + ((nb + wave) & 3) * 1024, 0)
                          : __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, lane * 16 + nb * 1024, sbase, 0);
                bf[i][nb] = make_uint4(v.x, v.y, v.z, v.w);
            }
        }
    };
    // Row-major gather: piece u = tid + 256 q is row u / PPR = tid / PPR +
    // q * RS, channels kc*KC + (u % PPR)*E .. +E.  The staged map holds, per
    // (row, offset), the neighbour's byte offset in x (plain gathers; out of
    // range when missing, which the buffer load answers with zeros) or its
    // row index (64-bit gathers; -1 when missing), laid out [offset][row %
    // RS][row / RS] so that a thread's APT rows of an offset are one vector
    // read.
    constexpr int RS = 256 / PPR;  // rows apart of a thread's pieces
    static_assert(RS * APT == BM, "a thread's pieces cover one row per RS rows");
    auto map_slot = [&](int r, int o) __attribute__((always_inline)) { return (o * RS + r % RS) * APT + r / RS; };
    constexpr int32_t kNoRow = XF == 0 ? static_cast<int32_t>(0x80000000u) : -1;
    auto rows_of = [&](const Task &t, int32_t (&jn)[APT]) __attribute__((always_inline)) {
        const int o = sub_o(t, my_sub);
        const int32_t *src = rows + (o * RS + tid / PPR) * APT;
        if constexpr (APT % 4 == 0) {
#pragma unroll
            for (int q4 = 0; q4 < APT / 4; ++q4) {
                const int4 v = reinterpret_cast<const int4 *>(src)[q4];
                jn[4 * q4] = v.x;
                jn[4 * q4 + 1] = v.y;
                jn[4 * q4 + 2] = v.z;
                jn[4 * q4 + 3] = v.w;
            }
        } else if constexpr (APT == 2) {
            const int2 v = *reinterpret_cast<const int2 *>(src);
            jn[0] = v.x;
            jn[1] = v.y;
        } else {
#pragma unroll
            for (int q = 0; q < APT; ++q) jn[q] = src[q];
        }
#pragma unroll
        for (int q = 0; q < APT; ++q)
            if constexpr (SUB > 1) jn[q] = my_sub < t.left ? jn[q] : kNoRow;
    };
    auto gather = [&](const Task &t, int32_t j, int q) __attribute__((always_inline)) {
        const int piece = (tid + q * 256) % PPR;
        if constexpr (SUB == 1) {
            if constexpr (XF == 0) {
                const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(
                    x_rsrc, static_cast<int32_t>(static_cast<uint32_t>(j) + piece * 16), t.kc * KC * ES, 0);
                return make_uint4(v.x, v.y, v.z, v.w);
            } else {
                return load_fragment<T>(a, j, t.kc * KC + piece * E);
            }
        } else {
            // the chunk is per lane: it goes into the vector offset
            const int c0 = sub_kc(t, my_sub) * KCS + (piece % PPS) * E;
            if constexpr (XF == 0) {
                const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(
                    x_rsrc, static_cast<int32_t>(static_cast<uint32_t>(j) + static_cast<uint32_t>(c0 * ES)), 0, 0);
                return make_uint4(v.x, v.y, v.z, v.w);
            } else {
                return load_fragment<T>(a, j, c0);
            }
        }
    };
    auto load_a = [&](const Task &c, uint4 (&ra)[APT]) __attribute__((always_inline)) {
        int32_t jn[APT];
        rows_of(c, jn);
#pragma unroll
        for (int q = 0; q < APT; ++q) ra[q] = gather(c, jn[q], q);
    };
    auto a_slot = [&](char *buf, int q) __attribute__((always_inline)) {
        const int u = tid + q * 256;
        return reinterpret_cast<uint4 *>(buf + (u / PPR) * SM::A_LD + (u % PPR) * 16);
    };

    f32x16 acc[MB][NB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x16{};
    // A fragments of k-step (wave + 4 i) from an LDS buffer (lane: row
    // mb*32 + lane%32, channels (wave + 4 i)*CPK + half*E .. +E).
    auto read_frags = [&](const char *buf, uint4 (&af)[KSW][4]) __attribute__((always_inline)) {
        const char *base = buf + (lane & 31) * SM::A_LD + half * 16 + wave * (CPK * static_cast<int>(sizeof(T)));
#pragma unroll
        for (int i = 0; i < KSW; ++i)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                af[i][mb] = *reinterpret_cast<const uint4 *>(base + mb * 32 * SM::A_LD +
                                                             i * 4 * CPK * static_cast<int>(sizeof(T)));
    };
    // MFMAs number lo .. hi-1 of a task in (k-step, row block, column block)
    // order; the bounds are compile-time, so the unrolled loop keeps only
    // those.
    auto mfma_range = [&](auto lo_c, auto hi_c, const uint4 (&af)[KSW][4], const uint4 (&bf)[KSW][NB])
        __attribute__((always_inline)) {
        constexpr int lo = decltype(lo_c)::value, hi = decltype(hi_c)::value;
#pragma unroll
        for (int i = 0; i < KSW; ++i)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const int idx = (i * MB + mb) * NB + nb;
                    if (idx >= lo && idx < hi) acc[mb][nb] = mfma_step<T>(af[i][mb], bf[i][nb], acc[mb][nb]);
                }
    };

    // One task body (task t, its A fragments already in afc, its weights in
    // bc), split by one barrier:
    //   first half   the first half of the MFMAs, alternating with the LDS
    //                stores of A(t+1) (in ra) to wbuf and, into the freed
    //                registers, the gathers of A(t+2) (cursor nx);
    //   barrier      A(t+1) visible to every wave;
    //   second half  the other MFMAs, alternating with the reads of A(t+1)'s
    //                fragments into afn; then the weight loads of task t+2
    //                into bc.
    // The next body starts its MFMAs at once: its fragments are in registers.
    constexpr int MPS = sizeof(T) == 2 ? 1 : 4;  // MFMA instructions per fragment pair
    constexpr int NPAIR = KSW * MB * NB;          // fragment pairs per task
    constexpr int HALF = NPAIR / 2;
    constexpr int NMF1 = HALF * MPS, NMF2 = (NPAIR - HALF) * MPS;
    constexpr int M0 = NMF1 < 4 ? NMF1 : 4;       // MFMAs before the first LDS store
    constexpr int MI = (NMF1 - M0) / APT;
    constexpr int MR = NMF1 - M0 - MI * APT;
    constexpr int NFR = KSW * MB;                 // fragment reads
    constexpr int MJ = NMF2 / (NFR + 1);
    constexpr int MK = NMF2 - MJ * NFR;
    auto body = [&](const uint4 (&afc)[KSW][4], uint4 (&afn)[KSW][4], uint4 (&bc)[KSW][NB], char *wbuf,
                    uint4 (&ra)[APT], Task &nx, Cursor &cur, int &left) __attribute__((always_inline)) {
        int32_t jn[APT];
        rows_of(nx, jn);
        mfma_range(std::integral_constant<int, 0>{}, std::integral_constant<int, HALF>{}, afc, bc);
#pragma unroll
        for (int q = 0; q < APT; ++q) {
            *a_slot(wbuf, q) = ra[q];
            ra[q] = gather(nx, jn[q], q);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, APT, 0);      // DS read: row indices
        __builtin_amdgcn_sched_group_barrier(0x008, M0, 0);       // MFMA
#pragma unroll
        for (int q = 0; q < APT; ++q) {
            if constexpr (MI > 0) __builtin_amdgcn_sched_group_barrier(0x008, MI, 0);
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);    // DS write
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);    // VMEM read: gather
        }
        if constexpr (MR > 0) __builtin_amdgcn_sched_group_barrier(0x008, MR, 0);
        lds_barrier();
        mfma_range(std::integral_constant<int, HALF>{}, std::integral_constant<int, NPAIR>{}, afc, bc);
        read_frags(wbuf, afn);
        load_b(nx, bc);
#pragma unroll
        for (int k = 0; k < NFR; ++k) {
            if constexpr (MJ > 0) __builtin_amdgcn_sched_group_barrier(0x008, MJ, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);    // DS read: next fragments
        }
        if constexpr (MK > 0) __builtin_amdgcn_sched_group_barrier(0x008, MK, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, KSW * NB, 0); // VMEM read: weights
        next_task(cur, left, nx);
    };

    // ---- stage this tile's neighbour rows and offset mask
    auto staged = [&](bool valid, int32_t j) __attribute__((always_inline)) {
        j >>= a.row_shift;
        if constexpr (XF == 0) return valid ? j * a.cin * ES : static_cast<int32_t>(0x80000000u);
        else return valid ? j : -1;
    };
    if (tid == 0) *omask = 0;
    uint32_t my_mask = 0;
    if (a.kmap) {
        const int count = tile_rows * kvol;
        const int4 *src = reinterpret_cast<const int4 *>(a.kmap + m0 * kvol);
        constexpr int Q = (BM * kMaxKvol / 4 + 255) / 256;
        int4 v[Q];
        if (tile_rows == BM) {
            // Full tile (every tile but the last): BM*kvol is a multiple of
            // 4, so clamped 16-byte loads cover it without branches.
            const int last4 = BM * kvol / 4 - 1;
#pragma unroll
            for (int q = 0; q < Q; ++q) v[q] = src[min(tid + q * 256, last4)];
        } else {
#pragma unroll
            for (int q = 0; q < Q; ++q) {
                const int e = (tid + q * 256) * 4;
                if (e + 3 < count) {
                    v[q] = src[tid + q * 256];
                } else {
                    v[q] = make_int4(-1, -1, -1, -1);
                    if (e < count) v[q].x = a.kmap[m0 * kvol + e];
                    if (e + 1 < count) v[q].y = a.kmap[m0 * kvol + e + 1];
                    if (e + 2 < count) v[q].z = a.kmap[m0 * kvol + e + 2];
                }
            }
        }
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int e0 = (tid + q * 256) * 4;
            const int jv[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int e = e0 + k;
                if (e >= BM * kvol) continue;
                const bool valid = e < count && jv[k] >= 0 && jv[k] < a.n_src;
                const int r = kvol == kMaxKvol ? e / kMaxKvol : e;
                rows[map_slot(r, kvol == kMaxKvol ? e - r * kMaxKvol : 0)] = staged(valid, jv[k]);
                const int o = kvol == kMaxKvol ? e % kMaxKvol : 0;
                if (valid) my_mask |= 1u << o;
            }
        }
    } else {
        for (int r = tid; r < BM; r += 256) {
            const int64_t j = m0 + r;
            const bool valid = r < tile_rows && j < a.n_src;
            rows[map_slot(r, 0)] = staged(valid, static_cast<int32_t>(j));
            if (valid) my_mask = 1u;
        }
    }
    // Wave OR: within each 16-lane DPP row, then across the four rows.
    {
        int m = static_cast<int>(my_mask);
        m |= __builtin_amdgcn_update_dpp(0, m, 0x128, 0xf, 0xf, false);
        m |= __builtin_amdgcn_update_dpp(0, m, 0x124, 0xf, 0xf, false);
        m |= __builtin_amdgcn_update_dpp(0, m, 0x122, 0xf, 0xf, false);
        m |= __builtin_amdgcn_update_dpp(0, m, 0x121, 0xf, 0xf, false);
        my_mask = static_cast<uint32_t>(__builtin_amdgcn_readlane(m, 0) | __builtin_amdgcn_readlane(m, 16) |
                                        __builtin_amdgcn_readlane(m, 32) | __builtin_amdgcn_readlane(m, 48));
    }
    lds_barrier();
    if (lane == 0 && my_mask) atomicOr(omask, my_mask);
    lds_barrier();
    const uint32_t mask = __builtin_amdgcn_readfirstlane(*omask);
    const int nsub = __popc(mask) * chunks;
    const int ntasks = (nsub + SUB - 1) / SUB;
    // this piece's tasks [tb, tb + cnt) (a stream-K range over the nominal
    // kvol * chunks tasks holds fewer where offsets are absent)
    const int tb = min(tb0, ntasks), cnt = min(tb1, ntasks) - tb;

    // ---- main loop.  Entering task t: A(t)'s fragments in registers, A(t+1)
    // on its way into ra, B(t) and B(t+1) in registers or on their way.
    if (cnt > 0) {
        char *buf0 = abuf, *buf1 = abuf + BM * SM::A_LD;
        uint4 b0[KSW][NB], b1[KSW][NB];
        uint4 fx[KSW][4], fy[KSW][4];
        uint4 ra[APT];
        // An odd task count peels task 0 before the loop, so the loop always
        // runs whole pairs; the peel's weights and fragments then live in the
        // other register sets, and the two LDS buffers swap roles.
        const bool odd = cnt & 1;
        Cursor cur{mask, -1, chunks - 1};
        if constexpr (SK) {
            // the cursor as task tb - 1 leaves it: its offset is the r-th
            // present one, its chunk (tb - 1) % chunks
            if (tb > 0) {
                const int r = (tb - 1) / chunks;
                uint32_t rest = mask;
                for (int k = 0; k < r; ++k) rest &= rest - 1u;
                const int o = __builtin_ctz(rest | 0x80000000u);
                cur = Cursor{rest & (rest - 1u), o, (tb - 1) - r * chunks};
            }
        }
        int left = nsub;
        Task nx;
        next_task(cur, left, nx);  // task 0
        load_a(nx, ra);
        if (odd) load_b(nx, b1);
        else load_b(nx, b0);
#pragma unroll
        for (int q = 0; q < APT; ++q) *a_slot(buf0, q) = ra[q];
        next_task(cur, left, nx);  // task 1
        load_a(nx, ra);
        // Gathers before weights, as in the loop body: the wait counts at the
        // loop head then match steady state (else the first body of each pair
        // also waits for the weights issued after its gathers).
        sched_fence();
        if (odd) load_b(nx, b0);
        else load_b(nx, b1);
        next_task(cur, left, nx);  // task 2
        lds_barrier();
        // The task loop at raised wave priority: where the other workgroup on
        // the CU is in its prologue, reduction or epilogue, this one's MFMA
        // stream issues first (same-box A/B: -1.4% BF16, -0.6% FP32).
        __builtin_amdgcn_s_setprio(1);
        if (odd) {
            read_frags(buf0, fy);
            body(fy, fx, b1, buf1, ra, nx, cur, left);
            char *tmp = buf0;
            buf0 = buf1;
            buf1 = tmp;
        } else {
            read_frags(buf0, fx);
        }
        for (int t = odd ? 1 : 0; t < cnt; t += 2) {
            body(fx, fy, b0, buf1, ra, nx, cur, left);
            body(fy, fx, b1, buf0, ra, nx, cur, left);
        }
        lds_barrier();  // the last fragment reads finish before the tile reuses LDS
        __builtin_amdgcn_s_setprio(0);
    }

    // ---- reduce the 4 partial tiles through LDS, in two phases ----
    // Phase p covers row blocks RPH*p .. RPH*p+RPH-1 (RPH = 2 for 128-row
    // tiles, 1 for 64-row ones); pair (h, c) = (block RPH*p+h, column
    // block c) is summed by wave (h*NB + c) % 4 into registers, the other
    // waves handing their partials over as float4 [4][lane] slots (16-byte
    // lane stride, conflict-free).  With ROT the owner keeps its own partial
    // (accumulator 0) and only three cross LDS.  Sums run in a fixed order,
    // so results are deterministic.  Accumulators are only indexed by
    // compile-time constants.
    constexpr int PPW = (RPH * NB + 3) / 4;  // pairs per wave per phase
    constexpr int NPH = MB / RPH;            // phases (one for 32-row tiles)
    auto slot_of = [&](int h, int c, int writer) __attribute__((always_inline)) {
        return red + ((h * NB + c) * 4 + writer) * (4 * 64);
    };
    float fin[NPH][PPW][16];
#pragma unroll
    for (int p = 0; p < NPH; ++p) {
        if (p) __syncthreads();
#pragma unroll
        for (int h = 0; h < RPH; ++h)
#pragma unroll
            for (int k = ROT ? 1 : 0; k < NB; ++k) {
                const int c = ROT ? ((k + wave) & 3) : k;
                float4 *slot = slot_of(h, c, wave);
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    slot[g * 64 + lane] = make_float4(acc[RPH * p + h][k][4 * g], acc[RPH * p + h][k][4 * g + 1],
                                                      acc[RPH * p + h][k][4 * g + 2], acc[RPH * p + h][k][4 * g + 3]);
            }
        __syncthreads();
        if constexpr (ROT) {
            // Wave w owns (h, w) for h = 0, 1: its accumulator 0 plus the
            // other three waves' slots.
#pragma unroll
            for (int h = 0; h < RPH; ++h)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    float4 sum = make_float4(acc[RPH * p + h][0][4 * g], acc[RPH * p + h][0][4 * g + 1],
                                             acc[RPH * p + h][0][4 * g + 2], acc[RPH * p + h][0][4 * g + 3]);
#pragma unroll
                    for (int s2 = 1; s2 < 4; ++s2) {
                        const float4 v = slot_of(h, wave, (wave + s2) & 3)[g * 64 + lane];
                        sum.x += v.x;
                        sum.y += v.y;
                        sum.z += v.z;
                        sum.w += v.w;
                    }
                    fin[p][h][4 * g] = sum.x;
                    fin[p][h][4 * g + 1] = sum.y;
                    fin[p][h][4 * g + 2] = sum.z;
                    fin[p][h][4 * g + 3] = sum.w;
                }
        } else {
#pragma unroll
            for (int i = 0; i < PPW; ++i) {
                const int q = wave + 4 * i;
                if (q >= RPH * NB) continue;
                const int h = q / NB, c = q - h * NB;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                    for (int src = 0; src < 4; ++src) {
                        const float4 v = slot_of(h, c, src)[g * 64 + lane];
                        sum.x += v.x;
                        sum.y += v.y;
                        sum.z += v.z;
                        sum.w += v.w;
                    }
                    fin[p][i][4 * g] = sum.x;
                    fin[p][i][4 * g + 1] = sum.y;
                    fin[p][i][4 * g + 2] = sum.z;
                    fin[p][i][4 * g + 3] = sum.w;
                }
            }
        }
    }
    __syncthreads();
    // Summed blocks -> FP32 tile in LDS (the tile aliases the slots).
#pragma unroll
    for (int p = 0; p < NPH; ++p)
#pragma unroll
        for (int i = 0; i < PPW; ++i) {
            const int q = wave + 4 * i;
            if (q >= RPH * NB) continue;
            const int h = q / NB, c = q - h * NB;
            const int col = c * 32 + (lane & 31);
            const int rb = (RPH * p + h) * 32 + 4 * half;
#pragma unroll
            for (int r = 0; r < 16; ++r) stg[(rb + 8 * (r >> 2) + (r & 3)) * SM::STG_LD + col] = fin[p][i][r];
        }
    if (SK && part_out) {
        // part of a tile: its FP32 tile, rows in order, to the partial slot
        constexpr int C4 = SM::NT / 4;
        static_assert(BM * C4 % 256 == 0, "whole 16-byte pieces per thread");
        __syncthreads();
#pragma unroll
        for (int k = 0; k < BM * C4 / 256; ++k) {
            const int pc = tid + k * 256, row = pc / C4, c4 = pc - row * C4;
            reinterpret_cast<float4 *>(part_out)[pc] =
                *reinterpret_cast<const float4 *>(stg + row * SM::STG_LD + 4 * c4);
        }
    } else {
        uint4 res[RowMap<SM::TPR, BM>::PASSES][2];
        load_residual<SM::TPR, BM>(a, m0, nb0, tile_rows, tid, res);
        __syncthreads();
        finish_rows<SM::TPR, BM, SM::STG_LD>(a, stg, part, m0, nb0, tile_rows, tid, res);
    }
    };
    if constexpr (!SK) {
        piece(xcd_tile(blockIdx.x, gridDim.x), blockIdx.y * NB, 0, INT32_MAX, nullptr);
    } else {
        const int64_t tiles = (a.n_out + BM - 1) / BM;
        const int64_t ntf = static_cast<int64_t>(a.kvol) * chunks_all;  // nominal tasks per tile
        const int g = xcd_tile(blockIdx.x, gridDim.x);  // XCD-contiguous runs
        const int64_t u1 = sk_run_begin(g + 1, a.sk_units, a.sk_wgs);
        int slot = 0;
        for (int64_t u = sk_run_begin(g, a.sk_units, a.sk_wgs); u < u1;) {
            const int64_t gt = u / ntf;  // column group * tiles + tile
            const int t0 = static_cast<int>(u - gt * ntf);
            const int t1 = static_cast<int>(min(ntf, t0 + (u1 - u)));
            const int grp = static_cast<int>(gt / tiles);
            const bool whole = t0 == 0 && t1 == ntf;
            __syncthreads();  // the previous piece is done with LDS
            piece(static_cast<int>(gt - grp * tiles), grp * NB, t0, t1,
                  whole ? nullptr : a.sk_partial + (static_cast<int64_t>(g) * 2 + slot) * (BM * SM::NT));
            slot += whole ? 0 : 1;
            u += t1 - t0;
        }
    }
}

template <class T, int NB, int KC, int XF, int SUB, int MB>
__global__ void __launch_bounds__(256, MB == 4 ? 1 : 2) conv_splitk_kernel(ConvArgs a) {
    splitk_body<T, NB, KC, XF, SUB, MB, false>(a);
}
template <class T, int NB, int KC, int XF, int SUB, int MB>
__global__ void __launch_bounds__(256, MB == 4 ? 1 : 2) conv_splitk_sk_kernel(ConvArgs a) {
    splitk_body<T, NB, KC, XF, SUB, MB, true>(a);
}

// The tiles that a split-K kernel's stream-K runs left in parts: the pieces'
// FP32 tiles added in task order (the runs in order), then the epilogue of
// the whole-tile path.  One workgroup per (tile, column group); tiles one
// run covers whole were finished by the conv kernel and are skipped.
template <class T, int NB, int KC, int MB>
__global__ void __launch_bounds__(256) splitk_combine_kernel(ConvArgs a) {
    using SM = SplitSmem<T, NB, KC, MB>;
    constexpr int BM = SM::BM, C4 = SM::NT / 4, K = BM * C4 / 256;
    __shared__ __align__(16) char smem[SM::STG_BYTES + SM::PART_BYTES];
    float *stg = reinterpret_cast<float *>(smem);
    float *part = reinterpret_cast<float *>(smem + SM::STG_BYTES);
    const int tid = threadIdx.x;
    const int64_t tiles = gridDim.x;
    const int tile = blockIdx.x, nb0 = blockIdx.y * NB;
    const int64_t ntf = static_cast<int64_t>(a.kvol) * (a.cin / KC);
    const int64_t uf = (static_cast<int64_t>(blockIdx.y) * tiles + tile) * ntf, ul = uf + ntf - 1;
    const int gf = sk_run_of(uf, a.sk_units, a.sk_wgs), gl = sk_run_of(ul, a.sk_units, a.sk_wgs);
    if (gf == gl) return;
    const int64_t m0 = static_cast<int64_t>(tile) * BM;
    const int tile_rows = static_cast<int>(min(static_cast<int64_t>(BM), a.n_out - m0));
    float4 sum[K];
    for (int g = gf; g <= gl; ++g) {
        // this tile's piece is run g's second partial one when the run began
        // in the middle of an earlier tile
        const int64_t b = sk_run_begin(g, a.sk_units, a.sk_wgs);
        const int slot = b < uf && b % ntf != 0 ? 1 : 0;
        const float4 *src = reinterpret_cast<const float4 *>(a.sk_partial + (static_cast<int64_t>(g) * 2 + slot) * (BM * SM::NT));
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const float4 v = src[tid + k * 256];
            if (g == gf) {
                sum[k] = v;
            } else {
                sum[k].x += v.x;
                sum[k].y += v.y;
                sum[k].z += v.z;
                sum[k].w += v.w;
            }
        }
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int pc = tid + k * 256, row = pc / C4, c4 = pc - row * C4;
        *reinterpret_cast<float4 *>(stg + row * SM::STG_LD + 4 * c4) = sum[k];
    }
    uint4 res[RowMap<SM::TPR, BM>::PASSES][2];
    load_residual<SM::TPR, BM>(a, m0, nb0, tile_rows, tid, res);
    __syncthreads();
    finish_rows<SM::TPR, BM, SM::STG_LD>(a, stg, part, m0, nb0, tile_rows, tid, res);
}

// Compiled tilings (tiling id -> MBW, NBW, WN, S); one task's weight chunk
// is at most 32 KiB.
//   0: 1,1,1,1  1: 1,1,2,1  2: 1,3,1,1  3: 1,2,2,1  4: 1,3,2,1  5: 1,4,2,1
//   6: 2,1,2,1  7: 2,3,1,1  8: 2,2,2,1  9: 2,3,2,1  10: 1,4,1,2
//   11-14: split-K, 128 rows x 128 / 64 / 96 / 32 columns
//   15, 16: split-K, 128 rows x 96 / 128 columns, 128-channel tasks joined
//           from 32- or 64-channel chunks; 19: 15 with 64 rows
//   17, 18: split-K, 64 rows x 128 columns, 128- / 64-channel tasks
//   23, 24: split-K, FP32, 64 / 32 rows x 32 columns
// 1x1 layers (kvol 1, no map): y[r] = W x[r >> row_shift] + bias, then SiLU
// and the residual.  Persistent workgroups: the packed weights (every k-step
// of all NBT column blocks) are copied to LDS once; each wave then takes
// 32-row blocks of the grid-stride sequence, streams its A fragments straight
// from the rows two k-steps ahead (a row past the end reads zeros through
// the buffer resource), and stores from the accumulators: no split-K
// reduction and no staging, which dominate a 27-offset kernel run on one
// offset.  Requires x_bytes < 2 GiB and at most kLinearMaxFrags packed
// weight fragments.
constexpr int kLinearMaxFrags = 4096;  // 64 KiB of LDS

// Stores one 32-row block of a 1x1 layer from its accumulators: bias,
// SiLU, residual, then the output dtype (EPC output elements per 16-byte
// store).  stg is this wave's 8 staging rows of NBT*32+4 floats.
template <int NBT, int EPC>
__device__ __forceinline__ void linear_store_block(const ConvArgs &a, const f32x16 (&acc)[NBT],
                                                   const float (&bias)[NBT], float *stg, int64_t blk,
                                                   int lane, int half) {
    constexpr int SLD = NBT * 32 + 4;
    // D layout: lane l holds column l % 32; register j holds row
    // 8*(j/4) + 4*(l/32) + j%4 of the block.  Rows 8g..8g+7 (registers
    // 4g..4g+3) go through this wave's LDS rows, then leave as one
    // contiguous, 16-byte-aligned span of 8*cout elements (8*cout*size is
    // a multiple of 16): full-width stores, not row pieces that straddle
    // cache lines.
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int64_t row0 = blk * 32 + 8 * g;
        if (row0 >= a.n_out) break;
#pragma unroll
        for (int cb = 0; cb < NBT; ++cb)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                stg[(4 * half + q) * SLD + cb * 32 + (lane & 31)] = acc[cb][4 * g + q] + bias[cb];
        const int elems = static_cast<int>(min(static_cast<int64_t>(8), a.n_out - row0)) * a.cout;
        for (int c = lane; c * EPC < elems; c += 64) {
            const int e0 = c * EPC;
            int rr = e0 / a.cout, cc = e0 - rr * a.cout;
            float v[EPC];
#pragma unroll
            for (int i = 0; i < EPC; ++i) {
                const bool in = e0 + i < elems;
                v[i] = in ? stg[rr * SLD + cc] : 0.0f;
                if (a.silu) v[i] = silu(v[i]);
                if (a.residual && in) {
                    const int64_t roff = ((row0 + rr) >> a.residual_shift) * a.cout + cc;
                    v[i] += a.y_bf16 ? bf16_to_f32(static_cast<const uint16_t *>(a.residual)[roff])
                                     : static_cast<const float *>(a.residual)[roff];
                }
                if (++cc == a.cout) {
                    cc = 0;
                    ++rr;
                }
            }
            const int64_t off = row0 * a.cout + e0;
            if (e0 + EPC <= elems) {
                if (a.y_bf16) {
                    uint32_t w[EPC / 2];
#pragma unroll
                    for (int i = 0; i < EPC / 2; ++i)
                        w[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
                    if constexpr (EPC == 8)
                        *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(a.y) + off) = make_uint4(w[0], w[1], w[2], w[3]);
                    else
                        *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(a.y) + off) = make_uint2(w[0], w[1]);
                } else {
                    if constexpr (EPC == 4)
                        *reinterpret_cast<float4 *>(static_cast<float *>(a.y) + off) = make_float4(v[0], v[1], v[2], v[3]);
                    else
#pragma unroll
                        for (int i = 0; i < EPC; ++i) static_cast<float *>(a.y)[off + i] = v[i];
                }
            } else {
#pragma unroll
                for (int i = 0; i < EPC; ++i) {
                    if (e0 + i >= elems) break;
                    if (a.y_bf16) static_cast<uint16_t *>(a.y)[off + i] = f32_to_bf16(v[i]);
                    else static_cast<float *>(a.y)[off + i] = v[i];
                }
            }
        }
    }
}

// XB (FP32 layers only): x holds BF16 rows, widened exactly as each A
// fragment is loaded (8 bytes per lane instead of 16).
template <class T, int NBT, bool XB = false>
__global__ void __launch_bounds__(256) linear_kernel(ConvArgs a) {
    static_assert(!XB || sizeof(T) == 4, "BF16 rows feed FP32 layers only");
    extern __shared__ uint4 wl[];
    constexpr int E = Frag<T>::E, CPK = 2 * E;
    constexpr int ES = XB ? 2 : static_cast<int>(sizeof(T));  // bytes per x element
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = lane >> 5;
    const int ks_total = a.cin / CPK;
    const uint4 *wg = static_cast<const uint4 *>(a.w);
    for (int f = tid; f < ks_total * NBT * 64; f += 256) wl[f] = wg[f];
    __syncthreads();
    // Output staging after the weights: 8 rows of SLD floats per wave.
    constexpr int SLD = NBT * 32 + 4;
    constexpr int EPC = sizeof(T) == 2 ? 8 : 4;  // output elements per 16-byte store (fp32 out: 4)
    float *stg = reinterpret_cast<float *>(wl + ks_total * NBT * 64) + wave * 8 * SLD;
    const auto x_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(a.x), static_cast<short>(0),
                                                          static_cast<int32_t>(a.x_bytes), 0x00020000);
    float bias[NBT];
#pragma unroll
    for (int cb = 0; cb < NBT; ++cb) {
        const int col = cb * 32 + (lane & 31);
        bias[cb] = a.bias && col < a.cout ? a.bias[col] : 0.0f;
    }
    const int64_t nblk = (a.n_out + 31) / 32;
    for (int64_t blk = static_cast<int64_t>(blockIdx.x) * 4 + wave; blk < nblk;
         blk += static_cast<int64_t>(gridDim.x) * 4) {
        const int64_t r = blk * 32 + (lane & 31);
        const uint32_t base = r < a.n_out
                                  ? static_cast<uint32_t>(((r >> a.row_shift) * a.cin + half * E) * ES)
                                  : 0x80000000u;
        auto load_a = [&](int st) __attribute__((always_inline)) {
            const int32_t off = static_cast<int32_t>(base + static_cast<uint32_t>(st * CPK * ES));
            if constexpr (XB) {
                typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
                const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(x_rsrc, off, 0, 0);
                return make_uint4(v.x << 16, v.x & 0xffff0000u, v.y << 16, v.y & 0xffff0000u);
            } else {
                const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, off, 0, 0);
                return make_uint4(v.x, v.y, v.z, v.w);
            }
        };
        f32x16 acc[NBT];
#pragma unroll
        for (int cb = 0; cb < NBT; ++cb) acc[cb] = f32x16{};
        // Loads run two k-steps ahead without a branch (one around a load
        // would make the compiler wait for every load at the join); the two
        // past the row's end read the next row or zeros and go unused.
        uint4 a0 = load_a(0);
        uint4 a1 = load_a(1);
        for (int st = 0; st < ks_total; ++st) {
            const uint4 cur = a0;
            a0 = a1;
            a1 = load_a(st + 2);
#pragma unroll
            for (int cb = 0; cb < NBT; ++cb) acc[cb] = mfma_step<T>(cur, wl[(st * NBT + cb) * 64 + lane], acc[cb]);
        }
        linear_store_block<NBT, EPC>(a, acc, bias, stg, blk, lane, half);
    }
}

// BF16 1x1 layers with Cin = 16 * KS (KS in {4, 8, 12, 16}), Cout a multiple
// of 8 and no residual, pipelined across a wave's row blocks.  Persistent
// workgroups of 4 waves with the weights in LDS, as in linear_kernel; wave w
// of G workgroups takes 32-row blocks w, w + 4G, ...  A wave holds all KS
// A fragments of its block in registers and loads the next block's (a second
// register set, the two used in turn) before the current block's MFMAs, so
// after the first block no block waits for its rows.  Rows 8g..8g+7 of a
// block go through this wave's 8 staging rows and leave as the same number
// of 16-byte buffer stores for every group (slots past the span get an
// offset the resource drops), and the first block's loads are followed by
// as many dropped stores: the compiler's count of the memory operations
// younger than a block's loads is then the same on every path, so the wait
// for them never covers the previous block's stores.
// Layers wider than NBT column blocks (NBT = 4, a multiple of 4 blocks) take
// one group of NBT blocks per blockIdx.y, with that group's weights in LDS.
template <int NBT, int KS>
__global__ void __launch_bounds__(256) linear_pipe_kernel(ConvArgs a) {
    extern __shared__ uint4 wl[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = lane >> 5;
    const int nbtot = a.cout_pad / 32;       // column blocks of the layer
    const int col0 = blockIdx.y * NBT * 32;  // this workgroup's first column
    constexpr int SLD = NBT * 32 + 4;                 // staging row stride (floats)
    constexpr int KP = (NBT * 32 + 63) / 64;          // 16-byte slots a lane per 8-row group
    constexpr int kStores = 4 * KP;                   // stores a block
    constexpr int kOut = int32_t(0x80000000);         // an offset every resource drops
    const int cout = a.cout;
    const auto x_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(a.x), static_cast<short>(0),
                                                          static_cast<int32_t>(a.x_bytes), 0x00020000);
    const auto y_rsrc = __builtin_amdgcn_make_buffer_rsrc(a.y, static_cast<short>(0),
                                                          static_cast<int32_t>(a.n_out * cout * 2), 0x00020000);
    const auto drop_rsrc = __builtin_amdgcn_make_buffer_rsrc(a.y, static_cast<short>(0), 0, 0x00020000);
    const int64_t nblk = (a.n_out + 31) / 32;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 4;
    // Lane: row lane % 32 of the block, channels ks*16 + half*8 .. +8; rows
    // past the end (blocks after the wave's last) read zeros.
    auto load_block = [&](int64_t blk, uint4 (&f)[KS]) __attribute__((always_inline)) {
        const int64_t r = blk * 32 + (lane & 31);
        const uint32_t base = r < a.n_out ? static_cast<uint32_t>(((r >> a.row_shift) * a.cin + half * 8) * 2)
                                          : 0x80000000u;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, static_cast<int32_t>(base + ks * 32), 0, 0);
            f[ks] = make_uint4(v.x, v.y, v.z, v.w);
            __builtin_amdgcn_sched_barrier(0);  // k-step order on every path
        }
    };
    // The bias first: the weight copy's waits then cover it, so no load
    // issued before the loop is still pending inside it.
    float bias[NBT];
#pragma unroll
    for (int cb = 0; cb < NBT; ++cb) {
        const int col = col0 + cb * 32 + (lane & 31);
        bias[cb] = a.bias && col < cout ? a.bias[col] : 0.0f;
    }
    // The group's fragments: [ks][cb][64] of the layer's [ks][nbtot][64].
    const uint4 *wg = static_cast<const uint4 *>(a.w);
    for (int f = tid; f < KS * NBT * 64; f += 256) {
        const int ks = f / (NBT * 64), rem = f - ks * (NBT * 64);
        wl[f] = wg[(ks * nbtot + blockIdx.y * NBT) * 64 + rem];
    }
    // The first block's rows stay in flight across the barrier below.
    int64_t blk = static_cast<int64_t>(blockIdx.x) * 4 + wave;
    uint4 fa[KS], fb[KS];
    load_block(blk, fa);
#pragma unroll
    for (int k = 0; k < kStores; ++k)
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, drop_rsrc, 16 * k, 0, 0);
    float *stg = reinterpret_cast<float *>(wl + KS * NBT * 64) + wave * 8 * SLD;
    // Slot k of a lane: 16-byte piece i = lane + 64k of an 8-row group's
    // columns col0 .. col0 + gcols, at staging row i / (gcols / 8), column
    // 8 * (i % (gcols / 8)); goff is its element offset from the group's row 0.
    const int ppr = min(cout - col0, NBT * 32) / 8;
    int soff[KP], goff[KP];
#pragma unroll
    for (int k = 0; k < KP; ++k) {
        const int i = min(lane + 64 * k, 8 * ppr - 1);
        soff[k] = (i / ppr) * SLD + (i % ppr) * 8;
        goff[k] = (i / ppr) * cout + col0 + (i % ppr) * 8;
    }
    __syncthreads();
    auto run_block = [&](int64_t b, const uint4 (&f)[KS]) __attribute__((always_inline)) {
        f32x16 acc[NBT];
#pragma unroll
        for (int cb = 0; cb < NBT; ++cb) acc[cb] = f32x16{};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int cb = 0; cb < NBT; ++cb) acc[cb] = mfma_step<uint16_t>(f[ks], wl[(ks * NBT + cb) * 64 + lane], acc[cb]);
        // D layout: lane l holds column l % 32; register j holds row
        // 8*(j/4) + 4*(l/32) + j%4 of the block.
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int64_t row0 = b * 32 + 8 * g;
#pragma unroll
            for (int cb = 0; cb < NBT; ++cb)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float v = acc[cb][4 * g + q] + bias[cb];
                    if (a.silu) v = silu(v);
                    stg[(4 * half + q) * SLD + cb * 32 + (lane & 31)] = v;
                }
            const int64_t left = a.n_out - row0;
            const int pieces = static_cast<int>(left <= 0 ? 0 : left >= 8 ? 8 * ppr : left * ppr);
#pragma unroll
            for (int k = 0; k < KP; ++k) {
                const int i = lane + 64 * k;
                const float4 p = *reinterpret_cast<const float4 *>(stg + soff[k]);
                const float4 q = *reinterpret_cast<const float4 *>(stg + soff[k] + 4);
                const u32x4 v = {pack_bf16x2(p.x, p.y), pack_bf16x2(p.z, p.w), pack_bf16x2(q.x, q.y),
                                 pack_bf16x2(q.z, q.w)};
                __builtin_amdgcn_raw_buffer_store_b128(
                    v, y_rsrc, i < pieces ? static_cast<int32_t>((row0 * cout + goff[k]) * 2) : kOut, 0, 0);
            }
        }
    };
    for (; blk < nblk; blk += 2 * stride) {
        load_block(blk + stride, fb);
        run_block(blk, fa);
        if (blk + stride >= nblk) break;
        load_block(blk + 2 * stride, fa);
        run_block(blk + stride, fb);
    }
}

// FP32 1x1 layer fed BF16 rows, on BF16 MFMAs.  Each FP32 weight w is held as
// three BF16 terms, w1 = bf16(w), w2 = bf16(w - w1), w3 = bf16(w - w1 - w2)
// (each difference is exact in FP32), so w - (w1 + w2 + w3) is below
// 2^-24 |w| (the 24 significand bits of w in three 8-bit pieces; terms too
// small for FP32's range aside).  A BF16 row element times a BF16 term is
// exact in the FP32 accumulator, so the layer keeps FP32 accuracy while
// three 32x32x16 BF16 MFMAs replace eight 32x32x2 FP32 ones per 16
// channels.
// Workgroup: one wave per 32-column block (64 * NBT threads), each holding
// its block's 3 * KSX term fragments in registers for the whole launch.  The
// workgroup takes 32-row blocks of a grid-stride sequence; every wave loads
// the next block's rows (Cin = 16 * KSX channels, one 16-byte fragment per
// k-step) into the registers of the current one as soon as its MFMAs are
// issued, so the loads overlap the block's epilogue while three waves per
// SIMD fit (a second register set for the next block would leave two;
// Cin = 128 keeps two).
// The finished values (bias, SiLU, residual) go into an LDS tile laid out
// exactly as the output rows (row * cout + col), so the block leaves as one
// contiguous span of 16-byte streaming stores.  Two tiles alternate: one
// barrier per block.
// RES: a.residual is set (a separate instantiation: the residual loads of
// the epilogue wait for every load in flight, so a kernel that has them
// cannot keep the next block's rows in flight across the epilogue).
template <int NBT, int KSX, bool RES>
__global__ void __launch_bounds__(64 * NBT) __attribute__((amdgpu_waves_per_eu(KSX <= 6 ? 3 : 2)))
linear_split_kernel(ConvArgs a) {
    __shared__ __align__(16) float tile[2][32 * 32 * NBT];
    const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5;
    const int cb = __builtin_amdgcn_readfirstlane(tid >> 6);  // this wave's column block
    const int cout = a.cout;
    const uint4 *wg = static_cast<const uint4 *>(a.w);
    uint4 wr[KSX][3];
#pragma unroll
    for (int ks = 0; ks < KSX; ++ks)
#pragma unroll
        for (int t = 0; t < 3; ++t) wr[ks][t] = wg[((ks * NBT + cb) * 3 + t) * 64 + lane];
    const int col = cb * 32 + (lane & 31);
    const bool col_ok = col < cout;
    const float bias = a.bias && col_ok ? a.bias[col] : 0.0f;
    const auto x_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(a.x), static_cast<short>(0),
                                                          static_cast<int32_t>(a.x_bytes), 0x00020000);
    const int64_t nblk = (a.n_out + 31) / 32;
    // Lane: row lane % 32 of the block, channels ks*16 + half*8 .. +8.  Rows
    // past the end (the block after the workgroup's last) read zeros
    // through the buffer resource.
    auto load_block = [&](int64_t blk, uint4 (&f)[KSX]) __attribute__((always_inline)) {
        const int64_t r = blk * 32 + (lane & 31);
        const uint32_t base = r < a.n_out ? static_cast<uint32_t>(((r >> a.row_shift) * a.cin + half * 8) * 2)
                                          : 0x80000000u;
        // Issued in k-step order everywhere (the barriers pin it): the wait
        // before a k-step's MFMAs then counts the later loads and the stores
        // as younger on every path into the loop.
#pragma unroll
        for (int ks = 0; ks < KSX; ++ks) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, static_cast<int32_t>(base + ks * 32), 0, 0);
            f[ks] = make_uint4(v.x, v.y, v.z, v.w);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // Every block ends with kStores stores per thread, whatever its output
    // type and row count (16-byte pieces, one single element, and for BF16
    // output stores to an empty buffer, which the resource drops), and the
    // first block's loads are followed by as many dropped stores (at
    // distinct offsets, so none is merged away): on both paths into the loop
    // each k-step's rows then have the same known number of younger memory
    // operations, so its wait covers its own load and never the previous
    // block's stores.
    constexpr int kSpan = 32 * 32 * NBT;  // tile elements
    constexpr int kStores = kSpan / 4 / (64 * NBT) + 1;  // FP32: 16-byte pieces, then one element
    constexpr int kNontemporal = 2;  // buffer store cache policy: nt
    const auto drop_rsrc = __builtin_amdgcn_make_buffer_rsrc(a.y, static_cast<short>(0), 0, 0x00020000);
    auto dropped_stores = [&](auto count) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < decltype(count)::value; ++k)
            __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, drop_rsrc, 16 * k, 0, 0);
    };
    uint4 cur[KSX];
    int buf = 0;
    load_block(blockIdx.x, cur);
    dropped_stores(std::integral_constant<int, kStores>{});
    for (int64_t blk = blockIdx.x; blk < nblk; blk += gridDim.x, buf ^= 1) {
        f32x16 acc = f32x16{};
        // Smallest terms first.
#pragma unroll
        for (int ks = 0; ks < KSX; ++ks)
#pragma unroll
            for (int t = 2; t >= 0; --t) acc = mfma_step<uint16_t>(cur[ks], wr[ks][t], acc);
        load_block(blk + gridDim.x, cur);
        const int64_t row0 = blk * 32;
        const int rows = static_cast<int>(min(static_cast<int64_t>(32), a.n_out - row0));
        float *tl = tile[buf];
        // D layout: lane l holds column l % 32; register j holds row
        // 8*(j/4) + 4*(l/32) + j%4 of the block.
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int r = 8 * (j >> 2) + 4 * half + (j & 3);
            if (!col_ok || r >= rows) continue;
            float v = acc[j] + bias;
            if (a.silu) v = silu(v);
            if constexpr (RES) {
                const int64_t roff = ((row0 + r) >> a.residual_shift) * cout + col;
                v += a.y_bf16 ? bf16_to_f32(static_cast<const uint16_t *>(a.residual)[roff])
                              : static_cast<const float *>(a.residual)[roff];
            }
            tl[r * cout + col] = v;
        }
        __syncthreads();
        // The block's rows are one span of rows * cout elements starting at
        // row0 * cout (16-byte aligned: 32 * cout elements per block).  Every
        // thread issues the same number of 16-byte buffer stores (a piece
        // outside the span gets an offset the buffer resource drops), so the
        // compiler can count them and the wait for the next block's rows,
        // loaded before these stores, leaves the stores in flight (with a
        // store count it cannot know it waits for them too).  A span that is
        // not whole pieces (a last block only) ends with single elements.
        const int elems = rows * cout;
        constexpr int kOut = int32_t(0x80000000);  // an offset every resource drops
        if (a.y_bf16) {
            const int pieces = elems / 8;
            const auto y_rsrc = __builtin_amdgcn_make_buffer_rsrc(static_cast<uint16_t *>(a.y) + row0 * cout,
                                                                  static_cast<short>(0), elems * 2, 0x00020000);
#pragma unroll
            for (int k = 0; k < kSpan / 8 / (64 * NBT); ++k) {
                const int i = tid + k * 64 * NBT;
                const float4 p = *reinterpret_cast<const float4 *>(tl + i * 8);
                const float4 q = *reinterpret_cast<const float4 *>(tl + i * 8 + 4);
                const u32x4 v = {pack_bf16x2(p.x, p.y), pack_bf16x2(p.z, p.w), pack_bf16x2(q.x, q.y),
                                 pack_bf16x2(q.z, q.w)};
                __builtin_amdgcn_raw_buffer_store_b128(v, y_rsrc, i < pieces ? i * 16 : kOut, 0, kNontemporal);
            }
            dropped_stores(std::integral_constant<int, kStores - 1 - kSpan / 8 / (64 * NBT)>{});
            // The span's last elems % 8 elements, one a thread.
            const int e = pieces * 8 + tid;
            __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(tl[min(e, kSpan - 1)]), y_rsrc,
                                                  tid < 8 && e < elems ? e * 2 : kOut, 0, 0);
        } else {
            const int pieces = elems / 4;
            const auto y_rsrc = __builtin_amdgcn_make_buffer_rsrc(static_cast<float *>(a.y) + row0 * cout,
                                                                  static_cast<short>(0), elems * 4, 0x00020000);
#pragma unroll
            for (int k = 0; k < kSpan / 4 / (64 * NBT); ++k) {
                const int i = tid + k * 64 * NBT;
                const u32x4 v = *reinterpret_cast<const u32x4 *>(tl + i * 4);
                __builtin_amdgcn_raw_buffer_store_b128(v, y_rsrc, i < pieces ? i * 16 : kOut, 0, kNontemporal);
            }
            dropped_stores(std::integral_constant<int, kStores - 1 - kSpan / 4 / (64 * NBT)>{});
            // The span's last elems % 4 elements, one a thread.
            const int e = pieces * 4 + tid;
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, tl[min(e, kSpan - 1)]), y_rsrc,
                                                  tid < 4 && e < elems ? e * 4 : kOut, 0, 0);
        }
    }
}

template <int NBT>
KernelFn pick_linear_pipe_ks(int ks) {
    switch (ks) {
    case 4: return linear_pipe_kernel<NBT, 4>;
    case 8: return linear_pipe_kernel<NBT, 8>;
    case 12: return linear_pipe_kernel<NBT, 12>;
    case 16: return linear_pipe_kernel<NBT, 16>;
    default: return nullptr;
    }
}

// Cin = 16 * ksx for ksx in {2, 4, 6, 8}; nbt column blocks in 1..4.
template <int NBT, bool RES>
KernelFn pick_linear_split_ks(int ksx) {
    switch (ksx) {
    case 2: return linear_split_kernel<NBT, 2, RES>;
    case 4: return linear_split_kernel<NBT, 4, RES>;
    case 6: return linear_split_kernel<NBT, 6, RES>;
    case 8: return linear_split_kernel<NBT, 8, RES>;
    default: return nullptr;
    }
}

template <class T, bool XB = false>
KernelFn pick_linear(int nbt) {
    switch (nbt) {
    case 1: return linear_kernel<T, 1, XB>;
    case 2: return linear_kernel<T, 2, XB>;
    case 3: return linear_kernel<T, 3, XB>;
    case 4: return linear_kernel<T, 4, XB>;
    case 6: return linear_kernel<T, 6, XB>;
    case 8: return linear_kernel<T, 8, XB>;
    default: return nullptr;
    }
}

template <class T, int KC, int XF>
KernelFn pick_tiling(int id) {
#define S3DX_T(MBW, NBW, WN, S)                                                     \
    if constexpr (KC * NBW * WN * 32 * static_cast<int>(sizeof(T)) <= 32768)        \
        return conv_mfma_kernel<T, MBW, NBW, WN, KC, XF, S>;                         \
    else                                                                             \
        return nullptr;
    switch (id) {
    case 0: S3DX_T(1, 1, 1, 1)
    case 1: S3DX_T(1, 1, 2, 1)
    case 2: S3DX_T(1, 3, 1, 1)
    case 3: S3DX_T(1, 2, 2, 1)
    case 4: S3DX_T(1, 3, 2, 1)
    case 5: S3DX_T(1, 4, 2, 1)
    case 6: S3DX_T(2, 1, 2, 1)
    case 7: S3DX_T(2, 3, 1, 1)
    case 8: S3DX_T(2, 2, 2, 1)
    case 9: S3DX_T(2, 3, 2, 1)
    case 10: S3DX_T(1, 4, 1, 2)
    case 11: case 12: case 13: case 14: {
        constexpr int KS = KC / (2 * Frag<T>::E);
        if constexpr (KS % 4 == 0) {
            // 128 x 128 tiles with 128-channel BF16 or 64-channel FP32 tasks
            // spill: not built (the host takes 64 / 32 channels for tiling 11).
            if (id == 11) {
                if constexpr (sizeof(T) == 2 ? KC <= 64 : KC <= 32) return conv_splitk_kernel<T, 4, KC, XF, 1, 4>;
                else return nullptr;
            }
            if (id == 12) return conv_splitk_kernel<T, 2, KC, XF, 1, 4>;
            if (id == 13) return conv_splitk_kernel<T, 3, KC, XF, 1, 4>;
            return conv_splitk_kernel<T, 1, KC, XF, 1, 4>;
        } else {
            return nullptr;
        }
    }
    case 15: case 16: {
        if constexpr (sizeof(T) == 2 && XF == 0 && (KC == 32 || KC == 64)) {
            if (id == 15) return conv_splitk_kernel<T, 3, 128, XF, 128 / KC, 4>;
            return conv_splitk_kernel<T, 4, 128, XF, 128 / KC, 4>;
        } else {
            return nullptr;
        }
    }
    case 19: {  // 15 with 64-row tiles, two workgroups per CU (16's 128 columns would spill)
        if constexpr (sizeof(T) == 2 && XF == 0 && (KC == 32 || KC == 64))
            return conv_splitk_kernel<T, 3, 128, XF, 128 / KC, 2>;
        else
            return nullptr;
    }
    case 23: case 24: {  // FP32 32-column tiles of 64 (23) or 32 (24) rows, for small sets
        constexpr int KS = KC / (2 * Frag<T>::E);
        if constexpr (sizeof(T) == 4 && XF == 0 && KS % 4 == 0)
            return id == 23 ? conv_splitk_kernel<T, 1, KC, XF, 1, 2> : conv_splitk_kernel<T, 1, KC, XF, 1, 1>;
        else
            return nullptr;
    }
    case 18: {  // 64-row tiles, two workgroups per CU, half-width tasks
        if constexpr (sizeof(T) == 2 && XF == 0 && KC == 64)
            return conv_splitk_kernel<T, 4, 64, XF, 1, 2>;
        else if constexpr (sizeof(T) == 4 && XF == 0 && KC == 32)
            return conv_splitk_kernel<T, 4, 32, XF, 1, 2>;
        else
            return nullptr;
    }
    default: return nullptr;
    }
#undef S3DX_T
}

template <class T, int KC>
KernelFn pick_kc(int id, bool xf) {
    return xf ? pick_tiling<T, KC, 1>(id) : pick_tiling<T, KC, 0>(id);
}

}  // namespace
}  // namespace s3dx
