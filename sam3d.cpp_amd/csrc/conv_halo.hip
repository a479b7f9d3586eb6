// Halo-staged BF16 submanifold conv: one workgroup per 32*MB-row x 128-column
// output tile, each distinct source row staged in LDS once per 64-channel
// chunk.  Tiling 20: 128-row tiles, one workgroup per CU; tiling 21: 64-row
// tiles, two workgroups per CU (one's prologue, halo copies, reduction and
// epilogue overlap the other's MFMAs).
//
// Why: the split-K kernels gather every neighbour row for every offset (27
// gathers per output row) and stream every weight fragment per workgroup:
// about 48 KB of vector-memory reads per 16 MFMAs per SIMD, so the CU's
// vector-memory path, not the MFMA pipes, sets their pace.  Here each distinct
// source row is read once per chunk (~470 rows for 128 output rows, ~285 for
// 64, on sphere-shell sets, against 27 gathers per row) and each weight
// fragment goes straight from memory into the one wave that uses it.
//
// Workgroup: 4 waves, split-K.  Wave w owns the whole tile in accumulators
// (MB x 4 blocks of 32 x 32) and k-step w (16 channels) of each 64-channel
// chunk, for every present offset.  The task loop has no barrier: A
// fragments come from the LDS halo (slot from a per-tile table), B fragments
// from memory two tasks ahead.
//
// Prologue (per tile): the map slice is deduplicated with an LDS bitmap over
// the range of source rows it names; a prefix count gives each distinct row
// its halo slot (ascending row order), and a [27][rows] table of slots (a zero
// row for missing neighbours) drives the gathers.  A slice whose rows span
// more than the bitmap, or name more distinct rows than the halo holds, is
// gathered from memory instead (same loop, 16-byte MFMA-order loads).
//
// Epilogue: the four partial tiles are summed through LDS in a fixed order
// (deterministic) and finished row-major (bias, LayerNorm, modulate, SiLU,
// residual) by the shared finish_rows.
#include "conv_kernels.hpp"
#include "kmap_table.hpp"

#include <type_traits>

namespace s3dx {
namespace {

// s_waitcnt immediate waiting for vmcnt <= n (expcnt, lgkmcnt left at their maxima).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }

// f(integral_constant<int, I>) for I = B..E-1, unrolled at compile time.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

constexpr int kHChunk = 64;              // channels per halo chunk
constexpr int kHRowBytes = kHChunk * 2;  // 128 bytes per halo row

// 16-byte piece p of halo slot s sits at position p ^ halo_swizzle(s) of
// the slot's 128-byte row, so eight consecutive slots (the usual neighbours
// of consecutive output rows) read by one 16-byte LDS access spread over
// the eight positions.  ((s >> 1) & 7, which also separates 16 consecutive
// slots, halves the bank-conflict cycles but measured 1.5% slower.)
__device__ __forceinline__ int halo_swizzle(int s) { return s & 7; }
// Byte offset of slot s's row with its swizzle folded in: piece p of the
// slot sits at halo_offset(s) ^ (p << 4) (the row offset has bits 4-6 clear).
__device__ __forceinline__ uint32_t halo_offset(uint32_t s) {
    return s * kHRowBytes | static_cast<uint32_t>(halo_swizzle(static_cast<int>(s))) << 4;
}

template <int MB>
struct HaloSmem {
    static constexpr int ROWS = 32 * MB;
    static constexpr int RPH = MB == 4 ? 2 : 1;                  // row blocks reduced per phase
    static constexpr int CAP = MB == 4 ? 1088 : 511;             // halo rows (slot CAP is the zero row)
    static constexpr int BITWORDS = MB == 4 ? 1024 : 512;        // bitmap words (32 source rows each)
    static constexpr int ENTRIES = ROWS * kMaxKvol;
    static constexpr int STG_LD = 128 + 8;                       // padded FP32 output-tile row
    static constexpr int HALO_BYTES = (CAP + 1) * kHRowBytes;
    static constexpr int RED_BYTES = RPH * 4 * 4 * 4096;         // one reduction phase
    static constexpr int STG_BYTES = ROWS * STG_LD * 4 + 2 * ROWS * 16 * 4;
    static constexpr int R0A = HALO_BYTES > RED_BYTES ? HALO_BYTES : RED_BYTES;
    static constexpr int REGION0 = R0A > STG_BYTES ? R0A : STG_BYTES;
    static constexpr int TABLE_OFF = REGION0;
    static constexpr int BITMAP_OFF = TABLE_OFF + (ENTRIES * 2 + 15) / 16 * 16;
    static constexpr int PREFIX_OFF = BITMAP_OFF + BITWORDS * 4;
    static constexpr int ROWS_OFF = PREFIX_OFF + BITWORDS * 4;
    static constexpr int MISC_OFF = ROWS_OFF + (CAP * 4 + 15) / 16 * 16;
    static constexpr int TOTAL = MISC_OFF + 64;
    static_assert(TOTAL <= (MB == 4 ? 160 * 1024 : 80 * 1024), "LDS budget (two workgroups per CU for MB 2)");
    // The global-gather mode keeps 32-bit source rows (or -1) in region0,
    // which that mode does not use as a halo.
    static_assert(ENTRIES * 4 <= REGION0, "32-bit table fits region0");
};

// Wave-wide reductions through DPP (each 16-lane row by rotations, then the
// four rows by readlane); the result is wave-uniform.
__device__ __forceinline__ int dpp_ror(int x, int n) {
    switch (n) {
    case 8: return __builtin_amdgcn_update_dpp(0, x, 0x128, 0xf, 0xf, false);
    case 4: return __builtin_amdgcn_update_dpp(0, x, 0x124, 0xf, 0xf, false);
    case 2: return __builtin_amdgcn_update_dpp(0, x, 0x122, 0xf, 0xf, false);
    default: return __builtin_amdgcn_update_dpp(0, x, 0x121, 0xf, 0xf, false);
    }
}
template <class Op>
__device__ __forceinline__ int wave_reduce(int x, Op op) {
    x = op(x, dpp_ror(x, 8));
    x = op(x, dpp_ror(x, 4));
    x = op(x, dpp_ror(x, 2));
    x = op(x, dpp_ror(x, 1));
    return op(op(__builtin_amdgcn_readlane(x, 0), __builtin_amdgcn_readlane(x, 16)),
              op(__builtin_amdgcn_readlane(x, 32), __builtin_amdgcn_readlane(x, 48)));
}

// Exclusive prefix over the workgroup (256 threads) of one value each;
// returns the prefix, writes the total to *total.  Every thread must call it.
template <int WAVES = 4>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t *wave_sums, uint32_t *total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t incl = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t t = __shfl_up(incl, d, 64);
        if (lane >= d) incl += t;
    }
    if (lane == 63) wave_sums[wave] = incl;
    __syncthreads();
    uint32_t base = 0, all = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
        base += w < wave ? wave_sums[w] : 0u;
        all += wave_sums[w];
    }
    *total = all;
    return base + incl - v;
}

// Steps 1-4 of a tile's prologue: the tile's map slice deduplicated into LDS
// -- the [27][ROWS] slot table (or, when the slice cannot be staged, the
// 32-bit source-row table), the source row of every slot -- and the offset
// mask.  Every thread of the workgroup must call it; ends with a barrier.
struct TileDedupe {
    uint32_t mask, distinct;
    bool global_a;
};
// The tile's map slice read from memory: entries 4u..4u+3 of the tile
// (16-byte aligned, ROWS * 108 bytes per tile) by one unconditional 16-byte
// buffer load, whose resource ends at the map's last entry: a buffer load
// zero-fills each dword past the resource (checked on gfx950), and
// dedupe_tile marks entries past `count` invalid whatever they read.  (A
// load under a condition would compile to a branch, and the compiler waits
// for each such load at its join.)
struct SliceLoad {
    const int32_t *kmap;
    int32_t bytes;  // the map's size in bytes (rows * 108, under 2 GiB)
    __device__ __forceinline__ int4 operator()(int64_t m0, int u, int) const {
        const auto r = __builtin_amdgcn_make_buffer_rsrc(const_cast<int32_t *>(kmap), static_cast<short>(0), bytes,
                                                         0x00020000);
        const u32x4 v =
            __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int32_t>((m0 * kMaxKvol + 4 * u) * 4), 0, 0);
        return make_int4(static_cast<int32_t>(v.x), static_cast<int32_t>(v.y), static_cast<int32_t>(v.z),
                         static_cast<int32_t>(v.w));
    }
};

template <int MB, bool ENTRY_ORDER = false, int NTH = 256, class Fetch = SliceLoad>
__device__ __forceinline__ TileDedupe dedupe_tile(Fetch fetch, int64_t n_src, int32_t row_shift, int64_t m0,
                                                  int tile_rows, uint16_t *table, int32_t *table32,
                                                  uint32_t *bitmap, uint32_t *prefix, uint32_t *slot_row,
                                                  int32_t *misc) {
    using SM = HaloSmem<MB>;
    constexpr int ROWS = SM::ROWS, CAP = SM::CAP, ENTRIES = SM::ENTRIES;
    const int tid = threadIdx.x, lane = tid & 63;
    // ---- 1. this tile's map slice (ROWS * 27 entries) from `fetch`, as
    // source rows (-1: missing)
    constexpr int V4 = ENTRIES / 4;
    constexpr int Q = (V4 + NTH - 1) / NTH;
    const int count = tile_rows * kMaxKvol;
    int sj[Q][4];
    {
        // (slots past the slice fetch its last piece again and are marked
        // invalid below: a fetch under `u < V4` would be a branch, and the
        // compiler waits for each such load at its join)
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int u = tid + q * NTH;
            const int4 v = fetch(m0, min(u, V4 - 1), count);
            const int jv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const bool valid = u < V4 && 4 * u + k < count && jv[k] >= 0 && jv[k] < n_src;
                sj[q][k] = valid ? (jv[k] >> row_shift) : -1;
            }
        }
    }
    // ---- 2. range of named source rows and the offset mask (the range,
    // mask and bitmap are reset while the slice's loads are in flight)
    if (tid == 0) {
        misc[0] = INT32_MAX;
        misc[1] = INT32_MIN;
        misc[2] = 0;
    }
    for (int w = tid; w < SM::BITWORDS; w += NTH) bitmap[w] = 0u;
    __syncthreads();
    {
        int lo = INT32_MAX, hi = INT32_MIN, m = 0;
#pragma unroll
        for (int q = 0; q < Q; ++q)
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (sj[q][k] >= 0) {
                    lo = min(lo, sj[q][k]);
                    hi = max(hi, sj[q][k]);
                    m |= 1 << ((4 * (tid + q * NTH) + k) % kMaxKvol);
                }
        lo = wave_reduce(lo, [](int x, int y) { return min(x, y); });
        hi = wave_reduce(hi, [](int x, int y) { return max(x, y); });
        m = wave_reduce(m, [](int x, int y) { return x | y; });
        if (lane == 0) {
            atomicMin(&misc[0], lo);
            atomicMax(&misc[1], hi);
            atomicOr(&misc[2], m);
        }
        __syncthreads();
    }
    const int rlo = misc[0], rhi = misc[1];
    const uint32_t mask = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(misc[2]));
    const int64_t span = rhi >= rlo ? static_cast<int64_t>(rhi) - rlo + 1 : 0;
    bool global_a = span > static_cast<int64_t>(SM::BITWORDS) * 32;
    uint32_t distinct = 0;
    if (!global_a && span > 0) {
        // ---- 3. bitmap of named rows -> slot = rank among them
        const int words = static_cast<int>((span + 31) / 32);
#pragma unroll
        for (int q = 0; q < Q; ++q)
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (sj[q][k] >= 0) {
                    const uint32_t r = static_cast<uint32_t>(sj[q][k] - rlo);
                    atomicOr(&bitmap[r >> 5], 1u << (r & 31));
                }
        __syncthreads();
        constexpr int WPT = SM::BITWORDS / NTH;  // words per thread
        uint32_t cnt[WPT], mine = 0;
#pragma unroll
        for (int k = 0; k < WPT; ++k) {
            const int w = tid * WPT + k;
            cnt[k] = w < words ? static_cast<uint32_t>(__popc(bitmap[w])) : 0u;
            mine += cnt[k];
        }
        uint32_t run = block_exclusive_scan<NTH / 64>(mine, reinterpret_cast<uint32_t *>(misc + 4), &distinct);
#pragma unroll
        for (int k = 0; k < WPT; ++k) {
            const int w = tid * WPT + k;
            if (w < words) prefix[w] = run;
            run += cnt[k];
        }
        global_a = distinct > static_cast<uint32_t>(CAP);
        __syncthreads();
    }
    // ---- 4. the slot (or, gathering from memory, the row) of every entry,
    // and the source row of every slot
#pragma unroll
    for (int q = 0; q < Q; ++q)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int e = 4 * (tid + q * NTH) + k;
            if (e >= ENTRIES) continue;
            const int r = e / kMaxKvol, o = e - r * kMaxKvol;
            const int ti = ENTRY_ORDER ? e : o * ROWS + r;
            if (global_a) {
                table32[ti] = sj[q][k];
            } else {
                uint32_t slot = CAP;
                if (sj[q][k] >= 0) {
                    const uint32_t d = static_cast<uint32_t>(sj[q][k] - rlo);
                    const uint32_t bits = bitmap[d >> 5];
                    slot = prefix[d >> 5] + static_cast<uint32_t>(__popc(bits & ((1u << (d & 31)) - 1u)));
                    slot_row[slot] = static_cast<uint32_t>(sj[q][k]);  // writers of one slot agree
                }
                table[ti] = static_cast<uint16_t>(slot);
            }
        }
    __syncthreads();
    return TileDedupe{mask, distinct, global_a};
}

// Gather plans: one record per 64-row tile of a kernel map, the result of
// dedupe_tile kept in memory so that every conv over the map skips it:
//   [0, 16)     mode (0: halo, 1: global gathers), distinct rows, offset mask, 0
//   [16, ...)   halo: the u16 slot table [27][64], then at kPlanSlots the
//               source row of each slot; global: the int32 row table [27][64]
constexpr int kPlanHeader = 16;
constexpr int kPlanSlots = kPlanHeader + 64 * kMaxKvol * 2;  // 3472
static_assert(kPlanSlots + HaloSmem<2>::CAP * 4 <= kGatherPlanRecord, "halo record fits");
static_assert(kPlanHeader + 64 * kMaxKvol * 4 <= kGatherPlanRecord, "global record fits");
static_assert(kGatherPlanRecord % 1024 == 0, "records copy as whole 1 KiB pieces");

// 128-row records (the 8-wave kernel): the same header; halo tiles hold the
// source row of each slot right after it, then at kPlan128Table the u32
// table [27][128] of halo byte offsets (halo_offset of each slot); global
// tiles the int32 row table [27][128] at kPlan128Table.  The header and the
// rows come first so that a kernel can start copying rows while the table
// is still on its way.
constexpr int kPlan128Slots = kPlanHeader;     // 16
constexpr int kPlan128Table = 4608;
constexpr int kPlan128HeadPieces = (kPlan128Slots + HaloSmem<4>::CAP * 4 + 1023) / 1024;  // 5 KiB
static_assert(kPlan128Slots + HaloSmem<4>::CAP * 4 <= kPlan128Table, "halo record fits");
static_assert(kPlan128Table + 128 * kMaxKvol * 4 <= kGatherPlanRecord128, "tables fit");
static_assert(kGatherPlanRecord128 % 1024 == 0, "records copy as whole 1 KiB pieces");
// Halo layout of the 8-wave kernel: two buffers of kH8BufRows rows (one per
// chunk, the next chunk's copied while the current one is in use) with the
// zero row at slot kH8Double, or, for tiles naming more distinct rows, one
// buffer with the zero row at kH8Single.
constexpr int kH8BufRows = 560;
constexpr int kH8Double = kH8BufRows - 1;        // 559
constexpr int kH8Single = HaloSmem<4>::CAP;      // 1088
constexpr int kH8HaloBytes = 2 * kH8BufRows * kHRowBytes;
// 1 KiB after the halo that nothing reads: the last chunk sends its unneeded
// copy pieces (zero fills, which read no memory) there.
constexpr int kH8Dump = kH8HaloBytes;
constexpr int kH8Bytes = 160 * 1024;  // the kernel's LDS: halo, dump, plan record, padding
static_assert(kH8Dump + 1024 + kGatherPlanRecord128 <= kH8Bytes, "halo, dump and record fit");
// The record header's last word, 0 as the plan builder writes it: in LDS,
// the 8-wave kernel's arrival counter for the four waves of column half 0.
constexpr int kHalfCounter = 12;
static_assert((kH8Single + 1) * kHRowBytes <= kH8HaloBytes, "single buffer fits");
static_assert(kH8BufRows % 8 == 0, "buffers keep the slot swizzle");

template <int MB, bool PLAN>
struct HaloLds {
    // Planned kernels keep region0 and the copied record; unplanned ones the
    // dedupe buffers of HaloSmem.
    static constexpr int TOTAL = PLAN ? HaloSmem<MB>::REGION0 + kGatherPlanRecord + 64 : HaloSmem<MB>::TOTAL;
    static_assert(!PLAN || MB == 2, "plans are for 64-row tiles");
    static_assert(TOTAL <= (MB == 4 ? 160 * 1024 : 80 * 1024), "LDS budget");
};

// NB 32-column blocks per tile: 4 (128 columns), or 3 (96 columns: wave w < 3
// owns column block w in the reduction, wave 3 only hands its partials over).
template <int MB, bool PLAN, int NB = 4>
__global__ void __launch_bounds__(256, MB == 4 ? 1 : 2) conv_halo_kernel(ConvArgs a) {
    static_assert(NB == 4 || NB == 3, "128- or 96-column tiles");
    using SM = HaloSmem<MB>;
    constexpr int ROWS = SM::ROWS, CAP = SM::CAP, RPH = SM::RPH;
    __shared__ __align__(16) char smem[HaloLds<MB, PLAN>::TOTAL];
    char *halo = smem;
    char *rec = smem + SM::REGION0;  // the tile's plan record (planned kernels)
    uint16_t *table = reinterpret_cast<uint16_t *>(PLAN ? rec + kPlanHeader : smem + SM::TABLE_OFF);
    uint32_t *bitmap = reinterpret_cast<uint32_t *>(smem + SM::BITMAP_OFF);
    uint32_t *prefix = reinterpret_cast<uint32_t *>(smem + SM::PREFIX_OFF);
    uint32_t *slot_row = reinterpret_cast<uint32_t *>(PLAN ? rec + kPlanSlots : smem + SM::ROWS_OFF);
    int32_t *misc = reinterpret_cast<int32_t *>(smem + SM::MISC_OFF);  // [0] lo, [1] hi, [2] mask, [4..7] scan
    int32_t *table32 = reinterpret_cast<int32_t *>(PLAN ? rec + kPlanHeader : smem);  // global-gather mode

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int half = lane >> 5;
    const int tile = xcd_tile(blockIdx.x, gridDim.x);
    const int64_t m0 = static_cast<int64_t>(tile) * ROWS;
    const int nb0 = blockIdx.y * NB;
    const int nbtot = a.cout_pad / 32;
    const int ksteps_total = a.cin / 16;
    // Cin a multiple of 64, or (64-row tiles) 32 more: the last chunk then
    // holds two k-steps, and wave w takes k-step w & 1 of it on every other
    // present offset (parity w >> 1), so the four waves still share it.
    const int chunks = (a.cin + kHChunk - 1) / kHChunk;
    const bool half_last = a.cin % kHChunk != 0;
    const int tile_rows = static_cast<int>(min(static_cast<int64_t>(ROWS), a.n_out - m0));
    const int32_t xbytes = static_cast<int32_t>(a.x_bytes < INT32_MAX ? a.x_bytes : INT32_MAX);
    const int64_t w_bytes = static_cast<int64_t>(kMaxKvol) * a.cin * a.cout_pad * 2;
    const auto w_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(a.w), static_cast<short>(0),
                                                          static_cast<int32_t>(w_bytes), 0x00020000);
    const auto x_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(a.x), static_cast<short>(0),
                                                          xbytes, 0x00020000);

    TileDedupe dd;
    if constexpr (PLAN) {
        // The tile's plan record, straight into LDS: 1 KiB per instruction.
        const int64_t plan_bytes = (a.n_out + 63) / 64 * kGatherPlanRecord;
        const auto p_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(a.plan), static_cast<short>(0),
                                                              static_cast<int32_t>(plan_bytes), 0x00020000);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int i = wave + 4 * k;
            if (i < kGatherPlanRecord / 1024)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(p_rsrc, (__attribute__((address_space(3))) void *)(rec + i * 1024),
                                                         16, lane * 16, tile * kGatherPlanRecord + i * 1024, 0, 0);
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
        const uint32_t *hdr = reinterpret_cast<const uint32_t *>(rec);
        dd.global_a = __builtin_amdgcn_readfirstlane(hdr[0]) != 0;
        dd.distinct = __builtin_amdgcn_readfirstlane(hdr[1]);
        dd.mask = __builtin_amdgcn_readfirstlane(hdr[2]);
    } else {
        dd = dedupe_tile<MB>(SliceLoad{a.kmap, static_cast<int32_t>(a.n_out * kMaxKvol * 4)}, a.n_src, a.row_shift, m0,
                             tile_rows, table, table32, bitmap, prefix, slot_row, misc);
    }
    const uint32_t mask = dd.mask, distinct = dd.distinct;
    const bool global_a = dd.global_a;
    if (!global_a)
        for (int i = tid; i < kHRowBytes / 16; i += 256)
            reinterpret_cast<uint4 *>(halo + CAP * kHRowBytes)[i] = make_uint4(0, 0, 0, 0);
    __syncthreads();

    f32x16 acc[MB][NB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x16{};

    const int ntasks = __popc(mask);
    // Fragment (k-step ks, column block cb) of the packed weights sits at
    // byte ((ks * nbtot + cb) * 64 + lane) * 16; wave w keeps column block
    // (k + w) mod NB in accumulator column k, so the block it owns in the
    // final reduction is always accumulator column 0.
    int32_t bvo[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) bvo[nb] = lane * 16 + ((nb + wave) % NB) * 1024;
    // Offsets walked by scalar cursors; past the last one a cursor repeats
    // it (prefetches beyond the end reload it harmlessly).  Offsets are
    // below 27, so bit 31 is free: the ctz of rest | bit 31 is 31 exactly
    // when rest is empty (testing rest itself beside rest - 1 would turn
    // into a vector subtract and a readfirstlane).
    auto mfmas = [&](const uint4 (&af)[MB], const uint4 (&bf)[NB]) __attribute__((always_inline)) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = mfma_step<uint16_t>(af[mb], bf[nb], acc[mb][nb]);
    };

    // The chunk loop, for A from the halo (GA false) or from memory (GA
    // true): one loop nest per mode, so the accumulators stay in place.
    auto chunk_loop = [&](auto ga) __attribute__((always_inline)) {
        constexpr bool GA = decltype(ga)::value;
        for (int c = 0; c < chunks && ntasks > 0; ++c) {
            const bool hc = half_last && c == chunks - 1;
            const int kl = hc ? (wave & 1) : wave;  // this wave's k-step within the chunk
            const int ks = c * 4 + kl;             // and over the whole Cin
            // This wave's offsets in chunk c: every present one, or in a
            // half-width chunk every other one (parity wave >> 1).
            uint32_t cmask = mask;
            if (hc) {
                cmask = 0u;
                int k = 0;
                for (uint32_t r = mask; r != 0u; r &= r - 1u, ++k)
                    if ((k & 1) == (wave >> 1)) cmask |= r & (0u - r);
            }
            const int cn = __popc(cmask);
            const int olast = cn > 0 ? 31 - __builtin_clz(cmask) : 0;
            auto advance = [&](uint32_t &rest) __attribute__((always_inline)) {
                const int o = __builtin_ctz(rest | 0x80000000u);
                rest &= rest - 1u;
                return o == 31 ? olast : o;
            };
            // channels of chunk c that exist (the half chunk's upper 32 are
            // never read; their copy pieces are zero fills)
            const int cpieces = hc ? (a.cin - c * kHChunk) / 8 : 8;
            if constexpr (!GA) {
                if (c > 0) __syncthreads();  // every wave is done with chunk c-1
                // ---- 5. chunk c of every distinct row into its slot,
                // straight from memory into LDS (no registers): one
                // instruction fills 8 consecutive slots (1 KiB, lane L -> byte
                // 16 L), so lane L loads piece (L % 8) ^ halo_swizzle(slot) of its
                // slot's row -- the swizzle that spreads a gather of 32 slots
                // over the banks.  Eight lanes read each 128-byte row chunk:
                // whole cache lines.  Four groups per wave per round: their
                // slot rows are read first, one LDS round trip for four copies.
                const int groups = (static_cast<int>(distinct) + 7) >> 3;
                for (int g0 = wave; g0 < groups; g0 += 16) {
                    uint32_t off[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int s = (g0 + 4 * k) * 8 + (lane >> 3);
                        const int p = (lane & 7) ^ halo_swizzle(s);
                        off[k] = s < static_cast<int>(distinct) && p < cpieces
                                     ? (slot_row[min(s, CAP - 1)] * static_cast<uint32_t>(a.cin) + c * kHChunk +
                                        p * 8) * 2u
                                     : 0x80000000u;  // past the buffer: zeros
                    }
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        if (g0 + 4 * k < groups)
                            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                                x_rsrc, (__attribute__((address_space(3))) void *)(halo + (g0 + 4 * k) * 1024), 16,
                                static_cast<int32_t>(off[k]), 0, 0, 0);
                }
                // vmcnt(0) (expcnt and lgkmcnt left at their maxima): this
                // wave's copies have landed; the barrier covers the others.
                __builtin_amdgcn_s_waitcnt(0x0F70);
                __syncthreads();
            }
            // ---- 6. tasks: the present offsets in ascending order.  Per
            // task t: A(t+1) is read and the slots of task t+2 looked up
            // while t's MFMAs run; the weights of task t+R are requested
            // right after them.  Scheduling fences keep the weight loads in
            // that order.
            auto load_b = [&](int o, uint4 (&bf)[NB]) __attribute__((always_inline)) {
                const int32_t sbase = ((o * ksteps_total + ks) * nbtot + nb0) * 1024;
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, bvo[nb], sbase, 0);
                    bf[nb] = make_uint4(v.x, v.y, v.z, v.w);
                }
            };
            // The source of row block mb's lane row (mb*32 + lane%32) at
            // offset o: its halo slot, or (GA) its source row or -1.
            auto load_idx = [&](int o, int (&ix)[MB]) __attribute__((always_inline)) {
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    if constexpr (GA) ix[mb] = table32[o * ROWS + mb * 32 + (lane & 31)];
                    else ix[mb] = table[o * ROWS + mb * 32 + (lane & 31)];
                }
            };
            // A fragments: channels ks*16 + half*8 .. +8, i.e. chunk piece
            // 2*wave + half.
            auto load_a = [&](const int (&ix)[MB], uint4 (&af)[MB]) __attribute__((always_inline)) {
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    if constexpr (GA) {
                        const uint32_t off = ix[mb] >= 0
                                                 ? (static_cast<uint32_t>(ix[mb]) * static_cast<uint32_t>(a.cin) +
                                                    static_cast<uint32_t>(ks * 16 + half * 8)) * 2u
                                                 : 0x80000000u;
                        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, static_cast<int32_t>(off), 0, 0);
                        af[mb] = make_uint4(v.x, v.y, v.z, v.w);
                    } else {
                        const int p = 2 * kl + half;
                        af[mb] = *reinterpret_cast<const uint4 *>(halo + ix[mb] * kHRowBytes + ((p ^ halo_swizzle(ix[mb])) << 4));
                    }
                }
            };
            // Ring of R task sets (B requested R-1 tasks ahead: three for
            // 64-row tiles, whose tasks are half as long, else two).
            constexpr int R = MB == 2 ? 4 : 3;
            uint4 bq[R][NB], aq[R][MB];
            int iq[R][MB];
            uint32_t rest_i = cmask, rest_b = cmask;
            // (issued in the loop's order, so the wait counts at the loop
            // head match the steady state)
#pragma unroll
            for (int k = 0; k < R; ++k) {
                load_b(advance(rest_b), bq[k]);
                sched_fence();
            }
            load_idx(advance(rest_i), iq[0]);
            load_idx(advance(rest_i), iq[1]);
            load_a(iq[0], aq[0]);
            sched_fence();
            // body of task t held in set K (t = K mod R)
            auto body = [&](auto kc) __attribute__((always_inline)) {
                constexpr int K = decltype(kc)::value, K1 = (K + 1) % R, K2 = (K + 2) % R;
                // The LDS reads for the next tasks go between this task's
                // MFMAs (the scheduler interleaves them); the weight loads
                // stay after the last MFMA that reads their registers.
                load_a(iq[K1], aq[K1]);
                load_idx(advance(rest_i), iq[K2]);
                mfmas(aq[K], bq[K]);
                sched_fence();
                load_b(advance(rest_b), bq[K]);
                sched_fence();
            };
            int t = 0;
            for (; t + R <= cn; t += R) {
                body(std::integral_constant<int, 0>{});
                body(std::integral_constant<int, 1>{});
                body(std::integral_constant<int, 2>{});
                if constexpr (R == 4) body(std::integral_constant<int, 3>{});
            }
            // Fewer than R tasks left: set k holds task t+k's weights; the
            // A of task t is in set 0 and the slots of task t+1 in set 1.
            const int left = cn - t;
            if (left >= 1) mfmas(aq[0], bq[0]);
            if (left >= 2) {
                load_a(iq[1], aq[1]);
                mfmas(aq[1], bq[1]);
            }
            if constexpr (R == 4) {
                if (left >= 3) {
                    load_idx(advance(rest_i), iq[2]);
                    load_a(iq[2], aq[2]);
                    mfmas(aq[2], bq[2]);
                }
            }
        }
    };
    if (global_a) chunk_loop(std::true_type{});
    else chunk_loop(std::false_type{});
    __syncthreads();  // the halo region becomes the reduction slots

    // ---- 7. reduce the 4 partial tiles in two phases of RPH row blocks;
    // pair (h, c) = (row block RPH*p + h, column block c) is summed by wave c,
    // the other waves handing their partials over as float4 [4][lane] slots.
    float4 *red = reinterpret_cast<float4 *>(smem);
    auto slot_of = [&](int h, int c, int writer) __attribute__((always_inline)) {
        return red + ((h * 4 + c) * 4 + writer) * (4 * 64);
    };
    float fin[2][RPH][16];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        if (p) __syncthreads();
#pragma unroll
        for (int h = 0; h < RPH; ++h)
#pragma unroll
            for (int k = 0; k < NB; ++k) {
                const int c = (k + wave) % NB;  // (waves below NB own block `wave`: column 0)
                if (c == wave) continue;
                float4 *slot = slot_of(h, c, wave);
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    slot[g * 64 + lane] = make_float4(acc[RPH * p + h][k][4 * g], acc[RPH * p + h][k][4 * g + 1],
                                                      acc[RPH * p + h][k][4 * g + 2], acc[RPH * p + h][k][4 * g + 3]);
            }
        __syncthreads();
        if (wave >= NB) continue;  // (a 96-column tile's wave 3 owns no block)
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
    }
    __syncthreads();
    float *stg = reinterpret_cast<float *>(smem);
    float *part = stg + ROWS * SM::STG_LD;
    if (wave < NB) {
#pragma unroll
        for (int p = 0; p < 2; ++p)
#pragma unroll
            for (int h = 0; h < RPH; ++h) {
                const int col = wave * 32 + (lane & 31);
                const int rb = (RPH * p + h) * 32 + 4 * half;
#pragma unroll
                for (int r = 0; r < 16; ++r) stg[(rb + 8 * (r >> 2) + (r & 3)) * SM::STG_LD + col] = fin[p][h][r];
            }
    }
    constexpr int TPR = NB * 4;  // threads per row: 8 columns each
    uint4 res[RowMap<TPR, ROWS>::PASSES][2];
    load_residual<TPR, ROWS>(a, m0, nb0, tile_rows, tid, res);
    __syncthreads();
    finish_rows<TPR, ROWS, SM::STG_LD>(a, stg, part, m0, nb0, tile_rows, tid, res);
}

// 128-row x 128-column tiles read through 128-row gather-plan records: one
// workgroup of 8 waves per CU, two waves per SIMD on the same tile.  Wave w
// holds k-step ks = w % 4 of every 64-channel chunk for column half
// ch = w / 4 (column blocks 2ch, 2ch+1): 4 x 2 accumulator blocks, two weight
// fragments and four A fragments per task, so every weight fragment feeds
// four row blocks (half the weight traffic per MFMA of the 64-row tiles).
// Tasks run chunk-major, offsets ascending; the weight loads of the next
// tasks flow on across chunk boundaries.  With two halo buffers (tiles naming
// at most kH8Double distinct rows) chunk c+1 is copied into the other buffer
// while chunk c is in use.
//
// Every output element is accumulated in the same order as by the 64-row
// kernel (k-step w's partial: chunks, then offsets, ascending) and the four
// k-step partials of column block c are summed as ((P_c + P_c+1) + P_c+2) +
// P_c+3 (indices mod 4), the order of the 64-row kernel's reduction, so the
// two kernels' results are bit-identical.
//
// Stream-K launches (SK, conv_halo8_sk_kernel): the (column group, tile,
// chunk) units of the layer, column-group-major, are cut into sk_wgs equal
// runs, one per workgroup (one workgroup per CU), so that every CU gets the
// same number of chunk-units whatever the tile count.  A run covers pieces
// of consecutive tiles: a piece that is a whole tile is finished here; a
// piece that is part of a tile (at most the first and the last of a run)
// leaves its FP32 tile in the run's partial slot 0 or 1, and
// halo8_combine_kernel adds a tile's pieces in chunk order and finishes it.
// A piece of chunks [c0, c1) reads x and the weights from chunk c0 on, so
// the chunk loop is the whole-tile loop on a narrower input.
template <bool SK>
__device__ __forceinline__ void halo8_body(const ConvArgs &a) {
    constexpr int ROWS = 128;
    constexpr int STG_LD = 128;
    __shared__ __align__(16) char smem[kH8Bytes];
    char *halo = smem;
    char *rec = smem + kH8Dump + 1024;
    // [27][128] u32: halo byte offsets, or source rows for global gathers
    const int32_t *table32 = reinterpret_cast<const int32_t *>(rec + kPlan128Table);
    const uint32_t *slot_row = reinterpret_cast<const uint32_t *>(rec + kPlan128Slots);

    const int nbtot = a.cout_pad / 32;
    const int ksteps_total = a.cin / 16;
    const int chunks_all = a.cin / kHChunk;
    const int wave_run = SK ? __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6) : 0;
    auto piece = [&](const int tile, const int nb0, const int cbeg, const int cend, float *const part_out)
        __attribute__((always_inline)) {
    // (stream-K: each piece forms the thread index from the wave index and an
    // mbcnt over an empty asm's zero, and the weight offset stride, the zero
    // row's value and 1/cout pass empty asms too, so that none of them, nor
    // what derives from them, is hoisted out of the run's loop and held --
    // spilled -- across every piece)
    int tid_v = static_cast<int>(threadIdx.x);
    if constexpr (SK) {
        int zero = 0;
        asm volatile("" : "+s"(zero));
        tid_v = wave_run * 64 + static_cast<int>(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, zero)));
    }
    const int tid = tid_v, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ks = wave & 3, ch = wave >> 2;
    const int half = lane >> 5;
    const int64_t m0 = static_cast<int64_t>(tile) * ROWS;
    const int chunks = cend - cbeg;
    const int tile_rows = static_cast<int>(min(static_cast<int64_t>(ROWS), a.n_out - m0));
    // x and the weights from chunk cbeg on
    const char *const xbase = static_cast<const char *>(a.x) + static_cast<int64_t>(cbeg) * kHRowBytes;
    const int64_t x_rest = a.x_bytes - static_cast<int64_t>(cbeg) * kHRowBytes;
    const int32_t xbytes = static_cast<int32_t>(x_rest < INT32_MAX ? x_rest : INT32_MAX);
    const int64_t w_skip = static_cast<int64_t>(cbeg) * 4 * nbtot * 1024;
    const int64_t w_bytes = static_cast<int64_t>(kMaxKvol) * a.cin * a.cout_pad * 2 - w_skip;
    const auto w_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char *>(static_cast<const char *>(a.w) + w_skip), static_cast<short>(0),
        static_cast<int32_t>(w_bytes), 0x00020000);
    const auto x_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(xbase), static_cast<short>(0),
                                                          xbytes, 0x00020000);

    // ---- 1. the tile's plan record, straight into LDS (1 KiB per instruction)
    {
        const int64_t plan_bytes = (a.n_out + ROWS - 1) / ROWS * kGatherPlanRecord128;
        const auto p_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(a.plan), static_cast<short>(0),
                                                              static_cast<int32_t>(plan_bytes), 0x00020000);
        // the header and the slot rows only: the table follows later
        static_assert(kPlan128HeadPieces <= 8, "one head piece per wave");
        if (wave < kPlan128HeadPieces)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(p_rsrc, (__attribute__((address_space(3))) void *)(rec + wave * 1024),
                                                     16, lane * 16, tile * kGatherPlanRecord128 + wave * 1024, 0, 0);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
    }
    // The rest of the record (the table) into LDS; a path waits for it
    // before its first table read.  The full loop requests it after its first
    // halo copy, so that the rows the first tasks need are first in line.
    auto load_table = [&]() __attribute__((always_inline)) {
        const int64_t plan_bytes = (a.n_out + ROWS - 1) / ROWS * kGatherPlanRecord128;
        const auto p_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(a.plan), static_cast<short>(0),
                                                              static_cast<int32_t>(plan_bytes), 0x00020000);
        constexpr int kRest = kGatherPlanRecord128 / 1024 - kPlan128HeadPieces;
#pragma unroll
        for (int k = 0; k < (kRest + 7) / 8; ++k) {
            const int i = kPlan128HeadPieces + wave + 8 * k;
            if (wave + 8 * k < kRest)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(p_rsrc, (__attribute__((address_space(3))) void *)(rec + i * 1024),
                                                         16, lane * 16, tile * kGatherPlanRecord128 + i * 1024, 0, 0);
        }
    };
    const uint32_t *hdr = reinterpret_cast<const uint32_t *>(rec);
    const bool global_a = __builtin_amdgcn_readfirstlane(hdr[0]) != 0;
    const uint32_t distinct = __builtin_amdgcn_readfirstlane(hdr[1]);
    const uint32_t mask = __builtin_amdgcn_readfirstlane(hdr[2]);
    const bool dbl = !global_a && distinct <= static_cast<uint32_t>(kH8Double);
    const int zrow = dbl ? kH8Double : kH8Single;
    if (!global_a && tid < 2 * (kHRowBytes / 16)) {  // the zero row of each buffer in use
        const int b = tid / (kHRowBytes / 16);
        if (b == 0 || dbl)
            reinterpret_cast<uint4 *>(halo + (b * kH8BufRows + zrow) * kHRowBytes)[tid % (kHRowBytes / 16)] =
                make_uint4(opaque_scalar<SK>(0), 0, 0, 0);
    }

    // Chunk c of every distinct row into its slot of `buf` (lane L of a
    // 1 KiB copy fills piece (L % 8) ^ halo_swizzle(slot) of slot 8g + L / 8).
    // The copies run from within the chunk bodies below, whose pointer
    // arguments are __restrict__: that tells the compiler that a copy into
    // one buffer does not alias the reads of the other, so it waits for the
    // copy only where the code says so (else it drains vmcnt before every
    // LDS read that follows a copy, and the next chunk's copy stops
    // overlapping the current chunk's MFMAs).
    auto halo_copy = [&](int c, char *buf, const uint32_t *slot_row, const char *xg) __attribute__((always_inline)) {
        const auto x_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(xg), static_cast<short>(0), xbytes,
                                                              0x00020000);
        const int groups = (static_cast<int>(distinct) + 7) >> 3;
        for (int g0 = wave; g0 < groups; g0 += 32) {
            uint32_t off[4], srow[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) srow[k] = slot_row[min((g0 + 8 * k) * 8 + (lane >> 3), kH8Single - 1)];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int sl = (g0 + 8 * k) * 8 + (lane >> 3);
                const int p = (lane & 7) ^ halo_swizzle(sl);
                off[k] = sl < static_cast<int>(distinct)
                             ? (srow[k] * static_cast<uint32_t>(a.cin) + c * kHChunk + p * 8) * 2u
                             : 0x80000000u;  // past the buffer: zeros
            }
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (g0 + 8 * k < groups)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(
                        x_rsrc, (__attribute__((address_space(3))) void *)(buf + (g0 + 8 * k) * 1024), 16,
                        static_cast<int32_t>(off[k]), 0, 0, 0);
        }
    };
    auto buf_of = [&](int c) __attribute__((always_inline)) {
        return halo + (dbl && (c & 1) ? kH8BufRows * kHRowBytes : 0);
    };

    f32x16 acc[4][2];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[mb][j] = f32x16{};

    const int ntasks = __popc(mask);
    const int olast = ntasks > 0 ? 31 - __builtin_clz(mask) : 0;
    // Offsets walked by scalar cursors, ascending; past the last one a
    // cursor repeats it (prefetches beyond the end reload it harmlessly).
    auto advance = [&](uint32_t &rest) __attribute__((always_inline)) {
        const int o = __builtin_ctz(rest | 0x80000000u);
        rest &= rest - 1u;
        return o == 31 ? olast : o;
    };
    // Fragment (k-step, column block) of the packed weights sits at byte
    // ((kstep * nbtot + cb) * 64 + lane) * 16: for (chunk c, offset o) this
    // wave's two fragments start at w_first + c * w_chunk + o * w_offset.
    const int32_t w_offset = opaque_scalar<SK>(ksteps_total * nbtot * 1024);
    const int32_t w_chunk = 4 * nbtot * 1024;
    const int32_t w_first = (ks * nbtot + nb0 + 2 * ch) * 1024;
    // (voff_extra 0x80000000 puts the loads out of range: zeros, no memory read)
    auto load_b_at = [&](int32_t sbase, uint4 (&bf)[2], uint32_t voff_extra = 0u) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(
                w_rsrc, static_cast<int32_t>((static_cast<uint32_t>(lane * 16) | voff_extra) + j * 1024), sbase, 0);
            bf[j] = make_uint4(v.x, v.y, v.z, v.w);
        }
    };
    auto load_b = [&](int c, int o, uint4 (&bf)[2]) __attribute__((always_inline)) {
        load_b_at(w_first + c * w_chunk + o * w_offset, bf);
    };
    auto mfmas = [&](const uint4 (&af)[4], const uint4 (&bf)[2]) __attribute__((always_inline)) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[mb][j] = mfma_step<uint16_t>(af[mb], bf[j], acc[mb][j]);
    };
    // This lane's 16-byte piece of the A fragment (channels 8p..8p+7 of the
    // chunk) from the halo rows whose offsets ix holds.
    const uint32_t p16 = static_cast<uint32_t>(2 * ks + half) << 4;
    auto load_a_halo = [&](const char *buf, const int (&ix)[4], uint4 (&af)[4]) __attribute__((always_inline)) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
            af[mb] = *reinterpret_cast<const uint4 *>(buf + (static_cast<uint32_t>(ix[mb]) ^ p16));
    };
    // Before chunk c's tasks its halo copy has landed and every wave is past
    // chunk c-1; with two buffers the copy of chunk c+1 then goes into the
    // buffer chunk c-1 used.  When NB weight loads were issued after the copy
    // of chunk c (the first NB of the cursor for c = 0, the last NB of chunk
    // c-1's tasks otherwise) vmcnt(NB) covers the copy; `few`: fewer were
    // (the cursor ran past the last chunk, or chunk c-1 had fewer tasks), so
    // wait for every load.
    auto chunk_sync = [&](int c, auto nb, bool few, char *cur, char *nxt, const uint32_t *rows,
                          const char *xg) __attribute__((always_inline)) {
        constexpr int NB = decltype(nb)::value;
        if (dbl) {
            if (!few) __builtin_amdgcn_s_waitcnt(vmcnt_imm(NB));
            else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            __syncthreads();
            if (c + 1 < chunks) halo_copy(c + 1, nxt, rows, xg);
        } else {
            if (c > 0) {
                __syncthreads();
                halo_copy(c, cur, rows, xg);
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            } else if (!few) {
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(NB));
            } else {
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            }
            __syncthreads();
        }
    };

    // The chunk loop over any offset mask, for A from the halo (GA false) or
    // from memory (GA true).
    auto chunk_loop = [&](auto ga) __attribute__((always_inline)) {
        constexpr bool GA = decltype(ga)::value;
        if (ntasks == 0) return;
        constexpr int R = 4;  // weight sets in flight (three tasks ahead)
        uint4 bq[R][2];
        // The weight cursor runs over (chunk, offset) chunk-major across the
        // whole loop, so the loads for the next chunk's first tasks go out while
        // the current chunk ends; past the last task it requests nothing.
        int cur_c = 0;
        uint32_t rest_b = mask;
        auto next_b = [&](uint4 (&bf)[2]) __attribute__((always_inline)) {
            if (rest_b == 0u) {
                ++cur_c;
                rest_b = mask;
            }
            const int o = advance(rest_b);
            if (cur_c < chunks) load_b(cur_c, o, bf);
        };
        // bq[i] <- bq[(i + n) % R]: after a chunk whose task count leaves n
        // over a multiple of R, the next chunk's task i sits in bq[(n + i) % R].
        auto rotate_b = [&](int n) __attribute__((always_inline)) {
            uint4 t[R][2];
    #pragma unroll
            for (int k = 0; k < R; ++k) t[k][0] = bq[k][0], t[k][1] = bq[k][1];
    #pragma unroll
            for (int r = 1; r < R; ++r)
                if (n == r)
    #pragma unroll
                    for (int k = 0; k < R; ++k) bq[k][0] = t[(k + r) % R][0], bq[k][1] = t[(k + r) % R][1];
        };
        if constexpr (!GA) halo_copy(0, halo, slot_row, xbase);
#pragma unroll
        for (int k = 0; k < R; ++k) {
            next_b(bq[k]);
            sched_fence();
        }
        auto chunk = [&](int c, char *__restrict__ buf, char *__restrict__ nxt, const int32_t *__restrict__ tbl,
                         const uint32_t *__restrict__ rows, const char *__restrict__ xg) __attribute__((always_inline)) {
            // (loads after chunk c's copy: for c = 0 the cursor's first R
            // sets, fewer when the tile has fewer than R (chunk, offset) tasks)
            if constexpr (!GA)
                chunk_sync(c, std::integral_constant<int, 2 * R>{}, c == 0 ? ntasks * chunks < R : ntasks < R, buf,
                           nxt, rows, xg);
            const int kch = (c * 4 + ks) * 16 + half * 8;  // this lane's first channel of the A fragment
            auto load_idx = [&](int o, int (&ix)[4]) __attribute__((always_inline)) {
#pragma unroll
                for (int mb = 0; mb < 4; ++mb) ix[mb] = tbl[o * ROWS + mb * 32 + (lane & 31)];
            };
            auto load_a = [&](const int (&ix)[4], uint4 (&af)[4]) __attribute__((always_inline)) {
                if constexpr (GA) {
#pragma unroll
                    for (int mb = 0; mb < 4; ++mb) {
                        const uint32_t off = ix[mb] >= 0 ? (static_cast<uint32_t>(ix[mb]) * static_cast<uint32_t>(a.cin) +
                                                            static_cast<uint32_t>(kch)) * 2u
                                                         : 0x80000000u;
                        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, static_cast<int32_t>(off), 0, 0);
                        af[mb] = make_uint4(v.x, v.y, v.z, v.w);
                    }
                } else {
                    load_a_halo(buf, ix, af);
                }
            };
            uint4 aq[2][4];
            int iq[2][4];
            uint32_t rest_i = mask;
            load_idx(advance(rest_i), iq[0]);
            load_idx(advance(rest_i), iq[1]);
            load_a(iq[0], aq[0]);
            sched_fence();
            // task t: A in aq[t & 1], slots of t + 1 in iq[(t + 1) & 1],
            // weights in bq[t % R]; A(t + 1) is read and the slots of t + 2
            // looked up while t's MFMAs run, the weights R tasks on
            // requested right after them.
            auto body = [&](auto kc) __attribute__((always_inline)) {
                constexpr int K = decltype(kc)::value, A0 = K & 1, A1 = (K + 1) & 1;
                load_a(iq[A1], aq[A1]);
                load_idx(advance(rest_i), iq[A0]);
                mfmas(aq[A0], bq[K]);
                sched_fence();
                next_b(bq[K]);
                sched_fence();
            };
            int t = 0;
            for (; t + R <= ntasks; t += R) {
                body(std::integral_constant<int, 0>{});
                body(std::integral_constant<int, 1>{});
                body(std::integral_constant<int, 2>{});
                body(std::integral_constant<int, 3>{});
            }
            // Fewer than R tasks left: bq[k] holds task t+k's weights, aq[0]
            // the A of task t and iq[1] the slots of task t+1; each set used
            // is refilled with the next weights in the sequence.
            const int left = ntasks - t;
            if (left >= 1) {
                mfmas(aq[0], bq[0]);
                sched_fence();
                next_b(bq[0]);
                sched_fence();
            }
            if (left >= 2) {
                load_a(iq[1], aq[1]);
                mfmas(aq[1], bq[1]);
                sched_fence();
                next_b(bq[1]);
                sched_fence();
            }
            if (left >= 3) {
                load_idx(advance(rest_i), iq[0]);
                load_a(iq[0], aq[0]);
                mfmas(aq[0], bq[2]);
                sched_fence();
                next_b(bq[2]);
                sched_fence();
            }
            rotate_b(left);
        };
        for (int c = 0; c < chunks; ++c)
            chunk(c, buf_of(c), buf_of(c + 1), table32, slot_row, xbase);
    };

    // Two-buffer halo tiles whose rows have neighbours at all 27 offsets
    // (every tile of a closed surface): the same task order with the offsets
    // known at compile time, so the table reads take immediate addresses and
    // no cursor runs.  Three weight sets in flight: 27 tasks a chunk leave
    // task t of every chunk in set t % 3.
    //
    // The copy of chunk c+1 goes out one 1 KiB piece per task over chunk
    // c's first tasks, each right after a weight load:
    // vmcnt retires loads in issue order, so a wait for weights requested
    // after a piece also waits for that piece, and spreading the pieces
    // gives each about RF tasks of MFMAs to land instead of stalling the
    // chunk's first task on the whole copy.
    auto full_loop = [&]() __attribute__((always_inline)) {
        constexpr int RF = 3;
        // Pieces a wave copies per chunk with two buffers: group
        // min(wave + 8j, groups - 1) (slots 8g..8g+7) for j < kPieces, so
        // every wave issues all of them (a clamped piece copies its group
        // again: the same bytes to the same place).
        constexpr int kPieces = (kH8Double + 1 + 63) / 64;  // 9
        static_assert(kPieces <= kMaxKvol - RF, "the pieces go out before the chunk's last weight loads");
        const int groups = (static_cast<int>(distinct) + 7) >> 3;
        uint32_t piece_off[kPieces];  // source byte offset of each piece at chunk 0
        int piece_group[kPieces];
        // (the slot rows are read unconditionally, at clamped indexes, so
        // that the nine LDS reads go out together)
        uint32_t srow[kPieces];
#pragma unroll
        for (int j = 0; j < kPieces; ++j) {
            piece_group[j] = min(wave + 8 * j, groups - 1);
            srow[j] = slot_row[min(piece_group[j] * 8 + (lane >> 3), kH8Double)];
        }
#pragma unroll
        for (int j = 0; j < kPieces; ++j) {
            const int sl = piece_group[j] * 8 + (lane >> 3);
            const int p = (lane & 7) ^ halo_swizzle(sl);
            piece_off[j] = sl < static_cast<int>(distinct) ? (srow[j] * static_cast<uint32_t>(a.cin) + p * 8) * 2u
                                                           : 0x80000000u;  // past the buffer: zeros
        }
        // piece j of chunk cc into buffer dst (soffset is outside the range
        // check: the zero-fill offset stays out of range)
        auto piece = [&](__amdgpu_buffer_rsrc_t rsrc, int j, int cc, uint32_t off, char *dst)
                         __attribute__((always_inline)) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)(dst), 16,
                                                     static_cast<int32_t>(off), cc * kHRowBytes, 0, 0);
        };
        uint4 bf[RF][2];
        int32_t wb = w_first;  // weights of the next task to request
        {
            const auto x_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(xbase), static_cast<short>(0),
                                                                  xbytes, 0x00020000);
#pragma unroll
            for (int j = 0; j < kPieces; ++j) piece(x_rsrc, j, 0, piece_off[j], halo + piece_group[j] * 1024);
        }
        load_table();
#pragma unroll
        for (int k = 0; k < RF; ++k) {
            load_b_at(wb, bf[k]);
            wb += w_offset;
            sched_fence();
        }
        // Chunk c's 27 tasks from `buf`; but for the last chunk, chunk
        // c+1's copy goes into `nxt` over the first tasks and the first
        // weights of chunk c+1 are requested over the last ones.  The last
        // chunk leaves the other buffer untouched (the epilogue uses it).
        auto chunk = [&](int c, const char *__restrict__ buf, char *__restrict__ nxt, const int32_t *__restrict__ tbl,
                         const char *__restrict__ xg) __attribute__((always_inline)) {
            const bool last = c + 1 == chunks;
            const auto x_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(xg), static_cast<short>(0),
                                                                  xbytes, 0x00020000);
            auto load_idx = [&](int o, int (&ix)[4]) __attribute__((always_inline)) {
#pragma unroll
                for (int mb = 0; mb < 4; ++mb) ix[mb] = tbl[o * ROWS + mb * 32 + (lane & 31)];
            };
            const int32_t w_next = w_first + (c + 1) * w_chunk;
            // The last chunk requests nothing for a next one: its pieces go
            // to the dump, its last weight loads out of range (zeros, no
            // memory read), so no wave waits on them after the loop.
            const uint32_t b_void = last ? 0x80000000u : 0u;
            uint4 aq[2][4];
            int iq[2][4];
            load_idx(0, iq[0]);
            load_idx(1, iq[1]);
            load_a_halo(buf, iq[0], aq[0]);
            sched_fence();
            static_for<0, kMaxKvol>([&](auto tc) __attribute__((always_inline)) {
                constexpr int t = decltype(tc)::value, A0 = t & 1, A1 = (t + 1) & 1;
                if constexpr (t + 1 < kMaxKvol) load_a_halo(buf, iq[A1], aq[A1]);
                if constexpr (t + 2 < kMaxKvol) load_idx(t + 2, iq[A0]);
                mfmas(aq[A0], bf[t % RF]);
                sched_fence();
                if constexpr (t + RF == kMaxKvol) wb = w_next;
                load_b_at(wb, bf[t % RF], t + RF < kMaxKvol ? 0u : b_void);
                wb += w_offset;
                if constexpr (t < kPieces)
                    piece(x_rsrc, t, c + 1, last ? 0x80000000u : piece_off[t],
                          last ? smem + kH8Dump : nxt + piece_group[t] * 1024);
                sched_fence();
            });
        };
        for (int c = 0; c < chunks; ++c) {
            // chunk c's pieces (and for c = 0 the table) precede the last
            // 2 RF weight loads, and after the barrier no wave reads the
            // buffer of chunk c-1
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * RF));
            __syncthreads();
            chunk(c, buf_of(c), buf_of(c + 1), table32, xbase);
        }
    };
    if (dbl && !global_a && mask == (1u << kMaxKvol) - 1u) {
        full_loop();  // requests the table itself; its first wait covers it
    } else {
        load_table();
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
        if (global_a) chunk_loop(std::true_type{});
        else chunk_loop(std::false_type{});
    }
    // the epilogue's column parameters, in flight during the reduction
    RowParams params;
    load_row_params(a, nb0 * 32 + (tid % 16) * 8, params);

    // ---- 3. reduce the four k-step partials of each 32 x 32 block: wave
    // (ks, ch) sums row block ks of column blocks 2ch, 2ch+1, the three
    // other waves of its column half handing theirs over through LDS as
    // float4 [4][lane] blocks.  The halves are independent: column half 0
    // (whose waves the SIMDs favour, so they leave the loop first) reduces
    // in the halo buffer the last chunk does not use while half 1 still
    // runs its MFMAs, synchronizing its four waves through an LDS counter;
    // half 1 then reduces both column blocks at once after the barrier.
    // With one large halo buffer (nothing free during the loop) both halves
    // take the second path in turn.
    float fin[2][16];
    // Writer w's block of row block rb: rank (w - rb - 1) & 3 among the
    // three writers, 4 KiB each, [rb][rank] per column block.
    auto block_of = [&](float4 *base, int rb, int w) __attribute__((always_inline)) {
        return base + (rb * 3 + ((w - rb - 1) & 3)) * (4 * 64);
    };
    auto write_partials = [&](float4 *base, int j) __attribute__((always_inline)) {
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            if (rb == ks) continue;
            float4 *sl = block_of(base, rb, ks);
#pragma unroll
            for (int g = 0; g < 4; ++g)
                sl[g * 64 + lane] = make_float4(acc[rb][j][4 * g], acc[rb][j][4 * g + 1], acc[rb][j][4 * g + 2],
                                                acc[rb][j][4 * g + 3]);
        }
    };
    // fin[j]: ((P_c + P_c+1) + P_c+2) + P_c+3 for column block c = 2ch + j
    // (indices mod 4), the order of the 64-row kernel's reduction.  The
    // code is instantiated per k-step KS (= ks, dispatched by with_ks) so
    // that the own partial acc[KS][j] is a constant index: a runtime pick
    // among the four gets folded into a load from a computed address, which
    // puts all of acc in scratch memory.
    auto reduce_block = [&](auto kc, const float4 *base, int j) __attribute__((always_inline)) {
        constexpr int KS = decltype(kc)::value;
        const int cbl = 2 * ch + j;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            float4 term[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int w = (cbl + i) & 3;
                term[i] = w == KS ? make_float4(acc[KS][j][4 * g], acc[KS][j][4 * g + 1], acc[KS][j][4 * g + 2],
                                                acc[KS][j][4 * g + 3])
                                  : block_of(const_cast<float4 *>(base), KS, w)[g * 64 + lane];
            }
            float4 sum = term[0];
#pragma unroll
            for (int i = 1; i < 4; ++i) {
                sum.x += term[i].x;
                sum.y += term[i].y;
                sum.z += term[i].z;
                sum.w += term[i].w;
            }
            fin[j][4 * g] = sum.x;
            fin[j][4 * g + 1] = sum.y;
            fin[j][4 * g + 2] = sum.z;
            fin[j][4 * g + 3] = sum.w;
        }
    };
    auto with_ks = [&](auto f) __attribute__((always_inline)) {
        switch (ks) {
        case 0: f(std::integral_constant<int, 0>{}); break;
        case 1: f(std::integral_constant<int, 1>{}); break;
        case 2: f(std::integral_constant<int, 2>{}); break;
        default: f(std::integral_constant<int, 3>{}); break;
        }
    };
    // The staged output tile, unpadded at the top of LDS (the slots of a
    // whole-half reduction take the 96 KiB below it): 16-byte group q of row
    // r sits at q ^ 8 when r & 4, so rows r and r + 4 (written by one
    // instruction) fall on opposite halves of the banks.
    constexpr int kSlotBytes = 2 * 4 * 3 * 4096;
    static_assert(kSlotBytes + ROWS * STG_LD * 4 <= kH8Bytes, "slots and tile fit");
    float *stg = reinterpret_cast<float *>(smem + kSlotBytes);
    auto write_stg = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = (2 * ch + j) * 32 + (lane & 31);
            const int rb = ks * 32 + 4 * half;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = rb + 8 * (r >> 2) + (r & 3);
                stg[row * STG_LD + (col ^ (((row >> 2) & 1) << 5))] = fin[j][r];
            }
        }
    };
    float4 *slots = reinterpret_cast<float4 *>(smem);
    if (dbl || global_a) {  // a halo buffer is free during the last chunk
        if (ch == 0) {
            float4 *region = reinterpret_cast<float4 *>(global_a ? halo : buf_of(chunks));
            uint32_t *ctr = reinterpret_cast<uint32_t *>(rec + kHalfCounter);
            // all four waves of the half have arrived `round` times
            auto half_sync = [&](uint32_t round) __attribute__((always_inline)) {
                if (lane == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
                while (__hip_atomic_load(ctr, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < 4u * round)
                    __builtin_amdgcn_s_sleep(1);
            };
            write_partials(region, 0);
            half_sync(1);
            with_ks([&](auto kc) __attribute__((always_inline)) { reduce_block(kc, region, 0); });
            half_sync(2);  // every wave has read column block 0's partials
            write_partials(region, 1);
            half_sync(3);
            with_ks([&](auto kc) __attribute__((always_inline)) { reduce_block(kc, region, 1); });
        }
        __syncthreads();  // the loop and half 0's reduction are over: LDS is free
        if (ch == 0) {
            write_stg();
        } else {
            write_partials(slots, 0);
            write_partials(slots + 12 * 256, 1);
        }
        __syncthreads();
        if (ch == 1) {
            with_ks([&](auto kc) __attribute__((always_inline)) {
                reduce_block(kc, slots, 0);
                reduce_block(kc, slots + 12 * 256, 1);
            });
            write_stg();
        }
    } else {  // both halves at once, one column block per phase
        __syncthreads();  // the halo region becomes the reduction slots
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            if (j) __syncthreads();  // phase 0's slots have been read
            write_partials(slots + ch * 12 * 256, j);
            __syncthreads();
            with_ks([&](auto kc) __attribute__((always_inline)) { reduce_block(kc, slots + ch * 12 * 256, j); });
        }
        write_stg();
    }
    if (SK && part_out) {
        // part of a tile: its FP32 tile, rows in order, to the partial slot
        __syncthreads();
#pragma unroll
        for (int k = 0; k < ROWS * STG_LD / 4 / kHalo8Threads; ++k) {
            const int pc = tid + k * kHalo8Threads, row = pc >> 5, col = (pc & 31) * 4;
            reinterpret_cast<float4 *>(part_out)[pc] =
                *reinterpret_cast<const float4 *>(stg + row * STG_LD + (col ^ (((row >> 2) & 1) << 5)));
        }
    } else {
        load_row_mod(a, nb0 * 32 + (tid % 16) * 8, params);
        uint4 res[RowMap<16, ROWS, kHalo8Threads>::PASSES][2];
        load_residual<16, ROWS, kHalo8Threads>(a, m0, nb0, tile_rows, tid, res);
        __syncthreads();
        // (stream-K: 1/cout formed per piece, not held across the run)
        float inv_cout = 0.0f;
        if constexpr (SK) {
            inv_cout = 1.0f / static_cast<float>(opaque_scalar<SK>(a.cout));
            __builtin_assume(inv_cout != 0.0f);
        }
        finish_rows<16, ROWS, STG_LD, kHalo8Threads, true>(a, stg, stg, m0, nb0, tile_rows, tid, res, params,
                                                           inv_cout);
    }
    };
    if constexpr (!SK) {
        piece(xcd_tile(blockIdx.x, gridDim.x), blockIdx.y * 4, 0, chunks_all, nullptr);
    } else {
        const int64_t tiles = (a.n_out + ROWS - 1) / ROWS;
        const int g = xcd_tile(blockIdx.x, gridDim.x);  // XCD-contiguous runs
        const int64_t u1 = sk_run_begin(g + 1, a.sk_units, a.sk_wgs);
        int slot = 0;
        for (int64_t u = sk_run_begin(g, a.sk_units, a.sk_wgs); u < u1;) {
            // (divisors opaque per piece: their reciprocals are not held
            // in vector registers across the run)
            int64_t ca = chunks_all, nt = tiles;
            asm volatile("" : "+s"(ca), "+s"(nt));
            const int64_t gt = u / ca;  // column group * tiles + tile
            const int cb = static_cast<int>(u - gt * ca);
            const int ce = static_cast<int>(min(ca, cb + (u1 - u)));
            const int grp = static_cast<int>(gt / nt);
            const bool whole = cb == 0 && ce == chunks_all;
            __syncthreads();  // the previous piece is done with LDS
            piece(static_cast<int>(gt - grp * tiles), grp * 4, cb, ce,
                  whole ? nullptr : a.sk_partial + (static_cast<int64_t>(g) * 2 + slot) * (ROWS * STG_LD));
            slot += whole ? 0 : 1;
            u += ce - cb;
        }
    }
}

__global__ void __launch_bounds__(kHalo8Threads, 1) conv_halo8_kernel(ConvArgs a) { halo8_body<false>(a); }
__global__ void __launch_bounds__(kHalo8Threads, 1) conv_halo8_sk_kernel(ConvArgs a) { halo8_body<true>(a); }

// The tiles that stream-K runs left in parts: the pieces' FP32 tiles added
// in chunk order (the runs in order), then the epilogue of the whole-tile
// path.  One workgroup per (tile, column group); tiles that one run covers
// whole were finished by the conv kernel and are skipped.
__global__ void __launch_bounds__(kHalo8Threads, 1) halo8_combine_kernel(ConvArgs a) {
    constexpr int ROWS = 128, STG_LD = 128;
    __shared__ __align__(16) float stg[ROWS * STG_LD];
    const int tid = threadIdx.x;
    const int64_t tiles = gridDim.x;
    const int tile = blockIdx.x, nb0 = blockIdx.y * 4;
    const int chunks = a.cin / kHChunk;
    const int64_t uf = (static_cast<int64_t>(blockIdx.y) * tiles + tile) * chunks, ul = uf + chunks - 1;
    const int gf = sk_run_of(uf, a.sk_units, a.sk_wgs), gl = sk_run_of(ul, a.sk_units, a.sk_wgs);
    if (gf == gl) return;
    const int64_t m0 = static_cast<int64_t>(tile) * ROWS;
    const int tile_rows = static_cast<int>(min(static_cast<int64_t>(ROWS), a.n_out - m0));
    RowParams params;
    load_row_params(a, nb0 * 32 + (tid % 16) * 8, params);
    load_row_mod(a, nb0 * 32 + (tid % 16) * 8, params);
    constexpr int K = ROWS * STG_LD / 4 / kHalo8Threads;
    float4 sum[K];
    for (int g = gf; g <= gl; ++g) {
        // this tile's piece is run g's second partial one when the run began
        // in the middle of an earlier tile
        const int64_t b = sk_run_begin(g, a.sk_units, a.sk_wgs);
        const int slot = b < uf && b % chunks != 0 ? 1 : 0;
        const float4 *src = reinterpret_cast<const float4 *>(a.sk_partial + (static_cast<int64_t>(g) * 2 + slot) * (ROWS * STG_LD));
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const float4 v = src[tid + k * kHalo8Threads];
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
        const int pc = tid + k * kHalo8Threads, row = pc >> 5, col = (pc & 31) * 4;
        *reinterpret_cast<float4 *>(stg + row * STG_LD + (col ^ (((row >> 2) & 1) << 5))) = sum[k];
    }
    uint4 res[RowMap<16, ROWS, kHalo8Threads>::PASSES][2];
    load_residual<16, ROWS, kHalo8Threads>(a, m0, nb0, tile_rows, tid, res);
    __syncthreads();
    finish_rows<16, ROWS, STG_LD, kHalo8Threads, true>(a, stg, stg, m0, nb0, tile_rows, tid, res, params);
}

// Threads of a plan build's workgroup (one per tile): the dedupe's short
// dependent steps run on 16 (128-row) or 8 (64-row) waves, one bitmap word
// and about four map entries per thread.
constexpr int kPlanBuild128Threads = 1024;
constexpr int kPlanBuild64Threads = 512;

// One workgroup per tile (64 or 128 rows): dedupe_tile, then the record to
// memory.  128-row records hold halo byte offsets and name missing
// neighbours by the zero row of the kernel's halo layout: slot kH8Single when
// the tile's distinct rows need the single large buffer, else kH8Double (two
// buffers, one per chunk).
template <int MB, int NTH, class Fetch>
__device__ __forceinline__ void plan_tile(Fetch fetch, int64_t n_out, int64_t n_src, int32_t row_shift, char *plan) {
    using SM = HaloSmem<MB>;
    constexpr int ROWS = SM::ROWS;
    constexpr int REC = MB == 2 ? kGatherPlanRecord : kGatherPlanRecord128;
    constexpr int SLOTS = MB == 2 ? kPlanSlots : kPlan128Slots;
    __shared__ __align__(16) int32_t table32[ROWS * kMaxKvol];
    __shared__ __align__(16) uint16_t table[ROWS * kMaxKvol];
    __shared__ __align__(16) uint32_t bitmap[SM::BITWORDS];
    __shared__ __align__(16) uint32_t prefix[SM::BITWORDS];
    __shared__ __align__(16) uint32_t slot_row[SM::CAP];
    __shared__ __align__(16) int32_t misc[4 + NTH / 64];
    const int tile = xcd_tile(blockIdx.x, gridDim.x), tid = threadIdx.x;
    const int64_t m0 = static_cast<int64_t>(tile) * ROWS;
    const int tile_rows = static_cast<int>(min(static_cast<int64_t>(ROWS), n_out - m0));
    // The tables come back in entry order (row-major, 27 per row: no LDS
    // bank conflicts on writing them); the record stores them offset-major.
    const TileDedupe dd = dedupe_tile<MB, true, NTH>(fetch, n_src, row_shift, m0, tile_rows, table, table32, bitmap,
                                                     prefix, slot_row, misc);
    char *rec = plan + static_cast<int64_t>(tile) * REC;
    if (tid == 0)
        *reinterpret_cast<uint4 *>(rec) = make_uint4(dd.global_a ? 1u : 0u, dd.distinct, dd.mask, 0u);
    auto entry = [](int i) { return (i % ROWS) * kMaxKvol + i / ROWS; };  // record index -> entry
    constexpr int TABLE = MB == 2 ? kPlanHeader : kPlan128Table;
    if (dd.global_a) {
        for (int i = tid; i < ROWS * kMaxKvol; i += NTH)
            reinterpret_cast<int32_t *>(rec + TABLE)[i] = table32[entry(i)];
    } else {
        if constexpr (MB == 4) {
            const uint32_t z = dd.distinct <= static_cast<uint32_t>(kH8Double) ? kH8Double : kH8Single;
            for (int i = tid; i < ROWS * kMaxKvol; i += NTH) {
                const uint32_t sl = table[entry(i)];
                reinterpret_cast<uint32_t *>(rec + TABLE)[i] = halo_offset(sl == static_cast<uint32_t>(SM::CAP) ? z : sl);
            }
        } else {
            for (int i = tid; i < ROWS * kMaxKvol / 2; i += NTH)  // two rows of one offset per word
                reinterpret_cast<uint32_t *>(rec + kPlanHeader)[i] =
                    static_cast<uint32_t>(table[entry(2 * i)]) | static_cast<uint32_t>(table[entry(2 * i + 1)]) << 16;
        }
        for (int i = tid; i < static_cast<int>(dd.distinct); i += NTH)
            reinterpret_cast<uint32_t *>(rec + SLOTS)[i] = slot_row[i];
    }
}

template <int MB, int NTH>
__global__ void __launch_bounds__(NTH) gather_plan_build_kernel(const int32_t *kmap, int64_t n_out, int64_t n_src,
                                                                int32_t row_shift, char *plan) {
    plan_tile<MB, NTH>(SliceLoad{kmap, static_cast<int32_t>(n_out * kMaxKvol * 4)}, n_out, n_src, row_shift, plan);
}

// The tile's map slice computed by the lookups of the kernel map (and stored
// into it) instead of read back: the map and its gather plan in one pass.
using SliceLookup = KmapLookup4;

template <int MB, int NTH>
__global__ void __launch_bounds__(NTH) kmap_plan_kernel(const int4 *coords, int32_t n, KmapHash h, int32_t missing,
                                                        int32_t *kmap, char *plan) {
    const SliceLookup fetch{coords, n, missing, h, kmap_wide(h), kmap_dup(h), kmap};
    plan_tile<MB, NTH>(fetch, n, n, 0, plan);
}

}  // namespace

void launch_kmap_plan(int rows, const int32_t *coords, int64_t n, int32_t missing, int32_t *kmap, void *workspace,
                      uint64_t workspace_bytes, void *plan, hipStream_t stream) {
    const KmapHash h = kmap_insert_launch(reinterpret_cast<const int4 *>(coords), static_cast<int32_t>(n), workspace,
                                          workspace_bytes, stream);
    const unsigned tiles = static_cast<unsigned>((n + rows - 1) / rows);
    if (rows == 128)
        hipLaunchKernelGGL(HIP_KERNEL_NAME(kmap_plan_kernel<4, kPlanBuild128Threads>), dim3(tiles),
                           dim3(kPlanBuild128Threads), 0, stream, reinterpret_cast<const int4 *>(coords),
                           static_cast<int32_t>(n), h, missing, kmap, static_cast<char *>(plan));
    else
        hipLaunchKernelGGL(HIP_KERNEL_NAME(kmap_plan_kernel<2, kPlanBuild64Threads>), dim3(tiles),
                           dim3(kPlanBuild64Threads), 0, stream, reinterpret_cast<const int4 *>(coords),
                           static_cast<int32_t>(n), h, missing, kmap, static_cast<char *>(plan));
}

KernelFn pick_halo_bf16(int rows, int nb) {
    if (nb == 3) return rows == 64 ? conv_halo_kernel<2, false, 3> : nullptr;
    return rows == 128 ? conv_halo_kernel<4, false> : rows == 64 ? conv_halo_kernel<2, false> : nullptr;
}

KernelFn pick_halo8_stream_k() { return conv_halo8_sk_kernel; }

void launch_halo8_combine(const ConvArgs &a, int64_t tiles, int groups, hipStream_t stream) {
    hipLaunchKernelGGL(halo8_combine_kernel, dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(groups)),
                       dim3(kHalo8Threads), 0, stream, a);
}

KernelFn pick_halo_bf16_planned(int rows, int nb) {
    if (nb == 3) return rows == 64 ? conv_halo_kernel<2, true, 3> : nullptr;
    return rows == 64 ? conv_halo_kernel<2, true> : rows == 128 ? conv_halo8_kernel : nullptr;
}

void launch_gather_plan_build(int rows, const int32_t *kmap, int64_t n_out, int64_t n_src, int32_t row_shift,
                              void *plan, hipStream_t stream) {
    const unsigned tiles = static_cast<unsigned>((n_out + rows - 1) / rows);
    if (rows == 128)
        hipLaunchKernelGGL(HIP_KERNEL_NAME(gather_plan_build_kernel<4, kPlanBuild128Threads>), dim3(tiles),
                           dim3(kPlanBuild128Threads), 0, stream, kmap, n_out, n_src, row_shift,
                           static_cast<char *>(plan));
    else
        hipLaunchKernelGGL(HIP_KERNEL_NAME(gather_plan_build_kernel<2, kPlanBuild64Threads>), dim3(tiles),
                           dim3(kPlanBuild64Threads), 0, stream, kmap, n_out, n_src, row_shift,
                           static_cast<char *>(plan));
}

}  // namespace s3dx
