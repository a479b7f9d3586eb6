// The 2x coarsen of a voxel set: SlatTables' downsample tables
// (sparse_ops.cpp:53-104) -- the coarse set, fine -> coarse rows, each coarse
// row's first 8 fine rows and 1 / (count + 1).
//
// The reference keys a std::map by (b, x/2, y/2, z/2) (C++ division, toward
// zero) and visits the fine rows in order, so the coarse rows are the
// distinct keys in lexicographic order and each key lists its fine rows
// ascending.  Here the keys are sorted instead: the key's four int32, sign
// bit flipped, form two unsigned 64-bit halves whose (hi, lo) order is that
// lexicographic order; a stable radix sort by lo, then by hi, of the row
// indices 0..n-1 leaves equal keys adjacent with their rows ascending.  A
// flag per new key and a scan give every sorted row its coarse rank.  Any
// int32 coordinates, any bounding box; O(n) work, one host synchronization
// (to return nc).
//
// Sets of batch 0 in [0, 128)^3 (the SLat grids) take a window instead, with
// no sort: their coarse cells index a 64^3 bitmap in (x, y, z) order -- the
// std::map order of the keys -- so a popcount scan over the bitmap ranks
// them; each fine row takes one of its coarse row's eight slots, and a pass
// per coarse row sorts its slots (its rows ascending).  A coarse cell with
// more than eight rows (duplicate coordinates) or a row outside the window
// raises a flag read at the synchronization, and the sort runs instead.
#include "coord_hash.hpp"

#include <rocprim/device/device_radix_sort.hpp>

#include <type_traits>

namespace s3dx {
namespace {

__device__ __forceinline__ uint64_t flip(int32_t v) { return static_cast<uint32_t>(v) ^ 0x80000000u; }
__device__ __forceinline__ int32_t unflip(uint64_t v) {
    return static_cast<int32_t>(static_cast<uint32_t>(v) ^ 0x80000000u);
}

__global__ void __launch_bounds__(kThreads)
coarse_key_halves_kernel(const int4 *__restrict__ coords, int32_t n, uint64_t *__restrict__ hi,
                         uint64_t *__restrict__ lo, int32_t *__restrict__ rows) {
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const int4 c = coords[i];
    // C++ integer division truncates toward zero (sparse_ops.cpp:63-64).
    hi[i] = (flip(c.x) << 32) | flip(c.y / 2);
    lo[i] = (flip(c.z / 2) << 32) | flip(c.w / 2);
    rows[i] = i;
}

__global__ void __launch_bounds__(kThreads)
gather_u64_kernel(const uint64_t *__restrict__ src, const int32_t *__restrict__ idx, int32_t n,
                  uint64_t *__restrict__ dst) {
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i < n) dst[i] = src[idx[i]];
}

// 1 where the sorted key differs from its predecessor.
__global__ void __launch_bounds__(kThreads)
new_key_kernel(const uint64_t *__restrict__ hi, const uint64_t *__restrict__ lo, int32_t n,
               int32_t *__restrict__ flag) {
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i < n) flag[i] = i == 0 || hi[i] != hi[i - 1] || lo[i] != lo[i - 1] ? 1 : 0;
}

// Sorted position i has coarse rank ex[i] + flag[i] - 1 (ex: exclusive scan
// of the flags); the first position of a rank records the coarse key and
// where the rank's rows start.
__global__ void __launch_bounds__(kThreads)
assign_kernel(const uint64_t *__restrict__ hi, const uint64_t *__restrict__ lo, const int32_t *__restrict__ rows,
              const int32_t *__restrict__ flag, const int32_t *__restrict__ ex, int32_t n,
              int32_t *__restrict__ f2c, int4 *__restrict__ coarse_coords, int32_t *__restrict__ starts) {
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const int32_t r = ex[i] + flag[i] - 1;
    f2c[rows[i]] = r;
    if (flag[i]) {
        starts[r] = i;
        coarse_coords[r] = make_int4(unflip(hi[i] >> 32), unflip(hi[i]), unflip(lo[i] >> 32), unflip(lo[i]));
    }
}

// Per coarse row: its first 8 fine rows (ascending; n pads) and
// 1 / (count + 1) (sparse_ops.cpp:82-104).  nc is read on the device.
__global__ void __launch_bounds__(kThreads)
children_kernel(const int32_t *__restrict__ rows, const int32_t *__restrict__ starts, const int32_t *nc_dev,
                int32_t n, int32_t *__restrict__ children, float *__restrict__ inv_count) {
    const int32_t r = blockIdx.x * kThreads + threadIdx.x;
    const int32_t nc = *nc_dev;
    if (r >= nc) return;
    const int32_t s = starts[r], e = r + 1 < nc ? starts[r + 1] : n, k = e - s;
#pragma unroll
    for (int j = 0; j < 8; ++j) children[static_cast<int64_t>(r) * 8 + j] = j < k ? rows[s + j] : n;
    inv_count[r] = 1.0f / static_cast<float>(k + 1);
}

// ---- window path ----------------------------------------------------------
constexpr int kCoarseWindowLog2 = 6;                                   // 64^3 coarse cells
constexpr int kCoarseWords = (1 << (3 * kCoarseWindowLog2)) / 32;       // 8,192 bitmap words
constexpr int kScanThreads = 1024;
static_assert(kCoarseWords % kScanThreads == 0, "whole words per scan thread");
enum { kOutside = 0, kOverflow = 1 };  // flag words

// Zeroes the bitmap, the flags and the slot counters (n).
__global__ void __launch_bounds__(kThreads)
window_clear_kernel(uint32_t *__restrict__ bitmap, uint32_t *__restrict__ flags, int32_t *__restrict__ cnt,
                    int32_t n) {
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i < kCoarseWords) bitmap[i] = 0u;
    if (i < 2) flags[i] = 0u;
    if (i < n) cnt[i] = 0;
}

__device__ __forceinline__ int32_t coarse_cell(int4 c) {
    constexpr int kFine = 2 << kCoarseWindowLog2;  // 128
    if (c.x != 0 || static_cast<uint32_t>(c.y) >= kFine || static_cast<uint32_t>(c.z) >= kFine ||
        static_cast<uint32_t>(c.w) >= kFine)
        return -1;
    // (nonnegative: C++ truncation is the shift)
    return ((((c.y >> 1) << kCoarseWindowLog2) + (c.z >> 1)) << kCoarseWindowLog2) + (c.w >> 1);
}

__global__ void __launch_bounds__(kThreads)
window_mark_kernel(const int4 *__restrict__ coords, int32_t n, uint32_t *__restrict__ bitmap,
                   uint32_t *__restrict__ flags) {
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const int32_t cell = coarse_cell(coords[i]);
    if (cell < 0) atomicOr(&flags[kOutside], 1u);
    else atomicOr(&bitmap[cell >> 5], 1u << (cell & 31));
}

// One workgroup: prefix[w] = occupied cells in words 0..w-1; *total = nc.
__global__ void __launch_bounds__(kScanThreads)
window_scan_kernel(const uint32_t *__restrict__ bitmap, uint32_t *__restrict__ prefix, int32_t *__restrict__ total) {
    constexpr int WPT = kCoarseWords / kScanThreads;
    __shared__ uint32_t wave_sums[kScanThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t cnt[WPT], mine = 0;
#pragma unroll
    for (int k = 0; k < WPT; ++k) {
        cnt[k] = static_cast<uint32_t>(__popc(bitmap[tid * WPT + k]));
        mine += cnt[k];
    }
    uint32_t incl = mine;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t t = __shfl_up(incl, d, 64);
        if (lane >= d) incl += t;
    }
    if (lane == 63) wave_sums[wave] = incl;
    __syncthreads();
    uint32_t base = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kScanThreads / 64; ++w) {
        base += w < wave ? wave_sums[w] : 0u;
        all += wave_sums[w];
    }
    uint32_t run = base + incl - mine;
#pragma unroll
    for (int k = 0; k < WPT; ++k) {
        prefix[tid * WPT + k] = run;
        run += cnt[k];
    }
    if (tid == 0) *total = static_cast<int32_t>(all);
}

// Fine row i: its coarse rank, the coarse key, and one of the rank's eight slots.
__global__ void __launch_bounds__(kThreads)
window_assign_kernel(const int4 *__restrict__ coords, int32_t n, const uint32_t *__restrict__ bitmap,
                     const uint32_t *__restrict__ prefix, uint32_t *__restrict__ flags, int32_t *__restrict__ f2c,
                     int4 *__restrict__ coarse_coords, int32_t *__restrict__ cnt, int32_t *__restrict__ slots) {
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n || flags[kOutside] != 0u) return;
    const int4 c = coords[i];
    const int32_t cell = coarse_cell(c);
    const uint32_t w = static_cast<uint32_t>(cell) >> 5, bit = static_cast<uint32_t>(cell) & 31u;
    const int32_t r = static_cast<int32_t>(prefix[w] + static_cast<uint32_t>(__popc(bitmap[w] & ((1u << bit) - 1u))));
    f2c[i] = r;
    coarse_coords[r] = make_int4(0, c.y >> 1, c.z >> 1, c.w >> 1);  // (every row of r writes the same key)
    const int32_t k = atomicAdd(&cnt[r], 1);
    if (k < 8) slots[static_cast<int64_t>(r) * 8 + k] = i;
    else atomicOr(&flags[kOverflow], 1u);
}

// Per coarse row: its rows ascending (at most eight here), padded with n, and
// 1 / (count + 1).
__global__ void __launch_bounds__(kThreads)
window_children_kernel(const int32_t *__restrict__ cnt, const int32_t *__restrict__ slots, const int32_t *nc_dev,
                       const uint32_t *__restrict__ flags, int32_t n, int32_t *__restrict__ children,
                       float *__restrict__ inv_count) {
    const int32_t r = blockIdx.x * kThreads + threadIdx.x;
    if (r >= *nc_dev || flags[kOutside] != 0u || flags[kOverflow] != 0u) return;
    const int32_t k = cnt[r];
    int32_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = j < k ? slots[static_cast<int64_t>(r) * 8 + j] : n;
    // the slots in arrival order; an insertion sort of the eight puts the rows ascending
#pragma unroll
    for (int a = 1; a < 8; ++a)
#pragma unroll
        for (int b = a; b > 0; --b)
            if (v[b] < v[b - 1]) {
                const int32_t t = v[b];
                v[b] = v[b - 1];
                v[b - 1] = t;
            }
#pragma unroll
    for (int j = 0; j < 8; ++j) children[static_cast<int64_t>(r) * 8 + j] = v[j];
    inv_count[r] = 1.0f / static_cast<float>(k + 1);
}

size_t sort_temp_bytes(int64_t n) {
    size_t bytes = 0;
    hip_check(rocprim::radix_sort_pairs(nullptr, bytes, static_cast<const uint64_t *>(nullptr),
                                        static_cast<uint64_t *>(nullptr), static_cast<const int32_t *>(nullptr),
                                        static_cast<int32_t *>(nullptr), static_cast<uint32_t>(n)),
              "radix_sort_pairs size");
    return bytes;
}

struct CoarsenLayout {
    uint64_t *hi0, *lo0, *hi1, *hi2, *lo2;
    int32_t *rows0, *rows1, *rows2, *flag, *ex, *starts, *totals;
    void *sort_ws, *scan_ws;
    size_t sort_bytes;
    // window path: bitmap, word prefixes, flags, slot counters and slots
    uint32_t *bitmap, *prefix, *wflags;
    int32_t *cnt, *slots;
};
template <class W>
void coarsen_layout(W &w, int64_t n, CoarsenLayout *l) {
    const uint64_t un = static_cast<uint64_t>(n);
    const size_t sort_bytes = sort_temp_bytes(n);
    if constexpr (std::is_same_v<W, Carver>) {
        l->hi0 = w.template take<uint64_t>(un);
        l->lo0 = w.template take<uint64_t>(un);
        l->hi1 = w.template take<uint64_t>(un);
        l->hi2 = w.template take<uint64_t>(un);
        l->lo2 = w.template take<uint64_t>(un);
        l->rows0 = w.template take<int32_t>(un);
        l->rows1 = w.template take<int32_t>(un);
        l->rows2 = w.template take<int32_t>(un);
        l->flag = w.template take<int32_t>(un);
        l->ex = w.template take<int32_t>(un);
        l->starts = w.template take<int32_t>(un);
        l->totals = w.template take<int32_t>(8);
        l->sort_ws = w.template take<char>(sort_bytes);
        l->scan_ws = w.template take<char>(scan_workspace_bytes(n));
        l->sort_bytes = sort_bytes;
        l->bitmap = w.template take<uint32_t>(kCoarseWords);
        l->prefix = w.template take<uint32_t>(kCoarseWords);
        l->wflags = w.template take<uint32_t>(2);
        l->cnt = w.template take<int32_t>(un);
        l->slots = w.template take<int32_t>(un * 8);
    } else {
        for (int k = 0; k < 5; ++k) w.template take<uint64_t>(un);
        for (int k = 0; k < 6; ++k) w.template take<int32_t>(un);
        w.template take<int32_t>(8);
        w.template take<char>(sort_bytes);
        w.template take<char>(scan_workspace_bytes(n));
        w.template take<uint32_t>(kCoarseWords);
        w.template take<uint32_t>(kCoarseWords);
        w.template take<uint32_t>(2);
        w.template take<int32_t>(un);
        w.template take<int32_t>(un * 8);
    }
}

}  // namespace
}  // namespace s3dx

using namespace s3dx;

extern "C" {

S3DX_API s3dx_status s3dx_coarsen2_workspace_size(int64_t n, uint64_t *bytes, char *error,
                                                  uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(bytes != nullptr, "bytes is NULL");
        require(n > 0 && n <= INT32_MAX / 27, "voxel count out of range");
        Sizer s;
        coarsen_layout(s, n, nullptr);
        *bytes = s.used;
    });
}

S3DX_API s3dx_status s3dx_coarsen2(const int32_t *coords, int64_t n, int32_t *coarse_coords,
                                   int32_t *fine_to_coarse, int32_t *coarse_children,
                                   float *coarse_inv_count, int64_t *nc_out, void *workspace,
                                   uint64_t workspace_bytes, s3dx_stream stream, char *error,
                                   uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(coords != nullptr, "coords is NULL");
        require(aligned(coords, 16), "coords must be 16-byte aligned");
        require(n > 0, "voxel count must be positive");
        require(n <= INT32_MAX / 27, "voxel count exceeds INT32_MAX / 27");
        require(coarse_coords && fine_to_coarse && coarse_children && coarse_inv_count && nc_out,
                "NULL output");
        require(aligned(coarse_coords, 16), "coarse_coords must be 16-byte aligned");
        require(workspace != nullptr, "workspace is NULL");
        const hipStream_t s = as_stream(stream);
        const int32_t ni = static_cast<int32_t>(n);
        const uint32_t un = static_cast<uint32_t>(n);
        Carver w(workspace, workspace_bytes);
        CoarsenLayout l;
        coarsen_layout(w, n, &l);
        const unsigned blocks = blocks_for(ni);

        // 0. the window path; its flags and nc come back at the one
        // synchronization, and only a flag sends the set through the sort
        window_clear_kernel<<<blocks_for(std::max<int64_t>(n, kCoarseWords)), kThreads, 0, s>>>(l.bitmap, l.wflags,
                                                                                              l.cnt, ni);
        launch_check("window_clear");
        window_mark_kernel<<<blocks, kThreads, 0, s>>>(reinterpret_cast<const int4 *>(coords), ni, l.bitmap, l.wflags);
        launch_check("window_mark");
        window_scan_kernel<<<1, kScanThreads, 0, s>>>(l.bitmap, l.prefix, l.totals);
        launch_check("window_scan");
        window_assign_kernel<<<blocks, kThreads, 0, s>>>(reinterpret_cast<const int4 *>(coords), ni, l.bitmap,
                                                         l.prefix, l.wflags, fine_to_coarse,
                                                         reinterpret_cast<int4 *>(coarse_coords), l.cnt, l.slots);
        launch_check("window_assign");
        window_children_kernel<<<blocks, kThreads, 0, s>>>(l.cnt, l.slots, l.totals, l.wflags, ni, coarse_children,
                                                           coarse_inv_count);
        launch_check("window_children");
        struct {
            int32_t nc;
            uint32_t flags[2];
        } back{};
        hip_check(hipMemcpyAsync(&back.nc, l.totals, sizeof(int32_t), hipMemcpyDeviceToHost, s), "hipMemcpyAsync nc");
        hip_check(hipMemcpyAsync(back.flags, l.wflags, sizeof(back.flags), hipMemcpyDeviceToHost, s),
                  "hipMemcpyAsync flags");
        hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
        if (back.flags[kOutside] == 0u && back.flags[kOverflow] == 0u) {
            require(back.nc > 0 && back.nc <= ni, "coarse row count out of range");
            *nc_out = back.nc;
            return;
        }

        // 1. the two key halves; rows 0..n-1
        coarse_key_halves_kernel<<<blocks, kThreads, 0, s>>>(reinterpret_cast<const int4 *>(coords), ni, l.hi0,
                                                             l.lo0, l.rows0);
        launch_check("coarse_key_halves");
        // 2. stable sort by lo, then by hi: (hi, lo) order, rows ascending per key
        size_t bytes = l.sort_bytes;
        hip_check(rocprim::radix_sort_pairs(l.sort_ws, bytes, l.lo0, l.hi2, l.rows0, l.rows1, un, 0, 64, s),
                  "radix_sort_pairs (lo)");
        gather_u64_kernel<<<blocks, kThreads, 0, s>>>(l.hi0, l.rows1, ni, l.hi1);
        launch_check("gather_hi");
        bytes = l.sort_bytes;
        hip_check(rocprim::radix_sort_pairs(l.sort_ws, bytes, l.hi1, l.hi2, l.rows1, l.rows2, un, 0, 64, s),
                  "radix_sort_pairs (hi)");
        gather_u64_kernel<<<blocks, kThreads, 0, s>>>(l.lo0, l.rows2, ni, l.lo2);
        launch_check("gather_lo");
        // 3. ranks, coarse keys, fine -> coarse, rank starts
        new_key_kernel<<<blocks, kThreads, 0, s>>>(l.hi2, l.lo2, ni, l.flag);
        launch_check("new_key");
        exclusive_scan_i32(l.flag, l.ex, n, l.totals, l.scan_ws, s);
        assign_kernel<<<blocks, kThreads, 0, s>>>(l.hi2, l.lo2, l.rows2, l.flag, l.ex, ni, fine_to_coarse,
                                                  reinterpret_cast<int4 *>(coarse_coords), l.starts);
        launch_check("assign");
        // 4. children and 1 / (count + 1)
        children_kernel<<<blocks, kThreads, 0, s>>>(l.rows2, l.starts, l.totals, ni, coarse_children,
                                                    coarse_inv_count);
        launch_check("children");
        int32_t nc = 0;
        hip_check(hipMemcpyAsync(&nc, l.totals, sizeof(nc), hipMemcpyDeviceToHost, s), "hipMemcpyAsync nc");
        hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
        require(nc > 0 && nc <= ni, "coarse row count out of range");
        *nc_out = nc;
    });
}

}  // extern "C"
