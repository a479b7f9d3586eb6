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
    } else {
        for (int k = 0; k < 5; ++k) w.template take<uint64_t>(un);
        for (int k = 0; k < 6; ++k) w.template take<int32_t>(un);
        w.template take<int32_t>(8);
        w.template take<char>(sort_bytes);
        w.template take<char>(scan_workspace_bytes(n));
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
