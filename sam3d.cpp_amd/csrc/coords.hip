// Occupancy -> sparse coordinates on the GPU: the steps between the sparse
// structure decoder's occupancy grid and the SLat stage's coordinate table.
//
// Reference (host C++, src/objects_runtime/session.cpp):
//   threshold occ > 0 in x-major order, batch 0        :1437-1441
//   prune_surface_coords (max_neighbor_axes_dist = 1)   :133-163
//   downsample_coords (max 42000, factor 2, seed 42)    :168-233
//
// Each is an ordered stream compaction (a flag per input row, an exclusive
// scan, a scatter), so outputs keep the reference's input order.  The
// reference identifies cells by coordinate_key (:122-127: b<<48 | x<<32 |
// y<<16 | z&0xffff, each field zero-extended, so the fields overlap); the
// hash here is keyed by that same 64-bit value, so cells that alias in the
// reference (negative or wide coordinates) alias here too.
#include "coord_hash.hpp"

#include <algorithm>
#include <cmath>
#include <numeric>
#include <random>
#include <vector>

namespace s3dx {
namespace {

// coordinate_key (session.cpp:122-127) as the hash's int4 key: its low and
// high 32-bit words.
__device__ __forceinline__ int4 cell_key(int32_t b, int32_t x, int32_t y, int32_t z) {
    const uint64_t k = (static_cast<uint64_t>(static_cast<uint32_t>(b)) << 48) |
                       (static_cast<uint64_t>(static_cast<uint32_t>(x)) << 32) |
                       (static_cast<uint64_t>(static_cast<uint32_t>(y)) << 16) |
                       static_cast<uint64_t>(static_cast<uint32_t>(z) & 0xffffu);
    return make_int4(static_cast<int32_t>(static_cast<uint32_t>(k)),
                     static_cast<int32_t>(static_cast<uint32_t>(k >> 32)), 0, 0);
}

__global__ void __launch_bounds__(kThreads)
cell_keys_kernel(const int4 *__restrict__ coords, int32_t n, int4 *__restrict__ keys) {
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const int4 c = coords[i];
    keys[i] = cell_key(c.x, c.y, c.z, c.w);
}

__global__ void __launch_bounds__(kThreads)
occ_flag_kernel(const float *__restrict__ occ, int64_t cells, int32_t *__restrict__ flag) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i < cells) flag[i] = occ[i] > 0.0f ? 1 : 0;
}

// Cell i = (x*ny + y)*nz + z becomes row pos[i] = (0, x, y, z).
__global__ void __launch_bounds__(kThreads)
occ_emit_kernel(const int32_t *__restrict__ flag, const int32_t *__restrict__ pos, int64_t cells,
                int32_t ny, int32_t nz, int4 *__restrict__ out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= cells || !flag[i]) return;
    const int64_t yz = static_cast<int64_t>(ny) * nz;
    const int64_t x = i / yz;
    const int64_t r = i - x * yz;
    out[pos[i]] = make_int4(0, static_cast<int32_t>(x), static_cast<int32_t>(r / nz),
                            static_cast<int32_t>(r % nz));
}

// One thread per (voxel, offset): flag[i] = 1 when the cell key of
// coords[i] + d(o) (same b; int32 arithmetic wrapping as on the host) is
// not among the voxels' keys (h built on them).  flag starts at zero; every
// writer writes 1.
__global__ void __launch_bounds__(kThreads)
surface_flag_kernel(const int4 *__restrict__ coords, int32_t n, Hash h, int32_t *__restrict__ flag) {
    const int32_t g = blockIdx.x * kThreads + threadIdx.x;
    if (g >= n * 27) return;
    const int32_t i = g / 27;
    const int32_t o = g - i * 27;
    const int4 c = coords[i];
    auto step = [](int32_t v, int d) {
        return static_cast<int32_t>(static_cast<uint32_t>(v) + static_cast<uint32_t>(d));
    };
    const int4 q = cell_key(c.x, step(c.y, o / 9 - 1), step(c.z, (o / 3) % 3 - 1), step(c.w, o % 3 - 1));
    if (hash_find(h, q) < 0) flag[i] = 1;
}

__global__ void __launch_bounds__(kThreads)
compact_rows_kernel(const int4 *__restrict__ in, int32_t n, const int32_t *__restrict__ flag,
                    const int32_t *__restrict__ pos, int4 *__restrict__ out) {
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i < n && flag[i]) out[pos[i]] = in[i];
}

// Bounding box of (x, y, z): bbox[0..2] min, bbox[3..5] max.
__global__ void __launch_bounds__(kThreads)
xyz_bbox_kernel(const int4 *__restrict__ coords, int32_t n, int32_t *bbox) {
    int v[6] = {INT32_MAX, INT32_MAX, INT32_MAX, INT32_MIN, INT32_MIN, INT32_MIN};
    for (int32_t i = blockIdx.x * kThreads + threadIdx.x; i < n; i += gridDim.x * kThreads) {
        const int4 c = coords[i];
        v[0] = min(v[0], c.y); v[1] = min(v[1], c.z); v[2] = min(v[2], c.w);
        v[3] = max(v[3], c.y); v[4] = max(v[4], c.z); v[5] = max(v[5], c.w);
    }
    block_bounds_atomic<3>(v, bbox);
}

// One axis of downsample_coords (session.cpp:180-211): the coordinate's
// position in [lo, hi] mapped onto the centred target range of
// (hi - lo + 1) / factor cells, rounded half up, clamped to the range's
// truncated ends.  Double precision, every operation rounded on its own (no
// fused multiply-add), so the results are the host's bit for bit.
__device__ __forceinline__ int32_t downsample_axis(int32_t v, int32_t lo, int32_t hi, int32_t factor) {
#pragma clang fp contract(off)
    const double original = static_cast<double>(hi - lo + 1);
    const double target = original / static_cast<double>(factor);
    const double offset = (original - target) * 0.5;
    const double target_min = static_cast<double>(lo) + offset;
    const double target_max = target_min + target - 1.0;
    const int32_t tmin = static_cast<int32_t>(target_min);  // truncation toward zero
    const int32_t tmax = static_cast<int32_t>(target_max);
    const double denom = static_cast<double>(hi - lo);
    const double normalized = denom > 0.0 ? (static_cast<double>(v) - lo) / denom : 0.0;
    const double value = normalized * (target - 1.0) + target_min;
    int64_t r = static_cast<int64_t>(floor(value + 0.5));
    r = r < tmin ? tmin : r;
    r = r > tmax ? tmax : r;
    return static_cast<int32_t>(r);
}

__global__ void __launch_bounds__(kThreads)
downsample_map_kernel(const int4 *__restrict__ coords, int32_t n, const int32_t *__restrict__ bbox,
                      int32_t factor, int4 *__restrict__ mapped) {
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const int4 c = coords[i];
    mapped[i] = make_int4(c.x, downsample_axis(c.y, bbox[0], bbox[3], factor),
                          downsample_axis(c.z, bbox[1], bbox[4], factor),
                          downsample_axis(c.w, bbox[2], bbox[5], factor));
}

// flag[i] = 1 for the first row of each key (after hash_build on keys).
__global__ void __launch_bounds__(kThreads)
first_flag_kernel(const int4 *__restrict__ keys, int32_t n, Hash h, int32_t *__restrict__ flag) {
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i < n) flag[i] = hash_find(h, keys[i]) == i ? 1 : 0;
}

__global__ void __launch_bounds__(kThreads)
gather_rows_kernel(const int4 *__restrict__ in, const int32_t *__restrict__ idx, int32_t m,
                   int4 *__restrict__ out) {
    const int32_t j = blockIdx.x * kThreads + threadIdx.x;
    if (j < m) out[j] = in[idx[j]];
}

void check_coord_rows(const int32_t *coords, int64_t n, int64_t max_n) {
    require(coords != nullptr, "coords is NULL");
    require(aligned(coords, 16), "coords must be 16-byte aligned");
    require(n > 0, "voxel count must be positive");
    require(n <= max_n, "voxel count out of range");
}

int64_t read_count(const int32_t *total, hipStream_t s) {
    int32_t v = 0;
    hip_check(hipMemcpyAsync(&v, total, sizeof(v), hipMemcpyDeviceToHost, s), "hipMemcpyAsync count");
    hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    return v;
}

// ---- workspace layouts ------------------------------------------------------
struct OccLayout {
    int32_t *flag, *pos, *totals;
    void *scan_ws;
};
template <class W>
void occ_layout(W &w, int64_t cells, OccLayout *l) {
    const uint64_t u = static_cast<uint64_t>(cells);
    if constexpr (std::is_same_v<W, Carver>) {
        l->flag = w.template take<int32_t>(u);
        l->pos = w.template take<int32_t>(u);
        l->totals = w.template take<int32_t>(8);
        l->scan_ws = w.template take<char>(scan_workspace_bytes(cells));
    } else {
        w.template take<int32_t>(u);
        w.template take<int32_t>(u);
        w.template take<int32_t>(8);
        w.template take<char>(scan_workspace_bytes(cells));
    }
}

struct PruneLayout {
    Hash hash;
    int4 *keys;
    int32_t *flag, *pos, *totals;
    void *scan_ws;
};
template <class W>
void prune_layout(W &w, int64_t n, PruneLayout *l) {
    const uint64_t u = static_cast<uint64_t>(n);
    if constexpr (std::is_same_v<W, Carver>) {
        hash_layout(w, n, &l->hash);
        l->keys = w.template take<int4>(u);
        l->flag = w.template take<int32_t>(u);
        l->pos = w.template take<int32_t>(u);
        l->totals = w.template take<int32_t>(8);
        l->scan_ws = w.template take<char>(scan_workspace_bytes(n));
    } else {
        hash_layout(w, n, static_cast<Hash *>(nullptr));
        w.template take<int4>(u);
        w.template take<int32_t>(u);
        w.template take<int32_t>(u);
        w.template take<int32_t>(8);
        w.template take<char>(scan_workspace_bytes(n));
    }
}

struct DownsampleLayout {
    Hash hash;
    int32_t *bbox, *flag, *pos, *idx, *totals;
    int4 *mapped, *keys, *unique;
    void *scan_ws;
};
template <class W>
void downsample_layout(W &w, int64_t n, DownsampleLayout *l) {
    const uint64_t u = static_cast<uint64_t>(n);
    if constexpr (std::is_same_v<W, Carver>) {
        hash_layout(w, n, &l->hash);
        l->bbox = w.template take<int32_t>(8);
        l->flag = w.template take<int32_t>(u);
        l->pos = w.template take<int32_t>(u);
        l->idx = w.template take<int32_t>(u);
        l->totals = w.template take<int32_t>(8);
        l->mapped = w.template take<int4>(u);
        l->keys = w.template take<int4>(u);
        l->unique = w.template take<int4>(u);
        l->scan_ws = w.template take<char>(scan_workspace_bytes(n));
    } else {
        hash_layout(w, n, static_cast<Hash *>(nullptr));
        w.template take<int32_t>(8);
        for (int k = 0; k < 3; ++k) w.template take<int32_t>(u);
        w.template take<int32_t>(8);
        for (int k = 0; k < 3; ++k) w.template take<int4>(u);
        w.template take<char>(scan_workspace_bytes(n));
    }
}

}  // namespace
}  // namespace s3dx

using namespace s3dx;

extern "C" {

S3DX_API s3dx_status s3dx_occupancy_workspace_size(int32_t nx, int32_t ny, int32_t nz, uint64_t *bytes,
                                                   char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(bytes != nullptr, "bytes is NULL");
        require(nx > 0 && ny > 0 && nz > 0, "grid extents must be positive");
        const int64_t cells = static_cast<int64_t>(nx) * ny * nz;
        require(cells <= INT32_MAX, "grid has more than INT32_MAX cells");
        Sizer s;
        occ_layout(s, cells, nullptr);
        *bytes = s.used;
    });
}

S3DX_API s3dx_status s3dx_occupancy_coords(const float *occupancy, int32_t nx, int32_t ny, int32_t nz,
                                           int32_t *coords, int64_t *count, void *workspace,
                                           uint64_t workspace_bytes, s3dx_stream stream, char *error,
                                           uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(occupancy && coords && count && workspace, "NULL argument");
        require(aligned(coords, 16), "coords must be 16-byte aligned");
        require(nx > 0 && ny > 0 && nz > 0, "grid extents must be positive");
        const int64_t cells = static_cast<int64_t>(nx) * ny * nz;
        require(cells <= INT32_MAX, "grid has more than INT32_MAX cells");
        const hipStream_t s = as_stream(stream);
        Carver w(workspace, workspace_bytes);
        OccLayout l;
        occ_layout(w, cells, &l);
        const unsigned blocks = static_cast<unsigned>((cells + kThreads - 1) / kThreads);
        occ_flag_kernel<<<blocks, kThreads, 0, s>>>(occupancy, cells, l.flag);
        launch_check("occ_flag");
        exclusive_scan_i32(l.flag, l.pos, cells, l.totals, l.scan_ws, s);
        occ_emit_kernel<<<blocks, kThreads, 0, s>>>(l.flag, l.pos, cells, ny, nz,
                                                    reinterpret_cast<int4 *>(coords));
        launch_check("occ_emit");
        *count = read_count(l.totals, s);
    });
}

S3DX_API s3dx_status s3dx_prune_surface_workspace_size(int64_t n, uint64_t *bytes, char *error,
                                                       uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(bytes != nullptr, "bytes is NULL");
        require(n > 0 && n <= INT32_MAX / 27, "voxel count out of range");
        Sizer s;
        prune_layout(s, n, nullptr);
        *bytes = s.used;
    });
}

S3DX_API s3dx_status s3dx_prune_surface(const int32_t *coords, int64_t n, int32_t *surface,
                                        int64_t *count, void *workspace, uint64_t workspace_bytes,
                                        s3dx_stream stream, char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        check_coord_rows(coords, n, INT32_MAX / 27);
        require(surface && count && workspace, "NULL argument");
        require(aligned(surface, 16), "surface must be 16-byte aligned");
        const hipStream_t s = as_stream(stream);
        const int32_t ni = static_cast<int32_t>(n);
        Carver w(workspace, workspace_bytes);
        PruneLayout l;
        prune_layout(w, n, &l);
        const int4 *c4 = reinterpret_cast<const int4 *>(coords);
        cell_keys_kernel<<<blocks_for(n), kThreads, 0, s>>>(c4, ni, l.keys);
        launch_check("cell_keys");
        hash_build(l.keys, ni, l.hash, s);
        fill_u32(reinterpret_cast<uint32_t *>(l.flag), static_cast<uint64_t>(n), 0u, s);
        surface_flag_kernel<<<blocks_for(n * 27), kThreads, 0, s>>>(c4, ni, l.hash, l.flag);
        launch_check("surface_flag");
        exclusive_scan_i32(l.flag, l.pos, n, l.totals, l.scan_ws, s);
        compact_rows_kernel<<<blocks_for(n), kThreads, 0, s>>>(c4, ni, l.flag, l.pos,
                                                              reinterpret_cast<int4 *>(surface));
        launch_check("compact_rows");
        *count = read_count(l.totals, s);
    });
}

S3DX_API s3dx_status s3dx_downsample_coords_workspace_size(int64_t n, uint64_t *bytes, char *error,
                                                           uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(bytes != nullptr, "bytes is NULL");
        require(n > 0 && n <= INT32_MAX, "voxel count out of range");
        Sizer s;
        downsample_layout(s, n, nullptr);
        *bytes = s.used;
    });
}

S3DX_API s3dx_status s3dx_downsample_coords(const int32_t *coords, int64_t n, int64_t max_coords,
                                            int32_t factor, uint32_t seed, int32_t *out, int64_t *count,
                                            void *workspace, uint64_t workspace_bytes, s3dx_stream stream,
                                            char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        check_coord_rows(coords, n, INT32_MAX);
        require(out && count && workspace, "NULL argument");
        require(aligned(out, 16), "out must be 16-byte aligned");
        require(max_coords >= 0, "max_coords must be non-negative");
        require(factor > 0, "downsample factor must be positive");
        const hipStream_t s = as_stream(stream);
        // At most max_coords rows: the set is returned as it is
        // (session.cpp:174), duplicates included.
        if (n <= max_coords) {
            hip_check(hipMemcpyAsync(out, coords, static_cast<size_t>(n) * 16, hipMemcpyDeviceToDevice, s),
                      "hipMemcpyAsync");
            *count = n;
            return;
        }
        const int32_t ni = static_cast<int32_t>(n);
        Carver w(workspace, workspace_bytes);
        DownsampleLayout l;
        downsample_layout(w, n, &l);
        const int4 *c4 = reinterpret_cast<const int4 *>(coords);
        fill_u32(reinterpret_cast<uint32_t *>(l.bbox), 3, static_cast<uint32_t>(INT32_MAX), s);
        fill_u32(reinterpret_cast<uint32_t *>(l.bbox) + 3, 3, static_cast<uint32_t>(INT32_MIN), s);
        xyz_bbox_kernel<<<bounds_blocks(n), kThreads, 0, s>>>(c4, ni, l.bbox);
        launch_check("xyz_bbox");
        downsample_map_kernel<<<blocks_for(n), kThreads, 0, s>>>(c4, ni, l.bbox, factor, l.mapped);
        launch_check("downsample_map");
        // First occurrence of each mapped cell key, in input order (:213-215).
        cell_keys_kernel<<<blocks_for(n), kThreads, 0, s>>>(l.mapped, ni, l.keys);
        launch_check("cell_keys");
        hash_build(l.keys, ni, l.hash, s);
        first_flag_kernel<<<blocks_for(n), kThreads, 0, s>>>(l.keys, ni, l.hash, l.flag);
        launch_check("first_flag");
        exclusive_scan_i32(l.flag, l.pos, n, l.totals, l.scan_ws, s);
        compact_rows_kernel<<<blocks_for(n), kThreads, 0, s>>>(l.mapped, ni, l.flag, l.pos, l.unique);
        launch_check("compact_rows");
        const int64_t unique_n = read_count(l.totals, s);
        if (unique_n <= max_coords) {
            hip_check(hipMemcpyAsync(out, l.unique, static_cast<size_t>(unique_n) * 16,
                                     hipMemcpyDeviceToDevice, s),
                      "hipMemcpyAsync");
            *count = unique_n;
            return;
        }
        // More than max_coords cells: the reference's sample, the first
        // max_coords entries of a std::shuffle of 0..unique_n-1 under
        // std::mt19937(seed) (:217-229).  The permutation depends only on
        // unique_n and the seed, so the host draws it with the same standard
        // library and the GPU gathers the rows.
        std::mt19937 rng(seed);
        std::vector<size_t> order(static_cast<size_t>(unique_n));
        std::iota(order.begin(), order.end(), size_t(0));
        std::shuffle(order.begin(), order.end(), rng);
        std::vector<int32_t> pick(static_cast<size_t>(max_coords));
        for (size_t j = 0; j < pick.size(); ++j) pick[j] = static_cast<int32_t>(order[j]);
        if (!pick.empty()) {
            hip_check(hipMemcpyAsync(l.idx, pick.data(), pick.size() * sizeof(int32_t), hipMemcpyHostToDevice, s),
                      "hipMemcpyAsync");
            gather_rows_kernel<<<blocks_for(max_coords), kThreads, 0, s>>>(
                l.unique, l.idx, static_cast<int32_t>(max_coords), reinterpret_cast<int4 *>(out));
            launch_check("gather_rows");
            hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");  // pick stays alive until the copy ends
        }
        *count = max_coords;
    });
}

}  // extern "C"
