// Kernel maps on the GPU: the 27-offset submanifold neighbour table and the
// exact 2x subdivide (the 2x coarsen is in coarsen.hip).
//
// Reference semantics (all host C++ in sam3d.cpp):
//   build_conv            src/objects_runtime/sparse_ops.cpp:117-142
//   SlatTables downsample src/objects_runtime/sparse_ops.cpp:53-104
//   MeshSubdivideTables   src/objects_runtime/sparse_ops.cpp:272-404
//
// The coordinate hash (coord_hash.hpp) gives every key its smallest row, as
// std::map::emplace's "first occurrence wins" does.
#include "kmap_table.hpp"

#include <atomic>
#include <mutex>
#include <vector>

namespace s3dx {
namespace {

// Hash path of the insert (coordinates outside the window): claim a slot
// for row i, or lower the row of the slot already holding its key.
__device__ __forceinline__ void kmap_hash_insert(const int4 *__restrict__ keys, int32_t n, const KmapHash &h, int32_t i,
                                         int4 c) {
    const bool fits = fits16(c);
    if (!fits) h.flags[kFlagWide] = flag_of(h.seed, kFlagWide);
    uint32_t pos = key_hash(c) & h.mask;
    for (uint32_t probe = 0; probe <= h.mask; ++probe) {
        const uint32_t tag = tag_of(h.seed, pos);
        auto *word = reinterpret_cast<unsigned long long *>(&h.slots[pos]) + 1;  // {row, tag}
        const unsigned long long mine = (static_cast<unsigned long long>(tag) << 32) | static_cast<uint32_t>(i);
        unsigned long long cur = *word;
        if (static_cast<uint32_t>(cur >> 32) != tag) {
            const unsigned long long prev = atomicCAS(word, cur, mine);
            if (prev == cur) {
                atomicExch(reinterpret_cast<unsigned long long *>(&h.slots[pos]),
                           static_cast<unsigned long long>(fits ? pack16(c) : 0ull));
                return;
            }
            cur = prev;  // claimed meanwhile, by a row of this build
        }
        // The slot's row is of this build (or a chance match of a word that
        // never held this build's table): compare coordinates through the
        // input, since its packed key may not be written yet.  A chance
        // word whose row has this key acts as the key's slot: lower its row
        // and write the packed key it may lack.
        const uint32_t r = static_cast<uint32_t>(cur);
        if (r < static_cast<uint32_t>(n) && same_key(keys[r], c)) {
            atomicMin(word, mine);
            if (fits)
                atomicExch(reinterpret_cast<unsigned long long *>(&h.slots[pos]),
                           static_cast<unsigned long long>(pack16(c)));
            if (r != static_cast<uint32_t>(i)) h.flags[kFlagDuplicate] = flag_of(h.seed, kFlagDuplicate);
            return;
        }
        pos = (pos + 1) & h.mask;
    }
    h.flags[kFlagOverflow] = flag_of(h.seed, kFlagOverflow);
}

// Thread per voxel: claim the cell (or, outside the window, a slot) for row
// i, or lower the row of the one already holding its key.
__global__ void __launch_bounds__(kThreads)
kmap_insert_kernel(const int4 *__restrict__ keys, int32_t n, KmapHash h) {
    // (voxel ranges per XCD as the lookups take them: their cells and rows
    // stay in that XCD's L2)
    const int32_t i = xcd_tile(blockIdx.x, gridDim.x) * kThreads + threadIdx.x;
    if (i >= n) return;
    const int4 c = keys[i];
    const int32_t cell = window_cell(c, h.wlog2);
    if (cell < 0) {
        kmap_hash_insert(keys, n, h, i, c);
        return;
    }
    const uint32_t tag = tag_of(h.seed, static_cast<uint32_t>(cell));
    unsigned long long *word = h.cells + cell;
    const unsigned long long mine = (static_cast<unsigned long long>(tag) << 32) | static_cast<uint32_t>(i);
    unsigned long long cur = *word;  // a stale read only fails the CAS
    for (;;) {
        // A current cell holds this key (one cell per key) unless its tag is
        // a stale word's chance match, whose row names other coordinates.
        const uint32_t r = static_cast<uint32_t>(cur);
        if (static_cast<uint32_t>(cur >> 32) == tag && r < static_cast<uint32_t>(n) && same_key(keys[r], c)) {
            atomicMin(word, mine);
            if (r != static_cast<uint32_t>(i)) h.flags[kFlagDuplicate] = flag_of(h.seed, kFlagDuplicate);
            return;
        }
        const unsigned long long prev = atomicCAS(word, cur, mine);
        if (prev == cur) return;
        cur = prev;  // claimed meanwhile by a row of this build (with this key)
    }
}

// One thread per (voxel, offset): kmap[i*27+o] = first row at coords[i]+d(o).
__global__ void __launch_bounds__(kThreads)
kmap_lookup_kernel(const int4 *__restrict__ coords, int32_t n, KmapHash h, int32_t missing,
                   int32_t *__restrict__ kmap) {
    const int32_t g = xcd_tile(blockIdx.x, gridDim.x) * kThreads + threadIdx.x;
    if (g >= n * 27) return;
    const int32_t i = g / 27;
    kmap[g] = kmap_entry(h, coords, n, i, g - i * 27, missing, kmap_wide(h), kmap_dup(h));
}

// Four map entries per thread (KmapLookup4): each thread's loads in flight
// together (a lookup is a chain of three dependent loads) and one 16-byte
// store.  kmap 16-byte aligned.
__global__ void __launch_bounds__(kThreads)
kmap_lookup4_kernel(const int4 *__restrict__ coords, int32_t n, KmapHash h, int32_t missing,
                    int32_t *__restrict__ kmap) {
    const int32_t u = xcd_tile(blockIdx.x, gridDim.x) * kThreads + threadIdx.x;
    const int32_t count = n * 27;
    if (int64_t(4) * u >= count) return;
    const KmapLookup4 lookup{coords, n, missing, h, kmap_wide(h), kmap_dup(h), kmap};
    lookup(0, u, count);
}

// ---- subdivide ------------------------------------------------------------
// For child slot ch (bits bx,by,bz) and offset o, the neighbour lives in the
// parent at parent-offset kAdjOffset and at child slot kAdjChild
// (sparse_ops.cpp:346-365): coordinate bits+d in {-1,0,1,2} splits into a
// parent step floor((bits+d)/2) and a child bit (bits+d) mod 2.
__device__ __forceinline__ void adjacent(int ch, int o, int *parent_offset, int *child_slot) {
    const int b[3] = {ch >> 2, (ch >> 1) & 1, ch & 1};
    const int d[3] = {o / 9 - 1, (o / 3) % 3 - 1, o % 3 - 1};
    int po = 0, cs = 0;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
        const int v = b[a] + d[a];
        const int step = v < 0 ? -1 : (v > 1 ? 1 : 0);
        po = po * 3 + (step + 1);
        cs = cs * 2 + (v - 2 * step);
    }
    *parent_offset = po;
    *child_slot = cs;
}

__global__ void __launch_bounds__(kThreads)
child_coords_kernel(const int4 *__restrict__ parents, int32_t p, int4 *__restrict__ children) {
    const int32_t r = blockIdx.x * kThreads + threadIdx.x;
    if (r >= p * 8) return;
    const int4 c = parents[r >> 3];
    const int ch = r & 7;
    int4 out;
    out.x = c.x;
    out.y = static_cast<int32_t>(static_cast<uint32_t>(c.y) * 2u + static_cast<uint32_t>(ch >> 2));
    out.z = static_cast<int32_t>(static_cast<uint32_t>(c.z) * 2u +
                                 static_cast<uint32_t>((ch >> 1) & 1));
    out.w = static_cast<int32_t>(static_cast<uint32_t>(c.w) * 2u + static_cast<uint32_t>(ch & 1));
    children[r] = out;
}

// One thread per (child, offset): neighbour = parent_nbr*8 + child slot.
__global__ void __launch_bounds__(kThreads)
child_kmap_kernel(const int32_t *__restrict__ parent_kmap, int32_t p, int32_t *__restrict__ kmap) {
    const int64_t g = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (g >= static_cast<int64_t>(p) * 8 * 27) return;
    const int32_t r = static_cast<int32_t>(g / 27);
    const int32_t o = static_cast<int32_t>(g - static_cast<int64_t>(r) * 27);
    int po, cs;
    adjacent(r & 7, o, &po, &cs);
    const int32_t t = parent_kmap[static_cast<int64_t>(r >> 3) * 27 + po];
    kmap[g] = t >= 0 ? t * 8 + cs : -1;
}

// Four entries per thread (32-bit indexes: 216 p below 2^31): the
// (child slot, offset) -> (parent offset, child slot) table from LDS instead
// of recomputed per entry, the four parent-map loads in flight together, one
// 16-byte store; XCD-contiguous ranges of entries.  kmap 16-byte aligned.
__global__ void __launch_bounds__(kThreads)
child_kmap4_kernel(const int32_t *__restrict__ parent_kmap, int32_t p, int32_t *__restrict__ kmap) {
    __shared__ uint8_t adj[8 * 27];  // parent offset | child slot << 5
    if (threadIdx.x < 8 * 27) {
        int po, cs;
        adjacent(static_cast<int>(threadIdx.x) / 27, static_cast<int>(threadIdx.x) % 27, &po, &cs);
        adj[threadIdx.x] = static_cast<uint8_t>(po | cs << 5);
    }
    __syncthreads();
    const int32_t u = xcd_tile(blockIdx.x, gridDim.x) * kThreads + threadIdx.x;
    const int32_t count = p * 8 * 27;
    if (int64_t(4) * u >= count) return;
    const int32_t g = 4 * u;
    int32_t r = g / 27, o = g - r * 27;
    int32_t e[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        e[k] = -1;
        if (g + k < count) {
            const uint32_t a = adj[(r & 7) * 27 + o];
            const int32_t t = parent_kmap[(r >> 3) * 27 + static_cast<int32_t>(a & 31u)];
            e[k] = t >= 0 ? t * 8 + static_cast<int32_t>(a >> 5) : -1;
        }
        if (++o == 27) o = 0, ++r;
    }
    if (g + 3 < count) {
        *reinterpret_cast<int4 *>(kmap + g) = make_int4(e[0], e[1], e[2], e[3]);
    } else {
#pragma unroll
        for (int k = 0; k < 3; ++k)
            if (g + k < count) kmap[g + k] = e[k];
    }
}

constexpr uint64_t kmap_capacity(int64_t n) {
    uint64_t cap = 256;
    while (cap < static_cast<uint64_t>(n) * 4) cap <<= 1;
    return cap;
}

// log2 of the window extent for n voxels: the largest of 64, 128, 256
// (at most max_log2) whose 8-byte cells take no more bytes than the
// 16-byte hash slots, so the window at most doubles the workspace.
constexpr int32_t window_log2(int64_t n, int32_t max_log2) {
    const uint64_t slot_bytes = kmap_capacity(n) * 16;
    int32_t lg = kWindowMinLog2;
    while (lg < max_log2 && (uint64_t(8) << (3 * (lg + 1))) <= slot_bytes) ++lg;
    return lg;
}

template <class W>
void kmap_layout(W &w, int64_t n, KmapHash *h, int32_t max_log2 = kWindowMaxLog2) {
    const uint64_t cap = kmap_capacity(n);
    const int32_t lg = window_log2(n, max_log2);
    const uint64_t cells = uint64_t(1) << (3 * lg);
    if constexpr (std::is_same_v<W, Carver>) {
        h->cells = w.template take<unsigned long long>(cells);
        h->slots = w.template take<uint4>(cap);
        h->flags = w.template take<int32_t>(64);
        h->mask = static_cast<uint32_t>(cap - 1);
        h->seed = 0;
        h->wlog2 = lg;
    } else {
        w.template take<unsigned long long>(cells);
        w.template take<uint4>(cap);
        w.template take<int32_t>(64);
    }
}

// A new seed for every build in the process (never repeated before 2^32
// builds), so slots of earlier builds read as empty.  Seeds whose flag value
// of some flag word is 0 are skipped (three of 2^32), so a zero-filled
// table never reads as a raised flag.
std::atomic<uint32_t> g_seed_counter{0x3C6EF372u};
uint32_t next_seed() {
    for (;;) {
        const uint32_t s = g_seed_counter.fetch_add(1, std::memory_order_relaxed);
        if (flag_of(s, kFlagDuplicate) != 0 && flag_of(s, kFlagOverflow) != 0 && flag_of(s, kFlagWide) != 0)
            return s;
    }
}

// Exact recount behind a raised flag (subdivide only, which reports it):
// counts[0] = rows whose key the table lost (an exhausted probe sequence),
// counts[1] = rows that are not the first row of their key.
__global__ void __launch_bounds__(kThreads)
kmap_confirm_kernel(const int4 *__restrict__ keys, int32_t n, KmapHash h, uint32_t *__restrict__ counts) {
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const bool wide = h.flags[kFlagWide] == flag_of(h.seed, kFlagWide);
    const int32_t r = kmap_find(h, keys, n, keys[i], wide);
    if (r < 0) atomicAdd(&counts[0], 1u);
    else if (r != i) atomicAdd(&counts[1], 1u);
}

// Insert + lookup (two launches, no clearing pass), leaving the flags of
// this build (h.seed) in the workspace.
void run_kmap(const int4 *coords, int32_t n, int32_t missing, int32_t *kmap, KmapHash &h, hipStream_t stream) {
    h.seed = next_seed();
    kmap_insert_kernel<<<blocks_for(n), kThreads, 0, stream>>>(coords, n, h);
    launch_check("kmap_insert");
    // (four entries a thread pays on large sets: 183 -> 174 us at 1.81M
    // voxels; at 28k voxels one entry a thread is 2% faster)
    if (aligned(kmap, 16) && n > (int32_t(1) << 17))
        kmap_lookup4_kernel<<<blocks_for((static_cast<int64_t>(n) * 27 + 3) / 4), kThreads, 0, stream>>>(
            coords, n, h, missing, kmap);
    else
        kmap_lookup_kernel<<<blocks_for(static_cast<int64_t>(n) * 27), kThreads, 0, stream>>>(coords, n, h, missing,
                                                                                               kmap);
    launch_check("kmap_lookup");
}

// Allocation-free kernel maps: the hash table lives in `scratch`, one array
// per device for the life of the process, sized for kStaticKmapMaxVoxels.
constexpr int64_t kStaticKmapMaxVoxels = int64_t(1) << 18;
// (its window stays 64^3: the array is sized for that layout)
constexpr uint64_t kStaticKmapBytes = (uint64_t(8) << (3 * kWindowMinLog2)) +
                                      (kmap_capacity(kStaticKmapMaxVoxels) * 16 + 255) / 256 * 256 +
                                      (64 * 4 + 255) / 256 * 256;
static __device__ __align__(256) unsigned char scratch[kStaticKmapBytes];

// The device address of `scratch` on the current device, looked up once per
// device (the array's name in host code is only a stand-in).
void *static_scratch() {
    constexpr int kMaxDevices = 64;
    static std::mutex lock;
    static void *addr[kMaxDevices] = {};
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    require(dev >= 0 && dev < kMaxDevices, "device index out of range");
    std::lock_guard<std::mutex> g(lock);
    if (addr[dev] == nullptr) {
        void *p = nullptr;
        hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        addr[dev] = p;
    }
    return addr[dev];
}

void check_coords(const int32_t *coords, int64_t n) {
    require(coords != nullptr, "coords is NULL");
    require(aligned(coords, 16), "coords must be 16-byte aligned");
    require(n > 0, "voxel count must be positive");
    require(n <= INT32_MAX / 27, "voxel count exceeds INT32_MAX / 27");
}

}  // namespace

KmapHash kmap_insert_launch(const int4 *coords, int32_t n, void *workspace, uint64_t workspace_bytes,
                            hipStream_t stream) {
    Carver w(workspace, workspace_bytes);
    KmapHash h;
    kmap_layout(w, n, &h);
    h.seed = next_seed();
    kmap_insert_kernel<<<blocks_for(n), kThreads, 0, stream>>>(coords, n, h);
    launch_check("kmap_insert");
    return h;
}

}  // namespace s3dx

namespace s3dx {
namespace {
struct SubdivideLayout {
    KmapHash hash;
    int32_t *parent_kmap;
};
template <class W>
void subdivide_layout(W &w, int64_t p, SubdivideLayout *l) {
    if constexpr (std::is_same_v<W, Carver>) {
        kmap_layout(w, p, &l->hash);
        l->parent_kmap = w.template take<int32_t>(static_cast<uint64_t>(p) * 27);
    } else {
        kmap_layout(w, p, static_cast<KmapHash *>(nullptr));
        w.template take<int32_t>(static_cast<uint64_t>(p) * 27);
    }
}
}  // namespace
}  // namespace s3dx

using namespace s3dx;

extern "C" {

S3DX_API s3dx_status s3dx_kmap_workspace_size(int64_t n, uint64_t *bytes, char *error,
                                              uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(bytes != nullptr, "bytes is NULL");
        require(n > 0 && n <= INT32_MAX / 27, "voxel count out of range");
        Sizer s;
        kmap_layout(s, n, static_cast<KmapHash *>(nullptr));
        *bytes = s.used;
    });
}

S3DX_API s3dx_status s3dx_kmap_subm3(const int32_t *coords, int64_t n, int32_t missing_value,
                                     int32_t *kmap, void *workspace, uint64_t workspace_bytes,
                                     s3dx_stream stream, char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        check_coords(coords, n);
        require(kmap != nullptr, "kmap is NULL");
        require(workspace != nullptr, "workspace is NULL");
        Carver w(workspace, workspace_bytes);
        KmapHash h;
        kmap_layout(w, n, &h);
        run_kmap(reinterpret_cast<const int4 *>(coords), static_cast<int32_t>(n), missing_value,
                 kmap, h, as_stream(stream));
    });
}

S3DX_API s3dx_status s3dx_kmap_subm3_static(const int32_t *coords, int64_t n, int32_t missing_value,
                                            int32_t *kmap, s3dx_stream stream, char *error,
                                            uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        check_coords(coords, n);
        require(kmap != nullptr, "kmap is NULL");
        require(n <= kStaticKmapMaxVoxels, "voxel count exceeds the static table's maximum (262144)");
        Carver w(static_scratch(), kStaticKmapBytes);
        KmapHash h;
        kmap_layout(w, n, &h, kWindowMinLog2);
        run_kmap(reinterpret_cast<const int4 *>(coords), static_cast<int32_t>(n), missing_value, kmap, h,
                 as_stream(stream));
    });
}

S3DX_API s3dx_status s3dx_subdivide2_workspace_size(int64_t parent_count, uint64_t *bytes,
                                                    char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(bytes != nullptr, "bytes is NULL");
        require(parent_count > 0 && parent_count <= INT32_MAX / 27,
                "parent count out of range");
        Sizer s;
        subdivide_layout(s, parent_count, nullptr);
        *bytes = s.used;
    });
}

S3DX_API s3dx_status s3dx_subdivide2(const int32_t *parent_coords, int64_t parent_count,
                                     int32_t *child_coords, int32_t *child_kmap, void *workspace,
                                     uint64_t workspace_bytes, s3dx_stream stream, char *error,
                                     uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        // sparse_ops.cpp:273 rejects count <= 0 and count > INT32_MAX / 8; the
        // child kmap additionally needs 8 * 27 * count to index in int32.
        require(parent_coords != nullptr, "parent_coords is NULL");
        require(parent_count > 0, "parent count must be positive");
        require(parent_count <= INT32_MAX / 8, "parent count exceeds INT32_MAX / 8");
        require(parent_count <= INT32_MAX / 27, "parent count exceeds INT32_MAX / 27");
        require(child_coords != nullptr, "child_coords is NULL");
        require(aligned(parent_coords, 16) && aligned(child_coords, 16),
                "coordinates must be 16-byte aligned");
        require(workspace != nullptr, "workspace is NULL");
        const hipStream_t s = as_stream(stream);
        const int32_t p = static_cast<int32_t>(parent_count);
        Carver w(workspace, workspace_bytes);
        SubdivideLayout l;
        subdivide_layout(w, parent_count, &l);
        run_kmap(reinterpret_cast<const int4 *>(parent_coords), p, -1, l.parent_kmap, l.hash, s);
        child_coords_kernel<<<blocks_for(static_cast<int64_t>(p) * 8), kThreads, 0, s>>>(
            reinterpret_cast<const int4 *>(parent_coords), p, reinterpret_cast<int4 *>(child_coords));
        launch_check("child_coords");
        if (child_kmap) {
            const int64_t entries = static_cast<int64_t>(p) * 8 * 27;
            if (aligned(child_kmap, 16) && entries < (int64_t(1) << 31) - 4)
                child_kmap4_kernel<<<blocks_for((entries + 3) / 4), kThreads, 0, s>>>(l.parent_kmap, p, child_kmap);
            else
                child_kmap_kernel<<<blocks_for(entries), kThreads, 0, s>>>(l.parent_kmap, p, child_kmap);
            launch_check("child_kmap");
        }
        int32_t flags[2] = {0, 0};
        hip_check(hipMemcpyAsync(flags, l.hash.flags, sizeof(flags), hipMemcpyDeviceToHost, s),
                  "hipMemcpyAsync flags");
        hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
        if (flags[kFlagDuplicate] == flag_of(l.hash.seed, kFlagDuplicate) ||
            flags[kFlagOverflow] == flag_of(l.hash.seed, kFlagOverflow)) {
            // A raised flag word may be a chance value of a workspace that
            // never held this build's table: recount exactly before failing.
            uint32_t *counts = reinterpret_cast<uint32_t *>(l.hash.flags + kConfirmWord);
            hip_check(hipMemsetAsync(counts, 0, 2 * sizeof(uint32_t), s), "hipMemsetAsync counts");
            kmap_confirm_kernel<<<blocks_for(p), kThreads, 0, s>>>(reinterpret_cast<const int4 *>(parent_coords), p,
                                                                   l.hash, counts);
            launch_check("kmap_confirm");
            uint32_t c[2] = {0, 0};
            hip_check(hipMemcpyAsync(c, counts, sizeof(c), hipMemcpyDeviceToHost, s), "hipMemcpyAsync counts");
            hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
            require(c[1] == 0, "duplicate parent coordinates");
            if (c[0] != 0) throw std::runtime_error("hash table overflow");
        }
    });
}

/* Test-only hooks, exported for the test suite and absent from the public
 * header: the seed of the next kernel-map build in this process (so a test
 * can replay a build whose tags collide with a zero-filled table), and a
 * clearing of the allocation-free entry point's static table on the current
 * device (so a test can start it from zeros as a fresh process does). */
S3DX_API s3dx_status s3dx_testing_set_kmap_seed(uint32_t seed, char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] { g_seed_counter.store(seed, std::memory_order_relaxed); });
}

S3DX_API s3dx_status s3dx_testing_zero_static_kmap(s3dx_stream stream, char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        const hipStream_t s = as_stream(stream);
        hip_check(hipMemsetAsync(static_scratch(), 0, kStaticKmapBytes, s), "hipMemsetAsync scratch");
        hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    });
}

}  // extern "C"
