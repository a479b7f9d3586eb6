// Kernel maps on the GPU: the coordinate hash, the 27-offset submanifold
// neighbour table, the 2x OR-pool (coarse set) and the exact 2x subdivide.
//
// Reference semantics (all host C++ in sam3d.cpp):
//   build_conv            src/objects_runtime/sparse_ops.cpp:117-142
//   SlatTables downsample src/objects_runtime/sparse_ops.cpp:53-104
//   MeshSubdivideTables   src/objects_runtime/sparse_ops.cpp:272-404
//
// The coordinate hash (coord_hash.hpp) gives every key its smallest row, as
// std::map::emplace's "first occurrence wins" does.
#include "coord_hash.hpp"

#include <atomic>
#include <mutex>
#include <vector>

namespace s3dx {
namespace {

// ---- the kernel-map table ----------------------------------------------------
// Two structures, chosen per coordinate:
//  - a direct-index window of 64^3 cells for batch 0 and x, y, z in [0, 64)
//    (the SLat grids: 64^3 fine, 32^3 coarse), one 64-bit word {row, tag} per
//    cell: a lookup is one 8-byte read, an insert a read and a CAS;
//  - for every other coordinate, open addressing with linear probing at load
//    <= 1/4 over 16-byte slots {key lo, key hi, row, tag}.  The key is
//    (b, x, y, z) packed as four int16 when the coordinate fits (a set with
//    any other coordinate raises the "wide" flag and its slots are matched
//    through the input rows instead).
// The {row, tag} word is claimed with one 64-bit CAS; a second row with the
// same coordinates lowers it with a 64-bit atomicMin, so every key keeps its
// smallest row -- std::map::emplace's "first occurrence wins"
// (sparse_ops.cpp:124-127).
//
// A cell or slot belongs to the current build only when its tag equals
// tag_of(seed, index), and every build draws a new seed: tag_of is a
// bijection of seed ^ f(index), so nothing written by another build carries
// the current tag, and the table needs no clearing pass between builds.
// Memory that never held the table (a fresh workspace) reads as empty except
// with probability 2^-32 per word; such a hash slot must still match the
// packed 64-bit key (or, wide, the input row's coordinates) before a lookup
// returns its row, and a window cell's row is checked against the input
// rows' coordinates on insert.
constexpr int kWindow = 64;                                 // cells per axis
constexpr int64_t kWindowCells = int64_t(kWindow) * kWindow * kWindow;

struct KmapHash {
    unsigned long long *cells;  // kWindowCells words {row, tag}
    uint4 *slots;               // mask + 1 slots
    int32_t *flags;             // [kFlag*] == flag_of(seed, k) when raised in this build
    uint32_t mask;
    uint32_t seed;
};

constexpr int kFlagWide = 2;  // some hashed coordinate does not fit int16

__device__ __host__ __forceinline__ uint32_t mix32(uint32_t h) {
    h ^= h >> 16;
    h *= 0x7FEB352Du;
    h ^= h >> 15;
    h *= 0x846CA68Bu;
    h ^= h >> 16;
    return h;
}
__device__ __forceinline__ uint32_t tag_of(uint32_t seed, uint32_t index) {
    return mix32(seed ^ (index * 0x9E3779B1u));
}
__device__ __host__ __forceinline__ int32_t flag_of(uint32_t seed, int k) {
    return static_cast<int32_t>(mix32(seed + 0x632BE5ABu * static_cast<uint32_t>(k + 1)));
}

// The window cell of c, or -1.
__device__ __forceinline__ int32_t window_cell(int4 c) {
    const uint32_t x = static_cast<uint32_t>(c.y), y = static_cast<uint32_t>(c.z), z = static_cast<uint32_t>(c.w);
    if (c.x != 0 || (x | y | z) >= static_cast<uint32_t>(kWindow)) return -1;
    return static_cast<int32_t>((x * kWindow + y) * kWindow + z);
}

__device__ __forceinline__ bool fits16(int4 c) {
    auto f = [](int32_t v) { return v >= -32768 && v <= 32767; };
    return f(c.x) && f(c.y) && f(c.z) && f(c.w);
}
__device__ __forceinline__ uint64_t pack16(int4 c) {
    return (static_cast<uint64_t>(static_cast<uint16_t>(c.x)) << 48) |
           (static_cast<uint64_t>(static_cast<uint16_t>(c.y)) << 32) |
           (static_cast<uint64_t>(static_cast<uint16_t>(c.z)) << 16) | static_cast<uint64_t>(static_cast<uint16_t>(c.w));
}

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
        // The slot's row is of this build (or a stale word's chance match,
        // whose row fails the comparison): compare coordinates through the
        // input, since its packed key may not be written yet.
        const uint32_t r = static_cast<uint32_t>(cur);
        if (r < static_cast<uint32_t>(n) && same_key(keys[r], c)) {
            atomicMin(word, mine);
            h.flags[kFlagDuplicate] = flag_of(h.seed, kFlagDuplicate);
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
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const int4 c = keys[i];
    const int32_t cell = window_cell(c);
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
            h.flags[kFlagDuplicate] = flag_of(h.seed, kFlagDuplicate);
            return;
        }
        const unsigned long long prev = atomicCAS(word, cur, mine);
        if (prev == cur) return;
        cur = prev;  // claimed meanwhile by a row of this build (with this key)
    }
}

// Hash path of kmap_find (coordinates outside the window).
__device__ __forceinline__ int32_t kmap_hash_find(const KmapHash &h, const int4 *__restrict__ keys, int32_t n, int4 q,
                                          bool wide) {
    if (!wide && !fits16(q)) return -1;
    const uint64_t kq = pack16(q);
    uint32_t pos = key_hash(q) & h.mask;
    for (uint32_t probe = 0; probe <= h.mask; ++probe) {
        const uint4 s = h.slots[pos];
        if (s.w != tag_of(h.seed, pos)) return -1;
        const bool hit = wide ? s.z < static_cast<uint32_t>(n) && same_key(keys[s.z], q)
                              : ((static_cast<uint64_t>(s.y) << 32) | s.x) == kq;
        if (hit) return static_cast<int32_t>(s.z);
        pos = (pos + 1) & h.mask;
    }
    return -1;
}

// Smallest row whose key equals q, or -1 (after kmap_insert_kernel).
__device__ __forceinline__ int32_t kmap_find(const KmapHash &h, const int4 *__restrict__ keys, int32_t n, int4 q,
                                             bool wide) {
    const int32_t cell = window_cell(q);
    if (cell < 0) return kmap_hash_find(h, keys, n, q, wide);
    const unsigned long long v = h.cells[cell];
    return static_cast<uint32_t>(v >> 32) == tag_of(h.seed, static_cast<uint32_t>(cell))
               ? static_cast<int32_t>(static_cast<uint32_t>(v))
               : -1;
}

// One thread per (voxel, offset): kmap[i*27+o] = first row at coords[i]+d(o).
__global__ void __launch_bounds__(kThreads)
kmap_lookup_kernel(const int4 *__restrict__ coords, int32_t n, KmapHash h, int32_t missing,
                   int32_t *__restrict__ kmap) {
    const int32_t g = blockIdx.x * kThreads + threadIdx.x;
    if (g >= n * 27) return;
    const int32_t i = g / 27;
    const int32_t o = g - i * 27;
    const int4 c = coords[i];
    const bool wide = h.flags[kFlagWide] == flag_of(h.seed, kFlagWide);
    const bool dup = h.flags[kFlagDuplicate] == flag_of(h.seed, kFlagDuplicate);
    int32_t result = missing;
    // Later duplicates of a coordinate keep an all-missing row
    // (sparse_ops.cpp:129-139 only visits each key's first row).
    const bool owner = !dup || kmap_find(h, coords, n, c, wide) == i;
    int4 q = c;
    if (owner && add_fits(c.y, o / 9 - 1, &q.y) && add_fits(c.z, (o / 3) % 3 - 1, &q.z) &&
        add_fits(c.w, o % 3 - 1, &q.w)) {
        const int32_t r = kmap_find(h, coords, n, q, wide);
        if (r >= 0) result = r;
    }
    kmap[g] = result;
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

// ---- coarsen ---------------------------------------------------------------
__global__ void __launch_bounds__(kThreads)
coarse_keys_kernel(const int4 *__restrict__ coords, int32_t n, int4 *__restrict__ ckeys,
                   int32_t *bbox) {
    int v[8] = {INT32_MAX, INT32_MAX, INT32_MAX, INT32_MAX, INT32_MIN, INT32_MIN, INT32_MIN, INT32_MIN};
    for (int32_t i = blockIdx.x * kThreads + threadIdx.x; i < n; i += gridDim.x * kThreads) {
        const int4 c = coords[i];
        // C++ integer division truncates toward zero (sparse_ops.cpp:63-64).
        const int4 k = make_int4(c.x, c.y / 2, c.z / 2, c.w / 2);
        ckeys[i] = k;
        v[0] = min(v[0], k.x); v[1] = min(v[1], k.y); v[2] = min(v[2], k.z); v[3] = min(v[3], k.w);
        v[4] = max(v[4], k.x); v[5] = max(v[5], k.y); v[6] = max(v[6], k.z); v[7] = max(v[7], k.w);
    }
    block_bounds_atomic<4>(v, bbox);
}

struct DenseGrid {
    int32_t lo[4];
    int64_t ext[4];
};

__device__ __forceinline__ int64_t dense_cell(const DenseGrid &g, int4 k) {
    return ((static_cast<int64_t>(k.x) - g.lo[0]) * g.ext[1] + (static_cast<int64_t>(k.y) - g.lo[1])) *
               g.ext[2] * g.ext[3] +
           (static_cast<int64_t>(k.z) - g.lo[2]) * g.ext[3] + (static_cast<int64_t>(k.w) - g.lo[3]);
}

// Dense path: every occupied coarse cell is marked; the exclusive scan over
// the row-major (b, x, y, z) cell index is then the lexicographic rank.
__global__ void __launch_bounds__(kThreads)
dense_mark_kernel(const int4 *__restrict__ ckeys, int32_t n, DenseGrid g, int32_t *mark) {
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i < n) mark[dense_cell(g, ckeys[i])] = 1;
}

__global__ void __launch_bounds__(kThreads)
dense_assign_kernel(const int4 *__restrict__ ckeys, int32_t n, DenseGrid g,
                    const int32_t *__restrict__ rank, int32_t *__restrict__ f2c,
                    int4 *__restrict__ coarse_coords) {
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const int4 k = ckeys[i];
    const int32_t r = rank[dense_cell(g, k)];
    f2c[i] = r;
    coarse_coords[r] = k;  // every writer of row r stores the same key
}

// General path (bounding box too large for a dense grid): representatives
// (the smallest fine row of each coarse key) are ranked by counting smaller
// keys, O(nc^2) comparisons tiled through LDS.
__global__ void __launch_bounds__(kThreads)
rep_flag_kernel(const int4 *__restrict__ ckeys, int32_t n, Hash h, int32_t *__restrict__ rep,
                int32_t *__restrict__ is_rep) {
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const int32_t r = hash_find(h, ckeys[i]);
    rep[i] = r;
    is_rep[i] = r == i ? 1 : 0;
}

__global__ void __launch_bounds__(kThreads)
rep_compact_kernel(const int32_t *__restrict__ is_rep, const int32_t *__restrict__ pos, int32_t n,
                   int32_t *__restrict__ reps) {
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i < n && is_rep[i]) reps[pos[i]] = i;
}

__device__ __forceinline__ bool key_less(int4 a, int4 b) {
    if (a.x != b.x) return a.x < b.x;
    if (a.y != b.y) return a.y < b.y;
    if (a.z != b.z) return a.z < b.z;
    return a.w < b.w;
}

__global__ void __launch_bounds__(kThreads)
rank_count_kernel(const int4 *__restrict__ ckeys, const int32_t *__restrict__ reps, int32_t nc,
                  int32_t *__restrict__ rank_of) {
    __shared__ int4 tile[kThreads];
    const int32_t u = blockIdx.x * kThreads + threadIdx.x;
    const int4 mine = u < nc ? ckeys[reps[u]] : make_int4(0, 0, 0, 0);
    int32_t rank = 0;
    for (int32_t t0 = 0; t0 < nc; t0 += kThreads) {
        const int32_t v = t0 + threadIdx.x;
        __syncthreads();
        if (v < nc) tile[threadIdx.x] = ckeys[reps[v]];
        __syncthreads();
        const int32_t m = min(kThreads, nc - t0);
        for (int32_t j = 0; j < m; ++j) rank += key_less(tile[j], mine) ? 1 : 0;
    }
    if (u < nc) rank_of[u] = rank;
}

__global__ void __launch_bounds__(kThreads)
general_assign_kernel(const int4 *__restrict__ ckeys, int32_t n, const int32_t *__restrict__ rep,
                      const int32_t *__restrict__ pos, const int32_t *__restrict__ rank_of,
                      int32_t *__restrict__ f2c, int4 *__restrict__ coarse_coords) {
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const int32_t r = rank_of[pos[rep[i]]];
    f2c[i] = r;
    if (rep[i] == i) coarse_coords[r] = ckeys[i];
}

// Children lists: counts -> offsets -> bucketed fine rows -> the 8 smallest
// per coarse row in ascending order (sparse_ops.cpp:82-104).
__global__ void __launch_bounds__(kThreads)
child_count_kernel(const int32_t *__restrict__ f2c, int32_t n, int32_t *counts) {
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i < n) atomicAdd(&counts[f2c[i]], 1);
}

__global__ void __launch_bounds__(kThreads)
child_bucket_kernel(const int32_t *__restrict__ f2c, int32_t n, const int32_t *__restrict__ start,
                    int32_t *fill, int32_t *__restrict__ bucket) {
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const int32_t c = f2c[i];
    bucket[start[c] + atomicAdd(&fill[c], 1)] = i;
}

__global__ void __launch_bounds__(kThreads)
child_select_kernel(const int32_t *__restrict__ bucket, const int32_t *__restrict__ start,
                    const int32_t *__restrict__ counts, int32_t nc, int32_t n,
                    int32_t *__restrict__ children, float *__restrict__ inv_count) {
    const int32_t c = blockIdx.x * kThreads + threadIdx.x;
    if (c >= nc) return;
    const int32_t s = start[c], k = counts[c];
    int32_t prev = -1;
    for (int j = 0; j < 8; ++j) {
        // j-th smallest: the smallest entry greater than the previous pick
        // (entries are distinct fine rows).
        int32_t best = INT32_MAX;
        for (int32_t t = 0; t < k; ++t) {
            const int32_t v = bucket[s + t];
            if (v > prev && v < best) best = v;
        }
        const bool have = j < k;
        children[static_cast<int64_t>(c) * 8 + j] = have ? best : n;
        if (have) prev = best;
    }
    inv_count[c] = 1.0f / static_cast<float>(k + 1);
}

// Dense coarse grids up to this many cells use the scan path.
uint64_t dense_cell_cap(int64_t n) {
    const uint64_t a = uint64_t(1) << 21;
    const uint64_t b = static_cast<uint64_t>(n) * 64;
    return a > b ? a : b;
}

constexpr uint64_t kmap_capacity(int64_t n) {
    uint64_t cap = 256;
    while (cap < static_cast<uint64_t>(n) * 4) cap <<= 1;
    return cap;
}

template <class W>
void kmap_layout(W &w, int64_t n, KmapHash *h) {
    const uint64_t cap = kmap_capacity(n);
    if constexpr (std::is_same_v<W, Carver>) {
        h->cells = w.template take<unsigned long long>(kWindowCells);
        h->slots = w.template take<uint4>(cap);
        h->flags = w.template take<int32_t>(64);
        h->mask = static_cast<uint32_t>(cap - 1);
        h->seed = 0;
    } else {
        w.template take<unsigned long long>(kWindowCells);
        w.template take<uint4>(cap);
        w.template take<int32_t>(64);
    }
}

// A new seed for every build in the process (never repeated before 2^32
// builds), so slots of earlier builds read as empty.
uint32_t next_seed() {
    static std::atomic<uint32_t> counter{0x3C6EF372u};
    return counter.fetch_add(1, std::memory_order_relaxed);
}

// Insert + lookup (two launches, no clearing pass), leaving the flags of
// this build (h.seed) in the workspace.
void run_kmap(const int4 *coords, int32_t n, int32_t missing, int32_t *kmap, KmapHash &h, hipStream_t stream) {
    h.seed = next_seed();
    kmap_insert_kernel<<<blocks_for(n), kThreads, 0, stream>>>(coords, n, h);
    launch_check("kmap_insert");
    kmap_lookup_kernel<<<blocks_for(static_cast<int64_t>(n) * 27), kThreads, 0, stream>>>(coords, n, h, missing,
                                                                                           kmap);
    launch_check("kmap_lookup");
}

// Allocation-free kernel maps: the hash table lives in `scratch`, one array
// per device for the life of the process, sized for kStaticKmapMaxVoxels.
constexpr int64_t kStaticKmapMaxVoxels = int64_t(1) << 18;
constexpr uint64_t kStaticKmapBytes = kWindowCells * 8 + (kmap_capacity(kStaticKmapMaxVoxels) * 16 + 255) / 256 * 256 +
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
namespace {
struct CoarsenLayout {
    int4 *ckeys;
    Hash hash;
    int32_t *bbox;
    int32_t *totals;
    int32_t *a, *b, *c, *d;  // n-sized scratch
    int32_t *counts, *start, *fill, *bucket;
    int32_t *dense_mark, *dense_rank;
    void *scan_ws;
};
template <class W>
void coarsen_layout(W &w, int64_t n, CoarsenLayout *l) {
    const uint64_t un = static_cast<uint64_t>(n);
    const uint64_t cells = dense_cell_cap(n);
    const uint64_t scan_items = cells > un ? cells : un;
    if constexpr (std::is_same_v<W, Carver>) {
        l->ckeys = w.template take<int4>(un);
        hash_layout(w, n, &l->hash);
        l->bbox = w.template take<int32_t>(8);
        l->totals = w.template take<int32_t>(8);
        l->a = w.template take<int32_t>(un);
        l->b = w.template take<int32_t>(un);
        l->c = w.template take<int32_t>(un);
        l->d = w.template take<int32_t>(un);
        l->counts = w.template take<int32_t>(un);
        l->start = w.template take<int32_t>(un);
        l->fill = w.template take<int32_t>(un);
        l->bucket = w.template take<int32_t>(un);
        l->dense_mark = w.template take<int32_t>(cells);
        l->dense_rank = w.template take<int32_t>(cells);
        l->scan_ws = w.template take<char>(scan_workspace_bytes(static_cast<int64_t>(scan_items)));
    } else {
        w.template take<int4>(un);
        hash_layout(w, n, static_cast<Hash *>(nullptr));
        w.template take<int32_t>(8);
        w.template take<int32_t>(8);
        for (int k = 0; k < 8; ++k) w.template take<int32_t>(un);
        w.template take<int32_t>(cells);
        w.template take<int32_t>(cells);
        w.template take<char>(scan_workspace_bytes(static_cast<int64_t>(scan_items)));
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
        kmap_layout(w, n, &h);
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
            child_kmap_kernel<<<blocks_for(static_cast<int64_t>(p) * 8 * 27), kThreads, 0, s>>>(
                l.parent_kmap, p, child_kmap);
            launch_check("child_kmap");
        }
        int32_t flags[2] = {0, 0};
        hip_check(hipMemcpyAsync(flags, l.hash.flags, sizeof(flags), hipMemcpyDeviceToHost, s),
                  "hipMemcpyAsync flags");
        hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
        require(flags[kFlagDuplicate] != flag_of(l.hash.seed, kFlagDuplicate), "duplicate parent coordinates");
        if (flags[kFlagOverflow] == flag_of(l.hash.seed, kFlagOverflow))
            throw std::runtime_error("hash table overflow");
    });
}


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
        check_coords(coords, n);
        require(coarse_coords && fine_to_coarse && coarse_children && coarse_inv_count && nc_out,
                "NULL output");
        require(aligned(coarse_coords, 16), "coarse_coords must be 16-byte aligned");
        require(workspace != nullptr, "workspace is NULL");
        const hipStream_t s = as_stream(stream);
        const int32_t ni = static_cast<int32_t>(n);
        Carver w(workspace, workspace_bytes);
        CoarsenLayout l;
        coarsen_layout(w, n, &l);
        const int4 *c4 = reinterpret_cast<const int4 *>(coords);
        int4 *cc4 = reinterpret_cast<int4 *>(coarse_coords);

        // 1. coarse keys + their bounding box.
        fill_u32(reinterpret_cast<uint32_t *>(l.bbox), 4, static_cast<uint32_t>(INT32_MAX), s);
        fill_u32(reinterpret_cast<uint32_t *>(l.bbox) + 4, 4, static_cast<uint32_t>(INT32_MIN), s);
        coarse_keys_kernel<<<bounds_blocks(ni), kThreads, 0, s>>>(c4, ni, l.ckeys, l.bbox);
        launch_check("coarse_keys");
        int32_t bbox[8];
        hip_check(hipMemcpyAsync(bbox, l.bbox, sizeof(bbox), hipMemcpyDeviceToHost, s),
                  "hipMemcpyAsync bbox");
        hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");

        DenseGrid g;
        bool dense = true;
        uint64_t cells = 1;
        for (int a = 0; a < 4; ++a) {
            g.lo[a] = bbox[a];
            g.ext[a] = static_cast<int64_t>(bbox[4 + a]) - bbox[a] + 1;
            const uint64_t e = static_cast<uint64_t>(g.ext[a]);
            if (cells > dense_cell_cap(n) / e) dense = false;
            else cells *= e;
        }
        dense = dense && cells <= dense_cell_cap(n);

        int32_t nc = 0;
        if (dense) {
            // 2a. mark occupied cells, scan -> lexicographic rank.
            fill_u32(reinterpret_cast<uint32_t *>(l.dense_mark), cells, 0, s);
            dense_mark_kernel<<<blocks_for(ni), kThreads, 0, s>>>(l.ckeys, ni, g, l.dense_mark);
            launch_check("dense_mark");
            exclusive_scan_i32(l.dense_mark, l.dense_rank, static_cast<int64_t>(cells), l.totals,
                               l.scan_ws, s);
            dense_assign_kernel<<<blocks_for(ni), kThreads, 0, s>>>(l.ckeys, ni, g, l.dense_rank,
                                                                    fine_to_coarse, cc4);
            launch_check("dense_assign");
        } else {
            // 2b. dedupe through the hash, rank representatives by counting.
            hash_build(l.ckeys, ni, l.hash, s);
            int32_t *rep = l.a, *is_rep = l.b, *pos = l.c, *rank_of = l.d;
            rep_flag_kernel<<<blocks_for(ni), kThreads, 0, s>>>(l.ckeys, ni, l.hash, rep, is_rep);
            launch_check("rep_flag");
            exclusive_scan_i32(is_rep, pos, ni, l.totals, l.scan_ws, s);
            int32_t *reps = l.bucket;  // free until the children pass
            rep_compact_kernel<<<blocks_for(ni), kThreads, 0, s>>>(is_rep, pos, ni, reps);
            launch_check("rep_compact");
            hip_check(hipMemcpyAsync(&nc, l.totals, sizeof(nc), hipMemcpyDeviceToHost, s),
                      "hipMemcpyAsync nc");
            hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
            rank_count_kernel<<<blocks_for(nc), kThreads, 0, s>>>(l.ckeys, reps, nc, rank_of);
            launch_check("rank_count");
            general_assign_kernel<<<blocks_for(ni), kThreads, 0, s>>>(l.ckeys, ni, rep, pos, rank_of,
                                                                      fine_to_coarse, cc4);
            launch_check("general_assign");
        }
        hip_check(hipMemcpyAsync(&nc, l.totals, sizeof(nc), hipMemcpyDeviceToHost, s),
                  "hipMemcpyAsync nc");
        hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
        require(nc > 0 && nc <= ni, "coarse row count out of range");

        // 3. children (8 smallest fine rows per coarse row) and 1/(count+1).
        fill_u32(reinterpret_cast<uint32_t *>(l.counts), static_cast<uint64_t>(nc), 0, s);
        fill_u32(reinterpret_cast<uint32_t *>(l.fill), static_cast<uint64_t>(nc), 0, s);
        child_count_kernel<<<blocks_for(ni), kThreads, 0, s>>>(fine_to_coarse, ni, l.counts);
        launch_check("child_count");
        exclusive_scan_i32(l.counts, l.start, nc, l.totals + 1, l.scan_ws, s);
        child_bucket_kernel<<<blocks_for(ni), kThreads, 0, s>>>(fine_to_coarse, ni, l.start, l.fill,
                                                                l.bucket);
        launch_check("child_bucket");
        child_select_kernel<<<blocks_for(nc), kThreads, 0, s>>>(l.bucket, l.start, l.counts, nc, ni,
                                                                coarse_children, coarse_inv_count);
        launch_check("child_select");
        *nc_out = nc;
    });
}

}  // extern "C"
