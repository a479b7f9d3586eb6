// The kernel-map table shared by the map's kernels (kmap.hip) and the
// one-pass map + gather-plan kernel (conv_halo.hip): its layout, tags and
// lookups.  The insert kernel and the host side are in kmap.hip.
#pragma once

#include "coord_hash.hpp"

namespace s3dx {

struct KmapHash {
    unsigned long long *cells;  // 2^(3 * wlog2) words {row, tag}
    uint4 *slots;               // mask + 1 slots
    int32_t *flags;             // [kFlag*] == flag_of(seed, k) when raised in this build
    uint32_t mask;
    uint32_t seed;
    int32_t wlog2;              // window extent 2^wlog2 cells per axis
};

// Lays out `workspace` for n voxels, draws a new seed and launches the
// insert; the returned table is ready for kmap_find once the launch has run
// (kmap.hip).
KmapHash kmap_insert_launch(const int4 *coords, int32_t n, void *workspace, uint64_t workspace_bytes,
                            hipStream_t stream);

namespace {

// ---- the kernel-map table ----------------------------------------------------
// Two structures, chosen per coordinate:
//  - a direct-index window of E^3 cells for batch 0 and x, y, z in [0, E),
//    one 64-bit word {row, tag} per cell: a lookup is one 8-byte read, an
//    insert a read and a CAS.  E is 64 (the SLat grids: 64^3 fine, 32^3
//    coarse, the mesh decoder's 64^3 parents), or 128 / 256 when the set is
//    large enough that the window takes no more bytes than the hash slots
//    (the mesh decoder's 128^3 and 256^3 child sets: 226k and 1.81M voxels);
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
// Memory that never held the table (a zero-filled or fresh workspace) can
// carry the current tag by chance: mix32(0) == 0, so for every seed exactly
// one index of a zero-filled table does, and random bytes do at 2^-32 per
// word.  So no row is ever taken on its tag alone: the insert and the
// lookup both return (or keep) a word's row r only when r < n and the input
// row r has the queried coordinates.  A chance word whose row names other
// coordinates reads as a foreign word (the insert claims it, the lookup
// moves on or reports a miss); one whose row has the queried coordinates is
// a row of that key, and the insert's atomicMin still leaves the key's
// smallest row.  The maps are therefore exact whatever the table holds on
// entry; the flag words alone are taken on their value, and a raised flag
// that decides an error (subdivide's duplicate test) is confirmed by an
// exact pass before it is reported.
constexpr int kWindowMinLog2 = 6;  // 64 cells per axis
constexpr int kWindowMaxLog2 = 8;  // 256 cells per axis


constexpr int kFlagWide = 2;     // some hashed coordinate does not fit int16
constexpr int kConfirmWord = 8;  // two counters of the exact recount behind a raised flag

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

// The window cell of c (x-major, z fastest), or -1.
__device__ __forceinline__ int32_t window_cell(int4 c, int32_t wlog2) {
    const uint32_t x = static_cast<uint32_t>(c.y), y = static_cast<uint32_t>(c.z), z = static_cast<uint32_t>(c.w);
    if (c.x != 0 || (x | y | z) >= (1u << wlog2)) return -1;
    return static_cast<int32_t>((((x << wlog2) | y) << wlog2) | z);
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

// Hash path of kmap_find (coordinates outside the window).
__device__ __forceinline__ int32_t kmap_hash_find(const KmapHash &h, const int4 *__restrict__ keys, int32_t n, int4 q,
                                          bool wide) {
    if (!wide && !fits16(q)) return -1;
    const uint64_t kq = pack16(q);
    uint32_t pos = key_hash(q) & h.mask;
    for (uint32_t probe = 0; probe <= h.mask; ++probe) {
        const uint4 s = h.slots[pos];
        if (s.w != tag_of(h.seed, pos)) return -1;
        // The packed key (when every key fits) screens the probe chain; the
        // row is returned only after its input coordinates match.
        if ((wide || ((static_cast<uint64_t>(s.y) << 32) | s.x) == kq) && s.z < static_cast<uint32_t>(n) &&
            same_key(keys[s.z], q))
            return static_cast<int32_t>(s.z);
        pos = (pos + 1) & h.mask;
    }
    return -1;
}

// Smallest row whose key equals q, or -1 (after kmap_insert_kernel).
__device__ __forceinline__ int32_t kmap_find(const KmapHash &h, const int4 *__restrict__ keys, int32_t n, int4 q,
                                             bool wide) {
    const int32_t cell = window_cell(q, h.wlog2);
    if (cell < 0) return kmap_hash_find(h, keys, n, q, wide);
    const unsigned long long v = h.cells[cell];
    const uint32_t r = static_cast<uint32_t>(v);
    return static_cast<uint32_t>(v >> 32) == tag_of(h.seed, static_cast<uint32_t>(cell)) &&
                   r < static_cast<uint32_t>(n) && same_key(keys[r], q)
               ? static_cast<int32_t>(r)
               : -1;
}


// Map entry (i, o): the first row at coords[i] + delta(o), or `missing`; a
// later duplicate of a coordinate keeps an all-missing row
// (sparse_ops.cpp:129-139 only visits each key's first row).
__device__ __forceinline__ int32_t kmap_entry(const KmapHash &h, const int4 *__restrict__ coords, int32_t n, int32_t i,
                                              int32_t o, int32_t missing, bool wide, bool dup) {
    const int4 c = coords[i];
    const bool owner = !dup || kmap_find(h, coords, n, c, wide) == i;
    int4 q = c;
    if (owner && add_fits(c.y, o / 9 - 1, &q.y) && add_fits(c.z, (o / 3) % 3 - 1, &q.z) &&
        add_fits(c.w, o % 3 - 1, &q.w)) {
        const int32_t r = kmap_find(h, coords, n, q, wide);
        if (r >= 0) return r;
    }
    return missing;
}
__device__ __forceinline__ bool kmap_wide(const KmapHash &h) { return h.flags[kFlagWide] == flag_of(h.seed, kFlagWide); }
__device__ __forceinline__ bool kmap_dup(const KmapHash &h) {
    return h.flags[kFlagDuplicate] == flag_of(h.seed, kFlagDuplicate);
}

// Entries 4u .. 4u+3 of the map slice from row m0 (count entries in all):
// the four entries' loads go out together, step by step (coordinates,
// window cells, then the rows' coordinates that confirm them), and the
// entries are stored (one 16-byte store when all four exist).  An entry
// outside the window, or any entry when the set holds duplicates, takes the
// general kmap_entry.  `kmap` is 16-byte aligned; m0 * 27 is a multiple of 4.
struct KmapLookup4 {
    static constexpr int kOffsets = 27;  // map entries per voxel
    const int4 *coords;
    int32_t n, missing;
    KmapHash h;
    bool wide, dup;
    int32_t *kmap;
    __device__ __forceinline__ int4 operator()(int64_t m0, int u, int count) const {
        // The four entries' loads go out together, step by step (coordinates,
        // window cells, then the rows' coordinates that confirm them); an
        // entry outside the window, or any entry when the set holds
        // duplicates, takes the general kmap_entry instead.
        int e[4], i[4], o[4], cell[4];
        int4 c[4];
        const int64_t g0 = m0 * kOffsets + 4 * u;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int64_t g = g0 + k;
            i[k] = static_cast<int32_t>(g / kOffsets);
            o[k] = static_cast<int32_t>(g - int64_t(i[k]) * kOffsets);
        }
        // Every load of a stage is unconditional (an index that is not
        // needed reads row 0 or window cell 0, both always present: a tile
        // has rows and the window at least 2^18 cells) and its value is
        // selected afterwards: a load under a condition compiles to a branch,
        // and the compiler waits for each such load at its join, one round
        // trip per entry.
#pragma unroll
        for (int k = 0; k < 4; ++k) c[k] = coords[min(i[k], n - 1)];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (4 * u + k >= count) c[k] = make_int4(-1, 0, 0, 0);
        unsigned long long v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            int4 q = c[k];
            cell[k] = -1;
            if (add_fits(c[k].y, o[k] / 9 - 1, &q.y) && add_fits(c[k].z, (o[k] / 3) % 3 - 1, &q.z) &&
                add_fits(c[k].w, o[k] % 3 - 1, &q.w))
                cell[k] = window_cell(q, h.wlog2);
            c[k] = q;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = h.cells[cell[k] >= 0 ? cell[k] : 0];
        int4 rc[4];
        uint32_t r[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            r[k] = static_cast<uint32_t>(v[k]);
            const bool tagged = cell[k] >= 0 && static_cast<uint32_t>(v[k] >> 32) ==
                                                    tag_of(h.seed, static_cast<uint32_t>(cell[k]));
            if (!tagged || r[k] >= static_cast<uint32_t>(n)) r[k] = 0xFFFFFFFFu;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) rc[k] = coords[r[k] != 0xFFFFFFFFu ? r[k] : 0u];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (4 * u + k >= count) {
                e[k] = -1;
            } else if (dup || cell[k] < 0) {
                e[k] = kmap_entry(h, coords, n, i[k], o[k], missing, wide, dup);
            } else {
                e[k] = r[k] != 0xFFFFFFFFu && same_key(rc[k], c[k]) ? static_cast<int32_t>(r[k]) : missing;
            }
        }
        if (4 * u + 3 < count) {
            *reinterpret_cast<int4 *>(kmap + g0) = make_int4(e[0], e[1], e[2], e[3]);
        } else {
#pragma unroll
            for (int k = 0; k < 3; ++k)
                if (4 * u + k < count) kmap[g0 + k] = e[k];
        }
        return make_int4(e[0], e[1], e[2], e[3]);
    }
};

}  // namespace
}  // namespace s3dx
