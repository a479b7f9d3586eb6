// Coordinate hash shared by the kernel-map and coordinate-set kernels.
//
// The hash is open addressing with linear probing at load <= 1/8.  A slot is
// one 32-bit row (0xFFFFFFFF = empty); the key of a slot is the row's
// (b, x, y, z) in the input, so a probe reads the slot, then the key it
// names.  The table (4 bytes a slot, 1 MB at 30k voxels) stays resident in
// L2 and clears with one coalesced fill.  A wave waits for its longest probe
// chain, which is what the low load keeps short.  A slot is claimed with a
// 32-bit CAS on the row; a second row with the same coordinates lowers it
// with atomicMin, so after the insert kernel every key maps to its smallest
// row -- exactly std::map::emplace's "first occurrence wins".  Any int32
// coordinates are handled exactly.
#pragma once

#include "common.hpp"

#include <type_traits>

namespace s3dx {
namespace {

constexpr uint32_t kEmpty = 0xFFFFFFFFu;
constexpr int kThreads = 256;

// Workspace flag words.
constexpr int kFlagDuplicate = 0;  // some coordinate occurs twice
constexpr int kFlagOverflow = 1;   // probe sequence exhausted (never at load <= 1/8)

// 32-bit hash of (b, x, y, z): a multiply-add chain over the four words and
// a murmur3-style finalizer (five 32-bit multiplies).
__device__ __forceinline__ uint32_t key_hash(int4 c) {
    uint32_t h = static_cast<uint32_t>(c.x) * 0x9E3779B1u + static_cast<uint32_t>(c.y);
    h = h * 0x85EBCA77u + static_cast<uint32_t>(c.z);
    h = h * 0xC2B2AE3Du + static_cast<uint32_t>(c.w);
    h ^= h >> 16;
    h *= 0x7FEB352Du;
    h ^= h >> 15;
    h *= 0x846CA68Bu;
    h ^= h >> 16;
    return h;
}

__device__ __forceinline__ bool same_key(int4 a, int4 b) {
    return a.x == b.x && a.y == b.y && a.z == b.z && a.w == b.w;
}

// Device view of the table: cap = mask + 1 slots of one row index each
// (kEmpty when free).  A slot's key is keys[row], read from the array the
// table was built from, so the table stays small (4 bytes a slot, load
// <= 1/8) and one coalesced fill clears it.
struct Hash {
    uint32_t *slots;
    const int4 *keys;
    int32_t *flags;
    uint32_t mask;
};

// Smallest inserted row whose key equals c, or -1 (after the insert kernel).
__device__ __forceinline__ int32_t hash_find(const Hash &h, int4 c) {
    uint32_t pos = key_hash(c) & h.mask;
    for (uint32_t probe = 0; probe <= h.mask; ++probe) {
        const uint32_t row = h.slots[pos];
        if (row == kEmpty) return -1;
        if (same_key(h.keys[row], c)) return static_cast<int32_t>(row);
        pos = (pos + 1) & h.mask;
    }
    return -1;
}

// Empties the slots and zeroes the flag words (one launch for both).
__global__ void __launch_bounds__(kThreads) hash_clear_kernel(Hash h) {
    const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i <= h.mask) h.slots[i] = kEmpty;
    if (i < 64) h.flags[i] = 0;
}

__global__ void __launch_bounds__(kThreads)
hash_insert_kernel(const int4 *__restrict__ keys, int32_t n, Hash h) {
    const int32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const int4 c = keys[i];
    uint32_t pos = key_hash(c) & h.mask;
    for (uint32_t probe = 0; probe <= h.mask; ++probe) {
        const uint32_t prev = atomicCAS(&h.slots[pos], kEmpty, static_cast<uint32_t>(i));
        if (prev == kEmpty) return;
        // Rows sharing a key only ever lower the slot's row, so any row seen
        // here carries the slot's key.
        if (same_key(keys[prev], c)) {
            atomicMin(&h.slots[pos], static_cast<uint32_t>(i));
            h.flags[kFlagDuplicate] = 1;
            return;
        }
        pos = (pos + 1) & h.mask;
    }
    h.flags[kFlagOverflow] = 1;
}

__device__ __forceinline__ bool add_fits(int32_t v, int32_t d, int32_t *out) {
    const int64_t s = static_cast<int64_t>(v) + d;
    *out = static_cast<int32_t>(s);
    return s >= INT32_MIN && s <= INT32_MAX;
}

unsigned blocks_for(int64_t items) { return static_cast<unsigned>((items + kThreads - 1) / kThreads); }

// Grid of a bounds reduction: at most 128 blocks, each thread striding over
// the items, so the per-block atomics stay few.
inline unsigned bounds_blocks(int64_t items) { return blocks_for(items) < 128u ? blocks_for(items) : 128u; }

// Block-wide min of v[0..M) and max of v[M..2M), committed with one atomic
// per value per block: a wave butterfly, then the block's waves through LDS.
// Every thread of the block must call it.
template <int M>
__device__ __forceinline__ void block_bounds_atomic(int (&v)[2 * M], int32_t *out) {
    __shared__ int part[kThreads / 64][2 * M];
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
#pragma unroll
        for (int a = 0; a < M; ++a) v[a] = min(v[a], __shfl_xor(v[a], d, 64));
#pragma unroll
        for (int a = M; a < 2 * M; ++a) v[a] = max(v[a], __shfl_xor(v[a], d, 64));
    }
    if ((threadIdx.x & 63) == 0)
#pragma unroll
        for (int a = 0; a < 2 * M; ++a) part[threadIdx.x >> 6][a] = v[a];
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int a = 0; a < 2 * M; ++a) {
            int r = part[0][a];
            for (int w = 1; w < kThreads / 64; ++w) r = a < M ? min(r, part[w][a]) : max(r, part[w][a]);
            if (a < M) atomicMin(&out[a], r);
            else atomicMax(&out[a], r);
        }
    }
}

constexpr uint64_t hash_capacity(int64_t n) {
    uint64_t cap = 256;
    while (cap < static_cast<uint64_t>(n) * 8) cap <<= 1;
    return cap;
}

template <class W>
void hash_layout(W &w, int64_t n, Hash *h) {
    const uint64_t cap = hash_capacity(n);
    if constexpr (std::is_same_v<W, Carver>) {
        h->slots = w.template take<uint32_t>(cap);
        h->keys = nullptr;
        h->flags = w.template take<int32_t>(64);
        h->mask = static_cast<uint32_t>(cap - 1);
    } else {
        w.template take<uint32_t>(cap);
        w.template take<int32_t>(64);
    }
}

// Clears the table and inserts n keys (first occurrence wins).
inline void hash_build(const int4 *keys, int32_t n, Hash &h, hipStream_t stream) {
    h.keys = keys;
    const uint64_t cap = static_cast<uint64_t>(h.mask) + 1;
    hash_clear_kernel<<<blocks_for(static_cast<int64_t>(cap)), kThreads, 0, stream>>>(h);
    launch_check("hash_clear");
    hash_insert_kernel<<<blocks_for(n), kThreads, 0, stream>>>(keys, n, h);
    launch_check("hash_insert");
}

}  // namespace
}  // namespace s3dx
