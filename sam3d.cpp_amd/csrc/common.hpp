// Shared internals of libs3dx_sparse: the ABI error boundary, HIP error
// checks, bfloat16 conversions and small device utilities.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <limits>
#include <new>
#include <stdexcept>
#include <string>

#include "s3dx_sparse.h"

namespace s3dx {

// ---------------------------------------------------------------------------
// ABI boundary: exceptions never cross the C ABI.  Same contract as the
// reference's s3d::boundary (src/error.hpp:15-22).
// ---------------------------------------------------------------------------
struct hip_error : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct oom_error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

inline void message(char *error, uint64_t capacity, const char *text) noexcept {
    if (!error || !capacity) return;
    const uint64_t n = std::min<uint64_t>(capacity - 1, std::strlen(text));
    std::memcpy(error, text, static_cast<size_t>(n));
    error[n] = '\0';
}

template <class F>
s3dx_status boundary(char *error, uint64_t capacity, F &&body) noexcept {
    if (!error && capacity) return S3DX_INVALID_ARGUMENT;
    try {
        body();
        message(error, capacity, "");
        return S3DX_OK;
    } catch (const std::invalid_argument &e) {
        message(error, capacity, e.what());
        return S3DX_INVALID_ARGUMENT;
    } catch (const oom_error &e) {
        message(error, capacity, e.what());
        return S3DX_OUT_OF_MEMORY;
    } catch (const std::bad_alloc &) {
        message(error, capacity, "allocation failed");
        return S3DX_OUT_OF_MEMORY;
    } catch (const std::exception &e) {
        message(error, capacity, e.what());
        return S3DX_INTERNAL_ERROR;
    } catch (...) {
        message(error, capacity, "unknown internal error");
        return S3DX_INTERNAL_ERROR;
    }
}

inline void require(bool condition, const char *text) {
    if (!condition) throw std::invalid_argument(text);
}

inline void hip_check(hipError_t e, const char *what) {
    if (e == hipSuccess) return;
    std::string m = std::string(what) + ": " + hipGetErrorString(e);
    if (e == hipErrorOutOfMemory) throw oom_error(m);
    throw hip_error(m);
}

// Launch-error check right after a kernel launch.
inline void launch_check(const char *what) { hip_check(hipGetLastError(), what); }

inline hipStream_t as_stream(s3dx_stream s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned(const void *p, uintptr_t a) {
    return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

inline uint64_t round_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

// Carves sub-buffers out of a caller workspace (256-byte aligned pieces).
struct Carver {
    char *base;
    uint64_t size;
    uint64_t used = 0;
    Carver(void *b, uint64_t s) : base(static_cast<char *>(b)), size(s) {}
    template <class T>
    T *take(uint64_t count) {
        const uint64_t bytes = round_up(count * sizeof(T), 256);
        if (used + bytes > size) throw std::invalid_argument("workspace too small");
        T *p = reinterpret_cast<T *>(base + used);
        used += bytes;
        return p;
    }
};
// Same sizes as Carver, for the *_workspace_size queries.
struct Sizer {
    uint64_t used = 0;
    template <class T>
    void take(uint64_t count) {
        used += round_up(count * sizeof(T), 256);
    }
};

// ---------------------------------------------------------------------------
// bfloat16 (stored as uint16_t) <-> float32, round to nearest even.
// ---------------------------------------------------------------------------
__host__ __device__ inline float bf16_to_f32(uint16_t h) {
    return __builtin_bit_cast(float, static_cast<uint32_t>(h) << 16);
}
__host__ __device__ inline uint16_t f32_to_bf16(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
        u |= 0x00400000u;
    } else {
        u += 0x7fffu + ((u >> 16) & 1u);
    }
    return static_cast<uint16_t>(u >> 16);
}

// Two floats as packed bfloat16 (lo in bits 0-15), each rounded to nearest
// even: one v_cvt_pk_bf16_f32 on gfx950 (f32_to_bf16 is the same rounding,
// written out for the host and for single elements).
__device__ inline uint32_t pack_bf16x2(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
    return __builtin_bit_cast(uint32_t, v);
}

template <class T>
__device__ inline float load_as_f32(const T *p);
template <>
__device__ inline float load_as_f32<float>(const float *p) {
    return *p;
}
template <>
__device__ inline float load_as_f32<uint16_t>(const uint16_t *p) {
    return bf16_to_f32(*p);
}
template <class T>
__device__ inline void store_from_f32(T *p, float v);
template <>
__device__ inline void store_from_f32<float>(float *p, float v) {
    *p = v;
}
template <>
__device__ inline void store_from_f32<uint16_t>(uint16_t *p, float v) {
    *p = f32_to_bf16(v);
}

// Workgroups are dealt round-robin over the 8 XCDs; workgroup `bid` of
// `nblocks` takes logical index xcd_tile(bid, nblocks), so that each XCD runs a
// contiguous run of logical indices (row tiles, voxel ranges) and neighbouring
// accesses share its L2.
__device__ __forceinline__ int xcd_tile(int bid, int nblocks) {
    const int q = nblocks / 8, r = nblocks % 8;
    const int xcd = bid % 8, local = bid / 8;
    return xcd * q + min(xcd, r) + local;
}

// x * sigmoid(x) with the hardware exponential and reciprocal (a few ulp; a
// large negative x gives exp = inf, rcp = 0, result -0).
__device__ inline float silu(float v) { return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }

inline int dtype_size(int32_t dt) { return dt == S3DX_BF16 ? 2 : 4; }
inline void require_dtype(int32_t dt) {
    require(dt == S3DX_F32 || dt == S3DX_BF16, "dtype must be S3DX_F32 or S3DX_BF16");
}

// Grid-stride fill kernels (no hipMemsetAsync, so callers may capture graphs).
void fill_u32(uint32_t *p, uint64_t count, uint32_t value, hipStream_t stream);
void fill_u64(uint64_t *p, uint64_t count, uint64_t value, hipStream_t stream);

// Exclusive prefix sum of int32 in[0..n) -> out[0..n), total written to
// *total (device).  Workspace from scan_workspace_bytes(n).
uint64_t scan_workspace_bytes(int64_t n);
void exclusive_scan_i32(const int32_t *in, int32_t *out, int64_t n, int32_t *total,
                        void *workspace, hipStream_t stream);

}  // namespace s3dx
