// Device plumbing entry points (the reference's Backend seam,
// src/objects_runtime/backend.hpp:16-58) and shared device utilities: fill
// kernels and a three-phase exclusive scan.
#include "common.hpp"

namespace s3dx {

namespace {

__global__ void fill_u32_kernel(uint32_t *p, uint64_t count, uint32_t value) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride)
        p[i] = value;
}

__global__ void fill_u64_kernel(uint64_t *p, uint64_t count, uint64_t value) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride)
        p[i] = value;
}

unsigned fill_blocks(uint64_t count) {
    const uint64_t b = (count + 255) / 256;
    return static_cast<unsigned>(b < 1 ? 1 : (b > 8192 ? 8192 : b));
}

// ---- scan: each block scans 1024 items (256 threads x 4) -----------------
constexpr int kScanThreads = 256;
constexpr int kScanItems = 4;
constexpr int kScanTile = kScanThreads * kScanItems;

__device__ int32_t block_exclusive_scan(int32_t v, int32_t *total) {
    // Wave64 inclusive scan with shuffles, then across the 4 waves via LDS.
    __shared__ int32_t wave_sums[kScanThreads / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int32_t x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int32_t y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
    }
    if (lane == 63) wave_sums[wave] = x;
    __syncthreads();
    int32_t before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kScanThreads / 64; ++w) {
        const int32_t s = wave_sums[w];
        if (w < wave) before += s;
        all += s;
    }
    __syncthreads();
    *total = all;
    return before + x - v;
}

__global__ void scan_tiles_kernel(const int32_t *in, int32_t *out, int64_t n,
                                  int32_t *tile_sums) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile + threadIdx.x * kScanItems;
    int32_t v[kScanItems];
    int32_t local = 0;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        v[k] = base + k < n ? in[base + k] : 0;
        local += v[k];
    }
    int32_t total;
    int32_t run = block_exclusive_scan(local, &total);
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        if (base + k < n) out[base + k] = run;
        run += v[k];
    }
    if (threadIdx.x == 0) tile_sums[blockIdx.x] = total;
}

__global__ void scan_add_kernel(int32_t *out, int64_t n, const int32_t *tile_offsets) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile + threadIdx.x * kScanItems;
    const int32_t add = tile_offsets[blockIdx.x];
#pragma unroll
    for (int k = 0; k < kScanItems; ++k)
        if (base + k < n) out[base + k] += add;
}

__global__ void scan_total_kernel(const int32_t *in, const int32_t *out, int64_t n,
                                  int32_t *total) {
    if (threadIdx.x == 0 && blockIdx.x == 0) *total = n > 0 ? out[n - 1] + in[n - 1] : 0;
}

}  // namespace

void fill_u32(uint32_t *p, uint64_t count, uint32_t value, hipStream_t stream) {
    if (!count) return;
    fill_u32_kernel<<<fill_blocks(count), 256, 0, stream>>>(p, count, value);
    launch_check("fill_u32");
}

void fill_u64(uint64_t *p, uint64_t count, uint64_t value, hipStream_t stream) {
    if (!count) return;
    fill_u64_kernel<<<fill_blocks(count), 256, 0, stream>>>(p, count, value);
    launch_check("fill_u64");
}

uint64_t scan_workspace_bytes(int64_t n) {
    // One (tile sums, tile offsets) pair per recursion level.
    uint64_t bytes = 256;
    if (n <= 0) return bytes;
    do {
        const int64_t tiles = (n + kScanTile - 1) / kScanTile;
        bytes += round_up(static_cast<uint64_t>(tiles) * sizeof(int32_t), 256) * 2;
        n = tiles;
    } while (n > 1);
    return bytes;
}

void exclusive_scan_i32(const int32_t *in, int32_t *out, int64_t n, int32_t *total,
                        void *workspace, hipStream_t stream) {
    if (n <= 0) {
        fill_u32(reinterpret_cast<uint32_t *>(total), 1, 0, stream);
        return;
    }
    const int64_t tiles = (n + kScanTile - 1) / kScanTile;
    char *ws = static_cast<char *>(workspace);
    int32_t *sums = reinterpret_cast<int32_t *>(ws);
    int32_t *offs = reinterpret_cast<int32_t *>(
        ws + round_up(static_cast<uint64_t>(tiles) * sizeof(int32_t), 256));
    char *rest = ws + 2 * round_up(static_cast<uint64_t>(tiles) * sizeof(int32_t), 256);
    scan_tiles_kernel<<<static_cast<unsigned>(tiles), kScanThreads, 0, stream>>>(in, out, n, sums);
    launch_check("scan_tiles");
    if (tiles > 1) {
        exclusive_scan_i32(sums, offs, tiles, total, rest, stream);
        scan_add_kernel<<<static_cast<unsigned>(tiles), kScanThreads, 0, stream>>>(out, n, offs);
        launch_check("scan_add");
    }
    scan_total_kernel<<<1, 64, 0, stream>>>(in, out, n, total);
    launch_check("scan_total");
}

}  // namespace s3dx

using namespace s3dx;

extern "C" {

S3DX_API uint32_t s3dx_abi_version(void) { return S3DX_ABI_VERSION; }

S3DX_API s3dx_status s3dx_device_info(int32_t *device_count, char *name, uint64_t name_capacity,
                                      char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(device_count != nullptr, "device_count is NULL");
        require(name != nullptr || name_capacity == 0, "name is NULL with nonzero capacity");
        int count = 0;
        hip_check(hipGetDeviceCount(&count), "hipGetDeviceCount");
        *device_count = count;
        if (name && name_capacity) {
            name[0] = '\0';
            if (count > 0) {
                int dev = 0;
                hip_check(hipGetDevice(&dev), "hipGetDevice");
                hipDeviceProp_t prop;
                hip_check(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties");
                std::string s = std::string(prop.name) + " " + prop.gcnArchName + " CUs=" +
                                std::to_string(prop.multiProcessorCount);
                message(name, name_capacity, s.c_str());
            }
        }
    });
}

S3DX_API s3dx_status s3dx_malloc(void **out, uint64_t bytes, char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(out != nullptr, "out is NULL");
        *out = nullptr;
        hip_check(hipMalloc(out, bytes ? bytes : 1), "hipMalloc");
    });
}

S3DX_API void s3dx_free(void *ptr) {
    if (ptr) (void)hipFree(ptr);
}

S3DX_API s3dx_status s3dx_memcpy_h2d(void *dst, const void *host_src, uint64_t bytes,
                                     s3dx_stream stream, char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        if (!bytes) return;
        require(dst && host_src, "NULL pointer");
        hip_check(hipMemcpyAsync(dst, host_src, bytes, hipMemcpyHostToDevice, as_stream(stream)),
                  "hipMemcpyAsync H2D");
        hip_check(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
    });
}

S3DX_API s3dx_status s3dx_memcpy_d2h(void *host_dst, const void *src, uint64_t bytes,
                                     s3dx_stream stream, char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        if (!bytes) return;
        require(host_dst && src, "NULL pointer");
        hip_check(hipMemcpyAsync(host_dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)),
                  "hipMemcpyAsync D2H");
        hip_check(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
    });
}

S3DX_API s3dx_status s3dx_stream_create(s3dx_stream *out, char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(out != nullptr, "out is NULL");
        hipStream_t s = nullptr;
        hip_check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
        *out = s;
    });
}

S3DX_API s3dx_status s3dx_stream_destroy(s3dx_stream stream, char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        if (stream) hip_check(hipStreamDestroy(as_stream(stream)), "hipStreamDestroy");
    });
}

S3DX_API s3dx_status s3dx_stream_synchronize(s3dx_stream stream, char *error,
                                             uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        hip_check(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
    });
}

S3DX_API s3dx_status s3dx_event_create(s3dx_event *out, char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(out != nullptr, "out is NULL");
        hipEvent_t e = nullptr;
        hip_check(hipEventCreate(&e), "hipEventCreate");
        *out = e;
    });
}

S3DX_API s3dx_status s3dx_timing_event_create(s3dx_event *out, char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(out != nullptr, "out is NULL");
        hipEvent_t e = nullptr;
        // No system-scope fence on record: no cache write-back / invalidate
        // between the timed launches, so the interval is the work's own.
        hip_check(hipEventCreateWithFlags(&e, hipEventDisableSystemFence), "hipEventCreateWithFlags");
        *out = e;
    });
}

S3DX_API s3dx_status s3dx_event_destroy(s3dx_event event, char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        if (event) hip_check(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)), "hipEventDestroy");
    });
}

S3DX_API s3dx_status s3dx_event_record(s3dx_event event, s3dx_stream stream, char *error,
                                       uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(event != nullptr, "event is NULL");
        hip_check(hipEventRecord(reinterpret_cast<hipEvent_t>(event), as_stream(stream)),
                  "hipEventRecord");
    });
}

S3DX_API s3dx_status s3dx_event_elapsed_ms(s3dx_event start, s3dx_event stop, float *ms,
                                           char *error, uint64_t error_capacity) {
    return boundary(error, error_capacity, [&] {
        require(start && stop && ms, "NULL argument");
        hip_check(hipEventSynchronize(reinterpret_cast<hipEvent_t>(stop)), "hipEventSynchronize");
        hip_check(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                      reinterpret_cast<hipEvent_t>(stop)),
                  "hipEventElapsedTime");
    });
}

}  // extern "C"
