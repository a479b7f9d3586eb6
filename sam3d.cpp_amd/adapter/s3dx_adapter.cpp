// A compiled consumer of include/s3dx_sparse.h: the adapter of
// s3dx_adapter.hpp exercised end to end.  Each entry point takes and returns
// HOST arrays so a caller without a device runtime of its own (the tests'
// ctypes) can compare them with the reference's tables and the oracle.
// Built with the host C++ compiler alone (no hipcc, no HIP headers).
#include "s3dx_adapter.hpp"

#include <algorithm>
#include <cstring>

namespace {

template <class F>
s3dx_status guarded(char *error, uint64_t capacity, F &&body) noexcept {
    auto put = [&](const char *text) {
        if (!error || !capacity) return;
        const size_t n = std::min<size_t>(capacity - 1, std::strlen(text));
        std::memcpy(error, text, n);
        error[n] = '\0';
    };
    if (!error && capacity) return S3DX_INVALID_ARGUMENT;
    try {
        const s3dx_status st = body();
        if (st == S3DX_OK) put("");
        return st;
    } catch (const s3d::s3dx_failure &e) {
        put(e.what());
        return e.status;
    } catch (const std::exception &e) {
        put(e.what());
        return S3DX_INTERNAL_ERROR;
    }
}

struct Stream {
    s3dx_stream s = nullptr;
    Stream() {
        char err[256];
        s3d::s3dx_check(s3dx_stream_create(&s, err, sizeof err), err);
    }
    ~Stream() { s3dx_stream_destroy(s, nullptr, 0); }
};

}  // namespace

extern "C" {

// DeviceSlatTables::build on host coords; the tables come back to the host
// (capacities as s3dx_coarsen2's: n rows).  INVALID_ARGUMENT when build()
// returns false.
__attribute__((visibility("default"))) s3dx_status s3dx_adapter_slat_tables(
    const int32_t *coords, int64_t n, int32_t *conv_fine, int64_t *nc, int32_t *coarse_coords,
    int32_t *fine_to_coarse, int32_t *coarse_children, float *coarse_inv_count, int32_t *conv_coarse,
    char *error, uint64_t error_capacity) {
    return guarded(error, error_capacity, [&]() -> s3dx_status {
        Stream st;
        s3d::DeviceSlatTables t;
        if (!t.build(coords, n, st.s)) throw s3d::s3dx_failure(S3DX_INVALID_ARGUMENT, "SlatTables build failed");
        *nc = t.nc;
        const uint64_t un = uint64_t(n), unc = uint64_t(t.nc);
        t.conv_fine.download(conv_fine, un * 27 * 4, st.s);
        t.coarse_coords.download(coarse_coords, unc * 16, st.s);
        t.fine_to_coarse.download(fine_to_coarse, un * 4, st.s);
        t.coarse_children.download(coarse_children, unc * 8 * 4, st.s);
        t.coarse_inv_count.download(coarse_inv_count, unc * 4, st.s);
        t.conv_coarse.download(conv_coarse, unc * 27 * 4, st.s);
        return S3DX_OK;
    });
}

// device_subdivide on host parents; children [8p][4] and kmap [8p][27] to the
// host.  INVALID_ARGUMENT where MeshSubdivideTables::build returns false.
__attribute__((visibility("default"))) s3dx_status s3dx_adapter_subdivide(const int32_t *parents, int64_t p,
                                                                          int32_t *child_coords,
                                                                          int32_t *child_kmap, char *error,
                                                                          uint64_t error_capacity) {
    return guarded(error, error_capacity, [&]() -> s3dx_status {
        if (p <= 0 || p > INT32_MAX / 8) throw s3d::s3dx_failure(S3DX_INVALID_ARGUMENT, "parent count out of range");
        Stream st;
        s3d::DeviceBuffer dp(uint64_t(p) * 16), dc(uint64_t(p) * 8 * 16), dk(uint64_t(p) * 8 * 27 * 4);
        dp.upload(parents, uint64_t(p) * 16, st.s);
        if (!s3d::device_subdivide(dp.get<int32_t>(), p, dc.get<int32_t>(), dk.get<int32_t>(), st.s))
            throw s3d::s3dx_failure(S3DX_INVALID_ARGUMENT, "MeshSubdivideTables build failed");
        dc.download(child_coords, uint64_t(p) * 8 * 16, st.s);
        dk.download(child_kmap, uint64_t(p) * 8 * 27 * 4, st.s);
        return S3DX_OK;
    });
}

// The SLat res_block on the fine set of `coords` (tables built by
// DeviceSlatTables), FP32 layers, `forwards` forwards with modulate
// scale/shift [forwards][cout] (host).  x [n][cin]; ws/bs NULL for the
// identity skip; y [forwards][n][cout] to the host.
__attribute__((visibility("default"))) s3dx_status s3dx_adapter_res_block(
    const int32_t *coords, int64_t n, int32_t cin, int32_t cout, const float *x, const float *n1w,
    const float *n1b, const float *w1, const float *b1, const float *w2, const float *b2, const float *ws,
    const float *bs, int32_t forwards, const float *scale, const float *shift, float *y, char *error,
    uint64_t error_capacity) {
    return guarded(error, error_capacity, [&]() -> s3dx_status {
        Stream st;
        s3d::DeviceSlatTables t;
        if (!t.build(coords, n, st.s)) throw s3d::s3dx_failure(S3DX_INVALID_ARGUMENT, "SlatTables build failed");
        s3d::SlatResBlock block(cin, cout, false, n1w, n1b, w1, b1, w2, b2, ws, bs, st.s);
        s3d::DeviceBuffer dx(uint64_t(n) * cin * 4), dy(uint64_t(n) * cout * 4), tmp;
        dx.upload(x, uint64_t(n) * cin * 4, st.s);
        // Odd forwards run with the fine map's gather plan: same results.
        s3d::GatherPlan plan(block.conv1, n, t.conv_fine.get<int32_t>(), st.s);
        for (int f = 0; f < forwards; ++f) {
            block.forward(dx.get(), n, t.conv_fine.get<int32_t>(), scale + uint64_t(f) * cout,
                          shift + uint64_t(f) * cout, dy.get(), tmp, st.s, f % 2 ? plan.get() : nullptr);
            dy.download(y + uint64_t(f) * n * cout, uint64_t(n) * cout * 4, st.s);
        }
        return S3DX_OK;
    });
}

}  // extern "C"
