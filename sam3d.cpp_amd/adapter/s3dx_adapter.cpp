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

// Host float32 rows -> device rows in the layers' dtype (and back): what a
// graph's get_tensor_f32 / set_input_f32 hand the stages between runs.
s3d::DeviceBuffer to_device(const float *host, uint64_t count, bool bf16, s3dx_stream s) {
    char err[256];
    s3d::DeviceBuffer f(count * 4);
    f.upload(host, count * 4, s);
    if (!bf16) return f;
    s3d::DeviceBuffer b(count * 2);
    s3d::s3dx_check(s3dx_convert(f.get(), S3DX_F32, int64_t(count), b.get(), S3DX_BF16, s, err, sizeof err), err);
    char e2[64];
    s3d::s3dx_check(s3dx_stream_synchronize(s, e2, sizeof e2), e2);  // f is freed on return
    return b;
}

void to_host(const void *dev, uint64_t count, bool bf16, float *host, s3dx_stream s) {
    char err[256];
    if (!bf16) {
        s3d::s3dx_check(s3dx_memcpy_d2h(host, dev, count * 4, s, err, sizeof err), err);
        return;
    }
    s3d::DeviceBuffer f(count * 4);
    s3d::s3dx_check(s3dx_convert(dev, S3DX_BF16, int64_t(count), f.get(), S3DX_F32, s, err, sizeof err), err);
    f.download(host, count * 4, s);
}

s3d::ResBlockWeights block_weights(const float *const *w) {
    s3d::ResBlockWeights b;
    b.n1w = w[0], b.n1b = w[1], b.w1 = w[2], b.b1 = w[3], b.w2 = w[4], b.b2 = w[5], b.ws = w[6], b.bs = w[7];
    return b;
}

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

// The SLat res_block on the fine set of `coords` (tables by DeviceSlatTables),
// FP32 or BF16 layers, `forwards` forwards.  w: the 8 pointers of
// ResBlockWeights (ws/bs NULL for the identity skip).  emb [forwards][2 *
// cout] (host): each forward's emb_layers output, uploaded to a device
// buffer as a graph's output would arrive; odd forwards run with the fine
// map's gather plan.  x [n][cin] and y [forwards][n][cout] host float32.
__attribute__((visibility("default"))) s3dx_status s3dx_adapter_res_block(
    const int32_t *coords, int64_t n, int32_t cin, int32_t cout, int32_t dtype, const float *x,
    const float *const *w, int32_t forwards, const float *emb, float *y, char *error, uint64_t error_capacity) {
    return guarded(error, error_capacity, [&]() -> s3dx_status {
        Stream st;
        const bool bf16 = dtype == S3DX_BF16;
        s3d::DeviceSlatTables t;
        if (!t.build(coords, n, st.s)) throw s3d::s3dx_failure(S3DX_INVALID_ARGUMENT, "SlatTables build failed");
        const s3d::SlatResBlock block(cin, cout, bf16, block_weights(w), st.s);
        s3d::DeviceBuffer dx = to_device(x, uint64_t(n) * cin, bf16, st.s);
        s3d::DeviceBuffer dy(uint64_t(n) * cout * (bf16 ? 2 : 4)), demb(uint64_t(2) * cout * 4), tmp;
        s3d::GatherPlan plan(block.conv1, n, t.conv_fine.get<int32_t>(), st.s);
        for (int f = 0; f < forwards; ++f) {
            demb.upload(emb + uint64_t(f) * 2 * cout, uint64_t(2) * cout * 4, st.s);
            block.forward(dx.get(), n, t.conv_fine.get<int32_t>(), demb.get<float>(), dy.get(), tmp, st.s,
                          f % 2 ? plan.get() : nullptr);
            to_host(dy.get(), uint64_t(n) * cout, bf16, y + uint64_t(f) * n * cout, st.s);
        }
        return S3DX_OK;
    });
}

// One SLat forward's sparse stages on the fine set of `coords`, driven as
// the reference's forward would be once its graph is split at them: the
// dense graph before them hands over h0 = input_layer(x) [nf][128] and the
// four res blocks' emb_layers outputs; input_stage runs; skip1 [nc][1024]
// goes to the trunk graph; the trunk's output h [nc][1024] comes back;
// output_stage runs; out [nf][128] goes to the final LayerNorm + out_layer.
// w: 4 x 8 ResBlockWeights pointers (input_blocks.0, input_blocks.1,
// out_blocks.0, out_blocks.1).  emb: [2*128 | 2*1024 | 2*128 | 2*128].
// nc is returned; skip1 and h hold n rows of capacity.
__attribute__((visibility("default"))) s3dx_status s3dx_adapter_slat_stages(
    const int32_t *coords, int64_t n, int32_t dtype, const float *const *w, const float *h0, const float *emb,
    const float *h_trunk, int64_t *nc_out, float *skip1, float *out, char *error, uint64_t error_capacity) {
    return guarded(error, error_capacity, [&]() -> s3dx_status {
        Stream st;
        const bool bf16 = dtype == S3DX_BF16;
        s3d::DeviceSlatTables t;
        if (!t.build(coords, n, st.s)) throw s3d::s3dx_failure(S3DX_INVALID_ARGUMENT, "SlatTables build failed");
        const s3d::ResBlockWeights bw[4] = {block_weights(w), block_weights(w + 8), block_weights(w + 16),
                                            block_weights(w + 24)};
        s3d::SlatSparseStages stages(bf16, bw, st.s);
        stages.bind(t, st.s);
        const int64_t nc = t.nc;
        *nc_out = nc;
        s3d::DeviceBuffer demb(2816 * 4), y(uint64_t(n) * 128 * (bf16 ? 2 : 4));
        demb.upload(emb, 2816 * 4, st.s);
        const float *e = demb.get<float>();
        s3d::DeviceBuffer dh0 = to_device(h0, uint64_t(n) * 128, bf16, st.s);
        stages.input_stage(dh0.get(), e, e + 256, st.s);
        to_host(stages.skip1.get(), uint64_t(nc) * 1024, bf16, skip1, st.s);  // -> the trunk graph
        s3d::DeviceBuffer dh = to_device(h_trunk, uint64_t(nc) * 1024, bf16, st.s);  // <- its output
        stages.output_stage(dh.get(), e + 2304, e + 2560, y.get(), st.s);
        to_host(y.get(), uint64_t(n) * 128, bf16, out, st.s);
        return S3DX_OK;
    });
}

// The mesh decoder's levels + head (MeshDecoderStack) from the dense base's
// output: parents [p][4] and features [p][768] host float32 in (what the
// base graph's get_tensor_f32 returns, session.cpp:922); raw
// [64p][101] and the level-1 child coordinates [64p][4] out (the inputs of
// extract_object_mesh).  w: 2 x 10 MeshLevelWeights pointers, then the
// head's weight [101][1][96] and bias.  INVALID_ARGUMENT where
// MeshSubdivideTables::build fails.
__attribute__((visibility("default"))) s3dx_status s3dx_adapter_mesh_decoder(
    const int32_t *parents, int64_t p, int32_t dtype, const float *features, const float *const *w, float *raw,
    int32_t *child_coords, char *error, uint64_t error_capacity) {
    return guarded(error, error_capacity, [&]() -> s3dx_status {
        if (p <= 0 || p > INT32_MAX / 64) throw s3d::s3dx_failure(S3DX_INVALID_ARGUMENT, "parent count out of range");
        Stream st;
        const bool bf16 = dtype == S3DX_BF16;
        s3d::MeshLevelWeights lw[2];
        for (int l = 0; l < 2; ++l) {
            const float *const *q = w + 10 * l;
            lw[l].gn1_w = q[0], lw[l].gn1_b = q[1], lw[l].w1 = q[2], lw[l].b1 = q[3], lw[l].ws = q[4];
            lw[l].bs = q[5], lw[l].gn2_w = q[6], lw[l].gn2_b = q[7], lw[l].w2 = q[8], lw[l].b2 = q[9];
        }
        const s3d::MeshDecoderStack stack(bf16, lw, w[20], w[21], st.s);
        s3d::DeviceBuffer dp(uint64_t(p) * 16), draw(uint64_t(p) * 64 * 101 * 4), dc(uint64_t(p) * 64 * 16);
        dp.upload(parents, uint64_t(p) * 16, st.s);
        s3d::DeviceBuffer df = to_device(features, uint64_t(p) * 768, bf16, st.s);
        if (!stack.run(dp.get<int32_t>(), p, df.get(), draw.get<float>(), dc.get<int32_t>(), st.s))
            throw s3d::s3dx_failure(S3DX_INVALID_ARGUMENT, "MeshSubdivideTables build failed");
        draw.download(raw, uint64_t(p) * 64 * 101 * 4, st.s);
        dc.download(child_coords, uint64_t(p) * 64 * 16, st.s);
        return S3DX_OK;
    });
}

}  // extern "C"
