// The C++ adapter a sam3d.cpp maintainer adds to src/objects_runtime/ to call
// libs3dx_sparse.so: RAII around the C ABI's device buffers and layer objects,
// and device-resident replacements for the reference's table builders and
// sparse blocks.  Plain C++17 over include/s3dx_sparse.h (no HIP headers).
//
//   DeviceSlatTables   SlatTables::build         sparse_ops.hpp:36, sparse_ops.cpp:49-173
//   device_subdivide   MeshSubdivideTables::build sparse_ops.hpp:77, sparse_ops.cpp:272-404
//   SlatResBlock       the res_block lambda       slat_flow_graph.cpp:216-275
//   make_layer         the conv lambda + weights  slat_flow_graph.cpp:105-155,
//                                                 mesh_decoder_graph.cpp:81-103
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "s3dx_sparse.h"

namespace s3d {

struct s3dx_failure : std::runtime_error {
    s3dx_status status;
    s3dx_failure(s3dx_status st, const std::string &m) : std::runtime_error(m), status(st) {}
};

inline void s3dx_check(s3dx_status st, const char *err) {
    if (st != S3DX_OK) throw s3dx_failure(st, std::string("s3dx: ") + err);
}

// One device allocation (s3dx_malloc / s3dx_free).
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(uint64_t bytes) : bytes_(bytes) {
        char err[256];
        s3dx_check(s3dx_malloc(&p_, bytes ? bytes : 1, err, sizeof err), err);
    }
    DeviceBuffer(const DeviceBuffer &) = delete;
    DeviceBuffer &operator=(const DeviceBuffer &) = delete;
    DeviceBuffer(DeviceBuffer &&o) noexcept : p_(std::exchange(o.p_, nullptr)), bytes_(std::exchange(o.bytes_, 0)) {}
    DeviceBuffer &operator=(DeviceBuffer &&o) noexcept {
        if (this != &o) {
            s3dx_free(p_);
            p_ = std::exchange(o.p_, nullptr);
            bytes_ = std::exchange(o.bytes_, 0);
        }
        return *this;
    }
    ~DeviceBuffer() { s3dx_free(p_); }
    template <class T = void>
    T *get() const { return static_cast<T *>(p_); }
    uint64_t bytes() const { return bytes_; }
    void upload(const void *host, uint64_t bytes, s3dx_stream s) const {
        char err[256];
        s3dx_check(s3dx_memcpy_h2d(p_, host, bytes, s, err, sizeof err), err);
    }
    void download(void *host, uint64_t bytes, s3dx_stream s) const {
        char err[256];
        s3dx_check(s3dx_memcpy_d2h(host, p_, bytes, s, err, sizeof err), err);
    }

private:
    void *p_ = nullptr;
    uint64_t bytes_ = 0;
};

// Device-resident SlatTables (the APE stays where it is).  build() keeps the
// reference's contract: false on invalid input, tables valid after true.
struct DeviceSlatTables {
    int64_t n = 0, nc = 0;
    DeviceBuffer coords, conv_fine, fine_to_coarse, coarse_coords, coarse_children, coarse_inv_count,
        conv_coarse;

    bool build(const int32_t *host_coords, int64_t n_fine, s3dx_stream s) {
        char err[512];
        uint64_t ws_k = 0, ws_c = 0;
        if (host_coords == nullptr || n_fine <= 0) return false;
        if (s3dx_kmap_workspace_size(n_fine, &ws_k, err, sizeof err) != S3DX_OK) return false;
        if (s3dx_coarsen2_workspace_size(n_fine, &ws_c, err, sizeof err) != S3DX_OK) return false;
        n = n_fine;
        DeviceBuffer ws(ws_k > ws_c ? ws_k : ws_c);
        coords = DeviceBuffer(uint64_t(n) * 16);
        conv_fine = DeviceBuffer(uint64_t(n) * 27 * 4);
        fine_to_coarse = DeviceBuffer(uint64_t(n) * 4);
        coarse_coords = DeviceBuffer(uint64_t(n) * 16);
        coarse_children = DeviceBuffer(uint64_t(n) * 8 * 4);
        coarse_inv_count = DeviceBuffer(uint64_t(n) * 4);
        conv_coarse = DeviceBuffer(uint64_t(n) * 27 * 4);
        coords.upload(host_coords, uint64_t(n) * 16, s);
        // conv_fine: sentinel n, byte-identical to build_conv (sparse_ops.cpp:126-142)
        s3dx_check(s3dx_kmap_subm3(coords.get<int32_t>(), n, static_cast<int32_t>(n), conv_fine.get<int32_t>(),
                                   ws.get(), ws.bytes(), s, err, sizeof err), err);
        // coarse set, fine_to_coarse, children, 1/(count+1) (sparse_ops.cpp:53-104)
        s3dx_check(s3dx_coarsen2(coords.get<int32_t>(), n, coarse_coords.get<int32_t>(),
                                 fine_to_coarse.get<int32_t>(), coarse_children.get<int32_t>(),
                                 coarse_inv_count.get<float>(), &nc, ws.get(), ws.bytes(), s, err, sizeof err),
                   err);
        // conv_coarse: sentinel nc (sparse_ops.cpp:142)
        s3dx_check(s3dx_kmap_subm3(coarse_coords.get<int32_t>(), nc, static_cast<int32_t>(nc),
                                   conv_coarse.get<int32_t>(), ws.get(), ws.bytes(), s, err, sizeof err),
                   err);
        char e2[64];
        s3dx_check(s3dx_stream_synchronize(s, e2, sizeof e2), e2);  // ws is freed on return
        return true;
    }
};

// Device-resident MeshSubdivideTables: children (b, 2x+bx, 2y+by, 2z+bz) and
// their neighbour rows (-1 when missing).  false for duplicate parents or
// p > INT32_MAX / 8, as the reference's build returns.
inline bool device_subdivide(const int32_t *d_parents, int64_t p, int32_t *d_child_coords, int32_t *d_child_kmap,
                             s3dx_stream s) {
    char err[512];
    uint64_t ws_bytes = 0;
    if (s3dx_subdivide2_workspace_size(p, &ws_bytes, err, sizeof err) != S3DX_OK) return false;
    DeviceBuffer ws(ws_bytes);
    const s3dx_status st =
        s3dx_subdivide2(d_parents, p, d_child_coords, d_child_kmap, ws.get(), ws_bytes, s, err, sizeof err);
    if (st == S3DX_INVALID_ARGUMENT) return false;
    s3dx_check(st, err);
    return true;
}

// A prepared layer (s3dx_conv), freed with the object.
class SparseConvLayer {
public:
    SparseConvLayer() = default;
    explicit SparseConvLayer(s3dx_conv *c) : c_(c) {}
    SparseConvLayer(const SparseConvLayer &) = delete;
    SparseConvLayer &operator=(const SparseConvLayer &) = delete;
    SparseConvLayer(SparseConvLayer &&o) noexcept : c_(std::exchange(o.c_, nullptr)) {}
    SparseConvLayer &operator=(SparseConvLayer &&o) noexcept {
        if (this != &o) {
            s3dx_conv_free(c_);
            c_ = std::exchange(o.c_, nullptr);
        }
        return *this;
    }
    ~SparseConvLayer() { s3dx_conv_free(c_); }
    s3dx_conv *get() const { return c_; }
    explicit operator bool() const { return c_ != nullptr; }
    // With a gather plan of kmap (GatherPlan below) the halo kernels skip
    // their per-tile dedupe; results are the same bits either way.
    void run(const void *x, int64_t n_in, const int32_t *kmap, int64_t n_out, const void *residual, void *y,
             int32_t y_dtype, s3dx_stream s, const s3dx_gather_plan *plan = nullptr) const {
        char err[512];
        if (plan)
            s3dx_check(s3dx_conv_run_planned(c_, plan, x, n_in, kmap, n_out, residual, y, y_dtype, s, err,
                                             sizeof err), err);
        else
            s3dx_check(s3dx_conv_run(c_, x, n_in, kmap, n_out, residual, y, y_dtype, s, err, sizeof err), err);
    }
    std::string plan(int64_t n_in, int64_t n_out) const {
        char buf[256], err[256];
        s3dx_check(s3dx_conv_plan(c_, n_in, n_out, buf, sizeof buf, err, sizeof err), err);
        return buf;
    }

private:
    s3dx_conv *c_ = nullptr;
};

// A kernel map's gather plan (s3dx_gather_plan): built once per map -- as
// SlatTables are, once per sample -- and shared by every conv over that map
// whose source rows are the map's rows (all SLat convs).  rebuild() refills
// it for the next sample's map without allocating (at most the rows it was
// built for).
class GatherPlan {
public:
    GatherPlan() = default;
    GatherPlan(const SparseConvLayer &layer, int64_t n, const int32_t *kmap, s3dx_stream s) {
        char err[512];
        s3dx_check(s3dx_gather_plan_create(layer.get(), n, kmap, n, s, &p_, err, sizeof err), err);
    }
    GatherPlan(const GatherPlan &) = delete;
    GatherPlan &operator=(const GatherPlan &) = delete;
    GatherPlan(GatherPlan &&o) noexcept : p_(std::exchange(o.p_, nullptr)) {}
    GatherPlan &operator=(GatherPlan &&o) noexcept {
        if (this != &o) {
            s3dx_gather_plan_free(p_);
            p_ = std::exchange(o.p_, nullptr);
        }
        return *this;
    }
    ~GatherPlan() { s3dx_gather_plan_free(p_); }
    void rebuild(const SparseConvLayer &layer, int64_t n, const int32_t *kmap, s3dx_stream s) {
        char err[512];
        s3dx_check(s3dx_gather_plan_rebuild(p_, layer.get(), n, kmap, n, s, err, sizeof err), err);
    }
    const s3dx_gather_plan *get() const { return p_; }

private:
    s3dx_gather_plan *p_ = nullptr;
};

// At weight load: SLat weights are [Cout][27][Cin] (gguf_schema.py:326-334),
// mesh weights [27][Cout][Cin] (convert_sam3d_to_gguf.py:486-492), mesh 1x1
// skips [1][Cout][Cin] as the converter already stored them
// (convert_sam3d_to_gguf.py:489-491: no further transpose).  kvol 27 or 1.
inline SparseConvLayer make_layer(const float *w, const float *b, int cin, int cout, int kvol, bool mesh,
                                  bool bf16) {
    char err[512];
    s3dx_conv *c = nullptr;
    s3dx_check(s3dx_conv_create(cin, cout, kvol, bf16 ? S3DX_BF16 : S3DX_F32, &c, err, sizeof err), err);
    SparseConvLayer layer(c);
    s3dx_check(s3dx_conv_set_weights(c, w, mesh ? S3DX_WEIGHT_MESH : S3DX_WEIGHT_SLAT, b, err, sizeof err), err);
    return layer;
}

// The SLat res_block (slat_flow_graph.cpp:216-275): LayerNorm(affine) + SiLU
// -> conv1 -> LayerNorm -> h*(1+scale)+shift -> SiLU -> conv2 -> + skip, the
// skip being x or Linear(x).  conv1's epilogue holds the norm, the modulate
// (device buffers read per forward) and the SiLU; conv2's the residual.
// Weights host float32: norm1 [cin] x2, w1 [cout][27][cin], b1, w2
// [cout][27][cout], b2, skip [cout][1][cin] + bias or NULL (identity).
struct SlatResBlock {
    int cin = 0, cout = 0;
    bool bf16 = false;
    DeviceBuffer norm1_w, norm1_b, mod_scale, mod_shift;
    SparseConvLayer conv1, conv2, skip;

    SlatResBlock(int cin_, int cout_, bool bf16_, const float *n1w, const float *n1b, const float *w1,
                 const float *b1, const float *w2, const float *b2, const float *ws, const float *bs,
                 s3dx_stream s)
        : cin(cin_), cout(cout_), bf16(bf16_), norm1_w(uint64_t(cin_) * 4), norm1_b(uint64_t(cin_) * 4),
          mod_scale(uint64_t(cout_) * 4), mod_shift(uint64_t(cout_) * 4) {
        char err[512];
        norm1_w.upload(n1w, uint64_t(cin) * 4, s);
        norm1_b.upload(n1b, uint64_t(cin) * 4, s);
        conv1 = make_layer(w1, b1, cin, cout, 27, false, bf16);
        s3dx_check(s3dx_conv_set_layernorm(conv1.get(), 1, 1e-6f, nullptr, nullptr, nullptr, nullptr, err,
                                           sizeof err), err);
        s3dx_check(s3dx_conv_set_modulate(conv1.get(), mod_scale.get<float>(), mod_shift.get<float>(), err,
                                          sizeof err), err);
        s3dx_check(s3dx_conv_set_silu(conv1.get(), 1, err, sizeof err), err);
        conv2 = make_layer(w2, b2, cout, cout, 27, false, bf16);
        if (ws) skip = make_layer(ws, bs, cin, cout, 1, false, bf16);
        else if (cin != cout) throw s3dx_failure(S3DX_INVALID_ARGUMENT, "s3d: res_block skip needs a Linear");
    }

    // One forward on n rows of x (device, the layers' dtype) over kmap (and
    // its gather plan, or NULL).  scale/shift: host [cout], this forward's
    // emb_layers halves.  The temporaries come from `tmp` (3 * n * max(cin,
    // cout) elements).
    void forward(const void *x, int64_t n, const int32_t *kmap, const float *scale, const float *shift, void *y,
                 DeviceBuffer &tmp, s3dx_stream s, const s3dx_gather_plan *plan = nullptr) {
        char err[512];
        const int32_t dt = bf16 ? S3DX_BF16 : S3DX_F32;
        const uint64_t es = bf16 ? 2 : 4, wide = uint64_t(cin > cout ? cin : cout);
        if (tmp.bytes() < 3 * uint64_t(n) * wide * es) tmp = DeviceBuffer(3 * uint64_t(n) * wide * es);
        char *h = tmp.get<char>(), *y1 = h + uint64_t(n) * wide * es, *sk = y1 + uint64_t(n) * wide * es;
        mod_scale.upload(scale, uint64_t(cout) * 4, s);
        mod_shift.upload(shift, uint64_t(cout) * 4, s);
        s3dx_check(s3dx_layernorm_rows(x, dt, n, cin, 1e-6f, norm1_w.get<float>(), norm1_b.get<float>(), nullptr,
                                       nullptr, 1, h, dt, s, err, sizeof err), err);
        conv1.run(h, n, kmap, n, nullptr, y1, dt, s, plan);
        const void *res = x;
        if (skip) {
            skip.run(x, n, nullptr, n, nullptr, sk, dt, s);
            res = sk;
        }
        conv2.run(y1, n, kmap, n, res, y, dt, s, plan);
    }
};

}  // namespace s3d
