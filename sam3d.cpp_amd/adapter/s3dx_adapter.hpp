// The C++ adapter a sam3d.cpp maintainer adds to src/objects_runtime/ to call
// libs3dx_sparse.so: RAII around the C ABI's device buffers and layer objects,
// and device-resident replacements for the reference's table builders and
// sparse blocks.  Plain C++17 over include/s3dx_sparse.h (no HIP headers).
//
//   DeviceSlatTables   SlatTables::build         sparse_ops.hpp:36, sparse_ops.cpp:49-173
//   device_subdivide   MeshSubdivideTables::build sparse_ops.hpp:77, sparse_ops.cpp:272-404
//   SlatResBlock       the res_block lambda       slat_flow_graph.cpp:216-275
//   SlatSparseStages   the SLat forward's sparse  slat_flow_graph.cpp:284-291, 441-503
//                      input and output stages
//   MeshDecoderStack   the mesh levels + head     session.cpp:927-975,
//                                                 mesh_decoder_graph.cpp:105-140
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

// Host float32 weights of one SLat res_block: norm1 [cin] x2, w1
// [cout][27][cin], b1, w2 [cout][27][cout], b2, skip [cout][1][cin] + bias
// (ws NULL: the identity skip).
struct ResBlockWeights {
    const float *n1w = nullptr, *n1b = nullptr, *w1 = nullptr, *b1 = nullptr, *w2 = nullptr, *b2 = nullptr,
                *ws = nullptr, *bs = nullptr;
};

// The SLat res_block (slat_flow_graph.cpp:216-275): LayerNorm(affine) + SiLU
// -> conv1 -> LayerNorm -> h*(1+scale)+shift -> SiLU -> conv2 -> + skip, the
// skip being x or Linear(x).  conv1's epilogue holds the norm, the modulate
// and the SiLU; conv2's the residual.
struct SlatResBlock {
    int cin = 0, cout = 0;
    bool bf16 = false;
    DeviceBuffer norm1_w, norm1_b;
    SparseConvLayer conv1, conv2, skip;

    SlatResBlock() = default;
    SlatResBlock(int cin_, int cout_, bool bf16_, const ResBlockWeights &w, s3dx_stream s)
        : cin(cin_), cout(cout_), bf16(bf16_), norm1_w(uint64_t(cin_) * 4), norm1_b(uint64_t(cin_) * 4) {
        char err[512];
        norm1_w.upload(w.n1w, uint64_t(cin) * 4, s);
        norm1_b.upload(w.n1b, uint64_t(cin) * 4, s);
        conv1 = make_layer(w.w1, w.b1, cin, cout, 27, false, bf16);
        s3dx_check(s3dx_conv_set_layernorm(conv1.get(), 1, 1e-6f, nullptr, nullptr, nullptr, nullptr, err,
                                           sizeof err), err);
        s3dx_check(s3dx_conv_set_silu(conv1.get(), 1, err, sizeof err), err);
        conv2 = make_layer(w.w2, w.b2, cout, cout, 27, false, bf16);
        if (w.ws) skip = make_layer(w.ws, w.bs, cin, cout, 1, false, bf16);
        else if (cin != cout) throw s3dx_failure(S3DX_INVALID_ARGUMENT, "s3d: res_block skip needs a Linear");
    }

    // One forward on n rows of x (device, the layers' dtype) over kmap (and
    // its gather plan, or NULL).  d_emb: this forward's emb_layers output on
    // the device, [2 * cout] float32 -- scale = d_emb[0, cout), shift =
    // d_emb[cout, 2 * cout), the reference's two views of `e` (:238-243) --
    // read by the kernel when it runs: no copy, no host synchronization.
    // The temporaries come from `tmp` (grown to 3 * n * max(cin, cout)
    // elements; growing it allocates, so size it once for the largest set).
    void forward(const void *x, int64_t n, const int32_t *kmap, const float *d_emb, void *y, DeviceBuffer &tmp,
                 s3dx_stream s, const s3dx_gather_plan *plan = nullptr) const {
        char err[512];
        const int32_t dt = bf16 ? S3DX_BF16 : S3DX_F32;
        const uint64_t es = bf16 ? 2 : 4, wide = uint64_t(cin > cout ? cin : cout);
        if (tmp.bytes() < 3 * uint64_t(n) * wide * es) tmp = DeviceBuffer(3 * uint64_t(n) * wide * es);
        char *h = tmp.get<char>(), *y1 = h + uint64_t(n) * wide * es, *sk = y1 + uint64_t(n) * wide * es;
        s3dx_check(s3dx_conv_set_modulate(conv1.get(), d_emb, d_emb + cout, err, sizeof err), err);
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

// The sparse stages of one SLat forward (slat_flow_graph.cpp:284-291 and
// 441-503) between the graph's dense parts, on device-resident tables:
//   input_stage:  h0 [nf][128] (input_layer's output) -> input_blocks.0 ->
//                 2x mean-pool -> input_blocks.1 -> skip1 [nc][1024]
//                 (skip0 [nf][128] and skip1 stay on the device)
//   output_stage: h [nc][1024] (the trunk's output) -> concat skip1 +
//                 upsample -> out_blocks.0 -> concat skip0 -> out_blocks.1
//                 -> [nf][128] (for the final LayerNorm + out_layer)
// Each block takes its emb_layers output (device [2 * cout] float32) per
// forward.  The fine and coarse maps' gather plans are built once per
// sample (bind) and shared by every conv over that map.
struct SlatSparseStages {
    static constexpr int kIo = 128, kModel = 1024;
    bool bf16 = false;
    SlatResBlock in0, in1, out0, out1;
    int64_t nf = 0, nc = 0;
    const DeviceSlatTables *t = nullptr;
    DeviceBuffer skip0, skip1, xc, xcat, h1, tmp;
    GatherPlan plan_f, plan_c;

    SlatSparseStages(bool bf16_, const ResBlockWeights w[4], s3dx_stream s)
        : bf16(bf16_), in0(kIo, kIo, bf16_, w[0], s), in1(kIo, kModel, bf16_, w[1], s),
          out0(2 * kModel, kIo, bf16_, w[2], s), out1(2 * kIo, kIo, bf16_, w[3], s) {}

    // Per sample: the tables (kept alive by the caller), the stage buffers
    // and the gather plans.  Allocates; the forwards that follow do not.
    void bind(const DeviceSlatTables &tables, s3dx_stream s) {
        t = &tables;
        nf = tables.n;
        nc = tables.nc;
        const uint64_t es = bf16 ? 2 : 4;
        skip0 = DeviceBuffer(uint64_t(nf) * kIo * es);
        skip1 = DeviceBuffer(uint64_t(nc) * kModel * es);
        xc = DeviceBuffer(uint64_t(nc) * kIo * es);
        xcat = DeviceBuffer(uint64_t(nf) * 2 * kModel * es);
        h1 = DeviceBuffer(uint64_t(nf) * kIo * es);
        tmp = DeviceBuffer(3 * uint64_t(nf) * 2 * kModel * es);
        plan_f = GatherPlan(in0.conv1, nf, tables.conv_fine.get<int32_t>(), s);
        plan_c = GatherPlan(in1.conv2, nc, tables.conv_coarse.get<int32_t>(), s);
    }

    void input_stage(const void *h0, const float *emb_in0, const float *emb_in1, s3dx_stream s) {
        char err[512];
        const int32_t dt = bf16 ? S3DX_BF16 : S3DX_F32;
        in0.forward(h0, nf, t->conv_fine.get<int32_t>(), emb_in0, skip0.get(), tmp, s, plan_f.get());
        s3dx_check(s3dx_downsample_mean(skip0.get(), dt, nf, kIo, t->coarse_children.get<int32_t>(),
                                        t->coarse_inv_count.get<float>(), nc, xc.get(), s, err, sizeof err), err);
        in1.forward(xc.get(), nc, t->conv_coarse.get<int32_t>(), emb_in1, skip1.get(), tmp, s, plan_c.get());
    }

    void output_stage(const void *h, const float *emb_out0, const float *emb_out1, void *y, s3dx_stream s) {
        char err[512];
        const int32_t dt = bf16 ? S3DX_BF16 : S3DX_F32;
        s3dx_check(s3dx_concat_rows(h, kModel, skip1.get(), kModel, dt, nc, t->fine_to_coarse.get<int32_t>(), nf,
                                    xcat.get(), s, err, sizeof err), err);
        out0.forward(xcat.get(), nf, t->conv_fine.get<int32_t>(), emb_out0, h1.get(), tmp, s, plan_f.get());
        s3dx_check(s3dx_concat_rows(h1.get(), kIo, skip0.get(), kIo, dt, nf, nullptr, nf, xcat.get(), s, err,
                                    sizeof err), err);
        out1.forward(xcat.get(), nf, t->conv_fine.get<int32_t>(), emb_out1, y, tmp, s, plan_f.get());
    }
};

// Host float32 weights of one mesh upsample block (mesh_decoder_graph.cpp:
// 105-132): GroupNorm32 affine [cin] x2, conv1 [27][cout][cin] + bias, the
// 1x1 skip [1][cout][cin] + bias, GroupNorm32 affine [cout] x2, conv2
// [27][cout][cout] + bias.
struct MeshLevelWeights {
    const float *gn1_w = nullptr, *gn1_b = nullptr, *w1 = nullptr, *b1 = nullptr, *ws = nullptr, *bs = nullptr,
                *gn2_w = nullptr, *gn2_b = nullptr, *w2 = nullptr, *b2 = nullptr;
};

// The mesh decoder's sparse stack after the dense base (session.cpp:927-975):
// for each of the two levels, MeshSubdivideTables on the current coordinates,
// then the upsample block -- GroupNorm32 + SiLU of the parents applied as
// the conv's input pass, conv1 gathering parent row j >> 3 (the repeat), the
// 1x1 skip once per parent (it commutes with the repeat), GroupNorm32 + SiLU
// of conv1's rows, conv2 + skip row i >> 3 -- and the 96 -> 101 head in FP32.
// Everything stays on the device between the levels; in the reference each
// level is a separate graph run with a host round trip of the features.
struct MeshDecoderStack {
    static constexpr int kCh[3] = {768, 192, 96};
    static constexpr int kOut = 101;
    bool bf16 = false;
    struct Level {
        DeviceBuffer gn1_w, gn1_b, gn2_w, gn2_b, s1, h1, s2, h2;
        SparseConvLayer conv1, skip, conv2;
    } lv[2];
    SparseConvLayer head;

    MeshDecoderStack(bool bf16_, const MeshLevelWeights w[2], const float *head_w, const float *head_b,
                     s3dx_stream s)
        : bf16(bf16_) {
        char err[512];
        for (int l = 0; l < 2; ++l) {
            const int cin = kCh[l], cout = kCh[l + 1];
            Level &L = lv[l];
            L.gn1_w = DeviceBuffer(uint64_t(cin) * 4);
            L.gn1_b = DeviceBuffer(uint64_t(cin) * 4);
            L.gn2_w = DeviceBuffer(uint64_t(cout) * 4);
            L.gn2_b = DeviceBuffer(uint64_t(cout) * 4);
            L.s1 = DeviceBuffer(uint64_t(cin) * 4);
            L.h1 = DeviceBuffer(uint64_t(cin) * 4);
            L.s2 = DeviceBuffer(uint64_t(cout) * 4);
            L.h2 = DeviceBuffer(uint64_t(cout) * 4);
            L.gn1_w.upload(w[l].gn1_w, uint64_t(cin) * 4, s);
            L.gn1_b.upload(w[l].gn1_b, uint64_t(cin) * 4, s);
            L.gn2_w.upload(w[l].gn2_w, uint64_t(cout) * 4, s);
            L.gn2_b.upload(w[l].gn2_b, uint64_t(cout) * 4, s);
            L.conv1 = make_layer(w[l].w1, w[l].b1, cin, cout, 27, true, bf16);
            s3dx_check(s3dx_conv_set_gather_parent(L.conv1.get(), 1, nullptr, err, sizeof err), err);
            s3dx_check(s3dx_conv_set_input_affine_silu(L.conv1.get(), L.s1.get<float>(), L.h1.get<float>(), err,
                                                       sizeof err), err);
            L.skip = make_layer(w[l].ws, w[l].bs, cin, cout, 1, true, bf16);
            L.conv2 = make_layer(w[l].w2, w[l].b2, cout, cout, 27, true, bf16);
            s3dx_check(s3dx_conv_set_input_affine_silu(L.conv2.get(), L.s2.get<float>(), L.h2.get<float>(), err,
                                                       sizeof err), err);
            s3dx_check(s3dx_conv_set_residual_parent(L.conv2.get(), 1, err, sizeof err), err);
        }
        head = make_layer(head_w, head_b, kCh[2], kOut, 1, false, false);
        if (bf16) s3dx_check(s3dx_conv_set_input_dtype(head.get(), S3DX_BF16, err, sizeof err), err);
    }

    // parents [p][4] and features [p][768] (the layers' dtype) on the device.
    // Writes raw [64p][101] float32 and the level-1 child coordinates
    // [64p][4]: the inputs of extract_object_mesh (session.cpp:986-990).
    // false where MeshSubdivideTables::build would fail (duplicate parents,
    // p > INT32_MAX / 64).
    bool run(const int32_t *d_parents, int64_t p, const void *d_features, float *d_raw, int32_t *d_child_coords,
             s3dx_stream s) const {
        char err[512];
        if (p <= 0 || p > INT32_MAX / 64) return false;
        const int32_t dt = bf16 ? S3DX_BF16 : S3DX_F32;
        const uint64_t es = bf16 ? 2 : 4;
        DeviceBuffer coords0(uint64_t(p) * 8 * 16), kmap(uint64_t(p) * 64 * 27 * 4);
        DeviceBuffer feat[2] = {DeviceBuffer(uint64_t(p) * 8 * kCh[1] * es), DeviceBuffer(uint64_t(p) * 64 * kCh[2] * es)};
        DeviceBuffer y1(uint64_t(p) * 64 * kCh[2] * es > uint64_t(p) * 8 * kCh[1] * es ? uint64_t(p) * 64 * kCh[2] * es
                                                                                     : uint64_t(p) * 8 * kCh[1] * es);
        DeviceBuffer ys(uint64_t(p) * 8 * kCh[1] * es);
        uint64_t gws = 0, g = 0;
        for (int l = 0; l < 2; ++l) {
            const int64_t n = p << (3 * (l + 1));
            for (int c : {kCh[l], kCh[l + 1]}) {
                s3dx_check(s3dx_groupnorm_workspace_size(n, c, 32, &g, err, sizeof err), err);
                gws = g > gws ? g : gws;
            }
        }
        DeviceBuffer gw(gws);
        const int32_t *par = d_parents;
        const void *x = d_features;
        for (int l = 0; l < 2; ++l) {
            const Level &L = lv[l];
            const int cin = kCh[l], cout = kCh[l + 1];
            const int64_t np = p << (3 * l), n = np * 8;
            int32_t *child = l == 0 ? coords0.get<int32_t>() : d_child_coords;
            if (!device_subdivide(par, np, child, kmap.get<int32_t>(), s)) return false;
            s3dx_check(s3dx_groupnorm_stats(x, dt, np, cin, 32, 1e-5f, L.gn1_w.get<float>(), L.gn1_b.get<float>(),
                                            L.s1.get<float>(), L.h1.get<float>(), gw.get(), gw.bytes(), s, err,
                                            sizeof err), err);
            L.conv1.run(x, np, kmap.get<int32_t>(), n, nullptr, y1.get(), dt, s);
            L.skip.run(x, np, nullptr, np, nullptr, ys.get(), dt, s);
            s3dx_check(s3dx_groupnorm_stats(y1.get(), dt, n, cout, 32, 1e-5f, L.gn2_w.get<float>(),
                                            L.gn2_b.get<float>(), L.s2.get<float>(), L.h2.get<float>(), gw.get(),
                                            gw.bytes(), s, err, sizeof err), err);
            L.conv2.run(y1.get(), n, kmap.get<int32_t>(), n, ys.get(), feat[l].get(), dt, s);
            par = child;
            x = feat[l].get();
        }
        head.run(x, p * 64, nullptr, p * 64, nullptr, d_raw, S3DX_F32, s);
        char e2[64];
        s3dx_check(s3dx_stream_synchronize(s, e2, sizeof e2), e2);  // the level buffers are freed on return
        return true;
    }
};

}  // namespace s3d
