"""Whole blocks through the C ABI against the oracle, at the shapes the
reference runs.

- The SLat sparse res_block exactly as slat_flow_graph.cpp:216-275 (and the
  out blocks at :441-503) builds it: [down/up] -> LayerNorm(affine) -> SiLU ->
  conv1 -> LayerNorm -> h*(1+scale)+shift -> SiLU -> conv2 -> + skip, the skip
  being the block input or a Linear of it, with scale/shift in device buffers
  that change between forwards (the emb_layers output).
- The benchmark's configurations at full size: the config-2 block chained at
  28,265 voxels in both dtypes, the config-3 1024-channel conv on all 5,086
  coarse rows, and the config-4 192-channel slot-offset conv over all 226,120
  children -- each asserting the launch plan the benchmark times.

BF16 layers round every stored tensor to BF16 (inputs, weights, the block's
intermediate outputs); the oracle rounds at the same points and runs in
float64.  Gates (rel-L2): 1e-5 FP32, 1e-2 BF16.  BF16 blocks are also held to
1e-2 against the unrounded float chain (the reference's F32 graph on the
BF16-rounded inputs and weights).
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import check_rel

pytestmark = pytest.mark.gpu

TOL = {0: 1e-5, 1: 1e-2}


def _r(W, a, dtype):
    return W.round_bf16(a) if dtype == 1 and a is not None else a


def _dev(s3dx, W, a, dtype):
    a = np.ascontiguousarray(a, np.float32)
    return s3dx.DeviceArray.from_host(W.f32_to_bf16_bits(a) if dtype == s3dx.BF16 else a)


def _host(s3dx, W, d, dtype):
    h = d.download()
    return W.bf16_bits_to_f32(h).reshape(h.shape) if dtype == s3dx.BF16 else h


def _buf(s3dx, rows, c, dtype):
    return s3dx.DeviceArray((rows, c), np.uint16 if dtype == s3dx.BF16 else np.float32)


class ResBlock:
    """The reference res_block on the GPU: one layer object per conv, the
    per-forward modulate in device buffers the caller rewrites."""

    def __init__(self, s3dx, W, dtype, cin, cout, seed):
        self.s3dx, self.W, self.dtype, self.cin, self.cout = s3dx, W, dtype, cin, cout
        g = lambda k, shape, s=1.0: W.normal_f32(seed, k, shape, s)  # noqa: E731
        self.p = dict(n1w=g(1, (cin,), 0.2) + 1.0, n1b=g(2, (cin,), 0.2),
                      w1=W.conv_weight(seed, 3, cin, cout), b1=g(4, (cout,), 0.1),
                      w2=W.conv_weight(seed, 5, cout, cout), b2=g(6, (cout,), 0.1),
                      ws=W.conv_weight(seed, 7, cin, cout, kvol=1) if cin != cout else None,
                      bs=g(8, (cout,), 0.1))
        p = self.p
        self.n1w, self.n1b = s3dx.DeviceArray.from_host(p["n1w"]), s3dx.DeviceArray.from_host(p["n1b"])
        self.mscale = s3dx.DeviceArray((cout,), np.float32)
        self.mshift = s3dx.DeviceArray((cout,), np.float32)
        self.conv1 = (s3dx.SparseConv(cin, cout, 27, dtype).set_weights(p["w1"], s3dx.WEIGHT_SLAT, p["b1"])
                      .set_layernorm(True, 1e-6).set_modulate(self.mscale, self.mshift).set_silu(True))
        self.conv2 = s3dx.SparseConv(cout, cout, 27, dtype).set_weights(p["w2"], s3dx.WEIGHT_SLAT, p["b2"])
        self.skip = (s3dx.SparseConv(cin, cout, 1, dtype).set_weights(p["ws"], s3dx.WEIGHT_SLAT, p["bs"])
                     if p["ws"] is not None else None)

    def run(self, xin, n, kmap, scale, shift):
        s3dx, dt = self.s3dx, self.dtype
        self.mscale.upload(scale)
        self.mshift.upload(shift)
        h = _buf(s3dx, n, self.cin, dt)
        s3dx.layernorm_rows(xin, dt, n, self.cin, 1e-6, self.n1w, self.n1b, silu=True, y=h, y_dtype=dt)
        y1 = _buf(s3dx, n, self.cout, dt)
        self.conv1.run(h, n, kmap, n, y1, dt)
        res = xin
        if self.skip is not None:
            res = _buf(s3dx, n, self.cout, dt)
            self.skip.run(xin, n, None, n, res, dt)
        y2 = _buf(s3dx, n, self.cout, dt)
        self.conv2.run(y1, n, kmap, n, y2, dt, res)
        return y2

    def oracle(self, O, xin, kmap, n, scale, shift, rounded):
        """rounded: round every stored tensor as the BF16 layers do; else the
        reference's float chain on rounded inputs and weights."""
        W, p = self.W, self.p
        rd = (lambda a: W.round_bf16(a)) if self.dtype == 1 else (lambda a: a)
        st = rd if rounded else (lambda a: a)
        h = st(O.silu(O.layernorm(xin, 1e-6, p["n1w"], p["n1b"])))
        y1 = O.conv(h, kmap, n, rd(p["w1"]), 0, self.cout, p["b1"])
        y1 = st(O.silu(O.modulate(O.layernorm(y1, 1e-6), scale, shift)))
        skip = xin if p["ws"] is None else st(O.conv(xin, None, n, rd(p["ws"]), 0, self.cout, p["bs"], kvol=1))
        return O.conv(y1, kmap, n, rd(p["w2"]), 0, self.cout, p["b2"]) + skip


def _slat_sets(W, O):
    fine = W.shell_64(res=24, centre=(12.0, 12.0, 12.0), radius=7.0)
    nf = fine.shape[0]
    nc, coarse, f2c, children, inv = O.coarsen2(fine)
    coarse = np.ascontiguousarray(coarse[:nc])
    return (fine, nf, O.kmap_subm3(fine, nf), nc, coarse, f2c, children[:8 * nc], inv[:nc],
            O.kmap_subm3(coarse, nc))


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("block,cin,cout", [
    ("input_blocks.0", 128, 128),    # fine, identity skip
    ("input_blocks.1", 128, 1024),   # 2x mean-pool down to the coarse set, Linear skip, LN as its own pass
    ("out_blocks.0", 2048, 128),     # nearest upsample of the coarse 2048 channels, Linear skip
    ("out_blocks.1", 256, 128),      # fine, Linear skip
])
def test_slat_res_block(s3dx, O, W, dtype, block, cin, cout):
    fine, nf, kf, nc, coarse, f2c, children, inv, kc = _slat_sets(W, O)
    seed = {"input_blocks.0": 60, "input_blocks.1": 61, "out_blocks.0": 62, "out_blocks.1": 63}[block]
    rb = ResBlock(s3dx, W, dtype, cin, cout, seed)
    plan1, plan2 = rb.conv1.plan(nf, nf), rb.conv2.plan(nf, nf)
    print(f"{block} dtype={dtype} nf={nf} nc={nc} conv1: {plan1} | conv2: {plan2}", flush=True)
    dk_f, dk_c = s3dx.DeviceArray.from_host(kf), s3dx.DeviceArray.from_host(kc)
    # The block input on the device, and its host copy as the layers store it.
    if block == "input_blocks.1":
        xf = _r(W, W.normal_f32(seed, 20, (nf, cin)), dtype)
        xd = _buf(s3dx, nc, cin, dtype)
        s3dx.downsample_mean(_dev(s3dx, W, xf, dtype), dtype, nf, cin, s3dx.DeviceArray.from_host(children),
                             s3dx.DeviceArray.from_host(inv), nc, xd)
        xin = _r(W, O.downsample_mean(xf, children, inv, nc), dtype)
        n, kmap, dk = nc, kc, dk_c
    elif block == "out_blocks.0":
        xcoarse = _r(W, W.normal_f32(seed, 20, (nc, cin)), dtype)
        xd = _buf(s3dx, nf, cin, dtype)
        s3dx.upsample_nearest(_dev(s3dx, W, xcoarse, dtype), dtype, nc, cin, s3dx.DeviceArray.from_host(f2c), nf, xd)
        xin = O.upsample_nearest(xcoarse, f2c)
        n, kmap, dk = nf, kf, dk_f
    else:
        xin = _r(W, W.normal_f32(seed, 20, (nf, cin)), dtype)
        xd = _dev(s3dx, W, xin, dtype)
        n, kmap, dk = nf, kf, dk_f
    check_rel(_host(s3dx, W, xd, dtype), xin, 0.0 if dtype == 1 else 1e-7, "block input")
    # Two forwards of the same layer objects with different modulate values.
    for fwd in range(2):
        scale = W.normal_f32(seed, 30 + fwd, (cout,), 0.3)
        shift = W.normal_f32(seed, 40 + fwd, (cout,), 0.3)
        got = _host(s3dx, W, rb.run(xd, n, dk, scale, shift), dtype)
        check_rel(got, rb.oracle(O, xin, kmap, n, scale, shift, True), TOL[dtype], f"forward {fwd}")
        if dtype == 1:
            check_rel(got, rb.oracle(O, xin, kmap, n, scale, shift, False), TOL[dtype],
                      f"forward {fwd} vs the float chain")


@pytest.mark.parametrize("cout", [128, 1024])
def test_modulate_buffers_reread_each_run(s3dx, O, W, cout):
    # One FP32 layer, LayerNorm fused (128) or as its own pass (1024): the
    # modulate buffers are rewritten between runs and each run follows them.
    coords = W.shells_union(4)[:1200]
    n = coords.shape[0]
    kmap = O.kmap_subm3(coords, n)
    x = W.normal_f32(70, 1, (n, 64))
    w = W.conv_weight(70, 2, 64, cout)
    b = W.normal_f32(70, 3, (cout,))
    ms, mh = s3dx.DeviceArray((cout,), np.float32), s3dx.DeviceArray((cout,), np.float32)
    conv = (s3dx.SparseConv(64, cout, 27, s3dx.F32).set_weights(w, s3dx.WEIGHT_SLAT, b)
            .set_layernorm(True, 1e-6).set_modulate(ms, mh).set_silu(True))
    print(f"modulate cout={cout}: {conv.plan(n, n)}", flush=True)
    xd, dk = s3dx.DeviceArray.from_host(x), s3dx.DeviceArray.from_host(kmap)
    h = O.conv(x, kmap, n, w, 0, cout, b)
    y = s3dx.DeviceArray((n, cout), np.float32)
    for k in range(3):
        scale, shift = W.normal_f32(71, k, (cout,), 0.5), W.normal_f32(72, k, (cout,), 0.5)
        ms.upload(scale)
        mh.upload(shift)
        conv.run(xd, n, dk, n, y, s3dx.F32)
        check_rel(y.download(), O.silu(O.modulate(O.layernorm(h, 1e-6), scale, shift)), 1e-5, f"run {k}")


@pytest.mark.parametrize("dtype", [0, 1])
def test_config2_block_full_size(s3dx, O, W, dtype):
    # The benchmark's step at its real size: conv(+LN+SiLU) -> conv(+x).
    coords = W.shells_union(0)
    n = coords.shape[0]
    assert n == 28265
    kmap = O.kmap_subm3(coords, n)
    c = 128
    x = _r(W, W.normal_f32(0, 100, (n, c)), dtype)
    w1, w2 = W.conv_weight(0, 101, c, c), W.conv_weight(0, 102, c, c)
    b = np.zeros(c, np.float32)
    conv1 = (s3dx.SparseConv(c, c, 27, dtype).set_weights(w1, s3dx.WEIGHT_SLAT, b)
             .set_layernorm(True, 1e-6).set_silu(True))
    conv2 = s3dx.SparseConv(c, c, 27, dtype).set_weights(w2, s3dx.WEIGHT_SLAT, b)
    # BF16: the halo-staged 64-row kernel; FP32: 64-row split-K tiles.
    head = "mfma tiling=21 split-k halo rows=64 cols=128 kc=64" if dtype == 1 else \
        "mfma tiling=18 split-k rows=64 cols=128 kc=32"
    for cv in (conv1, conv2):
        plan = cv.plan(n, n)
        print(f"config 2 dtype={dtype}: {plan}", flush=True)
        assert plan.startswith(head) and plan.endswith("grid=442x1"), plan
    xd, dk = _dev(s3dx, W, x, dtype), s3dx.DeviceArray.from_host(kmap)
    h, y = _buf(s3dx, n, c, dtype), _buf(s3dx, n, c, dtype)
    conv1.run(xd, n, dk, n, h, dtype)
    conv2.run(h, n, dk, n, y, dtype, xd)
    rd = (lambda a: W.round_bf16(a)) if dtype == 1 else (lambda a: a)
    h_ref = O.silu(O.layernorm(O.conv(x, kmap, n, rd(w1), 0, c, b), 1e-6))
    check_rel(_host(s3dx, W, h, dtype), h_ref, TOL[dtype], "conv1 + LayerNorm + SiLU")
    ref = O.conv(rd(h_ref), kmap, n, rd(w2), 0, c, b) + x
    check_rel(_host(s3dx, W, y, dtype), ref, TOL[dtype], "block output")
    if dtype == 1:
        check_rel(_host(s3dx, W, y, dtype), O.conv(h_ref, kmap, n, rd(w2), 0, c, b) + x, TOL[dtype],
                  "block output vs the float chain")


def test_config3_full_size(s3dx, O, W):
    fine = W.shells_union(0)
    nc, coarse, _, _, _ = O.coarsen2(fine)
    assert nc == 5086
    coarse = np.ascontiguousarray(coarse[:nc])
    kmap = O.kmap_subm3(coarse, nc)
    c = 1024
    conv = s3dx.SparseConv(c, c, 27, s3dx.BF16).set_weights(W.conv_weight(0, 301, c, c), s3dx.WEIGHT_SLAT, None)
    plan = conv.plan(nc, nc)
    print(f"config 3: {plan}", flush=True)
    assert plan.startswith("mfma tiling=21 split-k halo rows=64 cols=128 kc=64") and plan.endswith("grid=80x8"), plan
    x = W.round_bf16(W.normal_f32(0, 300, (nc, c)))
    y = _buf(s3dx, nc, c, s3dx.BF16)
    conv.run(_dev(s3dx, W, x, s3dx.BF16), nc, s3dx.DeviceArray.from_host(kmap), nc, y, s3dx.BF16)
    ref = O.conv(x, kmap, nc, W.round_bf16(W.conv_weight(0, 301, c, c)), 0, c, None)
    check_rel(_host(s3dx, W, y, s3dx.BF16), ref, 1e-2)


def test_config4_full_size(s3dx, O, W):
    parents = W.shells_union(0)
    p = parents.shape[0]
    child, kmap = O.subdivide2(parents)
    n = 8 * p
    c = 192
    w = W.conv_weight(0, 401, c, c, layout="mesh")
    slot = W.normal_f32(0, 402, (8, c), 0.02)
    conv = (s3dx.SparseConv(c, c, 27, s3dx.BF16).set_weights(w, s3dx.WEIGHT_MESH, None)
            .set_gather_parent(True, slot))
    plan = conv.plan(p, n)
    print(f"config 4 children={n}: {plan}", flush=True)
    assert plan.startswith("pre=children mfma tiling=21 split-k halo rows=64 cols=96") and plan.endswith("grid=3534x2"), plan
    xp = W.round_bf16(W.normal_f32(0, 400, (p, c)))
    y = _buf(s3dx, n, c, s3dx.BF16)
    conv.run(_dev(s3dx, W, xp, s3dx.BF16), p, s3dx.DeviceArray.from_host(kmap), n, y, s3dx.BF16)
    xc = W.round_bf16(O.repeat_children(xp) + np.tile(slot, (p, 1)))
    ref = O.conv(xc, kmap, n, W.round_bf16(w), 1, c, None)
    check_rel(_host(s3dx, W, y, s3dx.BF16), ref, 1e-2)
