"""Parity of the benchmark configs' larger shapes through the C ABI.

Config 3: a 1024 -> 1024 conv on the 2x OR-pooled (coarse) set.
Config 4/5: the mesh upsample block (mesh_decoder_graph.cpp:109-134) at its real
channel counts -- GroupNorm32 + SiLU of the parents fused into the children's
gather, conv, GroupNorm32 + SiLU fused into the next gather, conv, plus the 1x1
skip of the repeated input as the residual -- against the oracle's op-by-op
restatement.  Voxel counts are small so the oracle finishes in seconds.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import check_rel, rel_l2

pytestmark = pytest.mark.gpu

TOL = {0: 1e-5, 1: 1e-2}


def _rnd(W, a, dtype):
    return W.round_bf16(a) if dtype == 1 else a


def _dev(s3dx, W, x, dtype):
    if dtype == s3dx.BF16:
        return s3dx.DeviceArray.from_host(W.f32_to_bf16_bits(x))
    return s3dx.DeviceArray.from_host(np.ascontiguousarray(x, np.float32))


def _host(s3dx, W, d, dtype):
    h = d.download()
    return W.bf16_bits_to_f32(h).reshape(h.shape) if dtype == s3dx.BF16 else h


@pytest.mark.parametrize("dtype", [1])
def test_config3_coarse_1024_channels(s3dx, O, W, dtype):
    fine = W.shell_64(res=20, centre=(10.0, 10.0, 10.0), radius=6.0)
    nc, coarse, _, _, _ = O.coarsen2(fine)
    coarse = np.ascontiguousarray(coarse[:nc])
    kmap = O.kmap_subm3(coarse, nc)
    c = 1024
    print(f"config3 nc={nc}", flush=True)
    x = W.normal_f32(31, 1, (nc, c))
    w = W.conv_weight(31, 2, c, c)
    b = W.normal_f32(31, 3, (c,))
    conv = s3dx.SparseConv(c, c, 27, dtype).set_weights(w, s3dx.WEIGHT_SLAT, b)
    assert "split-k" in conv.plan(nc, nc)
    y = s3dx.DeviceArray((nc, c), np.uint16 if dtype == s3dx.BF16 else np.float32)
    conv.run(_dev(s3dx, W, x, dtype), nc, s3dx.DeviceArray.from_host(kmap), nc, y, dtype)
    ref = O.conv(_rnd(W, x, dtype), kmap, nc, _rnd(W, w, dtype), 0, c, b)
    check_rel(_host(s3dx, W, y, dtype), ref, TOL[dtype])


def _gn_dev(s3dx, x_dev, dtype, n, c, gamma, beta):
    g, bt = s3dx.DeviceArray.from_host(gamma), s3dx.DeviceArray.from_host(beta)
    scale, shift, ws = s3dx.groupnorm_stats(x_dev, dtype, n, c, 32, 1e-5, g, bt)
    return scale, shift, (g, bt, ws)


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("parent_skip", [False, True])
@pytest.mark.parametrize("level,cin,cout,radius", [(0, 768, 192, 2.0), (1, 192, 96, 4.0)])
def test_mesh_upsample_block(s3dx, O, W, level, cin, cout, radius, parent_skip, dtype):
    # dtype 0: FP32 layers, the reference mesh graph's own precision (F16
    # weights cast to F32 in the graph, mesh_decoder_graph.cpp:10-12, 89-102);
    # dtype 1: BF16 layers as the benchmark's config 5 runs them.
    parents = W.shell_64(res=12, centre=(6.0, 6.0, 6.0), radius=radius)
    p = parents.shape[0]
    child, kmap = O.subdivide2(parents)
    n = 8 * p
    et = np.uint16 if dtype == s3dx.BF16 else np.float32
    print(f"mesh block level={level} dtype={dtype} parents={p} children={n} parent_skip={parent_skip}",
          flush=True)
    seed = 40 + level
    x = W.normal_f32(seed, 1, (p, cin))
    g1, b1 = W.normal_f32(seed, 2, (cin,), 0.2) + 1.0, W.normal_f32(seed, 3, (cin,), 0.2)
    g2, b2 = W.normal_f32(seed, 4, (cout,), 0.2) + 1.0, W.normal_f32(seed, 5, (cout,), 0.2)
    w1 = W.conv_weight(seed, 6, cin, cout, layout="mesh")
    w2 = W.conv_weight(seed, 7, cout, cout, layout="mesh")
    ws = W.conv_weight(seed, 8, cin, cout, kvol=1, layout="mesh")
    c1, c2, cs = (W.normal_f32(seed, k, (cout,), 0.1) for k in (9, 10, 11))

    # GPU: GN stats of the parents -> conv1 gathers parent rows with the affine
    # + SiLU applied; GN stats of conv1 -> conv2 with affine + SiLU in its
    # gather; the 1x1 skip of the repeated raw input is conv2's residual.
    xd = _dev(s3dx, W, x, dtype)
    dk = s3dx.DeviceArray.from_host(kmap)
    s1, h1, keep1 = _gn_dev(s3dx, xd, dtype, p, cin, g1, b1)
    conv1 = (s3dx.SparseConv(cin, cout, 27, dtype).set_weights(w1, s3dx.WEIGHT_MESH, c1)
             .set_gather_parent(True).set_input_affine_silu(s1, h1))
    y1 = s3dx.DeviceArray((n, cout), et)
    conv1.run(xd, p, dk, n, y1, dtype)
    # The skip on the repeated input, or once per parent with conv2 reading
    # residual row i >> 3: the same values.
    skip = s3dx.SparseConv(cin, cout, 1, dtype).set_weights(ws, s3dx.WEIGHT_MESH, cs)
    skip.set_gather_parent(not parent_skip)
    ns = p if parent_skip else n
    ys = s3dx.DeviceArray((ns, cout), et)
    skip.run(xd, p, None, ns, ys, dtype)
    s2, h2, keep2 = _gn_dev(s3dx, y1, dtype, n, cout, g2, b2)
    conv2 = (s3dx.SparseConv(cout, cout, 27, dtype).set_weights(w2, s3dx.WEIGHT_MESH, c2)
             .set_input_affine_silu(s2, h2).set_residual_parent(parent_skip))
    y2 = s3dx.DeviceArray((n, cout), et)
    conv2.run(y1, n, dk, n, y2, dtype, ys)
    got = _host(s3dx, W, y2, dtype)

    # Oracle, op by op, on the same roundings of stored tensors (none in FP32).
    xr = _rnd(W, x, dtype)
    a1 = O.repeat_children(O.silu(O.groupnorm(xr, 32, 1e-5, g1, b1)))
    r1 = _rnd(W, O.conv(_rnd(W, a1, dtype), kmap, n, _rnd(W, w1, dtype), 1, cout, c1), dtype)
    a2 = O.silu(O.groupnorm(r1, 32, 1e-5, g2, b2))
    rs = _rnd(W, O.conv(O.repeat_children(xr), None, n, _rnd(W, ws, dtype), 1, cout, cs, kvol=1), dtype)
    ref = O.conv(_rnd(W, a2, dtype), kmap, n, _rnd(W, w2, dtype), 1, cout, c2) + rs
    check_rel(got, ref, TOL[dtype], f"{cin}->{cout} dtype {dtype}")


def _gn_f64(x, groups, eps, gamma, beta):
    """GroupNorm's per-channel scale/shift over all rows, in float64
    (statistics over every voxel x C/groups channels, mesh_decoder_graph.cpp:16-30)."""
    n, c = x.shape
    xg = x.astype(np.float64).reshape(n, groups, c // groups)
    mean = xg.mean(axis=(0, 2))
    var = np.square(xg - mean[None, :, None]).mean(axis=(0, 2))
    inv = np.repeat(1.0 / np.sqrt(var + eps), c // groups)
    scale = inv * gamma
    return scale, beta - np.repeat(mean, c // groups) * scale


def _parent_map(kmap):
    """A child map read at parent resolution: entry j -> j >> 3 (-1 stays)."""
    return np.where(kmap >= 0, kmap >> 3, -1).astype(np.int32)


# The launches the benchmark's config-5 stack makes (bench.py mesh_stack): per
# level (conv1 gathering parent rows after the GN affine + SiLU pass, the 1x1
# skip on the parents, conv2 after its GN pass).
CONFIG5_PLANS = {
    0: ("pre=rows parent-rows mfma tiling=21 split-k halo rows=64 cols=96 kc=64 xf=0 ln=none grid=3534x2",
        "mfma tiling=4 rows=64 cols=192 kc=64 xf=0 ln=none grid=442x1",
        "pre=rows mfma tiling=21 split-k halo rows=64 cols=96 kc=64 xf=0 ln=none grid=3534x2"),
    1: ("pre=rows parent-rows mfma tiling=21 split-k halo rows=64 cols=96 kc=64 xf=0 ln=none grid=28265x1",
        "linear pipe cols=96 ksteps=12 ln=none grid=512",
        "pre=rows mfma tiling=19 split-k rows=64 cols=96 kc=32 xf=0 ln=none grid=28265x1"),
}


def test_config5_chained_full_size(s3dx, O, W):
    # The mesh decoder's sparse stack at its real size, chained as the
    # reference runs it (session.cpp:927-975) and as the benchmark times it:
    # 28,265 parents (768 ch) -> subdivide -> block 768->192 on 226,120
    # children -> subdivide -> block 192->96 on 1,808,960 children -> FP32
    # head 96->101 fed the BF16 rows.  Every stage is checked against the
    # oracle on the GPU's own input to that stage: GroupNorm statistics in
    # float64 over all rows, convs on 2,000 sampled output rows (full input),
    # the 1x1 skip on all parents, the head on sampled rows.
    bf = s3dx.BF16
    seed = 0
    parents = W.shells_union(seed)
    p0 = parents.shape[0]
    dp = s3dx.DeviceArray.from_host(parents)
    xp = s3dx.DeviceArray.from_host(W.f32_to_bf16_bits(W.normal_f32(seed, 500, (p0, 768))))
    plans = {}
    for level, (cin, cout) in enumerate(((768, 192), (192, 96))):
        p = xp.shape[0]
        n = 8 * p
        child, dk = s3dx.subdivide2(dp, p, True)
        print(f"config 5 level {level}: parents={p} children={n}", flush=True)
        g1 = W.normal_f32(seed, 510 + level, (cin,), 0.2) + 1.0
        b1 = W.normal_f32(seed, 520 + level, (cin,), 0.2)
        g2 = W.normal_f32(seed, 530 + level, (cout,), 0.2) + 1.0
        b2 = W.normal_f32(seed, 540 + level, (cout,), 0.2)
        w1 = W.conv_weight(seed, 550 + level, cin, cout, layout="mesh")
        wsk = W.conv_weight(seed, 560 + level, cin, cout, kvol=1, layout="mesh")
        w2 = W.conv_weight(seed, 570 + level, cout, cout, layout="mesh")
        c1, cs, c2 = (W.normal_f32(seed, 580 + 3 * level + k, (cout,), 0.1) for k in range(3))
        s1, h1, keep1 = _gn_dev(s3dx, xp, bf, p, cin, g1, b1)
        conv1 = (s3dx.SparseConv(cin, cout, 27, bf).set_weights(w1, s3dx.WEIGHT_MESH, c1)
                 .set_gather_parent(True).set_input_affine_silu(s1, h1))
        skip = s3dx.SparseConv(cin, cout, 1, bf).set_weights(wsk, s3dx.WEIGHT_MESH, cs)
        y1 = s3dx.DeviceArray((n, cout), np.uint16)
        ys = s3dx.DeviceArray((p, cout), np.uint16)
        conv1.run(xp, p, dk, n, y1, bf)
        skip.run(xp, p, None, p, ys, bf)
        s2, h2, keep2 = _gn_dev(s3dx, y1, bf, n, cout, g2, b2)
        conv2 = (s3dx.SparseConv(cout, cout, 27, bf).set_weights(w2, s3dx.WEIGHT_MESH, c2)
                 .set_input_affine_silu(s2, h2).set_residual_parent(True))
        y2 = s3dx.DeviceArray((n, cout), np.uint16)
        conv2.run(y1, n, dk, n, y2, bf, ys)
        plans[level] = (conv1.plan(p, n), skip.plan(p, p), conv2.plan(n, n))
        print(f"  plans: conv1 {plans[level][0]} | skip {plans[level][1]} | conv2 {plans[level][2]}", flush=True)
        assert plans[level] == CONFIG5_PLANS[level], plans[level]

        kmap = dk.download()
        rows = np.sort(np.random.default_rng(level).choice(n, 2000, replace=False))
        xh = _host(s3dx, W, xp, bf)
        # GroupNorm 1 over the parents, conv1 over the children (parent row j >> 3)
        sc, sh = _gn_f64(xh, 32, 1e-5, g1, b1)
        check_rel(s1.download(), sc, 1e-5, f"level {level} GN1 scale")
        check_rel(h1.download(), sh, 1e-5, f"level {level} GN1 shift")
        a1 = W.round_bf16(O.silu((xh * sc + sh).astype(np.float32)))
        ref1 = O.conv(a1, _parent_map(kmap[rows]), p, W.round_bf16(w1), 1, cout, c1)
        check_rel(_host(s3dx, W, y1, bf)[rows], ref1, 1e-2, f"level {level} conv1 {cin}->{cout}")
        ysh = _host(s3dx, W, ys, bf)
        check_rel(ysh, O.conv(xh, None, p, W.round_bf16(wsk), 1, cout, cs, kvol=1), 1e-2,
                  f"level {level} 1x1 skip on the parents")
        # GroupNorm 2 over conv1's rows, conv2 + the skip's row i >> 3
        y1h = _host(s3dx, W, y1, bf)
        sc, sh = _gn_f64(y1h, 32, 1e-5, g2, b2)
        check_rel(s2.download(), sc, 1e-5, f"level {level} GN2 scale")
        check_rel(h2.download(), sh, 1e-5, f"level {level} GN2 shift")
        a2 = W.round_bf16(O.silu((y1h * sc + sh).astype(np.float32)))
        del y1h
        ref2 = O.conv(a2, kmap[rows], n, W.round_bf16(w2), 1, cout, c2) + ysh[rows >> 3]
        del a2
        check_rel(_host(s3dx, W, y2, bf)[rows], ref2, 1e-2, f"level {level} conv2 {cout}->{cout} + skip")
        xp, dp = y2, child
        del y1, ys, kmap
    n1 = xp.shape[0]
    assert n1 == 8 * 8 * p0
    head = (s3dx.SparseConv(96, 101, 1, s3dx.F32).set_weights(W.conv_weight(seed, 590, 96, 101, kvol=1),
                                                               s3dx.WEIGHT_SLAT, None).set_input_dtype(bf))
    out = s3dx.DeviceArray((n1, 101), np.float32)
    head.run(xp, n1, None, n1, out, s3dx.F32)
    print(f"  head: {head.plan(n1, n1)}", flush=True)
    assert head.plan(n1, n1) == "in=bf16 linear cols=128 ksteps=6 terms=3 ln=none grid=768"
    rows = np.sort(np.random.default_rng(7).choice(n1, 4000, replace=False))
    yh = _host(s3dx, W, xp, bf)[rows]
    ref = O.conv(yh, None, len(rows), W.conv_weight(seed, 590, 96, 101, kvol=1), 0, 101, None, kvol=1)
    check_rel(out.download()[rows], ref, 1e-5, "FP32 head 96->101 on the BF16 rows")
