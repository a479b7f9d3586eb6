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


@pytest.mark.parametrize("parent_skip", [False, True])
@pytest.mark.parametrize("level,cin,cout,radius", [(0, 768, 192, 2.0), (1, 192, 96, 4.0)])
def test_mesh_upsample_block(s3dx, O, W, level, cin, cout, radius, parent_skip):
    dtype = s3dx.BF16
    parents = W.shell_64(res=12, centre=(6.0, 6.0, 6.0), radius=radius)
    p = parents.shape[0]
    child, kmap = O.subdivide2(parents)
    n = 8 * p
    print(f"mesh block level={level} parents={p} children={n} parent_skip={parent_skip}", flush=True)
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
    y1 = s3dx.DeviceArray((n, cout), np.uint16)
    conv1.run(xd, p, dk, n, y1, dtype)
    # The skip on the repeated input, or once per parent with conv2 reading
    # residual row i >> 3: the same values.
    skip = s3dx.SparseConv(cin, cout, 1, dtype).set_weights(ws, s3dx.WEIGHT_MESH, cs)
    skip.set_gather_parent(not parent_skip)
    ns = p if parent_skip else n
    ys = s3dx.DeviceArray((ns, cout), np.uint16)
    skip.run(xd, p, None, ns, ys, dtype)
    s2, h2, keep2 = _gn_dev(s3dx, y1, dtype, n, cout, g2, b2)
    conv2 = (s3dx.SparseConv(cout, cout, 27, dtype).set_weights(w2, s3dx.WEIGHT_MESH, c2)
             .set_input_affine_silu(s2, h2).set_residual_parent(parent_skip))
    y2 = s3dx.DeviceArray((n, cout), np.uint16)
    conv2.run(y1, n, dk, n, y2, dtype, ys)
    got = _host(s3dx, W, y2, dtype)

    # Oracle, op by op, on the same bf16 roundings of stored tensors.
    xr = _rnd(W, x, 1)
    a1 = O.repeat_children(O.silu(O.groupnorm(xr, 32, 1e-5, g1, b1)))
    r1 = _rnd(W, O.conv(_rnd(W, a1, 1), kmap, n, _rnd(W, w1, 1), 1, cout, c1), 1)
    a2 = O.silu(O.groupnorm(r1, 32, 1e-5, g2, b2))
    rs = _rnd(W, O.conv(O.repeat_children(xr), None, n, _rnd(W, ws, 1), 1, cout, cs, kvol=1), 1)
    ref = O.conv(_rnd(W, a2, 1), kmap, n, _rnd(W, w2, 1), 1, cout, c2) + rs
    check_rel(got, ref, 1e-2)
