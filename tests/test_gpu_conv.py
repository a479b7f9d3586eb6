"""GPU sparse convolution through the C ABI against the oracle.

Tolerances (rel-L2): FP32 <= 1e-5; BF16 <= 1e-2 against the FP32 oracle run
on the BF16-rounded inputs and weights."""
import numpy as np
import pytest

from helpers import check_rel, rel_l2

pytestmark = pytest.mark.gpu

TOL = {0: 1e-5, 1: 1e-2}


def to_dev(s3dx, x, dtype):
    W = s3dx.workloads
    if dtype == s3dx.BF16:
        return s3dx.DeviceArray.from_host(W.f32_to_bf16_bits(x))
    return s3dx.DeviceArray.from_host(np.ascontiguousarray(x, np.float32))


def from_dev(s3dx, d, dtype):
    h = d.download()
    return s3dx.workloads.bf16_bits_to_f32(h).reshape(h.shape) if dtype == s3dx.BF16 else h


def rnd(s3dx, a, dtype):
    return s3dx.workloads.round_bf16(a) if dtype == s3dx.BF16 and a is not None else a


def gpu_conv(s3dx, x, kmap, n_in, w, layout, bias, dtype, cout, kvol=27, n_out=None,
             y_dtype=None, residual=None, setup=None):
    cin = x.shape[1]
    conv = s3dx.SparseConv(cin, cout, kvol, dtype).set_weights(w, layout, bias)
    if setup:
        setup(conv)
    n_out = n_out if n_out is not None else (kmap.shape[0] if kmap is not None else x.shape[0])
    yd = dtype if y_dtype is None else y_dtype
    y = s3dx.DeviceArray((n_out, cout), np.uint16 if yd == s3dx.BF16 else np.float32)
    dk = s3dx.DeviceArray.from_host(kmap) if kmap is not None else None
    dr = to_dev(s3dx, residual, yd) if residual is not None else None
    conv.run(to_dev(s3dx, x, dtype), n_in, dk, n_out, y, yd, dr)
    return from_dev(s3dx, y, yd)


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("cin,cout", [(32, 32), (64, 64), (128, 96), (128, 128), (64, 160),
                                      (96, 192), (256, 256), (16, 32)])
def test_linear_layer_lane_layout(s3dx, W, dtype, cin, cout):
    # kvol 1, no map: a plain GEMM, so any A/B/D lane-layout mistake shows.
    n = 517
    print(f"linear dtype={dtype} cin={cin} cout={cout}", flush=True)
    x = W.normal_f32(3, 1, (n, cin))
    w = W.normal_f32(3, 2, (cout, 1, cin), 1.0 / np.sqrt(cin))
    b = W.normal_f32(3, 3, (cout,))
    got = gpu_conv(s3dx, x, None, n, w, s3dx.WEIGHT_SLAT, b, dtype, cout, kvol=1)
    xr, wr = rnd(s3dx, x, dtype), rnd(s3dx, w, dtype)
    ref = xr.astype(np.float64) @ wr[:, 0, :].T.astype(np.float64) + b
    check_rel(got, ref, TOL[dtype] / (10 if dtype == 0 else 1))


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("cin,cout", [(64, 64), (128, 128), (32, 96), (192, 192), (96, 96),
                                      (256, 256), (8, 128), (20, 36), (128, 101)])
def test_subm_conv_matches_oracle(s3dx, O, W, dtype, cin, cout):
    coords = W.shells_union(1)[:3000]
    n = coords.shape[0]
    print(f"subm conv dtype={dtype} cin={cin} cout={cout} n={n}", flush=True)
    kmap = O.kmap_subm3(coords, n)
    x = W.normal_f32(4, 1, (n, cin))
    w = W.conv_weight(4, 2, cin, cout)
    b = W.normal_f32(4, 3, (cout,), 0.5)
    got = gpu_conv(s3dx, x, kmap, n, w, s3dx.WEIGHT_SLAT, b, dtype, cout)
    ref = O.conv(rnd(s3dx, x, dtype), kmap, n, rnd(s3dx, w, dtype), 0, cout, b)
    check_rel(got, ref, TOL[dtype])


def test_config1_fp32_conv(s3dx, O, W):
    coords = W.shell_64()
    n = coords.shape[0]
    kmap = O.kmap_subm3(coords, n)
    x = W.normal_f32(0, 1, (n, 64))
    w = W.conv_weight(0, 2, 64, 64)
    b = np.zeros(64, np.float32)
    got = gpu_conv(s3dx, x, kmap, n, w, s3dx.WEIGHT_SLAT, b, s3dx.F32, 64)
    ref = O.conv(x, kmap, n, w, 0, 64, b)
    check_rel(got, ref, 1e-5)


@pytest.mark.parametrize("dtype", [0, 1])
def test_mesh_layout_minus_one_sentinel(s3dx, O, W, dtype):
    coords = W.shell_64(res=32, centre=(16.0, 16.0, 16.0), radius=9.0)
    n = coords.shape[0]
    kmap = O.kmap_subm3(coords, -1)
    cin, cout = 96, 192
    x = W.normal_f32(5, 1, (n, cin))
    w = W.conv_weight(5, 2, cin, cout, layout="mesh")
    b = W.normal_f32(5, 3, (cout,))
    got = gpu_conv(s3dx, x, kmap, n, w, s3dx.WEIGHT_MESH, b, dtype, cout)
    ref = O.conv(rnd(s3dx, x, dtype), kmap, n, rnd(s3dx, w, dtype), 1, cout, b)
    check_rel(got, ref, TOL[dtype])


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("cin,cout", [(64, 64), (24, 40), (20, 64)])
@pytest.mark.parametrize("slot_on,affine_on", [(True, True), (True, False), (False, True)])
def test_gather_parent_slot_offset_and_input_affine(s3dx, O, W, dtype, cin, cout, slot_on, affine_on):
    # conv over subdivided children whose features are silu(GN-affine(parent))
    # repeated x8, plus a per-slot offset when set.  cin 20 takes the
    # per-element transform pass; without slot offsets the parent rows are
    # transformed and the gather reads row j >> 3.
    parents = W.shell_64(res=24, centre=(12.0, 12.0, 12.0), radius=7.0)
    p = parents.shape[0]
    child, kmap = O.subdivide2(parents)
    n = 8 * p
    print(f"gather-parent dtype={dtype} p={p} cin={cin} slot={slot_on} affine={affine_on}", flush=True)
    xp = W.normal_f32(6, 1, (p, cin))
    slot = W.normal_f32(6, 2, (8, cin), 0.02)
    scale = W.normal_f32(6, 3, (cin,), 0.5) + 1.0
    shift = W.normal_f32(6, 4, (cin,), 0.5)
    w = W.conv_weight(6, 5, cin, cout, layout="mesh")
    b = W.normal_f32(6, 6, (cout,))
    ds, dh = s3dx.DeviceArray.from_host(scale), s3dx.DeviceArray.from_host(shift)

    def setup(conv):
        conv.set_gather_parent(True, slot if slot_on else None)
        if affine_on:
            conv.set_input_affine_silu(ds, dh)
        plan = conv.plan(p, n)
        assert plan.startswith("pre=children " if slot_on else "pre=rows parent-rows "), plan

    got = gpu_conv(s3dx, xp, kmap, p, w, s3dx.WEIGHT_MESH, b, dtype, cout, n_out=n, setup=setup)
    xr = rnd(s3dx, xp, dtype)
    xc = O.repeat_children(xr) + (np.tile(slot, (p, 1)) if slot_on else 0.0)
    act = O.silu(xc * scale + shift) if affine_on else xc
    ref = O.conv(rnd(s3dx, act, dtype), kmap, n, rnd(s3dx, w, dtype), 1, cout, b)
    check_rel(got, ref, TOL[dtype])


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("cout,ln", [(128, True), (160, True), (64, False), (40, False)])
def test_residual_at_parent_resolution(s3dx, O, W, dtype, cout, ln):
    # Output row i adds residual row i >> 3, through the fused-LN (128),
    # separate-LN (160), plain MFMA (64) and generic (40) epilogues.
    parents = W.shell_64(res=20, centre=(10.0, 10.0, 10.0), radius=5.0)
    p = parents.shape[0]
    _, kmap = O.subdivide2(parents)
    n = 8 * p
    print(f"residual parent dtype={dtype} cout={cout} ln={ln} n={n}", flush=True)
    cin = 64
    x = W.normal_f32(9, 1, (n, cin))
    w = W.conv_weight(9, 2, cin, cout)
    b = W.normal_f32(9, 3, (cout,))
    res = W.normal_f32(9, 4, (p, cout))

    def setup(conv):
        conv.set_residual_parent(True)
        if ln:
            conv.set_layernorm(True, 1e-6).set_silu(True)

    got = gpu_conv(s3dx, x, kmap, n, w, s3dx.WEIGHT_SLAT, b, dtype, cout, residual=res, setup=setup)
    h = O.conv(rnd(s3dx, x, dtype), kmap, n, rnd(s3dx, w, dtype), 0, cout, b)
    if ln:
        h = O.silu(O.layernorm(h, 1e-6))
    ref = h + O.repeat_children(rnd(s3dx, res, dtype))
    check_rel(got, ref, TOL[dtype])


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("cin,cout,n,parent,res_parent,silu", [
    (96, 101, 300001, False, False, False),  # the head's shape; > 2 passes of the persistent grid
    (160, 96, 4099, True, True, True),       # parent rows, per-parent residual, SiLU
    (128, 128, 5, False, True, False),        # fewer rows than one 32-row block
    (64, 256, 777, False, False, True),
])
def test_linear_kernel(s3dx, O, W, dtype, cin, cout, n, parent, res_parent, silu):
    # 1x1 layers on the LDS-resident-weight kernel against a plain GEMM.
    rows_in = (n + 7) // 8 if parent else n
    x = W.normal_f32(18, 1, (rows_in, cin))
    w = W.conv_weight(18, 2, cin, cout, kvol=1)
    b = W.normal_f32(18, 3, (cout,))
    res = W.normal_f32(18, 4, ((n + 7) // 8 if res_parent else n, cout))

    def setup(conv):
        conv.set_gather_parent(parent).set_residual_parent(res_parent).set_silu(silu)
        plan = conv.plan(rows_in, n)
        print(f"linear cin={cin} cout={cout} n={n} dtype={dtype}: {plan}", flush=True)
        assert "linear" in plan, plan

    got = gpu_conv(s3dx, x, None, rows_in, w, s3dx.WEIGHT_SLAT, b, dtype, cout, kvol=1, n_out=n,
                   residual=res, setup=setup)
    xs = rnd(s3dx, x, dtype)
    xs = O.repeat_children(xs)[:n] if parent else xs
    h = O.conv(xs, None, n, rnd(s3dx, w, dtype), 0, cout, b, kvol=1)
    if silu:
        h = O.silu(h)
    rr = rnd(s3dx, res, dtype)
    ref = h + (O.repeat_children(rr)[:n] if res_parent else rr)
    check_rel(got, ref, TOL[dtype])


@pytest.mark.parametrize("cin,cout,n,parent,silu,bias", [
    (192, 96, 226120, True, False, True),    # the mesh level-1 skip (parent rows); several blocks a wave
    (256, 128, 28265, False, False, True),   # the SLat out-block skip
    (128, 128, 100003, False, True, False),  # last block of 3 rows; SiLU, no bias
    (64, 8, 33, False, True, True),          # one column block of 8 of 32 columns, a 1-row tail
    (128, 40, 1, False, False, True),        # a single row
    (192, 96, 4099, True, True, True),       # parent rows with a ragged last parent
    (128, 1024, 9503, False, False, True),   # the SLat 128->1024 skip: eight 128-column groups
    (64, 512, 777, False, True, True),       # four groups, SiLU
    (128, 1000, 301, False, False, True),    # eight groups, the last 104 columns wide
])
def test_linear_pipe_kernel(s3dx, O, W, cin, cout, n, parent, silu, bias):
    # BF16 1x1 layers with BF16 output and no residual run the pipelined
    # kernel.  Its rows must match the oracle and the same layer's FP32
    # output rounded to BF16: bit for bit up to four column blocks, where
    # that output comes from the plain linear kernel (same accumulation
    # order); for wider layers, whose FP32 output comes from an MFMA tiling
    # kernel that sums in another order, within BF16 rounding (2^-8
    # relative) of it plus 1e-5 of its largest magnitude for the sums'
    # FP32 differences.
    bf = s3dx.BF16
    rows_in = (n + 7) // 8 if parent else n
    x = W.normal_f32(19, 1, (rows_in, cin))
    w = W.conv_weight(19, 2, cin, cout, kvol=1)
    b = W.normal_f32(19, 3, (cout,)) if bias else None
    conv = s3dx.SparseConv(cin, cout, 1, bf).set_weights(w, s3dx.WEIGHT_SLAT, b)
    conv.set_gather_parent(parent).set_silu(silu)
    plan = conv.plan(rows_in, n)
    print(f"pipe cin={cin} cout={cout} n={n} parent={parent} silu={silu}: {plan}", flush=True)
    assert plan.startswith(("parent-rows linear pipe", "linear pipe")), plan
    xd = to_dev(s3dx, x, bf)
    y = s3dx.DeviceArray((n, cout), np.uint16)
    y32 = s3dx.DeviceArray((n, cout), np.float32)
    conv.run(xd, rows_in, None, n, y, bf)
    conv.run(xd, rows_in, None, n, y32, s3dx.F32)  # the plain kernel (FP32 output)
    got = y.download()
    rows = np.arange(n) if n <= 5000 else np.sort(np.random.default_rng(3).choice(n, 5000, replace=False))
    xs = rnd(s3dx, x, bf)
    xs = xs[rows >> 3] if parent else xs[rows]
    h = O.conv(xs, None, len(rows), rnd(s3dx, w, bf), 0, cout, b, kvol=1)
    if silu:
        h = O.silu(h)
    check_rel(W.bf16_bits_to_f32(got[rows]), h, TOL[bf])
    f32 = y32.download()
    if cout <= 128:
        assert np.array_equal(got, W.f32_to_bf16_bits(f32)), "pipe != plain kernel rounded"
    else:
        d = np.abs(W.bf16_bits_to_f32(got) - f32)
        assert np.all(d <= np.abs(f32) * 2.0 ** -8 + 1e-5 * np.abs(f32).max()), float(d.max())



def test_transform_buffer_regrows(s3dx, O, W):
    # One layer object run on a small, a larger, then the small parent set:
    # the transformed-input buffer grows once and stays valid.
    dtype, cin, cout = 1, 64, 64
    slot = W.normal_f32(8, 2, (8, cin), 0.02)
    w = W.conv_weight(8, 5, cin, cout, layout="mesh")
    conv = (s3dx.SparseConv(cin, cout, 27, dtype).set_weights(w, s3dx.WEIGHT_MESH, None)
            .set_gather_parent(True, slot))
    for radius in (4.0, 7.0, 4.0):
        parents = W.shell_64(res=24, centre=(12.0, 12.0, 12.0), radius=radius)
        p = parents.shape[0]
        _, kmap = O.subdivide2(parents)
        n = 8 * p
        print(f"regrow p={p}", flush=True)
        xp = W.normal_f32(8, int(radius), (p, cin))
        y = s3dx.DeviceArray((n, cout), np.uint16)
        conv.run(s3dx.DeviceArray.from_host(W.f32_to_bf16_bits(xp)), p,
                 s3dx.DeviceArray.from_host(kmap), n, y, dtype)
        h = y.download()
        got = W.bf16_bits_to_f32(h).reshape(h.shape)
        xc = O.repeat_children(rnd(s3dx, xp, dtype)) + np.tile(slot, (p, 1))
        ref = O.conv(rnd(s3dx, xc, dtype), kmap, n, rnd(s3dx, w, dtype), 1, cout, None)
        check_rel(got, ref, TOL[dtype])


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("cout", [128, 160, 101])
def test_layernorm_modulate_silu_residual_epilogue(s3dx, O, W, dtype, cout):
    # cout 128: fused into the MFMA epilogue; 160 and 101: separate LN pass.
    coords = W.shells_union(2)[:2500]
    n = coords.shape[0]
    print(f"ln epilogue dtype={dtype} cout={cout}", flush=True)
    kmap = O.kmap_subm3(coords, n)
    cin = 64
    x = W.normal_f32(7, 1, (n, cin))
    w = W.conv_weight(7, 2, cin, cout)
    b = W.normal_f32(7, 3, (cout,))
    lw, lb = W.normal_f32(7, 4, (cout,)), W.normal_f32(7, 5, (cout,))
    ms, mh = W.normal_f32(7, 6, (cout,), 0.3), W.normal_f32(7, 7, (cout,), 0.3)
    res = W.normal_f32(7, 8, (n, cout))

    def setup(conv):
        conv.set_layernorm(True, 1e-6, lw, lb, ms, mh)
        conv.set_silu(True)

    got = gpu_conv(s3dx, x, kmap, n, w, s3dx.WEIGHT_SLAT, b, dtype, cout, residual=res, setup=setup)
    h = O.conv(rnd(s3dx, x, dtype), kmap, n, rnd(s3dx, w, dtype), 0, cout, b)
    ref = O.silu(O.modulate(O.layernorm(h, 1e-6, lw, lb), ms, mh)) + rnd(s3dx, res, dtype)
    check_rel(got, ref, TOL[dtype])


def test_output_dtype_cross(s3dx, O, W):
    # bf16 arithmetic with fp32 output, and fp32 arithmetic with bf16 output.
    coords = W.shells_union(0)[:1500]
    n = coords.shape[0]
    kmap = O.kmap_subm3(coords, n)
    x = W.normal_f32(8, 1, (n, 128))
    w = W.conv_weight(8, 2, 128, 128)
    b = W.normal_f32(8, 3, (128,))
    ref = O.conv(W.round_bf16(x), kmap, n, W.round_bf16(w), 0, 128, b)
    got = gpu_conv(s3dx, x, kmap, n, w, 0, b, s3dx.BF16, 128, y_dtype=s3dx.F32)
    check_rel(got, ref, 1e-2)
    ref32 = O.conv(x, kmap, n, w, 0, 128, b)
    got2 = gpu_conv(s3dx, x, kmap, n, w, 0, b, s3dx.F32, 128, y_dtype=s3dx.BF16)
    check_rel(got2, ref32, 1e-2)


def test_deterministic_and_empty_rows(s3dx, O, W):
    coords = W.shells_union(0)[:2000]
    n = coords.shape[0]
    kmap = O.kmap_subm3(coords, n)
    kmap[::7] = n  # rows with no neighbour at all (bias only)
    x = W.normal_f32(9, 1, (n, 128))
    w = W.conv_weight(9, 2, 128, 128)
    b = W.normal_f32(9, 3, (128,))
    a1 = gpu_conv(s3dx, x, kmap, n, w, 0, b, s3dx.BF16, 128)
    a2 = gpu_conv(s3dx, x, kmap, n, w, 0, b, s3dx.BF16, 128)
    assert np.array_equal(a1, a2)
    assert np.allclose(a1[::7], W.round_bf16(np.broadcast_to(b, a1[::7].shape)), atol=0)


TILINGS = {  # cout -> tiling ids whose workgroup spans the whole row (11-14, 23, 24: split-K; 20, 21: halo)
    32: ["0", "14", "23", "24"], 64: ["1", "6", "12"], 96: ["2", "7", "13"],
    128: ["3", "8", "10", "11", "18", "20", "21"],
    192: ["4", "9"], 256: ["5"]}


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("cin,cout,tiling", [(c, o, t) for c, o in [(128, 128), (192, 192), (96, 96),
                                                                   (64, 64), (256, 128), (64, 256), (64, 32)]
                                             for t in TILINGS[o]])
def test_row_block_tilings(s3dx, O, W, monkeypatch, dtype, cin, cout, tiling):
    # Every compiled tiling on a tail-heavy row count, with the fused
    # LayerNorm + SiLU + residual epilogue.
    monkeypatch.setenv("S3DX_CONV_TILING", tiling)
    coords = W.shells_union(0)[:2900]
    n = coords.shape[0]
    print(f"tiling {tiling} dtype={dtype} cin={cin} cout={cout}", flush=True)
    kmap = O.kmap_subm3(coords, n)
    x = W.normal_f32(15, 1, (n, cin))
    w = W.conv_weight(15, 2, cin, cout)
    b = W.normal_f32(15, 3, (cout,))
    res = W.normal_f32(15, 4, (n, cout))

    def setup(conv):
        conv.set_layernorm(True, 1e-6)
        conv.set_silu(True)

    got = gpu_conv(s3dx, x, kmap, n, w, s3dx.WEIGHT_SLAT, b, dtype, cout, residual=res, setup=setup)
    h = O.conv(rnd(s3dx, x, dtype), kmap, n, rnd(s3dx, w, dtype), 0, cout, b)
    ref = O.silu(O.layernorm(h, 1e-6)) + rnd(s3dx, res, dtype)
    check_rel(got, ref, TOL[dtype])


@pytest.mark.parametrize("cin,cout,tiling,kvol", [
    (96, 96, "15", 27), (192, 96, "15", 27), (96, 128, "16", 27), (192, 128, "16", 27),
    (160, 96, "15", 27), (224, 128, "16", 27),  # 5 and 7 chunks: the last task is part empty
    (96, 96, "15", 1), (160, 128, "16", 1),     # one task holding an empty sub-task
    (96, 96, "19", 27), (192, 96, "19", 27), (160, 96, "19", 27),  # 15 with 64-row tiles
])
def test_subtask_tilings(s3dx, O, W, monkeypatch, cin, cout, tiling, kvol):
    # Split-K tasks of 128 channels made of 32- or 64-channel chunks (bf16),
    # with the fused LayerNorm + SiLU + residual epilogue.
    monkeypatch.setenv("S3DX_CONV_TILING", tiling)
    dtype = 1
    coords = W.shells_union(1)[:2900]
    n = coords.shape[0]
    kmap = O.kmap_subm3(coords, n) if kvol == 27 else None
    x = W.normal_f32(16, 1, (n, cin))
    w = W.conv_weight(16, 2, cin, cout, kvol=kvol)
    b = W.normal_f32(16, 3, (cout,))
    res = W.normal_f32(16, 4, (n, cout))

    def setup(conv):
        conv.set_layernorm(True, 1e-6)
        conv.set_silu(True)
        plan = conv.plan(n, n)
        print(f"subtask cin={cin} cout={cout} kvol={kvol}: {plan}", flush=True)
        assert plan.startswith(f"mfma tiling={tiling} split-k"), plan

    got = gpu_conv(s3dx, x, kmap, n, w, s3dx.WEIGHT_SLAT, b, dtype, cout, kvol=kvol, residual=res, setup=setup)
    h = O.conv(rnd(s3dx, x, dtype), kmap, n, rnd(s3dx, w, dtype), 0, cout, b, kvol=kvol)
    ref = O.silu(O.layernorm(h, 1e-6)) + rnd(s3dx, res, dtype)
    check_rel(got, ref, TOL[dtype])


@pytest.mark.parametrize("cin,cout,kvol,dtype,with_res", [
    (96, 101, 1, 0, False), (96, 101, 1, 1, True),  # the mesh output head's shape
    (64, 101, 27, 1, True), (64, 100, 27, 0, True), (64, 40, 27, 0, False),
    (64, 104, 27, 1, True), (32, 7, 27, 0, True),   # cout % 8 == 0 (16-byte rows), and a tiny cout
])
def test_padded_cout(s3dx, O, W, cin, cout, kvol, dtype, with_res):
    # Cout not a multiple of 32: zero-padded weight blocks on the MFMA path,
    # only the real columns stored (element stores when rows are not 16-byte
    # aligned).
    coords = W.shells_union(3)[:2600]
    n = coords.shape[0]
    kmap = O.kmap_subm3(coords, n) if kvol == 27 else None
    x = W.normal_f32(17, 1, (n, cin))
    w = W.conv_weight(17, 2, cin, cout, kvol=kvol)
    b = W.normal_f32(17, 3, (cout,))
    res = W.normal_f32(17, 4, (n, cout)) if with_res else None

    def setup(conv):
        plan = conv.plan(n, n)
        print(f"padded cout cin={cin} cout={cout} kvol={kvol} dtype={dtype}: {plan}", flush=True)
        assert plan.startswith(("mfma", "linear")), plan

    got = gpu_conv(s3dx, x, kmap, n, w, s3dx.WEIGHT_SLAT, b, dtype, cout, kvol=kvol, residual=res, setup=setup)
    ref = O.conv(rnd(s3dx, x, dtype), kmap, n, rnd(s3dx, w, dtype), 0, cout, b, kvol=kvol)
    if with_res:
        ref = ref + rnd(s3dx, res, dtype)
    check_rel(got, ref, TOL[dtype])


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [0, 1])
def test_centre_column_not_identity(s3dx, O, W, dtype):
    # The MFMA kernel fetches each tile's first task (the centre offset)
    # assuming kmap[i][13] == i.  Maps that break it -- a permuted centre
    # column, and later duplicates of a coordinate (all-sentinel rows) --
    # must give the same results as the oracle.
    rng = np.random.default_rng(21)
    coords = W.shells_union(2)[:3000]
    dup = np.concatenate([coords, coords[rng.integers(0, coords.shape[0], 200)]], 0)
    for name, c in (("permuted", coords), ("duplicates", dup)):
        n = c.shape[0]
        kmap = O.kmap_subm3(c, n)
        if name == "permuted":
            kmap[:, 13] = np.roll(kmap[:, 13], 5)
        x = W.normal_f32(22, 1, (n, 128))
        w = W.conv_weight(22, 2, 128, 128)
        b = W.normal_f32(22, 3, (128,))
        print(f"centre test {name} dtype={dtype} n={n}", flush=True)
        got = gpu_conv(s3dx, x, kmap, n, w, s3dx.WEIGHT_SLAT, b, dtype, 128)
        ref = O.conv(rnd(s3dx, x, dtype), kmap, n, rnd(s3dx, w, dtype), 0, 128, b)
        check_rel(got, ref, TOL[dtype], name)


@pytest.mark.parametrize("cin,cout,kvol,n,plan", [
    (96, 101, 1, 300001, "in=bf16 linear cols=128 ksteps=6 terms=3"),  # the mesh head, > 2 grid passes
    (128, 96, 1, 4099, "in=bf16 linear cols=96 ksteps=8 terms=3"),
    (32, 20, 1, 777, "in=bf16 linear cols=32 ksteps=2 terms=3"),
    (64, 64, 27, None, "in=bf16 pre=widen mfma"),
    (192, 96, 1, 5000, "in=bf16 pre=widen mfma"),
])
def test_bf16_rows_into_fp32_layer(s3dx, O, W, cin, cout, kvol, n, plan):
    # BF16 rows feeding an FP32 layer.  Widened plans are bit-identical to
    # widening the rows first (exact) and running the same FP32 layer.  The
    # three-term plans multiply on BF16 MFMAs: every product is exact and
    # the sums are FP32, so they stay within 1e-6 (rel-L2) of a float64
    # reference, like the FP32 kernel; dropping the smallest weight term
    # alone gives ~1e-5.  The weights span 2^-20 .. 2^20 so that every term
    # carries bits.
    coords = W.shells_union(2)[:3000] if kvol == 27 else None
    n = coords.shape[0] if kvol == 27 else n
    kmap = O.kmap_subm3(coords, n) if kvol == 27 else None
    xb = W.f32_to_bf16_bits(W.normal_f32(41, 1, (n, cin)))
    w = W.conv_weight(41, 2, cin, cout, kvol=kvol)
    if kvol == 1:
        w = (w * np.exp2(np.random.default_rng(43).integers(-20, 21, w.shape))).astype(np.float32)
    b = W.normal_f32(41, 3, (cout,))
    conv_b = s3dx.SparseConv(cin, cout, kvol, s3dx.F32).set_weights(w, s3dx.WEIGHT_SLAT, b).set_input_dtype(s3dx.BF16)
    got_plan = conv_b.plan(n, n)
    print(f"bf16 rows -> fp32 cin={cin} cout={cout} kvol={kvol} n={n}: {got_plan}", flush=True)
    assert got_plan.startswith(plan), got_plan
    conv_f = s3dx.SparseConv(cin, cout, kvol, s3dx.F32).set_weights(w, s3dx.WEIGHT_SLAT, b)
    dk = s3dx.DeviceArray.from_host(kmap) if kmap is not None else None
    y1 = s3dx.DeviceArray((n, cout), np.float32)
    y2 = s3dx.DeviceArray((n, cout), np.float32)
    conv_b.run(s3dx.DeviceArray.from_host(xb), n, dk, n, y1, s3dx.F32)
    conv_f.run(s3dx.DeviceArray.from_host(W.bf16_bits_to_f32(xb)), n, dk, n, y2, s3dx.F32)
    g1, g2 = y1.download(), y2.download()
    if "terms=3" not in plan:
        assert np.array_equal(g1, g2)
        return
    ref = W.bf16_bits_to_f32(xb).astype(np.float64) @ w.reshape(cout, cin).astype(np.float64).T + b
    e1, e2 = rel_l2(g1, ref), rel_l2(g2, ref)
    print(f"  rel-L2 vs float64: three-term {e1:.3g}, FP32 kernel {e2:.3g}", flush=True)
    assert e1 <= 1e-6 and e2 <= 1e-6


@pytest.mark.parametrize("y_dtype", [0, 1])
@pytest.mark.parametrize("cin,cout,p", [(64, 96, 1001), (128, 128, 333), (32, 101, 77), (64, 64, 5)])
def test_bf16_rows_three_term_epilogue(s3dx, W, y_dtype, cin, cout, p):
    # The three-term kernel's epilogue: parent rows (row i reads x[i >> 3]),
    # SiLU, a per-parent residual, FP32 or BF16 output, and a last block
    # shorter than 32 rows (8 * p rows).  Reference: float64.
    n = 8 * p
    xb = W.f32_to_bf16_bits(W.normal_f32(47, 1, (p, cin)))
    w = W.conv_weight(47, 2, cin, cout, kvol=1)
    b = W.normal_f32(47, 3, (cout,))
    res = W.normal_f32(47, 4, (p, cout))
    if y_dtype == s3dx.BF16:
        res = W.round_bf16(res)
    conv = (s3dx.SparseConv(cin, cout, 1, s3dx.F32).set_weights(w, s3dx.WEIGHT_SLAT, b)
            .set_input_dtype(s3dx.BF16).set_gather_parent(True).set_silu(True).set_residual_parent(True))
    plan = conv.plan(p, n)
    print(f"three-term epilogue cin={cin} cout={cout} p={p} y_dtype={y_dtype}: {plan}", flush=True)
    assert "terms=3" in plan and "parent-rows" in plan, plan
    y = s3dx.DeviceArray((n, cout), np.uint16 if y_dtype == s3dx.BF16 else np.float32)
    dr = s3dx.DeviceArray.from_host(W.f32_to_bf16_bits(res) if y_dtype == s3dx.BF16 else res)
    conv.run(s3dx.DeviceArray.from_host(xb), p, None, n, y, y_dtype, dr)
    got = from_dev(s3dx, y, y_dtype)
    h = W.bf16_bits_to_f32(xb).astype(np.float64) @ w.reshape(cout, cin).astype(np.float64).T + b
    h = h / (1.0 + np.exp(-h)) + res
    ref = np.repeat(h, 8, axis=0)
    check_rel(got, ref, 1e-6 if y_dtype == s3dx.F32 else 4e-3)


# FP32 split-K layers with long tiles (at least 256 tasks a tile) that take
# more than one pass over the CUs run in stream-K runs: equal runs of
# (column group, tile, task) units, two per CU, and a pass that adds the
# pieces of tiles split between runs.  Forced run counts cut tiles in many
# places (runs inside a tile, across several, the tail tile); the fused
# LayerNorm + SiLU, the residual and a LayerNorm pass over 512 columns come
# after the pieces are added.  FP32 gate against the oracle on sampled rows,
# the same bits on a second launch, and the 5,086-row 1024 -> 1024 layer
# picks the runs by itself.
SPLITK_STREAM_K = {
    # name: (set, cin, cout, LayerNorm+SiLU, residual, runs); "fine": the
    # 28,265-row config-2 set, "coarse": its 5,086 coarse rows (tail tile of 30)
    "fine_cin512_ln_300runs": ("fine", 512, 128, True, False, 300),
    "fine_cin512_res_97runs": ("fine", 512, 128, False, True, 97),
    "coarse_cin512_cout1024_res_1000runs": ("coarse", 512, 1024, False, True, 1000),  # runs inside tiles
    "coarse_cin512_cout512_ln_7runs": ("coarse", 512, 512, True, True, 7),  # LayerNorm as its own pass
}


@pytest.mark.parametrize("case", list(SPLITK_STREAM_K))
def test_splitk_stream_k_runs(s3dx, O, W, monkeypatch, case):
    which, cin, cout, ln, with_res, runs = SPLITK_STREAM_K[case]
    coords = W.shells_union(0)
    if which == "coarse":
        nc, coarse, _, _, _ = O.coarsen2(coords)
        coords = np.ascontiguousarray(coarse[:nc])
    n = coords.shape[0]
    kmap = O.kmap_subm3(coords, n)
    seed = 70 + runs % 50
    w, b = W.conv_weight(seed, 2, cin, cout), W.normal_f32(seed, 3, (cout,), 0.1)
    conv = s3dx.SparseConv(cin, cout, 27, s3dx.F32).set_weights(w, s3dx.WEIGHT_SLAT, b)
    if ln:
        conv.set_layernorm(True, 1e-6).set_silu(True)
    x = W.normal_f32(seed, 1, (n, cin))
    res = W.normal_f32(seed, 6, (n, cout)) if with_res else None
    xd, kd = to_dev(s3dx, x, s3dx.F32), s3dx.DeviceArray.from_host(kmap)
    rd = to_dev(s3dx, res, s3dx.F32) if with_res else None
    monkeypatch.setenv("S3DX_STREAM_K_RUNS", str(runs))
    plan = conv.plan(n, n)
    print(f"{case}: {plan}", flush=True)
    assert plan.startswith("mfma tiling=18 split-k stream-k rows=64") and f"grid={runs}x1" in plan, plan
    y1, y2 = s3dx.DeviceArray((n, cout), np.float32), s3dx.DeviceArray((n, cout), np.float32)
    conv.run(xd, n, kd, n, y1, s3dx.F32, rd)
    conv.run(xd, n, kd, n, y2, s3dx.F32, rd)
    assert np.array_equal(y1.download(), y2.download()), "stream-K runs differ between launches"
    rows = np.sort(np.concatenate([np.random.default_rng(seed).choice(n - 64, 300, replace=False), np.arange(n - 64, n)]))
    h = O.conv(x, kmap[rows], n, w, 0, cout, b)
    if ln:
        h = O.silu(O.layernorm(h, 1e-6))
    if with_res:
        h = h + res[rows]
    check_rel(y1.download()[rows], h, TOL[0], case)


def test_splitk_stream_k_config3_fp32(s3dx, O, W, monkeypatch):
    fine = W.shells_union(0)
    nc, coarse, _, _, _ = O.coarsen2(fine)
    coarse = np.ascontiguousarray(coarse[:nc])
    kmap = O.kmap_subm3(coarse, nc)
    c = 1024
    w = W.conv_weight(0, 311, c, c)
    conv = s3dx.SparseConv(c, c, 27, s3dx.F32).set_weights(w, s3dx.WEIGHT_SLAT, None)
    plan = conv.plan(nc, nc)
    print(f"FP32 config 3: {plan}", flush=True)
    assert plan.startswith("mfma tiling=18 split-k stream-k rows=64 cols=128") and plan.endswith("grid=512x1"), plan
    x = W.normal_f32(0, 310, (nc, c))
    xd, kd = to_dev(s3dx, x, s3dx.F32), s3dx.DeviceArray.from_host(kmap)
    y = s3dx.DeviceArray((nc, c), np.float32)
    conv.run(xd, nc, kd, nc, y, s3dx.F32)
    rows = np.sort(np.random.default_rng(5).choice(nc, 300, replace=False))
    check_rel(y.download()[rows], O.conv(x, kmap[rows], nc, w, 0, c, None), TOL[0], "FP32 1024 -> 1024 stream-K")
    monkeypatch.setenv("S3DX_STREAM_K", "0")
    assert not " stream-k" in conv.plan(nc, nc)
