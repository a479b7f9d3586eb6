"""GPU row ops (LayerNorm, GroupNorm statistics, affine+SiLU, SLat
down/upsample, conversions) against the oracle."""
import numpy as np
import pytest

from helpers import check_rel, rel_l2

pytestmark = pytest.mark.gpu


def dev(s3dx, a):
    return s3dx.DeviceArray.from_host(np.ascontiguousarray(a))


@pytest.mark.parametrize("c", [128, 96, 2048, 101])
def test_layernorm_rows(s3dx, O, W, c):
    n = 1000
    x = W.normal_f32(11, 1, (n, c), 2.0) + 0.5
    w, b = W.normal_f32(11, 2, (c,)), W.normal_f32(11, 3, (c,))
    ms, mh = W.normal_f32(11, 4, (c,)), W.normal_f32(11, 5, (c,))
    y = s3dx.DeviceArray((n, c), np.float32)
    s3dx.layernorm_rows(dev(s3dx, x), s3dx.F32, n, c, 1e-6, dev(s3dx, w), dev(s3dx, b),
                        dev(s3dx, ms), dev(s3dx, mh), True, y, s3dx.F32)
    ref = O.silu(O.modulate(O.layernorm(x, 1e-6, w, b), ms, mh))
    check_rel(y.download(), ref, 1e-5)
    # bf16 in, bf16 out, in place, no affine
    xb = dev(s3dx, W.f32_to_bf16_bits(x))
    s3dx.layernorm_rows(xb, s3dx.BF16, n, c, 1e-6)
    got = W.bf16_bits_to_f32(xb.download()).reshape(n, c)
    check_rel(got, O.layernorm(W.round_bf16(x), 1e-6), 1e-2)


@pytest.mark.parametrize("xd,yd,c", [
    (1, 1, 128), (1, 1, 256), (1, 1, 1024), (1, 1, 2048), (1, 1, 4096), (1, 1, 96), (1, 1, 6144),
    (0, 0, 128), (0, 0, 2048), (0, 1, 1024), (1, 0, 192), (0, 0, 20), (1, 1, 24)])
def test_layernorm_rows_vector_path(s3dx, O, W, xd, yd, c):
    # Out of place with 16-byte aligned rows: the register-resident kernel
    # (2^k lanes per row, 1-8 pieces per lane, several rows per wave for
    # narrow rows); rows wider than 512 pieces (BF16 6144) or not whole
    # pieces (FP32 20) take the element kernel.  Row count not a multiple of
    # the rows per block.  norm1's affine + SiLU, then the modulate form.
    n = 3001
    x = W.normal_f32(12, c, (n, c), 2.0) + 0.5
    w, b = W.normal_f32(12, 2, (c,)), W.normal_f32(12, 3, (c,))
    ms, mh = W.normal_f32(12, 4, (c,)), W.normal_f32(12, 5, (c,))
    store = {0: np.float32, 1: np.uint16}
    xin = W.f32_to_bf16_bits(x) if xd == 1 else x
    xr = W.round_bf16(x) if xd == 1 else x
    host = (lambda d: W.bf16_bits_to_f32(d.download()).reshape(n, c)) if yd == 1 else (lambda d: d.download())
    tol = 1e-2 if yd == 1 else 1e-5
    print(f"layernorm vector path x={xd} y={yd} c={c}", flush=True)
    dx = dev(s3dx, xin)
    y = s3dx.DeviceArray((n, c), store[yd])
    s3dx.layernorm_rows(dx, xd, n, c, 1e-6, dev(s3dx, w), dev(s3dx, b), silu=True, y=y, y_dtype=yd)
    check_rel(host(y), O.silu(O.layernorm(xr, 1e-6, w, b)), tol, "affine + SiLU")
    s3dx.layernorm_rows(dx, xd, n, c, 1e-6, None, None, dev(s3dx, ms), dev(s3dx, mh), y=y, y_dtype=yd)
    check_rel(host(y), O.modulate(O.layernorm(xr, 1e-6), ms, mh), tol, "modulate")


@pytest.mark.parametrize("n,c,groups,mean,std", [
    (5000, 96, 32, 2.0, 1.5), (40000, 192, 32, 2.0, 1.5), (3000, 768, 32, 2.0, 1.5),
    (20000, 96, 32, 300.0, 0.05),  # |mean| >> std: the shifted sums keep the variance
    (700, 36, 4, 1.0, 1.0),        # rows not whole 16-byte pieces: per-element loads
    (3, 64, 32, 0.0, 1.0),         # fewer rows than blocks
    (2000, 1024, 2, 1.0, 1.0),     # 512 channels a group: totals in two chunks of 256
    (500, 300, 1, 1.0, 1.0),       # 300 channels a group: a partial second chunk
])
def test_groupnorm_stats_and_affine(s3dx, O, W, n, c, groups, mean, std):
    x = W.normal_f32(12, 1, (n, c), std) + W.normal_f32(12, 2, (c,), 2.0) + np.float32(mean)
    x = x.astype(np.float32)
    g, b = W.normal_f32(12, 3, (c,)), W.normal_f32(12, 4, (c,))
    dx = dev(s3dx, x)
    scale, shift, _ = s3dx.groupnorm_stats(dx, s3dx.F32, n, c, groups, 1e-5, dev(s3dx, g), dev(s3dx, b))
    y = s3dx.DeviceArray((n, c), np.float32)
    s3dx.affine_rows(dx, s3dx.F32, n, c, scale, shift, True, y, s3dx.F32)
    ref = O.silu(O.groupnorm(x, groups, 1e-5, g, b))
    check_rel(y.download(), ref, 1e-5)


@pytest.mark.parametrize("n,c", [(30000, 768), (100000, 96), (999, 40)])
def test_groupnorm_stats_bf16_input(s3dx, O, W, n, c):
    # bf16 rows: statistics of the stored (rounded) values, in float.
    x = W.round_bf16(W.normal_f32(14, 1, (n, c), 1.5) + W.normal_f32(14, 2, (c,), 2.0))
    g, b = W.normal_f32(14, 3, (c,)), W.normal_f32(14, 4, (c,))
    dx = dev(s3dx, W.f32_to_bf16_bits(x))
    scale, shift, _ = s3dx.groupnorm_stats(dx, s3dx.BF16, n, c, 8, 1e-5, dev(s3dx, g), dev(s3dx, b))
    y = s3dx.DeviceArray((n, c), np.float32)
    s3dx.affine_rows(dx, s3dx.BF16, n, c, scale, shift, False, y, s3dx.F32)
    ref = O.groupnorm(x, 8, 1e-5, g, b)
    check_rel(y.download(), ref, 1e-5)


@pytest.mark.parametrize("dtype,c", [(0, 64), (1, 64), (1, 128), (0, 20), (1, 20), (0, 6)])
def test_down_up_sample(s3dx, O, W, dtype, c):
    # Rows of whole 16-byte pieces take the vector path (FP32 64/20, BF16
    # 64/128), the others one element per thread.  Children are summed in
    # order in FP32, as the oracle does: results are bit-identical (BF16 after
    # one rounding of the oracle's FP32 value).
    coords = W.shells_union(0)
    n = coords.shape[0]
    nc, cc, f2c, ch, inv = s3dx.coarsen2(dev(s3dx, coords), n)
    print(f"down/up dtype={dtype} c={c} n={n} nc={nc}", flush=True)
    x = W.normal_f32(13, 1, (n, c))
    bf = dtype == s3dx.BF16
    xr = W.round_bf16(x) if bf else x
    dx = dev(s3dx, W.f32_to_bf16_bits(x) if bf else x)
    store = np.uint16 if bf else np.float32
    host = (lambda d: W.bf16_bits_to_f32(d.download())) if bf else (lambda d: d.download())
    down = s3dx.DeviceArray((nc, c), store)
    s3dx.downsample_mean(dx, dtype, n, c, ch, inv, nc, down)
    ref = O.downsample_mean(xr, ch.download()[: 8 * nc], inv.download()[:nc], nc)
    assert np.array_equal(host(down), W.round_bf16(ref) if bf else ref)
    up = s3dx.DeviceArray((n, c), store)
    s3dx.upsample_nearest(down, dtype, nc, c, f2c, n, up)
    assert np.array_equal(host(up), O.upsample_nearest(host(down), f2c.download()))


@pytest.mark.parametrize("count", [4096, 4099, 13, 40_000_003])
def test_convert_roundtrip(s3dx, W, count):
    # 8-element vector steps plus a scalar tail; 40M elements also runs more
    # than one grid-stride pass.
    x = W.normal_f32(14, 1, (count,), 100.0)
    d = dev(s3dx, x)
    b = s3dx.DeviceArray((count,), np.uint16)
    s3dx.convert(d, s3dx.F32, count, b, s3dx.BF16)
    assert np.array_equal(b.download(), W.f32_to_bf16_bits(x))
    back = s3dx.DeviceArray((count,), np.float32)
    s3dx.convert(b, s3dx.BF16, count, back, s3dx.F32)
    assert np.array_equal(back.download(), W.round_bf16(x))
    same = s3dx.DeviceArray((count,), np.float32)
    s3dx.convert(back, s3dx.F32, count, same, s3dx.F32)
    assert np.array_equal(same.download(), back.download())


@pytest.mark.parametrize("dtype,ca,cb", [(1, 1024, 1024), (1, 128, 128), (0, 128, 128), (1, 24, 8), (0, 5, 3)])
@pytest.mark.parametrize("gather", [False, True])
def test_concat_rows(s3dx, W, dtype, ca, cb, gather):
    # The SLat out blocks' ggml_concat (slat_flow_graph.cpp:443, 477): with a
    # row index (fine_to_coarse) it is out_blocks.0's concat + upsample in one
    # pass.  Bit-exact against numpy; indices outside the source give zero rows.
    coords = W.shells_union(1)
    n = coords.shape[0]
    nc, cc, f2c, ch, inv = s3dx.coarsen2(dev(s3dx, coords), n)
    src = nc if gather else n
    store = np.uint16 if dtype == s3dx.BF16 else np.float32
    a = W.normal_f32(15, ca, (src, ca))
    b = W.normal_f32(16, cb, (src, cb))
    if dtype == s3dx.BF16:
        a, b = W.f32_to_bf16_bits(a), W.f32_to_bf16_bits(b)
    rows = f2c.download().copy() if gather else None
    if gather:
        rows[::97] = -1
        rows[1::89] = nc
    print(f"concat dtype={dtype} {ca}+{cb} gather={gather} rows={n}", flush=True)
    y = s3dx.DeviceArray((n, ca + cb), store)
    s3dx.concat_rows(dev(s3dx, a), ca, dev(s3dx, b), cb, dtype, src,
                     dev(s3dx, rows) if gather else None, n, y)
    want = np.concatenate([a, b], 1)
    if gather:
        ok = (rows >= 0) & (rows < nc)
        want = np.where(ok[:, None], want[np.clip(rows, 0, nc - 1)], 0).astype(store)
    assert np.array_equal(y.download(), want)
