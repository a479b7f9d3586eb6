"""The halo-staged BF16 conv kernels and per-map gather plans.

A halo tile stages each distinct source row of its 64 (or 128) output rows
once per 64-channel chunk into LDS; a tile whose rows reach more distinct
source rows than its LDS holds reads them from memory instead (global mode).
A gather plan (s3dx_gather_plan_create) precomputes each 64-row tile's
distinct rows and slot table once per map; s3dx_conv_run_planned then skips
that step.  A planned run must equal the unplanned run bit for bit (same
kernel body, same summation order), on tiles of either mode and on the tail
tile, and both meet the BF16 gate (rel-L2 1e-2) against the float64 oracle.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import check_rel

pytestmark = pytest.mark.gpu


def _bf(s3dx, W, a):
    return s3dx.DeviceArray.from_host(W.f32_to_bf16_bits(np.ascontiguousarray(a, np.float32)))


def _host(W, d):
    h = d.download()
    return W.bf16_bits_to_f32(h).reshape(h.shape)


def _dense_cube(side, shuffle_from=None, seed=0):
    """A dense side^3 cube, batch 0, x-major; rows [shuffle_from:] shuffled,
    so their tiles reach ~27 distinct source rows per output row."""
    g = np.stack(np.meshgrid(*(np.arange(side),) * 3, indexing="ij"), -1).reshape(-1, 3)
    c = np.concatenate([np.zeros((len(g), 1), np.int64), g], 1).astype(np.int32)
    if shuffle_from is not None:
        rng = np.random.default_rng(seed)
        tail = c[shuffle_from:].copy()
        rng.shuffle(tail)
        c[shuffle_from:] = tail
    return np.ascontiguousarray(c)


def _layer(s3dx, W, cin, cout, seed, ln):
    conv = (s3dx.SparseConv(cin, cout, 27, s3dx.BF16)
            .set_weights(W.conv_weight(seed, 2, cin, cout), s3dx.WEIGHT_SLAT, W.normal_f32(seed, 3, (cout,), 0.1)))
    if ln:
        conv.set_layernorm(True, 1e-6).set_silu(True)
    return conv


def _oracle(O, W, x, kmap, n, cin, cout, seed, ln, res=None):
    h = O.conv(x, kmap, n, W.round_bf16(W.conv_weight(seed, 2, cin, cout)), 0, cout, W.normal_f32(seed, 3, (cout,), 0.1))
    if ln:
        h = O.silu(O.layernorm(h, 1e-6))
    return h + res if res is not None else h


def _sparse_points(step, pair):
    """Points on a lattice of `step` (no neighbours: one present offset per
    tile), or (pair) z-adjacent pairs (three present offsets)."""
    g = np.stack(np.meshgrid(*(np.arange(0, 60, step),) * 3, indexing="ij"), -1).reshape(-1, 3)
    if pair:
        g = np.concatenate([g, g + np.array([0, 0, 1])])
        g = g[np.lexsort((g[:, 2], g[:, 1], g[:, 0]))]
    c = np.concatenate([np.zeros((len(g), 1), np.int64), g], 1).astype(np.int32)
    return np.ascontiguousarray(c)


CASES = {
    # name: (coords builder, cin, cout, LayerNorm+SiLU+residual)
    "isolated_points_cin256": (lambda W: _sparse_points(3, False), 256, 128, True),  # fewer tasks than in flight
    # one offset and one or two chunks: fewer weight loads than the wait
    # before chunk 0 counts on (the copy must still have landed)
    "isolated_points_cin128": (lambda W: _sparse_points(3, False), 128, 128, True),
    "isolated_points_cin64": (lambda W: _sparse_points(3, False), 64, 128, False),
    "point_pairs_cin256": (lambda W: _sparse_points(4, True), 256, 128, False),
    "shells_union_28265": (lambda W: W.shells_union(0), 128, 128, True),
    "shells_union_3000_cin256": (lambda W: W.shells_union(1)[:3000], 256, 128, False),
    "shuffled_cube_13824": (lambda W: _dense_cube(24, 0), 128, 128, True),          # every tile global
    "half_shuffled_cube_13824": (lambda W: _dense_cube(24, 6912), 128, 128, False),  # both modes
    "tiny_37": (lambda W: W.shells_union(2)[:37], 128, 128, True),                   # one partial tile
    # one chunk (the first chunk is the last), an odd chunk count, two column groups
    "shells_union_28265_cin64": (lambda W: W.shells_union(0), 64, 128, True),
    "shells_union_3000_cin192": (lambda W: W.shells_union(1)[:3000], 192, 128, True),
    "shells_union_3000_cout256": (lambda W: W.shells_union(1)[:3000], 128, 256, False),
}


@pytest.mark.parametrize("case", list(CASES))
def test_planned_run_equals_unplanned(s3dx, O, W, monkeypatch, case):
    monkeypatch.delenv("S3DX_CONV_TILING", raising=False)
    monkeypatch.delenv("S3DX_CONV_HALO", raising=False)
    build, cin, cout, ln = CASES[case]
    coords = build(W)
    n = coords.shape[0]
    kmap = O.kmap_subm3(coords, n)
    conv = _layer(s3dx, W, cin, cout, 40, ln)
    plan_text = conv.plan(n, n)
    print(f"{case} n={n}: {plan_text}", flush=True)
    assert plan_text.startswith("mfma tiling=21 split-k halo rows=64"), plan_text
    x = W.round_bf16(W.normal_f32(40, 1, (n, cin)))
    res = W.round_bf16(W.normal_f32(40, 4, (n, cout))) if ln else None
    xd, kd = _bf(s3dx, W, x), s3dx.DeviceArray.from_host(kmap)
    rd = _bf(s3dx, W, res) if ln else None
    gp = conv.gather_plan(n, kd, n)
    planned = conv.plan(n, n, gp)
    print(f"  planned: {planned}", flush=True)
    # one pass of 128-row tiles over the CUs: the 8-wave kernel
    assert planned.startswith("mfma tiling=22 split-k halo rows=128") and planned.endswith("plan=128"), planned
    y0 = s3dx.DeviceArray((n, cout), np.uint16)
    y1 = s3dx.DeviceArray((n, cout), np.uint16)
    conv.run(xd, n, kd, n, y0, s3dx.BF16, rd)
    conv.run(xd, n, kd, n, y1, s3dx.BF16, rd, plan=gp)
    a, b = y0.download(), y1.download()
    assert np.array_equal(a, b), f"planned run differs in {(a != b).sum()} of {a.size} values"
    # The plan serves every layer over the same map and source rows.
    other = _layer(s3dx, W, cin, cout, 41, False)
    other.run(xd, n, kd, n, y0, s3dx.BF16)
    other.run(xd, n, kd, n, y1, s3dx.BF16, plan=gp)
    assert np.array_equal(y0.download(), y1.download())
    check_rel(_host(W, y1), _oracle(O, W, x, kmap, n, cin, cout, 41, False), 1e-2, f"{case} (second layer)")
    # with a residual and no LayerNorm (the 8-wave kernel then finishes each
    # column half on its own)
    res2 = W.round_bf16(W.normal_f32(41, 4, (n, cout)))
    rd2 = _bf(s3dx, W, res2)
    other.run(xd, n, kd, n, y0, s3dx.BF16, rd2)
    other.run(xd, n, kd, n, y1, s3dx.BF16, rd2, plan=gp)
    assert np.array_equal(y0.download(), y1.download())
    check_rel(_host(W, y1), _oracle(O, W, x, kmap, n, cin, cout, 41, False, res2), 1e-2,
              f"{case} (second layer + residual)")
    conv.run(xd, n, kd, n, y1, s3dx.BF16, rd, plan=gp)
    check_rel(_host(W, y1), _oracle(O, W, x, kmap, n, cin, cout, 40, ln, res), 1e-2, case)


def test_planned_config3_rows(s3dx, O, W, monkeypatch):
    # 1024 -> 1024 on the 5,086 coarse rows.  40 x 8 128-row tiles are more
    # than the CUs: the planned run takes stream-K runs of the 8-wave kernel
    # (equal runs of (column group, tile, chunk) units, one per CU), the same
    # bits on every run and within BF16 rounding of the oracle.  With
    # stream-K off it takes 64-row records and equals the unplanned run bit
    # for bit, as every other planned run does.
    fine = W.shells_union(0)
    nc, coarse, _, _, _ = O.coarsen2(fine)
    coarse = np.ascontiguousarray(coarse[:nc])
    kmap = O.kmap_subm3(coarse, nc)
    c = 1024
    w = W.conv_weight(0, 301, c, c)
    conv = s3dx.SparseConv(c, c, 27, s3dx.BF16).set_weights(w, s3dx.WEIGHT_SLAT, None)
    x = W.round_bf16(W.normal_f32(0, 300, (nc, c)))
    xd, kd = _bf(s3dx, W, x), s3dx.DeviceArray.from_host(kmap)
    gp = conv.gather_plan(nc, kd, nc)
    planned = conv.plan(nc, nc, gp)
    print(f"config 3 planned: {planned}", flush=True)
    assert planned.startswith("mfma tiling=22 split-k halo stream-k rows=128 cols=128") and \
        planned.endswith(" plan=128"), planned
    y0, y1, y2 = (s3dx.DeviceArray((nc, c), np.uint16) for _ in range(3))
    conv.run(xd, nc, kd, nc, y0, s3dx.BF16)
    conv.run(xd, nc, kd, nc, y1, s3dx.BF16, plan=gp)
    conv.run(xd, nc, kd, nc, y2, s3dx.BF16, plan=gp)
    assert np.array_equal(y1.download(), y2.download()), "stream-K runs differ between launches"
    rows = np.sort(np.random.default_rng(3).choice(nc, 600, replace=False))
    ref = O.conv(x, kmap[rows], nc, W.round_bf16(w), 0, c, None)
    check_rel(_host(W, y1)[rows], ref, 1e-2, "config 3 stream-K")
    check_rel(_host(W, y0)[rows], ref, 1e-2, "config 3 unplanned")
    monkeypatch.setenv("S3DX_STREAM_K", "0")
    gp64 = conv.gather_plan(nc, kd, nc)
    planned = conv.plan(nc, nc, gp64)
    assert planned.startswith("mfma tiling=21 split-k halo rows=64") and planned.endswith("grid=80x8 plan=64"), planned
    conv.run(xd, nc, kd, nc, y2, s3dx.BF16, plan=gp64)
    assert np.array_equal(y0.download(), y2.download())


# Stream-K runs forced to a run count that cuts tiles at many places: runs
# that end mid-tile, runs covering several whole tiles, runs that fall
# inside one tile (a tile in four or more pieces), tiles in global-gather
# mode, two column groups with a residual, and the LayerNorm + modulate +
# SiLU epilogue after the pieces are added.  Each against the float64 oracle
# on sampled rows, and the same bits on a second launch.
STREAM_K = {
    # name: (coords builder, cin, cout, LayerNorm+modulate+SiLU, residual, runs, FP32 output)
    "shells_3000_cin512_ln_7runs": (lambda W: W.shells_union(1)[:3000], 512, 128, True, False, 7, False),
    "shells_3000_cin512_cout256_res_13runs": (lambda W: W.shells_union(1)[:3000], 512, 256, False, True, 13, False),
    "shells_3000_cin1024_100runs": (lambda W: W.shells_union(1)[:3000], 1024, 128, False, False, 100, False),
    "shuffled_cube_13824_cin512_ln_9runs": (lambda W: _dense_cube(24, 0), 512, 128, True, True, 9, False),
    "tiny_200_cin1024_res_3runs": (lambda W: W.shells_union(2)[:200], 1024, 128, False, True, 3, False),
    # FP32 rows out of both passes: a LayerNorm wider than the tile (its own
    # pass over the conv's FP32 rows), and FP32 output asked of a BF16 layer
    "shells_3000_cin512_cout512_ln_11runs": (lambda W: W.shells_union(1)[:3000], 512, 512, True, True, 11, False),
    "shells_3000_cin768_f32out_res_17runs": (lambda W: W.shells_union(1)[:3000], 768, 128, False, True, 17, True),
}


@pytest.mark.parametrize("case", list(STREAM_K))
def test_stream_k_runs(s3dx, O, W, monkeypatch, case):
    build, cin, cout, ln, with_res, runs, f32_out = STREAM_K[case]
    coords = build(W)
    n = coords.shape[0]
    kmap = O.kmap_subm3(coords, n)
    seed = 90 + runs
    w, b = W.conv_weight(seed, 2, cin, cout), W.normal_f32(seed, 3, (cout,), 0.1)
    conv = s3dx.SparseConv(cin, cout, 27, s3dx.BF16).set_weights(w, s3dx.WEIGHT_SLAT, b)
    scale, shift = W.normal_f32(seed, 4, (cout,), 0.3), W.normal_f32(seed, 5, (cout,), 0.3)
    if ln:
        conv.set_layernorm(True, 1e-6).set_modulate(s3dx.DeviceArray.from_host(scale),
                                                     s3dx.DeviceArray.from_host(shift)).set_silu(True)
    x = W.round_bf16(W.normal_f32(seed, 1, (n, cin)))
    res = W.round_bf16(W.normal_f32(seed, 6, (n, cout))) if with_res else None
    xd, kd = _bf(s3dx, W, x), s3dx.DeviceArray.from_host(kmap)
    # (the residual comes in the output's dtype)
    rd = None if not with_res else (s3dx.DeviceArray.from_host(np.ascontiguousarray(res, np.float32)) if f32_out
                                    else _bf(s3dx, W, res))
    monkeypatch.setenv("S3DX_STREAM_K_RUNS", str(runs))
    gp = conv.gather_plan(n, kd, n)
    plan = conv.plan(n, n, gp)
    print(f"{case}: {plan}", flush=True)
    assert " stream-k " in plan and f"grid={runs}x1" in plan and plan.endswith(" plan=128"), plan
    ydt, ystore = (s3dx.F32, np.float32) if f32_out else (s3dx.BF16, np.uint16)
    y1, y2 = s3dx.DeviceArray((n, cout), ystore), s3dx.DeviceArray((n, cout), ystore)
    conv.run(xd, n, kd, n, y1, ydt, rd, plan=gp)
    conv.run(xd, n, kd, n, y2, ydt, rd, plan=gp)
    assert np.array_equal(y1.download(), y2.download()), "stream-K runs differ between launches"
    rows = np.sort(np.random.default_rng(seed).choice(n, min(n, 500), replace=False))
    h = O.conv(x, kmap[rows], n, W.round_bf16(w), 0, cout, b)
    if ln:
        h = O.silu(O.modulate(O.layernorm(h, 1e-6), scale, shift))
    if with_res:
        h = h + res[rows]
    got = y1.download() if f32_out else _host(W, y1)
    check_rel(got[rows], h, 1e-2, case)


# Layers whose columns come in 96 but not 128 (the mesh decoder's 192 and 96
# outputs) run 64-row, 96-column halo tiles: the three owning waves and the
# fourth, which only hands its partials over.
COLS96 = {
    "shells_3000_cin192_cout192": (lambda W: W.shells_union(1)[:3000], 192, 192),
    "shells_3000_cin64_cout96": (lambda W: W.shells_union(1)[:3000], 64, 96),
    "shells_28265_cin128_cout192": (lambda W: W.shells_union(0), 128, 192),
    "shuffled_cube_13824_cout96": (lambda W: _dense_cube(24, 0), 128, 96),          # every tile global
    "half_shuffled_cube_13824_cout192": (lambda W: _dense_cube(24, 6912), 64, 192),  # both modes
    "tiny_37_cout96": (lambda W: W.shells_union(2)[:37], 128, 96),
}


@pytest.mark.parametrize("case", list(COLS96))
def test_96_column_tiles(s3dx, O, W, monkeypatch, case):
    monkeypatch.delenv("S3DX_CONV_TILING", raising=False)
    monkeypatch.delenv("S3DX_CONV_HALO", raising=False)
    monkeypatch.delenv("S3DX_PLAN_ROWS", raising=False)
    build, cin, cout = COLS96[case]
    coords = build(W)
    n = coords.shape[0]
    kmap = O.kmap_subm3(coords, n)
    conv = _layer(s3dx, W, cin, cout, 46, False)
    x = W.round_bf16(W.normal_f32(46, 1, (n, cin)))
    res = W.round_bf16(W.normal_f32(46, 4, (n, cout)))
    xd, kd, rd = _bf(s3dx, W, x), s3dx.DeviceArray.from_host(kmap), _bf(s3dx, W, res)
    gp = conv.gather_plan(n, kd, n)
    plan_text, planned = conv.plan(n, n), conv.plan(n, n, gp)
    print(f"{case} n={n}: {plan_text} | {planned}", flush=True)
    assert plan_text.startswith("mfma tiling=21 split-k halo rows=64 cols=96"), plan_text
    assert planned.endswith(f"grid={(n + 63) // 64}x{cout // 96} plan=64"), planned
    y0, y1 = s3dx.DeviceArray((n, cout), np.uint16), s3dx.DeviceArray((n, cout), np.uint16)
    conv.run(xd, n, kd, n, y0, s3dx.BF16, rd)
    conv.run(xd, n, kd, n, y1, s3dx.BF16, rd, plan=gp)
    assert np.array_equal(y0.download(), y1.download())
    check_rel(_host(W, y1), _oracle(O, W, x, kmap, n, cin, cout, 46, False, res), 1e-2, case)


@pytest.mark.parametrize("tiling", ["20", "21"])
@pytest.mark.parametrize("shuffle_from", [None, 0, 6912])
def test_halo_tilings_on_dense_and_shuffled_rows(s3dx, O, W, monkeypatch, tiling, shuffle_from):
    # Both tile heights on LDS-staged, global and mixed tiles (no plan).
    monkeypatch.setenv("S3DX_CONV_TILING", tiling)
    coords = _dense_cube(24, shuffle_from, seed=3)
    n = coords.shape[0]
    kmap = O.kmap_subm3(coords, n)
    conv = _layer(s3dx, W, 128, 128, 42, True)
    plan_text = conv.plan(n, n)
    print(f"tiling {tiling} shuffle_from={shuffle_from}: {plan_text}", flush=True)
    assert plan_text.startswith(f"mfma tiling={tiling} split-k halo"), plan_text
    x = W.round_bf16(W.normal_f32(42, 1, (n, 128)))
    res = W.round_bf16(W.normal_f32(42, 4, (n, 128)))
    y = s3dx.DeviceArray((n, 128), np.uint16)
    conv.run(_bf(s3dx, W, x), n, s3dx.DeviceArray.from_host(kmap), n, y, s3dx.BF16, _bf(s3dx, W, res))
    check_rel(_host(W, y), _oracle(O, W, x, kmap, n, 128, 128, 42, True, res), 1e-2)


def test_plan_rejects_another_map_size(s3dx, O, W, monkeypatch):
    monkeypatch.delenv("S3DX_CONV_TILING", raising=False)
    monkeypatch.delenv("S3DX_CONV_HALO", raising=False)
    coords = W.shells_union(0)[:2000]
    n = coords.shape[0]
    kd = s3dx.DeviceArray.from_host(O.kmap_subm3(coords, n))
    conv = _layer(s3dx, W, 128, 128, 43, False)
    gp = conv.gather_plan(n, kd, n)
    xd = _bf(s3dx, W, W.normal_f32(43, 1, (n, 128)))
    y = s3dx.DeviceArray((n, 128), np.uint16)
    with pytest.raises(s3dx.S3dxError) as e:
        conv.run(xd, n, kd, n - 1, y, s3dx.BF16, plan=gp)
    assert e.value.status == s3dx.INVALID_ARGUMENT and "gather plan" in str(e.value)
    # A layer reading parent rows (x >> 3) has other source rows.
    parent = _layer(s3dx, W, 128, 128, 43, False).set_gather_parent(True)
    with pytest.raises(s3dx.S3dxError) as e:
        parent.run(xd, n, kd, n, y, s3dx.BF16, plan=gp)
    assert e.value.status == s3dx.INVALID_ARGUMENT
    # A layer that runs another kernel ignores the plan.
    f32 = s3dx.SparseConv(128, 128, 27, s3dx.F32).set_weights(W.conv_weight(43, 2, 128, 128), s3dx.WEIGHT_SLAT, None)
    xf = s3dx.DeviceArray.from_host(W.normal_f32(43, 5, (n, 128)))
    yf0, yf1 = s3dx.DeviceArray((n, 128), np.float32), s3dx.DeviceArray((n, 128), np.float32)
    f32.run(xf, n, kd, n, yf0, s3dx.F32)
    f32.run(xf, n, kd, n, yf1, s3dx.F32, plan=gp)
    assert np.array_equal(yf0.download(), yf1.download())


def test_plan_rebuild_in_place(s3dx, O, W, monkeypatch):
    # A plan created for a larger map serves a smaller one after rebuild (no
    # allocation); a larger one is refused.
    monkeypatch.delenv("S3DX_CONV_TILING", raising=False)
    monkeypatch.delenv("S3DX_CONV_HALO", raising=False)
    big, small = W.shells_union(0)[:6000], W.shells_union(1)[:4100]
    conv = _layer(s3dx, W, 128, 128, 44, True)
    kb = s3dx.DeviceArray.from_host(O.kmap_subm3(big, big.shape[0]))
    gp = conv.gather_plan(big.shape[0], kb, big.shape[0])
    n = small.shape[0]
    kmap = O.kmap_subm3(small, n)
    ks = s3dx.DeviceArray.from_host(kmap)
    gp.rebuild(conv, n, ks, n)
    x = W.round_bf16(W.normal_f32(44, 1, (n, 128)))
    xd = _bf(s3dx, W, x)
    y0, y1 = s3dx.DeviceArray((n, 128), np.uint16), s3dx.DeviceArray((n, 128), np.uint16)
    conv.run(xd, n, ks, n, y0, s3dx.BF16)
    conv.run(xd, n, ks, n, y1, s3dx.BF16, plan=gp)
    assert np.array_equal(y0.download(), y1.download())
    check_rel(_host(W, y1), _oracle(O, W, x, kmap, n, 128, 128, 44, True), 1e-2)
    with pytest.raises(s3dx.S3dxError) as e:
        gp.rebuild(conv, 6001, kb, 6001)
    assert e.value.status == s3dx.INVALID_ARGUMENT


@pytest.mark.parametrize("rows", ["64", "128"])
def test_plan_tile_heights_agree(s3dx, O, W, monkeypatch, rows):
    # Both planned kernels (64-row records, 4 waves; 128-row records, 8
    # waves) on the config-2 block, bit-identical to the unplanned run.
    monkeypatch.delenv("S3DX_CONV_TILING", raising=False)
    monkeypatch.delenv("S3DX_CONV_HALO", raising=False)
    monkeypatch.setenv("S3DX_PLAN_ROWS", rows)
    coords = W.shells_union(0)
    n = coords.shape[0]
    kd = s3dx.DeviceArray.from_host(O.kmap_subm3(coords, n))
    conv = _layer(s3dx, W, 128, 128, 45, True)
    gp = conv.gather_plan(n, kd, n)
    planned = conv.plan(n, n, gp)
    print(f"rows {rows}: {planned}", flush=True)
    assert planned.endswith(f"plan={rows}") and f"rows={rows}" in planned, planned
    xd = _bf(s3dx, W, W.normal_f32(45, 1, (n, 128)))
    res = _bf(s3dx, W, W.normal_f32(45, 4, (n, 128)))
    y0, y1 = s3dx.DeviceArray((n, 128), np.uint16), s3dx.DeviceArray((n, 128), np.uint16)
    conv.run(xd, n, kd, n, y0, s3dx.BF16, res)
    conv.run(xd, n, kd, n, y1, s3dx.BF16, res, plan=gp)
    assert np.array_equal(y0.download(), y1.download())


@pytest.mark.parametrize("cin", [128, 2048])
def test_planned_layernorm_modulate_full_size(s3dx, O, W, cin):
    # The res_block's conv1 as the benchmark times it and as the SLat flow
    # runs it (slat_flow_graph.cpp:216-275, out_blocks.0 at :441-470): BF16,
    # LayerNorm (no affine) + h*(1+scale)+shift + SiLU fused, scale/shift in
    # device buffers rewritten between forwards, on the config-2 set with the
    # map's 128-row gather plan (the 8-wave kernel, tiling 22).  Each forward:
    # planned == unplanned bit for bit, and both against the float64 oracle
    # (all rows at 128 input channels, 3,000 sampled rows at 2048).
    coords = W.shells_union(0)
    n = coords.shape[0]
    kmap = O.kmap_subm3(coords, n)
    cout, seed = 128, 80 + cin // 128
    w, b = W.conv_weight(seed, 2, cin, cout), W.normal_f32(seed, 3, (cout,), 0.1)
    ms, mh = s3dx.DeviceArray((cout,), np.float32), s3dx.DeviceArray((cout,), np.float32)
    conv = (s3dx.SparseConv(cin, cout, 27, s3dx.BF16).set_weights(w, s3dx.WEIGHT_SLAT, b)
            .set_layernorm(True, 1e-6).set_modulate(ms, mh).set_silu(True))
    dk = s3dx.DeviceArray.from_host(kmap)
    gp = conv.gather_plan(n, dk, n)
    plan = conv.plan(n, n, gp)
    print(f"planned LN+modulate+SiLU {cin}->{cout}: {plan} | unplanned: {conv.plan(n, n)}", flush=True)
    assert plan == "mfma tiling=22 split-k halo rows=128 cols=128 kc=64 xf=0 ln=fused grid=221x1 plan=128", plan
    x = W.round_bf16(W.normal_f32(seed, 1, (n, cin)))
    xd = _bf(s3dx, W, x)
    rows = np.arange(n) if cin == 128 else np.sort(np.random.default_rng(seed).choice(n, 3000, replace=False))
    h = O.layernorm(O.conv(x, kmap[rows], n, W.round_bf16(w), 0, cout, b), 1e-6)
    yp, yu = s3dx.DeviceArray((n, cout), np.uint16), s3dx.DeviceArray((n, cout), np.uint16)
    for fwd in range(2):
        scale, shift = W.normal_f32(seed, 10 + fwd, (cout,), 0.3), W.normal_f32(seed, 20 + fwd, (cout,), 0.3)
        ms.upload(scale)
        mh.upload(shift)
        conv.run(xd, n, dk, n, yp, s3dx.BF16, plan=gp)
        conv.run(xd, n, dk, n, yu, s3dx.BF16)
        got = yp.download()
        assert np.array_equal(got, yu.download()), f"forward {fwd}: planned != unplanned"
        got = W.bf16_bits_to_f32(got).reshape(n, cout)[rows]
        check_rel(got, O.silu(O.modulate(h, scale, shift)), 1e-2, f"{cin}->{cout} forward {fwd}")


@pytest.mark.parametrize("rows", ["128", "64"])
def test_kmap_planned_one_pass(s3dx, O, W, golden, monkeypatch, rows):
    # s3dx_kmap_subm3_planned: the kernel map and its gather plan from the
    # same lookups.  The map is byte-identical to s3dx_kmap_subm3's (golden
    # SHA on config 2, the oracle on a set with duplicates and coordinates
    # outside the window, a zeroed workspace under the seed whose tag for an
    # empty cell next to the set is 0); its plan drives the planned conv to
    # the same bits as a plan rebuilt from the map and as the unplanned run.
    from helpers import colliding_seed, set_kmap_seed, sha, window_cell_index
    arrays, manifest = golden
    monkeypatch.setenv("S3DX_PLAN_ROWS", rows)
    base = W.shells_union(0)
    dup = np.concatenate([base[:9000], base[2000:2600], base[9000:12000] - np.array([0, 20, 0, 0], np.int32)])
    for name, coords in (("config 2", base), ("duplicates + hashed", np.ascontiguousarray(dup))):
        n = coords.shape[0]
        want = O.kmap_subm3(coords, n)
        conv = _layer(s3dx, W, 128, 128, 48, True)
        dc = s3dx.DeviceArray.from_host(coords)
        k_sep = s3dx.DeviceArray.from_host(want)
        plan_sep = conv.gather_plan(n, k_sep, n)
        plan_one = conv.gather_plan(n, k_sep, n)
        k_one = s3dx.DeviceArray((n, 27), np.int32)
        ws = s3dx.DeviceArray(s3dx.kmap_workspace_size(n), np.uint8)
        ws.upload(np.zeros(ws.nbytes, np.uint8))
        if name == "config 2":
            set_kmap_seed(s3dx, colliding_seed(window_cell_index(27, 22, 46)))
        s3dx.kmap_subm3_planned(dc, n, n, k_one, plan_one, conv, ws)
        got = k_one.download()
        print(f"kmap+plan one pass rows={rows} {name} n={n}: {conv.plan(n, n, plan_one)}", flush=True)
        assert np.array_equal(got, want), name
        if name == "config 2":
            assert sha(got) == manifest["shells_union_s0"]["conv_fine_sha256"]
        x = W.round_bf16(W.normal_f32(48, 1, (n, 128)))
        xd = _bf(s3dx, W, x)
        ys = [s3dx.DeviceArray((n, 128), np.uint16) for _ in range(3)]
        conv.run(xd, n, k_one, n, ys[0], s3dx.BF16, plan=plan_one)
        conv.run(xd, n, k_sep, n, ys[1], s3dx.BF16, plan=plan_sep)
        conv.run(xd, n, k_sep, n, ys[2], s3dx.BF16)
        a, b, c = (y.download() for y in ys)
        assert np.array_equal(a, b) and np.array_equal(a, c), name
        check_rel(_host(W, ys[0]), _oracle(O, W, x, want, n, 128, 128, 48, True), 1e-2, name)


HALF_CHUNK = {
    # name: (coords builder, cin, cout) -- Cin 32 above a multiple of 64
    "shells_union_3000_96_96": (lambda W: W.shells_union(1)[:3000], 96, 96),
    "shells_union_3000_96_192": (lambda W: W.shells_union(1)[:3000], 96, 192),
    "shells_union_3000_160_128": (lambda W: W.shells_union(1)[:3000], 160, 128),
    "shuffled_cube_13824_96_96": (lambda W: _dense_cube(24, 0), 96, 96),          # every tile global
    "half_shuffled_cube_13824_96_96": (lambda W: _dense_cube(24, 6912), 96, 96),  # both modes
    "isolated_points_96_96": (lambda W: _sparse_points(3, False), 96, 96),       # one offset: waves 2, 3 idle
    "point_pairs_96_128": (lambda W: _sparse_points(4, True), 96, 128),           # three offsets
    "tiny_37_96_96": (lambda W: W.shells_union(2)[:37], 96, 96),                  # one partial tile
}


@pytest.mark.parametrize("plan_rows", ["64", "128"])
@pytest.mark.parametrize("case", list(HALF_CHUNK))
def test_half_width_last_chunk(s3dx, O, W, monkeypatch, case, plan_rows):
    # The 64-row halo kernel with Cin 32 above a multiple of 64 (forced:
    # split-K is the default there): the last chunk's two k-steps split
    # over the four waves by offset parity.  Planned == unplanned bit for bit
    # (a 128-row plan is not used by this kernel and leaves the launch as it
    # is), both against the oracle.
    monkeypatch.setenv("S3DX_CONV_TILING", "21")
    monkeypatch.delenv("S3DX_CONV_HALO", raising=False)
    monkeypatch.setenv("S3DX_PLAN_ROWS", plan_rows)
    build, cin, cout = HALF_CHUNK[case]
    coords = build(W)
    n = coords.shape[0]
    kmap = O.kmap_subm3(coords, n)
    conv = _layer(s3dx, W, cin, cout, 47, False)
    x = W.round_bf16(W.normal_f32(47, 1, (n, cin)))
    res = W.round_bf16(W.normal_f32(47, 4, (n, cout)))
    xd, kd, rd = _bf(s3dx, W, x), s3dx.DeviceArray.from_host(kmap), _bf(s3dx, W, res)
    gp = conv.gather_plan(n, kd, n)
    plan_text, planned = conv.plan(n, n), conv.plan(n, n, gp)
    print(f"{case} n={n} plan rows {plan_rows}: {plan_text} | {planned}", flush=True)
    cols = 128 if cout % 128 == 0 else 96
    assert plan_text.startswith(f"mfma tiling=21 split-k halo rows=64 cols={cols} kc=64+32"), plan_text
    assert planned == (plan_text + " plan=64" if plan_rows == "64" else plan_text), planned
    y0, y1 = s3dx.DeviceArray((n, cout), np.uint16), s3dx.DeviceArray((n, cout), np.uint16)
    conv.run(xd, n, kd, n, y0, s3dx.BF16, rd)
    conv.run(xd, n, kd, n, y1, s3dx.BF16, rd, plan=gp)
    assert np.array_equal(y0.download(), y1.download())
    check_rel(_host(W, y1), _oracle(O, W, x, kmap, n, cin, cout, 47, False, res), 1e-2, case)
