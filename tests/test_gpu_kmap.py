"""GPU kernel maps, coarsen and subdivide through the C ABI: byte-identical to
the oracle and to the reference golden tables."""
import numpy as np
import pytest

from helpers import (SMALL, colliding_seed, flag_value, kmap_flags_offset, large_sets, set_kmap_seed, sha,
                     window_cell_index)

pytestmark = pytest.mark.gpu


def gpu_kmap(s3dx, coords, missing):
    n = coords.shape[0]
    d = s3dx.DeviceArray.from_host(np.ascontiguousarray(coords, np.int32))
    return s3dx.kmap_subm3(d, n, missing).download()


@pytest.mark.parametrize("name", SMALL)
def test_small_sets_match_reference(s3dx, O, golden, name):
    arrays, manifest = golden
    coords = arrays[f"{name}.coords"]
    n = coords.shape[0]
    print(f"kmap small set {name} n={n}", flush=True)
    assert np.array_equal(gpu_kmap(s3dx, coords, n), arrays[f"{name}.conv_fine"])
    assert np.array_equal(gpu_kmap(s3dx, coords, -1), O.kmap_subm3(coords, -1))
    nc, cc, f2c, ch, inv = s3dx.coarsen2(s3dx.DeviceArray.from_host(coords), n)
    assert nc == manifest[name]["nc"]
    assert np.array_equal(f2c.download(), arrays[f"{name}.fine_to_coarse"])
    ccoords = cc.download()[:nc]
    assert np.array_equal(gpu_kmap(s3dx, ccoords, nc), arrays[f"{name}.conv_coarse"])
    assert np.array_equal(ch.download()[: 8 * nc], arrays[f"{name}.coarse_children"])
    assert np.array_equal(inv.download()[:nc].view(np.uint32),
                          arrays[f"{name}.coarse_inv_count"].view(np.uint32))
    tables = s3dx.MeshSubdivideTables()
    ok = tables.build(coords)
    if manifest[name]["subdivide"] == "rejected":
        assert not ok
    else:
        assert ok
        assert np.array_equal(tables.child_coords.download(), arrays[f"{name}.child_coords"])
        assert np.array_equal(tables.neighbors.download(), arrays[f"{name}.neighbors"])


def test_large_sets_match_reference_sha(s3dx, O, W, golden):
    arrays, manifest = golden
    for name, coords in large_sets(W, O, arrays).items():
        m = manifest[name]
        n = coords.shape[0]
        print(f"kmap large set {name} n={n}", flush=True)
        t = s3dx.SlatTables()
        assert t.build(coords)
        assert sha(t.conv_fine.download()) == m["conv_fine_sha256"], name
        assert t.nc == m["nc"], name
        assert sha(t.fine_to_coarse.download()) == m["fine_to_coarse_sha256"], name
        assert sha(t.conv_coarse.download()) == m["conv_coarse_sha256"], name
        assert sha(t.coarse_children.download()[: 8 * t.nc]) == m["coarse_children_sha256"], name
        assert sha(t.coarse_inv_count.download()[: t.nc]) == m["coarse_inv_count_sha256"], name
        mt = s3dx.MeshSubdivideTables()
        assert mt.build(t.coords, n)
        assert sha(mt.child_coords.download()) == m["subdivide"]["child_coords_sha256"], name
        assert sha(mt.neighbors.download()) == m["subdivide"]["neighbors_sha256"], name


def test_random_sets_with_duplicates_and_batches(s3dx, O):
    rng = np.random.default_rng(2024)
    for trial in range(12):
        n = int(rng.integers(1, 5000))
        span = int(rng.integers(2, 40))
        c = rng.integers(-span, span, size=(n, 4)).astype(np.int32)
        c[:, 0] = rng.integers(0, 3, size=n)
        print(f"random trial {trial} n={n} span={span}", flush=True)
        assert np.array_equal(gpu_kmap(s3dx, c, n), O.kmap_subm3(c, n))
        nc, cc, f2c, ch, inv = s3dx.coarsen2(s3dx.DeviceArray.from_host(c), n)
        onc, occ, of2c, och, oinv = O.coarsen2(c)
        assert nc == onc
        assert np.array_equal(cc.download()[:nc], occ)
        assert np.array_equal(f2c.download(), of2c)
        assert np.array_equal(ch.download()[: 8 * nc], och)
        assert np.array_equal(inv.download()[:nc], oinv)


def _coarsen_cases():
    """Sets for the window path of s3dx_coarsen2 (batch 0 in [0, 128)^3, at
    most eight rows per coarse cell) and for each way out of it."""
    rng = np.random.default_rng(91)
    g = np.stack(np.meshgrid(*(np.arange(0, 128, 3),) * 3, indexing="ij"), -1).reshape(-1, 3)
    base = np.concatenate([np.zeros((len(g), 1), np.int64), g], 1).astype(np.int32)
    base = base[rng.permutation(len(base))]
    edge = base.copy()
    edge[:8, 1:] = [[0, 0, 0], [127, 127, 127], [0, 127, 0], [127, 0, 127],
                    [126, 1, 0], [1, 126, 127], [64, 63, 64], [63, 64, 63]]
    few_dups = np.concatenate([base, base[:500]])             # two rows on some fine cells: <= 8 a coarse cell
    cube = np.stack(np.meshgrid(*(np.arange(10, 12),) * 3, indexing="ij"), -1).reshape(-1, 3)
    full = np.concatenate([np.zeros((8, 1), np.int64), cube], 1).astype(np.int32)
    overflow = np.concatenate([base, full, full[:1]])        # nine rows on one coarse cell
    outside = base.copy()
    outside[17] = [0, 128, 5, 5]                              # one row past the window
    negative = base.copy()
    negative[3] = [0, -1, 4, 4]                               # (-1 / 2 == 0: the same coarse cell as 0, 1)
    batch1 = base.copy()
    batch1[::97, 0] = 1                                       # a second batch
    return {"window": base, "window_edges": edge, "window_duplicates": few_dups,
            "nine_rows_one_cell": overflow, "outside_window": outside, "negative": negative,
            "two_batches": batch1}


@pytest.mark.parametrize("case", list(_coarsen_cases()))
def test_coarsen_window_path(s3dx, O, case):
    # The window path (a bitmap ranked by a popcount scan, eight slots a
    # coarse row) and its fallback to the sort, byte-identical to the oracle
    # on the tables SlatTables::build returns (sparse_ops.cpp:53-104).
    c = np.ascontiguousarray(_coarsen_cases()[case])
    n = c.shape[0]
    nc, cc, f2c, ch, inv = s3dx.coarsen2(s3dx.DeviceArray.from_host(c), n)
    onc, occ, of2c, och, oinv = O.coarsen2(c)
    print(f"coarsen {case}: n={n} nc={nc}", flush=True)
    assert nc == onc
    assert np.array_equal(cc.download()[:nc], occ)
    assert np.array_equal(f2c.download(), of2c)
    assert np.array_equal(ch.download()[: 8 * nc], och)
    assert np.array_equal(inv.download()[:nc].view(np.uint32), oinv.view(np.uint32))


@pytest.mark.parametrize("n", [3000, 200000])
def test_coarsen_wide_bbox(s3dx, O, n):
    # Coordinates spread over ~2^30 (negative ones too, two batches, half the
    # rows repeated): the sort-based coarsen orders any int32 keys, in
    # O(n log n) -- 200k rows of 100k distinct wide keys in one call.
    rng = np.random.default_rng(77)
    c = rng.integers(-2**30, 2**30, size=(n, 4)).astype(np.int32)
    c[:, 0] = rng.integers(0, 2, size=n)
    c[n // 2:] = c[: n - n // 2]  # duplicates
    print(f"coarsen wide bbox n={n}", flush=True)
    nc, cc, f2c, ch, inv = s3dx.coarsen2(s3dx.DeviceArray.from_host(c), n)
    onc, occ, of2c, och, oinv = O.coarsen2(c)
    assert nc == onc
    assert np.array_equal(cc.download()[:nc], occ)
    assert np.array_equal(f2c.download(), of2c)
    assert np.array_equal(ch.download()[: 8 * nc], och)
    assert np.array_equal(inv.download()[:nc].view(np.uint32), oinv.view(np.uint32))
    if n <= 3000:
        assert np.array_equal(gpu_kmap(s3dx, c, n), O.kmap_subm3(c, n))


def test_subdivide_rejects_duplicates(s3dx):
    p = np.array([[0, 1, 2, 3], [0, 4, 4, 4], [0, 1, 2, 3]], np.int32)
    assert not s3dx.MeshSubdivideTables().build(p)
    with pytest.raises(s3dx.S3dxError, match="duplicate"):
        s3dx.subdivide2(s3dx.DeviceArray.from_host(p), 3)


def test_two_level_subdivide_properties(s3dx, W):
    # The mesh-decoder path at full size: 64^3 set -> 128^3 -> 256^3 (~1.8M).
    parents = W.shells_union(0)
    t0 = s3dx.MeshSubdivideTables()
    assert t0.build(parents)
    t1 = s3dx.MeshSubdivideTables()
    assert t1.build(t0.child_coords, t0.child_count)
    n1 = t1.child_count
    print(f"two-level subdivide children={n1}", flush=True)
    k = t1.neighbors.download()
    child = t1.child_coords.download()
    # centre tap is the row itself; neighbour relation is symmetric
    assert np.array_equal(k[:, 13], np.arange(n1))
    for o in (0, 4, 12, 22):
        have = np.nonzero(k[:, o] >= 0)[0]
        assert np.array_equal(k[k[have, o], 26 - o], have)
        d = child[k[have, o], 1:] - child[have, 1:]
        assert np.all(d == np.array([o // 9 - 1, (o // 3) % 3 - 1, o % 3 - 1]))
    # the subdivided map equals a from-scratch kernel map over the children
    assert np.array_equal(s3dx.kmap_subm3(t1.child_coords, n1, -1).download(), k)


def test_coarsen_subdivide_reused_buffers(s3dx, W):
    # Two calls into the same caller-owned outputs and workspace, the second
    # on a smaller set: each result equals a fresh call's, byte for byte, in
    # the meaningful rows (nothing is left over from the first call).
    big, small = W.shells_union(0), W.shells_union(1)[:5000]
    n = big.shape[0]
    c_out = (s3dx.DeviceArray((n, 4), np.int32), s3dx.DeviceArray((n,), np.int32),
             s3dx.DeviceArray((8 * n,), np.int32), s3dx.DeviceArray((n,), np.float32))
    c_ws = s3dx.DeviceArray(s3dx.coarsen2_workspace_size(n), np.uint8)
    s_out = (s3dx.DeviceArray((8 * n, 4), np.int32), s3dx.DeviceArray((8 * n, 27), np.int32))
    s_ws = s3dx.DeviceArray(s3dx.subdivide2_workspace_size(n), np.uint8)
    for coords in (big, small):
        m = coords.shape[0]
        d = s3dx.DeviceArray.from_host(coords)
        print(f"reused buffers n={m}", flush=True)
        nc, cc, f2c, ch, inv = s3dx.coarsen2(d, m, out=c_out, workspace=c_ws)
        nc2, cc2, f2c2, ch2, inv2 = s3dx.coarsen2(d, m)
        assert nc == nc2
        assert np.array_equal(cc.download()[:nc], cc2.download()[:nc])
        assert np.array_equal(f2c.download()[:m], f2c2.download()[:m])
        assert np.array_equal(ch.download()[: 8 * nc], ch2.download()[: 8 * nc])
        assert np.array_equal(inv.download()[:nc], inv2.download()[:nc])
        child, kmap = s3dx.subdivide2(d, m, True, out=s_out, workspace=s_ws)
        child2, kmap2 = s3dx.subdivide2(d, m, True)
        assert np.array_equal(child.download()[: 8 * m], child2.download())
        assert np.array_equal(kmap.download()[: 8 * m], kmap2.download())


def test_workspace_reuse_and_garbage(s3dx, O, W):
    # One workspace across builds of different sets -- window cells (batch 0,
    # [0, 64)^3), hashed coordinates (outside the window, other batches, wide
    # int32 values) and duplicates -- first as left by earlier builds, then
    # filled with random bytes: no word of an earlier build or of the bytes
    # may surface in a later map.
    rng = np.random.default_rng(5)
    big = W.shells_union(0)
    dup = np.concatenate([big[:3000], big[1000:2500]])
    rng.shuffle(dup)
    batch1 = big[:5000].copy()
    batch1[:, 0] = 1
    wide = big[:2000].copy()
    wide[::5, 1] += 70000  # beyond int16: matched through the input rows
    sets = {"shells": big, "shells_every_3rd": big[::3],
            "shifted_x40": big + np.array([0, 40, 0, 0], np.int32),
            "shifted_negative": big - np.array([0, 30, 30, 30], np.int32),
            "two_batches": np.concatenate([big[:5000], batch1]),
            "duplicates": dup, "wide": wide, "shells_again": big}
    n_max = max(c.shape[0] for c in sets.values())
    ws = s3dx.DeviceArray(s3dx.kmap_workspace_size(n_max), np.uint8)
    for garbage in (False, True):
        if garbage:
            ws.upload(rng.integers(0, 256, size=ws.nbytes, dtype=np.uint8))
        for name, c in sets.items():
            c = np.ascontiguousarray(c, np.int32)
            n = c.shape[0]
            print(f"kmap reuse garbage={garbage} {name} n={n}", flush=True)
            got = s3dx.kmap_subm3(s3dx.DeviceArray.from_host(c), n, -1, workspace=ws).download()
            assert np.array_equal(got, O.kmap_subm3(c, -1)), name


def _zeroed(s3dx, nbytes):
    ws = s3dx.DeviceArray(nbytes, np.uint8)
    ws.upload(np.zeros(nbytes, np.uint8))
    return ws


def test_zero_filled_table_tag_collision(s3dx, W, golden):
    # Window cell (0,27,22,46) is empty in config 2 (seed 0) but is the
    # neighbour of three voxels.  Under the build seed whose tag for that
    # cell is 0 (the 59,357th build of a process), a zero-filled table
    # carries the current tag there, and a lookup that trusted the tag would
    # return row 0 for those voxels.  The map must stay byte-identical to the
    # reference's (golden SHA), for the SLat sentinel and for subdivide.
    arrays, manifest = golden
    coords = W.shells_union(0)
    n = coords.shape[0]
    cell = (27, 22, 46)
    rows = {tuple(r): i for i, r in enumerate(coords[:, 1:].tolist())}
    assert cell not in rows
    near = [(rows[(cell[0] - dx, cell[1] - dy, cell[2] - dz)], (dx + 1) * 9 + (dy + 1) * 3 + (dz + 1))
            for dx in (-1, 0, 1) for dy in (-1, 0, 1) for dz in (-1, 0, 1)
            if (cell[0] - dx, cell[1] - dy, cell[2] - dz) in rows]
    assert len(near) == 3
    seed = colliding_seed(window_cell_index(*cell))
    assert seed == 0x3C6EF372 + 59356
    dc = s3dx.DeviceArray.from_host(coords)
    print(f"kmap zero-filled workspace, seed {seed:#x}, n={n}", flush=True)
    set_kmap_seed(s3dx, seed)
    got = s3dx.kmap_subm3(dc, n, n, workspace=_zeroed(s3dx, s3dx.kmap_workspace_size(n))).download()
    assert all(got[i, o] == n for i, o in near), [(i, o, got[i, o]) for i, o in near]
    assert sha(got) == manifest["shells_union_s0"]["conv_fine_sha256"]
    print("subdivide zero-filled workspace, same seed", flush=True)
    set_kmap_seed(s3dx, seed)
    child, kmap = s3dx.subdivide2(dc, n, True, workspace=_zeroed(s3dx, s3dx.subdivide2_workspace_size(n)))
    sub = manifest["shells_union_s0"]["subdivide"]
    assert sha(child.download()) == sub["child_coords_sha256"]
    assert sha(kmap.download()) == sub["neighbors_sha256"]


def test_subdivide_confirms_chance_flags(s3dx, W):
    # A workspace whose flag words hold, by chance, the values this build
    # raises them to (duplicate, overflow) on a duplicate-free set: the
    # exact recount behind a raised flag must clear it, and a set with a
    # real duplicate must still be rejected.
    parents = np.ascontiguousarray(W.shells_union(1)[:5000])
    n = parents.shape[0]
    seed = 0x51ED270B
    nbytes = s3dx.subdivide2_workspace_size(n)
    host = np.zeros(nbytes, np.uint8)
    off = kmap_flags_offset(n)
    host[off:off + 8] = np.array([flag_value(seed, 0), flag_value(seed, 1)], np.int32).view(np.uint8)
    ws = s3dx.DeviceArray(nbytes, np.uint8)
    ws.upload(host)
    dc = s3dx.DeviceArray.from_host(parents)
    print(f"subdivide with planted flag words, n={n}", flush=True)
    set_kmap_seed(s3dx, seed)
    child, kmap = s3dx.subdivide2(dc, n, True, workspace=ws)
    child2, kmap2 = s3dx.subdivide2(dc, n, True)
    assert np.array_equal(child.download(), child2.download())
    assert np.array_equal(kmap.download(), kmap2.download())
    dup = np.ascontiguousarray(np.concatenate([parents, parents[17:18]]))
    with pytest.raises(s3dx.S3dxError, match="duplicate"):
        s3dx.subdivide2(s3dx.DeviceArray.from_host(dup), n + 1)


@pytest.mark.parametrize("extent,n", [(128, 150_000), (256, 1_100_000)])
def test_wide_window_sets(s3dx, O, extent, n):
    # Sets large enough for a 128^3 or 256^3 direct-index window (above
    # 131,072 and 1,048,576 voxels): coordinates spread over the window,
    # some outside it (batch 1, negative, beyond the extent: the hashed
    # path), duplicated rows, a shuffled order; against the oracle, and on a
    # workspace refilled with random bytes.
    rng = np.random.default_rng(extent)
    c = rng.integers(0, extent, size=(n, 4)).astype(np.int32)
    c[:, 0] = 0
    out = rng.choice(n, n // 50, replace=False)
    c[out[: len(out) // 3], 0] = 1
    c[out[len(out) // 3: 2 * len(out) // 3], 1] -= extent
    c[out[2 * len(out) // 3:], 3] += extent
    c[rng.choice(n, n // 100, replace=False)] = c[rng.choice(n, n // 100, replace=False)]
    c = np.ascontiguousarray(c)
    print(f"wide window extent={extent} n={n}", flush=True)
    want = O.kmap_subm3(c, -1)
    ws = s3dx.DeviceArray(s3dx.kmap_workspace_size(n), np.uint8)
    for garbage in (False, True):
        if garbage:
            ws.upload(rng.integers(0, 256, size=ws.nbytes, dtype=np.uint8))
        got = s3dx.kmap_subm3(s3dx.DeviceArray.from_host(c), n, -1, workspace=ws).download()
        assert np.array_equal(got, want), f"garbage={garbage}"
