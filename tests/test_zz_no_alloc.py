"""The allocation-free kernel map (s3dx_kmap_subm3_static) through the C ABI.

Its table is a static device array that starts zeroed and keeps the last
call's contents; nothing clears it between calls (per-call tags, rows checked
against the input coordinates).  Checked against the workspace entry point
(s3dx_kmap_subm3) on two calls in a row, the second on a smaller set, then a
set with duplicated coordinates and the mesh sentinel; against the
reference's golden SHA and the oracle; and on a zeroed table under the build
seed whose tag collides with a zero word of a cell next to the set.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import colliding_seed, set_kmap_seed, sha, window_cell_index, zero_static_kmap

pytestmark = pytest.mark.gpu


def test_static_kmap_matches_workspace_entry_point(s3dx, W, O, golden):
    arrays, manifest = golden
    rng = np.random.default_rng(3)
    big = W.shells_union(0)
    small = W.shell_64()
    dup = np.concatenate([small[:4000], small[rng.integers(0, 4000, 300)]], 0)
    for name, coords, missing in (("28,265-voxel shells", big, None), ("10,366-voxel shell", small, None),
                                  ("duplicates, sentinel -1", dup, -1)):
        n = coords.shape[0]
        miss = n if missing is None else missing
        print(f"static kmap {name}: n={n}", flush=True)
        dc = s3dx.DeviceArray.from_host(np.ascontiguousarray(coords, np.int32))
        want = s3dx.kmap_subm3(dc, n, miss).download()
        got = s3dx.kmap_subm3_static(dc, n, miss).download()
        assert np.array_equal(got, want), name
        if n == big.shape[0]:
            assert sha(got) == manifest["shells_union_s0"]["conv_fine_sha256"]
        else:
            assert np.array_equal(got, O.kmap_subm3(np.ascontiguousarray(coords, np.int32), miss)), name


def test_static_kmap_zeroed_table_tag_collision(s3dx, W, golden):
    # The static table as a fresh process has it (all zeros), under the seed
    # whose tag for the empty cell (0,27,22,46) next to three voxels of
    # config 2 is 0: the map must still equal the reference's.
    arrays, manifest = golden
    coords = W.shells_union(0)
    n = coords.shape[0]
    seed = colliding_seed(window_cell_index(27, 22, 46))
    print(f"static kmap on a zeroed table, seed {seed:#x}, n={n}", flush=True)
    zero_static_kmap(s3dx)
    set_kmap_seed(s3dx, seed)
    dc = s3dx.DeviceArray.from_host(coords)
    got = s3dx.kmap_subm3_static(dc, n, n).download()
    assert sha(got) == manifest["shells_union_s0"]["conv_fine_sha256"]
