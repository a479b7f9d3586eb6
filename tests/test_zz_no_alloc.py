"""The allocation-free kernel map (s3dx_kmap_subm3_static) through the C ABI
against the workspace entry point (s3dx_kmap_subm3): byte-identical maps on
two calls in a row, the second on a smaller set (the static table keeps the
first call's contents and must be cleared by the second), then a set with
duplicated coordinates and the mesh sentinel."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_static_kmap_matches_workspace_entry_point(s3dx, W):
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
