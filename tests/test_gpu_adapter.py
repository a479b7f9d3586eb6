"""The compiled C++ consumer of the ABI (sam3d.cpp_amd/adapter, libs3dx_adapter.so):
the adapter a sam3d.cpp maintainer adds, built by the host C++ compiler
against include/s3dx_sparse.h alone, called in this process through ctypes.

- DeviceSlatTables reproduces the reference's own tables (SHA-256 of the
  golden manifest, written by the compiled sparse_ops.cpp);
- device_subdivide reproduces MeshSubdivideTables, and returns false where
  the reference does (duplicate parents);
- SlatResBlock runs the SLat res_block with a new modulate per forward, at
  the FP32 gate against the oracle.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np
import pytest

from helpers import check_rel, large_sets, sha

pytestmark = pytest.mark.gpu

_vp, _i32, _i64, _u64 = C.c_void_p, C.c_int32, C.c_int64, C.c_uint64


@pytest.fixture(scope="module")
def adapter(s3dx):
    s3dx.lib()  # the same libs3dx_sparse.so the adapter links to
    path = Path(s3dx.LIB_PATH).parent / "libs3dx_adapter.so"
    if not path.exists():
        pytest.fail(f"{path} is not built; run __graft_entry__.build()")
    lib = C.CDLL(str(path))
    lib.s3dx_adapter_slat_tables.argtypes = [_vp, _i64, _vp, C.POINTER(_i64), _vp, _vp, _vp, _vp, _vp, C.c_char_p, _u64]
    lib.s3dx_adapter_subdivide.argtypes = [_vp, _i64, _vp, _vp, C.c_char_p, _u64]
    lib.s3dx_adapter_res_block.argtypes = [_vp, _i64, _i32, _i32] + [_vp] * 9 + [_i32, _vp, _vp, _vp, C.c_char_p, _u64]
    for f in (lib.s3dx_adapter_slat_tables, lib.s3dx_adapter_subdivide, lib.s3dx_adapter_res_block):
        f.restype = C.c_uint32
    return lib


def _p(a):
    return None if a is None else a.ctypes.data_as(_vp)


def test_adapter_slat_tables_and_subdivide_match_reference(adapter, s3dx, O, W, golden):
    arrays, manifest = golden
    for name, coords in large_sets(W, O, arrays).items():
        coords = np.ascontiguousarray(coords, np.int32)
        n = coords.shape[0]
        m = manifest[name]
        print(f"adapter tables {name} n={n}", flush=True)
        fine = np.empty((n, 27), np.int32)
        cc = np.empty((n, 4), np.int32)
        f2c = np.empty(n, np.int32)
        ch = np.empty(8 * n, np.int32)
        inv = np.empty(n, np.float32)
        coarse = np.empty((n, 27), np.int32)
        nc = _i64(0)
        err = C.create_string_buffer(512)
        st = adapter.s3dx_adapter_slat_tables(_p(coords), n, _p(fine), C.byref(nc), _p(cc), _p(f2c), _p(ch), _p(inv),
                                              _p(coarse), err, len(err))
        assert st == 0, err.value
        nc = nc.value
        assert nc == m["nc"]
        assert sha(fine) == m["conv_fine_sha256"], name
        assert sha(f2c) == m["fine_to_coarse_sha256"], name
        assert sha(coarse[:nc]) == m["conv_coarse_sha256"], name
        assert sha(ch[: 8 * nc]) == m["coarse_children_sha256"], name
        assert sha(inv[:nc]) == m["coarse_inv_count_sha256"], name
        child = np.empty((8 * n, 4), np.int32)
        kmap = np.empty((8 * n, 27), np.int32)
        st = adapter.s3dx_adapter_subdivide(_p(coords), n, _p(child), _p(kmap), err, len(err))
        assert st == 0, err.value
        assert sha(child) == m["subdivide"]["child_coords_sha256"], name
        assert sha(kmap) == m["subdivide"]["neighbors_sha256"], name
    dup = np.ascontiguousarray(np.concatenate([coords[:50], coords[:1]]), np.int32)
    st = adapter.s3dx_adapter_subdivide(_p(dup), dup.shape[0], _p(child), _p(kmap), err, len(err))
    assert st == s3dx.INVALID_ARGUMENT, "duplicate parents must be rejected like MeshSubdivideTables::build"


@pytest.mark.parametrize("cin,cout", [(128, 128), (256, 128)])
def test_adapter_res_block(adapter, O, W, cin, cout):
    coords = np.ascontiguousarray(W.shell_64(res=24, centre=(12.0, 12.0, 12.0), radius=7.0), np.int32)
    n = coords.shape[0]
    g = lambda k, shape, s=1.0: W.normal_f32(90, k, shape, s)  # noqa: E731
    x = g(1, (n, cin))
    n1w, n1b = g(2, (cin,), 0.2) + 1.0, g(3, (cin,), 0.2)
    w1, b1 = W.conv_weight(90, 4, cin, cout), g(5, (cout,), 0.1)
    w2, b2 = W.conv_weight(90, 6, cout, cout), g(7, (cout,), 0.1)
    ws = W.conv_weight(90, 8, cin, cout, kvol=1) if cin != cout else None
    bs = g(9, (cout,), 0.1) if cin != cout else None
    fwd = 2
    scale, shift = g(10, (fwd, cout), 0.3), g(11, (fwd, cout), 0.3)
    y = np.empty((fwd, n, cout), np.float32)
    err = C.create_string_buffer(512)
    st = adapter.s3dx_adapter_res_block(_p(coords), n, cin, cout, _p(x), _p(n1w), _p(n1b), _p(w1), _p(b1), _p(w2),
                                        _p(b2), _p(ws), _p(bs), fwd, _p(scale), _p(shift), _p(y), err, len(err))
    assert st == 0, err.value
    kmap = O.kmap_subm3(coords, n)
    h = O.silu(O.layernorm(x, 1e-6, n1w, n1b))
    c1 = O.conv(h, kmap, n, w1, 0, cout, b1)
    skip = x if ws is None else O.conv(x, None, n, ws, 0, cout, bs, kvol=1)
    for f in range(fwd):
        y1 = O.silu(O.modulate(O.layernorm(c1, 1e-6), scale[f], shift[f]))
        ref = O.conv(y1, kmap, n, w2, 0, cout, b2) + skip
        check_rel(y[f], ref, 1e-5, f"adapter res_block {cin}->{cout} forward {f}")
