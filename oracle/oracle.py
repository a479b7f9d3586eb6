"""TEST INFRASTRUCTURE ONLY: ctypes bindings of the CPU oracle (liboracle.so)
and of the compiled reference checker (_ref/libref_sparse_ops.so).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
this module, as the checker or the CPU baseline -- never as the product path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_PATH = HERE / "liboracle.so"
REF_PATH = HERE / "_ref" / "libref_sparse_ops.so"

_vp, _i32, _i64, _f32 = C.c_void_p, C.c_int32, C.c_int64, C.c_float

_SIGS = {
    "orc_kmap_subm3": (_i32, [_vp, _i64, _i32, _vp]),
    "orc_coarsen2": (_i64, [_vp, _i64, _vp, _vp, _vp, _vp]),
    "orc_subdivide2": (_i32, [_vp, _i64, _vp, _vp]),
    "orc_conv_subm": (None, [_vp, _i64, _i32, _vp, _i64, _i32, _vp, _i32, _i32, _vp, _vp]),
    "orc_layernorm": (None, [_vp, _i64, _i32, _f32, _vp, _vp, _vp]),
    "orc_groupnorm": (None, [_vp, _i64, _i32, _i32, _f32, _vp, _vp, _vp]),
    "orc_silu": (None, [_vp, _i64, _vp]),
    "orc_modulate": (None, [_vp, _i64, _i32, _vp, _vp, _vp]),
    "orc_add": (None, [_vp, _vp, _i64, _vp]),
    "orc_downsample_mean": (None, [_vp, _i64, _i32, _vp, _vp, _i64, _vp]),
    "orc_upsample_nearest": (None, [_vp, _i64, _i32, _vp, _i64, _vp]),
    "orc_repeat_children": (None, [_vp, _i64, _i32, _vp]),
    "orc_occupancy_coords": (_i64, [_vp, _i32, _vp]),
    "orc_prune_surface": (_i64, [_vp, _i64, _vp]),
    "orc_downsample_coords": (_i64, [_vp, _i64, _i64, _i32, C.c_uint32, _vp]),
    "orc_mt19937_draw": (C.c_uint32, [C.c_uint32, _i64]),
    "orc_conv_im2col_gemm_f32": (None, [_vp, _i64, _i32, _vp, _i64, _vp, _i32, _vp, _vp, _i32]),
    "orc_round_bf16": (None, [_vp, _i64, _vp]),
}

_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        h = C.CDLL(str(ORACLE_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(h, name)
            fn.restype, fn.argtypes = res, args
        _lib = h
    return _lib


def ref_available() -> bool:
    return REF_PATH.exists()


def ref():
    global _ref
    if _ref is None:
        h = C.CDLL(str(REF_PATH))
        h.ref_slat_tables.restype = _i64
        h.ref_slat_tables.argtypes = [_vp, _i64, _i32, _vp, _vp, _vp, _vp, _vp]
        h.ref_mesh_subdivide.restype = _i32
        h.ref_mesh_subdivide.argtypes = [_vp, _i64, _vp, _vp]
        _ref = h
    return _ref


def _p(a):
    return None if a is None else a.ctypes.data_as(_vp)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


# ---- oracle ---------------------------------------------------------------
def kmap_subm3(coords: np.ndarray, missing: int) -> np.ndarray:
    c = _c(coords, np.int32)
    n = c.shape[0]
    out = np.empty((n, 27), dtype=np.int32)
    lib().orc_kmap_subm3(_p(c), n, missing, _p(out))
    return out


def coarsen2(coords: np.ndarray):
    c = _c(coords, np.int32)
    n = c.shape[0]
    cc = np.empty((n, 4), np.int32)
    f2c = np.empty(n, np.int32)
    ch = np.empty(8 * n, np.int32)
    inv = np.empty(n, np.float32)
    nc = lib().orc_coarsen2(_p(c), n, _p(cc), _p(f2c), _p(ch), _p(inv))
    return nc, cc[:nc].copy(), f2c, ch[: 8 * nc].copy(), inv[:nc].copy()


def subdivide2(parents: np.ndarray):
    p = _c(parents, np.int32)
    n = p.shape[0]
    child = np.empty((8 * n, 4), np.int32)
    nbr = np.empty((8 * n, 27), np.int32)
    ok = lib().orc_subdivide2(_p(p), n, _p(child), _p(nbr))
    return (child, nbr) if ok else None


def conv(x: np.ndarray, kmap, n_in: int, w: np.ndarray, layout: int, cout: int, bias=None,
         kvol: int = 27, n_out: int = None) -> np.ndarray:
    x = _c(x, np.float32)
    cin = x.shape[1]
    k = _c(kmap, np.int32)
    if n_out is None:
        n_out = k.shape[0] if k is not None else x.shape[0]
    w = _c(w, np.float32)
    b = _c(bias, np.float32)
    y = np.empty((n_out, cout), np.float32)
    lib().orc_conv_subm(_p(x), n_in, cin, _p(k), n_out, kvol, _p(w), layout, cout, _p(b), _p(y))
    return y


def layernorm(x, eps, w=None, b=None):
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().orc_layernorm(_p(x), x.shape[0], x.shape[1], eps, _p(_c(w, np.float32)), _p(_c(b, np.float32)), _p(y))
    return y


def groupnorm(x, groups, eps, w=None, b=None):
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().orc_groupnorm(_p(x), x.shape[0], x.shape[1], groups, eps, _p(_c(w, np.float32)),
                        _p(_c(b, np.float32)), _p(y))
    return y


def silu(x):
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().orc_silu(_p(x), x.size, _p(y))
    return y


def modulate(h, scale, shift):
    h = _c(h, np.float32)
    y = np.empty_like(h)
    lib().orc_modulate(_p(h), h.shape[0], h.shape[1], _p(_c(scale, np.float32)), _p(_c(shift, np.float32)), _p(y))
    return y


def downsample_mean(x, children, inv_count, nc):
    x = _c(x, np.float32)
    y = np.empty((nc, x.shape[1]), np.float32)
    lib().orc_downsample_mean(_p(x), x.shape[0], x.shape[1], _p(_c(children, np.int32)),
                              _p(_c(inv_count, np.float32)), nc, _p(y))
    return y


def upsample_nearest(coarse, f2c):
    coarse = _c(coarse, np.float32)
    f = _c(f2c, np.int32)
    y = np.empty((f.shape[0], coarse.shape[1]), np.float32)
    lib().orc_upsample_nearest(_p(coarse), coarse.shape[0], coarse.shape[1], _p(f), f.shape[0], _p(y))
    return y


def repeat_children(x):
    x = _c(x, np.float32)
    y = np.empty((8 * x.shape[0], x.shape[1]), np.float32)
    lib().orc_repeat_children(_p(x), x.shape[0], x.shape[1], _p(y))
    return y


def occupancy_coords(occ: np.ndarray) -> np.ndarray:
    o = _c(occ, np.float32)
    res = o.shape[0]
    out = np.empty((res ** 3, 4), np.int32)
    n = lib().orc_occupancy_coords(_p(o), res, _p(out))
    return out[:n].copy()


def prune_surface(coords: np.ndarray) -> np.ndarray:
    c = _c(coords, np.int32)
    out = np.empty_like(c)
    m = lib().orc_prune_surface(_p(c), c.shape[0], _p(out))
    return out[:m].copy()


def downsample_coords(coords: np.ndarray, max_coords: int = 42000, factor: int = 2,
                      seed: int = 42) -> np.ndarray:
    c = _c(coords, np.int32)
    n = c.shape[0]
    out = np.empty((max(1, min(n, max_coords)), 4), np.int32)
    m = lib().orc_downsample_coords(_p(c), n, max_coords, factor, seed, _p(out))
    return out[:m].copy()


def mt19937_draw(seed: int, k: int) -> int:
    return int(lib().orc_mt19937_draw(seed, k))


def conv_im2col_gemm_f32(x, kmap, n_in, w_slat, cout, bias, threads: int) -> np.ndarray:
    x = _c(x, np.float32)
    k = _c(kmap, np.int32)
    y = np.empty((k.shape[0], cout), np.float32)
    lib().orc_conv_im2col_gemm_f32(_p(x), n_in, x.shape[1], _p(k), k.shape[0], _p(_c(w_slat, np.float32)),
                                   cout, _p(_c(bias, np.float32)), _p(y), threads)
    return y


def round_bf16(x):
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().orc_round_bf16(_p(x), x.size, _p(y))
    return y


# ---- compiled reference (sparse_ops.cpp) ------------------------------------
def ref_slat_tables(coords: np.ndarray, channels: int = 6):
    """SlatTables::build -> (conv_fine, nc, f2c, conv_coarse, children, inv_count)."""
    c = _c(coords, np.int32)
    n = c.shape[0]
    cf = np.empty((n, 27), np.int32)
    f2c = np.empty(n, np.int32)
    cc = np.empty((n, 27), np.int32)
    ch = np.empty(8 * n, np.int32)
    inv = np.empty(n, np.float32)
    nc = ref().ref_slat_tables(_p(c), n, channels, _p(cf), _p(f2c), _p(cc), _p(ch), _p(inv))
    if nc < 0:
        return None
    return cf, int(nc), f2c, cc[:nc].copy(), ch[: 8 * nc].copy(), inv[:nc].copy()


def ref_mesh_subdivide(parents: np.ndarray):
    p = _c(parents, np.int32)
    n = p.shape[0]
    child = np.empty((8 * n, 4), np.int32)
    nbr = np.empty((8 * n, 27), np.int32)
    ok = ref().ref_mesh_subdivide(_p(p), n, _p(child), _p(nbr))
    return (child, nbr) if ok else None
