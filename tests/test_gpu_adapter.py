"""The compiled C++ consumer of the ABI (sam3d.cpp_amd/adapter, libs3dx_adapter.so):
the adapter a sam3d.cpp maintainer adds, built by the host C++ compiler
against include/s3dx_sparse.h alone, called in this process through ctypes.

- DeviceSlatTables reproduces the reference's own tables (SHA-256 of the
  golden manifest, written by the compiled sparse_ops.cpp);
- device_subdivide reproduces MeshSubdivideTables, and returns false where
  the reference does (duplicate parents);
- SlatResBlock runs the SLat res_block with a new device modulate per
  forward (FP32 and BF16 layers; odd forwards with the map's gather plan);
- SlatSparseStages runs one SLat forward's sparse input and output stages
  in the hand-off order of a graph split at them (host rows in and out, as
  Backend::get_tensor_f32 / set_input_f32 give them);
- MeshDecoderStack runs both mesh levels and the head from the dense base's
  host output to extract_object_mesh's inputs (raw rows + coordinates).
Gates against the oracle: rel-L2 1e-5 FP32, 1e-2 BF16 (the oracle rounds
every tensor the BF16 layers store).
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
    lib.s3dx_adapter_res_block.argtypes = [_vp, _i64, _i32, _i32, _i32, _vp, _vp, _i32, _vp, _vp, C.c_char_p, _u64]
    lib.s3dx_adapter_slat_stages.argtypes = [_vp, _i64, _i32, _vp, _vp, _vp, _vp, C.POINTER(_i64), _vp, _vp,
                                             C.c_char_p, _u64]
    lib.s3dx_adapter_mesh_decoder.argtypes = [_vp, _i64, _i32, _vp, _vp, _vp, _vp, C.c_char_p, _u64]
    for f in (lib.s3dx_adapter_slat_tables, lib.s3dx_adapter_subdivide, lib.s3dx_adapter_res_block,
              lib.s3dx_adapter_slat_stages, lib.s3dx_adapter_mesh_decoder):
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


def _ptrs(arrays):
    """A C array of float pointers (NULL for None); keeps the arrays alive."""
    keep = [None if a is None else np.ascontiguousarray(a, np.float32) for a in arrays]
    arr = (_vp * len(keep))(*[None if a is None else a.ctypes.data for a in keep])
    return arr, keep


def _block_params(W, seed, cin, cout):
    g = lambda k, shape, s=1.0: W.normal_f32(seed, k, shape, s)  # noqa: E731
    skip = cin != cout
    return [g(2, (cin,), 0.2) + 1.0, g(3, (cin,), 0.2), W.conv_weight(seed, 4, cin, cout), g(5, (cout,), 0.1),
            W.conv_weight(seed, 6, cout, cout), g(7, (cout,), 0.1),
            W.conv_weight(seed, 8, cin, cout, kvol=1) if skip else None, g(9, (cout,), 0.1) if skip else None]


def _block_oracle(O, W, prm, x, kmap, n, cout, emb, dtype):
    """The res_block (slat_flow_graph.cpp:216-275) in float64, rounding every
    tensor a BF16 layer stores (its input, the LayerNorm+SiLU rows, conv1's
    finished rows, the skip, the output)."""
    st = (lambda a: W.round_bf16(a)) if dtype == 1 else (lambda a: a)
    n1w, n1b, w1, b1, w2, b2, ws, bs = prm
    x = st(x)
    h = st(O.silu(O.layernorm(x, 1e-6, n1w, n1b)))
    y1 = O.conv(h, kmap, n, st(w1), 0, cout, b1)
    y1 = st(O.silu(O.modulate(O.layernorm(y1, 1e-6), emb[:cout], emb[cout:])))
    skip = x if ws is None else st(O.conv(x, None, n, st(ws), 0, cout, bs, kvol=1))
    return st(O.conv(y1, kmap, n, st(w2), 0, cout, b2) + skip)


TOLS = {0: 1e-5, 1: 1e-2}


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("cin,cout", [(128, 128), (256, 128)])
def test_adapter_res_block(adapter, O, W, cin, cout, dtype):
    coords = np.ascontiguousarray(W.shell_64(res=24, centre=(12.0, 12.0, 12.0), radius=7.0), np.int32)
    n = coords.shape[0]
    prm = _block_params(W, 90, cin, cout)
    x = W.normal_f32(90, 1, (n, cin))
    fwd = 2
    emb = W.normal_f32(90, 10, (fwd, 2 * cout), 0.3)
    y = np.empty((fwd, n, cout), np.float32)
    err = C.create_string_buffer(512)
    wp, keep = _ptrs(prm)
    st = adapter.s3dx_adapter_res_block(_p(coords), n, cin, cout, dtype, _p(x), wp, fwd, _p(emb), _p(y), err,
                                        len(err))
    assert st == 0, err.value
    kmap = O.kmap_subm3(coords, n)
    for f in range(fwd):
        ref = _block_oracle(O, W, prm, x, kmap, n, cout, emb[f], dtype)
        check_rel(y[f], ref, TOLS[dtype], f"adapter res_block {cin}->{cout} dtype {dtype} forward {f}")


@pytest.mark.parametrize("dtype", [0, 1])
def test_adapter_slat_stages(adapter, O, W, dtype):
    # One SLat forward's sparse stages through the adapter, in the order a
    # split graph would hand them rows, against the oracle's chain
    # (slat_flow_graph.cpp:284-291, 441-503): input_blocks.0 -> 2x mean-pool
    # -> input_blocks.1 = skip1; the trunk's output (random rows here) ->
    # concat skip1 -> upsample -> out_blocks.0 -> concat skip0 -> out_blocks.1.
    coords = np.ascontiguousarray(W.shell_64(res=24, centre=(12.0, 12.0, 12.0), radius=7.0), np.int32)
    n = coords.shape[0]
    dims = ((128, 128), (128, 1024), (2048, 128), (256, 128))
    prms = [_block_params(W, 120 + b, ci, co) for b, (ci, co) in enumerate(dims)]
    embs = [W.normal_f32(130 + b, 1, (2 * co,), 0.3) for b, (ci, co) in enumerate(dims)]
    h0 = W.normal_f32(140, 1, (n, 128))
    nc_o, cc, f2c, ch, inv = O.coarsen2(coords)
    h_trunk = W.normal_f32(141, 1, (nc_o, 1024))
    wp, keep = _ptrs(sum(prms, []))
    emb = np.concatenate(embs).astype(np.float32)
    nc = _i64(0)
    skip1 = np.empty((n, 1024), np.float32)
    out = np.empty((n, 128), np.float32)
    err = C.create_string_buffer(512)
    hp = np.zeros((n, 1024), np.float32)
    hp[:nc_o] = h_trunk
    st = adapter.s3dx_adapter_slat_stages(_p(coords), n, dtype, wp, _p(h0), _p(emb), _p(hp), C.byref(nc), _p(skip1),
                                          _p(out), err, len(err))
    assert st == 0, err.value
    assert nc.value == nc_o
    print(f"slat stages dtype={dtype} nf={n} nc={nc_o}", flush=True)
    rd = (lambda a: W.round_bf16(a)) if dtype == 1 else (lambda a: a)
    kf, kc = O.kmap_subm3(coords, n), O.kmap_subm3(np.ascontiguousarray(cc), nc_o)
    s0 = _block_oracle(O, W, prms[0], h0, kf, n, 128, embs[0], dtype)
    xc = rd(O.downsample_mean(s0, ch, inv, nc_o))
    s1 = _block_oracle(O, W, prms[1], xc, kc, nc_o, 1024, embs[1], dtype)
    check_rel(skip1[:nc_o], s1, TOLS[dtype], f"dtype {dtype} skip1 (input stage)")
    # the output stage from the adapter's own skip1, as the trunk would see it
    xcat = O.upsample_nearest(np.concatenate([rd(h_trunk), skip1[:nc_o]], 1), f2c)
    h1 = _block_oracle(O, W, prms[2], xcat, kf, n, 128, embs[2], dtype)
    ref = _block_oracle(O, W, prms[3], np.concatenate([h1, s0], 1), kf, n, 128, embs[3], dtype)
    check_rel(out, ref, TOLS[dtype], f"dtype {dtype} out (output stage)")


@pytest.mark.parametrize("dtype", [0, 1])
def test_adapter_mesh_decoder(adapter, O, W, dtype):
    # Both mesh levels and the head from the base graph's host output
    # (session.cpp:927-975): the raw rows and the child coordinates that
    # extract_object_mesh reads, against the oracle level by level.
    parents = np.ascontiguousarray(W.shell_64(res=12, centre=(6.0, 6.0, 6.0), radius=3.0), np.int32)
    p = parents.shape[0]
    g = lambda k, shape, s=1.0: W.normal_f32(150, k, shape, s)  # noqa: E731
    prm = []
    for lv, (ci, co) in enumerate(((768, 192), (192, 96))):
        o = 20 * lv
        prm += [g(o + 1, (ci,), 0.2) + 1.0, g(o + 2, (ci,), 0.2), W.conv_weight(150, o + 3, ci, co, layout="mesh"),
                g(o + 4, (co,), 0.1), W.conv_weight(150, o + 5, ci, co, kvol=1, layout="mesh"), g(o + 6, (co,), 0.1),
                g(o + 7, (co,), 0.2) + 1.0, g(o + 8, (co,), 0.2), W.conv_weight(150, o + 9, co, co, layout="mesh"),
                g(o + 10, (co,), 0.1)]
    prm += [W.conv_weight(150, 60, 96, 101, kvol=1), g(61, (101,), 0.1)]
    feats = g(0, (p, 768))
    wp, keep = _ptrs(prm)
    raw = np.empty((64 * p, 101), np.float32)
    child = np.empty((64 * p, 4), np.int32)
    err = C.create_string_buffer(512)
    st = adapter.s3dx_adapter_mesh_decoder(_p(parents), p, dtype, _p(feats), wp, _p(raw), _p(child), err, len(err))
    assert st == 0, err.value
    print(f"mesh decoder dtype={dtype} parents={p} children={64 * p}", flush=True)
    rd = (lambda a: W.round_bf16(a)) if dtype == 1 else (lambda a: a)
    x, par = rd(feats), parents
    for lv, (ci, co) in enumerate(((768, 192), (192, 96))):
        g1, b1, w1, c1, ws, cs, g2, b2, w2, c2 = prm[10 * lv: 10 * lv + 10]
        kids, kmap = O.subdivide2(par)
        n = kids.shape[0]
        a1 = rd(O.repeat_children(O.silu(O.groupnorm(x, 32, 1e-5, g1, b1))))
        r1 = rd(O.conv(a1, kmap, n, rd(w1), 1, co, c1))
        a2 = rd(O.silu(O.groupnorm(r1, 32, 1e-5, g2, b2)))
        sk = rd(O.conv(O.repeat_children(x), None, n, rd(ws), 1, co, cs, kvol=1))
        x, par = rd(O.conv(a2, kmap, n, rd(w2), 1, co, c2) + sk), kids
    assert np.array_equal(child, par)
    ref = O.conv(x, None, 64 * p, prm[20], 0, 101, prm[21], kvol=1)
    check_rel(raw, ref, TOLS[dtype], f"dtype {dtype} raw [{64 * p}][101]")
