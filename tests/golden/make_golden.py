"""Writes the committed golden fixtures under tests/golden/.

Run in the container that holds the reference tree, after `make -C oracle`:

    python tests/golden/make_golden.py

Sources of truth:
  * kernel maps, coarse tables and subdivide tables come from the reference's
    own sparse_ops.cpp (SlatTables::build, MeshSubdivideTables::build),
    compiled from /root/reference into oracle/_ref/libref_sparse_ops.so;
  * the real occupancy set comes from the reference fixture
    tests/objects_runtime/fixtures/ss_occ_f32.samt (upstream SS-decoder logits),
    stored here as a 64^3 occupancy bitmap;
  * dense-occupancy convolution and the LayerNorm / GroupNorm / SiLU vectors
    come from torch's CPU conv3d / layer_norm / group_norm / silu (a library
    routine; the sparse conv on a fully dense block equals a zero-padded 3x3x3
    conv3d).
Small cases are stored whole (npz, no pickles); full-size tables are pinned by
SHA-256 of their little-endian bytes in manifest.json.
"""
from __future__ import annotations

import hashlib
import json
import struct
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
import __graft_entry__ as ge  # noqa: E402

OUT = Path(__file__).resolve().parent
REF_FIXTURE = Path("/root/reference/tests/objects_runtime/fixtures/ss_occ_f32.samt")


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def read_samt_f32(path: Path) -> np.ndarray:
    # SAMT: magic "SAMT" | int32 ndims | int64 ne[ndims] | int32 type | data
    raw = path.read_bytes()
    magic, nd = struct.unpack_from("<Ii", raw, 0)
    assert magic == 0x544D4153, hex(magic)
    ne = struct.unpack_from(f"<{nd}q", raw, 8)
    (typ,) = struct.unpack_from("<i", raw, 8 + 8 * nd)
    assert typ == 0, typ  # GGML_TYPE_F32
    data = np.frombuffer(raw, dtype="<f4", offset=12 + 8 * nd)
    assert data.size == int(np.prod(ne))
    return data


def small_cases(W):
    rng = np.random.default_rng(1234)
    cases = {}
    xyz = np.stack(np.meshgrid(np.arange(30, 33), np.arange(30, 33), np.arange(30, 33),
                               indexing="ij"), -1).reshape(-1, 3)
    cases["window_block"] = np.concatenate([np.zeros((27, 1), int), xyz], 1)
    cases["isolated"] = np.array([[0, 5, 5, 5], [0, 9, 9, 9], [0, 5, 5, 7]])
    d = rng.integers(0, 6, size=(120, 3))
    dup = np.concatenate([np.zeros((120, 1), int), d], 1)
    cases["duplicates"] = dup  # many repeated coordinates, unsorted
    neg = rng.integers(-5, 5, size=(150, 3))
    cases["negative"] = np.unique(np.concatenate([np.zeros((150, 1), int), neg], 1), axis=0)
    mb = rng.integers(0, 7, size=(200, 4))
    mb[:, 0] = rng.integers(0, 3, size=200)
    cases["multibatch"] = np.unique(mb, axis=0)
    rng.shuffle(cases["multibatch"])  # unsorted input order
    sp = rng.integers(0, 40, size=(400, 3))
    cases["sparse_random"] = np.unique(np.concatenate([np.zeros((400, 1), int), sp], 1), axis=0)
    big = np.array([[0, 2**31 - 1, -2**31, 7], [0, 2**31 - 2, -2**31, 7], [1, 0, 0, 0],
                    [0, 2**31 - 1, -2**31 + 1, 7], [-3, 4, 4, 4], [-3, 5, 4, 4]])
    cases["int32_extremes"] = big
    cases["shell_r4"] = W.shell_64(res=12, centre=(6.0, 6.0, 6.0), radius=4.0)
    return {k: np.ascontiguousarray(v, dtype=np.int32) for k, v in cases.items()}


def write_tables(O, name: str, coords: np.ndarray, store: dict, manifest: dict, whole: bool):
    slat = O.ref_slat_tables(coords)
    assert slat is not None, name
    cf, nc, f2c, cc, ch, inv = slat
    entry = {"n": int(coords.shape[0]), "nc": nc, "coords_sha256": sha(coords),
             "conv_fine_sha256": sha(cf), "fine_to_coarse_sha256": sha(f2c),
             "conv_coarse_sha256": sha(cc), "coarse_children_sha256": sha(ch),
             "coarse_inv_count_sha256": sha(inv),
             "pairs": int(np.count_nonzero(cf != coords.shape[0]))}
    if whole:
        store[f"{name}.coords"] = coords
        store[f"{name}.conv_fine"] = cf
        store[f"{name}.fine_to_coarse"] = f2c
        store[f"{name}.conv_coarse"] = cc
        store[f"{name}.coarse_children"] = ch
        store[f"{name}.coarse_inv_count"] = inv
    sub = O.ref_mesh_subdivide(coords)
    if sub is None:
        entry["subdivide"] = "rejected"
    else:
        child, nbr = sub
        entry["subdivide"] = {"child_coords_sha256": sha(child), "neighbors_sha256": sha(nbr)}
        if whole:
            store[f"{name}.child_coords"] = child
            store[f"{name}.neighbors"] = nbr
    manifest[name] = entry


def conv_vectors(store: dict):
    import torch

    g = torch.Generator().manual_seed(7)
    res, cin, cout = 6, 8, 12
    x = torch.randn(cin, res, res, res, generator=g)
    w = torch.randn(cout, cin, 3, 3, 3, generator=g) * 0.2
    b = torch.randn(cout, generator=g)
    y = torch.nn.functional.conv3d(x[None], w, b, padding=1)[0]
    xyz = np.stack(np.meshgrid(*[np.arange(res)] * 3, indexing="ij"), -1).reshape(-1, 3)
    store["dense_conv.coords"] = np.concatenate([np.zeros((len(xyz), 1), int), xyz], 1).astype(np.int32)
    store["dense_conv.x"] = x.permute(1, 2, 3, 0).reshape(-1, cin).numpy()
    # SLat weight layout [cout][27][cin] with o = kd*9 + kh*3 + kw.
    store["dense_conv.w_slat"] = w.permute(0, 2, 3, 4, 1).reshape(cout, 27, cin).numpy()
    store["dense_conv.bias"] = b.numpy()
    store["dense_conv.y"] = y.permute(1, 2, 3, 0).reshape(-1, cout).numpy()

    xn = torch.randn(50, 96, generator=g) * 3 + 1
    wn = torch.randn(96, generator=g)
    bn = torch.randn(96, generator=g)
    store["norm.x"] = xn.numpy()
    store["norm.w"] = wn.numpy()
    store["norm.b"] = bn.numpy()
    store["norm.layer_norm"] = torch.nn.functional.layer_norm(xn, (96,), wn, bn, 1e-6).numpy()
    # SparseGroupNorm: all rows of one batch form the spatial extent.
    gn = torch.nn.functional.group_norm(xn.t()[None], 32, wn, bn, 1e-5)[0].t()
    store["norm.group_norm"] = gn.contiguous().numpy()
    store["norm.silu"] = torch.nn.functional.silu(xn).numpy()


def main():
    O = ge.load_oracle()
    W = ge.load_package().workloads
    assert O.ref_available(), "build oracle/_ref first (make -C oracle)"
    store, manifest = {}, {}
    for name, coords in small_cases(W).items():
        write_tables(O, name, coords, store, manifest, whole=True)
    write_tables(O, "shell_64", W.shell_64(), store, manifest, whole=False)
    for seed in (0, 1, 2):
        c = W.shells_union(seed)
        write_tables(O, f"shells_union_s{seed}", c, store, manifest, whole=False)
        write_tables(O, f"shells_union_s{seed}_pool2", W.or_pool2(c), store, manifest, whole=False)
    # Real occupancy: logits > 0 in x-major order, then the surface rule.
    occ = read_samt_f32(REF_FIXTURE).reshape(64, 64, 64)
    bits = np.packbits((occ > 0).reshape(-1))
    store["ss_occ.bits"] = bits
    coords = O.occupancy_coords(occ)
    surface = O.prune_surface(coords)
    manifest["ss_occ"] = {"occupied": int(coords.shape[0]), "surface": int(surface.shape[0]),
                          "occupied_sha256": sha(coords), "surface_sha256": sha(surface)}
    write_tables(O, "ss_occ_surface", surface, store, manifest, whole=False)
    conv_vectors(store)
    np.savez_compressed(OUT / "golden.npz", **store)
    (OUT / "manifest.json").write_text(json.dumps(manifest, indent=1, sort_keys=True) + "\n")
    print(f"wrote {len(store)} arrays, {len(manifest)} manifest entries")


if __name__ == "__main__":
    main()
