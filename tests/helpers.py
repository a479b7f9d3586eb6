"""Shared test helpers: named voxel sets rebuilt from the workload generators
and the golden fixtures."""
import hashlib
import struct

import numpy as np


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), np.finfo(np.float64).tiny))


SMALL = ["window_block", "isolated", "duplicates", "negative", "multibatch", "sparse_random",
         "int32_extremes", "shell_r4"]


def large_sets(W, O, arrays):
    """name -> coords for the full-size manifest entries."""
    sets = {"shell_64": W.shell_64()}
    for seed in (0, 1, 2):
        c = W.shells_union(seed)
        sets[f"shells_union_s{seed}"] = c
        sets[f"shells_union_s{seed}_pool2"] = W.or_pool2(c)
    occ = np.unpackbits(arrays["ss_occ.bits"]).reshape(64, 64, 64).astype(np.float32)
    sets["ss_occ_surface"] = O.prune_surface(O.occupancy_coords(occ))
    return sets


BF16_ROW_TOL = 1e-2  # worst row's rel-L2, BF16 gates
BF16_ABS_TOL = 1e-2  # worst element's |error| / max |ref|, BF16 gates


def row_errors(got, ref):
    """(worst row rel-L2, worst |error| / max |ref|) over the rows of 2-D
    arrays (1-D: one row).  A row's norm is floored at 0.1 x the RMS row norm,
    so near-zero rows are judged against the scale of the whole output."""
    a = np.asarray(got, np.float64)
    b = np.asarray(ref, np.float64)
    a = a.reshape(1, -1) if a.ndim == 1 else a.reshape(a.shape[0], -1)
    b = b.reshape(1, -1) if b.ndim == 1 else b.reshape(b.shape[0], -1)
    d = a - b
    rn = np.sqrt(np.einsum("ij,ij->i", b, b))
    floor = max(0.1 * float(np.sqrt(np.mean(rn * rn))), np.finfo(np.float64).tiny)
    row = float(np.max(np.sqrt(np.einsum("ij,ij->i", d, d)) / np.maximum(rn, floor))) if d.size else 0.0
    big = float(np.max(np.abs(b))) if b.size else 0.0
    mabs = float(np.max(np.abs(d)) / max(big, np.finfo(np.float64).tiny)) if d.size else 0.0
    return row, mabs


def check_rel(got, ref, tol, what="") -> float:
    """Asserts rel-L2(got, ref) <= tol, printing the measured value first.
    BF16-level gates (tol >= 1e-3) also bound the worst row (rel-L2 <= 1e-2)
    and the worst element (|error| <= 1e-2 max |ref|): a localized error --
    a wrong halo slot, a tail tile, a missed neighbour in 0.1% of rows --
    stays under a global 1e-2 but not under these (a row missing one of ~21
    neighbours is off by ~0.2)."""
    e = rel_l2(got, ref)
    if tol >= 1e-3:
        row, mabs = row_errors(got, ref)
        print(f"  rel-L2 {e:.3e} (gate {tol:.0e}), worst row {row:.3e}, max-abs/max {mabs:.3e} "
              f"(gates {BF16_ROW_TOL:.0e}) {what}", flush=True)
        assert e <= tol, (what, e, tol)
        assert row <= BF16_ROW_TOL, (what, "worst row", row)
        assert mabs <= BF16_ABS_TOL, (what, "max abs", mabs)
        return e
    print(f"  rel-L2 {e:.3e} (gate {tol:.0e}) {what}", flush=True)
    assert e <= tol, (what, e, tol)
    return e


def _coordinate_key(b, x, y, z):
    """session.cpp:122-127 in Python integers: the four fields as uint32,
    shifted by 48/32/16/0 into one uint64 (z masked to 16 bits), so fields
    wider than 16 bits overlap their neighbours' bits."""
    m32 = 0xFFFFFFFF
    return (((b & m32) << 48) | ((x & m32) << 32) | ((y & m32) << 16) | (z & 0xFFFF)) & 0xFFFFFFFFFFFFFFFF


def _wrap32(v):
    return (v + 2 ** 31) % 2 ** 32 - 2 ** 31


def prune_brute_force(coords):
    """prune_surface_coords (session.cpp:133-163) written independently of the
    oracle: a Python set of coordinate keys, and a row is kept (in input
    order) when some cell of its 3x3x3 neighbourhood in its own batch has a
    key outside the set."""
    rows = [tuple(int(v) for v in r) for r in coords]
    occupied = {_coordinate_key(*r) for r in rows}
    keep = []
    for b, x, y, z in rows:
        if any(_coordinate_key(b, _wrap32(x + dx), _wrap32(y + dy), _wrap32(z + dz)) not in occupied
               for dx in (-1, 0, 1) for dy in (-1, 0, 1) for dz in (-1, 0, 1)):
            keep.append((b, x, y, z))
    return np.array(keep, np.int32).reshape(-1, 4)


def prune_cases():
    """Sets the reference's prune is exercised on: two batches with negative
    coordinates and duplicated rows, a solid cube (only its shell survives),
    and cells whose coordinate_key aliases another cell's."""
    rng = np.random.default_rng(5)
    blobs = rng.integers(-5, 7, size=(2500, 4)).astype(np.int32)
    blobs[:, 0] = rng.integers(0, 2, size=blobs.shape[0])
    blobs = np.unique(blobs, axis=0)
    blobs = np.concatenate([blobs, blobs[::53]], 0)[rng.permutation(blobs.shape[0] + len(blobs[::53]))]
    g = np.arange(1, 8, dtype=np.int32)
    x, y, z = np.meshgrid(g, g, g, indexing="ij")
    cube = np.stack([np.full_like(x, 3), x, y, z], -1).reshape(-1, 4)
    # A cube at negative coordinates: y's sign bits spill into x's field
    # (y << 16 as uint64), so its keys alias one another.
    neg = cube.copy()
    neg[:, 1:] -= 9
    # Aliasing: the centre (0,6,6,6) of the block [5,7]^3 lacks its +x
    # neighbour (0,7,6,6), but (0,6,65542,6) has that key
    # ((6<<32) | ((65542<<16)) == (7<<32) | (6<<16)), so the reference sees
    # the neighbour as present and drops the centre.  (0,6,6,65542) shares
    # the centre's key through the 16-bit z mask.
    g3 = np.arange(5, 8, dtype=np.int32)
    x, y, z = np.meshgrid(g3, g3, g3, indexing="ij")
    block = np.stack([np.zeros_like(x), x, y, z], -1).reshape(-1, 4)
    block = block[~np.all(block == [0, 7, 6, 6], axis=1)]
    alias = np.concatenate([block, [[0, 6, 65542, 6], [0, 6, 6, 65542], [0, -1, 7, 2]]], 0).astype(np.int32)
    return {"blobs_two_batches_duplicates": blobs, "solid_cube": cube, "negative_cube": neg,
            "key_aliasing": alias}


def gguf_bytes(kv, tensors, align=32):
    """A GGUF v3 file: header, metadata, tensor infos, aligned data."""
    def s(x):
        b = x.encode()
        return struct.pack("<Q", len(b)) + b
    out = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kv))
    for k, (vt, v) in kv.items():
        out += s(k) + struct.pack("<I", vt)
        if vt == 8:
            out += s(v)
        elif vt == 9:
            out += struct.pack("<IQ", 4, len(v)) + b"".join(struct.pack("<I", e) for e in v)
        else:
            out += struct.pack({4: "<I", 6: "<f", 10: "<Q"}[vt], v)
    blobs, off = [], 0
    for name, (gtype, arr) in tensors.items():
        out += s(name) + struct.pack("<I", arr.ndim) + struct.pack(f"<{arr.ndim}Q", *reversed(arr.shape))
        out += struct.pack("<IQ", gtype, off)
        blob = arr.tobytes()
        pad = (-len(blob)) % align
        blobs.append(blob + b"\0" * pad)
        off += len(blob) + pad
    out += b"\0" * ((-len(out)) % align)
    return out + b"".join(blobs)


# ---- test-only hooks of libs3dx_sparse.so (exported, not in the public header)

def _mix32(h):
    m = 0xFFFFFFFF
    h ^= h >> 16
    h = (h * 0x7FEB352D) & m
    h ^= h >> 15
    h = (h * 0x846CA68B) & m
    h ^= h >> 16
    return h


def window_cell_index(x, y, z):
    """Index of batch-0 cell (x, y, z) in the kernel-map table's 64^3 window."""
    return (x * 64 + y) * 64 + z


def colliding_seed(cell_index):
    """The kernel-map seed whose tag for this window cell is 0: the tag is
    mix32(seed ^ cell * 0x9E3779B1), mix32 is a bijection with mix32(0) == 0,
    so a zero-filled word carries the current tag exactly for this seed."""
    seed = (cell_index * 0x9E3779B1) & 0xFFFFFFFF
    assert _mix32(seed ^ ((cell_index * 0x9E3779B1) & 0xFFFFFFFF)) == 0
    return seed


def flag_value(seed, k):
    """The value flag word k holds when raised by the build with this seed."""
    v = _mix32((seed + 0x632BE5AB * (k + 1)) & 0xFFFFFFFF)
    return v - (1 << 32) if v >= 1 << 31 else v


def kmap_flags_offset(n):
    """Byte offset of the flag words in a kernel-map workspace for n voxels:
    the window of 8-byte cells (64^3, or 128^3 / 256^3 when those take no
    more bytes than the slots), then the 16-byte slots (power of two, >= 4n,
    >= 256), each region a multiple of 256 bytes."""
    cap = 256
    while cap < 4 * n:
        cap <<= 1
    lg = 6
    while lg < 8 and 8 << (3 * (lg + 1)) <= cap * 16:
        lg += 1
    return (8 << (3 * lg)) + cap * 16


def set_kmap_seed(s3dx, seed):
    import ctypes as C
    fn = s3dx.lib().s3dx_testing_set_kmap_seed
    fn.restype = C.c_uint32
    fn.argtypes = [C.c_uint32, C.c_char_p, C.c_uint64]
    buf = C.create_string_buffer(256)
    assert fn(seed, buf, len(buf)) == 0, buf.value


def zero_static_kmap(s3dx):
    import ctypes as C
    fn = s3dx.lib().s3dx_testing_zero_static_kmap
    fn.restype = C.c_uint32
    fn.argtypes = [C.c_void_p, C.c_char_p, C.c_uint64]
    buf = C.create_string_buffer(256)
    assert fn(None, buf, len(buf)) == 0, buf.value
