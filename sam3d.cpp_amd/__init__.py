"""Python host mirror of the s3dx sparse-voxel C ABI (include/s3dx_sparse.h).

Loads the in-tree libs3dx_sparse.so with ctypes and exposes the reference's
operator interface for this path:

  SlatTables.build(coords)             sparse_ops.hpp:36  (fine/coarse maps,
                                       downsample tables; APE excluded)
  MeshSubdivideTables.build(parents)   sparse_ops.hpp:77
  SparseConv(...).run(...)             slat_flow_graph.cpp:112-155 conv lambda,
                                       mesh_decoder_graph.cpp:81-103 convolution

Device memory is plain device pointers owned by DeviceArray.  There is no
fallback: if the HIP library cannot be loaded, import fails loudly.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

from . import formats  # noqa: F401  (re-exported)
from . import workloads  # noqa: F401  (re-exported)

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libs3dx_sparse.so"

F32 = 0
BF16 = 1
WEIGHT_SLAT = 0
WEIGHT_MESH = 1

OK, INVALID_ARGUMENT, OUT_OF_MEMORY, INTERNAL_ERROR = 0, 1, 2, 3


class S3dxError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"s3dx status {status}: {message}")
        self.status = status


_vp, _i32, _i64, _u32, _u64, _f32 = C.c_void_p, C.c_int32, C.c_int64, C.c_uint32, C.c_uint64, C.c_float
_err = [C.c_char_p, _u64]

# name -> (restype, argtypes without the trailing error buffer, has_error_buffer)
SIGNATURES = {
    "s3dx_abi_version": (_u32, [], False),
    "s3dx_device_info": (_u32, [C.POINTER(_i32), C.c_char_p, _u64], True),
    "s3dx_malloc": (_u32, [C.POINTER(_vp), _u64], True),
    "s3dx_free": (None, [_vp], False),
    "s3dx_memcpy_h2d": (_u32, [_vp, _vp, _u64, _vp], True),
    "s3dx_memcpy_d2h": (_u32, [_vp, _vp, _u64, _vp], True),
    "s3dx_stream_create": (_u32, [C.POINTER(_vp)], True),
    "s3dx_stream_destroy": (_u32, [_vp], True),
    "s3dx_stream_synchronize": (_u32, [_vp], True),
    "s3dx_event_create": (_u32, [C.POINTER(_vp)], True),
    "s3dx_timing_event_create": (_u32, [C.POINTER(_vp)], True),
    "s3dx_event_destroy": (_u32, [_vp], True),
    "s3dx_event_record": (_u32, [_vp, _vp], True),
    "s3dx_event_elapsed_ms": (_u32, [_vp, _vp, C.POINTER(_f32)], True),
    "s3dx_kmap_workspace_size": (_u32, [_i64, C.POINTER(_u64)], True),
    "s3dx_kmap_subm3": (_u32, [_vp, _i64, _i32, _vp, _vp, _u64, _vp], True),
    "s3dx_kmap_subm3_static": (_u32, [_vp, _i64, _i32, _vp, _vp], True),
    "s3dx_coarsen2_workspace_size": (_u32, [_i64, C.POINTER(_u64)], True),
    "s3dx_coarsen2": (_u32, [_vp, _i64, _vp, _vp, _vp, _vp, C.POINTER(_i64), _vp, _u64, _vp], True),
    "s3dx_occupancy_workspace_size": (_u32, [_i32, _i32, _i32, C.POINTER(_u64)], True),
    "s3dx_occupancy_coords": (_u32, [_vp, _i32, _i32, _i32, _vp, C.POINTER(_i64), _vp, _u64, _vp], True),
    "s3dx_prune_surface_workspace_size": (_u32, [_i64, C.POINTER(_u64)], True),
    "s3dx_prune_surface": (_u32, [_vp, _i64, _vp, C.POINTER(_i64), _vp, _u64, _vp], True),
    "s3dx_downsample_coords_workspace_size": (_u32, [_i64, C.POINTER(_u64)], True),
    "s3dx_downsample_coords": (_u32, [_vp, _i64, _i64, _i32, _u32, _vp, C.POINTER(_i64), _vp, _u64, _vp],
                               True),
    "s3dx_subdivide2_workspace_size": (_u32, [_i64, C.POINTER(_u64)], True),
    "s3dx_subdivide2": (_u32, [_vp, _i64, _vp, _vp, _vp, _u64, _vp], True),
    "s3dx_conv_create": (_u32, [_i32, _i32, _i32, _i32, C.POINTER(_vp)], True),
    "s3dx_conv_free": (None, [_vp], False),
    "s3dx_conv_set_weights": (_u32, [_vp, _vp, _i32, _vp], True),
    "s3dx_conv_set_gather_parent": (_u32, [_vp, _i32, _vp], True),
    "s3dx_conv_set_input_affine_silu": (_u32, [_vp, _vp, _vp], True),
    "s3dx_conv_set_layernorm": (_u32, [_vp, _i32, _f32, _vp, _vp, _vp, _vp], True),
    "s3dx_conv_set_modulate": (_u32, [_vp, _vp, _vp], True),
    "s3dx_conv_set_silu": (_u32, [_vp, _i32], True),
    "s3dx_conv_set_residual_parent": (_u32, [_vp, _i32], True),
    "s3dx_conv_set_input_dtype": (_u32, [_vp, _i32], True),
    "s3dx_conv_run": (_u32, [_vp, _vp, _i64, _vp, _i64, _vp, _vp, _i32, _vp], True),
    "s3dx_conv_plan": (_u32, [_vp, _i64, _i64, C.c_char_p, _u64], True),
    "s3dx_gather_plan_create": (_u32, [_vp, _i64, _vp, _i64, _vp, C.POINTER(_vp)], True),
    "s3dx_gather_plan_free": (None, [_vp], False),
    "s3dx_gather_plan_rebuild": (_u32, [_vp, _vp, _i64, _vp, _i64, _vp], True),
    "s3dx_conv_plan_planned": (_u32, [_vp, _vp, _i64, _i64, C.c_char_p, _u64], True),
    "s3dx_kmap_subm3_planned": (_u32, [_vp, _i64, _i32, _vp, _vp, _vp, _vp, _u64, _vp], True),
    "s3dx_conv_run_planned": (_u32, [_vp, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _i32, _vp], True),
    "s3dx_layernorm_rows": (_u32, [_vp, _i32, _i64, _i32, _f32, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _vp], True),
    "s3dx_groupnorm_workspace_size": (_u32, [_i64, _i32, _i32, C.POINTER(_u64)], True),
    "s3dx_groupnorm_stats": (_u32, [_vp, _i32, _i64, _i32, _i32, _f32, _vp, _vp, _vp, _vp, _vp, _u64, _vp], True),
    "s3dx_affine_rows": (_u32, [_vp, _i32, _i64, _i32, _vp, _vp, _i32, _vp, _i32, _vp], True),
    "s3dx_downsample_mean": (_u32, [_vp, _i32, _i64, _i32, _vp, _vp, _i64, _vp, _vp], True),
    "s3dx_upsample_nearest": (_u32, [_vp, _i32, _i64, _i32, _vp, _i64, _vp, _vp], True),
    "s3dx_concat_rows": (_u32, [_vp, _i32, _vp, _i32, _i32, _i64, _vp, _i64, _vp, _vp], True),
    "s3dx_convert": (_u32, [_vp, _i32, _i64, _vp, _i32, _vp], True),
}

_lib = None


def lib() -> C.CDLL:
    """The loaded HIP library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
        handle = C.CDLL(str(LIB_PATH))
        for name, (res, args, has_err) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args + (_err if has_err else [])
        _lib = handle
    return _lib


def call(name: str, *args):
    """Call an error-buffer entry point; raise S3dxError on a non-OK status."""
    buf = C.create_string_buffer(512)
    status = getattr(lib(), name)(*args, buf, len(buf))
    if status != OK:
        raise S3dxError(status, buf.value.decode(errors="replace"))
    return status


def device_count() -> int:
    n = _i32(0)
    name = C.create_string_buffer(256)
    try:
        call("s3dx_device_info", C.byref(n), name, len(name))
    except S3dxError:
        return 0
    return int(n.value)


def device_name() -> str:
    n = _i32(0)
    name = C.create_string_buffer(256)
    call("s3dx_device_info", C.byref(n), name, len(name))
    return name.value.decode()


# ---------------------------------------------------------------------------
# Device memory / streams / events
# ---------------------------------------------------------------------------
class DeviceArray:
    """A device allocation with a numpy-like shape and dtype (uint16 = bf16 bits)."""

    def __init__(self, shape, dtype):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = _vp()
        call("s3dx_malloc", C.byref(p), _u64(max(self.nbytes, 1)))
        self.ptr = p.value

    @classmethod
    def from_host(cls, a: np.ndarray, stream=None) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        d.upload(a, stream)
        return d

    def upload(self, a: np.ndarray, stream=None):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.nbytes, self.nbytes)
        if self.nbytes:
            call("s3dx_memcpy_h2d", _vp(self.ptr), a.ctypes.data_as(_vp), _u64(self.nbytes), _sptr(stream))

    def download(self, stream=None) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        if self.nbytes:
            call("s3dx_memcpy_d2h", out.ctypes.data_as(_vp), _vp(self.ptr), _u64(self.nbytes), _sptr(stream))
        return out

    def free(self):
        if self.ptr:
            lib().s3dx_free(_vp(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        p = _vp()
        call("s3dx_stream_create", C.byref(p))
        self.handle = p.value

    def synchronize(self):
        call("s3dx_stream_synchronize", _vp(self.handle))

    def __del__(self):
        try:
            if self.handle:
                lib().s3dx_stream_destroy(_vp(self.handle), None, 0)
        except Exception:
            pass


class Event:
    """A HIP event; timing=True: for measuring intervals only (no system-scope
    fence on record, see s3dx_timing_event_create)."""

    def __init__(self, timing: bool = False):
        p = _vp()
        call("s3dx_timing_event_create" if timing else "s3dx_event_create", C.byref(p))
        self.handle = p.value

    def record(self, stream=None):
        call("s3dx_event_record", _vp(self.handle), _sptr(stream))

    def elapsed_ms(self, stop: "Event") -> float:
        ms = _f32(0)
        call("s3dx_event_elapsed_ms", _vp(self.handle), _vp(stop.handle), C.byref(ms))
        return float(ms.value)

    def __del__(self):
        try:
            if self.handle:
                lib().s3dx_event_destroy(_vp(self.handle), None, 0)
        except Exception:
            pass


def _sptr(stream):
    if stream is None:
        return _vp(None)
    return _vp(stream.handle if isinstance(stream, Stream) else stream)


def _dptr(a):
    if a is None:
        return _vp(None)
    return _vp(a.ptr if isinstance(a, DeviceArray) else a)


def _host_f32(a):
    if a is None:
        return None, _vp(None)
    arr = np.ascontiguousarray(a, dtype=np.float32)
    return arr, arr.ctypes.data_as(_vp)


# ---------------------------------------------------------------------------
# Kernel maps
# ---------------------------------------------------------------------------
def kmap_workspace_size(n: int) -> int:
    b = _u64(0)
    call("s3dx_kmap_workspace_size", _i64(n), C.byref(b))
    return int(b.value)


def kmap_subm3(coords: DeviceArray, n: int, missing: int, kmap: DeviceArray = None,
               workspace: DeviceArray = None, stream=None) -> DeviceArray:
    """Submanifold 3x3x3 neighbour table (build_conv, sparse_ops.cpp:117-142)."""
    if kmap is None:
        kmap = DeviceArray((n, 27), np.int32)
    if workspace is None:
        workspace = DeviceArray(kmap_workspace_size(n), np.uint8)
    call("s3dx_kmap_subm3", _dptr(coords), _i64(n), _i32(missing), _dptr(kmap), _dptr(workspace),
         _u64(workspace.nbytes), _sptr(stream))
    return kmap


def kmap_subm3_planned(coords: DeviceArray, n: int, missing: int, kmap: DeviceArray, plan: "GatherPlan",
                       conv: "SparseConv", workspace: DeviceArray = None, stream=None) -> DeviceArray:
    """kmap_subm3 and plan.rebuild(conv, n, kmap, n) in one pass (s3dx_kmap_subm3_planned)."""
    if workspace is None:
        workspace = DeviceArray(kmap_workspace_size(n), np.uint8)
    call("s3dx_kmap_subm3_planned", _dptr(coords), _i64(n), _i32(missing), _dptr(kmap), _vp(plan.handle),
         _vp(conv.handle), _dptr(workspace), _u64(workspace.nbytes), _sptr(stream))
    return kmap


def kmap_subm3_static(coords: DeviceArray, n: int, missing: int, kmap: DeviceArray = None,
                      stream=None) -> DeviceArray:
    """kmap_subm3 with the library's static table: no workspace, no allocation
    in the library (n <= 262144; calls overlapping on one GPU race)."""
    if kmap is None:
        kmap = DeviceArray((n, 27), np.int32)
    call("s3dx_kmap_subm3_static", _dptr(coords), _i64(n), _i32(missing), _dptr(kmap), _sptr(stream))
    return kmap


def subdivide2_workspace_size(p: int) -> int:
    b = _u64(0)
    call("s3dx_subdivide2_workspace_size", _i64(p), C.byref(b))
    return int(b.value)


def subdivide2(parents: DeviceArray, p: int, with_kmap: bool = True, stream=None, out=None,
               workspace: DeviceArray = None):
    """MeshSubdivideTables::build (sparse_ops.cpp:272-404): (child_coords, child_kmap).
    out = (child [8p, 4], kmap [8p, 27] or None) and workspace may be passed in to
    reuse them across calls."""
    ws = workspace if workspace is not None else DeviceArray(subdivide2_workspace_size(p), np.uint8)
    if out is not None:
        child, kmap = out
        kmap = kmap if with_kmap else None
    else:
        child = DeviceArray((8 * p, 4), np.int32)
        kmap = DeviceArray((8 * p, 27), np.int32) if with_kmap else None
    call("s3dx_subdivide2", _dptr(parents), _i64(p), _dptr(child), _dptr(kmap), _dptr(ws),
         _u64(ws.nbytes), _sptr(stream))
    return child, kmap


def coarsen2_workspace_size(n: int) -> int:
    b = _u64(0)
    call("s3dx_coarsen2_workspace_size", _i64(n), C.byref(b))
    return int(b.value)


def coarsen2(coords: DeviceArray, n: int, stream=None, out=None, workspace: DeviceArray = None):
    """SlatTables downsample tables (sparse_ops.cpp:53-104).

    Returns (nc, coarse_coords [n,4], fine_to_coarse [n], children [8n], inv_count [n]);
    only the first nc (8*nc) rows of the coarse outputs are meaningful.  out =
    (coarse_coords, fine_to_coarse, children, inv_count) and workspace may be
    passed in to reuse them across calls."""
    ws = workspace if workspace is not None else DeviceArray(coarsen2_workspace_size(n), np.uint8)
    if out is not None:
        cc, f2c, ch, inv = out
    else:
        cc = DeviceArray((n, 4), np.int32)
        f2c = DeviceArray((n,), np.int32)
        ch = DeviceArray((8 * n,), np.int32)
        inv = DeviceArray((n,), np.float32)
    nc = _i64(0)
    call("s3dx_coarsen2", _dptr(coords), _i64(n), _dptr(cc), _dptr(f2c), _dptr(ch), _dptr(inv),
         C.byref(nc), _dptr(ws), _u64(ws.nbytes), _sptr(stream))
    return int(nc.value), cc, f2c, ch, inv


def occupancy_workspace_size(shape) -> int:
    b = _u64(0)
    call("s3dx_occupancy_workspace_size", *(_i32(int(v)) for v in shape), C.byref(b))
    return int(b.value)


def prune_surface_workspace_size(n: int) -> int:
    b = _u64(0)
    call("s3dx_prune_surface_workspace_size", _i64(n), C.byref(b))
    return int(b.value)


def downsample_coords_workspace_size(n: int) -> int:
    b = _u64(0)
    call("s3dx_downsample_coords_workspace_size", _i64(n), C.byref(b))
    return int(b.value)


def occupancy_coords(occupancy: DeviceArray, shape, stream=None, out: DeviceArray = None,
                     workspace: DeviceArray = None):
    """Cells with occupancy > 0 in x-major order as (0, x, y, z) rows
    (session.cpp:1437-1441).  Returns (count, coords [cells, 4]); the first
    count rows are meaningful.  out / workspace may be passed in to reuse them."""
    nx, ny, nz = (int(v) for v in shape)
    b = _u64(0)
    call("s3dx_occupancy_workspace_size", _i32(nx), _i32(ny), _i32(nz), C.byref(b))
    ws = workspace if workspace is not None else DeviceArray(int(b.value), np.uint8)
    out = out if out is not None else DeviceArray((nx * ny * nz, 4), np.int32)
    cnt = _i64(0)
    call("s3dx_occupancy_coords", _dptr(occupancy), _i32(nx), _i32(ny), _i32(nz), _dptr(out),
         C.byref(cnt), _dptr(ws), _u64(ws.nbytes), _sptr(stream))
    return int(cnt.value), out


def prune_surface(coords: DeviceArray, n: int, stream=None, out: DeviceArray = None,
                  workspace: DeviceArray = None):
    """prune_surface_coords (session.cpp:133-163).  Returns (count, surface [n, 4])."""
    b = _u64(0)
    call("s3dx_prune_surface_workspace_size", _i64(n), C.byref(b))
    ws = workspace if workspace is not None else DeviceArray(int(b.value), np.uint8)
    out = out if out is not None else DeviceArray((n, 4), np.int32)
    cnt = _i64(0)
    call("s3dx_prune_surface", _dptr(coords), _i64(n), _dptr(out), C.byref(cnt), _dptr(ws),
         _u64(ws.nbytes), _sptr(stream))
    return int(cnt.value), out


def downsample_coords(coords: DeviceArray, n: int, max_coords: int = 42000, factor: int = 2,
                      seed: int = 42, stream=None, out: DeviceArray = None, workspace: DeviceArray = None):
    """downsample_coords (session.cpp:168-233).  Returns (count, out [min(n, max_coords), 4])."""
    b = _u64(0)
    call("s3dx_downsample_coords_workspace_size", _i64(n), C.byref(b))
    ws = workspace if workspace is not None else DeviceArray(int(b.value), np.uint8)
    out = out if out is not None else DeviceArray((max(1, min(n, max_coords)), 4), np.int32)
    cnt = _i64(0)
    call("s3dx_downsample_coords", _dptr(coords), _i64(n), _i64(max_coords), _i32(factor), _u32(seed),
         _dptr(out), C.byref(cnt), _dptr(ws), _u64(ws.nbytes), _sptr(stream))
    return int(cnt.value), out


def coords_from_occupancy(occupancy: DeviceArray, shape, max_coords: int = 42000, seed: int = 42,
                          stream=None):
    """The SLat stage's coordinate table from the decoder's occupancy, as
    session.cpp:1437-1474 builds it: threshold, surface prune, then the
    downsample when more than max_coords rows remain.  Returns (count, coords)."""
    n, coords = occupancy_coords(occupancy, shape, stream)
    if n == 0:
        return 0, coords
    n, coords = prune_surface(coords, n, stream)
    if n > max_coords:
        n, coords = downsample_coords(coords, n, max_coords, 2, seed, stream)
    return n, coords


class SlatTables:
    """Device-resident SLat tables (SlatTables, sparse_ops.hpp:11-37, minus the APE)."""

    def build(self, coords_host: np.ndarray, stream=None) -> bool:
        c = np.ascontiguousarray(coords_host, dtype=np.int32)
        self.nf = int(c.shape[0])
        if self.nf <= 0:
            return False
        self.coords = DeviceArray.from_host(c, stream)
        self.conv_fine = kmap_subm3(self.coords, self.nf, self.nf, stream=stream)
        (self.nc, self.coarse_coords, self.fine_to_coarse, self.coarse_children,
         self.coarse_inv_count) = coarsen2(self.coords, self.nf, stream)
        self.conv_coarse = kmap_subm3(self.coarse_coords, self.nc, self.nc, stream=stream)
        return True


class MeshSubdivideTables:
    """Device-resident subdivide tables (MeshSubdivideTables, sparse_ops.hpp:71-78)."""

    def build(self, parent_coords, count: int = None, stream=None) -> bool:
        if isinstance(parent_coords, DeviceArray):
            parents = parent_coords
            count = parent_coords.shape[0] if count is None else count
        else:
            p = np.ascontiguousarray(parent_coords, dtype=np.int32)
            count = p.shape[0]
            if count <= 0:
                return False
            parents = DeviceArray.from_host(p, stream)
        try:
            self.child_coords, self.neighbors = subdivide2(parents, count, True, stream)
        except S3dxError as e:
            if e.status == INVALID_ARGUMENT:
                return False
            raise
        self.parent_count = count
        self.child_count = 8 * count
        return True


# ---------------------------------------------------------------------------
# Convolution layer
# ---------------------------------------------------------------------------
class SparseConv:
    """A prepared sparse conv layer (s3dx_conv): packed weights + fused epilogue."""

    def __init__(self, cin: int, cout: int, kvol: int = 27, dtype: int = F32):
        p = _vp()
        call("s3dx_conv_create", _i32(cin), _i32(cout), _i32(kvol), _i32(dtype), C.byref(p))
        self.handle = p.value
        self.cin, self.cout, self.kvol, self.dtype = cin, cout, kvol, dtype

    def set_weights(self, weight: np.ndarray, layout: int = WEIGHT_SLAT, bias: np.ndarray = None):
        w, wp = _host_f32(weight)
        b, bp = _host_f32(bias)
        call("s3dx_conv_set_weights", _vp(self.handle), wp, _i32(layout), bp)
        return self

    def set_gather_parent(self, enable: bool = True, slot_offset: np.ndarray = None):
        s, sp = _host_f32(slot_offset)
        call("s3dx_conv_set_gather_parent", _vp(self.handle), _i32(int(enable)), sp)
        return self

    def set_input_affine_silu(self, scale: DeviceArray = None, shift: DeviceArray = None):
        call("s3dx_conv_set_input_affine_silu", _vp(self.handle), _dptr(scale), _dptr(shift))
        self._affine_refs = (scale, shift)
        return self

    def set_layernorm(self, enable: bool = True, eps: float = 1e-6, weight=None, bias=None,
                      mod_scale=None, mod_shift=None):
        hs = [_host_f32(a) for a in (weight, bias, mod_scale, mod_shift)]
        call("s3dx_conv_set_layernorm", _vp(self.handle), _i32(int(enable)), _f32(eps),
             *[p for _, p in hs])
        return self

    def set_modulate(self, scale: DeviceArray = None, shift: DeviceArray = None):
        """Per-run modulate h*scale + h + shift from DEVICE [cout] float32 buffers
        (the res_block's emb_layers output); read at run time."""
        call("s3dx_conv_set_modulate", _vp(self.handle), _dptr(scale), _dptr(shift))
        self._modulate_refs = (scale, shift)
        return self

    def set_silu(self, enable: bool = True):
        call("s3dx_conv_set_silu", _vp(self.handle), _i32(int(enable)))
        return self

    def set_residual_parent(self, enable: bool = True):
        """Residual of one row per parent: output row i adds residual row i >> 3."""
        call("s3dx_conv_set_residual_parent", _vp(self.handle), _i32(int(enable)))
        return self

    def set_input_dtype(self, dtype: int):
        """x in `dtype`: the layer's own, or BF16 rows for an FP32 layer (widened exactly)."""
        call("s3dx_conv_set_input_dtype", _vp(self.handle), _i32(dtype))
        return self

    def plan(self, n_in: int, n_out: int, gather_plan: "GatherPlan" = None) -> str:
        """The kernel variant run() launches for these row counts (host only);
        with `gather_plan`, the one run(plan=gather_plan) launches."""
        buf = C.create_string_buffer(256)
        if gather_plan is None:
            call("s3dx_conv_plan", _vp(self.handle), _i64(n_in), _i64(n_out), buf, len(buf))
        else:
            call("s3dx_conv_plan_planned", _vp(self.handle), _vp(gather_plan.handle), _i64(n_in), _i64(n_out), buf,
                 len(buf))
        return buf.value.decode()

    def gather_plan(self, n_in: int, kmap, n_out: int, stream=None) -> "GatherPlan":
        """The map's gather plan for this layer's source rows (s3dx_gather_plan_create)."""
        return GatherPlan(self, n_in, kmap, n_out, stream)

    def run(self, x: DeviceArray, n_in: int, kmap, n_out: int, y: DeviceArray, y_dtype: int = None,
            residual: DeviceArray = None, stream=None, plan: "GatherPlan" = None):
        yd = self.dtype if y_dtype is None else y_dtype
        if plan is None:
            call("s3dx_conv_run", _vp(self.handle), _dptr(x), _i64(n_in), _dptr(kmap), _i64(n_out),
                 _dptr(residual), _dptr(y), _i32(yd), _sptr(stream))
        else:
            call("s3dx_conv_run_planned", _vp(self.handle), _vp(plan.handle), _dptr(x), _i64(n_in), _dptr(kmap),
                 _i64(n_out), _dptr(residual), _dptr(y), _i32(yd), _sptr(stream))
        return y

    def __del__(self):
        try:
            if self.handle:
                lib().s3dx_conv_free(_vp(self.handle))
        except Exception:
            pass


class GatherPlan:
    """A kernel map's per-tile gather plan (s3dx_gather_plan): built once per map,
    passed to every run over that map by layers that read their input alike."""

    def __init__(self, conv: SparseConv, n_in: int, kmap, n_out: int, stream=None):
        p = _vp()
        call("s3dx_gather_plan_create", _vp(conv.handle), _i64(n_in), _dptr(kmap), _i64(n_out), _sptr(stream),
             C.byref(p))
        self.handle = p.value
        self._kmap = kmap

    def rebuild(self, conv: SparseConv, n_in: int, kmap, n_out: int, stream=None) -> "GatherPlan":
        """Rebuilds the plan in place for another map of at most the created rows
        (s3dx_gather_plan_rebuild; no allocation)."""
        call("s3dx_gather_plan_rebuild", _vp(self.handle), _vp(conv.handle), _i64(n_in), _dptr(kmap), _i64(n_out),
             _sptr(stream))
        self._kmap = kmap
        return self

    def __del__(self):
        try:
            if self.handle:
                lib().s3dx_gather_plan_free(_vp(self.handle))
        except Exception:
            pass


# ---------------------------------------------------------------------------
# Row ops
# ---------------------------------------------------------------------------
def layernorm_rows(x, x_dtype, n, c, eps, w=None, b=None, mod_scale=None, mod_shift=None,
                   silu=False, y=None, y_dtype=None, stream=None):
    yd = x_dtype if y_dtype is None else y_dtype
    call("s3dx_layernorm_rows", _dptr(x), _i32(x_dtype), _i64(n), _i32(c), _f32(eps), _dptr(w),
         _dptr(b), _dptr(mod_scale), _dptr(mod_shift), _i32(int(silu)), _dptr(y if y is not None else x),
         _i32(yd), _sptr(stream))


def groupnorm_stats(x, x_dtype, n, c, groups, eps, gamma=None, beta=None, stream=None, out=None):
    """Per-channel GroupNorm scale/shift (s3dx_groupnorm_stats); `out` = a previous
    call's (scale, shift, workspace) to reuse (no allocation)."""
    if out is None:
        b = _u64(0)
        call("s3dx_groupnorm_workspace_size", _i64(n), _i32(c), _i32(groups), C.byref(b))
        ws = DeviceArray(int(b.value), np.uint8)
        scale = DeviceArray((c,), np.float32)
        shift = DeviceArray((c,), np.float32)
    else:
        scale, shift, ws = out
    call("s3dx_groupnorm_stats", _dptr(x), _i32(x_dtype), _i64(n), _i32(c), _i32(groups), _f32(eps),
         _dptr(gamma), _dptr(beta), _dptr(scale), _dptr(shift), _dptr(ws), _u64(ws.nbytes), _sptr(stream))
    return scale, shift, ws


def affine_rows(x, x_dtype, n, c, scale, shift, silu, y, y_dtype, stream=None):
    call("s3dx_affine_rows", _dptr(x), _i32(x_dtype), _i64(n), _i32(c), _dptr(scale), _dptr(shift),
         _i32(int(silu)), _dptr(y), _i32(y_dtype), _sptr(stream))


def downsample_mean(x, dtype, nf, c, children, inv_count, nc, y, stream=None):
    call("s3dx_downsample_mean", _dptr(x), _i32(dtype), _i64(nf), _i32(c), _dptr(children),
         _dptr(inv_count), _i64(nc), _dptr(y), _sptr(stream))


def upsample_nearest(coarse, dtype, nc, c, f2c, nf, y, stream=None):
    call("s3dx_upsample_nearest", _dptr(coarse), _i32(dtype), _i64(nc), _i32(c), _dptr(f2c), _i64(nf),
         _dptr(y), _sptr(stream))


def concat_rows(a, ca, b, cb, dtype, n_src, rows, n, y, stream=None):
    """y[i] = [a[r], b[r]], r = rows[i] or i (ggml_concat, slat_flow_graph.cpp:443, 477)."""
    call("s3dx_concat_rows", _dptr(a), _i32(ca), _dptr(b), _i32(cb), _i32(dtype), _i64(n_src), _dptr(rows),
         _i64(n), _dptr(y), _sptr(stream))


def convert(x, x_dtype, count, y, y_dtype, stream=None):
    call("s3dx_convert", _dptr(x), _i32(x_dtype), _i64(count), _dptr(y), _i32(y_dtype), _sptr(stream))


def synchronize(stream=None):
    call("s3dx_stream_synchronize", _sptr(stream))
