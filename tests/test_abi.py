"""The C ABI library loads, exports every declared symbol, and rejects bad
arguments on the host (no device needed)."""
import ctypes as C
import re
from pathlib import Path

import pytest

HEADER = Path(__file__).resolve().parents[1] / "include" / "s3dx_sparse.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"S3DX_API\s+[\w\s\*]+?\b(s3dx_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported(s3dx):
    names = declared()
    assert len(names) >= 30
    lib = s3dx.lib()
    for name in names:
        assert hasattr(lib, name), name
        assert name in s3dx.SIGNATURES, f"{name} missing from the Python binding"
    assert set(s3dx.SIGNATURES) == set(names)


def test_abi_version(s3dx):
    assert s3dx.lib().s3dx_abi_version() == 1


def _status(s3dx, name, *args, cap=256):
    buf = C.create_string_buffer(cap)
    st = getattr(s3dx.lib(), name)(*args, buf, cap)
    return st, buf.value.decode()


def test_error_buffer_contract(s3dx):
    lib = s3dx.lib()
    b = C.c_uint64(0)
    # NULL buffer with nonzero capacity is itself invalid
    assert lib.s3dx_kmap_workspace_size(100, C.byref(b), None, 16) == s3dx.INVALID_ARGUMENT
    # NULL,0 discards diagnostics
    assert lib.s3dx_kmap_workspace_size(100, C.byref(b), None, 0) == s3dx.OK
    # success clears the buffer; failure NUL-terminates a truncated message
    buf = C.create_string_buffer(b"stale text", 32)
    assert lib.s3dx_kmap_workspace_size(100, C.byref(b), buf, 32) == s3dx.OK and buf.value == b""
    small = C.create_string_buffer(8)
    assert lib.s3dx_kmap_workspace_size(0, C.byref(b), small, 8) == s3dx.INVALID_ARGUMENT
    assert len(small.value) == 7


def test_workspace_sizes_grow(s3dx):
    a = s3dx.kmap_workspace_size(1000)
    b = s3dx.kmap_workspace_size(100000)
    assert 0 < a < b
    assert b >= 2 * 100000 * 8  # hash slots at load <= 1/2


@pytest.mark.parametrize("call", [
    ("s3dx_kmap_workspace_size", 0),
    ("s3dx_kmap_workspace_size", 2**31 // 27 + 1),
    ("s3dx_subdivide2_workspace_size", 0),
    ("s3dx_subdivide2_workspace_size", 2**31 // 27 + 1),
    ("s3dx_coarsen2_workspace_size", -5),
])
def test_size_queries_reject_bad_counts(s3dx, call):
    b = C.c_uint64(0)
    st, msg = _status(s3dx, call[0], C.c_int64(call[1]), C.byref(b))
    assert st == s3dx.INVALID_ARGUMENT and msg


def test_kmap_rejects_bad_pointers(s3dx):
    st, msg = _status(s3dx, "s3dx_kmap_subm3", None, 10, 10, None, None, 0, None)
    assert st == s3dx.INVALID_ARGUMENT and "coords" in msg
    st, msg = _status(s3dx, "s3dx_kmap_subm3", C.c_void_p(0x1004), 10, 10, C.c_void_p(0x2000),
                      C.c_void_p(0x3000), 1 << 20, None)
    assert st == s3dx.INVALID_ARGUMENT and "aligned" in msg
    st, msg = _status(s3dx, "s3dx_kmap_subm3", C.c_void_p(0x1000), 10, 10, C.c_void_p(0x2000),
                      C.c_void_p(0x3000), 64, None)
    assert st == s3dx.INVALID_ARGUMENT and "workspace" in msg


def test_subdivide_rejects_reference_limits(s3dx):
    # sparse_ops.cpp:273: count <= 0 and count > INT32_MAX / 8 are rejected
    for p in (0, -1, 2**31 // 8 + 1):
        st, msg = _status(s3dx, "s3dx_subdivide2", C.c_void_p(0x1000), C.c_int64(p), C.c_void_p(0x2000),
                          None, C.c_void_p(0x3000), 1 << 20, None)
        assert st == s3dx.INVALID_ARGUMENT, (p, msg)


def test_conv_create_validation(s3dx):
    p = C.c_void_p()
    for args in [(0, 8, 27, 0), (8, 8, 5, 0), (8, 8, 27, 7), (8, -1, 1, 1)]:
        st, msg = _status(s3dx, "s3dx_conv_create", *args, C.byref(p))
        assert st == s3dx.INVALID_ARGUMENT and msg, args
    st, _ = _status(s3dx, "s3dx_conv_create", 128, 128, 27, 1, C.byref(p))
    assert st == s3dx.OK and p.value
    st, msg = _status(s3dx, "s3dx_conv_run", p, C.c_void_p(0x1000), 10, C.c_void_p(0x2000), 10,
                      None, C.c_void_p(0x3000), 1, None)
    assert st == s3dx.INVALID_ARGUMENT and "weights" in msg
    s3dx.lib().s3dx_conv_free(p)


def test_conv_plan_names_the_launched_kernel(s3dx, monkeypatch):
    # Host-only query: which kernel variant s3dx_conv_run would launch.
    monkeypatch.delenv("S3DX_CONV_TILING", raising=False)
    monkeypatch.delenv("S3DX_CONV_HALO", raising=False)
    n = 28265  # 64^3 eight-shell union, seed 0
    c128 = s3dx.SparseConv(128, 128, 27, s3dx.BF16)
    # BF16 3x3x3 with 64-channel chunks and 128 columns: the halo-staged
    # kernel on 64-row tiles (442 > 256 CUs), 128-row tiles on request.
    assert c128.plan(n, n) == "mfma tiling=21 split-k halo rows=64 cols=128 kc=64 xf=0 ln=none grid=442x1"
    monkeypatch.setenv("S3DX_CONV_HALO", "128")
    assert c128.plan(n, n) == "mfma tiling=20 split-k halo rows=128 cols=128 kc=64 xf=0 ln=none grid=221x1"
    # Without it: one pass of 128-row tiles on 256 CUs: 64-row tiles, two per CU, 64-channel tasks
    monkeypatch.setenv("S3DX_CONV_HALO", "0")
    assert c128.plan(n, n) == "mfma tiling=18 split-k rows=64 cols=128 kc=64 xf=0 ln=none grid=442x1"
    monkeypatch.delenv("S3DX_CONV_HALO")
    c128.set_layernorm(True, 1e-6)
    assert "ln=fused" in c128.plan(n, n)
    # A fused LayerNorm over 256 columns is not the halo kernel's epilogue.
    assert "halo" not in s3dx.SparseConv(128, 256, 27, s3dx.BF16).set_layernorm(True, 1e-6).plan(n, n)
    assert "halo" in s3dx.SparseConv(1024, 1024, 27, s3dx.BF16).plan(5086, 5086)
    assert "halo" not in s3dx.SparseConv(128, 128, 27, s3dx.F32).plan(n, n)
    f64 = s3dx.SparseConv(64, 64, 27, s3dx.F32)
    assert f64.plan(n, n).startswith("mfma tiling=12 split-k rows=128 cols=64 kc=64")
    # The 10,366-voxel sphere shell: 81 x 2 tiles of 128 x 32 would leave CUs
    # idle; FP32 32-column tiles then take 32 rows each.
    assert f64.plan(10366, 10366) == "mfma tiling=24 split-k rows=32 cols=32 kc=64 xf=0 ln=none grid=324x2"
    # 96 bf16 channels: four 32-channel chunks make each 128-channel task;
    # forced, the 64-row halo kernel with a half-width last chunk.
    assert s3dx.SparseConv(96, 96, 27, s3dx.BF16).plan(n, n).startswith("mfma tiling=15 split-k rows=128 cols=96 kc=32")
    monkeypatch.setenv("S3DX_CONV_TILING", "21")
    assert s3dx.SparseConv(96, 96, 27, s3dx.BF16).plan(n, n) == \
        "mfma tiling=21 split-k halo rows=64 cols=96 kc=64+32 xf=0 ln=none grid=442x1"
    monkeypatch.delenv("S3DX_CONV_TILING")
    # 192 output columns without LayerNorm: two 96-column tiles of the
    # 64-row halo kernel (the split-K kernels with S3DX_CONV_HALO=0: 64-row
    # tiles, two per CU, as there are more 128-row tiles than CUs).
    assert s3dx.SparseConv(192, 192, 27, s3dx.BF16).plan(n, n) == \
        "mfma tiling=21 split-k halo rows=64 cols=96 kc=64 xf=0 ln=none grid=442x2"
    monkeypatch.setenv("S3DX_CONV_HALO", "0")
    assert s3dx.SparseConv(192, 192, 27, s3dx.BF16).plan(n, n) == \
        "mfma tiling=19 split-k rows=64 cols=96 kc=64 xf=0 ln=none grid=442x2"
    monkeypatch.delenv("S3DX_CONV_HALO")
    assert "cols=192" in s3dx.SparseConv(192, 192, 27, s3dx.BF16).set_layernorm(True, 1e-6).plan(n, n)
    # Cout not a multiple of 32: the generic kernel.
    assert s3dx.SparseConv(16, 40, 27, s3dx.F32).plan(100, 100) == "generic rows=64 cols=64 ln=none grid=2x1"
    # The parent repeat alone is a shift of the staged rows, no pre-pass.
    skip = s3dx.SparseConv(192, 192, 1, s3dx.BF16).set_gather_parent(True)
    assert skip.plan(n, 8 * n).startswith("parent-rows mfma tiling=")
    # BF16 rows into FP32 layers: the head reads them in its kernel; a
    # 27-offset layer widens them first.  Other combinations are refused.
    head = s3dx.SparseConv(96, 101, 1, s3dx.F32).set_input_dtype(s3dx.BF16)
    assert head.plan(8 * n, 8 * n).startswith("in=bf16 linear cols=128 ksteps=6 terms=3")
    assert s3dx.SparseConv(64, 64, 27, s3dx.F32).set_input_dtype(s3dx.BF16).plan(n, n).startswith("in=bf16 pre=widen mfma")
    with pytest.raises(s3dx.S3dxError, match="input dtype"):
        s3dx.SparseConv(64, 64, 27, s3dx.BF16).set_input_dtype(s3dx.F32)
    monkeypatch.setenv("S3DX_CONV_TILING", "10")
    assert c128.plan(n, n).startswith("mfma tiling=10 rows=128 cols=128")
    with pytest.raises(s3dx.S3dxError):
        c128.plan(0, n)


def test_missing_library_fails_loudly(s3dx, monkeypatch, tmp_path):
    monkeypatch.setattr(s3dx, "_lib", None)
    monkeypatch.setattr(s3dx, "LIB_PATH", tmp_path / "absent.so")
    with pytest.raises(RuntimeError, match="not built"):
        s3dx.lib()


def test_conv_modulate_needs_layernorm(s3dx):
    # Device modulate pointers are only recorded here (never read without a
    # run), so fake addresses suffice on a host without a GPU.
    conv = s3dx.SparseConv(64, 128, 27, s3dx.BF16)
    with pytest.raises(s3dx.S3dxError, match="LayerNorm"):
        conv.set_modulate(0x1000, 0x2000)
    with pytest.raises(s3dx.S3dxError, match="both"):
        conv.set_layernorm(True, 1e-6).set_modulate(0x1000, None)
    conv.set_modulate(0x1000, 0x2000)
    conv.set_modulate(None, None)


def test_linear_layer_rejects_rows_past_the_input(s3dx):
    # kvol 1 without a map: output row i reads input row i (row i >> 3 when
    # gathering parents), so n_out may not exceed the input rows.
    conv = s3dx.SparseConv(64, 64, 1, s3dx.BF16)
    assert "linear" in conv.plan(100, 100)
    with pytest.raises(s3dx.S3dxError, match="n_out exceeds"):
        conv.plan(100, 101)
    conv.set_gather_parent(True)
    conv.plan(100, 800)
    with pytest.raises(s3dx.S3dxError, match="n_out exceeds"):
        conv.plan(100, 801)


def test_static_kmap_rejects_sets_above_its_table(s3dx):
    # Checked before any device work: the static table holds 262144 voxels.
    st, msg = _status(s3dx, "s3dx_kmap_subm3_static", C.c_void_p(0x1000), C.c_int64(262145), C.c_int32(-1),
                      C.c_void_p(0x2000), C.c_void_p(None))
    assert st == s3dx.INVALID_ARGUMENT and "262144" in msg
