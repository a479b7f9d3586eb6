"""Weights replayed from on-disk GGUF layouts through the HIP conv.

A GGUF file is written with the converters' three sparse-conv layouts (F16,
as the converter stores them), read back by formats.GgufFile, turned into
set_weights layouts by formats.conv_weight, and run on the GPU.  The
expectation is computed from the original spconv tensors (Cout, KD, KH, KW,
Cin) by their own semantics, not through the converters' layouts:
  - SLat conv (convert_sam3d_to_gguf.py:295-301, gguf_schema.py:326-334) and
    mesh 3x3x3 conv (convert_sam3d_to_gguf.py:486-492): offset o = kd*9 +
    kh*3 + kw takes w[:, kd, kh, kw, :] as a (Cout, Cin) matrix;
  - mesh 1x1 skip (convert_sam3d_to_gguf.py:481-492): the pinned spconv's 1x1
    path reads the same buffer as an (IC, OC) matrix M, y = x @ M.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import check_rel, gguf_bytes

pytestmark = pytest.mark.gpu

GGML_F16 = 1


def _f16(a):
    return a.astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("kind,cin,cout", [("slat", 64, 96), ("mesh", 96, 64), ("mesh_1x1", 192, 96)])
def test_gguf_weights_through_hip_conv(s3dx, O, W, tmp_path, kind, cin, cout):
    F = s3dx.formats
    rng = np.random.default_rng(80)
    k = 1 if kind == "mesh_1x1" else 3
    w5 = _f16(rng.normal(0.0, 1.0 / np.sqrt(k ** 3 * cin), size=(cout, k, k, k, cin)))
    if kind == "slat":
        stored = w5.reshape(cout, 27 * cin)
    elif kind == "mesh":
        stored = np.transpose(w5, (1, 2, 3, 0, 4)).reshape(27, cout * cin)
    else:
        stored = w5.reshape(cin, cout).T.reshape(1, cout * cin)
    path = tmp_path / "w.gguf"
    path.write_bytes(gguf_bytes({"general.architecture": (8, "sam3d")},
                                {"blk.conv.weight": (GGML_F16, stored.astype(np.float16))}))
    wt = F.conv_weight(F.GgufFile(path).tensor("blk.conv.weight"), kind, cin, cout)
    layout = s3dx.WEIGHT_SLAT if kind == "slat" else s3dx.WEIGHT_MESH
    conv = s3dx.SparseConv(cin, cout, k ** 3, s3dx.F32).set_weights(wt, layout, None)

    coords = W.shells_union(5)[:1500]
    n = coords.shape[0]
    x = W.normal_f32(81, 1, (n, cin))
    y = s3dx.DeviceArray((n, cout), np.float32)
    if k == 3:
        kmap = O.kmap_subm3(coords, n)
        conv.run(s3dx.DeviceArray.from_host(x), n, s3dx.DeviceArray.from_host(kmap), n, y, s3dx.F32)
        ref = O.conv(x, kmap, n, w5.reshape(cout, 27, cin), 0, cout, None)
    else:
        conv.run(s3dx.DeviceArray.from_host(x), n, None, n, y, s3dx.F32)
        ref = x.astype(np.float64) @ w5.reshape(cin, cout).astype(np.float64)
    print(f"gguf {kind} {cin}->{cout}: {conv.plan(n, n)}", flush=True)
    check_rel(y.download(), ref, 1e-5, kind)
