"""SAMT and GGUF readers (host side) and the converters' conv-weight layouts.

SAMT is pinned by the reference's own fixture (ss_occ_f32.samt: 69,537 cells
above zero, the same bits as the committed golden set).  The GGUF reader is
checked by round trips through a writer built here from the published GGUF
layout: parity unpinned beyond that (no GGUF file ships with the reference)."""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np
import pytest

from helpers import gguf_bytes

FIXTURE = Path("/root/reference/tests/objects_runtime/fixtures/ss_occ_f32.samt")


@pytest.fixture(scope="module")
def F(s3dx):
    return s3dx.formats


@pytest.mark.skipif(not FIXTURE.exists(), reason="reference tree absent")
def test_samt_reference_fixture(F, golden):
    arrays, _ = golden
    occ = F.read_samt(FIXTURE)
    assert occ.shape == (64, 64, 64) and occ.dtype == np.float32
    assert int((occ > 0).sum()) == 69537
    assert np.array_equal(np.packbits((occ > 0).reshape(-1)), arrays["ss_occ.bits"])


@pytest.mark.parametrize("dtype,shape", [(np.float32, (7,)), (np.float16, (3, 5)), (np.int32, (4, 4)),
                                         (np.float32, (2, 3, 4, 5))])
def test_samt_round_trip(F, tmp_path, dtype, shape):
    a = (np.arange(np.prod(shape)) * 3 - 11).astype(dtype).reshape(shape)
    F.write_samt(tmp_path / "t.samt", a)
    raw = (tmp_path / "t.samt").read_bytes()
    assert raw[:4] == b"SAMT" and struct.unpack_from("<i", raw, 4)[0] == len(shape)
    assert struct.unpack_from(f"<{len(shape)}q", raw, 8) == tuple(reversed(shape))  # ne[0] fastest
    b = F.read_samt(tmp_path / "t.samt")
    assert b.dtype == a.dtype and np.array_equal(a, b)


def test_samt_int32_type_30_and_malformed(F, tmp_path):
    coords = np.array([[0, 1, 2, 3], [0, 4, 5, 6]], np.int32)
    head = struct.pack("<Ii", 0x544D4153, 2) + struct.pack("<2q", 4, 2) + struct.pack("<i", 30)
    (tmp_path / "c.samt").write_bytes(head + coords.tobytes())
    assert np.array_equal(F.read_samt(tmp_path / "c.samt"), coords)
    (tmp_path / "bad.samt").write_bytes(b"SAMX" + head[4:] + coords.tobytes())
    with pytest.raises(ValueError):
        F.read_samt(tmp_path / "bad.samt")
    (tmp_path / "short.samt").write_bytes(head + coords.tobytes()[:-4])
    with pytest.raises(ValueError):
        F.read_samt(tmp_path / "short.samt")


def test_gguf_round_trip(F, tmp_path):
    rng = np.random.default_rng(3)
    w = rng.normal(size=(40, 27 * 16)).astype(np.float32)
    h = rng.normal(size=(27, 8 * 4)).astype(np.float16)
    bf = rng.normal(size=(5, 6)).astype(np.float32)
    bf_bits = (bf.view(np.uint32) >> 16).astype(np.uint16)
    ids = np.arange(12, dtype=np.int32).reshape(3, 4)
    kv = {"general.architecture": (8, "sam3d"), "meshdec.resolution": (4, 256),
          "meshdec.mlp_ratio": (6, 4.0), "general.alignment": (4, 32), "list": (9, [1, 2, 3])}
    path = tmp_path / "m.gguf"
    path.write_bytes(gguf_bytes(kv, {"slat.conv.weight": (0, w), "meshdec.conv.weight": (1, h),
                                      "b": (30, bf_bits), "ids": (26, ids)}))
    g = F.GgufFile(path)
    assert g.version == 3 and g.kv["general.architecture"] == "sam3d" and g.kv["list"] == [1, 2, 3]
    assert g.kv["meshdec.resolution"] == 256 and g.kv["meshdec.mlp_ratio"] == 4.0
    assert np.array_equal(g.tensor("slat.conv.weight"), w)
    assert np.array_equal(g.tensor("meshdec.conv.weight"), h)
    assert np.array_equal(g.tensor("b"), (bf_bits.astype(np.uint32) << 16).view(np.float32))
    assert np.array_equal(g.tensor("ids"), ids)


def test_conv_weight_layouts(F):
    # spconv (Cout, KD, KH, KW, Cin): SLat keeps the C-order flatten
    # (gguf_schema.py:326-334); mesh 3x3x3 permutes to (KD, KH, KW, Cout, Cin)
    # (convert_sam3d_to_gguf.py:486-492); mesh 1x1 reads the buffer as (IC, OC).
    rng = np.random.default_rng(4)
    cout, cin = 6, 5
    w5 = rng.normal(size=(cout, 3, 3, 3, cin)).astype(np.float32)
    slat = F.conv_weight(w5.reshape(cout, 27 * cin), "slat", cin, cout)
    assert slat.shape == (cout, 27, cin) and slat[2, 13, 4] == w5[2, 1, 1, 1, 4]
    mesh = F.conv_weight(np.transpose(w5, (1, 2, 3, 0, 4)).reshape(27, cout * cin), "mesh", cin, cout)
    assert mesh.shape == (27, cout, cin) and mesh[5, 3, 1] == w5[3, 0, 1, 2, 1]
    w1 = rng.normal(size=(cout, 1, 1, 1, cin)).astype(np.float32)
    m1 = w1.reshape(cin, cout).T.copy().reshape(1, cout * cin)
    one = F.conv_weight(m1, "mesh_1x1", cin, cout)
    assert one.shape == (1, cout, cin) and one[0, 4, 2] == w1.reshape(-1)[2 * cout + 4]
    with pytest.raises(ValueError):
        F.conv_weight(m1, "mesh", cin, cout)
