"""Occupancy -> coordinates on the GPU through the C ABI, byte-identical to
the oracle (session.cpp:1437-1441 threshold, :133-163 prune_surface_coords,
:168-233 downsample_coords), on the reference's own occupancy fixture
(ss_occ_f32.samt, 64^3) and on synthetic grids and sets."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import prune_brute_force, prune_cases

pytestmark = pytest.mark.gpu


def _occ_fixture(golden):
    arrays, _ = golden
    return np.unpackbits(arrays["ss_occ.bits"]).reshape(64, 64, 64).astype(np.float32)


def _rows(dev, count):
    return dev.download()[:count]


def test_occupancy_threshold_fixture(s3dx, O, golden):
    occ = _occ_fixture(golden)
    n, coords = s3dx.occupancy_coords(s3dx.DeviceArray.from_host(occ), occ.shape)
    print(f"occupancy fixture n={n}", flush=True)
    assert n == 69537
    assert np.array_equal(_rows(coords, n), O.occupancy_coords(occ))


@pytest.mark.parametrize("shape", [(17, 17, 17), (5, 33, 8), (64, 64, 64)])
def test_occupancy_threshold_signed_values(s3dx, shape):
    # Logits of both signs, exact zeros and negative zeros: only > 0 is kept,
    # in x-major order (numpy's argwhere order).
    rng = np.random.default_rng(sum(shape))
    occ = rng.normal(size=shape).astype(np.float32)
    occ[rng.random(shape) < 0.1] = 0.0
    occ[rng.random(shape) < 0.05] = -0.0
    n, coords = s3dx.occupancy_coords(s3dx.DeviceArray.from_host(occ), shape)
    print(f"occupancy shape={shape} n={n}", flush=True)
    want = np.argwhere(occ > 0).astype(np.int32)
    want = np.concatenate([np.zeros((want.shape[0], 1), np.int32), want], 1)
    assert np.array_equal(_rows(coords, n), want)


def test_prune_surface_fixture(s3dx, O, golden):
    coords = O.occupancy_coords(_occ_fixture(golden))
    n, surf = s3dx.prune_surface(s3dx.DeviceArray.from_host(coords), coords.shape[0])
    print(f"prune fixture n={n}", flush=True)
    assert n == 67783
    assert np.array_equal(_rows(surf, n), O.prune_surface(coords))


@pytest.mark.parametrize("seed", [1, 2])
def test_prune_surface_random_sets(s3dx, O, seed):
    # Dense-ish random blobs over two batches, negative coordinates, and
    # duplicated rows (each copy is judged on its own, as the reference does).
    rng = np.random.default_rng(seed)
    c = rng.integers(-6, 10, size=(6000, 4)).astype(np.int32)
    c[:, 0] = rng.integers(0, 2, size=c.shape[0])
    c = np.unique(c, axis=0)
    c = np.concatenate([c, c[::97]], 0)
    c = c[rng.permutation(c.shape[0])]
    n, surf = s3dx.prune_surface(s3dx.DeviceArray.from_host(c), c.shape[0])
    print(f"prune random seed={seed} n={c.shape[0]} -> {n}", flush=True)
    want = O.prune_surface(c)
    assert 0 < want.shape[0] < c.shape[0]
    assert np.array_equal(_rows(surf, n), want)


def test_downsample_fixture_surface(s3dx, O, golden):
    # 67,783 surface voxels > 42,000: the reference's map + first-occurrence
    # dedupe (+ sample if still too many).
    surface = O.prune_surface(O.occupancy_coords(_occ_fixture(golden)))
    n, out = s3dx.downsample_coords(s3dx.DeviceArray.from_host(surface), surface.shape[0])
    want = O.downsample_coords(surface)
    print(f"downsample fixture {surface.shape[0]} -> {n} (oracle {want.shape[0]})", flush=True)
    assert np.array_equal(_rows(out, n), want)


@pytest.mark.parametrize("max_coords,seed", [(1000, 42), (1000, 7), (5000, 42), (10 ** 6, 42)])
def test_downsample_sample_and_passthrough(s3dx, O, max_coords, seed):
    # The sample (unique cells > max_coords) must be the reference's
    # std::shuffle draw; n <= max_coords returns the input, duplicates kept.
    rng = np.random.default_rng(11)
    c = rng.integers(0, 60, size=(30000, 4)).astype(np.int32)
    c[:, 0] = 0
    n, out = s3dx.downsample_coords(s3dx.DeviceArray.from_host(c), c.shape[0], max_coords, 2, seed)
    want = O.downsample_coords(c, max_coords, 2, seed)
    print(f"downsample max={max_coords} seed={seed}: {n} rows", flush=True)
    assert np.array_equal(_rows(out, n), want)


def test_downsample_dense_cube(s3dx, O):
    g = np.arange(64, dtype=np.int32)
    x, y, z = np.meshgrid(g, g, g, indexing="ij")
    cube = np.stack([np.zeros_like(x), x, y, z], -1).reshape(-1, 4)
    n, out = s3dx.downsample_coords(s3dx.DeviceArray.from_host(cube), cube.shape[0])
    assert n == 32 ** 3
    assert np.array_equal(_rows(out, n), O.downsample_coords(cube))


def test_coords_from_occupancy_pipeline(s3dx, O, golden):
    # session.cpp:1437-1474: threshold, prune, downsample above 42,000 rows.
    occ = _occ_fixture(golden)
    n, coords = s3dx.coords_from_occupancy(s3dx.DeviceArray.from_host(occ), occ.shape)
    want = O.downsample_coords(O.prune_surface(O.occupancy_coords(occ)))
    print(f"pipeline rows={n}", flush=True)
    assert np.array_equal(_rows(coords, n), want)


@pytest.mark.parametrize("case", ["blobs_two_batches_duplicates", "solid_cube", "negative_cube", "key_aliasing"])
def test_prune_surface_brute_force_cases(s3dx, case):
    # The GPU prune against the independent brute force (coordinate_key
    # aliasing, negative coordinates, batches and duplicated rows).
    c = prune_cases()[case]
    n, surf = s3dx.prune_surface(s3dx.DeviceArray.from_host(c), c.shape[0])
    print(f"prune {case} n={c.shape[0]} -> {n}", flush=True)
    assert np.array_equal(_rows(surf, n), prune_brute_force(c))
