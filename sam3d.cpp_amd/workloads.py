"""Seeded synthetic voxel sets and tensors for the sparse-voxel benchmark configs.

Portable on purpose: the random stream is splitmix64 (integer arithmetic only)
and occupancy tests use IEEE +,-,*,sqrt, so the same seed yields the same
coordinates on every machine and numpy version.  Normal variates use
Box-Muller on that stream.

Configs (sizes as in the benchmark definition):
  shell_64       one shell |d-20| <= 1 around (32,32,32) on 64^3 (10,366 voxels)
  shells_union   8 shells, centres U[12,52]^3, radii U[6,14], |d-r| <= 1.5,
                 on 64^3 (~25-35k voxels)
  or_pool2       2x OR-pool of a voxel set (unique (b, x//2, y//2, z//2))
Coordinates are int32 [n, 4] = (b, x, y, z) in lexicographic order, as the
SS-decoder occupancy produces them (session.cpp:1437-1441).
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


class SplitMix64:
    """splitmix64 stream; `tag` separates independent streams of one seed."""

    def __init__(self, seed: int, tag: int = 0):
        with np.errstate(over="ignore"):
            s = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) * _GOLDEN + np.uint64(tag & 0xFFFFFFFF)
            self.state = _mix(np.array([s], dtype=np.uint64))[0]

    def next_u64(self, count: int) -> np.ndarray:
        with np.errstate(over="ignore"):
            k = np.arange(1, count + 1, dtype=np.uint64)
            z = self.state + k * _GOLDEN
            self.state = self.state + np.uint64(count) * _GOLDEN
            return _mix(z)

    def uniform(self, count: int) -> np.ndarray:
        """Doubles in [0, 1) with 53 random bits."""
        return (self.next_u64(count) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)

    def normal(self, count: int) -> np.ndarray:
        u = self.next_u64(2 * count)
        u1 = ((u[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
        u2 = (u[1::2] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
        return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def _grid(res: int):
    ax = np.arange(res, dtype=np.float64)
    return np.meshgrid(ax, ax, ax, indexing="ij")


def _coords_from_mask(mask: np.ndarray, batch: int = 0) -> np.ndarray:
    xyz = np.argwhere(mask).astype(np.int32)  # C order: x slowest, z fastest
    b = np.full((xyz.shape[0], 1), batch, dtype=np.int32)
    return np.ascontiguousarray(np.concatenate([b, xyz], axis=1))


def shell_64(res: int = 64, centre=(32.0, 32.0, 32.0), radius: float = 20.0,
             half_thickness: float = 1.0) -> np.ndarray:
    """Integer shell |dist - radius| <= half_thickness (10,366 voxels by default)."""
    x, y, z = _grid(res)
    d = np.sqrt((x - centre[0]) ** 2 + (y - centre[1]) ** 2 + (z - centre[2]) ** 2)
    return _coords_from_mask(np.abs(d - radius) <= half_thickness)


def shells_union(seed: int = 0, res: int = 64, count: int = 8, half_thickness: float = 1.5):
    """Union of `count` shells with centres U[12,52]^3 and radii U[6,14]."""
    rng = SplitMix64(seed, tag=1)
    u = rng.uniform(count * 4).reshape(count, 4)
    centres = 12.0 + 40.0 * u[:, :3]
    radii = 6.0 + 8.0 * u[:, 3]
    x, y, z = _grid(res)
    mask = np.zeros((res, res, res), dtype=bool)
    for c, r in zip(centres, radii):
        d = np.sqrt((x - c[0]) ** 2 + (y - c[1]) ** 2 + (z - c[2]) ** 2)
        mask |= np.abs(d - r) <= half_thickness
    return _coords_from_mask(mask)


def occupancy_noise(seed: int = 0, res: int = 64, density: float = 0.265) -> np.ndarray:
    """A float32 [res]^3 occupancy field (x-major) with about `density` of the
    cells > 0, scattered like a noisy decoder output: N(0,1) shifted by the
    normal quantile of 1 - density (0.628 for the default)."""
    from statistics import NormalDist
    shift = NormalDist().inv_cdf(1.0 - density)
    return (normal_f32(seed, 7, (res, res, res)) - np.float32(shift)).astype(np.float32)


def or_pool2(coords: np.ndarray) -> np.ndarray:
    """Unique (b, x//2, y//2, z//2), lexicographically sorted (non-negative coords)."""
    c = coords.copy()
    c[:, 1:] //= 2
    return np.ascontiguousarray(np.unique(c, axis=0).astype(np.int32))


def normal_f32(seed: int, tag: int, shape, std: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    v = SplitMix64(seed, tag).normal(n).astype(np.float32) * np.float32(std)
    return v.reshape(shape)


def conv_weight(seed: int, tag: int, cin: int, cout: int, kvol: int = 27,
                layout: str = "slat") -> np.ndarray:
    """N(0, 1/sqrt(kvol*cin)) weights; slat layout [cout][kvol][cin], mesh [kvol][cout][cin]."""
    std = 1.0 / np.sqrt(kvol * cin)
    shape = (cout, kvol, cin) if layout == "slat" else (kvol, cout, cin)
    return normal_f32(seed, tag, shape, std)


# ---------------------------------------------------------------------------
# bfloat16 helpers (numpy has no bf16: values travel as uint16 bit patterns)
# ---------------------------------------------------------------------------
def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x007FFFFF) != 0)
    r = u + 0x7FFF + ((u >> 16) & 1)
    r = np.where(nan, u | 0x00400000, r)
    return ((r >> 16) & 0xFFFF).astype(np.uint16)


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(x)).reshape(np.shape(x))


def kmap_pairs(kmap: np.ndarray, n_in: int) -> int:
    """Present (voxel, offset) pairs P of a kernel map."""
    return int(np.count_nonzero((kmap >= 0) & (kmap < n_in)))
