"""Shared test helpers: named voxel sets rebuilt from the workload generators
and the golden fixtures."""
import hashlib

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
