#!/usr/bin/env python3
"""Sparse-voxel conv benchmark: effective TFLOP/s + kernel-map Mvox/s.

Workload (one step): on a seeded 64^3 union of 8 sphere shells (~28k voxels,
int32 coords resident in HBM), build the 27-offset kernel map and, from the
same lookups, its gather plan (per 128-row tile: the distinct source rows) on
the GPU, then run one SparseResBlock at C=128:
    conv3x3x3 -> LayerNorm -> SiLU -> conv3x3x3 -> + x
in BF16 with FP32 accumulation (LayerNorm/SiLU fused into the first conv's
epilogue, the residual into the second's).  The same block in FP32 is
reported beside it.

value        = effective conv TFLOP/s = 2 * (2*Cin*Cout*P) / (conv1 + conv2
               kernel time), P = present (voxel, offset) pairs of the map,
               kernel times from HIP events around each launch on its stream
kmap_mvox_s  = voxels / (device time of the kernel-map build alone)
kmap_plan_ms = device time of the step's one-pass map + plan build
gather_plan_ms = device time of a plan rebuild alone (reported beside the
               conv time, and in value_incl_gather_plan)
ms_per_step  = wall clock per step (kernel map + plan + block, host launches
               included)

The CPU baseline (rank 0, N=1 only) times the oracle's restatement of the
reference CPU path on the same inputs: im2col gather + FP32 GEMM (the GGML CPU
decomposition) at the reference's default 8 threads and on all usable cores,
and the fine kernel map alone single-threaded; the reference's own whole
SlatTables::build, compiled from its sources (oracle/_ref), is timed beside it.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
import __graft_entry__ as ge  # noqa: E402

METRIC = "sparse-conv effective TFLOP/s + kernel-map Mvox/s, 64^3 ~30k vox C=128"
PEAK_BF16_TFLOPS = 2516.6
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
KMAP_BYTES_PER_VOXEL = 124  # 16 B coords in + 108 B map out


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--channels", type=int, default=128)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--copy-calibration", action="store_true",
                   help="run only a 256 MiB copy kernel (HBM counter calibration)")
    p.add_argument("--no-extras", action="store_true",
                   help="skip the other configs (1, 3, 4, 5, coarsen, subdivide)")
    p.add_argument("--profile-only", action="store_true",
                   help="run --steps untimed steps (kernel map + BF16 block) and exit: a short "
                        "program for counter collection")
    p.add_argument("--profile-kmap", action="store_true",
                   help="run --steps untimed kernel maps on each of the mesh decoder's child sets "
                        "(226,120 and 1,808,960 voxels) and exit: for counter collection")
    return p.parse_args()


class Block:
    """SparseResBlock at one dtype: conv(+LN+SiLU) then conv(+residual)."""

    def __init__(self, s3dx, W, dtype, n, c, seed, stream):
        self.s3dx, self.n, self.c, self.dtype, self.stream = s3dx, n, c, dtype, stream
        x = W.normal_f32(seed, 100, (n, c))
        w1 = W.conv_weight(seed, 101, c, c)
        w2 = W.conv_weight(seed, 102, c, c)
        b = np.zeros(c, np.float32)
        self.host = dict(x=x, w1=w1, w2=w2, b=b)
        store = np.uint16 if dtype == s3dx.BF16 else np.float32
        xd = W.f32_to_bf16_bits(x) if dtype == s3dx.BF16 else x
        self.x = s3dx.DeviceArray.from_host(xd)
        self.h = s3dx.DeviceArray((n, c), store)
        self.y = s3dx.DeviceArray((n, c), store)
        self.conv1 = (s3dx.SparseConv(c, c, 27, dtype).set_weights(w1, s3dx.WEIGHT_SLAT, b)
                      .set_layernorm(True, 1e-6).set_silu(True))
        self.conv2 = s3dx.SparseConv(c, c, 27, dtype).set_weights(w2, s3dx.WEIGHT_SLAT, b)

    def run(self, kmap, ev=None, plan=None):
        s = self.stream
        if ev:
            ev[0].record(s)
        self.conv1.run(self.x, self.n, kmap, self.n, self.h, self.dtype, None, s, plan=plan)
        if ev:
            ev[1].record(s)
        self.conv2.run(self.h, self.n, kmap, self.n, self.y, self.dtype, self.x, s, plan=plan)
        if ev:
            ev[2].record(s)


def _event_us(s3dx, stream, fn, reps=10, warm=2):
    """Median device time of fn() on `stream`, HIP timing events around each
    call, after >= `warm` calls and ~50 ms of untimed calls (clocks settle)."""
    t0 = time.perf_counter()
    done = 0
    while done < warm or time.perf_counter() - t0 < 0.05:
        fn()
        done += 1
        if done % 8 == 0:
            stream.synchronize()
    ev = [(s3dx.Event(timing=True), s3dx.Event(timing=True)) for _ in range(reps)]
    for a, b in ev:
        a.record(stream)
        fn()
        b.record(stream)
    stream.synchronize()
    return statistics.median(a.elapsed_ms(b) * 1e3 for a, b in ev)


def _wall_us(fn, reps=5):
    fn()
    t = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        t.append(time.perf_counter() - t0)
    return statistics.median(t) * 1e6


def extras(s3dx, W, stream, seed):
    """The other configs of the path, timed on the same GPU (not the headline)."""
    out = {}
    bf, f32 = s3dx.BF16, s3dx.F32

    def conv_entry(name, conv, x, n_in, kmap, n_out, y, ydt, pairs, cin, cout, peak, residual=None,
                   planned=False):
        gp, plan_us = None, None
        if planned:  # the map's gather plan, built once per map (timed apart)
            gp = conv.gather_plan(n_in, kmap, n_out, stream)
            plan_us = _event_us(s3dx, stream, lambda: gp.rebuild(conv, n_in, kmap, n_out, stream))
        us = _event_us(s3dx, stream, lambda: conv.run(x, n_in, kmap, n_out, y, ydt, residual, stream, plan=gp))
        flops = 2.0 * cin * cout * pairs
        out[name] = {"us": us, "tflops": flops / us / 1e6, "peak_tflops": peak,
                     "frac": flops / us / 1e6 / peak, "rows": n_out, "pairs": pairs,
                     "plan": conv.plan(n_in, n_out, gp)}
        if planned:
            out[name]["gather_plan_us"] = plan_us

    # config 1: one FP32 64 -> 64 conv on the 20-radius shell (10,366 voxels)
    c1 = W.shell_64()
    n1 = c1.shape[0]
    k1 = s3dx.kmap_subm3(s3dx.DeviceArray.from_host(c1, stream), n1, n1, stream=stream)
    p1 = W.kmap_pairs(k1.download(stream), n1)
    conv = s3dx.SparseConv(64, 64, 27, f32).set_weights(W.conv_weight(seed, 201, 64, 64), s3dx.WEIGHT_SLAT, None)
    x = s3dx.DeviceArray.from_host(W.normal_f32(seed, 200, (n1, 64)), stream)
    y = s3dx.DeviceArray((n1, 64), np.float32)
    conv_entry("config1_fp32_conv_64", conv, x, n1, k1, n1, y, f32, p1, 64, 64, PEAK_FP32_TFLOPS)

    # coarsen (SlatTables downsample tables) and config 3: 1024 -> 1024 BF16 on the coarse set
    c2 = W.shells_union(seed)
    n2 = c2.shape[0]
    d2 = s3dx.DeviceArray.from_host(c2, stream)
    res = {}

    c_out = (s3dx.DeviceArray((n2, 4), np.int32), s3dx.DeviceArray((n2,), np.int32),
             s3dx.DeviceArray((8 * n2,), np.int32), s3dx.DeviceArray((n2,), np.float32))
    c_ws = s3dx.DeviceArray(s3dx.coarsen2_workspace_size(n2), np.uint8)

    def do_coarsen():
        res["c"] = s3dx.coarsen2(d2, n2, stream, out=c_out, workspace=c_ws)
    us = _wall_us(do_coarsen)
    nc, cc = res["c"][0], res["c"][1]
    out["coarsen2"] = {"us_wall": us, "fine": n2, "coarse": nc, "mvox_s": n2 / us,
                       "note": "wall clock including its one host synchronization, buffers reused"}
    k3 = s3dx.kmap_subm3(cc, nc, nc, stream=stream)
    p3 = W.kmap_pairs(k3.download(stream)[:nc], nc)
    conv = s3dx.SparseConv(1024, 1024, 27, bf).set_weights(W.conv_weight(seed, 301, 1024, 1024), s3dx.WEIGHT_SLAT, None)
    x = s3dx.DeviceArray.from_host(W.f32_to_bf16_bits(W.normal_f32(seed, 300, (nc, 1024))), stream)
    y = s3dx.DeviceArray((nc, 1024), np.uint16)
    conv_entry("config3_bf16_conv_1024", conv, x, nc, k3, nc, y, bf, p3, 1024, 1024, PEAK_BF16_TFLOPS,
               planned=True)

    # The SLat flow's largest conv, out_blocks.0.conv1 (slat_flow_graph.cpp:441-470):
    # 2048 -> 128 over the fine set, with the fused LayerNorm + modulate + SiLU.
    k2 = s3dx.kmap_subm3(d2, n2, n2, stream=stream)
    p2 = W.kmap_pairs(k2.download(stream), n2)
    mscale = s3dx.DeviceArray.from_host(W.normal_f32(seed, 322, (128,), 0.1), stream)
    mshift = s3dx.DeviceArray.from_host(W.normal_f32(seed, 324, (128,), 0.1), stream)
    conv = (s3dx.SparseConv(2048, 128, 27, bf).set_weights(W.conv_weight(seed, 321, 2048, 128), s3dx.WEIGHT_SLAT,
                                                            W.normal_f32(seed, 323, (128,), 0.1))
            .set_layernorm(True, 1e-6).set_modulate(mscale, mshift).set_silu(True))
    x = s3dx.DeviceArray.from_host(W.f32_to_bf16_bits(W.normal_f32(seed, 320, (n2, 2048))), stream)
    y = s3dx.DeviceArray((n2, 128), np.uint16)
    conv_entry("slat_out_block0_conv1_bf16_2048_128", conv, x, n2, k2, n2, y, bf, p2, 2048, 128, PEAK_BF16_TFLOPS,
               planned=True)

    # SLat sparse I/O (slat_flow_graph.cpp:159-190) at C=128 BF16: 2x mean-pool
    # of the fine rows onto the coarse set, then nearest upsample back.
    # Compulsory bytes: every source row, index and output row once.
    f2c, ch, inv = res["c"][2], res["c"][3], res["c"][4]
    xf = s3dx.DeviceArray.from_host(W.f32_to_bf16_bits(W.normal_f32(seed, 310, (n2, 128))), stream)
    yc = s3dx.DeviceArray((nc, 128), np.uint16)
    yf = s3dx.DeviceArray((n2, 128), np.uint16)
    for name, fn, nbytes in (
            ("downsample_mean_bf16_128", lambda: s3dx.downsample_mean(xf, bf, n2, 128, ch, inv, nc, yc, stream),
             n2 * 256 + nc * (8 * 4 + 4 + 256)),
            ("upsample_nearest_bf16_128", lambda: s3dx.upsample_nearest(yc, bf, nc, 128, f2c, n2, yf, stream),
             nc * 256 + n2 * (4 + 256))):
        us = _event_us(s3dx, stream, fn)
        out[name] = {"us": us, "gb_s": nbytes / us / 1e3, "peak_gb_s": PEAK_HBM_GBS,
                     "frac": nbytes / us / 1e3 / PEAK_HBM_GBS, "fine": n2, "coarse": nc, "bytes": nbytes}

    # occupancy -> coordinates (session.cpp:1437-1474) on a noisy 64^3 field
    # with the reference fixture's density (~27% occupied, mostly surface):
    # threshold, surface prune, downsample to 42,000 rows; buffers reused,
    # three host synchronizations (the row counts) inside the timed region.
    occ = s3dx.DeviceArray.from_host(W.occupancy_noise(seed), stream)
    cells = 64 ** 3
    b_occ = s3dx.DeviceArray((cells, 4), np.int32)
    b_surf = s3dx.DeviceArray((cells, 4), np.int32)
    b_down = s3dx.DeviceArray((42000, 4), np.int32)
    ws = {}

    def do_coords():
        n1, _ = s3dx.occupancy_coords(occ, (64, 64, 64), stream, out=b_occ, workspace=ws.get("o"))
        n2_, _ = s3dx.prune_surface(b_occ, n1, stream, out=b_surf, workspace=ws.get("p"))
        n3, _ = (s3dx.downsample_coords(b_surf, n2_, 42000, 2, 42, stream, out=b_down, workspace=ws.get("d"))
                 if n2_ > 42000 else (n2_, b_surf))
        res["coords"] = (n1, n2_, n3)
    do_coords()
    n1, n2_, n3 = res["coords"]
    ws["o"] = s3dx.DeviceArray(s3dx.occupancy_workspace_size((64, 64, 64)), np.uint8)
    ws["p"] = s3dx.DeviceArray(s3dx.prune_surface_workspace_size(n1), np.uint8)
    ws["d"] = s3dx.DeviceArray(s3dx.downsample_coords_workspace_size(n2_), np.uint8)
    us = _wall_us(do_coords)
    out["coords_from_occupancy_64"] = {"us_wall": us, "cells": cells, "occupied": n1, "surface": n2_,
                                       "rows": n3, "mvox_s": cells / us,
                                       "note": "threshold + prune + downsample, wall clock with their three "
                                               "host synchronizations, buffers reused"}

    # subdivide (MeshSubdivideTables) and config 4: 192 -> 192 BF16 over the children,
    # gathering parent rows (repeat x8) plus a per-slot offset
    s_out = (s3dx.DeviceArray((8 * n2, 4), np.int32), s3dx.DeviceArray((8 * n2, 27), np.int32))
    s_ws = s3dx.DeviceArray(s3dx.subdivide2_workspace_size(n2), np.uint8)

    def do_subdivide():
        res["s"] = s3dx.subdivide2(d2, n2, True, stream, out=s_out, workspace=s_ws)
    us = _wall_us(do_subdivide)
    ch, k4 = res["s"]
    n4 = 8 * n2
    out["subdivide2"] = {"us_wall": us, "parents": n2, "children": n4, "mvox_s": n4 / us,
                         "note": "wall clock including its one host synchronization, buffers reused"}
    p4 = W.kmap_pairs(k4.download(stream), n4)
    conv = (s3dx.SparseConv(192, 192, 27, bf).set_weights(W.conv_weight(seed, 401, 192, 192, layout="mesh"),
                                                           s3dx.WEIGHT_MESH, None)
            .set_gather_parent(True, W.normal_f32(seed, 402, (8, 192), 0.02)))
    x = s3dx.DeviceArray.from_host(W.f32_to_bf16_bits(W.normal_f32(seed, 400, (n2, 192))), stream)
    y = s3dx.DeviceArray((n4, 192), np.uint16)
    conv_entry("config4_bf16_conv_192_children", conv, x, n2, k4, n4, y, bf, p4, 192, 192, PEAK_BF16_TFLOPS)

    # Kernel maps (mesh sentinel -1) over the mesh decoder's child sets at
    # 128^3 and 256^3: outside the 64^3 window, so every voxel takes the
    # hashed path.  Algorithmic bytes: 16 B coordinates in + 108 B map out.
    ch1, _ = s3dx.subdivide2(ch, n4, False, stream)
    for name, cset, cn in (("kmap_subm3_mesh_children_128", ch, n4),
                           ("kmap_subm3_mesh_children_256", ch1, 8 * n4)):
        km = s3dx.DeviceArray((cn, 27), np.int32)
        kw = s3dx.DeviceArray(s3dx.kmap_workspace_size(cn), np.uint8)
        us = _event_us(s3dx, stream, lambda: s3dx.kmap_subm3(cset, cn, -1, km, kw, stream))
        gbs = cn * KMAP_BYTES_PER_VOXEL / us / 1e3
        out[name] = {"us": us, "voxels": cn, "mvox_s": cn / us, "gb_s": gbs, "peak_gb_s": PEAK_HBM_GBS,
                     "frac": gbs / PEAK_HBM_GBS}
        del km, kw
    del ch1

    # config 5: 768-channel parents -> upsample block (768 -> 192) -> upsample
    # block (192 -> 96) -> linear 96 -> 101 (FP32), the mesh decoder's sparse stack
    out["config5_stack"] = mesh_stack(s3dx, W, stream, seed, d2, n2, ch, k4)
    # one SLat flow forward's sparse stages, BF16 and FP32
    out["slat_forward_bf16"] = slat_forward(s3dx, W, stream, seed, s3dx.BF16)
    out["slat_forward_fp32"] = slat_forward(s3dx, W, stream, seed, s3dx.F32, reps=3)
    return out


def slat_forward(s3dx, W, stream, seed, dtype, reps=5):
    """One SLat flow forward's sparse stages at config-2 shapes (28,265 fine /
    5,086 coarse voxels), slat_flow_graph.cpp:284-291 and 441-503, each op
    timed by HIP events around it: input_blocks.0 (128 -> 128), 2x mean-pool,
    input_blocks.1 (128 -> 1024, Linear skip), concat skip1 + upsample,
    out_blocks.0 (2048 -> 128), concat skip0, out_blocks.1 (256 -> 128).  Each
    block: LayerNorm(affine) + SiLU pass, conv1 (+ LayerNorm + modulate +
    SiLU), Linear skip, conv2 (+ skip).  Convs run with the fine or coarse
    map's gather plan (built once per sample, timed apart).  The reference
    runs 38 such forwards per sample (session.cpp:1689-1763)."""
    bf = dtype == s3dx.BF16
    store = np.uint16 if bf else np.float32
    es = 2 if bf else 4
    peak = PEAK_BF16_TFLOPS if bf else PEAK_FP32_TFLOPS
    coords = W.shells_union(seed)
    t = s3dx.SlatTables()
    t.build(coords, stream)
    nf, nc = t.nf, t.nc
    pf = W.kmap_pairs(t.conv_fine.download(stream), nf)
    pc = W.kmap_pairs(t.conv_coarse.download(stream)[:nc], nc)

    def dev(a):
        a = np.ascontiguousarray(a, np.float32)
        return s3dx.DeviceArray.from_host(W.f32_to_bf16_bits(a) if bf else a, stream)

    blocks = []
    for b, (cin, cout, coarse) in enumerate(((128, 128, False), (128, 1024, True), (2048, 128, False),
                                             (256, 128, False))):
        k = 700 + 20 * b
        blk = {"cin": cin, "cout": cout, "coarse": coarse,
               "n1w": s3dx.DeviceArray.from_host(W.normal_f32(seed, k, (cin,), 0.2) + 1.0, stream),
               "n1b": s3dx.DeviceArray.from_host(W.normal_f32(seed, k + 1, (cin,), 0.2), stream),
               "ms": s3dx.DeviceArray.from_host(W.normal_f32(seed, k + 2, (cout,), 0.3), stream),
               "mh": s3dx.DeviceArray.from_host(W.normal_f32(seed, k + 9, (cout,), 0.3), stream)}
        blk["conv1"] = (s3dx.SparseConv(cin, cout, 27, dtype)
                        .set_weights(W.conv_weight(seed, k + 3, cin, cout), s3dx.WEIGHT_SLAT,
                                     W.normal_f32(seed, k + 4, (cout,), 0.1))
                        .set_layernorm(True, 1e-6).set_silu(True))
        blk["conv1"].set_modulate(blk["ms"], blk["mh"])
        blk["conv2"] = s3dx.SparseConv(cout, cout, 27, dtype).set_weights(
            W.conv_weight(seed, k + 5, cout, cout), s3dx.WEIGHT_SLAT, W.normal_f32(seed, k + 6, (cout,), 0.1))
        blk["skip"] = (s3dx.SparseConv(cin, cout, 1, dtype).set_weights(
            W.conv_weight(seed, k + 7, cin, cout, kvol=1), s3dx.WEIGHT_SLAT, W.normal_f32(seed, k + 8, (cout,), 0.1))
            if cin != cout else None)
        blocks.append(blk)
    plan_f = blocks[0]["conv1"].gather_plan(nf, t.conv_fine, nf, stream)
    plan_c = blocks[1]["conv2"].gather_plan(nc, t.conv_coarse, nc, stream)
    plan_us = {"fine": _event_us(s3dx, stream, lambda: plan_f.rebuild(blocks[0]["conv1"], nf, t.conv_fine, nf, stream)),
               "coarse": _event_us(s3dx, stream,
                                   lambda: plan_c.rebuild(blocks[1]["conv2"], nc, t.conv_coarse, nc, stream))}
    h0 = dev(W.normal_f32(seed, 790, (nf, 128)))
    trunk = dev(W.normal_f32(seed, 791, (nc, 1024)))
    buf = lambda rows, c: s3dx.DeviceArray((rows, c), store)  # noqa: E731
    skip0, xc, skip1 = buf(nf, 128), buf(nc, 128), buf(nc, 1024)
    xcat, h1, out = buf(nf, 2048), buf(nf, 128), buf(nf, 128)
    tmp_h, tmp_y1, tmp_s = buf(nf, 2048), buf(nf, 1024), buf(nf, 1024)
    ops = []  # (stage, op, fn, flops, bytes)

    def block_ops(stage, blk, x, y):
        n = nc if blk["coarse"] else nf
        kmap = t.conv_coarse if blk["coarse"] else t.conv_fine
        plan = plan_c if blk["coarse"] else plan_f
        pairs = pc if blk["coarse"] else pf
        cin, cout = blk["cin"], blk["cout"]
        h, y1, sk = tmp_h, tmp_y1, tmp_s
        ops.append((stage, "layernorm_silu", lambda: s3dx.layernorm_rows(
            x, dtype, n, cin, 1e-6, blk["n1w"], blk["n1b"], silu=True, y=h, y_dtype=dtype, stream=stream),
            0.0, 2.0 * n * cin * es))
        ops.append((stage, f"conv1_{cin}_{cout}", lambda: blk["conv1"].run(
            h, n, kmap, n, y1, dtype, None, stream, plan=plan), 2.0 * cin * cout * pairs, None))
        res = x
        if blk["skip"] is not None:
            ops.append((stage, f"skip_{cin}_{cout}", lambda: blk["skip"].run(x, n, None, n, sk, dtype, None, stream),
                        2.0 * cin * cout * n, None))
            res = sk
        ops.append((stage, f"conv2_{cout}_{cout}", lambda: blk["conv2"].run(
            y1, n, kmap, n, y, dtype, res, stream, plan=plan), 2.0 * cout * cout * pairs, None))

    block_ops("input_blocks.0", blocks[0], h0, skip0)
    ops.append(("input_blocks.1", "downsample_mean", lambda: s3dx.downsample_mean(
        skip0, dtype, nf, 128, t.coarse_children, t.coarse_inv_count, nc, xc, stream), 0.0,
        (nf * 128 + nc * 128) * es + nc * 36))
    block_ops("input_blocks.1", blocks[1], xc, skip1)
    ops.append(("out_blocks.0", "concat_upsample", lambda: s3dx.concat_rows(
        trunk, 1024, skip1, 1024, dtype, nc, t.fine_to_coarse, nf, xcat, stream), 0.0,
        (2 * nc * 1024 + nf * 2048) * es + nf * 4))
    block_ops("out_blocks.0", blocks[2], xcat, h1)
    ops.append(("out_blocks.1", "concat", lambda: s3dx.concat_rows(
        h1, 128, skip0, 128, dtype, nf, None, nf, xcat, stream), 0.0, 2 * nf * 256 * es))
    block_ops("out_blocks.1", blocks[3], xcat, out)

    def forward(ev=None):
        for i, (_, _, fn, _, _) in enumerate(ops):
            if ev:
                ev[i].record(stream)
            fn()
        if ev:
            ev[len(ops)].record(stream)

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.1:
        forward()
        stream.synchronize()
    times = [[] for _ in ops]
    for _ in range(reps):
        ev = [s3dx.Event(timing=True) for _ in range(len(ops) + 1)]
        forward(ev)
        stream.synchronize()
        for i in range(len(ops)):
            times[i].append(ev[i].elapsed_ms(ev[i + 1]) * 1e3)
    stages, total, total_flops = {}, 0.0, 0.0
    for (stage, op, _, fl, nbytes), tt in zip(ops, times):
        us = statistics.median(tt)
        e = {"us": us}
        if fl:
            e.update(tflops=fl / us / 1e6, frac=fl / us / 1e6 / peak)
        else:
            e.update(gb_s=nbytes / us / 1e3, frac=nbytes / us / 1e3 / PEAK_HBM_GBS)
        stages.setdefault(stage, {})[op] = e
        total += us
        total_flops += fl
    plans = {b: {"conv1": blk["conv1"].plan(nc if blk["coarse"] else nf, nc if blk["coarse"] else nf,
                                            plan_c if blk["coarse"] else plan_f),
                 "conv2": blk["conv2"].plan(nc if blk["coarse"] else nf, nc if blk["coarse"] else nf,
                                            plan_c if blk["coarse"] else plan_f)}
             for b, blk in zip(("input_blocks.0", "input_blocks.1", "out_blocks.0", "out_blocks.1"), blocks)}
    return {"us_per_forward": total, "tflops": total_flops / total / 1e6, "frac": total_flops / total / 1e6 / peak,
            "fine": nf, "coarse": nc, "pairs_fine": pf, "pairs_coarse": pc, "gather_plan_us": plan_us,
            "ms_per_sample_38_forwards": 38 * total / 1e3, "stages": stages, "plans": plans,
            "dtype": "bf16" if bf else "fp32"}


def mesh_stack(s3dx, W, stream, seed, d0, p0, ch0, k0):
    bf, f32 = s3dx.BF16, s3dx.F32
    stages, flops = {}, {}

    def block(level, xp, p, kmap, cin, cout):
        n = 8 * p
        g1 = s3dx.DeviceArray.from_host(W.normal_f32(seed, 510 + level, (cin,), 0.2) + 1.0, stream)
        b1 = s3dx.DeviceArray.from_host(W.normal_f32(seed, 520 + level, (cin,), 0.2), stream)
        g2 = s3dx.DeviceArray.from_host(W.normal_f32(seed, 530 + level, (cout,), 0.2) + 1.0, stream)
        b2 = s3dx.DeviceArray.from_host(W.normal_f32(seed, 540 + level, (cout,), 0.2), stream)
        conv1 = (s3dx.SparseConv(cin, cout, 27, bf)
                 .set_weights(W.conv_weight(seed, 550 + level, cin, cout, layout="mesh"), s3dx.WEIGHT_MESH, None)
                 .set_gather_parent(True))
        # 1x1 skip of repeat_children(x) == repeat_children(1x1 skip of x): run
        # it on the parents; conv2 adds residual row i >> 3.
        skip = s3dx.SparseConv(cin, cout, 1, bf).set_weights(
            W.conv_weight(seed, 560 + level, cin, cout, kvol=1, layout="mesh"), s3dx.WEIGHT_MESH, None)
        conv2 = (s3dx.SparseConv(cout, cout, 27, bf).set_weights(
            W.conv_weight(seed, 570 + level, cout, cout, layout="mesh"), s3dx.WEIGHT_MESH, None)
            .set_residual_parent(True))
        y1 = s3dx.DeviceArray((n, cout), np.uint16)
        ys = s3dx.DeviceArray((p, cout), np.uint16)
        y2 = s3dx.DeviceArray((n, cout), np.uint16)
        pairs = W.kmap_pairs(kmap.download(stream), n)
        flops[level] = 2.0 * pairs * (cin * cout + cout * cout) + 2.0 * p * cin * cout
        gn1 = s3dx.groupnorm_stats(xp, bf, p, cin, 32, 1e-5, g1, b1, stream)
        gn2 = s3dx.groupnorm_stats(y1, bf, n, cout, 32, 1e-5, g2, b2, stream)
        conv1.set_input_affine_silu(gn1[0], gn1[1])
        conv2.set_input_affine_silu(gn2[0], gn2[1])

        def run():
            s3dx.groupnorm_stats(xp, bf, p, cin, 32, 1e-5, g1, b1, stream, out=gn1)
            conv1.run(xp, p, kmap, n, y1, bf, None, stream)
            skip.run(xp, p, None, p, ys, bf, None, stream)
            s3dx.groupnorm_stats(y1, bf, n, cout, 32, 1e-5, g2, b2, stream, out=gn2)
            conv2.run(y1, n, kmap, n, y2, bf, ys, stream)
        run.keep = (g1, b1, g2, b2, gn1, gn2)
        return run, y2, n

    x0 = s3dx.DeviceArray.from_host(W.f32_to_bf16_bits(W.normal_f32(seed, 500, (p0, 768))), stream)
    run0, y0, n0 = block(0, x0, p0, k0, 768, 192)
    run0()
    ch1, k1 = s3dx.subdivide2(ch0, n0, True, stream)
    run1, y1, n1 = block(1, y0, n0, k1, 192, 96)
    # FP32 head fed the BF16 block output directly (rows widened exactly in the kernel)
    head = (s3dx.SparseConv(96, 101, 1, f32).set_weights(W.conv_weight(seed, 590, 96, 101, kvol=1), s3dx.WEIGHT_SLAT, None)
            .set_input_dtype(bf))
    out = s3dx.DeviceArray((n1, 101), np.float32)

    def run_head():
        head.run(y1, n1, None, n1, out, f32, None, stream)

    stages["level0_block_us"] = _event_us(s3dx, stream, run0, reps=5)
    stages["level1_block_us"] = _event_us(s3dx, stream, run1, reps=5)
    stages["head_us"] = _event_us(s3dx, stream, run_head, reps=5)
    total = stages["level0_block_us"] + stages["level1_block_us"] + stages["head_us"]
    # The two subdivides (children coordinates + their kernel maps) that feed the
    # blocks, timed on reused buffers, wall clock with their one host synchronization each.
    subs = {}
    for lv, (cin_d, cn) in enumerate(((d0, p0), (ch0, n0))):
        so = (s3dx.DeviceArray((8 * cn, 4), np.int32), s3dx.DeviceArray((8 * cn, 27), np.int32))
        sw = s3dx.DeviceArray(s3dx.subdivide2_workspace_size(cn), np.uint8)
        subs[f"subdivide{lv}_us_wall"] = _wall_us(
            lambda: s3dx.subdivide2(cin_d, cn, True, stream, out=so, workspace=sw))
    total_all = total + subs["subdivide0_us_wall"] + subs["subdivide1_us_wall"]
    fl = flops[0] + flops[1] + 2.0 * n1 * 96 * 101
    return {**stages, **subs, "total_us": total, "total_with_subdivides_us": total_all,
            "parents": p0, "level0_children": n0, "level1_children": n1,
            "tflops": fl / total / 1e6, "tflops_with_subdivides": fl / total_all / 1e6,
            "dtype": "bf16 blocks, fp32 head",
            "note": "per block: GN32 stats, conv (GN affine+SiLU pass over the parents, gather of "
                    "parent row j>>3), 1x1 skip over the parents, GN32 stats, conv (GN affine+SiLU "
                    "pass) + skip row i>>3 as residual; flops count the skip once per parent; "
                    "total_us is the three layer stages, total_with_subdivides_us adds the two "
                    "subdivides (children + child kernel maps) that build their tables"}


def profile_kmap(s3dx, W, seed, steps):
    """Kernel maps (mesh sentinel) on the 128^3 and 256^3 child sets of the
    8-shell union, `steps` builds each, untimed."""
    stream = s3dx.Stream()
    c = W.shells_union(seed)
    d = s3dx.DeviceArray.from_host(c, stream)
    ch, _ = s3dx.subdivide2(d, c.shape[0], False, stream)
    ch1, _ = s3dx.subdivide2(ch, 8 * c.shape[0], False, stream)
    for cset, n in ((ch, 8 * c.shape[0]), (ch1, 64 * c.shape[0])):
        km = s3dx.DeviceArray((n, 27), np.int32)
        ws = s3dx.DeviceArray(s3dx.kmap_workspace_size(n), np.uint8)
        for _ in range(steps):
            s3dx.kmap_subm3(cset, n, -1, km, ws, stream)
        stream.synchronize()
        print(json.dumps({"profile_kmap_voxels": n, "builds": steps}), flush=True)


def copy_calibration(s3dx):
    n = 64 * 1024 * 1024  # 256 MiB of f32
    a = s3dx.DeviceArray((n,), np.float32)
    b = s3dx.DeviceArray((n,), np.float32)
    for _ in range(3):
        s3dx.convert(a, s3dx.F32, n, b, s3dx.F32)
    s3dx.synchronize()
    print(json.dumps({"copy_calibration_bytes_read": n * 4, "copy_calibration_bytes_written": n * 4}))


def _timed_runs(fn, budget_s: float, max_runs: int):
    """Run fn until about budget_s seconds have passed; per-run times."""
    times, start = [], time.perf_counter()
    while len(times) < max_runs and (not times or time.perf_counter() - start < budget_s):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return times


def cpu_baseline(block, kmap_host, n, pairs, coords, W, conv_budget_s=6.0, kmap_budget_s=3.0):
    """Bounded CPU sample of the same workload (about 20 s of host work).

    conv: the oracle's im2col gather + FP32 GEMM (the GGML CPU op
    decomposition, slat_flow_graph.cpp:128-130) at the reference's default of
    8 threads (objects_native.hpp:29) -- the reported `value` -- and at every
    core this process may use (capped at 16, the host share of one GPU).
    kmap: the fine map alone, build_conv (sparse_ops.cpp:117-142) as the
    oracle restates it with ordered maps, single-threaded as the reference
    runs it -- compared with the GPU's fine-map build; the reference's whole
    SlatTables::build (fine + coarse maps + APE, compiled from
    sparse_ops.cpp) is timed beside it for context."""
    O = ge.load_oracle()
    h = block.host
    c = block.c
    flops = 2.0 * c * c * pairs
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    legs = {}
    for threads in (8, min(16, usable)):
        if threads in legs:
            continue
        O.conv_im2col_gemm_f32(h["x"], kmap_host, n, h["w1"], c, h["b"], threads)  # warm-up
        ts = _timed_runs(lambda: O.conv_im2col_gemm_f32(h["x"], kmap_host, n, h["w1"], c, h["b"], threads),
                         conv_budget_s, 2000)
        legs[threads] = (statistics.median(ts), len(ts), sum(ts))
    t8, runs8, tot8 = legs[8]
    kmap_t = _timed_runs(lambda: O.kmap_subm3(coords, n), kmap_budget_s, 2000)
    t_kmap = statistics.median(kmap_t)
    out = {
        "value": flops / t8 / 1e12, "unit": "TFLOP/s", "cores": 8, "kind": "port",
        "sample": (f"{runs8} runs ({tot8:.1f} s) of one {c}->{c} FP32 sparse conv over the same {n} voxels / "
                   f"{pairs} pairs: im2col gather + FP32 GEMM on 8 threads (the reference's default thread "
                   f"count; GGML CPU decomposition), median {t8 * 1e3:.1f} ms per conv"),
        "conv_ms": t8 * 1e3,
        "all_cores": {str(k): {"threads": k, "conv_ms": v[0] * 1e3, "value": flops / v[0] / 1e12, "runs": v[1]}
                      for k, v in legs.items()},
        "nproc": os.cpu_count(), "usable_cores": usable,
        "kmap": {"value": n / t_kmap / 1e6, "unit": "Mvox/s", "cores": 1, "kind": "port", "ms": t_kmap * 1e3,
                 "sample": (f"{len(kmap_t)} runs ({sum(kmap_t):.1f} s) of the fine kernel map alone "
                            "(build_conv, sparse_ops.cpp:117-142, the oracle's ordered-map restatement), "
                            "single thread, median")},
        "cpu_model": cpu_model(),
    }
    if O.ref_available():
        ref_t = _timed_runs(lambda: O.ref_slat_tables(coords, 6), kmap_budget_s, 2000)
        out["kmap_reference_slat_tables"] = {
            "value": n / statistics.median(ref_t) / 1e6, "unit": "Mvox/s", "cores": 1, "kind": "reference",
            "ms": statistics.median(ref_t) * 1e3,
            "sample": (f"{len(ref_t)} runs of the reference's whole SlatTables::build (fine + coarse maps, "
                       "downsample tables, 6-channel APE) compiled from sparse_ops.cpp; not like-for-like "
                       "with the GPU's fine map")}
    return out


def cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(every box has one GPU and the path has no multi-GPU leg)", file=sys.stderr)
        sys.exit(2)
    s3dx = ge.load_package()
    W = s3dx.workloads
    if args.copy_calibration:
        copy_calibration(s3dx)
        return
    if args.profile_kmap:
        profile_kmap(s3dx, W, args.seed, args.steps)
        return
    c = args.channels
    coords = W.shells_union(args.seed)
    n = coords.shape[0]
    stream = s3dx.Stream()
    dc = s3dx.DeviceArray.from_host(coords, stream)
    kmap = s3dx.DeviceArray((n, 27), np.int32)
    ws = s3dx.DeviceArray(s3dx.kmap_workspace_size(n), np.uint8)
    s3dx.kmap_subm3(dc, n, n, kmap, ws, stream)
    kmap_host = kmap.download(stream)
    pairs = W.kmap_pairs(kmap_host, n)
    flops = 2.0 * c * c * pairs  # effective FLOPs per conv

    bf = Block(s3dx, W, s3dx.BF16, n, c, args.seed, stream)
    # The map's gather plan (per 64-row tile: distinct source rows + slot
    # table), rebuilt in place after each map build and shared by both convs.
    gplan = bf.conv1.gather_plan(n, kmap, n, stream)

    def step(ev_k=None, ev_b=None):
        # the kernel map and its gather plan from the same lookups (one pass)
        if ev_k:
            ev_k[0].record(stream)
        s3dx.kmap_subm3_planned(dc, n, n, kmap, gplan, bf.conv1, ws, stream)
        if ev_k:
            ev_k[1].record(stream)
        bf.run(kmap, ev_b, gplan)

    if args.profile_only:
        for _ in range(args.steps):
            step()
        stream.synchronize()
        print(json.dumps({"profile_only_steps": args.steps, "voxels": n, "pairs": pairs,
                          "plan": {"conv1": bf.conv1.plan(n, n, gplan), "conv2": bf.conv2.plan(n, n, gplan)}}),
              flush=True)
        return
    f32 = Block(s3dx, W, s3dx.F32, n, c, args.seed, stream)

    # Clock settle: the GPU ramps its clocks over tens of milliseconds of
    # load, so the step runs untimed for ~150 ms before the W warm-up steps
    # (10 warm-up steps alone leave the timed region ~6% below steady state).
    t_settle = time.perf_counter()
    while time.perf_counter() - t_settle < 0.15:
        for _ in range(20):
            step()
        stream.synchronize()
    for _ in range(args.warmup):
        step()
        f32.run(kmap)
    stream.synchronize()

    K = args.steps
    evk = [[s3dx.Event(timing=True), s3dx.Event(timing=True)] for _ in range(K)]
    evb = [[s3dx.Event(timing=True), s3dx.Event(timing=True), s3dx.Event(timing=True)] for _ in range(K)]
    stream.synchronize()
    t0 = time.perf_counter()
    for i in range(K):
        step(evk[i], evb[i])
    stream.synchronize()
    wall = time.perf_counter() - t0

    kmap_plan_ms = statistics.mean(evk[i][0].elapsed_ms(evk[i][1]) for i in range(K))
    conv1_ms = [evb[i][0].elapsed_ms(evb[i][1]) for i in range(K)]
    conv2_ms = [evb[i][1].elapsed_ms(evb[i][2]) for i in range(K)]
    conv_ms = statistics.mean(conv1_ms + conv2_ms)
    block_ms = statistics.mean(a + b for a, b in zip(conv1_ms, conv2_ms))
    # The map alone (s3dx_kmap_subm3) and the plan rebuild alone, for the
    # map's Mvox/s and beside the one-pass figure.
    kmap_avg = _event_us(s3dx, stream, lambda: s3dx.kmap_subm3(dc, n, n, kmap, ws, stream), reps=K) / 1e3
    gplan_ms = _event_us(s3dx, stream, lambda: gplan.rebuild(bf.conv1, n, kmap, n, stream), reps=K) / 1e3

    # FP32 block, timed the same way after the BF16 region.
    evf = [[s3dx.Event(timing=True), s3dx.Event(timing=True), s3dx.Event(timing=True)] for _ in range(K)]
    for i in range(K):
        f32.run(kmap, evf[i])
    stream.synchronize()
    f1 = [evf[i][0].elapsed_ms(evf[i][1]) for i in range(K)]
    f2 = [evf[i][1].elapsed_ms(evf[i][2]) for i in range(K)]
    f32_conv_ms = statistics.mean(f1 + f2)

    tflops = 2 * flops / (block_ms * 1e-3) / 1e12
    achieved = flops / (conv_ms * 1e-3) / 1e12
    # HBM bytes per launch from the committed FETCH_SIZE/WRITE_SIZE passes,
    # only while they describe the kernel this run launches.
    planned = {"conv1": bf.conv1.plan(n, n, gplan), "conv2": bf.conv2.plan(n, n, gplan)}
    kernel = ("conv_halo8_kernel" if "tiling=22" in planned["conv1"] else
              "conv_halo_kernel<2, true>" if "plan=64" in planned["conv1"] else "unplanned")
    traffic = None
    tfile = ROOT / "profiles" / "conv_bf16_c128_shells64_traffic.json"
    if tfile.exists():
        t = json.loads(tfile.read_text())
        if t.get("kernel") == kernel:
            traffic = t.get("hbm_bytes_per_launch")
    out = {
        "metric": METRIC,
        "value": tflops,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": wall / K * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": (f"SparseResBlock C={c} (conv3x3x3 -> LayerNorm -> SiLU -> conv3x3x3 -> +x) "
                         f"plus its kernel-map build, 8-shell union on a 64^3 grid, seed {args.seed}"),
            "voxels": n, "pairs": pairs, "channels": c, "seed": args.seed,
            "effective_gflop_per_conv": flops / 1e9,
            "dense27_gflop_per_conv": 2.0 * 27 * n * c * c / 1e9,
        },
        "kmap_mvox_s": n / (kmap_avg * 1e-3) / 1e6,
        "kmap_ms": kmap_avg,
        "gather_plan_ms": gplan_ms,
        "kmap_plan_ms": kmap_plan_ms,
        "block_ms": block_ms,
        "conv_kernel_ms": conv_ms,
        "conv1_ms": statistics.mean(conv1_ms),
        "conv2_ms": statistics.mean(conv2_ms),
        # The plan is per map (like the kernel map): this step amortizes it
        # over its two convs only, the SLat flow over every conv of a sample.
        "value_incl_gather_plan": 2 * flops / ((block_ms + gplan_ms) * 1e-3) / 1e12,
        "value_incl_kmap_and_plan": 2 * flops / ((block_ms + kmap_plan_ms) * 1e-3) / 1e12,
        "roofline": {
            "bound": "mfma", "achieved": achieved, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": achieved / PEAK_BF16_TFLOPS, "traffic": traffic,
            "kernel": kernel,
            "plan": planned,
        },
        "kmap_roofline": {
            "bound": "hbm", "achieved": n * KMAP_BYTES_PER_VOXEL / (kmap_avg * 1e-3) / 1e9,
            "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": n * KMAP_BYTES_PER_VOXEL / (kmap_avg * 1e-3) / 1e9 / PEAK_HBM_GBS,
        },
        "fp32": {
            "value": flops / (f32_conv_ms * 1e-3) / 1e12, "unit": "TFLOP/s",
            "conv_kernel_ms": f32_conv_ms, "peak": PEAK_FP32_TFLOPS,
            "frac": flops / (f32_conv_ms * 1e-3) / 1e12 / PEAK_FP32_TFLOPS,
        },
        "device": s3dx.device_name(),
    }
    if not args.no_extras:
        out["extras"] = extras(s3dx, W, stream, args.seed)
    if not args.no_cpu:
        cb = cpu_baseline(f32, kmap_host, n, pairs, coords, W)
        out["cpu_baseline"] = cb
        best = max(v["value"] for v in cb["all_cores"].values())
        out["gpu_over_cpu"] = {"conv_vs_8_threads": out["value"] / cb["value"],
                               "conv_vs_all_cores": out["value"] / best,
                               "kmap_vs_fine_map": out["kmap_mvox_s"] / cb["kmap"]["value"]}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
