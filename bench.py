#!/usr/bin/env python3
"""Benchmark of the MI355X SPH / hash-grid hot path (one GPU).

    python bench.py [--steps K] [--warmup W] [--gpus 1]

A "step" is one SPH substep of BASELINE.json configs[3]: 1,048,576 particles (dam-break lattice
block, h = cell = 0.01, 100^3 cells), re-hash + stable radix sort + cell ranges + density +
fused pressure/viscosity force + gravity / integrate / box, replayed from a captured HIP graph of
`--graph-substeps` substeps.  Inputs are resident in HBM before the timed region.  Exactly W
substeps run untimed, then exactly K are timed (K // G graph replays, then the remainder as one
eager call of the same kernels).  The defaults (W = 100, K = 900) are the survey's c3 protocol
(1000 substeps, mean of the last 900); with other arguments that protocol is also run on a
fresh trajectory and reported in extra.c3_protocol_last_900_of_1000.

One JSON line on stdout:
  value        particle-steps/s over the K timed substeps (wall clock between synchronisations)
  roofline     the dominant kernel of the substep: algorithmic bytes per launch / its mean
               launch time from HIP events on the context stream (G further substeps launched
               eagerly with every kernel bracketed by events, right after the timed region)
  cpu_baseline the single-threaded CPU restatement (oracle/) of the same substep on a bounded
               sample, timed on this host
  extra.sph_c0   configs[0] (50,000 particles) throughput, 2000 substeps after 100
  extra.sort_c1  the standalone 16,777,216-pair 32-bit sort and the same count of
               full-entropy 32-bit keys: Gkeys/s, bytes of the survey formula (68 N) and bytes
               actually moved (passes whose digit is constant move nothing) against the HBM
               roofline
  extra.query_c2 HashGrid build + neighbour query of configs[2] (4,194,304 points)
  extra.sph_c4   one grid build + density + force pass of configs[4] (8,388,608 particles,
               skewed occupancy): time, candidate tests per second, occupancy max / p99
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (REPO, REPO / "forge-gpu_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, GB/s
METRIC = "SPH particle-steps/s @1M; radix sort Gkeys/s; achieved HBM GB/s vs peak"
KERNELS = ["hash", "hist", "sort", "gather", "scan", "plan", "density", "prep", "force",
           "finalize"]
# A "pass" groups the kernels of one stage of the substep; its duration per substep is the sum
# of its kernels' launch durations, or, for the two neighbour passes, its wall time from the
# pass timers (the density pass: one launch of heavy parts and light items; the force pass:
# k_prep and that launch).
PASSES = {"hash": ["hash", "hist"], "sort": ["sort"], "gather": ["gather"], "scan": ["scan"],
          "plan": ["plan"], "density": ["density"], "force": ["prep", "force"],
          "finalize": ["finalize"]}
PASS_TIMERS = {"density": "density_pass", "force": "force_pass"}


def algorithmic_bytes(n: int, cells: int, passes: int, substeps: int = 1) -> dict:
    """Bytes each pass must move at minimum per substep (neighbour re-reads counted once: they
    are served from L2/LDS), averaged over one call of `substeps` substeps: the first rebuilds
    from the caller's arrays, the later ones (resident) from the previous substep's sorted
    state, and only the last moves the state back to particle order."""
    G = max(1, int(substeps))
    C4 = 4 * (cells + 1)
    entry = {
        "hash": 12 * n + 4 * n,                      # positions in, cell keys out
        # passes of 8-bit digits, or two of 10-bit digits for 17..20-bit keys (c3):
        # pass 0 reads keys (values are the indices), middle passes read + write (key, value),
        # the last pass writes (key, value) and the rank of each particle
        "sort": 12 * n + 16 * n * max(passes - 2, 0) + 16 * n + 4 * n,
        "gather": 4 * n + 24 * n + 32 * n,           # rank, pos / vel in, float4 pairs out
        "scan": 4 * n + C4,                          # sorted keys in, cell_start out
    }
    resident = {
        "hash": 4 * n,                               # keys (written by k_finalize) in
        "sort": 12 * n + 16 * n * max(passes - 2, 0) + 16 * n,
        "gather": 4 * n + 32 * n + 32 * n + 4 * n + C4,  # slot map, state in and out, + cells
        "scan": 0,                                   # done by the gather kernel
    }
    per = {k: (entry[k] + (G - 1) * resident[k]) / G for k in entry}
    per.update({
        "plan": 16 * n,                              # sorted positions
        "density": 16 * n + 12 * n + C4,             # positions in, 3 slab partials out
        "force": 32 * n + 12 * n + 36 * n + C4,      # pos / vel / density in, 9 partials out
        # pos, vel, partials in, new state (32 B) out; + next keys (all but the last substep);
        # the last substep also moves the state to particle order (rank, 32 B in, 28 B out)
        "finalize": 80 * n + 32 * n + ((G - 1) * 4 * n + 64 * n) / G,
    })
    return {k: int(v) for k, v in per.items()}


def survey_step_bytes(n: int, cells: int, passes: int) -> int:
    """Whole-substep algorithmic bytes with the neighbour re-reads counted once:
    N·(168 + 16p) + 24C for p 8-bit sort passes (hash 20, sort 4 + 16p, bounds 4, gather 60,
    density 20, force + epilogue 60 bytes per particle; the cell table written once, read twice)."""
    return n * (168 + 16 * passes) + 24 * cells


def read_traffic(kernel_pass: str):
    """HBM bytes per launch of a pass, from the committed rocprofv3 PMC summary
    (profiles/traffic_c3.txt, lines `<pass> fetch_bytes=<B> write_bytes=<B>`), or None."""
    f = REPO / "profiles" / "traffic_c3.txt"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        parts = line.split()
        if len(parts) >= 3 and parts[0] == kernel_pass:
            kv = dict(q.split("=", 1) for q in parts[1:] if "=" in q)
            try:
                return int(float(kv["fetch_bytes"]) + float(kv["write_bytes"]))
            except (KeyError, ValueError):
                return None
    return None


VALU_PEAK_INSTS = 256 * 2.4e9  # MI355X: one non-packed VALU wave instruction per cycle per CU
# The highest VALU wave-instruction rate measured on this GPU (SQ_INSTS_VALU over the kernel
# trace's duration): the configs[4] force pass, profiles/sph_c4_kernel_stats.md.  It is above
# VALU_PEAK_INSTS, so that figure is not the counter's ceiling.
VALU_MEASURED_INSTS = 7.63e11


def read_valu(kernel_pass: str):
    """VALU wave instructions per substep of a pass, from the committed rocprofv3 PMC summary
    (profiles/valu_c3.txt, lines `<pass> valu_insts=<N>`), or None."""
    f = REPO / "profiles" / "valu_c3.txt"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        parts = line.split()
        if len(parts) >= 2 and parts[0] == kernel_pass and parts[1].startswith("valu_insts="):
            return int(parts[1].split("=", 1)[1])
    return None


def copy_calibration(torch, log, mib: int = 1024) -> None:
    """A plain copy kernel of known size (reads and writes `mib` MiB each) for scaling the PMC
    FETCH_SIZE / WRITE_SIZE readings; run alone under rocprofv3 --pmc."""
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    log(f"copy calibration: 3 launches, {mib} MiB read + {mib} MiB written each")


def stream_ceiling(torch, log, mib: int = 1024, reps: int = 10) -> dict:
    """A STREAM-style copy ceiling measured on this GPU: `mib` MiB read and written by one
    device copy, median of `reps` with HIP events; GB/s counts the bytes read plus written."""
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        torch.mul(src, 1.0, out=dst)  # an elementwise kernel (a copy_ may go through DMA)
        b.record()
        b.synchronize()
        ts.append(a.elapsed_time(b))
    t = sorted(ts)[len(ts) // 2]
    gbs = 2 * mib * (1 << 20) / (t * 1e-3) / 1e9
    del src, dst
    torch.cuda.empty_cache()
    log(f"copy ceiling: {mib} MiB copy in {t:.3f} ms -> {gbs:.0f} GB/s")
    return {"GBs": gbs, "bytes": 2 * mib * (1 << 20), "ms": t, "reps": reps,
            "frac_of_hbm_peak": gbs / HBM_PEAK_GBS,
            "kernel": "torch.mul(src, 1.0, out=dst) over a 1 GiB float32 tensor: one elementwise "
                      "kernel, read + write counted (the copy kernel the PMC byte counters are "
                      "scaled by)"}


def cpu_info() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def build_fields(fh, cfg, torch):
    f = fh.FieldSet(cfg.n)
    for nm, a in (("pos_x", cfg.x), ("pos_y", cfg.y), ("pos_z", cfg.z)):
        f.f32_fields[nm] = torch.from_numpy(a).cuda()
    for nm in ("vel_x", "vel_y", "vel_z"):
        f.f32_fields[nm] = torch.zeros(cfg.n, dtype=torch.float32, device="cuda")
    f.add_f32_zeros("density", cfg.n)
    return f


def build_pipe(fh, cfg):
    p = fh.Pipeline()
    p.add(fh.SphFusedModule(cfg.h, cfg.cell_size, cfg.dims, cfg.mass, cfg.gas_constant,
                            cfg.rest_density, cfg.viscosity))
    p.add(fh.GravityModule(*cfg.gravity))
    p.add(fh.IntegrateModule())
    p.add(fh.BoxColliderModule(*cfg.box_min, *cfg.box_max, cfg.restitution))
    return p


def run_substeps(pipe, fields, ctx, dt, count: int, G: int) -> None:
    """`count` substeps: count // G replays of the captured G-substep graph, then the remainder as
    one eager fh_sph_fused_steps call (the same kernels)."""
    if count >= G:
        pipe.replay(count // G)
    if count % G:
        pipe.run_async(fields, dt, count % G)


def timed_trajectory(fh, torch, cfg, W: int, K: int, G: int, log):
    """A fresh dam-break field set: W untimed substeps, then exactly K timed substeps between
    synchronisations (wall clock and HIP events on the context stream).  Returns the fields,
    pipeline, context and the two times."""
    fields = build_fields(fh, cfg, torch)
    pipe = build_pipe(fh, cfg)
    ctx = fields.context(cfg.num_cells)
    torch.cuda.synchronize()
    pipe.capture(fields, cfg.dt, G)
    if W:
        run_substeps(pipe, fields, ctx, cfg.dt, W, G)
    ctx.sync()
    torch.cuda.synchronize()
    ctx.event_record(0)
    t0 = time.perf_counter()
    run_substeps(pipe, fields, ctx, cfg.dt, K, G)
    ctx.event_record(1)
    ctx.sync()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev_ms = ctx.event_elapsed_ms(0, 1)
    log(f"{cfg.name}: {W} warm-up + {K} timed substeps (graph of {G}): wall "
        f"{wall * 1e3:.2f} ms, events {ev_ms:.2f} ms")
    return fields, pipe, ctx, wall, ev_ms


def bench_sph(args, fh, torch, log):
    from forge_hip import workloads

    cfg = workloads.config3()
    C = cfg.num_cells
    _, passes = fh.RadixSorter.digit_layout(max(1, (C - 1).bit_length()), cfg.n)
    G = max(1, args.graph_substeps)
    K, W = max(1, args.steps), max(0, args.warmup)
    fields, pipe, ctx, wall, ev_ms = timed_trajectory(fh, torch, cfg, W, K, G, log)
    # The survey's c3 protocol (1000 substeps, mean of the last 900) as its own figure, on a
    # fresh trajectory, unless the arguments already are that protocol.
    if args.no_protocol:
        proto = None
    elif (W, K) == (100, 900):
        proto = {"warmup": W, "steps": K, "ms_per_step": wall * 1e3 / K,
                 "value": cfg.n * K / wall, "same_as_headline": True}
    else:
        _, _, _, pwall, _ = timed_trajectory(fh, torch, cfg, 100, 900, G, log)
        proto = {"warmup": 100, "steps": 900, "ms_per_step": pwall * 1e3 / 900,
                 "value": cfg.n * 900 / pwall, "same_as_headline": False}
    # Per-kernel durations: the G substeps of the graph once more, launched eagerly on the same
    # stream with every kernel bracketed by HIP events (events recorded by graph nodes cannot be
    # timed on HIP).
    for k in KERNELS + list(PASS_TIMERS.values()):
        ctx.time_kernel(k, (passes if k == "sort" else 1) * G)
    pipe.run_async(fields, cfg.dt, G)
    ctx.sync()
    kern = {}
    for k in KERNELS + list(PASS_TIMERS.values()):
        t = ctx.kernel_times_ms(k)
        kern[k] = {"launches": len(t), "mean_us": 1e3 * sum(t) / max(len(t), 1),
                   "per_substep_us": 1e3 * sum(t) / G}
        ctx.time_kernel(k, 0)
    byts = algorithmic_bytes(cfg.n, C, passes, G)
    pas = {}
    for p, ks in PASSES.items():
        # the neighbour passes are timed as a whole (wall time)
        us = kern[PASS_TIMERS[p]]["per_substep_us"] if p in PASS_TIMERS else \
            sum(kern[k]["per_substep_us"] for k in ks)
        pas[p] = {"kernels": ks, "per_substep_us": us,
                  "kernel_sum_us": sum(kern[k]["per_substep_us"] for k in ks),
                  "alg_bytes": byts[p],
                  "alg_GBs": byts[p] / (us * 1e-6) / 1e9 if us > 0 else None}
    dom = max(pas, key=lambda p: pas[p]["per_substep_us"])
    achieved = pas[dom]["alg_GBs"]
    total_alg = sum(byts.values())
    return dict(cfg=cfg, C=C, passes=passes, G=G, K=K, W=W, wall=wall, ev_ms=ev_ms, kern=kern,
                pas=pas, dom=dom, achieved=achieved, total_alg=total_alg, digest=cfg.digest(),
                proto=proto)


def bench_sph_c0(args, fh, torch, log):
    """configs[0] (50,000 particles, the scale of the reference's published dam-break figure)
    as a throughput line: 100 warm-up substeps, then 2000 timed, graph of 10."""
    from forge_hip import workloads

    cfg = workloads.config0()
    W, K, G = 100, 2000, 10
    _, _, ctx, wall, ev_ms = timed_trajectory(fh, torch, cfg, W, K, G, log)
    return {"workload": "c0: SPH dam-break substep, 50,000 particles, h = cell = 0.025, 40^3 "
                        "cells, re-hash + sort every substep, hipGraph of 10 substeps",
            "warmup": W, "steps": K, "ms_per_step": wall * 1e3 / K,
            "particle_steps_per_s": cfg.n * K / wall, "substep_us_events": ev_ms * 1e3 / K,
            "input_sha256": cfg.digest(),
            "reference_published": {"value": 2.22e8, "hardware": "NVIDIA L40",
                                    "source": "ROADMAP.md:263 (50K particles, its own "
                                              "random-init manifest; context only)"}}


def time_sort(args, fh, torch, log, keys, vals, label):
    """Median of whole 32-bit fh_sort_pairs calls on (keys, vals) with HIP events, and the
    per-pass durations of further calls with every kernel bracketed by events."""
    n = keys.size
    ctx = fh.Context(max_n=n, max_cells=1)
    k0, v0 = fh.from_u32(keys), fh.from_u32(vals)
    k, v = k0.clone(), v0.clone()
    sorter = fh.RadixSorter(n, ctx=ctx)
    torch.cuda.synchronize()
    for _ in range(2):
        k.copy_(k0)
        v.copy_(v0)
        sorter.sort(k, v, n, 32)
    times = []
    reps = args.sort_reps
    for _ in range(reps):  # whole sorts, no per-kernel events in between
        k.copy_(k0)
        v.copy_(v0)
        ctx.torch_stream().wait_stream(torch.cuda.current_stream())
        # A ~100 us device-side delay ahead of the timed region, so that all the sort's launches
        # are queued before the device reaches it: the events time device execution, not the
        # host's launch rate (an eager call's 7 launches otherwise leave the device idle for
        # 10-30 us while the host catches up).
        with torch.cuda.stream(ctx.torch_stream()):
            torch.cuda._sleep(200_000)
        ctx.event_record(2)
        sorter.sort(k, v, n, 32, sync=False)
        ctx.event_record(3)
        times.append(ctx.event_elapsed_ms(2, 3))
    ctx.time_kernel("sort", 4 * reps)
    ctx.time_kernel("hist", reps)
    for _ in range(reps):
        k.copy_(k0)
        v.copy_(v0)
        ctx.torch_stream().wait_stream(torch.cuda.current_stream())
        sorter.sort(k, v, n, 32, sync=False)
        ctx.sync()  # the next copy_ must not overlap this sort
    passes_ms = ctx.kernel_times_ms("sort")
    hist_ms = ctx.kernel_times_ms("hist")
    # The device's pass plan (fh_sort_plan, bit p: pass p moved keys; a pass whose digit is
    # equal for every key returns at once: c1's top byte is always 0, so 3 of the 4 passes move
    # keys).  The timed launches are the 4 passes of each sort in order.
    plan = ctx.sort_plan()
    ctx.close()
    t = sorted(times)[len(times) // 2]
    moving = [x for q, x in enumerate(passes_ms) if (plan >> (q % 4)) & 1]
    mp = bin(plan & 0xF).count("1")
    pass_us = 1e3 * sum(moving) / max(len(moving), 1)
    moved = (4 + 16 * mp) * n
    out = {
        "workload": label,
        "median_ms": t, "gkeys_per_s": n / (t * 1e-3) / 1e9,
        # the survey's formula: a key read for the histograms + 4 passes reading and writing
        # (key, value), whether or not a pass moves anything
        "alg_bytes": 68 * n, "alg_GBs": 68 * n / (t * 1e-3) / 1e9,
        "frac_of_hbm_peak": 68 * n / (t * 1e-3) / 1e9 / HBM_PEAK_GBS,
        # the bytes actually moved: the histogram read + the passes that move keys
        "moving_passes_per_sort": mp, "pass_plan": plan,
        "moved_bytes": moved, "moved_GBs": moved / (t * 1e-3) / 1e9,
        "moved_frac_of_hbm_peak": moved / (t * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "onesweep_pass_mean_us": pass_us,
        "onesweep_pass_GBs": 16 * n / (pass_us * 1e-6) / 1e9,
        "hist_mean_us": 1e3 * sum(hist_ms) / max(len(hist_ms), 1),
        "reps": reps,
    }
    log(f"sort {label[:40]}: median {t:.3f} ms, {out['gkeys_per_s']:.2f} Gkeys/s, "
        f"{mp} moving passes, moved {out['moved_frac_of_hbm_peak']:.3f} of HBM peak")
    return out


def bench_sort(args, fh, torch, log):
    """configs[1] (keys < 2^24: the top byte is 0, so 3 of the 4 passes move data), and the same
    count of full-entropy 32-bit keys (all 4 passes move data)."""
    from forge_hip import workloads

    keys, vals = workloads.config1()
    out = time_sort(args, fh, torch, log, keys, vals,
                    "c1: 16,777,216 (u32 cell key, u32 index) pairs, 32-bit stable LSD sort")
    full = workloads.u32_stream(workloads.DEFAULT_SEED, 7, keys.size)
    out["full_entropy"] = time_sort(args, fh, torch, log, full, vals,
                                    "16,777,216 uniformly random u32 keys (all 4 passes move "
                                    "data), u32 index values, 32-bit stable LSD sort")
    return out


def sort_bytes(n: int, bits: int) -> int:
    """B_sort(N, bits) = N (4 + 16 ceil(bits / 8)): one key read for the all-digit histogram,
    then a read and write of (key, value) per 8-bit pass."""
    return n * (4 + 16 * ((bits + 7) // 8))


def bench_query_c2(args, fh, torch, log):
    """HashGrid build + 3x3x3 neighbour query (counts and poly6 weight sums) of
    4,194,304 uniform points, r = cell = 0.0122, 82^3 cells.  Each leg is timed with HIP
    events around `reps` back-to-back calls on the context stream."""
    from forge_hip import _lib, workloads
    from forge_hip._lib import check, f3, u3
    from forge_hip.runtime import ptr, u32_empty

    c = workloads.config2()
    n = c["n"]
    C = c["dims"][0] * c["dims"][1] * c["dims"][2]
    ctx = fh.Context(max_n=n, max_cells=C)
    grid = fh.HashGrid(c["cell_size"], c["dims"], c["origin"], n, ctx=ctx)
    P = tuple(torch.from_numpy(c[a]).cuda() for a in "xyz")
    counts = u32_empty(n, P[0].device)
    wsum = torch.empty(n, dtype=torch.float32, device=P[0].device)
    torch.cuda.synchronize()
    lib = _lib.load()
    bargs = (ctx.handle, ptr(P[0]), ptr(P[1]), ptr(P[2]), 1, n, grid.cell_size, f3(grid.origin),
             u3(grid.dims), ptr(grid.cell_start), ptr(grid.sorted_indices),
             ptr(grid.cell_indices))
    qargs = (ctx.handle, ptr(P[0]), ptr(P[1]), ptr(P[2]), 1, n, grid.cell_size, f3(grid.origin),
             u3(grid.dims), ptr(grid.cell_start), ptr(grid.sorted_indices), float(c["radius"]),
             ptr(counts), ptr(wsum))
    reps = max(args.sort_reps, 1)
    check(lib.fh_hashgrid_build(*bargs))
    check(lib.fh_neighbor_query(*qargs))
    ctx.sync()
    ctx.event_record(4)
    for _ in range(reps):
        check(lib.fh_hashgrid_build(*bargs))
    ctx.event_record(5)
    for _ in range(reps):
        check(lib.fh_neighbor_query(*qargs))
    ctx.event_record(6)
    ctx.sync()
    build_ms = ctx.event_elapsed_ms(4, 5) / reps
    query_ms = ctx.event_elapsed_ms(5, 6) / reps
    mean_count = float(counts.double().mean().item())
    ctx.close()
    bits = max(1, (C - 1).bit_length())
    b_build = 20 * n + sort_bytes(n, bits) + 4 * n + 8 * C
    b_query = 28 * n + 8 * C
    out = {
        "workload": "c2: HashGrid build + 3x3x3 neighbour query, 4,194,304 uniform points, "
                    "r = cell = 0.0122, 82^3 cells",
        "build_ms": build_ms, "query_ms": query_ms,
        "points_per_s": n / ((build_ms + query_ms) * 1e-3),
        "mean_neighbours": mean_count,
        "build_alg_bytes": b_build, "build_alg_GBs": b_build / (build_ms * 1e-3) / 1e9,
        "query_alg_bytes": b_query, "query_alg_GBs": b_query / (query_ms * 1e-3) / 1e9,
        "query_frac_of_hbm_peak": b_query / (query_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "reps": reps,
    }
    log(f"c2: build {build_ms:.3f} ms, query {query_ms:.3f} ms")
    return out


def candidate_tests(x, y, z, cs, dims):
    """Pair candidates of one neighbour pass: sum over particles of the occupancy of their
    clamped 3x3x3 cell neighbourhood."""
    import numpy as np

    nx, ny, nz = dims
    c = [np.clip(np.floor(a / np.float32(cs)).astype(np.int64), 0, d - 1)
         for a, d in ((x, nx), (y, ny), (z, nz))]
    occ = np.bincount(c[0] + nx * (c[1] + ny * c[2]), minlength=nx * ny * nz)
    o3 = occ.reshape(nz, ny, nx)
    p = np.pad(o3, 1)
    s = np.zeros_like(o3)
    for a in range(3):
        for b in range(3):
            for d in range(3):
                s += p[a:a + nz, b:b + ny, d:d + nx]
    return int((o3 * s).sum()), occ


def bench_sph_c4(args, fh, torch, log):
    """one HashGrid build + SPH density + pressure/viscosity pass over 8,388,608
    particles of 64 Gaussian clumps + 10 % uniform background (load-imbalance stress); the
    fused module alone (rebuild, density, force), timed with HIP events over `reps` calls."""
    import numpy as np
    from forge_hip import workloads

    cfg = workloads.config4()
    f = build_fields(fh, cfg, torch)
    p = fh.Pipeline()
    p.add(fh.SphFusedModule(cfg.h, cfg.cell_size, cfg.dims, cfg.mass, cfg.gas_constant,
                            cfg.rest_density, cfg.viscosity))
    ctx = f.context(cfg.num_cells)
    # c4's dense clumps make long heavy items: 8 wavefronts per heavy item instead of 4 (~9 %),
    # cells ordered by 8 sub-cells per axis, so that heavy items skip far candidates (~36 %),
    # items split above 384 candidates per particle rather than the default 192 (~1.5 %), and a
    # partial-sum slot for every item (most of c4's items are heavy; the default has one per 8)
    ctx.set_option(fh.FH_OPT_HEAVY_PARTS, 8)
    ctx.set_option(fh.FH_OPT_SUBCELL, 8)
    ctx.set_option(fh.FH_OPT_HEAVY_WORK, 384)
    ctx.set_option(fh.FH_OPT_HEAVY_SLOTS, 2**31 - 1)
    torch.cuda.synchronize()
    p.step(f, cfg.dt)  # warm-up (positions do not move: every call is the same workload)
    reps = 3
    ctx.event_record(7)
    for _ in range(reps):
        p.step_async(f, cfg.dt)
    ctx.event_record(8)
    ctx.sync()
    ms = ctx.event_elapsed_ms(7, 8) / reps
    ks = ["density", "force"]
    for k in ks:
        ctx.time_kernel(k, 1)
    p.step_async(f, cfg.dt)
    ctx.sync()
    kt = {k: 1e3 * sum(ctx.kernel_times_ms(k)) for k in ks}
    for k in ks:
        ctx.time_kernel(k, 0)
    cand, occ = candidate_tests(cfg.x, cfg.y, cfg.z, cfg.cell_size, cfg.dims)
    nz = occ[occ > 0]
    out = {
        "workload": "c4: 8,388,608 particles (64 Gaussian clumps + 10 % uniform), h = cell = "
                    "0.01, 100^3 cells: one grid build + density + fused force pass",
        "ms": ms, "particles_per_s": cfg.n / (ms * 1e-3),
        "candidate_tests_per_pass": cand,
        "candidate_tests_per_s": 2 * cand / (ms * 1e-3),
        "occupancy_max": int(occ.max()), "occupancy_p99_nonempty": float(np.percentile(nz, 99)),
        "kernels_us": {k: round(v, 1) for k, v in kt.items()},
        "heavy_parts": 8, "subcells_per_axis": 8, "heavy_work": 384, "heavy_slots": "every item", "reps": reps,
        "input_sha256": cfg.digest(),
    }
    log(f"c4: {ms:.2f} ms per build + density + force, max occupancy {occ.max()}")
    return out


def cpu_baseline(args, log):
    import numpy as np

    import oracle.oracle as O
    from forge_hip import workloads

    cfg = workloads.config3()
    prm = O.sph_params(cfg.h, cfg.cell_size, cfg.dims, cfg.mass, cfg.gas_constant,
                       cfg.rest_density, cfg.viscosity)
    z = np.zeros(cfg.n, np.float32)
    state = [cfg.x, cfg.y, cfg.z, z, z, z]
    steps = 0
    t0 = time.perf_counter()
    while True:
        r = O.sph_step(prm, 7, cfg.gravity, cfg.box_min, cfg.box_max, cfg.restitution,
                       *state, cfg.dt)
        state = list(r[:6])
        steps += 1
        el = time.perf_counter() - t0
        if el >= args.cpu_seconds or steps >= 50:
            break
    log(f"cpu baseline: {steps} substeps in {el:.2f} s")
    return {"value": cfg.n * steps / el, "unit": "particle-steps/s", "cores": 1, "kind": "port",
            "sample": f"{steps} consecutive substeps of configs[3] (1,048,576 particles) through "
                      f"oracle/oracle.c or_sph_step (single-threaded C, -O2 -ffp-contract=off)",
            "seconds": el, "cpu": cpu_info(), "host_cpus": os.cpu_count()}


def valu_block(insts, us):
    if not insts or not us:
        return None
    return {"insts_per_launch": insts, "peak_insts_per_s": VALU_PEAK_INSTS,
            "achieved_insts_per_s": insts / (us * 1e-6),
            "frac": insts / (us * 1e-6) / VALU_PEAK_INSTS,
            "measured_ceiling_insts_per_s": VALU_MEASURED_INSTS,
            "frac_of_measured_ceiling": insts / (us * 1e-6) / VALU_MEASURED_INSTS,
            "source": "profiles/valu_c3.txt"}


# Survey bytes per particle of each neighbour pass: density reads the
# sorted float4 positions and writes rho (20 B); force + epilogue read two float4 records and
# write the new position, velocity and index (60 B).
SURVEY_PASS_BYTES = {"density": 20, "force": 60}


def roofline_block(s, dom, n, stream):
    """The dominant pass against the HBM roofline (algorithmic bytes / its measured time), with
    the survey's byte count beside the builder's, the measured HBM traffic, the copy ceiling
    measured on this GPU, and the VALU issue fraction; `bound` names the resource closest to
    its limit."""
    p = s["pas"][dom]
    us = p["per_substep_us"]
    traffic = read_traffic(dom)
    valu = valu_block(read_valu(dom), us)
    frac = s["achieved"] / HBM_PEAK_GBS
    dram_frac = traffic / (us * 1e-6) / 1e9 / HBM_PEAK_GBS if traffic and us else None
    hbm_frac = max(frac, dram_frac or 0.0)
    bound = "valu" if valu and valu["frac"] > hbm_frac else "hbm"
    sb = SURVEY_PASS_BYTES.get(dom)
    out = {
        "bound": bound, "kernel": dom + " pass (" + " + ".join(p["kernels"]) + ")",
        "achieved": s["achieved"], "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": frac,
        "traffic": traffic,
        "alg_bytes_per_launch": p["alg_bytes"], "mean_launch_us": us,
        # the survey's per-particle bytes for the same pass
        "survey_bytes_per_launch": sb * n if sb else None,
        "survey_frac": sb * n / (us * 1e-6) / 1e9 / HBM_PEAK_GBS if sb and us else None,
        "dram_frac": dram_frac,
        # the SPH passes are limited by vector ALU issue, not HBM: VALU wave instructions of
        # the pass (PMC, profiles/valu_c3.txt) over the time measured here, against the issue
        # rate of 256 CUs at 2.4 GHz
        "valu": valu,
    }
    if stream:
        out["stream_ceiling_GBs"] = stream["GBs"]
        out["frac_of_stream_ceiling"] = s["achieved"] / stream["GBs"]
        out["stream_ceiling"] = stream
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=900)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--graph-substeps", type=int, default=10)
    ap.add_argument("--sort-reps", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-protocol", action="store_true",
                    help="skip the separate 1000-substep c3 protocol run (for profiling)")
    ap.add_argument("--no-sort", action="store_true", help="skip the c1 sort line")
    ap.add_argument("--no-extra-configs", action="store_true",
                    help="skip the c2 (grid build + query) and c4 (skewed SPH pass) lines")
    ap.add_argument("--no-stream", action="store_true", help="skip the copy-ceiling measurement")
    ap.add_argument("--quiet", action="store_true")
    ap.add_argument("--sort-only", action="store_true",
                    help="only the c1 sort line (for a profile of the sort alone)")
    ap.add_argument("--only", choices=["c0", "c1", "c2", "c4"],
                    help="only that configuration's line (for a profile of it alone)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB copy kernel (scale for PMC byte counters)")
    args = ap.parse_args(argv)

    def log(msg):
        if not args.quiet:
            print(f"[bench] {msg}", file=sys.stderr, flush=True)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (every GPU box "
              "here has one GPU); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    import forge_hip as fh

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 1
    if args.copy_calibration:
        copy_calibration(torch, log)
        return 0
    fh.load()
    log(f"device {torch.cuda.get_device_name(0)}")
    if args.sort_only:
        args.only = "c1"
    if args.only:
        fn = {"c0": bench_sph_c0, "c1": bench_sort, "c2": bench_query_c2, "c4": bench_sph_c4}
        print(json.dumps({"metric": METRIC, "only": args.only,
                          "result": fn[args.only](args, fh, torch, log)}), flush=True)
        return 0
    stream = None if args.no_stream else stream_ceiling(torch, log)
    s = bench_sph(args, fh, torch, log)
    c0 = None if args.no_extra_configs else bench_sph_c0(args, fh, torch, log)
    sort = None if args.no_sort else bench_sort(args, fh, torch, log)
    q2 = None if args.no_extra_configs else bench_query_c2(args, fh, torch, log)
    s4 = None if args.no_extra_configs else bench_sph_c4(args, fh, torch, log)
    cpu = None if args.no_cpu else cpu_baseline(args, log)

    cfg, K = s["cfg"], s["K"]
    ms_per_step = s["wall"] * 1e3 / K
    value = cfg.n * K / s["wall"]
    dom = s["dom"]
    kern = s["kern"]
    line = {
        "metric": METRIC,
        "value": value,
        "unit": "particle-steps/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": s["W"],
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "configs[3]: SPH dam-break substep, 1,048,576 particles, h = cell = 0.01, "
                        "100^3 cells, re-hash + sort every substep, hipGraph of "
                        f"{s['G']} substeps (one fh_sph_fused_steps call: state resident in "
                        "sorted order between them, fields written after the last); "
                        f"{s['W']} warm-up substeps, then {K} timed",
            "particles": cfg.n, "cells": s["C"], "sort_passes": s["passes"],
            "graph_substeps": s["G"], "input_sha256": s["digest"], "parallelism": "single GPU",
        },
        "roofline": roofline_block(s, dom, cfg.n, stream),
        "cpu_baseline": cpu,
        "extra": {
            "c3_protocol_last_900_of_1000": s["proto"],
            "substep_us_events": s["ev_ms"] * 1e3 / K,
            "substep_alg_bytes": s["total_alg"],
            "substep_alg_GBs": s["total_alg"] / (ms_per_step * 1e-3) / 1e9,
            "substep_survey_bytes": survey_step_bytes(cfg.n, s["C"], s["passes"]),
            "substep_survey_frac": survey_step_bytes(cfg.n, s["C"], s["passes"])
            / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "kernels": {k: {q: (round(v, 3) if isinstance(v, float) else v) for q, v in kern[k].items()}
                        for k in KERNELS},
            "passes": {p: {q: (round(v, 3) if isinstance(v, float) else v) for q, v in d.items()}
                       for p, d in s["pas"].items()},
            "sph_c0": c0,
            "sort_c1": sort,
            "query_c2": q2,
            "sph_c4": s4,
        },
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
