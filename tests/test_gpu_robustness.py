"""Failure handling and long-run state, forced from the host (no fault, no hang):

* epoch renewal: the rebuilds' work tags compare a 30-bit epoch that every start bumps, so a tag
  2^30 - 1 starts old would match again; the context renews (clears the tags, restarts the
  epoch) before its count of queued starts -- graph replays included -- reaches the period.
  With a period of a few starts the epochs cycle within the test, so a renewal that failed to
  clear a tag would alias a stale one (a skipped sub-tile, a stale group or cell run) and change
  the results; they must equal those of the default period bit for bit, and the renewal kernel
  must have run;
* a radix-sort look-back that gives up (FH_OPT_SPIN_LIMIT = 1: one poll) is reported by fh_sync
  as FH_ESTATE instead of passing silently, and the context sorts correctly afterwards.
"""
import numpy as np
import pytest
import torch

from test_gpu_sph import colocated_cfg, fields_from, sph_pipeline

pytestmark = pytest.mark.gpu


def _run_sph(fh, cfg, vel, period):
    f = fields_from(fh, cfg, vel)
    ctx = f.context(cfg.num_cells)
    ctx.set_option(fh.FH_OPT_EPOCH_PERIOD, period)
    ctx.time_kernel("epoch_reset", 1000)
    p = sph_pipeline(fh, cfg)
    p.resident = True
    torch.cuda.synchronize()
    p.run(f, cfg.dt, 7)             # one resident call: 7 starts
    p.step(f, cfg.dt)               # one eager substep
    p.capture(f, cfg.dt, 4)         # a graph of 4 resident substeps ...
    for _ in range(3):
        p.replay(1)                 # ... replayed with a sync in between
        ctx.sync()
    resets = len(ctx.kernel_times_ms("epoch_reset"))
    ctx.time_kernel("epoch_reset", 0)
    ctx.set_option(fh.FH_OPT_EPOCH_PERIOD, 0)
    return {k: t.cpu().numpy() for k, t in f.f32_fields.items()}, resets


def _expected_renewals(period, calls):
    """The host's renewal rule: before a start (or a replay of G starts) that would take the
    count past the period, renew and restart the count."""
    begins = renewals = 0
    for kind, k in calls:
        if kind == "start":
            for _ in range(k):
                if begins + 1 > period:
                    renewals, begins = renewals + 1, 0
                begins += 1
        else:
            if begins + k > period:
                renewals, begins = renewals + 1, 0
            begins += k
    return renewals


@pytest.mark.parametrize("period", [1, 3, 5])
def test_epoch_renewal_keeps_sph_results(fh, gpu_ctx, period):
    """Co-located groups (group tags, skipped sub-tiles, candidate cells) stepped 20 times:
    7 resident substeps, 1 eager one and 3 replays of a 4-substep graph, with renewals every
    `period` starts against the default period."""
    cfg, vel = colocated_cfg(seed=41)
    print(f"epoch renewal: period {period}", flush=True)
    ref, r0 = _run_sph(fh, cfg, vel, 0)
    got, r1 = _run_sph(fh, cfg, vel, period)
    assert r0 == 0
    assert r1 == _expected_renewals(period, [("start", 7), ("start", 1), ("replay", 4),
                                             ("replay", 4), ("replay", 4)]), r1
    for k in ref:
        assert np.array_equal(ref[k], got[k]), k


def test_epoch_renewal_keeps_hashgrid_builds(fh, gpu_ctx, oracle):
    """fh_hashgrid_build (each build is a start) on 6 point sets in a context renewing every 2
    starts, against the oracle: the renewals run between builds and change nothing."""
    ctx = fh.Context(max_n=50_000, max_cells=40 ** 3)
    ctx.set_option(fh.FH_OPT_EPOCH_PERIOD, 2)
    ctx.time_kernel("epoch_reset", 100)
    rng = np.random.default_rng(3)
    for t in range(6):
        n = 50_000 - 7_000 * t
        p = rng.uniform(0, 1, (n, 3)).astype(np.float32)
        p[: n // 4] = p[: n // 4] * np.float32(0.05)  # dense corner cells: long runs
        grid = fh.HashGrid(0.025, (40, 40, 40), (0, 0, 0), n, ctx=ctx)
        grid.build(torch.from_numpy(p).cuda())
        ocs, osi, oci = oracle.hashgrid_build(p[:, 0], p[:, 1], p[:, 2], 0.025, (0, 0, 0),
                                              (40, 40, 40))
        assert np.array_equal(fh.to_u32(grid.cell_start), ocs), t
        assert np.array_equal(fh.to_u32(grid.sorted_indices)[:n], osi), t
        assert np.array_equal(fh.to_u32(grid.cell_indices)[:n], oci), t
    assert len(ctx.kernel_times_ms("epoch_reset")) >= 2
    ctx.close()


def test_epoch_period_option(fh, gpu_ctx):
    for v in (0, 1, 1000, 2 ** 30 - 2):
        gpu_ctx.set_option(fh.FH_OPT_EPOCH_PERIOD, v)
    for bad in (-1, 2 ** 30 - 1, 2 ** 31 - 1):
        with pytest.raises(fh.ForgeError):
            gpu_ctx.set_option(fh.FH_OPT_EPOCH_PERIOD, bad)
    gpu_ctx.set_option(fh.FH_OPT_EPOCH_PERIOD, 0)


def test_lookback_failure_is_reported_by_sync(fh, gpu_ctx):
    """With one poll allowed, the look-backs of a 1,048,576-pair 32-bit sort give up: fh_sync
    reports it (FH_ESTATE) instead of FH_OK.  The scatter stays in bounds, so nothing faults;
    with the default limit restored the same context sorts correctly."""
    n = 1_048_576
    ctx = fh.Context(max_n=n, max_cells=1)
    rng = np.random.default_rng(12)
    keys = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)
    vals = np.arange(n, dtype=np.uint32)
    sorter = fh.RadixSorter(n, ctx=ctx)
    ctx.set_option(fh.FH_OPT_SPIN_LIMIT, 1)
    k, v = fh.from_u32(keys), fh.from_u32(vals)
    torch.cuda.synchronize()
    print("look-back failure forced: spin limit 1", flush=True)
    sorter.sort(k, v, n, 32, sync=False)
    with pytest.raises(fh.ForgeError) as ei:
        ctx.sync()
    assert ei.value.code == fh.FH_ESTATE and "look-back" in ei.value.message
    ctx.sync()  # reported once
    ctx.set_option(fh.FH_OPT_SPIN_LIMIT, 0)
    k, v = fh.from_u32(keys), fh.from_u32(vals)
    torch.cuda.synchronize()
    sorter.sort(k, v, n, 32)
    order = np.argsort(keys, kind="stable")
    assert np.array_equal(fh.to_u32(k), keys[order])
    assert np.array_equal(fh.to_u32(v), vals[order])
    ctx.close()
