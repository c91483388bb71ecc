"""bench.py -- one JSON line for the MI355X preemptible persistent GEMM.

Workload ("tile calibration"): persistent fp32 SGEMM
M=N=K=4096, 128x128 output tiles (MFMA128 engine), per-tile K chunk 32, one
worker per CU slot, no yields. A step is one full pass of the worker pool over
the 1024 output tiles; inputs are resident in HBM before the timed region.
`value` is whole-job GEMM throughput in TFLOP/s.

Also reported (same line): the roofline of the GEMM kernel (fp32 MFMA dense
peak 157.3 TFLOP/s; per-launch duration from HIP events on the launch stream),
the engine clock the launches ran at (device-side probe; the timed steps follow
an untimed pre-warm of back-to-back launches, --prewarm-ms, because the clock
climbs from its idle level over about a second of load), and the CPU
baseline: the reference's float64 host GEMM (i-k-j, src/persistent.cu:221-227,
restated in oracle/) timed on this host -- the whole GEMM with OpenMP on the
host threads this process may use, and a 1024-row sample on one thread -- whose
result also checks the whole GPU C.

The same line carries `preemption`: the cfg3 experiment (background fp32
SGEMM M=N=8192, K=4096, 128x128 tiles, k-chunk 128, on all 256 CUs; urgent
fp32 GEMM 256x256x256 at exponential arrivals, mean 2 ms) run by the
product binaries, 10,000 arrivals for every latency -- cooperative yield
latency at k-stage and tile-boundary polls (flag set -> last block observes,
the reference's latency), the retreat arm (one background job; flag raised ->
urgent GEMM starts on its own stream), the no-preemption baseline, the polling
overhead (ABAB drains) and the tile time at full residency they are measured
against, and the same latencies with the tile taken as a 32- and a 64-deep
k-chunk (`by_k_chunk`) -- and `bf16`: the cfg5 bf16 MFMA GEMM throughput
(M=N=K=8192, 256x256 tiles, no yields) with its engine clock: right after the preemption
runs (`tflops`, the poll-off preemptible kernel over two GEMMs), and
sustained (one GEMM per launch after a pre-warm of the same launches), beside
torch.matmul (hipBLASLt) on the same operands under the same conditions (the
sustained bf16 clock is set by the load on the whole chip; `--bf16-sweep`
times the GEMM on 64-256 workers), the retreat arm on the bf16 background
(10,000 arrivals; retreating tiles re-queued from k = 0), and cfg5 at 1, 2
and 4 blocks per CU (`occupancy`: each occupancy's tile, its throughput and
its cooperative stage-poll latency in k-chunk times).

Usage: python bench.py [--gpus 1] [--steps 10] [--warmup 3] [--no-preempt]
"""
import argparse
import json
import os
import re
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = ("urgent-task preempt latency p50/p99 (us); persistent GEMM TFLOP/s; "
          "yield overhead %")
PEAK_FP32_TF = 157.3


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def host_threads():
    """Threads for the all-core host baseline: the CPU share this process may
    use (OMP_NUM_THREADS when set, else the affinity mask)."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    return len(os.sched_getaffinity(0))


def cpu_baseline(A_host, B_host, C_gpu, rows_1t):
    """The reference's float64 host GEMM (i-k-j, src/persistent.cu:221-227,
    restated in oracle/) on this host: the whole GEMM on every host thread
    (OpenMP over rows), and rows 0..rows_1t-1 on one thread as the reference
    runs it. The all-core result checks the whole GPU C."""
    import oracle
    M, K = A_host.shape
    N = B_host.shape[1]
    threads = host_threads()
    t0 = time.perf_counter()
    ref = oracle.gemm_f64(A_host, B_host, threads=threads)
    dt_all = time.perf_counter() - t0
    t0 = time.perf_counter()
    ref1 = oracle.gemm_f64_rows(A_host, B_host, 0, rows_1t)
    dt_1 = time.perf_counter() - t0
    assert (ref1 == ref[:rows_1t]).all(), "float64 rows differ between thread counts"
    frob = oracle.rel_frobenius(C_gpu, ref)
    return {
        "value": 2.0 * M * N * K / dt_all / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"the whole {M}x{N}x{K} GEMM in float64, i-k-j order "
                   f"(src/persistent.cu:221-227), OpenMP over rows on {threads} host threads, "
                   f"{dt_all:.1f} s"),
        "host_cores": os.cpu_count(),
        "single_thread": {
            "value": 2.0 * rows_1t * N * K / dt_1 / 1e12, "unit": "TFLOP/s", "cores": 1,
            "sample": f"rows 0..{rows_1t - 1} of the same GEMM, 1 thread, {dt_1:.1f} s"},
        "seconds": dt_all + dt_1,
    }, frob


def clock_summary(raw, wall_mhz):
    """Engine clock from apk_clock_probe records (cycles, ticks, xcd, start)."""
    import numpy as np
    r = raw.reshape(-1, 4)
    ok = r[:, 1] > 0
    mhz = r[ok, 0] / r[ok, 1] * wall_mhz
    per_xcd = {}
    for x, f in zip(r[ok, 2], mhz):
        per_xcd.setdefault(int(x), []).append(float(f))
    return {"mean": round(float(mhz.mean()), 1), "min": round(float(mhz.min()), 1),
            "max": round(float(mhz.max()), 1),
            "per_xcd": {str(k): round(float(np.mean(v)), 1) for k, v in sorted(per_xcd.items())},
            "probes": int(ok.sum())}


def measured_traffic(profile="profiles/persistent_gemm_mfma128_cfg2.md"):
    """HBM-side bytes per launch of the GEMM kernel as measured by the two
    rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE, scaled by a plain copy) and
    recorded in the profile summary; None if not recorded."""
    path = os.path.join(ROOT, profile)
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":")[1])
    return None


BIN = os.path.join(ROOT, "apk_amd", "bin")
# cfg3: background 8192x8192 (64x64 tiles of 128), K=4096 in k-chunks of 128,
# one pass over the grid per trial; urgent 256x256x256 on 4 workers.
CFG3 = ["--engine", "mfma128", "--tiles-m", "64", "--tiles-n", "64", "--gemm-k", "4096",
        "--k", "128"]
CFG3_URGENT = ["--urgent-m", "256", "--urgent-n", "256", "--urgent-k", "256"]


def run_bin(name, args, timeout=300):
    """Run a product binary (apk_amd/bin) and return its stdout; its exit
    status must be 0 (every binary checks its own results)."""
    cmd = [os.path.join(BIN, name)] + [str(a) for a in args]
    log(f"$ apk_amd/bin/{name} " + " ".join(cmd[1:]))
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    if r.returncode != 0:
        raise RuntimeError(f"{name} exited {r.returncode}:\n{r.stdout[-2000:]}\n{r.stderr[-2000:]}")
    return r.stdout


def grab(text, pattern, cast=float):
    m = re.search(pattern, text)
    if not m:
        raise RuntimeError(f"pattern {pattern!r} not found in:\n{text[-2000:]}")
    return tuple(cast(g) for g in m.groups())


def preemption_metrics(events, trials):
    """cfg3 preemption figures from the product binaries (see module doc)."""
    out = {"workload": ("cfg3: bg fp32 SGEMM M=N=8192 K=4096, 128x128 tiles, k-chunk 128, "
                        "256 workers (1/CU); urgent fp32 GEMM 256x256x256; exponential "
                        "arrivals, mean 2 ms, seed 21")}
    # Polling overhead (ABAB drains, medians): flag sampled at tile (k-chunk)
    # boundaries, and at every k-stage; the tile time from the poll-off drain.
    ovh = {}
    for poll in ("chunk", "stage"):
        t = run_bin("yield", ["--mode", "overhead"] + CFG3 + ["--tasks", 4096, "--reps", 6,
                                                               "--poll", poll])
        on_ms, = grab(t, r"poll ON : ([\d.]+) ms")
        off_ms, = grab(t, r"poll OFF: ([\d.]+) ms")
        pct, = grab(t, r"polling overhead: ([-\d.]+)%")
        ovh[poll] = (pct, on_ms, off_ms)
    # 4096 tasks of 32 k-chunks each over 256 workers: chunk time per worker.
    tile_us = min(ovh["chunk"][2], ovh["stage"][2]) * 1e3 * 256 / 4096 / 32
    out["tile_us_full_residency"] = round(tile_us, 3)
    out["overhead_pct"] = {"tile_boundary": ovh["chunk"][0], "k_stage": ovh["stage"][0]}
    # Cooperative yield: set -> last block observes (the reference's
    # latency); urgent e2e. Flag polled at every k-stage, and at tile
    # boundaries only.
    for poll, key in (("stage", "coop"), ("chunk", "coop_tile_boundary")):
        # 100 more arrivals than reported: the first 100 are warm-up (discarded)
        lat = run_bin("yield", ["--mode", "latency"] + CFG3 + CFG3_URGENT +
                      ["--poll", poll, "--arrival", "exp", "--mean-gap-us", 2000,
                       "--events", events + 100], timeout=600)
        p50, p90, p99 = grab(lat, r"preemption latency set->last \(us\): p50 ([\d.]+) \| "
                                  r"p90 ([\d.]+) \| p99 ([\d.]+)")
        e50, e99 = grab(lat, r"urgent e2e set->done \(us\): p50 ([\d.]+) \| p99 ([\d.]+)")
        n_ev, = grab(lat, r"blocks\): (\d+) events \(", int)
        out[key + "_latency_us"] = {"p50": p50, "p99": p99, "events": n_ev,
                                    "p50_over_tile": round(p50 / tile_us, 3)}
        out[key + "_urgent_e2e_us"] = {"p50": e50, "p99": e99}
    # Retreat arm: CUs handed to the urgent GEMM on its own stream. One
    # background job on all workers; the host raises each arrival as it falls
    # due; accumulator-only checkpoints (the live stages are re-fetched).
    rt = run_bin("urgent_baseline", CFG3 + CFG3_URGENT +
                 ["--bg-tasks", 4096, "--urgent-blocks", 4, "--arrival", "exp",
                  "--mean-gap-us", 2000, "--yield", 1, "--retreat", 4, "--oracle", 1,
                  "--continuous", 1, "--events", events, "--resume", "acc"], timeout=600)
    r50, r99 = grab(rt, r"flag raised -> urgent GEMM starts \(us\): p50 ([\d.]+) \| "
                        r"p90 [\d.]+ \| p99 ([\d.]+)")
    n_in, = grab(rt, r"continuous retreat arm: (\d+) arrivals within the job", int)
    re50, re99 = grab(rt, r"urgent GEMM done after the flag \(us\): p50 ([\d.]+) \| p99 ([\d.]+)")
    bad, total = grab(rt, r"SAFETY: (\d+) of (\d+) task fingerprints", int)
    tf_job, = grab(rt, r"background: ([\d.]+) TFLOP/s over the job")
    tf_off, below, idle = grab(rt, r"background alone with polls off: ([\d.]+) TFLOP/s -> the "
                                   r"job with arrivals ([-\d.]+)% below it, the polled kernel "
                                   r"alone ([-\d.]+)% below it")
    out["retreat_latency_us"] = {"p50": r50, "p99": r99, "events": n_in,
                                 "p50_over_tile": round(r50 / tile_us, 3),
                                 "mode": "continuous job, accumulator-only checkpoints"}
    out["retreat_urgent_done_us"] = {"p50": re50, "p99": re99}
    out["retreat_background_tflops"] = tf_job
    # the whole cost of being preemptible this way: polls, retreats, resumes
    # and the urgent GEMMs' CUs, against the same kernel with polls off
    out["retreat_background_overhead_pct"] = {"vs_polls_off": below, "polls_off_tflops": tf_off,
                                              "no_arrivals_vs_polls_off": idle}
    # The same job with retreating tiles re-queued from k = 0 (no checkpoint:
    # the ring then holds an entry for every retreat of the job, so no
    # ticket waits for its entry), paying half a tile of redone work per
    # retreat instead of the accumulator save and restore.
    rr = run_bin("urgent_baseline", CFG3 + CFG3_URGENT +
                 ["--bg-tasks", 4096, "--urgent-blocks", 4, "--arrival", "exp",
                  "--mean-gap-us", 2000, "--yield", 1, "--retreat", 4, "--oracle", 1,
                  "--continuous", 1, "--events", events, "--resume", "restart"], timeout=600)
    q50, q99 = grab(rr, r"flag raised -> urgent GEMM starts \(us\): p50 ([\d.]+) \| "
                        r"p90 [\d.]+ \| p99 ([\d.]+)")
    tile_off, = grab(rr, r"tile \(k-chunk\) time at full residency: ([\d.]+) us")
    _, below_r, _ = grab(rr, r"background alone with polls off: ([\d.]+) TFLOP/s -> the "
                             r"job with arrivals ([-\d.]+)% below it, the polled kernel "
                             r"alone ([-\d.]+)% below it")
    bad_r, total_r = grab(rr, r"SAFETY: (\d+) of (\d+) task fingerprints", int)
    n_r, = grab(rr, r"continuous retreat arm: (\d+) arrivals within the job", int)
    out["retreat_restart"] = {"p50": q50, "p99": q99, "events": n_r,
                              "p50_over_tile": round(q50 / tile_off, 3), "tile_us": tile_off,
                              "background_below_polls_off_pct": below_r,
                              "corrupt_tasks": bad_r, "tasks_checked": total_r,
                              "oracle": "PASS" if ("ORACLE: PASS" in rr and
                                                   "yield: PASS" in rr) else "FAIL"}
    out["corrupt_yields"] = bad + bad_r
    out["retreat_tasks_checked"] = total
    out["oracle"] = "PASS" if ("ORACLE: PASS" in rt and "yield: PASS" in rt) else "FAIL"
    # No preemption: the urgent GEMM waits for the background to drain (one
    # background launch per arrival, src/urgent_baseline.cu:309-343).
    nb = run_bin("urgent_baseline", CFG3 + CFG3_URGENT +
                 ["--bg-tasks", 4096, "--urgent-blocks", 4, "--arrival", "exp",
                  "--mean-gap-us", 2000, "--trials", trials], timeout=900)
    n50, n99 = grab(nb, r"urgent e2e \(us\):\s+p50 ([\d.]+) \| p90 [\d.]+ \| p99 ([\d.]+)")
    out["no_preempt_urgent_e2e_us"] = {"p50": n50, "p99": n99, "trials": trials}
    out["by_k_chunk"] = latency_by_k_chunk(max(events // 5, 500), tile_us)
    return out


def latency_by_k_chunk(events, tile128_us):
    """The cfg3 latencies with the tile taken as a 32- and a 64-deep k-chunk
    (cfg2's per-tile K set {32, 64, 128}): the cooperative arm at every
    k-stage, and the retreat arm (accumulator checkpoints), each job walking
    K in chunks of that depth. Polls sit at every 32-deep k-stage in both, so
    the latency in us hardly moves with the chunk, and its ratio to a tile
    grows as the tile shrinks. The cooperative tile time is the 128-deep
    chunk's scaled by depth; the retreat arm measures its own (polls off)."""
    out = {}
    for kc in (32, 64):
        cfg = ["--engine", "mfma128", "--tiles-m", "64", "--tiles-n", "64", "--gemm-k", "4096",
               "--k", str(kc)]
        lat = run_bin("yield", ["--mode", "latency"] + cfg + CFG3_URGENT +
                      ["--poll", "stage", "--arrival", "exp", "--mean-gap-us", 2000,
                       "--events", events + 100], timeout=600)
        p50, p99 = grab(lat, r"preemption latency set->last \(us\): p50 ([\d.]+) \| "
                             r"p90 [\d.]+ \| p99 ([\d.]+)")
        tile = tile128_us * kc / 128
        rt = run_bin("urgent_baseline", cfg + CFG3_URGENT +
                     ["--bg-tasks", 4096, "--urgent-blocks", 4, "--arrival", "exp",
                      "--mean-gap-us", 2000, "--yield", 1, "--retreat", 4, "--oracle", 1,
                      "--continuous", 1, "--events", events, "--resume", "acc"], timeout=600)
        r50, r99 = grab(rt, r"flag raised -> urgent GEMM starts \(us\): p50 ([\d.]+) \| "
                            r"p90 [\d.]+ \| p99 ([\d.]+)")
        rtile, = grab(rt, r"tile \(k-chunk\) time at full residency: ([\d.]+) us")
        bad, total = grab(rt, r"SAFETY: (\d+) of (\d+) task fingerprints", int)
        out[str(kc)] = {
            "coop_k_stage": {"p50": p50, "p99": p99, "tile_us": round(tile, 3),
                             "p50_over_tile": round(p50 / tile, 3),
                             "p99_over_tile": round(p99 / tile, 3)},
            "retreat": {"p50": r50, "p99": r99, "tile_us": rtile,
                        "p50_over_tile": round(r50 / rtile, 3),
                        "p99_over_tile": round(r99 / rtile, 3), "corrupt_tasks": bad,
                        "tasks_checked": total,
                        "oracle": "PASS" if ("ORACLE: PASS" in rt and "yield: PASS" in rt)
                        else "FAIL"},
            "events": events}
    return out


def bf16_metrics():
    """cfg5 bf16 MFMA GEMM throughput (tcyield calibrate, no yields), and the
    retreat arm's latency on the bf16 background (urgent_baseline)."""
    t = run_bin("tcyield", ["--mode", "calibrate", "--tiles-m", 32, "--tiles-n", 32,
                            "--gemm-k", 8192, "--k", 256, "--tasks", 2048,
                            "--prewarm-ms", 1500])
    us, gf = grab(t, r"-> ([\d.]+) us/task/block \| ([\d.]+) GFLOP/s")
    mhz, = grab(t, r"engine clock during the run \(\d+ probes\): mean ([\d.]+) MHz")
    tf = gf / 1e3
    # Retreat arm on the bf16 background: one job, 10,000 exponential
    # arrivals (mean 2 ms), urgent bf16 GEMM 256^3 on its own stream; the
    # retreating blocks re-queue their tiles from k = 0 (no checkpoint of the
    # 256 KiB accumulators).
    rt = run_bin("urgent_baseline", ["--engine", "bf16x256", "--tiles-m", 32, "--tiles-n", 32,
                                     "--gemm-k", 8192, "--k", 256, "--urgent-m", 256,
                                     "--urgent-n", 256, "--urgent-k", 256, "--bg-tasks", 1024,
                                     "--urgent-blocks", 1, "--arrival", "exp", "--mean-gap-us",
                                     2000, "--verify-rows", 32, "--yield", 1, "--retreat", 1,
                                     "--oracle", 1, "--continuous", 1, "--events", 10000,
                                     "--resume", "restart"], timeout=600)
    r50, r99 = grab(rt, r"flag raised -> urgent GEMM starts \(us\): p50 ([\d.]+) \| "
                        r"p90 [\d.]+ \| p99 ([\d.]+)")
    n_in, = grab(rt, r"continuous retreat arm: (\d+) arrivals within the job", int)
    tile_us, = grab(rt, r"tile \(k-chunk\) time at full residency: ([\d.]+) us")
    bad, total = grab(rt, r"SAFETY: (\d+) of (\d+) task fingerprints", int)
    ovh, = grab(rt, r"retreat overhead ([-\d.]+)%")
    _, below = grab(rt, r"background alone with polls off: ([\d.]+) TFLOP/s -> the job "
                        r"with arrivals ([-\d.]+)% below it")
    occ = bf16_occupancy_points()
    return {"occupancy": occ,
            "workload": "cfg5: bf16 GEMM M=N=K=8192 (2 passes of 1024 256x256 tiles), fp32 "
                        "accumulate, 256 workers, no yields, after 1.5 s of the same runs",
            "tflops": round(tf, 2), "peak": 2516.6, "frac": round(tf / 2516.6, 4),
            "engine_clock_mhz": mhz,
            "frac_at_measured_clock": round(tf / (2516.6 * mhz / 2400.0), 4),
            "us_per_tile": us,
            "retreat_latency_us": {"p50": r50, "p99": r99, "events": n_in,
                                   "tile_us": tile_us, "p50_over_tile": round(r50 / tile_us, 3),
                                   "mode": "continuous job, tiles re-queued from k = 0",
                                   "background_overhead_pct": ovh,
                                   "background_below_polls_off_pct": below,
                                   "corrupt_tasks": bad,
                                   "tasks_checked": total,
                                   "oracle": "PASS" if ("ORACLE: PASS" in rt and
                                                        "yield: PASS" in rt) else "FAIL"}}


def bf16_occupancy_points(events=2000):
    """cfg5 at 1, 2 and 4 blocks per CU: the tile each occupancy runs
    (256x256 on 8 waves, 256x128 on 4 waves, 128x128 on one wave), its
    poll-off throughput with the engine clock (tcyield calibrate, after 1 s
    of the same runs), and the cooperative arm's stage-poll latency (set ->
    last block observes, `events` arrivals at U(150, 400) us gaps, urgent bf16
    GEMM 256^3, full checkpoints) in k-chunk times (256-deep chunks, 32 per
    tile). The latency runs hash no task fingerprints (as the reference
    measures it): their safety rests on every urgent output, the float64
    check of C and the exactly-once counts; fingerprints are checked by the
    GPU tests."""
    out = []
    for eng, blocks, tm, tn in (("bf16x256", 256, 32, 32), ("bf16x256x128", 512, 32, 64),
                                ("bf16x128", 1024, 64, 64)):
        g = ["--engine", eng, "--tiles-m", tm, "--tiles-n", tn, "--gemm-k", 8192, "--k", 256,
             "--blocks", blocks]
        t = run_bin("tcyield", ["--mode", "calibrate"] + g + ["--tasks", 2 * blocks * 8,
                                                              "--prewarm-ms", 1000])
        us, gf = grab(t, r"-> ([\d.]+) us/task/block \| ([\d.]+) GFLOP/s")
        mhz, = grab(t, r"engine clock during the run \(\d+ probes\): mean ([\d.]+) MHz")
        ev = run_bin("tcyield", ["--mode", "events"] + g +
                     ["--poll", "stage", "--events", events, "--urgent-m", 256, "--urgent-n",
                      256, "--urgent-k", 256, "--verify-rows", 8, "--oracle", 1,
                      "--fingerprints", 0], timeout=600)
        p50, p99 = grab(ev, r"latency set->last \(us\): p50 ([\d.]+) \| p90 [\d.]+ \| "
                            r"p99 ([\d.]+)")
        first, = grab(ev, r"first observer p50 ([\d.]+) us")
        bad, = grab(ev, r"SAFETY: (\d+)/\d+ urgent outputs corrupt", int)
        chunk_us = us / 32
        tf = gf / 1e3
        out.append({"engine": eng, "tile": [8192 // tm, 8192 // tn],
                    "blocks_per_cu": blocks // 256, "tflops": round(tf, 1),
                    "frac": round(tf / 2516.6, 4), "engine_clock_mhz": mhz,
                    "frac_at_measured_clock": round(tf / (2516.6 * mhz / 2400.0), 4),
                    "k_chunk_us": round(chunk_us, 3),
                    "coop_stage_latency_us": {"p50": p50, "p99": p99, "first_observer_p50": first,
                                              "p50_over_k_chunk": round(p50 / chunk_us, 3),
                                              "events": events},
                    "corrupt_urgent_outputs": bad,
                    "c_check": "PASS" if "bg C PASS" in ev else "FAIL",
                    "oracle": "PASS" if "ORACLE: PASS" in ev else "FAIL"})
    return out


def timed_sustained(launch, flop, steps, prewarm_ms, wall_mhz, torch, apk_amd, stream):
    """Per-launch time (HIP events on the launch stream) of `steps` launches
    that follow `prewarm_ms` of untimed back-to-back launches, with the
    engine clock read by apk_clock_probe on a side stream meanwhile. Returns
    (TFLOP/s from the mean launch time, clock summary)."""
    import numpy as np
    # The side stream's set-up and its first long probe (which perturbs the
    # GEMM beside it for a while) happen inside the pre-warm.
    probes = torch.zeros(32 * 4, dtype=torch.int64, device="cuda")
    side = torch.cuda.Stream()
    apk_amd.clock_probe(probes.data_ptr(), 32, 1, side.cuda_stream)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n = 0
    while (time.perf_counter() - t0) * 1e3 < prewarm_ms:
        for _ in range(20):
            launch(n)
            if n == 0:
                apk_amd.clock_probe(probes.data_ptr(), 32, int(20e3 * wall_mhz), side.cuda_stream)
            n += 1
        stream.synchronize()
    side.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    launch(n)
    ev[0][0].record(stream)
    launch(n + 1)
    ev[0][1].record(stream)
    stream.synchronize()
    est_ms = ev[0][0].elapsed_time(ev[0][1])
    window = max(1, int(0.6 * steps * est_ms * 1e3 * wall_mhz))
    for i in range(steps):
        ev[i][0].record(stream)
        launch(n + 2 + i)
        ev[i][1].record(stream)
        if i == 0:
            apk_amd.clock_probe(probes.data_ptr(), 32, window, side.cuda_stream)
    stream.synchronize()
    side.synchronize()
    ms = float(np.mean([a.elapsed_time(b) for a, b in ev]))
    return flop / (ms * 1e-3) / 1e12, clock_summary(probes.cpu().numpy(), wall_mhz)


def bf16_sustained(workers_list, steps, prewarm_ms, vendor):
    """The bf16x256 persistent GEMM (8192^3, one GEMM per launch, bf16
    operands, fp32 accumulate) on each worker count of `workers_list`, and
    with `vendor` torch.matmul (hipBLASLt) on the same operands, each timed
    after a sustained pre-warm of the same launches with the engine clock
    read beside it. Returns one dict per case."""
    import torch
    import apk_amd
    apk_amd.load()
    info = apk_amd.device_info()
    wall_mhz = info.wall_clock_khz / 1e3
    S = 8192
    flop = 2.0 * S ** 3
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    A = torch.randn((S, S), generator=gen, device="cuda").to(torch.bfloat16)
    Bt = torch.randn((S, S), generator=gen, device="cuda").to(torch.bfloat16)
    C = torch.empty((S, S), device="cuda", dtype=torch.float32)
    stream = torch.cuda.current_stream()
    eng = apk_amd.ENGINE_BF16X256
    ring = 8192  # queue counters per launch; zeroed again only when the ring wraps
    counters = torch.zeros((ring, apk_amd.QUEUE_WORDS), dtype=torch.int32, device="cuda")
    out = []
    for blocks in workers_list:
        counters.zero_()

        def launch(i, blocks=blocks):
            if i % ring == 0 and i > 0:
                counters.zero_()  # stream-ordered after every earlier launch
            apk_amd.persistent_gemm(eng, A.data_ptr(), Bt.data_ptr(), C.data_ptr(), S, S, S, S,
                                    counters[i % ring].data_ptr(), None, blocks,
                                    stream.cuda_stream)
        tf, clk = timed_sustained(launch, flop, steps, prewarm_ms, wall_mhz, torch, apk_amd,
                                  stream)
        out.append({"kernel": "bf16x256 persistent GEMM", "workers": blocks,
                    "tflops": round(tf, 1), "frac": round(tf / 2516.6, 4),
                    "tflops_per_worker": round(tf / blocks, 3), "engine_clock_mhz": clk,
                    "frac_at_measured_clock": round(tf / (2516.6 * clk["mean"] / 2400.0), 4)})
    if vendor:
        B = Bt.t().contiguous()
        Cv = torch.matmul(A, B)
        ours = C if workers_list else None
        tf, clk = timed_sustained(lambda i: torch.matmul(A, B, out=Cv), flop, steps,
                                  prewarm_ms, wall_mhz, torch, apk_amd, stream)
        case = {"kernel": "torch.matmul bf16 (hipBLASLt)", "tflops": round(tf, 1),
                "frac": round(tf / 2516.6, 4), "engine_clock_mhz": clk,
                "frac_at_measured_clock": round(tf / (2516.6 * clk["mean"] / 2400.0), 4)}
        if ours is not None:
            # both products of the same bf16 operands (fp32 accumulate, the
            # vendor's output rounded to bf16): agreement to bf16 rounding
            d = (ours - Cv.float()).norm() / Cv.float().norm()
            case["rel_frobenius_vs_ours"] = float(d)
        out.append(case)
    del A, Bt, C
    torch.cuda.empty_cache()
    return out


def bf16_power_sweep(steps, prewarm_ms):
    """Diagnostic (--bf16-sweep): is the bf16 GEMM's clock set by the load
    on the whole chip? The bf16x256 persistent GEMM on 256, 192, 128 and 64
    workers (one per CU), and torch.matmul on the same shape, each after a
    sustained pre-warm with the engine clock. One JSON line per case."""
    for case in bf16_sustained((256, 192, 128, 64), steps, prewarm_ms, vendor=True):
        print(json.dumps(case), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--prewarm-ms", type=float, default=1500,
                    help="back-to-back untimed launches before the warm-up steps, so that "
                         "the engine clock has left its idle level (it takes ~1 s to climb)")
    ap.add_argument("--size", type=int, default=4096)
    ap.add_argument("--k-chunk", type=int, default=32)
    ap.add_argument("--cpu-rows", type=int, default=1024)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-preempt", action="store_true",
                    help="skip the preemption and bf16 sections")
    ap.add_argument("--events", type=int, default=10000,
                    help="arrivals for the cooperative and retreat latencies")
    ap.add_argument("--trials", type=int, default=10000,
                    help="arrivals (one background launch each) for the no-preemption baseline")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="only time torch.matmul (rocBLAS/hipBLASLt) on the same shapes: bf16 "
                         "8192^3 and fp32 4096^3, for comparison")
    ap.add_argument("--bf16-sweep", action="store_true",
                    help="only run the bf16 clock-versus-load diagnostic (bf16x256 GEMM on "
                         "256/192/128/64 workers and torch.matmul, each after a sustained "
                         "pre-warm, with the engine clock)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB (the "
                         "known-size kernel that scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only; the preemptible persistent "
              "GEMM has no multi-GPU path (each GPU would run its own share of the "
              "tile grid with its own queue and flag).", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import apk_amd

    torch.cuda.set_device(0)
    if args.vendor_gemm:
        res = {}
        for dt, n in ((torch.bfloat16, 8192), (torch.float32, 4096)):
            a = torch.randn(n, n, device="cuda", dtype=dt)
            b = torch.randn(n, n, device="cuda", dtype=dt)
            for _ in range(3):
                a @ b
            torch.cuda.synchronize()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(10):
                a @ b
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / 10
            res[str(dt).split(".")[1]] = {"n": n, "ms": round(ms, 4),
                                          "tflops": round(2 * n ** 3 / ms / 1e9, 1)}
        print(json.dumps({"vendor_gemm": res}), flush=True)
        return
    if args.bf16_sweep:
        bf16_power_sweep(max(args.steps, 20), args.prewarm_ms)
        return
    if args.calibrate_copy:
        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copied {args.calibrate_copy} MiB x3")
        return
    apk_amd.load()
    info = apk_amd.device_info()
    eng = apk_amd.ENGINE_MFMA128
    occ = apk_amd.occupancy(eng)
    blocks = info.cu_count * occ
    S = args.size
    M = N = K = S
    kc = args.k_chunk
    flop = 2.0 * M * N * K

    gen = torch.Generator(device="cuda")
    gen.manual_seed(21)
    dA = torch.rand((M, K), generator=gen, device="cuda", dtype=torch.float32) * 2 - 1
    dB = torch.rand((K, N), generator=gen, device="cuda", dtype=torch.float32) * 2 - 1
    dC = torch.empty((M, N), device="cuda", dtype=torch.float32)
    total = args.warmup + args.steps
    counters = torch.zeros((total, apk_amd.QUEUE_WORDS), dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(total)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(total)]
    torch.cuda.synchronize()
    log(f"device {info.name.decode()} {info.arch.decode()} CUs={info.cu_count} "
        f"occupancy={occ}/CU blocks={blocks}")

    def step(i):
        starts[i].record(stream)
        apk_amd.persistent_gemm(eng, dA.data_ptr(), dB.data_ptr(), dC.data_ptr(),
                                M, N, K, kc, counters[i].data_ptr(), None, blocks,
                                stream.cuda_stream)
        ends[i].record(stream)

    # Engine clock probes: one-wave blocks on a side stream (default
    # priority). The side stream's first launch sets up its hardware queue,
    # and the first long probe beside the GEMM grid slows the GEMM and lowers
    # the clock for a while (measured: 1.03-1.04 against 0.99 ms per launch,
    # 2.22-2.26 against 2.38 GHz): both happen inside the pre-warm, never in
    # the timed steps.
    wall_mhz = info.wall_clock_khz / 1e3
    probes = torch.zeros(32 * 4, dtype=torch.int64, device="cuda")
    side = torch.cuda.Stream()
    apk_amd.clock_probe(probes.data_ptr(), 32, 1, side.cuda_stream)
    torch.cuda.synchronize()
    # Pre-warm: the engine clock climbs from its idle level over ~1 s of load
    # (profiles/engine_clock_readback.md); a few warm-up launches leave it
    # mid-climb. Untimed, on a counter set of its own.
    pre_counters = torch.zeros(apk_amd.QUEUE_WORDS, dtype=torch.int32, device="cuda")
    pre_launches = 0
    t_pre = time.perf_counter()
    while (time.perf_counter() - t_pre) * 1e3 < args.prewarm_ms:
        for _ in range(20):
            pre_counters.zero_()
            apk_amd.persistent_gemm(eng, dA.data_ptr(), dB.data_ptr(), dC.data_ptr(),
                                    M, N, K, kc, pre_counters.data_ptr(), None, blocks,
                                    stream.cuda_stream)
            if pre_launches == 0:
                apk_amd.clock_probe(probes.data_ptr(), 32, int(20e3 * wall_mhz), side.cuda_stream)
            pre_launches += 1
        stream.synchronize()
    side.synchronize()
    pre_ms = (time.perf_counter() - t_pre) * 1e3
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # Engine clock during the timed steps: the probes, beside the GEMM grid,
    # over 60% of the expected timed region (from the warm-up launches). The
    # window is shorter than the timed region, and the timed region waits
    # for the GEMM stream alone, so the probe never lengthens it.
    warm_ms = float(np.min([starts[i].elapsed_time(ends[i]) for i in range(args.warmup)]))
    window = max(1, int(0.6 * args.steps * warm_ms * 1e3 * wall_mhz))
    t0 = time.perf_counter()
    for i in range(args.warmup, total):
        step(i)
        if i == args.warmup:
            apk_amd.clock_probe(probes.data_ptr(), 32, window, side.cuda_stream)
    stream.synchronize()
    wall = time.perf_counter() - t0
    side.synchronize()
    ms_per_step = wall * 1e3 / args.steps
    launch_ms = [starts[i].elapsed_time(ends[i]) for i in range(args.warmup, total)]
    avg_launch_ms = float(np.mean(launch_ms))
    value = flop / (ms_per_step * 1e-3) / 1e12
    achieved = flop / (avg_launch_ms * 1e-3) / 1e12
    clock = clock_summary(probes.cpu().numpy(), wall_mhz)
    log(f"GEMM {M}x{N}x{K} kc={kc}: {ms_per_step:.3f} ms/step wall, "
        f"{avg_launch_ms:.3f} ms/launch (events) -> {value:.1f} TFLOP/s; engine clock "
        f"{clock['mean']:.0f} MHz (min {clock['min']:.0f}, max {clock['max']:.0f})")

    out = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": (f"cfg2 tile calibration: persistent fp32 SGEMM M=N=K={S}, "
                         f"128x128 tiles (MFMA128, v_mfma_f32_32x32x2_f32), "
                         f"k_chunk={kc}, {blocks} workers, no yields"),
            "M": M, "N": N, "K": K, "tile": [128, 128], "k_chunk": kc,
            "workers": blocks, "workers_per_cu": occ,
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": PEAK_FP32_TF,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_FP32_TF, 4),
            # the peak is quoted at 2.4 GHz; the clock the launches ran at:
            "engine_clock_mhz": clock,
            "frac_at_measured_clock": round(achieved / (PEAK_FP32_TF * clock["mean"] / 2400.0), 4),
            "traffic": measured_traffic() if (S, kc) == (4096, 32) else None,
        },
        "prewarm": {"ms": round(pre_ms, 1), "launches": pre_launches},
    }
    failed = []

    def section(name, fn):
        """A section's figures, or {"error": ...} in their place (and a
        non-zero exit status after the line is printed) if it fails: the
        GEMM line above is never lost to a later section."""
        try:
            return fn()
        except Exception as e:  # a binary's exit status, a missing pattern
            import traceback
            traceback.print_exc()
            failed.append(name)
            return {"error": f"{type(e).__name__}: {str(e)[:800]}"}

    if not args.no_preempt:
        out["preemption"] = section("preemption",
                                    lambda: preemption_metrics(args.events, args.trials))

        def bf16_all():
            b = bf16_metrics()
            blocks_bf16 = info.cu_count * apk_amd.occupancy(apk_amd.ENGINE_BF16X256)
            ours, vendor = bf16_sustained((blocks_bf16,), 20, args.prewarm_ms, vendor=True)
            b["sustained"] = {k: ours[k] for k in ("tflops", "frac", "engine_clock_mhz",
                                                   "frac_at_measured_clock")}
            b["sustained"]["workload"] = (
                "one 8192^3 GEMM per launch (apk_persistent_gemm, bf16x256), 20 launches timed "
                f"after {args.prewarm_ms:.0f} ms of the same launches")
            b["vendor_sustained"] = {k: vendor[k] for k in (
                "kernel", "tflops", "frac", "engine_clock_mhz", "frac_at_measured_clock")}
            return b
        out["bf16"] = section("bf16", bf16_all)
        log("preemption: " + json.dumps(out["preemption"]))
        log("bf16: " + json.dumps(out["bf16"]))
    if not args.no_cpu:
        A_host = dA.cpu().numpy()
        B_host = dB.cpu().numpy()
        C_gpu = dC.cpu().numpy()
        cb, frob = cpu_baseline(A_host, B_host, C_gpu, args.cpu_rows)
        out["cpu_baseline"] = {k: v for k, v in cb.items() if k != "seconds"}
        out["check"] = {"rows": M, "rel_frobenius_vs_f64": frob, "tol": 1e-5,
                        "pass": bool(frob <= 1e-5)}
        log(f"cpu baseline {cb['value'] * 1e3:.1f} GFLOP/s on {cb['cores']} threads "
            f"({cb['single_thread']['value'] * 1e3:.2f} on 1); whole C rel-Frobenius {frob:.2e}")
        if not out["check"]["pass"]:
            failed.append("check")
    print(json.dumps(out), flush=True)
    if failed:
        log("bench.py: failed: " + ", ".join(failed))
        sys.exit(1)


if __name__ == "__main__":
    main()
