"""Parity at the BASELINE configurations' full sizes, through the product
binaries (each one checks its own results against the oracle's definitions
and exits non-zero on any violation):

  cfg3  fp32 background M=N=8192, K=4096, 128x128 tiles on all 256 CUs; the
        urgent 256^3 GEMM on a second stream at exponential arrivals (mean
        2 ms), retreat arm: every task's fingerprint equals the unpreempted
        run's, the urgent output is bit-identical, every task runs once;
  cfg4  fp32 M=N=K=8192, 3-stage LDS ring, >= 25,000 k-stage yields with
        checkpoint/resume: C bit-identical to the unpreempted run, float64
        within 1e-5 rel-Frobenius, exactly-once; plus the issue site, where
        >= 25,000 checkpoints are taken while a live stage is still in flight
        (the buffer-conflicting yields) and the drain keeps every one exact;
  cfg5  bf16 M=N=K=8192, 256x256 tiles at 1 block per CU and the 128x128
        tile at 2 and 4 blocks per CU, yields at k-stage (and for 256x256
        tile-boundary) sites: C bit-identical, float64 (bf16-rounded inputs)
        within 1e-2, exactly-once; the 1e8-task tiny oracle at 1, 2 and 4
        blocks per CU; the retreat arm on the 256x256 background, one job of
        400 arrivals.
When tasks cycle the grid (more tasks than tiles) C holds the last pass, so
every task's fingerprint against its unpreempted tile is checked as well.
"""
import os
import re
import subprocess

import pytest

from gpu_util import say

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "apk_amd", "bin")

CFG4 = ["--engine", "mfma128", "--tiles-m", 64, "--tiles-n", 64, "--gemm-k", 8192, "--k", 32,
        "--urgent-m", 128, "--urgent-n", 128, "--urgent-k", 256, "--verify-rows", 64]
CFG5 = ["--tiles-m", 32, "--tiles-n", 32, "--gemm-k", 8192, "--k", 256, "--urgent-m", 256,
        "--urgent-n", 256, "--urgent-k", 256, "--verify-rows", 32]
CFG3 = ["--engine", "mfma128", "--tiles-m", 64, "--tiles-n", 64, "--gemm-k", 4096, "--k", 128,
        "--urgent-m", 256, "--urgent-n", 256, "--urgent-k", 256]


def run_bin(name, *args, timeout=300):
    cmd = [os.path.join(BIN, name)] + [str(a) for a in args]
    say("$ " + " ".join([f"apk_amd/bin/{name}"] + cmd[1:]))
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    tail = r.stdout[-2500:]
    assert r.returncode == 0, f"{name} exited {r.returncode}\n{tail}\n{r.stderr[-2000:]}"
    for line in r.stdout.splitlines():
        if re.match(r"(SAFETY|yields|resumed|ORACLE|C check|oracle|naive|events)", line):
            say("  " + line)
    return r.stdout


def grab(text, pattern, cast=int):
    m = re.search(pattern, text)
    assert m, f"{pattern!r} not in output:\n{text[-2000:]}"
    return tuple(cast(g) for g in m.groups())


def assert_identical(out):
    """C bit-identical to the unpreempted run (its last pass, when tasks cycle
    the grid) and no task fingerprint differing from its unpreempted tile."""
    bad, hashed = grab(out, r"resumed background: (\d+) of (\d+) task fingerprints differ")
    assert bad == 0 and hashed > 0, (bad, hashed)
    assert re.search(r"C bit-identical to the unpreempted run: (yes|last pass yes)", out), out[-2000:]


def test_cfg4_stage_yields_25k():
    out = run_bin("midyield", *CFG4, "--mode", "events", "--poll", "stage", "--events", 26000,
                  "--oracle", 1)
    yields, = grab(out, r"yields: (\d+)")
    assert yields >= 25000
    assert_identical(out)
    corrupt, = grab(out, r"SAFETY: (\d+)/")
    assert corrupt == 0
    assert "ORACLE: PASS" in out


@pytest.mark.parametrize("disc", ["drain", "naive"])
def test_cfg4_issue_site(disc):
    out = run_bin("midyield", *CFG4, "--mode", "events", "--poll", "issue", "--discipline",
                  disc, "--events", 4000, "--oracle", 1)
    assert "ORACLE: PASS" in out
    if disc == "drain":
        assert_identical(out)
        stale, = grab(out, r"stale checkpoints: (\d+)")
        assert stale == 0
        # every observer checkpoints at an issue site; the buffer-conflicting
        # ones found the newest stage's loads still landing when the drain began
        ckpts, inflight = grab(out, r"\(of all (\d+) checkpoints: (\d+)\)")
        say(f"  issue-site checkpoints {ckpts}, live stage in flight at {inflight}")
        assert inflight >= 25000, (ckpts, inflight)
    else:
        # the drain is load-bearing: without it some checkpoints are stale,
        # and exactly those resumes differ from the unpreempted tile
        assert "every corruption follows a stale checkpoint" in out
        stale, = grab(out, r"stale checkpoints resumed: (\d+)")
        bad, = grab(out, r"naive control: (\d+) corrupted tasks")
        assert stale > 0 and 0 < bad <= stale


@pytest.mark.parametrize("poll", ["stage", "pe"])
def test_cfg5_bf16_yields(poll):
    out = run_bin("tcyield", *CFG5, "--mode", "events", "--poll", poll, "--events", 1500,
                  "--oracle", 1)
    assert_identical(out)
    corrupt, = grab(out, r"SAFETY: (\d+)/")
    assert corrupt == 0
    assert "ORACLE: PASS" in out


CFG5_128 = ["--tiles-m", 64, "--tiles-n", 64, "--gemm-k", 8192, "--k", 256, "--urgent-m", 256,
            "--urgent-n", 256, "--urgent-k", 256, "--verify-rows", 32]


@pytest.mark.parametrize("engine,blocks", [("bf16x128", 1024), ("bf16x256x128", 512),
                                           ("bf16x128", 512)])
def test_cfg5_bf16_small_tiles_yields_multi_block(engine, blocks):
    """cfg5 at 4 and 2 blocks per CU (the 256x256 tile cannot hold them): the
    one-wave 128x128 tile at 4 (and 2), the 256x128 tile at 2; k-stage yields
    with checkpoint/resume."""
    tiles_m = ["--tiles-m", 32] if engine == "bf16x256x128" else []
    # flags are read first match first: the tile rows go ahead of CFG5_128's
    out = run_bin("tcyield", *tiles_m, *CFG5_128, "--engine", engine, "--blocks", blocks,
                  "--mode", "events", "--poll", "stage", "--events", 1500, "--oracle", 1)
    yields, = grab(out, r"yields: (\d+)")
    assert yields >= 1000
    assert_identical(out)
    corrupt, = grab(out, r"SAFETY: (\d+)/")
    assert corrupt == 0
    assert "ORACLE: PASS" in out


@pytest.mark.parametrize("bpc", [1, 2, 4])
def test_cfg5_tiny_oracle_1e8(bpc):
    out = run_bin("tcyield", "--mode", "tiny", "--tasks", 100000000, "--blocks-per-cu", bpc)
    assert "ORACLE: PASS" in out


def test_cfg3_retreat_arm_8192():
    out = run_bin("urgent_baseline", *CFG3, "--bg-tasks", 4096, "--urgent-blocks", 4,
                  "--arrival", "exp", "--mean-gap-us", 2000, "--trials", 100,
                  "--verify-rows", 64, "--yield", 1, "--retreat", 4, "--oracle", 1)
    bad, total = grab(out, r"SAFETY: (\d+) of (\d+) task fingerprints")
    assert bad == 0 and total == 100 * 4096
    assert "ORACLE: PASS" in out
    assert "yield: PASS" in out


def test_cfg3_no_preemption_baseline_8192():
    """The no-yield urgent baseline (src/urgent_baseline.cu:309-343) at cfg3:
    background and urgent GEMM run concurrently on two streams and both match
    float64 (the binary's correctness gate) before the trials."""
    out = run_bin("urgent_baseline", *CFG3, "--bg-tasks", 4096, "--urgent-blocks", 4,
                  "--arrival", "exp", "--mean-gap-us", 2000, "--trials", 50,
                  "--verify-rows", 64)
    assert "PASS:" in out
    assert "urgent e2e (us)" in out


@pytest.mark.parametrize("resume", ["ckpt", "acc"])
def test_cfg3_retreat_arm_continuous(resume):
    """cfg3 retreat arm as one background job (M=N=8192, K=4096 on all 256
    CUs) with 400 exponential arrivals raised by the host: every task's
    fingerprint matches its unpreempted tile, every task runs exactly once,
    the kept urgent outputs are bit-identical, no resume entry is lost."""
    out = run_bin("urgent_baseline", *CFG3, "--bg-tasks", 4096, "--urgent-blocks", 4,
                  "--arrival", "exp", "--mean-gap-us", 2000, "--yield", 1, "--retreat", 4,
                  "--oracle", 1, "--continuous", 1, "--events", 400, "--resume", resume)
    bad, = grab(out, r"SAFETY: (\d+) of \d+ task fingerprints")
    assert bad == 0
    n_in, = grab(out, r"continuous retreat arm: (\d+) arrivals within the job")
    assert n_in == 400
    assert "arrivals without a retreat 0" in out
    assert "ORACLE: PASS" in out and "yield: PASS" in out


@pytest.mark.parametrize("resume", ["restart", "acc"])
def test_cfg5_bf16_retreat_arm_continuous(resume):
    """cfg5 retreat arm on the bf16 256x256 background (M=N=K=8192, 1 block
    per CU) as one job with 400 exponential arrivals, tiles re-queued from
    k = 0 or resumed from their accumulators: the blocks that may retreat
    poll every pair of stages with the pairs software-pipelined, and every
    task's fingerprint matches its unpreempted tile, every task runs once,
    the kept urgent outputs are bit-identical."""
    out = run_bin("urgent_baseline", "--engine", "bf16x256", *CFG5, "--bg-tasks", 1024,
                  "--urgent-blocks", 1, "--arrival", "exp", "--mean-gap-us", 2000, "--yield", 1,
                  "--retreat", 1, "--oracle", 1, "--continuous", 1, "--events", 400,
                  "--resume", resume)
    bad, = grab(out, r"SAFETY: (\d+) of \d+ task fingerprints")
    assert bad == 0
    n_in, = grab(out, r"continuous retreat arm: (\d+) arrivals within the job")
    assert n_in == 400
    assert "arrivals without a retreat 0" in out
    assert "ORACLE: PASS" in out and "yield: PASS" in out
