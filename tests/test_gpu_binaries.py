"""The five measurement binaries as a drop-in for the reference's sweep drivers.

Each test runs a binary with a scaled-down version of an invocation from the
reference's own drivers (scripts/calibrate.sh, phase2.sh, phase3.sh,
phase5.sh, pareto.sh) and checks:
  * exit status 0 (every binary checks its own results and exits 1 on a
    failed float64 check, oracle or safety verdict);
  * the CSV header: the reference's columns, byte for byte, first (extra
    columns only appended at the end);
  * the OBS1 observation matrix: magic, shape, and that it holds exactly the
    per-event set / observation times the latency CSV summarises.

Scaling: fewer events / trials / tasks and smaller tile grids than the
drivers use, so that each binary runs for seconds.
"""
import os
import re
import struct
import subprocess

import numpy as np
import pytest

from apk_amd.analysis import common as an_common
from apk_amd.analysis import maxofn, visibility
from apk_amd.analysis import spread as an_spread
from gpu_util import say

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "apk_amd", "bin")

# The reference's CSV headers (the interface the analysis scripts read).
HDR_PERSISTENT = "task,block,smid,start_cyc,end_cyc,dur_cyc,dur_us"  # src/persistent.cu:252
HDR_URGENT = ("trial,delay_us,consumed_at_arrival,remaining_at_arrival,"
              "e2e_us,exec_us,gap_us,drain_us")  # src/urgent_baseline.cu:366-367
HDR_YIELD_OVH = "rep,poll,wall_ms"  # src/yield.cu:702
HDR_YIELD_LAT = ("event,set_ns,first_obs_ns,last_obs_ns,lat_us,spread_us,"
                 "claimer,e2e_us,complete,last_block,block0_delay_us,"
                 "lat_excl_setter_us")  # src/yield.cu:886-888
HDR_MIDYIELD = ("event,lat_us,lat_excl_setter_us,first_us,claimer,e2e_us,"
                "cu_max_rel,corrupt,complete,site")  # src/midyield.cu:699-700
HDR_TCYIELD = ("event,lat_us,lat_excl_setter_us,first_us,claimer,"
               "e2e_us,bad_elems,site,complete")  # src/tcyield.cu:762-763
OBS1_MAGIC = 0x3153424f  # src/yield.cu:452-466


def run_bin(name, *args, timeout=240):
    cmd = [os.path.join(BIN, name)] + [str(a) for a in args]
    say("$ " + " ".join([f"apk_amd/bin/{name}"] + cmd[1:]))
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, f"{name} exited {r.returncode}\n{r.stdout[-3000:]}\n{r.stderr[-3000:]}"
    return r.stdout


def assert_header(path, ref):
    with open(path, "rb") as f:
        first = f.readline().decode()
    assert first == ref + "\n" or first.startswith(ref + ","), (path, first, ref)
    return first.rstrip("\n").split(",")


def read_csv(path):
    import csv
    with open(path) as f:
        return list(csv.DictReader(f))


def read_obs1(path):
    raw = open(path, "rb").read()
    magic, events, blocks = struct.unpack_from("<3q", raw, 0)
    assert magic == OBS1_MAGIC
    assert len(raw) == 8 * (3 + events + events * blocks), (len(raw), events, blocks)
    body = np.frombuffer(raw, dtype="<i8", offset=24)
    return events, blocks, body[:events], body[events:].reshape(events, blocks)


@pytest.fixture(scope="module", autouse=True)
def binaries_built():
    for b in ("persistent", "urgent_baseline", "yield", "midyield", "tcyield"):
        assert os.access(os.path.join(BIN, b), os.X_OK), f"apk_amd/bin/{b} not built"


def test_calibrate_sh(tmp_path):
    """scripts/calibrate.sh:13-18: persistent --k K --sm-clock-mhz M --csv."""
    for k in (32, 64, 128, 256, 512):
        csv = tmp_path / f"calib_k{k}.csv"
        out = run_bin("persistent", "--k", k, "--sm-clock-mhz", 1695, "--tiles-m", 16,
                      "--tiles-n", 16, "--passes", 1, "--csv", csv)
        assert "PASS" in out or "verify" in out.lower(), out[-800:]
        assert_header(csv, HDR_PERSISTENT)
        rows = read_csv(csv)
        assert len(rows) == 16 * 16
        assert sorted(int(r["task"]) for r in rows) == list(range(256))
        assert all(int(r["end_cyc"]) >= int(r["start_cyc"]) for r in rows)


def test_persistent_prints_engine_clock(tmp_path):
    """The final pass's TFLOP/s comes with the engine clock read on the device
    during that pass (apk_clock_probe windows inside the pass's records)."""
    out = run_bin("persistent", "--engine", "mfma128", "--tiles-m", 32, "--tiles-n", 32,
                  "--gemm-k", 4096, "--k", 128, "--passes", 3, "--verify", 0,
                  "--csv", tmp_path / "p.csv")
    m = re.search(r"engine clock during the final pass \((\d+) probes\): mean (\d+) MHz", out)
    assert m, out[-1500:]
    assert int(m.group(1)) >= 1 and 500 <= int(m.group(2)) <= 3000, m.group(0)


@pytest.mark.parametrize("sel,tiles,bpc", [(("--engine", "bf16x256"), 4, 1),
                                            (("--dtype", "bf16"), 4, 1),
                                            (("--engine", "bf16x128"), 8, 2),
                                            (("--engine", "bf16x128"), 8, 4),
                                            (("--engine", "bf16x256x128"), 8, 2)])
def test_persistent_bf16_engines(tmp_path, sel, tiles, bpc):
    """persistent --engine bf16x256|bf16x128|bf16x256x128 (--dtype bf16 = bf16x256): the
    bf16 tiles on the reference's tcyield data (normal(0,1) rounded to bf16),
    float64 check passes, one record per (tile, chunk) in the reference's CSV
    schema."""
    csv = tmp_path / "bf16.csv"
    out = run_bin("persistent", *sel, "--tiles-m", tiles, "--tiles-n", tiles,
                  "--gemm-k", 1024, "--k", 256, "--passes", 2, "--blocks-per-cu", bpc,
                  "--verify", 1, "--csv", csv)
    assert "PASS:" in out and "bf16 peak" in out, out[-1500:]
    assert ("bf16x256" if sel[1] == "bf16" else sel[1]) in out
    assert_header(csv, HDR_PERSISTENT)
    assert len(read_csv(csv)) == tiles * tiles * 4


def test_phase2_sh(tmp_path):
    """scripts/phase2.sh: urgent_baseline --mode sat|sat-1|1persm --trials T."""
    for mode in ("sat", "sat-1", "1persm"):
        csv = tmp_path / f"phase2_{mode}.csv"
        out = run_bin("urgent_baseline", "--mode", mode, "--trials", 20, "--bg-tasks", 4000,
                      "--tiles-m", 16, "--tiles-n", 16, "--csv", csv)
        assert "PASS" in out
        assert_header(csv, HDR_URGENT)
        rows = read_csv(csv)
        assert len(rows) == 20
        assert all(float(r["e2e_us"]) > 0 for r in rows)


def test_phase3_sh(tmp_path):
    """scripts/phase3.sh: verify, overhead, latency --set dev and --set host."""
    out = run_bin("yield", "--mode", "verify", "--tasks", 4000, "--tiles-m", 16, "--tiles-n", 16)
    assert "PASS" in out
    ovh = tmp_path / "phase3_overhead.csv"
    run_bin("yield", "--mode", "overhead", "--tasks", 20000, "--reps", 4, "--tiles-m", 16,
            "--tiles-n", 16, "--csv", ovh)
    assert_header(ovh, HDR_YIELD_OVH)
    assert len(read_csv(ovh)) == 8
    for setter in ("dev", "host"):
        lat = tmp_path / f"phase3_lat_{setter}.csv"
        obs = tmp_path / f"phase3_lat_{setter}.obs"
        out = run_bin("yield", "--mode", "latency", "--set", setter, "--events", 300,
                      "--warmup-events", 20, "--tiles-m", 16, "--tiles-n", 16, "--csv", lat,
                      "--dump-obs", obs)
        assert "preemption latency set->last" in out, out[-1500:]
        if setter == "host":
            assert "host->device flag visibility" in out
        cols = assert_header(lat, HDR_YIELD_LAT)
        rows = read_csv(lat)
        assert len(rows) == 300
        events, blocks, set_ns, obs_ns = read_obs1(obs)
        assert events == 300 and blocks > 0
        complete = 0
        for e, r in enumerate(rows):
            assert int(r["event"]) == e
            if r["complete"] != "1":
                continue
            complete += 1
            o = obs_ns[e]
            assert (o > 0).all()
            # the CSV's first/last observation are the matrix row's min/max
            assert abs(int(r["first_obs_ns"]) - int(o.min())) <= 20, (e, r, o.min())
            assert abs(int(r["last_obs_ns"]) - int(o.max())) <= 20, (e, r, o.max())
            if setter == "dev":
                assert int(set_ns[e]) == int(r["set_ns"]) or abs(int(set_ns[e]) - int(r["set_ns"])) <= 20
        assert complete >= 250, complete
        assert "claim_site" in cols
        # the analysis ports read the binary's own files: the identity
        # lat == first + spread holds row by row, and the OBS1 matrix feeds
        # the held-out max-of-N model
        n = an_spread.analyse_rows(rows, 20, str(lat))[0]
        assert n == sum(1 for r in rows if r["complete"] == "1" and int(r["event"]) >= 20)
        d = an_common.delays_us(obs, 20)
        assert d.shape[1] == blocks - 1 and d.shape[0] >= 200
        for q, pred, meas in maxofn.heldout(d):
            assert pred > 0 and meas > 0


def test_phase5_sh(tmp_path):
    """scripts/phase5.sh: midyield verify (drain, poison), events per
    discipline at the stage site, the boundary comparator and the overhead
    pair; plus the issue site the reference's POLL_ISSUE defines."""
    run_bin("midyield", "--mode", "verify", "--discipline", "drain", "--tasks", 4000,
            "--tiles-m", 16, "--tiles-n", 16)
    run_bin("midyield", "--mode", "verify", "--discipline", "poison", "--tasks", 4000,
            "--tiles-m", 16, "--tiles-n", 16)
    for disc in ("drain", "naive", "poison"):
        csv = tmp_path / f"phase5_{disc}.csv"
        out = run_bin("midyield", "--mode", "events", "--discipline", disc, "--events", 200,
                      "--warmup-events", 10, "--tiles-m", 16, "--tiles-n", 16, "--csv", csv)
        assert "SAFETY:" in out
        assert_header(csv, HDR_MIDYIELD)
        rows = read_csv(csv)  # one row per fired event (src/midyield.cu:701-739)
        assert 0 < len(rows) <= 200
        assert len({r["event"] for r in rows}) == len(rows)
    for disc in ("drain", "naive"):
        out = run_bin("midyield", "--mode", "events", "--discipline", disc, "--poll", "issue",
                      "--events", 200, "--warmup-events", 10, "--tiles-m", 16, "--tiles-n", 16,
                      "--engine", "mfma128", "--k", 32, "--gemm-k", 512)
        assert "SAFETY:" in out
    csv = tmp_path / "phase5_drain_boundary.csv"
    run_bin("midyield", "--mode", "events", "--discipline", "drain", "--poll", "boundary",
            "--events", 200, "--warmup-events", 10, "--tiles-m", 16, "--tiles-n", 16,
            "--csv", csv)
    assert_header(csv, HDR_MIDYIELD)
    for poll in ("stage", "boundary"):
        out = run_bin("midyield", "--mode", "overhead", "--poll", poll, "--tasks", 20000,
                      "--reps", 4, "--tiles-m", 16, "--tiles-n", 16)
        assert "overhead" in out


def test_tcyield(tmp_path):
    """tcyield (src/tcyield.cu:384-842): verify, calibrate, overhead, events."""
    # 8 tasks per block: the setter (block 0) raises the 5 events at its own
    # sites, one per site, and a 256-deep task has only 4 of them
    run_bin("tcyield", "--mode", "verify", "--tasks", 2048)
    out = run_bin("tcyield", "--mode", "calibrate", "--tasks", 512)
    assert "GFLOP/s" in out
    run_bin("tcyield", "--mode", "overhead", "--poll", "pe", "--tasks", 512, "--reps", 4)
    csv = tmp_path / "tc_events.csv"
    out = run_bin("tcyield", "--mode", "events", "--poll", "stage", "--events", 100,
                  "--warmup-events", 10, "--csv", csv)
    assert "SAFETY:" in out
    assert_header(csv, HDR_TCYIELD)
    assert 0 < len(read_csv(csv)) <= 100
    # the latency runs' variant: no per-task fingerprints, same verdict
    out = run_bin("tcyield", "--mode", "events", "--poll", "stage", "--events", 100,
                  "--warmup-events", 10, "--fingerprints", 0, "--oracle", 1)
    assert "0 of 0 task fingerprints differ from the unpreempted tile (--fingerprints 0)" in out
    assert "ORACLE: PASS" in out and "events: PASS" in out


@pytest.mark.parametrize("loaded,iters", [(0, 0), (1, 64)])
def test_visibility(tmp_path, loaded, iters):
    """yield --mode visibility (src/yield.cu:470-568): the run ends on its own
    (the setter stores the stop value; every block also has a deadline) and
    every event is observed by every block, at or after its set time."""
    obs = tmp_path / f"vis_{loaded}.obs"
    out = run_bin("yield", "--mode", "visibility", "--events", 300, "--warmup-events", 20,
                  "--loaded", loaded, "--work-iters", iters, "--dump-obs", obs)
    assert "(0 unset, 0 anomalies)" in out, out[-1500:]
    events, blocks, set_ns, o = read_obs1(obs)
    assert events == 300 and blocks >= 256
    assert (set_ns > 0).all()
    assert (o > 0).all(), f"{int((o == 0).sum())} (event, block) pairs never observed"
    assert (o >= set_ns[:, None] - 20).all()
    p50, p99 = visibility.dmax_quantiles(obs, 20)
    dmax = ((o - set_ns[:, None]).max(axis=1) / 1e3)[20:]
    assert dmax.min() <= p50 <= p99 <= dmax.max()


def test_pareto_sh(tmp_path):
    """scripts/pareto.sh:10-24: reserved slots vs the cooperative arm."""
    for r_, u in ((8, 1), (32, 4)):
        csv = tmp_path / f"res_R{r_}_U{u}.csv"
        run_bin("urgent_baseline", "--mode", "sat", "--reserve", r_, "--urgent-blocks", u,
                "--trials", 20, "--bg-tasks", 4000, "--tiles-m", 16, "--tiles-n", 16,
                "--csv", csv)
        assert_header(csv, HDR_URGENT)
        assert len(read_csv(csv)) == 20
    for u in (1, 4):
        csv = tmp_path / f"coop_U{u}.csv"
        out = run_bin("yield", "--mode", "latency", "--set", "dev", "--events", 200,
                      "--warmup-events", 10, "--urgent-tiles", u, "--tiles-m", 16,
                      "--tiles-n", 16, "--csv", csv)
        assert "urgent e2e set->done" in out
        assert_header(csv, HDR_YIELD_LAT)
