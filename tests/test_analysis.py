"""CPU tests of apk_amd/analysis: the latency-CSV spread analysis, the
held-out max-of-N model, the visibility summary, the OBS1 reader and the
rocm-smi clock parser, on matrices and CSVs built here with known answers.
The GPU tests (test_gpu_binaries.py) run the same functions over the files
the binaries write."""
import bisect
import os
import sys
import time

import numpy as np
import pytest

from apk_amd.analysis import clock_readback, common, maxofn, spread, visibility

HDR = ("event,set_ns,first_obs_ns,last_obs_ns,lat_us,spread_us,claimer,e2e_us,complete,"
       "last_block,block0_delay_us,lat_excl_setter_us,claim_site")


def write_latency_csv(path, events):
    """events: list of (set_ns, first_ns, last_ns, complete); columns written
    with the binary's rounding (lat_us, spread_us to 0.01 us)."""
    with open(path, "w") as f:
        f.write(HDR + "\n")
        for e, (s, lo, hi, c) in enumerate(events):
            f.write(f"{e},{s},{lo},{hi},{(hi - s) / 1e3:.2f},{(hi - lo) / 1e3:.2f},0,-1.00,"
                    f"{int(c)},1,0.00,{(hi - s) / 1e3:.2f},0\n")


def test_nearest_rank_percentile():
    v = list(range(100, 0, -1))  # 1..100, unsorted
    assert common.pct(v, 0.5) == 51  # v[int(0.5 * 100)] of sorted 1..100
    assert common.pct(v, 0.99) == 100
    assert common.pct(v, 1.0) == 100  # clamped to the last element
    assert common.pct([7.0], 0.9) == 7.0
    with pytest.raises(ValueError):
        common.pct([], 0.5)


def test_spread_cell(tmp_path):
    # 1000 measured events: spread k * 10 ns (k = 0..999 shuffled), first
    # delay 2 us + k * 1 ns; 100 warm-up events and 5 incomplete events with
    # huge values that must not count.
    rng = np.random.default_rng(3)
    ks = rng.permutation(1000)
    ev = [(1_000_000 * i, 0, 0, True) for i in range(100)]
    ev = [(s, s + 50_000_000, s + 90_000_000, c) for s, _, _, c in ev]  # warm-up outliers
    for i, k in enumerate(ks):
        s = 10_000_000 + 1_000_000 * i
        first = s + 2000 + int(k)
        ev.append((s, first, first + 10 * int(k), True))
    for i in range(5):
        s = 2_000_000_000 + i
        ev.append((s, s + 1, s + 99_000_000, False))
    p = tmp_path / "phase4_lat_b32_p1.csv"
    write_latency_csv(p, ev)
    n, s50, s95, s99, f50, f99 = spread.analyse_rows(common.read_rows(p), 100, str(p))
    assert n == 1000
    # nearest-rank over k*0.01 us, k = 0..999: index int(q * 1000)
    assert (s50, s95, s99) == (5.0, 9.5, 9.9)
    assert f50 == pytest.approx(2.5) and f99 == pytest.approx(2.99)


def test_spread_identity_violation_is_caught(tmp_path):
    ev = [(1000 * i * 1000, 1000 * i * 1000 + 2000, 1000 * i * 1000 + 5000, True)
          for i in range(300)]
    p = tmp_path / "x.csv"
    write_latency_csv(p, ev)
    rows = common.read_rows(p)
    spread.analyse_rows(rows, 100)  # consistent: passes
    rows[150]["lat_us"] = f"{float(rows[150]['lat_us']) + 0.03:.2f}"  # planted error
    with pytest.raises(spread.IdentityError):
        spread.analyse_rows(rows, 100)
    rows[150]["lat_us"] = f"{float(rows[150]['lat_us']) - 0.02:.2f}"  # within rounding
    spread.analyse_rows(rows, 100)


def test_spread_grid_cli(tmp_path, capsys):
    raw = tmp_path / "raw"
    raw.mkdir()
    for b in (32, 64):
        for p in (1, 2):
            # spread grows with blocks x poll: every measured event spreads by b*p ns
            ev = [(10**6 * i, 10**6 * i + 1000, 10**6 * i + 1000 + 10 * b * p, True)
                  for i in range(400)]
            write_latency_csv(raw / f"phase4_lat_b{b}_p{p}.csv", ev)
    out = tmp_path / "sum" / "spread.csv"
    rc = spread.main(["--raw", str(raw), "--blocks", "64,32", "--poll", "2,1", "--out", str(out)])
    assert rc == 0
    lines = out.read_text().splitlines()
    assert lines[0] == spread.HEADER
    assert [l.split(",")[:3] for l in lines[1:]] == [
        ["32", "1", "300"], ["32", "2", "300"], ["64", "1", "300"], ["64", "2", "300"]]
    assert lines[1].split(",")[3] == "0.320"
    text = capsys.readouterr().out
    assert "spread p50 growth with blocks (poll=1): 2.00x" in text
    assert "spread p50 growth with poll period (blocks=64): 2.00x" in text
    assert spread.main(["--raw", str(raw), "--blocks", "128", "--poll", "1",
                        "--out", str(out)]) == 2


def test_obs1_round_trip_and_validation(tmp_path):
    set_ns = np.array([0, 1000, 2000], dtype=np.int64)
    obs = np.array([[0, 0], [1500, 1700], [2600, 0]], dtype=np.int64)
    p = tmp_path / "m.obs1"
    common.write_obs1(p, set_ns, obs)
    raw = p.read_bytes()
    assert len(raw) == 8 * (3 + 3 + 6)
    assert raw[:4] == b"OBS1"  # magic 0x3153424f little-endian
    s2, o2 = common.read_obs1(p)
    assert (s2 == set_ns).all() and (o2 == obs).all()
    # warm-up 0: event 0 unset, event 2 incomplete -> only event 1 is kept
    d = common.delays_us(p, warmup=0, exclude_setter=False)
    assert d.tolist() == [[0.5, 0.7]]
    assert common.delays_us(p, warmup=0).tolist() == [[0.7]]
    p.write_bytes(raw[:-8])
    with pytest.raises(ValueError):
        common.read_obs1(p)
    p.write_bytes(b"XXXX" + raw[4:])
    with pytest.raises(ValueError):
        common.read_obs1(p)


def bisection_quantile(fit_sorted, n, q):
    """The max-of-N predicted quantile by bisection over x on the step
    function F(x)^n (an independent method for the closed form)."""
    L = len(fit_sorted)
    lo, hi = float(fit_sorted[0]) - 1.0, float(fit_sorted[-1]) + 1.0
    for _ in range(200):
        mid = (lo + hi) / 2
        if (bisect.bisect_right(fit_sorted, mid) / L) ** n < q:
            lo = mid
        else:
            hi = mid
    return hi


@pytest.mark.parametrize("n", [1, 2, 7, 64])
def test_max_of_n_quantile_matches_bisection(n):
    rng = np.random.default_rng(n)
    fit = np.sort(rng.integers(0, 50, size=997).astype(np.float64))  # many ties
    for q in (0.01, 0.5, 0.9, 0.95, 0.99, 0.999):
        got = maxofn.predicted_max_quantile(fit, n, q)
        ref = bisection_quantile(fit.tolist(), n, q)
        assert got == pytest.approx(ref, abs=1e-9), (n, q, got, ref)


def test_heldout_independent_blocks(tmp_path):
    # iid U(0, 1) delays, 32 blocks: the model's median of the max is the
    # closed form 0.5^(1/32), and the held-out measurement agrees.
    rng = np.random.default_rng(11)
    events, blocks = 4000, 33  # block 0 = setter, dropped
    set_ns = np.arange(1, events + 1, dtype=np.int64) * 10_000_000
    obs = set_ns[:, None] + 1 + (rng.random((events, blocks)) * 1e6).astype(np.int64)
    p = tmp_path / "iid.obs1"
    common.write_obs1(p, set_ns, obs)
    d = common.delays_us(p, warmup=100)
    assert d.shape == (3900, 32)
    res = dict((q, (pr, me)) for q, pr, me in maxofn.heldout(d))
    assert res[0.5][0] == pytest.approx(1000 * 0.5 ** (1 / 32), rel=2e-3)
    for q, (pr, me) in res.items():
        assert me == pytest.approx(pr, rel=0.01), (q, pr, me)
    cors = maxofn.pair_correlations(d)
    assert len(cors) == 300 and max(abs(c) for c in cors) < 0.1


def test_heldout_correlated_blocks(tmp_path):
    # every block sees the same delay (fully correlated): the independence
    # model overpredicts the max, and the pair correlations are 1.
    rng = np.random.default_rng(5)
    events, blocks = 1000, 9
    set_ns = np.arange(1, events + 1, dtype=np.int64) * 10_000_000
    common_delay = (rng.random(events) * 1e6).astype(np.int64) + 1
    obs = set_ns[:, None] + np.repeat(common_delay[:, None], blocks, axis=1)
    p = tmp_path / "cor.obs1"
    common.write_obs1(p, set_ns, obs)
    d = common.delays_us(p, warmup=100)
    for q, pr, me in maxofn.heldout(d):
        assert pr > me
    cors = maxofn.pair_correlations(d)
    assert min(cors) == pytest.approx(1.0)
    lo, mid, hi = maxofn.block_medians(d)
    assert lo == mid == hi


def test_floor_check_and_visibility(tmp_path, capsys):
    events, blocks = 300, 4
    set_ns = np.arange(1, events + 1, dtype=np.int64) * 1_000_000
    delay = np.full((events, blocks), 500, dtype=np.int64)
    delay[:, 2] = 900
    delay[150, 3] = 2000   # two events over a 1.03 us bound
    delay[250, 0] = 2000
    delay[50, 1] = 99_000  # warm-up: ignored
    p = tmp_path / "floor.obs1"
    common.write_obs1(p, set_ns, set_ns[:, None] + delay)
    n, mx, over = maxofn.floor_check(common.delays_us(p, 100))
    assert (n, mx, over) == (200, 2.0, 1)  # block 0 (setter) dropped here
    # Dmax includes block 0: 198 events at 0.9, two at 2.0; p99 = sorted[198]
    assert visibility.dmax_quantiles(p, 100) == (0.9, 2.0)
    out = tmp_path / "vis.csv"
    assert visibility.main(["--run", f"MI355X:4:floor={p}", "--out", str(out)]) == 0
    assert out.read_text().splitlines() == [visibility.HEADER, "MI355X,4,floor,0.90,2.00,bin"]
    assert maxofn.main(["--floor", f"F={p}", "--part", f"P={p}",
                        "--out", str(tmp_path / "h.csv")]) == 0
    text = capsys.readouterr().out
    # the floor check drops the setter (block 0): only event 150 is over
    assert "F: n=200 absolute max 2.00 us, events over 1.03 us: 1" in text
    assert (tmp_path / "h.csv").read_text().splitlines()[0] == \
        "part,quantile,predicted_us,measured_us"


def test_rocm_smi_clock_parser():
    text = """
============================ ROCm System Management Interface ============================
================================ Current clock frequencies ================================
GPU[0]          : fclk clock level: 0: (1600Mhz)
GPU[0]          : mclk clock level: 0: (1900Mhz)
GPU[0]          : sclk clock level: 1: (2103Mhz)
GPU[0]          : socclk clock level: 0: (28Mhz)
GPU[1]          : sclk clock level: 0: (132Mhz)
============================================================================================
"""
    c = clock_readback.parse_rocm_smi(text)
    assert c[(0, "sclk")] == 2103 and c[(0, "mclk")] == 1900 and c[(0, "fclk")] == 1600
    assert c[(1, "sclk")] == 132
    assert clock_readback.parse_rocm_smi("no clocks here") == {}


def test_parse_rocm_smi_power():
    text = ("GPU[0]\t\t: Current Socket Graphics Package Power (W): 1198.0\n"
            "GPU[1]\t\t: Average Graphics Package Power (W): 301.5\n"
            "GPU[0]\t\t: Max Graphics Package Power (W): 1400.0\n"
            "GPU[0]\t\t: sclk clock level: 1: (1905Mhz)\n")
    c = clock_readback.parse_rocm_smi(text)
    assert c[(0, "power_w")] == 1198.0 and c[(1, "power_w")] == 301.5
    assert c[(0, "power_cap_w")] == 1400.0 and c[(0, "sclk")] == 1905


def test_default_load_is_a_built_binary_path():
    cmd = clock_readback.default_load(10.0)
    assert os.path.basename(cmd[0]) == "persistent"
    assert int(cmd[cmd.index("--passes") + 1]) >= 1000
    assert cmd[cmd.index("--verify") + 1] == "0"


def test_clock_readback_stops_its_load(tmp_path, capsys):
    """The load never outlives the read-back: past --max-seconds it is
    terminated, and the samples taken meanwhile are still reported."""
    smi = tmp_path / "fake-smi"
    smi.write_text("#!/bin/sh\necho 'GPU[0]\t\t: sclk clock level: 1: (1405Mhz)'\n"
                   "echo 'GPU[0]\t\t: mclk clock level: 0: (2000Mhz)'\n"
                   "echo 'GPU[0]\t\t: Current Socket Graphics Package Power (W): 990.0'\n")
    smi.chmod(0o755)
    pidfile = tmp_path / "pid"
    load = [sys.executable, "-c",
            f"import os, time; open({str(pidfile)!r}, 'w').write(str(os.getpid())); "
            "print('load up', flush=True); time.sleep(120)"]
    csv = tmp_path / "clk.csv"
    t0 = time.monotonic()
    rc = clock_readback.main(["--smi", str(smi), "--interval", "0.2", "--max-seconds", "2",
                              "--csv", str(csv), "--"] + load)
    assert time.monotonic() - t0 < 30
    assert rc == 0
    pid = int(pidfile.read_text())
    with pytest.raises(ProcessLookupError):
        for _ in range(50):  # reaped by the read-back; gone within a moment
            os.kill(pid, 0)
            time.sleep(0.1)
    out = capsys.readouterr()
    assert "load up" in out.out
    assert "sclk under load" in out.out and "median 1405" in out.out
    assert "package power under load" in out.out and "median 990" in out.out
    assert "stopped at the 2 s limit" in out.err
    rows = csv.read_text().splitlines()
    assert rows[0] == "t_s,mclk_mhz,power_w,sclk_mhz" and len(rows) > 3
