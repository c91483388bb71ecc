"""Observation spread of the flag across resident blocks, per event.

Reads the latency CSVs that `yield --mode latency --csv` writes (header
"event,set_ns,first_obs_ns,last_obs_ns,lat_us,spread_us,...", the
reference's src/yield.cu:886-888) for a grid of block counts and poll
periods, and reports per cell the spread (last observer - first observer)
p50/p95/p99 and the first-observer delay p50/p99 over complete events past
the warm-up, as the reference's scripts/reanalyze_spread.py:23-75 does.

Every row is also checked against the identity lat = first + spread: the
three columns derive from the same three timestamps, so they differ only by
the CSV's 0.01 us rounding of lat_us and spread_us; a larger difference
means the CSV was written or parsed wrongly.

    python -m apk_amd.analysis.spread --raw results/raw \
        --blocks 32,64,128,256 --poll 1,2,4,8 \
        --out results/summary/spread_scaling.csv

Output is deterministic: sorted grid, fixed warm-up cut, nearest-rank
percentiles, fixed formatting.
"""
import argparse
import os
import sys

from .common import fmt, pct, ratio, read_rows

HEADER = ("blocks,poll_every,n,spread_p50_us,spread_p95_us,spread_p99_us,"
          "first_p50_us,first_p99_us")
IDENTITY_TOL_US = 0.02  # two values rounded to 0.01 us


class IdentityError(ValueError):
    pass


def analyse_rows(rows, warmup=100, where=""):
    """Summary of one latency CSV's rows: (n, spread p50, p95, p99, first p50,
    p99). Raises IdentityError when lat != first + spread beyond rounding."""
    kept = [r for r in rows if r["complete"] == "1" and int(r["event"]) >= warmup]
    if not kept:
        raise ValueError(f"{where}: no complete events past warm-up {warmup}")
    spread = [float(r["spread_us"]) for r in kept]
    first = [(int(r["first_obs_ns"]) - int(r["set_ns"])) / 1e3 for r in kept]
    lat = [float(r["lat_us"]) for r in kept]
    worst = max(abs(l - f - s) for l, f, s in zip(lat, first, spread))
    if worst >= IDENTITY_TOL_US:
        raise IdentityError(f"{where}: lat != first + spread by {worst:.4f} us")
    return (len(kept), pct(spread, 0.50), pct(spread, 0.95), pct(spread, 0.99),
            pct(first, 0.50), pct(first, 0.99))


def analyse(raw, blocks, polls, pattern, warmup=100):
    out = []
    for b in sorted(blocks):
        for p in sorted(polls):
            path = os.path.join(raw, pattern.format(b=b, p=p))
            if not os.path.exists(path):
                raise FileNotFoundError(path)
            out.append((b, p) + analyse_rows(read_rows(path), warmup, path))
    return out


def write_csv(path, rows):
    d = os.path.dirname(path)
    if d:
        os.makedirs(d, exist_ok=True)
    with open(path, "w") as f:
        f.write(HEADER + "\n")
        for r in rows:
            f.write(",".join(fmt(x) for x in r) + "\n")


def report(rows, blocks, polls):
    lines = [f"{'blocks':>6} {'poll':>4} | {'spr_p50':>7} {'spr_p95':>7} {'spr_p99':>7} "
             f"| {'first_p50':>9}"]
    for r in rows:
        lines.append(f"{r[0]:>6} {r[1]:>4} | {r[3]:>7.2f} {r[4]:>7.2f} {r[5]:>7.2f} "
                     f"| {r[6]:>9.2f}")
    cell = {(r[0], r[1]): r for r in rows}
    bs, ps = sorted(blocks), sorted(polls)
    p0, bmax = ps[0], bs[-1]
    lines.append("")
    lines.append(f"spread p50 growth with blocks (poll={p0}): " + " ".join(
        f"{ratio(cell[(bs[i + 1], p0)][3], cell[(bs[i], p0)][3]):.2f}x"
        for i in range(len(bs) - 1)))
    lines.append(f"spread p50 growth with poll period (blocks={bmax}): " + " ".join(
        f"{ratio(cell[(bmax, ps[i + 1])][3], cell[(bmax, ps[i])][3]):.2f}x"
        for i in range(len(ps) - 1)))
    return "\n".join(lines)


def _ints(s):
    return [int(x) for x in s.split(",") if x]


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--raw", default="results/raw")
    ap.add_argument("--blocks", type=_ints, default=[32, 64, 128, 256])
    ap.add_argument("--poll", type=_ints, default=[1, 2, 4, 8])
    ap.add_argument("--pattern", default="phase4_lat_b{b}_p{p}.csv")
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--out", default="results/summary/spread_scaling.csv")
    a = ap.parse_args(argv)
    try:
        rows = analyse(a.raw, a.blocks, a.poll, a.pattern, a.warmup)
    except FileNotFoundError as e:
        print(f"missing {e}: run from the directory holding the raw CSVs", file=sys.stderr)
        return 2
    except IdentityError as e:
        print(f"FAIL: {e}", file=sys.stderr)
        return 1
    write_csv(a.out, rows)
    print(report(rows, a.blocks, a.poll))
    print(f"\nwrote {a.out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
