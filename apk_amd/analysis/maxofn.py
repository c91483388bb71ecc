"""Held-out max-of-N model and the every-event floor check, from OBS1
matrices (reference scripts/heldout_maxofn.py:12-96).

Model: if the N blocks' observation delays of one event were independent
draws from one marginal F, the latest observer would follow F^N. The first
half of the events fits F (the pooled per-block delays); the second half
tests it: predicted q-quantile of the max = the smallest fitted delay x with
F(x)^N >= q, against the measured nearest-rank q-quantile of the per-event
max. Per-block median delays and the correlation of 300 random block pairs
(Python's random.Random(21), as the reference draws them) say how far the
blocks are from independent.

Floor check: over every complete event of a no-work visibility run, the
largest delay and the number of events whose latest observer exceeds a
bound (default 1.03 us, the reference's one-timer-quantum bound; the device
clock here ticks at 10 ns, so the bound is a latency budget, not a quantum).

    python -m apk_amd.analysis.maxofn \
        --part MI355X-256=results/raw/obs_lat_b256.obs1 \
        --floor MI355X-256=results/raw/vis_floor.obs1 \
        --out results/summary/heldout_maxofn.csv
"""
import argparse
import os
import random
import sys

import numpy as np

from .common import delays_us, pct

QUANTILES = (0.5, 0.9, 0.95, 0.99)


def floor_check(d, bound_us=1.03):
    """(events, largest delay, events whose latest observer > bound_us)."""
    dmax = d.max(axis=1)
    return int(d.shape[0]), float(dmax.max()), int((dmax > bound_us).sum())


def predicted_max_quantile(fit_sorted, n_blocks, q):
    """Smallest x in the fitted sample with F(x)^n >= q, F the empirical CDF
    (count of fitted delays <= x over the sample size)."""
    L = fit_sorted.size
    # k = the smallest count with (k/L)^n >= q
    k = min(L, max(1, int(np.ceil(L * q ** (1.0 / n_blocks)))))
    while k > 1 and ((k - 1) / L) ** n_blocks >= q:
        k -= 1
    while k < L and (k / L) ** n_blocks < q:
        k += 1
    # F(fit_sorted[k-1]) >= k/L, and every smaller value has F <= (k-1)/L,
    # ties included, so this is the smallest x with F(x)^n >= q.
    return float(fit_sorted[k - 1])


def heldout(d, quantiles=QUANTILES):
    """Fit on the first half of the events, test on the second half.
    Returns [(q, predicted, measured)]."""
    n_blocks = d.shape[1]
    half = d.shape[0] // 2
    fit = np.sort(d[:half].ravel(), kind="stable")
    dmax_test = d[half:].max(axis=1)
    return [(q, predicted_max_quantile(fit, n_blocks, q), pct(dmax_test, q))
            for q in quantiles]


def block_medians(d):
    m = [pct(d[:, b], 0.5) for b in range(d.shape[1])]
    return min(m), pct(m, 0.5), max(m)


def pair_correlations(d, pairs=300, seed=21):
    rng = random.Random(seed)
    cors = []
    for _ in range(pairs):
        i, j = rng.sample(range(d.shape[1]), 2)
        xi, xj = d[:, i], d[:, j]
        si, sj = xi.std(), xj.std()
        if si * sj > 0:
            cors.append(float(((xi - xi.mean()) * (xj - xj.mean())).mean() / (si * sj)))
    return cors


def _named(s):
    name, _, path = s.partition("=")
    if not path:
        raise argparse.ArgumentTypeError(f"expected NAME=PATH, got {s!r}")
    return name, path


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--part", type=_named, action="append", default=[],
                    help="NAME=OBS1 latency matrix (held-out model)")
    ap.add_argument("--floor", type=_named, action="append", default=[],
                    help="NAME=OBS1 no-work visibility matrix (floor check)")
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--bound-us", type=float, default=1.03)
    ap.add_argument("--out", default="results/summary/heldout_maxofn.csv")
    a = ap.parse_args(argv)
    if not a.part and not a.floor:
        ap.error("give at least one --part or --floor")

    print("=== floor visibility: every-event check ===")
    for name, path in a.floor:
        n, mx, over = floor_check(delays_us(path, a.warmup), a.bound_us)
        print(f"{name}: n={n} absolute max {mx:.2f} us, events over {a.bound_us:.2f} us: {over}")

    out_rows = []
    print("=== held-out independence model (fit half A, test half B) ===")
    for name, path in a.part:
        d = delays_us(path, a.warmup)
        half = d.shape[0] // 2
        print(f"{name} (N={d.shape[1]}, fit n={half}, test n={d.shape[0] - half}):")
        for q, pr, me in heldout(d):
            print(f"  p{int(q * 100):02d}: predicted {pr:7.2f}  measured {me:7.2f}")
            out_rows.append(f"{name},{q},{pr:.2f},{me:.2f}")
        lo, mid, hi = block_medians(d)
        print(f"  per-block median delays: min {lo:.2f} p50 {mid:.2f} max {hi:.2f}")
        cors = pair_correlations(d)
        if cors:
            print(f"  pairwise corr, {len(cors)} pairs: min {min(cors):.3f} "
                  f"p50 {pct(cors, 0.5):.3f} max {max(cors):.3f}")
    if a.part:
        dname = os.path.dirname(a.out)
        if dname:
            os.makedirs(dname, exist_ok=True)
        with open(a.out, "w") as f:
            f.write("part,quantile,predicted_us,measured_us\n")
            f.write("".join(r + "\n" for r in out_rows))
        print(f"wrote {a.out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
