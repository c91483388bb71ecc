"""Visibility summary from OBS1 matrices (reference
scripts/make_visibility_summary.py:16-58): per run, the latest observer's
delay (Dmax: max over every block, the setter included) per complete event
past the warm-up, and its p50 / p99 over events. Every row is computed from
a matrix (source "bin"); the reference's rows transcribed from A10/A100 logs
have no counterpart here.

    python -m apk_amd.analysis.visibility \
        --run MI355X:256:floor=results/raw/vis_floor.obs1 \
        --run MI355X:256:loaded=results/raw/vis_loaded.obs1 \
        --out results/summary/visibility.csv
"""
import argparse
import os
import sys

from .common import delays_us, pct

HEADER = "part,blocks,variant,dmax_p50_us,dmax_p99_us,source"


def dmax_quantiles(path, warmup=100):
    d = delays_us(path, warmup, exclude_setter=False)
    if d.shape[0] == 0:
        raise ValueError(f"{path}: no complete events past warm-up {warmup}")
    dmax = d.max(axis=1)
    return pct(dmax, 0.5), pct(dmax, 0.99)


def _run(s):
    label, _, path = s.partition("=")
    parts = label.split(":")
    if not path or len(parts) != 3:
        raise argparse.ArgumentTypeError(f"expected PART:BLOCKS:VARIANT=PATH, got {s!r}")
    return parts[0], int(parts[1]), parts[2], path


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--run", type=_run, action="append", required=True)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--out", default="results/summary/visibility.csv")
    a = ap.parse_args(argv)
    lines = [HEADER]
    for part, blocks, variant, path in a.run:
        p50, p99 = dmax_quantiles(path, a.warmup)
        lines.append(f"{part},{blocks},{variant},{p50:.2f},{p99:.2f},bin")
    d = os.path.dirname(a.out)
    if d:
        os.makedirs(d, exist_ok=True)
    with open(a.out, "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))
    print(f"wrote {a.out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
