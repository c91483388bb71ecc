"""Shared readers for the analysis modules: the nearest-rank percentile and
the OBS1 observation matrix."""
import csv
import math

import numpy as np

OBS1_MAGIC = 0x3153424F  # "OBS1" little-endian


def pct(values, q):
    """Nearest-rank percentile, v[min(int(q * n), n - 1)] of the sorted
    values (reference scripts/analyze_pareto.py:7-9; the binaries'
    percentile() in apk_amd/host/host_common.cpp uses the same rule)."""
    v = np.sort(np.asarray(values, dtype=np.float64), kind="stable")
    if v.size == 0:
        raise ValueError("percentile of an empty sample")
    return float(v[min(int(q * v.size), v.size - 1)])


def read_obs1(path):
    """OBS1 file: int64 little-endian {magic, events, blocks}, then
    set[events], then obs[events * blocks] (ns on the device clock; 0 = never
    observed). Layout of the reference's dump (src/yield.cu:452-466), which
    apk_amd/host/yield_rig.cpp dump_obs1 writes. Returns (set_ns, obs_ns)
    as int64 arrays of shapes (events,) and (events, blocks)."""
    raw = np.fromfile(path, dtype="<i8")
    if raw.size < 3 or raw[0] != OBS1_MAGIC:
        raise ValueError(f"{path}: not an OBS1 file")
    events, blocks = int(raw[1]), int(raw[2])
    if events < 0 or blocks <= 0 or raw.size != 3 + events + events * blocks:
        raise ValueError(f"{path}: {raw.size} words for {events} events x {blocks} blocks")
    set_ns = raw[3:3 + events].copy()
    obs = raw[3 + events:].reshape(events, blocks).copy()
    return set_ns, obs


def write_obs1(path, set_ns, obs_ns):
    """Inverse of read_obs1 (used to build test matrices)."""
    set_ns = np.asarray(set_ns, dtype="<i8")
    obs_ns = np.asarray(obs_ns, dtype="<i8")
    events, blocks = obs_ns.shape
    hdr = np.array([OBS1_MAGIC, events, blocks], dtype="<i8")
    with open(path, "wb") as f:
        f.write(hdr.tobytes())
        f.write(set_ns.tobytes())
        f.write(obs_ns.tobytes())


def delays_us(path, warmup=100, exclude_setter=True, require_complete=True):
    """Per-event observation delays (us) of an OBS1 matrix: events before
    `warmup` and unset events dropped, events with an unobserved block dropped
    when require_complete, and block 0 (the device setter) dropped when
    exclude_setter. Returns an (events_kept, blocks_kept) float64 array."""
    set_ns, obs = read_obs1(path)
    keep = np.arange(set_ns.size) >= warmup
    keep &= set_ns != 0
    if require_complete:
        keep &= (obs != 0).all(axis=1)
    lo = 1 if exclude_setter else 0
    return (obs[keep, lo:] - set_ns[keep, None]).astype(np.float64) / 1e3


def read_rows(path):
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def fmt(x):
    return f"{x:.3f}" if isinstance(x, float) else str(x)


def ratio(a, b):
    return a / b if b else math.nan
