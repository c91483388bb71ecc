"""Engine clock read back while a GEMM load runs (the read-back half of the
reference's scripts/lock_clocks.sh:15-25).

The reference locks the SM clock with nvidia-smi and then reads it back
under load, because a lock is only evidence once it holds under load. On
MI355X the counterpart of the lock is rocm-smi's performance determinism
mode, which needs root; without it the engine clock follows power from one
dispatch to the next. This script does not change any GPU setting: it runs
a load (by default the persistent fp32 MFMA GEMM at 8192^3 for a few
seconds, whose last pass also prints the clock read on the device by
apk_clock_probe) and samples `rocm-smi --showclocks --showpower` every
--interval seconds meanwhile, then prints each sample and the min / median
/ max of the engine clock (sclk) and of the package power seen while the
load ran, beside the power cap (`--showmaxpower`): a clock that sags while
the power sits at the cap is power-bound.

    python -m apk_amd.analysis.clock_readback --seconds 10 --csv clock.csv
    python -m apk_amd.analysis.clock_readback -- apk_amd/bin/tcyield --mode calibrate ...
"""
import argparse
import os
import re
import shutil
import signal
import subprocess
import sys
import tempfile
import time

from .common import pct

_HERE = os.path.dirname(os.path.abspath(__file__))
BIN_DIR = os.path.join(os.path.dirname(_HERE), "bin")

# "GPU[0]          : sclk clock level: 1: (2100Mhz)" and the like: the clock
# name, then the first "(<n>Mhz)" or "<n> MHz" on the line.
_CLOCK_LINE = re.compile(r"GPU\[(\d+)\][^:]*:\s*(\w+)\b.*?\(?\s*(\d+(?:\.\d+)?)\s*M[Hh]z\)?")


# "GPU[0]          : Current Socket Graphics Package Power (W): 845.0",
# "... Average Graphics Package Power (W): 845.0", "... Max Graphics Package
# Power (W): 1400.0".
_POWER_LINE = re.compile(r"GPU\[(\d+)\][^:]*:\s*(.*?Power)\s*\(W\):\s*(\d+(?:\.\d+)?)")


def parse_rocm_smi(text):
    """{(gpu, clock name): MHz} from `rocm-smi --showclocks` text, plus
    {(gpu, "power_w"): W} for a current or average package power line and
    {(gpu, "power_cap_w"): W} for a maximum one."""
    out = {}
    for line in text.splitlines():
        m = _POWER_LINE.search(line)
        if m:
            key = "power_cap_w" if "max" in m.group(2).lower() else "power_w"
            out[(int(m.group(1)), key)] = float(m.group(3))
            continue
        m = _CLOCK_LINE.search(line)
        if m:
            out[(int(m.group(1)), m.group(2).lower())] = float(m.group(3))
    return out


def default_load(seconds):
    """Persistent fp32 MFMA GEMM, 8192^3 per pass (~8.5 ms), enough passes
    for `seconds`; no verification, records to /dev/null."""
    passes = max(2, int(seconds / 0.0085))
    return [os.path.join(BIN_DIR, "persistent"), "--engine", "mfma128", "--tiles-m", "64",
            "--tiles-n", "64", "--gemm-k", "8192", "--k", "128", "--passes", str(passes),
            "--verify", "0", "--csv", "/dev/null"]


def sample(smi, what=("--showclocks", "--showpower")):
    r = subprocess.run([smi, *what], capture_output=True, text=True, timeout=30)
    return r.returncode, parse_rocm_smi(r.stdout), r.stdout + r.stderr


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--seconds", type=float, default=10.0)
    ap.add_argument("--interval", type=float, default=0.5)
    ap.add_argument("--max-seconds", type=float, default=0,
                    help="stop the load after this long (default 3 x --seconds + 30)")
    ap.add_argument("--gpu", type=int, default=0)
    ap.add_argument("--csv", default="")
    ap.add_argument("--smi", default="", help="rocm-smi executable (default: on PATH)")
    ap.add_argument("load", nargs="*", help="load command (default: persistent mfma128 8192^3)")
    a = ap.parse_args(argv)

    smi = a.smi or shutil.which("rocm-smi") or "/opt/rocm/bin/rocm-smi"
    if not os.path.exists(smi):
        print("rocm-smi not found: no read-back", file=sys.stderr)
        return 2
    rc, _, text = sample(smi)
    print("--- idle read-back ---")
    print(text.strip())
    if rc != 0:
        print(f"rocm-smi exited {rc}: read-back denied on this host", file=sys.stderr)
        return 2
    _, cap, _ = sample(smi, ("--showmaxpower",))
    cap_w = cap.get((a.gpu, "power_cap_w"))

    cmd = a.load or default_load(a.seconds)
    limit = a.max_seconds if a.max_seconds > 0 else 3 * a.seconds + 30
    print("--- load: " + " ".join(cmd) + " ---", flush=True)
    # The load's output goes to a file (a pipe could fill and stall it), and
    # the load never outlives this script: stopped at the limit, and on
    # SIGTERM (e.g. from `timeout`) as on any other exit.
    log = tempfile.TemporaryFile(mode="w+")
    load = subprocess.Popen(cmd, stdout=log, stderr=subprocess.STDOUT, text=True)
    prev_term = signal.signal(signal.SIGTERM, lambda *_: sys.exit(143))
    rows = []
    stopped = False
    try:
        t0 = time.monotonic()
        time.sleep(min(1.0, a.interval * 2))  # past the load's set-up
        while load.poll() is None:
            rc, clocks, _ = sample(smi)
            t = time.monotonic() - t0
            if rc == 0 and clocks:
                rows.append((t, clocks))
                print(f"t={t:6.2f} s  " + "  ".join(
                    f"{name}={v:.0f}" for (g, name), v in sorted(clocks.items())
                    if g == a.gpu), flush=True)
            if t > limit:
                stopped = True
                load.terminate()
                break
            time.sleep(a.interval)
    finally:
        if load.poll() is None:
            load.terminate()
            try:
                load.wait(10)
            except subprocess.TimeoutExpired:
                load.kill()
                load.wait()
        signal.signal(signal.SIGTERM, prev_term)
    log.seek(0)
    lines = log.read().strip().splitlines()
    print("--- load output (first and last lines) ---")
    print("\n".join(lines[:6] + (["..."] if len(lines) > 14 else []) + lines[-8:]))
    if stopped:
        print(f"load stopped at the {limit:.0f} s limit", file=sys.stderr)
    elif load.returncode != 0:
        print(f"load exited {load.returncode}", file=sys.stderr)
        return load.returncode

    sclk = [c[(a.gpu, "sclk")] for _, c in rows if (a.gpu, "sclk") in c]
    if a.csv:
        names = sorted({k[1] for _, c in rows for k in c if k[0] == a.gpu})
        with open(a.csv, "w") as f:
            f.write("t_s," + ",".join(n if n.startswith("power") else f"{n}_mhz"
                                      for n in names) + "\n")
            for t, c in rows:
                f.write(f"{t:.3f}," + ",".join(
                    f"{c[(a.gpu, n)]:.0f}" if (a.gpu, n) in c else "" for n in names) + "\n")
    if not sclk:
        print("no sclk sample under load", file=sys.stderr)
        return 1
    print(f"sclk under load ({len(sclk)} samples): min {min(sclk):.0f} | median "
          f"{pct(sclk, 0.5):.0f} | max {max(sclk):.0f} MHz (not locked: determinism "
          f"mode needs root)")
    watts = [c[(a.gpu, "power_w")] for _, c in rows if (a.gpu, "power_w") in c]
    if watts:
        print(f"package power under load ({len(watts)} samples): min {min(watts):.0f} | "
              f"median {pct(watts, 0.5):.0f} | max {max(watts):.0f} W | cap "
              + (f"{cap_w:.0f} W" if cap_w else "not reported"))
    return 0


if __name__ == "__main__":
    sys.exit(main())
