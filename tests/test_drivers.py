"""CPU checks of the sweep drivers (apk_amd/drivers/*.sh), the counterparts
of the reference's scripts/*.sh: each parses as bash, names only binaries
the Makefile builds, and passes only flags those binaries read; the CSV
paths are the reference's (results/raw/<phase>_...csv)."""
import glob
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRV = os.path.join(ROOT, "apk_amd", "drivers")
HOST = os.path.join(ROOT, "apk_amd", "host")
SCRIPTS = sorted(glob.glob(os.path.join(DRV, "*.sh")))


def flags_read_by_binaries():
    """Every "--flag" string literal in the host sources (parse_arg/parse_str
    names and the modes they compare against)."""
    found = set()
    for f in glob.glob(os.path.join(HOST, "*.cpp")):
        found |= set(re.findall(r'"(--[a-z0-9-]+)"', open(f).read()))
    return found


def test_drivers_exist():
    names = {os.path.basename(p) for p in SCRIPTS}
    for n in ("calibrate.sh", "phase2.sh", "phase3.sh", "phase4.sh", "phase5.sh", "pareto.sh",
              "analyze.sh", "profile.sh"):
        assert n in names


@pytest.mark.parametrize("path", SCRIPTS, ids=os.path.basename)
def test_driver_parses(path):
    r = subprocess.run(["bash", "-n", path], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


@pytest.mark.parametrize("path", [p for p in SCRIPTS if "$BIN/" in open(p).read()],
                         ids=os.path.basename)
def test_driver_binaries_and_flags(path):
    text = open(path).read()
    bins = set(re.findall(r'\$BIN/([a-z_]+)', text))
    built = {os.path.basename(p)[4:-4] for p in glob.glob(os.path.join(HOST, "bin_*.cpp"))}
    assert bins and bins <= built, (bins, built)
    known = flags_read_by_binaries()
    used = set(re.findall(r'(?<![\w-])(--[a-z][a-z0-9-]*)', text))
    assert used <= known, sorted(used - known)
    for csv in re.findall(r'--csv "([^"]+)"', text):
        assert csv.startswith("$RAW/") and csv.endswith(".csv"), csv


BIN = os.path.join(ROOT, "apk_amd", "bin")


@pytest.mark.parametrize("binary,args,needle", [
    ("persistent", ["--dtype", "bf16", "--engine", "mfma128"], "--dtype bf16 does not name"),
    ("tcyield", ["--dtype", "fp16"], "--dtype fp16 does not name"),
    ("midyield", ["--dtype", "bf16", "--engine", "valu64"], "--dtype bf16 does not name"),
    ("urgent_baseline", ["--dtype", "fp32", "--engine", "bf16x256"], "--dtype fp32 does not name"),
    ("persistent", ["--engine", "fp64"], "unknown --engine"),
])
def test_binaries_reject_bad_engine_flags(binary, args, needle):
    """--dtype picks the engine when --engine is absent (fp32: the binary's
    default, bf16: bf16x256); a --dtype that contradicts --engine, an
    unknown --dtype or engine is a bad flag: exit 1 before any GPU call (the
    reference returns 1 on bad flags, src/midyield.cu:378-381)."""
    path = os.path.join(BIN, binary)
    if not os.access(path, os.X_OK):
        pytest.skip("binaries not built (python -c 'import __graft_entry__ as g; g.build()')")
    r = subprocess.run([path] + args, capture_output=True, text=True, timeout=60)
    assert r.returncode == 1, (r.returncode, r.stdout[-500:], r.stderr[-500:])
    assert needle in r.stderr, r.stderr[-500:]
