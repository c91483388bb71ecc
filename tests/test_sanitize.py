"""CPU sanitizer gate, the counterpart of the reference's `make sanitize`
(Makefile:33-38, compute-sanitizer memcheck over small configs of all five
binaries; GPU-side sanitizers are not available on this pool).

tests/native/Makefile builds, with g++ only:
  * the protocol simulator (apk_amd/sim/protocol_sim.cpp over the kernels'
    own queue and resume-ring code, apk_amd/csrc/protocol.hpp) under
    ThreadSanitizer and under AddressSanitizer + UBSan, run over the
    simulator's cases: both arms, every resume mode, rings smaller than one
    generation's retreats, every worker retreating at once;
  * the measurement binaries' host library (apk_amd/host/host_common.cpp)
    with the CPU oracle under AddressSanitizer + UBSan, whose self-test
    checks the two against each other exactly.
A run passes when the case passes and the sanitizer reports nothing; a
planted race (the simulator's publish-early mistake) must be reported by
ThreadSanitizer, so the gate is shown to see one."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NATIVE = os.path.join(ROOT, "tests", "native")
# One build folder per pytest-xdist worker: workers that rebuilt the same
# binaries at once ran a file another worker was still writing.
_WORKER = os.environ.get("PYTEST_XDIST_WORKER", "")
BUILD_NAME = "_build" + (f"_{_WORKER}" if _WORKER else "")
BUILD = os.path.join(NATIVE, BUILD_NAME)
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0",
           UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1",
           TSAN_OPTIONS="halt_on_error=0:exitcode=66")
# A job long enough for 40 generations at 0.5 ms on 16 blocks, short enough
# under the sanitizers' 5-15x slowdown. The ring's wait deadlines (20 ms in
# the kernels, there only to keep a stopped block from hanging the grid) are
# stretched to 2 s: under ThreadSanitizer, 32 threads on a few cores were
# seen to stall a consumer past 20 ms, and a deadline that runs out is
# reported as an error by design.
JOB = ["--tiles-m", "16", "--tiles-n", "16", "--passes", "32", "--stages", "16",
       "--mean-gap-us", "500", "--events", "40", "--blocks", "16", "--work-ns", "20000",
       "--rq-wait-us", "2000000"]


@pytest.fixture(scope="module")
def sanitized():
    r = subprocess.run(["make", "-s", "-C", NATIVE, "sanitize", f"B={BUILD_NAME}"],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    return BUILD


def run(path, args, timeout=300):
    r = subprocess.run([path] + [str(a) for a in args], capture_output=True, text=True,
                       env=ENV, timeout=timeout)
    return r.returncode, r.stdout, r.stderr


def clean(stderr):
    return not re.search(r"ERROR: AddressSanitizer|WARNING: ThreadSanitizer|runtime error:",
                         stderr)


def test_host_library_and_oracle_under_asan_ubsan(sanitized):
    rc, out, err = run(os.path.join(sanitized, "host_selftest_asan"), [])
    assert rc == 0 and clean(err), out[-2000:] + err[-4000:]
    assert out.startswith("PASS"), out


CASES = [
    ["--arm", "coop", "--resume", "full"],
    ["--arm", "coop", "--resume", "acc", "--poll-every", "4"],
    ["--arm", "retreat", "--resume", "full"],
    ["--arm", "retreat", "--resume", "acc"],
    ["--arm", "retreat", "--resume", "restart"],
    ["--arm", "retreat", "--resume", "full", "--retreat", 16, "--domains", 16, "--cap", 2],
    ["--arm", "retreat", "--resume", "restart", "--retreat", 16, "--domains", 16, "--cap", 3],
    ["--arm", "retreat", "--resume", "acc", "--blocks", 32, "--retreat", 32, "--cap", 8],
]


@pytest.mark.parametrize("san", ["tsan", "asan"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(str(x) for x in c[1::2]))
def test_protocol_simulator_sanitized(sanitized, san, case):
    # Every run must be clean and pass; a retreat case is run again (up to
    # four times) while a run had no retreat at all, which the host's thread
    # scheduling decides (tests/test_protocol_sim.py run_covering).
    for _ in range(4):
        rc, out, err = run(os.path.join(sanitized, f"protocol_sim_{san}"),
                           JOB + case + ["--seed", 4])
        assert clean(err), err[-6000:]
        assert rc == 0 and out.startswith("PASS"), out + err[-2000:]
        if "retreat" not in case:
            break
        n = int(re.search(r"retreats (\d+)", out).group(1))
        if n > 0:
            break
    if "retreat" in case:
        assert n > 0 and f"resumed {n}" in out, out


def test_tsan_sees_a_planted_race(sanitized):
    """publish-early writes the checkpoint slot after the entry is published:
    the consumer's read of the slot is then ordered by nothing, which
    ThreadSanitizer reports (and the end check sees as wrong results)."""
    rc, out, err = run(os.path.join(sanitized, "protocol_sim_tsan"),
                       JOB + ["--arm", "retreat", "--resume", "full", "--bug", "publish-early",
                              "--seed", 4])
    assert "WARNING: ThreadSanitizer: data race" in err, (rc, out, err[-2000:])
