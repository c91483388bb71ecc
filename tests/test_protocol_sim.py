"""CPU protocol simulator (apk_amd/bin/protocol_sim): the kernels' work
queue, resume ring and generation rules (apk_amd/csrc/protocol.hpp, compiled
here for the host) driven by std::thread blocks under random preemption.

Every arm and resume mode must pass its end checks (each task completed once
with the order-sensitive expected result, each fired event's urgent tiles
served once, the resume ring empty with nothing lost or refused), and each
planted protocol mistake must be caught by the check that names it."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SIM = os.path.join(ROOT, "apk_amd", "bin", "protocol_sim")
# A job that outlasts the events: 8192 tasks of 16 stages on 16 blocks.
JOB = ["--tiles-m", "16", "--tiles-n", "16", "--passes", "32", "--stages", "16",
       "--mean-gap-us", "100", "--events", "200", "--blocks", "16"]


def run(*args):
    assert os.access(SIM, os.X_OK), "apk_amd/bin/protocol_sim not built"
    r = subprocess.run([SIM] + JOB + [str(a) for a in args], capture_output=True, text=True,
                       timeout=120)
    line = r.stdout.strip().splitlines()[-1] if r.stdout.strip() else r.stderr
    fields = {k: int(v) for k, v in re.findall(r"([a-z]+(?: [a-z]+)?) (-?\d+)", line)}
    return r.returncode, line, fields


@pytest.mark.parametrize("arm", ["coop", "retreat"])
@pytest.mark.parametrize("resume", ["full", "acc", "restart"])
def test_protocol_passes(arm, resume):
    rc, line, f = run("--arm", arm, "--resume", resume, "--seed", 3)
    assert rc == 0, line
    assert line.startswith("PASS")
    fired = int(re.search(r"events fired=(\d+)", line).group(1))
    assert fired >= 20, line  # the job outlasted a good share of the events
    if arm == "retreat":
        n = int(re.search(r"retreats (\d+)", line).group(1))
        assert n > 0 and f"resumed {n}" in line, line
    else:
        assert int(re.search(r"yields (\d+)", line).group(1)) > 0, line


def test_retreat_quota_over_fewer_domains():
    """64 retreats per event over 16 domains (quota 4 per domain), 32 blocks."""
    rc, line, _ = run("--arm", "retreat", "--blocks", 32, "--retreat", 64, "--domains", 16,
                      "--seed", 5)
    assert rc == 0, line


@pytest.mark.parametrize("resume", ["full", "acc", "restart"])
def test_retreat_every_worker_many_events(resume):
    """Every one of 64 blocks retreats at each of up to 40 generations: whole
    grids reserve tickets together and whole continuations claim them
    together, the case a claim loop of compare-and-swaps serialised."""
    rc, line, f = run("--arm", "retreat", "--resume", resume, "--seed", 2, "--blocks", 64,
                      "--retreat", 64, "--passes", 32, "--events", 40, "--mean-gap-us", 500,
                      "--work-ns", 20000)
    assert rc == 0, line
    fired = int(re.search(r"events fired=(\d+)", line).group(1))
    n = int(re.search(r"retreats (\d+)", line).group(1))
    assert fired >= 20 and n >= 10 * 64 and f"resumed {n}" in line, line


def test_coop_poll_every_4():
    rc, line, _ = run("--arm", "coop", "--poll-every", 4, "--seed", 7)
    assert rc == 0, line


@pytest.mark.parametrize("bug,arm,extra,caught", [
    ("publish-early", "retreat", [], r"wrong [1-9]"),
    ("resume-skip", "retreat", [], r"wrong [1-9]"),
    ("resume-skip", "coop", [], r"wrong [1-9]"),
    ("no-release", "retreat", ["--cap", 16], r"refused [1-9]"),
    ("double-serve", "coop", [], r"urgent bad [1-9]"),
])
def test_planted_mistakes_are_caught(bug, arm, extra, caught):
    rc, line, _ = run("--arm", arm, "--bug", bug, "--seed", 11, *extra)
    assert rc == 1, line
    assert line.startswith("FAIL") and re.search(caught, line), line
