"""CPU protocol simulator (apk_amd/bin/protocol_sim): the kernels' work
queue, resume ring and generation rules (apk_amd/csrc/protocol.hpp, compiled
here for the host) driven by std::thread blocks under random preemption.

Every arm and resume mode must pass its end checks (each task completed once
with the order-sensitive expected result, each fired event's urgent tiles
served once, the resume ring empty: every ticket claimed and released, no
wait run out), also with a ring smaller than one generation's retreats, where
retreats are declined ("refused") and nothing may be lost; and each planted
protocol mistake must be caught by the check that names it."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SIM = os.path.join(ROOT, "apk_amd", "bin", "protocol_sim")
SIM_BIN = SIM  # the sanitizer gate reruns these cases on instrumented builds
# A job that outlasts the events: 8192 tasks of 16 stages on 16 blocks.
JOB = ["--tiles-m", "16", "--tiles-n", "16", "--passes", "32", "--stages", "16",
       "--mean-gap-us", "100", "--events", "200", "--blocks", "16"]


def run(*args, sim=None, job=True, timeout=120):
    sim = sim or SIM
    assert os.access(sim, os.X_OK), f"{sim} not built"
    r = subprocess.run([sim] + (JOB if job else []) + [str(a) for a in args],
                       capture_output=True, text=True, timeout=timeout)
    line = r.stdout.strip().splitlines()[-1] if r.stdout.strip() else r.stderr
    fields = {k: int(v) for k, v in re.findall(r"([a-z]+(?: [a-z]+)?) (-?\d+)", line)}
    return r.returncode, line, fields


def deadline_ran_out(rc, f):
    """A ring wait that ran out ("stuck") fails the run by design. The
    simulator's blocks are host threads, which the OS can deschedule in the
    middle of a publish for longer than a short deadline (on the GPU a wave
    is never descheduled, and the kernels' deadline is 20 ms): such a run
    says nothing about the protocol and is run again."""
    return rc == 1 and f.get("stuck", 0) > 0


def run_covering(*args, cover, attempts=4, **kw):
    """Runs the simulator until a run also exercises the path under test
    (`cover(line, fields)`), at most `attempts` times; every run must pass
    its end checks, except one whose deadline the OS ran out. Whether a given
    run retreats or is refused at all also depends on the OS scheduler: two
    events the setter raises close together can both land before the first
    grid reaches a site, and the first grid retreats at generation 1 only (on
    the GPU the next flag is raised on the urgent stream behind the urgent
    GEMM, which needs the freed CUs, so generation 1 is never skipped
    there)."""
    for _ in range(attempts):
        rc, line, f = run(*args, **kw)
        if deadline_ran_out(rc, f):
            continue
        assert rc == 0 and line.startswith("PASS"), line
        if cover(line, f):
            return rc, line, f
    raise AssertionError(f"no run of {attempts} exercised the path: {line}")


def retreated(line, f):
    n = int(re.search(r"retreats (\d+)", line).group(1))
    return n > 0 and f"resumed {n}" in line


def refused(line, f):
    return f["refused"] > 0


@pytest.mark.parametrize("arm", ["coop", "retreat"])
@pytest.mark.parametrize("resume", ["full", "acc", "restart"])
def test_protocol_passes(arm, resume):
    def cover(line, f):
        # the job outlasted a good share of the events, and some retreated or yielded
        fired = int(re.search(r"events fired=(\d+)", line).group(1))
        if arm == "retreat":
            return fired >= 20 and retreated(line, f)
        return fired >= 20 and int(re.search(r"yields (\d+)", line).group(1)) > 0
    run_covering("--arm", arm, "--resume", resume, "--seed", 3, cover=cover)


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
    def many(line, f):
        fired = int(re.search(r"events fired=(\d+)", line).group(1))
        n = int(re.search(r"retreats (\d+)", line).group(1))
        return fired >= 20 and n >= 10 * 64 and f"resumed {n}" in line
    run_covering("--arm", "retreat", "--resume", resume, "--seed", 2, "--blocks", 64,
                 "--retreat", 64, "--passes", 32, "--events", 40, "--mean-gap-us", 500,
                 "--work-ns", 20000, cover=many)


def test_coop_poll_every_4():
    rc, line, _ = run("--arm", "coop", "--poll-every", 4, "--seed", 7)
    assert rc == 0, line


@pytest.mark.parametrize("bug,arm,extra,caught", [
    ("publish-early", "retreat", [], r"wrong [1-9]"),
    ("resume-skip", "retreat", [], r"wrong [1-9]"),
    ("resume-skip", "coop", [], r"wrong [1-9]"),
    ("no-release", "retreat", ["--cap", 16], r"unreleased [1-9]"),
    # tasks of 320 us and a 50 us ring deadline: without the occupancy gate a
    # producer past the ring's capacity waits for a consumer's next task
    # boundary and times out holding a ticket (the hole); the gated ring
    # passes the same job (test_gate_passes_where_no_gate_leaves_a_hole)
    ("no-gate", "retreat", ["--cap", 2, "--retreat", 16, "--domains", 16, "--rq-wait-us", 50,
                            "--work-ns", 20000], r"ring left [1-9]"),
    ("double-serve", "coop", [], r"urgent bad [1-9]"),
])
def test_planted_mistakes_are_caught(bug, arm, extra, caught):
    # A run whose threads never reach the planted step (no retreat, say: see
    # run_covering) passes; one of four must reach it and be caught.
    for _ in range(4):
        rc, line, _ = run("--arm", arm, "--bug", bug, "--seed", 11, *extra)
        if rc != 0:
            break
    assert rc == 1, line
    assert line.startswith("FAIL") and re.search(caught, line), line


def test_gate_passes_where_no_gate_leaves_a_hole():
    """The planted no-gate job with the ring as built: the same 50 us
    deadline, 320 us tasks and 2-entry ring, and every task completes once
    with the ring left empty."""
    # 50 us is short enough for the OS to run it out on a busy host: up to
    # eight runs
    rc, line, f = run_covering("--arm", "retreat", "--seed", 11, "--cap", 2, "--retreat", 16,
                               "--domains", 16, "--rq-wait-us", 50, "--work-ns", 20000,
                               cover=retreated, attempts=8)
    assert f["miss"] == 0 and f["lost"] == 0 and f["ring left"] == 0 and f["stuck"] == 0, line


@pytest.mark.parametrize("resume", ["full", "acc", "restart"])
@pytest.mark.parametrize("cap", [2, 3])
def test_retreat_ring_smaller_than_a_generation(resume, cap):
    """16 retreats per generation into a ring of 2 or 3 entries: the ring
    declines retreats once it holds `cap` unreleased tickets (the block keeps
    its tile), and every task still completes exactly once with nothing lost,
    stuck, unclaimed or unreleased. The urgent kernel holds the freed CUs for
    2 ms, so that the generation's retreats reach the ring before the
    continuation claims any (on a loaded host they trickle in otherwise)."""
    rc, line, f = run_covering("--arm", "retreat", "--resume", resume, "--retreat", 16,
                               "--domains", 16, "--cap", cap, "--seed", 4, "--urgent-us", 2000,
                               cover=lambda line, f: refused(line, f) and retreated(line, f))
    assert f["miss"] == 0 and f["lost"] == 0 and f["ring left"] == 0, line
    assert f["stuck"] == 0 and f["unreleased"] == 0, line


@pytest.mark.parametrize("extra", [
    # a full ring while tiles are long (12 ms stages): one refusal per job
    ["--retreat", 4, "--domains", 4, "--work-ns", 12000000],
    # more retreats per generation than domains hold blocks
    ["--retreat", 6, "--domains", 2, "--work-ns", 8000000],
])
def test_retreat_full_ring_long_tiles(extra):
    """Small jobs whose ring fills while every other block is deep in a long
    tile: a declined retreat used to strand a later published ticket."""
    rc, line, f = run_covering("--arm", "retreat", "--resume", "full", "--blocks", 8, "--cap", 2,
                               "--tiles-m", 4, "--tiles-n", 4, "--passes", 4, "--stages", 4,
                               "--events", 4, "--mean-gap-us", 30000, "--seed", 1, *extra,
                               job=False, cover=refused)
    assert f["miss"] == 0 and f["lost"] == 0 and f["ring left"] == 0, line


def test_ring_of_one_entry_is_rejected():
    """With one entry, "published by ticket t" and "free for ticket t + 1"
    are the same sequence number: the simulator refuses it, as the C ABI does."""
    rc, line, _ = run("--arm", "retreat", "--cap", 1)
    assert rc == 2 and "bad configuration" in line, line


@pytest.mark.parametrize("seed", [6, 7])
def test_retreat_short_ring_waits(seed):
    """The ring's deadlines cut to 2 ms (the kernels use 20 ms): with the
    occupancy gate every wait ends on other blocks' progress, so nothing runs
    out. Six blocks, so that the threads fit the host's cores and none is
    descheduled for milliseconds in the middle of a publish (on the GPU a wave
    is never descheduled; on an oversubscribed CPU a 2 ms deadline can expire
    on the OS scheduler alone)."""
    rc, line, f = run_covering("--arm", "retreat", "--resume", "full", "--blocks", 6,
                               "--retreat", 6, "--domains", 6, "--cap", 2, "--seed", seed,
                               "--rq-wait-us", 2000, cover=refused, attempts=8)
    assert f["stuck"] == 0 and f["lost"] == 0, line
