"""GPU parity of the preemptible persistent GEMM (apk_persistent_yield)
through the C ABI.

What is pinned, per run:
  * C after yields (checkpoint / re-fetch / restart, chunk or stage polls) is
    bit-identical to the same kernel with polling off, and to the oracle
    (VALU64: sequential fmaf chain bit for bit; MFMA128: float64 within
    rel-Frobenius 1e-5);
  * every completed task's device fingerprint equals the oracle's fingerprint
    of that tile in the unpreempted C -- so a corrupted resume in any pass is
    caught even though later passes overwrite C;
  * every urgent tile of every fired event is bit-identical to the same tile
    computed by the plain persistent GEMM (poison control: all differ);
  * exactly-once: each task id completes once, each fired event runs exactly
    its urgent tile count, each fired event has a claimant.
"""
import numpy as np
import pytest

import oracle
from gpu_util import dev, run_persistent, say

pytestmark = pytest.mark.gpu


class Job:
    def __init__(self, torch, apk, engine, M, N, K, kc, Mu, Nu, Ku, events, blocks,
                 passes, seed=21):
        self.t, self.apk, self.engine = torch, apk, engine
        g = apk.geometry(engine)
        self.g = g
        self.M, self.N, self.K, self.kc = M, N, K, kc
        self.Mu, self.Nu, self.Ku = Mu, Nu, Ku
        self.tiles = (M // g.tile_m) * (N // g.tile_n)
        self.U = (Mu // g.tile_m) * (Nu // g.tile_n)
        self.num_tasks = self.tiles * passes
        self.events, self.blocks = events, blocks
        self.A, self.B = oracle.fill_uniform_pm1(seed, M, N, K)
        self.Au = np.ascontiguousarray(self.A[:Mu, :Ku])
        self.Bu = np.ascontiguousarray(self.B[:Ku, :Nu])
        T = torch
        self.dA, self.dB = dev(T, self.A), dev(T, self.B)
        self.dAu, self.dBu = dev(T, self.Au), dev(T, self.Bu)
        self.dC = T.empty((M, N), dtype=T.float32, device="cuda")
        self.dCu = T.empty((Mu, Nu), dtype=T.float32, device="cuda")
        E = max(events, 1)
        i32, i64 = T.int32, T.int64
        self.nxt = T.zeros(apk.QUEUE_WORDS, dtype=i32, device="cuda")
        self.flag = T.zeros(apk.FLAG_MAX_COPIES * apk.FLAG_STRIDE // 4, dtype=i32, device="cuda")
        self.sched = T.zeros(E, dtype=i64, device="cuda")
        self.set_gt = T.zeros(E, dtype=i64, device="cuda")
        self.obs = T.zeros(E * blocks, dtype=i64, device="cuda")
        self.claim = T.zeros(E, dtype=i32, device="cuda")
        self.site = T.zeros(E, dtype=i32, device="cuda")
        self.u_gt = T.zeros(2 * E, dtype=i64, device="cuda")
        self.u_end = T.zeros(E, dtype=i64, device="cuda")
        self.uq = T.zeros(E, dtype=i32, device="cuda")
        self.ckpt = T.zeros(blocks * apk.ckpt_floats(engine), dtype=T.float32, device="cuda")
        self.task_hash = T.zeros(self.num_tasks, dtype=i64, device="cuda")
        self.u_hash = T.zeros(E * max(self.U, 1), dtype=i64, device="cuda")
        self.stats = T.zeros(blocks * apk.STATS_PER_BLOCK, dtype=i64, device="cuda")
        self.exec_count = T.zeros(self.num_tasks, dtype=i32, device="cuda")
        self.u_exec = T.zeros(E, dtype=i32, device="cuda")

    def run(self, poll, resume=0, gap_ticks=300, poison=0, use_oracle=False, events=None,
            copies=1, poll_every=1, naive=0):
        T, apk = self.t, self.apk
        ev = self.events if events is None else events
        for x in (self.nxt, self.flag, self.set_gt, self.obs, self.claim, self.u_gt,
                  self.u_end, self.uq, self.task_hash, self.u_hash, self.stats,
                  self.exec_count, self.u_exec):
            x.zero_()
        self.site.fill_(-1)
        self.dC.fill_(float("nan"))
        self.dCu.fill_(float("nan"))
        self.sched.copy_(T.arange(1, max(self.events, 1) + 1, dtype=T.int64, device="cuda") * gap_ticks)
        T.cuda.synchronize()
        p = apk.YieldParams()
        p.A, p.B, p.C = self.dA.data_ptr(), self.dB.data_ptr(), self.dC.data_ptr()
        p.M, p.N, p.K, p.k_chunk = self.M, self.N, self.K, self.kc
        p.num_tasks, p.next_task = self.num_tasks, self.nxt.data_ptr()
        p.Au, p.Bu, p.Cu = self.dAu.data_ptr(), self.dBu.data_ptr(), self.dCu.data_ptr()
        p.Mu, p.Nu, p.Ku = self.Mu, self.Nu, self.Ku
        p.uq_next = self.uq.data_ptr()
        p.flag, p.flag_copies, p.flag_system = self.flag.data_ptr(), copies, 0
        p.flag_set = self.flag.data_ptr() if ev > 0 else None
        p.sched = self.sched.data_ptr() if ev > 0 else None
        p.num_events, p.stop_after, p.poll_every = ev, 0, poll_every
        p.set_gt, p.obs_gt = self.set_gt.data_ptr(), self.obs.data_ptr()
        p.claim, p.claim_site = self.claim.data_ptr(), self.site.data_ptr()
        p.u_gt, p.u_end_max = self.u_gt.data_ptr(), self.u_end.data_ptr()
        p.resume, p.ckpt, p.poison, p.naive = resume, self.ckpt.data_ptr(), poison, naive
        p.task_hash, p.u_hash, p.stats = (self.task_hash.data_ptr(), self.u_hash.data_ptr(),
                                          self.stats.data_ptr())
        p.exec_count = self.exec_count.data_ptr() if use_oracle else None
        p.u_exec_count = self.u_exec.data_ptr() if use_oracle else None
        apk.persistent_yield(self.engine, poll, use_oracle, p, self.blocks,
                             T.cuda.current_stream().cuda_stream)
        T.cuda.synchronize()
        return {
            "C": self.dC.cpu().numpy(), "Cu": self.dCu.cpu().numpy(),
            "task_hash": self.task_hash.cpu().numpy().view(np.uint64),
            "u_hash": self.u_hash.cpu().numpy().view(np.uint64),
            "set_gt": self.set_gt.cpu().numpy()[:ev], "claim": self.claim.cpu().numpy()[:ev],
            "site": self.site.cpu().numpy()[:ev],
            "obs": self.obs.cpu().numpy()[:ev * self.blocks].reshape(max(ev, 0), self.blocks),
            "stats": self.stats.cpu().numpy().reshape(self.blocks, self.apk.STATS_PER_BLOCK),
            "exec": self.exec_count.cpu().numpy(), "u_exec": self.u_exec.cpu().numpy()[:ev],
        }

    def tile_hashes(self, C):
        g = self.g
        tn = self.N // g.tile_n
        return np.array([oracle.tile_hash(C, (t // tn) * g.tile_m, (t % tn) * g.tile_n,
                                          g.tile_m, g.tile_n) for t in range(self.tiles)],
                        dtype=np.uint64)

    def urgent_reference(self):
        C, _, _ = run_persistent(self.t, self.apk, self.engine, self.Au, self.Bu, self.Ku,
                                 blocks=4, with_log=False)
        g = self.g
        un = self.Nu // g.tile_n
        return C, np.array([oracle.tile_hash(C, (u // un) * g.tile_m, (u % un) * g.tile_n,
                                             g.tile_m, g.tile_n) for u in range(self.U)],
                           dtype=np.uint64)


def _bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def _blocks(apk, engine, poll, per_cu=1):
    return apk.device_info().cu_count * min(per_cu, apk.yield_occupancy(engine, poll))


@pytest.fixture(scope="module")
def mfma_job(torch_gpu, apk):
    say("building mfma128 yield job M=N=512 K=1024 kc=32")
    return Job(torch_gpu, apk, apk.ENGINE_MFMA128, 512, 512, 1024, 32, 256, 256, 256,
               events=40, blocks=_blocks(apk, apk.ENGINE_MFMA128, apk.POLL_STAGE), passes=64)


def _assert_run_exact(job, r, ref_C, ref_hashes, urgent_hashes):
    fired = int((r["set_gt"] != 0).sum())
    assert fired >= 5, f"only {fired} events fired"
    assert (_bits(r["C"]) == _bits(ref_C)).all(), "C differs from the unpreempted run"
    th = r["task_hash"]
    want = ref_hashes[np.arange(job.num_tasks) % job.tiles]
    assert (th == want).all(), f"{int((th != want).sum())} task fingerprints differ"
    ok = r["set_gt"] != 0
    assert (r["claim"][ok] > 0).all()
    uh = r["u_hash"][:len(r["set_gt"]) * job.U].reshape(-1, job.U)[ok]
    assert (uh == urgent_hashes[None, :]).all(), "urgent tile differs"
    assert int(r["stats"][:, 0].sum()) >= fired
    # blocks that drained the queue early may miss late events; the claimer never does
    assert (r["obs"][ok] > 0).any(axis=1).all()
    return fired


@pytest.mark.parametrize("poll,resume", [(2, 0), (2, 1), (2, 2), (1, 0)])
def test_mfma128_yield_bit_identical(torch_gpu, apk, mfma_job, poll, resume):
    say(f"mfma128 yield poll={poll} resume={resume}")
    j = mfma_job
    off = j.run(apk.POLL_OFF, events=0)
    ref_h = j.tile_hashes(off["C"])
    # device fingerprint definition == oracle's, on the unpreempted run
    assert (off["task_hash"] == ref_h[np.arange(j.num_tasks) % j.tiles]).all()
    ref64 = oracle.gemm_f64(j.A, j.B, threads=8)
    assert oracle.rel_frobenius(off["C"], ref64) <= 1e-5
    _, u_ref_h = j.urgent_reference()
    r = j.run(poll, resume=resume)
    fired = _assert_run_exact(j, r, off["C"], ref_h, u_ref_h)
    uref64 = oracle.gemm_f64(j.Au, j.Bu)
    assert oracle.rel_frobenius(r["Cu"], uref64) <= 1e-5
    say(f"  fired {fired} events, {int(r['stats'][:, 0].sum())} yields, bit-identical")


def test_mfma128_poison_is_detected(torch_gpu, apk, mfma_job):
    say("mfma128 poison control")
    j = mfma_job
    off = j.run(apk.POLL_OFF, events=0)
    _, u_ref_h = j.urgent_reference()
    r = j.run(apk.POLL_STAGE, resume=0, poison=1)
    ok = r["set_gt"] != 0
    uh = r["u_hash"][:len(r["set_gt"]) * j.U].reshape(-1, j.U)[ok]
    # staged B[0][col0] + 1.0 changes column 0 of every urgent tile
    assert (uh != u_ref_h[None, :]).all(), "poison not detected in some urgent tile"
    assert (_bits(r["C"]) == _bits(off["C"])).all()


def test_mfma128_oracle_exactly_once(torch_gpu, apk, mfma_job):
    say("mfma128 oracle")
    j = mfma_job
    r = j.run(apk.POLL_STAGE, resume=0, use_oracle=True)
    dup, missed, first_bad = oracle.count_tasks(r["exec"])
    assert (dup, missed) == (0, 0), first_bad
    fired_mask = r["set_gt"] != 0
    ok, fired, bad_u, uncl = oracle.count_events(r["set_gt"][fired_mask], r["u_exec"][fired_mask],
                                                 r["claim"][fired_mask], j.U)
    assert ok and fired >= 5 and bad_u == 0 and uncl == 0


def test_mfma128_task_start_sites(torch_gpu, apk):
    """Tasks two k-stages deep: a large share of the events arrive while
    blocks are between tasks, where a new generation is first seen at the
    task-start site (the flag sample taken with the task pop). Those sites
    must be taken, and the run must stay bit-identical and exactly-once."""
    say("mfma128 task-start sites: M=N=512 K=64 kc=32, 400 passes")
    E = apk.ENGINE_MFMA128
    j = Job(torch_gpu, apk, E, 512, 512, 64, 32, 256, 256, 64, events=40,
            blocks=_blocks(apk, E, apk.POLL_STAGE), passes=400)
    off = j.run(apk.POLL_OFF, events=0)
    assert oracle.rel_frobenius(off["C"], oracle.gemm_f64(j.A, j.B, threads=8)) <= 1e-5
    ref_h = j.tile_hashes(off["C"])
    _, u_ref_h = j.urgent_reference()
    for resume in (apk.RESUME_CKPT_FULL, apk.RESUME_CKPT_ACC, apk.RESUME_RESTART):
        r = j.run(apk.POLL_STAGE, resume=resume, use_oracle=True)
        fired = _assert_run_exact(j, r, off["C"], ref_h, u_ref_h)
        dup, missed, first_bad = oracle.count_tasks(r["exec"])
        assert (dup, missed) == (0, 0), first_bad
        starts = _stat(r, apk, apk.ST_START_SITES)
        say(f"  resume {resume}: fired {fired}, yields {_stat(r, apk, apk.ST_YIELDS)}, "
            f"generations first seen at a task start {starts}")
        assert starts > 0
    # the naive discipline keeps its checkpoints after the stage wait: no
    # task-start sites
    r = j.run(apk.POLL_STAGE, resume=apk.RESUME_CKPT_FULL, naive=1)
    assert _stat(r, apk, apk.ST_START_SITES) == 0


def test_valu64_yield_bit_exact_vs_fmaf_chain(torch_gpu, apk):
    say("valu64 yield M=N=256 K=256 kc=64 chunk polls, restart and ckpt")
    E = apk.ENGINE_VALU64
    j = Job(torch_gpu, apk, E, 256, 256, 256, 64, 64, 128, 64, events=30,
            blocks=_blocks(apk, E, apk.POLL_CHUNK, per_cu=2), passes=200)
    chain = oracle.gemm_f32_chain(j.A, j.B)
    ref_h = j.tile_hashes(chain)
    _, u_ref_h = j.urgent_reference()
    for resume in (0, 2):
        r = j.run(apk.POLL_CHUNK, resume=resume, gap_ticks=150)
        _assert_run_exact(j, r, chain, ref_h, u_ref_h)
    assert (_bits(j.urgent_reference()[0]) == _bits(oracle.gemm_f32_chain(j.Au, j.Bu))).all()


@pytest.mark.parametrize("poll_every,copies", [(4, 16), (2, 1)])
def test_mfma128_sparse_polls_and_flag_copies(torch_gpu, apk, mfma_job, poll_every, copies):
    say(f"mfma128 chunk polls every {poll_every}, {copies} flag copies")
    j = mfma_job
    off = j.run(apk.POLL_OFF, events=0)
    ref_h = j.tile_hashes(off["C"])
    _, u_ref_h = j.urgent_reference()
    r = j.run(apk.POLL_CHUNK, resume=0, copies=copies, poll_every=poll_every)
    _assert_run_exact(j, r, off["C"], ref_h, u_ref_h)
    # yields only at chunk boundaries (every poll_every-th one the block
    # passes, counted across its tasks)
    sites = r["site"][r["set_gt"] != 0]
    assert (sites % (j.kc // apk.geometry(j.engine).k_stage) == 0).all(), sites


def _stat(r, apk, col):
    return int(r["stats"][:, col].sum())


def test_mfma128_issue_site_drain(torch_gpu, apk, mfma_job):
    """Issue sites (checkpoint before any wait, then pop): with the drain the
    result stays bit-identical and no checkpoint is ever stale."""
    say("mfma128 issue-site yields, drain")
    j = mfma_job
    off = j.run(apk.POLL_OFF, events=0)
    ref_h = j.tile_hashes(off["C"])
    _, u_ref_h = j.urgent_reference()
    # Events far enough apart that a block is back at a site before the next
    # one: every observer checkpoints and restores (~10 us), and a block that
    # sees several new generations serves only the newest (src/yield.cu:155-183).
    r = j.run(apk.POLL_ISSUE, resume=apk.RESUME_CKPT_FULL, gap_ticks=2000, use_oracle=True)
    fired = _assert_run_exact(j, r, off["C"], ref_h, u_ref_h)
    dup, missed, _ = oracle.count_tasks(r["exec"])
    assert (dup, missed) == (0, 0)
    assert _stat(r, apk, apk.ST_STALE_ALL) == 0
    # every block that sees an event checkpoints at the issue site and resumes
    assert _stat(r, apk, apk.ST_CHECKPOINTS) >= fired
    assert _stat(r, apk, apk.ST_INFLIGHT) == _stat(r, apk, apk.ST_INFLIGHT_ALL)
    say(f"  fired {fired}, checkpoints {_stat(r, apk, apk.ST_CHECKPOINTS)}, in flight at the "
        f"drain {_stat(r, apk, apk.ST_INFLIGHT_ALL)}")


def test_mfma128_issue_site_naive_control(torch_gpu, apk, mfma_job):
    """Naive at issue sites: the checkpoint may capture a stage still in
    flight; a resumed task differs from the unpreempted tile only if a
    checkpoint it resumed from was observed stale (a task resumed stale twice
    differs once). Urgent tiles are never affected (their loads land after the
    stale ones)."""
    say("mfma128 issue-site yields, naive")
    j = mfma_job
    off = j.run(apk.POLL_OFF, events=0)
    ref_h = j.tile_hashes(off["C"])
    _, u_ref_h = j.urgent_reference()
    r = j.run(apk.POLL_ISSUE, resume=apk.RESUME_CKPT_FULL, gap_ticks=2000, naive=1)
    ok = r["set_gt"] != 0
    fired = int(ok.sum())
    assert fired >= 5
    uh = r["u_hash"][:len(r["set_gt"]) * j.U].reshape(-1, j.U)[ok]
    assert (uh == u_ref_h[None, :]).all(), "urgent tile differs"
    want = ref_h[np.arange(j.num_tasks) % j.tiles]
    bad = int((r["task_hash"] != want).sum())
    stale = _stat(r, apk, apk.ST_STALE)
    assert bad <= stale and (bad == 0) == (stale == 0), (bad, stale)
    assert stale == _stat(r, apk, apk.ST_STALE_ALL)  # every checkpoint is resumed
    say(f"  fired {fired}, checkpoints {_stat(r, apk, apk.ST_CHECKPOINTS)}, in flight "
        f"{_stat(r, apk, apk.ST_INFLIGHT_ALL)}, stale {_stat(r, apk, apk.ST_STALE_ALL)}, "
        f"stale resumed {stale} = corrupted tasks {bad}")
