"""GPU parity of the retreat arm through the C ABI: the background persistent
GEMM hands CUs to an urgent GEMM queued on a second stream.

Per run, on the urgent stream: apk_raise_flag -> apk_persistent_gemm (the
urgent job) -> a continuation relaunch of the preemptible kernel; on the
background stream: the preemptible kernel with retreat = R. ceil(R/32)
blocks in each (XCD, shader engine) domain checkpoint their tile into the
HBM resume queue and exit; the tiles are finished by whichever worker pops
them. Pinned:
  * C bit-identical to the unpreempted run, and every task's fingerprint
    equal to its tile's fingerprint in that run (fp32 MFMA128 and bf16);
  * exactly-once: every task id completed once, 32 * ceil(R/32) tickets
    reserved and popped, none left counted as unclaimed, no resume error --
    also with every worker retreating at once;
  * the urgent output bit-identical to the same GEMM run alone;
  * the device timeline is ordered: flag raised <= first checkpoint start
    <= last retreat exit.
"""
import numpy as np
import pytest

import oracle
from gpu_util import dev, say

pytestmark = pytest.mark.gpu


class _HipStream:
    """A non-blocking HIP stream of its own (hipStreamCreateWithFlags, default
    priority), as the measurement binaries use: the background and urgent
    kernels must sit on different hardware queues to run concurrently."""
    def __init__(self):
        import ctypes
        self._hip = ctypes.CDLL("libamdhip64.so")
        s = ctypes.c_void_p()
        rc = self._hip.hipStreamCreateWithFlags(ctypes.byref(s), ctypes.c_uint(1))
        assert rc == 0, f"hipStreamCreateWithFlags: {rc}"
        self.cuda_stream = s.value


_STREAMS = []


def _streams():
    """The background and urgent streams, created once per process: HIP maps
    streams onto a few hardware queues (4 here), so a fifth stream shares a
    queue with an earlier one and its work would wait behind that queue's
    kernels -- the urgent stream must keep a hardware queue of its own."""
    if not _STREAMS:
        _STREAMS.extend([_HipStream(), _HipStream()])
    return _STREAMS


class RetreatJob:
    def __init__(self, torch, apk, engine, M, N, K, kc, Mu, Nu, Ku, passes, retreat, seed=21,
                 cap=None):
        T = torch
        self.t, self.apk, self.engine = T, apk, engine
        g = apk.geometry(engine)
        self.g = g
        self.M, self.N, self.K, self.kc = M, N, K, kc
        self.Mu, self.Nu, self.Ku = Mu, Nu, Ku
        self.tiles = (M // g.tile_m) * (N // g.tile_n)
        self.U = (Mu // g.tile_m) * (Nu // g.tile_n)
        self.num_tasks = self.tiles * passes
        self.R = retreat
        D = apk.RETREAT_DOMAINS
        self.RB = D * ((retreat + D - 1) // D)
        self.cap = cap or self.RB  # resume ring entries
        self.blocks = apk.device_info().cu_count * min(
            1, apk.yield_occupancy(engine, apk.POLL_STAGE))
        if g.elem_bytes == 2:   # bf16 bit patterns; B passed transposed (N x K)
            A, _, B, _ = oracle.fill_normal_bf16(seed, M, N, K)
            Au, _, Bu, _ = oracle.fill_normal_bf16(seed + 1, Mu, Nu, Ku)
            self.dA = dev(T, A.view(np.int16))
            self.dB = dev(T, np.ascontiguousarray(B.T).view(np.int16))
            self.dAu = dev(T, Au.view(np.int16))
            self.dBu = dev(T, np.ascontiguousarray(Bu.T).view(np.int16))
        else:
            A, B = oracle.fill_uniform_pm1(seed, M, N, K)
            Au, Bu = oracle.fill_uniform_pm1(seed + 1, Mu, Nu, Ku)
            self.dA, self.dB = dev(T, A), dev(T, B)
            self.dAu, self.dBu = dev(T, Au), dev(T, Bu)
        i32, i64 = T.int32, T.int64
        self.dC = T.empty((M, N), dtype=T.float32, device="cuda")
        self.dCu = T.empty((Mu, Nu), dtype=T.float32, device="cuda")
        self.nxt = T.zeros(apk.QUEUE_WORDS, dtype=i32, device="cuda")
        self.unxt = T.zeros(apk.QUEUE_WORDS, dtype=i32, device="cuda")
        self.flag = T.zeros(apk.FLAG_STRIDE // 4, dtype=i32, device="cuda")
        self.set_gt = T.zeros(1, dtype=i64, device="cuda")
        # one event's retreats, then the first grid's registrations
        self.rcount = T.zeros(2 * apk.RETREAT_DOMAINS, dtype=i32, device="cuda")
        self.rgt = T.zeros(2, dtype=i64, device="cuda")
        self.rq_ctl = T.zeros(apk.RQ_CTL_WORDS, dtype=i32, device="cuda")
        self.rq_entry = T.zeros(4 * self.cap, dtype=i32, device="cuda")
        self.rq_slots = T.zeros(self.cap * apk.ckpt_floats(engine), dtype=T.float32,
                                device="cuda")
        rows = 2 * self.blocks + self.RB
        self.stats = T.zeros(rows * apk.STATS_PER_BLOCK, dtype=i64, device="cuda")
        self.task_hash = T.zeros(self.num_tasks, dtype=i64, device="cuda")
        self.exec_count = T.zeros(self.num_tasks, dtype=i32, device="cuda")
        self.run_gt = T.zeros(2, dtype=i64, device="cuda")
        self.exit_count = T.zeros(1, dtype=i32, device="cuda")
        self.bg, self.us = _streams()

    def params(self, poll_every, resume, continuation, block_base):
        apk = self.apk
        p = apk.YieldParams()
        p.A, p.B, p.C = self.dA.data_ptr(), self.dB.data_ptr(), self.dC.data_ptr()
        p.M, p.N, p.K, p.k_chunk = self.M, self.N, self.K, self.kc
        p.num_tasks, p.next_task = self.num_tasks, self.nxt.data_ptr()
        p.flag, p.flag_copies = self.flag.data_ptr(), 1
        p.num_events, p.poll_every, p.resume = 1, poll_every, resume
        p.task_hash, p.stats = self.task_hash.data_ptr(), self.stats.data_ptr()
        p.exec_count = self.exec_count.data_ptr()
        p.retreat, p.retreat_count, p.retreat_gt = self.R, self.rcount.data_ptr(), self.rgt.data_ptr()
        p.rq_ctl, p.rq_entry = self.rq_ctl.data_ptr(), self.rq_entry.data_ptr()
        p.rq_slots, p.rq_capacity = self.rq_slots.data_ptr(), self.cap
        p.continuation, p.block_base = continuation, block_base
        if not continuation:
            p.run_gt, p.exit_count = self.run_gt.data_ptr(), self.exit_count.data_ptr()
        return p

    def reset(self):
        for x in (self.nxt, self.unxt, self.flag, self.set_gt, self.rcount, self.rq_ctl,
                  self.rq_entry, self.stats, self.task_hash, self.exec_count, self.run_gt,
                  self.exit_count):
            x.zero_()
        # resume ring: entry i starts free for ticket i (seq = i)
        self.rq_entry.view(self.cap, 4)[:, 2] = self.t.arange(self.cap, dtype=self.t.int32,
                                                              device="cuda")
        self.rgt[0] = np.iinfo(np.int64).max
        self.rgt[1] = 0
        self.dC.fill_(float("nan"))
        self.dCu.fill_(float("nan"))
        self.t.cuda.synchronize()

    def run(self, poll, resume, poll_every=1, preempt=True):
        T, apk = self.t, self.apk
        self.reset()
        say(f"retreat run engine={self.engine} poll={poll} resume={resume} preempt={preempt}")
        apk.persistent_yield(self.engine, poll, True, self.params(poll_every, resume, 0, 0),
                             self.blocks, self.bg.cuda_stream)
        if preempt:
            apk.raise_flag(self.flag.data_ptr(), 1, 1, self.set_gt.data_ptr(), self.us.cuda_stream)
            apk.persistent_gemm(self.engine, self.dAu.data_ptr(), self.dBu.data_ptr(),
                                self.dCu.data_ptr(), self.Mu, self.Nu, self.Ku, self.Ku,
                                self.unxt.data_ptr(), None, self.U, self.us.cuda_stream)
            apk.persistent_yield(self.engine, poll, True,
                                 self.params(poll_every, resume, 1, self.blocks),
                                 self.RB, self.us.cuda_stream)
        T.cuda.synchronize()
        late = 0
        ctl = self.rq_ctl.cpu().numpy()
        if ctl[1] > ctl[0]:   # a retreat after the continuation drained the queue
            late = 1
            apk.persistent_yield(self.engine, poll, True,
                                 self.params(poll_every, resume, 1, self.blocks + self.RB),
                                 self.blocks, self.bg.cuda_stream)
            T.cuda.synchronize()
        rows = 2 * self.blocks + self.RB
        return {
            "C": self.dC.cpu().numpy(), "Cu": self.dCu.cpu().numpy(),
            "task_hash": self.task_hash.cpu().numpy().view(np.uint64),
            "exec": self.exec_count.cpu().numpy(),
            "ctl": self.rq_ctl.cpu().numpy().view(np.uint32), "late": late,
            "set_gt": int(self.set_gt.cpu()[0]), "rgt": self.rgt.cpu().numpy(),
            "run_gt": self.run_gt.cpu().numpy(),
            "stats": self.stats.cpu().numpy().reshape(rows, apk.STATS_PER_BLOCK),
        }


def _bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def _check(job, ref, r):
    assert (_bits(r["C"]) == _bits(ref["C"])).all(), "C differs from the unpreempted run"
    want = ref["task_hash"][np.arange(job.num_tasks) % job.tiles]
    th = r["task_hash"]
    assert (th == want).all(), f"{int((th != want).sum())} task fingerprints differ"
    assert (r["exec"] == 1).all(), (f"exactly-once violated: {int((r['exec'] > 1).sum())} dup, "
                                   f"{int((r['exec'] == 0).sum())} missed")
    st = r["stats"]
    head, tail = int(r["ctl"][0]), int(r["ctl"][1])
    t0, t1 = (int(x) for x in r["run_gt"])
    assert t0 < r["set_gt"] < t1, (f"flag raised at {r['set_gt']} outside the background run "
                                   f"[{t0}, {t1}]: the two streams did not run concurrently")
    assert head == tail == job.RB, (head, tail, r["set_gt"] - t0, t1 - t0, r["rgt"] - t0)
    assert int(r["ctl"][2]) == 0, f"{int(r['ctl'][2])} reserved tickets left unclaimed"
    assert int(r["ctl"][3]) == 0, f"{int(r['ctl'][3])} reserved tickets left unreleased"
    assert int(st[:, 5].sum()) == job.RB and int(st[:, 6].sum()) == job.RB
    assert int(st[:, 7].sum()) == 0, "resume entries lost"
    assert r["set_gt"] > 0 and r["set_gt"] <= r["rgt"][0] <= r["rgt"][1]


@pytest.fixture(scope="module")
def fp32_job(torch_gpu, apk):
    say("building mfma128 retreat job M=N=1024 K=4096 kc=128, 16 passes")
    job = RetreatJob(torch_gpu, apk, apk.ENGINE_MFMA128, 1024, 1024, 4096, 128, 256, 256, 256,
                     passes=16, retreat=4)
    job.ref = job.run(apk.POLL_STAGE, apk.RESUME_CKPT_FULL, preempt=False)
    assert (job.ref["exec"] == 1).all()
    frob = oracle.rel_frobenius(job.ref["C"][:128],
                                oracle.gemm_f64_rows(job.dA[:128].cpu().numpy(),
                                                     job.dB.cpu().numpy(), 0, 128))
    assert frob <= 1e-5, frob
    from gpu_util import run_persistent
    job.uref, _, _ = run_persistent(torch_gpu, apk, apk.ENGINE_MFMA128, job.dAu.cpu().numpy(),
                                    job.dBu.cpu().numpy(), 256, blocks=4, with_log=False)
    return job


@pytest.mark.parametrize("poll,resume,pe", [(2, 0, 1), (2, 1, 1), (2, 2, 1), (1, 0, 1), (1, 0, 2)])
def test_retreat_bit_identical_exactly_once(fp32_job, apk, poll, resume, pe):
    r = fp32_job.run(poll, resume, poll_every=pe)
    _check(fp32_job, fp32_job.ref, r)
    assert (_bits(r["Cu"]) == _bits(fp32_job.uref)).all(), "urgent output differs"


def test_retreat_bf16(torch_gpu, apk):
    say("building bf16x256 retreat job M=N=1024 K=2048 kc=256")
    job = RetreatJob(torch_gpu, apk, apk.ENGINE_BF16X256, 1024, 1024, 2048, 256, 256, 256, 256,
                     passes=512, retreat=2)
    ref = job.run(apk.POLL_STAGE, apk.RESUME_CKPT_FULL, preempt=False)
    for resume in (apk.RESUME_CKPT_FULL, apk.RESUME_CKPT_ACC):
        _check(job, ref, job.run(apk.POLL_STAGE, resume))


@pytest.mark.parametrize("resume", [1, 2])
def test_retreat_every_worker(torch_gpu, apk, resume):
    """Every worker retreats at once (retreat = the grid): 256 tickets reserved
    together, then claimed together by the 256-block continuation."""
    say(f"building mfma128 mass-retreat job M=N=1024 K=4096 kc=128, resume={resume}")
    blocks = apk.device_info().cu_count
    job = RetreatJob(torch_gpu, apk, apk.ENGINE_MFMA128, 1024, 1024, 4096, 128, 256, 256, 256,
                     passes=16, retreat=blocks)
    ref = job.run(apk.POLL_STAGE, apk.RESUME_CKPT_FULL, preempt=False)
    r = job.run(apk.POLL_STAGE, resume)
    assert (_bits(r["C"]) == _bits(ref["C"])).all(), "C differs from the unpreempted run"
    assert (r["exec"] == 1).all(), "exactly-once violated"
    head, tail, left, held = (int(x) for x in r["ctl"])
    st = r["stats"]
    assert head == tail and left == 0 and held == 0, (head, tail, left, held)
    # every block on a CU of its own, 8 per (XCD, shader engine) domain: all retreat
    assert tail == job.RB == blocks, (tail, job.RB)
    assert int(st[:, 5].sum()) == tail and int(st[:, 6].sum()) == tail
    assert int(st[:, 7].sum()) == 0, "resume entries lost"


@pytest.mark.parametrize("resume", [1, 2])
def test_retreat_ring_smaller_than_a_generation(torch_gpu, apk, resume):
    """Every worker asks to retreat at once into a ring of 64 entries: the
    ring admits as many retreats as it has entries free and declines the rest
    before they take a ticket (the declining block keeps its tile), so nothing
    is lost -- C bit-identical, every task once, every ticket claimed and
    released, no resume error."""
    say(f"building mfma128 small-ring retreat job M=N=1024 K=4096 kc=128, cap 64, resume={resume}")
    blocks = apk.device_info().cu_count
    job = RetreatJob(torch_gpu, apk, apk.ENGINE_MFMA128, 1024, 1024, 4096, 128, 256, 256, 256,
                     passes=16, retreat=blocks, cap=64)
    ref = job.run(apk.POLL_STAGE, apk.RESUME_CKPT_FULL, preempt=False)
    r = job.run(apk.POLL_STAGE, resume)
    assert (_bits(r["C"]) == _bits(ref["C"])).all(), "C differs from the unpreempted run"
    assert (r["exec"] == 1).all(), (f"exactly-once violated: {int((r['exec'] > 1).sum())} dup, "
                                   f"{int((r['exec'] == 0).sum())} missed")
    want = ref["task_hash"][np.arange(job.num_tasks) % job.tiles]
    assert (r["task_hash"] == want).all(), "task fingerprints differ"
    head, tail, left, held = (int(x) for x in r["ctl"])
    st = r["stats"]
    retreats, declined = int(st[:, apk.ST_RETREATS].sum()), int(st[:, apk.ST_DECLINED].sum())
    say(f"retreats {retreats} declined {declined} tickets {tail}")
    assert head == tail == retreats and left == 0 and held == 0, (head, tail, left, held)
    assert int(st[:, apk.ST_RESUMED].sum()) == retreats
    assert int(st[:, apk.ST_ERRORS].sum()) == 0, "resume-ring wait ran out"
    assert retreats >= 64 and declined > 0 and retreats + declined == blocks, (retreats, declined)
