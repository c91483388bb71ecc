"""GPU parity of the bf16 MFMA engines (v_mfma_f32_32x32x16_bf16, fp32
accumulation) through the C ABI: APK_ENGINE_BF16X256 (256x256 tile, 1 block
per CU), APK_ENGINE_BF16X128 (128x128 tile on one wave, 4 blocks per CU) and
APK_ENGINE_BF16X256X128 (256x128 tile, 2 blocks per CU) -- the occupancies at
which the 256x256 tile cannot run.

What is pinned:
  * operand/accumulator lane layouts: small-integer bf16 inputs make every
    product and partial sum exact in fp32, so C must equal the integer GEMM
    bit for bit (a wrong row/column/k mapping cannot pass);
  * numerics on normal(0,1) bf16 inputs (the reference's tcyield data,
    src/tcyield.cu:459-473): rel-Frobenius <= 1e-2 against float64 on the
    bf16-quantized inputs (the bf16 bar), and in practice far below;
  * determinism: the k order is fixed, so C is bit-identical for every
    k_chunk and worker count, and across the three engines;
  * the yield path: stage and chunk polls with checkpoint/resume give C
    bit-identical to the unpreempted run, and the oracle counts are exact.
B is passed transposed (Bt = N x K row-major): C = A . Bt^T.
"""
import numpy as np
import pytest

import oracle
from gpu_util import assert_queue_drained, dev, say

pytestmark = pytest.mark.gpu

ENGS = ["bf16x256", "bf16x128", "bf16x256x128"]


def tile_of(apk, eng):
    g = apk.geometry(eng)
    return g.tile_m, g.tile_n


def bits_of_small_ints(rng, shape, lo=-3, hi=3):
    """bf16 bit patterns of small integers (exact in bf16) and their values."""
    v = rng.integers(lo, hi + 1, size=shape).astype(np.float32)
    bits = (v.view(np.uint32) >> 16).astype(np.uint16)  # exact: low mantissa bits are 0
    assert oracle.bf16_to_f32(int(bits.flat[0])) == v.flat[0]
    return bits, v


def run_bf16(torch, apk, A_bits, Bt_bits, k_chunk, blocks=None, eng=None):
    M, K = A_bits.shape
    N = Bt_bits.shape[0]
    eng = apk.ENGINE_BF16X256 if eng is None else eng
    if blocks is None:
        blocks = apk.device_info().cu_count * apk.occupancy(eng)
    dA, dB = dev(torch, A_bits.view(np.int16)), dev(torch, Bt_bits.view(np.int16))
    dC = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    nxt = torch.zeros(apk.QUEUE_WORDS, dtype=torch.int32, device="cuda")
    apk.persistent_gemm(eng, dA.data_ptr(), dB.data_ptr(), dC.data_ptr(), M, N, K, k_chunk,
                        nxt.data_ptr(), None, blocks, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return dC.cpu().numpy(), nxt.cpu().numpy()


@pytest.mark.parametrize("name", ENGS)
@pytest.mark.parametrize("K", [64, 128, 192])
def test_bf16_layout_exact_small_integers(torch_gpu, apk, name, K):
    """Exact products and sums of small integers. K = 64 is one pair of the
    256x256 tile's 32-deep stages, whose deferred k-step (the pipelined pair)
    then runs only before the epilogue; 192, an odd number of its pairs."""
    eng = apk.ENGINES[name]
    TM, TN = tile_of(apk, eng)
    M, N = 2 * TM, TN
    say(f"{name} layout: small integers, M={M} N={N} K={K}")
    rng = np.random.default_rng(5)
    A_bits, A = bits_of_small_ints(rng, (M, K))
    Bt_bits, Bt = bits_of_small_ints(rng, (N, K))
    C, nxt = run_bf16(torch_gpu, apk, A_bits, Bt_bits, k_chunk=K, blocks=3, eng=eng)
    ref = (A.astype(np.int64) @ Bt.astype(np.int64).T).astype(np.float32)
    assert_queue_drained(nxt, (M // TM) * (N // TN), blocks=3)
    assert np.array_equal(C, ref)


@pytest.mark.parametrize("name", ENGS)
def test_bf16_normal_inputs_vs_float64(torch_gpu, apk, name):
    say(f"{name} numerics: normal(0,1) bf16, M=N=512 K=1024")
    eng = apk.ENGINES[name]
    M, N, K = 512, 512, 1024
    A_bits, A, B_bits, B = oracle.fill_normal_bf16(7, M, N, K)
    Bt_bits = np.ascontiguousarray(B_bits.T)
    C, _ = run_bf16(torch_gpu, apk, A_bits, Bt_bits, k_chunk=256, eng=eng)
    ref = oracle.gemm_f64(A, B, threads=8)
    rf = oracle.rel_frobenius(C, ref)
    say(f"  rel-Frobenius {rf:.3e}")
    assert rf <= 1e-2
    assert rf <= 1e-5  # fp32 accumulation of exact bf16 products


@pytest.mark.parametrize("name", ENGS)
def test_bf16_bit_identical_across_chunks_and_workers(torch_gpu, apk, name):
    say(f"{name} determinism across k_chunk and worker counts")
    eng = apk.ENGINES[name]
    M, N, K = 512, 512, 512
    A_bits, _, B_bits, _ = oracle.fill_normal_bf16(11, M, N, K)
    Bt_bits = np.ascontiguousarray(B_bits.T)
    C0, _ = run_bf16(torch_gpu, apk, A_bits, Bt_bits, k_chunk=32, blocks=1, eng=eng)
    for kc, blocks in ((512, None), (64, 3), (128, 2)):
        C1, _ = run_bf16(torch_gpu, apk, A_bits, Bt_bits, k_chunk=kc, blocks=blocks, eng=eng)
        assert np.array_equal(C0.view(np.uint32), C1.view(np.uint32)), (kc, blocks)


@pytest.mark.parametrize("K", [512, 192])
def test_bf16_engines_bit_identical(torch_gpu, apk, K):
    """The three bf16 tiles form every output's sum in the same k order (k
    steps of 16, ascending), so C is bit-identical across them; K = 192 is 3
    load regions of 64 for the 256x256 tile and 6 of 32 for the other two."""
    say(f"bf16x256 vs bf16x128 vs bf16x256x128, M=N=512 K={K}")
    A_bits, A, B_bits, B = oracle.fill_normal_bf16(13, 512, 512, K)
    Bt_bits = np.ascontiguousarray(B_bits.T)
    C = {name: run_bf16(torch_gpu, apk, A_bits, Bt_bits, k_chunk=K, blocks=3,
                        eng=apk.ENGINES[name])[0] for name in ENGS}
    for name in ENGS[1:]:
        assert np.array_equal(C[name].view(np.uint32), C["bf16x256"].view(np.uint32)), name
    assert oracle.rel_frobenius(C["bf16x256"], oracle.gemm_f64(A, B, threads=8)) <= 1e-5


def test_bf16_small_tiles_run_at_2_and_4_blocks_per_cu(apk):
    """The one-wave 128x128 tile's plain and yield kernels fit 4 blocks per CU
    (32 KiB of LDS per block, one wave per SIMD), the 256x128 tile's 2 (48 KiB,
    two waves per SIMD); the 256x256 tile fits one."""
    e128, e256 = apk.ENGINES["bf16x128"], apk.ENGINES["bf16x256"]
    e256x128 = apk.ENGINES["bf16x256x128"]
    assert apk.occupancy(e128) >= 4 and apk.occupancy(e256x128) >= 2
    for poll in (apk.POLL_OFF, apk.POLL_CHUNK, apk.POLL_STAGE, apk.POLL_ISSUE):
        assert apk.yield_occupancy(e128, poll) >= 4, poll
        assert apk.yield_occupancy(e256x128, poll) >= 2, poll
    assert apk.occupancy(e256) == 1


class Bf16Job:
    """Preemptible bf16 GEMM with an urgent bf16 job, all through the C ABI."""

    def __init__(self, torch, apk, M, N, K, kc, Mu, Nu, Ku, events, blocks, passes, seed=3,
                 eng=None):
        T = torch
        self.t, self.apk = torch, apk
        self.eng = apk.ENGINE_BF16X256 if eng is None else eng
        self.tm, self.tn = tile_of(apk, self.eng)
        self.M, self.N, self.K, self.kc = M, N, K, kc
        self.Mu, self.Nu, self.Ku = Mu, Nu, Ku
        self.tiles = (M // self.tm) * (N // self.tn)
        self.U = (Mu // self.tm) * (Nu // self.tn)
        self.num_tasks = self.tiles * passes
        self.events, self.blocks = events, blocks
        A_bits, self.A, B_bits, self.B = oracle.fill_normal_bf16(seed, M, N, K)
        self.Abits, self.Btbits = A_bits, np.ascontiguousarray(B_bits.T)
        Au_bits, self.Au, Bu_bits, self.Bu = oracle.fill_normal_bf16(seed + 1, Mu, Nu, Ku)
        self.Aubits, self.Bubits = Au_bits, np.ascontiguousarray(Bu_bits.T)
        self.dA, self.dB = dev(T, self.Abits.view(np.int16)), dev(T, self.Btbits.view(np.int16))
        self.dAu = dev(T, self.Aubits.view(np.int16))
        self.dBu = dev(T, self.Bubits.view(np.int16))
        self.dC = T.empty((M, N), dtype=T.float32, device="cuda")
        self.dCu = T.empty((max(events, 1), Mu, Nu), dtype=T.float32, device="cuda")
        E = max(events, 1)
        i32, i64 = T.int32, T.int64
        z = lambda n, t: T.zeros(n, dtype=t, device="cuda")
        self.nxt, self.uq = z(apk.QUEUE_WORDS, i32), z(E, i32)
        self.flag = z(apk.FLAG_MAX_COPIES * apk.FLAG_STRIDE // 4, i32)
        self.sched, self.set_gt, self.obs = z(E, i64), z(E, i64), z(E * blocks, i64)
        self.claim, self.site, self.u_gt, self.u_end = z(E, i32), z(E, i32), z(2 * E, i64), z(E, i64)
        self.ckpt = T.zeros(blocks * apk.ckpt_floats(self.eng), dtype=T.float32, device="cuda")
        self.task_hash, self.u_hash = z(self.num_tasks, i64), z(E * max(self.U, 1), i64)
        self.stats = z(blocks * apk.STATS_PER_BLOCK, i64)
        self.exec_count, self.u_exec = z(self.num_tasks, i32), z(E, i32)

    def run(self, poll, resume=0, gap_ticks=300, use_oracle=False, events=None, poll_every=1):
        T, apk = self.t, self.apk
        ev = self.events if events is None else events
        for x in (self.nxt, self.flag, self.set_gt, self.obs, self.claim, self.u_gt, self.u_end,
                  self.uq, self.task_hash, self.u_hash, self.stats, self.exec_count, self.u_exec):
            x.zero_()
        self.site.fill_(-1)
        self.dC.fill_(float("nan"))
        self.dCu.fill_(float("nan"))
        self.sched.copy_(T.arange(1, max(self.events, 1) + 1, dtype=T.int64, device="cuda")
                         * gap_ticks)
        T.cuda.synchronize()
        p = apk.YieldParams()
        p.A, p.B, p.C = self.dA.data_ptr(), self.dB.data_ptr(), self.dC.data_ptr()
        p.M, p.N, p.K, p.k_chunk = self.M, self.N, self.K, self.kc
        p.num_tasks, p.next_task = self.num_tasks, self.nxt.data_ptr()
        p.Au, p.Bu, p.Cu = self.dAu.data_ptr(), self.dBu.data_ptr(), self.dCu.data_ptr()
        p.Mu, p.Nu, p.Ku = self.Mu, self.Nu, self.Ku
        p.cu_event_stride = self.Mu * self.Nu
        p.uq_next = self.uq.data_ptr()
        p.flag, p.flag_copies, p.flag_system = self.flag.data_ptr(), 1, 0
        p.flag_set = self.flag.data_ptr() if ev > 0 else None
        p.sched = self.sched.data_ptr() if ev > 0 else None
        p.num_events, p.stop_after, p.poll_every = ev, 0, poll_every
        p.set_gt, p.obs_gt = self.set_gt.data_ptr(), self.obs.data_ptr()
        p.claim, p.claim_site = self.claim.data_ptr(), self.site.data_ptr()
        p.u_gt, p.u_end_max = self.u_gt.data_ptr(), self.u_end.data_ptr()
        p.resume, p.ckpt = resume, self.ckpt.data_ptr()
        p.task_hash, p.u_hash = self.task_hash.data_ptr(), self.u_hash.data_ptr()
        p.stats = self.stats.data_ptr()
        p.exec_count = self.exec_count.data_ptr() if use_oracle else None
        p.u_exec_count = self.u_exec.data_ptr() if use_oracle else None
        apk.persistent_yield(self.eng, poll, use_oracle, p, self.blocks,
                             T.cuda.current_stream().cuda_stream)
        T.cuda.synchronize()
        return {
            "C": self.dC.cpu().numpy(), "Cu": self.dCu.cpu().numpy()[:max(ev, 1)],
            "task_hash": self.task_hash.cpu().numpy().view(np.uint64),
            "set_gt": self.set_gt.cpu().numpy()[:ev], "claim": self.claim.cpu().numpy()[:ev],
            "site": self.site.cpu().numpy()[:ev],
            "stats": self.stats.cpu().numpy().reshape(self.blocks, apk.STATS_PER_BLOCK),
            "exec": self.exec_count.cpu().numpy(), "u_exec": self.u_exec.cpu().numpy()[:ev],
        }


# (engine, blocks per CU or a block count): the 256x256 tile on 64 workers,
# the 128x128 tile at 4 (and 2) blocks on every CU, the 256x128 tile at 2.
JOBS = [("bf16x256", 64), ("bf16x128", "2/CU"), ("bf16x128", "4/CU"), ("bf16x256x128", "2/CU")]


@pytest.fixture(scope="module", params=JOBS, ids=lambda j: f"{j[0]}-{j[1]}".replace("/", "per"))
def bf16_job(torch_gpu, apk, request):
    name, b = request.param
    eng = apk.ENGINES[name]
    blocks = b if isinstance(b, int) else apk.device_info().cu_count * int(b.split("/")[0])
    for poll in (apk.POLL_CHUNK, apk.POLL_STAGE):  # every worker resident
        assert apk.yield_occupancy(eng, poll) * apk.device_info().cu_count >= blocks
    TM, TN = tile_of(apk, eng)
    # 9 tasks per block: the job outlasts the 24 events the setter (block 0)
    # raises 3 us apart at its own poll sites.
    tiles = (512 // TM) * (512 // TN)
    passes = -(-9 * blocks // tiles)
    say(f"building {name} yield job M=N=512 K=1024 kc=64 on {blocks} blocks ({passes} passes), "
        "urgent 256x512x256")
    return Bf16Job(torch_gpu, apk, 512, 512, 1024, 64, 256, 512, 256, events=24, blocks=blocks,
                   passes=passes, eng=eng)


@pytest.mark.parametrize("poll,resume", [(2, 0), (2, 1), (2, 2), (1, 0)])
def test_bf16_yield_bit_identical(bf16_job, apk, poll, resume):
    j = bf16_job
    say(f"engine {j.eng} on {j.blocks} blocks: yield poll={poll} resume={resume}")
    ref = j.run(apk.POLL_OFF, events=0)
    r = j.run(poll, resume=resume)
    fired = int((r["set_gt"] != 0).sum())
    yields = int(r["stats"][:, 0].sum())
    assert fired == j.events and yields >= fired
    assert np.array_equal(r["C"].view(np.uint32), ref["C"].view(np.uint32))
    # every task's fingerprint equals its tile's fingerprint in the unpreempted C
    tn = j.N // j.tn
    th = np.array([oracle.tile_hash(ref["C"], (t // tn) * j.tm, (t % tn) * j.tn, j.tm, j.tn)
                   for t in range(j.tiles)], dtype=np.uint64)
    assert np.array_equal(r["task_hash"], th[np.arange(j.num_tasks) % j.tiles])
    # every claimed event's urgent output equals the non-preemptible urgent GEMM
    uref = run_bf16_urgent(j)
    for e in range(j.events):
        assert r["claim"][e] != 0
        assert np.array_equal(r["Cu"][e].view(np.uint32), uref.view(np.uint32)), e
    say(f"  fired {fired} events, {yields} yields, bit-identical")


def run_bf16_urgent(j):
    C, _ = run_bf16(j.t, j.apk, j.Aubits, j.Bubits, k_chunk=j.Ku, blocks=2, eng=j.eng)
    return C


def test_bf16_float64_and_oracle(bf16_job, apk):
    j = bf16_job
    say(f"engine {j.eng} on {j.blocks} blocks: stage yields, float64 check and exactly-once "
        "oracle")
    r = j.run(apk.POLL_STAGE, resume=0, use_oracle=True)
    ref = oracle.gemm_f64(j.A, j.B, threads=8)
    assert oracle.rel_frobenius(r["C"], ref) <= 1e-5
    assert (r["exec"] == 1).all()
    assert (r["u_exec"] == j.U).all()


@pytest.fixture(scope="module", params=ENGS)
def bf16_odd_job(torch_gpu, apk, request):
    # An odd number of pairs (each pair is one load region): 5 (sites 0, 2,
    # ..., 8), the urgent job 3.
    eng = apk.ENGINES[request.param]
    ks = apk.geometry(eng).k_stage
    K, Ku = 10 * ks, 6 * ks
    TM, TN = tile_of(apk, eng)
    # 48 tasks per block: the job outlasts the 24 events the setter raises
    # 3 us apart (the one-wave tile finishes 24 short tiles in about 70 us)
    passes = 3072 // ((512 // TM) * (512 // TN))
    say(f"building {request.param} odd-length yield job M=N=512 K={K} kc={K // 5}, urgent "
        f"256x256x{Ku}")
    return Bf16Job(torch_gpu, apk, 512, 512, K, K // 5, 256, 256, Ku, events=24, blocks=64,
                   passes=passes, eng=eng)


@pytest.mark.parametrize("resume", [0, 1, 2])
def test_bf16_odd_length_pairs_yield(bf16_odd_job, apk, resume):
    """Yields at every site of tiles with an odd number of pairs, incl. the
    last pair: C bit-identical to the unpreempted run, within tolerance of
    float64, urgent outputs equal the non-preemptible urgent GEMM, every task
    and event counted once."""
    j = bf16_odd_job
    say(f"engine {j.eng} odd-length pairs, stage yields, resume={resume}")
    ref = j.run(apk.POLL_OFF, events=0)
    uref = run_bf16_urgent(j)
    assert oracle.rel_frobenius(uref, oracle.gemm_f64(j.Au, j.Bu, threads=8)) <= 1e-5
    c64 = oracle.gemm_f64(j.A, j.B, threads=8)
    # The setter (block 0) raises each event at its first poll site past the
    # event's time, so the site an event lands on depends on how long the
    # setter spends before each site; with the short 16-deep stages of the
    # small tiles, a job of 24 events can land none at the last site. Jobs
    # are repeated, each checked in full, until an event has.
    S = j.K // apk.geometry(j.eng).k_stage
    last = (S - 1) // 2 * 2
    sites = np.zeros(S, dtype=np.int64)
    for attempt in range(16):
        r = j.run(apk.POLL_STAGE, resume=resume, use_oracle=True)
        fired = int((r["set_gt"] != 0).sum())
        assert fired == j.events and int(r["stats"][:, 0].sum()) >= fired
        assert np.array_equal(r["C"].view(np.uint32), ref["C"].view(np.uint32))
        assert oracle.rel_frobenius(r["C"], c64) <= 1e-5
        for e in range(j.events):
            assert np.array_equal(r["Cu"][e].view(np.uint32), uref.view(np.uint32)), e
        assert (r["exec"] == 1).all() and (r["u_exec"] == j.U).all()
        # sites are the pair boundaries 0, 2, ..., last
        assert set(np.unique(r["site"]).tolist()) <= set(range(0, last + 1, 2))
        sites += np.bincount(r["site"], minlength=S)
        if sites[last] > 0:
            break
    assert sites[last] > 0
    say(f"  {attempt + 1} job(s), {j.events} events each, at sites {sites.tolist()}, "
        "bit-identical, float64 within 1e-5")
