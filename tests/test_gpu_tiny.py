"""GPU parity of the tiny-task scheduler oracle (apk_tiny_oracle) through the
C ABI: one v_mfma_f32_16x16x16_bf16 per task, popped by every wave of the
grid from the XCD-split fetch-add queue, under device-raised preemption
events that make waves checkpoint their in-flight tile to HBM, run urgent
tasks and restore.

Pinned:
  * the operand/result lane layout: the device's register-order dump of the
    first tasks equals the CPU restatement word for word (small integers,
    so the products are exact);
  * exactly-once: every task id counted once, every fired event's urgent
    mini-queue run exactly urgent_per_event times, all events fired;
  * bit-exactness through checkpoint/restore: the background and urgent
    checksums equal the CPU's predictions (a lost, duplicated or corrupted
    task changes them).
"""
import numpy as np
import pytest

import oracle
from gpu_util import dev, say

pytestmark = pytest.mark.gpu


def run_tiny(torch, apk, n, batch, events, gap_ticks, U, pa=8, pb=8, n_debug=0, blocks=None):
    T = torch
    A, _ = oracle.tiny_pool(11, pa)
    Bt, _ = oracle.tiny_pool(12, pb)
    if blocks is None:
        blocks = apk.device_info().cu_count * 2
    waves = blocks * 4
    E = max(events, 1)
    i32, i64 = T.int32, T.int64
    d = {
        "A": dev(T, A.view(np.int16)), "Bt": dev(T, Bt.view(np.int16)),
        "next": T.zeros(apk.QUEUE_WORDS, dtype=i32, device="cuda"),
        "exec": T.zeros(n, dtype=i32, device="cuda"),
        "sum": T.zeros(2, dtype=i64, device="cuda"),
        "flag": T.zeros(64, dtype=i32, device="cuda"),
        "sched": (T.arange(1, E + 1, dtype=i64, device="cuda") * gap_ticks),
        "set": T.zeros(E, dtype=i64, device="cuda"),
        "uq": T.zeros(E, dtype=i32, device="cuda"),
        "uexec": T.zeros(E, dtype=i32, device="cuda"),
        "ckpt": T.zeros(waves * 256, dtype=T.float32, device="cuda"),
        "stats": T.zeros(2, dtype=i64, device="cuda"),
        "dbg": T.full((max(n_debug, 1) * 256,), float("nan"), dtype=T.float32, device="cuda"),
    }
    p = apk.TinyParams()
    p.num_tasks, p.next_task, p.batch = n, d["next"].data_ptr(), batch
    p.A, p.Bt, p.pa, p.pb = d["A"].data_ptr(), d["Bt"].data_ptr(), pa, pb
    p.exec_count, p.checksum, p.flag = d["exec"].data_ptr(), d["sum"].data_ptr(), d["flag"].data_ptr()
    if events:
        p.sched, p.num_events, p.set_gt = d["sched"].data_ptr(), events, d["set"].data_ptr()
        p.uq_next, p.urgent_per_event, p.u_exec_count = d["uq"].data_ptr(), U, d["uexec"].data_ptr()
    p.ckpt, p.stats = d["ckpt"].data_ptr(), d["stats"].data_ptr()
    if n_debug:
        p.c_debug, p.n_debug = d["dbg"].data_ptr(), n_debug
    T.cuda.synchronize()
    say(f"tiny oracle n={n} batch={batch} events={events} U={U} blocks={blocks}")
    apk.tiny_oracle(p, blocks, T.cuda.current_stream().cuda_stream)
    T.cuda.synchronize()
    return A, Bt, {k: v.cpu().numpy() for k, v in d.items()}


def test_tiny_lane_layout_exact(torch_gpu, apk):
    A, Bt, r = run_tiny(torch_gpu, apk, n=64, batch=1, events=0, gap_ticks=0, U=0, pa=5, pb=3,
                        n_debug=64, blocks=4)
    dbg = r["dbg"].reshape(64, 256)
    for t in range(64):
        want = oracle.tiny_tile(A, Bt, t % 5, (t // 5) % 3)
        assert np.array_equal(dbg[t].view(np.uint32), want.view(np.uint32)), f"task {t}"
    assert (r["exec"] == 1).all()


@pytest.mark.parametrize("batch", [1, 4])
def test_tiny_exactly_once_under_preemption(torch_gpu, apk, batch):
    n, events, U = 4_000_000, 40, 32
    A, Bt, r = run_tiny(torch_gpu, apk, n=n, batch=batch, events=events, gap_ticks=200, U=U)
    fired = int((r["set"] != 0).sum())
    assert fired == events, f"only {fired} of {events} events fired"
    ex = r["exec"]
    assert (ex == 1).all(), f"{int((ex > 1).sum())} duplicated, {int((ex == 0).sum())} missed"
    assert (r["uexec"] == U).all(), r["uexec"]
    yields, urgent = (int(x) for x in r["stats"])
    assert urgent == events * U and yields >= events
    bg, u = oracle.tiny_expected(A, Bt, n, events * U)
    got = r["sum"].view(np.uint64)
    assert int(got[0]) == bg, "background checksum differs"
    assert int(got[1]) == u, "urgent checksum differs"
