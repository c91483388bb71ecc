"""Helpers for GPU parity tests: device buffers through torch (plumbing only)
and a runner for apk_persistent_gemm through the C ABI."""
import sys

import numpy as np


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(torch, arr):
    """numpy -> device tensor (same dtype, contiguous)."""
    return torch.from_numpy(np.ascontiguousarray(arr)).to("cuda")


def run_persistent(torch, apk, engine, A, B, k_chunk, blocks=None, with_log=True,
                   C=None):
    M, K = A.shape
    N = B.shape[1]
    g = apk.geometry(engine)
    if blocks is None:
        blocks = apk.device_info().cu_count * apk.occupancy(engine)
    dA, dB = dev(torch, A), dev(torch, B)
    dC = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda") if C is None else C
    nxt = torch.zeros(apk.QUEUE_WORDS, dtype=torch.int32, device="cuda")
    nrec = (M // g.tile_m) * (N // g.tile_n) * (K // k_chunk)
    log = torch.full((nrec * 3,), -1, dtype=torch.int64, device="cuda") if with_log else None
    stream = torch.cuda.current_stream().cuda_stream
    apk.persistent_gemm(engine, dA.data_ptr(), dB.data_ptr(), dC.data_ptr(), M, N, K,
                        k_chunk, nxt.data_ptr(), log.data_ptr() if with_log else None,
                        blocks, stream)
    torch.cuda.synchronize()
    out = dC.cpu().numpy()
    recs = None
    if with_log:
        raw = log.cpu().numpy().reshape(nrec, 3)
        recs = {"start": raw[:, 0], "end": raw[:, 1],
                "smid": (raw[:, 2] & 0xffffffff).astype(np.int64).astype(np.int32),
                "block": (raw[:, 2] >> 32).astype(np.int32)}
    return out, recs, nxt.cpu().numpy()


def assert_queue_drained(ctr, tasks, blocks, xcds=8):
    """Counters of the XCD-aware queue after a run with tasks == tiles: list
    q holds positions [q*T/8, (q+1)*T/8) and every one was handed out; every
    worker ends with one failed pop on each non-empty list."""
    T = tasks
    for q in range(xcds):
        n = (q + 1) * T // xcds - q * T // xcds
        if n:
            assert ctr[q] >= n + blocks, (q, ctr[q], n, blocks)
        else:
            assert ctr[q] == 0, (q, ctr[q])
    assert not ctr[xcds:].any()
