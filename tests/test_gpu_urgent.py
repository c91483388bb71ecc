"""apk_urgent_gemm, the reference's urgent_tile (src/urgent_baseline.cu:
100-112): one block per tile, no queue, start stamped at block 0's first
instruction, end raised by every block. Its C must be bit-identical to the
persistent GEMM's (same engine, same per-element k order), the fp32 tile
bit-identical to the fmaf-chain oracle, and the stamps ordered."""
import numpy as np
import pytest

import oracle
from gpu_util import dev, run_persistent, say

pytestmark = pytest.mark.gpu


def run_urgent(torch, apk, eng, A, B):
    M, K = A.shape
    N = B.shape[0] if apk.geometry(eng).b_transposed else B.shape[1]
    dA, dB = dev(torch, A), dev(torch, B)
    dC = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    t = torch.zeros(2, dtype=torch.int64, device="cuda")
    apk.urgent_gemm(eng, dA.data_ptr(), dB.data_ptr(), dC.data_ptr(), M, N, K,
                    t.data_ptr(), t.data_ptr() + 8, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    start, end = t.cpu().numpy().tolist()
    return dC.cpu().numpy(), start, end


@pytest.mark.parametrize("name", ["valu64", "mfma128"])
def test_urgent_fp32_matches_persistent(torch_gpu, apk, name):
    eng = apk.ENGINES[name]
    g = apk.geometry(eng)
    M, N, K = 2 * g.tile_m, 2 * g.tile_n, 256
    say(f"urgent_gemm {name} {M}x{N}x{K} vs persistent_gemm")
    A, B = oracle.fill_uniform_pm1(21, M, N, K)
    C, start, end = run_urgent(torch_gpu, apk, eng, A, B)
    # records at every k-stage: the persistent GEMM's one-stage-per-barrier
    # loop, against the urgent kernel's (stage pairs for the fp32 MFMA tile)
    Cp, _, _ = run_persistent(torch_gpu, apk, eng, A, B, g.k_stage, blocks=3)
    assert np.array_equal(C.view(np.uint32), Cp.view(np.uint32))
    if name == "valu64":
        assert np.array_equal(C.view(np.uint32), oracle.gemm_f32_chain(A, B).view(np.uint32))
    assert oracle.rel_frobenius(C, oracle.gemm_f64(A, B, threads=8)) <= 1e-5
    assert 0 < start <= end


@pytest.mark.parametrize("name", ["bf16x256", "bf16x128", "bf16x256x128"])
def test_urgent_bf16_matches_persistent(torch_gpu, apk, name):
    eng = apk.ENGINES[name]
    g = apk.geometry(eng)
    M, N, K = 2 * g.tile_m, g.tile_n, 512
    say(f"urgent_gemm {name} {M}x{N}x{K} vs persistent_gemm")
    A_bits, A, B_bits, B = oracle.fill_normal_bf16(9, M, N, K)
    Bt = np.ascontiguousarray(B_bits.T)
    C, start, end = run_urgent(torch_gpu, apk, eng, A_bits.view(np.int16), Bt.view(np.int16))
    dA, dB = dev(torch_gpu, A_bits.view(np.int16)), dev(torch_gpu, Bt.view(np.int16))
    dC = torch_gpu.empty((M, N), dtype=torch_gpu.float32, device="cuda")
    q = torch_gpu.zeros(apk.QUEUE_WORDS, dtype=torch_gpu.int32, device="cuda")
    apk.persistent_gemm(eng, dA.data_ptr(), dB.data_ptr(), dC.data_ptr(), M, N, K, K,
                        q.data_ptr(), None, 2, torch_gpu.cuda.current_stream().cuda_stream)
    torch_gpu.cuda.synchronize()
    assert np.array_equal(C.view(np.uint32), dC.cpu().numpy().view(np.uint32))
    assert oracle.rel_frobenius(C, oracle.gemm_f64(A, B, threads=8)) <= 1e-5
    assert 0 < start <= end


def test_urgent_rejects_bad_shape(torch_gpu, apk):
    # M = 100 is not a multiple of the 128-row tile: refused before any launch
    buf = torch_gpu.zeros(128 * 128, dtype=torch_gpu.float32, device="cuda")
    with pytest.raises(apk.ApkError):
        apk.urgent_gemm(apk.ENGINE_MFMA128, buf.data_ptr(), buf.data_ptr(), buf.data_ptr(),
                        100, 128, 128)
