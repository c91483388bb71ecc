"""GPU parity of the persistent GEMM (apk_persistent_gemm) against the CPU
oracle, through the C ABI.

Bars: VALU64 is bit-identical to the oracle's sequential fmaf chain (the
reference tile's arithmetic, src/tile.cuh:85-96); MFMA128 is within
rel-Frobenius <= 1e-5 and elementwise rtol=atol=1e-4 of the float64 reference
(src/persistent.cu:221-237), and bit-identical across worker counts and chunk
sizes (the per-tile accumulation order does not depend on scheduling)."""
import numpy as np
import pytest

import oracle
from gpu_util import assert_queue_drained, run_persistent, say

pytestmark = pytest.mark.gpu

FROB_F32 = 1e-5


def _bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def test_cfg1_valu64_bit_exact(torch_gpu, apk):
    # BASELINE cfg1: M=N=1024, K=128, 64x64 tiles, seed 0 (glibc: == seed 1)
    say("cfg1 valu64 M=N=1024 K=128 seed 0")
    A, B = oracle.fill_uniform_pm1(0, 1024, 1024, 128)
    C, recs, nxt = run_persistent(torch_gpu, apk, apk.ENGINE_VALU64, A, B, 128)
    ref32 = oracle.gemm_f32_chain(A, B)
    assert (_bits(C) == _bits(ref32)).all()
    ref = oracle.gemm_f64(A, B, threads=8)
    bad, nans, _ = oracle.check_elementwise(C, ref)
    assert bad == 0 and nans == 0
    assert oracle.rel_frobenius(C, ref) <= FROB_F32
    assert (recs["block"] >= 0).all() and (recs["end"] >= recs["start"]).all()
    assert nxt[:8].sum() >= 256


def test_valu64_chunked_bit_exact_reference_seed(torch_gpu, apk):
    say("valu64 chunked M=256 N=192 K=512 kc=64 seed 21")
    A, B = oracle.fill_uniform_pm1(21, 256, 192, 512)
    C, recs, _ = run_persistent(torch_gpu, apk, apk.ENGINE_VALU64, A, B, 64, blocks=7)
    assert (_bits(C) == _bits(oracle.gemm_f32_chain(A, B))).all()
    # records: 12 tiles x 8 chunks, each chunk of a tile on one block, in order
    st = recs["start"].reshape(12, 8)
    en = recs["end"].reshape(12, 8)
    assert (en >= st).all() and (st[:, 1:] >= en[:, :-1] - 1).all()
    assert (recs["block"].reshape(12, 8) == recs["block"].reshape(12, 8)[:, :1]).all()


@pytest.mark.parametrize("kc", [32, 64, 128])
def test_mfma128_parity_and_order_independence(torch_gpu, apk, kc):
    say(f"mfma128 M=512 N=384 K=512 kc={kc}")
    A, B = oracle.fill_uniform_pm1(21, 512, 384, 512)
    ref = oracle.gemm_f64(A, B, threads=8)
    C1, recs, _ = run_persistent(torch_gpu, apk, apk.ENGINE_MFMA128, A, B, kc)
    bad, nans, mr = oracle.check_elementwise(C1, ref)
    assert nans == 0 and bad == 0, (bad, mr)
    assert oracle.rel_frobenius(C1, ref) <= FROB_F32
    C2, _, _ = run_persistent(torch_gpu, apk, apk.ENGINE_MFMA128, A, B, kc, blocks=3)
    C3, _, _ = run_persistent(torch_gpu, apk, apk.ENGINE_MFMA128, A, B, 512, blocks=5,
                              with_log=False)
    assert (_bits(C1) == _bits(C2)).all() and (_bits(C1) == _bits(C3)).all()
    assert (recs["block"] >= 0).all()


@pytest.mark.parametrize("K", [96, 128, 32, 192])
def test_mfma128_stage_pairs_odd_stage_counts(torch_gpu, apk, K):
    """Without per-chunk records the fp32 MFMA tile runs its k-stages in
    pairs (one barrier per 64 k) when a tile has an even number of 32-deep
    stages, and one stage per barrier otherwise. C is bit-identical to the
    one-stage-per-barrier loop (records at every 32-k chunk) and within
    tolerance of float64."""
    say(f"mfma128 stage pairs vs single stages, M=256 N=384 K={K} ({K // 32} stages)")
    A, B = oracle.fill_uniform_pm1(8, 256, 384, K)
    Cp, _, _ = run_persistent(torch_gpu, apk, apk.ENGINE_MFMA128, A, B, K, blocks=5,
                              with_log=False)
    Cs, recs, _ = run_persistent(torch_gpu, apk, apk.ENGINE_MFMA128, A, B, 32, blocks=5)
    assert (_bits(Cp) == _bits(Cs)).all()
    assert (recs["block"] >= 0).all()
    assert oracle.rel_frobenius(Cp, oracle.gemm_f64(A, B)) <= FROB_F32


def test_mfma128_single_tile_and_idle_workers(torch_gpu, apk):
    say("mfma128 single tile, 64 workers")
    A, B = oracle.fill_uniform_pm1(4, 128, 128, 64)
    C, _, nxt = run_persistent(torch_gpu, apk, apk.ENGINE_MFMA128, A, B, 32, blocks=64)
    ref = oracle.gemm_f64(A, B)
    assert oracle.rel_frobenius(C, ref) <= FROB_F32
    assert_queue_drained(nxt, 1, 64)  # one tile taken; every worker's last pop failed


@pytest.fixture(scope="module")
def cfg2_operands():
    return oracle.fill_uniform_pm1(21, 4096, 4096, 4096)


@pytest.mark.parametrize("kc", [32, 64, 128])
def test_cfg2_full_size_sampled_rows(torch_gpu, apk, cfg2_operands, kc):
    # BASELINE cfg2 shape: M=N=K=4096, 128x128 tiles, K walked in kc-chunks
    # (the per-tile K set {32, 64, 128}).
    say(f"mfma128 cfg2 M=N=K=4096 kc={kc}")
    A, B = cfg2_operands
    C, recs, _ = run_persistent(torch_gpu, apk, apk.ENGINE_MFMA128, A, B, kc)
    assert not np.isnan(C).any()
    rows = [0, 127, 128, 2049, 4095]
    for r in rows:
        ref = oracle.gemm_f64_rows(A, B, r, 1)
        assert oracle.rel_frobenius(C[r:r + 1], ref) <= FROB_F32, r
    assert (recs["block"] >= 0).all()
    assert len(recs["block"]) == 32 * 32 * (4096 // kc)
