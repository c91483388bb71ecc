"""apk_persistent_gemm_noalloc (queue counters in the library's own device
array) against apk_persistent_gemm (caller's counter buffer), through the C
ABI: two calls in a row, the second on a smaller GEMM, each bit-identical to
the existing entry point on the same inputs (same kernel, same k order), for
the VALU64 and MFMA128 engines; the first call also against the oracle."""
import numpy as np
import pytest

import oracle
from gpu_util import dev, say

pytestmark = pytest.mark.gpu


def _bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("engine_name,shapes,kc", [
    ("ENGINE_VALU64", [(512, 512, 256), (128, 192, 64)], 64),
    ("ENGINE_MFMA128", [(1024, 768, 512), (256, 384, 128)], 32),
])
def test_noalloc_matches_existing_entry_point(torch_gpu, apk, engine_name, shapes, kc):
    T = torch_gpu
    engine = getattr(apk, engine_name)
    blocks = apk.device_info().cu_count * apk.occupancy(engine)
    stream = T.cuda.current_stream().cuda_stream
    for i, (M, N, K) in enumerate(shapes):
        say(f"noalloc {engine_name} call {i}: M={M} N={N} K={K} kc={kc}")
        A, B = oracle.fill_uniform_pm1(21 + i, M, N, K)
        dA, dB = dev(T, A), dev(T, B)
        c_ref = T.full((M, N), float("nan"), dtype=T.float32, device="cuda")
        c_new = T.full((M, N), float("nan"), dtype=T.float32, device="cuda")
        nxt = T.zeros(apk.QUEUE_WORDS, dtype=T.int32, device="cuda")
        apk.persistent_gemm(engine, dA.data_ptr(), dB.data_ptr(), c_ref.data_ptr(), M, N, K, kc,
                            nxt.data_ptr(), None, blocks, stream)
        apk.persistent_gemm_noalloc(engine, dA.data_ptr(), dB.data_ptr(), c_new.data_ptr(),
                                    M, N, K, kc, None, blocks, stream)
        T.cuda.synchronize()
        ref, new = c_ref.cpu().numpy(), c_new.cpu().numpy()
        assert not np.isnan(new).any(), "tiles never written"
        assert (_bits(new) == _bits(ref)).all(), "noalloc result differs from apk_persistent_gemm"
        if i == 0:
            if engine == apk.ENGINE_VALU64:
                assert (_bits(new) == _bits(oracle.gemm_f32_chain(A, B))).all()
            else:
                assert oracle.rel_frobenius(new, oracle.gemm_f64(A, B, threads=8)) <= 1e-5


def test_noalloc_rejects_bad_shape(torch_gpu, apk):
    T = torch_gpu
    d = T.zeros(64 * 64, dtype=T.float32, device="cuda")
    with pytest.raises(apk.ApkError, match="not multiples"):
        apk.persistent_gemm_noalloc(apk.ENGINE_MFMA128, d.data_ptr(), d.data_ptr(), d.data_ptr(),
                                    96, 128, 64, 32, None, 4, 0)
