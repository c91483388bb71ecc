"""Pins of the CPU oracle (oracle/oracle.cpp) against sources independent of
it: the golden fixtures (libc rand, numpy MT19937, libstdc++ distributions,
torch bf16 cast), numpy float64 matmul, exact rational arithmetic, and brute
force. Each test is chosen so that a plausible mistake in the restatement (a
dropped term, a wrong index, a transposed operand, a wrong rounding) fails."""
import json
import os
from fractions import Fraction

import numpy as np
import pytest

import oracle

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = json.load(open(os.path.join(HERE, "golden", "golden.json")))


# ---------------------------------------------------------------- generators
@pytest.mark.parametrize("seed", ["0", "1", "21", "12345"])
def test_glibc_rand_matches_libc(seed):
    g = GOLDEN["glibc_rand"][seed]
    far = g["far_index"]
    s = oracle.glibc_rand_stream(int(seed), far + 1)
    assert list(s[:8]) == g["first"]
    assert int(s[far]) == g["far"]


def test_glibc_seed0_is_seed1_and_known_answer():
    # published known answer of glibc: srand(1); rand() == 1804289383
    assert oracle.glibc_rand_stream(1, 1)[0] == 1804289383
    assert (oracle.glibc_rand_stream(0, 100) == oracle.glibc_rand_stream(1, 100)).all()


def test_fill_uniform_uses_one_stream_a_then_b():
    M, N, K = 3, 5, 4
    A, B = oracle.fill_uniform_pm1(21, M, N, K)
    r = oracle.glibc_rand_stream(21, M * K + K * N).astype(np.float64)
    v = (r / 2147483647.0 * 2.0 - 1.0).astype(np.float32)
    assert (A.ravel() == v[:M * K]).all()
    assert (B.ravel() == v[M * K:]).all()
    assert A.min() >= -1.0 and A.max() <= 1.0


@pytest.mark.parametrize("seed", ["5489", "21", "7"])
def test_mt19937_matches_numpy_legacy(seed):
    assert list(oracle.mt_stream(int(seed), 16)) == GOLDEN["mt19937_raw"][seed]


def test_mt19937_standard_10000th():
    assert int(oracle.mt_stream(5489, 10000)[-1]) == GOLDEN["mt19937_default_10000th"]


@pytest.mark.parametrize("seed", ["21", "7"])
def test_uniform_schedule_matches_libstdcxx(seed):
    got = oracle.uniform_gap_schedule(int(seed), 150.0, 400.0, 64)
    assert list(got) == GOLDEN["uniform_schedule_us_150_400"][seed]


@pytest.mark.parametrize("seed", ["21", "7"])
def test_exp_schedule_matches_libstdcxx(seed):
    got = oracle.exp_gap_schedule(int(seed), 2000.0, 64)
    assert list(got) == GOLDEN["exp_schedule_mean_2000us"][seed]


def test_exp_schedule_moments():
    cum = oracle.exp_gap_schedule(3, 2000.0, 200000)
    gaps = np.diff(np.concatenate([[0], cum])) / 1e3
    assert abs(gaps.mean() / 2000.0 - 1) < 0.01
    assert abs(gaps.std() / 2000.0 - 1) < 0.02   # exponential: sd == mean
    assert (gaps >= 0).all()


def test_uniform_schedule_bounds():
    cum = oracle.uniform_gap_schedule(21, 150.0, 400.0, 20000)
    gaps = np.diff(np.concatenate([[0], cum]))
    assert gaps.min() >= 150000 and gaps.max() < 400000
    assert abs(gaps.mean() / 275000 - 1) < 0.01


def test_abab_order():
    # pairs alternate which variant leads: on,off, off,on, on,off, ...
    seq = [oracle.abab_poll(r) for r in range(8)]
    assert seq == [1, 0, 0, 1, 1, 0, 0, 1]


@pytest.mark.parametrize("case", range(len(GOLDEN["bf16_rne"])))
def test_bf16_rne_matches_torch(case):
    c = GOLDEN["bf16_rne"][case]
    assert oracle.bf16_rne(c["x"]) == c["bits"]


def test_bf16_roundtrip_and_normal_moments():
    A, Ad, B, Bd = oracle.fill_normal_bf16(5, 256, 256, 256)
    back = (A.astype(np.uint32) << 16).view(np.float32)
    assert (back == Ad).all()
    allv = np.concatenate([Ad.ravel(), Bd.ravel()]).astype(np.float64)
    assert abs(allv.mean()) < 0.01 and abs(allv.std() - 1) < 0.01


# ---------------------------------------------------------------- GEMMs
def test_gemm_f64_matches_numpy():
    A, B = oracle.fill_uniform_pm1(21, 64, 48, 80)
    ref = A.astype(np.float64) @ B.astype(np.float64)
    got = oracle.gemm_f64(A, B)
    np.testing.assert_allclose(got, ref, rtol=1e-13, atol=1e-13)
    # a transposed operand (square case) must not pass
    A2, B2 = oracle.fill_uniform_pm1(3, 32, 32, 32)
    assert not np.allclose(oracle.gemm_f64(A2, B2), A2.astype(np.float64) @ B2.T.astype(np.float64))


def test_gemm_f64_threads_identical():
    A, B = oracle.fill_uniform_pm1(9, 37, 29, 53)
    assert (oracle.gemm_f64(A, B, 1) == oracle.gemm_f64(A, B, 4)).all()
    rows = oracle.gemm_f64_rows(A, B, 5, 7)
    assert (rows == oracle.gemm_f64(A, B)[5:12]).all()


def test_gemm_closed_forms():
    rng = np.random.default_rng(0)
    A = rng.integers(-8, 9, size=(16, 24)).astype(np.float32)
    eye = np.eye(24, dtype=np.float32)
    assert (oracle.gemm_f64(A, eye) == A).all()
    u = rng.integers(-5, 6, size=(16, 1)).astype(np.float32)
    v = rng.integers(-5, 6, size=(1, 12)).astype(np.float32)
    assert (oracle.gemm_f64(u, v) == (u.astype(np.float64) * v)).all()


def _round_f32(q):
    """Nearest float32 to the rational q, ties to even (exact)."""
    c = np.float32(float(q))
    best = None
    for cand in (np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))):
        d = abs(Fraction(float(cand)) - q)
        key = (d, int(np.array(cand, dtype=np.float32).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, cand)
    return best[1]


def test_gemm_f32_chain_exact_rational():
    A, B = oracle.fill_uniform_pm1(21, 3, 4, 37)
    got = oracle.gemm_f32_chain(A, B)
    for i in range(3):
        for j in range(4):
            acc = np.float32(0.0)
            for k in range(37):
                q = Fraction(float(A[i, k])) * Fraction(float(B[k, j])) + Fraction(float(acc))
                acc = _round_f32(q)
            assert got[i, j].view(np.uint32) == np.float32(acc).view(np.uint32), (i, j)


def test_gemm_f32_chain_differs_from_unfused():
    # a chain of separate multiply and add roundings must not reproduce fmaf
    A, B = oracle.fill_uniform_pm1(21, 16, 16, 64)
    got = oracle.gemm_f32_chain(A, B)
    unfused = np.zeros((16, 16), dtype=np.float32)
    for k in range(64):
        unfused = (unfused + (A[:, k:k + 1] * B[k:k + 1, :]).astype(np.float32)).astype(np.float32)
    assert (got != unfused).any()
    np.testing.assert_allclose(got, A.astype(np.float64) @ B.astype(np.float64), rtol=1e-5, atol=1e-5)


def test_gemm_f32_chain_integer_exact():
    rng = np.random.default_rng(1)
    A = rng.integers(-16, 17, size=(8, 40)).astype(np.float32)
    B = rng.integers(-16, 17, size=(40, 9)).astype(np.float32)
    assert (oracle.gemm_f32_chain(A, B) == (A.astype(np.int64) @ B.astype(np.int64))).all()


# ---------------------------------------------------------------- checks / stats
def test_rel_frobenius_numpy():
    rng = np.random.default_rng(2)
    ref = rng.standard_normal(1000)
    got = (ref + 1e-6 * rng.standard_normal(1000)).astype(np.float32)
    want = np.linalg.norm(got.astype(np.float64) - ref) / np.linalg.norm(ref)
    assert abs(oracle.rel_frobenius(got, ref) / want - 1) < 1e-9


def test_check_elementwise_boundary():
    ref = np.array([0.0, 1.0, 100.0, -3.0], dtype=np.float64)
    ok = np.array([1e-4 * 0.99, 1.0 + 2e-4 * 0.99, 100.0 + 0.0101 * 0.99, -3.0], dtype=np.float32)
    assert oracle.check_elementwise(ok, ref)[0] == 0
    bad = ok.copy()
    bad[2] = np.float32(100.0 + 0.0101 * 1.5)
    assert oracle.check_elementwise(bad, ref)[0] == 1
    nan = ok.copy()
    nan[0] = np.nan
    assert oracle.check_elementwise(nan, ref)[1] == 1


@pytest.mark.parametrize("n", [1, 2, 7, 100, 101])
def test_percentile_nearest_rank(n):
    rng = np.random.default_rng(n)
    v = rng.standard_normal(n)
    s = sorted(v)
    for q in (0.0, 0.5, 0.9, 0.99, 1.0):
        assert oracle.percentile(v, q) == s[min(int(q * n), n - 1)]


def test_count_tasks_planted():
    e = np.ones(1000, dtype=np.int32)
    assert oracle.count_tasks(e) == (0, 0, -1)
    e[17] = 2
    e[400] = 0
    e[401] = 3
    assert oracle.count_tasks(e) == (2, 1, 17)


def test_count_events_planted():
    set_gt = np.array([5, 6, 0, 9], dtype=np.int64)
    uexec = np.array([2, 2, 0, 2], dtype=np.int32)
    claim = np.array([1, 3, 0, 2], dtype=np.int32)
    ok, fired, bad, uncl = oracle.count_events(set_gt, uexec, claim, 2)
    assert (ok, fired, bad, uncl) == (False, 3, 0, 0)   # fired != events
    ok, fired, bad, uncl = oracle.count_events(set_gt[[0, 1, 3]], uexec[[0, 1, 3]], claim[[0, 1, 3]], 2)
    assert ok and fired == 3
    uexec[1] = 1
    claim[3] = 0
    ok, fired, bad, uncl = oracle.count_events(set_gt[[0, 1, 3]], uexec[[0, 1, 3]], claim[[0, 1, 3]], 2)
    assert (ok, bad, uncl) == (False, 1, 1)


def test_tile_hash_sensitivity():
    A, B = oracle.fill_uniform_pm1(21, 128, 128, 32)
    C = oracle.gemm_f32_chain(A, B)
    h = oracle.tile_hash(C, 0, 0, 64, 64)
    assert h == oracle.tile_hash(C.copy(), 0, 0, 64, 64)
    D = C.copy()
    D.view(np.uint32)[3, 5] ^= 1           # one ulp in one element
    assert oracle.tile_hash(D, 0, 0, 64, 64) != h
    E = C.copy()
    E[0, 0], E[0, 1] = C[0, 1], C[0, 0]    # same multiset, moved
    assert oracle.tile_hash(E, 0, 0, 64, 64) != h
    assert oracle.tile_hash(C, 64, 0, 64, 64) != h  # other tile


def _py_mix64(z):
    M = (1 << 64) - 1
    z &= M
    z = ((z ^ (z >> 30)) * 0xbf58476d1ce4e5b9) & M
    z = ((z ^ (z >> 27)) * 0x94d049bb133111eb) & M
    return z ^ (z >> 31)


def _py_tiny_value(Av, Btv, ia, ib):
    """Plain-Python restatement: C = A[ia] . B[ib] (Bt stored N x K) from the
    small-integer values, in lane-major register order, then the positional
    fingerprint."""
    a = Av[ia].reshape(16, 16)
    bt = Btv[ib].reshape(16, 16)
    C = a.astype(np.int64) @ bt.astype(np.int64).T            # exact integers
    v = 0
    for lane in range(64):
        for j in range(4):
            x = np.float32(C[4 * (lane // 16) + j][lane % 16])
            bits = int(x.view(np.uint32))
            v += _py_mix64(bits + ((4 * lane + j) << 32))
    return v & ((1 << 64) - 1)


def test_tiny_tile_layout_and_values():
    A, Av = oracle.tiny_pool(1, 3)
    Bt, Btv = oracle.tiny_pool(2, 2)
    out = oracle.tiny_tile(A, Bt, 2, 1)
    C = Av[2].reshape(16, 16) @ Btv[1].reshape(16, 16).T
    for lane in (0, 5, 17, 33, 63):
        for j in range(4):
            assert out[4 * lane + j] == C[4 * (lane // 16) + j][lane % 16]
    # a transposed operand (the plausible mistake) gives a different tile
    assert not np.array_equal(out.reshape(64, 4),
                              (Av[2].reshape(16, 16) @ Btv[1].reshape(16, 16))
                              [np.arange(4)[None, :] + 4 * (np.arange(64)[:, None] // 16),
                               np.arange(64)[:, None] % 16])


def test_tiny_expected_matches_python_restatement():
    A, Av = oracle.tiny_pool(3, 3)
    Bt, Btv = oracle.tiny_pool(4, 2)
    pa, pb, n, nu = 3, 2, 40, 9
    G, SALT, M = 0x9E3779B97F4A7C15, 0xD1B54A32D192ED03, (1 << 64) - 1
    bg = sum(_py_mix64(_py_tiny_value(Av, Btv, t % pa, (t // pa) % pb) + t * G)
             for t in range(n)) & M
    u = sum(_py_mix64(_py_tiny_value(Av, Btv, (i * 7 + 3) % pa, (i * 13 + 5) % pb) + i * G + SALT)
            for i in range(nu)) & M
    assert oracle.tiny_expected(A, Bt, n, nu, threads=3) == (bg, u)
    # the sum over tasks is order-free but not task-free: dropping one task changes it
    assert oracle.tiny_expected(A, Bt, n - 1, nu)[0] != bg
