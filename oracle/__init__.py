"""CPU oracle for the preemptible persistent-GEMM path -- TEST INFRASTRUCTURE.

ctypes binding of oracle/_build/liboracle.so (built from oracle.cpp by
oracle/Makefile). Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may use this package, and only as the checker or as the
timed CPU baseline; the product (apk_amd/) never imports it.

Parity status of each function is recorded in the header of oracle.cpp
(every function has an independent pin in tests/test_oracle.py).
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")

_lib = None
_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_U32 = ctypes.c_uint32
_D = ctypes.c_double


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle` "
                           "(__graft_entry__.build() does)")
    lib = ctypes.CDLL(LIB_PATH)
    sig = {
        "apko_glibc_rand_stream": (None, [_U32, _P, _I64]),
        "apko_fill_uniform_pm1": (None, [_U32, _P, _I64, _P, _I64]),
        "apko_gemm_f64": (None, [_P, _P, _P, _I, _I, _I, _I]),
        "apko_gemm_f64_rows": (None, [_P, _P, _P, _I, _I, _I, _I, _I]),
        "apko_gemm_f32_chain": (None, [_P, _P, _P, _I, _I, _I]),
        "apko_check_elementwise": (None, [_P, _P, _I64, _D, _D, _P, _P, _P]),
        "apko_rel_frobenius": (_D, [_P, _P, _I64]),
        "apko_percentile": (_D, [_P, _I64, _D]),
        "apko_mt_stream": (None, [_U32, _P, _I64]),
        "apko_uniform_gap_schedule": (None, [_U32, _D, _D, _I, _P]),
        "apko_exp_gap_schedule": (None, [_U32, _D, _I, _P]),
        "apko_abab_poll": (_I, [_I]),
        "apko_bf16_rne": (ctypes.c_uint16, [ctypes.c_float]),
        "apko_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
        "apko_fill_normal_bf16": (None, [_U32, _P, _P, _I64, _P, _P, _I64]),
        "apko_count_tasks": (None, [_P, _I64, _P, _P, _P]),
        "apko_count_events": (_I, [_P, _P, _P, _I, _I, _P, _P, _P]),
        "apko_tile_hash": (ctypes.c_uint64, [_P, _I, _I, _I, _I, _I]),
        "apko_tiny_tile": (None, [_P, _P, _I, _I, _P]),
        "apko_tiny_expected": (None, [_P, _P, _I, _I, ctypes.c_uint64, ctypes.c_uint64, _I,
                                      _P, _P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def glibc_rand_stream(seed, n):
    out = np.empty(n, dtype=np.int32)
    load().apko_glibc_rand_stream(seed, _ptr(out), n)
    return out


def fill_uniform_pm1(seed, M, N, K):
    """A (MxK) and B (KxN) as the reference generates them (srand(seed))."""
    A = np.empty((M, K), dtype=np.float32)
    B = np.empty((K, N), dtype=np.float32)
    load().apko_fill_uniform_pm1(seed, _ptr(A), A.size, _ptr(B), B.size)
    return A, B


def gemm_f64(A, B, threads=1):
    A = np.ascontiguousarray(A, dtype=np.float32)
    B = np.ascontiguousarray(B, dtype=np.float32)
    M, K = A.shape
    K2, N = B.shape
    assert K == K2
    C = np.empty((M, N), dtype=np.float64)
    load().apko_gemm_f64(_ptr(A), _ptr(B), _ptr(C), M, N, K, threads)
    return C


def gemm_f64_rows(A, B, row0, nrows):
    A = np.ascontiguousarray(A, dtype=np.float32)
    B = np.ascontiguousarray(B, dtype=np.float32)
    M, K = A.shape
    N = B.shape[1]
    nrows = min(nrows, M - row0)
    C = np.empty((nrows, N), dtype=np.float64)
    load().apko_gemm_f64_rows(_ptr(A), _ptr(B), _ptr(C), M, N, K, row0, nrows)
    return C


def gemm_f32_chain(A, B):
    A = np.ascontiguousarray(A, dtype=np.float32)
    B = np.ascontiguousarray(B, dtype=np.float32)
    M, K = A.shape
    N = B.shape[1]
    C = np.empty((M, N), dtype=np.float32)
    load().apko_gemm_f32_chain(_ptr(A), _ptr(B), _ptr(C), M, N, K)
    return C


def check_elementwise(got, ref, rtol=1e-4, atol=1e-4):
    got = np.ascontiguousarray(got, dtype=np.float32)
    ref = np.ascontiguousarray(ref, dtype=np.float64)
    bad, nans, mr = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_double()
    load().apko_check_elementwise(_ptr(got), _ptr(ref), got.size, rtol, atol,
                                  ctypes.byref(bad), ctypes.byref(nans),
                                  ctypes.byref(mr))
    return bad.value, nans.value, mr.value


def rel_frobenius(got, ref):
    got = np.ascontiguousarray(got, dtype=np.float32)
    ref = np.ascontiguousarray(ref, dtype=np.float64)
    return load().apko_rel_frobenius(_ptr(got), _ptr(ref), got.size)


def percentile(v, q):
    v = np.ascontiguousarray(v, dtype=np.float64)
    return load().apko_percentile(_ptr(v), v.size, q)


def mt_stream(seed, n):
    out = np.empty(n, dtype=np.uint32)
    load().apko_mt_stream(seed, _ptr(out), n)
    return out


def uniform_gap_schedule(seed, gmin_us, gmax_us, events):
    out = np.empty(events, dtype=np.int64)
    load().apko_uniform_gap_schedule(seed, gmin_us, gmax_us, events, _ptr(out))
    return out


def exp_gap_schedule(seed, mean_us, events):
    out = np.empty(events, dtype=np.int64)
    load().apko_exp_gap_schedule(seed, mean_us, events, _ptr(out))
    return out


def abab_poll(r):
    return load().apko_abab_poll(r)


def bf16_rne(x):
    return load().apko_bf16_rne(x)


def bf16_to_f32(h):
    return load().apko_bf16_to_f32(h)


def fill_normal_bf16(seed, M, N, K):
    A = np.empty((M, K), dtype=np.uint16)
    B = np.empty((K, N), dtype=np.uint16)
    Ad = np.empty((M, K), dtype=np.float32)
    Bd = np.empty((K, N), dtype=np.float32)
    load().apko_fill_normal_bf16(seed, _ptr(A), _ptr(Ad), A.size, _ptr(B),
                                 _ptr(Bd), B.size)
    return A, Ad, B, Bd


def count_tasks(exec_counts):
    e = np.ascontiguousarray(exec_counts, dtype=np.int32)
    d, m, fb = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    load().apko_count_tasks(_ptr(e), e.size, ctypes.byref(d), ctypes.byref(m),
                            ctypes.byref(fb))
    return d.value, m.value, fb.value


def count_events(set_gt, uexec, claim, urgent_per_event):
    s = np.ascontiguousarray(set_gt, dtype=np.int64)
    u = np.ascontiguousarray(uexec, dtype=np.int32)
    c = None if claim is None else np.ascontiguousarray(claim, dtype=np.int32)
    f, b, un = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    ok = load().apko_count_events(_ptr(s), _ptr(u), None if c is None else _ptr(c),
                                  s.size, urgent_per_event, ctypes.byref(f),
                                  ctypes.byref(b), ctypes.byref(un))
    return bool(ok), f.value, b.value, un.value


def tile_hash(C, row0, col0, tile_m, tile_n):
    C = np.ascontiguousarray(C, dtype=np.float32)
    return load().apko_tile_hash(_ptr(C), C.shape[1], row0, col0, tile_m, tile_n)


def tiny_pool(seed, tiles, lo=-2, hi=2):
    """`tiles` 16x16 tiles of small-integer bf16 bit patterns (exact in
    bf16), seeded; returns (bits uint16 [tiles, 256], values float32)."""
    rng = np.random.default_rng(seed)
    v = rng.integers(lo, hi + 1, size=(tiles, 256)).astype(np.float32)
    bits = (v.view(np.uint32) >> 16).astype(np.uint16)
    return np.ascontiguousarray(bits), v


def tiny_tile(A, Bt, ia, ib):
    """Product of A tile ia and B tile ib (Bt stored N x K) in the device's
    lane-major register order: out[4 l + j] = C[4 (l // 16) + j][l % 16]."""
    A = np.ascontiguousarray(A, dtype=np.uint16)
    Bt = np.ascontiguousarray(Bt, dtype=np.uint16)
    out = np.empty(256, dtype=np.float32)
    load().apko_tiny_tile(_ptr(A), _ptr(Bt), ia, ib, _ptr(out))
    return out


def tiny_expected(A, Bt, n, n_urgent, threads=8):
    """Expected (background, urgent) checksums of the tiny-task oracle."""
    A = np.ascontiguousarray(A, dtype=np.uint16)
    Bt = np.ascontiguousarray(Bt, dtype=np.uint16)
    bg, u = ctypes.c_uint64(), ctypes.c_uint64()
    load().apko_tiny_expected(_ptr(A), _ptr(Bt), A.shape[0], Bt.shape[0], n, n_urgent,
                              threads, ctypes.byref(bg), ctypes.byref(u))
    return bg.value, u.value
