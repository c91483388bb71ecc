"""apk_amd -- MI355X (gfx950) preemptible persistent GEMM.

Python access to the C ABI declared in include/apk.h (lib/libapk.so), used
by the tests, smoke() and bench.py. The product is the HIP library and the
C++ measurement binaries in bin/; this module only binds the library with
ctypes and fails loudly when it has not been built. There is no CPU
fallback: every compute call runs the gfx950 kernels.
"""
import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(_HERE)
LIB_PATH = os.path.join(_HERE, "lib", "libapk.so")
BIN_DIR = os.path.join(_HERE, "bin")
HEADER = os.path.join(ROOT, "include", "apk.h")

APK_OK, APK_EINVAL, APK_EHIP, APK_ERANGE = 0, 1, 2, 3
ENGINE_VALU64, ENGINE_MFMA128, ENGINE_BF16X256, ENGINE_BF16X128, ENGINE_BF16X256X128 = range(5)
ENGINES = {"valu64": ENGINE_VALU64, "mfma128": ENGINE_MFMA128, "bf16x256": ENGINE_BF16X256,
           "bf16x128": ENGINE_BF16X128, "bf16x256x128": ENGINE_BF16X256X128}


class ApkError(RuntimeError):
    pass


class TileRecord(ctypes.Structure):
    _fields_ = [("start", ctypes.c_int64), ("end", ctypes.c_int64),
                ("smid", ctypes.c_int32), ("block", ctypes.c_int32)]


class DeviceInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 128), ("arch", ctypes.c_char * 64),
                ("cu_count", ctypes.c_int), ("wall_clock_khz", ctypes.c_int),
                ("clock_khz", ctypes.c_int), ("lds_per_cu", ctypes.c_int),
                ("regs_per_cu", ctypes.c_int), ("xcc_count", ctypes.c_int)]


class EngineGeometry(ctypes.Structure):
    _fields_ = [("tile_m", ctypes.c_int), ("tile_n", ctypes.c_int),
                ("k_stage", ctypes.c_int), ("threads", ctypes.c_int),
                ("lds_bytes", ctypes.c_int), ("elem_bytes", ctypes.c_int),
                ("b_transposed", ctypes.c_int)]


POLL_OFF, POLL_CHUNK, POLL_STAGE, POLL_ISSUE = 0, 1, 2, 3
RESUME_CKPT_FULL, RESUME_CKPT_ACC, RESUME_RESTART = 0, 1, 2
FLAG_STRIDE, FLAG_MAX_COPIES = 4096, 256
STATS_PER_BLOCK = 16
# columns of a stats row (APK_ST_* in include/apk.h)
(ST_YIELDS, ST_SAVE, ST_URGENT, ST_RESTORE, ST_INFLIGHT, ST_RETREATS, ST_RESUMED, ST_ERRORS,
 ST_STALE, ST_CHECKPOINTS, ST_INFLIGHT_ALL, ST_STALE_ALL, ST_DECLINED, ST_START_SITES) = range(14)
QUEUE_WORDS, QUEUE_XCDS = 16, 8
RQ_CTL_WORDS = 4  # resume ring control words (APK_RQ_CTL_WORDS)
SES_PER_XCD, RETREAT_DOMAINS = 4, 32


class YieldParams(ctypes.Structure):
    """Mirror of apk_yield_params (include/apk.h); pointers are device
    addresses as ints."""
    _fields_ = [
        ("A", ctypes.c_void_p), ("B", ctypes.c_void_p), ("C", ctypes.c_void_p),
        ("M", ctypes.c_int), ("N", ctypes.c_int), ("K", ctypes.c_int), ("k_chunk", ctypes.c_int),
        ("num_tasks", ctypes.c_uint), ("next_task", ctypes.c_void_p),
        ("Au", ctypes.c_void_p), ("Bu", ctypes.c_void_p), ("Cu", ctypes.c_void_p),
        ("Mu", ctypes.c_int), ("Nu", ctypes.c_int), ("Ku", ctypes.c_int),
        ("uq_next", ctypes.c_void_p),
        ("flag", ctypes.c_void_p), ("flag_copies", ctypes.c_int), ("flag_system", ctypes.c_int),
        ("flag_set", ctypes.c_void_p),
        ("sched", ctypes.c_void_p), ("num_events", ctypes.c_int),
        ("stop_after", ctypes.c_longlong), ("poll_every", ctypes.c_int),
        ("set_gt", ctypes.c_void_p), ("obs_gt", ctypes.c_void_p), ("claim", ctypes.c_void_p),
        ("claim_site", ctypes.c_void_p), ("u_gt", ctypes.c_void_p), ("u_end_max", ctypes.c_void_p),
        ("resume", ctypes.c_int), ("ckpt", ctypes.c_void_p), ("poison", ctypes.c_int),
        ("task_hash", ctypes.c_void_p), ("u_hash", ctypes.c_void_p), ("stats", ctypes.c_void_p),
        ("exec_count", ctypes.c_void_p), ("u_exec_count", ctypes.c_void_p),
        ("cu_event_stride", ctypes.c_longlong), ("naive", ctypes.c_int),
        ("run_gt", ctypes.c_void_p), ("exit_count", ctypes.c_void_p),
        ("retreat", ctypes.c_int), ("retreat_count", ctypes.c_void_p),
        ("retreat_gt", ctypes.c_void_p), ("rq_ctl", ctypes.c_void_p),
        ("rq_entry", ctypes.c_void_p), ("rq_slots", ctypes.c_void_p),
        ("rq_capacity", ctypes.c_uint), ("continuation", ctypes.c_int),
        ("block_base", ctypes.c_int), ("obs_stride", ctypes.c_int),
        ("launch_epoch", ctypes.c_int),
    ]


class TinyParams(ctypes.Structure):
    """Mirror of apk_tiny_params (include/apk.h)."""
    _fields_ = [
        ("num_tasks", ctypes.c_uint), ("next_task", ctypes.c_void_p), ("batch", ctypes.c_int),
        ("A", ctypes.c_void_p), ("Bt", ctypes.c_void_p), ("pa", ctypes.c_int), ("pb", ctypes.c_int),
        ("exec_count", ctypes.c_void_p), ("checksum", ctypes.c_void_p), ("flag", ctypes.c_void_p),
        ("sched", ctypes.c_void_p), ("num_events", ctypes.c_int), ("set_gt", ctypes.c_void_p),
        ("uq_next", ctypes.c_void_p), ("urgent_per_event", ctypes.c_int),
        ("u_exec_count", ctypes.c_void_p), ("ckpt", ctypes.c_void_p), ("stats", ctypes.c_void_p),
        ("c_debug", ctypes.c_void_p), ("n_debug", ctypes.c_uint),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int
_SIGNATURES = {
    "apk_last_error": (ctypes.c_char_p, []),
    "apk_get_device_info": (_I, [_I, ctypes.POINTER(DeviceInfo)]),
    "apk_engine_geometry_of": (_I, [_I, ctypes.POINTER(EngineGeometry)]),
    "apk_persistent_gemm_occupancy": (_I, [_I, ctypes.POINTER(_I)]),
    "apk_persistent_gemm": (_I, [_I, _P, _P, _P, _I, _I, _I, _I, _P, _P, _I, _P]),
    "apk_persistent_gemm_noalloc": (_I, [_I, _P, _P, _P, _I, _I, _I, _I, _P, _I, _P]),
    "apk_urgent_gemm": (_I, [_I, _P, _P, _P, _I, _I, _I, _P, _P, _P]),
    "apk_persistent_yield": (_I, [_I, _I, _I, ctypes.POINTER(YieldParams), _I, _P]),
    "apk_yield_ckpt_floats": (ctypes.c_longlong, [_I]),
    "apk_persistent_yield_occupancy": (_I, [_I, _I, ctypes.POINTER(_I)]),
    "apk_raise_flag": (_I, [_P, _I, _I, _P, _P]),
    "apk_spin_flag": (_I, [_P, _I, ctypes.c_longlong, _P, _P]),
    "apk_clock_probe": (_I, [_P, _I, ctypes.c_longlong, _P]),
    "apk_tiny_oracle": (_I, [ctypes.POINTER(TinyParams), _I, _P]),
}

_lib = None


def header_symbols(path=HEADER):
    """Names of every function declared in include/apk.h."""
    text = open(path).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(apk_\w+)\s*\(", text, re.M)))


def load():
    """Load lib/libapk.so (once) and set argument types. Raises ApkError if
    the library has not been built: there is no fallback path."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ApkError(f"{LIB_PATH} is missing: run __graft_entry__.build() "
                       "(make -C apk_amd) first")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc):
    if rc != APK_OK:
        msg = load().apk_last_error().decode(errors="replace")
        raise ApkError(f"apk error {rc}: {msg}")


def device_info(device=0):
    info = DeviceInfo()
    check(load().apk_get_device_info(device, ctypes.byref(info)))
    return info


def geometry(engine):
    g = EngineGeometry()
    check(load().apk_engine_geometry_of(engine, ctypes.byref(g)))
    return g


def occupancy(engine):
    n = ctypes.c_int(0)
    check(load().apk_persistent_gemm_occupancy(engine, ctypes.byref(n)))
    return n.value


def persistent_gemm(engine, A, B, C, M, N, K, k_chunk, next_task, log, blocks,
                    stream=0):
    """Launch apk_persistent_gemm on device pointers (ints). Asynchronous."""
    check(load().apk_persistent_gemm(engine, A, B, C, M, N, K, k_chunk,
                                     next_task, log, blocks, stream))


def persistent_gemm_noalloc(engine, A, B, C, M, N, K, k_chunk, log, blocks, stream=0):
    """Launch apk_persistent_gemm_noalloc (queue counters in the library's own
    device array; no allocation). Asynchronous."""
    check(load().apk_persistent_gemm_noalloc(engine, A, B, C, M, N, K, k_chunk, log,
                                             blocks, stream))


def urgent_gemm(engine, A, B, C, M, N, K, start_gt=None, end_gt=None, stream=0):
    """Launch apk_urgent_gemm: one block per tile, no queue; optional device
    pointers receive the start (block 0's first instruction) and end ticks.
    Asynchronous."""
    check(load().apk_urgent_gemm(engine, A, B, C, M, N, K, start_gt, end_gt, stream))


def yield_occupancy(engine, poll):
    n = ctypes.c_int(0)
    check(load().apk_persistent_yield_occupancy(engine, poll, ctypes.byref(n)))
    return n.value


def ckpt_floats(engine):
    return int(load().apk_yield_ckpt_floats(engine))


def raise_flag(flag, copies, value, set_gt=None, stream=0):
    """Queue apk_raise_flag on `stream`: store `value` into every flag copy
    and the device tick into *set_gt. Asynchronous."""
    check(load().apk_raise_flag(flag, copies, value, set_gt, stream))


def spin_flag(flag, system_scope, max_ticks, out, stream=0):
    """Queue apk_spin_flag: one wave spins (bounded by max_ticks) until *flag
    reads non-zero; out[0] = device tick of that read (-1 on timeout),
    out[1] = the value. Asynchronous."""
    check(load().apk_spin_flag(flag, 1 if system_scope else 0, max_ticks, out, stream))


def clock_probe(out, blocks, window_ticks, stream=0):
    """Queue apk_clock_probe: `blocks` one-wave blocks count shader-clock
    cycles and wall ticks over window_ticks; out = 4 long longs per block
    (cycles, ticks, xcd, start tick). Asynchronous."""
    check(load().apk_clock_probe(out, blocks, window_ticks, stream))


def persistent_yield(engine, poll, oracle, params, blocks, stream=0):
    """Launch apk_persistent_yield with a YieldParams. Asynchronous."""
    check(load().apk_persistent_yield(engine, poll, 1 if oracle else 0,
                                      ctypes.byref(params), blocks, stream))


def tiny_oracle(params, blocks, stream=0):
    """Launch apk_tiny_oracle with a TinyParams. Asynchronous."""
    check(load().apk_tiny_oracle(ctypes.byref(params), blocks, stream))
