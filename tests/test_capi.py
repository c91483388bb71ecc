"""C ABI surface on the CPU: the library loads, exports every function that
include/apk.h declares, and rejects bad arguments before touching a GPU."""
import ctypes
import re
import subprocess

import pytest

import apk_amd


def test_header_declares_functions():
    syms = apk_amd.header_symbols()
    assert "apk_persistent_gemm" in syms and "apk_last_error" in syms
    assert len(syms) >= 5


def test_library_exports_every_header_symbol():
    lib = apk_amd.load()
    missing = [s for s in apk_amd.header_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    out = subprocess.check_output(["nm", "-D", "--defined-only", apk_amd.LIB_PATH]).decode()
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(apk_amd.header_symbols()) <= exported


def test_engine_geometry():
    g = apk_amd.geometry(apk_amd.ENGINE_VALU64)
    assert (g.tile_m, g.tile_n, g.k_stage, g.threads) == (64, 64, 32, 256)
    assert (g.elem_bytes, g.b_transposed) == (4, 0)
    g = apk_amd.geometry(apk_amd.ENGINE_MFMA128)
    assert (g.tile_m, g.tile_n, g.k_stage, g.threads) == (128, 128, 32, 256)
    assert g.lds_bytes <= 160 * 1024
    g = apk_amd.geometry(apk_amd.ENGINE_BF16X256)
    assert (g.tile_m, g.tile_n, g.k_stage, g.threads) == (256, 256, 32, 512)
    assert (g.elem_bytes, g.b_transposed) == (2, 1)
    assert g.lds_bytes <= 160 * 1024
    # the small bf16 tiles: 4 (one wave each) and 2 blocks per CU fit LDS
    g = apk_amd.geometry(apk_amd.ENGINE_BF16X128)
    assert (g.tile_m, g.tile_n, g.k_stage, g.threads) == (128, 128, 16, 64)
    assert (g.elem_bytes, g.b_transposed) == (2, 1) and 4 * g.lds_bytes <= 160 * 1024
    g = apk_amd.geometry(apk_amd.ENGINE_BF16X256X128)
    assert (g.tile_m, g.tile_n, g.k_stage, g.threads) == (256, 128, 16, 256)
    assert (g.elem_bytes, g.b_transposed) == (2, 1) and 2 * g.lds_bytes <= 160 * 1024
    with pytest.raises(apk_amd.ApkError):
        apk_amd.geometry(99)



@pytest.mark.parametrize("engine,M,N,K,kc,blocks,frag", [
    (apk_amd.ENGINE_VALU64, 100, 64, 64, 64, 4, "multiples"),
    (apk_amd.ENGINE_MFMA128, 128, 128, 96, 64, 4, "k_chunk"),
    (apk_amd.ENGINE_MFMA128, 128, 128, 64, 48, 4, "k_chunk"),
    (apk_amd.ENGINE_VALU64, 64, 64, 64, 64, 0, "blocks"),
    (apk_amd.ENGINE_VALU64, 0, 64, 64, 64, 1, "empty"),
    (apk_amd.ENGINE_BF16X256, 256, 128, 64, 64, 4, "multiples"),
    (apk_amd.ENGINE_BF16X256, 256, 256, 64, 48, 4, "k_chunk"),
    # the bf16 tiles load a pair of stages as one region: an even number of
    # stages (2 x 32 k for the 256x256 tile, 2 x 16 k for the others)
    (apk_amd.ENGINE_BF16X256, 256, 256, 96, 32, 4, "multiple of 64"),
    (apk_amd.ENGINE_BF16X128, 128, 128, 48, 48, 4, "multiple of 32"),
    (apk_amd.ENGINE_BF16X256X128, 256, 128, 80, 16, 4, "multiple of 32"),
    (apk_amd.ENGINE_BF16X256X128, 128, 128, 64, 16, 4, "multiples"),
    (7, 64, 64, 64, 64, 1, "engine"),
])
def test_persistent_gemm_rejects_bad_args(engine, M, N, K, kc, blocks, frag):
    lib = apk_amd.load()
    fake = ctypes.c_void_p(0x1000)   # never dereferenced: rejected on the host
    rc = lib.apk_persistent_gemm(engine, fake, fake, fake, M, N, K, kc, fake, None, blocks, None)
    assert rc == apk_amd.APK_EINVAL
    assert frag in lib.apk_last_error().decode()


def test_null_pointers_rejected():
    lib = apk_amd.load()
    rc = lib.apk_persistent_gemm(0, None, None, None, 64, 64, 64, 64, None, None, 1, None)
    assert rc == apk_amd.APK_EINVAL


def test_yield_params_layout_matches_header(tmp_path):
    """The ctypes mirror of apk_yield_params has the C compiler's layout."""
    src = tmp_path / "sz.c"
    fields = [f[0] for f in apk_amd.YieldParams._fields_]
    body = "".join(f'printf("%zu ", offsetof(apk_yield_params, {f}));' for f in fields)
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "apk.h"\n'
                   'int main(){' + body + 'printf("%zu\\n", sizeof(apk_yield_params));return 0;}\n')
    exe = tmp_path / "sz"
    subprocess.check_call(["gcc", "-I", apk_amd.os.path.join(apk_amd.ROOT, "include"),
                           str(src), "-o", str(exe)])
    got = [int(x) for x in subprocess.check_output([str(exe)]).split()]
    want = [getattr(apk_amd.YieldParams, f).offset for f in fields] + [ctypes.sizeof(apk_amd.YieldParams)]
    assert got == want


def test_yield_rejects_bad_args():
    lib = apk_amd.load()
    p = apk_amd.YieldParams()
    fake = 0x1000
    p.A = p.B = p.C = p.next_task = fake
    p.M, p.N, p.K, p.k_chunk = 128, 128, 64, 48
    rc = lib.apk_persistent_yield(apk_amd.ENGINE_MFMA128, apk_amd.POLL_STAGE, 0, ctypes.byref(p), 1, None)
    assert rc == apk_amd.APK_EINVAL and b"k_chunk" in lib.apk_last_error()
    p.k_chunk = 32
    rc = lib.apk_persistent_yield(apk_amd.ENGINE_MFMA128, apk_amd.POLL_STAGE, 0, ctypes.byref(p), 1, None)
    assert rc == apk_amd.APK_EINVAL and b"flag" in lib.apk_last_error()
    p.flag = fake
    p.resume = apk_amd.RESUME_CKPT_FULL
    rc = lib.apk_persistent_yield(apk_amd.ENGINE_MFMA128, apk_amd.POLL_STAGE, 0, ctypes.byref(p), 1, None)
    assert rc == apk_amd.APK_EINVAL and b"ckpt" in lib.apk_last_error()
    p.resume = apk_amd.RESUME_RESTART
    p.num_events = 3
    rc = lib.apk_persistent_yield(apk_amd.ENGINE_MFMA128, apk_amd.POLL_STAGE, 0, ctypes.byref(p), 1, None)
    assert rc == apk_amd.APK_EINVAL and b"event array" in lib.apk_last_error()
    p.num_events = 0
    p.Au = fake
    p.Bu = p.Cu = fake
    p.Mu, p.Nu, p.Ku = 100, 128, 32
    rc = lib.apk_persistent_yield(apk_amd.ENGINE_MFMA128, apk_amd.POLL_STAGE, 0, ctypes.byref(p), 1, None)
    assert rc == apk_amd.APK_EINVAL and b"urgent" in lib.apk_last_error()
    # accumulators (floats per thread x threads) + every ring slot (an issue
    # site keeps up to NS live stages: 3 x 32 KiB, 3 x 16 KiB, 4 x 32 KiB)
    assert apk_amd.ckpt_floats(apk_amd.ENGINE_MFMA128) == 64 * 256 + 3 * 32 * 1024 // 4
    assert apk_amd.ckpt_floats(apk_amd.ENGINE_VALU64) == 16 * 256 + 3 * 16 * 1024 // 4
    assert apk_amd.ckpt_floats(apk_amd.ENGINE_BF16X256) == 128 * 512 + 4 * 32 * 1024 // 4


def test_python_constants_match_header():
    text = open(apk_amd.HEADER).read()
    defines = dict(re.findall(r"#define (APK_\w+) (\d+)", text))
    assert int(defines["APK_FLAG_STRIDE"]) == apk_amd.FLAG_STRIDE
    assert int(defines["APK_FLAG_MAX_COPIES"]) == apk_amd.FLAG_MAX_COPIES
    assert int(defines["APK_STATS_PER_BLOCK"]) == apk_amd.STATS_PER_BLOCK
    assert int(defines["APK_QUEUE_WORDS"]) == apk_amd.QUEUE_WORDS
    assert int(defines["APK_QUEUE_XCDS"]) == apk_amd.QUEUE_XCDS
    assert int(defines["APK_SES_PER_XCD"]) == apk_amd.SES_PER_XCD
    assert int(defines["APK_RETREAT_DOMAINS"]) == apk_amd.RETREAT_DOMAINS == 32
    assert int(defines["APK_RQ_CTL_WORDS"]) == apk_amd.RQ_CTL_WORDS == 4
    stats = dict(re.findall(r"(APK_ST_\w+) = (\d+)", text))
    assert int(stats["APK_ST_DECLINED"]) == apk_amd.ST_DECLINED == 12
    assert int(stats["APK_ST_START_SITES"]) == apk_amd.ST_START_SITES == 13
    assert int(stats["APK_ST_ERRORS"]) == apk_amd.ST_ERRORS == 7


def test_retreat_arm_rejects_bad_args():
    lib = apk_amd.load()
    p = apk_amd.YieldParams()
    fake = 0x1000
    p.A = p.B = p.C = p.next_task = p.flag = fake
    p.M, p.N, p.K, p.k_chunk = 128, 128, 64, 32
    p.resume = apk_amd.RESUME_CKPT_FULL
    p.retreat = 2
    call = lambda: lib.apk_persistent_yield(apk_amd.ENGINE_MFMA128, apk_amd.POLL_STAGE, 0,
                                            ctypes.byref(p), 1, None)
    assert call() == apk_amd.APK_EINVAL and b"resume queue" in lib.apk_last_error()
    p.num_events = 1
    p.retreat_count = p.rq_ctl = p.rq_entry = fake
    # a ring of one entry cannot tell "published by ticket t" (seq t + 1)
    # from "free for ticket t + 1" (t + capacity): at least 2 entries
    for cap in (0, 1):
        p.rq_capacity = cap
        assert call() == apk_amd.APK_EINVAL and b"at least 2 entries" in lib.apk_last_error()
    p.rq_capacity = 2
    assert call() == apk_amd.APK_EINVAL and b"rq_slots" in lib.apk_last_error()
    p.rq_slots = fake
    p.Au = fake
    assert call() == apk_amd.APK_EINVAL and b"no urgent job" in lib.apk_last_error()
    p.Au = None
    p.retreat = -1
    assert call() == apk_amd.APK_EINVAL and b"retreat" in lib.apk_last_error()
    p.retreat = 0
    p.num_events = 0
    p.ckpt = fake
    p.block_base = 3
    assert call() == apk_amd.APK_EINVAL and b"block_base" in lib.apk_last_error()


def test_raise_flag_rejects_bad_args():
    lib = apk_amd.load()
    assert lib.apk_raise_flag(None, 1, 1, None, None) == apk_amd.APK_EINVAL
    assert lib.apk_raise_flag(ctypes.c_void_p(0x1000), 0, 1, None, None) == apk_amd.APK_EINVAL
    assert b"flag_copies" in lib.apk_last_error()


def test_tiny_params_layout_matches_header(tmp_path):
    src = tmp_path / "tz.c"
    fields = [f[0] for f in apk_amd.TinyParams._fields_]
    body = "".join(f'printf("%zu ", offsetof(apk_tiny_params, {f}));' for f in fields)
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "apk.h"\n'
                   'int main(){' + body + 'printf("%zu\\n", sizeof(apk_tiny_params));return 0;}\n')
    exe = tmp_path / "tz"
    subprocess.check_call(["gcc", "-I", apk_amd.os.path.join(apk_amd.ROOT, "include"),
                           str(src), "-o", str(exe)])
    got = [int(x) for x in subprocess.check_output([str(exe)]).split()]
    want = [getattr(apk_amd.TinyParams, f).offset for f in fields] + [ctypes.sizeof(apk_amd.TinyParams)]
    assert got == want


def test_tiny_oracle_rejects_bad_args():
    lib = apk_amd.load()
    p = apk_amd.TinyParams()
    call = lambda blocks=1: lib.apk_tiny_oracle(ctypes.byref(p), blocks, None)
    assert call() == apk_amd.APK_EINVAL and b"NULL" in lib.apk_last_error()
    fake = 0x1000
    p.next_task = p.A = p.Bt = p.exec_count = p.checksum = p.flag = p.ckpt = fake
    assert call() == apk_amd.APK_EINVAL and b"batch" in lib.apk_last_error()
    p.batch, p.pa, p.pb = 1, 4, 4
    assert call(0) == apk_amd.APK_EINVAL and b"blocks" in lib.apk_last_error()
    p.num_events = 3
    assert call() == apk_amd.APK_EINVAL and b"events need" in lib.apk_last_error()
