"""Static checks of the gfx950 assembly of every kernel of the library (see
tests/isa_barriers.py): no barrier inside a divergent loop, and no vmcnt
wait inside a k-stage compute block. Compiles each HIP source once."""
import glob
import os
import subprocess

import pytest

from isa_barriers import divergent_barrier_loops, vm_waits_in_compute_blocks

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SOURCES = sorted(glob.glob(os.path.join(ROOT, "apk_amd", "csrc", "*.hip")))


_ASM = {}


def _asm(src, tmp_path):
    if src in _ASM:
        return _ASM[src]
    out = tmp_path / "k.s"
    subprocess.check_call(
        ["/opt/rocm/bin/hipcc", "-std=c++17", "-O3", "--offload-arch=gfx950", "-fPIC",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "apk_amd", "csrc"),
         "-S", "--cuda-device-only", src, "-o", str(out)],
        stderr=subprocess.DEVNULL)
    _ASM[src] = out.read_text()
    return _ASM[src]


@pytest.mark.parametrize("src", SOURCES, ids=[os.path.basename(s) for s in SOURCES])
def test_no_barrier_in_divergent_loop(src, tmp_path):
    bad = divergent_barrier_loops(_asm(src, tmp_path))
    assert not bad, bad


@pytest.mark.parametrize("src", SOURCES, ids=[os.path.basename(s) for s in SOURCES])
def test_no_vm_wait_in_compute_block(src, tmp_path):
    bad = vm_waits_in_compute_blocks(_asm(src, tmp_path))
    assert not bad, bad[:8]


def test_checker_catches_the_pattern():
    # A loop with a per-lane exit and a barrier in its body must be flagged.
    asm = "\n".join([
        "_Z1kv:",
        ".LBB0_1:                                ; =>This Loop Header: Depth=1",
        "\ts_barrier",
        "\ts_andn2_b64 exec, exec, s[4:5]",
        "\ts_cbranch_execnz .LBB0_1",
        "; %bb.2:",
        "\ts_endpgm",
    ])
    assert divergent_barrier_loops(asm) == [("_Z1kv", ".LBB0_1", "BB0_1")]
    clean = asm.replace("\ts_barrier\n", "")
    assert divergent_barrier_loops(clean) == []


def test_vm_wait_checker_catches_the_pattern():
    body = ["\tv_mfma_f32_32x32x2_f32 a[0:15], v1, v2, a[0:15]"] * 40
    asm = "\n".join(["_Z1kv:", ".LBB0_1:", "\ts_waitcnt vmcnt(4)"] + body + ["\ts_endpgm"])
    assert divergent_barrier_loops(asm) == []
    assert vm_waits_in_compute_blocks(asm) == [("_Z1kv", ".LBB0_1", "s_waitcnt vmcnt(4)")]
    assert vm_waits_in_compute_blocks(asm.replace("\ts_waitcnt vmcnt(4)\n", "")) == []
    # The stage wait right before the barrier is the protocol's own; a wait
    # after the barrier, or a second one, is not.
    stage = ["_Z1kv:", ".LBB0_1:", "\ts_waitcnt vmcnt(4)", "\ts_barrier"] + body
    assert vm_waits_in_compute_blocks("\n".join(stage)) == []
    late = stage + ["\ts_waitcnt vmcnt(2)"]
    assert vm_waits_in_compute_blocks("\n".join(late)) == [("_Z1kv", ".LBB0_1", "s_waitcnt vmcnt(2)")]
    pair = ["_Z1kv:", ".LBB0_1:", "\ts_waitcnt vmcnt(0)", "\ts_barrier"] + body
    assert vm_waits_in_compute_blocks("\n".join(pair)) == []
    twice = ["_Z1kv:", ".LBB0_1:", "\ts_waitcnt vmcnt(4)", "\ts_waitcnt vmcnt(0)", "\ts_barrier"] + body
    assert vm_waits_in_compute_blocks("\n".join(twice)) == [("_Z1kv", ".LBB0_1", "s_waitcnt vmcnt(0)")]
    # one-wave workgroups: the compiler's "; wave barrier" marker stands for
    # the dropped s_barrier
    wave = ["_Z1kv:", ".LBB0_1:", "\ts_waitcnt vmcnt(0)", "\t; wave barrier"] + body
    assert vm_waits_in_compute_blocks("\n".join(wave)) == []
    wave_late = wave + ["\ts_waitcnt vmcnt(0)"]
    assert vm_waits_in_compute_blocks("\n".join(wave_late)) == [("_Z1kv", ".LBB0_1", "s_waitcnt vmcnt(0)")]
