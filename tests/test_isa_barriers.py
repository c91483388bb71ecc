"""Every gfx950 kernel of the library is free of barriers inside divergent
loops (see tests/isa_barriers.py). Compiles each HIP source to assembly."""
import glob
import os
import subprocess

import pytest

from isa_barriers import divergent_barrier_loops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SOURCES = sorted(glob.glob(os.path.join(ROOT, "apk_amd", "csrc", "*.hip")))


@pytest.mark.parametrize("src", SOURCES, ids=[os.path.basename(s) for s in SOURCES])
def test_no_barrier_in_divergent_loop(src, tmp_path):
    out = tmp_path / "k.s"
    subprocess.check_call(
        ["/opt/rocm/bin/hipcc", "-std=c++17", "-O3", "--offload-arch=gfx950", "-fPIC",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROOT, "apk_amd", "csrc"),
         "-S", "--cuda-device-only", src, "-o", str(out)],
        stderr=subprocess.DEVNULL)
    bad = divergent_barrier_loops(out.read_text())
    assert not bad, bad


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
