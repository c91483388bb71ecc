"""Generate tests/golden/golden.json: known answers from sources independent of
the oracle, used to pin oracle/oracle.cpp.

Sources (none of them is the oracle or the product):
  * libc's own srand()/rand() through ctypes -- the generator the reference
    calls for its inputs (src/persistent.cu:131-135);
  * numpy's MT19937 with legacy (init_genrand) seeding -- the same seeding as
    std::mt19937(seed);
  * libstdc++'s std::mt19937 + uniform_real_distribution +
    exponential_distribution, compiled here with g++ from the small program
    below -- the exact library calls of the reference's schedule
    (src/yield.cu:824-830);
  * torch's float32 -> bfloat16 cast (round to nearest even).

Run: python tests/golden/make_golden.py   (writes golden.json next to it)
"""
import ctypes
import json
import os
import subprocess
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

CXX_SRC = r"""
#include <cstdio>
#include <random>
int main() {
  const unsigned seeds[] = {21u, 7u};
  for (unsigned s : seeds) {
    std::mt19937 rng(s);
    std::uniform_real_distribution<double> gap(150.0 * 1000.0, 400.0 * 1000.0);
    long long acc = 0;
    printf("U %u", s);
    for (int e = 0; e < 64; ++e) { acc += (long long)gap(rng); printf(" %lld", acc); }
    printf("\n");
  }
  for (unsigned s : seeds) {
    std::mt19937 rng(s);
    std::exponential_distribution<double> gap(1.0 / (2000.0 * 1000.0));
    long long acc = 0;
    printf("E %u", s);
    for (int e = 0; e < 64; ++e) { acc += (long long)gap(rng); printf(" %lld", acc); }
    printf("\n");
  }
  return 0;
}
"""


def glibc_rand(seeds, n, idx_far):
    libc = ctypes.CDLL("libc.so.6")
    libc.rand.restype = ctypes.c_int
    out = {}
    for s in seeds:
        libc.srand(ctypes.c_uint(s))
        vals = [libc.rand() for _ in range(idx_far + 1)]
        out[str(s)] = {"first": vals[:n], "far_index": idx_far, "far": vals[idx_far]}
    return out


def mt_raw(seeds, n):
    out = {}
    for s in seeds:
        bg = np.random.MT19937()
        bg._legacy_seeding(s)
        out[str(s)] = [int(x) for x in bg.random_raw(n)]
    return out


def libstdcxx_schedules():
    with tempfile.TemporaryDirectory() as td:
        src = os.path.join(td, "sched.cpp")
        exe = os.path.join(td, "sched")
        open(src, "w").write(CXX_SRC)
        subprocess.check_call(["g++", "-O2", "-std=c++17", "-o", exe, src])
        text = subprocess.check_output([exe]).decode()
    uni, expo = {}, {}
    for line in text.strip().splitlines():
        kind, seed, *vals = line.split()
        (uni if kind == "U" else expo)[seed] = [int(v) for v in vals]
    return uni, expo


def bf16_cases():
    import torch
    xs = [0.0, -0.0, 1.0, -1.0, 1.00390625, 1.005859375, 1.0029296875,
          3.14159265, -2.71828182, 1e-40, -1e-40, 3.0e38, 65504.0, 1.0 / 3.0,
          0.1, -0.1, 255.5, 1.00048828125, 1.001953125]
    t = torch.tensor(xs, dtype=torch.float32).to(torch.bfloat16)
    bits = t.view(torch.int16).numpy().astype(np.uint16)
    return [{"x": float(np.float32(x)), "bits": int(b)} for x, b in zip(xs, bits)]


def main():
    uni, expo = libstdcxx_schedules()
    golden = {
        "glibc_rand": glibc_rand([0, 1, 21, 12345], 8, 100000),
        "mt19937_raw": mt_raw([5489, 21, 7], 16),
        # C++11 [rand.predef]: the 10000th consecutive invocation of a
        # default-constructed std::mt19937 produces 4123659995.
        "mt19937_default_10000th": 4123659995,
        "uniform_schedule_us_150_400": uni,
        "exp_schedule_mean_2000us": expo,
        "bf16_rne": bf16_cases(),
    }
    with open(os.path.join(HERE, "golden.json"), "w") as f:
        json.dump(golden, f, indent=1)
    print("wrote golden.json")


if __name__ == "__main__":
    main()
