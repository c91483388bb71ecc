"""bench.py -- one JSON line for the MI355X preemptible persistent GEMM.

Workload ("tile calibration"): persistent fp32 SGEMM
M=N=K=4096, 128x128 output tiles (MFMA128 engine), per-tile K chunk 32, one
worker per CU slot, no yields. A step is one full pass of the worker pool over
the 1024 output tiles; inputs are resident in HBM before the timed region.
`value` is whole-job GEMM throughput in TFLOP/s.

Also reported (same line): the roofline of the GEMM kernel (fp32 MFMA dense
peak 157.3 TFLOP/s; per-launch duration from HIP events on the launch stream),
and the CPU baseline: the reference's float64 host GEMM (i-k-j,
src/persistent.cu:221-227, restated in oracle/) timed on this host on a
bounded sample of the same GEMM's rows.

Usage: python bench.py [--gpus 1] [--steps 10] [--warmup 3]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = ("urgent-task preempt latency p50/p99 (us); persistent GEMM TFLOP/s; "
          "yield overhead %")
PEAK_FP32_TF = 157.3


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_baseline(A_host, B_host, C_gpu_rows, rows):
    """Reference float64 host GEMM on `rows` rows (single thread), timed; the
    same rows double as a correctness check of the GPU output."""
    import numpy as np
    import oracle
    t0 = time.perf_counter()
    ref = oracle.gemm_f64_rows(A_host, B_host, 0, rows)
    dt = time.perf_counter() - t0
    K = A_host.shape[1]
    N = B_host.shape[1]
    flop = 2.0 * rows * N * K
    frob = oracle.rel_frobenius(C_gpu_rows, ref)
    return {
        "value": flop / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"rows 0..{rows - 1} of the {A_host.shape[0]}x{N}x{K} GEMM in float64, "
                   f"i-k-j order (src/persistent.cu:221-227), 1 thread, {dt:.1f} s"),
        "seconds": dt,
    }, frob


def measured_traffic(profile="profiles/persistent_gemm_mfma128_cfg2.md"):
    """HBM-side bytes per launch of the GEMM kernel as measured by the two
    rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE, scaled by a plain copy) and
    recorded in the profile summary; None if not recorded."""
    path = os.path.join(ROOT, profile)
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":")[1])
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--size", type=int, default=4096)
    ap.add_argument("--k-chunk", type=int, default=32)
    ap.add_argument("--cpu-rows", type=int, default=1024)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB (the "
                         "known-size kernel that scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only; the preemptible persistent "
              "GEMM has no multi-GPU path (see DESIGN.md for how it would shard).",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import apk_amd

    torch.cuda.set_device(0)
    if args.calibrate_copy:
        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copied {args.calibrate_copy} MiB x3")
        return
    apk_amd.load()
    info = apk_amd.device_info()
    eng = apk_amd.ENGINE_MFMA128
    occ = apk_amd.occupancy(eng)
    blocks = info.cu_count * occ
    S = args.size
    M = N = K = S
    kc = args.k_chunk
    flop = 2.0 * M * N * K

    gen = torch.Generator(device="cuda")
    gen.manual_seed(21)
    dA = torch.rand((M, K), generator=gen, device="cuda", dtype=torch.float32) * 2 - 1
    dB = torch.rand((K, N), generator=gen, device="cuda", dtype=torch.float32) * 2 - 1
    dC = torch.empty((M, N), device="cuda", dtype=torch.float32)
    total = args.warmup + args.steps
    counters = torch.zeros((total, apk_amd.QUEUE_WORDS), dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(total)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(total)]
    torch.cuda.synchronize()
    log(f"device {info.name.decode()} {info.arch.decode()} CUs={info.cu_count} "
        f"occupancy={occ}/CU blocks={blocks}")

    def step(i):
        starts[i].record(stream)
        apk_amd.persistent_gemm(eng, dA.data_ptr(), dB.data_ptr(), dC.data_ptr(),
                                M, N, K, kc, counters[i].data_ptr(), None, blocks,
                                stream.cuda_stream)
        ends[i].record(stream)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.warmup, total):
        step(i)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    launch_ms = [starts[i].elapsed_time(ends[i]) for i in range(args.warmup, total)]
    avg_launch_ms = float(np.mean(launch_ms))
    value = flop / (ms_per_step * 1e-3) / 1e12
    achieved = flop / (avg_launch_ms * 1e-3) / 1e12
    log(f"GEMM {M}x{N}x{K} kc={kc}: {ms_per_step:.3f} ms/step wall, "
        f"{avg_launch_ms:.3f} ms/launch (events) -> {value:.1f} TFLOP/s")

    out = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": (f"cfg2 tile calibration: persistent fp32 SGEMM M=N=K={S}, "
                         f"128x128 tiles (MFMA128, v_mfma_f32_32x32x2_f32), "
                         f"k_chunk={kc}, {blocks} workers, no yields"),
            "M": M, "N": N, "K": K, "tile": [128, 128], "k_chunk": kc,
            "workers": blocks, "workers_per_cu": occ,
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": PEAK_FP32_TF,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_FP32_TF, 4),
            "traffic": measured_traffic() if (S, kc) == (4096, 32) else None,
        },
    }
    if not args.no_cpu:
        rows = args.cpu_rows
        A_host = dA[:rows].cpu().numpy()
        B_host = dB.cpu().numpy()
        C_rows = dC[:rows].cpu().numpy()
        cb, frob = cpu_baseline(A_host, B_host, C_rows, rows)
        out["cpu_baseline"] = {k: v for k, v in cb.items() if k != "seconds"}
        out["check"] = {"rows": rows, "rel_frobenius_vs_f64": frob, "tol": 1e-5,
                        "pass": bool(frob <= 1e-5)}
        log(f"cpu baseline {cb['value'] * 1e3:.3f} GFLOP/s ({cb['seconds']:.1f} s); "
            f"GPU rows rel-Frobenius {frob:.2e}")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
