"""Benchmark of the GGUF quantized matmul path on one MI355X.

Headline (BASELINE.json metric): Q4_K matvec GB/s at K->N = 4096->14336, M=1,
plus the M=512 Q4_K qmatmul in TOPS.  One "step" is one xn-style
`QTensor::matmul_t` call: quantize the f32 activation row to Q8_K, then the
Q4_K matvec, on weights already resident in HBM.  Weight copies are rotated
(> 512 MB in total) so every step streams its weight from HBM rather than
from the 256 MB Infinity Cache.  Steps are captured in a HIP graph and the
graph replay is timed with HIP events on the capture stream.

Prints one JSON line (see `result` below).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0

K_DIM, N_DIM = 4096, 14336
Q4K_BYTES_PER_SB = 144


def weight_bytes(n: int, k: int) -> int:
    return n * (k // 256) * Q4K_BYTES_PER_SB


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--copies", type=int, default=16, help="rotated weight copies (16 x 33 MB = 528 MB)")
    p.add_argument("--prefill-m", type=int, default=512)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--only", choices=["all", "matvec", "prefill", "copy"], default="all",
                   help="'copy' times a plain 512 MiB device copy (calibrates the HBM byte counters)")
    p.add_argument("--eager", action="store_true",
                   help="launch steps one by one instead of replaying a HIP graph (for counter runs)")
    return p.parse_args()


class Eager:
    """Stand-in for a captured graph: `replay` launches the steps directly."""

    def __init__(self, fn, steps: int):
        self.fn, self.steps = fn, steps

    def replay(self):
        for i in range(self.steps):
            self.fn(i)


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "hbm_traffic_q4k_matvec_k4096_n14336_m1.md")


def measured_traffic():
    """HBM bytes per launch of the matvec kernel, as recorded from the
    FETCH_SIZE / WRITE_SIZE counter runs (scaled by the copy calibration)."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def capture(fn, steps: int, stream, eager: bool = False):
    import torch

    if eager:
        return Eager(fn, steps)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(steps):
            fn(i)
    return g


def time_graph(g, stream, reps: int = 5) -> float:
    """Median over `reps` replays of the graph's duration in ms (HIP events on `stream`)."""
    import torch

    times = []
    for _ in range(reps):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            start.record(stream)
            g.replay()
            end.record(stream)
        end.synchronize()
        times.append(start.elapsed_time(end))
    return float(np.median(times))


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                          "(multi-GPU sharding is described in DESIGN.md, not implemented)"}))
        sys.exit(2)

    import torch

    from xn_amd import GgmlDType, QTensor
    from xn_amd.quantized import lhs_workspace, matmul_preq, quantize_lhs

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev).manual_seed(299792458)
    stream = torch.cuda.Stream(dev)

    result = {
        "metric": "Q4_K matvec GB/s (% HBM peak) at 4096x14336; M=512 qmatmul TOPS (% MFMA)",
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4k-weights x q8k-activations, int32 block dots, f32 combine",
        "data": "synthetic: weights N(0,0.02) quantized to Q4_K on device, activations N(0,1), seed 299792458",
        "config": {"workload": "q4k_matvec_k4096_n14336_m1", "k": K_DIM, "n": N_DIM, "m": 1,
                   "weight_copies": args.copies, "parallelism": "single GPU"},
    }

    if args.only == "copy":
        nbytes = 512 << 20
        src = torch.empty(nbytes // 4, device=dev, dtype=torch.float32).fill_(1.0)
        dst = torch.empty_like(src)
        with torch.cuda.stream(stream):
            for _ in range(3):
                dst.copy_(src)
            g = capture(lambda i: dst.copy_(src), 10, stream, args.eager)
        ms = time_graph(g, stream) / 10
        print(json.dumps({"metric": "device copy GB/s (read + write)", "bytes_read": nbytes,
                          "bytes_written": nbytes, "ms_per_copy": round(ms, 5),
                          "value": round(2 * nbytes / (ms * 1e-3) / 1e9, 1), "unit": "GB/s"}), flush=True)
        return

    # ---------------- weights: rotated copies, quantized on the device
    copies = []
    for _ in range(args.copies):
        w = torch.randn((N_DIM, K_DIM), generator=gen, device=dev, dtype=torch.float32) * 0.02
        copies.append(QTensor.quantize_f32(w, (N_DIM, K_DIM), GgmlDType.Q4K))
        del w
    torch.cuda.synchronize()
    wbytes = weight_bytes(N_DIM, K_DIM)
    algo_bytes = wbytes + K_DIM * 4 + N_DIM * 4  # weights + f32 x + f32 y

    if args.only in ("all", "matvec"):
        x = torch.randn((1, K_DIM), generator=gen, device=dev, dtype=torch.float32)
        y = torch.empty((1, N_DIM), device=dev, dtype=torch.float32)
        ws = lhs_workspace(GgmlDType.Q4K, 1, K_DIM, dev)

        def step(i):
            copies[i % len(copies)].matmul_t((1, K_DIM, N_DIM), x, y)

        def kernel_only(i):
            matmul_preq(copies[i % len(copies)], 1, ws, y)

        with torch.cuda.stream(stream):
            for i in range(args.warmup):
                step(i)
            quantize_lhs(GgmlDType.Q4K, x, ws, 1, K_DIM)
            for i in range(args.warmup):
                kernel_only(i)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            g_step = capture(step, args.steps, stream, args.eager)
            g_kern = capture(kernel_only, args.steps, stream, args.eager)
        torch.cuda.synchronize()
        ms_step = time_graph(g_step, stream) / args.steps
        ms_kern = time_graph(g_kern, stream) / args.steps
        value = algo_bytes / (ms_step * 1e-3) / 1e9
        achieved = algo_bytes / (ms_kern * 1e-3) / 1e9
        result.update({
            "value": round(value, 1),
            "ms_per_step": round(ms_step, 5),
            "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        })
        result["roofline"] = {
            "bound": "hbm",
            "kernel": "matvec_kernel<Q4K, MB=1>",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
            "traffic_source": "rocprofv3 --pmc FETCH_SIZE (x2.000) + WRITE_SIZE (x1.000), "
                              "profiles/hbm_traffic_q4k_matvec_k4096_n14336_m1.md",
            "algorithmic_bytes_per_launch": algo_bytes,
            "avg_launch_us": round(ms_kern * 1e3, 3),
        }
        del g_step, g_kern

    if args.only in ("all", "prefill"):
        m = args.prefill_m
        xp = torch.randn((m, K_DIM), generator=gen, device=dev, dtype=torch.float32)
        yp = torch.empty((m, N_DIM), device=dev, dtype=torch.float32)
        wsp = lhs_workspace(GgmlDType.Q4K, m, K_DIM, dev)
        psteps = max(5, min(50, args.steps // 4))

        def pstep(i):
            copies[i % len(copies)].matmul_t((m, K_DIM, N_DIM), xp, yp)

        def pkern(i):
            matmul_preq(copies[i % len(copies)], m, wsp, yp)

        with torch.cuda.stream(stream):
            for i in range(3):
                pstep(i)
            quantize_lhs(GgmlDType.Q4K, xp, wsp, m, K_DIM)
            for i in range(3):
                pkern(i)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            gp = capture(pstep, psteps, stream, args.eager)
            gk = capture(pkern, psteps, stream, args.eager)
        ms_p = time_graph(gp, stream) / psteps
        ms_k = time_graph(gk, stream) / psteps
        ops = 2.0 * m * N_DIM * K_DIM
        result["prefill"] = {
            "workload": f"q4k_qmatmul_m{m}_k{K_DIM}_n{N_DIM}",
            "ms_per_call": round(ms_p, 4),
            "tops": round(ops / (ms_p * 1e-3) / 1e12, 2),
            "kernel_ms": round(ms_k, 4),
            "kernel_tops": round(ops / (ms_k * 1e-3) / 1e12, 2),
            "frac_int8_peak": round(ops / (ms_k * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4),
            "peak_tops": INT8_PEAK_TOPS,
        }
        if args.only == "prefill":
            result["value"] = result["prefill"]["tops"]
            result["unit"] = "TOPS"
            result["ms_per_step"] = result["prefill"]["ms_per_call"]

    # ---------------- CPU baseline: the xn-style AVX2 path on the host cores
    if not args.no_cpu and args.only in ("all", "matvec"):
        import oracle

        threads = min(os.cpu_count() or 1, 16)
        oracle.cpu_pool_init(threads)
        ncopies = min(16, len(copies))  # > 512 MB, past any host L3
        host_w = [np.frombuffer(copies[i].data(), dtype=np.uint8) for i in range(ncopies)]
        xh = np.random.default_rng(1).normal(0, 1, (1, K_DIM)).astype(np.float32)
        scratch = np.zeros(oracle.nbytes(oracle.Q8K, K_DIM), dtype=np.uint8)
        oracle.cpu_matmul(oracle.Q4K, xh, host_w[0], N_DIM, scratch)
        times = []
        t_end = time.perf_counter() + args.cpu_seconds
        i = 0
        while time.perf_counter() < t_end or len(times) < 5:
            t0 = time.perf_counter()
            oracle.cpu_matmul(oracle.Q4K, xh, host_w[i % ncopies], N_DIM, scratch)
            times.append(time.perf_counter() - t0)
            i += 1
        med = float(np.median(times))
        # the same calls without the activation quantization (kernel only)
        lhs_q = oracle.quantize_lhs(oracle.Q4K, xh)
        times_k = []
        t_end = time.perf_counter() + args.cpu_seconds / 2
        while time.perf_counter() < t_end or len(times_k) < 5:
            t0 = time.perf_counter()
            oracle.cpu_matmul_preq(oracle.Q4K, lhs_q, host_w[i % ncopies], 1, K_DIM, N_DIM)
            times_k.append(time.perf_counter() - t0)
            i += 1
        med_k = float(np.median(times_k))
        result["cpu_baseline"] = {
            "value": round(algo_bytes / med / 1e9, 2),
            "unit": "GB/s",
            "cores": threads,
            "kind": "port",
            "value_excl_quantize": round(algo_bytes / med_k / 1e9, 2),
            "sample": f"{len(times)} calls of Q4_K 4096->14336 M=1 (quantize_lhs + AVX2 vec_dot_q4k_q8k over "
                      f"128-column tasks), {ncopies} rotated weight copies, median {med * 1e3:.3f} ms; "
                      f"value_excl_quantize: {len(times_k)} calls on pre-quantized lhs, median {med_k * 1e3:.3f} ms",
        }

    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
