"""Benchmark of the GGUF quantized matmul path on one MI355X.

Headline (BASELINE.json metric): Q4_K matvec GB/s at K->N = 4096->14336, M=1,
plus the M=512 Q4_K qmatmul in TOPS.  One "step" is one xn-style
`QTensor::matmul_t` call: quantize the f32 activation row to Q8_K and
multiply it with the Q4_K weight (at M=1, K=4096 one kernel that quantizes
the row in LDS, then streams the weight), on weights already resident in
HBM.  Weight copies are rotated
(> 512 MB in total) so every step streams its weight from HBM rather than
from the 256 MB Infinity Cache.  Steps are captured in a HIP graph and the
graph replay is timed with HIP events on the capture stream.

Unless --no-cpu is given, the outputs of the last timed replays (the M=1 row,
16 sampled rows of the M=512 product) are compared with the CPU oracle on the
same inputs and weights (`check` in the JSON line); bench.py exits with status
1 when they differ beyond the parity tolerance.

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


GPU_BOX_CPU_SHARE = 16  # CPUs a one-GPU job may keep busy on the GPU boxes


def host_threads() -> int:
    """Threads of the CPU baseline pool: xn sizes its pool from
    RAYON_NUM_THREADS, else num_cpus::get() (utils.rs:16-27); here the CPUs
    this process may run on, capped at the GPU box's per-GPU CPU share."""
    avail = len(os.sched_getaffinity(0))
    env = os.environ.get("RAYON_NUM_THREADS", "")
    want = int(env) if env.isdigit() and int(env) > 0 else avail
    return max(1, min(want, avail, GPU_BOX_CPU_SHARE))


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--copies", type=int, default=16, help="rotated weight copies (16 x 33 MB = 528 MB)")
    p.add_argument("--prefill-m", type=int, default=512)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--only", choices=["all", "matvec", "prefill", "copy", "stream", "sweep", "decode"],
                   default="all",
                   help="'copy' times a plain 512 MiB device copy (calibrates the HBM byte counters); "
                        "'stream' times a bare read of the headline weight's bytes (the matvec's ceiling); "
                        "'sweep' times every configured shape (matvec sweep, FFN, prefill, decode step)")
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


# The parity tolerance of the f32 outputs (the same as the GPU tests'):
# relative L2 over the whole output, and per row the largest absolute error
# relative to the row's largest |value|.
REL_L2, ROW_MAX_REL = 1e-3, 2e-3


def close_stats(got: np.ndarray, want: np.ndarray) -> tuple:
    got = got.reshape(want.shape).astype(np.float64)
    want = want.astype(np.float64)
    rel = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    row = np.abs(got - want).max(axis=1) / np.maximum(np.abs(want).max(axis=1), 1e-30)
    return float(rel), float(row.max())


WEIGHT_BYTES = {2: (32, 18), 8: (32, 34), 12: (256, 144), 14: (256, 210)}  # dtype: (block elems, block bytes)


def qbytes(dt: int, n: int, k: int) -> int:
    be, bb = WEIGHT_BYTES[dt]
    return n * (k // be) * bb


def sweep(args, dev, stream, gen) -> dict:
    """Every configured shape: the Q8_0 matvec, the Q4_0 FFN block with its
    SiLU gate, the Q4_K (and Q6_K / Q4_0) matvec sweep over M = 1, 2, 4, 8,
    the int8-MFMA prefill at M = 64 .. 2048, and all QMatMuls of one decode
    step of the 32-layer model (batch 1 and 16).  Rates use the algorithmic
    bytes of weights + f32 activations + f32 outputs; prefill uses 2*M*N*K."""
    import math

    import torch

    from xn_amd import GgmlDType, QTensor
    from xn_amd.quantized import matmul_preq, matmul_t_group, matmul_t_silu_gate, quantize_lhs

    decode_only = args.only == "decode"

    def make(dt, n, k):
        w = torch.randn((n, k), generator=gen, device=dev, dtype=torch.float32) * 0.02
        q = QTensor.quantize_f32(w, (n, k), GgmlDType(dt))
        del w
        return q

    def copies_for(nbytes):
        return max(2, min(16, math.ceil(600e6 / nbytes)))

    def timed(fn, steps):
        with torch.cuda.stream(stream):
            for i in range(3):
                fn(i)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            g = capture(fn, steps, stream, args.eager)
        ms = time_graph(g, stream) / steps
        del g
        return ms

    rows = []
    steps = 50

    def matvec_row(name, dt, k, n, ms_list):
        wb = qbytes(dt, n, k)
        ws = [make(dt, n, k) for _ in range(copies_for(wb))]
        for m in ms_list:
            x = torch.randn((m, k), generator=gen, device=dev)
            y = torch.empty((m, n), device=dev)
            a = ws[0].workspace(m)
            quantize_lhs(GgmlDType(dt), x, a, m, k)
            ms_step = timed(lambda i: ws[i % len(ws)].matmul_t((m, k, n), x, y), steps)
            ms_kern = timed(lambda i: matmul_preq(ws[i % len(ws)], m, a, y), steps)
            algo = wb + m * k * 4 + m * n * 4
            rows.append({"config": name, "dtype": GgmlDType(dt).name, "k": k, "n": n, "m": m,
                         "weight_copies": len(ws), "us_step": round(ms_step * 1e3, 2),
                         "us_kernel": round(ms_kern * 1e3, 2),
                         "gbs_step": round(algo / (ms_step * 1e-3) / 1e9, 1),
                         "gbs_kernel": round(algo / (ms_kern * 1e-3) / 1e9, 1),
                         "frac_hbm_kernel": round(algo / (ms_kern * 1e-3) / 1e9 / HBM_PEAK_GBS, 3)})
            print(json.dumps(rows[-1]), file=sys.stderr, flush=True)
        del ws

    if not decode_only:
        # config 1: Q8_0 4096 -> 4096
        matvec_row("1 q8_0 matvec", 8, 4096, 4096, [1])
        # config 3: Q4_K sweep
        for k, n in [(4096, 4096), (4096, 14336), (14336, 4096), (8192, 28672)]:
            matvec_row("3 q4k sweep", 12, k, n, [1, 2, 4, 8])
        # the other decode dtypes at the FFN shapes
        matvec_row("5 q6k ffn down", 14, 14336, 4096, [1, 4])
        matvec_row("2 q4_0 gate/up", 2, 4096, 14336, [1])
        matvec_row("2 q4_0 down", 2, 14336, 4096, [1])
        # one GPU's shard of an 8-way split FFN: gate/up column-parallel
        # (4096 -> 14336/8), down row-parallel (K = 14336/8 = 7 super-blocks)
        matvec_row("e shard/8 q4k gate/up (column-parallel)", 12, 4096, 1792, [1, 16])
        matvec_row("e shard/8 q6k down (row-parallel)", 14, 1792, 4096, [1, 16])

    # config 2: Q4_0 FFN block, h = silu(x Wg^T) * (x Wu^T), y = h Wd^T
    k, f = 4096, 14336
    sets = [(make(2, f, k), make(2, f, k), make(2, k, f)) for _ in range(4)]
    x = torch.randn((1, k), generator=gen, device=dev)
    g_ = torch.empty((1, f), device=dev)
    u_ = torch.empty((1, f), device=dev)
    h_ = torch.empty((1, f), device=dev)
    y_ = torch.empty((1, k), device=dev)

    def ffn(i):
        wg, wu, wd = sets[i % len(sets)]
        wg.matmul_t((1, k, f), x, g_)
        wu.matmul_t((1, k, f), x, u_)
        torch.mul(torch.nn.functional.silu(g_), u_, out=h_)
        wd.matmul_t((1, f, k), h_, y_)

    def ffn_fused(i):
        wg, wu, wd = sets[i % len(sets)]
        matmul_t_silu_gate(wg, wu, (1, k, f), x, h_)
        wd.matmul_t((1, f, k), h_, y_)

    algo = 3 * qbytes(2, f, k) + (2 * k + 3 * f) * 4 + f * 4
    for name, fn in (("2 q4_0 ffn block (gate, up, torch SiLU-mul, down)", ffn),
                     ("2 q4_0 ffn block (fused SiLU-gated gate/up kernel, down)", ffn_fused)):
        ms = timed(fn, steps)
        rows.append({"config": name, "m": 1, "us_step": round(ms * 1e3, 2),
                     "gbs_step": round(algo / (ms * 1e-3) / 1e9, 1)})
        print(json.dumps(rows[-1]), file=sys.stderr, flush=True)
    del sets

    # config 4: prefill on int8 MFMA
    k, n = 4096, 14336
    for dt in (() if decode_only else (12, 14)):
        ws = [make(dt, n, k) for _ in range(copies_for(qbytes(dt, n, k)))]
        for m in (64, 256, 512, 2048):
            x = torch.randn((m, k), generator=gen, device=dev)
            y = torch.empty((m, n), device=dev)
            a = ws[0].workspace(m)
            quantize_lhs(GgmlDType(dt), x, a, m, k)
            ps = 10 if m >= 2048 else 20
            ms_step = timed(lambda i: ws[i % len(ws)].matmul_t((m, k, n), x, y), ps)
            ms_kern = timed(lambda i: matmul_preq(ws[i % len(ws)], m, a, y), ps)
            ops = 2.0 * m * n * k
            rows.append({"config": "4 prefill", "dtype": GgmlDType(dt).name, "k": k, "n": n, "m": m,
                         "us_step": round(ms_step * 1e3, 1), "us_kernel": round(ms_kern * 1e3, 1),
                         "tops_step": round(ops / (ms_step * 1e-3) / 1e12, 1),
                         "tops_kernel": round(ops / (ms_kern * 1e-3) / 1e12, 1),
                         "frac_int8_peak_kernel": round(ops / (ms_kern * 1e-3) / 1e12 / INT8_PEAK_TOPS, 3)})
            print(json.dumps(rows[-1]), file=sys.stderr, flush=True)
        del ws

    # config 5: every QMatMul of one decode step (random weights; attention itself is out of scope)
    from xn_amd.decode import DecoderWeights, DecodeStep

    d, kv, ff, vocab, layers = 4096, 1024, 14336, 128256, 32
    dw = DecoderWeights.random(layers, d, kv, ff, vocab, dev, generator=gen)
    mats = [(q, q.shape()[1], q.shape()[0]) for lw in dw.layers for q in lw.all()] + \
           [(dw.lm_head, d, vocab)]
    wtotal = dw.weight_bytes()
    for b in (1, 16):
        xs = {kk: torch.randn((b, kk), generator=gen, device=dev) for kk in (d, ff)}
        ys = {n: torch.empty((b, n), device=dev) for n in (d, kv, ff, vocab)}

        def step(i):
            for q, kk, n in mats:
                q.matmul_t((b, kk, n), xs[kk], ys[n])

        ms = timed(step, 3)
        rows.append({"config": "5 decode step (225 QMatMuls, one call each)", "batch": b, "weight_bytes": wtotal,
                     "us_step": round(ms * 1e3, 1), "gbs_weights": round(wtotal / (ms * 1e-3) / 1e9, 1),
                     "frac_hbm": round(wtotal / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 3)})
        print(json.dumps(rows[-1]), file=sys.stderr, flush=True)
        # the product driver: q/k/v grouped, SiLU-gated gate/up, one captured graph per step
        ds = DecodeStep(dw, b, dev)
        ds.x.normal_(generator=gen)
        ds.capture(stream)
        for _ in range(3):
            ds.replay()
        torch.cuda.synchronize()
        times = []
        for _ in range(5):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(5):
                ds.replay()
            e1.record(stream)
            e1.synchronize()
            times.append(e0.elapsed_time(e1) / 5)
        ms = float(np.median(times))
        rows.append({"config": "5 decode step (DecodeStep: q/k/v grouped, one MLP call per layer, one graph)",
                     "batch": b, "weight_bytes": wtotal,
                     "us_step": round(ms * 1e3, 1), "gbs_weights": round(wtotal / (ms * 1e-3) / 1e9, 1),
                     "frac_hbm": round(wtotal / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 3)})
        print(json.dumps(rows[-1]), file=sys.stderr, flush=True)
        del ds
    del mats, dw
    return {"metric": "per-config sweep", "rows": rows}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                          "(sharding the weights across GPUs is not built; --only sweep times one GPU's "
                          "shard of an 8-way split FFN at its real shape)"}))
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

    if args.only == "stream":
        from xn_amd.measure import stream_read

        nbytes = weight_bytes(N_DIM, K_DIM)
        ncopy = max(2, (600 << 20) // nbytes + 1)  # past the 256 MB Infinity Cache
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(i + 1) for i in range(ncopy)]
        sink = torch.zeros(1, dtype=torch.int32, device=dev)
        with torch.cuda.stream(stream):
            for i in range(args.warmup):
                stream_read(bufs[i % ncopy], sink)
            g = capture(lambda i: stream_read(bufs[i % ncopy], sink), args.steps, stream, args.eager)
        ms = time_graph(g, stream) / args.steps
        print(json.dumps({"metric": "bare HBM read GB/s of the 4096x14336 Q4_K weight bytes",
                          "bytes_per_launch": nbytes, "copies": ncopy, "us_per_read": round(ms * 1e3, 3),
                          "value": round(nbytes / (ms * 1e-3) / 1e9, 1), "unit": "GB/s",
                          "frac_of_8TBs": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}), flush=True)
        return

    if args.only in ("sweep", "decode"):
        print(json.dumps(sweep(args, dev, stream, gen)), flush=True)
        return

    # ---------------- weights: rotated copies, quantized on the device
    timed_out = {}  # what the timed graphs computed last: (copy index, lhs, output)
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
        ws = copies[0].workspace(1)

        def step(i):
            copies[i % len(copies)].matmul_t((1, K_DIM, N_DIM), x, y)

        def kernel_only(i):
            matmul_preq(copies[i % len(copies)], 1, ws, y)

        def split_step(i):
            copies[i % len(copies)].matmul_t_split((1, K_DIM, N_DIM), x, y)

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
            g_split = capture(split_step, args.steps, stream, args.eager)
        torch.cuda.synchronize()
        ms_step = time_graph(g_step, stream) / args.steps
        ms_kern = time_graph(g_kern, stream) / args.steps
        ms_split = time_graph(g_split, stream) / args.steps
        # the last replayed step's output (every variant computes the same y
        # for step i), kept for the check against the CPU oracle
        timed_out["matvec"] = ((args.steps - 1) % len(copies), x.cpu().numpy(), y.cpu().numpy())
        result["matvec_variants_us"] = {
            "matmul_t_step": round(ms_step * 1e3, 3),
            "preq_kernel": round(ms_kern * 1e3, 3),
            "quantize_then_preq_step": round(ms_split * 1e3, 3),
        }
        value = algo_bytes / (ms_step * 1e-3) / 1e9
        # the step is one kernel (the fused matvec: the row quantized in LDS
        # by each workgroup), so its average launch duration is the step's
        achieved = value
        result.update({
            "value": round(value, 1),
            "ms_per_step": round(ms_step, 5),
            "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        })
        result["roofline"] = {
            "bound": "hbm",
            "kernel": "matvec_kernel<Q4K, MB=1, fused quantize>",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
            "traffic_source": "rocprofv3 --pmc FETCH_SIZE (x2.000) + WRITE_SIZE (x1.000), "
                              "profiles/hbm_traffic_q4k_matvec_k4096_n14336_m1.md",
            "algorithmic_bytes_per_launch": algo_bytes,
            "avg_launch_us": round(ms_step * 1e3, 3),
        }
        del g_step, g_kern, g_split

    if args.only in ("all", "prefill"):
        m = args.prefill_m
        xp = torch.randn((m, K_DIM), generator=gen, device=dev, dtype=torch.float32)
        yp = torch.empty((m, N_DIM), device=dev, dtype=torch.float32)
        wsp = copies[0].workspace(m)
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
        timed_out["prefill"] = ((psteps - 1) % len(copies), xp.cpu().numpy(), yp.cpu().numpy())
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

    # ---------------- check of the timed outputs against the CPU oracle
    cpu_threads = host_threads()
    if not args.no_cpu and timed_out:
        import oracle

        oracle.cpu_pool_init(cpu_threads)  # the first call fixes the pool size
        check = {"rel_l2_max": REL_L2, "row_max_rel_max": ROW_MAX_REL}
        ok = True
        for name, (ci, lhs, got) in timed_out.items():
            rows = np.arange(lhs.shape[0]) if lhs.shape[0] <= 16 else np.linspace(0, lhs.shape[0] - 1, 16).astype(int)
            want = oracle.cpu_matmul(oracle.Q4K, lhs[rows], np.frombuffer(copies[ci].data(), dtype=np.uint8), N_DIM)
            rel, row_rel = close_stats(got[rows], want)
            ok = ok and rel <= REL_L2 and row_rel <= ROW_MAX_REL
            check[name] = {"rows_checked": len(rows), "rel_l2": float(f"{rel:.3e}"), "row_max_rel": float(f"{row_rel:.3e}")}
        check["ok"] = bool(ok)
        result["check"] = check

    # ---------------- CPU baseline: the xn-style AVX2 path on the host cores
    if not args.no_cpu and args.only in ("all", "matvec"):
        import oracle

        threads = cpu_threads
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
            "host_cpus": os.cpu_count(),
            "affinity_cpus": len(os.sched_getaffinity(0)),
            "threads_rule": "xn's pool size (utils.rs:16-27: RAYON_NUM_THREADS, else every CPU the process may "
                            f"use) capped at the GPU box's CPU share of {GPU_BOX_CPU_SHARE} per GPU",
            "kind": "port",
            "value_excl_quantize": round(algo_bytes / med_k / 1e9, 2),
            "sample": f"{len(times)} calls of Q4_K 4096->14336 M=1 (quantize_lhs + AVX2 vec_dot_q4k_q8k over "
                      f"128-column tasks), {ncopies} rotated weight copies, median {med * 1e3:.3f} ms; "
                      f"value_excl_quantize: {len(times_k)} calls on pre-quantized lhs, median {med_k * 1e3:.3f} ms",
        }

    print(json.dumps(result), flush=True)
    if not result.get("check", {}).get("ok", True):
        print("bench: the timed outputs differ from the CPU oracle beyond the tolerance", file=sys.stderr, flush=True)
        sys.exit(1)


if __name__ == "__main__":
    main()
