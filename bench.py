"""Benchmark: int4 MatMulNBits on Qwen3-0.6B projection shapes.

One step = one pass of the q, k, v, o, gate, up, down and lm_head
MatMulNBits projections (block_size 128, packed uint4 zero points) at M = 512
tokens (prefill).  `value` is the whole pass's algorithmic TFLOP/s
(2*M*N*K per projection) with weights and activations resident in HBM.  The
same run times the M = 1 decode pass over the same weights (algorithmic HBM
GB/s), the dominant kernels' roofline fractions, and the CPU oracle (the
reference's algorithm restated in C, one thread, as the reference never pools
MatMulNBits) on a bounded sample.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2500.0

# (name, K, N) — Qwen3-0.6B: hidden 1024, 16 q heads x 128, 8 kv heads x 128,
# intermediate 3072, vocab 151936.
QWEN3_PROJ = [("q", 1024, 2048), ("k", 1024, 1024), ("v", 1024, 1024), ("o", 2048, 1024),
              ("gate", 1024, 3072), ("up", 1024, 3072), ("down", 3072, 1024),
              ("lm_head", 1024, 151936)]
BLOCK = 128
M_PREFILL = 512


def nbits_bytes(m, k, n, bs=BLOCK, a_bytes=4):
    """Algorithmic bytes of one MatMulNBits call: A, packed W, scales, packed
    zero points, Y (each tensor once)."""
    nb = (k + bs - 1) // bs
    return m * k * a_bytes + n * nb * bs // 2 + n * nb * 4 + n * ((nb + 1) // 2) + m * n * 4


def make_weight(rng, k, n, bs=BLOCK):
    nb = (k + bs - 1) // bs
    b = rng.integers(0, 256, (n, nb, bs // 2), dtype=np.uint8)
    s = rng.uniform(0.002, 0.02, (n, nb)).astype(np.float32)
    zp = rng.integers(0, 256, (n, (nb + 1) // 2), dtype=np.uint8)
    return b, s, zp


def cpu_baseline(weights, rng, budget_s=30.0):
    """Times the oracle (reference algorithm: 32-column dequantised tiles +
    4x16 f32 GEMM, one thread) at M = 512 on a bounded sample: projections in
    order, the lm_head on its first columns, until ~budget_s of CPU work."""
    import oracle

    oracle.lib()
    flops = 0.0
    t_total = 0.0
    parts = []
    for (name, k, n), (b, s, zp) in zip(QWEN3_PROJ, weights):
        cols = n if name != "lm_head" else 65536
        a = rng.standard_normal((M_PREFILL, k)).astype(np.float32)
        bb, ss, zz = b[:cols], s[:cols], zp[:cols]
        t0 = time.perf_counter()
        oracle.matmul_nbits(a, bb, ss, zz, k=k, n=cols, block_size=BLOCK)
        dt = time.perf_counter() - t0
        t_total += dt
        flops += 2.0 * M_PREFILL * cols * k
        parts.append(f"{name}[{cols}]")
        if t_total > budget_s:
            break
    return {"value": flops / t_total / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"M=512 int4 MatMulNBits bs128 zp, projections {'+'.join(parts)} "
                      f"({flops / 1e9:.1f} GFLOP in {t_total:.1f} s, 1 thread)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", choices=["lm512", "lm1", "copy"], default=None,
                    help="profiling mode: launch one workload --steps times and exit "
                         "(lm512: lm_head M=512, lm1: lm_head M=1, copy: 256 MiB device "
                         "copy used to calibrate the HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(the multi-GPU design is an N-split of weight columns, not measured here)",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from onnx_runtime_dart_amd import ops

    dev = torch.device("cuda:0")
    torch.cuda.init()
    stream = torch.cuda.Stream(device=dev)
    ctx = ops.Context(0)
    ctx.set_stream(stream.cuda_stream)

    if args.only == "copy":
        src = torch.empty(64 << 20, device=dev, dtype=torch.float32).fill_(1.0)
        dst = torch.empty_like(src)
        with torch.cuda.stream(stream):
            for _ in range(args.steps):
                dst.copy_(src)
        torch.cuda.synchronize()
        print(f"copy: {args.steps} x {src.numel() * 4} bytes read and written", flush=True)
        return
    rng = np.random.default_rng(0x5EED0003)
    t0 = time.perf_counter()
    if args.only in ("lm512", "lm1"):
        m = M_PREFILL if args.only == "lm512" else 1
        _, k, n = QWEN3_PROJ[-1]
        b, s, zp = make_weight(rng, k, n)
        w = ops.NBitsWeight(b, s, zp, k=k, n=n, block_size=BLOCK, ctx=ctx)
        a = torch.randn((m, k), device=dev, dtype=torch.float32)
        y = torch.empty((m, n), device=dev, dtype=torch.float32)
        with torch.cuda.stream(stream):
            for _ in range(args.steps):
                w.run_dev(a.data_ptr(), m, y.data_ptr())
        torch.cuda.synchronize()
        print(f"{args.only}: {args.steps} launches of lm_head M={m} K={k} N={n}", flush=True)
        w.release()
        return
    host_w = [make_weight(rng, k, n) for _, k, n in QWEN3_PROJ]
    weights = [ops.NBitsWeight(b, s, zp, k=k, n=n, block_size=BLOCK, ctx=ctx)
               for (_, k, n), (b, s, zp) in zip(QWEN3_PROJ, host_w)]
    print(f"# weights uploaded in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)

    g = torch.Generator(device=dev)
    g.manual_seed(0x5EED0003)
    acts = {}
    outs = {}
    for m in (M_PREFILL, 1):
        for _, k, n in QWEN3_PROJ:
            acts.setdefault((m, k), torch.randn((m, k), device=dev, dtype=torch.float32,
                                                generator=g))
            outs.setdefault((m, n), torch.empty((m, n), device=dev, dtype=torch.float32))

    def run_pass(m):
        for (_, k, n), w in zip(QWEN3_PROJ, weights):
            w.run_dev(acts[(m, k)].data_ptr(), m, outs[(m, n)].data_ptr())

    def timed(fn, steps, warmup):
        with torch.cuda.stream(stream):
            for _ in range(warmup):
                fn()
            torch.cuda.synchronize()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(steps):
                fn()
            e1.record(stream)
            torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    flops_step = sum(2.0 * M_PREFILL * n * k for _, k, n in QWEN3_PROJ)
    ms_step = timed(lambda: run_pass(M_PREFILL), args.steps, args.warmup)
    value = flops_step / (ms_step / 1e3) / 1e12

    bytes_m1 = sum(nbits_bytes(1, k, n) for _, k, n in QWEN3_PROJ)
    ms_m1 = timed(lambda: run_pass(1), args.steps, args.warmup)
    gbs_m1 = bytes_m1 / (ms_m1 / 1e3) / 1e9

    # Dominant kernels: lm_head at M=512 (MFMA) and at M=1 (HBM stream).
    k_lm, n_lm = QWEN3_PROJ[-1][1], QWEN3_PROJ[-1][2]
    w_lm = weights[-1]
    reps = max(args.steps, 10)
    ms_lm = timed(lambda: w_lm.run_dev(acts[(M_PREFILL, k_lm)].data_ptr(), M_PREFILL,
                                       outs[(M_PREFILL, n_lm)].data_ptr()), reps, 2)
    lm_flops = 2.0 * M_PREFILL * n_lm * k_lm
    lm_tflops = lm_flops / (ms_lm / 1e3) / 1e12
    ms_lm1 = timed(lambda: w_lm.run_dev(acts[(1, k_lm)].data_ptr(), 1,
                                        outs[(1, n_lm)].data_ptr()), reps * 5, 5)
    lm1_bytes = nbits_bytes(1, k_lm, n_lm)
    lm1_gbs = lm1_bytes / (ms_lm1 / 1e3) / 1e9

    result = {
        "metric": "int4 MatMulNBits TFLOP/s (M=512) + M=1 GEMV HBM GB/s, Qwen3-0.6B shapes",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights x fp32 activations (fp16 hi/lo MFMA, fp32 accumulate)",
        "data": "synthetic (seeded uniform nibbles, scales U(0.002,0.02), A ~ N(0,1))",
        "config": {"workload": "Qwen3-0.6B int4 MatMulNBits projections q,k,v,o,gate,up,"
                               "down,lm_head; block_size 128 with uint4 zero points",
                   "M": M_PREFILL, "block_size": BLOCK,
                   "gflop_per_step": round(flops_step / 1e9, 2)},
        "gemv_m1": {"value": round(gbs_m1, 1), "unit": "GB/s", "ms_per_pass": round(ms_m1, 4),
                    "bytes_per_pass": bytes_m1, "frac_hbm_peak": round(gbs_m1 / HBM_PEAK_GBS, 4)},
        "roofline": {"kernel": "k_gemm_f16split (lm_head 512x1024x151936, incl. activation "
                               "prepass)",
                     "bound": "mfma", "achieved": round(lm_tflops, 2),
                     "peak": FP16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(lm_tflops / FP16_MFMA_PEAK_TFLOPS, 4), "traffic": None,
                     "ms": round(ms_lm, 4)},
        "roofline_gemv": {"kernel": "k_gemv_dot8 (lm_head M=1, incl. activation prepass)",
                          "bound": "hbm", "achieved": round(lm1_gbs, 1), "peak": HBM_PEAK_GBS,
                          "unit": "GB/s", "frac": round(lm1_gbs / HBM_PEAK_GBS, 4),
                          "traffic": None, "bytes": lm1_bytes, "ms": round(ms_lm1, 4)},
    }
    if not args.no_cpu and os.environ.get("MIGEMM_BENCH_NO_CPU") != "1":
        result["cpu_baseline"] = cpu_baseline(host_w, np.random.default_rng(0x5EED0003))
    else:
        result["cpu_baseline"] = None
    for w in weights:
        w.release()
    ctx.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
