"""Benchmark of the matrix-multiply operator family on one MI355X.

Headline (`value`): int4 MatMulNBits on the Qwen3-0.6B projection shapes.  One
step = one pass of the q, k, v, o, gate, up, down and lm_head MatMulNBits
projections (block_size 128, packed uint4 zero points) at M = 512 tokens;
`value` is the pass's algorithmic TFLOP/s (2*M*N*K per projection) with
weights and activations resident in HBM.

The same run also measures, each with HIP events on the stream the library
launches on:
  roofline       the lm_head call at M = 512 (MFMA-bound), against fp16 peak
                 (the kernel issues three fp6 products per product: its
                 share of the fp6 peak is reported beside it), and the same
                 call on a weight without prefill images (the fp8 GEMM that
                 dequantises each tile);
  gemv_m1        the same eight projections at M = 1, algorithmic HBM GB/s;
                 four distinct weight sets are rotated so that the working set
                 (~370 MB) exceeds the 256 MB last-level cache and the weights
                 really stream from HBM;
  roofline_gemv  the lm_head launches at M = 1 inside those passes;
  decode_sweep   a Llama-style 1B decode step (16 layers of q/k/v/o/gate/up/
                 down + lm_head, block_size 32 with zero points, 0.79 GB of
                 distinct packed weights) at M = 1, 4 and 16;
  int8_prefill   the Qwen3 projections as MatMulInteger (u8 x i8 -> int32) at
                 M = 512, and the DynamicQuantizeLinear -> MatMulInteger ->
                 QLinearMatMul chain at M = 128, K = N = 1024;
  f32_encoder    one MiniLM-L6 encoder layer's Gemm/MatMul set (batch 32,
                 seq 128, hidden 384, 12 heads, FFN 1536) in fp32;
  cpu_baseline   the oracle (the reference's algorithms restated in C) on
                 bounded samples: the M = 512 int4 prefill on one thread (the
                 reference never pools MatMulNBits) as `value`, the M = 1
                 GEMV, and the fp32 MiniLM Gemm set on the GemmPool N-split
                 over the host's cores, with the host's CPU model.
`traffic` (HBM bytes per launch of the dominant kernels) comes from
profiles/traffic.json, written from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
runs of `bench.py --only ...` (commands and calibration in that file).

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu] [--quick]
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
FP8_MFMA_PEAK_TFLOPS = 5000.0
FP6_MFMA_PEAK_TFLOPS = 10100.0
INT8_MFMA_PEAK_TOPS = 5000.0
FP32_MFMA_PEAK_TFLOPS = 157.3

# (name, K, N) — Qwen3-0.6B: hidden 1024, 16 q heads x 128, 8 kv heads x 128,
# intermediate 3072, vocab 151936.
QWEN3_PROJ = [("q", 1024, 2048), ("k", 1024, 1024), ("v", 1024, 1024), ("o", 2048, 1024),
              ("gate", 1024, 3072), ("up", 1024, 3072), ("down", 3072, 1024),
              ("lm_head", 1024, 151936)]
# Sibling projections that read the same activations and run as one grouped
# launch (mg_matmul_nbits_group_dev), as the Dart shim issues them: q/k/v and
# gate/up.  Indices into QWEN3_PROJ.
QWEN3_GROUPS = [(0, 1, 2), (3,), (4, 5), (6,), (7,)]
BLOCK = 128
M_PREFILL = 512
GEMV_ROTATE = 4

# Llama-style 1B decoder: hidden 2048, 32 q heads and 8 kv heads of 64,
# intermediate 8192, 16 layers, vocab 128256; int4 block 32 with zero points.
LLAMA_LAYER = [("q", 2048, 2048), ("k", 2048, 512), ("v", 2048, 512), ("o", 2048, 2048),
               ("gate", 2048, 8192), ("up", 2048, 8192), ("down", 8192, 2048)]
LLAMA_LAYERS = 16
LLAMA_HEAD = ("lm_head", 2048, 128256)
LLAMA_BLOCK = 32

# MiniLM-L6 encoder layer: tokens = 32 x 128, hidden 384, 12 heads x 32, FFN 1536.
MINILM_B, MINILM_S, MINILM_H, MINILM_HEADS, MINILM_FFN = 32, 128, 384, 12, 1536


def nbits_bytes(m, k, n, bs=BLOCK, a_bytes=4):
    """Algorithmic bytes of one MatMulNBits call: A, packed W, scales, packed
    zero points, Y (each tensor once)."""
    nb = (k + bs - 1) // bs
    return m * k * a_bytes + n * nb * bs // 2 + n * nb * 4 + n * ((nb + 1) // 2) + m * n * 4


def make_weight(rng, k, n, bs=BLOCK, s_lo=0.002, s_hi=0.02):
    nb = (k + bs - 1) // bs
    b = np.frombuffer(rng.bytes(n * nb * (bs // 2)), dtype=np.uint8).reshape(n, nb, bs // 2)
    s = rng.uniform(s_lo, s_hi, (n, nb)).astype(np.float32)
    zp = np.frombuffer(rng.bytes(n * ((nb + 1) // 2)), dtype=np.uint8).reshape(n, (nb + 1) // 2)
    return b, s, zp


def host_info():
    """Host CPU model and the cores this process may use."""
    model = "unknown"
    try:
        for ln in Path("/proc/cpuinfo").read_text().splitlines():
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    return {"cpu_model": model, "cores_available": cores, "cpu_count": os.cpu_count()}


def cpu_baseline(weights, rng, budget_s=12.0):
    """The reference's CPU algorithms restated in C (the oracle), timed on
    bounded samples of the benchmark's workloads:
      int4 prefill  M = 512 MatMulNBits, 32-column dequantised tiles + the
                    4x16 f32 kernel, one thread (the reference never pools
                    MatMulNBits) -> `value`;
      int4 GEMV     M = 1 MatMulNBits, the f64 per-column decode, one thread;
      fp32 pool     the MiniLM-L6 Gemm set (config C3) on the GemmPool N-split
                    over the host's cores (lib/src/parallel_pool.dart).
    """
    import oracle

    oracle.lib()
    info = host_info()
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
    out = {"value": flops / t_total / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "port",
           "sample": f"M=512 int4 MatMulNBits bs128 zp, projections {'+'.join(parts)} "
                     f"({flops / 1e9:.1f} GFLOP in {t_total:.1f} s, 1 thread)",
           "host": info}
    # M = 1 GEMV over all eight projections (the whole lm_head).
    nbytes, t1 = 0, 0.0
    for (name, k, n), (b, s, zp) in zip(QWEN3_PROJ, weights):
        a = rng.standard_normal((1, k)).astype(np.float32)
        t0 = time.perf_counter()
        oracle.matmul_nbits(a, b, s, zp, k=k, n=n, block_size=BLOCK)
        t1 += time.perf_counter() - t0
        nbytes += nbits_bytes(1, k, n)
    out["gemv_m1"] = {"value": round(nbytes / t1 / 1e9, 3), "unit": "GB/s", "cores": 1,
                      "sample": f"M=1 int4 MatMulNBits, the eight Qwen3 projections "
                                f"({nbytes / 1e6:.1f} MB in {t1:.2f} s, 1 thread)"}
    # fp32 MiniLM Gemm set on the pool's N-split.
    workers = max(1, min(16, info["cores_available"]))
    H, F = MINILM_H, MINILM_FFN
    gemms = [("q", H, H), ("k", H, H), ("v", H, H), ("out", H, H), ("ffn1", H, F),
             ("ffn2", F, H)]
    rows = MINILM_B * MINILM_S
    fl, tp = 0.0, 0.0
    for _, k, n in gemms:
        w = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)  # prepacked B [K, N]
        x = rng.standard_normal((rows, k)).astype(np.float32)
        pool = oracle.GemmPool(w, workers)
        t0 = time.perf_counter()
        pool.matmul(x)
        tp += time.perf_counter() - t0
        pool.close()
        fl += 2.0 * rows * k * n
    out["f32_pool"] = {"value": round(fl / tp / 1e12, 5), "unit": "TFLOP/s", "cores": workers,
                       "sample": f"MiniLM-L6 layer Gemm set q/k/v/out/ffn1/ffn2 at {rows} rows "
                                 f"on the GemmPool N-split over {workers} threads "
                                 f"({fl / 1e9:.1f} GFLOP in {tp:.2f} s)"}
    return out


def load_traffic():
    p = ROOT / "profiles" / "traffic.json"
    if not p.exists():
        return {}
    return json.loads(p.read_text()).get("kernels", {})


class Timer:
    """HIP-event timing on one stream."""

    def __init__(self, torch, stream):
        self.torch, self.stream = torch, stream

    def event(self):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record(self.stream)
        return e

    def loop(self, fn, steps, warmup):
        torch = self.torch
        with torch.cuda.stream(self.stream):
            for _ in range(warmup):
                fn()
            torch.cuda.synchronize()
            e0 = self.event()
            for _ in range(steps):
                fn()
            e1 = self.event()
            torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true",
                    help="headline and lm_head measurements only")
    ap.add_argument("--only", default=None,
                    choices=["lm512", "lm1", "copy", "i8lm512", "f32ffn", "llama1", "llama16",
                             "attn", "conv", "qconv", "gqa512", "gqadec", "pass512", "dec1", "dec4",
                             "dec16"],
                    help="profiling mode: launch one workload --steps times and exit "
                         "(lm512 / lm1: Qwen3 lm_head MatMulNBits at M=512 / M=1; i8lm512: "
                         "the lm_head as MatMulInteger at M=512; f32ffn: the MiniLM FFN1 "
                         "Gemm; llama1 / llama16: the Llama lm_head at M=1 / M=16; attn: the MiniLM "
                         "fused attention; conv / qconv: the ResNet-50 3x3 conv as Conv / "
                         "QLinearConv; gqa512: the 512-token causal GroupQueryAttention "
                         "prefill; gqadec: its decode step over a 4096-token cache; pass512: the headline "
                         "M=512 pass of eight Qwen3 projections, grouped as timed; dec1 / dec4 / "
                         "dec16: the grouped Llama-style decode step at M=1 / 4 / 16; copy: 256 MiB "
                         "device copy used to calibrate the HBM byte counters)")
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
    T = Timer(torch, stream)
    g = torch.Generator(device=dev)
    g.manual_seed(0x5EED0003)

    def randn(*shape):
        return torch.randn(shape, device=dev, dtype=torch.float32, generator=g)

    if args.only:
        run_only(args, torch, ops, ctx, stream, dev, randn)
        return

    rng = np.random.default_rng(0x5EED0003)
    t0 = time.perf_counter()
    host_w = [make_weight(rng, k, n) for _, k, n in QWEN3_PROJ]
    weights = [ops.NBitsWeight(b, s, zp, k=k, n=n, block_size=BLOCK, ctx=ctx)
               for (_, k, n), (b, s, zp) in zip(QWEN3_PROJ, host_w)]
    print(f"# weights uploaded in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)

    acts, outs = {}, {}
    for m in (M_PREFILL, 1):
        for _, k, n in QWEN3_PROJ:
            if (m, k) not in acts:
                acts[(m, k)] = randn(m, k)
            if (m, n) not in outs:
                outs[(m, n)] = torch.empty((m, n), device=dev, dtype=torch.float32)

    # Grouped members write separate outputs (one per projection).
    for m in (M_PREFILL, 1):
        for name, _, n in QWEN3_PROJ:
            outs[(m, name)] = torch.empty((m, n), device=dev, dtype=torch.float32)

    def run_pass_separate(ws, m):
        for (_, k, n), w in zip(QWEN3_PROJ, ws):
            w.run_dev(acts[(m, k)].data_ptr(), m, outs[(m, n)].data_ptr())

    def run_pass(ws, m):
        for grp in QWEN3_GROUPS:
            k = QWEN3_PROJ[grp[0]][1]
            if len(grp) == 1:
                ws[grp[0]].run_dev(acts[(m, k)].data_ptr(), m,
                                   outs[(m, QWEN3_PROJ[grp[0]][0])].data_ptr())
            else:
                ops.matmul_nbits_group_dev([ws[i] for i in grp], acts[(m, k)].data_ptr(), m,
                                           [outs[(m, QWEN3_PROJ[i][0])].data_ptr() for i in grp],
                                           ctx=ctx)

    # ---- headline: M = 512 prefill pass (siblings grouped), and the same
    # eight projections launched one by one
    flops_step = sum(2.0 * M_PREFILL * n * k for _, k, n in QWEN3_PROJ)
    ms_step = T.loop(lambda: run_pass(weights, M_PREFILL), args.steps, args.warmup)
    value = flops_step / (ms_step / 1e3) / 1e12
    ms_step_sep = T.loop(lambda: run_pass_separate(weights, M_PREFILL), args.steps, args.warmup)
    print(f"# prefill pass {ms_step:.4f} ms, {value:.1f} TFLOP/s (separate launches "
          f"{ms_step_sep:.4f} ms)", file=sys.stderr, flush=True)

    # Resident weight bytes of the pass, with and without the prefill images.
    resident_img = int(sum(w.info()[2] for w in weights))
    images_bytes = int(sum(-(-n // 128) * 2 * 48 * (-(-k // 128) * 128) for _, k, n in QWEN3_PROJ))
    packed_bytes = int(sum(b.nbytes + s.nbytes + z.nbytes for b, s, z in host_w))

    # ---- dominant MFMA kernel: lm_head at M = 512
    traffic = load_traffic()
    _, k_lm, n_lm = QWEN3_PROJ[-1]
    w_lm = weights[-1]
    reps = max(args.steps, 10)
    ms_lm = T.loop(lambda: w_lm.run_dev(acts[(M_PREFILL, k_lm)].data_ptr(), M_PREFILL,
                                        outs[(M_PREFILL, n_lm)].data_ptr()), reps, 2)
    lm_tflops = 2.0 * M_PREFILL * n_lm * k_lm / (ms_lm / 1e3) / 1e12
    lm_alg_bytes = nbits_bytes(M_PREFILL, k_lm, n_lm)
    lm_ai = 2.0 * M_PREFILL * n_lm * k_lm / lm_alg_bytes
    lm_roof_tflops = min(FP6_MFMA_PEAK_TFLOPS, lm_ai * HBM_PEAK_GBS / 1e3)
    lm_gbs = lm_alg_bytes / (ms_lm / 1e3) / 1e9
    tr = traffic.get("lm512", {})
    # The same lm_head on a weight created without prefill images.
    ctx.set_prefill_images(False)
    w_lm8 = ops.NBitsWeight(*host_w[-1], k=k_lm, n=n_lm, block_size=BLOCK, ctx=ctx)
    ctx.set_prefill_images(True)
    ms_lm8 = T.loop(lambda: w_lm8.run_dev(acts[(M_PREFILL, k_lm)].data_ptr(), M_PREFILL,
                                          outs[(M_PREFILL, n_lm)].data_ptr()), reps, 2)
    w_lm8.release()
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
        "dtype": "int4 weights x fp32 activations (weights' (q - zp) / 2 as fp6 e2m3 prefill "
                 "images, activations as three e2m3 digits with per-32-k E8M0 scales, "
                 "block-scaled fp6 MFMA, fp32 accumulate)",
        "weight_format": {
            "form": "packed int4 (decode) + prefill images, 0.75 byte per weight, built on "
                    "the device at weight upload (outside the timed region)",
            "resident_bytes": resident_img,
            "resident_bytes_without_images": resident_img - images_bytes,
            "packed_onnx_bytes": packed_bytes,
            "image_bytes": images_bytes},
        "data": "synthetic (seeded uniform nibbles, scales U(0.002,0.02), A ~ N(0,1))",
        "config": {"workload": "Qwen3-0.6B int4 MatMulNBits projections q,k,v,o,gate,up,"
                               "down,lm_head; block_size 128 with uint4 zero points",
                   "M": M_PREFILL, "block_size": BLOCK,
                   "gflop_per_step": round(flops_step / 1e9, 2),
                   "launches": "q/k/v and gate/up as sibling groups (one launch each, as the "
                               "Dart shim issues them); o, down, lm_head alone"},
        "separate_launches": {"ms_per_step": round(ms_step_sep, 4),
                              "TFLOP/s": round(flops_step / (ms_step_sep / 1e3) / 1e12, 2)},
        "roofline": {"kernel": tr.get("kernel", "k_gemm_f6x3") +
                     " (lm_head 512x1024x151936; op time incl. activation prepass)",
                     # The kernel issues fp6 MFMAs (10.1 PFLOP/s dense); at its
                     # arithmetic intensity (159.3 GFLOP over 396.5 MB, 402
                     # FLOP/B) that is above min(peak, AI x 8 TB/s) = 3.21
                     # PFLOP/s, so the bound is HBM: achieved = algorithmic
                     # bytes / op time against 8 TB/s.
                     "bound": "hbm" if lm_ai * HBM_PEAK_GBS / 1e3 < FP6_MFMA_PEAK_TFLOPS
                              else "mfma",
                     "achieved": round(lm_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(lm_tflops / lm_roof_tflops, 4),
                     "arithmetic_intensity_flop_per_byte": round(lm_ai, 1),
                     "achieved_tflops": round(lm_tflops, 2),
                     "roofline_tflops": round(lm_roof_tflops, 1),
                     "frac_of_fp16_peak": round(lm_tflops / FP16_MFMA_PEAK_TFLOPS, 4),
                     "issued": "3 fp6 MFMA products per algorithmic product",
                     "mfma_issue_utilisation_fp6": round(3 * lm_tflops / FP6_MFMA_PEAK_TFLOPS,
                                                         4),
                     "without_images": {
                         "kernel": "k_gemm_f8x3 (three e4m3 digits, weight tiles dequantised "
                                   "in the GEMM)",
                         "ms": round(ms_lm8, 4),
                         "TFLOP/s": round(2.0 * M_PREFILL * n_lm * k_lm / (ms_lm8 / 1e3) / 1e12,
                                          2)},
                     "traffic": tr.get("bytes"),
                     "algorithmic_bytes": lm_alg_bytes,
                     "ms": round(ms_lm, 4)},
    }

    # ---- M = 1 decode pass over rotated weight sets
    rot = [weights]
    for r in range(1, GEMV_ROTATE):
        rng_r = np.random.default_rng(0x5EED0003 + r)
        rot.append([ops.NBitsWeight(*make_weight(rng_r, k, n), k=k, n=n, block_size=BLOCK,
                                    ctx=ctx) for _, k, n in QWEN3_PROJ])
    state = {"i": 0}

    def gemv_pass_on(ws):
        run_pass(ws, 1)

    def gemv_pass():
        gemv_pass_on(rot[state["i"] % GEMV_ROTATE])
        state["i"] += 1

    bytes_m1 = sum(nbits_bytes(1, k, n) for _, k, n in QWEN3_PROJ)
    gsteps = max(4 * args.steps, 40)
    # Host-issued passes (8 ctypes calls each; on a slow host the launch
    # rate, not the GPU, can bound this figure).
    ms_m1_eager = T.loop(gemv_pass, gsteps, 8)
    # The same passes replayed from a HIP graph (one pass per rotated weight
    # set captured once): the GPU time of the pass without host launch gaps.
    ms_m1_graph = None
    graph = None
    try:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for ws in rot:
                gemv_pass_on(ws)
        ms_m1_graph = T.loop(graph.replay, max(gsteps // GEMV_ROTATE, 10), 3) / GEMV_ROTATE
    except Exception as e:  # capture unsupported: report the host-issued figure only
        print(f"# gemv M=1 graph capture failed: {e}", file=sys.stderr, flush=True)
    ms_m1 = ms_m1_graph if ms_m1_graph is not None else ms_m1_eager
    # The eight projections launched one by one, replayed the same way.
    ms_m1_sep = None
    try:
        graph_sep = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph_sep, stream=stream):
            for ws in rot:
                run_pass_separate(ws, 1)
        ms_m1_sep = T.loop(graph_sep.replay, max(gsteps // GEMV_ROTATE, 10), 3) / GEMV_ROTATE
    except Exception as e:
        print(f"# gemv M=1 graph capture (separate) failed: {e}", file=sys.stderr, flush=True)
    # Per-projection times, each of the 8 projections launched alone between
    # its own pair of events (pre-created), averaged over the rotated sets.
    nsum = 4 * GEMV_ROTATE
    evs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            for _ in QWEN3_PROJ] for _ in range(nsum)]
    with torch.cuda.stream(stream):
        torch.cuda.synchronize()
        for it in range(nsum):
            ws = rot[it % GEMV_ROTATE]
            for j, ((_, k, n), w) in enumerate(zip(QWEN3_PROJ, ws)):
                evs[it][j][0].record(stream)
                w.run_dev(acts[(1, k)].data_ptr(), 1, outs[(1, n)].data_ptr())
                evs[it][j][1].record(stream)
        torch.cuda.synchronize()
    per_launch = [float(np.mean([evs[it][j][0].elapsed_time(evs[it][j][1])
                                 for it in range(nsum)])) for j in range(len(QWEN3_PROJ))]
    ms_lm1_pass = per_launch[-1]
    lm1_bytes = nbits_bytes(1, k_lm, n_lm)
    # Average launch duration of the lm_head GEMV alone: back-to-back launches
    # over the rotated weight sets (each launch streams its weights from HBM).
    state["j"] = 0

    def lm1_launch():
        ws = rot[state["j"] % GEMV_ROTATE]
        state["j"] += 1
        ws[-1].run_dev(acts[(1, k_lm)].data_ptr(), 1, outs[(1, n_lm)].data_ptr())

    ms_lm1 = T.loop(lm1_launch, gsteps, 8)
    lm1_gbs = lm1_bytes / (ms_lm1 / 1e3) / 1e9
    tr1 = traffic.get("lm1", {})
    result["gemv_m1"] = {"value": round(bytes_m1 / (ms_m1 / 1e3) / 1e9, 1), "unit": "GB/s",
                         "ms_per_pass": round(ms_m1, 4),
                         "timing": "HIP graph replay" if ms_m1_graph is not None
                                   else "host-issued launches",
                         "ms_per_pass_host_issued": round(ms_m1_eager, 4),
                         "launches": "q/k/v and gate/up as sibling groups, as the headline",
                         "ms_per_pass_separate_launches":
                             None if ms_m1_sep is None else round(ms_m1_sep, 4),
                         # Each projection launched alone between its own
                         # pair of events on host-issued passes: these include
                         # the event overhead (~2-4 us each), so they are not
                         # kernel times and their sum exceeds the pass.
                         "launch_event_pair_us": {name: round(t * 1e3, 2)
                                                  for (name, _, _), t in zip(QWEN3_PROJ,
                                                                             per_launch)},
                         "launch_event_pair_sum_ms": round(sum(per_launch), 4),
                         "bytes_per_pass": bytes_m1,
                         "weight_sets_rotated": GEMV_ROTATE,
                         "frac_hbm_peak": round(bytes_m1 / (ms_m1 / 1e3) / 1e9 / HBM_PEAK_GBS,
                                                4)}
    result["roofline_gemv"] = {
        "kernel": tr1.get("kernel", "k_gemv_dot8p") +
        " (lm_head M=1, 1024x151936; average of back-to-back launches over the rotated sets)",
        "bound": "hbm", "achieved": round(lm1_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(lm1_gbs / HBM_PEAK_GBS, 4), "traffic": tr1.get("bytes"),
        "algorithmic_bytes": lm1_bytes, "ms": round(ms_lm1, 4),
        "ms_in_pass_events": round(ms_lm1_pass, 4)}
    print(f"# gemv M=1 pass {ms_m1:.4f} ms (host-issued {ms_m1_eager:.4f} ms, event-pair sum "
          f"{sum(per_launch):.4f} ms); lm_head {ms_lm1 * 1e3:.2f} us {lm1_gbs:.0f} GB/s",
          file=sys.stderr, flush=True)
    graph = None
    for ws in rot[1:]:
        for w in ws:
            w.release()
    del rot

    if not args.quick:
        result["decode_sweep"] = decode_sweep(torch, ops, ctx, T, randn, dev, args, stream)
        result["int8_prefill"] = int8_prefill(torch, ops, ctx, T, dev, args)
        result["nbits_float_zp_prefill"] = nbits_float_zp(torch, ops, ctx, T, randn, dev, args)
        result["f32_encoder"] = f32_encoder(torch, ops, ctx, T, randn, dev, args)
        result["conv"] = conv_family(torch, ops, ctx, T, randn, dev, args)
        result["gqa"] = gqa_steps(torch, ops, ctx, T, randn, dev)
        result["load_path"] = load_path(ops, ctx, host_w[-1], QWEN3_PROJ[-1])

    if not args.no_cpu and not args.quick and os.environ.get("MIGEMM_BENCH_NO_CPU") != "1":
        result["cpu_baseline"] = cpu_baseline(host_w, np.random.default_rng(0x5EED0003))
    else:
        result["cpu_baseline"] = None
    for w in weights:
        w.release()
    ctx.close()
    print(json.dumps(result), flush=True)


def decode_sweep(torch, ops, ctx, T, randn, dev, args, stream):
    """Llama-style 1B decode step at M in {1, 4, 16}: 16 layers x 7 projections
    + lm_head, all distinct weights (0.79 GB packed), algorithmic HBM GB/s."""
    t0 = time.perf_counter()
    rng = np.random.default_rng(0x5EED0004)
    shapes = [s for _ in range(LLAMA_LAYERS) for s in LLAMA_LAYER] + [LLAMA_HEAD]
    ws = [ops.NBitsWeight(*make_weight(rng, k, n, LLAMA_BLOCK, 0.005, 0.02), k=k, n=n,
                          block_size=LLAMA_BLOCK, ctx=ctx) for _, k, n in shapes]
    print(f"# llama weights uploaded in {time.perf_counter() - t0:.1f} s", file=sys.stderr,
          flush=True)
    out = {"workload": "Llama-style 1B int4 decode step: 16 x (q 2048x2048, k/v 2048x512, "
                       "o 2048x2048, gate/up 2048x8192, down 8192x2048) + lm_head "
                       "2048x128256; block_size 32 with uint4 zero points",
           "grouped": "q/k/v and gate/up of each layer as one mg_matmul_nbits_group_dev "
                      "call each (the same products; 4 launches per layer instead of 7)"}
    for m in (1, 4, 16):
        a = {k: randn(m, k) for k in {k for _, k, _ in shapes}}
        y = {n: torch.empty((m, n), device=dev, dtype=torch.float32)
             for n in {n for _, _, n in shapes}}

        def step():
            for (_, k, n), w in zip(shapes, ws):
                w.run_dev(a[k].data_ptr(), m, y[n].data_ptr())

        nl = len(LLAMA_LAYER)

        def step_grouped():
            for li in range(LLAMA_LAYERS):
                lw = ws[li * nl:(li + 1) * nl]
                ops.matmul_nbits_group_dev(lw[0:3], a[2048].data_ptr(), m,
                                           [y[2048].data_ptr(), y[512].data_ptr(),
                                            y[512].data_ptr()], ctx=ctx)
                lw[3].run_dev(a[2048].data_ptr(), m, y[2048].data_ptr())
                ops.matmul_nbits_group_dev(lw[4:6], a[2048].data_ptr(), m,
                                           [y[8192].data_ptr(), y[8192].data_ptr()], ctx=ctx)
                lw[6].run_dev(a[8192].data_ptr(), m, y[2048].data_ptr())
            ws[-1].run_dev(a[LLAMA_HEAD[1]].data_ptr(), m, y[LLAMA_HEAD[2]].data_ptr())

        steps = max(args.steps // 2, 5)
        ms_g_eager = T.loop(step_grouped, steps, 2)
        ms_eager = T.loop(step, steps, 2)
        # The steps replayed from HIP graphs: GPU time without host launch gaps.
        ms, ms_g = ms_eager, ms_g_eager
        timing = "host-issued launches"
        try:
            g1, g2 = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
            with torch.cuda.graph(g1, stream=stream):
                step()
            with torch.cuda.graph(g2, stream=stream):
                step_grouped()
            ms = T.loop(g1.replay, steps, 2)
            ms_g = T.loop(g2.replay, steps, 2)
            timing = "HIP graph replay"
            del g1, g2
        except Exception as e:
            print(f"# decode M={m} graph capture failed: {e}", file=sys.stderr, flush=True)
        ms_head = T.loop(lambda: ws[-1].run_dev(a[LLAMA_HEAD[1]].data_ptr(), m,
                                                y[LLAMA_HEAD[2]].data_ptr()), steps, 2)
        nbytes = sum(nbits_bytes(m, k, n, LLAMA_BLOCK) for _, k, n in shapes)
        hb = nbits_bytes(m, LLAMA_HEAD[1], LLAMA_HEAD[2], LLAMA_BLOCK)
        out[f"M{m}"] = {"ms_per_step": round(ms, 4), "bytes_per_step": nbytes,
                        "GB/s": round(nbytes / (ms / 1e3) / 1e9, 1),
                        "frac_hbm_peak": round(nbytes / (ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
                        "grouped_ms_per_step": round(ms_g, 4),
                        "grouped_GB/s": round(nbytes / (ms_g / 1e3) / 1e9, 1),
                        "timing": timing,
                        "host_issued_ms_per_step": round(ms_eager, 4),
                        "host_issued_grouped_ms_per_step": round(ms_g_eager, 4),
                        "lm_head_us": round(ms_head * 1e3, 2),
                        "lm_head_GB/s": round(hb / (ms_head / 1e3) / 1e9, 1)}
        print(f"# decode M={m}: {out[f'M{m}']}", file=sys.stderr, flush=True)
    out["layer_with_producers"] = decode_layers_with_producers(torch, ops, ctx, T, randn, dev,
                                                               args, stream, ws, shapes)
    for w in ws:
        w.release()
    return out


def decode_layers_with_producers(torch, ops, ctx, T, randn, dev, args, stream, ws, shapes):
    """The decode step with the ops that produce each projection's input, as a
    layer runs them (lib/src/onnx_graph.dart:1227-1309; attention itself is
    left out: its output is a synthetic buffer): per layer SkipSimplified-
    LayerNormalization -> q/k/v, o on the attention output, the residual add
    fused into the next SkipSimplifiedLayerNormalization -> gate/up, SiLU
    gating (Sigmoid, Mul, Mul) -> down.  Timed twice: every GEMV converting
    its fp32 input in a prepass launch, and the two norms also writing the
    split activations their GEMVs read (no prepass launch for q/k/v and
    gate/up: 12 launches per layer instead of 14)."""
    H, I = LLAMA_LAYER[0][1], LLAMA_LAYER[4][2]
    nl = len(LLAMA_LAYER)
    rng = np.random.default_rng(0x5EED0005)
    gam = [torch.from_numpy(rng.uniform(0.5, 1.5, H).astype(np.float32)).to(dev)
           for _ in range(2 * LLAMA_LAYERS)]
    res = {}
    for m in (4, 16):
        x, resid, att = randn(m, H), randn(m, H), randn(m, H)
        h, ssum, q, o = (torch.empty((m, H), device=dev) for _ in range(4))
        kk = torch.empty((m, LLAMA_LAYER[1][2]), device=dev)
        vv = torch.empty((m, LLAMA_LAYER[2][2]), device=dev)
        g, u, sg, act = (torch.empty((m, I), device=dev) for _ in range(4))
        dn = torch.empty((m, H), device=dev)
        sp_h = torch.empty(ops.nbits_split_bytes(H, LLAMA_BLOCK), device=dev, dtype=torch.uint8)
        P = lambda t: t.data_ptr()  # noqa: E731

        def step(split):
            xin, rin = x, resid
            for li in range(LLAMA_LAYERS):
                lw = ws[li * nl:(li + 1) * nl]
                if split:
                    ops.skip_rms_norm_f32_split_dev(P(xin), P(rin), (m, H), P(gam[2 * li]), H, None,
                                                    1e-5, P(h), P(ssum), LLAMA_BLOCK, P(sp_h),
                                                    ctx=ctx)
                    ops.matmul_nbits_group_split_dev(lw[0:3], P(h), P(sp_h), m,
                                                     [P(q), P(kk), P(vv)], ctx=ctx)
                else:
                    ops.skip_rms_norm_f32_dev(P(xin), P(rin), (m, H), P(gam[2 * li]), H, None,
                                              1e-5, P(h), P(ssum), ctx=ctx)
                    ops.matmul_nbits_group_dev(lw[0:3], P(h), m, [P(q), P(kk), P(vv)], ctx=ctx)
                lw[3].run_dev(P(att), m, P(o))
                if split:
                    ops.skip_rms_norm_f32_split_dev(P(o), P(ssum), (m, H), P(gam[2 * li + 1]), H,
                                                    None, 1e-5, P(h), P(ssum), LLAMA_BLOCK,
                                                    P(sp_h), ctx=ctx)
                    ops.matmul_nbits_group_split_dev(lw[4:6], P(h), P(sp_h), m, [P(g), P(u)],
                                                     ctx=ctx)
                else:
                    ops.skip_rms_norm_f32_dev(P(o), P(ssum), (m, H), P(gam[2 * li + 1]), H, None,
                                              1e-5, P(h), P(ssum), ctx=ctx)
                    ops.matmul_nbits_group_dev(lw[4:6], P(h), m, [P(g), P(u)], ctx=ctx)
                ops.sigmoid_f32_dev(P(g), m * I, P(sg), ctx=ctx)
                ops.binary_f32_dev("mul", P(g), (m, I), P(sg), (m, I), P(sg), ctx=ctx)
                ops.binary_f32_dev("mul", P(sg), (m, I), P(u), (m, I), P(act), ctx=ctx)
                lw[6].run_dev(P(act), m, P(dn))
                xin, rin = dn, ssum
            ws[-1].run_dev(P(dn), m, P(y_head))

        y_head = torch.empty((m, LLAMA_HEAD[2]), device=dev)
        steps = max(args.steps // 2, 5)
        r = {}
        for tag, split in (("prepass", False), ("split", True)):
            ms = T.loop(lambda: step(split), steps, 2)
            timing = "host-issued launches"
            try:
                gr = torch.cuda.CUDAGraph()
                with torch.cuda.graph(gr, stream=stream):
                    step(split)
                ms = T.loop(gr.replay, steps, 2)
                timing = "HIP graph replay"
                del gr
            except Exception as e:
                print(f"# decode layer M={m} graph capture failed: {e}", file=sys.stderr,
                      flush=True)
            r[f"{tag}_ms_per_step"] = round(ms, 4)
            r["timing"] = timing
        r["launches_per_layer"] = {"prepass": 14, "split": 12}
        res[f"M{m}"] = r
        print(f"# decode layers with producers M={m}: {r}", file=sys.stderr, flush=True)
    res["workload"] = ("16 Llama-style layers (SkipSimplifiedLayerNormalization, q/k/v, o, "
                       "SkipSimplifiedLayerNormalization, gate/up, Sigmoid, Mul, Mul, down) + "
                       "lm_head; attention output synthetic")
    return res


def nbits_float_zp(torch, ops, ctx, T, randn, dev, args):
    """MatMulNBits with float zero points (the form some exporters write) at
    M = 512 on the Qwen3 gate and lm_head shapes: the fp6 GEMM on the prefill
    images (q / 2), the zero point taken out as z times the activations' row
    sums."""
    rng = np.random.default_rng(0x5EED0004)
    out = {}
    for name, k, n in (("gate", 1024, 3072), ("lm_head", 1024, 151936)):
        nb = k // BLOCK
        b = np.frombuffer(rng.bytes(n * nb * BLOCK // 2), np.uint8).reshape(n, nb, BLOCK // 2)
        s = rng.uniform(0.002, 0.02, (n, nb)).astype(np.float32)
        zp = (rng.standard_normal((n, nb)) + 8).astype(np.float32)
        w = ops.NBitsWeight(b, s, zp, k=k, n=n, block_size=BLOCK, ctx=ctx)
        a = randn(M_PREFILL, k)
        y = torch.empty((M_PREFILL, n), device=dev, dtype=torch.float32)
        ms = T.loop(lambda: w.run_dev(a.data_ptr(), M_PREFILL, y.data_ptr()),
                    max(args.steps // 2, 5), 2)
        out[name] = {"shape": [M_PREFILL, k, n], "ms": round(ms, 4),
                     "TFLOP/s": round(2.0 * M_PREFILL * k * n / (ms / 1e3) / 1e12, 2)}
        w.release()
    return out


def int8_prefill(torch, ops, ctx, T, dev, args):
    """Qwen3 projections as MatMulInteger (u8 activations x i8 weights, zero
    points 128 / 0) at M = 512, and the DQL -> MatMulInteger -> QLinearMatMul
    chain at M = 128, K = N = 1024."""
    rng = np.random.default_rng(0x5EED0002)
    ws = []
    for _, k, n in QWEN3_PROJ:
        b = np.frombuffer(rng.bytes(k * n), dtype=np.int8).reshape(k, n).copy()
        b[b == -128] = -127
        ws.append(ops.Int8Weight(b, np.zeros(1, np.int32), ctx=ctx))
    a = {k: torch.randint(0, 256, (M_PREFILL, k), device=dev, dtype=torch.uint8)
         for k in {k for _, k, _ in QWEN3_PROJ}}
    y = {n: torch.empty((M_PREFILL, n), device=dev, dtype=torch.int32)
         for n in {n for _, _, n in QWEN3_PROJ}}

    def run():
        for (_, k, n), w in zip(QWEN3_PROJ, ws):
            w.matmul_integer_dev(a[k].data_ptr(), False, M_PREFILL, y[n].data_ptr(),
                                 np.array([128], np.int32))

    ops_step = sum(2.0 * M_PREFILL * n * k for _, k, n in QWEN3_PROJ)
    ms = T.loop(run, max(args.steps // 2, 5), 2)
    _, k_lm, n_lm = QWEN3_PROJ[-1]
    ms_lm = T.loop(lambda: ws[-1].matmul_integer_dev(a[k_lm].data_ptr(), False, M_PREFILL,
                                                     y[n_lm].data_ptr(),
                                                     np.array([128], np.int32)), 10, 2)
    lm_tops = 2.0 * M_PREFILL * n_lm * k_lm / (ms_lm / 1e3) / 1e12
    # The lm_head shape is below the int8 ridge: its roofline is
    # min(peak, arithmetic intensity x HBM bandwidth) (A u8, B i8, Y int32).
    lm_bytes = M_PREFILL * k_lm + k_lm * n_lm + M_PREFILL * n_lm * 4
    ai = 2.0 * M_PREFILL * n_lm * k_lm / lm_bytes
    roof = min(INT8_MFMA_PEAK_TOPS, ai * HBM_PEAK_GBS / 1e3)
    out = {"workload": "Qwen3-0.6B projections as MatMulInteger u8 x i8 -> int32, M=512",
           "TOP/s": round(ops_step / (ms / 1e3) / 1e12, 1), "ms_per_pass": round(ms, 4),
           "lm_head": {"TOP/s": round(lm_tops, 1), "ms": round(ms_lm, 4),
                       "arithmetic_intensity_op_per_byte": round(ai, 1),
                       "roofline_TOP/s": round(roof, 1),
                       "bound": "hbm" if roof < INT8_MFMA_PEAK_TOPS else "mfma",
                       "frac_roofline": round(lm_tops / roof, 4),
                       "frac_int8_peak": round(lm_tops / INT8_MFMA_PEAK_TOPS, 4)}}
    for w in ws:
        w.release()
    # C2 chain: x f32 [128, 1024] -> DQL -> MatMulInteger (int32) and QLinearMatMul (u8).
    m, k, n = 128, 1024, 1024
    b = np.clip(rng.integers(-127, 128, (k, n)), -127, 127).astype(np.int8)
    w = ops.Int8Weight(b, np.zeros(1, np.int32), ctx=ctx)
    x = torch.randn((m, k), device=dev, dtype=torch.float32)
    xq = torch.empty((m, k), device=dev, dtype=torch.uint8)
    sz = torch.zeros(4, device=dev, dtype=torch.int32)  # scale, zp, non-finite flag
    y32 = torch.empty((m, n), device=dev, dtype=torch.int32)
    y8 = torch.empty((m, n), device=dev, dtype=torch.uint8)

    def chain():
        ops.dynamic_quantize_linear_dev(x.data_ptr(), m * k, xq.data_ptr(), sz.data_ptr(),
                                        ctx=ctx)
        w.matmul_integer_dq_dev(xq.data_ptr(), m, sz.data_ptr(), y32.data_ptr())
        w.qlinear_matmul_dq_dev(xq.data_ptr(), m, sz.data_ptr(), 2.0 ** -10, 0.05, 128,
                                y8.data_ptr(), lo=0, hi=255)

    ms_c = T.loop(chain, max(args.steps, 10), 3)
    out["dql_chain_M128_K1024_N1024"] = {
        "us_per_chain": round(ms_c * 1e3, 2),
        "ops": "DQL + MatMulInteger + QLinearMatMul, scale/zp read on the device"}
    w.release()
    print(f"# int8: {out}", file=sys.stderr, flush=True)
    return out


def f32_encoder(torch, ops, ctx, T, randn, dev, args):
    """One MiniLM-L6 encoder layer's matmuls in fp32: q/k/v/out Gemm (transB,
    bias) [4096,384]x[384,384]^T, FFN1 [4096,384]x[1536,384]^T, FFN2
    [4096,1536]x[384,1536]^T, and the attention as the graph runs it after its
    _FusedSDPA rewrite: softmax([384 x 128x32]x[32x128] * 1/sqrt(32) + padding
    mask [32,1,1,128]) x [128x32] in one fused launch.  The two attention
    MatMuls alone (no softmax) are timed beside it."""
    rng = np.random.default_rng(0x5EED0001)
    tok = MINILM_B * MINILM_S
    H, F = MINILM_H, MINILM_FFN
    gemms = [("q", H, H), ("k", H, H), ("v", H, H), ("out", H, H), ("ffn1", H, F),
             ("ffn2", F, H)]
    ws, bias = [], []
    for _, k, n in gemms:
        wt = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        ws.append(ops.F32Weight(wt, trans_b=True, ctx=ctx))
        bias.append(torch.from_numpy((rng.standard_normal(n) * 0.02).astype(np.float32)).to(dev))
    x = {k: randn(tok, k) for k in (H, F)}
    y = {n: torch.empty((tok, n), device=dev, dtype=torch.float32) for n in (H, F)}
    bh = MINILM_B * MINILM_HEADS
    dh = H // MINILM_HEADS
    q = randn(MINILM_B, MINILM_HEADS, MINILM_S, dh)
    kt = randn(MINILM_B, MINILM_HEADS, dh, MINILM_S)
    p = randn(MINILM_B, MINILM_HEADS, MINILM_S, MINILM_S)
    v = randn(MINILM_B, MINILM_HEADS, MINILM_S, dh)
    sc = torch.empty((MINILM_B, MINILM_HEADS, MINILM_S, MINILM_S), device=dev)
    ctxo = torch.empty((MINILM_B, MINILM_HEADS, MINILM_S, dh), device=dev)
    # BERT extended attention mask: 0 for tokens, -10000 for padding (the last
    # 16 positions of every other sequence).
    mask = torch.zeros((MINILM_B, 1, 1, MINILM_S), device=dev)
    mask[1::2, :, :, -16:] = -10000.0
    scale = 1.0 / float(np.sqrt(dh))

    def attention():
        ops.fused_sdpa_dev(q.data_ptr(), q.shape, kt.data_ptr(), kt.shape, v.data_ptr(),
                           v.shape, mask.data_ptr(), mask.shape, scale, ctxo.data_ptr(), ctx=ctx)

    def attention_unfused_matmuls():
        ops.matmul_f32_dev(q.data_ptr(), q.shape, kt.data_ptr(), kt.shape, sc.data_ptr(),
                           ctx=ctx)
        ops.matmul_f32_dev(p.data_ptr(), p.shape, v.data_ptr(), v.shape, ctxo.data_ptr(),
                           ctx=ctx)

    def run():
        for (_, k, n), w, bb in zip(gemms, ws, bias):
            w.gemm_dev(x[k].data_ptr(), tok, y[n].data_ptr(), bb.data_ptr(), [n])
        attention()

    attn_flops = 2 * (2.0 * bh * MINILM_S * MINILM_S * dh)
    flops = sum(2.0 * tok * k * n for _, k, n in gemms) + attn_flops
    ms = T.loop(run, max(args.steps // 2, 5), 2)
    attn_ms = T.loop(attention, 20, 3)
    unfused_ms = T.loop(attention_unfused_matmuls, 10, 2)
    attn_bytes = 4 * (3 * bh * MINILM_S * dh + MINILM_B * MINILM_S + bh * MINILM_S * dh)
    ffn_ms = T.loop(lambda: ws[4].gemm_dev(x[H].data_ptr(), tok, y[F].data_ptr(),
                                           bias[4].data_ptr(), [F]), 10, 2)
    ffn_tf = 2.0 * tok * H * F / (ffn_ms / 1e3) / 1e12
    out = {"workload": "MiniLM-L6 layer matmuls fp32 (batch 32, seq 128, hidden 384, "
                       "12x32 heads, FFN 1536)",
           "TFLOP/s": round(flops / (ms / 1e3) / 1e12, 2), "ms_per_layer": round(ms, 4),
           "gflop_per_layer": round(flops / 1e9, 2),
           "ffn1": {"TFLOP/s": round(ffn_tf, 2),
                    "frac_fp32_mfma_peak": round(ffn_tf / FP32_MFMA_PEAK_TFLOPS, 4),
                    "ms": round(ffn_ms, 4)},
           "attention_fused": {
               "kernel": "k_attn (_FusedSDPA, 384 heads x 128x128, head 32, padding mask)",
               "us": round(attn_ms * 1e3, 2),
               "TFLOP/s": round(attn_flops / (attn_ms / 1e3) / 1e12, 2),
               "frac_fp32_mfma_peak": round(attn_flops / (attn_ms / 1e3) / 1e12 /
                                            FP32_MFMA_PEAK_TFLOPS, 4),
               "GB/s": round(attn_bytes / (attn_ms / 1e3) / 1e9, 1),
               "unfused_two_matmuls_us": round(unfused_ms * 1e3, 2)}}
    for w in ws:
        w.release()
    print(f"# f32: {out}", file=sys.stderr, flush=True)
    return out


# Convolution workloads (no BASELINE config names one; these are common CNN
# shapes): ResNet-50 stage-3 3x3 conv, the ResNet stem, a stride-2 4x4
# ConvTranspose upsampler (VAE decoder) and the stage-3 conv as QLinearConv.
RESNET_3X3 = ((32, 256, 14, 14), (256, 256, 3, 3), dict(pads=[1, 1, 1, 1]))
RESNET_STEM = ((32, 3, 224, 224), (64, 3, 7, 7), dict(strides=[2, 2], pads=[3, 3, 3, 3]))
VAE_UP = ((8, 128, 32, 32), (128, 64, 4, 4), dict(strides=[2, 2], pads=[1, 1, 1, 1]))


def conv_flops(xs, ws, ys):
    """2 * N * M * out_positions * (C / group) * taps (taps in the padding
    count, as a GEMM over im2col would)."""
    return 2.0 * ys[0] * ys[1] * float(np.prod(ys[2:])) * ws[1] * float(np.prod(ws[2:]))


def conv_family(torch, ops, ctx, T, randn, dev, args):
    rng = np.random.default_rng(0x5EED0004)
    out = {}

    def f32_case(name, spec, transposed=False):
        xs, ws, at = spec
        x = randn(*xs)
        w = torch.from_numpy((rng.standard_normal(ws) * 0.05).astype(np.float32)).to(dev)
        if transposed:
            ys = ops.conv_transpose_output_shape(xs, ws, **at)
            flops = 2.0 * xs[0] * xs[1] * ws[1] * float(np.prod(xs[2:])) * float(np.prod(ws[2:]))
        else:
            ys = ops.conv_output_shape(xs, ws, **at)
            flops = conv_flops(xs, ws, ys)
        b = torch.zeros(ys[1], device=dev)
        y = torch.empty(ys, device=dev, dtype=torch.float32)
        fn = ops.conv_transpose_f32_dev if transposed else ops.conv_f32_dev
        ms = T.loop(lambda: fn(x.data_ptr(), xs, w.data_ptr(), ws, y.data_ptr(), b.data_ptr(),
                               ctx=ctx, **at), 20, 3)
        tf = flops / (ms / 1e3) / 1e12
        out[name] = {"x": list(xs), "w": list(ws), **{k: v for k, v in at.items()},
                     "us": round(ms * 1e3, 2), "TFLOP/s": round(tf, 2),
                     "frac_fp32_mfma_peak": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)}

    f32_case("resnet50_3x3_256", RESNET_3X3)
    f32_case("resnet50_stem_7x7", RESNET_STEM)
    f32_case("conv_transpose_4x4_s2", VAE_UP, transposed=True)
    out["conv_transpose_4x4_s2"]["note"] = ("FLOPs count the useful taps (4 of 16 per output); "
                                            "the four sub-pixel phases issue only those")

    xs, ws, at = RESNET_3X3
    x = torch.randint(0, 256, xs, device=dev, dtype=torch.uint8)
    w = torch.randint(-128, 128, ws, device=dev, dtype=torch.int8)
    ys = ops.conv_output_shape(xs, ws, **at)
    y = torch.empty(ys, device=dev, dtype=torch.uint8)
    wsc = rng.uniform(0.002, 0.02, ws[0]).astype(np.float32)
    wz = np.zeros(ws[0], np.int8)
    ms = T.loop(lambda: ops.qlinear_conv_dev(x.data_ptr(), False, xs, 0.05, 128, w.data_ptr(),
                                             True, ws, wsc, wz, 4.0, 128, y.data_ptr(),
                                             lo=0, hi=255, ctx=ctx, **at), 20, 3)
    tf = conv_flops(xs, ws, ys) / (ms / 1e3) / 1e12
    out["qlinear_conv_resnet50_3x3_256"] = {
        "us": round(ms * 1e3, 2), "TOP/s": round(tf, 2),
        "note": "int8 MFMA GEMM over a byte im2col (exact int32 sums); includes the per-call "
                "filter prepack and the upload of the per-channel requant table"}
    print(f"# conv: {out}", file=sys.stderr, flush=True)
    return out


def gqa_steps(torch, ops, ctx, T, randn, dev):
    """GroupQueryAttention at Llama-3.2-1B geometry (32 query heads, 8 KV heads
    of 64, RoPE): one decode step over a 1024- and a 4096-token cache (KV
    append, attention over the cache; algorithmic bytes = the cache read
    twice plus written once, the op's present-KV contract) and a 512-token
    causal prefill."""
    out = {}
    h, kv, hs = 32, 8, 64
    for name, b, s, past in (("decode_past1024", 1, 1, 1024), ("decode_past4096", 1, 1, 4096),
                             ("prefill_512", 1, 512, 0)):
        q, k, v = randn(b, s, h * hs), randn(b, s, kv * hs), randn(b, s, kv * hs)
        pk, pv = randn(b, kv, max(past, 1), hs), randn(b, kv, max(past, 1), hs)
        cos, sin = randn(past + s, hs // 2), randn(past + s, hs // 2)
        y = torch.empty_like(q)
        prk = torch.empty((b, kv, past + s, hs), device=dev)
        prv = torch.empty_like(prk)

        def step():
            ops.group_query_attention_dev(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), b, s, h * hs, h, kv, y.data_ptr(),
                prk.data_ptr(), prv.data_ptr(), past_key_ptr=pk.data_ptr() if past else 0,
                past_value_ptr=pv.data_ptr() if past else 0, past_len=past,
                cos_ptr=cos.data_ptr(), sin_ptr=sin.data_ptr(), max_pos=past + s,
                half_rot=hs // 2, do_rotary=True, ctx=ctx)

        ms = T.loop(step, 20, 3)
        kv_bytes = 2 * b * kv * (past + s) * hs * 4
        out[name] = {"us": round(ms * 1e3, 2),
                     "cache_GB/s": round(3 * kv_bytes / (ms / 1e3) / 1e9, 1)}
        if s > 1:
            flops = 4.0 * b * h * hs * s * (s + 1) / 2
            out[name]["TFLOP/s"] = round(flops / (ms / 1e3) / 1e12, 2)
    print(f"# gqa: {out}", file=sys.stderr, flush=True)
    return out


def load_path(ops, ctx, hw, proj):
    """Upload time of the Qwen lm_head's int4 tensors (B, scales, zero points)
    through the streamed path: from host arrays, and from a file (the ONNX
    external-data case; the file is written first, so it is read from the page
    cache).  GB/s counts the raw ONNX bytes."""
    import tempfile
    b, sc, zp = hw
    _, k, n = proj
    raw = b.nbytes + sc.nbytes + zp.nbytes
    out = {"workload": f"Qwen3 lm_head MatMulNBits {k}x{n} bs {BLOCK} uint4 zp, "
                       f"{raw / 1e6:.1f} MB raw"}
    srcs = [ops.TensorSource.from_array(np.ascontiguousarray(t)) for t in (b, sc, zp)]

    def timed(sources, chunk=0):
        best = None
        for _ in range(3):
            t0 = time.perf_counter()
            w = ops.NBitsWeight.streamed(*sources, zp_kind=ops.MG_ZP_UINT4, k=k, n=n,
                                         block_size=BLOCK, chunk_bytes=chunk, ctx=ctx)
            dt = time.perf_counter() - t0
            w.release()
            best = dt if best is None else min(best, dt)
        return best

    t_host = timed(srcs)
    with tempfile.TemporaryDirectory() as d:
        path = Path(d) / "lm_head.bin"
        with open(path, "wb") as f:
            for t in (b, sc, zp):
                f.write(np.ascontiguousarray(t).tobytes())
        offs = np.cumsum([0, b.nbytes, sc.nbytes])
        fsrc = [ops.TensorSource.from_file(path, int(o)) for o in offs]
        t_file = timed(fsrc)
    out["host_arrays"] = {"ms": round(t_host * 1e3, 2), "GB/s": round(raw / t_host / 1e9, 2)}
    out["file_page_cache"] = {"ms": round(t_file * 1e3, 2), "GB/s": round(raw / t_file / 1e9, 2)}
    print(f"# load path: {out}", file=sys.stderr, flush=True)
    return out


def run_only(args, torch, ops, ctx, stream, dev, randn):
    """Profiling mode: one workload launched --steps times on the library's
    stream."""
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
    with torch.cuda.stream(stream):
        if args.only in ("lm512", "lm1", "llama1", "llama16"):
            if args.only.startswith("llama"):
                m, (_, k, n), bs = int(args.only[5:]), LLAMA_HEAD, LLAMA_BLOCK
            else:
                m, (_, k, n), bs = (M_PREFILL if args.only == "lm512" else 1), QWEN3_PROJ[-1], BLOCK
            w = ops.NBitsWeight(*make_weight(rng, k, n, bs), k=k, n=n, block_size=bs, ctx=ctx)
            a = randn(m, k)
            y = torch.empty((m, n), device=dev, dtype=torch.float32)
            for _ in range(args.steps):
                w.run_dev(a.data_ptr(), m, y.data_ptr())
        elif args.only == "pass512":
            ws = [ops.NBitsWeight(*make_weight(rng, k, n), k=k, n=n, block_size=BLOCK, ctx=ctx)
                  for _, k, n in QWEN3_PROJ]
            acts = {k: randn(M_PREFILL, k) for _, k, _ in QWEN3_PROJ}
            outs = [torch.empty((M_PREFILL, n), device=dev, dtype=torch.float32)
                    for _, _, n in QWEN3_PROJ]
            for _ in range(args.steps):
                for grp in QWEN3_GROUPS:
                    k = QWEN3_PROJ[grp[0]][1]
                    ops.matmul_nbits_group_dev([ws[i] for i in grp], acts[k].data_ptr(),
                                               M_PREFILL, [outs[i].data_ptr() for i in grp],
                                               ctx=ctx)
            torch.cuda.synchronize()
            for x in ws:
                x.release()
            w = None
        elif args.only in ("dec1", "dec4", "dec16"):
            m = int(args.only[3:])
            shapes = [x for _ in range(LLAMA_LAYERS) for x in LLAMA_LAYER] + [LLAMA_HEAD]
            ws = [ops.NBitsWeight(*make_weight(rng, k, n, LLAMA_BLOCK, 0.005, 0.02), k=k, n=n,
                                  block_size=LLAMA_BLOCK, ctx=ctx) for _, k, n in shapes]
            a = {k: randn(m, k) for k in {k for _, k, _ in shapes}}
            y = {n: torch.empty((m, n), device=dev, dtype=torch.float32)
                 for n in {n for _, _, n in shapes}}
            nl = len(LLAMA_LAYER)
            for _ in range(args.steps):
                for li in range(LLAMA_LAYERS):
                    lw = ws[li * nl:(li + 1) * nl]
                    ops.matmul_nbits_group_dev(lw[0:3], a[2048].data_ptr(), m,
                                               [y[2048].data_ptr(), y[512].data_ptr(),
                                                y[512].data_ptr()], ctx=ctx)
                    lw[3].run_dev(a[2048].data_ptr(), m, y[2048].data_ptr())
                    ops.matmul_nbits_group_dev(lw[4:6], a[2048].data_ptr(), m,
                                               [y[8192].data_ptr(), y[8192].data_ptr()],
                                               ctx=ctx)
                    lw[6].run_dev(a[8192].data_ptr(), m, y[2048].data_ptr())
                ws[-1].run_dev(a[LLAMA_HEAD[1]].data_ptr(), m, y[LLAMA_HEAD[2]].data_ptr())
            torch.cuda.synchronize()
            for x in ws:
                x.release()
            w = None
        elif args.only == "i8lm512":
            m, (_, k, n) = M_PREFILL, QWEN3_PROJ[-1]
            b = np.frombuffer(rng.bytes(k * n), dtype=np.int8).reshape(k, n)
            w = ops.Int8Weight(b, np.zeros(1, np.int32), ctx=ctx)
            a = torch.randint(0, 256, (m, k), device=dev, dtype=torch.uint8)
            y = torch.empty((m, n), device=dev, dtype=torch.int32)
            for _ in range(args.steps):
                w.matmul_integer_dev(a.data_ptr(), False, m, y.data_ptr(),
                                     np.array([128], np.int32))
        elif args.only == "f32ffn":
            tok, k, n = MINILM_B * MINILM_S, MINILM_H, MINILM_FFN
            w = ops.F32Weight((rng.standard_normal((n, k)) * 0.02).astype(np.float32),
                              trans_b=True, ctx=ctx)
            bias = torch.zeros(n, device=dev)
            a = randn(tok, k)
            y = torch.empty((tok, n), device=dev, dtype=torch.float32)
            for _ in range(args.steps):
                w.gemm_dev(a.data_ptr(), tok, y.data_ptr(), bias.data_ptr(), [n])
        elif args.only == "conv":
            xs, ws, at = RESNET_3X3
            x = randn(*xs)
            wt = torch.from_numpy((rng.standard_normal(ws) * 0.05).astype(np.float32)).to(dev)
            y = torch.empty(ops.conv_output_shape(xs, ws, **at), device=dev, dtype=torch.float32)
            w = None
            for _ in range(args.steps):
                ops.conv_f32_dev(x.data_ptr(), xs, wt.data_ptr(), ws, y.data_ptr(), ctx=ctx, **at)
        elif args.only == "gqa512":
            h, kv, hs, s_ = 32, 8, 64, 512
            q, k, v = randn(1, s_, h * hs), randn(1, s_, kv * hs), randn(1, s_, kv * hs)
            cos, sin = randn(s_, hs // 2), randn(s_, hs // 2)
            y = torch.empty_like(q)
            prk = torch.empty((1, kv, s_, hs), device=dev)
            prv = torch.empty_like(prk)
            w = None
            for _ in range(args.steps):
                ops.group_query_attention_dev(
                    q.data_ptr(), k.data_ptr(), v.data_ptr(), 1, s_, h * hs, h, kv, y.data_ptr(),
                    prk.data_ptr(), prv.data_ptr(), cos_ptr=cos.data_ptr(),
                    sin_ptr=sin.data_ptr(), max_pos=s_, half_rot=hs // 2, do_rotary=True,
                    ctx=ctx)
        elif args.only == "gqadec":
            h, kv, hs, past = 32, 8, 64, 4096
            q, k, v = randn(1, 1, h * hs), randn(1, 1, kv * hs), randn(1, 1, kv * hs)
            pk, pv = randn(1, kv, past, hs), randn(1, kv, past, hs)
            cos, sin = randn(past + 1, hs // 2), randn(past + 1, hs // 2)
            y = torch.empty_like(q)
            prk = torch.empty((1, kv, past + 1, hs), device=dev)
            prv = torch.empty_like(prk)
            w = None
            for _ in range(args.steps):
                ops.group_query_attention_dev(
                    q.data_ptr(), k.data_ptr(), v.data_ptr(), 1, 1, h * hs, h, kv, y.data_ptr(),
                    prk.data_ptr(), prv.data_ptr(), past_key_ptr=pk.data_ptr(),
                    past_value_ptr=pv.data_ptr(), past_len=past, cos_ptr=cos.data_ptr(),
                    sin_ptr=sin.data_ptr(), max_pos=past + 1, half_rot=hs // 2, do_rotary=True,
                    ctx=ctx)
        elif args.only == "qconv":
            xs, ws, at = RESNET_3X3
            x = torch.randint(0, 256, xs, device=dev, dtype=torch.uint8)
            wt = torch.randint(-128, 128, ws, device=dev, dtype=torch.int8)
            y = torch.empty(ops.conv_output_shape(xs, ws, **at), device=dev, dtype=torch.uint8)
            wsc = rng.uniform(0.002, 0.02, ws[0]).astype(np.float32)
            wz = np.zeros(ws[0], np.int8)
            w = None
            for _ in range(args.steps):
                ops.qlinear_conv_dev(x.data_ptr(), False, xs, 0.05, 128, wt.data_ptr(), True, ws,
                                     wsc, wz, 4.0, 128, y.data_ptr(), lo=0, hi=255, ctx=ctx, **at)
        elif args.only == "attn":
            dh = MINILM_H // MINILM_HEADS
            q = randn(MINILM_B, MINILM_HEADS, MINILM_S, dh)
            kt = randn(MINILM_B, MINILM_HEADS, dh, MINILM_S)
            v = randn(MINILM_B, MINILM_HEADS, MINILM_S, dh)
            mask = torch.zeros((MINILM_B, 1, 1, MINILM_S), device=dev)
            y = torch.empty_like(v)
            w = None
            for _ in range(args.steps):
                ops.fused_sdpa_dev(q.data_ptr(), q.shape, kt.data_ptr(), kt.shape, v.data_ptr(),
                                   v.shape, mask.data_ptr(), mask.shape, 1.0 / np.sqrt(dh),
                                   y.data_ptr(), ctx=ctx)
    torch.cuda.synchronize()
    print(f"{args.only}: {args.steps} launches", flush=True)
    if w is not None:
        w.release()


if __name__ == "__main__":
    main()
