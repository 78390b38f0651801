#!/usr/bin/env python3
"""Benchmark: BERT-base encoder seqs/s on one MI355X through the zenith_amd
HIP kernels (BASELINE.json metric, config 5 at b32 s128 fp16).

One step = one forward of the 12-layer encoder over one batch of 32
sequences x 128 tokens (synthetic, seeded; key-padding lengths ~ U{64..128}),
replayed from a HIP graph, inputs resident in HBM. Prints ONE JSON line.

Also measured in the same run:
  roofline  - the dominant kernel (FFN GEMM, 4096x768 -> 3072 with the fused
              bias+GELU epilogue) timed with HIP events on its launch stream;
              achieved = 2*M*N*K / average launch time vs the 2.5 PFLOP/s fp16
              dense MFMA peak. `traffic` comes from the committed rocprofv3
              PMC summary (profiles/gemm_ffn_up_pmc.json) when present.
  cpu_baseline - the CPU oracle (numpy fp32 restatement of the reference's CPU
              path) on a bounded sample of the same workload (whole sequences
              of 128 tokens through 12 layers), on this host's cores.
  int8      - the INT8-FFN variant of the same encoder (extra field).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "BERT-base seqs/s (b32,s128,fp16/int8); GEMM & attn TFLOPS as % of MI355X peak"
PEAK_FP16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0


def _args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--seq", type=int, default=128)
    ap.add_argument("--layers", type=int, default=12)
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="bound on the CPU-baseline sample (whole sequences)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-int8", action="store_true")
    return ap.parse_args()


def time_kernel_events(torch, launch, n_iter=200, n_warm=20):
    """Average duration of `launch()` (one kernel) over n_iter back-to-back
    launches, bracketed by HIP events recorded on the launch stream."""
    stream = torch.cuda.current_stream()
    for _ in range(n_warm):
        launch()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(n_iter):
        launch()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / n_iter  # seconds per launch


def gemm_roofline(torch, dev):
    import numpy as np

    from zenith_amd import _lib as L
    from zenith_amd import synthetic

    M, K, N = 4096, 768, 3072
    a = torch.from_numpy(synthetic.normal((M, K), tag=1)).to(dev, torch.float16)
    w = torch.from_numpy(synthetic.normal((N, K), tag=2, std=0.02)).to(dev, torch.float16)
    b = torch.zeros(N, dtype=torch.float16, device=dev)
    c = torch.empty((M, N), dtype=torch.float16, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    args = (a.data_ptr(), w.data_ptr(), c.data_ptr(), M, N, K, K, K, N, 1, L.ZK_F16,
            b.data_ptr(), None, 0, L.ZK_EPI_BIAS_GELU_ERF, stream)
    fn = L.load().zk_gemm_f16

    def launch():
        rc = fn(*args)
        if rc:
            raise RuntimeError(L.last_error())

    t = time_kernel_events(torch, launch)
    flops = 2.0 * M * N * K
    achieved = flops / t / 1e12
    traffic = None
    pmc = os.path.join(ROOT, "profiles", "gemm_ffn_up_pmc.json")
    if os.path.exists(pmc):
        try:
            with open(pmc) as f:
                traffic = json.load(f).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    del np
    return {
        "kernel": "gemm_mfma_kernel<F16,128x128,bias+gelu_erf> M=4096 N=3072 K=768",
        "bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP16_TFLOPS,
        "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP16_TFLOPS, 4), "traffic": traffic,
        "avg_launch_us": round(t * 1e6, 3), "flops_per_launch": flops,
    }


def cpu_baseline(seq: int, layers: int, budget_s: float):
    """Oracle fp32 encoder on whole sequences until the time budget is used."""
    import numpy as np

    from oracle import bert as obert
    from zenith_amd import synthetic

    try:
        from threadpoolctl import threadpool_info

        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
        blas = ",".join(sorted({i.get("internal_api", "?") for i in threadpool_info()}))
    except Exception:  # pragma: no cover
        threads, blas = int(os.environ.get("OMP_NUM_THREADS", "1")), "unknown"
    w = synthetic.bert_weights(layers, seed=42)
    x = synthetic.hidden_states(4, seq, seed=42)
    lens = synthetic.padding_lengths(4, seq)
    obert.bert_encoder(x[:1], w[:1], lens[:1])  # warm-up (BLAS threads, caches)
    done, t0 = 0, time.perf_counter()
    while True:
        i = done % 4
        obert.bert_encoder(x[i:i + 1], w, lens[i:i + 1])
        done += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return {
        "value": round(done / el, 4), "unit": "seqs/s", "cores": int(threads), "kind": "port",
        "sample": f"{done} sequences x {seq} tokens through {layers} fp32 layers "
                  f"(numpy oracle, {blas} BLAS), {el:.1f} s; host cpus={len(os.sched_getaffinity(0))}",
    }


def main():
    args = _args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the encoder shards by batch; "
              "multi-GPU runs are not part of it). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    from zenith_amd import synthetic
    from zenith_amd.encoder import BertEncoder

    if not torch.cuda.is_available():
        print("bench.py: no GPU available", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    B, S = args.batch, args.seq
    layers = synthetic.bert_weights(args.layers, seed=42)
    enc = BertEncoder(layers, device=dev)
    x = torch.from_numpy(synthetic.hidden_states(B, S, seed=42)).to(dev, torch.float16)
    lens = torch.from_numpy(synthetic.padding_lengths(B, S)).to(dev)
    gx, gl, go = enc.capture(B, S)
    gx.copy_(x)
    gl.copy_(lens)

    def timed(steps, warmup):
        for _ in range(warmup):
            enc.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            enc.replay()
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    dt = timed(args.steps, args.warmup)
    seqs_s = B * args.steps / dt
    out = go.float()
    assert torch.isfinite(out).all(), "non-finite encoder output"

    int8 = None
    if not args.no_int8:
        # per-layer activation scales from one fp16 calibration pass
        s_x, s_h = _calibrate(enc, x, lens, torch)
        enc.enable_int8_ffn(s_x, s_h, layers_fp32=layers)
        enc.capture(B, S)
        enc._gx.copy_(x)
        enc._gl.copy_(lens)
        dt8 = timed(args.steps, args.warmup)
        int8 = {"value": round(B * args.steps / dt8, 2), "ms_per_step": round(dt8 / args.steps * 1e3, 4)}
        enc.disable_int8_ffn()

    roof = gemm_roofline(torch, dev)
    cpu = None if args.no_cpu else cpu_baseline(S, args.layers, args.cpu_seconds)
    fwd_flops = args.layers * (2 * B * S * 768 * (3 * 768 + 768 + 2 * 3072) + 4 * B * 12 * S * S * 64)
    line = {
        "metric": METRIC, "value": round(seqs_s, 2), "unit": "seqs/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(dt / args.steps * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (seeded N(0,1) tokens, N(0,0.02) random-init weights, lengths U{S/2..S})",
        "config": {"workload": f"BERT-base {args.layers}-layer post-LN encoder fwd, b{B} s{S}, fp16, "
                               "key-padding mask, HIP-graph replay",
                   "global_batch": B, "seq_len": S, "parallelism": "none (1 GPU)"},
        "encoder_tflops": round(fwd_flops * args.steps / dt / 1e12, 2),
        "int8_ffn": int8,
        "roofline": {k: roof[k] for k in ("bound", "achieved", "peak", "unit", "frac", "traffic")},
        "roofline_kernel": {k: roof[k] for k in ("kernel", "avg_launch_us", "flops_per_launch")},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def _calibrate(enc, x, lens, torch):
    """absmax/127 of the FFN-up input (h1) and GELU output (u) per layer from
    one eager fp16 pass (MinMax rule, zenith/optimization/quantization.py:101-107)."""
    from zenith_amd import _lib as L

    B, S, H = x.shape
    enc._buffers(B, S)
    bf = enc._bufs
    stream = torch.cuda.current_stream().cuda_stream
    cur = x.reshape(B * S, H).contiguous()
    s_x, s_h = [], []
    for i in range(len(enc.layers)):
        out = torch.empty_like(cur)
        enc._layer(i, cur, out, lens, B, S, stream)
        s_x.append(max(float(bf["h1"].abs().max()) / 127.0, 1e-8))
        s_h.append(max(float(bf["u"].abs().max()) / 127.0, 1e-8))
        cur = out
    del L
    return s_x, s_h


if __name__ == "__main__":
    main()
