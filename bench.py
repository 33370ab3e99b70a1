"""Throughput of the gfx950 BERT encoder forward (BASELINE.json metric).

One step = one ``ebh_encode_device`` forward of the whole batch (embeddings ->
6 layers -> mean pool -> L2 normalise) over ids / mask already resident in
HBM, ending with the stream synchronised.  Default workload: c3, MiniLM-L6
shape, batch 256 x seq 128, fp32, seeded synthetic ids, random-init weights.

Prints one JSON line.  ``roofline`` is measured live for the dominant kernel
(the FFN-up GEMM) with HIP events on the stream its launches go to;
``cpu_baseline`` times the repo's C restatement of the reference CPU path
(``oracle/``) on a bounded sample of the same workload on this host.
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

PEAK = {"fp32": (157.3, "TFLOP/s"), "bf16": (2500.0, "TFLOP/s")}   # MI355X dense MFMA peaks
HBM_PEAK_GBS = 8000.0


def gemm_flops(cfg, tokens: int, which: str) -> float:
    H, I = cfg.hidden_size, cfg.intermediate_size
    return {"gemm_qkv": 2.0 * tokens * H * 3 * H, "gemm_out": 2.0 * tokens * H * H,
            "gemm_ffn_up": 2.0 * tokens * H * I, "gemm_ffn_down": 2.0 * tokens * I * H}[which]


def forward_flops(cfg, lengths) -> float:
    """L * [2 l (4H^2 + 2HI) + 4 l^2 H] per sequence of valid length l."""
    H, I, L = cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers
    lengths = np.asarray(lengths, np.float64)
    return float(L * (2 * lengths * (4 * H * H + 2 * H * I) + 4 * lengths ** 2 * H).sum())


def cpu_baseline(spec, weights, ids, mask, budget_s: float):
    """Oracle (C port of the reference CPU path) on chunks of 16 sequences of
    the same workload until ``budget_s`` has elapsed (after one warm-up chunk)."""
    import oracle
    om = oracle.OracleModel(spec.model, weights)
    chunk = 16
    om.encode(ids[:chunk], mask[:chunk])           # warm-up
    done, t0, i = 0, time.perf_counter(), 0
    while True:
        lo = (i * chunk) % spec.batch
        om.encode(ids[lo:lo + chunk], mask[lo:lo + chunk])
        done += chunk
        i += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return {"value": round(done / el, 3), "unit": "sentences/s",
            "cores": oracle.get_num_threads(), "kind": "port",
            "sample": f"{done} sequences of the {spec.name} workload (seq {spec.seq_len}) in "
                      f"chunks of {chunk}, {el:.1f} s, oracle/liboracle.so on "
                      f"{oracle.get_num_threads()} OpenMP threads"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c3", choices=["c1", "c2", "c3", "c4", "c5"])
    ap.add_argument("--dtype", default=None, help="fp32 | bf16 (default: the config's)")
    ap.add_argument("--profile-kernel", default="gemm_ffn_up")
    ap.add_argument("--cpu-budget", type=float, default=12.0,
                    help="seconds of CPU baseline work (0 disables)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported "
              "(the path shards as pure data parallelism over the batch, see DESIGN.md)",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import edgebert_amd as eb

    spec = eb.CONFIGS[args.config]
    dtype = args.dtype or spec.dtype
    cfg = spec.model
    weights = eb.make_weights(cfg)
    ids, mask, lengths = eb.make_inputs(spec)
    B, S = ids.shape
    model = eb.Model.from_weights(weights, cfg, dtype)

    dev = torch.device("cuda:0")
    d_ids = torch.from_numpy(ids).to(dev)
    d_mask = torch.from_numpy(mask).to(dev)
    d_out = torch.empty((B, cfg.hidden_size), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream

    def step():
        model.encode_device(d_ids.data_ptr(), d_mask.data_ptr(), B, S, d_out.data_ptr(),
                            True, stream)

    for _ in range(args.warmup):
        step()
    model.synchronize()
    torch.cuda.synchronize()

    model.profile_enable(args.profile_kernel)
    times = []
    torch.cuda.synchronize()
    t_all = time.perf_counter()
    for _ in range(args.steps):
        t0 = time.perf_counter()
        step()
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_all
    model.synchronize()
    launches, prof_ms = model.profile_read()
    model.profile_enable("none")

    times = np.array(times)
    ms_per_step = 1e3 * wall / args.steps
    value = B * args.steps / wall
    tokens = int(mask.sum())
    avg_kernel_ms = prof_ms / max(launches, 1)
    flops = gemm_flops(cfg, tokens, args.profile_kernel)
    achieved = flops / (avg_kernel_ms * 1e-3) / 1e12
    peak, punit = PEAK[dtype]
    fwd_flops = forward_flops(cfg, lengths)

    result = {
        "metric": "sentences/sec at MiniLM-L6 shape batch 256x seq 128 fp32; p50 batch latency"
        if args.config == "c3" else f"sentences/sec ({args.config})",
        "value": round(value, 2),
        "unit": "sentences/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "p50_batch_latency_ms": round(float(np.median(times)) * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if dtype == "fp32" else "bf16",
        "data": "synthetic (seeded ids, random-init N(0,0.02) weights; no checkpoint offline)",
        "config": {"workload": f"{args.config}: {cfg.num_hidden_layers}L H{cfg.hidden_size} "
                               f"I{cfg.intermediate_size} heads{cfg.num_attention_heads} "
                               f"batch {B} x seq {S}",
                   "global_batch": B, "seq_len": S, "valid_tokens": tokens,
                   "parallelism": "single GPU"},
        "forward_tflops": round(fwd_flops / (ms_per_step * 1e-3) / 1e12, 2),
        "roofline": {"kernel": args.profile_kernel, "bound": "mfma", "achieved": round(achieved, 3),
                     "peak": peak, "unit": punit, "frac": round(achieved / peak, 4),
                     "traffic": None, "avg_launch_ms": round(avg_kernel_ms, 5),
                     "launches": launches},
    }
    if args.cpu_budget > 0:
        result["cpu_baseline"] = cpu_baseline(spec, weights, ids, mask, args.cpu_budget)
    print(json.dumps(result), flush=True)
    model.close()


if __name__ == "__main__":
    main()
