"""Throughput of the gfx950 BERT encoder forward: sentences/s at MiniLM-L6 shape,
batch 256 x seq 128, fp32, with the p50 batch latency.

One step = one ``ebh_encode_device`` forward of the whole batch (embeddings ->
L layers -> mean pool -> L2 normalise) over ids / mask already resident in
HBM, ending with the stream synchronised.  From the second call on, a forward
of the same shape on the same buffers replays as a HIP graph (the library's
default; ``--no-graph-replay`` times direct launches).  Default workload: c3, MiniLM-L6
shape, batch 256 x seq 128, fp32, seeded synthetic ids, random-init weights.

Prints one JSON line.  ``roofline`` is measured live, over as many forwards
again right after the timed region, for one kernel family
(default: the FFN-up GEMM, the largest single launch) with HIP events on the
stream its launches go to; its ``traffic`` (HBM bytes per launch) is read from
the committed rocprofv3 counter summary for the same workload and kernel, when
there is one.  ``cpu_baseline`` times the repo's C restatement of the
reference CPU path (``oracle/``) on a bounded sample of the same workload on
this host, with its built-in sgemm (the reference's default build) and with
OpenBLAS (its ``openblas`` feature).  ``host_api`` is the rate of the blocking host-buffer entry point
(``ebh_encode``: ids / mask copied in over PCIe, vectors copied back); it is
reported beside ``value``, never as it.  ``encode_texts`` is the rate from
texts (``Model::encode`` without its cache): the native tokenizer on host
threads writing into the pinned staging buffers, then the same forward; the
texts are the workload's ids spelled as words of a synthetic vocabulary, so
they tokenise back to exactly those ids (``matches_ids``).  Beside it, the
tokenisation alone, native and with the HF ``tokenizers`` library the
reference uses.

``kernels`` gives every kernel family of the headline forward the same way as
``roofline`` (HIP events, fraction of its roofline).  ``configs`` holds the
other benchmark configs (c5, c4, c2, c1 by default), each timed after the
headline with its own model exactly as the headline is (``value``,
``ms_per_step``, p50), with its dominant kernel family as ``roofline`` and
every family under ``kernels``; ``value`` and ``metric`` stay on c3.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

# MI355X published dense peaks: fp32 matrix 157.3 TFLOP/s, bf16 2.5 PFLOP/s; HBM3E 8 TB/s.
# Dense matrix peaks of MI355X per algorithmic flop: fp32 MFMA, bf16 MFMA, and
# fp32 products formed from six bf16 MFMA products (the bf16 peak / 6).
PEAK_TFLOPS = {"fp32": 157.3, "bf16": 2500.0, "fp32-bf16x6": 2500.0 / 6}
HBM_PEAK_GBS = 8000.0
KERNELS = ("gemm_qkv", "attention", "gemm_out", "gemm_ffn_up", "gemm_ffn_down", "layernorm",
           "embed", "pool")


def few_fused(cfg, B: int, S: int, dtype: str) -> bool:
    """Whether the library runs attention and the attention-output projection
    of this batch as one launch (the rule of few_attn_fits in
    edgebert_amd/csrc/few.hip): fp32 GEMMs, at most 64 positions, hidden 384
    in heads of 32.  Its profiled "attention" launch then includes the output
    projection's partials."""
    H, nh = cfg.hidden_size, cfg.num_attention_heads
    return dtype != "bf16" and 0 < B * S <= 64 and H == 384 and H == 32 * nh


def kernel_work(cfg, lengths, B: int, which: str, fused: bool = False, dtype: str = "fp32"):
    """Algorithmic work of ONE launch of a kernel family: (amount, bound, unit).

    GEMMs: 2*T*N*K FLOPs over the T valid tokens.  Attention: 4*H*sum(l^2)
    FLOPs (q.k^T and p.v at 2 FLOP per MAC); with bf16 q / k / v (bf16 models)
    the kernel is HBM-bound instead: q, k, v read and the context written once,
    4*T*H*2 bytes.  Row kernels: the HBM bytes the op must move at minimum
    (each operand read once, each result written once), in the activation
    encoding of the model (bf16 models keep the GEMM outputs and the residual
    stream in bf16).  Embeddings: a word row per token, but each of the
    max(l) position rows once (every sequence shares them, so after the first
    read they come from cache).  fused: the few-token layer's launches
    (few_fused).
    """
    H, I = cfg.hidden_size, cfg.intermediate_size
    lengths = np.asarray(lengths, np.float64)
    T = float(lengths.sum())
    P = float(lengths.max()) if lengths.size else 0.0   # distinct position rows
    if dtype == "bf16":
        if which == "attention":
            return 4.0 * T * H * 2, "hbm", "byte"
        if which == "layernorm":      # bf16 product and residual read, bf16 residual written
            return 3.0 * T * H * 2 + 3 * H * 4, "hbm", "byte"
        if which == "embed":          # fp32 word row in, bf16 row written per token
            return T * (8 + H * 4 + H * 2) + P * H * 4 + 3 * H * 4, "hbm", "byte"
        if which == "pool":           # the bf16 residual stream once, one fp32 vector per sequence
            return T * H * 2 + B * H * 4 + (B + 1) * 4, "hbm", "byte"
    if fused and which == "attention":
        return 2.0 * T * H * H + 4.0 * H * float((lengths ** 2).sum()), "mfma", "flop"
    if fused and which == "gemm_out":
        raise KeyError("gemm_out runs inside the attention launch at this size")
    if which == "gemm_qkv":
        return 2.0 * T * H * 3 * H, "mfma", "flop"
    if which == "gemm_out":
        return 2.0 * T * H * H, "mfma", "flop"
    if which == "gemm_ffn_up":
        return 2.0 * T * H * I, "mfma", "flop"
    if which == "gemm_ffn_down":
        return 2.0 * T * I * H, "mfma", "flop"
    if which == "attention":
        return 4.0 * H * float((lengths ** 2).sum()), "mfma", "flop"
    if which == "layernorm":          # read the GEMM output row, write the normalised row
        return 2.0 * T * H * 4 + 2 * H * 4, "hbm", "byte"
    if which == "embed":              # token id + position, word row in, row written per token
        return T * (8 + 2 * H * 4) + P * H * 4 + 3 * H * 4, "hbm", "byte"
    if which == "pool":               # every token row once, one vector per sequence
        return T * H * 4 + B * H * 4 + (B + 1) * 4, "hbm", "byte"
    raise KeyError(which)


def forward_flops(cfg, lengths) -> float:
    """L * [2 l (4H^2 + 2HI) + 4 l^2 H] per sequence of valid length l."""
    H, I, L = cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers
    lengths = np.asarray(lengths, np.float64)
    return float(L * (2 * lengths * (4 * H * H + 2 * H * I) + 4 * lengths ** 2 * H).sum())


def measured_traffic(config: str, kernel: str, dtype: str):
    """HBM bytes per launch from the committed counter summary
    (profiles/hbm_traffic_<config>.md, lines ``traffic[<kernel>][<dtype>] = <bytes>``)."""
    path = os.path.join(ROOT, "profiles", f"hbm_traffic_{config}.md")
    if not os.path.exists(path):
        return None
    pat = re.compile(r"^traffic\[(\w+)\]\[(\w+)\]\s*=\s*(\d+)")
    with open(path) as f:
        for line in f:
            m = pat.match(line.strip())
            if m and m.group(1) == kernel and m.group(2) == dtype:
                return int(m.group(3))
    return None


def cpu_baseline(spec, weights, ids, mask, budget_s: float):
    """Oracle (C port of the reference CPU path) on chunks of 16 sequences of
    the same workload, in the reference's two builds: the default features
    (matrixmultiply sgemm, restated in oracle.c) and ``--features openblas``
    (every product on OpenBLAS's cblas_sgemm, here the OpenBLAS numpy links).
    Each runs for half of ``budget_s`` after one warm-up chunk; ``value`` is
    the faster of the two."""
    import oracle
    om = oracle.OracleModel(spec.model, weights)
    chunk = 16

    def timed(seconds):
        om.encode(ids[:chunk], mask[:chunk])           # warm-up
        done, t0, i = 0, time.perf_counter(), 0
        while True:
            lo = (i * chunk) % spec.batch
            om.encode(ids[lo:lo + chunk], mask[lo:lo + chunk])
            done += chunk
            i += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                return done, el

    variants = {}
    done, el = timed(budget_s / 2)
    variants["default"] = {"value": round(done / el, 3), "sequences": done, "seconds": round(el, 1)}
    blas = None
    try:
        blas = oracle.use_openblas(True)
        done, el = timed(budget_s / 2)
        variants["openblas"] = {"value": round(done / el, 3), "sequences": done,
                                "seconds": round(el, 1), "library": os.path.basename(blas)}
    except oracle.OracleError as e:
        variants["openblas"] = {"value": None, "error": str(e)}
    finally:
        oracle.use_openblas(False)
    best = max((k for k in variants if variants[k]["value"]), key=lambda k: variants[k]["value"])
    n = oracle.get_num_threads()
    return {"value": variants[best]["value"], "unit": "sentences/s", "cores": n, "kind": "port",
            "sample": f"sequences of the {spec.name} workload (seq {spec.seq_len}) in chunks of "
                      f"{chunk}, about {budget_s / 2:.0f} s per build, oracle/liboracle.so on {n} "
                      f"OpenMP threads of {os.cpu_count()} host CPUs; value = the faster build "
                      f"({best})",
            "variants": variants}


def text_path(model, spec, ids, mask, lengths, steps: int) -> dict:
    """Texts -> vectors through ebh_encode_texts, and the tokenisers alone."""
    from edgebert_amd import synth
    from edgebert_amd.tokenizer import Tokenizer, hf_tokenizer_from_str

    doc = synth.tokenizer_json(spec.model)
    tok = Tokenizer.from_str(doc)
    texts = synth.make_texts(ids, lengths)
    B = len(texts)
    model.tokenizer = tok
    ref = model.encode_ids(ids, mask, normalize=True)
    got = model.encode_texts(texts, True)
    t0 = time.perf_counter()
    for _ in range(steps):
        model.encode_texts(texts, True)
    el = time.perf_counter() - t0
    t0 = time.perf_counter()
    for _ in range(steps):
        tok.encode_batch_ids(texts)
    el_tok = time.perf_counter() - t0
    # Several batches through encode_texts_many (encode_batch's schedule: two
    # host threads, one batch tokenising while the other's forward runs).
    many = [texts] * max(steps, 2)
    model.encode_texts_many(many[:2], True)
    t0 = time.perf_counter()
    model.encode_texts_many(many, True)
    el_many = time.perf_counter() - t0
    out = {"value": round(B * steps / el, 2), "unit": "sentences/s",
           "pipelined": round(B * len(many) / el_many, 2),
           "matches_ids": bool(np.array_equal(got, ref)),
           "tokenize_native": round(B * steps / el_tok, 2),
           "threads": min(16, os.cpu_count() or 1)}
    try:
        hf = hf_tokenizer_from_str(doc)
        hf.encode_batch(texts, add_special_tokens=True)
        t0 = time.perf_counter()
        for _ in range(steps):
            hf.encode_batch(texts, add_special_tokens=True)
        out["tokenize_hf_tokenizers"] = round(B * steps / (time.perf_counter() - t0), 2)
    except ImportError:
        out["tokenize_hf_tokenizers"] = None
    out["note"] = ("ebh_encode_texts: native tokenizer on host threads into pinned staging + H2D + "
                   "forward + D2H, one batch per call; pipelined: batches on two host threads, one "
                   "tokenising while the other's forward runs; tokenize_*: encode_batch alone")
    return out


def split_product_run(eb, torch, spec, weights, d_ids, d_mask, d_ref, lengths, steps, warmup,
                      profile_kernel, graph_replay):
    """The same workload on an EBH_DTYPE_F32_BF16X6 model: fp32 weights and
    activations, every large GEMM product formed from six bf16 MFMA products
    of three-way bf16 splits (fp32 accumulate).  Reported beside the headline,
    which stays on the fp32 MFMA path: sentences/s, its FFN-up roofline
    against the bf16 peak / 6, and the largest difference of its vectors from
    the fp32 path's on this batch."""
    cfg = spec.model
    B, S = d_ids.shape
    m = eb.Model.from_weights(weights, cfg, "fp32-bf16x6")
    out = torch.empty_like(d_ref)
    stream = torch.cuda.current_stream().cuda_stream
    if not graph_replay:
        m.set_graph_replay(False)

    def step():
        m.encode_device(d_ids.data_ptr(), d_mask.data_ptr(), B, S, out.data_ptr(), True, stream)

    for _ in range(warmup):
        step()
    m.synchronize()
    torch.cuda.synchronize()
    times = []
    t_all = time.perf_counter()
    for _ in range(steps):
        t0 = time.perf_counter()
        step()
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    wall = time.perf_counter() - t_all
    m.synchronize()
    max_abs = float((out - d_ref).abs().max())
    m.profile_enable(profile_kernel)
    for _ in range(steps):
        step()
    m.synchronize()
    torch.cuda.synchronize()
    launches, prof_ms = m.profile_read()
    m.profile_enable("none")
    m.close()
    # At most 64 positions the few-token kernels run plain fp32 MFMA products
    # for this dtype too (their products are memory round trips, not MFMA work).
    few = B * S <= 64
    work, bound, wunit = kernel_work(cfg, lengths, B, profile_kernel, few_fused(cfg, B, S, "fp32-bf16x6"))
    avg = prof_ms / max(launches, 1)
    peak = PEAK_TFLOPS["fp32" if few else "fp32-bf16x6"] if bound == "mfma" else HBM_PEAK_GBS
    achieved = work / (avg * 1e-3) / (1e12 if bound == "mfma" else 1e9)
    return {"value": round(B * steps / wall, 2), "unit": "sentences/s",
            "ms_per_step": round(1e3 * wall / steps, 4),
            "p50_batch_latency_ms": round(float(np.median(times)) * 1e3, 4),
            "max_abs_vs_fp32_path": max_abs,
            "gemm_arithmetic": "fp32 MFMA products: at most 64 positions the few-token kernels do not "
                               "split (EBH_DTYPE_F32_BF16X6)" if few else
                               "fp32 operands split into three bf16 parts, six bf16 MFMA products "
                               "per fp32 product, fp32 accumulate (EBH_DTYPE_F32_BF16X6)",
            "roofline": {"kernel": profile_kernel, "bound": bound, "achieved": round(achieved, 3),
                         "peak": round(peak, 1), "unit": "TFLOP/s" if bound == "mfma" else "GB/s",
                         "frac": round(achieved / peak, 4), "avg_launch_ms": round(avg, 5),
                         "launches": launches}}


LEG_DTYPE_NOTE = {
    "fp32": "f32 (GEMM operands, accumulation, residual stream, LayerNorm, softmax)",
    "bf16": "bf16 GEMM and attention operands with fp32 accumulation; bf16 residual stream "
            "(the skip connection carries bf16-rounded values); LayerNorm statistics, softmax "
            "and pooling in fp32",
}


def config_leg(eb, torch, name: str, steps: int, warmup: int, graph_replay: bool) -> dict:
    """One BASELINE config timed as the headline is (forwards over HBM-resident
    ids / mask, graph replay unless disabled), then every kernel family of its
    forward timed with HIP events over as many forwards again (direct
    launches), each as a fraction of its roofline: GEMMs and attention against
    the matrix peak of the config's dtype, row kernels against HBM.  ``traffic``
    is the committed counter summary's HBM bytes per launch, where one exists
    for that config."""
    spec = eb.CONFIGS[name]
    cfg, dtype = spec.model, spec.dtype
    weights = eb.make_weights(cfg)
    ids, mask, lengths = eb.make_inputs(spec)
    B, S = ids.shape
    model = eb.Model.from_weights(weights, cfg, dtype)
    del weights
    if not graph_replay:
        model.set_graph_replay(False)
    dev = torch.device("cuda:0")
    d_ids = torch.from_numpy(ids).to(dev)
    d_mask = torch.from_numpy(mask).to(dev)
    d_out = torch.empty((B, cfg.hidden_size), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream

    def step():
        model.encode_device(d_ids.data_ptr(), d_mask.data_ptr(), B, S, d_out.data_ptr(), True, stream)

    for _ in range(warmup):
        step()
    model.synchronize()
    torch.cuda.synchronize()
    times = []
    t_all = time.perf_counter()
    for _ in range(steps):
        t0 = time.perf_counter()
        step()
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    wall = time.perf_counter() - t_all
    model.synchronize()
    fused = few_fused(cfg, B, S, dtype)
    families = {}
    for fam in KERNELS:
        if fused and fam == "gemm_out":
            continue
        model.profile_enable(fam)
        for _ in range(steps):
            step()
        model.synchronize()
        torch.cuda.synchronize()
        launches, prof_ms = model.profile_read()
        model.profile_enable("none")
        if not launches:
            continue
        avg = prof_ms / launches
        work, bound, wunit = kernel_work(cfg, lengths, B, fam, fused, dtype)
        if bound == "mfma":
            achieved, peak, punit = work / (avg * 1e-3) / 1e12, PEAK_TFLOPS[dtype], "TFLOP/s"
        else:
            achieved, peak, punit = work / (avg * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s"
        families[fam] = {"bound": bound, "achieved": round(achieved, 3), "peak": peak, "unit": punit,
                         "frac": round(achieved / peak, 4), "avg_launch_ms": round(avg, 5),
                         "launches": launches, "per_forward": launches // steps,
                         "traffic": measured_traffic(name, fam, dtype)}
    model.close()
    ms = 1e3 * wall / steps
    top = max(families, key=lambda f: families[f]["avg_launch_ms"] * families[f]["per_forward"])
    return {"value": round(B * steps / wall, 2), "unit": "sentences/s", "steps": steps, "warmup": warmup,
            "ms_per_step": round(ms, 4), "p50_batch_latency_ms": round(float(np.median(times)) * 1e3, 4),
            "dtype": LEG_DTYPE_NOTE[dtype],
            "workload": f"{name}: {cfg.num_hidden_layers}L H{cfg.hidden_size} I{cfg.intermediate_size} "
                        f"heads{cfg.num_attention_heads} batch {B} x seq {S}, lengths "
                        f"{spec.len_lo}-{spec.len_hi}",
            "valid_tokens": int(mask.sum()),
            "forward_tflops": round(forward_flops(cfg, lengths) / (ms * 1e-3) / 1e12, 2),
            "graph_replay": graph_replay,
            "roofline": dict(kernel=top, **families[top]),
            "kernels": families}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c3", choices=["c1", "c2", "c3", "c4", "c5"])
    ap.add_argument("--dtype", default=None, help="fp32 | bf16 | fp32-bf16x6 (default: the config's)")
    ap.add_argument("--bf16x6-steps", type=int, default=None,
                    help="fp32 configs: also time an EBH_DTYPE_F32_BF16X6 model (fp32 GEMM products "
                         "from six bf16 MFMA products) for this many steps, reported under "
                         "fp32_bf16x6 beside the headline (default: --steps; 0 disables)")
    ap.add_argument("--profile-kernel", default="gemm_ffn_up", choices=KERNELS)
    ap.add_argument("--cpu-budget", type=float, default=16.0,
                    help="seconds of CPU baseline work, split over its two builds (0 disables)")
    ap.add_argument("--host-api-steps", type=int, default=5,
                    help="blocking host-buffer forwards timed for host_api (0 disables)")
    ap.add_argument("--text-steps", type=int, default=5,
                    help="batches timed for encode_texts and the tokenizers (0 disables)")
    ap.add_argument("--no-graph-replay", action="store_true",
                    help="run every forward as direct launches (no HIP graph replay)")
    ap.add_argument("--legs", default=None,
                    help="comma-separated BASELINE configs also timed, each with its own model, after "
                         "the headline and reported under `configs` (default with --config c3: "
                         "c5,c4,c2,c1; 'none' disables)")
    ap.add_argument("--leg-steps", type=int, default=10, help="timed forwards per leg")
    ap.add_argument("--copy-probe-mb", type=int, default=0,
                    help="after the timed region, run 3 plain device copies of this many MiB "
                         "(the calibration dispatch for rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported "
              "(the forward shards as pure data parallelism over the batch: one process per GPU, "
              "each with its own slice of sentences)",
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

    if args.no_graph_replay:
        model.set_graph_replay(False)
    for _ in range(args.warmup):
        step()
    model.synchronize()
    torch.cuda.synchronize()

    def timed(n):
        times = []
        torch.cuda.synchronize()
        t_all = time.perf_counter()
        for _ in range(n):
            t0 = time.perf_counter()
            step()
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
        torch.cuda.synchronize()
        return time.perf_counter() - t_all, times

    # The timed region: forwards as a caller runs them (graph replay on unless
    # --no-graph-replay).  Then the same number of forwards with one kernel
    # family timed by HIP events on its stream (those run as direct launches)
    # for the roofline.
    wall, times = timed(args.steps)
    model.synchronize()
    model.profile_enable(args.profile_kernel)
    timed(args.steps)
    model.synchronize()
    launches, prof_ms = model.profile_read()
    model.profile_enable("none")

    times = np.array(times)
    ms_per_step = 1e3 * wall / args.steps
    value = B * args.steps / wall
    tokens = int(mask.sum())
    avg_kernel_ms = prof_ms / max(launches, 1)
    fused = few_fused(cfg, B, S, dtype)
    work, bound, wunit = kernel_work(cfg, lengths, B, args.profile_kernel, fused, dtype)
    if bound == "mfma":
        achieved, peak, punit = work / (avg_kernel_ms * 1e-3) / 1e12, PEAK_TFLOPS[dtype], "TFLOP/s"
    else:
        achieved, peak, punit = work / (avg_kernel_ms * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s"
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
        "dtype": {"fp32": "f32", "bf16": "bf16", "fp32-bf16x6": "f32 (bf16x6 GEMM products)"}[dtype],
        "data": "synthetic (seeded ids, random-init N(0,0.02) weights; no checkpoint offline)",
        "config": {"workload": f"{args.config}: {cfg.num_hidden_layers}L H{cfg.hidden_size} "
                               f"I{cfg.intermediate_size} heads{cfg.num_attention_heads} "
                               f"batch {B} x seq {S}",
                   "global_batch": B, "seq_len": S, "valid_tokens": tokens,
                   "parallelism": "single GPU"},
        "forward_tflops": round(fwd_flops / (ms_per_step * 1e-3) / 1e12, 2),
        "graph_replay": not args.no_graph_replay,
        "roofline": {"kernel": args.profile_kernel + (" (with the output projection)"
                                                      if fused and args.profile_kernel == "attention" else ""),
                     "bound": bound, "achieved": round(achieved, 3),
                     "peak": peak, "unit": punit, "frac": round(achieved / peak, 4),
                     "traffic": measured_traffic(args.config, args.profile_kernel, dtype),
                     "work_per_launch": work, "work_unit": wunit,
                     "avg_launch_ms": round(avg_kernel_ms, 5), "launches": launches},
    }
    if args.host_api_steps > 0:
        model.encode_ids(ids, mask, normalize=True)           # warm the host staging buffers
        t0 = time.perf_counter()
        for _ in range(args.host_api_steps):
            model.encode_ids(ids, mask, normalize=True)
        el = time.perf_counter() - t0
        result["host_api"] = {"value": round(B * args.host_api_steps / el, 2),
                              "unit": "sentences/s",
                              "note": "ebh_encode on host buffers: validation + H2D + forward + D2H"}
    if args.text_steps > 0:
        result["encode_texts"] = text_path(model, spec, ids, mask, lengths, args.text_steps)
    if args.copy_probe_mb > 0:
        n = args.copy_probe_mb * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        result["copy_probe_bytes"] = n * 4
    x6_steps = args.steps if args.bf16x6_steps is None else args.bf16x6_steps
    if dtype == "fp32" and x6_steps > 0:
        result["fp32_bf16x6"] = split_product_run(eb, torch, spec, weights, d_ids, d_mask, d_out, lengths,
                                                  x6_steps, args.warmup, args.profile_kernel,
                                                  not args.no_graph_replay)
    # The headline's own kernel families, as the legs report theirs.
    fams = {}
    for fam in KERNELS:
        if fused and fam == "gemm_out":
            continue
        model.profile_enable(fam)
        timed(args.steps)
        model.synchronize()
        n, fms = model.profile_read()
        model.profile_enable("none")
        if n:
            fwork, fbound, _ = kernel_work(cfg, lengths, B, fam, fused, dtype)
            favg = fms / n
            if fbound == "mfma":
                fa, fp, fu = fwork / (favg * 1e-3) / 1e12, PEAK_TFLOPS[dtype], "TFLOP/s"
            else:
                fa, fp, fu = fwork / (favg * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s"
            fams[fam] = {"bound": fbound, "achieved": round(fa, 3), "peak": fp, "unit": fu,
                         "frac": round(fa / fp, 4), "avg_launch_ms": round(favg, 5), "launches": n,
                         "traffic": measured_traffic(args.config, fam, dtype)}
    result["kernels"] = fams
    if args.cpu_budget > 0:
        result["cpu_baseline"] = cpu_baseline(spec, weights, ids, mask, args.cpu_budget)
    model.close()
    legs = args.legs if args.legs is not None else ("c5,c4,c2,c1" if args.config == "c3" else "none")
    legs = [c for c in legs.split(",") if c and c != "none" and c != args.config]
    if legs:
        del weights
        result["configs"] = {}
        for name in legs:
            result["configs"][name] = config_leg(eb, torch, name, args.leg_steps, args.warmup,
                                                 not args.no_graph_replay)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
