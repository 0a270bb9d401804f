#!/usr/bin/env python3
"""Benchmark: residues/s of the ESM-2-650M W8A8 varlen packed forward on one
MI355X (varlen 256-sequence batch).

A step is one packed forward (embed, 33 encoder layers, final LN, lm head)
over the whole synthetic batch, with the batch already staged in HBM
(esm_gfx950_batch_upload before the timed region) and the logits left in
HBM. W warmup steps, then K timed steps bracketed by device syncs and HIP
events on the context stream. Every INT8 GEMM and attention launch inside
the timed region is also bracketed by HIP events (per-site timing), which
gives the dominant kernel's average launch duration for the roofline line.

cpu_baseline: the reference's own CPU path (its kernels compiled from source
into oracle/_ref/libesmref.so, driven in TransformerBlock order) on a
bounded sample of the same batch, timed on this host's cores. The same
sample is also run on the GPU in per-tensor (reference-parity) mode and the
logit correlation is reported.

Prints one JSON line. --gpus N > 1 exits: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "esm-cpp_amd"))

import esm_gfx950 as eg  # noqa: E402
from esm_gfx950 import synthetic as syn  # noqa: E402

MI355X_PEAK_INT8_TOPS = 5000.0  # dense int8, 5.0 POP/s
MI355X_PEAK_HBM_GBS = 8000.0
GEMM_SITES = ("qkv", "out", "fc1", "fc2")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gemm_ops(site, T, d, f):
    n, k = {"qkv": (3 * d, d), "out": (d, d), "fc1": (f, d), "fc2": (d, f)}[site]
    return 2.0 * T * n * k


def cpu_baseline(weights, batch, gpu_model, args):
    """Times the reference CPU forward on a sample; returns (record, parity)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from pyoracle import REF_LIB, RefLib, RefModel

    if not os.path.exists(REF_LIB):
        return None, None
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    threads = max(1, min(cores, args.cpu_threads))
    ref = RefLib(threads=threads)
    idx = list(range(0, len(batch.lengths), max(1, len(batch.lengths) // args.cpu_seqs)))[: args.cpu_seqs]
    sample = batch.subset(idx)
    t0 = time.time()
    rm = RefModel(ref, weights, int8=True)
    log(f"cpu: reference model built in {time.time() - t0:.1f}s (isa={ref.isa()}, threads={threads})")
    rm.forward_packed(sample)  # warmup
    times = []
    logits = None
    for _ in range(args.cpu_iters):
        t = time.perf_counter()
        logits = rm.forward_packed(sample)
        times.append(time.perf_counter() - t)
    rm.free()
    mean_s = float(np.mean(times))
    rec = {
        "value": round(sample.residues / mean_s, 1),
        "unit": "residues/s",
        "cores": threads,
        "kind": "reference",
        "sample": (f"{len(idx)} of {len(batch.lengths)} sequences ({sample.residues} residues, "
                   f"{sample.total_tokens} tokens), 1 warmup + {args.cpu_iters} timed ForwardPacked calls, "
                   f"mean {mean_s * 1000:.0f} ms; reference kernels isa={ref.isa()}"),
    }
    finite = bool(np.all(np.isfinite(logits)))
    gpu_model.set_act_mode(eg.ACT_PER_TENSOR)
    g = gpu_model.forward_packed(sample.ids, sample.cu)
    gpu_model.set_act_mode(eg.ACT_PER_TOKEN if args.act_mode == "token" else eg.ACT_PER_TENSOR)
    corr = float(np.corrcoef(g.ravel().astype(np.float64), logits.ravel().astype(np.float64))[0, 1])
    agree = float(np.mean(np.argmax(g, 1) == np.argmax(logits, 1)))
    parity = {"vs": "reference CPU path, per-tensor activation scale", "logit_corr": round(corr, 6),
              "argmax_agree": round(agree, 4), "cpu_finite": finite}
    return rec, parity


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=["varlen", "uniform"], default="varlen")
    ap.add_argument("--act-mode", choices=["token", "tensor"], default="token")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seqs", type=int, default=64)
    ap.add_argument("--cpu-iters", type=int, default=3)
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--parts", type=int, default=2,
                    help="concurrent sequence groups (streams) in the throughput pass")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on exactly one GPU (got --gpus {args.gpus}); the packed forward "
              "shards whole sequences across GPUs with no exchange -- see DESIGN.md.", file=sys.stderr)
        sys.exit(2)
    rank = int(os.environ.get("RANK", "0"))

    cfg = syn.ESM2_650M
    t0 = time.time()
    weights = syn.make_weights(cfg, seed=20261201 + 4, int8=True)
    batch = syn.config4_varlen_batch() if args.workload == "varlen" else syn.config4_uniform_batch()
    log(f"weights + batch in {time.time() - t0:.1f}s: T={batch.total_tokens} residues={batch.residues}")

    dev = eg.Device(0)
    mode = eg.ACT_PER_TOKEN if args.act_mode == "token" else eg.ACT_PER_TENSOR
    model = eg.Model(dev, weights, int8=True, act_mode=mode)
    T = batch.total_tokens
    logits = dev.empty((T, cfg.vocab_size), np.float32)
    model.set_parts(args.parts)
    model.upload_batch(batch.ids, batch.cu)
    for _ in range(args.warmup):
        model.forward_device(logits)
    dev.sync()
    log("warmup done")

    # Timed region without per-kernel events (throughput), then with them on
    # one stream (per-site kernel durations for the roofline).
    dev.sync()
    dev.timer_start()
    for _ in range(args.steps):
        model.forward_device(logits)
    ms_plain = dev.timer_stop() / args.steps
    if args.parts != 1:
        model.set_parts(1)
        model.upload_batch(batch.ids, batch.cu)
        model.forward_device(logits)
    dev.kernel_timing(True)
    dev.sync()
    dev.timer_start()
    for _ in range(args.steps):
        model.forward_device(logits)
    ms_events = dev.timer_stop() / args.steps
    sites = {}
    for site in GEMM_SITES + ("attention", "lm_dense"):
        n, tot = dev.kernel_timing_query(site)
        if n:
            sites[site] = {"launches": n, "avg_us": round(tot / n * 1000, 2), "ms_per_step": round(tot / args.steps, 3)}
    dev.kernel_timing(False)
    out = logits.numpy()
    if not np.all(np.isfinite(out)):
        raise SystemExit("bench: non-finite logits")
    log(f"ms/step {ms_plain:.3f} (with per-kernel events {ms_events:.3f}); sites {sites}")

    d, f = cfg.hidden_size, cfg.intermediate_size
    dom = max((s for s in GEMM_SITES if s in sites), key=lambda s: sites[s]["ms_per_step"])
    ops = gemm_ops(dom, T, d, f)
    achieved = ops / (sites[dom]["avg_us"] * 1e-6) / 1e12
    n_dom, k_dom = {"qkv": (3 * d, d), "out": (d, d), "fc1": (f, d), "fc2": (d, f)}[dom]
    # HBM bytes per launch of the dominant kernel, measured with rocprofv3
    # FETCH_SIZE / WRITE_SIZE passes scaled by a copy-kernel calibration (see
    # the profiles/ summaries); null when no measurement is recorded.
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as fh:
            rec_t = json.load(fh).get(f"{args.workload}:{dom}")
        if rec_t:
            traffic = rec_t.get("hbm_bytes_per_launch")
    roofline = {"bound": "mfma", "achieved": round(achieved, 1), "peak": MI355X_PEAK_INT8_TOPS,
                "unit": "TFLOP/s", "frac": round(achieved / MI355X_PEAK_INT8_TOPS, 4), "traffic": traffic,
                "kernel": f"gemm_i8_v3_kernel, {dom} GEMM M={T} N={n_dom} K={k_dom} (int8 ops: 2MNK = {ops:.4g})",
                "algorithmic_bytes": T * k_dom + n_dom * k_dom + 4 * T + 8 * n_dom + 4 * T * n_dom}
    total_gemm_ms = sum(sites[s]["ms_per_step"] for s in GEMM_SITES if s in sites)
    all_ops = sum(gemm_ops(s, T, d, f) for s in GEMM_SITES) * cfg.num_layers
    roofline["all_i8_gemms_frac"] = round(all_ops / (total_gemm_ms * 1e-3) / 1e12 / MI355X_PEAK_INT8_TOPS, 4)
    if "attention" in sites:
        # Attention: 4 * sum(L^2) * H * dh FLOP (QK^T + PV) against the bf16/fp16
        # dense peak; each split-fp16 product costs three MFMAs, so the matrix
        # cores execute 3x these FLOP.
        H, dh = cfg.num_heads, cfg.head_dim
        flop = 4.0 * float(np.sum(batch.lengths.astype(np.float64) ** 2)) * H * dh
        bytes_min = T * H * dh * (3 * 4 + 4)
        t = sites["attention"]["avg_us"] * 1e-6
        roofline["attention"] = {"flop": flop, "tflops": round(flop / t / 1e12, 1),
                                 "frac_of_2500": round(flop / t / 1e12 / 2500.0, 4),
                                 "min_bytes": bytes_min, "gbs": round(bytes_min / t / 1e9, 1),
                                 "frac_of_hbm": round(bytes_min / t / 1e9 / MI355X_PEAK_HBM_GBS, 4)}

    residues = batch.residues
    value = residues / (ms_plain * 1e-3)
    cpu = parity = None
    if not args.no_cpu_baseline and rank == 0:
        cpu, parity = cpu_baseline(weights, batch, model, args)
    model.free()
    dev.close()
    rec = {
        "metric": "residues/sec, ESM-2-650M W8A8 varlen packed fwd, 1 MI355X; %MFMA/HBM peak",
        "value": round(value, 1),
        "unit": "residues/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_plain, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (random-init ESM-2-650M weights with SmoothQuant folding, synthetic residues)",
        "config": {"workload": f"config4 {args.workload}: ESM-2-650M W8A8 packed forward, "
                               f"{len(batch.lengths)} sequences",
                   "tokens": T, "residues": residues, "sequences": int(len(batch.lengths)),
                   "act_quant": "per-token" if mode == eg.ACT_PER_TOKEN else "per-tensor",
                   "attention": "split-fp16 (hi+lo, 3 MFMAs per product) fp32-accurate MFMA", "parallelism": "single GPU",
                   "streams": args.parts},
        "tokens_per_s": round(T / (ms_plain * 1e-3), 1),
        "ms_per_step_with_kernel_events": round(ms_events, 3),
        "kernel_sites": sites,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "parity": parity,
    }
    if cpu:
        rec["gpu_over_cpu"] = round(value / cpu["value"], 1)
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
