#!/usr/bin/env python3
"""Benchmark: residues/s of the ESM-2-650M W8A8 varlen packed forward on one
MI355X (varlen 256-sequence batch).

A step is one packed forward (embed, 33 encoder layers, final LN, lm head)
over the whole synthetic batch, with the batch already staged in HBM
(esm_gfx950_batch_upload before the timed region) and the logits left in
HBM. W warmup steps, then K timed steps bracketed by device syncs and HIP
events on the context stream. A second pass brackets every INT8 GEMM and
attention launch with HIP events on the stream it runs on, which gives the
dominant kernel's average launch duration for the roofline line.

Extra records (same JSON line, "workloads"): config 4's uniform 8x256 batch
and config 5 (ESM-2 3B, 36 layers, 64 sequences of log-uniform 50..1024
tokens), each with residues/s and its dominant GEMM's roofline; the headline
batch with the reference's per-tensor activation scales (default numerics).

A further record times the x86-exact numerics (ESM_GFX950_NUMERICS_X86_AVX512,
or _X86_AMX on an AMX host) on the headline batch: the mode whose logits
equal the reference CPU path's bit for bit.

cpu_baseline: the reference's own CPU path (its kernels compiled from source
into oracle/_ref/libesmref.so, driven in ForwardPackedInto order) on the
identical packed batch (all 256 sequences by default), timed on this host
with the reference's protocol (python/esm_cpp/bench/compare.py:172-191:
warmup runs, then timed runs, p50 and mean; 1 + 3 by default instead of
compare.py's 2 + 5, which would hold the GPU box two minutes for the CPU
alone), both ForwardPacked and ForwardScheduled (PlanBatches groups).

parity: on that batch, the GPU in x86-exact numerics against the CPU run
(bit for bit), the GPU's per-tensor mode against it; and on the committed
33-layer fixture (tests/golden/full_depth_650m.npz) the GPU's default modes
against the oracle and the reference, next to the reference's own spread.

--act-mode tensor times the headline batch with per-tensor activation
scales, --numerics x86_avx512 / x86_amx in the x86-exact numerics (per-tensor
scales): the records the profiles of those modes come from.

Prints one JSON line. --gpus N > 1 exits: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
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
ROW_SITES = ("ln_quant", "ln_quant_first", "attn_quant", "gelu_quant")
FIXTURE = os.path.join(ROOT, "tests", "golden", "full_depth_650m.npz")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gemm_shape(site, cfg):
    d, f = cfg.hidden_size, cfg.intermediate_size
    return {"qkv": (3 * d, d), "out": (d, d), "fc1": (f, d), "fc2": (d, f)}[site]


def gemm_ops(site, T, cfg):
    n, k = gemm_shape(site, cfg)
    return 2.0 * T * n * k


def corr(a, b):
    return float(np.corrcoef(a.ravel().astype(np.float64), b.ravel().astype(np.float64))[0, 1])


def measure(dev, model, batch, cfg, steps, warmup, parts):
    """(ms per step with `parts` groups (0: the library's automatic count),
    per-step ms with per-kernel events and one group, per-site kernel times,
    groups the throughput pass used)."""
    T = batch.total_tokens
    logits = dev.empty((T, cfg.vocab_size), np.float32)
    model.set_parts(parts)
    model.upload_batch(batch.ids, batch.cu)
    used = model.staged_parts()
    for _ in range(warmup):
        model.forward_device(logits)
    dev.sync()
    dev.timer_start()
    for _ in range(steps):
        model.forward_device(logits)
    ms = dev.timer_stop() / steps
    if used != 1:
        model.set_parts(1)
        model.upload_batch(batch.ids, batch.cu)
        model.forward_device(logits)
    dev.kernel_timing(True)
    dev.sync()
    dev.timer_start()
    for _ in range(steps):
        model.forward_device(logits)
    ms_events = dev.timer_stop() / steps
    sites = {}
    for site in GEMM_SITES + ("attention", "lm_dense") + ROW_SITES:
        n, tot = dev.kernel_timing_query(site)
        if n:
            sites[site] = {"launches": n, "avg_us": round(tot / n * 1000, 2), "ms_per_step": round(tot / steps, 3)}
    dev.kernel_timing(False)
    out = logits.numpy()
    logits.free()
    if not np.all(np.isfinite(out)):
        raise SystemExit("bench: non-finite logits")
    return ms, ms_events, sites, used


# Bytes each GEMM moves per output value beyond its int8 operands: QKV
# writes split-fp16 hi + lo parts; out-proj and fc2 read and write hidden
# (the residual add); fc1 writes its 24-bit intermediate in per-token mode
# and fp32 GELU output per tensor.
def out_bytes(site, per_token):
    return {"qkv": 4, "out": 8, "fc1": 3 if per_token else 4, "fc2": 8}[site]


def roofline_of(sites, T, cfg, batch, workload, per_token=True):
    dom = max((s for s in GEMM_SITES if s in sites), key=lambda s: sites[s]["ms_per_step"])
    ops = gemm_ops(dom, T, cfg)
    achieved = ops / (sites[dom]["avg_us"] * 1e-6) / 1e12
    n_dom, k_dom = gemm_shape(dom, cfg)
    # HBM bytes per launch of the dominant kernel, measured with rocprofv3
    # FETCH_SIZE / WRITE_SIZE passes scaled by a copy-kernel calibration (the
    # profiles/ summaries); null when no measurement is recorded.
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as fh:
            rec_t = json.load(fh).get(f"{workload}:{dom}")
        if rec_t:
            traffic = rec_t.get("hbm_bytes_per_launch")
    r = {"bound": "mfma", "achieved": round(achieved, 1), "peak": MI355X_PEAK_INT8_TOPS, "unit": "TFLOP/s",
         "frac": round(achieved / MI355X_PEAK_INT8_TOPS, 4), "traffic": traffic,
         "kernel": f"gemm_i8_v3_kernel, {dom} GEMM M={T} N={n_dom} K={k_dom} (int8 ops: 2MNK = {ops:.4g})",
         "algorithmic_bytes": T * k_dom + n_dom * k_dom + 4 * T + 8 * n_dom + out_bytes(dom, per_token) * T * n_dom}
    total_gemm_ms = sum(sites[s]["ms_per_step"] for s in GEMM_SITES if s in sites)
    all_ops = sum(gemm_ops(s, T, cfg) for s in GEMM_SITES) * cfg.num_layers
    r["all_i8_gemms_frac"] = round(all_ops / (total_gemm_ms * 1e-3) / 1e12 / MI355X_PEAK_INT8_TOPS, 4)
    if "attention" in sites:
        # 4 * sum(L^2) * H * dh FLOP (QK^T + PV) against the fp16 dense peak;
        # each split-fp16 product costs three MFMAs, so the matrix cores run
        # 3x these FLOP. Minimum bytes: split-fp16 Q, K, V words in, fp32 out.
        H, dh = cfg.num_heads, cfg.head_dim
        flop = 4.0 * float(np.sum(batch.lengths.astype(np.float64) ** 2)) * H * dh
        bytes_min = T * H * dh * (3 * 4 + 4)
        t = sites["attention"]["avg_us"] * 1e-6
        r["attention"] = {"flop": flop, "tflops": round(flop / t / 1e12, 1),
                          "frac_of_2500": round(flop / t / 1e12 / 2500.0, 4), "min_bytes": bytes_min,
                          "gbs": round(bytes_min / t / 1e9, 1),
                          "frac_of_hbm": round(bytes_min / t / 1e9 / MI355X_PEAK_HBM_GBS, 4)}
    # HBM-bound row kernels (per-token mode): algorithmic bytes per launch
    # over the event-timed duration, against the 8 TB/s peak. RoPE has no
    # kernel of its own: it runs in the QKV GEMM's epilogue.
    d, f = cfg.hidden_size, cfg.intermediate_size
    row_bytes = {
        "ln_quant": T * d * (4 + 1) + 4 * T,           # hidden in, int8 out, scales (residual added by the GEMM)
        "ln_quant_first": T * d * (4 + 1) + 4 * T,     # hidden in, int8 out, scales
        "attn_quant": T * d * (4 + 1) + 4 * T,         # fp32 in, int8 out, scales
        "gelu_quant": T * f * (3 + 1) + 4 * T,         # fc1's 24-bit values in, int8 out, scales
    }
    rows = {}
    for site, b in row_bytes.items():
        if site in sites:
            t = sites[site]["avg_us"] * 1e-6
            rows[site] = {"bytes_per_launch": b, "avg_us": sites[site]["avg_us"], "gbs": round(b / t / 1e9, 1),
                          "frac_of_hbm": round(b / t / 1e9 / MI355X_PEAK_HBM_GBS, 4)}
    if rows:
        rows["rope"] = "fused into the QKV GEMM epilogue (no separate pass)"
        r["row_kernels"] = rows
    return r


def x86_workload(dev, weights, batch, cfg, isa, args):
    """The x86-exact numerics (logits equal to the reference CPU path's on an
    `isa` host) on the headline batch: residues/s and per-site kernel times."""
    numerics = eg.NUMERICS_X86_AMX if isa == "amx" else eg.NUMERICS_X86_AVX512
    model = eg.Model(dev, weights, int8=True, act_mode=eg.ACT_PER_TENSOR)
    try:
        model.set_numerics(numerics)
        ms, _, sites, used = measure(dev, model, batch, cfg, args.extra_steps, 1, 1)
    finally:
        model.free()
    T = batch.total_tokens
    return {"workload": f"x86-exact: config4 varlen, ESM-2-650M W8A8, numerics "
                        f"{'X86_AMX' if numerics == eg.NUMERICS_X86_AMX else 'X86_AVX512'} (per-tensor activation "
                        f"scales; logits equal the reference's {isa} CPU forward bit for bit)",
            "tokens": T, "residues": batch.residues, "sequences": int(len(batch.lengths)),
            "ms_per_step": round(ms, 3), "value": round(batch.residues / (ms * 1e-3), 1), "unit": "residues/s",
            "tokens_per_s": round(T / (ms * 1e-3), 1), "streams": used, "kernel_sites": sites}


def extra_workload(dev, name, cfg, weights, batch, args, act_mode=eg.ACT_PER_TOKEN):
    model = eg.Model(dev, weights, int8=True, act_mode=act_mode)
    try:
        ms, _, sites, used = measure(dev, model, batch, cfg, args.extra_steps, 2, args.parts)
    finally:
        model.free()
    T = batch.total_tokens
    return {"workload": name, "tokens": T, "residues": batch.residues, "sequences": int(len(batch.lengths)),
            "ms_per_step": round(ms, 3), "value": round(batch.residues / (ms * 1e-3), 1), "unit": "residues/s",
            "tokens_per_s": round(T / (ms * 1e-3), 1), "streams": used, "kernel_sites": sites,
            "roofline": roofline_of(sites, T, cfg, batch, name.split(":")[0],
                                    per_token=act_mode == eg.ACT_PER_TOKEN)}


def host_cpu():
    info = {"hardware_concurrency": os.cpu_count()}
    try:
        info["affinity_cpus"] = len(os.sched_getaffinity(0))
    except AttributeError:
        pass
    try:
        cores, model = set(), None
        phys = core = None
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and model is None:
                    model = v
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    core = v
                elif not k and phys is not None:
                    cores.add((phys, core))
                    phys = core = None
        if phys is not None:
            cores.add((phys, core))
        info["model"] = model
        info["physical_cores"] = len(cores) or None
        info["sockets"] = len({p for p, _ in cores}) or None
    except OSError:
        pass
    return info


def p50(xs):
    return float(statistics.median(xs))


def cpu_baseline(weights, batch, dev, args):
    """The reference CPU path on a sample: ForwardPacked and ForwardScheduled
    timed as compare.py does; returns (record, sample, cpu logits, isa)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from pyoracle import REF_LIB, RefLib, RefModel

    if not os.path.exists(REF_LIB):
        return None, None, None, None
    cpu = host_cpu()
    threads = max(1, min(cpu.get("affinity_cpus") or cpu["hardware_concurrency"] or 1, args.cpu_threads))
    ref = RefLib(threads=threads)
    nseq = len(batch.lengths) if args.cpu_seqs <= 0 else min(args.cpu_seqs, len(batch.lengths))
    idx = list(range(0, len(batch.lengths), max(1, len(batch.lengths) // nseq)))[:nseq]
    sample = batch if nseq == len(batch.lengths) else batch.subset(idx)
    rm = RefModel(ref, weights, int8=True)
    isa = ref.isa()
    log(f"cpu: isa={isa} threads={threads} host={cpu}")

    def timed(fn):
        for _ in range(args.cpu_warmup):
            fn()
        ts = []
        for _ in range(args.cpu_iters):
            t = time.perf_counter()
            out = fn()
            ts.append(time.perf_counter() - t)
        return ts, out

    packed_t, logits = timed(lambda: rm.forward_packed(sample))
    groups = ref.plan_batches(sample.lengths, 256, 1.2)
    subsets = [sample.subset(g) for g in groups]
    sched_t, _ = timed(lambda: [rm.forward_packed(s) for s in subsets])
    rm.free()
    best = min(p50(packed_t), p50(sched_t))
    rec = {
        "value": round(sample.residues / best, 1),
        "unit": "residues/s",
        "cores": threads,
        "kind": "reference",
        "sample": (f"{len(idx)} of {len(batch.lengths)} sequences ({sample.residues} residues, "
                   f"{sample.total_tokens} tokens); {args.cpu_warmup} warmup + {args.cpu_iters} timed runs each of "
                   f"ForwardPacked and ForwardScheduled ({len(groups)} PlanBatches groups); value = the faster p50; "
                   f"reference kernels isa={isa}, {threads} threads (ESM_NUM_THREADS; the GPU box grants one "
                   f"GPU's job 16 CPUs)"),
        "isa": isa,
        "threads": threads,
        "host": cpu,
        "forward_packed_ms": {"p50": round(p50(packed_t) * 1e3, 1), "mean": round(statistics.mean(packed_t) * 1e3, 1)},
        "forward_scheduled_ms": {"p50": round(p50(sched_t) * 1e3, 1),
                                 "mean": round(statistics.mean(sched_t) * 1e3, 1), "groups": len(groups)},
        "finite": bool(np.all(np.isfinite(logits))),
    }
    return rec, sample, logits, isa


def parity(dev, weights, sample, cpu_logits, isa):
    """GPU against the reference CPU run on the sample, and at full depth
    against the committed fixture."""
    out = {}
    numerics = eg.NUMERICS_X86_AMX if isa == "amx" else eg.NUMERICS_X86_AVX512
    if sample is not None:
        m = eg.Model(dev, weights, int8=True, act_mode=eg.ACT_PER_TENSOR)
        g = m.forward_packed(sample.ids, sample.cu)
        out["per_tensor_vs_reference_cpu"] = {"logit_corr": round(corr(g, cpu_logits), 6),
                                              "argmax_agree": round(float(np.mean(g.argmax(1) == cpu_logits.argmax(1))), 4)}
        m.set_numerics(numerics)
        g = m.forward_packed(sample.ids, sample.cu)
        m.free()
        out[f"x86_numerics_vs_reference_cpu"] = {
            "isa": isa, "tokens": sample.total_tokens, "layers": weights.cfg.num_layers,
            "bit_exact": bool(np.array_equal(g.view(np.uint32), cpu_logits.view(np.uint32))),
            "max_abs_diff": float(np.max(np.abs(g - cpu_logits))), "logit_corr": round(corr(g, cpu_logits), 8)}
    if os.path.exists(FIXTURE):
        with np.load(FIXTURE) as z:
            fx = {k: z[k] for k in z.files}
        ids, cu = fx["ids"], fx["cu"]
        res = {"batch": f"{len(cu) - 1} sequences, {int(cu[-1])} tokens, 33 layers (tests/golden/full_depth_650m.npz)"}
        for name, mode, numerics_, key in (
                ("per_token_vs_oracle_ffn24", eg.ACT_PER_TOKEN, eg.NUMERICS_DEFAULT, "oracle_per_token_ffn24"),
                ("per_token_vs_oracle_fp32_intermediate", eg.ACT_PER_TOKEN, eg.NUMERICS_DEFAULT, "oracle_per_token"),
                ("per_tensor_vs_oracle", eg.ACT_PER_TENSOR, eg.NUMERICS_DEFAULT, "oracle_per_tensor"),
                ("per_tensor_vs_reference_avx512vnni", eg.ACT_PER_TENSOR, eg.NUMERICS_DEFAULT, "ref_avx512vnni"),
                ("x86_avx512_vs_reference_avx512vnni", eg.ACT_PER_TENSOR, eg.NUMERICS_X86_AVX512, "ref_avx512vnni"),
                ("x86_amx_vs_reference_amx", eg.ACT_PER_TENSOR, eg.NUMERICS_X86_AMX, "ref_amx")):
            if key not in fx:
                continue
            m = eg.Model(dev, weights, int8=True, act_mode=mode)
            m.set_numerics(numerics_)
            g = m.forward_packed(ids, cu)
            m.free()
            res[name] = {"logit_corr": round(corr(g, fx[key]), 6),
                         "argmax_agree": round(float(np.mean(g.argmax(1) == fx[key].argmax(1))), 4),
                         "bit_exact": bool(np.array_equal(g.view(np.uint32), fx[key].view(np.uint32)))}
        spread = {}
        for a, b in (("ref_avx512vnni", "ref_amx"), ("ref_avx512vnni", "ref_isa_ref"), ("ref_amx", "ref_isa_ref")):
            if a in fx and b in fx:
                spread[f"{a[4:]}_vs_{b[4:]}"] = round(corr(fx[a], fx[b]), 6)
        res["reference_own_spread"] = spread
        out["full_depth_33_layers"] = res
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=["varlen", "uniform"], default="varlen")
    ap.add_argument("--act-mode", choices=["token", "tensor"], default="token")
    ap.add_argument("--numerics", choices=["default", "x86_avx512", "x86_amx"], default="default",
                    help="numerics of the timed forward; the x86-exact modes take per-tensor activation scales")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the uniform and config-5 records")
    ap.add_argument("--no-parity", action="store_true")
    ap.add_argument("--extra-steps", type=int, default=5)
    ap.add_argument("--cpu-seqs", type=int, default=0, help="sequences in the CPU baseline (0: the whole batch)")
    ap.add_argument("--cpu-warmup", type=int, default=1)
    ap.add_argument("--cpu-iters", type=int, default=3)
    ap.add_argument("--no-x86", action="store_true", help="skip the x86-exact numerics record")
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--parts", type=int, default=0,
                    help="concurrent sequence groups (streams) in the throughput pass; 0 = the library's "
                         "automatic count (one group per 6e11 int8 ops of a layer's linears, 1..3)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on exactly one GPU (got --gpus {args.gpus}); the packed forward "
              "would shard whole sequences across GPUs with no exchange; only one GPU is measured here.", file=sys.stderr)
        sys.exit(2)
    rank = int(os.environ.get("RANK", "0"))

    cfg = syn.ESM2_650M
    t0 = time.time()
    weights = syn.make_weights(cfg, seed=20261201 + 4, int8=True)
    batch = syn.config4_varlen_batch() if args.workload == "varlen" else syn.config4_uniform_batch()
    log(f"weights + batch in {time.time() - t0:.1f}s: T={batch.total_tokens} residues={batch.residues}")

    dev = eg.Device(0)
    numerics = {"default": eg.NUMERICS_DEFAULT, "x86_avx512": eg.NUMERICS_X86_AVX512,
                "x86_amx": eg.NUMERICS_X86_AMX}[args.numerics]
    mode = eg.ACT_PER_TOKEN if args.act_mode == "token" and numerics == eg.NUMERICS_DEFAULT else eg.ACT_PER_TENSOR
    model = eg.Model(dev, weights, int8=True, act_mode=mode)
    if numerics != eg.NUMERICS_DEFAULT:
        model.set_numerics(numerics)
    T = batch.total_tokens
    ms_plain, ms_events, sites, used = measure(dev, model, batch, cfg, args.steps, args.warmup, args.parts)
    model.free()
    log(f"ms/step {ms_plain:.3f} (with per-kernel events {ms_events:.3f}); sites {sites}")
    roofline = roofline_of(sites, T, cfg, batch, args.workload, per_token=mode == eg.ACT_PER_TOKEN)
    value = batch.residues / (ms_plain * 1e-3)

    workloads = []
    if not args.no_extra:
        other = "uniform" if args.workload == "varlen" else "varlen"
        ob = syn.config4_uniform_batch() if other == "uniform" else syn.config4_varlen_batch()
        workloads.append(extra_workload(dev, f"{other}: config4 {other}, ESM-2-650M W8A8", cfg, weights, ob, args))
        log(f"extra {workloads[-1]['workload']}: {workloads[-1]['ms_per_step']} ms")
        c5 = syn.ESM2_3B
        w5 = syn.make_weights(c5, seed=20261201 + 5, int8=True, keep_f32_linears=False)
        workloads.append(extra_workload(dev, "config5: ESM-2-3B W8A8, 64 sequences log-uniform 50..1024", c5, w5,
                                        syn.config5_batch(), args))
        del w5
        log(f"extra {workloads[-1]['workload']}: {workloads[-1]['ms_per_step']} ms")
        if args.workload == "varlen" and mode == eg.ACT_PER_TOKEN and numerics == eg.NUMERICS_DEFAULT:
            # The reference's own activation scaling (one dynamic scale per
            # tensor), default numerics: one sequence group (the scale spans
            # the batch).
            workloads.append(extra_workload(
                dev, "per-tensor: config4 varlen, ESM-2-650M W8A8, per-tensor activation scales (the reference's "
                     "dynamic per-tensor quantisation), default numerics", cfg, weights, batch, args,
                act_mode=eg.ACT_PER_TENSOR))
            log(f"extra {workloads[-1]['workload']}: {workloads[-1]['ms_per_step']} ms")

    cpu = par = None
    sample = cpu_logits = isa = None
    if not args.no_cpu_baseline and rank == 0:
        cpu, sample, cpu_logits, isa = cpu_baseline(weights, batch, dev, args)
    if not args.no_x86 and args.workload == "varlen":
        x86 = x86_workload(dev, weights, batch, cfg, isa or "avx512vnni", args)
        if cpu and cpu["sample"].startswith(f"{len(batch.lengths)} of {len(batch.lengths)}"):
            x86["gpu_over_cpu"] = round(x86["value"] / cpu["value"], 1)
        workloads.append(x86)
        log(f"extra {x86['workload']}: {x86['ms_per_step']} ms")
    if not args.no_parity and rank == 0:
        par = parity(dev, weights, sample, cpu_logits, isa or "avx512vnni")
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
                   "tokens": T, "residues": batch.residues, "sequences": int(len(batch.lengths)),
                   "act_quant": "per-token" if mode == eg.ACT_PER_TOKEN else "per-tensor",
                   "numerics": args.numerics,
                   "attention": "split-fp16 (hi+lo, 3 MFMAs per product) fp32-accurate MFMA", "parallelism": "single GPU",
                   "streams": used},
        "tokens_per_s": round(T / (ms_plain * 1e-3), 1),
        "ms_per_step_with_kernel_events": round(ms_events, 3),
        "kernel_sites": sites,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "parity": par,
        "workloads": workloads,
    }
    if cpu:
        rec["gpu_over_cpu"] = round(value / cpu["value"], 1)
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
