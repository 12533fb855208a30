#!/usr/bin/env python3
"""Headline benchmark: ESM-2 650M Q8_0 batched bidirectional forward,
B=16 sequences of L=512 tokens (BOS + 510 residues + EOS) on one MI355X.

One step = one cih_forward over the batch with tokens already resident in
HBM and logits written to HBM (device-pointer I/O).  Weights are seeded
N(0, 0.02) (biases 0, LayerNorm gamma 1 / beta 0), quantized to Q8_0 in-tree;
tokens are uniform over the 20 standard amino acids.

Prints one JSON line: residues/s, the roofline of the dominant kernel (the
Q8_0 dequantizing GEMMs, timed with HIP events on the library's stream over
a second pass of the same steps) and the CPU baseline (the oracle restatement
of the reference's multithreaded CPU path, timed on a bounded sample on this
host).
"""
import argparse
import ctypes
import json
import os
import re
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "codon-infer_amd"))
from codon_hip.devmem import Hip  # noqa: E402

METRIC = "residues/sec ESM-2 650M Q8_0 B=16 L=512; HBM GB/s & MFMA util vs peak"
PEAK_FP32_MFMA_TFLOPS = 157.3   # MI355X dense FP32 matrix peak
PEAK_BF16_MFMA_TFLOPS = 2500.0  # MI355X dense bf16 matrix peak
PEAK_HBM_GBS = 8000.0
TIMING = "HIP event pair around every launch on the library stream, over an instrumented second pass of the same steps"
GEMV_MAX_TOKENS = 8             # batches of at most this many tokens use the weight-streaming GEMV
PEAK_F16_MFMA_TFLOPS = 2500.0   # MI355X dense f16 matrix peak
# What the forward computes in: every GEMM input (activations, the exact
# integer quants, FP32 weights of the LM head as a pair copy) enters the
# MFMA units as f16 limbs, products are exact and accumulate in FP32;
# LayerNorm, softmax, GELU, residual stream and block scaling are FP32.
DTYPE = "f16x2/f32acc"
DTYPE_NOTE = ("GEMM activations as two f16 limbs (hi = f16(x), lo = f16(x - hi): ~22 significant bits) times exact "
              "integer quants in f16, FP32 accumulate and FP32 block scales; FP32 weights (LM head; the 8M FP32 "
              "model) as a 22-bit f16 pair copy; attention Q/K/V/P as f16 limb pairs (hi*hi + hi*lo + lo*hi), FP32 "
              "softmax; LayerNorm, GELU, residual stream FP32")
# The default quantized GEMM issues 2 f16 MFMA MACs per algorithmic MAC
# (activation split into two f16 limbs); CIH_LIMBS=bf16x3 issues 3 bf16 MACs,
# CIH_QGEMM=fp32 selects the FP32-MFMA kernel (1 MAC per MAC).


def qgemm_name(wname, T, d):
    """Which quantized GEMM the forward's projections take at T tokens: the
    LDS-staged kernel from 64 tokens on while the f16 copy of the quants is
    there (its plan picks 64 x 64 tiles below about five per CU, the large
    tiles above), or, for a model loaded with CIH_GEMM_F16=0, when even the
    narrowest projection (N = d) gives a full round of 128 x 128 tiles; else
    the register-staged one (split-K for small T)."""
    env = os.environ.get
    copy = env("CIH_GEMM_F16") != "0"
    if env("CIH_GEMM_LDS") == "0":
        lds = False
    elif env("CIH_GEMM_LDS") == "force":
        lds = True
    elif copy and env("CIH_GEMM_PLAN") != "0":
        lds = T >= 64
    else:
        lds = -(-T // 128) * -(-d // 128) >= 256
    if lds:
        src = "f16 copy of the quants" if copy else "quants"
        return f"k_gemm_lds<{wname}> f16 MFMA, 2 limbs, operands global->LDS, W from the {src} (QKV, Wo, FC1, FC2)"
    return f"k_gemm_x3<{wname}> f16 MFMA, 2 limbs (QKV, Wo, FC1, FC2)"


def measured_traffic(name):
    """HBM bytes per launch of the dominant kernel for this workload, from the
    committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary (copy-calibrated)."""
    path = os.path.join(REPO, "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                m = re.match(r"traffic_per_launch_bytes = ([0-9.eE+-]+)", line.strip())
                if m:
                    return float(m.group(1)), "profiles/" + name
    except OSError:
        pass
    return None, None


def copy_probe(hip, mb):
    """One device-to-device copy of mb MiB: the known-size transfer the
    FETCH_SIZE / WRITE_SIZE counters are calibrated against."""
    nbytes = mb << 20
    src, dst = hip.malloc(nbytes), hip.malloc(nbytes)
    hip.L.hipMemcpy(ctypes.c_void_p(dst), ctypes.c_void_p(src), nbytes, 3)
    hip.sync()
    hip.free(src)
    hip.free(dst)


def kernel_overrides():
    """CIH_* switches that change which kernels run (graph replay switches
    only change how the same kernels are launched)."""
    return any(k.startswith("CIH_") and k not in ("CIH_FORWARD_GRAPH", "CIH_DECODE_GRAPH") for k in os.environ)


def physical_cores():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("cpu cores"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return os.cpu_count() or 1


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(cfg, w, tokens, budget_s, contacts=None):
    """The oracle (the reference's CPU algorithm: row-partitioned 4-token FMA
    GEMMs on a thread pool, serial attention) on sequences of the same
    workload, with the reference's benchmark protocol: one untimed warm-up
    forward, then up to five timed forwards, one sequence each
    (examples/bench_metrics.rs:163-177), residues/s = residues of one
    sequence / the median forward time.  Fewer than five timed forwards are
    run when the warm-up shows five would exceed budget_s (stated in the
    sample string).  A sequence whose single forward would far exceed the
    budget (3B at L=2048) is cut to its first 256 tokens + EOS, which the
    sample string also states.  With contacts the oracle computes them as
    the reference does, from each head's map in turn (no map export)."""
    import statistics
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import cpu_ref as cr

    threads = max(1, min(16, physical_cores(), os.cpu_count() or 1))
    # ~ 2 * 12 d^2 flops per token at ~0.15 TFLOP/s on 16 host cores
    est = 24.0 * cfg.dim * cfg.dim * cfg.n_layers * len(tokens[0]) / 1.5e11
    cut = est > budget_s

    def seq(i):
        t = tokens[i % len(tokens)]
        return np.concatenate([t[:256], [2]]).astype(np.int32) if cut else t

    def run(t):
        t0 = time.perf_counter()
        cr.forward(cfg, w, t, threads, contacts=contacts, final_att=False, hidden=False)
        return time.perf_counter() - t0

    warm = run(seq(0))
    n = max(1, min(5, round(budget_s / max(warm, 1e-9))))
    times, res = [], []
    for i in range(n):
        t = seq(i + 1)
        times.append(run(t))
        res.append(len(t) - 2)
    med = statistics.median(times)
    rate = statistics.median([r / x for r, x in zip(res, times)])
    what = f"first 256 residues of each sequence" if cut else f"whole sequences of L={len(tokens[0])}"
    return {"value": rate, "unit": "residues/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "host_cpus": os.cpu_count(),
            "protocol": f"1 warm-up + median of {n} (reference: 1 + median of 5)",
            "median_forward_s": round(med, 3), "forward_s": [round(x, 3) for x in times],
            "sample": f"{what} of the same workload, one per forward, {threads} threads: one warm-up forward "
                      f"({warm:.1f} s) then {n} timed forwards, residues/s of the median "
                      f"(threads = min(16, physical cores): 16 is the CPU share one GPU's job gets on this host)"}


def load_bench(args, ch):
    """Model load: a CODQ file of --model / --dtype (seeded weights) written to
    the temp directory, then cih_model_create_from_file timed (median of
    --steps, page cache warm), i.e. file -> device-resident model.  With
    --dtype fp32 the FP32 file is also loaded with quantize_to = Q8_0."""
    import statistics
    import tempfile
    cfg = ch.EsmConfig.by_name(args.model)
    seeds = {"8M": 8, "35M": 35, "150M": 150, "650M": 650, "3B": 3000}
    w = ch.EsmWeights.random(cfg, seed=seeds[args.model], bias_std=0.02)
    w = w.quantize_q8() if args.dtype == "q8" else (w.quantize_q4() if args.dtype == "q4" else w)
    path = os.path.join(tempfile.gettempdir(), f"bench_{args.model}_{args.dtype}.codq")
    ch.save_codq(path, cfg, w)
    size = os.path.getsize(path)
    lib = ch._lib.lib()

    def timed(quantize_to):
        ts = []
        for i in range(args.warmup + args.steps):
            h = ctypes.c_void_p()
            t0 = time.perf_counter()
            ch._lib.check(lib.cih_model_create_from_file(path.encode(), quantize_to, None, 0.0, ctypes.byref(h)))
            dt = time.perf_counter() - t0
            lib.cih_model_destroy(h)
            if i >= args.warmup:
                ts.append(dt)
        return statistics.median(ts)

    t = timed(-1)
    line = {"metric": f"model load ms, ESM-2 {args.model} {args.dtype} CODQ file -> device", "value": round(t * 1e3, 1),
            "unit": "ms", "higher_is_better": False, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "file_bytes": size, "GB_per_s": round(size / t / 1e9, 2)}
    if args.dtype == "fp32":
        line["quantize_to_q8_ms"] = round(timed(1) * 1e3, 1)
    os.remove(path)
    print(json.dumps(line), flush=True)


def decode_bench(args, ch):
    """Autoregressive decoding (forward_q8 / forward_q4 with the KV cache,
    lib.rs:3741-4233) of --streams independent sequences: each gets a
    16-token prompt (prefilled in one call), then every step feeds one token
    per stream at its next position — the greedy choice among the ids
    sample() allows, <eos> excluded so every step does the same work.
    --warmup untimed steps, then --new-tokens timed steps; value = generated
    tokens per second over all streams (steps replay a captured graph); a
    second, instrumented pass of up to 64 steps gives the kernel breakdown."""
    cfg = ch.EsmConfig.by_name(args.model)
    seeds = {"8M": 8, "35M": 35, "150M": 150, "650M": 650, "3B": 3000}
    t0 = time.perf_counter()
    w = ch.EsmWeights.random(cfg, seed=seeds[args.model], bias_std=0.02)
    w = w.quantize_q8() if args.dtype == "q8" else (w.quantize_q4() if args.dtype == "q4" else w)
    n, P, K = args.streams, 16, args.new_tokens
    model = ch.GpuModel(cfg, w, max_batch=1, max_len=16)
    if args.copy_probe_mb:
        copy_probe(Hip(), args.copy_probe_mb)
    dec = ch.GpuDecoder(model, n_slots=n, max_len=cfg.max_seq_len, max_rows=max(16, n))
    assert P + args.warmup + K <= cfg.max_seq_len
    rng = np.random.default_rng(7)
    allowed = np.arange(4, 24)
    last = []
    for s in range(n):
        pr = np.concatenate([[0], 4 + rng.integers(0, 20, P - 1)]).astype(np.int32)
        last.append(dec.decode(np.full(P, s), pr, np.arange(P))[-1])
    print(f"[bench] decode model + prefill ready ({time.perf_counter() - t0:.1f} s)", file=sys.stderr, flush=True)
    slots = np.arange(n, dtype=np.int32)
    state = {"pos": P, "logits": np.stack(last)}

    def step():
        toks = allowed[np.argmax(state["logits"][:, allowed], axis=1)].astype(np.int32)
        state["logits"] = dec.decode(slots, toks, np.full(n, state["pos"], np.int32))
        state["pos"] += 1

    for _ in range(args.warmup):
        step()
    t1 = time.perf_counter()
    for _ in range(K):
        step()
    el = time.perf_counter() - t1
    # instrumented pass (kernel by kernel, an event pair per launch) at the
    # same positions for the breakdown and the roofline
    K2 = min(K, 64)
    state["pos"] -= K2
    model.profile(True)
    t2 = time.perf_counter()
    for _ in range(K2):
        step()
    el_instr = time.perf_counter() - t2
    model.profile(False)
    K_prof = K2
    q = model.profile_read(ch.KC_GEMM_QUANT if args.dtype != "fp32" else ch.KC_GEMM_FP32)
    a = model.profile_read(ch.KC_ATTENTION)
    o = model.profile_read(ch.KC_OTHER)
    f = model.profile_read(ch.KC_GEMM_FP32) if args.dtype != "fp32" else {"total_ms": 0.0, "bytes": 0.0}
    gbs = q["bytes"] / (q["total_ms"] * 1e-3) / 1e9 if q["total_ms"] > 0 else 0.0
    step_bytes = (q["bytes"] + a["bytes"] + o["bytes"] + f["bytes"]) / K_prof
    traffic, traffic_src = (None, None)
    if not kernel_overrides() and (args.model, args.dtype, n) == ("650M", "q4", 1):
        traffic, traffic_src = measured_traffic("gemv_decode_q4_650m.md")
    ms = el * 1e3 / K
    line = {
        "metric": f"decode tokens/s ESM-2 {args.model} {args.dtype} ({n} stream{'s' if n > 1 else ''})",
        "value": round(n * K / el, 1), "unit": "tokens/s",
        "n_gpus": 1, "steps": K, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "ms_per_step_instrumented": round(el_instr * 1e3 / K_prof, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": DTYPE if args.dtype != "fp32" else "f32", "data": "synthetic",
        "config": {"workload": f"ESM-2 {args.model} {args.dtype} autoregressive decode, {n} stream(s), 16-token "
                               f"prompts, positions {P + args.warmup}..{P + args.warmup + K - 1}, seeded weights",
                   "streams": n, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": ("k_gemv16 split-K GEMV on f16 MFMA" if args.dtype != "fp32" and n <= 8
                                                and os.environ.get("CIH_GEMV16") != "0" else "k_gemv")
                                               + " (weights streamed once per step for all streams)",
                     "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic, "traffic_source": traffic_src,
                     "timing": TIMING},
        "step_breakdown_ms": {"gemv": round(q["total_ms"] / K_prof, 4),
                              "attention": round(a["total_ms"] / K_prof, 4),
                              "other": round(o["total_ms"] / K_prof, 4),
                              "lm_head_fp32": round(f["total_ms"] / K_prof, 4)},
        "step_bytes": round(step_bytes), "step_GB_per_s": round(step_bytes / (ms * 1e-3) / 1e9, 1),
    }
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(REPO, "oracle"))
        import cpu_ref as cr
        threads = max(1, min(16, physical_cores(), os.cpu_count() or 1))
        rs = cr.RunState(cfg, w, max_len=cfg.max_seq_len, num_threads=threads)
        done, tc = 0, time.perf_counter()
        while time.perf_counter() - tc < args.cpu_budget and done < P + K:
            rs.step(4 + done % 20, done)
            done += 1
        ec = time.perf_counter() - tc
        line["cpu_baseline"] = {"value": done / ec, "unit": "tokens/s", "cores": threads, "kind": "port",
                                "sample": f"{done} one-token steps of one stream (positions 0..{done - 1}), "
                                          f"{threads} threads, {ec:.1f} s"}
    dec.close()
    model.close()
    print(json.dumps(line), flush=True)


def dms_bench(args, ch):
    """ESM-2 650M Q8_0 in-silico DMS: a seeded 400-residue protein, every
    position masked in turn (400 copies of L=402) in chunks of 32, scored on
    the GPU (canonical log-softmax, entropy, 19 deltas per position).  One
    step = one full scan; value = mutations (positions x 20) per second."""
    n, chunk = 400, 32
    cfg = ch.EsmConfig.esm2_650m()
    t0 = time.perf_counter()
    w = ch.EsmWeights.random(cfg, seed=650, bias_std=0.0).quantize_q8()
    rng = np.random.default_rng(400)
    res = (4 + rng.integers(0, 20, n)).astype(np.int32)
    model = ch.GpuModel(cfg, w, max_batch=chunk, max_len=n + 2, outputs=ch.OUT_LOGITS)
    print(f"[bench] dms model ready ({time.perf_counter() - t0:.1f} s)", file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        model.dms(res, 0, 0, ch.DMS_MASKED_MARGINAL, chunk)
    t1 = time.perf_counter()
    for _ in range(args.steps):
        model.dms(res, 0, 0, ch.DMS_MASKED_MARGINAL, chunk)
    el = time.perf_counter() - t1
    model.profile(True)
    t2 = time.perf_counter()
    for _ in range(args.steps):
        model.dms(res, 0, 0, ch.DMS_MASKED_MARGINAL, chunk)
    el_instr = time.perf_counter() - t2
    model.profile(False)
    q = model.profile_read(ch.KC_GEMM_QUANT)
    achieved = q["flops"] / (q["total_ms"] * 1e-3) / 1e12 if q["total_ms"] > 0 else 0.0
    mut = n * 20
    line = {
        "metric": "mutations/s ESM-2 650M Q8_0 in-silico DMS (masked marginal), 400 residues",
        "value": round(mut * args.steps / el, 1),
        "unit": "mutations/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(el * 1e3 / args.steps, 3),
        "ms_per_step_instrumented": round(el_instr * 1e3 / args.steps, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": DTYPE, "dtype_note": DTYPE_NOTE,
        "data": "synthetic",
        "config": {"workload": f"ESM-2 650M Q8_0 DMS: seeded {n}-residue protein, {n} masked copies of L={n + 2} "
                               f"in chunks of {chunk}, scored on the GPU",
                   "residues_per_step": n * n, "forwards_per_step": (n + chunk - 1) // chunk,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": qgemm_name("Q8_0", chunk * (n + 2), cfg.dim),
                     "achieved": round(achieved, 2), "peak": PEAK_F16_MFMA_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_F16_MFMA_TFLOPS, 4), "traffic": None, "timing": TIMING},
    }
    if not args.no_cpu_baseline:
        sys.path.insert(0, os.path.join(REPO, "oracle"))
        import cpu_ref as cr
        threads = max(1, min(16, physical_cores(), os.cpu_count() or 1))
        done, tc = 0, time.perf_counter()
        while time.perf_counter() - tc < args.cpu_budget and done < n:
            toks = np.concatenate([[0], res, [2]]).astype(np.int32)
            wt = int(toks[done + 1])
            toks[done + 1] = 32
            logits = cr.forward(cfg, w, toks, threads, final_att=False, hidden=False)["logits"]
            cr.dms_score(logits[done + 1], wt)
            done += 1
        ec = time.perf_counter() - tc
        line["cpu_baseline"] = {"value": done * 20 / ec, "unit": "mutations/s", "cores": threads, "kind": "port",
                                "sample": f"{done} masked position(s) of the same scan, one forward each, "
                                          f"{threads} threads, {ec:.1f} s"}
    model.close()
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--seq-len", type=int, default=512,
                    help="tokens per sequence; --batch 1 --seq-len 8 or less measures the weight-streaming GEMV")
    ap.add_argument("--cpu-budget", type=float, default=25.0,
                    help="seconds of CPU baseline work (the timed forwards after the warm-up)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--model", choices=["8M", "35M", "150M", "650M", "3B"], default="650M")
    ap.add_argument("--dtype", choices=["fp32", "q8", "q4"], default="q8")
    ap.add_argument("--ragged", type=int, nargs=2, metavar=("LO", "HI"),
                    help="residues per sequence uniform in [LO, HI] (padded to --seq-len)")
    ap.add_argument("--outputs", choices=["logits+final_att", "logits", "contacts", "maps", "maps+contacts"],
                    default="logits+final_att",
                    help="logits+final_att: what the reference's forward fills and the Rust drop-in requests on "
                         "every call (lib.rs:5201-5204, 5256-5261; the headline); logits: logits only; contacts: "
                         "+ contact probabilities; maps: + every layer's attention maps")
    ap.add_argument("--workload", choices=["forward", "dms", "load", "decode"], default="forward",
                    help="forward: batched forward (the headline); dms: in-silico deep mutational scan of a "
                         "400-residue protein (400 masked copies, L=402, chunks of 32); load: CODQ file -> device; "
                         "decode: autoregressive decoding with the KV cache")
    ap.add_argument("--streams", type=int, default=1, help="decode: independent sequences decoded together")
    ap.add_argument("--new-tokens", type=int, default=256, help="decode: timed steps (tokens per stream)")
    ap.add_argument("--copy-probe-mb", type=int, default=0,
                    help="issue one device-to-device copy of this many MiB first (a known-size kernel that "
                         "calibrates FETCH_SIZE / WRITE_SIZE counter runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): the ESM-2 forward is data parallel over "
              "sequences and this build runs on a single MI355X", file=sys.stderr)
        sys.exit(2)

    import codon_hip as ch

    if args.workload == "dms":
        return dms_bench(args, ch)
    if args.workload == "load":
        return load_bench(args, ch)
    if args.workload == "decode":
        return decode_bench(args, ch)
    B, S = args.batch, args.seq_len
    cfg = ch.EsmConfig.by_name(args.model)
    # the projections' kernels and traffic are the same with or without the
    # final map, so the committed traffic summaries serve both output sets
    base650 = (args.model, args.dtype, args.ragged) == ("650M", "q8", None) and args.outputs in (
        "logits", "logits+final_att")
    headline = base650 and args.outputs == "logits+final_att"
    seeds = {"8M": 8, "35M": 35, "150M": 150, "650M": 650, "3B": 3000}
    t0 = time.perf_counter()
    w = ch.EsmWeights.random(cfg, seed=seeds[args.model], bias_std=0.0)
    w = w.quantize_q8() if args.dtype == "q8" else (w.quantize_q4() if args.dtype == "q4" else w)
    print(f"[bench] weights ready in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    rng = np.random.default_rng(16)
    if args.ragged:
        lens = (rng.integers(args.ragged[0], args.ragged[1] + 1, B) + 2).astype(np.int32)
        assert lens.max() <= S, "--ragged HI + 2 must fit in --seq-len"
    else:
        lens = np.full(B, S, np.int32)
    toks = np.zeros((B, S), np.int32)
    for b in range(B):
        toks[b, 0], toks[b, lens[b] - 1] = 0, 2
        toks[b, 1:lens[b] - 1] = 4 + rng.integers(0, 20, lens[b] - 2)

    flags = ch.OUT_LOGITS
    if "final_att" in args.outputs:
        flags |= ch.OUT_FINAL_ATT
    if "contacts" in args.outputs:
        flags |= ch.OUT_CONTACTS
    if "maps" in args.outputs:
        flags |= ch.OUT_ATTN
    contact = cfg.contact_head_weights() if flags & ch.OUT_CONTACTS else None
    # reserved for host-pointer outputs too (staging buffers), so that the
    # same model also times a short host-I/O pass after the timed one
    model = ch.GpuModel(cfg, w, contact_head=contact, max_batch=B, max_len=S, outputs=flags)
    hip = Hip()
    d_tok = hip.malloc(toks.nbytes)
    d_log = hip.malloc(B * S * cfg.vocab_size * 4)
    hip.h2d(d_tok, toks)
    outs = {"logits": d_log}
    extra = []
    if flags & ch.OUT_FINAL_ATT:
        outs["final_att"] = hip.malloc(B * S * S * 4)
        extra.append(outs["final_att"])
    if flags & ch.OUT_CONTACTS:
        outs["contacts"] = hip.malloc(B * (S - 2) * (S - 2) * 4)
        extra.append(outs["contacts"])
    if flags & ch.OUT_ATTN:
        outs["attn"] = hip.malloc(B * cfg.n_layers * cfg.n_heads * S * S * 4)
        extra.append(outs["attn"])
    if args.copy_probe_mb:
        copy_probe(hip, args.copy_probe_mb)
    print(f"[bench] model resident ({time.perf_counter() - t0:.1f} s); warmup {args.warmup}", file=sys.stderr,
          flush=True)

    for _ in range(args.warmup):
        model.forward_device(d_tok, lens, S, flags, outs)
    hip.sync()
    # Timed pass: K steps as a caller runs them (no per-kernel events).
    t1 = time.perf_counter()
    for _ in range(args.steps):
        model.forward_device(d_tok, lens, S, flags, outs)
    hip.sync()
    el = time.perf_counter() - t1
    print(f"[bench] timed {args.steps} steps in {el:.3f} s", file=sys.stderr, flush=True)
    # The same steps asking for logits only (no attention probabilities of
    # the last layer, no head-mean map): reported beside the value.
    el_lo = None
    if flags & ch.OUT_FINAL_ATT:
        lo_flags = flags & ~ch.OUT_FINAL_ATT
        for _ in range(args.warmup):
            model.forward_device(d_tok, lens, S, lo_flags, outs)
        hip.sync()
        t4 = time.perf_counter()
        for _ in range(args.steps):
            model.forward_device(d_tok, lens, S, lo_flags, outs)
        hip.sync()
        el_lo = time.perf_counter() - t4
    # Instrumented pass: the same K steps with a HIP event pair around every
    # kernel on the library's stream (kernel classes, roofline).  The event
    # packets add a few microseconds per kernel boundary, so this pass is not
    # the one whose wall time is reported.
    model.profile(True)
    hip.sync()
    t2 = time.perf_counter()
    for _ in range(args.steps):
        model.forward_device(d_tok, lens, S, flags, outs)
    hip.sync()
    el_instr = time.perf_counter() - t2
    model.profile(False)

    ks = {name: model.profile_read(kc) for name, kc in
          (("gemm_q8", ch.KC_GEMM_QUANT), ("gemm_fp32", ch.KC_GEMM_FP32), ("attention", ch.KC_ATTENTION),
           ("other", ch.KC_OTHER))}
    T = int(lens.sum())
    fp32_model = args.dtype == "fp32"
    q = ks["gemm_fp32"] if fp32_model else ks["gemm_q8"]
    gemv = T <= GEMV_MAX_TOKENS and os.environ.get("CIH_GEMV") != "0"
    fp32_path = os.environ.get("CIH_QGEMM") == "fp32"
    wname = {"q8": "Q8_0", "q4": "Q4_0", "fp32": "FP32"}[args.dtype]
    if gemv:
        # weight streaming: algorithmic bytes = quantized weights + activations in/out
        achieved = q["bytes"] / (q["total_ms"] * 1e-3) / 1e9 if q["total_ms"] > 0 else 0.0
        if not fp32_model and os.environ.get("CIH_GEMV16") != "0" and not fp32_path:
            wo_in_att = cfg.dim // cfg.n_heads % 32 == 0 and os.environ.get("CIH_FEW_WO") != "0" and args.outputs in (
                "logits", "logits+final_att")
            kname = f"k_gemv16<{wname}> split-K GEMV on f16 MFMA " + (
                "(QKV, FC1, FC2; Wo inside the attention kernel"
                + (" except in the last layer, whose map is exported)" if flags & ch.OUT_FINAL_ATT else ")")
                if wo_in_att else "(QKV, Wo, FC1, FC2)")
        else:
            kname = f"k_gemv<{wname}> weight streaming (QKV, Wo, FC1, FC2)"
        peak, limbs = PEAK_HBM_GBS, None
    else:
        achieved = q["flops"] / (q["total_ms"] * 1e-3) / 1e12 if q["total_ms"] > 0 else 0.0
        env = os.environ.get
        fp32_mfma = fp32_path or (fp32_model and (env("CIH_F32_PAIR") == "0" or env("CIH_LIMBS") == "bf16x3"))
        if fp32_mfma:
            kname, peak, limbs = f"k_gemm<{wname}> FP32 MFMA (QKV, Wo, FC1, FC2, LM head)", PEAK_FP32_MFMA_TFLOPS, 1
        elif fp32_model:
            # the f16 pair copy of the FP32 weights (hi and lo halves, K doubled)
            # times the activations' two f16 limbs: 4 f16 MFMA MACs per MAC
            lds = T >= 64 and env("CIH_GEMM_LDS") != "0" and env("CIH_GEMM_PLAN") != "0" and env("CIH_ACT") != "f32"
            kname = (("k_gemm_lds" if lds else "k_gemm_x3") + "<FP32 pair copy> f16 MFMA, 2 activation limbs x "
                     "2 weight halves (QKV, Wo, FC1, FC2, LM head)")
            peak, limbs = PEAK_F16_MFMA_TFLOPS, 4
        elif env("CIH_LIMBS") == "bf16x3":
            kname, peak, limbs = f"k_gemm_x3<{wname}> bf16 MFMA, 3 limbs (QKV, Wo, FC1, FC2)", PEAK_BF16_MFMA_TFLOPS, 3
        else:
            kname, peak, limbs = qgemm_name(wname, T, cfg.dim), PEAK_F16_MFMA_TFLOPS, 2
    # traffic from the committed PMC summary, for the workloads it was measured on
    overrides = kernel_overrides()
    prof = None
    if not overrides and base650 and (B, S) == (16, 512):
        prof = "gemm_q8_650m_b16_l512.md"
    elif not overrides and base650 and (B, S) == (1, 8):
        prof = "gemv_q8_650m_b1_l8.md"
    traffic, traffic_src = measured_traffic(prof) if prof else (None, None)
    kernels = {k: {"launches": v["launches"] // max(1, args.steps),
                   "ms_per_step": v["total_ms"] / max(1, args.steps),
                   "tflops": (v["flops"] / (v["total_ms"] * 1e-3) / 1e12) if v["total_ms"] > 0 and v["flops"] else None}
               for k, v in ks.items()}
    for k, v in kernels.items():
        print(f"[bench] {k}: {v}", file=sys.stderr, flush=True)

    logits = np.empty((B, S, cfg.vocab_size), np.float32)
    hip.d2h(logits, d_log)
    assert np.isfinite(logits).all()
    # Host-pointer I/O (tokens from host memory, outputs copied back over
    # PCIe inside each call): reported beside the line, never as its value.
    # (Skipped when every layer's maps are exported: gigabytes per call.)
    seqs = [toks[b, :lens[b]] for b in range(B)]
    host_steps = 0 if flags & ch.OUT_ATTN else min(args.steps, 5)
    t3 = time.perf_counter()
    for _ in range(host_steps):
        model.forward(seqs, flags)
    el_host = time.perf_counter() - t3

    residues = int((lens - 2).sum())
    value = residues * args.steps / el
    outs_desc = {"logits+final_att": "logits + the last layer's head-mean attention map (final_layer_att)",
                 "logits": "logits", "contacts": "logits + contacts", "maps": "logits + every layer's attention maps",
                 "maps+contacts": "logits + every layer's attention maps + contacts"}[args.outputs]
    lens_desc = (f"{args.ragged[0]}-{args.ragged[1]} residues (uniform), padded to L={S}" if args.ragged
                 else f"L={S} (BOS+{S - 2}+EOS)")
    metric = METRIC if headline and (B, S) == (16, 512) else \
        f"residues/sec ESM-2 {args.model} {wname} B={B} {lens_desc}, {outs_desc}"
    line = {
        "metric": metric,
        "value": round(value, 1),
        "unit": "residues/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(el * 1e3 / args.steps, 3),
        "ms_per_step_instrumented": round(el_instr * 1e3 / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE if not fp32_path else "f32",
        "dtype_note": DTYPE_NOTE if not fp32_path else "FP32 MFMA (CIH_QGEMM=fp32)",
        "data": "synthetic",
        "config": {"workload": f"ESM-2 {args.model} {wname} bidirectional forward, B={B}, {lens_desc}, "
                               f"seeded N(0,0.02) weights{' quantized in-tree' if args.dtype != 'fp32' else ''}, "
                               f"uniform 20-AA tokens, {outs_desc} to HBM",
                   "batch": B, "seq_len": S, "residues_per_step": residues, "parallelism": "single GPU",
                   "io": "tokens read from and outputs written to HBM (CIH_IO_DEVICE): the timed region holds "
                         "no host transfer"},
        "logits_only": ({"value": round(residues * args.steps / el_lo, 1), "unit": "residues/s",
                         "ms_per_step": round(el_lo * 1e3 / args.steps, 3),
                         "note": "the same steps without OUT_FINAL_ATT"} if el_lo else None),
        "host_io": ({"value": round(residues * host_steps / el_host, 1), "unit": "residues/s",
                     "ms_per_step": round(el_host * 1e3 / host_steps, 3), "steps": host_steps,
                     "note": "host-pointer tokens and outputs, PCIe copies inside each call"} if host_steps else None),
        "roofline": ({"bound": "hbm", "kernel": kname,
                      "achieved": round(achieved, 1), "peak": peak, "unit": "GB/s",
                      "frac": round(achieved / peak, 4),
                      "traffic": traffic, "traffic_source": traffic_src, "timing": TIMING} if gemv else
                     {"bound": "mfma", "kernel": kname,
                      "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
                      "frac": round(achieved / peak, 4),
                      "traffic": traffic, "traffic_source": traffic_src,
                      "mfma_macs_per_mac": limbs,
                      "issued_frac": round(achieved * limbs / peak, 4), "timing": TIMING}),
        "kernels": kernels,
    }
    if not args.no_cpu_baseline:
        print("[bench] CPU baseline (oracle) ...", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_baseline(cfg, w, [toks[b, :lens[b]] for b in range(B)], args.cpu_budget,
                                            contact if "contacts" in args.outputs else None)
    model.close()
    hip.free(d_tok)
    hip.free(d_log)
    for p in extra:
        hip.free(p)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
