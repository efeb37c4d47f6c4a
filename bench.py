"""Benchmark of the INT8 TinyLlama-1.1B decoder hot path on one MI355X.

Workload (value): greedy decode at batch 1 of a TinyLlama-1.1B-shape INT8
model (22 layers, hidden 2048, 32/4 heads, FFN 5632, vocab 32000) with
random N(0, 0.02) weights quantized per output channel: a 128-token seeded
prompt is prefilled, then --steps greedy decode steps (default 256) are timed
as they run in production (one captured HIP graph replayed per step).
One "step" is one token through 22 decoder layers, the LM head and argmax.

Also reported, on the same model in the same run:
  roofline      the dominant decode kernel (SiLU-GLU gate/up GEMV): algorithmic
                bytes per launch / its dispatch duration from HIP events on the
                library's stream (the quantity rocprofv3's kernel trace
                reports), against 8 TB/s; plus its busy time in the graph
                regime from the device timeline
  timeline      the device timeline of graph-replayed steps: per kernel class
                the busy time (first wavefront start to last wavefront end)
                and the gap to the next kernel, which add up to the step
  kernels       per decode kernel class: dispatch duration and timeline busy
                time, with algorithmic GB/s of each
  prefill       512-token prefill (22 layers + LM head + argmax): wall time and
                per-role GEMM dispatch durations at M = 512, i8 MFMA
                utilisation against 5.0 POP/s dense
  eos_watch     decode rate with an EOS id set (the host keeps three steps in
                flight and reads the device's stop flag after every step)
  cpu_baseline  the CPU oracle (tl_oracle.c) decoding the same steps from the
                same KV cache on all host threads and on one; tokens must equal
                the GPU's
  workloads     config 1 (one GEMV + requantize), config 2 (one decoder layer)
                and config 5 (32 sequences x 2048 context, 64 steps)

    python bench.py [--gpus 1] [--steps 256] [--warmup 8] [--only decode|prefill|batch]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode tok/s + decode GEMV HBM GB/s + prefill i8 MFMA %, TinyLlama-1.1B bs=1"
HBM_PEAK_GBS = 8000.0
I8_PEAK_OPS = 5.0e15
CFG = dict(hidden=2048, intermediate=5632, n_layers=22, n_heads=32, n_kv_heads=4, head_dim=64,
           vocab=32000, max_pos=2048, rms_eps=np.float32(1e-5), rope_theta=10000.0)
DECODE_CLASSES = ("qkv", "attn", "o", "glu", "down", "lm_head", "other")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def decode_kernel_bytes(cfg):
    """Algorithmic HBM bytes of one launch of each decode kernel class (each
    byte counted once: weights, their fp32 scales, activations in and out)."""
    D, F, V = cfg["hidden"], cfg["intermediate"], cfg["vocab"]
    kvd = cfg["n_kv_heads"] * cfg["head_dim"]
    qkv = D + 2 * kvd
    return {
        "qkv": qkv * D + qkv * 4 + D + 8 + qkv * 4,
        "o": D * D + D * 4 + D + 8 + D * 4 * 2,
        "glu": 2 * F * D + 2 * F * 4 + D + 8 + F * 4,
        "down": D * F + D * 4 + F + 8 + D * 4 * 2,
        "lm_head": V * D + V * 4 + D + 8,
    }


def prefill_gemm_ops(cfg, m):
    """INT8 multiply-add ops (x2) of the Q|K|V, O, gate/up and down GEMMs of
    an m-token prefill, per role and in total."""
    D, F = cfg["hidden"], cfg["intermediate"]
    kvd = cfg["n_kv_heads"] * cfg["head_dim"]
    per = {"qkv": (D + 2 * kvd) * D, "o": D * D, "glu": 2 * F * D, "down": D * F}
    return {k: 2.0 * m * v * cfg["n_layers"] for k, v in per.items()}


def host_cpu():
    model = platform.processor() or "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return model, os.cpu_count() or 1, usable


def cpu_baseline(host, eng, prompt_len, first_token, gpu_tokens, steps_all, steps_one, threads):
    """The oracle continues the same sequence from the GPU's KV cache
    (positions 0..prompt_len-1), one token per step through every layer, on
    `threads` host threads for steps_all steps and on one thread for
    steps_one steps; its tokens must equal the GPU's."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    arrays = oracle.ModelArrays(**vars(host))
    kc, vc = arrays.new_cache()
    for layer in range(CFG["n_layers"]):
        for g in range(CFG["n_kv_heads"]):
            k, v = eng.kv_read(0, layer, g, 0, prompt_len)
            kc[layer, g, :prompt_len] = k
            vc[layer, g, :prompt_len] = v
    orc = oracle.Oracle(arrays)
    want = [int(t) for t in gpu_tokens]

    def run(n_threads, n_steps, cache):
        oracle.lib().or_set_threads(n_threads)
        tok, got = first_token, []
        t0 = time.perf_counter()
        for s in range(n_steps):
            x = orc.embed(tok)
            for layer in range(CFG["n_layers"]):
                x = orc.decode_row(layer, prompt_len + s, x, *cache)
            tok, _ = orc.lm_head(x)
            got.append(tok)
        return n_steps / (time.perf_counter() - t0), got == want[:n_steps]

    rate_one, match_one = run(1, steps_one, (kc.copy(), vc.copy()))
    rate_all, match_all = run(threads, steps_all, (kc, vc))
    return rate_all, rate_one, match_all and match_one


def bench_gemv_q_proj(eng, seed, launches=200, copies=96):
    """Single INT8 GEMV + per-channel requantize, the Q-projection shape: x int8
    [2048], W int8 [2048][2048] uniform in [-127, 127], m U[1e-3, 1e-2].  The
    weights rotate over `copies` distinct buffers (384 MB) so every launch
    streams from HBM rather than the 256 MB Infinity Cache; kernel time from
    HIP events on the library's stream."""
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    n = k = 2048
    ws = [torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda", generator=g) for _ in range(copies)]
    x = torch.randint(-127, 128, (k,), dtype=torch.int8, device="cuda", generator=g)
    m = torch.rand(n, device="cuda", generator=g) * 9e-3 + 1e-3
    y = torch.empty(n, dtype=torch.int8, device="cuda")
    acc = torch.empty(n, dtype=torch.int32, device="cuda")
    for i in range(copies):
        eng.rt.call("tl_gemv_i8_requant", x, ws[i], m, n, k, y, acc)
    eng.set_profiling(True)
    for i in range(launches):
        eng.rt.call("tl_gemv_i8_requant", x, ws[i % copies], m, n, k, y, acc)
    cnt, ms, _ = eng.profile("qkv")
    eng.set_profiling(False)
    avg_us = ms * 1e3 / cnt
    nbytes = n * k + k + n * 4 + n
    gbs = nbytes / (avg_us * 1e-6) / 1e9
    return {"workload": "INT8 GEMV + requantize, x[1x2048] . W[2048x2048]^T, per-channel fp32 multipliers",
            "launches": cnt, "avg_us": round(avg_us, 3), "bytes": nbytes, "gbs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "weights_rotated_over": copies}


def bench_decode_layer(eng, calls=64):
    """One TinyLlama-shape decoder layer, one decode step at position 512 over
    the 512 rows a prefill left in the cache: the sum of its five kernels'
    average dispatch durations (HIP events)."""
    import torch
    x = torch.randn(CFG["hidden"], device="cuda")
    x0 = x.clone()
    for _ in range(4):
        x.copy_(x0)
        eng.decode_layer(x, layer=0, pos=512)
    eng.set_profiling(True)
    for _ in range(calls):
        x.copy_(x0)
        eng.decode_layer(x, layer=0, pos=512)
    per = {}
    for name in ("qkv", "attn", "o", "glu", "down"):
        cnt, ms, _ = eng.profile(name)
        per[name] = round(ms * 1e3 / cnt, 3) if cnt else None
    eng.set_profiling(False)
    total_us = sum(v for v in per.values() if v)
    kb = decode_kernel_bytes(CFG)
    nbytes = kb["qkv"] + kb["o"] + kb["glu"] + kb["down"] + CFG["n_kv_heads"] * 512 * 128
    gbs = nbytes / (total_us * 1e-6) / 1e9
    return {"workload": "one TinyLlama-shape decoder layer, decode step at position 512 (512 cached rows)",
            "kernel_us": per, "us": round(total_us, 3), "bytes": nbytes, "gbs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4)}


def bench_prefill(eng, seed, n_tokens, reps):
    """n_tokens-token prefill of the whole model: wall time (median of reps
    after one warm-up), then one profiled prefill for per-role GEMM dispatch
    durations at M = n_tokens."""
    import torch
    pp = np.random.default_rng(seed).integers(0, CFG["vocab"], n_tokens).astype(np.int32)
    eng.prefill(pp)
    times = []
    for _ in range(reps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        eng.prefill(pp)
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
    eng.set_profiling(True)
    eng.prefill(pp)
    ops = prefill_gemm_ops(CFG, n_tokens)
    roles = {}
    for name in ("qkv", "o", "glu", "down"):
        cnt, ms, _ = eng.profile(name)
        roles[name] = {"launches": cnt, "avg_us": round(ms * 1e3 / max(cnt, 1), 3),
                       "tops": round(ops[name] / (ms * 1e-3) / 1e12, 1) if ms else None,
                       "mfma_frac": round(ops[name] / (ms * 1e-3) / I8_PEAK_OPS, 4) if ms else None}
    # the rest of the same profiled prefill: attention (Q|K|V post-processing
    # where it runs separately, the attention tiles), the row kernels (RMSNorm
    # and quantization of every GEMM's activations) and the final LM head
    others = {}
    for name in ("attn", "norm", "lm_head", "other"):
        cnt, ms, _ = eng.profile(name)
        if cnt:
            others[name] = {"launches": cnt, "avg_us": round(ms * 1e3 / cnt, 3), "ms": round(ms, 3)}
    eng.set_profiling(False)
    gemm_ms = sum(r["avg_us"] * r["launches"] for r in roles.values()) / 1e3
    kernel_ms = gemm_ms + sum(o["ms"] for o in others.values())
    total_ops = sum(ops.values())
    ms_med = float(np.median(times))
    return {"tokens": n_tokens, "ms": round(ms_med, 3), "tok_s": round(n_tokens / ms_med * 1e3, 1),
            "gemm_ms": round(gemm_ms, 3), "gemm_launches": sum(r["launches"] for r in roles.values()),
            "gemm_tops": round(total_ops / (gemm_ms * 1e-3) / 1e12, 1),
            "mfma_frac": round(total_ops / (gemm_ms * 1e-3) / I8_PEAK_OPS, 4), "gemms": roles,
            "other_kernels": others,
            "kernel_ms": round(kernel_ms, 3),
            "note": "gemms and other_kernels: dispatch durations (HIP events around every kernel) of one "
                    "profiled prefill; kernel_ms is their sum, ms the unprofiled wall time"}


def bench_batch(eng_factory, host_seed, B=32, ctx=2048, steps=64):
    """Batched decode: B sequences, each with a (ctx - steps)-row seeded INT8 KV
    cache, then `steps` decode steps of all B together (M = B GEMMs)."""
    import torch
    eng = eng_factory(B)
    rng = np.random.default_rng(host_seed)
    start = ctx - steps
    for b in range(B):
        for layer in range(CFG["n_layers"]):
            for g in range(CFG["n_kv_heads"]):
                k = rng.integers(-127, 128, (start, 64), dtype=np.int8)
                v = rng.integers(-127, 128, (start, 64), dtype=np.int8)
                eng.kv_write(b, layer, g, 0, k, v)
    toks = rng.integers(0, CFG["vocab"], B).astype(np.int32)
    pos = np.full(B, start, np.int32)
    eng.decode_batch(toks, pos - 8, 8)  # warm-up over rows start-8..start-1
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = eng.decode_batch(toks, pos, steps)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    eng.set_profiling(True)
    eng.decode_batch(toks, pos, 4)
    per = {}
    for name in ("qkv", "attn", "o", "glu", "down", "lm_head", "norm", "other"):
        cnt, ms, _ = eng.profile(name)
        if cnt:
            per[name] = {"launches_per_step": cnt // 4, "us_per_step": round(ms * 1e3 / 4, 1)}
    eng.set_profiling(False)
    eng.close()
    weights = sum(decode_kernel_bytes(CFG)[k] for k in ("qkv", "o", "glu", "down")) * CFG["n_layers"] \
        + decode_kernel_bytes(CFG)["lm_head"]
    kv = B * CFG["n_layers"] * CFG["n_kv_heads"] * 128 * (start + steps / 2)
    step_s = dt / steps
    return {"workload": f"batched INT8 decode, {B} sequences x {start}-row seeded KV cache, {steps} steps",
            "tok_s": round(B * steps / dt, 1), "ms_per_step": round(step_s * 1e3, 3),
            "hbm_bytes_per_step": int(weights + kv),
            "gbs": round((weights + kv) / step_s / 1e9, 1),
            "frac": round((weights + kv) / step_s / 1e9 / HBM_PEAK_GBS, 4), "tokens_out": int(out.size),
            "kernels_dispatch": per}


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, each scaled by the same counter's reading for a
    device-to-device copy of known size), or None when it has not been measured."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(kernel)
    except (OSError, ValueError):
        return None
    return None if rec is None else rec.get("traffic_bytes")


def decode_section(eng, host, args):
    """The headline: timed graph replay of K steps, then the per-kernel
    measurements of the same sequence."""
    import torch
    prompt = np.random.default_rng(args.seed).integers(0, CFG["vocab"], args.prompt).astype(np.int32)
    eng.prefill(prompt)
    if args.warmup > 0:
        eng.decode(args.warmup)
    first, _ = eng.prefill(prompt)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    toks, _ = eng.decode(args.steps)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    log(f"decode: {args.steps} steps in {dt * 1e3:.1f} ms -> {args.steps / dt:.1f} tok/s")
    step_us = dt * 1e6 / args.steps

    # the same steps with an EOS id that never comes (stop flag read per chunk)
    eng.prefill(prompt)
    never = next(t for t in range(CFG["vocab"] - 1, -1, -1) if t not in set(toks.tolist()) and t != first)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    toks_eos, stop = eng.decode(args.steps, eos_id=never)
    torch.cuda.synchronize()
    eos_dt = time.perf_counter() - t0
    assert stop == "max_tokens" and np.array_equal(toks_eos, toks), "EOS-watching decode changed the tokens"

    # dispatch durations: the profiled steps launch every kernel directly with
    # HIP events that the dispatch itself timestamps
    kbytes = decode_kernel_bytes(CFG)
    kernels = {}
    if args.profile_steps > 0:
        eng.prefill(prompt)
        eng.set_profiling(True)
        eng.decode(args.profile_steps)
        for name in DECODE_CLASSES:
            cnt, ms, _ = eng.profile(name)
            if cnt:
                kernels[name] = {"launches_per_step": round(cnt / args.profile_steps),
                                 "dispatch_us": round(ms * 1e3 / cnt, 3)}
        eng.set_profiling(False)

    # device timeline of graph-replayed steps (the production regime)
    tl = {"steps": 0, "kernels": 0, "step_us": 0.0, "classes": {}}
    if args.timeline_steps > 0:
        eng.prefill(prompt)
        tl = eng.decode_timeline(args.timeline_steps)
    for name, rec in tl["classes"].items():
        e = kernels.setdefault(name, {})
        n = max(rec["launches"], 1)
        e.update(busy_us=round(rec["busy_us"] / n, 3), gap_after_us=round(rec["gap_us"] / n, 3))
    for name, e in kernels.items():
        if name in kbytes:
            e["bytes"] = kbytes[name]
            for src, dst in (("dispatch_us", "dispatch"), ("busy_us", "busy")):
                if e.get(src):
                    gbs = kbytes[name] / (e[src] * 1e-6) / 1e9
                    e[f"{dst}_gbs"] = round(gbs, 1)
                    e[f"{dst}_frac"] = round(gbs / HBM_PEAK_GBS, 4)
    busy = sum(r["busy_us"] for r in tl["classes"].values())
    gaps = sum(r["gap_us"] for r in tl["classes"].values())
    accounting = {
        "step_us": round(step_us, 2),
        "timeline_step_us": round(tl["step_us"], 2),
        "busy_us": round(busy, 2), "gaps_us": round(gaps, 2),
        "between_steps_us": round(step_us - tl["step_us"], 2),
        "kernels_per_step": tl["kernels"], "timeline_steps": tl["steps"],
        "note": "timeline_step_us = busy_us + gaps_us (first kernel start to last kernel end of a step); "
                "between_steps_us = step_us - timeline_step_us is the boundary from one replayed step to the next",
    }
    per_step = {k: (CFG["n_layers"] if k != "lm_head" else 1) for k in kbytes}
    bytes_step = sum(kbytes[k] * per_step[k] for k in kbytes)
    # all decode GEMVs of a step together: their algorithmic bytes over their
    # summed durations (dispatch, and busy inside the replayed graph)
    gemv = {"classes": sorted(kbytes), "bytes_per_step": bytes_step}
    for src, dst in (("dispatch_us", "dispatch"), ("busy_us", "busy")):
        if all(kernels.get(k, {}).get(src) for k in kbytes):
            us = sum(kernels[k][src] * per_step[k] for k in kbytes)
            gbs = sum(kbytes[k] * per_step[k] for k in kbytes) / (us * 1e-6) / 1e9
            gemv.update({f"{dst}_us_per_step": round(us, 2), f"{dst}_gbs": round(gbs, 1),
                         f"{dst}_frac": round(gbs / HBM_PEAK_GBS, 4)})
    margin = lm_head_margin(eng, prompt, first, toks)
    return dict(prompt=prompt, first=first, toks=toks, dt=dt, kernels=kernels, accounting=accounting, margin=margin,
                eos_watch={"tok_s": round(args.steps / eos_dt, 2), "vs_no_eos": round(dt / eos_dt, 4),
                           "eos_id": int(never)},
                bytes_step=bytes_step, gemv=gemv)


def lm_head_margin(eng, prompt, first, toks):
    """Top-1 minus top-2 logit of every greedy choice of the timed run (the
    prompt's next token and each decode step's), from one untimed prefill of
    prompt + generated tokens through tl_prefill_logits; prefill rows equal
    token-by-token decode bit for bit, so each row's argmax must be the token
    the decode produced."""
    import torch
    seq = np.concatenate([prompt, [first], toks[:-1]]).astype(np.int32)
    n, V = int(seq.size), CFG["vocab"]
    logits = torch.empty((n, V), dtype=torch.float32, device="cuda")
    eng.rt.call("tl_prefill_logits", 0, seq, n, logits)
    rows = logits[prompt.size - 1:].cpu().numpy()
    top2 = np.partition(rows, V - 2, axis=1)[:, V - 2:]
    margin = top2[:, 1] - top2[:, 0]
    want = np.concatenate([[first], toks]).astype(np.int64)
    return {"choices": int(rows.shape[0]), "min": float(margin.min()), "p01": float(np.quantile(margin, 0.01)),
            "median": float(np.median(margin)), "argmin_step": int(margin.argmin()) - 1,
            "exact_ties": int((margin == 0).sum()),
            "argmax_matches_decode": bool(np.array_equal(rows.argmax(axis=1), want))}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--prefill-len", type=int, default=512)
    ap.add_argument("--prefill-reps", type=int, default=5)
    ap.add_argument("--profile-steps", type=int, default=32)
    ap.add_argument("--timeline-steps", type=int, default=32)
    ap.add_argument("--cpu-steps", type=int, default=0, help="all-thread oracle steps (default: --steps)")
    ap.add_argument("--cpu-single-steps", type=int, default=16)
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--no-extras", action="store_true", help="skip the GEMV, layer and batch-32 workloads")
    ap.add_argument("--only", choices=["all", "decode", "prefill", "batch"], default="all",
                    help="run one workload alone (for profiling it): prefill repeats the 512-token prefill")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="only copy this many MiB device to device once (a kernel of known traffic for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: it measures the single-GPU hot path only "
              f"(--gpus {args.gpus} requested; sharding is described, not run)", file=sys.stderr)
        sys.exit(2)
    if args.prompt + args.steps + args.warmup > CFG["max_pos"]:
        sys.exit("prompt + steps exceeds the 2048-position context")

    import torch
    if args.copy_calibration_mib > 0:
        n = args.copy_calibration_mib << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "read": n, "written": n}), flush=True)
        return
    import __graft_entry__
    __graft_entry__.load_package()
    from lpta.engine import Engine

    torch.cuda.set_device(0)
    t0 = time.time()
    eng = Engine(CFG, max_seqs=1)
    host = eng.load_random(args.seed)
    log(f"model ready in {time.time() - t0:.1f}s")

    def batch_engine(B):
        return Engine(CFG, max_seqs=B).load_model(host)

    if args.only == "prefill":
        pre = bench_prefill(eng, args.seed + 1, args.prefill_len, max(args.prefill_reps, 1))
        log(f"prefill {args.prefill_len}: {pre}")
        eng.close()
        print(json.dumps({"prefill": pre}), flush=True)
        return
    if args.only == "batch":
        eng.close()
        b = bench_batch(batch_engine, args.seed + 7)
        log(f"batch 32: {b}")
        print(json.dumps({"batch32": b}), flush=True)
        return

    d = decode_section(eng, host, args)
    tok_s = args.steps / d["dt"]
    kernels = d["kernels"]
    glu = kernels.get("glu", {})

    pre = None
    if args.only == "all" and args.prefill_len > 0:
        pre = bench_prefill(eng, args.seed + 1, args.prefill_len, max(args.prefill_reps, 1))
        log(f"prefill {args.prefill_len}: {pre}")

    extras = None
    if args.only == "all" and not args.no_extras:
        extras = {"gemv_q_proj": bench_gemv_q_proj(eng, args.seed)}
        log(f"gemv q_proj: {extras['gemv_q_proj']}")
        if args.prefill_len >= 512:
            extras["decode_layer"] = bench_decode_layer(eng)
            log(f"decode layer: {extras['decode_layer']}")

    cpu = None
    if args.only == "all" and not args.no_cpu:
        model, nproc, usable = host_cpu()
        threads = args.cpu_threads or min(16, usable)
        steps_all = min(args.cpu_steps or args.steps, args.steps)
        steps_one = min(args.cpu_single_steps, args.steps)
        eng.prefill(d["prompt"])
        rate_all, rate_one, match = cpu_baseline(host, eng, args.prompt, d["first"], d["toks"], steps_all,
                                                 steps_one, threads)
        cpu = {"value": round(rate_all, 3), "unit": "tok/s", "cores": threads, "kind": "port",
               "sample": f"oracle (tl_oracle.c, gcc -O3, OpenMP) decoding the first {steps_all} of the timed greedy "
                         f"steps from the GPU's {args.prompt}-token KV cache on {threads} threads; "
                         f"single_thread over the first {steps_one}",
               "single_thread": round(rate_one, 3), "cpu_model": model, "nproc": nproc,
               "usable_cpus": usable, "tokens_match_gpu": bool(match)}
        log(f"cpu baseline: {cpu}")

    if extras is not None:
        eng.close()
        eng = None
        torch.cuda.empty_cache()
        extras["batch32"] = bench_batch(batch_engine, args.seed + 7)
        log(f"batch 32: {extras['batch32']}")

    out = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(d["dt"] * 1e3 / args.steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "TinyLlama-1.1B-shape INT8 greedy decode, batch 1, 128-token prompt then "
                               f"{args.steps} timed decode steps (22 layers + LM head + argmax per step)",
                   "layers": 22, "hidden": 2048, "heads": "32q/4kv", "ffn": 5632, "vocab": 32000,
                   "prompt_tokens": args.prompt, "weights": "random N(0,0.02), per-output-channel int8",
                   "kv_cache": "int8, static per-layer/per-kv-head scales"},
        "roofline": {"bound": "hbm", "kernel": "gemv_glu (gate+up SiLU-GLU decode GEMV)",
                     "achieved": glu.get("dispatch_gbs"), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": glu.get("dispatch_frac"), "traffic": measured_traffic("gemv_glu"),
                     "bytes_per_launch": glu.get("bytes"), "avg_us": glu.get("dispatch_us"),
                     "busy_us": glu.get("busy_us"), "busy_frac": glu.get("busy_frac")},
        "decode_step_hbm_frac": round(d["bytes_step"] / (d["dt"] / args.steps) / 1e9 / HBM_PEAK_GBS, 4),
        "decode_gemv": d["gemv"],
        "lm_head_margin": d["margin"],
        "step_accounting": d["accounting"],
        "kernels": kernels,
        "eos_watch": d["eos_watch"],
        "prefill": pre,
        "cpu_baseline": cpu,
        "workloads": extras,
    }
    if eng is not None:
        eng.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
