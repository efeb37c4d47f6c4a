"""Benchmark of the INT8 TinyLlama-1.1B decoder hot path on one MI355X.

Workload (value): greedy decode at batch 1 of a TinyLlama-1.1B-shape INT8
model (22 layers, hidden 2048, 32/4 heads, FFN 5632, vocab 32000) with
random N(0, 0.02) weights quantized per output channel: a 128-token seeded
prompt is prefilled, then --steps greedy decode steps (default 256) are timed.
One "step" is one token through 22 decoder layers, the LM head and argmax.

Also reported, on the same model in the same run:
  roofline      the dominant decode kernel (SiLU-GLU gate/up GEMV) timed with
                HIP events on the library's stream: algorithmic bytes per
                launch / average launch time, against 8 TB/s;
  kernels       the same for every decode kernel class;
  prefill       512-token prefill (all 22 layers + LM head + argmax): i8 MFMA
                utilisation of the GEMM kernels against 5.0 POP/s dense;
  cpu_baseline  the CPU oracle (tl_oracle.c, OpenMP) decoding a bounded
                sample of the same steps from the same KV cache; its tokens
                must equal the GPU's.

    python bench.py [--gpus 1] [--steps 256] [--warmup 8]
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

METRIC = "decode tok/s + decode GEMV HBM GB/s + prefill i8 MFMA %, TinyLlama-1.1B bs=1"
HBM_PEAK_GBS = 8000.0
I8_PEAK_OPS = 5.0e15
CFG = dict(hidden=2048, intermediate=5632, n_layers=22, n_heads=32, n_kv_heads=4, head_dim=64,
           vocab=32000, max_pos=2048, rms_eps=np.float32(1e-5), rope_theta=10000.0)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_model_on_device(eng, cfg, seed):
    """Random-init weights drawn on the GPU (torch RNG, plumbing) and
    quantized per output channel by the library's own quantizer."""
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    D, F, V = cfg["hidden"], cfg["intermediate"], cfg["vocab"]
    kvd = cfg["n_kv_heads"] * cfg["head_dim"]
    shapes = [(D, D), (kvd, D), (kvd, D), (D, D), (F, D), (F, D), (D, F)]

    def qrows(rows, cols):
        w = torch.randn(rows, cols, generator=g, device="cuda", dtype=torch.float32) * 0.02
        q = torch.empty(rows, cols, dtype=torch.int8, device="cuda")
        s = torch.empty(rows, dtype=torch.float32, device="cuda")
        eng.rt.call("tl_quantize_weight_rows", w, rows, cols, q, s)
        return q, s

    host_layers = []
    for layer in range(cfg["n_layers"]):
        ws, ss = zip(*[qrows(*shp) for shp in shapes])
        g_in = 1.0 + 0.02 * torch.randn(D, generator=g, device="cuda")
        g_post = 1.0 + 0.02 * torch.randn(D, generator=g, device="cuda")
        L = dict(w=list(ws), s=list(ss), g_in=g_in, g_post=g_post)
        eng.load_layer(layer, L)
        host_layers.append({k: ([t.cpu().numpy() for t in v] if isinstance(v, list) else v.cpu().numpy())
                            for k, v in L.items()})
    lm_w, lm_s = qrows(V, D)
    emb, emb_s = qrows(V, D)
    g_final = 1.0 + 0.02 * torch.randn(D, generator=g, device="cuda")
    eng.load_lm_head(lm_w, lm_s, g_final)
    eng.load_embedding(emb, emb_s)
    rng = np.random.default_rng(seed)
    sk = rng.uniform(0.02, 0.06, (cfg["n_layers"], cfg["n_kv_heads"])).astype(np.float32)
    sv = rng.uniform(0.02, 0.06, (cfg["n_layers"], cfg["n_kv_heads"])).astype(np.float32)
    eng.set_kv_scales(sk, sv)
    from lpta import build_rope_cache
    cos, sin = build_rope_cache(cfg["max_pos"], cfg["head_dim"], cfg["rope_theta"])
    eng.set_rope_table(cos, sin)
    torch.cuda.synchronize()
    host = dict(layers=host_layers, lm_w=lm_w.cpu().numpy(), lm_s=lm_s.cpu().numpy(),
                g_final=g_final.cpu().numpy(), emb=emb.cpu().numpy(), emb_s=emb_s.cpu().numpy(),
                rope_cos=cos, rope_sin=sin, kv_sk=sk, kv_sv=sv)
    return host


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
    D, F = cfg["hidden"], cfg["intermediate"]
    kvd = cfg["n_kv_heads"] * cfg["head_dim"]
    per_layer = (D + 2 * kvd) * D + D * D + 2 * F * D + D * F
    return 2.0 * m * per_layer * cfg["n_layers"]


def cpu_baseline(host, cfg, eng, prompt_len, first_token, gpu_tokens, n_steps, threads):
    """The oracle continues the same sequence on the host cores from the GPU's
    KV cache (positions 0..prompt_len-1) for n_steps greedy steps."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    arrays = oracle.ModelArrays(cfg=dict(cfg), layers=host["layers"], lm_w=host["lm_w"], lm_s=host["lm_s"],
                                g_final=host["g_final"], emb=host["emb"], emb_s=host["emb_s"],
                                rope_cos=host["rope_cos"], rope_sin=host["rope_sin"],
                                kv_sk=host["kv_sk"], kv_sv=host["kv_sv"])
    kc, vc = arrays.new_cache()
    for layer in range(cfg["n_layers"]):
        for g in range(cfg["n_kv_heads"]):
            k, v = eng.kv_read(0, layer, g, 0, prompt_len)
            kc[layer, g, :prompt_len] = k
            vc[layer, g, :prompt_len] = v
    orc = oracle.Oracle(arrays)
    oracle.lib().or_set_threads(threads)
    tok = first_token
    got = []
    t0 = time.perf_counter()
    for s in range(n_steps):
        x = orc.embed(tok)
        for layer in range(cfg["n_layers"]):
            x = orc.decode_row(layer, prompt_len + s, x, kc, vc)
        tok, _ = orc.lm_head(x)
        got.append(tok)
    dt = time.perf_counter() - t0
    return n_steps / dt, got, got == [int(t) for t in gpu_tokens[:n_steps]]


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
    average HIP-event times."""
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


def bench_batch(model_eng_factory, host_seed, B=32, ctx=2048, steps=64):
    """Batched decode: B sequences, each with a (ctx - steps)-row seeded INT8 KV
    cache, then `steps` decode steps of all B together (M = B GEMMs)."""
    import torch
    eng = model_eng_factory(B)
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
    eng.close()
    weights = sum(decode_kernel_bytes(CFG)[k] for k in ("qkv", "o", "glu", "down")) * CFG["n_layers"] \
        + decode_kernel_bytes(CFG)["lm_head"]
    kv = B * CFG["n_layers"] * CFG["n_kv_heads"] * 128 * (start + steps / 2)
    step_s = dt / steps
    return {"workload": f"batched INT8 decode, {B} sequences x {start}-row seeded KV cache, {steps} steps",
            "tok_s": round(B * steps / dt, 1), "ms_per_step": round(step_s * 1e3, 3),
            "hbm_bytes_per_step": int(weights + kv),
            "gbs": round((weights + kv) / step_s / 1e9, 1),
            "frac": round((weights + kv) / step_s / 1e9 / HBM_PEAK_GBS, 4), "tokens_out": int(out.size)}


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, each scaled by the same counter's reading for a
    device-to-device copy of known size), or None when it has not been measured."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(kernel)
    except (OSError, ValueError):
        return None
    return None if rec is None else rec.get("traffic_bytes")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--prefill-len", type=int, default=512)
    ap.add_argument("--profile-steps", type=int, default=32)
    ap.add_argument("--cpu-steps", type=int, default=4)
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--no-extras", action="store_true", help="skip the GEMV, layer and batch-32 workloads")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="only copy this many MiB device to device once (a kernel of known traffic for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: this build measures the single-GPU hot path only "
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
    host = build_model_on_device(eng, CFG, args.seed)
    log(f"model ready in {time.time() - t0:.1f}s")
    prompt = np.random.default_rng(args.seed).integers(0, CFG["vocab"], args.prompt).astype(np.int32)

    # warmup (untimed): prefill + a few decode steps
    eng.prefill(prompt)
    if args.warmup > 0:
        eng.decode(args.warmup)
    # timed: K decode steps after a fresh prefill of the same prompt
    first, _ = eng.prefill(prompt)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    toks, _ = eng.decode(args.steps)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    tok_s = args.steps / dt
    log(f"decode: {args.steps} steps in {dt * 1e3:.1f} ms -> {tok_s:.1f} tok/s")

    # per-kernel timing with HIP events on the library's stream
    kbytes = decode_kernel_bytes(CFG)
    kernels = {}
    eng.prefill(prompt)
    eng.set_profiling(True)
    if args.profile_steps > 0:
        eng.decode(args.profile_steps)
    for name in ("qkv", "o", "glu", "down", "lm_head", "attn", "norm"):
        cnt, ms, _ = eng.profile(name)
        if cnt:
            avg_us = ms * 1e3 / cnt
            entry = {"launches": cnt, "avg_us": round(avg_us, 3)}
            if name in kbytes:
                gbs = kbytes[name] / (avg_us * 1e-6) / 1e9
                entry.update(bytes=kbytes[name], gbs=round(gbs, 1), frac=round(gbs / HBM_PEAK_GBS, 4))
            kernels[name] = entry
    eng.set_profiling(False)
    gemv_bytes = sum(kbytes[k] * kernels[k]["launches"] for k in kbytes if k in kernels)
    gemv_us = sum(kernels[k]["avg_us"] * kernels[k]["launches"] for k in kbytes if k in kernels)
    glu = kernels.get("glu", {"gbs": None, "frac": None, "bytes": kbytes["glu"], "avg_us": None})

    # prefill: 512 tokens, MFMA utilisation of the GEMM kernels
    pre = None
    if args.prefill_len > 0:
        pp = np.random.default_rng(args.seed + 1).integers(0, CFG["vocab"], args.prefill_len).astype(np.int32)
        eng.prefill(pp)  # warm
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        eng.prefill(pp)
        torch.cuda.synchronize()
        pre_ms = (time.perf_counter() - t0) * 1e3
        eng.set_profiling(True)
        eng.prefill(pp)
        cnt, gemm_ms, _ = eng.profile("gemm_prefill")
        eng.set_profiling(False)
        ops = prefill_gemm_ops(CFG, args.prefill_len)
        pre = {"tokens": args.prefill_len, "ms": round(pre_ms, 3), "tok_s": round(args.prefill_len / pre_ms * 1e3, 1),
               "gemm_ms": round(gemm_ms, 3), "gemm_launches": cnt,
               "gemm_tops": round(ops / (gemm_ms * 1e-3) / 1e12, 1),
               "mfma_frac": round(ops / (gemm_ms * 1e-3) / I8_PEAK_OPS, 4)}
        log(f"prefill {args.prefill_len}: {pre}")

    extras = None
    if not args.no_extras:
        extras = {"gemv_q_proj": bench_gemv_q_proj(eng, args.seed)}
        log(f"gemv q_proj: {extras['gemv_q_proj']}")
        if args.prefill_len >= 512:
            extras["decode_layer"] = bench_decode_layer(eng)
            log(f"decode layer: {extras['decode_layer']}")

    cpu = None
    if not args.no_cpu and args.cpu_steps > 0:
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        eng.prefill(prompt)
        rate, ctoks, match = cpu_baseline(host, CFG, eng, args.prompt, first, toks, args.cpu_steps, threads)
        cpu = {"value": round(rate, 3), "unit": "tok/s", "cores": threads, "kind": "port",
               "sample": f"oracle (tl_oracle.c, OpenMP) decoding {args.cpu_steps} greedy steps of the same "
                         f"sequence from the GPU's {args.prompt}-token KV cache",
               "tokens_match_gpu": bool(match)}
        log(f"cpu baseline: {cpu}")

    if extras is not None:
        # the batch needs its own handle (32 KV caches); free the batch-1 model first
        layers_host = host
        eng.close()
        del eng
        torch.cuda.empty_cache()

        def factory(B):
            e = Engine(CFG, max_seqs=B)
            for i, L in enumerate(layers_host["layers"]):
                e.load_layer(i, L)
            e.load_lm_head(layers_host["lm_w"], layers_host["lm_s"], layers_host["g_final"])
            e.load_embedding(layers_host["emb"], layers_host["emb_s"])
            e.set_kv_scales(layers_host["kv_sk"], layers_host["kv_sv"])
            return e

        extras["batch32"] = bench_batch(factory, args.seed + 7)
        log(f"batch 32: {extras['batch32']}")
        eng = None

    out = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dt * 1e3 / args.steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "TinyLlama-1.1B-shape INT8 greedy decode, batch 1, 128-token prompt then "
                               f"{args.steps} timed decode steps (22 layers + LM head + argmax per step)",
                   "layers": 22, "hidden": 2048, "heads": "32q/4kv", "ffn": 5632, "vocab": 32000,
                   "prompt_tokens": args.prompt, "weights": "random N(0,0.02), per-output-channel int8",
                   "kv_cache": "int8, static per-layer/per-kv-head scales"},
        "roofline": {"bound": "hbm", "kernel": "gemv_glu (gate+up SiLU-GLU decode GEMV)",
                     "achieved": glu["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": glu["frac"],
                     "traffic": measured_traffic("gemv_glu"), "bytes_per_launch": glu["bytes"],
                     "avg_us": glu["avg_us"]},
        "decode_gemv_gbs": round(gemv_bytes / (gemv_us * 1e-6) / 1e9, 1) if gemv_us else None,
        "decode_step_hbm_frac": (round(gemv_bytes / args.profile_steps / (dt / args.steps) / 1e9 / HBM_PEAK_GBS, 4)
                                 if args.profile_steps else None),
        "kernels": kernels,
        "prefill": pre,
        "cpu_baseline": cpu,
        "workloads": extras,
    }
    if eng is not None:
        eng.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
