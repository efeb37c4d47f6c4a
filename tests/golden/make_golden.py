"""Write the golden vectors under tests/golden/ from the reference's own NumPy code.

Run once, in a container that has the reference checkout:

    python tests/golden/make_golden.py [/path/to/reference]

It imports model/tinyllama.py (TL), model/tinyllama_gemm_int8.py (GI) and
model/export_fpga_vectors.py (EX) from the reference, calls them on seeded
inputs and saves inputs and outputs as small .npz fixtures.  The fixtures are
data only; the tests read them and never the reference itself.  It also turns
the reference's committed integer fixtures (sim/*.txt, sim/test_k*/ and a
subsample of rtl/compute/rope_{cos,sin}_rom.memh) into .npz files.

Functions covered and the reference lines they exercise:
  rms_norm TL:45-50, build_rope_cache TL:59-66, apply_rope TL:69-80,
  softmax TL:100-103, silu TL:159-161, quantize_int8 GI:36-42,
  dequantize_int32 GI:45-46, quantized_linear GI:59-88,
  mixed_precision_self_attention GI:136-182 (captured internals),
  mixed_precision_decoder_layer GI:256-281, forward_mixed GI:437-467,
  quantize_probability_tile EX:870-873.
"""
from __future__ import annotations

import os
import sys
import tempfile

import numpy as np

OUT = os.path.dirname(os.path.abspath(__file__))
REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
sys.path.insert(0, os.path.join(REF, "model"))

import tinyllama as TL                 # noqa: E402
import tinyllama_gemm_int8 as GI       # noqa: E402
import export_fpga_vectors as EX       # noqa: E402


def save(name, **arrays):
    path = os.path.join(OUT, name)
    np.savez_compressed(path, **arrays)
    print(f"wrote {path}: {sorted(arrays)}")


def golden_primitives():
    rng = np.random.default_rng(20240501)
    # RMSNorm at the model width and at awkward widths (pairwise-sum edge cases)
    rms = {}
    for n in (2048, 5632, 64, 100, 128, 129, 300, 1000):
        x = (rng.standard_normal((3, n)) * rng.uniform(0.1, 30.0, (3, 1))).astype(np.float32)
        w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        rms[f"x_{n}"] = x
        rms[f"w_{n}"] = w
        rms[f"y_{n}"] = TL.rms_norm(x, w, 1e-5)
    save("rms_norm.npz", **rms)

    # quantize_int8 / dequantize_int32
    q = {}
    cases = {
        "normal": rng.standard_normal((4, 2048)).astype(np.float32),
        "wide": (rng.standard_normal(5632) * 50).astype(np.float32),
        "ties": (np.arange(-300, 301, dtype=np.float32) * 0.5),
        "zeros": np.zeros(64, np.float32),
        "tiny": (rng.standard_normal(100) * 1e-30).astype(np.float32),
    }
    for k, x in cases.items():
        qx, s = GI.quantize_int8(x)
        q[f"x_{k}"] = x
        q[f"q_{k}"] = qx
        q[f"s_{k}"] = np.float64(s)
    acc = rng.integers(-(2 ** 26), 2 ** 26, (3, 777)).astype(np.int32)
    sx, sw = 0.01234567891234, 0.000987654321
    q["deq_acc"] = acc
    q["deq_sx"] = np.float64(sx)
    q["deq_sw"] = np.float64(sw)
    q["deq_y"] = GI.dequantize_int32(acc, sx, sw)
    save("quantize.npz", **q)

    # quantized_linear (per-tensor weights, golden [K][N] layout)
    x = rng.standard_normal((3, 256)).astype(np.float32)
    w = (rng.standard_normal((256, 96)) * 0.02).astype(np.float32)
    out, dbg = GI.quantized_linear(x, w, None, capture_arrays=True)
    save("quantized_linear.npz", x=x, w=w, out=out, input_scale=np.float64(dbg["input_scale"][0]),
         weight_scale=np.float64(dbg["weight_scale"][0]), input_q=dbg["input_q"],
         weight_q=dbg["weight_q"], accum_int32=dbg["accum_int32"])

    # RoPE table (subsampled positions) and apply_rope
    cos, sin = TL.build_rope_cache(2048, 64, 10000.0)
    pos = np.unique(np.concatenate([np.arange(64), np.arange(64, 2048, 37), [2047]])).astype(np.int32)
    q_h = rng.standard_normal((32, 5, 64)).astype(np.float32)
    k_h = rng.standard_normal((4, 5, 64)).astype(np.float32)
    qr, kr = TL.apply_rope(q_h, k_h, cos, sin)
    save("rope.npz", positions=pos, cos=cos[pos], sin=sin[pos], q=q_h, k=k_h, q_rot=qr, k_rot=kr)

    # softmax over float32 rows of several lengths, and SiLU
    sm = {}
    for n in (1, 7, 64, 65, 513, 2048):
        s = (rng.standard_normal((2, n)) * 4).astype(np.float32)
        sm[f"s_{n}"] = s
        sm[f"p_{n}"] = TL.softmax(s, axis=-1)
    xs = np.concatenate([rng.standard_normal(4000) * 4, [-80, -61, -60, -59.5, 0.0, 59.5, 60, 61, 80]]).astype(np.float32)
    sm["silu_x"] = xs
    sm["silu_y"] = TL.silu(xs)
    p = np.concatenate([rng.uniform(0, 1, 3000), (np.arange(128) + 0.5) / 127.0, [0.0, 1.0]]).astype(np.float32)
    sm["prob_p"] = p
    sm["prob_q"] = EX.quantize_probability_tile(p)
    save("softmax_silu.npz", **sm)


def tiny_cfg():
    return dict(hidden=256, intermediate=512, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64,
                vocab=512, max_pos=128, rms_eps=1e-5, rope_theta=10000.0)


def exact_int8_weight(rng, shape):
    """int8 values q with max |q| = 127; the float weight is q * 2**-9 exactly,
    so the golden's per-tensor quantize_int8 recovers q with scale 2**-9."""
    q = np.clip(np.rint(rng.standard_normal(shape) * 10.0), -127, 127).astype(np.int8)
    q.flat[rng.integers(q.size)] = 127
    return q


W_SCALE = 2.0 ** -9


def golden_model():
    """A small random model in the golden's .npz schema (TL:205-267, 322-377).
    Every weight is int8 * 2**-9, so the golden's per-tensor dequantization
    multiplier equals the per-channel one with all channel scales 2**-9."""
    rng = np.random.default_rng(7)
    c = tiny_cfg()
    D, F, H, Hkv, hd, V = c["hidden"], c["intermediate"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["vocab"]
    arrays = {
        "meta_model_id": np.array("synthetic/tiny-int8"),
        "meta_hidden_size": np.array(D, np.int32),
        "meta_intermediate_size": np.array(F, np.int32),
        "meta_num_hidden_layers": np.array(c["n_layers"], np.int32),
        "meta_num_attention_heads": np.array(H, np.int32),
        "meta_num_key_value_heads": np.array(Hkv, np.int32),
        "meta_head_dim": np.array(hd, np.int32),
        "meta_vocab_size": np.array(V, np.int32),
        "meta_max_position_embeddings": np.array(c["max_pos"], np.int32),
        "meta_rms_norm_eps": np.array(c["rms_eps"], np.float32),
        "meta_rope_theta": np.array(c["rope_theta"], np.float32),
    }
    qs = {}
    e8 = rng.integers(-127, 128, (V, D)).astype(np.int8)
    es = rng.uniform(2e-3, 8e-3, V).astype(np.float32)
    arrays["embed_w"] = (e8.astype(np.float32) * es[:, None]).astype(np.float32)
    arrays["final_norm_w"] = (1.0 + 0.05 * rng.standard_normal(D)).astype(np.float32)
    qs["lm_head_w"] = exact_int8_weight(rng, (D, V))
    shapes = {"q_w": (D, D), "k_w": (D, Hkv * hd), "v_w": (D, Hkv * hd), "o_w": (D, D),
              "gate_w": (D, F), "up_w": (D, F), "down_w": (F, D)}
    for i in range(c["n_layers"]):
        for name, shp in shapes.items():
            qs[f"layer{i}_{name}"] = exact_int8_weight(rng, shp)
        arrays[f"layer{i}_input_norm_w"] = (1.0 + 0.05 * rng.standard_normal(D)).astype(np.float32)
        arrays[f"layer{i}_post_norm_w"] = (1.0 + 0.05 * rng.standard_normal(D)).astype(np.float32)
    for k, q in qs.items():
        arrays[k] = (q.astype(np.float32) * np.float32(W_SCALE)).astype(np.float32)
    return c, arrays, qs, e8, es


def golden_composed():
    c, arrays, qs, e8, es = golden_model()
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "tiny.npz")
        np.savez(path, **arrays)
        weights = TL.load_weights(path, compute_dtype=np.float32, cache_arrays=True)
        cfg = weights.cfg
        cos, sin = TL.build_rope_cache(cfg["max_position_embeddings"], cfg["head_dim"], cfg["rope_theta"])

        out = {"embed_q": e8, "embed_s": es, "w_scale": np.float64(W_SCALE)}
        for k, q in qs.items():
            out[k + "_q"] = q          # the float weight is q * w_scale, [K][N] golden layout
        for k, v in arrays.items():
            if k.endswith("norm_w"):
                out[k] = v
        # one decoder layer at one token (position 0)
        tok = 17
        x0 = weights.embed([tok]).astype(np.float32)
        y, dbg = GI.mixed_precision_decoder_layer(x0, weights.layer(0), cfg, cos, sin, capture_arrays=True)
        out.update(layer_tok=np.int32(tok), layer_x=x0, layer_y=y,
                   layer_attn_input=dbg["attn_input_fp"], layer_x_after_attn=dbg["x_after_attn_fp"],
                   layer_ffn_input=dbg["ffn_input_fp"], layer_hidden=dbg["ffn"]["hidden_fp"],
                   layer_q=dbg["attn"]["q_proj_fp"], layer_k=dbg["attn"]["k_proj_fp"],
                   layer_v=dbg["attn"]["v_proj_fp"], layer_attended=dbg["attn"]["attended_fp"],
                   layer_q_acc=dbg["attn"]["q_proj"]["accum_int32"],
                   layer_down_acc=dbg["ffn"]["down_proj"]["accum_int32"])
        # attention internals over a short causal sequence (float attention of the golden)
        toks = [5, 301, 42, 42, 333, 7]
        xs = weights.embed(toks).astype(np.float32)
        a_in = TL.rms_norm(xs, weights.layer(0)["input_norm_w"], cfg["rms_norm_eps"])
        att, adbg = GI.mixed_precision_self_attention(a_in, weights.layer(0), cfg, cos, sin, capture_arrays=True)
        out.update(attn_tokens=np.asarray(toks, np.int32), attn_q=adbg["q_proj_fp"], attn_k=adbg["k_proj_fp"],
                   attn_v=adbg["v_proj_fp"], attn_weights=adbg["weights_fp"], attn_attended=adbg["attended_fp"])
        # full forward at one token, quantized LM head, greedy id
        for t in (17, 250, 511):
            logits = GI.forward_mixed([t], weights, cos, sin, cfg["num_hidden_layers"], True)
            out[f"fwd_logits_{t}"] = logits[-1]
            out[f"fwd_token_{t}"] = np.int32(np.argmax(logits[-1]))
        out["cfg"] = np.array([c["hidden"], c["intermediate"], c["n_layers"], c["n_heads"], c["n_kv_heads"],
                               c["head_dim"], c["vocab"], c["max_pos"]], np.int32)
    save("tiny_model.npz", **out)


def reference_fixtures():
    sim = os.path.join(REF, "sim")
    load = lambda p: np.loadtxt(p, dtype=np.int64).astype(np.int32)  # noqa: E731
    fx = {"x": load(os.path.join(sim, "x.txt")), "w": load(os.path.join(sim, "w.txt")),
          "expected": load(os.path.join(sim, "expected.txt"))}
    for k in (16, 64):
        d = os.path.join(sim, f"test_k{k}")
        for name in ("x_q", "W1_q", "W2_q", "y1_int", "y2_q", "y_expected"):
            fx[f"k{k}_{name}"] = load(os.path.join(d, f"{name}.txt"))
        with open(os.path.join(d, "scales.txt")) as fh:
            for line in fh:
                key, val = line.split()
                fx[f"k{k}_{key}"] = np.float64(val)
    save("sim_fixtures.npz", **fx)

    rom = {}
    for kind in ("cos", "sin"):
        with open(os.path.join(REF, "rtl", "compute", f"rope_{kind}_rom.memh")) as fh:
            words = np.array([int(s, 16) for s in fh.read().split()], np.uint32).view(np.int32)
        rom[kind] = words.reshape(2048, 32)
    pos = np.unique(np.concatenate([np.arange(64), np.arange(64, 2048, 29), [2047]])).astype(np.int32)
    save("rope_rom.npz", positions=pos, cos_q16=rom["cos"][pos], sin_q16=rom["sin"][pos])


if __name__ == "__main__":
    golden_primitives()
    golden_composed()
    reference_fixtures()
