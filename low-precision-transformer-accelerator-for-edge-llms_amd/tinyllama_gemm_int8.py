"""The operator surface of model/tinyllama_gemm_int8.py (GI) on the MI355X path.

Same function names, arguments, return values, debug-dict keys and errors as
the reference module, computed by the HIP library through its C-ABI:

- quantize_int8, dequantize_int32 and quantized_linear follow GI:36-88
  exactly (one scale per tensor, weights quantized on every call) and are
  bit-exact to the reference.
- mixed_precision_self_attention, mixed_precision_feed_forward,
  mixed_precision_decoder_layer, forward_mixed and run_generate run the INT8
  accelerator path this library implements: activations quantized per row,
  weights per output channel (design_decisions A10/B1), and attention over a
  symmetric INT8 KV cache with static per-layer/per-KV-head scales, INT8 score
  and probability x V contractions (A7/A9/B2; EX:870-888, 2082-2089).  At one
  token the projections coincide with the reference; the attention and what
  follows agree with it to within the INT8 cache's quantization error.
  Results are bit-exact to the CPU oracle of that path and to the library's
  fused kernels.

Static KV scales come from the caller (``kv_scales=(k, v)``, [Hkv] per layer)
or from the weight archive (``kv_k_scale``/``kv_v_scale``); otherwise they are
calibrated on the input, per KV head: s = f32(max|x| / 127) over the rotated
keys / the values of the sequence (1.0 for an all-zero head).

Only quantize_lm_head=True is supported by forward_mixed / run_generate: the
LM head is one of the INT8 GEMM roles of the path.
"""
from __future__ import annotations

import os
from typing import Any

import numpy as np

from ._native import Runtime
from . import tinyllama as TL
from .tinyllama import (TinyLlamaWeights, build_rope_cache, dev, empty, host, load_weights, op_runtime,
                        round_pos, set_rope_rows)

WEIGHTS = ("q_w", "k_w", "v_w", "o_w", "gate_w", "up_w", "down_w")


# ---------------------------------------------------------------------------
# GI:36-88
# ---------------------------------------------------------------------------
def _quantize_dev(x_dev, n: int):
    """Per-tensor quantization on the device: (int8 tensor, float scale)."""
    q = empty((n,), np.int8)
    s = empty((1,), np.float64)
    if n == 0:
        return q, 1.0
    op_runtime().call("tl_quantize_tensor", x_dev, n, q, s)
    return q, float(host(s)[0])


def quantize_int8(tensor: np.ndarray) -> tuple[np.ndarray, float]:
    """GI:36-42: s = max|x| / 127 (1.0 if 0), q = clip(rne(x / s), -127, 127)."""
    x = np.asarray(tensor, dtype=np.float32)
    q, s = _quantize_dev(dev(x.ravel()), x.size)
    return host(q).reshape(x.shape), s


def dequantize_int32(accum: np.ndarray, input_scale: float, weight_scale: float) -> np.ndarray:
    """GI:45-46: f32(accum) * (input_scale * weight_scale)."""
    acc = np.asarray(accum, dtype=np.int32)
    if acc.size == 0:
        return np.empty(acc.shape, np.float32)
    cols = acc.shape[-1] if acc.ndim else 1
    y = empty((acc.size,), np.float32)
    op_runtime().call("tl_dequantize_i32", dev(acc.ravel()), acc.size // cols, cols, float(input_scale),
                      float(weight_scale), None, y)
    return host(y).reshape(acc.shape)


def diff_stats(reference: np.ndarray, candidate: np.ndarray) -> dict[str, float]:
    """GI:49-56 (a host-side report, not part of the computation)."""
    diff = np.asarray(candidate, dtype=np.float32) - np.asarray(reference, dtype=np.float32)
    abs_diff = np.abs(diff)
    return {"mae": float(abs_diff.mean()), "rmse": float(np.sqrt(np.mean(diff * diff))),
            "max_abs": float(abs_diff.max())}


def _pad_k(t, k: int, kp: int):
    """int8 [rows][k] -> [rows][kp] with zero columns (zero products are exact)."""
    if kp == k:
        return t.contiguous()
    import torch
    out = torch.zeros((t.shape[0], kp), dtype=t.dtype, device=t.device)
    out[:, :k] = t
    return out


def quantized_linear(x: np.ndarray, w: np.ndarray, b: np.ndarray | None = None,
                     capture_arrays: bool = False) -> tuple[np.ndarray, dict[str, Any]]:
    """GI:59-88: per-tensor INT8 x @ W ([K][N]) with INT32 accumulation, then
    dequantization (+ bias)."""
    x_fp = np.asarray(x, dtype=np.float32)
    w_fp = np.asarray(w, dtype=np.float32)
    k, n = w_fp.shape
    x2 = x_fp.reshape(-1, k)
    m = x2.shape[0]
    rt = op_runtime()
    xq, x_scale = _quantize_dev(dev(x2.ravel()), x2.size)
    wq, w_scale = _quantize_dev(dev(w_fp.ravel()), w_fp.size)
    kp = max(64, -(-k // 64) * 64)
    out = empty((m, n), np.float32)
    acc = empty((m, n), np.int32)
    if m:
        a8 = _pad_k(xq.view(m, k), k, kp)
        w8 = _pad_k(wq.view(k, n).t(), k, kp)
        rt.call("tl_gemm_i8", a8, w8, m, n, kp, acc)
        bias = None if b is None else dev(np.broadcast_to(np.asarray(b, np.float32), (n,)))
        rt.call("tl_dequantize_i32", acc, m, n, x_scale, w_scale, bias, out)
    shape = x_fp.shape[:-1] + (n,)
    out_h = host(out).reshape(shape)
    debug: dict[str, Any] = {
        "input_scale": np.array([x_scale], dtype=np.float32),
        "weight_scale": np.array([w_scale], dtype=np.float32),
    }
    if capture_arrays:
        debug.update({
            "input_fp": x_fp,
            "input_q": host(xq).reshape(x_fp.shape),
            "weight_fp": w_fp,
            "weight_q": host(wq).reshape(w_fp.shape),
            "accum_int32": host(acc).reshape(shape),
            "output_fp": out_h,
        })
    return out_h, debug


# ---------------------------------------------------------------------------
# the INT8 accelerator path, staged through the C-ABI so every debug value
# of the reference exists
# ---------------------------------------------------------------------------
def _our_cfg(cfg: dict, n_layers: int, vocab: int | None = None) -> dict:
    return dict(hidden=cfg["hidden_size"], intermediate=cfg["intermediate_size"], n_layers=n_layers,
                n_heads=cfg["num_attention_heads"], n_kv_heads=cfg["num_key_value_heads"],
                head_dim=cfg["head_dim"], vocab=vocab if vocab is not None else cfg.get("vocab_size", 64),
                max_pos=round_pos(cfg["max_position_embeddings"]), rms_eps=np.float32(cfg["rms_norm_eps"]),
                rope_theta=float(cfg.get("rope_theta", 10000.0)))


def _check_no_bias(layer: dict) -> None:
    for key in ("q_b", "k_b", "v_b", "o_b", "gate_b", "up_b", "down_b"):
        if layer.get(key) is not None:
            raise ValueError(f"{key}: the INT8 path has no projection biases (TinyLlama has none)")


class _QLayer:
    """One decoder layer quantized per output channel on the device:
    int8 [N][K] + float32 [N] for q, k, v, o, gate, up, down."""

    def __init__(self, rt: Runtime, layer: dict):
        _check_no_bias(layer)
        self.w, self.s, self.fp = {}, {}, {}
        for name in WEIGHTS:
            w_kn = np.asarray(layer[name], dtype=np.float32)
            n, k = w_kn.shape[1], w_kn.shape[0]
            w_nk = dev(np.ascontiguousarray(w_kn.T))
            q = empty((n, k), np.int8)
            s = empty((n,), np.float32)
            rt.call("tl_quantize_weight_rows", w_nk, n, k, q, s)
            self.w[name], self.s[name], self.fp[name] = q, s, w_kn
        self.g_in = dev(np.asarray(layer["input_norm_w"], np.float32))
        self.g_post = dev(np.asarray(layer["post_norm_w"], np.float32))

    def load_into(self, rt: Runtime, index: int) -> None:
        rt.load_layer(index, [self.w[n] for n in WEIGHTS], [self.s[n] for n in WEIGHTS], self.g_in, self.g_post,
                      src=1)


def _quantize_rows(rt: Runtime, x, rows: int, n: int):
    q = empty((rows, n), np.int8)
    s = empty((rows,), np.float64)
    rt.call("tl_quantize_rows", x, rows, n, q, s)
    return q, s


def _linear_rows(rt: Runtime, a8, a_s, ql: _QLayer, name: str, rows: int, residual=None):
    w = ql.w[name]
    n, k = w.shape
    y = empty((rows, n), np.float32)
    rt.call("tl_gemm_i8_dequant", a8, a_s, w, ql.s[name], rows, n, k, residual, y)
    return y


def _proj_debug(rt: Runtime, a_fp, a8, a_s, ql: _QLayer, name: str, rows: int, out, capture: bool) -> dict:
    """The reference's quantized_linear debug dict for one projection: per-row
    input scales and per-channel weight scales in place of its two scalars."""
    d: dict[str, Any] = {"input_scale": host(a_s).astype(np.float32),
                         "weight_scale": host(ql.s[name]).astype(np.float32)}
    if capture:
        w = ql.w[name]
        n, k = w.shape
        acc = empty((rows, n), np.int32)
        kp = max(64, -(-k // 64) * 64)
        rt.call("tl_gemm_i8", _pad_k(a8, k, kp), _pad_k(w, k, kp), rows, n, kp, acc)
        d.update({"input_fp": host(a_fp), "input_q": host(a8), "weight_fp": ql.fp[name],
                  "weight_q": np.ascontiguousarray(host(w).T), "accum_int32": host(acc), "output_fp": host(out)})
    return d


def _calibrate_kv(rt: Runtime, k_rows, v_rows, rows: int, hkv: int, pos0: int, cos, sin):
    """Static per-KV-head scales from this sequence: rotated keys, raw values."""
    kr = k_rows.clone()
    rt_rope = op_runtime(max_pos=pos0 + rows)
    set_rope_rows(rt_rope, cos, sin, pos0 + rows)
    rt_rope.call("tl_rope", kr, rows, hkv, dev(np.arange(pos0, pos0 + rows, dtype=np.int32)))
    sk = np.empty(hkv, np.float32)
    sv = np.empty(hkv, np.float32)
    for g in range(hkv):
        for src, dst in ((kr, sk), (v_rows, sv)):
            head = src.view(rows, hkv, 64)[:, g, :].contiguous()
            _, s = _quantize_dev(head.view(-1), rows * 64)
            dst[g] = np.float32(s)
    return sk, sv


class _Model:
    """A handle holding layers of one geometry, its KV cache (sequence 0) and
    RoPE table; layers are loaded into slots 0.. in order."""

    def __init__(self, cfg: dict, n_layers: int, vocab: int, cos, sin):
        self.cfg = cfg
        self.ours = _our_cfg(cfg, n_layers, vocab)
        self.rt = Runtime(self.ours)
        n_pos = min(cos.shape[0], self.ours["max_pos"])
        if n_pos < cfg["max_position_embeddings"]:
            raise ValueError("RoPE table shorter than max_position_embeddings")
        self.cos = np.ascontiguousarray(cos[:n_pos], np.float32)
        self.sin = np.ascontiguousarray(sin[:n_pos], np.float32)
        set_rope_rows(self.rt, self.cos, self.sin, n_pos)
        self.L = n_layers
        self.sk = np.ones((n_layers, self.ours["n_kv_heads"]), np.float32)
        self.sv = np.ones((n_layers, self.ours["n_kv_heads"]), np.float32)

    def set_kv_scales(self, layer: int, sk, sv) -> None:
        self.sk[layer] = sk
        self.sv[layer] = sv
        self.rt.call("tl_set_kv_scales", self.sk, self.sv)

    # -- stages -----------------------------------------------------------
    def attention(self, ql: _QLayer, layer: int, a, a8, a_s, rows: int, kv_scales, capture: bool):
        """Q/K/V projections, RoPE, KV append, INT8 attention, O projection."""
        rt, c = self.rt, self.ours
        D, hkv = c["hidden"], c["n_kv_heads"]
        kvd = hkv * 64
        q = _linear_rows(rt, a8, a_s, ql, "q_w", rows)
        k = _linear_rows(rt, a8, a_s, ql, "k_w", rows)
        v = _linear_rows(rt, a8, a_s, ql, "v_w", rows)
        if kv_scales is None:
            sk, sv = _calibrate_kv(rt, k, v, rows, hkv, 0, self.cos, self.sin)
        else:
            sk, sv = (np.broadcast_to(np.asarray(s, np.float32), (hkv,)) for s in kv_scales)
        self.set_kv_scales(layer, sk, sv)
        import torch
        qkv = torch.cat([q, k, v], dim=1).contiguous()
        q8 = empty((rows, D), np.int8)
        qs = empty((rows,), np.float64)
        rt.call("tl_qkv_append", 0, layer, 0, rows, qkv, q8, qs, None)
        att = empty((rows, D), np.float32)
        rt.call("tl_attention", 0, layer, 0, rows, q8, qs, att)
        att8, att_s = _quantize_rows(rt, att, rows, D)
        out = _linear_rows(rt, att8, att_s, ql, "o_w", rows)
        debug: dict[str, Any] = {
            "q_proj": _proj_debug(rt, a, a8, a_s, ql, "q_w", rows, q, capture),
            "k_proj": _proj_debug(rt, a, a8, a_s, ql, "k_w", rows, k, capture),
            "v_proj": _proj_debug(rt, a, a8, a_s, ql, "v_w", rows, v, capture),
            "o_proj": _proj_debug(rt, att, att8, att_s, ql, "o_w", rows, out, capture),
            "q_proj_fp": host(q), "k_proj_fp": host(k), "v_proj_fp": host(v),
            "kv_scales": (np.array(sk, np.float32), np.array(sv, np.float32)),
        }
        if capture:
            debug.update({"attended_fp": host(att), "out_fp": host(out)})
        return out, (att8, att_s), debug

    def feed_forward(self, ql: _QLayer, f, f8, f_s, rows: int, capture: bool):
        rt, F = self.rt, self.ours["intermediate"]
        gate = _linear_rows(rt, f8, f_s, ql, "gate_w", rows)
        up = _linear_rows(rt, f8, f_s, ql, "up_w", rows)
        hid = empty((rows, F), np.float32)
        rt.call("tl_silu_mul", gate, up, rows * F, hid)
        h8, h_s = _quantize_rows(rt, hid, rows, F)
        out = _linear_rows(rt, h8, h_s, ql, "down_w", rows)
        debug: dict[str, Any] = {
            "gate_proj": _proj_debug(rt, f, f8, f_s, ql, "gate_w", rows, gate, capture),
            "up_proj": _proj_debug(rt, f, f8, f_s, ql, "up_w", rows, up, capture),
            "down_proj": _proj_debug(rt, hid, h8, h_s, ql, "down_w", rows, out, capture),
            "gate_proj_fp": host(gate), "up_proj_fp": host(up), "hidden_fp": host(hid),
        }
        if capture:
            debug["out_fp"] = host(out)
        return out, (h8, h_s), debug

    def norm(self, x, g, rows: int):
        D = self.ours["hidden"]
        y = empty((rows, D), np.float32)
        q8 = empty((rows, D), np.int8)
        s = empty((rows,), np.float64)
        self.rt.call("tl_rmsnorm_quant", x, g, rows, D, y, q8, s)
        return y, q8, s

    def decoder_layer(self, ql: _QLayer, layer: int, x, rows: int, kv_scales, capture: bool):
        """GI:256-281 on the INT8 path; residual adds happen in the O and down
        GEMM epilogues exactly as in the fused kernels."""
        rt = self.rt
        a, a8, a_s = self.norm(x, ql.g_in, rows)
        attn_out, (att8, att_s), attn_debug = self.attention(ql, layer, a, a8, a_s, rows, kv_scales, capture)
        x1 = _linear_rows(rt, att8, att_s, ql, "o_w", rows, residual=x)
        f, f8, f_s = self.norm(x1, ql.g_post, rows)
        ffn_out, (h8, h_s), ffn_debug = self.feed_forward(ql, f, f8, f_s, rows, capture)
        out = _linear_rows(rt, h8, h_s, ql, "down_w", rows, residual=x1)
        debug: dict[str, Any] = {"attn_input_fp": host(a), "x_after_attn_fp": host(x1), "ffn_input_fp": host(f),
                                 "attn": attn_debug, "ffn": ffn_debug}
        if capture:
            debug["layer_out_fp"] = host(out)
        return out, debug


_LAYER_MODELS: dict = {}


def _layer_model(cfg: dict, cos, sin) -> _Model:
    key = (cfg["hidden_size"], cfg["intermediate_size"], cfg["num_attention_heads"], cfg["num_key_value_heads"],
           cfg["max_position_embeddings"], float(np.float32(cfg["rms_norm_eps"])),
           hash(np.asarray(cos[:8], np.float32).tobytes()))
    m = _LAYER_MODELS.get(key)
    if m is None:
        m = _Model(cfg, 1, 64, cos, sin)
        _LAYER_MODELS[key] = m
    return m


def _rows_of(x: np.ndarray, D: int) -> tuple[np.ndarray, int]:
    x_fp = np.asarray(x, dtype=np.float32)
    if x_fp.ndim != 2 or x_fp.shape[1] != D:
        raise ValueError(f"x must be [seq, {D}]")
    return np.ascontiguousarray(x_fp), x_fp.shape[0]


def mixed_precision_self_attention(x: np.ndarray, layer: dict, cfg: dict, cos: np.ndarray, sin: np.ndarray,
                                   capture_arrays: bool = False, kv_scales=None) -> tuple[np.ndarray, dict[str, Any]]:
    """GI:136-182 on the INT8 path: x [seq][D] (the normed attention input) at
    positions 0..seq-1, causal GQA attention over the INT8 cache."""
    m = _layer_model(cfg, cos, sin)
    x_fp, rows = _rows_of(x, cfg["hidden_size"])
    if rows > cfg["max_position_embeddings"]:
        raise ValueError(f"Sequence length {rows} exceeds max_position_embeddings={cfg['max_position_embeddings']}")
    ql = _QLayer(m.rt, layer)
    a = dev(x_fp)
    a8, a_s = _quantize_rows(m.rt, a, rows, cfg["hidden_size"])
    out, _, debug = m.attention(ql, 0, a, a8, a_s, rows, kv_scales, capture_arrays)
    return host(out), debug


def mixed_precision_feed_forward(x: np.ndarray, layer: dict,
                                 capture_arrays: bool = False) -> tuple[np.ndarray, dict[str, Any]]:
    """GI:205-225 on the INT8 path: SiLU(gate) * up, then down."""
    _check_no_bias(layer)
    x_fp = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    squeeze = x_fp.ndim == 1
    x2 = x_fp.reshape(-1, x_fp.shape[-1])
    rows, D = x2.shape
    F = np.asarray(layer["gate_w"]).shape[1]
    # a handle of this width (any head split the library accepts); the
    # feed-forward uses no KV cache or RoPE rows
    heads = D // 64
    kv = next(g for g in range(1, heads + 1) if heads % g == 0 and heads // g <= 8)
    cfg = {"hidden_size": D, "intermediate_size": F, "num_attention_heads": heads, "num_key_value_heads": kv,
           "head_dim": 64, "max_position_embeddings": 1, "rms_norm_eps": 1e-5}
    m = _layer_model(cfg, *build_rope_cache(1, 64, 10000.0))
    ql = _QLayer(m.rt, layer)
    f = dev(x2)
    f8, f_s = _quantize_rows(m.rt, f, rows, D)
    out, _, debug = m.feed_forward(ql, f, f8, f_s, rows, capture_arrays)
    out_h = host(out)
    return (out_h[0] if squeeze else out_h), debug


def mixed_precision_decoder_layer(x: np.ndarray, layer: dict, cfg: dict, cos: np.ndarray, sin: np.ndarray,
                                  capture_arrays: bool = False, kv_scales=None) -> tuple[np.ndarray, dict[str, Any]]:
    """GI:256-281 on the INT8 path for x [seq][D] at positions 0..seq-1."""
    m = _layer_model(cfg, cos, sin)
    x_fp, rows = _rows_of(x, cfg["hidden_size"])
    if rows > cfg["max_position_embeddings"]:
        raise ValueError(f"Sequence length {rows} exceeds max_position_embeddings={cfg['max_position_embeddings']}")
    ql = _QLayer(m.rt, layer)
    out, debug = m.decoder_layer(ql, 0, dev(x_fp), rows, kv_scales, capture_arrays)
    return host(out), debug


# ---------------------------------------------------------------------------
# GI:91-133, 185-203, 228-253, 408-434: the float32 reference the analysis
# report compares against, on the library's float32 kernels (TL:106-197)
# ---------------------------------------------------------------------------
def _ref_attention_dev(rt: Runtime, a, layer: dict, cfg: dict, cos, sin, rows: int, capture: bool):
    att, parts = TL.self_attention_dev(rt, a, layer, cfg, cos, sin, rows, capture)
    out = TL.linear_dev(rt, att, layer["o_w"], layer.get("o_b"), rows)
    debug: dict[str, Any] = {"q_proj_fp": host(parts["q"]), "k_proj_fp": host(parts["k"]),
                             "v_proj_fp": host(parts["v"])}
    if capture:
        debug.update({"scores_fp": host(parts["scores"]), "weights_fp": host(parts["weights"]),
                      "attended_fp": host(att), "out_fp": host(out)})
    return att, out, debug


def _ref_ffn_dev(rt: Runtime, f, layer: dict, rows: int, capture: bool):
    out, gate, up, hid = TL.feed_forward_dev(rt, f, layer, rows)
    debug: dict[str, Any] = {"gate_proj_fp": host(gate), "up_proj_fp": host(up), "hidden_fp": host(hid)}
    if capture:
        debug["out_fp"] = host(out)
    return hid, out, debug


def reference_self_attention(x: np.ndarray, layer: dict, cfg: dict, cos: np.ndarray, sin: np.ndarray,
                             capture_arrays: bool = False) -> tuple[np.ndarray, dict[str, Any]]:
    """GI:91-133: float32 self-attention of x [seq][D] with its debug dict."""
    x_fp, rows = _rows_of(x, cfg["hidden_size"])
    _, out, debug = _ref_attention_dev(TL._float_runtime(cfg), dev(x_fp), layer, cfg, cos, sin, rows,
                                       capture_arrays)
    return host(out), debug


def reference_feed_forward(x: np.ndarray, layer: dict,
                           capture_arrays: bool = False) -> tuple[np.ndarray, dict[str, Any]]:
    """GI:185-202: float32 SwiGLU feed-forward with its debug dict."""
    x_fp = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    x2 = x_fp.reshape(-1, x_fp.shape[-1])
    _, out, debug = _ref_ffn_dev(op_runtime(), dev(x2), layer, x2.shape[0], capture_arrays)
    lead = x_fp.shape[:-1]
    debug = {k: v.reshape(lead + (-1,)) for k, v in debug.items()}
    return host(out).reshape(lead + (-1,)), debug


def reference_decoder_layer(x: np.ndarray, layer: dict, cfg: dict, cos: np.ndarray, sin: np.ndarray,
                            capture_arrays: bool = False) -> tuple[np.ndarray, dict[str, Any]]:
    """GI:228-253: the float32 decoder layer with its debug dict.  The
    residual adds run in the projections' epilogues (x + (a @ W + b), the
    reference's rounding); the projections are recomputed for that."""
    rt = TL._float_runtime(cfg)
    x_fp, rows = _rows_of(x, cfg["hidden_size"])
    D = cfg["hidden_size"]
    xd = dev(x_fp)
    a = TL.rms_norm_dev(rt, xd, layer["input_norm_w"], rows, D)
    att, _, attn_debug = _ref_attention_dev(rt, a, layer, cfg, cos, sin, rows, capture_arrays)
    x1 = TL.linear_dev(rt, att, layer["o_w"], layer.get("o_b"), rows, residual=xd)
    f = TL.rms_norm_dev(rt, x1, layer["post_norm_w"], rows, D)
    hid, _, ffn_debug = _ref_ffn_dev(rt, f, layer, rows, capture_arrays)
    out = host(TL.linear_dev(rt, hid, layer["down_w"], layer.get("down_b"), rows, residual=x1))
    debug: dict[str, Any] = {"attn_input_fp": host(a), "x_after_attn_fp": host(x1), "ffn_input_fp": host(f),
                             "attn": attn_debug, "ffn": ffn_debug}
    if capture_arrays:
        debug["layer_out_fp"] = out
    return out, debug


def forward_reference(token_ids, weights: TinyLlamaWeights, cos: np.ndarray, sin: np.ndarray,
                      layer_count: int) -> np.ndarray:
    """GI:408-434: float32 logits [seq][V] over the first layer_count layers."""
    return TL.forward(list(token_ids), weights, cos, sin, layer_count=layer_count)


# ---------------------------------------------------------------------------
# whole model: one device-resident engine per weight archive
# ---------------------------------------------------------------------------
class _Engine(_Model):
    """All layers, the INT8 LM head and the INT8 embedding of one archive."""

    def __init__(self, weights: TinyLlamaWeights, layer_count: int, cos, sin):
        cfg = weights.cfg
        super().__init__(cfg, layer_count, cfg["vocab_size"], cos, sin)
        rt = self.rt
        self.layers = []
        for i in range(layer_count):
            ql = _QLayer(rt, weights.layer(i))
            ql.load_into(rt, i)
            self.layers.append(ql)
        V, D = cfg["vocab_size"], cfg["hidden_size"]

        def rows_q(w_rows):
            n, k = w_rows.shape
            q = empty((n, k), np.int8)
            s = empty((n,), np.float32)
            rt.call("tl_quantize_weight_rows", dev(np.ascontiguousarray(w_rows, np.float32)), n, k, q, s)
            return q, s

        self.lm_w, self.lm_s = rows_q(np.asarray(weights.lm_head_w(), np.float32).T)
        self.g_final = dev(np.asarray(weights.final_norm_w(), np.float32))
        rt.call("tl_load_lm_head", self.lm_w, self.lm_s, self.g_final, 1)
        self.emb, self.emb_s = rows_q(np.asarray(weights._array("embed_w"), np.float32))
        rt.call("tl_load_embedding", self.emb, self.emb_s, 1)
        self.calibrated = False
        scales = weights.kv_scales()
        if scales is not None:
            self.sk[:] = scales[0][:layer_count]
            self.sv[:] = scales[1][:layer_count]
            rt.call("tl_set_kv_scales", self.sk, self.sv)
            self.calibrated = True
        self.V, self.D = V, D

    def staged_forward(self, token_ids: np.ndarray):
        """Embedding, every layer (calibrating its KV scales on the way), final
        RMSNorm and the INT8 LM head over all rows: logits [seq][V] (device)."""
        rt, rows = self.rt, token_ids.size
        x = empty((rows, self.D), np.float32)
        rt.call("tl_embed", dev(token_ids.astype(np.int32)), rows, x)
        for i, ql in enumerate(self.layers):
            scales = None if not self.calibrated else (self.sk[i], self.sv[i])
            x, _ = self.decoder_layer(ql, i, x, rows, scales, False)
        self.calibrated = True
        _, x8, xs = self.norm(x, self.g_final, rows)
        logits = empty((rows, self.V), np.float32)
        rt.call("tl_gemm_i8_dequant", x8, xs, self.lm_w, self.lm_s, rows, self.V, self.D, None, logits)
        return logits

    def forward(self, token_ids: np.ndarray) -> np.ndarray:
        if not self.calibrated:
            return host(self.staged_forward(token_ids))
        logits = empty((token_ids.size, self.V), np.float32)
        self.rt.call("tl_prefill_logits", 0, np.ascontiguousarray(token_ids, np.int32), token_ids.size, logits)
        return host(logits)


_ENGINES: dict = {}


def _engine(weights: TinyLlamaWeights, layer_count: int, cos, sin) -> _Engine:
    key = (id(weights), layer_count)
    e = _ENGINES.get(key)
    if e is None or e.weights_ref is not weights:
        e = _Engine(weights, layer_count, cos, sin)
        e.weights_ref = weights
        _ENGINES[key] = e
    return e


def validate_layer_count(cfg: dict, layer_count: int) -> None:
    if layer_count < 1 or layer_count > cfg["num_hidden_layers"]:
        raise ValueError(f"--layers must be between 1 and {cfg['num_hidden_layers']}")


def forward_mixed(token_ids, weights: TinyLlamaWeights, cos: np.ndarray, sin: np.ndarray, layer_count: int,
                  quantize_lm_head: bool) -> np.ndarray:
    """GI:437-467: logits [seq][V] of every position, on the INT8 path."""
    cfg = weights.cfg
    seq = len(token_ids)
    if seq > cfg["max_position_embeddings"]:
        raise ValueError(f"Sequence length {seq} exceeds max_position_embeddings={cfg['max_position_embeddings']}")
    if not quantize_lm_head:
        raise ValueError("the MI355X path runs the INT8 LM head: pass quantize_lm_head=True")
    if seq == 0:
        raise ValueError("Input token sequence is empty")
    validate_layer_count(cfg, layer_count)
    ids = np.asarray(token_ids, dtype=np.int32)
    return _engine(weights, layer_count, cos, sin).forward(ids)


def parse_token_ids(token_ids_arg: str | None) -> list[int] | None:
    """GI:340-348 interface: "1, 2,3" -> [1, 2, 3]; None stays None."""
    if token_ids_arg is None:
        return None
    fields = (f.strip() for f in token_ids_arg.split(","))
    return [int(f) for f in fields if f]


def resolve_token_ids(prompt: str | None, token_ids_arg: str | None, tokenizer) -> list[int]:
    """GI:361-375 interface: explicit ids win, else the prompt is tokenized;
    the reference's ValueError texts for a missing or empty input."""
    ids = parse_token_ids(token_ids_arg)
    if ids is None:
        if prompt is None:
            raise ValueError("Provide either --prompt or --token-ids")
        if tokenizer is None:
            raise ValueError("Tokenizer unavailable, so --token-ids is required")
        ids = list(tokenizer.encode(prompt))
    if len(ids) == 0:
        raise ValueError("Input token sequence is empty")
    return ids


def run_generate(prompt: str | None, token_ids_arg: str | None, weights_path, layer_count: int, max_tokens: int,
                 local_files_only: bool = True, quantize_lm_head: bool = True, cache_arrays: bool = False,
                 tokenizer=None, eos_token_id: int | None = None) -> list[int]:
    """GI:629-685 on the INT8 path: the prompt is prefilled once and each new
    token is one decode step over the KV cache (the reference recomputes the
    whole prefix per token).  Prints the reference's lines and returns the
    prompt followed by the generated ids.  ``weights_path`` may also be a
    TinyLlamaWeights.  No tokenizer is loaded (no network); pass one to get
    text."""
    if max_tokens < 1:
        raise ValueError("--max-tokens must be at least 1")
    if not quantize_lm_head:
        raise ValueError("the MI355X path runs the INT8 LM head: pass quantize_lm_head=True")
    weights = weights_path if isinstance(weights_path, TinyLlamaWeights) else load_weights(
        weights_path, cache_arrays=cache_arrays)
    cfg = weights.cfg
    validate_layer_count(cfg, layer_count)
    token_ids = resolve_token_ids(prompt, token_ids_arg, tokenizer)
    if len(token_ids) + max_tokens > cfg["max_position_embeddings"]:
        raise ValueError(f"Sequence length {len(token_ids) + max_tokens} exceeds "
                         f"max_position_embeddings={cfg['max_position_embeddings']}")
    cos, sin = build_rope_cache(cfg["max_position_embeddings"], cfg["head_dim"], cfg["rope_theta"])
    print(f"Token ids: {token_ids}")
    print("")
    if layer_count != cfg["num_hidden_layers"]:
        print(f"Generating with {layer_count} / {cfg['num_hidden_layers']} decoder layers. "
              "Use the full layer count for normal TinyLlama behavior.")
        print("")
    eng = _engine(weights, layer_count, cos, sin)
    ids = np.asarray(token_ids, dtype=np.int32)
    if not eng.calibrated:
        eng.staged_forward(ids)
    import ctypes as C
    out = np.empty(max_tokens, np.int32)
    n, stop = C.c_int32(), C.c_int32()
    eos = -1 if eos_token_id is None else int(eos_token_id)
    eng.rt.check(eng.rt.lib.tl_generate(eng.rt.h, 0, ids.ctypes.data, ids.size, max_tokens, eos, None,
                                        out.ctypes.data, C.byref(n), C.byref(stop)), "tl_generate")
    generated = list(token_ids)
    for step, tok in enumerate(out[:n.value].tolist()):
        generated.append(tok)
        piece = "" if tokenizer is None else tokenizer.decode([tok])
        print(f"  step {step + 1:2d}: token {tok:6d} -> '{piece.encode('unicode_escape').decode('ascii')}'")
        if eos_token_id is not None and tok == eos_token_id:
            print("  [EOS]")
    print("")
    print(f"Output token ids: {generated}")
    return generated


# ---------------------------------------------------------------------------
# The analysis report and the command line (GI:284-338, 351-353, 401-405,
# 470-626, 688-745).  What is kept from the reference is its interface: the
# CLI flags, the ValueError texts, the printed and summary line formats and
# the key schema of debug_arrays.npz (nested debug dicts joined with "_").
# The report is assembled from per-layer comparison records; both models run
# on the device (float32 kernels for the reference model, the INT8 path for
# the mixed one).
# ---------------------------------------------------------------------------
def safe_repr(text: str) -> str:
    """Printable ASCII form of token text (GI:290-291 format)."""
    return text.encode("unicode_escape").decode("ascii")


def decode_token(tokenizer, token_id: int) -> str:
    """Text of one token id; empty without a tokenizer (GI:284-287)."""
    return tokenizer.decode([int(token_id)]) if tokenizer is not None else ""


def top_tokens(logits: np.ndarray, tokenizer, k: int) -> list[tuple[int, float, str]]:
    """The k largest logits of a row as (id, logit, text), largest first
    (GI:294-299).  A partial partition finds the k, a sort orders them."""
    row = np.asarray(logits, dtype=np.float32).ravel()
    k = max(0, min(int(k), row.size))
    if k == 0:
        return []
    best = np.argpartition(row, row.size - k)[row.size - k:]
    best = best[np.argsort(-row[best], kind="stable")]
    return [(int(i), float(row[i]), decode_token(tokenizer, int(i))) for i in best]


def flatten_named_arrays(prefix: str, obj: Any) -> dict[str, np.ndarray]:
    """Nested debug dicts -> {"outer_inner_leaf": array} (the GI:302-310 key
    schema); leaves that are not arrays are left out."""
    flat: dict[str, np.ndarray] = {}
    pending = [(prefix, obj)]
    while pending:
        name, node = pending.pop()
        if isinstance(node, np.ndarray):
            flat[name] = node
        elif isinstance(node, dict):
            pending.extend(((f"{name}_{key}" if name else str(key)), child) for key, child in node.items())
    return flat


def dump_debug(dump_dir: str, token_ids: list[int], reference_debug: dict[str, Any], mixed_debug: dict[str, Any],
               summary_lines: list[str]) -> None:
    """Write debug_arrays.npz (token_ids, reference_*, mixed_*) and
    summary.txt into dump_dir (the GI:313-327 files)."""
    os.makedirs(dump_dir, exist_ok=True)
    payload = {"token_ids": np.asarray(token_ids, dtype=np.int32)}
    for side, tree in (("reference", reference_debug), ("mixed", mixed_debug)):
        payload.update(flatten_named_arrays(side, tree))
    np.savez(os.path.join(dump_dir, "debug_arrays.npz"), **payload)
    with open(os.path.join(dump_dir, "summary.txt"), "w", encoding="utf-8") as out:
        out.write("".join(line + "\n" for line in summary_lines))


def maybe_load_tokenizer(model_id: str, local_files_only: bool):
    """A tokenizer from the local cache, or None with a warning (GI:330-337
    behaviour; nothing is ever downloaded)."""
    try:
        from transformers import AutoTokenizer
        return AutoTokenizer.from_pretrained(model_id, local_files_only=local_files_only)
    except Exception as exc:   # transformers missing, or nothing cached
        print(f"Warning: could not load tokenizer for {model_id}: {exc}")
        return None


def projection_stats_line(name: str, ref_array: np.ndarray, mix_array: np.ndarray) -> str:
    """One line of the projection breakdown (GI:351-353 format)."""
    st = diff_stats(ref_array, mix_array)
    return f"{name}: mae={st['mae']:.6f}, max_abs={st['max_abs']:.6f}"


def print_token_context(token_ids: list[int], tokenizer) -> None:
    """The report's opening lines (GI:401-405 format)."""
    lines = [f"Token ids: {token_ids}"]
    if tokenizer is not None:
        lines.append(f"Decoded tokens: {[safe_repr(decode_token(tokenizer, t)) for t in token_ids]}")
    print("\n".join(lines + [""]))


# projection breakdown of the dumped layer: (debug block, key, label); the
# O and down rows are shown when both models captured them
_BREAKDOWN = (("attn", "q_proj_fp", "attn q_proj"), ("attn", "k_proj_fp", "attn k_proj"),
              ("attn", "v_proj_fp", "attn v_proj"), ("ffn", "gate_proj_fp", "ffn gate_proj"),
              ("ffn", "up_proj_fp", "ffn up_proj"), ("attn", "out_fp", "attn o_proj"),
              ("ffn", "out_fp", "ffn down_proj"))


class _Report:
    """Lines of an analysis run: ``say`` prints, ``note`` keeps a line for
    summary.txt, ``both`` does both."""

    def __init__(self, token_ids: list[int], layer_count: int):
        self.kept = [f"Token ids: {token_ids}", f"Layers analyzed: {layer_count}", "Layer stats:"]

    def say(self, line: str = "") -> None:
        print(line)

    def note(self, line: str) -> None:
        self.kept.append(line)

    def both(self, line: str) -> None:
        self.say(line)
        self.note(line)


class _LayerComparison:
    """Walks the decoder layers with the float32 model and the INT8 path side
    by side.  Each layer is compared twice: isolated (the INT8 layer fed the
    float32 model's input) and cumulative (the INT8 path fed its own previous
    output).  The dumped layer keeps both models' debug dicts."""

    def __init__(self, weights: TinyLlamaWeights, token_ids: list[int], cos, sin, dump_layer: int | None):
        self.w = weights
        self.cos, self.sin = cos, sin
        self.dump_layer = dump_layer
        self.float_x = np.asarray(weights.embed(token_ids), np.float32)
        self.int8_x = self.float_x.copy()
        self.kv = weights.kv_scales()
        self.dumped: tuple[dict, dict] | None = None

    def step(self, index: int) -> tuple[dict, dict, list[str]]:
        layer = self.w.layer(index)
        cfg = self.w.cfg
        keep = index == self.dump_layer
        kv = None if self.kv is None else (self.kv[0][index], self.kv[1][index])
        f_out, f_dbg = reference_decoder_layer(self.float_x, layer, cfg, self.cos, self.sin, capture_arrays=keep)
        iso, iso_dbg = mixed_precision_decoder_layer(self.float_x, layer, cfg, self.cos, self.sin,
                                                     capture_arrays=keep, kv_scales=kv)
        cum, _ = mixed_precision_decoder_layer(self.int8_x, layer, cfg, self.cos, self.sin, kv_scales=kv)
        lines: list[str] = []
        if keep:
            self.dumped = (f_dbg, iso_dbg)
            for block, key, label in _BREAKDOWN:
                if key in f_dbg[block] and key in iso_dbg[block]:
                    lines.append(projection_stats_line("  " + label, f_dbg[block][key], iso_dbg[block][key]))
        isolated, cumulative = diff_stats(f_out, iso), diff_stats(f_out, cum)
        self.float_x, self.int8_x = f_out, cum
        return isolated, cumulative, lines

    def final_logits(self, quantize_lm_head: bool, keep_debug: bool):
        """Final RMSNorm of each model's last hidden rows, then the LM head of
        the last position: float32 for the reference model; for the INT8 path
        the per-tensor quantized_linear (GI:59-88) when quantize_lm_head."""
        eps = self.w.cfg["rms_norm_eps"]
        g = self.w.final_norm_w()
        head = self.w.lm_head_w()
        ref_logits = TL.linear(TL.rms_norm(self.float_x, g, eps)[-1:], head)
        last = TL.rms_norm(self.int8_x, g, eps)[-1:]
        if quantize_lm_head:
            mix_logits, dbg = quantized_linear(last, head, None, capture_arrays=keep_debug)
            return ref_logits, mix_logits, dbg
        return ref_logits, TL.linear(last, head), {}


def run_analysis(prompt: str | None, token_ids_arg: str | None, weights_path, layer_count: int,
                 dump_layer: int | None = None, dump_dir: str | None = None, local_files_only: bool = True,
                 top_k: int = 5, quantize_lm_head: bool = False, cache_arrays: bool = False,
                 tokenizer=None) -> dict:
    """The GI:470-626 analysis: the float32 model and the INT8 path over the
    prompt, compared layer by layer and on the final logits of the last
    position; with dump_layer, that layer's debug dicts (and the quantized LM
    head's) are written to dump_dir.  The INT8 layers use the archive's static
    KV scales when it has them, else scales calibrated on the prompt.
    ``weights_path`` may also be a TinyLlamaWeights.  Returns the summary
    lines, both next tokens and both logit rows."""
    weights = weights_path if isinstance(weights_path, TinyLlamaWeights) else load_weights(
        weights_path, cache_arrays=cache_arrays)
    cfg = weights.cfg
    validate_layer_count(cfg, layer_count)
    wants_text = prompt is not None and token_ids_arg is None
    if tokenizer is None and wants_text:
        tokenizer = maybe_load_tokenizer(cfg["model_id"], local_files_only=local_files_only)
    token_ids = resolve_token_ids(prompt, token_ids_arg, tokenizer)
    if dump_layer is not None and not 0 <= dump_layer < layer_count:
        raise ValueError("--dump-layer must be within the executed layer range")
    cos, sin = build_rope_cache(cfg["max_position_embeddings"], cfg["head_dim"], cfg["rope_theta"])
    print_token_context(token_ids, tokenizer)

    rep = _Report(token_ids, layer_count)
    walk = _LayerComparison(weights, token_ids, cos, sin, dump_layer)
    for index in range(layer_count):
        iso, cum, breakdown = walk.step(index)
        rep.both(f"Layer {index}: isolated MAE={iso['mae']:.6f}, isolated max={iso['max_abs']:.6f}, "
                 f"cumulative MAE={cum['mae']:.6f}, cumulative max={cum['max_abs']:.6f}")
        for line in breakdown:
            rep.both(line)

    ref_logits, mix_logits, lm_dbg = walk.final_logits(quantize_lm_head, keep_debug=dump_dir is not None)
    st = diff_stats(ref_logits, mix_logits)
    picks = {"Float32": int(np.argmax(ref_logits[0])), "INT8 path": int(np.argmax(mix_logits[0]))}
    token_lines = [f"{who} next token: {tok} -> '{safe_repr(decode_token(tokenizer, tok))}'"
                   for who, tok in picks.items()]
    rep.say()
    rep.say(f"Final logits: MAE={st['mae']:.6f}, RMSE={st['rmse']:.6f}, max_abs={st['max_abs']:.6f}")
    for line in token_lines:
        rep.say(line)
    for title, row in ((f"Top {top_k} float32 tokens:", ref_logits[0]), (f"Top {top_k} INT8-path tokens:", mix_logits[0])):
        rep.say()
        rep.say(title)
        for tok, value, text in top_tokens(row, tokenizer, top_k):
            rep.say(f"  {tok:6d}  {value:12.6f}  '{safe_repr(text)}'")
    rep.note("")
    rep.note(f"Final logits: mae={st['mae']:.6f}, rmse={st['rmse']:.6f}, max_abs={st['max_abs']:.6f}")
    for line in token_lines:
        rep.note(line)

    if dump_dir is not None:
        f_dbg, m_dbg = walk.dumped if walk.dumped is not None else ({}, {})
        if lm_dbg:
            m_dbg = {**m_dbg, "lm_head": lm_dbg}
        dump_debug(dump_dir, token_ids, f_dbg, m_dbg, rep.kept)
        rep.say()
        rep.say(f"Saved debug dump to {dump_dir}")
    return {"summary_lines": rep.kept, "ref_token": picks["Float32"], "mix_token": picks["INT8 path"],
            "ref_logits": ref_logits, "mix_logits": mix_logits}


def build_arg_parser():
    """The reference's command line (GI:688-717 flags and defaults; --weights
    is required here: no weight archive ships with the package)."""
    import argparse
    ap = argparse.ArgumentParser(description="INT8 TinyLlama decoder path on MI355X: float32-vs-INT8 analysis "
                                             "or greedy generation")
    ap.add_argument("--mode", choices=["analysis", "generate"], default="analysis",
                    help="analysis = one-pass float32 vs INT8 comparison, generate = autoregressive INT8-path "
                         "generation")
    for flag, kind, default in (("--prompt", str, None), ("--token-ids", str, None), ("--layers", int, 1),
                                ("--max-tokens", int, 20), ("--dump-layer", int, None), ("--dump-dir", str, None),
                                ("--top-k", int, 5)):
        ap.add_argument(flag, type=kind, default=default)
    ap.add_argument("--weights", type=str, required=True)
    for flag in ("--local-files-only", "--cache-arrays"):
        ap.add_argument(flag, action="store_true")
    ap.add_argument("--quantize-lm-head", action="store_true",
                    help="Also quantize the final vocab projection (always on in --mode generate).")
    return ap


def main(argv: list[str] | None = None) -> None:
    """Command-line entry: --mode analysis (run_analysis) or --mode generate
    (run_generate)."""
    args = build_arg_parser().parse_args(argv)
    if not os.path.exists(args.weights):
        raise FileNotFoundError(f"Weights not found at {args.weights}. Run model/tinyllama.py --save-weights first.")
    if args.mode == "analysis":
        run_analysis(args.prompt, args.token_ids, args.weights, args.layers, dump_layer=args.dump_layer,
                     dump_dir=args.dump_dir, local_files_only=args.local_files_only, top_k=args.top_k,
                     quantize_lm_head=args.quantize_lm_head, cache_arrays=args.cache_arrays)
        return
    if args.dump_layer is not None or args.dump_dir is not None:
        raise ValueError("--dump-layer and --dump-dir are only supported in --mode analysis")
    tokenizer = None
    if args.prompt is not None and args.token_ids is None:
        tokenizer = maybe_load_tokenizer(load_weights(args.weights).cfg["model_id"], args.local_files_only)
    run_generate(args.prompt, args.token_ids, args.weights, args.layers, args.max_tokens,
                 local_files_only=args.local_files_only, quantize_lm_head=True, cache_arrays=args.cache_arrays,
                 tokenizer=tokenizer)
