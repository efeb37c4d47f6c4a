"""Model construction helpers shared by the tests (host-side NumPy only).

``tiny_from_golden`` rebuilds the small golden model whose vectors are in
tests/golden/tiny_model.npz; ``synthetic`` draws a seeded random model of any
geometry with the per-output-channel quantization the configurations use.
"""
from __future__ import annotations

import numpy as np

from conftest import golden
import oracle
from oracle import ModelArrays

WEIGHT_NAMES = ("q_w", "k_w", "v_w", "o_w", "gate_w", "up_w", "down_w")


def rope_cache(max_pos, hd, theta):
    """RoPE table through the product's own builder (lpta.tinyllama)."""
    import lpta
    return lpta.build_rope_cache(max_pos, hd, theta)


def tiny_from_golden(kv_sk=None, kv_sv=None):
    z = golden("tiny_model.npz")
    D, F, L, H, Hkv, hd, V, max_pos = (int(v) for v in z["cfg"])
    cfg = dict(hidden=D, intermediate=F, n_layers=L, n_heads=H, n_kv_heads=Hkv, head_dim=hd,
               vocab=V, max_pos=max_pos, rms_eps=np.float32(1e-5), rope_theta=10000.0)
    ws = np.float32(z["w_scale"])
    layers = []
    for i in range(L):
        w = [np.ascontiguousarray(z[f"layer{i}_{n}_q"].T) for n in WEIGHT_NAMES]
        s = [np.full(m.shape[0], ws, np.float32) for m in w]
        layers.append(dict(w=w, s=s, g_in=np.ascontiguousarray(z[f"layer{i}_input_norm_w"]),
                           g_post=np.ascontiguousarray(z[f"layer{i}_post_norm_w"])))
    cos, sin = rope_cache(max_pos, hd, 10000.0)
    sk = np.full((L, Hkv), 0.05, np.float32) if kv_sk is None else np.ascontiguousarray(kv_sk, np.float32)
    sv = np.full((L, Hkv), 0.05, np.float32) if kv_sv is None else np.ascontiguousarray(kv_sv, np.float32)
    return ModelArrays(cfg=cfg, layers=layers, lm_w=np.ascontiguousarray(z["lm_head_w_q"].T),
                       lm_s=np.full(V, ws, np.float32), g_final=np.ascontiguousarray(z["final_norm_w"]),
                       emb=np.ascontiguousarray(z["embed_q"]), emb_s=np.ascontiguousarray(z["embed_s"]),
                       rope_cos=cos, rope_sin=sin, kv_sk=sk, kv_sv=sv), z


synthetic = oracle.synthetic_model


SMALL = oracle.SMALL_CFG
TINYLLAMA = oracle.TINYLLAMA_CFG
