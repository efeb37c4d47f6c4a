"""The reference's Python operator surface on the GPU (lpta.tinyllama,
lpta.tinyllama_gemm_int8).  Operator-level functions are compared with the
golden vectors of model/tinyllama.py / model/tinyllama_gemm_int8.py; the
layer- and model-level functions (INT8 KV-cache path) bit for bit with the CPU
oracle and with the library's fused kernels."""
import numpy as np
import pytest

import oracle
from conftest import golden
from gpu_util import assert_bits_equal

pytestmark = pytest.mark.gpu
F32 = np.float32
NAMES = ("q_w", "k_w", "v_w", "o_w", "gate_w", "up_w", "down_w")


def gi():
    import lpta.tinyllama_gemm_int8 as m
    return m


def tl():
    import lpta.tinyllama as m
    return m


# ---- operator level: golden vectors --------------------------------------------------------

def test_quantize_int8_vs_golden():
    z = golden("quantize.npz")
    for name in ("normal", "wide", "ties", "zeros", "tiny"):
        q, s = gi().quantize_int8(z[f"x_{name}"])
        assert_bits_equal(q, z[f"q_{name}"], name)
        assert s == float(z[f"s_{name}"]), name
    y = gi().dequantize_int32(z["deq_acc"], float(z["deq_sx"]), float(z["deq_sw"]))
    assert_bits_equal(y, z["deq_y"], "dequantize_int32")


def test_quantized_linear_and_dequantize_vs_golden():
    z = golden("quantized_linear.npz")
    out, dbg = gi().quantized_linear(z["x"], z["w"], capture_arrays=True)
    assert_bits_equal(out, z["out"], "out")
    assert_bits_equal(dbg["input_q"], z["input_q"], "input_q")
    assert_bits_equal(dbg["weight_q"], z["weight_q"], "weight_q")
    assert_bits_equal(dbg["accum_int32"], z["accum_int32"], "accum")
    assert dbg["input_scale"].dtype == F32 and dbg["input_scale"][0] == F32(z["input_scale"])
    assert dbg["weight_scale"][0] == F32(z["weight_scale"])
    y = gi().dequantize_int32(z["accum_int32"], float(z["input_scale"]), float(z["weight_scale"]))
    assert_bits_equal(y, z["out"], "dequantize_int32")
    # bias adds in float32 after dequantization (GI:72-73)
    b = np.linspace(-1, 1, z["w"].shape[1]).astype(F32)
    out_b, _ = gi().quantized_linear(z["x"], z["w"], b)
    assert_bits_equal(out_b, (z["out"] + b).astype(F32), "bias")
    # a single row (decode shape) keeps its 1-D shape
    out1, _ = gi().quantized_linear(z["x"][0], z["w"])
    assert out1.shape == (z["w"].shape[1],)


def test_rms_norm_vs_golden():
    from lpta import TlError
    z = golden("rms_norm.npz")
    widths = sorted({int(k.split("_")[1]) for k in z.files if k.startswith("x_")})
    def perfect_tree(n):  # NumPy's pairwise halving splits evenly down to leaves of 8k <= 128
        while n > 128:
            if n % 16:
                return False
            n //= 2
        return n % 8 == 0

    checked = 0
    for n in widths:
        x, w, y = z[f"x_{n}"], z[f"w_{n}"], z[f"y_{n}"]
        if perfect_tree(n):
            assert_bits_equal(tl().rms_norm(x, w, 1e-5), y, f"width {n}")
            checked += 1
        else:
            with pytest.raises(TlError):  # no exact pairwise tree for this width
                tl().rms_norm(x, w, 1e-5)
    assert checked >= 4


def test_rope_vs_golden():
    z = golden("rope.npz")
    cos, sin = tl().build_rope_cache(2048, 64, 10000.0)
    assert_bits_equal(cos[z["positions"]], z["cos"], "cos table")
    qr, kr = tl().apply_rope(z["q"], z["k"], cos, sin)
    assert_bits_equal(qr, z["q_rot"], "q_rot")
    assert_bits_equal(kr, z["k_rot"], "k_rot")


def test_softmax_silu_vs_golden():
    z = golden("softmax_silu.npz")
    for n in (1, 7, 64, 65, 513, 2048):
        p = tl().softmax(z[f"s_{n}"])
        np.testing.assert_allclose(p, z[f"p_{n}"], rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(tl().silu(z["silu_x"]), z["silu_y"], rtol=1e-6, atol=1e-30)


# ---- layer / model level: a small float model in the reference's archive schema ------------

def float_archive(D=256, F=512, L=2, H=4, Hkv=2, V=512, max_pos=128, seed=3):
    rng = np.random.default_rng(seed)
    kvd = Hkv * 64
    a = {"meta_model_id": np.array("synthetic"), "meta_hidden_size": np.array(D),
         "meta_intermediate_size": np.array(F), "meta_num_hidden_layers": np.array(L),
         "meta_num_attention_heads": np.array(H), "meta_num_key_value_heads": np.array(Hkv),
         "meta_head_dim": np.array(64), "meta_vocab_size": np.array(V),
         "meta_max_position_embeddings": np.array(max_pos), "meta_rms_norm_eps": np.array(1e-5, np.float32),
         "meta_rope_theta": np.array(10000.0, np.float32)}
    shapes = {"q_w": (D, D), "k_w": (D, kvd), "v_w": (D, kvd), "o_w": (D, D), "gate_w": (D, F), "up_w": (D, F),
              "down_w": (F, D)}
    for i in range(L):
        for n, shp in shapes.items():
            a[f"layer{i}_{n}"] = (rng.standard_normal(shp) * 0.06).astype(F32)
        a[f"layer{i}_input_norm_w"] = (1 + 0.05 * rng.standard_normal(D)).astype(F32)
        a[f"layer{i}_post_norm_w"] = (1 + 0.05 * rng.standard_normal(D)).astype(F32)
    a["embed_w"] = rng.standard_normal((V, D)).astype(F32)
    a["lm_head_w"] = (rng.standard_normal((D, V)) * 0.06).astype(F32)
    a["final_norm_w"] = (1 + 0.05 * rng.standard_normal(D)).astype(F32)
    return a


def oracle_model(w, qlayers, sk, sv, lm=None, emb=None, g_final=None):
    """oracle.ModelArrays holding exactly the device's quantized weights."""
    import lpta
    c = w.cfg
    cfg = dict(hidden=c["hidden_size"], intermediate=c["intermediate_size"], n_layers=len(qlayers),
               n_heads=c["num_attention_heads"], n_kv_heads=c["num_key_value_heads"], head_dim=64,
               vocab=c["vocab_size"], max_pos=c["max_position_embeddings"], rms_eps=F32(c["rms_norm_eps"]),
               rope_theta=float(c["rope_theta"]))
    layers = [dict(w=[ql.w[n].cpu().numpy() for n in NAMES], s=[ql.s[n].cpu().numpy() for n in NAMES],
                   g_in=ql.g_in.cpu().numpy(), g_post=ql.g_post.cpu().numpy()) for ql in qlayers]
    V, D = cfg["vocab"], cfg["hidden"]
    cos, sin = lpta.build_rope_cache(cfg["max_pos"], 64, cfg["rope_theta"])
    zeros_w = np.zeros((V, D), np.int8)
    return oracle.ModelArrays(cfg=cfg, layers=layers,
                              lm_w=zeros_w if lm is None else lm[0], lm_s=np.ones(V, F32) if lm is None else lm[1],
                              g_final=np.ones(D, F32) if g_final is None else g_final,
                              emb=zeros_w if emb is None else emb[0], emb_s=np.ones(V, F32) if emb is None else emb[1],
                              rope_cos=cos, rope_sin=sin, kv_sk=np.ascontiguousarray(sk, F32),
                              kv_sv=np.ascontiguousarray(sv, F32))


def test_decoder_layer_equals_oracle_and_fused_path():
    """mixed_precision_decoder_layer over 40 positions == oracle token-by-token
    decode == the fused tl_layer_rows kernels, with given static KV scales."""
    w = tl().TinyLlamaWeights.from_arrays(float_archive())
    cfg = w.cfg
    cos, sin = tl().build_rope_cache(cfg["max_position_embeddings"], 64, 10000.0)
    x = np.random.default_rng(4).standard_normal((40, cfg["hidden_size"])).astype(F32)
    sk, sv = np.array([0.02, 0.03], F32), np.array([0.025, 0.015], F32)
    out, dbg = gi().mixed_precision_decoder_layer(x, w.layer(0), cfg, cos, sin, capture_arrays=True,
                                                  kv_scales=(sk, sv))
    assert set(dbg) >= {"attn_input_fp", "x_after_attn_fp", "ffn_input_fp", "attn", "ffn", "layer_out_fp"}
    assert set(dbg["attn"]) >= {"q_proj", "k_proj", "v_proj", "o_proj", "q_proj_fp", "k_proj_fp", "v_proj_fp"}
    assert set(dbg["ffn"]) >= {"gate_proj", "up_proj", "down_proj", "gate_proj_fp", "up_proj_fp", "hidden_fp"}
    assert set(dbg["attn"]["q_proj"]) >= {"input_scale", "weight_scale", "input_q", "weight_q", "accum_int32"}
    # oracle with the very int8 weights the device quantized
    m = gi()._layer_model(cfg, cos, sin)
    ql = gi()._QLayer(m.rt, w.layer(0))
    arrays = oracle_model(w, [ql], sk[None, :], sv[None, :])
    orc = oracle.Oracle(arrays)
    kc, vc = arrays.new_cache()
    want = np.stack([orc.decode_row(0, i, x[i], kc, vc) for i in range(x.shape[0])])
    assert_bits_equal(out, want, "layer output vs oracle")
    # the fused kernels over the same rows
    from lpta.engine import Engine
    import torch
    eng = Engine(dict(arrays.cfg), max_seqs=1)
    eng.load_layer(0, dict(w=[ql.w[n] for n in NAMES], s=[ql.s[n] for n in NAMES], g_in=ql.g_in, g_post=ql.g_post))
    eng.set_kv_scales(sk[None, :], sv[None, :])
    eng.set_rope_table(cos, sin)
    xd = torch.from_numpy(x).cuda()
    eng.rt.call("tl_layer_rows", 0, 0, 0, x.shape[0], xd)
    assert_bits_equal(xd.cpu().numpy(), out, "fused tl_layer_rows")
    for g in range(2):
        k, v = eng.kv_read(0, 0, g, 0, x.shape[0])
        assert_bits_equal(k, kc[0, g, :x.shape[0]], "K rows")
        assert_bits_equal(v, vc[0, g, :x.shape[0]], "V rows")
    eng.close()


def test_kv_scale_calibration():
    """Without kv_scales, each KV head's static scale is f32(max|x| / 127) over
    the sequence's rotated keys / values."""
    w = tl().TinyLlamaWeights.from_arrays(float_archive(seed=9))
    cfg = w.cfg
    cos, sin = tl().build_rope_cache(cfg["max_position_embeddings"], 64, 10000.0)
    x = np.random.default_rng(5).standard_normal((17, cfg["hidden_size"])).astype(F32)
    a = tl().rms_norm(x, w.layer(0)["input_norm_w"], 1e-5)
    _, dbg = gi().mixed_precision_self_attention(a, w.layer(0), cfg, cos, sin)
    sk, sv = dbg["kv_scales"]
    k = dbg["k_proj_fp"]
    v = dbg["v_proj_fp"].reshape(17, 2, 64)
    k_rot = np.stack([oracle.apply_rope(k[t], 2, 64, cos[t], sin[t]) for t in range(17)]).reshape(17, 2, 64)
    for g in range(2):
        assert sk[g] == F32(np.float64(np.abs(k_rot[:, g]).max()) / 127.0)
        assert sv[g] == F32(np.float64(np.abs(v[:, g]).max()) / 127.0)


def test_forward_mixed_and_run_generate_equal_oracle(tmp_path, capsys):
    arch = float_archive(seed=12)
    path = tmp_path / "weights.npz"
    np.savez(path, **arch)
    w = tl().load_weights(str(path))
    cfg = w.cfg
    cos, sin = tl().build_rope_cache(cfg["max_position_embeddings"], 64, cfg["rope_theta"])
    ids = [5, 77, 300, 2, 511, 64, 9]
    logits = gi().forward_mixed(ids, w, cos, sin, 2, quantize_lm_head=True)   # calibrates
    again = gi().forward_mixed(ids, w, cos, sin, 2, quantize_lm_head=True)    # fused tl_prefill_logits
    assert logits.shape == (len(ids), cfg["vocab_size"])
    assert_bits_equal(again, logits, "calibrated staged path vs fused prefill")
    eng = gi()._engine(w, 2, cos, sin)
    arrays = oracle_model(w, eng.layers, eng.sk, eng.sv, lm=(eng.lm_w.cpu().numpy(), eng.lm_s.cpu().numpy()),
                          emb=(eng.emb.cpu().numpy(), eng.emb_s.cpu().numpy()), g_final=eng.g_final.cpu().numpy())
    orc = oracle.Oracle(arrays)
    kc, vc = arrays.new_cache()
    for i, t in enumerate(ids):
        x = orc.embed(t)
        for layer in range(2):
            x = orc.decode_row(layer, i, x, kc, vc)
        _, _, want = orc.lm_head(x, want_logits=True)
        assert_bits_equal(logits[i], want, f"logits row {i}")
    # run_generate: prefill once + KV-cache decode, same ids as the oracle
    got = gi().run_generate(None, ",".join(map(str, ids)), str(path), 2, 6)
    want_ids, _ = orc.generate(np.asarray(ids, np.int32), 6)
    assert got == ids + [int(t) for t in want_ids]
    out = capsys.readouterr().out
    assert out.startswith(f"Token ids: {ids}") and "Output token ids:" in out
    with pytest.raises(ValueError, match="at least 1"):
        gi().run_generate(None, "1,2", str(path), 2, 0)
    with pytest.raises(ValueError, match="--layers must be between"):
        gi().run_generate(None, "1,2", str(path), 3, 2)
    with pytest.raises(ValueError, match="empty"):
        gi().run_generate(None, " , ", str(path), 2, 2)
    with pytest.raises(ValueError, match="exceeds max_position_embeddings"):
        gi().forward_mixed(list(range(200)), w, cos, sin, 2, quantize_lm_head=True)
