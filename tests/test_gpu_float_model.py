"""The float32 model of model/tinyllama.py on the library's float kernels
(tl_linear_f32, tl_attention_f32) and the analysis report built on it
(run_analysis with its per-layer debug dump, GI:302-327, 470-626).

Float32 results are compared with float64 NumPy at float32 accumulation
bounds and with the reference's own attention outputs (golden tiny_model.npz,
GI:136-182 internals: float64 softmax weights and attended rows); the dump's
INT8 arrays are bit-compared with direct calls of the INT8 path."""
import numpy as np
import pytest

from conftest import golden
from gpu_util import assert_bits_equal
from test_gpu_golden_surface import float_archive

pytestmark = pytest.mark.gpu
F32, F64 = np.float32, np.float64
EPS32 = 2.0 ** -24


def tl():
    import lpta.tinyllama as m
    return m


def gi():
    import lpta.tinyllama_gemm_int8 as m
    return m


@pytest.mark.parametrize("m,k,n,bias,res", [(7, 100, 77, True, True), (1, 2048, 256, False, False),
                                             (130, 64, 200, True, False), (3, 5632, 96, False, True)])
def test_linear_f32_within_float32_bound(m, k, n, bias, res):
    rng = np.random.default_rng(m * n + k)
    x = rng.standard_normal((m, k)).astype(F32)
    w = (rng.standard_normal((k, n)) * 0.05).astype(F32)
    b = rng.standard_normal(n).astype(F32) if bias else None
    r = rng.standard_normal((m, n)).astype(F32) if res else None
    rt = tl().op_runtime()
    y = tl().linear_dev(rt, tl().dev(x), w, b, m, None if r is None else tl().dev(r))
    got = tl().host(y)
    want = x.astype(F64) @ w.astype(F64)
    mag = np.abs(x).astype(F64) @ np.abs(w).astype(F64)
    if b is not None:
        want, mag = want + b, mag + np.abs(b)
    if r is not None:
        want, mag = want + r, mag + np.abs(r)
    bound = (k + 3) * EPS32 * mag + 1e-30
    assert (np.abs(got - want) <= bound).all()
    # the numpy-facing TL:106-110 entry point, 1-D and batched shapes
    np.testing.assert_allclose(tl().linear(x[0], w), x[0].astype(F64) @ w, rtol=0,
                               atol=float(((k + 2) * EPS32 * mag[0]).max()))


def test_attention_f32_vs_reference_golden():
    """The reference's mixed-path attention internals (float64 weights and
    attended rows over float32 projections) at 6 tokens, 4 heads, 2 KV heads."""
    z = golden("tiny_model.npz")
    q, k, v = z["attn_q"], z["attn_k"], z["attn_v"]
    S, Hq, Hkv = q.shape[0], q.shape[1] // 64, k.shape[1] // 64
    cos, sin = tl().build_rope_cache(128, 64, 10000.0)
    rt = tl().op_runtime(max_pos=128)
    tl().set_rope_rows(rt, cos, sin, 128)
    qd, kd, vd = tl().dev(q), tl().dev(k), tl().dev(v)
    pos = tl().dev(np.arange(S, dtype=np.int32))
    rt.call("tl_rope", qd, S, Hq, pos)
    rt.call("tl_rope", kd, S, Hkv, pos)
    out = tl().empty((S, Hq * 64), F32)
    sc = tl().empty((Hq, S, S), F32)
    wt = tl().empty((Hq, S, S), F32)
    rt.call("tl_attention_f32", qd, kd, vd, S, Hq, Hkv, 0.125, out, sc, wt)
    weights, scores, att = tl().host(wt), tl().host(sc), tl().host(out)
    # float32 scores (64-term dot products) against the reference's float64
    # softmax over float32 matmul scores
    np.testing.assert_allclose(weights, z["attn_weights"], rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(att, z["attn_attended"], rtol=1e-4, atol=1e-5)
    upper = ~np.tril(np.ones((S, S), bool))
    assert (weights[:, upper] == 0).all() and (scores[:, upper] == F32(-1e9)).all()
    np.testing.assert_allclose(weights.sum(-1), 1.0, rtol=1e-6)


def np_float_layer(x, L, cfg, cos, sin):
    """TL:177-189 in float64 (test restatement for the composition check)."""
    def rms(a, w):
        return a / np.sqrt(np.mean(a * a, -1, keepdims=True) + cfg["rms_norm_eps"]) * w

    def rope(t):
        S = t.shape[1]
        return t * cos[:S] + np.concatenate([-t[..., 32:], t[..., :32]], -1) * sin[:S]

    S, H, Hkv = x.shape[0], cfg["num_attention_heads"], cfg["num_key_value_heads"]
    x = x.astype(F64)
    a = rms(x, L["input_norm_w"])
    q = (a @ L["q_w"]).reshape(S, H, 64).transpose(1, 0, 2)
    k = (a @ L["k_w"]).reshape(S, Hkv, 64).transpose(1, 0, 2)
    v = (a @ L["v_w"]).reshape(S, Hkv, 64).transpose(1, 0, 2)
    q, k = rope(q), rope(k)
    k, v = np.repeat(k, H // Hkv, 0), np.repeat(v, H // Hkv, 0)
    s = q @ k.transpose(0, 2, 1) * 0.125
    s[:, ~np.tril(np.ones((S, S), bool))] = -1e9
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    att = (p @ v).transpose(1, 0, 2).reshape(S, H * 64)
    x1 = x + att @ L["o_w"]
    f = rms(x1, L["post_norm_w"])
    g, u = f @ L["gate_w"], f @ L["up_w"]
    return x1 + (g / (1 + np.exp(-np.clip(g, -60, 60))) * u) @ L["down_w"]


def test_float_decoder_layer_and_forward():
    w = tl().TinyLlamaWeights.from_arrays(float_archive(seed=21))
    cfg = w.cfg
    cos, sin = tl().build_rope_cache(cfg["max_position_embeddings"], 64, 10000.0)
    x = np.random.default_rng(8).standard_normal((33, cfg["hidden_size"])).astype(F32)
    got = tl().decoder_layer(x, w.layer(0), cfg, cos, sin)
    want = np_float_layer(x, {k: (v.astype(F64) if v is not None else None) for k, v in w.layer(0).items()}, cfg,
                          cos.astype(F64), sin.astype(F64))
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4)
    # the GI debug wrapper computes the same layer
    out, dbg = gi().reference_decoder_layer(x, w.layer(0), cfg, cos, sin, capture_arrays=True)
    assert_bits_equal(out, got, "reference_decoder_layer vs TL decoder_layer")
    assert_bits_equal(dbg["layer_out_fp"], got, "layer_out_fp")
    assert dbg["attn"]["scores_fp"].shape == (4, 33, 33) and dbg["attn"]["weights_fp"].shape == (4, 33, 33)
    assert_bits_equal(dbg["x_after_attn_fp"], (x + dbg["attn"]["out_fp"]).astype(F32), "x + attention out")
    assert_bits_equal(out, (dbg["x_after_attn_fp"] + dbg["ffn"]["out_fp"]).astype(F32), "x1 + ffn out")
    # TL:391-408 forward over both layers vs the float64 restatement
    ids = [3, 99, 250, 7, 511]
    logits = tl().forward(ids, w, cos, sin)
    xw = w.embed(ids).astype(F64)
    for i in range(2):
        xw = np_float_layer(xw, {k: (v.astype(F64) if v is not None else None) for k, v in w.layer(i).items()},
                            cfg, cos.astype(F64), sin.astype(F64))
    xw = xw / np.sqrt(np.mean(xw * xw, -1, keepdims=True) + 1e-5) * w.final_norm_w()
    np.testing.assert_allclose(logits, xw @ w.lm_head_w(), rtol=1e-3, atol=1e-3)
    assert_bits_equal(gi().forward_reference(ids, w, cos, sin, 2), logits, "forward_reference")


# keys of the reference's debug dicts after flatten_named_arrays (GI:75-87,
# 122-133, 166-181, 195-202, 215-224, 244-253, 272-281, 318-321)
PROJ_KEYS = ("input_scale", "weight_scale", "input_fp", "input_q", "weight_fp", "weight_q", "accum_int32",
             "output_fp")
REF_KEYS = ["reference_attn_input_fp", "reference_x_after_attn_fp", "reference_ffn_input_fp",
            "reference_layer_out_fp", "reference_attn_q_proj_fp", "reference_attn_k_proj_fp",
            "reference_attn_v_proj_fp", "reference_attn_scores_fp", "reference_attn_weights_fp",
            "reference_attn_attended_fp", "reference_attn_out_fp", "reference_ffn_gate_proj_fp",
            "reference_ffn_up_proj_fp", "reference_ffn_hidden_fp", "reference_ffn_out_fp"]
MIX_KEYS = (["mixed_attn_input_fp", "mixed_x_after_attn_fp", "mixed_ffn_input_fp", "mixed_layer_out_fp",
             "mixed_attn_q_proj_fp", "mixed_attn_k_proj_fp", "mixed_attn_v_proj_fp", "mixed_attn_attended_fp",
             "mixed_attn_out_fp", "mixed_ffn_gate_proj_fp", "mixed_ffn_up_proj_fp", "mixed_ffn_hidden_fp",
             "mixed_ffn_out_fp"]
            + [f"mixed_attn_{p}_{k}" for p in ("q_proj", "k_proj", "v_proj", "o_proj") for k in PROJ_KEYS]
            + [f"mixed_ffn_{p}_{k}" for p in ("gate_proj", "up_proj", "down_proj") for k in PROJ_KEYS]
            + [f"mixed_lm_head_{k}" for k in PROJ_KEYS])


def test_run_analysis_dump(tmp_path, capsys):
    arch = float_archive(seed=31)
    path = tmp_path / "weights.npz"
    np.savez(path, **arch)
    dump = tmp_path / "dump"
    ids = [5, 77, 300, 2, 511, 64, 9, 130]
    res = gi().run_analysis(None, ",".join(map(str, ids)), str(path), 2, dump_layer=1, dump_dir=str(dump),
                            top_k=4, quantize_lm_head=True)
    out = capsys.readouterr().out
    assert f"Token ids: {ids}" in out
    assert "Layer 0: isolated MAE=" in out and "Layer 1: isolated MAE=" in out
    assert "  attn q_proj: mae=" in out and "  ffn down_proj: mae=" in out
    assert "Top 4 float32 tokens:" in out and "Top 4 INT8-path tokens:" in out
    assert f"Saved debug dump to {dump}" in out
    summary = (dump / "summary.txt").read_text().splitlines()
    assert summary[:3] == [f"Token ids: {ids}", "Layers analyzed: 2", "Layer stats:"]
    assert summary == res["summary_lines"]
    with np.load(dump / "debug_arrays.npz", allow_pickle=False) as z:
        keys = set(z.files)
        missing = [k for k in ["token_ids"] + REF_KEYS + MIX_KEYS if k not in keys]
        assert not missing, missing
        assert_bits_equal(z["token_ids"], np.asarray(ids, np.int32), "token_ids")
        # the dumped layer is layer 1 run from the float32 model's layer-0 output
        w = tl().load_weights(str(path))
        cfg = w.cfg
        cos, sin = tl().build_rope_cache(cfg["max_position_embeddings"], 64, cfg["rope_theta"])
        x0, _ = gi().reference_decoder_layer(w.embed(ids).astype(F32), w.layer(0), cfg, cos, sin)
        r1, rdbg = gi().reference_decoder_layer(x0, w.layer(1), cfg, cos, sin, capture_arrays=True)
        assert_bits_equal(z["reference_layer_out_fp"], r1, "reference layer 1")
        assert_bits_equal(z["reference_attn_weights_fp"], rdbg["attn"]["weights_fp"], "reference weights")
        m1, mdbg = gi().mixed_precision_decoder_layer(x0, w.layer(1), cfg, cos, sin, capture_arrays=True)
        assert_bits_equal(z["mixed_layer_out_fp"], m1, "mixed layer 1 (isolated)")
        assert_bits_equal(z["mixed_attn_q_proj_accum_int32"], mdbg["attn"]["q_proj"]["accum_int32"], "q accum")
        assert z["mixed_lm_head_input_q"].shape == (1, cfg["hidden_size"])
        assert z["mixed_lm_head_weight_q"].dtype == np.int8
    # the INT8 path tracks the float32 model on this small model
    assert res["mix_logits"].shape == res["ref_logits"].shape == (1, cfg["vocab_size"])
    rel = np.abs(res["mix_logits"] - res["ref_logits"]).max() / np.abs(res["ref_logits"]).max()
    assert rel < 0.25


def test_run_analysis_argument_errors(tmp_path):
    arch = float_archive(seed=32)
    path = tmp_path / "weights.npz"
    np.savez(path, **arch)
    with pytest.raises(ValueError, match="dump-layer"):
        gi().run_analysis(None, "1,2", str(path), 1, dump_layer=1)
    with pytest.raises(ValueError, match="--layers"):
        gi().run_analysis(None, "1,2", str(path), 3)
    with pytest.raises(ValueError, match="--prompt or --token-ids"):
        gi().run_analysis(None, None, str(path), 1)
    with pytest.raises(FileNotFoundError):
        gi().main(["--weights", str(tmp_path / "missing.npz")])
    with pytest.raises(ValueError, match="only supported in --mode analysis"):
        gi().main(["--mode", "generate", "--weights", str(path), "--token-ids", "1", "--dump-layer", "0"])
