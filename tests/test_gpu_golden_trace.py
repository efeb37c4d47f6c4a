"""Decode-step debug capture (tl_capture_step) against the CPU oracle's trace
of the same step, the capture's export in the canonical case format, and the
replay of shared_gemm_engine cases written in the reference exporter's
layout (EX:259-386).  Integer tensors, float tensors and token ids must be
bit-identical to the oracle's."""
import numpy as np
import pytest

import oracle
from gpu_util import assert_bits_equal
from lpta import golden_trace as gt

pytestmark = pytest.mark.gpu


def engine_for(model):
    from lpta.engine import Engine
    return Engine(model.cfg).load_model(model)


def oracle_prefill(orc, m, prompt):
    kc, vc = m.new_cache()
    x = None
    for i, t in enumerate(prompt):
        x = orc.embed(int(t))
        for layer in range(m.cfg["n_layers"]):
            x = orc.decode_row(layer, i, x, kc, vc)
    return orc.lm_head(x)[0], kc, vc


def oracle_step(orc, m, tok, pos, kc, vc, layer):
    """The oracle's decode step at pos with layer's trace and the top-16 logits."""
    c = m.cfg
    D, Hq, V = c["hidden"], c["n_heads"], c["vocab"]
    KVD = c["n_kv_heads"] * 64
    tr = {"attn_in_q": np.zeros(D, np.int8), "attn_in_s": np.zeros(1), "qkv": np.zeros(D + 2 * KVD, np.float32),
          "q8": np.zeros(D, np.int8), "q_s": np.zeros(1), "scores": np.zeros(Hq * (pos + 1), np.int32),
          "probs": np.zeros(Hq * (pos + 1), np.int8), "attended": np.zeros(D, np.float32),
          "out": np.zeros(D, np.float32)}
    x = orc.embed(int(tok))
    x_in = None
    for li in range(c["n_layers"]):
        if li == layer:
            x_in = x.copy()
            x = orc.decode_row(li, pos, x, kc, vc, tr)
        else:
            x = orc.decode_row(li, pos, x, kc, vc)
    nxt, logit, logits = orc.lm_head(x, want_logits=True)
    top = np.lexsort((np.arange(V), -logits))[:16]
    tr["scores"] = tr["scores"].reshape(Hq, pos + 1)
    tr["probs"] = tr["probs"].reshape(Hq, pos + 1)
    return dict(tr, x_in=x_in, final=x, token=nxt, logit=logit, top_ids=top, top_logits=logits[top])


CASES = [
    # (geometry, prompt length, captured layer, key0, n_keys)
    ("small", 70, 1, 0, -1),
    ("small", 9, 0, 3, 5),
    ("tinyllama2", 33, 1, 0, -1),
]


def model_for(name):
    if name == "small":
        return oracle.synthetic_model(dict(oracle.SMALL_CFG), seed=11)
    cfg = dict(oracle.TINYLLAMA_CFG, n_layers=2, vocab=512)
    return oracle.synthetic_model(cfg, seed=12, kv_range=(0.01, 0.1))


@pytest.mark.parametrize("name,n_prompt,layer,key0,n_keys", CASES)
def test_capture_step_matches_oracle(name, n_prompt, layer, key0, n_keys, tmp_path):
    print(f"capture case {name} prompt={n_prompt} layer={layer} window={key0},{n_keys}", flush=True)
    m = model_for(name)
    c = m.cfg
    prompt = np.random.default_rng(n_prompt).integers(0, c["vocab"], n_prompt).astype(np.int32)
    eng = engine_for(m)
    first, _ = eng.prefill(prompt)
    cap = eng.capture_step(layer, key0=key0, n_keys=n_keys)
    orc = oracle.Oracle(m)
    tok0, kc, vc = oracle_prefill(orc, m, prompt)
    assert first == tok0
    pos = n_prompt
    want = oracle_step(orc, m, tok0, pos, kc, vc, layer)
    W = pos + 1 - key0 if n_keys < 0 else n_keys

    assert (cap["layer"], cap["pos"], cap["key0"], cap["n_keys"], cap["token_in"]) == (layer, pos, key0, W, tok0)
    assert_bits_equal(cap["layer_in"], want["x_in"], "layer input")
    assert_bits_equal(cap["attn_in_q"], want["attn_in_q"], "attention input (INT8)")
    assert cap["attn_in_scale"] == want["attn_in_s"][0]
    assert_bits_equal(cap["qkv"], want["qkv"], "Q|K|V projections")
    assert_bits_equal(cap["q8"], want["q8"], "query (INT8)")
    assert cap["q_scale"] == want["q_s"][0]
    G = c["n_heads"] // c["n_kv_heads"]
    for g in range(c["n_kv_heads"]):
        assert_bits_equal(cap["k_row"][g * 64:(g + 1) * 64], kc[layer, g, pos], f"K row head {g}")
        assert_bits_equal(cap["v_row"][g * 64:(g + 1) * 64], vc[layer, g, pos], f"V row head {g}")
        assert_bits_equal(cap["kv_scales"][0, g], m.kv_sk[layer, g], "K scale")
        assert_bits_equal(cap["kv_scales"][1, g], m.kv_sv[layer, g], "V scale")
        # score scale f32((s_q s_k) / sqrt(64)) of each query head of the group
        want_scl = np.float32((want["q_s"][0] * np.float64(m.kv_sk[layer, g])) * 0.125)
        assert_bits_equal(cap["score_scale"][g * G:(g + 1) * G], np.full(G, want_scl, np.float32), "score scale")
    assert_bits_equal(cap["scores"], want["scores"][:, key0:key0 + W], "INT32 score window")
    assert_bits_equal(cap["probs"], want["probs"][:, key0:key0 + W], "INT8 probability window")
    assert (cap["probs"] >= 0).all()
    assert_bits_equal(cap["attended"], want["attended"], "attention output")
    assert_bits_equal(cap["layer_out"], want["out"], "layer output")
    assert_bits_equal(cap["final_hidden"], want["final"], "final hidden state")
    assert cap["token"] == want["token"] and cap["top_ids"][0] == want["token"]
    assert_bits_equal(cap["top_ids"], want["top_ids"].astype(np.int32), "top-16 ids")
    assert_bits_equal(cap["top_logits"], want["top_logits"], "top-16 logits")
    assert_bits_equal(np.float32(cap["logit"]), np.float32(want["logit"]), "chosen logit")

    # the capture was one real decode step: the sequence continues as if
    # tl_decode had run it
    more, _ = eng.decode(3)
    eng.close()
    ref = engine_for(m)
    plain, _ = ref.generate(prompt, 5)
    ref.close()
    assert [first, cap["token"], *more.tolist()] == plain.tolist()

    # export in the canonical case format and read it back
    case_id = gt.export_capture(cap, tmp_path)
    entry, arrays = gt.load_case(tmp_path, case_id)
    assert entry["block"] == "decode_step" and entry["layer_id"] == layer and entry["token_start"] == pos
    for k in ("q8", "k_row", "scores", "probs", "attended", "top_ids"):
        assert_bits_equal(arrays[k], cap[k], f"exported {k}")
    assert int(arrays["token"][0]) == cap["token"]
    base = tmp_path / entry["rtl_fixture_base"]
    q8 = gt.read_packed_lane_memh(str(base) + ".q8_packed.memh", bits_per_lane=8, signed=True)
    assert_bits_equal(q8.astype(np.int8), cap["q8"].reshape(-1, 64), "q8 fixture")
    sc = gt.read_packed_lane_memh(str(base) + ".scores_packed.memh", bits_per_lane=32, signed=True)
    assert_bits_equal(sc.astype(np.int32), cap["scores"], "score fixture")
    meta = gt.read_scalar_memh_u32(str(base) + ".meta.memh")
    assert meta.tolist() == [layer, pos, key0, W, tok0, cap["token"]]


def test_capture_rejects_bad_windows():
    m = model_for("small")
    eng = engine_for(m)
    from lpta import TlValueError
    with pytest.raises(TlValueError, match="prefilled"):
        eng.capture_step(0)
    eng.prefill(np.arange(5, dtype=np.int32))
    with pytest.raises(TlValueError, match="window"):
        eng.capture_step(0, key0=2, n_keys=5)    # keys 2..6 but pos = 5
    with pytest.raises(TlValueError, match="layer"):
        eng.capture_step(2)
    cap = eng.capture_step(1, key0=6, n_keys=-1)  # empty window at the step's own key
    assert cap["n_keys"] == 0 and cap["scores"].shape == (m.cfg["n_heads"], 0)
    eng.close()


# ---- replay of exporter-format shared_gemm_engine cases ------------------------------

N_TILE, LANES = 32, 512   # EX:45-46


def write_ex_gemm_case(root, case_id, act, wt, acc):
    """A shared_gemm_engine case laid out as EX:259-386 writes it."""
    m, k = act.shape
    n = wt.shape[1]
    act_steps = np.zeros((k, LANES), np.int8)
    wt_steps = np.zeros((k, LANES), np.int8)
    acc_lane = np.zeros(LANES, np.int32)
    for mi in range(m):
        for ni in range(n):
            lane = mi * N_TILE + ni
            act_steps[:, lane] = act[mi]
            wt_steps[:, lane] = wt[:, ni]
            acc_lane[lane] = acc[mi, ni]
    gt.write_case(root, case_id, "phase3", "shared_gemm_engine",
                  dict(act=act, wt=wt, acc_expected=acc, act_steps=act_steps, wt_steps=wt_steps,
                       acc_expected_lane=acc_lane, active_lane_count=np.asarray([m * n], np.int32)),
                  {"k_total": k, "m_count": m, "n_count": n})
    base = root / "phase3" / "rtl" / case_id
    gt.write_hex_memh(str(base) + ".meta.memh", np.asarray([k, m * n, m, n], np.uint32), bits=32, signed=False)
    gt.write_hex_memh(str(base) + ".act_steps.memh", act_steps, bits=8, signed=True)
    gt.write_hex_memh(str(base) + ".wt_steps.memh", wt_steps, bits=8, signed=True)
    gt.write_hex_memh(str(base) + ".acc_expected_lane.memh", acc_lane, bits=32, signed=True)
    return base


@pytest.mark.parametrize("m,n,k", [(16, 32, 2048), (3, 7, 40), (16, 32, 5632)])
def test_replay_gemm_cases(m, n, k, tmp_path):
    print(f"replay case m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(k + m)
    act = rng.integers(-127, 128, (m, k)).astype(np.int8)
    wt = rng.integers(-127, 128, (k, n)).astype(np.int8)
    acc = oracle.gemm_i8(act, np.ascontiguousarray(wt.T))
    base = write_ex_gemm_case(tmp_path, "phase3_decode_layer0_q_gemm_m0_n0", act, wt, acc)
    bad = acc.copy()
    bad[m - 1, n - 1] += 1
    write_ex_gemm_case(tmp_path / "planted", "phase3_decode_layer0_q_gemm_m0_n0", act, wt, bad)
    gt.write_case(tmp_path, "phase3_other", "phase3", "softmax_wrapper", {"acc": acc})
    rt = gt.Runtime(dict(hidden=512, intermediate=1408, n_layers=1, n_heads=8, n_kv_heads=2, head_dim=64,
                         vocab=64, max_pos=64, rms_eps=np.float32(1e-5), rope_theta=1e4))
    _, arrays = gt.load_case(tmp_path, "phase3_decode_layer0_q_gemm_m0_n0")
    r = gt.replay_gemm_case(rt, arrays)
    assert r["match"]
    assert_bits_equal(r["acc"], acc, "replayed accumulators")
    f = gt.replay_gemm_fixture(rt, base)
    assert f["match"]
    assert gt.fixture_paths(tmp_path / "phase3") == [str(base)]
    res = gt.replay_manifest(rt, tmp_path)
    assert res == [{"case_id": "phase3_decode_layer0_q_gemm_m0_n0", "replayed": True, "match": True},
                   {"case_id": "phase3_other", "replayed": False}]
    # a planted wrong accumulator is reported as a mismatch
    _, arrays = gt.load_case(tmp_path / "planted", "phase3_decode_layer0_q_gemm_m0_n0")
    assert not gt.replay_gemm_case(rt, arrays)["match"]
    assert not gt.replay_gemm_fixture(rt, gt.fixture_paths(tmp_path / "planted")[0])["match"]
    rt.close()


# ---- replay of exporter-format requantize_unit cases --------------------------------

SCALES = 16   # EX:47 SCALE_VECTOR_ELEMS: one Q16.16 multiplier per 32 lanes


def write_ex_requant_case(root, case_id, acc_lane, scale, out_lane, active):
    """A requantize_unit case laid out as EX:528-653 writes it."""
    gt.write_case(root, case_id, "phase3", "requantize_unit",
                  dict(acc=acc_lane, scale=scale, out_expected=out_lane,
                       elem_count=np.asarray([active], np.int32)), {"active_lane_count": active})
    base = root / "phase3" / "rtl" / case_id
    gt.write_hex_memh(str(base) + ".meta.memh", np.asarray([active], np.uint32), bits=32, signed=False)
    gt.write_hex_memh(str(base) + ".acc.memh", acc_lane, bits=32, signed=True)
    gt.write_hex_memh(str(base) + ".scale.memh", scale, bits=32, signed=False)
    gt.write_hex_memh(str(base) + ".out_expected.memh", out_lane, bits=8, signed=True)
    return base


def oracle_requant(acc_lane, scale, active, nonneg=0):
    return np.array([oracle.lib().or_requant_q16(int(a), int(scale[i // 32]), nonneg) if i < active else 0
                     for i, a in enumerate(acc_lane)], np.int8)


@pytest.mark.parametrize("active", [512, 64, 37])
def test_replay_requant_cases(active, tmp_path):
    """Q16.16 requantization (requantize_unit.sv:39-115) of exporter-format
    cases: multipliers as EX:542-545 forms them (sx * sw / s_out in Q16.16),
    lanes past the element count zero, and a planted wrong lane reported."""
    print(f"replay requant case active={active}", flush=True)
    rng = np.random.default_rng(active)
    acc = rng.integers(-300000, 300001, LANES).astype(np.int32)
    mult_fp = rng.uniform(1e-4, 1e-3, SCALES)
    scale = np.array([int(round(m * 65536.0)) for m in mult_fp], np.uint32)
    out = oracle_requant(acc, scale, active)
    base = write_ex_requant_case(tmp_path, "phase3_prefill_layer0_q_requant_m0_n0", acc, scale, out, active)
    bad = out.copy()
    bad[active - 1] = np.int8(out[active - 1] ^ 1)
    write_ex_requant_case(tmp_path / "planted", "phase3_prefill_layer0_q_requant_m0_n0", acc, scale, bad, active)
    rt = gt.Runtime(dict(hidden=512, intermediate=1408, n_layers=1, n_heads=8, n_kv_heads=2, head_dim=64,
                         vocab=64, max_pos=64, rms_eps=np.float32(1e-5), rope_theta=1e4))
    _, arrays = gt.load_case(tmp_path, "phase3_prefill_layer0_q_requant_m0_n0")
    r = gt.replay_requant_case(rt, arrays)
    assert r["match"]
    assert_bits_equal(r["out"], out, "replayed lanes")
    assert gt.replay_fixture(rt, base)["match"]
    assert gt.replay_manifest(rt, tmp_path) == [{"case_id": "phase3_prefill_layer0_q_requant_m0_n0",
                                                 "replayed": True, "match": True}]
    _, arrays = gt.load_case(tmp_path / "planted", "phase3_prefill_layer0_q_requant_m0_n0")
    assert not gt.replay_requant_case(rt, arrays)["match"]
    assert not gt.replay_fixture(rt, gt.fixture_paths(tmp_path / "planted")[0])["match"]
    rt.close()


def test_requant_q16_edges():
    """tl_requant_q16 against the oracle at the integer edges: the largest
    accumulators times the largest multipliers (64-bit products), exact
    half-way products of both parities, both clamps, one multiplier per
    bank of 32 lanes, and the element count."""
    from gpu_util import dev, empty, host
    rt = gt.Runtime(dict(hidden=512, intermediate=1408, n_layers=1, n_heads=8, n_kv_heads=2, head_dim=64,
                         vocab=64, max_pos=64, rms_eps=np.float32(1e-5), rope_theta=1e4))
    acc = np.array([2**31 - 1, -2**31, 3, 5, -3, -5, 1, -1, 255, -255, 256, 0, 127, -128, 10, 11] * 8, np.int32)
    scale = np.array([0xFFFFFFFF, 0x8000, 0x10000, 0x7FFF, 0x1, 0x0, 0x12345, 0xFFFF], np.uint32)
    for nonneg in (0, 1):
        for active in (acc.size, 40):
            want = np.array([oracle.lib().or_requant_q16(int(a), int(scale[i // 32]), nonneg) if i < active else 0
                             for i, a in enumerate(acc)], np.int8)
            y = empty((acc.size,), np.int8)
            rt.call("tl_requant_q16", dev(acc), dev(scale.view(np.int32)), acc.size, active, 32, nonneg, y)
            assert_bits_equal(host(y), want, f"nonnegative_only={nonneg} active={active}")
    rt.close()


# ---- replay of exporter-format element-wise cases (phases 4-6) ----------------------

EX_CFG = dict(oracle.TINYLLAMA_CFG, n_layers=1, vocab=64)


def ex_rope_case(rng, base, tokens):
    """rope_unit (EX:930-1006): one head's INT8 Q and K rows at positions
    base .. base + tokens - 1, rotated by the oracle's or_rotate_q16 with
    cos / sin in Q16.16 as EX:656-668 forms the ROM."""
    cos, sin = oracle.rope_table(2048, 64, 1e4)
    cq, sq = gt.q16_signed_from_float(cos), gt.q16_signed_from_float(sin)
    L = oracle.lib()
    arrays = {}
    for name in ("q", "k"):
        x = rng.integers(-127, 128, (tokens, 64)).astype(np.int8)
        y = np.zeros_like(x)
        for t in range(tokens):
            for d in range(64):
                lower = d < 32
                pair = x[t, d + 32] if lower else x[t, d - 32]
                y[t, d] = L.or_rotate_q16(int(x[t, d]), int(pair), int(cq[base + t, d]), int(sq[base + t, d]),
                                          int(lower))
        arrays[f"{name}_in"], arrays[f"{name}_out_expected"] = x, y
    return dict(arrays, token_base=np.asarray([base], np.int32), token_count=np.asarray([tokens], np.int32),
                q_head_id=np.asarray([3], np.int32), kv_head_id=np.asarray([0], np.int32))


def ex_mask_case(rng, qb, kb, qrc, kcc):
    """causal_mask_unit (EX:1009-1086) on an 8 x 64 INT32 score tile."""
    s = rng.integers(-(1 << 20), 1 << 20, (8, 64)).astype(np.int32)
    out = np.empty_like(s)
    oracle.lib().or_causal_mask_tile(oracle.ptr(s, oracle.C.c_int32), 8, 64, qb, kb, qrc, kcc,
                                     oracle.ptr(out, oracle.C.c_int32))
    return dict(score_in=s, score_out_expected=out, query_pos_base=np.asarray([qb], np.int32),
                key_pos_base=np.asarray([kb], np.int32), query_row_count=np.asarray([qrc], np.int32),
                key_col_count=np.asarray([kcc], np.int32))


def ex_rmsnorm_case(rng, rows):
    """rmsnorm (EX:1705-1805): per-tensor INT8 input rows, Q16.16-exact input
    and gains, the oracle's RMSNorm (TL:45-50, NumPy's pairwise mean), output
    quantized at the Q16.16 output scale."""
    x_fp = rng.standard_normal((rows, 2048)).astype(np.float32)
    gamma = rng.uniform(0.8, 1.2, 2048).astype(np.float32)
    x_q, s_in = oracle.quantize_int8(x_fp)
    x_deq = gt.float_from_q16(x_q.astype(np.int64) * int(gt.q16_from_float(s_in)))
    gamma_core = gt.float_from_q16(gt.q16_signed_from_float(gamma))
    y_fp = oracle.rms_norm(x_deq, gamma_core, EX_CFG["rms_eps"])
    _, s_out = oracle.quantize_int8(oracle.rms_norm(x_q.astype(np.float32) * np.float32(s_in), gamma,
                                                    EX_CFG["rms_eps"]))
    s_out_q16 = int(gt.q16_from_float(s_out))
    y_q = gt.quantize_fixed_by_scale_q16(gt.q16_signed_from_float(y_fp), s_out_q16)
    return dict(x_q=x_q, x_deq=x_deq, gamma_fp=gamma, y_fp=y_fp, y_q=y_q,
                input_scale=np.asarray([s_in], np.float32),
                output_scale=np.asarray([gt.float_from_q16(s_out_q16)], np.float32))


def ex_softmax_case(rng, qrc, kcc, qb):
    """softmax (EX:1808-1893): masked INT32 scores times the Q16.16 score
    scale, the oracle's row softmax over the active rows, Q16.16 probabilities
    and their INT8 form."""
    raw = rng.integers(-3000, 3000, (8, 64)).astype(np.int32)
    masked = np.empty_like(raw)
    oracle.lib().or_causal_mask_tile(oracle.ptr(raw, oracle.C.c_int32), 8, 64, qb, 0, qrc, kcc,
                                     oracle.ptr(masked, oracle.C.c_int32))
    scale = 0.004
    core = np.clip(masked.astype(np.int64) * int(gt.q16_from_float(scale)), -(1 << 31), (1 << 31) - 1)
    score_fp = gt.float_from_q16(core)
    prob_fp = np.zeros((8, 64), np.float32)
    for r in range(qrc):
        prob_fp[r] = oracle.softmax_row(score_fp[r])
    prob_q = gt.quantize_probability_q16(gt.q16_signed_from_float(prob_fp))
    return dict(score_in=masked, score_fp=score_fp, prob_fp=prob_fp, prob_q=prob_q,
                score_scale=np.asarray([scale], np.float32))


def ex_silu_case(rng, rows):
    """silu (EX:1896-1990): per-tensor INT8 gate values through Q16.16, the
    oracle's SiLU (TL:159-161), output quantized at its Q16.16 scale."""
    x_fp = (rng.standard_normal((rows, 32)) * 4).astype(np.float32)
    x_q, s_in = oracle.quantize_int8(x_fp)
    x_deq = gt.float_from_q16(x_q.astype(np.int64) * int(gt.q16_from_float(s_in)))
    y_fp = oracle.silu(x_deq)
    s_out_q16 = int(gt.q16_from_float(oracle.quantize_int8(y_fp)[1]))
    y_q = gt.quantize_fixed_by_scale_q16(gt.q16_signed_from_float(y_fp), s_out_q16)
    return dict(x_q=x_q, x_deq=x_deq, y_fp=y_fp, y_q=y_q, input_scale=np.asarray([s_in], np.float32),
                output_scale=np.asarray([gt.float_from_q16(s_out_q16)], np.float32))


def ex_argmax_case(rng, tie):
    """argmax (EX:1651-1702): Q16.16 logits of the 32000-entry vocabulary;
    with `tie`, the maximum is planted at three ids across 128-wide tiles."""
    logits_fp = (rng.standard_normal(32000) * 3).astype(np.float32)
    q16 = gt.q16_signed_from_float(logits_fp)
    if tie:
        top = int(q16.max()) + 7
        q16[[31999, 20001, 20000]] = top
    best = np.asarray([0], np.int32)
    idx = oracle.lib().or_argmax_i32_tiles(oracle.ptr(q16, oracle.C.c_int32), 32000, 128,
                                           oracle.ptr(best, oracle.C.c_int32))
    assert idx == int(np.argmax(q16))
    return dict(logits_fp=logits_fp, logits_q16=q16, argmax_expected=np.asarray([idx], np.uint32),
                logit_expected=best)


def test_replay_elementwise_cases(tmp_path):
    """Cases of six more exporter block types, written in the exporter's
    .npz layout with a manifest (expected values from the oracle), replayed
    through the library's operators: rope_unit (INT8 RoPE), causal_mask_unit,
    rmsnorm, softmax, silu and argmax.  Each case matches; a planted error in
    each type is reported as a mismatch."""
    rng = np.random.default_rng(2024)
    cases = [
        ("phase4_prefill_layer0_rope_q3_kv0_t0", "phase4", "rope_unit", ex_rope_case(rng, 0, 8)),
        ("phase4_decode_layer0_rope_q3_kv0_t1500", "phase4", "rope_unit", ex_rope_case(rng, 1500, 8)),
        ("phase4_prefill_layer0_causal_mask_q0_kv0_qb8_kb0", "phase4", "causal_mask_unit",
         ex_mask_case(rng, 8, 0, 8, 64)),
        ("phase4_decode_layer0_causal_mask_q0_kv0_qb70_kb64", "phase4", "causal_mask_unit",
         ex_mask_case(rng, 70, 64, 1, 30)),
        ("phase5_prefill_layer0_rmsnorm1", "phase5", "rmsnorm", ex_rmsnorm_case(rng, 4)),
        ("phase5_prefill_layer0_softmax_q0_kv0_qb8_kb0", "phase5", "softmax", ex_softmax_case(rng, 8, 64, 8)),
        ("phase5_decode_layer0_softmax_q0_kv0_qb5_kb0", "phase5", "softmax", ex_softmax_case(rng, 1, 6, 5)),
        ("phase5_prefill_layer0_silu_gate_m0", "phase5", "silu", ex_silu_case(rng, 16)),
        ("phase6_prefill_argmax", "phase6", "argmax", ex_argmax_case(rng, False)),
        ("phase6_decode_argmax", "phase6", "argmax", ex_argmax_case(rng, True)),
    ]
    for cid, phase, block, arrays in cases:
        gt.write_case(tmp_path, cid, phase, block, arrays)
    rt = gt.Runtime(EX_CFG)
    res = gt.replay_manifest(rt, tmp_path)
    print("replay:", [(r["case_id"], r.get("match")) for r in res], flush=True)
    assert res == [{"case_id": cid, "replayed": True, "match": True} for cid, _, _, _ in cases]
    # planted errors: one element of an expected output per block type
    plants = {"rope_unit": "k_out_expected", "causal_mask_unit": "score_out_expected", "rmsnorm": "y_q",
              "softmax": "prob_q", "silu": "y_q", "argmax": "argmax_expected"}
    for cid, phase, block, arrays in cases:
        bad = dict(arrays)
        key = plants[block]
        v = np.array(bad[key], copy=True)
        flat = v.reshape(-1)
        flat[-1] = flat[-1] + 1 if block != "rmsnorm" else np.int8(flat[-1] ^ 1)
        bad[key] = v
        assert not gt.REPLAYERS[block](rt, bad)["match"], f"planted error in {cid} not reported"
    rt.close()
