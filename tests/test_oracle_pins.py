"""Pins the CPU oracle to the reference: golden vectors written by
tests/golden/make_golden.py from the reference's own NumPy functions, the
reference's committed integer fixtures (sim/), the SystemVerilog testbench
KATs, and closed-form / brute-force checks.  CPU only."""
import math

import numpy as np
import pytest

import oracle
from conftest import golden
from models import tiny_from_golden

F32 = np.float32


def bits_equal(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32 if a.dtype == np.float32 else a.dtype),
                                                 b.view(np.uint32 if b.dtype == np.float32 else b.dtype))


# ---- RMSNorm (TL:45-50): bit-exact, NumPy pairwise summation ---------------------

def test_rms_norm_bit_exact_vs_golden():
    z = golden("rms_norm.npz")
    for key in z.files:
        if not key.startswith("x_"):
            continue
        n = key[2:]
        y = oracle.rms_norm(z[f"x_{n}"], z[f"w_{n}"], F32(1e-5))
        assert bits_equal(y, z[f"y_{n}"]), f"rms_norm width {n}"


def test_pairwise_sum_is_not_a_plain_loop():
    # a sequential float32 sum differs from NumPy's pairwise tree on this input;
    # the oracle must follow the tree
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(2048) * 1e3).astype(F32)
    seq = F32(0)
    for v in x:
        seq = F32(seq + v)
    pw = oracle.lib().or_pairwise_sum(oracle.ptr(x, oracle.C.c_float), x.size)
    assert F32(pw) == np.sum(x, dtype=F32)
    assert F32(pw) != seq


# ---- quantize_int8 / dequantize_int32 / quantized_linear (GI:36-88) -----------------

def test_quantize_int8_bit_exact_vs_golden():
    z = golden("quantize.npz")
    for case in ("normal", "wide", "ties", "zeros", "tiny"):
        q, s = oracle.quantize_int8(z[f"x_{case}"])
        assert np.array_equal(q, z[f"q_{case}"]), case
        assert s == float(z[f"s_{case}"]), case


def test_quantize_never_emits_minus_128():
    x = np.array([-1.0, 1.0, -1.0000001, 0.5], F32)
    q, _ = oracle.quantize_int8(x)
    assert q.min() >= -127


def test_dequantize_bit_exact_vs_golden():
    z = golden("quantize.npz")
    m = oracle.lib().or_dequant_mult(float(z["deq_sx"]), float(z["deq_sw"]))
    y = z["deq_acc"].astype(F32) * F32(m)
    assert bits_equal(y, z["deq_y"])


def test_quantized_linear_chain_vs_golden():
    z = golden("quantized_linear.npz")
    xq, sx = oracle.quantize_int8(z["x"])            # per-tensor, as GI:68
    wq, sw = oracle.quantize_int8(z["w"])            # per-tensor, as GI:69
    # the golden's debug dict keeps the scales as float32 (GI:76-77)
    assert np.array_equal(xq, z["input_q"]) and F32(sx) == F32(z["input_scale"])
    assert np.array_equal(wq, z["weight_q"]) and F32(sw) == F32(z["weight_scale"])
    acc = oracle.gemm_i8(xq, np.ascontiguousarray(wq.T))
    assert np.array_equal(acc, z["accum_int32"])
    out = acc.astype(F32) * F32(oracle.lib().or_dequant_mult(sx, sw))
    assert bits_equal(out, z["out"])


# ---- integer contraction: sim fixtures and testbench KATs ---------------------------

def test_sim_matvec_fixture():
    z = golden("sim_fixtures.npz")
    w = z["w"].reshape(64, 64).astype(np.int8)
    x = z["x"].astype(np.int8)[None, :]
    assert np.array_equal(oracle.gemm_i8(x, w)[0], z["expected"])


@pytest.mark.parametrize("k", [16, 64])
def test_sim_two_layer_requant_chain(k):
    z = golden("sim_fixtures.npz")
    x = z[f"k{k}_x_q"].astype(np.int8)[None, :]
    w1 = z[f"k{k}_W1_q"].reshape(k, k).astype(np.int8)
    w2 = z[f"k{k}_W2_q"].reshape(k, k).astype(np.int8)
    y1 = oracle.gemm_i8(x, w1)[0]
    assert np.array_equal(y1, z[f"k{k}_y1_int"])
    mult = oracle.lib().or_dequant_mult(float(z[f"k{k}_scale_W1"]), float(z[f"k{k}_scale_x"]))
    y1_deq = np.maximum(y1.astype(F32) * F32(mult), F32(0))
    y2q, sy2 = oracle.quantize_int8(y1_deq)
    assert np.array_equal(y2q, z[f"k{k}_y2_q"].astype(np.int8))
    assert abs(sy2 - float(z[f"k{k}_scale_y2"])) <= 1e-7 * sy2
    assert np.array_equal(oracle.gemm_i8(y2q[None, :], w2)[0], z[f"k{k}_y_expected"])


def test_mac_kats():
    # tb_mac_lane.sv:20-47, tb_mac_array.sv:185-211, tb_shared_gemm_engine.sv:79-122
    a = np.array([[3, 1], [-7, -1]], np.int8)
    w = np.array([[-4, 10], [-6, 5]], np.int8)
    c = oracle.gemm_i8(a, w)
    assert c[0, 0] == -2 and c[1, 1] == 37
    a = np.array([[127, -128, -128]], np.int8)
    for i, (x, y, want) in enumerate([(127, 127, 16129), (-128, 127, -16256), (-128, -128, 16384)]):
        assert oracle.gemm_i8(np.array([[x]], np.int8), np.array([[y]], np.int8))[0, 0] == want
    ones = np.ones((1, 2), np.int8)
    rows = np.array([[1, 10], [2, 20], [3, 30], [4, 40]], np.int8)
    assert list(oracle.gemm_i8(ones, rows)[0]) == [11, 22, 33, 44]


def test_gemm_brute_force_with_extremes():
    rng = np.random.default_rng(11)
    for m, n, k in [(1, 37, 5632), (3, 64, 2048), (5, 9, 1)]:
        a = rng.integers(-128, 128, (m, k)).astype(np.int8)
        w = rng.integers(-128, 128, (n, k)).astype(np.int8)
        a[0, :] = -128
        w[0, :] = -128
        want = (a.astype(np.int64) @ w.astype(np.int64).T)
        assert np.array_equal(oracle.gemm_i8(a, w), want.astype(np.int32))


# ---- requantize (requantize_unit.sv) ----------------------------------------------

def q16(v):
    return int(round(v * 65536))


def test_requantize_unit_kats():
    L = oracle.lib()
    assert L.or_requant_q16(10, q16(1.0), 0) == 10
    assert L.or_requant_q16(300, q16(1.0), 0) == 127
    assert L.or_requant_q16(-300, q16(1.0), 0) == -127
    assert L.or_requant_q16(3, q16(0.5), 0) == 2        # 1.5 -> 2
    assert L.or_requant_q16(5, q16(0.5), 0) == 2        # 2.5 -> 2 (half to even)
    assert L.or_requant_q16(-4, q16(0.5), 1) == 0       # non-negative clamp
    assert L.or_requant_q16(10, q16(0.5), 0) == 5
    assert L.or_requant_q16(11, q16(0.5), 0) == 6       # 5.5 -> 6
    acc = np.array([10, 300, -300, 3, 5, -11, 11], np.int32)
    mult = np.array([1.0, 1.0, 1.0, 0.5, 0.5, 1.0, 0.5], F32)
    assert list(oracle.requant_f32(acc, mult)) == [10, 127, -127, 2, 2, -11, 6]


def test_requant_f32_equals_q16_where_exact():
    # for a Q16.16 multiplier m and |acc| < 2^15 the float32 product is exact,
    # so the fp32 requantizer must agree with the RTL's integer one everywhere
    rng = np.random.default_rng(5)
    L = oracle.lib()
    for _ in range(20):
        mq = int(rng.integers(1, 1 << 17))
        acc = rng.integers(-(1 << 15), 1 << 15, 2000).astype(np.int32)
        y = oracle.requant_f32(acc, np.full(acc.size, F32(mq / 65536.0)))
        want = [L.or_requant_q16(int(a), mq, 0) for a in acc]
        assert list(y) == want


# ---- argmax (argmax_reduction.sv, GI:671) ------------------------------------------

def test_argmax_kats():
    v = np.zeros(128, np.int32)
    v[0], v[1], v[2] = 10, 55, 55
    v[64], v[65] = 40, 100
    best = oracle.C.c_int32()
    L = oracle.lib()
    assert L.or_argmax_i32_tiles(oracle.ptr(v, oracle.C.c_int32), 128, 64, oracle.C.byref(best)) == 65
    assert best.value == 100
    assert L.or_argmax_i32_tiles(oracle.ptr(v, oracle.C.c_int32), 64, 64, oracle.C.byref(best)) == 1
    f = np.array([1.0, 3.0, -2.0, 3.0, 3.0], F32)
    assert L.or_argmax_first(oracle.ptr(f, oracle.C.c_float), 5) == int(np.argmax(f)) == 1


def test_argmax_i32_equals_numpy_argmax():
    """or_argmax_i32_tiles over 128-wide vocabulary tiles (EX:1651-1668) is
    np.argmax (first maximum) on INT32 vectors, including ties planted across
    tiles and at the last element."""
    rng = np.random.default_rng(17)
    L = oracle.lib()
    best = oracle.C.c_int32()
    for n in (1, 127, 128, 129, 32000):
        for _ in range(5):
            v = rng.integers(-(1 << 31), (1 << 31) - 1, n, dtype=np.int64).astype(np.int32)
            if n > 3:
                top = int(v.max())
                for i in rng.choice(n, 3, replace=False):
                    v[i] = top
            got = L.or_argmax_i32_tiles(oracle.ptr(v, oracle.C.c_int32), n, 128, oracle.C.byref(best))
            assert got == int(np.argmax(v)) and best.value == int(v.max())


# ---- causal mask (causal_mask_unit.sv, EX:1157-1184) -------------------------------

def causal_mask(s, qb, kb, qrc, kcc):
    out = np.empty_like(s)
    L = oracle.lib()
    L.or_causal_mask_tile(oracle.ptr(s, oracle.C.c_int32), s.shape[0], s.shape[1], qb, kb, qrc, kcc,
                          oracle.ptr(out, oracle.C.c_int32))
    return out


def test_causal_mask_kat():
    """tb_causal_mask_unit.sv:101-126: prefill, query base 0, key base 0, one
    active row, four active columns, scores 11..14: column 0 is kept, columns
    1-4 become MASK_NEG_INF, and the inactive second row is 0."""
    s = np.zeros((8, 64), np.int32)
    s[0, :4] = [11, 12, 13, 14]
    s[1, :] = 99
    out = causal_mask(s, 0, 0, 1, 4)
    assert out[0, 0] == 11
    assert list(out[0, 1:5]) == [-1000000000] * 4
    assert not out[1].any()


def test_causal_mask_rule():
    """Every (query base, key base, counts) of a small sweep against the rule
    written out element by element: kept when the row and column are active
    and key position <= query position."""
    rng = np.random.default_rng(3)
    for qb, kb, qrc, kcc in [(8, 0, 8, 64), (0, 0, 8, 64), (70, 64, 5, 30), (3, 10, 8, 64), (100, 40, 0, 64)]:
        s = rng.integers(-1000, 1000, (8, 64)).astype(np.int32)
        out = causal_mask(s, qb, kb, qrc, kcc)
        for r in range(8):
            for c in range(64):
                want = 0 if r >= qrc else (s[r, c] if c < kcc and kb + c <= qb + r else -1000000000)
                assert out[r, c] == want


# ---- RoPE (TL:59-80, rope_unit.sv, rope ROM) ---------------------------------------

def test_rope_table_bit_exact_vs_golden():
    z = golden("rope.npz")
    from models import rope_cache
    cos, sin = rope_cache(2048, 64, 10000.0)
    pos = z["positions"]
    assert bits_equal(cos[pos], z["cos"]) and bits_equal(sin[pos], z["sin"])


def test_rope_table_matches_rom_memh():
    """EX:656-681 wrote rope_{cos,sin}_rom.memh as int(round(65536 v)) of the
    golden table's first 32 dims.  Every sampled word matches except at one
    frequency (dim 5), where the ROM's NumPy computed theta ** (10/64) one ulp
    away from this one; the drift that causes grows with the position and
    stays within 4 Q16.16 LSBs (6e-5).  The golden vectors of this NumPy
    (test above) pin the table bit for bit."""
    z = golden("rope_rom.npz")
    from models import rope_cache
    cos, sin = rope_cache(2048, 64, 10000.0)
    pos = z["positions"]
    to_q16 = np.vectorize(lambda v: int(round(float(v) * 65536.0)))
    for tab, rom in ((cos, z["cos_q16"]), (sin, z["sin_q16"])):
        d = to_q16(tab[pos, :32]) - rom
        assert np.array_equal(np.delete(d, 5, axis=1), np.zeros((d.shape[0], 31), d.dtype))
        assert np.abs(d[:, 5]).max() <= 4


def test_apply_rope_bit_exact_vs_golden():
    z = golden("rope.npz")
    cos, sin = z["cos"], z["sin"]   # positions 0..63 are the first rows
    for p in range(z["q"].shape[1]):
        q = np.ascontiguousarray(z["q"][:, p, :])
        k = np.ascontiguousarray(z["k"][:, p, :])
        assert bits_equal(oracle.apply_rope(q, 32, 64, cos[p], sin[p]), z["q_rot"][:, p, :])
        assert bits_equal(oracle.apply_rope(k, 4, 64, cos[p], sin[p]), z["k_rot"][:, p, :])


def test_int8_rope_kats():
    # tb_rope_unit.sv:112-148: position 0 (cos = 1.0, sin = 0) is the identity
    L = oracle.lib()
    for v, pair in [(5, -3), (-127, 127), (64, 0)]:
        assert L.or_rotate_q16(v, pair, 65536, 0, 1) == v
        assert L.or_rotate_q16(v, pair, 65536, 0, 0) == v
    # a quarter turn: lower half -> -pair, upper half -> +pair
    assert L.or_rotate_q16(10, 20, 0, 65536, 1) == -20
    assert L.or_rotate_q16(10, 20, 0, 65536, 0) == 20


# ---- softmax / SiLU / exp / probabilities ------------------------------------------

def test_expf_close_to_libm():
    xs = np.concatenate([np.linspace(-80, 60, 200001), [0.0, -1e-8, 1e-8]]).astype(F32)
    ys = oracle.expf(xs)
    ref = np.array([math.exp(float(v)) for v in xs])
    ulp = np.spacing(ref.astype(F32)).astype(np.float64)
    err = np.abs(ys.astype(np.float64) - ref) / ulp
    assert err.max() <= 2.0, err.max()
    assert oracle.expf(np.array([0.0], F32))[0] == 1.0
    assert oracle.expf(np.array([-80.5], F32))[0] == 0.0


def test_softmax_close_to_golden():
    z = golden("softmax_silu.npz")
    for key in z.files:
        if key.startswith("s_"):
            n = key[2:]
            s, p = z[f"s_{n}"], z[f"p_{n}"]
            for r in range(s.shape[0]):
                got = oracle.softmax_row(s[r])
                assert np.allclose(got, p[r], rtol=1e-6, atol=1e-9), n


def test_silu_close_to_golden():
    z = golden("softmax_silu.npz")
    got = oracle.silu(z["silu_x"])
    assert np.allclose(got, z["silu_y"], rtol=1e-6, atol=1e-30)


def test_probability_quantization_bit_exact_vs_exporter():
    z = golden("softmax_silu.npz")
    assert np.array_equal(oracle.quantize_probs(z["prob_p"]), z["prob_q"])


def test_block_sum_is_butterfly_tree():
    rng = np.random.default_rng(2)
    v = (rng.standard_normal(64) * 10).astype(F32)
    a = v.copy()
    for off in (32, 16, 8, 4, 2, 1):
        a = np.array([F32(a[i] + a[i ^ off]) for i in range(64)], F32)
    got = oracle.lib().or_block_sum64(oracle.ptr(v, oracle.C.c_float))
    assert F32(got) == a[0]
    assert abs(float(got) - math.fsum(map(float, v))) < 1e-4


# ---- attention and composed layer vs the golden model -------------------------------

def test_int8_attention_tracks_golden_float_attention():
    """GI:136-182 computes attention in float; the build's attention runs the
    INT8 score and probability x V contractions over the INT8 cache.  On the
    golden's own Q/K/V (layer 0 of the tiny model, 6 causal tokens) the INT8
    result must stay within the INT8 quantization error of the golden."""
    arrays, z = tiny_from_golden()
    cfg = arrays.c_config()
    H, Hkv, hd = 4, 2, 64
    q, k, v = z["attn_q"], z["attn_k"], z["attn_v"]
    S = q.shape[0]
    cos, sin = arrays.rope_cos, arrays.rope_sin
    q_rot = np.stack([oracle.apply_rope(q[t], H, hd, cos[t], sin[t]) for t in range(S)])
    k_rot = np.stack([oracle.apply_rope(k[t], Hkv, hd, cos[t], sin[t]) for t in range(S)])
    sk = np.abs(k_rot).reshape(S, Hkv, hd).max(axis=(0, 2)) / 127.0
    sv = np.abs(v).reshape(S, Hkv, hd).max(axis=(0, 2)) / 127.0
    sk = np.tile(sk.astype(F32), (2, 1))
    sv = np.tile(sv.astype(F32), (2, 1))
    kc, vc = arrays.new_cache()
    for t in range(S):
        for g in range(Hkv):
            kc[0, g, t] = oracle.quantize_static(k_rot[t, g * hd:(g + 1) * hd], sk[0, g])
            vc[0, g, t] = oracle.quantize_static(v[t, g * hd:(g + 1) * hd], sv[0, g])
    L = oracle.lib()
    golden_att = z["attn_attended"]
    golden_w = z["attn_weights"]                      # [H][S][S], float64
    for t in range(S):
        q8, sq = oracle.quantize_int8(q_rot[t])
        att = np.empty(H * hd, F32)
        probs = np.empty((H, t + 1), np.int8)
        L.or_attention_row(oracle.C.byref(cfg), 0, t, oracle.ptr(q8, oracle.C.c_int8), sq,
                           oracle.ptr(kc, oracle.C.c_int8), oracle.ptr(vc, oracle.C.c_int8),
                           oracle.ptr(sk, oracle.C.c_float), oracle.ptr(sv, oracle.C.c_float),
                           oracle.ptr(att, oracle.C.c_float), None, oracle.ptr(probs, oracle.C.c_int8), None)
        # probabilities: within half an INT8 step plus the Q/K quantization error
        assert np.abs(probs / 127.0 - golden_w[:, t, :t + 1]).max() < 0.03
        # attended: within a few percent of the output range
        assert np.abs(att - golden_att[t]).max() < 0.04 * np.abs(golden_att[t]).max() + 1e-6


def _layer0_trace(arrays):
    D, F = arrays.cfg["hidden"], arrays.cfg["intermediate"]
    kvd = arrays.cfg["n_kv_heads"] * arrays.cfg["head_dim"]
    return dict(attn_in=np.empty(D, F32), attn_in_q=np.empty(D, np.int8), attn_in_s=np.empty(1),
                qkv_acc=np.empty(D + 2 * kvd, np.int32), qkv=np.empty(D + 2 * kvd, F32),
                attended=np.empty(D, F32), x_after_attn=np.empty(D, F32), hidden=np.empty(F, F32),
                out=np.empty(D, F32))


def test_decoder_layer_vs_golden_one_token():
    """GI:256-281 at one token (position 0), where per-row and per-tensor
    activation scales coincide.  Everything up to the attention is bit-exact;
    the INT8-KV attention output and what follows stay within its error."""
    arrays0, z = tiny_from_golden()
    kvd = 128
    k, v = z["layer_k"][0], z["layer_v"][0]
    sk = (np.abs(k).reshape(2, 64).max(axis=1) / 127.0).astype(F32)
    sv = (np.abs(v).reshape(2, 64).max(axis=1) / 127.0).astype(F32)
    arrays, _ = tiny_from_golden(kv_sk=np.tile(sk, (2, 1)), kv_sv=np.tile(sv, (2, 1)))
    orc = oracle.Oracle(arrays)
    kc, vc = arrays.new_cache()
    tr = _layer0_trace(arrays)
    x0 = orc.embed(int(z["layer_tok"]))
    assert bits_equal(x0, z["layer_x"][0])
    y = orc.decode_row(0, 0, x0, kc, vc, tr)
    D = 256
    assert bits_equal(tr["attn_in"], z["layer_attn_input"][0])
    assert np.array_equal(tr["qkv_acc"][:D], z["layer_q_acc"][0])
    assert bits_equal(tr["qkv"][:D], z["layer_q"][0])
    assert bits_equal(tr["qkv"][D:D + kvd], z["layer_k"][0])
    assert bits_equal(tr["qkv"][D + kvd:], z["layer_v"][0])
    # at one token the golden's attention returns V itself; the INT8 cache holds
    # V to within half a step of its static scale
    step = np.repeat(sv, 64 * 2)[:D]
    assert np.all(np.abs(tr["attended"] - z["layer_attended"][0]) <= 0.5 * step * 1.01 + 1e-7)
    ref_o = z["layer_x_after_attn"][0] - z["layer_x"][0]
    assert np.abs(tr["x_after_attn"] - z["layer_x_after_attn"][0]).max() < 0.05 * np.abs(ref_o).max()
    ref_h = z["layer_hidden"][0]
    assert np.abs(tr["hidden"] - ref_h).max() < 0.05 * np.abs(ref_h).max()
    ref_f = z["layer_y"][0] - z["layer_x_after_attn"][0]
    assert np.abs(y - z["layer_y"][0]).max() < 0.05 * (np.abs(ref_o).max() + np.abs(ref_f).max())


def test_forward_one_token_vs_golden():
    """GI:437-467 + GI:671 at one token through both layers with the quantized
    LM head: logits track the golden and the greedy id matches it."""
    arrays, z = tiny_from_golden(kv_sk=np.full((2, 2), 0.01, F32), kv_sv=np.full((2, 2), 0.01, F32))
    orc = oracle.Oracle(arrays)
    for t in (17, 250, 511):
        kc, vc = arrays.new_cache()
        x = orc.embed(t)
        for layer in range(2):
            x = orc.decode_row(layer, 0, x, kc, vc)
        tok, best, logits = orc.lm_head(x, want_logits=True)
        ref = z[f"fwd_logits_{t}"]
        assert np.abs(logits - ref).max() < 0.02 * np.abs(ref).max()
        srt = np.sort(ref)
        if srt[-1] - srt[-2] > 0.04 * np.abs(ref).max():
            assert tok == int(z[f"fwd_token_{t}"])


def test_generate_equals_token_by_token_forward():
    """Greedy generation with the KV cache equals the per-token definition
    (prefill rows are the same rows as sequential decode)."""
    arrays, _ = tiny_from_golden(kv_sk=np.full((2, 2), 0.01, F32), kv_sv=np.full((2, 2), 0.01, F32))
    orc = oracle.Oracle(arrays)
    prompt = [3, 77, 200, 5]
    toks, _ = orc.generate(prompt, 6)
    kc, vc = arrays.new_cache()
    seq = list(prompt)
    for step in range(6):
        for p in range(len(seq) - (1 if step else len(seq)), len(seq)):
            tok = oracle.lib().or_forward_token(oracle.C.byref(orc.cm), seq[p], p, 2,
                                                oracle.ptr(kc, oracle.C.c_int8), oracle.ptr(vc, oracle.C.c_int8), None)
        assert tok == toks[step]
        seq.append(int(tok))


def test_attention_pv_multiplier_closed_form():
    """Closed form for the P.V step (EX:1839, softmax_wrapper.sv:23: the
    probability scale is 1/127).  With an all-zero query every key scores 0,
    so softmax gives p = 1/n and the INT8 probability is rne(127/n) for every
    key; the accumulator is then rne(127/n) * sum_t v8[t][d] and the output
    is that integer times f32((1/127) * s_v), bit for bit.  A 1/128 scale,
    a dropped key or a transposed V index fails it."""
    cfg = dict(oracle.SMALL_CFG, n_layers=1)
    c = oracle.OrConfig(*(cfg[k] for k in ("hidden", "intermediate", "n_layers", "n_heads", "n_kv_heads",
                                            "head_dim", "vocab", "max_pos", "rms_eps", "rope_theta")))
    H, Hkv, hd = cfg["n_heads"], cfg["n_kv_heads"], 64
    rng = np.random.default_rng(4)
    sk = rng.uniform(0.01, 0.1, (1, Hkv)).astype(F32)
    sv = rng.uniform(0.01, 0.1, (1, Hkv)).astype(F32)
    kc = np.zeros((1, Hkv, cfg["max_pos"], hd), np.int8)
    vc = np.zeros_like(kc)
    q8 = np.zeros(H * hd, np.int8)
    for n in (1, 3, 5, 64, 65, 200):
        kc[0, :, :n] = rng.integers(-127, 128, (Hkv, n, hd))
        vc[0, :, :n] = rng.integers(-127, 128, (Hkv, n, hd))
        att = np.empty(H * hd, F32)
        acc = np.empty(H * hd, np.int32)
        probs = np.empty((H, n), np.int8)
        oracle.lib().or_attention_row(oracle.C.byref(c), 0, n - 1, oracle.ptr(q8, oracle.C.c_int8), 0.01,
                                      oracle.ptr(kc, oracle.C.c_int8), oracle.ptr(vc, oracle.C.c_int8),
                                      oracle.ptr(sk, oracle.C.c_float), oracle.ptr(sv, oracle.C.c_float),
                                      oracle.ptr(att, oracle.C.c_float), None, oracle.ptr(probs, oracle.C.c_int8),
                                      oracle.ptr(acc, oracle.C.c_int32))
        p8 = int(np.rint(np.float32(127.0) * (np.float32(1.0) / np.float32(n))))
        assert np.all(probs == p8), n
        for h in range(H):
            g = h // (H // Hkv)
            want_acc = p8 * vc[0, g, :n].astype(np.int64).sum(axis=0)
            assert np.array_equal(acc[h * hd:(h + 1) * hd], want_acc), (n, h)
            mult = np.float32(np.float64(1.0 / 127.0) * np.float64(sv[0, g]))
            want = want_acc.astype(F32) * mult
            assert bits_equal(att[h * hd:(h + 1) * hd], want), (n, h)
            wrong = want_acc.astype(F32) * np.float32(np.float64(1.0 / 128.0) * np.float64(sv[0, g]))
            assert not bits_equal(att[h * hd:(h + 1) * hd], wrong)


# ---- layer-major multi-row forms (used to check full-size runs) ----------------------

def test_decode_rows_equal_decode_row():
    """or_decode_rows (rows of one prompt, layer-major; and rows of different
    sequences at different positions) equals or_decode_row row by row: every
    output bit and every cache row."""
    m = oracle.synthetic_model(dict(oracle.SMALL_CFG), seed=3)
    orc = oracle.Oracle(m)
    L = m.cfg["n_layers"]
    prompt = np.random.default_rng(1).integers(0, m.cfg["vocab"], 37)
    # one prompt, layer-major vs token by token
    c1, c2 = m.new_cache(), m.new_cache()
    x = np.stack([orc.embed(int(t)) for t in prompt]).astype(F32)
    for layer in range(L):
        orc.decode_rows(layer, np.arange(prompt.size), x, [c1] * prompt.size)
    for i, t in enumerate(prompt):
        y = orc.embed(int(t))
        for layer in range(L):
            y = orc.decode_row(layer, i, y, *c2)
        assert bits_equal(x[i], y), i
    assert np.array_equal(c1[0], c2[0]) and np.array_equal(c1[1], c2[1])
    # three sequences at different positions (the batched-decode shape)
    rng = np.random.default_rng(2)
    caches = [m.new_cache() for _ in range(3)]
    for kc, vc in caches:
        kc[:, :, :100] = rng.integers(-127, 128, kc[:, :, :100].shape)
        vc[:, :, :100] = rng.integers(-127, 128, vc[:, :, :100].shape)
    copies = [(kc.copy(), vc.copy()) for kc, vc in caches]
    pos = np.array([7, 99, 40], np.int32)
    x = rng.standard_normal((3, m.cfg["hidden"])).astype(F32)
    want = [x[r].copy() for r in range(3)]
    for layer in range(L):
        orc.decode_rows(layer, pos, x, caches)
        for r in range(3):
            want[r] = orc.decode_row(layer, int(pos[r]), want[r], *copies[r])
    for r in range(3):
        assert bits_equal(x[r], want[r]), r
        assert np.array_equal(caches[r][0], copies[r][0]) and np.array_equal(caches[r][1], copies[r][1])
    tok, lg = orc.lm_head_rows(x)
    for r in range(3):
        assert (int(tok[r]), F32(lg[r])) == tuple(orc.lm_head(x[r])[:1]) + (F32(orc.lm_head(x[r])[1]),)


def test_generate_layer_major_equals_generate():
    m = oracle.synthetic_model(dict(oracle.SMALL_CFG), seed=4)
    orc = oracle.Oracle(m)
    prompt = np.array([5, 17, 1000, 3, 3, 2047, 64, 9, 9, 100], np.int32)
    c1, c2 = m.new_cache(), m.new_cache()
    want, _ = orc.generate(prompt, 9, cache=c1)
    got = orc.generate_layer_major(prompt, 9, cache=c2)
    assert np.array_equal(got, want)
    assert np.array_equal(c1[0], c2[0]) and np.array_equal(c1[1], c2[1])
