"""Decoder-layer and model-level parity through the C-ABI against the CPU
oracle: the TinyLlama-shape decode layer over a prefilled INT8 KV cache,
prefill vs token-by-token decode, greedy generation and batched decode.
Token ids, KV rows, INT8 values and float outputs must be bit-identical."""
import numpy as np
import pytest

import oracle
from gpu_util import assert_bits_equal, dev, host

pytestmark = pytest.mark.gpu
F32 = np.float32


def engine_for(model, max_seqs=1):
    from lpta.engine import Engine
    return Engine(model.cfg, max_seqs=max_seqs).load_model(model)


def fill_cache_random(eng, model, seq, n_tokens, seed, kc=None, vc=None):
    """Seeded uniform INT8 K/V rows at positions 0..n_tokens-1 (written to the
    engine and, when given, to the oracle's logical cache)."""
    rng = np.random.default_rng(seed)
    c = model.cfg
    for layer in range(c["n_layers"]):
        for g in range(c["n_kv_heads"]):
            k = rng.integers(-127, 128, (n_tokens, 64)).astype(np.int8)
            v = rng.integers(-127, 128, (n_tokens, 64)).astype(np.int8)
            eng.kv_write(seq, layer, g, 0, k, v)
            if kc is not None:
                kc[layer, g, :n_tokens] = k
                vc[layer, g, :n_tokens] = v


# ---- one TinyLlama-shape decoder layer, one decode step over a 512-token cache ----

@pytest.fixture(scope="module")
def layer_model():
    cfg = dict(oracle.TINYLLAMA_CFG, n_layers=1, vocab=64)
    return oracle.synthetic_model(cfg, seed=2024, kv_range=(0.01, 0.1))


def test_decode_layer_tinyllama_shape(layer_model):
    m = layer_model
    eng = engine_for(m)
    orc = oracle.Oracle(m)
    kc, vc = m.new_cache()
    fill_cache_random(eng, m, 0, 512, seed=77, kc=kc, vc=vc)
    x = np.random.default_rng(5).standard_normal(2048).astype(F32)
    xd = dev(x)
    eng.decode_layer(xd, layer=0, pos=512)
    want = orc.decode_row(0, 512, x, kc, vc)
    assert_bits_equal(host(xd), want, "layer output")
    for g in range(4):
        k, v = eng.kv_read(0, 0, g, 0, 513)
        assert_bits_equal(k, kc[0, g, :513], f"K cache head {g}")
        assert_bits_equal(v, vc[0, g, :513], f"V cache head {g}")
    eng.close()


@pytest.mark.parametrize("pos", [0, 63, 64, 127, 128, 511, 512, 2047])
def test_decode_layer_positions(layer_model, pos):
    """One TinyLlama-shape decode layer with `pos` cached rows (the new row at
    position pos): an empty cache, both sides of a 64-key block edge, both
    sides of the 512 keys the batch-1 attention keeps in registers, and the
    last position of a 2048-row cache.  The layer output and every K/V row
    equal the oracle bit for bit."""
    m = layer_model
    assert pos < m.cfg["max_pos"]
    eng = engine_for(m)
    orc = oracle.Oracle(m)
    kc, vc = m.new_cache()
    if pos:
        fill_cache_random(eng, m, 0, pos, seed=100 + pos, kc=kc, vc=vc)
    x = np.random.default_rng(pos).standard_normal(2048).astype(F32)
    xd = dev(x)
    eng.decode_layer(xd, layer=0, pos=pos)
    assert_bits_equal(host(xd), orc.decode_row(0, pos, x, kc, vc), f"layer output at position {pos}")
    for g in range(4):
        k, v = eng.kv_read(0, 0, g, 0, pos + 1)
        assert_bits_equal(k, kc[0, g, :pos + 1], f"K cache head {g}")
        assert_bits_equal(v, vc[0, g, :pos + 1], f"V cache head {g}")
    eng.close()


def test_decode_sharp_softmax_matches_oracle():
    """Decode attention with K/V scales of 1-3 (scores spread over hundreds,
    so most exponentials fall past the cut-off at -80): the batch-1 decode
    layer output and batched decode of three sequences over two layers equal
    the oracle bit for bit; the second layer's K/V rows are built from the
    first layer's attention output."""
    cfg = dict(oracle.TINYLLAMA_CFG, n_layers=2, vocab=512)
    m = oracle.synthetic_model(cfg, seed=31, kv_range=(1.0, 3.0))
    orc = oracle.Oracle(m)
    eng = engine_for(m)
    kc, vc = m.new_cache()
    fill_cache_random(eng, m, 0, 700, seed=8, kc=kc, vc=vc)
    x = np.random.default_rng(9).standard_normal(2048).astype(F32)
    xd = dev(x)
    eng.decode_layer(xd, layer=0, pos=700)
    assert_bits_equal(host(xd), orc.decode_row(0, 700, x, kc, vc), "batch-1 layer output")
    eng.close()
    B, steps = 3, 2
    eng = engine_for(m, max_seqs=B)
    start = np.array([100, 640, 1500], np.int32)
    toks = np.array([3, 77, 400], np.int32)
    caches = []
    for b in range(B):
        kc, vc = m.new_cache()
        fill_cache_random(eng, m, b, int(start[b]), seed=40 + b, kc=kc, vc=vc)
        caches.append((kc, vc))
    got = eng.decode_batch(toks, start, steps)
    for b in range(B):
        kc, vc = caches[b]
        tok = int(toks[b])
        for s in range(steps):
            x = orc.embed(tok)
            for layer in range(cfg["n_layers"]):
                x = orc.decode_row(layer, int(start[b]) + s, x, kc, vc)
            tok, _ = orc.lm_head(x)
            assert got[b, s] == tok, f"seq {b} step {s}"
        for layer in range(cfg["n_layers"]):
            for g in range(4):
                k, v = eng.kv_read(b, layer, g, 0, int(start[b]) + steps)
                assert_bits_equal(k, kc[layer, g, :int(start[b]) + steps], f"K seq {b} layer {layer}")
                assert_bits_equal(v, vc[layer, g, :int(start[b]) + steps], f"V seq {b} layer {layer}")
    eng.close()


# ---- small models: generation, prefill == decode, batched decode -------------------

@pytest.fixture(scope="module")
def small_model():
    return oracle.synthetic_model(dict(oracle.SMALL_CFG), seed=11)


def test_generate_matches_oracle(small_model):
    eng = engine_for(small_model)
    prompt = np.array([5, 17, 1000, 3, 3, 2047, 64], np.int32)
    got, stop = eng.generate(prompt, 24)
    want, _ = oracle.Oracle(small_model).generate(prompt, 24)
    assert stop == "max_tokens"
    assert_bits_equal(got, want, "token ids")
    eng.close()


def test_interleaved_sequences_match_oracle(small_model):
    """Batch-1 decode of two sequences in turns (3 steps of A, 5 of B, 4 of A,
    2 of B): every call starts from its own sequence's token and cursor, so
    each continuation equals the oracle's greedy generation of that prompt."""
    eng = engine_for(small_model, max_seqs=2)
    prompts = [np.array([5, 17, 1000, 3, 3, 2047, 64], np.int32), np.array([9, 8, 7, 300, 1], np.int32)]
    got = [[], []]
    for s, p in enumerate(prompts):
        tok, _ = eng.prefill(p, seq=s)
        got[s].append(tok)
    for s, n in ((0, 3), (1, 5), (0, 4), (1, 2)):
        toks, _ = eng.decode(n, seq=s)
        got[s].extend(int(t) for t in toks)
    orc = oracle.Oracle(small_model)
    for s, p in enumerate(prompts):
        want, _ = orc.generate(p, len(got[s]))
        assert_bits_equal(np.array(got[s], np.int32), want, f"sequence {s}")
    eng.close()


def test_prefill_cache_equals_sequential_decode(small_model):
    """Rows of a prefill are the same rows sequential decode would produce."""
    m = small_model
    eng = engine_for(m)
    prompt = np.random.default_rng(3).integers(0, m.cfg["vocab"], 70).astype(np.int32)
    tok, _ = eng.prefill(prompt)
    kc, vc = m.new_cache()
    orc = oracle.Oracle(m)
    x = None
    for i, t in enumerate(prompt):
        x = orc.embed(int(t))
        for layer in range(m.cfg["n_layers"]):
            x = orc.decode_row(layer, i, x, kc, vc)
    want_tok, _ = orc.lm_head(x)
    assert tok == want_tok
    for layer in range(m.cfg["n_layers"]):
        for g in range(m.cfg["n_kv_heads"]):
            k, v = eng.kv_read(0, layer, g, 0, prompt.size)
            assert_bits_equal(k, kc[layer, g, :prompt.size], "K")
            assert_bits_equal(v, vc[layer, g, :prompt.size], "V")
    eng.close()


def test_generate_eos_and_abort(small_model):
    import ctypes
    eng = engine_for(small_model)
    prompt = np.array([1, 2, 3], np.int32)
    free, _ = eng.generate(prompt, 12)
    eos = int(free[4])
    first = int(np.argmax(free == eos))
    got, stop = eng.generate(prompt, 12, eos_id=eos)
    assert stop == "eos" and got.tolist() == free[:first + 1].tolist()
    flag = ctypes.c_int32(1)
    got, stop = eng.generate(prompt, 12, abort_flag=flag)
    assert stop == "host_abort" and got.size == 0
    eng.close()


def test_decode_continues_after_eos_stop(small_model):
    """Steps replayed after the EOS stop record nothing and leave the cache
    and cursor as they were: decoding on from the stop gives the oracle's
    greedy continuation of the same sequence (EOS fed back like any token)."""
    eng = engine_for(small_model)
    prompt = np.array([3, 1, 4, 1, 5, 9, 2, 6], np.int32)
    free, _ = eng.generate(prompt, 30)
    eos = int(free[3])
    first = int(np.argmax(free == eos))
    got, stop = eng.generate(prompt, 30, eos_id=eos)      # stops inside the first 16-step chunk
    assert stop == "eos" and got.tolist() == free[:first + 1].tolist()
    more, stop2 = eng.decode(9, seq=0)
    assert stop2 == "max_tokens"
    want, _ = oracle.Oracle(small_model).generate(prompt, first + 1 + 9)
    assert_bits_equal(np.concatenate([got, more]), want, "tokens across the stop")
    eng.close()


def test_decode_batch_matches_oracle(small_model):
    m = small_model
    B, steps = 4, 6
    eng = engine_for(m, max_seqs=B)
    start = np.array([40, 100, 7, 180], np.int32)
    toks = np.array([9, 999, 2000, 0], np.int32)
    caches = []
    for b in range(B):
        kc, vc = m.new_cache()
        fill_cache_random(eng, m, b, int(start[b]), seed=100 + b, kc=kc, vc=vc)
        caches.append((kc, vc))
    got = eng.decode_batch(toks, start, steps)
    orc = oracle.Oracle(m)
    for b in range(B):
        kc, vc = caches[b]
        tok = int(toks[b])
        for s in range(steps):
            x = orc.embed(tok)
            for layer in range(m.cfg["n_layers"]):
                x = orc.decode_row(layer, int(start[b]) + s, x, kc, vc)
            tok, _ = orc.lm_head(x)
            assert got[b, s] == tok, f"seq {b} step {s}"
    eng.close()


def test_lm_head_argmax_operator(small_model):
    m = small_model
    eng = engine_for(m)
    x = np.random.default_rng(1).standard_normal(m.cfg["hidden"]).astype(F32)
    import ctypes
    tok, lg = ctypes.c_int32(), ctypes.c_float()
    logits = dev(np.zeros(m.cfg["vocab"], F32))
    eng.rt.call("tl_lm_head_argmax", dev(x), ctypes.byref(tok), ctypes.byref(lg), logits)
    want_tok, want_lg, want_logits = oracle.Oracle(m).lm_head(x, want_logits=True)
    assert_bits_equal(host(logits), want_logits, "logits")
    assert tok.value == want_tok and lg.value == want_lg
    eng.close()


def _leaf_sums(sq):
    """Sums of the 16 leaves of 128 squares each (NumPy's 8-accumulator leaf)."""
    import ctypes as C
    out = []
    for j in range(16):
        leaf = np.ascontiguousarray(sq[128 * j:128 * (j + 1)])
        out.append(np.float32(oracle.lib().or_pairwise_sum(oracle.ptr(leaf, C.c_float), 128)))
    return out


def _combine(lv, partner):
    """Pairwise levels 1, 2, 4, 8 over 16 leaf sums; partner(j, off) names the
    leaf position added to position j at level off; returns position 0."""
    v = list(lv)
    for off in (1, 2, 4, 8):
        v = [np.float32(v[j] + v[partner(j, off)]) for j in range(16)]
    return v[0]


def test_rmsnorm_leaf_order_lm_head(layer_model):
    """Rows whose 128-element leaves span 2^-4 .. 2^4 in magnitude, so that the
    float32 sum of squares depends on how the 16 leaf sums are paired.  The
    final RMSNorm + LM-head GEMV, whose prologue combines the leaf sums across
    lanes, must give the oracle's logits bit for bit.  The rows are first shown
    to tell NumPy's pairing (j ^ off) from a rotated one (j - off within 16)."""
    import ctypes
    m = layer_model
    eng = engine_for(m)
    rng = np.random.default_rng(77)
    told_apart = 0
    orc = oracle.Oracle(m)
    for r in range(24):
        x = rng.standard_normal(2048).astype(F32)
        x *= np.repeat(np.exp2(rng.integers(-4, 5, 16)), 128).astype(F32)
        sq = (x * x).astype(F32)
        lv = _leaf_sums(sq)
        right = _combine(lv, lambda j, off: j ^ off)
        assert right == np.float32(oracle.lib().or_pairwise_sum(oracle.ptr(sq, ctypes.c_float), sq.size))
        told_apart += right != _combine(lv, lambda j, off: (j & ~15) | ((j - off) & 15))
        tok, lg = ctypes.c_int32(), ctypes.c_float()
        logits = dev(np.zeros(m.cfg["vocab"], F32))
        eng.rt.call("tl_lm_head_argmax", dev(x), ctypes.byref(tok), ctypes.byref(lg), logits)
        want_tok, want_lg, want_logits = orc.lm_head(x, want_logits=True)
        assert_bits_equal(host(logits), want_logits, f"logits of row {r}")
        assert tok.value == want_tok and lg.value == want_lg
    assert told_apart >= 8
    eng.close()


def test_bad_arguments_raise_value_error(small_model):
    from lpta import TlValueError
    eng = engine_for(small_model)
    with pytest.raises(TlValueError):
        eng.prefill(np.array([], np.int32))
    with pytest.raises(TlValueError):
        eng.prefill(np.array([small_model.cfg["vocab"]], np.int32))
    with pytest.raises(TlValueError):
        eng.generate(np.arange(10, dtype=np.int32), small_model.cfg["max_pos"])
    with pytest.raises(TlValueError):
        eng.decode(1, seq=0)  # nothing prefilled
    eng.close()


@pytest.mark.parametrize("kslice,qkv_kslice,o_fuse", [("1", "1", "1"), ("1", "1", "0"), ("1", "0", "1"),
                                                    ("0", "1", "1")],
                         ids=["o_quantizing_itself", "qkv_and_down_k_sliced", "down_k_sliced", "whole_k"])
def test_decode_batch_tinyllama_heads(kslice, qkv_kslice, o_fuse, monkeypatch):
    """Batched decode with TinyLlama's attention geometry (32 query heads over
    4 KV heads, 4 query heads per attention workgroup): the
    down GEMM K-sliced with integer atomic adds folded by the next RMSNorm row
    prologue and the Q|K|V GEMM K-sliced with its sums dequantized by the
    attention kernel, with the O GEMM K-sliced too, quantizing the attention
    output itself at the row maxima the attention kernel writes per head
    (default) or after a quantization kernel (TL_BATCH_O_FUSE=0), the down
    GEMM alone K-sliced (TL_BATCH_QKV_KSLICE=0), and whole-K
    (TL_BATCH_KSLICE=0)."""
    monkeypatch.setenv("TL_BATCH_O_FUSE", o_fuse)
    monkeypatch.setenv("TL_BATCH_KSLICE", kslice)
    monkeypatch.setenv("TL_BATCH_QKV_KSLICE", qkv_kslice)
    cfg = dict(oracle.TINYLLAMA_CFG, n_layers=2, vocab=512)
    m = oracle.synthetic_model(cfg, seed=5)
    B, steps = 3, 3
    eng = engine_for(m, max_seqs=B)
    start = np.array([64, 300, 1000], np.int32)
    toks = np.array([1, 200, 511], np.int32)
    caches = []
    for b in range(B):
        kc, vc = m.new_cache()
        fill_cache_random(eng, m, b, int(start[b]), seed=300 + b, kc=kc, vc=vc)
        caches.append((kc, vc))
    got = eng.decode_batch(toks, start, steps)
    orc = oracle.Oracle(m)
    for b in range(B):
        kc, vc = caches[b]
        tok = int(toks[b])
        for s in range(steps):
            x = orc.embed(tok)
            for layer in range(cfg["n_layers"]):
                x = orc.decode_row(layer, int(start[b]) + s, x, kc, vc)
            tok, _ = orc.lm_head(x)
            assert got[b, s] == tok, f"seq {b} step {s}"
        for layer in range(cfg["n_layers"]):
            for g in range(4):
                k, v = eng.kv_read(b, layer, g, 0, int(start[b]) + steps)
                assert_bits_equal(k, kc[layer, g, :int(start[b]) + steps], f"K seq {b}")
                assert_bits_equal(v, vc[layer, g, :int(start[b]) + steps], f"V seq {b}")
    eng.close()


@pytest.mark.parametrize("B", [2, 17, 31])
def test_decode_batch_sizes_tinyllama_heads(B):
    """Batched decode at batch sizes 2, 17 and 31 (the M <= 32 GEMMs at row
    counts other than 32, the grouped attention's workgroup order at other
    grid sizes) with TinyLlama's geometry and ragged cache lengths: every id
    and every K/V row equals the oracle's (layer-major over the batch's rows,
    on up to 16 host threads)."""
    import os
    cfg = dict(oracle.TINYLLAMA_CFG, n_layers=2, vocab=512)
    m = oracle.synthetic_model(cfg, seed=900 + B)
    steps = 2
    eng = engine_for(m, max_seqs=B)
    rng = np.random.default_rng(B)
    start = rng.integers(1, 1500, B).astype(np.int32)
    toks = rng.integers(0, cfg["vocab"], B).astype(np.int32)
    caches = []
    for b in range(B):
        kc, vc = m.new_cache()
        fill_cache_random(eng, m, b, int(start[b]), seed=1000 + b, kc=kc, vc=vc)
        caches.append((kc, vc))
    got = eng.decode_batch(toks, start, steps)
    oracle.lib().or_set_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    orc = oracle.Oracle(m)
    tok = toks
    for s in range(steps):
        x = np.stack([orc.embed(int(t)) for t in tok]).astype(F32)
        for layer in range(cfg["n_layers"]):
            orc.decode_rows(layer, start + s, x, caches)
        want, _ = orc.lm_head_rows(x)
        assert_bits_equal(np.asarray(got[:, s], np.int32), want, f"ids of step {s}")
        tok = want
    for b in range(B):
        kc, vc = caches[b]
        n = int(start[b]) + steps
        for layer in range(cfg["n_layers"]):
            for g in range(cfg["n_kv_heads"]):
                k, v = eng.kv_read(b, layer, g, 0, n)
                assert_bits_equal(k, kc[layer, g, :n], f"K seq {b} layer {layer} head {g}")
                assert_bits_equal(v, vc[layer, g, :n], f"V seq {b} layer {layer} head {g}")
    eng.close()


def test_prefill_then_batched_decode():
    """Three prompts of 37, 128 and 300 tokens prefilled one sequence at a
    time (tl_prefill), continued together by tl_decode_batch from each
    prompt's predicted token, and the second sequence then alone by tl_decode
    (batch-1 graph replay from the batch's last token): the ids are the
    oracle's greedy generation over each prompt and the K/V rows of prompt and
    generated tokens the oracle's."""
    import os
    cfg = dict(oracle.TINYLLAMA_CFG, n_layers=2, vocab=1024)
    m = oracle.synthetic_model(cfg, seed=77)
    lens, steps = [37, 128, 300], 4
    eng = engine_for(m, max_seqs=len(lens))
    rng = np.random.default_rng(7)
    prompts = [rng.integers(0, cfg["vocab"], n).astype(np.int32) for n in lens]
    first = [eng.prefill(p, seq=b)[0] for b, p in enumerate(prompts)]
    got = eng.decode_batch(np.array(first, np.int32), np.array(lens, np.int32), steps)
    more = 5
    alone, stop = eng.decode(more, seq=1)
    assert stop == "max_tokens"
    oracle.lib().or_set_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    orc = oracle.Oracle(m)
    for b, p in enumerate(prompts):
        kc, vc = m.new_cache()
        extra = more if b == 1 else 0
        want = orc.generate_layer_major(p, steps + 1 + extra, cache=(kc, vc))
        assert first[b] == want[0], f"seq {b}: prefill token"
        assert_bits_equal(np.asarray(got[b], np.int32), want[1:steps + 1], f"seq {b}: batched ids")
        if extra:
            assert_bits_equal(np.asarray(alone, np.int32), want[steps + 1:], f"seq {b}: batch-1 ids after the batch")
        n = lens[b] + steps + extra
        for layer in range(cfg["n_layers"]):
            for g in range(cfg["n_kv_heads"]):
                k, v = eng.kv_read(b, layer, g, 0, n)
                assert_bits_equal(k, kc[layer, g, :n], f"K seq {b} layer {layer} head {g}")
                assert_bits_equal(v, vc[layer, g, :n], f"V seq {b} layer {layer} head {g}")
    eng.close()


def test_decode_timeline_steps_are_decode_steps(small_model):
    """tl_decode_timeline runs ordinary greedy steps from a graph captured
    with clock stamps: decoding on afterwards gives the tokens plain decode
    gives, every kernel of the step is stamped, gaps are non-negative and the
    per-class busy times and gaps add up to the step."""
    eng = engine_for(small_model)
    prompt = np.array([4, 8, 15, 16, 23, 42], np.int32)
    eng.prefill(prompt)
    want, _ = eng.decode(7)
    eng.prefill(prompt)
    tl = eng.decode_timeline(4)
    rest, _ = eng.decode(3)
    assert_bits_equal(rest, want[4:], "tokens after the timeline steps")
    L = small_model.cfg["n_layers"]
    assert tl["steps"] == 4 and tl["kernels"] == 5 * L + 2
    cls = tl["classes"]
    assert {k: v["launches"] for k, v in cls.items()} == {"qkv": L, "attn": L, "o": L, "glu": L, "down": L,
                                                         "lm_head": 1, "other": 1}
    busy = sum(v["busy_us"] for v in cls.values())
    gaps = sum(v["gap_us"] for v in cls.values())
    assert all(v["busy_us"] > 0 for v in cls.values())
    assert all(v["gap_us"] >= 0 for k, v in cls.items() if k != "other")
    assert abs(busy + gaps - tl["step_us"]) < 1e-6 * tl["step_us"] + 1e-3
    eng.close()


def test_graph_replay_equals_direct_launches(small_model):
    """The captured decode step (HIP graph) and direct launches give the same tokens."""
    import os
    eng = engine_for(small_model)
    prompt = np.array([4, 8, 15, 16, 23, 42], np.int32)
    graph_toks, _ = eng.generate(prompt, 12)
    eng.set_profiling(True)          # profiling launches kernels directly
    direct_toks, _ = eng.generate(prompt, 12)
    eng.set_profiling(False)
    assert_bits_equal(graph_toks, direct_toks, "tokens")
    eng.close()


def test_prefill_512_tinyllama_shape():
    """A 512-token prefill (M = 512 MFMA GEMMs, causal prefill attention) of a
    2-layer TinyLlama-shape model with the full 32000-entry vocabulary equals
    token-by-token decode in the oracle: next token, its logit and every K/V
    cache row."""
    cfg = dict(oracle.TINYLLAMA_CFG, n_layers=2)
    m = oracle.synthetic_model(cfg, seed=21)
    prompt = np.random.default_rng(8).integers(0, cfg["vocab"], 512).astype(np.int32)
    eng = engine_for(m)
    tok, lg = eng.prefill(prompt)
    orc = oracle.Oracle(m)
    kc, vc = m.new_cache()
    x = None
    for i, t in enumerate(prompt):
        x = orc.embed(int(t))
        for layer in range(cfg["n_layers"]):
            x = orc.decode_row(layer, i, x, kc, vc)
    want_tok, want_lg = orc.lm_head(x)
    assert (tok, lg) == (want_tok, want_lg)
    for layer in range(cfg["n_layers"]):
        for g in range(cfg["n_kv_heads"]):
            k, v = eng.kv_read(0, layer, g, 0, prompt.size)
            assert_bits_equal(k, kc[layer, g, :prompt.size], f"K layer {layer} head {g}")
            assert_bits_equal(v, vc[layer, g, :prompt.size], f"V layer {layer} head {g}")
    eng.close()


@pytest.mark.parametrize("n", [64, 100, 300])
def test_prefill_lengths_tinyllama_shape(n):
    """Prefills whose length is not a multiple of the GEMM row tiles (the
    packed-operand GEMMs pad A to 128 rows; the packed Q|K|V GEMM also
    rotates, quantizes and appends K/V and leaves Q for the attention tiles to
    quantize) on a 2-layer TinyLlama-shape model: next token, its logit and
    every K/V row equal token-by-token decode in the oracle."""
    cfg = dict(oracle.TINYLLAMA_CFG, n_layers=2, vocab=4096)
    m = oracle.synthetic_model(cfg, seed=40 + n)
    prompt = np.random.default_rng(n).integers(0, cfg["vocab"], n).astype(np.int32)
    eng = engine_for(m)
    tok, lg = eng.prefill(prompt)
    orc = oracle.Oracle(m)
    kc, vc = m.new_cache()
    x = None
    for i, t in enumerate(prompt):
        x = orc.embed(int(t))
        for layer in range(cfg["n_layers"]):
            x = orc.decode_row(layer, i, x, kc, vc)
    assert (tok, lg) == orc.lm_head(x)
    for layer in range(cfg["n_layers"]):
        for g in range(cfg["n_kv_heads"]):
            k, v = eng.kv_read(0, layer, g, 0, n)
            assert_bits_equal(k, kc[layer, g, :n], f"K layer {layer} head {g}")
            assert_bits_equal(v, vc[layer, g, :n], f"V layer {layer} head {g}")
    eng.close()


@pytest.mark.parametrize("n", [1000, 2048])
def test_prefill_long_tinyllama_shape(n):
    """Prefills past the 512 keys of the register-resident attention tiles
    (the general attention_tile_kernel, quantizing the float Q that the fused
    Q|K|V epilogue leaves), up to the 2048-position limit, on a 2-layer
    TinyLlama-shape model: next token, its logit and every K/V row equal the
    oracle's layer-major prefill (on up to 16 host threads) bit for bit."""
    import os
    cfg = dict(oracle.TINYLLAMA_CFG, n_layers=2, vocab=4096)
    m = oracle.synthetic_model(cfg, seed=70 + n)
    prompt = np.random.default_rng(n).integers(0, cfg["vocab"], n).astype(np.int32)
    eng = engine_for(m)
    tok, lg = eng.prefill(prompt)
    oracle.lib().or_set_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    orc = oracle.Oracle(m)
    kc, vc = m.new_cache()
    want_tok, want_lg = orc.prefill(prompt, (kc, vc))
    assert tok == want_tok
    assert F32(lg).view(np.uint32) == F32(want_lg).view(np.uint32)
    for layer in range(cfg["n_layers"]):
        for g in range(cfg["n_kv_heads"]):
            k, v = eng.kv_read(0, layer, g, 0, n)
            assert_bits_equal(k, kc[layer, g, :n], f"K layer {layer} head {g}")
            assert_bits_equal(v, vc[layer, g, :n], f"V layer {layer} head {g}")
    eng.close()


@pytest.mark.parametrize("pos0,rows", [(300, 100), (1000, 64), (1900, 148)])
def test_layer_rows_after_cached_rows(pos0, rows):
    """tl_layer_rows over `rows` tokens of a sequence that already holds pos0
    cached rows (the prefill path of a continuation: packed GEMMs, the fused
    Q|K|V epilogue, attention tiles that start mid-context): the layer output
    rows and every K/V row equal the oracle's layer-major rows at positions
    pos0 .. pos0 + rows - 1, bit for bit."""
    cfg = dict(oracle.TINYLLAMA_CFG, n_layers=1, vocab=64)
    m = oracle.synthetic_model(cfg, seed=500 + pos0)
    eng = engine_for(m)
    orc = oracle.Oracle(m)
    kc, vc = m.new_cache()
    fill_cache_random(eng, m, 0, pos0, seed=pos0, kc=kc, vc=vc)
    x = np.random.default_rng(rows).standard_normal((rows, cfg["hidden"])).astype(F32)
    xd = dev(x)
    eng.rt.call("tl_layer_rows", 0, 0, pos0, rows, xd)
    want = orc.decode_rows(0, np.arange(pos0, pos0 + rows, dtype=np.int32), x.copy(), [(kc, vc)] * rows)
    assert_bits_equal(host(xd), want, "layer output rows")
    n = pos0 + rows
    for g in range(cfg["n_kv_heads"]):
        k, v = eng.kv_read(0, 0, g, 0, n)
        assert_bits_equal(k, kc[0, g, :n], f"K head {g}")
        assert_bits_equal(v, vc[0, g, :n], f"V head {g}")
    eng.close()


@pytest.mark.parametrize("geom", [(1024, 3072, 16, 4), (512, 1536, 8, 2), (384, 1280, 6, 2)],
                         ids=["hidden1024", "hidden512", "hidden384_row_major"])
def test_prefill_other_geometry(geom):
    """Prefill of 200 rows at three more geometries.  Packed-operand GEMMs:
    hidden 1024, FFN 3072, 16 query / 4 KV heads (Q|K|V N = 1536, one 64-row
    tile per head, the 32 x 160 split tile not taken) and hidden 512, FFN
    1536, 8 / 2 heads (K = 512: each wavefront's quarter of K is the four
    register sets loaded before the main loop, which then never runs).
    Row-major GEMMs: hidden 384, FFN 1280 (K not a multiple of 512, so the
    packed path is not taken; Q|K|V post-processing in qkv_post_kernel, Q
    quantized there).  Next token, its logit and every K/V row equal
    token-by-token decode in the oracle."""
    hidden, ffn, nh, nkv = geom
    cfg = dict(oracle.TINYLLAMA_CFG, hidden=hidden, intermediate=ffn, n_heads=nh, n_kv_heads=nkv, n_layers=2,
               vocab=2048, max_pos=512)
    m = oracle.synthetic_model(cfg, seed=77)
    n = 200
    prompt = np.random.default_rng(77).integers(0, cfg["vocab"], n).astype(np.int32)
    eng = engine_for(m)
    tok, lg = eng.prefill(prompt)
    orc = oracle.Oracle(m)
    kc, vc = m.new_cache()
    x = None
    for i, t in enumerate(prompt):
        x = orc.embed(int(t))
        for layer in range(cfg["n_layers"]):
            x = orc.decode_row(layer, i, x, kc, vc)
    assert (tok, lg) == orc.lm_head(x)
    for layer in range(cfg["n_layers"]):
        for g in range(cfg["n_kv_heads"]):
            k, v = eng.kv_read(0, layer, g, 0, n)
            assert_bits_equal(k, kc[layer, g, :n], f"K layer {layer} head {g}")
            assert_bits_equal(v, vc[layer, g, :n], f"V layer {layer} head {g}")
    eng.close()


def test_generate_tinyllama_shape_matches_oracle():
    """Greedy generation on a 2-layer TinyLlama-shape model (hidden 2048, FFN
    5632, 32/4 heads, vocab 32000), on either decode path: the oracle's token
    ids and KV rows."""
    cfg = dict(oracle.TINYLLAMA_CFG, n_layers=2)
    m = oracle.synthetic_model(cfg, seed=31)
    prompt = np.random.default_rng(9).integers(0, cfg["vocab"], 20).astype(np.int32)
    eng = engine_for(m)
    got, stop = eng.generate(prompt, 12)
    assert stop == "max_tokens"
    orc = oracle.Oracle(m)
    kc, vc = m.new_cache()
    want, _ = orc.generate(prompt, 12, cache=(kc, vc))
    assert_bits_equal(got, want, "token ids")
    n = prompt.size + 11   # rows written: prompt + every fed-back token but the last
    for layer in range(2):
        for g in range(4):
            k, v = eng.kv_read(0, layer, g, 0, n)
            assert_bits_equal(k, kc[layer, g, :n], f"K layer {layer} head {g}")
            assert_bits_equal(v, vc[layer, g, :n], f"V layer {layer} head {g}")
    eng.close()


# ---- causal attention of a block of rows (prefill tiles) ----------------------------

@pytest.mark.parametrize("shape,pos0,rows,sharp", [
    ("tinyllama", 0, 1, False), ("tinyllama", 0, 77, False), ("tinyllama", 130, 64, False),
    ("tinyllama", 1900, 100, False), ("small", 5, 33, False), ("small", 0, 256, False),
    ("small", 96, 160, False), ("tinyllama", 0, 512, True), ("small", 96, 160, True),
    ("tinyllama", 1000, 200, True)])
def test_attention_rows_match_oracle(shape, pos0, rows, sharp):
    """tl_attention over rows at positions pos0 .. pos0 + rows - 1 of one
    sequence (the prefill path: INT8 MFMA tiles of 32 rows, partial last
    tiles, tiles that start mid-context) equals the oracle's per-row GQA
    attention over the same INT8 cache, bit for bit.  With `sharp`, Q scales
    of 0.5-2 put most of each row's scores more than 80 below its maximum,
    where the exponential is 0 by the cut-off rather than by the polynomial."""
    base = oracle.TINYLLAMA_CFG if shape == "tinyllama" else oracle.SMALL_CFG
    cfg = dict(base, n_layers=1, vocab=64)
    from lpta.engine import Engine
    eng = Engine(cfg, max_seqs=1)
    rng = np.random.default_rng(pos0 * 1000 + rows)
    Hkv, H = cfg["n_kv_heads"], cfg["n_heads"]
    D = H * 64
    sk = rng.uniform(0.01, 0.08, (1, Hkv)).astype(F32)
    sv = rng.uniform(0.01, 0.08, (1, Hkv)).astype(F32)
    eng.set_kv_scales(sk, sv)
    kc = np.zeros((1, Hkv, cfg["max_pos"], 64), np.int8)
    vc = np.zeros_like(kc)
    n = pos0 + rows
    for g in range(Hkv):
        kc[0, g, :n] = rng.integers(-127, 128, (n, 64))
        vc[0, g, :n] = rng.integers(-127, 128, (n, 64))
        eng.kv_write(0, 0, g, 0, kc[0, g, :n], vc[0, g, :n])
    q8 = rng.integers(-127, 128, (rows, D)).astype(np.int8)
    qs = rng.uniform(0.5, 2.0, rows) if sharp else rng.uniform(0.005, 0.05, rows)
    if sharp:   # the regime is reached: keys below max - 80 in the last row of head 0
        r = rows - 1
        s = (kc[0, 0, :pos0 + rows].astype(np.int64) @ q8[r, :64].astype(np.int64)).astype(F32)
        s = s * F32(qs[r] * float(sk[0, 0]) * 0.125)
        assert np.count_nonzero(s - s.max() < -80) > (pos0 + rows) // 2
    out = dev(np.zeros((rows, D), F32))
    eng.rt.call("tl_attention", 0, 0, pos0, rows, dev(q8), dev(qs), out)
    got = host(out)
    for r in range(rows):
        want = oracle.attention_row(cfg, 0, pos0 + r, q8[r], qs[r], kc, vc, sk, sv)
        assert_bits_equal(got[r], want, f"row {r} (position {pos0 + r})")
    eng.close()
