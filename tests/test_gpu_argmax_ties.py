"""Exact LM-head logit ties: the lower token id must win (GI:671 np.argmax;
rtl/compute/argmax_reduction.sv:49-56, KAT tb_argmax_reduction.sv:167-168).

Pairs of LM-head rows are made identical (same INT8 row, same scale), so the
two logits are equal to the bit.  The pairs' scales are raised eightfold so
that the greedy choice almost always falls on a pair.  Three pair layouts
cover the reductions the HIP path has:
  adjacent   (2i, 2i+1): the same wavefront and 32-column tile;
  tile_edge  (32j+31, 32j+32): neighbouring 32-column tiles (batched fold);
  far        (i, i+V/2): different LM-head workgroups (batch-1 key fold) and
             tiles.
Generation runs on every decode path: HIP-graph replay, direct launches,
batched decode and the standalone operator, and must
equal the oracle, whose argmax takes the first maximum.
"""
import ctypes

import numpy as np
import pytest

import oracle
from gpu_util import assert_bits_equal, dev, host

pytestmark = pytest.mark.gpu
F32 = np.float32
CFG = dict(oracle.TINYLLAMA_CFG, n_layers=2)
V = CFG["vocab"]


def pairs(layout):
    if layout == "adjacent":
        lo = np.arange(0, V, 2)
        return lo[::5], lo[::5] + 1
    if layout == "tile_edge":
        lo = np.arange(31, V - 1, 32)
        return lo, lo + 1
    lo = np.arange(0, V // 2, 3)
    return lo, lo + V // 2


@pytest.fixture(scope="module")
def base_model():
    return oracle.synthetic_model(CFG, seed=41)


def tied_model(base, layout):
    lo, hi = pairs(layout)
    lm_w = base.lm_w.copy()
    lm_s = base.lm_s.copy()
    lm_s[lo] *= F32(8.0)
    lm_w[hi] = lm_w[lo]
    lm_s[hi] = lm_s[lo]
    m = oracle.ModelArrays(cfg=dict(base.cfg), layers=base.layers, lm_w=lm_w, lm_s=lm_s, g_final=base.g_final,
                           emb=base.emb, emb_s=base.emb_s, rope_cos=base.rope_cos, rope_sin=base.rope_sin,
                           kv_sk=base.kv_sk, kv_sv=base.kv_sv)
    return m, set(lo.tolist()), set(hi.tolist())


LAYOUTS = pytest.mark.parametrize("layout", ["adjacent", "tile_edge", "far"])


def assert_ties_resolved(got, want, lo, hi, what):
    assert_bits_equal(np.asarray(got, np.int32), np.asarray(want, np.int32), what)
    ids = np.asarray(got).ravel().tolist()
    assert not (set(ids) & hi), f"{what}: a higher id of a tied pair won"
    assert sum(t in lo for t in ids) >= len(ids) // 2, f"{what}: too few steps fell on a tied pair to test the rule"


@LAYOUTS
def test_operator_ties(base_model, layout):
    """tl_lm_head_argmax (one key per row, atomicMax fold) on random rows."""
    from lpta.engine import Engine
    m, lo, hi = tied_model(base_model, layout)
    eng = Engine(CFG).load_model(m)
    orc = oracle.Oracle(m)
    rng = np.random.default_rng(6)
    got, want = [], []
    for _ in range(12):
        x = rng.standard_normal(CFG["hidden"]).astype(F32)
        tok, lg = ctypes.c_int32(), ctypes.c_float()
        logits = dev(np.zeros(V, F32))
        eng.rt.call("tl_lm_head_argmax", dev(x), ctypes.byref(tok), ctypes.byref(lg), logits)
        wt, wl, wlog = orc.lm_head(x, want_logits=True)
        assert_bits_equal(host(logits), wlog, "logits")
        got.append(tok.value)
        want.append(wt)
    assert_ties_resolved(got, want, lo, hi, f"operator ({layout})")
    eng.close()


@LAYOUTS
@pytest.mark.parametrize("path", ["graph", "direct"])
def test_generate_ties(base_model, layout, path):
    """Batch-1 generation: the fused LM-head GEMV keeps one argmax key per
    workgroup and the token bookkeeping kernel folds them."""
    from lpta.engine import Engine
    m, lo, hi = tied_model(base_model, layout)
    eng = Engine(CFG).load_model(m)
    if path == "direct":
        eng.set_profiling(True)   # profiling launches every kernel directly
    prompt = np.array([17, 4000, 31999, 2, 250], np.int32)
    got, _ = eng.generate(prompt, 10)
    want, _ = oracle.Oracle(m).generate(prompt, 10)
    assert_ties_resolved(got, want, lo, hi, f"{path} ({layout})")
    eng.close()


@LAYOUTS
def test_decode_batch_ties(base_model, layout):
    """Batched decode: the packed LM-head GEMM keeps one key per 32-column
    tile and row, and argmax_tiles folds them."""
    from lpta.engine import Engine
    m, lo, hi = tied_model(base_model, layout)
    B, steps = 4, 6
    eng = Engine(CFG, max_seqs=B).load_model(m)
    orc = oracle.Oracle(m)
    prompts = [np.array([5 + b, 900 * b + 1, 77], np.int32) for b in range(B)]
    first, caches = [], []
    for b, p in enumerate(prompts):
        tok, _ = eng.prefill(p, seq=b)
        cache = m.new_cache()
        want_tok, _ = orc.prefill(p, cache)
        assert tok == want_tok
        first.append(tok)
        caches.append(cache)
    got = eng.decode_batch(np.array(first, np.int32), np.array([p.size for p in prompts], np.int32), steps)
    x = np.stack([orc.embed(t) for t in first]).astype(F32)
    want = np.empty((B, steps), np.int32)
    for s in range(steps):
        for layer in range(CFG["n_layers"]):
            orc.decode_rows(layer, np.array([p.size + s for p in prompts], np.int32), x, caches)
        want[:, s], _ = orc.lm_head_rows(x)
        x = np.stack([orc.embed(int(t)) for t in want[:, s]]).astype(F32)
    assert_ties_resolved(got, want, lo, hi, f"batched ({layout})")
    eng.close()
