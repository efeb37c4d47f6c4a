"""Token-id parity at the full sizes of the benchmark workloads, on the
22-layer TinyLlama-1.1B-shape model (hidden 2048, 32/4 heads, FFN 5632,
vocab 32000; reference geometry model/tinyllama.py:205-221), against the CPU
oracle run on the host cores:

* 512-token prefill: next token, its logit and all 22 x 4 K/V planes x 512 rows
  (model/tinyllama_gemm_int8.py:437-467);
* 128-token prompt + 256 greedy tokens on both batch-1 decode paths: every id
  and every K/V row written (GI:629-685);
* 32 sequences x 1984 seeded cache rows x 64 batched decode steps: all 2048
  ids and the 64 rows each sequence appends.

The oracle runs layer-major over the rows it can batch (or_decode_rows, pinned
bit-exact to or_decode_row on the CPU), on up to 16 host threads.
"""
import os
import time

import numpy as np
import pytest

import oracle
from gpu_util import assert_bits_equal

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]
F32 = np.float32
FULL = dict(oracle.TINYLLAMA_CFG)
SEED = 1234


def log(msg):
    print(f"[fullsize] {msg}", flush=True)


def oracle_threads():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


@pytest.fixture(scope="module")
def full():
    from lpta.engine import Engine
    t = time.time()
    eng = Engine(FULL, max_seqs=32)
    host = eng.load_random(SEED)
    arrays = oracle.ModelArrays(**vars(host))
    oracle.lib().or_set_threads(oracle_threads())
    log(f"22-layer model loaded in {time.time() - t:.1f}s; oracle threads {oracle_threads()}")
    yield eng, arrays, oracle.Oracle(arrays)
    eng.close()


def check_kv(eng, seq, cache, t0, n, what):
    kc, vc = cache
    for layer in range(FULL["n_layers"]):
        for g in range(FULL["n_kv_heads"]):
            k, v = eng.kv_read(seq, layer, g, t0, n)
            assert_bits_equal(k, kc[layer, g, t0:t0 + n], f"{what}: K layer {layer} head {g}")
            assert_bits_equal(v, vc[layer, g, t0:t0 + n], f"{what}: V layer {layer} head {g}")


def test_prefill_512_22_layers(full):
    eng, arrays, orc = full
    prompt = np.random.default_rng(3).integers(0, FULL["vocab"], 512).astype(np.int32)
    tok, lg = eng.prefill(prompt, seq=0)
    t = time.time()
    cache = arrays.new_cache()
    want_tok, want_lg = orc.prefill(prompt, cache)
    log(f"prefill 512: gpu {tok} ({lg!r}), oracle {want_tok} ({want_lg!r}) in {time.time() - t:.1f}s")
    assert tok == want_tok
    assert F32(lg).view(np.uint32) == F32(want_lg).view(np.uint32)
    check_kv(eng, 0, cache, 0, 512, "prefill 512")


@pytest.fixture(scope="module")
def generation_128_256(full):
    _, arrays, orc = full
    prompt = np.random.default_rng(4).integers(0, FULL["vocab"], 128).astype(np.int32)
    t = time.time()
    cache = arrays.new_cache()
    want = orc.generate_layer_major(prompt, 256, cache=cache)
    log(f"oracle 128 + 256 generation in {time.time() - t:.1f}s")
    return prompt, want, cache


def test_generate_128_plus_256_22_layers(full, generation_128_256):
    """Batch-1 decode: the captured per-layer kernels replayed as a HIP graph
    give every token id and K/V row of the oracle's generation."""
    eng, _, _ = full
    prompt, want, cache = generation_128_256
    got, stop = eng.generate(prompt, 256, seq=0)
    assert stop == "max_tokens"
    assert_bits_equal(got, want, "token ids")
    check_kv(eng, 0, cache, 0, 128 + 255, "generation")


def _abort_after(flag, delay_s, stamp):
    import threading

    def run():
        time.sleep(delay_s)
        flag.value = 1
        stamp.append(time.perf_counter())

    t = threading.Thread(target=run)
    t.start()
    return t


def test_host_abort_stops_decode_within_steps(full, generation_128_256):
    """A host abort raised during batch-1 decode (stop_condition_unit.sv:18-37,
    HOST_ABORT outranks EOS): the decode stops with reason host_abort, the
    tokens it did record are the oracle's greedy ids, and it returns within a
    few steps of the flag (each 22-layer step is about 0.5 ms; the abort word
    is read by every step's token bookkeeping and the host keeps at most three
    steps in flight).  The same sequence then decodes on from where it
    stopped, so no abort is left behind."""
    import ctypes
    eng, _, orc = full
    prompt, want, _ = generation_128_256
    eng.prefill(prompt, seq=1)
    flag = ctypes.c_int32(0)
    stamp = []
    th = _abort_after(flag, 0.04, stamp)
    got, stop = eng.decode(1500, seq=1, abort_flag=flag)
    t_ret = time.perf_counter()
    th.join()
    latency_ms = (t_ret - stamp[0]) * 1e3
    log(f"abort after {got.size} decode steps; returned {latency_ms:.2f} ms after the flag")
    assert stop == "host_abort"
    assert 0 < got.size < 1500
    assert_bits_equal(got[:min(got.size, 255)], want[1:1 + min(got.size, 255)], "ids before the abort")
    assert latency_ms < 4.0
    more, stop2 = eng.decode(3, seq=1)
    assert stop2 == "max_tokens" and more.size == 3


def test_host_abort_stops_prefill_between_layers(full):
    """tl_generate with an abort flag launches the prefill one layer at a time
    and reads the flag between layers: an abort raised during a 2000-token
    prefill (about 0.4 ms per layer) returns host_abort with no token within
    about a layer, and the handle then generates normally."""
    import ctypes
    eng, _, orc = full
    prompt = np.random.default_rng(8).integers(0, FULL["vocab"], 2000).astype(np.int32)
    flag = ctypes.c_int32(0)
    stamp = []
    th = _abort_after(flag, 0.003, stamp)
    got, stop = eng.generate(prompt, 8, seq=2, abort_flag=flag)
    t_ret = time.perf_counter()
    th.join()
    latency_ms = (t_ret - stamp[0]) * 1e3 if stamp else 0.0
    log(f"prefill abort: {stop}, returned {latency_ms:.2f} ms after the flag")
    assert stop == "host_abort" and got.size == 0
    assert latency_ms < 2.0
    short = prompt[:16]
    got2, stop2 = eng.generate(short, 4, seq=2, abort_flag=ctypes.c_int32(0))
    want2, _ = orc.generate(short, 4)
    assert stop2 == "max_tokens"
    assert_bits_equal(got2, want2, "ids after the aborted prefill")


def test_decode_batch_32x2048_22_layers(full):
    """32 sequences, each with 1984 seeded INT8 cache rows at the model's
    per-layer / per-KV-head scales, 64 greedy steps at M = 32 (the batched
    decode kernels: packed-weight MFMA GEMMs, grouped attention over 2048 keys)."""
    eng, arrays, orc = full
    B, T0, steps = 32, 1984, 64
    rng = np.random.default_rng(5)
    t = time.time()
    caches = []
    for b in range(B):
        kc, vc = arrays.new_cache()
        kc[:, :, :T0] = rng.integers(-127, 128, kc[:, :, :T0].shape, dtype=np.int8)
        vc[:, :, :T0] = rng.integers(-127, 128, vc[:, :, :T0].shape, dtype=np.int8)
        for layer in range(FULL["n_layers"]):
            for g in range(FULL["n_kv_heads"]):
                eng.kv_write(b, layer, g, 0, kc[layer, g, :T0], vc[layer, g, :T0])
        caches.append((kc, vc))
    log(f"seeded {B} caches of {T0} rows in {time.time() - t:.1f}s")
    toks = rng.integers(0, FULL["vocab"], B).astype(np.int32)
    got = eng.decode_batch(toks, np.full(B, T0, np.int32), steps)
    t = time.time()
    x = np.stack([orc.embed(int(v)) for v in toks]).astype(F32)
    for s in range(steps):
        pos = np.full(B, T0 + s, np.int32)
        for layer in range(FULL["n_layers"]):
            orc.decode_rows(layer, pos, x, caches)
        want, _ = orc.lm_head_rows(x)
        assert_bits_equal(got[:, s], want, f"ids of step {s}")
        x = np.stack([orc.embed(int(v)) for v in want]).astype(F32)
        if s % 16 == 15:
            log(f"oracle batched step {s + 1}/{steps} at {time.time() - t:.1f}s")
    for b in range(B):
        check_kv(eng, b, caches[b], T0, steps, f"sequence {b}")
