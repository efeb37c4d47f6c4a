"""Operator-level parity: each HIP operator through the C-ABI against the CPU
oracle on the same seeded inputs.  Integer and float results must be
bit-identical (the kernels and the oracle follow the same operation order)."""
import numpy as np
import pytest

import oracle
from gpu_util import OPS_CFG, assert_bits_equal, dev, empty, host, runtime

pytestmark = pytest.mark.gpu
F32 = np.float32


@pytest.fixture(scope="module")
def rt():
    r = runtime()
    yield r
    r.close()


# ---- decode GEMV + requantize (the Q-projection operator, 2048 x 2048) ----------

@pytest.mark.parametrize("mlo,mhi", [(1e-3, 1e-2), (1e-5, 1e-4)])
def test_gemv_requant_q_projection(rt, mlo, mhi):
    rng = np.random.default_rng(1)
    x = rng.integers(-127, 128, 2048).astype(np.int8)
    w = rng.integers(-127, 128, (2048, 2048)).astype(np.int8)
    m = rng.uniform(mlo, mhi, 2048).astype(F32)
    y, acc = empty(2048, np.int8), empty(2048, np.int32)
    rt.call("tl_gemv_i8_requant", dev(x), dev(w), dev(m), 2048, 2048, y, acc)
    want_acc = oracle.gemm_i8(x[None, :], w)[0]
    assert_bits_equal(host(acc), want_acc, "acc")
    assert_bits_equal(host(y), oracle.requant_f32(want_acc, m), "y8")


@pytest.mark.parametrize("n,k", [(1, 16), (37, 5632), (5, 1040), (4099, 2048), (300, 6144), (8, 3072)])
def test_gemv_shapes(rt, n, k):
    rng = np.random.default_rng(n * 7 + k)
    x = rng.integers(-128, 128, k).astype(np.int8)
    w = rng.integers(-128, 128, (n, k)).astype(np.int8)
    m = rng.uniform(1e-5, 1e-3, n).astype(F32)
    y, acc = empty(n, np.int8), empty(n, np.int32)
    rt.call("tl_gemv_i8_requant", dev(x), dev(w), dev(m), n, k, y, acc)
    want = (x.astype(np.int64)[None, :] @ w.astype(np.int64).T)[0].astype(np.int32)
    assert_bits_equal(host(acc), want, "acc")
    assert_bits_equal(host(y), oracle.requant_f32(want, m), "y8")


def test_gemv_rejects_bad_k(rt):
    from lpta import TlValueError
    with pytest.raises(TlValueError):
        rt.call("tl_gemv_i8_requant", dev(np.zeros(24, np.int8)), dev(np.zeros((4, 24), np.int8)),
                dev(np.ones(4, F32)), 4, 24, empty(4, np.int8), None)


# ---- MFMA GEMM ---------------------------------------------------------------------

@pytest.mark.parametrize("m,n,k", [(2, 64, 64), (5, 128, 2048), (32, 2048, 2048), (20, 160, 5632), (33, 256, 5632),
                                   (64, 192, 128), (130, 320, 1024), (512, 2560, 2048), (7, 32000, 64)])
def test_gemm_i8_exact(rt, m, n, k):
    rng = np.random.default_rng(m * 1000 + n + k)
    a = rng.integers(-128, 128, (m, k)).astype(np.int8)
    w = rng.integers(-128, 128, (n, k)).astype(np.int8)
    c = empty((m, n), np.int32)
    rt.call("tl_gemm_i8", dev(a), dev(w), m, n, k, c)
    want = (a.astype(np.int64) @ w.astype(np.int64).T).astype(np.int32)
    assert_bits_equal(host(c), want, "gemm")


@pytest.mark.parametrize("m", [1, 3, 32, 200])
def test_gemm_dequant_residual(rt, m):
    n, k = 2048, 2048
    rng = np.random.default_rng(m)
    a = rng.integers(-127, 128, (m, k)).astype(np.int8)
    w = rng.integers(-127, 128, (n, k)).astype(np.int8)
    sa = rng.uniform(1e-3, 1e-1, m)
    sw = rng.uniform(1e-4, 1e-3, n).astype(F32)
    res = rng.standard_normal((m, n)).astype(F32)
    y = empty((m, n), np.float32)
    rt.call("tl_gemm_i8_dequant", dev(a), dev(sa), dev(w), dev(sw), m, n, k, dev(res), y)
    acc = oracle.gemm_i8(a, w)
    mult = np.array([[oracle.lib().or_dequant_mult(float(sa[i]), float(sw[j])) for j in range(n)]
                     for i in range(m)], F32)
    assert_bits_equal(host(y), res + acc.astype(F32) * mult, "dequant+residual")


# ---- RMSNorm / quantize / softmax / SiLU / RoPE ---------------------------------------

@pytest.mark.parametrize("n,rows", [(2048, 5), (512, 3), (256, 1), (5632, 2)])
def test_rmsnorm_quant(rt, n, rows):
    rng = np.random.default_rng(n + rows)
    x = (rng.standard_normal((rows, n)) * rng.uniform(0.1, 20, (rows, 1))).astype(F32)
    g = (1 + 0.1 * rng.standard_normal(n)).astype(F32)
    y, q, s = empty((rows, n), np.float32), empty((rows, n), np.int8), empty(rows, np.float64)
    rt.call("tl_rmsnorm_quant", dev(x), dev(g), rows, n, y, q, s)
    want_y = oracle.rms_norm(x, g, F32(1e-5))
    want_q, want_s = oracle.quantize_rows(want_y)
    assert_bits_equal(host(y), want_y, "rmsnorm")
    assert_bits_equal(host(q), want_q, "q")
    assert_bits_equal(host(s), want_s, "scale")
    # without the float output: the one-workgroup-per-row vectorized kernel
    q2, s2 = empty((rows, n), np.int8), empty(rows, np.float64)
    rt.call("tl_rmsnorm_quant", dev(x), dev(g), rows, n, None, q2, s2)
    assert_bits_equal(host(q2), want_q, "q (no float output)")
    assert_bits_equal(host(s2), want_s, "scale (no float output)")


@pytest.mark.parametrize("gain", [1e-30, 2.0 ** -58, 1e30], ids=["tiny", "near_2^-64", "huge"])
def test_rmsnorm_quant_extreme_scales(rt, gain):
    """Row scales below 2^-64 and above 2^64 take the quantizer's correctly
    rounded division; scales just above 2^-64 the reciprocal-and-corrections
    path.  Both equal the oracle bit for bit (2048-wide rows: the fused
    row prologue)."""
    n, rows = 2048, 4
    rng = np.random.default_rng(31)
    x = (rng.standard_normal((rows, n)) * rng.uniform(0.5, 4, (rows, 1))).astype(F32)
    g = ((1 + 0.1 * rng.standard_normal(n)) * gain).astype(F32)
    want_q, want_s = oracle.quantize_rows(oracle.rms_norm(x, g, F32(1e-5)))
    q, s = empty((rows, n), np.int8), empty(rows, np.float64)
    rt.call("tl_rmsnorm_quant", dev(x), dev(g), rows, n, None, q, s)
    assert_bits_equal(host(q), want_q, "q")
    assert_bits_equal(host(s), want_s, "scale")
    f32_scale = want_s.astype(np.float32)
    assert ((f32_scale < 2.0 ** -64) | (f32_scale > 2.0 ** 64)).all() == (gain != 2.0 ** -58)


def test_quantize_rows_and_tensor(rt):
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((4, 5632)) * 3).astype(F32)
    x[2] = 0.0
    q, s = empty((4, 5632), np.int8), empty(4, np.float64)
    rt.call("tl_quantize_rows", dev(x), 4, 5632, q, s)
    want_q, want_s = oracle.quantize_rows(x)
    assert_bits_equal(host(q), want_q, "rows q")
    assert_bits_equal(host(s), want_s, "rows s")
    # a width that is not a multiple of 64 takes the general row kernel
    xo = np.ascontiguousarray(x[:, :1000])
    qo, so = empty((4, 1000), np.int8), empty(4, np.float64)
    rt.call("tl_quantize_rows", dev(xo), 4, 1000, qo, so)
    want_qo, want_so = oracle.quantize_rows(xo)
    assert_bits_equal(host(qo), want_qo, "rows q (n = 1000)")
    assert_bits_equal(host(so), want_so, "rows s (n = 1000)")
    qt, st = empty((4, 5632), np.int8), empty(1, np.float64)
    rt.call("tl_quantize_tensor", dev(x), x.size, qt, st)
    wq, ws = oracle.quantize_int8(x)
    assert_bits_equal(host(qt), wq, "tensor q")
    assert host(st)[0] == ws


def near_half_integer_rows(rows, n, seed):
    """Rows whose quotients x / s sit on and within a few ulps of
    half-integers k + 1/2 (the rounding boundaries of the quantizers), with
    the row maximum fixing s = f32(max / 127)."""
    rng = np.random.default_rng(seed)
    out = np.empty((rows, n), F32)
    for r in range(rows):
        mx = F32(rng.uniform(0.05, 40.0))
        sf = F32(np.float64(mx) / 127.0)
        k = rng.integers(-127, 127, n).astype(np.float64)
        v = ((k + 0.5) * np.float64(sf)).astype(F32)
        ulps = rng.integers(-3, 4, n).astype(np.int32)
        v = (v.view(np.int32) + ulps).view(F32)
        v = np.clip(v, -mx, mx)
        v[0] = mx
        out[r] = v
    return out


@pytest.mark.parametrize("n", [2048, 5632, 1000])
def test_quantizers_at_rounding_boundaries(rt, n):
    """rint(RN(x / s)) exactly at and around every rounding boundary of the
    quantizers (row, tensor and RMSNorm-prologue paths)."""
    x = near_half_integer_rows(8, n, seed=n)
    q, s = empty((8, n), np.int8), empty(8, np.float64)
    rt.call("tl_quantize_rows", dev(x), 8, n, q, s)
    want_q, want_s = oracle.quantize_rows(x)
    assert_bits_equal(host(q), want_q, "rows q at half-integers")
    assert_bits_equal(host(s), want_s, "rows s")
    qt, st = empty((8, n), np.int8), empty(1, np.float64)
    rt.call("tl_quantize_tensor", dev(x), x.size, qt, st)
    wq, ws = oracle.quantize_int8(x)
    assert_bits_equal(host(qt), wq, "tensor q at half-integers")
    if n % 256 == 0:
        # the RMSNorm prologue with unit gains on rows already at unit RMS
        # keeps the quotients near the boundaries
        g = np.ones(n, F32)
        y, q2, s2 = empty((8, n), np.float32), empty((8, n), np.int8), empty(8, np.float64)
        rt.call("tl_rmsnorm_quant", dev(x), dev(g), 8, n, None, q2, s2)
        want_q2, want_s2 = oracle.quantize_rows(oracle.rms_norm(x, g, F32(1e-5)))
        assert_bits_equal(host(q2), want_q2, "rmsnorm prologue q")
        assert_bits_equal(host(s2), want_s2, "rmsnorm prologue s")


def test_quantize_weight_rows(rt):
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((300, 2048)) * 0.02).astype(F32)
    q, s = empty((300, 2048), np.int8), empty(300, np.float32)
    rt.call("tl_quantize_weight_rows", dev(w), 300, 2048, q, s)
    wq, ws = oracle.quantize_weight_rows(w)
    assert_bits_equal(host(q), wq, "q")
    assert_bits_equal(host(s), ws, "s")


@pytest.mark.parametrize("n", [1, 7, 64, 65, 513, 2048])
def test_softmax_rows(rt, n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((3, n)) * 6).astype(F32)
    p = empty((3, n), np.float32)
    rt.call("tl_softmax_rows", dev(x), 3, n, p)
    want = np.stack([oracle.softmax_row(x[r]) for r in range(3)])
    assert_bits_equal(host(p), want, "softmax")


def test_silu_and_glu(rt):
    rng = np.random.default_rng(3)
    g = np.concatenate([rng.standard_normal(5000) * 5, [-90, -60, -59.9, 0, 59.9, 60, 90]]).astype(F32)
    u = rng.standard_normal(g.size).astype(F32)
    y = empty(g.size, np.float32)
    rt.call("tl_silu_mul", dev(g), None, g.size, y)
    assert_bits_equal(host(y), oracle.silu(g), "silu")
    rt.call("tl_silu_mul", dev(g), dev(u), g.size, y)
    assert_bits_equal(host(y), oracle.silu(g) * u, "glu")


def test_rope_rows(rt):
    import lpta
    cos, sin = lpta.build_rope_cache(2048, 64, 10000.0)
    rt.call("tl_set_rope_table", cos, sin, 2048)
    rng = np.random.default_rng(8)
    pos = np.array([0, 1, 17, 511, 1024, 2047], np.int32)
    v = rng.standard_normal((pos.size, 32 * 64)).astype(F32)
    d = dev(v)
    rt.call("tl_rope", d, pos.size, 32, dev(pos))
    want = np.stack([oracle.apply_rope(v[i], 32, 64, cos[p], sin[p]) for i, p in enumerate(pos)])
    assert_bits_equal(host(d), want, "rope")
