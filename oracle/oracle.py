"""ctypes front end of the CPU oracle (TEST INFRASTRUCTURE ONLY).

The oracle (tl_oracle.c) restates the reference's INT8 decoder path in C; this
module loads oracle/_build/libtl_oracle.so and exposes it to the tests, to
``__graft_entry__.smoke()`` and to the ``cpu_baseline`` leg of ``bench.py``.
Nothing in the product package imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass, field

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libtl_oracle.so")

_i8p = C.POINTER(C.c_int8)
_i32p = C.POINTER(C.c_int32)
_f32p = C.POINTER(C.c_float)
_f64p = C.POINTER(C.c_double)


class OrConfig(C.Structure):
    _fields_ = [
        ("hidden", C.c_int32), ("intermediate", C.c_int32), ("n_layers", C.c_int32),
        ("n_heads", C.c_int32), ("n_kv_heads", C.c_int32), ("head_dim", C.c_int32),
        ("vocab", C.c_int32), ("max_pos", C.c_int32), ("rms_eps", C.c_float),
        ("rope_theta", C.c_float),
    ]


class OrLayer(C.Structure):
    _fields_ = [("w", _i8p * 7), ("s", _f32p * 7), ("g_in", _f32p), ("g_post", _f32p)]


class OrModel(C.Structure):
    _fields_ = [
        ("cfg", OrConfig), ("layers", C.POINTER(OrLayer)), ("lm_w", _i8p), ("lm_s", _f32p),
        ("g_final", _f32p), ("emb", _i8p), ("emb_s", _f32p), ("rope_cos", _f32p),
        ("rope_sin", _f32p), ("kv_sk", _f32p), ("kv_sv", _f32p),
    ]


class OrTrace(C.Structure):
    _fields_ = [
        ("attn_in", _f32p), ("attn_in_q", _i8p), ("attn_in_s", _f64p), ("qkv_acc", _i32p),
        ("qkv", _f32p), ("q_rot", _f32p), ("k_rot", _f32p), ("q8", _i8p), ("q_s", _f64p),
        ("scores", _i32p), ("probs", _i8p), ("pv_acc", _i32p), ("attended", _f32p),
        ("x_after_attn", _f32p), ("hidden", _f32p), ("out", _f32p),
    ]


def build(quiet: bool = True) -> str:
    """Compile the oracle with its Makefile (gcc only)."""
    subprocess.run(["make", "-C", HERE], check=True,
                   stdout=subprocess.DEVNULL if quiet else None)
    return LIB_PATH


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        sig = {
            "or_pairwise_sum": (C.c_float, [_f32p, C.c_int64]),
            "or_rms_norm": (None, [_f32p, _f32p, C.c_int32, C.c_float, _f32p]),
            "or_quantize_int8": (C.c_double, [_f32p, C.c_int64, _i8p]),
            "or_quantize_rows": (None, [_f32p, C.c_int32, C.c_int32, _i8p, _f64p]),
            "or_quantize_weight_rows": (None, [_f32p, C.c_int32, C.c_int32, _i8p, _f32p]),
            "or_quantize_static": (None, [_f32p, C.c_int64, C.c_float, _i8p]),
            "or_dequant_mult": (C.c_float, [C.c_double, C.c_double]),
            "or_gemm_i8": (None, [_i8p, _i8p, C.c_int32, C.c_int32, C.c_int32, _i32p]),
            "or_requant_f32": (None, [_i32p, _f32p, C.c_int32, _i8p]),
            "or_requant_q16": (C.c_int8, [C.c_int32, C.c_uint32, C.c_int32]),
            "or_rotate_q16": (C.c_int8, [C.c_int8, C.c_int8, C.c_int32, C.c_int32, C.c_int32]),
            "or_expf": (C.c_float, [C.c_float]),
            "or_silu": (C.c_float, [C.c_float]),
            "or_block_sum64": (C.c_float, [_f32p]),
            "or_softmax_row": (None, [_f32p, C.c_int32, _f32p]),
            "or_quantize_probs": (None, [_f32p, C.c_int32, _i8p]),
            "or_apply_rope": (None, [_f32p, C.c_int32, C.c_int32, _f32p, _f32p]),
            "or_argmax_first": (C.c_int32, [_f32p, C.c_int32]),
            "or_argmax_i32_tiles": (C.c_int32, [_i32p, C.c_int32, C.c_int32, _i32p]),
            "or_causal_mask_tile": (None, [_i32p, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                           C.c_int32, _i32p]),
            "or_attention_row": (None, [C.POINTER(OrConfig), C.c_int32, C.c_int32, _i8p, C.c_double,
                                        _i8p, _i8p, _f32p, _f32p, _f32p, _i32p, _i8p, _i32p]),
            "or_embed": (None, [C.POINTER(OrModel), C.c_int32, _f32p]),
            "or_decode_row": (None, [C.POINTER(OrModel), C.c_int32, C.c_int32, _f32p, _i8p, _i8p,
                                     C.POINTER(OrTrace)]),
            "or_lm_head_argmax": (C.c_int32, [C.POINTER(OrModel), _f32p, _f32p, _f32p]),
            "or_forward_token": (C.c_int32, [C.POINTER(OrModel), C.c_int32, C.c_int32, C.c_int32,
                                             _i8p, _i8p, _f32p]),
            "or_generate": (C.c_int32, [C.POINTER(OrModel), _i32p, C.c_int32, C.c_int32, C.c_int32,
                                        C.c_int32, _i8p, _i8p, _i32p, _f32p]),
            "or_decode_rows": (None, [C.POINTER(OrModel), C.c_int32, C.c_int32, _i32p, _f32p,
                                      C.POINTER(_i8p), C.POINTER(_i8p)]),
            "or_lm_head_rows": (None, [C.POINTER(OrModel), C.c_int32, _f32p, _i32p, _f32p]),
            "or_set_threads": (None, [C.c_int32]),
            "or_get_threads": (C.c_int32, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def ptr(a: np.ndarray | None, ctype):
    if a is None:
        return C.cast(None, C.POINTER(ctype))
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(C.POINTER(ctype))


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def i8(a):
    return np.ascontiguousarray(a, dtype=np.int8)


# ---- primitive wrappers -----------------------------------------------------

def rms_norm(x, w, eps):
    x = f32(x)
    w = f32(w)
    out = np.empty_like(x)
    rows = x.reshape(-1, x.shape[-1])
    o = out.reshape(-1, x.shape[-1])
    for r in range(rows.shape[0]):
        xr = np.ascontiguousarray(rows[r])
        orow = np.empty_like(xr)
        lib().or_rms_norm(ptr(xr, C.c_float), ptr(w, C.c_float), xr.size, eps, ptr(orow, C.c_float))
        o[r] = orow
    return out


def quantize_int8(x):
    x = f32(x)
    q = np.empty(x.shape, np.int8)
    s = lib().or_quantize_int8(ptr(x, C.c_float), x.size, ptr(q, C.c_int8))
    return q, s


def quantize_rows(x):
    x = f32(x)
    rows, cols = x.shape
    q = np.empty(x.shape, np.int8)
    s = np.empty(rows, np.float64)
    lib().or_quantize_rows(ptr(x, C.c_float), rows, cols, ptr(q, C.c_int8), ptr(s, C.c_double))
    return q, s


def quantize_weight_rows(w):
    w = f32(w)
    rows, cols = w.shape
    q = np.empty(w.shape, np.int8)
    s = np.empty(rows, np.float32)
    lib().or_quantize_weight_rows(ptr(w, C.c_float), rows, cols, ptr(q, C.c_int8), ptr(s, C.c_float))
    return q, s


def quantize_static(x, scale):
    x = f32(x)
    q = np.empty(x.shape, np.int8)
    lib().or_quantize_static(ptr(x, C.c_float), x.size, float(scale), ptr(q, C.c_int8))
    return q


def gemm_i8(a, w):
    a = i8(a)
    w = i8(w)
    m, k = a.shape
    n = w.shape[0]
    assert w.shape[1] == k
    c = np.empty((m, n), np.int32)
    lib().or_gemm_i8(ptr(a, C.c_int8), ptr(w, C.c_int8), m, n, k, ptr(c, C.c_int32))
    return c


def requant_f32(acc, mult):
    acc = np.ascontiguousarray(acc, np.int32)
    mult = f32(mult)
    y = np.empty(acc.shape, np.int8)
    lib().or_requant_f32(ptr(acc, C.c_int32), ptr(mult, C.c_float), acc.size, ptr(y, C.c_int8))
    return y


def softmax_row(s):
    s = f32(s)
    p = np.empty_like(s)
    lib().or_softmax_row(ptr(s, C.c_float), s.size, ptr(p, C.c_float))
    return p


def quantize_probs(p):
    p = f32(p)
    q = np.empty(p.shape, np.int8)
    lib().or_quantize_probs(ptr(p, C.c_float), p.size, ptr(q, C.c_int8))
    return q


def apply_rope(v, n_heads, hd, cos_p, sin_p):
    v = f32(v).copy()
    lib().or_apply_rope(ptr(v, C.c_float), n_heads, hd, ptr(f32(cos_p), C.c_float), ptr(f32(sin_p), C.c_float))
    return v


def attention_row(cfg: dict, layer, pos, q8, q_scale, kc, vc, sk, sv):
    """or_attention_row: GQA attention of one INT8 query row (all heads, at
    position pos, keys 0..pos of the logical cache kc / vc) -> float32 [D]."""
    c = OrConfig(cfg["hidden"], cfg["intermediate"], cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"],
                 cfg["head_dim"], cfg["vocab"], cfg["max_pos"], cfg["rms_eps"], cfg["rope_theta"])
    att = np.empty(cfg["n_heads"] * cfg["head_dim"], np.float32)
    lib().or_attention_row(C.byref(c), layer, pos, ptr(i8(q8), C.c_int8), float(q_scale),
                           ptr(kc, C.c_int8), ptr(vc, C.c_int8), ptr(f32(sk), C.c_float), ptr(f32(sv), C.c_float),
                           ptr(att, C.c_float), None, None, None)
    return att


def expf(x):
    return np.array([lib().or_expf(float(v)) for v in np.asarray(x, np.float32).ravel()],
                    np.float32).reshape(np.shape(x))


def silu(x):
    return np.array([lib().or_silu(float(v)) for v in np.asarray(x, np.float32).ravel()],
                    np.float32).reshape(np.shape(x))


# ---- model ------------------------------------------------------------------

def rope_table(max_pos, hd, theta):
    """TL:59-66 build_rope_cache restated with the same float32 NumPy steps."""
    inv_freq = 1.0 / (theta ** (np.arange(0, hd, 2, dtype=np.float32) / hd))
    ang = np.outer(np.arange(max_pos, dtype=np.float32), inv_freq)
    ang = np.concatenate([ang, ang], axis=-1)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)



@dataclass
class ModelArrays:
    """Host arrays of a quantized model, laid out the way the oracle reads them."""

    cfg: dict
    layers: list            # per layer: dict(w=[7 int8 [N][K]], s=[7 f32 [N]], g_in, g_post)
    lm_w: np.ndarray
    lm_s: np.ndarray
    g_final: np.ndarray
    emb: np.ndarray
    emb_s: np.ndarray
    rope_cos: np.ndarray
    rope_sin: np.ndarray
    kv_sk: np.ndarray
    kv_sv: np.ndarray
    _keep: list = field(default_factory=list)

    def c_config(self) -> OrConfig:
        c = self.cfg
        return OrConfig(c["hidden"], c["intermediate"], c["n_layers"], c["n_heads"],
                        c["n_kv_heads"], c["head_dim"], c["vocab"], c["max_pos"],
                        c["rms_eps"], c["rope_theta"])

    def c_model(self) -> OrModel:
        n = len(self.layers)
        arr = (OrLayer * n)()
        for i, L in enumerate(self.layers):
            for j in range(7):
                arr[i].w[j] = ptr(L["w"][j], C.c_int8)
                arr[i].s[j] = ptr(L["s"][j], C.c_float)
            arr[i].g_in = ptr(L["g_in"], C.c_float)
            arr[i].g_post = ptr(L["g_post"], C.c_float)
        self._keep = [arr]
        return OrModel(self.c_config(), C.cast(arr, C.POINTER(OrLayer)), ptr(self.lm_w, C.c_int8),
                       ptr(self.lm_s, C.c_float), ptr(self.g_final, C.c_float), ptr(self.emb, C.c_int8),
                       ptr(self.emb_s, C.c_float), ptr(self.rope_cos, C.c_float),
                       ptr(self.rope_sin, C.c_float), ptr(self.kv_sk, C.c_float), ptr(self.kv_sv, C.c_float))

    def new_cache(self):
        c = self.cfg
        shape = (c["n_layers"], c["n_kv_heads"], c["max_pos"], c["head_dim"])
        return np.zeros(shape, np.int8), np.zeros(shape, np.int8)


class Oracle:
    """Stateful convenience wrapper around one model."""

    def __init__(self, arrays: ModelArrays):
        self.a = arrays
        self.cm = arrays.c_model()

    def decode_row(self, layer, pos, x, kc, vc, trace: dict | None = None):
        x = f32(x).copy()
        tr = None
        if trace is not None:
            tr = OrTrace()
            for name, (ct, _) in _TRACE_TYPES.items():
                if name in trace:
                    setattr(tr, name, ptr(trace[name], ct))
        lib().or_decode_row(C.byref(self.cm), layer, pos, ptr(x, C.c_float), ptr(kc, C.c_int8),
                            ptr(vc, C.c_int8), C.byref(tr) if tr is not None else None)
        return x

    def decode_rows(self, layer, pos, x, caches):
        """or_decode_rows: rows x[r] (updated in place, float32 [rows][D]) at
        positions pos[r] of the sequences whose (K, V) caches are caches[r]."""
        pos = np.ascontiguousarray(pos, np.int32)
        assert x.dtype == np.float32 and x.flags["C_CONTIGUOUS"] and x.shape[0] == pos.size == len(caches)
        kp = (_i8p * pos.size)(*[ptr(k, C.c_int8) for k, _ in caches])
        vp = (_i8p * pos.size)(*[ptr(v, C.c_int8) for _, v in caches])
        lib().or_decode_rows(C.byref(self.cm), layer, pos.size, ptr(pos, C.c_int32), ptr(x, C.c_float), kp, vp)
        return x

    def lm_head_rows(self, x):
        """or_lm_head_rows: greedy token and its logit for every row of x."""
        x = f32(x)
        rows = x.shape[0]
        tok = np.empty(rows, np.int32)
        lg = np.empty(rows, np.float32)
        lib().or_lm_head_rows(C.byref(self.cm), rows, ptr(x, C.c_float), ptr(tok, C.c_int32), ptr(lg, C.c_float))
        return tok, lg

    def prefill(self, prompt, cache):
        """Every prompt row through every layer (layer-major), then the LM head
        of the last row: (next token, its logit); the prompt's K/V rows land
        in cache."""
        prompt = np.ascontiguousarray(prompt, np.int32)
        x = np.stack([self.embed(int(t)) for t in prompt]).astype(np.float32)
        pos = np.arange(prompt.size, dtype=np.int32)
        caches = [cache] * prompt.size
        for layer in range(self.a.cfg["n_layers"]):
            self.decode_rows(layer, pos, x, caches)
        tok, lg = self.lm_head_rows(x[-1:])
        return int(tok[0]), float(lg[0])

    def generate_layer_major(self, prompt, max_new, cache=None):
        """Greedy generation whose prompt runs layer-major (prefill) and whose
        new tokens run one row at a time: the same ids and cache rows as
        generate(), faster for long prompts."""
        kc, vc = cache if cache is not None else self.a.new_cache()
        tok, _ = self.prefill(prompt, (kc, vc))
        out = [tok]
        pos = len(prompt)
        while len(out) < max_new:
            x = self.embed(out[-1])[None, :].copy()
            for layer in range(self.a.cfg["n_layers"]):
                self.decode_rows(layer, [pos], x, [(kc, vc)])
            t, _ = self.lm_head_rows(x)
            out.append(int(t[0]))
            pos += 1
        return np.array(out, np.int32)

    def embed(self, tok):
        x = np.empty(self.a.cfg["hidden"], np.float32)
        lib().or_embed(C.byref(self.cm), int(tok), ptr(x, C.c_float))
        return x

    def lm_head(self, x, want_logits=False):
        x = f32(x)
        logits = np.empty(self.a.cfg["vocab"], np.float32) if want_logits else None
        best = C.c_float()
        tok = lib().or_lm_head_argmax(C.byref(self.cm), ptr(x, C.c_float), ptr(logits, C.c_float),
                                      C.byref(best))
        return (tok, best.value, logits) if want_logits else (tok, best.value)

    def generate(self, prompt, max_new, n_layers=None, eos=-1, cache=None):
        prompt = np.ascontiguousarray(prompt, np.int32)
        kc, vc = cache if cache is not None else self.a.new_cache()
        out = np.empty(max_new, np.int32)
        lg = np.empty(max_new, np.float32)
        n = lib().or_generate(C.byref(self.cm), ptr(prompt, C.c_int32), prompt.size, max_new,
                              self.a.cfg["n_layers"] if n_layers is None else n_layers, eos,
                              ptr(kc, C.c_int8), ptr(vc, C.c_int8), ptr(out, C.c_int32), ptr(lg, C.c_float))
        if n < 0:
            raise ValueError("bad generate arguments")
        return out[:n], lg[:n]


_TRACE_TYPES = {
    "attn_in": (C.c_float, None), "attn_in_q": (C.c_int8, None), "attn_in_s": (C.c_double, None),
    "qkv_acc": (C.c_int32, None), "qkv": (C.c_float, None), "q_rot": (C.c_float, None),
    "k_rot": (C.c_float, None), "q8": (C.c_int8, None), "q_s": (C.c_double, None),
    "scores": (C.c_int32, None), "probs": (C.c_int8, None), "pv_acc": (C.c_int32, None),
    "attended": (C.c_float, None), "x_after_attn": (C.c_float, None), "hidden": (C.c_float, None),
    "out": (C.c_float, None),
}


def synthetic_model(cfg: dict, seed: int, kv_range=(0.02, 0.06)) -> ModelArrays:
    """Seeded random model of any geometry: weights N(0, 0.02) quantized per
    output channel (or_quantize_weight_rows), RMSNorm gains N(1, 0.02),
    embedding N(0, 0.02) quantized per row, static KV scales uniform in
    kv_range."""
    rng = np.random.default_rng(seed)
    D, F, L, Hkv, hd, V = (cfg[k] for k in ("hidden", "intermediate", "n_layers", "n_kv_heads",
                                            "head_dim", "vocab"))
    kvd = Hkv * hd
    shapes = [(D, D), (kvd, D), (kvd, D), (D, D), (F, D), (F, D), (D, F)]
    sd = np.float32(0.02)
    layers = []
    for _ in range(L):
        w, s = [], []
        for shp in shapes:
            q, sc = quantize_weight_rows(rng.standard_normal(shp, dtype=np.float32) * sd)
            w.append(q)
            s.append(sc)
        layers.append(dict(w=w, s=s,
                           g_in=(1.0 + 0.02 * rng.standard_normal(D)).astype(np.float32),
                           g_post=(1.0 + 0.02 * rng.standard_normal(D)).astype(np.float32)))
    lm_w, lm_s = quantize_weight_rows(rng.standard_normal((V, D), dtype=np.float32) * sd)
    emb, emb_s = quantize_weight_rows(rng.standard_normal((V, D), dtype=np.float32) * sd)
    cos, sin = rope_table(cfg["max_pos"], hd, cfg["rope_theta"])
    sk = rng.uniform(*kv_range, (L, Hkv)).astype(np.float32)
    sv = rng.uniform(*kv_range, (L, Hkv)).astype(np.float32)
    return ModelArrays(cfg=dict(cfg), layers=layers, lm_w=lm_w, lm_s=lm_s,
                       g_final=(1.0 + 0.02 * rng.standard_normal(D)).astype(np.float32),
                       emb=emb, emb_s=emb_s, rope_cos=cos, rope_sin=sin, kv_sk=sk, kv_sv=sv)


SMALL_CFG = dict(hidden=512, intermediate=1408, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=64,
                 vocab=2048, max_pos=256, rms_eps=np.float32(1e-5), rope_theta=10000.0)

TINYLLAMA_CFG = dict(hidden=2048, intermediate=5632, n_layers=22, n_heads=32, n_kv_heads=4, head_dim=64,
                     vocab=32000, max_pos=2048, rms_eps=np.float32(1e-5), rope_theta=10000.0)
