"""The primitives of model/tinyllama.py (TL) on the MI355X path.

Same names, arguments and return types as the reference module: NumPy in,
NumPy out, with every per-element computation done by the HIP library.
- rms_norm and apply_rope are bit-exact to the reference;
- softmax and silu use the library's own exp and agree with the reference to
  about 1e-6 relative;
- build_rope_cache keeps the reference's float32 NumPy steps (the table is an
  input of the forward pass, not a per-token computation);
- causal_mask, repeat_kv and rotate_half are index operations.
TinyLlamaWeights / load_weights read the reference's .npz weight archive
(TL:198-267 key schema).

Device memory is torch CUDA tensors used as plain buffers.
"""
from __future__ import annotations

import numpy as np

from ._native import Runtime

# ---------------------------------------------------------------------------
# device plumbing: small operator handles and torch buffers
# ---------------------------------------------------------------------------
_OP_HANDLES: dict = {}


def round_pos(n: int) -> int:
    """Handle position counts are positive multiples of 64."""
    return max(64, -(-int(n) // 64) * 64)


def op_runtime(eps: float = 1e-5, max_pos: int = 64) -> Runtime:
    """A minimal handle for operator calls.  The library reads the RMSNorm
    epsilon from the handle's configuration and RoPE tables hold max_pos rows
    (rounded up to a multiple of 64), so handles are cached per (float32 eps,
    max_pos)."""
    key = (float(np.float32(eps)), round_pos(max_pos))
    rt = _OP_HANDLES.get(key)
    if rt is None:
        cfg = dict(hidden=64, intermediate=64, n_layers=1, n_heads=1, n_kv_heads=1, head_dim=64, vocab=64,
                   max_pos=key[1], rms_eps=np.float32(eps), rope_theta=10000.0)
        rt = Runtime(cfg)
        _OP_HANDLES[key] = rt
    return rt


def set_rope_rows(rt: Runtime, cos: np.ndarray, sin: np.ndarray, n: int) -> None:
    """Load rows 0..n-1 of a cos/sin table into rt's RoPE table (rows past n,
    up to the handle's size, are zero and never read)."""
    rows = rt.cfg["max_pos"]
    c = np.zeros((rows, 64), np.float32)
    s = np.zeros((rows, 64), np.float32)
    c[:n] = cos[:n]
    s[:n] = sin[:n]
    rt.call("tl_set_rope_table", c, s, rows)


def dev(a, dtype=None):
    """NumPy array -> torch CUDA tensor (a copy)."""
    import torch
    a = np.require(a if dtype is None else np.asarray(a, dtype=dtype), requirements=["C", "W"])
    return torch.from_numpy(a).cuda()


def empty(shape, dtype):
    import torch
    tdt = {np.float32: torch.float32, np.float64: torch.float64, np.int8: torch.int8,
           np.int32: torch.int32}[np.dtype(dtype).type]
    return torch.empty(tuple(int(s) for s in shape), dtype=tdt, device="cuda")


def host(t) -> np.ndarray:
    return t.detach().cpu().numpy()


# ---------------------------------------------------------------------------
# TL:45-50
# ---------------------------------------------------------------------------
def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """x * 1/sqrt(mean(x^2) + eps) * w over the last axis, in float32."""
    x_fp = np.asarray(x, dtype=np.float32)
    w_fp = np.asarray(w, dtype=np.float32)
    n = x_fp.shape[-1]
    rows = int(np.prod(x_fp.shape[:-1], dtype=np.int64))
    if rows == 0:
        return np.empty(x_fp.shape, np.float32)
    rt = op_runtime(eps)
    y = empty((rows, n), np.float32)
    q = empty((rows, n), np.int8)
    s = empty((rows,), np.float64)
    rt.call("tl_rmsnorm_quant", dev(x_fp.reshape(rows, n)), dev(np.broadcast_to(w_fp, (n,))), rows, n, y, q, s)
    return host(y).reshape(x_fp.shape)


# ---------------------------------------------------------------------------
# TL:59-80
# ---------------------------------------------------------------------------
def build_rope_cache(seq_len: int, head_dim: int, rope_theta: float) -> tuple[np.ndarray, np.ndarray]:
    """RoPE cos/sin tables [seq_len][head_dim] in float32 (TL:59-66).

    The table is an input of the reference's forward pass (GI:437 takes
    ``cos, sin``), so it is built with the same float32 NumPy steps: inverse
    frequencies theta ** -(2i/d), the outer product with the positions,
    duplicated across both halves of the head, then cos and sin.  The
    ``rope_{cos,sin}_rom.memh`` tables of the RTL are this table in Q16.16.
    """
    exponents = np.arange(0, head_dim, 2, dtype=np.float32) / head_dim
    inv_freq = 1.0 / (rope_theta ** exponents)
    angles = np.outer(np.arange(seq_len, dtype=np.float32), inv_freq)
    angles = np.concatenate([angles, angles], axis=-1)
    return np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)


def rotate_half(x: np.ndarray) -> np.ndarray:
    """TL:69-71: (x1, x2) -> (-x2, x1) over the last axis."""
    half = x.shape[-1] // 2
    return np.concatenate([-x[..., half:], x[..., :half]], axis=-1)


def _rope_heads(v: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """q or k [heads][seq][64] rotated at positions 0..seq-1 by the library."""
    heads, seq, hd = v.shape
    if hd != 64:
        raise ValueError("head_dim must be 64")
    if seq == 0:
        return np.empty(v.shape, np.float32)
    if cos.shape[0] < seq or sin.shape[0] < seq:
        raise ValueError("RoPE table shorter than the sequence")
    rt = op_runtime(max_pos=seq)
    set_rope_rows(rt, cos, sin, seq)
    rows = dev(np.ascontiguousarray(np.asarray(v, np.float32).transpose(1, 0, 2)).reshape(seq, heads * hd))
    rt.call("tl_rope", rows, seq, heads, dev(np.arange(seq, dtype=np.int32)))
    return host(rows).reshape(seq, heads, hd).transpose(1, 0, 2).copy()


def apply_rope(q: np.ndarray, k: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """TL:74-80: q [Hq][seq][hd], k [Hkv][seq][hd] rotated at positions 0..seq-1."""
    return _rope_heads(q, cos, sin), _rope_heads(k, cos, sin)


# ---------------------------------------------------------------------------
# TL:89-103
# ---------------------------------------------------------------------------
def causal_mask(seq_len: int) -> np.ndarray:
    return np.tril(np.ones((seq_len, seq_len), dtype=bool))


def repeat_kv(x: np.ndarray, n_rep: int) -> np.ndarray:
    """GQA index map: KV head h serves query heads h*n_rep .. h*n_rep+n_rep-1."""
    if n_rep == 1:
        return x
    return np.repeat(x, n_rep, axis=0)


def softmax(x: np.ndarray, axis: int = -1) -> np.ndarray:
    """Softmax over the last axis, in float32 on the library's kernel."""
    if axis not in (-1, np.ndim(x) - 1):
        raise ValueError("softmax runs over the last axis")
    x_fp = np.asarray(x, dtype=np.float32)
    n = x_fp.shape[-1]
    rows = int(np.prod(x_fp.shape[:-1], dtype=np.int64))
    if rows == 0 or n == 0:
        return np.empty(x_fp.shape, np.float32)
    p = empty((rows, n), np.float32)
    op_runtime().call("tl_softmax_rows", dev(x_fp.reshape(rows, n)), rows, n, p)
    return host(p).reshape(x_fp.shape)


# ---------------------------------------------------------------------------
# TL:159-161
# ---------------------------------------------------------------------------
def silu(x: np.ndarray) -> np.ndarray:
    """x / (1 + exp(-clip(x, -60, 60))) in float32."""
    x_fp = np.asarray(x, dtype=np.float32)
    if x_fp.size == 0:
        return np.empty(x_fp.shape, np.float32)
    y = empty((x_fp.size,), np.float32)
    op_runtime().call("tl_silu_mul", dev(x_fp.ravel()), None, x_fp.size, y)
    return host(y).reshape(x_fp.shape)


# ---------------------------------------------------------------------------
# TL:106-197, 391-408: the float32 model, the baseline the analysis report
# compares the INT8 path against (tl_linear_f32 / tl_attention_f32).  Sums
# run in the kernels' order, so results agree with the reference to float32
# rounding; the reference's scores and softmax are float64 (float32 scores
# times a float64 scale), here they stay float32.
# ---------------------------------------------------------------------------
def _float_runtime(cfg: dict) -> Runtime:
    return op_runtime(cfg["rms_norm_eps"], max_pos=cfg["max_position_embeddings"])


def _bias(b, n: int):
    return None if b is None else dev(np.broadcast_to(np.asarray(b, np.float32), (n,)))


def linear_dev(rt: Runtime, x, w: np.ndarray, b, rows: int, residual=None):
    """Device rows x [rows][K] @ w [K][N] (+ b) (+ residual) -> [rows][N]."""
    w_fp = np.asarray(w, np.float32)
    k, n = w_fp.shape
    y = empty((rows, n), np.float32)
    rt.call("tl_linear_f32", x, dev(w_fp), _bias(b, n), residual, rows, n, k, y)
    return y


def linear(x: np.ndarray, w: np.ndarray, b: np.ndarray | None = None) -> np.ndarray:
    """TL:106-110: x @ w (+ b) in float32, w [K][N]."""
    x_fp = np.asarray(x, dtype=np.float32)
    w_fp = np.asarray(w, dtype=np.float32)
    k, n = w_fp.shape
    rows = int(np.prod(x_fp.shape[:-1], dtype=np.int64))
    if rows == 0:
        return np.empty(x_fp.shape[:-1] + (n,), np.float32)
    y = linear_dev(op_runtime(), dev(x_fp.reshape(rows, k)), w_fp, b, rows)
    return host(y).reshape(x_fp.shape[:-1] + (n,))


def rms_norm_dev(rt: Runtime, x, w: np.ndarray, rows: int, n: int):
    """TL:45-50 on device rows (the handle's epsilon)."""
    y = empty((rows, n), np.float32)
    q = empty((rows, n), np.int8)
    s = empty((rows,), np.float64)
    rt.call("tl_rmsnorm_quant", x, dev(np.asarray(w, np.float32)), rows, n, y, q, s)
    return y


def self_attention_dev(rt: Runtime, x, layer: dict, cfg: dict, cos, sin, rows: int, capture: bool = False):
    """TL:122-156 on device rows x [rows][D]: (out, parts) where parts holds
    the Q/K/V projections and, when capture is set, the scores, weights and
    attended rows.  The attention output projection is not added to any
    residual here."""
    Hq, Hkv, hd = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"]
    if hd != 64:
        raise ValueError("head_dim must be 64")
    set_rope_rows(rt, cos, sin, rows)
    q = linear_dev(rt, x, layer["q_w"], layer.get("q_b"), rows)
    k = linear_dev(rt, x, layer["k_w"], layer.get("k_b"), rows)
    v = linear_dev(rt, x, layer["v_w"], layer.get("v_b"), rows)
    parts = {"q": q, "k": k, "v": v}
    qr, kr = q.clone(), k.clone()
    pos = dev(np.arange(rows, dtype=np.int32))
    rt.call("tl_rope", qr, rows, Hq, pos)
    rt.call("tl_rope", kr, rows, Hkv, pos)
    att = empty((rows, Hq * hd), np.float32)
    scores = empty((Hq, rows, rows), np.float32) if capture else None
    weights = empty((Hq, rows, rows), np.float32) if capture else None
    rt.call("tl_attention_f32", qr, kr, v, rows, Hq, Hkv, float(np.float32(cfg["attn_scale"])), att, scores, weights)
    parts.update(attended=att, scores=scores, weights=weights)
    return att, parts


def self_attention(x: np.ndarray, layer: dict, cfg: dict, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """TL:122-156: GQA self-attention of x [seq][D] at positions 0..seq-1."""
    rt = _float_runtime(cfg)
    x_fp = np.asarray(x, np.float32)
    rows = x_fp.shape[0]
    att, _ = self_attention_dev(rt, dev(x_fp), layer, cfg, cos, sin, rows)
    return host(linear_dev(rt, att, layer["o_w"], layer.get("o_b"), rows))


def feed_forward_dev(rt: Runtime, x, layer: dict, rows: int, residual=None):
    """TL:164-169 on device rows: (out, gate, up, hidden)."""
    gate = linear_dev(rt, x, layer["gate_w"], layer.get("gate_b"), rows)
    up = linear_dev(rt, x, layer["up_w"], layer.get("up_b"), rows)
    F = gate.shape[1]
    hid = empty((rows, F), np.float32)
    rt.call("tl_silu_mul", gate, up, rows * F, hid)
    out = linear_dev(rt, hid, layer["down_w"], layer.get("down_b"), rows, residual)
    return out, gate, up, hid


def feed_forward(x: np.ndarray, layer: dict) -> np.ndarray:
    """TL:164-169: down(silu(gate(x)) * up(x))."""
    x_fp = np.asarray(x, np.float32)
    rows = int(np.prod(x_fp.shape[:-1], dtype=np.int64))
    out, *_ = feed_forward_dev(op_runtime(), dev(x_fp.reshape(rows, -1)), layer, rows)
    return host(out).reshape(x_fp.shape[:-1] + (out.shape[1],))


def decoder_layer_dev(rt: Runtime, x, layer: dict, cfg: dict, cos, sin, rows: int):
    """TL:177-189 on device rows; the residual adds run in the O and down
    projections' epilogues (x + (a @ W + b), the reference's rounding)."""
    D = cfg["hidden_size"]
    a = rms_norm_dev(rt, x, layer["input_norm_w"], rows, D)
    att, _ = self_attention_dev(rt, a, layer, cfg, cos, sin, rows)
    x1 = linear_dev(rt, att, layer["o_w"], layer.get("o_b"), rows, residual=x)
    f = rms_norm_dev(rt, x1, layer["post_norm_w"], rows, D)
    out, *_ = feed_forward_dev(rt, f, layer, rows, residual=x1)
    return out


def decoder_layer(x: np.ndarray, layer: dict, cfg: dict, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """TL:177-189: pre-norm attention and feed-forward with residuals."""
    x_fp = np.asarray(x, np.float32)
    rt = _float_runtime(cfg)
    return host(decoder_layer_dev(rt, dev(x_fp), layer, cfg, cos, sin, x_fp.shape[0]))


def forward(token_ids: list[int], weights: "TinyLlamaWeights", cos: np.ndarray, sin: np.ndarray,
            layer_count: int | None = None) -> np.ndarray:
    """TL:391-408: logits [seq][V] of the float32 model (all layers unless
    layer_count is given)."""
    cfg = weights.cfg
    seq = len(token_ids)
    if seq > cfg["max_position_embeddings"]:
        raise ValueError(f"Sequence length {seq} exceeds max_position_embeddings={cfg['max_position_embeddings']}")
    rt = _float_runtime(cfg)
    x = dev(np.asarray(weights.embed(token_ids), np.float32))
    for i in range(cfg["num_hidden_layers"] if layer_count is None else layer_count):
        x = decoder_layer_dev(rt, x, weights.layer(i), cfg, cos, sin, seq)
    x = rms_norm_dev(rt, x, weights.final_norm_w(), seq, cfg["hidden_size"])
    return host(linear_dev(rt, x, weights.lm_head_w(), None, seq))


# ---------------------------------------------------------------------------
# TL:198-267: the weight archive
# ---------------------------------------------------------------------------
# the archive's geometry keys (``meta_<name>``, TL:205-217) and how each
# becomes a cfg value
_META_SCHEMA = (
    ("model_id", lambda v: str(np.asarray(v).item())),
    ("hidden_size", int),
    ("intermediate_size", int),
    ("num_hidden_layers", int),
    ("num_attention_heads", int),
    ("num_key_value_heads", int),
    ("head_dim", int),
    ("vocab_size", int),
    ("max_position_embeddings", int),
    ("rms_norm_eps", float),
    ("rope_theta", float),
)

class TinyLlamaWeights:
    """The reference's weight archive: ``meta_*`` geometry keys,
    ``embed_w`` [V][D], ``final_norm_w``, ``lm_head_w`` [D][V] and per layer
    ``layer{i}_{q,k,v,o,gate,up,down}_w`` ([K][N], x @ W) with optional
    ``_b`` biases and ``layer{i}_{input,post}_norm_w``.  Loaded with
    ``np.load`` (no pickle).  ``from_arrays`` builds the same object from a
    dict of arrays and a cfg (for synthetic models).

    Optional static KV-cache scales may ride along as ``kv_k_scale`` /
    ``kv_v_scale`` [L][Hkv] float32 arrays; without them the INT8 path
    calibrates them on the first prompt it sees.
    """

    def __init__(self, path: str | None = None, compute_dtype=np.float32, cache_arrays: bool = False,
                 data=None):
        self.path = path
        self.data = np.load(path) if data is None else data
        self.compute_dtype = compute_dtype
        self.cache_arrays = cache_arrays
        self._cache: dict = {}
        self.cfg = {name: conv(self.data["meta_" + name]) for name, conv in _META_SCHEMA}
        self.cfg["num_key_value_groups"] = self.cfg["num_attention_heads"] // self.cfg["num_key_value_heads"]
        self.cfg["attn_scale"] = 1.0 / np.sqrt(self.cfg["head_dim"])

    @classmethod
    def from_arrays(cls, arrays: dict) -> "TinyLlamaWeights":
        return cls(data=_DictArchive(arrays))

    def _files(self):
        return self.data.files

    def _array(self, key: str) -> np.ndarray:
        """Archive entry ``key`` in compute_dtype (no copy when it already is),
        memoised per key when cache_arrays is set."""
        arr = self._cache.get(key)
        if arr is None:
            arr = self.data[key].astype(self.compute_dtype, copy=False)
            if self.cache_arrays:
                self._cache[key] = arr
        return arr

    def _optional_array(self, key: str):
        return self._array(key) if key in self._files() else None

    def embed(self, token_ids) -> np.ndarray:
        return self._array("embed_w")[token_ids]

    def final_norm_w(self) -> np.ndarray:
        return self._array("final_norm_w")

    def lm_head_w(self) -> np.ndarray:
        return self._array("lm_head_w")

    def kv_scales(self):
        """(k_scales, v_scales) [L][Hkv] float32 if the archive carries them."""
        if "kv_k_scale" in self._files() and "kv_v_scale" in self._files():
            return (np.asarray(self.data["kv_k_scale"], np.float32), np.asarray(self.data["kv_v_scale"], np.float32))
        return None

    def layer(self, idx: int) -> dict:
        out = {}
        for n in ("q", "k", "v", "o"):
            out[f"{n}_w"] = self._array(f"layer{idx}_{n}_w")
        for n in ("q", "k", "v", "o"):
            out[f"{n}_b"] = self._optional_array(f"layer{idx}_{n}_b")
        for n in ("gate", "up", "down"):
            out[f"{n}_w"] = self._array(f"layer{idx}_{n}_w")
        for n in ("gate", "up", "down"):
            out[f"{n}_b"] = self._optional_array(f"layer{idx}_{n}_b")
        out["input_norm_w"] = self._array(f"layer{idx}_input_norm_w")
        out["post_norm_w"] = self._array(f"layer{idx}_post_norm_w")
        return out


class _DictArchive:
    """A dict of arrays with the ``files`` / ``__getitem__`` face of np.load."""

    def __init__(self, arrays: dict):
        self._a = {k: np.asarray(v) for k, v in arrays.items()}
        self.files = list(self._a)

    def __getitem__(self, k):
        return self._a[k]


def load_weights(path: str, compute_dtype=np.float32, cache_arrays: bool = False) -> TinyLlamaWeights:
    return TinyLlamaWeights(path, compute_dtype=compute_dtype, cache_arrays=cache_arrays)
