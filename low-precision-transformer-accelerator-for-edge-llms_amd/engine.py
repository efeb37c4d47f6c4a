"""Device-resident INT8 TinyLlama engine over the C-ABI (KV-cache generation).

``Engine`` owns one ``tl_handle``: the quantized weights, the INT8 KV cache
(static per-layer/per-KV-head scales) and the HIP stream.  It is the KV-cache
counterpart of the reference's host loop (model/tinyllama_gemm_int8.py:629-685
run_generate, 437-467 forward_mixed): the prompt is prefilled once, then each
new token runs 22 decoder layers at M = 1 against the cache.

Host arrays are NumPy; device buffers are torch CUDA tensors used only as
memory (``data_ptr()`` handed to the library).
"""
from __future__ import annotations

import ctypes as C
from types import SimpleNamespace

import numpy as np

from . import _native
from ._native import TL_MEM_DEVICE, TL_MEM_HOST, Runtime
from .tinyllama import build_rope_cache

WEIGHT_ORDER = ("q_w", "k_w", "v_w", "o_w", "gate_w", "up_w", "down_w")


def _np(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


class Engine:
    """INT8 decoder hot path on one MI355X.

    ``model`` is any object with the attributes of a quantized model:
    ``cfg`` (dict of TL:205-221 geometry), ``layers`` (per layer: ``w`` list
    of 7 int8 [N][K] arrays in q,k,v,o,gate,up,down order, ``s`` their float32
    scales, ``g_in``, ``g_post``), ``lm_w``, ``lm_s``, ``g_final``, ``emb``,
    ``emb_s``, ``kv_sk``, ``kv_sv`` and optionally ``rope_cos``/``rope_sin``.
    Arrays may be NumPy (host) or torch CUDA tensors (device).
    """

    def __init__(self, cfg: dict, max_seqs: int = 1):
        self.cfg = dict(cfg)
        self.rt = Runtime(cfg, max_seqs=max_seqs)
        self.lib = self.rt.lib
        self.h = self.rt.h

    # ---- loading -------------------------------------------------------------
    @staticmethod
    def _src(x) -> int:
        return TL_MEM_DEVICE if hasattr(x, "is_cuda") and x.is_cuda else TL_MEM_HOST

    def _keep(self, x, dt):
        if hasattr(x, "data_ptr"):
            return x.contiguous()
        return _np(x, dt)

    def load_model(self, model) -> "Engine":
        for i, L in enumerate(model.layers):
            self.load_layer(i, L)
        self.load_lm_head(model.lm_w, model.lm_s, model.g_final)
        self.load_embedding(model.emb, model.emb_s)
        self.set_kv_scales(model.kv_sk, model.kv_sv)
        cos = getattr(model, "rope_cos", None)
        if cos is None:
            cos, sin = build_rope_cache(self.cfg["max_pos"], self.cfg["head_dim"], self.cfg["rope_theta"])
        else:
            sin = model.rope_sin
        self.set_rope_table(cos, sin)
        return self

    def load_random(self, seed: int, kv_range=(0.02, 0.06)) -> SimpleNamespace:
        """Load a seeded random-init model of this engine's geometry and return
        host copies of what was loaded (the attributes ``load_model`` reads).

        Float weights are drawn N(0, 0.02) on the device (torch's generator,
        plumbing only) and quantized per output channel by the library's own
        ``tl_quantize_weight_rows``; RMSNorm gains are N(1, 0.02); static KV
        scales are uniform in ``kv_range`` (NumPy generator of the same seed).
        Drawing 1.1 G weights on the device takes well under a second, which
        is what makes full-size runs practical."""
        import torch
        g = torch.Generator(device="cuda")
        g.manual_seed(int(seed))
        c = self.cfg
        D, F, V = c["hidden"], c["intermediate"], c["vocab"]
        kvd = c["n_kv_heads"] * c["head_dim"]
        shapes = [(D, D), (kvd, D), (kvd, D), (D, D), (F, D), (F, D), (D, F)]

        def qrows(rows, cols):
            w = torch.randn(rows, cols, generator=g, device="cuda", dtype=torch.float32) * 0.02
            q = torch.empty(rows, cols, dtype=torch.int8, device="cuda")
            sc = torch.empty(rows, dtype=torch.float32, device="cuda")
            self.rt.call("tl_quantize_weight_rows", w, rows, cols, q, sc)
            return q, sc

        def gains():
            return 1.0 + 0.02 * torch.randn(D, generator=g, device="cuda")

        host_layers = []
        for layer in range(c["n_layers"]):
            ws, ss = zip(*[qrows(*shp) for shp in shapes])
            L = dict(w=list(ws), s=list(ss), g_in=gains(), g_post=gains())
            self.load_layer(layer, L)
            host_layers.append(dict(w=[t.cpu().numpy() for t in L["w"]], s=[t.cpu().numpy() for t in L["s"]],
                                    g_in=L["g_in"].cpu().numpy(), g_post=L["g_post"].cpu().numpy()))
        lm_w, lm_s = qrows(V, D)
        emb, emb_s = qrows(V, D)
        g_final = gains()
        self.load_lm_head(lm_w, lm_s, g_final)
        self.load_embedding(emb, emb_s)
        rng = np.random.default_rng(int(seed))
        sk = rng.uniform(*kv_range, (c["n_layers"], c["n_kv_heads"])).astype(np.float32)
        sv = rng.uniform(*kv_range, (c["n_layers"], c["n_kv_heads"])).astype(np.float32)
        self.set_kv_scales(sk, sv)
        cos, sin = build_rope_cache(c["max_pos"], c["head_dim"], c["rope_theta"])
        self.set_rope_table(cos, sin)
        torch.cuda.synchronize()
        return SimpleNamespace(cfg=dict(c), layers=host_layers, lm_w=lm_w.cpu().numpy(), lm_s=lm_s.cpu().numpy(),
                               g_final=g_final.cpu().numpy(), emb=emb.cpu().numpy(), emb_s=emb_s.cpu().numpy(),
                               rope_cos=cos, rope_sin=sin, kv_sk=sk, kv_sv=sv)

    def load_layer(self, i: int, L) -> None:
        w = [self._keep(t, np.int8) for t in L["w"]]
        s = [self._keep(t, np.float32) for t in L["s"]]
        g_in = self._keep(L["g_in"], np.float32)
        g_post = self._keep(L["g_post"], np.float32)
        self.rt.load_layer(i, w, s, g_in, g_post, self._src(w[0]))

    def load_lm_head(self, w, s, g_final) -> None:
        w, s, g = self._keep(w, np.int8), self._keep(s, np.float32), self._keep(g_final, np.float32)
        self.rt.call("tl_load_lm_head", w, s, g, self._src(w))

    def load_embedding(self, e, s) -> None:
        e, s = self._keep(e, np.int8), self._keep(s, np.float32)
        self.rt.call("tl_load_embedding", e, s, self._src(e))

    def set_kv_scales(self, sk, sv) -> None:
        sk = _np(sk.cpu().numpy() if hasattr(sk, "cpu") else sk, np.float32)
        sv = _np(sv.cpu().numpy() if hasattr(sv, "cpu") else sv, np.float32)
        self.rt.call("tl_set_kv_scales", sk, sv)

    def set_rope_table(self, cos, sin) -> None:
        cos, sin = _np(cos, np.float32), _np(sin, np.float32)
        self.rt.call("tl_set_rope_table", cos, sin, int(cos.shape[0]))

    # ---- KV cache ---------------------------------------------------------------
    def kv_write(self, seq, layer, kv_head, t0, k_rows=None, v_rows=None) -> None:
        ref = k_rows if k_rows is not None else v_rows
        n = int(np.asarray(ref).shape[0])
        k = None if k_rows is None else _np(k_rows, np.int8)
        v = None if v_rows is None else _np(v_rows, np.int8)
        self.rt.call("tl_kv_write", int(seq), int(layer), int(kv_head), int(t0), n, k, v)

    def kv_read(self, seq, layer, kv_head, t0, n):
        k = np.empty((n, 64), np.int8)
        v = np.empty((n, 64), np.int8)
        self.rt.call("tl_kv_read", int(seq), int(layer), int(kv_head), int(t0), int(n), k, v)
        return k, v

    # ---- generation ---------------------------------------------------------------
    def prefill(self, tokens, seq: int = 0) -> tuple[int, float]:
        t = _np(tokens, np.int32)
        tok, lg = C.c_int32(), C.c_float()
        self.rt.check(self.lib.tl_prefill(self.h, int(seq), t.ctypes.data, int(t.size), C.byref(tok), C.byref(lg)),
                      "tl_prefill")
        return tok.value, lg.value

    def decode(self, max_new: int, seq: int = 0, eos_id: int = -1, abort_flag=None):
        out = np.empty(max(int(max_new), 1), np.int32)
        n, stop = C.c_int32(), C.c_int32()
        flag = None if abort_flag is None else C.addressof(abort_flag)
        self.rt.check(self.lib.tl_decode(self.h, int(seq), int(max_new), int(eos_id), flag, out.ctypes.data,
                                         C.byref(n), C.byref(stop)), "tl_decode")
        return out[:n.value], _native.STOP_REASONS[stop.value]

    def generate(self, prompt, max_new: int, seq: int = 0, eos_id: int = -1, abort_flag=None):
        p = _np(prompt, np.int32)
        out = np.empty(max(int(max_new), 1), np.int32)
        n, stop = C.c_int32(), C.c_int32()
        flag = None if abort_flag is None else C.addressof(abort_flag)
        self.rt.check(self.lib.tl_generate(self.h, int(seq), p.ctypes.data, int(p.size), int(max_new), int(eos_id),
                                           flag, out.ctypes.data, C.byref(n), C.byref(stop)), "tl_generate")
        return out[:n.value], _native.STOP_REASONS[stop.value]

    def decode_batch(self, tokens, start_pos, n_steps: int):
        t = _np(tokens, np.int32)
        p = _np(start_pos, np.int32)
        out = np.empty((t.size, int(n_steps)), np.int32)
        self.rt.call("tl_decode_batch", int(t.size), t, p, int(n_steps), out)
        return out

    def capture_step(self, layer: int, seq: int = 0, key0: int = 0, n_keys: int = -1) -> dict:
        """One greedy decode step (as one step of ``decode``) with the tensors
        of decoder layer ``layer`` copied out (golden_trace.capture_step)."""
        from .golden_trace import capture_step
        return capture_step(self.rt, seq, layer, key0, n_keys)

    def decode_layer(self, x_dev, layer: int, pos: int, seq: int = 0) -> None:
        """One decoder layer on a device row x_dev (torch float32 [D]) in place."""
        self.rt.call("tl_decode_layer", int(seq), int(layer), int(pos), x_dev)

    def sync(self) -> None:
        self.rt.call("tl_sync")

    def set_profiling(self, on: bool) -> None:
        self.rt.call("tl_set_profiling", int(bool(on)))

    def decode_timeline(self, n_steps: int, seq: int = 0) -> dict:
        """Device timeline of n_steps greedy decode steps (tl_decode_timeline):
        per kernel class, mean busy and following-gap microseconds per step."""
        return self.rt.decode_timeline(seq, n_steps)

    def profile(self, kclass: str):
        return self.rt.profile(kclass)

    def close(self) -> None:
        self.rt.close()
