"""ctypes binding of libtl_int8.so (the C-ABI declared in include/tl_int8.h).

There is no CPU fallback: loading fails with an error when the library has not
been built, and ``Runtime`` fails when no gfx950 device is present.
"""
from __future__ import annotations

import ctypes as C
import os
import re

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB_PATH = os.path.join(PKG, "_lib", "libtl_int8.so")
HEADER = os.path.join(ROOT, "include", "tl_int8.h")

TL_OK, TL_ERR_BAD_DESCRIPTOR, TL_ERR_UNSUPPORTED, TL_ERR_INTERNAL = 0, 1, 6, 7
TL_MEM_HOST, TL_MEM_DEVICE = 0, 1
STOP_REASONS = {0: "none", 1: "eos", 2: "max_tokens", 3: "host_abort", 4: "internal_error"}
KCLASS = {"qkv": 0, "attn": 1, "o": 2, "glu": 3, "down": 4, "lm_head": 5, "norm": 6,
          "gemm_prefill": 7, "other": 8}


class TlConfig(C.Structure):
    _fields_ = [
        ("hidden", C.c_int32), ("intermediate", C.c_int32), ("n_layers", C.c_int32),
        ("n_heads", C.c_int32), ("n_kv_heads", C.c_int32), ("head_dim", C.c_int32),
        ("vocab", C.c_int32), ("max_pos", C.c_int32), ("rms_eps", C.c_float),
        ("rope_theta", C.c_float),
    ]

    @classmethod
    def from_dict(cls, d: dict) -> "TlConfig":
        return cls(int(d["hidden"]), int(d["intermediate"]), int(d["n_layers"]), int(d["n_heads"]),
                   int(d["n_kv_heads"]), int(d["head_dim"]), int(d["vocab"]), int(d["max_pos"]),
                   float(d["rms_eps"]), float(d["rope_theta"]))


CAPTURE_TOPK = 16   # TL_CAPTURE_TOPK


class TlCapture(C.Structure):
    """struct tl_capture: one decode step's tensors of one layer."""
    _fields_ = [
        ("layer", C.c_int32), ("key0", C.c_int32), ("n_keys", C.c_int32),
        ("pos", C.c_int32), ("token_in", C.c_int32), ("token", C.c_int32), ("logit", C.c_float),
        ("attn_in_scale", C.c_double), ("q_scale", C.c_double),
        ("layer_in", C.c_void_p), ("attn_in_q", C.c_void_p), ("qkv", C.c_void_p), ("q8", C.c_void_p),
        ("k_row", C.c_void_p), ("v_row", C.c_void_p), ("kv_scales", C.c_void_p), ("score_scale", C.c_void_p),
        ("scores", C.c_void_p), ("probs", C.c_void_p), ("attended", C.c_void_p), ("layer_out", C.c_void_p),
        ("final_hidden", C.c_void_p), ("top_ids", C.c_void_p), ("top_logits", C.c_void_p),
    ]


class TlTimeline(C.Structure):
    """struct tl_timeline: device timeline of batch-1 decode steps."""
    _fields_ = [("steps", C.c_int32), ("kernels", C.c_int32), ("step_us", C.c_double),
                ("busy_us", C.c_double * 9), ("gap_us", C.c_double * 9), ("launches", C.c_int32 * 9)]


class TlError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{message} (status {status})")
        self.status = status


class TlValueError(TlError, ValueError):
    """Bad arguments: raised where the reference raises ValueError."""


_vp = C.c_void_p
_i32 = C.c_int32
_i64 = C.c_int64
_i32p = C.POINTER(C.c_int32)
_f32p = C.POINTER(C.c_float)
_f64p = C.POINTER(C.c_double)

SIGNATURES = {
    "tl_create": (_i32, [C.POINTER(TlConfig), _i32, C.POINTER(_vp)]),
    "tl_destroy": (None, [_vp]),
    "tl_last_error": (C.c_char_p, [_vp]),
    "tl_status_string": (C.c_char_p, [_i32]),
    "tl_get_config": (_i32, [_vp, C.POINTER(TlConfig)]),
    "tl_sync": (_i32, [_vp]),
    "tl_load_layer": (_i32, [_vp, _i32, _vp * 7, _vp * 7, _vp, _vp, _i32]),
    "tl_load_lm_head": (_i32, [_vp, _vp, _vp, _vp, _i32]),
    "tl_load_embedding": (_i32, [_vp, _vp, _vp, _i32]),
    "tl_set_kv_scales": (_i32, [_vp, _vp, _vp]),
    "tl_set_rope_table": (_i32, [_vp, _vp, _vp, _i32]),
    "tl_kv_write": (_i32, [_vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp]),
    "tl_kv_read": (_i32, [_vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp]),
    "tl_quantize_rows": (_i32, [_vp, _vp, _i32, _i32, _vp, _vp]),
    "tl_quantize_tensor": (_i32, [_vp, _vp, _i64, _vp, _vp]),
    "tl_quantize_weight_rows": (_i32, [_vp, _vp, _i32, _i32, _vp, _vp]),
    "tl_rmsnorm_quant": (_i32, [_vp, _vp, _vp, _i32, _i32, _vp, _vp, _vp]),
    "tl_gemv_i8_requant": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _vp, _vp]),
    "tl_requant_q16": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp]),
    "tl_causal_mask_i32": (_i32, [_vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _vp]),
    "tl_rope_q16": (_i32, [_vp, _vp, _i32, _i32, _vp, _vp]),
    "tl_argmax_i32": (_i32, [_vp, _vp, _i32, _i32p, _i32p]),
    "tl_gemm_i8": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _vp]),
    "tl_gemm_i8_noalloc": (_i32, [_vp, _vp, _vp, _i32, _i32, _i32, _vp]),
    "tl_gemm_i8_dequant": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _vp]),
    "tl_rope": (_i32, [_vp, _vp, _i32, _i32, _vp]),
    "tl_linear_f32": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp]),
    "tl_attention_f32": (_i32, [_vp, _vp, _vp, _vp, _i32, _i32, _i32, C.c_float, _vp, _vp, _vp]),
    "tl_softmax_rows": (_i32, [_vp, _vp, _i32, _i32, _vp]),
    "tl_silu_mul": (_i32, [_vp, _vp, _vp, _i64, _vp]),
    "tl_attention": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp]),
    "tl_qkv_append": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp]),
    "tl_lm_head_argmax": (_i32, [_vp, _vp, _i32p, _f32p, _vp]),
    "tl_embed": (_i32, [_vp, _vp, _i32, _vp]),
    "tl_decode_layer": (_i32, [_vp, _i32, _i32, _i32, _vp]),
    "tl_layer_rows": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp]),
    "tl_prefill_logits": (_i32, [_vp, _i32, _vp, _i32, _vp]),
    "tl_dequantize_i32": (_i32, [_vp, _vp, C.c_int64, _i32, C.c_double, C.c_double, _vp, _vp]),
    "tl_prefill": (_i32, [_vp, _i32, _vp, _i32, _i32p, _f32p]),
    "tl_decode": (_i32, [_vp, _i32, _i32, _i32, _vp, _vp, _i32p, _i32p]),
    "tl_generate": (_i32, [_vp, _i32, _vp, _i32, _i32, _i32, _vp, _vp, _i32p, _i32p]),
    "tl_decode_batch": (_i32, [_vp, _i32, _vp, _vp, _i32, _vp]),
    "tl_capture_step": (_i32, [_vp, _i32, C.POINTER(TlCapture)]),
    "tl_set_profiling": (_i32, [_vp, _i32]),
    "tl_get_profile": (_i32, [_vp, _i32, C.POINTER(C.c_int64), _f64p, _f64p]),
    "tl_decode_timeline": (_i32, [_vp, _i32, _i32, C.POINTER(TlTimeline)]),
}


def header_symbols(path: str = HEADER) -> list[str]:
    """Function names declared in include/tl_int8.h."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tl_[a-z0-9_]+)\s*\(", text)))


_lib = None


def _bind_torch_runtime() -> None:
    """PyTorch-ROCm ships its own HIP runtime (SONAME libamdhip64.so.7) and
    loads it under another file name.  Importing torch before this library
    makes the dynamic linker resolve our libamdhip64.so.7 dependency to that
    already-loaded copy, so the process has a single HIP runtime and torch
    device pointers are valid here.  Without torch the library binds to the
    system ROCm runtime."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def library_path() -> str:
    return LIB_PATH


def load_library() -> C.CDLL:
    """Load libtl_int8.so and declare every entry point.  Needs no GPU."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build the HIP library first (__graft_entry__.build())")
    _bind_torch_runtime()
    L = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _fence(args) -> None:
    """The library runs on its own non-blocking stream: device inputs written
    by torch on torch's current stream must be complete before a call reads
    them, so wait for that stream when any argument is a CUDA tensor."""
    for a in args:
        if getattr(a, "is_cuda", False):
            import torch
            torch.cuda.current_stream(a.device).synchronize()
            return


def _addr(x) -> int | None:
    """Device or host address of a torch tensor, a NumPy array or an int."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    if hasattr(x, "ctypes"):
        return x.ctypes.data
    raise TypeError(f"cannot take the address of {type(x)}")


class Runtime:
    """One tl_handle: a device-resident model, its KV cache and a HIP stream."""

    def __init__(self, cfg: dict, max_seqs: int = 1):
        self.lib = load_library()
        self.cfg = dict(cfg)
        h = _vp()
        st = self.lib.tl_create(C.byref(TlConfig.from_dict(cfg)), int(max_seqs), C.byref(h))
        if st != TL_OK:
            msg = self.lib.tl_last_error(None).decode()
            raise (TlValueError if st == TL_ERR_BAD_DESCRIPTOR else TlError)(st, f"tl_create: {msg}")
        self.h = h
        self.max_seqs = max_seqs

    def close(self):
        if getattr(self, "h", None):
            self.lib.tl_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def check(self, status: int, what: str = "") -> None:
        if status != TL_OK:
            msg = self.lib.tl_last_error(self.h).decode()
            cls = TlValueError if status == TL_ERR_BAD_DESCRIPTOR else TlError
            raise cls(status, f"{what}: {msg}" if what else msg)

    def call(self, name: str, *args) -> None:
        """Call tl_<name>(h, *args): tensors and arrays become their addresses,
        everything else (ints, floats, ctypes objects, None) passes through."""
        fn = getattr(self.lib, name)
        _fence(args)
        conv = [_addr(a) if hasattr(a, "data_ptr") or hasattr(a, "__array_interface__") else a for a in args]
        self.check(fn(self.h, *conv), name)

    # ---- model state -------------------------------------------------------
    def load_layer(self, layer: int, w: list, s: list, g_in, g_post, src: int) -> None:
        _fence([*w, *s, g_in, g_post])
        wa = (_vp * 7)(*[_addr(t) for t in w])
        sa = (_vp * 7)(*[_addr(t) for t in s])
        self.check(self.lib.tl_load_layer(self.h, layer, wa, sa, _addr(g_in), _addr(g_post), src), "tl_load_layer")

    def decode_timeline(self, seq: int, n_steps: int) -> dict:
        """tl_decode_timeline: mean per-step device busy time and following gap
        per kernel class, in microseconds."""
        t = TlTimeline()
        self.check(self.lib.tl_decode_timeline(self.h, int(seq), int(n_steps), C.byref(t)), "tl_decode_timeline")
        classes = {name: {"launches": t.launches[k], "busy_us": t.busy_us[k], "gap_us": t.gap_us[k]}
                   for name, k in KCLASS.items() if t.launches[k]}
        return {"steps": t.steps, "kernels": t.kernels, "step_us": t.step_us, "classes": classes}

    def profile(self, kclass: str) -> tuple[int, float, float]:
        cnt, ms, by = C.c_int64(), C.c_double(), C.c_double()
        self.check(self.lib.tl_get_profile(self.h, KCLASS[kclass], C.byref(cnt), C.byref(ms), C.byref(by)))
        return cnt.value, ms.value, by.value
