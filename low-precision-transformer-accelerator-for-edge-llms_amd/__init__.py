"""MI355X-native INT8 TinyLlama decoder hot path.

A from-scratch gfx950 implementation of the shared INT8 decoder path of
samarthbs27/Low-Precision-Transformer-Accelerator-for-Edge-LLMs: INT8 x INT8 ->
INT32 GEMV/GEMM with fused requantize/dequantize epilogues, GQA attention over
an INT8 KV cache with static per-layer/per-KV-head scales, RMSNorm, RoPE,
softmax, SiLU-GLU, residuals and greedy argmax.  Hand-written HIP kernels sit
behind a C-ABI (include/tl_int8.h, libtl_int8.so); this package is the Python
host side (ctypes): ``engine.Engine`` (device-resident model, KV-cache
generation) and, with the reference's own names and arguments, ``tinyllama``
(model/tinyllama.py primitives, weight archive) and ``tinyllama_gemm_int8``
(model/tinyllama_gemm_int8.py operator surface).

The package directory name is not a Python identifier; load it with
``__graft_entry__.load_package()`` (it registers the alias ``lpta``).
"""
from . import _native
from ._native import Runtime, TlConfig, TlError, TlValueError, header_symbols, library_path, load_library
from .tinyllama import build_rope_cache

__all__ = ["Runtime", "TlConfig", "TlError", "TlValueError", "header_symbols", "library_path",
           "load_library", "build_rope_cache", "Engine"]


def __getattr__(name):
    if name == "Engine":
        from .engine import Engine
        return Engine
    raise AttributeError(name)
