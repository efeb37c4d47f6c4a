"""Helpers for the GPU parity tests: device tensors and a per-geometry engine."""
from __future__ import annotations

import numpy as np

import lpta  # noqa: F401  (registered by conftest)


def torch():
    import torch as t
    return t


def dev(a):
    """NumPy -> torch CUDA tensor (plumbing only)."""
    t = torch()
    return t.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.detach().cpu().numpy()


def empty(shape, dtype):
    t = torch()
    tdt = {np.float32: t.float32, np.int8: t.int8, np.int32: t.int32, np.float64: t.float64}[dtype]
    return t.empty(shape, dtype=tdt, device="cuda")


OPS_CFG = dict(hidden=2048, intermediate=5632, n_layers=1, n_heads=32, n_kv_heads=4, head_dim=64,
               vocab=64, max_pos=2048, rms_eps=np.float32(1e-5), rope_theta=10000.0)


def runtime(cfg=OPS_CFG, max_seqs=1):
    from lpta import Runtime
    return Runtime(cfg, max_seqs=max_seqs)


def bits(a):
    a = np.asarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else (a.view(np.uint64) if a.dtype == np.float64 else a)


def assert_bits_equal(got, want, what=""):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    if not np.array_equal(bits(got), bits(want)):
        diff = np.argwhere(bits(got) != bits(want))
        i = tuple(diff[0])
        raise AssertionError(f"{what}: {len(diff)} mismatches, first at {i}: got {got[i]!r} want {want[i]!r}")
