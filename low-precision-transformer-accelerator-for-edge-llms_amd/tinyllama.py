"""Host-side counterparts of model/tinyllama.py (TL) needed by the INT8 path.

Only table construction lives here; every per-token computation runs in the
HIP library (see ops.py for the operator surface of TL's primitives).
"""
from __future__ import annotations

import numpy as np


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
