"""Golden-trace I/O and decode-step debug capture.

- memh files in the reference's text format: one hexadecimal word per line,
  lower case, zero padded to ceil(bits / 4) digits, two's complement for
  negative values (EX:199-217 write_hex_memh); packed-lane rows with lane 0 in
  the least significant (right-most) position (EX:220-244
  write_packed_lane_memh); readers with the sign extension of
  hls/common/test_memh.hpp:14-76.
- The canonical case format of docs/golden_trace_plan.md (section 5): one
  manifest.json listing the cases, one .npz of numeric arrays per case, and
  packed RTL fixtures under <phase>/rtl/ (EX:292-415 build_gemm_case).
- capture_step: one greedy decode step with the tensors of one decoder layer
  copied out (the capture list of docs/design_decisions.txt:366-392, B8),
  through tl_capture_step.
- replay_gemm_case / replay_gemm_fixture: run an exported shared_gemm_engine
  case (EX:292-415) through the library's INT8 GEMM and compare the INT32
  accumulators.
- replay_requant_case / replay_requant_fixture: run an exported
  requantize_unit case (EX:528-653: 512 accumulator lanes, 16 Q16.16
  multipliers) through tl_requant_q16 and compare the INT8 lanes.
- replay of the element-wise case types: rope_unit (tl_rope_q16),
  causal_mask_unit (tl_causal_mask_i32), rmsnorm (tl_rmsnorm_quant), softmax
  (tl_softmax_rows), silu (tl_silu_mul) and argmax (tl_argmax_i32), with the
  exporter's Q16.16 conversions on the host (EX:152-161, 191-192, 875-927).
"""
from __future__ import annotations

import ctypes as C
import json
import os
from pathlib import Path

import numpy as np

from ._native import CAPTURE_TOPK, Runtime, TlCapture

_HEX = np.frombuffer(b"0123456789abcdef", dtype=np.uint8)


def _ceil_div(a: int, b: int) -> int:
    return -(-a // b)


def _as_words(values, bits: int) -> np.ndarray:
    """Integer values -> uint64 words masked to `bits` (two's complement).
    For integers, the signed branch of EX:210-214 ((v + 2**bits) & mask for
    v < 0) and the unsigned one (v & mask) give the same word."""
    a = np.asarray(values)
    if a.dtype.kind == "u":
        u = a.astype(np.uint64)
    elif a.dtype.kind in "ib":
        u = a.astype(np.int64).view(np.uint64)
    elif a.dtype.kind == "f":   # int(raw_value) truncates toward zero
        u = np.trunc(a).astype(np.int64).view(np.uint64)
    else:
        raise TypeError(f"memh values must be numeric, got {a.dtype}")
    if bits < 64:
        u = u & np.uint64((1 << bits) - 1)
    return u


def _hex_digits(words: np.ndarray, width: int) -> np.ndarray:
    """[n] uint64 -> [n][width] ASCII hex digits, most significant first."""
    shifts = np.arange(width - 1, -1, -1, dtype=np.uint64) * np.uint64(4)
    nib = (words.reshape(-1, 1) >> shifts) & np.uint64(0xF)
    return _HEX[nib.astype(np.intp)]


def _write_rows(path, digits: np.ndarray) -> None:
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    rows = np.concatenate([digits, np.full((digits.shape[0], 1), ord("\n"), np.uint8)], axis=1)
    path.write_bytes(rows.tobytes())


def write_hex_memh(path, values, *, bits: int, signed: bool) -> None:
    """EX:199-217: one word of `bits` per line, every value of the flattened
    array in order.  `signed` is kept for the reference's signature: the
    masked word does not depend on it."""
    del signed
    flat = np.asarray(values).reshape(-1)
    _write_rows(path, _hex_digits(_as_words(flat, bits), _ceil_div(bits, 4)))


def write_packed_lane_memh(path, values, *, bits_per_lane: int, signed: bool) -> None:
    """EX:220-244: one line per row (a 1-D array is one row), lanes written
    from the last to the first so lane 0 is the right-most word."""
    del signed
    arr = np.asarray(values)
    if arr.ndim == 1:
        arr = arr.reshape(1, -1)
    rows, lanes = arr.shape[0], int(np.prod(arr.shape[1:]))
    width = _ceil_div(bits_per_lane, 4)
    words = _as_words(arr.reshape(rows, lanes)[:, ::-1].reshape(-1), bits_per_lane)
    _write_rows(path, _hex_digits(words, width).reshape(rows, lanes * width))


def read_memh_lines(path) -> list[str]:
    """test_memh.hpp:14-28: the non-empty lines of the file."""
    p = Path(path)
    if not p.is_file():
        raise FileNotFoundError(f"Failed to open memh file: {path}")
    return [ln for ln in p.read_text().split("\n") if ln]


def _hex_prefix(token: str) -> int:
    """Leading hexadecimal digits of a token as an unsigned integer (what
    `stream >> std::hex` extracts; 0 when there are none), wrapped to 64 bits."""
    t = token.strip()
    if t[:2].lower() == "0x":
        t = t[2:]
    n = 0
    while n < len(t) and t[n] in "0123456789abcdefABCDEF":
        n += 1
    return int(t[:n], 16) & ((1 << 64) - 1) if n else 0


def parse_hex_unsigned(token: str) -> int:
    """test_memh.hpp:46-52."""
    return _hex_prefix(token)


def parse_hex_signed(token: str, bits: int) -> int:
    """test_memh.hpp:30-44: sign-extend from bit bits-1 (only that bit is
    tested; digits above it are kept), as a signed 64-bit value."""
    v = _hex_prefix(token)
    if bits < 64 and v & (1 << (bits - 1)):
        v |= ((1 << 64) - 1) & ~((1 << bits) - 1)
    return v - (1 << 64) if v >> 63 else v


_NIBBLE = np.full(256, 255, np.uint8)
_NIBBLE[np.frombuffer(b"0123456789abcdef", np.uint8)] = np.arange(16, dtype=np.uint8)
_NIBBLE[np.frombuffer(b"ABCDEF", np.uint8)] = np.arange(10, 16, dtype=np.uint8)


def _nibbles_to_words(nib: np.ndarray) -> np.ndarray:
    """[..., width] nibbles, most significant first -> [...] uint64."""
    words = np.zeros(nib.shape[:-1], np.uint64)
    for i in range(nib.shape[-1]):
        words = (words << np.uint64(4)) | nib[..., i].astype(np.uint64)
    return words


def _read_words(path) -> np.ndarray:
    """The unsigned word of every line (parse_hex_unsigned), vectorized when
    every line is 1..16 plain hex digits."""
    lines = read_memh_lines(path)
    if not lines:
        return np.zeros(0, np.uint64)
    if max(len(ln) for ln in lines) <= 16:
        try:
            b = np.char.rjust(np.char.encode(np.array(lines), "ascii"), 16, b"0")
        except UnicodeEncodeError:
            b = None
        if b is not None:
            nib = _NIBBLE[np.frombuffer(b.astype("S16").tobytes(), np.uint8).reshape(-1, 16)]
            if not (nib == 255).any():
                return _nibbles_to_words(nib)
    return np.array([_hex_prefix(ln) for ln in lines], np.uint64)


# The casts of test_memh.hpp:54-76 keep the low bits of the parsed value, which
# the sign extension of parse_hex_signed leaves unchanged.
def read_scalar_memh_i32(path) -> np.ndarray:
    """test_memh.hpp:54-60."""
    return (_read_words(path) & np.uint64(0xFFFFFFFF)).astype(np.uint32).view(np.int32)


def read_scalar_memh_u32(path) -> np.ndarray:
    """test_memh.hpp:62-68."""
    return (_read_words(path) & np.uint64(0xFFFFFFFF)).astype(np.uint32)


def read_scalar_memh_i8(path) -> np.ndarray:
    """test_memh.hpp:70-76."""
    return (_read_words(path) & np.uint64(0xFF)).astype(np.uint8).view(np.int8)


def read_packed_lane_memh(path, *, bits_per_lane: int, signed: bool, lanes: int | None = None) -> np.ndarray:
    """Inverse of write_packed_lane_memh: [rows][lanes] (int64 when signed,
    uint64 otherwise).  Every line must hold lanes * ceil(bits / 4) digits."""
    width = _ceil_div(bits_per_lane, 4)
    lines = read_memh_lines(path)
    if not lines:
        return np.zeros((0, lanes or 0), np.int64 if signed else np.uint64)
    n_chars = len(lines[0])
    if lanes is None:
        if n_chars % width:
            raise ValueError(f"{path}: line of {n_chars} digits is not a whole number of {width}-digit lanes")
        lanes = n_chars // width
    if any(len(ln) != lanes * width for ln in lines):
        raise ValueError(f"{path}: every line must hold {lanes} lanes of {width} hex digits")
    raw = np.frombuffer("".join(lines).encode("ascii"), dtype=np.uint8).reshape(len(lines), lanes, width)
    nib = _NIBBLE[raw]
    if (nib == 255).any():
        raise ValueError(f"{path}: non-hexadecimal character")
    words = _nibbles_to_words(nib)[:, ::-1]
    if not signed:
        return np.ascontiguousarray(words)
    if bits_per_lane >= 64:
        return np.ascontiguousarray(words.view(np.int64))
    sign = np.uint64(1 << (bits_per_lane - 1))
    ext = np.uint64(((1 << 64) - 1) & ~((1 << bits_per_lane) - 1))
    return np.ascontiguousarray(np.where(words & sign, words | ext, words).view(np.int64))


# ---------------------------------------------------------------------------
# canonical case format: manifest.json + one .npz per case
# ---------------------------------------------------------------------------
TRACE_FORMAT_VERSION = 1


def _manifest_path(root) -> Path:
    return Path(root) / "manifest.json"


def read_manifest(root) -> dict:
    p = _manifest_path(root)
    if not p.is_file():
        return {"trace_format_version": TRACE_FORMAT_VERSION, "cases": []}
    return json.loads(p.read_text())


def write_case(root, case_id: str, phase: str, block: str, arrays: dict, meta: dict | None = None) -> Path:
    """Write <root>/<phase>/<case_id>.npz and add (or replace) its manifest
    entry: case id, phase, block, path (relative to root), dtype and shape
    summaries and the caller's metadata."""
    root = Path(root)
    case_path = root / phase / f"{case_id}.npz"
    case_path.parent.mkdir(parents=True, exist_ok=True)
    arrays = {k: np.asarray(v) for k, v in arrays.items()}
    np.savez(case_path, **arrays)
    entry = {
        "case_id": case_id,
        "phase": phase,
        "block": block,
        "path": case_path.relative_to(root).as_posix(),
        "dtype_summary": {k: str(v.dtype) for k, v in arrays.items()},
        "shape_summary": {k: list(v.shape) for k, v in arrays.items()},
    }
    entry.update(meta or {})
    man = read_manifest(root)
    man["cases"] = [c for c in man.get("cases", []) if c.get("case_id") != case_id] + [entry]
    _manifest_path(root).write_text(json.dumps(man, indent=2) + "\n")
    return case_path


def _resolve(root: Path, path: str) -> Path:
    p = Path(path)
    if p.is_absolute() and p.exists():
        return p
    for base in (root, root.parent):
        if (base / p).exists():
            return base / p
    # the reference exporter records paths under its own output root
    for parent in [p] + list(p.parents):
        if parent.name == root.name:
            cand = root / p.relative_to(parent)
            if cand.exists():
                return cand
    raise FileNotFoundError(f"case file {path} not found under {root}")


def load_case(root, case_id: str) -> tuple[dict, dict[str, np.ndarray]]:
    """(manifest entry, arrays) of one case; arrays load without pickle."""
    root = Path(root)
    for entry in read_manifest(root).get("cases", []):
        if entry.get("case_id") == case_id:
            with np.load(_resolve(root, entry["path"]), allow_pickle=False) as z:
                return entry, {k: z[k] for k in z.files}
    raise KeyError(f"case {case_id} not in {_manifest_path(root)}")


# ---------------------------------------------------------------------------
# decode-step capture (design_decisions.txt:366-392)
# ---------------------------------------------------------------------------
def capture_step(rt: Runtime, seq: int, layer: int, key0: int = 0, n_keys: int = -1) -> dict:
    """One greedy decode step of sequence `seq` (as one step of tl_decode)
    with the tensors of decoder layer `layer` copied out.  The attention
    window holds keys key0 .. key0 + n_keys - 1 (n_keys < 0: through the
    step's position).  Returns a dict of NumPy arrays and scalars."""
    cfg = rt.cfg
    D, Hq, Hkv = cfg["hidden"], cfg["n_heads"], cfg["n_kv_heads"]
    KVD = Hkv * cfg["head_dim"]
    W = cfg["max_pos"] if n_keys < 0 else int(n_keys)
    out = {
        "layer_in": np.zeros(D, np.float32),
        "attn_in_q": np.zeros(D, np.int8),
        "qkv": np.zeros(D + 2 * KVD, np.float32),
        "q8": np.zeros(D, np.int8),
        "k_row": np.zeros(KVD, np.int8),
        "v_row": np.zeros(KVD, np.int8),
        "kv_scales": np.zeros(2 * Hkv, np.float32),
        "score_scale": np.zeros(Hq, np.float32),
        "scores": np.zeros(Hq * max(W, 1), np.int32),
        "probs": np.zeros(Hq * max(W, 1), np.int8),
        "attended": np.zeros(D, np.float32),
        "layer_out": np.zeros(D, np.float32),
        "final_hidden": np.zeros(D, np.float32),
        "top_ids": np.zeros(CAPTURE_TOPK, np.int32),
        "top_logits": np.zeros(CAPTURE_TOPK, np.float32),
    }
    cap = TlCapture()
    cap.layer, cap.key0, cap.n_keys = int(layer), int(key0), int(n_keys)
    for k, v in out.items():
        setattr(cap, k, v.ctypes.data)
    rt.check(rt.lib.tl_capture_step(rt.h, int(seq), C.byref(cap)), "tl_capture_step")
    W = cap.n_keys
    out["scores"] = out["scores"][:Hq * W].reshape(Hq, W)
    out["probs"] = out["probs"][:Hq * W].reshape(Hq, W)
    out["kv_scales"] = out["kv_scales"].reshape(2, Hkv)
    out.update(layer=int(layer), pos=cap.pos, key0=cap.key0, n_keys=W, token_in=cap.token_in, token=cap.token,
               logit=np.float32(cap.logit), attn_in_scale=cap.attn_in_scale, q_scale=cap.q_scale)
    return out


_SCALARS = ("layer", "pos", "key0", "n_keys", "token_in", "token")


def export_capture(capture: dict, root, case_id: str | None = None, memh: bool = True) -> str:
    """Write a capture as a decode-step case (phase7, block "decode_step"):
    the .npz holds every array and scalar, the manifest entry its layer,
    position and window, and with memh=True the integer tensors are also
    written as packed RTL fixtures under phase7/rtl/ (one 64-lane row per
    head for q8 / K / V, one row per head of the score and probability
    windows).  Returns the case id."""
    layer, pos = int(capture["layer"]), int(capture["pos"])
    case_id = case_id or f"phase7_decode_layer{layer}_pos{pos}"
    arrays = {k: v for k, v in capture.items() if isinstance(v, np.ndarray)}
    for k in _SCALARS:
        arrays[k] = np.asarray([capture[k]], np.int32)
    arrays["logit"] = np.asarray([capture["logit"]], np.float32)
    arrays["attn_in_scale"] = np.asarray([capture["attn_in_scale"]], np.float64)
    arrays["q_scale"] = np.asarray([capture["q_scale"]], np.float64)
    meta = {"layer_id": layer, "token_start": pos, "token_count": 1, "key0": int(capture["key0"]),
            "n_keys": int(capture["n_keys"])}
    if memh:
        base = Path(root) / "phase7" / "rtl" / case_id
        hd = 64
        write_hex_memh(base.with_suffix(".meta.memh"),
                       np.asarray([layer, pos, capture["key0"], capture["n_keys"], capture["token_in"],
                                   capture["token"]], np.uint32), bits=32, signed=False)
        write_packed_lane_memh(base.with_suffix(".q8_packed.memh"), capture["q8"].reshape(-1, hd), bits_per_lane=8,
                               signed=True)
        write_packed_lane_memh(base.with_suffix(".k_row_packed.memh"), capture["k_row"].reshape(-1, hd),
                               bits_per_lane=8, signed=True)
        write_packed_lane_memh(base.with_suffix(".v_row_packed.memh"), capture["v_row"].reshape(-1, hd),
                               bits_per_lane=8, signed=True)
        if capture["n_keys"] > 0:
            write_packed_lane_memh(base.with_suffix(".scores_packed.memh"), capture["scores"], bits_per_lane=32,
                                   signed=True)
            write_packed_lane_memh(base.with_suffix(".probs_packed.memh"), capture["probs"], bits_per_lane=8,
                                   signed=True)
        write_hex_memh(base.with_suffix(".top_ids.memh"), capture["top_ids"], bits=32, signed=False)
        meta["rtl_fixture_base"] = base.relative_to(Path(root)).as_posix()
    write_case(root, case_id, "phase7", "decode_step", arrays, meta)
    return case_id


# ---------------------------------------------------------------------------
# replay of exported shared_gemm_engine cases (EX:259-415)
# ---------------------------------------------------------------------------
GEMM_N_TILE = 32      # EX:45 N_TILE: lane = m_local * N_TILE + n_local (EX:283-289)
GEMM_LANES = 512      # EX:46


def _gemm_i8(rt: Runtime, act: np.ndarray, wt: np.ndarray) -> np.ndarray:
    """act [m][K] int8 . wt [K][n] int8 -> [m][n] int32 on the device (K is
    zero-padded to the GEMM's multiple of 64, which leaves every sum as is)."""
    from .tinyllama import dev, empty, host
    m, k = act.shape
    n = wt.shape[1]
    kp = max(64, _ceil_div(k, 64) * 64)
    a = np.zeros((m, kp), np.int8)
    a[:, :k] = act
    w = np.zeros((n, kp), np.int8)
    w[:, :k] = wt.T
    c = empty((m, n), np.int32)
    rt.call("tl_gemm_i8", dev(a), dev(w), m, n, kp, c)
    return host(c)


def replay_gemm_case(rt: Runtime, arrays: dict) -> dict:
    """A case .npz of EX:328-336 (act [m][K], wt [K][n], acc_expected [m][n]):
    the library's accumulators and whether they equal the expected ones."""
    act = np.asarray(arrays["act"], np.int8)
    wt = np.asarray(arrays["wt"], np.int8)
    acc = _gemm_i8(rt, act, wt)
    exp = np.asarray(arrays["acc_expected"], np.int32)
    return {"acc": acc, "match": bool(acc.shape == exp.shape and np.array_equal(acc, exp))}


def replay_gemm_fixture(rt: Runtime, fixture_base) -> dict:
    """The RTL fixture files of EX:338-386 (<base>.meta.memh = K, active
    lanes, m, n; .act_steps.memh / .wt_steps.memh = [K][512] int8 lane
    steps; .acc_expected_lane.memh = [512] int32): rebuild the operand tiles
    from the lanes, run them through the library and compare lane by lane."""
    base = str(fixture_base)
    k_total, active, m, n = (int(v) for v in read_scalar_memh_u32(base + ".meta.memh")[:4])
    if active != m * n or m * GEMM_N_TILE > GEMM_LANES or n > GEMM_N_TILE:
        raise ValueError(f"{base}: meta {k_total, active, m, n} does not fit the lane packing")
    act_steps = read_scalar_memh_i8(base + ".act_steps.memh").reshape(k_total, GEMM_LANES)
    wt_steps = read_scalar_memh_i8(base + ".wt_steps.memh").reshape(k_total, GEMM_LANES)
    acc_lane = read_scalar_memh_i32(base + ".acc_expected_lane.memh")
    act = np.ascontiguousarray(act_steps[:, [mi * GEMM_N_TILE for mi in range(m)]].T)
    wt = np.ascontiguousarray(wt_steps[:, :n])
    acc = _gemm_i8(rt, act, wt)
    lanes = np.zeros(GEMM_LANES, np.int32)
    for mi in range(m):
        lanes[mi * GEMM_N_TILE:mi * GEMM_N_TILE + n] = acc[mi]
    return {"acc": acc, "acc_lane": lanes, "match": bool(np.array_equal(lanes, acc_lane))}


# ---------------------------------------------------------------------------
# replay of exported requantize_unit cases (EX:528-653)
# ---------------------------------------------------------------------------
REQUANT_LANES_PER_SCALE = 32   # requantize_unit.sv:109: multiplier of lane i is scale[i / BANK_SLICE_INT8]


def _requant_q16(rt: Runtime, acc: np.ndarray, scale: np.ndarray, elem_count: int) -> np.ndarray:
    """tl_requant_q16 over the lanes; an element count of 0 means every lane
    (requantize_unit.sv effective_elem_count)."""
    from .tinyllama import dev, empty, host
    acc = np.ascontiguousarray(acc, np.int32)
    n = acc.size
    active = n if elem_count == 0 else min(int(elem_count), n)
    y = empty((n,), np.int8)
    rt.call("tl_requant_q16", dev(acc), dev(np.ascontiguousarray(scale, np.uint32).view(np.int32)), n, active,
            REQUANT_LANES_PER_SCALE, 0, y)
    return host(y)


def replay_requant_case(rt: Runtime, arrays: dict) -> dict:
    """A case .npz of EX:560-568 (acc [512] int32 lanes, scale [16] uint32
    Q16.16, elem_count [1], out_expected [512] int8): the library's output
    lanes and whether they equal the expected ones."""
    out = _requant_q16(rt, arrays["acc"], arrays["scale"], int(np.asarray(arrays["elem_count"]).ravel()[0]))
    exp = np.asarray(arrays["out_expected"], np.int8)
    return {"out": out, "match": bool(out.shape == exp.shape and np.array_equal(out, exp))}


def replay_requant_fixture(rt: Runtime, fixture_base) -> dict:
    """The RTL fixture files of EX:578-625 (<base>.meta.memh = active lanes;
    .acc.memh [512] int32; .scale.memh [16] uint32 Q16.16;
    .out_expected.memh [512] int8), replayed lane by lane."""
    base = str(fixture_base)
    active = int(read_scalar_memh_u32(base + ".meta.memh")[0])
    acc = read_scalar_memh_i32(base + ".acc.memh")
    scale = read_scalar_memh_u32(base + ".scale.memh")
    exp = read_scalar_memh_i8(base + ".out_expected.memh")
    out = _requant_q16(rt, acc, scale, active)
    return {"out": out, "match": bool(out.shape == exp.shape and np.array_equal(out, exp))}


# ---------------------------------------------------------------------------
# Q16.16 conversions of the exporter's fixed-point cases, vectorised
# restatements of EX:152-161, 191-192, 875-927
# ---------------------------------------------------------------------------
Q16 = 1 << 16
MASK_NEG_INF = -1000000000   # tinyllama_pkg.sv (EX:73)


def q16_from_float(v) -> np.ndarray:
    """EX:152-155: round(max(0, v) 2^16) clamped to uint32 (round half to
    even, as Python's round on a float)."""
    x = np.rint(np.maximum(np.asarray(v, np.float64), 0.0) * Q16)
    return np.clip(x, 0, 0xFFFFFFFF).astype(np.uint32)


def q16_signed_from_float(v) -> np.ndarray:
    """EX:158-161: round(v 2^16) clamped to int32."""
    x = np.rint(np.asarray(v, np.float64) * Q16)
    return np.clip(x, -(1 << 31), (1 << 31) - 1).astype(np.int32)


def float_from_q16(raw) -> np.ndarray:
    """EX:191-192: float32(raw / 2^16)."""
    return (np.asarray(raw, np.int64).astype(np.float64) / Q16).astype(np.float32)


def quantize_fixed_by_scale_q16(values_q16, scale_q16: int, nonnegative_only: bool = False) -> np.ndarray:
    """EX:900-927: |v| / scale rounded half to even on the exact integer
    quotient and remainder, sign restored, clamped to +-127 or [0, 127]."""
    den = int(scale_q16) if int(scale_q16) != 0 else 1
    v = np.asarray(values_q16, np.int64)
    mag = np.abs(v)
    q, rem = mag // den, mag % den
    q = q + ((2 * rem > den) | ((2 * rem == den) & (q & 1 == 1))).astype(np.int64)
    r = np.where(v < 0, -q, q)
    return np.clip(r, 0 if nonnegative_only else -127, 127).astype(np.int8)


def quantize_probability_q16(prob_q16) -> np.ndarray:
    """EX:875-888: round_half_even(p 127 / 2^16) of Q16.16 probabilities,
    clamped to [0, 127]."""
    prod = np.asarray(prob_q16, np.int64) * 127
    q, rem = prod >> 16, prod & (Q16 - 1)
    q = q + ((rem > Q16 // 2) | ((rem == Q16 // 2) & (q & 1 == 1))).astype(np.int64)
    return np.clip(q, 0, 127).astype(np.int8)


def _scalar(arrays: dict, key: str) -> float:
    return np.asarray(arrays[key]).ravel()[0].item()


def _fp_close(got, want, rtol: float = 1e-6, atol: float = 1e-9) -> bool:
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return bool(got.shape == want.shape and np.all(np.abs(got - want) <= atol + rtol * np.abs(want)))


# ---------------------------------------------------------------------------
# replay of the exporter's phase-4/5/6 element-wise case types
# ---------------------------------------------------------------------------
def replay_rope_case(rt: Runtime, arrays: dict) -> dict:
    """rope_unit case (EX:930-1006: q_in / k_in [tokens][64] int8 of one head
    at positions token_base + t, q_out_expected / k_out_expected) through
    tl_rope_q16, the accelerator's INT8 RoPE."""
    from .tinyllama import dev, empty, host
    base = int(_scalar(arrays, "token_base"))
    out = {}
    for name in ("q", "k"):
        x = np.ascontiguousarray(arrays[f"{name}_in"], np.int8)
        rows = x.shape[0]
        pos = np.arange(base, base + rows, dtype=np.int32)
        y = empty(x.shape, np.int8)
        rt.call("tl_rope_q16", dev(x), rows, x.shape[1] // 64, dev(pos), y)
        out[name] = host(y)
    match = all(np.array_equal(out[n], np.asarray(arrays[f"{n}_out_expected"], np.int8)) for n in ("q", "k"))
    return {"q_out": out["q"], "k_out": out["k"], "match": bool(match)}


def replay_causal_mask_case(rt: Runtime, arrays: dict) -> dict:
    """causal_mask_unit case (EX:1009-1086: score_in [8][64] int32 with the
    query / key position bases and active row / column counts) through
    tl_causal_mask_i32."""
    from .tinyllama import dev, empty, host
    s = np.ascontiguousarray(arrays["score_in"], np.int32)
    out = empty(s.shape, np.int32)
    rt.call("tl_causal_mask_i32", dev(s), s.shape[0], s.shape[1], int(_scalar(arrays, "query_pos_base")),
            int(_scalar(arrays, "key_pos_base")), int(_scalar(arrays, "query_row_count")),
            int(_scalar(arrays, "key_col_count")), out)
    got = host(out)
    return {"score_out": got, "match": bool(np.array_equal(got, np.asarray(arrays["score_out_expected"], np.int32)))}


def replay_rmsnorm_case(rt: Runtime, arrays: dict) -> dict:
    """rmsnorm case (EX:1705-1805): the golden RMSNorm of the Q16.16-exact
    input rows x_deq with the gains rounded through Q16.16 (EX:1722-1724) runs
    on the device (tl_rmsnorm_quant, TL:45-50 arithmetic); its output goes to
    Q16.16 and is quantized at the case's output scale as EX:1725-1727 does.
    Match: y_fp bit for bit and y_q equal."""
    from .tinyllama import dev, empty, host
    x = np.ascontiguousarray(arrays["x_deq"], np.float32)
    rows, n = x.shape
    gamma = float_from_q16(q16_signed_from_float(np.asarray(arrays["gamma_fp"], np.float32)))
    y = empty((rows, n), np.float32)
    q = empty((rows, n), np.int8)
    sc = empty((rows,), np.float64)
    rt.call("tl_rmsnorm_quant", dev(x), dev(gamma), rows, n, y, q, sc)
    y_fp = host(y)
    y_q = quantize_fixed_by_scale_q16(q16_signed_from_float(y_fp), int(q16_from_float(_scalar(arrays, "output_scale"))))
    fp_ok = bool(np.array_equal(y_fp.view(np.uint32), np.asarray(arrays["y_fp"], np.float32).view(np.uint32)))
    q_ok = bool(np.array_equal(y_q, np.asarray(arrays["y_q"], np.int8)))
    return {"y_fp": y_fp, "y_q": y_q, "match_fp": fp_ok, "match": fp_ok and q_ok}


def replay_softmax_case(rt: Runtime, arrays: dict) -> dict:
    """softmax case (EX:1808-1893): the active rows of score_fp (the masked
    scores times the Q16.16 score scale) through tl_softmax_rows (TL:100-103
    arithmetic), then Q16.16 probabilities and their INT8 form (EX:1820-1824).
    The golden's softmax agrees with the library's within 1e-6 relative, so
    the float match is to that tolerance; prob_q must be equal."""
    from .tinyllama import dev, empty, host
    s = np.ascontiguousarray(arrays["score_fp"], np.float32)
    rows = int(np.count_nonzero(np.asarray(arrays["prob_fp"], np.float32).any(axis=1)))
    prob = np.zeros_like(s)
    if rows:
        p = empty((rows, s.shape[1]), np.float32)
        rt.call("tl_softmax_rows", dev(np.ascontiguousarray(s[:rows])), rows, s.shape[1], p)
        prob[:rows] = host(p)
    prob_q = quantize_probability_q16(q16_signed_from_float(prob))
    fp_ok = _fp_close(prob, arrays["prob_fp"])
    q_ok = bool(np.array_equal(prob_q, np.asarray(arrays["prob_q"], np.int8)))
    return {"prob_fp": prob, "prob_q": prob_q, "match_fp": fp_ok, "match": fp_ok and q_ok}


def replay_silu_case(rt: Runtime, arrays: dict) -> dict:
    """silu case (EX:1896-1990): SiLU of x_deq through tl_silu_mul (TL:159-161
    arithmetic), then Q16.16 and the fixed-point quantization at the case's
    output scale (EX:1905-1907).  Float match within 1e-6 relative (the
    golden's np.exp), y_q equal."""
    from .tinyllama import dev, empty, host
    x = np.ascontiguousarray(arrays["x_deq"], np.float32)
    y = empty(x.shape, np.float32)
    rt.call("tl_silu_mul", dev(x), None, int(x.size), y)
    y_fp = host(y)
    y_q = quantize_fixed_by_scale_q16(q16_signed_from_float(y_fp), int(q16_from_float(_scalar(arrays, "output_scale"))))
    fp_ok = _fp_close(y_fp, arrays["y_fp"])
    q_ok = bool(np.array_equal(y_q, np.asarray(arrays["y_q"], np.int8)))
    return {"y_fp": y_fp, "y_q": y_q, "match_fp": fp_ok, "match": fp_ok and q_ok}


def replay_argmax_case(rt: Runtime, arrays: dict) -> dict:
    """argmax case (EX:1651-1702: Q16.16 logits of the whole vocabulary)
    through tl_argmax_i32 (argmax_reduction.sv, lowest id wins a tie)."""
    from .tinyllama import dev
    v = np.ascontiguousarray(arrays["logits_q16"], np.int32)
    idx, val = C.c_int32(), C.c_int32()
    rt.call("tl_argmax_i32", dev(v), int(v.size), C.byref(idx), C.byref(val))
    match = idx.value == int(_scalar(arrays, "argmax_expected")) and val.value == int(_scalar(arrays, "logit_expected"))
    return {"token": idx.value, "logit": val.value, "match": bool(match)}


def replay_fixture(rt: Runtime, fixture_base) -> dict:
    """Replay one RTL fixture: a requantize_unit fixture has .acc.memh, a
    shared_gemm_engine fixture .act_steps.memh."""
    base = str(fixture_base)
    if os.path.exists(base + ".acc.memh"):
        return replay_requant_fixture(rt, base)
    return replay_gemm_fixture(rt, base)


REPLAYERS = {"shared_gemm_engine": replay_gemm_case, "requantize_unit": replay_requant_case,
             "rope_unit": replay_rope_case, "causal_mask_unit": replay_causal_mask_case,
             "rmsnorm": replay_rmsnorm_case, "softmax": replay_softmax_case, "silu": replay_silu_case,
             "argmax": replay_argmax_case}


def replay_manifest(rt: Runtime, root) -> list[dict]:
    """Replay every case a manifest lists whose block has a replayer
    (REPLAYERS); other blocks are reported as not replayed."""
    root = Path(root)
    results = []
    for entry in read_manifest(root).get("cases", []):
        replay = REPLAYERS.get(entry.get("block"))
        if replay is None:
            results.append({"case_id": entry.get("case_id"), "replayed": False})
            continue
        _, arrays = load_case(root, entry["case_id"])
        r = replay(rt, arrays)
        results.append({"case_id": entry["case_id"], "replayed": True, "match": r["match"]})
    return results


def fixture_paths(root) -> list[str]:
    """Sorted fixture bases (<...>/rtl/<case_id>) found under root."""
    out = set()
    for dirpath, _, files in os.walk(root):
        for f in files:
            if f.endswith(".meta.memh"):
                out.add(os.path.join(dirpath, f[: -len(".meta.memh")]))
    return sorted(out)
