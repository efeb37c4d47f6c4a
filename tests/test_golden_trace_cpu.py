"""Golden-trace I/O without a GPU: the memh writers and readers against the
reference's own memh text (rtl/compute/rope_{cos,sin}_rom.memh lines kept in
tests/golden/), against the reference's C++ readers (hls/common/test_memh.hpp,
built into oracle/_ref/ when the reference checkout is present) and against
hand-worked words; the manifest + .npz case format round trip."""
import json
import os
import subprocess

import numpy as np
import pytest

from conftest import GOLDEN, ROOT, golden
from lpta import golden_trace as gt

SLICE_POSITIONS = (0, 1, 93, 1021, 2047)   # tests/golden/make_memh_slices.py
MEMH_READER = os.path.join(ROOT, "oracle", "_ref", "memh_reader")


def _rom_rows(kind):
    d = golden("rope_rom.npz")
    pos = list(d["positions"])
    return np.stack([d[f"{kind}_q16"][pos.index(p)] for p in SLICE_POSITIONS]).reshape(-1)


@pytest.mark.parametrize("kind", ["cos", "sin"])
def test_reader_decodes_reference_rom_text(kind):
    got = gt.read_scalar_memh_i32(os.path.join(GOLDEN, f"rope_{kind}_rom_slice.memh"))
    want = _rom_rows(kind)
    assert got.dtype == np.int32 and got.shape == want.shape
    np.testing.assert_array_equal(got, want)
    if kind == "sin":
        assert (got < 0).any()   # two's complement words are in the slice


@pytest.mark.parametrize("kind", ["cos", "sin"])
def test_writer_reproduces_reference_rom_text(kind, tmp_path):
    # EX:669-680 writes the ROM with write_hex_memh(bits=32, signed=True)
    path = tmp_path / "rom.memh"
    gt.write_hex_memh(path, _rom_rows(kind), bits=32, signed=True)
    with open(os.path.join(GOLDEN, f"rope_{kind}_rom_slice.memh"), "rb") as fh:
        assert path.read_bytes() == fh.read()


def test_hand_worked_words(tmp_path):
    p = tmp_path / "a.memh"
    gt.write_hex_memh(p, np.array([0, 1, -1, 127, -128], np.int8), bits=8, signed=True)
    assert p.read_text() == "00\n01\nff\n7f\n80\n"
    gt.write_hex_memh(p, np.array([-2, 65535], np.int64), bits=16, signed=True)
    assert p.read_text() == "fffe\nffff\n"
    gt.write_hex_memh(p, np.array([5, 6], np.uint32), bits=12, signed=False)   # width ceil(12 / 4) = 3
    assert p.read_text() == "005\n006\n"
    # lane 0 is the right-most word of a packed row
    gt.write_packed_lane_memh(p, np.array([[1, -1, 2], [3, 4, -128]], np.int8), bits_per_lane=8, signed=True)
    assert p.read_text() == "02ff01\n800403\n"
    gt.write_packed_lane_memh(p, np.array([-1, 2], np.int32), bits_per_lane=32, signed=True)
    assert p.read_text() == "00000002ffffffff\n"


def test_parse_hex_signed_edges():
    assert gt.parse_hex_signed("80", 8) == -128
    assert gt.parse_hex_signed("7f", 8) == 127
    assert gt.parse_hex_signed("1ff", 8) == -1        # bit 7 set: every bit above is set
    assert gt.parse_hex_signed("100", 8) == 256       # bit 7 clear: the extra digit stays
    assert gt.parse_hex_signed("ffffffff", 32) == -1
    assert gt.parse_hex_signed("ffffffffffffffff", 64) == -1
    assert gt.parse_hex_unsigned("0x10") == 16


EDGE_LINES = ["80", "1ff", "100", "7fffffff", "ffffffff", "FF", "0x10", "deadbeef", "123456789", "0", "7f"]


def test_readers_match_hand_casts(tmp_path):
    p = tmp_path / "e.memh"
    p.write_text("\n".join(EDGE_LINES) + "\n\n")
    assert gt.read_scalar_memh_i32(p).tolist() == [128, 511, 256, 2147483647, -1, 255, 16, -559038737,
                                                    591751049, 0, 127]
    assert gt.read_scalar_memh_i8(p).tolist() == [-128, -1, 0, -1, -1, -1, 16, -17, -119, 0, 127]
    assert gt.read_scalar_memh_u32(p).tolist()[4] == 0xFFFFFFFF


@pytest.mark.skipif(not os.path.exists(MEMH_READER), reason="oracle/_ref/memh_reader not built (needs the reference)")
@pytest.mark.parametrize("mode", ["i32", "u32", "i8"])
def test_readers_match_reference_cpp(mode, tmp_path):
    rng = np.random.default_rng(7)
    p = tmp_path / "r.memh"
    words = [f"{int(v):x}" for v in rng.integers(0, 1 << 36, 200)] + EDGE_LINES
    p.write_text("\n".join(words) + "\n")
    out = subprocess.run([MEMH_READER, mode, str(p)], capture_output=True, text=True, check=True).stdout
    want = [int(v) for v in out.split()]
    fn = {"i32": gt.read_scalar_memh_i32, "u32": gt.read_scalar_memh_u32, "i8": gt.read_scalar_memh_i8}[mode]
    assert fn(p).tolist() == want
    rom = os.path.join(GOLDEN, "rope_sin_rom_slice.memh")
    out = subprocess.run([MEMH_READER, mode, rom], capture_output=True, text=True, check=True).stdout
    assert fn(rom).tolist() == [int(v) for v in out.split()]


@pytest.mark.parametrize("bits,signed,dtype", [(8, True, np.int8), (16, False, np.uint16), (32, True, np.int32),
                                               (4, False, np.uint8)])
def test_round_trips(bits, signed, dtype, tmp_path):
    rng = np.random.default_rng(bits)
    info = np.iinfo(dtype)
    hi = min(int(info.max), (1 << bits) - 1)
    v = rng.integers(int(info.min), hi + 1, size=(7, 13)).astype(dtype)
    p = tmp_path / "x.memh"
    gt.write_packed_lane_memh(p, v, bits_per_lane=bits, signed=signed)
    back = gt.read_packed_lane_memh(p, bits_per_lane=bits, signed=signed)
    np.testing.assert_array_equal(back, v.astype(np.int64 if signed else np.uint64))
    gt.write_hex_memh(p, v, bits=bits, signed=signed)
    words = gt._read_words(p)
    np.testing.assert_array_equal(words, v.reshape(-1).astype(np.int64).view(np.uint64) & np.uint64((1 << bits) - 1))


def test_packed_reader_rejects_ragged_rows(tmp_path):
    p = tmp_path / "bad.memh"
    p.write_text("0102\n010\n")
    with pytest.raises(ValueError):
        gt.read_packed_lane_memh(p, bits_per_lane=8, signed=True)
    with pytest.raises(FileNotFoundError):
        gt.read_memh_lines(tmp_path / "missing.memh")


def test_case_manifest_round_trip(tmp_path):
    a = np.arange(12, dtype=np.int8).reshape(3, 4)
    b = np.array([1.5], np.float32)
    gt.write_case(tmp_path, "phase3_x", "phase3", "shared_gemm_engine", {"act": a, "s": b}, {"layer_id": 2})
    gt.write_case(tmp_path, "phase3_y", "phase3", "requantize_unit", {"act": a})
    gt.write_case(tmp_path, "phase3_x", "phase3", "shared_gemm_engine", {"act": a + 1}, {"layer_id": 3})
    man = json.loads((tmp_path / "manifest.json").read_text())
    assert [c["case_id"] for c in man["cases"]] == ["phase3_y", "phase3_x"]
    entry, arrays = gt.load_case(tmp_path, "phase3_x")
    assert entry["layer_id"] == 3 and entry["block"] == "shared_gemm_engine"
    assert entry["path"] == "phase3/phase3_x.npz"
    assert entry["shape_summary"]["act"] == [3, 4] and entry["dtype_summary"]["act"] == "int8"
    np.testing.assert_array_equal(arrays["act"], a + 1)
    with pytest.raises(KeyError):
        gt.load_case(tmp_path, "nope")
    # a path recorded under the exporter's own output root resolves too
    man["cases"][1]["path"] = f"sim/{tmp_path.name}/phase3/phase3_x.npz"
    (tmp_path / "manifest.json").write_text(json.dumps(man))
    np.testing.assert_array_equal(gt.load_case(tmp_path, "phase3_x")[1]["act"], a + 1)


# ---- Q16.16 conversions of the exporter's fixed-point cases --------------------------

def _rne_div(num: int, den: int) -> int:
    """num / den rounded half to even, exactly (Fraction arithmetic)."""
    from fractions import Fraction
    return round(Fraction(num, den))


def test_q16_conversions_match_scalar_definitions():
    """The vectorised conversions against the scalar arithmetic they restate
    (EX:152-161, 191-192), element by element, on random values, exact
    half-LSB ties and the clamping ends."""
    rng = np.random.default_rng(5)
    v = np.concatenate([rng.standard_normal(2000) * 10, rng.uniform(-40000, 40000, 500),
                        (np.arange(-40, 40) + 0.5) / 65536.0, [0.0, -0.0, 1e12, -1e12, 32767.99999]])
    v32 = v.astype(np.float32)
    want_s = [max(-(1 << 31), min(int(round(float(x) * 65536.0)), (1 << 31) - 1)) for x in v32]
    want_u = [max(0, min(int(round(max(0.0, float(x)) * 65536.0)), 0xFFFFFFFF)) for x in v32]
    assert gt.q16_signed_from_float(v32).tolist() == want_s
    assert gt.q16_from_float(v32).tolist() == want_u
    raw = np.concatenate([rng.integers(-(1 << 31), (1 << 31) - 1, 1000), [0, 1, -1, 65536, -(1 << 31)]])
    got = gt.float_from_q16(raw)
    assert got.dtype == np.float32
    assert all(g == np.float32(int(r) / 65536.0) for g, r in zip(got, raw))


def test_fixed_point_quantizers_match_exact_rounding():
    """quantize_fixed_by_scale_q16 (EX:900-927) and quantize_probability_q16
    (EX:875-888) against exact rational rounding half to even, with ties
    planted, both clamps and a zero scale (treated as 1)."""
    rng = np.random.default_rng(6)
    for den in (1, 2, 3, 65536, 77777, 1234567):
        vals = rng.integers(-(1 << 28), 1 << 28, 3000).astype(np.int64)
        ties = (np.arange(-20, 20) * 2 + 1) * den // 2 if den % 2 == 0 else np.arange(-20, 20) * den
        vals = np.concatenate([vals, ties, [0]])
        for nonneg in (False, True):
            got = gt.quantize_fixed_by_scale_q16(vals, den, nonnegative_only=nonneg)
            lo = 0 if nonneg else -127
            want = [max(lo, min(127, (-1 if x < 0 else 1) * _rne_div(abs(int(x)), den))) for x in vals]
            assert got.tolist() == want
    z = gt.quantize_fixed_by_scale_q16(np.array([5, -5, 130]), 0)
    assert z.tolist() == [5, -5, 127]
    p = np.concatenate([rng.integers(-1000, 70000, 5000), [0, 65536, 32768 // 127 * 127]]).astype(np.int64)
    p = np.concatenate([p, [x for x in range(0, 70000) if (x * 127) % 65536 == 32768][:50]])
    got = gt.quantize_probability_q16(p)
    want = [max(0, min(127, _rne_div(int(x) * 127, 65536))) for x in p]
    assert got.tolist() == want
