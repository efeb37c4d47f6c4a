"""C-ABI checks that need no GPU: the library loads, exports every function
include/tl_int8.h declares, and refuses to run without a gfx950 device
instead of falling back to the CPU."""
import ctypes
import os

import pytest

import lpta
from lpta import _native


def test_library_exports_every_header_symbol():
    lib = lpta.load_library()
    declared = lpta.header_symbols()
    assert len(declared) >= 30
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, f"declared in tl_int8.h but not exported: {missing}"
    # and the Python binding declares a signature for each of them
    assert sorted(_native.SIGNATURES) == declared


def test_status_strings():
    lib = lpta.load_library()
    assert lib.tl_status_string(0) == b"ok"
    assert lib.tl_status_string(1) == b"bad descriptor"
    assert lib.tl_status_string(7) == b"internal error"


def test_config_layout_matches_header():
    # ten 4-byte fields, as tl_config in include/tl_int8.h and or_config in the oracle
    assert ctypes.sizeof(_native.TlConfig) == 40
    import oracle
    assert ctypes.sizeof(oracle.OrConfig) == 40


def _has_gpu():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.mark.skipif(_has_gpu(), reason="checks the no-device path")
def test_no_cpu_fallback_without_gpu():
    with pytest.raises(_native.TlError) as e:
        _native.Runtime(dict(hidden=512, intermediate=1408, n_layers=1, n_heads=8, n_kv_heads=2,
                             head_dim=64, vocab=64, max_pos=128, rms_eps=1e-5, rope_theta=1e4))
    assert e.value.status == _native.TL_ERR_INTERNAL


def test_bad_geometry_rejected_before_device_use():
    lib = lpta.load_library()
    h = ctypes.c_void_p()
    bad = _native.TlConfig(512, 1408, 1, 8, 2, 128, 64, 128, 1e-5, 1e4)   # head_dim 128
    assert lib.tl_create(ctypes.byref(bad), 1, ctypes.byref(h)) == _native.TL_ERR_UNSUPPORTED
    assert b"head_dim" in lib.tl_last_error(None)
    bad = _native.TlConfig(520, 1408, 1, 8, 2, 64, 64, 128, 1e-5, 1e4)    # hidden != heads * 64
    assert lib.tl_create(ctypes.byref(bad), 1, ctypes.byref(h)) == _native.TL_ERR_BAD_DESCRIPTOR
    bad = _native.TlConfig(1536, 1408, 1, 24, 2, 64, 64, 128, 1e-5, 1e4)  # 24 heads per kv head
    assert lib.tl_create(ctypes.byref(bad), 1, ctypes.byref(h)) == _native.TL_ERR_UNSUPPORTED
    assert not h.value


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setattr(_native, "LIB_PATH", os.path.join(tmp_path, "nope.so"))
    with pytest.raises(RuntimeError, match="missing"):
        _native.load_library()


def test_pairwise_plan_widths():
    # widths the device RMSNorm accepts: halving chain on multiples of 8
    lib = lpta.load_library()
    h = ctypes.c_void_p()
    bad = _native.TlConfig(64 * 3 * 7, 1408, 1, 21, 3, 64, 64, 128, 1e-5, 1e4)  # 1344 -> 672 -> 336 -> 168 -> 84
    assert lib.tl_create(ctypes.byref(bad), 1, ctypes.byref(h)) == _native.TL_ERR_UNSUPPORTED


def test_golden_surface_host_logic(tmp_path):
    """Host-only parts of the reference-surface mirror: token-id parsing and
    its errors (GI:340-375), the layer-count check (GI:356-358) and the weight
    archive reader (TL:198-267 key schema)."""
    import numpy as np
    import lpta.tinyllama as tl
    import lpta.tinyllama_gemm_int8 as gi
    assert gi.parse_token_ids(" 1, 2 ,3,") == [1, 2, 3] and gi.parse_token_ids(None) is None
    with pytest.raises(ValueError, match="Provide either"):
        gi.resolve_token_ids(None, None, None)
    with pytest.raises(ValueError, match="--token-ids is required"):
        gi.resolve_token_ids("hello", None, None)
    with pytest.raises(ValueError, match="empty"):
        gi.resolve_token_ids(None, ",", None)
    with pytest.raises(ValueError, match="between 1 and 22"):
        gi.validate_layer_count({"num_hidden_layers": 22}, 0)
    meta = {"meta_model_id": np.array("m"), "meta_hidden_size": np.array(64), "meta_intermediate_size": np.array(128),
            "meta_num_hidden_layers": np.array(1), "meta_num_attention_heads": np.array(1),
            "meta_num_key_value_heads": np.array(1), "meta_head_dim": np.array(64), "meta_vocab_size": np.array(10),
            "meta_max_position_embeddings": np.array(32), "meta_rms_norm_eps": np.array(1e-5, np.float32),
            "meta_rope_theta": np.array(10000.0, np.float32)}
    arrays = dict(meta, embed_w=np.ones((10, 64), np.float16), layer0_q_w=np.zeros((64, 64), np.float16),
                  layer0_q_b=np.zeros(64, np.float16), layer0_input_norm_w=np.ones(64, np.float16))
    np.savez(tmp_path / "w.npz", **arrays)
    w = tl.load_weights(str(tmp_path / "w.npz"))
    assert w.cfg["num_key_value_groups"] == 1 and w.cfg["hidden_size"] == 64 and w.cfg["model_id"] == "m"
    assert w.embed([1, 3]).shape == (2, 64) and w.embed([1]).dtype == np.float32
    assert w.kv_scales() is None
    assert w._optional_array("layer0_k_b") is None and w._optional_array("layer0_q_b").dtype == np.float32


def test_capture_layout_matches_header(tmp_path):
    # offsets of struct tl_capture as the C compiler lays it out from the header
    fields = [f for f, _ in _native.TlCapture._fields_]
    src = tmp_path / "layout.c"
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "tl_int8.h"\nint main(void) {\n'
                   + "".join(f'    printf("%zu\\n", offsetof(tl_capture, {f}));\n' for f in fields)
                   + '    printf("%zu\\n", sizeof(tl_capture));\n    printf("%d\\n", TL_CAPTURE_TOPK);\n'
                   + "    return 0;\n}\n")
    exe = tmp_path / "layout"
    import subprocess
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(os.path.dirname(_native.HEADER)), "-o", str(exe),
                    str(src)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    want = [getattr(_native.TlCapture, f).offset for f in fields] + [ctypes.sizeof(_native.TlCapture),
                                                                     _native.CAPTURE_TOPK]
    assert got == want


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures the single-GPU hot path: --gpus N > 1 exits non-zero
    with a message saying so, before touching any device."""
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], cwd=root,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)
