"""tl_gemm_i8_noalloc (the entry point that allocates nothing: its split-K
scratch is a fixed per-GPU device array) against tl_gemm_i8 through the
C-ABI, INT32 accumulators bit for bit, on two calls in a row with the second
smaller, and against the oracle's integer GEMM.  The second and third calls
leave the device's free memory unchanged."""
import numpy as np
import pytest

import oracle
from gpu_util import assert_bits_equal, dev, empty, host, runtime

pytestmark = pytest.mark.gpu


def _operands(rng, m, n, k):
    a = rng.integers(-127, 128, (m, k)).astype(np.int8)
    w = rng.integers(-127, 128, (n, k)).astype(np.int8)
    return a, w


@pytest.mark.parametrize("shapes", [
    ((32, 2048, 5632), (7, 1000, 4096)),     # split-K small-M path (scratch used), then a smaller one
    ((24, 256, 6144), (1, 64, 2112)),        # few tiles: the most K slices
    ((96, 512, 2048), (40, 96, 128)),        # paths without scratch (MFMA tiles, 33..63 rows)
], ids=["split_k", "few_tiles", "no_scratch_paths"])
def test_noalloc_gemm_equals_gemm(shapes):
    import torch
    rt = runtime()
    rng = np.random.default_rng(sum(sum(s) for s in shapes))
    for call, (m, n, k) in enumerate(shapes):
        a, w = _operands(rng, m, n, k)
        da, dw = dev(a), dev(w)
        want = empty((m, n), np.int32)
        got = empty((m, n), np.int32)
        got.fill_(-1)
        rt.call("tl_gemm_i8", da, dw, m, n, k, want)
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        rt.call("tl_gemm_i8_noalloc", da, dw, m, n, k, got)
        rt.call("tl_gemm_i8_noalloc", da, dw, m, n, k, got)
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info()[0] == free0, f"call {call}: device memory changed"
        assert_bits_equal(host(got), host(want), f"call {call} {m}x{n}x{k}")
        if m * n * k <= 32 * 2048 * 5632:
            assert_bits_equal(host(got), oracle.gemm_i8(a, w), f"call {call} vs oracle")
    rt.close()
