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


def test_noalloc_two_handles_concurrently():
    """Two handles on one GPU calling tl_gemm_i8_noalloc from two host threads
    at once (ctypes releases the GIL during the call): the calls share the
    GPU's one scratch array and are put in order, so every result equals
    tl_gemm_i8's."""
    import threading
    import torch
    rts = [runtime(), runtime()]
    shapes = [(32, 2048, 5632), (24, 256, 6144)]   # both use the split-K scratch
    rng = np.random.default_rng(71)
    ops = []
    for (m, n, k) in shapes:
        a, w = _operands(rng, m, n, k)
        want = empty((m, n), np.int32)
        rts[0].call("tl_gemm_i8", dev(a), dev(w), m, n, k, want)
        ops.append((dev(a), dev(w), m, n, k, want))
    torch.cuda.synchronize()
    errors = []

    def worker(i):
        da, dw, m, n, k, want = ops[i]
        got = empty((m, n), np.int32)
        try:
            for it in range(40):
                got.fill_(-1)
                torch.cuda.synchronize()
                rts[i].call("tl_gemm_i8_noalloc", da, dw, m, n, k, got)
                if not torch.equal(got, want):
                    errors.append(f"handle {i} call {it}")
                    return
        except Exception as e:   # noqa: BLE001 -- reported below
            errors.append(f"handle {i}: {e}")

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    for rt in rts:
        rt.close()
    assert errors == []
