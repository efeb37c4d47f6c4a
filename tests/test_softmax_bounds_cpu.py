"""The attention kernels quantize probabilities as rne(127 RN(e / total))
without clipping to [0, 127], because a float32 sum of nonnegative terms is
never below any of its terms, whatever the order (each partial sum is a
rounding of a value at least as large as every term in it, and rounding is
monotonic), so e <= total and RN(e / total) <= 1.  Checked in float32 numpy
arithmetic for sums in sequential, pairwise (block butterfly) and shuffled
orders, on random, equal, tiny and one-dominant exponentials."""
import numpy as np

F32 = np.float32


def sum_sequential(v):
    s = F32(0)
    for x in v:
        s = F32(s + x)
    return s


def sum_pairwise(v):
    v = list(v)
    while len(v) > 1:
        if len(v) % 2:
            v.append(F32(0))
        v = [F32(v[i] + v[i + 1]) for i in range(0, len(v), 2)]
    return v[0]


def probability_bytes_unclipped(e, total):
    q = (e / total).astype(F32)                       # RN(e / total)
    return np.rint((q * F32(127)).astype(F32))        # rne(RN(127 q))


def test_probability_needs_no_clip():
    rng = np.random.default_rng(2027)
    cases = []
    for n in (1, 2, 3, 63, 64, 65, 256, 1000):
        cases.append(rng.random(n).astype(F32))
        cases.append(np.exp(-rng.random(n).astype(F32) * F32(100)).astype(F32))
        cases.append(np.full(n, F32(1)))
        cases.append(np.full(n, F32(np.nextafter(F32(1), F32(0)))))
        tiny = np.full(n, F32(1e-38))
        tiny[0] = F32(1)
        cases.append(tiny)
        cases.append(np.concatenate([[F32(1)], np.zeros(n - 1, F32)]).astype(F32))
    for e in cases:
        for order in ("sequential", "pairwise", "shuffled"):
            if order == "shuffled":
                total = sum_sequential(rng.permutation(e))
            elif order == "pairwise":
                total = sum_pairwise(e)
            else:
                total = sum_sequential(e)
            assert np.all(e <= total), order
            p = probability_bytes_unclipped(e, total)
            assert p.min() >= 0 and p.max() <= 127, order
