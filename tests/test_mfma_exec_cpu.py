"""MFMA instructions ignore EXEC: an MFMA issued while the EXEC mask is
narrowed (inside a lane-divergent branch) still multiplies and writes its whole
accumulator, and the compiler drops the s_cbranch_execz that would skip a
short masked block.  A guard such as ``if (wave * per + j < kch)`` with
``wave = threadIdx.x >> 6`` therefore does not stop the MFMA: it adds a
product that should have been skipped.  That made one build of the batched
decode's K-sliced GEMM add extra K chunks (a wrong greedy token).

These CPU tests compile every HIP source of the library to gfx950 assembly
with the library's own flags and check that no MFMA is issued after an EXEC
narrowing with no execz skip in between.  Every kernel's MFMA guards are
built from wave_id() (a scalar, wavefront-uniform value) and kernel
arguments, so they compile to scalar branches.
"""
from __future__ import annotations

import importlib.util
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "low-precision-transformer-accelerator-for-edge-llms_amd")
CSRC = os.path.join(PKG, "csrc")


def _build_module():
    spec = importlib.util.spec_from_file_location("_lpta_build_flags", os.path.join(PKG, "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _hipcc():
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    return None


def exposed_mfmas(asm: str) -> list[tuple[str, int]]:
    """(kernel, line) of every MFMA issued after an instruction that narrows
    EXEC (v_cmpx*, s_*saveexec*, or a write to exec other than a restoring
    s_or_b64 / s_mov_b64) with no s_cbranch_execz since that write."""
    hits = []
    fn, masked, skipped = "?", False, False
    for ln, line in enumerate(asm.splitlines(), 1):
        t = line.strip()
        m = re.match(r"^(_Z\w+):", t)
        if m:
            fn, masked, skipped = m.group(1), False, False
            continue
        if not t or t.startswith(";") or t.startswith("."):
            continue
        parts = t.split(None, 1)
        op, args = parts[0], (parts[1] if len(parts) > 1 else "")
        dst = args.split(",")[0].strip()
        if op.startswith("v_cmpx") or op.endswith("saveexec_b64") or op.endswith("saveexec_b32") or (
                dst == "exec" and not op.startswith(("s_or_b64", "s_mov_b64"))):
            masked, skipped = True, False
        elif dst == "exec":
            masked, skipped = False, False
        if op == "s_cbranch_execz":
            skipped = True
        if "mfma" in op and masked and not skipped:
            hits.append((fn, ln))
    return hits


def _asm(src: str, workdir: str, extra_inc: list[str] | None = None) -> str:
    b = _build_module()
    out = os.path.join(workdir, os.path.basename(src) + ".s")
    inc = ["-I", os.path.join(ROOT, "include"), "-I", CSRC] + (extra_inc or [])
    cmd = [_hipcc(), *b.HIPCC_FLAGS, *inc, "--cuda-device-only", "-S", "-o", out, src]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout[-2000:]
    with open(out) as f:
        return f.read()


pytestmark = pytest.mark.skipif(_hipcc() is None, reason="hipcc is needed to compile the kernels")

PLANTED = r"""
#include <hip/hip_runtime.h>
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
// the guard is lane-divergent to the compiler: the MFMA lands under an EXEC
// mask with no skip
__global__ __launch_bounds__(64) void planted(const v4i* a, const v4i* b, int n, int* out, int* pre) {
    const int lane = threadIdx.x;
    const v4i x = a[lane], y = b[lane];
    pre[lane] = x[0] + y[0];
    v16i acc = {};
    if (lane >= n) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(x, y, acc, 0, 0, 0);
    for (int i = 0; i < 16; i++) out[lane * 16 + i] = acc[i];
}
// the same guard on a wavefront-uniform value: a scalar branch
__global__ __launch_bounds__(64) void uniform(const v4i* a, const v4i* b, int n, int* out, int* pre) {
    const int lane = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const v4i x = a[lane], y = b[lane];
    pre[lane] = x[0] + y[0];
    v16i acc = {};
    if (w >= n) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(x, y, acc, 0, 0, 0);
    for (int i = 0; i < 16; i++) out[lane * 16 + i] = acc[i];
}
"""


def test_scanner_finds_a_planted_masked_mfma():
    """The checker sees the pattern: a lane-divergent guard leaves the MFMA
    under EXEC with no skip; the same guard on a uniform value does not."""
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "planted.hip")
        with open(src, "w") as f:
            f.write(PLANTED)
        hits = exposed_mfmas(_asm(src, d))
    kernels = {k for k, _ in hits}
    assert any("planted" in k for k in kernels), hits
    assert not any("uniform" in k for k in kernels), hits


@pytest.mark.parametrize("src", ["tl_kernels.hip", "tl_gemm.hip", "tl_decode.hip", "tl_float.hip"])
def test_no_mfma_runs_under_a_narrowed_exec(src):
    with tempfile.TemporaryDirectory() as d:
        hits = exposed_mfmas(_asm(os.path.join(CSRC, src), d))
    assert hits == [], f"MFMAs under a narrowed EXEC with no skip in {src}: {hits[:10]}"
