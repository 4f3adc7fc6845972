"""Ahead-of-time build of the HIP library for gfx950.

Replaces the reference's JIT build (/root/reference/nanonemo/kernels/cuda/__init__.py:15-18, which runs
nvcc through torch.utils.cpp_extension.load on first use): here ``hipcc`` compiles
``nanonemo_amd/csrc/*.hip`` once, in-tree, into ``nanonemo_amd/lib/libnanonemo_fa.so``, a plain C-ABI
shared library with no torch types in its signatures (include/nanonemo_fa.h, include/nanonemo_rope.h, include/nanonemo_rmsnorm.h). The library is loaded
with ctypes (nanonemo_amd/kernels/hip/__init__.py), so the same .so runs on any box with the ROCm
runtime.

    python -m nanonemo_amd.build
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
SRCS = [PKG / "csrc" / "flash_attn.hip", PKG / "csrc" / "rope.hip", PKG / "csrc" / "rmsnorm.hip"]
LIB_DIR = PKG / "lib"
LIB = LIB_DIR / "libnanonemo_fa.so"
# Block timelines for `bench.py --timeline`: the attention kernels built with NN_TIMELINE=1, so that every block
# records clock stamps at its phase boundaries (the product library compiles those stamps to nothing).
TIMELINE_SRCS = [PKG / "csrc" / "flash_attn.hip"]
TIMELINE_LIB = LIB_DIR / "libnanonemo_fa_timeline.so"
ARCH = "gfx950"

# -packed-fp32-ops: keep v_pk_{add,mul,fma}_f32 out of the generated code (those packed forms have
# produced intermittent wrong results on the target boxes). hipcc's host pass warns that it does not
# know the feature; that warning is harmless.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-shared",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # Device code never relies on NaN semantics (masked scores are -inf, never NaN); without this
    # every fmaxf of an MFMA result is preceded by a canonicalising v_max_f32 x, x.
    "-Xarch_device",
    "-fno-honor-nans",
    # Select MFMAs in their VGPR form and let register allocation move accumulators to AGPRs where it
    # must: the dK / dV kernel then keeps dK^T / dV^T in AGPRs while S and dP stay in VGPRs, where
    # the softmax reads them, instead of copying every S / dP element out of an AGPR (2-3 % faster;
    # no other kernel's code changes).
    "-mllvm",
    "-amdgpu-mfma-vgpr-form=1",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (looked at $HIPCC, /opt/rocm/bin/hipcc and PATH)")


def _start(srcs: list[Path], lib: Path, verbose: bool, defines: tuple[str, ...] = ()):
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    tmp = lib.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, *defines, f"-I{ROOT / 'include'}", "-o", str(tmp), *(str(s) for s in srcs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True), tmp, lib


def _finish(job, verbose: bool) -> Path:
    proc, tmp, lib = job
    out, _ = proc.communicate()
    noise = "'-packed-fp32-ops' is not a recognized feature"
    log = "\n".join(l for l in out.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {lib.name} ({proc.returncode}):\n{log}")
    if verbose and log.strip():
        print(log, flush=True)
    os.replace(tmp, lib)  # atomic: a process that already mapped the old file keeps it
    return lib


def build(verbose: bool = False) -> Path:
    """Compile the HIP library and the timeline build of the attention kernels, in parallel (always
    recompiles); return the library's path."""
    jobs = [_start(SRCS, LIB, verbose), _start(TIMELINE_SRCS, TIMELINE_LIB, verbose, ("-DNN_TIMELINE=1",))]
    errors = []
    for job in jobs:
        try:
            _finish(job, verbose)
        except RuntimeError as e:
            errors.append(str(e))
    if errors:
        raise RuntimeError("\n".join(errors))
    return LIB


if __name__ == "__main__":
    print(build(verbose="-q" not in sys.argv))
