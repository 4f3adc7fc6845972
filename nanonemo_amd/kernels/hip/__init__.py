"""ctypes binding of the gfx950 HIP library (libnanonemo_fa.so, C ABI in include/nanonemo_fa.h).

Replaces the reference's ``build(name)`` (/root/reference/nanonemo/kernels/cuda/__init__.py:15-18), which
JIT-compiled a pybind11 torch extension. Here the library is built ahead of time by
``nanonemo_amd.build`` and only loaded: no compiler runs on first use, and no torch type crosses the
boundary (raw device pointers, int64 sizes, a dtype code, the scale and a hipStream_t).

There is no fallback: if the library is missing, :func:`lib` raises, so a GPU run can never silently
use another implementation.
"""

from __future__ import annotations

import ctypes
from functools import cache
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parents[2] / "lib" / "libnanonemo_fa.so"

DTYPE_F16 = 0
DTYPE_BF16 = 1
DTYPE_F32 = 2  # nn_rope_* only

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_int = ctypes.c_int
_f32 = ctypes.c_float
_sz = ctypes.c_size_t
_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); must match include/nanonemo_fa.h, nanonemo_rope.h and nanonemo_rmsnorm.h
SIGNATURES: dict[str, tuple] = {
    "nn_fa_fwd": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _int, _f32, _vp]),
    "nn_fa_fwd_strided": (
        _int,
        [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64p, _i64p, _int, _f32, _vp],
    ),
    "nn_fa_bwd_workspace_size": (_sz, [_i64, _i64, _i64, _i64, _i64]),
    "nn_fa_bwd": (
        _int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _i64, _i64, _i64, _i64, _i64, _int, _f32, _vp],
    ),
    "nn_fa_bwd_strided": (
        _int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _i64, _i64, _i64, _i64, _i64, _i64p, _i64p, _int, _f32,
         _vp],
    ),
    "nn_fa_fwd_rope_strided": (
        _int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64p, _i64p, _int, _f32, _vp],
    ),
    "nn_fa_bwd_rope_strided": (
        _int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64p, _i64p,
         _int, _f32, _vp],
    ),
    "nn_fa_bwd_pre": (_int, [_vp, _vp, _vp, _vp, _sz, _i64, _i64, _i64, _i64, _i64, _int, _f32, _vp]),
    "nn_fa_bwd_dkdv": (_int, [_vp, _vp, _vp, _vp, _vp, _sz, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _int, _f32, _vp]),
    "nn_fa_bwd_dq": (
        _int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp, _i64, _i64, _i64, _i64, _i64, _int, _f32, _vp]
    ),
    "nn_fa_bwd_noalloc": (
        _int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _int, _f32, _vp]
    ),
    "nn_fa_bwd_plan": (
        _int, [_i64, _i64, _i64, _i64, ctypes.POINTER(_int), ctypes.POINTER(_int), ctypes.POINTER(_int), _i64p]
    ),
    "nn_fa_last_error": (ctypes.c_char_p, []),
    "nn_fa_abi_version": (_int, []),
    # include/nanonemo_rope.h
    "nn_rope_qk": (
        _int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64p, _i64p, _i64, _int, _vp],
    ),
    "nn_rope_qk_bwd": (
        _int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64p, _i64p, _i64, _int, _vp],
    ),
    "nn_rope_last_error": (ctypes.c_char_p, []),
    # include/nanonemo_rmsnorm.h
    "nn_add_rmsnorm_fwd": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _f32, _int, _int, _int, _vp]),
    "nn_add_rmsnorm_bwd_workspace_size": (_sz, [_i64, _i64]),
    "nn_add_rmsnorm_bwd": (
        _int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _i64, _i64, _int, _int, _int, _int, _vp]
    ),
    "nn_rmsnorm_last_error": (ctypes.c_char_p, []),
}

ABI_VERSION = 10


@cache
def lib() -> ctypes.CDLL:
    """Load libnanonemo_fa.so once per process and declare every entry point's C signature."""
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"HIP library {LIB_PATH} is not built; run `python -m nanonemo_amd.build` "
            "(or __graft_entry__.build()) first. There is no non-HIP fallback."
        )
    handle = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    if handle.nn_fa_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{LIB_PATH} has ABI {handle.nn_fa_abi_version()}, expected {ABI_VERSION}; rebuild it")
    return handle


def eager(*ts) -> bool:
    """Whether a public function may run its eager path: a plain autograd.Function around the library call instead
    of its torch.library op. The ops' dispatch (the dispatcher's Python kernel, the autograd.Function that
    register_autograd generates, and a second op's dispatch in the backward) costs several tens of microseconds of
    host time per forward + backward; the eager paths call the same launch code, so their results are the same
    bits. True only for plain CUDA tensors outside torch.compile tracing, torch.func transforms and dispatch modes,
    which need the ops (an opaque traced node, a transform rule, the op visible to the mode); meta and CPU tensors
    take the ops too, whose fake impls and checks handle them."""
    import torch

    if torch.compiler.is_compiling():
        return False
    for t in ts:
        if type(t) is not torch.Tensor or not t.is_cuda:
            return False
    # Both queries are PyTorch internals; where this PyTorch lacks one, the ops take every call.
    transforms = getattr(getattr(torch._C, "_functorch", None), "peek_interpreter_stack", None)
    modes = getattr(torch._C, "_len_torch_dispatch_stack", None)
    if transforms is None or modes is None:
        return False
    return transforms() is None and not modes()


def stream_of(t) -> int:
    """PyTorch's current HIP stream on t's device, as the hipStream_t the library takes (the handle alone, without
    building a torch.cuda.Stream object where this PyTorch offers that)."""
    import torch

    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is not None:
        return raw(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


def on_device(t):
    """A context that makes t's device current for a launch (a no-op when it already is)."""
    import contextlib

    import torch

    return contextlib.nullcontext() if t.device.index == torch.cuda.current_device() else torch.cuda.device(t.device)


def records(*ts) -> bool:
    """Whether autograd records a call on these inputs (grad mode on and one of them requires grad)."""
    import torch

    return torch.is_grad_enabled() and any(t.requires_grad for t in ts)


def strides3(b: int, h: int, t: int) -> ctypes.Array:
    """An int64[3] {batch, head, row} element-stride array for the *_strided entry points."""
    return (ctypes.c_int64 * 3)(b, h, t)


def check(rc: int) -> None:
    """Raise RuntimeError with the library's message when an nn_fa_* entry point returns non-zero."""
    if rc != 0:
        msg = lib().nn_fa_last_error().decode(errors="replace")
        raise RuntimeError(msg or f"nanonemo_fa call failed with code {rc}")


def check_rope(rc: int) -> None:
    """Raise RuntimeError with the library's message when an nn_rope_* entry point returns non-zero."""
    if rc != 0:
        msg = lib().nn_rope_last_error().decode(errors="replace")
        raise RuntimeError(msg or f"nanonemo_rope call failed with code {rc}")


def check_rmsnorm(rc: int) -> None:
    """Raise RuntimeError with the library's message when an nn_add_rmsnorm_* entry point returns non-zero."""
    if rc != 0:
        msg = lib().nn_rmsnorm_last_error().decode(errors="replace")
        raise RuntimeError(msg or f"nanonemo_rmsnorm call failed with code {rc}")
