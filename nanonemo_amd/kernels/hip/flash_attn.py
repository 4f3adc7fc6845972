"""torch.library boundary of the gfx950 causal GQA FlashAttention-2 kernels.

Drop-in for /root/reference/nanonemo/kernels/cuda/flash_attn.py: the same op names and schemas
(``nanonemo::flash_attn`` :18-22 and ``nanonemo::flash_attn_bwd`` :31-35), the same fake impls
(contiguous outputs, :25-28 and :38-40), the same autograd wiring (save q, k, v, o, lse; ignore the
gradient of lse, :43-54) and the same public ``flash_attn(q, k, v) -> o`` (:57-60). Under
``torch.compile(fullgraph=True)`` each op is one opaque node traced through its fake impl.

Differences from the reference, all widening: fp16 **and** bf16 inputs (the reference accepts fp16
only, flash_attn.cu:344-346), and the compute is the HIP library behind a C ABI
(include/nanonemo_fa.h) called through ctypes on PyTorch's current HIP stream. Every output and the
backward workspace is allocated here by PyTorch's caching allocator; the library never allocates,
synchronises or copies to the host, so both ops can be captured into a HIP graph. In eager mode the public
functions reach the same launches through a plain autograd.Function instead of the ops' dispatch, which
halves their host time (see "the eager path" below).
"""

from __future__ import annotations

import ctypes
import math

import torch
from torch import Tensor
from torch.autograd.function import once_differentiable

from nanonemo_amd.kernels.hip import DTYPE_BF16, DTYPE_F16, check, lib, strides3
from nanonemo_amd.kernels.hip import eager as _eager
from nanonemo_amd.kernels.hip import on_device as _on
from nanonemo_amd.kernels.hip import records as _records
from nanonemo_amd.kernels.hip import stream_of as _stream

_DTYPES = {torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}


def _check_inputs(q: Tensor, k: Tensor, v: Tensor, seq_dim: int = 2) -> None:
    """The reference's check_inputs (flash_attn.cu:342-356) with the dtype set widened to {fp16, bf16}.

    ``seq_dim`` is 2 for the reference's (B, heads, T, hd) tensors and 1 for the (B, T, heads, hd)
    tensors of the layout-fused ops; the head dimension is the other one of dims 1 and 2."""
    head_dim_idx = 3 - seq_dim
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise RuntimeError("inputs must be CUDA tensors")
    if q.dtype not in _DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise RuntimeError("inputs must be float16 or bfloat16 (all the same dtype)")
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise RuntimeError("expected (B, H, T, hd) / (B, KVH, T, hd)")
    if not (q.is_contiguous() and k.is_contiguous() and v.is_contiguous()):
        raise RuntimeError("inputs must be contiguous")
    if q.size(0) != k.size(0) or q.size(seq_dim) != k.size(seq_dim) or k.shape != v.shape:
        raise RuntimeError("K and V must share shape; Q must share batch and length")
    if q.size(3) != k.size(3):
        raise RuntimeError("Q and K must share head_dim")
    if q.size(3) not in (32, 64):
        raise RuntimeError("head_dim must be 32 or 64")
    if k.size(head_dim_idx) == 0 or q.size(head_dim_idx) % k.size(head_dim_idx) != 0:
        raise RuntimeError("query heads must group evenly over KV heads")
    if q.device != k.device or q.device != v.device:
        raise RuntimeError("inputs must be on the same device")
    for t in (q, k, v):
        if t.numel() and t.data_ptr() % 16 != 0:
            raise RuntimeError("inputs must be 16-byte aligned")


def _contig(t: Tensor) -> Tensor:
    return t if t.is_contiguous() else t.contiguous()


_CAPTURE_MSG = (
    "{}: capturing this op into a HIP graph while autograd records it (torch.cuda.graph around the forward and its "
    "autograd backward, or torch.compile(mode='reduce-overhead')) is not supported: such a capture once ended in a "
    "host fault in capture_end and no cause has been shown. Capture the C ABI calls (nn_fa_fwd / nn_fa_bwd / "
    "nn_fa_bwd_noalloc) instead, or run the ops eagerly (torch.compile(fullgraph=True) without graphs is supported)."
)


def _refuse_capture_with_autograd(where: str, *inputs: Tensor) -> None:
    """Raise when the current stream is capturing and autograd will record this op: before any launch in the
    public functions (grad mode on and an input requires grad), and in setup_context / the backward as a
    backstop for direct op calls. Capture without autograd, and capture of the C ABI, are unaffected. Skipped
    while torch.compile traces (the check is a host query, and no capture runs at trace time)."""
    # A capture needs PyTorch's initialised HIP state: is_initialized is a flag read, where the capture query is a
    # runtime call, and this runs on every op call.
    if not torch.cuda.is_initialized():
        return
    if inputs and not (torch.is_grad_enabled() and any(t.requires_grad for t in inputs)):
        return
    if torch.compiler.is_compiling() or not torch.cuda.is_current_stream_capturing():
        return
    raise RuntimeError(_CAPTURE_MSG.format(where))


def _refuse_capture_from_autograd_engine(where: str) -> None:
    """In the backward ops' bodies: raise when the autograd engine runs them (directly, or inside a compiled
    backward such as torch.compile's mode='reduce-overhead' records) while the current stream is capturing."""
    if torch._C._current_autograd_node() is not None:
        _refuse_capture_with_autograd(where)


def _launch_fwd(q: Tensor, k: Tensor, v: Tensor) -> tuple[Tensor, Tensor]:
    """Allocates (o, lse) and launches the forward on contiguous, checked inputs."""
    B, H, T, D = q.shape
    o = torch.empty_like(q)
    lse = torch.empty((B, H, T), dtype=torch.float32, device=q.device)
    if B == 0 or T == 0 or H == 0:
        return o, lse
    with _on(q):
        rc = lib().nn_fa_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
            B, H, k.size(1), T, D, _DTYPES[q.dtype], 1.0 / math.sqrt(D), _stream(q),
        )
    check(rc)
    return o, lse


def _prep(q: Tensor, k: Tensor, v: Tensor, seq_dim: int = 2) -> tuple[Tensor, Tensor, Tensor]:
    """Contiguous copies where needed, then the checks: the forward's inputs as the launch takes them."""
    q, k, v = _contig(q), _contig(k), _contig(v)
    _check_inputs(q, k, v, seq_dim)
    return q, k, v


def _fwd(q: Tensor, k: Tensor, v: Tensor) -> tuple[Tensor, Tensor]:
    """The forward on any strides: (o, lse)."""
    return _launch_fwd(*_prep(q, k, v))


@torch.library.custom_op("nanonemo::flash_attn", mutates_args=())
def _flash_attn(q: Tensor, k: Tensor, v: Tensor) -> tuple[Tensor, Tensor]:
    return _fwd(q, k, v)


@_flash_attn.register_fake
def _(q, k, v):
    B, H, T, _ = q.shape  # the kernel returns contiguous tensors whatever the input strides
    return (
        torch.empty(q.shape, dtype=q.dtype, device=q.device),
        torch.empty((B, H, T), dtype=torch.float32, device=q.device),
    )


def _launch_bwd(d_o: Tensor, q: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """Allocates (dq, dk, dv) and the workspace and launches the backward on contiguous, checked inputs."""
    B, H, T, D = q.shape
    KVH = k.size(1)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    if B == 0 or T == 0 or H == 0:
        return dq, dk, dv
    L = lib()
    ws_bytes = L.nn_fa_bwd_workspace_size(B, H, KVH, T, D)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    with _on(q):
        rc = L.nn_fa_bwd(
            d_o.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
            dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws_bytes,
            B, H, KVH, T, D, _DTYPES[q.dtype], 1.0 / math.sqrt(D), _stream(q),
        )
    check(rc)
    return dq, dk, dv


@torch.library.custom_op("nanonemo::flash_attn_bwd", mutates_args=())
def _flash_attn_bwd(d_o: Tensor, q: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    _refuse_capture_from_autograd_engine("flash_attn backward op")
    d_o, q, k, v, o, lse = (_contig(t) for t in (d_o, q, k, v, o, lse))
    _check_inputs(q, k, v)
    if d_o.shape != q.shape or d_o.dtype != q.dtype or o.shape != q.shape or o.dtype != q.dtype:
        raise RuntimeError("d_o must be a contiguous float16/bfloat16 tensor shaped like q")
    B, H, T, D = q.shape
    if lse.shape != (B, H, T) or lse.dtype != torch.float32:
        raise RuntimeError("lse must be a float32 tensor of shape (B, H, T)")
    return _launch_bwd(d_o, q, k, v, o, lse)


@_flash_attn_bwd.register_fake
def _(d_o, q, k, v, o, lse):
    return tuple(torch.empty(t.shape, dtype=t.dtype, device=t.device) for t in (q, k, v))


def _setup_context(ctx, inputs, output):
    _refuse_capture_with_autograd("flash_attn (autograd)")
    q, k, v = inputs
    o, lse = output
    ctx.save_for_backward(q, k, v, o, lse)
    # lse's gradient is ignored, so autograd need not fill a zero tensor for it on every backward.
    ctx.set_materialize_grads(False)


def _d_out(d_o, o):
    """The gradient reaching o; zeros when o itself was not used (only lse was), as a materialised grad would be."""
    return torch.zeros_like(o) if d_o is None else d_o


def _backward(ctx, d_o, _d_lse):
    _refuse_capture_with_autograd("flash_attn backward")
    q, k, v, o, lse = ctx.saved_tensors
    return _flash_attn_bwd(_d_out(d_o, o), q, k, v, o, lse)


_flash_attn.register_autograd(_backward, setup_context=_setup_context)


# ---- the eager path of the public functions ----------------------------------------------------
# The custom ops are what torch.compile traces (one opaque node each, through their fake impls) and what callers
# of torch.ops.nanonemo.* reach. Run eagerly under autograd, an op pays for the dispatcher's Python kernel, the
# autograd.Function that register_autograd generates and, in the backward, a second op's dispatch and checks: tens
# of microseconds of host time per forward + backward, which at the model's shape is about the GPU time of the
# three kernels. The public functions therefore run plain CUDA tensors in eager mode through the
# autograd.Functions below (``eager``): the same checks and launches in the forward, and in the backward the
# launch alone, on the contiguous inputs the forward checked and saved (the gradient autograd hands over has o's
# shape and dtype). Outputs and gradients are the same bits as the ops'. Everything else (torch.compile tracing,
# torch.func transforms, dispatch modes, tensor subclasses, meta and CPU tensors) goes through the custom ops.


class _FlashAttnFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v):
        q, k, v = _prep(q, k, v)
        o, lse = _launch_fwd(q, k, v)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.set_materialize_grads(False)
        return o

    @staticmethod
    @once_differentiable
    def backward(ctx, d_o):
        _refuse_capture_with_autograd("flash_attn backward")
        q, k, v, o, lse = ctx.saved_tensors
        return _launch_bwd(_contig(_d_out(d_o, o)), q, k, v, o, lse)


def flash_attn(q: Tensor, k: Tensor, v: Tensor) -> Tensor:
    """Causal GQA attention. q: (B, H, T, hd), k/v: (B, KVH, T, hd), fp16 or bf16, H % KVH == 0, hd in {32, 64}."""
    _refuse_capture_with_autograd("flash_attn", q, k, v)
    if _eager(q, k, v):
        return _FlashAttnFn.apply(q, k, v) if _records(q, k, v) else _fwd(q, k, v)[0]
    o, _ = _flash_attn(q, k, v)
    return o


# ---- layout-fused ops: (B, T, heads, hd) in and out -------------------------------------------
# The reference model projects x to (B, T, heads * hd), views it as (B, T, heads, hd), transposes to
# (B, heads, T, hd) for the op (which then copies each input to contiguous memory,
# /root/reference/nanonemo/kernels/cuda/flash_attn.py:20,33) and transposes + reshapes o back for
# the output projection (/root/reference/nanonemo/model/layers.py:97-104,116), one more copy per
# direction. These ops take and return the projection layout itself through the library's strided
# entry points: q (B, T, H, hd), k / v (B, T, KVH, hd), o / dq (B, T, H, hd), dk / dv (B, T, KVH, hd),
# all contiguous in that layout (so o.view(B, T, H * hd) feeds the output projection directly);
# lse stays (B, H, T). Not in the reference: an addition that the same model code can select.


def _bthd_strides(t: Tensor) -> ctypes.Array:
    B, T, Hh, D = t.shape
    return strides3(T * Hh * D, D, Hh * D)


def _launch_fwd_bthd(q: Tensor, k: Tensor, v: Tensor) -> tuple[Tensor, Tensor]:
    """Allocates (o, lse) and launches the projection-layout forward on contiguous, checked inputs."""
    B, T, H, D = q.shape
    o = torch.empty_like(q)
    lse = torch.empty((B, H, T), dtype=torch.float32, device=q.device)
    if B == 0 or T == 0 or H == 0:
        return o, lse
    with _on(q):
        rc = lib().nn_fa_fwd_strided(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
            B, H, k.size(2), T, D, _bthd_strides(q), _bthd_strides(k), _DTYPES[q.dtype], 1.0 / math.sqrt(D),
            _stream(q),
        )
    check(rc)
    return o, lse


@torch.library.custom_op("nanonemo::flash_attn_bthd", mutates_args=())
def _flash_attn_bthd(q: Tensor, k: Tensor, v: Tensor) -> tuple[Tensor, Tensor]:
    return _launch_fwd_bthd(*_prep(q, k, v, seq_dim=1))


@_flash_attn_bthd.register_fake
def _(q, k, v):
    B, T, H, _ = q.shape
    return (
        torch.empty(q.shape, dtype=q.dtype, device=q.device),
        torch.empty((B, H, T), dtype=torch.float32, device=q.device),
    )


def _launch_bwd_bthd(d_o: Tensor, q: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """Allocates (dq, dk, dv) and the workspace and launches the projection-layout backward on contiguous, checked
    inputs."""
    B, T, H, D = q.shape
    KVH = k.size(2)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    if B == 0 or T == 0 or H == 0:
        return dq, dk, dv
    L = lib()
    ws_bytes = L.nn_fa_bwd_workspace_size(B, H, KVH, T, D)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    with _on(q):
        rc = L.nn_fa_bwd_strided(
            d_o.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
            dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws_bytes,
            B, H, KVH, T, D, _bthd_strides(q), _bthd_strides(k), _DTYPES[q.dtype], 1.0 / math.sqrt(D), _stream(q),
        )
    check(rc)
    return dq, dk, dv


@torch.library.custom_op("nanonemo::flash_attn_bthd_bwd", mutates_args=())
def _flash_attn_bthd_bwd(
    d_o: Tensor, q: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor
) -> tuple[Tensor, Tensor, Tensor]:
    _refuse_capture_from_autograd_engine("flash_attn_bthd backward op")
    d_o, q, k, v, o, lse = (_contig(t) for t in (d_o, q, k, v, o, lse))
    _check_inputs(q, k, v, seq_dim=1)
    if d_o.shape != q.shape or d_o.dtype != q.dtype or o.shape != q.shape or o.dtype != q.dtype:
        raise RuntimeError("d_o must be a contiguous float16/bfloat16 tensor shaped like q")
    B, T, H, D = q.shape
    if lse.shape != (B, H, T) or lse.dtype != torch.float32:
        raise RuntimeError("lse must be a float32 tensor of shape (B, H, T)")
    return _launch_bwd_bthd(d_o, q, k, v, o, lse)


@_flash_attn_bthd_bwd.register_fake
def _(d_o, q, k, v, o, lse):
    return tuple(torch.empty(t.shape, dtype=t.dtype, device=t.device) for t in (q, k, v))


def _backward_bthd(ctx, d_o, _d_lse):
    _refuse_capture_with_autograd("flash_attn_bthd backward")
    q, k, v, o, lse = ctx.saved_tensors
    return _flash_attn_bthd_bwd(_d_out(d_o, o), q, k, v, o, lse)


_flash_attn_bthd.register_autograd(_backward_bthd, setup_context=_setup_context)


class _FlashAttnBthdFn(torch.autograd.Function):
    """The eager path of flash_attn_bthd (see flash_attn's)."""

    @staticmethod
    def forward(ctx, q, k, v):
        q, k, v = _prep(q, k, v, seq_dim=1)
        o, lse = _launch_fwd_bthd(q, k, v)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.set_materialize_grads(False)
        return o

    @staticmethod
    @once_differentiable
    def backward(ctx, d_o):
        _refuse_capture_with_autograd("flash_attn_bthd backward")
        q, k, v, o, lse = ctx.saved_tensors
        return _launch_bwd_bthd(_contig(_d_out(d_o, o)), q, k, v, o, lse)


def flash_attn_bthd(q: Tensor, k: Tensor, v: Tensor) -> Tensor:
    """Causal GQA attention in the projection layout: q (B, T, H, hd), k/v (B, T, KVH, hd) -> o (B, T, H, hd)."""
    _refuse_capture_with_autograd("flash_attn_bthd", q, k, v)
    if _eager(q, k, v):
        if _records(q, k, v):
            return _FlashAttnBthdFn.apply(q, k, v)
        return _launch_fwd_bthd(*_prep(q, k, v, seq_dim=1))[0]
    o, _ = _flash_attn_bthd(q, k, v)
    return o


# ---- RoPE of q folded into the layout-fused ops ------------------------------------------------
# The reference rotates q and k beside the op (/root/reference/nanonemo/model/layers.py:99-101) and the op
# then reads the rotated tensors. Here the forward takes q *before* RoPE, rotates each query row in registers
# (the same fp32 operation order as nanonemo::rope_qk, so the result is bit-identical) and also returns the
# rotated q, which the backward reads; the backward's dQ kernel rotates its gradient back by -theta before
# storing it, so dq is the gradient of the unrotated q. k is rotated beforehand (rope_k). Not in the reference:
# an addition the same model code can select (rope_kernel="fused"). The gradients of lse and of the rotated q
# output are not propagated (the model uses neither), as the reference ignores lse's.


def _check_tables(cos: Tensor, sin: Tensor, T: int, D: int, device: torch.device) -> tuple[Tensor, Tensor]:
    """The RoPE tables: float32 (T_max >= T, hd/2), on the inputs' GPU. Checked before any launch, since the
    library reads them through raw device pointers (a host table would be read as device memory)."""
    if not (cos.is_cuda and sin.is_cuda) or cos.device != device or sin.device != device:
        raise RuntimeError("cos/sin must be float32 (T_max >= T, hd/2) tables on the inputs' device")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32 or cos.shape != sin.shape or cos.dim() != 2 \
            or cos.shape[1] != D // 2 or cos.shape[0] < T:
        raise RuntimeError("cos/sin must be float32 (T_max >= T, hd/2) tables on the inputs' device")
    return _contig(cos), _contig(sin)


def _prep_rope(q: Tensor, k: Tensor, v: Tensor, cos: Tensor, sin: Tensor) -> tuple[Tensor, ...]:
    """Contiguous copies where needed and the checks of the RoPE-fused forward's inputs."""
    q, k, v = _prep(q, k, v, seq_dim=1)
    cos, sin = _check_tables(cos, sin, q.size(1), q.size(3), q.device)
    return q, k, v, cos, sin


def _launch_fwd_rope(q: Tensor, k: Tensor, v: Tensor, cos: Tensor, sin: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """Allocates (o, lse, q_rot) and launches the RoPE-fused forward on contiguous, checked inputs."""
    B, T, H, D = q.shape
    o, q_rot = torch.empty_like(q), torch.empty_like(q)
    lse = torch.empty((B, H, T), dtype=torch.float32, device=q.device)
    if B == 0 or T == 0 or H == 0:
        return o, lse, q_rot
    with _on(q):
        rc = lib().nn_fa_fwd_rope_strided(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), q_rot.data_ptr(),
            cos.data_ptr(), sin.data_ptr(), cos.shape[0], B, H, k.size(2), T, D, _bthd_strides(q), _bthd_strides(k),
            _DTYPES[q.dtype], 1.0 / math.sqrt(D), _stream(q),
        )
    check(rc)
    return o, lse, q_rot


@torch.library.custom_op("nanonemo::flash_attn_bthd_rope", mutates_args=())
def _flash_attn_bthd_rope(q: Tensor, k: Tensor, v: Tensor, cos: Tensor, sin: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    return _launch_fwd_rope(*_prep_rope(q, k, v, cos, sin))


@_flash_attn_bthd_rope.register_fake
def _(q, k, v, cos, sin):
    B, T, H, _ = q.shape
    return (
        torch.empty(q.shape, dtype=q.dtype, device=q.device),
        torch.empty((B, H, T), dtype=torch.float32, device=q.device),
        torch.empty(q.shape, dtype=q.dtype, device=q.device),
    )


def _launch_bwd_rope(
    d_o: Tensor, q_rot: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor, cos: Tensor, sin: Tensor
) -> tuple[Tensor, Tensor, Tensor]:
    """Allocates (dq of the unrotated q, dk, dv) and the workspace and launches the RoPE-fused backward on
    contiguous, checked inputs."""
    B, T, H, D = q_rot.shape
    KVH = k.size(2)
    dq, dk, dv = torch.empty_like(q_rot), torch.empty_like(k), torch.empty_like(v)
    if B == 0 or T == 0 or H == 0:
        return dq, dk, dv
    L = lib()
    ws_bytes = L.nn_fa_bwd_workspace_size(B, H, KVH, T, D)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q_rot.device)
    with _on(q_rot):
        rc = L.nn_fa_bwd_rope_strided(
            d_o.data_ptr(), q_rot.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
            dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws_bytes, cos.data_ptr(), sin.data_ptr(),
            cos.shape[0], B, H, KVH, T, D, _bthd_strides(q_rot), _bthd_strides(k), _DTYPES[q_rot.dtype],
            1.0 / math.sqrt(D), _stream(q_rot),
        )
    check(rc)
    return dq, dk, dv


@torch.library.custom_op("nanonemo::flash_attn_bthd_rope_bwd", mutates_args=())
def _flash_attn_bthd_rope_bwd(
    d_o: Tensor, q_rot: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor, cos: Tensor, sin: Tensor
) -> tuple[Tensor, Tensor, Tensor]:
    _refuse_capture_from_autograd_engine("flash_attn_bthd_rope backward op")
    d_o, q_rot, k, v, o, lse = (_contig(t) for t in (d_o, q_rot, k, v, o, lse))
    _check_inputs(q_rot, k, v, seq_dim=1)
    if d_o.shape != q_rot.shape or d_o.dtype != q_rot.dtype or o.shape != q_rot.shape or o.dtype != q_rot.dtype:
        raise RuntimeError("d_o must be a contiguous float16/bfloat16 tensor shaped like q")
    B, T, H, D = q_rot.shape
    if lse.shape != (B, H, T) or lse.dtype != torch.float32:
        raise RuntimeError("lse must be a float32 tensor of shape (B, H, T)")
    cos, sin = _check_tables(cos, sin, T, D, q_rot.device)
    return _launch_bwd_rope(d_o, q_rot, k, v, o, lse, cos, sin)


@_flash_attn_bthd_rope_bwd.register_fake
def _(d_o, q_rot, k, v, o, lse, cos, sin):
    return tuple(torch.empty(t.shape, dtype=t.dtype, device=t.device) for t in (q_rot, k, v))


def _setup_context_rope(ctx, inputs, output):
    _refuse_capture_with_autograd("flash_attn_bthd_rope (autograd)")
    _, k, v, cos, sin = inputs
    o, lse, q_rot = output
    ctx.save_for_backward(q_rot, k, v, o, lse, cos, sin)
    ctx.set_materialize_grads(False)  # the gradients of lse and q_rot are ignored


def _backward_rope(ctx, d_o, _d_lse, _d_q_rot):
    _refuse_capture_with_autograd("flash_attn_bthd_rope backward")
    q_rot, k, v, o, lse, cos, sin = ctx.saved_tensors
    dq, dk, dv = _flash_attn_bthd_rope_bwd(_d_out(d_o, o), q_rot, k, v, o, lse, cos, sin)
    return dq, dk, dv, None, None


_flash_attn_bthd_rope.register_autograd(_backward_rope, setup_context=_setup_context_rope)


class _FlashAttnBthdRopeFn(torch.autograd.Function):
    """The eager path of flash_attn_bthd_rope (see flash_attn's)."""

    @staticmethod
    def forward(ctx, q, k, v, cos, sin):
        q, k, v, cos, sin = _prep_rope(q, k, v, cos, sin)
        o, lse, q_rot = _launch_fwd_rope(q, k, v, cos, sin)
        ctx.save_for_backward(q_rot, k, v, o, lse, cos, sin)
        ctx.set_materialize_grads(False)
        return o

    @staticmethod
    @once_differentiable
    def backward(ctx, d_o):
        _refuse_capture_with_autograd("flash_attn_bthd_rope backward")
        q_rot, k, v, o, lse, cos, sin = ctx.saved_tensors
        dq, dk, dv = _launch_bwd_rope(_contig(_d_out(d_o, o)), q_rot, k, v, o, lse, cos, sin)
        return dq, dk, dv, None, None


def flash_attn_bthd_rope(q: Tensor, k: Tensor, v: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """Causal GQA attention in the projection layout with q's RoPE folded in: q (B, T, H, hd) *before* RoPE,
    k (B, T, KVH, hd) already rotated, v (B, T, KVH, hd), cos/sin fp32 (T_max, hd/2) -> o (B, T, H, hd)."""
    _refuse_capture_with_autograd("flash_attn_bthd_rope", q, k, v)
    if _eager(q, k, v, cos, sin):
        if _records(q, k, v, cos, sin):
            return _FlashAttnBthdRopeFn.apply(q, k, v, cos, sin)
        return _launch_fwd_rope(*_prep_rope(q, k, v, cos, sin))[0]
    o, _, _ = _flash_attn_bthd_rope(q, k, v, cos, sin)
    return o
