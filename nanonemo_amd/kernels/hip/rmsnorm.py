"""torch.library ops for the gfx950 fused residual add + RMSNorm (include/nanonemo_rmsnorm.h).

Drop-in for /root/reference/nanonemo/kernels/cuda/rmsnorm.py: the same op names and schemas
(``nanonemo::cuda_add_rms_norm_fwd`` :17-22 and ``nanonemo::cuda_add_rms_norm_bwd`` :31-38), the same fake
impls (:25-28, :41-44), the same autograd wiring (save h, or x when there is no delta, with weight and
rstd; :47-61) and the same public ``add_rms_norm(x, delta, weight, eps) -> (y, x + delta)`` (:64-68), whose
output dtype follows autocast. The model selects it with ``norm_kernel="hip"`` where the reference uses
``norm_kernel="cuda"`` (/root/reference/nanonemo/model/layers.py:36-56).

Differences from the reference: bfloat16 as well as float16 / float32 tensors (widening), and dw is summed
on the device by the library in a fixed order (the reference sums its partials with torch on the host
side). Hidden sizes are the reference's: a multiple of 8 up to 4096, or any size up to 1024.
"""

from __future__ import annotations

import torch
from torch import Tensor
from torch.autograd.function import once_differentiable

from nanonemo_amd.kernels.hip import check_rmsnorm, eager, lib, on_device, records, stream_of

_CODES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def _code(dtype: torch.dtype) -> int:
    if dtype not in _CODES:
        raise RuntimeError(f"only float32, float16 and bfloat16 are supported, got {dtype}")
    return _CODES[dtype]




def _fwd_impl(
    x: Tensor, delta: Tensor | None, weight: Tensor, eps: float, out_dtype: torch.dtype
) -> tuple[Tensor, Tensor, Tensor]:
    """Checks, allocates and launches the forward: (y, h, rstd). The body of the op and of the eager path."""
    if not x.is_cuda:
        raise RuntimeError("x must be a CUDA tensor")
    x = x.contiguous()
    delta = delta.contiguous() if delta is not None else None
    weight = weight.contiguous()
    if weight.dtype != torch.float32:
        raise RuntimeError("weight must be contiguous float32")
    if delta is not None and delta.shape != x.shape:
        raise RuntimeError("delta must match x")
    N = x.size(-1)
    if weight.numel() != N:
        raise RuntimeError("weight must have hidden-size elements")
    M = x.numel() // N if N else 0
    y = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    h = torch.empty(x.shape, dtype=torch.promote_types(x.dtype, delta.dtype), device=x.device) if delta is not None \
        else x.new_empty(0)
    rstd = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    with on_device(x):
        rc = lib().nn_add_rmsnorm_fwd(
            x.data_ptr(), delta.data_ptr() if delta is not None else None, weight.data_ptr(), y.data_ptr(),
            h.data_ptr() if delta is not None else None, rstd.data_ptr(), M, N, eps, _code(x.dtype),
            _code(delta.dtype) if delta is not None else 0, _code(out_dtype), stream_of(x),
        )
    check_rmsnorm(rc)
    return y, h, rstd


@torch.library.custom_op("nanonemo::cuda_add_rms_norm_fwd", mutates_args=())
def _fwd(x: Tensor, delta: Tensor | None, weight: Tensor, eps: float, out_dtype: torch.dtype) -> tuple[Tensor, Tensor, Tensor]:
    return _fwd_impl(x, delta, weight, eps, out_dtype)


@_fwd.register_fake
def _(x, delta, weight, eps, out_dtype):
    h = x.new_empty(x.shape, dtype=torch.promote_types(x.dtype, delta.dtype)) if delta is not None else x.new_empty(0)
    return x.new_empty(x.shape, dtype=out_dtype), h, x.new_empty(x.shape[:-1], dtype=torch.float32)


def _bwd_impl(
    dy: Tensor, dh: Tensor | None, h: Tensor, weight: Tensor, rstd: Tensor,
    dx_dtype: torch.dtype, ddelta_dtype: torch.dtype | None,
) -> tuple[Tensor, Tensor, Tensor]:
    """Checks, allocates and launches the backward: (dx, ddelta, dw). The body of the op and of the eager path."""
    dy, h, weight, rstd = dy.contiguous(), h.contiguous(), weight.contiguous(), rstd.contiguous()
    dh = dh.contiguous() if dh is not None else None
    if dy.shape != h.shape:
        raise RuntimeError("dy and h must be contiguous, same shape")
    if (dh is None) != (ddelta_dtype is None):
        raise RuntimeError("dh and ddelta_dtype go together")
    if dh is not None and dh.dtype != h.dtype:
        raise RuntimeError("dh must be contiguous, h's dtype")
    N = h.size(-1)
    M = h.numel() // N if N else 0
    dx = torch.empty(h.shape, dtype=dx_dtype, device=h.device)
    dd = torch.empty(h.shape, dtype=ddelta_dtype, device=h.device) if dh is not None else h.new_empty(0)
    dw = torch.empty(N, dtype=torch.float32, device=h.device)
    L = lib()
    ws_bytes = L.nn_add_rmsnorm_bwd_workspace_size(M, N)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=h.device)
    with on_device(h):
        rc = L.nn_add_rmsnorm_bwd(
            dy.data_ptr(), dh.data_ptr() if dh is not None else None, h.data_ptr(), weight.data_ptr(),
            rstd.data_ptr(), dx.data_ptr(), dd.data_ptr() if dh is not None else None, dw.data_ptr(), ws.data_ptr(),
            ws_bytes, M, N, _code(dy.dtype), _code(h.dtype), _code(dx_dtype),
            _code(ddelta_dtype) if ddelta_dtype is not None else 0, stream_of(h),
        )
    check_rmsnorm(rc)
    return dx, dd, dw.to(weight.dtype)


@torch.library.custom_op("nanonemo::cuda_add_rms_norm_bwd", mutates_args=())
def _bwd(
    dy: Tensor, dh: Tensor | None, h: Tensor, weight: Tensor, rstd: Tensor,
    dx_dtype: torch.dtype, ddelta_dtype: torch.dtype | None,
) -> tuple[Tensor, Tensor, Tensor]:
    return _bwd_impl(dy, dh, h, weight, rstd, dx_dtype, ddelta_dtype)


@_bwd.register_fake
def _(dy, dh, h, weight, rstd, dx_dtype, ddelta_dtype):
    dd = h.new_empty(h.shape, dtype=ddelta_dtype) if ddelta_dtype is not None else h.new_empty(0)
    return h.new_empty(h.shape, dtype=dx_dtype), dd, torch.empty_like(weight)


def _save(ctx, x, delta, weight, y, h, rstd):
    ctx.save_for_backward(h if delta is not None else x, weight, rstd)
    ctx.x_dtype = x.dtype
    ctx.y_dtype = y.dtype
    ctx.delta_dtype = delta.dtype if delta is not None else None
    # rstd's gradient is ignored, so autograd need not fill a zero tensor for it on every backward.
    ctx.set_materialize_grads(False)


def _setup_context(ctx, inputs, output):
    x, delta, weight, eps, out_dtype = inputs
    _save(ctx, x, delta, weight, *output)


def _grads(ctx, dy, dh, bwd):
    h, weight, rstd = ctx.saved_tensors
    has_delta = ctx.delta_dtype is not None
    if dy is None:  # y unused downstream
        dy = torch.zeros(h.shape, dtype=ctx.y_dtype, device=h.device)
    if has_delta and dh is None:  # h unused downstream
        dh = torch.zeros_like(h)
    dx, dd, dw = bwd(dy, dh if has_delta else None, h, weight, rstd, ctx.x_dtype, ctx.delta_dtype)
    return dx, (dd if has_delta else None), dw, None, None


def _backward(ctx, dy, dh, _drstd):
    return _grads(ctx, dy, dh, _bwd)


_fwd.register_autograd(_backward, setup_context=_setup_context)


class _AddRmsNormFn(torch.autograd.Function):
    """The eager path of add_rms_norm (plain CUDA tensors outside tracing; ``eager``): the op's launches and
    autograd wiring without its dispatch, so the same bits for less host time. Outputs y and h (an empty tensor
    when delta is None); rstd is saved, not returned."""

    @staticmethod
    def forward(ctx, x, delta, weight, eps, out_dtype):
        y, h, rstd = _fwd_impl(x, delta, weight, eps, out_dtype)
        _save(ctx, x, delta, weight, y, h, rstd)
        if delta is None:
            ctx.mark_non_differentiable(h)
        return y, h

    @staticmethod
    @once_differentiable
    def backward(ctx, dy, dh):
        return _grads(ctx, dy, dh, _bwd_impl)


def add_rms_norm(x: Tensor, delta: Tensor | None, weight: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    """Returns (rmsnorm(x + delta) * weight, x + delta); delta=None normalizes x alone. Under autocast
    the normalized output takes the autocast dtype (the residual keeps its own)."""
    out_dtype = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else x.dtype
    ins = (x, weight) if delta is None else (x, delta, weight)
    if eager(*ins):
        if records(*ins):
            y, h = _AddRmsNormFn.apply(x, delta, weight, eps, out_dtype)
        else:
            y, h, _ = _fwd_impl(x, delta, weight, eps, out_dtype)
    else:
        y, h, _ = _fwd(x, delta, weight, eps, out_dtype)
    return y, (x if delta is None else h)
