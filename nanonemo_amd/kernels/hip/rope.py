"""torch.library op for the gfx950 RoPE kernel (include/nanonemo_rope.h): q and k rotated in one launch.

Replaces the reference's RoPE on either side of the attention op: the plain-PyTorch apply_rope
(/root/reference/nanonemo/model/layers.py:67-74, upcast, two muls and an add per half, a cat and a
downcast per tensor) and its fused Triton apply_rope_qk (nanonemo/kernels/triton/rope.py, used at
layers.py:99-101), which rotates q and k in the (B, T, heads, hd) projection layout in one launch.

    rope_qk(q, k, cos, sin) -> (q', k')      q (B, T, H, hd), k (B, T, KVH, hd); cos/sin fp32 (T_max, hd/2)

The result is bit-identical to the reference's torch formula (fp32 products and sums rounded one at a
time, then one rounding to the input dtype), and so is the gradient (the rotation by -theta).
"""

from __future__ import annotations

import torch
from torch import Tensor
from torch.autograd.function import once_differentiable

from nanonemo_amd.kernels.hip import DTYPE_BF16, DTYPE_F16, DTYPE_F32, check_rope, eager, lib, on_device, records
from nanonemo_amd.kernels.hip import stream_of, strides3

_DTYPES = {torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16, torch.float32: DTYPE_F32}


def _prep(q: Tensor, k: Tensor, cos: Tensor, sin: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    if not (q.is_cuda and k.is_cuda and cos.is_cuda and sin.is_cuda):
        raise RuntimeError("inputs must be CUDA tensors")
    if q.dim() != 4 or k.dim() != 4 or q.shape[0] != k.shape[0] or q.shape[1] != k.shape[1] or q.shape[3] != k.shape[3]:
        raise RuntimeError("expected q (B, T, H, hd) and k (B, T, KVH, hd)")
    if q.dtype not in _DTYPES or k.dtype != q.dtype:
        raise RuntimeError("q and k must share a dtype in {float16, bfloat16, float32}")
    D = q.shape[3]
    if D % 16:
        raise RuntimeError("head_dim must be a multiple of 16")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32 or cos.shape != sin.shape or cos.dim() != 2 \
            or cos.shape[1] != D // 2 or cos.shape[0] < q.shape[1]:
        raise RuntimeError("cos/sin must be float32 (T_max >= T, hd/2) tables")
    q, k = q.contiguous(), k.contiguous()
    return q, k, cos.contiguous(), sin.contiguous()


def _call(fn_name: str, q: Tensor, k: Tensor, cos: Tensor, sin: Tensor) -> tuple[Tensor, Tensor]:
    B, T, H, D = q.shape
    KVH = k.shape[2]
    qo, ko = torch.empty_like(q), torch.empty_like(k)
    if q.numel() == 0 and k.numel() == 0:
        return qo, ko
    with on_device(q):
        rc = getattr(lib(), fn_name)(
            q.data_ptr(), qo.data_ptr(), k.data_ptr(), ko.data_ptr(), cos.data_ptr(), sin.data_ptr(),
            B, T, H, KVH, D, strides3(T * H * D, H * D, D), strides3(T * KVH * D, KVH * D, D), cos.shape[0],
            _DTYPES[q.dtype], stream_of(q),
        )
    check_rope(rc)
    return qo, ko


@torch.library.custom_op("nanonemo::rope_qk", mutates_args=())
def _rope_qk(q: Tensor, k: Tensor, cos: Tensor, sin: Tensor) -> tuple[Tensor, Tensor]:
    return _call("nn_rope_qk", *_prep(q, k, cos, sin))


@_rope_qk.register_fake
def _(q, k, cos, sin):
    return torch.empty(q.shape, dtype=q.dtype, device=q.device), torch.empty(k.shape, dtype=k.dtype, device=k.device)


@torch.library.custom_op("nanonemo::rope_qk_bwd", mutates_args=())
def _rope_qk_bwd(dq: Tensor, dk: Tensor, cos: Tensor, sin: Tensor) -> tuple[Tensor, Tensor]:
    return _call("nn_rope_qk_bwd", *_prep(dq, dk, cos, sin))


@_rope_qk_bwd.register_fake
def _(dq, dk, cos, sin):
    return torch.empty(dq.shape, dtype=dq.dtype, device=dq.device), torch.empty(dk.shape, dtype=dk.dtype, device=dk.device)


def _setup_context(ctx, inputs, output):
    _, _, cos, sin = inputs
    ctx.save_for_backward(cos, sin)


def _backward(ctx, dq, dk):
    cos, sin = ctx.saved_tensors
    gq, gk = _rope_qk_bwd(dq, dk, cos, sin)
    return gq, gk, None, None


_rope_qk.register_autograd(_backward, setup_context=_setup_context)


class _RopeQkFn(torch.autograd.Function):
    """The eager path of rope_qk (plain CUDA tensors outside tracing; ``eager``): the op's launches and autograd
    wiring without its dispatch, so the same bits for less host time."""

    @staticmethod
    def forward(ctx, q, k, cos, sin):
        ctx.save_for_backward(cos, sin)
        return _call("nn_rope_qk", *_prep(q, k, cos, sin))

    @staticmethod
    @once_differentiable
    def backward(ctx, dq, dk):
        cos, sin = ctx.saved_tensors
        gq, gk = _call("nn_rope_qk_bwd", *_prep(dq, dk, cos, sin))
        return gq, gk, None, None


def _rope(q: Tensor, k: Tensor, cos: Tensor, sin: Tensor) -> tuple[Tensor, Tensor]:
    if eager(q, k, cos, sin):
        if records(q, k, cos, sin):
            return _RopeQkFn.apply(q, k, cos, sin)
        return _call("nn_rope_qk", *_prep(q, k, cos, sin))
    return _rope_qk(q, k, cos, sin)


def rope_qk(q: Tensor, k: Tensor, cos: Tensor, sin: Tensor) -> tuple[Tensor, Tensor]:
    """Rotate q (B, T, H, hd) and k (B, T, KVH, hd) by the positions' angles (cos/sin: fp32 (T_max, hd/2))."""
    return _rope(q, k, cos, sin)


def rope_k(k: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """Rotate k (B, T, KVH, hd) alone (the q half of the pass is folded into the attention op)."""
    q = k.new_empty(k.shape[0], k.shape[1], 0, k.shape[3])
    return _rope(q, k, cos, sin)[1]
