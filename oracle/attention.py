"""CPU oracle for causal grouped-query attention, forward and backward, in float64.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker (or, in bench.py, as the timed CPU baseline). The product
path (nanonemo_amd) never imports it and has no CPU fallback.

This is the build's own numpy restatement of the reference's plain-PyTorch attention and of the math
its CUDA kernel implements. The reference holds no golden vectors for this path (its tests compare
against PyTorch at run time), so every function here is pinned in tests/test_oracle.py by independent
checks: torch's scaled_dot_product_attention (math backend) plus autograd in float64, brute-force
Python loops on tiny shapes, closed forms (T = 1, Q = 0, GQA == MHA with repeated K/V), and planted
mistakes that those checks must catch.

Conventions (all from the reference):
  * q: (B, H, T, D); k, v: (B, KVH, T, D); query head h reads KV head h // (H // KVH)
    (/root/reference/nanonemo/kernels/cuda/flash_attn.cu:59, nanonemo/model/layers.py:109-113).
  * Causal, square, top-left aligned: key j is visible to query i iff j <= i
    (flash_attn.cu:103,126; tests/kernels/test_flash_attn.py:28 uses SDPA is_causal=True).
  * scale = 1 / sqrt(D) (flash_attn.cu:370).
  * lse is the natural-log logsumexp of the scaled, masked scores, shape (B, H, T)
    (flash_attn.cu:162, :366).
  * The backward ignores the gradient of lse (flash_attn.py:49) and returns gradients summed over
    the query heads of each KV group (flash_attn.cu:235,256).
"""

from __future__ import annotations

import numpy as np


def kv_head_index(H: int, KVH: int) -> np.ndarray:
    """KV head read by each query head: h // (H // KVH) (flash_attn.cu:59; repeat_interleave order)."""
    return np.arange(H) // (H // KVH)


def causal_mask(T: int) -> np.ndarray:
    """Boolean (T, T) mask, True where key j is in the future of query i (j > i) (flash_attn.cu:126)."""
    return np.triu(np.ones((T, T), dtype=bool), k=1)


def _expand(x: np.ndarray, H: int) -> np.ndarray:
    return x[:, kv_head_index(H, x.shape[1])]


def _scores(qb: np.ndarray, kb: np.ndarray, scale: float) -> np.ndarray:
    s = np.matmul(qb, np.swapaxes(kb, -1, -2)) * scale
    s[..., causal_mask(qb.shape[-2])] = -np.inf
    return s


def forward(q, k, v, scale: float | None = None):
    """(o, lse) of causal GQA attention in float64.

    Restates flash_attn.cu:52-174 (fwd_kernel) without tiling: o = softmax(scale * Q K_h^T + M) V_h,
    lse = ln sum_j exp(scale * s_ij) over visible j. Loops over the batch to bound memory.
    """
    q, k, v = (np.asarray(t, dtype=np.float64) for t in (q, k, v))
    B, H, T, D = q.shape
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    o = np.empty_like(q)
    lse = np.empty((B, H, T))
    for b in range(B):
        s = _scores(q[b : b + 1], _expand(k[b : b + 1], H), scale)
        m = s.max(-1, keepdims=True)
        e = np.exp(s - m)
        l = e.sum(-1, keepdims=True)
        o[b] = np.matmul(e / l, _expand(v[b : b + 1], H))[0]
        lse[b] = (m + np.log(l))[0, ..., 0]
    return o, lse


def group_sum(x: np.ndarray, KVH: int) -> np.ndarray:
    """Sum (B, H, T, D) per-query-head gradients into (B, KVH, T, D) per KV head (flash_attn.cu:235,256)."""
    B, H, T, D = x.shape
    return x.reshape(B, KVH, H // KVH, T, D).sum(2)


def backward(do, q, k, v, o=None, lse=None, scale: float | None = None):
    """(dq, dk, dv) in float64 from the closed forms the reference kernel implements (flash_attn.cu:176-340).

    P = exp(scale * S - lse); D = rowsum(dO * O) (flash_attn.cu:388); dP = dO V_h^T;
    dS = P * (dP - D); dQ = scale * dS K_h; dK_h = scale * dS^T Q; dV_h = P^T dO; dK, dV are then
    summed over the query heads of each KV group. ``o`` and ``lse`` default to this module's forward.
    """
    do, q, k, v = (np.asarray(t, dtype=np.float64) for t in (do, q, k, v))
    B, H, T, D = q.shape
    KVH = k.shape[1]
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    if o is None or lse is None:
        o, lse = forward(q, k, v, scale)
    o = np.asarray(o, dtype=np.float64)
    lse = np.asarray(lse, dtype=np.float64)
    dq = np.empty_like(q)
    dk = np.empty_like(k)
    dv = np.empty_like(v)
    for b in range(B):
        kb, vb = _expand(k[b : b + 1], H)[0], _expand(v[b : b + 1], H)[0]
        s = _scores(q[b : b + 1], kb[None], scale)[0]
        p = np.exp(s - lse[b][..., None])
        dvec = preprocess(do[b], o[b])[..., None]
        dp = np.matmul(do[b], np.swapaxes(vb, -1, -2))
        ds = p * (dp - dvec)
        dq[b] = scale * np.matmul(ds, kb)
        dk[b] = group_sum((scale * np.matmul(np.swapaxes(ds, -1, -2), q[b]))[None], KVH)[0]
        dv[b] = group_sum(np.matmul(np.swapaxes(p, -1, -2), do[b])[None], KVH)[0]
    return dq, dk, dv


def preprocess(do, o):
    """D = rowsum(dO * O) in float64, shape (B, H, T) (flash_attn.cu:388)."""
    return (np.asarray(do, dtype=np.float64) * np.asarray(o, dtype=np.float64)).sum(-1)


def flops(B: int, H: int, T: int, D: int, which: str = "fwd+bwd") -> float:
    """Algorithmic FLOPs, 2 per multiply-add over the causal (query, key) pairs, recompute not counted.

    Pairs = B*H*T*(T+1)/2. The forward does 2 products (QK^T, PV): 4*D flop per pair; the backward 4
    (dV, dP, dQ, dK): 8*D flop per pair. So fwd = 2*B*H*D*T*(T+1), bwd = 4*B*H*D*T*(T+1),
    fwd+bwd = 6*B*H*D*T*(T+1).
    """
    per = {"fwd": 2, "bwd": 4, "fwd+bwd": 6}[which]
    return float(per) * B * H * D * T * (T + 1)


def torch_reference_fwd_bwd(q, k, v, do, explicit: bool = False):
    """The reference's plain-PyTorch attention, forward plus autograd backward, in the inputs' dtype.

    Restates /root/reference/nanonemo/model/layers.py:109-115 and tests/kernels/test_flash_attn.py:24-28:
    repeat_interleave K/V over the group, then F.scaled_dot_product_attention(is_causal=True) pinned
    to the math backend; with ``explicit`` the per-head loop form of tests/model/test_layers.py:107-123
    (matmul, triu mask, softmax, matmul) batched over heads. Used as the timed CPU baseline.
    Returns (o, dq, dk, dv).
    """
    import torch
    import torch.nn.functional as F

    q, k, v = (t.detach().requires_grad_() for t in (q, k, v))
    group = q.shape[1] // k.shape[1]
    kr, vr = k.repeat_interleave(group, dim=1), v.repeat_interleave(group, dim=1)
    if explicit:
        T = q.shape[2]
        s = torch.matmul(q, kr.transpose(-1, -2)) / (q.shape[-1] ** 0.5)
        s = s.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
        o = torch.matmul(s.softmax(-1), vr)
    else:
        with torch.nn.attention.sdpa_kernel(torch.nn.attention.SDPBackend.MATH):
            o = F.scaled_dot_product_attention(q, kr, vr, is_causal=True)
    dq, dk, dv = torch.autograd.grad(o, (q, k, v), do)
    return o.detach(), dq, dk, dv
