"""GPU tests of the layout-fused boundary: the strided C-ABI entry points (nn_fa_fwd_strided,
nn_fa_bwd_strided) and the (B, T, heads, hd) ops nanonemo::flash_attn_bthd / _bwd.

Strides only change addressing, never arithmetic, so every result here must be bit-identical to the
dense [B, heads, T, hd] path, whose parity against the float64 oracle is established in
test_flash_attn_gpu.py; one shape is also checked against the oracle directly.
"""

from __future__ import annotations

import ctypes
import math

import pytest
import torch

from oracle import attention as oracle
from tests.common import LSE_ATOL, TOL, TOL_GRAD, assert_close_tol, errors, make_inputs

pytestmark = pytest.mark.gpu

DEV = "cuda"

SHAPES = [(2, 12, 4, 200, 64), (1, 4, 2, 37, 32), (3, 8, 8, 65, 64), (1, 6, 2, 1, 64)]


def _fa():
    from nanonemo_amd.kernels.hip import flash_attn as fa

    return fa


def _bhtd(q, k, v, do):
    fa = _fa()
    q, k, v = (t.to(DEV).requires_grad_() for t in (q, k, v))
    o, lse = fa._flash_attn(q, k, v)
    o.backward(do.to(DEV))
    return o.detach(), lse, q.grad, k.grad, v.grad


def _bthd(q, k, v, do):
    """The same problem through the (B, T, heads, hd) ops; results returned in [B, heads, T, hd]."""
    fa = _fa()
    qt, kt, vt = (t.transpose(1, 2).contiguous().to(DEV).requires_grad_() for t in (q, k, v))
    o, lse = fa._flash_attn_bthd(qt, kt, vt)
    assert o.shape == qt.shape and o.is_contiguous()
    o.backward(do.transpose(1, 2).contiguous().to(DEV))
    for g, t in ((qt.grad, qt), (kt.grad, kt), (vt.grad, vt)):
        assert g.shape == t.shape and g.is_contiguous()
    return o.detach().transpose(1, 2), lse, qt.grad.transpose(1, 2), kt.grad.transpose(1, 2), vt.grad.transpose(1, 2)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B, H, KVH, T, hd", SHAPES)
def test_bthd_ops_bit_identical_to_dense(B, H, KVH, T, hd, dtype):
    print(f"\n[case] bthd B={B} H={H} KVH={KVH} T={T} hd={hd} {dtype}", flush=True)
    q, k, v, do = make_inputs(B, H, KVH, T, hd, dtype, seed=3)
    ref = _bhtd(q, k, v, do)
    got = _bthd(q, k, v, do)
    torch.cuda.synchronize()
    for name, a, b in zip(("o", "lse", "dq", "dk", "dv"), got, ref):
        assert torch.equal(a, b), f"{name} differs from the dense path"


def test_bthd_matches_oracle():
    dtype = torch.bfloat16
    q, k, v, do = make_inputs(2, 12, 4, 130, 64, dtype, seed=5)
    o, lse, dq, dk, dv = (t.cpu() for t in _bthd(q, k, v, do))
    qd, kd, vd, dod = (t.double().numpy() for t in (q, k, v, do))
    ro, rlse = oracle.forward(qd, kd, vd)
    rdq, rdk, rdv = oracle.backward(dod, qd, kd, vd, ro, rlse)
    assert_close_tol(o, torch.from_numpy(ro), TOL[dtype], "bthd o")
    assert errors(lse, torch.from_numpy(rlse))["max_abs"] <= LSE_ATOL
    for name, x, r in (("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv)):
        assert_close_tol(x, torch.from_numpy(r), TOL_GRAD[dtype], f"bthd {name}")


def _padded(t: torch.Tensor, pad_row: int, pad_head: int, pad_batch: int) -> torch.Tensor:
    """A [B, h, T, D] view of t with padded rows, heads and batches (strides multiples of 8)."""
    B, h, T, D = t.shape
    st = D + pad_row
    sh = T * st + pad_head
    sb = h * sh + pad_batch
    buf = torch.full((B * sb + 64,), float("nan"), dtype=t.dtype, device=DEV)
    view = buf.as_strided((B, h, T, D), (sb, sh, st, 1))
    view.copy_(t.to(DEV))
    return view


def test_strided_c_abi_with_padded_rows():
    from nanonemo_amd.kernels.hip import DTYPE_BF16, check, lib, strides3

    B, H, KVH, T, D = 2, 6, 3, 150, 64
    dtype = torch.bfloat16
    q, k, v, do = make_inputs(B, H, KVH, T, D, dtype, seed=9)
    ref = _bhtd(q, k, v, do)
    torch.cuda.synchronize()

    pq, pk, pv, pdo = _padded(q, 8, 16, 24), _padded(k, 8, 16, 24), _padded(v, 8, 16, 24), _padded(do, 8, 16, 24)
    # o / dq share q's layout, dk / dv share k's; pre-fill with NaN so unwritten padding shows up
    po, pdq = _padded(torch.full_like(q, float("nan")), 8, 16, 24), _padded(torch.full_like(q, float("nan")), 8, 16, 24)
    pdk, pdv = _padded(torch.full_like(k, float("nan")), 8, 16, 24), _padded(torch.full_like(k, float("nan")), 8, 16, 24)
    sq = strides3(*pq.stride()[:3])
    sk = strides3(*pk.stride()[:3])
    assert tuple(pq.stride()[:3]) == tuple(po.stride()[:3]) and tuple(pk.stride()[:3]) == tuple(pdk.stride()[:3])
    lse = torch.empty(B, H, T, dtype=torch.float32, device=DEV)
    L = lib()
    sp = torch.cuda.current_stream().cuda_stream
    scale = 1.0 / math.sqrt(D)
    print(f"\n[case] strided C ABI B={B} H={H} KVH={KVH} T={T} D={D} strides q {pq.stride()} k {pk.stride()}", flush=True)
    check(L.nn_fa_fwd_strided(pq.data_ptr(), pk.data_ptr(), pv.data_ptr(), po.data_ptr(), lse.data_ptr(),
                              B, H, KVH, T, D, sq, sk, DTYPE_BF16, scale, sp))
    ws_bytes = L.nn_fa_bwd_workspace_size(B, H, KVH, T, D)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    check(L.nn_fa_bwd_strided(pdo.data_ptr(), pq.data_ptr(), pk.data_ptr(), pv.data_ptr(), po.data_ptr(), lse.data_ptr(),
                              pdq.data_ptr(), pdk.data_ptr(), pdv.data_ptr(), ws.data_ptr(), ws_bytes,
                              B, H, KVH, T, D, sq, sk, DTYPE_BF16, scale, sp))
    torch.cuda.synchronize()
    for name, a, b in zip(("o", "lse", "dq", "dk", "dv"), (po, lse, pdq, pdk, pdv), ref):
        assert torch.equal(a, b), f"{name} differs from the dense path"


def test_bthd_compiles_without_graph_breaks():
    fa = _fa()
    B, H, KVH, T, D = 2, 12, 4, 96, 64

    def attn_block(x, wq, wk, wv, wo):
        q = (x @ wq).view(B, T, H, D)
        k = (x @ wk).view(B, T, KVH, D)
        v = (x @ wv).view(B, T, KVH, D)
        return fa.flash_attn_bthd(q, k, v).view(B, T, H * D) @ wo

    g = torch.Generator(device=DEV).manual_seed(0)
    x = torch.randn(B, T, 256, device=DEV, generator=g, dtype=torch.bfloat16)
    ws = [torch.randn(256, n, device=DEV, generator=g, dtype=torch.bfloat16) * 0.05 for n in (H * D, KVH * D, KVH * D)]
    wo = torch.randn(H * D, 256, device=DEV, generator=g, dtype=torch.bfloat16) * 0.05
    params = [w.requires_grad_() for w in (*ws, wo)]
    eager = attn_block(x, *params)
    eager.float().square().sum().backward()
    grads = [p.grad.clone() for p in params]
    for p in params:
        p.grad = None
    compiled = torch.compile(attn_block, fullgraph=True)
    out = compiled(x, *params)
    out.float().square().sum().backward()
    torch.cuda.synchronize()
    assert torch.equal(out, eager)
    for a, b in zip((p.grad for p in params), grads):
        torch.testing.assert_close(a, b, rtol=1e-2, atol=1e-2)
