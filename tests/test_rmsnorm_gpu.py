"""GPU parity of the HIP fused residual add + RMSNorm against the float64 oracle (oracle/rmsnorm.py).

Mirrors the reference's kernel test (/root/reference/tests/kernels/test_rmsnorm.py): its SHAPES and
dtype pairs, with and without delta, upstream gradients into both outputs (as in the model: the next
sublayer and the residual stream), the autocast output dtype, opcheck and torch.compile(fullgraph=True).
Adds: bfloat16 pairs; the backward pipelined over two rows per team at both ends of its grid range (8192 x 768, the
114 M model's full-size shape, 256 blocks; 16384 x 768, 512 blocks) and at a ragged row count (12289 x 768: the last
block's teams hold one row or none); a width just past the two-rows-per-wave backward (2056); and the empty input.
The oracle sees the same rounded inputs and the residual as the kernel stores it; tolerances are the
reference's (fp32 1e-5; fp16 rtol 1e-3, atol 4e-3, i.e. 2 ulps at magnitude 2-4), with bf16 at the same
two ulps of its own precision.
"""

from __future__ import annotations

import pytest
import torch

from oracle import rmsnorm as R

pytestmark = pytest.mark.gpu

EPS = 1e-5
SHAPES = [(2048, 768), (7, 768), (1, 33), (130, 1000), (64, 4096), (8192, 768), (12289, 768), (16384, 768), (3, 2056),
          (520, 768)]
DTYPES = [
    (torch.float32, torch.float32),
    (torch.float32, torch.float16),
    (torch.float16, torch.float16),
    (torch.float32, torch.bfloat16),
    (torch.bfloat16, torch.bfloat16),
]
# (x dtype, delta dtype or None): every pair with a delta, and each x dtype alone
CASES = [(x, d) for x, d in DTYPES] + [(x, None) for x in (torch.float32, torch.float16, torch.bfloat16)]
TOL = {
    torch.float32: dict(rtol=1e-5, atol=1e-5),
    torch.float16: dict(rtol=1e-3, atol=4e-3),
    torch.bfloat16: dict(rtol=8e-3, atol=3.2e-2),
}


def _mod():
    from nanonemo_amd.kernels.hip import rmsnorm

    return rmsnorm


def _inputs(M, N, x_dtype, d_dtype, with_delta=True, seed=0):
    torch.manual_seed(seed)
    x = torch.randn(M, N, device="cuda", dtype=x_dtype, requires_grad=True)
    d = torch.randn(M, N, device="cuda", dtype=d_dtype, requires_grad=True) if with_delta else None
    w = (1 + 0.1 * torch.randn(N, device="cuda")).requires_grad_()
    return x, d, w


def _np(t):
    return t.detach().double().cpu().numpy()


@pytest.mark.parametrize("M, N", SHAPES)
@pytest.mark.parametrize("x_dtype, d_dtype", CASES)
def test_matches_oracle(M, N, x_dtype, d_dtype):
    print(f"\n[case] add_rms_norm M={M} N={N} x={x_dtype} delta={d_dtype}", flush=True)
    with_delta = d_dtype is not None
    x, d, w = _inputs(M, N, x_dtype, d_dtype, with_delta)
    y, h = _mod().add_rms_norm(x, d, w, EPS)
    tol = TOL[x_dtype]
    h_dtype = torch.promote_types(x_dtype, d_dtype) if with_delta else x_dtype
    assert y.dtype == x_dtype and h.dtype == h_dtype
    # the residual as stored: x + delta in fp32, rounded once to h's dtype
    h_ref = (x.detach().float() + d.detach().float()).to(h_dtype) if with_delta else x.detach()
    torch.testing.assert_close(h, h_ref, rtol=0, atol=0)
    ry, _ = R.forward(_np(h_ref), _np(w), EPS)
    torch.testing.assert_close(y.double().cpu(), torch.from_numpy(ry), **tol)

    gy, gh = torch.randn_like(y), torch.randn_like(h)
    if with_delta:
        torch.autograd.backward([y, h], [gy, gh])
    else:
        y.backward(gy)
    rdx, rdw = R.backward(_np(gy), _np(h_ref), _np(w), EPS, _np(gh) if with_delta else None)
    torch.testing.assert_close(x.grad.double().cpu(), torch.from_numpy(rdx), **tol)
    if with_delta:
        torch.testing.assert_close(d.grad.double().cpu(), torch.from_numpy(rdx), **TOL[d_dtype])
    # dw sums over all rows, so its error grows with M (the reference's allowance)
    torch.testing.assert_close(w.grad.double().cpu(), torch.from_numpy(rdw), rtol=tol["rtol"] * 10,
                               atol=tol["atol"] * M**0.5)


def test_backward_is_deterministic():
    x, d, w = _inputs(8192, 768, torch.float32, torch.bfloat16)
    gy = torch.randn(8192, 768, device="cuda", dtype=torch.float32)
    grads = []
    for _ in range(2):
        xs, ds, ws = (t.detach().clone().requires_grad_() for t in (x, d, w))
        y, h = _mod().add_rms_norm(xs, ds, ws, EPS)
        (y.float() * gy).sum().backward()
        grads.append((xs.grad, ds.grad, ws.grad))
    for a, b in zip(*grads):
        assert torch.equal(a, b)


def test_gradient_through_one_output_only():
    # Autograd passes no gradient for an unused output (the op does not ask it to fill zeros): only the
    # residual used gives dx = ddelta = 1 and dw = 0; only the normalised output used gives the same
    # gradients as an explicit zero gradient for the residual.
    x, d, w = _inputs(520, 768, torch.float32, torch.bfloat16)
    y, h = _mod().add_rms_norm(x, d, w, EPS)
    h.sum().backward()
    assert torch.equal(x.grad, torch.ones_like(x)) and torch.equal(d.grad, torch.ones_like(d))
    assert torch.equal(w.grad, torch.zeros_like(w))
    gy = torch.randn(520, 768, device="cuda")
    grads = []
    for with_zero_dh in (False, True):
        xs, ds, ws = (t.detach().clone().requires_grad_() for t in (x, d, w))
        y, h = _mod().add_rms_norm(xs, ds, ws, EPS)
        loss = (y.float() * gy).sum()
        if with_zero_dh:
            loss = loss + (h * 0).sum()
        loss.backward()
        grads.append((xs.grad, ds.grad, ws.grad))
    for a, b in zip(*grads):
        assert torch.equal(a, b)


def test_empty_rows():
    x = torch.empty(0, 768, device="cuda", requires_grad=True)
    d = torch.empty(0, 768, device="cuda", requires_grad=True)
    w = torch.ones(768, device="cuda", requires_grad=True)
    y, h = _mod().add_rms_norm(x, d, w, EPS)
    (y.sum() + h.sum()).backward()
    assert y.shape == (0, 768) and torch.equal(w.grad, torch.zeros_like(w))


def test_autocast_writes_normalized_output_in_autocast_dtype():
    x, d, w = _inputs(16, 768, torch.float32, torch.bfloat16)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y, h = _mod().add_rms_norm(x, d, w, EPS)
    assert y.dtype == torch.bfloat16 and h.dtype == torch.float32
    ry, _ = R.forward(_np(h), _np(w), EPS)
    torch.testing.assert_close(y.double().cpu(), torch.from_numpy(ry), **TOL[torch.bfloat16])


@pytest.mark.parametrize("with_delta", [True, False])
def test_opcheck(with_delta):
    # schema, fake (meta) implementation and autograd registration
    x, d, w = _inputs(8, 64, torch.float32, torch.float16, with_delta)
    torch.library.opcheck(_mod()._fwd, (x, d, w, EPS, torch.float32))


def test_compiles_without_graph_breaks():
    m = _mod()
    x, d, w = _inputs(64, 768, torch.float32, torch.bfloat16)
    torch._dynamo.reset()
    compiled = torch.compile(lambda x, d, w: m.add_rms_norm(x, d, w, EPS), fullgraph=True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y, h = compiled(x, d, w)
        ry, rh = m.add_rms_norm(x, d, w, EPS)
    torch.testing.assert_close(y, ry)
    torch.testing.assert_close(h, rh)
