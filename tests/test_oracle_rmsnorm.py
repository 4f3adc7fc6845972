"""Pins the float64 add + RMSNorm oracle (oracle/rmsnorm.py) on the CPU, independently of it:

* torch autograd in float64 of the reference's plain-PyTorch formula (/root/reference/nanonemo/model/
  layers.py:19-33: x * rsqrt(mean(x^2) + eps) * w), a separate implementation of the derivative;
* central finite differences of the oracle's own forward;
* closed forms at eps = 0: y is unchanged by scaling a row (so the gradient is orthogonal to h when
  w = 1), and a constant row c maps to sign(c) * w;
* planted mistakes in the oracle (a sum for a mean, a dropped projection term, rstd squared) that these
  checks must catch.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import rmsnorm as R

EPS = 1e-5


def _rand(M, N, seed=0):
    g = np.random.default_rng(seed)
    return g.standard_normal((M, N)), 1 + 0.1 * g.standard_normal(N), g.standard_normal((M, N)), g.standard_normal((M, N))


def _torch(h, w, dy, dh, eps):
    ht = torch.tensor(h, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    y = ht * torch.rsqrt(ht.pow(2).mean(dim=-1, keepdim=True) + eps) * wt
    (y * torch.tensor(dy)).sum().backward()
    return y.detach().numpy(), ht.grad.numpy() + dh, wt.grad.numpy()


@pytest.mark.parametrize("M, N", [(7, 768), (1, 33), (130, 1000), (3, 8)])
def test_matches_torch_autograd(M, N):
    h, w, dy, dh = _rand(M, N)
    y, _ = R.forward(h, w, EPS)
    dx, dw = R.backward(dy, h, w, EPS, dh)
    ty, tdx, tdw = _torch(h, w, dy, dh, EPS)
    np.testing.assert_allclose(y, ty, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(dx, tdx, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(dw, tdw, rtol=1e-10, atol=1e-10)


def test_matches_finite_differences():
    h, w, dy, _ = _rand(3, 10, seed=1)
    dx, dw = R.backward(dy, h, w, EPS)
    step = 1e-6
    f = lambda hh, ww: float((R.forward(hh, ww, EPS)[0] * dy).sum())  # noqa: E731
    for (r, c) in [(0, 0), (1, 7), (2, 9)]:
        e = np.zeros_like(h)
        e[r, c] = step
        assert abs((f(h + e, w) - f(h - e, w)) / (2 * step) - dx[r, c]) < 1e-7
    for c in (0, 4, 9):
        e = np.zeros_like(w)
        e[c] = step
        assert abs((f(h, w + e) - f(h, w - e)) / (2 * step) - dw[c]) < 1e-7


def test_scale_invariance_closed_forms():
    h, w, dy, _ = _rand(4, 16, seed=2)
    y, rstd = R.forward(h, w, 0.0)
    y2, _ = R.forward(3.5 * h, w, 0.0)
    np.testing.assert_allclose(y, y2, rtol=1e-13)
    np.testing.assert_allclose(rstd, 1 / np.sqrt((h * h).mean(-1)), rtol=1e-13)
    dx, _ = R.backward(dy, h, np.ones(16), 0.0)
    np.testing.assert_allclose((dx * h).sum(-1), 0.0, atol=1e-12)  # y(a h) = y(h): no gradient along h
    c = np.array([[2.5] * 16, [-0.75] * 16])
    np.testing.assert_allclose(R.forward(c, w, 0.0)[0], np.sign(c) * w, rtol=1e-13)


def _fails(check) -> bool:
    try:
        check()
    except AssertionError:
        return True
    return False


def _check_all():
    test_matches_torch_autograd(7, 768)
    test_matches_finite_differences()


def test_planted_sum_instead_of_mean_is_caught(monkeypatch):
    def bad(h, w, eps):
        hd = np.asarray(h, dtype=np.float64)
        rstd = 1 / np.sqrt((hd * hd).sum(axis=-1, keepdims=True) + eps)
        return hd * rstd * w, rstd[..., 0]

    monkeypatch.setattr(R, "forward", bad)
    assert _fails(_check_all)


def test_planted_dropped_projection_term_is_caught(monkeypatch):
    def bad(dy, h, w, eps, dh=None):
        rstd = 1 / np.sqrt((h * h).mean(-1, keepdims=True) + eps)
        dx = rstd * dy * w + (dh if dh is not None else 0)
        return dx, (dy * h * rstd).sum(0)

    monkeypatch.setattr(R, "backward", bad)
    assert _fails(_check_all)


def test_planted_rstd_squared_is_caught(monkeypatch):
    good = R.backward

    def bad(dy, h, w, eps, dh=None):
        dx, dw = good(dy, h, w, eps, dh)
        rstd = 1 / np.sqrt((h * h).mean(-1, keepdims=True) + eps)
        return (dx - (dh if dh is not None else 0)) * rstd + (dh if dh is not None else 0), dw

    monkeypatch.setattr(R, "backward", bad)
    assert _fails(_check_all)
