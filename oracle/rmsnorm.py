"""CPU oracle for the fused residual add + RMSNorm, forward and backward, in float64.

TEST INFRASTRUCTURE ONLY. Only tests/ may import this module, and only as the checker. The product path
(nanonemo_amd) never imports it and has no CPU fallback.

The build's own numpy restatement of the reference's plain-PyTorch RMSNorm / AddRMSNorm
(/root/reference/nanonemo/model/layers.py:19-56) and of the math its fused kernel implements
(/root/reference/nanonemo/kernels/cuda/rmsnorm.cu:1-9, fwd :62-98, bwd :102-154). The reference holds
no golden vectors for this path (its tests compare against PyTorch at run time), so every function here
is pinned in tests/test_oracle_rmsnorm.py by independent checks: torch autograd in float64 of the
reference formula, central finite differences, the scale-invariance closed forms at eps = 0, and planted
mistakes those checks must catch.

Conventions (all from the reference):
  * rows are the last dimension; h = x + delta is the residual as stored (rounded to its dtype by the
    caller: the kernels normalise the stored residual, rmsnorm.cu:84-86);
  * y = (h * rstd) * w with rstd = 1 / sqrt(mean(h^2) + eps) (layers.py:29-31, rmsnorm.cu:91-96);
  * backward with n = h * rstd, dn = dy * w: dh = rstd * (dn - n * mean(dn * n)) + dh_residual and
    dw = sum over rows of dy * n (rmsnorm.cu:3-4, :130-149).
"""

from __future__ import annotations

import numpy as np


def forward(h, w, eps: float):
    """(y, rstd) of RMSNorm over the last dimension of the stored residual h, float64."""
    hd = np.asarray(h, dtype=np.float64)
    rstd = 1.0 / np.sqrt((hd * hd).mean(axis=-1, keepdims=True) + eps)
    return hd * rstd * np.asarray(w, dtype=np.float64), rstd[..., 0]


def backward(dy, h, w, eps: float, dh=None):
    """(dx, dw): the gradient into the residual (plus dh, the gradient arriving at h itself) and into w."""
    hd = np.asarray(h, dtype=np.float64)
    wd = np.asarray(w, dtype=np.float64)
    g = np.asarray(dy, dtype=np.float64)
    rstd = 1.0 / np.sqrt((hd * hd).mean(axis=-1, keepdims=True) + eps)
    n = hd * rstd
    dn = g * wd
    dx = rstd * (dn - n * (dn * n).mean(axis=-1, keepdims=True))
    if dh is not None:
        dx = dx + np.asarray(dh, dtype=np.float64)
    dw = (g * n).reshape(-1, hd.shape[-1]).sum(axis=0)
    return dx, dw
