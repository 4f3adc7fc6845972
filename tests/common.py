"""Helpers shared by the tests: seeded inputs, golden fixtures, error metrics, tolerances."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"

# (B, H, KVH, T, hd) from the reference's tests/kernels/test_flash_attn.py:12: the model shape, MHA with
# an odd T, T=1 with a short head_dim, and 4:1 GQA with T one past a tile.
REF_SHAPES = [(2, 12, 4, 1024, 64), (2, 4, 4, 37, 64), (1, 1, 1, 1, 32), (3, 8, 2, 65, 32)]

# Tolerances against the float64 oracle on the same rounded inputs. Elementwise (assert_close
# semantics with a scale-aware absolute term):
#     |x - ref| <= max(atol, atol_rel * max|ref|) + rtol * |ref|
# plus a relative Frobenius-norm bound on the whole tensor.
#   fp16: atol = rtol = 2e-2 is the reference's own TOL (tests/kernels/test_flash_attn.py:13), which it
#         applied against fp16 SDPA; here it is applied against float64.
#   bf16: 8 mantissa bits instead of 11, so P, dS and the outputs round 8x coarser.
#   atol_rel: errors scale with the data. D = rowsum(dO * O) is built from the 16-bit rounded O (as
#         in the reference, flash_attn.cu:388) and P / dS are rounded to 16 bits before their
#         products, so with inputs x3 (config 3) gradients reach ~35 and their errors grow with
#         them; about 2 half-ulps of the tensor's largest magnitude covers that.
TOL = {
    torch.float16: dict(rtol=2e-2, atol=2e-2, atol_rel=2e-3, fro=5e-3),
    torch.bfloat16: dict(rtol=5e-2, atol=6e-2, atol_rel=1.5e-2, fro=1e-2),
}
TOL_GRAD = {
    torch.float16: dict(rtol=2e-2, atol=2e-2, atol_rel=2e-3, fro=5e-3),
    torch.bfloat16: dict(rtol=5e-2, atol=1e-1, atol_rel=1.5e-2, fro=1e-2),
}
LSE_ATOL = 1e-2  # natural-log units; config 3 (inputs x3) asks for lse within 1e-2


def make_inputs(B, H, KVH, T, D, dtype, mult=1.0, seed=0):
    """Seeded CPU inputs in the reference's draw order (q, k, v, then dO), rounded to ``dtype``."""
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, H, T, D, generator=g) * mult).to(dtype)
    k = (torch.randn(B, KVH, T, D, generator=g) * mult).to(dtype)
    v = (torch.randn(B, KVH, T, D, generator=g) * mult).to(dtype)
    do = torch.randn(B, H, T, D, generator=g).to(dtype)
    return q, k, v, do


def load_golden(name: str) -> dict:
    z = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    dtype = getattr(torch, str(z["dtype"]))
    out = {"shape": tuple(int(x) for x in z["shape"]), "dtype": dtype, "mult": float(z["mult"])}
    for key in ("q", "k", "v", "do"):
        out[key] = torch.from_numpy(z[key].view(np.int16).copy()).view(dtype)
    for key in ("o", "lse", "dq", "dk", "dv"):
        out[key] = torch.from_numpy(z[key].astype(np.float64))
    return out


def golden_names() -> list[str]:
    return sorted(p.stem for p in GOLDEN.glob("*.npz"))


def errors(x: torch.Tensor, ref: torch.Tensor) -> dict:
    x = x.double().cpu()
    ref = ref.double().cpu()
    diff = (x - ref).abs()
    # Relative to the reference's norm, floored at an RMS of 1e-3 so that an all-zero reference
    # (e.g. dq and dk at T = 1) compares on absolute error instead of dividing by zero.
    floor = 1e-3 * max(ref.numel(), 1) ** 0.5
    fro = (diff.norm() / ref.norm().clamp_min(floor)).item()
    return {"max_abs": diff.max().item() if diff.numel() else 0.0, "rel_fro": fro}


def assert_close_tol(x: torch.Tensor, ref: torch.Tensor, tol: dict, what: str = "") -> dict:
    x = x.double().cpu()
    ref = ref.double().cpu()
    e = errors(x, ref)
    print(f"[err] {what}: max_abs={e['max_abs']:.3e} rel_fro={e['rel_fro']:.3e}", flush=True)
    atol = max(tol["atol"], tol["atol_rel"] * (ref.abs().max().item() if ref.numel() else 0.0))
    torch.testing.assert_close(x, ref, rtol=tol["rtol"], atol=atol, msg=lambda m: f"{what}: {m} {e}")
    assert e["rel_fro"] <= tol["fro"], f"{what}: relative Frobenius error {e['rel_fro']:.3e} > {tol['fro']:.1e}"
    return e
