"""GPU parity of the HIP kernels against the float64 oracle and the committed golden fixtures.

Mirrors the reference's kernel tests (/root/reference/tests/kernels/test_flash_attn.py:31-78): parity of
the output and all three input gradients over its SHAPES, the causal-leak test (bit-exact prefix),
opcheck, torch.compile(fullgraph=True) with contiguous and strided inputs. Adds: bf16, the golden
fixtures, ragged T / every GQA group size / both head dims, HIP-graph capture and replay, and the
BASELINE configs 2-4 at full size against a float32 PyTorch reference on the GPU.

Every comparison is against a higher-precision reference on the SAME rounded 16-bit inputs; tolerances
are in tests/common.py (TOL, TOL_GRAD, LSE_ATOL).
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import attention as oracle
from tests.common import (
    LSE_ATOL,
    REF_SHAPES,
    TOL,
    TOL_GRAD,
    assert_close_tol,
    errors,
    golden_names,
    load_golden,
    make_inputs,
)

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _fa():
    from nanonemo_amd.kernels.hip import flash_attn as fa

    return fa


def _run(q, k, v, do):
    """Forward + backward through the ops on the GPU; returns CPU tensors (o, lse, dq, dk, dv)."""
    fa = _fa()
    q, k, v = (t.to(DEV).requires_grad_() for t in (q, k, v))
    o, lse = fa._flash_attn(q, k, v)
    o.backward(do.to(DEV))
    torch.cuda.synchronize()
    return o.detach().cpu(), lse.cpu(), q.grad.cpu(), k.grad.cpu(), v.grad.cpu()


# Accuracy relative to PyTorch's own attention: the kernel's error against the reference, next to PyTorch's own
# attention in the same dtype on the same rounded inputs, measured in the same run, on max-abs and relative-Frobenius
# error:
#   * at most SDPA_RATIO times the error of PyTorch's FlashAttention kernel (SDPA's flash backend, else its
#     mem-efficient one): the same algorithm class, which like this kernel (and the reference's,
#     /root/reference/nanonemo/kernels/cuda/flash_attn.cu:129-138,287-293) rounds P and dS to 16 bits before their
#     products and builds D from the 16-bit o;
#   * at most SDPA_MATH_RATIO times the error of SDPA's math backend, which computes in fp32 and rounds only its
#     outputs. dq is where the two differ: dq = scale * sum_j dS_ij K_j with sum_j dS_ij = 0, so the 16-bit rounding
#     of dS shows through the cancellation (measured up to 2.7x max-abs and 3.3x relative-Frobenius at inputs x3, the
#     same ratios PyTorch's own flash kernel shows against the math path).
# SDPA_FLOOR absorbs max-abs errors at the level of fp32 rounding noise (dq at T = 1, which both SDPA paths return as
# exact zeros); the relative-Frobenius ratio is not taken for an all-zero reference.
SDPA_RATIO = 2.0
SDPA_MATH_RATIO = 4.0
SDPA_FLOOR = 1e-5


def _sdpa(q, k, v, do, backends):
    """PyTorch's attention in the inputs' dtype on the GPU: repeat_interleave'd K/V through SDPA restricted to the
    first of ``backends`` that runs, with autograd; returns (backend name, (o, dq, dk, dv) on the CPU)."""
    from torch.nn.attention import sdpa_kernel

    group = q.shape[1] // k.shape[1]
    for backend in backends:
        qs, ks, vs = (t.to(DEV).requires_grad_() for t in (q, k, v))
        try:
            with sdpa_kernel(backend):
                o = torch.nn.functional.scaled_dot_product_attention(
                    qs, ks.repeat_interleave(group, dim=1), vs.repeat_interleave(group, dim=1), is_causal=True)
        except RuntimeError:  # the backend does not take this shape or dtype
            continue
        grads = torch.autograd.grad(o, (qs, ks, vs), do.to(DEV))
        torch.cuda.synchronize()
        return backend.name, tuple(t.detach().cpu() for t in (o, *grads))
    raise RuntimeError(f"no SDPA backend of {backends} ran")


def _sdpa_bound(report, refs, inputs, label):
    """Assert the bounds relative to PyTorch's attention (see SDPA_RATIO) for o, dq, dk, dv and print the ratios."""
    from torch.nn.attention import SDPBackend

    lines = []
    for backends, ratio in (((SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION), SDPA_RATIO),
                            ((SDPBackend.MATH,), SDPA_MATH_RATIO)):
        name, outs = _sdpa(*inputs, backends)
        parts = []
        for n, x in zip(("o", "dq", "dk", "dv"), outs):
            r = refs[n]
            es = errors(x, r)
            ours = report[n]
            metrics = ("max_abs", "rel_fro") if bool((r != 0).any()) else ("max_abs",)
            for m in metrics:
                floor = SDPA_FLOOR if m == "max_abs" else 0.0
                assert ours[m] <= ratio * es[m] + floor, (
                    f"{label} {n}: {m} {ours[m]:.3e} is more than {ratio} x SDPA {name}'s {es[m]:.3e}")
            parts.append(f"{n} {ours['max_abs'] / max(es['max_abs'], SDPA_FLOOR):.2f}x/"
                         f"{ours['rel_fro'] / max(es['rel_fro'], 1e-12):.2f}x")
        lines.append(f"vs {name} (bound {ratio}x): " + ", ".join(parts))
    print(f"[sdpa] {label} (max-abs/rel-fro ratios) " + "; ".join(lines), flush=True)


def _check(got, ref, dtype, label, inputs=None):
    """Tolerances of tests/common.py against ``ref``; with ``inputs`` (the rounded q, k, v, dO) also the bounds
    relative to PyTorch's same-dtype attention (SDPA_RATIO) for o, dq, dk, dv."""
    o, lse, dq, dk, dv = got
    ro, rlse, rdq, rdk, rdv = ref
    assert o.dtype == dtype and dq.dtype == dtype and dk.dtype == dtype and dv.dtype == dtype
    report = {"o": assert_close_tol(o, ro, TOL[dtype], f"{label} o")}
    e = errors(lse, rlse)
    assert e["max_abs"] <= LSE_ATOL, f"{label} lse {e}"
    report["lse"] = e
    for name, x, r in (("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv)):
        report[name] = assert_close_tol(x, r, TOL_GRAD[dtype], f"{label} {name}")
    print(f"\n[parity] {label}: " + ", ".join(f"{k} max_abs={v['max_abs']:.2e} fro={v['rel_fro']:.1e}" for k, v in report.items()), flush=True)
    if inputs is not None:
        _sdpa_bound(report, {"o": ro, "dq": rdq, "dk": rdk, "dv": rdv}, inputs, label)


def _oracle(q, k, v, do):
    qd, kd, vd, dod = (t.double().numpy() for t in (q, k, v, do))
    o, lse = oracle.forward(qd, kd, vd)
    dq, dk, dv = oracle.backward(dod, qd, kd, vd, o, lse)
    return tuple(torch.from_numpy(x) for x in (o, lse, dq, dk, dv))


@pytest.mark.parametrize("name", golden_names())
def test_golden_fixture(name):
    g = load_golden(name)
    got = _run(g["q"], g["k"], g["v"], g["do"])
    _check(got, tuple(g[x] for x in ("o", "lse", "dq", "dk", "dv")), g["dtype"], f"golden {name}",
           inputs=(g["q"], g["k"], g["v"], g["do"]))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B, H, KVH, T, hd", REF_SHAPES)
def test_matches_oracle(B, H, KVH, T, hd, dtype):
    q, k, v, do = make_inputs(B, H, KVH, T, hd, dtype, seed=0)
    _check(_run(q, k, v, do), _oracle(q, k, v, do), dtype, f"{(B, H, KVH, T, hd)} {dtype}", inputs=(q, k, v, do))


# Ragged lengths around every tile size (64-key forward tiles, 128-query forward blocks, 64-query /
# 128-key backward tiles), every group size of 12 query heads, and both head dims.
EDGE = [
    (1, 1, 1, 2, 64),
    (1, 2, 1, 63, 64),
    (1, 2, 2, 64, 32),
    (1, 3, 1, 65, 64),
    (2, 4, 2, 127, 64),
    (1, 6, 3, 128, 32),
    (1, 12, 1, 129, 64),
    (1, 12, 6, 191, 64),
    (1, 12, 12, 257, 32),
    (1, 4, 4, 300, 64),
    (1, 6, 2, 513, 64),
]


@pytest.mark.parametrize("B, H, KVH, T, hd", EDGE)
def test_edge_shapes(B, H, KVH, T, hd):
    dtype = torch.bfloat16
    q, k, v, do = make_inputs(B, H, KVH, T, hd, dtype, seed=T)
    _check(_run(q, k, v, do), _oracle(q, k, v, do), dtype, f"edge {(B, H, KVH, T, hd)}")


def _random_shapes(n, seed=2024):
    """n seeded (B, H, KVH, T, hd, dtype) draws: T in 1..400, every divisor of H as KVH, both head dims."""
    import random

    rng = random.Random(seed)
    out = []
    for i in range(n):
        H = rng.choice([1, 2, 3, 4, 6, 8, 12, 16])
        KVH = rng.choice([d for d in range(1, H + 1) if H % d == 0])
        out.append((rng.choice([1, 2]), H, KVH, rng.randint(1, 400), rng.choice([32, 64]),
                    (torch.bfloat16, torch.float16)[i % 2]))
    return out


@pytest.mark.parametrize("B, H, KVH, T, hd, dtype", _random_shapes(16))
def test_random_shapes_match_oracle(B, H, KVH, T, hd, dtype):
    q, k, v, do = make_inputs(B, H, KVH, T, hd, dtype, seed=1000 + T)
    _check(_run(q, k, v, do), _oracle(q, k, v, do), dtype, f"random {(B, H, KVH, T, hd, dtype)}")


def test_long_sequence_prefix_and_zero_tail():
    """T=65536 (B=1, 12 Q / 4 KV heads, d=64, bf16), checked through properties that hold at any length.

    * Causal prefix: o, lse and dq of the first P rows depend only on rows and keys < P, so they are bit-identical
      to a run on the P-row prefix.
    * dO is zero past row P, so every dS of those rows is 0. dK/dV of keys < P then match the prefix run's, up to the
      order of their fp32 sums (the two shapes split the work differently), and dK/dV of keys >= P are exactly 0.
    * Each output row is a convex combination of V rows, so it stays within V's range.
    """
    torch.manual_seed(7)
    B, H, KVH, T, hd, P = 1, 12, 4, 65536, 64, 1024
    dt = torch.bfloat16
    q = torch.randn(B, H, T, hd, device=DEV).to(dt)
    k = torch.randn(B, KVH, T, hd, device=DEV).to(dt)
    v = torch.randn(B, KVH, T, hd, device=DEV).to(dt)
    do = torch.randn(B, H, T, hd, device=DEV).to(dt)
    do[:, :, P:] = 0
    fa = _fa()
    o, lse = fa._flash_attn(q, k, v)
    dq, dk, dv = fa._flash_attn_bwd(do, q, k, v, o, lse)
    qp, kp, vp, dop = (t[:, :, :P].contiguous() for t in (q, k, v, do))
    op_, lsep = fa._flash_attn(qp, kp, vp)
    dqp, dkp, dvp = fa._flash_attn_bwd(dop, qp, kp, vp, op_, lsep)
    torch.cuda.synchronize()
    assert torch.equal(o[:, :, :P], op_) and torch.equal(lse[:, :, :P], lsep)
    assert torch.equal(dq[:, :, :P], dqp)
    assert not dq[:, :, P:].any() and not dk[:, :, P:].any() and not dv[:, :, P:].any()
    assert_close_tol(dk[:, :, :P], dkp, TOL_GRAD[dt], "dk prefix")
    assert_close_tol(dv[:, :, :P], dvp, TOL_GRAD[dt], "dv prefix")
    assert torch.isfinite(lse).all() and torch.isfinite(o).all()
    vmax = v.float().abs().amax(dim=(0, 2)).repeat_interleave(H // KVH, dim=0)  # [H, hd]
    assert (o.float().abs() <= vmax[None, :, None, :] * (1 + 2 ** -7) + 1e-6).all()


@pytest.mark.parametrize("B, T", [(0, 64), (2, 0)])
def test_empty_problem_through_the_ops(B, T):
    """No batch or no rows: both layouts' forward and backward return empty results of the right shapes."""
    fa = _fa()
    q = torch.randn(B, 12, T, 64, device=DEV).to(torch.bfloat16).requires_grad_()
    k = torch.randn(B, 4, T, 64, device=DEV).to(torch.bfloat16).requires_grad_()
    v = torch.randn(B, 4, T, 64, device=DEV).to(torch.bfloat16).requires_grad_()
    o, lse = fa._flash_attn(q, k, v)
    assert o.shape == q.shape and lse.shape == (B, 12, T) and lse.dtype == torch.float32
    dq, dk, dv = torch.autograd.grad(o, (q, k, v), torch.ones_like(o))
    assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape
    qt, kt, vt = (t.detach().transpose(1, 2).contiguous().requires_grad_() for t in (q, k, v))
    ot = fa.flash_attn_bthd(qt, kt, vt)
    assert ot.shape == qt.shape
    grads = torch.autograd.grad(ot, (qt, kt, vt), torch.ones_like(ot))
    assert [g.shape for g in grads] == [qt.shape, kt.shape, vt.shape]
    torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_extreme_score_range_matches_oracle(dtype):
    # Inputs x12: scores with standard deviation ~144, so a row's running max jumps by hundreds (base 2)
    # between sub-tiles; the forward's p against the stale max overflows to inf there, which must send the
    # wave through its rescale path. Softmax is nearly one-hot; O, lse and every gradient still follow
    # the float64 oracle on the same rounded inputs.
    mult = 12.0 if dtype == torch.bfloat16 else 4.0  # fp16 q*k products stay far below its range at x4
    q, k, v, do = make_inputs(1, 4, 2, 300, 64, dtype, mult=mult, seed=5)
    got = _run(q, k, v, do)
    assert all(torch.isfinite(t).all() for t in got)
    _check(got, _oracle(q, k, v, do), dtype, f"extreme x{mult:g} {dtype}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rows_past_T_with_a_very_negative_last_lse(dtype):
    # T % 64 != 0, so the last 64-row query tile has rows past T, and the last row's scores are all about
    # -110 (natural-log units): keys are positive, and q[T-1] = -12. Its lse is then about -105, and a row
    # past T that started its scores from that lse (zero Q) would get p = e^105, which overflows fp32. Such
    # rows must contribute nothing: every output finite and on the float64 oracle.
    B, H, KVH, T, hd = 1, 4, 2, 300, 64
    q, k, v, do = make_inputs(B, H, KVH, T, hd, dtype, seed=7)
    k = (k.float().abs() + 0.5).to(dtype)
    q[:, :, T - 1, :] = -12.0
    got = _run(q, k, v, do)
    assert all(torch.isfinite(t).all() for t in got)
    assert got[1][:, :, T - 1].max() < -100.0  # the case is the intended one
    _check(got, _oracle(q, k, v, do), dtype, f"rows past T, very negative last lse {dtype}")


def test_causal_future_keys_dont_leak():
    # Changing a key/value strictly after position i must not change output i (bit-exact).
    fa = _fa()
    for dtype in (torch.float16, torch.bfloat16):
        q, k, v, _ = (t.to(DEV) for t in make_inputs(1, 4, 1, 200, 64, dtype))
        y = fa.flash_attn(q, k, v)
        k2, v2 = k.clone(), v.clone()
        k2[:, :, 70:] = torch.randn_like(k2[:, :, 70:])
        v2[:, :, 70:] = torch.randn_like(v2[:, :, 70:])
        y2 = fa.flash_attn(q, k2, v2)
        torch.testing.assert_close(y[:, :, :70], y2[:, :, :70], rtol=0, atol=0)
        assert not torch.equal(y[:, :, 70:], y2[:, :, 70:])


def test_deterministic_forward():
    fa = _fa()
    q, k, v, _ = (t.to(DEV) for t in make_inputs(2, 12, 4, 333, 64, torch.bfloat16))
    assert torch.equal(fa.flash_attn(q, k, v), fa.flash_attn(q, k, v))


# Shapes whose dK/dV work units (B * KVH * ceil(T / 128)) are too few to fill the chip, so that each unit
# pair is split over several blocks whose fp32 partials are summed afterwards (16 and 9 splits here).
SPLIT = [(2, 12, 1, 1024, 64), (1, 12, 2, 700, 32)]


@pytest.mark.parametrize("B, H, KVH, T, hd", SPLIT)
def test_split_dkdv_matches_oracle(B, H, KVH, T, hd):
    dtype = torch.bfloat16
    q, k, v, do = make_inputs(B, H, KVH, T, hd, dtype, seed=11)
    _check(_run(q, k, v, do), _oracle(q, k, v, do), dtype, f"split {(B, H, KVH, T, hd)}")


# Shapes with enough unit pairs that fewer waves share each (B*KVH*ceil(T/128) >= 768: one wave per pair, four
# pairs per block; >= 512: two waves per pair). The second leaves two waves of its last block idle (130
# pairs), the third one pair in its last block (91 pairs of two).
WPP = [(12, 8, 8, 1024, 32), (65, 4, 2, 700, 32), (91, 2, 1, 700, 32)]


@pytest.mark.parametrize("B, H, KVH, T, hd", WPP)
def test_fewer_waves_per_unit_pair_matches_oracle(B, H, KVH, T, hd):
    dtype = torch.bfloat16
    q, k, v, do = make_inputs(B, H, KVH, T, hd, dtype, seed=13)
    _check(_run(q, k, v, do), _oracle(q, k, v, do), dtype, f"waves per pair {(B, H, KVH, T, hd)}")


# Small unsplit shapes whose dK/dV blocks take single units (B * KVH * ceil(T / 64) units): one per block (config
# 1's shape, 16 units), or two per block with two waves each (512 and 396 units; the second leaves two waves of its
# last block idle).
SINGLE_UNITS = [(1, 12, 4, 256, 64, torch.bfloat16), (32, 12, 4, 256, 64, torch.bfloat16),
                (33, 3, 3, 256, 32, torch.float16), (64, 12, 4, 128, 64, torch.float16)]


@pytest.mark.parametrize("B, H, KVH, T, hd, dtype", SINGLE_UNITS)
def test_single_unit_dkdv_blocks_match_oracle(B, H, KVH, T, hd, dtype):
    q, k, v, do = make_inputs(B, H, KVH, T, hd, dtype, seed=17)
    _check(_run(q, k, v, do), _oracle(q, k, v, do), dtype, f"single units {(B, H, KVH, T, hd, dtype)}")


# Paired dK/dV blocks with four waves whose K / V rows go through LDS (head_dim 64, at most 32 units per head)
# and an odd unit count, so that the middle block carries one unit alone (it takes its K / V through LDS too):
# 15 and 31 units per head. Against the float32 reference on the GPU (the float64 oracle is slow at these sizes).
KVL_ODD = [(8, 12, 4, 960, 64, torch.bfloat16), (4, 12, 4, 1984, 64, torch.float16)]


@pytest.mark.parametrize("B, H, KVH, T, hd, dtype", KVL_ODD)
def test_paired_kv_through_lds_with_a_middle_unit(B, H, KVH, T, hd, dtype):
    import ctypes

    from nanonemo_amd.kernels.hip import lib

    n, w, p, g = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int64()
    assert lib().nn_fa_bwd_plan(B, H, KVH, T, ctypes.byref(n), ctypes.byref(w), ctypes.byref(p), ctypes.byref(g)) == 0
    assert (n.value, w.value, p.value) == (1, 4, 1), (n.value, w.value, p.value)  # unsplit, paired, 4 waves
    print(f"\n[case] paired K/V-through-LDS dK/dV with a middle unit {(B, H, KVH, T, hd, dtype)}", flush=True)
    torch.manual_seed(21)
    q, do = (torch.randn(B, H, T, hd, device=DEV).to(dtype) for _ in range(2))
    k, v = (torch.randn(B, KVH, T, hd, device=DEV).to(dtype) for _ in range(2))
    fa = _fa()
    qs, ks, vs = (t.clone().requires_grad_() for t in (q, k, v))
    o, lse = fa._flash_attn(qs, ks, vs)
    dq, dk, dv = torch.autograd.grad(o, (qs, ks, vs), do)
    got = (o.detach(), lse, dq, dk, dv)
    ref = _torch_fp32_reference(q, k, v, do)
    _check(tuple(t.cpu() for t in got), tuple(t.cpu() for t in ref), dtype, f"kvl odd {(B, H, KVH, T, hd, dtype)}",
           inputs=(q, k, v, do))
    del ref
    torch.cuda.empty_cache()


# A plain shape, an fp16 head_dim-32 MQA shape whose dK/dV work is split, and a bf16 split shape.
SEPARATE = [(2, 12, 4, 300, 64, torch.bfloat16), (1, 12, 1, 700, 32, torch.float16), (2, 12, 1, 1024, 64, torch.bfloat16)]


@pytest.mark.parametrize("B, H, KVH, T, hd, dtype", SEPARATE)
def test_separate_backward_entry_points(B, H, KVH, T, hd, dtype):
    """nn_fa_bwd_pre then nn_fa_bwd_dkdv, and nn_fa_bwd_dq, called on their own through the C ABI, give the
    gradients of nn_fa_bwd (which runs nn_fa_bwd_dq's kernel, with the preprocessing fused, then dK/dV's).
    dq is the same kernel on the same inputs: bit for bit. dk and dv match the oracle; against nn_fa_bwd's they
    differ only in rounding, because the standalone pass sums D = rowsum(dO * o) in another order."""
    from nanonemo_amd.kernels.hip import DTYPE_BF16, DTYPE_F16, check, lib

    L = lib()
    dt = DTYPE_BF16 if dtype == torch.bfloat16 else DTYPE_F16
    print(f"\n[case] separate backward entry points B={B} H={H} KVH={KVH} T={T} hd={hd} {dtype}", flush=True)
    qc, kc, vc, doc = make_inputs(B, H, KVH, T, hd, dtype, seed=5)
    q, k, v, do = (t.to(DEV) for t in (qc, kc, vc, doc))
    o, lse = torch.empty_like(q), torch.empty(B, H, T, device=DEV)
    scale = 1.0 / math.sqrt(hd)
    st = torch.cuda.current_stream().cuda_stream
    p = lambda t: t.data_ptr()  # noqa: E731
    check(L.nn_fa_fwd(p(q), p(k), p(v), p(o), p(lse), B, H, KVH, T, hd, dt, scale, st))
    wsb = L.nn_fa_bwd_workspace_size(B, H, KVH, T, hd)
    ws, ws2 = (torch.empty(wsb, dtype=torch.uint8, device=DEV) for _ in range(2))
    dq, dq2 = torch.empty_like(q), torch.empty_like(q)
    dk, dk2, dv, dv2 = torch.empty_like(k), torch.empty_like(k), torch.empty_like(v), torch.empty_like(v)
    check(L.nn_fa_bwd(p(do), p(q), p(k), p(v), p(o), p(lse), p(dq), p(dk), p(dv), p(ws), wsb, B, H, KVH, T, hd,
                      dt, scale, st))
    check(L.nn_fa_bwd_pre(p(o), p(do), p(lse), p(ws2), wsb, B, H, KVH, T, hd, dt, scale, st))
    check(L.nn_fa_bwd_dkdv(p(q), p(k), p(v), p(do), p(ws2), wsb, p(dk2), p(dv2), B, H, KVH, T, hd, dt, scale, st))
    check(L.nn_fa_bwd_dq(p(q), p(k), p(v), p(o), p(do), p(lse), p(ws2), wsb, p(dq2), B, H, KVH, T, hd, dt, scale,
                         st))
    torch.cuda.synchronize()
    assert torch.equal(dq2, dq)
    ro, rlse = oracle.forward(*(t.double().numpy() for t in (qc, kc, vc)))
    _, rdk, rdv = oracle.backward(*(t.double().numpy() for t in (doc, qc, kc, vc)), ro, rlse)
    for name, x, x_fused, r in (("dk", dk2, dk, rdk), ("dv", dv2, dv, rdv)):
        assert_close_tol(x.cpu(), torch.from_numpy(r), TOL_GRAD[dtype], f"separate {name}")
        e = errors(x.double().cpu(), x_fused.double().cpu())
        assert e["rel_fro"] <= 2e-3, f"separate {name} vs nn_fa_bwd: {e}"


def test_deterministic_backward():
    # The backward has no atomics: the split dK/dV partials are summed in split order, the unsplit ones
    # through LDS in wave order, so repeated calls agree bit for bit.
    fa = _fa()
    for shape in (SPLIT[0], (8, 12, 4, 1024, 64)):
        q, k, v, do = (t.to(DEV) for t in make_inputs(*shape, torch.bfloat16, seed=3))
        o, lse = fa._flash_attn(q, k, v)
        g1 = fa._flash_attn_bwd(do, q, k, v, o, lse)
        g2 = fa._flash_attn_bwd(do, q, k, v, o, lse)
        assert all(torch.equal(a, b) for a, b in zip(g1, g2)), shape


def test_backward_when_only_lse_is_used():
    # lse's gradient is ignored (as in the reference), and autograd passes no gradient for an unused o: the
    # backward then runs on a zero dO, so every input gradient is exactly zero.
    fa = _fa()
    q, k, v, _ = (t.to(DEV).requires_grad_() for t in make_inputs(2, 12, 4, 200, 64, torch.bfloat16, seed=4))
    _, lse = fa._flash_attn(q, k, v)
    lse.sum().backward()
    for t in (q, k, v):
        assert t.grad is not None and torch.equal(t.grad, torch.zeros_like(t))
    # and with o used, autograd's result is the backward op's on the same dO, bit for bit
    q2, k2, v2 = (t.detach().clone().requires_grad_() for t in (q, k, v))
    do = torch.randn_like(q)
    o = fa.flash_attn(q2, k2, v2)
    o.backward(do)
    o_, lse_ = fa._flash_attn(q.detach(), k.detach(), v.detach())
    for a, b in zip((q2.grad, k2.grad, v2.grad), fa._flash_attn_bwd(do, q.detach(), k.detach(), v.detach(), o_, lse_)):
        assert torch.equal(a, b)


def test_opcheck():
    fa = _fa()
    for dtype in (torch.float16, torch.bfloat16):
        q, k, v, _ = (t.to(DEV).requires_grad_() for t in make_inputs(1, 4, 2, 48, 32, dtype))
        torch.library.opcheck(fa._flash_attn, (q, k, v))


def test_compiles_without_graph_breaks():
    fa = _fa()
    q, k, v, _ = (t.to(DEV) for t in make_inputs(2, 12, 4, 64, 64, torch.bfloat16))
    torch._dynamo.reset()
    fn = torch.compile(fa.flash_attn, fullgraph=True)
    torch.testing.assert_close(fn(q, k, v), fa.flash_attn(q, k, v), rtol=0, atol=0)


def test_compiles_with_strided_inputs():
    # In the model q/k arrive as transposed views; the fake impl must match the real output strides.
    fa = _fa()
    q, k, v, _ = make_inputs(2, 12, 4, 64, 64, torch.float16)
    q, k, v = (t.to(DEV).transpose(1, 2).contiguous().transpose(1, 2).requires_grad_() for t in (q, k, v))
    assert not q.is_contiguous()
    torch._dynamo.reset()
    y = torch.compile(fa.flash_attn, fullgraph=True)(q, k, v)
    y.sum().backward()
    torch.testing.assert_close(y, fa.flash_attn(q, k, v), rtol=0, atol=0)
    assert q.grad is not None and q.grad.shape == q.shape


@pytest.mark.skip(
    reason="capturing fwd+bwd (with autograd) in torch.cuda.graph ended in a host segmentation fault inside "
    "capture_end on the MI355X box; no cause has been shown in this code yet, so the case stays off the GPU and the "
    "ops refuse it before any launch (tests/test_boundary.py::test_capture_through_autograd_is_refused)"
)
def test_hip_graph_capture_and_replay():
    # fwd+bwd captured once, replayed several times with eager work in between; every replay must
    # equal the eager result bit for bit (the library allocates, syncs and copies nothing itself).
    fa = _fa()
    dtype = torch.bfloat16
    q, k, v, do = (t.to(DEV) for t in make_inputs(2, 12, 4, 256, 64, dtype, seed=1))
    qs, ks, vs = (t.clone().requires_grad_() for t in (q, k, v))

    def step():
        o = fa.flash_attn(qs, ks, vs)
        return (o, *torch.autograd.grad(o, (qs, ks, vs), do))

    ref = [t.clone() for t in step()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    for i in range(4):
        junk = torch.randn(1 << 20, device=DEV) * i  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs, ref):
            assert torch.equal(a, b), f"replay {i} differs from eager"
        del junk


# ---- BASELINE configs at full size, against a float32 reference on the GPU -------------------


def _torch_fp32_reference(q, k, v, do):
    """Explicit matmul + masked softmax in float32 with autograd (the reference's math path, fp32)."""
    qf, kf, vf = (t.float().requires_grad_() for t in (q, k, v))
    group = q.shape[1] // k.shape[1]
    kr = kf.repeat_interleave(group, dim=1)
    vr = vf.repeat_interleave(group, dim=1)
    T = q.shape[2]
    s = torch.matmul(qf, kr.transpose(-1, -2).contiguous()) / math.sqrt(q.shape[-1])
    s = s.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool, device=q.device), 1), float("-inf"))
    lse = torch.logsumexp(s, -1)
    o = torch.matmul(torch.softmax(s, -1), vr)
    dq, dk, dv = torch.autograd.grad(o, (qf, kf, vf), do.float())
    return tuple(t.detach() for t in (o, lse, dq, dk, dv))


@pytest.mark.parametrize(
    "B, H, KVH, T, hd, dtype, mult",
    [
        (8, 12, 4, 1024, 64, torch.float16, 1.0),  # config 2
        (8, 12, 4, 1024, 64, torch.bfloat16, 1.0),  # the north-star shape in bf16
        (32, 12, 4, 1024, 64, torch.bfloat16, 3.0),  # config 3
        (2, 12, 4, 8192, 64, torch.bfloat16, 1.0),  # config 4
    ],
)
def test_baseline_configs_full_size(B, H, KVH, T, hd, dtype, mult):
    torch.manual_seed(0)
    q = (torch.randn(B, H, T, hd, device=DEV) * mult).to(dtype)
    k = (torch.randn(B, KVH, T, hd, device=DEV) * mult).to(dtype)
    v = (torch.randn(B, KVH, T, hd, device=DEV) * mult).to(dtype)
    do = torch.randn(B, H, T, hd, device=DEV).to(dtype)
    fa = _fa()
    qs, ks, vs = (t.clone().requires_grad_() for t in (q, k, v))
    o, lse = fa._flash_attn(qs, ks, vs)
    dq, dk, dv = torch.autograd.grad(o, (qs, ks, vs), do)
    got = (o.detach(), lse, dq, dk, dv)
    ref = _torch_fp32_reference(q, k, v, do)
    _check(tuple(t.cpu() for t in got), tuple(t.cpu() for t in ref), dtype, f"config {(B, H, KVH, T, hd, dtype, mult)}",
           inputs=(q, k, v, do))
    del ref
    torch.cuda.empty_cache()
