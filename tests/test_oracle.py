"""Pins the float64 oracle (oracle/attention.py) without the GPU.

The reference holds no golden vectors for attention, so the oracle is pinned by checks that do not
retype its formulas:
  * torch's scaled_dot_product_attention (math backend) with repeat_interleave of K/V, the reference's
    own plain-PyTorch attention (/root/reference/tests/kernels/test_flash_attn.py:24-28,
    nanonemo/model/layers.py:109-115), and torch autograd through it, all in float64;
  * brute-force Python loops on tiny shapes (the per-head loop of
    /root/reference/tests/model/test_layers.py:107-123, written element by element);
  * closed forms: T = 1, Q = 0, GQA == MHA on repeated K/V with group-summed gradients, and
    causality (a future perturbation leaves the prefix bit-identical, test_flash_attn.py:48-56);
  * planted mistakes (wrong KV-head mapping, wrong mask diagonal, dropped D term, mean instead of
    group sum, missing scale) that these checks must catch.
"""

from __future__ import annotations

import itertools
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as A
from tests.common import golden_names, load_golden, make_inputs


def _rand(B, H, KVH, T, D, seed=0, mult=1.0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, H, T, D)) * mult
    k = rng.standard_normal((B, KVH, T, D)) * mult
    v = rng.standard_normal((B, KVH, T, D)) * mult
    do = rng.standard_normal((B, H, T, D))
    return q, k, v, do


def _torch_reference(q, k, v, do):
    """The reference's plain-PyTorch attention (repeat_interleave + SDPA math), fp64, with autograd."""
    tq, tk, tv = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v))
    group = tq.shape[1] // tk.shape[1]
    with torch.nn.attention.sdpa_kernel(torch.nn.attention.SDPBackend.MATH):
        o = F.scaled_dot_product_attention(
            tq, tk.repeat_interleave(group, dim=1), tv.repeat_interleave(group, dim=1), is_causal=True
        )
    o.backward(torch.tensor(do))
    s = tq @ tk.repeat_interleave(group, dim=1).transpose(-1, -2) / math.sqrt(q.shape[-1])
    T = q.shape[2]
    s = s.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
    lse = torch.logsumexp(s, -1)
    return (o.detach().numpy(), lse.detach().numpy(), tq.grad.numpy(), tk.grad.numpy(), tv.grad.numpy())


SHAPES = [(1, 4, 1, 16, 32), (2, 4, 4, 37, 64), (1, 1, 1, 1, 32), (3, 8, 2, 65, 32), (1, 12, 4, 128, 64)]


def _check_against_torch(shape, seed=0, mult=1.0):
    q, k, v, do = _rand(*shape, seed=seed, mult=mult)
    o, lse = A.forward(q, k, v)
    dq, dk, dv = A.backward(do, q, k, v, o, lse)
    ro, rlse, rdq, rdk, rdv = _torch_reference(q, k, v, do)
    for name, x, r in (("o", o, ro), ("lse", lse, rlse), ("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv)):
        np.testing.assert_allclose(x, r, rtol=1e-10, atol=1e-10, err_msg=name)


@pytest.mark.parametrize("shape", SHAPES)
def test_matches_torch_sdpa_and_autograd(shape):
    _check_against_torch(shape)


def test_matches_torch_with_large_scores():
    # Config 3 multiplies the inputs by 3 (score std ~ 9): a peaked softmax.
    _check_against_torch((1, 6, 2, 96, 64), seed=3, mult=3.0)


def _brute_force(q, k, v, do):
    """Element-by-element loops: softmax by hand per (b, h, i), gradients from the chain rule."""
    B, H, T, D = q.shape
    KVH = k.shape[1]
    group = H // KVH
    sc = 1.0 / math.sqrt(D)
    o = np.zeros_like(q)
    lse = np.zeros((B, H, T))
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    for b, h, i in itertools.product(range(B), range(H), range(T)):
        kh = h // group
        s = [sum(q[b, h, i, d] * k[b, kh, j, d] for d in range(D)) * sc for j in range(i + 1)]
        mx = max(s)
        w = [math.exp(x - mx) for x in s]
        z = sum(w)
        p = [x / z for x in w]
        lse[b, h, i] = mx + math.log(z)
        for d in range(D):
            o[b, h, i, d] = sum(p[j] * v[b, kh, j, d] for j in range(i + 1))
        # dL/dp_j = dO_i . v_j ; softmax Jacobian: ds_j = p_j (dp_j - sum_l p_l dp_l)
        dp = [sum(do[b, h, i, d] * v[b, kh, j, d] for d in range(D)) for j in range(i + 1)]
        dot = sum(p[j] * dp[j] for j in range(i + 1))
        for j in range(i + 1):
            ds = p[j] * (dp[j] - dot)
            for d in range(D):
                dq[b, h, i, d] += ds * k[b, kh, j, d] * sc
                dk[b, kh, j, d] += ds * q[b, h, i, d] * sc
                dv[b, kh, j, d] += p[j] * do[b, h, i, d]
    return o, lse, dq, dk, dv


@pytest.mark.parametrize("shape", [(1, 2, 1, 5, 4), (2, 4, 2, 3, 2), (1, 3, 3, 4, 3), (1, 1, 1, 1, 2)])
def test_matches_brute_force_loops(shape):
    q, k, v, do = _rand(*shape, seed=7)
    o, lse = A.forward(q, k, v)
    got = (o, lse, *A.backward(do, q, k, v, o, lse))
    want = _brute_force(q, k, v, do)
    for name, x, r in zip(("o", "lse", "dq", "dk", "dv"), got, want):
        np.testing.assert_allclose(x, r, rtol=1e-10, atol=1e-12, err_msg=name)


def test_t1_closed_form():
    # One token attends only to itself: o = v of its KV head, dq = dk = 0, dv = sum of dO over the group.
    q, k, v, do = _rand(2, 6, 2, 1, 32, seed=1)
    o, lse = A.forward(q, k, v)
    dq, dk, dv = A.backward(do, q, k, v, o, lse)
    np.testing.assert_allclose(o, np.repeat(v, 3, axis=1), rtol=0, atol=1e-15)
    np.testing.assert_allclose(lse, (q * np.repeat(k, 3, axis=1)).sum(-1) / math.sqrt(32), atol=1e-12)
    assert np.abs(dq).max() < 1e-14 and np.abs(dk).max() < 1e-14
    np.testing.assert_allclose(dv, do.reshape(2, 2, 3, 1, 32).sum(2), atol=1e-14)


def test_zero_query_closed_form():
    # q = 0: uniform attention over the visible prefix, o_t = mean_{j<=t} v_j, lse_t = ln(t + 1).
    _, k, v, _ = _rand(1, 4, 2, 20, 64, seed=2)
    q = np.zeros((1, 4, 20, 64))
    o, lse = A.forward(q, k, v)
    prefix_mean = np.cumsum(v, axis=2) / np.arange(1, 21)[None, None, :, None]
    np.testing.assert_allclose(o, np.repeat(prefix_mean, 2, axis=1), atol=1e-13)
    np.testing.assert_allclose(lse, np.broadcast_to(np.log(np.arange(1, 21)), lse.shape), atol=1e-13)


def test_gqa_equals_mha_on_repeated_kv():
    # GQA must equal MHA on explicitly repeated K/V, with dK/dV summed over each group.
    q, k, v, do = _rand(2, 12, 4, 33, 64, seed=4)
    o, lse = A.forward(q, k, v)
    dq, dk, dv = A.backward(do, q, k, v, o, lse)
    kr, vr = np.repeat(k, 3, axis=1), np.repeat(v, 3, axis=1)
    o2, lse2 = A.forward(q, kr, vr)
    dq2, dk2, dv2 = A.backward(do, q, kr, vr, o2, lse2)
    np.testing.assert_allclose(o, o2, atol=1e-14)
    np.testing.assert_allclose(dq, dq2, atol=1e-13)
    np.testing.assert_allclose(dk, dk2.reshape(2, 4, 3, 33, 64).sum(2), atol=1e-12)
    np.testing.assert_allclose(dv, dv2.reshape(2, 4, 3, 33, 64).sum(2), atol=1e-12)


def test_future_keys_do_not_leak():
    q, k, v, _ = _rand(1, 4, 1, 16, 32, seed=5)
    o, lse = A.forward(q, k, v)
    k2, v2 = k.copy(), v.copy()
    k2[:, :, 8:] = np.random.default_rng(9).standard_normal(k2[:, :, 8:].shape)
    v2[:, :, 8:] = np.random.default_rng(10).standard_normal(v2[:, :, 8:].shape)
    o2, lse2 = A.forward(q, k2, v2)
    assert np.array_equal(o[:, :, :8], o2[:, :, :8]) and np.array_equal(lse[:, :, :8], lse2[:, :, :8])
    assert not np.allclose(o[:, :, 8:], o2[:, :, 8:])


def test_flops_counts_causal_pairs():
    for B, H, T, D in [(1, 1, 1, 64), (2, 3, 5, 32), (8, 12, 1024, 64)]:
        pairs = B * H * sum(i + 1 for i in range(T))
        assert A.flops(B, H, T, D, "fwd") == 4 * D * pairs
        assert A.flops(B, H, T, D, "bwd") == 8 * D * pairs
        assert A.flops(B, H, T, D) == 12 * D * pairs
    assert abs(A.flops(8, 12, 1024, 64) - 38.69e9) < 0.01e9


# ---- planted mistakes: each must be caught by at least one of the checks above ----------------


def _fails(check) -> bool:
    try:
        check()
    except AssertionError:
        return True
    return False


def test_planted_wrong_kv_head_mapping_is_caught(monkeypatch):
    monkeypatch.setattr(A, "kv_head_index", lambda H, KVH: np.arange(H) % KVH)
    assert _fails(lambda: _check_against_torch((1, 12, 4, 24, 32)))


def test_planted_wrong_mask_diagonal_is_caught(monkeypatch):
    monkeypatch.setattr(A, "causal_mask", lambda T: np.triu(np.ones((T, T), dtype=bool), k=2))
    assert _fails(lambda: _check_against_torch((1, 2, 1, 9, 16)))


def test_planted_dropped_d_term_is_caught(monkeypatch):
    monkeypatch.setattr(A, "preprocess", lambda do, o: np.zeros(np.shape(do)[:-1]))
    assert _fails(lambda: _check_against_torch((1, 2, 1, 9, 16)))


def test_planted_mean_instead_of_group_sum_is_caught(monkeypatch):
    monkeypatch.setattr(A, "group_sum", lambda x, KVH: x.reshape(x.shape[0], KVH, -1, *x.shape[2:]).mean(2))
    assert _fails(lambda: _check_against_torch((1, 6, 2, 9, 16)))
    assert _fails(test_gqa_equals_mha_on_repeated_kv)


def test_planted_missing_scale_is_caught():
    q, k, v, do = _rand(1, 2, 1, 7, 16, seed=11)
    o, lse = A.forward(q, k, v, scale=1.0)  # forgot 1/sqrt(D)
    ro, rlse, *_ = _torch_reference(q, k, v, do)
    assert not np.allclose(o, ro, atol=1e-6)


# ---- committed golden fixtures -----------------------------------------------------------------


@pytest.mark.parametrize("name", golden_names())
def test_golden_fixture_reproduces(name):
    g = load_golden(name)
    B, H, KVH, T, D = g["shape"]
    # The stored inputs are exactly the seeded draw, so any box can regenerate them.
    q, k, v, do = make_inputs(B, H, KVH, T, D, g["dtype"], g["mult"], seed=0)
    for key, t in (("q", q), ("k", k), ("v", v), ("do", do)):
        assert torch.equal(g[key].view(torch.int16), t.view(torch.int16)), key
    qd, kd, vd, dod = (g[x].double().numpy() for x in ("q", "k", "v", "do"))
    o, lse = A.forward(qd, kd, vd)
    dq, dk, dv = A.backward(dod, qd, kd, vd, o, lse)
    for key, x in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
        np.testing.assert_allclose(x, g[key].numpy(), rtol=1e-6, atol=1e-6, err_msg=key)


# ---- the timed CPU baseline (torch_reference_fwd_bwd), both forms ------------------------------


def _check_torch_reference_fn(shape, explicit, seed=12):
    """torch_reference_fwd_bwd in float64 against the pinned forward / backward at 1e-10."""
    q, k, v, do = _rand(*shape, seed=seed)
    o, lse = A.forward(q, k, v)
    dq, dk, dv = A.backward(do, q, k, v, o, lse)
    got = A.torch_reference_fwd_bwd(*(torch.tensor(x, dtype=torch.float64) for x in (q, k, v, do)), explicit=explicit)
    for name, x, r in zip(("o", "dq", "dk", "dv"), got, (o, dq, dk, dv)):
        assert x.dtype == torch.float64, name
        np.testing.assert_allclose(x.numpy(), r, rtol=1e-10, atol=1e-10, err_msg=f"{name} explicit={explicit}")


@pytest.mark.parametrize("explicit", [False, True])
@pytest.mark.parametrize("shape", [(1, 12, 4, 40, 64), (2, 6, 2, 17, 32), (1, 4, 1, 9, 16), (1, 3, 3, 5, 8)])
def test_torch_reference_fwd_bwd_matches_pinned_oracle(shape, explicit):
    _check_torch_reference_fn(shape, explicit)


def test_torch_reference_fwd_bwd_config1_shape():
    # BASELINE config 1 (B=1, T=256, 12 Q / 4 KV heads, d=64), the shape the CPU baseline times.
    _check_torch_reference_fn((1, 12, 4, 256, 64), explicit=False, seed=0)
    _check_torch_reference_fn((1, 12, 4, 256, 64), explicit=True, seed=0)


@pytest.mark.parametrize("explicit", [False, True])
def test_planted_repeat_instead_of_repeat_interleave_is_caught(monkeypatch, explicit):
    # K/V tiled [kv0, kv1, kv0, kv1, ...] instead of [kv0, kv0, ..., kv1, ...]: the wrong GQA grouping.
    def tiled(self, repeats, dim=None, **kw):
        reps = [1] * self.dim()
        reps[dim] = repeats
        return self.repeat(*reps)

    monkeypatch.setattr(torch.Tensor, "repeat_interleave", tiled)
    assert _fails(lambda: _check_torch_reference_fn((1, 12, 4, 24, 32), explicit))


def test_planted_dropped_is_causal_is_caught(monkeypatch):
    sdpa = F.scaled_dot_product_attention
    monkeypatch.setattr(F, "scaled_dot_product_attention", lambda *a, is_causal=False, **kw: sdpa(*a, **kw))
    assert _fails(lambda: _check_torch_reference_fn((1, 4, 2, 24, 32), explicit=False))


def test_planted_wrong_explicit_mask_diagonal_is_caught(monkeypatch):
    triu = torch.triu
    monkeypatch.setattr(torch, "triu", lambda x, diagonal=0: triu(x, diagonal + 1))
    assert _fails(lambda: _check_torch_reference_fn((1, 4, 2, 24, 32), explicit=True))

