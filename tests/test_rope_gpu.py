"""GPU tests of the HIP RoPE kernel (include/nanonemo_rope.h, nanonemo::rope_qk) against the
reference's RoPE formula (/root/reference/nanonemo/model/layers.py:67-74, restated in
nanonemo_amd.model.rope), the pattern of /root/reference/tests/kernels/test_rope.py.

The kernel rounds exactly where the torch formula does (fp32 products and sums one at a time, then
one rounding to the dtype), so forward and gradients must be bit-identical to it."""

from __future__ import annotations

import pytest
import torch

from nanonemo_amd.model import ModelConfig, NanoNemo, rope, rope_tables

pytestmark = pytest.mark.gpu

SHAPES = [(2, 37, 12, 4, 64), (1, 1, 4, 2, 32), (3, 130, 8, 8, 128), (2, 1024, 12, 4, 64)]


def _rope_qk():
    from nanonemo_amd.kernels.hip.rope import rope_qk

    return rope_qk


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("B, T, H, KVH, D", SHAPES)
def test_forward_and_backward_bit_identical_to_the_formula(B, T, H, KVH, D, dtype):
    print(f"\n[case] rope B={B} T={T} H={H} KVH={KVH} D={D} {dtype}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(0)
    cos, sin = (t.cuda() for t in rope_tables(D, T + 5, 10000.0))  # tables longer than T
    q = (torch.randn(B, T, H, D, device="cuda", generator=g) * 3).to(dtype).requires_grad_()
    k = (torch.randn(B, T, KVH, D, device="cuda", generator=g) * 3).to(dtype).requires_grad_()
    qr, kr = (t.detach().clone().requires_grad_() for t in (q, k))
    qo, ko = _rope_qk()(q, k, cos, sin)
    rq, rk = rope(qr, cos, sin, seq_dim=1), rope(kr, cos, sin, seq_dim=1)
    assert torch.equal(qo, rq) and torch.equal(ko, rk)
    gq = torch.randn(qo.shape, device="cuda", generator=g).to(dtype)
    gk = torch.randn(ko.shape, device="cuda", generator=g).to(dtype)
    torch.autograd.backward((qo, ko), (gq, gk))
    torch.autograd.backward((rq, rk), (gq, gk))
    assert torch.equal(q.grad, qr.grad) and torch.equal(k.grad, kr.grad)


def test_model_with_hip_rope_is_bit_identical():
    small = dict(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, d_ff=512, vocab_size=512, max_seq_len=128)
    torch.manual_seed(0)
    a = NanoNemo(ModelConfig(**small, attn_kernel="hip_bthd")).cuda()
    b = NanoNemo(ModelConfig(**small, attn_kernel="hip_bthd", rope_kernel="hip")).cuda()
    b.load_state_dict(a.state_dict())
    idx = torch.randint(0, 512, (2, 128), device="cuda")
    with torch.autocast("cuda", dtype=torch.bfloat16):
        la, lb = a(idx, idx.roll(-1, 1))[1], b(idx, idx.roll(-1, 1))[1]
    la.backward()
    lb.backward()
    assert torch.equal(la, lb)
    for (n, pa), pb in zip(a.named_parameters(), b.parameters()):
        assert torch.equal(pa.grad, pb.grad), n


def test_compiles_without_graph_breaks():
    rope_qk = _rope_qk()
    cos, sin = (t.cuda() for t in rope_tables(64, 64, 10000.0))
    q = torch.randn(2, 64, 12, 64, device="cuda", dtype=torch.bfloat16)
    k = torch.randn(2, 64, 4, 64, device="cuda", dtype=torch.bfloat16)
    f = torch.compile(lambda q, k: rope_qk(q, k, cos, sin), fullgraph=True)
    a, b = f(q, k)
    c, d = rope_qk(q, k, cos, sin)
    assert torch.equal(a, c) and torch.equal(b, d)
