"""q's RoPE folded into the attention (nanonemo::flash_attn_bthd_rope / _bwd, nn_fa_{fwd,bwd}_rope_strided):
bit-identical to the unfused flow — nanonemo::rope_qk on q and k, the layout-fused attention on the rotated
tensors, and nanonemo::rope_qk_bwd on the gradients — on every output (o, lse, the rotated q, dq of the
unrotated q, dk, dv), in bf16 and fp16, head_dim 64 and 32, MHA / GQA / MQA (a split dK/dV) and ragged T;
through autograd; in the model (rope_kernel="fused" against "hip"); and under torch.compile."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _inputs(B, T, H, KVH, D, dtype, seed):
    from nanonemo_amd.model import rope_tables

    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(B, T, H, D, generator=g).to(dtype).to(DEV)
    k = torch.randn(B, T, KVH, D, generator=g).to(dtype).to(DEV)
    v = torch.randn(B, T, KVH, D, generator=g).to(dtype).to(DEV)
    do = torch.randn(B, T, H, D, generator=g).to(dtype).to(DEV)
    cos, sin = (t.to(DEV) for t in rope_tables(D, T + 17, 10000.0))  # tables longer than T
    return q, k, v, do, cos, sin


@pytest.mark.parametrize(
    "B, T, H, KVH, D, dtype",
    [
        (2, 256, 12, 4, 64, torch.bfloat16),
        (2, 256, 12, 4, 64, torch.float16),
        (1, 333, 8, 2, 32, torch.bfloat16),
        (2, 1024, 12, 1, 64, torch.bfloat16),  # MQA: the dK/dV work is split
        (1, 65, 4, 4, 64, torch.float16),
        (3, 1, 6, 3, 32, torch.bfloat16),
    ],
)
def test_fused_rope_is_bit_identical_to_rope_then_attention(B, T, H, KVH, D, dtype):
    from nanonemo_amd.kernels.hip import flash_attn as fa
    from nanonemo_amd.kernels.hip import rope as rp

    print(f"\n[case] fused RoPE vs rope_qk + flash_attn_bthd B={B} T={T} H={H} KVH={KVH} D={D} {dtype}", flush=True)
    q, k, v, do, cos, sin = _inputs(B, T, H, KVH, D, dtype, seed=7)
    # unfused: rotate q and k, attend, then rotate the gradients back
    qr, kr = rp._rope_qk(q, k, cos, sin)
    o_ref, lse_ref = fa._flash_attn_bthd(qr, kr, v)
    dqr, dkr, dv_ref = fa._flash_attn_bthd_bwd(do, qr, kr, v, o_ref, lse_ref)
    dq_ref, dk_ref = rp._rope_qk_bwd(dqr, dkr, cos, sin)
    # fused: k alone through the RoPE kernel, q inside the attention
    kr2 = rp.rope_k(k, cos, sin)
    o, lse, q_rot = fa._flash_attn_bthd_rope(q, kr2, v, cos, sin)
    dq, dk_rot, dv = fa._flash_attn_bthd_rope_bwd(do, q_rot, kr2, v, o, lse, cos, sin)
    dk = rp._rope_qk_bwd(q.new_empty(B, T, 0, D), dk_rot, cos, sin)[1]
    torch.cuda.synchronize()
    for name, a, r in (("k_rot", kr2, kr), ("q_rot", q_rot, qr), ("o", o, o_ref), ("lse", lse, lse_ref),
                       ("dk_rot", dk_rot, dkr), ("dq", dq, dq_ref), ("dk", dk, dk_ref), ("dv", dv, dv_ref)):
        assert torch.equal(a, r), f"{name}: max |diff| {(a.float() - r.float()).abs().max().item()}"


def test_fused_rope_autograd_matches_the_unfused_composition():
    from nanonemo_amd.kernels.hip import flash_attn as fa
    from nanonemo_amd.kernels.hip import rope as rp

    q, k, v, do, cos, sin = _inputs(2, 200, 12, 4, 64, torch.bfloat16, seed=3)
    grads = []
    for fused in (False, True):
        qs, ks, vs = (t.clone().requires_grad_() for t in (q, k, v))
        if fused:
            o = fa.flash_attn_bthd_rope(qs, rp.rope_k(ks, cos, sin), vs, cos, sin)
        else:
            qr, kr = rp.rope_qk(qs, ks, cos, sin)
            o = fa.flash_attn_bthd(qr, kr, vs)
        grads.append((o.detach(), *torch.autograd.grad(o, (qs, ks, vs), do)))
    for name, a, b in zip(("o", "dq", "dk", "dv"), *grads):
        assert torch.equal(a, b), name


def test_model_with_fused_rope_is_bit_identical_to_separate_rope():
    from nanonemo_amd.model import ModelConfig, NanoNemo

    small = dict(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, d_ff=512, vocab_size=512, max_seq_len=128)
    torch.manual_seed(0)
    a = NanoNemo(ModelConfig(**small, attn_kernel="hip_bthd", rope_kernel="hip")).cuda()
    b = NanoNemo(ModelConfig(**small, attn_kernel="hip_bthd", rope_kernel="fused")).cuda()
    b.load_state_dict(a.state_dict())
    idx = torch.randint(0, 512, (2, 128), device=DEV)
    tgt = torch.roll(idx, -1, dims=1)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        la, lb = a(idx, tgt)[1], b(idx, tgt)[1]
    la.backward()
    lb.backward()
    assert torch.equal(la, lb)
    for (n, pa), pb in zip(a.named_parameters(), b.parameters()):
        assert torch.equal(pa.grad, pb.grad), n


def test_fused_rope_compiles_without_graph_breaks():
    from nanonemo_amd.kernels.hip import flash_attn as fa
    from nanonemo_amd.kernels.hip import rope as rp

    q, k, v, do, cos, sin = _inputs(2, 128, 12, 4, 64, torch.bfloat16, seed=5)
    torch._dynamo.reset()
    fn = torch.compile(lambda q, k, v: fa.flash_attn_bthd_rope(q, rp.rope_k(k, cos, sin), v, cos, sin), fullgraph=True)
    eager = fa.flash_attn_bthd_rope(q, rp.rope_k(k, cos, sin), v, cos, sin)
    assert torch.equal(fn(q, k, v), eager)
    # the backward under AOTAutograd: the three-output op with its ignored gradients (lse, q_rot) and the
    # rope_k backward, bit for bit against eager autograd
    outs = []
    for f in (fn, lambda q, k, v: fa.flash_attn_bthd_rope(q, rp.rope_k(k, cos, sin), v, cos, sin)):
        qs, ks, vs = (t.clone().requires_grad_() for t in (q, k, v))
        o = f(qs, ks, vs)
        outs.append((o.detach(), *torch.autograd.grad(o, (qs, ks, vs), do)))
    for name, a, b in zip(("o", "dq", "dk", "dv"), *outs):
        assert torch.equal(a, b), name
