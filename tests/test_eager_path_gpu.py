"""The public functions' eager path (flash_attn, flash_attn_bthd, flash_attn_bthd_rope through plain
autograd.Functions that call the library's launch helpers) against the custom ops they bypass
(torch.ops.nanonemo.* with their registered autograd): the same outputs and gradients, bit for bit, in bf16 and
fp16, for strided inputs, for an unused output, and without autograd; and the routing: torch.func transforms and
dispatch modes go through the custom ops."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _grads(fn, inputs, do):
    o = fn(*inputs)
    return (o, *torch.autograd.grad(o, [t for t in inputs if t.requires_grad], do))


def _leaves(*ts):
    return [t.detach().clone().requires_grad_() for t in ts]


CASES = [
    (2, 256, 12, 4, 64, torch.bfloat16),
    (2, 256, 12, 4, 64, torch.float16),
    (1, 333, 8, 2, 32, torch.bfloat16),
    (2, 1024, 12, 1, 64, torch.bfloat16),  # MQA: a split dK/dV
]


@pytest.mark.parametrize("B, T, H, KVH, D, dtype", CASES)
def test_eager_path_matches_the_custom_ops_bit_for_bit(B, T, H, KVH, D, dtype):
    from nanonemo_amd.kernels.hip import flash_attn as fa
    from nanonemo_amd.model import rope_tables

    print(f"\n[case] eager path vs custom ops B={B} T={T} H={H} KVH={KVH} D={D} {dtype}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(3)
    q, do = (torch.randn(B, T, H, D, generator=g).to(dtype).to(DEV) for _ in range(2))
    k, v = (torch.randn(B, T, KVH, D, generator=g).to(dtype).to(DEV) for _ in range(2))
    cos, sin = (t.to(DEV) for t in rope_tables(D, T, 10000.0))
    # (B, H, T, hd) views of the projection layout: strided inputs for the dense op
    dense = lambda t: t.transpose(1, 2)  # noqa: E731
    pairs = [
        ("flash_attn", fa.flash_attn, lambda *a: torch.ops.nanonemo.flash_attn(*a)[0],
         (dense(q), dense(k), dense(v)), dense(do)),
        ("flash_attn_bthd", fa.flash_attn_bthd, lambda *a: torch.ops.nanonemo.flash_attn_bthd(*a)[0], (q, k, v), do),
        ("flash_attn_bthd_rope", fa.flash_attn_bthd_rope,
         lambda *a: torch.ops.nanonemo.flash_attn_bthd_rope(*a)[0], (q, k, v, cos, sin), do),
    ]
    for name, eager, op, ins, dout in pairs:
        a = _leaves(*ins[:3]) + list(ins[3:])
        b = _leaves(*ins[:3]) + list(ins[3:])
        got = _grads(eager, a, dout)
        ref = _grads(op, b, dout)
        assert type(got[0].grad_fn).__name__.startswith("_FlashAttn"), f"{name}: eager path not taken ({got[0].grad_fn})"
        torch.cuda.synchronize()
        for what, x, y in zip(("o", "dq", "dk", "dv"), got, ref):
            assert torch.equal(x, y), f"{name} {what}: max |diff| {(x.float() - y.float()).abs().max().item()}"
        with torch.no_grad():  # no autograd: the forward alone, nothing recorded
            o = eager(*a)
        assert o.grad_fn is None and torch.equal(o, got[0])


def test_eager_path_backward_when_only_part_of_the_output_is_used():
    # d_o arrives as a sparse slice's gradient (zeros elsewhere) and, for an output that is not used at all, the
    # backward is not called; the results must equal the custom op's.
    from nanonemo_amd.kernels.hip import flash_attn as fa

    g = torch.Generator(device="cpu").manual_seed(5)
    q = torch.randn(1, 4, 128, 64, generator=g).bfloat16().to(DEV)
    k, v = (torch.randn(1, 2, 128, 64, generator=g).bfloat16().to(DEV) for _ in range(2))
    a, b = _leaves(q, k, v), _leaves(q, k, v)
    ga = torch.autograd.grad(fa.flash_attn(*a)[:, :, :7].sum(), a)
    gb = torch.autograd.grad(torch.ops.nanonemo.flash_attn(*b)[0][:, :, :7].sum(), b)
    for x, y in zip(ga, gb):
        assert torch.equal(x, y)


def test_transforms_and_dispatch_modes_take_the_custom_ops():
    from torch.utils._python_dispatch import TorchDispatchMode

    from nanonemo_amd.kernels.hip import flash_attn as fa

    x = torch.ones(4, device=DEV)
    assert fa._eager(x)
    assert not fa._eager(x, torch.ones(4))  # a CPU tensor among the inputs
    seen = []

    def f(t):
        seen.append(fa._eager(t))
        return (t * t).sum()

    def h(t):
        seen.append(fa._eager(t))
        return t * 2

    torch.func.grad(f)(x)
    torch.func.vmap(h)(x.view(2, 2))
    assert seen == [False, False]

    class Mode(TorchDispatchMode):
        def __torch_dispatch__(self, func, types, args=(), kwargs=None):
            return func(*args, **(kwargs or {}))

    with Mode():
        assert not fa._eager(x)
    assert fa._eager(x)


def test_eager_path_under_torch_compile_uses_the_ops():
    # Traced by dynamo, the public function must take the custom op (one opaque node), not the autograd.Function.
    from nanonemo_amd.kernels.hip import flash_attn as fa

    g = torch.Generator(device="cpu").manual_seed(9)
    q = torch.randn(1, 4, 64, 64, generator=g).bfloat16().to(DEV)
    k, v = (torch.randn(1, 2, 64, 64, generator=g).bfloat16().to(DEV) for _ in range(2))
    seen = []

    def backend(gm, example_inputs):
        seen.extend(str(n.target) for n in gm.graph.nodes if n.op == "call_function")
        return gm

    torch._dynamo.reset()
    out = torch.compile(fa.flash_attn, backend=backend, fullgraph=True)(q, k, v)
    assert any("nanonemo.flash_attn" in t for t in seen), seen
    assert torch.equal(out, fa.flash_attn(q, k, v))


def test_rope_eager_path_matches_the_op_bit_for_bit():
    from nanonemo_amd.kernels.hip import rope as rp
    from nanonemo_amd.model import rope_tables

    print("\n[case] rope_qk / rope_k eager path vs nanonemo::rope_qk", flush=True)
    g = torch.Generator(device="cpu").manual_seed(11)
    q, dq = (torch.randn(2, 200, 12, 64, generator=g).bfloat16().to(DEV) for _ in range(2))
    k, dk = (torch.randn(2, 200, 4, 64, generator=g).bfloat16().to(DEV) for _ in range(2))
    cos, sin = (t.to(DEV) for t in rope_tables(64, 256, 10000.0))
    a, b = _leaves(q, k), _leaves(q, k)
    ea = rp.rope_qk(a[0], a[1], cos, sin)
    eb = torch.ops.nanonemo.rope_qk(b[0], b[1], cos, sin)
    assert type(ea[0].grad_fn).__name__.startswith("_RopeQkFn")
    ga = torch.autograd.grad(ea, a, (dq, dk))
    gb = torch.autograd.grad(eb, b, (dq, dk))
    for x, y in zip((*ea, *ga), (*eb, *gb)):
        assert torch.equal(x, y)
    ka, kb = _leaves(k)[0], _leaves(k)[0]
    oa, ob = rp.rope_k(ka, cos, sin), torch.ops.nanonemo.rope_qk(q[:, :, :0], kb, cos, sin)[1]
    assert torch.equal(oa, ob)
    assert torch.equal(torch.autograd.grad(oa, ka, dk)[0], torch.autograd.grad(ob, kb, dk)[0])
    # only one output used: the other's gradient is a zero tensor on both paths
    assert torch.equal(torch.autograd.grad(rp.rope_qk(a[0], a[1], cos, sin)[0], a, dq)[1],
                       torch.autograd.grad(torch.ops.nanonemo.rope_qk(b[0], b[1], cos, sin)[0], b, dq)[1])


@pytest.mark.parametrize("with_delta", [True, False])
@pytest.mark.parametrize("autocast", [False, True])
def test_add_rms_norm_eager_path_matches_the_op_bit_for_bit(with_delta, autocast):
    from nanonemo_amd.kernels.hip import rmsnorm as rn

    print(f"\n[case] add_rms_norm eager path vs op delta={with_delta} autocast={autocast}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(13)
    x, dy, dh = (torch.randn(4, 96, 768, generator=g).to(DEV) for _ in range(3))
    d = torch.randn(4, 96, 768, generator=g).to(DEV) if with_delta else None
    w = (1 + 0.1 * torch.randn(768, generator=g)).to(DEV)
    leaves = lambda: [t.detach().clone().requires_grad_() for t in (x, d, w) if t is not None]  # noqa: E731

    def run(fn, ins):
        xs, ds, ws = (ins[0], ins[1], ins[2]) if with_delta else (ins[0], None, ins[1])
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
            y, h = fn(xs, ds, ws)
        outs, grads = (y, h), (dy.to(y.dtype), dh.to(h.dtype))
        if not with_delta:
            outs, grads = (y,), (dy.to(y.dtype),)
        return (y, h, *torch.autograd.grad(outs, ins, grads))

    def op(xs, ds, ws):
        out_dtype = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else xs.dtype
        y, h, _ = torch.ops.nanonemo.cuda_add_rms_norm_fwd(xs, ds, ws, 1e-5, out_dtype)
        return y, (xs if ds is None else h)

    ra = run(lambda *t: rn.add_rms_norm(*t, 1e-5), leaves())
    rb = run(op, leaves())
    assert type(ra[0].grad_fn).__name__.startswith("_AddRmsNormFn")
    for i, (p, r) in enumerate(zip(ra, rb)):
        assert torch.equal(p, r), f"output {i}: max |diff| {(p.float() - r.float()).abs().max().item()}"


def test_eager_path_under_activation_checkpointing():
    # torch.utils.checkpoint runs the forward again inside the backward: the gradients equal a plain run's, bit for
    # bit (the kernels are deterministic).
    from torch.utils.checkpoint import checkpoint

    from nanonemo_amd.kernels.hip import flash_attn as fa

    g = torch.Generator(device="cpu").manual_seed(19)
    q, do = (torch.randn(2, 300, 8, 64, generator=g).bfloat16().to(DEV) for _ in range(2))
    k, v = (torch.randn(2, 300, 2, 64, generator=g).bfloat16().to(DEV) for _ in range(2))
    a, b = _leaves(q, k, v), _leaves(q, k, v)
    ga = torch.autograd.grad(fa.flash_attn_bthd(*a), a, do)
    gb = torch.autograd.grad(checkpoint(fa.flash_attn_bthd, *b, use_reentrant=False), b, do)
    for x, y in zip(ga, gb):
        assert torch.equal(x, y)
