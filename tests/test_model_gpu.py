"""The model with this build's attention against the same model on the plain-PyTorch attention, on
identical weights and inputs (the pattern of /root/reference/tests/kernels/test_model_kernels.py:54-78),
plus the layout-fused path's exact agreement with the drop-in path, torch.compile, and a short
training run (BASELINE config 5 in miniature)."""

from __future__ import annotations

import pytest
import torch

from nanonemo_amd.model import ModelConfig, NanoNemo
from nanonemo_amd.train import make_optimizer, synthetic_batches, train_step

pytestmark = pytest.mark.gpu

# attn_backend only affects the "torch" attention: the reference model attends in fp32 (SDPA math on upcast q, k, v)
SMALL = dict(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, d_ff=512, vocab_size=512, max_seq_len=128,
             attn_backend="math_fp32")


def _pair(attn: str, cfg: dict = SMALL, batch: int = 2):
    """The plain model and one with this build's kernels ("+rope" / "+qrope" / "+norm": also the HIP RoPE, q's RoPE
    inside the attention op, the fused add + RMSNorm), on identical weights, with a batch of uniform token ids and
    their next-token targets."""
    kernel, *extras = attn.split("+")
    torch.manual_seed(0)
    ref = NanoNemo(ModelConfig(**cfg)).cuda()
    rope = "hip" if "rope" in extras else "fused" if "qrope" in extras else "torch"
    fast = NanoNemo(ModelConfig(**cfg, attn_kernel=kernel, rope_kernel=rope,
                                norm_kernel="hip" if "norm" in extras else "torch")).cuda()
    fast.load_state_dict(ref.state_dict())
    idx = torch.randint(0, ref.cfg.vocab_size, (batch, ref.cfg.max_seq_len), device="cuda")
    return ref, fast, idx, torch.roll(idx, -1, dims=1)


def _grads(model):
    return {n: p.grad for n, p in model.named_parameters()}


@pytest.mark.parametrize("attn", ["hip", "hip_bthd", "hip_bthd+norm"])
def test_bf16_autocast_loss_and_grads_match_torch_attention(attn):
    print(f"\n[case] model {attn} vs torch attention, bf16 autocast", flush=True)
    ref, fast, idx, tgt = _pair(attn)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        _, ref_loss = ref(idx, tgt)
        _, loss = fast(idx, tgt)
    # bf16 rounds 8x coarser than the reference's fp16 test (loss 1e-3, grads 5e-2 * max)
    torch.testing.assert_close(loss, ref_loss, rtol=5e-3, atol=5e-3)
    ref_loss.backward()
    loss.backward()
    for name, g in _grads(fast).items():
        r = _grads(ref)[name]
        torch.testing.assert_close(g, r, rtol=5e-2, atol=5e-2 * r.abs().max().item(), msg=name)


# the full 114 M model (12 layers, d_model 768, 12 Q / 4 KV heads, SwiGLU 2048, vocab 50,304,
# tied embeddings) at B=8, T=1024 under bf16 autocast, random init (seed 0), uniform token ids.
CONFIG5 = dict(max_seq_len=1024, attn_backend="math_fp32")


@pytest.mark.parametrize("attn", ["hip_bthd", "hip", "hip_bthd+rope+norm", "hip_bthd+qrope+norm"])
def test_config5_full_size_loss_and_grads_match_torch_attention(attn):
    # The pattern of /root/reference/tests/kernels/test_model_kernels.py:54-66 (loss 1e-3, every gradient within
    # 5e-2 of its largest magnitude) at the full model and batch, widened for bf16: loss 5e-3.
    print(f"\n[case] config 5 full size, {attn} vs torch attention (fp32 math), bf16 autocast", flush=True)
    ref, fast, idx, tgt = _pair(attn, CONFIG5, batch=8)
    assert ref.num_params() == 114_150_144
    with torch.autocast("cuda", dtype=torch.bfloat16):
        _, ref_loss = ref(idx, tgt)
        _, loss = fast(idx, tgt)
    print(f"[loss] torch {ref_loss.item():.6f} {attn} {loss.item():.6f}", flush=True)
    torch.testing.assert_close(loss, ref_loss, rtol=5e-3, atol=5e-3)
    ref_loss.backward()
    loss.backward()
    worst = 0.0
    for name, g in _grads(fast).items():
        r = _grads(ref)[name]
        assert g is not None and torch.isfinite(g).all(), name
        worst = max(worst, ((g - r).abs().max() / r.abs().max()).item())
        torch.testing.assert_close(g, r, rtol=5e-2, atol=5e-2 * r.abs().max().item(), msg=name)
    print(f"[grads] largest |g - ref| / max|ref| over parameters: {worst:.3e}", flush=True)
    del ref, fast
    torch.cuda.empty_cache()


def test_layout_fused_model_is_bit_identical_to_the_drop_in_model():
    _, a, idx, tgt = _pair("hip")
    torch.manual_seed(0)
    b = NanoNemo(ModelConfig(**SMALL, attn_kernel="hip_bthd")).cuda()
    b.load_state_dict(a.state_dict())
    with torch.autocast("cuda", dtype=torch.bfloat16):
        la = a(idx, tgt)[1]
        lb = b(idx, tgt)[1]
    la.backward()
    lb.backward()
    assert torch.equal(la, lb)
    for (n, ga), gb in zip(_grads(a).items(), _grads(b).values()):
        assert torch.equal(ga, gb), n


def test_compiled_model_has_no_graph_breaks():
    _, fast, idx, tgt = _pair("hip_bthd")
    torch._dynamo.reset()
    compiled = torch.compile(fast, fullgraph=True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        _, loss = compiled(idx, tgt)
        _, eager_loss = fast(idx, tgt)
    loss.backward()
    torch.testing.assert_close(loss, eager_loss, rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("attn", ["hip_bthd+rope+norm", "hip_bthd+qrope+norm"])
def test_compiled_model_with_every_hip_kernel(attn):
    # The whole model compiled with every kernel of this build on (the pattern of
    # /root/reference/tests/kernels/test_model_kernels.py:69-78): no graph break under fullgraph=True, and the
    # compiled forward and backward agree with the same model run eagerly.
    print(f"\n[case] torch.compile(fullgraph=True) of the model with {attn}", flush=True)
    _, fast, idx, tgt = _pair(attn)
    torch.manual_seed(0)
    eager = NanoNemo(fast.cfg).cuda()
    eager.load_state_dict(fast.state_dict())
    torch._dynamo.reset()
    compiled = torch.compile(fast, fullgraph=True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        _, loss = compiled(idx, tgt)
        _, eager_loss = eager(idx, tgt)
    loss.backward()
    eager_loss.backward()
    torch.testing.assert_close(loss, eager_loss, rtol=1e-3, atol=1e-3)
    for (name, g), r in zip(_grads(fast).items(), _grads(eager).values()):
        assert g is not None and torch.isfinite(g).all(), name
        torch.testing.assert_close(g, r, rtol=5e-2, atol=5e-2 * r.abs().max().item(), msg=name)


def test_short_training_run_tracks_torch_attention():
    curves = {}
    for attn in ("torch", "hip_bthd"):
        torch.manual_seed(0)
        model = NanoNemo(ModelConfig(**SMALL, attn_kernel=attn)).cuda()
        opt = make_optimizer(model, lr=2e-3)
        # one fixed batch, so that the loss has something to learn (uniform random streams do not)
        batch = synthetic_batches(1, 4, 128, SMALL["vocab_size"], "cuda")[0]
        curves[attn] = torch.stack([train_step(model, opt, [batch])[0] for _ in range(10)]).cpu()
    print(f"\n[train] torch {curves['torch'].tolist()}\n[train] hip   {curves['hip_bthd'].tolist()}", flush=True)
    assert torch.isfinite(curves["hip_bthd"]).all()
    # Two bf16 runs drift apart step by step (different rounding, then different updates), as any two
    # kernels do: the first steps agree closely, the whole curve within a few percent.
    torch.testing.assert_close(curves["hip_bthd"][:5], curves["torch"][:5], rtol=0, atol=2e-2)
    torch.testing.assert_close(curves["hip_bthd"], curves["torch"], rtol=5e-2, atol=0)
    assert curves["hip_bthd"][-1] < curves["hip_bthd"][0] - 0.5


def test_fused_norm_model_tracks_the_plain_norm_model():
    # The whole model with the fused add + RMSNorm (and the layout-fused attention) against the same model
    # with plain-PyTorch norms, bf16 autocast: the norms' outputs differ only in rounding order.
    _, a, idx, tgt = _pair("hip_bthd")
    torch.manual_seed(0)
    b = NanoNemo(ModelConfig(**SMALL, attn_kernel="hip_bthd", norm_kernel="hip")).cuda()
    b.load_state_dict(a.state_dict())
    with torch.autocast("cuda", dtype=torch.bfloat16):
        la = a(idx, tgt)[1]
        lb = b(idx, tgt)[1]
    la.backward()
    lb.backward()
    torch.testing.assert_close(lb, la, rtol=2e-3, atol=2e-3)
    for (n, ga), gb in zip(_grads(a).items(), _grads(b).values()):
        torch.testing.assert_close(gb, ga, rtol=5e-2, atol=5e-2 * ga.abs().max().item(), msg=n)
