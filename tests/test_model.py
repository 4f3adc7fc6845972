"""CPU tests of the 114 M model that carries the attention op: structure, init,
RoPE in both layouts, FLOP count, and the train step on the plain-PyTorch attention.

Mirrors /root/reference/tests/model/test_model.py:11-40 and tests/model/test_layers.py:50-87."""

from __future__ import annotations

import math

import pytest
import torch

from nanonemo_amd.model import ModelConfig, NanoNemo, rope, rope_tables
from nanonemo_amd.train import make_optimizer, synthetic_batches, train_step

SMALL = dict(n_layers=2, d_model=96, n_heads=6, n_kv_heads=2, d_ff=256, vocab_size=128, max_seq_len=32)


def test_param_count_is_exact():
    cfg = ModelConfig()
    d, kv = cfg.d_model, cfg.n_kv_heads * cfg.head_dim
    per_block = (d * d + 2 * d * kv + d * d) + 3 * d * cfg.d_ff + 2 * d
    expected = cfg.vocab_size * d + cfg.n_layers * per_block + d
    model = NanoNemo(cfg)
    assert model.num_params() == expected == 114_150_144
    assert model.num_params(non_embedding=True) == expected - cfg.vocab_size * d


def test_flops_per_token_matches_the_reference_count():
    # /root/reference/nanonemo/train/mfu.py:24-26 quotes 798.0 MFLOP/token for this model at T = 1024
    assert NanoNemo(ModelConfig()).flops_per_token(1024) / 1e6 == pytest.approx(798.0, abs=0.2)


def test_tied_embedding_and_scaled_residual_init():
    torch.manual_seed(0)
    cfg = ModelConfig()
    model = NanoNemo(cfg)
    assert model.lm_head.weight is model.tok_emb.weight
    resid = 0.02 / math.sqrt(2 * cfg.n_layers)
    assert abs(model.blocks[0].attn.wo.weight.std().item() - resid) < 2e-4
    assert abs(model.blocks[0].mlp.w_down.weight.std().item() - resid) < 2e-4
    assert abs(model.blocks[0].attn.wq.weight.std().item() - 0.02) < 2e-4
    assert not any("rope" in k for k in model.state_dict())


def test_rope_is_the_same_in_both_layouts():
    cos, sin = rope_tables(64, 50, 10000.0)
    x = torch.randn(2, 50, 12, 64, dtype=torch.bfloat16)  # (B, T, H, hd)
    a = rope(x, cos, sin, seq_dim=1)
    b = rope(x.transpose(1, 2), cos, sin, seq_dim=2).transpose(1, 2)
    assert torch.equal(a, b)


def test_rope_tables_are_bit_identical_to_the_reference_formula():
    # The reference's rope_cache (/root/reference/nanonemo/model/layers.py:59-64): inv_freq as the reciprocal
    # of an fp32 power, angles as torch.outer of fp32 positions and inv_freq. base**(-x) differs from
    # 1/(base**x) in the last bit for some i, which moves thousands of cos/sin entries at T=1024.
    for hd, T, base in ((64, 1024, 10000.0), (32, 300, 10000.0), (64, 64, 500000.0)):
        inv = 1.0 / (base ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))
        ang = torch.outer(torch.arange(T, dtype=torch.float32), inv)
        cos, sin = rope_tables(hd, T, base)
        assert cos.dtype == sin.dtype == torch.float32 and cos.shape == (T, hd // 2)
        assert torch.equal(cos, ang.cos()) and torch.equal(sin, ang.sin()), (hd, T, base)
    # and the negative-power form is not the same table (so the check above can tell them apart)
    neg = 10000.0 ** (-torch.arange(0, 64, 2, dtype=torch.float32) / 64)
    assert not torch.equal(torch.outer(torch.arange(1024, dtype=torch.float32), neg).cos(), rope_tables(64, 1024, 10000.0)[0])


def test_rope_closed_forms():
    cos, sin = rope_tables(8, 16, 10000.0)
    x = torch.randn(1, 1, 16, 8, dtype=torch.float64).float()
    y = rope(x, cos, sin, seq_dim=2)
    assert torch.equal(y[:, :, 0], x[:, :, 0])  # position 0 is the identity
    # rotations preserve each (i, i + hd/2) pair's norm
    n = lambda t: t[..., :4].square() + t[..., 4:].square()  # noqa: E731
    torch.testing.assert_close(n(y), n(x), rtol=1e-5, atol=1e-6)
    # the score between rotated q at m and k at n depends only on m - n
    q, k = torch.randn(8), torch.randn(8)
    qs = rope(q.expand(1, 1, 16, 8).contiguous(), cos, sin, seq_dim=2)[0, 0]
    ks = rope(k.expand(1, 1, 16, 8).contiguous(), cos, sin, seq_dim=2)[0, 0]
    assert torch.dot(qs[7], ks[3]).item() == pytest.approx(torch.dot(qs[9], ks[5]).item(), rel=1e-5, abs=1e-5)
    # the pairing is i <-> i + hd/2 with angle m * base^(-2i/hd)
    m, i = 5, 1
    theta = m * 10000.0 ** (-2 * i / 8)
    e = torch.zeros(1, 1, 16, 8)
    e[0, 0, m, i] = 1.0
    r = rope(e, cos, sin, seq_dim=2)[0, 0, m]
    assert r[i].item() == pytest.approx(math.cos(theta), abs=1e-6)
    assert r[i + 4].item() == pytest.approx(math.sin(theta), abs=1e-6)


def test_initial_loss_is_near_uniform():
    torch.manual_seed(0)
    model = NanoNemo(ModelConfig(**SMALL))
    idx = torch.randint(0, 128, (2, 32))
    _, loss = model(idx, torch.roll(idx, -1, dims=1))
    assert abs(loss.item() - math.log(128)) < 0.1


def test_train_step_on_torch_attention():
    torch.manual_seed(0)
    model = NanoNemo(ModelConfig(**SMALL))
    opt = make_optimizer(model) if torch.cuda.is_available() else torch.optim.AdamW(model.parameters(), lr=3e-3)
    data = synthetic_batches(4, 2, 32, 128, "cpu")
    losses = []
    for x, y in data:
        loss, norm = train_step(model, opt, [(x, y)], amp_dtype=None)
        assert torch.isfinite(norm)
        losses.append(loss.item())
    assert all(math.isfinite(v) for v in losses)
    # the same batch again after training on it: its loss went down
    x, y = data[0]
    with torch.no_grad():
        assert model(x, y)[1].item() < losses[0]


def test_unknown_attention_kernel_is_rejected():
    with pytest.raises(ValueError):
        ModelConfig(attn_kernel="cuda_v2")


@pytest.mark.parametrize("field", ["rope_kernel", "norm_kernel"])
def test_unknown_neighbour_kernel_is_rejected(field):
    with pytest.raises(ValueError):
        ModelConfig(**{field: "triton"})
