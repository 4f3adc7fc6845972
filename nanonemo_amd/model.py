"""The 114 M-parameter Llama-style decoder that calls the attention ops (the workload of BASELINE config 5).

Mirrors the reference model (/root/reference/nanonemo/model/config.py:6-53, layers.py:13-161,
model.py:13-70) so that a run of it exercises the attention path the way NanoNemo's training does:
pre-norm blocks with the residual stream carried as (x, pending delta), RMSNorm reduced in fp32,
rotate-half RoPE with fp32 tables, GQA attention (12 query / 4 KV heads, head_dim 64), SwiGLU MLP,
tied input/output embedding, GPT-2 style init with the residual projections scaled by
1/sqrt(2 n_layers), and the cross entropy on fp32 logits.

``attn_kernel`` selects the attention:
  * "torch": the reference's plain-PyTorch path, repeat_interleave + SDPA (math backend by default);
  * "hip":   this build's drop-in op nanonemo::flash_attn on (B, heads, T, hd) views (the reference's
             "cuda" setting, layers.py:89-93,106-108, including its transposes and copies);
  * "hip_bthd": the layout-fused op nanonemo::flash_attn_bthd, which reads the projections and RoPE
             output in their (B, T, heads, hd) layout and writes o where the output projection reads it.
``rope_kernel="hip"`` rotates q and k with this build's RoPE kernel (nanonemo::rope_qk), ``rope_kernel="fused"``
rotates k with it and q inside the layout-fused attention op (nanonemo::flash_attn_bthd_rope), and
``norm_kernel="hip"`` runs the residual add + RMSNorm on either side of attention as this build's fused
kernel (nanonemo::cuda_add_rms_norm_fwd / _bwd, the reference's norm_kernel="cuda"); everything else
is plain PyTorch.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn
from torch.nn.attention import SDPBackend, sdpa_kernel


@dataclass
class ModelConfig:
    """Hyperparameters of /root/reference/nanonemo/model/config.py:6-53 (the attention-relevant subset)."""

    n_layers: int = 12
    d_model: int = 768
    n_heads: int = 12
    n_kv_heads: int = 4
    d_ff: int = 2048
    vocab_size: int = 50304
    max_seq_len: int = 1024
    norm_eps: float = 1e-5
    rope_base: float = 10000.0
    init_std: float = 0.02
    # SDPA backend of the "torch" attention: "math" and "mem_efficient" as in the reference (config.py:30),
    # "math_fp32": the math backend on q, k, v upcast to fp32 (autocast off inside), output cast back; the
    # reference attention that the tests and the config-5 comparison use (an fp32 reference, and no 16-bit
    # batched products on transposed operands, which the math backend's forward and backward make)
    attn_backend: str = "math"
    attn_kernel: str = "torch"  # "torch" | "hip" | "hip_bthd"
    # "torch" | "hip" (q and k rotated in one launch, nanonemo::rope_qk) | "fused" (q rotated inside the attention
    # op nanonemo::flash_attn_bthd_rope, k alone by nanonemo::rope_qk; needs attn_kernel="hip_bthd")
    rope_kernel: str = "torch"
    norm_kernel: str = "torch"  # "torch" | "hip" (fused residual add + RMSNorm, nanonemo::cuda_add_rms_norm_*)

    def __post_init__(self):
        if self.d_model % self.n_heads:
            raise ValueError("d_model must divide evenly into heads")
        if self.n_heads % self.n_kv_heads:
            raise ValueError("query heads must group evenly over KV heads")
        if self.head_dim % 2:
            raise ValueError("RoPE rotates pairs of dimensions")
        if self.attn_backend not in ("math", "mem_efficient", "math_fp32"):
            raise ValueError(f"unknown attn_backend {self.attn_backend!r}")
        if self.attn_kernel not in ("torch", "hip", "hip_bthd"):
            raise ValueError(f"unknown attn_kernel {self.attn_kernel!r}")
        if self.rope_kernel not in ("torch", "hip", "fused"):
            raise ValueError(f"unknown rope_kernel {self.rope_kernel!r}")
        if self.rope_kernel == "fused" and self.attn_kernel != "hip_bthd":
            raise ValueError('rope_kernel="fused" needs attn_kernel="hip_bthd"')
        if self.norm_kernel not in ("torch", "hip"):
            raise ValueError(f"unknown norm_kernel {self.norm_kernel!r}")

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads


class RMSNorm(nn.Module):
    """x / rms(x) * w, reduced in fp32 (as layers.py:23-33) and returned in x's dtype."""

    def __init__(self, dim: int, eps: float):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        return (xf * torch.rsqrt(xf.square().mean(-1, keepdim=True) + self.eps) * self.weight.float()).to(x.dtype)


class AddRMSNorm(RMSNorm):
    """(rmsnorm(x + delta), x + delta): the pending sublayer output joins the stream here (layers.py:36-56).
    kernel="hip" does both in one pass with this build's fused kernel."""

    def __init__(self, dim: int, eps: float, kernel: str = "torch"):
        super().__init__(dim, eps)
        self.fused = None
        if kernel == "hip":
            from nanonemo_amd.kernels.hip.rmsnorm import add_rms_norm  # raises without the library

            self.fused = add_rms_norm

    def forward(self, x: torch.Tensor, delta: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        if self.fused is not None:
            return self.fused(x, delta, self.weight, self.eps)
        if delta is not None:
            x = x + delta
        return super().forward(x), x


def rope_tables(head_dim: int, max_seq_len: int, base: float) -> tuple[torch.Tensor, torch.Tensor]:
    """cos, sin of m * theta_i, shape (max_seq_len, head_dim // 2), fp32 (layers.py:59-64).

    theta_i = 1 / base^(2i / head_dim), rounded as the reference rounds it (a reciprocal of the fp32 power,
    not a negative power: the two differ in the last bit for some i), and m * theta_i as one fp32 product."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    ang = torch.outer(torch.arange(max_seq_len, dtype=torch.float32), inv_freq)
    return ang.cos(), ang.sin()


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, seq_dim: int) -> torch.Tensor:
    """Rotate-half RoPE (dimension i pairs with i + hd/2, layers.py:67-74) along ``seq_dim`` of a 4-D x."""
    T, half = x.shape[seq_dim], x.shape[-1] // 2
    shape = [1, 1, 1, half]
    shape[seq_dim] = T
    c, s = cos[:T].view(shape), sin[:T].view(shape)
    xf = x.float()
    a, b = xf[..., :half], xf[..., half:]
    return torch.cat((a * c - b * s, a * s + b * c), dim=-1).to(x.dtype)


class Attention(nn.Module):
    """Causal GQA self-attention (layers.py:77-116)."""

    def __init__(self, cfg: ModelConfig):
        super().__init__()
        self.cfg = cfg
        self.H, self.KVH, self.hd = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        self.wq = nn.Linear(cfg.d_model, self.H * self.hd, bias=False)
        self.wk = nn.Linear(cfg.d_model, self.KVH * self.hd, bias=False)
        self.wv = nn.Linear(cfg.d_model, self.KVH * self.hd, bias=False)
        self.wo = nn.Linear(self.H * self.hd, cfg.d_model, bias=False)
        if cfg.attn_kernel != "torch":
            from nanonemo_amd.kernels.hip import flash_attn as fa  # registers the ops; raises without the library

            self._fa = fa
        if cfg.rope_kernel in ("hip", "fused"):
            from nanonemo_amd.kernels.hip.rope import rope_k, rope_qk

            self._rope_qk, self._rope_k = rope_qk, rope_k

    def forward(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        B, T, _ = x.shape
        q = self.wq(x).view(B, T, self.H, self.hd)
        k = self.wk(x).view(B, T, self.KVH, self.hd)
        v = self.wv(x).view(B, T, self.KVH, self.hd)
        if self.cfg.rope_kernel == "fused":  # k rotated here, q inside the attention op
            k = self._rope_k(k, cos, sin)
            return self.wo(self._fa.flash_attn_bthd_rope(q, k, v, cos, sin).view(B, T, -1))
        hip_rope = self.cfg.rope_kernel == "hip"
        if hip_rope:  # in the projection layout, q and k in one launch
            q, k = self._rope_qk(q, k, cos, sin)
        if self.cfg.attn_kernel == "hip_bthd":
            if not hip_rope:
                q, k = rope(q, cos, sin, seq_dim=1), rope(k, cos, sin, seq_dim=1)
            return self.wo(self._fa.flash_attn_bthd(q, k, v).view(B, T, -1))
        q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)  # (B, heads, T, hd) views
        if not hip_rope:
            q, k = rope(q, cos, sin, seq_dim=2), rope(k, cos, sin, seq_dim=2)
        if self.cfg.attn_kernel == "hip":
            y = self._fa.flash_attn(q, k, v)
        else:
            g = self.H // self.KVH
            kr, vr = k.repeat_interleave(g, dim=1), v.repeat_interleave(g, dim=1)
            if self.cfg.attn_backend == "math_fp32":
                with torch.autocast(q.device.type, enabled=False), sdpa_kernel(SDPBackend.MATH):
                    y = F.scaled_dot_product_attention(q.float(), kr.float(), vr.float(), is_causal=True).to(q.dtype)
            else:
                backend = {"math": SDPBackend.MATH, "mem_efficient": SDPBackend.EFFICIENT_ATTENTION}[self.cfg.attn_backend]
                with sdpa_kernel(backend):
                    y = F.scaled_dot_product_attention(q, kr, vr, is_causal=True)
        return self.wo(y.transpose(1, 2).reshape(B, T, -1))


class MLP(nn.Module):
    """SwiGLU: down(silu(gate(x)) * up(x)) (layers.py:119-137)."""

    def __init__(self, cfg: ModelConfig):
        super().__init__()
        self.w_gate = nn.Linear(cfg.d_model, cfg.d_ff, bias=False)
        self.w_up = nn.Linear(cfg.d_model, cfg.d_ff, bias=False)
        self.w_down = nn.Linear(cfg.d_ff, cfg.d_model, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.w_down(F.silu(self.w_gate(x)) * self.w_up(x))


class Block(nn.Module):
    """Pre-norm block; returns (stream, pending MLP output) like layers.py:140-161."""

    def __init__(self, cfg: ModelConfig):
        super().__init__()
        self.norm_attn = AddRMSNorm(cfg.d_model, cfg.norm_eps, cfg.norm_kernel)
        self.attn = Attention(cfg)
        self.norm_mlp = AddRMSNorm(cfg.d_model, cfg.norm_eps, cfg.norm_kernel)
        self.mlp = MLP(cfg)

    def forward(self, x, cos, sin, delta=None):
        h, x = self.norm_attn(x, delta)
        h, x = self.norm_mlp(x, self.attn(h, cos, sin))
        return x, self.mlp(h)


class NanoNemo(nn.Module):
    """Decoder-only LM (model.py:13-70): embedding, n_layers blocks, final norm, tied lm_head."""

    def __init__(self, cfg: ModelConfig):
        super().__init__()
        self.cfg = cfg
        self.tok_emb = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.blocks = nn.ModuleList(Block(cfg) for _ in range(cfg.n_layers))
        self.norm_out = AddRMSNorm(cfg.d_model, cfg.norm_eps, cfg.norm_kernel)
        self.lm_head = nn.Linear(cfg.d_model, cfg.vocab_size, bias=False)
        self.lm_head.weight = self.tok_emb.weight
        cos, sin = rope_tables(cfg.head_dim, cfg.max_seq_len, cfg.rope_base)
        self.register_buffer("rope_cos", cos, persistent=False)
        self.register_buffer("rope_sin", sin, persistent=False)
        for m in self.modules():
            if isinstance(m, (nn.Linear, nn.Embedding)):
                nn.init.normal_(m.weight, std=cfg.init_std)
        resid_std = cfg.init_std / math.sqrt(2 * cfg.n_layers)
        for blk in self.blocks:
            nn.init.normal_(blk.attn.wo.weight, std=resid_std)
            nn.init.normal_(blk.mlp.w_down.weight, std=resid_std)

    def forward(self, idx: torch.Tensor, targets: torch.Tensor | None = None):
        T = idx.shape[1]
        if T > self.cfg.max_seq_len:
            raise ValueError(f"sequence length {T} > max_seq_len {self.cfg.max_seq_len}")
        x, delta = self.tok_emb(idx), None
        for blk in self.blocks:
            x, delta = blk(x, self.rope_cos, self.rope_sin, delta)
        h = self.norm_out(x, delta)[0]
        logits = self.lm_head(h)
        loss = None
        if targets is not None:
            loss = F.cross_entropy(logits.float().view(-1, logits.size(-1)), targets.reshape(-1))
        return logits, loss

    def num_params(self, non_embedding: bool = False) -> int:
        n = sum(p.numel() for p in self.parameters())  # the tied weight counts once
        return n - self.tok_emb.weight.numel() if non_embedding else n

    def flops_per_token(self, seq_len: int) -> float:
        """Training FLOPs per token: 6 per non-embedding parameter and per lm_head weight, plus the
        attention products in the full-square convention (12 * n_layers * d_model * T)."""
        cfg = self.cfg
        return 6.0 * (self.num_params(non_embedding=True) + cfg.vocab_size * cfg.d_model) + 12.0 * cfg.n_layers * cfg.d_model * seq_len
