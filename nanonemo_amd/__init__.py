"""nanonemo_amd: MI355X (gfx950) causal grouped-query FlashAttention-2 for NanoNemo.

The public entry point mirrors /root/reference/nanonemo/kernels/cuda/flash_attn.py:57-60:

    from nanonemo_amd.kernels.hip.flash_attn import flash_attn
    o = flash_attn(q, k, v)   # q (B, H, T, hd), k/v (B, KVH, T, hd), fp16 or bf16, causal

Importing the op module registers the torch.library ops ``nanonemo::flash_attn`` and
``nanonemo::flash_attn_bwd`` (same names and schemas as the reference).
"""

__version__ = "0.1.0"
