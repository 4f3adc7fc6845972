"""Writes the committed golden fixtures tests/golden/*.npz from the float64 oracle (oracle/attention.py).

The reference holds no stored vectors for this path (tests/kernels/test_flash_attn.py draws seeded
inputs and compares against PyTorch at run time), so the fixtures are this build's own: inputs drawn
the reference's way (torch.manual_seed(seed), then randn for q, k, v and dO in that order,
/root/reference/tests/kernels/test_flash_attn.py:16-21), rounded to the case's 16-bit dtype, and the
oracle's float64 outputs on exactly those rounded inputs, stored as float32.

Shapes: the reference test SHAPES (test_flash_attn.py:12) that fit a small file, plus BASELINE config 1
(B=1, T=256, 12 Q / 4 KV heads, d=64) and a bf16 case with inputs x3 (config 3's softmax stress).

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import attention as oracle  # noqa: E402

# name: (B, H, KVH, T, D, dtype, input scale)
CASES = {
    "mha_t37_f16": (2, 4, 4, 37, 64, torch.float16, 1.0),
    "t1_d32_f16": (1, 1, 1, 1, 32, torch.float16, 1.0),
    "gqa4_t65_d32_f16": (3, 8, 2, 65, 32, torch.float16, 1.0),
    "gqa4_t65_d32_bf16": (3, 8, 2, 65, 32, torch.bfloat16, 1.0),
    "gqa3_t200_bf16_x3": (1, 6, 2, 200, 64, torch.bfloat16, 3.0),
    "cfg1_t256_bf16": (1, 12, 4, 256, 64, torch.bfloat16, 1.0),
}


def make_inputs(B, H, KVH, T, D, dtype, mult=1.0, seed=0):
    """Seeded CPU inputs in the reference's draw order (q, k, v, then dO), rounded to ``dtype``."""
    torch.manual_seed(seed)
    q = (torch.randn(B, H, T, D) * mult).to(dtype)
    k = (torch.randn(B, KVH, T, D) * mult).to(dtype)
    v = (torch.randn(B, KVH, T, D) * mult).to(dtype)
    do = torch.randn(B, H, T, D).to(dtype)
    return q, k, v, do


def bits(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.int16).numpy().view(np.uint16)


def main() -> None:
    for name, (B, H, KVH, T, D, dtype, mult) in CASES.items():
        q, k, v, do = make_inputs(B, H, KVH, T, D, dtype, mult)
        qd, kd, vd, dod = (t.double().numpy() for t in (q, k, v, do))
        o, lse = oracle.forward(qd, kd, vd)
        dq, dk, dv = oracle.backward(dod, qd, kd, vd, o, lse)
        np.savez_compressed(
            HERE / f"{name}.npz",
            shape=np.array([B, H, KVH, T, D]),
            dtype=np.array(str(dtype).replace("torch.", "")),
            mult=np.array(mult),
            q=bits(q), k=bits(k), v=bits(v), do=bits(do),
            o=o.astype(np.float32), lse=lse.astype(np.float32),
            dq=dq.astype(np.float32), dk=dk.astype(np.float32), dv=dv.astype(np.float32),
        )
        print(name, (HERE / f"{name}.npz").stat().st_size, "bytes")


if __name__ == "__main__":
    main()
