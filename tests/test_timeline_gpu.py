"""The timeline build (libnanonemo_fa_timeline.so, the attention kernels with NN_TIMELINE=1, behind
`bench.py --timeline`): its outputs equal the product library's bit for bit (the stamps change nothing the
kernels compute), and every block of each launch leaves a consistent record: the 100 MHz clock's end after its
start, the shader clock's first-tile stamp between the block's start and end, an XCD id below 8, and, for the
forward and dQ, the block's tile count."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from tests.common import make_inputs

pytestmark = pytest.mark.gpu


def test_timeline_build_matches_product_and_records_every_block():
    from nanonemo_amd.build import TIMELINE_LIB
    from nanonemo_amd.kernels.hip import DTYPE_BF16, SIGNATURES, check, lib

    B, H, KVH, T, D = 2, 12, 4, 384, 64
    print(f"\n[case] timeline build vs product B={B} H={H} KVH={KVH} T={T} D={D} bf16", flush=True)
    TL = ctypes.CDLL(str(TIMELINE_LIB))
    for name in ("nn_fa_fwd", "nn_fa_bwd", "nn_fa_bwd_workspace_size", "nn_fa_last_error"):
        fn = getattr(TL, name)
        fn.restype, fn.argtypes = SIGNATURES[name]
    TL.nn_fa_timeline_read.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int]

    def ok(rc):
        assert rc == 0, TL.nn_fa_last_error()

    q, k, v, do = (t.cuda() for t in make_inputs(B, H, KVH, T, D, torch.bfloat16, seed=11))
    sp = torch.cuda.current_stream().cuda_stream
    p = lambda t: t.data_ptr()  # noqa: E731
    wsb = lib().nn_fa_bwd_workspace_size(B, H, KVH, T, D)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    outs = {}
    for name, L, chk in (("product", lib(), check), ("timeline", TL, ok)):
        o, lse = torch.empty_like(q), torch.empty(B, H, T, device="cuda")
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        if name == "timeline":
            ok(TL.nn_fa_timeline_clear())
        chk(L.nn_fa_fwd(p(q), p(k), p(v), p(o), p(lse), B, H, KVH, T, D, DTYPE_BF16, D ** -0.5, sp))
        chk(L.nn_fa_bwd(p(do), p(q), p(k), p(v), p(o), p(lse), p(dq), p(dk), p(dv), p(ws), wsb, B, H, KVH, T, D,
                        DTYPE_BF16, D ** -0.5, sp))
        torch.cuda.synchronize()
        outs[name] = (o, lse, dq, dk, dv)
    for n, a, b in zip(("o", "lse", "dq", "dk", "dv"), outs["product"], outs["timeline"]):
        assert torch.equal(a, b), f"{n} differs between the product and the timeline build"

    nqb = (T + 127) // 128
    for kern, name in enumerate(("fwd", "dq", "dkdv")):
        r = np.zeros((16384, 16), dtype=np.uint64)
        ok(TL.nn_fa_timeline_read(kern, r.ctypes.data, 16384))
        r = r.astype(np.int64)
        used = r[:, 0] != 0
        n = int(used.sum())
        if name in ("fwd", "dq"):
            assert n == nqb * B * H and used[:n].all(), f"{name}: {n} records"
            # tile counts: every query block index once per head, qb + 1 tiles of 128 keys (T = 3 * 128)
            assert sorted(np.bincount(r[:n, 7], minlength=nqb + 1)[1:].tolist()) == [B * H] * nqb
        else:
            assert n > 0 and used[:n].all(), f"{name}: {n} records"
        r = r[:n]
        assert (r[:, 1] > r[:, 0]).all(), f"{name}: a block ends before it starts"
        assert (r[:, 4] >= r[:, 2]).all(), f"{name}: shader-clock end before start"
        ready = (r[:, 3] >= r[:, 2]) & (r[:, 4] >= r[:, 3])
        if name == "dkdv":  # wave 0 stamps its first tile only if it has an iteration (a split may leave it none)
            ready |= r[:, 3] == 0
        assert ready.all(), f"{name}: first-tile stamp outside the block's lifetime"
        assert (((r[:, 5] >> 32) & 0xF) < 8).all(), f"{name}: XCD id out of range"
