"""HIP-graph capture of the C ABI (the launch pattern the reference's benchmark times, benchmarks/kernels/
common.py:30-54, and that compile(mode="reduce-overhead") relies on, trainer.py:48-55).

The library allocates, frees, synchronises and memsets nothing, so its calls can be captured. Here the
calls themselves are captured with torch.cuda.graph on buffers allocated beforehand (no autograd inside
the capture): one nn_fa_fwd + nn_fa_bwd pair (also at a shape whose dK/dV work is split, which adds the
partial-sum kernel), and the RoPE and fused add + RMSNorm kernels beside it.
Each graph is replayed several times with eager work and synchronisations in between, outputs poisoned
before every replay; every replay must equal the eager result bit for bit.
"""

from __future__ import annotations

import pytest
import torch

from tests.common import make_inputs

pytestmark = pytest.mark.gpu


def _replays_match(launch, outs, n=4, names=None):
    """Eager run, capture, then n poisoned replays compared bit for bit with the eager outputs. A mismatch is
    reported with the output it is in, how many elements differ, the largest difference and any NaNs."""
    names = names or [f"output {i}" for i in range(len(outs))]
    launch(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ref = [t.clone() for t in outs]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # a warm call on a side stream before capture, as torch recommends
        launch(side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for i in range(n):
        for t in outs:  # eager work between replays, and no stale result can pass
            t.fill_(float("nan")) if t.is_floating_point() else t.fill_(0)
        junk = torch.randn(1 << 20, device="cuda") * i
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        bad = []
        for name, a, r in zip(names, outs, ref):
            if not torch.equal(a, r):
                d = (a.float() - r.float()).abs()
                ne = (a != r).nonzero()
                bad.append(f"{name}: {ne.shape[0]} of {a.numel()} elements differ, max |diff| {d.nan_to_num(float('inf')).max().item():.3e}, "
                           f"NaNs in the replay {a.isnan().sum().item()}, first at {ne[0].tolist()}")
        assert not bad, f"replay {i} differs from the eager result: " + "; ".join(bad)
        del junk


@pytest.mark.parametrize("B, H, KVH, T, D", [(2, 12, 4, 256, 64), (2, 12, 1, 1024, 64)])  # the second splits dK/dV
def test_captured_fwd_bwd_c_abi_calls_replay_bit_identically(B, H, KVH, T, D):
    from nanonemo_amd.kernels.hip import DTYPE_BF16, check, lib

    L = lib()
    print(f"\n[case] graph capture of nn_fa_fwd + nn_fa_bwd B={B} H={H} KVH={KVH} T={T} D={D}", flush=True)
    q, k, v, do = (t.cuda() for t in make_inputs(B, H, KVH, T, D, torch.bfloat16, seed=2))
    o, dq = torch.empty_like(q), torch.empty_like(q)
    dk, dv = torch.empty_like(k), torch.empty_like(v)
    lse = torch.empty(B, H, T, device="cuda")
    wsb = L.nn_fa_bwd_workspace_size(B, H, KVH, T, D)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    p = lambda t: t.data_ptr()  # noqa: E731

    def launch(stream):
        check(L.nn_fa_fwd(p(q), p(k), p(v), p(o), p(lse), B, H, KVH, T, D, DTYPE_BF16, 0.125, stream))
        check(L.nn_fa_bwd(p(do), p(q), p(k), p(v), p(o), p(lse), p(dq), p(dk), p(dv), p(ws), wsb, B, H, KVH, T, D,
                          DTYPE_BF16, 0.125, stream))

    _replays_match(launch, [o, lse, dq, dk, dv], names=["o", "lse", "dq", "dk", "dv"])


def test_captured_rope_and_rmsnorm_c_abi_calls_replay_bit_identically():
    from nanonemo_amd.kernels.hip import check_rmsnorm, check_rope, lib, strides3
    from nanonemo_amd.model import rope_tables

    L = lib()
    B, T, H, KVH, D, N = 2, 128, 12, 4, 64, 768
    print(f"\n[case] graph capture of nn_rope_qk + nn_add_rmsnorm_fwd / _bwd", flush=True)
    g = torch.Generator(device="cuda").manual_seed(3)
    q = torch.randn(B, T, H, D, device="cuda", generator=g).bfloat16()
    k = torch.randn(B, T, KVH, D, device="cuda", generator=g).bfloat16()
    qo, ko = torch.empty_like(q), torch.empty_like(k)
    cos, sin = (t.cuda() for t in rope_tables(D, T, 10000.0))
    M = B * T
    x = torch.randn(M, N, device="cuda", generator=g)
    d = torch.randn(M, N, device="cuda", generator=g).bfloat16()
    w = 1 + 0.1 * torch.randn(N, device="cuda", generator=g)
    y, h, rstd = torch.empty(M, N, device="cuda", dtype=torch.bfloat16), torch.empty(M, N, device="cuda"), torch.empty(M, device="cuda")
    dy = torch.randn(M, N, device="cuda", generator=g).bfloat16()
    dh = torch.randn(M, N, device="cuda", generator=g)
    dx, dd, dw = torch.empty(M, N, device="cuda"), torch.empty(M, N, device="cuda", dtype=torch.bfloat16), torch.empty(N, device="cuda")
    wsb = L.nn_add_rmsnorm_bwd_workspace_size(M, N)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    p = lambda t: t.data_ptr()  # noqa: E731

    def launch(stream):
        check_rope(L.nn_rope_qk(p(q), p(qo), p(k), p(ko), p(cos), p(sin), B, T, H, KVH, D,
                                strides3(T * H * D, H * D, D), strides3(T * KVH * D, KVH * D, D), T, 1, stream))
        check_rmsnorm(L.nn_add_rmsnorm_fwd(p(x), p(d), p(w), p(y), p(h), p(rstd), M, N, 1e-5, 2, 1, 1, stream))
        check_rmsnorm(L.nn_add_rmsnorm_bwd(p(dy), p(dh), p(h), p(w), p(rstd), p(dx), p(dd), p(dw), p(ws), wsb, M, N,
                                           1, 2, 2, 1, stream))

    _replays_match(launch, [qo, ko, y, h, rstd, dx, dd, dw])
