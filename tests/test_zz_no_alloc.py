"""nn_fa_bwd_noalloc (the backward whose workspace is the library's own device array) against nn_fa_bwd with a
caller workspace, through the C ABI: bit-identical outputs (the same kernels on the same inputs), on two calls
in a row where the second is smaller (the array keeps the first call's contents), at an unsplit shape and at a
shape whose dK/dV work is split (partials in the array), and a shape too large for the array is rejected."""

from __future__ import annotations

import pytest
import torch

from tests.common import make_inputs

pytestmark = pytest.mark.gpu


def _run_both(L, B, H, KVH, T, D, seed, dtype=torch.bfloat16):
    from nanonemo_amd.kernels.hip import DTYPE_BF16, DTYPE_F16, check

    code = DTYPE_BF16 if dtype == torch.bfloat16 else DTYPE_F16
    print(f"\n[case] nn_fa_bwd_noalloc vs nn_fa_bwd B={B} H={H} KVH={KVH} T={T} D={D} {dtype} seed={seed}", flush=True)
    q, k, v, do = (t.cuda() for t in make_inputs(B, H, KVH, T, D, dtype, seed=seed))
    o, lse = torch.empty_like(q), torch.empty(B, H, T, device="cuda")
    sp = torch.cuda.current_stream().cuda_stream
    p = lambda t: t.data_ptr()  # noqa: E731
    check(L.nn_fa_fwd(p(q), p(k), p(v), p(o), p(lse), B, H, KVH, T, D, code, D ** -0.5, sp))
    wsb = L.nn_fa_bwd_workspace_size(B, H, KVH, T, D)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    ref = [torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)]
    check(L.nn_fa_bwd(p(do), p(q), p(k), p(v), p(o), p(lse), *(p(t) for t in ref), p(ws), wsb, B, H, KVH, T, D,
                      code, D ** -0.5, sp))
    got = [torch.full_like(t, float("nan")) for t in ref]
    check(L.nn_fa_bwd_noalloc(p(do), p(q), p(k), p(v), p(o), p(lse), *(p(t) for t in got), B, H, KVH, T, D,
                              code, D ** -0.5, sp))
    torch.cuda.synchronize()
    for name, a, r in zip(("dq", "dk", "dv"), got, ref):
        assert torch.equal(a, r), f"{name} differs at B={B} H={H} KVH={KVH} T={T}: max |diff| {(a.float() - r.float()).abs().max().item()}"


@pytest.mark.parametrize(
    "first, second",
    [
        ((8, 12, 4, 1024, 64), (2, 12, 4, 200, 64)),  # unsplit, then a smaller ragged one
        ((2, 12, 1, 1024, 64), (1, 12, 1, 300, 32)),  # split dK/dV (partials in the array), then smaller
    ],
)
def test_noalloc_backward_matches_workspace_backward_twice(first, second):
    from nanonemo_amd.kernels.hip import lib

    L = lib()
    _run_both(L, *first, seed=5)
    _run_both(L, *second, seed=6)


def test_noalloc_backward_matches_workspace_backward_in_fp16():
    from nanonemo_amd.kernels.hip import lib

    L = lib()
    _run_both(L, 2, 12, 1, 1024, 64, seed=9, dtype=torch.float16)  # split dK/dV
    _run_both(L, 3, 8, 4, 129, 64, seed=10, dtype=torch.float16)


def test_noalloc_backward_rejects_shapes_beyond_its_array():
    from nanonemo_amd.kernels.hip import DTYPE_BF16, lib

    L = lib()
    B, H, KVH, T, D = 64, 16, 4, 8192, 64  # -D and -lse/scale alone need 64 MiB
    assert L.nn_fa_bwd_workspace_size(B, H, KVH, T, D) > 32 << 20
    rc = L.nn_fa_bwd_noalloc(*([None] * 9), B, H, KVH, T, D, DTYPE_BF16, 0.125, torch.cuda.current_stream().cuda_stream)
    assert rc != 0 and b"scratch" in L.nn_fa_last_error()


def test_noalloc_backward_captures_into_a_graph_without_a_workspace():
    # The caller it exists for: a HIP-graph capture of fwd + bwd whose only buffers are the inputs and outputs
    # (nothing is allocated for the backward). Replays, with the outputs poisoned and eager work in between, equal
    # the eager nn_fa_bwd with a caller workspace bit for bit.
    from nanonemo_amd.kernels.hip import DTYPE_BF16, check, lib

    L = lib()
    B, H, KVH, T, D = 2, 12, 4, 384, 64
    print(f"\n[case] graph capture of nn_fa_fwd + nn_fa_bwd_noalloc B={B} H={H} KVH={KVH} T={T} D={D}", flush=True)
    q, k, v, do = (t.cuda() for t in make_inputs(B, H, KVH, T, D, torch.bfloat16, seed=8))
    o, lse = torch.empty_like(q), torch.empty(B, H, T, device="cuda")
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    p = lambda t: t.data_ptr()  # noqa: E731

    def launch(st):
        check(L.nn_fa_fwd(p(q), p(k), p(v), p(o), p(lse), B, H, KVH, T, D, DTYPE_BF16, 0.125, st))
        check(L.nn_fa_bwd_noalloc(p(do), p(q), p(k), p(v), p(o), p(lse), p(dq), p(dk), p(dv), B, H, KVH, T, D,
                                  DTYPE_BF16, 0.125, st))

    wsb = L.nn_fa_bwd_workspace_size(B, H, KVH, T, D)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    ref = [torch.empty_like(t) for t in (dq, dk, dv)]
    sp = torch.cuda.current_stream().cuda_stream
    launch(sp)  # first call on the device looks the array up, outside the capture
    check(L.nn_fa_bwd(p(do), p(q), p(k), p(v), p(o), p(lse), *(p(t) for t in ref), p(ws), wsb, B, H, KVH, T, D,
                      DTYPE_BF16, 0.125, sp))
    o_ref, lse_ref = o.clone(), lse.clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for i in range(3):
        for t in (o, lse, dq, dk, dv):
            t.fill_(float("nan"))
        junk = torch.randn(1 << 20, device="cuda") * i
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, a, r in (("o", o, o_ref), ("lse", lse, lse_ref), ("dq", dq, ref[0]), ("dk", dk, ref[1]),
                           ("dv", dv, ref[2])):
            assert torch.equal(a, r), f"replay {i}: {name} differs"
        del junk
