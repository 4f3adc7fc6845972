"""CPU tests of the drop-in boundary: the C-ABI library, its exports, its argument checks, and the
torch.library ops' schemas, fake impls and input validation. No GPU compute is launched here."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from nanonemo_amd.kernels.hip import ABI_VERSION, LIB_PATH, SIGNATURES, lib

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))


def _declared_symbols() -> list[str]:
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(nn_\w+)\s*\(", text))
    return sorted(names)


def test_library_is_built():
    assert LIB_PATH.exists(), "run `python -m nanonemo_amd.build` (or __graft_entry__.build()) first"


def test_library_exports_every_header_symbol():
    handle = ctypes.CDLL(str(LIB_PATH))
    declared = _declared_symbols()
    assert declared, "no declarations parsed from the header"
    for name in declared:
        assert hasattr(handle, name), f"{name} declared in include/ but not exported"
    # and the Python binding declares a signature for each of them
    assert sorted(SIGNATURES) == declared


def test_abi_version():
    assert lib().nn_fa_abi_version() == ABI_VERSION


def test_timeline_build_is_separate_and_rejects_bad_arguments():
    # bench.py --timeline's library is the attention library built with NN_TIMELINE=1: it exports the same
    # attention entry points plus nn_fa_timeline_*, which the product library does not have; its record read
    # refuses arguments outside the record array before any device call.
    from nanonemo_amd.build import TIMELINE_LIB

    assert TIMELINE_LIB.exists(), "run `python -m nanonemo_amd.build` first"
    TL = ctypes.CDLL(str(TIMELINE_LIB))
    for name in ("nn_fa_timeline_dims", "nn_fa_timeline_clear", "nn_fa_timeline_read"):
        assert hasattr(TL, name) and not hasattr(lib(), name), name
    for name in _declared_symbols():
        if name.startswith("nn_fa_"):
            assert hasattr(TL, name), f"{name} missing from the timeline build"
    dims = [ctypes.c_int() for _ in range(3)]
    TL.nn_fa_timeline_dims.argtypes = [ctypes.POINTER(ctypes.c_int)] * 3
    assert TL.nn_fa_timeline_dims(*(ctypes.byref(d) for d in dims)) == 0
    assert [d.value for d in dims] == [3, 16384, 16]
    TL.nn_fa_timeline_read.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
    TL.nn_fa_last_error.restype = ctypes.c_char_p
    buf = (ctypes.c_uint64 * 16)()
    for kern, n in ((3, 1), (-1, 1), (0, 16385), (0, -1)):
        assert TL.nn_fa_timeline_read(kern, buf, n) != 0 and b"invalid" in TL.nn_fa_last_error()
    assert TL.nn_fa_timeline_read(0, None, 1) != 0


def _dkdv_split(B, H, KVH, T):
    """Blocks sharing one dK/dV unit pair: 1 when the B*KVH*ceil(nkb/2) pairs fill 256 CUs, else up to 16,
    keeping at least 8 of a pair's (H/KVH)*(nkb+1) iterations per split, and none where 16 times a unit's
    (H/KVH)*nkb iterations would overflow the kernel's 32-bit split bounds."""
    nkb = (T + 63) // 64
    base = B * KVH * ((nkb + 1) // 2)
    if base <= 0 or base >= 256 or (H // KVH) * nkb * 16 >= 2**31:
        return 1
    return max(1, min(16, -(-256 // base), (H // KVH) * (nkb + 1) // 8))


@pytest.mark.parametrize(
    "B, H, KVH, T, D, split",
    [(8, 12, 4, 1024, 64, 1), (32, 12, 4, 1024, 64, 1), (8, 12, 1, 1024, 64, 4), (1, 12, 4, 1024, 64, 6),
     (1, 12, 4, 256, 64, 1), (2, 12, 1, 1024, 64, 16), (1, 8, 8, 700, 32, 1), (1, 1, 1, 1, 32, 1),
     (1, 1 << 27, 1, 64, 32, 1), (1, (1 << 27) - 8, 1, 64, 32, 16)],
)
def test_workspace_size(B, H, KVH, T, D, split):
    L = lib()
    assert _dkdv_split(B, H, KVH, T) == split
    vec = 4 * B * H * T  # -rowsum(dO * o) and -lse/scale, fp32 per query row
    rnd = lambda n: (n + 255) // 256 * 256  # noqa: E731
    part = split * 2 * 4 * B * KVH * T * D if split > 1 else 0  # fp32 dK / dV partials of each split
    assert L.nn_fa_bwd_workspace_size(B, H, KVH, T, D) == 2 * rnd(vec) + rnd(part)
    assert L.nn_fa_bwd_workspace_size(0, H, KVH, T, D) == 0


@pytest.mark.parametrize(
    "args, msg",
    [
        ((1, 4, 2, 16, 48, 1), "head_dim must be 32 or 64"),
        ((1, 4, 3, 16, 64, 1), "query heads must group evenly"),
        ((1, 4, 2, 16, 64, 7), "float16 or bfloat16"),
        ((1, 4, 0, 16, 64, 1), "invalid sizes"),
        ((-1, 4, 2, 16, 64, 1), "invalid sizes"),
    ],
)
def test_c_abi_rejects_bad_arguments_before_any_launch(args, msg):
    L = lib()
    B, H, KVH, T, D, dt = args
    rc = L.nn_fa_fwd(16, 16, 16, 16, 16, B, H, KVH, T, D, dt, 0.125, None)
    assert rc != 0
    assert msg in L.nn_fa_last_error().decode()
    rc = L.nn_fa_bwd(16, 16, 16, 16, 16, 16, 16, 16, 16, 256, 1 << 30, B, H, KVH, T, D, dt, 0.125, None)
    assert rc != 0 and msg in L.nn_fa_last_error().decode()


def test_c_abi_rejects_misaligned_and_small_workspace():
    L = lib()
    rc = L.nn_fa_fwd(8, 16, 16, 16, 16, 1, 4, 2, 16, 64, 1, 0.125, None)
    assert rc != 0 and "16-byte aligned" in L.nn_fa_last_error().decode()
    rc = L.nn_fa_bwd_dkdv(16, 16, 16, 16, 256, 10, 16, 16, 1, 4, 2, 16, 64, 1, 0.125, None)
    assert rc != 0 and "workspace too small" in L.nn_fa_last_error().decode()
    rc = L.nn_fa_bwd_dq(16, 16, 16, 16, 16, 16, 256, 10, 16, 1, 4, 2, 16, 64, 1, 0.125, None)
    assert rc != 0 and "workspace too small" in L.nn_fa_last_error().decode()
    rc = L.nn_fa_bwd_pre(16, 16, 16, 0, 1 << 20, 1, 4, 2, 16, 64, 1, 0.125, None)
    assert rc != 0 and "null workspace" in L.nn_fa_last_error().decode()


@pytest.mark.parametrize(
    "qs, ks, msg",
    [
        ((4096, 1024, 60), (4096, 1024, 64), "q/o strides must be positive multiples of 8"),
        ((4096, 1024, 64), (4096, 0, 64), "k/v strides must be positive multiples of 8"),
        ((4096, 1024, 32), (4096, 1024, 64), "q/o row stride is smaller than head_dim"),
        ((4096, 1024, 1 << 27), (4096, 1024, 64), "q/o strides too large"),
    ],
)
def test_strided_c_abi_rejects_bad_strides_before_any_launch(qs, ks, msg):
    from nanonemo_amd.kernels.hip import strides3

    L = lib()
    B, H, KVH, T, D = 1, 4, 2, 16, 64
    rc = L.nn_fa_fwd_strided(16, 16, 16, 16, 16, B, H, KVH, T, D, strides3(*qs), strides3(*ks), 1, 0.125, None)
    assert rc != 0 and msg in L.nn_fa_last_error().decode()
    rc = L.nn_fa_bwd_strided(16, 16, 16, 16, 16, 16, 16, 16, 16, 256, 1 << 30, B, H, KVH, T, D,
                             strides3(*qs), strides3(*ks), 1, 0.125, None)
    assert rc != 0 and msg in L.nn_fa_last_error().decode()
    rc = L.nn_fa_fwd_strided(16, 16, 16, 16, 16, B, H, KVH, T, D, None, strides3(*ks), 1, 0.125, None)
    assert rc != 0 and "null strides" in L.nn_fa_last_error().decode()


@pytest.mark.parametrize(
    "kw, msg",
    [
        (dict(D=56), "head_dim must be a multiple of 16"),
        (dict(dtype=5), "dtype must be float16, bfloat16 or float32"),
        (dict(T=40), "exceeds the 32 rows of the tables"),
        (dict(qs=(4096, 768, 60)), "q strides must be positive multiples of 8"),
        (dict(qp=24), "q must be 16-byte aligned"),
        (dict(cosp=None), "null table"),
    ],
)
def test_rope_c_abi_rejects_bad_arguments_before_any_launch(kw, msg):
    from nanonemo_amd.kernels.hip import strides3

    L = lib()
    a = dict(D=64, dtype=1, T=16, qs=(4096, 768, 64), qp=16, cosp=256)
    a.update(kw)
    rc = L.nn_rope_qk(a["qp"], 32, 64, 96, a["cosp"], 512, 1, a["T"], 12, 4, a["D"], strides3(*a["qs"]),
                      strides3(1024, 256, 64), 32, a["dtype"], None)
    assert rc != 0 and msg in L.nn_rope_last_error().decode()
    rc = L.nn_rope_qk_bwd(a["qp"], 32, 64, 96, a["cosp"], 512, 1, a["T"], 12, 4, a["D"], strides3(*a["qs"]),
                          strides3(1024, 256, 64), 32, a["dtype"], None)
    assert rc != 0 and msg in L.nn_rope_last_error().decode()


@pytest.mark.parametrize(
    "kw, msg",
    [
        (dict(N=4100), "hidden size must be <= 1024, or a multiple of 8 and <= 4096"),
        (dict(N=4104), "hidden size must be <= 1024, or a multiple of 8 and <= 4096"),
        (dict(N=0), "invalid sizes"),
        (dict(M=-1), "invalid sizes"),
        (dict(xdt=3), "dtype must be float16, bfloat16 or float32"),
        (dict(x=24), "tensors must be 16-byte aligned"),
        (dict(x=None), "null pointer argument"),
        (dict(eps=-1.0), "eps must be non-negative"),
    ],
)
def test_rmsnorm_c_abi_rejects_bad_arguments_before_any_launch(kw, msg):
    L = lib()
    a = dict(M=16, N=768, x=256, xdt=2, eps=1e-5)
    a.update(kw)
    rc = L.nn_add_rmsnorm_fwd(a["x"], 512, 1024, 2048, 4096, 8192, a["M"], a["N"], a["eps"], a["xdt"], 1, 1, None)
    assert rc != 0 and msg in L.nn_rmsnorm_last_error().decode()


def test_rmsnorm_c_abi_backward_checks_and_workspace():
    L = lib()
    # one fp32 dw row per block: a block of 8 waves has 16 teams (32-lane teams) for N <= 1024 with N % 8 == 0,
    # else 8 (64-lane teams); above 3072 (more than 48 values per lane) a block has 4 waves and 4 teams. One row per
    # team, or two for 3 units of 8 elements per lane (the pipelined kernel) where that gives 256 to 512 blocks; at
    # most 512 blocks, whose teams then walk further rows
    assert L.nn_add_rmsnorm_bwd_workspace_size(8192, 768) == 256 * 768 * 4
    assert L.nn_add_rmsnorm_bwd_workspace_size(16384, 768) == 512 * 768 * 4  # pipelined, the top of its range
    assert L.nn_add_rmsnorm_bwd_workspace_size(7, 768) == 1 * 768 * 4
    assert L.nn_add_rmsnorm_bwd_workspace_size(7, 4096) == 2 * 4096 * 4
    assert L.nn_add_rmsnorm_bwd_workspace_size(7, 3072) == 1 * 3072 * 4
    assert L.nn_add_rmsnorm_bwd_workspace_size(520, 768) == 33 * 768 * 4
    assert L.nn_add_rmsnorm_bwd_workspace_size(8160, 768) == 510 * 768 * 4  # two rows per team would leave 255 blocks
    assert L.nn_add_rmsnorm_bwd_workspace_size(520, 2048) == 65 * 2048 * 4
    assert L.nn_add_rmsnorm_bwd_workspace_size(1 << 20, 33) == 512 * 33 * 4
    assert L.nn_add_rmsnorm_bwd_workspace_size(0, 768) == 0
    args = (256, 512, 768, 1024, 2048, 4096, 8192, 16384)
    rc = L.nn_add_rmsnorm_bwd(*args, 32768, 10, 64, 768, 1, 2, 2, 1, None)
    assert rc != 0 and "workspace too small" in L.nn_rmsnorm_last_error().decode()
    rc = L.nn_add_rmsnorm_bwd(*args, None, 1 << 20, 64, 768, 1, 2, 2, 1, None)
    assert rc != 0 and "null workspace" in L.nn_rmsnorm_last_error().decode()
    rc = L.nn_add_rmsnorm_bwd(*args, 32768, 1 << 20, 64, 768, 1, 9, 2, 1, None)
    assert rc != 0 and "dtype" in L.nn_rmsnorm_last_error().decode()


def test_rmsnorm_ops_registered_with_reference_schemas():
    from nanonemo_amd.kernels.hip import rmsnorm  # noqa: F401

    fwd = str(torch.ops.nanonemo.cuda_add_rms_norm_fwd.default._schema)
    bwd = str(torch.ops.nanonemo.cuda_add_rms_norm_bwd.default._schema)
    assert fwd == ("nanonemo::cuda_add_rms_norm_fwd(Tensor x, Tensor? delta, Tensor weight, float eps, "
                   "ScalarType out_dtype) -> (Tensor, Tensor, Tensor)")
    assert bwd == ("nanonemo::cuda_add_rms_norm_bwd(Tensor dy, Tensor? dh, Tensor h, Tensor weight, Tensor rstd, "
                   "ScalarType dx_dtype, ScalarType? ddelta_dtype) -> (Tensor, Tensor, Tensor)")


def test_rmsnorm_fakes_follow_the_reference():
    from nanonemo_amd.kernels.hip import rmsnorm  # noqa: F401

    x = torch.empty(4, 16, 768, device="meta")
    d = torch.empty(4, 16, 768, dtype=torch.bfloat16, device="meta")
    w = torch.empty(768, device="meta")
    y, h, rstd = torch.ops.nanonemo.cuda_add_rms_norm_fwd(x, d, w, 1e-5, torch.bfloat16)
    assert y.dtype == torch.bfloat16 and h.dtype == torch.float32 and rstd.shape == (4, 16) and y.shape == x.shape
    y, h, _ = torch.ops.nanonemo.cuda_add_rms_norm_fwd(x, None, w, 1e-5, torch.float32)
    assert h.numel() == 0
    dx, dd, dw = torch.ops.nanonemo.cuda_add_rms_norm_bwd(y, h.new_empty(x.shape), x, w, rstd, torch.float32,
                                                          torch.bfloat16)
    assert dx.dtype == torch.float32 and dd.dtype == torch.bfloat16 and dw.shape == w.shape


def test_c_abi_empty_problem_is_a_no_op():
    # T == 0 and B == 0 return success without touching device memory (flash_attn.cu:367).
    L = lib()
    assert L.nn_fa_fwd(None, None, None, None, None, 1, 4, 2, 0, 64, 1, 0.125, None) == 0
    assert L.nn_fa_fwd(None, None, None, None, None, 0, 4, 2, 16, 64, 1, 0.125, None) == 0
    assert L.nn_fa_last_error().decode() == ""


# ---- torch.library ops -----------------------------------------------------------------------


def _ops():
    from nanonemo_amd.kernels.hip import flash_attn as fa

    return fa


def test_ops_registered_with_reference_schemas():
    _ops()
    fwd = torch.ops.nanonemo.flash_attn.default._schema
    bwd = torch.ops.nanonemo.flash_attn_bwd.default._schema
    assert str(fwd) == "nanonemo::flash_attn(Tensor q, Tensor k, Tensor v) -> (Tensor, Tensor)"
    assert str(bwd) == (
        "nanonemo::flash_attn_bwd(Tensor d_o, Tensor q, Tensor k, Tensor v, Tensor o, Tensor lse)"
        " -> (Tensor, Tensor, Tensor)"
    )


def test_layout_fused_ops_registered():
    _ops()
    fwd = torch.ops.nanonemo.flash_attn_bthd.default._schema
    bwd = torch.ops.nanonemo.flash_attn_bthd_bwd.default._schema
    assert str(fwd) == "nanonemo::flash_attn_bthd(Tensor q, Tensor k, Tensor v) -> (Tensor, Tensor)"
    assert str(bwd) == (
        "nanonemo::flash_attn_bthd_bwd(Tensor d_o, Tensor q, Tensor k, Tensor v, Tensor o, Tensor lse)"
        " -> (Tensor, Tensor, Tensor)"
    )


def test_layout_fused_fakes_keep_the_projection_layout():
    fa = _ops()
    B, T, H, KVH, D = 2, 64, 12, 4, 64
    q = torch.empty(B, T, H, D, dtype=torch.bfloat16, device="meta")
    k = torch.empty(B, T, KVH, D, dtype=torch.bfloat16, device="meta")
    o, lse = torch.ops.nanonemo.flash_attn_bthd(q, k, k)
    assert o.shape == (B, T, H, D) and o.is_contiguous() and lse.shape == (B, H, T) and lse.dtype == torch.float32
    dq, dk, dv = torch.ops.nanonemo.flash_attn_bthd_bwd(o, q, k, k, o, lse)
    assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == k.shape
    assert fa.flash_attn_bthd(q, k, k).view(B, T, H * D).shape == (B, T, H * D)


def test_rope_fused_ops_registered_and_faked():
    fa = _ops()
    fwd = str(torch.ops.nanonemo.flash_attn_bthd_rope.default._schema)
    bwd = str(torch.ops.nanonemo.flash_attn_bthd_rope_bwd.default._schema)
    assert fwd == "nanonemo::flash_attn_bthd_rope(Tensor q, Tensor k, Tensor v, Tensor cos, Tensor sin) -> (Tensor, Tensor, Tensor)"
    assert bwd == ("nanonemo::flash_attn_bthd_rope_bwd(Tensor d_o, Tensor q_rot, Tensor k, Tensor v, Tensor o, Tensor lse, "
                   "Tensor cos, Tensor sin) -> (Tensor, Tensor, Tensor)")
    B, T, H, KVH, D = 2, 64, 12, 4, 64
    q = torch.empty(B, T, H, D, dtype=torch.bfloat16, device="meta")
    k = torch.empty(B, T, KVH, D, dtype=torch.bfloat16, device="meta")
    cos = torch.empty(T, D // 2, device="meta")
    o, lse, q_rot = torch.ops.nanonemo.flash_attn_bthd_rope(q, k, k, cos, cos)
    assert o.shape == q_rot.shape == q.shape and o.is_contiguous() and lse.shape == (B, H, T)
    dq, dk, dv = torch.ops.nanonemo.flash_attn_bthd_rope_bwd(o, q_rot, k, k, o, lse, cos, cos)
    assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == k.shape
    assert fa.flash_attn_bthd_rope(q, k, k, cos, cos).shape == q.shape


def test_rope_fused_c_abi_checks_tables_before_any_launch():
    L = lib()
    s3 = (ctypes.c_int64 * 3)(1024 * 12 * 64, 64, 12 * 64)
    k3 = (ctypes.c_int64 * 3)(1024 * 4 * 64, 64, 4 * 64)
    args = (256, 512, 768, 1024, 2048, 4096)
    rc = L.nn_fa_fwd_rope_strided(*args, None, 8192, 1024, 1, 12, 4, 1024, 64, s3, k3, 1, 0.125, None)
    assert rc != 0 and b"null RoPE table" in L.nn_fa_last_error()
    rc = L.nn_fa_fwd_rope_strided(*args, 8192, 16384, 512, 1, 12, 4, 1024, 64, s3, k3, 1, 0.125, None)
    assert rc != 0 and b"exceeds the 512 rows" in L.nn_fa_last_error()
    rc = L.nn_fa_fwd_rope_strided(*args, 8200, 16384, 1024, 1, 12, 4, 1024, 64, s3, k3, 1, 0.125, None)
    assert rc != 0 and b"16-byte aligned" in L.nn_fa_last_error()
    ws = L.nn_fa_bwd_workspace_size(1, 12, 4, 1024, 64)
    rc = L.nn_fa_bwd_rope_strided(*args, 256, 512, 768, 256, ws, 8192, 16384, 1000, 1, 12, 4, 1024, 64, s3, k3, 1,
                                  0.125, None)
    assert rc != 0 and b"exceeds the 1000 rows" in L.nn_fa_last_error()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fake_impls_give_contiguous_outputs_for_strided_inputs(dtype):
    fa = _ops()
    B, H, KVH, T, D = 2, 12, 4, 64, 64
    q = torch.empty(B, T, H, D, dtype=dtype, device="meta").transpose(1, 2)
    k = torch.empty(B, T, KVH, D, dtype=dtype, device="meta").transpose(1, 2)
    v = torch.empty(B, KVH, T, D, dtype=dtype, device="meta")
    assert not q.is_contiguous()
    o, lse = torch.ops.nanonemo.flash_attn(q, k, v)
    assert o.shape == q.shape and o.dtype == dtype and o.is_contiguous()
    assert lse.shape == (B, H, T) and lse.dtype == torch.float32 and lse.is_contiguous()
    dq, dk, dv = torch.ops.nanonemo.flash_attn_bwd(o, q, k, v, o, lse)
    for g, t in ((dq, q), (dk, k), (dv, v)):
        assert g.shape == t.shape and g.dtype == t.dtype and g.is_contiguous()
    assert fa.flash_attn(q, k, v).shape == q.shape


@pytest.mark.parametrize(
    "make, msg",
    [
        (lambda: [torch.zeros(1, 4, 8, 64, dtype=torch.float16)] * 3, "inputs must be CUDA tensors"),
    ],
)
def test_op_rejects_cpu_tensors(make, msg):
    fa = _ops()
    q, k, v = make()
    with pytest.raises(RuntimeError, match=msg):
        fa.flash_attn(q, k, v)


def test_product_never_imports_the_oracle():
    pkg = ROOT / "nanonemo_amd"
    for path in pkg.rglob("*"):
        if path.suffix in {".py", ".hip", ".h", ".cpp"}:
            text = path.read_text()
            assert not re.search(r"^\s*(from|import)\s+oracle\b", text, re.M), path
            assert "oracle/" not in text, path


def test_noalloc_backward_checks_shape_before_touching_the_device():
    # The argument checks of nn_fa_bwd_noalloc run before any HIP call: an empty problem is a no-op and a shape
    # whose workspace exceeds the library's 32 MiB array is rejected with a message, here without a GPU.
    L = lib()
    assert L.nn_fa_bwd_noalloc(*([None] * 9), 0, 12, 4, 1024, 64, 1, 0.125, None) == 0
    B, H, KVH, T, D = 64, 16, 4, 8192, 64
    assert L.nn_fa_bwd_workspace_size(B, H, KVH, T, D) > 32 << 20
    assert L.nn_fa_bwd_noalloc(*([None] * 9), B, H, KVH, T, D, 1, 0.125, None) == -1
    assert b"32 MiB" in L.nn_fa_last_error() or b"scratch" in L.nn_fa_last_error()
    assert L.nn_fa_bwd_noalloc(*([None] * 9), 1, 12, 5, 64, 64, 1, 0.125, None) == -1  # 12 % 5 != 0


# ---- HIP-graph capture through autograd is refused before any launch ---------------------------


class _Ctx:
    """Stands in for an autograd context: the guard must raise before touching it."""

    @property
    def saved_tensors(self):
        raise AssertionError("the guard must raise before the saved tensors are read")

    def save_for_backward(self, *a):
        raise AssertionError("the guard must raise before anything is saved")


def test_capture_through_autograd_is_refused(monkeypatch):
    from nanonemo_amd.kernels.hip import flash_attn as fa

    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    monkeypatch.setattr(torch.cuda, "is_initialized", lambda: True)
    q = torch.zeros(1, 2, 4, 64, requires_grad=True)  # CPU tensors: the guard comes before the device check
    k = torch.zeros(1, 1, 4, 64, requires_grad=True)
    cos = torch.zeros(4, 32)
    for call in (lambda: fa.flash_attn(q, k, k), lambda: fa.flash_attn_bthd(q, k, k),
                 lambda: fa.flash_attn_bthd_rope(q, k, k, cos, cos)):
        with pytest.raises(RuntimeError, match="not supported"):
            call()
    for f in (fa._setup_context, fa._setup_context_rope):
        with pytest.raises(RuntimeError, match="capture_end"):
            f(_Ctx(), (q, k, k, cos, cos)[: 5 if f is fa._setup_context_rope else 3], (q, q, q))
    for f, grads in ((fa._backward, (q, None)), (fa._backward_bthd, (q, None)), (fa._backward_rope, (q, None, None))):
        with pytest.raises(RuntimeError, match="HIP graph"):
            f(_Ctx(), *grads)


def test_capture_without_autograd_is_not_refused(monkeypatch):
    # No input requires grad (or grad mode is off): nothing is recorded, so the guard lets the call through to the
    # op's own checks (here the CPU-tensor check, since no GPU is needed to show the guard passed).
    from nanonemo_amd.kernels.hip import flash_attn as fa

    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    monkeypatch.setattr(torch.cuda, "is_initialized", lambda: True)
    q, k = torch.zeros(1, 2, 4, 64), torch.zeros(1, 1, 4, 64)
    with pytest.raises(RuntimeError, match="CUDA tensors"):
        fa.flash_attn(q, k, k)
    qg = q.clone().requires_grad_()
    with torch.no_grad(), pytest.raises(RuntimeError, match="CUDA tensors"):
        fa.flash_attn(qg, k, k)


def test_capture_guard_is_off_when_not_capturing():
    from nanonemo_amd.kernels.hip import flash_attn as fa

    q = torch.zeros(1, 2, 4, 64, requires_grad=True)
    fa._refuse_capture_with_autograd("x", q)  # not capturing: returns


def test_rope_fused_ops_reject_host_tables():
    # cos / sin must be GPU tensors on q's device; a host table would reach the library as a host address.
    from nanonemo_amd.kernels.hip import flash_attn as fa

    cos = torch.zeros(8, 32)
    with pytest.raises(RuntimeError, match="inputs' device"):
        fa._check_tables(cos, cos, 8, 64, torch.device("cuda", 0))
    with pytest.raises(RuntimeError, match="inputs' device"):
        fa._check_tables(cos, cos.clone(), 8, 64, torch.device("cpu"))  # CPU "inputs" still need CUDA tables


def test_backward_ops_refuse_capture_only_inside_the_autograd_engine(monkeypatch):
    # The backward ops' own guard: a capture driven by the autograd engine (eager autograd, or a compiled backward
    # as mode="reduce-overhead" records) is refused; the same call outside the engine is not (a manual op pair).
    from nanonemo_amd.kernels.hip import flash_attn as fa

    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    monkeypatch.setattr(torch.cuda, "is_initialized", lambda: True)
    fa._refuse_capture_from_autograd_engine("outside the engine")  # returns

    class F(torch.autograd.Function):
        @staticmethod
        def forward(ctx, a):
            return a * 2

        @staticmethod
        def backward(ctx, g):
            fa._refuse_capture_from_autograd_engine("inside the engine")
            return g

    x = torch.ones(3, requires_grad=True)
    with pytest.raises(RuntimeError, match="inside the engine: capturing"):
        F.apply(x).sum().backward()


def test_eager_path_routing_without_a_gpu():
    # The public functions' eager autograd.Functions are for plain CUDA tensors only: meta and CPU tensors (and,
    # on a GPU, transforms, dispatch modes and tracing) take the custom ops, whose fake impls and checks serve them.
    from nanonemo_amd.kernels.hip import eager, records

    meta, cpu = torch.empty(2, device="meta"), torch.zeros(2)
    assert not eager(meta) and not eager(cpu)
    g = torch.zeros(2, requires_grad=True)
    assert records(cpu, g) and not records(cpu)
    with torch.no_grad():
        assert not records(g)
