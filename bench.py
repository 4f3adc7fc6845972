"""Benchmark of the causal GQA FlashAttention-2 forward + backward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--dtype bf16|fp16] [--batch 8] [--seq 1024]
    python bench.py --sweep        # step and per-kernel times over the SWEEP shapes, one JSON line each
    python bench.py --timeline     # per-block timelines of the three attention kernels (timeline build)

A step is one forward + backward of the hot path through the drop-in torch.library ops (nanonemo::flash_attn
then nanonemo::flash_attn_bwd, which call the C ABI of include/nanonemo_fa.h) on synthetic N(0,1) inputs
resident in HBM. Default workload: B=8, T=1024, 12 query / 4 KV heads, head_dim 64, bf16 (the north-star shape
of BASELINE.json). W untimed warmup steps, about 1 s of settling steps, then K timed steps between device
synchronisations. Each timed step follows a 512 MiB cache-flush write (twice the Infinity Cache, the reference
benchmark's method, benchmarks/kernels/common.py:30-54) and is timed alone with HIP events on the launch
stream; value and ms_per_step come from the median step. The flush keeps the device busy while the host
enqueues the op pair, so the pair runs back to back as from a graph replay.

value = algorithmic FLOPs per step / time per step, with F_alg = 6*B*H*D*T*(T+1) (12*D flop per causal
(query, key) pair: 2 forward and 4 backward products; the backward's recompute of S is not counted).

The JSON line also carries:
  c_abi_warm_*  the same pair through the C ABI on preallocated outputs, back to back with warm caches
                (op_warm_ms_per_step: through the ops, back to back; graph_ms_per_step: the C-ABI pair
                replayed from a HIP graph; ref_method: graph replays after a flush, median / p20 / p80);
  roofline      the dominant kernel (the longest of the forward, dK/dV and dQ kernels), timed alone
                with HIP events on the stream it is launched on: achieved = its algorithmic FLOPs per
                launch (forward 4*D, dK/dV 6*D, dQ 2*D per causal pair) / its mean launch time, against
                the dense BF16/FP16 MFMA peak of 2.5 PFLOP/s; traffic is null (HBM bytes need rocprofv3
                counters, which this run does not collect);
  traffic_committed  the dominant kernel's HBM bytes per launch from the committed rocprofv3 FETCH_SIZE /
                WRITE_SIZE summary of this workload (profiles/), labelled as such;
  clock         the GFX clock (median of the SMU's per-XCD readings through amdsmi) and socket power while
                the dK/dV kernel alone, then the whole step, run back to back; roofline.frac_at_sclk is the
                dominant kernel's fraction of the peak scaled to that clock (the published peak assumes 2.4 GHz);
  same_node     PyTorch's own attention on the same GPU (SDPA flash with native GQA, and the reference
                benchmark's providers: SDPA mem-efficient and math on repeat_interleave'd K/V) beside this
                build's op, each as fwd + autograd.grad back to back;
  cpu_baseline  the reference's plain-PyTorch attention on BASELINE config 1 (fp32, B=1, T=256), forward +
                autograd backward, both of its forms (SDPA math and explicit matmuls), on the host CPUs;
  kernels       per-kernel mean times (nn_fa_bwd = the dQ kernel, which also runs the preprocessing pass,
                then the dK/dV kernel) and the HBM rate of the standalone preprocessing entry point;
  layout_fusion the same fwd+bwd from (B, T, heads, hd) projections: through transposed views and the
                dense ops (the reference model's flow, with its copies) vs the layout-fused
                nanonemo::flash_attn_bthd ops, with the host's time per step beside each;
  rope_qk       the HIP RoPE kernel on the workload's q and k (projection layout, one launch) and its
                HBM rate, beside the plain-PyTorch formula;
  other_dtype   the headline's measurement in the other 16-bit type (fp16 for the default bf16 run: BASELINE
                config 2's own dtype);
  config5       BASELINE config 5 in brief (default workload only): a few 114 M-model bf16 train steps per
                attention path (plain PyTorch, and every HIP kernel with q's RoPE separate or folded in):
                tokens/s and the loss differences against the plain-PyTorch path (step 0 and largest);
  add_rmsnorm   the HIP fused residual add + RMSNorm forward and backward (dx, ddelta and dw) on the
                114 M model's stream at this workload's tokens (B*T rows of 768, fp32 residual, bf16
                sublayer output and normalised output) and their HBM rates.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "causal GQA attn fwd+bwd TFLOP/s at T=1024; % of BF16 MFMA peak"
PEAK_TFLOPS = 2500.0  # MI355X dense BF16/FP16 MFMA, published
PEAK_HBM_GBPS = 8000.0
COPY_CALIB_BYTES = 256 << 20  # size of the calibration copy run by --profile-only


NORM_D = 768  # d_model of the 114 M model


def _norm_launches(L, M, dev, sp):
    """C-ABI launches of the fused add + RMSNorm on M rows of the model's residual stream (fp32 x, bf16
    delta and output, fp32 weight), with their algorithmic HBM bytes."""
    import torch

    from nanonemo_amd.kernels.hip import check_rmsnorm

    N = NORM_D
    g = torch.Generator(device=dev).manual_seed(1)
    x = torch.randn(M, N, device=dev, generator=g)
    d = torch.randn(M, N, device=dev, generator=g).bfloat16()
    w = torch.ones(N, device=dev)
    y = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    h = torch.empty(M, N, device=dev)
    rstd = torch.empty(M, device=dev)
    dy = torch.randn(M, N, device=dev, generator=g).bfloat16()
    dh = torch.randn(M, N, device=dev, generator=g)
    dx = torch.empty(M, N, device=dev)
    dd = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    dw = torch.empty(N, device=dev)
    wsb = L.nn_add_rmsnorm_bwd_workspace_size(M, N)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    keep = (x, d, w, y, h, rstd, dy, dh, dx, dd, dw, ws)
    return {
        "fwd": lambda: check_rmsnorm(L.nn_add_rmsnorm_fwd(x.data_ptr(), d.data_ptr(), w.data_ptr(), y.data_ptr(),
                                                          h.data_ptr(), rstd.data_ptr(), M, N, 1e-5, 2, 1, 1, sp)),
        "bwd": lambda: check_rmsnorm(L.nn_add_rmsnorm_bwd(dy.data_ptr(), dh.data_ptr(), h.data_ptr(), w.data_ptr(),
                                                          rstd.data_ptr(), dx.data_ptr(), dd.data_ptr(), dw.data_ptr(),
                                                          ws.data_ptr(), wsb, M, N, 1, 2, 2, 1, sp)),
        # read x, delta; write h, y, rstd  |  read dy, dh, h, rstd; write dx, ddelta (dw and its partials aside)
        "fwd_bytes": M * N * (4 + 2 + 4 + 2) + 4 * M,
        "bwd_bytes": M * N * (2 + 4 + 4 + 4 + 2) + 4 * M,
        "keep": keep,
    }


def gfx_clock(dev, enqueue, seconds=2.5):
    """The GFX (shader) clock the device runs at under a given load: enqueue() (device work, issued back to back
    in batches) repeats for about `seconds` while a thread samples the SMU's per-XCD current GFX clock and the
    socket power through amdsmi every few ms. The SMU refreshes those readings about once a second, so only the
    tables published after the load started count. Returns the median (and p10 / p90) over the samples of the
    mean over the XCDs, the median power, the number of distinct tables and the clock ceiling; {"error": ...}
    where amdsmi is unavailable or no table was published in the window."""
    import threading

    import torch

    try:
        import amdsmi

        amdsmi.amdsmi_init()
    except Exception as exc:  # noqa: BLE001 -- the measurement is optional
        return {"error": f"amdsmi unavailable: {exc}"}
    try:
        handles = amdsmi.amdsmi_get_processor_handles()
        handle = handles[0] if len(handles) == 1 else None
        if handle is None:  # several GPUs visible: the one whose PCI address is cuda's device
            props = torch.cuda.get_device_properties(dev)
            want = f"{getattr(props, 'pci_domain_id', 0):04x}:{getattr(props, 'pci_bus_id', -1):02x}:"
            handle = next((h for h in handles if amdsmi.amdsmi_get_gpu_device_bdf(h).lower().startswith(want)), None)
        if handle is None:
            return {"error": "no amdsmi handle matches the device"}
        ceiling = amdsmi.amdsmi_get_clock_info(handle, amdsmi.AmdSmiClkType.GFX).get("max_clk")
        samples, stop = [], threading.Event()

        def sampler():
            while not stop.is_set():
                m = amdsmi.amdsmi_get_gpu_metrics_info(handle)
                clks = [c for c in (m.get("current_gfxclks") or []) if isinstance(c, int)]
                pw = m.get("current_socket_power")
                if clks:
                    samples.append((time.perf_counter(), sum(clks) / len(clks), pw if isinstance(pw, int) else None,
                                    m.get("system_clock_counter")))
                time.sleep(0.003)

        th = threading.Thread(target=sampler, daemon=True)
        torch.cuda.synchronize()
        # The SMU refreshes its table about once a second: the table current now describes the time before the
        # load, so its samples are dropped.
        before = amdsmi.amdsmi_get_gpu_metrics_info(handle).get("system_clock_counter")
        th.start()
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            enqueue()
            torch.cuda.synchronize()
        t1 = time.perf_counter()
        stop.set()
        th.join()
        window = [x for x in samples if t0 < x[0] < t1 and x[3] != before]
        inside = sorted(x[1] for x in window)
        power = [x[2] for x in window if x[2] is not None]
        if not inside:
            return {"error": f"the SMU metrics table did not refresh during the {seconds} s window"}
        updates = len({x[3] for x in window})
        return {
            "gfx_mhz_median": round(statistics.median(inside)),
            "gfx_mhz_p10": round(inside[len(inside) // 10]),
            "gfx_mhz_p90": round(inside[(9 * len(inside)) // 10]),
            "samples": len(inside),
            # distinct SMU metric tables among the samples (its timestamp), i.e. how many readings are independent
            "smu_updates": updates,
            "socket_power_w_median": statistics.median(power) if power else None,
            "gfx_mhz_max": ceiling,
        }
    except Exception as exc:  # noqa: BLE001
        return {"error": f"amdsmi query failed: {exc}"}
    finally:
        try:
            amdsmi.amdsmi_shut_down()
        except Exception:  # noqa: BLE001
            pass


def same_node(q, k, v, do, fa, reps):
    """PyTorch's own attention on the same GPU, as the reference benchmark's providers run it
    (/root/reference/benchmarks/kernels/flash_attn.py:27-49: SDPA mem-efficient and SDPA math on
    repeat_interleave'd K/V), plus SDPA's flash backend with native GQA (enable_gqa) where this PyTorch has one,
    and this build's attention through autograd the same way (this_build_autograd: the public flash_attn, whose
    eager path is a plain autograd.Function; this_build_autograd_ops: the custom op torch.ops.nanonemo.flash_attn
    with its registered autograd, as torch.compile and op-level callers reach it), each as fwd + autograd.grad
    w.r.t. q, k, v, back to back on warm
    caches; ms: time per call from HIP events, host_ms: the host's time per call in the same loop (where host_ms
    reaches ms, the host, not the GPU, sets the pace). Neither a spin kernel that holds the device while the host
    enqueues nor the profiler's kernel records give the device time of a host-paced loop faithfully here: the
    nearly idle device lowers its clock during a spin (the next milliseconds run up to about 15 % slower), and
    per-kernel tracing lengthens the kernels."""
    import warnings

    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    B, H, T = q.shape[0], q.shape[1], q.shape[2]
    group = H // k.shape[1]
    qs, ks, vs = (t.detach().clone().requires_grad_() for t in (q, k, v))

    def sdpa(backend, gqa):
        def step():
            with sdpa_kernel([backend]):
                if gqa:
                    o = F.scaled_dot_product_attention(qs, ks, vs, is_causal=True, enable_gqa=True)
                else:
                    kk, vv = ks.repeat_interleave(group, dim=1), vs.repeat_interleave(group, dim=1)
                    o = F.scaled_dot_product_attention(qs, kk, vv, is_causal=True)
            return torch.autograd.grad(o, (qs, ks, vs), do)

        return step

    def ours():
        return torch.autograd.grad(fa.flash_attn(qs, ks, vs), (qs, ks, vs), do)

    def ours_ops():
        return torch.autograd.grad(torch.ops.nanonemo.flash_attn(qs, ks, vs)[0], (qs, ks, vs), do)

    providers = {"this_build_autograd": ours, "this_build_autograd_ops": ours_ops,
                 "sdpa_flash_gqa": sdpa(SDPBackend.FLASH_ATTENTION, True),
                 "sdpa_mem_efficient": sdpa(SDPBackend.EFFICIENT_ATTENTION, False)}
    if B * H * T * T <= 1 << 27:  # math materialises the B*H*T*T scores
        providers["sdpa_math"] = sdpa(SDPBackend.MATH, False)
    out = {}
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        for name, fn in providers.items():
            try:
                for _ in range(3):
                    fn()
                torch.cuda.synchronize()
                n = reps if name != "sdpa_math" else max(3, reps // 10)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                t0 = time.perf_counter()
                e0.record()
                for _ in range(n):
                    fn()
                t1 = time.perf_counter()
                e1.record()
                e1.synchronize()
                out[name] = {"ms": round(e0.elapsed_time(e1) / n, 5), "host_ms": round((t1 - t0) * 1e3 / n, 5)}
            except Exception as exc:  # noqa: BLE001 -- a backend this PyTorch lacks
                out[name] = {"error": str(exc).splitlines()[0][:200]}
    return out


def parse():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--dtype", choices=["bf16", "fp16"], default="bf16")
    p.add_argument("--batch", type=int, default=8)
    p.add_argument("--seq", type=int, default=1024)
    p.add_argument("--heads", type=int, default=12)
    p.add_argument("--kv-heads", type=int, default=4)
    p.add_argument("--head-dim", type=int, default=64)
    p.add_argument("--input-scale", type=float, default=1.0, help="q, k, v ~ N(0,1) times this (BASELINE config 3: 3.0)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=16.0, help="budget of the CPU baseline sample (both forms)")
    p.add_argument("--no-config5", action="store_true", help="skip the config5 block (114 M model train steps)")
    p.add_argument("--config5-steps", type=int, default=10, help="train steps per attention path in the config5 block")
    p.add_argument("--profile-only", action="store_true", help="only the timed steps (for rocprofv3)")
    p.add_argument("--prewarm", type=float, default=1.0, help="seconds of untimed steps after the warmup")
    p.add_argument("--sweep", action="store_true",
                   help="instead of the headline line: one JSON line per shape of SWEEP (step and per-kernel times)")
    p.add_argument("--timeline", action="store_true",
                   help="instead of the headline line: per-block timelines of the forward, dQ and dK/dV kernels at "
                   "the workload's shape, from libnanonemo_fa_timeline.so, one JSON line")
    p.add_argument("--timeline-out", default=None, help="with --timeline: also save the raw records (.npz)")
    return p.parse_args()


# --sweep shapes: (label, B, T, H, KVH, D, dtype, input scale). The BASELINE.json configurations 2-4 first
# (config 2 in its fp16 and the headline's bf16), then other head dims, GQA ratios and lengths.
SWEEP = [
    ("config 2 (fp16)", 8, 1024, 12, 4, 64, "fp16", 1.0),
    ("config 2 (bf16, the headline)", 8, 1024, 12, 4, 64, "bf16", 1.0),
    ("config 3", 32, 1024, 12, 4, 64, "bf16", 3.0),
    ("config 4", 2, 8192, 12, 4, 64, "bf16", 1.0),
    ("config 1 shape", 1, 256, 12, 4, 64, "bf16", 1.0),
    ("head_dim 32", 8, 1024, 12, 4, 32, "bf16", 1.0),
    ("MHA (12 KV heads)", 8, 1024, 12, 12, 64, "bf16", 1.0),
    ("MQA (1 KV head)", 8, 1024, 12, 1, 64, "bf16", 1.0),
    # the reference benchmark's (B, T) ladder at fixed tokens (benchmarks/kernels/flash_attn.py:54); (8, 1024) is config 2
    ("T=256 (ladder)", 32, 256, 12, 4, 64, "bf16", 1.0),
    ("T=512 (ladder)", 16, 512, 12, 4, 64, "bf16", 1.0),
    ("T=2048", 4, 2048, 12, 4, 64, "bf16", 1.0),
    ("T=4096", 2, 4096, 12, 4, 64, "bf16", 1.0),
    ("T=16384", 1, 16384, 12, 4, 64, "bf16", 1.0),
]


def sweep(args):
    """Per shape: the fwd+bwd step through the C ABI and each kernel alone, HIP events on the launch
    stream, after warm-up and about 0.3 s of settling steps. One JSON line per shape."""
    import torch

    from nanonemo_amd.kernels.hip import DTYPE_BF16, DTYPE_F16, check, lib

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    L = lib()
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    for label, B, T, H, KVH, D, dts, mult in SWEEP:
        dtype = torch.bfloat16 if dts == "bf16" else torch.float16
        code = DTYPE_BF16 if dts == "bf16" else DTYPE_F16
        scale = 1.0 / math.sqrt(D)
        torch.manual_seed(0)
        q, do = ((torch.randn(B, H, T, D, device=dev) * mult).to(dtype) for _ in range(2))
        k, v = ((torch.randn(B, KVH, T, D, device=dev) * mult).to(dtype) for _ in range(2))
        o, dq = torch.empty_like(q), torch.empty_like(q)
        dk, dv = torch.empty_like(k), torch.empty_like(v)
        lse = torch.empty(B, H, T, dtype=torch.float32, device=dev)
        wsb = L.nn_fa_bwd_workspace_size(B, H, KVH, T, D)
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        a = (B, H, KVH, T, D, code, scale, sp)
        fwd = lambda: L.nn_fa_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), *a)  # noqa: E731
        bwd = lambda: L.nn_fa_bwd(do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),  # noqa: E731
                                  lse.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), wsb, *a)
        dqk = lambda: L.nn_fa_bwd_dq(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(),  # noqa: E731
                                     lse.data_ptr(), ws.data_ptr(), wsb, dq.data_ptr(), *a)
        dkdv = lambda: L.nn_fa_bwd_dkdv(q.data_ptr(), k.data_ptr(), v.data_ptr(), do.data_ptr(), ws.data_ptr(),  # noqa: E731
                                        wsb, dk.data_ptr(), dv.data_ptr(), *a)

        def step():
            check(fwd())
            check(bwd())

        for _ in range(max(args.warmup, 3)):
            step()
        t_end = time.perf_counter() + 0.3
        while time.perf_counter() < t_end:
            for _ in range(20):
                step()
            torch.cuda.synchronize()

        def events(fn, reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(reps):
                fn()
            e1.record(stream)
            e1.synchronize()
            return e0.elapsed_time(e1) * 1e3 / reps

        pairs = B * H * T * (T + 1) / 2
        reps = max(5, min(args.steps, int(30000 / events(step, 3))))  # about 30 ms of each measurement
        step_us = events(step, reps)
        # the reference benchmark's method: each step after a 512 MiB cache flush, timed alone (median)
        flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(30)]
        for i, (e0, e1) in enumerate(ev):
            flush.fill_(i & 0xFF)
            e0.record(stream)
            step()
            e1.record(stream)
        torch.cuda.synchronize()
        flushed_us = statistics.median(e0.elapsed_time(e1) for e0, e1 in ev) * 1e3
        del flush
        us = {n: events(lambda fn=fn: check(fn()), reps) for n, fn in (("fwd", fwd), ("dq", dqk), ("dkdv", dkdv))}
        tf = lambda flop, t: round(flop / t / 1e6, 1)  # noqa: E731
        print(json.dumps({
            "shape": label, "B": B, "T": T, "H": H, "KVH": KVH, "D": D, "dtype": dts, "input_scale": mult,
            "step_us": round(step_us, 2), "tflops": tf(12 * D * pairs, step_us),
            "flushed_step_us": round(flushed_us, 2), "flushed_tflops": tf(12 * D * pairs, flushed_us),
            "pct_of_peak": round(100 * 12 * D * pairs / step_us / 1e6 / PEAK_TFLOPS, 2),
            "fwd_us": round(us["fwd"], 2), "fwd_tflops": tf(4 * D * pairs, us["fwd"]),
            "dq_us": round(us["dq"], 2), "dq_tflops": tf(2 * D * pairs, us["dq"]),
            "dkdv_us": round(us["dkdv"], 2), "dkdv_tflops": tf(6 * D * pairs, us["dkdv"]),
        }), flush=True)
        del q, k, v, do, o, dq, dk, dv, lse, ws
        torch.cuda.empty_cache()


def config5(steps: int, warmup: int = 4):
    """BASELINE config 5 in brief: the 114 M model (12 layers, d_model 768, 12 Q / 4 KV heads, vocab 50,304, tied
    embeddings) trained from the seed-0 init on the seed-0 uniform token stream at B=8, T=1024 under bf16 autocast,
    ``steps`` AdamW steps per attention path (nanonemo_amd.train.run, the same weights and batches for every path).
    tokens/s over the steps after ``warmup``; loss differences against the plain-PyTorch attention (SDPA math on fp32
    q, k, v), at step 0 (identical weights and batch) and the largest over the steps. The 50-step curves come from
    ``python -m nanonemo_amd.train``."""
    import torch

    from nanonemo_amd.train import run

    paths = ("torch", "hip_bthd+rope+norm", "hip_bthd+qrope+norm")
    res = {}
    for attn in paths:
        losses, tps, fpt = run(attn, steps, 8, 1024, dict(max_seq_len=1024, attn_backend="math_fp32"), warmup=warmup)
        res[attn] = {"tokens_per_s": round(tps, 1), "model_tflops": round(tps * fpt / 1e12, 2),
                     "losses": [round(v, 5) for v in losses]}
        torch.cuda.empty_cache()
    for attn in paths[1:]:
        d = [abs(a - b) for a, b in zip(res[attn]["losses"], res["torch"]["losses"])]
        res[attn]["step0_abs_loss_diff_vs_torch"] = round(d[0], 6)
        res[attn]["max_abs_loss_diff_vs_torch"] = round(max(d), 5)
        res[attn]["speedup_vs_torch"] = round(res[attn]["tokens_per_s"] / res["torch"]["tokens_per_s"], 3)
    return {"workload": f"114M NanoNemo, bf16 autocast, B=8 T=1024, {steps} AdamW steps per path (tokens/s over the "
                        f"last {steps - warmup}), seed-0 init, uniform synthetic tokens; torch = SDPA math on fp32 q, k, v",
            "results": res}


def _cpu_topology():
    """(usable logical CPUs, physical cores among them, CPU model) of this host, from the process's CPU
    affinity and /proc/cpuinfo (a core is a distinct (physical id, core id) pair)."""
    usable = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else list(range(os.cpu_count() or 1))
    model, cores, cur = platform.processor() or platform.machine(), set(), {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" not in line:
                if cur.get("processor") in usable:
                    cores.add((cur.get("physical id", "0"), cur.get("core id", cur.get("processor"))))
                cur = {}
                continue
            key, val = (x.strip() for x in line.split(":", 1))
            if key == "processor":
                cur["processor"] = int(val)
            elif key in ("physical id", "core id"):
                cur[key] = val
            elif key == "model name":
                model = val
        if cur.get("processor") in usable:
            cores.add((cur.get("physical id", "0"), cur.get("core id", cur.get("processor"))))
    except OSError:
        pass
    return len(usable), len(cores) or len(usable), model


def cpu_baseline(budget_s):
    """Times the reference's plain-PyTorch CPU path on BASELINE config 1, in the same process.

    Config 1: fp32, B=1, T=256, 12 query / 4 KV heads, head_dim 64, torch.manual_seed(0) then randn q, k, v,
    dO in that order, scale 1/sqrt(64). Both of the reference's forms (oracle.attention.torch_reference_fwd_bwd):
    repeat_interleave + SDPA math (nanonemo/model/layers.py:109-115) and the explicit matmul / triu mask /
    softmax form (tests/model/test_layers.py:107-123), each forward + autograd backward, timed for about
    budget_s / 2 seconds after 3 warm-ups on every usable host CPU. The median of each is scaled to TFLOP/s
    with the GPU figure's algorithmic FLOP count; ``value`` is the faster form.
    """
    import torch

    from oracle.attention import flops, torch_reference_fwd_bwd

    B, H, KVH, T, D = 1, 12, 4, 256, 64
    usable, phys, model = _cpu_topology()
    torch.set_num_threads(usable)
    torch.manual_seed(0)
    q = torch.randn(B, H, T, D)
    k = torch.randn(B, KVH, T, D)
    v = torch.randn(B, KVH, T, D)
    do = torch.randn(B, H, T, D)
    forms = {}
    for name, explicit in (("sdpa_math", False), ("explicit", True)):
        for _ in range(3):
            torch_reference_fwd_bwd(q, k, v, do, explicit=explicit)
        times = []
        t_end = time.perf_counter() + budget_s / 2
        while time.perf_counter() < t_end or len(times) < 5:
            t0 = time.perf_counter()
            torch_reference_fwd_bwd(q, k, v, do, explicit=explicit)
            times.append(time.perf_counter() - t0)
            if len(times) >= 20000:
                break
        t = statistics.median(times)
        forms[name] = {"median_ms": round(t * 1e3, 4), "reps": len(times), "tflops": flops(B, H, T, D) / t / 1e12}
    best = max(forms, key=lambda n: forms[n]["tflops"])
    return {
        "value": round(forms[best]["tflops"], 5),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"BASELINE config 1: plain-PyTorch causal GQA fwd + autograd bwd, fp32, B={B} T={T} {H}Q/{KVH}KV "
        f"d={D}, seed 0; value = the faster of the reference's two forms ({best}); medians over about "
        f"{budget_s / 2:.0f} s each",
        "forms": {n: {"median_ms": f["median_ms"], "reps": f["reps"], "tflops": round(f["tflops"], 5)} for n, f in forms.items()},
        "threads": torch.get_num_threads(),
        "physical_cores": phys,
        "cpu_model": model,
    }


def timeline(args):
    """Per-block timelines of the forward, dQ and dK/dV kernels at the workload's shape, from the timeline build
    (libnanonemo_fa_timeline.so: the same kernels, each block stamping the 100 MHz constant clock at its start and
    end and the shader clock at its phase boundaries). The records come from the last of 20 back-to-back
    fwd + nn_fa_bwd steps after about 1 s of steps. Per kernel: when it ran (µs from the forward's first block),
    how many blocks ran at once and what fraction of that slot-time held a block, when its first block ended and
    its last block started, the shader clock over a block, its blocks' phase lengths in shader cycles (forward and
    dQ: start to first tile ready, dQ's row-load and preprocessing prologue within it; dK/dV: prologue, the
    spread of the 4 waves' loop ends in a unit, which the slowest sets, and the first unit's reduction), and, for
    the forward and dQ, per tile count when those blocks started and ended. One JSON line."""
    import numpy as np
    import torch

    from nanonemo_amd.build import TIMELINE_LIB
    from nanonemo_amd.kernels.hip import DTYPE_BF16, DTYPE_F16, SIGNATURES

    if not TIMELINE_LIB.exists():
        raise RuntimeError(f"{TIMELINE_LIB} is not built; run `python -m nanonemo_amd.build`")
    TL = ctypes.CDLL(str(TIMELINE_LIB))
    for name in ("nn_fa_fwd", "nn_fa_bwd", "nn_fa_bwd_workspace_size", "nn_fa_last_error"):
        fn = getattr(TL, name)
        fn.restype, fn.argtypes = SIGNATURES[name]
    TL.nn_fa_timeline_dims.argtypes = [ctypes.POINTER(ctypes.c_int)] * 3
    TL.nn_fa_timeline_read.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int]

    def ok(rc):
        if rc != 0:
            raise RuntimeError(TL.nn_fa_last_error().decode(errors="replace"))

    nk, nb, nw = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    ok(TL.nn_fa_timeline_dims(ctypes.byref(nk), ctypes.byref(nb), ctypes.byref(nw)))
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    sp = torch.cuda.current_stream().cuda_stream
    B, T, H, KVH, D = args.batch, args.seq, args.heads, args.kv_heads, args.head_dim
    dtype = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    a = (B, H, KVH, T, D, DTYPE_BF16 if args.dtype == "bf16" else DTYPE_F16, 1.0 / math.sqrt(D), sp)
    torch.manual_seed(0)
    q, do = ((torch.randn(B, H, T, D, device=dev) * args.input_scale).to(dtype) for _ in range(2))
    k, v = ((torch.randn(B, KVH, T, D, device=dev) * args.input_scale).to(dtype) for _ in range(2))
    o, dq, dk, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    lse = torch.empty(B, H, T, dtype=torch.float32, device=dev)
    wsb = TL.nn_fa_bwd_workspace_size(B, H, KVH, T, D)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)

    def step():
        ok(TL.nn_fa_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), *a))
        ok(TL.nn_fa_bwd(do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                        dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), wsb, *a))

    for _ in range(max(args.warmup, 3)):
        step()
    t_end = time.perf_counter() + args.prewarm
    while time.perf_counter() < t_end:
        for _ in range(50):
            step()
        torch.cuda.synchronize()
    ok(TL.nn_fa_timeline_clear())
    for _ in range(20):
        step()
    torch.cuda.synchronize()
    rec = {}
    for kern, name in enumerate(("fwd", "dq", "dkdv")):
        r = np.zeros((nb.value, nw.value), dtype=np.uint64)
        ok(TL.nn_fa_timeline_read(kern, r.ctypes.data, nb.value))
        rec[name] = r[r[:, 0] != 0].astype(np.int64)  # blocks of the last launch (a cleared record reads 0)
    if args.timeline_out:
        np.savez(args.timeline_out, **rec)
    t0 = rec["fwd"][:, 0].min()
    us = lambda ticks: ticks / 100.0  # noqa: E731  (s_memrealtime runs at 100 MHz)
    rnd = lambda x: round(float(x), 2)  # noqa: E731

    def summary(r, name):
        start, end = us(r[:, 0] - t0), us(r[:, 1] - t0)
        ev = sorted([(s_, 1) for s_ in start] + [(e_, -1) for e_ in end], key=lambda x: (x[0], x[1]))
        live = peak = 0
        for _, d in ev:
            live += d
            peak = max(peak, live)
        k0, k1 = start.min(), end.max()
        out = {
            "blocks": int(len(r)), "start_us": rnd(k0), "end_us": rnd(k1), "span_us": rnd(k1 - k0),
            "blocks_at_once_max": peak,
            "slot_time_used": rnd((end - start).sum() / (peak * (k1 - k0))),
            "first_block_end_us": rnd(end.min() - k0), "last_block_start_us": rnd(start.max() - k0),
            "shader_mhz_median": round(float(np.median((r[:, 4] - r[:, 2]) / us(r[:, 1] - r[:, 0])))),
            "blocks_per_xcd": np.bincount((r[:, 5] >> 32) & 0xF, minlength=8).tolist(),
        }
        first = start < k0 + 1.0  # the first wave of blocks (started within 1 us of the kernel's start)
        pro = r[:, 3] - r[:, 2]
        out["prologue_cycles_median"] = {"first_wave": int(np.median(pro[first])),
                                         "later": int(np.median(pro[~first])) if (~first).any() else None}
        if name == "dq":
            rows = r[:, 6] - r[:, 2]
            out["row_prologue_cycles_median"] = {"first_wave": int(np.median(rows[first])),
                                                 "later": int(np.median(rows[~first])) if (~first).any() else None}
        if name in ("fwd", "dq"):
            by = {}
            for nt in sorted(set(r[:, 7].tolist())):
                m = r[:, 7] == nt
                by[f"{int(nt)} tiles"] = {
                    "blocks": int(m.sum()),
                    "start_us_min_med_max": [rnd(start[m].min() - k0), rnd(np.median(start[m]) - k0),
                                             rnd(start[m].max() - k0)],
                    "end_us_min_med_max": [rnd(end[m].min() - k0), rnd(np.median(end[m]) - k0), rnd(end[m].max() - k0)],
                    "duration_us_median": rnd(np.median(end[m] - start[m])),
                }
            out["by_128_key_tiles"] = by
        if name == "dkdv":
            loop0, loop1 = r[:, 6:10], r[:, 10:14]
            out["unit0_loop_end_spread_cycles_median"] = int(np.median(loop0.max(1) - loop0.min(1)))
            two = (loop1 > 0).all(1)
            if two.any():
                out["unit1_loop_end_spread_cycles_median"] = int(np.median(loop1[two].max(1) - loop1[two].min(1)))
            out["unit0_reduction_cycles_median"] = int(np.median(r[:, 14] - loop0.max(1)))
            out["block_cycles_median"] = int(np.median(r[:, 4] - r[:, 2]))
        return out

    print(json.dumps({"timeline": {
        "workload": {"batch": B, "seq_len": T, "heads": H, "kv_heads": KVH, "head_dim": D, "dtype": args.dtype},
        "how": "last of 20 back-to-back fwd + nn_fa_bwd steps from libnanonemo_fa_timeline.so; times in us from "
               "the forward's first block start (100 MHz clock), cycles in shader clocks",
        **{n: summary(r, n) for n, r in rec.items()},
    }}), flush=True)


def main():
    args = parse()
    if args.timeline and args.gpus == 1:
        timeline(args)
        return
    if args.sweep and args.gpus == 1:
        sweep(args)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py measures one GPU only: this build's hot path (causal GQA attention) runs per GPU on its "
            "own heads/batch shard with no exchange, and no multi-GPU figure is produced. Use --gpus 1.",
            file=sys.stderr,
        )
        sys.exit(2)

    import torch

    from nanonemo_amd.kernels.hip import DTYPE_BF16, DTYPE_F16, check, lib
    from nanonemo_amd.kernels.hip import flash_attn as fa

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    dtype = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    B, H, KVH, T, D = args.batch, args.heads, args.kv_heads, args.seq, args.head_dim
    scale = 1.0 / math.sqrt(D)
    f_fwd = 2.0 * B * H * D * T * (T + 1)
    f_bwd = 2.0 * f_fwd
    f_all = f_fwd + f_bwd

    torch.manual_seed(0)
    q = (torch.randn(B, H, T, D, device=dev) * args.input_scale).to(dtype)
    k = (torch.randn(B, KVH, T, D, device=dev) * args.input_scale).to(dtype)
    v = (torch.randn(B, KVH, T, D, device=dev) * args.input_scale).to(dtype)
    do = torch.randn(B, H, T, D, device=dev).to(dtype)

    L = lib()
    dt_code = DTYPE_BF16 if dtype == torch.bfloat16 else DTYPE_F16
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    o = torch.empty_like(q)
    lse = torch.empty(B, H, T, dtype=torch.float32, device=dev)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws_bytes = L.nn_fa_bwd_workspace_size(B, H, KVH, T, D)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    ptr = {n: t.data_ptr() for n, t in dict(q=q, k=k, v=v, do=do, o=o, lse=lse, dq=dq, dk=dk, dv=dv, ws=ws).items()}

    def step_abi_on(st):
        """One fwd+bwd through the C ABI (the drop-in boundary) on stream st, outputs already allocated."""
        check(L.nn_fa_fwd(ptr["q"], ptr["k"], ptr["v"], ptr["o"], ptr["lse"], B, H, KVH, T, D, dt_code, scale, st))
        check(L.nn_fa_bwd(ptr["do"], ptr["q"], ptr["k"], ptr["v"], ptr["o"], ptr["lse"], ptr["dq"], ptr["dk"],
                          ptr["dv"], ptr["ws"], ws_bytes, B, H, KVH, T, D, dt_code, scale, st))

    def step_abi():
        step_abi_on(sp)

    def step_op():
        """The same pair through the torch.library ops (allocates outputs with the caching allocator)."""
        o2, lse2 = fa._flash_attn(q, k, v)
        return fa._flash_attn_bwd(do, q, k, v, o2, lse2)

    def timed(fn, n):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / n

    # The last-level-cache flush of the reference benchmark's method (benchmarks/kernels/common.py:30-54): a
    # 512 MiB write, twice the 256 MB Infinity Cache, before every timed step, so each step reads its inputs
    # from HBM. Allocated before the warmup so that its allocation settles with the others.
    flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev)

    def flushed_op_steps(n):
        """n steps, each a cache flush and then the op pair timed alone with events on the launch stream.
        The flush keeps the device busy for about 0.1 ms while the host enqueues the op pair behind it, so
        the op pair runs back to back on the device as it would from a graph replay."""
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
        torch.cuda.synchronize()
        for i, (a, b_) in enumerate(ev):
            flush.fill_(i & 0xFF)
            a.record(stream)
            step_op()
            b_.record(stream)
        torch.cuda.synchronize()
        return [a.elapsed_time(b_) for a, b_ in ev]

    # Untimed: the W warmup steps of every path (which make every allocation the timed steps reuse), then
    # about 1 s of back-to-back steps. After a new device allocation the step time stays up to 15 %
    # longer for some 300 steps (~117 -> ~103 us at the default workload), so this settling run comes
    # after the last allocation and before the timed region.
    for _ in range(args.warmup):
        step_abi()
        step_op()
    if not args.profile_only:
        flushed_op_steps(max(args.warmup, 3))
    t_end = time.perf_counter() + args.prewarm
    while time.perf_counter() < t_end:
        for _ in range(200):  # the device never idles between these (the host runs ahead)
            step_abi()
        torch.cuda.synchronize()
    # The headline: K steps through the torch.library ops, each after a cache flush, bracketed by device
    # synchronisations; value from the median step.
    # (--profile-only: warm steps only, so that the per-kernel averages of a trace match the bench's own
    # per-kernel event timings, which are taken on warm caches)
    step_ms = flushed_op_steps(args.steps) if not args.profile_only else [float("nan")]
    ms = statistics.median(step_ms)
    # Beside it, warm-cache back-to-back steps: through the C ABI on resident outputs, and through the ops.
    abi_ms = timed(step_abi, args.steps)
    op_ms = timed(step_op, args.steps)
    if args.profile_only:
        # The standalone preprocessing pass (nn_fa_bwd runs it fused into the dQ kernel), so that its
        # HBM traffic and rate have rocprofv3 records of their own.
        for _ in range(args.steps):
            check(L.nn_fa_bwd_pre(ptr["o"], ptr["do"], ptr["lse"], ptr["ws"], ws_bytes, B, H, KVH, T, D, dt_code,
                                  scale, sp))
        # The RoPE kernel on the workload's q and k in the projection layout.
        from nanonemo_amd.kernels.hip import check_rope, strides3
        from nanonemo_amd.model import rope_tables

        qp, kp = q.transpose(1, 2).contiguous(), k.transpose(1, 2).contiguous()
        qr, kr = torch.empty_like(qp), torch.empty_like(kp)
        cos_t, sin_t = (t.to(dev) for t in rope_tables(D, T, 10000.0))
        for _ in range(args.steps):
            check_rope(L.nn_rope_qk(qp.data_ptr(), qr.data_ptr(), kp.data_ptr(), kr.data_ptr(), cos_t.data_ptr(),
                                    sin_t.data_ptr(), B, T, H, KVH, D, strides3(T * H * D, H * D, D),
                                    strides3(T * KVH * D, KVH * D, D), T, dt_code, sp))
        # The fused add + RMSNorm, forward and backward, on the model's residual stream at these tokens.
        norm = _norm_launches(L, B * T, dev, sp)
        for _ in range(args.steps):
            norm["fwd"]()
            norm["bwd"]()
        # A plain device copy of known size, for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings.
        src = torch.empty(COPY_CALIB_BYTES // 2, dtype=torch.bfloat16, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"ms_per_step": ms, "c_abi_warm_ms_per_step": abi_ms, "op_warm_ms_per_step": op_ms,
                          "copy_calib_bytes": COPY_CALIB_BYTES}), flush=True)
        return


    # ---- each kernel alone, HIP events on the launch stream ----
    launches = {
        "fwd": lambda: L.nn_fa_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                                   B, H, KVH, T, D, dt_code, scale, sp),
        "bwd_pre": lambda: L.nn_fa_bwd_pre(o.data_ptr(), do.data_ptr(), lse.data_ptr(), ws.data_ptr(), ws_bytes,
                                           B, H, KVH, T, D, dt_code, scale, sp),
        "bwd_dkdv": lambda: L.nn_fa_bwd_dkdv(q.data_ptr(), k.data_ptr(), v.data_ptr(), do.data_ptr(), ws.data_ptr(),
                                             ws_bytes, dk.data_ptr(), dv.data_ptr(), B, H, KVH, T, D, dt_code, scale, sp),
        "bwd_dq": lambda: L.nn_fa_bwd_dq(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(),
                                         lse.data_ptr(), ws.data_ptr(), ws_bytes, dq.data_ptr(), B, H, KVH, T, D,
                                         dt_code, scale, sp),
    }
    reps = max(20, args.steps)
    kern_us = {}
    for name, fn in launches.items():
        for _ in range(5):
            check(fn())
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            check(fn())
        e1.record(stream)
        e1.synchronize()
        kern_us[name] = e0.elapsed_time(e1) * 1e3 / reps
    # The clock the chip holds under this load (the 2.5 PFLOP/s peak assumes 2.4 GHz): sampled while the dK/dV
    # kernel alone, then the whole C-ABI step, run back to back.
    clocks = {
        "bwd_dkdv": gfx_clock(dev, lambda: [check(launches["bwd_dkdv"]()) for _ in range(100)]),
        "step": gfx_clock(dev, lambda: [step_abi() for _ in range(50)]),
    }

    # ---- layout fusion: the same fwd+bwd starting from the projection layout (B, T, heads, hd) ----
    # (after the per-kernel timings: its new allocations slow the next ~300 steps, see the warmup note)
    # "views": the reference model's flow (layers.py:97-104,116) -- transposed views into the dense ops,
    # which copy them to contiguous memory, then o transposed + reshaped for the output projection and
    # the gradients transposed back to the projection layout. "fused": nanonemo::flash_attn_bthd, which
    # reads and writes that layout directly.
    qp, kp, vp, dop = (t.transpose(1, 2).contiguous() for t in (q, k, v, do))

    def step_views():
        o2, lse2 = fa._flash_attn(qp.transpose(1, 2), kp.transpose(1, 2), vp.transpose(1, 2))
        y = o2.transpose(1, 2).reshape(B, T, H * D)
        g = fa._flash_attn_bwd(dop.transpose(1, 2), qp.transpose(1, 2), kp.transpose(1, 2), vp.transpose(1, 2), o2, lse2)
        return y, [t.transpose(1, 2).contiguous() for t in g]

    def step_fused():
        o2, lse2 = fa._flash_attn_bthd(qp, kp, vp)
        y = o2.view(B, T, H * D)
        return y, fa._flash_attn_bthd_bwd(dop, qp, kp, vp, o2, lse2)

    for _ in range(3):
        step_views()
        step_fused()
    t_end = time.perf_counter() + args.prewarm / 2
    while time.perf_counter() < t_end:
        for _ in range(50):
            step_views()
            step_fused()
        torch.cuda.synchronize()
    def host_ms(fn, n):  # the host's time per call in a loop of n calls (device work enqueued, not waited for)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        return (t1 - t0) * 1e3 / n

    views_ms = timed(step_views, args.steps)
    fused_ms = timed(step_fused, args.steps)
    views_host_ms, fused_host_ms = host_ms(step_views, args.steps), host_ms(step_fused, args.steps)

    # ---- q's RoPE folded into the attention, against the separate RoPE kernel, as GPU time: the C-ABI flows
    # back to back, timed with HIP events on the launch stream (the ops' host cost would set the pace of a loop of
    # op calls). Separate: nn_rope_qk(q, k) + the strided pair + nn_rope_qk_bwd(dq, dk). Fused: nn_rope_qk on k
    # alone + nn_fa_fwd_rope_strided / nn_fa_bwd_rope_strided (q rotated in the forward's registers, dq rotated
    # back in the dQ kernel) + nn_rope_qk_bwd on dk alone. ----
    from nanonemo_amd.kernels.hip import check_rope as _chk_rope
    from nanonemo_amd.kernels.hip import strides3 as _s3
    from nanonemo_amd.model import rope_tables as _tables

    cos_f, sin_f = (t.to(dev) for t in _tables(D, T, 10000.0))
    rq, rk, rdq, rdk, rdq2, rdk2 = (torch.empty_like(t) for t in (qp, kp, qp, kp, qp, kp))
    ro, rlse, rqrot = torch.empty_like(qp), torch.empty(B, H, T, device=dev), torch.empty_like(qp)
    rdv = torch.empty_like(vp)
    s_att_q, s_att_kv = _s3(T * H * D, D, H * D), _s3(T * KVH * D, D, KVH * D)   # (batch, head, row) strides
    s_rope_q, s_rope_kv = _s3(T * H * D, H * D, D), _s3(T * KVH * D, KVH * D, D)  # (batch, row, head) strides
    P = lambda t: t.data_ptr()  # noqa: E731

    def rope_flow(fused):
        hq = 0 if fused else H  # the fused flow rotates k alone
        _chk_rope(L.nn_rope_qk(P(qp), P(rq), P(kp), P(rk), P(cos_f), P(sin_f), B, T, hq, KVH, D, s_rope_q, s_rope_kv,
                               T, dt_code, sp))
        if fused:
            check(L.nn_fa_fwd_rope_strided(P(qp), P(rk), P(vp), P(ro), P(rlse), P(rqrot), P(cos_f), P(sin_f), T, B, H,
                                           KVH, T, D, s_att_q, s_att_kv, dt_code, scale, sp))
            check(L.nn_fa_bwd_rope_strided(P(dop), P(rqrot), P(rk), P(vp), P(ro), P(rlse), P(rdq), P(rdk), P(rdv),
                                           P(ws), ws_bytes, P(cos_f), P(sin_f), T, B, H, KVH, T, D, s_att_q,
                                           s_att_kv, dt_code, scale, sp))
        else:
            check(L.nn_fa_fwd_strided(P(rq), P(rk), P(vp), P(ro), P(rlse), B, H, KVH, T, D, s_att_q, s_att_kv, dt_code,
                                      scale, sp))
            check(L.nn_fa_bwd_strided(P(dop), P(rq), P(rk), P(vp), P(ro), P(rlse), P(rdq), P(rdk), P(rdv), P(ws),
                                      ws_bytes, B, H, KVH, T, D, s_att_q, s_att_kv, dt_code, scale, sp))
        _chk_rope(L.nn_rope_qk_bwd(P(rdq), P(rdq2), P(rdk), P(rdk2), P(cos_f), P(sin_f), B, T, hq, KVH, D, s_rope_q,
                                   s_rope_kv, T, dt_code, sp))

    rope_us = {}
    for fused in (False, True):
        for _ in range(5):
            rope_flow(fused)
    for trial in range(3):  # interleaved
        for fused in (False, True):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(args.steps):
                rope_flow(fused)
            e1.record(stream)
            e1.synchronize()
            rope_us.setdefault(fused, []).append(e0.elapsed_time(e1) * 1e3 / args.steps)
    rope_sep_us, rope_fused_us = (statistics.median(rope_us[f]) for f in (False, True))
    qbytes = B * T * H * D * dtype.itemsize

    # ---- the RoPE kernel beside the op (q and k in the projection layout, one launch) ----
    from nanonemo_amd.kernels.hip.rope import rope_qk
    from nanonemo_amd.model import rope, rope_tables

    from nanonemo_amd.kernels.hip import check_rope, strides3

    cos_t, sin_t = (t.to(dev) for t in rope_tables(D, T, 10000.0))
    for _ in range(5):
        rope_qk(qp, kp, cos_t, sin_t)
    rope_op_us = timed(lambda: rope_qk(qp, kp, cos_t, sin_t), max(20, args.steps)) * 1e3
    torch_rope_us = timed(lambda: (rope(qp, cos_t, sin_t, 1), rope(kp, cos_t, sin_t, 1)), max(20, args.steps)) * 1e3
    # the kernel alone: C-ABI launches with prepared arguments, events on the launch stream
    qr, kr = torch.empty_like(qp), torch.empty_like(kp)
    rope_args = (qp.data_ptr(), qr.data_ptr(), kp.data_ptr(), kr.data_ptr(), cos_t.data_ptr(), sin_t.data_ptr(),
                 B, T, H, KVH, D, strides3(T * H * D, H * D, D), strides3(T * KVH * D, KVH * D, D), T, dt_code, sp)
    for _ in range(5):
        check_rope(L.nn_rope_qk(*rope_args))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(200):
        check_rope(L.nn_rope_qk(*rope_args))
    e1.record(stream)
    e1.synchronize()
    rope_us = e0.elapsed_time(e1) * 1e3 / 200
    rope_bytes = 2 * (qp.numel() + kp.numel()) * qp.element_size()  # read and write q and k

    # ---- the fused add + RMSNorm on the model's residual stream (B*T rows of d_model) ----
    norm = _norm_launches(L, B * T, dev, sp)
    norm_us = {}
    for name in ("fwd", "bwd"):
        for _ in range(5):
            norm[name]()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(200):
            norm[name]()
        e1.record(stream)
        e1.synchronize()
        norm_us[name] = e0.elapsed_time(e1) * 1e3 / 200

    # The same C-ABI step captured once into a HIP graph and replayed (no host launch cost per kernel).
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        step_abi_on(side.cuda_stream)
    stream.wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        step_abi_on(torch.cuda.current_stream().cuda_stream)
    # (last of the measurements: the graph's memory pool and the flush buffer are new allocations, so the
    # replays settle for a while before they are timed, as the direct steps do)
    t_end = time.perf_counter() + args.prewarm / 2
    while time.perf_counter() < t_end:
        for _ in range(200):
            graph.replay()
        torch.cuda.synchronize()
    graph_ms = timed(graph.replay, args.steps)
    # The reference benchmark's method (benchmarks/kernels/common.py:30-54): every replay preceded by a
    # cache flush (a 512 MiB write, past the 256 MB Infinity Cache) and timed alone with events; median,
    # p20 and p80 over the replays.
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(max(100, args.steps))]
    for i, (a, b_) in enumerate(ev):
        flush.fill_(i & 0xFF)
        a.record(stream)
        graph.replay()
        b_.record(stream)
    torch.cuda.synchronize()
    ref_ms = sorted(a.elapsed_time(b_) for a, b_ in ev)
    # PyTorch's own attention on this GPU, beside this build's (last: SDPA math's scores are a large new
    # allocation, which would slow the measurements after it)
    sdpa_cmp = same_node(q, k, v, do, fa, max(20, args.steps // 2))

    # BASELINE config 2's own dtype: the same op pair on the same seeded inputs in the other 16-bit type, timed as the
    # headline (warm-up, settling steps, then K steps each after a cache flush, median).
    other = torch.float16 if dtype == torch.bfloat16 else torch.bfloat16
    q2, k2, v2, do2 = (t.to(other) for t in (q, k, v, do))

    def step_op2():
        o3, lse3 = fa._flash_attn(q2, k2, v2)
        return fa._flash_attn_bwd(do2, q2, k2, v2, o3, lse3)

    for _ in range(args.warmup):
        step_op2()
    t_end = time.perf_counter() + args.prewarm / 2
    while time.perf_counter() < t_end:
        for _ in range(100):
            step_op2()
        torch.cuda.synchronize()
    ev2 = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    for i, (a, b_) in enumerate(ev2):
        flush.fill_(i & 0xFF)
        a.record(stream)
        step_op2()
        b_.record(stream)
    torch.cuda.synchronize()
    other_ms = statistics.median(a.elapsed_time(b_) for a, b_ in ev2)
    del q2, k2, v2, do2

    e = 2  # bytes per 16-bit element
    pre_alg_bytes = 2 * B * H * T * D * e + 4 * B * H * T
    pre_all_bytes = pre_alg_bytes + 8 * B * H * T  # also reads lse and writes -lse/scale
    # Algorithmic FLOPs (8*D per causal pair for the backward) split by the products each kernel owns:
    # dV, dP, dK -> dk/dv kernel (6*D), dQ -> dq kernel (2*D); the dP and S recomputed by each are not counted.
    f_dkdv = 3.0 * B * H * D * T * (T + 1)
    f_dq = 1.0 * B * H * D * T * (T + 1)
    kern_tflops = {
        "fwd": f_fwd / (kern_us["fwd"] * 1e-6) / 1e12,
        "bwd_dkdv": f_dkdv / (kern_us["bwd_dkdv"] * 1e-6) / 1e12,
        "bwd_dq": f_dq / (kern_us["bwd_dq"] * 1e-6) / 1e12,
    }
    dominant = max(("fwd", "bwd_dkdv", "bwd_dq"), key=lambda n: kern_us[n])
    kernel_names = {"fwd": "fa_fwd_kernel", "bwd_dkdv": "fa_bwd_dkdv_kernel", "bwd_dq": "fa_bwd_dq_kernel"}

    # HBM bytes per launch of the dominant kernel are not measured in this run (that needs rocprofv3 counters): the
    # committed FETCH_SIZE / WRITE_SIZE summary of this workload (profiles/) is reported beside the roofline block,
    # labelled with its source, and roofline.traffic stays null.
    traffic_committed = None
    tfile = ROOT / "profiles" / f"fa_causal_gqa_b{B}_t{T}_{args.dtype}.traffic.json"
    if tfile.exists() and (H, KVH, D) == (12, 4, 64):
        measured = json.loads(tfile.read_text())
        key = f"{kernel_names[dominant]}<{D},{args.dtype}>"
        if key in measured:
            traffic_committed = {"kernel": kernel_names[dominant], "bytes_per_launch": round(measured[key]),
                                 "source": f"profiles/{tfile.name}: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of this "
                                 "workload, scaled by a device copy's readings; committed, not measured in this run"}

    value = f_all / (ms * 1e-3) / 1e12
    props = torch.cuda.get_device_properties(dev)
    sclk = (clocks["bwd_dkdv"] if dominant == "bwd_dkdv" else clocks["step"]).get("gfx_mhz_median")
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic",
        "config": {
            "workload": f"causal GQA attention fwd+bwd, B={B} T={T} {H}Q/{KVH}KV heads d={D} {args.dtype}: one "
            "nanonemo::flash_attn + nanonemo::flash_attn_bwd op pair per step on inputs resident in HBM, each step "
            "after a 512 MiB last-level-cache flush and timed alone with HIP events (median of the K steps)",
            "B": B, "T": T, "H": H, "KVH": KVH, "D": D, "input_scale": args.input_scale,
        },
        "pct_of_bf16_peak": round(100 * value / PEAK_TFLOPS, 2),
        "step_ms": {
            "median": round(ms, 5),
            "p20": round(sorted(step_ms)[len(step_ms) // 5], 5),
            "p80": round(sorted(step_ms)[(4 * len(step_ms)) // 5], 5),
            "mean": round(statistics.fmean(step_ms), 5),
        },
        # warm caches, back to back (the inputs stay in the 256 MB Infinity Cache between steps)
        "other_dtype": {
            "dtype": "fp16" if other == torch.float16 else "bf16",
            "how": "the same op pair on the same seeded inputs cast to the other 16-bit type, timed as the headline",
            "ms_per_step": round(other_ms, 5),
            "value": round(f_all / (other_ms * 1e-3) / 1e12, 2),
        },
        "c_abi_warm_ms_per_step": round(abi_ms, 5),
        "c_abi_warm_tflops": round(f_all / (abi_ms * 1e-3) / 1e12, 2),
        "op_warm_ms_per_step": round(op_ms, 5),
        "graph_ms_per_step": round(graph_ms, 5),
        "ref_method": {
            "how": "HIP-graph replay of the C-ABI step, each after a 512 MiB cache-flush write, timed alone with events",
            "replays": len(ref_ms),
            "median_ms": round(statistics.median(ref_ms), 5),
            "p20_ms": round(ref_ms[len(ref_ms) // 5], 5),
            "p80_ms": round(ref_ms[(4 * len(ref_ms)) // 5], 5),
            "tflops_at_median": round(f_all / (statistics.median(ref_ms) * 1e-3) / 1e12, 2),
            # the FlashAttention-paper convention, 3.5 x 2*B*H*T^2*D, for comparison only
            "paper_convention_tflops_at_median": round(3.5 * 2 * B * H * T * T * D / (statistics.median(ref_ms) * 1e-3) / 1e12, 2),
        },
        "rope_qk": {
            "kernel_us": round(rope_us, 2),
            "GBps": round(rope_bytes / (rope_us * 1e-6) / 1e9, 1),
            "op_us": round(rope_op_us, 2),
            "torch_formula_us": round(torch_rope_us, 2),
        },
        "add_rmsnorm": {
            "shape": f"{B * T} x {NORM_D}, x fp32 + delta bf16 -> y bf16, h fp32",
            "fwd_us": round(norm_us["fwd"], 2),
            "fwd_GBps": round(norm["fwd_bytes"] / (norm_us["fwd"] * 1e-6) / 1e9, 1),
            "bwd_us": round(norm_us["bwd"], 2),
            "bwd_GBps": round(norm["bwd_bytes"] / (norm_us["bwd"] * 1e-6) / 1e9, 1),
        },
        "rope_fusion": {
            "how": "GPU time of the C-ABI flows back to back (HIP events, median of 3 interleaved runs): nn_rope_qk(q, "
            "k) + nn_fa_fwd_strided + nn_fa_bwd_strided + nn_rope_qk_bwd(dq, dk), against nn_rope_qk(k) + "
            "nn_fa_fwd_rope_strided + nn_fa_bwd_rope_strided (q rotated in the forward's registers, dq rotated back "
            "in the dQ kernel) + nn_rope_qk_bwd(dk)",
            "separate_us_per_step": round(rope_sep_us, 2),
            "fused_us_per_step": round(rope_fused_us, 2),
            "saved_us": round(rope_sep_us - rope_fused_us, 2),
            # the RoPE kernel's read of q (its q_rot write moves into the forward) and rope_qk_bwd's read and
            # write of dq
            "q_trip_bytes_removed": 3 * qbytes,
        },
        "same_node": {
            "how": "fwd + autograd.grad back to back, warm caches, HIP events (host_ms: the host's time per call in the "
            "same loop); SDPA as the reference benchmark runs it (repeat_interleave'd K/V), flash with native GQA; "
            "op_pair = this build's two ops without autograd",
            "this_build_op_pair_ms": round(op_ms, 5),
            **sdpa_cmp,
        },
        "layout_fusion": {
            "from": "projection layout (B, T, heads, hd)",
            "views_ms_per_step": round(views_ms, 5),
            "fused_ms_per_step": round(fused_ms, 5),
            "speedup": round(views_ms / fused_ms, 3),
            # the host's time per step in the same loops: where it reaches the step time, the host sets the pace
            "views_host_ms_per_step": round(views_host_ms, 5),
            "fused_host_ms_per_step": round(fused_host_ms, 5),
        },
        "roofline": {
            "kernel": kernel_names[dominant],
            "bound": "mfma",
            "achieved": round(kern_tflops[dominant], 2),
            "peak": PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(kern_tflops[dominant] / PEAK_TFLOPS, 4),
            "traffic": None,
            # the same peak scaled to the GFX clock measured while the kernel ran back to back
            "sclk_mhz": sclk,
            "peak_at_sclk": round(PEAK_TFLOPS * sclk / 2400.0, 1) if sclk else None,
            "frac_at_sclk": round(kern_tflops[dominant] / (PEAK_TFLOPS * sclk / 2400.0), 4) if sclk else None,
        },
        "traffic_committed": traffic_committed,
        "clock": clocks,
        "kernels": {
            "fwd_us": round(kern_us["fwd"], 2),
            "fwd_tflops": round(kern_tflops["fwd"], 2),
            # the standalone preprocessing entry point (nn_fa_bwd fuses the same pass into the dQ kernel)
            "bwd_pre_standalone_us": round(kern_us["bwd_pre"], 2),
            "bwd_pre_alg_GBps": round(pre_alg_bytes / (kern_us["bwd_pre"] * 1e-6) / 1e9, 1),
            "bwd_pre_moved_GBps": round(pre_all_bytes / (kern_us["bwd_pre"] * 1e-6) / 1e9, 1),
            "bwd_dkdv_us": round(kern_us["bwd_dkdv"], 2),
            "bwd_dkdv_tflops": round(kern_tflops["bwd_dkdv"], 2),
            "bwd_dq_us": round(kern_us["bwd_dq"], 2),
            "bwd_dq_tflops": round(kern_tflops["bwd_dq"], 2),
            "bwd_tflops": round(f_bwd / ((kern_us["bwd_dkdv"] + kern_us["bwd_dq"]) * 1e-6) / 1e12, 2),
        },
        "device": {"name": props.name, "cus": props.multi_processor_count, "arch": getattr(props, "gcnArchName", "")},
    }
    if not args.no_config5 and (B, T, H, KVH, D) == (8, 1024, 12, 4, 64):
        del graph, flush
        torch.cuda.empty_cache()
        out["config5"] = config5(args.config5_steps)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
