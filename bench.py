"""Benchmark of the FP8 sliding-window-attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c3|c4|c1|c2|c5|c2_train|ref_fp8|swa_bf16|swa_bf16_450m|fp8_train_450m|fp8_block_train_450m]

Default workload (the headline metric): fp8_swa_attention_forward on
B=4, H=16, T=8192, D=64, window=1024, causal; Q/K/V bf16 ~ N(0, 1) with each head scaled by a
lognormal(0, 1) factor (seeded), per-head e4m3 scales. One step = the whole operator as
flw_fp8_swa_attention_forward runs it: one amax + e4m3 quantise launch pair for Q, K and V (V into
the MFMA tile layout; Q's codes deferred: the pair writes Q's scale and reciprocal only) and the
fused FP8 attention kernel, which reads Q in bf16 and quantises it on load, on inputs already
resident in HBM. Everything runs through the C ABI of libflower_amd.so on torch's current stream.

Before the W warm-up steps, the step runs untimed for SPIN_UP_S seconds (clock spin-up).

Printed (one JSON line):
  value      -- in-window attention FLOP/s of the whole step, TFLOP/s (4*D per in-window pair)
  roofline   -- the attention kernel alone (a HIP event pair per launch, recorded from the
                kernel's own dispatch on the stream it runs on, via flw_time_next_launch): achieved TFLOP/s against MI355X dense FP8 MFMA peak
                (5.0 PFLOP/s); traffic = its measured HBM bytes per launch (TRAFFIC below)
  quant      -- the quantise launch pair: algorithmic bytes (Q, K, V read by the amax pass; K, V
                read again and their codes written by the quantise pass) / their time (event pair
                recorded by the pair's own dispatches), against 8 TB/s HBM
  cpu_baseline -- the CPU oracle of the FP8-simulated reference path (e4m3 quantise, dequantise,
                banded fp32 softmax attention) on a bounded sample of the same workload, host
                cores, scaled linearly to the same unit.

--workload c2 measures the FP8 weight-cache linear of BASELINE.json config 2 instead (bf16
x[8192, 1024] with 0.1 % outliers at 20x, cached e4m3 weight [4096, 1024] with per-output-channel
scales): the headline is the weight-only GEMM (e4m3 weight x bf16 activations on bf16 MFMA, one
kernel per step); the A8W8 recipe (per-row activation quantisation + FP8 GEMM) is reported
beside it, in GEMM TFLOP/s.
--workload swa_bf16 / swa_bf16_450m measure the bf16 sliding-window attention training op (forward
with log-sum-exp, then the backward) at the reference's measurement shape B1 H20 T4096 D64 W2048 /
its 450M model shape B2 H20 T8192 D64 W2048; roofline = the backward entry point.
--workload fp8_train_450m measures the differentiable FP8 attention (fp8_swa_attention: FP8 forward,
bf16 backward at the dequantised Q, K, V) as one autograd training step at the 450M model shape.
--workload c2_train measures the C2 linear as an FP8 training step (forward, dgrad and wgrad GEMMs
with their quantisers), beside torch's bf16 matmuls of the same three products.
--workload fp8_block_train_450m measures one 450M block (d 1280, 20 heads, SwiGLU 3392, W 2048,
QK-norm + RoPE; B2 x T8192) forward + backward with its Linears converted to FP8 (tensorwise, the
reference's configs' recipe), beside rowwise and bf16 Linears, in ms per block: the reference's
own FP8-linear training measurement (precision.py:3-9, an RTX 5090, reported as context).
Other configs are parity-test cases; c1 / c4 are accepted here for measurement only.
--library-gemm-reference runs no workload: it times hipBLASLt (through torch) at the GEMM shapes,
the reference point for the library's own GEMMs.
--issue-probe runs no workload: it measures, on one SIMD at four waves, the issue cost of each
instruction class of the attention loop (v_fma, v_exp, v_max3, v_cvt_pk_fp8, v_mul,
v_permlane32_swap, the FP8 MFMA) and how much of the MFMA hides under each VALU class, the
figures the attention kernel's time is accounted with.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "FP8 SWA attn fwd TFLOPS + % FP8 MFMA peak at T=8192,W=1024; quant GB/s"
FP8_PEAK_TFLOPS = 5000.0     # MI355X dense FP8 MFMA
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA
HBM_PEAK_GBPS = 8000.0       # MI355X HBM3E
COPY_PROBE_BYTES = 256 << 20

WORKLOADS = {
    "c3": dict(B=4, H=16, T=8192, D=64, W=1024, granularity="head", inputs="lognormal_heads"),
    "c4": dict(B=1, H=16, T=32768, D=64, W=4096, granularity="head", inputs="student_t_channels"),
    "c1": dict(B=1, H=8, T=1024, D=64, W=256, granularity="tensor", inputs="randn_fp32"),
    # the reference's own published FP8 measurement shape (fp8_swa_attention.py:39-46: 0.431 ms
    # on an RTX 5090, per-tensor scales) -- other hardware, so context only, not a baseline
    "ref_fp8": dict(B=1, H=20, T=4096, D=64, W=2048, granularity="tensor", inputs="randn_bf16",
                    label="the reference's published FP8 measurement shape B1 H20 T4096 D64 W2048"),
    "c2": dict(M=8192, N=4096, K=1024, outlier_frac=0.001, outlier_scale=20.0, w_std=0.02),
    "c5": dict(B=1, T=32768, d_model=1024, num_heads=16, ffn_dim=4096, W=4096, w_std=0.02),
    # the C2 linear as a training step: forward + FP8 dgrad + FP8 wgrad (rowwise recipe)
    "c2_train": dict(M=8192, N=4096, K=1024, outlier_frac=0.001, outlier_scale=20.0, w_std=0.02),
    # bf16 sliding-window attention as a training op (forward with log-sum-exp + backward): the
    # reference's own measurement shape (swa_attention.py:10-14, :40-43) and its 450M model shape
    "swa_bf16": dict(B=1, H=20, T=4096, D=64, W=2048, ref="B1 H20 T4096 D64 W2048"),
    "swa_bf16_450m": dict(B=2, H=20, T=8192, D=64, W=2048, ref="B2 H20 T8192 D64 W2048"),
    # the differentiable FP8 attention (FP8 forward, bf16 backward) as a training step, 450M shape
    "fp8_train_450m": dict(B=2, H=20, T=8192, D=64, W=2048, granularity="head", ref="B2 H20 T8192 D64 W2048"),
    # one 450M block (vanilla_matched: d 1280, 20 heads, SwiGLU 3392, W 2048) forward + backward
    # with its Linears converted to FP8: the reference's own FP8-linear training measurement
    # (precision.py:3-9: 13.61 ms tensorwise, 18.72 rowwise, 18.87 bf16 per block on an RTX 5090,
    # compiled) -- other hardware, so context only, not a baseline
    "fp8_block_train_450m": dict(B=2, T=8192, recipe="tensorwise", w_std=0.02,
                                 reference_rtx5090_ms={"tensorwise": 13.61, "rowwise": 18.72, "bf16": 18.87}),
}
DATA = {
    "lognormal_heads": "synthetic (seeded; bf16 N(0,1) x a lognormal(0,1) factor per head)",
    "student_t_channels": "synthetic (seeded; bf16 N(0,1), 4 of 64 channels Student-t nu=4)",
    "randn_fp32": "synthetic (seeded; fp32 N(0,1))",
    "randn_bf16": "synthetic (seeded; bf16 N(0,1))",
    "c2": "synthetic (seeded; bf16 x N(0,1) with 0.1% outliers x20; weight N(0,0.02), random init)",
    "c5": "synthetic (seeded; bf16 x N(0,1); every Linear weight N(0,0.02), random init)",
    "swa_bf16": "synthetic (seeded; bf16 q, k, v, dO ~ N(0,1))",
    "block_train": "synthetic (seeded; bf16 x, dy ~ N(0,1); every Linear weight N(0,0.02), random init)",
}

# HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE on each workload, as
# recorded in profiles/ (swa_fwd_c3.md, swa_fwd_c4.md, fp8_gemm_c2.md, w8a16_gemm_c2.md,
# swa_bf16_450m.md). FETCH_SIZE is scaled by 2.0: a plain 256 MiB device copy reads back
# 131,088 KiB of FETCH_SIZE against 262,144 KiB of WRITE_SIZE (scale 1.0). The attention kernel
# reads Q in bf16 (quantised on load); "quant" is the deferred-Q quantise pair.
TRAFFIC = {
    "c3": {"swa_fwd": 209_343_898, "quant": 403_801_190},
    "c4": {"swa_fwd": 209_952_154, "quant": 403_344_998},
    "c2": {"gemm": 117_834_752, "w8a16": 134_490_112},
    "swa_bf16_450m": {"bwd": 554_757_120, "fwd": 169_459_712},
}


def make_inputs(cfg, seed=0):
    B, H, T, D = cfg["B"], cfg["H"], cfg["T"], cfg["D"]
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(3):
        if cfg["inputs"] == "lognormal_heads":
            x = torch.randn(B, H, T, D, generator=g) * torch.randn(1, H, 1, 1, generator=g).exp()
            out.append(x.to(torch.bfloat16))
        elif cfg["inputs"] == "student_t_channels":
            x = torch.randn(B, H, T, D, generator=g)
            ch = torch.randperm(D, generator=g)[:4]
            # Student-t, nu = 4: z / sqrt(chi2_4 / 4), chi2_4 as a sum of four squared normals
            z = torch.randn(B, H, T, 4, generator=g)
            chi2 = torch.randn(B, H, T, 4, 4, generator=g).square().sum(-1)
            x[..., ch] = z / (chi2 / 4.0).sqrt()
            out.append(x.to(torch.bfloat16))
        elif cfg["inputs"] == "randn_bf16":
            out.append(torch.randn(B, H, T, D, generator=g).to(torch.bfloat16))
        else:
            out.append(torch.randn(B, H, T, D, generator=g))
    return out


def make_gemm_inputs(cfg, seed=0):
    """bf16 activations with 0.1 % outliers at 20x, bf16 weight N(0, 0.02)."""
    M, N, K = cfg["M"], cfg["N"], cfg["K"]
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    n_out = int(round(cfg["outlier_frac"] * M * K))
    pos = torch.randperm(M * K, generator=g)[:n_out]
    x.view(-1)[pos] *= cfg["outlier_scale"]
    w = torch.randn(N, K, generator=g) * cfg["w_std"]
    return x.to(torch.bfloat16), w.to(torch.bfloat16)


def host_threads() -> int:
    """Host threads the CPU baseline runs on: the cores this process may use (its CPU affinity,
    i.e. os.cpu_count() where no affinity limit applies), further capped by OMP_NUM_THREADS when
    the launcher sets it (a shared GPU box grants each job a share of the host that way). The
    number is reported with the baseline."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def in_window_pairs(T, W):
    ramp = min(T, W)
    return ramp * (ramp + 1) // 2 + max(0, T - W) * W


def _events(n, per=2):
    """n tuples of `per` timing events, created up front (torch creates an event lazily, on its
    first record) so their handles can be passed to the library before the timed region."""
    ev = [tuple(torch.cuda.Event(enable_timing=True) for _ in range(per)) for _ in range(n)]
    for t in ev:
        for e in t:
            e.record()
    return ev


SPIN_UP_S = 0.3


def _spin_up(step, seconds=SPIN_UP_S):
    """Run the step, untimed, until `seconds` of wall time have passed. An idle MI355X needs
    ~20-30 ms of sustained work to leave its low clock state: the first ~100 attention launches
    of a fresh process run ~15 % slower than the rest, so W short warm-up steps alone would time
    the clock ramp rather than the kernels."""
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            step()
        torch.cuda.synchronize()


def _wall_ms(step, steps):
    """Mean wall time of `steps` back-to-back steps in ms, bracketed by device synchronisation,
    with nothing else in the loop: the whole-job throughput (`value`). Kernel times come from a
    separate loop with the dispatch-recorded event pairs, whose recording would otherwise sit
    inside this interval."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps * 1e3


def _arm(lib, pair):
    """The next entry point called records this event pair from its own dispatches
    (flw_time_next_launch -> hipExtLaunchKernel): start with its first kernel, stop with its last,
    so the interval holds those kernels and no marker packets."""
    from flower_amd import _lib
    _lib.check(lib.flw_time_next_launch(pair[0].cuda_event, pair[1].cuda_event), "timer")


class AttentionStep:
    """The operator as C-ABI launches, as flw_fp8_swa_attention_forward runs it: one quantise pass
    pair over Q, K, V with Q's codes deferred (flw_quant_qkv_e4m3_deferq: the amax pass reads all
    three, the quantise pass writes K / V codes and the scales), then the attention kernel, which
    reads Q in bf16 and quantises it on load (flw_fp8_swa_fwd_qx)."""

    def __init__(self, q, k, v, cfg):
        from flower_amd import _lib
        self.L, self.lib = _lib, _lib.load()
        self.q, self.k, self.v = q, k, v
        B, H, T, D = q.shape
        self.shape = (B, H, T, D)
        self.W = cfg["W"]
        self.gran = _lib.GRANULARITY[cfg["granularity"]]
        G = {0: 1, 1: H, 2: B * H}[self.gran]
        dev = q.device
        self.q8 = torch.empty((B, H, T, D), dtype=torch.uint8, device=dev)   # non-finite groups only
        self.k8 = torch.empty_like(self.q8)
        self.vt = torch.empty(self.lib.flw_vtile_bytes(B, H, T, D), dtype=torch.uint8, device=dev)
        self.sc = torch.empty(3 * G, dtype=torch.float32, device=dev)
        self.qr = torch.empty(G, dtype=torch.float32, device=dev)
        self.G = G
        self.ws = _lib.workspace(3 * self.lib.flw_quant_workspace_bytes(B, H, T, D), dev)
        self.out = torch.empty((B, H, T, D), dtype=q.dtype, device=dev)
        self.dt = _lib.dtype_code(q.dtype)
        self.s8 = _lib.i64s(H * T * D, T * D, D)
        self.so = _lib.i64s(*self.out.stride()[:3])
        self.sq = _lib.i64s(*q.stride()[:3])
        self.sx = _lib.i64s(*q.stride()[:3], *k.stride()[:3], *v.stride()[:3])

    def quant(self, stream):
        B, H, T, D = self.shape
        rc = self.lib.flw_quant_qkv_e4m3_deferq(self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), self.dt,
                                                B, H, T, D, self.sx, self.gran, self.q8.data_ptr(),
                                                self.k8.data_ptr(), self.vt.data_ptr(), self.sc.data_ptr(),
                                                self.qr.data_ptr(), self.ws.data_ptr(), self.ws.numel(), stream)
        self.L.check(rc, "quant")

    def attend(self, stream):
        B, H, T, D = self.shape
        G, base = self.G, self.sc.data_ptr()
        rc = self.lib.flw_fp8_swa_fwd_qx(self.q.data_ptr(), self.sq, self.q8.data_ptr(), self.qr.data_ptr(),
                                         self.k8.data_ptr(), self.s8, self.vt.data_ptr(), base, base + 4 * G,
                                         base + 8 * G, self.gran, self.out.data_ptr(), self.dt, self.so,
                                         B, H, T, D, self.W, stream)
        self.L.check(rc, "swa")


def bench_attention(cfg, steps, warmup):
    q, k, v = (t.cuda() for t in make_inputs(cfg))
    step = AttentionStep(q, k, v, cfg)
    stream = torch.cuda.current_stream().cuda_stream
    _spin_up(lambda: (step.quant(stream), step.attend(stream)))
    for _ in range(warmup):
        step.quant(stream)
        step.attend(stream)
    wall_ms = _wall_ms(lambda: (step.quant(stream), step.attend(stream)), steps)
    ev, kev = _events(steps), _events(steps)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        _arm(step.lib, ev[i])
        step.quant(stream)
        _arm(step.lib, kev[i])
        step.attend(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    quant_ms = np.array([e[0].elapsed_time(e[1]) for e in ev])
    attn_ms = np.array([e[0].elapsed_time(e[1]) for e in kev])
    B, H, T, D = q.shape
    return dict(wall_s=wall, ms_per_step=wall_ms, quant_ms=float(np.mean(quant_ms)),
                attn_ms=float(np.mean(attn_ms)), attn_ms_min=float(np.min(attn_ms)),
                flops=4 * D * B * H * in_window_pairs(T, cfg["W"]),
                # amax pass: Q, K, V read; quantise pass: K, V read, their codes written
                quant_bytes=B * H * T * D * (5 * q.element_size() + 2), dtype=q.dtype)


def bench_gemm(cfg, steps, warmup):
    """BASELINE config 2 through the C ABI: weight quantised once (the FP8 weight cache), then per
    step per-row activation quantisation + the scaled FP8 GEMM, events around the GEMM."""
    from flower_amd import _lib
    lib = _lib.load()
    x, w = (t.cuda() for t in make_gemm_inputs(cfg))
    M, N, K = cfg["M"], cfg["N"], cfg["K"]
    stream = torch.cuda.current_stream().cuda_stream
    w8 = torch.empty((N, K), dtype=torch.uint8, device="cuda")
    ws_ = torch.empty(N, dtype=torch.float32, device="cuda")
    _lib.check(lib.flw_quant_rows_e4m3(w.data_ptr(), _lib.BF16, N, K, K, w8.data_ptr(), ws_.data_ptr(), stream), "w")
    x8 = torch.empty((M, K), dtype=torch.uint8, device="cuda")
    sx = torch.empty(M, dtype=torch.float32, device="cuda")
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")

    def quant():
        _lib.check(lib.flw_quant_rows_e4m3(x.data_ptr(), _lib.BF16, M, K, K, x8.data_ptr(), sx.data_ptr(), stream), "x")

    def gemm():
        _lib.check(lib.flw_fp8_scaled_mm(x8.data_ptr(), M, K, w8.data_ptr(), N, sx.data_ptr(), M,
                                         ws_.data_ptr(), N, y.data_ptr(), N, stream), "gemm")

    _spin_up(lambda: (quant(), gemm()))
    for _ in range(warmup):
        quant()
        gemm()
    wall_ms = _wall_ms(lambda: (quant(), gemm()), steps)
    kev = _events(steps)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        quant()
        _arm(lib, kev[i])
        gemm()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    g_ms = np.array([e[0].elapsed_time(e[1]) for e in kev])
    # the row quantiser alone, timed after the steps (it has no timing hook of its own)
    qev = _events(steps)
    for a, b in qev:
        a.record()
        quant()
        b.record()
    torch.cuda.synchronize()
    q_ms = np.array([a.elapsed_time(b) for a, b in qev])
    return dict(wall_s=wall, ms_per_step=wall_ms, quant_ms=float(q_ms.mean()),
                gemm_ms=float(g_ms.mean()), gemm_ms_min=float(g_ms.min()), flops=2 * M * N * K,
                quant_bytes=M * K * (2 * 2 + 1) + 4 * M, gemm_bytes=M * K + N * K + 2 * M * N + 4 * (M + N),
                x=x, w=w)


def bench_gemm_w8a16(cfg, steps, warmup):
    """BASELINE config 2, weight-only: the cached per-channel e4m3 weight times the bf16
    activations as they are (flw_fp8_linear, FLW_GEMM_W8A16: one kernel per step)."""
    from flower_amd import _lib
    lib = _lib.load()
    x, w = (t.cuda() for t in make_gemm_inputs(cfg))
    M, N, K = cfg["M"], cfg["N"], cfg["K"]
    stream = torch.cuda.current_stream().cuda_stream
    w8 = torch.empty((N, K), dtype=torch.uint8, device="cuda")
    ws_ = torch.empty(N, dtype=torch.float32, device="cuda")
    _lib.check(lib.flw_quant_rows_e4m3(w.data_ptr(), _lib.BF16, N, K, K, w8.data_ptr(), ws_.data_ptr(), stream), "w")
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")

    def gemm():
        _lib.check(lib.flw_fp8_linear(x.data_ptr(), M, K, K, w8.data_ptr(), N, ws_.data_ptr(), N,
                                      _lib.GEMM_W8A16, y.data_ptr(), N, None, 0, stream), "w8a16")

    _spin_up(gemm)
    for _ in range(warmup):
        gemm()
    wall_ms = _wall_ms(gemm, steps)
    kev = _events(steps)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        _arm(lib, kev[i])
        gemm()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    g_ms = np.array([e[0].elapsed_time(e[1]) for e in kev])
    return dict(wall_s=wall, ms_per_step=wall_ms, gemm_ms=float(g_ms.mean()),
                gemm_ms_min=float(g_ms.min()), flops=2 * M * N * K,
                gemm_bytes=2 * M * K + N * K + 2 * M * N + 4 * N, x=x, w=w)


def cpu_baseline(cfg, budget_s=20.0):
    """Oracle of the FP8-simulated reference path on the host: e4m3 quantise, dequantise, banded
    fp32 attention, head by head (all B of each) until the time budget, scaled linearly."""
    from threadpoolctl import threadpool_limits
    from oracle.quant import dequant, per_tensor_fp8
    from oracle.swa import swa_banded
    cores = host_threads()
    B, H, T, D, W = cfg["B"], cfg["H"], cfg["T"], cfg["D"], cfg["W"]
    q, k, v = (t.float().numpy() for t in make_inputs(cfg))
    gran = cfg["granularity"]
    done_heads, t_total = 0, 0.0
    with threadpool_limits(cores):
        if gran == "tensor":                     # one scale over all heads: quantise once, timed
            t0 = time.perf_counter()
            full = [dequant(*per_tensor_fp8(x, "tensor")) for x in (q, k, v)]
            t_total += time.perf_counter() - t0
        for h in range(H):
            t0 = time.perf_counter()
            if gran == "tensor":
                deq = [x[:, h:h + 1] for x in full]
            else:
                deq = [dequant(*per_tensor_fp8(x[:, h:h + 1], gran)) for x in (q, k, v)]
            swa_banded(*deq, W, chunk=512)
            t_total += time.perf_counter() - t0
            done_heads += 1
            if t_total > budget_s:
                break
    flops = 4 * D * B * done_heads * in_window_pairs(T, W)
    return {"value": flops / t_total / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"{done_heads} of {H} heads (all {B} batches each) of the same workload in "
                      f"{t_total:.1f} s: oracle e4m3 quantise + dequantise + banded fp32 softmax "
                      f"attention (numpy / multithreaded BLAS), FLOPs counted as in-window 4*D per pair"}


def cpu_baseline_gemm(x, w, budget_s=15.0, weight_only=False):
    """The oracle on the host: per-row e4m3 of W (once, outside the timing, as the weight cache
    does), then per row block of x either the _fp8_head recipe (per-row e4m3 of x, closed-form
    scaled GEMM) or the weight-only product, until the time budget."""
    from threadpoolctl import threadpool_limits
    from oracle.gemm import fp8_linear_a8w8, fp8_linear_w8a16
    from oracle.quant import rowwise_fp8
    cores = host_threads()
    xf, wf = x.float().cpu().numpy(), w.float().cpu().numpy()
    w8, sw = rowwise_fp8(wf)
    rows, t_total = 0, 0.0
    with threadpool_limits(cores):
        for r0 in range(0, xf.shape[0], 512):
            t0 = time.perf_counter()
            if weight_only:
                fp8_linear_w8a16(xf[r0:r0 + 512], w8, sw.reshape(-1))
            else:
                fp8_linear_a8w8(xf[r0:r0 + 512], w8, sw.reshape(-1))
            t_total += time.perf_counter() - t0
            rows += min(512, xf.shape[0] - r0)
            if t_total > budget_s:
                break
    flops = 2 * rows * wf.shape[0] * wf.shape[1]
    return {"value": flops / t_total / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"{rows} of {xf.shape[0]} activation rows in {t_total:.1f} s: oracle " +
                      ("weight-only product (float64 x @ dequant(w8)^T, numpy / BLAS)" if weight_only else
                       "per-row e4m3 quantisation + float64 closed-form scaled GEMM (numpy / BLAS)") +
                      "; weight quantised once outside the timing, as the weight cache does"}


# Instruction classes of flw_diag_issue_probe (bit mask) and the attention loop's count of each per
# 64-key tile and wave (steady state, from the kernel's assembly).
ISSUE_CLASSES = {1: "v_fma_f32", 2: "v_exp_f32", 4: "v_max3_f32", 8: "v_cvt_pk_fp8_f32", 16: "v_mul_f32",
                 32: "v_permlane32_swap_b32", 64: "v_mfma_scale_f32_32x32x64_f8f6f4"}
ISSUE_PROBES = [1, 2, 4, 8, 16, 32, 64, 65, 66, 68, 72, 80, 3, 67]


LIBRARY_GEMM_SHAPES = {"c2": (8192, 4096, 1024), "c5_qkv": (32768, 3072, 1024), "c5_ff1": (32768, 4096, 1024),
                       "c5_ff2": (32768, 1024, 4096), "c5_o": (32768, 1024, 1024)}


def library_gemm_reference(steps=50):
    """The vendor GEMM at this build's GEMM shapes (M, N, K): torch's bf16 matmul and FP8
    torch._scaled_mm (e4m3 operands, bf16 out) with per-row x per-column scales (the A8W8 recipe's
    scaling) and with per-tensor scales, all on hipBLASLt. Timed with events over `steps` calls
    after 5 warm-up calls. A reference point only: no epilogue (residual, amax) is included."""
    for name, (M, N, K) in LIBRARY_GEMM_SHAPES.items():
        g = torch.Generator(device="cuda").manual_seed(0)
        a = torch.randn(M, K, device="cuda", dtype=torch.bfloat16, generator=g)
        b = torch.randn(N, K, device="cuda", dtype=torch.bfloat16, generator=g)
        a8, b8 = a.to(torch.float8_e4m3fn), b.to(torch.float8_e4m3fn)
        sa, sb = torch.ones(M, 1, device="cuda"), torch.ones(1, N, device="cuda")
        one = torch.ones((), device="cuda")
        calls = {"bf16_matmul": lambda: a @ b.t(),
                 "fp8_scaled_mm_rowwise": lambda: torch._scaled_mm(a8, b8.t(), scale_a=sa, scale_b=sb,
                                                                   out_dtype=torch.bfloat16),
                 "fp8_scaled_mm_tensorwise": lambda: torch._scaled_mm(a8, b8.t(), scale_a=one, scale_b=one,
                                                                      out_dtype=torch.bfloat16)}
        rec = {"shape": name, "M": M, "N": N, "K": K}
        for key, fn in calls.items():
            try:
                for _ in range(5):
                    fn()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(steps):
                    fn()
                e1.record()
                torch.cuda.synchronize()
                us = e0.elapsed_time(e1) / steps * 1e3
                rec[key] = {"us": round(us, 2), "tflops": round(2 * M * N * K / us / 1e6, 1)}
            except RuntimeError as e:                 # a recipe this torch build lacks
                rec[key] = {"error": str(e)[:120]}
        print(json.dumps(rec), flush=True)


def issue_probe():
    """Per-SIMD issue cost of single instruction classes and of MFMA + VALU mixes (four waves per
    SIMD, the attention kernel's occupancy). A probe kernel runs `iters` iterations per wave of 32
    independent VALU instructions per class in its mask and / or 2 independent MFMAs; the cost of
    one iteration on one SIMD is the kernel time divided by the iterations all waves of a SIMD run.
    For a mix, `overlap` is the fraction of the smaller component hidden under the larger."""
    from flower_amd import _lib
    lib = _lib.load_diag()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    blocks = 4 * cus                              # 4 workgroups of 4 waves per CU = 4 waves per SIMD
    iters = lib.flw_diag_issue_probe_iters()
    out = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    waves_per_simd = blocks * 4 / (4 * cus)
    per_iter = {}
    for mask in ISSUE_PROBES:
        call = lambda: _lib.check(lib.flw_diag_issue_probe(mask, out.data_ptr(), out.numel(), blocks, stream), "probe", lib)
        call()
        torch.cuda.synchronize()
        ev = _events(5)
        for a, b in ev:
            a.record()
            call()
            b.record()
        torch.cuda.synchronize()
        ms = float(np.median([a.elapsed_time(b) for a, b in ev]))
        ns = ms * 1e6 / (iters * waves_per_simd)
        per_iter[mask] = ns
        parts = [m for m in ISSUE_CLASSES if mask & m]
        rec = {"probe": "+".join(ISSUE_CLASSES[m] for m in parts), "mask": mask, "ns_per_iter_per_simd": round(ns, 3)}
        if len(parts) == 1:
            n = 2 if mask == 64 else 32
            rec["ns_per_instruction"] = round(ns / n, 4)
            rec["cycles_at_2.4GHz"] = round(ns / n * 2.4, 2)
        else:
            comp = [per_iter[m] for m in parts if m in per_iter]
            if len(comp) == len(parts):
                rec["sum_of_parts_ns"] = round(sum(comp), 3)
                rec["overlap"] = round((sum(comp) - ns) / min(comp), 3)
        rec.update(iters=iters, waves_per_simd=waves_per_simd, device=torch.cuda.get_device_name(0))
        print(json.dumps(rec), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="c3", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="first run one plain 256 MiB device copy, the reference point that scales "
                         "the HBM byte counters of a rocprofv3 --pmc run")
    ap.add_argument("--library-gemm-reference", action="store_true",
                    help="instead of a workload, time the vendor GEMM (hipBLASLt through torch: bf16 "
                         "matmul, FP8 _scaled_mm with per-row x per-column and per-tensor scales) at "
                         "the C2 shape and C5's four linear shapes, the reference point for the "
                         "library's own GEMMs; prints one JSON line per shape")
    ap.add_argument("--qk-route", choices=("epilogue", "quantiser"), default="epilogue",
                    help="c5 only: where the block applies HeadRMSNorm + RoPE to q and k -- in the QKV "
                         "GEMM's epilogue (the default) or in both quantiser passes")
    ap.add_argument("--issue-probe", action="store_true",
                    help="instead of a workload, measure the per-SIMD issue cost of the attention "
                         "loop's instruction classes and their overlap with the FP8 MFMA "
                         "(flw_diag_issue_probe); prints one JSON line per probe")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on exactly one GPU (every box here has one); it measures "
              "one GPU's share of the work (attention shards by batch and head with no "
              "communication). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.issue_probe:
        issue_probe()
        return
    if args.library_gemm_reference:
        library_gemm_reference()
        return
    cfg = WORKLOADS[args.workload]
    if args.copy_probe:
        src = torch.empty(COPY_PROBE_BYTES, dtype=torch.uint8, device="cuda").fill_(1)
        torch.empty_like(src).copy_(src)
        torch.cuda.synchronize()
        del src
    if args.workload == "c2":
        line = run_gemm(cfg, args)
    elif args.workload == "c5":
        line = run_block(cfg, args)
    elif args.workload.startswith("swa_bf16"):
        line = run_swa_bf16(cfg, args)
    elif args.workload == "c2_train":
        line = run_linear_train(cfg, args)
    elif args.workload == "fp8_train_450m":
        line = run_fp8_train(cfg, args)
    elif args.workload == "fp8_block_train_450m":
        line = run_block_train(cfg, args)
    else:
        line = run_attention(cfg, args)
    print(json.dumps(line), flush=True)


def run_attention(cfg, args):
    r = bench_attention(cfg, args.steps, args.warmup)
    value = r["flops"] / (r["ms_per_step"] * 1e-3) / 1e12
    attn_tflops = r["flops"] / (r["attn_ms"] * 1e-3) / 1e12
    quant_gbps = r["quant_bytes"] / (r["quant_ms"] * 1e-3) / 1e9
    traffic = TRAFFIC.get(args.workload, {})
    dt = {torch.bfloat16: "bf16", torch.float32: "fp32"}[r["dtype"]]
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup, "spin_up_s": SPIN_UP_S,
        "ms_per_step": round(r["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 (fp32 accumulate)",
        "data": DATA[cfg["inputs"]],
        "config": {"workload": "fp8_swa_attention_forward, " + cfg.get("label", f"BASELINE {args.workload.upper()}"),
                   "B": cfg["B"], "H": cfg["H"], "T": cfg["T"], "D": cfg["D"], "window": cfg["W"],
                   "causal": True, "scales": cfg["granularity"], "input_dtype": dt},
        "roofline": {"bound": "mfma", "achieved": round(attn_tflops, 2), "peak": FP8_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(attn_tflops / FP8_PEAK_TFLOPS, 4),
                     "traffic": traffic.get("swa_fwd"),
                     "kernel": f"swa_fwd_kernel<{cfg['D']}, {dt}>", "kernel_ms": round(r["attn_ms"], 4),
                     "kernel_ms_min": round(r["attn_ms_min"], 4), "flop_per_launch": r["flops"]},
        "quant": {"bound": "hbm", "achieved": round(quant_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                  "frac": round(quant_gbps / HBM_PEAK_GBPS, 4), "ms": round(r["quant_ms"], 4),
                  "algorithmic_bytes": r["quant_bytes"], "traffic": traffic.get("quant")},
        "attention_pct_fp8_peak": round(100 * attn_tflops / FP8_PEAK_TFLOPS, 2),
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(cfg)
    return line


def run_gemm(cfg, args):
    """BASELINE config 2. Headline: the weight-only FP8 linear (e4m3 cached weight x bf16
    activations, bf16 MFMA); alongside: the A8W8 recipe (per-row e4m3 activations, FP8 MFMA)."""
    r = bench_gemm_w8a16(cfg, args.steps, args.warmup)
    value = r["flops"] / (r["ms_per_step"] * 1e-3) / 1e12
    g_tflops = r["flops"] / (r["gemm_ms"] * 1e-3) / 1e12
    a = bench_gemm(cfg, args.steps, args.warmup)
    a_tflops = a["flops"] / (a["gemm_ms"] * 1e-3) / 1e12
    line = {
        "metric": "FP8 weight-cache linear TFLOPS (e4m3 per-channel weight x bf16 activations), BASELINE config 2",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup, "spin_up_s": SPIN_UP_S,
        "ms_per_step": round(r["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 MFMA (e4m3 weight widened exactly to bf16), fp32 accumulate",
        "data": DATA["c2"],
        "config": {"workload": "fp8 weight-only linear from the weight cache, BASELINE C2", "M": cfg["M"],
                   "N": cfg["N"], "K": cfg["K"], "scales": "per-output-channel weight"},
        "roofline": {"bound": "mfma", "achieved": round(g_tflops, 2), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(g_tflops / BF16_PEAK_TFLOPS, 4),
                     "traffic": TRAFFIC["c2"].get("w8a16"), "algorithmic_bytes": r["gemm_bytes"],
                     "kernel": "w8a16_gemm_kernel", "kernel_ms": round(r["gemm_ms"], 4),
                     "kernel_ms_min": round(r["gemm_ms_min"], 4), "flop_per_launch": r["flops"]},
        "a8w8": {"value": round(a["flops"] / (a["ms_per_step"] * 1e-3) / 1e12, 2), "unit": "TFLOP/s",
                 "ms_per_step": round(a["ms_per_step"], 4),
                 "roofline": {"bound": "mfma", "achieved": round(a_tflops, 2), "peak": FP8_PEAK_TFLOPS,
                              "unit": "TFLOP/s", "frac": round(a_tflops / FP8_PEAK_TFLOPS, 4),
                              "traffic": TRAFFIC["c2"]["gemm"], "algorithmic_bytes": a["gemm_bytes"],
                              "kernel": "fp8_gemm_256_kernel", "kernel_ms": round(a["gemm_ms"], 4),
                              "kernel_ms_min": round(a["gemm_ms_min"], 4)},
                 "quant": {"bound": "hbm", "achieved": round(a["quant_bytes"] / (a["quant_ms"] * 1e-3) / 1e9, 1),
                           "peak": HBM_PEAK_GBPS, "unit": "GB/s", "ms": round(a["quant_ms"], 4),
                           "algorithmic_bytes": a["quant_bytes"]}},
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_gemm(r["x"], r["w"], weight_only=True)
    return line


def run_block(cfg, args):
    """one FP8 decoder block forward (RMSNorm -> QKV -> HeadRMSNorm + RoPE of q, k
    (the reference block's qkv_heads) -> per-head FP8 SWA -> O -> residual -> RMSNorm -> GELU MLP ->
    residual), every Linear from the FP8 weight cache."""
    from flower_amd.block import Fp8DecoderBlock, block_flops, init_block_
    from flower_amd.precision import fp8_weight_cache
    B, T, d = cfg["B"], cfg["T"], cfg["d_model"]
    blk = Fp8DecoderBlock(d, cfg["num_heads"], cfg["ffn_dim"], cfg["W"])
    init_block_(blk, std=cfg["w_std"], seed=0)
    blk = blk.to("cuda", torch.bfloat16)
    blk.fuse_qk_epilogue = args.qk_route == "epilogue"
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, T, d, generator=g).to("cuda", torch.bfloat16)
    flops = block_flops(T, B, d, cfg["ffn_dim"], cfg["num_heads"], cfg["W"])
    with fp8_weight_cache(blk):
        _spin_up(lambda: blk(x))
        for _ in range(args.warmup):
            blk(x)
        wall_ms = _wall_ms(lambda: blk(x), args.steps)
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
        torch.cuda.synchronize()
        for a, b in ev:
            a.record()
            blk(x)
            b.record()
        torch.cuda.synchronize()
    ms = float(np.mean([a.elapsed_time(b) for a, b in ev]))
    wall = wall_ms * 1e-3 * args.steps
    value = flops / (wall / args.steps) / 1e12
    return {
        "metric": "FP8 decoder block forward TFLOPS (linear + in-window attention FLOPs), BASELINE config 5",
        "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "spin_up_s": SPIN_UP_S, "ms_per_step": round(wall / args.steps * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp8_e4m3 (fp32 accumulate), bf16 activations",
        "data": DATA["c5"],
        "config": {"workload": "Fp8DecoderBlock forward, BASELINE C5", "B": B, "T": T, "d_model": d,
                   "num_heads": cfg["num_heads"], "ffn_dim": cfg["ffn_dim"], "window": cfg["W"],
                   "qk_norm": blk.attn.qk_norm is not None, "rope_base": blk.attn.rope._base,
                   "qk_route": args.qk_route,
                   "scales": "per-head attention, per-row x per-channel linears"},
        "roofline": {"bound": "mfma", "achieved": round(flops / (ms * 1e-3) / 1e12, 2), "peak": FP8_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(flops / (ms * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4),
                     "traffic": None, "kernel": "whole block (HIP events around each forward)",
                     "kernel_ms": round(ms, 4), "flop_per_launch": flops},
    }


def bench_swa_bf16(cfg, steps, warmup):
    """One training step of the attention op through the C ABI: flw_swa_bf16_fwd (O and the
    log-sum-exp) then flw_swa_bf16_bwd (Delta, dK/dV, dQ), each timed by its own dispatches."""
    from flower_amd import _lib
    lib = _lib.load()
    B, H, T, D, W = cfg["B"], cfg["H"], cfg["T"], cfg["D"], cfg["W"]
    g = torch.Generator().manual_seed(0)
    q, k, v, do = (torch.randn(B, H, T, D, generator=g).to("cuda", torch.bfloat16) for _ in range(4))
    out = torch.empty_like(q)
    lse = torch.empty((B, H, T), dtype=torch.float32, device="cuda")
    dq, dk, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
    ws = _lib.workspace(lib.flw_swa_bf16_bwd_workspace_bytes(B, H, T, D), q.device)
    stream = torch.cuda.current_stream().cuda_stream

    def fwd():
        _lib.check(lib.flw_swa_bf16_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), B, H, T, D, W,
                                        out.data_ptr(), lse.data_ptr(), stream), "fwd")

    def bwd():
        _lib.check(lib.flw_swa_bf16_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), do.data_ptr(),
                                        lse.data_ptr(), B, H, T, D, W, dq.data_ptr(), dk.data_ptr(),
                                        dv.data_ptr(), ws.data_ptr(), ws.numel(), stream), "bwd")

    _spin_up(lambda: (fwd(), bwd()))
    for _ in range(warmup):
        fwd()
        bwd()
    wall_ms = _wall_ms(lambda: (fwd(), bwd()), steps)
    fev, bev = _events(steps), _events(steps)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        _arm(lib, fev[i])
        fwd()
        _arm(lib, bev[i])
        bwd()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    f_ms = np.array([a.elapsed_time(b) for a, b in fev])
    b_ms = np.array([a.elapsed_time(b) for a, b in bev])
    pairs = B * H * in_window_pairs(T, W)
    return dict(wall_s=wall, ms_per_step=wall_ms, fwd_ms=float(f_ms.mean()), fwd_ms_min=float(f_ms.min()),
                bwd_ms=float(b_ms.mean()), bwd_ms_min=float(b_ms.min()), fwd_flops=4 * D * pairs,
                bwd_flops=10 * D * pairs)


def cpu_baseline_swa_bf16(cfg, budget_s=20.0):
    """The float64 oracle of the same op (oracle/swa_grad.py: banded forward + log-sum-exp, then
    the backward) on the host, (b, h) slice by slice until the time budget, scaled linearly."""
    from threadpoolctl import threadpool_limits
    from oracle.swa_grad import swa_backward, swa_forward_lse
    cores = host_threads()
    B, H, T, D, W = cfg["B"], cfg["H"], cfg["T"], cfg["D"], cfg["W"]
    g = torch.Generator().manual_seed(0)
    q, k, v, do = (torch.randn(1, 1, T, D, generator=g).to(torch.bfloat16).double().numpy() for _ in range(4))
    done, t_total = 0, 0.0
    with threadpool_limits(cores):
        while t_total < budget_s and done < B * H:
            t0 = time.perf_counter()
            o, lse = swa_forward_lse(q, k, v, W, chunk=512)
            swa_backward(q, k, v, o, lse, do, W, chunk=512)
            t_total += time.perf_counter() - t0
            done += 1
    flops = 14 * D * done * in_window_pairs(T, W)
    return {"value": flops / t_total / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"{done} of {B * H} (b, h) slices of the same workload in {t_total:.1f} s: oracle "
                      f"float64 banded forward + log-sum-exp + backward (numpy / multithreaded BLAS), "
                      f"FLOPs counted as 4*D + 10*D per in-window pair"}


def run_swa_bf16(cfg, args):
    """bf16 sliding-window attention, forward (with log-sum-exp) + backward, one training step.
    FLOPs per in-window (query, key) pair: forward 4*D (Q K^T, P V), backward 10*D (S recomputed,
    dP, dV, dK, dQ), as FlashAttention counts them; the dQ kernel's second S / dP (14*D in all) is
    not counted."""
    r = bench_swa_bf16(cfg, args.steps, args.warmup)
    flops = r["fwd_flops"] + r["bwd_flops"]
    value = flops / (r["ms_per_step"] * 1e-3) / 1e12
    b_tf = r["bwd_flops"] / (r["bwd_ms"] * 1e-3) / 1e12
    f_tf = r["fwd_flops"] / (r["fwd_ms"] * 1e-3) / 1e12
    line = {
        "metric": "bf16 SWA attention forward+backward TFLOPS (training op), % bf16 MFMA peak",
        "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "spin_up_s": SPIN_UP_S, "ms_per_step": round(r["ms_per_step"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 MFMA, fp32 softmax / accumulate", "data": DATA["swa_bf16"],
        "config": {"workload": f"swa_attention forward + backward, {cfg['ref']}", "B": cfg["B"], "H": cfg["H"],
                   "T": cfg["T"], "D": cfg["D"], "window": cfg["W"], "causal": True},
        "roofline": {"bound": "mfma", "achieved": round(b_tf, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(b_tf / BF16_PEAK_TFLOPS, 4),
                     "traffic": TRAFFIC.get(args.workload, {}).get("bwd"),
                     "kernel": "flw_swa_bf16_bwd (delta + dkdv + dq kernels)", "kernel_ms": round(r["bwd_ms"], 4),
                     "kernel_ms_min": round(r["bwd_ms_min"], 4), "flop_per_launch": r["bwd_flops"]},
        "forward": {"bound": "mfma", "achieved": round(f_tf, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(f_tf / BF16_PEAK_TFLOPS, 4), "kernel": "swa_bf16_fwd_kernel<64>",
                    "traffic": TRAFFIC.get(args.workload, {}).get("fwd"),
                    "ms": round(r["fwd_ms"], 4), "ms_min": round(r["fwd_ms_min"], 4), "flop_per_launch": r["fwd_flops"]},
        "fwd_plus_bwd_kernel_ms": round(r["fwd_ms"] + r["bwd_ms"], 4),
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_swa_bf16(cfg)
    return line


def bench_fp8_train(cfg, steps, warmup):
    """One autograd training step of fp8_swa_attention (bf16 q, k, v with requires_grad, a seeded
    dO): the forward (the e4m3 quantiser pair over Q, K, V, then the FP8 kernel) and the backward
    (three e4m3 dequantisers, the bf16 forward recomputing O and the log-sum-exp at the dequantised
    values, the bf16 backward), each bracketed by events on the current stream."""
    from flower_amd.kernels import fp8_swa_attention
    B, H, T, D, W = cfg["B"], cfg["H"], cfg["T"], cfg["D"], cfg["W"]
    g = torch.Generator().manual_seed(0)
    q, k, v, do = (torch.randn(B, H, T, D, generator=g).to("cuda", torch.bfloat16) for _ in range(4))
    for t in (q, k, v):
        t.requires_grad_(True)

    def fwd():
        return fp8_swa_attention(q, k, v, W, granularity=cfg["granularity"])

    def step():
        q.grad = k.grad = v.grad = None
        fwd().backward(do)

    _spin_up(step)
    for _ in range(warmup):
        step()
    wall_ms = _wall_ms(step, steps)
    ev = _events(steps, per=3)
    torch.cuda.synchronize()
    for i in range(steps):
        q.grad = k.grad = v.grad = None
        ev[i][0].record()
        out = fwd()
        ev[i][1].record()
        out.backward(do)
        ev[i][2].record()
    torch.cuda.synchronize()
    f_ms = np.array([a.elapsed_time(b) for a, b, _ in ev])
    b_ms = np.array([b.elapsed_time(c) for _, b, c in ev])
    pairs = B * H * in_window_pairs(T, W)
    return dict(ms_per_step=wall_ms, fwd_ms=float(f_ms.mean()), bwd_ms=float(b_ms.mean()),
                fwd_flops=4 * D * pairs, bwd_flops=10 * D * pairs)


def run_fp8_train(cfg, args):
    """The differentiable FP8 attention, one training step. FLOPs per in-window pair: forward 4*D
    (on the FP8 MFMA), backward 10*D (bf16 MFMA); the backward's recomputed bf16 forward (4*D more)
    is not counted. roofline = the FP8 forward (its share of the step on the FP8 peak)."""
    r = bench_fp8_train(cfg, args.steps, args.warmup)
    flops = r["fwd_flops"] + r["bwd_flops"]
    value = flops / (r["ms_per_step"] * 1e-3) / 1e12
    f_tf = r["fwd_flops"] / (r["fwd_ms"] * 1e-3) / 1e12
    b_tf = r["bwd_flops"] / (r["bwd_ms"] * 1e-3) / 1e12
    return {
        "metric": "FP8 SWA attention training step TFLOPS (FP8 forward, bf16 backward at the dequantised "
                  "Q/K/V), 450M model shape",
        "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "spin_up_s": SPIN_UP_S, "ms_per_step": round(r["ms_per_step"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp8_e4m3 forward, bf16 backward (fp32 softmax / accumulate)", "data": DATA["swa_bf16"],
        "config": {"workload": f"fp8_swa_attention forward + backward, {cfg['ref']}", "B": cfg["B"], "H": cfg["H"],
                   "T": cfg["T"], "D": cfg["D"], "window": cfg["W"], "causal": True,
                   "scales": cfg["granularity"]},
        "roofline": {"bound": "mfma", "achieved": round(f_tf, 2), "peak": 5000.0, "unit": "TFLOP/s",
                     "frac": round(f_tf / 5000.0, 4), "traffic": None,
                     "kernel": "the FP8 forward (quantiser pair + swa_fwd_kernel<64, bf16>), events around it",
                     "kernel_ms": round(r["fwd_ms"], 4), "flop_per_launch": r["fwd_flops"]},
        "backward": {"bound": "mfma", "achieved": round(b_tf, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(b_tf / BF16_PEAK_TFLOPS, 4), "ms": round(r["bwd_ms"], 4),
                     "kernels": "3 x dequant + swa_bf16_fwd (recompute) + flw_swa_bf16_bwd"},
    }


def bench_block_train(cfg, steps, warmup, recipe):
    """One training step (forward + backward, weight gradients included) of the 450M block
    (flower_amd.block.TransformerBlock, block_config()): its five Linears converted by
    convert_model_to_fp8 with ``recipe`` (None: left in bf16, torch's GEMMs), the attention on the
    HIP bf16 sliding-window kernels, RMSNorm, the head split with QK-norm + RoPE and the SwiGLU
    product on the HIP row kernels (forward and backward), the residual adds folded into the norms'
    passes and (FP8 tensorwise) the down projection's GEMM epilogue."""
    import copy
    import torch.nn as nn
    from flower_amd.block import TransformerBlock, block_config, init_block_
    from flower_amd.precision import convert_model_to_fp8
    B, T = cfg["B"], cfg["T"]
    conf = block_config()
    block = init_block_(TransformerBlock(conf), std=cfg["w_std"], seed=0).to("cuda", torch.bfloat16)
    stack = nn.Module()
    stack.blocks = nn.ModuleList([copy.deepcopy(block)])
    if recipe is not None:
        convert_model_to_fp8(stack, recipe=recipe, keep_bf16_blocks=0, verbose=False)
    blk = stack.blocks[0]
    g = torch.Generator().manual_seed(1)
    x = torch.randn(B, T, conf.d_model, generator=g).to("cuda", torch.bfloat16).requires_grad_(True)
    dy = torch.randn(B, T, conf.d_model, generator=g).to("cuda", torch.bfloat16)

    def step():
        x.grad = None
        for prm in blk.parameters():
            prm.grad = None
        blk(x)[0].backward(dy)

    _spin_up(step)
    for _ in range(warmup):
        step()
    wall_ms = _wall_ms(step, steps)
    ev = _events(steps, per=3)
    torch.cuda.synchronize()
    for i in range(steps):
        x.grad = None
        for prm in blk.parameters():
            prm.grad = None
        ev[i][0].record()
        out = blk(x)[0]
        ev[i][1].record()
        out.backward(dy)
        ev[i][2].record()
    torch.cuda.synchronize()
    f_ms = np.array([a.elapsed_time(b) for a, b, _ in ev])
    b_ms = np.array([b.elapsed_time(c) for _, b, c in ev])
    lin = sum(m.weight.numel() for m in blk.modules() if isinstance(m, nn.Linear))
    D, H, W = conf.d_model // conf.num_heads, conf.num_heads, conf.local_window
    pairs = B * H * in_window_pairs(T, W)
    return dict(ms_per_step=wall_ms, fwd_ms=float(f_ms.mean()), bwd_ms=float(b_ms.mean()),
                linear_flops=6 * lin * B * T, attn_flops=14 * D * pairs,
                converted=sum(type(m).__name__ == "Fp8Linear" for m in blk.modules()))


def run_block_train(cfg, args):
    """The 450M block's training step with FP8 Linears (cfg recipe, tensorwise as the reference's
    configs), beside the same block with rowwise FP8 and with bf16 Linears, each in ms per block
    (the reference's unit); FLOPs counted as 6 x Linear weights x tokens plus 14 D per in-window
    attention pair (forward 4 D, backward 10 D). ``value`` is the FP8 block's TFLOP/s."""
    runs = {name: bench_block_train(cfg, args.steps, args.warmup, rec)
            for name, rec in (("tensorwise", "tensorwise"), ("rowwise", "rowwise"), ("bf16", None))}
    main = runs[cfg["recipe"]]
    flops = main["linear_flops"] + main["attn_flops"]
    ref = cfg["reference_rtx5090_ms"]
    return {
        "metric": "450M block training step (forward + backward) with FP8 Linears, TFLOPS and ms per block",
        "value": round(flops / (main["ms_per_step"] * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "spin_up_s": SPIN_UP_S,
        "ms_per_step": round(main["ms_per_step"], 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"fp8_e4m3 Linears ({cfg['recipe']}; FP8 forward, dgrad and wgrad), bf16 attention and elementwise",
        "data": DATA["block_train"],
        "config": {"workload": "TransformerBlock forward + backward, 450M vanilla_matched", "B": cfg["B"],
                   "T": cfg["T"], "d_model": 1280, "num_heads": 20, "ffn": "swiglu 3392", "window": 2048,
                   "qk_norm": True, "recipe": cfg["recipe"], "converted_linears": main["converted"]},
        "roofline": {"bound": "mfma", "achieved": round(flops / (main["ms_per_step"] * 1e-3) / 1e12, 2),
                     "peak": FP8_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(flops / (main["ms_per_step"] * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4),
                     "traffic": None, "kernel": "the whole block step (wall time)",
                     "kernel_ms": round(main["ms_per_step"], 4), "flop_per_launch": flops},
        "ms_per_block": {k: round(v["ms_per_step"], 4) for k, v in runs.items()},
        "forward_ms": {k: round(v["fwd_ms"], 4) for k, v in runs.items()},
        "backward_ms": {k: round(v["bwd_ms"], 4) for k, v in runs.items()},
        "speedup_vs_bf16": {k: round(runs["bf16"]["ms_per_step"] / v["ms_per_step"], 3)
                            for k, v in runs.items() if k != "bf16"},
        "reference_rtx5090_ms_per_block": ref,
    }


def bench_linear_train(cfg, steps, warmup):
    """One FP8 training step of the C2 linear through the C ABI, rowwise recipe, weights quantised
    once outside the steps (the weight cache: row codes for the forward, column codes for dgrad):
      forward  x8 = rows(x); y = x8 . w8^T                          (2 launches)
      dgrad    g8 = rows(g); dx = g8 . w8c^T                        (2)
      wgrad    g8c = cols(g), x8c = cols(x) (transposed); dW = g8c . x8c^T   (3)
    Each entry point is timed by the event pair its own dispatches record."""
    from flower_amd import _lib
    lib = _lib.load()
    M, N, K = cfg["M"], cfg["N"], cfg["K"]
    x, w = (t.cuda() for t in make_gemm_inputs(cfg))
    g = torch.randn(M, N, generator=torch.Generator().manual_seed(1)).to("cuda", torch.bfloat16)
    stream = torch.cuda.current_stream().cuda_stream
    Mp = (M + 127) // 128 * 128
    u8 = lambda *sh: torch.empty(sh, dtype=torch.uint8, device="cuda")
    f32 = lambda n: torch.empty(n, dtype=torch.float32, device="cuda")
    bf = lambda *sh: torch.empty(sh, dtype=torch.bfloat16, device="cuda")
    w8, sw, w8c, swc = u8(N, K), f32(N), u8(K, N), f32(K)
    x8, sx, y = u8(M, K), f32(M), bf(M, N)
    g8, sg, dx = u8(M, N), f32(M), bf(M, K)
    g8c, sgc, x8c, sxc, dw = u8(N, Mp), f32(N), u8(K, Mp), f32(K), bf(N, K)
    ws = torch.empty(max(lib.flw_quant_cols_workspace_bytes(M, N), lib.flw_quant_cols_workspace_bytes(M, K),
                         lib.flw_quant_cols_workspace_bytes(N, K)), dtype=torch.uint8, device="cuda")
    C = _lib.check
    C(lib.flw_quant_rows_e4m3(w.data_ptr(), _lib.BF16, N, K, K, w8.data_ptr(), sw.data_ptr(), stream), "w rows")
    C(lib.flw_quant_cols_e4m3(w.data_ptr(), _lib.BF16, N, K, K, _lib.SCALE_COLUMN, w8c.data_ptr(), N,
                              swc.data_ptr(), ws.data_ptr(), ws.numel(), stream), "w cols")

    mws = torch.empty(max(256, lib.flw_fp8_scaled_mm_workspace_bytes(M, N, K), lib.flw_fp8_scaled_mm_workspace_bytes(M, K, N),
                          lib.flw_fp8_scaled_mm_workspace_bytes(N, K, Mp)), dtype=torch.uint8, device="cuda")

    def mm(a8, sa, b8, sb, out, m, n, k):     # split over K into mws when [m, n] has few tiles
        C(lib.flw_fp8_scaled_mm_ws(a8.data_ptr(), m, k, b8.data_ptr(), n, sa.data_ptr(), sa.numel(),
                                   sb.data_ptr(), sb.numel(), out.data_ptr(), n, mws.data_ptr(), mws.numel(),
                                   stream), "mm")

    calls = [
        ("fwd_quant", lambda: C(lib.flw_quant_rows_e4m3(x.data_ptr(), _lib.BF16, M, K, K, x8.data_ptr(),
                                                        sx.data_ptr(), stream), "x rows")),
        ("fwd_gemm", lambda: mm(x8, sx, w8, sw, y, M, N, K)),
        ("dgrad_quant", lambda: C(lib.flw_quant_rows_e4m3(g.data_ptr(), _lib.BF16, M, N, N, g8.data_ptr(),
                                                          sg.data_ptr(), stream), "g rows")),
        ("dgrad_gemm", lambda: mm(g8, sg, w8c, swc, dx, M, K, N)),
        ("wgrad_quant_g", lambda: C(lib.flw_quant_cols_e4m3(g.data_ptr(), _lib.BF16, M, N, N, _lib.SCALE_COLUMN,
                                                            g8c.data_ptr(), Mp, sgc.data_ptr(), ws.data_ptr(),
                                                            ws.numel(), stream), "g cols")),
        ("wgrad_quant_x", lambda: C(lib.flw_quant_cols_e4m3(x.data_ptr(), _lib.BF16, M, K, K, _lib.SCALE_COLUMN,
                                                            x8c.data_ptr(), Mp, sxc.data_ptr(), ws.data_ptr(),
                                                            ws.numel(), stream), "x cols")),
        ("wgrad_gemm", lambda: mm(g8c, sgc, x8c, sxc, dw, N, K, Mp)),
    ]

    def step():
        for _, f in calls:
            f()

    _spin_up(step)
    for _ in range(warmup):
        step()
    wall_ms = _wall_ms(step, steps)
    ev = [_events(steps) for _ in calls]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        for j, (_, f) in enumerate(calls):
            _arm(lib, ev[j][i])
            f()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = {name: float(np.mean([a.elapsed_time(b) for a, b in ev[j]])) for j, (name, _) in enumerate(calls)}
    # the same three products in bf16 through torch (hipBLASLt), for comparison
    wt = w.t()
    for _ in range(3):                      # library heuristics / first-call set-up outside the timing
        torch.matmul(x, wt)
        torch.matmul(g, w)
        torch.matmul(g.t(), x)
    torch.cuda.synchronize()
    tev = _events(steps, per=4)
    for a, b, c_, d in tev:
        a.record()
        torch.matmul(x, wt)
        b.record()
        torch.matmul(g, w)
        c_.record()
        torch.matmul(g.t(), x)
        d.record()
    torch.cuda.synchronize()
    bf16 = {"fwd_ms": float(np.median([a.elapsed_time(b) for a, b, _, _ in tev])),
            "dgrad_ms": float(np.median([b.elapsed_time(c_) for _, b, c_, _ in tev])),
            "wgrad_ms": float(np.median([c_.elapsed_time(d) for _, _, c_, d in tev]))}
    return dict(wall_s=wall, ms_per_step=wall_ms, ms=ms, bf16=bf16, flops_gemm=2 * M * N * K,
                x=x, w=w, g=g)


def cpu_baseline_linear_train(x, w, g, budget_s=15.0):
    """The oracle's FP8 forward + backward (oracle/gemm.py: per-row / per-column e4m3, float64
    closed-form GEMMs) on a sub-batch of token rows, scaled to the same FLOPs unit."""
    from threadpoolctl import threadpool_limits
    from oracle.gemm import fp8_linear_a8w8, fp8_linear_backward
    from oracle.quant import rowwise_fp8
    cores = host_threads()
    xf, wf, gf = (t.float().cpu().numpy() for t in (x, w, g))
    w8, sw = rowwise_fp8(wf)
    rows, t_total = 0, 0.0
    with threadpool_limits(cores):
        for r0 in range(0, xf.shape[0], 1024):
            t0 = time.perf_counter()
            fp8_linear_a8w8(xf[r0:r0 + 1024], w8, sw.reshape(-1))
            fp8_linear_backward(gf[r0:r0 + 1024], xf[r0:r0 + 1024], wf, "rowwise")
            t_total += time.perf_counter() - t0
            rows += min(1024, xf.shape[0] - r0)
            if t_total > budget_s:
                break
    flops = 3 * 2 * rows * wf.shape[0] * wf.shape[1]
    return {"value": flops / t_total / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"{rows} of {xf.shape[0]} token rows in {t_total:.1f} s, 1024 at a time: oracle per-row / "
                      f"per-column e4m3 + float64 closed-form forward, dgrad and wgrad GEMMs (numpy / BLAS); "
                      f"the weight's column codes re-made per sub-batch"}


def run_linear_train(cfg, args):
    r = bench_linear_train(cfg, args.steps, args.warmup)
    ms, f = r["ms"], r["flops_gemm"]
    value = 3 * f / (r["ms_per_step"] * 1e-3) / 1e12
    tf = lambda t: round(f / (t * 1e-3) / 1e12, 2)
    gemms = {k: ms[k] for k in ("fwd_gemm", "dgrad_gemm", "wgrad_gemm")}
    dom = max(gemms, key=gemms.get)
    line = {
        "metric": "FP8 linear training step TFLOPS (forward + dgrad + wgrad, rowwise e4m3), BASELINE C2 shape",
        "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "spin_up_s": SPIN_UP_S, "ms_per_step": round(r["ms_per_step"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp8_e4m3 (fp32 accumulate), bf16 in / out", "data": DATA["c2"],
        "config": {"workload": "Fp8Linear training step at the C2 shape", "M": cfg["M"], "N": cfg["N"],
                   "K": cfg["K"], "recipe": "rowwise (per-row x / g for forward / dgrad, per-column g / x for wgrad)"},
        "roofline": {"bound": "mfma", "achieved": tf(gemms[dom]), "peak": FP8_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(f / (gemms[dom] * 1e-3) / 1e12 / FP8_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": f"fp8_gemm_256_kernel ({dom})", "kernel_ms": round(gemms[dom], 4),
                     "flop_per_launch": f},
        "kernels_ms": {k: round(v, 4) for k, v in ms.items()},
        "gemm_tflops": {k: tf(v) for k, v in gemms.items()},
        "bf16_torch_ms": {k: round(v, 4) for k, v in r["bf16"].items()},
        "bf16_torch_tflops": {k: tf(v) for k, v in r["bf16"].items()},
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_linear_train(r["x"], r["w"], r["g"])
    return line


if __name__ == "__main__":
    main()
