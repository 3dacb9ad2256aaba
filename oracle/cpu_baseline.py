"""CPU baseline of the A8W8 path (TEST/BENCH INFRASTRUCTURE ONLY).

Timed by bench.py's cpu_baseline leg, never shipped or called by the product.
It is this repo's port of the reference's own CPU formula: per-token E4M3FN
quantization of bf16 activations (tests/test_misc.py:532-536 with QMAX 448 and
float8_e4m3fn in place of 127/int8) followed by the fp32 dequant matmul of
tests/test_gemm.py:116, in PyTorch on the host's cores.
"""
from __future__ import annotations

import os
import statistics
import time

import torch


def quantize_per_token(x: torch.Tensor):
    """bf16 [M, K] -> (float8_e4m3fn [M, K], fp32 [M, 1])."""
    xf = x.float()
    s = (xf.abs().amax(dim=1, keepdim=True) / 448.0).clamp(min=1e-10)
    q = (xf * (1.0 / s)).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q, s


def dequant_matmul(q: torch.Tensor, s: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor) -> torch.Tensor:
    """C = (A.f @ B.f^T) * a_s * b_s -> bf16 (tests/test_gemm.py:116)."""
    return ((q.float() @ wq.float().T) * s * ws.reshape(1, -1)).to(torch.bfloat16)


def run(M: int = 128, N: int = 4096, K: int = 4096, seed: int = 0, budget_s: float = 12.0, warmup: int = 3,
        min_reps: int = 10):
    """Time quant + dequant matmul on config 0 of BASELINE (X [M,K] ~ N(0,1),
    W [N,K] ~ N(0,0.02) quantized per output channel). Returns a dict with the
    median times and TFLOP/s of the total."""
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    wq, ws = quantize_per_token(w)  # per output channel = per row of W
    for _ in range(warmup):
        dequant_matmul(*quantize_per_token(x), wq, ws)
    tq, tm = [], []
    t_start = time.perf_counter()
    while len(tq) < min_reps or (time.perf_counter() - t_start < budget_s and len(tq) < 1000):
        t0 = time.perf_counter()
        q, s = quantize_per_token(x)
        t1 = time.perf_counter()
        dequant_matmul(q, s, wq, ws)
        t2 = time.perf_counter()
        tq.append(t1 - t0)
        tm.append(t2 - t1)
    total = [a + b for a, b in zip(tq, tm)]
    med = statistics.median(total)
    return {
        "threads": threads,
        "reps": len(total),
        "quant_ms": statistics.median(tq) * 1e3,
        "matmul_ms": statistics.median(tm) * 1e3,
        "total_ms": med * 1e3,
        "tflops": 2.0 * M * N * K / med / 1e12,
        "sample": f"X bf16 [{M},{K}] ~N(0,1) per-token E4M3FN quant + dequant matmul with W [{N},{K}] ~N(0,0.02) "
                  f"per-channel E4M3FN, fp32, bf16 out; median of {len(total)} reps",
    }
