"""hkq_gemm_a8w8_noalloc (split-K partials in the library's own device scratch)
against hkq_gemm_a8w8_ws (the same plan on a caller workspace), through the C
ABI: two calls in a row, the second with a smaller input, each bit-exact with
the workspace entry point and within the GEMM tolerance of the oracle."""
import numpy as np
import pytest
import torch

import hkq
from gpu_util import assert_gemm_close, dev_f32, dev_u8, host_bf16_f32, require_gpu

pytestmark = pytest.mark.gpu


def _inputs(orc, M, N, K, seed):
    A, sa = orc.quant_rowwise(orc.randn_bf16((M, K), seed=seed), None, "fp8")
    B, sb = orc.quant_rowwise(orc.randn_bf16((N, K), seed=seed + 1, std=0.02), None, "fp8")
    return A, B, sa.reshape(-1), sb.reshape(-1)


def _run(name, A, B, sa, sb, M, N, K, ws=None):
    Ad, Bd, sad, sbd = dev_u8(A), dev_u8(B), dev_f32(sa), dev_f32(sb)
    C = torch.full((M, N), 3.0, dtype=torch.bfloat16, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    args = [Ad.data_ptr(), Bd.data_ptr(), sad.data_ptr(), sbd.data_ptr(), C.data_ptr(), M, N, K, K, K, N]
    if ws is None:
        hkq.call(name, *args, stream)
    else:
        hkq.call(name, *args, ws.data_ptr(), ws.numel(), stream)
    torch.cuda.synchronize()
    return C


def test_gemm_a8w8_noalloc_matches_workspace_entry(orc):
    require_gpu()
    L = hkq.lib()
    cap = L.hkq_gemm_a8w8_noalloc_max_workspace()
    # a split-K plan with a large workspace, then a smaller split shape
    for (M, N, K) in ((128, 4096, 14336), (64, 2048, 4096)):
        need = L.hkq_gemm_a8w8_workspace(M, N, K)
        assert 0 < need <= cap, (M, N, K, need)
        A, B, sa, sb = _inputs(orc, M, N, K, seed=M + N)
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        ref = _run("hkq_gemm_a8w8_ws", A, B, sa, sb, M, N, K, ws)
        got = _run("hkq_gemm_a8w8_noalloc", A, B, sa, sb, M, N, K)
        assert torch.equal(got, ref), f"{M}x{N}x{K}: noalloc differs from the workspace entry point"
        assert_gemm_close(host_bf16_f32(got), orc.gemm_a8w8_ref_f32(A, B, sa, sb), f"noalloc {M}x{N}x{K}")
