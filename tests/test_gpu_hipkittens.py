"""The hipkittens (pybind11) surface on the GPU: each reference-named entry
point gives the same bytes as the C-ABI call it forwards to, with the
reference's argument orders."""
import numpy as np
import pytest
import torch

import hkq
from gpu_util import dev_bf16, dev_f32, dev_u8, host_bf16_bits, host_u8, require_gpu

pytestmark = pytest.mark.gpu


def test_per_token_quant_fwd(orc):
    require_gpu()
    import hipkittens as hk

    xb = orc.randn_bf16((64, 4096), seed=2)
    x = dev_bf16(xb)
    for dt, kind in ((torch.int8, "int8"), (torch.float8_e4m3fn, "fp8"), (torch.uint8, "fp8")):
        out = torch.empty((64, 4096), dtype=dt, device="cuda")
        sc = torch.empty((64, 1), dtype=torch.float32, device="cuda")
        hk.per_token_quant_fwd(x, out, sc)
        torch.cuda.synchronize()
        qo, so = orc.quant_rowwise(xb, None, kind)
        assert np.array_equal(host_u8(out), qo) and np.array_equal(sc.cpu().numpy(), so)


def test_group_quant_fwd(orc):
    require_gpu()
    import hipkittens as hk

    xb = orc.randn_bf16((32, 2048), seed=3)
    out = torch.empty((32, 2048), dtype=torch.float8_e4m3fn, device="cuda")
    sc = torch.empty((32, 16), dtype=torch.float32, device="cuda")
    hk.group_quant_fwd(dev_bf16(xb), out, sc, group_size=128)
    torch.cuda.synchronize()
    qo, so = orc.quant_rowwise(xb, 128, "fp8")
    assert np.array_equal(host_u8(out), qo) and np.array_equal(sc.cpu().numpy(), so)


def test_gemm_dispatch_argument_orders(orc):
    require_gpu()
    import hipkittens as hk

    M, N, K = 256, 512, 1024
    A, sa = orc.quant_rowwise(orc.randn_bf16((M, K), seed=4), None, "fp8")
    B, sb = orc.quant_rowwise(orc.randn_bf16((N, K), seed=5, std=0.02), None, "fp8")
    Ad = dev_u8(A).view(torch.float8_e4m3fn)
    Bd = dev_u8(B).view(torch.float8_e4m3fn)
    sad, sbd = dev_f32(sa.reshape(-1)), dev_f32(sb.reshape(-1))
    ref = hkq.gemm_a8w8(Ad, Bd, sad, sbd)
    C1 = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    C2 = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    hk.gemm.a8w8.dispatch(Ad, Bd, sad, sbd, C1)                 # gemm_a8w8_tk: C last
    hk.gemm.a8w8_per_token.dispatch(Ad, Bd, C2, sad, sbd)       # per_token_scale_tk: C third
    torch.cuda.synchronize()
    assert torch.equal(C1, ref) and torch.equal(C2, ref)
    with pytest.raises(TypeError):
        hk.gemm.a8w8.dispatch(Ad.view(torch.uint8).to(torch.bfloat16), Bd, sad, sbd, C1)


def test_afp4wfp4_dispatch(orc):
    require_gpu()
    import hipkittens as hk

    M, N, K = 128, 256, 1024
    Aq, As = orc.mx_quant_fp4(orc.randn_bf16((M, K), seed=6))
    Bq, Bs = orc.mx_quant_fp4(orc.randn_bf16((N, K), seed=7, std=0.02))
    args = [dev_u8(a) for a in (Aq, As, Bq, Bs)]
    ref = hkq.gemm_mxfp4(*args)
    C = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    hk.gemm.afp4wfp4.dispatch(args[0], args[2], C, args[1], args[3])
    torch.cuda.synchronize()
    assert torch.equal(C, ref)


def test_quant_moe_module(orc):
    require_gpu()
    import hipkittens as hk

    M, K = 64, 1024
    xb = orc.randn_bf16((M, K), seed=8)
    x = dev_bf16(xb)
    qm = hk.moe_routing.quant
    for is_fp4 in (True, False):
        q = torch.empty((M, K // 2 if is_fp4 else K), dtype=torch.uint8, device="cuda")
        s = torch.empty((M, K // 32), dtype=torch.uint8, device="cuda")
        qm.downcast_to_mxfp(mx_tensor=q, mx_scale=s, src=x, outer_dim=M, quant_dim=K, is_fp4=is_fp4)
        out = torch.empty((M, K), dtype=torch.bfloat16, device="cuda")
        qm.upcast_from_mxfp(out, s, q, M, K, is_fp4)
        torch.cuda.synchronize()
        qo, so = orc.mx_quant_fp4(xb) if is_fp4 else orc.mx_quant_fp8(xb)
        assert np.array_equal(host_u8(q), qo) and np.array_equal(host_u8(s), so)
        assert np.array_equal(host_bf16_bits(out), orc.mx_dequant(qo, so, M, K, is_fp4))
    y = torch.empty((M, K), dtype=torch.uint8, device="cuda")
    qm.downcast_to_static_fp8(x, y, dev_f32(np.array([0.25], np.float32)), M, K)
    torch.cuda.synchronize()
    assert np.array_equal(host_u8(y), orc.quant_static_fp8(xb, 0.25))


def test_blockscale_dispatch(orc):
    require_gpu()
    import hipkittens as hk

    M, N, K = 128, 256, 512
    A, sa = orc.quant_rowwise(orc.randn_bf16((M, K), seed=9), 128, "fp8")
    B, sbr = orc.quant_rowwise(orc.randn_bf16((N, K), seed=10, std=0.02), 128, "fp8")
    sb = np.ascontiguousarray(sbr.T)  # [K/128, N]: the reference test's per-column layout
    Ad, Bd = dev_u8(A).view(torch.float8_e4m3fn), dev_u8(B).view(torch.float8_e4m3fn)
    sad, sbd = dev_f32(sa), dev_f32(sb)
    ref = hkq.gemm_blockscale(Ad, Bd, sad, sbd, group_n=1)
    C = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    hk.gemm.a8w8_blockscale.dispatch(Ad, Bd, C, sad, sbd)     # C third, as in the reference
    torch.cuda.synchronize()
    assert torch.equal(C, ref)
