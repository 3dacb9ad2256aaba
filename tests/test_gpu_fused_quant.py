"""GPU parity of the fused quantizers against the CPU oracle, through the C ABI
and the reference-named modules.

RMSNorm + 1x128 FP8 / MXFP4 (nearest and the reference module's floor ladder):
codes and scales bit-exact (the reduction order, sqrt and division are fixed,
so nothing is left to rounding luck).
SwiGLU + FP8: the activation uses the device exp2 and reciprocal, so codes may
differ from the oracle's by one E4M3 step where the activation sits at a
rounding boundary; scales within 4 fp32 ulp; at least 99.9% of codes equal.
"""
import numpy as np
import pytest
import torch

import hkq
from gpu_util import assert_gemm_close, dev_bf16, dev_f32, dev_u8, host_bf16_bits, host_u8, require_gpu

pytestmark = pytest.mark.gpu


def rms_inputs(orc, M, D, seed):
    xb = orc.randn_bf16((M, D), seed=seed)
    wb = orc.randn_bf16((D,), seed=seed + 1)
    if M > 2:
        xb[1, :] = 0                                                              # all-zero row: r = 1/sqrt(eps)
        xb[2, : D // 2] = (np.linspace(-60, 60, D // 2).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    return xb, wb


# FP8 1x128 (kind 0) needs D % 128 == 0, MXFP4 (kinds 1, 2) D % 32 == 0: only
# valid combinations are generated
RMS_SHAPES = [(1, 128), (7, 1024), (256, 4096), (33, 5120), (64, 7168), (130, 8192), (5, 2080)]


@pytest.mark.parametrize("kind,M,D", [(k, M, D) for k in (0, 1, 2) for (M, D) in RMS_SHAPES
                                      if D % (128 if k == 0 else 32) == 0])
def test_rmsnorm_quant_bitexact(orc, kind, M, D):
    require_gpu()
    xb, wb = rms_inputs(orc, M, D, M + D + kind)
    eps = 1e-6
    q, s = hkq.rmsnorm_quant(dev_bf16(xb), dev_bf16(wb), eps, kind)
    torch.cuda.synchronize()
    oq, os_ = orc.rmsnorm_quant(xb, wb, eps, kind)
    assert np.array_equal(host_u8(q), oq)
    if kind == 0:
        assert np.array_equal(s.cpu().numpy().view(np.uint32), os_.view(np.uint32))
    else:
        assert np.array_equal(host_u8(s), os_)


def test_rmsnorm_mxfp4_floor_differs_from_nearest(orc):
    """The two MXFP4 element rules share scales and differ on codes: the floor
    ladder never rounds a magnitude up, so |floor code| <= |nearest code|."""
    require_gpu()
    M, D = 64, 4096
    xb, wb = rms_inputs(orc, M, D, 11)
    x, w = dev_bf16(xb), dev_bf16(wb)
    qn, sn = hkq.rmsnorm_quant(x, w, 1e-6, 1)
    qf, sf = hkq.rmsnorm_quant(x, w, 1e-6, 2)
    torch.cuda.synchronize()
    assert np.array_equal(host_u8(sn), host_u8(sf))
    a, b = host_u8(qn), host_u8(qf)
    na = np.stack([a & 0xF, a >> 4]) & 7
    nb = np.stack([b & 0xF, b >> 4]) & 7
    assert np.all(nb <= na) and np.any(nb < na)


def test_rmsnorm_quant_strided_rows(orc):
    """Input, code and scale rows with padding (ldx, ldq, lds past the row)."""
    require_gpu()
    M, D = 40, 1024
    xb, wb = rms_inputs(orc, M, D, 3)
    xpad = np.zeros((M, D + 64), np.uint16)
    xpad[:, :D] = xb
    x = dev_bf16(xpad)
    q = torch.full((M, D + 32), 0x5A, dtype=torch.uint8, device="cuda")
    s = torch.full((M, D // 128 + 3), -1.0, dtype=torch.float32, device="cuda")
    hkq.call("hkq_rmsnorm_quant", x.data_ptr(), dev_bf16(wb).data_ptr(), q.data_ptr(), s.data_ptr(), M, D, D + 64,
             D + 32, D // 128 + 3, 1e-6, 0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    oq, os_ = orc.rmsnorm_quant(xb, wb, 1e-6, 0)
    qh, sh = host_u8(q), s.cpu().numpy()
    assert np.array_equal(qh[:, :D], oq) and np.all(qh[:, D:] == 0x5A)
    assert np.array_equal(sh[:, : D // 128], os_) and np.all(sh[:, D // 128:] == -1.0)


@pytest.mark.parametrize("kind", [0, 1, 2])
def test_rmsnorm_quant_special_values(orc, kind):
    """Rows and weights that drive the group scale to its edges, bit-exact
    against the oracle: a row holding +inf (the norm's r becomes 0, the inf
    element NaN), a row holding NaN, weights near the bf16 maximum (y
    overflows to +-inf: amax = inf, FP8 scale inf, reciprocal 0), weights near
    the bf16 minimum normal (FP8 scale floored at 1e-10) and a weight group
    whose amax / 448 lies around the 1e-10 floor."""
    require_gpu()
    M, D = 12, 2048
    xb, wb = rms_inputs(orc, M, D, 77)
    xb[3, 17] = 0x7F80                                          # +inf
    xb[4, 300] = 0x7FC1                                         # NaN
    xb[5, 1000] = 0xFF80                                        # -inf
    wf = orc.bf16_bits_to_f32(wb).copy()
    wf[0:128] = np.sign(wf[0:128]) * 3.0e38                     # y overflows in the first FP8 group
    wf[128:256] *= 1e-36                                        # amax / 448 far below 1e-10
    wf[256:384] = np.sign(wf[256:384]) * np.geomspace(5e-9, 3e-8, 128)  # amax / 448 at 1.0-1.5e-10
    wf[384:416] = 0.0                                           # a zero MXFP4 block
    wb = orc.f32_to_bf16_bits(wf.astype(np.float32))
    eps = 1e-6
    q, s = hkq.rmsnorm_quant(dev_bf16(xb), dev_bf16(wb), eps, kind)
    torch.cuda.synchronize()
    oq, os_ = orc.rmsnorm_quant(xb, wb, eps, kind)
    assert np.array_equal(host_u8(q), oq)
    if kind == 0:
        sh = s.cpu().numpy()
        assert np.isinf(os_[:, 0]).any() and (os_ == np.float32(1e-10)).any()  # both scale edges are reached
        assert np.array_equal(sh.view(np.uint32), os_.view(np.uint32))
    else:
        assert np.array_equal(host_u8(s), os_)


@pytest.mark.parametrize("kind", [0, 1])
def test_fused_rmsnorm_modules_reference_call(orc, kind):
    """tests/test_misc.py:552-601 of the reference as written: M=256, N=4096,
    eps=1e-6, randn bf16 input and weight (seed 42), uint8 outputs."""
    require_gpu()
    import hipkittens as hk
    M, N, eps = 256, 4096, 1e-6
    torch.manual_seed(42)
    x = torch.randn(M, N, dtype=torch.bfloat16)
    weight = torch.randn(N, dtype=torch.bfloat16)
    xb, wb = x.view(torch.int16).numpy().view(np.uint16), weight.view(torch.int16).numpy().view(np.uint16)
    if kind == 0:
        out = torch.zeros(M, N, dtype=torch.uint8, device="cuda")
        scales = torch.zeros(M, N // 128, dtype=torch.float32, device="cuda")
        hk.fused_rmsnorm_fp8_quant_fwd(x.cuda(), weight.cuda(), out, scales, eps)
    else:
        out = torch.zeros(M, N // 2, dtype=torch.uint8, device="cuda")
        scales = torch.zeros(M, N // 32, dtype=torch.uint8, device="cuda")
        hk.fused_rmsnorm_mxfp4_quant_fwd(x.cuda(), weight.cuda(), out, scales, eps)
    torch.cuda.synchronize()
    # the module keeps the reference's floor ladder for MXFP4 elements (kind 2)
    oq, os_ = orc.rmsnorm_quant(xb, wb, eps, 2 if kind else 0)
    assert (out != 0).sum().item() > 0  # the reference test's own check
    assert np.array_equal(host_u8(out), oq)
    assert np.array_equal(scales.cpu().numpy().view(np.uint8 if kind else np.uint32), os_.view(np.uint8 if kind else np.uint32))


def e4m3_step_diff(a, b):
    """Distance in E4M3 steps between code arrays of equal sign (inf where signs differ)."""
    sa, sb = a >> 7, b >> 7
    ma, mb = (a & 0x7F).astype(np.int32), (b & 0x7F).astype(np.int32)
    d = np.abs(ma - mb)
    return np.where((sa == sb) | ((ma == 0) & (mb == 0)), d, np.where(ma + mb <= 1, 1, 99))


# 1x128 groups need F % 128 == 0: only valid combinations are generated
SWIGLU_SHAPES = [(1, 128, 1.0), (64, 14336, 1.0), (300, 1024, 1.702), (17, 6144, 1.0), (8, 32768, 1.0), (40, 200, 1.0)]


@pytest.mark.parametrize("interleaved", [False, True])
@pytest.mark.parametrize("group,M,F,alpha", [(g, M, F, a) for g in (0, 128) for (M, F, a) in SWIGLU_SHAPES
                                             if g == 0 or F % g == 0])
def test_swiglu_quant(orc, interleaved, group, M, F, alpha):
    require_gpu()
    yb = orc.randn_bf16((M, 2 * F), seed=M + F + group)
    q, s = hkq.swiglu_quant(dev_bf16(yb), alpha, interleaved, group)
    torch.cuda.synchronize()
    oq, os_, act = orc.swiglu_quant(yb, alpha, interleaved, group)
    gs = s.cpu().numpy()
    assert np.all(np.abs(gs.view(np.int32).astype(np.int64) - os_.view(np.int32).astype(np.int64)) <= 4)
    d = e4m3_step_diff(host_u8(q), oq)
    assert d.max() <= 1
    assert (d == 0).mean() >= 0.999


def test_swiglu_module_call(orc):
    require_gpu()
    import hipkittens as hk
    M, F = 128, 2048
    yb = orc.randn_bf16((M, 2 * F), seed=21)
    out = torch.empty(M, F, dtype=torch.float8_e4m3fn, device="cuda")
    sc = torch.empty(M, 1, dtype=torch.float32, device="cuda")
    hk.swiglu_quant_fwd(dev_bf16(yb), out, sc)
    q, s = hkq.swiglu_quant(dev_bf16(yb))
    torch.cuda.synchronize()
    assert np.array_equal(host_u8(out), host_u8(q))
    assert torch.equal(sc.view(-1), s)


def test_moe_layer_chain(orc):
    """Router logits -> GPU routing -> gate/up MoE GEMM -> SwiGLU + per-token FP8
    -> down MoE GEMM (rows in expert-sorted order, no gather): the down output
    matches the fp64 reference of the down GEMM on the oracle's requantization
    of the GPU gate/up output."""
    require_gpu()
    T, E, K, H, F = 512, 8, 2, 256, 512
    logits = orc.randn_bf16((T, E), seed=31)
    r = hkq.moe_routing(dev_bf16(logits), K, 128)
    X, xs = orc.quant_rowwise(orc.randn_bf16((T, H), seed=32), None, "fp8")
    W1, ws1 = orc.quant_rowwise(orc.randn_bf16((E * 2 * F, H), seed=33, std=0.05), None, "fp8")
    W2, ws2 = orc.quant_rowwise(orc.randn_bf16((E * H, F), seed=34, std=0.05), None, "fp8")
    Y1 = hkq.moe_a8w8(dev_u8(X).view(torch.float8_e4m3fn), dev_u8(W1.reshape(E, 2 * F, H)).view(torch.float8_e4m3fn),
                      r["hist"], r["offs"], r["expt_data"], K, gather=r["gather"], x_scale=dev_f32(xs.reshape(-1)),
                      w_scale=dev_f32(ws1.reshape(E, 2 * F)))
    q2, s2 = hkq.swiglu_quant(Y1)
    Y2 = hkq.moe_a8w8(q2, dev_u8(W2.reshape(E, H, F)).view(torch.float8_e4m3fn), r["hist"], r["offs"],
                      r["expt_data"], 1, gather=None, x_scale=s2, w_scale=dev_f32(ws2.reshape(E, H)))
    torch.cuda.synchronize()
    y1b = host_bf16_bits(Y1)
    oq, os_, _ = orc.swiglu_quant(y1b)
    d = e4m3_step_diff(host_u8(q2), oq)
    assert d.max() <= 1 and (d == 0).mean() >= 0.999
    hist = r["hist"].cpu().numpy()
    offs = r["offs"].cpu().numpy()
    ed = r["expt_data"].cpu().numpy()
    ed = ed[ed != -1]
    ref = orc.moe_ref(host_u8(q2), W2.reshape(E, H, F), s2.cpu().numpy(), ws2.reshape(E, H), None,
                      np.arange(T * K), hist, offs, ed, 1, w_layout="enk")
    assert_gemm_close(Y2.float().cpu().numpy(), ref, "down projection")
