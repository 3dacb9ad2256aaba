"""Pin the oracle's fused quantizers (RMSNorm + 1x128 FP8 / MXFP4, SwiGLU +
FP8) on the CPU.

RMSNorm: against an fp64 restatement of the formula in the reference's
test_parity.py (x / sqrt(mean(x^2) + eps) * w) through independent decoders
(torch.float8_e4m3fn, the E2M1 value table), against exact known answers
(constant rows: rms = |c|), and the quantization half against the pinned
1x128 quantizer. SwiGLU: against torch's silu in fp64 and torch's E4M3FN
encoder.
"""
import math

import numpy as np
import pytest
import torch

E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def bf16_bits(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def bits_f64(b):
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def e4m3_decode(c):
    return torch.from_numpy(np.ascontiguousarray(c, np.uint8)).view(torch.float8_e4m3fn).float().numpy().astype(np.float64)


def e4m3_encode(v):
    return torch.from_numpy(np.ascontiguousarray(v, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def rms_ref(xb, wb, eps):
    x, w = bits_f64(xb), bits_f64(wb)
    return x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + eps) * w[None, :]


@pytest.mark.parametrize("M,D", [(8, 128), (16, 1024), (4, 4096), (3, 5120), (2, 8192)])
def test_rmsnorm_fp8_against_fp64(orc, M, D):
    xb = orc.randn_bf16((M, D), seed=D)
    wb = orc.randn_bf16((D,), seed=D + 1)
    xb[0, : D // 2] = bf16_bits(np.linspace(-30, 30, D // 2))  # wide range in one row
    eps = 1e-6
    q, s = orc.rmsnorm_quant(xb, wb, eps, 0)
    y = rms_ref(xb, wb, eps)
    amax = np.abs(y).reshape(M, D // 128, 128).max(2)
    assert np.allclose(s, amax / 448.0, rtol=1e-6, atol=0)
    deq = e4m3_decode(q).reshape(M, D // 128, 128) * s[:, :, None].astype(np.float64)
    yg = y.reshape(M, D // 128, 128)
    # E4M3: half an ulp is 2^-4 relative for normals, 2^-10 absolute (x scale) for subnormals
    bound = np.maximum(np.abs(yg) * 2.0 ** -4, s[:, :, None] * 2.0 ** -10) * (1 + 1e-5) + 1e-30
    assert np.all(np.abs(deq - yg) <= bound)


@pytest.mark.parametrize("M,D", [(8, 128), (4, 4096), (2, 8192), (5, 800)])
def test_rmsnorm_mxfp4_against_fp64(orc, M, D):
    xb = orc.randn_bf16((M, D), seed=3 * D)
    wb = orc.randn_bf16((D,), seed=3 * D + 1)
    eps = 1e-5
    q, s = orc.rmsnorm_quant(xb, wb, eps, 1)
    y = rms_ref(xb, wb, eps).reshape(M, D // 32, 32)
    e = s.astype(np.int64) - 127
    lo, hi = q & 0xF, q >> 4
    codes = np.stack([lo, hi], axis=-1).reshape(M, D // 32, 32)
    vals = E2M1[codes & 7] * np.where(codes & 8, -1.0, 1.0)
    t = y * 2.0 ** (-e[:, :, None].astype(np.float64))
    # each code is a nearest grid point of y * 2^-e (fp32 y vs fp64: ties may go either way)
    dist = np.abs(np.abs(t)[..., None] - E2M1[None, None, None, :]).min(-1)
    assert np.all(np.abs(np.abs(t) - np.abs(vals)) <= dist + 1e-5 * np.abs(t) + 1e-30)
    assert np.all((np.sign(vals) == np.sign(t)) | (vals == 0))
    # the shared exponent puts the block maximum in [4, 8) (above 6 saturates to 6)
    m = np.abs(t).max(-1)
    assert np.all((m < 8.0) & ((m >= 3.5) | (np.abs(y).max(-1) == 0)))


@pytest.mark.parametrize("M,D", [(8, 4096), (5, 8192), (3, 160)])
def test_rmsnorm_mxfp4_floor_against_fp64(orc, M, D):
    """kind 2 (the reference module's element rule): the scales of kind 1, and
    each code the largest grid magnitude at or below |y * 2^-e| of the fp64
    RMSNorm (values within 1e-5 of a grid point may fall either side)."""
    xb = orc.randn_bf16((M, D), seed=5 * D)
    wb = orc.randn_bf16((D,), seed=5 * D + 1)
    eps = 1e-5
    q, s = orc.rmsnorm_quant(xb, wb, eps, 2)
    _, s1 = orc.rmsnorm_quant(xb, wb, eps, 1)
    assert np.array_equal(s, s1)
    y = rms_ref(xb, wb, eps).reshape(M, D // 32, 32)
    t = y * 2.0 ** (-(s.astype(np.int64) - 127)[:, :, None].astype(np.float64))
    codes = np.stack([q & 0xF, q >> 4], axis=-1).reshape(M, D // 32, 32)
    got = E2M1[codes & 7]
    idx = np.searchsorted(E2M1, np.abs(t), side="right") - 1
    want = E2M1[np.clip(idx, 0, 7)]
    near = np.abs(np.abs(t)[..., None] - E2M1[None, None, None, :]).min(-1) <= 1e-5 * np.maximum(np.abs(t), 1e-30)
    assert np.all((got == want) | near)
    assert np.all(((codes & 8) != 0) == np.signbit(t))


@pytest.mark.parametrize("kind", [0, 1])
def test_rmsnorm_constant_rows_known_answer(orc, kind):
    """x = c (a power of two) in every column, eps = 0: sum(x^2) = D c^2 exactly,
    r = 1/|c|, y = sign(c) * w; the result is the plain quantizer of +-w."""
    D = 4096
    wb = orc.randn_bf16((D,), seed=77)
    xb = np.stack([np.full(D, v, np.uint16) for v in bf16_bits(np.array([0.5, -4.0, 2.0 ** -10, 1.0]))])
    q, s = orc.rmsnorm_quant(xb, wb, 0.0, kind)
    signs = np.array([1, -1, 1, 1])
    wsig = np.stack([wb if sg > 0 else wb ^ np.uint16(0x8000) for sg in signs])
    if kind == 0:
        q2, s2 = orc.quant_rowwise(wsig, 128, "fp8")
    else:
        q2, s2 = orc.mx_quant_fp4(wsig)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


def test_rmsnorm_sum_order_close_to_fsum(orc):
    """The fixed-order fp32 sum of squares is within fp32 rounding of the exact sum:
    checked through r on a row whose y is exactly representable."""
    D = 8192
    xb = orc.randn_bf16((1, D), seed=5)
    x = bits_f64(xb[0])
    exact = math.fsum(x * x)
    # w = 1: amax(y) over the first group relative to amax(x) gives r
    wb = np.full(D, 0x3F80, np.uint16)
    _, s = orc.rmsnorm_quant(xb, wb, 0.0, 0)
    r = (s[0, 0] * 448.0) / np.abs(x[:128]).max()
    assert abs(r - 1.0 / math.sqrt(exact / D)) <= 1e-6 / math.sqrt(exact / D)


@pytest.mark.parametrize("interleaved", [False, True])
@pytest.mark.parametrize("group", [0, 128])
@pytest.mark.parametrize("alpha", [1.0, 1.702])
def test_swiglu_quant_against_torch(orc, interleaved, group, alpha):
    M, F = 6, 1024
    yb = orc.randn_bf16((M, 2 * F), seed=F + group)
    q, s, act = orc.swiglu_quant(yb, alpha, interleaved, group)
    y = torch.from_numpy(bits_f64(yb))
    g, u = (y[:, 0::2], y[:, 1::2]) if interleaved else (y[:, :F], y[:, F:])
    ref = (g * torch.sigmoid(alpha * g) * u).numpy()
    assert np.allclose(act, ref, rtol=2e-6, atol=1e-30)
    G = F if group == 0 else group
    a32 = act.reshape(M, F // G, G)
    sc = np.maximum(np.abs(a32).max(-1) / np.float32(448.0), np.float32(1e-10)).astype(np.float32)
    assert np.array_equal(s.reshape(M, -1), sc)
    rc = (np.float32(1.0) / sc).astype(np.float32)
    codes = e4m3_encode(np.clip((a32 * rc[:, :, None]).astype(np.float32), -448, 448)).reshape(M, F)
    assert np.array_equal(q, codes)


def test_swiglu_interleaved_is_a_column_permutation(orc):
    M, F = 4, 512
    yb = orc.randn_bf16((M, 2 * F), seed=9)
    inter = np.empty_like(yb)
    inter[:, 0::2], inter[:, 1::2] = yb[:, :F], yb[:, F:]
    a = orc.swiglu_quant(yb, 1.0, False, 0)
    b = orc.swiglu_quant(inter, 1.0, True, 0)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
