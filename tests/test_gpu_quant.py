"""GPU parity of the quantizers against the CPU oracle, through the C ABI.

Bar: bit-exact codes and scales (integer/byte work). Inputs are seeded on the
CPU and copied, so both sides see identical bf16 bytes. Edge rows cover what
the reference kernels meet: all-zero rows/blocks, bf16 subnormals, extreme
dynamic range, +-inf and NaN, M = 1, ragged K, and BASELINE sizes.
"""
import numpy as np
import pytest
import torch

import hkq
from gpu_util import dev_bf16, dev_f32, dev_u8, host_bf16_bits, host_u8, require_gpu

pytestmark = pytest.mark.gpu


def edge_rows(orc, xb):
    """Overwrite the first rows of xb (uint16 [M, K]) with edge cases."""
    M, K = xb.shape
    rows = [
        np.zeros(K, np.float32),
        (np.arange(K, dtype=np.float32) - K / 2) * 1e-40,                 # bf16 subnormals
        np.linspace(-3e4, 3e4, K, dtype=np.float32),                     # wide range
        np.where(np.arange(K) % 7 == 0, np.float32(1e-30), np.float32(2.5e3)),
    ]
    for i, r in enumerate(rows[:M]):
        xb[i] = orc.f32_to_bf16_bits(r.astype(np.float32))
    if M > 4:
        xb[4, 3] = 0x7F80   # +inf
        xb[4, 5] = 0xFF80   # -inf
    if M > 5:
        xb[5, 1] = 0x7FC1   # NaN
        xb[5, 2] = 0xFFC3   # -NaN
    return xb


QUANT_SHAPES = [(1, 8), (3, 24), (7, 4096), (16, 4096), (128, 1024), (333, 2048), (64, 8192), (9, 14336),
                (5, 18432), (2, 32768)]


@pytest.mark.parametrize("kind", ["fp8", "int8"])
@pytest.mark.parametrize("M,K", QUANT_SHAPES)
def test_per_token_quant(orc, kind, M, K):
    require_gpu()
    xb = edge_rows(orc, orc.randn_bf16((M, K), seed=M * 131 + K))
    q, s = hkq.per_token_quant(dev_bf16(xb), hkq.KIND_FP8 if kind == "fp8" else hkq.KIND_INT8)
    torch.cuda.synchronize()
    qo, so = orc.quant_rowwise(xb, None, kind)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.reshape(-1).view(np.uint32))
    assert np.array_equal(host_u8(q), qo)


def test_per_token_quant_strided_rows(orc):
    require_gpu()
    M, K, ld = 33, 1024, 1536
    xb = orc.randn_bf16((M, ld), seed=3)
    x = dev_bf16(xb)[:, :K]
    q = torch.full((M, ld), 0xAB, dtype=torch.uint8, device="cuda")
    s = torch.empty(M, device="cuda")
    hkq.call("hkq_per_token_quant", x.data_ptr(), q.data_ptr(), s.data_ptr(), M, K, ld, ld, hkq.KIND_FP8,
             torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    qo, so = orc.quant_rowwise(np.ascontiguousarray(xb[:, :K]), None, "fp8")
    qh = q.cpu().numpy()
    assert np.array_equal(qh[:, :K], qo) and np.all(qh[:, K:] == 0xAB)
    assert np.array_equal(s.cpu().numpy(), so.reshape(-1))


def test_e4m3_encoder_every_bf16_value(orc):
    """Rows [448, v_1 .. v_4095]: amax 448 gives s = 1, r = 1, so each code is
    E4M3FN(v) for every finite bf16 value |v| <= 448."""
    require_gpu()
    bits = np.arange(1 << 16, dtype=np.uint32)
    v = (bits << 16).view(np.float32)
    v = v[np.isfinite(v) & (np.abs(v) <= 448.0)]
    per = 4095
    n_rows = (len(v) + per - 1) // per
    vals = np.zeros(n_rows * per, np.float32)
    vals[: len(v)] = v
    rows = np.concatenate([np.full((n_rows, 1), 448.0, np.float32), vals.reshape(n_rows, per)], axis=1)
    xb = orc.f32_to_bf16_bits(rows)
    q, s = hkq.per_token_quant(dev_bf16(xb), hkq.KIND_FP8)
    torch.cuda.synchronize()
    assert np.all(s.cpu().numpy() == 1.0)
    ref = torch.from_numpy(rows).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(host_u8(q), ref)


@pytest.mark.parametrize("group", [32, 64, 128, 256, 512])
@pytest.mark.parametrize("kind", ["fp8", "int8"])
def test_group_quant(orc, group, kind):
    require_gpu()
    M, K = 37, 2048
    xb = edge_rows(orc, orc.randn_bf16((M, K), seed=group))
    q, s = hkq.group_quant(dev_bf16(xb), group, hkq.KIND_FP8 if kind == "fp8" else hkq.KIND_INT8)
    torch.cuda.synchronize()
    qo, so = orc.quant_rowwise(xb, group, kind)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))
    assert np.array_equal(host_u8(q), qo)


@pytest.mark.parametrize("M,K", [(2048, 1536), (2048, 18432), (1, 128)])
def test_group_quant_1x128_blockscale_shapes(orc, M, K):
    require_gpu()
    xb = orc.randn_bf16((M, K), seed=K)
    q, s = hkq.group_quant(dev_bf16(xb), 128, hkq.KIND_FP8)
    torch.cuda.synchronize()
    qo, so = orc.quant_rowwise(xb, 128, "fp8")
    assert np.array_equal(s.cpu().numpy(), so) and np.array_equal(host_u8(q), qo)


@pytest.mark.parametrize("K", [524288 - 128, 524288, 524288 + 1024])
def test_group_and_mx_quant_wide_rows(orc, K):
    """Rows of about 2^19 elements: from K / 8 = 2^16 chunks per row the
    kernels take a chunk's row from a 64-bit division instead of the double
    reciprocal (which needs fewer than 2^16 chunks per row); both sides of the
    switch, and rows that end inside a workgroup's chunks."""
    require_gpu()
    M = 3
    xb = orc.randn_bf16((M, K), seed=K % 1000)
    q, s = hkq.group_quant(dev_bf16(xb), 128, hkq.KIND_FP8)
    q4, s4 = hkq.mx_quant(dev_bf16(xb), True)
    torch.cuda.synchronize()
    qo, so = orc.quant_rowwise(xb, 128, "fp8")
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32)) and np.array_equal(host_u8(q), qo)
    qo4, so4 = orc.mx_quant_fp4(xb)
    assert np.array_equal(host_u8(s4), so4) and np.array_equal(host_u8(q4), qo4)


def mx_edge(orc, xb):
    xb[0, :32] = 0                                                               # zero block -> code 0
    xb[0, 32:64] = orc.f32_to_bf16_bits(np.full(32, 7.0, np.float32))          # amax rounds up
    xb[1, :32] = orc.f32_to_bf16_bits(np.linspace(-1e-38, 1e-38, 32).astype(np.float32))
    xb[1, 32:64] = orc.f32_to_bf16_bits(np.linspace(-3e38, 3e38, 32).astype(np.float32))
    xb[2, 5] = 0xFF80                                                           # -inf
    xb[2, 40] = 0x7F80                                                          # +inf
    ties = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0] * 4, np.float32)  # amax 6 -> scale 2^0
    xb[3, :32] = orc.f32_to_bf16_bits(ties * np.where(np.arange(32) % 2, -1, 1))
    return xb


@pytest.mark.parametrize("M,K", [(4, 64), (37, 1024), (128, 8192), (4096, 8192)])
def test_mx_quant_fp4(orc, M, K):
    require_gpu()
    xb = mx_edge(orc, orc.randn_bf16((M, K), seed=M + K))
    q, s = hkq.mx_quant(dev_bf16(xb), True)
    torch.cuda.synchronize()
    qo, so = orc.mx_quant_fp4(xb)
    assert np.array_equal(host_u8(s), so)
    assert np.array_equal(host_u8(q), qo)


@pytest.mark.parametrize("M,K", [(4, 64), (37, 1024), (256, 4096)])
def test_mx_quant_fp8(orc, M, K):
    require_gpu()
    xb = mx_edge(orc, orc.randn_bf16((M, K), seed=M * 3 + K))
    q, s = hkq.mx_quant(dev_bf16(xb), False)
    torch.cuda.synchronize()
    qo, so = orc.mx_quant_fp8(xb)
    assert np.array_equal(host_u8(s), so)
    assert np.array_equal(host_u8(q), qo)


@pytest.mark.parametrize("is_fp4", [True, False])
def test_mx_dequant_all_codes(orc, is_fp4):
    """Every element byte and every scale byte (0 and 0xFF included)."""
    require_gpu()
    M, K = 256, 512
    rng = np.random.default_rng(5 + is_fp4)
    q = rng.integers(0, 256, (M, K // 2 if is_fp4 else K), dtype=np.uint8)
    q[0, : q.shape[1]] = np.arange(q.shape[1]) % 256
    s = rng.integers(0, 256, (M, K // 32), dtype=np.uint8)
    s[:, 0] = np.arange(M) % 256
    out = hkq.mx_dequant(dev_u8(q), dev_u8(s), K, is_fp4)
    torch.cuda.synchronize()
    ref = orc.mx_dequant(q, s, M, K, is_fp4)
    got = host_bf16_bits(out)
    nan_ref = (ref & 0x7FFF) > 0x7F80
    nan_got = (got & 0x7FFF) > 0x7F80
    assert np.array_equal(nan_ref, nan_got)
    assert np.array_equal(got[~nan_ref], ref[~nan_ref])


def test_static_fp8(orc):
    require_gpu()
    xb = edge_rows(orc, orc.randn_bf16((64, 4096), seed=9, std=100.0))
    for scale in (0.5, 0.37, 3.0, 1e-3):
        y = hkq.static_quant_fp8(dev_bf16(xb), dev_f32(np.array([scale], np.float32)))
        torch.cuda.synchronize()
        assert np.array_equal(host_u8(y), orc.quant_static_fp8(xb, scale)), scale


def test_per_token_quant_baseline_size(orc):
    """BASELINE quantizer size: bf16 [4096, 4096], full comparison."""
    require_gpu()
    xb = orc.randn_bf16((4096, 4096), seed=1)
    q, s = hkq.per_token_quant(dev_bf16(xb), hkq.KIND_FP8)
    torch.cuda.synchronize()
    qo, so = orc.quant_rowwise(xb, None, "fp8")
    assert np.array_equal(s.cpu().numpy(), so.reshape(-1)) and np.array_equal(host_u8(q), qo)
