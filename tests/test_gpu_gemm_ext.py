"""GPU parity of the batched and fused GEMM entry points against the CPU
oracle, through the C ABI and the reference-named modules:

- bf16 GEMM (gemm_a16w16_tk; tests/test_gemm.py:21-42 of the reference) and
  batched bf16 GEMM with bias (batched_gemm_bf16_tk; :316-347);
- batched A8W8 GEMM with per-token x per-channel scales and bias
  (batched_gemm_a8w8_tk; :349-390);
- block-scale FP8 GEMM with the multiply-add epilogue
  (fused_gemm_a8w8_blockscale_mul_add_tk; :498-533) and next to a bf16 GEMM
  (fused_gemm_a8w8_blockscale_a16w16_tk; :454-496).

Bar: the north-star GEMM tolerance (|C - ref| <= 2e-2 + 1e-2 |ref|, Frobenius
relative error < 1e-2) against the fp64 oracle on the same codes, scales and
bf16 values. The reference tests' own inputs are bf16 tensors; the FP8 paths
take their E4M3FN quantization (oracle quantizers), as the dense modules do.
"""
import numpy as np
import pytest
import torch

import hkq
from gpu_util import assert_gemm_close, dev_bf16, dev_f32, dev_u8, host_bf16_f32, require_gpu

pytestmark = pytest.mark.gpu


def fp8_rows(orc, shape, seed, std=1.0):
    """Per-row E4M3FN quantization of N(0, std) bf16 values: (codes, scales)."""
    x = orc.randn_bf16(shape, seed=seed, std=std).reshape(-1, shape[-1])
    q, s = orc.quant_rowwise(x, None, "fp8")
    return q.reshape(shape), s.reshape(shape[:-1])


# ---------------------------------------------------------------- bf16 GEMM

@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (1, 256, 512), (33, 100, 96), (300, 520, 384), (64, 512, 8192),
                                   (1000, 2056, 800), (512, 4096, 4096)])
def test_gemm_bf16(orc, M, N, K):
    require_gpu()
    A = orc.randn_bf16((M, K), seed=M + K)
    B = orc.randn_bf16((N, K), seed=N + K + 1, std=0.05)
    C = hkq.gemm_bf16(dev_bf16(A), dev_bf16(B))
    torch.cuda.synchronize()
    assert_gemm_close(host_bf16_f32(C), orc.gemm_bf16_ref(A, B), f"bf16 {M}x{N}x{K}")


def test_gemm_bf16_split_equals_unsplit(orc):
    """A grid small enough to split K (workspace plan) gives the same bits as the
    unsplit plan up to fp32 summation order: both within the bar, and close."""
    require_gpu()
    M, N, K = 32, 256, 16384
    A = orc.randn_bf16((M, K), seed=1)
    B = orc.randn_bf16((N, K), seed=2, std=0.05)
    C1 = host_bf16_f32(hkq.gemm_bf16(dev_bf16(A), dev_bf16(B), split=True))
    C2 = host_bf16_f32(hkq.gemm_bf16(dev_bf16(A), dev_bf16(B), split=False))
    ref = orc.gemm_bf16_ref(A, B)
    assert_gemm_close(C1, ref, "split")
    assert_gemm_close(C2, ref, "unsplit")


def test_gemm_bf16_identity_closed_form(orc):
    """B = I: C = A bit for bit (one product per sum, exact in fp32)."""
    require_gpu()
    M, K = 300, 256
    A = orc.randn_bf16((M, K), seed=3)
    eye = orc.f32_to_bf16_bits(np.eye(K, dtype=np.float32))
    C = hkq.gemm_bf16(dev_bf16(A), dev_bf16(eye))
    torch.cuda.synchronize()
    assert np.array_equal(C.view(torch.int16).cpu().numpy().view(np.uint16), A)


def test_gemm_a16w16_module_reference_call(orc):
    """tests/test_gemm.py:21-42 as written: M = N = K = 256, torch.randn bf16
    (seed 42), rel-err bar 0.02 of the reference plus the north-star bar."""
    require_gpu()
    import hipkittens as hk
    M, N, K = 256, 256, 256
    torch.manual_seed(42)
    A = torch.randn(M, K, dtype=torch.bfloat16, device="cuda")
    B = torch.randn(N, K, dtype=torch.bfloat16, device="cuda")
    C = torch.zeros(M, N, dtype=torch.bfloat16, device="cuda")
    hk.gemm.a16w16.dispatch(A, B, C)
    torch.cuda.synchronize()
    ref = orc.gemm_bf16_ref(A.view(torch.int16).cpu().numpy().view(np.uint16),
                            B.view(torch.int16).cpu().numpy().view(np.uint16))
    got = host_bf16_f32(C)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 0.02
    assert_gemm_close(got, ref, "a16w16 module")


@pytest.mark.parametrize("Z,M,N,K,bias", [(4, 128, 128, 128, True), (3, 300, 520, 384, True), (2, 64, 256, 1024, False),
                                          (5, 1, 128, 256, True)])
def test_batched_gemm_bf16(orc, Z, M, N, K, bias):
    require_gpu()
    A = orc.randn_bf16((Z, M, K), seed=Z + M)
    B = orc.randn_bf16((Z, N, K), seed=Z + N, std=0.05)
    bb = orc.randn_bf16((Z, N), seed=Z + K) if bias else None
    C = hkq.gemm_bf16(dev_bf16(A), dev_bf16(B), bias=dev_bf16(bb) if bias else None)
    torch.cuda.synchronize()
    got = host_bf16_f32(C)
    for z in range(Z):
        assert_gemm_close(got[z], orc.gemm_bf16_ref(A[z], B[z], bb[z] if bias else None), f"batch {z}")


def test_batched_gemm_bf16_module_reference_call(orc):
    """tests/test_gemm.py:316-347 as written: the (1, B, ., .) layout, bias
    (1, B, 1, N)."""
    require_gpu()
    import hipkittens as hk
    BATCH, M, N, K = 4, 128, 128, 128
    torch.manual_seed(42)
    A = torch.randn(BATCH, M, K, dtype=torch.bfloat16, device="cuda")
    B = torch.randn(BATCH, K, N, dtype=torch.bfloat16, device="cuda")
    bias = torch.randn(BATCH, 1, N, dtype=torch.bfloat16, device="cuda")
    A_hk = A.unsqueeze(0).contiguous()
    B_hk = B.transpose(-2, -1).unsqueeze(0).contiguous()
    C_hk = torch.zeros(1, BATCH, M, N, dtype=torch.bfloat16, device="cuda")
    hk.batched_gemm.bf16.dispatch(A_hk, B_hk, C_hk, bias.unsqueeze(0).contiguous())
    torch.cuda.synchronize()
    got = host_bf16_f32(C_hk.squeeze(0))
    bits = lambda t: t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    for z in range(BATCH):
        ref = orc.gemm_bf16_ref(bits(A[z]), bits(B[z].T), bits(bias[z, 0]))
        assert_gemm_close(got[z], ref, f"batch {z}")


# --------------------------------------------------------- batched A8W8

@pytest.mark.parametrize("Z,M,N,K,bias", [(4, 128, 128, 128, True), (3, 300, 516, 320, True), (2, 512, 1024, 2048, False),
                                          (6, 17, 64, 64, True), (1, 256, 256, 256, True), (5, 16, 200, 256, True),
                                          (3, 32, 96, 512, False)])
def test_batched_gemm_a8w8(orc, Z, M, N, K, bias):
    require_gpu()
    A, sa = fp8_rows(orc, (Z, M, K), seed=Z + M + K)
    B, sb = fp8_rows(orc, (Z, N, K), seed=Z + N, std=0.02)
    bb = orc.randn_bf16((Z, N), seed=K) if bias else None
    C = hkq.batched_gemm_a8w8(dev_u8(A), dev_u8(B), dev_f32(sa), dev_f32(sb), bias=dev_bf16(bb) if bias else None)
    torch.cuda.synchronize()
    ref = orc.batched_gemm_a8w8_ref(A, B, sa, sb, bb)
    got = host_bf16_f32(C)
    for z in range(Z):
        assert_gemm_close(got[z], ref[z], f"batch {z}")


@pytest.mark.parametrize("M,K", [(100, 192), (9, 256)])
def test_batched_gemm_a8w8_strided_batches(orc, M, K):
    """Batches placed with gaps (batch strides larger than the matrices), rows
    padded (lda, ldc > K, N): the bytes between batches stay untouched."""
    require_gpu()
    Z, N = 3, 136
    A, sa = fp8_rows(orc, (Z, M, K), seed=4)
    B, sb = fp8_rows(orc, (Z, N, K), seed=5, std=0.02)
    Ap = np.zeros((Z, M + 7, K + 64), np.uint8)
    Ap[:, :M, :K] = A
    Bp = np.zeros((Z, N + 3, K + 32), np.uint8)
    Bp[:, :N, :K] = B
    Cp = torch.full((Z, M + 5, N + 8), 3.0, dtype=torch.bfloat16, device="cuda")
    a, b = dev_u8(Ap), dev_u8(Bp)
    s_a, s_b = dev_f32(sa), dev_f32(sb)
    hkq.call("hkq_batched_gemm_a8w8", a.data_ptr(), b.data_ptr(), s_a.data_ptr(), s_b.data_ptr(), None,
             Cp.data_ptr(), Z, M, N, K, K + 64, K + 32, N + 8, (M + 7) * (K + 64), (N + 3) * (K + 32),
             (M + 5) * (N + 8), M, N, 0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got = host_bf16_f32(Cp)
    ref = orc.batched_gemm_a8w8_ref(A, B, sa, sb)
    for z in range(Z):
        assert_gemm_close(got[z, :M, :N], ref[z], f"batch {z}")
    assert np.all(got[:, M:, :] == 3.0) and np.all(got[:, :, N:] == 3.0)


def test_batched_gemm_a8w8_module_reference_call(orc):
    """tests/test_gemm.py:349-390: the (1, B, ., .) layout, a_scale (1, B, 1, M),
    b_scale (1, B, 1, N), bias (1, B, 1, N); A and B as E4M3FN codes (the
    reference passes bf16 tensors holding int8 values, which this build
    rejects with TypeError)."""
    require_gpu()
    import hipkittens as hk
    BATCH, M, N, K = 4, 128, 128, 128
    A, sa = fp8_rows(orc, (BATCH, M, K), seed=42)
    B, sb = fp8_rows(orc, (BATCH, N, K), seed=43, std=0.02)
    bias = orc.randn_bf16((BATCH, N), seed=44)
    A_hk = dev_u8(A).view(torch.float8_e4m3fn).unsqueeze(0)
    B_hk = dev_u8(B).view(torch.float8_e4m3fn).unsqueeze(0)
    a_scale_hk = dev_f32(sa).reshape(1, BATCH, 1, M)
    b_scale_hk = dev_f32(sb).reshape(1, BATCH, 1, N)
    bias_hk = dev_bf16(bias).reshape(1, BATCH, 1, N)
    C_hk = torch.zeros(1, BATCH, M, N, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(TypeError, match="E4M3FN"):
        hk.batched_gemm.a8w8.dispatch(A_hk.float().bfloat16(), B_hk.float().bfloat16(), a_scale_hk, b_scale_hk, C_hk,
                                      bias_hk)
    hk.batched_gemm.a8w8.dispatch(A_hk, B_hk, a_scale_hk, b_scale_hk, C_hk, bias_hk)
    torch.cuda.synchronize()
    ref = orc.batched_gemm_a8w8_ref(A, B, sa, sb, bias)
    got = host_bf16_f32(C_hk.squeeze(0))
    assert np.abs(got - ref).max() / np.abs(ref).max() < 0.10  # the reference test's own bar
    for z in range(BATCH):
        assert_gemm_close(got[z], ref[z], f"batch {z}")


# ------------------------------------------------ block-scale multiply-add

def blockscale_operands(orc, M, N, K, seed, group_n):
    """The reference tests' fused-GEMM inputs (tests/test_gemm.py:468-472,
    510-514): a, b ~ 0.1 N(0, 1), here as their E4M3FN values (unit scale),
    with independent scales in [0, 2) per 128-group."""
    rng = np.random.default_rng(seed)
    A = orc.e4m3_encode(orc.bf16_bits_to_f32(orc.randn_bf16((M, K), seed=seed, std=0.1)))
    B = orc.e4m3_encode(orc.bf16_bits_to_f32(orc.randn_bf16((N, K), seed=seed + 1, std=0.1)))
    sa = (rng.random((M, K // 128)) * 2.0).astype(np.float32)
    sb = (rng.random((K // 128, N if group_n == 1 else (N + 127) // 128)) * 2.0).astype(np.float32)
    return A, B, sa, sb


@pytest.mark.parametrize("group_n", [1, 128])
@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (333, 516, 384), (1, 256, 1024), (600, 772, 2048), (9, 4160, 256),
                                   (40, 200, 512), (129, 264, 256)])
def test_blockscale_mul_add(orc, M, N, K, group_n):
    require_gpu()
    A, B, sa, sb = blockscale_operands(orc, M, N, K, M + N, group_n)
    ca = orc.randn_bf16((M, N), seed=K, std=0.5)
    cb = orc.randn_bf16((M, N), seed=K + 1, std=0.5)
    C = hkq.gemm_blockscale_mul_add(dev_u8(A), dev_u8(B), dev_f32(sa), dev_f32(sb), dev_bf16(ca), dev_bf16(cb),
                                    group_n=group_n)
    torch.cuda.synchronize()
    ref = orc.gemm_blockscale_mul_add_ref(A, B, sa, sb, ca, cb, 128, group_n)
    assert_gemm_close(host_bf16_f32(C), ref, f"mul_add {M}x{N}x{K} gn{group_n}")


def test_blockscale_mul_add_unit_and_zero_factors(orc):
    """c_a = 1, c_b = 0 gives the block-scale GEMM's own bits; c_a = 0 gives c_b."""
    require_gpu()
    M, N, K = 200, 264, 512
    A, B, sa, sb = blockscale_operands(orc, M, N, K, 7, 128)
    one = dev_bf16(np.full((M, N), 0x3F80, np.uint16))
    zero = dev_bf16(np.zeros((M, N), np.uint16))
    cb = orc.randn_bf16((M, N), seed=8)
    args = (dev_u8(A), dev_u8(B), dev_f32(sa), dev_f32(sb))
    C0 = hkq.gemm_blockscale(*args, group_n=128)
    C1 = hkq.gemm_blockscale_mul_add(*args, one, zero, group_n=128)
    C2 = hkq.gemm_blockscale_mul_add(*args, zero, dev_bf16(cb), group_n=128)
    torch.cuda.synchronize()
    assert torch.equal(C0, C1)
    assert np.array_equal(C2.view(torch.int16).cpu().numpy().view(np.uint16), cb)


def test_fused_blockscale_mul_add_module_reference_call(orc):
    """tests/test_gemm.py:498-533: M = N = K = 256, a_scale [M, K/128] and
    b_scale [K/128, N] in [0, 2), c_a / c_b ~ 0.5 N(0, 1); the reference's bf16
    a / b are passed as their per-row E4M3FN quantization."""
    require_gpu()
    import hipkittens as hk
    M, N, K = 256, 256, 256
    A, B, sa, sb = blockscale_operands(orc, M, N, K, 42, 1)
    ca = orc.randn_bf16((M, N), seed=43, std=0.5)
    cb = orc.randn_bf16((M, N), seed=44, std=0.5)
    c = torch.zeros(M, N, dtype=torch.bfloat16, device="cuda")
    hk.fused_gemm.a8w8_blockscale_mul_add.dispatch(dev_u8(A).view(torch.float8_e4m3fn),
                                                   dev_u8(B).view(torch.float8_e4m3fn), c, dev_f32(sa), dev_f32(sb),
                                                   dev_bf16(ca), dev_bf16(cb))
    torch.cuda.synchronize()
    ref = orc.gemm_blockscale_mul_add_ref(A, B, sa, sb, ca, cb, 128, 1)
    got = host_bf16_f32(c)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 0.10
    assert_gemm_close(got, ref, "mul_add module")


def test_fused_blockscale_a16w16_module_reference_call(orc):
    """tests/test_gemm.py:454-496: the block-scale GEMM and the bf16 GEMM over the
    same M = 256 rows (N_fp8 = N_bf16 = K = 256)."""
    require_gpu()
    import hipkittens as hk
    M, N8, N16, K = 256, 256, 256, 256
    A, B, sa, sb = blockscale_operands(orc, M, N8, K, 52, 1)
    a16 = orc.randn_bf16((M, K), seed=53, std=0.1)
    b16 = orc.randn_bf16((N16, K), seed=54, std=0.1)
    c8 = torch.zeros(M, N8, dtype=torch.bfloat16, device="cuda")
    c16 = torch.zeros(M, N16, dtype=torch.bfloat16, device="cuda")
    hk.fused_gemm.a8w8_blockscale_a16w16.dispatch(dev_u8(A).view(torch.float8_e4m3fn),
                                                  dev_u8(B).view(torch.float8_e4m3fn), c8, dev_f32(sa), dev_f32(sb),
                                                  dev_bf16(a16), dev_bf16(b16), c16)
    torch.cuda.synchronize()
    ref8 = orc.gemm_blockscale_ref(A, B, sa, sb, 128, 1)
    ref16 = orc.gemm_bf16_ref(a16, b16)
    assert_gemm_close(host_bf16_f32(c8), ref8, "block-scale part")
    assert_gemm_close(host_bf16_f32(c16), ref16, "bf16 part")
