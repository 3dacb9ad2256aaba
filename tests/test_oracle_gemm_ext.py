"""Pin the oracle's bf16, batched A8W8 and block-scale multiply-add GEMM
references on the CPU, against torch (an independent fp32 implementation of
the reference tests' formulas) and closed forms."""
import numpy as np
import torch


def bf16_tensor(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def e4m3_tensor(codes):
    return torch.from_numpy(np.ascontiguousarray(codes, np.uint8)).view(torch.float8_e4m3fn)


def test_gemm_bf16_ref_against_torch(orc):
    """tests/test_gemm.py:21-42: C_ref = A.float() @ B.float().T."""
    A = orc.randn_bf16((96, 160), seed=1)
    B = orc.randn_bf16((72, 160), seed=2)
    bias = orc.randn_bf16((72,), seed=3)
    ref = orc.gemm_bf16_ref(A, B, bias)
    t = (bf16_tensor(A).double() @ bf16_tensor(B).double().T + bf16_tensor(bias).double()).numpy()
    assert np.allclose(ref, t, rtol=1e-12, atol=1e-12)
    t32 = (bf16_tensor(A).float() @ bf16_tensor(B).float().T).numpy()
    assert np.allclose(orc.gemm_bf16_ref(A, B), t32, rtol=1e-5, atol=1e-4)


def test_gemm_bf16_ref_identity(orc):
    """B = I: C = A exactly; a one-hot bias adds to one column only."""
    K = 64
    A = orc.randn_bf16((10, K), seed=4)
    eye = orc.f32_to_bf16_bits(np.eye(K, dtype=np.float32))
    bias = np.zeros(K, np.uint16)
    bias[5] = 0x4000  # 2.0
    C = orc.gemm_bf16_ref(A, eye, bias)
    a = orc.bf16_bits_to_f32(A).astype(np.float64)
    a[:, 5] += 2.0
    assert np.array_equal(C, a)


def test_batched_gemm_a8w8_ref_against_torch(orc):
    """tests/test_gemm.py:362-366: C_ref = bmm(A, B) * a_scale * b_scale + bias,
    here with B given as [Z, N, K] (the kernel's layout: B_hk = B.transpose(-2, -1))."""
    Z, M, N, K = 3, 40, 24, 128
    rng = np.random.default_rng(7)
    A = rng.integers(0, 256, (Z, M, K), dtype=np.uint8) & 0xF7  # no NaN codes (0x7F / 0xFF)
    B = rng.integers(0, 256, (Z, N, K), dtype=np.uint8) & 0xF7
    sa = rng.random((Z, M)).astype(np.float32) * 0.1
    sb = rng.random((Z, N)).astype(np.float32) * 0.1
    bias = orc.randn_bf16((Z, N), seed=8)
    ref = orc.batched_gemm_a8w8_ref(A, B, sa, sb, bias)
    a, b = e4m3_tensor(A).double(), e4m3_tensor(B).double()
    t = torch.bmm(a, b.transpose(1, 2).contiguous()) * torch.from_numpy(sa).double()[:, :, None] \
        * torch.from_numpy(sb).double()[:, None, :] + bf16_tensor(bias).double()[:, None, :]
    assert np.allclose(ref, t.numpy(), rtol=1e-12, atol=1e-12)
    # each batch is the 2-D A8W8 reference plus the bias
    for z in range(Z):
        two_d = orc.gemm_a8w8_ref(A[z], B[z], sa[z], sb[z]) + orc.bf16_bits_to_f32(bias[z]).astype(np.float64)
        assert np.allclose(ref[z], two_d, rtol=1e-12, atol=1e-12)


def test_blockscale_mul_add_ref(orc):
    """tests/test_gemm.py:519-525: ref = c_a * gemm_out + c_b; c_a = 1, c_b = 0
    is the block-scale GEMM itself; c_a = 0 gives c_b exactly; torch restatement."""
    M, N, K = 64, 256, 384
    rng = np.random.default_rng(9)
    A = rng.integers(0, 256, (M, K), dtype=np.uint8) & 0xF7
    B = rng.integers(0, 256, (N, K), dtype=np.uint8) & 0xF7
    sa = rng.random((M, K // 128)).astype(np.float32) * 2
    sb = rng.random((K // 128, N)).astype(np.float32) * 2
    ca = orc.randn_bf16((M, N), seed=10, std=0.5)
    cb = orc.randn_bf16((M, N), seed=11, std=0.5)
    ref = orc.gemm_blockscale_mul_add_ref(A, B, sa, sb, ca, cb, 128, 1)
    a, b = e4m3_tensor(A).double(), e4m3_tensor(B).double()
    g = torch.zeros(M, N, dtype=torch.float64)
    for kb in range(K // 128):
        ks, ke = kb * 128, (kb + 1) * 128
        g += (a[:, ks:ke] @ b[:, ks:ke].T) * torch.from_numpy(sa).double()[:, kb:kb + 1] \
            * torch.from_numpy(sb).double()[kb:kb + 1, :]
    t = bf16_tensor(ca).double() * g + bf16_tensor(cb).double()
    assert np.allclose(ref, t.numpy(), rtol=1e-12, atol=1e-12)
    one = np.full((M, N), 0x3F80, np.uint16)
    zero = np.zeros((M, N), np.uint16)
    assert np.array_equal(orc.gemm_blockscale_mul_add_ref(A, B, sa, sb, one, zero, 128, 1),
                          orc.gemm_blockscale_ref(A, B, sa, sb, 128, 1))
    assert np.array_equal(orc.gemm_blockscale_mul_add_ref(A, B, sa, sb, zero, cb, 128, 1),
                          orc.bf16_bits_to_f32(cb).astype(np.float64))


def _close_to_fp64(f32, f64, a_abs_b_abs):
    """fp32-product reference within 2^-16 of the sum of |terms| of the fp64 one."""
    assert f32.dtype == np.float32 and f32.shape == f64.shape
    assert np.all(np.abs(f32.astype(np.float64) - f64) <= 2.0 ** -16 * a_abs_b_abs + 1e-30)


def test_fp32_references_match_fp64(orc):
    """The fp32 full-output references (used at BASELINE sizes) against the
    fp64 ones on ragged shapes with per-row/column/group scales that differ
    everywhere, so a transposed or mis-indexed scale would fail."""
    M, N, K = 200, 260, 1024
    xa = orc.randn_bf16((M, K), seed=11)
    xw = orc.randn_bf16((N, K), seed=12, std=0.02)
    A, sa = orc.quant_rowwise(xa, None, "fp8")
    B, sb = orc.quant_rowwise(xw, None, "fp8")
    a, b = orc.e4m3_decode(A).astype(np.float64), orc.e4m3_decode(B).astype(np.float64)
    absum = (np.abs(a) @ np.abs(b).T) * np.abs(sa).reshape(-1, 1) * np.abs(sb).reshape(1, -1)
    _close_to_fp64(orc.gemm_a8w8_ref_f32(A, B, sa, sb), orc.gemm_a8w8_ref(A, B, sa, sb), absum)

    A1, sa1 = orc.quant_rowwise(xa, 128, "fp8")              # [M, K/128]
    for gn in (128, 1):
        Np = (N + 127) // 128 * 128
        xw2 = orc.randn_bf16((Np, K), seed=13, std=0.02)
        if gn == 128:
            B1, sbt = orc.quant_block_2d(xw2)
            sb1 = np.ascontiguousarray(sbt.T)                   # [K/128, N/128]
        else:
            B1, sbr = orc.quant_rowwise(xw2, 128, "fp8")
            sb1 = np.ascontiguousarray(sbr.T[:, :N])            # [K/128, N]
        B1 = np.ascontiguousarray(B1[:N])
        ref = orc.gemm_blockscale_ref(A1, B1, sa1, sb1, 128, gn)
        a1, b1 = orc.e4m3_decode(A1).astype(np.float64), orc.e4m3_decode(B1).astype(np.float64)
        absum = np.zeros((M, N))
        for g in range(K // 128):
            s = slice(128 * g, 128 * g + 128)
            absum += (np.abs(a1[:, s]) @ np.abs(b1[:, s]).T) * np.abs(sa1[:, g:g + 1]) * \
                np.abs(np.repeat(sb1[g], gn)[:N])[None, :]
        _close_to_fp64(orc.gemm_blockscale_ref_f32(A1, B1, sa1, sb1, 128, gn), ref, absum)

    Aq, As = orc.mx_quant_fp4(xa)
    Bq, Bs = orc.mx_quant_fp4(xw)
    da, db = orc.mx_fp4_dequant_f32(Aq, As).astype(np.float64), orc.mx_fp4_dequant_f32(Bq, Bs).astype(np.float64)
    _close_to_fp64(orc.gemm_mxfp4_ref_f32(Aq, As, Bq, Bs), orc.gemm_mxfp4_ref(Aq, As, Bq, Bs),
                   np.abs(da) @ np.abs(db).T)
