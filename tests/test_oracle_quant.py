"""Pin the oracle's quantizers and GEMM/MoE references (CPU only).

Each oracle routine is compared against a second, independently written
restatement (vectorised numpy + torch's float8 encoder) of the same reference
formula, against the reference tests' own formulas, and against closed forms.
"""
import numpy as np
import pytest
import torch


def torch_e4m3(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def numpy_rowwise(x32: np.ndarray, group: int, qmax: float):
    """Vectorised restatement of quant/kernel.cpp:46-107 (per group of columns)."""
    M, K = x32.shape
    xg = x32.reshape(M, K // group, group)
    amax = np.abs(xg).max(axis=2)
    s = np.maximum(amax / np.float32(qmax), np.float32(1e-10)).astype(np.float32)
    r = (np.float32(1.0) / s).astype(np.float32)
    v = (xg * r[:, :, None]).astype(np.float32)
    if qmax == 448.0:
        q = torch_e4m3(np.clip(v, -448.0, 448.0)).reshape(M, K)
    else:
        q = np.clip(np.rint(v), -127, 127).astype(np.int8).view(np.uint8).reshape(M, K)
    return q, s


@pytest.mark.parametrize("group", [None, 128])
@pytest.mark.parametrize("kind", ["fp8", "int8"])
def test_rowwise_matches_numpy(orc, group, kind):
    M, K = 64, 1024
    xb = orc.randn_bf16((M, K), seed=11)
    # rows with extreme dynamic range, an all-zero row and a row of bf16 subnormals
    xb[1, :] = orc.f32_to_bf16_bits(np.linspace(-3e4, 3e4, K, dtype=np.float32))
    xb[2, :] = 0
    xb[3, :] = orc.f32_to_bf16_bits((np.arange(K, dtype=np.float32) - K / 2) * 1e-40)
    q, s = orc.quant_rowwise(xb, group, kind)
    g = K if group is None else group
    qn, sn = numpy_rowwise(orc.bf16_bits_to_f32(xb), g, 448.0 if kind == "fp8" else 127.0)
    assert np.array_equal(s.view(np.uint32), sn.view(np.uint32))
    assert np.array_equal(q, qn)


def test_rowwise_int8_vs_reference_test_formula(orc):
    # reference test oracle (tests/test_misc.py:532-536) divides x / s; the kernel
    # multiplies by 1/s (quant/kernel.cpp:94,105): scales equal, codes within 1
    xb = orc.randn_bf16((256, 4096), seed=5)
    q, s = orc.quant_rowwise(xb, None, "int8")
    x = torch.from_numpy(orc.bf16_bits_to_f32(xb))
    ref_s = (x.abs().max(dim=1, keepdim=True).values / 127.0).clamp(min=1e-10)
    ref_q = (x / ref_s).round().clamp(-127, 127).to(torch.int8).numpy()
    assert np.array_equal(s, ref_s.numpy())
    assert np.abs(q.view(np.int8).astype(np.int32) - ref_q.astype(np.int32)).max() <= 1


def test_rowwise_known_answers(orc):
    K = 128
    x = np.zeros((2, K), np.float32)
    x[0, :4] = [448.0, 1.0, -0.5, 0.015625]  # amax 448 -> s = 1, r = 1
    x[1, :3] = [-0.0, 0.0, 0.0]              # all-zero row -> s = 1e-10
    q, s = orc.quant_rowwise(orc.f32_to_bf16_bits(x), None, "fp8")
    assert s[0, 0] == 1.0 and s[1, 0] == np.float32(1e-10)
    assert q[0, :4].tolist() == [0x7E, 0x38, 0xB0, 0x08]
    assert q[1, 0] == 0x80 and q[1, 1] == 0x00


def test_static_fp8_vs_reference_test_formula(orc):
    # tests/test_moe.py:997-999: (x / scale).clamp(-448, 448).to(float8_e4m3fn)
    xb = orc.randn_bf16((256, 128), seed=42, std=100.0)
    for scale in (0.5, 0.37, 3.0):
        y = orc.quant_static_fp8(xb, scale)
        x = torch.from_numpy(orc.bf16_bits_to_f32(xb))
        ref = (x / scale).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        assert np.array_equal(y, ref)


def numpy_mx_fp4(x32: np.ndarray):
    """Vectorised restatement: scale from the float formula, elements by
    nearest-even search over the e2m1 grid."""
    M, K = x32.shape
    xb = x32.reshape(M, K // 32, 32)
    amax = np.abs(xb).max(axis=2)
    p = ((amax.view(np.uint32).astype(np.uint64) + 0x200000) & 0xFF800000).astype(np.uint32).view(np.float32)
    with np.errstate(divide="ignore"):
        e = np.floor(np.log2(p.astype(np.float64))) - 2
    e = np.clip(np.nan_to_num(e, neginf=-1e9), -127, 127).astype(np.int32)
    qx = np.ldexp(xb.astype(np.float64), -e[:, :, None])
    grid = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
    a = np.minimum(np.abs(qx), 6.0)
    d = np.abs(a[..., None] - grid)
    dmin = d.min(axis=-1, keepdims=True)
    cand = d == dmin
    # ties -> even code: prefer the even index among candidates
    idx = np.where(cand[..., ::2].any(-1), np.argmax(cand * (np.arange(8) % 2 == 0), -1), np.argmax(cand, -1))
    code = idx.astype(np.uint8) | (np.signbit(xb).astype(np.uint8) << 3)
    code = code.reshape(M, K)
    packed = (code[:, 0::2] | (code[:, 1::2] << 4)).astype(np.uint8)
    return packed, (e + 127).astype(np.uint8)


def test_mx_fp4_quant_matches_numpy(orc):
    xb = orc.randn_bf16((64, 1024), seed=7)
    xb[0, :32] = 0  # all-zero block
    xb[1, :32] = orc.f32_to_bf16_bits(np.full(32, 7.0, np.float32))  # amax rounds up
    q, s = orc.mx_quant_fp4(xb)
    qn, sn = numpy_mx_fp4(orc.bf16_bits_to_f32(xb))
    assert np.array_equal(s, sn)
    assert np.array_equal(q, qn)
    assert s[0, 0] == 0 and s[1, 0] == 128


def test_mx_fp4_round_trip_property(orc):
    # decode(encode(x)) is the nearest representable point of the block's grid
    xb = orc.randn_bf16((32, 512), seed=9)
    q, s = orc.mx_quant_fp4(xb)
    deq = orc.mx_fp4_dequant_f32(q, s)
    x = orc.bf16_bits_to_f32(xb)
    scale = np.repeat(orc.e8m0_decode(s), 32, axis=1)
    grid = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
    err = np.abs(deq - x)
    best = np.abs(np.abs(x)[..., None] - grid * scale[..., None]).min(-1)
    sat = np.abs(x) > 6 * scale
    assert np.all((err <= best + 1e-12) | sat)


def test_mx_fp8_quant_and_dequant(orc):
    # downcast_to_mxfp / upcast_from_mxfp FP8 round trip (tests/test_moe.py:1022-1054):
    # mean abs error well under the reference's 0.5 bound; the scale is the
    # ceil power of two of amax/448 (quant_moe/kernel.cpp:152-160)
    xb = orc.randn_bf16((128, 256), seed=42)
    q, s = orc.mx_quant_fp8(xb)
    out = orc.mx_dequant(q, s, 128, 256, False)
    x = orc.bf16_bits_to_f32(xb)
    err = np.abs(orc.bf16_bits_to_f32(out) - x)
    assert err.mean() < 0.02
    amax = np.abs(x.reshape(128, 8, 32)).max(-1)
    scale = orc.e8m0_decode(s)
    assert np.all(scale >= amax / 448) and np.all(scale / 2 < amax / 448)


def test_mx_fp4_dequant_bf16(orc):
    xb = orc.randn_bf16((16, 256), seed=2)
    q, s = orc.mx_quant_fp4(xb)
    out = orc.mx_dequant(q, s, 16, 256, True)
    assert np.array_equal(orc.bf16_bits_to_f32(out), orc.mx_fp4_dequant_f32(q, s))


def test_gemm_a8w8_ref(orc):
    rng = np.random.default_rng(0)
    M, N, K = 64, 96, 256
    A = orc.e4m3_encode(rng.standard_normal((M, K)).astype(np.float32) * 30)
    B = orc.e4m3_encode(rng.standard_normal((N, K)).astype(np.float32) * 30)
    sa = rng.random(M).astype(np.float32) * 0.1 + 0.01
    sb = rng.random(N).astype(np.float32) * 0.1 + 0.01
    C = orc.gemm_a8w8_ref(A, B, sa, sb)
    # reference formula, torch fp32 (tests/test_gemm.py:116)
    a = torch.from_numpy(A).view(torch.float8_e4m3fn).float()
    b = torch.from_numpy(B).view(torch.float8_e4m3fn).float()
    ref = (a @ b.T) * torch.from_numpy(sa)[:, None] * torch.from_numpy(sb)[None, :]
    np.testing.assert_allclose(C, ref.double().numpy(), rtol=1e-5, atol=1e-3)
    # closed form: all codes 1.0 (0x38) -> C = K * sa * sb
    C1 = orc.gemm_a8w8_ref(np.full((M, K), 0x38, np.uint8), np.full((N, K), 0x38, np.uint8), sa, sb)
    np.testing.assert_array_equal(C1, K * sa.astype(np.float64)[:, None] * sb.astype(np.float64)[None, :])


def test_gemm_blockscale_ref(orc):
    rng = np.random.default_rng(1)
    M, N, K = 32, 256, 384
    A = orc.e4m3_encode(rng.standard_normal((M, K)).astype(np.float32) * 10)
    B = orc.e4m3_encode(rng.standard_normal((N, K)).astype(np.float32) * 10)
    sa = rng.random((M, K // 128)).astype(np.float32) * 0.1 + 0.01
    sb = rng.random((K // 128, N // 128)).astype(np.float32) * 0.1 + 0.01
    C = orc.gemm_blockscale_ref(A, B, sa, sb, 128, 128)
    # torch restatement of tests/test_gemm.py:148-153 with b_scale expanded per 128 cols
    a = torch.from_numpy(A).view(torch.float8_e4m3fn).double()
    b = torch.from_numpy(B).view(torch.float8_e4m3fn).double()
    ref = torch.zeros(M, N, dtype=torch.float64)
    for kg in range(K // 128):
        part = a[:, kg * 128:(kg + 1) * 128] @ b[:, kg * 128:(kg + 1) * 128].T
        bs = torch.from_numpy(sb[kg]).double().repeat_interleave(128)
        ref += part * torch.from_numpy(sa[:, kg]).double()[:, None] * bs[None, :]
    np.testing.assert_allclose(C, ref.numpy(), rtol=1e-12, atol=1e-9)
    # uniform scales reduce to the plain GEMM times the product of scales
    C2 = orc.gemm_blockscale_ref(A, B, np.full((M, 3), 0.5, np.float32), np.full((3, 2), 0.25, np.float32))
    np.testing.assert_allclose(C2, orc.gemm_a8w8_ref(A, B, np.full(M, 0.5), np.full(N, 0.25)), rtol=1e-12)


def test_gemm_mxfp4_ref(orc):
    M, N, K = 16, 32, 256
    # closed form: every element 1.0 (code 2), scales 127 (x1) -> C = K
    Aq = np.full((M, K // 2), 0x22, np.uint8)
    Bq = np.full((N, K // 2), 0x22, np.uint8)
    As = np.full((M, K // 32), 127, np.uint8)
    Bs = np.full((N, K // 32), 127, np.uint8)
    assert np.all(orc.gemm_mxfp4_ref(Aq, As, Bq, Bs) == K)
    # one block scaled by 2^3 on A row 0 -> that block contributes 8x
    As2 = As.copy()
    As2[0, 1] = 130
    C = orc.gemm_mxfp4_ref(Aq, As2, Bq, Bs)
    assert np.all(C[0] == K + 7 * 32) and np.all(C[1:] == K)
    # matches dequantized fp32 matmul of random data
    xa = orc.randn_bf16((M, K), seed=3)
    xb = orc.randn_bf16((N, K), seed=4, std=0.02)
    qa, sa = orc.mx_quant_fp4(xa)
    qb, sb = orc.mx_quant_fp4(xb)
    ref = torch.from_numpy(orc.mx_fp4_dequant_f32(qa, sa)) @ torch.from_numpy(orc.mx_fp4_dequant_f32(qb, sb)).T
    np.testing.assert_allclose(orc.gemm_mxfp4_ref(qa, sa, qb, sb), ref.double().numpy(), rtol=1e-5, atol=1e-5)


def loop_routing(assigns, E, block_m):
    """Literal restatement of tests/test_moe.py:97-128 (python loops)."""
    T, topk = assigns.shape
    hist = [0] * E
    for t in range(T):
        for k in range(topk):
            hist[assigns[t, k]] += 1
    offs = [0] * E
    for e in range(1, E):
        offs[e] = offs[e - 1] + hist[e - 1]
    gather = [0] * (T * topk)
    pos = list(offs)
    for t in range(T):
        for k in range(topk):
            e = assigns[t, k]
            gather[pos[e]] = t * topk + k
            pos[e] += 1
    tiles = [e | (b << 16) for e in range(E) for b in range((hist[e] + block_m - 1) // block_m)]
    return hist, offs, gather, tiles


def test_ogs_routing(orc):
    rng = np.random.default_rng(4)
    assigns = rng.integers(0, 8, (300, 2))
    hist, offs, gather, ed = orc.ogs_routing(assigns, 8, 128)
    h2, o2, g2, t2 = loop_routing(assigns, 8, 128)
    assert hist.tolist() == h2 and offs.tolist() == o2 and gather.tolist() == g2 and ed.tolist() == t2
    assert hist.sum() == 600 and sorted(gather.tolist()) == list(range(600))


@pytest.mark.parametrize("layout", ["ekn", "enk"])
def test_moe_ref_matches_dense(orc, layout):
    rng = np.random.default_rng(5)
    T, E, topk, K, N = 200, 4, 2, 128, 64
    X = orc.e4m3_encode(rng.standard_normal((T, K)).astype(np.float32))
    W = orc.e4m3_encode(rng.standard_normal((E, K, N)).astype(np.float32) * 0.1)
    xs = rng.random(T).astype(np.float32) + 0.5
    ws = rng.random((E, N)).astype(np.float32) + 0.5
    bias = rng.standard_normal((E, N)).astype(np.float32)
    assigns = np.stack([rng.permutation(E)[:topk] for _ in range(T)])
    hist, offs, gather, ed = orc.ogs_routing(assigns, E, 128)
    Wl = W if layout == "ekn" else np.ascontiguousarray(W.transpose(0, 2, 1))
    Y = orc.moe_ref(X, Wl, xs, ws, bias, gather, hist, offs, ed, topk, 128, layout)
    assert not np.isnan(Y).any()
    x = orc.e4m3_decode(X).astype(np.float64)
    w = orc.e4m3_decode(W).astype(np.float64)
    for slot in range(T * topk):
        t, k = divmod(int(gather[slot]), topk)
        e = assigns[t, k]
        ref = (x[t] @ w[e]) * xs[t] * ws[e] + bias[e]
        np.testing.assert_allclose(Y[slot], ref, rtol=1e-12, atol=1e-12)


def test_quant_block_2d(orc):
    """Each 128x128 block quantized like one 16384-wide row (loop over blocks),
    with known answers for a block of constant magnitude."""
    xb = orc.randn_bf16((256, 384), seed=21, std=0.02)
    xb[:128, 128:256] = orc.f32_to_bf16_bits(np.full((128, 128), -0.5, np.float32))
    q, s = orc.quant_block_2d(xb)
    assert q.shape == (256, 384) and s.shape == (2, 3)
    x = orc.bf16_bits_to_f32(xb)
    for nb in range(2):
        for kb in range(3):
            blk = x[nb * 128:(nb + 1) * 128, kb * 128:(kb + 1) * 128]
            qn, sn = numpy_rowwise(blk.reshape(1, -1), 128 * 128, 448.0)
            assert s[nb, kb] == sn[0, 0]
            assert np.array_equal(q[nb * 128:(nb + 1) * 128, kb * 128:(kb + 1) * 128], qn.reshape(128, 128))
    # constant block: amax 0.5 -> s = 0.5/448, every code is -448 (0xFE)
    assert s[0, 1] == np.float32(np.float32(0.5) / np.float32(448.0))
    assert np.all(q[:128, 128:256] == 0xFE)
