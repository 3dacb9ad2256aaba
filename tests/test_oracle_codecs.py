"""Pin the oracle's element codecs (CPU only).

e4m3fn is checked against torch.float8_e4m3fn, the encoder the reference's own
test uses as its oracle (reference tests/test_moe.py:997-999); e2m1 against the
reference's value table (moe-gemm/moe_op_mxfp4/kernel.cpp:32-35) plus a brute
force nearest-even search; the MX scale rule against the reference's float
formula (quantization/fused_mxfp4_quant/kernel.cpp:99-105) evaluated in numpy.
"""
import numpy as np
import pytest
import torch


def torch_e4m3(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def all_bf16_values() -> np.ndarray:
    bits = np.arange(1 << 16, dtype=np.uint32)
    v = (bits << 16).view(np.float32)
    return v[np.isfinite(v)]


def test_e4m3_decode_all_codes(orc):
    codes = np.arange(256, dtype=np.uint8)
    ours = orc.e4m3_decode(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert set(codes[nan].tolist()) == {0x7F, 0xFF}
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # known answers: max normal 448 (fused_fp8_quant/kernel.cpp:12), min subnormal 2^-9
    assert ours[0x7E] == 448.0 and ours[0xFE] == -448.0 and ours[0x01] == 2.0 ** -9 and ours[0x08] == 2.0 ** -6


def test_e4m3_encode_every_bf16(orc):
    v = np.clip(all_bf16_values(), -448.0, 448.0).astype(np.float32)
    assert np.array_equal(orc.e4m3_encode(v), torch_e4m3(v))


def test_e4m3_encode_rounding_boundaries(orc):
    # every midpoint between adjacent positive e4m3 values, +-2 fp32 ulp, both signs
    pos = np.sort(orc.e4m3_decode(np.arange(0, 0x7F, dtype=np.uint8)))
    mids = ((pos[:-1].astype(np.float64) + pos[1:]) / 2).astype(np.float32)
    pts = [mids, pos]
    u = mids.view(np.int32)
    for d in (-2, -1, 1, 2):
        pts.append((u + d).view(np.float32))
    x = np.concatenate(pts)
    x = np.concatenate([x, -x, [0.0, -0.0, 448.0, -448.0]]).astype(np.float32)
    x = x[np.abs(x) <= 448.0]
    assert np.array_equal(orc.e4m3_encode(x), torch_e4m3(x))


def test_e4m3_encode_random_fp32(orc):
    rng = np.random.default_rng(1)
    mant = rng.uniform(1.0, 2.0, 1 << 22)
    expo = rng.integers(-30, 9, 1 << 22)
    sign = rng.choice([-1.0, 1.0], 1 << 22)
    x = np.clip(sign * mant * np.exp2(expo), -448.0, 448.0).astype(np.float32)
    assert np.array_equal(orc.e4m3_encode(x), torch_e4m3(x))


def test_e4m3_encode_special(orc):
    x = np.array([np.nan, -np.nan, 1e30, -1e30, 449.0, 0.0, -0.0], dtype=np.float32)
    c = orc.e4m3_encode(x)
    assert (c[0] & 0x7F) == 0x7F and (c[1] & 0x7F) == 0x7F
    assert c[2] == 0x7E and c[3] == 0xFE and c[4] == 0x7E and c[5] == 0x00 and c[6] == 0x80


E2M1_GRID = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def test_e2m1_table(orc):
    # reference LUT (moe-gemm/moe_op_mxfp4/kernel.cpp:32-35)
    ref = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])
    ours = orc.e2m1_decode(np.arange(16))
    assert np.array_equal(ours, ref) and np.array_equal(np.signbit(ours), np.signbit(ref))


def brute_e2m1(a: float) -> int:
    """Nearest grid point by exhaustive search; ties to the even code; saturate."""
    if a >= 6.0:
        return 7
    d = np.abs(E2M1_GRID - a)
    best = np.flatnonzero(d == d.min())
    if len(best) == 1:
        return int(best[0])
    return int(best[0] if best[0] % 2 == 0 else best[1])


def test_e2m1_encode_brute_force(orc):
    vals = [v for v in all_bf16_values() if abs(v) <= 8.0]
    ties = [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]
    extra = []
    for t in ties:
        u = np.float32(t).view(np.int32)
        extra += [np.float32(t), (u - 1).view(np.float32), (u + 1).view(np.float32)]
    x = np.array(vals + extra + [-t for t in extra] + [6.5, 7.0, 100.0, -7.0], dtype=np.float32)
    ours = orc.e2m1_encode(x)
    ref = np.array([brute_e2m1(abs(float(v))) | (8 if np.signbit(v) else 0) for v in x], dtype=np.uint8)
    assert np.array_equal(ours, ref)
    assert orc.e2m1_encode(np.array([np.nan], np.float32))[0] == 0x7


def brute_e2m1_floor(a: float) -> int:
    """Largest grid magnitude at or below a, by exhaustive search (a >= 0)."""
    below = np.flatnonzero(E2M1_GRID <= a)
    return int(below[-1]) if len(below) else 0


def test_e2m1_floor_brute_force(orc):
    """The reference fused quantizer's ladder (fused_mxfp4_quant/kernel.cpp:
    128-150): every bf16 value of magnitude <= 8, every grid point and its
    neighbours one ulp away, saturation, signed zeros, infinities and NaN."""
    vals = [v for v in all_bf16_values() if abs(v) <= 8.0]
    extra = []
    for g in E2M1_GRID[1:]:
        u = np.float32(g).view(np.int32)
        extra += [np.float32(g), (u - 1).view(np.float32), (u + 1).view(np.float32)]
    x = np.array(vals + extra + [-t for t in extra] + [6.5, 100.0, -7.0, np.inf, -np.inf, 0.0, -0.0],
                 dtype=np.float32)
    ours = orc.e2m1_floor(x)
    ref = np.array([brute_e2m1_floor(abs(float(v))) | (8 if np.signbit(v) else 0) for v in x], dtype=np.uint8)
    assert np.array_equal(ours, ref)
    # known answers of the ladder, and NaN (every comparison false): magnitude 0, sign kept
    known = np.array([1.4, 1.5, 5.99, 6.0, 0.49, 0.5, -2.9, -3.0], np.float32)
    assert orc.e2m1_floor(known).tolist() == [0x2, 0x3, 0x6, 0x7, 0x0, 0x1, 0xC, 0xD]
    nan = np.array([np.float32(np.nan), -np.float32(np.nan)], np.float32)
    assert orc.e2m1_floor(nan).tolist() == [0x0, 0x8]
    # the floor and round-to-nearest-even rules meet exactly on the grid
    g = np.array(list(E2M1_GRID) + [-v for v in E2M1_GRID[1:]], np.float32)
    assert np.array_equal(orc.e2m1_floor(g), orc.e2m1_encode(g))


def test_mx_scale_rule_matches_float_formula(orc):
    # the reference's float formula: P = (bits + 0x200000) & 0xFF800000;
    # e = clamp(floor(log2(P)) - 2, -127, 127) (fused_mxfp4_quant/kernel.cpp:99-105)
    v = all_bf16_values()
    v = v[v > 0]
    p = ((v.view(np.uint32).astype(np.uint64) + 0x200000) & 0xFF800000).astype(np.uint32).view(np.float32)
    with np.errstate(divide="ignore", over="ignore"):
        e = np.floor(np.log2(p.astype(np.float64))) - 2
    e = np.clip(np.nan_to_num(e, posinf=1e9, neginf=-1e9), -127, 127).astype(np.int32)
    assert np.array_equal(orc.mx_scale_exp(v), e)
    # defined where the float rule is not: amax = 0 -> e = -127 (code 0); inf -> 127
    assert orc.mx_scale_exp(np.array([0.0, np.inf], np.float32)).tolist() == [-127, 127]
    # known answers: amax 6 -> e=0 (6 = 1.5*2^2); amax 7 rounds to 8 -> e=1; amax 1 -> e=-2
    assert orc.mx_scale_exp(np.array([6.0, 7.0, 1.0, 1.74], np.float32)).tolist() == [0, 1, -2, -2]


def test_e8m0_decode(orc):
    s = np.arange(256)
    d = orc.e8m0_decode(s)
    assert d[127] == 1.0 and d[128] == 2.0 and d[0] == 2.0 ** -127 and np.isnan(d[255])


def test_bf16_round_matches_torch(orc):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(1 << 20) * np.exp2(rng.integers(-20, 20, 1 << 20))).astype(np.float32)
    ours = orc.f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
