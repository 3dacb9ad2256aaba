"""CPU oracle for the quantized-GEMM hot path. TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker (or the timed CPU
baseline). The product path (``amd-kernels_amd``) never imports it.

The element-level arithmetic lives in ``hkq_oracle.c`` (plain scalar C, built
by ``oracle/Makefile`` into ``oracle/_build/liboracle.so``); this file wraps it
with numpy and adds the fp32/fp64 dequant-matmul references of the GEMMs.

How each function is pinned (tests/test_oracle_*.py):

=====================  ==========================================================
e4m3_encode/decode     torch.float8_e4m3fn (the reference test's own encoder,
                       tests/test_moe.py:997-999): every bf16 value, every fp32
                       within +-2 ulp of every e4m3 rounding boundary, 4M random
                       fp32; all 256 codes decoded.
e2m1_encode/decode     value table (moe-gemm/moe_op_mxfp4/kernel.cpp:32-35) and
                       brute-force nearest-even search over the grid.
e2m1_floor             the reference quantizer's ladder (fused_mxfp4_quant/
                       kernel.cpp:128-150) against a brute-force search for the
                       largest grid magnitude <= |x| over every bf16 value of
                       magnitude <= 8, every grid point +-1 ulp, NaN / +-inf /
                       +-0, and known answers (1.4 -> 1.0, 5.99 -> 4, 0.49 -> 0).
mx_scale_exp           the reference's float formula (fused_mxfp4_quant/
                       kernel.cpp:99-105) evaluated with numpy log2/floor over
                       every positive bf16 value.
quant_block_2d         per-block loop in numpy against the per-token rule on
                       each flattened block (tests/test_oracle_quant.py).
quant_rowwise          an independent vectorised numpy/torch restatement of
                       quant/kernel.cpp:46-107 (and of the reference test
                       formula tests/test_misc.py:532-536, within 1 code);
                       hand-computed known answers.
mx_quant_fp4/fp8       vectorised numpy restatement + round-trip property
                       (decode(encode(x)) is the nearest grid point).
static_fp8             torch reference formula (tests/test_moe.py:997-999).
gemm refs              reference formulas (tests/test_gemm.py:116,148-153,
                       gemm_a8w8_blockscale/test_parity.py:57-76), torch fp32,
                       plus closed forms (rank-1 / identity operands).
gemm_bf16_ref,         torch fp32 matmul / bmm on the same decoded values (the
batched_gemm_a8w8_ref, reference tests' formulas, tests/test_gemm.py:21-42,
gemm_blockscale_mul_   316-390, 498-533); identity and all-ones closed forms;
add_ref                c_a = 1, c_b = 0 reduces to the block-scale GEMM and
                       c_a = 0 to c_b exactly.
moe_ref / ogs_routing  tests/test_moe.py:97-128,733-753 restated; invariants
                       (histogram sum, exclusive scan, gather permutation) and
                       agreement with per-expert dense GEMMs.
moe_mxfp4_ref          per-expert dense gemm_mxfp4_ref on the gathered rows
                       (tests/test_oracle_moe.py); routed-weight and -1 block cases.
moe_blockscale_ref     per-expert dense gemm_blockscale_ref on the gathered rows
                       with each group's scales (group_k 64 / 128, group_n 1 /
                       64 / 128), and for [E, K, N] weights the same result
                       (tests/test_oracle_moe.py).
*_ref_f32              fp32 restatements used at BASELINE sizes (gemm_a8w8,
                       gemm_blockscale, gemm_mxfp4, moe, moe_mxfp4): against
                       the fp64 references within 2^-16 of the sum of |terms|
                       (tests/test_oracle_gemm_ext.py, tests/test_oracle_moe.py).
rmsnorm_quant          fp64 numpy RMSNorm (the test_parity.py formula of
                       fused_fp8_quant) then the pinned group / MX quantizers
                       (kind 2: the MX scale then e2m1_floor):
                       codes equal except where y sits within an ulp of a
                       rounding boundary; known answers for constant rows
                       (rms = |c| exactly); the fixed-order sum against math.fsum.
swiglu_quant           torch.nn.functional.silu(g) * u in fp64 then the pinned
                       per-token quantizer (codes within one step; scales within
                       4 ulp); alpha scaling; interleaved == split after a
                       column permutation.
topk                   torch.topk + torch.softmax (fp64) on tie-free logits;
                       brute-force sort by (-value, expert) on logits with many
                       ties, signed zeros, -inf and NaN (tests/test_oracle_routing.py).
sum_bitmatrix_rows     numpy unpackbits column sums and an exclusive cumsum of
                       per-tile sums; known answer of tests/test_moe.py:323-370.
expt_data              numpy cumsum / repeat construction; the reference test's
                       known-answer case (tests/test_moe.py:385-436).
compute_indx           numpy stable argsort (gather) and its inverse (scatter)
                       with the true per-block partials; carried == partial form.
align_block_size       numpy stable argsort per expert plus padding; the
                       reference test's own check (tests/test_moe.py:167-226).
=====================  ==========================================================
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None


def build():
    """Compile hkq_oracle.c with gcc (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        L.orc_e4m3fn_encode.restype = ctypes.c_uint8
        L.orc_e4m3fn_encode.argtypes = [ctypes.c_float]
        L.orc_e4m3fn_decode.restype = ctypes.c_float
        L.orc_e4m3fn_decode.argtypes = [ctypes.c_uint8]
        L.orc_e2m1_encode.restype = ctypes.c_uint8
        L.orc_e2m1_encode.argtypes = [ctypes.c_float]
        L.orc_e2m1_decode.restype = ctypes.c_float
        L.orc_e2m1_decode.argtypes = [ctypes.c_uint8]
        L.orc_mx_scale_exp.restype = ctypes.c_int
        L.orc_mx_scale_exp.argtypes = [ctypes.c_float]
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        L.orc_quant_rowwise.restype = None
        L.orc_quant_rowwise.argtypes = [P, I64, I64, I64, I64, ctypes.c_int, P, I64, P, I64]
        L.orc_static_fp8.restype = None
        L.orc_static_fp8.argtypes = [P, I64, ctypes.c_float, P]
        L.orc_mx_quant_fp4.restype = None
        L.orc_mx_quant_fp4.argtypes = [P, I64, I64, P, P]
        L.orc_mx_quant_fp8.restype = None
        L.orc_mx_quant_fp8.argtypes = [P, I64, I64, P, P]
        L.orc_mx_dequant.restype = None
        L.orc_mx_dequant.argtypes = [P, P, I64, I64, ctypes.c_int, P]
        L.orc_e4m3fn_decode_array.restype = None
        L.orc_e4m3fn_decode_array.argtypes = [P, I64, P]
        L.orc_mx_fp4_dequant_f32.restype = None
        L.orc_mx_fp4_dequant_f32.argtypes = [P, P, I64, I64, P]
        for name in ("orc_e4m3fn_encode_array", "orc_e2m1_encode_array", "orc_mx_scale_exp_array"):
            getattr(L, name).restype = None
            getattr(L, name).argtypes = [P, I64, P]
        I = ctypes.c_int
        L.orc_e2m1_floor_array.restype = None
        L.orc_e2m1_floor_array.argtypes = [P, I64, P]
        L.orc_rmsnorm_quant.restype = None
        L.orc_rmsnorm_quant.argtypes = [P, P, I64, I64, ctypes.c_float, I, P, P]
        L.orc_swiglu_quant.restype = None
        L.orc_swiglu_quant.argtypes = [P, I64, I64, ctypes.c_float, I, I, P, P, P]
        L.orc_topk.restype = None
        L.orc_topk.argtypes = [P, I64, I64, I64, I, I, P, P, I64, P]
        L.orc_sum_bitmatrix_rows.restype = None
        L.orc_sum_bitmatrix_rows.argtypes = [P, I64, I64, P, P]
        L.orc_expt_data.restype = None
        L.orc_expt_data.argtypes = [P, I64, I64, I64, I, I, P, P, P]
        L.orc_compute_indx.restype = None
        L.orc_compute_indx.argtypes = [P, P, I64, I, P, I64, P, P, P, P]
        L.orc_align_block_size.restype = I64
        L.orc_align_block_size.argtypes = [P, I64, I64, I64, P, P, P]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


# ----------------------------------------------------------------------------
# bf16 helpers (numpy has no bf16: bf16 tensors travel as uint16 bit patterns)
# ----------------------------------------------------------------------------

def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round fp32 to bf16 (nearest even), returned as uint16 bits."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Values of x (any float dtype) after rounding to fp32 then bf16."""
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(x, dtype=np.float32)))


# ----------------------------------------------------------------------------
# Codecs
# ----------------------------------------------------------------------------

def e4m3_encode(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().orc_e4m3fn_encode_array(_p(x), x.size, _p(out))
    return out


_E4M3_TABLE = None


def e4m3_decode(c: np.ndarray) -> np.ndarray:
    global _E4M3_TABLE
    if _E4M3_TABLE is None:
        codes = np.arange(256, dtype=np.uint8)
        out = np.empty(256, dtype=np.float32)
        lib().orc_e4m3fn_decode_array(_p(codes), 256, _p(out))
        _E4M3_TABLE = out
    return _E4M3_TABLE[np.asarray(c, dtype=np.uint8)]


def e2m1_encode(q: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.empty(q.shape, dtype=np.uint8)
    lib().orc_e2m1_encode_array(_p(q), q.size, _p(out))
    return out


def e2m1_decode(n: np.ndarray) -> np.ndarray:
    f = lib().orc_e2m1_decode
    table = np.array([f(i) for i in range(16)], dtype=np.float32)
    return table[np.asarray(n, dtype=np.uint8) & 0xF]


def mx_scale_exp(amax) -> np.ndarray:
    """Unbiased e8m0 exponent(s) of the MXFP4 scale rule for amax value(s)."""
    a = np.ascontiguousarray(amax, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.int32)
    lib().orc_mx_scale_exp_array(_p(a), a.size, _p(out))
    return out


def e8m0_decode(s: np.ndarray) -> np.ndarray:
    s = np.asarray(s, dtype=np.int32)
    v = np.ldexp(np.float32(1.0), np.minimum(s, 254) - 127).astype(np.float32)
    return np.where(s == 255, np.float32(np.nan), v)


# ----------------------------------------------------------------------------
# Quantizers (inputs: bf16 bit patterns, uint16 [M, K] C-contiguous)
# ----------------------------------------------------------------------------

def quant_rowwise(xb: np.ndarray, group: int | None = None, kind: str = "fp8"):
    """Per-token (group=None) or 1 x group quantization. Returns (q uint8
    [M,K], s float32 [M, K//group])."""
    xb = np.ascontiguousarray(xb, dtype=np.uint16)
    M, K = xb.shape
    g = K if group is None else group
    assert K % g == 0
    q = np.empty((M, K), dtype=np.uint8)
    s = np.empty((M, K // g), dtype=np.float32)
    lib().orc_quant_rowwise(_p(xb), M, K, K, g, 0 if kind == "fp8" else 1, _p(q), K, _p(s), K // g)
    return q, s


def quant_block_2d(xb: np.ndarray, block: int = 128):
    """128 x 128 block quantization of a weight matrix (DeepSeek-V3 weights):
    s[nb, kb] = max(amax(block) / 448, 1e-10), q = E4M3FN(clamp(w * (1/s)))
    -- the rule of quant/kernel.cpp:46-107 with the group taken over a 2-D
    block instead of a row. xb bf16 bits [N, K] (N, K multiples of `block`).
    Returns (q uint8 [N, K], s float32 [N/block, K/block])."""
    xb = np.ascontiguousarray(xb, dtype=np.uint16)
    N, K = xb.shape
    assert N % block == 0 and K % block == 0
    nb, kb = N // block, K // block
    blocks = xb.reshape(nb, block, kb, block).transpose(0, 2, 1, 3).reshape(nb * kb, block * block)
    q, s = quant_rowwise(np.ascontiguousarray(blocks), None, "fp8")
    q = q.reshape(nb, kb, block, block).transpose(0, 2, 1, 3).reshape(N, K)
    return np.ascontiguousarray(q), s.reshape(nb, kb)


def quant_static_fp8(xb: np.ndarray, scale: float) -> np.ndarray:
    xb = np.ascontiguousarray(xb, dtype=np.uint16)
    y = np.empty(xb.shape, dtype=np.uint8)
    lib().orc_static_fp8(_p(xb), xb.size, float(scale), _p(y))
    return y


def mx_quant_fp4(xb: np.ndarray):
    """Returns (q uint8 [M, K/2], s uint8 e8m0 [M, K/32])."""
    xb = np.ascontiguousarray(xb, dtype=np.uint16)
    M, K = xb.shape
    assert K % 32 == 0
    q = np.empty((M, K // 2), dtype=np.uint8)
    s = np.empty((M, K // 32), dtype=np.uint8)
    lib().orc_mx_quant_fp4(_p(xb), M, K, _p(q), _p(s))
    return q, s


def mx_quant_fp8(xb: np.ndarray):
    xb = np.ascontiguousarray(xb, dtype=np.uint16)
    M, K = xb.shape
    q = np.empty((M, K), dtype=np.uint8)
    s = np.empty((M, K // 32), dtype=np.uint8)
    lib().orc_mx_quant_fp8(_p(xb), M, K, _p(q), _p(s))
    return q, s


def mx_dequant(q: np.ndarray, s: np.ndarray, M: int, K: int, is_fp4: bool) -> np.ndarray:
    """bf16 bits [M, K]."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    s = np.ascontiguousarray(s, dtype=np.uint8)
    out = np.empty((M, K), dtype=np.uint16)
    lib().orc_mx_dequant(_p(q), _p(s), M, K, int(is_fp4), _p(out))
    return out


def mx_fp4_dequant_f32(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    s = np.ascontiguousarray(s, dtype=np.uint8)
    R, Kh = q.shape
    K = Kh * 2
    out = np.empty((R, K), dtype=np.float32)
    lib().orc_mx_fp4_dequant_f32(_p(q), _p(s), R, K, _p(out))
    return out


# ----------------------------------------------------------------------------
# GEMM references (fp64 accumulation of exactly decoded operands)
# ----------------------------------------------------------------------------

def gemm_a8w8_ref(A: np.ndarray, B: np.ndarray, sa: np.ndarray, sb: np.ndarray) -> np.ndarray:
    """C = (A . B^T) * sa[:,None] * sb[None,:] (tests/test_gemm.py:116) on
    e4m3fn codes A [M,K], B [N,K]; fp64 result [M, N]."""
    a = e4m3_decode(A).astype(np.float64)
    b = e4m3_decode(B).astype(np.float64)
    return (a @ b.T) * np.asarray(sa, np.float64).reshape(-1, 1) * np.asarray(sb, np.float64).reshape(1, -1)


def gemm_blockscale_ref(A, B, sa, sb, group_k: int = 128, group_n: int = 128) -> np.ndarray:
    """C = sum_kg (A_kg . B_kg^T) * sa[:, kg] * sb[kg, n // group_n]
    (gemm_a8w8_blockscale/test_parity.py:57-76; tests/test_gemm.py:148-153)."""
    a = e4m3_decode(A).astype(np.float64)
    b = e4m3_decode(B).astype(np.float64)
    M, K = a.shape
    N = b.shape[0]
    sa = np.asarray(sa, np.float64).reshape(M, -1)
    sb = np.asarray(sb, np.float64)
    sb = sb.reshape(sa.shape[1], -1)
    C = np.zeros((M, N), dtype=np.float64)
    for kg in range(sa.shape[1]):
        ks, ke = kg * group_k, min((kg + 1) * group_k, K)
        part = a[:, ks:ke] @ b[:, ks:ke].T
        bs = np.repeat(sb[kg], group_n)[:N]
        C += part * sa[:, kg:kg + 1] * bs[None, :]
    return C


# Full-output references at BASELINE sizes: the same formulas with the decoded
# operands multiplied in fp32 by torch on all host threads (seconds instead of
# minutes for 10^11-10^12 flops). Products of E4M3 / E2M1 values are exact in
# fp32; the fp32 sums differ from the fp64 ones by ~sqrt(K) * 2^-24 of the sum
# of |terms|, far inside the GEMM tolerance. Pinned against the fp64 functions
# above on small shapes (tests/test_oracle_gemm_ext.py).

def _matmul_f32(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """a [M, K] . b[N, K]^T in fp32 on the host (torch CPU, all threads)."""
    import torch
    torch.set_num_threads(max(1, len(os.sched_getaffinity(0))))
    ta = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    tb = torch.from_numpy(np.ascontiguousarray(b, dtype=np.float32))
    return (ta @ tb.T).numpy()


def gemm_a8w8_ref_f32(A, B, sa, sb) -> np.ndarray:
    """gemm_a8w8_ref with an fp32 product: float32 [M, N]."""
    C = _matmul_f32(e4m3_decode(A), e4m3_decode(B))
    C *= np.asarray(sa, np.float32).reshape(-1, 1)
    C *= np.asarray(sb, np.float32).reshape(1, -1)
    return C


def gemm_blockscale_ref_f32(A, B, sa, sb, group_k: int = 128, group_n: int = 128) -> np.ndarray:
    """gemm_blockscale_ref as one fp32 product of pre-scaled operands:
    sum_g (A_g sa[:, g]) . (B_g sb[g, n/gn])^T = (A * SA) . (B * SB)^T with
    SA[m, k] = sa[m, k/gk], SB[n, k] = sb[k/gk, n/gn] (each scaled operand
    rounds once to fp32: 2^-24 relative). float32 [M, N]."""
    a = e4m3_decode(A)
    b = e4m3_decode(B)
    M, K = a.shape
    N = b.shape[0]
    sa = np.asarray(sa, np.float32).reshape(M, -1)
    sb = np.asarray(sb, np.float32).reshape(sa.shape[1], -1)
    kidx = np.arange(K) // group_k
    a = a * sa[:, kidx]
    b = b * sb[kidx][:, np.arange(N) // group_n].T
    return _matmul_f32(a, b)


def gemm_mxfp4_ref_f32(Aq, As, Bq, Bs) -> np.ndarray:
    """gemm_mxfp4_ref with an fp32 product (decoded values are exact): float32 [M, N]."""
    return _matmul_f32(mx_fp4_dequant_f32(Aq, As), mx_fp4_dequant_f32(Bq, Bs))


def gemm_bf16_ref(A_bits, B_bits, bias_bits=None) -> np.ndarray:
    """C = A . B^T (+ bias[n]) on bf16 bit patterns A [M, K], B [N, K]
    (tests/test_gemm.py:21-42 and, with bias, :316-347); fp64 [M, N]."""
    a = bf16_bits_to_f32(np.asarray(A_bits)).astype(np.float64)
    b = bf16_bits_to_f32(np.asarray(B_bits)).astype(np.float64)
    C = a @ b.T
    if bias_bits is not None:
        C = C + bf16_bits_to_f32(np.asarray(bias_bits)).astype(np.float64).reshape(1, -1)
    return C


def batched_gemm_a8w8_ref(A, B, sa, sb, bias_bits=None) -> np.ndarray:
    """C[z] = (A[z] . B[z]^T) * sa[z][m] * sb[z][n] (+ bias[z][n]) over E4M3FN
    codes A [Z, M, K], B [Z, N, K] (tests/test_gemm.py:349-390); fp64 [Z, M, N]."""
    a = e4m3_decode(A).astype(np.float64)
    b = e4m3_decode(B).astype(np.float64)
    C = np.einsum("zmk,znk->zmn", a, b)
    Z = a.shape[0]
    C = C * np.asarray(sa, np.float64).reshape(Z, -1, 1) * np.asarray(sb, np.float64).reshape(Z, 1, -1)
    if bias_bits is not None:
        C = C + bf16_bits_to_f32(np.asarray(bias_bits)).astype(np.float64).reshape(Z, 1, -1)
    return C


def gemm_blockscale_mul_add_ref(A, B, sa, sb, ca_bits, cb_bits, group_k: int = 128, group_n: int = 128) -> np.ndarray:
    """C = c_a * G + c_b with G = gemm_blockscale_ref (unrounded), c_a / c_b
    bf16 bits [M, N] (tests/test_gemm.py:498-533); fp64 [M, N]."""
    G = gemm_blockscale_ref(A, B, sa, sb, group_k, group_n)
    ca = bf16_bits_to_f32(np.asarray(ca_bits)).astype(np.float64)
    cb = bf16_bits_to_f32(np.asarray(cb_bits)).astype(np.float64)
    return ca * G + cb


def gemm_mxfp4_ref(Aq, As, Bq, Bs) -> np.ndarray:
    """C = sum_k e2m1(a) 2^(sa-127) e2m1(b) 2^(sb-127) (moe-gemm/moe_op_mxfp4/
    kernel.cpp:191-207 with dense indexing); fp64 [M, N]."""
    a = mx_fp4_dequant_f32(Aq, As).astype(np.float64)
    b = mx_fp4_dequant_f32(Bq, Bs).astype(np.float64)
    return a @ b.T


# ----------------------------------------------------------------------------
# MoE: OGS routing metadata and the grouped GEMM reference
# ----------------------------------------------------------------------------

def ogs_routing(assigns: np.ndarray, num_experts: int, block_m: int = 128):
    """OGS metadata from top-k expert assignments [T, topk]
    (tests/test_moe.py:97-128): hist[e], offs[e] (exclusive scan), gather
    (sorted slot -> t*topk+k, token-major within an expert), expt_data
    (e | block << 16 per block_m rows)."""
    assigns = np.asarray(assigns, dtype=np.int64)
    T, topk = assigns.shape
    hist = np.bincount(assigns.ravel(), minlength=num_experts).astype(np.int32)
    offs = np.zeros(num_experts, dtype=np.int32)
    offs[1:] = np.cumsum(hist)[:-1]
    flat = assigns.ravel()  # index t*topk + k
    order = np.argsort(flat, kind="stable")  # stable: token-major within expert
    gather = order.astype(np.int32)
    tiles = []
    for e in range(num_experts):
        for b in range((int(hist[e]) + block_m - 1) // block_m):
            tiles.append(e | (b << 16))
    return hist, offs, gather, np.array(tiles, dtype=np.int32)


def moe_ref(X, W, x_scale, w_scale, bias, gather, hist, offs, expt_data, topk,
            block_m: int = 128, w_layout: str = "ekn"):
    """Y[start+gm] = (X[gather[start+gm] // topk] . W[e]) * xs * ws + bias[e]
    (tests/test_moe.py:733-753; rows gm >= hist[e] skipped, no % M wrap).

    X: e4m3 codes [T, K]; W: e4m3 codes [E, K, N] ("ekn") or [E, N, K] ("enk").
    x_scale: fp32 broadcastable to [T] (per-token) or scalar;
    w_scale: fp32 [E] (per-expert) or [E, N] (per-channel).
    Returns fp64 [T*topk, N] with untouched rows left as NaN."""
    x = e4m3_decode(X).astype(np.float64)
    w = e4m3_decode(W).astype(np.float64)
    if w_layout == "enk":
        w = np.transpose(w, (0, 2, 1))
    E, K, N = w.shape
    T = x.shape[0]
    xs = np.broadcast_to(np.asarray(x_scale, np.float64).reshape(-1), (T,)) if np.size(x_scale) in (1, T) else None
    ws = np.asarray(w_scale, np.float64)
    Y = np.full((T * topk, N), np.nan, dtype=np.float64)
    for ed in np.asarray(expt_data).tolist():
        e, b = ed & 0xFFFF, ed >> 16
        rows = [b * block_m + lm for lm in range(block_m) if b * block_m + lm < hist[e]]
        if not rows:
            continue
        sidx = offs[e] + np.array(rows)
        tok = np.asarray(gather)[sidx] // topk
        r = x[tok] @ w[e]
        r = r * xs[tok][:, None]
        r = r * (ws[e] if ws.ndim == 1 else ws[e][None, :])
        if bias is not None:
            r = r + np.asarray(bias, np.float64)[e][None, :]
        Y[sidx] = r
    return Y


def _tiles_rows(gather, hist, offs, expt_data, topk, E, block_m=128):
    """Per routing tile (e, sorted rows, tokens), skipping -1 / malformed entries."""
    out = []
    for ed in np.asarray(expt_data).tolist():
        if ed < 0 or (ed & 0xFFFF) >= E:
            continue
        e, b = ed & 0xFFFF, ed >> 16
        n = min(int(hist[e]) - b * block_m, block_m)
        if n <= 0:
            continue
        sidx = int(offs[e]) + b * block_m + np.arange(n)
        # no gather: sorted row s reads row s of X (the down projection's input)
        out.append((e, sidx, sidx if gather is None else np.asarray(gather)[sidx] // topk))
    return out


def moe_blockscale_ref(X, W, x_scale, w_scale, bias, gather, hist, offs, expt_data, topk, group_k, group_n,
                       block_m: int = 128, w_layout: str = "enk"):
    """moe-gemm/moe_op_gemm_a8w8_blockscale/kernel.cpp:93-167 restated: for each
    routing tile, Y[s, n] = sum_g (X[tok, g-part] . W[e, n, g-part]) *
    x_scale[tok, g] * w_scale[e, g, n // group_n] + bias[e, n]. X e4m3 codes
    [T, K]; W [E, N, K] ("enk") or [E, K, N] ("ekn"); x_scale [T, G];
    w_scale [E, G, ceil(N / group_n)]. fp64 [T*topk, N], untouched rows NaN."""
    x = e4m3_decode(X).astype(np.float64)
    w = e4m3_decode(W).astype(np.float64)
    if w_layout == "ekn":
        w = np.transpose(w, (0, 2, 1))
    E, N, K = w.shape
    T = x.shape[0]
    xs = np.asarray(x_scale, np.float64).reshape(T, -1)
    ws = np.asarray(w_scale, np.float64).reshape(E, xs.shape[1], -1)
    G = xs.shape[1]
    Y = np.full((T * topk, N), np.nan)
    for e, sidx, tok in _tiles_rows(gather, hist, offs, expt_data, topk, E, block_m):
        acc = np.zeros((len(sidx), N))
        for g in range(G):
            ks = slice(g * group_k, min((g + 1) * group_k, K))
            part = x[tok][:, ks] @ w[e][:, ks].T
            wcol = ws[e, g][np.arange(N) // group_n]
            acc += part * xs[tok, g][:, None] * wcol[None, :]
        if bias is not None:
            acc += np.asarray(bias, np.float64)[e][None, :]
        Y[sidx] = acc
    return Y


def moe_ref_f32(X, W, x_scale, w_scale, gather, hist, offs, expt_data, topk, group_k=None, group_n=1,
                block_m: int = 128):
    """fp32 full-output MoE reference for BASELINE sizes: per expert one fp32
    product of pre-scaled operands (W [E, N, K] e4m3 codes). x_scale: [T]
    (per token) or [T, G]; w_scale: [E, N] (per channel) or [E, G, C] with
    group_k / group_n. Rows of the listed tiles only; the rest NaN (float32)."""
    E, N, K = W.shape
    T = X.shape[0]
    gk = K if group_k is None else group_k
    xs = np.asarray(x_scale, np.float32).reshape(T, -1)      # [T, 1] or [T, G]
    ws = np.asarray(w_scale, np.float32)
    gn = 1 if ws.ndim == 2 else group_n
    ws = ws.reshape(E, 1, N) if ws.ndim == 2 else ws          # [E, 1 or G, C]
    kidx = np.arange(K) // gk
    kx = kidx if xs.shape[1] > 1 else np.zeros(K, np.int64)
    kw = kidx if ws.shape[1] > 1 else np.zeros(K, np.int64)
    Y = np.full((T * topk, N), np.nan, np.float32)
    rows = {}
    for e, sidx, tok in _tiles_rows(gather, hist, offs, expt_data, topk, E, block_m):
        s0, t0 = rows.get(e, (np.zeros(0, np.int64), np.zeros(0, np.int64)))
        rows[e] = (np.concatenate([s0, sidx]), np.concatenate([t0, tok]))
    for e, (sidx, tok) in rows.items():
        a = e4m3_decode(X[tok]) * xs[tok][:, kx]
        b = e4m3_decode(W[e]) * ws[e][kw][:, np.arange(N) // gn].T
        Y[sidx] = _matmul_f32(a, b)
    return Y


def moe_mxfp4_ref_f32(Aq, As, Bq, Bs, a_scale, b_scale, topk_w, sorted_ids, expert_ids, N, num_valid, topk,
                      mul_routed_weight, c_rows):
    """moe_mxfp4_ref with one fp32 product per expert over all of its rows
    (decoded E2M1 values are exact): float32 [c_rows, N], unwritten rows NaN."""
    a = mx_fp4_dequant_f32(Aq, As)
    E = Bq.shape[0]
    C = np.full((c_rows, N), np.nan, np.float32)
    sorted_ids = np.asarray(sorted_ids)
    per_e = {}
    for pm, e in enumerate(np.asarray(expert_ids).tolist()):
        ids = sorted_ids[pm * 128:(pm + 1) * 128]
        ids = ids[(ids >= 0) & (ids < num_valid)]
        if len(ids) == 0:
            continue
        if e == -1:
            C[ids] = 0.0
        elif 0 <= e < E:
            per_e.setdefault(e, []).append(ids)
    for e, lst in per_e.items():
        ids = np.concatenate(lst)
        r = _matmul_f32(a[ids // topk], mx_fp4_dequant_f32(Bq[e], Bs[e]))
        g = (1.0 if a_scale is None else float(np.float32(a_scale))) * (1.0 if b_scale is None else float(b_scale[e]))
        r *= np.float32(g)
        if mul_routed_weight:
            r *= np.asarray(topk_w, np.float32)[ids][:, None]
        C[ids] = r
    return C


# ----------------------------------------------------------------------------
# Quantizers fused with their producer
# ----------------------------------------------------------------------------

def e2m1_floor(x: np.ndarray) -> np.ndarray:
    """E2M1 codes of fp32 values by the reference fused quantizer's threshold
    ladder (quantization/fused_mxfp4_quant/kernel.cpp:128-150): largest grid
    magnitude at or below |x|, the sign bit of x kept, NaN -> magnitude 0."""
    a = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.zeros(a.size, np.uint8)
    lib().orc_e2m1_floor_array(_p(a), a.size, _p(out))
    return out.reshape(np.shape(x))


def rmsnorm_quant(xb: np.ndarray, wb: np.ndarray, eps: float, kind: int):
    """RMSNorm + quantization of bf16 bits [M, D] (weight bits [D]); kind 0:
    (E4M3FN codes [M, D], fp32 scales [M, D/128]); kind 1 (E2M1 elements
    rounded to nearest even) and kind 2 (floored, the reference module's
    rule): (packed E2M1 [M, D/2], e8m0 [M, D/32])."""
    x = np.ascontiguousarray(xb, dtype=np.uint16)
    w = np.ascontiguousarray(wb, dtype=np.uint16)
    M, D = x.shape
    if kind == 0:
        q = np.zeros((M, D), np.uint8)
        s = np.zeros((M, D // 128), np.float32)
    else:
        q = np.zeros((M, D // 2), np.uint8)
        s = np.zeros((M, D // 32), np.uint8)
    lib().orc_rmsnorm_quant(_p(x), _p(w), M, D, eps, kind, _p(q), _p(s))
    return q, s


def swiglu_quant(yb: np.ndarray, alpha: float = 1.0, interleaved: bool = False, group: int = 0):
    """SwiGLU + FP8 of bf16 bits [M, 2F] -> (codes [M, F], scales [M] or [M, F/128], act fp32 [M, F])."""
    y = np.ascontiguousarray(yb, dtype=np.uint16)
    M, F2 = y.shape
    F = F2 // 2
    q = np.zeros((M, F), np.uint8)
    s = np.zeros((M,) if group == 0 else (M, F // group), np.float32)
    act = np.zeros((M, F), np.float32)
    lib().orc_swiglu_quant(_p(y), M, F, alpha, int(interleaved), group, _p(q), _p(s), _p(act))
    return q, s, act


# ----------------------------------------------------------------------------
# MoE routing metadata producers (routing_oracle.c)
# ----------------------------------------------------------------------------

def _opt(a):
    return None if a is None else _p(a)


def topk(x_bits: np.ndarray, K: int, softmax: bool, bitmatrix: bool = True):
    """moe_topk: x_bits bf16 bits [rows, E] -> (Yv bf16 bits [rows, K],
    Yi int32 [rows, K], bits uint32 [rows, ceil(E/32)] or None)."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    rows, E = x.shape
    yv = np.zeros((rows, K), np.uint16)
    yi = np.zeros((rows, K), np.int32)
    bits = np.zeros((rows, (E + 31) // 32), np.uint32) if bitmatrix else None
    lib().orc_topk(_p(x), E, rows, E, K, int(softmax), _p(yv), _p(yi), K, _opt(bits))
    return yv, yi, bits


def sum_bitmatrix_rows(bits: np.ndarray, partials: bool = True):
    """bits uint32 [rows, nwords] -> (ret uint32 [32*nwords], partials uint32
    [ceil(rows/128), 32*nwords] (exclusive over 128-row tiles) or None)."""
    b = np.ascontiguousarray(bits, dtype=np.uint32)
    rows, nw = b.shape
    ret = np.zeros(32 * nw, np.uint32)
    part = np.zeros(((rows + 127) // 128, 32 * nw), np.uint32) if partials else None
    lib().orc_sum_bitmatrix_rows(_p(b), rows, nw, _p(ret), _opt(part))
    return ret, part


def expt_data(hist: np.ndarray, max_tiles: int, n_gates: int, log2: int, mode: int, md_init: int = 0x5A5A5A5A):
    """mode 0: stage 1; 1: stage 1 + 2; 2: stage 1 + fused stage 2.
    Returns (token_start [E+1], tile_start [E+1], md uint32 [max_tiles]) with md
    pre-filled with md_init where the mode writes nothing."""
    h = np.ascontiguousarray(hist, dtype=np.int32)
    E = h.shape[0]
    ts = np.zeros(E + 1, np.int32)
    tl = np.zeros(E + 1, np.int32)
    md = np.full(max(max_tiles, 1), md_init, np.uint32)
    lib().orc_expt_data(_p(h), E, max_tiles, n_gates, log2, mode, _p(ts), _p(tl), _p(md))
    return ts, tl, md[:max_tiles]


def compute_indx(indx: np.ndarray, scal_bits, K: int, tokens_start: np.ndarray, partial_offs=None,
                 n_slots: int | None = None):
    """routing_compute_indx over flattened gates indx [n_gates]; partial_offs
    int32 [nblocks, E] or None (counts carried). Returns (gather [n_slots],
    scatter [n_gates], gate_scal bits [n_slots] or None); untouched gather
    slots hold -7."""
    ind = np.ascontiguousarray(indx, dtype=np.int32).ravel()
    n = ind.shape[0]
    n_slots = n if n_slots is None else n_slots
    ts = np.ascontiguousarray(tokens_start, dtype=np.int32)
    gather = np.full(max(n_slots, 1), -7, np.int32)
    scatter = np.zeros(max(n, 1), np.int32)
    sc = None if scal_bits is None else np.ascontiguousarray(scal_bits, dtype=np.uint16).ravel()
    gs = None if sc is None else np.zeros(max(n_slots, 1), np.uint16)
    po = None if partial_offs is None else np.ascontiguousarray(partial_offs, dtype=np.int32)
    E = 0 if po is None else po.shape[1]
    lib().orc_compute_indx(_p(ind), _opt(sc), n, K, _opt(po), E, _p(ts), _p(gather), _p(scatter), _opt(gs))
    return gather[:n_slots], scatter[:n], (None if gs is None else gs[:n_slots])


def align_block_size(ids: np.ndarray, E: int, bs: int):
    """moe_align_block_size -> (sorted [total], expert_ids [total/bs], cumsum [E+1], total)."""
    x = np.ascontiguousarray(ids, dtype=np.int32).ravel()
    n = x.shape[0]
    cap = n + E * (bs - 1) + 1
    sorted_ = np.zeros(cap, np.int32)
    eids = np.zeros(cap // bs + 1, np.int32)
    cum = np.zeros(E + 1, np.int32)
    total = int(lib().orc_align_block_size(_p(x), n, E, bs, _p(sorted_), _p(eids), _p(cum)))
    return sorted_[:total], eids[: total // bs], cum, total


def moe_mxfp4_ref(Aq, As, Bq, Bs, a_scale, b_scale, topk_w, sorted_ids, expert_ids, N, num_valid, topk,
                  mul_routed_weight, c_rows):
    """The MXFP4 MoE of moe-gemm/moe_op_mxfp4/kernel.cpp:90-237 on the block-sorted
    routing of moe_align_block_size: for 128-row block pm with expert e =
    expert_ids[pm] and row id = sorted_ids[pm*128 + r] < num_valid,
    C[id] = (A[id // topk] . B[e]^T) * a_scale * b_scale[e] * (w[id] if mul), or 0
    when e == -1. Aq [T, K/2], As [T, K/32], Bq [E, N, K/2], Bs [E, N, K/32]
    (K contiguous). fp64 [c_rows, N], rows never written are NaN."""
    a = mx_fp4_dequant_f32(Aq, As).astype(np.float64)
    E = Bq.shape[0]
    b = [mx_fp4_dequant_f32(Bq[e], Bs[e]).astype(np.float64) for e in range(E)]
    C = np.full((c_rows, N), np.nan)
    sorted_ids = np.asarray(sorted_ids)
    for pm, e in enumerate(np.asarray(expert_ids).tolist()):
        ids = sorted_ids[pm * 128:(pm + 1) * 128]
        ids = ids[(ids >= 0) & (ids < num_valid)]
        if len(ids) == 0:
            continue
        if e == -1:
            C[ids] = 0.0
            continue
        r = a[ids // topk] @ b[e].T
        g = (1.0 if a_scale is None else float(np.float32(a_scale))) * (1.0 if b_scale is None else float(b_scale[e]))
        r = r * g
        if mul_routed_weight:
            r = r * np.asarray(topk_w, np.float64)[ids][:, None]
        C[ids] = r
    return C


# ----------------------------------------------------------------------------
# Input generation (seeded CPU generator, so CPU and GPU see identical bytes)
# ----------------------------------------------------------------------------

def randn_bf16(shape, std: float = 1.0, seed: int = 0) -> np.ndarray:
    """bf16 bits of N(0, std) drawn with torch's CPU generator."""
    import torch
    g = torch.Generator(device="cpu").manual_seed(seed)
    t = (torch.randn(*shape, generator=g, dtype=torch.float32) * std).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16).copy()
