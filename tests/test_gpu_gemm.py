"""GPU parity of the dense GEMMs against the CPU oracle, through the C ABI.

Bar (north star): bf16 C within |C - ref| <= 2e-2 + 1e-2 |ref| of the fp64
dequant matmul of the same codes and scales, and Frobenius relative error
< 1e-2. Inputs follow BASELINE's distributions (acts ~N(0,1), weights
~N(0,0.02)) through the oracle quantizers, so the GEMM test does not depend on
the GPU quantizer. Small shapes and every BASELINE size (the A8W8 headline and 20-shape sweep,
both MXFP4 sizes, the three block-scale shapes) are compared in full, the
latter against fp32 products of the decoded operands; plus closed forms.
"""
import numpy as np
import pytest
import torch

import hkq
from gpu_util import assert_gemm_close, dev_f32, dev_u8, host_bf16_f32, require_gpu

pytestmark = pytest.mark.gpu


def a8w8_inputs(orc, M, N, K, seed):
    xa = orc.randn_bf16((M, K), seed=seed)
    xw = orc.randn_bf16((N, K), seed=seed + 1, std=0.02)
    A, sa = orc.quant_rowwise(xa, None, "fp8")
    B, sb = orc.quant_rowwise(xw, None, "fp8")
    return A, B, sa.reshape(-1), sb.reshape(-1)


def run_a8w8(A, B, sa, sb):
    C = hkq.gemm_a8w8(dev_u8(A), dev_u8(B), dev_f32(sa), dev_f32(sb))
    torch.cuda.synchronize()
    return host_bf16_f32(C)


A8W8_SHAPES = [(256, 256, 64), (256, 256, 128), (1, 256, 256), (16, 512, 512), (100, 260, 4160), (333, 1000, 576),
               (513, 772, 1088), (128, 4096, 4096), (1024, 1024, 2048), (300, 300, 320)]


@pytest.mark.parametrize("M,N,K", A8W8_SHAPES)
def test_gemm_a8w8(orc, M, N, K):
    require_gpu()
    A, B, sa, sb = a8w8_inputs(orc, M, N, K, seed=M + N + K)
    C = run_a8w8(A, B, sa, sb)
    assert_gemm_close(C, orc.gemm_a8w8_ref(A, B, sa, sb), f"a8w8 {M}x{N}x{K}")


def test_gemm_a8w8_closed_form(orc):
    """All codes 1.0 (0x38): C = K * sa[m] * sb[n] exactly representable pattern."""
    require_gpu()
    M, N, K = 300, 516, 1024
    rng = np.random.default_rng(1)
    sa = (rng.integers(1, 8, M) / 64).astype(np.float32)
    sb = (rng.integers(1, 8, N) / 64).astype(np.float32)
    C = run_a8w8(np.full((M, K), 0x38, np.uint8), np.full((N, K), 0x38, np.uint8), sa, sb)
    assert np.array_equal(C, (K * sa[:, None].astype(np.float64) * sb[None, :]).astype(np.float32))


def test_gemm_a8w8_strided_and_out_of_place_rows(orc):
    """lda/ldb/ldc larger than K/N; bytes outside the logical matrices untouched."""
    require_gpu()
    M, N, K = 200, 132, 384
    A, B, sa, sb = a8w8_inputs(orc, M, N, K, seed=77)
    Ad = torch.zeros((M, K + 128), dtype=torch.uint8, device="cuda")
    Bd = torch.zeros((N, K + 64), dtype=torch.uint8, device="cuda")
    Ad[:, :K] = dev_u8(A)
    Bd[:, :K] = dev_u8(B)
    Cd = torch.full((M, N + 12), 7.0, dtype=torch.bfloat16, device="cuda")
    sad, sbd = dev_f32(sa), dev_f32(sb)  # keep the tensors alive while the kernel reads them
    hkq.call("hkq_gemm_a8w8", Ad.data_ptr(), Bd.data_ptr(), sad.data_ptr(), sbd.data_ptr(),
             Cd.data_ptr(), M, N, K, K + 128, K + 64, N + 12, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    C = host_bf16_f32(Cd)
    assert_gemm_close(C[:, :N], orc.gemm_a8w8_ref(A, B, sa, sb), "strided")
    assert np.all(C[:, N:] == 7.0)


# Full-output parity at every BASELINE A8W8 size: the headline shape and the
# 20-shape sweep (N, K) x M, each checked element by element against the fp32
# dequant matmul of the same codes (oracle.gemm_a8w8_ref_f32, pinned against
# the fp64 reference in tests/test_oracle_gemm_ext.py). These shapes select
# every A8W8 plan: narrow (M <= 16), skinny / 128 x 64 tiles with split K
# (M = 128), 128 x 128 tiles (M = 1024) and 256 x 256 tiles (M = 4096).
SWEEP_NK = [(6144, 4096), (4096, 4096), (28672, 4096), (4096, 14336)]
SWEEP_M = [1, 16, 128, 1024, 4096]
BASELINE_A8W8 = [(4096, 14336, 4096)] + [(M, N, K) for (N, K) in SWEEP_NK for M in SWEEP_M]

_weight_cache = {}


def _weights(orc, N, K, seed):
    """Per-channel FP8 weights ~N(0, 0.02), shared by the sweep's M values."""
    key = (N, K, seed)
    if key not in _weight_cache:
        _weight_cache.clear()
        B, sb = orc.quant_rowwise(orc.randn_bf16((N, K), seed=seed, std=0.02), None, "fp8")
        _weight_cache[key] = (B, sb.reshape(-1))
    return _weight_cache[key]


@pytest.mark.parametrize("M,N,K", BASELINE_A8W8)
def test_gemm_a8w8_baseline_sizes_full(orc, M, N, K):
    require_gpu()
    A, sa = orc.quant_rowwise(orc.randn_bf16((M, K), seed=M + K), None, "fp8")
    sa = sa.reshape(-1)
    B, sb = _weights(orc, N, K, seed=N + K + 1)
    C = run_a8w8(A, B, sa, sb)
    assert_gemm_close(C, orc.gemm_a8w8_ref_f32(A, B, sa, sb), f"a8w8 {M}x{N}x{K}")


# Smaller-tile and split-K plans: M <= 64 uses (32 or 64) x 256 tiles, few
# 256 x 256 tiles become 128 x 128 tiles (128 x 64 for FP8 with M <= 128 and
# K <= 8192), and if those are still few (with a long enough K) K is split
# into fp32 partials that the last split of each tile to finish adds up.
SPLIT_SHAPES = [(1, 4096, 14336), (16, 2048, 4096), (48, 1024, 2048), (128, 4096, 4096), (96, 28672, 4096), (24, 28672, 4096),
                (1024, 4096, 14336), (640, 1000, 8192), (256, 1024, 8192), (300, 2052, 2048), (100, 1000, 2048),
                (128, 6144, 4096)]


@pytest.mark.parametrize("M,N,K", SPLIT_SHAPES)
def test_gemm_a8w8_split_and_skinny(orc, M, N, K):
    """The split plan and the same shape through the plain entry point (no
    workspace) both agree with the oracle on every output element."""
    require_gpu()
    A, B, sa, sb = a8w8_inputs(orc, M, N, K, seed=M + 3 * N + K)
    Ad, Bd, sad, sbd = dev_u8(A), dev_u8(B), dev_f32(sa), dev_f32(sb)
    C1 = hkq.gemm_a8w8(Ad, Bd, sad, sbd)
    C0 = hkq.gemm_a8w8(Ad, Bd, sad, sbd, split=False)
    torch.cuda.synchronize()
    ref = orc.gemm_a8w8_ref_f32(A, B, sa, sb)
    assert_gemm_close(host_bf16_f32(C1), ref, f"a8w8 split {M}x{N}x{K}")
    assert_gemm_close(host_bf16_f32(C0), ref, f"a8w8 unsplit {M}x{N}x{K}")


def _a8w8_ws_launcher(Ad, Bd, sad, sbd, C, ws):
    M, K = Ad.shape
    N = Bd.shape[0]
    return lambda: hkq.call("hkq_gemm_a8w8_ws", Ad.data_ptr(), Bd.data_ptr(), sad.data_ptr(), sbd.data_ptr(),
                            C.data_ptr(), M, N, K, K, K, N, ws.data_ptr(), ws.numel(),
                            torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("M,N,K", [(128, 4096, 4096), (64, 4096, 14336), (1024, 1024, 8192)])
def test_gemm_a8w8_split_workspace_states(orc, M, N, K):
    """The split plan's per-tile arrival counters live in the workspace and
    need no clearing: a workspace full of 0xFF bytes, one left by a call of
    another shape, and the same call repeated all give the same bytes, which
    match the oracle (the partials are added in split order, whichever split
    finishes last)."""
    require_gpu()
    A, B, sa, sb = a8w8_inputs(orc, M, N, K, seed=M + N + K + 5)
    Ad, Bd, sad, sbd = dev_u8(A), dev_u8(B), dev_f32(sa), dev_f32(sb)
    need = hkq.lib().hkq_gemm_a8w8_workspace(M, N, K)
    assert need > 0
    ws = torch.full((need + (1 << 20),), 0xFF, dtype=torch.uint8, device="cuda")
    C = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    run = _a8w8_ws_launcher(Ad, Bd, sad, sbd, C, ws)
    run()
    torch.cuda.synchronize()
    first = C.clone()
    assert_gemm_close(host_bf16_f32(first), orc.gemm_a8w8_ref_f32(A, B, sa, sb), f"a8w8 split {M}x{N}x{K}")
    # another shape's split plan on the same workspace, then this one again, twice
    A2, B2, sa2, sb2 = a8w8_inputs(orc, 96, 2048, 4096, seed=9)
    C2 = torch.empty((96, 2048), dtype=torch.bfloat16, device="cuda")
    _a8w8_ws_launcher(dev_u8(A2), dev_u8(B2), dev_f32(sa2), dev_f32(sb2), C2, ws)()
    for _ in range(2):
        C.fill_(0)
        run()
        torch.cuda.synchronize()
        assert torch.equal(C.view(torch.int16), first.view(torch.int16))


def test_gemm_a8w8_split_graph_replay(orc):
    """A split GEMM captured in a HIP graph replays with one tag: every replay
    (with eager work and synchronization between them) equals the eager call."""
    require_gpu()
    M, N, K = 128, 4096, 4096
    A, B, sa, sb = a8w8_inputs(orc, M, N, K, seed=77)
    Ad, Bd, sad, sbd = dev_u8(A), dev_u8(B), dev_f32(sa), dev_f32(sb)
    ws = torch.empty((hkq.lib().hkq_gemm_a8w8_workspace(M, N, K),), dtype=torch.uint8, device="cuda")
    C = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    run = _a8w8_ws_launcher(Ad, Bd, sad, sbd, C, ws)
    run()
    torch.cuda.synchronize()
    eager = C.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            run()
    torch.cuda.current_stream().wait_stream(s)
    for i in range(4):
        C.fill_(0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(C.view(torch.int16), eager.view(torch.int16)), f"replay {i}"
        run()  # an eager call (a new tag) between replays
        torch.cuda.synchronize()
        assert torch.equal(C.view(torch.int16), eager.view(torch.int16))


def test_gemm_workspace_plans():
    """Shapes that fill the GPU and the narrow (M <= 16) path need no
    workspace; underfilled tiled shapes do."""
    require_gpu()
    L = hkq.lib()
    assert L.hkq_gemm_a8w8_workspace(4096, 14336, 4096) == 0
    assert L.hkq_gemm_a8w8_workspace(16, 4096, 14336) == 0
    assert L.hkq_gemm_a8w8_workspace(64, 4096, 14336) > 0
    assert L.hkq_gemm_a8w8_workspace(256, 1024, 8192) > 0
    assert L.hkq_gemm_mxfp4_workspace(4096, 8192, 8192) == 0
    assert L.hkq_gemm_mxfp4_workspace(16, 8192, 8192) == 0
    assert L.hkq_gemm_mxfp4_workspace(64, 8192, 8192) > 0


# Narrow path (M <= 16, and M <= 32 with few columns and a short K): one
# workgroup per 16 * NT columns, K split over its 4 waves (S = K/128 steps,
# S < 4 leaves waves idle), NT = 1, 2 or 4 by the number of workgroups,
# ragged N (rows past N read as zeros), ragged M.
NARROW_SHAPES = [(1, 16, 128), (1, 64, 640), (5, 1000, 4096), (16, 4096, 4096), (13, 6144, 256), (16, 28672, 512),
                 (32, 4096, 4096), (20, 6000, 1024), (3, 200, 384)]


@pytest.mark.parametrize("M,N,K", NARROW_SHAPES)
def test_gemm_a8w8_narrow(orc, M, N, K):
    require_gpu()
    A, B, sa, sb = a8w8_inputs(orc, M, N, K, seed=11 * M + N + K)
    C = run_a8w8(A, B, sa, sb)
    assert_gemm_close(C, orc.gemm_a8w8_ref(A, B, sa, sb), f"a8w8 narrow {M}x{N}x{K}")


def test_gemm_a8w8_narrow_strided(orc):
    """Narrow path with lda/ldb/ldc past K/N: bytes outside C untouched."""
    require_gpu()
    M, N, K = 7, 40, 512
    A, B, sa, sb = a8w8_inputs(orc, M, N, K, seed=78)
    Ad = torch.zeros((M, K + 256), dtype=torch.uint8, device="cuda")
    Bd = torch.zeros((N, K + 48), dtype=torch.uint8, device="cuda")
    Ad[:, :K] = dev_u8(A)
    Bd[:, :K] = dev_u8(B)
    Cd = torch.full((M, N + 20), 5.0, dtype=torch.bfloat16, device="cuda")
    sad, sbd = dev_f32(sa), dev_f32(sb)
    hkq.call("hkq_gemm_a8w8", Ad.data_ptr(), Bd.data_ptr(), sad.data_ptr(), sbd.data_ptr(),
             Cd.data_ptr(), M, N, K, K + 256, K + 48, N + 20, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    C = host_bf16_f32(Cd)
    assert_gemm_close(C[:, :N], orc.gemm_a8w8_ref(A, B, sa, sb), "narrow strided")
    assert np.all(C[:, N:] == 5.0)


def mx_inputs(orc, M, N, K, seed):
    xa = orc.randn_bf16((M, K), seed=seed)
    xw = orc.randn_bf16((N, K), seed=seed + 1, std=0.02)
    Aq, As = orc.mx_quant_fp4(xa)
    Bq, Bs = orc.mx_quant_fp4(xw)
    return Aq, As, Bq, Bs


def run_mxfp4(Aq, As, Bq, Bs):
    C = hkq.gemm_mxfp4(dev_u8(Aq), dev_u8(As), dev_u8(Bq), dev_u8(Bs))
    torch.cuda.synchronize()
    return host_bf16_f32(C)


@pytest.mark.parametrize("M,N,K", [(256, 256, 128), (256, 256, 256), (1, 256, 512), (128, 512, 8192), (77, 300, 768),
                                   (600, 1028, 1536), (260, 264, 384), (7, 1000, 256), (16, 8192, 1024), (32, 2048, 4096),
                                   (2, 48, 128)])
def test_gemm_mxfp4(orc, M, N, K):
    require_gpu()
    Aq, As, Bq, Bs = mx_inputs(orc, M, N, K, seed=M * 7 + K)
    C = run_mxfp4(Aq, As, Bq, Bs)
    assert_gemm_close(C, orc.gemm_mxfp4_ref(Aq, As, Bq, Bs), f"mxfp4 {M}x{N}x{K}")


def test_gemm_mxfp4_closed_form_scales(orc):
    """Elements 1.0, per-block scales 2^(r%5 - 2) on A and 2^(c%3 - 1) on B:
    C[m, n] = sum_blocks 32 * sA * sB is exact in fp32, so the bf16 output is
    exactly that sum rounded to nearest even."""
    require_gpu()
    M, N, K = 256, 256, 1024
    Aq = np.full((M, K // 2), 0x22, np.uint8)
    Bq = np.full((N, K // 2), 0x22, np.uint8)
    As = (127 + (np.arange(M)[:, None] + np.arange(K // 32)[None, :]) % 5 - 2).astype(np.uint8)
    Bs = (127 + (np.arange(N)[:, None] * 3 + np.arange(K // 32)[None, :]) % 3 - 1).astype(np.uint8)
    C = run_mxfp4(Aq, As, Bq, Bs)
    ref = orc.bf16_round(orc.gemm_mxfp4_ref(Aq, As, Bq, Bs))
    assert np.array_equal(C, ref)


@pytest.mark.parametrize("M", [128, 4096])
def test_gemm_mxfp4_baseline_sizes_full(orc, M):
    """BASELINE MXFP4 sizes, every output element against the fp32 product of
    the decoded operands (oracle.gemm_mxfp4_ref_f32)."""
    require_gpu()
    N = K = 8192
    Aq, As, Bq, Bs = mx_inputs(orc, M, N, K, seed=M)
    C = run_mxfp4(Aq, As, Bq, Bs)
    assert_gemm_close(C, orc.gemm_mxfp4_ref_f32(Aq, As, Bq, Bs), f"mxfp4 {M}x{N}x{K}")


# ---------------------------------------------------------------------------
# Block-scale FP8 GEMM (1x128 activation scales, 128x128 or 128x1 weight scales)
# ---------------------------------------------------------------------------

def blockscale_inputs(orc, M, N, K, seed, group_n):
    xa = orc.randn_bf16((M, K), seed=seed)
    A, sa = orc.quant_rowwise(xa, 128, "fp8")              # [M, K/128]
    Np = (N + 127) // 128 * 128
    xw = orc.randn_bf16((Np, K), seed=seed + 1, std=0.02)
    if group_n == 128:
        B, sbt = orc.quant_block_2d(xw)                    # sbt [N/128, K/128]
        sb = np.ascontiguousarray(sbt.T)                   # [K/128, N/128]
    else:
        B, sbr = orc.quant_rowwise(xw, 128, "fp8")         # per (n, k-group)
        sb = np.ascontiguousarray(sbr.T)                   # [K/128, N]
    return A, np.ascontiguousarray(B[:N]), sa, (sb if group_n == 128 else np.ascontiguousarray(sb[:, :N]))


def run_blockscale(A, B, sa, sb, group_n):
    C = hkq.gemm_blockscale(dev_u8(A), dev_u8(B), dev_f32(sa), dev_f32(sb), group_n=group_n)
    torch.cuda.synchronize()
    return host_bf16_f32(C)


# (1, 256, 1024) and M <= 64 below run the narrow block-scale kernel: 16-row
# tiles (MT = 1, 2, 4), 16- or 32-column slices (N/16 > CUs), one K group
# (S = 1 < 4 waves), ragged N; (100, 1000, 512) and (192, 2112, 1024) run it in
# row groups of 64 (few 256 x 256 tiles).
@pytest.mark.parametrize("group_n", [128, 1])
@pytest.mark.parametrize("M,N,K", [(128, 128, 256), (256, 256, 128), (333, 516, 384), (1, 256, 1024),
                                   (600, 772, 2048), (5, 1000, 512), (16, 4160, 1536), (20, 136, 128),
                                   (33, 300, 384), (64, 516, 640), (100, 1000, 512), (192, 2112, 1024)])
def test_gemm_blockscale(orc, M, N, K, group_n):
    require_gpu()
    A, B, sa, sb = blockscale_inputs(orc, M, N, K, M + N + K, group_n)
    C = run_blockscale(A, B, sa, sb, group_n)
    assert_gemm_close(C, orc.gemm_blockscale_ref(A, B, sa, sb, 128, group_n), f"blockscale {M}x{N}x{K} gn{group_n}")


# The tiled kernel with C rows 16-byte aligned: C with a row pitch of N + pad
# (a multiple of 8) whose extra columns must stay untouched, N % 8 == 4 (the
# last 16-byte piece of a row straddles N) and ragged M.
@pytest.mark.parametrize("M,N,K,pad,group_n", [(600, 772, 2048, 4, 128), (333, 516, 384, 12, 1),
                                               (520, 1028, 256, 4, 1)])
def test_gemm_blockscale_padded_rows(orc, M, N, K, pad, group_n):
    require_gpu()
    A, B, sa, sb = blockscale_inputs(orc, M, N, K, M + N + K + 7, group_n)
    sentinel = 7.0
    Cp = torch.full((M, N + pad), sentinel, dtype=torch.bfloat16, device="cuda")
    C = hkq.gemm_blockscale(dev_u8(A), dev_u8(B), dev_f32(sa), dev_f32(sb), Cp[:, :N], group_n=group_n)
    torch.cuda.synchronize()
    assert bool((Cp[:, N:] == sentinel).all()), "stores past N reached the row padding"
    assert_gemm_close(host_bf16_f32(C), orc.gemm_blockscale_ref(A, B, sa, sb, 128, group_n),
                      f"blockscale padded {M}x{N}x{K} gn{group_n}")


# Tile widths: grids that 256-column tiles leave a CU short run 256 x 224
# tiles (waves 4-7 with three n-tiles); HKQ_BLOCKSCALE_W224=0 forces 256-column
# tiles. Both compute every element with the same K steps and promotions, so
# their outputs agree bit for bit. Shapes: ragged N (1000 = 4*224 + 104: the
# last tile's waves 4-7 lie wholly past N), a 128-block boundary inside a
# 224-column tile (GN 128), per-column scales, and the 2048 x 7168 BASELINE grid.
@pytest.mark.parametrize("M,N,K,group_n", [(256, 1000, 512, 1), (600, 772, 2048, 128), (333, 516, 384, 1),
                                           (520, 1792, 640, 128), (2048, 7168, 2048, 128)])
def test_gemm_blockscale_tile_widths(orc, monkeypatch, M, N, K, group_n):
    require_gpu()
    A, B, sa, sb = blockscale_inputs(orc, M, N, K, M + N + K + 11, group_n)
    C224 = run_blockscale(A, B, sa, sb, group_n)
    monkeypatch.setenv("HKQ_BLOCKSCALE_W224", "0")
    C256 = run_blockscale(A, B, sa, sb, group_n)
    assert np.array_equal(C224, C256), f"tile widths disagree {M}x{N}x{K} gn{group_n}"
    assert_gemm_close(C224, orc.gemm_blockscale_ref_f32(A, B, sa, sb, 128, group_n), f"blockscale {M}x{N}x{K}")


def test_gemm_blockscale_uniform_scales_reduce_to_a8w8(orc):
    """Scales constant over K groups: the block-scale GEMM equals the A8W8 GEMM
    with the same per-row / per-column factors."""
    require_gpu()
    M, N, K = 256, 512, 1024
    A, B, sa1, sb1 = a8w8_inputs(orc, M, N, K, seed=5)
    sa = np.repeat(sa1[:, None], K // 128, axis=1).astype(np.float32)
    sb = np.repeat(sb1[None, :], K // 128, axis=0).astype(np.float32)
    C = run_blockscale(A, B, sa, sb, 1)
    assert_gemm_close(C, orc.gemm_a8w8_ref(A, B, sa1, sb1), "blockscale uniform")


@pytest.mark.parametrize("N,K", [(24576, 1536), (7168, 18432), (7168, 2048)])
def test_gemm_blockscale_baseline_sizes_full(orc, N, K):
    """The three DeepSeek-V3 shapes at M = 2048 (plus M = 1 and 16 on the
    narrow path), every output element against oracle.gemm_blockscale_ref_f32."""
    require_gpu()
    for M in (2048, 16, 1):
        A, B, sa, sb = blockscale_inputs(orc, M, N, K, K + M, 128)
        C = run_blockscale(A, B, sa, sb, 128)
        assert_gemm_close(C, orc.gemm_blockscale_ref_f32(A, B, sa, sb, 128, 128), f"blockscale {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(1, 4096, 8192), (32, 2048, 8192), (128, 8192, 8192), (512, 1024, 16384)])
def test_gemm_mxfp4_split_and_skinny(orc, M, N, K):
    require_gpu()
    Aq, As, Bq, Bs = mx_inputs(orc, M, N, K, seed=M + K + 5)
    args = [dev_u8(a) for a in (Aq, As, Bq, Bs)]
    C1 = hkq.gemm_mxfp4(*args)
    C0 = hkq.gemm_mxfp4(*args, split=False)
    torch.cuda.synchronize()
    ref = orc.gemm_mxfp4_ref_f32(Aq, As, Bq, Bs)
    assert_gemm_close(host_bf16_f32(C1), ref, f"mxfp4 split {M}x{N}x{K}")
    assert_gemm_close(host_bf16_f32(C0), ref, f"mxfp4 unsplit {M}x{N}x{K}")


# The persistent streaming kernel (256 x 256 tiles with K a multiple of 1024
# bytes, C's rows 16-byte aligned): several tiles per workgroup, the last round
# as M halves, ragged M and N at the grid edge (N % 8 == 4: the last 16-byte
# store of a row straddles N), the minimum of 8 K-tiles per tile, and a round
# count that leaves some workgroups one tile short; every output element
# against the oracle. pad > 0 gives C a row pitch of N + pad (a multiple of 8,
# so the streaming kernel takes it) whose extra columns must stay untouched;
# pad == 0 with N % 8 == 4 takes the one-tile-per-workgroup kernel.
@pytest.mark.parametrize("M,N,K,pad", [(4000, 14300, 4096, 4), (4000, 14300, 4096, 0), (4608, 14336, 1024, 0),
                                       (3000, 8196, 2048, 12), (8192, 4100, 1024, 4)])
def test_gemm_a8w8_stream_tiles(orc, M, N, K, pad):
    require_gpu()
    A, B, sa, sb = a8w8_inputs(orc, M, N, K, seed=M + N + K + 1)
    sentinel = 7.0
    Cp = torch.full((M, N + pad), sentinel, dtype=torch.bfloat16, device="cuda")
    C = hkq.gemm_a8w8(dev_u8(A), dev_u8(B), dev_f32(sa), dev_f32(sb), Cp[:, :N])
    torch.cuda.synchronize()
    if pad:
        assert bool((Cp[:, N:] == sentinel).all()), "stores past N reached the row padding"
    assert_gemm_close(host_bf16_f32(C), orc.gemm_a8w8_ref_f32(A, B, sa, sb), f"a8w8 stream {M}x{N}x{K} pad {pad}")


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 512), (8200, 4096, 1024)])
def test_gemm_bf16_stream_tiles(orc, M, N, K):
    require_gpu()
    A = orc.randn_bf16((M, K), seed=M)
    B = orc.randn_bf16((N, K), seed=N + 1)
    from gpu_util import dev_bf16
    C = hkq.gemm_bf16(dev_bf16(A), dev_bf16(B))
    torch.cuda.synchronize()
    a = torch.from_numpy(orc.bf16_bits_to_f32(A))
    b = torch.from_numpy(orc.bf16_bits_to_f32(B))
    assert_gemm_close(host_bf16_f32(C), (a @ b.T).numpy(), f"bf16 stream {M}x{N}x{K}")
