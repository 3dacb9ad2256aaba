"""GPU parity of the MXFP4 MoE GEMM (block-sorted routing) against the CPU
oracle (oracle.moe_mxfp4_ref: moe-gemm/moe_op_mxfp4/kernel.cpp:90-237
restated over exactly decoded operands), through the C ABI and the
reference-named module. Bar: the north-star GEMM tolerance on every written
row; rows no block names stay untouched."""
import numpy as np
import pytest
import torch

import hkq
from gpu_util import assert_gemm_close, dev_f32, dev_u8, require_gpu

pytestmark = pytest.mark.gpu


def dev_i32(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()


def routed(orc, T, E, topk, seed):
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.permutation(E)[:topk] for _ in range(T)]).astype(np.int32).ravel()
    s, eids, _, total = orc.align_block_size(ids, E, 128)
    return ids, s, eids


def problem(orc, T, E, K, N, seed):
    Aq, As = orc.mx_quant_fp4(orc.randn_bf16((T, K), seed=seed))
    Bq, Bs = orc.mx_quant_fp4(orc.randn_bf16((E * N, K), seed=seed + 1, std=0.05))
    return Aq, As, Bq.reshape(E, N, K // 2), Bs.reshape(E, N, K // 32)


# (1, ...) and (16, ...) have at most 32 valid gate ids and a small tiled grid:
# the decode (streaming) kernel, with K-steps uneven over its 4 waves and 16
# columns per workgroup, or 64 (N > 4096: (1, 8, 2, 512, 8192));
# (5, 8, 2, 384, 4160) has few ids but a large tiled grid, so it stays tiled.
@pytest.mark.parametrize("T,E,topk,K,N", [(64, 8, 2, 256, 256), (1024, 8, 2, 2048, 1024), (300, 4, 1, 384, 520),
                                          (77, 16, 4, 512, 64), (1, 8, 2, 256, 512), (5, 8, 2, 384, 4160),
                                          (16, 8, 2, 640, 1000), (1, 8, 2, 512, 8192), (2, 8, 2, 384, 4400)])
def test_moe_mxfp4(orc, T, E, topk, K, N):
    require_gpu()
    Aq, As, Bq, Bs = problem(orc, T, E, K, N, T + K)
    ids, s, eids = routed(orc, T, E, topk, T)
    rng = np.random.default_rng(5)
    w = rng.random(T * topk).astype(np.float32)
    bsc = (rng.random(E) * 0.5 + 0.5).astype(np.float32)
    C = hkq.moe_mxfp4(dev_u8(Aq), dev_u8(As), dev_u8(Bq), dev_u8(Bs), dev_i32(s), dev_i32(eids), T * topk, topk,
                      a_scale=dev_f32([0.75]), b_scale=dev_f32(bsc), topk_weights=dev_f32(w))
    torch.cuda.synchronize()
    ref = orc.moe_mxfp4_ref(Aq, As, Bq, Bs, 0.75, bsc, w, s, eids, N, T * topk, topk, True, T * topk)
    assert not np.isnan(ref).any()
    assert_gemm_close(C.float().cpu().numpy(), ref, "moe mxfp4")


@pytest.mark.parametrize("N", [9216, 11264])
def test_moe_mxfp4_whole_and_split_tiles(orc, N):
    """Enough 256-column tiles that most run as whole pairs of blocks while the
    sparse last round runs block by block: on 256 CUs, 8 pairs x 36 = 288
    tiles = 256 + 32 and 8 pairs x 44 = 352 = 256 + 96."""
    require_gpu()
    T, E, topk, K = 1000, 4, 2, 256
    Aq, As, Bq, Bs = problem(orc, T, E, K, N, 31)
    ids, s, eids = routed(orc, T, E, topk, 31)
    C = hkq.moe_mxfp4(dev_u8(Aq), dev_u8(As), dev_u8(Bq), dev_u8(Bs), dev_i32(s), dev_i32(eids), T * topk, topk)
    torch.cuda.synchronize()
    ref = orc.moe_mxfp4_ref(Aq, As, Bq, Bs, None, None, None, s, eids, N, T * topk, topk, False, T * topk)
    assert_gemm_close(C.float().cpu().numpy(), ref, f"moe mxfp4 whole + split N={N}")


def test_moe_mxfp4_gpu_routing_and_special_blocks(orc):
    """Sorted ids from the GPU align_block_size; a block whose expert is -1
    (zeros for its valid rows) and rows that no block names (left untouched)."""
    require_gpu()
    T, E, topk, K, N = 200, 4, 2, 256, 128
    Aq, As, Bq, Bs = problem(orc, T, E, K, N, 9)
    ids, _, _ = routed(orc, T, E, topk, 9)
    s_d, e_d, _, total_d = hkq.align_block_size(dev_i32(ids), E, 128)
    total = int(total_d.item())
    s_d, e_d = s_d[:total].clone(), e_d[: total // 128].clone()
    e_d[1] = -1                               # block 1 has no expert
    s_h = s_d.cpu().numpy()
    dropped = s_h[256:384][s_h[256:384] < T * topk]
    s_d[256:384] = T * topk                   # block 2: padding only, so its rows are never written
    C = torch.full((T * topk, N), 7.0, dtype=torch.bfloat16, device="cuda")
    hkq.moe_mxfp4(dev_u8(Aq), dev_u8(As), dev_u8(Bq), dev_u8(Bs), s_d, e_d, T * topk, topk, C=C)
    torch.cuda.synchronize()
    ref = orc.moe_mxfp4_ref(Aq, As, Bq, Bs, None, None, None, s_d.cpu().numpy(), e_d.cpu().numpy(), N, T * topk,
                            topk, False, T * topk)
    got = C.float().cpu().numpy()
    written = ~np.isnan(ref).any(axis=1)
    assert_gemm_close(got[written], ref[written], "moe mxfp4 written rows")
    assert np.all(got[dropped] == 7.0) and np.all(got[~written] == 7.0)
    blk1 = s_h[128:256][s_h[128:256] < T * topk]
    assert len(blk1) and np.all(got[blk1] == 0.0)


def test_moe_mxfp4_decode_layouts(orc):
    """Decode kernel on hand-made blocks: a valid id past the first 16 entries
    of its block (a later 16-entry group), a block of expert -1 (zeros for its
    valid rows) and rows no block names (left untouched)."""
    require_gpu()
    T, E, topk, K, N = 4, 2, 2, 256, 96
    Aq, As, Bq, Bs = problem(orc, T, E, K, N, 41)
    nv = T * topk
    s = np.full(3 * 128, nv, np.int32)
    s[[0, 1, 2, 37]] = [0, 1, 2, 3]          # block 0, expert 0: entry 37 is in group 2
    s[[128, 129]] = [4, 5]                   # block 1, expert -1: zeros
    s[[256, 300]] = [6, 7]                   # block 2, expert 1
    eids = np.array([0, -1, 1], np.int32)
    C = torch.full((nv + 2, N), 7.0, dtype=torch.bfloat16, device="cuda")
    hkq.moe_mxfp4(dev_u8(Aq), dev_u8(As), dev_u8(Bq), dev_u8(Bs), dev_i32(s), dev_i32(eids), nv, topk, C=C)
    torch.cuda.synchronize()
    ref = orc.moe_mxfp4_ref(Aq, As, Bq, Bs, None, None, None, s, eids, N, nv, topk, False, nv)
    got = C.float().cpu().numpy()
    rows = [0, 1, 2, 3, 6, 7]
    assert_gemm_close(got[rows], ref[rows], "moe mxfp4 decode layouts")
    assert np.all(got[[4, 5]] == 0.0) and np.all(got[nv:] == 7.0)


def test_moe_mxfp4_module_reference_call(orc):
    """tests/test_moe.py:902-936 of the reference, argument list unchanged:
    random E2M1 bytes and e8m0 scales in [120, 134), B [E, K/2, N] and B_mx_scale
    [E, K/32, N] (N-contiguous), per-tensor and per-expert scales, routed
    weights; against the oracle on the same codes. The K-contiguous form of the
    same weights gives the same bytes."""
    require_gpu()
    import hipkittens as hk
    num_tokens, num_experts, top_k, K, N, block_m, mx = 64, 8, 2, 256, 256, 128, 32
    g = torch.Generator().manual_seed(42)
    A = torch.randint(0, 255, (num_tokens, K // 2), dtype=torch.uint8, generator=g)
    B = torch.randint(0, 255, (num_experts, K // 2, N), dtype=torch.uint8, generator=g)
    A_mx = torch.randint(120, 134, (num_tokens, K // mx), dtype=torch.uint8, generator=g)
    B_mx = torch.randint(120, 134, (num_experts, K // mx, N), dtype=torch.uint8, generator=g)
    A_scale = torch.tensor([0.01], dtype=torch.float32)
    B_scale = torch.rand(num_experts, dtype=torch.float32, generator=g) * 0.01
    ids, s, eids = routed(orc, num_tokens, num_experts, top_k, 42)
    num_padded = len(s)
    w = torch.rand(num_padded, dtype=torch.float32, generator=g)
    C = torch.zeros(num_padded, N, dtype=torch.bfloat16, device="cuda")
    keep = (dev_u8(A.numpy()), dev_u8(B.numpy()), dev_u8(A_mx.numpy()), dev_u8(B_mx.numpy()), A_scale.cuda(),
            B_scale.cuda(), w.cuda(), dev_i32(s), dev_i32(eids))
    Ad, Bd, Amd, Bmd, asd, bsd, wd, sd, ed = keep
    hk.moe.mxfp4.moe_mxfp4(Ad, Bd, C, Amd, Bmd, asd, bsd, wd, sd, ed, N, K, num_tokens * top_k, top_k, True,
                           K // 2, 1, (K // 2) * N, N, 1, N, 1, K // mx, 1, (K // mx) * N, N, 1,
                           num_padded // block_m, (N + 127) // 128)
    torch.cuda.synchronize()
    Bt = B.transpose(1, 2).contiguous()
    Bmt = B_mx.transpose(1, 2).contiguous()
    ref = orc.moe_mxfp4_ref(A.numpy(), A_mx.numpy(), Bt.numpy(), Bmt.numpy(), 0.01, B_scale.numpy(), w.numpy(), s,
                            eids, N, num_tokens * top_k, top_k, True, num_padded)
    got = C.float().cpu().numpy()
    rows = ~np.isnan(ref).any(axis=1)
    assert_gemm_close(got[rows], ref[rows], "reference call")
    assert np.all(got[~rows] == 0)
    C2 = torch.zeros_like(C)
    Btd, Bmtd = dev_u8(Bt.numpy()), dev_u8(Bmt.numpy())
    hk.moe.mxfp4.moe_mxfp4(Ad, Btd, C2, Amd, Bmtd, asd, bsd, wd, sd, ed, N, K, num_tokens * top_k, top_k, True,
                           K // 2, 1, (K // 2) * N, 1, K // 2, N, 1, K // mx, 1, (K // mx) * N, 1, K // mx,
                           num_padded // block_m, (N + 127) // 128)
    torch.cuda.synchronize()
    assert torch.equal(C, C2)


# The reference's N-contiguous B [E, K/2, N] and B_mx_scale [E, K/32, N] read
# in place (hkq_moe_mxfp4_kn: K-tiles of E2M1 pairs staged as rows of K, the
# operands and the e8m0 scale operands built with transposed LDS reads): the
# same bits as the K-contiguous layout. Whole 256-row tiles, lone and 64-row
# blocks, the last round split in blocks, decode-sized routing (the tiled
# kernel), N not a multiple of 256 or 16, rows of K padded past N.
@pytest.mark.parametrize("T,E,topk,K,N,pad", [(600, 4, 2, 512, 512, 0), (300, 3, 2, 1024, 1000, 24),
                                              (4, 8, 2, 512, 256, 0), (2000, 8, 2, 256, 4104, 8)])
def test_moe_mxfp4_kn_matches_kmajor(orc, T, E, topk, K, N, pad):
    require_gpu()
    ids, s, eids = routed(orc, T, E, topk, 71)
    rng = np.random.default_rng(72)
    Aq = rng.integers(0, 256, (T, K // 2), dtype=np.uint8)
    As = rng.integers(120, 134, (T, K // 32), dtype=np.uint8)
    Bq = rng.integers(0, 256, (E, N, K // 2), dtype=np.uint8)
    Bs = rng.integers(120, 134, (E, N, K // 32), dtype=np.uint8)
    Bkn = np.zeros((E, K // 2, N + pad), np.uint8)
    Bkn[:, :, :N] = Bq.transpose(0, 2, 1)
    Bskn = np.zeros((E, K // 32, N + pad), np.uint8)
    Bskn[:, :, :N] = Bs.transpose(0, 2, 1)
    w = rng.random(len(s)).astype(np.float32)
    args = (dev_i32(s), dev_i32(eids), T * topk, topk)
    C = hkq.moe_mxfp4(dev_u8(Aq), dev_u8(As), dev_u8(Bq), dev_u8(Bs), *args, topk_weights=dev_f32(w))
    Ckn = hkq.moe_mxfp4(dev_u8(Aq), dev_u8(As), dev_u8(Bkn)[:, :, :N], dev_u8(Bskn)[:, :, :N], *args,
                        topk_weights=dev_f32(w), b_kn=True)
    torch.cuda.synchronize()
    assert torch.equal(C, Ckn), "N-contiguous weights give other bits than K-contiguous ones"
    ref = orc.moe_mxfp4_ref(Aq, As, Bq, Bs, None, None, w, s, eids, N, T * topk, topk, True, T * topk)
    got = Ckn.float().cpu().numpy()
    rows = ~np.isnan(ref).any(axis=1)
    assert_gemm_close(got[rows], ref[rows], "moe mxfp4 [E, K/2, N]")


def test_moe_pack_kmajor(orc):
    """The prepack entry point on ragged shapes and padded strides: an exact
    byte transpose of every expert plane, bytes outside the destination rows
    untouched."""
    require_gpu()
    rng = np.random.default_rng(3)
    for E, R, N, pad_r, pad_n in ((3, 100, 70, 0, 0), (2, 256, 512, 16, 32), (1, 64, 17, 5, 3)):
        src = rng.integers(0, 256, (E, R, N + pad_r), dtype=np.uint8)
        dst = torch.full((E, N, R + pad_n), 0xAB, dtype=torch.uint8, device="cuda")
        sd = dev_u8(src)
        hkq.call("hkq_moe_pack_kmajor", sd.data_ptr(), dst.data_ptr(), E, R, N, sd.stride(0), sd.stride(1),
                 dst.stride(0), dst.stride(1), torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        got = dst.cpu().numpy()
        assert np.array_equal(got[:, :, :R], src[:, :, :N].transpose(0, 2, 1))
        assert np.all(got[:, :, R:] == 0xAB)


@pytest.mark.parametrize("K,N", [(4096, 28672), (14336, 4096)])
def test_moe_mxfp4_mixtral_full(orc, K, N):
    """Mixtral-8x7B sizes (T=4096, E=8, top-2; gate/up K=4096, N=28672; down
    K=14336, N=4096) on align_block_size routing from seeded softmax top-2:
    weights ~N(0, 0.02) drawn on the device and MX-quantized by the GPU
    quantizer (bit-exact with the oracle's, tests/test_gpu_quant.py), every
    output row against the fp32 oracle (oracle.moe_mxfp4_ref_f32)."""
    require_gpu()
    T, E, topk = 4096, 8, 2
    gl = torch.Generator(device="cpu").manual_seed(K)
    logits = torch.randn(T, E, generator=gl)
    ids = torch.topk(torch.softmax(logits, -1), topk, dim=-1).indices.numpy().astype(np.int32).ravel()
    s, eids, _, _ = orc.align_block_size(ids, E, 128)
    Aq, As = orc.mx_quant_fp4(orc.randn_bf16((T, K), seed=K + 1))
    g = torch.Generator(device="cuda").manual_seed(K + 2)
    wb = (torch.randn(E * N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    Bq_d, Bs_d = hkq.mx_quant(wb, True)
    torch.cuda.synchronize()
    del wb
    Bq = Bq_d.cpu().numpy().reshape(E, N, K // 2)
    Bs = Bs_d.cpu().numpy().reshape(E, N, K // 32)
    rng = np.random.default_rng(K)
    w = rng.random(T * topk).astype(np.float32)
    C = hkq.moe_mxfp4(dev_u8(Aq), dev_u8(As), Bq_d.view(E, N, K // 2), Bs_d.view(E, N, K // 32), dev_i32(s),
                      dev_i32(eids), T * topk, topk, topk_weights=dev_f32(w))
    torch.cuda.synchronize()
    ref = orc.moe_mxfp4_ref_f32(Aq, As, Bq, Bs, None, None, w, s, eids, N, T * topk, topk, True, T * topk)
    assert not np.isnan(ref).any()
    assert_gemm_close(C.float().cpu().numpy(), ref, f"moe mxfp4 mixtral K={K} N={N}")


@pytest.mark.parametrize("K,N", [(4096, 28672), (14336, 4096)])
def test_moe_mxfp4_mixtral_reference_layout_module(orc, K, N):
    """Mixtral sizes through moe_op_mxfp4_tk with the reference's own layouts,
    B [E, K/2, N] and B_mx_scale [E, K/32, N] (stride_bn = stride_bmxn = 1,
    tests/test_moe.py:909-925), read in place by the kernels; every output row
    against the fp32 oracle."""
    require_gpu()
    import hipkittens as hk

    T, E, topk = 4096, 8, 2
    gl = torch.Generator(device="cpu").manual_seed(K + 5)
    logits = torch.randn(T, E, generator=gl)
    ids = torch.topk(torch.softmax(logits, -1), topk, dim=-1).indices.numpy().astype(np.int32).ravel()
    s, eids, _, _ = orc.align_block_size(ids, E, 128)
    Aq, As = orc.mx_quant_fp4(orc.randn_bf16((T, K), seed=K + 6))
    g = torch.Generator(device="cuda").manual_seed(K + 7)
    wb = (torch.randn(E * N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    Bq_d, Bs_d = hkq.mx_quant(wb, True)
    del wb
    Bkn = Bq_d.view(E, N, K // 2).transpose(1, 2).contiguous()
    Bskn = Bs_d.view(E, N, K // 32).transpose(1, 2).contiguous()
    torch.cuda.synchronize()
    Bq = Bq_d.cpu().numpy().reshape(E, N, K // 2)
    Bs = Bs_d.cpu().numpy().reshape(E, N, K // 32)
    del Bq_d, Bs_d
    C = torch.zeros(len(s), N, dtype=torch.bfloat16, device="cuda")
    hk.moe.mxfp4.moe_mxfp4(dev_u8(Aq), Bkn, C, dev_u8(As), Bskn, None, None, None, dev_i32(s), dev_i32(eids), N, K,
                           T * topk, topk, False, K // 2, 1, (K // 2) * N, N, 1, N, 1, K // 32, 1, (K // 32) * N, N, 1,
                           len(s) // 128, (N + 127) // 128)
    torch.cuda.synchronize()
    ref = orc.moe_mxfp4_ref_f32(Aq, As, Bq, Bs, None, None, None, s, eids, N, T * topk, topk, False, len(s))
    got = C.float().cpu().numpy()
    rows = ~np.isnan(ref).any(axis=1)
    assert rows.sum() == T * topk
    assert_gemm_close(got[rows], ref[rows], f"moe mxfp4 mixtral [E, K/2, N] module K={K} N={N}")
