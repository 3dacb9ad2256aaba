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
# the decode (streaming) kernel, with K-steps uneven over its 4 waves;
# (5, 8, 2, 384, 4160) has few ids but a large tiled grid, so it stays tiled.
@pytest.mark.parametrize("T,E,topk,K,N", [(64, 8, 2, 256, 256), (1024, 8, 2, 2048, 1024), (300, 4, 1, 384, 520),
                                          (77, 16, 4, 512, 64), (1, 8, 2, 256, 512), (5, 8, 2, 384, 4160),
                                          (16, 8, 2, 640, 1000)])
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


def test_moe_mxfp4_whole_and_split_tiles(orc):
    """Enough 256-column tiles that most run as whole pairs of blocks while the
    sparse last round (on 256 CUs: 8 pairs x 36 = 288 tiles = 256 + 32) runs block by block."""
    require_gpu()
    T, E, topk, K, N = 1000, 4, 2, 256, 9216
    Aq, As, Bq, Bs = problem(orc, T, E, K, N, 31)
    ids, s, eids = routed(orc, T, E, topk, 31)
    C = hkq.moe_mxfp4(dev_u8(Aq), dev_u8(As), dev_u8(Bq), dev_u8(Bs), dev_i32(s), dev_i32(eids), T * topk, topk)
    torch.cuda.synchronize()
    ref = orc.moe_mxfp4_ref(Aq, As, Bq, Bs, None, None, None, s, eids, N, T * topk, topk, False, T * topk)
    assert_gemm_close(C.float().cpu().numpy(), ref, "moe mxfp4 whole + split")


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
    """tests/test_moe.py:902-936 of the reference: random E2M1 bytes and e8m0
    scales in [120, 134), per-tensor and per-expert scales, routed weights. The
    reference's [E, K/2, N] weights raise ValueError naming the transpose; the
    transposed call matches the oracle."""
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
    args = (dev_u8(A.numpy()), dev_u8(B.numpy()), C, dev_u8(A_mx.numpy()), dev_u8(B_mx.numpy()), A_scale.cuda(),
            B_scale.cuda(), w.cuda(), dev_i32(s), dev_i32(eids), N, K, num_tokens * top_k, top_k, True)
    with pytest.raises(ValueError, match="transpose"):
        hk.moe.mxfp4.moe_mxfp4(*args, K // 2, 1, (K // 2) * N, N, 1, N, 1, K // mx, 1, (K // mx) * N, N, 1,
                               num_padded // block_m, (N + 127) // 128)
    Bt = B.transpose(1, 2).contiguous()
    Bmt = B_mx.transpose(1, 2).contiguous()
    args = args[:1] + (dev_u8(Bt.numpy()),) + args[2:4] + (dev_u8(Bmt.numpy()),) + args[5:]
    hk.moe.mxfp4.moe_mxfp4(*args, K // 2, 1, (K // 2) * N, 1, K // 2, N, 1, K // mx, 1, (K // mx) * N, 1, K // mx,
                           num_padded // block_m, (N + 127) // 128)
    torch.cuda.synchronize()
    ref = orc.moe_mxfp4_ref(A.numpy(), A_mx.numpy(), Bt.numpy(), Bmt.numpy(), 0.01, B_scale.numpy(), w.numpy(), s,
                            eids, N, num_tokens * top_k, top_k, True, num_padded)
    got = C.float().cpu().numpy()
    rows = ~np.isnan(ref).any(axis=1)
    assert_gemm_close(got[rows], ref[rows], "reference call")
    assert np.all(got[~rows] == 0)
