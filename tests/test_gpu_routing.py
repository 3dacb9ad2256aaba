"""GPU parity of the MoE routing producers against the CPU oracle
(oracle/routing_oracle.c), through the C ABI and through the reference-named
modules with the reference tests' own calls (tests/test_moe.py:167-470).

Bar: every index, count and tile word bit-exact; top-k values bit-exact
without softmax and within one bf16 ulp with it (device vs host expf).
"""
import numpy as np
import pytest
import torch

import hkq
from gpu_util import require_gpu

pytestmark = pytest.mark.gpu


def dev(a, dtype=np.int32):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=dtype)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bf16_dev(bits):
    return dev(bits.view(np.int16), np.int16).view(torch.bfloat16)


def bf16_host(t):
    return host(t.view(torch.int16)).view(np.uint16)


def logits_with_specials(orc, T, E, seed):
    xb = orc.randn_bf16((T, E), seed=seed)
    rng = np.random.default_rng(seed)
    ties = rng.random((T, E)) < 0.3  # integer-valued logits: many ties
    xb[ties] = (rng.integers(-2, 3, size=int(ties.sum())).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    z = (xb == 0) & (rng.random((T, E)) < 0.5)
    xb[z] = 0x8000
    xb[rng.random((T, E)) < 0.01] = 0xFF80  # -inf
    xb[rng.random((T, E)) < 0.01] = 0x7FC0  # NaN
    xb[0, :] = 0xFF80                       # nothing eligible
    return xb


def ulp_close(a_bits, b_bits):
    """bf16 values equal or one ulp apart (same sign)."""
    a, b = a_bits.astype(np.int32), b_bits.astype(np.int32)
    return np.all(np.abs(a - b) <= 1)


@pytest.mark.parametrize("T,E,K", [(4096, 8, 2), (1000, 64, 6), (4096, 256, 8), (333, 128, 4), (257, 512, 10),
                                   (100, 1024, 16), (50, 5, 8), (64, 20, 1), (700, 16, 3), (129, 60, 8),
                                   (200, 384, 8), (90, 1000, 2)])
def test_topk(orc, T, E, K):
    require_gpu()
    xb = logits_with_specials(orc, T, E, T + E + K)
    x = bf16_dev(xb)
    for softmax in (False, True):
        yv, yi, bits = hkq.moe_topk(x, K, softmax=softmax)
        ov, oi, ob = orc.topk(xb, K, softmax)
        assert np.array_equal(host(yi), oi)
        assert np.array_equal(host(bits).view(np.uint32), ob)
        gv = bf16_host(yv)
        if softmax:
            assert ulp_close(gv, ov)
        else:
            assert np.array_equal(gv, ov)


def test_topk_strided_and_column_major_bits(orc):
    """Row strides past the data and the reference test's column-major bitmatrix."""
    require_gpu()
    T, E, K = 300, 256, 4
    xb = orc.randn_bf16((T, E), seed=5)
    xpad = np.zeros((T, E + 40), np.uint16)
    xpad[:, :E] = xb
    x = bf16_dev(xpad)
    sy = 7
    Yv = torch.zeros((T, sy), dtype=torch.bfloat16, device="cuda")
    Yi = torch.full((T, sy), -5, dtype=torch.int32, device="cuda")
    nw = (E + 31) // 32
    Bits = torch.zeros(nw * T, dtype=torch.int32, device="cuda")
    hkq.call("hkq_moe_topk", x.data_ptr(), E + 40, Yv.data_ptr(), Yi.data_ptr(), sy, Bits.data_ptr(), 1, T, T, E, K, 1,
             torch.cuda.current_stream().cuda_stream)
    ov, oi, ob = orc.topk(xb, K, True)
    yi = host(Yi)
    assert np.array_equal(yi[:, :K], oi) and np.all(yi[:, K:] == -5)
    assert ulp_close(bf16_host(Yv)[:, :K], ov)
    assert np.array_equal(host(Bits).view(np.uint32).reshape(nw, T).T, ob)


def test_topk_module_reference_call(orc):
    """tests/test_moe.py:263-315 as written: 128 x 256 bf16 logits, K = 4, softmax."""
    require_gpu()
    import hipkittens as hk
    num_tokens, num_experts, K = 128, 256, 4
    xb = orc.randn_bf16((num_tokens, num_experts), seed=42)
    X = bf16_dev(xb)
    Yv = torch.empty(num_tokens, K, dtype=torch.bfloat16, device="cuda")
    Yi = torch.empty(num_tokens, K, dtype=torch.int32, device="cuda")
    Bits = torch.zeros((num_experts + 31) // 32 * num_tokens, dtype=torch.int32, device="cuda")
    hk.moe_routing.topk.moe_topk(X, num_experts, Yv, Yi, K, Bits, 1, num_tokens, num_tokens, num_experts, K, True)
    ov, oi, _ = orc.topk(xb, K, True)
    assert np.array_equal(host(Yi), oi)
    assert ulp_close(bf16_host(Yv), ov)
    with pytest.raises(ValueError):  # Yv too small for n_rows x K
        hk.moe_routing.topk.moe_topk(X, num_experts, Yv[:10], Yi, K, Bits, 1, num_tokens, num_tokens, num_experts, K,
                                     True)


@pytest.mark.parametrize("rows,nw", [(0, 1), (1, 1), (128, 2), (129, 1), (4096, 8), (128 * 300 + 5, 1), (40000, 3)])
def test_sum_bitmatrix_rows(orc, rows, nw):
    require_gpu()
    rng = np.random.default_rng(rows + nw)
    bits = rng.integers(0, 2**32, size=(rows, nw), dtype=np.uint64).astype(np.uint32)
    bits &= rng.integers(0, 2**32, size=(rows, nw), dtype=np.uint64).astype(np.uint32)
    ret, part = hkq.sum_bitmatrix_rows(dev(bits.view(np.int32)), partials=True)
    oret, opart = orc.sum_bitmatrix_rows(bits)
    assert np.array_equal(host(ret).view(np.uint32), oret)
    assert np.array_equal(host(part).view(np.uint32), opart)
    ret2, _ = hkq.sum_bitmatrix_rows(dev(bits.view(np.int32)), partials=False)
    assert np.array_equal(host(ret2).view(np.uint32), oret)


def test_sum_bitmatrix_rows_module_reference_call(orc):
    """tests/test_moe.py:323-370 as written (column-major, fused), plus the
    partials form with column-major partials and shape_pn below 32 * shape_bn."""
    require_gpu()
    import hipkittens as hk
    num_tokens, num_experts, num_blocks = 128, 64, 2
    np.random.seed(42)
    bitmatrix = np.zeros((num_tokens, num_blocks), np.uint32)
    for t in range(num_tokens):
        for eid in np.random.choice(num_experts, 2, replace=False):
            bitmatrix[t, eid // 32] |= np.uint32(1 << (eid % 32))
    bm_col = dev(bitmatrix.T.copy().view(np.int32))
    ret = torch.zeros(num_experts, dtype=torch.int32, device="cuda")
    hk.moe_routing.bitmatrix.sum_bitmatrix_rows_fused(bm_col, num_tokens, 1, num_tokens, ret, num_blocks)
    oret, _ = orc.sum_bitmatrix_rows(bitmatrix, partials=False)
    assert np.array_equal(host(ret).view(np.uint32), oret)

    T, nw = 1000, 2
    rng = np.random.default_rng(9)
    b = rng.integers(0, 2**32, size=(T, nw), dtype=np.uint64).astype(np.uint32)
    ntiles, pcols = (T + 127) // 128, 50
    part = torch.full((pcols * ntiles,), -3, dtype=torch.int32, device="cuda")  # [pcols, ntiles]
    ret = torch.zeros(32 * nw, dtype=torch.int32, device="cuda")
    hk.moe_routing.bitmatrix.sum_bitmatrix_rows(dev(b.T.copy().view(np.int32)), T, 1, T, ret, part, 1, ntiles, pcols,
                                                nw)
    oret, opart = orc.sum_bitmatrix_rows(b)
    assert np.array_equal(host(ret).view(np.uint32), oret)
    assert np.array_equal(host(part).view(np.uint32).reshape(pcols, ntiles).T, opart[:, :pcols])


@pytest.mark.parametrize("E,log2,slack", [(8, 6, 10), (1, 7, 0), (256, 7, 3), (64, 7, -5), (4096, 4, 100)])
def test_expt_data(orc, E, log2, slack):
    require_gpu()
    rng = np.random.default_rng(E * 7 + log2)
    hist = rng.integers(0, 700, size=E).astype(np.int32)
    hist[rng.random(E) < 0.3] = 0
    tile = 1 << log2
    total = int(((hist + tile - 1) // tile).sum())
    max_tiles = max(0, total + slack)
    n_gates = int(hist.sum())
    canary = 0x5A5A5A5A
    for mode in (0, 1, 2):
        ts = torch.zeros(E + 1, dtype=torch.int32, device="cuda")
        tl = torch.zeros(E + 1, dtype=torch.int32, device="cuda")
        md = torch.full((max_tiles + 1,), canary, dtype=torch.int32, device="cuda")
        h = dev(hist)
        if mode == 0:
            hkq.call("hkq_expt_data_stage1", h.data_ptr(), ts.data_ptr(), tl.data_ptr(), md.data_ptr(), E, max_tiles,
                     n_gates, log2, torch.cuda.current_stream().cuda_stream)
        else:
            hkq.call("hkq_expt_data_compute", h.data_ptr(), ts.data_ptr(), tl.data_ptr(), md.data_ptr(), E, max_tiles,
                     n_gates, log2, int(mode == 2), torch.cuda.current_stream().cuda_stream)
        ots, otl, omd = orc.expt_data(hist, max_tiles, n_gates, log2, mode, md_init=canary)
        assert np.array_equal(host(ts), ots) and np.array_equal(host(tl), otl)
        g = host(md).view(np.uint32)
        assert np.array_equal(g[:max_tiles], omd)
        assert g[max_tiles] == canary  # nothing written past max_num_tiles


def test_expt_data_module_reference_call(orc):
    """tests/test_moe.py:385-436 as written, then the stage-wise calls."""
    require_gpu()
    import hipkittens as hk
    num_experts, tile_dim_log2 = 8, 6
    torch.manual_seed(42)
    hist = torch.randint(0, 200, (num_experts,), dtype=torch.int32)
    n_gates = int(hist.sum())
    max_num_tiles = sum((int(h) + 63) // 64 for h in hist) + 10
    token_start = torch.zeros(num_experts + 1, dtype=torch.int32, device="cuda")
    tile_start = torch.zeros(num_experts + 1, dtype=torch.int32, device="cuda")
    md = torch.full((max_num_tiles,), -1, dtype=torch.int32, device="cuda")
    hk.moe_routing.expt_data.expt_data_compute(hist.cuda(), token_start, tile_start, md, num_experts, max_num_tiles,
                                               n_gates, tile_dim_log2, False)
    ots, otl, omd = orc.expt_data(hist.numpy(), max_num_tiles, n_gates, tile_dim_log2, 1)
    assert np.array_equal(host(token_start), ots) and np.array_equal(host(tile_start), otl)
    assert np.array_equal(host(md).view(np.uint32), omd)
    # stage 1 then stage 2 (and the fused stage 2) from the device TileStart
    md2 = torch.full((max_num_tiles,), 7, dtype=torch.int32, device="cuda")
    hk.moe_routing.expt_data.expt_data_stage1(hist.cuda(), token_start, tile_start, md2, num_experts, max_num_tiles,
                                              n_gates, tile_dim_log2)
    md3 = md2.clone()
    hk.moe_routing.expt_data.expt_data_stage2(hist.cuda(), tile_start, md2, num_experts, tile_dim_log2)
    assert np.array_equal(host(md2).view(np.uint32), omd)
    hk.moe_routing.expt_data.expt_data_stage2_fused(hist.cuda(), tile_start, md3, num_experts)
    _, _, omd3 = orc.expt_data(hist.numpy(), max_num_tiles, n_gates, tile_dim_log2, 2, md_init=7)
    assert np.array_equal(host(md3).view(np.uint32), omd3)


def partials_for(indx_flat, K, E):
    G = 128 * K
    nb = (len(indx_flat) + G - 1) // G
    cnt = np.zeros((nb, E), np.int64)
    for b in range(nb):
        v = indx_flat[b * G:(b + 1) * G]
        v = v[(v >= 0) & (v < E)]
        cnt[b] = np.bincount(v, minlength=E)
    return (np.cumsum(cnt, 0) - cnt).astype(np.int32), cnt.sum(0)


@pytest.mark.parametrize("T,K,E", [(1, 2, 8), (4096, 2, 8), (4096, 8, 256), (5000, 4, 1024), (77, 16, 40),
                                   (1000, 1, 3), (2048, 10, 512)])
def test_compute_indx(orc, T, K, E):
    require_gpu()
    rng = np.random.default_rng(T + K + E)
    indx = rng.integers(0, E, size=(T, K)).astype(np.int32)
    indx[rng.random((T, K)) < 0.03] = -1
    flat = indx.ravel()
    scal = rng.integers(0, 0x7F00, size=T * K).astype(np.uint16)
    po, hist = partials_for(flat, K, E)
    ts = np.concatenate([[0], np.cumsum(hist)[:-1]]).astype(np.int32)
    nv = int(hist.sum())
    og, osc, ogs = orc.compute_indx(flat, scal, K, ts, po, n_slots=nv)
    for use_partials in (True, False):
        g, s, gs = hkq.compute_indx(dev(indx), dev(ts), dev(po) if use_partials else None,
                                    expt_scal=bf16_dev(scal.reshape(T, K)), n_slots=nv)
        assert np.array_equal(host(g), og)
        assert np.array_equal(host(s), osc)
        assert np.array_equal(bf16_host(gs), ogs)


def test_compute_indx_module_and_strided_partials(orc):
    """Column-major PartialOffs through moe_routing_tk, gate scales skipped."""
    require_gpu()
    import hipkittens as hk
    T, K, E = 3000, 2, 8
    rng = np.random.default_rng(4)
    indx = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
    flat = indx.ravel()
    po, hist = partials_for(flat, K, E)
    ts = np.concatenate([[0], np.cumsum(hist)[:-1]]).astype(np.int32)
    og, osc, _ = orc.compute_indx(flat, None, K, ts, po)
    G = torch.empty(T * K, dtype=torch.int32, device="cuda")
    S = torch.empty(T * K, dtype=torch.int32, device="cuda")
    nb = po.shape[0]
    pcol = dev(po.T.copy())
    hk.moe_routing.routing.routing_compute_indx(G, S, None, None, dev(flat), pcol, 1, nb, dev(ts), T * K, K)
    assert np.array_equal(host(G), og) and np.array_equal(host(S), osc)
    hk.moe_routing.routing.routing_compute_indx_fused(G, S, None, None, dev(flat), dev(ts), T * K, K)
    assert np.array_equal(host(G), og) and np.array_equal(host(S), osc)


@pytest.mark.parametrize("n,E,bs", [(0, 8, 64), (1, 1, 16), (256, 8, 64), (8192, 8, 128), (32768, 256, 128),
                                    (100000, 64, 64), (3000, 1024, 16), (999, 3, 7), (70000, 2, 256)])
def test_align_block_size(orc, n, E, bs):
    require_gpu()
    rng = np.random.default_rng(n + E + bs)
    ids = rng.integers(0, E, size=n).astype(np.int32)
    if n:
        ids[rng.random(n) < 0.02] = -1
    s, eids, cum, total = hkq.align_block_size(dev(ids) if n else torch.empty(0, dtype=torch.int32, device="cuda"),
                                               E, bs)
    os_, oe, oc, ot = orc.align_block_size(ids, E, bs)
    assert int(host(total)[0]) == ot
    assert np.array_equal(host(cum), oc)
    assert np.array_equal(host(s)[:ot], os_)
    assert np.array_equal(host(eids)[: ot // bs], oe)


def test_align_block_size_module_reference_call(orc):
    """tests/test_moe.py:167-226 as written (256 ids, 8 experts, block 64)."""
    require_gpu()
    import hipkittens as hk
    num_tokens, num_experts, block_size = 256, 8, 64
    torch.manual_seed(42)
    topk_ids = torch.randint(0, num_experts, (num_tokens,), dtype=torch.int32, device="cuda")
    tpe = torch.bincount(topk_ids.cpu().long(), minlength=num_experts)
    expected_total = int(((tpe + block_size - 1) // block_size * block_size).sum())
    sorted_token_ids = torch.zeros(expected_total, dtype=torch.int32, device="cuda")
    expert_ids_out = torch.zeros(expected_total // block_size, dtype=torch.int32, device="cuda")
    tokens_cnts_buffer = torch.zeros((num_experts + 1) * num_experts, dtype=torch.int32, device="cuda")
    cumsum_buffer = torch.zeros(num_experts + 1, dtype=torch.int32, device="cuda")
    total_tokens_post_pad = torch.zeros(1, dtype=torch.int32, device="cuda")
    hk.moe_routing.align_block_size.moe_align_block_size(topk_ids, sorted_token_ids, expert_ids_out,
                                                         tokens_cnts_buffer, cumsum_buffer, total_tokens_post_pad,
                                                         num_experts, block_size, num_tokens)
    os_, oe, oc, ot = orc.align_block_size(topk_ids.cpu().numpy(), num_experts, block_size)
    assert int(host(total_tokens_post_pad)[0]) == ot == expected_total
    assert np.array_equal(host(sorted_token_ids), os_)
    assert np.array_equal(host(expert_ids_out), oe)
    assert np.array_equal(host(cumsum_buffer), oc)


def test_routing_pipeline_feeds_moe_gemm(orc):
    """Router logits -> GPU routing -> the OGS metadata the MoE GEMM consumes:
    equal to the host construction of tests/test_moe.py:97-128 (top-2 of 8,
    4096 tokens), and the MoE GEMM gives identical output with either."""
    require_gpu()
    T, E, K, hidden, N = 4096, 8, 2, 256, 256
    xb = orc.randn_bf16((T, E), seed=8)
    r = hkq.moe_routing(bf16_dev(xb), K, block_m=128)
    _, oi, _ = orc.topk(xb, K, True)
    hist, offs, gather, ed = orc.ogs_routing(oi, E, 128)
    assert np.array_equal(host(r["hist"]), hist)
    assert np.array_equal(host(r["offs"]), offs)
    assert np.array_equal(host(r["gather"]), gather)
    md = host(r["expt_data"])
    assert np.array_equal(md[: len(ed)], ed) and np.all(md[len(ed):] == -1)
    X, xs = orc.quant_rowwise(orc.randn_bf16((T, hidden), seed=9), None, "fp8")
    W, ws = orc.quant_rowwise(orc.randn_bf16((E * N, hidden), seed=10, std=0.02), None, "fp8")
    Xd = torch.from_numpy(X).cuda()
    Wd = torch.from_numpy(W.reshape(E, N, hidden)).cuda()
    xsd, wsd = dev(xs.reshape(-1), np.float32), dev(ws.reshape(E, N), np.float32)
    Y1 = hkq.moe_a8w8(Xd, Wd, r["hist"], r["offs"], r["expt_data"], K, gather=r["gather"], x_scale=xsd, w_scale=wsd)
    Y2 = hkq.moe_a8w8(Xd, Wd, dev(hist), dev(offs), dev(ed), K, gather=dev(gather), x_scale=xsd, w_scale=wsd)
    torch.cuda.synchronize()
    assert torch.equal(Y1.view(torch.int16), Y2.view(torch.int16))
