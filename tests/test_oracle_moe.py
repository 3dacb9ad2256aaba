"""Pin the oracle's MXFP4 MoE reference (CPU only) against per-expert dense
MXFP4 GEMM references on the gathered rows, and check its special cases
(routed weights, blocks without an expert, padding rows)."""
import numpy as np


def test_moe_mxfp4_ref_matches_dense_per_expert(orc):
    T, E, topk, K, N = 100, 4, 2, 256, 64
    rng = np.random.default_rng(1)
    Aq, As = orc.mx_quant_fp4(orc.randn_bf16((T, K), seed=1))
    Bq, Bs = orc.mx_quant_fp4(orc.randn_bf16((E * N, K), seed=2, std=0.05))
    Bq, Bs = Bq.reshape(E, N, K // 2), Bs.reshape(E, N, K // 32)
    ids = rng.integers(0, E, size=T * topk).astype(np.int32)
    sorted_ids, eids, _, total = orc.align_block_size(ids, E, 128)
    w = rng.random(T * topk).astype(np.float32)
    bsc = rng.random(E).astype(np.float32)
    C = orc.moe_mxfp4_ref(Aq, As, Bq, Bs, 0.5, bsc, w, sorted_ids, eids, N, T * topk, topk, True, T * topk)
    assert not np.isnan(C).any()  # every gate written once
    for e in range(E):
        g = np.nonzero(ids == e)[0]
        dense = orc.gemm_mxfp4_ref(Aq[g // topk], As[g // topk], Bq[e], Bs[e])
        np.testing.assert_allclose(C[g], dense * 0.5 * float(bsc[e]) * w[g][:, None].astype(np.float64), rtol=1e-12)


def test_moe_mxfp4_ref_special_blocks(orc):
    T, topk, K, N = 10, 1, 128, 8
    Aq, As = orc.mx_quant_fp4(orc.randn_bf16((T, K), seed=3))
    Bq, Bs = orc.mx_quant_fp4(orc.randn_bf16((N, K), seed=4))
    sorted_ids = np.full(256, T, np.int32)  # padding everywhere ...
    sorted_ids[:4] = [0, 1, 2, 3]           # ... but four rows of block 0
    sorted_ids[128:130] = [4, 5]            # and two of block 1
    C = orc.moe_mxfp4_ref(Aq, As, Bq[None], Bs[None], None, None, None, sorted_ids, np.array([0, -1]), N, T, topk,
                          False, T)
    np.testing.assert_allclose(C[:4], orc.gemm_mxfp4_ref(Aq[:4], As[:4], Bq, Bs))
    assert np.all(C[4:6] == 0) and np.isnan(C[6:]).all()


def _routing(orc, T, E, topk, seed):
    rng = np.random.default_rng(seed)
    assigns = np.stack([rng.permutation(E)[:topk] for _ in range(T)])
    return orc.ogs_routing(assigns, E, 128)


def test_moe_blockscale_ref_matches_dense_per_expert(orc):
    """The block-scale MoE reference (per-K-group scales, moe_op_gemm_a8w8_
    blockscale/kernel.cpp:114-145) equals, expert by expert, the dense
    block-scale GEMM reference on that expert's gathered rows, for group_k 64
    and 128 and group_n 1 / 64 / 128 with scales that differ per (token, group)
    and per (expert, group, column block)."""
    T, E, topk, K, N = 300, 4, 2, 256, 192
    hist, offs, gather, ed = _routing(orc, T, E, topk, 3)
    X, _ = orc.quant_rowwise(orc.randn_bf16((T, K), seed=4), None, "fp8")
    W, _ = orc.quant_rowwise(orc.randn_bf16((E * N, K), seed=5, std=0.05), None, "fp8")
    W = W.reshape(E, N, K)
    rng = np.random.default_rng(6)
    bias = rng.standard_normal((E, N)).astype(np.float32)
    for gk, gn in ((64, 64), (128, 1), (64, 128)):
        G, C = K // gk, (N + gn - 1) // gn
        xs = (rng.random((T, G)) + 0.5).astype(np.float32)
        ws = (rng.random((E, G, C)) + 0.5).astype(np.float32)
        Y = orc.moe_blockscale_ref(X, W, xs, ws, bias, gather, hist, offs, ed, topk, gk, gn)
        assert not np.isnan(Y).any()
        for e in range(E):
            s = offs[e] + np.arange(hist[e])
            tok = gather[s] // topk
            dense = orc.gemm_blockscale_ref(X[tok], W[e], xs[tok], ws[e], gk, gn) + bias[e][None, :]
            np.testing.assert_allclose(Y[s], dense, rtol=1e-12, atol=1e-12)
        # the reference's [E, K, N] layout gives the same result
        Yk = orc.moe_blockscale_ref(X, np.ascontiguousarray(W.transpose(0, 2, 1)), xs, ws, bias, gather, hist, offs,
                                    ed, topk, gk, gn, w_layout="ekn")
        np.testing.assert_array_equal(Y, Yk)


def test_moe_fp32_references_match_fp64(orc):
    """The fp32 full-output MoE references (BASELINE sizes) against the fp64
    ones: per-token x per-channel, per-K-group scales, and MXFP4."""
    T, E, topk, K, N = 200, 4, 2, 512, 160
    hist, offs, gather, ed = _routing(orc, T, E, topk, 7)
    X, xs = orc.quant_rowwise(orc.randn_bf16((T, K), seed=8), None, "fp8")
    W, ws = orc.quant_rowwise(orc.randn_bf16((E * N, K), seed=9, std=0.02), None, "fp8")
    W, ws, xs = W.reshape(E, N, K), ws.reshape(E, N), xs.reshape(-1)
    ref = orc.moe_ref(X, W, xs, ws, None, gather, hist, offs, ed, topk, 128, "enk")
    got = orc.moe_ref_f32(X, W, xs, ws, gather, hist, offs, ed, topk)
    assert got.dtype == np.float32
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)
    rng = np.random.default_rng(10)
    xsg = (rng.random((T, K // 128)) * 0.01).astype(np.float32)
    wsg = (rng.random((E, K // 128, (N + 63) // 64)) * 0.01).astype(np.float32)
    ref = orc.moe_blockscale_ref(X, W, xsg, wsg, None, gather, hist, offs, ed, topk, 128, 64)
    got = orc.moe_ref_f32(X, W, xsg, wsg, gather, hist, offs, ed, topk, group_k=128, group_n=64)
    # within 2^-16 of the sum of |terms| (E4M3 sign bit cleared: |codes|)
    absum = orc.moe_blockscale_ref(X & 0x7F, W & 0x7F, xsg, wsg, None, gather, hist, offs, ed, topk, 128, 64)
    assert np.all(np.abs(got - ref) <= 2.0 ** -16 * absum)
    Aq, As = orc.mx_quant_fp4(orc.randn_bf16((T, K), seed=11))
    Bq, Bs = orc.mx_quant_fp4(orc.randn_bf16((E * N, K), seed=12, std=0.05))
    Bq, Bs = Bq.reshape(E, N, K // 2), Bs.reshape(E, N, K // 32)
    ids = rng.integers(0, E, size=T * topk).astype(np.int32)
    s, eids, _, _ = orc.align_block_size(ids, E, 128)
    w = rng.random(T * topk).astype(np.float32)
    bsc = rng.random(E).astype(np.float32)
    ref = orc.moe_mxfp4_ref(Aq, As, Bq, Bs, 0.5, bsc, w, s, eids, N, T * topk, topk, True, T * topk)
    got = orc.moe_mxfp4_ref_f32(Aq, As, Bq, Bs, 0.5, bsc, w, s, eids, N, T * topk, topk, True, T * topk)
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)


def test_moe_refs_without_gather(orc):
    """Without a gather list (the down projection: X holds the expert-sorted
    rows) sorted row s reads row s of X: the same outputs as a gather list
    that names row s for every s (gather[s] = s * topk), for the fp32 and
    fp64 references."""
    T, E, topk, K, N = 150, 4, 2, 256, 96
    hist, offs, gather, ed = _routing(orc, T, E, topk, 13)
    rows = T * topk
    X, xs = orc.quant_rowwise(orc.randn_bf16((rows, K), seed=14), 128, "fp8")
    W, _ = orc.quant_rowwise(orc.randn_bf16((E * N, K), seed=15, std=0.05), None, "fp8")
    W = W.reshape(E, N, K)
    rng = np.random.default_rng(16)
    ws = (rng.random((E, K // 128, (N + 127) // 128)) + 0.5).astype(np.float32)
    ident = (np.arange(rows, dtype=np.int32) * topk).astype(np.int32)
    a = orc.moe_ref_f32(X, W, xs, ws, None, hist, offs, ed, 1, group_k=128, group_n=128)
    b = orc.moe_ref_f32(X, W, xs, ws, ident, hist, offs, ed, topk, group_k=128, group_n=128)
    assert not np.isnan(a).any()
    np.testing.assert_array_equal(a, b[:rows])  # b has X.shape[0] * topk rows, the ones past `rows` unlisted
    c = orc.moe_blockscale_ref(X, W, xs, ws, None, None, hist, offs, ed, 1, 128, 128)
    d = orc.moe_blockscale_ref(X, W, xs, ws, None, ident, hist, offs, ed, topk, 128, 128)
    np.testing.assert_array_equal(c, d[:rows])
