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
