"""Pin the oracle's MoE routing producers (CPU only).

Each routine of oracle/routing_oracle.c is checked against an independent
formulation built from library routines (torch.topk / softmax, numpy
unpackbits / cumsum / stable argsort / repeat), against brute force on inputs
full of ties, and against the known answers the reference's own tests define
(tests/test_moe.py:167-470 of the reference).
"""
import numpy as np
import pytest
import torch


def bf16_bits(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def bits_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- topk

@pytest.mark.parametrize("E,K", [(8, 2), (64, 4), (256, 8), (384, 10), (33, 16)])
def test_topk_matches_torch_on_distinct_logits(orc, E, K):
    rows = 96
    rng = np.random.default_rng(E * 100 + K)
    # distinct bf16 values per row: a random permutation of a strictly increasing grid
    grid = np.linspace(-4.0, 4.0, 4096, dtype=np.float32)
    grid = np.unique(bits_f32(bf16_bits(grid)))
    x = np.stack([rng.permutation(grid)[:E] for _ in range(rows)])
    xb = bf16_bits(x)
    assert all(len(np.unique(r)) == E for r in xb)
    xt = torch.from_numpy(bits_f32(xb))
    kk = min(K, E)
    ref_v, ref_i = torch.topk(xt, kk, dim=1, largest=True, sorted=True)
    yv, yi, bits = orc.topk(xb, K, softmax=False)
    assert np.array_equal(yi[:, :kk], ref_i.numpy().astype(np.int32))
    assert np.array_equal(bits_f32(yv[:, :kk]), ref_v.numpy())
    yv2, yi2, _ = orc.topk(xb, K, softmax=True)
    assert np.array_equal(yi2, yi)
    sm = torch.softmax(ref_v.double(), dim=1).numpy()
    got = bits_f32(yv2[:, :kk]).astype(np.float64)
    assert np.max(np.abs(got - sm) / sm) <= 2.0 ** -8  # bf16 rounding of the fp32 softmax
    # bitmatrix: exactly the chosen experts
    for r in range(rows):
        want = np.zeros((E + 31) // 32, np.uint32)
        for e in ref_i[r].tolist():
            want[e // 32] |= np.uint32(1 << (e % 32))
        assert np.array_equal(bits[r], want)


def brute_topk(vals: np.ndarray, K: int):
    """Sort eligible (not NaN, not -inf) experts by (-value, expert); -0 == +0."""
    el = [(float(v), e) for e, v in enumerate(vals) if not np.isnan(v) and v != -np.inf]
    el.sort(key=lambda t: (-t[0], t[1]))
    idx = [e for _, e in el[:K]] + [-1] * max(0, K - len(el))
    return idx


@pytest.mark.parametrize("E,K", [(8, 2), (8, 8), (5, 8), (40, 6), (256, 8)])
def test_topk_ties_and_specials_brute_force(orc, E, K):
    rows = 200
    rng = np.random.default_rng(7 + E + K)
    x = rng.integers(-2, 3, size=(rows, E)).astype(np.float32)  # heavy ties
    xb = bf16_bits(x)
    neg0 = rng.random((rows, E)) < 0.2
    xb[neg0 & (x == 0)] = 0x8000                                   # -0 among +0
    xb[rng.random((rows, E)) < 0.05] = 0xFF80                      # -inf
    xb[rng.random((rows, E)) < 0.05] = 0x7FC0                      # NaN
    xb[rng.random((rows, E)) < 0.02] = 0x7F80                      # +inf
    xb[0, :] = 0xFF80                                              # a row with nothing eligible
    yv, yi, bits = orc.topk(xb, K, softmax=False)
    f = bits_f32(xb)
    for r in range(rows):
        want = brute_topk(f[r], K)
        assert yi[r].tolist() == want, r
        for k, e in enumerate(want):
            assert yv[r, k] == (xb[r, e] if e >= 0 else 0xFF80)  # the logit's own bits (-0 kept)
    # softmax of a row with nothing eligible: every slot exp(0) / K
    yv2, _, _ = orc.topk(xb[:1], K, softmax=True)
    assert np.all(bits_f32(yv2) == np.float32(bits_f32(bf16_bits(np.float32(1.0) / np.float32(K)))))


def test_topk_reference_case(orc):
    """The reference test's setting (tests/test_moe.py:263-315): 128 x 256 logits ~ N(0,1), K = 4, softmax."""
    xb = orc.randn_bf16((128, 256), seed=42)
    yv, yi, _ = orc.topk(xb, 4, softmax=True)
    ref_v, ref_i = torch.topk(torch.from_numpy(bits_f32(xb)), 4, dim=1)
    # the reference test's acceptance: index sets agree on > 95% of rows (bf16 ties
    # may pick another expert of equal logit), values within 0.05
    same = np.mean([set(a) == set(b) for a, b in zip(yi.tolist(), ref_i.tolist())])
    assert same > 0.95
    sm = torch.softmax(ref_v, 1).numpy()
    assert np.max(np.abs(bits_f32(yv) - sm)) < 0.05


# ---------------------------------------------------------------- bitmatrix sums

@pytest.mark.parametrize("rows,nw", [(0, 1), (1, 1), (128, 2), (129, 1), (1000, 3), (128 * 300 + 5, 1)])
def test_sum_bitmatrix_rows_numpy(orc, rows, nw):
    rng = np.random.default_rng(rows + nw)
    bits = rng.integers(0, 2**32, size=(rows, nw), dtype=np.uint64).astype(np.uint32)
    bits &= rng.integers(0, 2**32, size=(rows, nw), dtype=np.uint64).astype(np.uint32)  # sparser
    ret, part = orc.sum_bitmatrix_rows(bits)
    unp = np.unpackbits(bits.view(np.uint8).reshape(rows, nw * 4), axis=1, bitorder="little").reshape(rows, 32 * nw)
    assert np.array_equal(ret, unp.sum(0).astype(np.uint32))
    nt = (rows + 127) // 128
    pad = np.zeros((nt * 128, 32 * nw), np.int64)
    pad[:rows] = unp
    per_tile = pad.reshape(nt, 128, 32 * nw).sum(1)
    excl = np.cumsum(per_tile, 0) - per_tile
    assert np.array_equal(part, excl.astype(np.uint32))


def test_sum_bitmatrix_rows_reference_case(orc):
    """tests/test_moe.py:323-370: 128 tokens, 64 experts, 2 distinct experts per token."""
    np.random.seed(42)
    bits = np.zeros((128, 2), np.uint32)
    want = np.zeros(64, np.uint32)
    for t in range(128):
        for e in np.random.choice(64, 2, replace=False):
            bits[t, e // 32] |= np.uint32(1 << (e % 32))
            want[e] += 1
    ret, _ = orc.sum_bitmatrix_rows(bits, partials=False)
    assert np.array_equal(ret, want)


# ---------------------------------------------------------------- expt_data

def numpy_expt_data(hist, log2, max_tiles, n_gates):
    tile = 1 << log2
    ntiles = (hist + tile - 1) // tile
    ts = np.concatenate([[0], np.cumsum(hist)[:-1], [n_gates]]).astype(np.int32)
    tl = np.concatenate([[0], np.cumsum(ntiles)]).astype(np.int32)
    e = np.repeat(np.arange(len(hist)), ntiles)
    i = np.concatenate([np.arange(n) for n in ntiles]) if len(e) else np.zeros(0, np.int64)
    md = np.full(max_tiles, 0xFFFFFFFF, np.uint32)
    md[: min(len(e), max_tiles)] = ((e | (i << 16)).astype(np.uint32))[:max_tiles]
    return ts, tl, md


@pytest.mark.parametrize("E,log2,slack", [(8, 6, 10), (1, 7, 0), (256, 4, 3), (64, 7, -5)])
def test_expt_data_numpy(orc, E, log2, slack):
    rng = np.random.default_rng(E * 7 + log2)
    hist = rng.integers(0, 300, size=E).astype(np.int32)
    hist[rng.random(E) < 0.3] = 0
    tile = 1 << log2
    total = int(((hist + tile - 1) // tile).sum())
    max_tiles = max(0, total + slack)
    n_gates = int(hist.sum())
    ts, tl, md = orc.expt_data(hist, max_tiles, n_gates, log2, mode=1)
    wts, wtl, wmd = numpy_expt_data(hist, log2, max_tiles, n_gates)
    assert np.array_equal(ts, wts) and np.array_equal(tl, wtl) and np.array_equal(md, wmd)
    # stage 1 only: the tail sentinels and nothing else
    _, _, md0 = orc.expt_data(hist, max_tiles, n_gates, log2, mode=0, md_init=7)
    assert np.all(md0[: min(total, max_tiles)] == 7) and np.all(md0[total:] == 0xFFFFFFFF)
    # fused stage 2: the first tile of each non-empty expert only
    _, _, md2 = orc.expt_data(hist, max_tiles, n_gates, log2, mode=2, md_init=7)
    first = {int(wtl[e]) for e in range(E) if hist[e] > 0 and wtl[e] < max_tiles}
    for t in range(min(total, max_tiles)):
        assert md2[t] == (wmd[t] if t in first else 7)


def test_expt_data_reference_case(orc):
    """tests/test_moe.py:385-436: 8 experts, hist ~ randint(0, 200) seed 42, tile 64, 10 spare tiles."""
    torch.manual_seed(42)
    hist = torch.randint(0, 200, (8,), dtype=torch.int32).numpy()
    max_tiles = int(sum((h + 63) // 64 for h in hist)) + 10
    ts, tl, md = orc.expt_data(hist, max_tiles, int(hist.sum()), 6, mode=1)
    acc, tacc = 0, 0
    for e in range(8):
        assert ts[e] == acc and tl[e] == tacc
        for t in range((int(hist[e]) + 63) // 64):
            assert md[tacc + t] == (t << 16) | e
        acc += int(hist[e])
        tacc += (int(hist[e]) + 63) // 64
    assert ts[8] == hist.sum() and tl[8] == tacc


# ---------------------------------------------------------------- compute_indx

def numpy_partials(indx_flat, K, E):
    G = 128 * K
    nb = (len(indx_flat) + G - 1) // G
    cnt = np.zeros((nb, E), np.int64)
    for b in range(nb):
        v = indx_flat[b * G:(b + 1) * G]
        v = v[(v >= 0) & (v < E)]
        cnt[b] = np.bincount(v, minlength=E)
    return (np.cumsum(cnt, 0) - cnt).astype(np.int32), cnt.sum(0)


@pytest.mark.parametrize("T,K,E", [(1, 2, 8), (300, 2, 8), (1000, 8, 256), (129, 4, 1024), (77, 16, 40), (500, 1, 3)])
def test_compute_indx_stable_argsort(orc, T, K, E):
    rng = np.random.default_rng(T + K + E)
    indx = rng.integers(0, E, size=(T, K)).astype(np.int32)
    indx[rng.random((T, K)) < 0.05] = -1  # dropped gates
    flat = indx.ravel()
    scal = rng.integers(0, 0x7F00, size=T * K).astype(np.uint16)
    po, hist = numpy_partials(flat, K, E)
    tokens_start = np.concatenate([[0], np.cumsum(hist)[:-1]]).astype(np.int32)
    n_valid = int(hist.sum())
    g, s, gs = orc.compute_indx(flat, scal, K, tokens_start, po, n_slots=n_valid)
    valid = np.nonzero(flat >= 0)[0]
    order = valid[np.argsort(flat[valid], kind="stable")]
    assert np.array_equal(g, order.astype(np.int32))
    inv = np.full(T * K, -1, np.int32)
    inv[order] = np.arange(n_valid)
    assert np.array_equal(s, inv)
    assert np.array_equal(gs, scal[order])
    # the carried form (no partials) gives the same placement
    g2, s2, gs2 = orc.compute_indx(flat, scal, K, tokens_start, None, n_slots=n_valid)
    assert np.array_equal(g2, g) and np.array_equal(s2, s) and np.array_equal(gs2, gs)


def test_compute_indx_matches_ogs_routing(orc):
    """The gather index of the OGS test helper (tests/test_moe.py:97-128) for top-2 of 8."""
    rng = np.random.default_rng(3)
    assigns = np.stack([rng.choice(8, 2, replace=False) for _ in range(700)]).astype(np.int32)
    hist, offs, gather, _ = orc.ogs_routing(assigns, 8)
    g, _, _ = orc.compute_indx(assigns.ravel(), None, 2, offs, None)
    assert np.array_equal(g, gather)


# ---------------------------------------------------------------- align_block_size

@pytest.mark.parametrize("n,E,bs", [(0, 8, 64), (1, 1, 16), (256, 8, 64), (5000, 256, 128), (3000, 1024, 16), (999, 3, 7)])
def test_align_block_size_numpy(orc, n, E, bs):
    rng = np.random.default_rng(n + E + bs)
    ids = rng.integers(0, E, size=n).astype(np.int32)
    if n:
        ids[rng.random(n) < 0.03] = -1
    s, eids, cum, total = orc.align_block_size(ids, E, bs)
    cnt = np.bincount(ids[ids >= 0], minlength=E)
    padded = (cnt + bs - 1) // bs * bs
    assert np.array_equal(cum, np.concatenate([[0], np.cumsum(padded)]).astype(np.int32))
    assert total == padded.sum()
    order = np.nonzero(ids >= 0)[0]
    order = order[np.argsort(ids[order], kind="stable")]
    want = np.full(total, n, np.int32)
    pos = np.concatenate([cum[e] + np.arange(cnt[e]) for e in range(E)]) if E else np.zeros(0, np.int64)
    want[pos.astype(np.int64)] = order
    assert np.array_equal(s, want)
    assert np.array_equal(eids, np.repeat(np.arange(E), padded // bs).astype(np.int32))


def test_align_block_size_reference_case(orc):
    """tests/test_moe.py:167-226: 256 ids over 8 experts (seed 42), block 64; the test's own check."""
    torch.manual_seed(42)
    ids = torch.randint(0, 8, (256,), dtype=torch.int32).numpy()
    s, eids, cum, total = orc.align_block_size(ids, 8, 64)
    cnt = np.bincount(ids, minlength=8)
    assert total == int(((cnt + 63) // 64 * 64).sum())
    assert np.array_equal(np.sort(s[s < 256]), np.arange(256))
