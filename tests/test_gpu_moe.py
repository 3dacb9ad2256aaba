"""GPU parity of the A8W8 MoE grouped GEMM against the CPU oracle
(oracle.moe_ref: tests/test_moe.py:733-753 restated, no % M wrap), through the
C ABI and through the reference-named modules.

Routing metadata follows the OGS contract (tests/test_moe.py:97-128) built by
oracle.ogs_routing. Bar: the north-star GEMM tolerance on every routed row;
rows that no tile covers stay untouched.
"""
import numpy as np
import pytest
import torch

import hkq
from gpu_util import assert_gemm_close, dev_f32, dev_u8, host_bf16_f32, require_gpu

pytestmark = pytest.mark.gpu


def dev_i32(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()


def make_problem(orc, T, E, topk, K, N, seed, skew=None):
    rng = np.random.default_rng(seed)
    if skew is None:
        assigns = np.stack([rng.permutation(E)[:topk] for _ in range(T)])
    else:
        assigns = skew(rng, T, E, topk)
    hist, offs, gather, ed = orc.ogs_routing(assigns, E, 128)
    X, xs = orc.quant_rowwise(orc.randn_bf16((T, K), seed=seed + 1), None, "fp8")
    Wf = orc.randn_bf16((E * N, K), seed=seed + 2, std=0.02)
    Wq, ws = orc.quant_rowwise(Wf, None, "fp8")
    return assigns, hist, offs, gather, ed, X, xs.reshape(-1), Wq.reshape(E, N, K), ws.reshape(E, N)


def run_moe(X, W, hist, offs, gather, ed, topk, xs=None, ws=None, bias=None, y_rows=None):
    Xd, Wd = dev_u8(X), dev_u8(W)
    args = dict(gather=dev_i32(gather) if gather is not None else None,
                x_scale=dev_f32(xs) if xs is not None else None,
                w_scale=dev_f32(ws) if ws is not None else None,
                bias=dev_f32(bias) if bias is not None else None)
    Y = hkq.moe_a8w8(Xd, Wd, dev_i32(hist), dev_i32(offs), dev_i32(ed), topk, y_rows=y_rows, **args)
    torch.cuda.synchronize()
    return host_bf16_f32(Y)


def check_rows(orc, Y, ref):
    routed = ~np.isnan(ref).any(axis=1)
    assert_gemm_close(Y[routed], ref[routed], "moe routed rows")
    assert np.all(Y[~routed] == 0)  # output preallocated with zeros: untouched rows stay zero


def test_moe_reference_setup(orc):
    """The reference test's setup (tests/test_moe.py:689-764): T=64, E=8, top-2,
    K=N=256, per-tensor activation scale, per-expert weight scale, bias."""
    require_gpu()
    T, E, topk, K, N = 64, 8, 2, 256, 256
    _, hist, offs, gather, ed, X, _, W, _ = make_problem(orc, T, E, topk, K, N, 1)
    rng = np.random.default_rng(2)
    xs = np.array([0.01], np.float32)
    ws = (rng.random(E) * 0.01).astype(np.float32)
    bias = (rng.standard_normal((E, N)) * 0.1).astype(np.float32)
    Y = run_moe(X, W, hist, offs, gather, ed, topk, xs, ws, bias)
    ref = orc.moe_ref(X, W, xs, ws, bias, gather, hist, offs, ed, topk, 128, "enk")
    check_rows(orc, Y, ref)


# At most 32 routed rows (or 64 with N <= 4096): the decode (streaming)
# kernel, with 16 or 64 columns per workgroup (N > 4096), one, two or four
# 16-row groups, ragged N and K-steps uneven over the 4 waves; (24, 2, 2, 384,
# 4104) has 48 rows and a wide N, so it takes the tiled kernel. N >= 8192 (32
# or more column tiles) walks the columns in XCD-aligned blocks of 8: 8320 has
# 33 column tiles (a last block of one), 700 x 3 with topk 2 odd pair groups.
@pytest.mark.parametrize("T,E,topk,K,N", [(300, 4, 2, 512, 520), (1, 8, 2, 256, 512), (1000, 8, 2, 1024, 1024),
                                          (257, 3, 1, 384, 260), (77, 4, 2, 320, 256), (5, 8, 2, 512, 4100),
                                          (16, 8, 2, 384, 1000), (16, 4, 2, 640, 4200), (30, 8, 2, 256, 520),
                                          (24, 2, 2, 384, 4104), (300, 4, 2, 256, 8320), (700, 3, 2, 384, 9216)])
def test_moe_per_token_per_channel(orc, T, E, topk, K, N):
    require_gpu()
    _, hist, offs, gather, ed, X, xs, W, ws = make_problem(orc, T, E, topk, K, N, T + N)
    Y = run_moe(X, W, hist, offs, gather, ed, topk, xs, ws)
    ref = orc.moe_ref(X, W, xs, ws, None, gather, hist, offs, ed, topk, 128, "enk")
    check_rows(orc, Y, ref)


def test_moe_skewed_routing_and_padding(orc):
    """Most tokens on one expert (several 128-row blocks), two experts empty,
    and -1 padding entries appended to ExptData."""
    require_gpu()
    T, E, topk, K, N = 600, 6, 2, 256, 512

    def skew(rng, T, E, topk):
        a = np.zeros((T, topk), np.int64)
        a[:, 0] = 0
        a[:, 1] = np.where(rng.random(T) < 0.8, 1, 3)
        return a

    _, hist, offs, gather, ed, X, xs, W, ws = make_problem(orc, T, E, topk, K, N, 7, skew)
    assert hist[2] == 0 and hist[4] == 0 and hist[0] == T
    ed_pad = np.concatenate([ed, np.full(5, -1, np.int32)])
    Y = run_moe(X, W, hist, offs, gather, ed_pad, topk, xs, ws)
    ref = orc.moe_ref(X, W, xs, ws, None, gather, hist, offs, ed, topk, 128, "enk")
    check_rows(orc, Y, ref)


# The persistent stream (at least two work units per CU, K a multiple of
# 1024): stream tiles over whole block pairs (entries (e, b even), (e, b + 1)),
# the lone blocks before or after them; the same products and epilogue as the tiled
# kernel, which pairs entries by position, so the outputs agree bit for bit
# (HKQ_MOE_STREAM=0 selects the tiled kernel). Uneven routing (odd block
# counts) with per-token, per-tensor and absent scales, one per expert or per
# channel; the entries in the producers' order, rotated by one (a pair across
# the list's wrap) and reversed (no pair: every block lone). Every case is also
# checked against the oracle. Without scales the outputs are raw code-product
# sums (terms up to 448^2, results far smaller than the sum of |terms|), which
# the FP8 MFMA does not accumulate exactly: that case is held to the bf16 bar
# plus 2^-14 of the sum of |terms| (the |codes| products; measured on MI355X:
# at most ~2^-17.7 of it).
@pytest.mark.parametrize("xs_kind,ws_kind,order", [("token", "channel", "sorted"), ("tensor", "expert", "sorted"),
                                                   ("none", "none", "sorted"), ("token", "channel", "rotated"),
                                                   ("token", "expert", "reversed")])
def test_moe_stream_matches_tiled(orc, monkeypatch, xs_kind, ws_kind, order):
    require_gpu()
    T, E, topk, K, N = 2304, 5, 2, 1024, 16384

    def uneven(rng, T, E, topk):
        p = np.array([0.35, 0.25, 0.2, 0.12, 0.08])
        out = np.zeros((T, topk), np.int64)
        for t in range(T):
            out[t] = rng.choice(E, size=topk, replace=False, p=p)
        return out

    _, hist, offs, gather, ed, X, xs, W, ws = make_problem(orc, T, E, topk, K, N, 31, uneven)
    assert len(ed) // 2 * (N // 256) >= 1024  # four units per CU: the stream runs (two suffice)
    assert any(np.bincount(ed[ed >= 0] & 0xFFFF) % 2 == 1)  # an expert with an odd block count
    if order == "rotated":
        ed = np.roll(ed, 1)
    elif order == "reversed":
        ed = ed[::-1].copy()
    if xs_kind == "tensor":
        xs = np.array([0.02], np.float32)
    if ws_kind == "expert":
        ws = (np.random.default_rng(32).random(E) * 0.01 + 0.001).astype(np.float32)
    xs_a = None if xs_kind == "none" else xs
    ws_a = None if ws_kind == "none" else ws
    Y = run_moe(X, W, hist, offs, gather, ed, topk, xs_a, ws_a)
    monkeypatch.setenv("HKQ_MOE_STREAM", "0")
    Y0 = run_moe(X, W, hist, offs, gather, ed, topk, xs_a, ws_a)
    assert np.array_equal(Y, Y0), "stream and tiled kernels disagree"
    if xs_a is not None and ws_a is not None:
        ref = orc.moe_ref(X, W, xs_a, ws_a, None, gather, hist, offs, ed, topk, 128, "enk")
        check_rows(orc, Y, ref)
    else:
        one, ones = np.array([1.0], np.float32), np.ones(E, np.float32)
        ref = orc.moe_ref(X, W, one, ones, None, gather, hist, offs, ed, topk, 128, "enk")
        absum = orc.moe_ref(X & 0x7F, W & 0x7F, one, ones, None, gather, hist, offs, ed, topk, 128, "enk")
        routed = ~np.isnan(ref).any(axis=1)
        err = np.abs(Y[routed].astype(np.float64) - ref[routed])
        assert np.all(err <= 0.02 + 0.01 * np.abs(ref[routed]) + 2.0 ** -14 * absum[routed])
        assert np.all(Y[~routed] == 0)


# The stream kernel's ragged store branch: N % 8 == 4 (a row's last 8-column
# piece holds 4 columns inside C) and Y rows padded past N, the padding checked
# untouched. Still four units per CU, so the stream runs.
def test_moe_stream_ragged_n_padded_y(orc, monkeypatch):
    require_gpu()
    T, E, topk, K, N, pad = 2304, 5, 2, 1024, 16388, 12
    _, hist, offs, gather, ed, X, xs, W, ws = make_problem(orc, T, E, topk, K, N, 41)
    assert len(ed) // 2 * ((N + 255) // 256) >= 1024 and N % 8 == 4
    sentinel = 0x7F7F  # a bf16 NaN pattern no kernel writes

    def run():
        Yp = torch.full((T * topk, N + pad), sentinel, dtype=torch.int16, device="cuda").view(torch.bfloat16)
        Yp[:, :N] = 0
        hkq.moe_a8w8(dev_u8(X), dev_u8(W), dev_i32(hist), dev_i32(offs), dev_i32(ed), topk, gather=dev_i32(gather),
                     x_scale=dev_f32(xs), w_scale=dev_f32(ws), Y=Yp[:, :N])
        torch.cuda.synchronize()
        assert torch.all(Yp[:, N:].view(torch.int16) == sentinel), "padding of Y rows written"
        return host_bf16_f32(Yp[:, :N])

    Y = run()
    monkeypatch.setenv("HKQ_MOE_STREAM", "0")
    Y0 = run()
    assert np.array_equal(Y, Y0), "stream and tiled kernels disagree"
    check_rows(orc, Y, orc.moe_ref(X, W, xs, ws, None, gather, hist, offs, ed, topk, 128, "enk"))


# The reference's N-contiguous [E, K, N] weights read in place (hkq_moe_a8w8_kn:
# K-tiles staged as rows of K, the MFMA operand built with transposed LDS
# reads): the products and their order are those of the K-contiguous path, so
# every output element is the same bits. Cases: the persistent stream (uneven
# routing: lone blocks, 64-row tiles), the tiled kernel, decode-sized routing,
# a bias and per-channel scales (the general epilogue), N that is not a
# multiple of 256 or 16 (the last column chunk reads the next row's bytes into
# columns that are never stored), and rows of K padded past N.
@pytest.mark.parametrize("T,E,topk,K,N,pad,stream,bias", [(2304, 5, 2, 1024, 16384, 0, True, False),
                                                          (2304, 5, 2, 1024, 16384, 0, False, False),
                                                          (4, 8, 2, 1024, 512, 0, True, False),
                                                          (300, 4, 2, 512, 1000, 24, True, True),
                                                          (700, 3, 2, 2048, 4104, 8, True, False)])
def test_moe_kn_matches_kmajor(orc, monkeypatch, T, E, topk, K, N, pad, stream, bias):
    require_gpu()

    def uneven(rng, T, E, topk):
        p = np.linspace(2.0, 1.0, E)
        p /= p.sum()
        out = np.zeros((T, topk), np.int64)
        for t in range(T):
            out[t] = rng.choice(E, size=topk, replace=False, p=p)
        return out

    _, hist, offs, gather, ed, X, xs, W, ws = make_problem(orc, T, E, topk, K, N, 51, uneven)
    Wkn = np.zeros((E, K, N + pad), np.uint8)
    Wkn[:, :, :N] = W.transpose(0, 2, 1)
    b = (np.random.default_rng(52).standard_normal((E, N)) * 0.1).astype(np.float32) if bias else None
    if not stream:
        monkeypatch.setenv("HKQ_MOE_STREAM", "0")
    args = dict(gather=dev_i32(gather), x_scale=dev_f32(xs), w_scale=dev_f32(ws),
                bias=dev_f32(b) if b is not None else None)
    Xd, hd, od, edd = dev_u8(X), dev_i32(hist), dev_i32(offs), dev_i32(ed)
    Y = hkq.moe_a8w8(Xd, dev_u8(W), hd, od, edd, topk, **args)
    Wkn_d = dev_u8(Wkn)[:, :, :N]  # [E, K, N] view with row stride N + pad
    Ykn = hkq.moe_a8w8(Xd, Wkn_d, hd, od, edd, topk, w_kn=True, **args)
    torch.cuda.synchronize()
    assert torch.equal(Y, Ykn), "N-contiguous weights give other bits than K-contiguous ones"
    check_rows(orc, host_bf16_f32(Ykn), orc.moe_ref(X, W, xs, ws, b, gather, hist, offs, ed, topk, 128, "enk"))


def test_moe_entry_order_and_pairing(orc):
    """ExptData in another order than the producers write it: consecutive
    entries that are blocks b, b+1 of one expert run as one 256-row tile, any
    other entry as a 128-row tile; every listed block is computed once either
    way (an expert with an odd block count puts a pair across two experts)."""
    require_gpu()
    T, E, topk, K, N = 700, 5, 2, 256, 256
    _, hist, offs, gather, ed, X, xs, W, ws = make_problem(orc, T, E, topk, K, N, 17)
    ref = orc.moe_ref(X, W, xs, ws, None, gather, hist, offs, ed, topk, 128, "enk")
    rng = np.random.default_rng(3)
    for order in (np.arange(len(ed))[::-1], rng.permutation(len(ed)), np.roll(np.arange(len(ed)), 1)):
        Y = run_moe(X, W, hist, offs, gather, ed[order], topk, xs, ws)
        check_rows(orc, Y, ref)


@pytest.mark.parametrize("bias", [False, True])
def test_moe_per_expert_weight_scale_tiled(orc, bias):
    """One weight scale per expert on the tiled kernel, without a bias (the
    lean epilogue's per-expert branch) and with one (the general epilogue)."""
    require_gpu()
    T, E, topk, K, N = 600, 4, 2, 512, 1040
    _, hist, offs, gather, ed, X, xs, W, _ = make_problem(orc, T, E, topk, K, N, 23)
    rng = np.random.default_rng(24)
    ws = (rng.random(E) * 0.01 + 0.001).astype(np.float32)
    b = (rng.standard_normal((E, N)) * 0.1).astype(np.float32) if bias else None
    Y = run_moe(X, W, hist, offs, gather, ed, topk, xs, ws, b)
    ref = orc.moe_ref(X, W, xs, ws, b, gather, hist, offs, ed, topk, 128, "enk")
    check_rows(orc, Y, ref)


def test_moe_decode_reference_setup(orc):
    """The reference test's scale and bias layout (per-tensor activation scale,
    per-expert weight scale, bias) at a decode size (8 tokens, top-2)."""
    require_gpu()
    T, E, topk, K, N = 8, 8, 2, 256, 320
    _, hist, offs, gather, ed, X, _, W, _ = make_problem(orc, T, E, topk, K, N, 21)
    rng = np.random.default_rng(22)
    xs = np.array([0.01], np.float32)
    ws = (rng.random(E) * 0.01).astype(np.float32)
    bias = (rng.standard_normal((E, N)) * 0.1).astype(np.float32)
    Y = run_moe(X, W, hist, offs, gather, ed, topk, xs, ws, bias)
    ref = orc.moe_ref(X, W, xs, ws, bias, gather, hist, offs, ed, topk, 128, "enk")
    check_rows(orc, Y, ref)


@pytest.mark.parametrize("hist", [[130, 0, 70, 256], [3, 0, 9, 8]])
def test_moe_without_gather(orc, hist):
    """GatherIndx None: tile rows read X[start + gm] directly (pre-sorted X);
    20 rows in all take the decode kernel."""
    require_gpu()
    E, K, N = 4, 256, 256
    hist = np.array(hist, np.int32)
    offs = np.concatenate([[0], np.cumsum(hist)[:-1]]).astype(np.int32)
    ed = np.array([e | (b << 16) for e in range(E) for b in range((hist[e] + 127) // 128)], np.int32)
    rows = int(hist.sum())
    X, xs = orc.quant_rowwise(orc.randn_bf16((rows, K), seed=3), None, "fp8")
    Wq, ws = orc.quant_rowwise(orc.randn_bf16((E * N, K), seed=4, std=0.02), None, "fp8")
    W, ws = Wq.reshape(E, N, K), ws.reshape(E, N)
    Y = run_moe(X, W, hist, offs, None, ed, 1, xs.reshape(-1), ws)
    ident = np.arange(rows, dtype=np.int32)  # gather = s with topk 1 is the same thing
    ref = orc.moe_ref(X, W, xs.reshape(-1), ws, None, ident, hist, offs, ed, 1, 128, "enk")
    check_rows(orc, Y, ref)


def test_moe_malformed_metadata_does_not_fault(orc):
    """Entries naming an expert >= E, gather values past T and an offset past
    the gather index are skipped or read zero; the valid tiles are exact."""
    require_gpu()
    T, E, topk, K, N = 128, 2, 1, 128, 256
    _, hist, offs, gather, ed, X, xs, W, ws = make_problem(orc, T, E, topk, K, N, 11)
    # expert 7, block 9 of expert 1, and words with bit 31 set other than -1
    # (their block id would be negative)
    bad = np.concatenate([ed, np.array([7 | (0 << 16), 1 | (9 << 16), -0x7FFFFFFF, -0x7FFF0000], np.int32)])
    g2 = gather.copy()
    g2[5] = T * topk + 40  # token past T: the row reads zero
    Y = run_moe(X, W, hist, offs, g2, bad, topk, xs, ws)
    ref = orc.moe_ref(X, W, xs, ws, None, gather, hist, offs, ed, topk, 128, "enk")
    ref[5] = 0.0
    check_rows(orc, Y, ref)


def test_moe_gather_division_bounds(orc):
    """Gather values are divided by top_k through a reciprocal multiply: values
    at the top of the int32 range give tokens past T (rows read zero), and
    2T - 1 with top_k 2 gives the last token exactly."""
    require_gpu()
    T, E, topk, K, N = 128, 2, 2, 128, 256
    _, hist, offs, gather, ed, X, xs, W, ws = make_problem(orc, T, E, topk, K, N, 12)
    g2 = gather.copy()
    g2[3] = 0x7FFFFFFF  # token 2^30 - 1, past T
    g2[4] = 0x7FFFFFFE
    g2[6] = 2 * T - 1  # token T - 1
    g2[7] = 2 * T      # token T, past T
    Y = run_moe(X, W, hist, offs, g2, ed, topk, xs, ws)
    g_ref = g2.copy()
    g_ref[[3, 4, 7]] = 0  # any valid value: those rows are zeroed below
    ref = orc.moe_ref(X, W, xs, ws, None, g_ref, hist, offs, ed, topk, 128, "enk")
    ref[[3, 4, 7]] = 0.0
    check_rows(orc, Y, ref)


def mixtral_routing(orc, T, E, topk, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    logits = torch.randn(T, E, generator=g)
    assigns = torch.topk(torch.softmax(logits, -1), topk, dim=-1).indices.numpy()
    return orc.ogs_routing(assigns, E, 128)


def device_weights_fp8(E, N, K, seed):
    """E*N x K weights ~N(0, 0.02) drawn on the device and quantized per row
    by the GPU quantizer (bit-exact with the oracle's, tests/test_gpu_quant.py);
    returns the codes [E, N, K] and scales [E, N] on the host."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn(E * N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    Wq_d, ws_d = hkq.per_token_quant(w)
    torch.cuda.synchronize()
    del w
    return Wq_d.view(torch.uint8).cpu().numpy().reshape(E, N, K), ws_d.cpu().numpy().reshape(E, N)


@pytest.mark.parametrize("K,N", [(4096, 28672), (14336, 4096)])
def test_moe_mixtral_full(orc, K, N):
    """BASELINE MoE shapes (Mixtral-8x7B: T=4096, E=8, top-2; gate/up K=4096,
    N=28672 and down K=14336, N=4096), softmax top-2 routing from seeded logits,
    per-token x per-channel scales: every routed output row against the fp32
    oracle (oracle.moe_ref_f32, pinned in tests/test_oracle_moe.py)."""
    require_gpu()
    T, E, topk = 4096, 8, 2
    hist, offs, gather, ed = mixtral_routing(orc, T, E, topk, K)
    X, xs = orc.quant_rowwise(orc.randn_bf16((T, K), seed=K + 1), None, "fp8")
    xs = xs.reshape(-1)
    W, ws = device_weights_fp8(E, N, K, seed=K + 2)
    Y = run_moe(X, W, hist, offs, gather, ed, topk, xs, ws)
    ref = orc.moe_ref_f32(X, W, xs, ws, gather, hist, offs, ed, topk)
    assert not np.isnan(ref).any()  # every (token, choice) routed
    assert_gemm_close(Y, ref, f"moe mixtral K={K} N={N}")


@pytest.mark.parametrize("K,N", [(4096, 28672), (14336, 4096)])
def test_moe_mixtral_reference_layout_module(orc, K, N):
    """The reference's own call shape at Mixtral size: moe_op_gemm_a8w8_tk with
    N-contiguous [E, K, N] weights (stride_wk = N, stride_wn = 1,
    tests/test_moe.py:723-729), read in place by the kernels; every routed row
    against the fp32 oracle."""
    require_gpu()
    import hipkittens as hk

    T, E, topk = 4096, 8, 2
    hist, offs, gather, ed = mixtral_routing(orc, T, E, topk, K)
    X, xs = orc.quant_rowwise(orc.randn_bf16((T, K), seed=K + 11), None, "fp8")
    xs = xs.reshape(-1)
    W, ws = device_weights_fp8(E, N, K, seed=K + 12)
    Wkn = dev_u8(W).transpose(1, 2).contiguous().view(torch.float8_e4m3fn)  # [E, K, N]
    Y = torch.zeros((T * topk, N), dtype=torch.bfloat16, device="cuda")
    grid_m, grid_n = len(ed), (N + 127) // 128
    hk.moe.a8w8.moe_a8w8(dev_u8(X).view(torch.float8_e4m3fn), Wkn, Y, dev_f32(xs), dev_f32(ws), None,
                         dev_i32(gather), dev_i32(hist), dev_i32(offs), dev_i32(ed), N, K, grid_m, grid_n, topk,
                         N, 1, K, 1, K * N, N, 1, False, 0.0)
    torch.cuda.synchronize()
    del Wkn
    ref = orc.moe_ref_f32(X, W, xs, ws, gather, hist, offs, ed, topk)
    assert not np.isnan(ref).any()
    assert_gemm_close(host_bf16_f32(Y), ref, f"moe mixtral [E, K, N] module K={K} N={N}")


# ---------------------------------------------------------------------------
# Block-scale MoE (per-K-group scales): moe_op_gemm_a8w8_blockscale with
# group_k < K (kernel.cpp:114-145 of the reference)
# ---------------------------------------------------------------------------

def run_moe_bs(X, W, hist, offs, gather, ed, topk, xs, ws, gk, gn, bias=None, y_rows=None):
    Y = hkq.moe_a8w8_blockscale(dev_u8(X), dev_u8(W), dev_i32(hist), dev_i32(offs), dev_i32(ed), topk, dev_f32(xs),
                                dev_f32(ws), gk, gn, gather=dev_i32(gather) if gather is not None else None,
                                bias=dev_f32(bias) if bias is not None else None, y_rows=y_rows)
    torch.cuda.synchronize()
    return host_bf16_f32(Y)


# group_k 64 / 128 / 192 (one, two, three K-tiles per group), group_n 1 (per
# column), 7 (groups across sub-tiles), 64 and 128 (one scale per sub-tile),
# ragged N, decode-sized and multi-block routing, a bias. group_k = 128 * 2^j
# with K % 128 == 0 takes the 8-wave kernel (128-wide K-tiles, routing blocks
# in pairs): (300, ..., 128, 1), (700, ..., 128, 128), (600, ..., 256, 7),
# (900, ..., 128, 64), (500, ..., 512, 1), and group_k past K (100, ..., 128,
# 256, 256, 128); group_k 384 (3 K-tiles), 192, and 128 with K % 128 == 64
# (300, ..., 320, 264, 128, 64) take the 64-wide kernel.
@pytest.mark.parametrize("T,E,topk,K,N,gk,gn", [(64, 8, 2, 256, 256, 64, 64), (300, 4, 2, 512, 520, 128, 1),
                                                (130, 3, 1, 384, 260, 192, 7), (5, 8, 2, 640, 1000, 64, 128),
                                                (700, 5, 2, 1024, 512, 128, 128), (16, 2, 2, 128, 4100, 64, 1),
                                                (600, 3, 2, 512, 1000, 256, 7), (900, 4, 2, 768, 264, 128, 64),
                                                (500, 2, 2, 1024, 512, 512, 1), (200, 2, 2, 768, 256, 384, 128),
                                                (300, 4, 2, 320, 264, 128, 64), (100, 3, 2, 128, 256, 256, 128)])
def test_moe_blockscale(orc, T, E, topk, K, N, gk, gn):
    require_gpu()
    _, hist, offs, gather, ed, X, _, W, _ = make_problem(orc, T, E, topk, K, N, T + K + gn)
    rng = np.random.default_rng(T + N)
    G, C = (K + gk - 1) // gk, (N + gn - 1) // gn
    xs = (rng.random((T, G)) * 0.02 + 0.005).astype(np.float32)
    ws = (rng.random((E, G, C)) * 0.002 + 0.0005).astype(np.float32)
    bias = (rng.standard_normal((E, N)) * 0.1).astype(np.float32) if T % 2 == 0 else None
    Y = run_moe_bs(X, W, hist, offs, gather, ed, topk, xs, ws, gk, gn, bias)
    ref = orc.moe_blockscale_ref(X, W, xs, ws, bias, gather, hist, offs, ed, topk, gk, gn)
    check_rows(orc, Y, ref)


# N-contiguous [E, K, N] weights through both block-scale kernels (the 8-wave
# one for group_k = 128 * 2^j, the 64-wide one otherwise), read in place: the
# same bits as the K-contiguous weights, ragged N and padded rows of K
# included.
@pytest.mark.parametrize("T,E,topk,K,N,gk,gn,pad", [(700, 5, 2, 1024, 512, 128, 128, 0),
                                                     (600, 3, 2, 512, 1000, 256, 7, 24),
                                                     (300, 4, 2, 320, 264, 64, 64, 8),
                                                     (64, 8, 2, 256, 256, 64, 64, 0)])
def test_moe_blockscale_kn_matches_kmajor(orc, T, E, topk, K, N, gk, gn, pad):
    require_gpu()
    _, hist, offs, gather, ed, X, _, W, _ = make_problem(orc, T, E, topk, K, N, 61)
    rng = np.random.default_rng(62)
    G, C = -(-K // gk), -(-N // gn)
    xs = (rng.random((T, G)) * 0.02 + 0.001).astype(np.float32)
    ws = (rng.random((E, G, C)) * 0.02 + 0.001).astype(np.float32)
    Wkn = np.zeros((E, K, N + pad), np.uint8)
    Wkn[:, :, :N] = W.transpose(0, 2, 1)
    Xd, hd, od, edd, gd = dev_u8(X), dev_i32(hist), dev_i32(offs), dev_i32(ed), dev_i32(gather)
    xsd, wsd = dev_f32(xs), dev_f32(ws)
    Y = hkq.moe_a8w8_blockscale(Xd, dev_u8(W), hd, od, edd, topk, xsd, wsd, gk, gn, gather=gd)
    Ykn = hkq.moe_a8w8_blockscale(Xd, dev_u8(Wkn)[:, :, :N], hd, od, edd, topk, xsd, wsd, gk, gn, gather=gd, w_kn=True)
    torch.cuda.synchronize()
    assert torch.equal(Y, Ykn), "N-contiguous weights give other bits than K-contiguous ones"
    ref = orc.moe_blockscale_ref(X, W, xs, ws, None, gather, hist, offs, ed, topk, gk, gn)
    check_rows(orc, host_bf16_f32(Ykn), ref)


def test_moe_blockscale_padding_and_malformed_entries(orc):
    """-1 padding, an expert past E and words with bit 31 set are skipped; a
    token past T reads zero."""
    require_gpu()
    T, E, topk, K, N = 200, 3, 2, 256, 256
    _, hist, offs, gather, ed, X, _, W, _ = make_problem(orc, T, E, topk, K, N, 5)
    rng = np.random.default_rng(6)
    xs = (rng.random((T, 4)) * 0.01).astype(np.float32)
    ws = (rng.random((E, 4, 4)) * 0.001).astype(np.float32)
    bad = np.concatenate([ed, np.array([-1, 9, -0x7FFFFFFF], np.int32)])
    g2 = gather.copy()
    g2[3] = T * topk + 10
    Y = run_moe_bs(X, W, hist, offs, g2, bad, topk, xs, ws, 64, 64)
    ref = orc.moe_blockscale_ref(X, W, xs, ws, None, gather, hist, offs, ed, topk, 64, 64)
    ref[3] = 0.0
    check_rows(orc, Y, ref)


@pytest.mark.parametrize("shift", [0, 1])
def test_moe_blockscale_many_words(orc, shift):
    """More than 512 ExptData words (64 experts x top-8 over 8192 tokens): the
    8-wave kernel's workgroups find their computing word 512 words at a time,
    so pairs sit across lane groups and across the 512-word steps; shift 1
    puts a -1 word first, moving every pair by one position."""
    require_gpu()
    T, E, topk, K, N = 8192, 64, 8, 256, 256
    _, hist, offs, gather, ed, X, _, W, _ = make_problem(orc, T, E, topk, K, N, 71)
    assert len(ed) > 512
    words = np.concatenate([np.full(shift, -1, np.int32), ed]).astype(np.int32)
    rng = np.random.default_rng(72)
    xs = (rng.random((T, K // 128)) * 0.02 + 0.005).astype(np.float32)
    ws = (rng.random((E, K // 128, N // 128)) * 0.002 + 0.0005).astype(np.float32)
    Y = run_moe_bs(X, W, hist, offs, gather, words, topk, xs, ws, 128, 128)
    ref = orc.moe_blockscale_ref(X, W, xs, ws, None, gather, hist, offs, words, topk, 128, 128)
    assert (~np.isnan(ref).any(axis=1)).all()  # every (token, choice) routed
    check_rows(orc, Y, ref)


@pytest.mark.parametrize("gk,gn", [(128, 128), (256, 1)])
def test_moe_blockscale_block_pairs(orc, gk, gn):
    """The 8-wave kernel computes two routing blocks of an expert per workgroup
    when their ExptData words are adjacent (b even, then b + 1). Words
    shuffled, a pair split by a -1, a duplicated word and dropped words: every
    listed block is computed, the blocks of dropped words stay untouched."""
    require_gpu()
    T, E, topk, K, N = 700, 2, 2, 512, 384
    _, hist, offs, gather, ed, X, _, W, _ = make_problem(orc, T, E, topk, K, N, 31)
    rng = np.random.default_rng(32)
    G, C = K // gk, (N + gn - 1) // gn
    xs = (rng.random((T, G)) * 0.02 + 0.005).astype(np.float32)
    ws = (rng.random((E, G, C)) * 0.002 + 0.0005).astype(np.float32)
    live = [int(w) for w in ed if w >= 0]
    assert len(live) >= 10  # several blocks per expert
    # drop expert 0's block 3 (block 2 then runs alone) and expert 1's block 0
    # (its block 1 has no partner), duplicate one word, split a pair with -1,
    # and put the rest in a shuffled order
    kept = [w for w in live if w not in (0 | (3 << 16), 1 | (0 << 16))]
    order = list(rng.permutation(len(kept)))
    words = [kept[i] for i in order] + [0 | (4 << 16), -1, 0 | (5 << 16), kept[0]]
    # and one adjacent pair in place: expert 1, blocks 2 and 3
    words = [1 | (2 << 16), 1 | (3 << 16)] + words
    bad = np.array(words, np.int32)
    Y = run_moe_bs(X, W, hist, offs, gather, bad, topk, xs, ws, gk, gn)
    ref = orc.moe_blockscale_ref(X, W, xs, ws, None, gather, hist, offs, bad, topk, gk, gn)
    dropped = orc.moe_blockscale_ref(X, W, xs, ws, None, gather, hist, offs,
                                     np.array([0 | (3 << 16), 1], np.int32), topk, gk, gn)
    assert (~np.isnan(dropped).any(axis=1)).sum() > 0  # the dropped blocks hold routed rows
    check_rows(orc, Y, ref)


def test_moe_blockscale_padded_rows(orc):
    """The 8-wave kernel with Y rows of pitch N + 4 (16-byte aligned rows, N %
    8 == 4: the last 16-byte piece of a row straddles N): the padding stays
    untouched, unrouted rows stay zero, routed rows match the oracle."""
    require_gpu()
    T, E, topk, K, N, gk, gn = 400, 3, 2, 512, 772, 128, 128
    _, hist, offs, gather, ed, X, _, W, _ = make_problem(orc, T, E, topk, K, N, 61)
    rng = np.random.default_rng(62)
    G, C = K // gk, (N + gn - 1) // gn
    xs = (rng.random((T, G)) * 0.02 + 0.005).astype(np.float32)
    ws = (rng.random((E, G, C)) * 0.002 + 0.0005).astype(np.float32)
    sentinel = 7.0
    Yp = torch.zeros((T * topk, N + 4), dtype=torch.bfloat16, device="cuda")
    Yp[:, N:] = sentinel
    hkq.moe_a8w8_blockscale(dev_u8(X), dev_u8(W), dev_i32(hist), dev_i32(offs), dev_i32(ed), topk, dev_f32(xs),
                            dev_f32(ws), gk, gn, gather=dev_i32(gather), Y=Yp[:, :N])
    torch.cuda.synchronize()
    assert bool((Yp[:, N:] == sentinel).all()), "stores past N reached the row padding"
    ref = orc.moe_blockscale_ref(X, W, xs, ws, None, gather, hist, offs, ed, topk, gk, gn)
    check_rows(orc, host_bf16_f32(Yp[:, :N].contiguous()), ref)


@pytest.mark.parametrize("proj", ["gate_up", "down"])
def test_moe_blockscale_mixtral_group128(orc, proj):
    """Mixtral-8x7B gate/up (T=4096, E=8, top-2, K=4096, N=28672) and down
    (the 8192 expert-sorted rows, K=14336, N=4096: few enough tiles that the
    last round's block pairs are computed as single blocks) with 1x128
    activation groups and 128x128 weight blocks, every routed row against the
    fp32 oracle with the same group scales."""
    require_gpu()
    T, E, topk = 4096, 8, 2
    hist, offs, gather, ed = mixtral_routing(orc, T, E, topk, 77)
    if proj == "gate_up":
        K, N, rows, tk, gat = 4096, 28672, T, topk, gather
    else:
        K, N, rows, tk, gat = 14336, 4096, T * topk, 1, None
    X, xs = orc.quant_rowwise(orc.randn_bf16((rows, K), seed=78), 128, "fp8")   # xs [rows, K/128]
    W, _ = device_weights_fp8(E, N, K, seed=79)
    rng = np.random.default_rng(80)
    ws = (rng.random((E, K // 128, N // 128)) * 2e-4 + 1e-4).astype(np.float32)
    Y = run_moe_bs(X, W, hist, offs, gat, ed, tk, xs, ws, 128, 128)
    ref = orc.moe_ref_f32(X, W, xs, ws, gat, hist, offs, ed, tk, group_k=128, group_n=128)
    assert not np.isnan(ref).any()
    assert_gemm_close(Y, ref, f"moe blockscale mixtral g128 {proj}")


def test_moe_hipkittens_modules(orc):
    """moe_op_gemm_a8w8_tk.moe_a8w8 and moe_op_gemm_a8w8_blockscale_tk with the
    reference argument orders give the C-ABI bytes, with K-contiguous [E, N, K]
    weights and with the reference test's N-contiguous [E, K, N] ones
    (stride_wk = N, stride_wn = 1, tests/test_moe.py:723-729)."""
    require_gpu()
    import hipkittens as hk

    T, E, topk, K, N = 96, 4, 2, 256, 256
    _, hist, offs, gather, ed, X, xs, W, ws = make_problem(orc, T, E, topk, K, N, 21)
    Xd, Wd = dev_u8(X).view(torch.float8_e4m3fn), dev_u8(W).view(torch.float8_e4m3fn)
    Wkn = Wd.transpose(1, 2).contiguous()  # [E, K, N]
    hd, od, gd, edd = dev_i32(hist), dev_i32(offs), dev_i32(gather), dev_i32(ed)
    xsd, wsd = dev_f32(np.array([0.02], np.float32)), dev_f32(ws[:, 0].copy())
    bias = dev_f32(np.random.default_rng(1).standard_normal((E, N)).astype(np.float32))
    ref = hkq.moe_a8w8(Xd, Wd, hd, od, edd, topk, gather=gd, x_scale=xsd, w_scale=wsd, bias=bias)
    grid_m, grid_n = len(ed), (N + 127) // 128
    for Wx, swk, swn in ((Wd, 1, K), (Wkn, N, 1)):
        Y = torch.zeros((T * topk, N), dtype=torch.bfloat16, device="cuda")
        hk.moe.a8w8.moe_a8w8(Xd, Wx, Y, xsd, wsd, bias, gd, hd, od, edd, N, K, grid_m, grid_n, topk,
                             N, 1, K, 1, N * K, swk, swn, False, 0.0)
        torch.cuda.synchronize()
        assert torch.equal(Y, ref)
    # blockscale module, group_k == K: per-token x per-channel scales (strided [T,1] / [E,1,N])
    xs_t = dev_f32(xs.reshape(T, 1))
    ws_c = dev_f32(ws.reshape(E, 1, N))
    ref2 = hkq.moe_a8w8(Xd, Wd, hd, od, edd, topk, gather=gd, x_scale=dev_f32(xs.reshape(-1)), w_scale=dev_f32(ws))
    for Wx, swk, swn in ((Wd, 1, K), (Wkn, N, 1)):
        Y2 = torch.zeros((T * topk, N), dtype=torch.bfloat16, device="cuda")
        hk.moe.a8w8_blockscale.moe_a8w8_blockscale(Xd, Wx, Y2, xs_t, ws_c, None, gd, hd, od, edd, N, K, K, 1,
                                                    grid_m, grid_n, topk, N, 1, K, 1, N * K, swk, swn, 1, 1, N, N, 1)
        torch.cuda.synchronize()
        assert torch.equal(Y2, ref2)


def test_moe_blockscale_reference_call(orc):
    """The reference's own call (tests/test_moe.py:771-815): 64 tokens, 8
    experts, top-2, K = N = 256, group_k = group_n = 64, W [E, K, N]
    (N-contiguous), X_scale [T, K/64], W_scale [E, K/64, N/64], grid_n over
    64-column tiles, through moe_op_gemm_a8w8_blockscale_tk with its argument
    list unchanged (E4M3FN codes in place of the int8 values), against the
    oracle."""
    require_gpu()
    import hipkittens as hk

    num_tokens, num_experts, top_k, K_dim, N_dim, group_k, group_n = 64, 8, 2, 256, 256, 64, 64
    _, hist, offs, gather, ed, X, _, W, _ = make_problem(orc, num_tokens, num_experts, top_k, K_dim, N_dim, 42)
    g = torch.Generator().manual_seed(42)
    X_scale = torch.rand(num_tokens, K_dim // group_k, generator=g) * 0.01
    W_scale = torch.rand(num_experts, K_dim // group_k, N_dim // group_n, generator=g) * 0.01
    Wkn = np.ascontiguousarray(W.transpose(0, 2, 1))  # [E, K, N]
    grid_m, grid_n = len(ed), (N_dim + 63) // 64
    Y = torch.zeros(num_tokens * top_k, N_dim, dtype=torch.bfloat16, device="cuda")
    keep = (dev_u8(X).view(torch.float8_e4m3fn), dev_u8(Wkn).view(torch.float8_e4m3fn), X_scale.cuda(),
            W_scale.cuda(), dev_i32(gather), dev_i32(hist), dev_i32(offs), dev_i32(ed))
    Xd, Wd, xsd, wsd, gd, hd, od, edd = keep
    hk.moe.a8w8_blockscale.moe_a8w8_blockscale(
        Xd, Wd, Y, xsd, wsd, None, gd, hd, od, edd,
        N_dim, K_dim, group_k, group_n, grid_m, grid_n, top_k,
        N_dim, 1,
        K_dim, 1,
        K_dim * N_dim, N_dim, 1,
        K_dim // group_k, 1,
        (K_dim // group_k) * (N_dim // group_n), N_dim // group_n, 1)
    torch.cuda.synchronize()
    ref = orc.moe_blockscale_ref(X, Wkn, X_scale.numpy(), W_scale.numpy(), None, gather, hist, offs, ed, top_k,
                                 group_k, group_n, w_layout="ekn")
    check_rows(orc, host_bf16_f32(Y), ref)
