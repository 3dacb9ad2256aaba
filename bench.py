#!/usr/bin/env python3
"""Headline benchmark: FP8 A8W8 GEMM (per-token x per-channel scales) at
M=4096, N=14336, K=4096 on one MI355X, plus the MXFP4 A4W4 GEMM at
M=4096, N=K=8192 and the per-token FP8 quantizer at [4096, 4096].

A step is one launch of the A8W8 GEMM over resident HBM inputs (synthetic,
seeded on the CPU: acts ~N(0,1), weights ~N(0,0.02), quantized by this
library's own quantizers). Kernel time comes from HIP events recorded on the
stream the kernels are launched on (torch's current stream), bracketing
exactly --steps launches after --warmup untimed ones.

Prints ONE JSON line. `roofline` describes the dominant kernel (the A8W8
GEMM): algorithmic flops per launch / average launch duration against the
MI355X dense FP8 peak; `traffic` is the HBM bytes per launch measured with
rocprofv3 PMC counters (FETCH_SIZE + WRITE_SIZE) and read from the committed
profile summary. `cpu_baseline` times the CPU port of the reference formula
(oracle/cpu_baseline.py) on BASELINE config 0.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "amd-kernels_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_FP8_TFLOPS = 5000.0   # MI355X dense FP8 (e4m3) MFMA
PEAK_FP4_TFLOPS = 10100.0  # MI355X dense MXFP4 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA

HEADLINE = dict(M=4096, N=14336, K=4096)
MXFP4 = dict(M=4096, N=8192, K=8192)
BLOCKSCALE = [(2048, 24576, 1536), (2048, 7168, 18432), (2048, 7168, 2048)]
MOE = dict(T=4096, E=8, topk=2, hidden=4096, ffn=14336)
# batched A8W8 (batch, M, N, K)
BATCHED = (8, 1024, 4096, 4096)
# routing pipelines timed beside the Mixtral one: (tokens, experts, top-k)
ROUTING_EXTRA = [(4096, 256, 8), (32768, 256, 8)]
# fused RMSNorm + quantizer cases: (rows, hidden, kind 0 = FP8 1x128 / 1 = MXFP4)
RMSNORM_CASES = [(4096, 4096, 0), (16384, 7168, 0), (4096, 8192, 1), (16384, 7168, 1)]
# A8W8 shape sweep (N, K) x M of the reference's GEMM benchmark configuration
SWEEP_NK = [(6144, 4096), (4096, 4096), (28672, 4096), (4096, 14336)]
SWEEP_M = [1, 16, 128, 1024, 4096]
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemm_a8w8_4096x14336x4096_pmc.txt")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def seeded_bf16(shape, std, seed):
    import torch

    g = torch.Generator(device="cpu").manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16).cuda()


PREHEAT_S = 0.3  # untimed device load before the warmup steps


def seeded_bf16_dev(shape, std, seed):
    """Like seeded_bf16 but drawn with a seeded device generator (large weights)."""
    import torch

    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(*shape, generator=g, device="cuda") * std).to(torch.bfloat16)


def time_launches(fn, steps, warmup, preheat=PREHEAT_S):
    """Average ms per launch over `steps` back-to-back launches on the current stream.

    Before the `warmup` launches, the kernel runs untimed for `preheat` seconds:
    MI355X engine clocks take tens of milliseconds of sustained load to settle,
    and a handful of warmup launches would otherwise time a ramping clock."""
    import time

    import torch

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < preheat:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def read_traffic():
    """HBM bytes per launch from the committed PMC summary (null if absent)."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    m = re.search(r"^traffic_bytes_per_launch\s*=\s*([0-9.eE+]+)", open(TRAFFIC_FILE).read(), re.M)
    return float(m.group(1)) if m else None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", choices=["a8w8", "mxfp4", "quant", "blockscale", "moe", "fused", "ext", "sweep", "copy"],
                    default=None,
                    help="run one kernel only (for profiling); prints no JSON line. 'copy' is a plain "
                         "1 GiB device copy used to calibrate the HBM byte counters")
    ap.add_argument("--shape", default=None,
                    help="with --only a8w8 / mxfp4 / blockscale: profile this M,N,K instead of the "
                         "benchmark's shape(s) (the block-scale decode rows are skipped)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no multi-GPU path.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import hkq

    torch.cuda.set_device(0)
    steps, warmup = args.steps, args.warmup

    if args.only == "copy":
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        ms = time_launches(lambda: dst.copy_(src), steps, warmup)
        log(json.dumps({"copy_bytes": 1 << 30, "us": round(ms * 1e3, 2), "GB/s": round(2 * (1 << 30) / ms / 1e6, 1)}))
        return

    # ---- A8W8 headline ----
    shape = None
    if args.shape:
        if args.only not in ("a8w8", "mxfp4", "blockscale"):
            print("--shape needs --only a8w8, mxfp4 or blockscale", file=sys.stderr)
            sys.exit(2)
        shape = tuple(int(v) for v in args.shape.split(","))
    M, N, K = shape if shape and args.only == "a8w8" else (HEADLINE["M"], HEADLINE["N"], HEADLINE["K"])
    x = seeded_bf16((M, K), 1.0, 1)
    w = seeded_bf16((N, K), 0.02, 2)
    qa, sa = hkq.per_token_quant(x)
    qb, sb = hkq.per_token_quant(w)
    C = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    torch.cuda.synchronize()
    res = {}
    if args.only in (None, "a8w8"):
        log(f"a8w8 {M}x{N}x{K}: warmup {warmup}, steps {steps}")
        ms = time_launches(lambda: hkq.gemm_a8w8(qa, qb, sa, sb, C), steps, warmup)
        res["a8w8"] = ms
    del x, w

    # ---- MXFP4 ----
    if args.only in (None, "mxfp4"):
        m4, n4, k4 = shape if shape else (MXFP4["M"], MXFP4["N"], MXFP4["K"])
        xa = seeded_bf16((m4, k4), 1.0, 3)
        xw = seeded_bf16((n4, k4), 0.02, 4)
        Aq, As = hkq.mx_quant(xa, True)
        Bq, Bs = hkq.mx_quant(xw, True)
        C4 = torch.empty((m4, n4), dtype=torch.bfloat16, device="cuda")
        torch.cuda.synchronize()
        log(f"mxfp4 {m4}x{n4}x{k4}")
        res["mxfp4"] = time_launches(lambda: hkq.gemm_mxfp4(Aq, As, Bq, Bs, C4), steps, warmup)
        del xa, xw

    # ---- per-token FP8 quantizer, bf16 [4096, 4096] ----
    if args.only in (None, "quant"):
        xq = seeded_bf16((4096, 4096), 1.0, 5)
        q = torch.empty((4096, 4096), dtype=torch.float8_e4m3fn, device="cuda")
        s = torch.empty((4096,), dtype=torch.float32, device="cuda")
        log("per-token quant 4096x4096")
        # pre-bound C-ABI call: a ~10 us kernel would otherwise be timed at the
        # rate Python can enqueue it
        launch = hkq.bind("hkq_per_token_quant", xq.data_ptr(), q.data_ptr(), s.data_ptr(), 4096, 4096, xq.stride(0),
                          q.stride(0), hkq.KIND_FP8, torch.cuda.current_stream().cuda_stream)
        res["quant"] = time_launches(launch, steps, warmup)

    # ---- block-scale FP8 GEMM at the DeepSeek-V3 shapes (1x128 act / 128x128 weight scales) ----
    bs_res = []
    if args.only in (None, "blockscale"):
        for (bm, bn, bk) in ([shape] if shape else BLOCKSCALE):
            xa = seeded_bf16((bm, bk), 1.0, 6)
            xw = seeded_bf16((bn, bk), 0.02, 7)
            qa_b, sa_b = hkq.group_quant(xa, 128)
            qw_b, sw_rows = hkq.group_quant(xw, 128)  # per (n, k-group)
            # 128x128 weight blocks: one scale per (k-group, n-block)
            sb_b = sw_rows.view(bn // 128, 128, bk // 128).amax(dim=1).t().contiguous()
            Cb = torch.empty((bm, bn), dtype=torch.bfloat16, device="cuda")
            torch.cuda.synchronize()
            log(f"blockscale {bm}x{bn}x{bk}")
            ms_b = time_launches(lambda: hkq.gemm_blockscale(qa_b, qw_b, sa_b, sb_b, Cb, 128), steps, warmup)
            bs_res.append({"M": bm, "N": bn, "K": bk, "ms": round(ms_b, 5),
                           "tflops": round(2.0 * bm * bn * bk / (ms_b * 1e-3) / 1e12, 2)})
            # decode-size rows on the same weights (the narrow path): HBM-bound, GB/s of weights + activations
            for dm in (() if shape else (1, 16)):
                qa_d, sa_d = qa_b[:dm].contiguous(), sa_b[:dm].contiguous()
                Cd = torch.empty((dm, bn), dtype=torch.bfloat16, device="cuda")
                launch = hkq.bind("hkq_gemm_blockscale", qa_d.data_ptr(), qw_b.data_ptr(), sa_d.data_ptr(),
                                  sb_b.data_ptr(), Cd.data_ptr(), dm, bn, bk, bk, bk, sa_d.stride(0), sb_b.stride(0), bn,
                                  128, torch.cuda.current_stream().cuda_stream)
                ms_d = time_launches(launch, steps, warmup, preheat=0.05)
                byts = dm * bk + bn * bk + 4 * (dm + bn // 128) * (bk // 128) + 2 * dm * bn
                bs_res.append({"M": dm, "N": bn, "K": bk, "us": round(ms_d * 1e3, 2),
                               "GB/s": round(byts / (ms_d * 1e-3) / 1e9, 1)})
            del xa, xw, qa_b, qw_b
        res["blockscale"] = sum(r.get("ms", 0.0) for r in bs_res)

    # ---- A8W8 MoE grouped GEMM, Mixtral-8x7B (E=8, top-2, 4096 tokens, 4096 -> 14336 gate/up, down) ----
    moe_res, routing_res, fused_res = [], [], []
    if args.only in (None, "moe"):
        T, E, topk, hidden, ffn = MOE["T"], MOE["E"], MOE["topk"], MOE["hidden"], MOE["ffn"]
        # routing on the GPU from seeded router logits ~N(0,1): top-2 (with softmax over
        # the chosen logits), tile counts, expert data and gate placement
        logits = seeded_bf16((T, E), 1.0, 8)
        rt, route = hkq.moe_routing_plan(logits, topk, 128)
        route()
        hist, offs, gather, expt_data = rt["hist"], rt["offs"], rt["gather"], rt["expt_data"]
        torch.cuda.synchronize()
        log(f"moe routing T={T} E={E} top-{topk}")
        ms_r = time_launches(route, steps, warmup, preheat=0.05)
        routing_res.append({"T": T, "E": E, "topk": topk, "us": round(ms_r * 1e3, 2), "calls": 4})
        xm = seeded_bf16((T, hidden), 1.0, 9)
        qx, sx = hkq.per_token_quant(xm)

        def expert_weights(nn, kk, seed):
            wq = torch.empty((E, nn, kk), dtype=torch.float8_e4m3fn, device="cuda")
            ws_m = torch.empty((E, nn), dtype=torch.float32, device="cuda")
            for e in range(E):  # per-channel quantization of each expert's [N, K] weights
                hkq.per_token_quant(seeded_bf16_dev((nn, kk), 0.02, seed + e), hkq.KIND_FP8, wq[e], ws_m[e])
            return wq, ws_m

        # the layer: gate/up over gathered tokens -> SwiGLU + per-token FP8 of the
        # expert-sorted rows -> down over those rows (no gather)
        w1, ws1 = expert_weights(2 * ffn, hidden, 10)
        w2, ws2 = expert_weights(hidden, ffn, 40)
        Y1 = torch.empty((T * topk, 2 * ffn), dtype=torch.bfloat16, device="cuda")
        Y2 = torch.empty((T * topk, hidden), dtype=torch.bfloat16, device="cuda")
        q2 = torch.empty((T * topk, ffn), dtype=torch.float8_e4m3fn, device="cuda")
        s2 = torch.empty((T * topk,), dtype=torch.float32, device="cuda")
        hkq.moe_a8w8(qx, w1, hist, offs, expt_data, topk, gather=gather, x_scale=sx, w_scale=ws1, Y=Y1)
        hkq.swiglu_quant(Y1, q=q2, s=s2)
        torch.cuda.synchronize()
        steps_fns = (
            ("gate_up", 2 * ffn, hidden, lambda: hkq.moe_a8w8(qx, w1, hist, offs, expt_data, topk, gather=gather,
                                                              x_scale=sx, w_scale=ws1, Y=Y1)),
            ("down", hidden, ffn, lambda: hkq.moe_a8w8(q2, w2, hist, offs, expt_data, 1, gather=None, x_scale=s2,
                                                       w_scale=ws2, Y=Y2)),
        )
        for name, nn, kk, fn in steps_fns:
            log(f"moe {name} N={nn} K={kk}")
            ms_m = time_launches(fn, steps, warmup)
            moe_res.append({"proj": name, "N": nn, "K": kk, "ms": round(ms_m, 5),
                            "tflops": round(2.0 * T * topk * nn * kk / (ms_m * 1e-3) / 1e12, 2)})
        log(f"swiglu + FP8 [{T * topk}, 2x{ffn}]")
        launch = hkq.bind("hkq_swiglu_quant", Y1.data_ptr(), q2.data_ptr(), s2.data_ptr(), T * topk, ffn, 2 * ffn, ffn,
                          0, 1.0, 0, 0, torch.cuda.current_stream().cuda_stream)
        ms_sw = time_launches(launch, steps, warmup)
        sw_bytes = T * topk * (4 * ffn + ffn + 4)
        fused_res.append({"op": "swiglu_fp8_per_token", "M": T * topk, "F": ffn, "us": round(ms_sw * 1e3, 2),
                          "GB/s": round(sw_bytes / (ms_sw * 1e-3) / 1e9, 1),
                          "pct_hbm_peak": round(100 * sw_bytes / (ms_sw * 1e-3) / 1e9 / PEAK_HBM_GBS, 1)})
        layer_ms = ms_r + sum(r["ms"] for r in moe_res) + ms_sw
        moe_res.append({"proj": "layer (routing + gate_up + swiglu/quant + down)", "ms": round(layer_ms, 5)})
        # decode sizes (the streaming MoE kernel): HBM-bound, GB/s of the active experts' weights
        for td in (1, 8):
            rtd, route_d = hkq.moe_routing_plan(logits[:td].contiguous(), topk, 128)
            route_d()
            hd = rtd["hist"]
            qd, sd = qx[:td].contiguous(), sx[:td].contiguous()
            q2d = q2[: td * topk].contiguous()
            s2d = s2[: td * topk].contiguous()
            Y1d = torch.empty((td * topk, 2 * ffn), dtype=torch.bfloat16, device="cuda")
            Y2d = torch.empty((td * topk, hidden), dtype=torch.bfloat16, device="cuda")
            torch.cuda.synchronize()
            act = int((hd[:E] > 0).sum().item())
            for name, nn, kk, fn in (
                ("gate_up", 2 * ffn, hidden, lambda: hkq.moe_a8w8(qd, w1, hd, rtd["offs"], rtd["expt_data"], topk,
                                                                  gather=rtd["gather"], x_scale=sd, w_scale=ws1,
                                                                  Y=Y1d)),
                ("down", hidden, ffn, lambda: hkq.moe_a8w8(q2d, w2, hd, rtd["offs"], rtd["expt_data"], 1, gather=None,
                                                           x_scale=s2d, w_scale=ws2, Y=Y2d))):
                log(f"moe decode T={td} {name}")
                ms_d = time_launches(fn, steps, warmup, preheat=0.05)
                moe_res.append({"proj": f"decode {name}", "T": td, "active_experts": act, "N": nn, "K": kk,
                                "us": round(ms_d * 1e3, 2), "GB/s": round(act * nn * kk / (ms_d * 1e-3) / 1e9, 1)})
        # block-scale MoE on the same weights: 1x128 activation scales and
        # 128x128 weight-block scales (group_k = group_n = 128)
        g = torch.Generator(device="cuda").manual_seed(50)
        xs_g = torch.rand((T, hidden // 128), generator=g, device="cuda") + 0.5
        s2_g = torch.rand((T * topk, ffn // 128), generator=g, device="cuda") + 0.5
        for name, nn, kk, xx, xsc, wq, gat, tk, yy in (
                ("blockscale gate_up", 2 * ffn, hidden, qx, xs_g, w1, gather, topk, Y1),
                ("blockscale down", hidden, ffn, q2, s2_g, w2, None, 1, Y2)):
            wsc = torch.rand((E, kk // 128, nn // 128), generator=g, device="cuda") + 0.5
            fn = (lambda xx=xx, xsc=xsc, wq=wq, gat=gat, tk=tk, yy=yy, wsc=wsc:
                  hkq.moe_a8w8_blockscale(xx, wq, hist, offs, expt_data, tk, xsc, wsc, 128, 128, gather=gat, Y=yy))
            fn()
            torch.cuda.synchronize()
            log(f"moe {name} N={nn} K={kk}")
            ms_b = time_launches(fn, steps, warmup)
            moe_res.append({"proj": name, "N": nn, "K": kk, "group_k": 128, "group_n": 128, "ms": round(ms_b, 5),
                            "tflops": round(2.0 * T * topk * nn * kk / (ms_b * 1e-3) / 1e12, 2)})
        # the reference's N-contiguous [E, K, N] weights: read in place by the
        # kernels (hkq_moe_a8w8_kn), and the K-major prepack a caller may run once
        w1_kn = w1.view(torch.uint8).transpose(1, 2).contiguous()
        w2_kn = w2.view(torch.uint8).transpose(1, 2).contiguous()
        for name, nn, kk, fn in (
                ("gate_up [E,K,N]", 2 * ffn, hidden, lambda: hkq.moe_a8w8(qx, w1_kn, hist, offs, expt_data, topk,
                                                                          gather=gather, x_scale=sx, w_scale=ws1, Y=Y1,
                                                                          w_kn=True)),
                ("down [E,K,N]", hidden, ffn, lambda: hkq.moe_a8w8(q2, w2_kn, hist, offs, expt_data, 1, gather=None,
                                                                    x_scale=s2, w_scale=ws2, Y=Y2, w_kn=True))):
            log(f"moe {name} N={nn} K={kk}")
            ms_m = time_launches(fn, steps, warmup)
            moe_res.append({"proj": name, "N": nn, "K": kk, "ms": round(ms_m, 5),
                            "tflops": round(2.0 * T * topk * nn * kk / (ms_m * 1e-3) / 1e12, 2)})
        del w2_kn
        w1_nk = torch.empty((E, 2 * ffn, hidden), dtype=torch.uint8, device="cuda")
        pack = hkq.bind("hkq_moe_pack_kmajor", w1_kn.data_ptr(), w1_nk.data_ptr(), E, hidden, 2 * ffn,
                        w1_kn.stride(0), w1_kn.stride(1), w1_nk.stride(0), w1_nk.stride(1),
                        torch.cuda.current_stream().cuda_stream)
        log("moe pack_kmajor [E, K, N] -> [E, N, K]")
        ms_p = time_launches(pack, steps, warmup)
        moe_res.append({"proj": "pack_kmajor", "E": E, "K": hidden, "N": 2 * ffn, "us": round(ms_p * 1e3, 2),
                        "GB/s": round(2 * w1_kn.numel() / (ms_p * 1e-3) / 1e9, 1)})
        del w1, w2, w1_kn, w1_nk

        # MXFP4 experts over the block-sorted routing of the same top-2 choice
        # (moe_align_block_size, 128-row blocks)
        sids, eids, _, tot = hkq.align_block_size(rt["topk_idx"], E, 128)
        total = int(tot.item())
        sids, eids = sids[:total], eids[: total // 128]
        a4, as4 = hkq.mx_quant(xm, True)
        for name, (nn, kk) in (("gate_up", (2 * ffn, hidden)), ("down", (hidden, ffn))):
            xa4, xs4 = (a4, as4) if kk == hidden else hkq.mx_quant(seeded_bf16((T, kk), 1.0, 60), True)
            wq4 = torch.empty((E, nn, kk // 2), dtype=torch.uint8, device="cuda")
            ws4 = torch.empty((E, nn, kk // 32), dtype=torch.uint8, device="cuda")
            for e in range(E):
                hkq.call("hkq_mx_quant", seeded_bf16_dev((nn, kk), 0.02, 70 + e).data_ptr(), wq4[e].data_ptr(),
                         ws4[e].data_ptr(), nn, kk, kk, 1, torch.cuda.current_stream().cuda_stream)
            C4 = torch.empty((T * topk, nn), dtype=torch.bfloat16, device="cuda")
            launch = hkq.bind("hkq_moe_mxfp4", xa4.data_ptr(), wq4.data_ptr(), C4.data_ptr(), xs4.data_ptr(),
                              ws4.data_ptr(), None, None, None,
                              sids.data_ptr(), eids.data_ptr(), nn, kk, T * topk, topk, 0, xa4.stride(0),
                              wq4.stride(0), wq4.stride(1), C4.stride(0), xs4.stride(0), ws4.stride(0), ws4.stride(1),
                              T, E, total // 128, torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            log(f"moe mxfp4 {name} N={nn} K={kk}")
            ms_4 = time_launches(launch, steps, warmup)
            moe_res.append({"proj": f"mxfp4 {name}", "N": nn, "K": kk, "ms": round(ms_4, 5),
                            "tflops": round(2.0 * T * topk * nn * kk / (ms_4 * 1e-3) / 1e12, 2)})
            # the reference's N-contiguous B [E, K/2, N] and scales [E, K/32, N], read in place
            wq4_kn = wq4.transpose(1, 2).contiguous()
            ws4_kn = ws4.transpose(1, 2).contiguous()
            del wq4, ws4
            launch = hkq.bind("hkq_moe_mxfp4_kn", xa4.data_ptr(), wq4_kn.data_ptr(), C4.data_ptr(), xs4.data_ptr(),
                              ws4_kn.data_ptr(), None, None, None,
                              sids.data_ptr(), eids.data_ptr(), nn, kk, T * topk, topk, 0, xa4.stride(0),
                              wq4_kn.stride(0), wq4_kn.stride(1), C4.stride(0), xs4.stride(0), ws4_kn.stride(0),
                              ws4_kn.stride(1), T, E, total // 128, torch.cuda.current_stream().cuda_stream)
            log(f"moe mxfp4 {name} [E,K/2,N] N={nn} K={kk}")
            ms_4 = time_launches(launch, steps, warmup)
            moe_res.append({"proj": f"mxfp4 {name} [E,K/2,N]", "N": nn, "K": kk, "ms": round(ms_4, 5),
                            "tflops": round(2.0 * T * topk * nn * kk / (ms_4 * 1e-3) / 1e12, 2)})
            del wq4_kn, ws4_kn, C4
        res["moe"] = layer_ms
        for (Tr, Er, Kr) in ROUTING_EXTRA:
            lg = seeded_bf16((Tr, Er), 1.0, 30)
            _, route = hkq.moe_routing_plan(lg, Kr, 128)
            ms_r = time_launches(route, steps, warmup, preheat=0.05)
            routing_res.append({"T": Tr, "E": Er, "topk": Kr, "us": round(ms_r * 1e3, 2), "calls": 4})

    # ---- fused RMSNorm + quantizers (HBM-bound) ----
    if args.only in (None, "fused"):
        for (mm, dd, kind) in RMSNORM_CASES:
            xr = seeded_bf16((mm, dd), 1.0, 50)
            wr = seeded_bf16((dd,), 1.0, 51)
            qr, sr = hkq.rmsnorm_quant(xr, wr, 1e-6, kind)
            torch.cuda.synchronize()
            log(f"rmsnorm + {'fp8 1x128' if kind == 0 else 'mxfp4'} [{mm}, {dd}]")
            launch = hkq.bind("hkq_rmsnorm_quant", xr.data_ptr(), wr.data_ptr(), qr.data_ptr(), sr.data_ptr(), mm, dd,
                              dd, qr.stride(0), sr.stride(0), 1e-6, kind, torch.cuda.current_stream().cuda_stream)
            ms_n = time_launches(launch, steps, warmup)
            nb = mm * dd * (2 + (1 + 4 / 128 if kind == 0 else 0.5 + 1 / 32)) + 2 * dd
            fused_res.append({"op": "rmsnorm_fp8_1x128" if kind == 0 else "rmsnorm_mxfp4", "M": mm, "D": dd,
                              "us": round(ms_n * 1e3, 2), "GB/s": round(nb / (ms_n * 1e-3) / 1e9, 1),
                              "pct_hbm_peak": round(100 * nb / (ms_n * 1e-3) / 1e9 / PEAK_HBM_GBS, 1)})
            del xr, qr, sr
        # the plain quantizers of the same family, for comparison
        for (mm, dd) in ((4096, 8192), (16384, 7168)):
            xr = seeded_bf16((mm, dd), 1.0, 52)
            q4 = torch.empty((mm, dd // 2), dtype=torch.uint8, device="cuda")
            s4 = torch.empty((mm, dd // 32), dtype=torch.uint8, device="cuda")
            log(f"mx quant fp4 [{mm}, {dd}]")
            launch = hkq.bind("hkq_mx_quant", xr.data_ptr(), q4.data_ptr(), s4.data_ptr(), mm, dd, dd, 1,
                              torch.cuda.current_stream().cuda_stream)
            ms_q = time_launches(launch, steps, warmup)
            nb = mm * dd * (2 + 0.5 + 1 / 32)
            fused_res.append({"op": "mx_quant_fp4", "M": mm, "D": dd, "us": round(ms_q * 1e3, 2),
                              "GB/s": round(nb / (ms_q * 1e-3) / 1e9, 1),
                              "pct_hbm_peak": round(100 * nb / (ms_q * 1e-3) / 1e9 / PEAK_HBM_GBS, 1)})
            qg = torch.empty((mm, dd), dtype=torch.float8_e4m3fn, device="cuda")
            sg = torch.empty((mm, dd // 128), dtype=torch.float32, device="cuda")
            log(f"group quant fp8 1x128 [{mm}, {dd}]")
            launch = hkq.bind("hkq_group_quant", xr.data_ptr(), qg.data_ptr(), sg.data_ptr(), mm, dd, dd, dd,
                              dd // 128, 128, hkq.KIND_FP8, torch.cuda.current_stream().cuda_stream)
            ms_g = time_launches(launch, steps, warmup)
            nb = mm * dd * (2 + 1 + 4 / 128)
            fused_res.append({"op": "group_quant_fp8_1x128", "M": mm, "D": dd, "us": round(ms_g * 1e3, 2),
                              "GB/s": round(nb / (ms_g * 1e-3) / 1e9, 1),
                              "pct_hbm_peak": round(100 * nb / (ms_g * 1e-3) / 1e9 / PEAK_HBM_GBS, 1)})
            del xr, qg, sg, q4, s4
        res["fused"] = sum(r["us"] for r in fused_res) * 1e-3

    # ---- bf16, batched A8W8 and block-scale multiply-add GEMMs ----
    ext_res = []
    if args.only in (None, "ext"):
        stream = torch.cuda.current_stream().cuda_stream
        mm, nn, kk = HEADLINE["M"], HEADLINE["N"], HEADLINE["K"]
        a16 = seeded_bf16((mm, kk), 1.0, 80)
        b16 = seeded_bf16((nn, kk), 0.02, 81)
        c16 = torch.empty((mm, nn), dtype=torch.bfloat16, device="cuda")
        log(f"bf16 gemm {mm}x{nn}x{kk}")
        launch = hkq.bind("hkq_gemm_bf16", a16.data_ptr(), b16.data_ptr(), c16.data_ptr(), mm, nn, kk, kk, kk, nn,
                          stream)
        ms_e = time_launches(launch, steps, warmup)
        tf = 2.0 * mm * nn * kk / (ms_e * 1e-3) / 1e12
        ext_res.append({"op": "gemm_bf16", "M": mm, "N": nn, "K": kk, "ms": round(ms_e, 5), "tflops": round(tf, 1),
                        "pct_bf16_peak": round(100 * tf / PEAK_BF16_TFLOPS, 1)})
        del a16, b16, c16
        zb, mb, nb_, kb_ = BATCHED
        xb = seeded_bf16((zb * mb, kb_), 1.0, 82)
        wb = seeded_bf16((zb * nb_, kb_), 0.02, 83)
        qxb, sxb = hkq.per_token_quant(xb)
        qwb, swb = hkq.per_token_quant(wb)
        biasb = seeded_bf16((zb, nb_), 1.0, 84)
        cb = torch.empty((zb, mb, nb_), dtype=torch.bfloat16, device="cuda")
        log(f"batched a8w8 {zb}x{mb}x{nb_}x{kb_}")
        launch = hkq.bind("hkq_batched_gemm_a8w8", qxb.data_ptr(), qwb.data_ptr(), sxb.data_ptr(), swb.data_ptr(),
                          biasb.data_ptr(), cb.data_ptr(), zb, mb, nb_, kb_, kb_, kb_, nb_, mb * kb_, nb_ * kb_,
                          mb * nb_, mb, nb_, nb_, stream)
        ms_e = time_launches(launch, steps, warmup)
        tf = 2.0 * zb * mb * nb_ * kb_ / (ms_e * 1e-3) / 1e12
        ext_res.append({"op": "batched_gemm_a8w8", "batch": zb, "M": mb, "N": nb_, "K": kb_, "ms": round(ms_e, 5),
                        "tflops": round(tf, 1), "pct_fp8_peak": round(100 * tf / PEAK_FP8_TFLOPS, 1)})
        del xb, wb, qxb, qwb, cb
        bm, bn, bk = BLOCKSCALE[2]
        qa_b, sa_b = hkq.group_quant(seeded_bf16((bm, bk), 1.0, 85), 128)
        qw_b, sw_rows = hkq.group_quant(seeded_bf16((bn, bk), 0.02, 86), 128)
        sb_b = sw_rows.view(bn // 128, 128, bk // 128).amax(dim=1).t().contiguous()
        ca = seeded_bf16((bm, bn), 1.0, 87)
        cbb = seeded_bf16((bm, bn), 1.0, 88)
        Cm = torch.empty((bm, bn), dtype=torch.bfloat16, device="cuda")
        log(f"blockscale mul_add {bm}x{bn}x{bk}")
        launch = hkq.bind("hkq_gemm_blockscale_mul_add", qa_b.data_ptr(), qw_b.data_ptr(), sa_b.data_ptr(),
                          sb_b.data_ptr(), Cm.data_ptr(), ca.data_ptr(), cbb.data_ptr(), bm, bn, bk, bk, bk,
                          sa_b.stride(0), sb_b.stride(0), bn, bn, bn, 128, stream)
        ms_e = time_launches(launch, steps, warmup)
        ext_res.append({"op": "gemm_blockscale_mul_add", "M": bm, "N": bn, "K": bk, "ms": round(ms_e, 5),
                        "tflops": round(2.0 * bm * bn * bk / (ms_e * 1e-3) / 1e12, 1)})
        res["ext"] = sum(r["ms"] for r in ext_res)

    # ---- A8W8 shape sweep and the MXFP4 M=128 configuration (plans with smaller tiles / split K) ----
    sweep = []
    if args.only in (None, "sweep"):
        log("a8w8 sweep")
        # BASELINE's data: bf16 activations ~N(0,1) and weights ~N(0,0.02),
        # quantized per token / per channel to E4M3FN by this library
        for si, (nn, kk) in enumerate(SWEEP_NK):
            wb, wsb = hkq.per_token_quant(seeded_bf16_dev((nn, kk), 0.02, 100 + si))
            xall, xsall = hkq.per_token_quant(seeded_bf16_dev((max(SWEEP_M), kk), 1.0, 110 + si))
            for mm in SWEEP_M:
                if (mm, nn, kk) == (M, N, K):
                    continue
                xa, xsa = xall[:mm], xsall[:mm]
                Cs = torch.empty((mm, nn), dtype=torch.bfloat16, device="cuda")
                nws = hkq.lib().hkq_gemm_a8w8_workspace(mm, nn, kk)
                wsp = torch.empty(max(nws, 16), dtype=torch.uint8, device="cuda")
                launch = hkq.bind("hkq_gemm_a8w8_ws", xa.data_ptr(), wb.data_ptr(), xsa.data_ptr(), wsb.data_ptr(),
                                  Cs.data_ptr(), mm, nn, kk, kk, kk, nn, wsp.data_ptr(), nws,
                                  torch.cuda.current_stream().cuda_stream)
                ms_s = time_launches(launch, 20, 3, preheat=0.05)
                byts = mm * kk + nn * kk + 2 * mm * nn + 4 * (mm + nn)
                sweep.append({"M": mm, "N": nn, "K": kk, "us": round(ms_s * 1e3, 2),
                              "tflops": round(2.0 * mm * nn * kk / (ms_s * 1e-3) / 1e12, 1),
                              "GB/s": round(byts / (ms_s * 1e-3) / 1e9, 1)})
        m4, n4, k4 = 128, MXFP4["N"], MXFP4["K"]
        xa4, xw4 = seeded_bf16((m4, k4), 1.0, 11), seeded_bf16((n4, k4), 0.02, 12)
        Aq4, As4 = hkq.mx_quant(xa4, True)
        Bq4, Bs4 = hkq.mx_quant(xw4, True)
        C4s = torch.empty((m4, n4), dtype=torch.bfloat16, device="cuda")
        nws = hkq.lib().hkq_gemm_mxfp4_workspace(m4, n4, k4)
        wsp = torch.empty(max(nws, 16), dtype=torch.uint8, device="cuda")
        launch = hkq.bind("hkq_gemm_mxfp4_ws", Aq4.data_ptr(), As4.data_ptr(), Bq4.data_ptr(), Bs4.data_ptr(),
                          C4s.data_ptr(), m4, n4, k4, Aq4.stride(0), Bq4.stride(0), As4.stride(0), Bs4.stride(0), n4,
                          wsp.data_ptr(), nws, torch.cuda.current_stream().cuda_stream)
        ms_s = time_launches(launch, 20, 3, preheat=0.05)
        sweep.append({"kind": "mxfp4", "M": m4, "N": n4, "K": k4, "us": round(ms_s * 1e3, 2),
                      "tflops": round(2.0 * m4 * n4 * k4 / (ms_s * 1e-3) / 1e12, 1)})
        res["sweep"] = sum(r["us"] for r in sweep) * 1e-3

    if args.only is not None:
        log(json.dumps({k: round(v * 1e3, 2) for k, v in res.items()}) + "  (us per launch)")
        for r in routing_res:
            log(json.dumps({"routing": r}))
        for r in bs_res + moe_res + fused_res + ext_res:
            log(json.dumps(r))
        if sweep:
            for r in sweep:
                log(json.dumps(r))
        return

    ms = res["a8w8"]
    flops = 2.0 * M * N * K
    tflops = flops / (ms * 1e-3) / 1e12
    m4, n4, k4 = MXFP4["M"], MXFP4["N"], MXFP4["K"]
    tflops4 = 2.0 * m4 * n4 * k4 / (res["mxfp4"] * 1e-3) / 1e12
    qbytes = 4096 * 4096 * 3 + 4096 * 4
    quant_gbs = qbytes / (res["quant"] * 1e-3) / 1e9

    cpu = None
    if not args.no_cpu:
        log("cpu baseline (oracle/cpu_baseline.py, BASELINE config 0)")
        from oracle import cpu_baseline

        r = cpu_baseline.run()
        cpu = {"value": round(r["tflops"], 6), "unit": "TFLOP/s", "cores": r["threads"], "kind": "port",
               "sample": r["sample"], "quant_ms": round(r["quant_ms"], 3), "matmul_ms": round(r["matmul_ms"], 3),
               "total_ms": round(r["total_ms"], 3)}

    out = {
        "metric": "FP8 A8W8 GEMM TFLOPS & % MFMA peak (4096x14336x4096); MXFP4 TFLOPS",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3fn",
        "data": "synthetic (seeded CPU generator: acts ~N(0,1), weights ~N(0,0.02); per-token / per-channel "
                "E4M3FN quantization by this library)",
        "config": {"workload": "A8W8 GEMM, per-token x per-channel fp32 scales, bf16 out", "M": M, "N": N, "K": K,
                   "parallelism": "single GPU"},
        "pct_fp8_peak": round(100 * tflops / PEAK_FP8_TFLOPS, 2),
        "mxfp4": {"M": m4, "N": n4, "K": k4, "tflops": round(tflops4, 2), "ms": round(res["mxfp4"], 5),
                  "pct_fp4_peak": round(100 * tflops4 / PEAK_FP4_TFLOPS, 2)},
        "quant_per_token_fp8": {"M": 4096, "K": 4096, "GB/s": round(quant_gbs, 1), "ms": round(res["quant"], 5),
                                "pct_hbm_peak": round(100 * quant_gbs / PEAK_HBM_GBS, 2)},
        "blockscale": bs_res,
        "moe_mixtral": moe_res,
        "moe_routing": routing_res,
        "fused_quant": fused_res,
        "gemm_ext": ext_res,
        "sweep": sweep,
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_FP8_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_FP8_TFLOPS, 4), "traffic": read_traffic()},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
