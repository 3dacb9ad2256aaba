"""ctypes binding of libhkq.so (the C ABI declared in include/hkq.h).

This is the layer the parity tests and bench.py call: plain device pointers,
explicit sizes and an explicit stream. Torch is used only to allocate device
memory and to name the stream. If the library is missing, loading raises -- there
is no fallback path.
"""
from __future__ import annotations

import ctypes
import os

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG, "lib", "libhkq.so")

KIND_FP8 = 0
KIND_INT8 = 1

# Every entry point declared in include/hkq.h, with its ctypes signature.
_P, _I64, _I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
SIGNATURES = {
    "hkq_last_error": (ctypes.c_char_p, []),
    "hkq_version": (_I, []),
    "hkq_per_token_quant": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _I, _P]),
    "hkq_group_quant": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P]),
    "hkq_static_quant_fp8": (_I, [_P, _P, _P, _I64, _P]),
    "hkq_mx_quant": (_I, [_P, _P, _P, _I64, _I64, _I64, _I, _P]),
    "hkq_mx_dequant": (_I, [_P, _P, _P, _I64, _I64, _I, _P]),
    "hkq_gemm_a8w8": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P]),
    "hkq_gemm_mxfp4": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P]),
    "hkq_gemm_a8w8_workspace": (ctypes.c_size_t, [_I64, _I64, _I64]),
    "hkq_gemm_a8w8_ws": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, ctypes.c_size_t, _P]),
    "hkq_gemm_a8w8_noalloc_max_workspace": (ctypes.c_size_t, []),
    "hkq_gemm_a8w8_noalloc": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P]),
    "hkq_gemm_mxfp4_workspace": (ctypes.c_size_t, [_I64, _I64, _I64]),
    "hkq_gemm_mxfp4_ws": (_I, [_P, _P, _P, _P, _P] + [_I64] * 8 + [_P, ctypes.c_size_t, _P]),
    "hkq_gemm_blockscale": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P]),
    "hkq_gemm_blockscale_mul_add": (_I, [_P] * 7 + [_I64] * 11 + [_P]),
    "hkq_batched_gemm_a8w8": (_I, [_P] * 6 + [_I64] * 13 + [_P]),
    "hkq_gemm_bf16": (_I, [_P, _P, _P] + [_I64] * 6 + [_P]),
    "hkq_gemm_bf16_workspace": (ctypes.c_size_t, [_I64, _I64, _I64]),
    "hkq_batched_gemm_bf16": (_I, [_P] * 4 + [_I64] * 11 + [_P, ctypes.c_size_t, _P]),
    "hkq_moe_a8w8": (_I, [_P, _P, _P, _P, _I64, _P, _I64, _I64, _I64, _P, _I64, _P, _P, _P, _P]
                     + [_I64] * 12 + [_P]),
    "hkq_moe_a8w8_kn": (_I, [_P, _P, _P, _P, _I64, _P, _I64, _I64, _I64, _P, _I64, _P, _P, _P, _P]
                        + [_I64] * 12 + [_P]),
    "hkq_moe_a8w8_blockscale": (_I, [_P, _P, _P, _P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64,
                                     _P, _P, _P, _P] + [_I64] * 12 + [_P]),
    "hkq_moe_a8w8_blockscale_kn": (_I, [_P, _P, _P, _P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64,
                                     _P, _P, _P, _P] + [_I64] * 12 + [_P]),
    "hkq_moe_pack_kmajor": (_I, [_P, _P] + [_I64] * 7 + [_P]),
    "hkq_rmsnorm_quant": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, ctypes.c_float, _I, _P]),
    "hkq_swiglu_quant": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, ctypes.c_float, _I, _I, _P]),
    "hkq_moe_mxfp4": (_I, [_P] * 10 + [_I64, _I64, _I64, _I64, _I] + [_I64] * 10 + [_P]),
    "hkq_moe_mxfp4_kn": (_I, [_P] * 10 + [_I64, _I64, _I64, _I64, _I] + [_I64] * 10 + [_P]),
    "hkq_moe_topk": (_I, [_P, _I64, _P, _P, _I64, _P, _I64, _I64, _I64, _I64, _I, _I, _P]),
    "hkq_sum_bitmatrix_rows": (_I, [_P, _I64, _I64, _I64, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "hkq_sum_bitmatrix_rows_fused": (_I, [_P, _I64, _I64, _I64, _P, _I64, _P]),
    "hkq_expt_data_stage1": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I, _P]),
    "hkq_expt_data_stage2": (_I, [_P, _P, _P, _I64, _I, _P]),
    "hkq_expt_data_stage2_fused": (_I, [_P, _P, _P, _I64, _P]),
    "hkq_expt_data_compute": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _P]),
    "hkq_routing_compute_indx": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _P, _I64, _I, _P]),
    "hkq_routing_compute_indx_fused": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I, _P]),
    "hkq_moe_align_block_size": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
}


class HkqError(RuntimeError):
    """A C-ABI call returned a non-zero hipError_t."""


_lib = None


def lib() -> ctypes.CDLL:
    """Load libhkq.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HkqError(f"{LIB_PATH} is missing: build it with `python amd-kernels_amd/build.py`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().hkq_last_error().decode(errors="replace")
        raise HkqError(f"{name} failed with code {rc}: {msg}")


def bind(name: str, *args):
    """Zero-argument callable that repeats one C-ABI call with fixed arguments:
    the arguments are converted to ctypes once, so back-to-back launches of a
    short kernel are not limited by Python-side argument handling."""
    fn = getattr(lib(), name)
    cargs = [t(a) if a is not None else None for t, a in zip(SIGNATURES[name][1], args)]

    def run():
        rc = fn(*cargs)
        if rc != 0:
            msg = lib().hkq_last_error().decode(errors="replace")
            raise HkqError(f"{name} failed with code {rc}: {msg}")

    return run


# ----------------------------------------------------------------------------
# torch-tensor conveniences over the C ABI (device pointers + current stream)
# ----------------------------------------------------------------------------

def _ptr(t) -> int:
    return t.data_ptr()


def _opt_ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


def _stream(stream=None) -> int:
    import torch

    s = torch.cuda.current_stream() if stream is None else stream
    return s.cuda_stream


def per_token_quant(x, kind: int = KIND_FP8, q=None, s=None, stream=None):
    """x bf16 [M, K] -> (q [M, K] float8_e4m3fn / int8, s fp32 [M])."""
    import torch

    M, K = x.shape
    if q is None:
        q = torch.empty((M, K), dtype=torch.float8_e4m3fn if kind == KIND_FP8 else torch.int8, device=x.device)
    if s is None:
        s = torch.empty((M,), dtype=torch.float32, device=x.device)
    call("hkq_per_token_quant", _ptr(x), _ptr(q), _ptr(s), M, K, x.stride(0), q.stride(0), kind, _stream(stream))
    return q, s


def group_quant(x, group: int = 128, kind: int = KIND_FP8, q=None, s=None, stream=None):
    """x bf16 [M, K] -> (q [M, K], s fp32 [M, K/group])."""
    import torch

    M, K = x.shape
    if q is None:
        q = torch.empty((M, K), dtype=torch.float8_e4m3fn if kind == KIND_FP8 else torch.int8, device=x.device)
    if s is None:
        s = torch.empty((M, K // group), dtype=torch.float32, device=x.device)
    call("hkq_group_quant", _ptr(x), _ptr(q), _ptr(s), M, K, x.stride(0), q.stride(0), s.stride(0), group, kind,
         _stream(stream))
    return q, s


def static_quant_fp8(x, scale, y=None, stream=None):
    import torch

    if y is None:
        y = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    call("hkq_static_quant_fp8", _ptr(x), _ptr(y), _ptr(scale), x.numel(), _stream(stream))
    return y


def mx_quant(x, is_fp4: bool = True, stream=None):
    """x bf16 [M, K] -> (q uint8 [M, K/2 or K], s uint8 [M, K/32])."""
    import torch

    M, K = x.shape
    q = torch.empty((M, K // 2 if is_fp4 else K), dtype=torch.uint8, device=x.device)
    s = torch.empty((M, K // 32), dtype=torch.uint8, device=x.device)
    call("hkq_mx_quant", _ptr(x), _ptr(q), _ptr(s), M, K, x.stride(0), int(is_fp4), _stream(stream))
    return q, s


def mx_dequant(q, s, K: int, is_fp4: bool = True, stream=None):
    import torch

    M = q.shape[0]
    out = torch.empty((M, K), dtype=torch.bfloat16, device=q.device)
    call("hkq_mx_dequant", _ptr(q), _ptr(s), _ptr(out), M, K, int(is_fp4), _stream(stream))
    return out


def rmsnorm_quant(x, w, eps: float = 1e-6, kind: int = 0, q=None, s=None, stream=None):
    """RMSNorm + quantization of bf16 [M, D] with weight bf16 [D]. kind 0: 1x128
    FP8 -> (q float8_e4m3fn [M, D], s fp32 [M, D/128]); kind 1: MXFP4 ->
    (q uint8 [M, D/2], s uint8 e8m0 [M, D/32]), elements rounded to nearest
    even; kind 2: MXFP4 with elements floored by the threshold ladder of
    kernels/quantization/fused_mxfp4_quant/kernel.cpp:128-150."""
    import torch

    M, D = x.shape
    if q is None:
        q = (torch.empty((M, D), dtype=torch.float8_e4m3fn, device=x.device) if kind == 0
             else torch.empty((M, D // 2), dtype=torch.uint8, device=x.device))
    if s is None:
        s = (torch.empty((M, D // 128), dtype=torch.float32, device=x.device) if kind == 0
             else torch.empty((M, D // 32), dtype=torch.uint8, device=x.device))
    call("hkq_rmsnorm_quant", _ptr(x), _ptr(w), _ptr(q), _ptr(s), M, D, x.stride(0), q.stride(0), s.stride(0),
         eps, kind, _stream(stream))
    return q, s


def swiglu_quant(y, alpha: float = 1.0, interleaved: bool = False, group: int = 0, q=None, s=None, stream=None):
    """SiLU-and-mul of a gate/up output bf16 [M, 2F] + FP8 quantization:
    (q float8_e4m3fn [M, F], s fp32 [M] (group 0) or [M, F/128] (group 128))."""
    import torch

    M, F2 = y.shape
    F = F2 // 2
    if q is None:
        q = torch.empty((M, F), dtype=torch.float8_e4m3fn, device=y.device)
    if s is None:
        s = torch.empty((M,) if group == 0 else (M, F // 128), dtype=torch.float32, device=y.device)
    call("hkq_swiglu_quant", _ptr(y), _ptr(q), _ptr(s), M, F, y.stride(0), q.stride(0),
         s.stride(0) if group else 0, alpha, int(interleaved), group, _stream(stream))
    return q, s


def _workspace(nbytes: int, like):
    import torch

    return torch.empty(nbytes, dtype=torch.uint8, device=like.device) if nbytes else None


def gemm_a8w8(A, B, sa, sb, C=None, stream=None, split: bool = True):
    """A [M, K], B [N, K] E4M3FN codes; sa [M], sb [N] fp32 -> C bf16 [M, N].
    split=False runs the plain entry point (no workspace, no split-K)."""
    import torch

    M, K = A.shape
    N = B.shape[0]
    if C is None:
        C = torch.empty((M, N), dtype=torch.bfloat16, device=A.device)
    if not split:
        call("hkq_gemm_a8w8", _ptr(A), _ptr(B), _ptr(sa), _ptr(sb), _ptr(C), M, N, K, A.stride(0), B.stride(0),
             C.stride(0), _stream(stream))
        return C
    ws = _workspace(lib().hkq_gemm_a8w8_workspace(M, N, K), A)
    call("hkq_gemm_a8w8_ws", _ptr(A), _ptr(B), _ptr(sa), _ptr(sb), _ptr(C), M, N, K, A.stride(0), B.stride(0),
         C.stride(0), _ptr(ws) if ws is not None else None, ws.numel() if ws is not None else 0, _stream(stream))
    return C


def gemm_mxfp4(A, As, B, Bs, C=None, stream=None, split: bool = True):
    """A u8 [M, K/2], As u8 [M, K/32], B u8 [N, K/2], Bs u8 [N, K/32] -> C bf16 [M, N].
    split=False runs the plain entry point (no workspace, no split-K)."""
    import torch

    M, K = A.shape[0], A.shape[1] * 2
    N = B.shape[0]
    if C is None:
        C = torch.empty((M, N), dtype=torch.bfloat16, device=A.device)
    if not split:
        call("hkq_gemm_mxfp4", _ptr(A), _ptr(As), _ptr(B), _ptr(Bs), _ptr(C), M, N, K, A.stride(0), B.stride(0),
             As.stride(0), Bs.stride(0), C.stride(0), _stream(stream))
        return C
    ws = _workspace(lib().hkq_gemm_mxfp4_workspace(M, N, K), A)
    call("hkq_gemm_mxfp4_ws", _ptr(A), _ptr(As), _ptr(B), _ptr(Bs), _ptr(C), M, N, K, A.stride(0), B.stride(0),
         As.stride(0), Bs.stride(0), C.stride(0), _ptr(ws) if ws is not None else None,
         ws.numel() if ws is not None else 0, _stream(stream))
    return C


def gemm_blockscale(A, B, sa, sb, C=None, group_n: int = 128, stream=None):
    """A [M, K], B [N, K] E4M3FN codes; sa fp32 [M, K/128]; sb fp32 [K/128, N/group_n]
    -> C bf16 [M, N]."""
    import torch

    M, K = A.shape
    N = B.shape[0]
    if C is None:
        C = torch.empty((M, N), dtype=torch.bfloat16, device=A.device)
    call("hkq_gemm_blockscale", _ptr(A), _ptr(B), _ptr(sa), _ptr(sb), _ptr(C), M, N, K, A.stride(0), B.stride(0),
         sa.stride(0), sb.stride(0), C.stride(0), group_n, _stream(stream))
    return C


def gemm_blockscale_mul_add(A, B, sa, sb, c_a, c_b, C=None, group_n: int = 128, stream=None):
    """C = bf16(c_a * G + c_b), G the fp32 block-scale GEMM of gemm_blockscale;
    c_a, c_b bf16 [M, N]."""
    import torch

    M, K = A.shape
    N = B.shape[0]
    if C is None:
        C = torch.empty(M, N, dtype=torch.bfloat16, device=A.device)
    call("hkq_gemm_blockscale_mul_add", _ptr(A), _ptr(B), _ptr(sa), _ptr(sb), _ptr(C), _ptr(c_a), _ptr(c_b), M, N, K,
         A.stride(0), B.stride(0), sa.stride(0), sb.stride(0), C.stride(0), c_a.stride(0), c_b.stride(0), group_n,
         _stream(stream))
    return C


def batched_gemm_a8w8(A, B, sa, sb, bias=None, C=None, stream=None):
    """A [Z, M, K], B [Z, N, K] E4M3FN codes; sa fp32 [Z, M], sb fp32 [Z, N];
    bias bf16 [Z, N] or None -> C bf16 [Z, M, N]."""
    import torch

    Z, M, K = A.shape
    N = B.shape[1]
    if C is None:
        C = torch.empty(Z, M, N, dtype=torch.bfloat16, device=A.device)
    call("hkq_batched_gemm_a8w8", _ptr(A), _ptr(B), _ptr(sa), _ptr(sb), _opt_ptr(bias), _ptr(C), Z, M, N, K,
         A.stride(1), B.stride(1), C.stride(1), A.stride(0), B.stride(0), C.stride(0), sa.stride(0), sb.stride(0),
         bias.stride(0) if bias is not None else 0, _stream(stream))
    return C


def gemm_bf16(A, B, C=None, bias=None, stream=None, split: bool = True):
    """A [M, K] or [Z, M, K], B [N, K] or [Z, N, K] bf16; bias bf16 [N] / [Z, N]
    or None -> C bf16 [M, N] / [Z, M, N]. split=False (or a batch or bias) runs
    without a workspace, so without split-K."""
    import torch

    batched = A.dim() == 3
    A3 = A if batched else A.unsqueeze(0)
    B3 = B if batched else B.unsqueeze(0)
    Z, M, K = A3.shape
    N = B3.shape[1]
    if C is None:
        C = torch.empty(Z, M, N, dtype=torch.bfloat16, device=A.device)
        if not batched:
            C = C[0]
    C3 = C if batched else C.unsqueeze(0)
    b2 = None if bias is None else (bias if bias.dim() == 2 else bias.unsqueeze(0))
    ws = None
    if split and Z == 1 and bias is None:
        n = int(lib().hkq_gemm_bf16_workspace(M, N, K))
        ws = torch.empty(n, dtype=torch.uint8, device=A.device) if n else None
    call("hkq_batched_gemm_bf16", _ptr(A3), _ptr(B3), _opt_ptr(b2), _ptr(C3), Z, M, N, K, A3.stride(1),
         B3.stride(1), C3.stride(1), A3.stride(0), B3.stride(0), C3.stride(0), b2.stride(0) if b2 is not None else 0,
         _ptr(ws) if ws is not None else None, ws.numel() if ws is not None else 0, _stream(stream))
    return C


def moe_a8w8(X, W, hist, offs, expt_data, topk, gather=None, x_scale=None, w_scale=None, bias=None, Y=None,
             y_rows=None, stream=None, w_kn=False):
    """OGS-routed A8W8 MoE GEMM. X [T, K] E4M3FN; W [E, N, K] E4M3FN (K contiguous),
    or with w_kn the reference's [E, K, N] (N contiguous, read in place);
    x_scale: None, [1] (per tensor) or [T] (per token); w_scale: None, [E] (per
    expert) or [E, N] (per channel); bias: None or fp32 [E, N]; int32 routing
    tensors as in the reference (gather [T*topk], hist [E], offs [E],
    expt_data [grid_m]). Returns Y bf16 [y_rows (default T*topk), N]."""
    import torch

    T, K = X.shape
    E, N = (W.shape[0], W.shape[2]) if w_kn else (W.shape[0], W.shape[1])
    rows = T * topk if y_rows is None else y_rows
    if Y is None:
        Y = torch.zeros((rows, N), dtype=torch.bfloat16, device=X.device)
    xs_tok = 0 if (x_scale is None or x_scale.numel() == 1) else 1
    if w_scale is None or w_scale.numel() == E:
        ws_e, ws_n = 1, 0
    else:
        ws_e, ws_n = N, 1
    null = 0
    call("hkq_moe_a8w8_kn" if w_kn else "hkq_moe_a8w8", _ptr(X), _ptr(W), _ptr(Y),
         _ptr(x_scale) if x_scale is not None else null, xs_tok,
         _ptr(w_scale) if w_scale is not None else null, ws_e, ws_n, 1,
         _ptr(bias) if bias is not None else null, N, _ptr(gather) if gather is not None else null,
         _ptr(hist), _ptr(offs), _ptr(expt_data), T, E, N, K, expt_data.numel(), topk, X.stride(0), W.stride(0),
         W.stride(1), Y.stride(0), rows, gather.numel() if gather is not None else 0, _stream(stream))
    return Y


def moe_a8w8_blockscale(X, W, hist, offs, expt_data, topk, x_scale, w_scale, group_k: int, group_n: int,
                        gather=None, bias=None, Y=None, y_rows=None, stream=None, w_kn=False):
    """OGS-routed A8W8 MoE GEMM with per-K-group scales. X [T, K] E4M3FN;
    W [E, N, K] E4M3FN (K contiguous), or with w_kn the reference's [E, K, N]
    (N contiguous, read in place); x_scale fp32 [T, ceil(K/group_k)];
    w_scale fp32 [E, ceil(K/group_k), ceil(N/group_n)] (any strides); bias None
    or fp32 [E, N]. Returns Y bf16 [y_rows (default T*topk), N]."""
    import torch

    T, K = X.shape
    E, N = (W.shape[0], W.shape[2]) if w_kn else (W.shape[0], W.shape[1])
    rows = T * topk if y_rows is None else y_rows
    if Y is None:
        Y = torch.zeros((rows, N), dtype=torch.bfloat16, device=X.device)
    call("hkq_moe_a8w8_blockscale_kn" if w_kn else "hkq_moe_a8w8_blockscale", _ptr(X), _ptr(W), _ptr(Y),
         _ptr(x_scale), x_scale.stride(0), x_scale.stride(1),
         _ptr(w_scale), w_scale.stride(0), w_scale.stride(1), w_scale.stride(2), group_k, group_n, _opt_ptr(bias), N,
         _opt_ptr(gather), _ptr(hist), _ptr(offs), _ptr(expt_data), T, E, N, K, expt_data.numel(), topk,
         X.stride(0), W.stride(0), W.stride(1), Y.stride(0), rows, gather.numel() if gather is not None else 0,
         _stream(stream))
    return Y


def moe_pack_kmajor(W, out=None, stream=None):
    """[E, R, N] byte planes (N contiguous, e.g. the reference's [E, K, N] MoE
    weights) -> contiguous [E, N, R] (uint8 view of the same codes)."""
    import torch

    E, R, N = W.shape
    assert W.stride(2) == 1, "the source's last dimension must be contiguous"
    if out is None:
        out = torch.empty((E, N, R), dtype=torch.uint8, device=W.device)
    call("hkq_moe_pack_kmajor", _ptr(W), _ptr(out), E, R, N, W.stride(0), W.stride(1), out.stride(0), out.stride(1),
         _stream(stream))
    return out


def moe_mxfp4(A, As, B, Bs, sorted_ids, expert_ids, num_valid: int, topk: int, a_scale=None, b_scale=None,
              topk_weights=None, C=None, c_rows=None, stream=None, b_kn=False):
    """MXFP4 MoE over block-sorted routing (align_block_size output, 128-row
    blocks). A uint8 [T, K/2], As uint8 [T, K/32], B uint8 [E, N, K/2], Bs uint8
    [E, N, K/32] (K contiguous), or with b_kn the reference's B [E, K/2, N] and
    Bs [E, K/32, N] (N contiguous, read in place); topk_weights (fp32, indexed by
    gate id) turns on the routed-weight multiply. Returns C bf16
    [c_rows (default num_valid), N] with row = gate id."""
    import torch

    T, Kh = A.shape
    E, N = (B.shape[0], B.shape[2]) if b_kn else (B.shape[0], B.shape[1])
    K = 2 * Kh
    rows = num_valid if c_rows is None else c_rows
    if C is None:
        C = torch.zeros((rows, N), dtype=torch.bfloat16, device=A.device)
    grid_m = sorted_ids.numel() // 128
    call("hkq_moe_mxfp4_kn" if b_kn else "hkq_moe_mxfp4", _ptr(A), _ptr(B), _ptr(C), _ptr(As), _ptr(Bs),
         _opt_ptr(a_scale), _opt_ptr(b_scale),
         _opt_ptr(topk_weights), _ptr(sorted_ids), _ptr(expert_ids), N, K, num_valid, topk,
         int(topk_weights is not None), A.stride(0), B.stride(0), B.stride(1), C.stride(0), As.stride(0),
         Bs.stride(0), Bs.stride(1), T, E, grid_m, _stream(stream))
    return C


# ----------------------------------------------------------------------------
# MoE routing metadata (GPU producers of the tensors moe_a8w8 consumes)
# ----------------------------------------------------------------------------

def moe_topk(logits, K: int, softmax: bool = True, bitmatrix: bool = True, stream=None):
    """Top-K experts per row of bf16 logits [T, E]: (values bf16 [T, K],
    experts int32 [T, K], bitmatrix int32 [T, ceil(E/32)] or None)."""
    import torch

    T, E = logits.shape
    Yv = torch.empty((T, K), dtype=torch.bfloat16, device=logits.device)
    Yi = torch.empty((T, K), dtype=torch.int32, device=logits.device)
    nw = (E + 31) // 32
    bits = torch.empty((T, nw), dtype=torch.int32, device=logits.device) if bitmatrix else None
    call("hkq_moe_topk", _ptr(logits), logits.stride(0), _ptr(Yv), _ptr(Yi), K, _opt_ptr(bits), nw, 1, T, E, K,
         int(softmax), _stream(stream))
    return Yv, Yi, bits


def sum_bitmatrix_rows(bits, partials: bool = True, stream=None):
    """Column sums of a row-major bitmatrix int32 [T, nw]: (hist int32 [32*nw],
    partials int32 [ceil(T/128), 32*nw] (exclusive over 128-row tiles) or None)."""
    import torch

    T, nw = bits.shape
    ret = torch.empty(32 * nw, dtype=torch.int32, device=bits.device)
    if not partials:
        call("hkq_sum_bitmatrix_rows_fused", _ptr(bits), T, bits.stride(0), 1, _ptr(ret), nw, _stream(stream))
        return ret, None
    part = torch.empty(((T + 127) // 128, 32 * nw), dtype=torch.int32, device=bits.device)
    call("hkq_sum_bitmatrix_rows", _ptr(bits), T, bits.stride(0), 1, _ptr(ret), _ptr(part), part.stride(0), 1,
         32 * nw, nw, _stream(stream))
    return ret, part


def expt_data(hist, n_gates: int, tile_log2: int = 7, max_tiles: int | None = None, stream=None):
    """OGS expert data: (token_start int32 [E+1], tile_start int32 [E+1], tile
    metadata int32 [max_tiles], -1 past the last tile). The default max_tiles,
    n_gates // 2^tile_log2 + E, bounds the tile count for any histogram."""
    import torch

    E = hist.numel()
    if max_tiles is None:
        max_tiles = n_gates // (1 << tile_log2) + E
    ts = torch.empty(E + 1, dtype=torch.int32, device=hist.device)
    tl = torch.empty(E + 1, dtype=torch.int32, device=hist.device)
    md = torch.empty(max(max_tiles, 1), dtype=torch.int32, device=hist.device)
    call("hkq_expt_data_compute", _ptr(hist), _ptr(ts), _ptr(tl), _ptr(md), E, max_tiles, n_gates, tile_log2, 0,
         _stream(stream))
    return ts, tl, md[:max_tiles]


def compute_indx(expt_indx, tokens_start, partial_offs=None, expt_scal=None, n_slots: int | None = None,
                 stream=None):
    """Gate placement for expert ids [T, K]: (gather int32 [n_slots], scatter
    int32 [T*K], gate_scal bf16 [n_slots] or None); partial_offs int32
    [ceil(T/128), E] from sum_bitmatrix_rows, or None (counted in one workgroup)."""
    import torch

    T, K = expt_indx.shape
    n = T * K
    n_slots = n if n_slots is None else n_slots
    dev = expt_indx.device
    gather = torch.empty(max(n_slots, 1), dtype=torch.int32, device=dev)
    scatter = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    gs = torch.empty(max(n_slots, 1), dtype=torch.bfloat16, device=dev) if expt_scal is not None else None
    if partial_offs is None:
        call("hkq_routing_compute_indx_fused", _ptr(gather), _ptr(scatter), _opt_ptr(gs), _opt_ptr(expt_scal),
             _ptr(expt_indx), _ptr(tokens_start), n, K, _stream(stream))
    else:
        call("hkq_routing_compute_indx", _ptr(gather), _ptr(scatter), _opt_ptr(gs), _opt_ptr(expt_scal),
             _ptr(expt_indx), _ptr(partial_offs), partial_offs.stride(0), partial_offs.stride(1),
             _ptr(tokens_start), n, K, _stream(stream))
    return gather[:n_slots], scatter[:n], (None if gs is None else gs[:n_slots])


def moe_routing_plan(logits, topk: int, block_m: int = 128, softmax: bool = True, stream=None):
    """Allocate the routing outputs for router logits bf16 [T, E] and bind the
    five launches that fill them (top-k + bitmatrix, tile counts and their
    scan, expert data, gate placement). Returns (outputs, run): run() enqueues
    the launches on the stream, with no host synchronisation and no
    allocation. outputs: topk_vals, topk_idx, bits, hist, partials, offs,
    token_start, tile_start, expt_data (tiles of block_m rows, -1 past the
    last), gather, scatter, gate_scal."""
    import torch

    T, E = logits.shape
    K = topk
    log2 = block_m.bit_length() - 1
    if (1 << log2) != block_m:
        raise ValueError("block_m must be a power of two")
    dev = logits.device
    nw = (E + 31) // 32
    ntiles = (T + 127) // 128
    max_tiles = T * K // block_m + E
    o = {
        "topk_vals": torch.empty((T, K), dtype=torch.bfloat16, device=dev),
        "topk_idx": torch.empty((T, K), dtype=torch.int32, device=dev),
        "bits": torch.empty((T, nw), dtype=torch.int32, device=dev),
        "hist_all": torch.empty(32 * nw, dtype=torch.int32, device=dev),
        "partials": torch.empty((ntiles, 32 * nw), dtype=torch.int32, device=dev),
        "token_start": torch.empty(E + 1, dtype=torch.int32, device=dev),
        "tile_start": torch.empty(E + 1, dtype=torch.int32, device=dev),
        "expt_data": torch.empty(max(max_tiles, 1), dtype=torch.int32, device=dev),
        "gather": torch.empty(max(T * K, 1), dtype=torch.int32, device=dev),
        "scatter": torch.empty(max(T * K, 1), dtype=torch.int32, device=dev),
        "gate_scal": torch.empty(max(T * K, 1), dtype=torch.bfloat16, device=dev),
    }
    st = _stream(stream)
    P = {k: v.data_ptr() for k, v in o.items()}
    calls = [
        bind("hkq_moe_topk", logits.data_ptr(), logits.stride(0), P["topk_vals"], P["topk_idx"], K, P["bits"], nw, 1,
             T, E, K, int(softmax), st),
        bind("hkq_sum_bitmatrix_rows", P["bits"], T, nw, 1, P["hist_all"], P["partials"], 32 * nw, 1, 32 * nw, nw, st),
        bind("hkq_expt_data_compute", P["hist_all"], P["token_start"], P["tile_start"], P["expt_data"], E, max_tiles,
             T * K, log2, 0, st),
        bind("hkq_routing_compute_indx", P["gather"], P["scatter"], P["gate_scal"], P["topk_vals"], P["topk_idx"],
             P["partials"], 32 * nw, 1, P["token_start"], T * K, K, st),
    ]

    def run():
        for c in calls:
            c()

    o["hist"] = o["hist_all"][:E]
    o["offs"] = o["token_start"][:E]
    o["expt_data"] = o["expt_data"][:max_tiles]
    return o, run


def moe_routing(logits, topk: int, block_m: int = 128, softmax: bool = True, stream=None):
    """Router logits bf16 [T, E] -> the OGS metadata of moe_a8w8, on the GPU and
    without a host synchronisation (see moe_routing_plan for the outputs)."""
    o, run = moe_routing_plan(logits, topk, block_m, softmax, stream)
    run()
    return o


def align_block_size(topk_ids, num_experts: int, block_size: int, stream=None):
    """moe_align_block_size over flattened expert ids: (sorted_token_ids int32
    [numel + E*(block_size-1)], expert_ids int32 [len(sorted) // block_size],
    cumsum int32 [E+1], total int32 [1]); only the first total entries of
    sorted_token_ids (and total // block_size of expert_ids) are written."""
    import torch

    numel = topk_ids.numel()
    dev = topk_ids.device
    cap = numel + num_experts * (block_size - 1)
    sorted_ids = torch.empty(max(cap, 1), dtype=torch.int32, device=dev)
    eids = torch.empty(max(cap // block_size, 1), dtype=torch.int32, device=dev)
    cnts = torch.empty((num_experts + 1) * num_experts, dtype=torch.int32, device=dev)
    cum = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    total = torch.empty(1, dtype=torch.int32, device=dev)
    call("hkq_moe_align_block_size", _ptr(topk_ids), _ptr(sorted_ids), _ptr(eids), _ptr(cnts), _ptr(cum),
         _ptr(total), num_experts, block_size, numel, _stream(stream))
    return sorted_ids, eids, cum, total

