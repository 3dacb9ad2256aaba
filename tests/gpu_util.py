"""Helpers shared by the GPU parity tests (bf16 bit patterns <-> device tensors,
seeded inputs, the north-star GEMM tolerance)."""
import numpy as np
import torch

# GEMM tolerance of the north star: bf16 output within 1e-2 relative / 2e-2
# absolute of the fp32-dequant matmul, elementwise |C - ref| <= ATOL + RTOL*|ref|.
GEMM_RTOL = 1e-2
GEMM_ATOL = 2e-2


def require_gpu():
    assert torch.cuda.is_available(), "GPU tests need an MI355X; run with -m 'not gpu' on CPU"


def dev_bf16(bits: np.ndarray) -> torch.Tensor:
    """uint16 bf16 bit patterns -> cuda bfloat16 tensor (same bytes)."""
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).cuda()


def dev_u8(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).cuda()


def dev_f32(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def host_u8(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.uint8).cpu().numpy()


def host_bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def host_bf16_f32(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


def assert_gemm_close(C: np.ndarray, ref: np.ndarray, what: str = "", rows_per_chunk: int = 512):
    """Elementwise |C - ref| <= ATOL + RTOL |ref| and Frobenius relative error
    < RTOL, checked in row chunks so that full outputs at BASELINE sizes
    (10^8 elements) need no fp64 copies of the whole matrix."""
    C = np.asarray(C)
    ref = np.asarray(ref)
    assert C.shape == ref.shape, f"{what}: shape {C.shape} vs {ref.shape}"
    if C.ndim != 2:
        C, ref = C.reshape(-1, C.shape[-1]), ref.reshape(-1, ref.shape[-1])
    n_bad, worst, worst_at = 0, -np.inf, None
    d2 = r2 = 0.0
    for r0 in range(0, C.shape[0], rows_per_chunk):
        c = np.asarray(C[r0:r0 + rows_per_chunk], np.float64)
        f = np.asarray(ref[r0:r0 + rows_per_chunk], np.float64)
        err = np.abs(c - f)
        excess = err - (GEMM_ATOL + GEMM_RTOL * np.abs(f))
        excess[np.isnan(excess)] = np.inf  # NaN on either side fails
        n_bad += int((excess > 0).sum())
        i = np.unravel_index(np.argmax(excess), excess.shape)
        if excess[i] > worst:
            worst, worst_at = excess[i], (r0 + i[0], i[1], c[i], f[i])
        d2 += float(np.sum((c - f) ** 2))
        r2 += float(np.sum(f ** 2))
    if n_bad:
        r, col, got, want = worst_at
        raise AssertionError(f"{what}: {n_bad} / {C.size} outside |d| <= {GEMM_ATOL} + {GEMM_RTOL}|ref|; "
                             f"worst at ({r}, {col}): got {got!r} ref {want!r}")
    rel = np.sqrt(d2) / max(np.sqrt(r2), 1e-30)
    assert rel < GEMM_RTOL, f"{what}: relative Frobenius error {rel}"
