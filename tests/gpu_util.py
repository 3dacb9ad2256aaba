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


def assert_gemm_close(C: np.ndarray, ref: np.ndarray, what: str = ""):
    C = np.asarray(C, np.float64)
    err = np.abs(C - ref)
    bound = GEMM_ATOL + GEMM_RTOL * np.abs(ref)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} / {bad.size} outside |d| <= {GEMM_ATOL} + {GEMM_RTOL}|ref|; "
                             f"worst at {i}: got {C[i]!r} ref {ref[i]!r}")
    rel = np.linalg.norm(C - ref) / max(np.linalg.norm(ref), 1e-30)
    assert rel < GEMM_RTOL, f"{what}: relative Frobenius error {rel}"
