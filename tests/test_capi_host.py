"""Host-side checks of the C ABI and the hipkittens loader (no GPU needed).

* libhkq.so loads and exports every function include/hkq.h declares, and the
  ctypes signature table covers exactly that set;
* argument validation happens before any HIP call and reports through
  hkq_last_error() (so it is exercised here without a device);
* the hipkittens package discovers the reference-named modules, loads them,
  and raises the reference's exception types.
"""
import ctypes
import os
import re

import pytest

import hkq

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hkq.h")


def declared_functions():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(hkq_[a-z0-9_]+)\s*\(", txt)))


def test_header_matches_binding_table():
    assert declared_functions() == sorted(hkq.SIGNATURES)


def test_library_exports_every_declared_symbol():
    L = hkq.lib()
    for name in declared_functions():
        assert hasattr(L, name), name
        assert ctypes.cast(getattr(L, name), ctypes.c_void_p).value


def test_version():
    assert hkq.lib().hkq_version() >= 1


def _expect_invalid(name, *args, match):
    with pytest.raises(hkq.HkqError, match=match) as ei:
        hkq.call(name, *args)
    assert "code 1" in str(ei.value)


def test_argument_errors_are_reported_before_launch():
    p = 0x1000  # never dereferenced: validation fails first
    _expect_invalid("hkq_per_token_quant", p, p, p, 4, 12, 12, 12, 0, None, match="multiple of 8")
    _expect_invalid("hkq_per_token_quant", p, p, p, 4, 16, 16, 16, 7, None, match="kind")
    _expect_invalid("hkq_per_token_quant", p, p, p, 4, 65536, 65536, 65536, 0, None, match="32768")
    _expect_invalid("hkq_group_quant", p, p, p, 4, 256, 256, 256, 2, 96, 0, None, match="group")
    _expect_invalid("hkq_group_quant", p, p, p, 4, 200, 200, 200, 2, 128, 0, None, match="multiple of group")
    _expect_invalid("hkq_mx_quant", p, p, p, 4, 48, 48, 1, None, match="multiple of 32")
    _expect_invalid("hkq_gemm_a8w8", p, p, p, p, p, 16, 16, 96, 96, 96, 16, None, match="multiple of 64")
    _expect_invalid("hkq_gemm_a8w8", p, p, p, p, p, 16, 18, 64, 64, 64, 24, None, match="N must be a multiple of 4")
    _expect_invalid("hkq_gemm_a8w8", p, p, p, p, p, 16, 20, 64, 64, 64, 18, None, match="ldc")
    _expect_invalid("hkq_gemm_a8w8", p + 4, p, p, p, p, 16, 16, 64, 64, 64, 16, None, match="aligned")
    _expect_invalid("hkq_gemm_a8w8", p, p, p, p, p + 4, 16, 16, 64, 64, 64, 16, None, match="aligned")
    _expect_invalid("hkq_gemm_mxfp4", p, p, p, p, p, 16, 16, 192, 96, 96, 8, 8, 16, None, match="multiple of 128")
    assert "multiple of 128" in hkq.lib().hkq_last_error().decode()


def test_gemm_workspace_queries():
    """Host-side GEMM plans (no GPU needed): the narrow path (M <= 16, and
    M <= 32 on narrow short shapes) and full grids need no workspace; split-K
    plans of the tiled path do (sizes for 256 CUs when no GPU is visible)."""
    L = hkq.lib()
    assert L.hkq_gemm_a8w8_workspace(1, 4096, 4096) == 0
    assert L.hkq_gemm_a8w8_workspace(16, 4096, 14336) == 0
    assert L.hkq_gemm_a8w8_workspace(32, 4096, 4096) == 0
    assert L.hkq_gemm_a8w8_workspace(4096, 14336, 4096) == 0
    assert L.hkq_gemm_a8w8_workspace(32, 28672, 4096) > 0   # wide N: tiled skinny path, split K
    assert L.hkq_gemm_a8w8_workspace(64, 4096, 14336) > 0
    assert L.hkq_gemm_mxfp4_workspace(16, 8192, 8192) == 0
    assert L.hkq_gemm_mxfp4_workspace(64, 8192, 8192) > 0


def test_hipkittens_discovery_and_errors():
    import hipkittens as hk

    for name in ("quant_tk", "quant_moe_tk", "gemm_a8w8_tk", "gemm_a8w8_per_token_scale_tk", "gemm_afp4wfp4_tk"):
        assert name in hk.modules, name
    assert hasattr(hk.modules["quant_tk"], "per_token_quant_fwd")
    assert hasattr(hk.gemm.a8w8, "dispatch") and hasattr(hk.gemm.afp4wfp4, "dispatch")
    assert hasattr(hk.moe_routing.quant, "downcast_to_mxfp")
    with pytest.raises(RuntimeError, match="not found"):
        hk.modules["no_such_module_tk"]
    assert hk.modules.get("no_such_module_tk") is None


def test_hipkittens_rejects_host_tensors_and_bf16_codes():
    import torch

    import hipkittens as hk

    a = torch.zeros(4, 64, dtype=torch.bfloat16)
    c = torch.zeros(4, 4, dtype=torch.bfloat16)
    s = torch.zeros(4)
    with pytest.raises(ValueError, match="GPU tensor"):
        hk.gemm.a8w8.dispatch(a, a, s, s, c)
    with pytest.raises(ValueError, match="GPU tensor"):
        hk.per_token_quant_fwd(a, a, s)


def test_moe_a8w8_rejects_x_past_2gib():
    """The MoE kernels address gathered X rows with 32-bit buffer offsets, so
    an X spanning 2^31 bytes or more is rejected before any launch instead of
    reading zeros or other tokens' rows."""
    p = 0x1000  # never dereferenced: validation fails first
    K = 4096
    T = (1 << 31) // K  # T * K == 2^31
    args = [p, p, p, None, 0, None, 0, 0, 1, None, 0, None, p, p, p,
            T, 8, 4096, K, 16, 2, K, 4096 * K, K, 4096, T * 2, 0, None]
    _expect_invalid("hkq_moe_a8w8", *args, match="2\\^31")


def test_moe_a8w8_rejects_topk_past_65535():
    """The MoE kernels divide gather indices by top_k through a reciprocal
    multiply that is exact for top_k < 2^16; larger values are rejected before
    any launch."""
    p = 0x1000  # never dereferenced: validation fails first
    K = 256
    args = [p, p, p, None, 0, None, 0, 0, 1, None, 0, None, p, p, p,
            16, 8, 256, K, 16, 1 << 16, K, 256 * K, K, 256, 16, 0, None]
    _expect_invalid("hkq_moe_a8w8", *args, match="topk")
