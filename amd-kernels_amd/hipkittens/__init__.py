"""hipkittens -- drop-in Python surface of the quantized-GEMM path.

Mirrors the reference loader (hipkittens/__init__.py of m8than/amd-kernels) for
the modules this build provides:

    import hipkittens as hk
    hk.per_token_quant_fwd(x, out, scales)                 # quant_tk
    hk.gemm.a8w8.dispatch(A, B, a_scale, b_scale, C)       # gemm_a8w8_tk
    hk.gemm.a8w8_per_token.dispatch(A, B, C, a_s, b_s)     # gemm_a8w8_per_token_scale_tk
    hk.gemm.afp4wfp4.dispatch(A, B, C, A_scale, B_scale)   # gemm_afp4wfp4_tk
    hk.gemm.a16w16.dispatch(A, B, C)                       # gemm_a16w16_tk
    hk.batched_gemm.a8w8.dispatch(A, B, a_s, b_s, C, bias) # batched_gemm_a8w8_tk (also .bf16)
    hk.fused_gemm.a8w8_blockscale_mul_add.dispatch(a, b, c, a_s, b_s, c_a, c_b)
                                                           # (also .a8w8_blockscale_a16w16)
    hk.moe_routing.quant.downcast_to_mxfp(...)             # quant_moe_tk
    hk.moe_routing.topk.moe_topk(X, ...)                   # moe_topk_tk (also bitmatrix,
                                                           # expt_data, align_block_size)
    hk.modules["gemm_a8w8_tk"]                             # any module by name

Discovery contract (reference hipkittens/__init__.py:31-62): extension files
named ``<module><EXT_SUFFIX>`` under ``<pkg>/kernels``, else ``<pkg>/../kernels``,
else ``$HIPKITTENS_KERNELS_DIR``; debug prefixes are skipped; modules load
lazily on first use and a missing module raises RuntimeError. Every module is
a thin pybind11 layer over libhkq.so (include/hkq.h); nothing here computes.
"""
from __future__ import annotations

import importlib.util
import os
import sysconfig
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))


def _kernels_dir() -> str:
    for cand in (os.path.join(_HERE, "kernels"), os.path.join(_HERE, "..", "kernels")):
        if os.path.isdir(cand):
            return cand
    return os.environ.get("HIPKITTENS_KERNELS_DIR", os.path.join(_HERE, "kernels"))


_KERNELS_DIR = _kernels_dir()
_EXT_SUFFIX = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
_SKIP_PREFIXES = ("ds_read_test", "hk_", "mfma_", "gemm_debug", "test_")

_so_paths: dict[str, str] = {}
_loaded: dict[str, object] = {}
_lock = threading.Lock()


def _discover() -> None:
    if not os.path.isdir(_KERNELS_DIR):
        return
    for root, _dirs, files in os.walk(_KERNELS_DIR):
        for f in sorted(files):
            if not f.endswith(_EXT_SUFFIX):
                continue
            name = f[: -len(_EXT_SUFFIX)]
            if name.startswith(_SKIP_PREFIXES):
                continue
            _so_paths[name] = os.path.join(root, f)


_discover()


def _load(name: str):
    with _lock:
        mod = _loaded.get(name)
        if mod is not None:
            return mod
        path = _so_paths.get(name)
        if path is None:
            raise RuntimeError(f"Kernel module '{name}' not found. Did you compile it? "
                               f"(python amd-kernels_amd/build.py)")
        spec = importlib.util.spec_from_file_location(name, path)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _loaded[name] = mod
        return mod


class _Modules:
    """Dict-like, lazily loading view of the discovered modules."""

    def __getitem__(self, name):
        return _load(name)

    def __contains__(self, name):
        return name in _so_paths

    def __len__(self):
        return len(_so_paths)

    def keys(self):
        return _so_paths.keys()

    def items(self):
        for name in list(_so_paths):
            yield name, _load(name)

    def get(self, name, default=None):
        try:
            return _load(name)
        except RuntimeError:
            return default

    def __repr__(self):
        return f"<hipkittens.modules: {len(_so_paths)} available, {len(_loaded)} loaded>"


modules = _Modules()


def _call(mod_name: str, func_name: str, *args, **kwargs):
    fn = getattr(_load(mod_name), func_name, None)
    if fn is None:
        raise RuntimeError(f"Function '{func_name}' not found in '{mod_name}'")
    return fn(*args, **kwargs)


# ---- quantization (top-level functions, as in the reference) ----

def per_token_quant_fwd(*args, **kwargs):
    """per_token_quant_fwd(input bf16 [M,D], output int8|float8_e4m3fn [M,D], scales f32 [M,1])"""
    return _call("quant_tk", "per_token_quant_fwd", *args, **kwargs)


def fused_rmsnorm_fp8_quant_fwd(*args, **kwargs):
    """fused_rmsnorm_fp8_quant_fwd(input bf16 [M,D], weight bf16 [D], output e4m3 [M,D], scales f32 [M,D/128], eps)"""
    return _call("fused_fp8_quant_tk", "fused_rmsnorm_fp8_quant_fwd", *args, **kwargs)


def fused_rmsnorm_mxfp4_quant_fwd(*args, **kwargs):
    """fused_rmsnorm_mxfp4_quant_fwd(input bf16 [M,D], weight bf16 [D], output u8 [M,D/2], scales u8 [M,D/32], eps)"""
    return _call("fused_mxfp4_quant_tk", "fused_rmsnorm_mxfp4_quant_fwd", *args, **kwargs)


def swiglu_quant_fwd(*args, **kwargs):
    """swiglu_quant_fwd(input bf16 [M,2F], output e4m3 [M,F], scales f32 [M] or [M,F/128], alpha=1.0,
    interleaved=False, group_size=0) (extension)"""
    return _call("quant_tk", "swiglu_quant_fwd", *args, **kwargs)


def group_quant_fwd(*args, **kwargs):
    """group_quant_fwd(input bf16 [M,K], output [M,K], scales f32 [M,K/g], group_size=128) (extension)"""
    return _call("quant_tk", "group_quant_fwd", *args, **kwargs)


# ---- namespaces ----

class _SubModule:
    """Namespace entry bound to one extension module, loaded on first attribute access."""

    def __init__(self, mod_name: str):
        self._mod_name = mod_name

    def __getattr__(self, name):
        if name.startswith("_"):
            raise AttributeError(name)
        return getattr(_load(self._mod_name), name)

    def __repr__(self):
        return f"<hipkittens.{self._mod_name}>"


class _GemmNamespace:
    a16w16 = _SubModule("gemm_a16w16_tk")
    a8w8 = _SubModule("gemm_a8w8_tk")
    a8w8_per_token = _SubModule("gemm_a8w8_per_token_scale_tk")
    a8w8_blockscale = _SubModule("gemm_a8w8_blockscale_tk")
    afp4wfp4 = _SubModule("gemm_afp4wfp4_tk")


class _BatchedGemmNamespace:
    bf16 = _SubModule("batched_gemm_bf16_tk")
    a8w8 = _SubModule("batched_gemm_a8w8_tk")


class _FusedGemmNamespace:
    a8w8_blockscale_a16w16 = _SubModule("fused_gemm_a8w8_blockscale_a16w16_tk")
    a8w8_blockscale_mul_add = _SubModule("fused_gemm_a8w8_blockscale_mul_add_tk")


class _MoeGemmNamespace:
    a8w8 = _SubModule("moe_op_gemm_a8w8_tk")
    a8w8_blockscale = _SubModule("moe_op_gemm_a8w8_blockscale_tk")
    mxfp4 = _SubModule("moe_op_mxfp4_tk")


class _MoeRoutingNamespace:
    align_block_size = _SubModule("moe_align_block_size_tk")
    bitmatrix = _SubModule("moe_bitmatrix_tk")
    expt_data = _SubModule("moe_expt_data_tk")
    topk = _SubModule("moe_topk_tk")
    quant = _SubModule("quant_moe_tk")
    # extension: the gate placement the reference compiles without a binding
    routing = _SubModule("moe_routing_tk")


gemm = _GemmNamespace()
batched_gemm = _BatchedGemmNamespace()
fused_gemm = _FusedGemmNamespace()
moe = _MoeGemmNamespace()
moe_routing = _MoeRoutingNamespace()
