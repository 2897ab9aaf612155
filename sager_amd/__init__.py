"""sager_amd - MI355X (gfx950) implementation of SAGER's quantized MoE
decode hot path.

The product is the C-ABI library ``libsager_hip.so`` (declared in
``include/sager_hip.h``); :mod:`sager_amd.ops` mirrors the reference's
``sager::cuda`` launcher API (include/sager/kernels/cuda_ops.hpp) on torch
device tensors for Python callers and tests.  There is no CPU fallback:
loading fails loudly when the HIP library is missing.
"""
import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libsager_hip.so")
_lib = None

Q4K_BYTES = 144
Q8K_BYTES = 276
QK = 256

_VP = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/sager_hip.h
SIGNATURES = {
    "sg_last_error": (ctypes.c_char_p, []),
    "sg_version": (ctypes.c_char_p, []),
    "sg_quantize_q8_k": (_I, [_VP, _VP, _I, _I, _VP]),
    "sg_quantize_q8_k_f16": (_I, [_VP, _VP, _I, _I, _VP]),
    "sg_gemv_q4_k_q8": (_I, [_VP, _VP, _VP, _I, _I, _VP]),
    "sg_gemv_q4_k_q8_batched": (_I, [_VP, _VP, _VP, _I, _I, _I, _VP]),
    "sg_gemv_ptrs_q4_k_q8": (_I, [_VP, _VP, _VP, _I, _I, _I, _VP]),
    "sg_gemv_q6_k_q8": (_I, [_VP, _VP, _VP, _I, _I, _VP]),
    "sg_gemv_q4_k_q8_f16out": (_I, [_VP, _VP, _VP, _I, _I, _VP]),
    "sg_gemv2m_q4_k_q8_f16out": (_I, [_VP, _VP, _VP, _VP, _VP, _I, _I, _I, _VP]),
    "sg_gemv3m_q4_k_q8_f16out": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _I, _I, _I, _I, _VP]),
    "sg_gemv_q4_k_q8_f16out_resadd": (_I, [_VP, _VP, _VP, _VP, _I, _I, _VP]),
    "sg_q4k_subblock_dots": (_I, [_VP, _VP, _VP, _I, _I, _VP]),
    "sg_router_topk": (_I, [_VP, _VP, _VP, _I, _I, _I, _I, _F, _VP]),
    "sg_silu_mul": (_I, [_VP, _VP, _VP, _I, _VP]),
    "sg_moe_combine": (_I, [_VP, _VP, _VP, _VP, _I, _I, _I, _VP]),
    "sg_silu_mul_f16": (_I, [_VP, _VP, _VP, _I, _I, _VP]),
    "sg_moe_combine_batched_f16": (_I, [_VP, _VP, _VP, _I, _I, _I, _VP]),
    "sg_sigmoid_gate_scalar_f16": (_I, [_VP, _VP, _I, _VP]),
    "sg_sigmoid_gate_scalar_batched_f16": (_I, [_VP, _VP, _I, _I, _VP]),
    "sg_gemv_f32_out_f16x": (_I, [_VP, _VP, _VP, _I, _I, _I, _VP]),
    "sg_gemv_ptrs_q4_k_q8_f16out": (_I, [_VP, _VP, _VP, _I, _I, _I, _VP]),
    "sg_gemv_q4_k_q8_f16out_batched": (_I, [_VP, _VP, _VP, _I, _I, _I, _VP]),
    "sg_moe_layer_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I]),
    "sg_moe_layer": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
                          _VP, _SZ, _I, _I, _I, _I, _I, _F, _VP]),
    "sg_moe_layer_f16": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
                              _VP, _VP, _SZ, _I, _I, _I, _I, _I, _F, _VP]),
    "sg_moe_prefill_f16": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
                                _VP, _VP, _SZ, _I, _I, _I, _I, _I, _F, _VP]),
    "sg_moe_layer_noalloc": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
                                  _VP, _I, _I, _I, _I, _I, _F, _VP]),
    "sg_moe_layer_stages": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
                                 _VP, _VP, _SZ, _I, _I, _I, _I, _I, _F, _I, _VP]),
    "sg_moe_dispatch_scan": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _I, _I, _I, _I, _VP]),
    "sg_router_topk_fused": (_I, [_VP, _VP, _VP, _VP, _I, _I, _I, _VP]),
    "sg_gather_rows_q8": (_I, [_VP, _VP, _VP, _I, _I, _VP]),
    "sg_gather_rows_q8_n": (_I, [_VP, _VP, _VP, _VP, _I, _I, _VP]),
    "sg_gather_rows_f16_n": (_I, [_VP, _VP, _VP, _VP, _I, _I, _VP]),
    "sg_silu_mul_f16_n": (_I, [_VP, _VP, _VP, _VP, _I, _I, _VP]),
    "sg_quantize_q8_k_n": (_I, [_VP, _VP, _VP, _I, _I, _VP]),
    "sg_gemv_grouped2_tab_q4_k_q8_f16out": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _I, _VP, _VP,
                                                 _VP, _I, _I, _I, _I, _VP]),
    "sg_gemv_grouped_tab_q4_k_q8_f16out": (_I, [_VP, _VP, _VP, _VP, _I, _VP, _VP, _I, _I, _I, _I,
                                                _VP]),
    "sg_scatter_routed_f16": (_I, [_VP, _VP, _VP, _I, _I, _I, _VP]),
    "sg_scatter_rows_f16": (_I, [_VP, _VP, _VP, _I, _I, _VP]),
    "sg_moe_dispatch_plan_workspace_bytes": (_SZ, [_I, _I]),
    "sg_moe_dispatch_plan": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _SZ, _I, _I, _I,
                                  _I, _I, _VP]),
    "sg_moe_prefill_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I]),
    "sg_moe_prefill": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
                            _VP, _SZ, _I, _I, _I, _I, _I, _F, _VP]),
    "sg_gguf_expert_dims": (_I, [ctypes.c_char_p, _VP, _VP, _VP, _VP, _VP]),
    "sg_expert_pool_load_gguf": (_I, [ctypes.c_char_p, _VP]),
    "sg_expert_pool_dims": (_I, [_VP, _VP, _VP, _VP, _VP]),
    "sg_expert_pool_table": (_VP, [_VP]),
    "sg_expert_pool_free": (None, [_VP]),
    "sg_q4k_quantize_row": (_I, [_VP, _VP, _I]),
}


def load(path=None):
    """Load libsager_hip.so and bind every C-ABI entry point.

    Raises OSError if the library has not been built (run
    ``python -m sager_amd.build_lib``)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise OSError(f"{p} not found: build it with `python -m sager_amd.build_lib`")
    lib = ctypes.CDLL(p)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib
