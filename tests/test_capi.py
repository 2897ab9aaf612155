"""C-ABI boundary checks that need no GPU: the library loads, exports every
entry point include/sager_hip.h declares, the Python bindings cover exactly
that set, and argument validation rejects bad geometry before any launch."""
import ctypes
import os
import re

import pytest

import sager_amd

HDR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                   "sager_hip.h")


def declared():
    text = open(HDR).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sg_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return sager_amd.load()


def test_exports_every_declared_symbol(lib):
    names = declared()
    assert len(names) >= 13
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(sager_amd.SIGNATURES) == names


def test_version(lib):
    assert b"gfx950" in lib.sg_version()


def test_validation_without_launch(lib):
    bad = ctypes.c_void_p(16)
    assert lib.sg_gemv_q4_k_q8(None, bad, bad, 8, 2048, None) == 1
    assert b"null" in lib.sg_last_error()
    assert lib.sg_gemv_q4_k_q8(bad, bad, bad, 8, 2000, None) == 4
    assert lib.sg_gemv_q4_k_q8(bad, bad, bad, 8, 256 * 65, None) == 8
    assert lib.sg_gemv_q4_k_q8_batched(bad, bad, bad, 8, 2048, 17, None) == 8
    assert lib.sg_quantize_q8_k(bad, bad, 100, 1, None) == 4
    assert lib.sg_router_topk(bad, bad, bad, 2000, 8, 9, 1, 1.0, None) == 4
    assert lib.sg_router_topk(bad, bad, bad, 256, 8, 8, 1, 1.0, None) == 4   # stride < k+1
    ws = lib.sg_moe_layer_workspace_bytes(1, 2048, 512, 256, 8)
    assert ws > 0
    args = [bad] * 3 + [None] * 3 + [None] + [bad, bad, None, bad, bad, bad, bad]
    assert lib.sg_moe_layer(*args, ws - 1, 1, 2048, 512, 256, 8, 1.0, None) == 1
    assert lib.sg_moe_layer(*args, ws, 17, 2048, 512, 256, 8, 1.0, None) == 8
    assert lib.sg_moe_layer(*args, ws, 1, 2048, 512, 256, 33, 1.0, None) == 4
    sh = [bad, None, None]
    args2 = [bad] * 3 + sh + [None] + [bad, bad, None, bad, bad, bad, bad]
    assert lib.sg_moe_layer(*args2, ws, 1, 2048, 512, 256, 8, 1.0, None) == 1
    # fp16-buffer launchers and the fp32 x fp16 GEMV reject bad geometry
    assert lib.sg_silu_mul_f16(bad, bad, bad, 0, 512, None) == 4
    assert lib.sg_moe_combine_batched_f16(bad, bad, bad, 8, 2048, 70000, None) == 4
    assert lib.sg_sigmoid_gate_scalar_batched_f16(None, bad, 1, 2048, None) == 1
    assert lib.sg_gemv_f32_out_f16x(bad, bad, bad, 256, 0, 1, None) == 4
    assert lib.sg_gemv_ptrs_q4_k_q8_f16out(bad, bad, bad, 0, 512, 2048, None) == 4
    assert lib.sg_gemv_q4_k_q8_f16out_batched(bad, bad, bad, 8, 2048, 17, None) == 8
