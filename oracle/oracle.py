"""numpy front end of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker.  The product path
(sager_amd/) never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        L.orc_half_to_float.restype = ctypes.c_float
        L.orc_half_to_float.argtypes = [ctypes.c_uint16]
        L.orc_expf.restype = ctypes.c_float
        L.orc_expf.argtypes = [ctypes.c_float]
        L.orc_count_expf_mismatch.restype = ctypes.c_int64
        L.orc_count_expf_mismatch.argtypes = [ctypes.c_int64, ctypes.c_uint64, ctypes.c_float,
                                              ctypes.c_float]
        L.orc_dequant.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.orc_dequant_q6k.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.orc_sigmoid.restype = ctypes.c_float
        L.orc_sigmoid.argtypes = [ctypes.c_float]
        L.orc_float_to_half.restype = ctypes.c_uint16
        L.orc_float_to_half.argtypes = [ctypes.c_float]
        _lib = L
    return _lib


def P(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def quantize_q8_k(x):
    """fp32 [rows, n] -> uint8 [rows, n/256*276]."""
    x = _c(np.atleast_2d(x), np.float32)
    rows, n = x.shape
    out = np.zeros((rows, n // 256 * 276), np.uint8)
    lib().orc_quantize_q8_k(P(x), P(out), n, rows)
    return out


def subblock_dots(w, xq, n_rows, k):
    w, xq = _c(w, np.uint8), _c(xq, np.uint8)
    d = np.zeros((n_rows, k // 256, 8), np.int32)
    lib().orc_subblock_dots(P(w), P(xq), P(d), n_rows, k)
    return d


def gemv(w, xq, n_rows, k, n_tokens=1):
    w, xq = _c(w, np.uint8), _c(xq, np.uint8)
    y = np.zeros((n_tokens, n_rows), np.float32)
    lib().orc_gemv_q4k_q8(P(w), P(xq), P(y), n_rows, k, n_tokens)
    return y


def dequant_q6k(w6, n):
    """Q6_K bytes (210 per 256 weights) -> fp32 [n]."""
    w6 = _c(w6, np.uint8)
    out = np.zeros(n, np.float32)
    lib().orc_dequant_q6k(P(w6), P(out), n)
    return out


def q6k_subgroup_dots(w6, xq, n_rows, k):
    """int32 [n_rows, k/256, 16]: sum over each 16-weight sub-group of (q6 - 32) * xq."""
    w6, xq = _c(w6, np.uint8), _c(xq, np.uint8)
    d = np.zeros((n_rows, k // 256, 16), np.int32)
    lib().orc_q6k_subgroup_dots(P(w6), P(xq), P(d), n_rows, k)
    return d


def gemv_q6k(w6, xq, n_rows, k):
    """y fp32 [n_rows] = W6 . xq (one token), the reference GPU kernel's order."""
    w6, xq = _c(w6, np.uint8), _c(xq, np.uint8)
    y = np.zeros(n_rows, np.float32)
    lib().orc_gemv_q6k_q8(P(w6), P(xq), P(y), n_rows, k)
    return y


def gemv_int(w, xq, n_rows, k, n_tokens=1):
    """The GEMV with the prefill path's integer-first super-block epilogue."""
    w, xq = _c(w, np.uint8), _c(xq, np.uint8)
    y = np.zeros((n_tokens, n_rows), np.float32)
    lib().orc_gemv_q4k_q8_int(P(w), P(xq), P(y), n_rows, k, n_tokens)
    return y


def dequant(w, n):
    w = _c(w, np.uint8)
    out = np.zeros(n, np.float32)
    lib().orc_dequant(P(w), P(out), n)
    return out


def silu_mul(g, u):
    g, u = _c(g, np.float32), _c(u, np.float32)
    h = np.zeros_like(g)
    lib().orc_silu_mul(P(g), P(u), P(h), g.size)
    return h


def expert_ffn(wg, wu, wd, x, hidden, n_ff):
    wg, wu, wd, x = _c(wg, np.uint8), _c(wu, np.uint8), _c(wd, np.uint8), _c(x, np.float32)
    y = np.zeros(hidden, np.float32)
    lib().orc_expert_ffn(P(wg), P(wu), P(wd), P(x), P(y), hidden, n_ff)
    return y


def router_topk(logits, k, shared_w=1.0, stride=None):
    logits = _c(np.atleast_2d(logits), np.float32)
    n_rows, n_expert = logits.shape
    stride = stride or k + 1
    idx = np.full((n_rows, stride), -1, np.int32)
    w = np.zeros((n_rows, stride), np.float32)
    lib().orc_router_topk(P(logits), P(idx), P(w), n_expert, k, stride, n_rows,
                          ctypes.c_float(shared_w))
    return idx, w


def moe_combine(expert_y, weight, residual=None):
    expert_y, weight = _c(expert_y, np.float32), _c(weight, np.float32)
    n_rows, slots, hidden = expert_y.shape
    out = np.zeros((n_rows, hidden), np.float32)
    res = _c(residual, np.float32) if residual is not None else None
    lib().orc_moe_combine(P(out), P(res) if res is not None else None, P(expert_y), P(weight),
                          slots - 1, hidden, n_rows)
    return out


def gemv_f32_lanes(w, x):
    """y [T, n_rows] = W fp32 [n_rows, k] . x fp32 [T, k] in the reference
    fp32 GEMV's lane order (q4_k.cu:133-149)."""
    w = _c(w, np.float32)
    x = _c(np.atleast_2d(x), np.float32)
    n_rows, k = w.shape
    y = np.zeros((x.shape[0], n_rows), np.float32)
    lib().orc_gemv_f32_lanes(P(w), P(x), P(y), n_rows, k, x.shape[0])
    return y


def sigmoid(g):
    return np.float32(lib().orc_sigmoid(ctypes.c_float(float(g))))


def _ptr_table(mats):
    arr = (ctypes.c_void_p * len(mats))()
    for i, m in enumerate(mats):
        arr[i] = None if m is None else m.ctypes.data
    return arr


def moe_layer(gate, up, down, shared, x, logits=None, idx=None, weight=None, residual=None,
              hidden=2048, n_ff=512, k=8, shared_w=1.0, n_threads=1, prefill=False,
              shared_gate_w=None):
    """gate/up/down: lists of per-expert uint8 arrays (None = absent);
    shared: (g, u, d) or None; shared_gate_w: fp32 [hidden] gate row of the
    shared expert or None.  Returns out [T, hidden], idx, weight.
    prefill=True: every GEMV in the integer-first epilogue order of the
    MFMA prefill path (orc_moe_prefill)."""
    x = _c(np.atleast_2d(x), np.float32)
    T = x.shape[0]
    n_expert = len(gate)
    for lst in (gate, up, down):
        for i, m in enumerate(lst):
            if m is not None:
                lst[i] = _c(m, np.uint8)
    tg, tu, td = _ptr_table(gate), _ptr_table(up), _ptr_table(down)
    sg = su = sd = None
    if shared is not None:
        shared = tuple(_c(m, np.uint8) for m in shared)
        sg, su, sd = (m.ctypes.data for m in shared)
    out = np.zeros((T, hidden), np.float32)
    res = _c(residual, np.float32) if residual is not None else None
    sgw = _c(shared_gate_w, np.float32) if shared_gate_w is not None else None
    psgw = P(sgw) if sgw is not None else None
    if prefill:
        if logits is not None:
            logits = _c(np.atleast_2d(logits), np.float32)
            idx = np.full((T, k + 1), -1, np.int32)
            weight = np.zeros((T, k + 1), np.float32)
        else:
            idx, weight = _c(idx, np.int32), _c(weight, np.float32).copy()
        lib().orc_moe_prefill(tg, tu, td, ctypes.c_void_p(sg), ctypes.c_void_p(su),
                              ctypes.c_void_p(sd), psgw, P(x),
                              P(logits) if logits is not None else None,
                              P(res) if res is not None else None, P(out), P(idx), P(weight), T,
                              hidden, n_ff, n_expert, k, ctypes.c_float(shared_w), n_threads)
        bad = ((idx[:, :k] < 0) | (idx[:, :k] >= n_expert)).any(axis=1)
        weight[bad] = 0.0
    elif logits is not None:
        logits = _c(np.atleast_2d(logits), np.float32)
        idx = np.full((T, k + 1), -1, np.int32)
        weight = np.zeros((T, k + 1), np.float32)
        lib().orc_moe_layer(tg, tu, td, ctypes.c_void_p(sg), ctypes.c_void_p(su),
                            ctypes.c_void_p(sd), psgw, P(x), P(logits),
                            P(res) if res is not None else None, P(out), P(idx), P(weight), T,
                            hidden, n_ff, n_expert, k, ctypes.c_float(shared_w), n_threads)
    else:
        idx, weight = _c(idx, np.int32), _c(weight, np.float32).copy()
        lib().orc_moe_layer_routed(tg, tu, td, ctypes.c_void_p(sg), ctypes.c_void_p(su),
                                   ctypes.c_void_p(sd), psgw, P(x), P(idx), P(weight),
                                   P(res) if res is not None else None, P(out), T, hidden,
                                   n_ff, n_expert, k, n_threads)
        # the oracle zeroes weights of bounds-killed rows on its own copy
        bad = ((idx[:, :k] < 0) | (idx[:, :k] >= n_expert)).any(axis=1)
        weight[bad] = 0.0
    return out, idx, weight


def float_to_half(x):
    """fp32 -> fp16 bits, round to nearest even (orc_float_to_half)."""
    x = _c(np.atleast_1d(x), np.float32)
    h = np.zeros(x.shape, np.uint16)
    lib().orc_float_to_half_n(P(x), P(h), ctypes.c_int64(x.size))
    return h


def moe_layer_f16(gate, up, down, shared, xn16, logits=None, idx=None, weight=None,
                  residual16=None, hidden=2048, n_ff=512, k=8, shared_w=1.0, n_threads=1,
                  prefill=False, shared_gate_w=None):
    """The layer on the session's fp16 buffers (orc_moe_layer_f16io): xn16
    fp16 [T, hidden] (normed activations), residual16 fp16 [T, hidden] or
    None.  Returns out fp16 [T, hidden], idx, weight."""
    x = _c(np.atleast_2d(xn16).astype(np.float16).astype(np.float32), np.float32)
    T = x.shape[0]
    n_expert = len(gate)
    for lst in (gate, up, down):
        for i, m in enumerate(lst):
            if m is not None:
                lst[i] = _c(m, np.uint8)
    tg, tu, td = _ptr_table(gate), _ptr_table(up), _ptr_table(down)
    sg = su = sd = None
    if shared is not None:
        shared = tuple(_c(m, np.uint8) for m in shared)
        sg, su, sd = (m.ctypes.data for m in shared)
    out = np.zeros((T, hidden), np.float32)
    res = (_c(np.asarray(residual16).astype(np.float16).astype(np.float32), np.float32)
           if residual16 is not None else None)
    sgw = _c(shared_gate_w, np.float32) if shared_gate_w is not None else None
    if logits is not None:
        logits = _c(np.atleast_2d(logits), np.float32)
        idx = np.full((T, k + 1), -1, np.int32)
        weight = np.zeros((T, k + 1), np.float32)
    else:
        idx, weight = _c(idx, np.int32), _c(weight, np.float32).copy()
    lib().orc_moe_layer_f16io(tg, tu, td, ctypes.c_void_p(sg), ctypes.c_void_p(su),
                              ctypes.c_void_p(sd), P(sgw) if sgw is not None else None, P(x),
                              P(logits) if logits is not None else None,
                              P(res) if res is not None else None, P(out), P(idx), P(weight), T,
                              hidden, n_ff, n_expert, k, ctypes.c_float(shared_w), n_threads,
                              int(prefill))
    bad = ((idx[:, :k] < 0) | (idx[:, :k] >= n_expert)).any(axis=1)
    weight[bad] = 0.0
    return out.astype(np.float16), idx, weight


def dispatch_scan(idx, weight, k, n_expert, tok_per=1):
    idx, weight = _c(idx, np.int32), _c(weight, np.float32).copy()
    n_rows = idx.shape[0]
    gslot = np.zeros(n_rows * k, np.int32)
    grows = np.zeros(n_rows * k, np.int32)
    off = np.zeros(n_expert + 1, np.int32)
    toff = np.zeros(n_expert + 1, np.int32)
    meta = np.zeros(4, np.int32)
    lib().orc_dispatch_scan(P(idx), P(weight), P(gslot), P(grows), P(off), P(toff), P(meta),
                            n_rows, k, n_expert, tok_per)
    return dict(weight=weight, gslot=gslot, grows=grows, off=off, toff=toff, meta=meta)
