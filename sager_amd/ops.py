"""Host-side mirror of the reference's launcher API over libsager_hip.so.

Each function keeps the name and argument meaning of the ``sager::cuda``
launcher it replaces (include/sager/kernels/cuda_ops.hpp) and takes torch
tensors that live on the GPU; it enqueues on torch's current stream and
never synchronizes.  Errors raise :class:`SagerError` with the library's
message (the reference's launchers return void and surface failures through
cudaGetLastError).  Block tensors are uint8 views of the packed formats:
Q4_K ``[..., 144]`` per 256 weights, Q8_K ``[..., 276]`` per 256 values.
"""
import ctypes

import numpy as np
import torch

from . import Q4K_BYTES, Q8K_BYTES, QK, load


class SagerError(RuntimeError):
    pass


def _stream():
    return torch.cuda.current_stream().cuda_stream


class DeviceAddress:
    """A raw device address the library owns (e.g. an expert pool's pointer
    table), usable wherever a device tensor argument is expected."""

    def __init__(self, addr, device):
        self.addr, self.device = int(addr), torch.device(device)
        self.is_cuda = True

    def data_ptr(self):
        return self.addr

    def is_contiguous(self):
        return True


def _ptr(t):
    if t is None:
        return None
    if not t.is_cuda:
        raise SagerError("tensor must be on the GPU")
    if not t.is_contiguous():
        raise SagerError("tensor must be contiguous")
    return t.data_ptr()


def _dtypes(name, **args):
    """Raise unless every (tensor, dtype) pair matches and the tensor is a
    contiguous GPU tensor: the launchers read raw bits."""
    for arg, (t, dt) in args.items():
        if t.dtype != dt:
            raise SagerError(f"{name}: {arg} must be {dt}, got {t.dtype}")
        _ptr(t)


def _check(status):
    if status != 0:
        raise SagerError(f"status {status}: {load().sg_last_error().decode()}")


def q8k_empty(n_tokens, n, device="cuda"):
    return torch.empty((n_tokens, (n // QK) * Q8K_BYTES), dtype=torch.uint8, device=device)


def quantize_q8_k(x, out=None):
    """cuda::quantize_q8_k (cuda_ops.hpp:271-273): rows of x (fp32 or fp16,
    [..., n]) -> Q8_K blocks [rows, n/256*276]."""
    n = x.shape[-1]
    rows = x.numel() // n
    if out is None:
        out = q8k_empty(rows, n, x.device)
    fn = load().sg_quantize_q8_k_f16 if x.dtype == torch.float16 else load().sg_quantize_q8_k
    if x.dtype not in (torch.float16, torch.float32):
        raise SagerError("x must be fp32 or fp16")
    _check(fn(_ptr(x), _ptr(out), n, rows, _stream()))
    return out


def gemv_q4_k_q8(w, x_q8, n_rows, k, y=None):
    """cuda::gemv_q4_k_q8 (cuda_ops.hpp:41-42): y[n_rows] fp32 = W . x."""
    if y is None:
        y = torch.empty(n_rows, dtype=torch.float32, device=w.device)
    _check(load().sg_gemv_q4_k_q8(_ptr(w), _ptr(x_q8), _ptr(y), n_rows, k, _stream()))
    return y


def gemv_q4_k_q8_f16out(w, x_q8, n_rows, k, y=None):
    """cuda::gemv_q4_k_q8_f16out (cuda_ops.hpp:53-54): y fp16 [n_rows]."""
    if y is None:
        y = torch.empty(n_rows, dtype=torch.float16, device=w.device)
    _check(load().sg_gemv_q4_k_q8_f16out(_ptr(w), _ptr(x_q8), _ptr(y), n_rows, k, _stream()))
    return y


def gemv_nm_q4_k_q8_f16out(ws, x_q8, rows, k, ys=None):
    """cuda::gemv2m / gemv3m_q4_k_q8_f16out (cuda_ops.hpp:156-164): the two or
    three projections of one x in one launch; returns the fp16 outputs."""
    if len(ws) not in (2, 3) or len(rows) != len(ws):
        raise SagerError("two or three matrices")
    if ys is None:
        ys = [torch.empty(r, dtype=torch.float16, device=x_q8.device) for r in rows]
    if len(ws) == 2:
        _check(load().sg_gemv2m_q4_k_q8_f16out(_ptr(ws[0]), _ptr(ws[1]), _ptr(x_q8), _ptr(ys[0]),
                                               _ptr(ys[1]), rows[0], rows[1], k, _stream()))
    else:
        _check(load().sg_gemv3m_q4_k_q8_f16out(_ptr(ws[0]), _ptr(ws[1]), _ptr(ws[2]), _ptr(x_q8),
                                               _ptr(ys[0]), _ptr(ys[1]), _ptr(ys[2]), rows[0],
                                               rows[1], rows[2], k, _stream()))
    return ys


def gemv_q4_k_q8_f16out_resadd(w, x_q8, res_inout, n_rows, k, y=None):
    """cuda::gemv_q4_k_q8_f16out_resadd (cuda_ops.hpp:166-171): y = f16(W.x),
    res_inout += y in fp16 (in place)."""
    if y is None:
        y = torch.empty(n_rows, dtype=torch.float16, device=w.device)
    _check(load().sg_gemv_q4_k_q8_f16out_resadd(_ptr(w), _ptr(x_q8), _ptr(y), _ptr(res_inout),
                                                n_rows, k, _stream()))
    return y


def gemv_q6_k_q8(w6, x_q8, n_rows, k, y=None):
    """cuda::gemv_q6_k_q8 (cuda_ops.hpp:44-48): y[n_rows] fp32 = W6 . x, W6 raw
    block_q6_K bytes (210 per 256 weights)."""
    if y is None:
        y = torch.empty(n_rows, dtype=torch.float32, device=w6.device)
    _check(load().sg_gemv_q6_k_q8(_ptr(w6), _ptr(x_q8), _ptr(y), n_rows, k, _stream()))
    return y


def gemv_q4_k_q8_batched(w, x_q8, n_rows, k, n_tokens, y=None):
    """cuda::gemv_q4_k_q8_batched (cuda_ops.hpp:72-74): y[n_tokens, n_rows]."""
    if y is None:
        y = torch.empty((n_tokens, n_rows), dtype=torch.float32, device=w.device)
    _check(load().sg_gemv_q4_k_q8_batched(_ptr(w), _ptr(x_q8), _ptr(y), n_rows, k, n_tokens,
                                          _stream()))
    return y


def gemv_ptrs_q4_k_q8(ptrs, x_q8, n_ptrs, rows_per, k, y=None):
    """cuda::gemv_ptrs_q4_k_q8_f16out (cuda_ops.hpp:60-63), fp32 out.
    ptrs: int64 device tensor of n_ptrs matrix addresses."""
    if y is None:
        y = torch.empty(n_ptrs * rows_per, dtype=torch.float32, device=x_q8.device)
    _check(load().sg_gemv_ptrs_q4_k_q8(_ptr(ptrs), _ptr(x_q8), _ptr(y), n_ptrs, rows_per, k,
                                       _stream()))
    return y


def gemv_ptrs_q4_k_q8_f16out(ptrs, x_q8, n_ptrs, rows_per, k, y=None):
    """cuda::gemv_ptrs_q4_k_q8_f16out (cuda_ops.hpp:60-63): fp16 y."""
    if y is None:
        y = torch.empty(n_ptrs * rows_per, dtype=torch.float16, device=x_q8.device)
    _check(load().sg_gemv_ptrs_q4_k_q8_f16out(_ptr(ptrs), _ptr(x_q8), _ptr(y), n_ptrs, rows_per,
                                              k, _stream()))
    return y


def gemv_q4_k_q8_f16out_batched(w, x_q8, n_rows, k, n_tokens, y=None):
    """cuda::gemv_q4_k_q8_f16out_batched (cuda_ops.hpp:67-70): fp16 y[n_tokens, n_rows]."""
    if y is None:
        y = torch.empty((n_tokens, n_rows), dtype=torch.float16, device=w.device)
    _check(load().sg_gemv_q4_k_q8_f16out_batched(_ptr(w), _ptr(x_q8), _ptr(y), n_rows, k,
                                                 n_tokens, _stream()))
    return y


def gemv_f32_out_f16x(w, x, y=None):
    """cuda::gemv_f32_out_f16x / _batched (q4_k.cu:1713-1718, 1987-1991):
    W fp32 [n_rows, k] . x fp16 [n_tokens, k] -> y fp32 [n_tokens, n_rows]
    (router logits, the shared expert's gate logit)."""
    n_rows, k = w.shape
    x2 = x.reshape(-1, k)
    if x2.dtype != torch.float16 or w.dtype != torch.float32:
        raise SagerError("w must be fp32 and x fp16")
    if y is None:
        y = torch.empty((x2.shape[0], n_rows), dtype=torch.float32, device=w.device)
    _check(load().sg_gemv_f32_out_f16x(_ptr(w), _ptr(x2), _ptr(y), n_rows, k, x2.shape[0],
                                       _stream()))
    return y


def subblock_dots(w, x_q8, n_rows, k):
    """int32 sub-block dot sums [n_rows, k/256, 8] (test hook)."""
    d = torch.empty((n_rows, k // QK, 8), dtype=torch.int32, device=w.device)
    _check(load().sg_q4k_subblock_dots(_ptr(w), _ptr(x_q8), _ptr(d), n_rows, k, _stream()))
    return d


def router_topk_batched(logits, n_expert_used, shared_w=1.0, idx_stride=None):
    """cuda::router_topk_batched (cuda_ops.hpp:175-177 / 351-360):
    logits [n_rows, n_expert] -> idx int32, weight fp32 [n_rows, idx_stride]."""
    n_rows, n_expert = logits.shape
    stride = idx_stride or n_expert_used + 1
    idx = torch.full((n_rows, stride), -1, dtype=torch.int32, device=logits.device)
    w = torch.zeros((n_rows, stride), dtype=torch.float32, device=logits.device)
    _check(load().sg_router_topk(_ptr(logits), _ptr(idx), _ptr(w), n_expert, n_expert_used,
                                 stride, n_rows, float(shared_w), _stream()))
    return idx, w


def router_topk(logits, n_expert_used, shared_w=1.0):
    """cuda::router_topk (cuda_ops.hpp:351-352): one row."""
    idx, w = router_topk_batched(logits.reshape(1, -1), n_expert_used, shared_w)
    return idx[0], w[0]


def silu_mul(g, u, out=None):
    """cuda::silu_mul_f16 (cuda_ops.hpp:305-306), fp32."""
    if out is None:
        out = torch.empty_like(g)
    _check(load().sg_silu_mul(_ptr(out), _ptr(g), _ptr(u), g.numel(), _stream()))
    return out


def moe_combine_batched(expert_y, weight, residual=None, out=None):
    """cuda::moe_combine_batched_f16 (cuda_ops.hpp:397-399), fp32:
    expert_y [n_rows, n_used+1, hidden], weight [n_rows, n_used+1]."""
    n_rows, slots, hidden = expert_y.shape
    if out is None:
        out = torch.empty((n_rows, hidden), dtype=torch.float32, device=expert_y.device)
    _check(load().sg_moe_combine(_ptr(out), _ptr(residual), _ptr(expert_y), _ptr(weight),
                                 slots - 1, hidden, n_rows, _stream()))
    return out


def silu_mul_f16(g, u, out=None):
    """cuda::silu_mul_f16 (cuda_ops.hpp:305-306) on fp16 [rows, n_ff] buffers."""
    if g.dtype != torch.float16 or u.dtype != torch.float16:
        raise SagerError("g and u must be fp16")
    if out is None:
        out = torch.empty_like(g)
    n_ff = g.shape[-1]
    _check(load().sg_silu_mul_f16(_ptr(out), _ptr(g), _ptr(u), g.numel() // n_ff, n_ff,
                                  _stream()))
    return out


def moe_combine_batched_f16(out, expert_y, weight):
    """cuda::moe_combine_batched_f16 (cuda_ops.hpp:379-381): out fp16
    [n_rows, hidden] holds the residual and receives the sum in place;
    expert_y fp16 [n_rows, n_used+1, hidden], weight fp32 [n_rows, n_used+1]."""
    _dtypes("moe_combine_batched_f16", out=(out, torch.float16),
            expert_y=(expert_y, torch.float16), weight=(weight, torch.float32))
    n_rows, slots, hidden = expert_y.shape
    if out.shape != (n_rows, hidden) or weight.shape != (n_rows, slots):
        raise SagerError("moe_combine_batched_f16: out [n_rows, hidden], weight [n_rows, slots]")
    _check(load().sg_moe_combine_batched_f16(_ptr(out), _ptr(expert_y), _ptr(weight), slots - 1,
                                             hidden, n_rows, _stream()))
    return out


def sigmoid_gate_scalar_batched_f16(out, g):
    """cuda::sigmoid_gate_scalar_batched_f16 (cuda_ops.hpp:384-386):
    out fp16 [n_rows, hidden] *= sigmoid(g[row]) in place."""
    _dtypes("sigmoid_gate_scalar_batched_f16", out=(out, torch.float16), g=(g, torch.float32))
    out2 = out.reshape(g.numel(), -1)
    _check(load().sg_sigmoid_gate_scalar_batched_f16(_ptr(out2), _ptr(g), out2.shape[0],
                                                     out2.shape[1], _stream()))
    return out


def sigmoid_gate_scalar_f16(out, g):
    """cuda::sigmoid_gate_scalar_f16 (cuda_ops.hpp:315-316): out fp16 [n] *= sigmoid(g[0])."""
    _dtypes("sigmoid_gate_scalar_f16", out=(out, torch.float16), g=(g, torch.float32))
    _check(load().sg_sigmoid_gate_scalar_f16(_ptr(out), _ptr(g), out.numel(), _stream()))
    return out


class MoeLayer:
    """One MoE layer's device-side pointer tables and workspace; ``forward``
    is the device-path dispatch of Session::moe_dispatch_device
    (session.cpp:2482-3030) as one call.  ``stages``: 3 = front and back (the
    whole layer), 1 / 2 = one of the two launches.  ``shared_gate_w``: the
    shared expert's fp32 [hidden] gate row (LayerWeights::shared_gate_w), or
    None."""

    def __init__(self, tab_gate, tab_up, tab_down, shared=None, hidden=2048, n_ff=512,
                 n_expert=256, k=8, max_tokens=1, shared_w=1.0, shared_gate_w=None):
        self.tab_gate, self.tab_up, self.tab_down = tab_gate, tab_up, tab_down
        self.shared = shared
        self.shared_gate_w = shared_gate_w
        self.hidden, self.n_ff, self.n_expert, self.k = hidden, n_ff, n_expert, k
        self.shared_w = float(shared_w)
        self.max_tokens = max_tokens
        nbytes = load().sg_moe_layer_workspace_bytes(max_tokens, hidden, n_ff, n_expert, k)
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=tab_gate.device)

    def forward(self, x, logits=None, residual=None, out=None, idx=None, weight=None,
                stages=3, workspace=None):
        T = x.shape[0]
        if T > self.max_tokens:
            raise SagerError(f"{T} tokens > max_tokens={self.max_tokens}")
        dev = x.device
        if out is None:
            out = torch.empty((T, self.hidden), dtype=torch.float32, device=dev)
        if idx is None:
            idx = torch.full((T, self.k + 1), -1, dtype=torch.int32, device=dev)
        if weight is None:
            weight = torch.zeros((T, self.k + 1), dtype=torch.float32, device=dev)
        sg, su, sd = self.shared if self.shared is not None else (None, None, None)
        ws = self.workspace if workspace is None else workspace
        _check(load().sg_moe_layer_stages(
            _ptr(self.tab_gate), _ptr(self.tab_up), _ptr(self.tab_down), _ptr(sg), _ptr(su),
            _ptr(sd), _ptr(self.shared_gate_w), _ptr(x), _ptr(logits), _ptr(residual), _ptr(out),
            _ptr(idx), _ptr(weight), _ptr(ws), ws.numel(), T, self.hidden, self.n_ff,
            self.n_expert, self.k, self.shared_w, stages, _stream()))
        return out, idx, weight

    _F16_ENTRY = "sg_moe_layer_f16"

    def forward_f16(self, xn=None, xq=None, logits=None, residual=None, out=None, idx=None,
                    weight=None, workspace=None):
        """The layer on the session's fp16 buffers (sg_moe_layer_f16 /
        sg_moe_prefill_f16): xn fp16 [T, hidden] and/or xq, a Q8_K of it
        (uint8 [T, hidden/256*276], used as is); residual/out fp16 [T, hidden]
        (may be the same tensor)."""
        src = xn if xn is not None else xq
        if src is None:
            raise SagerError("forward_f16 needs xn or xq")
        T = src.shape[0]
        if T > self.max_tokens:
            raise SagerError(f"{T} tokens > max_tokens={self.max_tokens}")
        if xn is not None:
            _dtypes(self._F16_ENTRY, xn=(xn, torch.float16))
        if xq is not None:
            _dtypes(self._F16_ENTRY, xq=(xq, torch.uint8))
            if xq.numel() != T * (self.hidden // QK) * Q8K_BYTES:
                raise SagerError("xq must hold T x hidden/256 Q8_K blocks")
        dev = src.device
        if out is None:
            out = torch.empty((T, self.hidden), dtype=torch.float16, device=dev)
        _dtypes(self._F16_ENTRY, out=(out, torch.float16))
        if residual is not None:
            _dtypes(self._F16_ENTRY, residual=(residual, torch.float16))
        if idx is None:
            idx = torch.full((T, self.k + 1), -1, dtype=torch.int32, device=dev)
        if weight is None:
            weight = torch.zeros((T, self.k + 1), dtype=torch.float32, device=dev)
        sg, su, sd = self.shared if self.shared is not None else (None, None, None)
        ws = self.workspace if workspace is None else workspace
        _check(getattr(load(), self._F16_ENTRY)(
            _ptr(self.tab_gate), _ptr(self.tab_up), _ptr(self.tab_down), _ptr(sg), _ptr(su),
            _ptr(sd), _ptr(self.shared_gate_w), _ptr(xn), _ptr(xq), _ptr(logits),
            _ptr(residual), _ptr(out), _ptr(idx), _ptr(weight), _ptr(ws), ws.numel(), T,
            self.hidden, self.n_ff, self.n_expert, self.k, self.shared_w, _stream()))
        return out, idx, weight


def moe_dispatch_scan(idx, weight, n_expert, k, tok_per=64):
    """cuda::moe_dispatch_scan (cuda_ops.hpp:219-222) on the device: returns
    dict(gslot, grows, off, toff, meta); `weight` is bounds-killed in place."""
    n_rows = idx.shape[0]
    dev = idx.device
    gslot = torch.empty(n_rows * k, dtype=torch.int32, device=dev)
    grows = torch.empty(n_rows * k, dtype=torch.int32, device=dev)
    off = torch.empty(n_expert + 2, dtype=torch.int32, device=dev)
    toff = torch.empty(n_expert + 2, dtype=torch.int32, device=dev)
    meta = torch.zeros(4, dtype=torch.int32, device=dev)
    _check(load().sg_moe_dispatch_scan(_ptr(idx), _ptr(weight), _ptr(gslot), _ptr(grows),
                                       _ptr(off), _ptr(toff), _ptr(meta), n_rows, k, n_expert,
                                       tok_per, _stream()))
    return dict(gslot=gslot, grows=grows, off=off, toff=toff, meta=meta)


def router_topk_fused(w, x, k, idx=None, weight=None):
    """cuda::router_topk_fused (cuda_ops.hpp:173-177): the router GEMV of one
    fp16 token x [hidden] with fp32 W [n_expert, hidden] and its top-k in one
    launch; idx/weight rows of k+1 slots (the shared slot is not written)."""
    n_expert, hidden = w.shape
    if idx is None:
        idx = torch.full((k + 1,), -1, dtype=torch.int32, device=w.device)
    if weight is None:
        weight = torch.zeros(k + 1, dtype=torch.float32, device=w.device)
    _dtypes("router_topk_fused", w=(w, torch.float32), x=(x, torch.float16),
            idx=(idx, torch.int32), weight=(weight, torch.float32))
    _check(load().sg_router_topk_fused(_ptr(w), _ptr(x), _ptr(idx), _ptr(weight), n_expert, k,
                                       hidden, _stream()))
    return idx, weight


# ---- stage-by-stage launchers of the grouped path (sg_stages.hip) -------------

def gather_rows_q8(src, src_rows, row_blocks, meta=None, r_max=None, out=None):
    """cuda::gather_rows_q8 / gather_rows_q8_n (cuda_ops.hpp:364-366,
    226-228): out[r] = src[src_rows[r]] for whole Q8_K rows (uint8 tensors of
    row_blocks*276 bytes per row); with meta, only r < meta[0] (r_max rows
    bound the grid)."""
    n = r_max if meta is not None else src_rows.numel()
    if out is None:
        out = torch.empty((n, row_blocks * Q8K_BYTES), dtype=torch.uint8, device=src.device)
    _dtypes("gather_rows_q8", src=(src, torch.uint8), out=(out, torch.uint8),
            src_rows=(src_rows, torch.int32))
    if meta is None:
        _check(load().sg_gather_rows_q8(_ptr(out), _ptr(src), _ptr(src_rows), n, row_blocks,
                                        _stream()))
    else:
        _dtypes("gather_rows_q8_n", meta=(meta, torch.int32))
        _check(load().sg_gather_rows_q8_n(_ptr(out), _ptr(src), _ptr(src_rows), _ptr(meta), n,
                                          row_blocks, _stream()))
    return out


def gather_rows_f16_n(src, src_rows, meta, r_max, out=None):
    """cuda::gather_rows_f16_n (cuda_ops.hpp:229-231): out[r] = src[src_rows[r]]
    for r < meta[0], fp16 rows."""
    hidden = src.shape[-1]
    if out is None:
        out = torch.empty((r_max, hidden), dtype=torch.float16, device=src.device)
    _dtypes("gather_rows_f16_n", src=(src, torch.float16), out=(out, torch.float16),
            src_rows=(src_rows, torch.int32), meta=(meta, torch.int32))
    _check(load().sg_gather_rows_f16_n(_ptr(out), _ptr(src), _ptr(src_rows), _ptr(meta), r_max,
                                       hidden, _stream()))
    return out


def silu_mul_f16_n(g, u, d_rows, out=None):
    """cuda::silu_mul_f16_n (cuda_ops.hpp:232-234): the first d_rows[0] rows of
    fp16 [rows_max, n_ff] buffers."""
    if out is None:
        out = torch.empty_like(g)
    _dtypes("silu_mul_f16_n", g=(g, torch.float16), u=(u, torch.float16),
            out=(out, torch.float16), d_rows=(d_rows, torch.int32))
    n_ff = g.shape[-1]
    _check(load().sg_silu_mul_f16_n(_ptr(out), _ptr(g), _ptr(u), _ptr(d_rows), g.numel() // n_ff,
                                    n_ff, _stream()))
    return out


def quantize_q8_k_n(x, d_rows, row_mult, n_max, out=None):
    """cuda::quantize_q8_k_n (cuda_ops.hpp:235-237): Q8_K of the first
    d_rows[0] * row_mult fp16 values of x."""
    if out is None:
        out = torch.empty((n_max * Q8K_BYTES,), dtype=torch.uint8, device=x.device)
    _dtypes("quantize_q8_k_n", x=(x, torch.float16), out=(out, torch.uint8),
            d_rows=(d_rows, torch.int32))
    _check(load().sg_quantize_q8_k_n(_ptr(x), _ptr(out), _ptr(d_rows), row_mult, n_max,
                                     _stream()))
    return out


def gemv_grouped2_tab_q4_k_q8_f16out(wg_tab, wu_tab, plan, tiles_max, xq, n_rows, k, n_expert,
                                     tok_per, yg, yu, mail, mail_n):
    """cuda::gemv_grouped2_tab_q4_k_q8_f16out_mtok (cuda_ops.hpp:240-244) over
    a moe_dispatch_scan plan; yg/yu fp16 [positions, n_rows]."""
    _dtypes("gemv_grouped2_tab", yg=(yg, torch.float16), yu=(yu, torch.float16),
            mail=(mail, torch.int32), mail_n=(mail_n, torch.int32), xq=(xq, torch.uint8))
    _check(load().sg_gemv_grouped2_tab_q4_k_q8_f16out(
        _ptr(wg_tab), _ptr(wu_tab), _ptr(plan["off"]), _ptr(plan["toff"]), _ptr(plan["meta"]),
        _ptr(mail), _ptr(mail_n), tiles_max, _ptr(xq), _ptr(yg), _ptr(yu), n_rows, k, n_expert,
        tok_per, _stream()))
    return yg, yu


def gemv_grouped_tab_q4_k_q8_f16out(w_tab, plan, tiles_max, xq, n_rows, k, n_expert, tok_per, y):
    """cuda::gemv_grouped_tab_q4_k_q8_f16out_mtok (cuda_ops.hpp:247-250)."""
    _dtypes("gemv_grouped_tab", y=(y, torch.float16), xq=(xq, torch.uint8))
    _check(load().sg_gemv_grouped_tab_q4_k_q8_f16out(
        _ptr(w_tab), _ptr(plan["off"]), _ptr(plan["toff"]), _ptr(plan["meta"]), tiles_max,
        _ptr(xq), _ptr(y), n_rows, k, n_expert, tok_per, _stream()))
    return y


def scatter_routed_f16(expert_y, grouped_out, gslot, n_rows, n_used):
    """cuda::scatter_routed_f16 (cuda_ops.hpp:372-374): expert_y fp16
    [n_rows, n_used+1, hidden] receives grouped_out[gslot[row*n_used+kk]]."""
    hidden = expert_y.shape[-1]
    _dtypes("scatter_routed_f16", expert_y=(expert_y, torch.float16),
            grouped_out=(grouped_out, torch.float16), gslot=(gslot, torch.int32))
    _check(load().sg_scatter_routed_f16(_ptr(expert_y), _ptr(grouped_out), _ptr(gslot), n_rows,
                                        n_used, hidden, _stream()))
    return expert_y


def scatter_rows_f16(dst, src, dst_rows):
    """cuda::scatter_rows_f16 (cuda_ops.hpp:408-409): dst[dst_rows[i]] = src[i]."""
    hidden = src.shape[-1]
    _dtypes("scatter_rows_f16", dst=(dst, torch.float16), src=(src, torch.float16),
            dst_rows=(dst_rows, torch.int32))
    _check(load().sg_scatter_rows_f16(_ptr(dst), _ptr(src), _ptr(dst_rows), src.shape[0], hidden,
                                      _stream()))
    return dst


def moe_dispatch_plan(idx, weight, n_expert, k, tok_per=64, shared_tail=0, tiles=True):
    """The multi-workgroup plan (sg_moe_dispatch_plan): the arrays of
    moe_dispatch_scan plus the grouped kernels' tile list; `weight` is
    bounds-killed in place."""
    n_rows = idx.shape[0]
    dev = idx.device
    gslot = torch.empty(n_rows * k, dtype=torch.int32, device=dev)
    grows = torch.empty(n_rows * k + shared_tail, dtype=torch.int32, device=dev)
    off = torch.empty(n_expert + 2, dtype=torch.int32, device=dev)
    toff = torch.empty(n_expert + 2, dtype=torch.int32, device=dev)
    meta = torch.zeros(4, dtype=torch.int32, device=dev)
    n_tiles = (2 + (n_rows * k + tok_per - 1) // tok_per + n_expert
               + (shared_tail + tok_per - 1) // tok_per)
    tl = torch.empty(n_tiles, dtype=torch.int32, device=dev) if tiles else None
    nbytes = load().sg_moe_dispatch_plan_workspace_bytes(n_rows, n_expert)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    _check(load().sg_moe_dispatch_plan(_ptr(idx), _ptr(weight), _ptr(gslot), _ptr(grows),
                                       _ptr(off), _ptr(toff), _ptr(meta), _ptr(tl), _ptr(ws),
                                       nbytes, n_rows, k, n_expert, tok_per, shared_tail,
                                       _stream()))
    return dict(gslot=gslot, grows=grows, off=off, toff=toff, meta=meta, tiles=tl)


class MoePrefill(MoeLayer):
    """The same layer for a prefill chunk of up to max_tokens tokens: the
    device plan and int8-MFMA grouped contractions (sg_moe_prefill)."""

    _F16_ENTRY = "sg_moe_prefill_f16"

    def __init__(self, tab_gate, tab_up, tab_down, shared=None, hidden=2048, n_ff=512,
                 n_expert=256, k=8, max_tokens=2048, shared_w=1.0, shared_gate_w=None):
        self.tab_gate, self.tab_up, self.tab_down = tab_gate, tab_up, tab_down
        self.shared = shared
        self.shared_gate_w = shared_gate_w
        self.hidden, self.n_ff, self.n_expert, self.k = hidden, n_ff, n_expert, k
        self.shared_w = float(shared_w)
        self.max_tokens = max_tokens
        nbytes = load().sg_moe_prefill_workspace_bytes(max_tokens, hidden, n_ff, n_expert, k)
        self.workspace = torch.empty(nbytes, dtype=torch.uint8, device=tab_gate.device)

    def forward(self, x, logits=None, residual=None, out=None, idx=None, weight=None,
                workspace=None):
        T = x.shape[0]
        if T > self.max_tokens:
            raise SagerError(f"{T} tokens > max_tokens={self.max_tokens}")
        dev = x.device
        if out is None:
            out = torch.empty((T, self.hidden), dtype=torch.float32, device=dev)
        if idx is None:
            idx = torch.full((T, self.k + 1), -1, dtype=torch.int32, device=dev)
        if weight is None:
            weight = torch.zeros((T, self.k + 1), dtype=torch.float32, device=dev)
        sg, su, sd = self.shared if self.shared is not None else (None, None, None)
        ws = self.workspace if workspace is None else workspace
        _check(load().sg_moe_prefill(
            _ptr(self.tab_gate), _ptr(self.tab_up), _ptr(self.tab_down), _ptr(sg), _ptr(su),
            _ptr(sd), _ptr(self.shared_gate_w), _ptr(x), _ptr(logits), _ptr(residual), _ptr(out),
            _ptr(idx), _ptr(weight), _ptr(ws), ws.numel(), T, self.hidden, self.n_ff,
            self.n_expert, self.k, self.shared_w, _stream()))
        return out, idx, weight


def q4k_quantize_row(x):
    """Host Q4_K quantizer (the reference's quantize_row, q4_k.cpp:62-174):
    fp32 numpy [n] (n a multiple of 256) -> uint8 [n/256, 144]."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros((x.size // QK, Q4K_BYTES), np.uint8)
    _check(load().sg_q4k_quantize_row(x.ctypes.data_as(ctypes.c_void_p),
                                      out.ctypes.data_as(ctypes.c_void_p), x.size))
    return out


def gguf_expert_dims(path):
    """(n_layers, n_expert, hidden, n_ff, q6_down_layers) of a GGUF v3 file's
    blk.L.ffn_{gate,up,down}_exps tensors; host only."""
    v = [ctypes.c_int(0) for _ in range(5)]
    _check(load().sg_gguf_expert_dims(str(path).encode(), *[ctypes.byref(c) for c in v]))
    return tuple(c.value for c in v)


class ExpertPool:
    """Every MoE layer's experts of a GGUF v3 file resident in HBM, with the
    device pointer table [gate|up|down][layer][expert] (replaces
    Weights::load_expert_pool, weights.cpp:800-870, and the session's table
    upload, session.cpp:3596-3597)."""

    def __init__(self, path):
        h = ctypes.c_void_p(0)
        _check(load().sg_expert_pool_load_gguf(str(path).encode(), ctypes.byref(h)))
        self._h = h
        v = [ctypes.c_int(0) for _ in range(4)]
        _check(load().sg_expert_pool_dims(h, *[ctypes.byref(c) for c in v]))
        self.n_layers, self.n_expert, self.hidden, self.n_ff = (c.value for c in v)
        self.table = load().sg_expert_pool_table(h)
        self.device = torch.device("cuda", torch.cuda.current_device())

    def layer_tables(self, layer):
        """(tab_gate, tab_up, tab_down) of one layer: device arrays of n_expert pointers."""
        if not 0 <= layer < self.n_layers:
            raise SagerError(f"layer {layer} not in [0, {self.n_layers})")
        step = self.n_layers * self.n_expert * 8
        base = self.table + layer * self.n_expert * 8
        return tuple(DeviceAddress(base + m * step, self.device) for m in range(3))

    def close(self):
        if self._h:
            load().sg_expert_pool_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
