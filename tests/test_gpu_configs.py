"""GPU parity at the benchmark configurations' full workloads (BASELINE.json
configs 3, 4 and 5), through the C ABI against the pinned CPU oracle:

  config 3 - verify window: 4 tokens through the 256-expert layer with a
             shared expert, router logits N(0, 1.5), 8 seeded windows;
  config 4 - 40 x 256 experts (18.1 GB) resident behind the device pointer
             tables, Zipf(1.1) routing given by the caller, one token through
             every layer, then Q8_K and the full 248320 x 2048 Q4_K LM head;
  config 5 - a 2048-token prefill chunk, top-8 of 256 experts from U(0,1)
             logits, through the device plan and the int8-MFMA grouped
             contractions, every token compared.

The stage order matched is Session::moe_dispatch_device's
(session.cpp:2482-3030).  Every index and output is compared bit for bit;
the north star's max relative error 1e-4 is asserted on top."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from sager_amd import ops
from sager_amd.synth import q4k_random_dev, zipf_routes

pytestmark = pytest.mark.gpu
H, F, E, K = 2048, 512, 256, 8
BLOCKS = F * H // 256


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rel_err(got, ref):
    floor = 1e-3 * max(float(np.abs(ref).max()), 1e-30)
    return float((np.abs(got.astype(np.float64) - ref) / np.maximum(np.abs(ref), floor)).max())


def assert_fp32_parity(got, ref):
    assert rel_err(got, ref) <= 1e-4
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


def _tabs(pool, n):
    return [torch.tensor([pool[m, e].data_ptr() for e in range(n)], dtype=torch.int64,
                         device="cuda") for m in range(3)]


def _threads():
    return max(1, min(16, os.cpu_count() or 2) // 2)


def test_config3_verify_window_256_experts():
    gen = torch.Generator(device="cuda").manual_seed(33)
    pool = q4k_random_dev(3 * (E + 1) * BLOCKS, gen).view(3, E + 1, BLOCKS, 144)
    layer = ops.MoeLayer(*_tabs(pool, E), (pool[0, E], pool[1, E], pool[2, E]), hidden=H,
                         n_ff=F, n_expert=E, k=K, max_tokens=4)
    p = host(pool)
    g, u, d = ([p[m, e] for e in range(E)] for m in range(3))
    sh = (p[0, E], p[1, E], p[2, E])
    rng = np.random.default_rng(3)
    shared_ids = 0
    for win in range(8):
        x = rng.normal(0, 1, (4, H)).astype(np.float32)
        lg = rng.normal(0, 1.5, (4, E)).astype(np.float32)
        out, idx, w = layer.forward(torch.from_numpy(x).cuda(), torch.from_numpy(lg).cuda())
        ref, ri, rw = orc.moe_layer(g, u, d, sh, x, logits=lg, hidden=H, n_ff=F, k=K,
                                    n_threads=_threads())
        np.testing.assert_array_equal(host(idx)[:, :K], ri[:, :K])
        np.testing.assert_array_equal(host(w).view(np.uint32), rw.view(np.uint32))
        assert_fp32_parity(host(out), ref)
        shared_ids += 4 * K - len(set(ri[:, :K].ravel().tolist()))
    assert shared_ids > 0  # N(0, 1.5) logits: tokens of a window share experts


def test_config4_stack_and_lm_head():
    NL = 40
    gen = torch.Generator(device="cuda").manual_seed(44)
    pool = torch.empty((NL, 3, E, BLOCKS, 144), dtype=torch.uint8, device="cuda")
    for L in range(NL):
        q4k_random_dev(3 * E * BLOCKS, gen, out=pool[L].view(-1, 144))
    rng = np.random.default_rng(4)
    routes = zipf_routes(rng, NL, E, K)
    wr = rng.uniform(0.5, 1.5, (NL, K)).astype(np.float32)
    wr /= wr.sum(1, keepdims=True)
    idx = np.full((NL, 1, K + 1), -1, np.int32)
    idx[:, 0, :K] = routes
    w = np.zeros((NL, 1, K + 1), np.float32)
    w[:, 0, :K] = wr
    x = rng.normal(0, 1, (NL, 1, H)).astype(np.float32)
    idx_d, w_d, x_d = (torch.from_numpy(a).cuda() for a in (idx, w, x))
    acts = torch.empty((NL, 1, H), dtype=torch.float32, device="cuda")
    stack = [ops.MoeLayer(*_tabs(pool[L], E), None, hidden=H, n_ff=F, n_expert=E, k=K)
             for L in range(NL)]
    head_rows = 248320
    head = q4k_random_dev(head_rows * 8, gen)
    xq = ops.q8k_empty(1, H)
    y = torch.empty(head_rows, dtype=torch.float32, device="cuda")
    # one token through the 40 layers in order on one stream, then the head
    for L in range(NL):
        stack[L].forward(x_d[L], None, out=acts[L], idx=idx_d[L], weight=w_d[L])
    ops.quantize_q8_k(acts[NL - 1], out=xq)
    ops.gemv_q4_k_q8(head, xq, head_rows, H, y=y)
    acts_h = host(acts)
    for L in range(NL):
        gl, ul, dl = [None] * E, [None] * E, [None] * E
        for e in routes[L]:
            gl[e], ul[e], dl[e] = (host(pool[L, m, e]) for m in range(3))
        ref, _, _ = orc.moe_layer(gl, ul, dl, None, x[L], idx=idx[L], weight=w[L], hidden=H,
                                  n_ff=F, k=K)
        assert_fp32_parity(acts_h[L], ref)
    xq_h = host(xq)
    np.testing.assert_array_equal(xq_h, orc.quantize_q8_k(acts_h[NL - 1]))
    yref = orc.gemv(host(head), xq_h, head_rows, H)[0]
    assert_fp32_parity(host(y), yref)


def test_config5_prefill_all_tokens():
    T = 2048
    gen = torch.Generator(device="cuda").manual_seed(55)
    pool = q4k_random_dev(3 * E * BLOCKS, gen).view(3, E, BLOCKS, 144)
    pre = ops.MoePrefill(*_tabs(pool, E), None, hidden=H, n_ff=F, n_expert=E, k=K,
                         max_tokens=T)
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, (T, H)).astype(np.float32)
    lg = rng.uniform(0, 1, (T, E)).astype(np.float32)
    out, idx, w = pre.forward(torch.from_numpy(x).cuda(), torch.from_numpy(lg).cuda())
    p = host(pool)
    ref, ri, rw = orc.moe_layer([p[0, e] for e in range(E)], [p[1, e] for e in range(E)],
                                [p[2, e] for e in range(E)], None, x, logits=lg, hidden=H,
                                n_ff=F, k=K, prefill=True, n_threads=_threads())
    np.testing.assert_array_equal(host(idx)[:, :K], ri[:, :K])
    np.testing.assert_array_equal(host(w).view(np.uint32), rw.view(np.uint32))
    assert len(np.unique(ri[:, :K])) == E  # every expert is touched
    assert_fp32_parity(host(out), ref)
