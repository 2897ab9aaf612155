"""GPU parity of the boundary's fp16-buffer launchers, the fp32 x fp16 GEMV
(router / shared-gate logits), the shared expert's sigmoid gate inside the
fused decode layer and the prefill chunk, and the multi-workgroup dispatch
plan - each through the C ABI against the pinned CPU oracle.

Bar: bit-exact (fp16 outputs compared as bits; fp32 outputs as bits, with
the north star's max relative error 1e-4 asserted on top)."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from sager_amd import ops
from sager_amd.synth import q4k_random_np

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rel_err(got, ref):
    floor = 1e-3 * max(float(np.abs(ref).max()), 1e-30)
    return float((np.abs(got.astype(np.float64) - ref) / np.maximum(np.abs(ref), floor)).max())


def assert_fp32_parity(got, ref):
    assert rel_err(got, ref) <= 1e-4
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


def assert_f16_bits(got, ref32):
    np.testing.assert_array_equal(got.view(np.uint16), ref32.astype(np.float16).view(np.uint16))


# ---- fp16-buffer launchers ---------------------------------------------------

@pytest.mark.parametrize("rows,n_ff", [(1, 512), (9, 512), (3, 1000)])
def test_silu_mul_f16_bit_exact(rows, n_ff):
    rng = np.random.default_rng(rows * n_ff)
    g = (rng.normal(0, 3, (rows, n_ff))).astype(np.float16)
    u = (rng.normal(0, 3, (rows, n_ff))).astype(np.float16)
    g[0, :4] = [0.0, -0.0, 60000.0, -60000.0]
    got = host(ops.silu_mul_f16(dev(g), dev(u)))
    ref = orc.silu_mul(g.astype(np.float32), u.astype(np.float32))
    assert_f16_bits(got, ref)


@pytest.mark.parametrize("n_rows,n_used,hidden", [(1, 8, 2048), (4, 8, 2048), (3, 2, 300)])
def test_moe_combine_batched_f16_bit_exact(n_rows, n_used, hidden):
    rng = np.random.default_rng(n_rows + hidden)
    y = rng.normal(0, 1, (n_rows, n_used + 1, hidden)).astype(np.float16)
    w = rng.uniform(0, 1, (n_rows, n_used + 1)).astype(np.float32)
    res = rng.normal(0, 1, (n_rows, hidden)).astype(np.float16)
    out = dev(res)
    ops.moe_combine_batched_f16(out, dev(y), dev(w))
    ref = orc.moe_combine(y.astype(np.float32), w, res.astype(np.float32))
    assert_f16_bits(host(out), ref)


@pytest.mark.parametrize("n_rows,hidden", [(1, 2048), (5, 2048), (2, 700)])
def test_sigmoid_gate_scalar_f16_bit_exact(n_rows, hidden):
    rng = np.random.default_rng(hidden + n_rows)
    y = rng.normal(0, 2, (n_rows, hidden)).astype(np.float16)
    y[0, :3] = [-0.0, 0.0, 65504.0]
    g = rng.normal(0, 3, n_rows).astype(np.float32)
    g[0] = 0.0
    out = dev(y)
    if n_rows == 1:
        ops.sigmoid_gate_scalar_f16(out, dev(g))
    else:
        ops.sigmoid_gate_scalar_batched_f16(out, dev(g))
    ref = np.stack([y[r].astype(np.float32) * orc.sigmoid(g[r]) for r in range(n_rows)])
    assert_f16_bits(host(out), ref.astype(np.float32))


@pytest.mark.parametrize("n_rows,k,T", [(256, 2048, 1), (256, 2048, 16), (1, 2048, 3),
                                        (13, 100, 2)])
def test_gemv_f32_out_f16x_bit_exact(n_rows, k, T):
    rng = np.random.default_rng(n_rows * 7 + k + T)
    w = rng.normal(0, 0.05, (n_rows, k)).astype(np.float32)
    x = rng.normal(0, 1, (T, k)).astype(np.float16)
    got = host(ops.gemv_f32_out_f16x(dev(w), dev(x)))
    ref = orc.gemv_f32_lanes(w, x.astype(np.float32))
    assert_fp32_parity(got, ref)


def test_gemv_f32_out_f16x_order():
    """The cancellation vector that pins the oracle's lane order gives the
    same 1.0 on the GPU."""
    k = 128
    x = np.zeros((1, k), np.float32)
    x[0, [0, 32, 64, 96]] = [2.0**14, 1.0, 1.0, -2.0**14]  # fp16-representable
    w = np.ones((1, k), np.float32)
    w[0, [0, 96]] = 2.0**10                                  # lane 0: 2^24, 1, 1, -2^24
    x[0, [1, 17, 9]] = [2.0**15, -2.0**15, 1.0]
    w[0, [1, 17]] = 2.0**10                                  # lanes 1, 17: +-2^25
    ref = orc.gemv_f32_lanes(w, x)
    assert ref[0, 0] == np.float32(1.0)
    got = host(ops.gemv_f32_out_f16x(dev(w), dev(x.astype(np.float16))))
    assert got[0, 0] == np.float32(1.0)


@pytest.mark.parametrize("n_ptrs,rows_per,k", [(9, 512, 2048), (256, 2048, 2048), (3, 100, 512)])
def test_gemv_ptrs_f16out_bit_exact(n_ptrs, rows_per, k):
    rng = np.random.default_rng(n_ptrs + rows_per)
    mats = [q4k_random_np(rng, rows_per * k // 256) for _ in range(n_ptrs)]
    x = rng.normal(0, 1, k).astype(np.float32)
    xq = orc.quantize_q8_k(x)
    dm = [dev(m) for m in mats]
    ptrs = torch.tensor([m.data_ptr() for m in dm], dtype=torch.int64, device="cuda")
    got = host(ops.gemv_ptrs_q4_k_q8_f16out(ptrs, dev(xq), n_ptrs, rows_per, k))
    ref = np.concatenate([orc.gemv(m, xq, rows_per, k)[0] for m in mats])
    assert_f16_bits(got, ref)


@pytest.mark.parametrize("n_rows,k,T", [(512, 2048, 4), (2048, 512, 16), (37, 768, 1)])
def test_gemv_f16out_batched_bit_exact(n_rows, k, T):
    rng = np.random.default_rng(n_rows + k + T)
    w = q4k_random_np(rng, n_rows * k // 256)
    xq = orc.quantize_q8_k(rng.normal(0, 1, (T, k)).astype(np.float32))
    got = host(ops.gemv_q4_k_q8_f16out_batched(dev(w), dev(xq), n_rows, k, T))
    assert_f16_bits(got, orc.gemv(w, xq, n_rows, k, T))


# ---- the shared expert's sigmoid gate in the fused layer and the prefill ----

def _pool(rng, n, hidden, n_ff):
    g = [q4k_random_np(rng, n_ff * hidden // 256) for _ in range(n)]
    u = [q4k_random_np(rng, n_ff * hidden // 256) for _ in range(n)]
    d = [q4k_random_np(rng, hidden * n_ff // 256) for _ in range(n)]
    return g, u, d


def _tables(mats):
    t = [dev(m) if m is not None else None for m in mats]
    ptrs = torch.tensor([m.data_ptr() if m is not None else 0 for m in t], dtype=torch.int64,
                        device="cuda")
    return ptrs, t


def _build(cls, g, u, d, shared, gate_w, hidden, n_ff, k, max_tokens):
    tg, kg = _tables(g)
    tu, ku = _tables(u)
    td, kd = _tables(d)
    sh = tuple(dev(m) for m in shared) if shared is not None else None
    layer = cls(tg, tu, td, sh, hidden=hidden, n_ff=n_ff, n_expert=len(g), k=k,
                max_tokens=max_tokens, shared_w=0.75,
                shared_gate_w=dev(gate_w) if gate_w is not None else None)
    layer._keep = (kg, ku, kd)
    return layer


@pytest.mark.parametrize("T,routed", [(1, False), (4, False), (16, False), (3, True)])
def test_moe_layer_shared_gate(T, routed):
    """hidden 2048, n_ff 512, top-8 of 32 experts + a gated shared expert."""
    rng = np.random.default_rng(900 + T)
    H, F, E, K = 2048, 512, 32, 8
    g, u, d = _pool(rng, E + 1, H, F)
    shared = (g.pop(), u.pop(), d.pop())
    gw = rng.normal(0, 0.03, H).astype(np.float32)
    x = rng.normal(0, 1, (T, H)).astype(np.float32)
    res = rng.normal(0, 1, (T, H)).astype(np.float32)
    layer = _build(ops.MoeLayer, g, u, d, shared, gw, H, F, K, T)
    if routed:
        lg = None
        idx = np.stack([np.append(rng.choice(E, K, replace=False), -1) for _ in range(T)])
        idx = idx.astype(np.int32)
        w = rng.uniform(0.1, 1, (T, K + 1)).astype(np.float32)
        w[:, K] = 0.75
        out, _, _ = layer.forward(dev(x), None, residual=dev(res), idx=dev(idx), weight=dev(w))
        ref, _, _ = orc.moe_layer(g, u, d, shared, x, idx=idx, weight=w, residual=res, hidden=H,
                                  n_ff=F, k=K, shared_gate_w=gw)
    else:
        lg = rng.normal(0, 1, (T, E)).astype(np.float32)
        out, idx, w = layer.forward(dev(x), dev(lg), residual=dev(res))
        ref, ri, rw = orc.moe_layer(g, u, d, shared, x, logits=lg, residual=res, hidden=H,
                                    n_ff=F, k=K, shared_w=0.75, shared_gate_w=gw)
        np.testing.assert_array_equal(host(idx)[:, :K], ri[:, :K])
        np.testing.assert_array_equal(host(w).view(np.uint32), rw.view(np.uint32))
    assert_fp32_parity(host(out), ref)
    # the same layer without the gate is a different, also exact, result
    layer.shared_gate_w = None
    if routed:
        out0, _, _ = layer.forward(dev(x), None, residual=dev(res), idx=dev(idx), weight=dev(w))
        ref0, _, _ = orc.moe_layer(g, u, d, shared, x, idx=idx, weight=w, residual=res,
                                   hidden=H, n_ff=F, k=K)
    else:
        out0, _, _ = layer.forward(dev(x), dev(lg), residual=dev(res))
        ref0, _, _ = orc.moe_layer(g, u, d, shared, x, logits=lg, residual=res, hidden=H,
                                   n_ff=F, k=K, shared_w=0.75)
    assert_fp32_parity(host(out0), ref0)
    assert not np.array_equal(ref0, ref)


def test_moe_layer_gate_without_shared_expert_is_ignored():
    rng = np.random.default_rng(77)
    H, F, E, K, T = 1024, 512, 16, 4, 2
    g, u, d = _pool(rng, E, H, F)
    gw = rng.normal(0, 0.03, H).astype(np.float32)
    x = rng.normal(0, 1, (T, H)).astype(np.float32)
    lg = rng.normal(0, 1, (T, E)).astype(np.float32)
    layer = _build(ops.MoeLayer, g, u, d, None, gw, H, F, K, T)
    out, _, _ = layer.forward(dev(x), dev(lg))
    ref, _, _ = orc.moe_layer(g, u, d, None, x, logits=lg, hidden=H, n_ff=F, k=K)
    assert_fp32_parity(host(out), ref)


@pytest.mark.parametrize("T", [1, 64, 200])
def test_moe_prefill_shared_gate(T):
    rng = np.random.default_rng(950 + T)
    H, F, E, K = 2048, 512, 32, 8
    g, u, d = _pool(rng, E + 1, H, F)
    shared = (g.pop(), u.pop(), d.pop())
    gw = rng.normal(0, 0.03, H).astype(np.float32)
    x = rng.normal(0, 1, (T, H)).astype(np.float32)
    lg = rng.normal(0, 1, (T, E)).astype(np.float32)
    res = rng.normal(0, 1, (T, H)).astype(np.float32)
    layer = _build(ops.MoePrefill, g, u, d, shared, gw, H, F, K, max(T, 16))
    out, idx, w = layer.forward(dev(x), dev(lg), residual=dev(res))
    ref, ri, rw = orc.moe_layer(g, u, d, shared, x, logits=lg, residual=res, hidden=H, n_ff=F,
                                k=K, shared_w=0.75, shared_gate_w=gw, prefill=True, n_threads=8)
    np.testing.assert_array_equal(host(idx)[:, :K], ri[:, :K])
    assert_fp32_parity(host(out), ref)


# ---- the multi-workgroup dispatch plan (what sg_moe_prefill builds) --------

def _routes(rng, n_rows, E, k):
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(n_rows)]).astype(np.int32)
    return np.concatenate([idx, np.full((n_rows, 1), -1, np.int32)], axis=1)


def _check_plan(idx, w, E, k, tok_per, shared_tail=0):
    ref = orc.dispatch_scan(idx, w, k, E, tok_per=tok_per)
    wd = dev(w)
    got = ops.moe_dispatch_plan(dev(idx), wd, E, k, tok_per=tok_per, shared_tail=shared_tail)
    R = int(ref["meta"][0])
    np.testing.assert_array_equal(host(got["meta"])[:3], ref["meta"][:3])
    off = host(got["off"])
    np.testing.assert_array_equal(off[:E + 1], ref["off"])
    assert off[E + 1] == off[E] + shared_tail
    np.testing.assert_array_equal(host(got["toff"])[:E + 1], ref["toff"])
    np.testing.assert_array_equal(host(got["gslot"]), ref["gslot"])
    grows = host(got["grows"])
    np.testing.assert_array_equal(grows[:R], ref["grows"][:R])
    np.testing.assert_array_equal(grows[R:R + shared_tail], np.arange(shared_tail))
    np.testing.assert_array_equal(host(wd), ref["weight"])
    # the tile list: every tile of every group in expert order, then the shared one's
    tiles = host(got["tiles"])
    hist = np.diff(ref["off"])
    want = [(e << 16) | j for e in range(E) for j in range((hist[e] + tok_per - 1) // tok_per)]
    want += [(E << 16) | j for j in range((shared_tail + tok_per - 1) // tok_per)]
    assert tiles[0] == len(want)
    np.testing.assert_array_equal(tiles[1:1 + len(want)], want)


@pytest.mark.parametrize("n_rows,E,k,shared", [(2048, 256, 8, 0), (2048, 256, 8, 1),
                                               (4096, 256, 8, 0), (300, 1024, 4, 1),
                                               (33, 32, 8, 0), (9000, 64, 4, 1),
                                               (60000, 16, 2, 0)])
def test_dispatch_plan_matches_oracle(n_rows, E, k, shared):
    """T=2048, E=256 is config 5's plan; T=4096, E=256 takes the global-memory
    bitmap path (n_w * E beyond the LDS copy); invalid ids sit past token 32.
    9000 rows take two bitmap words per expert and workgroup (byte counts),
    60000 rows eight (counts in words: 32 * 8 > 255)."""
    rng = np.random.default_rng(n_rows * 3 + E + shared)
    idx = _routes(rng, n_rows, E, k)
    idx[3, 1] = E + 5
    idx[min(40, n_rows - 1), 0] = -2
    idx[n_rows - 1, k - 1] = E
    w = rng.uniform(0, 1, (n_rows, k + 1)).astype(np.float32)
    _check_plan(idx, w, E, k, 64, n_rows if shared else 0)


@pytest.mark.parametrize("n_rows", [70, 2048])
def test_dispatch_plan_duplicate_ids_serial(n_rows):
    """Rows that name one expert twice (caller routing), beyond token 32 and
    across several scan workgroups: serial placement in (token, slot) order."""
    rng = np.random.default_rng(n_rows + 5)
    E, k = 64, 4
    idx = _routes(rng, n_rows, E, k)
    idx[40, 1] = idx[40, 0]
    idx[n_rows - 2, 3] = idx[n_rows - 2, 2]
    idx[50, 2] = 999
    w = rng.uniform(0, 1, (n_rows, k + 1)).astype(np.float32)
    _check_plan(idx, w, E, k, 16)


# ---- the fp16-buffer entry points: argument checks -------------------------

def test_layer_f16_argument_errors():
    rng = np.random.default_rng(7)
    H, F, E, K = 512, 256, 8, 2
    g, u, d = _pool(rng, E + 1, H, F)
    shared = (g.pop(), u.pop(), d.pop())
    gw = rng.normal(0, 0.03, H).astype(np.float32)
    layer = _build(ops.MoeLayer, g, u, d, shared, gw, H, F, K, 1)
    xn = dev(rng.normal(0, 0.02, (1, H)).astype(np.float16))  # finite fp16 outputs
    xq = ops.quantize_q8_k(xn)
    lg = dev(rng.normal(0, 1, (1, E)).astype(np.float32))
    with pytest.raises(ops.SagerError, match="shared gate needs xn"):
        layer.forward_f16(None, xq, lg)
    with pytest.raises(ops.SagerError, match="must be torch.float16"):
        layer.forward_f16(xn.float(), None, lg)
    # with the gate off, the Q8_K alone is enough, and equals xn alone
    layer.shared_gate_w = None
    o1, _, _ = layer.forward_f16(None, xq, lg)
    o2, _, _ = layer.forward_f16(xn, None, lg)
    assert torch.isfinite(o1).all()
    np.testing.assert_array_equal(host(o1).view(np.uint16), host(o2).view(np.uint16))
