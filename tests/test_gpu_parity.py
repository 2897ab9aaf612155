"""GPU parity: libsager_hip.so (through its C ABI, via sager_amd.ops) against
the pinned CPU oracle and the reference's golden vectors, on the same seeded
inputs.

Bar: Q8_K blocks, int32 sub-block dots, router indices - bit-exact.  fp32
outputs (GEMV, SiLU, combine, expert/layer outputs) - the kernels replay the
oracle's operation order, so they are checked bit-exact too; the tolerance
of the north star (max relative error 1e-4, denominator floored at
1e-3 * max|ref|) is asserted on top as the contract.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from sager_amd import ops
from sager_amd.synth import q4k_random_np

pytestmark = pytest.mark.gpu
GOLD = "tests/golden/q4k_golden.npz"


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


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)


# ---- Q8_K ------------------------------------------------------------------

def test_quantize_golden(gold):
    got = host(ops.quantize_q8_k(dev(gold["q8_x"])))
    np.testing.assert_array_equal(got, gold["q8_out"])


def test_quantize_fp16_input():
    rng = np.random.default_rng(21)
    x16 = rng.normal(0, 0.6, (5, 2048)).astype(np.float16)
    got = host(ops.quantize_q8_k(dev(x16)))
    np.testing.assert_array_equal(got, orc.quantize_q8_k(x16.astype(np.float32)))


@pytest.mark.parametrize("rows,n", [(1, 256), (3, 512), (16, 2048), (1, 16384)])
def test_quantize_shapes(rows, n):
    rng = np.random.default_rng(rows * n)
    x = (rng.normal(0, 1, (rows, n)) * rng.uniform(1e-3, 1e3, (rows, 1))).astype(np.float32)
    x[0, :256:7] = 0.0
    np.testing.assert_array_equal(host(ops.quantize_q8_k(dev(x))), orc.quantize_q8_k(x))


# ---- sub-block dots and GEMV ----------------------------------------------

def _case(rng, n_rows, k):
    w = q4k_random_np(rng, n_rows * k // 256)
    x = rng.normal(0, 1, k).astype(np.float32)
    return w, orc.quantize_q8_k(x)


@pytest.mark.parametrize("n_rows,k", [(128, 2048), (2048, 512), (37, 768), (5, 256),
                                      (9, 16384)])
def test_subblock_dots_bit_exact(n_rows, k):
    rng = np.random.default_rng(n_rows + k)
    w, xq = _case(rng, n_rows, k)
    got = host(ops.subblock_dots(dev(w), dev(xq), n_rows, k))
    np.testing.assert_array_equal(got, orc.subblock_dots(w, xq[0], n_rows, k))


@pytest.mark.parametrize("case", ["gemv_a", "gemv_b", "gemv_c"])
def test_gemv_golden(gold, case):
    n_rows, k = (int(v) for v in gold[case + "_shape"])
    w, xq = dev(gold[case + "_w"]), gold[case + "_xq"]
    for t in range(xq.shape[0]):
        y = host(ops.gemv_q4_k_q8(w, dev(xq[t]), n_rows, k))
        assert_fp32_parity(y, gold[case + "_y"][t])


@pytest.mark.parametrize("n_rows,k", [(2048, 2048), (512, 2048), (2048, 512), (1001, 768),
                                      (3, 256), (70, 16384), (4096, 4096), (777, 2304),
                                      (32768, 2048), (32769, 2048)])
def test_gemv_shapes(n_rows, k):
    rng = np.random.default_rng(7 * n_rows + k)
    w, xq = _case(rng, n_rows, k)
    y = host(ops.gemv_q4_k_q8(dev(w), dev(xq), n_rows, k))
    assert_fp32_parity(y, orc.gemv(w, xq, n_rows, k)[0])


@pytest.mark.parametrize("n_rows,k", [(65536, 2048), (20000, 4096)])
def test_gemv_many_groups_per_wave(n_rows, k):
    """More row groups than waves in the grid: every wave loops over several
    groups through its LDS buffer (the LM-head regime).  Bit-identical across
    runs and within the fp32 bar against the oracle."""
    rng = np.random.default_rng(n_rows + 3 * k)
    w, xq = _case(rng, n_rows, k)
    wd, xd = dev(w), dev(xq)
    ys = [host(ops.gemv_q4_k_q8(wd, xd, n_rows, k)) for _ in range(3)]
    for y in ys[1:]:
        np.testing.assert_array_equal(y, ys[0])
    assert_fp32_parity(ys[0], orc.gemv(w, xq, n_rows, k)[0])


def test_gemv_ptrs_many_groups_per_wave():
    rng = np.random.default_rng(32)
    n_ptrs, rows_per, k = 40, 2048, 2048
    mats = [dev(q4k_random_np(rng, rows_per * k // 256)) for _ in range(n_ptrs)]
    ptrs = torch.tensor([m.data_ptr() for m in mats], dtype=torch.int64, device="cuda")
    xq = orc.quantize_q8_k(rng.normal(0, 1, k).astype(np.float32))
    ys = [host(ops.gemv_ptrs_q4_k_q8(ptrs, dev(xq), n_ptrs, rows_per, k)) for _ in range(2)]
    np.testing.assert_array_equal(ys[1], ys[0])
    ref = np.concatenate([orc.gemv(m.cpu().numpy(), xq, rows_per, k)[0] for m in mats])
    assert_fp32_parity(ys[0], ref)


@pytest.mark.parametrize("n_rows,k", [(64, 2048), (1, 256), (7, 768), (33, 4096),
                                      (3, 8192), (50000, 2048), (9001, 1280)])
def test_gemv_q6k_bit_exact(n_rows, k):
    """Q6_K head GEMV against the oracle's restatement of the reference
    kernel's order: bit-identical, including shapes where every wave loops
    over several row groups and rows that start off 16-B boundaries."""
    from sager_amd.synth import q6k_random_np
    rng = np.random.default_rng(n_rows * 7 + k)
    w6 = q6k_random_np(rng, n_rows * k // 256)
    xq = orc.quantize_q8_k(rng.normal(0, 1, k).astype(np.float32))
    wd = dev(w6)
    y = host(ops.gemv_q6_k_q8(wd, dev(xq), n_rows, k))
    np.testing.assert_array_equal(y, orc.gemv_q6k(w6, xq[0], n_rows, k))
    np.testing.assert_array_equal(host(ops.gemv_q6_k_q8(wd, dev(xq), n_rows, k)), y)


@pytest.mark.parametrize("rows,k", [((4096, 512, 512), 2048), ((8192, 64), 2048),
                                    ((33, 7, 250), 768), ((60000, 4000, 1), 2048)])
def test_gemv_nm_f16out(rows, k):
    """gemv2m / gemv3m: each projection equals the fp32 GEMV (AVX2 order)
    rounded to fp16 (nearest even), including segments that start inside a
    row group and a 1-row segment."""
    rng = np.random.default_rng(sum(rows) + k)
    ws = [q4k_random_np(rng, r * k // 256) for r in rows]
    xq = orc.quantize_q8_k(rng.normal(0, 1, k).astype(np.float32))
    ys = ops.gemv_nm_q4_k_q8_f16out([dev(w) for w in ws], dev(xq), list(rows), k)
    for w, r, y in zip(ws, rows, ys):
        ref = orc.gemv(w, xq, r, k)[0].astype(np.float16)
        np.testing.assert_array_equal(host(y).view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("n_rows,k", [(2048, 4096), (777, 512), (70000, 2048)])
def test_gemv_f16out_and_resadd(n_rows, k):
    """fp16 GEMV and the fused residual add: res = f16(f32(res) + f32(f16(y)))."""
    rng = np.random.default_rng(n_rows + 5 * k)
    w = q4k_random_np(rng, n_rows * k // 256)
    xq = orc.quantize_q8_k(rng.normal(0, 1, k).astype(np.float32))
    ref = orc.gemv(w, xq, n_rows, k)[0].astype(np.float16)
    y = ops.gemv_q4_k_q8_f16out(dev(w), dev(xq), n_rows, k)
    np.testing.assert_array_equal(host(y).view(np.uint16), ref.view(np.uint16))
    res = (rng.normal(0, 4, n_rows)).astype(np.float16)
    res_d = torch.from_numpy(res.copy()).cuda()
    y2 = ops.gemv_q4_k_q8_f16out_resadd(dev(w), dev(xq), res_d, n_rows, k)
    np.testing.assert_array_equal(host(y2).view(np.uint16), ref.view(np.uint16))
    want = (res.astype(np.float32) + ref.astype(np.float32)).astype(np.float16)
    np.testing.assert_array_equal(res_d.cpu().numpy().view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("n_tokens", [1, 2, 4, 5, 16])
def test_gemv_batched(n_tokens):
    rng = np.random.default_rng(100 + n_tokens)
    n_rows, k = 777, 2048
    w = q4k_random_np(rng, n_rows * k // 256)
    xq = orc.quantize_q8_k(rng.normal(0, 1, (n_tokens, k)).astype(np.float32))
    y = host(ops.gemv_q4_k_q8_batched(dev(w), dev(xq), n_rows, k, n_tokens))
    assert_fp32_parity(y, orc.gemv(w, xq, n_rows, k, n_tokens))


def test_gemv_ptrs():
    rng = np.random.default_rng(31)
    n_ptrs, rows_per, k = 9, 512, 2048
    mats = [dev(q4k_random_np(rng, rows_per * k // 256)) for _ in range(n_ptrs)]
    ptrs = torch.tensor([m.data_ptr() for m in mats], dtype=torch.int64, device="cuda")
    xq = orc.quantize_q8_k(rng.normal(0, 1, k).astype(np.float32))
    y = host(ops.gemv_ptrs_q4_k_q8(ptrs, dev(xq), n_ptrs, rows_per, k))
    ref = np.concatenate([orc.gemv(m.cpu().numpy(), xq, rows_per, k)[0] for m in mats])
    assert_fp32_parity(y, ref)


# ---- router, SiLU, combine ---------------------------------------------------

@pytest.mark.parametrize("n_rows,n_expert,k,sigma", [(1, 256, 8, 1.0), (4, 256, 8, 1.5),
                                                     (64, 256, 8, 1.0), (3, 1024, 32, 2.0),
                                                     (2, 60, 7, 1.0)])
def test_router_bit_exact(n_rows, n_expert, k, sigma):
    rng = np.random.default_rng(n_rows * 1000 + n_expert)
    lg = rng.normal(0, sigma, (n_rows, n_expert)).astype(np.float32)
    idx, w = ops.router_topk_batched(dev(lg), k, shared_w=1.0)
    ri, rw = orc.router_topk(lg, k, 1.0)
    np.testing.assert_array_equal(host(idx)[:, :k], ri[:, :k])
    np.testing.assert_array_equal(host(w).view(np.uint32), rw.view(np.uint32))


def test_router_ties_nan_degenerate():
    lg = np.zeros((4, 256), np.float32)
    lg[0, [7, 3, 200, 100]] = 2.0
    lg[1, :] = 0.25                       # all equal: lower index wins every round
    lg[2, 9] = np.nan                     # NaN poisons the normalizer
    lg[3] = np.random.default_rng(0).normal(0, 1, 256)
    lg[3, 17] = lg[3, 200] = lg[3].max() + 1.0   # exact duplicate at the top
    idx, w = ops.router_topk_batched(dev(lg), 8, shared_w=0.5)
    ri, rw = orc.router_topk(lg, 8, 0.5)
    np.testing.assert_array_equal(host(idx)[:, :8], ri[:, :8])
    np.testing.assert_array_equal(host(w).view(np.uint32), rw.view(np.uint32))
    assert list(ri[3, :2]) == [17, 200]


def test_router_near_ties_model_shape():
    """256 experts, top-8 (the shape whose rounds run on the exps beside the
    normalizer): rows where two logits are equal or one or two ulps apart,
    at the top-k boundary and inside it, with the larger one at the higher
    index - their exps differ by an ulp or two and their probabilities may
    round equal, when the reference's lower-index rule decides the order."""
    rng = np.random.default_rng(99)
    rows = []
    for n in range(96):
        r = rng.normal(0, 1, 256).astype(np.float32)
        o = np.argsort(-r, kind="stable")
        pos = [0, 3, 6, 7, 8, 2][n % 6]
        a, b = o[pos], o[pos + 1]
        lo, hi = (a, b) if a < b else (b, a)  # hi: the higher index
        base = r[lo]
        r[hi] = base
        for _ in range(n % 3):  # 0, 1 or 2 ulps above, at the higher index
            r[hi] = np.nextafter(r[hi], np.float32(np.inf))
        rows.append(r)
    lg = np.stack(rows)
    idx, w = ops.router_topk_batched(dev(lg), 8, shared_w=1.0)
    ri, rw = orc.router_topk(lg, 8, 1.0)
    np.testing.assert_array_equal(host(idx)[:, :8], ri[:, :8])
    np.testing.assert_array_equal(host(w).view(np.uint32), rw.view(np.uint32))


def test_silu_bit_exact():
    rng = np.random.default_rng(12)
    g = (rng.normal(0, 4, 100000)).astype(np.float32)
    g[:6] = [0.0, -0.0, 88.0, -88.0, -104.0, 20.0]
    u = rng.normal(0, 1, g.size).astype(np.float32)
    h = host(ops.silu_mul(dev(g), dev(u)))
    np.testing.assert_array_equal(h.view(np.uint32), orc.silu_mul(g, u).view(np.uint32))


def test_combine_bit_exact():
    rng = np.random.default_rng(13)
    y = rng.normal(0, 1, (4, 9, 2048)).astype(np.float32)
    w = rng.uniform(0, 1, (4, 9)).astype(np.float32)
    res = rng.normal(0, 1, (4, 2048)).astype(np.float32)
    out = host(ops.moe_combine_batched(dev(y), dev(w), dev(res)))
    assert_fp32_parity(out, orc.moe_combine(y, w, res))
    out0 = host(ops.moe_combine_batched(dev(y), dev(w)))
    assert_fp32_parity(out0, orc.moe_combine(y, w))


# ---- fused MoE layer ---------------------------------------------------------

def _expert_pool(rng, n, hidden, n_ff):
    g = [q4k_random_np(rng, n_ff * hidden // 256) for _ in range(n)]
    u = [q4k_random_np(rng, n_ff * hidden // 256) for _ in range(n)]
    d = [q4k_random_np(rng, hidden * n_ff // 256) for _ in range(n)]
    return g, u, d


def _tables(mats):
    t = [dev(m) if m is not None else None for m in mats]
    ptrs = torch.tensor([m.data_ptr() if m is not None else 0 for m in t], dtype=torch.int64,
                        device="cuda")
    return ptrs, t


def _layer(g, u, d, shared, hidden, n_ff, k, max_tokens):
    tg, kg = _tables(g)
    tu, ku = _tables(u)
    td, kd = _tables(d)
    sh = tuple(dev(m) for m in shared) if shared is not None else None
    layer = ops.MoeLayer(tg, tu, td, sh, hidden=hidden, n_ff=n_ff, n_expert=len(g), k=k,
                         max_tokens=max_tokens)
    layer._keep = (kg, ku, kd)
    return layer


@pytest.mark.parametrize("T,sigma", [(1, 1.0), (4, 1.5), (16, 1.0)])
def test_moe_layer_small_pool(T, sigma):
    """hidden 2048, n_ff 512, top-8 of 32 experts + shared expert."""
    rng = np.random.default_rng(50 + T)
    H, F, E, K = 2048, 512, 32, 8
    g, u, d = _expert_pool(rng, E + 1, H, F)
    shared = (g.pop(), u.pop(), d.pop())
    x = rng.normal(0, 1, (T, H)).astype(np.float32)
    lg = rng.normal(0, sigma, (T, E)).astype(np.float32)
    res = rng.normal(0, 1, (T, H)).astype(np.float32)
    layer = _layer(g, u, d, shared, H, F, K, T)
    out, idx, w = layer.forward(dev(x), dev(lg), residual=dev(res))
    ref, ri, rw = orc.moe_layer(g, u, d, shared, x, logits=lg, residual=res, hidden=H, n_ff=F,
                                k=K)
    np.testing.assert_array_equal(host(idx)[:, :K], ri[:, :K])
    np.testing.assert_array_equal(host(w).view(np.uint32), rw.view(np.uint32))
    assert_fp32_parity(host(out), ref)
    # a second call on the same workspace gives the same bits (counters reset)
    out2, _, _ = layer.forward(dev(x), dev(lg), residual=dev(res))
    np.testing.assert_array_equal(host(out2), host(out))


def test_moe_layer_workspace_shared_by_sizes():
    """One workspace, calls of 4, 1, 3, 1 and 4 tokens in a row, the last
    split into its two launches: every call matches the oracle."""
    rng = np.random.default_rng(4242)
    H, F, E, K = 1024, 512, 32, 8
    g, u, d = _expert_pool(rng, E + 1, H, F)
    shared = (g.pop(), u.pop(), d.pop())
    layer = _layer(g, u, d, shared, H, F, K, 4)
    for T, stages in [(4, 3), (1, 3), (3, 3), (1, 3), (4, None)]:
        x = rng.normal(0, 1, (T, H)).astype(np.float32)
        lg = rng.normal(0, 1.5, (T, E)).astype(np.float32)
        out, idx, w = layer.forward(dev(x), dev(lg))
        ref, ri, rw = orc.moe_layer(g, u, d, shared, x, logits=lg, hidden=H, n_ff=F, k=K)
        np.testing.assert_array_equal(host(idx)[:, :K], ri[:, :K])
        np.testing.assert_array_equal(host(out).view(np.uint32), ref.view(np.uint32))


def test_moe_layer_config2_full_pool():
    """Config 2: 256 experts x (gate, up [512x2048], down [2048x512]) resident,
    top-8 from N(0,1) logits, shared expert, residual 0."""
    H, F, E, K = 2048, 512, 256, 8
    gen = torch.Generator(device="cuda").manual_seed(2)
    from sager_amd.synth import q4k_random_dev
    blocks = F * H // 256
    pool = q4k_random_dev(3 * (E + 1) * blocks, gen).view(3, E + 1, blocks, 144)
    tg = torch.tensor([pool[0, e].data_ptr() for e in range(E)], dtype=torch.int64,
                      device="cuda")
    tu = torch.tensor([pool[1, e].data_ptr() for e in range(E)], dtype=torch.int64,
                      device="cuda")
    td = torch.tensor([pool[2, e].data_ptr() for e in range(E)], dtype=torch.int64,
                      device="cuda")
    layer = ops.MoeLayer(tg, tu, td, (pool[0, E], pool[1, E], pool[2, E]), hidden=H, n_ff=F,
                         n_expert=E, k=K, max_tokens=1)
    rng = np.random.default_rng(3)
    for step in range(3):
        x = rng.normal(0, 1, (1, H)).astype(np.float32)
        lg = rng.normal(0, 1, (1, E)).astype(np.float32)
        out, idx, w = layer.forward(dev(x), dev(lg))
        ri, rw = orc.router_topk(lg, K)
        np.testing.assert_array_equal(host(idx)[0, :K], ri[0, :K])
        used = list(ri[0, :K])
        gh = [None] * E
        uh = [None] * E
        dh = [None] * E
        for e in used:
            gh[e], uh[e], dh[e] = (pool[m, e].cpu().numpy() for m in range(3))
        sh = tuple(pool[m, E].cpu().numpy() for m in range(3))
        ref, _, _ = orc.moe_layer(gh, uh, dh, sh, x, logits=lg, hidden=H, n_ff=F, k=K)
        assert_fp32_parity(host(out), ref)


def test_moe_layer_routed_edge_cases():
    """Caller-supplied routing (logits=None) with an out-of-range id, an absent
    expert (null table entry), no shared expert, residual aliasing out."""
    rng = np.random.default_rng(77)
    H, F, E, K, T = 512, 256, 8, 2, 3
    g, u, d = _expert_pool(rng, E, H, F)
    g[3] = None
    x = rng.normal(0, 1, (T, H)).astype(np.float32)
    idx = np.array([[1, 99, -1], [2, 3, -1], [3, 5, -1]], np.int32)
    w = np.array([[0.6, 0.4, 1.0], [0.7, 0.3, 1.0], [0.5, 0.5, 1.0]], np.float32)
    res = rng.normal(0, 1, (T, H)).astype(np.float32)
    layer = _layer(g, u, d, None, H, F, K, T)
    io = dev(res)
    wd = dev(w)
    out, _, wgt = layer.forward(dev(x), None, residual=io, out=io, idx=dev(idx), weight=wd)
    ref, _, rw = orc.moe_layer(g, u, d, None, x, idx=idx, weight=w, residual=res, hidden=H,
                               n_ff=F, k=K)
    np.testing.assert_array_equal(host(wgt), rw)
    assert_fp32_parity(host(out), ref)


@pytest.mark.parametrize("T,K", [(2, 4), (8, 8)])
def test_moe_layer_routed_duplicate_ids(T, K):
    """Caller routing that repeats an id inside a row and across rows (the
    plan's one-wave sort for up to 64 routes, and the general build past
    it): each (token, slot) is its own entry of its expert's group."""
    rng = np.random.default_rng(3100 + T)
    H, F, E = 2048, 512, K  # (the layer takes at least k experts)
    g, u, d = _expert_pool(rng, E + 1, H, F)
    shared = (g.pop(), u.pop(), d.pop())
    x = rng.normal(0, 1, (T, H)).astype(np.float32)
    idx = np.full((T, K + 1), -1, np.int32)
    idx[:, :K] = rng.integers(0, 3, (T, K))        # three experts: heavy repetition
    idx[0, :K] = 1                                   # one row entirely on one expert
    w = rng.uniform(0.05, 1.0, (T, K + 1)).astype(np.float32)
    w[:, K] = 1.0
    layer = _layer(g, u, d, shared, H, F, K, T)
    out, _, wgt = layer.forward(dev(x), None, idx=dev(idx), weight=dev(w))
    ref, _, rw = orc.moe_layer(g, u, d, shared, x, idx=idx, weight=w, hidden=H, n_ff=F, k=K)
    np.testing.assert_array_equal(host(wgt), rw)
    np.testing.assert_array_equal(host(out).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("T", [2, 3, 4, 5])
def test_moe_layer_routing_edge_cases(T):
    """Fused routing against the oracle where the logit order and the
    probability order can part: boundary ties, all-equal rows, a NaN row
    (degenerate selection), -inf logits; T = 2..5 covers the 2-wave teams,
    an idle team and two routing passes."""
    rng = np.random.default_rng(900 + T)
    H, F, E, K = 512, 256, 32, 8
    g, u, d = _expert_pool(rng, E + 1, H, F)
    shared = (g.pop(), u.pop(), d.pop())
    x = rng.normal(0, 1, (T, H)).astype(np.float32)
    lg = rng.normal(0, 1, (T, E)).astype(np.float32)
    lg[0, [4, 9, 20]] = lg[0].max() + 0.5          # 3-way tie at the top
    o = np.argsort(-lg[0], kind="stable")
    lg[0, o[8]] = lg[0, o[7]]                        # tie across the k boundary
    lg[1] = 0.125                                    # all equal
    if T > 2:
        lg[2, 7] = np.nan                            # degenerate row
    if T > 3:
        lg[3, :5] = -np.inf
    layer = _layer(g, u, d, shared, H, F, K, T)
    out, idx, w = layer.forward(dev(x), dev(lg))
    ref, ri, rw = orc.moe_layer(g, u, d, shared, x, logits=lg, hidden=H, n_ff=F, k=K)
    np.testing.assert_array_equal(host(idx)[:, :K], ri[:, :K])
    np.testing.assert_array_equal(host(w).view(np.uint32), rw.view(np.uint32))
    np.testing.assert_array_equal(host(out).view(np.uint32), ref.view(np.uint32))


def _t1_edge_rows(E, K):
    rng = np.random.default_rng(4711)
    rows = []
    base = rng.normal(0, 1, E).astype(np.float32)
    o = np.argsort(-base, kind="stable")
    r = base.copy(); r[o[3]] = r[o[2]]; rows.append(r)              # interior tie
    r = base.copy(); r[o[K]] = r[o[K - 1]]; rows.append(r)          # tie across the boundary
    r = np.zeros(E, np.float32) - 3.0
    r[[2, 5, 11]] = [0.0, -0.0, 0.0]; r[[1, 30]] = [-0.0, 0.0]      # signed zeros at the top
    rows.append(r)
    r = base.copy(); r[[0, 6]] = -np.inf; rows.append(r)            # -inf: not all finite
    r = base.copy(); r[9] = np.nan; rows.append(r)                  # degenerate
    r = base.copy(); r[o[1]] = np.nextafter(r[o[0]], np.float32(-9.0)); rows.append(r)  # 1 ulp apart
    r = base.copy(); r[o[K]] = r[o[K - 1]] - np.float32(2e-6); rows.append(r)   # near the margin
    r = (base * 40.0).astype(np.float32); rows.append(r)           # tiny tail probabilities
    return rows


def test_moe_layer_t1_routing_edge_cases():
    """One token: rows where the logit-order shortcut of the compute
    workgroups must hold or must hand over to the exact routing - ties inside
    and across the top-k boundary, signed zeros, -inf, NaN, logits one ulp
    apart, a gap near the shortcut's margin, very small probabilities."""
    H, F, E, K = 512, 256, 64, 8
    rng = np.random.default_rng(61)
    g, u, d = _expert_pool(rng, E + 1, H, F)
    shared = (g.pop(), u.pop(), d.pop())
    layer = _layer(g, u, d, shared, H, F, K, 1)
    x = rng.normal(0, 1, (1, H)).astype(np.float32)
    for lg in _t1_edge_rows(E, K):
        out, idx, w = layer.forward(dev(x), dev(lg[None]))
        ref, ri, rw = orc.moe_layer(g, u, d, shared, x, logits=lg[None], hidden=H, n_ff=F, k=K)
        np.testing.assert_array_equal(host(idx)[:, :K], ri[:, :K])
        np.testing.assert_array_equal(host(w).view(np.uint32), rw.view(np.uint32))
        np.testing.assert_array_equal(host(out).view(np.uint32), ref.view(np.uint32))


def _collision_logits(E, K, seed):
    """Search (on the oracle) for a logit row where two distinct logits, one
    float ulp apart, give the same probability, so the probability order
    (lower index first) differs from the logit order."""
    rng = np.random.default_rng(seed)
    for _ in range(20000):
        lg = (rng.normal(0, 1, E) - 4.0).astype(np.float32)
        top = rng.choice(E, 2, replace=False)
        hi_i, lo_i = max(top), min(top)               # higher index gets the larger logit
        base = np.float32(rng.uniform(0.5, 2.0))
        lg[lo_i] = base
        lg[hi_i] = np.nextafter(base, np.float32(9.0))
        idx, _ = orc.router_topk(lg[None], K)
        if idx[0, 0] == lo_i:                         # probabilities tied -> lower index first
            return lg[None]
    raise AssertionError("no collision found")


def test_moe_layer_near_collision_probabilities():
    """Distinct logits whose probabilities round to the same float: the fused
    routing must fall back from the logit order to the exact selection."""
    H, F, E, K = 512, 256, 64, 8
    rng = np.random.default_rng(5150)
    g, u, d = _expert_pool(rng, E, H, F)
    x = rng.normal(0, 1, (1, H)).astype(np.float32)
    lg = _collision_logits(E, K, 77)
    layer = _layer(g, u, d, None, H, F, K, 1)
    out, idx, w = layer.forward(dev(x), dev(lg))
    ref, ri, rw = orc.moe_layer(g, u, d, None, x, logits=lg, hidden=H, n_ff=F, k=K)
    np.testing.assert_array_equal(host(idx)[:, :K], ri[:, :K])
    np.testing.assert_array_equal(host(w).view(np.uint32), rw.view(np.uint32))
    np.testing.assert_array_equal(host(out).view(np.uint32), ref.view(np.uint32))


# ---- prefill chunk: device plan + int8-MFMA grouped contractions ----------

@pytest.mark.parametrize("n_rows,n_expert,k", [(64, 32, 8), (2048, 256, 8), (300, 1024, 4)])
def test_dispatch_scan_matches_oracle(n_rows, n_expert, k):
    rng = np.random.default_rng(n_rows + n_expert)
    idx = np.stack([rng.choice(n_expert, k, replace=False) for _ in range(n_rows)]).astype(
        np.int32)
    idx = np.concatenate([idx, np.full((n_rows, 1), -1, np.int32)], axis=1)
    idx[3, 1] = n_expert + 5           # invalid ids: bounds-kill of rows 3 and 7
    idx[7, 0] = -2
    w = rng.uniform(0, 1, (n_rows, k + 1)).astype(np.float32)
    ref = orc.dispatch_scan(idx, w, k, n_expert, tok_per=64)
    wd = dev(w)
    got = ops.moe_dispatch_scan(dev(idx), wd, n_expert, k, tok_per=64)
    R = int(ref["meta"][0])
    np.testing.assert_array_equal(host(got["meta"])[:3], ref["meta"][:3])
    np.testing.assert_array_equal(host(got["off"])[:n_expert + 1], ref["off"])
    np.testing.assert_array_equal(host(got["toff"])[:n_expert + 1], ref["toff"])
    np.testing.assert_array_equal(host(got["gslot"]), ref["gslot"])
    np.testing.assert_array_equal(host(got["grows"])[:R], ref["grows"][:R])
    np.testing.assert_array_equal(host(wd), ref["weight"])


def test_dispatch_scan_duplicate_ids():
    """Caller routing may name one expert twice in a row: the serial
    placement keeps (token, slot) order."""
    idx = np.array([[1, 1, 2, -1], [2, 0, 2, -1], [0, 1, 2, -1]], np.int32)
    w = np.ones((3, 4), np.float32)
    ref = orc.dispatch_scan(idx, w, 3, 4, tok_per=2)
    got = ops.moe_dispatch_scan(dev(idx), dev(w), 4, 3, tok_per=2)
    np.testing.assert_array_equal(host(got["gslot"]), ref["gslot"])
    np.testing.assert_array_equal(host(got["grows"])[:9], ref["grows"][:9])


def _prefill(g, u, d, shared, hidden, n_ff, k, max_tokens):
    tg, kg = _tables(g)
    tu, ku = _tables(u)
    td, kd = _tables(d)
    sh = tuple(dev(m) for m in shared) if shared is not None else None
    layer = ops.MoePrefill(tg, tu, td, sh, hidden=hidden, n_ff=n_ff, n_expert=len(g), k=k,
                           max_tokens=max_tokens)
    layer._keep = (kg, ku, kd)
    return layer


@pytest.mark.parametrize("T,shared", [(1, True), (7, False), (64, True), (200, True)])
def test_moe_prefill_small_pool(T, shared):
    """hidden 2048, n_ff 512, top-8 of 32 experts: the MFMA path bit-exact
    against the integer-first oracle (routing, plan, grouped GEMMs, combine)."""
    rng = np.random.default_rng(700 + T)
    H, F, E, K = 2048, 512, 32, 8
    g, u, d = _expert_pool(rng, E + 1, H, F)
    sh = (g.pop(), u.pop(), d.pop())
    if not shared:
        sh = None
    x = rng.normal(0, 1, (T, H)).astype(np.float32)
    lg = rng.normal(0, 1, (T, E)).astype(np.float32)
    res = rng.normal(0, 1, (T, H)).astype(np.float32)
    layer = _prefill(g, u, d, sh, H, F, K, max(T, 16))
    out, idx, w = layer.forward(dev(x), dev(lg), residual=dev(res))
    ref, ri, rw = orc.moe_layer(g, u, d, sh, x, logits=lg, residual=res, hidden=H, n_ff=F, k=K,
                                prefill=True, n_threads=8)
    np.testing.assert_array_equal(host(idx)[:, :K], ri[:, :K])
    np.testing.assert_array_equal(host(w).view(np.uint32), rw.view(np.uint32))
    assert_fp32_parity(host(out), ref)


@pytest.mark.parametrize("E", [64, 100, 384, 600])
def test_moe_prefill_router_widths(E):
    """The prefill's routing at every router width: up to 512 experts it runs
    in the launch that also quantizes x (64, 128, 256 and 512 experts per
    wave), above that in its own launch.  Eight distinct matrices are cycled
    over the pool to keep host memory small; the routing, plan and outputs are
    bit-exact against the oracle."""
    rng = np.random.default_rng(900 + E)
    H, F, K, T = 2048, 512, 8, 40
    g0, u0, d0 = _expert_pool(rng, 8, H, F)
    g = [g0[e % 8] for e in range(E)]
    u = [u0[(e // 8) % 8] for e in range(E)]
    d = [d0[(e * 3) % 8] for e in range(E)]
    x = rng.normal(0, 1, (T, H)).astype(np.float32)
    lg = rng.normal(0, 1.5, (T, E)).astype(np.float32)
    layer = _prefill(g, u, d, None, H, F, K, T)
    out, idx, w = layer.forward(dev(x), dev(lg))
    ref, ri, rw = orc.moe_layer(g, u, d, None, x, logits=lg, hidden=H, n_ff=F, k=K,
                                prefill=True, n_threads=8)
    np.testing.assert_array_equal(host(idx)[:, :K], ri[:, :K])
    np.testing.assert_array_equal(host(w).view(np.uint32), rw.view(np.uint32))
    assert_fp32_parity(host(out), ref)


def test_moe_prefill_routed_edge_cases():
    """Caller routing: an out-of-range id (bounds-kill), an absent expert,
    a token routed twice to one expert, no shared expert, residual = out."""
    rng = np.random.default_rng(78)
    H, F, E, K, T = 512, 256, 8, 2, 5
    g, u, d = _expert_pool(rng, E, H, F)
    g[3] = None
    x = rng.normal(0, 1, (T, H)).astype(np.float32)
    idx = np.array([[1, 99, -1], [2, 3, -1], [3, 5, -1], [4, 4, -1], [0, 7, -1]], np.int32)
    w = rng.uniform(0.1, 1, (T, K + 1)).astype(np.float32)
    res = rng.normal(0, 1, (T, H)).astype(np.float32)
    layer = _prefill(g, u, d, None, H, F, K, T)
    io = dev(res)
    wd = dev(w)
    out, _, wgt = layer.forward(dev(x), None, residual=io, out=io, idx=dev(idx), weight=wd)
    ref, _, rw = orc.moe_layer(g, u, d, None, x, idx=idx, weight=w, residual=res, hidden=H,
                               n_ff=F, k=K, prefill=True)
    np.testing.assert_array_equal(host(wgt), rw)
    assert_fp32_parity(host(out), ref)


def test_moe_prefill_f16_routed_edge_cases():
    """The same caller routing on the session's fp16 buffers (fp16 g, u and
    h, fp16 slot outputs; the absent expert's zeroed h rows are fp16 there),
    the fp16 residual updated in place."""
    rng = np.random.default_rng(79)
    H, F, E, K, T = 512, 256, 8, 2, 5
    g, u, d = _expert_pool(rng, E, H, F)
    g[3] = None
    xn = rng.normal(0, 0.02, (T, H)).astype(np.float16)
    idx = np.array([[1, 99, -1], [2, 3, -1], [3, 5, -1], [4, 4, -1], [0, 7, -1]], np.int32)
    w = rng.uniform(0.1, 1, (T, K + 1)).astype(np.float32)
    res = rng.normal(0, 1, (T, H)).astype(np.float16)
    layer = _prefill(g, u, d, None, H, F, K, T)
    io = dev(res)
    wd = dev(w)
    out, _, wgt = layer.forward_f16(dev(xn), None, None, residual=io, out=io, idx=dev(idx),
                                    weight=wd)
    ref, _, rw = orc.moe_layer_f16(g, u, d, None, xn, idx=idx, weight=w, residual16=res,
                                   hidden=H, n_ff=F, k=K, prefill=True)
    assert np.isfinite(ref.astype(np.float32)).all()
    np.testing.assert_array_equal(host(wgt), rw)
    np.testing.assert_array_equal(host(out).view(np.uint16), ref.view(np.uint16))


def test_moe_prefill_f16_unaligned_buffers():
    """The fp16 combine reads and writes 16 B per thread only when the
    residual and output are 16-B aligned; buffers 8 B off that alignment
    take the 8-B path, with the same bits."""
    rng = np.random.default_rng(81)
    H, F, E, K, T = 512, 256, 8, 2, 7
    g, u, d = _expert_pool(rng, E, H, F)
    xn = rng.normal(0, 0.02, (T, H)).astype(np.float16)
    lg = rng.normal(0, 1, (T, E)).astype(np.float32)
    res = rng.normal(0, 1, (T, H)).astype(np.float16)
    layer = _prefill(g, u, d, None, H, F, K, T)
    out_a, _, _ = layer.forward_f16(dev(xn), None, dev(lg), residual=dev(res))
    flat_r = torch.zeros(T * H + 4, dtype=torch.float16, device="cuda")
    flat_o = torch.zeros(T * H + 4, dtype=torch.float16, device="cuda")
    r_u = flat_r[4:].view(T, H)
    o_u = flat_o[4:].view(T, H)
    r_u.copy_(dev(res))
    assert r_u.data_ptr() % 16 == 8 and o_u.data_ptr() % 16 == 8
    out_u, _, _ = layer.forward_f16(dev(xn), None, dev(lg), residual=r_u, out=o_u)
    np.testing.assert_array_equal(host(out_u).view(np.uint16), host(out_a).view(np.uint16))
    ref, _, _ = orc.moe_layer_f16(g, u, d, None, xn, logits=lg, residual16=res, hidden=H,
                                  n_ff=F, k=K, prefill=True)
    np.testing.assert_array_equal(host(out_a).view(np.uint16), ref.view(np.uint16))


def test_moe_prefill_vs_decode_path():
    """The prefill path and the decode path agree on indices and weights and,
    through their different fp32 epilogue orders, on the outputs to within
    what one flipped Q8_K code of h can move (both are checked bit-exact
    against their own oracle elsewhere)."""
    rng = np.random.default_rng(4321)
    H, F, E, K, T = 2048, 512, 32, 8, 16
    g, u, d = _expert_pool(rng, E + 1, H, F)
    sh = (g.pop(), u.pop(), d.pop())
    x = rng.normal(0, 1, (T, H)).astype(np.float32)
    lg = rng.normal(0, 1, (T, E)).astype(np.float32)
    pre = _prefill(g, u, d, sh, H, F, K, T)
    dec = _layer(g, u, d, sh, H, F, K, T)
    o1, i1, w1 = pre.forward(dev(x), dev(lg))
    o2, i2, w2 = dec.forward(dev(x), dev(lg))
    np.testing.assert_array_equal(host(i1), host(i2))
    np.testing.assert_array_equal(host(w1), host(w2))
    assert rel_err(host(o1), host(o2)) < 5e-3


def test_silu_exp_table_sweep():
    """The table exp (expf_tab, with its exact fallback near float rounding
    midpoints and outside [-87, 88]) against the oracle's expf_sg through
    SiLU: every 256th float bit pattern (all exponents, both signs, inf and
    NaN patterns) with u = 1, bit for bit."""
    bits = (np.arange(1 << 24, dtype=np.uint64) << np.uint64(8)).astype(np.uint32)
    bits |= np.uint32(0x5A)  # low mantissa bits set, so patterns are not all round
    g = bits.view(np.float32)
    u = np.ones_like(g)
    h = host(ops.silu_mul(dev(g), dev(u)))
    ref = orc.silu_mul(g, u)
    nan = np.isnan(ref)  # NaN payloads are not compared, only NaN-ness
    np.testing.assert_array_equal(np.isnan(h), nan)
    np.testing.assert_array_equal(h[~nan].view(np.uint32), ref[~nan].view(np.uint32))
