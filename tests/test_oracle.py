"""Pins the CPU oracle (oracle/sg_oracle.c) before anything is checked
against it.

Sources of truth, per function:
  - golden vectors written by tests/golden/make_golden.py from the
    reference's own CPU sources (q4_k.cpp, q4_avx2.cpp compiled here);
  - closed forms and brute force in numpy (int64 / float64);
  - libm expf and a float64 exp for the exp routine;
  - an independent numpy softmax + stable sort for the router.
"""
import math
import os

import numpy as np
import pytest

from oracle import oracle as orc
from sager_amd.synth import q4k_random_np

GOLD = os.path.join(os.path.dirname(__file__), "golden", "q4k_golden.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)


# ---- formats -------------------------------------------------------------

def test_half_to_float_all_patterns(gold):
    got = np.array([np.float32(orc.lib().orc_half_to_float(h)).view(np.uint32)
                    for h in range(65536)], dtype=np.uint32)
    np.testing.assert_array_equal(got, gold["half_f32_bits"])
    # closed form: numpy's own fp16 decode agrees on every non-NaN pattern
    h = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    fin = ~np.isnan(h)
    np.testing.assert_array_equal(got[fin], h[fin].view(np.uint32))


def test_scale_unpack(gold):
    sb, sv = gold["scale_bytes"], gold["scale_vals"]
    import ctypes
    d, m = ctypes.c_uint8(), ctypes.c_uint8()
    for i in range(sb.shape[0]):
        row = np.ascontiguousarray(sb[i])
        for j in range(8):
            orc.lib().orc_get_scale_min(j, orc.P(row), ctypes.byref(d), ctypes.byref(m))
            assert (d.value, m.value) == tuple(sv[i, j])
    # closed form: the 12 bytes are a bijection onto sixteen 6-bit fields
    bits = np.unpackbits(sb, axis=1, bitorder="little").sum()
    assert sv.max() <= 63 and bits > 0


def test_dequant_matches_reference(gold):
    w = gold["gemv_c_w"]
    n = w.shape[0] * 256
    np.testing.assert_array_equal(orc.dequant(w, n), gold["real_dequant"])


# ---- Q8_K ------------------------------------------------------------------

def test_q8k_bit_exact_vs_reference(gold):
    got = orc.quantize_q8_k(gold["q8_x"])
    np.testing.assert_array_equal(got, gold["q8_out"])
    np.testing.assert_array_equal(got, gold["q8_out_avx2"])


def _q8_fields(b):
    b = b.reshape(-1, 276)
    d = b[:, 0:4].copy().view(np.float32)[:, 0]
    qs = b[:, 4:260].view(np.int8)
    bs = b[:, 260:276].copy().view(np.int16)
    return d, qs, bs


def test_q8k_invariants():
    rng = np.random.default_rng(99)
    x = rng.normal(0, 1, (7, 2048)).astype(np.float32)
    d, qs, bs = _q8_fields(orc.quantize_q8_k(x))
    xb = x.reshape(-1, 256)
    amax = np.maximum(np.abs(xb).max(axis=1), np.float32(1e-30))
    np.testing.assert_array_equal(d, (amax / np.float32(127)).astype(np.float32))
    assert np.abs(qs.astype(int)).max() <= 127
    np.testing.assert_array_equal(bs, qs.reshape(-1, 8, 32).astype(np.int64).sum(axis=2))
    # code = round-half-even(x * (1/d)) away from the clamp
    idf = (np.float32(1) / d).astype(np.float32)
    want = np.rint((xb * idf[:, None]).astype(np.float32)).clip(-127, 127)
    np.testing.assert_array_equal(qs, want.astype(np.int8))


# ---- integer dots and the GEMV ---------------------------------------------

def _brute_dots(w, xq, n_rows, k):
    nb = k // 256
    wb = w.reshape(n_rows, nb, 144)
    qs = wb[:, :, 16:].reshape(n_rows, nb, 4, 32)
    lo = (qs & 15).astype(np.int64)
    hi = (qs >> 4).astype(np.int64)
    nib = np.stack([lo, hi], axis=3).reshape(n_rows, nb, 8, 32)  # sub-block 2g, 2g+1
    _, xqs, _ = _q8_fields(xq)
    xv = xqs.reshape(nb, 8, 32).astype(np.int64)
    return (nib * xv[None]).sum(axis=3)


@pytest.mark.parametrize("case", ["gemv_a", "gemv_b", "gemv_c"])
def test_subblock_dots_brute_force(gold, case):
    n_rows, k = (int(v) for v in gold[case + "_shape"])
    w, xq = gold[case + "_w"], gold[case + "_xq"][0]
    np.testing.assert_array_equal(orc.subblock_dots(w, xq, n_rows, k),
                                  _brute_dots(w, xq, n_rows, k))


@pytest.mark.parametrize("case", ["gemv_a", "gemv_b", "gemv_c"])
def test_gemv_bit_exact_vs_reference(gold, case):
    n_rows, k = (int(v) for v in gold[case + "_shape"])
    w, xq = gold[case + "_w"], gold[case + "_xq"]
    y = orc.gemv(w, xq, n_rows, k, n_tokens=xq.shape[0])
    np.testing.assert_array_equal(y.view(np.uint32), gold[case + "_y"].view(np.uint32))
    np.testing.assert_array_equal(y.view(np.uint32), gold[case + "_y_scalar"].view(np.uint32))


@pytest.mark.parametrize("case", ["gemv_a", "gemv_c"])
def test_gemv_vs_fp64_dequant_dot(gold, case):
    """Independent float64 evaluation of the same quantized operands."""
    n_rows, k = (int(v) for v in gold[case + "_shape"])
    w, xq = gold[case + "_w"], gold[case + "_xq"][0]
    nb = k // 256
    dots = _brute_dots(w, xq, n_rows, k).astype(np.float64)
    wb = w.reshape(n_rows, nb, 144)
    d = wb[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    dm = wb[:, :, 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    sc = np.zeros((n_rows, nb, 8)); mn = np.zeros((n_rows, nb, 8))
    s12 = wb[:, :, 4:16].astype(np.int64)
    for j in range(8):
        if j < 4:
            sc[..., j] = s12[..., j] & 63
            mn[..., j] = s12[..., j + 4] & 63
        else:
            sc[..., j] = (s12[..., j + 4] & 15) | ((s12[..., j - 4] >> 6) << 4)
            mn[..., j] = (s12[..., j + 4] >> 4) | ((s12[..., j] >> 6) << 4)
    xd, _, bs = _q8_fields(xq)
    ref = (xd[None, :, None] * (d[..., None] * sc * dots - dm[..., None] * mn * bs[None])).sum(
        axis=(1, 2))
    y = orc.gemv(w, xq, n_rows, k)[0].astype(np.float64)
    scale = np.abs(ref).max()
    assert np.abs(y - ref).max() <= 1e-5 * scale
    # the reference's per-sub-block vec_dot_ref order lands in the same band
    assert np.abs(gold[case + "_vecdot"] - ref).max() <= 1e-5 * scale


@pytest.mark.parametrize("case", ["gemv_a", "gemv_c"])
def test_gemv_int_first_vs_fp64(gold, case):
    """The prefill GEMV (integer-first epilogue: exact I = sum sc*ip and
    M = sum mn*bsum per super-block, then two fmas) against the same float64
    evaluation; it is at least as close as the AVX2 order."""
    n_rows, k = (int(v) for v in gold[case + "_shape"])
    w, xq = gold[case + "_w"], gold[case + "_xq"][0]
    nb = k // 256
    dots = _brute_dots(w, xq, n_rows, k).astype(np.int64)
    wb = w.reshape(n_rows, nb, 144)
    d = wb[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    dm = wb[:, :, 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    s12 = wb[:, :, 4:16].astype(np.int64)
    sc = np.zeros((n_rows, nb, 8), np.int64); mn = np.zeros((n_rows, nb, 8), np.int64)
    for j in range(8):
        if j < 4:
            sc[..., j] = s12[..., j] & 63
            mn[..., j] = s12[..., j + 4] & 63
        else:
            sc[..., j] = (s12[..., j + 4] & 15) | ((s12[..., j - 4] >> 6) << 4)
            mn[..., j] = (s12[..., j + 4] >> 4) | ((s12[..., j] >> 6) << 4)
    xd, _, bs = _q8_fields(xq)
    I = (sc * dots).sum(axis=2)                       # exact integers per super-block
    M = (mn * bs[None].astype(np.int64)).sum(axis=2)
    ref = (xd[None, :] * (d * I - dm * M)).sum(axis=1)
    y = orc.gemv_int(w, xq, n_rows, k)[0].astype(np.float64)
    y_avx = orc.gemv(w, xq, n_rows, k)[0].astype(np.float64)
    scale = np.abs(ref).max()
    assert np.abs(y - ref).max() <= 1e-5 * scale
    assert np.abs(y - ref).max() <= np.abs(y_avx - ref).max() * 1.5 + 1e-7 * scale


def test_moe_prefill_is_router_ffn_int_combine():
    """orc_moe_prefill = router + per-route expert FFN with the integer-first
    GEMV (each stage by its own oracle function) + slot-order combine."""
    rng = np.random.default_rng(31)
    H, F, E, K, T = 512, 256, 8, 2, 3
    g = [q4k_random_np(rng, F * H // 256) for _ in range(E)]
    u = [q4k_random_np(rng, F * H // 256) for _ in range(E)]
    d = [q4k_random_np(rng, H * F // 256) for _ in range(E)]
    x = rng.normal(0, 1, (T, H)).astype(np.float32)
    lg = rng.normal(0, 1, (T, E)).astype(np.float32)
    out, idx, w = orc.moe_layer(g, u, d, None, x, logits=lg, hidden=H, n_ff=F, k=K, prefill=True)
    ri, rw = orc.router_topk(lg, K)
    np.testing.assert_array_equal(idx, ri)
    ys = np.zeros((T, K + 1, H), np.float32)
    for t in range(T):
        xq = orc.quantize_q8_k(x[t])
        for kk in range(K):
            e = ri[t, kk]
            gg = orc.gemv_int(g[e], xq, F, H)[0]
            uu = orc.gemv_int(u[e], xq, F, H)[0]
            hq = orc.quantize_q8_k(orc.silu_mul(gg, uu))
            ys[t, kk] = orc.gemv_int(d[e], hq, H, F)[0]
    ref = orc.moe_combine(ys, rw)
    np.testing.assert_array_equal(out.view(np.uint32), ref.view(np.uint32))


# ---- exp, SiLU, expert FFN ------------------------------------------------

def test_expf_correctly_rounded_sample():
    rng = np.random.default_rng(5)
    xs = np.concatenate([rng.uniform(-104, 89, 20000), rng.uniform(-1, 1, 20000),
                         [0.0, -0.0, 88.72283, 88.7228394, -87.33654, -103.97, 1e-30, -1e-30]])
    for x in xs.astype(np.float32):
        want = np.float32(math.exp(float(x))) if x < 88.73 else np.float32(np.inf)
        assert np.float32(orc.lib().orc_expf(float(x))) == want, x
    assert math.isnan(orc.lib().orc_expf(float("nan")))
    assert orc.lib().orc_expf(float("inf")) == float("inf")
    assert orc.lib().orc_expf(float("-inf")) == 0.0


def test_expf_vs_libm_expf():
    """The reference's std::exp(float) is the platform expf: they differ only
    by rare 1-ulp roundings (glibc's expf is not correctly rounded)."""
    n = 2_000_000
    bad = orc.lib().orc_count_expf_mismatch(n, 11, -104.0, 89.0)
    assert bad <= n * 2e-3


def test_silu_closed_form():
    rng = np.random.default_rng(3)
    g = rng.normal(0, 3, 4096).astype(np.float32)
    u = rng.normal(0, 1, 4096).astype(np.float32)
    h = orc.silu_mul(g, u)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    np.testing.assert_allclose(h, ref, rtol=3e-7, atol=1e-30)


def test_expert_ffn_vs_reference(gold):
    H, F = (int(v) for v in gold["ffn_shape"])
    for t in range(gold["ffn_x"].shape[0]):
        y = orc.expert_ffn(gold["ffn_wg"], gold["ffn_wu"], gold["ffn_wd"], gold["ffn_x"][t], H, F)
        ref = gold["ffn_y"][t]
        # exp() is the only deliberate difference (see test_expf_vs_libm_expf)
        floor = 1e-3 * np.abs(ref).max()
        rel = np.abs(y - ref) / np.maximum(np.abs(ref), floor)
        assert rel.max() <= 1e-4
        assert np.mean(y == ref) > 0.9


# ---- router ---------------------------------------------------------------

def _router_np(logits, k, shared_w):
    """Independent restatement: float64 softmax for the ordering, stable sort
    by (-prob, index); weights renormalized."""
    idx = np.zeros((logits.shape[0], k), np.int32)
    w = np.zeros((logits.shape[0], k))
    for r, lg in enumerate(logits.astype(np.float64)):
        p = np.exp(lg - lg.max())
        p /= p.sum()
        order = np.lexsort((np.arange(lg.size), -p))[:k]
        idx[r] = order
        w[r] = p[order] / p[order].sum()
    return idx, w


def test_router_random_logits():
    rng = np.random.default_rng(17)
    for n_expert, k, sigma in [(256, 8, 1.0), (256, 8, 1.5), (64, 4, 1.0), (1000, 32, 2.0)]:
        lg = rng.normal(0, sigma, (16, n_expert)).astype(np.float32)
        idx, w = orc.router_topk(lg, k, shared_w=1.0)
        ri, rw = _router_np(lg, k, 1.0)
        np.testing.assert_array_equal(idx[:, :k], ri)
        np.testing.assert_allclose(w[:, :k], rw, rtol=2e-6)
        assert (w[:, k] == 1.0).all()
        # weights sorted descending, sum to 1
        assert (np.diff(w[:, :k], axis=1) <= 0).all()
        np.testing.assert_allclose(w[:, :k].sum(axis=1), 1.0, rtol=1e-5)


def test_router_ties_lower_index():
    lg = np.zeros((1, 256), np.float32)
    lg[0, [7, 3, 200, 100]] = 2.0          # four-way tie at the top
    lg[0, [50, 9]] = 1.0
    idx, w = orc.router_topk(lg, 8, shared_w=0.0)
    assert list(idx[0, :8]) == [3, 7, 100, 200, 9, 50, 0, 1]
    assert w[0, 8] == 0.0
    eq = np.full((1, 16), 0.5, np.float32)
    idx, w = orc.router_topk(eq, 4)
    assert list(idx[0, :4]) == [0, 1, 2, 3]
    np.testing.assert_array_equal(w[0, :4], np.float32(0.25))


def test_router_nan_and_degenerate():
    lg = np.random.default_rng(1).normal(0, 1, (2, 32)).astype(np.float32)
    lg[0, 5] = np.nan   # NaN logit poisons the normalizer: every prob is NaN
    lg[1, :] = np.nan
    idx, w = orc.router_topk(lg, 4)
    for r in range(2):
        assert list(idx[r, :4]) == [0, 1, 2, 3]     # kk % n_expert
        assert (w[r, :4] == -1.0).all()             # sum <= 0: not renormalized


# ---- combine, layer, plan -------------------------------------------------

def test_combine_closed_form():
    rng = np.random.default_rng(4)
    y = rng.normal(0, 1, (3, 9, 2048)).astype(np.float32)
    w = rng.uniform(0, 1, (3, 9)).astype(np.float32)
    res = rng.normal(0, 1, (3, 2048)).astype(np.float32)
    out = orc.moe_combine(y, w, res)
    ref = res.astype(np.float64) + np.einsum("rk,rkh->rh", w.astype(np.float64), y)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)
    # slot order: the result equals the left-to-right fma chain
    acc = res.copy()
    for kk in range(9):
        acc = (w[:, kk:kk + 1].astype(np.float64) * y[:, kk] + acc).astype(np.float32)
    np.testing.assert_array_equal(out, acc)


def _experts(rng, n, hidden, n_ff):
    g = [q4k_random_np(rng, n_ff * hidden // 256) for _ in range(n)]
    u = [q4k_random_np(rng, n_ff * hidden // 256) for _ in range(n)]
    d = [q4k_random_np(rng, hidden * n_ff // 256) for _ in range(n)]
    return g, u, d


def test_moe_layer_is_router_ffn_combine():
    rng = np.random.default_rng(8)
    H, F, E, K = 512, 256, 16, 4
    g, u, d = _experts(rng, E + 1, H, F)
    sh = (g[E], u[E], d[E])
    x = rng.normal(0, 1, (3, H)).astype(np.float32)
    lg = rng.normal(0, 1, (3, E)).astype(np.float32)
    out, idx, w = orc.moe_layer(g[:E], u[:E], d[:E], sh, x, logits=lg, hidden=H, n_ff=F, k=K)
    ri, rw = orc.router_topk(lg, K)
    np.testing.assert_array_equal(idx[:, :K], ri[:, :K])
    for t in range(3):
        ys = [orc.expert_ffn(g[e], u[e], d[e], x[t], H, F) for e in idx[t, :K]]
        ys.append(orc.expert_ffn(*sh, x[t], H, F))
        ref = orc.moe_combine(np.stack(ys)[None], w[t:t + 1])
        np.testing.assert_array_equal(out[t], ref[0])
    # the worker pool gives the same bits
    out_mt, _, _ = orc.moe_layer(g[:E], u[:E], d[:E], sh, x, logits=lg, hidden=H, n_ff=F, k=K,
                                 n_threads=4)
    np.testing.assert_array_equal(out, out_mt)


def test_moe_layer_bad_ids_and_absent_experts():
    rng = np.random.default_rng(9)
    H, F, E, K = 256, 256, 8, 2
    g, u, d = _experts(rng, E, H, F)
    x = rng.normal(0, 1, (2, H)).astype(np.float32)
    idx = np.array([[1, 99, -1], [2, 3, -1]], np.int32)    # row 0 has an out-of-range id
    w = np.array([[0.6, 0.4, 1.0], [0.7, 0.3, 1.0]], np.float32)
    g2 = list(g)
    g2[3] = None                                            # expert 3 absent
    out, _, wk = orc.moe_layer(g2, u, d, None, x, idx=idx, weight=w, hidden=H, n_ff=F, k=K)
    np.testing.assert_array_equal(out[0], 0.0)              # bounds-kill zeroes the row
    np.testing.assert_array_equal(wk[0], 0.0)
    y2 = orc.expert_ffn(g[2], u[2], d[2], x[1], H, F)
    np.testing.assert_array_equal(out[1], (np.float32(0.7) * y2).astype(np.float32) + 0.0)


def test_dispatch_scan_invariants():
    rng = np.random.default_rng(2)
    n_rows, k, E = 64, 8, 256
    idx = np.stack([rng.permutation(E)[:k] for _ in range(n_rows)]).astype(np.int32)
    idx = np.concatenate([idx, np.full((n_rows, 1), -1, np.int32)], axis=1)
    idx[5, 2] = 300
    w = np.ones((n_rows, k + 1), np.float32)
    r = orc.dispatch_scan(idx, w, k, E, tok_per=4)
    valid = idx[:, :k][(idx[:, :k] >= 0) & (idx[:, :k] < E)]
    hist = np.bincount(valid, minlength=E)
    np.testing.assert_array_equal(np.diff(r["off"]), hist)
    np.testing.assert_array_equal(np.diff(r["toff"]), (hist + 3) // 4)
    assert tuple(r["meta"][:3]) == (valid.size, ((hist + 3) // 4).sum(), 1)
    assert (r["weight"][5] == 0).all() and (r["weight"][4] == 1).all()
    # every valid route lands in its expert's segment, rows ascending within it
    for rr in range(n_rows):
        for kk in range(k):
            e, gs = idx[rr, kk], r["gslot"][rr * k + kk]
            if 0 <= e < E:
                assert r["off"][e] <= gs < r["off"][e + 1] and r["grows"][gs] == rr
            else:
                assert gs == -1


# ---- Q6_K head GEMV ----------------------------------------------------------

def _q6_codes_by_subgroup(w6, n_blocks):
    """q6 - 32 per weight, decoded through the GPU kernel's sub-group view
    (q4_k.cu:1595-1613: sub-group t = half*8 + 2*quarter + is, 16 weights
    each) - a different indexing from the dequant loops of weights.cpp."""
    b = w6.reshape(n_blocks, 210).astype(np.int64)
    out = np.zeros((n_blocks, 256), np.int64)
    scale = np.zeros((n_blocks, 256), np.int64)
    sc = b[:, 192:208].astype(np.uint8).view(np.int8).astype(np.int64)
    for t in range(16):
        n, q, is_ = t >> 3, (t & 7) >> 1, t & 1
        for j in range(16):
            lo = (b[:, n * 64 + (q & 1) * 32 + is_ * 16 + j] >> (4 if q & 2 else 0)) & 15
            hi = (b[:, 128 + n * 32 + is_ * 16 + j] >> (2 * q)) & 3
            col = n * 128 + q * 32 + is_ * 16 + j
            out[:, col] = (lo | (hi << 4)) - 32
            scale[:, col] = sc[:, t]
    return out, scale


def test_q6k_dequant_matches_subgroup_view():
    rng = np.random.default_rng(61)
    from sager_amd.synth import q6k_random_np
    w6 = q6k_random_np(rng, 40)
    codes, scale = _q6_codes_by_subgroup(w6, 40)
    d = w6[:, 208:210].copy().view(np.float16)[:, 0].astype(np.float32)
    ref = (d[:, None] * scale.astype(np.float32)) * codes.astype(np.float32)
    np.testing.assert_array_equal(orc.dequant_q6k(w6, 40 * 256), ref.reshape(-1))


def test_q6k_dequant_hand_block():
    """One block built by hand: weight 0 = ql[0] low nibble | qh[0] bits 0-1,
    weight 64 = ql[0] high nibble | qh[0] bits 4-5, weight 160 (second half,
    quarter 1) = ql[64+32] low | qh[32] bits 2-3; scales sc[0], sc[4], sc[10]."""
    blk = np.zeros(210, np.uint8)
    blk[0] = 0x5A            # low 0xA, high 0x5
    blk[128] = 0b00_10_00_11  # bits 0-1 = 3, bits 4-5 = 2
    blk[96] = 0x07
    blk[160] = 0b0000_01_00  # bits 2-3 = 1
    sc = np.zeros(16, np.int8)
    sc[0], sc[4], sc[10] = 3, -2, 5
    blk[192:208] = sc.view(np.uint8)
    blk[208:210] = np.array([1.0], np.float16).view(np.uint8)
    y = orc.dequant_q6k(blk, 256)
    assert y[0] == 3 * ((0xA | 3 << 4) - 32)
    assert y[64] == -2 * ((0x5 | 2 << 4) - 32)
    assert y[160] == 5 * ((0x7 | 1 << 4) - 32)
    assert y[1] == 3 * (0 - 32)


def test_q6k_subgroup_dots_brute_force():
    rng = np.random.default_rng(62)
    from sager_amd.synth import q6k_random_np
    n_rows, k = 7, 768
    w6 = q6k_random_np(rng, n_rows * k // 256)
    xq = orc.quantize_q8_k(rng.normal(0, 1, k).astype(np.float32))[0]
    codes, _ = _q6_codes_by_subgroup(w6, n_rows * k // 256)
    x = np.concatenate([_q8_fields(xq)[1][b] for b in range(k // 256)]).astype(np.int64)
    ref = (codes.reshape(n_rows, k) * x[None]).reshape(n_rows, k // 256, 16, 16).sum(-1)
    np.testing.assert_array_equal(orc.q6k_subgroup_dots(w6, xq, n_rows, k), ref)


@pytest.mark.parametrize("n_rows,k", [(64, 2048), (5, 256), (3, 4096)])
def test_q6k_gemv_vs_fp64(n_rows, k):
    """Float64 dequant-dot of the same quantized operands: the 32-lane fp32
    order stays within 1e-5 of the row scale."""
    rng = np.random.default_rng(n_rows + k)
    from sager_amd.synth import q6k_random_np
    w6 = q6k_random_np(rng, n_rows * k // 256)
    xq = orc.quantize_q8_k(rng.normal(0, 1, k).astype(np.float32))[0]
    codes, scale = _q6_codes_by_subgroup(w6, n_rows * k // 256)
    d = w6[:, 208:210].copy().view(np.float16)[:, 0].astype(np.float64)
    wf = (d[:, None] * scale * codes).reshape(n_rows, k)
    xd = np.repeat(_q8_fields(xq)[0].astype(np.float64), 256)
    xv = np.concatenate([_q8_fields(xq)[1][b] for b in range(k // 256)]).astype(np.float64)
    ref = wf @ (xd * xv)
    y = orc.gemv_q6k(w6, xq, n_rows, k).astype(np.float64)
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()


# ---- fp32 GEMV in the reference lane order, sigmoid, the shared gate -------

def test_gemv_f32_lanes_order_pinned():
    """Values chosen so that the lane-strided sequential fma chain and the
    shfl_down tree (q4_k.cu:133-149) give exactly 1.0 while other orders do
    not: lane 0 sums 2^24, 1, 1, -2^24 in index order (the 1s are absorbed:
    0), lanes 1 and 17 cancel at the first tree step (off 16) before lane
    9's 1 is added at the second (off 8)."""
    k = 128
    w = np.ones((1, k), np.float32)
    x = np.zeros(k, np.float32)
    x[0], x[32], x[64], x[96] = 2.0**24, 1.0, 1.0, -2.0**24
    x[1], x[17], x[9] = 2.0**25, -2.0**25, 1.0
    assert orc.gemv_f32_lanes(w, x)[0, 0] == np.float32(1.0)
    # a plain index-order float32 sum loses both 1s and lane 9's
    acc = np.float32(0)
    for v in x:
        acc = np.float32(acc + v)
    assert acc != np.float32(1.0)


def test_gemv_f32_lanes_vs_fp64():
    rng = np.random.default_rng(31)
    for n_rows, k, T in ((7, 2048, 3), (256, 2048, 1), (5, 96, 2), (3, 40, 1)):
        w = rng.normal(0, 0.05, (n_rows, k)).astype(np.float32)
        x = rng.normal(0, 1, (T, k)).astype(np.float32)
        y = orc.gemv_f32_lanes(w, x)
        ref = x.astype(np.float64) @ w.astype(np.float64).T
        bound = 1e-6 * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T) + 1e-30
        assert (np.abs(y - ref) <= bound).all()
        # exact on integers small enough that every partial sum is exact
        wi = rng.integers(-8, 9, (n_rows, k)).astype(np.float32)
        xi = rng.integers(-8, 9, (T, k)).astype(np.float32)
        np.testing.assert_array_equal(orc.gemv_f32_lanes(wi, xi),
                                      (xi.astype(np.int64) @ wi.astype(np.int64).T))


def test_sigmoid_closed_form():
    assert orc.sigmoid(0.0) == np.float32(0.5)
    assert orc.sigmoid(200.0) == np.float32(1.0)
    assert orc.sigmoid(-200.0) == np.float32(0.0)
    rng = np.random.default_rng(5)
    for g in rng.normal(0, 4, 2000).astype(np.float32):
        ref = 1.0 / (1.0 + math.exp(-float(g)))
        got = float(orc.sigmoid(g))
        # exp correctly rounded, then two float32 roundings (add, divide)
        assert abs(got - ref) <= 3 * np.spacing(np.float32(ref)), (g, got, ref)


@pytest.mark.parametrize("prefill", [False, True])
def test_moe_layer_shared_gate_is_scaled_shared_slot(prefill):
    """The gated layer = the ungated experts, with the shared slot's output
    multiplied by sigmoid(gate_w . x[t]) before the combine."""
    rng = np.random.default_rng(44)
    H, F, E, K, T = 512, 256, 8, 3, 3
    g, u, d = _experts(rng, E + 1, H, F)
    sh = (g[E], u[E], d[E])
    x = rng.normal(0, 1, (T, H)).astype(np.float32)
    lg = rng.normal(0, 1, (T, E)).astype(np.float32)
    gw = rng.normal(0, 0.05, H).astype(np.float32)
    res = rng.normal(0, 1, (T, H)).astype(np.float32)
    out, idx, w = orc.moe_layer(g[:E], u[:E], d[:E], sh, x, logits=lg, residual=res, hidden=H,
                                n_ff=F, k=K, shared_gate_w=gw, prefill=prefill, shared_w=0.5)
    out0, idx0, _ = orc.moe_layer(g[:E], u[:E], d[:E], sh, x, logits=lg, residual=res, hidden=H,
                                  n_ff=F, k=K, prefill=prefill, shared_w=0.5)
    np.testing.assert_array_equal(idx, idx0)
    assert not np.array_equal(out, out0)
    gl = orc.gemv_f32_lanes(gw[None], x)[:, 0]
    xq = orc.quantize_q8_k(x)
    for t in range(T):
        ys = []
        for m in list(idx[t, :K]) + [None]:
            wg, wu, wd = sh if m is None else (g[m], u[m], d[m])
            if prefill:
                gg = orc.gemv_int(wg, xq[t], F, H)[0]
                uu = orc.gemv_int(wu, xq[t], F, H)[0]
                hh = orc.quantize_q8_k(orc.silu_mul(gg, uu))
                ys.append(orc.gemv_int(wd, hh, H, F)[0])
            else:
                ys.append(orc.expert_ffn(wg, wu, wd, x[t], H, F))
        s = orc.sigmoid(gl[t])
        ys[-1] = (ys[-1] * s).astype(np.float32)
        ref = orc.moe_combine(np.stack(ys)[None], w[t:t + 1], res[t:t + 1])
        np.testing.assert_array_equal(out[t], ref[0])
    # without a shared expert the gate has nothing to scale
    o1, _, _ = orc.moe_layer(g[:E], u[:E], d[:E], None, x, logits=lg, hidden=H, n_ff=F, k=K,
                             shared_gate_w=gw, prefill=prefill)
    o2, _, _ = orc.moe_layer(g[:E], u[:E], d[:E], None, x, logits=lg, hidden=H, n_ff=F, k=K,
                             prefill=prefill)
    np.testing.assert_array_equal(o1, o2)


# ---- the session's fp16 buffers ----------------------------------------------

def test_float_to_half_matches_numpy():
    """orc_float_to_half (round to nearest even) against numpy's float16
    conversion: the boundaries (largest half, the overflow midpoint 65520,
    subnormal and normal ranges, ties at every mantissa position) and 4M
    random bit patterns."""
    edge = np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, -65520.0, 1e30, -1e30,
                     2.0**-14, 2.0**-24, 2.0**-25, 2.0**-25 * 1.0000001, 3 * 2.0**-25,
                     2.0**-26, 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, 1.0 + 2.0**-11 + 2.0**-20,
                     2049.0, 2051.0, 6.1e-5, 5.96e-8, np.inf, -np.inf], np.float32)
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 2**32, 1 << 22, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([edge, bits.view(np.float32)])
    got = orc.float_to_half(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    np.testing.assert_array_equal(got[~nan], ref[~nan])
    assert (got[nan] & 0x7c00 == 0x7c00).all() and (got[nan] & 0x3ff != 0).all()


@pytest.mark.parametrize("prefill,gate", [(False, False), (False, True), (True, True)])
def test_moe_layer_f16_is_rounded_composition(prefill, gate):
    """The fp16-buffer layer = the fp32 layer's GEMVs with each expert's g
    and u stored as fp16, h = fp16(SiLU(g) * u) quantized, the slot outputs
    stored as fp16 (numpy's own conversion here), the shared slot gated on
    its fp16 value and stored again, combined in fp32 from the fp16
    residual, stored as fp16."""
    rng = np.random.default_rng(45)
    H, F, E, K, T = 512, 256, 8, 3, 3
    g, u, d = _experts(rng, E + 1, H, F)
    sh = (g[E], u[E], d[E])
    xn = rng.normal(0, 0.02, (T, H)).astype(np.float16)  # outputs stay finite in fp16
    lg = rng.normal(0, 1, (T, E)).astype(np.float32)
    gw = rng.normal(0, 0.05, H).astype(np.float32) if gate else None
    res = rng.normal(0, 1, (T, H)).astype(np.float16)
    out, idx, w = orc.moe_layer_f16(g[:E], u[:E], d[:E], sh, xn, logits=lg, residual16=res,
                                    hidden=H, n_ff=F, k=K, shared_gate_w=gw, prefill=prefill,
                                    shared_w=0.5)
    assert out.dtype == np.float16
    assert np.isfinite(out.astype(np.float32)).all()
    x = xn.astype(np.float32)
    xq = orc.quantize_q8_k(x)
    gl = orc.gemv_f32_lanes(gw[None], x)[:, 0] if gate else None
    f16 = lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float32)
    mv = orc.gemv_int if prefill else orc.gemv
    n_differ = 0
    for t in range(T):
        refs = []
        for r_mid in (f16, lambda a: np.asarray(a, np.float32)):
            ys = []
            for m in list(idx[t, :K]) + [None]:
                wg, wu, wd = sh if m is None else (g[m], u[m], d[m])
                # g and u stored as fp16, h = fp16(SiLU(g) * u), Q8_K of those values
                gg = r_mid(mv(wg, xq[t], F, H)[0])
                uu = r_mid(mv(wu, xq[t], F, H)[0])
                hh = orc.quantize_q8_k(r_mid(orc.silu_mul(gg, uu)))
                ys.append(f16(mv(wd, hh, H, F)[0]))
            if gate:
                ys[-1] = f16(ys[-1] * orc.sigmoid(gl[t]))
            ref = orc.moe_combine(np.stack(ys)[None], w[t:t + 1], res[t:t + 1].astype(np.float32))
            refs.append(ref[0].astype(np.float16).view(np.uint16))
        np.testing.assert_array_equal(out[t].view(np.uint16), refs[0])
        n_differ += int((refs[0] != refs[1]).sum())
    # the intermediate fp16 roundings change the output: this test tells the
    # two compositions apart
    assert n_differ > 0
