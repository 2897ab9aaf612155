"""GPU checks of the stage-by-stage launchers (sg_stages.hip): the row
gathers and scatters against numpy indexing, the device-count SiLU and Q8_K
against the oracle, and the plan-driven grouped GEMVs against the oracle's
GEMV (reference CPU order) rounded to fp16, over a real dispatch plan with an
absent expert (zeroed outputs, mailbox).  Bar: bit-exact."""
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


@pytest.mark.parametrize("counted", [False, True])
def test_gather_rows_q8(counted):
    rng = np.random.default_rng(1)
    rb, n_src, n = 3, 50, 37
    src = rng.integers(0, 256, (n_src, rb * 276), dtype=np.uint8)
    rows = rng.integers(0, n_src, n).astype(np.int32)
    if counted:
        live = 29
        out = dev(np.full((n, rb * 276), 0xAB, np.uint8))
        ops.gather_rows_q8(dev(src), dev(rows), rb, meta=dev(np.array([live, 7], np.int32)),
                           r_max=n, out=out)
        got = host(out)
        np.testing.assert_array_equal(got[:live], src[rows[:live]])
        assert (got[live:] == 0xAB).all()  # rows past the device count untouched
    else:
        got = host(ops.gather_rows_q8(dev(src), dev(rows), rb))
        np.testing.assert_array_equal(got, src[rows])


@pytest.mark.parametrize("hidden", [2048, 100])
def test_gather_rows_f16_n(hidden):
    rng = np.random.default_rng(2)
    src = rng.normal(0, 1, (40, hidden)).astype(np.float16)
    rows = rng.integers(0, 40, 24).astype(np.int32)
    out = dev(np.zeros((24, hidden), np.float16))
    ops.gather_rows_f16_n(dev(src), dev(rows), dev(np.array([20], np.int32)), 24, out=out)
    got = host(out)
    np.testing.assert_array_equal(got[:20].view(np.uint16), src[rows[:20]].view(np.uint16))
    assert (got[20:] == 0).all()


@pytest.mark.parametrize("hidden", [512, 36])
def test_scatter_routed_and_rows_f16(hidden):
    rng = np.random.default_rng(3)
    n_rows, n_used = 9, 4
    grouped = rng.normal(0, 1, (n_rows * n_used, hidden)).astype(np.float16)
    gslot = rng.permutation(n_rows * n_used).astype(np.int32)
    gslot[[3, 17]] = -1  # killed routes: their slots keep what was there
    ey0 = rng.normal(0, 1, (n_rows, n_used + 1, hidden)).astype(np.float16)
    ey = dev(ey0)
    ops.scatter_routed_f16(ey, dev(grouped), dev(gslot), n_rows, n_used)
    want = ey0.copy()
    for r in range(n_rows):
        for kk in range(n_used):
            gs = gslot[r * n_used + kk]
            if gs >= 0:
                want[r, kk] = grouped[gs]
    np.testing.assert_array_equal(host(ey).view(np.uint16), want.view(np.uint16))

    dst0 = np.zeros((30, hidden), np.float16)
    src = rng.normal(0, 1, (12, hidden)).astype(np.float16)
    drows = rng.choice(30, 12, replace=False).astype(np.int32)
    dst = dev(dst0)
    ops.scatter_rows_f16(dst, dev(src), dev(drows))
    want = dst0.copy()
    want[drows] = src
    np.testing.assert_array_equal(host(dst).view(np.uint16), want.view(np.uint16))


def test_silu_and_quantize_device_count():
    rng = np.random.default_rng(4)
    rows_max, live, n_ff = 12, 7, 512
    g = rng.normal(0, 3, (rows_max, n_ff)).astype(np.float16)
    u = rng.normal(0, 1, (rows_max, n_ff)).astype(np.float16)
    out = dev(np.full((rows_max, n_ff), 7.0, np.float16))
    d_rows = dev(np.array([live], np.int32))
    ops.silu_mul_f16_n(dev(g), dev(u), d_rows, out=out)
    got = host(out)
    ref = orc.float_to_half(orc.silu_mul(g[:live].astype(np.float32),
                                         u[:live].astype(np.float32)))
    np.testing.assert_array_equal(got[:live].view(np.uint16), ref)
    assert (got[live:] == 7.0).all()

    nb = n_ff // 256
    q = dev(np.full(rows_max * nb * 276, 0x5A, np.uint8))
    ops.quantize_q8_k_n(out, d_rows, n_ff, rows_max * nb, out=q)
    gq = host(q).reshape(rows_max, nb * 276)
    refq = orc.quantize_q8_k(got[:live].astype(np.float32))
    np.testing.assert_array_equal(gq[:live], refq)
    assert (gq[live:] == 0x5A).all()


@pytest.mark.parametrize("hidden,n_ff,tok_per", [(512, 256, 8), (2048, 512, 64)])
def test_grouped_tab_gemvs_over_plan(hidden, n_ff, tok_per):
    """Plan (sg_moe_dispatch_scan) -> gather -> grouped gate+up -> SiLU ->
    Q8_K of h -> grouped down, each stage against the oracle; expert 3 is
    absent from the gate table (zeroed rows, posted to the mailbox once per
    tile)."""
    rng = np.random.default_rng(5 + hidden)
    E, k, T = 16, 4, 40
    nbh, nbf = hidden // 256, n_ff // 256
    gate = [q4k_random_np(rng, n_ff * nbh) for _ in range(E)]
    up = [q4k_random_np(rng, n_ff * nbh) for _ in range(E)]
    down = [q4k_random_np(rng, hidden * nbf) for _ in range(E)]
    gd = [dev(m) for m in gate]
    ud = [dev(m) for m in up]
    dd = [dev(m) for m in down]
    absent = 3
    tab_g = torch.tensor([0 if e == absent else gd[e].data_ptr() for e in range(E)],
                         dtype=torch.int64, device="cuda")
    tab_u = torch.tensor([t.data_ptr() for t in ud], dtype=torch.int64, device="cuda")
    tab_d = torch.tensor([t.data_ptr() for t in dd], dtype=torch.int64, device="cuda")
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    ids[:6, 0] = absent  # make sure the absent expert has routes
    for t in range(6):   # (distinct ids per row)
        ids[t, 1:] = [e for e in rng.permutation(E) if e != absent][:k - 1]
    idx = np.concatenate([ids, np.full((T, 1), -1, np.int32)], 1)
    w = np.ones((T, k + 1), np.float32)
    plan = ops.moe_dispatch_scan(dev(idx), dev(w), E, k, tok_per=tok_per)
    off, toff, meta = host(plan["off"]), host(plan["toff"]), host(plan["meta"])
    grows = host(plan["grows"])
    R, tiles = int(meta[0]), int(meta[1])
    assert R == T * k

    x = rng.normal(0, 0.002, (T, hidden)).astype(np.float32)  # fp16 outputs stay finite
    xq = orc.quantize_q8_k(x)
    xg = ops.gather_rows_q8(dev(xq), plan["grows"], nbh, meta=plan["meta"], r_max=T * k)
    np.testing.assert_array_equal(host(xg)[:R], xq[grows[:R]])

    tiles_max = tiles + 3  # spare grid rows exit on meta[1]
    yg = dev(np.full((T * k, n_ff), 9.0, np.float16))
    yu = dev(np.full((T * k, n_ff), 9.0, np.float16))
    mail = torch.full((E,), -1, dtype=torch.int32, device="cuda")
    mail_n = torch.zeros(1, dtype=torch.int32, device="cuda")
    ops.gemv_grouped2_tab_q4_k_q8_f16out(tab_g, tab_u, plan, tiles_max, xg, n_ff, hidden, E,
                                         tok_per, yg, yu, mail, mail_n)
    yg_h, yu_h = host(yg), host(yu)
    xg_h = host(xg)
    for e in range(E):
        p0, p1 = int(off[e]), int(off[e + 1])
        if p1 == p0:
            continue
        if e == absent:
            assert (yg_h[p0:p1] == 0).all() and (yu_h[p0:p1] == 0).all()
            continue
        rg = orc.float_to_half(orc.gemv(gate[e], xg_h[p0:p1], n_ff, hidden, p1 - p0))
        ru = orc.float_to_half(orc.gemv(up[e], xg_h[p0:p1], n_ff, hidden, p1 - p0))
        np.testing.assert_array_equal(yg_h[p0:p1].view(np.uint16), rg, err_msg=f"gate e={e}")
        np.testing.assert_array_equal(yu_h[p0:p1].view(np.uint16), ru, err_msg=f"up e={e}")
    n_tiles_absent = int(toff[absent + 1] - toff[absent])
    assert int(host(mail_n)[0]) == n_tiles_absent
    assert (host(mail)[:n_tiles_absent] == absent).all()

    # SiLU and Q8_K of h over the routed rows (device count), then the down pass
    h = ops.silu_mul_f16_n(yg, yu, plan["meta"])
    hq = ops.quantize_q8_k_n(h, plan["meta"], n_ff, T * k * nbf)
    y = dev(np.full((T * k, hidden), 9.0, np.float16))
    ops.gemv_grouped_tab_q4_k_q8_f16out(tab_d, plan, tiles_max, hq.view(T * k, nbf * 276),
                                        hidden, n_ff, E, tok_per, y)
    y_h, hq_h = host(y), host(hq).reshape(T * k, nbf * 276)
    for e in range(E):
        p0, p1 = int(off[e]), int(off[e + 1])
        if p1 == p0:
            continue
        rd = orc.float_to_half(orc.gemv(down[e], hq_h[p0:p1], hidden, n_ff, p1 - p0))
        assert np.isfinite(rd.view(np.float16).astype(np.float32)).all()
        np.testing.assert_array_equal(y_h[p0:p1].view(np.uint16), rd, err_msg=f"down e={e}")


@pytest.mark.parametrize("n_expert,k,hidden", [(256, 8, 2048), (64, 4, 512), (1000, 8, 256)])
def test_router_topk_fused(n_expert, k, hidden):
    """Router GEMV + top-k in one launch against the two launches it fuses
    (sg_gemv_f32_out_f16x, sg_router_topk) and the oracle; three calls in a
    row (the arrival counter resets itself), the shared slot untouched."""
    rng = np.random.default_rng(n_expert + k)
    w = rng.normal(0, 0.05, (n_expert, hidden)).astype(np.float32)
    wd = dev(w)
    for call in range(3):
        x = rng.normal(0, 1, hidden).astype(np.float16)
        xd = dev(x)
        idx = torch.full((k + 1,), -7, dtype=torch.int32, device="cuda")
        wt = torch.full((k + 1,), 5.0, dtype=torch.float32, device="cuda")
        ops.router_topk_fused(wd, xd, k, idx=idx, weight=wt)
        lg = ops.gemv_f32_out_f16x(wd, xd.reshape(1, -1))
        i2, w2 = ops.router_topk(lg[0], k, shared_w=0.25)
        got_i, got_w = host(idx), host(wt)
        np.testing.assert_array_equal(got_i[:k], host(i2)[:k], err_msg=f"call {call}")
        np.testing.assert_array_equal(got_w[:k].view(np.uint32), host(w2)[:k].view(np.uint32))
        assert got_i[k] == -7 and got_w[k] == 5.0
        ref_lg = orc.gemv_f32_lanes(w, x.astype(np.float32))
        np.testing.assert_array_equal(host(lg).view(np.uint32), ref_lg.view(np.uint32))
        ri, rw = orc.router_topk(ref_lg, k)
        np.testing.assert_array_equal(got_i[:k], ri[0, :k])
        np.testing.assert_array_equal(got_w[:k].view(np.uint32), rw[0, :k].view(np.uint32))
