"""GGUF v3 expert loading: the host parser (CPU) and the Q4_K requantizer
against the reference's own quantize_row outputs (golden, bit-exact)."""
import os

import numpy as np
import pytest

from sager_amd import ops
from gguf_writer import ARRAY, BOOL, F32, F64, I8, I16, I32, I64, STRING, U8, U16, U32, U64
from gguf_writer import expert_file, write_gguf


GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "q4k_golden.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN)


@pytest.mark.parametrize("case", ["gauss", "q6", "edge"])
def test_q4k_quantize_row_bit_exact_vs_reference(gold, case):
    """The loader's requantizer equals the reference's quantize_row
    (q4_k.cpp:62-174) byte for byte: gaussian rows, rows dequantized from
    Q6_K, and edge rows (constant sub-blocks, zeros, spikes, one-sided and
    extreme ranges)."""
    x, q = gold[f"requant_{case}_x"], gold[f"requant_{case}_q"]
    np.testing.assert_array_equal(ops.q4k_quantize_row(x), q)


def test_gguf_expert_dims_reads_every_kv_type(tmp_path):
    rng = np.random.default_rng(1)
    kvs = [("k.u8", U8, 7), ("k.i8", I8, -3), ("k.u16", U16, 65535), ("k.i16", I16, -2),
           ("k.u32", U32, 1 << 31), ("k.i32", I32, -5), ("k.f32", F32, 1.5), ("k.bool", BOOL, True),
           ("k.str", STRING, "hello"), ("k.u64", U64, 1 << 40), ("k.i64", I64, -7),
           ("k.f64", F64, 2.25), ("k.arr", ARRAY, (U32, [1, 2, 3])),
           ("k.strs", ARRAY, (STRING, ["a", "bc", ""]))]
    p = tmp_path / "m.gguf"
    expert_file(p, rng, 3, 4, 256, 512, q6_down=(1,), alignment=64, extra_kvs=kvs)
    assert ops.gguf_expert_dims(p) == (3, 4, 256, 512, 1)


def test_gguf_rejects_malformed_files(tmp_path):
    rng = np.random.default_rng(2)
    good = tmp_path / "good.gguf"
    expert_file(good, rng, 2, 2, 256, 256)
    raw = good.read_bytes()
    cases = {
        "magic": b"GGUX" + raw[4:],
        "version": raw[:4] + (2).to_bytes(4, "little") + raw[8:],
        "truncated": raw[: len(raw) // 3],
        "tensor past end": raw[: len(raw) - 100],
    }
    for name, data in cases.items():
        p = tmp_path / f"{name.replace(' ', '_')}.gguf"
        p.write_bytes(data)
        with pytest.raises(ops.SagerError):
            ops.gguf_expert_dims(p)
    with pytest.raises(ops.SagerError, match="status 2"):
        ops.gguf_expert_dims(tmp_path / "missing.gguf")


def test_gguf_rejects_inconsistent_experts(tmp_path):
    from sager_amd.synth import q4k_random_np
    rng = np.random.default_rng(3)
    g = q4k_random_np(rng, 2 * 256 * 256 // 256).tobytes()
    # down with the wrong shape
    p = tmp_path / "shape.gguf"
    write_gguf(p, [], [("blk.0.ffn_gate_exps", (256, 256, 2), 12, g),
                       ("blk.0.ffn_up_exps", (256, 256, 2), 12, g),
                       ("blk.0.ffn_down_exps", (256, 512, 1), 12, g)])
    with pytest.raises(ops.SagerError, match="status 4"):
        ops.gguf_expert_dims(p)
    # an F32 gate
    p = tmp_path / "type.gguf"
    f32 = np.zeros(256 * 256 * 2, np.float32).tobytes()
    write_gguf(p, [], [("blk.0.ffn_gate_exps", (256, 256, 2), 0, f32),
                       ("blk.0.ffn_up_exps", (256, 256, 2), 12, g),
                       ("blk.0.ffn_down_exps", (256, 256, 2), 12, g)])
    with pytest.raises(ops.SagerError, match="status 8"):
        ops.gguf_expert_dims(p)
    # no expert tensors at all
    p = tmp_path / "none.gguf"
    write_gguf(p, [], [("token_embd.weight", (256, 1), 0, np.zeros(256, np.float32).tobytes())])
    with pytest.raises(ops.SagerError, match="status 3"):
        ops.gguf_expert_dims(p)


# ---- the pool on the GPU -------------------------------------------------------

@pytest.mark.gpu
def test_expert_pool_from_gguf(tmp_path):
    """Load a 3-layer, 16-expert file (layer 1's down projection in Q6_K) into
    HBM; every expert matrix behind the pointer table reproduces the file's
    bytes (or the requantized Q6_K rows) - checked through the pointer-table
    GEMV against the oracle - and a layer run on the pool's tables matches
    the oracle's MoE layer on the file's weights."""
    import torch
    from oracle import oracle as orc
    rng = np.random.default_rng(9)
    L, E, H, F, K = 3, 16, 512, 256, 4
    path = tmp_path / "experts.gguf"
    data = expert_file(path, rng, L, E, H, F, q6_down=(1,), alignment=64)
    pool = ops.ExpertPool(path)
    assert (pool.n_layers, pool.n_expert, pool.hidden, pool.n_ff) == (L, E, H, F)
    x = rng.normal(0, 1, H).astype(np.float32)
    xh = rng.normal(0, 1, F).astype(np.float32)
    xq, xqh = orc.quantize_q8_k(x), orc.quantize_q8_k(xh)
    expect = {}
    for l in range(L):
        tabs = pool.layer_tables(l)
        for m in range(3):
            w = data[(l, m)]
            if m == 2 and l == 1:  # Q6_K in the file: requantized at load
                w = ops.q4k_quantize_row(orc.dequant_q6k(w, E * H * F))
            w = w.reshape(E, -1, 144)
            expect[(l, m)] = w
            rows, k, xm = (F, H, xq) if m < 2 else (H, F, xqh)
            y = ops.gemv_ptrs_q4_k_q8(tabs[m], torch.from_numpy(xm).cuda(), E, rows, k)
            ref = np.concatenate([orc.gemv(w[e], xm, rows, k)[0] for e in range(E)])
            np.testing.assert_array_equal(y.cpu().numpy(), ref)
    # one decode token through layer 2 on the pool's tables
    xl = rng.normal(0, 1, (1, H)).astype(np.float32)
    lg = rng.normal(0, 1, (1, E)).astype(np.float32)
    layer = ops.MoeLayer(*pool.layer_tables(2), None, hidden=H, n_ff=F, n_expert=E, k=K)
    out, idx, w = layer.forward(torch.from_numpy(xl).cuda(), torch.from_numpy(lg).cuda())
    ref, ri, rw = orc.moe_layer([expect[(2, 0)][e] for e in range(E)],
                                [expect[(2, 1)][e] for e in range(E)],
                                [expect[(2, 2)][e] for e in range(E)], None, xl, logits=lg,
                                hidden=H, n_ff=F, k=K)
    np.testing.assert_array_equal(idx.cpu().numpy()[:, :K], ri[:, :K])
    np.testing.assert_array_equal(out.cpu().numpy(), ref)
    pool.close()
