"""Write tests/golden/q4k_golden.npz from the reference's own CPU sources.

Run in the build container (where /root/reference exists) after
`make -C oracle ref`, which compiles the reference's
src/kernels/q4_k.cpp and src/kernels/cpu/q4_avx2.cpp (with the reference's
Release flags) plus oracle/ref_shim.cpp into oracle/_ref/libsager_ref.so.

The fixture holds only data: seeded inputs and the outputs the reference's
functions produced for them. The tests compare the oracle (and, on the GPU,
the HIP library) against these arrays; nothing from the reference travels.

Reference functions exercised (all under /root/reference):
  half_to_float        include/sager/kernels/q4_k.hpp:66-88
  get_scale_min_k4     include/sager/kernels/q4_k.hpp:110-118
  dequant_row          src/kernels/q4_k.cpp:13-42
  quantize_row_q8_K    src/kernels/q4_k.cpp:44-61
  quantize_row (Q4_K)  src/kernels/q4_k.cpp:68-174   (realistic weights)
  vec_dot_ref          src/kernels/q4_k.cpp:176-207
  quantize_row_q8_k_avx2, gemv_q4_k_q8_avx2, gemv_q4_k_q8_scalar,
  expert_ffn_q4        src/kernels/cpu/q4_avx2.cpp:47-196

Usage:  python tests/golden/make_golden.py
"""
import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libsager_ref.so")
OUT = os.path.join(HERE, "q4k_golden.npz")


def P(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def orc_dequant_q6k(w6, n):
    """Q6_K -> fp32 through the repository's oracle (input generation only)."""
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", ".."))
    from oracle import oracle as orc
    return orc.dequant_q6k(w6, n)


def random_q4k(rng, n_blocks):
    """Synthetic Q4_K blocks as the configs specify: fp16 d, dmin from
    |N(0, 0.02)|, 12 uniform random scale bytes, 128 uniform random qs bytes."""
    b = rng.integers(0, 256, size=(n_blocks, 144), dtype=np.uint8)
    dd = np.abs(rng.normal(0.0, 0.02, size=(n_blocks, 2))).astype(np.float16)
    b[:, 0:4] = dd.view(np.uint8).reshape(n_blocks, 4)
    return b


def main():
    if not os.path.exists(REF_SO):
        sys.exit("build the reference shim first: make -C oracle ref")
    ref = ctypes.CDLL(REF_SO)
    ref.ref_half_to_float.restype = ctypes.c_float
    ref.ref_half_to_float.argtypes = [ctypes.c_uint16]
    ref.ref_vec_dot.restype = ctypes.c_float
    rng = np.random.default_rng(20261201)
    g = {}

    # fp16 -> fp32 over every bit pattern.
    g["half_f32_bits"] = np.array(
        [np.float32(ref.ref_half_to_float(h)).view(np.uint32) for h in range(65536)],
        dtype=np.uint32)

    # 6-bit scale/min unpack on random packed bytes.
    sb = rng.integers(0, 256, size=(1000, 12), dtype=np.uint8)
    sv = np.zeros((1000, 8, 2), dtype=np.uint8)
    d = ctypes.c_uint8()
    m = ctypes.c_uint8()
    for i in range(1000):
        row = np.ascontiguousarray(sb[i])
        for j in range(8):
            ref.ref_get_scale_min(j, P(row), ctypes.byref(d), ctypes.byref(m))
            sv[i, j] = (d.value, m.value)
    g["scale_bytes"], g["scale_vals"] = sb, sv

    # Q8_K quantization: N(0,1) rows plus edge rows.
    K = 2048
    rows = [rng.normal(0, 1, K).astype(np.float32) for _ in range(6)]
    rows.append(np.zeros(K, np.float32))                                  # all zero
    rows.append((rng.integers(-254, 255, K) * 0.5).astype(np.float32))    # .5 ties
    rows.append((rng.normal(0, 1, K) * 1e30).astype(np.float32))          # huge
    rows.append((rng.normal(0, 1, K) * 1e-38).astype(np.float32))         # tiny
    rows.append(rng.normal(0, 0.6, K).astype(np.float16).astype(np.float32))  # fp16 inputs
    r = np.full(K, 3.0, np.float32)
    r[::256] = -127.0
    rows.append(r)                                                        # exact grid
    xq_in = np.ascontiguousarray(np.stack(rows))
    n_r = xq_in.shape[0]
    q8 = np.zeros((n_r, (K // 256) * 276), np.uint8)
    q8b = np.zeros_like(q8)
    for i in range(n_r):
        xi = np.ascontiguousarray(xq_in[i])
        oi = np.zeros(q8.shape[1], np.uint8)
        ob = np.zeros(q8.shape[1], np.uint8)
        ref.ref_quantize_q8_k(P(xi), P(oi), K)
        ref.ref_quantize_q8_k_avx2(P(xi), P(ob), K)
        q8[i], q8b[i] = oi, ob
    g["q8_x"], g["q8_out"], g["q8_out_avx2"] = xq_in, q8, q8b

    def q8_of(x):
        out = np.zeros((x.shape[0], (x.shape[1] // 256) * 276), np.uint8)
        for i in range(x.shape[0]):
            xi = np.ascontiguousarray(x[i])
            oi = np.zeros(out.shape[1], np.uint8)
            ref.ref_quantize_q8_k(P(xi), P(oi), x.shape[1])
            out[i] = oi
        return out

    def gemv_case(name, w, n_rows, k, x):
        xq = q8_of(x)
        y = np.zeros((x.shape[0], n_rows), np.float32)
        ys = np.zeros_like(y)
        for t in range(x.shape[0]):
            yt = np.zeros(n_rows, np.float32)
            yst = np.zeros(n_rows, np.float32)
            xt = np.ascontiguousarray(xq[t])
            ref.ref_gemv_avx2(P(w), P(xt), P(yt), n_rows, k)
            ref.ref_gemv_scalar(P(w), P(xt), P(yst), n_rows, k)
            y[t], ys[t] = yt, yst
        vd = np.zeros(n_rows, np.float32)
        nb = k // 256
        xt = np.ascontiguousarray(xq[0])
        for rr in range(n_rows):
            wr = np.ascontiguousarray(w.reshape(n_rows, nb * 144)[rr])
            vd[rr] = ref.ref_vec_dot(P(wr), P(xt), k)
        g[name + "_w"], g[name + "_x"], g[name + "_xq"] = w, x, xq
        g[name + "_y"], g[name + "_y_scalar"], g[name + "_vecdot"] = y, ys, vd
        g[name + "_shape"] = np.array([n_rows, k], np.int32)

    # gate/up shape slice (K=2048), down shape slice (K=512), odd row count.
    gemv_case("gemv_a", random_q4k(rng, 128 * 8), 128, 2048,
              rng.normal(0, 1, (3, 2048)).astype(np.float32))
    gemv_case("gemv_b", random_q4k(rng, 257 * 2), 257, 512,
              rng.normal(0, 1, (2, 512)).astype(np.float32))
    # realistic weights from the reference's own Q4_K quantizer
    wf = (rng.normal(0, 1, 64 * 2048) * 0.05).astype(np.float32)
    wq = np.zeros((64 * 8, 144), np.uint8)
    ref.ref_quantize_row_q4k(P(wf), P(wq), wf.size)
    deq = np.zeros(wf.size, np.float32)
    ref.ref_dequant(P(wq), P(deq), wf.size)
    g["real_dequant"] = deq
    gemv_case("gemv_c", wq, 64, 2048, rng.normal(0, 1, (2, 2048)).astype(np.float32))

    # Expert FFN, hidden 2048, n_ff 256 (gate/up [256x2048], down [2048x256]).
    H, F = 2048, 256
    wg = random_q4k(rng, F * H // 256)
    wu = random_q4k(rng, F * H // 256)
    wd = random_q4k(rng, H * F // 256)
    xs = rng.normal(0, 1, (3, H)).astype(np.float32)
    ys = np.zeros((3, H), np.float32)
    scratch = np.zeros(2 * F, np.float32)
    for t in range(3):
        xt = np.ascontiguousarray(xs[t])
        yt = np.zeros(H, np.float32)
        ref.ref_expert_ffn(P(wg), P(wu), P(wd), P(xt), P(yt), P(scratch), H, F)
        ys[t] = yt
    g["ffn_wg"], g["ffn_wu"], g["ffn_wd"] = wg, wu, wd
    g["ffn_x"], g["ffn_y"] = xs, ys
    g["ffn_shape"] = np.array([H, F], np.int32)

    # Q4_K requantization (the GGUF loader's path for Q6_K expert tensors):
    # fp32 rows -> quantize_row.  Its own seed, so the cases above keep their
    # values.  Rows: gaussian weights, weights dequantized from random Q6_K
    # blocks, and edge rows (constant sub-blocks, zeros, one spike, a
    # one-sided range, large magnitudes).
    rq = np.random.default_rng(20261202)
    gauss = (rq.normal(0, 1, 16 * 2048) * 0.05).astype(np.float32)
    q6 = rq.integers(0, 256, size=(64, 210), dtype=np.uint8)
    q6[:, 208:210] = np.abs(rq.normal(0, 0.002, (64, 1))).astype(np.float16).view(np.uint8)
    from_q6 = orc_dequant_q6k(q6, 64 * 256)
    edge = np.zeros(8 * 256, np.float32)
    edge[0:32] = 0.25                                         # constant sub-block
    edge[256:512] = rq.normal(0, 1, 256).astype(np.float32)
    edge[300] = 40.0                                          # spike
    edge[512:768] = np.abs(rq.normal(0, 1, 256)).astype(np.float32) + 3.0  # positive only
    edge[768:1024] = -np.abs(rq.normal(0, 1, 256)).astype(np.float32)     # negative only
    edge[1024:1280] = (rq.normal(0, 1, 256) * 1e4).astype(np.float32)     # large
    edge[1280:1536] = (rq.normal(0, 1, 256) * 1e-6).astype(np.float32)    # tiny
    # 1536..2047 stay zero (an all-zero super-block)
    for name, x in (("gauss", gauss), ("q6", from_q6), ("edge", edge)):
        x = np.ascontiguousarray(x, np.float32)
        q = np.zeros((x.size // 256, 144), np.uint8)
        ref.ref_quantize_row_q4k(P(x), P(q), x.size)
        g["requant_" + name + "_x"], g["requant_" + name + "_q"] = x, q

    np.savez_compressed(OUT, **g)
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
