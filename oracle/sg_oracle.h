/* sg_oracle.h - CPU oracle for the quantized MoE decode path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP product
 * library (libsager_hip.so). Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product path never calls it.
 *
 * It restates, in plain C, the reference's CPU semantics for:
 *   - the Q4_K / Q8_K formats          include/sager/kernels/q4_k.hpp:39-118
 *   - Q8_K activation quantization     src/kernels/q4_k.cpp:44-61
 *   - int32 sub-block dots             src/kernels/q4_k.cpp:195-199
 *   - the fp32 Q4_K x Q8_K GEMV        src/kernels/cpu/q4_avx2.cpp:124-145
 *   - the Q6_K format and head GEMV    src/core/weights.cpp:168-209,
 *                                      src/kernels/cuda/q4_k.cu:1578-1652
 *   - the fp32 expert FFN              src/kernels/cpu/q4_avx2.cpp:175-196
 *   - router softmax/top-k/renorm      src/kernels/cuda/moe.cu:25-85
 *   - the fp32 combine                 src/kernels/cuda/moe.cu:265-280
 *   - the MoE layer stage order        src/core/session.cpp:2482-3030
 *   - fp32 x GEMV (router, shared gate) src/kernels/cuda/q4_k.cu:133-149
 *   - the shared-expert sigmoid gate   src/core/session.cpp:2904-2909
 *
 * Every function is pinned by a test (golden vectors from the reference's own
 * CPU sources, closed forms, brute force, or order-free invariants); see the
 * oracle tests under tests/.
 */
#ifndef SG_ORACLE_H
#define SG_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK_K 256
#define ORC_Q4K_BYTES 144
#define ORC_Q8K_BYTES 276
#define ORC_Q6K_BYTES 210

/* fp16 bits -> fp32 (exact). q4_k.hpp:66-88 */
float orc_half_to_float(uint16_t h);
/* 6-bit scale/min of sub-block j (0..7) from the 12 packed bytes. q4_k.hpp:110-118 */
void orc_get_scale_min(int j, const uint8_t* q, uint8_t* d, uint8_t* m);
/* Q4_K row(s) -> fp32 weights. q4_k.cpp:13-42 */
void orc_dequant(const void* w, float* out, int64_t n);

/* fp32 [n_rows][n] -> Q8_K blocks (n % 256 == 0). q4_k.cpp:44-61 */
void orc_quantize_q8_k(const float* x, void* out, int n, int n_rows);

/* int32 dots per sub-block: dots[r][b*8+s] = sum_l nib * xq. q4_k.cpp:195-199 */
void orc_subblock_dots(const void* w, const void* xq, int32_t* dots, int n_rows,
                       int k);

/* y[tok][r] = W[r] . xq[tok], fp32 in the AVX2 order (q4_avx2.cpp:124-145):
 * per super-block sum_s xd*(sd*ip - sm*bsum), then acc += block sum. */
/* Same GEMV with the integer-first super-block epilogue of the prefill
 * path: t = fma(d, (float)sum_s sc*ip, -(dmin * (float)sum_s mn*bsum)),
 * acc = fma(xd, t, acc) per super-block. */
void orc_gemv_q4k_q8_int(const void* w, const void* xq, float* y, int n_rows, int k,
                         int n_tokens);

void orc_gemv_q4k_q8(const void* w, const void* xq, float* y, int n_rows, int k,
                     int n_tokens);

/* Q6_K (210 B per 256 weights, weights.cpp:168-209) -> fp32 weights. */
void orc_dequant_q6k(const void* w6, float* out, int64_t n);
/* int32 sum_j (q6 - 32) * xq over each 16-weight sub-group:
 * dots[r][b*16 + t] (q4_k.cu:1595-1640). */
void orc_q6k_subgroup_dots(const void* w6, const void* xq, int32_t* dots, int n_rows, int k);
/* y[r] = W6[r] . xq (one token) in the order of gemv_q6_k_q8_kernel
 * (q4_k.cu:1578-1652): 32-lane strided sub-groups, fma accumulate, shfl_down tree. */
void orc_gemv_q6k_q8(const void* w6, const void* xq, float* y, int n_rows, int k);

/* exp for float arguments, evaluated in double and rounded once (stands in
 * for std::exp(float) of q4_avx2.cpp:189 and expf of moe.cu:38-43). */
float orc_expf(float x);
/* h = g/(1+exp(-g))*u, the fp32 chain of q4_avx2.cpp:187-191 */
void orc_silu_mul(const float* g, const float* u, float* h, int n);

/* Full fp32 expert FFN on one token. q4_avx2.cpp:175-196 */
void orc_expert_ffn(const void* wg, const void* wu, const void* wd,
                    const float* x, float* y, int hidden, int n_ff);

/* Router: softmax, k rounds of first-strict-max (NaN skipped, lower index
 * wins ties), renormalize, weight[k] = shared_w. Outputs use stride `stride`
 * (>= k+1). moe.cu:25-85, 165-234 */
void orc_router_topk(const float* logits, int* idx, float* weight, int n_expert,
                     int k, int stride, int n_rows, float shared_w);

/* out[r][i] = residual[r][i] + sum_{kk=0..n_used} w[r][kk]*y[r][kk][i], fp32,
 * kk order. out may alias residual. moe.cu:265-280 */
void orc_moe_combine(float* out, const float* residual, const float* expert_y,
                     const float* weight, int n_used, int hidden, int n_rows);

/* y[t][r] = W[r] . x[t], W fp32 [n_rows][k], x fp32 [n_tokens][k], in the
 * reference kernel's order (q4_k.cu:133-149): 32 lane-strided fma chains,
 * then the shfl_down tree 16, 8, 4, 2, 1. */
void orc_gemv_f32_lanes(const float* w, const float* x, float* y, int n_rows, int k,
                        int n_tokens);
/* 1 / (1 + exp(-g)) with orc_expf. */
float orc_sigmoid(float g);

/* One MoE layer for n_tokens tokens, device-path stage order
 * (session.cpp:2482-3030): quantize x, route, each routed expert and the
 * shared expert through orc_expert_ffn semantics, combine with slot k =
 * shared (weight shared_w). tab_* are [n_expert] pointers; sh_* may be NULL
 * (no shared expert: slot k contributes 0). residual may be NULL (= 0).
 * idx/weight outputs: [n_tokens][k+1]. n_threads > 1 runs the expert jobs
 * on a worker pool (same results).  sh_gate_w (fp32 [hidden] or NULL):
 * the shared output of token t is multiplied by
 * orc_sigmoid(orc_gemv_f32_lanes(sh_gate_w, x[t])) before the combine
 * (session.cpp:2904-2909); ignored without a shared expert. */
void orc_moe_layer(const void* const* tab_gate, const void* const* tab_up,
                   const void* const* tab_down, const void* sh_gate,
                   const void* sh_up, const void* sh_down, const float* sh_gate_w,
                   const float* x, const float* logits, const float* residual, float* out,
                   int* idx, float* weight, int n_tokens, int hidden, int n_ff,
                   int n_expert, int k, float shared_w, int n_threads);

/* Prefill layer: orc_moe_layer's routing/experts/combine with every GEMV
 * in the integer-first order (orc_gemv_q4k_q8_int).  logits may be NULL
 * (idx/weight then inputs). */
void orc_moe_prefill(const void* const* tab_gate, const void* const* tab_up,
                     const void* const* tab_down, const void* sh_gate, const void* sh_up,
                     const void* sh_down, const float* sh_gate_w, const float* x,
                     const float* logits, const float* residual, float* out, int* idx,
                     float* weight, int n_tokens, int hidden, int n_ff, int n_expert, int k,
                     float shared_w, int n_threads);

/* fp32 -> fp16 bits, round to nearest even (__float2half). */
uint16_t orc_float_to_half(float f);
void orc_float_to_half_n(const float* x, uint16_t* h, int64_t n);

/* The layer on the session's fp16 buffers (x: fp16 values of xn as floats,
 * residual: fp16 values or NULL, out: the fp16-rounded result as floats):
 * slot outputs stored as fp16, the shared slot gated on its fp16 value,
 * moe_combine_batched_f16's fp32 accumulation and fp16 store
 * (moe.cu:249-292).  logits may be NULL (idx/weight then inputs);
 * int_first selects the prefill's GEMV order. */
void orc_moe_layer_f16io(const void* const* tab_gate, const void* const* tab_up,
                         const void* const* tab_down, const void* sh_gate, const void* sh_up,
                         const void* sh_down, const float* sh_gate_w, const float* x,
                         const float* logits, const float* residual, float* out, int* idx,
                         float* weight, int n_tokens, int hidden, int n_ff, int n_expert, int k,
                         float shared_w, int n_threads, int int_first);

/* Same as orc_moe_layer but with routing given (idx/weight [n_tokens][k+1]
 * already filled, e.g. sampled routing); no softmax. */
void orc_moe_layer_routed(const void* const* tab_gate,
                          const void* const* tab_up,
                          const void* const* tab_down, const void* sh_gate,
                          const void* sh_up, const void* sh_down, const float* sh_gate_w,
                          const float* x, const int* idx, const float* weight,
                          const float* residual, float* out, int n_tokens,
                          int hidden, int n_ff, int n_expert, int k,
                          int n_threads);

/* Device-plan semantics of moe_dispatch_scan (moe.cu:366-444), made
 * deterministic: routes ordered by (expert, row, kk). off/toff [n_expert+1],
 * meta {R, tiles, bad}, gslot [n_rows*k], grows [n_rows*k]. Bad ids zero
 * that row's weights (stride k+1). */
void orc_dispatch_scan(const int* idx, float* weight, int* gslot, int* grows,
                       int* off, int* toff, int* meta, int n_rows, int k,
                       int n_expert, int tok_per);

/* Test helper: number of x in a sample where orc_expf(x) != libm expf(x). */
int64_t orc_count_expf_mismatch(int64_t n_samples, uint64_t seed, float lo,
                                float hi);
/* Test helper: 1 if this build took the AVX2 integer-dot path. */
int orc_have_avx2(void);

#ifdef __cplusplus
}
#endif
#endif /* SG_ORACLE_H */
