/* sager_hip.h - C ABI of libsager_hip.so, the MI355X (gfx950) implementation
 * of SAGER's quantized MoE decode hot path.
 *
 * This header is the drop-in boundary. It replaces the hot subset of the
 * reference's launcher API `namespace sager::cuda` in
 * include/sager/kernels/cuda_ops.hpp (the "ONLY surface the session loop
 * sees", cuda_ops.hpp:1-7) with extern "C" functions on plain pointers:
 *
 *   - every pointer argument is a DEVICE pointer unless stated otherwise;
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream);
 *   - every call is stream-ordered and never synchronizes (cuda_ops.hpp:4-6);
 *   - the caller owns every buffer; no function allocates device memory
 *     (the fused layer takes a caller-provided workspace);
 *   - the return value is a status (0 = ok) instead of the reference's
 *     `void` + cudaGetLastError; sg_last_error() gives the message of the
 *     last failure on the calling thread.
 *
 * Formats (include/sager/kernels/q4_k.hpp:39-62), both byte-packed:
 *   sg_block_q4k: 256 weights in 144 B  - fp16 d | fp16 dmin | 12 B packed
 *                 6-bit scales/mins | 128 B nibbles (group g = bytes
 *                 32g..32g+31: low nibbles are sub-block 2g, high 2g+1).
 *   sg_block_q8k: 256 activations in 276 B - fp32 d | 256 x int8 |
 *                 8 x int16 sub-block sums.
 * A matrix is n_rows x (k/256) blocks, row-major; k must be a multiple of
 * 256. Activation rows are k/256 consecutive Q8_K blocks per token.
 */
#ifndef SAGER_HIP_H
#define SAGER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#pragma pack(push, 1)
typedef struct sg_block_q4k {
  uint16_t d;
  uint16_t dmin;
  uint8_t scales[12];
  uint8_t qs[128];
} sg_block_q4k;

typedef struct sg_block_q8k {
  float d;
  int8_t qs[256];
  int16_t bsums[8];
} sg_block_q8k;
#pragma pack(pop)

/* Status codes; numeric values follow sager::Status (common.hpp:68-79). */
enum {
  SG_OK = 0,
  SG_ERR_INVALID_ARGUMENT = 1,
  SG_ERR_FILE_NOT_FOUND = 2,
  SG_ERR_GGUF_PARSE = 3,
  SG_ERR_GEOMETRY = 4,
  SG_ERR_OOM_VRAM = 5,
  SG_ERR_HIP = 7,
  SG_ERR_UNSUPPORTED = 8
};

/* Message of the last non-zero status returned on this thread ("" if none). */
const char* sg_last_error(void);
/* Library version string. */
const char* sg_version(void);

/* ---- Q8_K activation quantization ------------------------------------
 * out[r] = Q8_K(x[r]) for n_rows rows of n values (n % 256 == 0):
 * per block amax (start 1e-30), d = amax/127, q = round-half-even(x/d)
 * clamped to +-127, bsums = per-32 sums.  Bit-exact with
 * quantize_row_q8_K (q4_k.cpp:44-61).
 * Replaces cuda::quantize_q8_k (cuda_ops.hpp:271-273), which takes fp16
 * input; this one takes fp32 rows (the CPU chain's input, q4_avx2.cpp:180). */
int sg_quantize_q8_k(const float* x, sg_block_q8k* out, int n, int n_rows,
                     void* stream);
/* fp16 input, the exact argument meaning of cuda::quantize_q8_k. */
int sg_quantize_q8_k_f16(const uint16_t* x, sg_block_q8k* out, int n,
                         int n_rows, void* stream);

/* ---- Q4_K x Q8_K GEMV family -----------------------------------------
 * Row result, fp32, in the reference CPU order (q4_avx2.cpp:124-145 as
 * built): per super-block sum_s fma(xd, fma(sd, ip_s, -(sm*bsum_s)), .),
 * then the block sums added in block order. */

/* y[r] = W[r] . x.  Replaces cuda::gemv_q4_k_q8 (cuda_ops.hpp:41-42). */
int sg_gemv_q4_k_q8(const sg_block_q4k* w, const sg_block_q8k* x, float* y,
                    int n_rows, int k, void* stream);

/* y[t*n_rows + r] = W[r] . x[t] for t < n_tokens (1..16); each weight row is
 * read once for all tokens.  Replaces cuda::gemv_q4_k_q8_batched
 * (cuda_ops.hpp:72-74) and the mtok tiled variants (cuda_ops.hpp:88-90). */
int sg_gemv_q4_k_q8_batched(const sg_block_q4k* w, const sg_block_q8k* x,
                            float* y, int n_rows, int k, int n_tokens,
                            void* stream);
/* The same with fp16 y.  Replaces cuda::gemv_q4_k_q8_f16out_batched
 * (cuda_ops.hpp:67-70). */
int sg_gemv_q4_k_q8_f16out_batched(const sg_block_q4k* w, const sg_block_q8k* x,
                                   uint16_t* y, int n_rows, int k, int n_tokens,
                                   void* stream);

/* ---- dense-projection GEMVs (fp16 outputs) ---------------------------
 * The same Q4_K x Q8_K row dot (bit-identical to sg_gemv_q4_k_q8), rounded
 * to fp16 (nearest even).  Replaces cuda::gemv_q4_k_q8_f16out
 * (cuda_ops.hpp:53-54). */
int sg_gemv_q4_k_q8_f16out(const sg_block_q4k* w, const sg_block_q8k* x, uint16_t* y,
                           int n_rows, int k, void* stream);
/* The layer's two (GDN qkvz | ba) or three (GQA q | k | v) projections of
 * one x in ONE launch: y_m[r] = f16(W_m[r] . x), rows_m rows each.  Replaces
 * cuda::gemv2m / gemv3m_q4_k_q8_f16out (cuda_ops.hpp:156-164); the
 * reference's graph-parameter `slot` has no counterpart (nothing is stored
 * per layer). */
int sg_gemv2m_q4_k_q8_f16out(const sg_block_q4k* w1, const sg_block_q4k* w2,
                             const sg_block_q8k* x, uint16_t* y1, uint16_t* y2, int rows1,
                             int rows2, int k, void* stream);
int sg_gemv3m_q4_k_q8_f16out(const sg_block_q4k* w1, const sg_block_q4k* w2,
                             const sg_block_q4k* w3, const sg_block_q8k* x, uint16_t* y1,
                             uint16_t* y2, uint16_t* y3, int rows1, int rows2, int rows3,
                             int k, void* stream);
/* y[r] = f16(W[r] . x) and res_inout[r] = f16(f32(res_inout[r]) + f32(y[r]))
 * (add_kernel's semantics) in one launch.  Replaces
 * cuda::gemv_q4_k_q8_f16out_resadd (cuda_ops.hpp:166-171). */
int sg_gemv_q4_k_q8_f16out_resadd(const sg_block_q4k* w, const sg_block_q8k* x, uint16_t* y,
                                  uint16_t* res_inout, int n_rows, int k, void* stream);

/* Q6_K x Q8_K GEMV (the real model's LM head).  w6 points at raw
 * block_q6_K bytes (210 per 256 weights: ql[128] | qh[64] | int8 sc[16] |
 * fp16 d, weights.cpp:168-209); y[r] fp32 for r < n_rows.  The fp32 order
 * is the reference kernel's (q4_k.cu:1578-1652): per row 32 lanes, lane l
 * accumulating sub-groups l, l+32, ... as fma((xd*d)*sc, (float)isum, acc),
 * then the shfl_down tree.  k <= 8192; the matrix must be under 2 GiB.  Replaces
 * cuda::gemv_q6_k_q8 (cuda_ops.hpp:44-48) and its x-in-shared twin
 * gemv_q6_k_q8_smx (cuda_ops.hpp:179-182). */
int sg_gemv_q6_k_q8(const void* w6, const sg_block_q8k* x, float* y, int n_rows,
                    int k, void* stream);

/* Pointer-table GEMV: row r is row (r % rows_per) of matrix ptrs[r/rows_per]
 * (ptrs is a DEVICE array of n_ptrs device pointers); y[r] fp32 for
 * r < n_ptrs*rows_per.  Replaces cuda::gemv_ptrs_q4_k_q8_f16out
 * (cuda_ops.hpp:60-63) with an fp32 output. */
int sg_gemv_ptrs_q4_k_q8(const sg_block_q4k* const* ptrs,
                         const sg_block_q8k* x, float* y, int n_ptrs,
                         int rows_per, int k, void* stream);
/* The same with fp16 y (the fp32 row result rounded to nearest even), the
 * argument meaning of cuda::gemv_ptrs_q4_k_q8_f16out (cuda_ops.hpp:60-63,
 * q4_k.cu:184-213). */
int sg_gemv_ptrs_q4_k_q8_f16out(const sg_block_q4k* const* ptrs,
                                const sg_block_q8k* x, uint16_t* y, int n_ptrs,
                                int rows_per, int k, void* stream);

/* Test hook: the int32 sub-block dot sums the GEMVs use,
 * dots[(r*(k/256) + b)*8 + s] = sum_l nibble * xq for sub-block s of block b.
 * No launcher counterpart; the device routine it exposes is the reference's
 * dp4a_subblock (q4_k.cu:38-53). */
int sg_q4k_subblock_dots(const sg_block_q4k* w, const sg_block_q8k* x,
                         int32_t* dots, int n_rows, int k, void* stream);

/* ---- router, SiLU, combine -------------------------------------------- */

/* Per row: softmax over n_expert logits, n_expert_used rounds of argmax
 * (NaN skipped, lower index wins ties), weights renormalized by their sum,
 * weight[row*idx_stride + n_expert_used] = shared_w.  idx/weight rows have
 * stride idx_stride >= n_expert_used + 1.  n_expert <= 1024.
 * Replaces cuda::router_topk / router_topk_batched (cuda_ops.hpp:351-360),
 * moe.cu:25-85, 165-234. */
int sg_router_topk(const float* logits, int* idx, float* weight, int n_expert,
                   int n_expert_used, int idx_stride, int n_rows,
                   float shared_w, void* stream);

/* out[i] = g[i] / (1 + exp(-g[i])) * u[i], fp32 (q4_avx2.cpp:187-191).
 * Replaces cuda::silu_mul_f16 (cuda_ops.hpp:305-306) with fp32 buffers. */
int sg_silu_mul(float* out, const float* g, const float* u, int n,
                void* stream);

/* out[r][i] = residual[r][i] + sum_{kk=0..n_used} weight[r][kk] *
 * expert_y[r][kk][i] (one fma per slot, kk order); weight rows have stride
 * n_used+1 and expert_y is [n_rows][n_used+1][hidden]. residual may be NULL
 * (zero) and may alias out.  Replaces cuda::moe_combine_batched_f16
 * (cuda_ops.hpp:397-399, moe.cu:265-280) with fp32 buffers. */
int sg_moe_combine(float* out, const float* residual, const float* expert_y,
                   const float* weight, int n_used, int hidden, int n_rows,
                   void* stream);

/* Router GEMV (fp32 W [n_expert][hidden] times the fp16 x of one token) and
 * top-k in one launch: the logits bit for bit sg_gemv_f32_out_f16x's, the
 * selection and weights sg_router_topk's; writes idx[0..k) and
 * weight[0..k) only (the shared slot is left as it is).  Uses a file-scope
 * device array of logits and an arrival counter per GPU: calls that overlap
 * on one GPU race.  n_expert <= 1024, n_expert_used <= 64.  Replaces
 * cuda::router_topk_fused (cuda_ops.hpp:173-177, mmq.cu:459-522). */
int sg_router_topk_fused(const float* w, const uint16_t* x, int* idx, float* weight,
                         int n_expert, int n_expert_used, int hidden, void* stream);

/* ---- fp16-buffer launchers (the session loop's own buffers) ------------
 * fp16 values are IEEE binary16 bits; every conversion to fp16 rounds to
 * nearest even (__float2half), conversions to fp32 are exact. */

/* out[i] = f16(g/(1+exp(-g))*u) over rows*n_ff values, g, u fp16.
 * Replaces cuda::silu_mul_f16 (cuda_ops.hpp:305-306, norm_rotary.cu:133-141). */
int sg_silu_mul_f16(uint16_t* out, const uint16_t* g, const uint16_t* u, int rows, int n_ff,
                    void* stream);

/* out[r][i] = f16(f32(out[r][i]) + sum_{kk=0..n_used} fma(weight[r][kk],
 * f32(expert_y[r][kk][i]), .)) in kk order; out holds the residual on entry.
 * weight rows have stride n_used+1, expert_y is fp16 [n_rows][n_used+1][hidden].
 * Replaces cuda::moe_combine_batched_f16 (cuda_ops.hpp:379-381,
 * moe.cu:265-280). */
int sg_moe_combine_batched_f16(uint16_t* out, const uint16_t* expert_y, const float* weight,
                               int n_used, int hidden, int n_rows, void* stream);

/* out[i] *= sigmoid(g[0]) on fp16 out[n] (the shared expert's scalar gate,
 * fp32 logit g).  Replaces cuda::sigmoid_gate_scalar_f16 (cuda_ops.hpp:315-316,
 * norm_rotary.cu:177-184). */
int sg_sigmoid_gate_scalar_f16(uint16_t* out, const float* g, int n, void* stream);
/* out[r*hidden + i] *= sigmoid(g[r]).  Replaces
 * cuda::sigmoid_gate_scalar_batched_f16 (cuda_ops.hpp:384-386, moe.cu:282-292). */
int sg_sigmoid_gate_scalar_batched_f16(uint16_t* out, const float* g, int n_rows, int hidden,
                                       void* stream);

/* y[t*n_rows + r] = sum_i w[r][i] * f32(x[t][i]) for W fp32 [n_rows][k] and
 * x fp16 [n_tokens][k]: the router logits and the shared-expert gate logit.
 * Per row, lane l of 32 accumulates i = l, l+32, ... with fma, then a
 * shfl_down tree (16, 8, 4, 2, 1): the reference kernel's order
 * (q4_k.cu:133-149, 285-303; the mtok variant keeps the same order,
 * q4_k.cu:1434-1438).  Replaces cuda::gemv_f32_out_f16x (n_tokens = 1) and
 * gemv_f32_out_f16x_batched / _mtok. */
int sg_gemv_f32_out_f16x(const float* w, const uint16_t* x, float* y, int n_rows, int k,
                         int n_tokens, void* stream);

/* ---- fused MoE layer (decode step / verify window) --------------------
 * One MoE layer for n_tokens (1..16) tokens, in the stage order of the
 * reference's device path Session::moe_dispatch_device
 * (session.cpp:2482-3030): Q8_K(x) -> router top-k -> every routed expert
 * and the shared expert as gate/up GEMV, h = SiLU(g)*u, Q8_K(h), down GEMV
 * -> combine with slot k = shared expert (weight shared_w).  Experts shared
 * by several tokens are read from HBM once for all of them.
 *
 *   tab_gate/up/down: DEVICE arrays [n_expert] of expert matrices
 *                     (gate/up n_ff x hidden, down hidden x n_ff) - one
 *                     layer's slice of the [3][layer][E] pointer table
 *                     (session.cpp:2787-2796).
 *   sh_gate/up/down:  shared expert (n_ff x hidden etc.), or all NULL.
 *   sh_gate_w: fp32 [hidden] scalar gate row of the shared expert (qwen3.5
 *             files, LayerWeights::shared_gate_w, weights.hpp:54), or NULL.
 *             When set, the shared expert's output of token t is scaled by
 *             sigmoid(sh_gate_w . x[t]) before the combine, as
 *             gemv_f32_out_f16x_batched + sigmoid_gate_scalar_batched_f16
 *             do (session.cpp:2904-2909, layer.cpp:128-134).  The dot is
 *             taken in the reference kernel's fp32 lane order (q4_k.cu:
 *             133-149, 285-303); ignored without a shared expert.
 *   x:        fp32 [n_tokens][hidden] layer input.
 *   logits:   fp32 [n_tokens][n_expert]; if NULL, idx/weight are INPUTS
 *             (routing decided by the caller, e.g. sampled routing).
 *   residual: fp32 [n_tokens][hidden] or NULL (zero); may alias out.
 *   out:      fp32 [n_tokens][hidden].
 *   idx, weight: [n_tokens][k+1] (slot k of weight = shared_w).
 *   workspace: device buffer of at least sg_moe_layer_workspace_bytes()
 *             (scratch: the plan and h between the two launches).
 * The reference applies the gate to the shared output before the combine,
 * so slot k adds fma(shared_w, y_shared * sigmoid(g), acc); weight[t][k]
 * stays shared_w.
 * Routes with an id outside [0, n_expert) zero that token's whole weight row
 * (shared slot included), as moe_dispatch_scan does (moe.cu:385-396); a null
 * table entry is an absent expert and contributes zero (q4_k.cu:697-710).
 * Limits: hidden <= 8192 and n_ff <= 16384 (multiples of 256), k <= 32,
 * n_expert <= 1024.  Calls that share a workspace must be stream-ordered. */
size_t sg_moe_layer_workspace_bytes(int n_tokens, int hidden, int n_ff,
                                    int n_expert, int k);
int sg_moe_layer(const sg_block_q4k* const* tab_gate,
                 const sg_block_q4k* const* tab_up,
                 const sg_block_q4k* const* tab_down,
                 const sg_block_q4k* sh_gate, const sg_block_q4k* sh_up,
                 const sg_block_q4k* sh_down, const float* sh_gate_w, const float* x,
                 const float* logits, const float* residual, float* out,
                 int* idx, float* weight, void* workspace,
                 size_t workspace_bytes, int n_tokens, int hidden, int n_ff,
                 int n_expert, int k, float shared_w, void* stream);

/* sg_moe_layer on the session's own fp16 buffers (Session::moe_dispatch_
 * device, session.cpp:2482-3030, over x_ / xn_ of session.hpp:240):
 *   xn       fp16 [n_tokens][hidden], the normed activations (the shared
 *            gate's input; quantized to Q8_K when xq is NULL);
 *   xq       optional Q8_K of xn the caller already made (the fused
 *            norm+quantize's moe_xq_in_, session.cpp:1022, 1131), used as is
 *            instead of quantizing xn again; xn may then be NULL unless the
 *            shared gate is on;
 *   residual fp16 [n_tokens][hidden] or NULL (0); may alias out (x_ is both
 *            in the reference);
 *   out      fp16 [n_tokens][hidden].
 * The expert chain rounds where the session stores fp16: each expert's
 * gate and up outputs are rounded to fp16 (the f16out GEMVs), h =
 * fp16(SiLU(g) * u) (silu_mul_f16) and Q8_K of h is taken from those
 * values (session.cpp:1862-1869, 2791-2803, 2893-2898); the GEMVs' own
 * arithmetic is sg_moe_layer's.  The slot outputs are stored as fp16, as the
 * reference's f16out GEMVs store them, the shared one is gated on its fp16
 * value and stored again
 * (sigmoid_gate_scalar_batched_f16), and the combine accumulates in fp32
 * from the fp16 residual in slot order and stores fp16
 * (moe_combine_batched_f16, moe.cu:265-280; session.cpp:3029).  Everything
 * else (routing, idx/weight, workspace, limits) as sg_moe_layer. */
int sg_moe_layer_f16(const sg_block_q4k* const* tab_gate,
                     const sg_block_q4k* const* tab_up,
                     const sg_block_q4k* const* tab_down,
                     const sg_block_q4k* sh_gate, const sg_block_q4k* sh_up,
                     const sg_block_q4k* sh_down, const float* sh_gate_w,
                     const uint16_t* xn, const sg_block_q8k* xq, const float* logits,
                     const uint16_t* residual, uint16_t* out, int* idx, float* weight,
                     void* workspace, size_t workspace_bytes, int n_tokens, int hidden,
                     int n_ff, int n_expert, int k, float shared_w, void* stream);

/* sg_moe_layer without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * library keeps one 1 MiB scratch array per GPU (a file-scope device array,
 * held until the process ends) and uses it as the workspace; shapes whose
 * sg_moe_layer_workspace_bytes() exceeds 1 MiB are rejected with
 * SG_ERR_UNSUPPORTED (at hidden 2048, n_ff 512, top-8 + shared: up to 16
 * tokens).  Allocates nothing.  Every call on one GPU shares that GPU's
 * array, so calls that overlap on one GPU (two streams, two threads) race:
 * order them on one stream. */
int sg_moe_layer_noalloc(const sg_block_q4k* const* tab_gate,
                         const sg_block_q4k* const* tab_up,
                         const sg_block_q4k* const* tab_down,
                         const sg_block_q4k* sh_gate, const sg_block_q4k* sh_up,
                         const sg_block_q4k* sh_down, const float* sh_gate_w,
                         const float* x, const float* logits, const float* residual,
                         float* out, int* idx, float* weight, int n_tokens, int hidden,
                         int n_ff, int n_expert, int k, float shared_w, void* stream);

/* The two launches of sg_moe_layer, selectable: bit 0 = front (top-k,
 * Q8_K of x, the expert-major plan, gate/up GEMV + SiLU), bit 1 = back
 * (Q8_K of h, down GEMV, combine).  The back stage reads what the front left
 * in `workspace`, so a caller may run them separately on one stream (to put
 * other work between them, or to time one); stages = 3 is sg_moe_layer.
 * The reference issues these steps as separate launchers from
 * Session::moe_dispatch_device (session.cpp:2524-2556 route, :2791-2803
 * gate/up + SiLU + requant, :2820-2843 down + scatter, :3029 combine). */
int sg_moe_layer_stages(const sg_block_q4k* const* tab_gate,
                        const sg_block_q4k* const* tab_up,
                        const sg_block_q4k* const* tab_down,
                        const sg_block_q4k* sh_gate, const sg_block_q4k* sh_up,
                        const sg_block_q4k* sh_down, const float* sh_gate_w,
                        const float* x, const float* logits,
                        const float* residual, float* out, int* idx,
                        float* weight, void* workspace,
                        size_t workspace_bytes, int n_tokens, int hidden,
                        int n_ff, int n_expert, int k, float shared_w,
                        int stages, void* stream);

/* ---- prefill chunk (many tokens): device plan + int8-MFMA grouped GEMMs -- */

/* Expert-major plan of n_rows tokens x k routes, on the device, in one
 * launch.  Replaces cuda::moe_dispatch_scan (cuda_ops.hpp:219-222,
 * moe.cu:366-444) with the same outputs - off[E+1] row prefix, toff[E+1]
 * tile prefix (tok_per rows per tile), meta = {R, tiles, bad routes},
 * gslot[n_rows*k] (-1 for an invalid id), grows[R] (the token of each
 * grouped position) - and the same bounds-kill (an invalid id zeroes its
 * row of `weight`, stride k+1).  Unlike the reference, the order inside an
 * expert is deterministic: token order, then slot.  No mailbox: absent
 * experts are handled by the grouped kernels themselves.  off needs E+2
 * entries (off[E+1] = off[E]).  n_expert <= 1024 and
 * 2 * n_expert * (ceil(n_rows/32) + 1) + 1024 <= 38,912 (the plan is built in
 * LDS; 2048 tokens x 256 experts fit). */
int sg_moe_dispatch_scan(const int* idx, float* weight, int* gslot, int* grows,
                         int* off, int* toff, int* meta, int n_rows, int k,
                         int n_expert, int tok_per, void* stream);

/* The same plan built by two launches over many workgroups (32 tokens
 * each: bitmaps, then offsets and placement), with no
 * limit on n_rows beyond int indexing; the order inside an expert is the
 * same (token, then slot), so every array equals sg_moe_dispatch_scan's.
 * It is the plan sg_moe_prefill builds.  Extra outputs:
 *   shared_tail: the shared expert's rows (0 = none, else n_rows) appended
 *                after the routed ones: off[E+1] = off[E] + shared_tail and
 *                grows[off[E] + t] = t;
 *   tiles:       NULL, or the grouped kernels' work list: tiles[0] = count,
 *                then (expert << 16 | tile) for each tok_per-row tile of each
 *                group (the shared expert as expert E); it needs
 *                2 + (n_rows*k + tok_per-1)/tok_per + n_expert +
 *                (shared_tail + tok_per-1)/tok_per entries.
 * workspace: at least sg_moe_dispatch_plan_workspace_bytes(n_rows,
 * n_expert) bytes of scratch.  n_expert <= 1024, k <= 32.  Replaces
 * cuda::moe_dispatch_scan (cuda_ops.hpp:219-222) for large prefill chunks. */
size_t sg_moe_dispatch_plan_workspace_bytes(int n_rows, int n_expert);
int sg_moe_dispatch_plan(const int* idx, float* weight, int* gslot, int* grows, int* off,
                         int* toff, int* meta, int* tiles, void* workspace,
                         size_t workspace_bytes, int n_rows, int k, int n_expert, int tok_per,
                         int shared_tail, void* stream);

/* A whole MoE layer for a prefill chunk of n_tokens tokens (n_expert <=
 * 1024, k <= 32, n_tokens * (k + 1) < 2^31), same arguments and semantics as sg_moe_layer: Q8_K(x),
 * router top-k (logits != NULL) or caller routing, the device plan, gate/up
 * + SiLU and down as grouped int8-MFMA contractions over every routed expert
 * (the shared expert as one more group), combine in slot order.  Replaces
 * the reference's prefill MoE (session.cpp:2643-2840: the TC dequant+GEMM
 * path and its dp4a grouped twin, cuda_ops.hpp:190-250).  The super-block
 * sums are exact int32 (int8 MFMAs); the fp32 epilogue is the
 * integer-first super-block order (t = fma(d, sum sc*ip, -(dmin * sum
 * mn*bsum)), acc = fma(xd, t, acc)).  workspace: at least
 * sg_moe_prefill_workspace_bytes(). */
size_t sg_moe_prefill_workspace_bytes(int n_tokens, int hidden, int n_ff,
                                      int n_expert, int k);
int sg_moe_prefill(const sg_block_q4k* const* tab_gate,
                   const sg_block_q4k* const* tab_up,
                   const sg_block_q4k* const* tab_down,
                   const sg_block_q4k* sh_gate, const sg_block_q4k* sh_up,
                   const sg_block_q4k* sh_down, const float* sh_gate_w, const float* x,
                   const float* logits, const float* residual, float* out,
                   int* idx, float* weight, void* workspace,
                   size_t workspace_bytes, int n_tokens, int hidden, int n_ff,
                   int n_expert, int k, float shared_w, void* stream);

/* sg_moe_prefill on the session's fp16 buffers: the arguments and the
 * fp16 roundings of sg_moe_layer_f16 (g, u and h of every expert, the slot
 * outputs, the combine; xn fp16, xq an optional Q8_K of it used as is,
 * residual/out fp16; session.cpp:2643-2840 then moe_combine_batched_f16 at
 * :3029). */
int sg_moe_prefill_f16(const sg_block_q4k* const* tab_gate,
                       const sg_block_q4k* const* tab_up,
                       const sg_block_q4k* const* tab_down,
                       const sg_block_q4k* sh_gate, const sg_block_q4k* sh_up,
                       const sg_block_q4k* sh_down, const float* sh_gate_w,
                       const uint16_t* xn, const sg_block_q8k* xq, const float* logits,
                       const uint16_t* residual, uint16_t* out, int* idx, float* weight,
                       void* workspace, size_t workspace_bytes, int n_tokens, int hidden,
                       int n_ff, int n_expert, int k, float shared_w, void* stream);

/* ---- stage-by-stage launchers of the grouped path ----------------------
 * For a session that keeps the reference's own stage order (plan, gather,
 * grouped gate+up, SiLU, Q8_K of h, grouped down, scatter, combine) instead
 * of calling sg_moe_layer / sg_moe_prefill.  The plan arrays are
 * sg_moe_dispatch_scan's (meta[0] = routed rows, meta[1] = tiles).  Counts
 * decided by the plan are read on the device; r_max / rows_max / n_max /
 * tiles_max only bound the grids.  n_rows, r_max, tiles_max <= 65535. */

/* dst[r] = src[src_rows[r]], whole Q8_K rows of row_blocks blocks.
 * Replaces cuda::gather_rows_q8 (cuda_ops.hpp:364-366, moe.cu:237-247). */
int sg_gather_rows_q8(sg_block_q8k* dst, const sg_block_q8k* src, const int* src_rows,
                      int n_rows, int row_blocks, void* stream);
/* The same for r < meta[0].  Replaces cuda::gather_rows_q8_n
 * (cuda_ops.hpp:226-228, moe.cu:446-467). */
int sg_gather_rows_q8_n(sg_block_q8k* dst, const sg_block_q8k* src, const int* src_rows,
                        const int* meta, int r_max, int row_blocks, void* stream);
/* fp16 rows of hidden values, r < meta[0].  Replaces cuda::gather_rows_f16_n
 * (cuda_ops.hpp:229-231, moe.cu:472-491). */
int sg_gather_rows_f16_n(uint16_t* dst, const uint16_t* src, const int* src_rows,
                         const int* meta, int r_max, int hidden, void* stream);
/* out = f16(SiLU(g) * u) over the first d_rows[0] * n_ff values (the SiLU
 * of sg_silu_mul_f16).  Replaces cuda::silu_mul_f16_n (cuda_ops.hpp:232-234,
 * norm_rotary.cu:145-156). */
int sg_silu_mul_f16_n(uint16_t* out, const uint16_t* g, const uint16_t* u, const int* d_rows,
                      int rows_max, int n_ff, void* stream);
/* Q8_K of the first d_rows[0] * row_mult fp16 values (row_mult a multiple of
 * 256; n_max = the most blocks), bit-exact as sg_quantize_q8_k_f16.
 * Replaces cuda::quantize_q8_k_n (cuda_ops.hpp:235-237, q4_k.cu:1869-1924). */
int sg_quantize_q8_k_n(const uint16_t* x, sg_block_q8k* out, const int* d_rows, int row_mult,
                       int n_max, void* stream);
/* Grouped gate+up over the plan: for tile t < meta[1] (expert e = the last
 * with toff[e] <= t, positions off[e] + (t - toff[e]) * tok_per + j, at most
 * tok_per of them), yg[p][r] = f16(Wg_e[r] . xq[p]) and yu[p][r] likewise,
 * rows r < n_rows, each dot in the reference CPU order (as sg_gemv_q4_k_q8)
 * rounded once.  A null wg_tab[e] or wu_tab[e] zeroes the tile's outputs and
 * posts e to the mailbox (mail[atomicAdd(mail_n, 1)] = e while below
 * n_expert).  k <= 4096.  Replaces cuda::gemv_grouped2_tab_q4_k_q8_f16out_mtok
 * (cuda_ops.hpp:240-244, q4_k.cu:666-763, 1926-1957). */
int sg_gemv_grouped2_tab_q4_k_q8_f16out(const sg_block_q4k* const* wg_tab,
                                        const sg_block_q4k* const* wu_tab, const int* off,
                                        const int* toff, const int* meta, int* mail, int* mail_n,
                                        int tiles_max, const sg_block_q8k* xq, uint16_t* yg,
                                        uint16_t* yu, int n_rows, int k, int n_expert, int tok_per,
                                        void* stream);
/* The same with one matrix table (the down projection), no mailbox.
 * Replaces cuda::gemv_grouped_tab_q4_k_q8_f16out_mtok (cuda_ops.hpp:247-250,
 * q4_k.cu:765-836, 1959-1987). */
int sg_gemv_grouped_tab_q4_k_q8_f16out(const sg_block_q4k* const* w_tab, const int* off,
                                       const int* toff, const int* meta, int tiles_max,
                                       const sg_block_q8k* xq, uint16_t* y, int n_rows, int k,
                                       int n_expert, int tok_per, void* stream);
/* expert_y[row][kk] = grouped_out[gslot[row*n_used + kk]] for gslot >= 0
 * (expert_y rows of n_used + 1 slots, the last the shared expert's, left as
 * is).  Replaces cuda::scatter_routed_f16 (cuda_ops.hpp:372-374,
 * moe.cu:249-262). */
int sg_scatter_routed_f16(uint16_t* expert_y, const uint16_t* grouped_out, const int* gslot,
                          int n_rows, int n_used, int hidden, void* stream);
/* dst[dst_rows[i]] = src[i], fp16 rows.  Replaces cuda::scatter_rows_f16
 * (cuda_ops.hpp:408-409, moe.cu:142-156). */
int sg_scatter_rows_f16(uint16_t* dst, const uint16_t* src, const int* dst_rows, int n_rows,
                        int hidden, void* stream);

/* ---- GGUF expert pool (load time, host + HBM) ------------------------
 * Replaces Weights::load_expert_pool (weights.cpp:800-870, over the GGUF v3
 * reader of gguf.hpp/gguf.cpp) and the device pointer table the session
 * uploads (session.cpp:2787-2796, 3596-3597).  Every blk.L.ffn_{gate,up,
 * down}_exps (stacked [n_expert][rows][cols]; gate/up Q4_K, down Q4_K or
 * Q6_K) of L = 0, 1, ... is copied once into one HBM allocation laid out
 * [layer][expert][gate | up | down]; a Q6_K down projection is requantized to
 * Q4_K per row on the host first, as the reference does (weights.cpp:841-857).
 * The table is [gate|up|down][layer][expert] device pointers: layer l's three
 * slices are table + (m*L + l)*E, m = 0, 1, 2 - the tab_gate/tab_up/tab_down
 * arguments of sg_moe_layer and sg_moe_prefill.  Synchronous; not for the
 * hot path. */
typedef struct sg_expert_pool sg_expert_pool;

/* Parse a GGUF v3 file's header and expert tensors without touching the GPU. */
int sg_gguf_expert_dims(const char* path, int* n_layers, int* n_expert, int* hidden,
                        int* n_ff, int* q6_down_layers);
/* Load the expert pool of a GGUF v3 file onto the current device. */
int sg_expert_pool_load_gguf(const char* path, sg_expert_pool** out);
int sg_expert_pool_dims(const sg_expert_pool* p, int* n_layers, int* n_expert, int* hidden,
                        int* n_ff);
/* Device pointer table [3][n_layers][n_expert] (a device address). */
const sg_block_q4k* const* sg_expert_pool_table(const sg_expert_pool* p);
void sg_expert_pool_free(sg_expert_pool* p);

/* Host Q4_K quantizer of one fp32 row (n a multiple of 256): the
 * reference's quantize_row (q4_k.cpp:62-174), used to requantize Q6_K
 * expert tensors at load time. */
int sg_q4k_quantize_row(const float* x, sg_block_q4k* out, int n);

#ifdef __cplusplus
}
#endif
#endif /* SAGER_HIP_H */
