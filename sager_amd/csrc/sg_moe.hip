// sg_moe.hip - standalone router top-k, SiLU and combine launchers on gfx950
// (the per-stage operators of the reference's MoE dispatch; the fused layer
// is in sg_layer.hip).  Router moe.cu:25-85 / 165-234, SiLU
// norm_rotary.cu:133-160 with the CPU chain's fp32 order q4_avx2.cpp:187-191,
// combine moe.cu:265-280; fp16-buffer twins of SiLU and the combine, the
// shared-expert sigmoid gate (norm_rotary.cu:177-184, moe.cu:282-292) and
// the fp32 x fp16 GEMV that produces gate and router logits
// (q4_k.cu:133-149, 285-303).
#include "sg_common.hpp"
#include "sg_router.hpp"

namespace sg {

constexpr int kMaxExperts = 1024;
constexpr int kMaxK = 32;

__host__ __device__ inline int round4(int n) { return (n + 3) & ~3; }
__host__ __device__ inline int lpr_of(int nb) {
  int l = 1;
  while (l < nb) l <<= 1;
  return l;
}

template <int PL>
__global__ void __launch_bounds__(64) router_kernel(const float* __restrict__ logits,
                                                    int* __restrict__ idx,
                                                    float* __restrict__ weight, int n_expert,
                                                    int k, int stride, float shared_w) {
  __shared__ __attribute__((aligned(16))) float ev[64 * PL];
  const long long row = blockIdx.x;
  router_wave<PL>(logits + row * n_expert, n_expert, k, shared_w, idx + row * stride,
                  weight + row * stride, ev, threadIdx.x);
}

// four SiLU products per thread through the table exp (silu_mul_tab_n),
// the prefill gate/up kernel's arithmetic
__global__ void __launch_bounds__(256) silu_kernel(float* __restrict__ out,
                                                   const float* __restrict__ g,
                                                   const float* __restrict__ u, long long n) {
  __shared__ double tab[64];
  if (threadIdx.x < 64) tab[threadIdx.x] = kExp2Tab64[threadIdx.x];
  __syncthreads();
  const long long i0 = (static_cast<long long>(blockIdx.x) * 256 + threadIdx.x) * 4;
  float gv[4], uv[4], hv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const long long i = i0 + j < n ? i0 + j : n - 1;
    gv[j] = g[i];
    uv[j] = u[i];
  }
  silu_mul_tab_n<4>(gv, uv, hv, tab);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (i0 + j < n) out[i0 + j] = hv[j];
}

__global__ void __launch_bounds__(256) combine_kernel(float* out, const float* residual,
                                                      const float* __restrict__ ys,
                                                      const float* __restrict__ w, int n_used,
                                                      int hidden) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  const long long r = blockIdx.y;
  if (i >= hidden) return;
  float acc = residual ? residual[r * hidden + i] : 0.f;
  const float* yr = ys + r * (n_used + 1) * static_cast<long long>(hidden) + i;
  const float* wr = w + r * (n_used + 1);
  for (int kk = 0; kk <= n_used; ++kk)
    acc = __builtin_fmaf(wr[kk], yr[static_cast<long long>(kk) * hidden], acc);
  out[r * hidden + i] = acc;
}


// out = f16(SiLU(g) * u) on fp16 buffers (norm_rotary.cu:133-141)
__global__ void __launch_bounds__(256) silu_f16_kernel(uint16_t* __restrict__ out,
                                                       const uint16_t* __restrict__ g,
                                                       const uint16_t* __restrict__ u,
                                                       long long n) {
  const long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) out[i] = f16b(silu_mul(f16v(g[i]), f16v(u[i])));
}

// out[r][i] = f16(f32(out[r][i]) + sum_kk fma(w[r][kk], f32(y[r][kk][i])))
// in slot order on fp16 buffers (moe.cu:265-280)
__global__ void __launch_bounds__(256) combine_f16_kernel(uint16_t* out,
                                                          const uint16_t* __restrict__ ys,
                                                          const float* __restrict__ w,
                                                          int n_used, int hidden) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  const long long r = blockIdx.y;
  if (i >= hidden) return;
  float acc = f16v(out[r * hidden + i]);
  const uint16_t* yr = ys + r * (n_used + 1) * static_cast<long long>(hidden) + i;
  const float* wr = w + r * (n_used + 1);
  for (int kk = 0; kk <= n_used; ++kk)
    acc = __builtin_fmaf(wr[kk], f16v(yr[static_cast<long long>(kk) * hidden]), acc);
  out[r * hidden + i] = f16b(acc);
}

// out[r][i] = f16(f32(out[r][i]) * sigmoid(g[r])) (moe.cu:282-292)
__global__ void __launch_bounds__(256) sigmoid_gate_f16_kernel(uint16_t* __restrict__ out,
                                                               const float* __restrict__ g,
                                                               int hidden) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  const long long r = blockIdx.y;
  if (i >= hidden) return;
  const float s = sigmoid_sg(g[r]);
  out[r * hidden + i] = f16b(f16v(out[r * hidden + i]) * s);
}

// y[t][r] = W[r] . f32(x[t]) with W fp32 [n_rows][k], x fp16 [T][k]: eight
// rows per workgroup, one per 32-lane half-wave, in the reference's lane
// order (rowdot_f32_lanes32).
__global__ void __launch_bounds__(256) gemv_f32_f16x_kernel(const float* __restrict__ w,
                                                            const uint16_t* __restrict__ x,
                                                            float* __restrict__ y, int n_rows,
                                                            int k) {
  const int l = threadIdx.x & 31;
  const int row = blockIdx.x * 8 + (threadIdx.x >> 5);
  const long long t = blockIdx.y;
  const int r = row < n_rows ? row : n_rows - 1;  // whole halves stay active for the shuffles
  const uint16_t* xt = x + t * k;
  const float v = rowdot_f32_lanes32(w + static_cast<long long>(r) * k,
                                     [&](int i) { return f16v(xt[i]); }, k, l);
  if (l == 0 && row < n_rows) y[t * n_rows + row] = v;
}

// Router GEMV and top-k of one token in one launch (mmq.cu:459-511): the
// logits y[e] = W[e] . f32(x) in gemv_f32_f16x_kernel's lane order (so bit
// for bit sg_gemv_f32_out_f16x's), eight rows per workgroup; the workgroup
// that arrives last (a counter, no waiting) routes them with router_wave
// (sg_router_topk's semantics) and resets the counter.  Logits and counter
// are file-scope device arrays: one set per GPU, so calls that overlap on
// one GPU race.  Only the k routed slots are written (the shared slot k of
// weight is left as it is, as the reference's fused kernel does).
__device__ float g_router_logits[kMaxExperts];
__device__ unsigned int g_router_arrivals;

template <int PL>
__global__ void __launch_bounds__(256) router_fused_kernel(const float* __restrict__ w,
                                                           const uint16_t* __restrict__ x,
                                                           int* __restrict__ idx,
                                                           float* __restrict__ weight,
                                                           int n_expert, int k, int hidden) {
  __shared__ __attribute__((aligned(16))) float ev[64 * PL];
  __shared__ bool s_last;
  const int l = threadIdx.x & 31;
  const int row = blockIdx.x * 8 + (threadIdx.x >> 5);
  const int r = row < n_expert ? row : n_expert - 1;
  const float v = rowdot_f32_lanes32(w + static_cast<long long>(r) * hidden,
                                     [&](int i) { return f16v(x[i]); }, hidden, l);
  if (l == 0 && row < n_expert) g_router_logits[row] = v;
  __threadfence();  // this workgroup's logits, visible before its arrival
  __syncthreads();
  if (threadIdx.x == 0)
    s_last = atomicAdd(&g_router_arrivals, 1u) == gridDim.x - 1;
  __syncthreads();
  if (!s_last) return;
  __threadfence();  // every other workgroup's logits
  if (threadIdx.x < 64)
    router_wave<PL>(g_router_logits, n_expert, k, 0.f, idx, weight, ev, threadIdx.x, false);
  if (threadIdx.x == 0) atomicExch(&g_router_arrivals, 0u);  // for the next launch
}

}  // namespace sg

using namespace sg;

extern "C" {

int sg_router_topk_fused(const float* w, const uint16_t* x, int* idx, float* weight, int n_expert,
                         int n_expert_used, int hidden, void* stream) {
  const char* nm = "sg_router_topk_fused";
  if (!w || !x || !idx || !weight) return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  if (n_expert <= 0 || n_expert > kMaxExperts || n_expert_used <= 0 ||
      n_expert_used > n_expert || n_expert_used > 64 || hidden <= 0)
    return set_error(SG_ERR_GEOMETRY, "%s: n_expert=%d (<=%d) n_expert_used=%d hidden=%d", nm,
                     n_expert, kMaxExperts, n_expert_used, hidden);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((n_expert + 7) / 8);
  auto launch = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, s, w, x, idx, weight, n_expert, n_expert_used,
                       hidden);
  };
  if (n_expert <= 64) launch(router_fused_kernel<1>);
  else if (n_expert <= 128) launch(router_fused_kernel<2>);
  else if (n_expert <= 256) launch(router_fused_kernel<4>);
  else if (n_expert <= 512) launch(router_fused_kernel<8>);
  else launch(router_fused_kernel<16>);
  return check_launch(nm);
}


int sg_router_topk(const float* logits, int* idx, float* weight, int n_expert, int n_expert_used,
                   int idx_stride, int n_rows, float shared_w, void* stream) {
  if (!logits || !idx || !weight)
    return set_error(SG_ERR_INVALID_ARGUMENT, "sg_router_topk: null pointer");
  if (n_expert <= 0 || n_expert > kMaxExperts || n_expert_used <= 0 ||
      n_expert_used > n_expert || idx_stride < n_expert_used + 1 || n_rows <= 0)
    return set_error(SG_ERR_GEOMETRY,
                     "sg_router_topk: n_expert=%d (<=%d) n_expert_used=%d idx_stride=%d n_rows=%d",
                     n_expert, kMaxExperts, n_expert_used, idx_stride, n_rows);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // experts per lane: the smallest power of two that covers n_expert
  auto launch = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(n_rows), dim3(64), 0, s, logits, idx, weight, n_expert,
                       n_expert_used, idx_stride, shared_w);
  };
  if (n_expert <= 64) launch(router_kernel<1>);
  else if (n_expert <= 128) launch(router_kernel<2>);
  else if (n_expert <= 256) launch(router_kernel<4>);
  else if (n_expert <= 512) launch(router_kernel<8>);
  else launch(router_kernel<16>);
  return check_launch("sg_router_topk");
}

int sg_silu_mul(float* out, const float* g, const float* u, int n, void* stream) {
  if (!out || !g || !u) return set_error(SG_ERR_INVALID_ARGUMENT, "sg_silu_mul: null pointer");
  if (n <= 0) return set_error(SG_ERR_GEOMETRY, "sg_silu_mul: n=%d", n);
  hipLaunchKernelGGL(silu_kernel, dim3((n + 1023) / 1024), dim3(256), 0,
                     static_cast<hipStream_t>(stream), out, g, u, static_cast<long long>(n));
  return check_launch("sg_silu_mul");
}

int sg_moe_combine(float* out, const float* residual, const float* expert_y, const float* weight,
                   int n_used, int hidden, int n_rows, void* stream) {
  if (!out || !expert_y || !weight)
    return set_error(SG_ERR_INVALID_ARGUMENT, "sg_moe_combine: null pointer");
  if (n_used < 0 || hidden <= 0 || n_rows <= 0 || n_rows > 65535)
    return set_error(SG_ERR_GEOMETRY, "sg_moe_combine: n_used=%d hidden=%d n_rows=%d", n_used,
                     hidden, n_rows);
  hipLaunchKernelGGL(combine_kernel, dim3((hidden + 255) / 256, n_rows), dim3(256), 0,
                     static_cast<hipStream_t>(stream), out, residual, expert_y, weight, n_used,
                     hidden);
  return check_launch("sg_moe_combine");
}

int sg_silu_mul_f16(uint16_t* out, const uint16_t* g, const uint16_t* u, int rows, int n_ff,
                    void* stream) {
  if (!out || !g || !u) return set_error(SG_ERR_INVALID_ARGUMENT, "sg_silu_mul_f16: null pointer");
  if (rows <= 0 || n_ff <= 0)
    return set_error(SG_ERR_GEOMETRY, "sg_silu_mul_f16: rows=%d n_ff=%d", rows, n_ff);
  const long long n = static_cast<long long>(rows) * n_ff;
  if ((n + 255) / 256 > 0x7fffffffLL)
    return set_error(SG_ERR_GEOMETRY, "sg_silu_mul_f16: rows*n_ff=%lld too large", n);
  hipLaunchKernelGGL(silu_f16_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), out, g, u, n);
  return check_launch("sg_silu_mul_f16");
}

int sg_moe_combine_batched_f16(uint16_t* out, const uint16_t* expert_y, const float* weight,
                               int n_used, int hidden, int n_rows, void* stream) {
  if (!out || !expert_y || !weight)
    return set_error(SG_ERR_INVALID_ARGUMENT, "sg_moe_combine_batched_f16: null pointer");
  if (n_used < 0 || hidden <= 0 || n_rows <= 0 || n_rows > 65535)
    return set_error(SG_ERR_GEOMETRY, "sg_moe_combine_batched_f16: n_used=%d hidden=%d n_rows=%d",
                     n_used, hidden, n_rows);
  hipLaunchKernelGGL(combine_f16_kernel, dim3((hidden + 255) / 256, n_rows), dim3(256), 0,
                     static_cast<hipStream_t>(stream), out, expert_y, weight, n_used, hidden);
  return check_launch("sg_moe_combine_batched_f16");
}

int sg_sigmoid_gate_scalar_batched_f16(uint16_t* out, const float* g, int n_rows, int hidden,
                                       void* stream) {
  if (!out || !g)
    return set_error(SG_ERR_INVALID_ARGUMENT, "sg_sigmoid_gate_scalar_f16: null pointer");
  if (n_rows <= 0 || n_rows > 65535 || hidden <= 0)
    return set_error(SG_ERR_GEOMETRY, "sg_sigmoid_gate_scalar_f16: n_rows=%d hidden=%d", n_rows,
                     hidden);
  hipLaunchKernelGGL(sigmoid_gate_f16_kernel, dim3((hidden + 255) / 256, n_rows), dim3(256), 0,
                     static_cast<hipStream_t>(stream), out, g, hidden);
  return check_launch("sg_sigmoid_gate_scalar_f16");
}

int sg_sigmoid_gate_scalar_f16(uint16_t* out, const float* g, int n, void* stream) {
  return sg_sigmoid_gate_scalar_batched_f16(out, g, 1, n, stream);
}

int sg_gemv_f32_out_f16x(const float* w, const uint16_t* x, float* y, int n_rows, int k,
                         int n_tokens, void* stream) {
  if (!w || !x || !y) return set_error(SG_ERR_INVALID_ARGUMENT, "sg_gemv_f32_out_f16x: null pointer");
  if (n_rows <= 0 || k <= 0 || n_tokens <= 0 || n_tokens > 65535)
    return set_error(SG_ERR_GEOMETRY, "sg_gemv_f32_out_f16x: n_rows=%d k=%d n_tokens=%d", n_rows,
                     k, n_tokens);
  hipLaunchKernelGGL(gemv_f32_f16x_kernel, dim3((n_rows + 7) / 8, n_tokens), dim3(256), 0,
                     static_cast<hipStream_t>(stream), w, x, y, n_rows, k);
  return check_launch("sg_gemv_f32_out_f16x");
}

}  // extern "C"
