// sg_moe.hip - router top-k, SiLU, combine and the fused MoE layer on gfx950.
//
// The fused layer runs one MoE layer for 1..16 tokens in three launches:
//
//   route   (1 workgroup)   per token: softmax/top-k with one wave; Q8_K of
//                           x; the expert-major plan (unique experts, their
//                           routes in (expert, token, slot) order, the shared
//                           expert as a last group); clears the combine
//                           counters.
//   gate/up (chunks x groups) one workgroup = 16 rows of one expert group:
//                           each lane holds one super-block of a gate row
//                           (lanes 0-31) or of the same up row (lanes 32-63)
//                           in registers and runs it against every token of
//                           the group, so an expert shared by tokens is read
//                           from HBM once; h = SiLU(g)*u in the CPU chain's
//                           order.
//   down    (chunks x groups) requantizes the group's h rows into LDS, runs
//                           the down rows, writes the slot outputs; the last
//                           workgroup to finish a row chunk (atomic counter,
//                           release/acquire fences) combines that chunk for
//                           every token in slot order - deterministic, no
//                           floating-point atomics.
//
// Stage order and semantics: Session::moe_dispatch_device
// (session.cpp:2482-3030), router moe.cu:25-85 / 165-234, dispatch plan
// moe.cu:366-444, combine moe.cu:265-280, expert chain q4_avx2.cpp:175-196.
#include "sg_common.hpp"

namespace sg {

constexpr int kMaxExperts = 1024;
constexpr int kMaxK = 32;
constexpr int kMaxLayerTokens = 16;
constexpr int kPerLane = kMaxExperts / 64;

__host__ __device__ inline int round4(int n) { return (n + 3) & ~3; }
__host__ __device__ inline int lpr_of(int nb) {
  int l = 1;
  while (l < nb) l <<= 1;
  return l;
}

// ---- router: one wave per token row ----------------------------------------
// Softmax with the max and the normalizer sum taken in index order, k rounds
// of (value desc, index asc) argmax over non-NaN probabilities, degenerate
// rounds pick kk % n_expert, weights renormalized by their k-order sum,
// slot k = shared_w.  e_lds: round4(n_expert) floats of this wave.
__device__ void router_wave(const float* __restrict__ lg, int n_expert, int k, float shared_w,
                            int* __restrict__ oi, float* __restrict__ ow, float* e_lds,
                            int* oi_lds, int lane) {
  float p[kPerLane];
  float mx = -1e30f;
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) {
    const int i = lane + 64 * j;
    p[j] = i < n_expert ? lg[i] : 0.f;
    if (i < n_expert) mx = fmaxf(mx, p[j]);
  }
  mx = wave_max(mx);
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) {
    const int i = lane + 64 * j;
    if (i < n_expert) {
      p[j] = expf_sg(p[j] - mx);
      e_lds[i] = p[j];
    }
  }
  const int n4 = round4(n_expert);
  if (n_expert + lane < n4) e_lds[n_expert + lane] = 0.f;  // +0 leaves the sum unchanged
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float z = 0.f;
  if (lane == 0) {
    const float4* e4 = reinterpret_cast<const float4*>(e_lds);
    for (int i = 0; i < n4 / 4; ++i) {
      const float4 v = e4[i];
      z += v.x;
      z += v.y;
      z += v.z;
      z += v.w;
    }
  }
  z = __shfl(z, 0, 64);
#pragma unroll
  for (int j = 0; j < kPerLane; ++j)
    if (lane + 64 * j < n_expert) p[j] = p[j] / z;

  float wsum = 0.f;
  for (int kk = 0; kk < k; ++kk) {
    float bv = -1.f;
    int bi = -1;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
      const int i = lane + 64 * j;
      if (i < n_expert && p[j] == p[j] && p[j] > bv) {
        bv = p[j];
        bi = i;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int oj = __shfl_xor(bi, o, 64);
      if (oj >= 0 && (bi < 0 || ov > bv || (ov == bv && oj < bi))) {
        bv = ov;
        bi = oj;
      }
    }
    if (bi < 0) bi = kk % n_expert;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j)
      if (lane + 64 * j == bi) p[j] = -1.f;
    if (lane == 0) {
      oi[kk] = bi;
      ow[kk] = bv;
      if (oi_lds) oi_lds[kk] = bi;
    }
    wsum += bv;
  }
  if (lane == 0) {
    if (wsum > 0.f)
      for (int kk = 0; kk < k; ++kk) ow[kk] = ow[kk] / wsum;
    ow[k] = shared_w;
  }
}

__global__ void __launch_bounds__(64) router_kernel(const float* __restrict__ logits,
                                                    int* __restrict__ idx,
                                                    float* __restrict__ weight, int n_expert,
                                                    int k, int stride, float shared_w) {
  extern __shared__ __attribute__((aligned(16))) float e_dyn[];
  const long long row = blockIdx.x;
  router_wave(logits + row * n_expert, n_expert, k, shared_w, idx + row * stride,
              weight + row * stride, e_dyn, nullptr, threadIdx.x);
}

__global__ void __launch_bounds__(256) silu_kernel(float* __restrict__ out,
                                                   const float* __restrict__ g,
                                                   const float* __restrict__ u, long long n) {
  const long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) out[i] = silu_mul(g[i], u[i]);
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

// ---- fused layer ------------------------------------------------------------

struct LayerPlan {
  int* meta;    // [0] groups, [1] has_shared, [2] valid routes
  int* off;     // [gmax+1] route offsets per group
  int* expert;  // [gmax] expert id per group, -1 = shared expert
  int* tok;     // [T*k + T] route token, expert-major
  int* slot;    // [T*k + T] route slot
};

struct LayerWs {
  size_t xq, meta, off, expert, tok, slot, h, ys, counters, total;
  int gmax, chunks;
};

static size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

static int down_rows_per_wg(int n_ff) { return 4 * (64 / lpr_of(n_ff / kQK)); }

static LayerWs layer_ws(int T, int hidden, int n_ff, int n_expert, int k) {
  LayerWs w{};
  const int gmax = (T * k < n_expert ? T * k : n_expert) + 1;
  const int rmax = T * k + T;
  const int rows_wg = down_rows_per_wg(n_ff);
  w.gmax = gmax;
  w.chunks = (hidden + rows_wg - 1) / rows_wg;
  size_t o = 0;
  w.xq = o;       o = align256(o + static_cast<size_t>(T) * (hidden / kQK) * kQ8Bytes);
  w.meta = o;     o = align256(o + 4 * sizeof(int));
  w.off = o;      o = align256(o + (gmax + 1) * sizeof(int));
  w.expert = o;   o = align256(o + gmax * sizeof(int));
  w.tok = o;      o = align256(o + rmax * sizeof(int));
  w.slot = o;     o = align256(o + rmax * sizeof(int));
  w.h = o;        o = align256(o + static_cast<size_t>(T) * (k + 1) * n_ff * sizeof(float));
  w.ys = o;       o = align256(o + static_cast<size_t>(T) * (k + 1) * hidden * sizeof(float));
  w.counters = o; o = align256(o + w.chunks * sizeof(int));
  w.total = o;
  return w;
}

// Route + quantize + plan.  One workgroup of 16 waves.
__global__ void __launch_bounds__(1024) layer_route_kernel(
    const float* __restrict__ x, const float* __restrict__ logits, int* __restrict__ idx,
    float* __restrict__ weight, unsigned char* __restrict__ xq, LayerPlan plan,
    int* __restrict__ counters, int n_chunks, int T, int hidden, int n_expert, int k,
    float shared_w, int has_shared) {
  extern __shared__ __attribute__((aligned(16))) float e_dyn[];  // T * round4(n_expert)
  __shared__ int route_e[kMaxLayerTokens * kMaxK];
  __shared__ int present[kMaxExperts];
  __shared__ int gid[kMaxExperts];
  __shared__ int wtot[16];
  __shared__ int n_valid;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int stride = k + 1;

  // 1) routing (one wave per token) and clearing of the per-call state
  if (logits && wave < T)
    router_wave(logits + static_cast<long long>(wave) * n_expert, n_expert, k, shared_w,
                idx + wave * stride, weight + wave * stride, e_dyn + wave * round4(n_expert),
                route_e + wave * k, lane);
  if (tid < n_expert) present[tid] = 0;
  for (int c = tid; c < n_chunks; c += blockDim.x) counters[c] = 0;
  if (tid == 0) n_valid = 0;

  // 2) Q8_K of every token's x, one wave per block
  const int nbh = hidden / kQK;
  for (int b = wave; b < T * nbh; b += 16) {
    const float* xb = x + static_cast<long long>(b) * kQK + 4 * lane;
    float v[4] = {xb[0], xb[1], xb[2], xb[3]};
    quantize_block_wave(v, xq + static_cast<long long>(b) * kQ8Bytes, lane);
  }
  __threadfence_block();
  __syncthreads();

  // 3) expert-major plan
  const int R = T * k;
  bool valid = false;
  int e = -1;
  if (tid < R) {
    e = logits ? route_e[tid] : idx[(tid / k) * stride + (tid % k)];
    valid = e >= 0 && e < n_expert;
    route_e[tid] = valid ? e : -1;
    if (valid) {
      present[e] = 1;
      atomicAdd(&n_valid, 1);
    }
  }
  __syncthreads();
  // exclusive scan of present[] -> group id per expert (wave w covers 64w..64w+63)
  {
    const int ex = tid;
    const bool pr = ex < n_expert && present[ex];
    const unsigned long long bal = __ballot(pr);
    const int below = __builtin_amdgcn_mbcnt_hi(static_cast<unsigned>(bal >> 32),
                                                 __builtin_amdgcn_mbcnt_lo(static_cast<unsigned>(bal), 0));
    if (lane == 0) wtot[wave] = __popcll(bal);
    __syncthreads();
    int base = 0;
    for (int w = 0; w < wave; ++w) base += wtot[w];
    if (ex < n_expert) gid[ex] = base + below;
  }
  int n_groups_routed = 0;
  for (int w = 0; w < 16; ++w) n_groups_routed += wtot[w];
  __syncthreads();
  const int rv = n_valid;
  if (valid) {
    int rank = 0;
    bool first = true;
    for (int j = 0; j < R; ++j) {
      const int ej = route_e[j];
      if (ej < 0) continue;
      if (ej < e || (ej == e && j < tid)) ++rank;
      if (ej == e && j < tid) first = false;
    }
    plan.tok[rank] = tid / k;
    plan.slot[rank] = tid % k;
    if (first) {
      plan.off[gid[e]] = rank;
      plan.expert[gid[e]] = e;
    }
  }
  if (tid < T) {
    bool bad = false;
    for (int kk = 0; kk < k; ++kk) bad |= route_e[tid * k + kk] < 0;
    if (bad)  // bounds-kill: the whole row's weights, shared slot included
      for (int q = 0; q <= k; ++q) weight[tid * stride + q] = 0.f;
    if (has_shared) {
      plan.tok[rv + tid] = tid;
      plan.slot[rv + tid] = k;
    }
  }
  if (tid == 0) {
    plan.off[n_groups_routed] = rv;
    if (has_shared) {
      plan.expert[n_groups_routed] = -1;
      plan.off[n_groups_routed + 1] = rv + T;
    }
    plan.meta[0] = n_groups_routed + has_shared;
    plan.meta[1] = has_shared;
    plan.meta[2] = rv;
  }
}

// gate/up + SiLU for one (row chunk, group).  Lanes 0-31: gate rows,
// lanes 32-63: the same up rows.
__global__ void __launch_bounds__(256) layer_gateup_kernel(
    const sg_block_q4k* const* __restrict__ tab_gate, const sg_block_q4k* const* __restrict__ tab_up,
    const sg_block_q4k* sh_gate, const sg_block_q4k* sh_up, const unsigned char* __restrict__ xq,
    LayerPlan plan, float* __restrict__ h, int T, int hidden, int n_ff, int k) {
  extern __shared__ __attribute__((aligned(16))) uint32_t xs_dyn[];  // T * nbh * kXStride
  __shared__ int toks[kMaxLayerTokens];
  const int g = blockIdx.y;
  if (g >= plan.meta[0]) return;
  const int e = plan.expert[g];
  const sg_block_q4k* wg = e >= 0 ? tab_gate[e] : sh_gate;
  const sg_block_q4k* wu = e >= 0 ? tab_up[e] : sh_up;
  const bool present = wg != nullptr && wu != nullptr;
  const int beg = plan.off[g], end = plan.off[g + 1];

  const int nbh = hidden / kQK, lpr = lpr_of(nbh);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, hl = lane & 31;
  const int blk = hl & (lpr - 1);
  const int rpw = 32 / lpr;
  const int row = blockIdx.x * 4 * rpw + wave * rpw + hl / lpr;
  const bool live = present && blk < nbh && row < n_ff;

  uint32_t w36[36];
  ScaleMins sm8{};
  if (live) {
    load_q4k((half ? wu : wg) + static_cast<long long>(row) * nbh + blk, w36);
    sm8 = unpack_scales(w36[1], w36[2], w36[3]);
  }
  for (int e0 = beg; e0 < end; e0 += T) {
    const int n = end - e0 < T ? end - e0 : T;
    __syncthreads();
    if (threadIdx.x < n) toks[threadIdx.x] = plan.tok[e0 + threadIdx.x];
    __syncthreads();
    stage_q8k_rows(xq, toks, n, nbh, xs_dyn, threadIdx.x, blockDim.x);
    __syncthreads();
    for (int j = 0; j < n; ++j) {
      float s = 0.f;
      if (live) {
        int32_t xr[64], ip[8];
        float xd, bsf[8];
        load_x_regs(xs_dyn + (j * nbh + blk) * kXStride, xr, xd, bsf);
        subblock_dots(w36 + 4, xr, ip);
        s = block_sum(w36[0], sm8, ip, xd, bsf);
      }
      const float acc = row_sum_in_order(s, lane, lpr, nbh);
      const float up = __shfl_xor(acc, 32, 64);
      if (half == 0 && blk == 0 && row < n_ff) {
        const long long hs = static_cast<long long>(toks[j]) * (k + 1) + plan.slot[e0 + j];
        h[hs * n_ff + row] = present ? silu_mul(acc, up) : 0.f;
      }
    }
  }
}

// down projection for one (row chunk, group) + last-arriver combine.
__global__ void __launch_bounds__(256) layer_down_kernel(
    const sg_block_q4k* const* __restrict__ tab_gate, const sg_block_q4k* const* __restrict__ tab_up,
    const sg_block_q4k* const* __restrict__ tab_down, const sg_block_q4k* sh_gate,
    const sg_block_q4k* sh_up, const sg_block_q4k* sh_down, LayerPlan plan,
    const float* __restrict__ h, float* __restrict__ ys, const int* __restrict__ idx,
    const float* __restrict__ weight, const float* residual, float* out, int* counters, int T,
    int hidden, int n_ff, int n_expert, int k) {
  extern __shared__ __attribute__((aligned(16))) uint32_t hs_dyn[];  // T * nbf * kXStride
  __shared__ int toks[kMaxLayerTokens];
  __shared__ int slots[kMaxLayerTokens];
  __shared__ int last;
  const int g = blockIdx.y;
  const int n_groups = plan.meta[0];
  if (g >= n_groups) return;
  const int e = plan.expert[g];
  const sg_block_q4k* wd = e >= 0 ? tab_down[e] : sh_down;
  const bool present =
      wd != nullptr && (e >= 0 ? tab_gate[e] : sh_gate) != nullptr &&
      (e >= 0 ? tab_up[e] : sh_up) != nullptr;
  const int beg = plan.off[g], end = plan.off[g + 1];

  const int nbf = n_ff / kQK, lpr = lpr_of(nbf);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int blk = lane & (lpr - 1);
  const int rpw = 64 / lpr;
  const int rows_wg = 4 * rpw;
  const int row = blockIdx.x * rows_wg + wave * rpw + lane / lpr;
  const bool live = present && blk < nbf && row < hidden;

  uint32_t w36[36];
  ScaleMins sm8{};
  if (live) {
    load_q4k(wd + static_cast<long long>(row) * nbf + blk, w36);
    sm8 = unpack_scales(w36[1], w36[2], w36[3]);
  }
  for (int e0 = beg; e0 < end; e0 += T) {
    const int n = end - e0 < T ? end - e0 : T;
    __syncthreads();
    if (threadIdx.x < n) {
      toks[threadIdx.x] = plan.tok[e0 + threadIdx.x];
      slots[threadIdx.x] = plan.slot[e0 + threadIdx.x];
    }
    __syncthreads();
    for (int b = wave; b < n * nbf; b += 4) {  // Q8_K(h) of the batch into LDS
      const int j = b / nbf, bb = b - j * nbf;
      const long long hs = static_cast<long long>(toks[j]) * (k + 1) + slots[j];
      const float* hp = h + hs * n_ff + bb * kQK + 4 * lane;
      float v[4] = {hp[0], hp[1], hp[2], hp[3]};
      quantize_block_wave_lds(v, hs_dyn + b * kXStride, lane);
    }
    __syncthreads();
    for (int j = 0; j < n; ++j) {
      float s = 0.f;
      if (live) {
        int32_t xr[64], ip[8];
        float xd, bsf[8];
        load_x_regs(hs_dyn + (j * nbf + blk) * kXStride, xr, xd, bsf);
        subblock_dots(w36 + 4, xr, ip);
        s = block_sum(w36[0], sm8, ip, xd, bsf);
      }
      const float acc = row_sum_in_order(s, lane, lpr, nbf);
      if (blk == 0 && row < hidden) {
        const long long ysl = static_cast<long long>(toks[j]) * (k + 1) + slots[j];
        ys[ysl * hidden + row] = present ? acc : 0.f;
      }
    }
  }

  // last workgroup to finish this row chunk combines it
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) last = atomicAdd(&counters[blockIdx.x], 1) == n_groups - 1;
  __syncthreads();
  if (!last) return;
  __threadfence();
  const int has_shared = plan.meta[1];
  const int stride = k + 1;
  for (int q = threadIdx.x; q < T * rows_wg; q += blockDim.x) {
    const int t = q / rows_wg;
    const int r = blockIdx.x * rows_wg + (q - t * rows_wg);
    if (r >= hidden) continue;
    float acc = residual ? residual[static_cast<long long>(t) * hidden + r] : 0.f;
    for (int kk = 0; kk <= k; ++kk) {
      bool ok;
      if (kk < k) {
        const int ee = idx[t * stride + kk];
        ok = ee >= 0 && ee < n_expert;
      } else {
        ok = has_shared != 0;
      }
      const float yv = ok ? ys[(static_cast<long long>(t) * stride + kk) * hidden + r] : 0.f;
      acc = __builtin_fmaf(weight[t * stride + kk], yv, acc);
    }
    out[static_cast<long long>(t) * hidden + r] = acc;
  }
}

}  // namespace sg

using namespace sg;

extern "C" {

int sg_router_topk(const float* logits, int* idx, float* weight, int n_expert, int n_expert_used,
                   int idx_stride, int n_rows, float shared_w, void* stream) {
  if (!logits || !idx || !weight)
    return set_error(SG_ERR_INVALID_ARGUMENT, "sg_router_topk: null pointer");
  if (n_expert <= 0 || n_expert > kMaxExperts || n_expert_used <= 0 ||
      n_expert_used > n_expert || idx_stride < n_expert_used + 1 || n_rows <= 0)
    return set_error(SG_ERR_GEOMETRY,
                     "sg_router_topk: n_expert=%d (<=%d) n_expert_used=%d idx_stride=%d n_rows=%d",
                     n_expert, kMaxExperts, n_expert_used, idx_stride, n_rows);
  hipLaunchKernelGGL(router_kernel, dim3(n_rows), dim3(64), round4(n_expert) * sizeof(float),
                     static_cast<hipStream_t>(stream), logits, idx, weight, n_expert,
                     n_expert_used, idx_stride, shared_w);
  return check_launch("sg_router_topk");
}

int sg_silu_mul(float* out, const float* g, const float* u, int n, void* stream) {
  if (!out || !g || !u) return set_error(SG_ERR_INVALID_ARGUMENT, "sg_silu_mul: null pointer");
  if (n <= 0) return set_error(SG_ERR_GEOMETRY, "sg_silu_mul: n=%d", n);
  hipLaunchKernelGGL(silu_kernel, dim3((n + 255) / 256), dim3(256), 0,
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

size_t sg_moe_layer_workspace_bytes(int n_tokens, int hidden, int n_ff, int n_expert, int k) {
  if (n_tokens <= 0 || hidden <= 0 || n_ff <= 0 || n_expert <= 0 || k <= 0) return 0;
  return layer_ws(n_tokens, hidden, n_ff, n_expert, k).total;
}

int sg_moe_layer_stages(const sg_block_q4k* const* tab_gate, const sg_block_q4k* const* tab_up,
                        const sg_block_q4k* const* tab_down, const sg_block_q4k* sh_gate,
                        const sg_block_q4k* sh_up, const sg_block_q4k* sh_down, const float* x,
                        const float* logits, const float* residual, float* out, int* idx,
                        float* weight, void* workspace, size_t workspace_bytes, int n_tokens,
                        int hidden, int n_ff, int n_expert, int k, float shared_w, int stages,
                        void* stream) {
  const char* nm = "sg_moe_layer";
  if (stages <= 0 || stages > 7)
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: stages=%d not in 1..7", nm, stages);
  if (!tab_gate || !tab_up || !tab_down || !x || !out || !idx || !weight || !workspace)
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  const int n_sh = (sh_gate != nullptr) + (sh_up != nullptr) + (sh_down != nullptr);
  if (n_sh != 0 && n_sh != 3)
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: shared expert needs gate, up and down", nm);
  if (n_tokens <= 0 || n_tokens > kMaxLayerTokens)
    return set_error(SG_ERR_UNSUPPORTED, "%s: n_tokens=%d not in [1,%d]", nm, n_tokens,
                     kMaxLayerTokens);
  if (hidden <= 0 || hidden % kQK || n_ff <= 0 || n_ff % kQK)
    return set_error(SG_ERR_GEOMETRY, "%s: hidden=%d n_ff=%d must be multiples of 256", nm, hidden,
                     n_ff);
  if (hidden > 32 * kQK || n_ff > 64 * kQK)
    return set_error(SG_ERR_UNSUPPORTED, "%s: hidden=%d (<=8192) n_ff=%d (<=16384)", nm, hidden,
                     n_ff);
  if (k <= 0 || k > kMaxK || n_expert < k || n_expert > kMaxExperts)
    return set_error(SG_ERR_GEOMETRY, "%s: k=%d (<=%d) n_expert=%d (k..%d)", nm, k, kMaxK,
                     n_expert, kMaxExperts);
  const size_t lds_x = static_cast<size_t>(n_tokens) * (hidden / kQK) * kXStride * 4;
  const size_t lds_h = static_cast<size_t>(n_tokens) * (n_ff / kQK) * kXStride * 4;
  const size_t lds_e = static_cast<size_t>(n_tokens) * round4(n_expert) * 4;
  if (lds_x > 64 * 1024 || lds_h > 64 * 1024 || lds_e > 48 * 1024)
    return set_error(SG_ERR_UNSUPPORTED, "%s: n_tokens*hidden or n_tokens*n_ff too large", nm);
  const LayerWs ws = layer_ws(n_tokens, hidden, n_ff, n_expert, k);
  if (workspace_bytes < ws.total)
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: workspace %zu < %zu bytes", nm,
                     workspace_bytes, ws.total);
  unsigned char* base = static_cast<unsigned char*>(workspace);
  LayerPlan plan{reinterpret_cast<int*>(base + ws.meta), reinterpret_cast<int*>(base + ws.off),
                 reinterpret_cast<int*>(base + ws.expert), reinterpret_cast<int*>(base + ws.tok),
                 reinterpret_cast<int*>(base + ws.slot)};
  unsigned char* xq = base + ws.xq;
  float* h = reinterpret_cast<float*>(base + ws.h);
  float* ys = reinterpret_cast<float*>(base + ws.ys);
  int* counters = reinterpret_cast<int*>(base + ws.counters);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int has_shared = n_sh == 3;

  if (stages & 1) {
    hipLaunchKernelGGL(layer_route_kernel, dim3(1), dim3(1024), lds_e, s, x, logits, idx, weight,
                       xq, plan, counters, ws.chunks, n_tokens, hidden, n_expert, k, shared_w,
                       has_shared);
    if (int st = check_launch("sg_moe_layer/route")) return st;
  }
  if (stages & 2) {
    const int gu_rows_wg = 4 * (32 / lpr_of(hidden / kQK));
    hipLaunchKernelGGL(layer_gateup_kernel, dim3((n_ff + gu_rows_wg - 1) / gu_rows_wg, ws.gmax),
                       dim3(256), lds_x, s, tab_gate, tab_up, sh_gate, sh_up, xq, plan, h,
                       n_tokens, hidden, n_ff, k);
    if (int st = check_launch("sg_moe_layer/gateup")) return st;
  }
  if (stages & 4) {
    hipLaunchKernelGGL(layer_down_kernel, dim3(ws.chunks, ws.gmax), dim3(256), lds_h, s,
                       tab_gate, tab_up, tab_down, sh_gate, sh_up, sh_down, plan, h, ys, idx,
                       weight, residual, out, counters, n_tokens, hidden, n_ff, n_expert, k);
    if (int st = check_launch("sg_moe_layer/down")) return st;
  }
  return SG_OK;
}

int sg_moe_layer(const sg_block_q4k* const* tab_gate, const sg_block_q4k* const* tab_up,
                 const sg_block_q4k* const* tab_down, const sg_block_q4k* sh_gate,
                 const sg_block_q4k* sh_up, const sg_block_q4k* sh_down, const float* x,
                 const float* logits, const float* residual, float* out, int* idx,
                 float* weight, void* workspace, size_t workspace_bytes, int n_tokens, int hidden,
                 int n_ff, int n_expert, int k, float shared_w, void* stream) {
  return sg_moe_layer_stages(tab_gate, tab_up, tab_down, sh_gate, sh_up, sh_down, x, logits,
                             residual, out, idx, weight, workspace, workspace_bytes, n_tokens,
                             hidden, n_ff, n_expert, k, shared_w, 7, stream);
}

}  // extern "C"
