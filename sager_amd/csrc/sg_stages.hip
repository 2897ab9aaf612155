// sg_stages.hip - the reference's stage-by-stage launchers of the grouped
// MoE path, for a session that keeps its own stage order instead of the
// fused layer (sg_moe_layer / sg_moe_prefill):
//   dispatch plan -> gather the routed Q8_K rows expert-major ->
//   grouped gate+up (fp16 out) -> SiLU*up -> Q8_K of h -> grouped down ->
//   scatter the outputs back into the combine slab -> batched combine.
// Row and element counts that the plan decides live in device memory (the
// plan's meta block); the host only bounds the grids.  Every kernel here is
// a plain stream of rows: copies are 16-B (fp16 rows) or dword (Q8_K
// blocks) wide, and a launch's bound is checked before anything is issued.
//
// Reference launchers replaced (cuda_ops.hpp): gather_rows_q8 (:364-366),
// gather_rows_q8_n / gather_rows_f16_n (:226-231), silu_mul_f16_n
// (:232-234), quantize_q8_k_n (:235-237), gemv_grouped2_tab_q4_k_q8_f16out_mtok
// (:240-244), gemv_grouped_tab_q4_k_q8_f16out_mtok (:247-250),
// scatter_routed_f16 (:372-374), scatter_rows_f16 (:408-409).  Their
// kernels: moe.cu:152-156, 237-330, 446-491; norm_rotary.cu:145-156,
// 278-284; q4_k.cu:640-836, 1869-1990.
#include "sg_common.hpp"

namespace sg {

// ---- row copies -------------------------------------------------------------

// dst[r] = src[src_rows[r]] for r < n (n = *count when count is given),
// whole rows of `words` dwords.  Grid (chunks of 256 words, rows).
__global__ void __launch_bounds__(256) gather_words_kernel(uint32_t* __restrict__ dst,
                                                           const uint32_t* __restrict__ src,
                                                           const int* __restrict__ src_rows,
                                                           const int* __restrict__ count,
                                                           int words) {
  const int r = blockIdx.y;
  if (count && r >= *count) return;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= words) return;
  const long long s = src_rows[r];
  dst[static_cast<long long>(r) * words + i] = src[s * words + i];
}

// The same for fp16 rows of `hidden` values: 16-B chunks when vec (hidden a
// multiple of 8 and both buffers 16-B aligned: the model's rows), element by
// element otherwise.
__global__ void __launch_bounds__(256) gather_f16_kernel(uint16_t* __restrict__ dst,
                                                         const uint16_t* __restrict__ src,
                                                         const int* __restrict__ src_rows,
                                                         const int* __restrict__ count,
                                                         int hidden, bool vec) {
  const int r = blockIdx.y;
  if (count && r >= *count) return;
  const long long s = src_rows[r];
  if (vec) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= hidden / 8) return;
    reinterpret_cast<uint4*>(dst + static_cast<long long>(r) * hidden)[c] =
        reinterpret_cast<const uint4*>(src + s * hidden)[c];
  } else {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= hidden) return;
    dst[static_cast<long long>(r) * hidden + i] = src[s * hidden + i];
  }
}

// expert_y[row][kk] = grouped_out[gslot[row*n_used + kk]] (gslot < 0: the
// slot is left as it is); grid (chunks, rows, n_used).
__global__ void __launch_bounds__(256) scatter_routed_kernel(uint16_t* __restrict__ expert_y,
                                                             const uint16_t* __restrict__ grouped,
                                                             const int* __restrict__ gslot,
                                                             int n_used, int hidden, bool vec) {
  const int row = blockIdx.y, kk = blockIdx.z;
  const int gs = gslot[static_cast<long long>(row) * n_used + kk];
  if (gs < 0) return;
  const long long d = (static_cast<long long>(row) * (n_used + 1) + kk) * hidden;
  const long long s = static_cast<long long>(gs) * hidden;
  if (vec) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= hidden / 8) return;
    reinterpret_cast<uint4*>(expert_y + d)[c] = reinterpret_cast<const uint4*>(grouped + s)[c];
  } else {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < hidden) expert_y[d + i] = grouped[s + i];
  }
}

// dst[dst_rows[i]] = src[i], fp16 rows; grid (chunks, rows).
__global__ void __launch_bounds__(256) scatter_rows_kernel(uint16_t* __restrict__ dst,
                                                           const uint16_t* __restrict__ src,
                                                           const int* __restrict__ dst_rows,
                                                           int hidden, bool vec) {
  const int r = blockIdx.y;
  const long long d = static_cast<long long>(dst_rows[r]) * hidden;
  const long long s = static_cast<long long>(r) * hidden;
  if (vec) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= hidden / 8) return;
    reinterpret_cast<uint4*>(dst + d)[c] = reinterpret_cast<const uint4*>(src + s)[c];
  } else {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < hidden) dst[d + i] = src[s + i];
  }
}

// ---- device-count element-wise stages ------------------------------------------

// out[i] = f16(SiLU(g[i]) * u[i]) for i < *rows * n_ff (norm_rotary.cu:145-156;
// the same SiLU as sg_silu_mul_f16)
__global__ void __launch_bounds__(256) silu_f16_n_kernel(uint16_t* out, const uint16_t* g,
                                                         const uint16_t* u,
                                                         const int* __restrict__ rows, int n_ff) {
  const long long n = static_cast<long long>(*rows) * n_ff;
  const long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) out[i] = f16b(silu_mul(f16v(g[i]), f16v(u[i])));
}

// Q8_K of the first *rows * row_mult fp16 values (row_mult a multiple of
// 256): one wave per block, the arithmetic of sg_quantize_q8_k_f16
// (quantize_row_q8_K, q4_k.cpp:44-61); blocks past the count are not written.
__global__ void __launch_bounds__(256) quantize_f16_n_kernel(const uint16_t* __restrict__ x,
                                                             unsigned char* __restrict__ out,
                                                             const int* __restrict__ rows,
                                                             int row_mult) {
  const long long n_blocks = static_cast<long long>(*rows) * (row_mult / kQK);
  const long long blk = static_cast<long long>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (blk >= n_blocks) return;
  const uint16_t* xb = x + blk * kQK + 4 * lane;
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = half_bits_to_float(xb[i]);
  quantize_block_wave(v, out + blk * kQ8Bytes, lane);
}

// ---- grouped GEMVs driven by the dispatch plan ----------------------------------
// Tile t of the plan (t < meta[1]) is rows [tok0, tok0 + nt) of expert e's
// positions, e the last expert with toff[e] <= t, tok0 = (t - toff[e]) *
// tok_per (q4_k.cu:640-660 ff.).  Workgroup (x, t): four waves, wave w the
// rpw = 64 / lpr rows (4x + w) * rpw ..; lane = (row, super-block) as in
// the GEMV family, so each output is the fp32 row dot in the reference CPU
// order (q4_avx2.cpp:124-145) rounded once to fp16.  The tile's Q8_K rows
// (consecutive positions) are staged kTabTok at a time; the lane's weight
// block stays in registers for all of them.  With M = 2 the gate and the up
// matrix are done in turn.  An absent expert (a null matrix) zeroes the
// tile's outputs and, for the gate/up launch, posts its id once to the
// mailbox (mail[atomicAdd(mail_n, 1)] = e while that index < n_expert), as
// the reference does for its CPU fallback.
constexpr int kTabTok = 16;

__device__ __forceinline__ int expert_of_tile(const int* toff, int n_expert, int tile) {
  int lo = 0, hi = n_expert - 1, res = n_expert - 1;
  while (lo <= hi) {  // the last e with toff[e] <= tile
    const int mid = (lo + hi) >> 1;
    if (toff[mid + 1] <= tile) {
      lo = mid + 1;
    } else {
      res = mid;
      hi = mid - 1;
    }
  }
  return res;
}

template <int M>
__global__ void __launch_bounds__(256) grouped_tab_kernel(
    const sg_block_q4k* const* __restrict__ tab0, const sg_block_q4k* const* __restrict__ tab1,
    const int* __restrict__ off, const int* __restrict__ toff, const int* __restrict__ meta,
    int* __restrict__ mail, int* __restrict__ mail_n, const unsigned char* __restrict__ xq,
    uint16_t* __restrict__ y0, uint16_t* __restrict__ y1, int n_rows, int nb, int lpr,
    int n_expert, int tok_per) {
  __shared__ __attribute__((aligned(16))) uint32_t wbuf[4][64 * 36];
  extern __shared__ __attribute__((aligned(16))) uint32_t xs[];  // kTabTok * nb * kXStride
  const int tile = blockIdx.y;
  if (tile >= meta[1]) return;
  const int e = expert_of_tile(toff, n_expert, tile);
  const int joff = off[e], jm = off[e + 1] - joff;
  const int tok0 = (tile - toff[e]) * tok_per;
  const int nt = min(tok_per, jm - tok0);
  if (nt <= 0) return;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int rpw = 64 / lpr;
  const int r0 = (blockIdx.x * 4 + wv) * rpw;
  const int nr = max(0, min(rpw, n_rows - r0));
  const sg_block_q4k* w[2] = {tab0[e], M == 2 ? tab1[e] : nullptr};
  const long long p0 = static_cast<long long>(joff) + tok0;  // the tile's first position
  if (!w[0] || (M == 2 && !w[1])) {
    for (int i = lane; i < nt * nr; i += 64) {
      const long long o = (p0 + i / nr) * n_rows + r0 + i % nr;
      y0[o] = 0;
      if (M == 2) y1[o] = 0;
    }
    if (M == 2 && blockIdx.x == 0 && tid == 0) {
      const int mi = atomicAdd(mail_n, 1);
      if (mi < n_expert) mail[mi] = e;
    }
    return;
  }
  const int blk = lane & (lpr - 1), rr = lane / lpr;
  const bool live = blk < nb && rr < nr;
#pragma unroll 1
  for (int m = 0; m < M; ++m) {
    // the wave's rows are contiguous: nr * nb * 9 (<= 576) 16-B chunks
    const char* base = reinterpret_cast<const char*>(w[m] + static_cast<long long>(r0) * nb);
    if (nr > 0) dma_chunks<kNt>([&](int c) { return base + 16 * c; }, nr * nb * 9, wbuf[wv], lane);
    wait_vm();
    uint32_t w36[36];
    if (live) read_block_lds(wbuf[wv] + (rr * nb + blk) * 36, w36);
    ScaleMins sm8{};
    if (live) sm8 = unpack_scales(w36[1], w36[2], w36[3]);
    uint16_t* y = m == 0 ? y0 : y1;
#pragma unroll 1
    for (int c0 = 0; c0 < nt; c0 += kTabTok) {
      const int tc = min(kTabTok, nt - c0);
      __syncthreads();  // the previous chunk's reads are done
      stage_q8k(xq + (p0 + c0) * nb * kQ8Bytes, tc * nb, xs, tid, 256);
      __syncthreads();
      for (int t = 0; t < tc; ++t) {
        float s = 0.f;
        if (live) {
          int32_t xr[64], ip[8];
          float xd, bsf[8];
          load_x_regs(xs + (t * nb + blk) * kXStride, xr, xd, bsf);
          subblock_dots(w36 + 4, xr, ip);
          s = block_sum(w36[0], sm8, ip, xd, bsf);
        }
        const float acc = row_sum_last(s, blk, nb);
        if (blk == nb - 1 && rr < nr) y[(p0 + c0 + t) * n_rows + r0 + rr] = f16b(acc);
      }
    }
  }
}

}  // namespace sg

using namespace sg;

// 16-B copies of fp16 rows: whole rows of 8-value chunks, both buffers aligned
static bool vec16(const void* a, const void* b, int hidden) {
  return (hidden & 7) == 0 && ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15) == 0;
}

extern "C" {

int sg_gather_rows_q8(sg_block_q8k* dst, const sg_block_q8k* src, const int* src_rows,
                      int n_rows, int row_blocks, void* stream) {
  const char* nm = "sg_gather_rows_q8";
  if (!dst || !src || !src_rows) return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  if (n_rows <= 0 || n_rows > 65535 || row_blocks <= 0 || row_blocks > (1 << 20))
    return set_error(SG_ERR_GEOMETRY, "%s: n_rows=%d row_blocks=%d", nm, n_rows, row_blocks);
  const int words = row_blocks * (kQ8Bytes / 4);
  hipLaunchKernelGGL(gather_words_kernel, dim3((words + 255) / 256, n_rows), dim3(256), 0,
                     static_cast<hipStream_t>(stream), reinterpret_cast<uint32_t*>(dst),
                     reinterpret_cast<const uint32_t*>(src), src_rows, nullptr, words);
  return check_launch(nm);
}

int sg_gather_rows_q8_n(sg_block_q8k* dst, const sg_block_q8k* src, const int* src_rows,
                        const int* meta, int r_max, int row_blocks, void* stream) {
  const char* nm = "sg_gather_rows_q8_n";
  if (!dst || !src || !src_rows || !meta)
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  if (r_max <= 0 || r_max > 65535 || row_blocks <= 0 || row_blocks > (1 << 20))
    return set_error(SG_ERR_GEOMETRY, "%s: r_max=%d row_blocks=%d", nm, r_max, row_blocks);
  const int words = row_blocks * (kQ8Bytes / 4);
  hipLaunchKernelGGL(gather_words_kernel, dim3((words + 255) / 256, r_max), dim3(256), 0,
                     static_cast<hipStream_t>(stream), reinterpret_cast<uint32_t*>(dst),
                     reinterpret_cast<const uint32_t*>(src), src_rows, meta, words);
  return check_launch(nm);
}

int sg_gather_rows_f16_n(uint16_t* dst, const uint16_t* src, const int* src_rows,
                         const int* meta, int r_max, int hidden, void* stream) {
  const char* nm = "sg_gather_rows_f16_n";
  if (!dst || !src || !src_rows || !meta)
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  if (r_max <= 0 || r_max > 65535 || hidden <= 0)
    return set_error(SG_ERR_GEOMETRY, "%s: r_max=%d hidden=%d", nm, r_max, hidden);
  const bool vec = vec16(dst, src, hidden);
  const int per = vec ? hidden / 8 : hidden;
  hipLaunchKernelGGL(gather_f16_kernel, dim3((per + 255) / 256, r_max), dim3(256), 0,
                     static_cast<hipStream_t>(stream), dst, src, src_rows, meta, hidden, vec);
  return check_launch(nm);
}

int sg_scatter_routed_f16(uint16_t* expert_y, const uint16_t* grouped_out, const int* gslot,
                          int n_rows, int n_used, int hidden, void* stream) {
  const char* nm = "sg_scatter_routed_f16";
  if (!expert_y || !grouped_out || !gslot)
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  if (n_rows <= 0 || n_rows > 65535 || n_used <= 0 || n_used > 65535 || hidden <= 0)
    return set_error(SG_ERR_GEOMETRY, "%s: n_rows=%d n_used=%d hidden=%d", nm, n_rows, n_used,
                     hidden);
  const bool vec = vec16(expert_y, grouped_out, hidden);
  const int per = vec ? hidden / 8 : hidden;
  hipLaunchKernelGGL(scatter_routed_kernel, dim3((per + 255) / 256, n_rows, n_used), dim3(256),
                     0, static_cast<hipStream_t>(stream), expert_y, grouped_out, gslot, n_used,
                     hidden, vec);
  return check_launch(nm);
}

int sg_scatter_rows_f16(uint16_t* dst, const uint16_t* src, const int* dst_rows, int n_rows,
                        int hidden, void* stream) {
  const char* nm = "sg_scatter_rows_f16";
  if (!dst || !src || !dst_rows) return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  if (n_rows <= 0 || n_rows > 65535 || hidden <= 0)
    return set_error(SG_ERR_GEOMETRY, "%s: n_rows=%d hidden=%d", nm, n_rows, hidden);
  const bool vec = vec16(dst, src, hidden);
  const int per = vec ? hidden / 8 : hidden;
  hipLaunchKernelGGL(scatter_rows_kernel, dim3((per + 255) / 256, n_rows), dim3(256), 0,
                     static_cast<hipStream_t>(stream), dst, src, dst_rows, hidden, vec);
  return check_launch(nm);
}

int sg_silu_mul_f16_n(uint16_t* out, const uint16_t* g, const uint16_t* u, const int* d_rows,
                      int rows_max, int n_ff, void* stream) {
  const char* nm = "sg_silu_mul_f16_n";
  if (!out || !g || !u || !d_rows) return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  if (rows_max <= 0 || n_ff <= 0)
    return set_error(SG_ERR_GEOMETRY, "%s: rows_max=%d n_ff=%d", nm, rows_max, n_ff);
  const long long n = static_cast<long long>(rows_max) * n_ff;
  if ((n + 255) / 256 > 0x7fffffffLL)
    return set_error(SG_ERR_GEOMETRY, "%s: rows_max*n_ff=%lld too large", nm, n);
  hipLaunchKernelGGL(silu_f16_n_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256),
                     0, static_cast<hipStream_t>(stream), out, g, u, d_rows, n_ff);
  return check_launch(nm);
}

int sg_quantize_q8_k_n(const uint16_t* x, sg_block_q8k* out, const int* d_rows, int row_mult,
                       int n_max, void* stream) {
  const char* nm = "sg_quantize_q8_k_n";
  if (!x || !out || !d_rows) return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  if (row_mult <= 0 || row_mult % kQK != 0 || n_max <= 0)
    return set_error(SG_ERR_GEOMETRY,
                     "%s: row_mult=%d must be a positive multiple of 256, n_max=%d", nm, row_mult,
                     n_max);
  hipLaunchKernelGGL(quantize_f16_n_kernel, dim3((n_max + 3) / 4), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, reinterpret_cast<unsigned char*>(out),
                     d_rows, row_mult);
  return check_launch(nm);
}

}  // extern "C"

namespace sg {
template <int M>
static int grouped_tab_launch(const sg_block_q4k* const* tab0, const sg_block_q4k* const* tab1,
                              const int* off, const int* toff, const int* meta, int* mail,
                              int* mail_n, int tiles_max, const sg_block_q8k* xq, uint16_t* y0,
                              uint16_t* y1, int n_rows, int k, int n_expert, int tok_per,
                              void* stream, const char* nm) {
  if (!tab0 || !off || !toff || !meta || !xq || !y0 || (M == 2 && (!tab1 || !y1 || !mail || !mail_n)))
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  if (n_rows <= 0 || k <= 0 || k % kQK != 0 || k / kQK > 16 || n_expert <= 0 || tok_per <= 0 ||
      tiles_max <= 0 || tiles_max > 65535)
    return set_error(SG_ERR_GEOMETRY,
                     "%s: n_rows=%d k=%d (a multiple of 256, at most 4096) n_expert=%d "
                     "tok_per=%d tiles_max=%d",
                     nm, n_rows, k, n_expert, tok_per, tiles_max);
  const int nb = k / kQK;
  int lpr = 1;
  while (lpr < nb) lpr <<= 1;
  const int rows_wg = 4 * (64 / lpr);
  const size_t lds = static_cast<size_t>(kTabTok) * nb * kXStride * 4;
  hipLaunchKernelGGL(grouped_tab_kernel<M>, dim3((n_rows + rows_wg - 1) / rows_wg, tiles_max),
                     dim3(256), lds, static_cast<hipStream_t>(stream), tab0, tab1, off, toff, meta,
                     mail, mail_n, reinterpret_cast<const unsigned char*>(xq), y0, y1, n_rows, nb,
                     lpr, n_expert, tok_per);
  return check_launch(nm);
}
}  // namespace sg

extern "C" {

int sg_gemv_grouped2_tab_q4_k_q8_f16out(const sg_block_q4k* const* wg_tab,
                                        const sg_block_q4k* const* wu_tab, const int* off,
                                        const int* toff, const int* meta, int* mail, int* mail_n,
                                        int tiles_max, const sg_block_q8k* xq, uint16_t* yg,
                                        uint16_t* yu, int n_rows, int k, int n_expert, int tok_per,
                                        void* stream) {
  return grouped_tab_launch<2>(wg_tab, wu_tab, off, toff, meta, mail, mail_n, tiles_max, xq, yg,
                               yu, n_rows, k, n_expert, tok_per, stream,
                               "sg_gemv_grouped2_tab_q4_k_q8_f16out");
}

int sg_gemv_grouped_tab_q4_k_q8_f16out(const sg_block_q4k* const* w_tab, const int* off,
                                       const int* toff, const int* meta, int tiles_max,
                                       const sg_block_q8k* xq, uint16_t* y, int n_rows, int k,
                                       int n_expert, int tok_per, void* stream) {
  return grouped_tab_launch<1>(w_tab, nullptr, off, toff, meta, nullptr, nullptr, tiles_max, xq,
                               y, nullptr, n_rows, k, n_expert, tok_per, stream,
                               "sg_gemv_grouped_tab_q4_k_q8_f16out");
}

}  // extern "C"
