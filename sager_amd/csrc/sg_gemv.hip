// sg_gemv.hip - the Q4_K x Q8_K GEMV family on gfx950.
//
// Work unit: a wave owns a row group of 64/lpr rows, lpr = the power of two
// >= nb (nb = k/256 super-blocks per row).  The group's bytes are contiguous
// in HBM, so the wave streams them into its own 9 KB LDS buffer with
// global_load_lds_dwordx4 (1 KB of consecutive memory per instruction, no
// registers held while in flight).  Lane l then reads super-block (l mod
// lpr) of row (l / lpr) from LDS (144-B stride: conflict-free), computes the
// eight int32 sub-block dots with v_dot4_i32_i8 against its Q8_K activation
// block kept in registers, applies the fp32 super-block epilogue, and the
// lpr block sums of a row are added in block order (the reference's
// acc += sum order, q4_avx2.cpp:130-143) with DPP lane shifts.  The next group's copy is issued
// as soon as the block is in registers, so it overlaps the arithmetic.
//
// Small matrices (up to 262144 super-blocks) take gemv_lat_kernel instead:
// four lanes per super-block, loads straight into registers, one pass.
//
// Reference kernels replaced: gemv_q4_k_q8 / gemv_mtok_ro_f32_kernel
// (q4_k.cu:57-91, 1360-1422, 1534-1562), gemv_q4_k_q8_batched and the mtok
// variants (q4_k.cu:218-282, 359-498), gemv_ptrs_q4_k_q8_f16out
// (q4_k.cu:184-213).
#include <type_traits>

#include "sg_common.hpp"

namespace sg {

constexpr int kMaxNb = 64;       // k <= 16384
constexpr int kMaxTokens = 16;   // batched GEMV token tile
constexpr int kWaves = 4;        // waves per workgroup
constexpr int kBufWords = 64 * 36;  // one wave's 9216-B weight buffer
constexpr int kWgPerCu = 2;        // grid cap: workgroups per CU

struct PlainRows {
  const sg_block_q4k* w;
  int nb;
  __device__ const char* row(int r) const {
    return reinterpret_cast<const char*>(w + static_cast<long long>(r) * nb);
  }
  __device__ void stage(uint32_t*, int, int) {}
  __device__ void attach(const uint32_t*) {}
  __device__ bool contiguous(int, int) const { return true; }
  __device__ int table_words() const { return 0; }
};

// Rows of n_ptrs matrices of rows_per rows each, matrix e at ptrs[e].  With
// n_ptrs <= kMaxLdsPtrs the table is copied to LDS once per workgroup, so
// the address of a row group costs an LDS read instead of a dependent
// global load in front of every weight stream.
constexpr int kMaxLdsPtrs = 2048;
// Up to three matrices of the same K stacked: rows [0, end[0]) of w[0],
// [end[0], end[1]) of w[1], [end[1], end[2]) of w[2] (the layer's q|k|v or
// qkvz|ba projections, gemv2m/gemv3m).
struct SegRows {
  const sg_block_q4k* w[3];
  int end[3];
  int nb;
  __device__ int seg(int r) const { return r < end[0] ? 0 : (r < end[1] ? 1 : 2); }
  __device__ const char* row(int r) const {
    const int m = seg(r);
    const int lr = r - (m ? end[m - 1] : 0);
    return reinterpret_cast<const char*>(w[m] + static_cast<long long>(lr) * nb);
  }
  __device__ void stage(uint32_t*, int, int) {}
  __device__ void attach(const uint32_t*) {}
  __device__ bool contiguous(int r0, int n) const { return seg(r0) == seg(r0 + n - 1); }
  __device__ int table_words() const { return 0; }
};
typedef __attribute__((address_space(3))) const unsigned long long lds_u64;
struct TableRows {
  const sg_block_q4k* const* ptrs;
  int rows_per, nb, n_ptrs;
  int shift;  // log2(rows_per) when it is a power of two, else -1
  // the staged table, as an LDS pointer: a generic pointer would make the
  // lookup a flat load, which joins the vector-memory queue and is waited
  // for together with the weight copies in flight
  lds_u64* lds = nullptr;
  __device__ int matrix(int r) const { return shift >= 0 ? r >> shift : r / rows_per; }
  __device__ const char* row(int r) const {
    const int e = matrix(r);
    const unsigned long long base =
        lds ? lds[e] : reinterpret_cast<unsigned long long>(ptrs[e]);
    return reinterpret_cast<const char*>(base) +
           static_cast<long long>(r - e * rows_per) * nb * kQ4Bytes;
  }
  // copy the table to LDS (visible after the caller's barrier)
  __device__ void stage(uint32_t* dst, int tid, int nthreads) {
    if (n_ptrs > kMaxLdsPtrs) return;
    unsigned long long* d = reinterpret_cast<unsigned long long*>(dst);
    for (int i = tid; i < n_ptrs; i += nthreads) d[i] = reinterpret_cast<unsigned long long>(ptrs[i]);
  }
  __device__ void attach(const uint32_t* src) {
    if (n_ptrs <= kMaxLdsPtrs) lds = (lds_u64*)(src);
  }
  __device__ bool contiguous(int r0, int n) const { return matrix(r0) == matrix(r0 + n - 1); }
  // LDS words the staged table occupies (2 per pointer, when it is staged)
  __device__ int table_words() const { return n_ptrs <= kMaxLdsPtrs ? 2 * n_ptrs : 0; }
};

__host__ __device__ inline int lanes_per_row(int nb) {
  int l = 1;
  while (l < nb) l <<= 1;
  return l;
}

// Issue the copy of rows r0 .. r0+n-1 into buf.  Rows that are contiguous
// in memory (always for a plain matrix; for a table when the group does not
// straddle two matrices) stream as one range: chunk c at base + 16c, with no
// per-chunk division.
template <typename Rows>
__device__ __forceinline__ void dma_rows(const Rows& rows, int r0, int n, int nb, uint32_t* buf,
                                         int lane) {
  const int cpr = nb * 9;  // 16-B chunks per row
  if (rows.contiguous(r0, n)) {
    const char* base = rows.row(r0);
    dma_chunks<kNt>([&](int c) { return base + 16 * c; }, n * cpr, buf, lane);
  } else {
    dma_chunks<kNt>([&](int c) { return rows.row(r0 + c / cpr) + 16 * (c % cpr); }, n * cpr, buf,
               lane);
  }
}

// y[r] = W[r] . x, one token.  Wave W of the NW takes the row groups W,
// W + NW, W + 2 NW, ... (a group = 64/lpr rows, one 9 KB buffer), so that the
// chip reads one window of the matrix at a time (contiguous ranges per wave
// measured 2-4 % slower); it issues the
// next group's copy as soon as the current one has been read into
// registers, so one group is always in flight while it computes.  The row
// results stay in LDS until the wave's last group and are then written
// together: a global store between the copies would sit in the vmcnt queue
// that each copy is waited on with.  Two workgroups per CU.
// Where a row result goes: fp32 y[r] (F32Out); fp16 into the row's segment
// output (F16SegOut, gemv2m/3m); fp16 y[r] and the residual add
// res[r] = f16(f32(res[r]) + f32(y[r])) (F16ResAddOut, add_kernel's
// semantics).  fp16 conversions round to nearest even (__float2half).
struct F32Out {
  float* y;
  __device__ void store(int r, float v) const { y[r] = v; }
};
struct F16Out {
  uint16_t* y;
  __device__ void store(int r, float v) const { y[r] = f16b(v); }
};
struct F16SegOut {
  uint16_t* y[3];
  int end[3];
  __device__ void store(int r, float v) const {
    const int m = r < end[0] ? 0 : (r < end[1] ? 1 : 2);
    y[m][r - (m ? end[m - 1] : 0)] = f16b(v);
  }
};
struct F16ResAddOut {
  uint16_t* y;
  uint16_t* res;
  __device__ void store(int r, float v) const {
    const uint16_t h = f16b(v);
    y[r] = h;
    res[r] = f16b(f16v(res[r]) + f16v(h));
  }
};

template <typename Rows, typename Out, int NWV>
__global__ void __launch_bounds__(64 * NWV) gemv1_kernel(Rows rows,
                                                         const unsigned char* __restrict__ xq,
                                                         Out out, int n_rows, int nb, int lpr,
                                                         int gpw) {
  __shared__ __attribute__((aligned(16))) uint32_t wbuf[NWV][kBufWords];
  extern __shared__ __attribute__((aligned(16))) uint32_t xs_dyn[];  // nb * kXStride, table, results
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int rpw = 64 / lpr;
  const int n_groups = (n_rows + rpw - 1) / rpw;
  const int NW = gridDim.x * NWV;
  const int g_begin = blockIdx.x * NWV + wv, g_end = n_groups;
  auto rows_of = [&](int gg) { return min(rpw, n_rows - gg * rpw); };
  // the first group's weights first: their HBM latency overlaps the staging
  if (g_begin < g_end) dma_rows(rows, g_begin * rpw, rows_of(g_begin), nb, wbuf[wv], lane);
  stage_q8k(xq, nb, xs_dyn, threadIdx.x, blockDim.x);
  uint32_t* tab = xs_dyn + nb * kXStride;  // row table, when the rows have one
  rows.stage(tab, threadIdx.x, blockDim.x);
  float* res = reinterpret_cast<float*>(tab + rows.table_words()) + wv * gpw * rpw;
  bar();
  rows.attach(tab);

  const int blk = lane & (lpr - 1);
  const int rr = lane / lpr;
  const bool active = blk < nb;
  int32_t xr[64];
  float xd = 0.f, bsf[8];
  load_x_regs(xs_dyn + (active ? blk : 0) * kXStride, xr, xd, bsf);

  for (int g = g_begin, li = 0; g < g_end; g += NW, ++li) {
    const int n = rows_of(g);
    wait_vm();  // group g has landed
    uint32_t w36[36];
    const bool live = active && rr < n;
    if (live) read_block_lds(wbuf[wv] + (rr * nb + blk) * 36, w36);
    wait_lds();
    if (g + NW < g_end) dma_rows(rows, (g + NW) * rpw, rows_of(g + NW), nb, wbuf[wv], lane);
    const float s = live ? q4k_block_dot(w36, xr, xd, bsf) : 0.f;
    const float acc = row_sum_last(s, blk, nb);
    if (blk == nb - 1 && rr < n) res[li * rpw + rr] = acc;
  }
  wait_lds();  // this wave's result writes (read back by its own lanes)
  // result li * rpw + row of the wave belongs to group g_begin + li * NW
  for (int i = lane; i < gpw * rpw; i += 64) {
    const int r = (g_begin + (i / rpw) * NW) * rpw + i % rpw;
    if (r < n_rows) out.store(r, res[i]);
  }
}

// y[r] = W[r] . x for a small matrix (latency-bound: a few MB, read in one
// pass by the whole chip).  Four lanes share a super-block, each taking one
// sub-block pair (8 qs words of weights, 16 qs words of activations), so a
// 2048 x 2048 matrix spreads over 1024 one-wave workgroups instead of 256
// waves.  Every lane loads its weight and activation words straight into
// registers at entry: no LDS, no barrier, one memory latency before the
// arithmetic.  The super-block epilogue keeps the reference's order
// (sum = fma(xd, t_s, sum) for s = 0..7, q4_avx2.cpp:30-39,134-141): the
// running sum moves from the lane of pair p to that of pair p+1 with a DPP
// row shift, and the row's block sums are then added in block order by
// row_sum_last after one lane permute.  nb <= 16 (k <= 4096).
constexpr int kLatMaxNb = 16;
constexpr int kLatWaves = 4;  // waves per workgroup
constexpr int kDppRowShr1 = 0x111;
typedef uint32_t u32x4u __attribute__((ext_vector_type(4), aligned(4)));

template <typename Rows, typename Out>
__device__ __forceinline__ void gemv_lat_body(const Rows& rows, const unsigned char* __restrict__ xq,
                                              const Out& out, int n_rows, int nb, int lg) {
  const int lpr = 1 << lg;
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * kLatWaves + (threadIdx.x >> 6);
  const int part = lane & 3, blk = (lane >> 2) & (lpr - 1), rr = lane >> (2 + lg);
  const int rpw = 16 >> lg;
  const int r = wave * rpw + rr;
  const bool live = blk < nb && r < n_rows;
  // every lane loads (clamped to a valid block) and dead lanes zero their
  // words afterwards: no branch, so all arguments are fetched in one round
  const u32x4* wp = reinterpret_cast<const u32x4*>(rows.row(min(r, n_rows - 1)) +
                                                   min(blk, nb - 1) * kQ4Bytes);
  u32x4 h = wp[0], qa = wp[1 + 2 * part], qb = wp[2 + 2 * part];
  const unsigned char* xb = xq + min(blk, nb - 1) * kQ8Bytes;
  const u32x4u* xp = reinterpret_cast<const u32x4u*>(xb + 4 + 64 * part);
  uint32_t xw[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x4u v = xp[i];
    xw[4 * i] = v.x;
    xw[4 * i + 1] = v.y;
    xw[4 * i + 2] = v.z;
    xw[4 * i + 3] = v.w;
  }
  float xd = *reinterpret_cast<const float*>(xb);
  uint32_t bs = *reinterpret_cast<const uint32_t*>(xb + 260 + 4 * part);
  if (!live) {
    h = u32x4{0u, 0u, 0u, 0u};
    qa = h;
    qb = h;
    bs = 0;
    xd = 0.f;
  }
  const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
  int32_t lo = 0, hi = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    lo = __builtin_amdgcn_sdot4(static_cast<int>(q[j] & 0x0F0F0F0Fu), static_cast<int>(xw[j]), lo,
                                false);
    hi = __builtin_amdgcn_sdot4(static_cast<int>((q[j] >> 4) & 0x0F0F0F0Fu),
                                static_cast<int>(xw[8 + j]), hi, false);
  }
  const ScaleMins sm8 = unpack_scales(h.y, h.z, h.w);
  const float d = half_bits_to_float(h.x & 0xFFFFu);
  const float dmin = half_bits_to_float(h.x >> 16);
  const uint32_t scw = part < 2 ? sm8.sc_lo : sm8.sc_hi;
  const uint32_t mnw = part < 2 ? sm8.mn_lo : sm8.mn_hi;
  const int i0 = (2 * part) & 3;
  const float b0 = static_cast<float>(static_cast<int16_t>(bs & 0xFFFFu));
  const float b1 = static_cast<float>(static_cast<int16_t>(bs >> 16));
  const float t0 = __builtin_fmaf(d * byte_f(scw, i0), static_cast<float>(lo),
                                  -((dmin * byte_f(mnw, i0)) * b0));
  const float t1 = __builtin_fmaf(d * byte_f(scw, i0 + 1), static_cast<float>(hi),
                                  -((dmin * byte_f(mnw, i0 + 1)) * b1));
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float prev = j == 0 ? 0.f : dpp_f<kDppRowShr1>(acc);
    if (part == j) acc = __builtin_fmaf(xd, t1, __builtin_fmaf(xd, t0, prev));
  }
  // block sums (lane 4b+3 of each row) to lanes row*lpr + b
  const int c = lane & 15;
  const int src = ((c >> lg) << (2 + lg)) + 4 * (c & (lpr - 1)) + 3;
  const float sb = __builtin_bit_cast(
      float, __builtin_amdgcn_ds_bpermute(src << 2, __builtin_bit_cast(int, acc)));
  const int cb = c & (lpr - 1);
  const float row = row_sum_last(sb, cb, nb);
  const int ro = wave * rpw + (c >> lg);
  if (lane < 16 && cb == nb - 1 && ro < n_rows) out.store(ro, row);
}
template <typename Rows, typename Out>
__global__ void __launch_bounds__(64 * kLatWaves) gemv_lat_kernel(
    Rows rows, const unsigned char* __restrict__ xq, Out out, int n_rows, int nb, int lg) {
  gemv_lat_body(rows, xq, out, n_rows, nb, lg);
}
// The plain fp32 GEMV with scalar arguments only, which the code object can
// preload into SGPRs (no kernel-argument load before the first address).
__global__ void __launch_bounds__(64 * kLatWaves) gemv_lat_plain_kernel(
    const sg_block_q4k* __restrict__ w, const unsigned char* __restrict__ xq, float* y, int n_rows,
    int nb, int lg) {
  gemv_lat_body(PlainRows{w, nb}, xq, F32Out{y}, n_rows, nb, lg);
}

// y[t*n_rows + r] = W[r] . x[t] for t < n_tokens; weights read once.  The
// row result goes out through Out (fp32, or rounded to fp16).
template <typename Out>
__global__ void __launch_bounds__(256) gemv_batched_kernel(const sg_block_q4k* __restrict__ w,
                                                           const unsigned char* __restrict__ xq,
                                                           Out y, int n_rows,
                                                           int nb, int lpr, int n_tokens) {
  __shared__ __attribute__((aligned(16))) uint32_t wbuf[kWaves][kBufWords];
  extern __shared__ __attribute__((aligned(16))) uint32_t xs_dyn[];  // T * nb * kXStride
  const PlainRows rows{w, nb};
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int rpw = 64 / lpr;
  const int n_groups = (n_rows + rpw - 1) / rpw;
  const int n_waves = gridDim.x * kWaves;
  int g = blockIdx.x * kWaves + wv;
  uint32_t* buf = wbuf[wv];
  if (g < n_groups) dma_rows(rows, g * rpw, min(rpw, n_rows - g * rpw), nb, buf, lane);
  stage_q8k(xq, nb * n_tokens, xs_dyn, threadIdx.x, blockDim.x);
  __syncthreads();

  const int blk = lane & (lpr - 1);
  const int rr = lane / lpr;
  const bool active = blk < nb;
  for (; g < n_groups; g += n_waves) {
    const int r0 = g * rpw;
    const int n = min(rpw, n_rows - r0);
    wait_vm();
    uint32_t w36[36];
    const bool live = active && rr < n;
    if (live) read_block_lds(buf + (rr * nb + blk) * 36, w36);
    wait_lds();
    const int gn = g + n_waves;
    if (gn < n_groups) dma_rows(rows, gn * rpw, min(rpw, n_rows - gn * rpw), nb, buf, lane);
    ScaleMins sm8{};
    if (live) sm8 = unpack_scales(w36[1], w36[2], w36[3]);
    for (int t = 0; t < n_tokens; ++t) {
      float s = 0.f;
      if (live) {
        int32_t xr[64], ip[8];
        float xd, bsf[8];
        load_x_regs(xs_dyn + (t * nb + blk) * kXStride, xr, xd, bsf);
        subblock_dots(w36 + 4, xr, ip);
        s = block_sum(w36[0], sm8, ip, xd, bsf);
      }
      const float acc = row_sum_last(s, blk, nb);
      if (blk == nb - 1 && rr < n) y.store(t * n_rows + r0 + rr, acc);
    }
  }
}

// dots[(r*nb + b)*8 + s] = int32 sub-block dot (test hook).
__global__ void __launch_bounds__(256) subblock_dots_kernel(const sg_block_q4k* __restrict__ w,
                                                            const unsigned char* __restrict__ xq,
                                                            int32_t* __restrict__ dots,
                                                            int n_rows, int nb, int lpr) {
  __shared__ __attribute__((aligned(16))) uint32_t wbuf[kWaves][kBufWords];
  extern __shared__ __attribute__((aligned(16))) uint32_t xs_dyn[];
  const PlainRows rows{w, nb};
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int rpw = 64 / lpr;
  const int g = blockIdx.x * kWaves + wv;
  const int n_groups = (n_rows + rpw - 1) / rpw;
  const int r0 = g * rpw;
  const int n = g < n_groups ? min(rpw, n_rows - r0) : 0;
  if (n > 0) dma_rows(rows, r0, n, nb, wbuf[wv], lane);
  stage_q8k(xq, nb, xs_dyn, threadIdx.x, blockDim.x);
  __syncthreads();
  const int blk = lane & (lpr - 1);
  const int rr = lane / lpr;
  if (blk >= nb || rr >= n) return;
  int32_t xr[64];
  float xd, bsf[8];
  load_x_regs(xs_dyn + blk * kXStride, xr, xd, bsf);
  wait_vm();
  uint32_t w36[36];
  read_block_lds(wbuf[wv] + (rr * nb + blk) * 36, w36);
  int32_t ip[8];
  subblock_dots(w36 + 4, xr, ip);
  int32_t* o = dots + (static_cast<long long>(r0 + rr) * nb + blk) * 8;
#pragma unroll
  for (int s = 0; s < 8; ++s) o[s] = ip[s];
}

// Grid for a grid-stride row loop: every row group once, capped at two
// workgroups of four waves per CU (256 CUs) - enough copies in flight to
// stream HBM at full rate.
static unsigned gemv_grid(long long n_groups) {
  const long long wgs = (n_groups + kWaves - 1) / kWaves;
  const long long cap = 256LL * kWgPerCu;
  return static_cast<unsigned>(wgs < cap ? (wgs > 0 ? wgs : 1) : cap);
}

// gemv1_kernel's launch: waves per workgroup, grid, groups per wave and the
// LDS its per-wave results take.  (One wave per workgroup over more CUs was
// measured slower on the 2048 x 2048 matrix: each workgroup stages x again,
// with a quarter of the threads.)
struct Gemv1Launch {
  int nwv;
  unsigned grid;
  int gpw;
  size_t res_bytes;
};
static Gemv1Launch gemv1_launch(long long n_groups, int rpw) {
  Gemv1Launch l{};
  l.nwv = kWaves;
  l.grid = gemv_grid(n_groups);
  const long long waves = static_cast<long long>(l.grid) * l.nwv;
  l.gpw = static_cast<int>((n_groups + waves - 1) / waves);
  l.res_bytes = static_cast<size_t>(l.nwv) * l.gpw * rpw * 4;
  return l;
}

// Matrices of at most this many super-blocks (and nb <= 16) take
// gemv_lat_kernel.  Measured with cold matrices (graph replays over rotated
// copies), it is faster up to 32768 x 2048 (2048 x 2048: 3.35 against
// 4.84 us); from 65536 x 2048 on, the streaming kernel is (248320 x 2048:
// 52 against 57 us).
constexpr long long kLatMaxBlocks = 262144;
static bool use_lat(int n_rows, int nb) {
  return nb <= kLatMaxNb && static_cast<long long>(n_rows) * nb <= kLatMaxBlocks;
}
template <typename Rows, typename Out>
static void gemv_lat_go(hipStream_t s, Rows rows, const sg_block_q8k* x, Out out, int n_rows,
                        int nb) {
  const int lpr = lanes_per_row(nb), rpw = 16 / lpr;
  const int waves = (n_rows + rpw - 1) / rpw;
  const dim3 grid((waves + kLatWaves - 1) / kLatWaves), block(64 * kLatWaves);
  const unsigned char* xb = reinterpret_cast<const unsigned char*>(x);
  const int lg = __builtin_ctz(lpr);
  if constexpr (std::is_same_v<Rows, PlainRows> && std::is_same_v<Out, F32Out>)
    hipLaunchKernelGGL(gemv_lat_plain_kernel, grid, block, 0, s, rows.w, xb, out.y, n_rows, nb, lg);
  else
    hipLaunchKernelGGL((gemv_lat_kernel<Rows, Out>), grid, block, 0, s, rows, xb, out, n_rows, nb,
                       lg);
}

template <typename Rows, typename Out>
static void gemv1_go(const Gemv1Launch& L, size_t lds, hipStream_t s, Rows rows,
                     const sg_block_q8k* x, Out out, int n_rows, int nb, int lpr) {
  if (use_lat(n_rows, nb)) return gemv_lat_go(s, rows, x, out, n_rows, nb);
  const unsigned char* xb = reinterpret_cast<const unsigned char*>(x);
  if (L.nwv == 1)
    hipLaunchKernelGGL((gemv1_kernel<Rows, Out, 1>), dim3(L.grid), dim3(64), lds, s, rows, xb, out,
                       n_rows, nb, lpr, L.gpw);
  else
    hipLaunchKernelGGL((gemv1_kernel<Rows, Out, kWaves>), dim3(L.grid), dim3(64 * kWaves), lds, s,
                       rows, xb, out, n_rows, nb, lpr, L.gpw);
}

static int check_gemv_geometry(const char* name, int n_rows, int k) {
  if (n_rows <= 0 || k <= 0 || k % kQK != 0)
    return set_error(SG_ERR_GEOMETRY, "%s: n_rows=%d k=%d (k must be a positive multiple of 256)",
                     name, n_rows, k);
  if (k / kQK > kMaxNb)
    return set_error(SG_ERR_UNSUPPORTED, "%s: k=%d exceeds %d", name, k, kMaxNb * kQK);
  return SG_OK;
}

// one gemv1 launch over a row source and an output policy (shared by the
// fp16-output entry points)
template <typename Rows, typename Out>
static int launch_gemv1(Rows rows, const sg_block_q8k* x, Out out, int n_rows, int k,
                        hipStream_t s, const char* nm) {
  if (int st = check_gemv_geometry(nm, n_rows, k)) return st;
  const int nb = k / kQK, lpr = lanes_per_row(nb);
  const long long n_groups = (n_rows + (64 / lpr) - 1) / (64 / lpr);
  const Gemv1Launch L = gemv1_launch(n_groups, 64 / lpr);
  const size_t lds = static_cast<size_t>(nb) * kXStride * 4 + L.res_bytes;
  if (lds > 96 * 1024)
    return set_error(SG_ERR_UNSUPPORTED, "%s: n_rows=%d k=%d needs %zu B of LDS", nm, n_rows, k,
                     lds);
  gemv1_go(L, lds, s, rows, x, out, n_rows, nb, lpr);
  return check_launch(nm);
}

// the pointer-table GEMV over an output policy
template <typename Out>
static int launch_ptrs(const sg_block_q4k* const* ptrs, const sg_block_q8k* x, Out y, int n_ptrs,
                       int rows_per, int k, hipStream_t s, const char* nm) {
  if (!ptrs || !x) return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  if (n_ptrs <= 0 || rows_per <= 0 || static_cast<long long>(n_ptrs) * rows_per > 0x7fffffffLL)
    return set_error(SG_ERR_GEOMETRY, "%s: n_ptrs=%d rows_per=%d", nm, n_ptrs, rows_per);
  const int n_rows = n_ptrs * rows_per;
  if (int st = check_gemv_geometry(nm, n_rows, k)) return st;
  const int nb = k / kQK, lpr = lanes_per_row(nb);
  const long long n_groups = (n_rows + (64 / lpr) - 1) / (64 / lpr);
  const Gemv1Launch L = gemv1_launch(n_groups, 64 / lpr);
  const size_t lds = static_cast<size_t>(nb) * kXStride * 4 +
                     (n_ptrs <= kMaxLdsPtrs ? static_cast<size_t>(n_ptrs) * 8 : 0) + L.res_bytes;
  if (lds > 96 * 1024)
    return set_error(SG_ERR_UNSUPPORTED, "%s: n_rows=%d k=%d needs %zu B of LDS", nm, n_rows, k,
                     lds);
  gemv1_go(L, lds, s,
           TableRows{ptrs, rows_per, nb, n_ptrs,
                     (rows_per & (rows_per - 1)) == 0 ? __builtin_ctz(rows_per) : -1},
           x, y, n_rows, nb, lpr);
  return check_launch(nm);
}

// the batched GEMV over an output policy (fp32 or fp16 rows)
template <typename Out>
static int launch_batched(const sg_block_q4k* w, const sg_block_q8k* x, Out y, int n_rows, int k,
                          int n_tokens, hipStream_t s, const char* nm) {
  if (!w || !x) return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  if (int st = check_gemv_geometry(nm, n_rows, k)) return st;
  if (n_tokens <= 0 || n_tokens > kMaxTokens)
    return set_error(SG_ERR_UNSUPPORTED, "%s: n_tokens=%d not in [1,%d]", nm, n_tokens,
                     kMaxTokens);
  if (static_cast<long long>(n_rows) * n_tokens > 0x7fffffffLL)
    return set_error(SG_ERR_GEOMETRY, "%s: n_rows*n_tokens too large", nm);
  const int nb = k / kQK, lpr = lanes_per_row(nb);
  const size_t lds = static_cast<size_t>(nb) * n_tokens * kXStride * 4;
  if (lds > 96 * 1024)
    return set_error(SG_ERR_UNSUPPORTED, "%s: k*n_tokens too large for LDS", nm);
  const long long n_groups = (n_rows + (64 / lpr) - 1) / (64 / lpr);
  hipLaunchKernelGGL((gemv_batched_kernel<Out>), dim3(gemv_grid(n_groups)), dim3(256), lds, s, w,
                     reinterpret_cast<const unsigned char*>(x), y, n_rows, nb, lpr, n_tokens);
  return check_launch(nm);
}

}  // namespace sg

using namespace sg;

extern "C" {

int sg_gemv_q4_k_q8(const sg_block_q4k* w, const sg_block_q8k* x, float* y, int n_rows, int k,
                    void* stream) {
  const char* nm = "sg_gemv_q4_k_q8";
  if (!w || !x || !y) return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  return launch_gemv1(PlainRows{w, k / kQK}, x, F32Out{y}, n_rows, k,
                      static_cast<hipStream_t>(stream), nm);
}

int sg_gemv_ptrs_q4_k_q8(const sg_block_q4k* const* ptrs, const sg_block_q8k* x, float* y,
                         int n_ptrs, int rows_per, int k, void* stream) {
  if (!y) return set_error(SG_ERR_INVALID_ARGUMENT, "sg_gemv_ptrs_q4_k_q8: null pointer");
  return launch_ptrs(ptrs, x, F32Out{y}, n_ptrs, rows_per, k, static_cast<hipStream_t>(stream),
                     "sg_gemv_ptrs_q4_k_q8");
}

int sg_gemv_ptrs_q4_k_q8_f16out(const sg_block_q4k* const* ptrs, const sg_block_q8k* x,
                                uint16_t* y, int n_ptrs, int rows_per, int k, void* stream) {
  if (!y) return set_error(SG_ERR_INVALID_ARGUMENT, "sg_gemv_ptrs_q4_k_q8_f16out: null pointer");
  return launch_ptrs(ptrs, x, F16Out{y}, n_ptrs, rows_per, k, static_cast<hipStream_t>(stream),
                     "sg_gemv_ptrs_q4_k_q8_f16out");
}

int sg_gemv_q4_k_q8_batched(const sg_block_q4k* w, const sg_block_q8k* x, float* y, int n_rows,
                            int k, int n_tokens, void* stream) {
  if (!y) return set_error(SG_ERR_INVALID_ARGUMENT, "sg_gemv_q4_k_q8_batched: null pointer");
  return launch_batched(w, x, F32Out{y}, n_rows, k, n_tokens, static_cast<hipStream_t>(stream),
                        "sg_gemv_q4_k_q8_batched");
}

int sg_gemv_q4_k_q8_f16out_batched(const sg_block_q4k* w, const sg_block_q8k* x, uint16_t* y,
                                   int n_rows, int k, int n_tokens, void* stream) {
  if (!y) return set_error(SG_ERR_INVALID_ARGUMENT, "sg_gemv_q4_k_q8_f16out_batched: null pointer");
  return launch_batched(w, x, F16Out{y}, n_rows, k, n_tokens, static_cast<hipStream_t>(stream),
                        "sg_gemv_q4_k_q8_f16out_batched");
}

int sg_q4k_subblock_dots(const sg_block_q4k* w, const sg_block_q8k* x, int32_t* dots, int n_rows,
                         int k, void* stream) {
  if (!w || !x || !dots)
    return set_error(SG_ERR_INVALID_ARGUMENT, "sg_q4k_subblock_dots: null pointer");
  if (int st = check_gemv_geometry("sg_q4k_subblock_dots", n_rows, k)) return st;
  const int nb = k / kQK, lpr = lanes_per_row(nb);
  const long long n_groups = (n_rows + (64 / lpr) - 1) / (64 / lpr);
  hipLaunchKernelGGL(subblock_dots_kernel, dim3(static_cast<unsigned>((n_groups + 3) / 4)),
                     dim3(256), nb * kXStride * 4, static_cast<hipStream_t>(stream), w,
                     reinterpret_cast<const unsigned char*>(x), dots, n_rows, nb, lpr);
  return check_launch("sg_q4k_subblock_dots");
}

int sg_gemv_q4_k_q8_f16out(const sg_block_q4k* w, const sg_block_q8k* x, uint16_t* y, int n_rows,
                           int k, void* stream) {
  const char* nm = "sg_gemv_q4_k_q8_f16out";
  if (!w || !x || !y) return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  F16SegOut o{{y, y, y}, {n_rows, n_rows, n_rows}};
  return launch_gemv1(PlainRows{w, k / kQK}, x, o, n_rows, k, static_cast<hipStream_t>(stream),
                      nm);
}

int sg_gemv3m_q4_k_q8_f16out(const sg_block_q4k* w1, const sg_block_q4k* w2,
                             const sg_block_q4k* w3, const sg_block_q8k* x, uint16_t* y1,
                             uint16_t* y2, uint16_t* y3, int rows1, int rows2, int rows3, int k,
                             void* stream) {
  const char* nm = "sg_gemv3m_q4_k_q8_f16out";
  if (!w1 || !w2 || !x || !y1 || !y2 || (rows3 > 0 && (!w3 || !y3)))
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  if (rows1 <= 0 || rows2 <= 0 || rows3 < 0 ||
      static_cast<long long>(rows1) + rows2 + rows3 > 0x7fffffffLL)
    return set_error(SG_ERR_GEOMETRY, "%s: rows %d/%d/%d", nm, rows1, rows2, rows3);
  const int e0 = rows1, e1 = rows1 + rows2, e2 = e1 + rows3;
  SegRows rs{{w1, w2, rows3 > 0 ? w3 : w2}, {e0, e1, e2}, k / kQK};
  F16SegOut o{{y1, y2, rows3 > 0 ? y3 : y2}, {e0, e1, e2}};
  return launch_gemv1(rs, x, o, e2, k, static_cast<hipStream_t>(stream), nm);
}

int sg_gemv2m_q4_k_q8_f16out(const sg_block_q4k* w1, const sg_block_q4k* w2,
                             const sg_block_q8k* x, uint16_t* y1, uint16_t* y2, int rows1,
                             int rows2, int k, void* stream) {
  return sg_gemv3m_q4_k_q8_f16out(w1, w2, nullptr, x, y1, y2, nullptr, rows1, rows2, 0, k,
                                  stream);
}

int sg_gemv_q4_k_q8_f16out_resadd(const sg_block_q4k* w, const sg_block_q8k* x, uint16_t* y,
                                  uint16_t* res_inout, int n_rows, int k, void* stream) {
  const char* nm = "sg_gemv_q4_k_q8_f16out_resadd";
  if (!w || !x || !y || !res_inout) return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  return launch_gemv1(PlainRows{w, k / kQK}, x, F16ResAddOut{y, res_inout}, n_rows, k,
                      static_cast<hipStream_t>(stream), nm);
}

}  // extern "C"
