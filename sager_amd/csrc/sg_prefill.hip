// sg_prefill.hip - the multi-token (prefill chunk) MoE layer on gfx950 with
// int8 matrix cores.
//
// Stage order of the reference's grouped device path
// (Session::moe_dispatch_device, session.cpp:2643-2840):
//   Q8_K(x) -> router top-k (batched) -> dispatch scan into an expert-major
//   plan (moe.cu:366-444) -> grouped gate/up + SiLU -> Q8_K(h) -> grouped
//   down -> combine in slot order (moe.cu:265-280).
//
// The grouped contractions run on v_mfma_i32_16x16x32_i8: one MFMA is one
// Q4_K sub-block (32 weights) for 16 tokens x 16 weight rows, so every
// int32 sub-block dot is exact.  Per super-block each output keeps
// I = sum_s sc_s * ip_s and M = sum_s mn_s * bsum_s as exact integers; the
// fp32 epilogue is t = fma(d, I, -(dmin * M)), acc = fma(xd, t, acc) over
// the super-blocks in order (the integer-first order; the CPU oracle's
// orc_gemv_q4k_q8_int is the same arithmetic).
//
// Workgroup tile: 64 tokens x 128 weight rows (gate/up: 64 h rows of gate
// and the same 64 of up; down: 128 output rows), eight waves of 16 tokens x
// 64 rows each (gate/up: 32 h rows of gate and their up rows, so SiLU pairs
// meet in one lane), K streamed one super-block at a time through two LDS
// buffers (weights by global_load_lds, token rows gathered through
// registers).
#include "sg_common.hpp"
#include "sg_router.hpp"

namespace sg {

// ---- dispatch scan --------------------------------------------------------------
constexpr int kScanPerThread = 32;  // routes per thread: n_rows * k <= 32768
// One workgroup of 1024 threads.  Pass 1: per-expert route counts and a
// [expert][token] bitmap in LDS; invalid ids zero their row's weights
// (bounds-kill, moe.cu:385-396).  The exclusive scans give off/toff/meta.
// Pass 2 places every route at off[e] + (its rank among the expert's routes
// in token order) - a per-word prefix plus a popcount over the bitmap - so
// the plan is deterministic (the reference's atomic placement is not).  A token routed
// twice to one expert (caller-supplied ids) takes a serial placement.
// With shared_tail > 0, positions off[E] .. off[E] + shared_tail - 1 are the
// shared expert's (token t at off[E] + t) and off[E+1] closes them.
// Exclusive prefix sum of v over a 1024-thread workgroup (thread order);
// *total gets the sum.  tmp: 16 ints of LDS.  Contains three barriers.
__device__ __forceinline__ int block_exclusive_scan(int v, int* tmp, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;  // inclusive scan inside the wave
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) tmp[wave] = x;
  __syncthreads();
  int before = 0, all = 0;
  for (int w = 0; w < 16; ++w) {
    const int t = tmp[w];
    before += w < wave ? t : 0;
    all += t;
  }
  __syncthreads();  // tmp is reused by the caller's next scan
  *total = all;
  return before + x - v;
}

// One tile of the grouped kernels' work list: a group (expert, or E for the
// shared expert; -1 past the list), its positions [p0, p1), and the group's
// three matrices (absent: 0 when any of them is null).
struct TileRec {
  int g, p0, p1, pad;
  unsigned long long wg, wu, wd, pad2;
};

__global__ void __launch_bounds__(1024) dispatch_scan_kernel(
    const int* __restrict__ idx, float* __restrict__ weight, int* __restrict__ gslot,
    int* __restrict__ grows, int* __restrict__ off, int* __restrict__ toff,
    int* __restrict__ meta, int* __restrict__ tiles, int n_rows, int k, int n_expert, int tok_per,
    int shared_tail) {
  extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
  __shared__ int s_bad, s_dup, s_total;
  // W bitmap words per expert, stored at an odd stride WS: a wave's routes
  // share a token word, and an even stride would put all their experts' words
  // in one LDS bank
  const int E = n_expert, W = (n_rows + 31) / 32, WS = W | 1;
  int* hist = reinterpret_cast<int*>(lds);       // [E]
  int* offl = hist + E;                          // [E]
  int* part = offl + E;                          // [1024]
  uint32_t* bm = reinterpret_cast<uint32_t*>(part + 1024);  // [E][W] token bitmap
  int* pre = reinterpret_cast<int*>(bm + E * WS);           // [E][W] routes before each word
  const int tid = threadIdx.x, nth = blockDim.x;
  for (int i = tid; i < E; i += nth) hist[i] = 0;
  for (int i = tid; i < E * WS; i += nth) bm[i] = 0u;
  if (tid == 0) {
    s_bad = 0;
    s_dup = 0;
  }
  __syncthreads();
  const int total = n_rows * k;
  // route i = tid + nth j is (row i / k, slot i % k); when k divides nth the
  // row advances by nth / k per j and the slot is fixed (no division per route)
  const bool kdiv = nth % k == 0;
  const int r0 = tid / k, kk0 = tid - r0 * k, rstep = nth / k;
  auto row_of = [&](int j, int i) { return kdiv ? r0 + j * rstep : i / k; };
  // every route id this thread handles, loaded up front (independent loads
  // in flight together)
  int ids[kScanPerThread];
#pragma unroll
  for (int j = 0; j < kScanPerThread; ++j) {
    const int i = tid + nth * j;
    const int r = row_of(j, i), kk = kdiv ? kk0 : i - r * k;
    ids[j] = i < total ? idx[static_cast<long long>(r) * (k + 1) + kk] : -1;
  }
#pragma unroll
  for (int j = 0; j < kScanPerThread; ++j) {
    const int i = tid + nth * j;
    if (i >= total) break;
    const int r = row_of(j, i);
    const int e = ids[j];
    if (e < 0 || e >= E) {
      for (int q = 0; q <= k; ++q) weight[static_cast<long long>(r) * (k + 1) + q] = 0.f;
      gslot[i] = -1;
      atomicAdd(&s_bad, 1);
      continue;
    }
    const uint32_t bit = 1u << (r & 31);
    if (atomicOr(&bm[e * WS + (r >> 5)], bit) & bit) s_dup = 1;
  }
  __syncthreads();
  // the expert histogram: with distinct ids per row, the popcounts of the
  // expert's bitmap words (thread group of expert e, tpe threads, counts
  // its share of the words into part[]); with a duplicated id the bitmap
  // undercounts, so the ids are counted one by one
  const int tpe = max(1, nth / E);  // threads per expert
  const int pe = tid / tpe, pq = tid - pe * tpe;
  const int wpt = (W + tpe - 1) / tpe;
  const int pw0 = min(W, pq * wpt), pw1 = min(W, pw0 + wpt);
  if (!s_dup) {
    int c = 0;
    if (pe < E)
      for (int w = pw0; w < pw1; ++w) c += __popc(bm[pe * WS + w]);
    part[tid] = c;
    __syncthreads();
    if (tid < E) {
      int h = 0;
      for (int j = 0; j < tpe; ++j) h += part[tid * tpe + j];
      hist[tid] = h;
    }
  } else {
#pragma unroll
    for (int j = 0; j < kScanPerThread; ++j) {
      const int i = tid + nth * j;
      if (i >= total) break;
      const int e = ids[j];
      if (e >= 0 && e < E) atomicAdd(&hist[e], 1);
    }
  }
  __syncthreads();
  {  // exclusive prefix sums over the experts (E <= 1024: one per thread)
    const int h = tid < E ? hist[tid] : 0;
    const int tl = (h + tok_per - 1) / tok_per;
    int tot_h, tot_t;
    const int ph = block_exclusive_scan(h, part, &tot_h);
    const int pt = block_exclusive_scan(tl, part, &tot_t);
    if (tid < E) {
      off[tid] = ph;
      offl[tid] = ph;
      toff[tid] = pt;
    }
    if (tid == 0) {
      off[E] = tot_h;
      toff[E] = tot_t;
      off[E + 1] = tot_h + shared_tail;
      meta[0] = tot_h;
      meta[1] = tot_t;
      meta[2] = s_bad;
      s_total = tot_h;
    }
    if (tiles) {  // the work list: tiles[0] = count, then (group << 16 | tile) in group order
      if (tid < E)
        for (int j = 0; j < tl; ++j) tiles[1 + pt + j] = (tid << 16) | j;
      const int sh_t = (shared_tail + tok_per - 1) / tok_per;
      for (int j = tid; j < sh_t; j += nth) tiles[1 + tot_t + j] = (E << 16) | j;
      if (tid == 0) tiles[0] = tot_t + sh_t;
    }
  }
  __syncthreads();
  if (!s_dup) {
    // per-(expert, word) prefix of route counts, in place of the bitmap's
    // companion array pre[]: thread group of expert e scans its words (the
    // per-thread word counts are in part[] from the histogram; the scans
    // above used part[] as scratch, so they are counted again)
    int c = 0;
    if (pe < E)
      for (int w = pw0; w < pw1; ++w) c += __popc(bm[pe * WS + w]);
    part[tid] = c;
    __syncthreads();
    if (pe < E) {
      int run = offl[pe];
      for (int j = 0; j < pq; ++j) run += part[pe * tpe + j];
      for (int w = pw0; w < pw1; ++w) {
        pre[pe * WS + w] = run;
        run += __popc(bm[pe * WS + w]);
      }
    }
    __syncthreads();
    // every route independently: its position is the expert's offset plus
    // the routes of lower tokens (a popcount of the word's lower bits)
#pragma unroll
    for (int j = 0; j < kScanPerThread; ++j) {
      const int i = tid + nth * j;
      if (i >= total) break;
      const int r = row_of(j, i);
      const int ee = ids[j];
      if (ee < 0 || ee >= E) continue;
      const uint32_t word = bm[ee * WS + (r >> 5)];
      const int pos = pre[ee * WS + (r >> 5)] + __popc(word & ((1u << (r & 31)) - 1u));
      gslot[i] = pos;
      grows[pos] = r;
    }
  } else if (tid == 0) {  // duplicated ids in a row: serial placement in (token, slot) order
    for (int e = 0; e < E; ++e) hist[e] = offl[e];
    for (int i = 0; i < total; ++i) {
      const int r = i / k, kk = i - r * k;
      const int e = idx[static_cast<long long>(r) * (k + 1) + kk];
      if (e < 0 || e >= E) continue;
      const int pos = hist[e]++;
      gslot[i] = pos;
      grows[pos] = r;
    }
  }
  for (int t = tid; t < shared_tail; t += nth) grows[s_total + t] = t;
}

// ---- grouped int8-MFMA contraction ------------------------------------------------
// Positions of one group per tile, in blocks of 16: 96 holds every expert's
// routes at the config-5 shape (64 +- 8 per expert) in one tile, so each
// expert's weights are unpacked once per column slice, and two workgroups
// still fit a CU's LDS.
constexpr int kTokTile = 96;
constexpr int kTokBlocks = kTokTile / 16;
constexpr int kRowsWg = 128;                 // weight rows per workgroup
constexpr int kWRowWords = 36;               // one 144-B block
constexpr int kWBufWords = kRowsWg * kWRowWords;   // 18 KB
// prefill Q8 block ("Q8P", written by the prefill's own quantizers): a
// 16-B header (fp32 d, 12 B zero), the 256 qs bytes, then each sub-block sum
// s as two fp16 integers a = s >> 1 and b = s & 1 (eight a's, then eight
// b's): the operands of the exact fp16 MFMA for the mins term.  19 16-B
// chunks.
constexpr int kQ8PBytes = 304;
// staged Q8P block: qs (words 0-63), the a's (64-67), the b's (68-71), the
// header (d in word 72).  76 words = 19 16-B chunks: the stride is 12 banks
// mod 32, so eight lanes reading 16 B of eight consecutive rows (one
// ds_read_b128 pass) touch every bank once.
constexpr int kXRow = 76;
// a whole number of 64-lane copy instructions (1 KB each): the last one may
// run past the tile's rows, into this padding
constexpr int kXBufWords = (kTokTile * kXRow + 255) / 256 * 256;  // 29 KB
constexpr int kThreads = 512;                 // eight waves
constexpr int kDownSlicesPerWg = 8;  // down pass, nb <= 2
// LDS: one weight buffer (each wave refills its own rows once it has read
// them), two token buffers, the tile's token rows and the SiLU's exp table
// (64 doubles): 78 KB
constexpr size_t kGroupedLds = (kWBufWords + 2 * kXBufWords + kTokTile + 128) * 4;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

struct GroupedArgs {
  const unsigned char* xq;  // Q8P rows: x [T][nb] (gate/up) or h [P][nb] (down)
  const int* off;           // [G+1] position range of each group
  const int* grows;         // [P] token of each position (gate/up only)
  const TileRec* trec;      // work list: one record per tile, group -1 past it
  int n_rec;                // records in trec
  float* out;               // [P][n_out]: h (gate/up pass) or y (down)
  uint16_t* out16;          // [P][n_out] fp16 y (the down pass's kF16Out instances), or
                            // fp16 h (gate/up pass with r16: h is an fp16 value there)
  int nb;                   // super-blocks per weight row
  int n_rows;               // rows of each weight matrix
  int n_out;                // output row stride (= n_rows)
  int n_groups;
  int n_slices;             // column slices per tile
  int spw;                  // slices per workgroup (the kMulti down pass, nb <= 2: the
                            // token rows stay in LDS across them), a divisor of n_slices
  int r16;                  // gate/up pass on the session's fp16 buffers: g, u and h rounded
                            // to fp16 as the session stores them (session.cpp:2791-2803)
};

// One workgroup = one column slice of one tile (up to 128 positions of one
// group).  The 1-D grid is laid out so that every slice of a tile runs on
// one XCD and is dispatched together: workgroup L runs on XCD L % 8, and
// XCD x's j-th workgroup takes tile x + 8 (j / S), slice j % S.  The tile's
// token rows are then fetched from HBM once and served to its other slices
// from that XCD's L2.
// kF16Out (down pass): y is stored rounded to fp16 in out16, the form the
// session's fp16 combine reads it in (its f16out GEMVs, moe.cu:265-292).
template <bool kGateUp, bool kMulti = false, bool kF16Out = false>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4, 8)))
grouped_mfma_kernel(GroupedArgs a) {
  static_assert(!(kGateUp && kF16Out), "h stays fp32 (it is quantized next)");
  extern __shared__ __attribute__((aligned(16))) uint32_t gl_lds[];
  uint32_t* wbuf0 = gl_lds;
  uint32_t* xbuf0 = gl_lds + kWBufWords;
  int* trow = reinterpret_cast<int*>(gl_lds + kWBufWords + 2 * kXBufWords);
  double* etab = reinterpret_cast<double*>(trow + kTokTile);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  static_assert(kThreads == 512, "eight waves, one 16-row block each");
  // the workgroup's slices: sgrp * spw .. sgrp * spw + spw - 1, in turn
  const int spw = kMulti ? a.spw : 1, S = a.n_slices / spw;
  const int L = blockIdx.x, xcd = L & 7, jx = L >> 3;
  const int tile = xcd + 8 * (jx / S), sgrp = jx - (jx / S) * S;
  if (tile >= a.n_rec) return;
  const TileRec rec = a.trec[tile];
  const int g = rec.g, p0 = rec.p0, p1 = rec.p1;
  if (g < 0 || g >= a.n_groups || p0 >= p1) return;
  // gate/up pass: gate rows (a) and up rows (b); down pass: down rows
  const sg_block_q4k* ma = reinterpret_cast<const sg_block_q4k*>(kGateUp ? rec.wg : rec.wd);
  const sg_block_q4k* mb = reinterpret_cast<const sg_block_q4k*>(kGateUp ? rec.wu : rec.wd);
  const int nb = a.nb;
  // down: output columns [c0, c0 + 128) from weight rows c0 ..; gate/up:
  // h columns [c0, c0 + 64) from gate rows c0 .. (waves 0-3) and the same
  // up rows (waves 4-7)
  constexpr int kCols = kGateUp ? kRowsWg / 2 : kRowsWg;  // output columns per slice
  int c0 = sgrp * spw * kCols;
  const int lr = lane & 15, lq = lane >> 4;     // MFMA: row/column in the tile, K quarter

  if (!ma) {  // absent expert (a null gate, up or down matrix): its outputs are zero
    for (long long p = p0; p < p1; ++p)
      for (int r = tid; r < spw * kCols; r += kThreads) {
        if (kF16Out || (kGateUp && a.r16)) a.out16[p * a.n_out + c0 + r] = 0;
        else a.out[p * a.n_out + c0 + r] = 0.f;
      }
    return;
  }

  // the 128 weight rows of super-block b into buffer s (gate/up: 64 gate
  // rows, then the same 64 up rows).  Wave w copies chunks [144w, 144w+144)
  // (16 B each, chunk c = part c%9 of row c/9), rows of one matrix; the
  // per-lane offsets are fixed for the kernel, the block's offset b*144 goes
  // in the scalar offset (buffer_load ... lds).
  constexpr int kWChunks = kRowsWg * 9 / 8;  // 144 per wave
  const sg_block_q4k* mw = uniform_ptr((kGateUp && wave >= 4) ? mb : ma);
  const u32x4 rw4 = buffer_desc(mw, a.n_rows * nb * kQ4Bytes);
  uint32_t wofs[3];
  auto set_wofs = [&](int cs) {  // the per-lane chunk offsets of slice columns cs ..
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int cc = min(wave * kWChunks + lane + 64 * i, kRowsWg * 9 - 1);
      const int row = cc / 9, part = cc - row * 9;
      const int rr = kGateUp ? (row & 63) : row;
      wofs[i] = static_cast<uint32_t>((cs + rr) * nb) * kQ4Bytes + 16 * part;
    }
  };
  set_wofs(c0);
  auto stage_w = [&](int b) {  // into the wave's own rows of the weight buffer
#pragma unroll
    for (int i = 0; i < 3; ++i)
      if (64 * i + lane < kWChunks)
        dma16(wbuf0 + 4 * (wave * kWChunks + 64 * i), wofs[i], rw4, b * kQ4Bytes);
  };
  stage_w(0);  // the first weight block needs only the record: issued before the token rows
  // the tile's token rows of super-block b into token buffer s, 76 words per
  // token in 16-B chunks: LDS chunk c = 19t + j is filled from chunk
  // (j + 1) % 19 of token t's Q8P block (buffer_load_dwordx4 ... lds:
  // lane-consecutive chunks land LDS-consecutive); offsets are set per tile,
  // b*304 is the scalar offset.  Only the 16-token blocks that hold tokens
  // are copied.
  const int t0 = p0, nt = p1 - p0;
  const int ntb = (nt + 15) >> 4;  // token blocks holding tokens (wave-uniform)
  const int xchunks = ntb * 16 * 19;
  constexpr int kXInstr = (kTokTile * 19 / 64 + 7) / 8;  // per wave: 3
  const u32x4 rx4 = buffer_desc(a.xq, 0x7FFFFFFFu);
  uint32_t xofs[kXInstr];
  auto stage_x = [&](int b, int s) {
#pragma unroll
    for (int i = 0; i < kXInstr; ++i) {
      const int q = wave + 8 * i;  // the instruction's 64-chunk slice
      if (64 * q < xchunks)
        dma16(xbuf0 + s * kXBufWords + 256 * q, xofs[i], rx4, b * kQ8PBytes);
    }
  };

  if (kGateUp && tid < 64) etab[tid] = kExp2Tab64[tid];  // the SiLU's exp table
  if (tid < kTokTile) {  // block index of each token row (rows past nt repeat the first)
    const int t = tid < nt ? tid : 0;
    trow[tid] = (kGateUp ? a.grows[t0 + t] : t0 + t) * nb;
  }
  bar();
#pragma unroll
  for (int i = 0; i < kXInstr; ++i) {
    const int c = min(64 * (wave + 8 * i) + lane, kTokTile * 19 - 1);
    const int t = c / 19, j = c - t * 19;
    xofs[i] = static_cast<uint32_t>(trow[t]) * kQ8PBytes + 16 * (j == 18 ? 0 : j + 1);
  }
  // the wave's MFMA tiles: token blocks ti < ntb (16 tokens each) of weight
  // row block `wave`; the lane's four output tokens of block ti are the MFMA
  // result rows 16ti + 4lq + i, its weight row is 16 wave + lr.  The
  // weight-side work (nibble unpack, scales) is done once per super-block
  // and shared by every token block.
  float acc[kTokBlocks][4];
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  auto pmul = [](uint32_t q, uint32_t s2) -> int {  // 4 bytes x s2 (the same 16 bits twice)
    return __builtin_bit_cast(int, __builtin_bit_cast(u16x2, q) * __builtin_bit_cast(u16x2, s2));
  };

  stage_x(0, 0);
  if (kMulti && nb > 1) stage_x(1, 1);  // the whole tile's rows, kept for every slice
#pragma unroll 1
  for (int q = 0; q < spw; ++q, c0 += kCols) {
#pragma unroll
  for (int ti = 0; ti < kTokBlocks; ++ti)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[ti][i] = 0.f;
  for (int b = 0; b < nb; ++b) {
    const int s = b & 1;
    wait_vm();  // this wave's copies of block b have landed
    bar();      // ... and every wave's
    // the lane's weight words of block b into registers: the header and,
    // per K group, 16 qs bytes; then the wave refills its rows with block
    // b + 1 while it computes (the rows are the wave's own: no barrier)
    const uint32_t* Wl = wbuf0 + (16 * wave + lr) * kWRowWords;
    const uint4 whdr = *reinterpret_cast<const uint4*>(Wl);
    uint4 wq[4];
#pragma unroll
    for (int gq = 0; gq < 4; ++gq)
      wq[gq] = *reinterpret_cast<const uint4*>(Wl + 4 + 8 * gq + 4 * (lq & 1));
    wait_lds();
    if (b + 1 < nb) {  // the next block streams in while this one computes
      stage_w(b + 1);
      if (!kMulti) stage_x(b + 1, s ^ 1);
    } else if (kMulti && q + 1 < spw) {  // the next slice's first block
      set_wofs(c0 + kCols);
      stage_w(0);
    }
    const uint32_t* X = xbuf0 + s * kXBufWords;
    // I = sum_s sc_s * ip_s with the 6-bit scale split as sc = 8*sh + sl
    // (sh, sl in [0, 7]) and folded into the weight operand: nibble * sl
    // and nibble * sh are at most 105, so each byte of the packed product
    // stays an exact int8 and the products of four nibbles come from one
    // packed 16-bit multiply (no carry crosses a byte).  Then
    // I = 8 * C(sh) + C(sl), where each chain accumulates all eight
    // sub-blocks inside the MFMA (16x16x64, four K groups of 64; a lane's
    // A and B bytes only need to agree on the K order).  |C(sl)|, |C(sh)|
    // <= 8*7*32*15*127 fit int32, so I is exact.
    // The lane's 16 K bytes of group gq (64 weights) are 16 consecutive
    // ones: k = 64gq + 16lq + j, i.e. sub-block 2gq + (lq >> 1), the low
    // (lq < 2) or high nibbles of qs bytes 32gq + 16(lq & 1) + j - one
    // ds_read_b128 on each side.
    const ScaleMins sm = unpack_scales(whdr.y, whdr.z, whdr.w);
    const uint32_t scl[2] = {sm.sc_lo & 0x07070707u, sm.sc_hi & 0x07070707u};
    const uint32_t sch[2] = {(sm.sc_lo >> 3) & 0x07070707u, (sm.sc_hi >> 3) & 0x07070707u};
    const uint32_t nsh = 4 * (lq >> 1);                          // nibble of this lane
    const uint32_t sel_l = 0x0C000C00u + 0x00010001u * (lq >> 1);  // its sub-block's byte
    v4i bl[4], bh[4];
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const uint4 q = wq[gq];
      // sl and sh of sub-block 2gq + (lq >> 1), spread to both 16-bit halves
      const uint32_t sel = sel_l + 0x00010001u * ((2 * gq) & 3);
      const uint32_t sl = __builtin_amdgcn_perm(0u, scl[gq >> 1], sel);
      const uint32_t sh = __builtin_amdgcn_perm(0u, sch[gq >> 1], sel);
      const uint32_t n0 = (q.x >> nsh) & 0x0F0F0F0Fu, n1 = (q.y >> nsh) & 0x0F0F0F0Fu;
      const uint32_t n2 = (q.z >> nsh) & 0x0F0F0F0Fu, n3 = (q.w >> nsh) & 0x0F0F0F0Fu;
      bl[gq] = v4i{pmul(n0, sl), pmul(n1, sl), pmul(n2, sl), pmul(n3, sl)};
      bh[gq] = v4i{pmul(n0, sh), pmul(n1, sh), pmul(n2, sh), pmul(n3, sh)};
    }
    // M = sum_s mn_s * bsum_s by one fp16 MFMA, exactly: with bsum = 2 a + b
    // (a = bsum >> 1, b = bsum & 1, fp16 integers from the quantizer), K
    // quarters 0-1 pair 2 mn_s with a_s and quarters 2-3 pair mn_s with b_s
    // (s = 4 (lq & 1) + 0..3).  Every product and partial sum is an integer
    // below 2^24 (|M| <= 8 * 63 * 4064), so the fp32 accumulation is exact
    // and M arrives as the float the epilogue needs.
    const uint32_t dd = whdr.x;
    v4h bmn;
    {
      const uint32_t mw = (lq & 1) ? sm.mn_hi : sm.mn_lo;
      const uint32_t m2 = lq < 2 ? mw << 1 : mw;  // bytes <= 126: no carry
      // fp16 bits 0x6400 + v = 1024 + v; subtract 1024 exactly
      const h2 k1024 = {static_cast<_Float16>(-1024.f), static_cast<_Float16>(-1024.f)};
      const h2 f0 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, m2, 0x04010400u)) + k1024;
      const h2 f1 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, m2, 0x04030402u)) + k1024;
      bmn = v4h{f0.x, f0.y, f1.x, f1.y};
    }
    const float d = half_bits_to_float(dd & 0xFFFFu);
    const float dmin = half_bits_to_float(dd >> 16);
#pragma unroll
    for (int ti = 0; ti < kTokBlocks; ++ti) {
      if (ti >= ntb) continue;  // wave-uniform: a token block past the tile's end
      const uint32_t* Xt = X + (16 * ti + lr) * kXRow;
      const v4i z = {0, 0, 0, 0};
      v4i cl = z, ch = z;
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const uint4 xv = *reinterpret_cast<const uint4*>(Xt + 16 * gq + 4 * lq);
        const v4i av = {static_cast<int>(xv.x), static_cast<int>(xv.y), static_cast<int>(xv.z),
                        static_cast<int>(xv.w)};
        cl = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bl[gq], cl, 0, 0, 0);
        ch = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bh[gq], ch, 0, 0, 0);
      }
      const v4h ab = *reinterpret_cast<const v4h*>(Xt + 64 + 2 * lq);
      const v4f mf = __builtin_amdgcn_mfma_f32_16x16x16f16(ab, bmn, v4f{}, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int I = ch[i] * 8 + cl[i];
        const float xd = __builtin_bit_cast(float, X[(16 * ti + 4 * lq + i) * kXRow + 72]);
        const float t = __builtin_fmaf(d, static_cast<float>(I), -(dmin * mf[i]));
        acc[ti][i] = __builtin_fmaf(xd, t, acc[ti][i]);
      }
    }
  }
  // outputs of the lane's tokens
  if (kGateUp) {  // h = silu(gate) * up; wave w (gate) and w + 4 (up) hold the same h
    // positions and each takes half of them: the first half of the token
    // blocks in the gate wave, the second in the up wave, swapping the other
    // half through LDS
    bar();  // every wave is done with the token buffers
    float* pair = reinterpret_cast<float*>(xbuf0);  // [8 waves][kTokBlocks / 2 * 4][64 lanes]
    const bool up_wave = wave >= 4;
#pragma unroll
    for (int tj = 0; tj < kTokBlocks / 2; ++tj)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        pair[(wave * 2 * kTokBlocks + 4 * tj + i) * 64 + lane] =
            acc[up_wave ? tj : kTokBlocks / 2 + tj][i];
    bar();
    const int partner = wave ^ 4;
#pragma unroll
    for (int tj = 0; tj < kTokBlocks / 2; ++tj) {
      const int ti = up_wave ? kTokBlocks / 2 + tj : tj;
      if (ti >= ntb) continue;
      float gv[4], uv[4], hv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float other = pair[(partner * 2 * kTokBlocks + 4 * tj + i) * 64 + lane];
        gv[i] = up_wave ? other : acc[ti][i];
        uv[i] = up_wave ? acc[ti][i] : other;
      }
      if (a.r16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          gv[i] = f16r(gv[i]);
          uv[i] = f16r(uv[i]);
        }
      }
      silu_mul_tab_n<4>(gv, uv, hv, etab);
      if (a.r16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) hv[i] = f16r(hv[i]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tt = 16 * ti + 4 * lq + i;
        if (tt < nt)
        {
          const long long o = static_cast<long long>(t0 + tt) * a.n_out + c0 + 16 * (wave & 3) + lr;
          if (a.r16) a.out16[o] = f16b(hv[i]);
          else a.out[o] = hv[i];
        }
      }
    }
  } else {
    // the lane's first output row, opaque to the compiler: otherwise it
    // hoists the 24 store addresses out of the slice loop and spills
    int tl0 = t0 + 4 * lq;
    asm volatile("" : "+v"(tl0));
    float* ob = a.out + c0 + 16 * wave + lr;
    uint16_t* ob16 = a.out16 + c0 + 16 * wave + lr;
#pragma unroll
    for (int ti = 0; ti < kTokBlocks; ++ti) {
      if (ti >= ntb) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tt = 16 * ti + 4 * lq + i;
        if (tt < nt) {
          const long long o = static_cast<long long>(tl0 + 16 * ti + i) * a.n_out;
          if (kF16Out) ob16[o] = f16b(acc[ti][i]);
          else ob[o] = acc[ti][i];
        }
      }
    }
  }
  }  // slices
}

// ---- the dispatch plan over many workgroups (prefill path) ------------------
// The same arrays as dispatch_scan_kernel, in two launches:
// 1. plan_bits_kernel: workgroup w takes the R = 32 m tokens [R w, R w + R)
//    and writes wbits[w][e] (m words: the bitmap of its tokens routed to
//    expert e) and wflags[w] = bad routes | (duplicate id in a row) << 16;
//    an invalid id zeroes its row's weights (bounds-kill) and gets gslot -1;
// 2. plan_place_kernel: every workgroup sums the popcounts of each expert's
//    bitmap column - all of it (hist) and the part before its own tokens
//    (pre) - takes the exclusive scans (off, toff) and places its own
//    routes: a route of token r to expert e goes to off[e] + pre[e] + the
//    own routes of e from tokens below r, the token order within each expert,
//    as in the scan.  Workgroup 0 also writes off/toff/meta, the tile list
//    and the tile records.  A row with a duplicated id (caller routing only)
//    is placed serially in (token, slot) order by workgroup 0 alone, as
//    dispatch_scan_kernel does.
constexpr int kPlanThreads = 512;
constexpr int kPlanMaxWg = 256;   // bitmap workgroups; m grows with T beyond 256 * 32 tokens

__device__ __forceinline__ int plan_scan(int v, int* tmp, int* total) {
  // exclusive prefix sum over the workgroup (thread order); tmp: 16 ints
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) tmp[wave] = x;
  __syncthreads();
  int before = 0, all = 0;
  for (int w = 0; w < nw; ++w) {
    const int t = tmp[w];
    before += w < wave ? t : 0;
    all += t;
  }
  __syncthreads();
  *total = all;
  return before + x - v;
}

__global__ void __launch_bounds__(kPlanThreads) plan_bits_kernel(
    const int* __restrict__ idx, float* __restrict__ weight, int* __restrict__ gslot,
    uint32_t* __restrict__ wbits, int* __restrict__ wflags, int n_rows, int k, int E, int m) {
  extern __shared__ __attribute__((aligned(16))) uint32_t pb_lds[];  // [E][m]
  __shared__ int s_bad, s_dup;
  const int w = blockIdx.x, tid = threadIdx.x, nth = blockDim.x;
  const int R = 32 * m, lo = w * R, hi = min(n_rows, lo + R);
  for (int i = tid; i < E * m; i += nth) pb_lds[i] = 0u;
  if (tid == 0) {
    s_bad = 0;
    s_dup = 0;
  }
  __syncthreads();
  for (int i = tid; i < (hi - lo) * k; i += nth) {
    const int r = lo + i / k, kk = i - (i / k) * k;
    const int e = idx[static_cast<long long>(r) * (k + 1) + kk];
    if (e < 0 || e >= E) {
      for (int q = 0; q <= k; ++q) weight[static_cast<long long>(r) * (k + 1) + q] = 0.f;
      gslot[r * k + kk] = -1;
      atomicAdd(&s_bad, 1);
      continue;
    }
    const uint32_t bit = 1u << ((r - lo) & 31);
    if (atomicOr(&pb_lds[e * m + ((r - lo) >> 5)], bit) & bit) s_dup = 1;
  }
  __syncthreads();
  for (int i = tid; i < E * m; i += nth) wbits[static_cast<long long>(w) * E * m + i] = pb_lds[i];
  if (tid == 0) wflags[w] = s_bad | (s_dup << 16);
}

// Everything a workgroup reads is issued up front, so its latency is paid
// about once: the flags, each expert's bitmap column (up to kColWords words
// per thread in flight), its own bitmaps (into LDS), its own routes' ids and,
// in workgroup 0, the experts' matrix pointers.
constexpr int kColWords = 32;  // bitmap words of one expert's column per thread

__global__ void __launch_bounds__(kPlanThreads) plan_place_kernel(
    const int* __restrict__ idx, const uint32_t* __restrict__ wbits,
    const int* __restrict__ wflags, int* __restrict__ gslot, int* __restrict__ grows,
    int* __restrict__ off, int* __restrict__ toff, int* __restrict__ meta, int* __restrict__ tiles,
    TileRec* __restrict__ trec, int n_rec, const sg_block_q4k* const* tab_g,
    const sg_block_q4k* const* tab_u, const sg_block_q4k* const* tab_d, const sg_block_q4k* sh_g,
    const sg_block_q4k* sh_u, const sg_block_q4k* sh_d, int n_rows, int k, int E, int m,
    int n_w, int tok_per, int shared_tail) {
  extern __shared__ __attribute__((aligned(16))) uint32_t pp_lds[];  // own bitmaps [E][m]
  __shared__ int hist[1024], pre[1024], offl[1024], part[kPlanThreads];
  __shared__ int s_bad, s_dup, s_tmp[16];
  const int tid = threadIdx.x, nth = blockDim.x, w = blockIdx.x;
  const int R = 32 * m, lo = w * R, hi = min(n_rows, lo + R);
  const int nwords = n_w * m;  // words of one expert's column
  // thread group of expert pe: tpe threads, thread pq of it words
  // [pq * wpt, pq * wpt + wpt) of the column (kColWords at a time)
  const int tpe = max(1, nth / E), pe = tid / tpe, pq = tid - pe * tpe;
  const int wpt = (nwords + tpe - 1) / tpe;
  const int j0 = min(nwords, pq * wpt), j1 = min(nwords, j0 + wpt);
  // --- loads
  const int f = tid < n_w ? wflags[tid] : 0;  // n_w <= kPlanMaxWg <= nth
  const int ni = (hi - lo) * k;
  int my_e[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {  // own routes: (hi - lo) * k <= 32 m k, usually <= 2 per thread
    const int i = tid + q * nth;
    const int r = lo + i / k;
    my_e[q] = i < ni ? idx[static_cast<long long>(r) * (k + 1) + (i - (i / k) * k)] : -1;
  }
  for (int i = tid; i < E * m; i += nth) pp_lds[i] = wbits[static_cast<long long>(w) * E * m + i];
  const bool recs = w == 0 && trec;
  const sg_block_q4k* mgp[2] = {nullptr, nullptr};
  const sg_block_q4k* mup[2] = {nullptr, nullptr};
  const sg_block_q4k* mdp[2] = {nullptr, nullptr};
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int e = 2 * tid + q;
    if (recs && e < E) {
      mgp[q] = tab_g[e];
      mup[q] = tab_u[e];
      mdp[q] = tab_d[e];
    }
  }
  if (tid == 0) {
    s_bad = 0;
    s_dup = 0;
  }
  // experts eb + pe, nth / tpe of them per pass (E > nth: one each, several passes)
  for (int eb = 0; eb < E; eb += nth / tpe) {
    const int e = eb + pe;
    int h = 0, p = 0;
    if (e < E) {
      for (int c0 = j0; c0 < j1; c0 += kColWords) {
        // unconditional loads of clamped addresses (a load under a condition
        // is issued and waited for one at a time), masked afterwards
        uint32_t v[kColWords];
        int jw = c0 / m, jr = c0 - jw * m;  // word c0 of the column: workgroup jw, word jr
#pragma unroll
        for (int u = 0; u < kColWords; ++u) {
          v[u] = wbits[(static_cast<long long>(jw) * E + e) * m + jr];
          if (c0 + u + 1 < j1 && ++jr == m) {  // past the end: re-read the last word
            jr = 0;
            ++jw;
          }
        }
#pragma unroll
        for (int u = 0; u < kColWords; ++u) {
          const int c = (c0 + u) < j1 ? __popc(v[u]) : 0;
          h += c;
          p += (c0 + u) < w * m ? c : 0;
        }
      }
    }
    __syncthreads();  // part[] of the previous pass consumed; s_bad, s_dup set
    part[tid] = h;
    __syncthreads();
    if (pq == 0 && e < E) {
      int hh = 0;
      for (int j = 0; j < tpe; ++j) hh += part[tid + j];
      hist[e] = hh;
    }
    __syncthreads();
    part[tid] = p;
    __syncthreads();
    if (pq == 0 && e < E) {
      int pp = 0;
      for (int j = 0; j < tpe; ++j) pp += part[tid + j];
      pre[e] = pp;
    }
  }
  if (f & 0xFFFF) atomicAdd(&s_bad, f & 0xFFFF);
  if (f >> 16) s_dup = 1;
  __syncthreads();
  if (s_dup) {  // duplicated ids in a row: workgroup 0 does it all, serially
    if (w != 0) return;
    if (tid == 0) {  // the bitmaps undercount a duplicated id: count the routes
      for (int e = 0; e < E; ++e) hist[e] = 0;
      for (int i = 0; i < n_rows * k; ++i) {
        const int e = idx[static_cast<long long>(i / k) * (k + 1) + i % k];
        if (e >= 0 && e < E) ++hist[e];
      }
    }
    __syncthreads();
  }
  int tot_h = 0, tot_t = 0;
  {  // exclusive scans over the experts (E <= 1024: two per thread)
    const int e0 = 2 * tid, e1 = 2 * tid + 1;
    const int h0 = e0 < E ? hist[e0] : 0, h1 = e1 < E ? hist[e1] : 0;
    const int t0 = (h0 + tok_per - 1) / tok_per, t1 = (h1 + tok_per - 1) / tok_per;
    const int ph = plan_scan(h0 + h1, s_tmp, &tot_h);
    const int pt = plan_scan(t0 + t1, s_tmp, &tot_t);
    if (e0 < E) offl[e0] = ph;
    if (e1 < E) offl[e1] = ph + h0;
    if (w == 0) {
      if (e0 < E) {
        off[e0] = ph;
        toff[e0] = pt;
      }
      if (e1 < E) {
        off[e1] = ph + h0;
        toff[e1] = pt + t0;
      }
      auto put = [&](int t, int g, int p0, int p1, const sg_block_q4k* mg, const sg_block_q4k* mu,
                     const sg_block_q4k* md) {
        const bool present = mg && mu && md;
        trec[t] = TileRec{g, p0, p1, 0,
                          present ? reinterpret_cast<unsigned long long>(mg) : 0ull,
                          present ? reinterpret_cast<unsigned long long>(mu) : 0ull,
                          present ? reinterpret_cast<unsigned long long>(md) : 0ull, 0ull};
      };
#pragma unroll
      for (int q = 0; q < 2; ++q) {  // the tiles of experts e0 and e1
        const int e = q ? e1 : e0, hq = q ? h1 : h0, tl = q ? t1 : t0;
        const int pb = q ? ph + h0 : ph, tb = q ? pt + t0 : pt;
        if (e >= E) continue;
        if (tiles)
          for (int j = 0; j < tl; ++j) tiles[1 + tb + j] = (e << 16) | j;
        if (trec)
          for (int j = 0; j < tl; ++j)
            put(tb + j, e, pb + tok_per * j, min(pb + hq, pb + tok_per * (j + 1)), mgp[q], mup[q],
                mdp[q]);
      }
      const int sh_t = (shared_tail + tok_per - 1) / tok_per;
      if (tiles)
        for (int j = tid; j < sh_t; j += nth) tiles[1 + tot_t + j] = (E << 16) | j;
      if (trec) {
        for (int j = tid; j < sh_t; j += nth)
          put(tot_t + j, E, tot_h + tok_per * j,
              min(tot_h + shared_tail, tot_h + tok_per * (j + 1)), sh_g, sh_u, sh_d);
        for (int t = tot_t + sh_t + tid; t < n_rec; t += nth)
          trec[t] = TileRec{-1, 0, 0, 0, 0ull, 0ull, 0ull, 0ull};
      }
      if (tid == 0) {
        off[E] = tot_h;
        toff[E] = tot_t;
        off[E + 1] = tot_h + shared_tail;
        meta[0] = tot_h;
        meta[1] = tot_t;
        meta[2] = s_bad;
        if (tiles) tiles[0] = tot_t + sh_t;
      }
    }
  }
  __syncthreads();
  if (s_dup) {  // workgroup 0 only: serial placement, then the shared tail
    if (tid == 0) {
      for (int e = 0; e < E; ++e) hist[e] = offl[e];
      for (int i = 0; i < n_rows * k; ++i) {
        const int r = i / k, kk = i - r * k;
        const int e = idx[static_cast<long long>(r) * (k + 1) + kk];
        if (e < 0 || e >= E) continue;
        const int pos = hist[e]++;
        gslot[i] = pos;
        grows[pos] = r;
      }
    }
    for (int t = tid; t < shared_tail; t += nth) grows[tot_h + t] = t;
    return;
  }
  // the shared expert's positions of this workgroup's tokens: t at off[E] + t
  for (int t = lo + tid; t < min(hi, shared_tail); t += nth) grows[tot_h + t] = t;
  // this workgroup's routes (their ids were loaded at the start)
  auto place = [&](int i, int e) {
    const int r = lo + i / k, kk = i - (i / k) * k;
    if (e < 0 || e >= E) return;
    const int d = r - lo, wi = d >> 5;
    const uint32_t* be = pp_lds + e * m;
    int c = offl[e] + pre[e] + __popc(be[wi] & ((1u << (d & 31)) - 1u));
    for (int j = 0; j < wi; ++j) c += __popc(be[j]);
    gslot[r * k + kk] = c;
    grows[c] = r;
  };
#pragma unroll
  for (int q = 0; q < 2; ++q)
    if (tid + q * nth < ni) place(tid + q * nth, my_e[q]);
  for (int i = tid + 2 * nth; i < ni; i += nth)
    place(i, idx[static_cast<long long>(lo + i / k) * (k + 1) + (i - (i / k) * k)]);
}

// Q8P blocks (the grouped kernels' input, see kQ8PBytes): one block per
// 16-lane row (four per wave, 16 per workgroup); the lane's 16 values are
// four 16-B loads and the block's max and sums reduce inside a DPP row.
// The codes and d are quantize_row_q8_K's (q4_k.cpp:44-61), as in
// quantize_block_wave; only the layout differs.
// quantize_rows16 quantizes block `blk` in the lane's 16-lane row (blocks at
// or past n_blocks store nothing) from the lane's 16 values v.
__device__ __forceinline__ void quantize_rows16(const float (&v)[16], unsigned char* __restrict__ out,
                                                long long n_blocks, long long blk, int lane) {
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = fmaxf(amax, dpp_f<kDppXor1>(amax));
  amax = fmaxf(amax, dpp_f<kDppXor2>(amax));
  amax = fmaxf(amax, dpp_f<kDppHalfMirror>(amax));
  amax = fmaxf(amax, dpp_f<kDppMirror>(amax));
  amax = fmaxf(amax, 1e-30f);
  const float d = amax / 127.f;
  const float id = d > 0 ? 1.f / d : 0.f;
  uint32_t packed[4];
  int qsum = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    packed[w] = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = q8_code(v[4 * w + i] * id);
      qsum += q;
      packed[w] |= (static_cast<uint32_t>(q) & 0xFFu) << (8 * i);
    }
  }
  qsum += dpp_i<kDppXor1>(qsum);  // a sub-block sum's 32 values: this lane and its neighbour
  if (blk >= n_blocks) return;
  unsigned char* ob = out + blk * kQ8PBytes;
  const int r = lane & 15;
  *reinterpret_cast<u32x4*>(ob + 16 + 16 * r) = (u32x4){packed[0], packed[1], packed[2], packed[3]};
  if (r == 0) *reinterpret_cast<u32x4*>(ob) = (u32x4){__builtin_bit_cast(uint32_t, d), 0u, 0u, 0u};
  if ((r & 1) == 0) {  // sum = 2 a + b as fp16 integers (|a| <= 2032: exact)
    *reinterpret_cast<_Float16*>(ob + 272 + r) = static_cast<_Float16>(static_cast<float>(qsum >> 1));
    *reinterpret_cast<_Float16*>(ob + 288 + r) = static_cast<_Float16>(static_cast<float>(qsum & 1));
  }
}

// the lane's 16 values of block bc (fp32)
__device__ __forceinline__ void load16(const float* __restrict__ in, long long bc, int lane,
                                       float (&v)[16]) {
  const float* src = in + bc * kQK + 16 * (lane & 15);
#pragma unroll
  for (int i = 0; i < 16; i += 4) {
    const float4 f = *reinterpret_cast<const float4*>(src + i);
    v[i] = f.x;
    v[i + 1] = f.y;
    v[i + 2] = f.z;
    v[i + 3] = f.w;
  }
}

// the prefill's x: fp32, the session's fp16 xn, or a Q8_K of it the caller
// made (moe_xq_in_, session.cpp:1022, 1131), used as is
struct XSrc {
  const float* f32;
  const uint16_t* f16;
  const unsigned char* q8;
};

// Q8P block blk of x in the lane's 16-lane row: quantized from fp32 or
// fp16 values, or the caller's Q8_K block rearranged (its codes, d and
// sub-block sums unchanged)
__device__ __forceinline__ void x_block_q8p(const XSrc& x, unsigned char* __restrict__ out,
                                            long long n_blocks, long long blk, int lane) {
  const long long bc = blk < n_blocks ? blk : n_blocks - 1;  // rows past the end compute, never store
  if (x.q8) {
    if (blk >= n_blocks) return;
    const int r = lane & 15;
    const uint32_t* q = reinterpret_cast<const uint32_t*>(x.q8 + bc * kQ8Bytes);
    unsigned char* ob = out + blk * kQ8PBytes;
    *reinterpret_cast<u32x4*>(ob + 16 + 16 * r) =
        (u32x4){q[1 + 4 * r], q[2 + 4 * r], q[3 + 4 * r], q[4 + 4 * r]};
    if (r == 0) *reinterpret_cast<u32x4*>(ob) = (u32x4){q[0], 0u, 0u, 0u};
    if ((r & 1) == 0) {
      const int sum = static_cast<int16_t>(q[65 + (r >> 2)] >> (16 * ((r >> 1) & 1)));
      *reinterpret_cast<_Float16*>(ob + 272 + r) = static_cast<_Float16>(static_cast<float>(sum >> 1));
      *reinterpret_cast<_Float16*>(ob + 288 + r) = static_cast<_Float16>(static_cast<float>(sum & 1));
    }
    return;
  }
  float v[16];
  if (x.f16) {
    const uint16_t* src = x.f16 + bc * kQK + 16 * (lane & 15);
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = f16v(src[i]);
  } else {
    load16(x.f32, bc, lane, v);
  }
  quantize_rows16(v, out, n_blocks, blk, lane);
}
// rows_used (optional, device): only the first *rows_used rows hold data
// (the positions the plan filled); whole 16-lane rows past them exit before
// any lane exchange.
// in16 (instead of in): fp16 values (h of the fp16-buffer path).
__global__ void __launch_bounds__(256) prefill_quantize_kernel(const float* __restrict__ in,
                                                               const uint16_t* __restrict__ in16,
                                                               unsigned char* __restrict__ out,
                                                               long long n_blocks,
                                                               const int* __restrict__ rows_used,
                                                               int nb_row) {
  const int lane = threadIdx.x & 63;
  const long long blk =
      (static_cast<long long>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * 4 + (lane >> 4);
  if (rows_used && blk >= static_cast<long long>(*rows_used) * nb_row) return;
  const long long bc = blk < n_blocks ? blk : n_blocks - 1;
  float v[16];
  if (in16) {
    const uint4* src = reinterpret_cast<const uint4*>(in16 + bc * kQK + 16 * (lane & 15));
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint4 w = src[q];
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[8 * q + 2 * i] = f16v(ww[i] & 0xFFFFu);
        v[8 * q + 2 * i + 1] = f16v(ww[i] >> 16);
      }
    }
  } else {
    load16(in, bc, lane, v);
  }
  quantize_rows16(v, out, n_blocks, blk, lane);
}

// Q8P of x (caller routing, or routers wider than route_quantize_kernel's)
__global__ void __launch_bounds__(256) prefill_x_kernel(XSrc x, unsigned char* __restrict__ out,
                                                        long long n_blocks) {
  const int lane = threadIdx.x & 63;
  const long long blk =
      (static_cast<long long>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * 4 + (lane >> 4);
  x_block_q8p(x, out, n_blocks, blk, lane);
}

// The prefill's first launch: four-wave workgroups.  The first
// ceil(n_rows / 4) route one token per wave (router_wave, the standalone
// router's routine); the following ones quantize four blocks of x per wave,
// so the router's chains and the quantization share one launch.
constexpr int kRqWaves = 4;
template <int PL>
__global__ void __launch_bounds__(64 * kRqWaves) route_quantize_kernel(
    const float* __restrict__ logits, int* __restrict__ idx, float* __restrict__ weight,
    int n_rows, int n_expert, int k, float shared_w, XSrc x, unsigned char* __restrict__ xq,
    long long n_blocks) {
  __shared__ __attribute__((aligned(16))) float ev[kRqWaves][64 * PL];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_rwg = (n_rows + kRqWaves - 1) / kRqWaves;  // routing workgroups
  if (static_cast<int>(blockIdx.x) < n_rwg) {
    const long long w = static_cast<long long>(blockIdx.x) * kRqWaves + wave;
    if (w < n_rows)
      router_wave<PL>(logits + w * n_expert, n_expert, k, shared_w, idx + w * (k + 1),
                      weight + w * (k + 1), ev[wave], lane);
    return;
  }
  const long long qw = (static_cast<long long>(blockIdx.x) - n_rwg) * kRqWaves + wave;
  x_block_q8p(x, xq, n_blocks, qw * 4 + (lane >> 4), lane);
}

// out[t] = residual[t] + sum_kk fma(w[t][kk], y[pos(t, kk)]) in slot order;
// pos(t, k) = the shared expert's position off[E] + t when present.  A thread
// owns four consecutive columns; the positions and weights of eight slots are
// read first (uniform per workgroup), then their eight 16-B rows are loaded
// together before the ordered fma chain, so each thread has eight loads in
// flight instead of one.
// With out16 (the session's fp16 buffers) the slot outputs are taken as
// stored in fp16, the shared one gated on its fp16 value and stored again,
// the accumulation starts from the fp16 res16 and the sum is stored as fp16
// (sigmoid_gate_scalar_batched_f16, moe_combine_batched_f16: moe.cu:265-292);
// the down pass then stores y in fp16 already (y16), half the bytes to read.
__global__ void __launch_bounds__(256) prefill_combine_kernel(
    float* __restrict__ out, const float* __restrict__ residual, uint16_t* __restrict__ out16,
    const uint16_t* __restrict__ res16, const float* __restrict__ y,
    const uint16_t* __restrict__ y16,
    const float* __restrict__ weight, const int* __restrict__ gslot, const int* __restrict__ off,
    const float* __restrict__ sgate, int n_expert, int k, int hidden, int has_shared) {
  // 1-D grid, token-major: ceil(hidden / 1024) workgroups per token, so the
  // token count has no grid-dimension limit
  const int nbx = (hidden + 1023) / 1024;
  const int t = blockIdx.x / nbx;
  const int i = ((blockIdx.x - t * nbx) * 256 + threadIdx.x) * 4;
  if (i >= hidden) return;
  const long long o = static_cast<long long>(t) * hidden + i;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (residual) {
    acc = *reinterpret_cast<const float4*>(residual + o);
  } else if (res16) {
    const uint2 r4 = *reinterpret_cast<const uint2*>(res16 + o);
    acc = make_float4(f16v(r4.x & 0xFFFFu), f16v(r4.x >> 16), f16v(r4.y & 0xFFFFu), f16v(r4.y >> 16));
  }
  const int shared_pos = off[n_expert] + t;
  // the shared slot's output scaled by its gate first (1.0 without a gate
  // leaves it unchanged), as sigmoid_gate_scalar_batched_f16 does before
  // the combine (session.cpp:2904-2909)
  const float gs = sgate ? sgate[t] : 1.f;
  for (int k0 = 0; k0 <= k; k0 += 8) {
    int pos[8];
    float wv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int kk = k0 + u;
      pos[u] = kk < k ? gslot[t * k + kk] : (kk == k && has_shared ? shared_pos : -1);
      wv[u] = kk <= k ? weight[t * (k + 1) + kk] : 0.f;
    }
    float4 yv[8];
    if (y16) {
      uint2 yh[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        yh[u] = pos[u] >= 0
                    ? *reinterpret_cast<const uint2*>(y16 + static_cast<long long>(pos[u]) * hidden + i)
                    : make_uint2(0u, 0u);
#pragma unroll
      for (int u = 0; u < 8; ++u)
        yv[u] = make_float4(f16v(yh[u].x & 0xFFFFu), f16v(yh[u].x >> 16), f16v(yh[u].y & 0xFFFFu),
                            f16v(yh[u].y >> 16));
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u)
        yv[u] = pos[u] >= 0
                    ? *reinterpret_cast<const float4*>(y + static_cast<long long>(pos[u]) * hidden + i)
                    : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (out16) {
      auto r16 = [](float v) { return f16v(f16b(v)); };
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        yv[u] = make_float4(r16(yv[u].x), r16(yv[u].y), r16(yv[u].z), r16(yv[u].w));
        if (k0 + u == k)
          yv[u] = make_float4(r16(yv[u].x * gs), r16(yv[u].y * gs), r16(yv[u].z * gs),
                              r16(yv[u].w * gs));
      }
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (k0 + u == k) {
          yv[u].x *= gs;
          yv[u].y *= gs;
          yv[u].z *= gs;
          yv[u].w *= gs;
        }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (k0 + u <= k) {
        acc.x = __builtin_fmaf(wv[u], yv[u].x, acc.x);
        acc.y = __builtin_fmaf(wv[u], yv[u].y, acc.y);
        acc.z = __builtin_fmaf(wv[u], yv[u].z, acc.z);
        acc.w = __builtin_fmaf(wv[u], yv[u].w, acc.w);
      }
    }
  }
  if (out16) {
    *reinterpret_cast<uint2*>(out16 + o) =
        make_uint2(f16b(acc.x) | (static_cast<uint32_t>(f16b(acc.y)) << 16),
                   f16b(acc.z) | (static_cast<uint32_t>(f16b(acc.w)) << 16));
  } else {
    *reinterpret_cast<float4*>(out + o) = acc;
  }
}

// The combine on the fp16 buffers with fp16 slot outputs (the session's
// path): the arithmetic of prefill_combine_kernel's out16 branch, eight
// columns per thread so every slot row is read with 16-B loads, one
// workgroup of 256 threads per 2048 columns of a token.
__global__ void __launch_bounds__(256) prefill_combine16_kernel(
    uint16_t* __restrict__ out16, const uint16_t* __restrict__ res16,
    const uint16_t* __restrict__ y16, const float* __restrict__ weight,
    const int* __restrict__ gslot, const int* __restrict__ off, const float* __restrict__ sgate,
    int n_expert, int k, int hidden, int has_shared) {
  const int nbx = (hidden + 2047) / 2048;
  const int t = blockIdx.x / nbx;
  const int i = ((blockIdx.x - t * nbx) * 256 + threadIdx.x) * 8;
  if (i >= hidden) return;
  const long long o = static_cast<long long>(t) * hidden + i;
  auto unpack = [](const uint4 v, float (&f)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f[2 * j] = f16v(w[j] & 0xFFFFu);
      f[2 * j + 1] = f16v(w[j] >> 16);
    }
  };
  float acc[8];
  if (res16) {
    unpack(*reinterpret_cast<const uint4*>(res16 + o), acc);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.f;
  }
  const int shared_pos = off[n_expert] + t;
  const float gs = sgate ? sgate[t] : 1.f;
  for (int k0 = 0; k0 <= k; k0 += 8) {
    int pos[8];
    float wv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int kk = k0 + u;
      pos[u] = kk < k ? gslot[t * k + kk] : (kk == k && has_shared ? shared_pos : -1);
      wv[u] = kk <= k ? weight[t * (k + 1) + kk] : 0.f;
    }
    uint4 yh[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      yh[u] = pos[u] >= 0
                  ? *reinterpret_cast<const uint4*>(y16 + static_cast<long long>(pos[u]) * hidden + i)
                  : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (k0 + u > k) continue;
      float yv[8];
      unpack(yh[u], yv);
      if (k0 + u == k) {  // the shared slot, gated on its fp16 value and rounded again
#pragma unroll
        for (int j = 0; j < 8; ++j) yv[j] = f16v(f16b(yv[j] * gs));
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = __builtin_fmaf(wv[u], yv[j], acc[j]);
    }
  }
  uint4 r;
  r.x = f16b(acc[0]) | (static_cast<uint32_t>(f16b(acc[1])) << 16);
  r.y = f16b(acc[2]) | (static_cast<uint32_t>(f16b(acc[3])) << 16);
  r.z = f16b(acc[4]) | (static_cast<uint32_t>(f16b(acc[5])) << 16);
  r.w = f16b(acc[6]) | (static_cast<uint32_t>(f16b(acc[7])) << 16);
  *reinterpret_cast<uint4*>(out16 + o) = r;
}

// sgate[t] = sigmoid(w . x[t]): the shared expert's scalar gate
// (session.cpp:2904-2909, gemv_f32_out_f16x_batched then
// sigmoid_gate_scalar_batched_f16), one token per 32-lane half-wave in the
// reference's fp32 lane order.
__global__ void __launch_bounds__(256) shared_gate_kernel(const float* __restrict__ w, XSrc x,
                                                          float* __restrict__ sgate, int n_tokens,
                                                          int hidden) {
  const int l = threadIdx.x & 31;
  const int t0 = blockIdx.x * 8 + (threadIdx.x >> 5);
  const int t = t0 < n_tokens ? t0 : n_tokens - 1;  // whole halves stay active for the shuffles
  const long long o = static_cast<long long>(t) * hidden;
  const float g = x.f16 ? rowdot_f32_lanes32(w, [&](int i) { return f16v(x.f16[o + i]); }, hidden, l)
                        : rowdot_f32_lanes32(w, [&](int i) { return x.f32[o + i]; }, hidden, l);
  if (l == 0 && t0 < n_tokens) sgate[t0] = sigmoid_sg(g);
}

// ---- workspace ------------------------------------------------------------------
static size_t al256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

// the plan's workgroups (R = 32 m tokens each) and its scratch: wbits
// [n_w][E][m], wflags [n_w]
struct PlanWs {
  int m, n_w;
  size_t wbits, wflags, total, lds_bits;
};
static PlanWs plan_ws(int n_rows, int E) {
  PlanWs p{};
  p.m = (n_rows + 32 * kPlanMaxWg - 1) / (32 * kPlanMaxWg);
  p.n_w = (n_rows + 32 * p.m - 1) / (32 * p.m);
  size_t o = 0;
  p.wbits = o;  o = al256(o + static_cast<size_t>(p.n_w) * E * p.m * 4);
  p.wflags = o; o = al256(o + static_cast<size_t>(p.n_w) * 4);
  p.total = o;
  p.lds_bits = static_cast<size_t>(E) * p.m * 4;
  return p;
}

struct PrefillWs {
  size_t xq, gslot, grows, off, toff, meta, tiles, trec, plan, sgate, h, hq, y, total;
  int P;          // positions: T*k routes + T shared
  int max_tiles;  // bound on the work list: every group's last tile may be partial
};

static PrefillWs prefill_ws(int T, int hidden, int n_ff, int E, int k) {
  PrefillWs w{};
  w.P = T * k + T;
  size_t o = 0;
  w.xq = o;    o = al256(o + static_cast<size_t>(T) * (hidden / kQK) * kQ8PBytes);
  w.gslot = o; o = al256(o + static_cast<size_t>(T) * k * 4);
  w.grows = o; o = al256(o + static_cast<size_t>(w.P) * 4);
  w.off = o;   o = al256(o + static_cast<size_t>(E + 2) * 4);
  w.toff = o;  o = al256(o + static_cast<size_t>(E + 2) * 4);
  w.meta = o;  o = al256(o + 4 * 4);
  w.max_tiles = (T * k + kTokTile - 1) / kTokTile + E + (T + kTokTile - 1) / kTokTile;
  w.tiles = o; o = al256(o + static_cast<size_t>(1 + w.max_tiles) * 4);
  w.trec = o;  o = al256(o + static_cast<size_t>(w.max_tiles) * sizeof(TileRec));
  w.plan = o;  o = al256(o + plan_ws(T, E).total);
  w.sgate = o; o = al256(o + static_cast<size_t>(T) * 4);
  w.h = o;     o = al256(o + static_cast<size_t>(w.P) * n_ff * 4);
  w.hq = o;    o = al256(o + static_cast<size_t>(w.P) * (n_ff / kQK) * kQ8PBytes);
  w.y = o;     o = al256(o + static_cast<size_t>(w.P) * hidden * 4);
  w.total = o;
  return w;
}

// the grouped kernels' Q8P input
static int quantize_split(const float* in, const uint16_t* in16, unsigned char* out, int nb_row,
                          int n_rows, hipStream_t s, const char* nm,
                          const int* rows_used = nullptr) {
  const long long n_blocks = static_cast<long long>(nb_row) * n_rows;
  const unsigned grid = static_cast<unsigned>((n_blocks + 15) / 16);
  hipLaunchKernelGGL(prefill_quantize_kernel, dim3(grid), dim3(256), 0, s, in, in16, out,
                     n_blocks, rows_used, nb_row);
  return check_launch(nm);
}

constexpr int kScanLdsWords = 38 * 1024;  // dispatch scan: hist, offsets, parts, bitmap

static int scan_lds_words(int n_rows, int E) {
  return 2 * E + 1024 + 2 * E * (((n_rows + 31) / 32) | 1);
}

static int scan_launch(const int* idx, float* weight, int* gslot, int* grows, int* off, int* toff,
                       int* meta, int* tiles, int n_rows, int k, int E, int tok_per,
                       int shared_tail, hipStream_t s, const char* nm) {
  const int words = scan_lds_words(n_rows, E);
  if (words > kScanLdsWords)
    return set_error(SG_ERR_UNSUPPORTED, "%s: n_rows=%d x n_expert=%d too large for one scan",
                     nm, n_rows, E);
  hipLaunchKernelGGL(dispatch_scan_kernel, dim3(1), dim3(1024), words * 4, s, idx, weight, gslot,
                     grows, off, toff, meta, tiles, n_rows, k, E, tok_per, shared_tail);
  return check_launch(nm);
}

// the plan over many workgroups (bitmaps, then offsets and placement) on
// scratch `ws`
struct PlanTables {  // the matrices the tile records carry (all null: no records)
  const sg_block_q4k* const* g;
  const sg_block_q4k* const* u;
  const sg_block_q4k* const* d;
  const sg_block_q4k *sg, *su, *sd;
};

static int plan_launch(const int* idx, float* weight, int* gslot, int* grows, int* off,
                       int* toff, int* meta, int* tiles, TileRec* trec, int n_rec,
                       const PlanTables& pt, unsigned char* ws, int n_rows, int k, int E,
                       int tok_per, int shared_tail, hipStream_t s, const char* nm) {
  const PlanWs p = plan_ws(n_rows, E);
  if (p.lds_bits > 128 * 1024)
    return set_error(SG_ERR_UNSUPPORTED, "%s: n_rows=%d x n_expert=%d: plan too large", nm,
                     n_rows, E);
  uint32_t* wbits = reinterpret_cast<uint32_t*>(ws + p.wbits);
  int* wflags = reinterpret_cast<int*>(ws + p.wflags);
  hipLaunchKernelGGL(plan_bits_kernel, dim3(p.n_w), dim3(kPlanThreads), p.lds_bits, s, idx,
                     weight, gslot, wbits, wflags, n_rows, k, E, p.m);
  if (int st = check_launch(nm)) return st;
  hipLaunchKernelGGL(plan_place_kernel, dim3(p.n_w), dim3(kPlanThreads), p.lds_bits, s, idx, wbits, wflags,
                     gslot, grows, off, toff, meta, tiles, trec, n_rec, pt.g, pt.u, pt.d, pt.sg,
                     pt.su, pt.sd, n_rows, k, E, p.m, p.n_w, tok_per, shared_tail);
  return check_launch(nm);
}

// limits of the plan: E <= 1024, k <= 32, int route and tile indices
static int plan_check(int n_rows, int k, int E, int tok_per, const char* nm) {
  if (n_rows <= 0 || k <= 0 || k > 32 || E <= 0 || E > 1024 || tok_per <= 0)
    return set_error(SG_ERR_GEOMETRY, "%s: n_rows=%d k=%d (<=32) n_expert=%d (<=1024) tok_per=%d",
                     nm, n_rows, k, E, tok_per);
  if (static_cast<long long>(n_rows) * (k + 1) > 0x7fffffffLL)
    return set_error(SG_ERR_UNSUPPORTED, "%s: n_rows=%d x k=%d routes too many", nm, n_rows, k);
  return SG_OK;
}

}  // namespace sg

using namespace sg;

extern "C" {

int sg_moe_dispatch_scan(const int* idx, float* weight, int* gslot, int* grows, int* off,
                         int* toff, int* meta, int n_rows, int k, int n_expert, int tok_per,
                         void* stream) {
  const char* nm = "sg_moe_dispatch_scan";
  if (!idx || !weight || !gslot || !grows || !off || !toff || !meta)
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  if (n_rows <= 0 || k <= 0 || n_expert <= 0 || n_expert > 1024 || tok_per <= 0)
    return set_error(SG_ERR_GEOMETRY, "%s: n_rows=%d k=%d n_expert=%d (<=1024) tok_per=%d", nm,
                     n_rows, k, n_expert, tok_per);
  if (n_rows * k > 1024 * kScanPerThread)
    return set_error(SG_ERR_UNSUPPORTED, "%s: n_rows*k=%d > %d", nm, n_rows * k,
                     1024 * kScanPerThread);
  return scan_launch(idx, weight, gslot, grows, off, toff, meta, nullptr, n_rows, k, n_expert,
                     tok_per, 0,
                     static_cast<hipStream_t>(stream), nm);
}

size_t sg_moe_dispatch_plan_workspace_bytes(int n_rows, int n_expert) {
  if (n_rows <= 0 || n_expert <= 0) return 0;
  return plan_ws(n_rows, n_expert).total;
}

int sg_moe_dispatch_plan(const int* idx, float* weight, int* gslot, int* grows, int* off,
                         int* toff, int* meta, int* tiles, void* workspace,
                         size_t workspace_bytes, int n_rows, int k, int n_expert, int tok_per,
                         int shared_tail, void* stream) {
  const char* nm = "sg_moe_dispatch_plan";
  if (!idx || !weight || !gslot || !grows || !off || !toff || !meta || !workspace)
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  if (int st = plan_check(n_rows, k, n_expert, tok_per, nm)) return st;
  if (shared_tail < 0 || shared_tail > n_rows)
    return set_error(SG_ERR_GEOMETRY, "%s: shared_tail=%d not in [0, n_rows]", nm, shared_tail);
  if (workspace_bytes < plan_ws(n_rows, n_expert).total)
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: workspace %zu < %zu bytes", nm,
                     workspace_bytes, plan_ws(n_rows, n_expert).total);
  return plan_launch(idx, weight, gslot, grows, off, toff, meta, tiles, nullptr, 0, PlanTables{},
                     static_cast<unsigned char*>(workspace), n_rows, k, n_expert, tok_per,
                     shared_tail, static_cast<hipStream_t>(stream), nm);
}

size_t sg_moe_prefill_workspace_bytes(int n_tokens, int hidden, int n_ff, int n_expert, int k) {
  if (n_tokens <= 0 || hidden <= 0 || n_ff <= 0 || n_expert <= 0 || k <= 0) return 0;
  return prefill_ws(n_tokens, hidden, n_ff, n_expert, k).total;
}

}  // extern "C"

namespace sg {

// the chunk's output: fp32 (residual, out) or the session's fp16 buffers
struct PrefillOut {
  const float* residual;
  float* out;
  const uint16_t* res16;
  uint16_t* out16;
};

static int prefill_launch(const sg_block_q4k* const* tab_gate, const sg_block_q4k* const* tab_up,
                          const sg_block_q4k* const* tab_down, const sg_block_q4k* sh_gate,
                          const sg_block_q4k* sh_up, const sg_block_q4k* sh_down,
                          const float* sh_gate_w, const XSrc& x, const float* logits,
                          const PrefillOut& po, int* idx, float* weight, void* workspace,
                          size_t workspace_bytes, int n_tokens, int hidden, int n_ff, int n_expert,
                          int k, float shared_w, void* stream, const char* nm) {
  if (!tab_gate || !tab_up || !tab_down || !idx || !weight || !workspace)
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  const int n_sh = (sh_gate != nullptr) + (sh_up != nullptr) + (sh_down != nullptr);
  if (n_sh != 0 && n_sh != 3)
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: shared expert needs gate, up and down", nm);
  if (n_tokens <= 0 || hidden <= 0 || hidden % kQK || n_ff <= 0 || n_ff % kQK)
    return set_error(SG_ERR_GEOMETRY, "%s: n_tokens=%d hidden=%d n_ff=%d (multiples of 256)", nm,
                     n_tokens, hidden, n_ff);
  if (k <= 0 || k > 32 || n_expert < k || n_expert > 1024)
    return set_error(SG_ERR_GEOMETRY, "%s: k=%d n_expert=%d", nm, k, n_expert);
  const PrefillWs ws = prefill_ws(n_tokens, hidden, n_ff, n_expert, k);
  if (workspace_bytes < ws.total)
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: workspace %zu < %zu bytes", nm,
                     workspace_bytes, ws.total);
  if (int st = plan_check(n_tokens, k, n_expert, kTokTile, nm)) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  unsigned char* base = static_cast<unsigned char*>(workspace);
  unsigned char* xq = base + ws.xq;
  int* gslot = reinterpret_cast<int*>(base + ws.gslot);
  int* grows = reinterpret_cast<int*>(base + ws.grows);
  int* off = reinterpret_cast<int*>(base + ws.off);
  int* toff = reinterpret_cast<int*>(base + ws.toff);
  int* meta = reinterpret_cast<int*>(base + ws.meta);
  int* tiles = reinterpret_cast<int*>(base + ws.tiles);
  TileRec* trec = reinterpret_cast<TileRec*>(base + ws.trec);
  float* h = reinterpret_cast<float*>(base + ws.h);
  unsigned char* hq = base + ws.hq;
  float* y = reinterpret_cast<float*>(base + ws.y);
  // fp16 session buffers: y in fp16 (the combine rounds it to fp16 on use anyway)
  uint16_t* y16 = po.out16 ? reinterpret_cast<uint16_t*>(base + ws.y) : nullptr;
  const int has_shared = n_sh == 3;
  // the gate scales the shared expert only: without one it has nothing to scale
  float* sgate = has_shared && sh_gate_w ? reinterpret_cast<float*>(base + ws.sgate) : nullptr;

  if (logits && n_expert <= 512) {  // routing and Q8_K of x in one launch
    const long long nxb = static_cast<long long>(hidden / kQK) * n_tokens;
    const long long qwaves = (nxb + 3) / 4;  // four blocks per wave
    const unsigned grid = static_cast<unsigned>((n_tokens + kRqWaves - 1) / kRqWaves +
                                                (qwaves + kRqWaves - 1) / kRqWaves);
    auto launch = [&](auto kern) {
      hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * kRqWaves), 0, s, logits, idx, weight, n_tokens,
                         n_expert, k, shared_w, x, xq, nxb);
    };
    if (n_expert <= 64) launch(route_quantize_kernel<1>);
    else if (n_expert <= 128) launch(route_quantize_kernel<2>);
    else if (n_expert <= 256) launch(route_quantize_kernel<4>);
    else launch(route_quantize_kernel<8>);
    if (int st = check_launch("sg_moe_prefill/route_quantize")) return st;
  } else {
    const long long nxb = static_cast<long long>(hidden / kQK) * n_tokens;
    hipLaunchKernelGGL(prefill_x_kernel, dim3(static_cast<unsigned>((nxb + 15) / 16)), dim3(256),
                       0, s, x, xq, nxb);
    if (int st = check_launch(nm)) return st;
    if (logits)
      if (int st = sg_router_topk(logits, idx, weight, n_expert, k, k + 1, n_tokens, shared_w,
                                  stream))
        return st;
  }
  if (sgate) {
    hipLaunchKernelGGL(shared_gate_kernel, dim3((n_tokens + 7) / 8), dim3(256), 0, s, sh_gate_w, x,
                       sgate, n_tokens, hidden);
    if (int st = check_launch("sg_moe_prefill/shared_gate")) return st;
  }
  if (int st = plan_launch(idx, weight, gslot, grows, off, toff, meta, tiles, trec, ws.max_tiles,
                           PlanTables{tab_gate, tab_up, tab_down, sh_gate, sh_up, sh_down},
                           base + ws.plan, n_tokens, k, n_expert, kTokTile,
                           has_shared ? n_tokens : 0, s,
                           "sg_moe_prefill/plan"))
    return st;
  const int G = n_expert + has_shared;
  GroupedArgs ga{};
  ga.xq = xq;
  ga.off = off;
  ga.grows = grows;
  ga.trec = trec;
  ga.n_rec = ws.max_tiles;
  ga.out = h;
  ga.nb = hidden / kQK;
  ga.n_rows = n_ff;
  ga.n_out = n_ff;
  ga.n_groups = G;
  // 1-D grids: a multiple of 8 tiles (one per XCD) times the slices
  const int tiles8 = (ws.max_tiles + 7) / 8 * 8;
  ga.n_slices = n_ff / (kRowsWg / 2);
  ga.spw = 1;
  ga.r16 = po.out16 != nullptr;
  // fp16 h on the fp16 buffers (its values are fp16 there): half the bytes
  uint16_t* h16 = ga.r16 ? reinterpret_cast<uint16_t*>(h) : nullptr;
  ga.out16 = h16;
  hipLaunchKernelGGL(grouped_mfma_kernel<true>, dim3(tiles8 * ga.n_slices), dim3(kThreads),
                     kGroupedLds, s, ga);
  if (int st = check_launch("sg_moe_prefill/gate_up")) return st;
  // h rows of the filled positions only: off[E + 1] = routes + shared rows
  if (int st = quantize_split(h16 ? nullptr : h, h16, hq, n_ff / kQK, ws.P, s, nm,
                              off + n_expert + 1))
    return st;
  GroupedArgs gd = ga;
  gd.xq = hq;
  gd.grows = nullptr;
  gd.out = y;
  gd.out16 = y16;
  gd.nb = n_ff / kQK;
  gd.n_rows = hidden;
  gd.n_out = hidden;
  gd.n_slices = hidden / kRowsWg;
  // with at most two super-blocks per row the tile's token rows fit both
  // token buffers, so one workgroup runs several column slices on them
  gd.spw = 1;
  if (gd.nb <= 2)
    while (gd.spw < kDownSlicesPerWg && gd.n_slices % (2 * gd.spw) == 0) gd.spw *= 2;
  auto down = [&](auto kern, int n_wg) {
    hipLaunchKernelGGL(kern, dim3(tiles8 * n_wg), dim3(kThreads), kGroupedLds, s, gd);
  };
  if (gd.spw > 1) {
    if (y16) down(grouped_mfma_kernel<false, true, true>, gd.n_slices / gd.spw);
    else down(grouped_mfma_kernel<false, true>, gd.n_slices / gd.spw);
  } else {
    if (y16) down(grouped_mfma_kernel<false, false, true>, gd.n_slices);
    else down(grouped_mfma_kernel<false, false>, gd.n_slices);
  }
  if (int st = check_launch("sg_moe_prefill/down")) return st;
  // (16-B loads of the caller's fp16 buffers need them 16-B aligned)
  const bool al16 = (reinterpret_cast<uintptr_t>(po.out16) | reinterpret_cast<uintptr_t>(po.res16)) % 16 == 0;
  if (y16 && al16) {
    hipLaunchKernelGGL(prefill_combine16_kernel, dim3((hidden + 2047) / 2048 * n_tokens), dim3(256),
                       0, s, po.out16, po.res16, y16, weight, gslot, off, sgate, n_expert, k,
                       hidden, has_shared);
    return check_launch("sg_moe_prefill/combine");
  }
  hipLaunchKernelGGL(prefill_combine_kernel, dim3((hidden + 1023) / 1024 * n_tokens), dim3(256), 0, s,
                     po.out, po.residual, po.out16, po.res16, y, y16, weight, gslot, off, sgate,
                     n_expert, k, hidden, has_shared);
  return check_launch("sg_moe_prefill/combine");
}

}  // namespace sg

extern "C" {

int sg_moe_prefill(const sg_block_q4k* const* tab_gate, const sg_block_q4k* const* tab_up,
                   const sg_block_q4k* const* tab_down, const sg_block_q4k* sh_gate,
                   const sg_block_q4k* sh_up, const sg_block_q4k* sh_down,
                   const float* sh_gate_w, const float* x, const float* logits,
                   const float* residual, float* out, int* idx, float* weight, void* workspace,
                   size_t workspace_bytes, int n_tokens, int hidden, int n_ff, int n_expert, int k,
                   float shared_w, void* stream) {
  const char* nm = "sg_moe_prefill";
  if (!x || !out) return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  return prefill_launch(tab_gate, tab_up, tab_down, sh_gate, sh_up, sh_down, sh_gate_w,
                        XSrc{x, nullptr, nullptr}, logits,
                        PrefillOut{residual, out, nullptr, nullptr}, idx, weight, workspace,
                        workspace_bytes, n_tokens, hidden, n_ff, n_expert, k, shared_w, stream,
                        nm);
}

int sg_moe_prefill_f16(const sg_block_q4k* const* tab_gate, const sg_block_q4k* const* tab_up,
                       const sg_block_q4k* const* tab_down, const sg_block_q4k* sh_gate,
                       const sg_block_q4k* sh_up, const sg_block_q4k* sh_down,
                       const float* sh_gate_w, const uint16_t* xn, const sg_block_q8k* xq,
                       const float* logits, const uint16_t* residual, uint16_t* out, int* idx,
                       float* weight, void* workspace, size_t workspace_bytes, int n_tokens,
                       int hidden, int n_ff, int n_expert, int k, float shared_w, void* stream) {
  const char* nm = "sg_moe_prefill_f16";
  if ((!xn && !xq) || !out) return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  if (!xn && sh_gate_w && sh_gate && sh_up && sh_down)
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: the shared gate needs xn", nm);
  return prefill_launch(tab_gate, tab_up, tab_down, sh_gate, sh_up, sh_down, sh_gate_w,
                        XSrc{nullptr, xn, reinterpret_cast<const unsigned char*>(xq)}, logits,
                        PrefillOut{nullptr, nullptr, residual, out}, idx, weight, workspace,
                        workspace_bytes, n_tokens, hidden, n_ff, n_expert, k, shared_w, stream,
                        nm);
}

}  // extern "C"
