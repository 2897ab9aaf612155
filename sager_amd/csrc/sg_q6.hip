// sg_q6.hip - the Q6_K x Q8_K GEMV (the real model's LM head) on gfx950.
//
// Reference: gemv_q6_k_q8 (cuda_ops.hpp:44-48; q4_k.cu:1565-1658), block
// layout block_q6_K (weights.cpp:168-209): ql[128] | qh[64] | i8 sc[16] |
// fp16 d, 210 B per 256 weights.  Sub-group t (16 weights) of a block:
// half n = t>>3, quarter q = (t&7)>>1, is = t&1 covers weights
// n*128 + q*32 + is*16 + j, code (ql nibble q>>1 | qh bits 2q..2q+1 << 4)
// - 32, scale sc[t].
//
// Arithmetic (the reference kernel's, so the fp32 bits are reproducible):
// the int32 sub-group sum I = sum_j (code_j) * xq_j is exact; 32 lanes per
// row, lane l accumulating sub-groups sg = l, l+32, ... (block sg>>4) as
// acc = fma((xd*d)*sc, (float)I, acc), then the shfl_down tree over offsets
// 16, 8, 4, 2, 1.  Here one wave holds two rows (a half-wave each, lane l of
// the half = reference lane l).
//
// Memory: each wave streams row groups (R rows, about 4 KB) into its two LDS
// buffers with buffer_load_dwordx4 ... lds (the copy of the next group is in
// flight while the current one is computed), each 210-B block into a 224-B
// slot so that its 16-B fields are aligned (the copy reads from 2-byte
// aligned offsets).  The activation (Q8_K) is staged once per workgroup with
// the per-16 sums the zero point needs: I = sum code'*x - 32 * sum x.
#include "sg_common.hpp"

namespace sg {

constexpr int kQ6Bytes = 210;
constexpr int kQ6Waves = 4;
constexpr int kQ6GroupBytes = 4096;  // target bytes per row group
constexpr int kQ6WgPerCu = 3;        // grid cap (LDS allows three at K = 2048)
constexpr int kQ6XWords = 84;        // staged Q8_K block: 64 qs words, d, 16 sums, pad

__host__ __device__ constexpr int q6_rows_per_group(int nb) {
  return ((kQ6GroupBytes / (nb * kQ6Bytes)) & ~1) < 2 ? 2
                                                    : ((kQ6GroupBytes / (nb * kQ6Bytes)) & ~1);
}
// words per LDS buffer: one 224-B slot per block of the group
static int q6_buf_words(int nb) { return q6_rows_per_group(nb) * nb * 224 / 4; }

// LDS slot of one block: its 210 bytes copied as 14 16-B chunks (the last
// one runs 14 bytes into the next block), so every 16-B field is aligned
constexpr int kQ6Slot = 224;
constexpr int kQ6SlotChunks = kQ6Slot / 16;

// kNb > 0: the super-blocks per row fixed at compile time (the head's
// K = 2048); 0: taken from nb_arg.  kQ6Depth: row groups in flight per
// wave (the LDS ring's slots).
template <int kNb, int kQ6Depth>
__global__ void __launch_bounds__(256) gemv_q6_kernel(const unsigned char* __restrict__ w6,
                                                      const unsigned char* __restrict__ xq,
                                                      float* __restrict__ y, int n_rows, int nb_arg,
                                                      int R_arg, int buf_words, int gpw) {
  const int nb = kNb > 0 ? kNb : nb_arg;
  const int R = kNb > 0 ? q6_rows_per_group(kNb) : R_arg;
  extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  uint32_t* xs = lds;  // nb * kQ6XWords
  uint32_t* ring = lds + nb * kQ6XWords + wv * kQ6Depth * buf_words;
  // the wave's results, written out once at the end: a global store between
  // the copies would join the vmcnt queue that the copies are waited on with
  float* ys = reinterpret_cast<float*>(lds + nb * kQ6XWords + kQ6Waves * kQ6Depth * buf_words) +
              wv * gpw * R;
  const uint32_t row_bytes = static_cast<uint32_t>(nb) * kQ6Bytes;
  const int n_groups = (n_rows + R - 1) / R;
  // wave W of the NW takes groups W, W + NW, W + 2 NW, ...: at any moment the
  // chip reads one window of the matrix (a contiguous range per wave, its
  // waves far apart in HBM, measured 7 % slower on the 418 MB head)
  const int NW = gridDim.x * kQ6Waves;
  const int g_begin = blockIdx.x * kQ6Waves + wv, g_end = n_groups;
  const u32x4 rw = buffer_desc(w6, static_cast<uint32_t>(n_rows) * row_bytes);
  const uint32_t last_blk = static_cast<uint32_t>(n_rows) * nb - 1;

  // copy of row group gg: block slot s (row s / nb, block s % nb) from the
  // group's byte offset + 210 s, chunk by chunk; the per-lane part of the
  // offset is fixed, the group's goes in the scalar offset.  Bytes past the
  // matrix end (the buffer's size) read as zeros.
  const int n_slots = R * nb;
  const int n_instr = (n_slots * kQ6SlotChunks + 63) / 64;
  auto issue = [&](int gg, uint32_t* buf) {
    const int nr = min(R, n_rows - gg * R);
    const int nch = nr * nb * kQ6SlotChunks;
    const uint32_t base = static_cast<uint32_t>(gg) * R * row_bytes;
    for (int i = 0; i < n_instr; ++i) {
      const int c = 64 * i + lane;
      const int slot = c / kQ6SlotChunks, j = c - slot * kQ6SlotChunks;
      if (64 * i < nch && c < nch)
        dma16<true>(buf + 256 * i, slot * kQ6Bytes + 16 * j, rw, base);
    }
  };
  // instructions a copy of group gg issues (for the vmcnt waits)
  auto instrs = [&](int gg) { return (min(R, n_rows - gg * R) * nb * kQ6SlotChunks + 63) / 64; };
  int g = g_begin;
  for (int j = 0; j < kQ6Depth - 1; ++j)
    if (g + j * NW < g_end) issue(g + j * NW, ring + j * buf_words);

  // the matrix's last d sits in a dword that ends past the buffer's size
  // when the size is 2 mod 4 (the copy then returns zeros for it): it is
  // read from memory here, once, so that no global load joins the copies'
  // vmcnt queue inside the loop (its wait would drain every copy in flight)
  // (the aligned dword holding it, by a scalar load: the vector loads' queue
  // stays the copies' alone)
  const size_t last_off = static_cast<size_t>(last_blk) * kQ6Bytes + 208;
  const unsigned long long last_a =
      reinterpret_cast<unsigned long long>(w6) + (last_off & ~static_cast<size_t>(3));
  uint32_t last_w;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(last_w) : "s"(last_a));
  const uint32_t last_d = (last_off & 2) ? last_w >> 16 : last_w & 0xFFFFu;
  // stage x: qs words, d, and the 16 sums of 16 codes per block
  for (int i = threadIdx.x; i < nb * 65; i += blockDim.x) {
    const int b = i / 65, j = i - b * 65;
    const uint32_t v = reinterpret_cast<const uint32_t*>(xq + static_cast<long long>(b) * kQ8Bytes)[j];
    xs[b * kQ6XWords + (j == 0 ? 64 : j - 1)] = v;
  }
  bar();
  for (int i = threadIdx.x; i < nb * 16; i += blockDim.x) {
    const int b = i >> 4, t = i & 15;
    int s = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      s = __builtin_amdgcn_sdot4(static_cast<int>(xs[b * kQ6XWords + 4 * t + j]), 0x01010101, s,
                                 false);
    xs[b * kQ6XWords + 65 + t] = static_cast<uint32_t>(s);
  }
  bar();

  // the lane's fixed sub-group position (sg & 15 == l & 15 for every sg of the lane)
  const int half = lane >> 5, l = lane & 31;
  const int t = l & 15, qn = t >> 3, qq = (t & 7) >> 1, is = t & 1;
  const int ql_w = (qn * 64 + (qq & 1) * 32 + is * 16) / 4, qh_w = (128 + qn * 32 + is * 16) / 4;
  const uint32_t nib = (qq & 2) ? 4 : 0, hsh = 2 * qq;
  const int xw = (qn * 128 + qq * 32 + is * 16) / 4;  // first qs word of the sub-group

  for (int cur = 0, li = 0; g < g_end; g += NW, ++li, cur = cur + 1 == kQ6Depth ? 0 : cur + 1) {
    // group g has landed: only the copies of the next kQ6Depth - 2 groups may
    // still be in flight
    int younger = 0;
#pragma unroll
    for (int j = 1; j < kQ6Depth - 1; ++j)
      if (g + j * NW < g_end) younger += instrs(g + j * NW);
    wait_vm_n(younger);
    // refill the slot of group g - 1 (read in the previous iteration) with
    // g + depth - 1 before computing on g
    const int g2 = g + (kQ6Depth - 1) * NW;
    if (g2 < g_end) {
      wait_lds();  // every read of the ring so far has returned
      issue(g2, ring + (cur == 0 ? kQ6Depth - 1 : cur - 1) * buf_words);
    }
    const uint32_t* buf = ring + cur * buf_words;
    const int r0 = g * R, nr = min(R, n_rows - r0);
    for (int p = 0; p < nr; p += 2) {
      const int row = p + half;
      float acc = 0.f;
      if (row < nr) {
#pragma unroll 4
        for (int sg = l; sg < nb * 16; sg += 32) {
          const int blk = sg >> 4;
          const uint32_t* sl = buf + (row * nb + blk) * (kQ6Slot / 4);
          const u32x4 ql = *reinterpret_cast<const u32x4*>(sl + ql_w);
          const u32x4 qh = *reinterpret_cast<const u32x4*>(sl + qh_w);
          const float sc = static_cast<float>(reinterpret_cast<const int8_t*>(sl)[192 + t]);
          const uint32_t gblk = static_cast<uint32_t>(r0 + row) * nb + blk;
          const uint32_t dh = gblk == last_blk ? last_d : reinterpret_cast<const uint16_t*>(sl)[104];
          const uint32_t* xb = xs + blk * kQ6XWords;
          const u32x4 xv = *reinterpret_cast<const u32x4*>(xb + xw);
          int isum = 0;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t code =
                ((ql[j] >> nib) & 0x0F0F0F0Fu) | (((qh[j] >> hsh) & 0x03030303u) << 4);
            isum = __builtin_amdgcn_sdot4(static_cast<int>(code), static_cast<int>(xv[j]), isum,
                                          false);
          }
          isum -= 32 * static_cast<int>(xb[65 + t]);
          const float xd = __builtin_bit_cast(float, xb[64]);
          const float d = half_bits_to_float(dh);
          acc = __builtin_fmaf(xd * d * sc, static_cast<float>(isum), acc);
        }
      }
      // shfl_down tree over the half's 32 lanes (offsets 16, 8, 4, 2, 1; only
      // lane 0's sum is used): xor-16 swizzle, then DPP row shifts
      acc += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, acc), 0x401F));
      acc += dpp_f<0x108>(acc);  // row_shl:8
      acc += dpp_f<0x104>(acc);
      acc += dpp_f<0x102>(acc);
      acc += dpp_f<0x101>(acc);
      if (l == 0 && row < nr) ys[li * R + row] = acc;
    }
  }
  wait_lds();  // this wave's result writes (read back by its own lanes)
  // result li * R + row of the wave belongs to group g_begin + li * NW
  for (int i = lane; i < gpw * R; i += 64) {
    const int r = (g_begin + (i / R) * NW) * R + i % R;
    if (r < n_rows) y[r] = ys[i];
  }
}

}  // namespace sg

using namespace sg;

extern "C" {

int sg_gemv_q6_k_q8(const void* w6, const sg_block_q8k* x, float* y, int n_rows, int k,
                    void* stream) {
  const char* nm = "sg_gemv_q6_k_q8";
  if (!w6 || !x || !y) return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  if (n_rows <= 0 || k <= 0 || k % kQK != 0)
    return set_error(SG_ERR_GEOMETRY, "%s: n_rows=%d k=%d (k must be a positive multiple of 256)",
                     nm, n_rows, k);
  const int nb = k / kQK;
  // LDS: the staged activation plus two buffers of at least two rows per wave
  if (nb > 32) return set_error(SG_ERR_UNSUPPORTED, "%s: k=%d exceeds 8192", nm, k);
  if (static_cast<long long>(n_rows) * nb * kQ6Bytes >= (1LL << 31))
    return set_error(SG_ERR_UNSUPPORTED, "%s: matrix of %lld bytes exceeds 2 GiB", nm,
                     static_cast<long long>(n_rows) * nb * kQ6Bytes);
  const int R = q6_rows_per_group(nb), bw = q6_buf_words(nb);
  const long long n_groups = (n_rows + R - 1) / R;
  const long long wgs = (n_groups + kQ6Waves - 1) / kQ6Waves;
  const long long cap = 256LL * kQ6WgPerCu;
  const unsigned grid = static_cast<unsigned>(wgs < cap ? wgs : cap);
  // three groups in flight at K = 2048; two otherwise (the ring must fit LDS)
  const int depth = nb == 8 ? 3 : 2;
  const int gpw = static_cast<int>((n_groups + grid * kQ6Waves - 1) / (grid * kQ6Waves));
  const size_t lds_bytes =
      (static_cast<size_t>(nb) * kQ6XWords + kQ6Waves * depth * bw + kQ6Waves * gpw * R) * 4;
  if (lds_bytes > 160 * 1024)
    return set_error(SG_ERR_UNSUPPORTED, "%s: n_rows=%d needs %zu B of LDS", nm, n_rows, lds_bytes);
  auto kern = nb == 8 ? gemv_q6_kernel<8, 3> : gemv_q6_kernel<0, 2>;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), lds_bytes, static_cast<hipStream_t>(stream),
                     static_cast<const unsigned char*>(w6),
                     reinterpret_cast<const unsigned char*>(x), y, n_rows, nb, R, bw, gpw);
  return check_launch(nm);
}

}  // extern "C"
