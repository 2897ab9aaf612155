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
// Memory: each wave streams row groups (R rows, about 8 KB) into its two LDS
// buffers with buffer_load_dwordx4 ... lds (the copy of the next group is in
// flight while the current one is computed); the 210-B blocks sit at 2-byte
// alignment in LDS, so 16-B fields are read as five dwords and byte-aligned
// (v_alignbyte).  The activation (Q8_K) is staged once per workgroup with
// the per-16 sums the zero point needs: I = sum code'*x - 32 * sum x.
#include "sg_common.hpp"

namespace sg {

constexpr int kQ6Bytes = 210;
constexpr int kQ6Waves = 4;
constexpr int kQ6GroupBytes = 8192;  // target bytes per row group
constexpr int kQ6XWords = 84;        // staged Q8_K block: 64 qs words, d, 16 sums, pad

static int q6_rows_per_group(int nb) {
  const int r = (kQ6GroupBytes / (nb * kQ6Bytes)) & ~1;
  return r < 2 ? 2 : r;
}
// words per LDS buffer: the group's bytes, its start offset (< 16) and the
// over-read of the last 16-B field (one dword), rounded to 16 B
static int q6_buf_words(int nb) {
  const int bytes = q6_rows_per_group(nb) * nb * kQ6Bytes + 16 + 16;
  return (bytes + 15) / 16 * 4;
}

// 16 bytes at byte offset off (2-byte aligned) of LDS
__device__ __forceinline__ u32x4 lds_read16(const uint32_t* base, uint32_t off) {
  const uint32_t* p = base + (off >> 2);
  const uint32_t sh = off & 3;
  const uint32_t w0 = p[0], w1 = p[1], w2 = p[2], w3 = p[3], w4 = p[4];
  return (u32x4){__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh),
                 __builtin_amdgcn_alignbyte(w3, w2, sh), __builtin_amdgcn_alignbyte(w4, w3, sh)};
}

__global__ void __launch_bounds__(256) gemv_q6_kernel(const unsigned char* __restrict__ w6,
                                                      const unsigned char* __restrict__ xq,
                                                      float* __restrict__ y, int n_rows, int nb,
                                                      int R, int buf_words) {
  extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  uint32_t* xs = lds;  // nb * kQ6XWords
  uint32_t* bufs[2] = {lds + nb * kQ6XWords + wv * 2 * buf_words,
                       lds + nb * kQ6XWords + wv * 2 * buf_words + buf_words};
  const uint32_t row_bytes = static_cast<uint32_t>(nb) * kQ6Bytes;
  const int n_groups = (n_rows + R - 1) / R;
  const int n_waves = gridDim.x * kQ6Waves;
  const u32x4 rw = buffer_desc(w6, static_cast<uint32_t>(n_rows) * row_bytes);
  const uint32_t last_blk = static_cast<uint32_t>(n_rows) * nb - 1;

  // copy of row group gg into buf: bytes [start & ~15, end) in 16-B chunks
  // (dwords past the matrix end - the buffer's size - read as zeros)
  auto n_chunks = [&](int gg) {
    const uint32_t start = static_cast<uint32_t>(gg) * R * row_bytes;
    const int nr = min(R, n_rows - gg * R);
    return static_cast<int>(((start & 15u) + nr * row_bytes + 15) / 16);
  };
  auto issue = [&](int gg, uint32_t* buf) {
    const uint32_t a0 = (static_cast<uint32_t>(gg) * R * row_bytes) & ~15u;
    const int nch = n_chunks(gg);
    for (int c0 = 0; c0 < nch; c0 += 64)
      if (c0 + lane < nch) dma16(buf + 4 * c0, a0 + 16 * (c0 + lane), rw, 0);
  };
  int g = blockIdx.x * kQ6Waves + wv;
  if (g < n_groups) issue(g, bufs[0]);
  if (g + n_waves < n_groups) issue(g + n_waves, bufs[1]);

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
  const uint32_t ql_off = qn * 64 + (qq & 1) * 32 + is * 16, qh_off = 128 + qn * 32 + is * 16;
  const uint32_t nib = (qq & 2) ? 4 : 0, hsh = 2 * qq;
  const int xw = (qn * 128 + qq * 32 + is * 16) / 4;  // first qs word of the sub-group
  const int8_t* lds8 = nullptr;

  for (int cur = 0; g < n_groups; g += n_waves, cur ^= 1) {
    const int gn = g + n_waves;
    // group g has landed: only the next group's copy may still be in flight
    wait_vm_n(gn < n_groups ? (n_chunks(gn) + 63) / 64 : 0);
    const uint32_t* buf = bufs[cur];
    lds8 = reinterpret_cast<const int8_t*>(buf);
    const int r0 = g * R, nr = min(R, n_rows - r0);
    const uint32_t o0 = (static_cast<uint32_t>(r0) * row_bytes) & 15u;
    for (int p = 0; p < nr; p += 2) {
      const int row = p + half;
      float acc = 0.f;
      if (row < nr) {
        const uint32_t rb = o0 + static_cast<uint32_t>(row) * row_bytes;
        for (int sg = l; sg < nb * 16; sg += 32) {
          const int blk = sg >> 4;
          const uint32_t bb = rb + blk * kQ6Bytes;
          const u32x4 ql = lds_read16(buf, bb + ql_off);
          const u32x4 qh = lds_read16(buf, bb + qh_off);
          const float sc = static_cast<float>(lds8[bb + 192 + t]);
          // the matrix's last d sits in a dword that ends past the buffer's
          // size when the size is 2 mod 4 (the copy then returns zeros for
          // it): read that one from memory
          const uint32_t gblk = static_cast<uint32_t>(r0 + row) * nb + blk;
          const uint32_t dh = gblk == last_blk
                                  ? *reinterpret_cast<const uint16_t*>(w6 + static_cast<size_t>(gblk) * kQ6Bytes + 208)
                                  : reinterpret_cast<const uint16_t*>(buf)[(bb + 208) >> 1];
          const uint32_t* xb = xs + blk * kQ6XWords;
          const u32x4 xv = *reinterpret_cast<const u32x4*>(xb + xw);
          int isum = 0;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t code = ((ql[j] >> nib) & 0x0F0F0F0Fu) | (((qh[j] >> hsh) & 0x03030303u) << 4);
            isum = __builtin_amdgcn_sdot4(static_cast<int>(code), static_cast<int>(xv[j]), isum, false);
          }
          isum -= 32 * static_cast<int>(xb[65 + t]);
          const float xd = __builtin_bit_cast(float, xb[64]);
          const float d = half_bits_to_float(dh);
          acc = __builtin_fmaf(xd * d * sc, static_cast<float>(isum), acc);
        }
      }
#pragma unroll
      for (int off = 16; off > 0; off >>= 1) acc += __shfl_down(acc, off, 32);
      if (l == 0 && row < nr) y[r0 + row] = acc;
    }
    const int g2 = g + 2 * n_waves;
    if (g2 < n_groups) {
      wait_lds();  // every read of this buffer has returned
      issue(g2, bufs[cur]);
    }
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
  const unsigned grid = static_cast<unsigned>(wgs < 512 ? wgs : 512);  // two per CU
  const size_t lds_bytes = (static_cast<size_t>(nb) * kQ6XWords + kQ6Waves * 2 * bw) * 4;
  hipLaunchKernelGGL(gemv_q6_kernel, dim3(grid), dim3(256), lds_bytes,
                     static_cast<hipStream_t>(stream), static_cast<const unsigned char*>(w6),
                     reinterpret_cast<const unsigned char*>(x), y, n_rows, nb, R, bw);
  return check_launch(nm);
}

}  // extern "C"
