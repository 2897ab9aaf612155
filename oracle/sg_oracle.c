/* sg_oracle.c - CPU oracle for the quantized MoE decode path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for libsager_hip.so, never part of the
 * product path. Built with -ffp-contract=off so every fp32 operation rounds
 * exactly as written. The reference's Release build (g++ -O3 -mavx2 -mfma,
 * CMakeLists.txt:13-15,73-76) lets GCC contract a*b+c into FMAs; the places
 * where it does so on this path are written here as explicit fmaf() calls,
 * which makes the GEMV and expert FFN bit-identical to that build.
 * The one deliberate difference is exp(): orc_expf is correctly rounded
 * (double evaluation), while the reference calls the platform libm.
 *
 * Pinning (tests/test_oracle.py):
 *   orc_half_to_float, orc_get_scale_min   - closed form + reference goldens
 *   orc_quantize_q8_k                      - reference goldens (bit-exact),
 *                                            d = amax/127, bsums = sum q
 *   orc_subblock_dots                      - brute force in numpy int64
 *   orc_gemv_q4k_q8                        - reference goldens (bit-exact),
 *                                            fp64 dequant-dot tolerance
 *   orc_expf                               - libm expf over 1e7 samples
 *   orc_expert_ffn                         - reference goldens (bit-exact)
 *   orc_router_topk                        - numpy softmax + stable argsort,
 *                                            duplicated logits, NaN rows
 *   orc_moe_combine                        - fp64 closed form
 *   orc_float_to_half                      - numpy float16 conversion (RNE)
 *                                            over edge and random values
 *   orc_moe_layer_f16io                    - composition: the fp32 layer's
 *                                            GEMVs with g, u, h and the
 *                                            slot outputs rounded, combined
 *                                            as written here
 *   orc_dispatch_scan                      - counting invariants
 *   orc_dequant_q6k                        - closed form per field (numpy)
 *   orc_q6k_subgroup_dots                  - brute force from the dequant
 *   orc_gemv_q6k_q8                        - fp64 dequant-dot tolerance,
 *                                            32-lane order replayed in numpy
 */
#include "sg_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#if defined(__AVX2__)
#include <immintrin.h>
#endif

#pragma GCC optimize("fp-contract=off")

/* Byte layout of the two block formats (q4_k.hpp:46-62):
 *   Q4_K: u16 d | u16 dmin | u8 scales[12] | u8 qs[128]            144 B
 *   Q8_K: f32 d | i8 qs[256] | i16 bsums[8]                         276 B */
typedef struct {
  uint16_t d, dmin;
  uint8_t scales[12];
  uint8_t qs[128];
} orc_q4k;
typedef struct {
  float d;
  int8_t qs[256];
  int16_t bsums[8];
} __attribute__((packed)) orc_q8k;

_Static_assert(sizeof(orc_q4k) == 144, "Q4_K block is 144 B");
_Static_assert(sizeof(orc_q8k) == 276, "Q8_K block is 276 B");

/* ---- formats ---------------------------------------------------------- */

float orc_half_to_float(uint16_t h) {
  /* IEEE binary16 -> binary32; every fp16 value is exact in fp32. */
  const uint32_t sign = (uint32_t)(h >> 15) << 31;
  const int e = (h >> 10) & 31;
  const uint32_t f = h & 1023u;
  float mag;
  if (e == 0) {
    mag = ldexpf((float)f, -24);               /* zero / subnormal */
  } else if (e == 31) {
    uint32_t b = 0x7f800000u | (f << 13);
    memcpy(&mag, &b, 4);
  } else {
    mag = ldexpf((float)(1024u + f), e - 25);  /* (1.f) * 2^(e-15) */
  }
  uint32_t bits;
  memcpy(&bits, &mag, 4);
  bits |= sign;
  memcpy(&mag, &bits, 4);
  return mag;
}

/* fp32 -> fp16, round to nearest even (the __float2half of the reference's
 * sth(), moe.cu:12-14): infinities and NaN map to fp16 inf / quiet NaN,
 * values from 65520 up overflow to inf, values below 2^-14 become fp16
 * subnormals (multiples of 2^-24, rounded by rintf, which rounds to
 * nearest even). */
uint16_t orc_float_to_half(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u);
  if (ax >= 0x477ff000u) return sign | 0x7c00u;                 /* >= 65520: inf */
  if (ax < 0x38800000u) {                                        /* < 2^-14 */
    float a;
    memcpy(&a, &ax, 4);
    return sign | (uint16_t)rintf(a * 16777216.0f);              /* exact scaling by 2^24 */
  }
  uint32_t h = ((((ax >> 23) - 127u + 15u) << 10)) | ((ax >> 13) & 0x3ffu);
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;  /* a carry bumps the exponent */
  return sign | (uint16_t)h;
}

void orc_float_to_half_n(const float* x, uint16_t* h, int64_t n) {
  for (int64_t i = 0; i < n; ++i) h[i] = orc_float_to_half(x[i]);
}

static float f16_round(float v) { return orc_half_to_float(orc_float_to_half(v)); }

void orc_get_scale_min(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
  /* Sub-blocks 0..3: low 6 bits of bytes j and j+4. Sub-blocks 4..7: a
   * nibble of byte j+4 plus the top two bits of byte j-4 (d) or j (m). */
  if (j < 4) {
    *d = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *d = (uint8_t)((q[j + 4] & 15) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

void orc_dequant(const void* w, float* out, int64_t n) {
  const orc_q4k* b = (const orc_q4k*)w;
  for (int64_t blk = 0; blk < n / 256; ++blk) {
    const float d = orc_half_to_float(b[blk].d);
    const float dm = orc_half_to_float(b[blk].dmin);
    for (int s = 0; s < 8; ++s) {
      uint8_t sc, mn;
      orc_get_scale_min(s, b[blk].scales, &sc, &mn);
      const float sd = d * (float)sc, sm = dm * (float)mn;
      const uint8_t* qg = b[blk].qs + (s >> 1) * 32;
      for (int l = 0; l < 32; ++l) {
        const int nib = (s & 1) ? (qg[l] >> 4) : (qg[l] & 15);
        out[blk * 256 + s * 32 + l] = sd * (float)nib - sm;
      }
    }
  }
}

/* ---- Q8_K quantization (q4_k.cpp:44-61) -------------------------------- */

static int8_t q8_code(float v) {
  /* nearbyintf under the default round-to-nearest-even mode, then the
   * float->int conversion of x86 (NaN -> INT_MIN), then the +-127 clamp. */
  const float r = nearbyintf(v);
  int q;
  if (r != r || r >= 2147483648.0f || r < -2147483648.0f)
    q = INT32_MIN;
  else
    q = (int)r;
  return (int8_t)(q > 127 ? 127 : (q < -127 ? -127 : q));
}

void orc_quantize_q8_k(const float* x, void* out, int n, int n_rows) {
  orc_q8k* o = (orc_q8k*)out;
  const int nb = n / 256;
  for (int64_t r = 0; r < n_rows; ++r) {
    for (int b = 0; b < nb; ++b) {
      const float* xb = x + r * n + (int64_t)b * 256;
      orc_q8k* ob = o + r * nb + b;
      float amax = 1e-30f;
      for (int i = 0; i < 256; ++i) amax = fmaxf(amax, fabsf(xb[i]));
      const float d = amax / 127.f;
      const float id = d > 0 ? 1.f / d : 0.f;
      ob->d = d;
      int16_t bs[8] = {0};
      for (int i = 0; i < 256; ++i) {
        ob->qs[i] = q8_code(xb[i] * id);
        bs[i >> 5] = (int16_t)(bs[i >> 5] + ob->qs[i]);
      }
      memcpy(ob->bsums, bs, sizeof bs);
    }
  }
}

/* ---- integer sub-block dot -------------------------------------------- */

static int32_t sub_dot(const uint8_t* q32, const int8_t* x32, int high) {
#if defined(__AVX2__)
  const __m256i raw = _mm256_loadu_si256((const __m256i*)q32);
  const __m256i m4 = _mm256_set1_epi8(0x0F);
  const __m256i nib =
      high ? _mm256_and_si256(_mm256_srli_epi16(raw, 4), m4) : _mm256_and_si256(raw, m4);
  const __m256i xv = _mm256_loadu_si256((const __m256i*)x32);
  /* u8 x s8 pair sums fit s16 (2*15*127); widen with a multiply by 1. */
  const __m256i p16 = _mm256_maddubs_epi16(nib, xv);
  const __m256i p32 = _mm256_madd_epi16(p16, _mm256_set1_epi16(1));
  __m128i s = _mm_add_epi32(_mm256_castsi256_si128(p32), _mm256_extracti128_si256(p32, 1));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
  return _mm_cvtsi128_si32(s);
#else
  int32_t acc = 0;
  for (int l = 0; l < 32; ++l) acc += (high ? (q32[l] >> 4) : (q32[l] & 15)) * x32[l];
  return acc;
#endif
}

int orc_have_avx2(void) {
#if defined(__AVX2__)
  return 1;
#else
  return 0;
#endif
}

void orc_subblock_dots(const void* w, const void* xq, int32_t* dots, int n_rows,
                       int k) {
  const int nb = k / 256;
  const orc_q4k* W = (const orc_q4k*)w;
  const orc_q8k* X = (const orc_q8k*)xq;
  for (int64_t r = 0; r < n_rows; ++r)
    for (int b = 0; b < nb; ++b)
      for (int s = 0; s < 8; ++s)
        dots[(r * nb + b) * 8 + s] =
            sub_dot(W[r * nb + b].qs + (s >> 1) * 32, X[b].qs + s * 32, s & 1);
}

/* ---- fp32 GEMV in the AVX2 order (q4_avx2.cpp:124-145) ----------------- */

static float row_dot(const orc_q4k* row, const orc_q8k* x, int nb) {
  float acc = 0.f;
  for (int b = 0; b < nb; ++b) {
    const orc_q4k* blk = row + b;
    const float d = orc_half_to_float(blk->d);
    const float dm = orc_half_to_float(blk->dmin);
    float sum = 0.f;
    for (int s = 0; s < 8; ++s) {
      uint8_t sc, mn;
      orc_get_scale_min(s, blk->scales, &sc, &mn);
      const float sd = d * (float)sc;
      const float sm = dm * (float)mn;
      const int32_t ip = sub_dot(blk->qs + (s >> 1) * 32, x[b].qs + s * 32, s & 1);
      /* The reference's Release build (g++ -O3 -mavx2 -mfma) contracts this
       * epilogue into two FMAs: t = sd*ip - (sm*bsum) and sum += xd*t. */
      const float t = fmaf(sd, (float)ip, -(sm * (float)x[b].bsums[s]));
      sum = fmaf(x[b].d, t, sum);
    }
    acc += sum;
  }
  return acc;
}

void orc_gemv_q4k_q8(const void* w, const void* xq, float* y, int n_rows, int k,
                     int n_tokens) {
  const int nb = k / 256;
  const orc_q4k* W = (const orc_q4k*)w;
  const orc_q8k* X = (const orc_q8k*)xq;
  for (int64_t t = 0; t < n_tokens; ++t)
    for (int64_t r = 0; r < n_rows; ++r)
      y[t * n_rows + r] = row_dot(W + r * nb, X + t * nb, nb);
}

/* ---- fp32 GEMV, integer-first super-block epilogue (prefill path) -------
 * The reference's grouped prefill kernels compute the same exact integer
 * sub-block dots as every other path (q4_k.cu:733-741, dp4a_subblock) and
 * differ from the AVX2 path only in fp32 order.  The MFMA prefill kernels
 * here fix one order that maps onto integer matrix cores: per super-block
 * the exact integers I = sum_s sc_s * ip_s and M = sum_s mn_s * bsum_s
 * (|I| < 2^25, |M| < 2^21), then
 *   t = fma(d, (float)I, -(dmin * (float)M));  acc = fma(xd, t, acc)
 * over the super-blocks in order.  Same quantities as q4_avx2.cpp:30-39 and
 * q4_k.cpp:195-203; within ~1e-6 relative of the AVX2 order. */
static float row_dot_int(const orc_q4k* row, const orc_q8k* x, int nb) {
  float acc = 0.f;
  for (int b = 0; b < nb; ++b) {
    const orc_q4k* blk = row + b;
    int32_t I = 0, M = 0;
    for (int s = 0; s < 8; ++s) {
      uint8_t sc, mn;
      orc_get_scale_min(s, blk->scales, &sc, &mn);
      I += (int32_t)sc * sub_dot(blk->qs + (s >> 1) * 32, x[b].qs + s * 32, s & 1);
      M += (int32_t)mn * (int32_t)x[b].bsums[s];
    }
    const float t = fmaf(orc_half_to_float(blk->d), (float)I,
                         -(orc_half_to_float(blk->dmin) * (float)M));
    acc = fmaf(x[b].d, t, acc);
  }
  return acc;
}

void orc_gemv_q4k_q8_int(const void* w, const void* xq, float* y, int n_rows, int k,
                         int n_tokens) {
  const int nb = k / 256;
  const orc_q4k* W = (const orc_q4k*)w;
  const orc_q8k* X = (const orc_q8k*)xq;
  for (int64_t t = 0; t < n_tokens; ++t)
    for (int64_t r = 0; r < n_rows; ++r)
      y[t * n_rows + r] = row_dot_int(W + r * nb, X + t * nb, nb);
}

/* ---- exp (double evaluation, one final rounding) ----------------------- */

/* ---- Q6_K (the LM head) -----------------------------------------------
 * block_q6_K, 210 B per 256 weights (weights.cpp:168-209):
 *   u8 ql[128] | u8 qh[64] | i8 scales[16] | u16 d (bytes 208-209).
 * Weight n*128 + q*32 + l (half n, quarter q, l < 32) is
 *   ((ql[n*64 + (q&1)*32 + l] >> 4*(q>>1)) & 15) | ((qh[n*32 + l] >> 2q) & 3) << 4,
 * minus 32, with scale sc[n*8 + 2q + l/16]. */
void orc_dequant_q6k(const void* w6, float* out, int64_t n) {
  const uint8_t* b = (const uint8_t*)w6;
  for (int64_t blk = 0; blk < n / ORC_QK_K; ++blk, b += ORC_Q6K_BYTES) {
    const int8_t* sc = (const int8_t*)(b + 192);
    uint16_t dh;
    memcpy(&dh, b + 208, 2);
    const float d = orc_half_to_float(dh);
    for (int i = 0; i < ORC_QK_K; ++i) {
      const int nh = i >> 7, q = (i >> 5) & 3, l = i & 31;
      const int lo = (b[nh * 64 + (q & 1) * 32 + l] >> (4 * (q >> 1))) & 15;
      const int hi = (b[128 + nh * 32 + l] >> (2 * q)) & 3;
      out[blk * ORC_QK_K + i] = d * (float)sc[nh * 8 + 2 * q + l / 16] * (float)((lo | hi << 4) - 32);
    }
  }
}

/* int32 sum over sub-group t (16 weights) of block b: sum (q6 - 32) * xq.
 * Sub-group t: half n = t>>3, quarter q = (t&7)>>1, is = t&1 covers weights
 * n*128 + q*32 + is*16 + j (j < 16) with scale sc[t] (q4_k.cu:1595-1613). */
static int32_t q6_subgroup_dot(const uint8_t* blk6, const int8_t* x256, int t) {
  const int n = t >> 3, q = (t & 7) >> 1, is = t & 1;
  const uint8_t* ql = blk6 + n * 64 + (q & 1) * 32 + is * 16;
  const uint8_t* qh = blk6 + 128 + n * 32 + is * 16;
  const int8_t* x = x256 + n * 128 + q * 32 + is * 16;
  int32_t s = 0;
  for (int j = 0; j < 16; ++j) {
    const int v = (((ql[j] >> (4 * (q >> 1))) & 15) | (((qh[j] >> (2 * q)) & 3) << 4)) - 32;
    s += v * (int32_t)x[j];
  }
  return s;
}

void orc_q6k_subgroup_dots(const void* w6, const void* xq, int32_t* dots, int n_rows, int k) {
  const int nb = k / ORC_QK_K;
  const uint8_t* w = (const uint8_t*)w6;
  const orc_q8k* x = (const orc_q8k*)xq;
  for (int r = 0; r < n_rows; ++r)
    for (int b = 0; b < nb; ++b)
      for (int t = 0; t < 16; ++t)
        dots[((int64_t)r * nb + b) * 16 + t] =
            q6_subgroup_dot(w + ((int64_t)r * nb + b) * ORC_Q6K_BYTES, x[b].qs, t);
}

/* y[r] = W6[r] . xq in the reference GPU kernel's fp32 order
 * (gemv_q6_k_q8_kernel, q4_k.cu:1578-1652): 32 lanes per row, lane l takes
 * sub-groups sg = l, l+32, ... (block sg>>4, sub-group sg&15) in order,
 * acc = fma((xd*d)*sc, (float)isum, acc) - nvcc's default contraction of
 * acc += xd*d*sc*isum - then the shfl_down tree over offsets 16..1. */
void orc_gemv_q6k_q8(const void* w6, const void* xq, float* y, int n_rows, int k) {
  const int nb = k / ORC_QK_K;
  const uint8_t* w = (const uint8_t*)w6;
  const orc_q8k* x = (const orc_q8k*)xq;
  for (int r = 0; r < n_rows; ++r) {
    float lane[32] = {0};
    const uint8_t* row = w + (int64_t)r * nb * ORC_Q6K_BYTES;
    for (int sg = 0; sg < nb * 16; ++sg) {
      const int b = sg >> 4, t = sg & 15;
      const uint8_t* blk6 = row + (int64_t)b * ORC_Q6K_BYTES;
      uint16_t dh;
      memcpy(&dh, blk6 + 208, 2);
      const float d = orc_half_to_float(dh);
      const float sc = (float)((const int8_t*)(blk6 + 192))[t];
      const int32_t is = q6_subgroup_dot(blk6, x[b].qs, t);
      lane[sg & 31] = fmaf(x[b].d * d * sc, (float)is, lane[sg & 31]);
    }
    for (int off = 16; off > 0; off >>= 1)
      for (int l = 0; l < off; ++l) lane[l] = lane[l] + lane[l + off];
    y[r] = lane[0];
  }
}

float orc_expf(float xf) {
  if (xf != xf) return xf;
  if (xf > 100.f) return INFINITY;
  if (xf < -110.f) return 0.f;
  const double x = (double)xf;
  /* x = k*ln2 + r, |r| <= ln2/2; ln2 split in two doubles. */
  const double kd = nearbyint(x * 1.4426950408889634);
  const double r = fma(-kd, 2.3190468138462996e-17, fma(-kd, 6.9314718055994529e-01, x));
  /* Taylor series of e^r to degree 13 (remainder < 5e-18 on |r| <= 0.35). */
  /* Estrin evaluation (short dependency chain): pairs, then r^2, r^4, r^8. */
  const double r2 = r * r, r4 = r2 * r2, r8 = r4 * r4;
  const double q0 = fma(1.0, r, 1.0);
  const double q1 = fma(1.0 / 6.0, r, 0.5);
  const double q2 = fma(1.0 / 120.0, r, 1.0 / 24.0);
  const double q3 = fma(1.0 / 5040.0, r, 1.0 / 720.0);
  const double q4 = fma(1.0 / 362880.0, r, 1.0 / 40320.0);
  const double q5 = fma(1.0 / 39916800.0, r, 1.0 / 3628800.0);
  const double q6 = fma(1.0 / 6227020800.0, r, 1.0 / 479001600.0);
  const double s0 = fma(q1, r2, q0), s1 = fma(q3, r2, q2), s2 = fma(q5, r2, q4);
  const double u0 = fma(s1, r4, s0), u1 = fma(q6, r4, s2);
  const double p = fma(u1, r8, u0);
  const int64_t k = (int64_t)kd;
  uint64_t sb = (uint64_t)(k + 1023) << 52;
  double scale;
  memcpy(&scale, &sb, 8);
  return (float)(p * scale);
}

void orc_silu_mul(const float* g, const float* u, float* h, int n) {
  for (int i = 0; i < n; ++i) {
    const float gv = g[i];
    h[i] = gv / (1.f + orc_expf(-gv)) * u[i];
  }
}

/* ---- expert FFN (q4_avx2.cpp:175-196) ---------------------------------- */

/* f16_mid: the session's fp16 buffers - g and u stored as fp16 by the
 * f16out GEMVs, h = fp16(SiLU(g) * u) by silu_mul_f16, and h quantized from
 * those fp16 values (session.cpp:1862-1869, 2791-2803, 2893-2898). */
static void ffn_q8(const void* wg, const void* wu, const void* wd,
                   const orc_q8k* xq, float* y, int hidden, int n_ff, int int_first,
                   int f16_mid) {
  float* g = (float*)malloc(sizeof(float) * 3 * (size_t)n_ff);
  float* u = g + n_ff;
  float* h = u + n_ff;
  orc_q8k* hq = (orc_q8k*)malloc(sizeof(orc_q8k) * (size_t)(n_ff / 256));
  void (*gemv)(const void*, const void*, float*, int, int, int) =
      int_first ? orc_gemv_q4k_q8_int : orc_gemv_q4k_q8;
  gemv(wg, xq, g, n_ff, hidden, 1);
  gemv(wu, xq, u, n_ff, hidden, 1);
  if (f16_mid)
    for (int i = 0; i < n_ff; ++i) {
      g[i] = f16_round(g[i]);
      u[i] = f16_round(u[i]);
    }
  orc_silu_mul(g, u, h, n_ff);
  if (f16_mid)
    for (int i = 0; i < n_ff; ++i) h[i] = f16_round(h[i]);
  orc_quantize_q8_k(h, hq, n_ff, 1);
  gemv(wd, hq, y, hidden, n_ff, 1);
  free(hq);
  free(g);
}

void orc_expert_ffn(const void* wg, const void* wu, const void* wd,
                    const float* x, float* y, int hidden, int n_ff) {
  orc_q8k* xq = (orc_q8k*)malloc(sizeof(orc_q8k) * (size_t)(hidden / 256));
  orc_quantize_q8_k(x, xq, hidden, 1);
  ffn_q8(wg, wu, wd, xq, y, hidden, n_ff, 0, 0);
  free(xq);
}

/* ---- router (moe.cu:25-85) --------------------------------------------- */

void orc_router_topk(const float* logits, int* idx, float* weight, int n_expert,
                     int k, int stride, int n_rows, float shared_w) {
  float* prob = (float*)malloc(sizeof(float) * (size_t)n_expert);
  for (int64_t row = 0; row < n_rows; ++row) {
    const float* lg = logits + row * n_expert;
    int* oi = idx + row * stride;
    float* ow = weight + row * stride;
    float mx = -1e30f;
    for (int i = 0; i < n_expert; ++i) mx = fmaxf(mx, lg[i]);
    float z = 0.f;
    for (int i = 0; i < n_expert; ++i) z += orc_expf(lg[i] - mx);
    for (int i = 0; i < n_expert; ++i) prob[i] = orc_expf(lg[i] - mx) / z;
    float wsum = 0.f;
    for (int kk = 0; kk < k; ++kk) {
      float bv = -1.f;
      int bi = -1;
      for (int i = 0; i < n_expert; ++i) {
        const float p = prob[i];
        if (p == p && p > bv) { bv = p; bi = i; }
      }
      if (bi < 0) bi = kk % n_expert; /* degenerate logits */
      prob[bi] = -1.f;
      oi[kk] = bi;
      ow[kk] = bv;
      wsum += bv;
    }
    if (wsum > 0.f)
      for (int kk = 0; kk < k; ++kk) ow[kk] /= wsum;
    ow[k] = shared_w;
  }
  free(prob);
}

/* ---- combine (moe.cu:265-280, fp32) ------------------------------------ */

void orc_moe_combine(float* out, const float* residual, const float* expert_y,
                     const float* weight, int n_used, int hidden, int n_rows) {
  for (int64_t r = 0; r < n_rows; ++r) {
    const float* yr = expert_y + r * (int64_t)(n_used + 1) * hidden;
    const float* wr = weight + r * (n_used + 1);
    for (int i = 0; i < hidden; ++i) {
      float acc = residual ? residual[r * hidden + i] : 0.f;
      /* nvcc's default --fmad=true contracts the reference's
       * `acc += w * y` (moe.cu:276-277) into one FMA per slot. */
      for (int kk = 0; kk <= n_used; ++kk) acc = fmaf(wr[kk], yr[(int64_t)kk * hidden + i], acc);
      out[r * hidden + i] = acc;
    }
  }
}

/* ---- fp32 weight x activation GEMV: router logits and the shared gate ----
 * gemv_f32_out_kernel / gemv_f32_out_batched_kernel (q4_k.cu:133-149,
 * 285-303): per row, lane l of a 32-lane warp accumulates elements
 * l, l+32, ... (nvcc contracts `acc += w * x` into one FMA), then
 * `acc += __shfl_down_sync(acc, off)` for off = 16, 8, 4, 2, 1; lane 0's
 * value is the row.  A lane whose partner l+off is past 31 keeps its own
 * value, so lane 0's result depends only on lanes 0..31 as written below. */
static float rowdot_lanes32(const float* w, const float* x, int k) {
  float acc[32];
  for (int l = 0; l < 32; ++l) {
    float a = 0.f;
    for (int i = l; i < k; i += 32) a = fmaf(w[i], x[i], a);
    acc[l] = a;
  }
  for (int off = 16; off > 0; off >>= 1)
    for (int l = 0; l + off < 32; ++l) acc[l] = acc[l] + acc[l + off];
  return acc[0];
}

void orc_gemv_f32_lanes(const float* w, const float* x, float* y, int n_rows, int k,
                        int n_tokens) {
  for (int t = 0; t < n_tokens; ++t)
    for (int r = 0; r < n_rows; ++r)
      y[(int64_t)t * n_rows + r] = rowdot_lanes32(w + (int64_t)r * k, x + (int64_t)t * k, k);
}

/* 1 / (1 + exp(-g)) (moe.cu:289, norm_rotary.cu:182) */
float orc_sigmoid(float g) { return 1.f / (1.f + orc_expf(-g)); }

/* ---- worker pool (pool.cpp semantics: one job per expert FFN) ----------- */

typedef struct {
  const void *wg, *wu, *wd;
  const orc_q8k* xq;
  float* y;
  int hidden, n_ff, int_first, f16_mid;
} ffn_job;

typedef struct {
  pthread_mutex_t mu;
  pthread_cond_t cv_work, cv_done;
  ffn_job* jobs;
  int n_jobs, next, done, gen, nthreads, stop;
  pthread_t th[256];
} orc_pool;

static orc_pool g_pool = {.mu = PTHREAD_MUTEX_INITIALIZER,
                          .cv_work = PTHREAD_COND_INITIALIZER,
                          .cv_done = PTHREAD_COND_INITIALIZER};

static void run_job(const ffn_job* j) {
  if (j->wg == NULL || j->wu == NULL || j->wd == NULL) { /* absent expert: zero output */
    memset(j->y, 0, sizeof(float) * (size_t)j->hidden);
    return;
  }
  ffn_q8(j->wg, j->wu, j->wd, j->xq, j->y, j->hidden, j->n_ff, j->int_first, j->f16_mid);
}

static void* worker(void* arg) {
  (void)arg;
  pthread_mutex_lock(&g_pool.mu);
  for (;;) {
    while (!g_pool.stop && g_pool.next >= g_pool.n_jobs)
      pthread_cond_wait(&g_pool.cv_work, &g_pool.mu);
    if (g_pool.stop) break;
    const int j = g_pool.next++;
    pthread_mutex_unlock(&g_pool.mu);
    run_job(&g_pool.jobs[j]);
    pthread_mutex_lock(&g_pool.mu);
    if (++g_pool.done == g_pool.n_jobs) pthread_cond_signal(&g_pool.cv_done);
  }
  pthread_mutex_unlock(&g_pool.mu);
  return NULL;
}

static void pool_run(ffn_job* jobs, int n_jobs, int n_threads) {
  if (n_threads <= 1) {
    for (int j = 0; j < n_jobs; ++j) run_job(&jobs[j]);
    return;
  }
  if (n_threads > 256) n_threads = 256;
  pthread_mutex_lock(&g_pool.mu);
  while (g_pool.nthreads < n_threads) {
    pthread_create(&g_pool.th[g_pool.nthreads], NULL, worker, NULL);
    g_pool.nthreads++;
  }
  g_pool.jobs = jobs;
  g_pool.n_jobs = n_jobs;
  g_pool.next = 0;
  g_pool.done = 0;
  pthread_cond_broadcast(&g_pool.cv_work);
  while (g_pool.done < g_pool.n_jobs) pthread_cond_wait(&g_pool.cv_done, &g_pool.mu);
  g_pool.n_jobs = 0;
  g_pool.next = 0;
  pthread_mutex_unlock(&g_pool.mu);
}

/* ---- MoE layer (session.cpp:2482-3030 stage order) --------------------- */

static void moe_layer_routed(const void* const* tab_gate, const void* const* tab_up,
                             const void* const* tab_down, const void* sh_gate,
                             const void* sh_up, const void* sh_down, const float* sh_gate_w,
                             const float* x,
                             const int* idx, const float* weight, const float* residual,
                             float* out, int n_tokens, int hidden, int n_ff, int n_expert,
                             int k, int n_threads, int int_first, int f16_io) {
  const int nbh = hidden / 256;
  const int slots = k + 1;
  orc_q8k* xq = (orc_q8k*)malloc(sizeof(orc_q8k) * (size_t)nbh * n_tokens);
  orc_quantize_q8_k(x, xq, hidden, n_tokens);
  float* ys = (float*)calloc((size_t)n_tokens * slots * hidden, sizeof(float));
  ffn_job* jobs = (ffn_job*)calloc((size_t)n_tokens * slots, sizeof(ffn_job));
  float* w = (float*)malloc(sizeof(float) * (size_t)n_tokens * slots);
  memcpy(w, weight, sizeof(float) * (size_t)n_tokens * slots);
  int nj = 0;
  for (int t = 0; t < n_tokens; ++t) {
    for (int kk = 0; kk < slots; ++kk) {
      ffn_job* j = &jobs[nj++];
      j->xq = xq + (size_t)t * nbh;
      j->y = ys + ((size_t)t * slots + kk) * hidden;
      j->hidden = hidden;
      j->n_ff = n_ff;
      j->int_first = int_first;
      j->f16_mid = f16_io;
      if (kk < k) {
        const int e = idx[t * slots + kk];
        if (e < 0 || e >= n_expert) {
          /* bounds-kill (moe.cu:391-396): the whole row's weights go to 0 */
          for (int q = 0; q < slots; ++q) w[t * slots + q] = 0.f;
          continue;
        }
        j->wg = tab_gate[e];
        j->wu = tab_up[e];
        j->wd = tab_down[e];
      } else {
        j->wg = sh_gate;
        j->wu = sh_up;
        j->wd = sh_down;
      }
    }
  }
  pool_run(jobs, nj, n_threads);
  /* qwen3.5 shared-expert gate (session.cpp:2904-2909): the shared output
   * of token t is scaled by sigmoid(sh_gate_w . x[t]) before the combine */
  if (f16_io) {
    /* the session's fp16 buffers (session.cpp:2850-2930, moe.cu:249-292):
     * each expert's g, u and h were fp16 (ffn_q8's f16_mid above); every
     * slot output is stored as fp16 (the f16out GEMVs), the shared
     * slot is gated in place on its fp16 value (sigmoid_gate_scalar_batched
     * _f16: fp16(fp16(y) * s)), then moe_combine_batched_f16 accumulates
     * acc = fp32(residual fp16), acc = fma(w, fp32(y fp16), acc) in slot
     * order and stores fp16(acc).  residual holds fp16 values. */
    for (size_t i = 0; i < (size_t)n_tokens * slots * hidden; ++i) ys[i] = f16_round(ys[i]);
    if (sh_gate_w && sh_gate && sh_up && sh_down)
      for (int t = 0; t < n_tokens; ++t) {
        const float s = orc_sigmoid(rowdot_lanes32(sh_gate_w, x + (int64_t)t * hidden, hidden));
        float* yk = ys + ((size_t)t * slots + k) * hidden;
        for (int i = 0; i < hidden; ++i) yk[i] = f16_round(yk[i] * s);
      }
    orc_moe_combine(out, residual, ys, w, k, hidden, n_tokens);
    for (size_t i = 0; i < (size_t)n_tokens * hidden; ++i) out[i] = f16_round(out[i]);
  } else {
    if (sh_gate_w && sh_gate && sh_up && sh_down)
      for (int t = 0; t < n_tokens; ++t) {
        const float s = orc_sigmoid(rowdot_lanes32(sh_gate_w, x + (int64_t)t * hidden, hidden));
        float* yk = ys + ((size_t)t * slots + k) * hidden;
        for (int i = 0; i < hidden; ++i) yk[i] = yk[i] * s;
      }
    orc_moe_combine(out, residual, ys, w, k, hidden, n_tokens);
  }
  free(w);
  free(jobs);
  free(ys);
  free(xq);
}

void orc_moe_layer_routed(const void* const* tab_gate, const void* const* tab_up,
                          const void* const* tab_down, const void* sh_gate, const void* sh_up,
                          const void* sh_down, const float* sh_gate_w, const float* x,
                          const int* idx,
                          const float* weight, const float* residual, float* out,
                          int n_tokens, int hidden, int n_ff, int n_expert, int k,
                          int n_threads) {
  moe_layer_routed(tab_gate, tab_up, tab_down, sh_gate, sh_up, sh_down, sh_gate_w, x, idx,
                   weight, residual, out, n_tokens, hidden, n_ff, n_expert, k, n_threads, 0, 0);
}

/* The prefill layer: the same routing, experts and combine as
 * orc_moe_layer, with every GEMV in the integer-first epilogue order of
 * orc_gemv_q4k_q8_int (what the MFMA prefill kernels compute). */
void orc_moe_prefill(const void* const* tab_gate, const void* const* tab_up,
                     const void* const* tab_down, const void* sh_gate, const void* sh_up,
                     const void* sh_down, const float* sh_gate_w, const float* x,
                     const float* logits, const float* residual, float* out, int* idx,
                     float* weight, int n_tokens, int hidden, int n_ff, int n_expert, int k,
                     float shared_w, int n_threads) {
  if (logits) orc_router_topk(logits, idx, weight, n_expert, k, k + 1, n_tokens, shared_w);
  moe_layer_routed(tab_gate, tab_up, tab_down, sh_gate, sh_up, sh_down, sh_gate_w, x, idx,
                   weight, residual, out, n_tokens, hidden, n_ff, n_expert, k, n_threads, 1, 0);
}

/* The layer on the session's fp16 buffers: x holds the fp16 values of xn
 * (as floats; quantized exactly as the Q8_K the session's fused norm makes
 * from them), residual the fp16 values of the residual stream (NULL: 0),
 * out receives the fp16-rounded combine (as floats).  logits != NULL routes
 * first (idx/weight outputs); else idx/weight are inputs.  int_first: the
 * prefill's GEMV order. */
void orc_moe_layer_f16io(const void* const* tab_gate, const void* const* tab_up,
                         const void* const* tab_down, const void* sh_gate, const void* sh_up,
                         const void* sh_down, const float* sh_gate_w, const float* x,
                         const float* logits, const float* residual, float* out, int* idx,
                         float* weight, int n_tokens, int hidden, int n_ff, int n_expert, int k,
                         float shared_w, int n_threads, int int_first) {
  if (logits) orc_router_topk(logits, idx, weight, n_expert, k, k + 1, n_tokens, shared_w);
  moe_layer_routed(tab_gate, tab_up, tab_down, sh_gate, sh_up, sh_down, sh_gate_w, x, idx,
                   weight, residual, out, n_tokens, hidden, n_ff, n_expert, k, n_threads,
                   int_first, 1);
}

void orc_moe_layer(const void* const* tab_gate, const void* const* tab_up,
                   const void* const* tab_down, const void* sh_gate,
                   const void* sh_up, const void* sh_down, const float* sh_gate_w,
                   const float* x, const float* logits, const float* residual, float* out,
                   int* idx, float* weight, int n_tokens, int hidden, int n_ff,
                   int n_expert, int k, float shared_w, int n_threads) {
  orc_router_topk(logits, idx, weight, n_expert, k, k + 1, n_tokens, shared_w);
  orc_moe_layer_routed(tab_gate, tab_up, tab_down, sh_gate, sh_up, sh_down, sh_gate_w, x,
                       idx, weight, residual, out, n_tokens, hidden, n_ff,
                       n_expert, k, n_threads);
}

/* ---- dispatch plan (moe.cu:366-444, deterministic order) --------------- */

void orc_dispatch_scan(const int* idx, float* weight, int* gslot, int* grows,
                       int* off, int* toff, int* meta, int n_rows, int k,
                       int n_expert, int tok_per) {
  int* hist = (int*)calloc((size_t)n_expert, sizeof(int));
  int bad = 0;
  for (int r = 0; r < n_rows; ++r)
    for (int kk = 0; kk < k; ++kk) {
      const int e = idx[r * (k + 1) + kk];
      if (e < 0 || e >= n_expert) {
        for (int q = 0; q <= k; ++q) weight[r * (k + 1) + q] = 0.f;
        ++bad;
        continue;
      }
      hist[e]++;
    }
  int acc = 0, tacc = 0;
  for (int e = 0; e < n_expert; ++e) {
    off[e] = acc;
    toff[e] = tacc;
    acc += hist[e];
    tacc += (hist[e] + tok_per - 1) / tok_per;
  }
  off[n_expert] = acc;
  toff[n_expert] = tacc;
  meta[0] = acc;
  meta[1] = tacc;
  meta[2] = bad;
  memset(hist, 0, sizeof(int) * (size_t)n_expert);
  for (int r = 0; r < n_rows; ++r)
    for (int kk = 0; kk < k; ++kk) {
      const int e = idx[r * (k + 1) + kk];
      if (e < 0 || e >= n_expert) {
        gslot[r * k + kk] = -1;
        continue;
      }
      const int pos = off[e] + hist[e]++;
      gslot[r * k + kk] = pos;
      grows[pos] = r;
    }
  free(hist);
}

/* ---- test helpers ------------------------------------------------------- */

static uint64_t splitmix(uint64_t* s) {
  uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

int64_t orc_count_expf_mismatch(int64_t n_samples, uint64_t seed, float lo,
                                float hi) {
  int64_t bad = 0;
  uint64_t s = seed;
  for (int64_t i = 0; i < n_samples; ++i) {
    const double u = (double)(splitmix(&s) >> 11) * (1.0 / 9007199254740992.0);
    const float x = (float)(lo + (hi - lo) * u);
    const float a = orc_expf(x), b = expf(x);
    if (memcmp(&a, &b, 4) != 0) ++bad;
  }
  return bad;
}
