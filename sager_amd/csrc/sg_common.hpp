// sg_common.hpp - device helpers shared by the gfx950 kernels: block
// formats, exact fp16 decode, 6-bit scale unpack, the int8 sub-block dot,
// the super-block epilogue, exp, and wave64 helpers.
//
// Numerics contract (all kernels): compiled with -ffp-contract=off; every
// fused multiply-add below is written as an explicit fmaf so the fp32 results
// are bit-identical to the reference's CPU build on the same Q8_K input.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/sager_hip.h"

namespace sg {

constexpr int kQK = 256;          // weights per super-block
constexpr int kQ4Bytes = 144;     // Q4_K super-block
constexpr int kQ8Bytes = 276;     // Q8_K block
constexpr int kWave = 64;

// ---- status plumbing (host) -------------------------------------------
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

// ---- exact fp16 -> fp32 --------------------------------------------------
__device__ __forceinline__ float half_bits_to_float(uint32_t h16) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h16)));
}

// ---- the 8 sub-block scales and mins of one super-block ----------------
// The 12 packed bytes are words A (bytes 0-3), B (4-7), C (8-11):
//   scale j<4 = A.byte j & 63          min j<4 = B.byte j & 63
//   scale j>=4 = (C.byte(j-4) & 15) | (A.byte(j-4) >> 6) << 4
//   min   j>=4 = (C.byte(j-4) >> 4) | (B.byte(j-4) >> 6) << 4
// (q4_k.hpp:110-118, evaluated four sub-blocks per 32-bit operation.)
struct ScaleMins {
  uint32_t sc_lo, sc_hi, mn_lo, mn_hi;  // one 6-bit value per byte
};
__device__ __forceinline__ ScaleMins unpack_scales(uint32_t A, uint32_t B, uint32_t C) {
  ScaleMins r;
  r.sc_lo = A & 0x3F3F3F3Fu;
  r.mn_lo = B & 0x3F3F3F3Fu;
  r.sc_hi = (C & 0x0F0F0F0Fu) | ((A >> 2) & 0x30303030u);
  r.mn_hi = ((C >> 4) & 0x0F0F0F0Fu) | ((B >> 2) & 0x30303030u);
  return r;
}
__device__ __forceinline__ float byte_f(uint32_t w, int i) {
  return static_cast<float>((w >> (8 * i)) & 0xFFu);
}

// ---- int8 sub-block dots of one super-block -----------------------------
// q: the 32 qs words of the block; x: the 64 qs words of the matching Q8_K
// block. ip[s] = sum over the 32 weights of sub-block s of nibble * x.
// Nibbles (0..15) are exact as signed int8, so v_dot4 i8 x i8 is exact.
__device__ __forceinline__ void subblock_dots(const uint32_t* q, const int32_t* x,
                                              int32_t ip[8]) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    int32_t lo = 0, hi = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t w = q[8 * g + j];
      lo = __builtin_amdgcn_sdot4(static_cast<int>(w & 0x0F0F0F0Fu), x[16 * g + j], lo, false);
      hi = __builtin_amdgcn_sdot4(static_cast<int>((w >> 4) & 0x0F0F0F0Fu), x[16 * g + 8 + j], hi,
                                  false);
    }
    ip[2 * g] = lo;
    ip[2 * g + 1] = hi;
  }
}

// ---- super-block epilogue in the reference order -------------------------
// sum_s fma(xd, fma(sd_s, ip_s, -(sm_s * bsum_s)), sum), sd = d*scale,
// sm = dmin*min (q4_avx2.cpp:30-39,112-121,134-141 as compiled).
__device__ __forceinline__ float block_sum(uint32_t dd, const ScaleMins& sm8, const int32_t ip[8],
                                           float xd, const float bsf[8]) {
  const float d = half_bits_to_float(dd & 0xFFFFu);
  const float dmin = half_bits_to_float(dd >> 16);
  float sum = 0.f;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const uint32_t scw = s < 4 ? sm8.sc_lo : sm8.sc_hi;
    const uint32_t mnw = s < 4 ? sm8.mn_lo : sm8.mn_hi;
    const float sd = d * byte_f(scw, s & 3);
    const float smv = dmin * byte_f(mnw, s & 3);
    const float t = __builtin_fmaf(sd, static_cast<float>(ip[s]), -(smv * bsf[s]));
    sum = __builtin_fmaf(xd, t, sum);
  }
  return sum;
}

// Full dot of one Q4_K block (36 words) with one Q8_K block held as
// 64 qs words + d + float bsums.
__device__ __forceinline__ float q4k_block_dot(const uint32_t* w36, const int32_t* xq64, float xd,
                                               const float bsf[8]) {
  int32_t ip[8];
  subblock_dots(w36 + 4, xq64, ip);
  const ScaleMins sm8 = unpack_scales(w36[1], w36[2], w36[3]);
  return block_sum(w36[0], sm8, ip, xd, bsf);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// Cache policy of a weight stream read once per launch (the GEMVs' and the
// decode layer's weights): non-temporal, so that it does not displace what
// is re-read from the caches.  Measured on the 256-matrix pointer-table GEMV:
// 104 -> 92 us; the decode layer about 0.15 us per token faster.  Not for
// the prefill's grouped weights, whose column slices re-read each expert's
// rows from L2 (8 % slower with it).
constexpr int kNt = 2;
typedef __attribute__((address_space(3))) void* lds_void_p;
typedef __attribute__((address_space(1))) void* glb_void_p;

// ---- weight streaming: global -> LDS without passing through VGPRs ---------
// A wave copies n_chunks (<= 576) 16-B chunks with global_load_lds_dwordx4:
// instruction i moves chunk c = lane + 64*i to dst + 16*c, so each
// instruction reads 1 KB of consecutive global memory when the source is
// contiguous (fully coalesced), and nothing occupies registers while the
// data is in flight.  src(c) returns the global address of chunk c.
// With part/nparts, only instructions i = part, part + nparts, ... (several
// waves sharing one copy).  kAux: the copies' cache policy bits (kNt for a
// weight stream that nothing re-reads).
template <int kAux = 0, typename Src>
__device__ __forceinline__ void dma_chunks(Src src, int n_chunks, uint32_t* dst, int lane,
                                           int part = 0, int nparts = 1) {
#pragma unroll
  for (int i = 0; i < 9; ++i) {
    const int c = lane + 64 * i;
    if (i % nparts == part && i * 64 < n_chunks && c < n_chunks)
      __builtin_amdgcn_global_load_lds((glb_void_p)src(c), (lds_void_p)(dst + 256 * i), 16, 0,
                                       kAux);
  }
}
// Same for any number of chunks (576 per round).
template <typename Src>
__device__ __forceinline__ void dma_range(Src src, int n_chunks, uint32_t* dst, int lane) {
  for (int c0 = 0; c0 < n_chunks; c0 += 576)
    dma_chunks([&](int c) { return src(c0 + c); }, min(576, n_chunks - c0), dst + 4 * c0, lane);
}
// raw buffer descriptor: base address, stride 0, size in bytes, dword format
// (wave-uniform arguments; the words are moved to scalar registers)
__device__ __forceinline__ u32x4 buffer_desc(const void* base, uint32_t bytes) {
  const uint64_t v = reinterpret_cast<uintptr_t>(base);
  auto rfl = [](uint32_t x) { return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(x)); };
  return (u32x4){rfl(static_cast<uint32_t>(v)), rfl(static_cast<uint32_t>(v >> 32) & 0xFFFFu),
                 rfl(bytes), 0x00020000u};
}

// 16 B per lane from buffer rsrc at voff + soff into LDS at lds + 16 * lane
// (buffer_load_dwordx4 ... lds; with kStream, non-temporal as kNt).  Inline asm on purpose: the compiler then
// does not treat it as an LDS store in flight, which would make it wait for
// every outstanding copy before each LDS read; the kernels order these
// copies themselves (vmcnt waits and barriers).  Sets M0, which the
// compiler uses for nothing else in these kernels.
template <bool kStream = false>
__device__ __forceinline__ void dma16(const uint32_t* lds, uint32_t voff, u32x4 rsrc,
                                      uint32_t soff) {
  const uint32_t l =
      __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)));
  soff = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(soff));
  if (kStream)
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen nt lds"
                 :
                 : "s"(l), "v"(voff), "s"(rsrc), "s"(soff)
                 : "memory");
  else
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(l), "v"(voff), "s"(rsrc), "s"(soff)
                 : "memory");
}

// a pointer the caller knows to be wave-uniform, moved to scalar registers
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  const uint64_t v = reinterpret_cast<uintptr_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<T*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Wait for every outstanding global load of this wave (the DMA included).
__device__ __forceinline__ void wait_vm() {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
// Wait until at most n (0..15) of this wave's vector memory operations are
// outstanding: with two weight streams in flight, the older has landed once
// only the newer one's instructions remain.
__device__ __forceinline__ void wait_vm_n(int n) {
  switch (n) {
    case 15: __builtin_amdgcn_s_waitcnt(0x0F7F); break;  // vmcnt(15)
    case 14: __builtin_amdgcn_s_waitcnt(0x0F7E); break;
    case 13: __builtin_amdgcn_s_waitcnt(0x0F7D); break;
    case 12: __builtin_amdgcn_s_waitcnt(0x0F7C); break;
    case 11: __builtin_amdgcn_s_waitcnt(0x0F7B); break;
    case 10: __builtin_amdgcn_s_waitcnt(0x0F7A); break;
    case 9: __builtin_amdgcn_s_waitcnt(0x0F79); break;
    case 8: __builtin_amdgcn_s_waitcnt(0x0F78); break;
    case 7: __builtin_amdgcn_s_waitcnt(0x0F77); break;
    case 6: __builtin_amdgcn_s_waitcnt(0x0F76); break;
    case 5: __builtin_amdgcn_s_waitcnt(0x0F75); break;
    case 4: __builtin_amdgcn_s_waitcnt(0x0F74); break;
    case 3: __builtin_amdgcn_s_waitcnt(0x0F73); break;
    case 2: __builtin_amdgcn_s_waitcnt(0x0F72); break;
    case 1: __builtin_amdgcn_s_waitcnt(0x0F71); break;
    default: __builtin_amdgcn_s_waitcnt(0x0F70); break;
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
// Wait for this wave's LDS reads, so the buffer can be refilled.
__device__ __forceinline__ void wait_lds() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
}
// Workgroup barrier for LDS data: this wave's LDS operations complete,
// then s_barrier.  Unlike __syncthreads it does not wait for outstanding
// global loads - the LDS DMA included - so a weight stream issued before it
// keeps flowing; a wave reads LDS it filled by DMA only after wait_vm().
__device__ __forceinline__ void bar() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
// One 144-B block from LDS (16-B aligned) into 36 registers.
__device__ __forceinline__ void read_block_lds(const uint32_t* b, uint32_t* w36) {
  const u32x4* p = reinterpret_cast<const u32x4*>(b);
#pragma unroll
  for (int i = 0; i < 9; ++i) {
    const u32x4 v = p[i];
    w36[4 * i + 0] = v.x;
    w36[4 * i + 1] = v.y;
    w36[4 * i + 2] = v.z;
    w36[4 * i + 3] = v.w;
  }
}

// A double constant built in scalar registers (two s_mov_b32 through asm):
// the compiler then keeps it there, as a scalar operand of the vector
// instructions, instead of in a pair of vector registers.
template <unsigned long long B>
__device__ __forceinline__ double sconst() {
  unsigned lo, hi;
  asm("s_mov_b32 %0, %1" : "=s"(lo) : "n"(static_cast<unsigned>(B & 0xFFFFFFFFull)));
  asm("s_mov_b32 %0, %1" : "=s"(hi) : "n"(static_cast<unsigned>(B >> 32)));
  return __builtin_bit_cast(double, (static_cast<unsigned long long>(hi) << 32) | lo);
}
#define SG_SCONST(v) sconst<__builtin_bit_cast(unsigned long long, static_cast<double>(v))>()

// ---- exp: double evaluation, one rounding to float ------------------------
// x = k ln2 + r (|r| <= ln2/2, ln2 split in two doubles), e^r by its Taylor
// series to degree 13 (remainder < 5e-18), scaled by 2^k, rounded once.
// Correctly rounded except for arguments within ~1e-16 relative of a float
// rounding boundary.  Host and device evaluate the same IEEE operations.
__host__ __device__ __forceinline__ float expf_sg(float xf) {
  if (xf != xf) return xf;
  if (xf > 100.f) return __builtin_inff();
  if (xf < -110.f) return 0.f;
  const double x = static_cast<double>(xf);
  const double kd = __builtin_rint(x * 1.4426950408889634);
  double r = __builtin_fma(-kd, 6.9314718055994529e-01, x);
  r = __builtin_fma(-kd, 2.3190468138462996e-17, r);
  /* Estrin evaluation (short dependency chain): pairs, then r^2, r^4, r^8. */
  const double r2 = r * r, r4 = r2 * r2, r8 = r4 * r4;
  const double q0 = __builtin_fma(1.0, r, 1.0);
  const double q1 = __builtin_fma(1.0 / 6.0, r, 0.5);
  const double q2 = __builtin_fma(1.0 / 120.0, r, 1.0 / 24.0);
  const double q3 = __builtin_fma(1.0 / 5040.0, r, 1.0 / 720.0);
  const double q4 = __builtin_fma(1.0 / 362880.0, r, 1.0 / 40320.0);
  const double q5 = __builtin_fma(1.0 / 39916800.0, r, 1.0 / 3628800.0);
  const double q6 = __builtin_fma(1.0 / 6227020800.0, r, 1.0 / 479001600.0);
  const double s0 = __builtin_fma(q1, r2, q0), s1 = __builtin_fma(q3, r2, q2), s2 = __builtin_fma(q5, r2, q4);
  const double u0 = __builtin_fma(s1, r4, s0), u1 = __builtin_fma(q6, r4, s2);
  const double p = __builtin_fma(u1, r8, u0);
  const long long k = static_cast<long long>(kd);
  const double scale = __builtin_bit_cast(double, static_cast<unsigned long long>(k + 1023) << 52);
  return static_cast<float>(p * scale);
}

// expf_sg for the router and the window's gate/up kernel: the same
// operations on the same constants (so the same results), with the double
// constants built in scalar registers (sconst) rather than copied into
// vector registers (four exps per lane in the router took 62 such moves,
// and in the gate/up kernel the copies pushed it into spilling), and
// branch-free: out-of-range and NaN arguments evaluate the polynomial at 0
// and are replaced at the end, instead of a divergent region per exp.
__device__ __forceinline__ float expf_sg_kc(float xf) {
#define SG_EXPC(v) SG_SCONST(v)
  const bool nan = !(xf == xf), big = xf > 100.f, small = xf < -110.f;
  const float xs = (nan || big || small) ? 0.f : xf;
  const double x = static_cast<double>(xs);
  const double kd = __builtin_rint(x * SG_EXPC(1.4426950408889634));
  double r = __builtin_fma(-kd, SG_EXPC(6.9314718055994529e-01), x);
  r = __builtin_fma(-kd, SG_EXPC(2.3190468138462996e-17), r);
  /* Estrin evaluation (short dependency chain): pairs, then r^2, r^4, r^8. */
  const double r2 = r * r, r4 = r2 * r2, r8 = r4 * r4;
  const double q0 = __builtin_fma(1.0, r, 1.0);
  const double q1 = __builtin_fma(SG_EXPC(1.0 / 6.0), r, 0.5);
  const double q2 = __builtin_fma(SG_EXPC(1.0 / 120.0), r, SG_EXPC(1.0 / 24.0));
  const double q3 = __builtin_fma(SG_EXPC(1.0 / 5040.0), r, SG_EXPC(1.0 / 720.0));
  const double q4 = __builtin_fma(SG_EXPC(1.0 / 362880.0), r, SG_EXPC(1.0 / 40320.0));
  const double q5 = __builtin_fma(SG_EXPC(1.0 / 39916800.0), r, SG_EXPC(1.0 / 3628800.0));
  const double q6 = __builtin_fma(SG_EXPC(1.0 / 6227020800.0), r, SG_EXPC(1.0 / 479001600.0));
  const double s0 = __builtin_fma(q1, r2, q0), s1 = __builtin_fma(q3, r2, q2), s2 = __builtin_fma(q5, r2, q4);
  const double u0 = __builtin_fma(s1, r4, s0), u1 = __builtin_fma(q6, r4, s2);
  const double p = __builtin_fma(u1, r8, u0);
  const long long k = static_cast<long long>(kd);
  const double scale = __builtin_bit_cast(double, static_cast<unsigned long long>(k + 1023) << 52);
  float y = static_cast<float>(p * scale);
  y = small ? 0.f : y;
  y = big ? __builtin_inff() : y;
  return nan ? xf : y;
}
#undef SG_EXPC

// ---- exp from a 64-entry table: expf_sg's results, in fewer operations ----
// 2^(j/64), j = 0..63: each the double nearest the exact value (evaluated
// to 60 decimal digits).  Kernels that use expf_tab copy it into LDS.
static __constant__ double kExp2Tab64[64] = {
    0x1.0000000000000p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0, 0x1.0874518759bc8p+0,
    0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0, 0x1.11301d0125b51p+0, 0x1.1429aaea92de0p+0,
    0x1.172b83c7d517bp+0, 0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0,
    0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0, 0x1.2d285a6e4030bp+0,
    0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0, 0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0,
    0x1.3dea64c123422p+0, 0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cd0p+0,
    0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0, 0x1.56f4736b527dap+0,
    0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0, 0x1.6247eb03a5585p+0, 0x1.6623882552225p+0,
    0x1.6a09e667f3bcdp+0, 0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0,
    0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0, 0x1.868d99b4492edp+0,
    0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0, 0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e50p+0,
    0x1.9c49182a3f090p+0, 0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0,
    0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0, 0x1.bcc1e904bc1d2p+0,
    0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0, 0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0,
    0x1.d5818dcfba487p+0, 0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0,
    0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4540p+0, 0x1.fa7c1819e90d8p+0};

// e^x for x in [-87, 88] (normal float results): x = (64 k + j) ln2/64 + r
// with |r| <= ln2/128 (k j from rint(x * 64/ln2); ln2/64 split into a
// 39-bit head, so k * head is exact, and a tail), e^x = 2^k * T[j] * e^r
// with e^r to degree 5 (remainder below 2^-54 relative).  The double result
// is within 2^-49 (relative) of e^x.  A lane whose result lies within 2^14
// double ulps (at least 2^-39 relative) of a float rounding midpoint, or
// whose x is outside the range or NaN, takes expf_sg_kc instead.  For every
// other lane the exact e^x is at least 2^-40 from the midpoint, so rounding
// this result gives the correctly rounded float - which expf_sg also returns
// there, its own error being below 2^-50: the two agree bit for bit.
// tab: kExp2Tab64 in LDS.
// The fast evaluation alone; *ok tells whether its rounding is certain.
__device__ __forceinline__ float expf_tab_fast(float xf, const double* tab, bool* ok) {
  const bool in = xf >= -87.f && xf <= 88.f;
  const double x = in ? static_cast<double>(xf) : 0.0;
  const double kd = __builtin_rint(x * SG_SCONST(0x1.71547652b82fep+6));  // 64 / ln2
  double r = __builtin_fma(-kd, SG_SCONST(0x1.62e42fefa4000p-7), x);     // ln2/64, head
  r = __builtin_fma(-kd, SG_SCONST(-0x1.8432a1b0e2634p-49), r);           // ln2/64, tail
  double p = __builtin_fma(SG_SCONST(1.0 / 120.0), r, SG_SCONST(1.0 / 24.0));
  p = __builtin_fma(p, r, SG_SCONST(1.0 / 6.0));
  p = __builtin_fma(p, r, 0.5);
  p = __builtin_fma(p, r, 1.0);
  p = __builtin_fma(p, r, 1.0);
  const int ki = static_cast<int>(kd);
  const double scale =
      __builtin_bit_cast(double, static_cast<unsigned long long>((ki >> 6) + 1023) << 52);
  const double y = tab[ki & 63] * p * scale;
  // the 29 double fraction bits that rounding to float drops: the midpoint
  // between two floats is 0x10000000
  const uint32_t lo = static_cast<uint32_t>(__builtin_bit_cast(unsigned long long, y)) & 0x1FFFFFFFu;
  *ok = in && (lo - (0x10000000u - 0x4000u)) > 0x8000u;
  return static_cast<float>(y);
}

__device__ __forceinline__ float expf_tab(float xf, const double* tab) {
  bool ok;
  float res = expf_tab_fast(xf, tab, &ok);
  if (!ok) res = expf_sg_kc(xf);
  return res;
}

// N SiLU products at once: the fast exps are independent chains that the
// compiler interleaves, and the exact fallback runs only if some lane needs
// it for some element.
template <int N>
__device__ __forceinline__ void silu_mul_tab_n(const float (&g)[N], const float (&u)[N],
                                               float (&h)[N], const double* tab) {
  float e[N];
  bool ok[N], all = true;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    e[i] = expf_tab_fast(-g[i], tab, &ok[i]);
    all = all && ok[i];
  }
  if (!all) {
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (!ok[i]) e[i] = expf_sg_kc(-g[i]);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) h[i] = g[i] / (1.f + e[i]) * u[i];
}

// silu_mul with expf_tab (tab: kExp2Tab64 in LDS): the same bits
__device__ __forceinline__ float silu_mul_tab(float g, float u, const double* tab) {
  return g / (1.f + expf_tab(-g, tab)) * u;
}

// SiLU(g) * u in the CPU chain's operation order (q4_avx2.cpp:187-191).
__device__ __forceinline__ float silu_mul(float g, float u) {
  return g / (1.f + expf_sg(-g)) * u;
}
// silu_mul with expf_sg_kc
__device__ __forceinline__ float silu_mul_kc(float g, float u) {
  return g / (1.f + expf_sg_kc(-g)) * u;
}


// fp16 bits <-> fp32; the conversion to fp16 rounds the fp32 value to
// nearest even (__float2half of the reference's sth(), moe.cu:12-14).
__device__ __forceinline__ float f16v(uint16_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, b));
}
__device__ __forceinline__ uint16_t f16b(float v) {
  // v is materialized as an fp32 value first: otherwise the compiler fuses
  // the producing multiply or fma with the conversion into one mixed-
  // precision fma (v_fma_mix*_f16), which rounds once instead of twice and
  // adds +0 to a -0 product.
  asm("" : "+v"(v));
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

// v rounded to fp16 and read back as fp32 (a value stored in an fp16 buffer)
__device__ __forceinline__ float f16r(float v) { return f16v(f16b(v)); }

// sigmoid(g) = 1 / (1 + exp(-g)), the shared-expert gate
// (moe.cu:289, norm_rotary.cu:182).
__host__ __device__ __forceinline__ float sigmoid_sg(float g) {
  return 1.f / (1.f + expf_sg(-g));
}

// fp32 weight row . activation row in the order of the reference's fp32
// GEMV (gemv_f32_out_kernel, q4_k.cu:133-149; the shared-expert gate and
// router logits): lane l of 32 accumulates elements l, l+32, l+64, ... as
// acc = fma(w, x, acc) (nvcc contracts `acc += w * x`), then a shfl_down
// tree over offsets 16, 8, 4, 2, 1.  Run by 32 lanes together (l = lane
// & 31, all 32 active); the row value is in lane l = 0.  xv(i) gives x[i]
// as fp32.
template <typename XV>
__device__ __forceinline__ float rowdot_f32_lanes32(const float* __restrict__ w, XV xv, int k,
                                                    int l) {
  float acc = 0.f;
#pragma unroll 8
  for (int i = l; i < k; i += 32) acc = __builtin_fmaf(w[i], xv(i), acc);
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) acc += __shfl_down(acc, off, 32);
  return acc;
}

// ---- Q8_K code of one scaled value ----------------------------------------
// round-half-even, then the x86 float->int conversion the reference runs on
// (NaN and out-of-range -> INT_MIN), then the +-127 clamp.
__device__ __forceinline__ int q8_code(float v) {
  const float r = __builtin_rintf(v);
  int q;
  if (!(r == r) || r >= 2147483648.0f || r < -2147483648.0f)
    q = INT32_MIN;
  else
    q = static_cast<int>(r);
  return q > 127 ? 127 : (q < -127 ? -127 : q);
}

// ---- wave64 helpers ---------------------------------------------------------
// DPP lane exchanges within a 16-lane row: xor 1, xor 2 (quad_perm), the
// 8-lane and 16-lane mirrors.  Applied in that order they reduce a row with
// any associative, commutative combine; the four row results are then read
// with v_readlane and combined in a fixed order, so every lane returns the
// same value regardless of how the reduction is scheduled.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, v)));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

__device__ __forceinline__ float readlane_f(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// Maximum over the wave (NaN ignored as by fmaxf), same value in every lane.
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_f<kDppXor1>(v));
  v = fmaxf(v, dpp_f<kDppXor2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppMirror>(v));
  return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)),
               fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

// Maximum of an int over the wave, same value in every lane.
__device__ __forceinline__ int wave_max_i32(int v) {
  v = max(v, dpp_i<kDppXor1>(v));
  v = max(v, dpp_i<kDppXor2>(v));
  v = max(v, dpp_i<kDppHalfMirror>(v));
  v = max(v, dpp_i<kDppMirror>(v));
  return max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// Sum over each aligned group of 8 lanes (every lane of the group gets it).
__device__ __forceinline__ int sum8_dpp(int v) {
  v += dpp_i<kDppXor1>(v);
  v += dpp_i<kDppXor2>(v);
  v += dpp_i<kDppHalfMirror>(v);
  return v;
}

// (value, index) argmax: a valid index (>= 0) beats an invalid one, then the
// larger value, then the lower index.  Total order, so the result is exact.
__device__ __forceinline__ void argmax_take(float& bv, int& bi, float ov, int oi) {
  if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) {
    bv = ov;
    bi = oi;
  }
}
template <int CTRL>
__device__ __forceinline__ void argmax_step(float& bv, int& bi) {
  argmax_take(bv, bi, dpp_f<CTRL>(bv), dpp_i<CTRL>(bi));
}
__device__ __forceinline__ void wave_argmax_dpp(float& bv, int& bi) {
  argmax_step<kDppXor1>(bv, bi);
  argmax_step<kDppXor2>(bv, bi);
  argmax_step<kDppHalfMirror>(bv, bi);
  argmax_step<kDppMirror>(bv, bi);
  float v = readlane_f(bv, 0);
  int i = __builtin_amdgcn_readlane(bi, 0);
#pragma unroll
  for (int r = 16; r < 64; r += 16)
    argmax_take(v, i, readlane_f(bv, r), __builtin_amdgcn_readlane(bi, r));
  bv = v;
  bi = i;
}


// Quantize one 256-value block with the calling wave; `lane` in 0..63.
// v[0..3] are the lane's values 4*lane..4*lane+3 of the block.
__device__ __forceinline__ void quantize_block_wave(const float v[4], unsigned char* ob, int lane) {
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  amax = fmaxf(wave_max_dpp(amax), 1e-30f);
  const float d = amax / 127.f;
  const float id = d > 0 ? 1.f / d : 0.f;
  int q[4];
  uint32_t packed = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    q[i] = q8_code(v[i] * id);
    packed |= (static_cast<uint32_t>(q[i]) & 0xFFu) << (8 * i);
  }
  const int s = sum8_dpp(q[0] + q[1] + q[2] + q[3]);
  *reinterpret_cast<uint32_t*>(ob + 4 + 4 * lane) = packed;
  if (lane == 0) *reinterpret_cast<float*>(ob) = d;
  if ((lane & 7) == 0) *reinterpret_cast<int16_t*>(ob + 260 + 2 * (lane >> 3)) = static_cast<int16_t>(s);
}


// ---- Q8_K activations staged in LDS ------------------------------------------
// Each 276-B block becomes 80 dwords: [0,64) qs words, [64] d, [65,73) the
// eight bsums as floats (exact), rest padding; stride 320 B keeps the qs
// words 16-B aligned for ds_read_b128.
constexpr int kXStride = 80;

__device__ __forceinline__ void stage_q8k(const unsigned char* __restrict__ xq, int n_blocks,
                                          uint32_t* lds, int tid, int nthreads) {
  const uint32_t* src = reinterpret_cast<const uint32_t*>(xq);  // 276 B blocks are 4-B aligned
  for (int j = tid; j < n_blocks * 69; j += nthreads) {
    const int b = j / 69, w = j - b * 69;
    const uint32_t v = src[j];
    uint32_t* dst = lds + b * kXStride;
    if (w == 0) {
      dst[64] = v;
    } else if (w <= 64) {
      dst[w - 1] = v;
    } else {
      const int p = 2 * (w - 65);
      dst[65 + p] = __builtin_bit_cast(uint32_t, static_cast<float>(static_cast<int16_t>(v & 0xFFFFu)));
      dst[66 + p] = __builtin_bit_cast(uint32_t, static_cast<float>(static_cast<int16_t>(v >> 16)));
    }
  }
}

// Read one staged block into registers.
__device__ __forceinline__ void load_x_regs(const uint32_t* lds_blk, int32_t* xq64, float& xd,
                                            float* bsf) {
  const u32x4* p = reinterpret_cast<const u32x4*>(lds_blk);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const u32x4 v = p[i];
    xq64[4 * i + 0] = static_cast<int32_t>(v.x);
    xq64[4 * i + 1] = static_cast<int32_t>(v.y);
    xq64[4 * i + 2] = static_cast<int32_t>(v.z);
    xq64[4 * i + 3] = static_cast<int32_t>(v.w);
  }
  xd = __builtin_bit_cast(float, lds_blk[64]);
#pragma unroll
  for (int s = 0; s < 8; ++s) bsf[s] = __builtin_bit_cast(float, lds_blk[65 + s]);
}

// Sum the per-block partial sums of a row in block order
// (acc = 0; acc += s_0; ...; acc += s_{nb-1}), the reference's row
// accumulation (q4_avx2.cpp:130-143).  Lane `blk` of the row holds s_blk;
// each step moves the running sum one lane up with a DPP wave shift, so the
// complete row sum ends in the lane with blk == nb - 1.  All lanes active.
constexpr int kDppWaveShr1 = 0x138;
__device__ __forceinline__ float row_sum_last(float s, int blk, int nb) {
  float acc = 0.f + s;
  for (int j = 1; j < nb; ++j) {
    const float prev = dpp_f<kDppWaveShr1>(acc);
    if (blk == j) acc = prev + s;
  }
  return acc;
}

// Quantize one 256-value block with the calling wave straight into the LDS
// staging layout (qs words, d, float bsums); same arithmetic as
// quantize_block_wave.
__device__ __forceinline__ void quantize_block_wave_lds(const float v[4], uint32_t* dst,
                                                        int lane) {
  float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  amax = fmaxf(wave_max_dpp(amax), 1e-30f);
  const float d = amax / 127.f;
  const float id = d > 0 ? 1.f / d : 0.f;
  uint32_t packed = 0;
  int qsum = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = q8_code(v[i] * id);
    qsum += q;
    packed |= (static_cast<uint32_t>(q) & 0xFFu) << (8 * i);
  }
  const int s = sum8_dpp(qsum);
  dst[lane] = packed;
  if (lane == 0) dst[64] = __builtin_bit_cast(uint32_t, d);
  if ((lane & 7) == 0) dst[65 + (lane >> 3)] = __builtin_bit_cast(uint32_t, static_cast<float>(s));
}

// N blocks at once with the calling wave (same arithmetic as
// quantize_block_wave_lds, chains interleaved for latency); blocks b >=
// n_act are computed but not stored.  v[b][0..3] = the lane's 4 values of
// block b.
template <int N>
__device__ __forceinline__ void quantize_n_lds(const float (&v)[N][4], uint32_t* const (&dst)[N],
                                               int n_act, int lane) {
  float amax[N], d[N], id[N];
#pragma unroll
  for (int b = 0; b < N; ++b)
    amax[b] = fmaxf(fmaxf(fabsf(v[b][0]), fabsf(v[b][1])), fmaxf(fabsf(v[b][2]), fabsf(v[b][3])));
#pragma unroll
  for (int b = 0; b < N; ++b) amax[b] = fmaxf(wave_max_dpp(amax[b]), 1e-30f);
#pragma unroll
  for (int b = 0; b < N; ++b) d[b] = amax[b] / 127.f;
#pragma unroll
  for (int b = 0; b < N; ++b) id[b] = d[b] > 0 ? 1.f / d[b] : 0.f;
  uint32_t packed[N];
  int qsum[N];
#pragma unroll
  for (int b = 0; b < N; ++b) {
    packed[b] = 0;
    qsum[b] = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = q8_code(v[b][i] * id[b]);
      qsum[b] += q;
      packed[b] |= (static_cast<uint32_t>(q) & 0xFFu) << (8 * i);
    }
  }
#pragma unroll
  for (int b = 0; b < N; ++b) qsum[b] = sum8_dpp(qsum[b]);
#pragma unroll
  for (int b = 0; b < N; ++b) {
    if (b < n_act) {
      dst[b][lane] = packed[b];
      if (lane == 0) dst[b][64] = __builtin_bit_cast(uint32_t, d[b]);
      if ((lane & 7) == 0)
        dst[b][65 + (lane >> 3)] = __builtin_bit_cast(uint32_t, static_cast<float>(qsum[b]));
    }
  }
}

// One Q8_K block per 16-lane DPP row: lane l holds values 16*(l & 15) ..
// 16*(l & 15) + 15 of its row's block in v[].  Same arithmetic as
// quantize_n_lds (amax over the block, d = amax / 127, q = q8_code(v / d
// by the reciprocal), bsums over 32 values), with the block's reductions
// inside one DPP row: no cross-row steps and no lane reads.  Writes the
// block to dst (LDS, kXStride layout) when `active`.
__device__ __forceinline__ void quantize_row16_lds(const float (&v)[16], uint32_t* dst, bool active,
                                                   int lane) {
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
  qsum += dpp_i<kDppXor1>(qsum);  // the 32 values of a bsum: this lane and its neighbour
  if (active) {
    const int r = lane & 15;
    *reinterpret_cast<u32x4*>(dst + 4 * r) = (u32x4){packed[0], packed[1], packed[2], packed[3]};
    if (r == 0) dst[64] = __builtin_bit_cast(uint32_t, d);
    if ((r & 1) == 0) dst[65 + (r >> 1)] = __builtin_bit_cast(uint32_t, static_cast<float>(qsum));
  }
}

// Stage the Q8_K rows of n tokens (token ids in `tok`, nb blocks per row)
// into LDS: token j's block b goes to lds + (j*nb + b)*kXStride.
__device__ __forceinline__ void stage_q8k_rows(const unsigned char* __restrict__ xq,
                                               const int* tok, int n, int nb, uint32_t* lds,
                                               int tid, int nthreads) {
  const int per = nb * 69;
  for (int j = tid; j < n * per; j += nthreads) {
    const int r = j / per, jj = j - r * per;
    const int b = jj / 69, w = jj - b * 69;
    const uint32_t v =
        reinterpret_cast<const uint32_t*>(xq + static_cast<long long>(tok[r]) * nb * kQ8Bytes)[jj];
    uint32_t* dst = lds + (r * nb + b) * kXStride;
    if (w == 0) {
      dst[64] = v;
    } else if (w <= 64) {
      dst[w - 1] = v;
    } else {
      const int p = 2 * (w - 65);
      dst[65 + p] = __builtin_bit_cast(uint32_t, static_cast<float>(static_cast<int16_t>(v & 0xFFFFu)));
      dst[66 + p] = __builtin_bit_cast(uint32_t, static_cast<float>(static_cast<int16_t>(v >> 16)));
    }
  }
}

}  // namespace sg
