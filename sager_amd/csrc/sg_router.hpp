// sg_router.hpp - top-k selection building blocks for the fused MoE layer.
//
// Selection order everywhere: value descending, then index ascending - the
// order the reference's k rounds of first-strict-max produce
// (moe.cu:46-76).  A candidate is a 64-bit key, high word = the value mapped
// to an unsigned int that orders like the float (NaN lowest), low word =
// ~index, so "larger key" is exactly "earlier in the selection" and keys are
// distinct.
#pragma once

#include "sg_common.hpp"

namespace sg {

__device__ __forceinline__ uint64_t sel_key(float v, int i) {
  // -0 keys as +0: the two compare equal, so the lower index goes first
  const uint32_t b = v == 0.f ? 0u : __builtin_bit_cast(uint32_t, v);
  const uint32_t o = (v != v) ? 0u : ((b & 0x80000000u) ? ~b : (b | 0x80000000u));
  return (static_cast<uint64_t>(o) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(i));
}
__device__ __forceinline__ int sel_idx(uint64_t key) {
  return static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(key));
}
// The value of a key made from a non-NaN float (-0 comes back as +0).
__device__ __forceinline__ float sel_val(uint64_t key) {
  const uint32_t o = static_cast<uint32_t>(key >> 32);
  return __builtin_bit_cast(float, (o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}

// Largest 32-bit value over the wave, the same in every lane (DPP within
// each 16-lane row, then the four row maxima).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, static_cast<uint32_t>(dpp_i<kDppXor1>(static_cast<int>(v))));
  v = max(v, static_cast<uint32_t>(dpp_i<kDppXor2>(static_cast<int>(v))));
  v = max(v, static_cast<uint32_t>(dpp_i<kDppHalfMirror>(static_cast<int>(v))));
  v = max(v, static_cast<uint32_t>(dpp_i<kDppMirror>(static_cast<int>(v))));
  const uint32_t a = __builtin_amdgcn_readlane(static_cast<int>(v), 0);
  const uint32_t b = __builtin_amdgcn_readlane(static_cast<int>(v), 16);
  const uint32_t c = __builtin_amdgcn_readlane(static_cast<int>(v), 32);
  const uint32_t d = __builtin_amdgcn_readlane(static_cast<int>(v), 48);
  return max(max(a, b), max(c, d));
}

// Largest 64-bit key over the wave, the same in every lane: DPP exchanges
// within each 16-lane row, then the four row maxima.  No branches.
__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const int lo = dpp_i<CTRL>(static_cast<int>(static_cast<uint32_t>(v)));
  const int hi = dpp_i<CTRL>(static_cast<int>(static_cast<uint32_t>(v >> 32)));
  return (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo);
}
__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v)), l);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v >> 32)), l);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = max_u64(v, dpp_u64<kDppXor1>(v));
  v = max_u64(v, dpp_u64<kDppXor2>(v));
  v = max_u64(v, dpp_u64<kDppHalfMirror>(v));
  v = max_u64(v, dpp_u64<kDppMirror>(v));
  return max_u64(max_u64(readlane_u64(v, 0), readlane_u64(v, 16)),
                 max_u64(readlane_u64(v, 32), readlane_u64(v, 48)));
}

// Top-m keys (m <= 33) of keys[0..n) for a team of nthr threads (thread tt).
// Two levels: the top m of every 64-key group (rank by direct comparison
// inside the group), then the top m of those candidates.  Results in
// top[0..m) in selection order (0 = missing).  cand holds ceil(n/64)*m keys.
// Every thread of the workgroup must call this together: it contains three
// barriers.
__device__ void team_top_m(const uint64_t* keys, int n, int m, uint64_t* cand, uint64_t* top,
                           int tt, int nthr) {
  const int ng = (n + 63) >> 6;
  for (int i = tt; i < ng * m; i += nthr) cand[i] = 0;
  for (int i = tt; i < m; i += nthr) top[i] = 0;
  bar();
  for (int i = tt; i < n; i += nthr) {
    const uint64_t ki = keys[i];
    const int g0 = i & ~63, g1 = min(n, g0 + 64);
    int r = 0;
    for (int j = g0; j < g1; ++j) r += keys[j] > ki;
    if (r < m && ki != 0) cand[(g0 >> 6) * m + r] = ki;
  }
  bar();
  const int nc = ng * m;
  for (int c = tt; c < nc; c += nthr) {
    const uint64_t kc = cand[c];
    if (kc == 0) continue;
    int r = 0;
    for (int d = 0; d < nc; ++d) r += cand[d] > kc;
    if (r < m) top[r] = kc;
  }
  bar();
}

// Maximum of v over a team of nw waves (fmaxf semantics); `red` holds nw
// floats of team scratch.  Contains one workgroup barrier.
__device__ __forceinline__ float team_max(float v, float* red, int wave_in_team, int nw, int lane) {
  v = wave_max_dpp(v);
  if (lane == 0) red[wave_in_team] = v;
  bar();
  float m = red[0];
  for (int w = 1; w < nw; ++w) m = fmaxf(m, red[w]);
  return m;
}

// Serial sum x[0] + x[1] + ... + x[n-1] in index order by ONE thread, from
// LDS padded with +0 to a multiple of 32 (adding +0 changes nothing).
__device__ __forceinline__ float serial_sum(const float* x, int n32) {
  const float4* x4 = reinterpret_cast<const float4*>(x);
  float z = 0.f;
  for (int i = 0; i < n32 / 4; i += 8) {
    float4 v[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = x4[i + q];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      z += v[q].x;
      z += v[q].y;
      z += v[q].z;
      z += v[q].w;
    }
  }
  return z;
}

// ---- router: one wave per token row ----------------------------------------
// Softmax with the max and the normalizer sum taken in index order, k rounds
// of (value desc, index asc) argmax over non-NaN probabilities, degenerate
// rounds pick kk % n_expert, weights renormalized by their k-order sum,
// slot k = shared_w.  oi/ow may point to LDS or global memory; lane 0
// writes them.  All 64 lanes must be active.  PL = experts per lane
// (n_expert <= 64 PL).
//
// The model shape (256 experts, top-8, PL = 4) first tries a shorter chain:
// the k + 1 selection rounds run on the exps e_i, interleaved with the
// serial normalizer (every lane adds the same values, so no lane waits for
// another), since p_i = e_i / z orders like e_i.  Let c_0 .. c_k be the
// picks in e order.  If no two consecutive ones have equal probabilities,
// then p(c_0) > ... > p(c_k) and every other expert has p <= p(c_k), so the
// reference's k picks are c_0 .. c_(k-1) in that order.  An equality (from
// equal logits, or from the division's rounding), a NaN normalizer or a
// degenerate round among the first k falls back to the exact rounds below
// with the same z.
template <int PL>
__device__ __forceinline__ void router_wave(const float* __restrict__ lg, int n_expert, int k, float shared_w,
                            int* oi, float* ow, float* ev, int lane, bool shared_slot = true) {
  constexpr int kPerLane = PL;
  float p[kPerLane];
  float mx = -1e30f;
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) {
    const int i = lane + 64 * j;
    const float v = lg[i < n_expert ? i : n_expert - 1];  // no branch: one wait for all
    p[j] = i < n_expert ? v : 0.f;
    if (i < n_expert) mx = fmaxf(mx, p[j]);
  }
  mx = wave_max_dpp(mx);
  const int e32 = (n_expert + 31) & ~31;
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) {
    const int i = lane + 64 * j;
    if (i < n_expert) p[j] = expf_sg_kc(p[j] - mx);
    if (i < e32) ev[i] = i < n_expert ? p[j] : 0.f;  // +0 padding leaves the sum unchanged
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float z = 0.f;
  bool have_z = false;
  if constexpr (PL == 4) {
    constexpr int kE = 256, kK = 8, kR = kK + 1, kNb = kE / 32;
    if (n_expert == kE && k == kK) {
      uint32_t he[kPerLane];
#pragma unroll
      for (int j = 0; j < kPerLane; ++j)
        he[j] = p[j] == p[j] ? static_cast<uint32_t>(sel_key(p[j], lane + 64 * j) >> 32) : 0u;
      const float4* x4 = reinterpret_cast<const float4*>(ev);
      int my_i = 0;
      float my_e = -1.f;
      bool degen = false;
#pragma unroll
      for (int r = 0; r < (kR > kNb ? kR : kNb); ++r) {
        if (r < kNb) {  // 32 more terms of the normalizer, in index order
          float4 v[8];
#pragma unroll
          for (int q = 0; q < 8; ++q) v[q] = x4[8 * r + q];
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            z += v[q].x;
            z += v[q].y;
            z += v[q].z;
            z += v[q].w;
          }
        }
        if (r < kR) {  // selection round r on the exps
          uint32_t h = he[0];
#pragma unroll
          for (int j = 1; j < kPerLane; ++j) h = max(h, he[j]);
          h = wave_max_u32(h);
          int jb = kPerLane;
          uint64_t mb = 0;
#pragma unroll
          for (int j = kPerLane - 1; j >= 0; --j) {
            const uint64_t m = __ballot(he[j] == h);
            jb = m ? j : jb;
            mb = m ? m : mb;
          }
          const bool none = h == 0u;
          const int bi = none ? r % kE : 64 * jb + __builtin_ctzll(mb | (1ull << 63));
          const float be = none ? -1.f : sel_val(static_cast<uint64_t>(h) << 32);
          degen = degen || (none && r < kK);
#pragma unroll
          for (int j = 0; j < kPerLane; ++j) he[j] = lane + 64 * j == bi ? 0u : he[j];
          my_i = lane == r ? bi : my_i;
          my_e = lane == r ? be : my_e;
        }
      }
      have_z = true;
      // p of the picks (lane r), and the check of consecutive picks
      const float pp = my_e < 0.f ? -1.f : my_e / z;
      const float pn = __shfl_down(pp, 1, 64);
      const bool tie = lane < kK && pp == pn;
      if (z == z && !degen && __ballot(tie) == 0ull) {
        float wsum = 0.f;
#pragma unroll
        for (int r = 0; r < kK; ++r) wsum += readlane_f(pp, r);
        if (lane < kK) {
          oi[lane] = my_i;
          ow[lane] = wsum > 0.f ? pp / wsum : pp;
        }
        if (lane == 0 && shared_slot) ow[k] = shared_w;
        return;
      }
    }
  }
  if (!have_z) {
    // normalizer z = (((0 + e_0) + e_1) + ...) in index order, by one lane
    z = lane == 0 ? serial_sum(ev, e32) : 0.f;
    z = readlane_f(z, 0);
  }
#pragma unroll
  for (int j = 0; j < kPerLane; ++j)
    if (lane + 64 * j < n_expert) p[j] = p[j] / z;

  // k rounds of first-strict-max over the non-NaN probabilities, without
  // branches: each value is held as its order-preserving 32-bit image (0 =
  // not selectable: NaN, past n_expert or already taken; every other
  // probability maps above 0x7FFFFFFF).  A round takes the wave maximum of
  // the images, then among the experts holding it the lowest index (the
  // lowest j, then the lowest lane, since index = lane + 64 j).  Lane kk
  // keeps round kk's pick.
  uint32_t hv[kPerLane];
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) {
    const int i = lane + 64 * j;
    hv[j] = (i < n_expert && p[j] == p[j]) ? static_cast<uint32_t>(sel_key(p[j], i) >> 32) : 0u;
  }
  float wsum = 0.f;
  int my_i = 0;
  float my_w = 0.f;
  for (int kk = 0; kk < k; ++kk) {
    uint32_t h = hv[0];
#pragma unroll
    for (int j = 1; j < kPerLane; ++j) h = max(h, hv[j]);
    h = wave_max_u32(h);
    int bi = kk % n_expert;  // nothing selectable: the degenerate pick
    float bv = -1.f;
    if (h != 0u) {
      int jb = kPerLane;
      uint64_t mb = 0;
#pragma unroll
      for (int j = kPerLane - 1; j >= 0; --j) {
        const uint64_t m = __ballot(hv[j] == h);
        if (m) {
          jb = j;
          mb = m;
        }
      }
      bi = 64 * jb + __builtin_ctzll(mb);
      bv = sel_val(static_cast<uint64_t>(h) << 32);
    }
#pragma unroll
    for (int j = 0; j < kPerLane; ++j)
      if (lane + 64 * j == bi) hv[j] = 0u;
    if (lane == kk) {
      my_i = bi;
      my_w = bv;
    }
    wsum += bv;
  }
  if (lane < k) {
    oi[lane] = my_i;
    ow[lane] = wsum > 0.f ? my_w / wsum : my_w;
  }
  if (lane == 0 && shared_slot) ow[k] = shared_w;
}

}  // namespace sg
