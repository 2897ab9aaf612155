// sg_layer.hip - one fused MoE layer (decode step or verify window) on gfx950.
//
// Two launches per layer, on one stream:
//
//   front  grid (row chunks of 16, groups + 1): every routed workgroup finds
//          its expert from the top-k by logit, starts streaming that
//          expert's gate and up rows, and meanwhile derives the exact
//          selection from the probabilities (a different expert only on a
//          probability collision - then it streams the right one); then
//          h = SiLU(g) * u for every token of its group.  The last row of the
//          grid is one publisher workgroup that writes idx, weight and the
//          expert-major plan for the back kernel.
//   back   grid (row chunks of hidden/256 rows): every group's down rows for
//          the chunk, the Q8_K of h done in the workgroup, and the combine of
//          the chunk for every token in slot order - all inside one
//          workgroup, so there are no cross-workgroup counters or fences.
//
// Weights stream from HBM into LDS with global_load_lds_dwordx4 (1 KB of
// consecutive memory per instruction) and are read back per lane at the
// 144-B super-block stride.  A group is the shared expert (group 0, tokens
// 0..T-1 in slot k) or one distinct routed expert (ascending id) with its
// (token, slot) routes; an expert shared by several tokens is streamed once.
// Loads that do not depend on routing (x, h, residual) are issued at kernel
// start so their latency overlaps the routing and the plan load.
//
// Stage order and semantics: Session::moe_dispatch_device
// (session.cpp:2482-3030); router moe.cu:25-85 / 165-234; dispatch plan
// moe.cu:366-444 (made deterministic); combine moe.cu:265-280; expert chain
// q4_avx2.cpp:175-196.
#include <mutex>

#include "sg_common.hpp"
#include "sg_router.hpp"

namespace sg {

constexpr int kLMaxExperts = 1024;
constexpr int kLMaxK = 32;
constexpr int kLMaxTokens = 16;
constexpr int kMaxEpt = 16;        // experts per routing thread (1-wave teams, E = 1024)

__host__ __device__ constexpr inline int pow2_ceil(int n) {
  int l = 1;
  while (l < n) l <<= 1;
  return l;
}

// ---- workspace ------------------------------------------------------------------

struct LayerPlan {
  int* meta;    // [0] groups, [1] has_shared, [2] valid routes
  int* off;     // [gmax+1] entry offsets per group
  int* expert;  // [gmax] expert id per group, -1 = shared expert
  int* tok;     // [emax] entry token
  int* slot;    // [emax] entry slot
  unsigned long long* wdown;  // [gmax] down matrix of the group, 0 = absent expert
  unsigned long long* wgate;  // [gmax] gate matrix of the group, 0 = absent expert
  unsigned long long* wup;    // [gmax] up matrix of the group, 0 = absent expert
};

struct LayerWs {
  size_t meta, off, expert, tok, slot, wdown, wgate, wup, sgate, h, xq, total;
  int gmax, emax;
};

static size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

static LayerWs layer_ws(int T, int hidden, int n_ff, int E, int k) {
  LayerWs w{};
  w.gmax = (T * k < E ? T * k : E) + 1;
  w.emax = T * k + T;
  size_t o = 0;
  w.meta = o;   o = align256(o + 4 * sizeof(int));
  w.off = o;    o = align256(o + (w.gmax + 1) * sizeof(int));
  w.expert = o; o = align256(o + w.gmax * sizeof(int));
  w.tok = o;    o = align256(o + w.emax * sizeof(int));
  w.slot = o;   o = align256(o + w.emax * sizeof(int));
  w.wdown = o;  o = align256(o + w.gmax * sizeof(unsigned long long));
  w.wgate = o;  o = align256(o + w.gmax * sizeof(unsigned long long));
  w.wup = o;    o = align256(o + w.gmax * sizeof(unsigned long long));
  w.sgate = o;  o = align256(o + static_cast<size_t>(T) * sizeof(float));
  w.h = o;      o = align256(o + static_cast<size_t>(T) * (k + 1) * n_ff * sizeof(float));
  // several tokens: Q8_K of x in the LDS block layout (written by the routing
  // launch, read by the gate/up launch)
  w.xq = o;     o = align256(o + (T > 1 ? static_cast<size_t>(T) * (hidden / kQK) * kXStride * 4 : 0));
  w.total = o;
  return w;
}

struct FrontLds {
  int nteams, tw, TT, ept, m, e32, ncp;
  int tabg, tabu, tabd, lv, ev, cand, top, red, zs, spec, ridx, rw, re, rfirst, poff, pexp,
      ptok, pslot, ctrl, kw, xs, total;
};

struct LayerArgs {
  const sg_block_q4k* const* tab_gate;
  const sg_block_q4k* const* tab_up;
  const sg_block_q4k* const* tab_down;
  const sg_block_q4k* sh_gate;
  const sg_block_q4k* sh_up;
  const sg_block_q4k* sh_down;
  const float* sh_gate_w;  // fp32 [hidden] shared-expert gate row, or null
  const float* x;  // fp32 [T][hidden] (or null: x16 / xq_in below)
  const float* logits;
  const float* residual;
  float* out;
  int* idx;
  float* weight;
  LayerPlan plan;
  float* h;
  float* sgate;  // [T] sigmoid(sh_gate_w . x[t]) when sh_gate_w is set
  uint32_t* xq;  // T > 1: Q8_K of x, kXStride words per block (token-major)
  int T, hidden, n_ff, n_expert, k, has_shared, gmax, emax;
  float shared_w;
  int back_rows, back_lrow;  // rows per back workgroup, lanes per row there
  int back_bufs;             // back waves with a down-row buffer (8, or 4 when LDS is short)
  int publish_only;          // front launch of the publisher alone (the routing launch)
  FrontLds front_routed, front_shared;  // front LDS layouts (routing groups, shared group)
  // the session's fp16 buffers (after the fields above, whose layout the
  // fp32 kernels read): fp16 x16 instead of x, or (with either, or alone
  // without a shared gate) xq_in, a Q8_K of x made by the caller and used as
  // is; fp16 res16 / out16 instead of residual / out, with the slot outputs
  // stored as fp16 and combined as moe_combine_batched_f16
  const uint16_t* x16;
  const unsigned char* xq_in;
  const uint16_t* res16;
  uint16_t* out16;
};

// ---- front kernel LDS layout (dwords) -----------------------------------------------
// Routing runs in teams: one team of 4 waves per token for T = 1, two teams
// of 2 waves for T = 2, four one-wave teams otherwise (tokens in passes).

__host__ __device__ constexpr FrontLds front_lds(int T, int nbh, int E, int k, bool routed) {
  FrontLds L{};
  L.nteams = T == 1 ? 1 : (T == 2 ? 2 : 4);
  L.tw = 4 / L.nteams;
  L.TT = 64 * L.tw;
  L.ept = (E + L.TT - 1) / L.TT;
  L.m = k + 1;
  L.e32 = (E + 31) & ~31;
  L.ncp = (L.tw * L.m + 3) & ~3;  // a team's candidates: m per wave
  const int gmax = (T * k < E ? T * k : E) + 1;
  int o = 0;
  auto take = [&](int words) {
    o = (o + 3) & ~3;  // 16-B alignment for every array
    const int at = o;
    o += words;
    return at;
  };
  L.xs = take(T * nbh * kXStride);
  if (routed) {
    L.tabg = take(E * 2);
    L.tabu = take(E * 2);
    L.tabd = take(E * 2);
    L.lv = take(L.nteams * L.e32);
    L.ev = take(4 * L.e32);  // a team's (one token) or a wave's (routing launch) exps
    L.cand = take(L.nteams * L.ncp * 2);
    L.top = take(L.nteams * L.m * 2);
    L.red = take(L.nteams * 4);
    L.zs = take(L.nteams);
    L.spec = take(T * L.m);
    L.ridx = take(T * k);
    L.rw = take(T * (k + 1));
    L.re = take(T * k);
    L.rfirst = take(T * k);
    L.poff = take(gmax + 1);
    L.pexp = take(gmax);
    L.ptok = take(T * k + T);
    L.pslot = take(T * k + T);
    L.ctrl = take(8 + T * k);
    L.kw = take(4 * 64 + 4 * 128);  // team_select, one key per thread: value words, then keys
  }
  L.total = o;
  return L;
}

// rank among n (multiple of 4) keys, 16-B aligned.
__device__ __forceinline__ int rank_n(const uint64_t* c, int n, uint64_t key) {
  const u32x4* p = reinterpret_cast<const u32x4*>(c);
  int r = 0;
  int q = 0;
  for (; q + 8 <= n / 2; q += 8) {  // eight reads in flight
    u32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = p[q + u];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const uint64_t a = (static_cast<uint64_t>(v[u].y) << 32) | v[u].x;
      const uint64_t b = (static_cast<uint64_t>(v[u].w) << 32) | v[u].z;
      r += (a > key) + (b > key);
    }
  }
  for (; q < n / 2; ++q) {
    const u32x4 v = p[q];
    const uint64_t a = (static_cast<uint64_t>(v.y) << 32) | v.x;
    const uint64_t b = (static_cast<uint64_t>(v.w) << 32) | v.z;
    r += (a > key) + (b > key);
  }
  return r;
}

constexpr int kWaves4 = 4;  // waves of a front workgroup

// Top-m selection of a team (tw waves) over the keys kr[] its threads hold
// (0 = no key; keys are otherwise distinct).  Stage 1, per wave: the wave's
// m largest keys go to cand[wave * m ...) (zero-padded).  With one key per
// thread each key takes its rank among the wave's 64 keys, read back from
// kwbase (LDS, 128 words per wave) with broadcast reads; with more, a
// bitwise radix search over ballot counts finds the wave's m-th largest key
// - first on the value word, then, only when several keys share the
// boundary value, on the index word.  Stage 2: each candidate's rank among
// the team's tw*m candidates places it in top[rank] (0 = missing); when
// they fit one wave every wave of the team does this and writes the same
// top[], so it is readable by each wave on return after one barrier,
// otherwise the candidates are shared out and a second barrier follows.
// Every thread of the workgroup takes part.
template <int EPT>
__device__ __forceinline__ void team_select(const FrontLds& L, const uint64_t* kr, uint64_t* cand, uint64_t* top,
                            uint32_t* kwbase, int tt, bool wait_before_rank = false) {
  const int m = L.m, lane = tt & 63, wit = tt >> 6;
  uint32_t hi[EPT], lo[EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    hi[j] = static_cast<uint32_t>(kr[j] >> 32);
    lo[j] = static_cast<uint32_t>(kr[j]);
  }
  uint64_t* wc = cand + wit * m;
  int base = 0;
  if constexpr (EPT == 1) {
    // one key per lane: its rank among the wave's 64 keys by comparison
    // with all of them, read back from LDS (the wave's own writes, 16-B
    // broadcast reads, no barrier); ranks below m place the key.  First on
    // the value word without its lowest bit (31 bits: a comparison is then
    // the sign bit of a difference, plain arithmetic with no lane masks);
    // two keys equal there take the same rank, so one overwrites the other
    // in the candidate slots, which a read-back finds: then (rarely) the
    // ranks are taken again on the whole keys.
    uint32_t* kh = kwbase + 64 * (threadIdx.x >> 6);  // value words >> 1
    const uint32_t hm = static_cast<uint32_t>(kr[0] >> 33);
    kh[lane] = hm;
    const u32x4* p = reinterpret_cast<const u32x4*>(kh);
    int r = 0;
#pragma unroll
    for (int q = 0; q < 16; q += 8) {
      u32x4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = p[q + u];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        r += static_cast<int>(__builtin_amdgcn_ubfe(hm - v[u].x, 31, 1)) +
             static_cast<int>(__builtin_amdgcn_ubfe(hm - v[u].y, 31, 1)) +
             static_cast<int>(__builtin_amdgcn_ubfe(hm - v[u].z, 31, 1)) +
             static_cast<int>(__builtin_amdgcn_ubfe(hm - v[u].w, 31, 1));
      }
    }
    const bool place = kr[0] != 0 && r < m;
    if (place) wc[r] = kr[0];
    // (read through volatile: the compiler would otherwise forward this
    // lane's own store, which another lane's may have overwritten; and as an
    // LDS pointer: a generic one makes it a flat load, whose wait would also
    // drain the vector loads in flight)
    typedef __attribute__((address_space(3))) volatile uint64_t lds_vu64;
    const bool lost = place && ((lds_vu64*)(wc))[r] != kr[0];
    if (__ballot(lost)) {
      uint64_t* kw = reinterpret_cast<uint64_t*>(kwbase + 64 * kWaves4) + 64 * (threadIdx.x >> 6);
      kw[lane] = kr[0];
      const u32x4* p2 = reinterpret_cast<const u32x4*>(kw);
      r = 0;
      for (int q = 0; q < 32; ++q) {
        const u32x4 v = p2[q];
        const uint64_t a = (static_cast<uint64_t>(v.y) << 32) | v.x;
        const uint64_t b = (static_cast<uint64_t>(v.w) << 32) | v.z;
        r += (a > kr[0]) + (b > kr[0]);
      }
      if (kr[0] != 0 && r < m) wc[r] = kr[0];
    }
    base = __popcll(__ballot(kr[0] != 0));
  } else {
    // th: the largest value word v with at least m keys of value >= v (0 when
    // the wave has fewer than m keys of nonzero value)
    uint32_t th = 0;
    for (int b = 31; b >= 0; --b) {
      const uint32_t c = th | (1u << b);
      int n = 0;
#pragma unroll
      for (int j = 0; j < EPT; ++j) n += __popcll(__ballot(hi[j] >= c));
      if (n >= m) th = c;
    }
    int n_gt = 0, n_eq = 0;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      n_gt += __popcll(__ballot(hi[j] > th));
      n_eq += __popcll(__ballot(hi[j] == th && kr[j] != 0));
    }
    const int need = m - n_gt;  // >= 1
    // at the boundary value, the `need` largest index words (lowest experts)
    uint32_t tl = 0;
    if (n_eq > need) {
      for (int b = 31; b >= 0; --b) {
        const uint32_t c = tl | (1u << b);
        int n = 0;
#pragma unroll
        for (int j = 0; j < EPT; ++j) n += __popcll(__ballot(hi[j] == th && kr[j] != 0 && lo[j] >= c));
        if (n >= need) tl = c;
      }
    }
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const bool sel = kr[j] != 0 && (hi[j] > th || (hi[j] == th && lo[j] >= tl));
      const uint64_t bm = __ballot(sel);
      const int below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bm >> 32),
                                                  __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bm), 0));
      if (sel) wc[base + below] = kr[j];
      base += __popcll(bm);
    }
  }
  if (lane >= base && lane < m) wc[lane] = 0;
  const int nc = L.tw * m;
  if (tt >= nc && tt < L.ncp) cand[tt] = 0;  // rank_n reads whole 16-B pairs
  if (tt < m) top[tt] = 0;
  if (wait_before_rank) wait_vm();  // the caller's copies are visible after the barrier
  bar();
  if (nc <= 64) {
    // every wave of the team ranks all candidates and writes the same
    // top[]: each wave reads its own writes, so no second barrier
    if (lane < nc) {
      const uint64_t key = cand[lane];
      if (key != 0) {
        const int r = rank_n(cand, L.ncp, key);
        if (r < m) top[r] = key;
      }
    }
  } else {
    if (tt < nc) {
      const uint64_t key = cand[tt];
      if (key != 0) {
        const int r = rank_n(cand, L.ncp, key);
        if (r < m) top[r] = key;
      }
    }
    bar();
  }
}

// Expert-major plan from ridx[T*k] (ids outside [0, E) skipped): group 0 =
// shared expert when present, then distinct routed experts ascending;
// entries in (expert, token, slot) order.  ctrl[0] = valid routes,
// ctrl[1] = distinct experts.  Runs on wave 0 when T*k <= 64 (cross-lane
// reads), else on the whole workgroup; ends with a workgroup barrier.
__device__ __forceinline__ void build_plan(uint32_t* dyn, const FrontLds& L, int T, int k, int E, int has_shared,
                           int tid) {
  const int* ridx = reinterpret_cast<const int*>(dyn + L.ridx);
  int* re = reinterpret_cast<int*>(dyn + L.re);
  int* rfirst = reinterpret_cast<int*>(dyn + L.rfirst);
  int* poff = reinterpret_cast<int*>(dyn + L.poff);
  int* pexp = reinterpret_cast<int*>(dyn + L.pexp);
  int* ptok = reinterpret_cast<int*>(dyn + L.ptok);
  int* pslot = reinterpret_cast<int*>(dyn + L.pslot);
  int* ctrl = reinterpret_cast<int*>(dyn + L.ctrl);
  const int R = T * k;
  const int gbase = has_shared, ebase = has_shared ? T : 0;
  if (R <= 64) {
    if (tid < 64) {
      // One wave sorts the routes by key = (expert, route index): each
      // lane's rank is the count of smaller keys, read back from LDS with
      // broadcast 16-B reads (the wave's own writes, visible to its later
      // reads without a barrier).  Keys are below 2^17, so the comparison
      // is the sign bit of an integer difference (no lane masks).  An
      // invalid id sorts last and is left out.  Then the sorted keys come
      // back in lane order: lane r holds the r-th entry, its expert starts
      // a group when the previous entry's differs, and its group is the
      // count of group starts below it (a ballot).
      const int lane = tid;
      int e = lane < R ? ridx[lane] : -1;
      if (e < 0 || e >= E) e = -1;
      if (lane < R) re[lane] = e;
      const int key = lane < R ? (e >= 0 ? e : 1024) * 64 + lane : 0x7FFFFFFF;
      int* keys = rfirst;  // the sort's scratch: R keys, then the sorted ones
      if (lane < R) keys[lane] = key;
      int rank = 0;
      for (int j0 = 0; j0 < R; j0 += 4) {
        const int4 v = *reinterpret_cast<const int4*>(keys + j0);
        const int kv4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (j0 + u < R)
            rank += static_cast<int>(__builtin_amdgcn_ubfe(static_cast<unsigned>(kv4[u] - key), 31, 1));
      }
      int* sorted = ptok;  // placed here, then overwritten below with the entries' tokens
      const int nv = __popcll(__ballot(e >= 0));
      if (lane < R) sorted[rank] = key;
      const int sk = lane < nv ? sorted[lane] : 0;
      const int sp = lane > 0 && lane < nv ? sorted[lane - 1] : -64;
      const int se = sk >> 6, si = sk & 63;
      const bool first = lane < nv && (lane == 0 || (sp >> 6) != se);
      const uint64_t fm = __ballot(first);
      const int grp = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(fm >> 32),
                                                __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(fm), 0));
      const int nf = __popcll(fm);
      wait_lds();  // the sorted keys are read before the entries overwrite them
      if (lane < nv) {
        ptok[ebase + lane] = si / k;
        pslot[ebase + lane] = si % k;
        if (first) {
          poff[gbase + grp] = ebase + lane;
          pexp[gbase + grp] = se;
        }
      }
      if (has_shared && lane < T) {
        ptok[lane] = lane;
        pslot[lane] = k;
      }
      if (lane == 0) {
        poff[0] = 0;
        poff[gbase + nf] = ebase + nv;
        if (has_shared) pexp[0] = -1;
        ctrl[0] = nv;
        ctrl[1] = nf;
      }
    }
    bar();
    return;
  }
  if (tid == 0) ctrl[0] = ctrl[1] = 0;
  for (int i = tid; i < R; i += 256) {
    const int e = ridx[i];
    re[i] = (e >= 0 && e < E) ? e : -1;
  }
  bar();
  for (int i = tid; i < R; i += 256) {
    const int e = re[i];
    int first = e >= 0;
    for (int j = 0; j < i && first; ++j) first = re[j] != e;
    rfirst[i] = first;
    if (e >= 0) atomicAdd(&ctrl[0], 1);
    if (first) atomicAdd(&ctrl[1], 1);
  }
  bar();
  for (int i = tid; i < R; i += 256) {
    const int e = re[i];
    if (e < 0) continue;
    int rank = 0, grp = 0;
    for (int j = 0; j < R; ++j) {
      const int ej = re[j];
      if (ej < 0) continue;
      rank += ej < e || (ej == e && j < i);
      grp += rfirst[j] && ej < e;
    }
    ptok[ebase + rank] = i / k;
    pslot[ebase + rank] = i % k;
    if (rfirst[i]) {
      poff[gbase + grp] = ebase + rank;
      pexp[gbase + grp] = e;
    }
  }
  if (has_shared && tid < T) {
    ptok[tid] = tid;
    pslot[tid] = k;
  }
  bar();
  if (tid == 0) {
    poff[0] = 0;
    poff[gbase + ctrl[1]] = ebase + ctrl[0];
    if (has_shared) pexp[0] = -1;
  }
  bar();
}

// ---- front kernel ---------------------------------------------------------------------

// gate/up + SiLU of one wave's rows [row0, row0+nrw) of (wg, wu), whose
// bytes the wave already copied into buf (gate rows, then up rows), for the
// n entries (tok[j], slot[j]); x in LDS as staged Q8_K (xs).  Lanes 0-31
// hold gate super-blocks, lanes 32-63 the same up rows.
// r16 (the layer on the session's fp16 buffers): g and u are rounded to
// fp16 before the SiLU and h after it, as the session stores them
// (gemv_ptrs_q4_k_q8_f16out, then silu_mul_f16: session.cpp:1862-1869).
template <typename Entry>
__device__ __forceinline__ void gateup_wave(bool present, int row0, int nrw, int nbh, int lpr,
                                            const uint32_t* buf, const uint32_t* xs, Entry entry,
                                            int n, int stride, int n_ff, float* h, int lane,
                                            bool r16) {
  const int half = lane >> 5, hl = lane & 31;
  const int blk = hl & (lpr - 1), rr = hl / lpr;
  const bool live = present && blk < nbh && rr < nrw;
  wait_vm();
  uint32_t w36[36];
  ScaleMins sm8{};
  if (live) {
    read_block_lds(buf + 36 * (half * nrw * nbh + rr * nbh + blk), w36);
    sm8 = unpack_scales(w36[1], w36[2], w36[3]);
  }
  for (int j = 0; j < n; ++j) {
    int t, sl;
    entry(j, t, sl);
    float s = 0.f;
    if (live) {
      int32_t xr[64], ip[8];
      float xd, bsf[8];
      load_x_regs(xs + (t * nbh + blk) * kXStride, xr, xd, bsf);
      subblock_dots(w36 + 4, xr, ip);
      s = block_sum(w36[0], sm8, ip, xd, bsf);
    }
    const float acc = row_sum_last(s, blk, nbh);
    const float up = __shfl_xor(acc, 32, 64);
    if (half == 0 && blk == nbh - 1 && rr < nrw)
      h[(static_cast<long long>(t) * stride + sl) * n_ff + row0 + rr] =
          !present ? 0.f : r16 ? f16r(silu_mul(f16r(acc), f16r(up))) : silu_mul(acc, up);
  }
}

// One wave's share of a gate/up workgroup of the several-token launch: its
// nrw gate rows and the same up rows (in buf, landed and visible) against
// the Q8_K x of each of the group's n entries, h = SiLU(g) * u per entry.
// x comes from xq (global, kXStride words per block, token-major): entry
// 0's token is already in x0 (LDS); the others are copied into the weight
// buffers xspace (every wave's, kSpaceWords words) once every wave holds
// its weights in registers, as many per round as fit.  x is read from LDS
// one sub-block group at a time, which keeps the kernel within 128
// registers (four workgroups per CU).  Every wave of the workgroup calls
// this with the same n.  r16: fp16 g, u and h, as in gateup_wave (the
// session's grouped path: session.cpp:2791-2803).
constexpr int kSpaceWords = 4 * 64 * 36;
template <typename Entry>
__device__ __forceinline__ void gateup_group(bool present, int row0, int nrw, int nbh, int lpr,
                                             const uint32_t* buf, uint32_t* xspace,
                                             const uint32_t* x0, const uint32_t* xq, Entry entry,
                                             int n, int stride, int n_ff, float* h, int lane,
                                             int wave, bool r16) {
  const int half = lane >> 5, hl = lane & 31;
  const int blk = hl & (lpr - 1), rr = hl / lpr;
  const bool live = present && blk < nbh && rr < nrw;
  uint32_t w36[36];
  ScaleMins sm8{};
  if (live) {
    read_block_lds(buf + 36 * (half * nrw * nbh + rr * nbh + blk), w36);
    sm8 = unpack_scales(w36[1], w36[2], w36[3]);
  }
  auto dot_store = [&](const uint32_t* xtok, int t, int sl) {
    float s = 0.f;
    if (live) {
      const uint32_t* xb = xtok + blk * kXStride;
      int32_t ip[8];
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const u32x4* p4 = reinterpret_cast<const u32x4*>(xb + 16 * gq);
        int32_t xg[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const u32x4 v = p4[i];
          xg[4 * i] = static_cast<int32_t>(v.x);
          xg[4 * i + 1] = static_cast<int32_t>(v.y);
          xg[4 * i + 2] = static_cast<int32_t>(v.z);
          xg[4 * i + 3] = static_cast<int32_t>(v.w);
        }
        int32_t lo = 0, hi = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t w = w36[4 + 8 * gq + j];
          lo = __builtin_amdgcn_sdot4(static_cast<int>(w & 0x0F0F0F0Fu), xg[j], lo, false);
          hi = __builtin_amdgcn_sdot4(static_cast<int>((w >> 4) & 0x0F0F0F0Fu), xg[8 + j], hi,
                                      false);
        }
        ip[2 * gq] = lo;
        ip[2 * gq + 1] = hi;
      }
      float bsf[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) bsf[q] = __builtin_bit_cast(float, xb[65 + q]);
      s = block_sum(w36[0], sm8, ip, __builtin_bit_cast(float, xb[64]), bsf);
    }
    const float acc = row_sum_last(s, blk, nbh);
    const float up = __shfl_xor(acc, 32, 64);
    if (half == 0 && blk == nbh - 1 && rr < nrw)
      h[(static_cast<long long>(t) * stride + sl) * n_ff + row0 + rr] =
          !present ? 0.f : r16 ? f16r(silu_mul_kc(f16r(acc), f16r(up))) : silu_mul_kc(acc, up);
  };
  if (n > 0) {
    int t, sl;
    entry(0, t, sl);
    dot_store(x0, t, sl);
  }
  const int xw = nbh * kXStride;    // words of one token's x
  const int cw = xw / 4;            // its 16-B chunks
  const int cap = kSpaceWords / xw;  // tokens per round in the weight buffers
#pragma unroll 1
  for (int e0 = 1; e0 < n; e0 += cap) {
    const int ne = min(cap, n - e0);
    bar();  // every wave's weights are in registers: the buffers are free
    const int nch = ne * cw;
#pragma unroll 1
    for (int c0 = 64 * wave; c0 < nch; c0 += 256) {
      const int c = min(c0 + lane, nch - 1);
      const int ei = c / cw;
      int t, sl;
      entry(e0 + ei, t, sl);
      const uint32_t* src = xq + static_cast<long long>(t) * xw + 4 * (c - ei * cw);
      __builtin_amdgcn_global_load_lds((glb_void_p)src, (lds_void_p)(xspace + 4 * c0), 16, 0, 0);
    }
    wait_vm();
    bar();
#pragma unroll 1
    for (int i = 0; i < ne; ++i) {
      int t, sl;
      entry(e0 + i, t, sl);
      dot_store(xspace + i * xw, t, sl);
    }
  }
}

// Copy gate rows [row0, row0+nrw) and the same up rows into a wave buffer.
// (part/nparts: this wave's share of the copy instructions, as dma_chunks)
__device__ __forceinline__ void dma_gateup(const sg_block_q4k* wg, const sg_block_q4k* wu,
                                           int row0, int nrw, int nbh, uint32_t* buf, int lane,
                                           int part = 0, int nparts = 1) {
  const char* pg = reinterpret_cast<const char*>(wg + static_cast<long long>(row0) * nbh);
  const char* pu = reinterpret_cast<const char*>(wu + static_cast<long long>(row0) * nbh);
  const int ncg = nrw * nbh * 9;
  dma_chunks<kNt>([&](int c) { return c < ncg ? pg + 16 * c : pu + 16 * (c - ncg); }, 2 * ncg,
                  buf, lane, part, nparts);
}

// The lane's 16 values of x block b (16-lane row layout: lane & 15 holds
// values 16 (lane & 15) .. + 15) from the fp32 or fp16 x, or - with a
// caller-made Q8_K - the lane's part of that block as raw words: v[0..3]
// its 16 qs bytes, v[4] d, v[5] the block's bsum of its 32 values (even
// lanes; int16 in the low half).
__device__ __forceinline__ void x_load16(const LayerArgs& a, int b, int lane, float (&v)[16]) {
  const int r = lane & 15;
  if (a.xq_in) {
    const uint32_t* q = reinterpret_cast<const uint32_t*>(a.xq_in + static_cast<long long>(b) * kQ8Bytes);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __builtin_bit_cast(float, q[1 + 4 * r + i]);
    v[4] = __builtin_bit_cast(float, q[0]);
    v[5] = __builtin_bit_cast(float, q[65 + (r >> 2)] >> (16 * ((r >> 1) & 1)));
  } else if (a.x16) {
    const uint16_t* xb = a.x16 + static_cast<long long>(b) * kQK + 16 * r;
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = f16v(xb[i]);
  } else {
    const float* xb = a.x + static_cast<long long>(b) * kQK + 16 * r;
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = xb[i];
  }
}

// x_load16's values of block b into LDS in the kXStride layout: quantized
// (quantize_row16_lds), or the caller's Q8_K block rearranged (the same
// layout quantize_row16_lds writes).
__device__ __forceinline__ void x_row16_lds(const LayerArgs& a, const float (&v)[16], uint32_t* dst,
                                            bool active, int lane) {
  if (a.xq_in) {
    const int r = lane & 15;
    if (active) {
      *reinterpret_cast<u32x4*>(dst + 4 * r) =
          (u32x4){__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[1]),
                  __builtin_bit_cast(uint32_t, v[2]), __builtin_bit_cast(uint32_t, v[3])};
      if (r == 0) dst[64] = __builtin_bit_cast(uint32_t, v[4]);
      if ((r & 1) == 0)
        dst[65 + (r >> 1)] = __builtin_bit_cast(
            uint32_t, static_cast<float>(static_cast<int16_t>(__builtin_bit_cast(uint32_t, v[5]))));
    }
  } else {
    quantize_row16_lds(v, dst, active, lane);
  }
}

// x values of a wave's first P quantization passes, loaded at kernel start
// so their latency overlaps the routing or the plan: one Q8_K block per
// 16-lane row, pass p taking block 4 (p nw + w) + (lane >> 4), the lane's 16
// values.  Waves w < nw take part.
template <int P>
__device__ __forceinline__ void x_preload(const LayerArgs& a, int n_blocks, int w, int nw, int lane,
                                          float (&pre)[P][16]) {
  if (w >= nw) return;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int b = 4 * (p * nw + w) + (lane >> 4);
    x_load16(a, b < n_blocks ? b : 0, lane, pre[p]);
  }
}

// Q8_K of the x rows into LDS (kXStride layout), one block per 16-lane row:
// pass p of wave w takes block 4 (p nw + w) + (lane >> 4); the first P
// passes' values come from x_preload.
template <int P>
__device__ __forceinline__ void quantize_x(const LayerArgs& a, int n_blocks, uint32_t* xs, int w,
                                           int nw, int lane, const float (&pre)[P][16]) {
  if (w >= nw) return;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int b = 4 * (p * nw + w) + (lane >> 4);
    if (p > 0 && 4 * p * nw >= n_blocks) break;  // wave-uniform
    x_row16_lds(a, pre[p], xs + (b < n_blocks ? b : 0) * kXStride, b < n_blocks, lane);
  }
  for (int b0 = 4 * nw * P; b0 < n_blocks; b0 += 4 * nw) {
    const int b = b0 + 4 * w + (lane >> 4);
    const int bc = b < n_blocks ? b : 0;
    float v[16];
    x_load16(a, bc, lane, v);
    x_row16_lds(a, v, xs + bc * kXStride, b < n_blocks, lane);
  }
}

// Logit-order top-(k+1) of every token: spec[t*m + r] = r-th expert (or -1).
// Logits of the first routing pass into lr[] (what spec_select's pass 0
// reads): thread tt of team `team` holds experts tt + TT*j of token `team`,
// 0 outside.  Same team geometry as front_lds.
template <int EPT>
__device__ __forceinline__ void logits_preload(const LayerArgs& a, int T, int tid, float* lr) {
  const int E = a.n_expert;
  const int nteams = T == 1 ? 1 : (T == 2 ? 2 : 4);
  const int TT = 64 * (4 / nteams);
  const int ept = (E + TT - 1) / TT;
  const int team = tid / TT, tt = tid - team * TT;
  const bool ok = team < T;
  const float* lg = a.logits + static_cast<long long>(team) * E;
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int i = tt + TT * j;
    lr[j] = (j < ept && i < E && ok) ? lg[i] : 0.f;
  }
}

// Logit-order top-(k+1) of every token: teams of tw waves, one token per
// team per pass; each thread keeps its logits in lr[] (pass 0's from
// logits_preload, then the last pass's token).  Workgroup-wide; the last
// pass's top[] is readable on return, spec[] only after the caller's next
// barrier.  wait_copies: the calling wave waits for its outstanding copies
// before the selection's barrier (so they are visible on return).
template <int EPT>
__device__ __forceinline__ void spec_select(const LayerArgs& a, int T, uint32_t* dyn, const FrontLds& L,
                            float* lr, int tid, bool wait_copies = false) {
  const int E = a.n_expert, m = L.m;
  const int wave = tid >> 6, team = wave / L.tw, tt = tid - team * L.TT;
  float* lv = reinterpret_cast<float*>(dyn + L.lv) + team * L.e32;
  uint64_t* cand = reinterpret_cast<uint64_t*>(dyn + L.cand) + team * L.ncp;
  uint64_t* top = reinterpret_cast<uint64_t*>(dyn + L.top) + team * m;
  int* spec = reinterpret_cast<int*>(dyn + L.spec);
  for (int t0 = 0; t0 < T; t0 += L.nteams) {
    const int t = t0 + team;
    const bool ok = t < T;
    const float* lg = a.logits + static_cast<long long>(t) * E;
    uint64_t kr[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const int i = tt + L.TT * j;
      const bool in = j < L.ept && i < E && ok;
      if (t0 > 0) lr[j] = in ? lg[i] : 0.f;  // pass 0: logits_preload
      kr[j] = in ? sel_key(lr[j], i) : 0;
      if (j < L.ept && i < L.e32) lv[i] = lr[j];
    }
    team_select<EPT>(L, kr, cand, top, dyn + L.kw, tt, wait_copies && t0 == 0);
    if (ok && tt < m) spec[t * m + tt] = top[tt] ? sel_idx(top[tt]) : -1;
    if (t0 + L.nteams < T) bar();  // the next pass reuses cand/top
  }
}

// Plan for T == 1 straight from k distinct, valid ids id(0..k-1): group
// gbase + r = the expert of rank r, its single entry (token 0, slot j).
// Ends with a barrier unless the caller places one.
template <typename Id>
__device__ __forceinline__ void plan_t1(uint32_t* dyn, const FrontLds& L, int k, int has_shared, int tid, Id id,
                        bool barrier = true) {
  int* re = reinterpret_cast<int*>(dyn + L.re);
  int* poff = reinterpret_cast<int*>(dyn + L.poff);
  int* pexp = reinterpret_cast<int*>(dyn + L.pexp);
  int* ptok = reinterpret_cast<int*>(dyn + L.ptok);
  int* pslot = reinterpret_cast<int*>(dyn + L.pslot);
  int* ctrl = reinterpret_cast<int*>(dyn + L.ctrl);
  const int gbase = has_shared, ebase = has_shared ? 1 : 0;
  if (tid < k) {
    const int e = id(tid);
    int r = 0;
    for (int j = 0; j < k; ++j) r += id(j) < e;
    re[tid] = e;
    poff[gbase + r] = ebase + r;
    pexp[gbase + r] = e;
    ptok[ebase + r] = 0;
    pslot[ebase + r] = tid;
  }
  if (tid == 0) {
    if (has_shared) {
      poff[0] = 0;
      pexp[0] = -1;
      ptok[0] = 0;
      pslot[0] = k;
    }
    poff[gbase + k] = ebase + k;
    ctrl[0] = k;
    ctrl[1] = k;
  }
  if (barrier) bar();
}

// True when ridx[0..n) are distinct valid ids (what routing produces for
// one token); then the T == 1 plan needs no general build.
__device__ __forceinline__ bool ids_distinct_valid(const int* ridx, int n, int E) {
  bool ok = true;
  for (int i = 0; i < n; ++i) {
    ok &= ridx[i] >= 0 && ridx[i] < E;
    for (int j = 0; j < i; ++j) ok &= ridx[j] != ridx[i];
  }
  return ok;
}

// The plan of ridx[0..T*k): the one-token form when the ids are distinct
// and valid, else the general build.  Ends with a barrier.
__device__ __forceinline__ void make_plan(uint32_t* dyn, const FrontLds& L, int T, int k, int E,
                                          int has_shared, int tid) {
  const int* ridx = reinterpret_cast<const int*>(dyn + L.ridx);
  if (T == 1 && ids_distinct_valid(ridx, k, E))
    plan_t1(dyn, L, k, has_shared, tid, [&](int j) { return ridx[j]; });
  else
    build_plan(dyn, L, T, k, E, has_shared, tid);
}

// Whether the exact routing of one token (route_wave) is sure to select the
// logit-order ids top[0..k) in that order, decided by one wave from the
// k+1 leading logits alone, without the normalizer: every logit finite
// (so z = sum e lies in [1, E], nothing degenerates), and along the logit
// order each e_j = exp(l_j - max) either equals its successor's logit
// (tie: index order on both sides) or exceeds the successor's e by more
// than 2^-19 relative with the successor >= 2^-100 (the boundary pair k-1,
// k always strictly).  Then p_j = e_j / z > p_{j+1} for any z in [1, E]:
// the quotients are normal and more than two floats apart, so route_wave's
// check (p strictly decreasing or equal logits) passes.  A false result
// only means "run route_wave".  Wave-uniform.
__device__ __forceinline__ bool route_is_logit_order(const LayerArgs& a, const uint32_t* dyn,
                                                     const FrontLds& L, int lane) {
  const int E = a.n_expert, k = a.k, m = L.m;
  const float* lv = reinterpret_cast<const float*>(dyn + L.lv);
  const uint64_t* top = reinterpret_cast<const uint64_t*>(dyn + L.top);
  bool fin = true;
  for (int i = lane; i < E; i += 64) fin &= __builtin_isfinite(lv[i]);
  const int ik = lane < m && top[lane] != 0ull ? sel_idx(top[lane]) : -1;
  const float lk = ik >= 0 ? lv[ik] : 0.f;
  const float mx = readlane_f(lk, 0);
  const float ek = expf_sg(lk - mx);
  const float en = __shfl(ek, lane + 1, 64);
  const float ln = __shfl(lk, lane + 1, 64);
  const int in = __shfl(ik, lane + 1, 64);
  const bool gap = ek > en * 1.0000019073486328f && en >= 7.8886090522101181e-31f;  // 2^-19, 2^-100
  bool ok = true;
  if (lane + 1 < k) ok = ik >= 0 && in >= 0 && (lk == ln || gap);
  else if (lane + 1 == k && E > k) ok = ik >= 0 && in >= 0 && gap;
  return __ballot(!(ok && fin)) == 0ull;
}

// Exact routing of ONE token by one wave, no workgroup barrier (moe.cu:25-85):
// same arithmetic and checks as exact_route below.  Logits come from lv[]
// (LDS, filled by spec_select), lane l holds experts l + 64j.  Writes ridx,
// rw and ctrl[3] (1 when an id differs from the logit order).
template <int EPL>
__device__ __forceinline__ void route_wave(const LayerArgs& a, uint32_t* dyn, const FrontLds& L, int lane) {
  const int E = a.n_expert, k = a.k, m = L.m;
  const float* lv = reinterpret_cast<const float*>(dyn + L.lv);
  float* ev = reinterpret_cast<float*>(dyn + L.ev);
  const uint64_t* top = reinterpret_cast<const uint64_t*>(dyn + L.top);
  int* ridx = reinterpret_cast<int*>(dyn + L.ridx);
  float* rw = reinterpret_cast<float*>(dyn + L.rw);
  int* ctrl = reinterpret_cast<int*>(dyn + L.ctrl);
  float v[EPL];
  float mx = -1e30f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int i = lane + 64 * j;
    v[j] = i < E ? lv[i] : 0.f;
    if (i < E) mx = fmaxf(mx, v[j]);
  }
  mx = wave_max_dpp(mx);
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int i = lane + 64 * j;
    if (i < L.e32) ev[i] = i < E ? expf_sg(v[j] - mx) : 0.f;
  }
  // the wave's LDS writes complete in order before its own reads
  const float z = readlane_f(lane == 0 ? serial_sum(ev, L.e32) : 0.f, 0);
  const bool degen = !(z == z) || z == 0.f;
  const int ik = lane < m && top[lane] != 0ull ? sel_idx(top[lane]) : -1;  // logit order
  const float pk = (ik >= 0 && !degen) ? ev[ik] / z : -1.f;
  const float lk = ik >= 0 ? lv[ik] : 0.f;
  const float pn = __shfl(pk, lane + 1, 64);
  const float ln = __shfl(lk, lane + 1, 64);
  const int in = __shfl(ik, lane + 1, 64);
  bool cond = true;
  if (lane + 1 < k) cond = ik >= 0 && in >= 0 && (pk > pn || lk == ln);
  else if (lane + 1 == k && E > k) cond = ik >= 0 && in >= 0 && pk > pn;
  const bool fast = !degen && __ballot(!cond) == 0;
  int fi;
  float pv;
  if (degen) {
    fi = lane % E;
    pv = -1.f;
  } else if (fast) {
    fi = ik;
    pv = pk;
  } else {  // a probability collision: k rounds of argmax on p itself
    uint64_t kv[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int i = lane + 64 * j;
      kv[j] = i < E ? sel_key(ev[i] / z, i) : 0ull;
    }
    fi = 0;
    for (int kk = 0; kk < k; ++kk) {
      uint64_t best = 0;
#pragma unroll
      for (int j = 0; j < EPL; ++j) best = kv[j] > best ? kv[j] : best;
      best = wave_max_u64(best);
      if (lane == kk) fi = best ? sel_idx(best) : 0;
#pragma unroll
      for (int j = 0; j < EPL; ++j)
        if (kv[j] == best) kv[j] = 0;
    }
    pv = ev[fi] / z;
  }
  float wsum = 0.f;
  for (int kk = 0; kk < k; ++kk) wsum += readlane_f(pv, kk);
  const float wv = wsum > 0.f ? pv / wsum : pv;
  bool changed = false;
  if (lane < k) {
    changed = fi != ik;
    ridx[lane] = fi;
    rw[lane] = wv;
  }
  const bool any = __ballot(changed) != 0ull;
  if (lane == 0) {
    rw[k] = a.shared_w;
    ctrl[3] = any;
  }
}

// Exact routing of ONE token by the whole workgroup straight from the
// logits (moe.cu:25-85), for the publisher: max, one exp per expert per
// thread, the normalizer summed serially in index order, then the top k of
// the probability keys (value desc, index asc: the reference's k rounds of
// first-strict-max) by team_select; a degenerate row (NaN, empty
// normalizer) takes kk % E with weight -1.  Weights renormalized by their
// k-order sum.  Writes ridx[0..k), rw[0..k] and the one-token plan; ends
// with a barrier.
template <int EPT>
__device__ __forceinline__ void route_direct_t1(const LayerArgs& a, uint32_t* dyn, const FrontLds& L,
                                                const float* lr, int tid) {
  const int E = a.n_expert, k = a.k;
  const int lane = tid & 63, wave = tid >> 6;
  float* ev = reinterpret_cast<float*>(dyn + L.ev);
  uint64_t* cand = reinterpret_cast<uint64_t*>(dyn + L.cand);
  uint64_t* top = reinterpret_cast<uint64_t*>(dyn + L.top);
  float* red = reinterpret_cast<float*>(dyn + L.red);
  float* zs = reinterpret_cast<float*>(dyn + L.zs);
  int* ridx = reinterpret_cast<int*>(dyn + L.ridx);
  float* rw = reinterpret_cast<float*>(dyn + L.rw);
  float mx = -1e30f;
#pragma unroll
  for (int j = 0; j < EPT; ++j)
    if (j < L.ept && tid + L.TT * j < E) mx = fmaxf(mx, lr[j]);
  mx = team_max(mx, red, wave, L.tw, lane);
  float e[EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int i = tid + L.TT * j;
    e[j] = (j < L.ept && i < E) ? expf_sg(lr[j] - mx) : 0.f;
    if (j < L.ept && i < L.e32) ev[i] = e[j];
  }
  bar();
  if (tid == 0) zs[0] = serial_sum(ev, L.e32);
  bar();
  const float z = zs[0];
  const bool degen = !(z == z) || z == 0.f;
  if (!degen) {
    uint64_t kr[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const int i = tid + L.TT * j;
      kr[j] = (j < L.ept && i < E) ? sel_key(e[j] / z, i) : 0ull;
    }
    team_select<EPT>(L, kr, cand, top, dyn + L.kw, tid);
  }
  if (wave == 0) {
    int fi = 0;
    float pv = -1.f;
    if (lane < k) {
      fi = degen ? lane % E : (top[lane] ? sel_idx(top[lane]) : 0);
      if (!degen) pv = ev[fi] / z;
    }
    float wsum = 0.f;
    for (int kk = 0; kk < k; ++kk) wsum += readlane_f(pv, kk);
    const float wv = wsum > 0.f ? pv / wsum : pv;
    if (lane < k) {
      ridx[lane] = fi;
      rw[lane] = wv;
    }
    if (lane == 0) rw[k] = a.shared_w;
    // the plan straight from the ids in registers (distinct and valid: k
    // of E distinct keys, or kk % E with k <= E), as plan_t1 builds it
    int* re = reinterpret_cast<int*>(dyn + L.re);
    int* poff = reinterpret_cast<int*>(dyn + L.poff);
    int* pexp = reinterpret_cast<int*>(dyn + L.pexp);
    int* ptok = reinterpret_cast<int*>(dyn + L.ptok);
    int* pslot = reinterpret_cast<int*>(dyn + L.pslot);
    int* ctrl = reinterpret_cast<int*>(dyn + L.ctrl);
    const int gbase = a.has_shared, ebase = a.has_shared ? 1 : 0;
    int r = 0;
    for (int j = 0; j < k; ++j) r += __builtin_amdgcn_readlane(fi, j) < fi;
    if (lane < k) {
      re[lane] = fi;
      poff[gbase + r] = ebase + r;
      pexp[gbase + r] = fi;
      ptok[ebase + r] = 0;
      pslot[ebase + r] = lane;
    }
    if (lane == 0) {
      if (a.has_shared) {
        poff[0] = 0;
        pexp[0] = -1;
        ptok[0] = 0;
        pslot[0] = k;
      }
      poff[gbase + k] = ebase + k;
      ctrl[0] = k;
      ctrl[1] = k;
    }
  }
  bar();
}

// Exact routing of every token (moe.cu:25-85): max, exp, the normalizer
// summed serially in index order, p = e / z.  p is a monotone function of
// the logit, so the logit order (spec[]) is the probability order unless two
// neighbours collide on one float; the check is p strictly decreasing
// across the k+1 leading candidates (or equal logits).  A collision selects
// on the probabilities themselves; a degenerate row (NaN, empty normalizer)
// takes kk % E with weight -1.  Writes ridx (replacing the logit-order ids)
// and rw; ctrl[3] = 1 when any id changed.  Workgroup-wide, barriers only
// (no wait on the weight stream in flight).
template <int EPT>
__device__ __forceinline__ void exact_route(const LayerArgs& a, uint32_t* dyn, const FrontLds& L, float* lr,
                            int tid) {
  const int T = a.T, E = a.n_expert, k = a.k, stride = k + 1, m = L.m;
  const int lane = tid & 63, wave = tid >> 6;
  const int tw = L.tw, team = wave / tw, wit = wave - team * tw;
  const int tt = tid - team * L.TT;
  float* lv = reinterpret_cast<float*>(dyn + L.lv) + team * L.e32;
  float* ev = reinterpret_cast<float*>(dyn + L.ev) + team * L.e32;
  uint64_t* cand = reinterpret_cast<uint64_t*>(dyn + L.cand) + team * L.ncp;
  uint64_t* top = reinterpret_cast<uint64_t*>(dyn + L.top) + team * m;
  float* red = reinterpret_cast<float*>(dyn + L.red) + team * 4;
  float* zs = reinterpret_cast<float*>(dyn + L.zs);
  int* spec = reinterpret_cast<int*>(dyn + L.spec);
  int* ridx = reinterpret_cast<int*>(dyn + L.ridx);
  float* rw = reinterpret_cast<float*>(dyn + L.rw);
  int* ctrl = reinterpret_cast<int*>(dyn + L.ctrl);
  if (tid == 0) ctrl[3] = 0;
  for (int t0 = 0; t0 < T; t0 += L.nteams) {
    const int t = t0 + team;
    const bool ok = t < T;
    if (T > L.nteams) {  // several passes: (re)load this token's logits
      const float* lg = a.logits + static_cast<long long>(t) * E;
#pragma unroll
      for (int j = 0; j < EPT; ++j) {
        const int i = tt + L.TT * j;
        lr[j] = (j < L.ept && i < E && ok) ? lg[i] : 0.f;
        if (j < L.ept && i < L.e32) lv[i] = lr[j];
      }
    }
    if (tid == 0) ctrl[2] = 0;
    float mx = -1e30f;
#pragma unroll
    for (int j = 0; j < EPT; ++j)
      if (j < L.ept && tt + L.TT * j < E && ok) mx = fmaxf(mx, lr[j]);
    mx = team_max(mx, red, wit, tw, lane);
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const int i = tt + L.TT * j;
      if (j < L.ept && i < L.e32) ev[i] = (ok && i < E) ? expf_sg(lr[j] - mx) : 0.f;
    }
    bar();
    if (tt == 0) zs[team] = serial_sum(ev, L.e32);
    bar();
    const float z = zs[team];
    const bool degen = !(z == z) || z == 0.f;
    bool fast = false;
    float pk = -1.f;
    int ik = -1;
    if (wit == 0) {
      ik = (ok && lane < m) ? spec[t * m + lane] : -1;
      pk = (ik >= 0 && !degen) ? ev[ik] / z : -1.f;
      const float lk = ik >= 0 ? lv[ik] : 0.f;
      const float pn = __shfl(pk, lane + 1, 64);
      const float ln = __shfl(lk, lane + 1, 64);
      const int in = __shfl(ik, lane + 1, 64);
      bool cond = true;
      if (lane + 1 < k) cond = ik >= 0 && in >= 0 && (pk > pn || lk == ln);
      else if (lane + 1 == k && E > k) cond = ik >= 0 && in >= 0 && pk > pn;
      fast = ok && !degen && __ballot(!cond) == 0;
      if (lane == 0) {
        ctrl[4 + team] = ok && !degen && !fast;
        if (ok && !degen && !fast) atomicOr(&ctrl[2], 1);
      }
    }
    bar();
    if (ctrl[2] != 0) {  // selection on the probabilities for the colliding rows
      const bool slow_team = ctrl[4 + team] != 0;
      uint64_t kr[EPT];
#pragma unroll
      for (int j = 0; j < EPT; ++j) {
        const int i = tt + L.TT * j;
        kr[j] = (j < L.ept && i < E && slow_team) ? sel_key(ev[i] / z, i) : 0;
      }
      team_select<EPT>(L, kr, cand, top, dyn + L.kw, tt);
    }
    if (wit == 0 && ok) {
      int fi;
      float pv;
      if (degen) {
        fi = lane % E;
        pv = -1.f;
      } else if (fast) {
        fi = ik;
        pv = pk;
      } else {
        fi = lane < m && top[lane] ? sel_idx(top[lane]) : 0;
        pv = ev[fi] / z;
      }
      float wsum = 0.f;
      for (int kk = 0; kk < k; ++kk) wsum += readlane_f(pv, kk);
      const float wv = wsum > 0.f ? pv / wsum : pv;
      if (lane < k) {
        if (fi != ridx[t * k + lane]) atomicOr(&ctrl[3], 1);
        ridx[t * k + lane] = fi;
        rw[t * stride + lane] = wv;
      }
      if (lane == 0) rw[t * stride + k] = a.shared_w;
    }
    bar();
  }
}

// Compute workgroups (blockIdx.y < gmax): one (group, chunk of 16 rows).
// The shared expert's group streams at once; a routed group streams the
// expert the logit order gives it, then checks that against the exact
// routing (streaming the exact expert instead when they differ) and writes
// h for the (token, slot) entries of its group in the exact plan.  The
// publisher workgroup (blockIdx.y == gmax, x == 0) runs the same routing
// and writes idx, weight and the plan.
// NBH: hidden / 256 when compiled for it (0 = read from a).
// The shared expert's scalar gate of every token (session.cpp:2904-2909),
// sgate[t] = sigmoid(sh_gate_w . x[t]) in the reference's fp32 lane order:
// one token per 32-lane half-wave of the workgroup; read by the back kernel.
__device__ __forceinline__ void shared_gate_tokens(const LayerArgs& a, int tid) {
  const int l = tid & 31, half = tid >> 5;
  for (int t0 = 0; t0 < a.T; t0 += 8) {
    const int t = min(t0 + half, a.T - 1);
    const long long o = static_cast<long long>(t) * a.hidden;
    const float gl =
        a.x16 ? rowdot_f32_lanes32(a.sh_gate_w, [&](int i) { return f16v(a.x16[o + i]); }, a.hidden, l)
              : rowdot_f32_lanes32(a.sh_gate_w, [&](int i) { return a.x[o + i]; }, a.hidden, l);
    if (l == 0 && t0 + half < a.T) a.sgate[t] = sigmoid_sg(gl);
  }
}

// kOne: the one-token decode instance (T = 1 at compile time, so the
// several-token paths are not compiled into it)
template <int EPT, int NBH, bool kOne>
__device__ __forceinline__ void front_body(const LayerArgs& a, int bx, int g, uint32_t (*wbuf)[64 * 36],
                           uint32_t* dyn) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int T = kOne ? 1 : a.T, k = a.k, E = a.n_expert, stride = k + 1;
  const int nbh = NBH ? NBH : a.hidden / kQK, lpr = NBH ? pow2_ceil(NBH) : pow2_ceil(nbh);
  const bool publisher = g == a.gmax;
  if (publisher && bx != 0) return;  // one publisher per launch
  const bool shared_grp = a.has_shared && g == 0;
  const bool tabd_regs = publisher && E <= 256;
  // expert pointer tables into LDS (gate and up; down for the publisher),
  // issued first: the wait for the logits covers every load in flight, so
  // copies issued after the logits would hold up the selection
  if (!shared_grp && (wave < 2 || (wave == 2 && publisher && !tabd_regs))) {
    // (one branch per table: a select between the argument block's pointer
    // fields would make the compiler keep that block in scratch memory)
    auto copy_table = [&](const sg_block_q4k* const* tab, int at) {
      uint32_t* dst = dyn + at;
      const char* src = reinterpret_cast<const char*>(tab);
      dma_range([&](int c) { return src + 16 * c; }, E / 2, dst, lane);
      if ((E & 1) && lane == 0)  // odd table length: the last pointer by a plain load
        reinterpret_cast<unsigned long long*>(dst)[E - 1] =
            reinterpret_cast<unsigned long long>(tab[E - 1]);
    };
    if (wave == 0)
      copy_table(a.tab_gate, a.front_routed.tabg);
    else if (wave == 1)
      copy_table(a.tab_up, a.front_routed.tabu);
    else
      copy_table(a.tab_down, a.front_routed.tabd);
  }
  // the first routing pass's logits are the head of the routing chain
  float lr[EPT];
  if (a.logits && !shared_grp) logits_preload<EPT>(a, T, tid, lr);
  const FrontLds& L = shared_grp ? a.front_shared : a.front_routed;
  const int rpw = 32 / lpr;
  const int row0 = bx * 4 * rpw + wave * rpw;
  // (every chunk full when n_ff is a multiple of the workgroup's rows: then
  // a constant in the shape instances, and the copies need no lane masks)
  const bool full = a.n_ff % (4 * rpw) == 0;
  const int nrw = full ? rpw : max(0, min(rpw, a.n_ff - row0));
  const int gbase = a.has_shared;
  uint32_t* buf = wbuf[wave];
  uint32_t* xs = dyn + L.xs;
  const int nxb = T * nbh;
  // one token with router logits: wave 3 does the exact routing on its own
  // while waves 0-2 issue the weight stream and quantize x
  const bool t1w = T == 1 && a.logits != nullptr && !shared_grp;
  const int nqw = t1w ? 3 : 4;
  float xpre[1][16];
  if (!publisher) x_preload(a, nxb, wave, nqw, lane, xpre);

  if (shared_grp) {
    if (nrw > 0) dma_gateup(a.sh_gate, a.sh_up, row0, nrw, nbh, buf, lane);
    quantize_x(a, nxb, xs, wave, nqw, lane, xpre);
    bar();
    // entries: tokens 0..T-1 in slot k, no plan needed
    gateup_wave(true, row0, nrw, nbh, lpr, buf, xs,
                [&](int j, int& t, int& sl) { t = j; sl = k; }, T, stride, a.n_ff, a.h, lane,
                a.out16 != nullptr);
    if (a.sh_gate_w && bx == 0) shared_gate_tokens(a, tid);
    return;
  }

  const unsigned long long* tabg = reinterpret_cast<const unsigned long long*>(dyn + L.tabg);
  const unsigned long long* tabu = reinterpret_cast<const unsigned long long*>(dyn + L.tabu);
  const unsigned long long* tabd = reinterpret_cast<const unsigned long long*>(dyn + L.tabd);
  int* ridx = reinterpret_cast<int*>(dyn + L.ridx);
  int* spec = reinterpret_cast<int*>(dyn + L.spec);
  float* rw = reinterpret_cast<float*>(dyn + L.rw);
  int* ctrl = reinterpret_cast<int*>(dyn + L.ctrl);
  const int* pexp = reinterpret_cast<const int*>(dyn + L.pexp);
  const int* poff = reinterpret_cast<const int*>(dyn + L.poff);
  const int* ptok = reinterpret_cast<const int*>(dyn + L.ptok);
  const int* pslot = reinterpret_cast<const int*>(dyn + L.pslot);

  // The publisher's down table goes through registers when E <= 256: it is
  // written to LDS only when publishing, long after it landed, so no LDS
  // access of wave 2 waits for it meanwhile.
  unsigned long long tdv[4];
  if (tabd_regs && wave == 2) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      tdv[j] = lane + 64 * j < E ? reinterpret_cast<unsigned long long>(a.tab_down[lane + 64 * j])
                                 : 0ull;
  }

  // stream the gate/up rows of expert e (none when e < 0 or it is absent)
  // for wave w's rows into wave w's buffer
  // (returns whether expert e is present: both its matrices non-null)
  auto stream_rows = [&](int e, int w, int part = 0, int nparts = 1) {
    if (e < 0) return false;
    const int r0 = bx * 4 * rpw + w * rpw;
    const int n = full ? rpw : min(rpw, a.n_ff - r0);
    const sg_block_q4k* wg = reinterpret_cast<const sg_block_q4k*>(tabg[e]);
    const sg_block_q4k* wu = reinterpret_cast<const sg_block_q4k*>(tabu[e]);
    if (wg && wu && n > 0) dma_gateup(wg, wu, r0, n, nbh, wbuf[w], lane, part, nparts);
    return wg && wu;
  };

  int e_mine = -1, slot_mine = -1;
  bool present_mine = false;
  int n_groups;
  if (a.logits && publisher && T > 1) {
    // the routing launch of several tokens: one wave per token, each the
    // standalone router's exact routing (router_wave), then the plan
    // experts per lane: E <= 64 PL (the launch picks EPT with E <= 64 EPT
    // for three or more tokens, E <= 128 EPT for two)
    constexpr int kPl1 = EPT < 16 ? EPT : 16, kPl2 = 2 * EPT < 16 ? 2 * EPT : 16;
    float* evw = reinterpret_cast<float*>(dyn + L.ev) + wave * L.e32;
    // x of the window for waves 1-3 to quantize while wave 0 builds the plan
    float xw[3][16];
    if (wave > 0) x_preload(a, nxb, wave - 1, 3, lane, xw);
    for (int t = wave; t < T; t += 4) {
      const float* lg = a.logits + static_cast<long long>(t) * E;
      if (T == 2)
        router_wave<kPl2>(lg, E, k, a.shared_w, ridx + t * k, rw + t * stride, evw, lane);
      else
        router_wave<kPl1>(lg, E, k, a.shared_w, ridx + t * k, rw + t * stride, evw, lane);
    }
    bar();
    if (wave > 0) quantize_x(a, nxb, a.xq, wave - 1, 3, lane, xw);
    build_plan(dyn, L, T, k, E, a.has_shared, tid);
    n_groups = gbase + ctrl[1];
  } else if (a.logits && publisher && T == 1) {
    // the publisher routes exactly from the logits with every wave; it has
    // no stream to start and needs the weights, not the logit order
    route_direct_t1<EPT>(a, dyn, L, lr, tid);  // and the plan
    n_groups = gbase + ctrl[1];
  } else if (a.logits) {
    // waves 0-1 wait for the pointer tables inside the selection, so they
    // are readable when it returns
    spec_select<EPT>(a, T, dyn, L, lr, tid, wave < 2);
    bool streamed = false, routed = false;
    if (T == 1) {
      // top[] of the single token is readable now: with k valid ids the
      // plan is made here, in the same phase as spec[] and ridx[]
      const uint64_t* top = reinterpret_cast<const uint64_t*>(dyn + L.top);
      const uint64_t tk = lane < k ? top[lane] : 1ull;  // lane j: key of slot j
      const bool valid = __ballot(tk == 0ull) == 0ull;
      if (valid) {
        if (!publisher) {
          // speculative: the logit-order expert of this group, i.e. the one
          // of id rank g - gbase among top[] (what plan_t1 assigns), and its
          // slot, read straight from top[] so the stream starts before the
          // plan round.  Waves 0-2 issue it (each also a third of wave 3's
          // rows) so wave 3 routes unblocked.
          const int want = g - gbase;
          const int idl = lane < k ? sel_idx(tk) : 0x7FFFFFFF;
          // its rank among the k ids, which every lane reads from top[]
          // (broadcast reads; ids < 2^16, so a comparison is the sign bit
          // of a difference)
          int r = 0;
          const uint32_t* tw = reinterpret_cast<const uint32_t*>(top);
          for (int i = 0; i < k; ++i)
            r += static_cast<int>(__builtin_amdgcn_ubfe(
                static_cast<unsigned>(sel_idx(tw[2 * i]) - idl), 31, 1));
          const uint64_t hit = __ballot(lane < k && r == want);
          slot_mine = hit ? __builtin_ctzll(hit) : -1;
          e_mine = hit ? __builtin_amdgcn_readlane(idl, slot_mine) : -1;
          if (wave < 3) present_mine = stream_rows(e_mine, wave);
          if (wave < 3) stream_rows(e_mine, 3, wave, 3);
          if (wave == 3 && e_mine >= 0) present_mine = tabg[e_mine] != 0ull && tabu[e_mine] != 0ull;
          streamed = true;
        }
        // wave 3 routes exactly now (it reads top[] and lv[], complete since
        // the selection's last barrier) and writes ridx[] itself; the plan
        // is published by the barrier after the x quantization below.
        // wave 2 (the one with the fewest x blocks to quantize) writes the
        // plan, its lanes in the roles of threads 0..63
        // (a compute workgroup skips it when the logit order is provably
        // the exact one: only the publisher needs the weights; the
        // publisher routes with all four waves below)
        if (wave == 3 && !publisher) {
          if (route_is_logit_order(a, dyn, L, lane)) {
            if (lane == 0) ctrl[3] = 0;
          } else {
            route_wave<4 * EPT>(a, dyn, L, lane);
          }
        }
        if (wave == 2) {
          plan_t1(dyn, L, k, a.has_shared, lane, [&](int j) { return sel_idx(top[j]); }, false);
          if (publisher && lane < k) ridx[lane] = sel_idx(top[lane]);  // what exact_route compares
        }
        routed = true;
      } else {
        if (tid < k) ridx[tid] = top[tid] ? sel_idx(top[tid]) : -1;
        bar();
        build_plan(dyn, L, T, k, E, a.has_shared, tid);
      }
    } else {
      bar();
      for (int i = tid; i < T * k; i += 256) ridx[i] = spec[(i / k) * L.m + (i % k)];
      bar();
      build_plan(dyn, L, T, k, E, a.has_shared, tid);
    }
    if (!publisher && !streamed) {
      e_mine = g < gbase + ctrl[1] ? pexp[g] : -1;
      // speculative: the logit-order expert.  One token: waves 0-2 issue
      // the stream (each also a third of wave 3's rows) so wave 3 routes
      // unblocked.
      if (!t1w) {
        stream_rows(e_mine, wave);
      } else if (wave < 3) {
        stream_rows(e_mine, wave);
        stream_rows(e_mine, 3, wave, 3);
      }
    }
    if (t1w && publisher) {
      // no weight stream to overlap: the whole workgroup routes exactly (one
      // exp per thread instead of four per lane of one wave)
      exact_route<EPT>(a, dyn, L, lr, tid);
    } else if (t1w) {
      if (wave == 3) {
        if (!routed) route_wave<4 * EPT>(a, dyn, L, lane);
      } else {
        quantize_x(a, nxb, xs, wave, nqw, lane, xpre);  // overlaps the weight stream
        wait_vm();  // this wave's share of wave 3's rows
      }
      bar();
    } else {
      exact_route<EPT>(a, dyn, L, lr, tid);
    }
    const bool moved = ctrl[3] != 0;  // the exact routing changed an id
    if (moved) make_plan(dyn, L, T, k, E, a.has_shared, tid);
    if (streamed && !moved) {
      // one token, routing as the logits ordered it: this group's expert,
      // presence and single entry (token 0, slot_mine) are known already
      if (e_mine < 0) {
        wait_vm();
        return;
      }
      gateup_wave(present_mine, row0, nrw, nbh, lpr, buf, xs,
                  [&](int, int& t, int& sl) { t = 0; sl = slot_mine; }, 1, stride, a.n_ff, a.h,
                  lane, a.out16 != nullptr);
      return;
    }
    n_groups = gbase + ctrl[1];
    if (!publisher) {
      const int e_x = g < n_groups ? pexp[g] : -1;
      if (e_x != e_mine) {  // a collision moved this group to another expert
        wait_vm();          // the speculative stream has landed; reuse the buffers
        bar();
        stream_rows(e_x, wave);
        e_mine = e_x;
      }
    }
  } else {
    if (publisher && T > 1) {  // the gate/up launch reads x quantized
      float xw[1][16];
      x_preload(a, nxb, wave, 4, lane, xw);
      quantize_x(a, nxb, a.xq, wave, 4, lane, xw);
    }
    for (int i = tid; i < T * k; i += 256) ridx[i] = a.idx[(i / k) * stride + (i % k)];
    for (int i = tid; i < T * stride; i += 256) rw[i] = a.weight[i];
    bar();
    make_plan(dyn, L, T, k, E, a.has_shared, tid);
    n_groups = gbase + ctrl[1];
    if (!publisher) {
      if (wave < 2) wait_vm();  // pointer tables
      bar();
      e_mine = g < n_groups ? pexp[g] : -1;
      stream_rows(e_mine, wave);
    }
  }

  if (publisher) {
    // publish idx, weight, plan and down pointers
    if (tabd_regs && wave == 2) {
      unsigned long long* td = reinterpret_cast<unsigned long long*>(dyn + L.tabd);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (lane + 64 * j < E) td[lane + 64 * j] = tdv[j];
    }
    wait_vm();  // pointer tables
    bar();
    // one array per wave, each lane's loads independent of the others' (a
    // single wave doing all of it waited on one LDS read after another)
    const int* re = reinterpret_cast<const int*>(dyn + L.re);
    const int nv = ctrl[0];
    if (wave == 0) {
      for (int i = lane; i < T * stride; i += 64) {
        const int t = i / stride, q = i - t * stride;
        bool bad = false;  // bounds-kill: a row with an invalid id loses all its weights
        for (int kk = 0; kk < k; ++kk) bad |= re[t * k + kk] < 0;
        a.weight[i] = bad ? 0.f : rw[i];
        if (a.logits && q < k) a.idx[i] = ridx[t * k + q];
      }
    } else if (wave == 1) {
      for (int i = lane; i <= n_groups; i += 64) {
        a.plan.off[i] = poff[i];
        if (i < n_groups) {
          const int e = pexp[i];
          a.plan.expert[i] = e;
          const unsigned long long gp =
              e >= 0 ? tabg[e] : reinterpret_cast<unsigned long long>(a.sh_gate);
          const unsigned long long up =
              e >= 0 ? tabu[e] : reinterpret_cast<unsigned long long>(a.sh_up);
          const unsigned long long dp =
              e >= 0 ? tabd[e] : reinterpret_cast<unsigned long long>(a.sh_down);
          a.plan.wdown[i] = (gp && up) ? dp : 0ull;
          a.plan.wgate[i] = (gp && up) ? gp : 0ull;
          a.plan.wup[i] = (gp && up) ? up : 0ull;
        }
      }
    } else if (wave == 2) {
      for (int i = lane; i < (a.has_shared ? T : 0) + nv; i += 64) {
        a.plan.tok[i] = ptok[i];
        a.plan.slot[i] = pslot[i];
      }
    } else if (lane == 0) {
      a.plan.meta[0] = n_groups;
      a.plan.meta[1] = a.has_shared;
      a.plan.meta[2] = nv;
    }
    return;
  }
  if (g >= n_groups) {
    wait_vm();  // a stream may still be landing in this LDS
    return;
  }
  const int e = pexp[g];
  const bool present = tabg[e] != 0ull && tabu[e] != 0ull;
  if (!t1w) {
    quantize_x(a, nxb, xs, wave, nqw, lane, xpre);  // overlaps the weight stream
    bar();
  }
  const int j0 = poff[g];
  gateup_wave(present, row0, nrw, nbh, lpr, buf, xs,
              [&](int j, int& t, int& sl) { t = ptok[j0 + j]; sl = pslot[j0 + j]; },
              poff[g + 1] - j0, stride, a.n_ff, a.h, lane, a.out16 != nullptr);
}

// The decode model shape (one token, hidden 2048, n_ff 512, 256 experts,
// top-8): its instance sees these and the LDS layout as constants.
constexpr int kShapeHidden = 2048, kShapeFf = 512, kShapeE = 256, kShapeK = 8;
constexpr int kShapeWindow = 4;  // the verify window's tokens (one plus three drafts)

// The model shape with kT tokens, with or without a shared expert, as the
// launcher derives it (kT = 0: none).
// kIo: 0 = the buffers' precision read from the arguments; 1 = the fp32
// buffers (x, residual, out) and 2 = the fp16 ones, fixed at compile time so
// the other kind's branches compile away (their argument loads and tests
// otherwise sit on the one-token critical chain)
template <int kT, bool kSh, int kIo = 0>
__device__ __forceinline__ void apply_shape(LayerArgs& a) {
  if constexpr (kIo == 1) {
    a.x16 = nullptr;
    a.xq_in = nullptr;
    a.res16 = nullptr;
    a.out16 = nullptr;
  } else if constexpr (kIo == 2) {
    a.x = nullptr;
    a.residual = nullptr;
    a.out = nullptr;
  }
  if constexpr (kT > 0) {
    a.T = kT;
    a.has_shared = kSh;
    a.hidden = kShapeHidden;
    a.n_ff = kShapeFf;
    a.n_expert = kShapeE;
    a.k = kShapeK;
    a.gmax = (kT * kShapeK < kShapeE ? kT * kShapeK : kShapeE) + 1;
    a.emax = kT * kShapeK + kT;
    a.front_routed = front_lds(kT, kShapeHidden / kQK, kShapeE, kShapeK, true);
    a.front_shared = front_lds(kT, kShapeHidden / kQK, kShapeE, kShapeK, false);
  }
}
__host__ inline bool is_shape(int T, int hidden, int n_ff, int E, int k, int kT) {
  return T == kT && hidden == kShapeHidden && n_ff == kShapeFf && E == kShapeE && k == kShapeK;
}

template <int EPT, int NBH, bool kOne = false, int kShapeT = 0, bool kSh = false, int kIo = 0>
__global__ void __launch_bounds__(256) layer_front_kernel(LayerArgs args) {
  LayerArgs a = args;
  apply_shape<kShapeT, kSh, kIo>(a);
  __shared__ __attribute__((aligned(16))) uint32_t wbuf[4][64 * 36];
  extern __shared__ __attribute__((aligned(16))) uint32_t dyn[];
  // Row y of the grid runs group g.  With a shared expert its row comes
  // after the routed ones: workgroups are placed on CUs in grid order, so the
  // routed workgroups (the long routing chain) each get a CU of their own
  // and the shared expert's (no routing, done early) double up.
  // (one token only: the grid is then about one workgroup per CU; with more
  // tokens the shared expert's row stays first so it is not the tail)
  const int y = blockIdx.y;
  const int g = !kOne && a.publish_only
                    ? a.gmax
                    : ((!kOne && a.T != 1) || !a.has_shared || y >= a.gmax
                           ? y
                           : (y + 1 == a.gmax ? 0 : y + 1));
  front_body<EPT, NBH, kOne>(a, blockIdx.x, g, wbuf, dyn);
}

// Gate/up + SiLU of one (row chunk, group) from the plan the routing launch
// left in the workspace: several tokens (a verify window), where routing in
// every compute workgroup would cost more than a launch.  Grid (row chunks
// of 16, gmax); groups beyond the plan's count exit.
template <int NBH, int kShapeT = 0, bool kSh = false, int kIo = 0>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 8)))
layer_gateup_kernel(LayerArgs args) {
  LayerArgs a = args;
  apply_shape<kShapeT, kSh, kIo>(a);
  __shared__ __attribute__((aligned(16))) uint32_t wbuf[4][64 * 36];
  extern __shared__ __attribute__((aligned(16))) uint32_t dyn[];  // x0, then entry tok / slot
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int k = a.k, stride = k + 1, g = blockIdx.y, bx = blockIdx.x;
  const int nbh = NBH ? NBH : a.hidden / kQK, lpr = NBH ? pow2_ceil(NBH) : pow2_ceil(nbh);
  const int rpw = 32 / lpr;
  const int row0 = bx * 4 * rpw + wave * rpw;
  // (every chunk full when n_ff is a multiple of the workgroup's rows: then
  // a constant in the shape instances, and the copies need no lane masks)
  const bool full = a.n_ff % (4 * rpw) == 0;
  const int nrw = full ? rpw : max(0, min(rpw, a.n_ff - row0));
  const int xw = nbh * kXStride;
  // every plan word this workgroup needs in one round (g < gmax: inside
  // the plan arrays even past the live groups); the entry list too when it
  // fits one wave (lane = entry, the same in every wave), so no load waits
  // for off[]
  const int n_groups = a.plan.meta[0];
  const unsigned long long wg = a.plan.wgate[g], wu = a.plan.wup[g];
  const int off0 = a.plan.off[g], off1 = a.plan.off[g + 1];
  const bool ent1 = a.emax <= 64;
  const int v_tok = ent1 ? a.plan.tok[min(lane, a.emax - 1)] : 0;
  const int v_slot = ent1 ? a.plan.slot[min(lane, a.emax - 1)] : 0;
  if (g >= n_groups) return;
  const bool present = wg != 0ull && wu != 0ull;
  // entries of the group (clamped to the plan's capacity), at etok/eslot[j0 ..]
  const int j0 = min(max(off0, 0), a.emax);
  const int n = min(max(off1, j0), a.emax) - j0;
  if (present && nrw > 0)
    dma_gateup(reinterpret_cast<const sg_block_q4k*>(wg), reinterpret_cast<const sg_block_q4k*>(wu),
               row0, nrw, nbh, wbuf[wave], lane);
  // the first entry's x (quantized by the routing launch) beside the
  // weights, one copy instruction per wave
  uint32_t* x0 = dyn;
  if (n > 0) {
    const int t0 = ent1 ? __shfl(v_tok, j0, 64) : a.plan.tok[j0];
    const uint32_t* src = a.xq + static_cast<long long>(t0) * xw;
    dma_chunks([&](int c) { return reinterpret_cast<const char*>(src) + 16 * c; }, xw / 4, x0,
               lane, wave, 4);
  }
  int* etok = reinterpret_cast<int*>(dyn + ((xw + 3) & ~3));
  int* eslot = etok + a.emax;
  if (ent1) {
    if (tid < a.emax) {
      etok[tid] = v_tok;
      eslot[tid] = v_slot;
    }
  } else {
    for (int i = tid; i < n; i += 256) {
      etok[j0 + i] = a.plan.tok[j0 + i];
      eslot[j0 + i] = a.plan.slot[j0 + i];
    }
  }
  wait_vm();  // this wave's weights and its share of x0
  bar();
  gateup_group(present, row0, nrw, nbh, lpr, wbuf[wave], &wbuf[0][0], x0, a.xq,
               [&](int j, int& t, int& sl) { t = etok[j0 + j]; sl = eslot[j0 + j]; }, n, stride,
               a.n_ff, a.h, lane, wave, a.out16 != nullptr);
  if (g == 0 && a.has_shared && a.sh_gate_w && bx == 0) shared_gate_tokens(a, tid);
}

// ---- back kernel ------------------------------------------------------------------------
// One workgroup per chunk of `rows` output rows (hidden/rows >= 256 where the
// shape allows).  A wave packs `gpw` groups side by side - lane = (group,
// row, super-block) - and streams their down rows for the chunk into its LDS
// buffer while all eight waves quantize every (token, slot) h row to Q8_K in
// LDS (h was loaded at kernel start, beside the plan).  The slot outputs of
// the chunk go to LDS; then the workgroup combines
// out = residual + sum_kk fma(w_kk, y_kk) in slot order.
constexpr int kBackWaves = 8;                    // waves per back workgroup
constexpr int kBackThreads = 64 * kBackWaves;
constexpr int kBackPreCopies = 3;  // copy instructions per wave issued at kernel start
constexpr int kBackHSlots = 3;  // h blocks per wave preloaded at kernel start (T = 1, k = 8: 18)

struct BackLds {
  int hq, ys, off, wdown, tok, slot, wt, sg, meta, total;
};

__host__ __device__ constexpr BackLds back_lds(int T, int k, int n_ff, int rows, int gmax,
                                               int emax) {
  BackLds L{};
  const int nbf = n_ff / kQK;
  int o = 0;
  auto take = [&](int words) {
    o = (o + 3) & ~3;
    const int at = o;
    o += words;
    return at;
  };
  L.hq = take(T * (k + 1) * nbf * kXStride);
  L.ys = take(T * (k + 1) * rows);
  L.off = take(gmax + 1);
  L.wdown = take(gmax * 2);
  L.tok = take(emax);
  L.slot = take(emax);
  L.wt = take(T * (k + 1));
  L.sg = take(T);
  L.meta = take(4);
  L.total = (o + 3) & ~3;  // the down-row buffers follow, 16-B aligned
  return L;
}

// Q8_K of every (token, slot) h row of the back kernel into hq (LDS): wave w
// quantizes blocks e = w + 8j, j < HS from hpre (its registers) in
// one interleaved pass (every block of a one-token layer with k <= 8), later
// ones in passes of four loaded here.
template <int HS>
__device__ __forceinline__ void back_quantize_h(const LayerArgs& a, uint32_t* hq,
                                                const float (&hpre)[HS][4], int nq,
                                                int wave, int lane) {
  if (wave < nq) {
    uint32_t* dst[HS];
    int n = 0;
#pragma unroll
    for (int j = 0; j < HS; ++j) {
      const int e = wave + kBackWaves * j;
      dst[j] = hq + (e < nq ? e : wave) * kXStride;
      n += e < nq;
    }
    quantize_n_lds<HS>(hpre, dst, n, lane);
  }
  for (int e0 = wave + kBackWaves * HS; e0 < nq; e0 += 4 * kBackWaves) {
    float v[4][4];
    uint32_t* dst[4];
    int n = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int e = e0 + kBackWaves * u < nq ? e0 + kBackWaves * u : e0;
      const float* hp = a.h + static_cast<long long>(e) * kQK + 4 * lane;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[u][i] = hp[i];
      dst[u] = hq + e * kXStride;
      n += e0 + kBackWaves * u < nq;
    }
    quantize_n_lds<4>(v, dst, n, lane);
  }
}

// The down rows, Q8_K of h and combine of one chunk of `rows` output rows,
// with the plan in LDS (off, wdown, tok, slot, wt, meta).  Wave w
// quantizes h blocks w + 8j; hpre[j] holds the lane's 4 values of block
// w + 8j for j < HS (loaded at kernel start).
// NBF, ROWS: n_ff / 256 and the rows per workgroup when known at compile
// time (0 = read from a).  pre: the kernel start has already issued every
// group's down-row copies (the packed one-pass layout) and quantized h,
// and the barrier after them has passed.
template <int NBF, int ROWS, int HS>
__device__ __forceinline__ void back_core(const LayerArgs& a, const BackLds& L, uint32_t* bd,
                          uint32_t (*wbuf)[64 * 36], int row0, int nr, float res0,
                          const float (&hpre)[HS][4], bool pre) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int T = a.T, k = a.k, stride = k + 1;
  const int nbf = NBF ? NBF : a.n_ff / kQK;
  const int rows = ROWS ? ROWS : a.back_rows;
  const int lrow = NBF ? pow2_ceil(NBF) : a.back_lrow;
  const int gpw = 64 / (rows * lrow);  // groups per wave per pass
  uint32_t* hq = bd + L.hq;
  float* ys = reinterpret_cast<float*>(bd + L.ys);
  const int* off = reinterpret_cast<const int*>(bd + L.off);
  const unsigned long long* wdown = reinterpret_cast<const unsigned long long*>(bd + L.wdown);
  const int* tok = reinterpret_cast<const int*>(bd + L.tok);
  const int* slot = reinterpret_cast<const int*>(bd + L.slot);
  const float* wt = reinterpret_cast<const float*>(bd + L.wt);
  const float* sgl = reinterpret_cast<const float*>(bd + L.sg);
  const int* meta = reinterpret_cast<const int*>(bd + L.meta);
  const int nq = T * stride * nbf;
  const int n_out = T * nr;
  const int G = __builtin_amdgcn_readfirstlane(meta[0]);
  const int gwords = rows * nbf * 36;  // one group's rows in the buffer
  uint32_t* buf = wbuf[wave];
  const int q = lane / (rows * lrow);  // this lane's group within the wave
  const int rr = (lane / lrow) % rows, blk = lane & (lrow - 1);

  const int nbw = a.back_bufs;  // waves that stream and dot down rows
  // one pass with every buffer packed end to end: the copies are dealt to
  // all waves rather than issued by the waves that will read them
  const bool spread = G <= nbw * gpw && gpw * gwords == 64 * 36;
  // The packed one-pass layout with every group in one pass (the one-token
  // model shape): each super-block dot is split over two lanes, so that the
  // dots of the G groups spread over 16 G lanes (up to eight waves) instead
  // of 8 G.  Lane (rr, blk, hf) of a 32-lane group computes sub-blocks
  // 4 hf .. 4 hf + 3 of row rr's block blk; the block's fp32 chain (sum =
  // fma(xd, t_s, sum), s = 0..7) runs over lane hf = 0 and then, one DPP
  // shift later, lane hf = 1; the row's block sums are added in block order
  // one more shift later (row_sum_last's order).  The same operations as the
  // one-lane form, so the same bits.
  if (pre && spread && NBF == 2 && G <= 2 * kBackWaves) {
    const int gq = 2 * wave + (lane >> 5);
    const int rr2 = (lane >> 2) & 7, blk2 = (lane >> 1) & 1, hf = lane & 1;
    const bool has = gq < G && rr2 < rows;
    const bool present = has && wdown[gq] != 0ull;
    const bool live = present && rr2 < nr;
    const uint32_t* wb = wbuf[0] + gq * gwords + 36 * (rr2 * 2 + blk2);
    uint32_t wq[16];
    uint32_t dd = 0;
    ScaleMins sm8{};
    if (live) {
      const u32x4* w4 = reinterpret_cast<const u32x4*>(wb);
      const u32x4 hd = w4[0];
      dd = hd.x;
      sm8 = unpack_scales(hd.y, hd.z, hd.w);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4 v = w4[1 + 4 * hf + i];
        wq[4 * i] = v.x;
        wq[4 * i + 1] = v.y;
        wq[4 * i + 2] = v.z;
        wq[4 * i + 3] = v.w;
      }
    }
    const float d = half_bits_to_float(dd & 0xFFFFu);
    const float dmin = half_bits_to_float(dd >> 16);
    const int jb = has ? min(max(off[gq], 0), a.emax) : 0;
    const int je = has ? min(max(off[gq + 1], jb), a.emax) : 0;
    const int cnt = wave_max_i32(je - jb);
    for (int ji = 0; ji < cnt; ++ji) {
      const int j = jb + ji;
      const bool ok = j < je;
      const int hs = ok ? tok[j] * stride + slot[j] : 0;
      float part = 0.f;  // hf = 0: the chain of sub-blocks 0..3 from 0
      float tv[4] = {0.f, 0.f, 0.f, 0.f};
      float xd = 0.f;
      if (live && ok) {
        const uint32_t* xb = hq + (hs * 2 + blk2) * kXStride;
        const u32x4* x4 = reinterpret_cast<const u32x4*>(xb + 32 * hf);
        int32_t xw[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const u32x4 v = x4[i];
          xw[4 * i] = static_cast<int32_t>(v.x);
          xw[4 * i + 1] = static_cast<int32_t>(v.y);
          xw[4 * i + 2] = static_cast<int32_t>(v.z);
          xw[4 * i + 3] = static_cast<int32_t>(v.w);
        }
        xd = __builtin_bit_cast(float, xb[64]);
        int32_t ip[4];
#pragma unroll
        for (int g = 0; g < 2; ++g) {  // sub-block group 2 hf + g: sub-blocks 4 hf + 2g, + 1
          int32_t lo = 0, hi = 0;
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) {
            const uint32_t w = wq[8 * g + jj];
            lo = __builtin_amdgcn_sdot4(static_cast<int>(w & 0x0F0F0F0Fu), xw[16 * g + jj], lo,
                                        false);
            hi = __builtin_amdgcn_sdot4(static_cast<int>((w >> 4) & 0x0F0F0F0Fu),
                                        xw[16 * g + 8 + jj], hi, false);
          }
          ip[2 * g] = lo;
          ip[2 * g + 1] = hi;
        }
        const uint32_t scw = hf ? sm8.sc_hi : sm8.sc_lo;
        const uint32_t mnw = hf ? sm8.mn_hi : sm8.mn_lo;
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
          const float sd = d * byte_f(scw, s4);
          const float smv = dmin * byte_f(mnw, s4);
          const float bs = __builtin_bit_cast(float, xb[65 + 4 * hf + s4]);
          tv[s4] = __builtin_fmaf(sd, static_cast<float>(ip[s4]), -(smv * bs));
        }
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) part = __builtin_fmaf(xd, tv[s4], part);
      }
      // hf = 1 continues the chain from lane hf = 0's partial sum
      const float prev = dpp_f<0x111>(part);  // row_shr:1 (lane - 1, within 16-lane rows)
      float bsum = part;
      if (hf == 1) {
        bsum = prev;
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) bsum = __builtin_fmaf(xd, tv[s4], bsum);
      }
      // row sum in block order: 0 + block 0, then + block 1 (lanes hf = 1)
      const float acc0 = 0.f + bsum;
      const float prev2 = dpp_f<0x112>(acc0);  // row_shr:2: block 0's lane to block 1's
      const float acc = blk2 == 1 ? prev2 + bsum : acc0;
      if (ok && has && hf == 1 && blk2 == 1 && rr2 < nr) ys[hs * rows + rr2] = present ? acc : 0.f;
    }
  } else
  for (int gb = 0; gb < G; gb += nbw * gpw) {
    if (spread) {
      // every group's down rows as one run of 16-B chunks over all the
      // buffers (chunk c = group c / cpg, chunk c % cpg of its rows, at
      // wbuf[0] + 4c), the 1-KB copy instructions dealt round-robin to the
      // waves; each waits for its own before the barrier below
      if (gb == 0 && !pre) {
        const int cpg = gwords / 4, cval = nr * nbf * 9, total = G * cpg;
        const uint64_t inv = ((1ull << 24) + cpg - 1) / cpg;  // c / cpg exact for c < 2^24 / cpg
        const long long roff = static_cast<long long>(row0) * nbf * kQ4Bytes;
        for (int t = wave; 64 * t < total; t += kBackWaves) {
          const int c = 64 * t + lane;
          const int gq = static_cast<int>((static_cast<uint64_t>(c) * inv) >> 24);
          const int w = c - gq * cpg;
          const unsigned long long wd = c < total ? wdown[gq] : 0ull;
          if (wd && w < cval)
            __builtin_amdgcn_global_load_lds(
                (glb_void_p)(reinterpret_cast<const char*>(wd) + roff + 16 * w),
                (lds_void_p)(wbuf[0] + 256 * t), 16, 0, kNt);
        }
      }
    } else {
      // down rows of this wave's gpw groups as one run of 16-B chunks: chunk
      // c = group c / cpg, chunk c % cpg of the group's rows; LDS destination
      // buf + 4c (group qq at buf + qq * gwords).  At most 9 copy
      // instructions, no loop over groups.
      const int cpg = gwords / 4;       // chunks per group slot
      const int cval = nr * nbf * 9;    // chunks present (nr < rows at the edge)
      const uint32_t inv = ((1u << 20) + cpg - 1) / cpg;  // c / cpg exact for c < 576
      const long long roff = static_cast<long long>(row0) * nbf * kQ4Bytes;
#pragma unroll
      for (int i = 0; i < 9; ++i) {
        const int c = lane + 64 * i;
        if (64 * i >= gpw * cpg) break;
        const int qq = static_cast<int>((static_cast<uint32_t>(c) * inv) >> 20);
        const int w = c - qq * cpg;
        const int gq = gb + wave * gpw + qq;
        const unsigned long long wd = qq < gpw && gq < G && wave < nbw ? wdown[gq] : 0ull;
        if (wd && w < cval)
          __builtin_amdgcn_global_load_lds(
              (glb_void_p)(reinterpret_cast<const char*>(wd) + roff + 16 * w),
              (lds_void_p)(buf + 256 * i), 16, 0, kNt);
      }
    }
    if (gb == 0 && !pre) {  // Q8_K of every (token, slot) h row while the rows stream in
      back_quantize_h<HS>(a, hq, hpre, nq, wave, lane);
      if (spread) wait_vm();  // this wave's share of the copies
      bar();
    }
    wait_vm();
    const int gq = gb + wave * gpw + q;
    const bool has = gq < G && wave < nbw;
    const bool present = has && wdown[gq] != 0ull;
    const bool live = present && blk < nbf && rr < nr;
    uint32_t w36[36];
    ScaleMins sm8{};
    if (live) {
      read_block_lds(buf + q * gwords + 36 * (rr * nbf + blk), w36);
      sm8 = unpack_scales(w36[1], w36[2], w36[3]);
    }
    // entries of the group, clamped to the plan's capacity (a plan is only
    // ever read here, never trusted to bound a loop)
    const int jb = has ? min(max(off[gq], 0), a.emax) : 0;
    const int je = has ? min(max(off[gq + 1], jb), a.emax) : 0;
    const int cnt = wave_max_i32(je - jb);
    for (int ji = 0; ji < cnt; ++ji) {
      const int j = jb + ji;
      const bool ok = j < je;
      const int hs = ok ? tok[j] * stride + slot[j] : 0;
      float s = 0.f;
      if (live && ok) {
        int32_t xr[64], ip[8];
        float xd, bsf[8];
        load_x_regs(hq + (hs * nbf + blk) * kXStride, xr, xd, bsf);
        subblock_dots(w36 + 4, xr, ip);
        s = block_sum(w36[0], sm8, ip, xd, bsf);
      }
      const float acc = row_sum_last(s, blk, nbf);
      if (ok && blk == nbf - 1 && rr < nr) ys[hs * rows + rr] = present ? acc : 0.f;
    }
    wait_lds();
  }
  bar();
  // out = residual + sum over slots 0..k of fma(w, y) in slot order.  A slot
  // whose id was invalid (bounds-killed), whose expert is absent, or the
  // shared slot without a shared expert has no plan entry, so its y is the
  // 0 the prologue stored.
  for (int qo = tid; qo < n_out; qo += kBackThreads) {
    const int t = qo / nr, r = qo - t * nr;
    const long long o = static_cast<long long>(t) * a.hidden + row0 + r;
    float acc = qo == tid ? res0
                          : (a.residual ? a.residual[o] : (a.res16 ? f16v(a.res16[o]) : 0.f));
    // the shared slot's output scaled by its gate first (1.0 without a
    // gate, which leaves it unchanged), as sigmoid_gate_scalar_batched_f16
    // does before the combine (session.cpp:2904-2909)
    const float gs = sgl[t];
    for (int k0 = 0; k0 <= k; k0 += 16) {  // gather 16 slots, then the ordered fma chain
      float yv[16], wv[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int i = t * stride + (k0 + u <= k ? k0 + u : k);
        yv[u] = ys[i * rows + r];
        wv[u] = wt[i];
        if (a.out16) {  // fp16 slot outputs; the shared one gated on its fp16 value
          yv[u] = f16v(f16b(yv[u]));
          if (k0 + u == k) yv[u] = f16v(f16b(yv[u] * gs));
        } else if (k0 + u == k) {
          yv[u] *= gs;
        }
      }
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (k0 + u <= k) acc = __builtin_fmaf(wv[u], yv[u], acc);
    }
    if (a.out16) a.out16[o] = f16b(acc);
    else a.out[o] = acc;
  }
}

// residual of the first combine pass (qo = tid), loaded early
__device__ __forceinline__ float residual_pre(const LayerArgs& a, int row0, int nr) {
  const int tid = threadIdx.x;
  if ((!a.residual && !a.res16) || tid >= a.T * nr) return 0.f;
  const int t = tid / nr, r = tid - t * nr;
  const long long o = static_cast<long long>(t) * a.hidden + row0 + r;
  return a.residual ? a.residual[o] : f16v(a.res16[o]);
}

template <int NBF, int ROWS, int kShapeT = 0, bool kSh = false, int kIo = 0>
__global__ void __launch_bounds__(kBackThreads) layer_back_kernel(LayerArgs args) {
  // kShapeT > 0 (the model shape with kShapeT tokens, as in the front
  // kernel): the shape and the LDS layout are constants
  LayerArgs a = args;
  apply_shape<kShapeT, kSh, kIo>(a);
  if constexpr (kShapeT > 0) {
    a.back_rows = 8;
    a.back_lrow = 2;
    a.back_bufs = kBackWaves;
  }
  extern __shared__ __attribute__((aligned(16))) uint32_t dyn[];  // BackLds arrays, then the buffers
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int T = a.T, k = a.k, stride = k + 1;
  const int nbf = NBF ? NBF : a.n_ff / kQK;
  const int rows = ROWS ? ROWS : a.back_rows;
  const BackLds L = back_lds(T, k, a.n_ff, rows, a.gmax, a.emax);
  int* off = reinterpret_cast<int*>(dyn + L.off);
  unsigned long long* wdown = reinterpret_cast<unsigned long long*>(dyn + L.wdown);
  int* tok = reinterpret_cast<int*>(dyn + L.tok);
  int* slot = reinterpret_cast<int*>(dyn + L.slot);
  float* wt = reinterpret_cast<float*>(dyn + L.wt);
  float* sgl = reinterpret_cast<float*>(dyn + L.sg);
  int* meta = reinterpret_cast<int*>(dyn + L.meta);
  float* ys = reinterpret_cast<float*>(dyn + L.ys);
  const int row0 = blockIdx.x * rows;
  const int nr = max(0, min(rows, a.hidden - row0));

  // loads that do not depend on the plan: this wave's first HS h
  // blocks (block wave + 8j of the (token, slot) rows) and the residual
  const int nq = T * stride * nbf;
  constexpr int HS = kShapeT == kShapeWindow ? 9 : kBackHSlots;  // the window: every block
  float hpre[HS][4];
  if (wave < nq) {
#pragma unroll
    for (int j = 0; j < HS; ++j) {
      const int e0 = wave + kBackWaves * j;
      const int e = e0 < nq ? e0 : wave;
      const float* hp = a.h + static_cast<long long>(e) * kQK + 4 * lane;
#pragma unroll
      for (int i = 0; i < 4; ++i) hpre[j][i] = hp[i];
    }
  }
  const float res0 = residual_pre(a, row0, nr);

  // The packed one-pass copy layout of back_core, when the plan fits it
  // (its groups within the copy instructions issued here): each thread
  // loads the down pointers of its
  // chunks and the group count straight from the plan in global memory, so
  // the copies are issued as soon as those land, and h is quantized before
  // the first barrier.
  const int lrow = NBF ? pow2_ceil(NBF) : a.back_lrow;
  const int gpw = 64 / (rows * lrow);
  const int gwords = rows * nbf * 36, cpg = gwords / 4;
  // (PC copy instructions per wave: the groups they hold, cap, cover every
  // plan of the one-token shape; whether a plan fits is decided once its
  // group count has landed.  Nine per wave for the window's 32 groups
  // measured slower than the copies of back_core.)
  constexpr int PC = kBackPreCopies;
  const int cap = min(a.back_bufs * gpw, 64 * kBackWaves * PC / cpg);
  const bool pre_cand = kShapeT != kShapeWindow && gpw * gwords == 64 * 36 && cap > 0;
  const uint64_t inv = ((1ull << 24) + cpg - 1) / cpg;  // c / cpg exact for c < 2^24 / cpg
  // (with up to 64 groups every wave loads them all, lane = group, and
  // takes each chunk's pointer by a lane permute; otherwise one load per
  // chunk)
  const bool wd_lanes = a.gmax <= 64;
  unsigned long long wdl = 0ull;
  unsigned long long wdp[PC];
  int gpre = 0;
  if (pre_cand) {
    gpre = max(0, min(a.plan.meta[0], a.gmax));
    if (wd_lanes) {
      wdl = a.plan.wdown[min(lane, a.gmax - 1)];
    } else {
#pragma unroll
      for (int i = 0; i < PC; ++i) {
        const int c = 64 * (wave + kBackWaves * i) + lane;
        const int gq = static_cast<int>((static_cast<uint64_t>(c) * inv) >> 24);
        wdp[i] = a.plan.wdown[min(gq, a.gmax - 1)];
      }
    }
  }

  // the plan and routing weights.  When every array fits one element per
  // thread, each thread issues all of its loads (clamped indices, no
  // branches) before it waits once; loads inside separate guarded loops
  // would each wait for the previous one.
  const int nw = T * stride;
  if (a.gmax + 1 <= kBackThreads && a.emax <= kBackThreads && nw <= kBackThreads) {
    const int v_meta = a.plan.meta[min(tid, 1)];
    const int v_off = a.plan.off[min(tid, a.gmax)];
    const unsigned long long v_wd = a.plan.wdown[min(tid, a.gmax - 1)];
    const int v_tok = a.plan.tok[min(tid, a.emax - 1)];
    const int v_slot = a.plan.slot[min(tid, a.emax - 1)];
    const float v_wt = a.weight[min(tid, nw - 1)];
    const float v_sg = a.sgate ? a.sgate[min(tid, T - 1)] : 1.f;
    if (tid < 2) meta[tid] = v_meta;
    if (tid <= a.gmax) off[tid] = v_off;
    if (tid < a.gmax) wdown[tid] = v_wd;
    if (tid < a.emax) {
      tok[tid] = v_tok;
      slot[tid] = v_slot;
    }
    if (tid < nw) wt[tid] = v_wt;
    if (tid < T) sgl[tid] = v_sg;
  } else {
    if (tid < 2) meta[tid] = a.plan.meta[tid];
    for (int i = tid; i <= a.gmax; i += kBackThreads) off[i] = a.plan.off[i];
    for (int i = tid; i < a.gmax; i += kBackThreads) wdown[i] = a.plan.wdown[i];
    for (int i = tid; i < a.emax; i += kBackThreads) {
      tok[i] = a.plan.tok[i];
      slot[i] = a.plan.slot[i];
    }
    for (int i = tid; i < nw; i += kBackThreads) wt[i] = a.weight[i];
    for (int i = tid; i < T; i += kBackThreads) sgl[i] = a.sgate ? a.sgate[i] : 1.f;
  }
  uint32_t(*wbuf)[64 * 36] = reinterpret_cast<uint32_t(*)[64 * 36]>(dyn + L.total);
  const bool pre = pre_cand && gpre <= cap;
  if (pre) {
    // chunk c = 64 t + lane, t = wave + 8i: group c / cpg, chunk c % cpg of
    // its rows, to wbuf[0] + 4c (what back_core's packed layout reads)
    const int cval = nr * nbf * 9, total = gpre * cpg;
    const long long roff = static_cast<long long>(row0) * nbf * kQ4Bytes;
#pragma unroll
    for (int i = 0; i < PC; ++i) {
      const int t = wave + kBackWaves * i;
      const int c = 64 * t + lane;
      const int gq = static_cast<int>((static_cast<uint64_t>(c) * inv) >> 24);
      const int w = c - gq * cpg;
      unsigned long long wd;
      if (wd_lanes) {
        const int src = 4 * min(gq, 63);
        const unsigned lo = __builtin_amdgcn_ds_bpermute(src, static_cast<int>(wdl));
        const unsigned hi = __builtin_amdgcn_ds_bpermute(src, static_cast<int>(wdl >> 32));
        wd = (static_cast<unsigned long long>(hi) << 32) | lo;
      } else {
        wd = wdp[i];
      }
      if (c < total && wd && w < cval)
        __builtin_amdgcn_global_load_lds(
            (glb_void_p)(reinterpret_cast<const char*>(wd) + roff + 16 * w),
            (lds_void_p)(wbuf[0] + 256 * t), 16, 0, kNt);
    }
    if (tid == 0) meta[0] = gpre;
  }
  for (int i = tid; i < T * stride * rows; i += kBackThreads) ys[i] = 0.f;
  if (pre) {
    back_quantize_h<HS>(a, dyn + L.hq, hpre, nq, wave, lane);
    wait_vm();  // this wave's copies, visible to all after the barrier
  }
  bar();
  back_core<NBF, ROWS, HS>(a, L, dyn, wbuf, row0, nr, res0, hpre, pre);
}

static void back_geometry(int hidden, int n_ff, int& rows, int& lrow) {
  lrow = pow2_ceil(n_ff / kQK);      // lanes per row: one per super-block
  int r = 64 / lrow;                 // rows that fill a wave for one group
  while (r > 1 && hidden / r < 256) r >>= 1;  // at least 256 workgroups when possible
  rows = r;
}

// ---- the allocation-free layer: scratch in a file-scope device array ------------
// One 1 MiB array per GPU, held until the process ends; sg_moe_layer_noalloc
// uses it as the layer workspace.  Its device address is looked up once per
// device (hipGetSymbolAddress with that device current) and kept per device:
// in host code `scratch` names a host-side stand-in, never the device memory.
constexpr size_t kScratchBytes = size_t(1) << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// the current device's address of `scratch`
static int scratch_address(void** out, const char* nm) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return set_error(SG_ERR_HIP, "%s: hipGetDevice: %s", nm, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(SG_ERR_UNSUPPORTED, "%s: device %d beyond %d", nm, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(SG_ERR_HIP, "%s: hipGetSymbolAddress(scratch): %s", nm,
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SG_OK;
}

// the layer's activation and output buffers: fp32 (x, residual, out) or the
// session's fp16 ones (x16 and/or its Q8_K xq, res16, out16)
struct LayerIo {
  const float* x;
  const uint16_t* x16;
  const unsigned char* xq;
  const float* residual;
  float* out;
  const uint16_t* res16;
  uint16_t* out16;
};

static int layer_launch(const sg_block_q4k* const* tab_gate, const sg_block_q4k* const* tab_up,
                        const sg_block_q4k* const* tab_down, const sg_block_q4k* sh_gate,
                        const sg_block_q4k* sh_up, const sg_block_q4k* sh_down,
                        const float* sh_gate_w, const LayerIo& io, const float* logits, int* idx,
                        float* weight, void* workspace, size_t workspace_bytes, int n_tokens,
                        int hidden, int n_ff, int n_expert, int k, float shared_w, int stages,
                        void* stream, const char* nm);

}  // namespace sg

using namespace sg;

extern "C" {

size_t sg_moe_layer_workspace_bytes(int n_tokens, int hidden, int n_ff, int n_expert, int k) {
  if (n_tokens <= 0 || hidden <= 0 || n_ff <= 0 || n_expert <= 0 || k <= 0) return 0;
  return layer_ws(n_tokens, hidden, n_ff, n_expert, k).total;
}

int sg_moe_layer_stages(const sg_block_q4k* const* tab_gate, const sg_block_q4k* const* tab_up,
                        const sg_block_q4k* const* tab_down, const sg_block_q4k* sh_gate,
                        const sg_block_q4k* sh_up, const sg_block_q4k* sh_down,
                        const float* sh_gate_w, const float* x, const float* logits,
                        const float* residual, float* out, int* idx, float* weight,
                        void* workspace, size_t workspace_bytes, int n_tokens, int hidden,
                        int n_ff, int n_expert, int k, float shared_w, int stages,
                        void* stream) {
  const char* nm = "sg_moe_layer";
  if (!x || !out) return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  return layer_launch(tab_gate, tab_up, tab_down, sh_gate, sh_up, sh_down, sh_gate_w,
                      LayerIo{x, nullptr, nullptr, residual, out, nullptr, nullptr}, logits, idx,
                      weight, workspace, workspace_bytes, n_tokens, hidden, n_ff, n_expert, k,
                      shared_w, stages, stream, nm);
}

int sg_moe_layer_f16(const sg_block_q4k* const* tab_gate, const sg_block_q4k* const* tab_up,
                     const sg_block_q4k* const* tab_down, const sg_block_q4k* sh_gate,
                     const sg_block_q4k* sh_up, const sg_block_q4k* sh_down,
                     const float* sh_gate_w, const uint16_t* xn, const sg_block_q8k* xq,
                     const float* logits, const uint16_t* residual, uint16_t* out, int* idx,
                     float* weight, void* workspace, size_t workspace_bytes, int n_tokens,
                     int hidden, int n_ff, int n_expert, int k, float shared_w, void* stream) {
  const char* nm = "sg_moe_layer_f16";
  if ((!xn && !xq) || !out) return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  if (!xn && sh_gate_w && sh_gate && sh_up && sh_down)
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: the shared gate needs xn", nm);
  return layer_launch(tab_gate, tab_up, tab_down, sh_gate, sh_up, sh_down, sh_gate_w,
                      LayerIo{nullptr, xn, reinterpret_cast<const unsigned char*>(xq), nullptr,
                              nullptr, residual, out},
                      logits, idx, weight, workspace, workspace_bytes, n_tokens, hidden, n_ff,
                      n_expert, k, shared_w, 3, stream, nm);
}

}  // extern "C"

namespace sg {

static int layer_launch(const sg_block_q4k* const* tab_gate, const sg_block_q4k* const* tab_up,
                        const sg_block_q4k* const* tab_down, const sg_block_q4k* sh_gate,
                        const sg_block_q4k* sh_up, const sg_block_q4k* sh_down,
                        const float* sh_gate_w, const LayerIo& io, const float* logits, int* idx,
                        float* weight, void* workspace, size_t workspace_bytes, int n_tokens,
                        int hidden, int n_ff, int n_expert, int k, float shared_w, int stages,
                        void* stream, const char* nm) {
  if (stages <= 0 || stages > 3)
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: stages=%d not in 1..3", nm, stages);
  if (!tab_gate || !tab_up || !tab_down || !idx || !weight || !workspace)
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", nm);
  const int n_sh = (sh_gate != nullptr) + (sh_up != nullptr) + (sh_down != nullptr);
  if (n_sh != 0 && n_sh != 3)
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: shared expert needs gate, up and down", nm);
  if (n_tokens <= 0 || n_tokens > kLMaxTokens)
    return set_error(SG_ERR_UNSUPPORTED, "%s: n_tokens=%d not in [1,%d]", nm, n_tokens,
                     kLMaxTokens);
  if (hidden <= 0 || hidden % kQK || n_ff <= 0 || n_ff % kQK)
    return set_error(SG_ERR_GEOMETRY, "%s: hidden=%d n_ff=%d must be multiples of 256", nm, hidden,
                     n_ff);
  if (hidden > 32 * kQK || n_ff > 64 * kQK)
    return set_error(SG_ERR_UNSUPPORTED, "%s: hidden=%d (<=8192) n_ff=%d (<=16384)", nm, hidden,
                     n_ff);
  if (k <= 0 || k > kLMaxK || n_expert < k || n_expert > kLMaxExperts)
    return set_error(SG_ERR_GEOMETRY, "%s: k=%d (<=%d) n_expert=%d (k..%d)", nm, k, kLMaxK,
                     n_expert, kLMaxExperts);
  int rows = 1, lrow = 64;
  back_geometry(hidden, n_ff, rows, lrow);
  const LayerWs ws = layer_ws(n_tokens, hidden, n_ff, n_expert, k);
  if (workspace_bytes < ws.total)
    return set_error(SG_ERR_INVALID_ARGUMENT, "%s: workspace %zu < %zu bytes", nm,
                     workspace_bytes, ws.total);
  const size_t lds_f =
      static_cast<size_t>(front_lds(n_tokens, hidden / kQK, n_expert, k, true).total) * 4;
  const size_t lds_b =
      static_cast<size_t>(back_lds(n_tokens, k, n_ff, rows, ws.gmax, ws.emax).total) * 4;
  // the back kernel's down-row buffers: one per wave when they fit, else four
  const size_t buf_b = 64 * 36 * 4;
  const int back_bufs = lds_b + kBackWaves * buf_b <= 160 * 1024 ? kBackWaves : 4;
  if (lds_f + 4 * buf_b > 160 * 1024 || lds_b + back_bufs * buf_b > 160 * 1024)
    return set_error(SG_ERR_UNSUPPORTED, "%s: this shape needs more LDS than a workgroup has",
                     nm);
  unsigned char* base = static_cast<unsigned char*>(workspace);
  LayerArgs a{};
  a.tab_gate = tab_gate;
  a.tab_up = tab_up;
  a.tab_down = tab_down;
  a.sh_gate = sh_gate;
  a.sh_up = sh_up;
  a.sh_down = sh_down;
  // the gate scales the shared expert only: without one it has nothing to scale
  a.sh_gate_w = n_sh == 3 ? sh_gate_w : nullptr;
  a.x = io.x;
  a.x16 = io.x16;
  a.xq_in = io.xq;
  a.logits = logits;
  a.residual = io.residual;
  a.out = io.out;
  a.res16 = io.res16;
  a.out16 = io.out16;
  const bool f32io = io.x != nullptr;  // the fp32 entry (else the fp16 one)
  a.idx = idx;
  a.weight = weight;
  a.plan = LayerPlan{reinterpret_cast<int*>(base + ws.meta), reinterpret_cast<int*>(base + ws.off),
                     reinterpret_cast<int*>(base + ws.expert),
                     reinterpret_cast<int*>(base + ws.tok), reinterpret_cast<int*>(base + ws.slot),
                     reinterpret_cast<unsigned long long*>(base + ws.wdown),
                     reinterpret_cast<unsigned long long*>(base + ws.wgate),
                     reinterpret_cast<unsigned long long*>(base + ws.wup)};
  a.h = reinterpret_cast<float*>(base + ws.h);
  a.xq = n_tokens > 1 ? reinterpret_cast<uint32_t*>(base + ws.xq) : nullptr;
  a.sgate = a.sh_gate_w ? reinterpret_cast<float*>(base + ws.sgate) : nullptr;
  a.T = n_tokens;
  a.hidden = hidden;
  a.n_ff = n_ff;
  a.n_expert = n_expert;
  a.k = k;
  a.has_shared = n_sh == 3;
  a.gmax = ws.gmax;
  a.emax = ws.emax;
  a.shared_w = shared_w;
  a.back_rows = rows;
  a.back_lrow = lrow;
  a.back_bufs = back_bufs;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int rows_wg = 4 * (32 / pow2_ceil(hidden / kQK));
  const FrontLds fl = front_lds(n_tokens, hidden / kQK, n_expert, k, true);
  a.front_routed = fl;
  a.front_shared = front_lds(n_tokens, hidden / kQK, n_expert, k, false);
  // several tokens: routing launch (the publisher alone), then the gate/up
  // launch reading its plan; one token: one fused launch whose compute
  // workgroups route speculatively beside their weight stream
  // the gate/up launch: the first entry's x, then the entries
  const size_t lds_g = static_cast<size_t>((((hidden / kQK) * kXStride + 3) & ~3) + 2 * ws.emax) * 4;
  a.publish_only = n_tokens > 1;
  if (a.publish_only && lds_g + 4 * buf_b > 160 * 1024)
    return set_error(SG_ERR_UNSUPPORTED, "%s: this shape needs more LDS than a workgroup has",
                     nm);
  if (stages & 1) {
    // y < gmax: compute workgroups of group y; y == gmax: the publisher
    const dim3 grid = a.publish_only ? dim3(1, 1)
                                     : dim3((n_ff + rows_wg - 1) / rows_wg, ws.gmax + 1);
    if (is_shape(n_tokens, hidden, n_ff, n_expert, k, 1) && a.has_shared) {  // the model shape
      if (f32io)
        hipLaunchKernelGGL((layer_front_kernel<1, 8, true, 1, true, 1>), grid, dim3(256), lds_f, s, a);
      else
        hipLaunchKernelGGL((layer_front_kernel<1, 8, true, 1, true, 2>), grid, dim3(256), lds_f, s, a);
    } else if (is_shape(n_tokens, hidden, n_ff, n_expert, k, 1)) {
      if (f32io)
        hipLaunchKernelGGL((layer_front_kernel<1, 8, true, 1, false, 1>), grid, dim3(256), lds_f, s, a);
      else
        hipLaunchKernelGGL((layer_front_kernel<1, 8, true, 1, false, 2>), grid, dim3(256), lds_f, s, a);
    } else if (is_shape(n_tokens, hidden, n_ff, n_expert, k, kShapeWindow) && a.has_shared) {
      if (f32io)  // its verify window
        hipLaunchKernelGGL((layer_front_kernel<4, 8, false, kShapeWindow, true, 1>), grid, dim3(256),
                           lds_f, s, a);
      else
        hipLaunchKernelGGL((layer_front_kernel<4, 8, false, kShapeWindow, true, 2>), grid, dim3(256),
                           lds_f, s, a);
    }
    else if (fl.ept <= 1 && hidden / kQK == 8 && n_tokens == 1)  // one-token decode, hidden 2048
      hipLaunchKernelGGL((layer_front_kernel<1, 8, true>), grid, dim3(256), lds_f, s, a);
    else if (fl.ept <= 1 && hidden / kQK == 8)  // the decode shape, compiled for hidden 2048
      hipLaunchKernelGGL((layer_front_kernel<1, 8>), grid, dim3(256), lds_f, s, a);
    else if (fl.ept <= 1)
      hipLaunchKernelGGL((layer_front_kernel<1, 0>), grid, dim3(256), lds_f, s, a);
    else if (fl.ept <= 2)
      hipLaunchKernelGGL((layer_front_kernel<2, 0>), grid, dim3(256), lds_f, s, a);
    else if (fl.ept <= 4)
      hipLaunchKernelGGL((layer_front_kernel<4, 0>), grid, dim3(256), lds_f, s, a);
    else
      hipLaunchKernelGGL((layer_front_kernel<kMaxEpt, 0>), grid, dim3(256), lds_f, s, a);
    if (int st = check_launch("sg_moe_layer/front")) return st;
    if (a.publish_only) {
      const dim3 gg((n_ff + rows_wg - 1) / rows_wg, ws.gmax);
      if (is_shape(n_tokens, hidden, n_ff, n_expert, k, kShapeWindow) && a.has_shared && f32io)
        hipLaunchKernelGGL((layer_gateup_kernel<8, kShapeWindow, true, 1>), gg, dim3(256), lds_g, s,
                           a);
      else if (is_shape(n_tokens, hidden, n_ff, n_expert, k, kShapeWindow) && a.has_shared)
        hipLaunchKernelGGL((layer_gateup_kernel<8, kShapeWindow, true, 2>), gg, dim3(256), lds_g, s,
                           a);
      else if (hidden / kQK == 8)
        hipLaunchKernelGGL((layer_gateup_kernel<8>), gg, dim3(256), lds_g, s, a);
      else
        hipLaunchKernelGGL((layer_gateup_kernel<0>), gg, dim3(256), lds_g, s, a);
      if (int st = check_launch("sg_moe_layer/gateup")) return st;
    }
  }
  if (stages & 2) {
    // the decode geometry of n_ff = 512 at hidden >= 2048 compiled for its
    // constants; other shapes read them from the arguments
    const dim3 gb((hidden + rows - 1) / rows);
    const bool geo = rows == 8 && back_bufs == kBackWaves;
    const size_t lds_bb = lds_b + back_bufs * buf_b;
    if (geo && is_shape(n_tokens, hidden, n_ff, n_expert, k, 1) && a.has_shared) {  // model shape
      if (f32io)
        hipLaunchKernelGGL((layer_back_kernel<2, 8, 1, true, 1>), gb, dim3(kBackThreads), lds_bb, s, a);
      else
        hipLaunchKernelGGL((layer_back_kernel<2, 8, 1, true, 2>), gb, dim3(kBackThreads), lds_bb, s, a);
    } else if (geo && is_shape(n_tokens, hidden, n_ff, n_expert, k, 1)) {
      if (f32io)
        hipLaunchKernelGGL((layer_back_kernel<2, 8, 1, false, 1>), gb, dim3(kBackThreads), lds_bb, s, a);
      else
        hipLaunchKernelGGL((layer_back_kernel<2, 8, 1, false, 2>), gb, dim3(kBackThreads), lds_bb, s, a);
    } else if (geo && is_shape(n_tokens, hidden, n_ff, n_expert, k, kShapeWindow) &&
               a.has_shared) {  // its verify window
      if (f32io)
        hipLaunchKernelGGL((layer_back_kernel<2, 8, kShapeWindow, true, 1>), gb, dim3(kBackThreads),
                           lds_bb, s, a);
      else
        hipLaunchKernelGGL((layer_back_kernel<2, 8, kShapeWindow, true, 2>), gb, dim3(kBackThreads),
                           lds_bb, s, a);
    }
    else if (n_ff / kQK == 2 && rows == 8)
      hipLaunchKernelGGL((layer_back_kernel<2, 8>), gb, dim3(kBackThreads),
                         lds_b + back_bufs * buf_b, s, a);
    else
      hipLaunchKernelGGL((layer_back_kernel<0, 0>), gb, dim3(kBackThreads),
                         lds_b + back_bufs * buf_b, s, a);
    if (int st = check_launch("sg_moe_layer/back")) return st;
  }
  return SG_OK;
}

}  // namespace sg

extern "C" {

int sg_moe_layer(const sg_block_q4k* const* tab_gate, const sg_block_q4k* const* tab_up,
                 const sg_block_q4k* const* tab_down, const sg_block_q4k* sh_gate,
                 const sg_block_q4k* sh_up, const sg_block_q4k* sh_down,
                 const float* sh_gate_w, const float* x, const float* logits,
                 const float* residual, float* out, int* idx, float* weight, void* workspace,
                 size_t workspace_bytes, int n_tokens, int hidden, int n_ff, int n_expert, int k,
                 float shared_w, void* stream) {
  return sg_moe_layer_stages(tab_gate, tab_up, tab_down, sh_gate, sh_up, sh_down, sh_gate_w, x,
                             logits, residual, out, idx, weight, workspace, workspace_bytes,
                             n_tokens, hidden, n_ff, n_expert, k, shared_w, 3, stream);
}

int sg_moe_layer_noalloc(const sg_block_q4k* const* tab_gate, const sg_block_q4k* const* tab_up,
                         const sg_block_q4k* const* tab_down, const sg_block_q4k* sh_gate,
                         const sg_block_q4k* sh_up, const sg_block_q4k* sh_down,
                         const float* sh_gate_w, const float* x, const float* logits,
                         const float* residual, float* out, int* idx, float* weight,
                         int n_tokens, int hidden, int n_ff, int n_expert, int k,
                         float shared_w, void* stream) {
  const char* nm = "sg_moe_layer_noalloc";
  const size_t need = sg_moe_layer_workspace_bytes(n_tokens, hidden, n_ff, n_expert, k);
  if (need > kScratchBytes)
    return set_error(SG_ERR_UNSUPPORTED,
                     "%s: this shape needs %zu B of workspace, more than the %zu B scratch "
                     "(use sg_moe_layer with a caller workspace)",
                     nm, need, kScratchBytes);
  void* ws = nullptr;
  if (int st = scratch_address(&ws, nm)) return st;
  // nothing in the workspace has to start at zero: the front launch writes
  // the plan, h and the gates that the back launch then reads
  return sg_moe_layer_stages(tab_gate, tab_up, tab_down, sh_gate, sh_up, sh_down, sh_gate_w, x,
                             logits, residual, out, idx, weight, ws, kScratchBytes, n_tokens,
                             hidden, n_ff, n_expert, k, shared_w, 3, stream);
}

}  // extern "C"
