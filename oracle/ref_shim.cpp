// ref_shim.cpp - C entry points over the reference's own CPU sources.
//
// TEST INFRASTRUCTURE ONLY. Compiled together with the reference's
// src/kernels/q4_k.cpp and src/kernels/cpu/q4_avx2.cpp where they lie under
// /root/reference (see oracle/Makefile, target `ref`), into oracle/_ref/. It
// is used in this build container to write the golden fixtures under
// tests/golden/ and to cross-check the oracle; it never ships.
#include <cstdint>
#include <cstring>
#include <vector>

#include "sager/kernels/cpu_ops.hpp"
#include "sager/kernels/q4_k.hpp"

using sager::q4k::BlockQ4K;
using sager::q4k::BlockQ8K;

extern "C" {

// q4_k.hpp:66-88
float ref_half_to_float(uint16_t h) { return sager::q4k::half_to_float(h); }

// q4_k.hpp:110-118
void ref_get_scale_min(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
  sager::q4k::get_scale_min_k4(j, q, d, m);
}

// q4_k.cpp:13-42
void ref_dequant(const void* w, float* out, int n) {
  sager::q4k::dequant_row(static_cast<const BlockQ4K*>(w), out, n);
}

// q4_k.cpp:44-61 (host reference quantizer)
void ref_quantize_q8_k(const float* x, void* out, int n) {
  sager::q4k::quantize_row_q8_K(x, static_cast<BlockQ8K*>(out), n);
}

// q4_avx2.cpp:77-94 (AVX2 pool quantizer)
void ref_quantize_q8_k_avx2(const float* x, void* out, int n) {
  sager::cpu::quantize_row_q8_k_avx2(x, static_cast<BlockQ8K*>(out), n);
}

// q4_avx2.cpp:124-145
void ref_gemv_avx2(const void* w, const void* x, float* y, int n_rows, int k) {
  sager::cpu::gemv_q4_k_q8_avx2(static_cast<const BlockQ4K*>(w),
                                static_cast<const BlockQ8K*>(x), y, n_rows, k);
}

// q4_avx2.cpp:47-73
void ref_gemv_scalar(const void* w, const void* x, float* y, int n_rows, int k) {
  sager::cpu::gemv_q4_k_q8_scalar(static_cast<const BlockQ4K*>(w),
                                  static_cast<const BlockQ8K*>(x), y, n_rows, k);
}

// q4_k.cpp:176-207
float ref_vec_dot(const void* w, const void* x, int n) {
  return sager::q4k::vec_dot_ref(static_cast<const BlockQ4K*>(w),
                                 static_cast<const BlockQ8K*>(x), n);
}

// q4_avx2.cpp:175-196 (scratch >= 2*n_ff floats)
void ref_expert_ffn(const void* wg, const void* wu, const void* wd,
                    const float* x, float* y, float* scratch, int hidden,
                    int n_ff) {
  sager::cpu::expert_ffn_q4(static_cast<const BlockQ4K*>(wg),
                            static_cast<const BlockQ4K*>(wu),
                            static_cast<const BlockQ4K*>(wd), x, y, scratch,
                            hidden, n_ff);
}

// q4_k.cpp:68-174 (converter-side M-flavor quantizer; returns 0 on success)
int ref_quantize_row_q4k(const float* x, void* out, int n) {
  const std::vector<BlockQ4K> q = sager::q4k::quantize_row(x, n);
  std::memcpy(out, q.data(), q.size() * sizeof(BlockQ4K));
  return 0;
}

}  // extern "C"
