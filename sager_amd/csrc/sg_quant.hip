// sg_quant.hip - Q8_K activation quantization on gfx950, plus the library's
// status plumbing.
//
// One wave per 256-value block: each lane owns 4 consecutive values, the
// block amax is a wave max (exact in any order), and the codes of lanes
// 8s..8s+7 form sub-block s, whose sum is an 8-lane reduction.  Semantics:
// quantize_row_q8_K, q4_k.cpp:44-61 (bit-exact).
#include <stdarg.h>
#include <stdio.h>

#include "sg_common.hpp"

namespace sg {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SG_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return SG_OK;
}

template <typename In>
__device__ __forceinline__ float load_act(const In* p);
template <>
__device__ __forceinline__ float load_act<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_act<uint16_t>(const uint16_t* p) {
  return half_bits_to_float(*p);
}

template <typename In>
__global__ void __launch_bounds__(256) quantize_q8k_kernel(const In* __restrict__ x,
                                                           unsigned char* __restrict__ out,
                                                           long long n_blocks) {
  const long long blk = static_cast<long long>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (blk >= n_blocks) return;
  const In* xb = x + blk * kQK + 4 * lane;
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = load_act<In>(xb + i);
  quantize_block_wave(v, out + blk * kQ8Bytes, lane);
}

template <typename In>
static int quantize_launch(const In* x, sg_block_q8k* out, int n, int n_rows, void* stream,
                           const char* name) {
  if (!x || !out) return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null pointer", name);
  if (n <= 0 || n % kQK != 0 || n_rows <= 0)
    return set_error(SG_ERR_GEOMETRY, "%s: n=%d must be a positive multiple of 256, n_rows=%d",
                     name, n, n_rows);
  const long long n_blocks = static_cast<long long>(n / kQK) * n_rows;
  const long long grid = (n_blocks + 3) / 4;
  if (grid > 0x7fffffffLL) return set_error(SG_ERR_UNSUPPORTED, "%s: too many rows", name);
  hipLaunchKernelGGL(quantize_q8k_kernel<In>, dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x,
                     reinterpret_cast<unsigned char*>(out), n_blocks);
  return check_launch(name);
}

}  // namespace sg

extern "C" {

const char* sg_last_error(void) { return sg::g_err; }
const char* sg_version(void) { return "sager-hip 0.1.0 (gfx950)"; }

int sg_quantize_q8_k(const float* x, sg_block_q8k* out, int n, int n_rows, void* stream) {
  return sg::quantize_launch<float>(x, out, n, n_rows, stream, "sg_quantize_q8_k");
}

int sg_quantize_q8_k_f16(const uint16_t* x, sg_block_q8k* out, int n, int n_rows,
                         void* stream) {
  return sg::quantize_launch<uint16_t>(x, out, n, n_rows, stream, "sg_quantize_q8_k_f16");
}

}  // extern "C"
