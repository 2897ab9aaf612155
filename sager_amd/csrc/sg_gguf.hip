// sg_gguf.hip - GGUF v3 expert loader into HBM (host code).
//
// Replaces the reference's expert-pool load (Weights::load_expert_pool,
// weights.cpp:800-870, over gguf::File, gguf.hpp/gguf.cpp) and the device
// pointer table the session uploads (session.cpp:2787-2796, 3596-3597).
// MI355X-first: every expert of every MoE layer is copied once into ONE HBM
// allocation (18.1 GB for 40 x 256 experts of the 288 GB), laid out
// [layer][expert][gate | up | down], and the [gate|up|down][layer][expert]
// table of device pointers that sg_moe_layer / sg_moe_prefill take is built
// next to it - no host pool, no pump, no offload.
//
// The GGUF v3 container (gguf.hpp:7-11): magic "GGUF" | u32 version (3) |
// u64 n_tensors | u64 n_kv | KVs (string key, u32 type, payload) | tensor
// infos (string name, u32 n_dims, u64 dims[], u32 type, u64 offset) | data
// at the next multiple of general.alignment (default 32).  The expert tensors
// are blk.L.ffn_{gate,up,down}_exps, stacked [n_expert][rows][cols]: gate/up
// Q4_K (type 12), down Q4_K or Q6_K (type 14).  A Q6_K down projection is
// requantized to Q4_K on the host per row, as the reference does
// (weights.cpp:841-857): Q6_K -> fp32 (weights.cpp:168-209) -> the
// reference's Q4_K quantizer (q4_k.cpp:62-174, restated below).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "sg_common.hpp"

namespace sg {

// ---- Q4_K requantization (host) ----------------------------------------------
// fp32 -> fp16 by truncation, subnormals by shifting (q4_k.hpp:90-105)
static uint16_t f32_to_f16_trunc(float f) {
  uint32_t b;
  std::memcpy(&b, &f, 4);
  const uint32_t sign = (b >> 16) & 0x8000u;
  const int32_t e = static_cast<int32_t>((b >> 23) & 0xFF) - 127 + 15;
  uint32_t m = b & 0x7FFFFFu;
  if (e >= 0x1F) return static_cast<uint16_t>(sign | 0x7C00u);
  if (e <= 0) {
    if (e < -10) return static_cast<uint16_t>(sign);
    m |= 0x800000u;
    return static_cast<uint16_t>(sign | (m >> (14 - e)));
  }
  return static_cast<uint16_t>(sign | (static_cast<uint32_t>(e) << 10) | (m >> 13));
}

// 6-bit scale d and min m of sub-block j into the 12 packed bytes (the
// inverse of get_scale_min_k4, q4_k.hpp:120-130)
static void put_scale_min(int j, uint8_t* q, uint8_t d, uint8_t m) {
  if (j < 4) {
    q[j] = static_cast<uint8_t>((q[j] & 0xC0) | (d & 63));
    q[j + 4] = static_cast<uint8_t>((q[j + 4] & 0xC0) | (m & 63));
  } else {
    q[j + 4] = static_cast<uint8_t>((q[j + 4] & 0xF0) | (d & 0xF));
    q[j - 4] = static_cast<uint8_t>((q[j - 4] & 0x3F) | ((d >> 4) << 6));
    q[j + 4] = static_cast<uint8_t>((q[j + 4] & 0x0F) | ((m & 0xF) << 4));
    q[j] = static_cast<uint8_t>((q[j] & 0x3F) | ((m >> 4) << 6));
  }
}

// float -> int as x86's cvttss2si (the reference's build): NaN and values
// outside int32 give INT32_MIN
static int f2i_x86(float f) {
  if (!(f >= -2147483648.0f && f < 2147483648.0f)) return INT32_MIN;
  return static_cast<int>(f);
}
static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// Squared error of sub-block sb reconstructed as dd*q - mm, q = rint((x + mm)/dd)
// clamped to [0, 15].  The reference's Release build contracts dd*q - mm and
// err + e*e into fmas; they are written as such.
static float q4k_sub_err(const float* sb, float dd, float mm) {
  const float id = dd > 0.f ? 1.f / dd : 0.f;
  float err = 0.f;
  for (int j = 0; j < 32; ++j) {
    const int q = clampi(f2i_x86(std::nearbyint((sb[j] + mm) * id)), 0, 15);
    const float w = std::fma(dd, static_cast<float>(q), -mm);
    const float e = sb[j] - w;
    err = std::fma(e, e, err);
  }
  return err;
}

// One row of n (multiple of 256) fp32 weights -> Q4_K blocks: per super-block
// d = dmin = (largest sub-block range) / 63; per sub-block the 6-bit
// (scale, min) pair from an anchor (range/15, -min) refined by a step-4 grid
// within +-16 and a step-1 grid within +-2 of the running winner, keeping
// the first pair of least squared error (q4_k.cpp:62-174).  The search order
// and tie rule decide the bytes, so they follow the reference step for step.
static void q4k_quantize_row(const float* x, uint8_t* out, int n) {
  const int nb = n / 256;
  for (int b = 0; b < nb; ++b) {
    const float* xb = x + static_cast<size_t>(b) * 256;
    uint8_t* bl = out + static_cast<size_t>(b) * kQ4Bytes;
    std::memset(bl, 0, kQ4Bytes);
    uint8_t codes[8][32] = {};
    float max_abs = 1e-30f;
    for (int s = 0; s < 8; ++s) {
      float mn = xb[32 * s], mx = xb[32 * s];
      for (int j = 1; j < 32; ++j) {
        mn = std::fmin(mn, xb[32 * s + j]);
        mx = std::fmax(mx, xb[32 * s + j]);
      }
      max_abs = std::fmax(max_abs, mx - mn);
    }
    const float d = max_abs / 63.f, dmin = max_abs / 63.f;
    const uint16_t dh = f32_to_f16_trunc(d), mh = f32_to_f16_trunc(dmin);
    std::memcpy(bl, &dh, 2);
    std::memcpy(bl + 2, &mh, 2);
    uint8_t* sc = bl + 4;
    for (int s = 0; s < 8; ++s) {
      const float* sb = xb + 32 * s;
      float mn = sb[0], mx = sb[0];
      for (int j = 1; j < 32; ++j) {
        mn = std::fmin(mn, sb[j]);
        mx = std::fmax(mx, sb[j]);
      }
      if (mx == mn) {
        put_scale_min(s, sc, 1, 0);
        continue;
      }
      const float d_ideal = (mx - mn) / 15.f;
      const int is0 = clampi(f2i_x86(std::nearbyint(d_ideal / d)), 1, 63);
      const int im0 = clampi(f2i_x86(std::nearbyint(-mn / dmin)), 0, 63);
      float best = q4k_sub_err(sb, d * static_cast<float>(is0), dmin * static_cast<float>(im0));
      int b_is = is0, b_im = im0;
      for (int is = std::max(1, is0 - 16); is <= std::min(63, is0 + 16); is += 4)
        for (int im = std::max(0, im0 - 16); im <= std::min(63, im0 + 16); im += 4) {
          const float err = q4k_sub_err(sb, d * static_cast<float>(is), dmin * static_cast<float>(im));
          if (err < best) {
            best = err;
            b_is = is;
            b_im = im;
          }
        }
      // the step-1 pass re-reads its bounds from the running winner, as the
      // reference's loop conditions do (the window moves with each improvement)
      for (int is = std::max(1, b_is - 2); is <= std::min(63, b_is + 2); ++is)
        for (int im = std::max(0, b_im - 2); im <= std::min(63, b_im + 2); ++im) {
          const float err = q4k_sub_err(sb, d * static_cast<float>(is), dmin * static_cast<float>(im));
          if (err < best) {
            best = err;
            b_is = is;
            b_im = im;
          }
        }
      const float bd = d * static_cast<float>(b_is), bm = dmin * static_cast<float>(b_im);
      const float id = bd > 0.f ? 1.f / bd : 0.f;
      for (int j = 0; j < 32; ++j)
        codes[s][j] = static_cast<uint8_t>(clampi(f2i_x86(std::nearbyint((sb[j] + bm) * id)), 0, 15));
      put_scale_min(s, sc, static_cast<uint8_t>(b_is), static_cast<uint8_t>(b_im));
    }
    for (int g = 0; g < 4; ++g)  // group g: sub-block 2g in the low nibbles, 2g+1 in the high
      for (int l = 0; l < 32; ++l)
        bl[16 + 32 * g + l] = static_cast<uint8_t>((codes[2 * g][l] & 0xF) | ((codes[2 * g + 1][l] & 0xF) << 4));
  }
}

// IEEE binary16 -> binary32 on the host (exact)
static float h2f(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h >> 15) << 31;
  const uint32_t e = (h >> 10) & 0x1F, m = h & 0x3FF;
  uint32_t b;
  if (e == 0x1F) {
    b = sign | 0x7F800000u | (m << 13);
  } else if (e != 0) {
    b = sign | ((e + 112) << 23) | (m << 13);
  } else if (m == 0) {
    b = sign;
  } else {  // subnormal: m * 2^-24, exact in fp32
    const float v = static_cast<float>(m) * 5.9604644775390625e-8f;
    std::memcpy(&b, &v, 4);
    b |= sign;
  }
  float f;
  std::memcpy(&f, &b, 4);
  return f;
}

// Q6_K row -> fp32 (weights.cpp:168-209): weight n*128 + q*32 + l of a block
// is d * sc[n*8 + 2q + l/16] * (code - 32), code = (ql nibble q>>1 of byte
// n*64 + (q&1)*32 + l) | (qh bits 2q..2q+1 of byte n*32 + l) << 4.  The
// reference multiplies left to right: (d * sc) * (code - 32).
static void q6k_dequant_row(const uint8_t* src, float* out, int cols) {
  for (int b = 0; b < cols / 256; ++b) {
    const uint8_t* ql = src + static_cast<size_t>(b) * 210;
    const uint8_t* qh = ql + 128;
    const int8_t* sc = reinterpret_cast<const int8_t*>(qh + 64);
    uint16_t dh;
    std::memcpy(&dh, ql + 208, 2);
    const float d = h2f(dh);
    for (int i = 0; i < 256; ++i) {
      const int n = i >> 7, q = (i >> 5) & 3, l = i & 31;
      const int lo = (ql[n * 64 + (q & 1) * 32 + l] >> (4 * (q >> 1))) & 15;
      const int hi = (qh[n * 32 + l] >> (2 * q)) & 3;
      out[static_cast<size_t>(b) * 256 + i] = d * static_cast<float>(sc[n * 8 + 2 * q + l / 16]) *
                                              static_cast<float>((lo | (hi << 4)) - 32);
    }
  }
}

// ---- GGUF v3 reader ------------------------------------------------------------
constexpr int kGgufQ4K = 12, kGgufQ6K = 14;

struct GgufTensor {
  uint32_t n_dims = 0;
  uint64_t dims[4] = {0, 0, 0, 0};  // dims[0] fastest (ne0)
  uint32_t type = 0;
  uint64_t offset = 0;  // from the data section's start
  uint64_t nbytes = 0;
};

class GgufFile {
 public:
  ~GgufFile() {
    if (map_) munmap(map_, len_);
  }
  // status 0, or an SG_ERR_* with the message set
  int open(const char* path);
  const GgufTensor* tensor(const std::string& name) const {
    auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
  }
  const uint8_t* data(const GgufTensor& t) const { return data_ + t.offset; }
  uint64_t alignment() const { return alignment_; }

 private:
  bool take(void* dst, size_t n) {  // bounds-checked read at the cursor
    if (n > static_cast<size_t>(end_ - cur_)) return false;
    std::memcpy(dst, cur_, n);
    cur_ += n;
    return true;
  }
  bool skip(uint64_t n) {
    if (n > static_cast<uint64_t>(end_ - cur_)) return false;
    cur_ += n;
    return true;
  }
  bool take_str(std::string* s) {
    uint64_t len = 0;
    if (!take(&len, 8) || len > (1ull << 24)) return false;  // no key or name is 16 MB
    if (len > static_cast<uint64_t>(end_ - cur_)) return false;
    s->assign(reinterpret_cast<const char*>(cur_), static_cast<size_t>(len));
    cur_ += len;
    return true;
  }
  bool skip_value(uint32_t type, int depth);

  uint8_t* map_ = nullptr;
  size_t len_ = 0;
  const uint8_t* cur_ = nullptr;
  const uint8_t* end_ = nullptr;
  const uint8_t* data_ = nullptr;
  uint64_t alignment_ = 32;
  std::unordered_map<std::string, GgufTensor> tensors_;
};

// byte size of a scalar KV type (gguf_type: u8 i8 u16 i16 u32 i32 f32 bool
// string array u64 i64 f64 = 0..12, gguf.hpp:28-32); 0 for string/array
static int gguf_scalar_bytes(uint32_t t) {
  switch (t) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    default: return 0;
  }
}

bool GgufFile::skip_value(uint32_t type, int depth) {
  if (type == 8) {  // string
    std::string s;
    return take_str(&s);
  }
  if (type == 9) {  // array: u32 element type, u64 count, elements
    uint32_t et = 0;
    uint64_t count = 0;
    if (depth > 2 || !take(&et, 4) || !take(&count, 8)) return false;
    const int eb = gguf_scalar_bytes(et);
    if (eb > 0) return count <= (1ull << 40) && skip(count * static_cast<uint64_t>(eb));
    if (et != 8) return false;  // arrays of strings only among the variable-size types
    for (uint64_t j = 0; j < count; ++j)
      if (!skip_value(8, depth + 1)) return false;
    return true;
  }
  const int b = gguf_scalar_bytes(type);
  return b > 0 && skip(b);
}

// ggml tensor types the loader sizes (gguf.cpp:23-31): block size, bytes per block
static bool gguf_type_size(uint32_t type, uint64_t* block, uint64_t* bytes) {
  switch (type) {
    case 0: *block = 1; *bytes = 4; return true;       // F32
    case 1: *block = 1; *bytes = 2; return true;       // F16
    case 8: *block = 32; *bytes = 34; return true;     // Q8_0
    case 12: *block = 256; *bytes = 144; return true;  // Q4_K
    case 14: *block = 256; *bytes = 210; return true;  // Q6_K
    case 30: *block = 1; *bytes = 2; return true;      // BF16
    default: return false;
  }
}

int GgufFile::open(const char* path) {
  const char* nm = "gguf";
  const int fd = ::open(path, O_RDONLY);
  if (fd < 0) return set_error(SG_ERR_FILE_NOT_FOUND, "%s: cannot open %s", nm, path);
  struct stat st{};
  if (fstat(fd, &st) != 0 || st.st_size < 24) {
    ::close(fd);
    return set_error(SG_ERR_GGUF_PARSE, "%s: %s is too small", nm, path);
  }
  len_ = static_cast<size_t>(st.st_size);
  void* m = mmap(nullptr, len_, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (m == MAP_FAILED) return set_error(SG_ERR_GGUF_PARSE, "%s: mmap of %s failed", nm, path);
  map_ = static_cast<uint8_t*>(m);
  cur_ = map_;
  end_ = map_ + len_;
  char magic[4];
  uint32_t version = 0;
  uint64_t n_tensors = 0, n_kv = 0;
  if (!take(magic, 4) || std::memcmp(magic, "GGUF", 4) != 0)
    return set_error(SG_ERR_GGUF_PARSE, "%s: %s is not a GGUF file", nm, path);
  if (!take(&version, 4) || version != 3)
    return set_error(SG_ERR_GGUF_PARSE, "%s: version %u (only 3 is read)", nm, version);
  if (!take(&n_tensors, 8) || !take(&n_kv, 8))
    return set_error(SG_ERR_GGUF_PARSE, "%s: truncated header", nm);
  for (uint64_t i = 0; i < n_kv; ++i) {
    std::string key;
    uint32_t type = 0;
    if (!take_str(&key) || !take(&type, 4))
      return set_error(SG_ERR_GGUF_PARSE, "%s: kv %llu: truncated", nm, (unsigned long long)i);
    if (key == "general.alignment" && (type == 4 || type == 5)) {
      uint32_t a = 0;
      if (!take(&a, 4)) return set_error(SG_ERR_GGUF_PARSE, "%s: truncated alignment", nm);
      alignment_ = a ? a : 32;
      continue;
    }
    if (type > 12 || !skip_value(type, 0))
      return set_error(SG_ERR_GGUF_PARSE, "%s: kv %llu (%s): bad value of type %u", nm,
                       (unsigned long long)i, key.c_str(), type);
  }
  for (uint64_t i = 0; i < n_tensors; ++i) {
    std::string name;
    GgufTensor t;
    if (!take_str(&name) || !take(&t.n_dims, 4) || t.n_dims == 0 || t.n_dims > 4)
      return set_error(SG_ERR_GGUF_PARSE, "%s: tensor %llu: bad name or rank", nm,
                       (unsigned long long)i);
    for (uint32_t d = 0; d < t.n_dims; ++d)
      if (!take(&t.dims[d], 8)) return set_error(SG_ERR_GGUF_PARSE, "%s: %s: truncated", nm, name.c_str());
    if (!take(&t.type, 4) || !take(&t.offset, 8))
      return set_error(SG_ERR_GGUF_PARSE, "%s: %s: truncated", nm, name.c_str());
    uint64_t block = 0, bytes = 0;
    if (!gguf_type_size(t.type, &block, &bytes) || t.dims[0] % block != 0)
      return set_error(SG_ERR_GGUF_PARSE, "%s: %s: unsupported type %u", nm, name.c_str(), t.type);
    t.nbytes = t.dims[0] / block * bytes;
    for (uint32_t d = 1; d < t.n_dims; ++d) t.nbytes *= t.dims[d];
    tensors_.emplace(std::move(name), t);
  }
  uint64_t start = static_cast<uint64_t>(cur_ - map_);
  start = (start + alignment_ - 1) / alignment_ * alignment_;
  if (start > len_) return set_error(SG_ERR_GGUF_PARSE, "%s: data section past the end", nm);
  data_ = map_ + start;
  for (const auto& kv : tensors_)
    if (kv.second.offset > len_ - start || kv.second.nbytes > len_ - start - kv.second.offset)
      return set_error(SG_ERR_GGUF_PARSE, "%s: tensor %s runs past the end of the file", nm,
                       kv.first.c_str());
  return SG_OK;
}

// ---- the expert tensors of a file ------------------------------------------------
struct ExpertDims {
  int n_layers = 0, n_expert = 0, hidden = 0, n_ff = 0;
  int q6_down_layers = 0;  // layers whose down projection is Q6_K (requantized)
};

static std::string exps_name(int L, const char* m) {
  return "blk." + std::to_string(L) + ".ffn_" + m + "_exps";
}

// every blk.L.ffn_{gate,up,down}_exps for L = 0, 1, ... until the first
// layer without them; all layers must agree on the shapes
static int expert_dims(const GgufFile& f, ExpertDims* out) {
  const char* nm = "gguf experts";
  ExpertDims d;
  for (int L = 0;; ++L) {
    const GgufTensor* g = f.tensor(exps_name(L, "gate"));
    const GgufTensor* u = f.tensor(exps_name(L, "up"));
    const GgufTensor* dn = f.tensor(exps_name(L, "down"));
    if (!g && !u && !dn) break;
    if (!g || !u || !dn)
      return set_error(SG_ERR_GGUF_PARSE, "%s: layer %d lacks one of gate/up/down", nm, L);
    if (g->n_dims != 3 || u->n_dims != 3 || dn->n_dims != 3)
      return set_error(SG_ERR_GEOMETRY, "%s: layer %d: expert tensors must be 3-D", nm, L);
    if (g->type != kGgufQ4K || u->type != kGgufQ4K || (dn->type != kGgufQ4K && dn->type != kGgufQ6K))
      return set_error(SG_ERR_UNSUPPORTED, "%s: layer %d: types %u/%u/%u (gate/up Q4_K, down Q4_K or Q6_K)",
                       nm, L, g->type, u->type, dn->type);
    const uint64_t hidden = g->dims[0], n_ff = g->dims[1], E = g->dims[2];
    if (u->dims[0] != hidden || u->dims[1] != n_ff || u->dims[2] != E || dn->dims[0] != n_ff ||
        dn->dims[1] != hidden || dn->dims[2] != E)
      return set_error(SG_ERR_GEOMETRY, "%s: layer %d: gate/up/down shapes disagree", nm, L);
    if (hidden % 256 || n_ff % 256 || hidden > (1u << 20) || n_ff > (1u << 20) || E == 0 || E > 1024)
      return set_error(SG_ERR_GEOMETRY, "%s: layer %d: hidden %llu n_ff %llu experts %llu", nm, L,
                       (unsigned long long)hidden, (unsigned long long)n_ff, (unsigned long long)E);
    if (L == 0) {
      d.hidden = static_cast<int>(hidden);
      d.n_ff = static_cast<int>(n_ff);
      d.n_expert = static_cast<int>(E);
    } else if (d.hidden != static_cast<int>(hidden) || d.n_ff != static_cast<int>(n_ff) ||
               d.n_expert != static_cast<int>(E)) {
      return set_error(SG_ERR_GEOMETRY, "%s: layer %d differs from layer 0", nm, L);
    }
    d.q6_down_layers += dn->type == kGgufQ6K;
    d.n_layers = L + 1;
  }
  if (d.n_layers == 0) return set_error(SG_ERR_GGUF_PARSE, "%s: no blk.0.ffn_*_exps tensors", nm);
  *out = d;
  return SG_OK;
}

}  // namespace sg

// the pool: one HBM allocation [layer][expert][gate|up|down] and the device
// pointer table [gate|up|down][layer][expert]
struct sg_expert_pool {
  void* base = nullptr;
  void* table = nullptr;
  int n_layers = 0, n_expert = 0, hidden = 0, n_ff = 0;
  size_t expert_bytes = 0;
};

using namespace sg;

extern "C" {

int sg_q4k_quantize_row(const float* x, sg_block_q4k* out, int n) {
  if (!x || !out) return set_error(SG_ERR_INVALID_ARGUMENT, "sg_q4k_quantize_row: null pointer");
  if (n <= 0 || n % 256)
    return set_error(SG_ERR_GEOMETRY, "sg_q4k_quantize_row: n=%d (a positive multiple of 256)", n);
  q4k_quantize_row(x, reinterpret_cast<uint8_t*>(out), n);
  return SG_OK;
}

int sg_gguf_expert_dims(const char* path, int* n_layers, int* n_expert, int* hidden, int* n_ff,
                        int* q6_down_layers) {
  if (!path) return set_error(SG_ERR_INVALID_ARGUMENT, "sg_gguf_expert_dims: null path");
  GgufFile f;
  if (int st = f.open(path)) return st;
  ExpertDims d;
  if (int st = expert_dims(f, &d)) return st;
  if (n_layers) *n_layers = d.n_layers;
  if (n_expert) *n_expert = d.n_expert;
  if (hidden) *hidden = d.hidden;
  if (n_ff) *n_ff = d.n_ff;
  if (q6_down_layers) *q6_down_layers = d.q6_down_layers;
  return SG_OK;
}

void sg_expert_pool_free(sg_expert_pool* p) {
  if (!p) return;
  if (p->table) (void)hipFree(p->table);
  if (p->base) (void)hipFree(p->base);
  delete p;
}

int sg_expert_pool_load_gguf(const char* path, sg_expert_pool** out) {
  const char* nm = "sg_expert_pool_load_gguf";
  if (!path || !out) return set_error(SG_ERR_INVALID_ARGUMENT, "%s: null argument", nm);
  *out = nullptr;
  GgufFile f;
  if (int st = f.open(path)) return st;
  ExpertDims d;
  if (int st = expert_dims(f, &d)) return st;
  const size_t gu = static_cast<size_t>(d.n_ff) * (d.hidden / 256) * kQ4Bytes;   // gate or up
  const size_t dn = static_cast<size_t>(d.hidden) * (d.n_ff / 256) * kQ4Bytes;   // down (Q4_K)
  const size_t eb = 2 * gu + dn;
  const size_t E = static_cast<size_t>(d.n_expert), L = static_cast<size_t>(d.n_layers);
  sg_expert_pool* p = new sg_expert_pool;
  p->n_layers = d.n_layers;
  p->n_expert = d.n_expert;
  p->hidden = d.hidden;
  p->n_ff = d.n_ff;
  p->expert_bytes = eb;
  auto fail = [&](int code, const char* what) {
    sg_expert_pool_free(p);
    return set_error(code, "%s: %s", nm, what);
  };
  if (hipMalloc(&p->base, L * E * eb) != hipSuccess) return fail(SG_ERR_OOM_VRAM, "pool allocation failed");
  if (hipMalloc(&p->table, 3 * L * E * sizeof(void*)) != hipSuccess)
    return fail(SG_ERR_OOM_VRAM, "table allocation failed");
  // one layer's stacked tensor at a time through a pinned staging buffer,
  // scattered into the expert slots by one 2-D copy
  const size_t stage_bytes = E * std::max(gu, dn);
  void* stage = nullptr;
  if (hipHostMalloc(&stage, stage_bytes, hipHostMallocDefault) != hipSuccess)
    return fail(SG_ERR_OOM_VRAM, "pinned staging allocation failed");
  int st = SG_OK;
  std::vector<float> row(d.n_ff);
  for (size_t l = 0; l < L && st == SG_OK; ++l) {
    const char* mats[3] = {"gate", "up", "down"};
    for (int m = 0; m < 3 && st == SG_OK; ++m) {
      const GgufTensor* t = f.tensor(exps_name(static_cast<int>(l), mats[m]));
      const size_t mb = m < 2 ? gu : dn;
      if (t->type == kGgufQ4K) {
        std::memcpy(stage, f.data(*t), E * mb);
      } else {  // Q6_K down: requantize row by row
        const size_t rb6 = static_cast<size_t>(d.n_ff / 256) * 210;
        const uint8_t* src = f.data(*t);
        uint8_t* dst = static_cast<uint8_t*>(stage);
        for (size_t r = 0; r < E * static_cast<size_t>(d.hidden); ++r) {
          q6k_dequant_row(src + r * rb6, row.data(), d.n_ff);
          q4k_quantize_row(row.data(), dst + r * (d.n_ff / 256) * kQ4Bytes, d.n_ff);
        }
      }
      uint8_t* dst0 = static_cast<uint8_t*>(p->base) + l * E * eb + (m == 0 ? 0 : m == 1 ? gu : 2 * gu);
      if (hipMemcpy2D(dst0, eb, stage, mb, mb, E, hipMemcpyHostToDevice) != hipSuccess)
        st = set_error(SG_ERR_HIP, "%s: copy of layer %zu failed", nm, l);
    }
  }
  (void)hipHostFree(stage);
  if (st != SG_OK) {
    sg_expert_pool_free(p);
    return st;
  }
  std::vector<uint64_t> tab(3 * L * E);
  for (size_t m = 0; m < 3; ++m)
    for (size_t l = 0; l < L; ++l)
      for (size_t e = 0; e < E; ++e)
        tab[(m * L + l) * E + e] = reinterpret_cast<uint64_t>(static_cast<uint8_t*>(p->base) +
                                                            (l * E + e) * eb + m * gu);
  if (hipMemcpy(p->table, tab.data(), tab.size() * 8, hipMemcpyHostToDevice) != hipSuccess)
    return fail(SG_ERR_HIP, "table upload failed");
  *out = p;
  return SG_OK;
}

int sg_expert_pool_dims(const sg_expert_pool* p, int* n_layers, int* n_expert, int* hidden,
                        int* n_ff) {
  if (!p) return set_error(SG_ERR_INVALID_ARGUMENT, "sg_expert_pool_dims: null pool");
  if (n_layers) *n_layers = p->n_layers;
  if (n_expert) *n_expert = p->n_expert;
  if (hidden) *hidden = p->hidden;
  if (n_ff) *n_ff = p->n_ff;
  return SG_OK;
}

const sg_block_q4k* const* sg_expert_pool_table(const sg_expert_pool* p) {
  return p ? static_cast<const sg_block_q4k* const*>(p->table) : nullptr;
}

}  // extern "C"
