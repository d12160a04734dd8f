// kmoe_oracle.cpp — CPU oracle for the MoE FFN hot path (test infrastructure).
//
// The HIP path's results are compared against it, and bench.py times it as
// the CPU baseline; it is never linked into the product library. It restates
// kestrel's native CPU executor (crates/kestrel-engine, Rust + AVX2/FMA):
//   quant.rs   — dequant_row, quant::dot, matmul regime switch, bench_gemv
//   qdot.rs    — Q8Row / Q8KRow activation quantizers, unpack, scalar dot
//   avx2.rs    — fused AVX2 dot kernels, gemm_f32, dot_f32, hsum
//   transformer.rs:472-570 — route, dispatch, expert loop, combine
// The AVX2 kernels use the same intrinsics in the same order as the
// reference, because the fp32 result of a dot product depends on the order
// of its additions; bit-identical floats need identical order. Build with
// -O2 -mavx2 -mfma -mf16c -ffp-contract=off (no fast-math): Rust neither
// contracts a*b+c into an FMA nor reassociates, so neither may this file.
//
// Rust's f32::exp lowers to glibc's expf on x86_64 Linux; this file calls
// the same expf.

#include "kmoe_oracle.h"

#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <chrono>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

namespace {

// ---------------------------------------------------------------------------
// A small persistent worker pool. The reference parallelises matmul over
// 16-row (int path) or 48-row (GEMM path) tiles with rayon (quant.rs:244,264);
// every output element is still computed by one serial call, so results do
// not depend on the thread count.
class Pool {
 public:
  explicit Pool(int n) {
    for (int i = 0; i < n; ++i) workers_.emplace_back([this, i] { loop(i); });
  }
  ~Pool() {
    {
      std::lock_guard<std::mutex> g(m_);
      stop_ = true;
    }
    cv_.notify_all();
    for (auto &t : workers_) t.join();
  }
  int size() const { return (int)workers_.size(); }

  // Run fn(i) for i in [0, n) on the caller plus up to `helpers` workers.
  void run(size_t n, int helpers, const std::function<void(size_t)> &fn) {
    if (n == 0) return;
    helpers = std::min<int>(helpers, (int)workers_.size());
    if (helpers <= 0 || n == 1) {
      for (size_t i = 0; i < n; ++i) fn(i);
      return;
    }
    std::unique_lock<std::mutex> lk(run_m_);  // one job at a time
    {
      std::lock_guard<std::mutex> g(m_);
      job_ = &fn;
      n_ = n;
      next_.store(0);
      helpers_ = helpers;
      pending_ = helpers;
      ++gen_;
    }
    cv_.notify_all();
    drain(fn);
    std::unique_lock<std::mutex> g(m_);
    done_cv_.wait(g, [this] { return pending_ == 0; });
    job_ = nullptr;
  }

 private:
  void drain(const std::function<void(size_t)> &fn) {
    for (;;) {
      size_t i = next_.fetch_add(1);
      if (i >= n_) break;
      fn(i);
    }
  }
  void loop(int id) {
    uint64_t seen = 0;
    for (;;) {
      const std::function<void(size_t)> *job;
      {
        std::unique_lock<std::mutex> g(m_);
        cv_.wait(g, [&] { return stop_ || gen_ != seen; });
        if (stop_) return;
        seen = gen_;
        if (id >= helpers_) continue;
        job = job_;
      }
      drain(*job);
      {
        std::lock_guard<std::mutex> g(m_);
        if (--pending_ == 0) done_cv_.notify_all();
      }
    }
  }
  std::vector<std::thread> workers_;
  std::mutex m_, run_m_;
  std::condition_variable cv_, done_cv_;
  const std::function<void(size_t)> *job_ = nullptr;
  size_t n_ = 0;
  std::atomic<size_t> next_{0};
  int helpers_ = 0, pending_ = 0;
  uint64_t gen_ = 0;
  bool stop_ = false;
};

Pool &pool() {
  static Pool p(std::max(1u, std::thread::hardware_concurrency()) - 1);
  return p;
}

int resolve_threads(int threads) {
  int hw = (int)std::max(1u, std::thread::hardware_concurrency());
  if (threads <= 0 || threads > hw) return hw;
  return threads;
}

void par_for(size_t n, int threads, const std::function<void(size_t)> &fn) {
  pool().run(n, resolve_threads(threads) - 1, fn);
}

// ---------------------------------------------------------------------------
// f16 <-> f32 (IEEE binary16; half 2.7.1's to_f32 is the exact conversion)

float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {  // subnormal: normalise
      int e = -1;
      do {
        man <<= 1;
        ++e;
      } while ((man & 0x400u) == 0);
      man &= 0x3ffu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

uint16_t f32_to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t absx = x & 0x7fffffffu;
  if (absx >= 0x7f800000u) {  // inf / nan
    return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u : 0));
  }
  if (absx >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to inf
  int e = (int)(absx >> 23) - 127;
  uint32_t man = absx & 0x7fffffu;
  if (e < -14) {  // subnormal half (or zero)
    if (e < -25) return (uint16_t)sign;
    man |= 0x800000u;
    int shift = -14 - e + 13;  // bits to drop
    uint32_t res = man >> shift;
    uint32_t rem = man & ((1u << shift) - 1);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (res & 1))) ++res;
    return (uint16_t)(sign | res);
  }
  uint32_t res = ((uint32_t)(e + 15) << 10) | (man >> 13);
  uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (res & 1))) ++res;
  return (uint16_t)(sign | res);
}

inline float f16at(const uint8_t *b) { return f16_to_f32((uint16_t)(b[0] | (b[1] << 8))); }

// Rust's f32::max: the non-NaN operand when one is NaN.
inline float rmax(float a, float b) {
  if (std::isnan(a)) return b;
  if (std::isnan(b)) return a;
  return a > b ? a : b;
}

// Rust `(v).round() as i32` then clamp(-127, 127) (qdot.rs:43, :360).
// round() is half away from zero; `as i32` saturates and maps NaN to 0.
inline int8_t q8_round(float v) {
  float r = std::round(v);
  int32_t i;
  if (std::isnan(r)) i = 0;
  else if (r >= 2147483647.0f) i = 2147483647;
  else if (r <= -2147483648.0f) i = (-2147483647 - 1);
  else i = (int32_t)r;
  if (i < -127) i = -127;
  if (i > 127) i = 127;
  return (int8_t)i;
}

// scale_min_k4, quant.rs:54-61 (same in qdot.rs:66-72, avx2.rs:78-84)
inline void scale_min_k4(int j, const uint8_t *q, uint8_t &sc, uint8_t &m) {
  if (j < 4) {
    sc = q[j] & 63;
    m = q[j + 4] & 63;
  } else {
    sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
    m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

// ---------------------------------------------------------------------------
// AVX2 building blocks, avx2.rs:19-46

inline float hsum(__m256 v) {  // avx2.rs:20-27
  __m128 lo = _mm256_castps256_ps128(v);
  __m128 hi = _mm256_extractf128_ps(v, 1);
  __m128 s = _mm_add_ps(lo, hi);
  s = _mm_add_ps(s, _mm_movehl_ps(s, s));
  s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
  return _mm_cvtss_f32(s);
}
inline __m256i mul_u8_i8(__m256i w, __m256i x) {  // avx2.rs:31-33
  return _mm256_madd_epi16(_mm256_maddubs_epi16(w, x), _mm256_set1_epi16(1));
}
inline __m256i mul_i8_i8(__m256i w, __m256i x) {  // avx2.rs:37-41
  __m256i aw = _mm256_sign_epi8(w, w);
  __m256i sx = _mm256_sign_epi8(x, w);
  return mul_u8_i8(aw, sx);
}
inline __m256i load(const void *p) { return _mm256_loadu_si256((const __m256i *)p); }

bool has_fused_k(int t) { return t == ORC_Q4_K || t == ORC_Q6_K; }             // qdot.rs:371-378
bool qdot_supports(int t) {  // qdot.rs:60-63
  return t == ORC_Q8_0 || t == ORC_Q4_0 || t == ORC_Q4_1 || t == ORC_Q5_0 || t == ORC_Q5_1 || t == ORC_Q4_K ||
         t == ORC_Q5_K || t == ORC_Q6_K;
}

}  // namespace

extern "C" {

int orc_hw_threads(void) { return (int)std::max(1u, std::thread::hardware_concurrency()); }

int64_t orc_block_size(int t) {  // types.rs:151-160
  switch (t) {
    case ORC_F32: case ORC_F16: case ORC_BF16: return 1;
    case ORC_Q4_0: case ORC_Q4_1: case ORC_Q5_0: case ORC_Q5_1: case ORC_Q8_0: return 32;
    case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: return 256;
    default: return -1;
  }
}
int64_t orc_type_size(int t) {  // types.rs:163-181
  switch (t) {
    case ORC_F32: return 4;
    case ORC_F16: case ORC_BF16: return 2;
    case ORC_Q4_0: return 18;
    case ORC_Q4_1: return 20;
    case ORC_Q5_0: return 22;
    case ORC_Q5_1: return 24;
    case ORC_Q8_0: return 34;
    case ORC_Q4_K: return 144;
    case ORC_Q5_K: return 176;
    case ORC_Q6_K: return 210;
    default: return -1;
  }
}
int64_t orc_bytes_for(int t, int64_t n) {  // types.rs:184-191
  int64_t bs = orc_block_size(t);
  if (bs <= 0 || n < 0 || n % bs != 0) return -1;
  return n / bs * orc_type_size(t);
}

float orc_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
uint16_t orc_f32_to_f16(float f) { return f32_to_f16(f); }
void orc_f32_to_f16_n(const float *x, uint16_t *out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = f32_to_f16(x[i]);
}

// ---------------------------------------------------------------------------
// Generators

void orc_fill_normal(uint64_t seed, float mean, float std_, float *out, size_t n) {
  // splitmix64 stream; each pair of uniforms gives two normals (Box-Muller).
  uint64_t s = seed;
  auto next = [&s]() {
    s += 0x9e3779b97f4a7c15ull;
    uint64_t z = s;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
  };
  auto uni = [&]() { return ((double)(next() >> 11) + 0.5) * (1.0 / 9007199254740992.0); };
  const double two_pi = 6.283185307179586476925286766559;
  size_t i = 0;
  while (i < n) {
    double u1 = uni(), u2 = uni();
    double r = std::sqrt(-2.0 * std::log(u1));
    double z0 = r * std::cos(two_pi * u2);
    double z1 = r * std::sin(two_pi * u2);
    out[i++] = (float)((double)mean + (double)std_ * z0);
    if (i < n) out[i++] = (float)((double)mean + (double)std_ * z1);
  }
}

void orc_fill_xorshift_bytes(uint32_t seed, uint8_t *out, size_t n, uint8_t mask) {
  // qdot.rs:277-285, avx2.rs:172-182, quant.rs:352-358
  uint32_t x = seed ? seed : 1;
  for (size_t i = 0; i < n; ++i) {
    x ^= x << 13;
    x ^= x >> 17;
    x ^= x << 5;
    out[i] = (uint8_t)(x & mask);
  }
}

// ---------------------------------------------------------------------------
// Quantizers. kestrel has none (it only reads GGUF blocks); these write the
// ggml layouts of quant.rs:82-89 (Q8_0) and quant.rs:138-155 (Q4_K).

void orc_quantize_q8_0(const float *x, size_t n, uint8_t *out) {
  for (size_t b = 0; b < n / 32; ++b) {
    const float *xs = x + 32 * b;
    uint8_t *blk = out + 34 * b;
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) amax = rmax(amax, std::fabs(xs[j]));
    float d = amax / 127.0f;
    float id = d > 0.0f ? 1.0f / d : 0.0f;
    uint16_t dh = f32_to_f16(d);
    blk[0] = (uint8_t)(dh & 0xff);
    blk[1] = (uint8_t)(dh >> 8);
    for (int j = 0; j < 32; ++j) blk[2 + j] = (uint8_t)q8_round(xs[j] * id);
  }
}

void orc_quantize_q4_k(const float *x, size_t n, uint8_t *out) {
  for (size_t b = 0; b < n / 256; ++b) {
    const float *xs = x + 256 * b;
    uint8_t *blk = out + 144 * b;
    float sub_scale[8], sub_min[8];
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; ++j) {
      float mn = xs[32 * j], mx = xs[32 * j];
      for (int l = 1; l < 32; ++l) {
        mn = std::min(mn, xs[32 * j + l]);
        mx = std::max(mx, xs[32 * j + l]);
      }
      if (mn > 0.0f) mn = 0.0f;
      sub_scale[j] = (mx - mn) / 15.0f;
      sub_min[j] = -mn;
      max_scale = std::max(max_scale, sub_scale[j]);
      max_min = std::max(max_min, sub_min[j]);
    }
    uint16_t dh = f32_to_f16(max_scale / 63.0f);
    uint16_t mh = f32_to_f16(max_min / 63.0f);
    float df = f16_to_f32(dh), mf = f16_to_f32(mh);
    uint8_t sc[8], m[8];
    for (int j = 0; j < 8; ++j) {
      float s = df > 0.0f ? std::round(sub_scale[j] / df) : 0.0f;
      float mm = mf > 0.0f ? std::round(sub_min[j] / mf) : 0.0f;
      sc[j] = (uint8_t)std::min(63.0f, std::max(0.0f, s));
      m[j] = (uint8_t)std::min(63.0f, std::max(0.0f, mm));
    }
    blk[0] = (uint8_t)(dh & 0xff);
    blk[1] = (uint8_t)(dh >> 8);
    blk[2] = (uint8_t)(mh & 0xff);
    blk[3] = (uint8_t)(mh >> 8);
    uint8_t *scales = blk + 4;
    // Inverse of scale_min_k4 (quant.rs:54-61).
    for (int j = 0; j < 4; ++j) {
      scales[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
      scales[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
      scales[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
    }
    uint8_t q[256];
    for (int j = 0; j < 8; ++j) {
      float dl = df * (float)sc[j];
      float ml = mf * (float)m[j];
      for (int l = 0; l < 32; ++l) {
        float v = dl > 0.0f ? std::round((xs[32 * j + l] + ml) / dl) : 0.0f;
        q[32 * j + l] = (uint8_t)std::min(15.0f, std::max(0.0f, v));
      }
    }
    uint8_t *qs = blk + 16;
    for (int k = 0; k < 4; ++k)
      for (int l = 0; l < 32; ++l) qs[32 * k + l] = (uint8_t)(q[64 * k + l] | (q[64 * k + 32 + l] << 4));
  }
}

void orc_quantize_q6_k(const float *x, size_t n, uint8_t *out) {
  // Ours (kestrel only reads Q6_K). Sub-block j (16 elements) gets a signed
  // scale sc_j = round(amax_j / 32 / d) with d = max_j(amax_j / 32) / 127;
  // q = clamp(round(x / (d sc_j)), -32, 31) + 32, packed as quant.rs:180-201
  // reads it: element h*128 + 32*ri + l -> low (ri < 2) or high nibble of
  // ql[h*64 + 32*(ri&1) + l] and bits 2*ri..2*ri+1 of qh[h*32 + l].
  for (size_t b = 0; b < n / 256; ++b) {
    const float *xs = x + 256 * b;
    uint8_t *blk = out + 210 * b;
    float sub[16], mx = 0.0f;
    for (int j = 0; j < 16; ++j) {
      float a = 0.0f;
      for (int l = 0; l < 16; ++l) a = std::max(a, std::fabs(xs[16 * j + l]));
      sub[j] = a / 32.0f;
      mx = std::max(mx, sub[j]);
    }
    const uint16_t dh = f32_to_f16(mx / 127.0f);
    const float df = f16_to_f32(dh);
    int8_t sc[16];
    for (int j = 0; j < 16; ++j) {
      float v = df > 0.0f ? std::round(sub[j] / df) : 0.0f;
      sc[j] = (int8_t)std::min(127.0f, std::max(-127.0f, v));
    }
    uint8_t q[256];
    for (int i = 0; i < 256; ++i) {
      const float dl = df * (float)sc[i / 16];
      float v = dl != 0.0f ? std::round(xs[i] / dl) : 0.0f;
      q[i] = (uint8_t)(std::min(31.0f, std::max(-32.0f, v)) + 32.0f);
    }
    std::memset(blk, 0, 210);
    for (int h = 0; h < 2; ++h)
      for (int ri = 0; ri < 4; ++ri)
        for (int l = 0; l < 32; ++l) {
          const uint8_t v = q[h * 128 + 32 * ri + l];
          uint8_t &ql = blk[h * 64 + 32 * (ri & 1) + l];
          ql |= (uint8_t)((v & 0xF) << (ri < 2 ? 0 : 4));
          blk[128 + h * 32 + l] |= (uint8_t)(((v >> 4) & 3) << (2 * ri));
        }
    for (int j = 0; j < 16; ++j) blk[192 + j] = (uint8_t)sc[j];
    blk[208] = (uint8_t)(dh & 0xff);
    blk[209] = (uint8_t)(dh >> 8);
  }
}

void orc_quantize_rows(int t, const float *x, size_t rows, size_t cols, uint8_t *out, int threads) {
  int64_t rb = orc_bytes_for(t, (int64_t)cols);
  if (rb < 0) return;
  size_t chunk = 64;
  par_for((rows + chunk - 1) / chunk, threads, [&](size_t c) {
    size_t r1 = std::min(rows, (c + 1) * chunk);
    for (size_t r = c * chunk; r < r1; ++r) {
      if (t == ORC_Q8_0) orc_quantize_q8_0(x + r * cols, cols, out + r * rb);
      else if (t == ORC_Q4_K) orc_quantize_q4_k(x + r * cols, cols, out + r * rb);
      else if (t == ORC_Q6_K) orc_quantize_q6_k(x + r * cols, cols, out + r * rb);
      else if (t == ORC_F32) std::memcpy(out + r * rb, x + r * cols, cols * 4);
    }
  });
}

// ---------------------------------------------------------------------------
// dequant_row, quant.rs:63-205

int orc_dequant_row(int t, const uint8_t *src, float *y, size_t n) {
  switch (t) {
    case ORC_F32:
      std::memcpy(y, src, n * 4);
      return 0;
    case ORC_F16:
      for (size_t i = 0; i < n; ++i) y[i] = f16at(src + 2 * i);
      return 0;
    case ORC_BF16:
      for (size_t i = 0; i < n; ++i) {
        uint32_t bits = (uint32_t)(src[2 * i] | (src[2 * i + 1] << 8)) << 16;
        std::memcpy(&y[i], &bits, 4);
      }
      return 0;
    case ORC_Q8_0:  // quant.rs:82-89
      for (size_t b = 0; b < n / 32; ++b) {
        const uint8_t *blk = src + 34 * b;
        float d = f16at(blk);
        for (int j = 0; j < 32; ++j) y[32 * b + j] = (float)(int8_t)blk[2 + j] * d;
      }
      return 0;
    case ORC_Q4_0:  // quant.rs:90-99
      for (size_t b = 0; b < n / 32; ++b) {
        const uint8_t *blk = src + 18 * b;
        float d = f16at(blk);
        const uint8_t *qs = blk + 2;
        for (int j = 0; j < 16; ++j) {
          y[32 * b + j] = (float)((int)(qs[j] & 0xF) - 8) * d;
          y[32 * b + j + 16] = (float)((int)(qs[j] >> 4) - 8) * d;
        }
      }
      return 0;
    case ORC_Q4_1:  // quant.rs:100-111
      for (size_t b = 0; b < n / 32; ++b) {
        const uint8_t *blk = src + 20 * b;
        float d = f16at(blk), m = f16at(blk + 2);
        const uint8_t *qs = blk + 4;
        for (int j = 0; j < 16; ++j) {
          y[32 * b + j] = (float)(qs[j] & 0xF) * d + m;
          y[32 * b + j + 16] = (float)(qs[j] >> 4) * d + m;
        }
      }
      return 0;
    case ORC_Q5_0:  // quant.rs:112-123
      for (size_t b = 0; b < n / 32; ++b) {
        const uint8_t *blk = src + 22 * b;
        float d = f16at(blk);
        uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) | ((uint32_t)blk[5] << 24);
        const uint8_t *qs = blk + 6;
        for (int j = 0; j < 16; ++j) {
          uint8_t h0 = (uint8_t)(((qh >> j) << 4) & 0x10), h1 = (uint8_t)((qh >> (j + 12)) & 0x10);
          y[32 * b + j] = (float)((int)((qs[j] & 0xF) | h0) - 16) * d;
          y[32 * b + j + 16] = (float)((int)((qs[j] >> 4) | h1) - 16) * d;
        }
      }
      return 0;
    case ORC_Q5_1:  // quant.rs:124-137
      for (size_t b = 0; b < n / 32; ++b) {
        const uint8_t *blk = src + 24 * b;
        float d = f16at(blk), m = f16at(blk + 2);
        uint32_t qh = (uint32_t)blk[4] | ((uint32_t)blk[5] << 8) | ((uint32_t)blk[6] << 16) | ((uint32_t)blk[7] << 24);
        const uint8_t *qs = blk + 8;
        for (int j = 0; j < 16; ++j) {
          uint8_t h0 = (uint8_t)(((qh >> j) << 4) & 0x10), h1 = (uint8_t)((qh >> (j + 12)) & 0x10);
          y[32 * b + j] = (float)((qs[j] & 0xF) | h0) * d + m;
          y[32 * b + j + 16] = (float)((qs[j] >> 4) | h1) * d + m;
        }
      }
      return 0;
    case ORC_Q5_K:  // quant.rs:156-179
      for (size_t b = 0; b < n / 256; ++b) {
        const uint8_t *blk = src + 176 * b;
        float d = f16at(blk), dmin = f16at(blk + 2);
        const uint8_t *scales = blk + 4, *qh = blk + 16, *ql = blk + 48;
        float *yy = y + 256 * b;
        uint8_t u1 = 1, u2 = 2;
        for (int k = 0; k < 4; ++k) {
          uint8_t s1, m1, s2, m2;
          scale_min_k4(2 * k, scales, s1, m1);
          scale_min_k4(2 * k + 1, scales, s2, m2);
          float d1 = d * (float)s1, mm1 = dmin * (float)m1;
          float d2 = d * (float)s2, mm2 = dmin * (float)m2;
          const uint8_t *q = ql + 32 * k;
          for (int l = 0; l < 32; ++l) {
            int hi1 = (qh[l] & u1) ? 16 : 0, hi2 = (qh[l] & u2) ? 16 : 0;
            yy[64 * k + l] = d1 * (float)((q[l] & 0xF) + hi1) - mm1;
            yy[64 * k + l + 32] = d2 * (float)((q[l] >> 4) + hi2) - mm2;
          }
          u1 = (uint8_t)(u1 << 2);
          u2 = (uint8_t)(u2 << 2);
        }
      }
      return 0;
    case ORC_Q4_K:  // quant.rs:138-155
      for (size_t b = 0; b < n / 256; ++b) {
        const uint8_t *blk = src + 144 * b;
        float d = f16at(blk), dmin = f16at(blk + 2);
        const uint8_t *scales = blk + 4, *qs = blk + 16;
        float *yy = y + 256 * b;
        for (int k = 0; k < 4; ++k) {
          uint8_t s1, m1, s2, m2;
          scale_min_k4(2 * k, scales, s1, m1);
          scale_min_k4(2 * k + 1, scales, s2, m2);
          float d1 = d * (float)s1, mm1 = dmin * (float)m1;
          float d2 = d * (float)s2, mm2 = dmin * (float)m2;
          const uint8_t *q = qs + 32 * k;
          for (int l = 0; l < 32; ++l) {
            yy[64 * k + l] = d1 * (float)(q[l] & 0xF) - mm1;
            yy[64 * k + l + 32] = d2 * (float)(q[l] >> 4) - mm2;
          }
        }
      }
      return 0;
    case ORC_Q6_K:  // quant.rs:180-201
      for (size_t b = 0; b < n / 256; ++b) {
        const uint8_t *blk = src + 210 * b;
        float d = f16at(blk + 208);
        for (int h = 0; h < 2; ++h) {
          const uint8_t *ql = blk + h * 64, *qh = blk + 128 + h * 32, *sc = blk + 192 + h * 8;
          float *yy = y + 256 * b + h * 128;
          for (int l = 0; l < 32; ++l) {
            int is = l / 16;
            int q1 = (int)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
            int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            yy[l] = d * (float)(int8_t)sc[is] * (float)q1;
            yy[l + 32] = d * (float)(int8_t)sc[is + 2] * (float)q2;
            yy[l + 64] = d * (float)(int8_t)sc[is + 4] * (float)q3;
            yy[l + 96] = d * (float)(int8_t)sc[is + 6] * (float)q4;
          }
        }
      }
      return 0;
    default:
      return -1;
  }
}

// ---------------------------------------------------------------------------
// Activation quantizers, qdot.rs:30-49 (Q8Row) and qdot.rs:347-367 (Q8KRow)

void orc_q8row_quantize(const float *x, size_t n, int8_t *q, float *d, int32_t *s16) {
  for (size_t b = 0; b < n / 32; ++b) {
    const float *xs = x + 32 * b;
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) amax = rmax(amax, std::fabs(xs[j]));
    float scale = amax / 127.0f;
    float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    d[b] = scale;
    for (int j = 0; j < 32; ++j) q[32 * b + j] = q8_round(xs[j] * inv);
    int32_t a = 0, c = 0;
    for (int j = 0; j < 16; ++j) a += q[32 * b + j];
    for (int j = 16; j < 32; ++j) c += q[32 * b + j];
    s16[2 * b] = a;
    s16[2 * b + 1] = c;
  }
}

void orc_q8krow_quantize(const float *x, size_t n, int8_t *q, float *d, int32_t *bsums) {
  for (size_t b = 0; b < n / 256; ++b) {
    const float *xs = x + 256 * b;
    float amax = 0.0f;
    for (int j = 0; j < 256; ++j) amax = rmax(amax, std::fabs(xs[j]));
    float scale = amax / 127.0f;
    float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    d[b] = scale;
    for (int j = 0; j < 256; ++j) q[256 * b + j] = q8_round(xs[j] * inv);
  }
  for (size_t k = 0; k < n / 16; ++k) {
    int32_t s = 0;
    for (int j = 0; j < 16; ++j) s += q[16 * k + j];
    bsums[k] = s;
  }
}

// ---------------------------------------------------------------------------
// Unpacked representation, qdot.rs:75-184

int orc_unpack(int t, const uint8_t *w, size_t n, int8_t *q, float *sc, float *mn) {
  switch (t) {
    case ORC_Q8_0:
      for (size_t b = 0; b < n / 32; ++b) {
        const uint8_t *blk = w + 34 * b;
        float d = f16at(blk);
        for (int j = 0; j < 32; ++j) q[32 * b + j] = (int8_t)blk[2 + j];
        sc[2 * b] = d;
        sc[2 * b + 1] = d;
        mn[2 * b] = 0.0f;
        mn[2 * b + 1] = 0.0f;
      }
      return 0;
    case ORC_Q4_0:
      for (size_t b = 0; b < n / 32; ++b) {
        const uint8_t *blk = w + 18 * b;
        float d = f16at(blk);
        const uint8_t *qs = blk + 2;
        for (int j = 0; j < 16; ++j) {
          q[32 * b + j] = (int8_t)((int8_t)(qs[j] & 0xF) - 8);
          q[32 * b + j + 16] = (int8_t)((int8_t)(qs[j] >> 4) - 8);
        }
        sc[2 * b] = d;
        sc[2 * b + 1] = d;
        mn[2 * b] = 0.0f;
        mn[2 * b + 1] = 0.0f;
      }
      return 0;
    case ORC_Q4_1:  // qdot.rs:93-108 (bias 0, min = -m)
      for (size_t b = 0; b < n / 32; ++b) {
        const uint8_t *blk = w + 20 * b;
        float d = f16at(blk), m = -f16at(blk + 2);
        const uint8_t *qs = blk + 4;
        for (int j = 0; j < 16; ++j) {
          q[32 * b + j] = (int8_t)(qs[j] & 0xF);
          q[32 * b + j + 16] = (int8_t)(qs[j] >> 4);
        }
        sc[2 * b] = d;
        sc[2 * b + 1] = d;
        mn[2 * b] = m;
        mn[2 * b + 1] = m;
      }
      return 0;
    case ORC_Q5_0:
    case ORC_Q5_1:  // qdot.rs:109-128 (Q5_0: bias 16, min 0; Q5_1: bias 0, min = -m)
      for (size_t b = 0; b < n / 32; ++b) {
        const size_t bs = t == ORC_Q5_0 ? 22 : 24, off = t == ORC_Q5_0 ? 2 : 4;
        const uint8_t *blk = w + bs * b;
        float d = f16at(blk);
        const int8_t bias = t == ORC_Q5_0 ? 16 : 0;
        float m = t == ORC_Q5_0 ? 0.0f : -f16at(blk + 2);
        uint32_t qh = (uint32_t)blk[off] | ((uint32_t)blk[off + 1] << 8) | ((uint32_t)blk[off + 2] << 16) |
                      ((uint32_t)blk[off + 3] << 24);
        const uint8_t *qs = blk + off + 4;
        for (int j = 0; j < 16; ++j) {
          uint8_t h0 = (uint8_t)(((qh >> j) << 4) & 0x10), h1 = (uint8_t)((qh >> (j + 12)) & 0x10);
          q[32 * b + j] = (int8_t)((int8_t)((qs[j] & 0xF) | h0) - bias);
          q[32 * b + j + 16] = (int8_t)((int8_t)((qs[j] >> 4) | h1) - bias);
        }
        sc[2 * b] = d;
        sc[2 * b + 1] = d;
        mn[2 * b] = m;
        mn[2 * b + 1] = m;
      }
      return 0;
    case ORC_Q4_K:
    case ORC_Q5_K:  // qdot.rs:129-153
      for (size_t sb = 0; sb < n / 256; ++sb) {
        const bool k5 = t == ORC_Q5_K;
        const uint8_t *blk = w + (k5 ? 176 : 144) * sb;
        float d = f16at(blk), dmin = f16at(blk + 2);
        const uint8_t *scales = blk + 4, *qh = blk + 16, *qs = blk + (k5 ? 48 : 16);
        for (int k = 0; k < 4; ++k) {
          const uint8_t *src = qs + 32 * k;
          size_t base = sb * 256 + k * 64;
          for (int j = 0; j < 32; ++j) {
            uint8_t lo = src[j] & 0xF, hi = src[j] >> 4;
            if (k5) {
              lo = (uint8_t)(lo | (((qh[j] >> (2 * k)) & 1) << 4));
              hi = (uint8_t)(hi | (((qh[j] >> (2 * k + 1)) & 1) << 4));
            }
            q[base + j] = (int8_t)lo;
            q[base + 32 + j] = (int8_t)hi;
          }
          uint8_t s0, m0, s1, m1;
          scale_min_k4(2 * k, scales, s0, m0);
          scale_min_k4(2 * k + 1, scales, s1, m1);
          size_t i16b = base / 16;
          for (int h = 0; h < 2; ++h) {
            sc[i16b + h] = d * (float)s0;
            mn[i16b + h] = dmin * (float)m0;
            sc[i16b + 2 + h] = d * (float)s1;
            mn[i16b + 2 + h] = dmin * (float)m1;
          }
        }
      }
      return 0;
    case ORC_Q6_K:
      for (size_t sb = 0; sb < n / 256; ++sb) {
        const uint8_t *blk = w + 210 * sb;
        float d = f16at(blk + 208);
        for (int h = 0; h < 2; ++h) {
          const uint8_t *ql = blk + h * 64, *qh = blk + 128 + h * 32, *s = blk + 192 + h * 8;
          size_t base = sb * 256 + h * 128;
          for (int l = 0; l < 32; ++l) {
            q[base + l] = (int8_t)((int8_t)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32);
            q[base + l + 32] = (int8_t)((int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
            q[base + l + 64] = (int8_t)((int8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
            q[base + l + 96] = (int8_t)((int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
          }
          for (int r = 0; r < 4; ++r)
            for (int hf = 0; hf < 2; ++hf) {
              size_t i16b = (base + 32 * r + 16 * hf) / 16;
              sc[i16b] = d * (float)(int8_t)s[2 * r + hf];
              mn[i16b] = 0.0f;
            }
        }
      }
      return 0;
    default:
      return -1;
  }
}

float orc_dot_unpacked_scalar(const int8_t *uq, const float *usc, const float *umn, size_t n, const int8_t *aq,
                              const float *ad, const int32_t *as16) {
  // qdot.rs:187-200
  float sum = 0.0f;
  for (size_t k = 0; k < n / 16; ++k) {
    int32_t p = 0;
    for (int j = 0; j < 16; ++j) p += (int32_t)uq[16 * k + j] * (int32_t)aq[16 * k + j];
    sum += ad[k / 2] * (usc[k] * (float)p - umn[k] * (float)as16[k]);
  }
  return sum;
}

float orc_dot_unpacked_avx2(const int8_t *uq, const float *usc, const float *umn, size_t n, const int8_t *aq,
                            const float *ad, const int32_t *as16) {
  // avx2.rs:151-164
  __m256 acc = _mm256_setzero_ps();
  float mins = 0.0f;
  for (size_t b = 0; b < n / 32; ++b) {
    __m256i qw = load(uq + 32 * b);
    __m256i qx = load(aq + 32 * b);
    __m256 p = _mm256_cvtepi32_ps(mul_i8_i8(qw, qx));
    __m256 sc = _mm256_set_m128(_mm_set1_ps(usc[2 * b + 1] * ad[b]), _mm_set1_ps(usc[2 * b] * ad[b]));
    acc = _mm256_fmadd_ps(p, sc, acc);
    float t1 = umn[2 * b] * (float)as16[2 * b];
    float t2 = umn[2 * b + 1] * (float)as16[2 * b + 1];
    mins += ad[b] * (t1 + t2);
  }
  return hsum(acc) - mins;
}

// ---------------------------------------------------------------------------
// Fused AVX2 kernels, avx2.rs

float orc_dot_q8_0(const uint8_t *w, size_t n, const int8_t *aq, const float *ad) {
  // avx2.rs:49-58
  __m256 acc = _mm256_setzero_ps();
  for (size_t b = 0; b < n / 32; ++b) {
    const uint8_t *blk = w + 34 * b;
    __m256i qw = load(blk + 2);
    __m256i qx = load(aq + 32 * b);
    __m256 p = _mm256_cvtepi32_ps(mul_i8_i8(qw, qx));
    acc = _mm256_fmadd_ps(p, _mm256_set1_ps(f16at(blk) * ad[b]), acc);
  }
  return hsum(acc);
}

float orc_dot_q4_0(const uint8_t *w, size_t n, const int8_t *aq, const float *ad) {
  // avx2.rs:61-75
  __m256 acc = _mm256_setzero_ps();
  const __m256i m4 = _mm256_set1_epi8(0x0F);
  const __m256i eight = _mm256_set1_epi8(8);
  for (size_t b = 0; b < n / 32; ++b) {
    const uint8_t *blk = w + 18 * b;
    __m128i q = _mm_loadu_si128((const __m128i *)(blk + 2));
    __m256i both = _mm256_set_m128i(_mm_srli_epi16(q, 4), q);
    __m256i qw = _mm256_sub_epi8(_mm256_and_si256(both, m4), eight);
    __m256i qx = load(aq + 32 * b);
    __m256 p = _mm256_cvtepi32_ps(mul_i8_i8(qw, qx));
    acc = _mm256_fmadd_ps(p, _mm256_set1_ps(f16at(blk) * ad[b]), acc);
  }
  return hsum(acc);
}

float orc_dot_q4_k(const uint8_t *w, size_t n, const int8_t *aq, const float *ad, const int32_t *as16) {
  // avx2.rs:87-112 (Q4_K against 32-block Q8 activations)
  __m256 acc = _mm256_setzero_ps();
  float mins = 0.0f;
  const __m256i m4 = _mm256_set1_epi8(0x0F);
  for (size_t sb = 0; sb < n / 256; ++sb) {
    const uint8_t *blk = w + 144 * sb;
    float d = f16at(blk), dmin = f16at(blk + 2);
    const uint8_t *scales = blk + 4, *qs = blk + 16;
    for (int k = 0; k < 4; ++k) {
      __m256i q = load(qs + 32 * k);
      __m256i lo = _mm256_and_si256(q, m4);
      __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q, 4), m4);
      size_t b0 = sb * 8 + 2 * k, b1 = b0 + 1;
      __m256i x0 = load(aq + b0 * 32);
      __m256i x1 = load(aq + b1 * 32);
      uint8_t s0, m0, s1, m1;
      scale_min_k4(2 * k, scales, s0, m0);
      scale_min_k4(2 * k + 1, scales, s1, m1);
      acc = _mm256_fmadd_ps(_mm256_cvtepi32_ps(mul_u8_i8(lo, x0)), _mm256_set1_ps(d * (float)s0 * ad[b0]), acc);
      acc = _mm256_fmadd_ps(_mm256_cvtepi32_ps(mul_u8_i8(hi, x1)), _mm256_set1_ps(d * (float)s1 * ad[b1]), acc);
      float t0 = (float)m0 * ad[b0] * (float)(as16[2 * b0] + as16[2 * b0 + 1]);
      float t1 = (float)m1 * ad[b1] * (float)(as16[2 * b1] + as16[2 * b1 + 1]);
      mins += dmin * (t0 + t1);
    }
  }
  return hsum(acc) - mins;
}

float orc_dot_q4_k_8k(const uint8_t *w, size_t n, const int8_t *aq, const float *ad, const int32_t *abs) {
  // avx2.rs:351-379
  const __m256i m4 = _mm256_set1_epi8(0x0F);
  __m256 acc = _mm256_setzero_ps();
  float summs = 0.0f;
  for (size_t b = 0; b < n / 256; ++b) {
    const uint8_t *blk = w + 144 * b;
    float d = f16at(blk) * ad[b];
    float dmin = f16at(blk + 2) * ad[b];
    const uint8_t *scales = blk + 4, *qs = blk + 16;
    const int8_t *xq = aq + 256 * b;
    __m256i sumi = _mm256_setzero_si256();
    int32_t mins = 0;
    for (int k = 0; k < 4; ++k) {
      uint8_t s0, m0, s1, m1;
      scale_min_k4(2 * k, scales, s0, m0);
      scale_min_k4(2 * k + 1, scales, s1, m1);
      __m256i q = load(qs + 32 * k);
      __m256i lo = _mm256_and_si256(q, m4);
      __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q, 4), m4);
      __m256i p0 = _mm256_madd_epi16(_mm256_maddubs_epi16(lo, load(xq + 64 * k)), _mm256_set1_epi16((int16_t)s0));
      __m256i p1 = _mm256_madd_epi16(_mm256_maddubs_epi16(hi, load(xq + 64 * k + 32)), _mm256_set1_epi16((int16_t)s1));
      sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(p0, p1));
      const int32_t *bs = abs + b * 16 + 4 * k;
      mins += (int32_t)m0 * (bs[0] + bs[1]) + (int32_t)m1 * (bs[2] + bs[3]);
    }
    acc = _mm256_fmadd_ps(_mm256_cvtepi32_ps(sumi), _mm256_set1_ps(d), acc);
    summs += dmin * (float)mins;
  }
  return hsum(acc) - summs;
}

void orc_q4k_block_acc(const uint8_t *w, size_t n, const int8_t *aq, const int32_t *abs, int32_t *sumi_out,
                       int32_t *mins_out) {
  // The integer part of avx2.rs:361-374, lanes summed.
  const __m256i m4 = _mm256_set1_epi8(0x0F);
  for (size_t b = 0; b < n / 256; ++b) {
    const uint8_t *blk = w + 144 * b;
    const uint8_t *scales = blk + 4, *qs = blk + 16;
    const int8_t *xq = aq + 256 * b;
    __m256i sumi = _mm256_setzero_si256();
    int32_t mins = 0;
    for (int k = 0; k < 4; ++k) {
      uint8_t s0, m0, s1, m1;
      scale_min_k4(2 * k, scales, s0, m0);
      scale_min_k4(2 * k + 1, scales, s1, m1);
      __m256i q = load(qs + 32 * k);
      __m256i lo = _mm256_and_si256(q, m4);
      __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q, 4), m4);
      __m256i p0 = _mm256_madd_epi16(_mm256_maddubs_epi16(lo, load(xq + 64 * k)), _mm256_set1_epi16((int16_t)s0));
      __m256i p1 = _mm256_madd_epi16(_mm256_maddubs_epi16(hi, load(xq + 64 * k + 32)), _mm256_set1_epi16((int16_t)s1));
      sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(p0, p1));
      const int32_t *bs = abs + b * 16 + 4 * k;
      mins += (int32_t)m0 * (bs[0] + bs[1]) + (int32_t)m1 * (bs[2] + bs[3]);
    }
    alignas(32) int32_t lanes[8];
    _mm256_store_si256((__m256i *)lanes, sumi);
    int32_t s = 0;
    for (int i = 0; i < 8; ++i) s += lanes[i];
    sumi_out[b] = s;
    mins_out[b] = mins;
  }
}

void orc_q4k_block_acc_bruteforce(const uint8_t *w, size_t n, const int8_t *aq, const int32_t *abs, int64_t *sumi,
                                  int64_t *mins) {
  // sumi = sum_j sc_j * sum_{i in sub-block j} q_i * x_i ; mins = sum_j m_j * sum_{i in j} x_i
  for (size_t b = 0; b < n / 256; ++b) {
    const uint8_t *blk = w + 144 * b;
    int64_t s = 0, m = 0;
    for (int j = 0; j < 8; ++j) {
      uint8_t sc, mm;
      scale_min_k4(j, blk + 4, sc, mm);
      int64_t dot = 0, xs = 0;
      for (int i = 0; i < 32; ++i) {
        int e = 32 * j + i;  // element within the superblock
        int k = e / 64, l = e % 64;
        uint8_t byte = blk[16 + 32 * k + (l % 32)];
        int qv = l < 32 ? (byte & 0xF) : (byte >> 4);
        dot += (int64_t)qv * aq[256 * b + e];
        xs += aq[256 * b + e];
      }
      (void)abs;
      s += (int64_t)sc * dot;
      m += (int64_t)mm * xs;
    }
    sumi[b] = s;
    mins[b] = m;
  }
}

// avx2.rs:384-419, integer part: per block the 8 i32 lanes of `sumi` and the
// offset sum `offs`. The four 32-byte rows r of half h hold 6-bit values
// (0..63); maddubs pairs them with x, madd applies sc[2r] to bytes 0-15 and
// sc[2r+1] to bytes 16-31.
static void q6k_block_lanes(const uint8_t *blk, const int8_t *xq, const int32_t *bsums, __m256i &sumi,
                            int32_t &offs) {
  const __m256i m4 = _mm256_set1_epi8(0x0F);
  const __m256i m3 = _mm256_set1_epi8(0x03);
  sumi = _mm256_setzero_si256();
  offs = 0;
  for (int h = 0; h < 2; ++h) {
    const uint8_t *ql = blk + h * 64;
    const __m256i qh = load(blk + 128 + h * 32);
    const uint8_t *sc = blk + 192 + h * 8;
    const __m256i qa = load(ql), qb = load(ql + 32);
    const __m256i r[4] = {
        _mm256_or_si256(_mm256_and_si256(qa, m4), _mm256_slli_epi16(_mm256_and_si256(qh, m3), 4)),
        _mm256_or_si256(_mm256_and_si256(qb, m4),
                        _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 2), m3), 4)),
        _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(qa, 4), m4),
                        _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 4), m3), 4)),
        _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(qb, 4), m4),
                        _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 6), m3), 4)),
    };
    for (int ri = 0; ri < 4; ++ri) {
      const int16_t s0 = (int16_t)(int8_t)sc[2 * ri], s1 = (int16_t)(int8_t)sc[2 * ri + 1];
      const __m256i x = load(xq + h * 128 + ri * 32);
      const __m256i p = _mm256_madd_epi16(_mm256_maddubs_epi16(r[ri], x),
                                          _mm256_set_m128i(_mm_set1_epi16(s1), _mm_set1_epi16(s0)));
      sumi = _mm256_add_epi32(sumi, p);
      const int k16 = h * 8 + ri * 2;
      offs += (int32_t)s0 * bsums[k16] + (int32_t)s1 * bsums[k16 + 1];
    }
  }
}

float orc_dot_q6_k_8k(const uint8_t *w, size_t n, const int8_t *aq, const float *ad, const int32_t *abs) {
  // avx2.rs:384-419
  __m256 acc = _mm256_setzero_ps();
  for (size_t b = 0; b < n / 256; ++b) {
    const uint8_t *blk = w + 210 * b;
    const float d = f16at(blk + 208) * ad[b];
    __m256i sumi;
    int32_t offs;
    q6k_block_lanes(blk, aq + 256 * b, abs + 16 * b, sumi, offs);
    // sum sc (q - 32) x = sum sc q x - 32 sum sc sum x
    acc = _mm256_fmadd_ps(_mm256_cvtepi32_ps(sumi), _mm256_set1_ps(d), acc);
    acc = _mm256_add_ps(acc, _mm256_set_ps(0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, -32.0f * d * (float)offs));
  }
  return hsum(acc);
}

void orc_q6k_block_acc(const uint8_t *w, size_t n, const int8_t *aq, const int32_t *abs, int32_t *sumi_out,
                       int32_t *offs_out) {
  for (size_t b = 0; b < n / 256; ++b) {
    __m256i sumi;
    int32_t offs;
    q6k_block_lanes(w + 210 * b, aq + 256 * b, abs + 16 * b, sumi, offs);
    alignas(32) int32_t lanes[8];
    _mm256_store_si256((__m256i *)lanes, sumi);
    int32_t s = 0;
    for (int i = 0; i < 8; ++i) s += lanes[i];
    sumi_out[b] = s;
    offs_out[b] = offs;
  }
}

void orc_q6k_block_acc_bruteforce(const uint8_t *w, size_t n, const int8_t *aq, int64_t *sumi, int64_t *offs) {
  // sumi = sum_j sc_j * sum_{i in 16-block j} q6_i * x_i (q6 in 0..63, read
  // bit by bit from ql/qh); offs = sum_j sc_j * sum_{i in j} x_i.
  for (size_t b = 0; b < n / 256; ++b) {
    const uint8_t *blk = w + 210 * b;
    int64_t s = 0, o = 0;
    for (int j = 0; j < 16; ++j) {
      const int64_t sc = (int8_t)blk[192 + j];
      int64_t dot = 0, xs = 0;
      for (int i = 0; i < 16; ++i) {
        const int e = 16 * j + i, h = e / 128, ri = (e % 128) / 32, l = e % 32;
        const uint8_t qlb = blk[h * 64 + 32 * (ri & 1) + l];
        const int lo4 = ri < 2 ? (qlb & 0xF) : (qlb >> 4);
        const int hi2 = (blk[128 + h * 32 + l] >> (2 * ri)) & 3;
        const int q6 = lo4 | (hi2 << 4);
        dot += (int64_t)q6 * aq[256 * b + e];
        xs += aq[256 * b + e];
      }
      s += sc * dot;
      o += sc * xs;
    }
    sumi[b] = s;
    offs[b] = o;
  }
}

void orc_q8_0_block_acc(const uint8_t *w, size_t n, const int8_t *aq, int32_t *p) {
  for (size_t b = 0; b < n / 32; ++b) {
    __m256i qw = load(w + 34 * b + 2);
    __m256i qx = load(aq + 32 * b);
    alignas(32) int32_t lanes[8];
    _mm256_store_si256((__m256i *)lanes, mul_i8_i8(qw, qx));
    int32_t s = 0;
    for (int i = 0; i < 8; ++i) s += lanes[i];
    p[b] = s;
  }
}

// ---------------------------------------------------------------------------
// f32 kernels

float orc_quant_dot(const float *a, const float *b, size_t n) {
  // quant.rs:208-224: eight accumulators, multiply then add (no FMA), summed
  // in order starting from -0.0 (Rust's float Sum), then the tail.
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  size_t nc = n / 8 * 8;
  for (size_t c = 0; c < nc; c += 8)
    for (int i = 0; i < 8; ++i) {
      float p = a[c + i] * b[c + i];
      acc[i] = acc[i] + p;
    }
  float s = -0.0f;
  for (int i = 0; i < 8; ++i) s = s + acc[i];
  for (size_t c = nc; c < n; ++c) {
    float p = a[c] * b[c];
    s = s + p;
  }
  return s;
}

float orc_dot_f32(const float *a, const float *b, size_t n) {
  // avx2.rs:289-308
  __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
  size_t c = 0;
  while (c + 16 <= n) {
    acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + c), _mm256_loadu_ps(b + c), acc0);
    acc1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + c + 8), _mm256_loadu_ps(b + c + 8), acc1);
    c += 16;
  }
  while (c + 8 <= n) {
    acc0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + c), _mm256_loadu_ps(b + c), acc0);
    c += 8;
  }
  float s = hsum(_mm256_add_ps(acc0, acc1));
  while (c < n) {
    float p = a[c] * b[c];
    s = s + p;
    ++c;
  }
  return s;
}

void orc_gemm_f32(const float *w, size_t rows, const float *x, size_t s_rows, size_t cols, float *res) {
  // avx2.rs:230-286: 3 weight rows x 4 activation rows register-blocked.
  size_t rows3 = rows / 3 * 3;
  size_t s = 0;
  while (s + 4 <= s_rows) {
    const float *x0 = x + s * cols, *x1 = x + (s + 1) * cols, *x2 = x + (s + 2) * cols, *x3 = x + (s + 3) * cols;
    size_t r = 0;
    while (r < rows3) {
      __m256 acc[12];
      for (int i = 0; i < 12; ++i) acc[i] = _mm256_setzero_ps();
      const float *w0 = w + r * cols, *w1 = w + (r + 1) * cols, *w2 = w + (r + 2) * cols;
      for (size_t c = 0; c < cols; c += 8) {
        __m256 a0 = _mm256_loadu_ps(w0 + c);
        __m256 a1 = _mm256_loadu_ps(w1 + c);
        __m256 a2 = _mm256_loadu_ps(w2 + c);
        __m256 bb = _mm256_loadu_ps(x0 + c);
        acc[0] = _mm256_fmadd_ps(a0, bb, acc[0]);
        acc[1] = _mm256_fmadd_ps(a1, bb, acc[1]);
        acc[2] = _mm256_fmadd_ps(a2, bb, acc[2]);
        bb = _mm256_loadu_ps(x1 + c);
        acc[3] = _mm256_fmadd_ps(a0, bb, acc[3]);
        acc[4] = _mm256_fmadd_ps(a1, bb, acc[4]);
        acc[5] = _mm256_fmadd_ps(a2, bb, acc[5]);
        bb = _mm256_loadu_ps(x2 + c);
        acc[6] = _mm256_fmadd_ps(a0, bb, acc[6]);
        acc[7] = _mm256_fmadd_ps(a1, bb, acc[7]);
        acc[8] = _mm256_fmadd_ps(a2, bb, acc[8]);
        bb = _mm256_loadu_ps(x3 + c);
        acc[9] = _mm256_fmadd_ps(a0, bb, acc[9]);
        acc[10] = _mm256_fmadd_ps(a1, bb, acc[10]);
        acc[11] = _mm256_fmadd_ps(a2, bb, acc[11]);
      }
      for (int si = 0; si < 4; ++si)
        for (int ri = 0; ri < 3; ++ri) res[(r + ri) * s_rows + s + si] = hsum(acc[si * 3 + ri]);
      r += 3;
    }
    for (size_t rr = rows3; rr < rows; ++rr)
      for (int si = 0; si < 4; ++si) res[rr * s_rows + s + si] = orc_dot_f32(w + rr * cols, x + (s + si) * cols, cols);
    s += 4;
  }
  for (; s < s_rows; ++s)
    for (size_t r = 0; r < rows; ++r) res[r * s_rows + s] = orc_dot_f32(w + r * cols, x + s * cols, cols);
}

// ---------------------------------------------------------------------------
// quant::matmul, quant.rs:229-328

int orc_matmul(int t, const uint8_t *w, size_t w_len, size_t rows, size_t cols, const float *x, size_t s_rows,
               float *out, int regime, int threads) {
  int64_t rb = orc_bytes_for(t, (int64_t)cols);
  if (rb < 0) return -1;
  size_t row_bytes = (size_t)rb;
  if (w_len < row_bytes * rows) return -1;
  if (s_rows == 0 || rows == 0) return 0;
  const size_t TILE = 16;
  auto scatter_tile = [&](size_t r0, size_t n, const std::vector<float> &res) {  // quant.rs:330-339
    for (size_t i = 0; i < n; ++i)
      for (size_t s = 0; s < s_rows; ++s) out[s * rows + r0 + i] = res[i * s_rows + s];
  };
  // quant.rs:242-260: batched rows -> dequantized 48-row tiles + gemm_f32.
  // KESTREL_EXACT does not reach this branch (it is tested first), so EXACT
  // takes it too; the INT8 regime keeps it only for unquantized weights.
  bool quantized = t != ORC_F32 && t != ORC_F16 && t != ORC_BF16;
  if (s_rows >= 4 && cols % 8 == 0 && !(regime == ORC_REGIME_INT8 && quantized)) {
    const size_t GT = 48;
    size_t nt = (rows + GT - 1) / GT;
    par_for(nt, threads, [&](size_t ti) {
      size_t r0 = ti * GT, r1 = std::min(rows, r0 + GT);
      std::vector<float> wf((r1 - r0) * cols);
      for (size_t r = r0; r < r1; ++r) orc_dequant_row(t, w + r * row_bytes, wf.data() + (r - r0) * cols, cols);
      std::vector<float> res((r1 - r0) * s_rows);
      orc_gemm_f32(wf.data(), r1 - r0, x, s_rows, cols, res.data());
      scatter_tile(r0, r1 - r0, res);
    });
    return 0;
  }
  bool exact = regime == ORC_REGIME_EXACT;
  // quant.rs:262-281: K-quants against Q8_K activations.
  if (!exact && has_fused_k(t) && cols % 256 == 0) {
    std::vector<int8_t> q(s_rows * cols);
    std::vector<float> d(s_rows * (cols / 256));
    std::vector<int32_t> bs(s_rows * (cols / 16));
    for (size_t s = 0; s < s_rows; ++s)
      orc_q8krow_quantize(x + s * cols, cols, q.data() + s * cols, d.data() + s * (cols / 256),
                          bs.data() + s * (cols / 16));
    size_t nt = (rows + TILE - 1) / TILE;
    par_for(nt, threads, [&](size_t ti) {
      size_t r0 = ti * TILE, r1 = std::min(rows, r0 + TILE);
      std::vector<float> res((r1 - r0) * s_rows);
      for (size_t r = r0; r < r1; ++r)
        for (size_t s = 0; s < s_rows; ++s) {
          float v;
          if (t == ORC_Q4_K)  // dot_fused_k, qdot.rs:382-390
            v = orc_dot_q4_k_8k(w + r * row_bytes, cols, q.data() + s * cols, d.data() + s * (cols / 256),
                                bs.data() + s * (cols / 16));
          else
            v = orc_dot_q6_k_8k(w + r * row_bytes, cols, q.data() + s * cols, d.data() + s * (cols / 256),
                                bs.data() + s * (cols / 16));
          res[(r - r0) * s_rows + s] = v;
        }
      scatter_tile(r0, r1 - r0, res);
    });
    return 0;
  }
  // quant.rs:282-310: 32-block Q8 activations.
  if (!exact && qdot_supports(t) && cols % 32 == 0) {
    std::vector<int8_t> q(s_rows * cols);
    std::vector<float> d(s_rows * (cols / 32));
    std::vector<int32_t> s16(s_rows * (cols / 16));
    for (size_t s = 0; s < s_rows; ++s)
      orc_q8row_quantize(x + s * cols, cols, q.data() + s * cols, d.data() + s * (cols / 32),
                         s16.data() + s * (cols / 16));
    size_t nt = (rows + TILE - 1) / TILE;
    par_for(nt, threads, [&](size_t ti) {
      size_t r0 = ti * TILE, r1 = std::min(rows, r0 + TILE);
      std::vector<float> res((r1 - r0) * s_rows);
      for (size_t r = r0; r < r1; ++r)
        for (size_t s = 0; s < s_rows; ++s) {
          const int8_t *aq = q.data() + s * cols;
          const float *ad = d.data() + s * (cols / 32);
          const int32_t *as = s16.data() + s * (cols / 16);
          const uint8_t *wr = w + r * row_bytes;
          float v;
          switch (t) {  // dot_fused, qdot.rs:252-268
            case ORC_Q8_0: v = orc_dot_q8_0(wr, cols, aq, ad); break;
            case ORC_Q4_0: v = orc_dot_q4_0(wr, cols, aq, ad); break;
            case ORC_Q4_K: v = orc_dot_q4_k(wr, cols, aq, ad, as); break;
            default: {  // qdot::unpack + dot (avx2 dot_unpacked), quant.rs:295-302
              std::vector<int8_t> uq(cols);
              std::vector<float> usc(cols / 16), umn(cols / 16);
              orc_unpack(t, wr, cols, uq.data(), usc.data(), umn.data());
              v = orc_dot_unpacked_avx2(uq.data(), usc.data(), umn.data(), cols, aq, ad, as);
            }
          }
          res[(r - r0) * s_rows + s] = v;
        }
      scatter_tile(r0, r1 - r0, res);
    });
    return 0;
  }
  // quant.rs:311-327: dequantize + scalar dot.
  size_t nt = (rows + TILE - 1) / TILE;
  par_for(nt, threads, [&](size_t ti) {
    size_t r0 = ti * TILE, r1 = std::min(rows, r0 + TILE);
    std::vector<float> buf(cols), res((r1 - r0) * s_rows);
    for (size_t r = r0; r < r1; ++r) {
      orc_dequant_row(t, w + r * row_bytes, buf.data(), cols);
      for (size_t s = 0; s < s_rows; ++s) res[(r - r0) * s_rows + s] = orc_quant_dot(buf.data(), x + s * cols, cols);
    }
    scatter_tile(r0, r1 - r0, res);
  });
  return 0;
}

// ---------------------------------------------------------------------------
// MoE layer, transformer.rs:472-570

void orc_route_from_logits(const float *logits, size_t s_rows, int ne, int k, int norm_topk, float weights_scale,
                           uint32_t *idx_out, float *w_out) {
  // transformer.rs:479-495
  std::vector<float> p(ne);
  std::vector<int> idx(ne);
  for (size_t s = 0; s < s_rows; ++s) {
    const float *row = logits + s * ne;
    float m = -INFINITY;
    for (int e = 0; e < ne; ++e) m = rmax(m, row[e]);
    for (int e = 0; e < ne; ++e) p[e] = expf(row[e] - m);
    float sum = -0.0f;
    for (int e = 0; e < ne; ++e) sum = sum + p[e];
    for (int e = 0; e < ne; ++e) p[e] = p[e] / sum;
    for (int e = 0; e < ne; ++e) idx[e] = e;
    // Descending p; NaN compares Equal; ties by ascending index.
    std::stable_sort(idx.begin(), idx.end(), [&](int a, int b) {
      if (p[b] < p[a]) return true;
      if (p[a] < p[b]) return false;
      return a < b;
    });
    for (int j = 0; j < k; ++j) {
      idx_out[s * k + j] = (uint32_t)idx[j];
      w_out[s * k + j] = p[idx[j]];
    }
    if (norm_topk) {
      float ssum = -0.0f;
      for (int j = 0; j < k; ++j) ssum = ssum + w_out[s * k + j];
      ssum = rmax(ssum, 6.103515625e-05f);
      for (int j = 0; j < k; ++j) w_out[s * k + j] = w_out[s * k + j] / ssum;
    }
    if (weights_scale != 0.0f && weights_scale != 1.0f)
      for (int j = 0; j < k; ++j) w_out[s * k + j] = w_out[s * k + j] * weights_scale;
  }
}

int orc_route(const orc_moe_layer *L, const float *h, size_t s_rows, uint32_t *idx, float *w, int regime,
              int threads) {
  // transformer.rs:474-476: logits = matmul(F32 router [E, d], h)
  int ne = L->n_expert;
  std::vector<float> logits(s_rows * ne);
  int rc = orc_matmul(ORC_F32, (const uint8_t *)L->router, (size_t)ne * L->n_embd * 4, ne, L->n_embd, h, s_rows,
                      logits.data(), regime, threads);
  if (rc) return rc;
  orc_route_from_logits(logits.data(), s_rows, ne, L->n_expert_used, L->norm_topk, L->weights_scale, idx, w);
  return 0;
}

void orc_dispatch(const uint32_t *idx, size_t s_rows, int k, int ne, uint32_t *perm, uint32_t *offsets) {
  // transformer.rs:525-530: BTreeMap<expert, Vec<(token, w)>> filled in token
  // order == stable sort of the flat (token, slot) list by expert id.
  std::vector<uint32_t> counts(ne, 0);
  for (size_t i = 0; i < s_rows * (size_t)k; ++i) counts[idx[i]]++;
  offsets[0] = 0;
  for (int e = 0; e < ne; ++e) offsets[e + 1] = offsets[e] + counts[e];
  std::vector<uint32_t> fill(offsets, offsets + ne);
  for (size_t i = 0; i < s_rows * (size_t)k; ++i) perm[fill[idx[i]]++] = (uint32_t)i;
}

int orc_moe_ffn(const orc_moe_layer *L, const float *h, size_t s_rows, float *out, int regime, int threads) {
  const int ne = L->n_expert, k = L->n_expert_used;
  const size_t d = (size_t)L->n_embd, ff = (size_t)L->n_ff;
  std::vector<uint32_t> idx(s_rows * k);
  std::vector<float> wsel(s_rows * k);
  int rc = orc_route(L, h, s_rows, idx.data(), wsel.data(), regime, threads);
  if (rc) return rc;
  std::vector<uint32_t> perm(s_rows * k), offsets(ne + 1);
  orc_dispatch(idx.data(), s_rows, k, ne, perm.data(), offsets.data());
  int64_t gb = orc_bytes_for(L->gate_type, (int64_t)d), ub = orc_bytes_for(L->up_type, (int64_t)d),
          db = orc_bytes_for(L->down_type, (int64_t)ff);
  if (gb < 0 || ub < 0 || db < 0) return -1;
  std::vector<std::vector<float>> ys(ne);
  for (int e = 0; e < ne; ++e) {  // transformer.rs:544-565
    size_t n = offsets[e + 1] - offsets[e];
    if (n == 0) continue;
    std::vector<float> xs(n * d);
    for (size_t i = 0; i < n; ++i) {
      size_t s = perm[offsets[e] + i] / k;
      std::memcpy(xs.data() + i * d, h + s * d, d * 4);
    }
    std::vector<float> g(n * ff), u(n * ff);
    rc = orc_matmul(L->gate_type, L->gate[e], (size_t)gb * ff, ff, d, xs.data(), n, g.data(), regime, threads);
    if (!rc) rc = orc_matmul(L->up_type, L->up[e], (size_t)ub * ff, ff, d, xs.data(), n, u.data(), regime, threads);
    if (rc) return rc;
    for (size_t i = 0; i < n * ff; ++i) {  // SwiGLU: g / (1 + exp(-g)) * u
      float gv = g[i];
      float den = 1.0f + expf(-gv);
      float q = gv / den;
      g[i] = q * u[i];
    }
    ys[e].assign(n * d, 0.0f);
    rc = orc_matmul(L->down_type, L->down[e], (size_t)db * d, d, ff, g.data(), n, ys[e].data(), regime, threads);
    if (rc) return rc;
  }
  // transformer.rs:566-570: combine in ascending expert id, out += w * y.
  std::memset(out, 0, s_rows * d * 4);
  for (int e = 0; e < ne; ++e) {
    for (uint32_t i = offsets[e]; i < offsets[e + 1]; ++i) {
      size_t flat = perm[i], s = flat / k;
      float wv = wsel[flat];
      const float *y = ys[e].data() + (size_t)(i - offsets[e]) * d;
      float *o = out + s * d;
      for (size_t c = 0; c < d; ++c) {
        float p = wv * y[c];
        o[c] = o[c] + p;
      }
    }
  }
  return 0;
}

// ---------------------------------------------------------------------------
// Shared expert, transformer.rs:572-587: g = mm(gate, h), u = mm(up, h),
// g = g / (1 + exp(-g)) * u, y = mm(down, g); scale per token by
// 1 / (1 + exp(-quant::dot(gate_inp, h[s]))) (or 1); out[s] += scale * y[s].

int orc_shared_expert_add(const orc_shared_expert *S, const float *h, size_t s_rows, float *out, int regime,
                          int threads) {
  const size_t d = (size_t)S->n_embd, ff = (size_t)S->n_ff;
  const int64_t gb = orc_bytes_for(S->gate_type, (int64_t)d), ub = orc_bytes_for(S->up_type, (int64_t)d),
                db = orc_bytes_for(S->down_type, (int64_t)ff);
  if (gb < 0 || ub < 0 || db < 0) return -1;
  std::vector<float> g(s_rows * ff), u(s_rows * ff), y(s_rows * d);
  int rc = orc_matmul(S->gate_type, S->gate, (size_t)gb * ff, ff, d, h, s_rows, g.data(), regime, threads);
  if (!rc) rc = orc_matmul(S->up_type, S->up, (size_t)ub * ff, ff, d, h, s_rows, u.data(), regime, threads);
  if (rc) return rc;
  for (size_t i = 0; i < s_rows * ff; ++i) {
    float gv = g[i];
    float den = 1.0f + expf(-gv);
    float q = gv / den;
    g[i] = q * u[i];
  }
  rc = orc_matmul(S->down_type, S->down, (size_t)db * d, d, ff, g.data(), s_rows, y.data(), regime, threads);
  if (rc) return rc;
  for (size_t s = 0; s < s_rows; ++s) {
    float scale = 1.0f;
    if (S->gate_inp) {
      float t = orc_quant_dot(S->gate_inp, h + s * d, d);
      float den = 1.0f + expf(-t);
      scale = 1.0f / den;
    }
    for (size_t c = 0; c < d; ++c) {
      float p = scale * y[s * d + c];
      out[s * d + c] = out[s * d + c] + p;
    }
  }
  return 0;
}

// ---------------------------------------------------------------------------
// The rest of the decoder layer, transformer.rs:216-226, 330-467, 591-631

void orc_rmsnorm(const float *x, const float *w, size_t rows, size_t dim, float eps, float *out) {
  for (size_t r = 0; r < rows; ++r) {
    const float *xi = x + r * dim;
    float ss = -0.0f;  // Rust's float Sum starts from -0.0 and adds in order
    for (size_t j = 0; j < dim; ++j) {
      float p = xi[j] * xi[j];
      ss = ss + p;
    }
    ss = ss / (float)dim;
    const float rr = 1.0f / std::sqrt(ss + eps);
    for (size_t j = 0; j < dim; ++j) {
      float t = xi[j] * rr;
      out[r * dim + j] = t * w[j];
    }
  }
}

void orc_rope_inv_freq(float base, size_t rope_dim, const float *freqs, float *inv_freq) {
  for (size_t i = 0; i < rope_dim / 2; ++i) {
    const float e = -(2.0f * (float)i) / (float)rope_dim;
    inv_freq[i] = powf(base, e);
    if (freqs) inv_freq[i] = inv_freq[i] / freqs[i];
  }
}

void orc_rope(float *x, size_t s_rows, size_t n_heads, size_t hd, size_t rd, size_t pos0, const float *inv_freq,
              int neox) {
  for (size_t s = 0; s < s_rows; ++s) {
    const float p = (float)(pos0 + s);
    for (size_t h = 0; h < n_heads; ++h) {
      float *v = x + (s * n_heads + h) * hd;
      for (size_t i = 0; i < rd / 2; ++i) {
        const float ang = p * inv_freq[i];
        const float sn = sinf(ang), cs = cosf(ang);
        const size_t a = neox ? i : 2 * i, b = neox ? i + rd / 2 : 2 * i + 1;
        const float x0 = v[a], x1 = v[b];
        float t0 = x0 * cs, t1 = x1 * sn;
        v[a] = t0 - t1;
        t0 = x0 * sn;
        t1 = x1 * cs;
        v[b] = t0 + t1;
      }
    }
  }
}

void orc_attention(const float *q, const uint16_t *k_cache, const uint16_t *v_cache, size_t s_rows, size_t nh,
                   size_t nkv, size_t hd, size_t pos0, float *out) {
  const size_t group = nh / nkv, kvw = nkv * hd, n_tot = pos0 + s_rows;
  const float scale = 1.0f / std::sqrt((float)hd);
  std::vector<float> kf(n_tot * kvw), vf(n_tot * kvw);
  for (size_t i = 0; i < n_tot * kvw; ++i) {
    kf[i] = f16_to_f32(k_cache[i]);
    vf[i] = f16_to_f32(v_cache[i]);
  }
  std::vector<float> scores;
  for (size_t i = 0; i < s_rows * nh; ++i) {
    const size_t s = i / nh, h = i % nh, kvh = h / group, n = pos0 + s + 1;
    const float *qv = q + (s * nh + h) * hd;
    float *o = out + i * hd;
    for (size_t j = 0; j < hd; ++j) o[j] = 0.0f;
    scores.assign(n, 0.0f);
    float m = -INFINITY;
    for (size_t p = 0; p < n; ++p) {
      scores[p] = orc_quant_dot(qv, kf.data() + p * kvw + kvh * hd, hd) * scale;
      m = std::max(m, scores[p]);  // f32::max over the fold, NaN-free inputs
    }
    float sum = 0.0f;
    for (size_t p = 0; p < n; ++p) {
      scores[p] = expf(scores[p] - m);
      sum = sum + scores[p];
    }
    const float inv = 1.0f / sum;
    for (size_t p = 0; p < n; ++p) {
      const float w = scores[p] * inv;
      const float *vr = vf.data() + p * kvw + kvh * hd;
      for (size_t j = 0; j < hd; ++j) {
        float t = w * vr[j];
        o[j] = o[j] + t;
      }
    }
  }
}

void orc_swiglu(const float *g, const float *u, size_t n, float *out) {
  for (size_t i = 0; i < n; ++i) {
    const float gv = g[i];
    const float den = 1.0f + expf(-gv);
    const float t = gv / den;
    out[i] = t * u[i];
  }
}

uint32_t orc_argmax(const float *l, size_t n) {
  size_t best = 0;
  for (size_t i = 1; i < n; ++i)
    if (l[i] > l[best]) best = i;
  return (uint32_t)best;
}

// ---------------------------------------------------------------------------
// bench_gemv, quant.rs:348-368

double orc_bench_gemv(int t, size_t rows, size_t cols, size_t iters, int threads) {
  int64_t rb = orc_bytes_for(t, (int64_t)cols);
  if (rb < 0) return -1.0;
  std::vector<uint8_t> w(rows * (size_t)rb);
  orc_fill_xorshift_bytes(0x12345678u, w.data(), w.size(), 0x3f);
  std::vector<float> act(cols), out(rows);
  for (size_t i = 0; i < cols; ++i) act[i] = (float)(i % 7) * 0.01f;
  orc_matmul(t, w.data(), w.size(), rows, cols, act.data(), 1, out.data(), ORC_REGIME_AVX2, threads);
  auto t0 = std::chrono::steady_clock::now();
  for (size_t i = 0; i < iters; ++i)
    orc_matmul(t, w.data(), w.size(), rows, cols, act.data(), 1, out.data(), ORC_REGIME_AVX2, threads);
  double el = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
  return (double)(w.size() * iters) / el;
}

}  // extern "C"
