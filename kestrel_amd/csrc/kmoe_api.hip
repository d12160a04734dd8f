// kmoe_api.hip — the C ABI of include/kmoe.h: context, Tier::Vram ledger,
// HBM-resident expert tier, workspace, and the moe_ffn pipeline.
//
// One context = one device + one stream. Calls that take device pointers
// enqueue work and return; errors from argument checks are reported before
// anything is enqueued.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/kmoe.h"
#include "kmoe_launch.h"

namespace kmoe {
thread_local LaunchTiming g_timing;
}  // namespace kmoe

using namespace kmoe;

namespace {

// GgmlType block geometry (types.rs:151-181) of the types quant::matmul accepts.
int64_t block_size(int t) {
  switch (t) {
    case KMOE_F32: case KMOE_F16: case KMOE_BF16: return 1;
    case KMOE_Q4_0: case KMOE_Q4_1: case KMOE_Q5_0: case KMOE_Q5_1: case KMOE_Q8_0: return 32;
    case KMOE_Q4_K: case KMOE_Q5_K: case KMOE_Q6_K: return 256;
    default: return -1;
  }
}
int64_t type_size(int t) {
  switch (t) {
    case KMOE_F32: return 4;
    case KMOE_F16: case KMOE_BF16: return 2;
    case KMOE_Q4_0: return 18;
    case KMOE_Q4_1: return 20;
    case KMOE_Q5_0: return 22;
    case KMOE_Q5_1: return 24;
    case KMOE_Q8_0: return 34;
    case KMOE_Q4_K: return 144;
    case KMOE_Q5_K: return 176;
    case KMOE_Q6_K: return 210;
    default: return -1;
  }
}
// GgmlType::bytes_for (types.rs:184-191); -1 when cols is not a block multiple.
int64_t bytes_for(int t, int64_t n) {
  const int64_t bs = block_size(t);
  if (bs <= 0 || n < 0 || n % bs != 0) return -1;
  return n / bs * type_size(t);
}

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct Layer {
  kmoe_moe_desc desc{};
  uint8_t *arena = nullptr;  // n_expert contiguous experts: [gate | up | down]
  float *router = nullptr;
  size_t part_len[3] = {0, 0, 0};
  size_t part_off[3] = {0, 0, 0};
  size_t expert_stride = 0;
  bool tiled[3] = {false, false, false};  // Q4_K and Q6_K parts are stored as tiled rows
  int64_t part_rows[3] = {0, 0, 0}, part_nb[3] = {0, 0, 0};
  int32_t part_type[3] = {0, 0, 0};
  size_t reserved = 0;
  bool router_ok = false;
  std::vector<uint8_t> loaded;  // bit p set when part p of expert e is resident
  struct Shared {  // qwen2moe shared expert (transformer.rs:572-587), GGUF bytes verbatim
    bool on = false;
    int64_t n_ff = 0;
    int32_t type[3] = {0, 0, 0};
    uint8_t *arena = nullptr;
    size_t off[3] = {0, 0, 0}, len[3] = {0, 0, 0};
    float *gate_inp = nullptr;  // [n_embd] f32, inside the arena
    bool gate_ok = false;
    uint8_t loaded = 0;
    size_t reserved = 0;
  } sh;
};

struct Event2 {
  std::string name;
  hipEvent_t a, b;
};

}  // namespace

// Workspace of kmoe_moe_ffn_noalloc: a fixed device array, one per GPU (each
// device holds its own copy at its own address), shared by every call on that
// GPU and kept until the process ends. Host code never uses this name as an
// address: the device's address comes from hipGetSymbolAddress at
// kmoe_create (g_scratch below).
constexpr size_t kScratchBytes = size_t(16) << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
constexpr int kMaxDevices = 64;
static void *g_scratch[kMaxDevices];  // device address of scratch per device, null until looked up
static std::mutex g_scratch_mu;

// Device completion counters per context (words used by the decode router).
constexpr int kCounterWords = 64;
constexpr int kNormDone = 1;  // the decode router's residual writer (kmoe_norm_moe_ffn)
constexpr int kFewRows = 3;   // decode batches over narrow rows: experts of 1..3 rows take launch_few_int

struct kmoe_ctx {
  int device = 0;
  hipStream_t own = nullptr;
  hipStream_t stream = nullptr;
  std::string err;
  int regime = KMOE_REGIME_AVX2;
  uint32_t *counters = nullptr;  // device, kCounterWords completion counters, zero between calls
  uint64_t vram_limit = 0;
  uint64_t vram_reserved = 0;
  std::map<uint32_t, Layer> layers;
  std::map<void *, size_t> user_allocs;
  // workspace
  uint8_t *ws = nullptr;
  size_t ws_size = 0;
  // bumped whenever ws, dws or aws is (re)allocated: device addresses a
  // captured graph may hold change only then
  uint64_t ws_gen = 0;
  // device staging for host uploads of tiled parts and whole expert extents
  uint8_t *stage = nullptr;
  size_t stage_size = 0;
  // device staging of the host-slice entry points (kmoe_matmul_host, kmoe_moe_ffn_host)
  uint8_t *hio = nullptr;
  size_t hio_size = 0;
  // decoder ops: token ids copied from the host; attention counters
  // (zero between calls) followed by its cross-work-group partials
  uint8_t *dws = nullptr;
  size_t dws_size = 0;
  uint8_t *aws = nullptr;
  size_t aws_size = 0, aws_counters = 0;
  // last moe_ffn routing (pointers into ws) and its sizes
  uint32_t *last_idx = nullptr, *last_perm = nullptr, *last_off = nullptr;
  float *last_w = nullptr;
  int64_t last_slots = 0;
  int32_t last_E = 0;
  // profiling
  bool prof = false;
  std::vector<Event2> pending;
  std::map<std::string, std::pair<double, int64_t>> prof_acc;
};

namespace {

int fail(kmoe_ctx *c, int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (c) c->err = buf;
  return code;
}

#define HIP_OK(ctx, expr)                                                                                   \
  do {                                                                                                      \
    hipError_t e_ = (expr);                                                                                 \
    if (e_ != hipSuccess) return fail((ctx), KMOE_E_HIP, "%s: %s (%s:%d)", #expr, hipGetErrorString(e_), \
                                      __FILE__, __LINE__);                                                  \
  } while (0)

struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) (void)hipSetDevice(dev);
  }
  ~DeviceGuard() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};

// Ledger::reserve (ledger.rs:75-102): an error value, never an OOM.
int reserve(kmoe_ctx *c, uint64_t bytes, const char *purpose) {
  if (c->vram_reserved + bytes > c->vram_limit)
    return fail(c, KMOE_E_BUDGET,
                "VRAM budget exhausted: requested %llu bytes for %s, %llu/%llu reserved",
                (unsigned long long)bytes, purpose, (unsigned long long)c->vram_reserved,
                (unsigned long long)c->vram_limit);
  c->vram_reserved += bytes;
  return KMOE_OK;
}
void release(kmoe_ctx *c, uint64_t bytes) { c->vram_reserved -= bytes < c->vram_reserved ? bytes : c->vram_reserved; }

int dev_alloc(kmoe_ctx *c, size_t bytes, void **p, const char *purpose) {
  int rc = reserve(c, bytes, purpose);
  if (rc) return rc;
  hipError_t e = hipMalloc(p, bytes ? bytes : 1);
  if (e != hipSuccess) {
    release(c, bytes);
    return fail(c, KMOE_E_HIP, "hipMalloc(%zu) for %s: %s", bytes, purpose, hipGetErrorString(e));
  }
  return KMOE_OK;
}

// Accumulate finished profiling events.
void prof_drain(kmoe_ctx *c) {
  for (auto &ev : c->pending) {
    float ms = 0.0f;
    if (hipEventSynchronize(ev.b) == hipSuccess && hipEventElapsedTime(&ms, ev.a, ev.b) == hipSuccess) {
      auto &acc = c->prof_acc[ev.name];
      acc.first += ms;
      acc.second += 1;
    }
    (void)hipEventDestroy(ev.a);
    (void)hipEventDestroy(ev.b);
  }
  c->pending.clear();
}

// Run one launch, bracketed by events when profiling.
template <class F>
hipError_t timed(kmoe_ctx *c, const char *name, F &&launch) {
  if (!c->prof) return launch();
  Event2 ev{name, nullptr, nullptr};
  hipError_t e = hipEventCreate(&ev.a);
  if (e == hipSuccess) e = hipEventCreate(&ev.b);
  if (e != hipSuccess) return e;
  g_timing = LaunchTiming{ev.a, ev.b};
  e = launch();
  const bool used = g_timing.start == nullptr;  // a kernel took the events
  g_timing = LaunchTiming{};
  if (e != hipSuccess || !used) {
    (void)hipEventDestroy(ev.a);
    (void)hipEventDestroy(ev.b);
    return e;
  }
  c->pending.push_back(ev);
  if (c->pending.size() > 4096) prof_drain(c);
  return e;
}

#define LAUNCH(ctx, name, expr) HIP_OK(ctx, timed((ctx), (name), [&]() -> hipError_t { return (expr); }))

// Workspace carving.
struct Carver {
  uint8_t *base;
  size_t off = 0;
  template <class T>
  T *take(size_t n) {
    T *p = reinterpret_cast<T *>(base ? base + off : nullptr);
    off = align_up(off + n * sizeof(T));
    return p;
  }
};

struct MoeWs {
  int8_t *xq;
  float *xd;
  int32_t *xs;
  float *logits;
  uint32_t *idx;
  float *wsel;
  uint32_t *perm, *offsets, *inv, *rank;
  int32_t *n_active, *active;
  float *h;
  int8_t *hq;
  float *hd;
  int32_t *hs;
  float *y;
  float *part;  // partial sums of the f32 path's column splits
  int64_t part_floats;
};

MoeWs carve_moe(uint8_t *base, int64_t S, int64_t E, int64_t k, int64_t d, int64_t F, size_t *total) {
  Carver cv{base};
  MoeWs w{};
  const int64_t slots = S * k;
  w.xq = cv.take<int8_t>(S * d);
  w.xd = cv.take<float>(S * (d / 32));
  w.xs = cv.take<int32_t>(S * (d / 16));
  w.logits = cv.take<float>(S * E);
  w.idx = cv.take<uint32_t>(slots);
  w.wsel = cv.take<float>(slots);
  w.perm = cv.take<uint32_t>(slots);
  w.offsets = cv.take<uint32_t>(E + 1);
  w.inv = cv.take<uint32_t>(slots);
  w.rank = cv.take<uint32_t>(slots);
  w.n_active = cv.take<int32_t>(1);
  w.active = cv.take<int32_t>(E);
  w.h = cv.take<float>(slots * F);
  w.hq = cv.take<int8_t>(slots * F);
  w.hd = cv.take<float>(slots * (F / 32));
  w.hs = cv.take<int32_t>(slots * (F / 16));
  w.y = cv.take<float>(slots * d);
  const int64_t ma = slots < E ? slots : E;
  const int64_t pg = gemm_f32_part_floats(F, d, ma, S, slots), pd = gemm_f32_part_floats(d, F, ma, S, slots);
  w.part_floats = pg > pd ? pg : pd;
  w.part = w.part_floats > 0 ? cv.take<float>(w.part_floats) : nullptr;
  *total = cv.off;
  return w;
}

int ensure_ws(kmoe_ctx *c, size_t need) {
  if (need <= c->ws_size) return KMOE_OK;
  size_t sz = align_up(need + need / 4);
  if (c->ws) {
    HIP_OK(c, hipStreamSynchronize(c->stream));
    HIP_OK(c, hipFree(c->ws));
    release(c, c->ws_size);
    c->ws = nullptr;
    c->ws_size = 0;
    c->last_idx = c->last_perm = c->last_off = nullptr;
    c->last_w = nullptr;
  }
  void *p = nullptr;
  int rc = dev_alloc(c, sz, &p, "workspace");
  if (rc) return rc;
  c->ws = (uint8_t *)p;
  c->ws_size = sz;
  ++c->ws_gen;
  return KMOE_OK;
}

// Decoder-op workspace, grown on demand (a call that would grow it must not
// be inside a graph capture: callers run one call of each size first).
int ensure_dws(kmoe_ctx *c, size_t need) {
  if (need <= c->dws_size) return KMOE_OK;
  const size_t sz = align_up(need + need / 4);
  if (c->dws) {
    HIP_OK(c, hipStreamSynchronize(c->stream));
    HIP_OK(c, hipFree(c->dws));
    release(c, c->dws_size);
    c->dws = nullptr;
    c->dws_size = 0;
  }
  void *p = nullptr;
  int rc = dev_alloc(c, sz, &p, "decoder workspace");
  if (rc) return rc;
  c->dws = (uint8_t *)p;
  c->dws_size = sz;
  ++c->ws_gen;
  return KMOE_OK;
}

// Attention workspace: `counters` zero words, then partials. Grown (and its
// counters cleared) outside any graph capture: callers run one call of each
// size first.
int ensure_aws(kmoe_ctx *c, size_t counters, size_t part_bytes) {
  const size_t cb = align_up(counters * 4);
  if (cb <= c->aws_counters && cb + part_bytes <= c->aws_size) return KMOE_OK;
  const size_t ncb = std::max(cb, c->aws_counters);
  const size_t need = ncb + std::max(part_bytes, c->aws_size - c->aws_counters);
  const size_t sz = align_up(need + need / 4);
  if (c->aws) {
    HIP_OK(c, hipStreamSynchronize(c->stream));
    HIP_OK(c, hipFree(c->aws));
    release(c, c->aws_size);
    c->aws = nullptr;
    c->aws_size = c->aws_counters = 0;
  }
  void *p = nullptr;
  int rc = dev_alloc(c, sz, &p, "attention workspace");
  if (rc) return rc;
  HIP_OK(c, hipMemset(p, 0, ncb));
  c->aws = (uint8_t *)p;
  c->aws_size = sz;
  c->aws_counters = ncb;
  ++c->ws_gen;
  return KMOE_OK;
}

// Device staging for host uploads, grown to the largest request and kept until
// kmoe_destroy (counted in the ledger). nullptr, with no error left behind,
// when the budget or hipMalloc refuses it: callers then take the host route.
uint8_t *staging(kmoe_ctx *c, size_t need) {
  if (need <= c->stage_size) return c->stage;
  const std::string keep = c->err;
  if (c->stage) {
    if (hipStreamSynchronize(c->stream) != hipSuccess) return nullptr;
    (void)hipFree(c->stage);
    release(c, c->stage_size);
    c->stage = nullptr;
    c->stage_size = 0;
  }
  constexpr size_t kGrain = size_t(2) << 20;
  const size_t sz = (need + kGrain - 1) / kGrain * kGrain;
  void *p = nullptr;
  if (dev_alloc(c, sz, &p, "upload staging")) {
    (void)hipGetLastError();  // a failed hipMalloc must not surface at the next launch check
    c->err = keep;
    return nullptr;
  }
  c->stage = (uint8_t *)p;
  c->stage_size = sz;
  return c->stage;
}

// Device staging of the host-slice entry points, grown on demand (counted in
// the ledger, kept until kmoe_destroy).
int ensure_hio(kmoe_ctx *c, size_t need) {
  if (need <= c->hio_size) return KMOE_OK;
  const size_t sz = align_up(need + need / 4);
  if (c->hio) {
    HIP_OK(c, hipStreamSynchronize(c->stream));
    HIP_OK(c, hipFree(c->hio));
    release(c, c->hio_size);
    c->hio = nullptr;
    c->hio_size = 0;
  }
  void *p = nullptr;
  int rc = dev_alloc(c, sz, &p, "host-slice staging");
  if (rc) return rc;
  c->hio = (uint8_t *)p;
  c->hio_size = sz;
  return KMOE_OK;
}

// Whether p is device memory (hipMalloc'd, on any device); host memory, pinned
// or pageable, is not.
bool is_device_ptr(const void *p) {
  hipPointerAttribute_t a{};
  if (hipPointerGetAttributes(&a, p) != hipSuccess) {
    (void)hipGetLastError();  // an unknown (pageable host) pointer is not an error here
    return false;
  }
  return a.type == hipMemoryTypeDevice;
}

bool supported_weight(int t) { return t == KMOE_Q4_K || t == KMOE_Q6_K || t == KMOE_Q8_0; }
// K-quants take Q8_K activations (quant.rs:262-281); Q8_0 takes Q8 rows.
bool is_kq(int t) { return t == KMOE_Q4_K || t == KMOE_Q6_K; }

// Row-shape checks shared by the quantized kernels.
int check_quant_shape(kmoe_ctx *c, int t, int64_t cols) {
  if (!supported_weight(t)) return fail(c, KMOE_E_UNSUPPORTED, "ggml type %d has no kernel (Q8_0=8, Q4_K=12, Q6_K=14)", t);
  if (bytes_for(t, cols) < 0) return fail(c, KMOE_E_INVALID, "cols %lld not a multiple of the block size", (long long)cols);
  if (t == KMOE_Q8_0 && cols % 64 != 0)
    return fail(c, KMOE_E_UNSUPPORTED, "Q8_0 rows need cols %% 64 == 0 (dword-aligned row starts), got %lld",
                (long long)cols);
  if (cols % 64 != 0) return fail(c, KMOE_E_UNSUPPORTED, "cols %% 64 != 0");
  const int64_t per = cols + cols / 4 + cols / 8 + 48;
  if (3 * per > 65536) return fail(c, KMOE_E_UNSUPPORTED, "cols %lld too wide for the LDS-staged kernels", (long long)cols);
  return KMOE_OK;
}

// A raw weight pointer at a tiled (Q4_K / Q6_K) part of an expert tier, as
// kmoe_expert_part hands it out: the raw-pointer kernels read GGUF rows, so
// such a pointer is refused instead of giving wrong results.
int reject_tiled(kmoe_ctx *c, const void *w) {
  const uint8_t *p = (const uint8_t *)w;
  for (auto &kv : c->layers) {
    const Layer &L = kv.second;
    if (!L.arena || !L.expert_stride) continue;
    const uint8_t *b = L.arena, *e = L.arena + (size_t)L.desc.n_expert * L.expert_stride;
    if (p < b || p >= e) continue;
    const size_t o = (size_t)(p - b) % L.expert_stride;
    for (int k = 0; k < 3; ++k)
      if (L.tiled[k] && o >= L.part_off[k] && o < L.part_off[k] + L.part_len[k])
        return fail(c, KMOE_E_INVALID,
                    "weight pointer lies in layer %u's tiled expert part %d (KMOE_LAYOUT_TILED, see "
                    "kmoe_expert_part_layout); this entry point reads GGUF rows",
                    kv.first, k);
  }
  return KMOE_OK;
}

bool int_path(int regime, int64_t s_rows) {
  return regime == KMOE_REGIME_INT8 || (regime == KMOE_REGIME_AVX2 && s_rows < 4);
}

// int8-activation matvec: one activation row -> register-resident decode
// kernel; otherwise (or if the row is too wide for it) the LDS-staged kernel.
int matvec_q8_impl(kmoe_ctx *c, int t, const uint8_t *w, int64_t rows, int64_t cols, const int8_t *q, const float *d,
                   const int32_t *s, int64_t s_rows, float *out) {
  const char *name = t == KMOE_Q4_K ? "matvec_q4k" : (t == KMOE_Q6_K ? "matvec_q6k" : "matvec_q8_0");
  if (t == KMOE_Q4_K && s_rows >= kMfmaMinRows) {  // int8 matrix cores
    hipError_t e = timed(c, "matvec_q4k_mfma", [&]() {
      return launch_plain_mfma(c->stream, w, rows, cols, q, d, s, s_rows, out, nullptr, nullptr);
    });
    if (e == hipSuccess) return KMOE_OK;
    if (e != hipErrorNotSupported) HIP_OK(c, e);
  }
  if (s_rows == 1) {
    hipError_t e = timed(c, name, [&]() { return launch_decode_plain(c->stream, t, w, rows, cols, q, d, s, out); });
    if (e == hipSuccess) return KMOE_OK;
    if (e != hipErrorNotSupported) HIP_OK(c, e);
  }
  LAUNCH(c, name, launch_matvec_int(c->stream, t, w, rows, cols, q, d, s, s_rows, out));
  return KMOE_OK;
}

// Scratch for one int8-quantized activation matrix [s_rows, cols], plus the
// f32 path's partial sums (part_floats, 0 for none).
struct QRows {
  int8_t *q;
  float *d;
  int32_t *s;
  float *part;
  int64_t part_floats;
};
QRows carve_qrows(uint8_t *base, int64_t s_rows, int64_t cols, size_t *total, int64_t part_floats = 0) {
  Carver cv{base};
  QRows r{cv.take<int8_t>(s_rows * cols), cv.take<float>(s_rows * (cols / 32)), cv.take<int32_t>(s_rows * (cols / 16)),
          nullptr, part_floats};
  r.part = part_floats > 0 ? cv.take<float>(part_floats) : nullptr;
  *total = cv.off;
  return r;
}

// The f32 path's partial sums for the shared expert's three products.
int64_t sh_part_floats(int64_t Fs, int64_t d, int64_t S) {
  const int64_t a = gemm_f32_part_floats(Fs, d, 1, S, S), b = gemm_f32_part_floats(d, Fs, 1, S, S);
  return a > b ? a : b;
}

// quant::matmul (quant.rs:229-328) on validated arguments: F32 weights in the
// reference's summation order; otherwise the context's regime picks the f32
// GEMM or int8 activations (quantized into qr) and the int8 matvec.
int matmul_core(kmoe_ctx *c, int t, const uint8_t *w, int64_t rows, int64_t cols, const float *x, int64_t s_rows,
                float *out, const QRows &qr, float *wf = nullptr) {
  if (xtype(t)) {  // F16, BF16, Q4_0, Q4_1, Q5_0, Q5_1, Q5_K
    const int64_t rb = bytes_for(t, cols);
    if (t == KMOE_F16 || t == KMOE_BF16 || !int_path(c->regime, s_rows)) {
      // dequant_row into wf, then the F32 weights' path (quant.rs:242-260, :311-327)
      if (!wf) return fail(c, KMOE_E_INVALID, "no f32 staging for type %d", t);
      if (rows > (int64_t)INT32_MAX) return fail(c, KMOE_E_INVALID, "too many rows");
      LAUNCH(c, "dequant_x", launch_dequant_x(c->stream, t, w, rows, cols, rb, wf));
      LAUNCH(c, "matmul_f32_ordered", launch_router_logits(c->stream, wf, (int32_t)rows, cols, x, s_rows, out));
      return KMOE_OK;
    }
    LAUNCH(c, "quant_q8", launch_quant_q8(c->stream, x, s_rows, cols, qr.q, qr.d, qr.s));  // quant.rs:282-310
    LAUNCH(c, "matvec_unpacked", launch_mv_unpacked(c->stream, t, w, rows, cols, rb, qr.q, qr.d, qr.s, s_rows, out));
    return KMOE_OK;
  }
  if (t == KMOE_F32) {  // quant.rs:242 (s_rows >= 4) or :311-327 (dequant + quant::dot): summation order kept
    if (rows > (int64_t)INT32_MAX) return fail(c, KMOE_E_INVALID, "too many rows");
    LAUNCH(c, "matmul_f32_ordered",
           launch_router_logits(c->stream, (const float *)w, (int32_t)rows, cols, x, s_rows, out));
    return KMOE_OK;
  }
  if (!int_path(c->regime, s_rows)) {
    // Q4_K rows: the bf16-split kernel (exact products on the bf16 matrix
    // cores); other types, or unaligned buffers, the fp32 GEMM
    if (t == KMOE_Q4_K) {
      const hipError_t e = timed(c, "f32_rows_plain", [&]() {
        return launch_f32_rows_plain(c->stream, t, w, rows, cols, x, s_rows, out);
      });
      if (e == hipSuccess) return KMOE_OK;
      if (e != hipErrorNotSupported) HIP_OK(c, e);
    }
    LAUNCH(c, "gemm_f32", launch_matmul_f32(c->stream, t, w, rows, cols, x, s_rows, out, qr.part, qr.part_floats));
    return KMOE_OK;
  }
  // One row of at most 4096 columns: Q8_K of x inside the matvec kernel (every
  // work-group quantizes the row into LDS), no kernel before it. Measured:
  // 4096x4096 6.5 -> 5.3 µs, 14336x4096 13.9 -> 12.4 µs per call; at 14336
  // columns the per-work-group quantization (56 KB of x each) made it slower
  // (13.6 -> 16.7 µs), so wider rows keep the separate quantization.
  if (t == KMOE_Q4_K && s_rows == 1 && cols <= 4096) {
    const hipError_t e = timed(c, "matvec_q4k", [&]() {
      return launch_dec_rows(c->stream, w, rows, cols, nullptr, nullptr, nullptr, out, nullptr, x);
    });
    if (e == hipSuccess) return KMOE_OK;
    if (e != hipErrorNotSupported) HIP_OK(c, e);
  }
  // Narrower Q4_K rows and Q6_K rows of at most 4096 columns: the register
  // kernel quantizes x itself (the kernel the separate quantization would
  // feed, so the same bits).
  if ((t == KMOE_Q4_K || t == KMOE_Q6_K) && s_rows == 1 && cols <= 4096) {
    const hipError_t e = timed(c, t == KMOE_Q4_K ? "matvec_q4k" : "matvec_q6k", [&]() {
      return launch_decode_plain_fx(c->stream, t, w, rows, cols, x, out);
    });
    if (e == hipSuccess) return KMOE_OK;
    if (e != hipErrorNotSupported) HIP_OK(c, e);
  }
  if (is_kq(t)) LAUNCH(c, "quant_q8k", launch_quant_q8k(c->stream, x, s_rows, cols, qr.q, qr.d, qr.s));
  else LAUNCH(c, "quant_q8", launch_quant_q8(c->stream, x, s_rows, cols, qr.q, qr.d, qr.s));
  return matvec_q8_impl(c, t, w, rows, cols, qr.q, qr.d, qr.s, s_rows, out);
}

}  // namespace

extern "C" {

int kmoe_abi_version(void) { return KMOE_ABI_VERSION; }

int kmoe_create(int device, kmoe_ctx **out) {
  if (!out) return KMOE_E_INVALID;
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return KMOE_E_INVALID;
  DeviceGuard g(device);
  kmoe_ctx *c = new kmoe_ctx();
  c->device = device;
  if (hipStreamCreateWithFlags(&c->own, hipStreamNonBlocking) != hipSuccess) {
    delete c;
    return KMOE_E_HIP;
  }
  c->stream = c->own;
  // completion counters of multi-work-group kernels; zero between calls
  if (hipMalloc((void **)&c->counters, kCounterWords * 4) != hipSuccess ||
      hipMemset(c->counters, 0, kCounterWords * 4) != hipSuccess) {
    (void)hipStreamDestroy(c->own);
    delete c;
    return KMOE_E_HIP;
  }
  size_t fr = 0, tot = 0;
  if (hipMemGetInfo(&fr, &tot) == hipSuccess) c->vram_limit = tot;
  if (device < kMaxDevices) {  // this device's copy of the no-alloc scratch (device current here)
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[device]) {
      void *p = nullptr;
      if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
        (void)hipGetLastError();
        (void)hipFree(c->counters);
        (void)hipStreamDestroy(c->own);
        delete c;
        return KMOE_E_HIP;
      }
      g_scratch[device] = p;
    }
  }
  *out = c;
  return KMOE_OK;
}

int kmoe_destroy(kmoe_ctx *c) {
  if (!c) return KMOE_OK;
  DeviceGuard g(c->device);
  (void)hipStreamSynchronize(c->stream);
  prof_drain(c);
  for (auto &kv : c->layers) {
    (void)hipFree(kv.second.arena);
    (void)hipFree(kv.second.router);
    if (kv.second.sh.arena) (void)hipFree(kv.second.sh.arena);
  }
  for (auto &kv : c->user_allocs) (void)hipFree(kv.first);
  if (c->ws) (void)hipFree(c->ws);
  if (c->stage) (void)hipFree(c->stage);
  if (c->hio) (void)hipFree(c->hio);
  if (c->dws) (void)hipFree(c->dws);
  if (c->aws) (void)hipFree(c->aws);
  if (c->counters) (void)hipFree(c->counters);
  if (c->own) (void)hipStreamDestroy(c->own);
  delete c;
  return KMOE_OK;
}

const char *kmoe_last_error(const kmoe_ctx *c) { return c ? c->err.c_str() : "null context"; }

int kmoe_set_stream(kmoe_ctx *c, void *s) {
  if (!c) return KMOE_E_INVALID;
  c->stream = (hipStream_t)s;  // NULL is the null stream, not "our own"
  return KMOE_OK;
}
int kmoe_use_own_stream(kmoe_ctx *c) {
  if (!c) return KMOE_E_INVALID;
  c->stream = c->own;
  return KMOE_OK;
}
void *kmoe_get_stream(kmoe_ctx *c) { return c ? (void *)c->stream : nullptr; }

int kmoe_synchronize(kmoe_ctx *c) {
  if (!c) return KMOE_E_INVALID;
  DeviceGuard g(c->device);
  HIP_OK(c, hipStreamSynchronize(c->stream));
  return KMOE_OK;
}

int kmoe_workspace_generation(const kmoe_ctx *c, uint64_t *gen) {
  if (!c || !gen) return KMOE_E_INVALID;
  *gen = c->ws_gen;
  return KMOE_OK;
}

int kmoe_set_regime(kmoe_ctx *c, int regime) {
  if (!c) return KMOE_E_INVALID;
  if (regime < KMOE_REGIME_AVX2 || regime > KMOE_REGIME_EXACT) return fail(c, KMOE_E_INVALID, "bad regime %d", regime);
  c->regime = regime;
  return KMOE_OK;
}
int kmoe_get_regime(const kmoe_ctx *c) { return c ? c->regime : -1; }

int kmoe_vram_set_limit(kmoe_ctx *c, uint64_t limit) {
  if (!c) return KMOE_E_INVALID;
  if (limit == 0) {
    DeviceGuard g(c->device);
    size_t fr = 0, tot = 0;
    HIP_OK(c, hipMemGetInfo(&fr, &tot));
    limit = tot;
  }
  if (limit < c->vram_reserved)
    return fail(c, KMOE_E_BUDGET, "limit %llu below the %llu bytes already reserved", (unsigned long long)limit,
                (unsigned long long)c->vram_reserved);
  c->vram_limit = limit;
  return KMOE_OK;
}

int kmoe_vram_usage(const kmoe_ctx *c, uint64_t *reserved, uint64_t *limit) {
  if (!c) return KMOE_E_INVALID;
  if (reserved) *reserved = c->vram_reserved;
  if (limit) *limit = c->vram_limit;
  return KMOE_OK;
}

int kmoe_device_alloc(kmoe_ctx *c, size_t bytes, void **dev) {
  if (!c || !dev) return KMOE_E_INVALID;
  DeviceGuard g(c->device);
  int rc = dev_alloc(c, bytes, dev, "caller buffer");
  if (rc) return rc;
  c->user_allocs[*dev] = bytes;
  return KMOE_OK;
}

int kmoe_device_free(kmoe_ctx *c, void *dev) {
  if (!c) return KMOE_E_INVALID;
  auto it = c->user_allocs.find(dev);
  if (it == c->user_allocs.end()) return fail(c, KMOE_E_INVALID, "pointer not allocated by kmoe_device_alloc");
  DeviceGuard g(c->device);
  HIP_OK(c, hipStreamSynchronize(c->stream));
  HIP_OK(c, hipFree(dev));
  release(c, it->second);
  c->user_allocs.erase(it);
  return KMOE_OK;
}

int kmoe_copy_h2d(kmoe_ctx *c, void *dst, const void *src, size_t bytes) {
  if (!c || (!dst && bytes) || (!src && bytes)) return KMOE_E_INVALID;
  DeviceGuard g(c->device);
  HIP_OK(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
  HIP_OK(c, hipStreamSynchronize(c->stream));
  return KMOE_OK;
}

int kmoe_copy_d2h(kmoe_ctx *c, void *dst, const void *src, size_t bytes) {
  if (!c || (!dst && bytes) || (!src && bytes)) return KMOE_E_INVALID;
  DeviceGuard g(c->device);
  HIP_OK(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
  HIP_OK(c, hipStreamSynchronize(c->stream));
  return KMOE_OK;
}

// ------------------------------------------------------------------ kernels

int kmoe_quantize_q8k(kmoe_ctx *c, const float *x, int64_t s_rows, int64_t cols, int8_t *q, float *d, int32_t *bs) {
  if (!c) return KMOE_E_INVALID;
  if (s_rows < 0 || cols <= 0 || cols % 256 != 0) return fail(c, KMOE_E_INVALID, "Q8_K needs cols %% 256 == 0");
  if (s_rows == 0) return KMOE_OK;
  if (!x || !q || !d || !bs) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  LAUNCH(c, "quant_q8k", launch_quant_q8k(c->stream, x, s_rows, cols, q, d, bs));
  return KMOE_OK;
}

int kmoe_quantize_q8(kmoe_ctx *c, const float *x, int64_t s_rows, int64_t cols, int8_t *q, float *d, int32_t *s16) {
  if (!c) return KMOE_E_INVALID;
  if (s_rows < 0 || cols <= 0 || cols % 32 != 0) return fail(c, KMOE_E_INVALID, "Q8 needs cols %% 32 == 0");
  if (s_rows == 0) return KMOE_OK;
  if (!x || !q || !d || !s16) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  LAUNCH(c, "quant_q8", launch_quant_q8(c->stream, x, s_rows, cols, q, d, s16));
  return KMOE_OK;
}

int kmoe_matvec_q8(kmoe_ctx *c, int t, const void *w, size_t w_len, int64_t rows, int64_t cols, const int8_t *q,
                   const float *d, const int32_t *bs, int64_t s_rows, float *out) {
  if (!c) return KMOE_E_INVALID;
  if (int rc_ = reject_tiled(c, w)) return rc_;
  int rc = check_quant_shape(c, t, cols);
  if (rc) return rc;
  if (rows < 0 || s_rows < 0) return fail(c, KMOE_E_INVALID, "negative size");
  if ((uint64_t)w_len < (uint64_t)bytes_for(t, cols) * (uint64_t)rows)
    return fail(c, KMOE_E_INVALID, "weight buffer %zu < %lld x %lld", w_len, (long long)rows,
                (long long)bytes_for(t, cols));
  if (rows == 0 || s_rows == 0) return KMOE_OK;
  if (!w || !q || !d || !out || (is_kq(t) && !bs)) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  return matvec_q8_impl(c, t, (const uint8_t *)w, rows, cols, q, d, bs, s_rows, out);
}

int kmoe_q4k_block_sums(kmoe_ctx *c, const void *w, int64_t rows, int64_t cols, const int8_t *q, const int32_t *bs,
                        int64_t s_rows, int32_t *sumi, int32_t *mins) {
  if (!c) return KMOE_E_INVALID;
  if (int rc_ = reject_tiled(c, w)) return rc_;
  int rc = check_quant_shape(c, KMOE_Q4_K, cols);
  if (rc) return rc;
  if (rows == 0 || s_rows == 0) return KMOE_OK;
  if (!w || !q || !bs || !sumi || !mins) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  if (s_rows >= kMfmaMinRows) {  // the matrix-core kernel's integers (same rows as the matmul above)
    hipError_t e = timed(c, "block_sums_q4k_mfma", [&]() {
      return launch_plain_mfma(c->stream, (const uint8_t *)w, rows, cols, q, nullptr, bs, s_rows, nullptr, sumi,
                               mins);
    });
    if (e == hipSuccess) return KMOE_OK;
    if (e != hipErrorNotSupported) HIP_OK(c, e);
  }
  LAUNCH(c, "block_sums_q4k",
         launch_block_sums(c->stream, KMOE_Q4_K, (const uint8_t *)w, rows, cols, q, bs, s_rows, sumi, mins));
  return KMOE_OK;
}

int kmoe_q6k_block_sums(kmoe_ctx *c, const void *w, int64_t rows, int64_t cols, const int8_t *q, const int32_t *bs,
                        int64_t s_rows, int32_t *sumi, int32_t *offs) {
  if (!c) return KMOE_E_INVALID;
  if (int rc_ = reject_tiled(c, w)) return rc_;
  int rc = check_quant_shape(c, KMOE_Q6_K, cols);
  if (rc) return rc;
  if (rows == 0 || s_rows == 0) return KMOE_OK;
  if (!w || !q || !bs || !sumi || !offs) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  LAUNCH(c, "block_sums_q6k",
         launch_block_sums(c->stream, KMOE_Q6_K, (const uint8_t *)w, rows, cols, q, bs, s_rows, sumi, offs));
  return KMOE_OK;
}

int kmoe_q8_0_block_sums(kmoe_ctx *c, const void *w, int64_t rows, int64_t cols, const int8_t *q, int64_t s_rows,
                         int32_t *p) {
  if (!c) return KMOE_E_INVALID;
  if (int rc_ = reject_tiled(c, w)) return rc_;
  int rc = check_quant_shape(c, KMOE_Q8_0, cols);
  if (rc) return rc;
  if (rows == 0 || s_rows == 0) return KMOE_OK;
  if (!w || !q || !p) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  LAUNCH(c, "block_sums_q8_0",
         launch_block_sums(c->stream, KMOE_Q8_0, (const uint8_t *)w, rows, cols, q, nullptr, s_rows, p, nullptr));
  return KMOE_OK;
}

int kmoe_matmul(kmoe_ctx *c, int t, const void *w, size_t w_len, int64_t rows, int64_t cols, const float *x,
                int64_t s_rows, float *out) {
  if (!c) return KMOE_E_INVALID;
  if (int rc_ = reject_tiled(c, w)) return rc_;
  if (rows < 0 || cols <= 0 || s_rows < 0) return fail(c, KMOE_E_INVALID, "bad shape");
  const int64_t rb = bytes_for(t, cols);
  if (block_size(t) < 0) return fail(c, KMOE_E_UNSUPPORTED, "ggml type %d has no kernel", t);
  if (rb < 0) return fail(c, KMOE_E_INVALID, "cols %lld not a multiple of the block size", (long long)cols);
  if ((uint64_t)w_len < (uint64_t)rb * (uint64_t)rows)
    return fail(c, KMOE_E_INVALID, "weight buffer %zu < %lld x %lld", w_len, (long long)rows, (long long)rb);
  if (rows == 0 || s_rows == 0) return KMOE_OK;
  if (!w || !x || !out) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  const bool xt = xtype(t);
  if (t != KMOE_F32 && !xt) {
    int rc = check_quant_shape(c, t, cols);
    if (rc) return rc;
  }
  // int8 activations (or the f32 path's partial sums) go to the workspace;
  // the other types' f32 path also stages the dequantized rows there
  const int64_t pf = gemm_f32_part_floats(rows, cols, 1, s_rows, s_rows);
  const bool staged = xt && (t == KMOE_F16 || t == KMOE_BF16 || !int_path(c->regime, s_rows));
  size_t need = 0;
  carve_qrows(nullptr, s_rows, cols, &need, pf);
  const size_t wf_off = need;
  if (staged) need = wf_off + align_up((size_t)rows * (size_t)cols * 4);
  int rc = ensure_ws(c, need);
  if (rc) return rc;
  size_t qn = 0;
  QRows qr = carve_qrows(c->ws, s_rows, cols, &qn, pf);
  return matmul_core(c, t, (const uint8_t *)w, rows, cols, x, s_rows, out, qr,
                     staged ? (float *)(c->ws + wf_off) : nullptr);
}

int kmoe_matmul_host(kmoe_ctx *c, int t, const void *w, size_t w_len, int64_t rows, int64_t cols, const float *x,
                     int64_t s_rows, float *out) {
  if (!c) return KMOE_E_INVALID;
  if (rows < 0 || cols <= 0 || s_rows < 0) return fail(c, KMOE_E_INVALID, "bad shape");
  const int64_t rb = bytes_for(t, cols);
  if (block_size(t) < 0) return fail(c, KMOE_E_UNSUPPORTED, "ggml type %d has no kernel", t);
  if (rb < 0) return fail(c, KMOE_E_INVALID, "cols %lld not a multiple of the block size", (long long)cols);
  if ((uint64_t)w_len < (uint64_t)rb * (uint64_t)rows)
    return fail(c, KMOE_E_INVALID, "weight buffer %zu < %lld x %lld", w_len, (long long)rows, (long long)rb);
  if (rows == 0 || s_rows == 0) return KMOE_OK;
  if (!w || !x || !out) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  const bool wdev = is_device_ptr(w);
  const size_t wb = wdev ? 0 : align_up((size_t)(rb * rows)), xb = align_up((size_t)(s_rows * cols) * 4);
  const size_t ob = (size_t)(s_rows * rows) * 4;
  int rc = ensure_hio(c, wb + xb + ob);
  if (rc) return rc;
  uint8_t *wd = wdev ? (uint8_t *)w : c->hio;
  float *xd = (float *)(c->hio + wb), *od = (float *)(c->hio + wb + xb);
  if (!wdev) HIP_OK(c, hipMemcpyAsync(wd, w, (size_t)(rb * rows), hipMemcpyHostToDevice, c->stream));
  HIP_OK(c, hipMemcpyAsync(xd, x, (size_t)(s_rows * cols) * 4, hipMemcpyHostToDevice, c->stream));
  rc = kmoe_matmul(c, t, wd, wdev ? w_len : (size_t)(rb * rows), rows, cols, xd, s_rows, od);
  if (rc) return rc;
  HIP_OK(c, hipMemcpyAsync(out, od, ob, hipMemcpyDeviceToHost, c->stream));
  HIP_OK(c, hipStreamSynchronize(c->stream));
  return KMOE_OK;
}

int kmoe_route(kmoe_ctx *c, const float *router, int32_t E, int64_t d, const float *h, int64_t S, int32_t k,
               int32_t norm_topk, float weights_scale, uint32_t *idx, float *w, float *logits) {
  if (!c) return KMOE_E_INVALID;
  if (E <= 0 || E > 512 || k <= 0 || k > 16 || k > E || d <= 0 || S < 0)
    return fail(c, KMOE_E_INVALID, "route: need 0 < k <= min(E, 16), E <= 512");
  if (S == 0) return KMOE_OK;
  if (!router || !h || !idx || !w) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  if (S < 4) {  // fused decode routing; its dispatch outputs go to scratch
    const size_t n = (size_t)S * k;
    int rc = ensure_ws(c, 4 * align_up(n * 4) + 3 * align_up(((size_t)E + 1) * 4) + align_up((size_t)S * E * 4));
    if (rc) return rc;
    Carver cv{c->ws};
    uint32_t *perm = cv.take<uint32_t>(n), *inv = cv.take<uint32_t>(n);
    uint32_t *off = cv.take<uint32_t>(E + 1);
    int32_t *na = cv.take<int32_t>(1), *act = cv.take<int32_t>(E);
    float *lgs = cv.take<float>(S * E);
    float *lg_out = logits ? logits : lgs;
    hipError_t e = timed(c, "route_decode", [&]() {
      return launch_route_decode(c->stream, router, E, d, h, (int32_t)S, k, norm_topk, weights_scale, lg_out, idx, w,
                                 perm, off, inv, na, act, 0, nullptr, nullptr, nullptr, c->counters);
    });
    if (e == hipSuccess) return KMOE_OK;
    if (e != hipErrorNotSupported) HIP_OK(c, e);
  }
  float *lg = logits;
  if (!lg) {
    int rc = ensure_ws(c, align_up((size_t)S * E * 4));
    if (rc) return rc;
    lg = (float *)c->ws;
  }
  LAUNCH(c, "router_logits", launch_router_logits(c->stream, router, E, d, h, S, lg));
  LAUNCH(c, "route_topk", launch_route_topk(c->stream, lg, S, E, k, norm_topk, weights_scale, idx, w));
  return KMOE_OK;
}

int kmoe_dispatch(kmoe_ctx *c, const uint32_t *idx, int64_t S, int32_t k, int32_t E, uint32_t *perm, uint32_t *off) {
  if (!c) return KMOE_E_INVALID;
  if (E <= 0 || E > 512 || k <= 0 || S < 0) return fail(c, KMOE_E_INVALID, "dispatch: bad sizes");
  if (!idx || !perm || !off) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  int rc = ensure_ws(c, align_up((size_t)S * k * 4));
  if (rc) return rc;
  LAUNCH(c, "dispatch",
         launch_dispatch(c->stream, idx, S * k, E, perm, off, nullptr, nullptr, nullptr, (uint32_t *)c->ws));
  return KMOE_OK;
}

// ------------------------------------------------------------ expert tier

int kmoe_layer_create(kmoe_ctx *c, uint32_t layer, const kmoe_moe_desc *desc) {
  if (!c || !desc) return KMOE_E_INVALID;
  const kmoe_moe_desc &D = *desc;
  if (c->layers.count(layer)) return fail(c, KMOE_E_INVALID, "layer %u already exists", layer);
  if (D.n_expert == 0 || D.n_expert > 512 || D.n_expert_used == 0 || D.n_expert_used > 16 ||
      D.n_expert_used > D.n_expert)
    return fail(c, KMOE_E_INVALID, "need 0 < n_expert_used <= min(n_expert, 16), n_expert <= 512");
  if (D.gate_type != D.up_type) return fail(c, KMOE_E_UNSUPPORTED, "gate and up must share a ggml type");
  int rc = check_quant_shape(c, D.gate_type, D.n_embd);
  if (!rc) rc = check_quant_shape(c, D.down_type, D.n_ff);
  if (rc) return rc;
  if (D.n_ff % 64 != 0) return fail(c, KMOE_E_UNSUPPORTED, "n_ff %% 64 != 0");
  Layer L;
  L.desc = D;
  L.part_len[0] = (size_t)bytes_for(D.gate_type, D.n_embd) * D.n_ff;
  L.part_len[1] = (size_t)bytes_for(D.up_type, D.n_embd) * D.n_ff;
  L.part_len[2] = (size_t)bytes_for(D.down_type, D.n_ff) * D.n_embd;
  L.part_off[0] = 0;
  L.part_off[1] = align_up(L.part_len[0]);
  L.part_off[2] = L.part_off[1] + align_up(L.part_len[1]);
  L.expert_stride = L.part_off[2] + align_up(L.part_len[2]);
  const int32_t ptype[3] = {D.gate_type, D.up_type, D.down_type};
  for (int p = 0; p < 3; ++p) {
    L.part_type[p] = ptype[p];
    L.tiled[p] = ptype[p] == KMOE_Q4_K || ptype[p] == KMOE_Q6_K;
    L.part_rows[p] = p < 2 ? D.n_ff : D.n_embd;
    L.part_nb[p] = (p < 2 ? D.n_embd : D.n_ff) / 256;
  }
  const size_t arena = L.expert_stride * D.n_expert;
  const size_t router = align_up((size_t)D.n_expert * D.n_embd * 4);
  DeviceGuard g(c->device);
  void *p = nullptr;
  rc = dev_alloc(c, arena, &p, "expert tier");
  if (rc) return rc;
  L.arena = (uint8_t *)p;
  rc = dev_alloc(c, router, &p, "router");
  if (rc) {
    (void)hipFree(L.arena);
    release(c, arena);
    return rc;
  }
  L.router = (float *)p;
  L.reserved = arena + router;
  L.loaded.assign(D.n_expert, 0);
  c->layers[layer] = L;
  return KMOE_OK;
}

int kmoe_layer_destroy(kmoe_ctx *c, uint32_t layer) {
  if (!c) return KMOE_E_INVALID;
  auto it = c->layers.find(layer);
  if (it == c->layers.end()) return fail(c, KMOE_E_NOT_LOADED, "layer %u not created", layer);
  DeviceGuard g(c->device);
  HIP_OK(c, hipStreamSynchronize(c->stream));
  (void)hipFree(it->second.arena);
  (void)hipFree(it->second.router);
  release(c, it->second.reserved);
  if (it->second.sh.arena) {
    (void)hipFree(it->second.sh.arena);
    release(c, it->second.sh.reserved);
  }
  c->layers.erase(it);
  return KMOE_OK;
}

static Layer *find_layer(kmoe_ctx *c, uint32_t layer) {
  auto it = c->layers.find(layer);
  return it == c->layers.end() ? nullptr : &it->second;
}

int kmoe_router_upload(kmoe_ctx *c, uint32_t layer, const float *router, size_t bytes) {
  if (!c) return KMOE_E_INVALID;
  Layer *L = find_layer(c, layer);
  if (!L) return fail(c, KMOE_E_NOT_LOADED, "layer %u not created", layer);
  const size_t need = (size_t)L->desc.n_expert * L->desc.n_embd * 4;
  if (bytes != need || !router) return fail(c, KMOE_E_INVALID, "router bytes %zu != %zu", bytes, need);
  DeviceGuard g(c->device);
  HIP_OK(c, hipMemcpyAsync(L->router, router, bytes, hipMemcpyHostToDevice, c->stream));
  HIP_OK(c, hipStreamSynchronize(c->stream));
  L->router_ok = true;
  return KMOE_OK;
}

// Enqueue the placement of part `part` of expert e from device memory: a copy
// for verbatim parts, the tiling kernel for Q4_K / Q6_K.
static int place_from_device(kmoe_ctx *c, Layer *L, uint32_t e, int part, const uint8_t *src) {
  uint8_t *dst = L->arena + e * L->expert_stride + L->part_off[part];
  if (!L->tiled[part])
    HIP_OK(c, hipMemcpyAsync(dst, src, L->part_len[part], hipMemcpyDeviceToDevice, c->stream));
  else if (L->part_type[part] == KMOE_Q6_K)
    HIP_OK(c, launch_tq6_convert(c->stream, src, dst, L->part_rows[part], L->part_nb[part], true));
  else
    HIP_OK(c, launch_tq4_convert(c->stream, src, dst, L->part_rows[part], L->part_nb[part], true));
  return KMOE_OK;
}

// Enqueue the placement of a part from host memory. Verbatim parts go straight
// into the tier; tiled parts go through the device staging and the tiling
// kernel, or are tiled on the host when no staging can be had. Returns with
// the stream synchronized only on the host-tiling route.
static int place_from_host(kmoe_ctx *c, Layer *L, uint32_t e, int part, const uint8_t *src) {
  const size_t len = L->part_len[part];
  uint8_t *dst = L->arena + e * L->expert_stride + L->part_off[part];
  if (!L->tiled[part]) {
    HIP_OK(c, hipMemcpyAsync(dst, src, len, hipMemcpyHostToDevice, c->stream));
    return KMOE_OK;
  }
  if (uint8_t *st = staging(c, len)) {
    HIP_OK(c, hipMemcpyAsync(st, src, len, hipMemcpyHostToDevice, c->stream));
    return place_from_device(c, L, e, part, st);
  }
  std::vector<uint8_t> t(len);
  if (L->part_type[part] == KMOE_Q6_K)
    tq6_convert_host(src, t.data(), L->part_rows[part], L->part_nb[part], true);
  else
    tq4_convert_host(src, t.data(), L->part_rows[part], L->part_nb[part], true);
  HIP_OK(c, hipMemcpyAsync(dst, t.data(), len, hipMemcpyHostToDevice, c->stream));
  HIP_OK(c, hipStreamSynchronize(c->stream));  // t is released on return
  return KMOE_OK;
}

static int expert_upload(kmoe_ctx *c, uint32_t layer, uint32_t e, int32_t part, const void *bytes, size_t len,
                         bool from_device) {
  if (!c) return KMOE_E_INVALID;
  Layer *L = find_layer(c, layer);
  if (!L) return fail(c, KMOE_E_NOT_LOADED, "layer %u not created", layer);
  if (e >= L->desc.n_expert || part < 0 || part > 2) return fail(c, KMOE_E_INVALID, "expert %u part %d", e, part);
  if (len != L->part_len[part] || !bytes)
    return fail(c, KMOE_E_INVALID, "expert part bytes %zu != %zu", len, L->part_len[part]);
  DeviceGuard g(c->device);
  const uint8_t *src = (const uint8_t *)bytes;
  int rc = from_device ? place_from_device(c, L, e, part, src) : place_from_host(c, L, e, part, src);
  if (rc) return rc;
  HIP_OK(c, hipStreamSynchronize(c->stream));
  L->loaded[e] |= (uint8_t)(1u << part);
  return KMOE_OK;
}

int kmoe_expert_upload_buf(kmoe_ctx *c, uint32_t layer, uint32_t e, const void *buf, size_t len,
                           const uint64_t part_pos[3]) {
  if (!c) return KMOE_E_INVALID;
  Layer *L = find_layer(c, layer);
  if (!L) return fail(c, KMOE_E_NOT_LOADED, "layer %u not created", layer);
  if (e >= L->desc.n_expert || !buf || !part_pos) return fail(c, KMOE_E_INVALID, "expert %u buffer", e);
  for (int k = 0; k < 3; ++k)
    if (part_pos[k] > len || L->part_len[k] > len - part_pos[k])
      return fail(c, KMOE_E_INVALID, "part %d at %llu + %zu bytes overruns the %zu-byte buffer", k,
                  (unsigned long long)part_pos[k], L->part_len[k], len);
  DeviceGuard g(c->device);
  const uint8_t *host = (const uint8_t *)buf;
  if (uint8_t *st = staging(c, len)) {
    HIP_OK(c, hipMemcpyAsync(st, host, len, hipMemcpyHostToDevice, c->stream));
    for (int k = 0; k < 3; ++k) {
      int rc = place_from_device(c, L, e, k, st + part_pos[k]);
      if (rc) return rc;
    }
  } else {
    for (int k = 0; k < 3; ++k) {
      int rc = place_from_host(c, L, e, k, host + part_pos[k]);
      if (rc) return rc;
    }
  }
  HIP_OK(c, hipStreamSynchronize(c->stream));
  L->loaded[e] = 7;
  return KMOE_OK;
}

namespace {
struct HostRange {
  uintptr_t start, end;
};
}  // namespace

int kmoe_layer_preload(kmoe_ctx *c, uint32_t layer, const void *const part_base[3], const uint64_t part_stride[3],
                       uint64_t *copies) {
  if (!c) return KMOE_E_INVALID;
  Layer *L = find_layer(c, layer);
  if (!L) return fail(c, KMOE_E_NOT_LOADED, "layer %u not created", layer);
  if (!part_base || !part_stride || !part_base[0] || !part_base[1] || !part_base[2])
    return fail(c, KMOE_E_INVALID, "need three part bases and strides");
  constexpr uintptr_t kMergeGap = 4096;  // DIRECT_ALIGN: closer ranges are read as one
  DeviceGuard g(c->device);
  uint64_t n_copies = 0;
  for (uint32_t e = 0; e < L->desc.n_expert; ++e) {
    HostRange r[3];
    for (int k = 0; k < 3; ++k) {
      r[k].start = (uintptr_t)part_base[k] + (uintptr_t)e * part_stride[k];
      r[k].end = r[k].start + L->part_len[k];
    }
    std::sort(r, r + 3, [](const HostRange &a, const HostRange &b) { return a.start < b.start; });
    HostRange m[3];
    int nm = 0;
    for (int k = 0; k < 3; ++k) {
      if (nm && r[k].start < m[nm - 1].end + kMergeGap) {
        m[nm - 1].end = std::max(m[nm - 1].end, r[k].end);
        continue;
      }
      m[nm++] = r[k];
    }
    size_t pos[3], need = 0;
    for (int i = 0; i < nm; ++i) {
      pos[i] = need;
      need += align_up(m[i].end - m[i].start);
    }
    uint8_t *st = staging(c, need);
    if (!st) {  // no room for the extents: part by part
      for (int k = 0; k < 3; ++k) {
        const uint8_t *src = (const uint8_t *)part_base[k] + (size_t)e * part_stride[k];
        int rc = place_from_host(c, L, e, k, src);
        if (rc) return rc;
      }
      n_copies += 3;
      continue;
    }
    for (int i = 0; i < nm; ++i)
      HIP_OK(c, hipMemcpyAsync(st + pos[i], (const void *)m[i].start, m[i].end - m[i].start,
                               hipMemcpyHostToDevice, c->stream));
    n_copies += nm;
    for (int k = 0; k < 3; ++k) {
      const uintptr_t s = (uintptr_t)part_base[k] + (uintptr_t)e * part_stride[k];
      int i = 0;
      while (!(s >= m[i].start && s + L->part_len[k] <= m[i].end)) ++i;
      int rc = place_from_device(c, L, e, k, st + pos[i] + (s - m[i].start));
      if (rc) return rc;
    }
  }
  HIP_OK(c, hipStreamSynchronize(c->stream));
  std::fill(L->loaded.begin(), L->loaded.end(), (uint8_t)7);
  if (copies) *copies = n_copies;
  return KMOE_OK;
}

int kmoe_expert_upload(kmoe_ctx *c, uint32_t layer, uint32_t e, int32_t part, const void *bytes, size_t len) {
  return expert_upload(c, layer, e, part, bytes, len, false);
}
int kmoe_expert_upload_dev(kmoe_ctx *c, uint32_t layer, uint32_t e, int32_t part, const void *bytes, size_t len) {
  return expert_upload(c, layer, e, part, bytes, len, true);
}

int kmoe_expert_is_ready(kmoe_ctx *c, uint32_t layer, uint32_t e) {
  if (!c) return 0;
  Layer *L = find_layer(c, layer);
  if (!L || e >= L->desc.n_expert) return 0;
  return L->loaded[e] == 7 ? 1 : 0;
}

int kmoe_expert_part(kmoe_ctx *c, uint32_t layer, uint32_t e, int32_t part, const void **dev, size_t *len) {
  if (!c || !dev || !len) return KMOE_E_INVALID;
  Layer *L = find_layer(c, layer);
  if (!L) return fail(c, KMOE_E_NOT_LOADED, "layer %u not created", layer);
  if (e >= L->desc.n_expert || part < 0 || part > 2) return fail(c, KMOE_E_INVALID, "expert %u part %d", e, part);
  if (!(L->loaded[e] & (1u << part))) return fail(c, KMOE_E_NOT_LOADED, "expert %u part %d not resident", e, part);
  *dev = L->arena + e * L->expert_stride + L->part_off[part];
  *len = L->part_len[part];
  return KMOE_OK;
}

int kmoe_expert_part_layout(kmoe_ctx *c, uint32_t layer, uint32_t e, int32_t part, int32_t *layout) {
  if (!c || !layout) return KMOE_E_INVALID;
  Layer *L = find_layer(c, layer);
  if (!L) return fail(c, KMOE_E_NOT_LOADED, "layer %u not created", layer);
  if (e >= L->desc.n_expert || part < 0 || part > 2) return fail(c, KMOE_E_INVALID, "expert %u part %d", e, part);
  *layout = L->tiled[part] ? KMOE_LAYOUT_TILED : KMOE_LAYOUT_GGUF;
  return KMOE_OK;
}

int kmoe_shared_expert_create(kmoe_ctx *c, uint32_t layer, int64_t n_ff, int32_t gate_type, int32_t up_type,
                              int32_t down_type) {
  if (!c) return KMOE_E_INVALID;
  Layer *L = find_layer(c, layer);
  if (!L) return fail(c, KMOE_E_NOT_LOADED, "layer %u not created", layer);
  if (L->sh.arena) return fail(c, KMOE_E_INVALID, "layer %u already has a shared expert", layer);
  if (n_ff <= 0) return fail(c, KMOE_E_INVALID, "bad n_ff");
  const int64_t d = L->desc.n_embd;
  const int32_t ty[3] = {gate_type, up_type, down_type};
  const int64_t cols[3] = {d, d, n_ff}, rows[3] = {n_ff, n_ff, d};
  auto &S = L->sh;
  size_t off = 0;
  for (int p = 0; p < 3; ++p) {
    if (block_size(ty[p]) < 0) return fail(c, KMOE_E_UNSUPPORTED, "ggml type %d has no kernel", ty[p]);
    if (ty[p] != KMOE_F32) {
      int rc = check_quant_shape(c, ty[p], cols[p]);
      if (rc) return rc;
    }
    const int64_t rb = bytes_for(ty[p], cols[p]);
    if (rb < 0) return fail(c, KMOE_E_INVALID, "cols %lld not a multiple of the block size", (long long)cols[p]);
    S.len[p] = (size_t)rb * (size_t)rows[p];
    S.off[p] = off;
    off += align_up(S.len[p]);
  }
  const size_t gate_off = off;
  off += align_up((size_t)d * 4);
  DeviceGuard g(c->device);
  void *p = nullptr;
  int rc = dev_alloc(c, off, &p, "shared expert");
  if (rc) return rc;
  S.arena = (uint8_t *)p;
  S.reserved = off;
  S.gate_inp = (float *)(S.arena + gate_off);
  S.n_ff = n_ff;
  for (int i = 0; i < 3; ++i) S.type[i] = ty[i];
  S.on = true;
  S.loaded = 0;
  S.gate_ok = false;
  return KMOE_OK;
}

int kmoe_shared_expert_upload(kmoe_ctx *c, uint32_t layer, int32_t part, const void *bytes, size_t len) {
  if (!c) return KMOE_E_INVALID;
  Layer *L = find_layer(c, layer);
  if (!L) return fail(c, KMOE_E_NOT_LOADED, "layer %u not created", layer);
  auto &S = L->sh;
  if (!S.arena) return fail(c, KMOE_E_NOT_LOADED, "layer %u has no shared expert", layer);
  if (part < 0 || part > 2) return fail(c, KMOE_E_INVALID, "part %d", part);
  if (!bytes || len != S.len[part]) return fail(c, KMOE_E_INVALID, "shared part bytes %zu != %zu", len, S.len[part]);
  DeviceGuard g(c->device);
  HIP_OK(c, hipMemcpyAsync(S.arena + S.off[part], bytes, len, hipMemcpyHostToDevice, c->stream));
  HIP_OK(c, hipStreamSynchronize(c->stream));
  S.loaded |= (uint8_t)(1u << part);
  return KMOE_OK;
}

int kmoe_shared_gate_upload(kmoe_ctx *c, uint32_t layer, const float *gate_inp, size_t bytes) {
  if (!c) return KMOE_E_INVALID;
  Layer *L = find_layer(c, layer);
  if (!L) return fail(c, KMOE_E_NOT_LOADED, "layer %u not created", layer);
  auto &S = L->sh;
  if (!S.arena) return fail(c, KMOE_E_NOT_LOADED, "layer %u has no shared expert", layer);
  const size_t need = (size_t)L->desc.n_embd * 4;
  if (!gate_inp || bytes != need) return fail(c, KMOE_E_INVALID, "gate bytes %zu != %zu", bytes, need);
  DeviceGuard g(c->device);
  HIP_OK(c, hipMemcpyAsync(S.gate_inp, gate_inp, bytes, hipMemcpyHostToDevice, c->stream));
  HIP_OK(c, hipStreamSynchronize(c->stream));
  S.gate_ok = true;
  return KMOE_OK;
}

int kmoe_expert_read(kmoe_ctx *c, uint32_t layer, uint32_t e, int32_t part, void *host, size_t len) {
  if (!c) return KMOE_E_INVALID;
  const void *src = nullptr;
  size_t n = 0;
  int rc = kmoe_expert_part(c, layer, e, part, &src, &n);
  if (rc) return rc;
  if (!host || len != n) return fail(c, KMOE_E_INVALID, "expert part bytes %zu != %zu", len, n);
  Layer *L = find_layer(c, layer);
  DeviceGuard g(c->device);
  if (!L->tiled[part]) {
    HIP_OK(c, hipMemcpyAsync(host, src, n, hipMemcpyDeviceToHost, c->stream));
    HIP_OK(c, hipStreamSynchronize(c->stream));
    return KMOE_OK;
  }
  std::vector<uint8_t> t(n);
  HIP_OK(c, hipMemcpyAsync(t.data(), src, n, hipMemcpyDeviceToHost, c->stream));
  HIP_OK(c, hipStreamSynchronize(c->stream));
  if (L->part_type[part] == KMOE_Q6_K)
    tq6_convert_host(t.data(), (uint8_t *)host, L->part_rows[part], L->part_nb[part], false);
  else
    tq4_convert_host(t.data(), (uint8_t *)host, L->part_rows[part], L->part_nb[part], false);
  return KMOE_OK;
}

int kmoe_bytes_per_expert(kmoe_ctx *c, uint32_t layer, uint64_t *bytes) {
  if (!c || !bytes) return KMOE_E_INVALID;
  Layer *L = find_layer(c, layer);
  if (!L) return fail(c, KMOE_E_NOT_LOADED, "layer %u not created", layer);
  *bytes = L->part_len[0] + L->part_len[1] + L->part_len[2];
  return KMOE_OK;
}

// --------------------------------------------------------------- moe_ffn

// The MoE FFN of h; with norm, h is norm->f and is produced here first
// (x += y, f = rmsnorm(x) * w), folded into the single-token router kernel
// where it supports the shapes, else by the norm kernel.
static int moe_ffn(kmoe_ctx *c, uint32_t layer, const float *h, int64_t S, float *out, const RouteNorm *norm,
                   const kmoe_moe_dbg *dbg = nullptr, uint8_t *fixed_ws = nullptr, size_t fixed_size = 0) {
  if (!c) return KMOE_E_INVALID;
  Layer *L = find_layer(c, layer);
  if (!L) return fail(c, KMOE_E_NOT_LOADED, "layer %u not created", layer);
  if (S < 0) return fail(c, KMOE_E_INVALID, "negative s_rows");
  if (S == 0) return KMOE_OK;
  if (!h || !out) return fail(c, KMOE_E_INVALID, "null pointer");
  if (!L->router_ok) return fail(c, KMOE_E_NOT_LOADED, "layer %u router not uploaded", layer);
  for (uint32_t e = 0; e < L->desc.n_expert; ++e)
    if (L->loaded[e] != 7) return fail(c, KMOE_E_NOT_LOADED, "layer %u expert %u not resident", layer, e);
  if (L->sh.on && L->sh.loaded != 7) return fail(c, KMOE_E_NOT_LOADED, "layer %u shared expert not resident", layer);
  const kmoe_moe_desc &D = L->desc;
  const int64_t E = D.n_expert, k = D.n_expert_used, d = D.n_embd, F = D.n_ff;
  const int64_t slots = S * k;
  if (slots > (int64_t)UINT32_MAX / 2) return fail(c, KMOE_E_INVALID, "too many tokens");
  size_t need = 0;
  carve_moe(nullptr, S, E, k, d, F, &need);
  const size_t moe_need = align_up(need);
  size_t sh_need = 0;
  const int64_t Fs = L->sh.n_ff, mx = d > Fs ? d : Fs;
  if (L->sh.on) {  // gs, us [S, Fs] (one span), ys [S, d], gate logits [S], int8 scratch [S, max(d, Fs)]
    Carver cv{nullptr};
    cv.take<float>(2 * S * Fs);
    cv.take<float>(S * d);
    cv.take<float>(S);
    size_t q = 0;
    carve_qrows(nullptr, S, mx, &q, sh_part_floats(Fs, d, S));
    sh_need = cv.off + align_up(q);
  }
  DeviceGuard g(c->device);
  int rc = KMOE_OK;
  uint8_t *wsb = fixed_ws;  // the caller's fixed workspace, or the context's (grown here)
  if (fixed_ws) {
    if (moe_need + sh_need > fixed_size)
      return fail(c, KMOE_E_INVALID,
                  "%lld tokens of layer %u need %zu bytes of workspace, past the %zu-byte static scratch",
                  (long long)S, layer, moe_need + sh_need, fixed_size);
  } else {
    rc = ensure_ws(c, moe_need + sh_need);
    if (rc) return rc;
    wsb = c->ws;
  }
  size_t tmp;
  MoeWs w = carve_moe(wsb, S, E, k, d, F, &tmp);
  const int regime = c->regime;
  hipStream_t st = c->stream;
  // The shared expert's workspace: gate/up outputs [S, 2 Fs], ys [S, d], its
  // gate logits [S] and its int8 rows.
  float *sh_gs = nullptr, *sh_us = nullptr, *sh_ys = nullptr, *sh_gl = nullptr;
  QRows sh_qr{};
  if (L->sh.on) {
    Carver cv{wsb + moe_need};
    sh_gs = cv.take<float>(2 * S * Fs);
    sh_us = sh_gs + S * Fs;
    sh_ys = cv.take<float>(S * d);
    sh_gl = cv.take<float>(S);
    size_t q = 0;
    sh_qr = carve_qrows(wsb + moe_need + cv.off, S, mx, &q, sh_part_floats(Fs, d, S));
  }
  // One token on the int8 path, the shared gate and up of one type stored
  // back to back (one [2 Fs, d] matrix): one product over both reads the int8
  // row of h made for the routed experts (the same Q8KRow / Q8Row
  // quantization) and one kernel applies SwiGLU and quantizes its output.
  auto sh_fast = [&](bool x_is_int) {
    const auto &SH = L->sh;
    return L->sh.on && S == 1 && x_is_int && int_path(regime, 1) && SH.type[0] != KMOE_F32 &&
           SH.type[1] == SH.type[0] && SH.type[2] != KMOE_F32 && is_kq(SH.type[0]) == is_kq(D.gate_type) &&
           SH.off[1] == SH.off[0] + SH.len[0];
  };
  bool sh_front_done = false;  // the shared gate/up and SwiGLU + int8 rows are done
  bool sh_done = false;        // and its add into out
  auto sh_front = [&]() -> int {
    const auto &SH = L->sh;
    if (SH.gate_ok) LAUNCH(c, "shared_gate", launch_router_logits(st, SH.gate_inp, 1, d, h, S, sh_gl, true));
    const int r = matvec_q8_impl(c, SH.type[0], SH.arena + SH.off[0], 2 * Fs, d, w.xq, w.xd, w.xs, 1, sh_gs);
    if (r) return r;
    LAUNCH(c, "shared_swiglu_quant", launch_swiglu_quant(st, SH.type[2], sh_gs, Fs, sh_qr.q, sh_qr.d, sh_qr.s));
    sh_front_done = true;
    return KMOE_OK;
  };
  // Capture of the int-path integers (kmoe_moe_ffn_dbg): zeroed here, added to by the kernels.
  BlockDbg gdbg, ddbg;
  const BlockDbg *gd = nullptr, *dd = nullptr;
  const int64_t bel_g = D.gate_type == KMOE_Q8_0 ? 32 : 256, bel_d = D.down_type == KMOE_Q8_0 ? 32 : 256;
  if (dbg) {
    const size_t ng = (size_t)slots * F * (d / bel_g) * 4, nd = (size_t)slots * d * (F / bel_d) * 4;
    int32_t *const arr[6] = {dbg->gate_sumi, dbg->gate_mins, dbg->up_sumi, dbg->up_mins, dbg->down_sumi,
                             dbg->down_mins};
    for (int i = 0; i < 6; ++i)
      if (arr[i]) HIP_OK(c, hipMemsetAsync(arr[i], 0, i < 4 ? ng : nd, st));
    gdbg.s[0] = dbg->gate_sumi;
    gdbg.m[0] = dbg->gate_mins;
    gdbg.s[1] = dbg->up_sumi;
    gdbg.m[1] = dbg->up_mins;
    ddbg.s[0] = dbg->down_sumi;
    ddbg.m[0] = dbg->down_mins;
    gd = &gdbg;
    dd = &ddbg;
  }
  bool x_int = false, h_int = false;  // int8 rows of x / h were produced (for the capture)
  // the norm, where the router kernel does not take it
  bool norm_pending = norm != nullptr;
  auto run_norm = [&]() -> int {
    if (!norm_pending) return KMOE_OK;
    norm_pending = false;
    LAUNCH(c, "rmsnorm", launch_add_rmsnorm(st, norm->x, norm->y, norm->w, S, d, norm->eps, norm->f));
    return KMOE_OK;
  };
  if (norm_pending && !route_norm_supported(norm, (int32_t)S, d)) {
    rc = run_norm();
    if (rc) return rc;
  }

  const int gt = D.gate_type, dt = D.down_type;
  {
  // route (transformer.rs:474-496) and dispatch (transformer.rs:525-531). With
  // s_rows < 4 one fused work-group also quantizes x for the int8 path.
  bool x_quantized = false;
  // Single token on the int8 path with Q4_K experts: the router kernel only
  // produces the logits (and the int8 row) and the gate/up kernel selects the
  // experts itself, publishing the routing for the kernels after it.
  bool select_in_gate_up = S == 1 && regime != KMOE_REGIME_EXACT &&
                           decode_gate_up_can_select(gt, d, (int32_t)E, (int32_t)k);
  {
    const int qtype = regime == KMOE_REGIME_EXACT ? 0 : gt;
    hipError_t e = timed(c, "route_decode", [&]() {
      return launch_route_decode(st, L->router, (int32_t)E, d, h, (int32_t)S, (int32_t)k, D.norm_topk,
                                 D.weights_scale, w.logits, w.idx, w.wsel, w.perm, w.offsets, w.inv, w.n_active,
                                 w.active, qtype, w.xq, w.xd, w.xs, select_in_gate_up ? nullptr : c->counters,
                                 norm_pending ? norm : nullptr);
    });
    if (e == hipSuccess) {
      x_quantized = qtype != 0;
      norm_pending = false;
    } else {
      if (e != hipErrorNotSupported) HIP_OK(c, e);
      rc = run_norm();
      if (rc) return rc;
      select_in_gate_up = false;
      // the int8 rows of x come from extra work-groups of the router launch
      const int qkind = regime == KMOE_REGIME_EXACT ? 0 : is_kq(gt) ? 1 : 2;
      LAUNCH(c, "router_logits", launch_router_logits(st, L->router, (int32_t)E, d, h, S, w.logits, false, qkind,
                                                      w.xq, w.xd, w.xs));
      x_quantized = qkind != 0;
      LAUNCH(c, "route_topk", launch_route_topk(st, w.logits, S, (int32_t)E, (int32_t)k, D.norm_topk,
                                                D.weights_scale, w.idx, w.wsel));
      LAUNCH(c, "dispatch", launch_dispatch(st, w.idx, slots, (int32_t)E, w.perm, w.offsets, w.inv, w.n_active,
                                            w.active, w.rank));
    }
  }
  Routing rt{w.n_active, w.active, w.offsets, w.perm, w.inv, w.wsel, (int32_t)k};
  ExpertTier tier{L->arena, (int64_t)L->expert_stride,
                  {(int64_t)L->part_off[0], (int64_t)L->part_off[1], (int64_t)L->part_off[2]}};
  const int max_active = (int)(slots < E ? slots : E);
  // Which regimes can occur: an expert has at most S rows.
  const bool any_int = regime == KMOE_REGIME_INT8 || (regime == KMOE_REGIME_AVX2);
  const bool any_f32 = regime == KMOE_REGIME_EXACT || (regime == KMOE_REGIME_AVX2 && S >= 4);
  // Int8 regime with many token rows: grouped products on the int8 matrix cores;
  // while experts average at most 20 rows, those with at most 32 take the
  // streaming kernel (more rows per expert leave too many on the other one).
  const bool mfma = regime == KMOE_REGIME_INT8 && S >= kMfmaMinRows;
  const int ring_rows = slots <= 20 * E ? 32 : 0;

  // Single token, int8 path: every routed expert has one row. gate/up+SwiGLU
  // and down+combine run as register-resident decode kernels.
  if (S == 1 && regime != KMOE_REGIME_EXACT) {
    if (!x_quantized) {
      if (is_kq(gt)) LAUNCH(c, "quant_q8k", launch_quant_q8k(st, h, 1, d, w.xq, w.xd, w.xs));
      else LAUNCH(c, "quant_q8", launch_quant_q8(st, h, 1, d, w.xq, w.xd, w.xs));
      x_quantized = true;
    }
    DecSelect ds;
    ds.logits = w.logits;
    ds.E = (int32_t)E;
    ds.K = (int32_t)k;
    ds.norm_topk = D.norm_topk;
    ds.weights_scale = D.weights_scale;
    ds.idx = w.idx;
    ds.wsel = w.wsel;
    ds.perm = w.perm;
    ds.offsets = w.offsets;
    ds.inv = w.inv;
    ds.n_active = w.n_active;
    ds.active = w.active;
    x_int = true;
    // The shared expert's gate/up as extra items of the same launch, where the
    // experts take the register kernel (SwiGLU into its row).
    bool sgu_done = false;
    hipError_t e = hipErrorNotSupported;
    if (!gd && sh_fast(true) && L->sh.type[0] == gt) {
      const SharedGateUp sgu{L->sh.arena + L->sh.off[0], Fs, sh_gs};
      e = timed(c, "moe_gate_up_dec", [&]() {
        return launch_decode_gate_up(st, gt, tier, F, d, rt, max_active, w.xq, w.xd, w.xs, w.h,
                                     select_in_gate_up ? &ds : nullptr, gd, &sgu);
      });
      if (e == hipSuccess) sgu_done = true;
      else if (e != hipErrorNotSupported) HIP_OK(c, e);
    }
    if (!sgu_done)
      e = timed(c, "moe_gate_up_dec", [&]() {
        return launch_decode_gate_up(st, gt, tier, F, d, rt, max_active, w.xq, w.xd, w.xs, w.h,
                                     select_in_gate_up ? &ds : nullptr, gd);
      });
    if (e == hipErrorNotSupported && select_in_gate_up) {  // complete the routing from the logits, then as below
      LAUNCH(c, "route_topk", launch_route_topk(st, w.logits, S, (int32_t)E, (int32_t)k, D.norm_topk,
                                                D.weights_scale, w.idx, w.wsel));
      LAUNCH(c, "dispatch", launch_dispatch(st, w.idx, slots, (int32_t)E, w.perm, w.offsets, w.inv, w.n_active,
                                            w.active, w.rank));
      select_in_gate_up = false;
      e = timed(c, "moe_gate_up_dec", [&]() {
        return launch_decode_gate_up(st, gt, tier, F, d, rt, max_active, w.xq, w.xd, w.xs, w.h, nullptr, gd);
      });
    }
    if (e != hipErrorNotSupported) {
      HIP_OK(c, e);
      // one row per expert: every slot is on the int8 path in either int8 regime
      if (sgu_done) {  // the slots' and the shared row's int8 rows in one launch
        const auto &SH = L->sh;
        LAUNCH(c, "quant_slots_shared", launch_quant_two(st, dt, w.h, slots * F, w.hq, w.hd, w.hs, SH.type[2],
                                                          sh_gs, Fs, sh_qr.q, sh_qr.d, sh_qr.s));
        if (SH.gate_ok) LAUNCH(c, "shared_gate", launch_router_logits(st, SH.gate_inp, 1, d, h, S, sh_gl, true));
        sh_front_done = true;
      } else {
        LAUNCH(c, is_kq(dt) ? "quant_slots_q8k" : "quant_slots_q8",
               launch_quant_slots(st, dt, w.h, slots, F, rt, w.idx, KMOE_REGIME_INT8, w.hq, w.hd, w.hs));
      }
      h_int = true;
      if (!dd && sh_fast(x_int)) {  // the shared expert's down row in the routed down kernel
        if (!sh_front_done) {
          rc = sh_front();
          if (rc) return rc;
        }
        const auto &SH = L->sh;
        const SharedDown sd{SH.type[2], SH.arena + SH.off[2], Fs, sh_qr.q, sh_qr.d, sh_qr.s,
                            SH.gate_ok ? sh_gl : nullptr};
        e = timed(c, "moe_down_shared", [&]() {
          return launch_decode_down_shared(st, dt, tier, d, F, rt, w.hq, w.hd, w.hs, out, sd);
        });
        if (e == hipSuccess) {
          sh_done = true;
          goto done;
        }
        if (e != hipErrorNotSupported) HIP_OK(c, e);
      }
      e = timed(c, "moe_down_dec",
                [&]() { return launch_decode_down_combine(st, dt, tier, d, F, rt, w.hq, w.hd, w.hs, out, dd); });
      if (e != hipErrorNotSupported) {
        HIP_OK(c, e);
        goto done;
      }
      // down too wide for registers: finish with the general kernels below
      LAUNCH(c, "moe_down_int",
             launch_moe_int(st, 1, dt, tier, d, F, rt, regime, max_active, S, w.hq, w.hd, w.hs, w.y, 0, dd));
      LAUNCH(c, "combine", launch_combine(st, w.y, rt, S, d, out));
      goto done;
    }
  }
  // Experts with a few rows on the int path (decode batches), tiled Q4_K:
  // the few-rows kernels; experts with more rows take the kernels after them.
  const bool small_ok = S >= 2;
  // expert gate/up + SwiGLU (transformer.rs:551-558)
  if (any_int) {
    if (!x_quantized) {
      if (is_kq(gt)) LAUNCH(c, "quant_q8k", launch_quant_q8k(st, h, S, d, w.xq, w.xd, w.xs));
      else LAUNCH(c, "quant_q8", launch_quant_q8(st, h, S, d, w.xq, w.xd, w.xs));
    }
    x_int = true;
    int small_rows = 0;  // experts with 1..small_rows rows are done
    if (small_ok && gt == KMOE_Q4_K && L->tiled[0] && small_supported(F, d, 0)) {
      const hipError_t e = timed(c, "moe_gate_up_small", [&]() {
        return launch_small(st, 0, tier, F, d, rt, regime, max_active, S, w.xq, w.xd, w.xs, w.h, gd);
      });
      if (e == hipSuccess) small_rows = small_rows_for(d, 0, S);
      else if (e != hipErrorNotSupported) HIP_OK(c, e);
    }
    if (small_ok && small_rows == 0 && (gt == KMOE_Q8_0 || (L->tiled[0] && L->tiled[1]))) {  // narrow rows, 1-3 rows
      const hipError_t e = timed(c, "moe_gate_up_few", [&]() {
        return launch_few_int(st, 0, gt, tier, F, d, rt, regime, max_active, w.xq, w.xd, w.xs, w.h, kFewRows, gd);
      });
      if (e == hipSuccess) small_rows = kFewRows;
      else if (e != hipErrorNotSupported) HIP_OK(c, e);
    }
    // AVX2 regime: experts of 4 or more rows are the f32 path's
    const bool more_int = regime == KMOE_REGIME_INT8 || small_rows < 3;
    if (S > small_rows && more_int) {
      hipError_t e = hipErrorNotSupported;
      if (mfma && gt == KMOE_Q4_K)
        e = timed(c, "moe_gate_up_mfma", [&]() {
          return launch_moe_mfma(st, 0, tier, F, d, rt, regime, max_active, w.xq, w.xd, w.xs, w.h, small_rows + 1,
                                 (int)S, ring_rows, gd);
        });
      if (e != hipErrorNotSupported) HIP_OK(c, e);
      else
        LAUNCH(c, "moe_gate_up_int", launch_moe_int(st, 0, gt, tier, F, d, rt, regime, max_active, S, w.xq, w.xd,
                                                    w.xs, w.h, small_rows + 1, gd));
    }
  }
  // The f32 regime's experts (quant.rs:242-260): tiled Q4_K rows stream
  // through the bf16-split kernels (blocks of up to 64 token rows), gate and
  // up in one launch; other row types take the staged GEMM.
  const int f32_lo = regime == KMOE_REGIME_EXACT ? 1 : 4;
  const int f32_hi = (int)S;
  if (any_f32) {
    int f32_done = 0;  // experts with f32_lo..f32_done rows are done
    if (gt == KMOE_Q4_K && L->tiled[0] && L->tiled[1] && f32_hi >= f32_lo) {
      const hipError_t e = timed(c, "moe_gate_up_f32_rows", [&]() {
        return launch_f32_rows(st, 0, gt, tier, F, d, rt, regime, max_active, slots, f32_lo, f32_hi, h, w.h);
      });
      if (e == hipSuccess) f32_done = f32_hi;
      else if (e != hipErrorNotSupported) HIP_OK(c, e);
    }
    if (S > f32_done) {
      LAUNCH(c, "moe_gate_f32", launch_moe_f32(st, 0, gt, tier, F, d, rt, regime, max_active, S, slots, h, w.h,
                                               w.part, w.part_floats, f32_done + 1));
      LAUNCH(c, "moe_up_f32", launch_moe_f32(st, 1, gt, tier, F, d, rt, regime, max_active, S, slots, h, w.h,
                                             w.part, w.part_floats, f32_done + 1));
    }
  }
  // down (transformer.rs:559-560)
  if (any_int) {
    LAUNCH(c, is_kq(dt) ? "quant_slots_q8k" : "quant_slots_q8",
           launch_quant_slots(st, dt, w.h, slots, F, rt, w.idx, regime, w.hq, w.hd, w.hs));
    h_int = true;
    int small_rows = 0;
    if (small_ok && dt == KMOE_Q4_K && L->tiled[2] && small_supported(d, F, 1)) {
      const hipError_t e = timed(c, "moe_down_small", [&]() {
        return launch_small(st, 1, tier, d, F, rt, regime, max_active, S, w.hq, w.hd, w.hs, w.y, dd);
      });
      if (e == hipSuccess) small_rows = small_rows_for(F, 1, S);
      else if (e != hipErrorNotSupported) HIP_OK(c, e);
    }
    if (small_ok && small_rows == 0 && (dt == KMOE_Q8_0 || L->tiled[2])) {
      const hipError_t e = timed(c, "moe_down_few", [&]() {
        return launch_few_int(st, 1, dt, tier, d, F, rt, regime, max_active, w.hq, w.hd, w.hs, w.y, kFewRows, dd);
      });
      if (e == hipSuccess) small_rows = kFewRows;
      else if (e != hipErrorNotSupported) HIP_OK(c, e);
    }
    if (S > small_rows && (regime == KMOE_REGIME_INT8 || small_rows < 3)) {
      hipError_t e = hipErrorNotSupported;
      if (mfma && dt == KMOE_Q4_K)
        e = timed(c, "moe_down_mfma", [&]() {
          return launch_moe_mfma(st, 1, tier, d, F, rt, regime, max_active, w.hq, w.hd, w.hs, w.y, small_rows + 1,
                                 (int)S, ring_rows, dd);
        });
      if (e != hipErrorNotSupported) HIP_OK(c, e);
      else
        LAUNCH(c, "moe_down_int", launch_moe_int(st, 1, dt, tier, d, F, rt, regime, max_active, S, w.hq, w.hd,
                                                 w.hs, w.y, small_rows + 1, dd));
    }
  }
  if (any_f32) {
    int f32_done = 0;
    if (dt == KMOE_Q4_K && L->tiled[2] && f32_hi >= f32_lo) {
      const hipError_t e = timed(c, "moe_down_f32_rows", [&]() {
        return launch_f32_rows(st, 1, dt, tier, d, F, rt, regime, max_active, slots, f32_lo, f32_hi, w.h, w.y);
      });
      if (e == hipSuccess) f32_done = f32_hi;
      else if (e != hipErrorNotSupported) HIP_OK(c, e);
    }
    if (S > f32_done)
      LAUNCH(c, "moe_down_f32", launch_moe_f32(st, 2, dt, tier, d, F, rt, regime, max_active, S, slots, w.h, w.y,
                                               w.part, w.part_floats, f32_done + 1));
  }
  // combine (transformer.rs:566-570)
  LAUNCH(c, "combine", launch_combine(st, w.y, rt, S, d, out));
  }

done:
  if (dbg) {  // the int8 rows the products read, as the workspace holds them
    auto cp = [&](void *dst, const void *src, size_t n) -> int {
      if (dst && n) HIP_OK(c, hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, st));
      return KMOE_OK;
    };
    if (x_int) {
      rc = cp(dbg->xq, w.xq, (size_t)S * d);
      if (!rc) rc = cp(dbg->xd, w.xd, (size_t)S * (d / bel_g) * 4);
      if (!rc) rc = cp(dbg->xs, w.xs, (size_t)S * (d / 16) * 4);
      if (rc) return rc;
    }
    if (h_int) {
      rc = cp(dbg->hq, w.hq, (size_t)slots * F);
      if (!rc) rc = cp(dbg->hd, w.hd, (size_t)slots * (F / bel_d) * 4);
      if (!rc) rc = cp(dbg->hs, w.hs, (size_t)slots * (F / 16) * 4);
      if (rc) return rc;
    }
  }
  if (L->sh.on && !sh_done) {  // shared expert after the routed combine (transformer.rs:572-587)
    auto &SH = L->sh;
    float *gs = sh_gs, *us = sh_us, *ys = sh_ys, *gl = sh_gl;
    const QRows &qr = sh_qr;
    // One token on the int8 path: the fast front (above), then the down
    // product adds its gated result into out. Same arithmetic as the general
    // sequence below.
    const int t2 = SH.type[2];
    if (sh_fast(x_int)) {
      if (!sh_front_done) {
        rc = sh_front();
        if (rc) return rc;
      }
      const AddEpi epi{SH.gate_ok ? gl : nullptr};
      const hipError_t e = timed(c, "shared_down_add", [&]() {
        return launch_decode_plain(st, t2, SH.arena + SH.off[2], d, Fs, qr.q, qr.d, qr.s, out, &epi);
      });
      if (e == hipErrorNotSupported) {  // row too wide for registers: plain product, then the add
        rc = matvec_q8_impl(c, t2, SH.arena + SH.off[2], d, Fs, qr.q, qr.d, qr.s, 1, ys);
        if (rc) return rc;
        LAUNCH(c, "shared_add", launch_shared_add(st, out, ys, SH.gate_ok ? gl : nullptr, S, d));
      } else {
        HIP_OK(c, e);
      }
      goto shared_done;
    }
    // f32 regime, Q4_K gate and up: both products and SwiGLU in one launch
    hipError_t ef = hipErrorNotSupported;
    if (!int_path(c->regime, S) && SH.type[0] == KMOE_Q4_K && SH.type[1] == KMOE_Q4_K)
      ef = timed(c, "shared_gate_up_f32", [&]() {
        return launch_f32_rows_plain(st, KMOE_Q4_K, SH.arena + SH.off[0], Fs, d, h, S, gs, SH.arena + SH.off[1]);
      });
    if (ef != hipErrorNotSupported) {
      HIP_OK(c, ef);
    } else {
      rc = matmul_core(c, SH.type[0], SH.arena + SH.off[0], Fs, d, h, S, gs, qr);
      if (!rc) rc = matmul_core(c, SH.type[1], SH.arena + SH.off[1], Fs, d, h, S, us, qr);
      if (rc) return rc;
      LAUNCH(c, "shared_swiglu", launch_swiglu(st, gs, us, S * Fs));
    }
    rc = matmul_core(c, SH.type[2], SH.arena + SH.off[2], d, Fs, gs, S, ys, qr);
    if (rc) return rc;
    if (SH.gate_ok) LAUNCH(c, "shared_gate", launch_router_logits(st, SH.gate_inp, 1, d, h, S, gl, true));
    LAUNCH(c, "shared_add", launch_shared_add(st, out, ys, SH.gate_ok ? gl : nullptr, S, d));
  }
shared_done:
  c->last_idx = w.idx;
  c->last_w = w.wsel;
  c->last_perm = w.perm;
  c->last_off = w.offsets;
  c->last_slots = slots;
  c->last_E = (int32_t)E;
  return KMOE_OK;
}

int kmoe_moe_ffn(kmoe_ctx *c, uint32_t layer, const float *h, int64_t S, float *out) {
  return moe_ffn(c, layer, h, S, out, nullptr);
}

int kmoe_moe_ffn_dbg(kmoe_ctx *c, uint32_t layer, const float *h, int64_t S, float *out, const kmoe_moe_dbg *dbg) {
  if (!c) return KMOE_E_INVALID;
  if (!dbg || !dbg->gate_sumi || !dbg->up_sumi || !dbg->down_sumi)
    return fail(c, KMOE_E_INVALID, "kmoe_moe_ffn_dbg: null capture buffer");
  Layer *L = find_layer(c, layer);
  if (!L) return fail(c, KMOE_E_NOT_LOADED, "layer %u not created", layer);
  if ((is_kq(L->desc.gate_type) && (!dbg->gate_mins || !dbg->up_mins)) ||
      (is_kq(L->desc.down_type) && !dbg->down_mins))
    return fail(c, KMOE_E_INVALID, "kmoe_moe_ffn_dbg: K-quant parts need their mins/offs buffers");
  return moe_ffn(c, layer, h, S, out, nullptr, dbg);
}

int kmoe_moe_ffn_host(kmoe_ctx *c, uint32_t layer, const float *h, int64_t S, float *out) {
  if (!c) return KMOE_E_INVALID;
  Layer *L = find_layer(c, layer);
  if (!L) return fail(c, KMOE_E_NOT_LOADED, "layer %u not created", layer);
  if (S < 0) return fail(c, KMOE_E_INVALID, "negative s_rows");
  if (S == 0) return KMOE_OK;
  if (!h || !out) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  const size_t n = (size_t)S * L->desc.n_embd * 4, nb = align_up(n);
  int rc = ensure_hio(c, 2 * nb);
  if (rc) return rc;
  float *hd = (float *)c->hio, *od = (float *)(c->hio + nb);
  HIP_OK(c, hipMemcpyAsync(hd, h, n, hipMemcpyHostToDevice, c->stream));
  rc = moe_ffn(c, layer, hd, S, od, nullptr);
  if (rc) return rc;
  HIP_OK(c, hipMemcpyAsync(out, od, n, hipMemcpyDeviceToHost, c->stream));
  HIP_OK(c, hipStreamSynchronize(c->stream));
  return KMOE_OK;
}

int kmoe_moe_ffn_noalloc(kmoe_ctx *c, uint32_t layer, const float *h, int64_t S, float *out) {
  if (!c) return KMOE_E_INVALID;
  if (c->device >= kMaxDevices || !g_scratch[c->device])
    return fail(c, KMOE_E_HIP, "no static scratch on device %d", c->device);
  // no events either: profiling is suspended for the call
  const bool prof = c->prof;
  c->prof = false;
  const int rc = moe_ffn(c, layer, h, S, out, nullptr, nullptr, (uint8_t *)g_scratch[c->device], kScratchBytes);
  c->prof = prof;
  return rc;
}

int kmoe_norm_moe_ffn(kmoe_ctx *c, uint32_t layer, float *x, const float *y, const float *norm_w, float eps,
                      int64_t S, float *f, float *out) {
  if (!c) return KMOE_E_INVALID;
  if (S > 0 && (!x || !norm_w || !f)) return fail(c, KMOE_E_INVALID, "null pointer");
  const RouteNorm n{x, y, norm_w, eps, f, c->counters + kNormDone};
  return moe_ffn(c, layer, f, S, out, &n);
}

int kmoe_moe_last_routing(kmoe_ctx *c, uint32_t *idx, float *wv, uint32_t *perm, uint32_t *off) {
  if (!c) return KMOE_E_INVALID;
  if (!c->last_idx) return fail(c, KMOE_E_NOT_LOADED, "no kmoe_moe_ffn call yet");
  DeviceGuard g(c->device);
  const size_t n = (size_t)c->last_slots;
  if (idx) HIP_OK(c, hipMemcpyAsync(idx, c->last_idx, n * 4, hipMemcpyDeviceToDevice, c->stream));
  if (wv) HIP_OK(c, hipMemcpyAsync(wv, c->last_w, n * 4, hipMemcpyDeviceToDevice, c->stream));
  if (perm) HIP_OK(c, hipMemcpyAsync(perm, c->last_perm, n * 4, hipMemcpyDeviceToDevice, c->stream));
  if (off) HIP_OK(c, hipMemcpyAsync(off, c->last_off, (size_t)(c->last_E + 1) * 4, hipMemcpyDeviceToDevice, c->stream));
  return KMOE_OK;
}

// ------------------------------------------------------------- the rest of the decoder layer

static int check_table(kmoe_ctx *c, int32_t t, size_t table_len, int64_t n_rows, int64_t cols, int64_t *rb) {
  if (t != KMOE_F32 && t != KMOE_F16 && t != KMOE_Q8_0 && t != KMOE_Q4_K && t != KMOE_Q6_K)
    return fail(c, KMOE_E_UNSUPPORTED, "ggml type %d has no row kernel", t);
  *rb = t == KMOE_F16 ? 2 * cols : bytes_for(t, cols);
  if (n_rows <= 0 || cols <= 0 || *rb < 0)
    return fail(c, KMOE_E_INVALID, "cols %lld not a multiple of the block size", (long long)cols);
  if ((uint64_t)table_len < (uint64_t)*rb * (uint64_t)n_rows)
    return fail(c, KMOE_E_INVALID, "table buffer %zu < %lld x %lld", table_len, (long long)n_rows, (long long)*rb);
  return KMOE_OK;
}

int kmoe_get_rows(kmoe_ctx *c, int32_t t, const void *table, size_t table_len, int64_t n_rows, int64_t cols,
                  const uint32_t *ids, int64_t s_rows, float *out) {
  if (!c) return KMOE_E_INVALID;
  if (int rc_ = reject_tiled(c, table)) return rc_;
  int64_t rb = 0;
  int rc = check_table(c, t, table_len, n_rows, cols, &rb);
  if (rc) return rc;
  if (s_rows < 0) return fail(c, KMOE_E_INVALID, "negative size");
  if (s_rows == 0) return KMOE_OK;
  if (!table || !ids || !out) return fail(c, KMOE_E_INVALID, "null pointer");
  for (int64_t s = 0; s < s_rows; ++s)
    if (ids[s] >= (uint64_t)n_rows) return fail(c, KMOE_E_INVALID, "token id %u out of range", ids[s]);
  DeviceGuard g(c->device);
  rc = ensure_dws(c, (size_t)s_rows * 4);
  if (rc) return rc;
  uint32_t *ids_dev = (uint32_t *)c->dws;
  HIP_OK(c, hipMemcpyAsync(ids_dev, ids, (size_t)s_rows * 4, hipMemcpyHostToDevice, c->stream));
  LAUNCH(c, "get_rows", launch_get_rows(c->stream, t, (const uint8_t *)table, rb, n_rows, cols, ids_dev, s_rows, out));
  HIP_OK(c, hipStreamSynchronize(c->stream));  // the ids buffer is reused by the next call
  return KMOE_OK;
}

int kmoe_get_rows_dev(kmoe_ctx *c, int32_t t, const void *table, size_t table_len, int64_t n_rows, int64_t cols,
                      const uint32_t *ids_dev, int64_t s_rows, float *out) {
  if (!c) return KMOE_E_INVALID;
  if (int rc_ = reject_tiled(c, table)) return rc_;
  int64_t rb = 0;
  int rc = check_table(c, t, table_len, n_rows, cols, &rb);
  if (rc) return rc;
  if (s_rows < 0) return fail(c, KMOE_E_INVALID, "negative size");
  if (s_rows == 0) return KMOE_OK;
  if (!table || !ids_dev || !out) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  LAUNCH(c, "get_rows", launch_get_rows(c->stream, t, (const uint8_t *)table, rb, n_rows, cols, ids_dev, s_rows, out));
  return KMOE_OK;
}

int kmoe_rmsnorm(kmoe_ctx *c, float *x, const float *y, const float *w, int64_t rows, int64_t dim, float eps,
                 float *out) {
  if (!c) return KMOE_E_INVALID;
  if (rows < 0 || dim <= 0) return fail(c, KMOE_E_INVALID, "bad shape");
  if (rows == 0) return KMOE_OK;
  if (!x || !w || !out) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  LAUNCH(c, "rmsnorm", launch_add_rmsnorm(c->stream, x, y, w, rows, dim, eps, out));
  return KMOE_OK;
}

int kmoe_norm_matmul(kmoe_ctx *c, float *x, const float *y, const float *norm_w, float eps, int t, const void *w,
                     size_t w_len, int64_t rows, int64_t cols, int64_t s_rows, float *h, float *out) {
  if (!c) return KMOE_E_INVALID;
  if (int rc_ = reject_tiled(c, w)) return rc_;
  if (rows < 0 || cols <= 0 || s_rows < 0) return fail(c, KMOE_E_INVALID, "bad shape");
  const int64_t rb = bytes_for(t, cols);
  if (block_size(t) < 0) return fail(c, KMOE_E_UNSUPPORTED, "ggml type %d has no kernel", t);
  if (rb < 0) return fail(c, KMOE_E_INVALID, "cols %lld not a multiple of the block size", (long long)cols);
  if ((uint64_t)w_len < (uint64_t)rb * (uint64_t)rows)
    return fail(c, KMOE_E_INVALID, "weight buffer %zu < %lld x %lld", w_len, (long long)rows, (long long)rb);
  if (s_rows == 0) return KMOE_OK;
  if (!x || !norm_w || !w || !h || !out) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  if (t != KMOE_F32) {
    int rc = check_quant_shape(c, t, cols);
    if (rc) return rc;
  }
  const int64_t pf = gemm_f32_part_floats(rows, cols, 1, s_rows, s_rows);
  size_t need = 0;
  carve_qrows(nullptr, s_rows, cols, &need, pf);
  int rc = ensure_ws(c, need);
  if (rc) return rc;
  QRows qr = carve_qrows(c->ws, s_rows, cols, &need, pf);
  if (t != KMOE_F32 && int_path(c->regime, s_rows) && rows > 0) {
    hipError_t e = timed(c, "rmsnorm_quant", [&]() {
      return launch_rmsnorm_quant(c->stream, x, y, norm_w, s_rows, cols, eps, h, is_kq(t), qr.q, qr.d, qr.s);
    });
    if (e == hipSuccess) return matvec_q8_impl(c, t, (const uint8_t *)w, rows, cols, qr.q, qr.d, qr.s, s_rows, out);
    if (e != hipErrorNotSupported) HIP_OK(c, e);
  }
  LAUNCH(c, "rmsnorm", launch_add_rmsnorm(c->stream, x, y, norm_w, s_rows, cols, eps, h));
  if (rows == 0) return KMOE_OK;
  return matmul_core(c, t, (const uint8_t *)w, rows, cols, h, s_rows, out, qr);
}

// Position checks shared by rope, kv_store and attention: with a host
// position the rows must fit the context (EngineError::ContextFull,
// transformer.rs:278-282); a device position is checked by the kernels.
static int check_pos(kmoe_ctx *c, int64_t pos0, const int32_t *pos_dev, int64_t s_rows, int64_t n_ctx) {
  if (pos0 < 0 || s_rows < 0) return fail(c, KMOE_E_INVALID, "negative position or size");
  if (!pos_dev && n_ctx > 0 && pos0 + s_rows > n_ctx)
    return fail(c, KMOE_E_INVALID, "context full: need %lld positions, n_ctx %lld", (long long)(pos0 + s_rows),
                (long long)n_ctx);
  return KMOE_OK;
}

int kmoe_rope(kmoe_ctx *c, float *x, int64_t s_rows, int32_t n_heads, int32_t head_dim, int32_t rope_dim,
              int64_t pos0, const int32_t *pos_dev, const float *inv_freq, int32_t neox) {
  if (!c) return KMOE_E_INVALID;
  if (n_heads <= 0 || head_dim <= 0 || rope_dim <= 0 || rope_dim > head_dim || rope_dim % 2)
    return fail(c, KMOE_E_INVALID, "rope: need 0 < rope_dim <= head_dim, rope_dim even");
  int rc = check_pos(c, pos0, pos_dev, s_rows, 0);
  if (rc) return rc;
  if (s_rows == 0) return KMOE_OK;
  if (!x || !inv_freq) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  LAUNCH(c, "rope", launch_rope(c->stream, x, s_rows, n_heads, head_dim, rope_dim, pos0, pos_dev, inv_freq, neox));
  return KMOE_OK;
}

int kmoe_kv_store(kmoe_ctx *c, const float *k, const float *v, int64_t s_rows, int64_t kv_width, int64_t pos0,
                  const int32_t *pos_dev, int64_t n_ctx, uint16_t *k_cache, uint16_t *v_cache) {
  if (!c) return KMOE_E_INVALID;
  if (kv_width <= 0 || n_ctx <= 0) return fail(c, KMOE_E_INVALID, "bad shape");
  int rc = check_pos(c, pos0, pos_dev, s_rows, n_ctx);
  if (rc) return rc;
  if (s_rows == 0) return KMOE_OK;
  if (!k || !v || !k_cache || !v_cache) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  LAUNCH(c, "kv_store", launch_kv_store(c->stream, k, v, s_rows, kv_width, pos0, pos_dev, n_ctx, k_cache, v_cache));
  return KMOE_OK;
}

int kmoe_attention(kmoe_ctx *c, const float *q, const uint16_t *k_cache, const uint16_t *v_cache, int64_t s_rows,
                   int32_t n_head, int32_t n_kv, int32_t head_dim, int64_t pos0, const int32_t *pos_dev,
                   int64_t n_ctx, float *out) {
  if (!c) return KMOE_E_INVALID;
  if (n_head <= 0 || n_kv <= 0 || n_head % n_kv || n_ctx <= 0)
    return fail(c, KMOE_E_INVALID, "attention: need n_head %% n_kv == 0 and n_ctx > 0");
  if (!attn_supported(head_dim, n_head / n_kv))
    return fail(c, KMOE_E_UNSUPPORTED, "head_dim %d, %d query heads per kv head (kernels: 64 or 128, <= 16)",
                head_dim, n_head / n_kv);
  int rc = check_pos(c, pos0, pos_dev, s_rows, n_ctx);
  if (rc) return rc;
  if (s_rows == 0) return KMOE_OK;
  if (!q || !k_cache || !v_cache || !out) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  const int supers = attn_supers(pos_dev ? n_ctx : std::min(n_ctx, pos0 + s_rows));
  rc = ensure_aws(c, (size_t)s_rows * n_head, (size_t)attn_part_floats(s_rows, n_head, head_dim, supers) * 4);
  if (rc) return rc;
  LAUNCH(c, "attention",
         launch_attention(c->stream, q, k_cache, v_cache, s_rows, n_head, n_kv, head_dim, pos0, pos_dev, n_ctx,
                          supers, (float *)(c->aws + c->aws_counters), (uint32_t *)c->aws, out));
  return KMOE_OK;
}

int kmoe_attention_matmul(kmoe_ctx *c, const float *q, const uint16_t *k_cache, const uint16_t *v_cache,
                          int64_t s_rows, int32_t n_head, int32_t n_kv, int32_t head_dim, int64_t pos0,
                          const int32_t *pos_dev, int64_t n_ctx, float *attn, int t, const void *w, size_t w_len,
                          int64_t rows, float *out) {
  if (!c) return KMOE_E_INVALID;
  if (int rc_ = reject_tiled(c, w)) return rc_;
  if (n_head <= 0 || n_kv <= 0 || n_head % n_kv || n_ctx <= 0)
    return fail(c, KMOE_E_INVALID, "attention: need n_head %% n_kv == 0 and n_ctx > 0");
  if (!attn_supported(head_dim, n_head / n_kv))
    return fail(c, KMOE_E_UNSUPPORTED, "head_dim %d, %d query heads per kv head (kernels: 64 or 128, <= 16)",
                head_dim, n_head / n_kv);
  const int64_t cols = (int64_t)n_head * head_dim;
  const int64_t rb = bytes_for(t, cols);
  if (block_size(t) < 0) return fail(c, KMOE_E_UNSUPPORTED, "ggml type %d has no kernel", t);
  if (rb < 0 || rows < 0) return fail(c, KMOE_E_INVALID, "output projection shape");
  if ((uint64_t)w_len < (uint64_t)rb * (uint64_t)rows)
    return fail(c, KMOE_E_INVALID, "weight buffer %zu < %lld x %lld", w_len, (long long)rows, (long long)rb);
  int rc = check_pos(c, pos0, pos_dev, s_rows, n_ctx);
  if (rc) return rc;
  if (s_rows == 0) return KMOE_OK;
  if (!q || !k_cache || !v_cache || !attn || !w || !out) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  if (t != KMOE_F32) {
    rc = check_quant_shape(c, t, cols);
    if (rc) return rc;
  }
  const int supers = attn_supers(pos_dev ? n_ctx : std::min(n_ctx, pos0 + s_rows));
  rc = ensure_aws(c, (size_t)s_rows * n_head, (size_t)attn_part_floats(s_rows, n_head, head_dim, supers) * 4);
  if (rc) return rc;
  const int64_t pf = gemm_f32_part_floats(rows, cols, 1, s_rows, s_rows);
  size_t need = 0;
  carve_qrows(nullptr, s_rows, cols, &need, pf);
  rc = ensure_ws(c, need);
  if (rc) return rc;
  QRows qr = carve_qrows(c->ws, s_rows, cols, &need, pf);
  float *part = (float *)(c->aws + c->aws_counters);
  uint32_t *counters = (uint32_t *)c->aws;
  // Where the projection takes the integer path, the attention kernel writes
  // its int8 rows too (same values as the projection's own quantization).
  const int qt = t != KMOE_F32 && int_path(c->regime, s_rows) && rows > 0 ? (is_kq(t) ? 1 : 2) : 0;
  if (qt) {
    hipError_t e = timed(c, "attention_q8", [&]() {
      return launch_attention(c->stream, q, k_cache, v_cache, s_rows, n_head, n_kv, head_dim, pos0, pos_dev, n_ctx,
                              supers, part, counters, attn, qt, qr.q, qr.d, qr.s);
    });
    if (e == hipSuccess) return matvec_q8_impl(c, t, (const uint8_t *)w, rows, cols, qr.q, qr.d, qr.s, s_rows, out);
    if (e != hipErrorNotSupported) HIP_OK(c, e);
  }
  LAUNCH(c, "attention", launch_attention(c->stream, q, k_cache, v_cache, s_rows, n_head, n_kv, head_dim, pos0,
                                          pos_dev, n_ctx, supers, part, counters, attn));
  if (rows == 0) return KMOE_OK;
  return matmul_core(c, t, (const uint8_t *)w, rows, cols, attn, s_rows, out, qr);
}

int kmoe_rope_kv_store(kmoe_ctx *c, const float *q, const float *k, const float *v, int64_t s_rows, int32_t n_head,
                       int32_t n_kv, int32_t head_dim, int32_t rope_dim, int64_t pos0, const int32_t *pos_dev,
                       const float *inv_freq, int32_t neox, int64_t n_ctx, float *q_out, uint16_t *k_cache,
                       uint16_t *v_cache) {
  if (!c) return KMOE_E_INVALID;
  if (n_head <= 0 || n_kv <= 0 || head_dim <= 0 || rope_dim <= 0 || rope_dim > head_dim || rope_dim % 2 ||
      rope_dim > 256 || n_ctx <= 0)
    return fail(c, KMOE_E_INVALID, "rope: need 0 < rope_dim <= min(head_dim, 256), rope_dim even");
  int rc = check_pos(c, pos0, pos_dev, s_rows, n_ctx);
  if (rc) return rc;
  if (s_rows == 0) return KMOE_OK;
  if (!q || !k || !v || !inv_freq || !q_out || !k_cache || !v_cache)
    return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  LAUNCH(c, "rope_kv",
         launch_rope_kv(c->stream, q, k, v, s_rows, n_head, n_kv, head_dim, rope_dim, pos0, pos_dev, inv_freq, neox,
                        n_ctx, q_out, k_cache, v_cache));
  return KMOE_OK;
}

int kmoe_norm_matmul_rope_kv(kmoe_ctx *c, float *x, const float *y, const float *norm_w, float eps, int t,
                             const void *w, size_t w_len, int64_t cols, float *h, float *qkv, int32_t n_head,
                             int32_t n_kv, int32_t head_dim, int32_t rope_dim, int64_t pos0, const int32_t *pos_dev,
                             const float *inv_freq, int32_t neox, int64_t n_ctx, float *q_out, uint16_t *k_cache,
                             uint16_t *v_cache, float *x_out) {
  if (!c) return KMOE_E_INVALID;
  if (int rc_ = reject_tiled(c, w)) return rc_;
  if (x_out && x_out == x) x_out = nullptr;  // in place
  if (n_head <= 0 || n_kv <= 0 || head_dim <= 0 || rope_dim <= 0 || rope_dim > head_dim || rope_dim % 2 ||
      rope_dim > 256 || n_ctx <= 0)
    return fail(c, KMOE_E_INVALID, "rope: need 0 < rope_dim <= min(head_dim, 256), rope_dim even");
  int rc = check_pos(c, pos0, pos_dev, 1, n_ctx);
  if (rc) return rc;
  if (!qkv || !inv_freq || !q_out || !k_cache || !v_cache) return fail(c, KMOE_E_INVALID, "null pointer");
  const int64_t nq = (int64_t)n_head * head_dim, kvw = (int64_t)n_kv * head_dim, rows = nq + 2 * kvw;
  const bool int1 = t != KMOE_F32 && int_path(c->regime, 1) && block_size(t) > 0 && bytes_for(t, cols) > 0 &&
                    (uint64_t)w_len >= (uint64_t)bytes_for(t, cols) * (uint64_t)rows && x && norm_w && w && h &&
                    !check_quant_shape(c, t, cols);
  const QkvRope rp{n_head, n_kv, head_dim, rope_dim, neox, pos0, pos_dev, inv_freq, n_ctx, q_out, k_cache, v_cache};
  if (x_out) {
    if (!x) return fail(c, KMOE_E_INVALID, "null pointer");
    DeviceGuard g(c->device);
    if (int1) {  // one kernel: the norm inside the projection (K-quant rows), x + y into x_out
      const hipError_t e = timed(c, "matvec_qkv_rope", [&]() {
        const QkvNorm nm{x, y, norm_w, eps, h, x_out};
        return launch_matvec_qkv_rope_norm(c->stream, t, (const uint8_t *)w, rows, cols, nm, qkv, rp);
      });
      if (e == hipSuccess) return KMOE_OK;
      if (e != hipErrorNotSupported) HIP_OK(c, e);
    }
    // otherwise the in-place calls below on a copy of x in x_out
    HIP_OK(c, hipMemcpyAsync(x_out, x, (size_t)cols * 4, hipMemcpyDeviceToDevice, c->stream));
    x = x_out;
  }
  // one token on the integer path: norm + int8 rows, then the projection with
  // RoPE and the cache store in its epilogue
  if (int1) {
    DeviceGuard g(c->device);
    size_t need = 0;
    carve_qrows(nullptr, 1, cols, &need, 0);
    rc = ensure_ws(c, need);
    if (rc) return rc;
    QRows qr = carve_qrows(c->ws, 1, cols, &need, 0);
    hipError_t e = timed(c, "rmsnorm_quant", [&]() {
      return launch_rmsnorm_quant(c->stream, x, y, norm_w, 1, cols, eps, h, is_kq(t), qr.q, qr.d, qr.s);
    });
    if (e == hipSuccess) {
      e = timed(c, "matvec_qkv_rope", [&]() {
        return launch_matvec_qkv_rope(c->stream, t, (const uint8_t *)w, rows, cols, qr.q, qr.d, qr.s, qkv, rp);
      });
      if (e == hipSuccess) return KMOE_OK;
      if (e != hipErrorNotSupported) HIP_OK(c, e);
      rc = matvec_q8_impl(c, t, (const uint8_t *)w, rows, cols, qr.q, qr.d, qr.s, 1, qkv);
      if (rc) return rc;
      return kmoe_rope_kv_store(c, qkv, qkv + nq, qkv + nq + kvw, 1, n_head, n_kv, head_dim, rope_dim, pos0, pos_dev,
                                inv_freq, neox, n_ctx, q_out, k_cache, v_cache);
    }
    if (e != hipErrorNotSupported) HIP_OK(c, e);
  }
  rc = kmoe_norm_matmul(c, x, y, norm_w, eps, t, w, w_len, rows, cols, 1, h, qkv);
  if (rc) return rc;
  return kmoe_rope_kv_store(c, qkv, qkv + nq, qkv + nq + kvw, 1, n_head, n_kv, head_dim, rope_dim, pos0, pos_dev,
                            inv_freq, neox, n_ctx, q_out, k_cache, v_cache);
}

int kmoe_swiglu(kmoe_ctx *c, const float *gate, const float *up, int64_t n, float *out) {
  if (!c) return KMOE_E_INVALID;
  if (n < 0) return fail(c, KMOE_E_INVALID, "negative size");
  if (n == 0) return KMOE_OK;
  if (!gate || !up || !out) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  LAUNCH(c, "swiglu", launch_swiglu(c->stream, gate, up, n, out));
  return KMOE_OK;
}

int kmoe_add_rows(kmoe_ctx *c, float *x, const float *b, int64_t rows, int64_t cols) {
  if (!c) return KMOE_E_INVALID;
  if (rows < 0 || cols <= 0) return fail(c, KMOE_E_INVALID, "bad shape");
  if (rows == 0) return KMOE_OK;
  if (!x || !b) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  LAUNCH(c, "add_rows", launch_add_rows(c->stream, x, b, rows, cols));
  return KMOE_OK;
}

int kmoe_argmax(kmoe_ctx *c, const float *logits, int64_t n, uint32_t *out, int32_t *pos_dev, int32_t advance) {
  if (!c) return KMOE_E_INVALID;
  if (n <= 0) return fail(c, KMOE_E_INVALID, "argmax of an empty vector");
  if (!logits || !out) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  LAUNCH(c, "argmax", launch_argmax(c->stream, logits, n, out, pos_dev, advance));
  return KMOE_OK;
}

int kmoe_pos_advance(kmoe_ctx *c, int32_t *pos_dev, int32_t by) {
  if (!c) return KMOE_E_INVALID;
  if (!pos_dev) return fail(c, KMOE_E_INVALID, "null pointer");
  DeviceGuard g(c->device);
  LAUNCH(c, "pos_advance", launch_pos_advance(c->stream, pos_dev, by));
  return KMOE_OK;
}

// ------------------------------------------------------------- measurements for the planner

extern "C++" {
namespace {
// Seconds per call of f, from HIP events around `reps` calls on the stream.
template <class F>
int time_calls(kmoe_ctx *c, int reps, double *sec, F &&f) {
  hipEvent_t a = nullptr, b = nullptr;
  HIP_OK(c, hipEventCreate(&a));
  HIP_OK(c, hipEventCreate(&b));
  int rc = KMOE_OK;
  for (int i = 0; i < 2 && !rc; ++i) rc = f(i);  // warm-up
  if (!rc) {
    (void)hipEventRecord(a, c->stream);
    for (int i = 0; i < reps && !rc; ++i) rc = f(i);
    (void)hipEventRecord(b, c->stream);
    (void)hipEventSynchronize(b);
    float ms = 0.0f;
    (void)hipEventElapsedTime(&ms, a, b);
    *sec = ms * 1e-3 / reps;
  }
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  return rc;
}
}  // namespace
}  // extern "C++"

int kmoe_measure(kmoe_ctx *c, kmoe_gpu_measurements *m) {
  if (!c || !m) return KMOE_E_INVALID;
  DeviceGuard g(c->device);
  *m = kmoe_gpu_measurements{};
  size_t fr = 0, tot = 0;
  HIP_OK(c, hipMemGetInfo(&fr, &tot));
  m->vram_total = tot;
  m->vram_free = fr;
  // Four copies of a Mixtral-sized expert matrix (14336 x 4096), rotated so
  // repeats miss the 256 MB Infinity Cache; the same buffer serves the copy.
  constexpr int64_t kRows = 14336, kCols = 4096, kCopies = 4;
  const int types[3] = {KMOE_Q4_K, KMOE_Q6_K, KMOE_Q8_0};
  size_t mat = 0;  // room for the largest of the three matrices (Q8_0: 34 bytes per 32 weights)
  for (int t : types) mat = std::max(mat, (size_t)kRows * (size_t)bytes_for(t, kCols));
  const size_t buf = mat * kCopies;
  const size_t pb = std::min(buf, size_t(128) << 20);  // the PCIe copies land in the same buffer
  void *w = nullptr;
  int rc = dev_alloc(c, buf, &w, "measurement");
  if (rc) return rc;
  auto done = [&](int r) {
    (void)hipStreamSynchronize(c->stream);
    (void)hipFree(w);
    release(c, buf);
    return r;
  };
  if (hipMemsetAsync(w, 0x11, buf, c->stream) != hipSuccess) return done(fail(c, KMOE_E_HIP, "memset"));
  // device copy: half the buffer onto the other half
  double sec = 0.0;
  rc = time_calls(c, 10, &sec, [&](int) -> int {
    HIP_OK(c, hipMemcpyAsync((uint8_t *)w + buf / 2, w, buf / 2, hipMemcpyDeviceToDevice, c->stream));
    return KMOE_OK;
  });
  if (rc) return done(rc);
  m->hbm_copy_bps = (double)buf / sec;  // bytes read + bytes written
  // decode GEMV (one activation row) per type: weight bytes per second
  float *x = nullptr, *out = nullptr;
  rc = ensure_ws(c, 0);
  const int64_t pf = gemm_f32_part_floats(kRows, kCols, 1, 1, 1);
  size_t need = 0;
  carve_qrows(nullptr, 1, kCols, &need, pf);
  need += align_up((size_t)kCols * 4) + align_up((size_t)kRows * 4);
  if (!rc) rc = ensure_ws(c, need);
  if (rc) return done(rc);
  QRows qr = carve_qrows(c->ws, 1, kCols, &need, pf);
  x = (float *)(c->ws + need);
  out = (float *)(c->ws + need + align_up((size_t)kCols * 4));
  if (hipMemsetAsync(x, 0, (size_t)kCols * 4, c->stream) != hipSuccess) return done(fail(c, KMOE_E_HIP, "memset"));
  for (int i = 0; i < 3; ++i) {
    const int t = types[i];
    const size_t tb = (size_t)kRows * (size_t)bytes_for(t, kCols);  // <= mat: copy k ends by (k + 1) * mat
    const int saved = c->regime;
    c->regime = KMOE_REGIME_AVX2;  // one row: the integer path, as a decode step takes it
    rc = time_calls(c, 20, &sec, [&](int k) -> int {
      return matmul_core(c, t, (const uint8_t *)w + (size_t)(k % kCopies) * mat, kRows, kCols, x, 1, out, qr);
    });
    c->regime = saved;
    if (rc) return done(rc);
    m->gemv_bps[i] = (double)tb / sec;
  }
  // launch cost: a stream of minimal kernels, per launch
  rc = time_calls(c, 200, &sec, [&](int) -> int {
    HIP_OK(c, launch_pos_advance(c->stream, (int32_t *)out, 0));
    return KMOE_OK;
  });
  if (rc) return done(rc);
  m->launch_s = sec;
  // PCIe: a pinned host buffer of pb <= buf bytes each way
  void *host = nullptr;
  if (hipHostMalloc(&host, pb, hipHostMallocDefault) != hipSuccess)
    return done(fail(c, KMOE_E_HIP, "hipHostMalloc(%zu)", pb));
  rc = time_calls(c, 4, &sec, [&](int) -> int {
    HIP_OK(c, hipMemcpyAsync(w, host, pb, hipMemcpyHostToDevice, c->stream));
    return KMOE_OK;
  });
  if (!rc) {
    m->h2d_bps = (double)pb / sec;
    rc = time_calls(c, 4, &sec, [&](int) -> int {
      HIP_OK(c, hipMemcpyAsync(host, w, pb, hipMemcpyDeviceToHost, c->stream));
      return KMOE_OK;
    });
    if (!rc) m->d2h_bps = (double)pb / sec;
  }
  (void)hipStreamSynchronize(c->stream);
  (void)hipHostFree(host);
  return done(rc);
}

// ------------------------------------------------------------- profiling

int kmoe_profile_enable(kmoe_ctx *c, int on) {
  if (!c) return KMOE_E_INVALID;
  DeviceGuard g(c->device);
  prof_drain(c);
  c->prof_acc.clear();
  c->prof = on != 0;
  return KMOE_OK;
}

int kmoe_profile_read(kmoe_ctx *c, const char *kernel, double *total_ms, int64_t *launches) {
  if (!c || !kernel) return KMOE_E_INVALID;
  DeviceGuard g(c->device);
  prof_drain(c);
  auto it = c->prof_acc.find(kernel);
  if (total_ms) *total_ms = it == c->prof_acc.end() ? 0.0 : it->second.first;
  if (launches) *launches = it == c->prof_acc.end() ? 0 : it->second.second;
  return KMOE_OK;
}

}  // extern "C"
