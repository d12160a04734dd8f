// kmoe_launch.h — host-side launchers of the gfx950 kernels (internal).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kmoe {

// Kernel timing hook (profiling): while start is set, the next kernel launched
// through KMOE_LAUNCH on this thread records start/stop at its own dispatch
// (hipExtLaunchKernelGGL: the begin/end timestamps of the dispatch packet, the
// ones a kernel trace reports) and clears the hook.
struct LaunchTiming {
  hipEvent_t start = nullptr, stop = nullptr;
};
extern thread_local LaunchTiming g_timing;

#define KMOE_LAUNCH(K, G, B, SH, ST, ...)                                                              \
  do {                                                                                               \
    if (::kmoe::g_timing.start) {                                                                    \
      const ::kmoe::LaunchTiming t_ = ::kmoe::g_timing;                                              \
      ::kmoe::g_timing = ::kmoe::LaunchTiming{};                                                     \
      hipExtLaunchKernelGGL(K, G, B, SH, ST, t_.start, t_.stop, 0, __VA_ARGS__);                     \
    } else {                                                                                         \
      hipLaunchKernelGGL(K, G, B, SH, ST, __VA_ARGS__);                                              \
    }                                                                                                \
  } while (0)

enum { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_Q4_K = 12, T_Q6_K = 14 };
// K-quants read Q8_K activations (256-blocks with 16-sums): Q4_K and Q6_K.
constexpr bool is_kquant(int t) { return t == T_Q4_K || t == T_Q6_K; }
enum { REGIME_AVX2 = 0, REGIME_INT8 = 1, REGIME_EXACT = 2 };

// ---- activation quantizers (kmoe_quant.hip)
hipError_t launch_quant_q8k(hipStream_t st, const float *x, int64_t rows, int64_t cols, int8_t *q, float *d,
                            int32_t *bsums);
hipError_t launch_quant_q8(hipStream_t st, const float *x, int64_t rows, int64_t cols, int8_t *q, float *d,
                           int32_t *s16);

// ---- routing on-device state produced by dispatch, read by the grouped kernels
struct Routing {
  const int32_t *n_active;  // [1] number of experts with rows
  const int32_t *active;    // [n_expert] their ids, ascending
  const uint32_t *offsets;  // [n_expert+1]
  const uint32_t *perm;     // [S*k] flat (token*k + slot), sorted by expert then token
  const uint32_t *inv;      // [S*k] position of flat index in perm
  const float *wsel;        // [S*k] routing weights, flat
  int32_t topk;
};

// Expert tier addressing: expert e's part p starts at base + e*stride + off[p].
struct ExpertTier {
  const uint8_t *base;
  int64_t stride;
  int64_t off[3];
};

// Per-block integer accumulators of the int-path expert products, written by
// the kernels of one captured moe_ffn: per (slot p in dispatch order, weight
// row r, block b) at [(p*rows + r)*nblk + b], nblk = cols / block elements,
// the integers of dot_q4_k_8k (sumi, mins), dot_q6_k_8k (sumi, offs) or
// dot_q8_0 (p; m unused). s[0]/m[0]: gate (or down), s[1]/m[1]: up. The
// caller zeroes them; kernels add their quarter-superblock parts with integer
// atomics (exact in any order). All null: no capture.
struct BlockDbg {
  int32_t *s[2] = {nullptr, nullptr};
  int32_t *m[2] = {nullptr, nullptr};
};
__device__ __forceinline__ void dbg_add(int32_t *base, int64_t o, int v) {
  if (base) atomicAdd(base + o, v);
}

// ---- expert tier layout (kmoe_layout.hip): GGUF Q4_K rows <-> tiled Q4_K rows
// (rows of nb superblocks; src and dst must not overlap).
hipError_t launch_tq4_convert(hipStream_t st, const uint8_t *src, uint8_t *dst, int64_t rows, int64_t nb,
                              bool to_tiled);
void tq4_convert_host(const uint8_t *src, uint8_t *dst, int64_t rows, int64_t nb, bool to_tiled);
// The same for Q6_K rows (210 bytes per superblock in both layouts).
hipError_t launch_tq6_convert(hipStream_t st, const uint8_t *src, uint8_t *dst, int64_t rows, int64_t nb,
                              bool to_tiled);
void tq6_convert_host(const uint8_t *src, uint8_t *dst, int64_t rows, int64_t nb, bool to_tiled);

// ---- int8 matvecs (kmoe_matvec.hip)
// Plain: out[s*rows + r] for s < s_rows; activations pre-quantized.
hipError_t launch_matvec_int(hipStream_t st, int type, const uint8_t *w, int64_t rows, int64_t cols, const int8_t *xq,
                             const float *xd, const int32_t *xbs, int64_t s_rows, float *out);
// Epilogue of a one-row matvec that adds into out instead of storing:
// out[r] = out[r] + scale * y[r], scale = 1 / (1 + exp(-*logit)) or 1 when
// logit is null (the shared expert's gated add, transformer.rs:584-586).
struct AddEpi {
  const float *logit = nullptr;
};
// Single activation row (decode, one token): activation slice held in registers.
// Return hipErrorNotSupported when the row is too wide for that; callers then
// use the LDS-staged kernels. epi: add into out (see AddEpi).
hipError_t launch_decode_plain(hipStream_t st, int type, const uint8_t *w, int64_t rows, int64_t cols,
                               const int8_t *xq, const float *xd, const int32_t *xbs, float *out,
                               const AddEpi *epi = nullptr);
// The same for one f32 activation row quantized to Q8_K inside the kernel
// (Q4_K and Q6_K rows of at most 4096 columns; the same bits as
// launch_quant_q8k followed by launch_decode_plain where the rows take the
// register kernel). hipErrorNotSupported otherwise.
hipError_t launch_decode_plain_fx(hipStream_t st, int type, const uint8_t *w, int64_t rows, int64_t cols,
                                  const float *xf, float *out);
struct DecSelect;
// sel: the kernel selects the token's experts from its logits and writes the
// routing (hipErrorNotSupported where decode_gate_up_can_select is false).
// The shared expert's gate rows (GGUF, `rows` of them, its up rows right
// after: one [2 rows, cols] matrix) computed with the routed experts' gate/up
// (one launch), SwiGLU into h [rows].
struct SharedGateUp {
  const uint8_t *w;
  int64_t rows;
  float *h;
};
// sgu (one token, Q4_K or Q8_0 rows on the register kernel, no dbg): the
// shared expert's gate/up as extra items; hipErrorNotSupported (nothing
// launched) where the experts take another kernel.
hipError_t launch_decode_gate_up(hipStream_t st, int type, const ExpertTier &tier, int64_t rows, int64_t cols,
                                 const Routing &rt, int max_active, const int8_t *xq, const float *xd,
                                 const int32_t *xbs, float *h, const DecSelect *sel = nullptr,
                                 const BlockDbg *dbg = nullptr, const SharedGateUp *sgu = nullptr);
// Two int8 quantizations in one launch: rows A (the routed slots' h, all on
// the int path, launch_quant_slots' arithmetic for one token) and row B (the
// shared expert's SwiGLU row), each as Q8_K (K-quant down types) or Q8.
hipError_t launch_quant_two(hipStream_t st, int type_a, const float *ha, int64_t n_a, int8_t *qa, float *da,
                            int32_t *sa, int type_b, const float *hb, int64_t n_b, int8_t *qb, float *db,
                            int32_t *sb);
// Whether launch_decode_gate_up can select the experts for this layer shape.
bool decode_gate_up_can_select(int type, int64_t cols, int32_t E, int32_t K);
// Expert selection done inside the decode gate/up kernel: the token's logits
// [E] and where to publish the routing (the arrays of Routing, writable).
struct DecSelect {
  const float *logits = nullptr;
  int32_t E = 0, K = 0, norm_topk = 0;
  float weights_scale = 0.0f;
  uint32_t *idx = nullptr;
  float *wsel = nullptr;
  uint32_t *perm = nullptr, *offsets = nullptr, *inv = nullptr;
  int32_t *n_active = nullptr, *active = nullptr;
};
// Tiled Q4_K gate/up + SwiGLU for one token (kmoe_decode.hip): 2 rows per
// wave step, about 2 work-groups per CU. With sel the kernel selects the
// experts itself (E <= 256, max_active == K) and writes the routing; without
// it the routing is read from rt. hipErrorNotSupported for rows narrower than
// 48 quarters or wider than 128.
bool dec_gate_up_tq4_supported(int64_t cols);
hipError_t launch_dec_gate_up_tq4(hipStream_t st, const ExpertTier &tier, int64_t rows, int64_t cols,
                                  const Routing &rt, int max_active, const int8_t *xq, const float *xd,
                                  const int32_t *xbs, float *h, const DecSelect *sel = nullptr,
                                  const BlockDbg *dbg = nullptr);
// Q4_K rows of one matrix (GGUF bytes) against one Q8_K row: out[r]
// (kmoe_decode.hip). hipErrorNotSupported for rows narrower than 48 or wider
// than 256 quarter-superblocks or misaligned pointers (activations 16 bytes,
// rows 4).
bool dec_rows_supported(int64_t cols);
// xf non-null: the f32 row instead of xq/xd/xbs, quantized to Q8_K inside the
// kernel (at most 16 superblocks, xf 16-byte aligned).
hipError_t launch_dec_rows(hipStream_t st, const uint8_t *w, int64_t rows, int64_t cols, const int8_t *xq,
                           const float *xd, const int32_t *xbs, float *out, const AddEpi *epi = nullptr,
                           const float *xf = nullptr);
// Down projection + combine for one token: out[r] = sum_e (asc) w_e * y_e[r].
hipError_t launch_decode_down_combine(hipStream_t st, int type, const ExpertTier &tier, int64_t rows, int64_t cols,
                                      const Routing &rt, const int8_t *hq, const float *hd, const int32_t *hbs,
                                      float *out, const BlockDbg *dbg = nullptr);
// The shared expert's down rows (GGUF, type Q4_K or Q6_K) against its int8 row
// (sh.xq/xd/xbs: Q8_K of SwiGLU(gate, up), as launch_swiglu_quant writes it);
// logit: its gate's logit (sigmoid scale), or null for an ungated one.
struct SharedDown {
  int type;
  const uint8_t *w;
  int64_t cols;
  const int8_t *xq;
  const float *xd;
  const int32_t *xbs;
  const float *logit;
};
// launch_decode_down_combine with the shared expert added in the same kernel:
// out[r] = (sum_e (asc) w_e * y_e[r]) + scale * shared[r], the arithmetic and
// order of the down + combine kernel followed by the shared add.
// hipErrorNotSupported (nothing launched) where the two rows do not share a
// launch shape; then the caller runs them separately.
hipError_t launch_decode_down_shared(hipStream_t st, int type, const ExpertTier &tier, int64_t rows, int64_t cols,
                                     const Routing &rt, const int8_t *hq, const float *hd, const int32_t *hbs,
                                     float *out, const SharedDown &sh);
// Block sums (debug path of the same device code).
hipError_t launch_block_sums(hipStream_t st, int type, const uint8_t *w, int64_t rows, int64_t cols,
                             const int8_t *xq, const int32_t *xbs, int64_t s_rows, int32_t *sumi, int32_t *mins);
// Grouped MoE, int path: gate+up+SwiGLU -> h [slots, F] f32 (mode 0) or down -> y [slots, d] f32 (mode 1).
// Experts handled: those whose row count the regime sends to the int path.
// min_rows: experts with fewer rows are left to another kernel.
hipError_t launch_moe_int(hipStream_t st, int mode, int type, const ExpertTier &tier, int64_t rows, int64_t cols,
                          const Routing &rt, int regime, int max_active, int64_t s_rows, const int8_t *xq,
                          const float *xd, const int32_t *xbs, float *out, int min_rows = 0,
                          const BlockDbg *dbg = nullptr);

// Experts with 1..max_rows (at most 3) rows on the int path, rows of at most
// 64 task slots (the one-token register kernel's geometry, each weight task
// dotted with all of the expert's rows): as launch_moe_int, for those experts.
// hipErrorNotSupported for wider rows or max_rows outside 1..3.
hipError_t launch_few_int(hipStream_t st, int mode, int type, const ExpertTier &tier, int64_t rows, int64_t cols,
                          const Routing &rt, int regime, int max_active, const int8_t *xq, const float *xd,
                          const int32_t *xbs, float *out, int max_rows, const BlockDbg *dbg = nullptr);

// ---- int8 matrix-core path (kmoe_mfma.hip), Q4_K weights x Q8_K rows
// Token rows at which the matrix-core kernels take over.
constexpr int kMfmaMinRows = 8;
bool moe_mfma_supported(int64_t rows, int64_t cols);
// Grouped over the expert tier, as launch_moe_int (mode 0 gate/up + SwiGLU, 1 down),
// for the experts with min_rows..max_rows rows (max_rows: the most any expert can hold);
// those with at most ring_rows (<= 32; 0: none) rows take the streaming kernel.
// hipErrorNotSupported: shape or activation alignment (16 B) not covered.
hipError_t launch_moe_mfma(hipStream_t st, int mode, const ExpertTier &tier, int64_t rows, int64_t cols,
                           const Routing &rt, int regime, int max_active, const int8_t *aq, const float *ad,
                           const int32_t *abs, float *out, int min_rows, int max_rows, int ring_rows,
                           const BlockDbg *dbg = nullptr);
// Plain GGUF rows: out[s*rows + r], or, with sumi/mins set, the per-block
// integer accumulators at [(s*rows + r)*nb + b] (ad unused).
hipError_t launch_plain_mfma(hipStream_t st, const uint8_t *w, int64_t rows, int64_t cols, const int8_t *aq,
                             const float *ad, const int32_t *abs, int64_t s_rows, float *out, int32_t *sumi,
                             int32_t *mins);

// ---- few rows per expert (kmoe_small.hip): tiled Q4_K experts on the int
// path with 1..small_rows_for() rows (0: the batch is too large for these
// kernels). mode 0: gate/up + SwiGLU into h [slots, rows]; 1: down into y
// [slots, rows]. hipErrorNotSupported for row widths outside
// small_supported() or batches without a few-rows kernel.
bool small_supported(int64_t rows, int64_t cols, int mode);
int small_rows_for(int64_t cols, int mode, int64_t max_rows);
hipError_t launch_small(hipStream_t st, int mode, const ExpertTier &tier, int64_t rows, int64_t cols,
                        const Routing &rt, int regime, int max_active, int64_t max_rows, const int8_t *xq,
                        const float *xd, const int32_t *xbs, float *out, const BlockDbg *dbg = nullptr);

// ---- f32 path (kmoe_gemm_f32.hip): dequantized weights x f32 activations
// Partial-sum floats the launchers below use for this shape (0: no column
// split); groups = 1 (plain) or max_active, max_rows = most activation rows of
// one group, n_slots = all activation rows (plain) or slots (grouped). With a
// smaller buffer (or none) they run unsplit.
int64_t gemm_f32_part_floats(int64_t rows, int64_t cols, int64_t groups, int64_t max_rows, int64_t n_slots);
// Plain: out[s*rows + r].
hipError_t launch_matmul_f32(hipStream_t st, int type, const uint8_t *w, int64_t rows, int64_t cols, const float *x,
                             int64_t s_rows, float *out, float *part, int64_t part_floats);
// Grouped: mode 0 = gate (store g into h), 1 = up (h = silu(h) * u), 2 = down (store y).
hipError_t launch_moe_f32(hipStream_t st, int mode, int type, const ExpertTier &tier, int64_t rows, int64_t cols,
                          const Routing &rt, int regime, int max_active, int64_t max_rows_per_expert,
                          int64_t n_slots, const float *x, float *out, float *part, int64_t part_floats,
                          int min_rows = 0);
// The f32 regime for experts with min_rows..max_rows rows over tiled Q4_K
// rows (kmoe_f32rows.hip): mode 0 gate/up + SwiGLU into out [slots, rows],
// mode 1 down into out [slots, rows]. n_slots (S*k) bounds how many experts
// can hold a given number of rows. hipErrorNotSupported for other weight types.
bool f32_rows_supported(int type, int64_t rows, int64_t cols);
// The same kernel over plain GGUF Q4_K rows w [rows, cols] (16-byte aligned)
// and x [s_rows, cols] (16-byte aligned): out [s_rows, rows], the f32 regime of
// quant::matmul. With w_up (the same shape), w is the gate and out receives
// SwiGLU(w . x, w_up . x). hipErrorNotSupported for other types or alignments.
hipError_t launch_f32_rows_plain(hipStream_t st, int type, const uint8_t *w, int64_t rows, int64_t cols,
                                 const float *x, int64_t s_rows, float *out, const uint8_t *w_up = nullptr);
hipError_t launch_f32_rows(hipStream_t st, int mode, int type, const ExpertTier &tier, int64_t rows, int64_t cols,
                           const Routing &rt, int regime, int max_active, int64_t n_slots, int min_rows,
                           int max_rows, const float *x, float *out);

// ---- routing (kmoe_route.hip)
// logits [S, E] = router [E, d] . x [S, d] in the reference's summation order
// for s_rows (quant::matmul), or always in quant::dot order when qdot is set.
// qkind 1 / 2: the same launch also writes x's Q8_K / Q8 rows (xq, xd, xs as
// launch_quant_q8k / launch_quant_q8 write them).
hipError_t launch_router_logits(hipStream_t st, const float *router, int32_t n_expert, int64_t d, const float *x,
                                int64_t s_rows, float *logits, bool qdot = false, int qkind = 0,
                                int8_t *xq = nullptr, float *xd = nullptr, int32_t *xs = nullptr);
hipError_t launch_route_topk(hipStream_t st, const float *logits, int64_t s_rows, int32_t n_expert, int32_t k,
                             int32_t norm_topk, float weights_scale, uint32_t *idx, float *w);
// Decode routing (s_rows < 4): quant::dot-order logits (one work-group per
// expert), then in the last work-group to finish softmax, top-k, dispatch
// (perm/offsets/inv/active); int8 quantization of x when qtype is T_Q4_K
// (Q8_K rows) or T_Q8_0 (Q8 rows). logits [S, E] is required; *done must be 0
// and is 0 again when the kernel ends (calls on one counter must not overlap).
// With done null only the logits and the int8 rows are produced (the caller's
// next kernel selects the experts). hipErrorNotSupported when out of range.
// The one-token q/k/v projection with RoPE (interleaved pairs, or neox pairs
// when rope_dim == head_dim) and the KV store in its epilogue
// (kmoe_matvec.hip): rows [0, nh*hd) are q, then k, then v; out also receives
// the raw projection. hipErrorNotSupported for partial neox rotation or row
// geometries that do not keep a pair in one wave.
struct QkvRope {
  int32_t nh, nkv, hd, rd, neox;
  int64_t pos0;
  const int32_t *pos_dev;
  const float *inv_freq;
  int64_t n_ctx;
  float *q_out;
  uint16_t *kc, *vc;
};
hipError_t launch_matvec_qkv_rope(hipStream_t st, int type, const uint8_t *w, int64_t rows, int64_t cols,
                                  const int8_t *xq, const float *xd, const int32_t *xbs, float *out,
                                  const QkvRope &rope);
// The same with the residual add and RMSNorm in front (one token, K-quant
// rows of at most 4096 columns, 16-byte aligned rows): xo = x + y (y may be
// null; xo another buffer, x is not written), h = rmsnorm(xo) * w with
// k_rmsnorm_regs' bits, quantized to Q8_K inside the projection kernel;
// hipErrorNotSupported outside that.
struct QkvNorm {
  const float *x;
  const float *y, *w;
  float eps;
  float *h;
  float *xo;
};
hipError_t launch_matvec_qkv_rope_norm(hipStream_t st, int type, const uint8_t *w, int64_t rows, int64_t cols,
                                       const QkvNorm &nm, float *out, const QkvRope &rope);
// The FFN norm folded into the single-token router (RouteNorm): x += y (y
// may be null), f = rmsnorm(x) * w with k_rmsnorm_regs' arithmetic, and the
// router reads f. Needs S == 1, d % 256 == 0, 16-byte aligned rows.
struct RouteNorm {
  float *x;
  const float *y;
  const float *w;
  float eps;
  float *f;
  uint32_t *done;  // work-groups that have read x; 0 between calls (the last one stores x + y and resets it)
};
bool route_norm_supported(const RouteNorm *n, int32_t S, int64_t d);
hipError_t launch_route_decode(hipStream_t st, const float *router, int32_t E, int64_t d, const float *x, int32_t S,
                               int32_t k, int32_t norm_topk, float weights_scale, float *logits, uint32_t *idx,
                               float *w, uint32_t *perm, uint32_t *offsets, uint32_t *inv, int32_t *n_active,
                               int32_t *active, int qtype, int8_t *xq, float *xd, int32_t *xs, uint32_t *done,
                               const RouteNorm *norm = nullptr);
// Stable counting sort by expert. inv/n_active/active may be null.
hipError_t launch_dispatch(hipStream_t st, const uint32_t *idx, int64_t n_slots, int32_t n_expert, uint32_t *perm,
                           uint32_t *offsets, uint32_t *inv, int32_t *n_active, int32_t *active, uint32_t *rank_tmp);
// Q8_K / Q8 quantization of the slot rows of h that go to the int path.
hipError_t launch_quant_slots(hipStream_t st, int type, const float *h, int64_t n_slots, int64_t cols,
                              const Routing &rt, const uint32_t *idx_flat, int regime, int8_t *q, float *d,
                              int32_t *sums);
// ---- the other weight types of quant::matmul (kmoe_xtypes.hip): F16, BF16,
// Q4_0, Q4_1, Q5_0, Q5_1, Q5_K (ggml type ids).
bool xtype(int t);
// out [rows, cols] f32 = dequant_row of every row (quantized types: cols % 32 == 0).
hipError_t launch_dequant_x(hipStream_t st, int t, const uint8_t *w, int64_t rows, int64_t cols, int64_t row_bytes,
                            float *out);
// out [s_rows, rows] = the reference's int8 dot of each row with each Q8 row
// (the quantized types except F16/BF16; cols % 32 == 0).
hipError_t launch_mv_unpacked(hipStream_t st, int t, const uint8_t *w, int64_t rows, int64_t cols,
                              int64_t row_bytes, const int8_t *xq, const float *xd, const int32_t *s16, int64_t s_rows,
                              float *out);

// ---- shared expert (kmoe_shared.hip)
// g = g / (1 + exp(-g)) * u over n elements.
hipError_t launch_swiglu(hipStream_t st, float *g, const float *u, int64_t n);
// SwiGLU of one row whose gate and up values sit side by side (gu [2F]: g
// then u), quantized for the next product: Q8_K rows (K-quant type) or Q8 rows
// (Q8_0), written to q, d, s as the activation quantizers write them.
hipError_t launch_swiglu_quant(hipStream_t st, int type, const float *gu, int64_t F, int8_t *q, float *d, int32_t *s);
// out[s] += sigmoid(logits[s]) * y[s] (logits null: scale 1).
hipError_t launch_shared_add(hipStream_t st, float *out, const float *y, const float *logits, int64_t S, int64_t d);

// out[s] = sum over the token's experts in ascending id of w * y[slot].
hipError_t launch_combine(hipStream_t st, const float *y, const Routing &rt, int64_t s_rows, int64_t d, float *out);


// ---- the rest of the decoder layer (kmoe_decoder.hip) ----
// Rows ids[0..s_rows) of a GGUF table [n_rows, cols] of type t (F32, F16,
// Q8_0, Q4_K, Q6_K), dequantized to f32 out [s_rows, cols].
hipError_t launch_get_rows(hipStream_t st, int t, const uint8_t *table, int64_t row_bytes, int64_t n_rows,
                           int64_t cols, const uint32_t *ids, int64_t s_rows, float *out);
hipError_t launch_add_rmsnorm(hipStream_t st, float *x, const float *y, const float *w, int64_t rows, int64_t dim,
                              float eps, float *out);
// RMSNorm followed by the Q8_K (q8k) or Q8 quantization of its output, in one
// kernel; hipErrorNotSupported when the shape or alignment does not allow it.
hipError_t launch_rmsnorm_quant(hipStream_t st, float *x, const float *y, const float *w, int64_t rows, int64_t dim,
                                float eps, float *out, bool q8k, int8_t *q, float *qd, int32_t *qs);
hipError_t launch_rope(hipStream_t st, float *x, int64_t s_rows, int n_heads, int hd, int rd, int64_t pos0,
                       const int32_t *pos_dev, const float *inv_freq, int neox);
hipError_t launch_kv_store(hipStream_t st, const float *k, const float *v, int64_t s_rows, int64_t kvw,
                           int64_t pos0, const int32_t *pos_dev, int64_t n_ctx, uint16_t *kc, uint16_t *vc);
// Attention: chunks of 64 positions covering n_max positions, the
// cross-work-group partials' size (0 for one super-chunk), supported shapes.
// counters: s_rows * nh zero words (zero again when the kernel ends).
int attn_supers(int64_t n_max);
int64_t attn_part_floats(int64_t s_rows, int nh, int hd, int supers);
bool attn_supported(int hd, int group);
// qt 1 / 2 also writes the Q8_K / Q8 rows of out into xq, xd, xs (qt 1 needs
// more than one row and (nh / nkv) * hd % 256 == 0, else
// hipErrorNotSupported: one row runs a work-group per head); qt 0 writes none.
hipError_t launch_attention(hipStream_t st, const float *q, const uint16_t *kc, const uint16_t *vc, int64_t s_rows,
                            int nh, int nkv, int hd, int64_t pos0, const int32_t *pos_dev, int64_t n_ctx, int supers,
                            float *part, uint32_t *counters, float *out, int qt = 0, int8_t *xq = nullptr,
                            float *xd = nullptr, int32_t *xs = nullptr);
// RoPE of q (into q_out) and k, and the f16 store of k and v into the caches.
hipError_t launch_rope_kv(hipStream_t st, const float *q, const float *k, const float *v, int64_t s_rows, int nh,
                          int nkv, int hd, int rd, int64_t pos0, const int32_t *pos_dev, const float *inv_freq,
                          int neox, int64_t n_ctx, float *q_out, uint16_t *kc, uint16_t *vc);
hipError_t launch_swiglu(hipStream_t st, const float *g, const float *u, int64_t n, float *out);
hipError_t launch_add_rows(hipStream_t st, float *x, const float *b, int64_t rows, int64_t cols);
// argmax of l[0..n) into out[0]; pos_dev (may be null) += advance afterwards.
hipError_t launch_argmax(hipStream_t st, const float *l, int64_t n, uint32_t *out, int32_t *pos_dev,
                         int32_t advance);
hipError_t launch_pos_advance(hipStream_t st, int32_t *pos_dev, int32_t by);

}  // namespace kmoe
