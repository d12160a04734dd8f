/*
 * kmoe.h — C ABI of the MI355X (gfx950) MoE FFN hot path.
 *
 * This is the seam a Rust FFI crate (kestrel-hip-sys) binds. It replaces,
 * behind kestrel's unchanged InferenceSession trait
 * (crates/kestrel-backends/src/lib.rs:60-74):
 *   - quant::matmul                (crates/kestrel-engine/src/quant.rs:229)
 *   - Q8Row / Q8KRow::quantize     (crates/kestrel-engine/src/qdot.rs:30, :347)
 *   - Transformer::route           (crates/kestrel-engine/src/transformer.rs:472)
 *   - the dispatch of moe_ffn      (transformer.rs:525-531)
 *   - Transformer::moe_ffn         (transformer.rs:513), without the shared expert
 *   - ExpertStore's resident tier  (crates/kestrel-memory/src/expert.rs:223-641),
 *     as an HBM-resident expert tier with Tier::Vram accounting
 *     (crates/kestrel-memory/src/ledger.rs:10-14, :75)
 *   - the rest of the decoder layer of Transformer::forward_chunk_inner
 *     (transformer.rs:330-467, :591-631): embedding rows, RMSNorm, RoPE, the
 *     f16 KV cache, causal GQA attention, dense SwiGLU; and greedy
 *     sampler::argmax (crates/kestrel-engine/src/sampler.rs:104-112)
 *
 * Conventions
 *   - Every entry point returns a kmoe_status (0 = ok). On error the context
 *     keeps a message, kmoe_last_error(). Sizes that the reference asserts on
 *     (quant.rs:231-234) return KMOE_E_INVALID instead of aborting.
 *   - Pointers named *_dev are device (HBM) pointers. Calls that take them are
 *     asynchronous on the context's stream; kmoe_synchronize() waits.
 *   - Weights are GGUF bytes verbatim (ggml order: a [rows, cols] matrix is
 *     row-major, cols contiguous; kestrel-gguf lib.rs:151, quant.rs:226-228).
 *   - A context is one device and one stream. It is not thread-safe: callers
 *     serialise, as Transformer::forward(&mut self) does. Several contexts may
 *     coexist.
 */
#ifndef KMOE_H
#define KMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KMOE_ABI_VERSION 1

/* Status codes; the mapping to EngineError (transformer.rs:15-27) is
 * INVALID/UNSUPPORTED -> Unsupported or Other, BUDGET -> Budget,
 * NOT_LOADED -> Store, HIP -> Other. */
typedef enum {
  KMOE_OK = 0,
  KMOE_E_INVALID = -1,     /* bad argument or size mismatch */
  KMOE_E_UNSUPPORTED = -2, /* ggml type or shape without a kernel */
  KMOE_E_BUDGET = -3,      /* Tier::Vram reservation past the limit */
  KMOE_E_HIP = -4,         /* HIP runtime error */
  KMOE_E_NOT_LOADED = -5   /* layer, router or expert not uploaded */
} kmoe_status;

/* ggml type ids, kestrel-gguf types.rs:67-107. kmoe_matmul takes every type
 * quant::matmul does (quant.rs:48-51): F32, F16, BF16, Q4_0, Q4_1, Q5_0, Q5_1,
 * Q8_0, Q4_K, Q5_K, Q6_K. The expert tier, kmoe_matvec_q8 and the block-sum
 * entry points take Q8_0, Q4_K and Q6_K; get_rows F32, F16 and those. */
enum {
  KMOE_F32 = 0, KMOE_F16 = 1, KMOE_Q4_0 = 2, KMOE_Q4_1 = 3, KMOE_Q5_0 = 6, KMOE_Q5_1 = 7, KMOE_Q8_0 = 8,
  KMOE_Q4_K = 12, KMOE_Q5_K = 13, KMOE_Q6_K = 14, KMOE_BF16 = 30
};

/* Arithmetic regime of the quantized matmuls (quant.rs:229-328).
 * KMOE_REGIME_AVX2 (default): the reference on an AVX2+FMA host. A matmul
 *   (one expert) with s_rows >= 4 dequantizes weights to f32 and multiplies
 *   f32 activations (quant.rs:242-260); with s_rows < 4 it quantizes
 *   activations to int8 (Q8_K per 256 for Q4_K, quant.rs:262-281; Q8 per 32
 *   for Q8_0, quant.rs:282-310) and takes integer dots.
 * KMOE_REGIME_INT8: int8 activations for every row count: the per-row integer
 *   kernels of the reference applied to every row (batched/prefill regime).
 * KMOE_REGIME_EXACT: KESTREL_EXACT=1 (quant.rs:29-46): f32 for every row. */
enum { KMOE_REGIME_AVX2 = 0, KMOE_REGIME_INT8 = 1, KMOE_REGIME_EXACT = 2 };

typedef struct kmoe_ctx kmoe_ctx;

/* ------------------------------------------------------------------ context */
/* Replaces nothing one-to-one: NativeSession::load builds the engine
 * (backends/src/lib.rs:125-187); this creates the device side of it. */
int kmoe_create(int device, kmoe_ctx **out);
int kmoe_destroy(kmoe_ctx *ctx);
/* Message of the last failed call on ctx ("" if none). Valid until the next call. */
const char *kmoe_last_error(const kmoe_ctx *ctx);
int kmoe_abi_version(void);
/* Run on the caller's hipStream_t instead of the context's own stream. The
 * handle is used as given: NULL is HIP's default (null) stream, which is
 * where PyTorch's default stream lives. */
int kmoe_set_stream(kmoe_ctx *ctx, void *hip_stream);
/* Go back to the context's own (non-blocking) stream. */
int kmoe_use_own_stream(kmoe_ctx *ctx);
void *kmoe_get_stream(kmoe_ctx *ctx);
int kmoe_synchronize(kmoe_ctx *ctx);
int kmoe_set_regime(kmoe_ctx *ctx, int regime);
int kmoe_get_regime(const kmoe_ctx *ctx);
/* No counterpart in the reference (its host path has no device graphs). The
 * context's workspaces grow on demand, and growing one frees it and
 * allocates anew; *gen counts those (re)allocations. Work captured into a
 * HIP graph on this context holds workspace addresses: the graph may be
 * replayed only while the generation is the one read after its capture, and
 * must be captured again (after one uncaptured call at the new sizes) once
 * the generation has moved. */
int kmoe_workspace_generation(const kmoe_ctx *ctx, uint64_t *gen);

/* ------------------------------------------------- Tier::Vram accounting */
/* Ledger::reserve for Tier::Vram (ledger.rs:75): every device byte the context
 * owns (expert tier, routers, workspace, kmoe_device_alloc) is reserved
 * against `limit` first; past it, calls fail with KMOE_E_BUDGET.
 * limit 0 = the device's total memory. */
int kmoe_vram_set_limit(kmoe_ctx *ctx, uint64_t limit_bytes);
int kmoe_vram_usage(const kmoe_ctx *ctx, uint64_t *reserved, uint64_t *limit);

/* Device buffers for callers without their own allocator (counted in Tier::Vram). */
int kmoe_device_alloc(kmoe_ctx *ctx, size_t bytes, void **dev);
int kmoe_device_free(kmoe_ctx *ctx, void *dev);
int kmoe_copy_h2d(kmoe_ctx *ctx, void *dst_dev, const void *src, size_t bytes);  /* stream-ordered, synchronous */
int kmoe_copy_d2h(kmoe_ctx *ctx, void *dst, const void *src_dev, size_t bytes);  /* stream-ordered, synchronous */

/* -------------------------------------------------------------- kernel seam */
/* quant::matmul (quant.rs:229): out[s*rows + r] = W[r] . x[s] for W of
 * ggml_type with shape [rows, cols], x [s_rows, cols] f32, out [s_rows, rows] f32.
 * w_len must be >= rows * bytes_for(cols) (quant.rs:233-234). The regime of
 * the context picks the arithmetic as the reference does for s_rows. F16,
 * BF16, Q4_0, Q4_1, Q5_0, Q5_1 and Q5_K give the reference's bits in every
 * regime: the f32 path dequantizes the rows into the workspace (rows * cols
 * * 4 bytes) and sums in the reference's order; the int8 path replays the
 * AVX2 dot of qdot's unpacked rows. */
int kmoe_matmul(kmoe_ctx *ctx, int ggml_type, const void *w_dev, size_t w_len, int64_t rows, int64_t cols,
                const float *x_dev, int64_t s_rows, float *out_dev);

/* quant::matmul with its own signature (quant.rs:229): matmul(t, w: &[u8],
 * rows, cols, x: &[f32], out: &mut [f32]). x and out are host memory; w is
 * host memory (copied to the device for the call) or device memory (a
 * resident weight, e.g. from kmoe_device_alloc; used in place). Synchronous:
 * returns once out holds the result. Same arithmetic as kmoe_matmul. */
int kmoe_matmul_host(kmoe_ctx *ctx, int ggml_type, const void *w, size_t w_len, int64_t rows, int64_t cols,
                     const float *x, int64_t s_rows, float *out);

/* Q8KRow::quantize (qdot.rs:347-367) per row of x [s_rows, cols], cols % 256 == 0:
 * q [s_rows, cols] i8, d [s_rows, cols/256] f32, bsums [s_rows, cols/16] i32. */
int kmoe_quantize_q8k(kmoe_ctx *ctx, const float *x_dev, int64_t s_rows, int64_t cols, int8_t *q_dev, float *d_dev,
                      int32_t *bsums_dev);
/* Q8Row::quantize (qdot.rs:30-49) per row, cols % 32 == 0:
 * q [s_rows, cols] i8, d [s_rows, cols/32] f32, s16 [s_rows, cols/16] i32. */
int kmoe_quantize_q8(kmoe_ctx *ctx, const float *x_dev, int64_t s_rows, int64_t cols, int8_t *q_dev, float *d_dev,
                     int32_t *s16_dev);

/* Integer accumulators of the Q4_K x Q8_K dot (avx2.rs:361-374), per
 * (token s, row r, superblock b): sumi = sum_j sc_j * sum(q . x) and
 * mins = sum_j m_j * (bsum pair), both int32, written at [(s*rows + r)*nsb + b],
 * nsb = cols/256. Computed by the same device code as the matvec. */
int kmoe_q4k_block_sums(kmoe_ctx *ctx, const void *w_dev, int64_t rows, int64_t cols, const int8_t *q_dev,
                        const int32_t *bsums_dev, int64_t s_rows, int32_t *sumi_dev, int32_t *mins_dev);
/* Integer accumulators of the Q6_K x Q8_K dot (avx2.rs:398-414), per
 * (token s, row r, superblock b): sumi = sum_g sc_g * sum(q . x) over the 16
 * groups of 16 weights (q the unsigned 6-bit values) and offs = sum_g sc_g *
 * bsum_g, so the block's dot is d * xd * (sumi - 32 * offs). Layout as
 * kmoe_q4k_block_sums. Computed by the same device code as the matvec. */
int kmoe_q6k_block_sums(kmoe_ctx *ctx, const void *w_dev, int64_t rows, int64_t cols, const int8_t *q_dev,
                        const int32_t *bsums_dev, int64_t s_rows, int32_t *sumi_dev, int32_t *offs_dev);
/* Per-block int32 dot of Q8_0 x Q8 (avx2.rs:51-56), at [(s*rows + r)*nb + b], nb = cols/32. */
int kmoe_q8_0_block_sums(kmoe_ctx *ctx, const void *w_dev, int64_t rows, int64_t cols, const int8_t *q_dev,
                         int64_t s_rows, int32_t *p_dev);
/* Matvec on pre-quantized activations: the int8 path of kmoe_matmul with the
 * caller's Q8_K (Q4_K, Q6_K weights) or Q8 (Q8_0 weights, bsums unused) rows. */
int kmoe_matvec_q8(kmoe_ctx *ctx, int ggml_type, const void *w_dev, size_t w_len, int64_t rows, int64_t cols,
                   const int8_t *q_dev, const float *d_dev, const int32_t *bsums_dev, int64_t s_rows, float *out_dev);

/* ------------------------------------------------------ routing + dispatch */
/* Transformer::route (transformer.rs:472-496) on a router given by pointer:
 * logits = matmul(F32 router [n_expert, d], h [s_rows, d]) in the reference's
 * summation order for s_rows, softmax, top-k (descending p, ties to the lower
 * index), optional renormalisation (floor 2^-14) and weights_scale.
 * idx [s_rows, k] u32 and w [s_rows, k] f32 in selection order;
 * logits_dev (optional, may be NULL) receives [s_rows, n_expert]. */
int kmoe_route(kmoe_ctx *ctx, const float *router_dev, int32_t n_expert, int64_t d, const float *h_dev,
               int64_t s_rows, int32_t k, int32_t norm_topk, float weights_scale, uint32_t *idx_dev, float *w_dev,
               float *logits_dev);
/* The dispatch of moe_ffn (transformer.rs:525-531): a stable counting sort of
 * the s_rows*k (token, slot) pairs by expert id. perm [s_rows*k] holds flat
 * indices s*k + j; offsets [n_expert+1] is the exclusive scan of the counts. */
int kmoe_dispatch(kmoe_ctx *ctx, const uint32_t *idx_dev, int64_t s_rows, int32_t k, int32_t n_expert,
                  uint32_t *perm_dev, uint32_t *offsets_dev);

/* ------------------------------------------------------ HBM expert tier */
/* One MoE layer (MoeInfo, kestrel-model lib.rs:103-117, and the stacked
 * ffn_{gate,up,down}_exps geometry). */
typedef struct {
  uint32_t n_expert;
  uint32_t n_expert_used;
  int32_t norm_topk;   /* renormalise selected weights (default: all but qwen2moe) */
  float weights_scale; /* 0 or 1 = none */
  int64_t n_embd;      /* d */
  int64_t n_ff;        /* expert FFN width */
  int32_t gate_type, up_type, down_type;
} kmoe_moe_desc;

/* Reserve the layer's expert tier: n_expert * (gate + up + down) bytes, one
 * contiguous extent per expert (the prepared-container layout,
 * docs/prepared-format.md), plus the f32 router. Fails with KMOE_E_BUDGET past
 * the Tier::Vram limit. */
int kmoe_layer_create(kmoe_ctx *ctx, uint32_t layer, const kmoe_moe_desc *desc);
int kmoe_layer_destroy(kmoe_ctx *ctx, uint32_t layer);
/* Router tensor blk.L.ffn_gate_inp.weight, F32 [n_expert, n_embd], host bytes. */
int kmoe_router_upload(kmoe_ctx *ctx, uint32_t layer, const float *router, size_t bytes);
/* ExpertStore::load/preload_all (expert.rs:251-303, :620-641): copy expert e's
 * part (0 gate, 1 up, 2 down) GGUF bytes from host memory. Q8_0 and F32 parts
 * are stored verbatim; Q4_K and Q6_K parts are stored as tiled rows (same
 * size, regrouped so a wave's loads are contiguous), tiled on the device after
 * a copy into the context's upload staging (or on the host when the VRAM
 * budget leaves no room for it); kmoe_expert_read gives back the GGUF bytes. */
int kmoe_expert_upload(kmoe_ctx *ctx, uint32_t layer, uint32_t expert, int32_t part, const void *bytes, size_t len);
/* Same from device memory (device-to-device copy, tiled on the device). */
int kmoe_expert_upload_dev(kmoe_ctx *ctx, uint32_t layer, uint32_t expert, int32_t part, const void *bytes_dev,
                           size_t len);
/* ExpertBuf as ExpertStore::load fills it (expert.rs:62-76, :293-303): one
 * host buffer of len bytes holding expert e's file extents, part k (gate, up,
 * down) at byte part_pos[k]. The whole buffer goes to the device in one
 * host-to-device copy, then each part is placed into the tier on the device.
 * The upload staging (device memory counted in the VRAM ledger, kept until
 * kmoe_destroy) grows to the largest buffer seen; without room for it the
 * parts are uploaded one by one. Synchronous; all three parts are resident
 * on return. */
int kmoe_expert_upload_buf(kmoe_ctx *ctx, uint32_t layer, uint32_t expert, const void *buf, size_t len,
                           const uint64_t part_pos[3]);
/* ExpertStore::preload_all (expert.rs:620-641) over a mapped model image:
 * every expert of the layer, part k of expert e at part_base[k] + e *
 * part_stride[k] (TensorInfo::slice_offset, kestrel-gguf/src/lib.rs:187-189).
 * A plain GGUF passes each stacked ffn_{gate,up,down}_exps tensor's data and
 * its slice bytes; a prepared KGUF passes data offset + o_k and the shared
 * stride, so an expert's three parts lie together. Per expert the three
 * ranges are sorted and merged when less than 4096 bytes apart
 * (ExpertStore::extents_of and coalesce, expert.rs:263-267,
 * kestrel-model/src/lib.rs:323-336; the bytes between merged ranges are read
 * too, so they must be readable), and each merged range is one host-to-device
 * copy: 1 per expert for a KGUF, 3 for a plain GGUF. *copies (may be NULL)
 * receives the number of copies. Synchronous. */
int kmoe_layer_preload(kmoe_ctx *ctx, uint32_t layer, const void *const part_base[3], const uint64_t part_stride[3],
                       uint64_t *copies);
/* ExpertStore::is_ready (expert.rs:445): 1 when all three parts are resident, else 0. */
int kmoe_expert_is_ready(kmoe_ctx *ctx, uint32_t layer, uint32_t expert);
/* ExpertBuf::part (expert.rs:72-76): device pointer and length of a resident
 * part, in the tier's layout (kmoe_expert_part_layout): tiled rows for Q4_K
 * and Q6_K parts, GGUF bytes for the others. The entry points that take a raw
 * weight pointer (kmoe_matmul, kmoe_matvec_q8, the block sums, the decoder
 * ops) read GGUF rows and refuse a pointer to a tiled part with
 * KMOE_E_INVALID. */
int kmoe_expert_part(kmoe_ctx *ctx, uint32_t layer, uint32_t expert, int32_t part, const void **dev, size_t *len);
/* Layout of a tier part's bytes on the device. No counterpart in the
 * reference, whose ExpertBuf::part is always GGUF bytes: KMOE_LAYOUT_TILED
 * rows keep each row's size and bytes in another order (kmoe_expert_read
 * returns the GGUF bytes). */
enum { KMOE_LAYOUT_GGUF = 0, KMOE_LAYOUT_TILED = 1 };
int kmoe_expert_part_layout(kmoe_ctx *ctx, uint32_t layer, uint32_t expert, int32_t part, int32_t *layout);
/* ExpertBuf::part bytes as the reference hands them out (expert.rs:72-76):
 * copy a resident part to host memory in GGUF layout; len must equal the
 * part's length. Synchronous. */
int kmoe_expert_read(kmoe_ctx *ctx, uint32_t layer, uint32_t expert, int32_t part, void *host, size_t len);
/* Shared expert of a layer (qwen2moe, transformer.rs:572-587): dense
 * ffn_{gate,up}_shexp [n_ff, n_embd] and ffn_down_shexp [n_embd, n_ff] of the
 * given ggml types, stored as GGUF bytes. kmoe_moe_ffn then adds, after the
 * routed experts, scale_s * SwiGLU-FFN(h[s]) for every token s (three
 * quant::matmul over all s_rows rows, in the context's regime), where
 * scale_s = 1 / (1 + exp(-quant::dot(ffn_gate_inp_shexp, h[s]))) once
 * kmoe_shared_gate_upload has given that F32 [n_embd] vector, else 1. */
int kmoe_shared_expert_create(kmoe_ctx *ctx, uint32_t layer, int64_t n_ff, int32_t gate_type, int32_t up_type,
                              int32_t down_type);
/* Host GGUF bytes of part 0 (gate), 1 (up) or 2 (down); synchronous. */
int kmoe_shared_expert_upload(kmoe_ctx *ctx, uint32_t layer, int32_t part, const void *bytes, size_t len);
int kmoe_shared_gate_upload(kmoe_ctx *ctx, uint32_t layer, const float *gate_inp, size_t bytes);
/* ExpertStore::bytes_per_expert (expert.rs:269). */
int kmoe_bytes_per_expert(kmoe_ctx *ctx, uint32_t layer, uint64_t *bytes);

/* ------------------------------------------------------------ layer seam */
/* Transformer::moe_ffn (transformer.rs:513-570) for one layer: route, dispatch
 * (batch union: each routed expert's weights are read once for all its rows),
 * per-expert SwiGLU FFN in the context's regime, and the combine
 * out[s] = sum over the token's experts in ascending id of w * y.
 * h [s_rows, n_embd] f32 in, out [s_rows, n_embd] f32 out (device). */
int kmoe_moe_ffn(kmoe_ctx *ctx, uint32_t layer, const float *h_dev, int64_t s_rows, float *out_dev);
/* kmoe_moe_ffn without any allocation. No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, hosts that forbid hipMalloc). Same kernels,
 * routing, dispatch and output bits as kmoe_moe_ffn, but the workspace is a
 * fixed 16 MiB device array per GPU (allocated with the library's code
 * object, held until the process ends) instead of the context's grown one;
 * a call needing more (many tokens) fails with KMOE_E_INVALID and names the
 * size. It calls no hipMalloc / hipFree and creates no events (profiling is
 * suspended for the call). Every call on one GPU, from any context, shares
 * that array and leaves its contents behind: calls that overlap on one GPU
 * (other streams, other threads) race, and the caller must order them.
 * kmoe_moe_last_routing reads the routing from that array until the next
 * such call. */
int kmoe_moe_ffn_noalloc(kmoe_ctx *ctx, uint32_t layer, const float *h_dev, int64_t s_rows, float *out_dev);
/* Transformer::moe_ffn with its own signature (transformer.rs:513): h:
 * &[f32] in, the Vec<f32> out, both host memory [s_rows, n_embd] (the
 * caller's out buffer). Synchronous; same arithmetic as kmoe_moe_ffn. */
int kmoe_moe_ffn_host(kmoe_ctx *ctx, uint32_t layer, const float *h, int64_t s_rows, float *out);
/* The feed-forward half of a MoE decoder layer (transformer.rs:430-444):
 * x += y when y_dev is non-NULL (the attention output, :430), f =
 * rmsnorm(x, norm_w) (:442, as kmoe_rmsnorm) into f_dev [s_rows, n_embd],
 * then out = kmoe_moe_ffn(f) (:444). Bit-identical to kmoe_rmsnorm followed
 * by kmoe_moe_ffn; for one token with 16-byte aligned rows and n_embd % 256
 * == 0 the router kernel computes the norm itself (one launch fewer). */
int kmoe_norm_moe_ffn(kmoe_ctx *ctx, uint32_t layer, float *x_dev, const float *y_dev, const float *norm_w_dev,
                      float eps, int64_t s_rows, float *f_dev, float *out_dev);
/* Transformer::moe_ffn as kmoe_moe_ffn, observed from inside (the layer
 * seam's debug outputs). The reference computes these integers
 * inside dot_q4_k_8k / dot_q6_k_8k / dot_q8_0 (avx2.rs:49-58, :351-379,
 * :384-419) on the rows moe_ffn gathers (transformer.rs:544-560); this call
 * returns them from the kernels that produce the layer's output, so parity
 * of the integer part can be checked bit for bit. Device buffers:
 *   xq/xd/xs  int8 rows of h (token order) the gate/up products read: Q8_K
 *             (q [S, d], d [S, d/256], bsums [S, d/16]) for K-quant gate/up,
 *             Q8 (q [S, d], d [S, d/32], s16 [S, d/16]) for Q8_0;
 *   hq/hd/hs  int8 rows of the SwiGLU output per slot in dispatch order
 *             (position p of the permutation), typed by the down part;
 *   *_sumi, *_mins  per (slot p, weight row r, block b) at [(p*rows + r)*nblk
 *             + b]: gate and up rows = n_ff, nblk = n_embd / block; down rows
 *             = n_embd, nblk = n_ff / block. Q4_K: sumi and mins of
 *             avx2.rs:361-374; Q6_K: sumi and offs (the block's dot is
 *             d * xd * (sumi - 32 * offs)); Q8_0: p in *_sumi (*_mins unused,
 *             may be NULL).
 * Only products on the int path write integers; slots of experts on the f32
 * path read 0, and their hq rows are not written. xq.. and hq.. may be NULL.
 * Same routing, dispatch and output bits as kmoe_moe_ffn; slower (integer
 * atomics). No counterpart entry point in the reference. */
typedef struct {
  int8_t *xq;
  float *xd;
  int32_t *xs;
  int8_t *hq;
  float *hd;
  int32_t *hs;
  int32_t *gate_sumi, *gate_mins, *up_sumi, *up_mins, *down_sumi, *down_mins;
} kmoe_moe_dbg;
int kmoe_moe_ffn_dbg(kmoe_ctx *ctx, uint32_t layer, const float *h_dev, int64_t s_rows, float *out_dev,
                     const kmoe_moe_dbg *dbg);
/* Routing state of the last kmoe_moe_ffn on ctx (device copies; any may be NULL):
 * idx/w [s_rows*k], perm [s_rows*k], offsets [n_expert+1]. */
int kmoe_moe_last_routing(kmoe_ctx *ctx, uint32_t *idx_dev, float *w_dev, uint32_t *perm_dev,
                          uint32_t *offsets_dev);

/* ---- The rest of the decoder layer (Transformer::forward_chunk_inner,
 * transformer.rs:375-467) on device buffers, on the context's stream. ----
 *
 * Positions: row s of a call sits at position pos0 + s, plus *pos_dev when
 * pos_dev (a device int32) is non-NULL. A decode step that reads its
 * position from pos_dev can be captured once as a HIP graph and replayed;
 * kmoe_argmax / kmoe_pos_advance move the counter on the device. With a
 * host position, pos0 + s_rows > n_ctx fails with KMOE_E_INVALID ("context
 * full", EngineError::ContextFull, transformer.rs:278-282); with a device
 * position, rows past n_ctx are skipped by the kernels. A call that grows the
 * context's decoder workspace (kmoe_get_rows, and kmoe_attention at a larger
 * size) allocates: run one call of each size before capturing a graph. */

/* quant::get_row (quant.rs:342-345) for the token embedding lookup
 * (transformer.rs:381-389): out[s] = row ids[s] of the GGUF table
 * [n_rows, cols] of type F32, F16, Q8_0, Q4_K or Q6_K, dequantized in
 * dequant_row's expression order (bit-identical). ids are host token ids;
 * an id >= n_rows fails with KMOE_E_INVALID ("token id out of range").
 * Synchronous. */
int kmoe_get_rows(kmoe_ctx *ctx, int32_t type, const void *table_dev, size_t table_len, int64_t n_rows,
                  int64_t cols, const uint32_t *ids, int64_t s_rows, float *out_dev);
/* Same with the ids on the device (a graph-captured decode step); an id
 * >= n_rows gives a row of zeros. Asynchronous. */
int kmoe_get_rows_dev(kmoe_ctx *ctx, int32_t type, const void *table_dev, size_t table_len, int64_t n_rows,
                      int64_t cols, const uint32_t *ids_dev, int64_t s_rows, float *out_dev);
/* Transformer::rmsnorm (transformer.rs:330-340) over rows of dim: out = x *
 * (1 / sqrt(mean(x^2) + eps)) * w. When y_dev is non-NULL the residual add
 * of forward_chunk_inner (transformer.rs:427, :463) comes first: x += y is
 * stored in x and the norm is taken of the sum. out may be x. */
int kmoe_rmsnorm(kmoe_ctx *ctx, float *x_dev, const float *y_dev, const float *w_dev, int64_t rows, int64_t dim,
                 float eps, float *out_dev);
/* Transformer::rmsnorm then Transformer::mm of the normed rows (the
 * attention projections, transformer.rs:391-393, and the head, :462-466):
 * h = rmsnorm(x, norm_w) after x += y when y_dev is non-NULL (as
 * kmoe_rmsnorm), out = quant::matmul(W, h) as kmoe_matmul. Where the
 * context's regime takes the integer path, the norm kernel also writes the
 * int8 rows the matvec reads, one pass fewer; the results are bit-identical
 * to kmoe_rmsnorm followed by kmoe_matmul. h_dev [s_rows, cols] receives the
 * normed rows. */
int kmoe_norm_matmul(kmoe_ctx *ctx, float *x_dev, const float *y_dev, const float *norm_w_dev, float eps,
                     int ggml_type, const void *w_dev, size_t w_len, int64_t rows, int64_t cols, int64_t s_rows,
                     float *h_dev, float *out_dev);
/* Transformer::rope (transformer.rs:342-358), in place on x [s_rows,
 * n_heads, head_dim]: pairs (i, i + rope_dim/2) when neox (every
 * architecture but llama, transformer.rs:242), else (2i, 2i+1), rotated by
 * position * inv_freq[i] (inv_freq [rope_dim/2] f32 on the device, built as
 * at transformer.rs:216-226). */
int kmoe_rope(kmoe_ctx *ctx, float *x_dev, int64_t s_rows, int32_t n_heads, int32_t head_dim, int32_t rope_dim,
              int64_t pos0, const int32_t *pos_dev, const float *inv_freq_dev, int32_t neox);
/* KV cache store (transformer.rs:411-418): k, v [s_rows, kv_width] f32 to
 * f16 (round to nearest even, half::f16::from_f32) at rows position + s of
 * the caches [n_ctx, kv_width]. */
int kmoe_kv_store(kmoe_ctx *ctx, const float *k_dev, const float *v_dev, int64_t s_rows, int64_t kv_width,
                  int64_t pos0, const int32_t *pos_dev, int64_t n_ctx, uint16_t *k_cache_dev,
                  uint16_t *v_cache_dev);
/* Transformer::attention (transformer.rs:591-631): causal GQA for s_rows
 * queries q [s_rows, n_head, head_dim] (after RoPE) over the f16 caches
 * [n_ctx, n_kv * head_dim]; query s attends positions 0 ..= position(s),
 * head h reads kv head h / (n_head / n_kv). out [s_rows, n_head * head_dim].
 * Scores use quant::dot's summation order (bit-identical); the softmax is
 * taken over chunks of 64 positions and merged, within 1e-6 relative of the
 * reference's single pass. head_dim 64 or 128, at most 16 query heads per
 * kv head. */
int kmoe_attention(kmoe_ctx *ctx, const float *q_dev, const uint16_t *k_cache_dev, const uint16_t *v_cache_dev,
                   int64_t s_rows, int32_t n_head, int32_t n_kv, int32_t head_dim, int64_t pos0,
                   const int32_t *pos_dev, int64_t n_ctx, float *out_dev);
/* Transformer::attention then the output projection, self.mm(attn_output)
 * (transformer.rs:419-424): attn_dev receives the attention rows as
 * kmoe_attention writes them, out_dev [s_rows, rows] the projection as
 * kmoe_matmul computes it. Where the context's regime takes the integer
 * path, the attention kernel also writes the int8 rows the matvec reads, one
 * pass fewer; the results are bit-identical to kmoe_attention followed by
 * kmoe_matmul. */
int kmoe_attention_matmul(kmoe_ctx *ctx, const float *q_dev, const uint16_t *k_cache_dev,
                          const uint16_t *v_cache_dev, int64_t s_rows, int32_t n_head, int32_t n_kv, int32_t head_dim,
                          int64_t pos0, const int32_t *pos_dev, int64_t n_ctx, float *attn_dev, int ggml_type,
                          const void *w_dev, size_t w_len, int64_t rows, float *out_dev);
/* RoPE of q and k followed by the KV cache store (transformer.rs:406-418) in
 * one pass: q is rotated into q_out [s_rows, n_head * head_dim] (q_out must
 * not overlap q), k is rotated and stored with v as f16 at rows position + s
 * of the caches; k itself is left as it was. Same values as kmoe_rope on q
 * and k followed by kmoe_kv_store. rope_dim <= 256. */
int kmoe_rope_kv_store(kmoe_ctx *ctx, const float *q_dev, const float *k_dev, const float *v_dev, int64_t s_rows,
                       int32_t n_head, int32_t n_kv, int32_t head_dim, int32_t rope_dim, int64_t pos0,
                       const int32_t *pos_dev, const float *inv_freq_dev, int32_t neox, int64_t n_ctx,
                       float *q_out_dev, uint16_t *k_cache_dev, uint16_t *v_cache_dev);
/* Dense SwiGLU (transformer.rs:455): out = g / (1 + exp(-g)) * u, n elements. */
/* One decode step's attention input (transformer.rs:391-418): kmoe_norm_matmul
 * of x over the concatenated q/k/v rows (rows = (n_head + 2 n_kv) head_dim)
 * into qkv_dev [rows] (h_dev [cols] receives the normed row), followed by
 * kmoe_rope_kv_store of its q, k and v parts. Bit-identical to those two
 * calls; on the integer path with interleaved pairs (neox == 0), or neox
 * pairs over the whole head (rope_dim == head_dim), the projection kernel
 * applies RoPE and stores k and v itself. One token. x_out_dev NULL (or
 * x_dev): x += y in place. Otherwise x + y goes to x_out_dev [cols] and
 * x_dev is left as it was (a residual stream kept in two buffers); then, for
 * K-quant rows of at most 4096 columns on the integer path, the residual add,
 * the norm and its Q8_K row are formed inside the projection kernel itself:
 * one launch, the same bits. */
int kmoe_norm_matmul_rope_kv(kmoe_ctx *ctx, float *x_dev, const float *y_dev, const float *norm_w_dev, float eps,
                             int ggml_type, const void *w_dev, size_t w_len, int64_t cols, float *h_dev,
                             float *qkv_dev, int32_t n_head, int32_t n_kv, int32_t head_dim, int32_t rope_dim,
                             int64_t pos0, const int32_t *pos_dev, const float *inv_freq_dev, int32_t neox,
                             int64_t n_ctx, float *q_out_dev, uint16_t *k_cache_dev, uint16_t *v_cache_dev,
                             float *x_out_dev);
int kmoe_swiglu(kmoe_ctx *ctx, const float *gate_dev, const float *up_dev, int64_t n, float *out_dev);
/* Bias rows (transformer.rs:394-401): x[r] += b for rows of cols. */
int kmoe_add_rows(kmoe_ctx *ctx, float *x_dev, const float *b_dev, int64_t rows, int64_t cols);
/* sampler::argmax (sampler.rs:104-112, greedy sampling): out_dev[0] = the
 * first index of the largest of logits[0..n). When pos_dev is non-NULL,
 * *pos_dev += advance afterwards (the end of a graph-captured decode step). */
int kmoe_argmax(kmoe_ctx *ctx, const float *logits_dev, int64_t n, uint32_t *out_dev, int32_t *pos_dev,
                int32_t advance);
/* *pos_dev += by on the device (no counterpart: the position counter of
 * graph-captured steps). */
int kmoe_pos_advance(kmoe_ctx *ctx, int32_t *pos_dev, int32_t by);

/* ---- Measured figures for the planner's cost model ----
 * kestrel's planner prices a GPU tier with Bandwidths.vram / .pcie and a
 * fixed per-layer overhead (crates/kestrel-planner/src/cost.rs:26-83, :102,
 * :123), and takes the memory bandwidth from a table of known parts marked
 * as an estimate (crates/kestrel-hw/src/gpu.rs:28-34, :100-113), because it
 * has no compute API to measure with. kmoe_measure measures them on the
 * context's device, as kestrel-hw's bench.rs measures the host
 * (Measurements, bench.rs:13-25):
 *   hbm_copy_bps   device-to-device copy, bytes read + written per second
 *   gemv_bps[i]    decode GEMV (one row, the integer path) weight bytes per
 *                  second for Q4_K, Q6_K, Q8_0 over 14336 x 4096 matrices
 *                  rotated past the Infinity Cache: the GPU's counterpart of
 *                  Measurements.cpu_gemv_bytes_per_s
 *   h2d_bps/d2h_bps pinned host <-> device copies of 128 MiB
 *   launch_s       cost of one kernel in a stream of launches
 * It allocates about 250 MB of device memory (through the VRAM ledger) and
 * 128 MiB of pinned host memory for the duration of the call, and takes
 * about half a second. Synchronous. */
typedef struct {
  uint64_t vram_total, vram_free;
  double hbm_copy_bps;
  double gemv_bps[3]; /* KMOE_Q4_K, KMOE_Q6_K, KMOE_Q8_0 */
  double h2d_bps, d2h_bps;
  double launch_s;
} kmoe_gpu_measurements;
int kmoe_measure(kmoe_ctx *ctx, kmoe_gpu_measurements *out);

/* Per-kernel timing (0 = off): each kernel is launched with start/stop HIP
 * events taken from its own dispatch packet (hipExtLaunchKernelGGL), on the
 * context's stream. */
int kmoe_profile_enable(kmoe_ctx *ctx, int on);
/* Accumulated time and launch count of the kernel named `kernel` since enable. */
int kmoe_profile_read(kmoe_ctx *ctx, const char *kernel, double *total_ms, int64_t *launches);

#ifdef __cplusplus
}
#endif
#endif /* KMOE_H */
