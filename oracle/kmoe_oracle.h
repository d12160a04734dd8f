/*
 * kmoe_oracle.h — CPU oracle for the MoE FFN hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP path is
 * compared against, and the CPU baseline that bench.py times. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The
 * product library (kestrel_amd/libkmoe.so) never links or calls it.
 *
 * It restates the arithmetic of kestrel's native CPU executor (Rust, AVX2+FMA)
 * in C++ with the same AVX2 intrinsics in the same order, compiled with
 * -ffp-contract=off so that no multiply-add is fused unless the reference
 * fuses it. Every function cites the reference file:line it follows.
 *
 * Pinning status (what checks each function; see tests/test_oracle.py):
 *   - dequant_row Q8_0/Q4_0: known values from quant.rs:375-394; Q4_1, Q5_0,
 *     Q5_1, Q5_K: hand-built blocks whose values follow from the formats.
 *   - unpack of every qdot type == dequant within 1e-5 (qdot.rs:301-315), the
 *     unpacked dot against the float dot (qdot.rs:318-334).
 *   - bytes_for / block geometry: types.rs:300-307 (Q4_K 512 -> 288 B).
 *   - unpack == dequant (qdot.rs:301-315), fused == unpacked (avx2.rs:184-223),
 *     Q8_K kernels vs f64 dequantized math (avx2.rs:425-460),
 *     gemm vs naive (avx2.rs:312-330), matmul vs naive (quant.rs:397-411).
 *   - per-superblock integer accumulators (Q4_K, Q6_K): brute-force int64 loops.
 *   - Q6_K: dequant known values (hand-built blocks), dot_q6_k_8k vs f64
 *     dequantized math (avx2.rs:425-460), integers vs brute force.
 *   - route: brute-force O(E^2) selection + closed-form softmax order.
 *   - dispatch: std::stable_sort by expert id.
 *   - quantizers (ours; the reference only reads blocks): round-trip bounds.
 *   - glibc expf (via Rust f32::exp) in route and SwiGLU: parity unpinned by
 *     any reference test (the reference checks them only by tolerance).
 */
#ifndef KMOE_ORACLE_H
#define KMOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids, kestrel-gguf types.rs:67-107 */
enum {
  ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q4_1 = 3, ORC_Q5_0 = 6, ORC_Q5_1 = 7, ORC_Q8_0 = 8, ORC_Q4_K = 12,
  ORC_Q5_K = 13, ORC_Q6_K = 14, ORC_BF16 = 30
};

/* Arithmetic regimes of quant::matmul (quant.rs:229-328).
 *  ORC_REGIME_AVX2 : the reference on an AVX2+FMA host: s_rows>=4 -> f32 GEMM,
 *                    else int8 activations (Q8_K for K-quants, Q8 for Q8_0).
 *  ORC_REGIME_INT8 : the per-row int8 kernels applied to every row.
 *  ORC_REGIME_EXACT: KESTREL_EXACT=1 (quant.rs:29-46): f32 for every row.  */
enum { ORC_REGIME_AVX2 = 0, ORC_REGIME_INT8 = 1, ORC_REGIME_EXACT = 2 };

/* ---- block geometry (types.rs:132-191) ---- */
int64_t orc_block_size(int t);
int64_t orc_type_size(int t);
int64_t orc_bytes_for(int t, int64_t n); /* -1 if n is not a multiple of the block size */

/* ---- f16 (half 2.7.1 semantics: exact IEEE conversion) ---- */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f); /* round to nearest even */
void orc_f32_to_f16_n(const float *x, uint16_t *out, size_t n); /* half::f16::from_f32 per element */

/* ---- deterministic generators ---- */
/* splitmix64 -> uniform in (0,1) -> Box-Muller in double -> float */
void orc_fill_normal(uint64_t seed, float mean, float std, float *out, size_t n);
/* xorshift32 byte stream, as in the reference's tests and bench_gemv */
void orc_fill_xorshift_bytes(uint32_t seed, uint8_t *out, size_t n, uint8_t mask);

/* ---- quantizers (ours: kestrel reads blocks but never writes them) ---- */
void orc_quantize_q8_0(const float *x, size_t n, uint8_t *out);
void orc_quantize_q4_k(const float *x, size_t n, uint8_t *out);
void orc_quantize_q6_k(const float *x, size_t n, uint8_t *out);
void orc_quantize_rows(int t, const float *x, size_t rows, size_t cols, uint8_t *out, int threads);

/* ---- dequantization, quant.rs:63-205 ---- */
int orc_dequant_row(int t, const uint8_t *src, float *out, size_t n);

/* ---- activation quantizers, qdot.rs:30-49 and qdot.rs:347-367 ---- */
void orc_q8row_quantize(const float *x, size_t n, int8_t *q, float *d, int32_t *s16);
void orc_q8krow_quantize(const float *x, size_t n, int8_t *q, float *d, int32_t *bsums);

/* ---- unpacked representation, qdot.rs:75-184; scalar dot qdot.rs:187-200 ---- */
int orc_unpack(int t, const uint8_t *w, size_t n, int8_t *q, float *scale, float *min);
float orc_dot_unpacked_scalar(const int8_t *uq, const float *uscale, const float *umin, size_t n,
                              const int8_t *aq, const float *ad, const int32_t *as16);
float orc_dot_unpacked_avx2(const int8_t *uq, const float *uscale, const float *umin, size_t n,
                            const int8_t *aq, const float *ad, const int32_t *as16);

/* ---- fused AVX2 kernels, avx2.rs ---- */
float orc_dot_q8_0(const uint8_t *w, size_t n, const int8_t *aq, const float *ad);
float orc_dot_q4_0(const uint8_t *w, size_t n, const int8_t *aq, const float *ad);
float orc_dot_q4_k(const uint8_t *w, size_t n, const int8_t *aq, const float *ad, const int32_t *as16);
float orc_dot_q4_k_8k(const uint8_t *w, size_t n, const int8_t *aq, const float *ad, const int32_t *abs);

/* Per-superblock integer accumulators of dot_q4_k_8k (avx2.rs:361-374):
 * sumi[b] = sum of the 8 i32 lanes of `sumi`, mins[b] = `mins`. */
void orc_q4k_block_acc(const uint8_t *w, size_t n, const int8_t *aq, const int32_t *abs, int32_t *sumi, int32_t *mins);
/* The same integers by brute force in int64 (the pin for the above). */
void orc_q4k_block_acc_bruteforce(const uint8_t *w, size_t n, const int8_t *aq, const int32_t *abs, int64_t *sumi,
                                  int64_t *mins);
/* Q6_K x Q8_K, avx2.rs:384-419. */
float orc_dot_q6_k_8k(const uint8_t *w, size_t n, const int8_t *aq, const float *ad, const int32_t *abs);
/* Its per-superblock integers: sumi[b] = sum of the 8 i32 lanes of `sumi`,
 * offs[b] = `offs` (sum over 16-blocks of sc * bsum). */
void orc_q6k_block_acc(const uint8_t *w, size_t n, const int8_t *aq, const int32_t *abs, int32_t *sumi, int32_t *offs);
/* The same integers by brute force in int64 from the raw activations. */
void orc_q6k_block_acc_bruteforce(const uint8_t *w, size_t n, const int8_t *aq, int64_t *sumi, int64_t *offs);
/* Per-block integer dot of dot_q8_0 (avx2.rs:51-56): p[b] = sum of i8*i8 over the block. */
void orc_q8_0_block_acc(const uint8_t *w, size_t n, const int8_t *aq, int32_t *p);

/* ---- f32 kernels ---- */
float orc_quant_dot(const float *a, const float *b, size_t n);             /* quant.rs:208-224 */
float orc_dot_f32(const float *a, const float *b, size_t n);               /* avx2.rs:289-308 */
void orc_gemm_f32(const float *w, size_t rows, const float *x, size_t s_rows, size_t cols,
                  float *res);                                             /* avx2.rs:230-286 */

/* ---- quant::matmul, quant.rs:229-328 ---- */
/* out[s*rows + r] = W[r] . x[s]. threads: worker count (0 = all hardware threads). */
int orc_matmul(int t, const uint8_t *w, size_t w_len, size_t rows, size_t cols, const float *x, size_t s_rows,
               float *out, int regime, int threads);

/* ---- MoE layer, transformer.rs:472-570 ---- */
typedef struct {
  int32_t n_expert;
  int32_t n_expert_used;
  int32_t norm_topk;     /* MoeInfo.norm_topk, model/src/lib.rs:113-114 */
  float weights_scale;   /* MoeInfo.weights_scale, model/src/lib.rs:115-116 */
  int64_t n_embd;        /* d */
  int64_t n_ff;          /* expert FFN width */
  int32_t gate_type, up_type, down_type;
  const float *router;   /* [n_expert, n_embd] f32 */
  const uint8_t *const *gate; /* per expert: [n_ff, n_embd] GGUF bytes */
  const uint8_t *const *up;   /* per expert: [n_ff, n_embd] */
  const uint8_t *const *down; /* per expert: [n_embd, n_ff] */
} orc_moe_layer;

/* Transformer::route (transformer.rs:472-496). idx/w: [S, k] in selection order. */
int orc_route(const orc_moe_layer *L, const float *h, size_t s_rows, uint32_t *idx, float *w, int regime,
              int threads);
/* Softmax + top-k + renorm + scale on given logits (transformer.rs:479-495). */
void orc_route_from_logits(const float *logits, size_t s_rows, int n_expert, int k, int norm_topk,
                           float weights_scale, uint32_t *idx, float *w);
/* The dispatch of moe_ffn (transformer.rs:525-531): perm[j] = s*k + slot, sorted by
 * expert id then token; offsets[e]..offsets[e+1] is expert e's range. */
void orc_dispatch(const uint32_t *idx, size_t s_rows, int k, int n_expert, uint32_t *perm, uint32_t *offsets);
/* Transformer::moe_ffn without the shared expert (transformer.rs:513-570). */
int orc_moe_ffn(const orc_moe_layer *L, const float *h, size_t s_rows, float *out, int regime, int threads);

/* Shared expert of a layer (qwen2moe, transformer.rs:572-587): dense tensors
 * ffn_{gate,up}_shexp [n_ff, n_embd], ffn_down_shexp [n_embd, n_ff] (GGUF bytes)
 * and the optional F32 gate vector ffn_gate_inp_shexp [n_embd]. */
typedef struct {
  int64_t n_embd, n_ff;
  int32_t gate_type, up_type, down_type;
  const uint8_t *gate, *up, *down;
  const float *gate_inp; /* NULL: scale 1 */
} orc_shared_expert;
/* out[s] += g_s * SwiGLU-FFN(h[s]), g_s = 1/(1+exp(-quant::dot(gate_inp, h[s]))) or 1;
 * the three products are quant::matmul over all s_rows rows (Transformer::mm). */
int orc_shared_expert_add(const orc_shared_expert *S, const float *h, size_t s_rows, float *out, int regime,
                          int threads);

/* ---- the rest of the decoder layer, transformer.rs:216-226, 330-467, 591-631 ---- */
/* Transformer::rmsnorm (transformer.rs:330-340): per row of dim, the sum of
 * squares in order, r = 1/sqrt(ss/dim + eps), out = x * r * w. */
void orc_rmsnorm(const float *x, const float *w, size_t rows, size_t dim, float eps, float *out);
/* RoPE frequencies (transformer.rs:216-226): inv_freq[i] = base^(-(2i)/rope_dim),
 * divided by freqs[i] when freqs (rope_freqs.weight) is non-NULL. */
void orc_rope_inv_freq(float base, size_t rope_dim, const float *freqs, float *inv_freq);
/* Transformer::rope (transformer.rs:342-358), in place on x [s_rows, n_heads, head_dim]:
 * row s at position pos0 + s; pairs (i, i + rope_dim/2) when neox, else (2i, 2i+1). */
void orc_rope(float *x, size_t s_rows, size_t n_heads, size_t head_dim, size_t rope_dim, size_t pos0,
              const float *inv_freq, int neox);
/* Transformer::attention (transformer.rs:591-631): causal GQA for s_rows queries
 * q [s_rows, n_head, head_dim] at positions pos0.., over the f16 caches
 * [>= pos0 + s_rows, n_kv * head_dim]; out [s_rows, n_head * head_dim]. */
void orc_attention(const float *q, const uint16_t *k_cache, const uint16_t *v_cache, size_t s_rows, size_t n_head,
                   size_t n_kv, size_t head_dim, size_t pos0, float *out);
/* Dense SwiGLU (transformer.rs:455): out = g / (1 + exp(-g)) * u. */
void orc_swiglu(const float *g, const float *u, size_t n, float *out);
/* sampler::argmax (sampler.rs:104-112): the first index of the largest value. */
uint32_t orc_argmax(const float *l, size_t n);

/* ---- bench_gemv, quant.rs:348-368: weight bytes per second ---- */
double orc_bench_gemv(int t, size_t rows, size_t cols, size_t iters, int threads);

int orc_hw_threads(void);

#ifdef __cplusplus
}
#endif
#endif
