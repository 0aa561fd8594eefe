/*
 * qnn_oracle.h -- CPU restatement of QuickNN's quantized-decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP backend
 * (libqnn_hip.so) is compared against.  Only tests/, __graft_entry__.smoke()
 * and the cpu_baseline leg of bench.py may load it.  Nothing in the product
 * package links or calls it.
 *
 * Every function names the reference file:line it restates (paths relative to
 * the QuickNN source tree).  Pinning of each function (known answers,
 * invariants, brute force) lives in tests/test_oracle_*.py.
 *
 * Encodings follow TQNNWeightEncoding (src/core/QuickNN.Common.pas:130-131):
 *   0 native, 1 Q8_0, 2 Q4_K, 3 Q6_K, 4 Q3_K, 5 Q5_K, 6 IQ4_NL, 7 IQ3_S, 8 IQ4_XS,
 *   9 Q2_K, 10 IQ2_XXS, 11 IQ2_S, 12 Q2_0, 13 IQ3_XXS.
 * The oracle uses QO_ENC_INT4 (-1) for QuickNN's native packed INT4 rows.
 */
#ifndef QNN_ORACLE_H
#define QNN_ORACLE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

#define QO_ENC_INT4 (-1)
#define QO_ENC_Q8_0 1
#define QO_ENC_Q4_K 2
#define QO_ENC_Q6_K 3
#define QO_ENC_Q3_K 4
#define QO_ENC_Q5_K 5
#define QO_ENC_IQ4_NL 6
#define QO_ENC_IQ4_XS 8
#define QO_ENC_Q2_K 9
#define QO_ENC_Q2_0 12
#define QO_ENC_IQ3_S 7
#define QO_ENC_IQ2_XXS 10
#define QO_ENC_IQ2_S 11
#define QO_ENC_IQ3_XXS 13

/* Status codes: 0 ok, -1 argument error (EArgumentException). */

/* ---- INT4 (src/core/QuickNN.Quantization.Int4.pas) ---- */
int qo_int4_row_bytes(int cols);                                      /* :25-33 */
int qo_quantize_int4(const void *src, int is_bf16, int rows, int cols, uint8_t *dst); /* :35-144 */
float qo_int4_value(const uint8_t *row, int k);          /* CPU.Inference.pas:413-420 */
void qo_int4_dequant_row(const uint8_t *row, int cols, float *out);

/* ---- GGUF formats (src/io/QuickNN.GGUF.Quantization.pas) ---- */
int qo_gguf_block_elements(int enc);                                  /* :67-75 */
int qo_gguf_block_bytes(int enc);                                     /* :77-93 */
float qo_gguf_value(const uint8_t *data, int enc, int64_t index);     /* :136-253 */
int qo_gguf_decode_block(const uint8_t *block, int enc, float *out);  /* :274-368 */
int qo_gguf_dequantize(const uint8_t *data, int enc, int64_t count, float *out); /* :370-383 */
int qo_gguf_read4(const uint8_t *data, int enc, int64_t index, float *out4);
/* The IQ2/IQ3 tables as little-endian bytes: 0 IQ2_XXS_GRID, 1 IQ2_S_GRID,
   2 IQ3_XXS_GRID, 3 IQ3_S_GRID, 4 IQ2_SIGNS (Tables.inc:20-309); returns the
   byte count (out may be NULL), -1 for another index. */
int qo_iq_table(int which, uint8_t *out);
                                /* shaders/gguf.glsl:591-655 (readGGUF4) */

/* ---- AVX2 dots (CPU.Inference.AVX2.inc, GGUF.Dot.AVX2.inc) ---- */
float qo_vector_dot(int n, const float *a, const float *b);           /* AVX2.inc:7-67 */
float qo_int4_vector_dot(int n, const float *x, const uint8_t *w);    /* AVX2.inc:210-285 */
float qo_packed_dot(const uint8_t *data, int enc, const float *x, int count);
            /* GGUFTryDot (GGUF.Quantization.pas:255-272) -> PackedDot* (Dot.AVX2.inc) */

/* ---- CPU projection (src/backends/cpu/QuickNN.CPU.Inference.pas) ---- */
void *qo_pool_create(int threads);                                    /* :109-116 */
void qo_pool_destroy(void *pool);
int qo_pool_threads(void *pool);
int qo_cpu_linear(void *pool, const uint8_t *w, int enc, const float *x, float *y,
                  int in_dim, int out_dim);                            /* :316-428 */

/* ---- Decode-layer composites (src/models/QuickNN.Models.QwenHybrid.CPU.pas) ---- */
int qo_rmsnorm(const float *x, const float *gamma, int rows, int dim, float eps,
               int add_one, float *out);                              /* :110-120 */
float qo_silu(float g);                      /* :78-82 + :242-246 (clamps +-20) */
int qo_cpu_mlp(void *pool, const uint8_t *gate, const uint8_t *up, const uint8_t *down,
               int enc, const float *x, int rows, int hidden, int inter, float *out);
                                                                       /* :238-248 */

/* ---- MoE (src/backends/vulkan/shaders/moe.comp:25-50, LLM.MoE.pas:230-449) ---- */
int qo_moe_route(const float *logits, int rows, int experts, int k, int normalize,
                 int select_on_logits, uint32_t *ids, float *probs);
int qo_cpu_moe(void *pool, const uint8_t *const *gate, const uint8_t *const *up,
               const uint8_t *const *down, const float *x, const uint32_t *ids,
               const float *probs, int rows, int topk, int hidden, int inter, float *out);

/* ---- Multi-row GGUF (src/core/QuickNN.Quantization.pas:247-258) ---- */
int qo_gguf_gemm_scalar(const uint8_t *w, int enc, const float *a, int m, int k, int n,
                        float *c, int row_begin, int row_end);

/* ---- int8-activation prefill GEMM (the benchmark's configs[4] path; no reference counterpart) ---- */
int qo_q8_act_quant(const float *a, int m, int k, int8_t *q, float *d);          /* GGML Q8_0 rule, fp32 d */
int qo_q8_gemm_i8(const uint8_t *w, const int8_t *q, const float *d, int m, int k, int n, float *c);

/* ---- the rest of a decode layer ---- */
/* RoPE as the reference's CPU statement (src/models/QuickNN.Models.QwenHybrid.CPU.pas:51-67, RotaryDim = dim):
 * pairs (j, j + dim/2) of each of rows*heads head rows rotated by (position + row) * theta^(-2j/dim),
 * angle, sine, cosine and rotation in double, rounded once.  In place. */
int qo_rope(float *x, int rows, int heads, int dim, int position, float theta);
/* KV-cache append (tensor.comp:313-317; CPU statement QwenHybrid.CPU.pas:198-204):
 * K transposed [kv_heads][dim][cap], then V [kv_heads][cap][dim]. */
int qo_cache_write(float *cache, const float *k, const float *v, int rows, int kv_heads, int dim, int cap,
                   int position);
/* CachedAttention (attention.comp, mask modes 2 and 4) in double: out fp32 [rows][heads][dim]. */
int qo_cached_attention(const float *q, const float *cache, int rows, int cap, int heads, int kv_heads, int dim,
                        int position, int window, float softcap, float scale, int masked, float *out);
/* SampleToken's top-k (tensor.comp:123-176): k best (score after penalty, id) ranked by score then id;
 * tokens with seen == 0xffffffff excluded; unfilled ranks are (-FLT_MAX, 0xffffffff). */
int qo_sample_topk(const float *logits, const uint32_t *seen, int vocab, int k, float penalty, float *scores,
                   uint32_t *ids);
/* SampleToken (Context.Implementation.inc:1137-1187, tensor.comp:177-197): the selected token id. */
uint32_t qo_sample_token(const float *logits, const uint32_t *seen, int vocab, int top_k, float temperature,
                         float top_p, float penalty, float uniform);

/* ---- numerics helpers ---- */
float qo_half_to_float(uint16_t h);            /* src/core/QuickNN.Common.pas:1799+ */
uint16_t qo_float_to_half(float f);            /* round-to-nearest-even (test helper) */

#ifdef __cplusplus
}
#endif
#endif
