/*
 * CPU oracle for the Qwen3-0.6B decode step (the ops around the GEMVs).
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP decode kernels; only the
 * tests, the smoke check and the benchmark's CPU-baseline leg load it.
 * f16 values travel as raw IEEE binary16 bits (uint16_t).
 */
#ifndef QWEN3_DECODE_ORACLE_H
#define QWEN3_DECODE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* model/qwen3_full.mlir:29-64 */
#define QW_LAYERS 28
#define QW_HIDDEN 1024
#define QW_Q_HEADS 16
#define QW_KV_HEADS 8
#define QW_HEAD_DIM 128
#define QW_Q_DIM (QW_Q_HEADS * QW_HEAD_DIM)
#define QW_KV_DIM (QW_KV_HEADS * QW_HEAD_DIM)
#define QW_FFN 3072
#define QW_VOCAB 151936
#define QW_EPS 9.99999997e-7f
#define QW_ROPE_BASE 1.0e6f
/* rsqrt(128) of qwen3_full.mlir:721-723, rounded to nearest f32 */
#define QW_ATTN_SCALE ((float)(1.0 / 11.313708498984761))

/* Host copies of the weights in the reference's parameter layout
 * (create_q8_irpa.py:149-224): Q8_0 stacked [28, BPL] bytes; f16 norms
 * stacked [28, n]; f16 embedding [151936, 1024]; f16 output weight
 * [151936, 1024] (output_T.weight, qwen3_full.mlir:76-79). */
typedef struct oracle_qwen3_weights {
  const uint16_t* token_embd;
  const uint16_t* attn_norm;
  const uint16_t* ffn_norm;
  const uint16_t* q_norm;
  const uint16_t* k_norm;
  const uint8_t* wq;
  const uint8_t* wk;
  const uint8_t* wv;
  const uint8_t* wo;
  const uint8_t* wgu;
  const uint8_t* wdn;
  const uint16_t* output_norm;
  const uint16_t* output_w;
} oracle_qwen3_weights;

/* Intermediates of one layer, for per-op comparisons. */
typedef struct oracle_layer_trace {
  uint16_t q_roped[QW_Q_DIM];
  uint16_t k_roped[QW_KV_DIM];
  uint16_t v[QW_KV_DIM];
  uint16_t attn[QW_Q_DIM];
  uint16_t res1[QW_HIDDEN];
  uint16_t act[QW_FFN];
} oracle_layer_trace;

void oracle_rmsnorm(const uint16_t* x, const uint16_t* w, int n, float eps, uint16_t* out);
void oracle_head_rmsnorm(const uint16_t* x, int n_heads, const uint16_t* w, float eps,
                         uint16_t* out);
void oracle_rope(const uint16_t* x, int n_heads, int32_t pos, uint16_t* out);
void oracle_attention(const uint16_t* q, const uint16_t* k_rows, const uint16_t* v_rows, int ctx,
                      float scale, uint16_t* out);
void oracle_swiglu(const uint16_t* gate, const uint16_t* up, int n, uint16_t* out);
void oracle_add_f16(const uint16_t* a, const uint16_t* b, int n, uint16_t* out);
void oracle_decode_layer(const oracle_qwen3_weights* w, int layer, uint16_t* k_cache,
                         uint16_t* v_cache, int64_t max_seq, int32_t pos, const uint16_t* h_in,
                         uint16_t* h_out, oracle_layer_trace* trace);
int64_t oracle_decode_step(const oracle_qwen3_weights* w, uint16_t* k_cache, uint16_t* v_cache,
                           int64_t max_seq, int32_t token, int32_t pos, uint16_t* logits,
                           uint16_t* h_layers);

#ifdef __cplusplus
}
#endif
#endif
