/*
 * CPU oracle for the Qwen3-0.6B decode step around the GEMVs.  TEST
 * INFRASTRUCTURE ONLY (the checker; see q8_oracle.c).
 *
 * Restates model/qwen3_full.mlir's decode path op by op, with the reference's
 * f16 / f32 mix: f16 tensors between ops, f32 inside reductions and
 * transcendental math, every f32 -> f16 step rounding to nearest even.
 */
#include "decode_oracle.h"
#include "q8_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define H2F oracle_f16_to_f32
#define F2H oracle_f32_to_f16

/* qwen3_full.mlir:134-165 (@rms_norm_1x1024), also the per-head QK norm of
 * :648-702 with n = 128: ss = sequential f32 sum of squares; r =
 * sqrt(ss / n + eps); out = f16((x / r) * w). */
void oracle_rmsnorm(const uint16_t* x, const uint16_t* w, int n, float eps, uint16_t* out) {
  float ss = 0.0f;
  for (int i = 0; i < n; ++i) {
    float v = H2F(x[i]);
    ss = ss + v * v;
  }
  float r = sqrtf(ss / (float)n + eps);
  for (int i = 0; i < n; ++i) out[i] = F2H((H2F(x[i]) / r) * H2F(w[i]));
}

void oracle_head_rmsnorm(const uint16_t* x, int n_heads, const uint16_t* w, float eps,
                         uint16_t* out) {
  for (int h = 0; h < n_heads; ++h)
    oracle_rmsnorm(x + h * QW_HEAD_DIM, w, QW_HEAD_DIM, eps, out + h * QW_HEAD_DIM);
}

/* qwen3_full.mlir:324-388 / 390-454 (rope_decode_q / _k), rotate-half:
 * theta_i = f32(pos) * powf(1e6, -(2i / 128)), i = d mod 64;
 * d < 64: x[d] cos - x[d+64] sin;  d >= 64: x[d-64] sin + x[d] cos. */
void oracle_rope(const uint16_t* x, int n_heads, int32_t pos, uint16_t* out) {
  const float posf = (float)pos;
  for (int h = 0; h < n_heads; ++h) {
    const uint16_t* xh = x + h * QW_HEAD_DIM;
    uint16_t* oh = out + h * QW_HEAD_DIM;
    for (int d = 0; d < QW_HEAD_DIM; ++d) {
      const int i = d < 64 ? d : d - 64;
      const float e = -((2.0f * (float)i) / 128.0f);
      const float inv = powf(QW_ROPE_BASE, e) * 1.0f;
      const float th = posf * inv;
      const float c = cosf(th), s = sinf(th);
      float r;
      if (d < 64) {
        float a = H2F(xh[d]) * c;
        float b = H2F(xh[d + 64]) * s;
        r = a - b;
      } else {
        float a = H2F(xh[d - 64]) * s;
        float b = H2F(xh[d]) * c;
        r = a + b;
      }
      oh[d] = F2H(r);
    }
  }
}

/* qwen3_full.mlir:456-530: softmax(scale * q k^T) v over positions 0..ctx-1
 * for 16 query heads, query head h reading kv head h / 2 (the 8 -> 16 copy
 * expansion at :483-496).  k_rows / v_rows: [ctx, 8, 128] f16.  Computed in
 * f32: s_j = (sum_d q_d k_jd) * scale, m = max s, p_j = exp(s_j - m),
 * out = (sum_j p_j v_j) / (sum_j p_j), rounded to f16. */
void oracle_attention(const uint16_t* q, const uint16_t* k_rows, const uint16_t* v_rows, int ctx,
                      float scale, uint16_t* out) {
  float* s = (float*)malloc(sizeof(float) * (size_t)(ctx > 0 ? ctx : 1));
  for (int h = 0; h < QW_Q_HEADS; ++h) {
    const int g = h / (QW_Q_HEADS / QW_KV_HEADS);
    const uint16_t* qh = q + h * QW_HEAD_DIM;
    float m = -INFINITY;
    for (int j = 0; j < ctx; ++j) {
      const uint16_t* kj = k_rows + ((size_t)j * QW_KV_HEADS + g) * QW_HEAD_DIM;
      float dot = 0.0f;
      for (int d = 0; d < QW_HEAD_DIM; ++d) dot = dot + H2F(qh[d]) * H2F(kj[d]);
      s[j] = dot * scale;
      if (s[j] > m) m = s[j];
    }
    float l = 0.0f;
    for (int j = 0; j < ctx; ++j) {
      s[j] = expf(s[j] - m);
      l = l + s[j];
    }
    for (int d = 0; d < QW_HEAD_DIM; ++d) {
      float acc = 0.0f;
      for (int j = 0; j < ctx; ++j)
        acc = acc + s[j] * H2F(v_rows[((size_t)j * QW_KV_HEADS + g) * QW_HEAD_DIM + d]);
      out[h * QW_HEAD_DIM + d] = F2H(acc / l);
    }
  }
  free(s);
}

/* qwen3_full.mlir:829-839, every op in f16: e = exp(-g); den = 1 + e;
 * sig = 1 / den; silu = g * sig; out = silu * up.  f16 arithmetic is the
 * f32 result rounded once to f16 (exact for the add and the multiplies;
 * exp and the reciprocal evaluated in f32). */
void oracle_swiglu(const uint16_t* gate, const uint16_t* up, int n, uint16_t* out) {
  for (int i = 0; i < n; ++i) {
    const float g = H2F(gate[i]);
    const uint16_t e = F2H(expf(-g));
    const uint16_t den = F2H(1.0f + H2F(e));
    const uint16_t sig = F2H(1.0f / H2F(den));
    const uint16_t silu = F2H(g * H2F(sig));
    out[i] = F2H(H2F(silu) * H2F(up[i]));
  }
}

/* f16 + f16 (arith.addf on f16, qwen3_full.mlir:801-805, 858-862). */
void oracle_add_f16(const uint16_t* a, const uint16_t* b, int n, uint16_t* out) {
  for (int i = 0; i < n; ++i) out[i] = F2H(H2F(a[i]) + H2F(b[i]));
}

static const uint8_t* layer_q8(const uint8_t* stacked, int layer, int64_t n, int64_t k) {
  return stacked + (int64_t)layer * (n * k / 32 * 34);
}

/* @transformer_layer_decode_static (qwen3_full.mlir:751-864) with
 * @attention_block_decode_static (591-748) for one layer at position pos:
 * attention reads cache slots [0, pos) of this layer plus the new k/v, which
 * are written to slot pos (slot = layer*max_seq + pos, :792-797). */
void oracle_decode_layer(const oracle_qwen3_weights* w, int layer, uint16_t* k_cache,
                         uint16_t* v_cache, int64_t max_seq, int32_t pos, const uint16_t* h_in,
                         uint16_t* h_out, oracle_layer_trace* trace) {
  uint16_t normed[QW_HIDDEN], q[QW_Q_DIM], k[QW_KV_DIM], v[QW_KV_DIM];
  uint16_t qn[QW_Q_DIM], kn[QW_KV_DIM], qr[QW_Q_DIM], kr[QW_KV_DIM];
  uint16_t attn[QW_Q_DIM], o[QW_HIDDEN], res1[QW_HIDDEN], fnorm[QW_HIDDEN];
  uint16_t gu[2 * QW_FFN], act[QW_FFN], dn[QW_HIDDEN];

  oracle_rmsnorm(h_in, w->attn_norm + layer * QW_HIDDEN, QW_HIDDEN, QW_EPS, normed);
  oracle_q8_gemv(layer_q8(w->wq, layer, QW_Q_DIM, QW_HIDDEN), QW_Q_DIM, QW_HIDDEN, normed, q);
  oracle_q8_gemv(layer_q8(w->wk, layer, QW_KV_DIM, QW_HIDDEN), QW_KV_DIM, QW_HIDDEN, normed, k);
  oracle_q8_gemv(layer_q8(w->wv, layer, QW_KV_DIM, QW_HIDDEN), QW_KV_DIM, QW_HIDDEN, normed, v);
  oracle_head_rmsnorm(q, QW_Q_HEADS, w->q_norm + layer * QW_HEAD_DIM, QW_EPS, qn);
  oracle_head_rmsnorm(k, QW_KV_HEADS, w->k_norm + layer * QW_HEAD_DIM, QW_EPS, kn);
  oracle_rope(qn, QW_Q_HEADS, pos, qr);
  oracle_rope(kn, QW_KV_HEADS, pos, kr);
  uint16_t* kl = k_cache + (size_t)layer * max_seq * QW_KV_DIM;
  uint16_t* vl = v_cache + (size_t)layer * max_seq * QW_KV_DIM;
  memcpy(kl + (size_t)pos * QW_KV_DIM, kr, sizeof(kr));
  memcpy(vl + (size_t)pos * QW_KV_DIM, v, sizeof(v));
  oracle_attention(qr, kl, vl, pos + 1, QW_ATTN_SCALE, attn);
  oracle_q8_gemv(layer_q8(w->wo, layer, QW_HIDDEN, QW_Q_DIM), QW_HIDDEN, QW_Q_DIM, attn, o);
  oracle_add_f16(h_in, o, QW_HIDDEN, res1);
  oracle_rmsnorm(res1, w->ffn_norm + layer * QW_HIDDEN, QW_HIDDEN, QW_EPS, fnorm);
  oracle_q8_gemv(layer_q8(w->wgu, layer, 2 * QW_FFN, QW_HIDDEN), 2 * QW_FFN, QW_HIDDEN, fnorm, gu);
  oracle_swiglu(gu, gu + QW_FFN, QW_FFN, act);
  oracle_q8_gemv(layer_q8(w->wdn, layer, QW_HIDDEN, QW_FFN), QW_HIDDEN, QW_FFN, act, dn);
  oracle_add_f16(res1, dn, QW_HIDDEN, h_out);
  if (trace) {
    memcpy(trace->q_roped, qr, sizeof(qr));
    memcpy(trace->k_roped, kr, sizeof(kr));
    memcpy(trace->v, v, sizeof(v));
    memcpy(trace->attn, attn, sizeof(attn));
    memcpy(trace->res1, res1, sizeof(res1));
    memcpy(trace->act, act, sizeof(act));
  }
}

/* One token of @generate's inner loop (qwen3_full.mlir:1431-1511): embedding
 * gather (:86-94, 1436), 28 layers, final rms_norm (:1456), vocab GEMV (:1467)
 * and the tiled argmax (:1469-1511).  Writes the f16 logits if `logits` is not
 * NULL and the hidden state after every layer if `h_layers` is not NULL
 * ([29][1024]: the embedding row, then layer 0..27).  Returns the token. */
int64_t oracle_decode_step(const oracle_qwen3_weights* w, uint16_t* k_cache, uint16_t* v_cache,
                           int64_t max_seq, int32_t token, int32_t pos, uint16_t* logits,
                           uint16_t* h_layers) {
  uint16_t h[QW_HIDDEN], h2[QW_HIDDEN], normed[QW_HIDDEN];
  memcpy(h, w->token_embd + (size_t)token * QW_HIDDEN, sizeof(h));
  if (h_layers) memcpy(h_layers, h, sizeof(h));
  for (int l = 0; l < QW_LAYERS; ++l) {
    oracle_decode_layer(w, l, k_cache, v_cache, max_seq, pos, h, h2, NULL);
    memcpy(h, h2, sizeof(h));
    if (h_layers) memcpy(h_layers + (size_t)(l + 1) * QW_HIDDEN, h, sizeof(h));
  }
  oracle_rmsnorm(h, w->output_norm, QW_HIDDEN, QW_EPS, normed);
  uint16_t* lg = logits ? logits : (uint16_t*)malloc(sizeof(uint16_t) * QW_VOCAB);
  oracle_f16_gemv(w->output_w, QW_VOCAB, QW_HIDDEN, normed, lg);
  int64_t tok = oracle_argmax_tiled(lg, QW_VOCAB, 256);
  if (!logits) free(lg);
  return tok;
}
