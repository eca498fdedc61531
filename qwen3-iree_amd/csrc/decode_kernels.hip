// gfx950 kernels for the rest of the Qwen3-0.6B decode step, built around the
// Q8_0 GEMV engine of q8_device.h.  One layer
// (model/qwen3_full.mlir:751-864 with @attention_block_decode_static 591-748)
// is six launches:
//
//   dec_qkv          rms_norm(h, attn_norm) fused into the q/k/v GEMVs
//   dec_attn_split   q/k head norms + RoPE, the new k/v written to the flat
//                    KV cache, and split-K GQA attention partials (8 kv heads
//                    x 32 position splits)
//   dec_attn_combine the per-split softmax partials merged per query head
//   dec_o_res        attn_o GEMV + residual add
//   dec_gu_swiglu    rms_norm(res, ffn_norm) fused into gate_up; each wave
//                    computes a gate quad and the matching up quad and applies
//                    SwiGLU in its epilogue
//   dec_down_res     ffn_down GEMV + residual add
//
// plus dec_embed (token row gather), dec_vocab_argmax (final rms_norm fused
// into the vocab GEMV + argmax) and dec_finalize (token, position).
//
// Numerics follow the reference op by op: f16 tensors between ops, f32 in
// reductions and transcendental math, RNE to f16.  Normalisation multiplies by
// 1/rms where the reference divides by rms (one f32 rounding apart).
#include "q8_device.h"

namespace {

constexpr int kHidden = 1024;
constexpr int kHeadDim = 128;
constexpr int kKvHeads = 8;
constexpr int kFfn = 3072;
constexpr int kVocab = 151936;
constexpr int kAttnSplits = 32;
constexpr int kPartStride = 2 + kHeadDim;  // m, l, acc[128] per (query head, split)
constexpr float kEps = 9.99999997e-7f;    // qwen3_full.mlir:63
constexpr float kRopeBase = 1.0e6f;       // qwen3_full.mlir:59
// rsqrt(128) of qwen3_full.mlir:721-723, the f32 nearest 2^-3.5 (0x3DB504F3)
constexpr float kAttnScale = 0.0883883461356163f;

__device__ __forceinline__ float wave_sum(float v) {
  v = reduce_row16(v);
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

__device__ __forceinline__ float max32(float v) {  // over the 32 lanes of a wave half
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  return fmaxf(v, __shfl_xor(v, 16, 64));
}

__device__ __forceinline__ float sum32(float v) {
  v = reduce_row16(v);
  return v + __shfl_xor(v, 16, 64);
}

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  return (uint32_t)f32_to_f16_bits(a) | ((uint32_t)f32_to_f16_bits(b) << 16);
}

__device__ __forceinline__ _Float16 as_half(uint16_t b) { return __builtin_bit_cast(_Float16, b); }

// rms_norm of a 1024-vector (qwen3_full.mlir:134-165) for the 64 columns
// col(m, j) of this lane: the 16 lanes of a DPP row together hold all 1024
// columns, so their partial sums of squares meet in a row reduction.
template <class ColOf>
__device__ __forceinline__ void rmsnorm_cols(const uint16_t* __restrict__ h,
                                             const uint16_t* __restrict__ w, ColOf col,
                                             u32x4 (&xr)[8]) {
  u32x4 hv[8], wv[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    hv[m] = load_global(reinterpret_cast<const u32x4*>(h + col(m)));
    wv[m] = load_global(reinterpret_cast<const u32x4*>(w + col(m)));
  }
  float ss = 0.0f;
#pragma unroll
  for (int m = 0; m < 8; ++m) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f16x2 hp = as_f16x2(hv[m][j]);
      const float a = (float)hp.x, b = (float)hp.y;
      ss = ss + a * a;
      ss = ss + b * b;
    }
  }
  ss = reduce_row16(ss);
  const float inv = 1.0f / sqrtf(ss / 1024.0f + kEps);
#pragma unroll
  for (int m = 0; m < 8; ++m) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f16x2 hp = as_f16x2(hv[m][j]), wp = as_f16x2(wv[m][j]);
      const float a = ((float)hp.x * inv) * (float)wp.x;
      const float b = ((float)hp.y * inv) * (float)wp.y;
      xr[m][j] = pack_f16x2(a, b);
    }
  }
}

// The Q8_0 GEMV lane layout: columns [64 p16, 64 p16 + 64) in 8 pieces of 8.
__device__ __forceinline__ void rmsnorm_gemv_x(const uint16_t* __restrict__ h,
                                               const uint16_t* __restrict__ w, u32x4 (&xr)[8]) {
  const int p16 = threadIdx.x & 15;
  rmsnorm_cols(h, w, [=](int m) { return 64 * p16 + 8 * m; }, xr);
}

// SwiGLU of qwen3_full.mlir:829-839, every op in f16: e = exp(-g),
// den = 1 + e, sig = 1 / den, silu = g * sig, out = silu * up (exp and the
// reciprocal evaluated in f32 and rounded once).
__device__ __forceinline__ uint16_t swiglu_f16(float gate_acc, float up_acc) {
  const _Float16 g = (_Float16)gate_acc;
  const _Float16 u = (_Float16)up_acc;
  const _Float16 e = (_Float16)expf(-(float)g);
  const _Float16 den = (_Float16)1.0f + e;
  const _Float16 sig = (_Float16)(1.0f / (float)den);
  const _Float16 silu = g * sig;
  return __builtin_bit_cast(uint16_t, (_Float16)(silu * u));
}

}  // namespace

// ------------------------------------------------------------- kernels ----

// h = token_embd[token] (qwen3_full.mlir:86-94); the token is read on the
// device so a captured step can consume the previous step's argmax.  An id
// outside [0, 151936) reads row 0.
extern "C" __global__ __launch_bounds__(128) void dec_embed(const int32_t* __restrict__ token,
                                                            const uint16_t* __restrict__ embd,
                                                            uint16_t* __restrict__ h) {
  int t = *token;
  t = (t < 0 || t >= kVocab) ? 0 : t;
  reinterpret_cast<u32x4*>(h)[threadIdx.x] =
      load_global(reinterpret_cast<const u32x4*>(embd + (size_t)t * kHidden) + threadIdx.x);
}

// Workgroup 0 also stores the normalised vector it computed (every workgroup
// computes the same one) so the step's intermediate can be inspected.
__device__ __forceinline__ void store_gemv_x(const u32x4 (&xr)[8], uint16_t* __restrict__ out) {
  const int lane = threadIdx.x;
  if (blockIdx.x == 0 && lane < 16) {
#pragma unroll
    for (int m = 0; m < 8; ++m) reinterpret_cast<u32x4*>(out + 64 * lane + 8 * m)[0] = xr[m];
  }
}

// q, k, v = W{q,k,v}[layer] . rms_norm(h, attn_norm[layer]); workgroups
// 0..511 the q quads, 512..767 k, 768..1023 v (weights are layer bases).
// xn receives the normalised h (f16[1024]).
extern "C" __global__ __launch_bounds__(64) void dec_qkv(
    const uint8_t* __restrict__ wq, const uint8_t* __restrict__ wk,
    const uint8_t* __restrict__ wv, const uint16_t* __restrict__ h,
    const uint16_t* __restrict__ norm_w, uint16_t* __restrict__ q, uint16_t* __restrict__ k,
    uint16_t* __restrict__ v, uint16_t* __restrict__ xn) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[QuadShape<1>::LDS_BYTES];
  const int b = blockIdx.x;
  const uint8_t* w = b < 512 ? wq : (b < 768 ? wk : wv);
  uint16_t* y = b < 512 ? q : (b < 768 ? k : v);
  const int n = b < 512 ? 2048 : 1024;
  const int quad = b < 512 ? b : (b < 768 ? b - 512 : b - 768);
  q8_quad_core<1>(
      w, n, quad, lds,
      [&](u32x4 (&xr)[1][8]) {
        rmsnorm_gemv_x(h, norm_w, xr[0]);
        store_gemv_x(xr[0], xn);
      },
      [&](int row, float acc) { y[row] = f32_to_f16_bits(acc); });
}

// Attention for kv head g = block / 32 and position split s = block % 32.
//  1. q heads 2g, 2g+1 and k head g: per-head rms_norm with q_norm / k_norm
//     (qwen3_full.mlir:648-702), then RoPE (:324-454) at position pos;
//  2. the split owning position pos writes the roped k and the raw v to
//     cache slot pos (layer base passed in; slot layout [max_seq, 8, 128]);
//  3. positions [s*ctx/32, (s+1)*ctx/32) of ctx = pos + 1: scores
//     s_j = (q . k_j) * rsqrt(128), then an online softmax over chunks of 32
//     positions (lanes 0-31 score head 2g, 32-63 head 2g+1) and the weighted
//     sum of v (each lane owns dims 2*lane, 2*lane+1 of both heads);
//  4. partial (m, l, acc[128]) per query head -> part[head][split].
// Split 0 also stores the roped q heads (f16) to q_roped.
extern "C" __global__ __launch_bounds__(64) void dec_attn_split(
    const uint16_t* __restrict__ q_raw, const uint16_t* __restrict__ k_raw,
    const uint16_t* __restrict__ v_raw, const uint16_t* __restrict__ qn_w,
    const uint16_t* __restrict__ kn_w, const int32_t* __restrict__ pos_ptr, int max_seq,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache, float* __restrict__ part,
    uint16_t* __restrict__ q_roped) {
  const int lane = threadIdx.x;
  const int g = blockIdx.x / kAttnSplits;
  const int s = blockIdx.x % kAttnSplits;
  int pos = *pos_ptr;
  pos = pos < 0 ? 0 : (pos >= max_seq ? max_seq - 1 : pos);
  const int ctx = pos + 1;
  const int start = (int)((int64_t)s * ctx / kAttnSplits);
  const int end = (int)((int64_t)(s + 1) * ctx / kAttnSplits);

  __shared__ float xs[3][kHeadDim];   // normed q_A, q_B, k (f16 values)
  __shared__ uint32_t qh[2][64];      // roped q_A, q_B as f16 pairs
  __shared__ uint32_t kh[64], vh[64]; // roped new k, new v as f16 pairs
  __shared__ float pbuf[2][32];
  __shared__ float cbuf[2];

  // ---- 1. head norms: lane owns dims 2*lane, 2*lane+1 ----
  const uint16_t* src[3] = {q_raw + (2 * g) * kHeadDim, q_raw + (2 * g + 1) * kHeadDim,
                            k_raw + g * kHeadDim};
  const uint16_t* nw[3] = {qn_w, qn_w, kn_w};
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    const f16x2 xv = as_f16x2(reinterpret_cast<const uint32_t*>(src[t])[lane]);
    const f16x2 wv = as_f16x2(reinterpret_cast<const uint32_t*>(nw[t])[lane]);
    const float a = (float)xv.x, b = (float)xv.y;
    float ss = a * a;
    ss = ss + b * b;
    ss = wave_sum(ss);
    const float r = sqrtf(ss / 128.0f + kEps);
    xs[t][2 * lane] = (float)(_Float16)((a / r) * (float)wv.x);
    xs[t][2 * lane + 1] = (float)(_Float16)((b / r) * (float)wv.y);
  }
  const uint32_t v_new = reinterpret_cast<const uint32_t*>(v_raw + g * kHeadDim)[lane];
  __syncthreads();

  // ---- 1b. RoPE (rotate-half) ----
  const float posf = (float)pos;
  float cs[2], sn[2];
#pragma unroll
  for (int dd = 0; dd < 2; ++dd) {
    const int d = 2 * lane + dd;
    const int i = d < 64 ? d : d - 64;
    const float e = -((2.0f * (float)i) / 128.0f);
    const float th = posf * (powf(kRopeBase, e) * 1.0f);
    cs[dd] = cosf(th);
    sn[dd] = sinf(th);
  }
  uint32_t roped[3];
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    float r2[2];
#pragma unroll
    for (int dd = 0; dd < 2; ++dd) {
      const int d = 2 * lane + dd;
      if (d < 64) {
        const float a = xs[t][d] * cs[dd];
        const float b = xs[t][d + 64] * sn[dd];
        r2[dd] = a - b;
      } else {
        const float a = xs[t][d - 64] * sn[dd];
        const float b = xs[t][d] * cs[dd];
        r2[dd] = a + b;
      }
    }
    roped[t] = pack_f16x2(r2[0], r2[1]);
  }
  qh[0][lane] = roped[0];
  qh[1][lane] = roped[1];
  kh[lane] = roped[2];
  vh[lane] = v_new;

  // ---- 2. the new position into the cache (and the roped q heads, once) ----
  if (s == 0) {
    reinterpret_cast<uint32_t*>(q_roped + (2 * g) * kHeadDim)[lane] = roped[0];
    reinterpret_cast<uint32_t*>(q_roped + (2 * g + 1) * kHeadDim)[lane] = roped[1];
  }
  if (start <= pos && pos < end) {
    reinterpret_cast<uint32_t*>(k_cache + ((size_t)pos * kKvHeads + g) * kHeadDim)[lane] = roped[2];
    reinterpret_cast<uint32_t*>(v_cache + ((size_t)pos * kKvHeads + g) * kHeadDim)[lane] = v_new;
  }
  __syncthreads();

  // ---- 3. scores, online softmax, weighted v ----
  const int hsel = lane >> 5;
  const int pl = lane & 31;
  float m = -__builtin_inff(), l = 0.0f;
  float accA0 = 0.0f, accA1 = 0.0f, accB0 = 0.0f, accB1 = 0.0f;
  for (int c0 = start; c0 < end; c0 += 32) {
    const int p = c0 + pl;
    const bool valid = p < end;
    float sc = -__builtin_inff();
    if (valid) {
      float dot = 0.0f;
      if (p == pos) {
#pragma unroll 8
        for (int i = 0; i < 64; ++i)
          dot = __builtin_amdgcn_fdot2(as_f16x2(qh[hsel][i]), as_f16x2(kh[i]), dot, false);
      } else {
        const u32x4* krow =
            reinterpret_cast<const u32x4*>(k_cache + ((size_t)p * kKvHeads + g) * kHeadDim);
#pragma unroll
        for (int mm = 0; mm < 16; ++mm) {
          const u32x4 kv = load_global(krow + mm);
#pragma unroll
          for (int j = 0; j < 4; ++j)
            dot = __builtin_amdgcn_fdot2(as_f16x2(qh[hsel][4 * mm + j]), as_f16x2(kv[j]), dot,
                                         false);
        }
      }
      sc = dot * kAttnScale;
    }
    const float mn = fmaxf(m, max32(sc));  // finite: a chunk holds >= 1 valid position
    const float corr = expf(m - mn);       // exp(-inf) = 0 on the first chunk
    const float pj = valid ? expf(sc - mn) : 0.0f;
    l = l * corr + sum32(pj);
    m = mn;
    pbuf[hsel][pl] = pj;
    if (pl == 0) cbuf[hsel] = corr;
    __syncthreads();
    const float cA = cbuf[0], cB = cbuf[1];
    accA0 *= cA;
    accA1 *= cA;
    accB0 *= cB;
    accB1 *= cB;
    const int n = end - c0 < 32 ? end - c0 : 32;
    for (int j = 0; j < n; ++j) {
      const int pp = c0 + j;
      const uint32_t vw = (pp == pos)
          ? vh[lane]
          : reinterpret_cast<const uint32_t*>(v_cache + ((size_t)pp * kKvHeads + g) * kHeadDim)[lane];
      const f16x2 vv = as_f16x2(vw);
      const float v0 = (float)vv.x, v1 = (float)vv.y;
      const float pa = pbuf[0][j], pb = pbuf[1][j];
      accA0 = accA0 + pa * v0;
      accA1 = accA1 + pa * v1;
      accB0 = accB0 + pb * v0;
      accB1 = accB1 + pb * v1;
    }
    __syncthreads();
  }

  // ---- 4. partials ----
  float* pa = part + ((size_t)(2 * g) * kAttnSplits + s) * kPartStride;
  float* pb = part + ((size_t)(2 * g + 1) * kAttnSplits + s) * kPartStride;
  if (lane == 0) {
    pa[0] = m;
    pa[1] = l;
  }
  if (lane == 32) {
    pb[0] = m;
    pb[1] = l;
  }
  pa[2 + 2 * lane] = accA0;
  pa[3 + 2 * lane] = accA1;
  pb[2 + 2 * lane] = accB0;
  pb[3 + 2 * lane] = accB1;
}

// out[head*128 + d] = f16(sum_s w_s acc_s[d] / sum_s w_s l_s), w_s = exp(m_s - M).
extern "C" __global__ __launch_bounds__(128) void dec_attn_combine(const float* __restrict__ part,
                                                                   uint16_t* __restrict__ out) {
  const int h = blockIdx.x;
  const int d = threadIdx.x;
  const float* ph = part + (size_t)h * kAttnSplits * kPartStride;
  float M = -__builtin_inff();
  for (int s = 0; s < kAttnSplits; ++s) M = fmaxf(M, ph[s * kPartStride]);
  float L = 0.0f, acc = 0.0f;
  for (int s = 0; s < kAttnSplits; ++s) {
    const float ms = ph[s * kPartStride];
    if (ms != -__builtin_inff()) {
      const float w = expf(ms - M);
      L = L + ph[s * kPartStride + 1] * w;
      acc = acc + ph[s * kPartStride + 2 + d] * w;
    }
  }
  out[h * kHeadDim + d] = f32_to_f16_bits(acc / L);
}

// res = h + f16(W_o[layer] . attn)   (qwen3_full.mlir:739, 801-805)
extern "C" __global__ __launch_bounds__(64) void dec_o_res(const uint8_t* __restrict__ wo,
                                                           const uint16_t* __restrict__ attn,
                                                           const uint16_t* __restrict__ h,
                                                           uint16_t* __restrict__ res) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[QuadShape<2>::LDS_BYTES];
  q8_quad_core<2>(
      wo, kHidden, blockIdx.x, lds, [&](u32x4 (&xr)[2][8]) { load_x_cols<2>(attn, xr); },
      [&](int row, float acc) {
        res[row] = __builtin_bit_cast(uint16_t, (_Float16)(as_half(h[row]) + (_Float16)acc));
      });
}

// act[i] = swiglu(gate_i, up_i) with [gate; up] = W_gu[layer] . rms_norm(res,
// ffn_norm[layer]) (qwen3_full.mlir:807-839).  Wave b computes gate quad b
// (rows 4b..4b+3) and up quad b (rows 3072+4b..), so both operands of its
// four outputs are in its own lanes.  xn receives the normalised res.
extern "C" __global__ __launch_bounds__(64) void dec_gu_swiglu(const uint8_t* __restrict__ wgu,
                                                               const uint16_t* __restrict__ res,
                                                               const uint16_t* __restrict__ norm_w,
                                                               uint16_t* __restrict__ act,
                                                               uint16_t* __restrict__ xn) {
  constexpr int LDSB = QuadShape<1>::LDS_BYTES;
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * LDSB];
  const int b = blockIdx.x;
  u32x4 bg[QuadShape<1>::LOADS], bu[QuadShape<1>::LOADS];
  q8_quad_load<1>(wgu, 2 * kFfn, b, bg);
  q8_quad_load<1>(wgu, 2 * kFfn, kFfn / 4 + b, bu);
  u32x4 xr[1][8];
  rmsnorm_gemv_x(res, norm_w, xr[0]);
  store_gemv_x(xr[0], xn);
  q8_quad_stage<1>(bg, lds);
  q8_quad_stage<1>(bu, lds + LDSB);
  __syncthreads();
  const float ag = q8_quad_dot<1>(lds, xr);
  const float au = q8_quad_dot<1>(lds + LDSB, xr);
  const int lane = threadIdx.x;
  if ((lane & 15) == 0) act[4 * b + (lane >> 4)] = swiglu_f16(ag, au);
}

// h_out = res + f16(W_dn[layer] . act)   (qwen3_full.mlir:852, 858-862)
extern "C" __global__ __launch_bounds__(64) void dec_down_res(const uint8_t* __restrict__ wdn,
                                                              const uint16_t* __restrict__ act,
                                                              const uint16_t* __restrict__ res,
                                                              uint16_t* __restrict__ h_out) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[QuadShape<3>::LDS_BYTES];
  q8_quad_core<3>(
      wdn, kHidden, blockIdx.x, lds, [&](u32x4 (&xr)[3][8]) { load_x_cols<3>(act, xr); },
      [&](int row, float acc) {
        h_out[row] = __builtin_bit_cast(uint16_t, (_Float16)(as_half(res[row]) + (_Float16)acc));
      });
}

// logits = W_out . rms_norm(h, output_norm) (qwen3_full.mlir:1456-1467) with
// the fused argmax into ws (see vocab_body_x).  xn receives the normalised h.
extern "C" __global__ __launch_bounds__(256) void dec_vocab_argmax(
    const uint16_t* __restrict__ W, const uint16_t* __restrict__ h,
    const uint16_t* __restrict__ norm_w, uint16_t* __restrict__ logits, uint8_t* __restrict__ ws,
    uint16_t* __restrict__ xn) {
  vocab_body_x<VOCAB_NT_LOADS != 0, true>(
      W,
      [&](int li, u32x4 (&xr)[8]) {
        rmsnorm_cols(h, norm_w, [=](int m) { return 128 * m + 8 * li; }, xr);
        if (blockIdx.x == 0 && threadIdx.x < 16) {
#pragma unroll
          for (int m = 0; m < 8; ++m)
            reinterpret_cast<u32x4*>(xn + 128 * m + 8 * li)[0] = xr[m];
        }
      },
      logits, kVocab, ws);
}

// *token = the argmax (the key's row, -1 for none), the key zeroed; with
// advance, *pos moves to the next slot unless the cache is full (then
// status bit 0 is set and *pos stays).
extern "C" __global__ void dec_finalize(uint64_t* __restrict__ ws, int32_t* __restrict__ token,
                                        int32_t* __restrict__ pos, int advance, int max_seq,
                                        uint32_t* __restrict__ status) {
  if (threadIdx.x == 0) {
    const uint64_t key = ws[0];
    *token = key == 0 ? -1 : (int32_t)(0xffffffffu - (uint32_t)(key & 0xffffffffu));
    ws[0] = 0;
    if (advance) {
      const int p = *pos;
      if (p + 1 < max_seq) *pos = p + 1;
      else *status |= 1u;
    }
  }
}
