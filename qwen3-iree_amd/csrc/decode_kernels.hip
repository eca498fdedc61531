// gfx950 kernels for the rest of the Qwen3-0.6B decode step, built around the
// Q8_0 GEMV engine of q8_device.h.  One layer
// (model/qwen3_full.mlir:751-864 with @attention_block_decode_static 591-748)
// is five launches:
//
//   dec_qkv          rms_norm(h, attn_norm) fused into the q/k/v GEMVs
//   dec_attention    q/k head norms + RoPE, the new k/v written to the flat
//                    KV cache, split-K GQA attention partials (8 kv heads x 32
//                    position splits), merged by the last split of each kv
//                    head
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
constexpr int kAttnSplits = 32;      // position splits per kv head (one wave each)
constexpr int kAttnWaves = 4;        // splits per workgroup, merged in LDS
constexpr int kAttnGroups = kAttnSplits / kAttnWaves;  // partials per query head
constexpr int kPartStride = 4 + kHeadDim;  // m, l, 2 pad, acc[128] (16-byte aligned acc)
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

// Attention for kv head g = block / 8 and split group sg = block % 8: four
// waves, wave w taking position split s = 4 sg + w of the 32 equal splits of
// ctx = pos + 1; the four results merge in LDS into one partial per query
// head and group (the attn_o kernel merges the 8 groups).  Per wave:
//  0. the split's first 32 cache rows (K: half a row per lane, V: the lane's
//     two dims for each of the 32 positions) are requested before anything
//     else, so their latency overlaps steps 1-2;
//  1. q heads 2g, 2g+1 and k head g: per-head rms_norm with q_norm / k_norm
//     (qwen3_full.mlir:648-702), then RoPE (:324-454) at position pos;
//  2. the wave owning position pos writes the roped k and the raw v to cache
//     slot pos (layer base passed in; slot layout [max_seq, 8, 128]); split 0
//     stores the roped q heads (f16) to q_roped;
//  3. chunks of 32 positions: lane (j, half) scores position j of the chunk
//     on dims [64*half, 64*half + 64) for both q heads, the halves meet in one
//     cross-half add; s_j = (q . k_j) * rsqrt(128); online softmax; the
//     weighted sum of v (each lane owns dims 2*lane, 2*lane+1 of both heads).
//     The chunk count is uniform over the workgroup (splits differ by at most
//     one position), so every wave meets every barrier;
//  4. partial (m, l, acc[128]) per query head -> part[head][sg]: m = max over
//     the 4 waves, l and acc rescaled by exp(m_w - m).  An empty split (ctx <
//     32) contributes m = -inf, l = 0, acc = 0.
extern "C" __global__ __launch_bounds__(256) void dec_attention(
    const uint16_t* __restrict__ q_raw, const uint16_t* __restrict__ k_raw,
    const uint16_t* __restrict__ v_raw, const uint16_t* __restrict__ qn_w,
    const uint16_t* __restrict__ kn_w, const int32_t* __restrict__ pos_ptr, int max_seq,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache, float* __restrict__ part,
    uint16_t* __restrict__ q_roped) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int g = blockIdx.x / kAttnGroups;
  const int sg = blockIdx.x % kAttnGroups;
  const int s = sg * kAttnWaves + wave;
  const int half = lane >> 5;
  const int pl = lane & 31;

  // ---- inputs that do not depend on the position ----
  const uint16_t* src[3] = {q_raw + (2 * g) * kHeadDim, q_raw + (2 * g + 1) * kHeadDim,
                            k_raw + g * kHeadDim};
  uint32_t xw[3], nwv[3];
#pragma unroll
  for (int t = 0; t < 3; ++t) xw[t] = load_global(reinterpret_cast<const uint32_t*>(src[t]) + lane);
  nwv[0] = load_global(reinterpret_cast<const uint32_t*>(qn_w) + lane);
  nwv[2] = load_global(reinterpret_cast<const uint32_t*>(kn_w) + lane);
  nwv[1] = nwv[0];
  const uint32_t v_new = load_global(reinterpret_cast<const uint32_t*>(v_raw + g * kHeadDim) + lane);
  __builtin_amdgcn_sched_barrier(0);  // keep these loads ahead of the position-dependent ones

  int pos = *pos_ptr;
  pos = pos < 0 ? 0 : (pos >= max_seq ? max_seq - 1 : pos);
  const int ctx = pos + 1;
  const int start = (int)((int64_t)s * ctx / kAttnSplits);
  const int end = (int)((int64_t)(s + 1) * ctx / kAttnSplits);
  const int n_chunks = ((ctx + kAttnSplits - 1) / kAttnSplits + 31) / 32;  // workgroup-uniform

  // ---- 0. first chunk of the cache ----
  // Every lane issues every load (rows clamped into [start, end - 1], row 0
  // for an empty split) so the compiler's waits stay exact.
  const int last = end - 1 > 0 ? end - 1 : 0;
  u32x4 kreg[8];
  uint32_t vreg[32];
  auto load_chunk = [&](int c0) {
    const int p = c0 + pl < last ? c0 + pl : last;
    const u32x4* krow = reinterpret_cast<const u32x4*>(
        k_cache + ((size_t)p * kKvHeads + g) * kHeadDim + 64 * half);
#pragma unroll
    for (int m = 0; m < 8; ++m) kreg[m] = load_global(krow + m);
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const int pj = c0 + j < last ? c0 + j : last;
      vreg[j] = load_global(
          reinterpret_cast<const uint32_t*>(v_cache + ((size_t)pj * kKvHeads + g) * kHeadDim) + lane);
    }
  };
  load_chunk(start);
  __builtin_amdgcn_sched_barrier(0);

  __shared__ float xs[kAttnWaves][3][kHeadDim];  // normed q_A, q_B, k (f16 values)
  __shared__ uint32_t qh[kAttnWaves][2][64];     // roped q_A, q_B as f16 pairs
  __shared__ uint32_t kh[kAttnWaves][64];        // roped new k as f16 pairs
  __shared__ float pbuf[kAttnWaves][2][32];
  __shared__ float mrg[kAttnWaves][2][2 + kHeadDim];

  // ---- 1. head norms: lane owns dims 2*lane, 2*lane+1 ----
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    const f16x2 xv = as_f16x2(xw[t]);
    const f16x2 wv = as_f16x2(nwv[t]);
    const float a = (float)xv.x, b = (float)xv.y;
    float ss = a * a;
    ss = ss + b * b;
    ss = wave_sum(ss);
    const float r = sqrtf(ss / 128.0f + kEps);
    xs[wave][t][2 * lane] = (float)(_Float16)((a / r) * (float)wv.x);
    xs[wave][t][2 * lane + 1] = (float)(_Float16)((b / r) * (float)wv.y);
  }
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
        const float a = xs[wave][t][d] * cs[dd];
        const float b = xs[wave][t][d + 64] * sn[dd];
        r2[dd] = a - b;
      } else {
        const float a = xs[wave][t][d - 64] * sn[dd];
        const float b = xs[wave][t][d] * cs[dd];
        r2[dd] = a + b;
      }
    }
    roped[t] = pack_f16x2(r2[0], r2[1]);
  }
  qh[wave][0][lane] = roped[0];
  qh[wave][1][lane] = roped[1];
  kh[wave][lane] = roped[2];

  // ---- 2. the new position into the cache, the roped q heads once ----
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
  float m = -__builtin_inff(), l = 0.0f;  // per q head; identical in all lanes
  float mB = -__builtin_inff(), lB = 0.0f;
  float accA0 = 0.0f, accA1 = 0.0f, accB0 = 0.0f, accB1 = 0.0f;
  for (int c = 0; c < n_chunks; ++c) {
    const int c0 = start + 32 * c;
    const int p = c0 + pl;
    const bool valid = p < end;
    // the row of position pos is this step's k (in LDS; the cache slot was
    // requested before it was written)
    const bool is_new = p == pos;
    float dA = 0.0f, dB = 0.0f;
#pragma unroll
    for (int mm = 0; mm < 8; ++mm) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = 32 * half + 4 * mm + j;
        const f16x2 kv = as_f16x2(is_new ? kh[wave][i] : kreg[mm][j]);
        dA = __builtin_amdgcn_fdot2(as_f16x2(qh[wave][0][i]), kv, dA, false);
        dB = __builtin_amdgcn_fdot2(as_f16x2(qh[wave][1][i]), kv, dB, false);
      }
    }
    dA = dA + __shfl_xor(dA, 32, 64);
    dB = dB + __shfl_xor(dB, 32, 64);
    const float sA = valid ? dA * kAttnScale : -__builtin_inff();
    const float sB = valid ? dB * kAttnScale : -__builtin_inff();
    const float mnA = fmaxf(m, max32(sA));
    const float mnB = fmaxf(mB, max32(sB));
    // mn = -inf only while the split has seen no valid position (acc, l = 0)
    const float cA = mnA == -__builtin_inff() ? 1.0f : expf(m - mnA);
    const float cB = mnB == -__builtin_inff() ? 1.0f : expf(mB - mnB);
    const float pA = valid ? expf(sA - mnA) : 0.0f;
    const float pB = valid ? expf(sB - mnB) : 0.0f;
    l = l * cA + sum32(pA);
    lB = lB * cB + sum32(pB);
    m = mnA;
    mB = mnB;
    if (half == 0) {
      pbuf[wave][0][pl] = pA;
      pbuf[wave][1][pl] = pB;
    }
    __syncthreads();
    accA0 *= cA;
    accA1 *= cA;
    accB0 *= cB;
    accB1 *= cB;
    const int n = end - c0 < 32 ? end - c0 : 32;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      // positions past the split hold weight 0 and a clamped (valid) row,
      // selected to 0 so a non-finite value there cannot leak in
      const uint32_t vw = c0 + j == pos ? v_new : (j < n ? vreg[j] : 0u);
      const f16x2 vv = as_f16x2(vw);
      const float v0 = (float)vv.x, v1 = (float)vv.y;
      const float wa = pbuf[wave][0][j], wb = pbuf[wave][1][j];
      accA0 = accA0 + wa * v0;
      accA1 = accA1 + wa * v1;
      accB0 = accB0 + wb * v0;
      accB1 = accB1 + wb * v1;
    }
    __syncthreads();
    if (c + 1 < n_chunks) load_chunk(c0 + 32);
  }

  // ---- 4. the four waves' results -> one partial per query head ----
  if (lane == 0) {
    mrg[wave][0][0] = m;
    mrg[wave][0][1] = l;
    mrg[wave][1][0] = mB;
    mrg[wave][1][1] = lB;
  }
  mrg[wave][0][2 + 2 * lane] = accA0;
  mrg[wave][0][3 + 2 * lane] = accA1;
  mrg[wave][1][2 + 2 * lane] = accB0;
  mrg[wave][1][3 + 2 * lane] = accB1;
  __syncthreads();
  if (wave < 2) {  // wave hh merges query head 2g + hh
    const int hh = wave;
    float M = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, mrg[w][hh][0]);
    float L = 0.0f, a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) {
      const float mw = mrg[w][hh][0];
      const float ww = mw == -__builtin_inff() ? 0.0f : expf(mw - M);
      L = L + mrg[w][hh][1] * ww;
      a0 = a0 + mrg[w][hh][2 + 2 * lane] * ww;
      a1 = a1 + mrg[w][hh][3 + 2 * lane] * ww;
    }
    float* dst = part + ((size_t)(2 * g + hh) * kAttnGroups + sg) * kPartStride;
    if (lane == 0) {
      dst[0] = M;
      dst[1] = L;
    }
    reinterpret_cast<float2*>(dst + 4)[lane] = float2{a0, a1};
  }
}

// attn = the merged attention output: head h, dim d =
// sum_g w_g acc_g[d] / sum_g w_g l_g over the 8 partials g of head h, w_g =
// exp(m_g - max m); then res = h + f16(W_o[layer] . attn)
// (qwen3_full.mlir:739, 801-805).  Four waves per workgroup, one row quad
// each; the workgroup's 256 threads merge 8 dims each into LDS while the
// weight loads are in flight.  Workgroup 0 also stores attn.
extern "C" __global__ __launch_bounds__(256) void dec_o_res(const uint8_t* __restrict__ wo,
                                                            const float* __restrict__ part,
                                                            const uint16_t* __restrict__ h,
                                                            uint16_t* __restrict__ res,
                                                            uint16_t* __restrict__ attn_out) {
  constexpr int LDSB = QuadShape<2>::LDS_BYTES;
  __shared__ __attribute__((aligned(16))) uint8_t lds[4 * LDSB];
  __shared__ __attribute__((aligned(16))) uint16_t attn[2 * kHidden];
  const int t = threadIdx.x;
  const int wave = t >> 6;
  // the residual of this lane's row, requested up front; all 1024 rows exist,
  // and every lane of a row group stores the (same) result, so nothing here
  // is conditional and the load stays ahead of the GEMV
  const int row = 4 * (4 * blockIdx.x + wave) + ((t & 63) >> 4);
  const _Float16 h_row = as_half(load_global_u16(h + row));
  const float acc = q8_quad_core_acc<2>(
      wo, kHidden, 4 * blockIdx.x + wave, lds + wave * LDSB,
      [&](u32x4 (&xr)[2][8]) {
        const int head = t >> 4;
        const int d0 = 8 * (t & 15);
        const float* ph = part + (size_t)head * kAttnGroups * kPartStride;
        float2 ml[kAttnGroups];
        u32x4 av[kAttnGroups][2];
#pragma unroll
        for (int gi = 0; gi < kAttnGroups; ++gi) {
          const float* pg = ph + (size_t)gi * kPartStride;
          ml[gi] = *reinterpret_cast<const float2*>(pg);
          av[gi][0] = load_global(reinterpret_cast<const u32x4*>(pg + 4 + d0));
          av[gi][1] = load_global(reinterpret_cast<const u32x4*>(pg + 4 + d0) + 1);
        }
        float M = -__builtin_inff();
#pragma unroll
        for (int gi = 0; gi < kAttnGroups; ++gi) M = fmaxf(M, ml[gi].x);
        float wg[kAttnGroups], L = 0.0f;
#pragma unroll
        for (int gi = 0; gi < kAttnGroups; ++gi) {
          wg[gi] = ml[gi].x == -__builtin_inff() ? 0.0f : expf(ml[gi].x - M);
          L = L + ml[gi].y * wg[gi];
        }
        float a[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int gi = 0; gi < kAttnGroups; ++gi) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            // copy the element out first: __builtin_bit_cast of a vector
            // element lvalue reads element 0 with this compiler
            const uint32_t bits = av[gi][e >> 2][e & 3];
            a[e] = a[e] + __builtin_bit_cast(float, bits) * wg[gi];
          }
        }
        const u32x4 packed = {pack_f16x2(a[0] / L, a[1] / L), pack_f16x2(a[2] / L, a[3] / L),
                              pack_f16x2(a[4] / L, a[5] / L), pack_f16x2(a[6] / L, a[7] / L)};
        reinterpret_cast<u32x4*>(attn)[t] = packed;
        if (blockIdx.x == 0) reinterpret_cast<u32x4*>(attn_out)[t] = packed;
        __syncthreads();
        // x for this lane's GEMV columns, from the merged vector in LDS
        const int p16 = t & 15;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const u32x4* xs4 = reinterpret_cast<const u32x4*>(attn + 1024 * c + 64 * p16);
#pragma unroll
          for (int m8 = 0; m8 < 8; ++m8) xr[c][m8] = xs4[m8];
        }
      });
  res[row] = __builtin_bit_cast(uint16_t, (_Float16)(h_row + (_Float16)acc));
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
  // residual requested up front; unconditional store by the whole row group
  const int row = 4 * blockIdx.x + (threadIdx.x >> 4);
  const _Float16 r_row = as_half(load_global_u16(res + row));
  const float acc = q8_quad_core_acc<3>(
      wdn, kHidden, blockIdx.x, lds, [&](u32x4 (&xr)[3][8]) { load_x_cols<3>(act, xr); });
  h_out[row] = __builtin_bit_cast(uint16_t, (_Float16)(r_row + (_Float16)acc));
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

// *token = the argmax (the key's row, -1 for none), the key zeroed, and the
// token also stored to *out when out is not null (a generation loop's output
// slot); with advance, *pos moves to the next slot unless the cache is full
// (then status bit 0 is set and *pos stays).
extern "C" __global__ void dec_finalize(uint64_t* __restrict__ ws, int32_t* __restrict__ token,
                                        int32_t* __restrict__ pos, int advance, int max_seq,
                                        uint32_t* __restrict__ status, int32_t* __restrict__ out) {
  if (threadIdx.x == 0) {
    const uint64_t key = ws[0];
    const int32_t t = key == 0 ? -1 : (int32_t)(0xffffffffu - (uint32_t)(key & 0xffffffffu));
    *token = t;
    if (out != nullptr) *out = t;
    ws[0] = 0;
    if (advance) {
      const int p = *pos;
      if (p + 1 < max_seq) *pos = p + 1;
      else *status |= 1u;
    }
  }
}

// *pos moves to the next slot (as dec_finalize's advance) without a token:
// the end of a prompt step whose logits are not needed.
extern "C" __global__ void dec_advance(int32_t* __restrict__ pos, int max_seq,
                                       uint32_t* __restrict__ status) {
  if (threadIdx.x == 0) {
    const int p = *pos;
    if (p + 1 < max_seq) *pos = p + 1;
    else *status |= 1u;
  }
}
