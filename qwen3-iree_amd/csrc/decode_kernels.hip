// gfx950 kernels for the rest of the Qwen3-0.6B decode step, built around the
// Q8_0 GEMV engine of q8_device.h, in two forms that compute the same values
// with the same operations (shared code in decode_device.h):
//
// Launch per phase: one layer (model/qwen3_full.mlir:751-864 with
// @attention_block_decode_static 591-748) is five launches,
//   dec_qkv          rms_norm(h, attn_norm) fused into the q/k/v GEMVs
//   dec_attention    q/k head norms + RoPE, the new k/v written to the flat
//                    KV cache, split-K GQA attention (8 kv heads x 32
//                    position splits, 4 splits merged per workgroup)
//   dec_o_res        the 8 partials per head merged, attn_o GEMV + residual
//   dec_gu_swiglu    rms_norm(res, ffn_norm) fused into gate_up; each wave
//                    computes a gate quad and the matching up quad and applies
//                    SwiGLU in its epilogue
//   dec_down_res     ffn_down GEMV + residual add
// plus dec_embed (token row gather), dec_vocab_argmax (final rms_norm fused
// into the vocab GEMV + argmax) and dec_finalize (token, position).
//
// Single launch: dec_step runs the whole step in one launch of 448
// workgroups, two per CU and all resident at once, phases handing activations
// over through tagged 8-byte words instead of kernel boundaries (see its
// comment).
//
// Numerics follow the reference op by op: f16 tensors between ops, f32 in
// reductions and transcendental math, RNE to f16.  Normalisation multiplies by
// 1/rms where the reference divides by rms (one f32 rounding apart).
#include "decode_device.h"

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
        rmsnorm_gemv_x<false>(h, norm_w, xr[0]);
        store_gemv_x(xr[0], xn);
      },
      [&](int row, float acc) { y[row] = f32_to_f16_bits(acc); });
}

// Attention for kv head g = block / 8 and split group sg = block % 8 (see
// attention_group): q/k/v from global memory, the partial (m, l, acc[128]) of
// each query head to part[head][sg] (the attn_o kernel merges the 8 groups).
extern "C" __global__ __launch_bounds__(256) void dec_attention(
    const uint16_t* __restrict__ q_raw, const uint16_t* __restrict__ k_raw,
    const uint16_t* __restrict__ v_raw, const uint16_t* __restrict__ qn_w,
    const uint16_t* __restrict__ kn_w, const int32_t* __restrict__ pos_ptr, int max_seq,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache, float* __restrict__ part,
    uint16_t* __restrict__ q_roped) {
  __shared__ AttnLds lds;
  __shared__ __attribute__((aligned(16))) uint8_t kv[kAttnWaves][kKvPrefetchBytes];
  const int g = blockIdx.x / kAttnGroups;
  const int sg = blockIdx.x % kAttnGroups;
  const int lane = threadIdx.x & 63;
  const int pos_raw = *pos_ptr;
  float cs[2], sn[2];
  rope_angles(pos_raw < 0 ? 0 : (pos_raw >= max_seq ? max_seq - 1 : pos_raw), cs, sn);
  attention_group(
      lds, g, sg, pos_raw, cs, sn, max_seq, qn_w, kn_w, k_cache, v_cache, q_roped,
      kv[threadIdx.x >> 6], false, [] {},
      [&](uint32_t (&xw)[3], uint32_t& v_new) {
        xw[0] = load_global(reinterpret_cast<const uint32_t*>(q_raw + (2 * g) * kHeadDim) + lane);
        xw[1] = load_global(reinterpret_cast<const uint32_t*>(q_raw + (2 * g + 1) * kHeadDim) + lane);
        xw[2] = load_global(reinterpret_cast<const uint32_t*>(k_raw + g * kHeadDim) + lane);
        v_new = load_global(reinterpret_cast<const uint32_t*>(v_raw + g * kHeadDim) + lane);
      },
      [&](int hh, float M, float L, float a0, float a1) {
        float* dst = part + ((size_t)(2 * g + hh) * kAttnGroups + sg) * kPartStride;
        if (lane == 0) {
          dst[0] = M;
          dst[1] = L;
        }
        reinterpret_cast<float2*>(dst + 4)[lane] = float2{a0, a1};
      });
}

// attn = the merged attention output: head h, dim d =
// sum_g w_g acc_g[d] / sum_g w_g l_g over the 8 partials g of head h, w_g =
// 2^(m_g - max m) (m in base-2 units); then res = h + f16(W_o[layer] . attn)
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
        float mg[kAttnGroups], lg[kAttnGroups], wg[kAttnGroups], L;
#pragma unroll
        for (int gi = 0; gi < kAttnGroups; ++gi) {
          mg[gi] = ml[gi].x;
          lg[gi] = ml[gi].y;
        }
        merge_weights(mg, lg, wg, L);
        float a[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          // copy the elements out first: __builtin_bit_cast of a vector
          // element lvalue reads element 0 with this compiler
          float accg[kAttnGroups];
#pragma unroll
          for (int gi = 0; gi < kAttnGroups; ++gi) {
            const uint32_t bits = av[gi][e >> 2][e & 3];
            accg[gi] = __builtin_bit_cast(float, bits);
          }
          a[e] = merge_dim(accg, wg);
        }
        const u32x4 packed = {pack_f16x2(a[0] / L, a[1] / L), pack_f16x2(a[2] / L, a[3] / L),
                              pack_f16x2(a[4] / L, a[5] / L), pack_f16x2(a[6] / L, a[7] / L)};
        reinterpret_cast<u32x4*>(attn)[t] = packed;
        if (blockIdx.x == 0) reinterpret_cast<u32x4*>(attn_out)[t] = packed;
        __syncthreads();
        lds_x_cols<2>(attn, xr);  // x from the merged vector in LDS
      });
  res[row] = residual_f16(h_row, acc);
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
  rmsnorm_gemv_x<false>(res, norm_w, xr[0]);
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
  h_out[row] = residual_f16(r_row, acc);
}

// logits = W_out . rms_norm(h, output_norm) (qwen3_full.mlir:1456-1467) with
// the fused argmax into ws (see vocab_body_x).  xn receives the normalised h.
extern "C" __global__ __launch_bounds__(256) void dec_vocab_argmax(
    const uint16_t* __restrict__ W, const uint16_t* __restrict__ h,
    const uint16_t* __restrict__ norm_w, uint16_t* __restrict__ logits, uint8_t* __restrict__ ws,
    uint16_t* __restrict__ xn) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[kHidden];
  __shared__ float red[4];
  vocab_body_x<VOCAB_NT_LOADS != 0, true>(
      W,
      [&](int li, u32x4 (&xr)[8]) {
        const int t = threadIdx.x;
        const uint2 x = rmsnorm_wg(load_global(reinterpret_cast<const uint2*>(h) + t),
                                   norm_weights4(norm_w), red);
        reinterpret_cast<uint2*>(xs)[t] = x;
        if (blockIdx.x == 0) reinterpret_cast<uint2*>(xn)[t] = x;
        __syncthreads();
#pragma unroll
        for (int m = 0; m < 8; ++m) xr[m] = *reinterpret_cast<const u32x4*>(xs + 128 * m + 8 * li);
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

// Zeroes n words of a decode scratch (graph-capture safe: a kernel).
extern "C" __global__ __launch_bounds__(256) void dec_scratch_clear(uint32_t* __restrict__ p,
                                                                   uint32_t n) {
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < n; i += gridDim.x * 256u) p[i] = 0u;
}

// ======================================================= single launch ====
//
// dec_step: the whole decode step in one launch of kStepWgs = 448 workgroups
// x 256 threads, two per CU, all resident at once (the launcher checks the
// occupancy; there is no grid barrier, and every wait is bounded).  Work
// moves between workgroups as tagged words: a 64-bit word holds 32 bits of
// data (an f16 pair or an f32) and a 32-bit tag naming (step, layer, phase); a
// producer stores the word with one agent-scope atomic store, a consumer polls
// it with agent-scope atomic loads until the tag matches.  A word is its own
// flag, so no fence, counter or barrier is needed between workgroups.
//
// Each workgroup keeps one role for the whole step: one phase per layer (or
// two that lie far apart), so it requests the weights of its next phase
// straight into LDS (global_load_lds) right after finishing the current one,
// a layer (or most of one) ahead of use.  The weights have landed long before
// the phase's input arrives, and a wave's in-order load queue holds no weight
// load ahead of a poll whose answer is on the critical path.  Roles:
//   AD  0..255    A: q/k/v quad 4 wg + w: rms_norm(h) (h = the embedding row
//                 for layer 0, else the previous layer's H words), GEMV -> Q,
//                 K, V words.  D on workgroups 0..191: gate/up quad pair
//                 4 wg + w + SwiGLU -> ACT words.  Right after A the D weights
//                 of this layer and the A weights of the next are requested.
//   B   256..319  attention for kv head b % 8, split group b / 8 (b = wg -
//                 256: a head's 8 groups on one XCD, wg mod 8; attention_group,
//                 q/k/v from the tagged words) -> PART; split group 0 then
//                 merges its kv head's 8 partials of both query heads -> ATT
//                 words; then the next layer's first cache chunk is requested
//                 into LDS.
//   CE  320..447  C: attn_o + residual, row quads 2 c, 2 c + 1 (c = wg - 320),
//                 one 1024-column chunk per wave, summed in LDS -> RES words;
//                 then E: ffn_down + residual over the same two row quads,
//                 the 3072 columns in three chunks over the waves -> H words.
// Every row is computed with the per-phase kernels' operations in their order
// (same device functions), so both step modes give the same bits.  Then the
// vocab GEMV over all 448 workgroups (each publishes its best key as two
// words), and workgroup 0 reduces the 448 keys: token, optional output slot,
// position advance, sequence number.  Layer-indexed words alternate between
// two buffers by layer parity (a word of layer l is rewritten at layer l + 2,
// after every reader of it has published something the writer waited for).
// Every wait is bounded: on timeout a workgroup sets status bit 1 and an abort
// word, and every waiting workgroup gives up.
namespace {

constexpr int kStepWgs = 448;
constexpr int kAdBase = 0, kDCount = 192;  // A on all 256, D on the first 192
constexpr int kBBase = 256;                // 64 attention workgroups
constexpr int kCBase = 320;                // 128 attn_o + ffn_down workgroups
// The vocab GEMV runs on the first kVocabWgs workgroups.
#ifndef DEC_VOCAB_WGS
#define DEC_VOCAB_WGS 448
#endif
constexpr int kVocabWgs = DEC_VOCAB_WGS;
// Vocab batches (4 rows) each wave stages into LDS before the last layer's h
// arrives, on top of the two it loads into registers.
#ifndef DEC_VOCAB_PRE
#define DEC_VOCAB_PRE 2
#endif
constexpr int kVocabPre = DEC_VOCAB_PRE;
// Workgroups 0..255 hold the first slot of every CU and finish their vocab
// rows well before 256..447, which share CUs with them: each of their waves
// takes kVocabHeavy16 / 16 times the rows of a later wave.
#ifndef DEC_VOCAB_HEAVY16
#define DEC_VOCAB_HEAVY16 24
#endif
constexpr int kVocabHeavy16 = DEC_VOCAB_HEAVY16;
// Vectors that every (or nearly every) workgroup waits for -- h, the
// attention output, the attn_o + residual output, the SwiGLU output -- are
// published in kRep replicas and workgroup w polls replica w % kRep: with one
// copy, hundreds of workgroups polling the same few cache lines queue at the
// same memory channels.
constexpr int kRep = 4;
constexpr int kNH = 512, kNAtt = 1024, kNRes = 512, kNAct = 1536;  // words per replica
// tagged-word map (u64 words) per layer parity
constexpr int kWH = 0;                                     // kRep x 512: h (E output)
constexpr int kWQ = kWH + kRep * kNH;                      // 1024: q row pairs
constexpr int kWK = kWQ + 1024;                            // 512
constexpr int kWV = kWK + 512;                             // 512
constexpr int kWPart = kWV + 512;                          // 16 x 8 x 130
constexpr int kWAtt = kWPart + kQHeads * kAttnGroups * 130;  // kRep x 1024
constexpr int kWRes = kWAtt + kRep * kNAtt;                // kRep x 512
constexpr int kWAct = kWRes + kRep * kNRes;                // kRep x 1536
constexpr int kWParity = kWAct + kRep * kNAct;
constexpr int kWArg = 2 * kWParity;                        // 2 per workgroup
constexpr int kWTotal = kWArg + 2 * kStepWgs;
// phases in a tag
constexpr int kPhQKV = 0, kPhPart = 1, kPhAtt = 2, kPhRes = 3, kPhAct = 4, kPhH = 5, kPhArg = 6;

struct StepParams {
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
  uint16_t* k_cache;
  uint16_t* v_cache;
  const int32_t* token_in;  // input token (device)
  int32_t* token_out;       // argmax written here (head only)
  int32_t* pos;
  uint16_t* logits;         // may be null
  int32_t* out;             // extra copy of the token, may be null
  uint64_t* words;          // kWTotal tagged words
  uint32_t* seq;            // step sequence number (persists across launches)
  uint32_t* last_started;   // sequence number of the launch whose last workgroup started
  uint32_t* status;
  uint16_t* on_out;         // the final rms_norm(h, output_norm) (f16[1024])
  uint32_t* stamps;         // timestamp build only (DEC_STEP_STAMPS): per-phase clock reads
  int max_seq;
  int advance;
  int head;                 // 0: no vocab / argmax (a prompt step); pos still advances
  uint32_t spin_limit;      // poll rounds after which a wait gives up (2^20 by default);
                            // 0: workgroup 0 gives up at its start (the host forcing the
                            // abort path, for tests)
};

__device__ __forceinline__ uint32_t step_tag(uint32_t seq, int layer, int phase) {
  return (seq << 8) | (uint32_t)(1 + (layer + 1) * 8 + phase);
}

__device__ __forceinline__ void put_word(uint64_t* p, uint32_t data, uint32_t tag) {
  __hip_atomic_store(p, ((uint64_t)tag << 32) | data, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t get_word(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// *p = v unless *p already holds v or a newer sequence number (compared
// modulo 2^32).  The workgroup that gives up moves the word to its own
// number, so the next launch tags its words with a number no word of the
// aborted launch carries.  (A workgroup that starts after the give-up reads
// the status word after the sequence word, in the same cache line, and the
// status bit is set before the sequence word moves: it sees the bit and
// returns at its start, so no workgroup runs with a newer number.)
__device__ __forceinline__ void advance_seq_word(uint32_t* p, uint32_t v) {
  uint32_t cur = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  while ((int32_t)(v - cur) > 0 &&
         !__hip_atomic_compare_exchange_strong(p, &cur, v, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT)) {
  }
}

// A wait that cannot complete: status bit 1 (sticky until the host clears
// it) makes every other waiter stop at its next check and every later launch
// on this scratch return at its start; then the sequence word moves to this
// workgroup's number.
__device__ __forceinline__ void give_up(uint32_t* status, uint32_t* seq_word, uint32_t seq) {
  __hip_atomic_fetch_or(status, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  advance_seq_word(seq_word, seq);
}

struct Waiter {
  const uint32_t* last_started;
  uint32_t* status;
  uint32_t* seq_word;  // the step sequence number in the scratch
  uint32_t seq;
  uint32_t spin_limit;
  int* s_abort;  // LDS flag of the workgroup

  static constexpr int kMax = 9;  // words per thread: n <= 2304

  // The first round of a wait: this thread's words (i = threadIdx.x + 256 k)
  // requested at once.  Issued before a phase's own weight loads, the round
  // trip overlaps them (vector loads complete in issue order, so a poll
  // issued after them could not return before them).
  // (Rounds that every thread has are issued unconditionally: the compiler
  // then waits for them precisely instead of draining all memory operations
  // after a per-lane branch.)
  template <class Src>
  __device__ __forceinline__ void poll_begin(int n, Src src, uint64_t (&w)[kMax]) const {
    const int t = threadIdx.x;
#pragma unroll
    for (int k = 0; k < kMax; ++k)
      if (256 * (k + 1) <= n || t + 256 * k < n) w[k] = get_word(src(t + 256 * k));
  }

  // Every thread of the workgroup calls this with the same arguments, after
  // poll_begin: the data halves of words src(0..n-1), once each carries tag
  // `tag`, land in dst[0, n).  Only words not ready yet are requested again,
  // so a wait costs one round trip once the data is there.  Returns false (in
  // every thread) when the step was aborted.
  template <class Src>
  __device__ __forceinline__ bool poll_finish(int n, uint32_t tag, uint32_t* __restrict__ dst,
                                              Src src, uint64_t (&w)[kMax]) const {
    const int t = threadIdx.x;
    bool ok = true;
    uint32_t spins = 0;
    while (true) {
      bool pending = false;
#pragma unroll
      for (int k = 0; k < kMax; ++k)
        if (t + 256 * k < n && (uint32_t)(w[k] >> 32) != tag) pending = true;
      if (!pending) break;
      ++spins;
      // another workgroup gave up (it already moved the sequence word past
      // this launch's number)
      if ((spins & 31u) == 0u &&
          (__hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 2u) != 0) {
        ok = false;
        break;
      }
      // ~1 ms into a wait and not every workgroup of the launch has started:
      // the grid is not resident at once (a kernel on another stream holds
      // CUs), so the started ones could wait forever for the others
      if ((spins & 1023u) == 0u &&
          __hip_atomic_load(last_started, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != seq)
        spins = spin_limit + 1u;
      if (spins > spin_limit) {
        give_up(status, seq_word, seq);
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int k = 0; k < kMax; ++k)
        if (t + 256 * k < n && (uint32_t)(w[k] >> 32) != tag) w[k] = get_word(src(t + 256 * k));
    }
    // every thread is past its previous reads of dst (a phase may read the
    // last vector right up to its next wait) before any overwrites it
    __syncthreads();
    if (ok) {
#pragma unroll
      for (int k = 0; k < kMax; ++k)
        if (t + 256 * k < n) dst[t + 256 * k] = (uint32_t)w[k];
    } else {
      *s_abort = 1;
    }
    __syncthreads();
    if (*s_abort != 0) {
      // the workgroup is about to end: its LDS copies in flight land first
      wait_vm<0>();
      return false;
    }
    return true;
  }

  // poll_begin + poll_finish.
  template <class Src>
  __device__ __forceinline__ bool wait_map(int n, uint32_t tag, uint32_t* __restrict__ dst,
                                           Src src) const {
    uint64_t w[kMax];
    poll_begin(n, src, w);
    return poll_finish(n, tag, dst, src, w);
  }

  __device__ __forceinline__ bool wait(const uint64_t* __restrict__ src, int n, uint32_t tag,
                                       uint32_t* __restrict__ dst) const {
    return wait_map(n, tag, dst, [=](int i) { return src + i; });
  }
};

// Row sums of a quad (rows q4, q4+1, q4+2, q4+3; row r's sum in lanes
// 16(r - q4)..) published as two f16-pair words, 2 quad and 2 quad + 1, in
// REP replicas `stride` words apart: lanes 0..REP-1 write the first word,
// lanes 32..32+REP-1 the second.  f(acc) maps a row sum to its f16 bits.
template <int REP, class F>
__device__ __forceinline__ void put_quad(uint64_t* __restrict__ words, int stride, int quad,
                                         float acc, uint32_t tag, F f) {
  const int lane = threadIdx.x & 63;
  const uint32_t mine = f(acc, 4 * quad + (lane >> 4));
  const uint32_t next = __shfl(mine, (lane + 16) & 63, 64);
  if ((lane & 31) < REP)
    put_word(words + (lane & 31) * stride + 2 * quad + (lane >> 5), mine | (next << 16), tag);
}

// u64 max over the 64 lanes of a wave.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)v, d, 64);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), d, 64);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    v = o > v ? o : v;
  }
  return v;
}

// Timestamp build (-DDEC_STEP_STAMPS=1, for measuring where a step's time
// goes; the product build compiles none of this): thread 0 of the workgroups
// listed in stamp_slot reads the 100 MHz real-time counter at the phase
// boundaries below into LDS (its low 32 bits: differences stay exact for 42
// s), [layer 0..27, or 28 for the vocab phase][point], and copies them to
// P.stamps[slot][29][21] (u32) at the end.
//   per layer: 0 layer start, 1 h ready (A), 13 x normalised (A), 2 q/k/v
//   published, 15 gate/up weights requested (D), 9 residual ready (D), 10
//   SwiGLU published, 3 q/k/v ready (B), inside B's attention_group: 16
//   head norms + RoPE done, 17 score MFMAs issued, 18 softmax done, 19
//   chunk loop done, 20 the four waves' results in LDS (after the
//   barrier), then 4 partial published, 5 partials ready (merge), 6 attention output
//   published, 14 h rows ready (C), 7 attention output ready (C), 8 residual
//   published, 11 SwiGLU ready (E), 12 h published
//   vocab: 0 start, 1 h ready, 2 key published, 3 keys ready (wg 0), 4 token
#ifndef DEC_STEP_STAMPS
#define DEC_STEP_STAMPS 0
#endif
constexpr int kStampWgs[16] = {0,   1,   100, 191, 192, 255, 256, 257,
                               264, 319, 320, 321, 383, 384, 446, 447};
constexpr int kStampPoints = 21;
__device__ __forceinline__ int stamp_slot(int wg) {
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (kStampWgs[i] == wg) return i;
  return -1;
}

constexpr int kVecWords = 2 * kAttnGroups * 130;  // 2080: the largest polled vector
// Weight prefetches sleep 64 kPace* cycles between 1 KiB pieces, each set
// spread over the time its role has before the weights are needed (the gate/up
// weights are requested right after A, the next q/k/v weights right after D,
// the next attn_o weights right after C, the next ffn_down weights right after
// E, the next cache chunk right after attention).  Unpaced bursts from
// hundreds of workgroups fill the memory queues and delay the hand-offs in
// flight; paced too slowly, a prefetch still being issued delays its wave's
// next poll.  Measured at context 1024 (us/token, 539 with E at 32): A 16 / 48
// 550 / 592, D 24 / 40 551 / 600, C 8 / 16 / 40 554 / 557 / 568, E 12-24
// 535-536, E 48 653, the cache chunk 4 / 16 unchanged; with E at 16 (536):
// A 28 / 36 539 / 552, D 28 / 36 547 / 561, C 28 / 36 539 / 554; with the
// gate/up touch and D at 30 (518): C 26 / 28 / 30 / 34 519 / 517 / 516 / 531,
// E 12 / 20 518, A 30 522.  Again with the cache rows copied whole and the
// kernel arguments preloaded (508.5 / 511.4 as below): D 26 / 34 526.8 /
// 542.6, A 28 / 36 515.1 / 524.4, C 26 / 34 515.3 / 529.5, E 12 / 20 512.2 /
// 510.9.
#ifndef DEC_PACE_A
#define DEC_PACE_A 32
#endif
#ifndef DEC_PACE_D
#define DEC_PACE_D 30
#endif
#ifndef DEC_PACE_C
#define DEC_PACE_C 30
#endif
#ifndef DEC_PACE_E
#define DEC_PACE_E 16
#endif
#ifndef DEC_PACE_KV
#define DEC_PACE_KV 8
#endif
constexpr int kPaceA = DEC_PACE_A, kPaceD = DEC_PACE_D, kPaceC = DEC_PACE_C, kPaceE = DEC_PACE_E,
              kPaceKV = DEC_PACE_KV;

// LDS of one workgroup, by role (a union: each workgroup uses one member).
// Weight buffers are per wave and filled by that wave's global_load_lds.
struct StepLdsAd {
  uint8_t wa[4][QuadShape<1>::LDS_BYTES];     // the q/k/v quad of each wave
  uint8_t wd[4][2][QuadShape<1>::LDS_BYTES];  // its gate quad and up quad
  uint8_t sink[4][256];                       // kv_touch's never-read landing area
};
struct StepLdsB {
  uint8_t kv[kAttnWaves][kKvPrefetchBytes];  // each wave's first cache chunk
  AttnLds attn;
};
struct StepLdsCE {
  uint8_t wc[4][QuadShape<1>::LDS_BYTES];     // C: each wave's chunk of its quad
  uint8_t we[4][2][QuadShape<1>::LDS_BYTES];  // E: chunks 0, 1 (even waves) or 2 (odd)
  float c_part[2][128];                       // C: the chunk sums of the two quads
  float e_part[2][64];                        // E: chunk 2's lane sums of the two quads
};
union StepLds {
  StepLdsAd ad;
  StepLdsB b;
  StepLdsCE ce;
};
// two workgroups per CU: 80 KiB each (the vocab phase adds 160 bytes)
static_assert(sizeof(StepLds) + 4 * kVecWords <= 81920 - 256, "dec_step LDS");
static_assert(sizeof(StepLds) >= 4 * kVocabPre * 8192, "vocab stage area");
// the fewest batches a wave owns (a wave of workgroups 256 .. kVocabWgs - 1)
static_assert(kVocabWgs > 256 || kVocabHeavy16 == 16,
              "the weighted split assumes more than 256 vocab workgroups");
static_assert(kVocab / 4 * 16 / (4 * (256 * kVocabHeavy16 + (kVocabWgs - 256) * 16)) - 1 >=
                  kVocabPre + 2,
              "vocab batches per wave");
static_assert(kKvHeads == 8 && kBBase % 8 == 0, "one kv head's attention workgroups per XCD (wg mod 8)");

}  // namespace

extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void dec_step(StepParams P) {
  __shared__ __attribute__((aligned(16))) StepLds S;
  __shared__ __attribute__((aligned(16))) uint32_t vec[kVecWords];  // polled words' data
  __shared__ int s_abort;
  __shared__ float s_red[4];  // rms_norm: the waves' sums
  const int wg = blockIdx.x;
  const int rep = wg % kRep;  // the replica this workgroup polls
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  if (t == 0) s_abort = 0;
#if DEC_STEP_STAMPS
  __shared__ uint32_t s_stamp[kLayers + 1][kStampPoints];
  const int stamp_i = stamp_slot(wg);
  if (t == 0)
    for (int i = 0; i < (kLayers + 1) * kStampPoints; ++i) (&s_stamp[0][0])[i] = 0;
#define STAMP(layer, k)                                                                    \
  do {                                                                                     \
    if (t == 0 && stamp_i >= 0)                                                            \
      s_stamp[layer][k] = (uint32_t)__builtin_amdgcn_s_memrealtime();                       \
  } while (0)
#else
#define STAMP(layer, k) \
  do {                  \
  } while (0)
#endif

  // The sequence number, then the status word (same cache line): a step of
  // this scratch gave up (status bit 1, until the host clears it) and this
  // launch does nothing, so a step queued behind an aborted one neither
  // advances the position nor writes a token.  A thread that reads a number a
  // give-up has already advanced also sees the bit (set before the number
  // moves), so a workgroup that runs has one number in every thread.
  const uint32_t seq = __hip_atomic_load(P.seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
  const uint32_t status_in = __hip_atomic_load(P.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();  // s_abort is 0 in every thread's view
  if ((status_in & 2u) != 0u) s_abort = 1;
  if (P.spin_limit == 0u && wg == 0 && t == 0 && (status_in & 2u) == 0u) {
    give_up(P.status, P.seq, seq);  // the host forces a give-up
    s_abort = 1;
  }
  // Workgroups start in index order: the last one marks the launch as
  // resident (a wait that finds another number after ~1 ms knows the grid
  // is not resident at once).
  if (wg == kStepWgs - 1 && t == 0)
    __hip_atomic_store(P.last_started, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int pos_raw = *P.pos;
  int tok = *P.token_in;
  tok = (tok < 0 || tok >= kVocab) ? 0 : tok;
  const uint16_t* emb = P.token_embd + (size_t)tok * kHidden;
  const Waiter W{P.last_started, P.status, P.seq, seq, P.spin_limit, &s_abort};
  const int pos_c = pos_raw < 0 ? 0 : (pos_raw >= P.max_seq ? P.max_seq - 1 : pos_raw);
  __syncthreads();
  if (s_abort) return;

  if (wg < kBBase) {
    // ================= AD: q/k/v of every layer; gate/up on 0..191 =================
    const int quad = 4 * wg + wave;  // 0..1023: q quads, then k, then v
    const uint8_t* wsel = quad < 512 ? P.wq : (quad < 768 ? P.wk : P.wv);
    const int n = quad < 512 ? 2048 : 1024;
    const int qd = quad < 512 ? quad : (quad < 768 ? quad - 512 : quad - 768);
    const int64_t bpl = (int64_t)n * (kHidden / 32 * 34);
    const bool has_d = wg < kDCount;
    const int b = 4 * wg + wave;  // gate/up quad pair (has_d)
    constexpr int64_t bpl_gu = (int64_t)(2 * kFfn) * (kHidden / 32 * 34);
    uint8_t* const la = S.ad.wa[wave];
    // kv_touch task of this wave: head wg mod 8, task (wg / 8) * 4 + wave of
    // that head's 128 = split (task mod 32), chunk 1 + task / 32 (1-4)
    const int touch_task = (wg >> 3) * 4 + wave;
    const int n_split_chunks = ((pos_c + 1 + kAttnSplits - 1) / kAttnSplits + 31) / 32;
    uint8_t* const lg = S.ad.wd[wave][0];
    uint8_t* const lu = S.ad.wd[wave][1];
    q8_quad_prefetch<1>(wsel, n, qd, la);
    for (int layer = 0; layer < kLayers; ++layer) {
      uint64_t* cur = P.words + (layer & 1) * kWParity;
      const uint64_t* prev = P.words + ((layer & 1) ^ 1) * kWParity;
      STAMP(layer, 0);
      // ---- A ----
      u32x4 xr[1][8];
      const uint16_t* an = P.attn_norm + layer * kHidden;
      // the norm weights first: the polled words come back after them (in
      // order), so once h has arrived its norm never waits on these loads
      const uint2 aw4 = norm_weights4(an);
      uint2 h4;
      if (layer == 0) {
        h4 = load_global(reinterpret_cast<const uint2*>(emb) + t);
      } else {
        const auto h_src = [=](int i) { return prev + kWH + rep * kNH + i; };
        uint64_t hp[Waiter::kMax];
        W.poll_begin(512, h_src, hp);
        if (!W.poll_finish(512, step_tag(seq, layer - 1, kPhH), vec, h_src, hp)) return;
        STAMP(layer, 1);
        h4 = reinterpret_cast<const uint2*>(vec)[t];
      }
      norm_to_vec(h4, aw4, vec, s_red, xr[0]);
      STAMP(layer, 13);
      const float acc = q8_quad_dot<1>(la, xr);
      uint64_t* dst = quad < 512 ? cur + kWQ : (quad < 768 ? cur + kWK : cur + kWV);
      put_quad<1>(dst, 0, qd, acc, step_tag(seq, layer, kPhQKV),
                  [](float a, int) { return (uint32_t)f32_to_f16_bits(a); });
      STAMP(layer, 2);
      // Splits of more than one chunk (context past 1024): this layer's cache
      // chunks 1-4 of every split into the L2 of the XCD whose attention
      // workgroups read them (head wg mod 8), one chunk per wave, about 2 us
      // before the attention copies them (which then hit L2 instead of HBM):
      // us/token at context 2048 636.6 -> 619.1, 4096 826.7 -> 761.1, 8192
      // 1158.6 -> 1094.6, 16384 1763.7 -> 1714.0, 1024 unchanged.  Touching
      // the later chunks too (two tasks per wave) measured slower (8192:
      // 1123.0, 16384: 1749.1): L2 holds only so much beside the weights.
      if (touch_task < 32 * (n_split_chunks - 1)) {
        const SplitRange tr = split_range(touch_task & 31, pos_c);
        kv_touch(S.ad.sink[wave], P.k_cache + (int64_t)layer * P.max_seq * (kKvHeads * kHeadDim),
                 P.v_cache + (int64_t)layer * P.max_seq * (kKvHeads * kHeadDim), wg & 7,
                 tr.start + 32 * (1 + (touch_task >> 5)), tr.last);
      }
      // The A-only workgroups (idle until the next layer's h) bring the
      // gate/up quads of the 24 D workgroups on their XCD (wg mod 8) into its
      // L2, one dword per 128-byte line into the never-read sink, while the D
      // workgroups' own paced copies into LDS (below) follow: us/token at
      // context 1024 535.7 -> 518.6 (with the D pace 32 -> 30; with the touch
      // the D pace measured 20 / 24 / 26 / 28 / 32 / 36: 542 / 539 / 535 / 522
      // / 528 / 568).
      if (!has_d) {
        const int k = (wg - kDCount) >> 3;  // this one's rank among the 8 on its XCD
        const uint8_t* wl = P.wgu + layer * bpl_gu;
        for (int i = 0; i < 6; ++i) {
          const int tq = wave * 6 + i;  // D workgroup tq / 8 of 3, its wave, gate or up
          const int j = (wg & 7) + 8 * (3 * k + tq / 8);
          const int b = 4 * j + ((tq >> 1) & 3);
          const int quad = (tq & 1) ? kFfn / 4 + b : b;
          // a quad is 4 x 1088 = 4352 bytes: lines 0..33
          const uint8_t* src =
              wl + (size_t)quad * (4 * (kHidden / 32 * 34)) + 128 * (lane < 34 ? lane : 33);
          __builtin_amdgcn_global_load_lds((const GLOBAL_AS void*)src, (LDS_AS void*)S.ad.sink[wave],
                                           4, 0, 0);
          __builtin_amdgcn_s_sleep(16);
        }
      }
      // this layer's gate/up weights (the next layer's q/k/v weights follow D)
      if (has_d) {
        const uint8_t* wl = P.wgu + layer * bpl_gu;
        q8_quad_prefetch<1, kPaceD>(wl, 2 * kFfn, b, lg);
        q8_quad_prefetch<1, kPaceD>(wl, 2 * kFfn, kFfn / 4 + b, lu);
        STAMP(layer, 15);
      }
      // ---- D: gate/up + SwiGLU ----
      if (has_d) {
        const uint2 dw4 = norm_weights4(P.ffn_norm + layer * kHidden);  // before the wait
        if (!W.wait(cur + kWRes + rep * kNRes, 512, step_tag(seq, layer, kPhRes), vec)) return;
        STAMP(layer, 9);
        u32x4 xd[1][8];
        norm_to_vec(reinterpret_cast<const uint2*>(vec)[t], dw4, vec, s_red, xd[0]);
        const float ag = q8_quad_dot<1>(lg, xd);
        const float au = q8_quad_dot<1>(lu, xd);
        const uint32_t act = swiglu_f16(ag, au);
        const uint32_t next = __shfl(act, (lane + 16) & 63, 64);
        if ((lane & 31) < kRep)
          put_word(cur + kWAct + (lane & 31) * kNAct + 2 * b + (lane >> 5), act | (next << 16),
                   step_tag(seq, layer, kPhAct));
        STAMP(layer, 10);
      }
      if (layer + 1 < kLayers) q8_quad_prefetch<1, kPaceA>(wsel + (layer + 1) * bpl, n, qd, la);
    }
  } else if (wg < kCBase) {
    // ================= B: attention (+ merge on split group 0) =================
    // kv head g's split groups, its merge (split group 0) among them, on
    // workgroups wg = g (mod 8): the partials' hand-off stays within one XCD
    // (one L2)
    const int bw = wg - kBBase;
    const int g = bw % kKvHeads;
    const int sg = bw / kKvHeads;
    uint8_t* const kv_mine = S.b.kv[wave];
    // the first chunk of each wave's split stays in LDS: requested for layer 0
    // now, for layer l + 1 as soon as layer l's attention (and merge) is done
    const SplitRange my_split = split_range(sg * kAttnWaves + wave, pos_c);
    kv_prefetch(kv_mine, P.k_cache, P.v_cache, g, my_split);
    float rope_cs[2], rope_sn[2];  // the position's RoPE angles, for every layer
    rope_angles(pos_c, rope_cs, rope_sn);
    for (int layer = 0; layer < kLayers; ++layer) {
      uint64_t* cur = P.words + (layer & 1) * kWParity;
      STAMP(layer, 0);
      const int64_t cache_layer = (int64_t)layer * P.max_seq * (kKvHeads * kHeadDim);
      bool ok = true;
      const uint32_t tq = step_tag(seq, layer, kPhQKV);
      // q heads 2g, 2g+1 (words 128g..), k head g, v head g (words 64g..)
      const auto qkv_src = [=](int i) {
        return i < 128 ? cur + kWQ + 128 * g + i
                       : (i < 192 ? cur + kWK + 64 * g + (i - 128) : cur + kWV + 64 * g + (i - 192));
      };
      uint64_t qkv_poll[Waiter::kMax];
      attention_group(
          S.b.attn, g, sg, pos_raw, rope_cs, rope_sn, P.max_seq, P.q_norm + layer * kHeadDim,
          P.k_norm + layer * kHeadDim, P.k_cache + cache_layer, P.v_cache + cache_layer, nullptr,
          kv_mine, true, [&] { W.poll_begin(256, qkv_src, qkv_poll); },
          [&](uint32_t (&xw)[3], uint32_t& v_new) {
            ok = W.poll_finish(256, tq, vec, qkv_src, qkv_poll);
            STAMP(layer, 3);
            xw[0] = vec[lane];
            xw[1] = vec[64 + lane];
            xw[2] = vec[128 + lane];
            v_new = vec[192 + lane];
          },
          [&](int hh, float M, float Ls, float a0, float a1) {
            uint64_t* d = cur + kWPart + ((2 * g + hh) * kAttnGroups + sg) * 130;
            const uint32_t tp = step_tag(seq, layer, kPhPart);
            if (lane == 0) {
              put_word(d, __builtin_bit_cast(uint32_t, M), tp);
              put_word(d + 1, __builtin_bit_cast(uint32_t, Ls), tp);
            }
            put_word(d + 2 + 2 * lane, __builtin_bit_cast(uint32_t, a0), tp);
            put_word(d + 3 + 2 * lane, __builtin_bit_cast(uint32_t, a1), tp);
          },
#if DEC_STEP_STAMPS
          // the timestamp build's points inside the attention (kept in place)
          [&](int k) {
            __builtin_amdgcn_sched_barrier(0);
            STAMP(layer, k);
            __builtin_amdgcn_sched_barrier(0);
          }
#else
          NoStamp()
#endif
      );
      if (!ok) {
        wait_vm<0>();  // attention_group's copies after the failed wait
        return;
      }
      STAMP(layer, 4);
      if (sg == 0) {
        // the 8 groups' partials of query heads 2g, 2g+1 (contiguous words)
        if (!W.wait(cur + kWPart + 2 * g * kAttnGroups * 130, 2 * kAttnGroups * 130,
                    step_tag(seq, layer, kPhPart), vec))
          return;
        STAMP(layer, 5);
        if (wave < 2) {
          const int hh = wave;
          const float* pv = reinterpret_cast<const float*>(vec) + hh * kAttnGroups * 130;
          float mg[kAttnGroups], lg[kAttnGroups], wgt[kAttnGroups], Ls;
#pragma unroll
          for (int gi = 0; gi < kAttnGroups; ++gi) {
            mg[gi] = pv[gi * 130];
            lg[gi] = pv[gi * 130 + 1];
          }
          merge_weights(mg, lg, wgt, Ls);
          float a[2];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            float accg[kAttnGroups];
#pragma unroll
            for (int gi = 0; gi < kAttnGroups; ++gi) accg[gi] = pv[gi * 130 + 2 + 2 * lane + e];
            a[e] = merge_dim(accg, wgt);
          }
          const uint32_t att = pack_f16x2(a[0] / Ls, a[1] / Ls);
#pragma unroll
          for (int r = 0; r < kRep; ++r)
            put_word(cur + kWAtt + r * kNAtt + (2 * g + hh) * 64 + lane, att,
                     step_tag(seq, layer, kPhAtt));
        }
        STAMP(layer, 6);
        __syncthreads();  // vec is reused by the next wait
      }
      if (layer + 1 < kLayers) {  // the next layer's first chunk, into this wave's LDS region
        const int64_t next = (int64_t)(layer + 1) * P.max_seq * (kKvHeads * kHeadDim);
        kv_prefetch<kPaceKV>(kv_mine, P.k_cache + next, P.v_cache + next, g, my_split);
      }
    }
  } else {
    // ================= CE: attn_o + residual, then ffn_down + residual =================
    // C: row quads 2 cw and 2 cw + 1 (waves 0-1 and 2-3), one 1024-column
    // chunk per wave, the two chunk sums added in LDS in the per-phase
    // kernel's order.  E: the same two quads of W_down, waves 2 qi (chunks 0
    // and 1) and 2 qi + 1 (chunk 2), the lane sums added in chunk order; the
    // residual of each row is the value this workgroup's C just published.
    const int cw = wg - kCBase;  // 0..127
    const int qi = wave >> 1;
    const int quad = 2 * cw + qi;  // 0..255
    const int c = wave & 1;
    constexpr int64_t bpl_o = (int64_t)kHidden * (2 * kHidden / 32 * 34);
    constexpr int64_t bpl_dn = (int64_t)kHidden * (kFfn / 32 * 34);
    uint8_t* const lwc = S.ce.wc[wave];
    uint8_t* const lwe0 = S.ce.we[wave][0];
    uint8_t* const lwe1 = S.ce.we[wave][1];
    auto prefetch_e = [&](int layer) {
      const uint8_t* wl = P.wdn + layer * bpl_dn;
      if (c == 0) {
        q8_chunk_prefetch<3, kPaceE>(wl, kHidden, quad, 0, lwe0);
        q8_chunk_prefetch<3, kPaceE>(wl, kHidden, quad, 1, lwe1);
      } else {
        q8_chunk_prefetch<3, kPaceE>(wl, kHidden, quad, 2, lwe0);
      }
    };
    q8_chunk_prefetch<2>(P.wo, kHidden, quad, c, lwc);
    prefetch_e(0);
    const int row = 4 * quad + (lane >> 4);
    for (int layer = 0; layer < kLayers; ++layer) {
      uint64_t* cur = P.words + (layer & 1) * kWParity;
      const uint64_t* prev = P.words + ((layer & 1) ^ 1) * kWParity;
      STAMP(layer, 0);
      // ---- C ----
      _Float16 h_row;
      if (layer == 0) {
        h_row = as_half(load_global_u16(emb + row));
      } else {
        // this workgroup's 8 residual rows = h words [4 cw, +4)
        if (!W.wait(prev + kWH + rep * kNH + 4 * cw, 4, step_tag(seq, layer - 1, kPhH),
                    vec + 1024))
          return;
        STAMP(layer, 14);
        h_row = as_half(reinterpret_cast<const uint16_t*>(vec + 1024)[row - 8 * cw]);
      }
      if (!W.wait(cur + kWAtt + rep * kNAtt, 1024, step_tag(seq, layer, kPhAtt), vec)) return;
      STAMP(layer, 7);
      {
        u32x4 xr[1][8];
        lds_x_cols<1>(reinterpret_cast<const uint16_t*>(vec) + 1024 * c, xr);
        S.ce.c_part[qi][lane + 64 * c] = q8_quad_lane_dot<1>(lwc, xr);
      }
      __syncthreads();
      uint16_t res_row = 0;  // this row's attn_o + residual (waves with c == 0)
      if (c == 0) {
        float acc = 0.0f;
        acc += S.ce.c_part[qi][lane];
        acc += S.ce.c_part[qi][lane + 64];
        acc = reduce_row16(acc);
        res_row = residual_f16(h_row, acc);
        put_quad<kRep>(cur + kWRes, kNRes, quad, acc, step_tag(seq, layer, kPhRes),
                       [&](float, int) { return (uint32_t)res_row; });
        STAMP(layer, 8);
      }
      if (layer + 1 < kLayers)
        q8_chunk_prefetch<2, kPaceC>(P.wo + (layer + 1) * bpl_o, kHidden, quad, c, lwc);
      // ---- E ----
      if (!W.wait(cur + kWAct + rep * kNAct, 1536, step_tag(seq, layer, kPhAct), vec)) return;
      STAMP(layer, 11);
      float e = 0.0f;
      if (c == 0) {
        u32x4 xr[1][8];
        lds_x_cols<1>(reinterpret_cast<const uint16_t*>(vec), xr);
        e += q8_quad_lane_dot<1>(lwe0, xr);
        lds_x_cols<1>(reinterpret_cast<const uint16_t*>(vec) + 1024, xr);
        e += q8_quad_lane_dot<1>(lwe1, xr);
      } else {
        u32x4 xr[1][8];
        lds_x_cols<1>(reinterpret_cast<const uint16_t*>(vec) + 2048, xr);
        S.ce.e_part[qi][lane] = q8_quad_lane_dot<1>(lwe0, xr);
      }
      __syncthreads();
      if (c == 0) {
        e += S.ce.e_part[qi][lane];
        e = reduce_row16(e);
        put_quad<kRep>(cur + kWH, kNH, quad, e, step_tag(seq, layer, kPhH),
                       [&](float a, int) { return (uint32_t)residual_f16(as_half(res_row), a); });
        STAMP(layer, 12);
      }
      if (layer + 1 < kLayers) prefetch_e(layer + 1);
    }
  }

  // ---- vocab GEMV + argmax over all workgroups ----
  const uint64_t* hfin = P.words + ((kLayers - 1) & 1) * kWParity + kWH + rep * kNH;
  const uint32_t tag_h = step_tag(seq, kLayers - 1, kPhH);
  const uint32_t tag_arg = step_tag(seq, kLayers, kPhArg);
  STAMP(kLayers, 0);
  if (P.head && wg < kVocabWgs) {
    bool ok = true;
    // The stage area is the role LDS: every wave is done with its role (and
    // its DMAs into it) before any wave stages vocab rows there.
    if constexpr (kVocabPre > 0) {
      wait_vm<0>();
      __syncthreads();
    }
    vocab_body_xp<VOCAB_NT_LOADS != 0, true, kVocabPre>(
        P.output_w,
        [&](int li, u32x4 (&xr)[8]) -> bool {
          const uint2 w4 = norm_weights4(P.output_norm);  // requested before the wait
          ok = W.wait(hfin, 512, tag_h, vec);
          STAMP(kLayers, 1);
          if (!ok) return false;  // no row is computed or stored
          uint2* v2 = reinterpret_cast<uint2*>(vec);
          const uint2 x = rmsnorm_wg(v2[t], w4, s_red);
          v2[t] = x;
          if (wg == 0) reinterpret_cast<uint2*>(P.on_out)[t] = x;
          __syncthreads();
          const uint16_t* xs = reinterpret_cast<const uint16_t*>(vec);
#pragma unroll
          for (int m = 0; m < 8; ++m)
            xr[m] = *reinterpret_cast<const u32x4*>(xs + 128 * m + 8 * li);
          return true;
        },
        P.logits, kVocab, [&](uint64_t key) {
          put_word(P.words + kWArg + 2 * wg, (uint32_t)(key >> 32), tag_arg);
          put_word(P.words + kWArg + 2 * wg + 1, (uint32_t)key, tag_arg);
        }, kVocabWgs, reinterpret_cast<uint8_t*>(&S), 256, kVocabHeavy16);
    if (!ok) return;
    STAMP(kLayers, 2);
  }

#if DEC_STEP_STAMPS
  if (t == 0 && stamp_i >= 0 && wg != 0)
    for (int i = 0; i < (kLayers + 1) * kStampPoints; ++i)
      P.stamps[stamp_i * (kLayers + 1) * kStampPoints + i] = (&s_stamp[0][0])[i];
#endif
  // ---- workgroup 0: token, position, sequence number ----
  if (wg != 0) return;
  if (P.head) {
    if (!W.wait(P.words + kWArg, 2 * kVocabWgs, tag_arg, vec)) return;
    STAMP(kLayers, 3);
    // keys of workgroups t and t + 256
    uint64_t key = t < kVocabWgs ? ((uint64_t)vec[2 * t] << 32) | vec[2 * t + 1] : 0;
    if (t + 256 < kVocabWgs) {
      const uint64_t key2 = ((uint64_t)vec[512 + 2 * t] << 32) | vec[512 + 2 * t + 1];
      key = key2 > key ? key2 : key;
    }
    key = wave_max_u64(key);
    __shared__ uint64_t s_key[4];
    if (lane == 0) s_key[wave] = key;
    __syncthreads();
    if (t == 0) {
      uint64_t k = s_key[0];
      for (int i = 1; i < 4; ++i) k = s_key[i] > k ? s_key[i] : k;
      const int32_t token = k == 0 ? -1 : (int32_t)(0xffffffffu - (uint32_t)(k & 0xffffffffu));
      *P.token_out = token;
      if (P.out != nullptr) *P.out = token;
    }
  } else if (!W.wait(hfin, 512, tag_h, vec)) {  // the last layer is done
    return;
  }
  if (t == 0) {
    if (P.advance) {
      if (pos_raw + 1 < P.max_seq) *P.pos = pos_raw + 1;
      else __hip_atomic_fetch_or(P.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __hip_atomic_store(P.seq, seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  STAMP(kLayers, 4);
#if DEC_STEP_STAMPS
  if (t == 0)
    for (int i = 0; i < (kLayers + 1) * kStampPoints; ++i)
      P.stamps[i] = (&s_stamp[0][0])[i];  // workgroup 0 is slot 0
#endif
}
