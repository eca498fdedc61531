// gfx950 kernels for batched prompt ingestion: the reference's @prefill
// (model/qwen3_full.mlir:2032-2111, one @transformer_layer_prefill per layer,
// :1731-2030) runs all prompt tokens of a layer together, so the layer
// matrices become GEMMs [n_tokens, K] x [K, N] instead of n_tokens GEMVs.
//
// Per layer (eight launches):
//   pf_rmsnorm       rms_norm(h, attn_norm) of every token row
//   pf_gemm_q8 x3    q, k, v projections (MFMA, Q8_0 weights dequantized in
//                    registers, the per-block scale applied in f32)
//   pf_qk_rope_cache per-head rms_norm of q and k, RoPE at each token's
//                    position, k and v written to their cache slots
//   pf_attention     causal GQA attention of every token over the cache
//   pf_gemm_q8       attn_o + residual
//   pf_rmsnorm       rms_norm(res, ffn_norm)
//   pf_gemm_q8       gate/up with SwiGLU in the epilogue
//   pf_gemm_q8       ffn_down + residual
// plus pf_embed (token rows) before the first layer.  The vocab GEMV + argmax
// of the last token reuses the decode kernels.
//
// Numerics follow the decode step op for op (f16 tensors between ops, f32 in
// sums, norms and transcendental math): the norms, RoPE, SwiGLU and residual
// adds are the same device functions the decode kernels call, the GEMMs form
// each Q8_0 block's 32 products exactly (int8 and f16 inputs, f32 MFMA
// accumulation) and add them into an f32 sum with the block's scale, as the
// GEMV does; only the order of the f32 additions differs.
#include "decode_device.h"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- GEMM ----
//
// Y[m, n] = sum_k X[m, k] W[n, k], W a [N, K] matrix of Q8_0 blocks (row n:
// K/32 blocks of 34 bytes, f16 scale + 32 int8).  Workgroup tile 64 (m) x 64
// (n), four waves of 32 x 32 (2 x 2 tiles of v_mfma_f32_16x16x32_f16, one
// Q8_0 block per instruction).  A stage covers 8 blocks (256 k): X rows (512
// bytes, padded to 528 in LDS so the 16 rows a fragment read touches fall in
// distinct banks) and the tile's 64 W rows (8 blocks = 272 contiguous bytes,
// 16-byte aligned) go through registers into LDS; the next stage's loads are
// in flight while the current one is multiplied.
//
// Lane layout of the MFMA (checked on the device): A[i][k] in lane i + 16
// (k / 8), element k % 8; B[k][j] in lane j + 16 (k / 8), element k % 8;
// C[i][j] in lane j + 16 (i / 4), element i % 4.

constexpr int kGemmBM = 64;
constexpr int kGemmBN = 64;
constexpr int kStageBlocks = 8;
constexpr int kXRow = 2 * 32 * kStageBlocks + 16;  // 528
constexpr int kWRow = 34 * kStageBlocks;           // 272
constexpr int kXLds = kGemmBM * kXRow;
constexpr int kWLds = kGemmBN * kWRow;
constexpr int kXPieces = kGemmBM * 32;             // 16-byte pieces per stage
constexpr int kWPieces = kGemmBN * 17;

enum { kEpiStore = 0, kEpiResidual = 1, kEpiSwiGLU = 2 };

struct GemmArgs {
  const uint16_t* x;  // [M, ldx] f16
  const uint8_t* w;   // Q8_0 rows of the layer
  uint16_t* y;        // [M, ldy] f16
  const uint16_t* r;  // residual [M, ldr] (kEpiResidual)
  int M, K;
  int n_tiles;        // output tiles of 64 columns (kEpiSwiGLU: 32 gate + 32 up rows)
  int ldx, ldy, ldr;
  int up_row;         // kEpiSwiGLU: first up row of W (gate rows are 0..up_row-1)
};

template <int EPI>
__device__ __forceinline__ void gemm_q8(const GemmArgs& A) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kXLds + kWLds];
  uint8_t* xl = lds;
  uint8_t* wl = lds + kXLds;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int g = lane >> 4;
  const int c16 = lane & 15;

  // Workgroups are dealt to the 8 XCDs round robin; the m tiles of one n tile
  // go to the same XCD, one after another, so its weight rows are fetched
  // from HBM once and then hit that XCD's L2.
  const int mt = (A.M + kGemmBM - 1) / kGemmBM;
  const int xcd = blockIdx.x & 7;
  const int slot = blockIdx.x >> 3;
  const int n_tile = (slot / mt) * 8 + xcd;
  const int m0 = (slot % mt) * kGemmBM;
  const int row_bytes = A.K / 32 * 34;
  const int stages = A.K / (32 * kStageBlocks);

  auto w_row = [&](int r) -> int {
    if constexpr (EPI == kEpiSwiGLU)
      return r < 32 ? 32 * n_tile + r : A.up_row + 32 * n_tile + (r - 32);
    else
      return kGemmBN * n_tile + r;
  };

  u32x4 xp[kXPieces / 256], wp[(kWPieces + 255) / 256];
  auto gload = [&](int s) {
#pragma unroll
    for (int j = 0; j < kXPieces / 256; ++j) {
      const int piece = t + 256 * j;
      const int row = piece >> 5;
      const int m = m0 + row < A.M ? m0 + row : A.M - 1;
      xp[j] = load_global(reinterpret_cast<const u32x4*>(
          A.x + (size_t)m * A.ldx + 256 * s + 8 * (piece & 31)));
    }
#pragma unroll
    for (int j = 0; j < (kWPieces + 255) / 256; ++j) {
      const int piece = t + 256 * j;
      if (piece < kWPieces) {
        const int row = piece / 17;
        wp[j] = load_global(reinterpret_cast<const u32x4*>(
            A.w + (size_t)w_row(row) * row_bytes + kWRow * s + 16 * (piece - 17 * row)));
      }
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int j = 0; j < kXPieces / 256; ++j) {
      const int piece = t + 256 * j;
      *reinterpret_cast<u32x4*>(xl + (piece >> 5) * kXRow + 16 * (piece & 31)) = xp[j];
    }
#pragma unroll
    for (int j = 0; j < (kWPieces + 255) / 256; ++j) {
      const int piece = t + 256 * j;
      if (piece < kWPieces) {
        const int row = piece / 17;
        *reinterpret_cast<u32x4*>(wl + row * kWRow + 16 * (piece - 17 * row)) = wp[j];
      }
    }
  };

  const int wm = wave & 1, wn = wave >> 1;
  int nrow[2];  // LDS W rows of this lane's column in the two n tiles
  if constexpr (EPI == kEpiSwiGLU) {
    nrow[0] = 16 * wn + c16;       // gate row
    nrow[1] = 32 + 16 * wn + c16;  // the matching up row
  } else {
    nrow[0] = 32 * wn + c16;
    nrow[1] = 32 * wn + 16 + c16;
  }
  f32x4 acc[2][2];
#pragma unroll
  for (int ms = 0; ms < 2; ++ms)
#pragma unroll
    for (int ns = 0; ns < 2; ++ns) acc[ms][ns] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
  const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};

  // Block b's four products are issued before block b - 1's are scaled into
  // the sums, so the matrix unit works while the scale FMAs run.
  f32x4 prev[2][2];
  float prev_sc[2] = {0.0f, 0.0f};
#pragma unroll
  for (int ms = 0; ms < 2; ++ms)
#pragma unroll
    for (int ns = 0; ns < 2; ++ns) prev[ms][ns] = zero;
  auto scale_in = [&]() {
#pragma unroll
    for (int ms = 0; ms < 2; ++ms)
#pragma unroll
      for (int ns = 0; ns < 2; ++ns)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[ms][ns][i] = __builtin_fmaf(prev_sc[ns], prev[ms][ns][i], acc[ms][ns][i]);
  };

  gload(0);
  for (int s = 0; s < stages; ++s) {
    __syncthreads();  // every wave is done reading the previous stage
    lstore();
    __syncthreads();
    if (s + 1 < stages) gload(s + 1);
#pragma unroll
    for (int b = 0; b < kStageBlocks; ++b) {
      f16x8 a[2];
#pragma unroll
      for (int ms = 0; ms < 2; ++ms)
        a[ms] = *reinterpret_cast<const f16x8*>(xl + (32 * wm + 16 * ms + c16) * kXRow +
                                                2 * (32 * b + 8 * g));
      f16x8 bq[2];
      float sc[2];
#pragma unroll
      for (int ns = 0; ns < 2; ++ns) {
        const uint8_t* wr = wl + nrow[ns] * kWRow + 34 * b;
        sc[ns] = (float)*reinterpret_cast<const _Float16*>(wr);
        // the block's int8 k = 8 g .. 8 g + 7 sit at wr + 2 + 8 g: 4-byte
        // aligned for odd b, 2 bytes past a dword boundary for even b
        uint32_t lo, hi;
        if (b % 2 == 0) {
          const uint32_t* p = reinterpret_cast<const uint32_t*>(wr + 8 * g);
          const uint32_t d0 = p[0], d1 = p[1], d2 = p[2];
          lo = __builtin_amdgcn_alignbyte(d1, d0, 2);
          hi = __builtin_amdgcn_alignbyte(d2, d1, 2);
        } else {
          const uint32_t* p = reinterpret_cast<const uint32_t*>(wr + 2 + 8 * g);
          lo = p[0];
          hi = p[1];
        }
        const uint32_t bl = lo ^ 0x80808080u, bh = hi ^ 0x80808080u;
        const f16x2 v0 = q8x2_to_f16x2(bl, kSelLo), v1 = q8x2_to_f16x2(bl, kSelHi);
        const f16x2 v2 = q8x2_to_f16x2(bh, kSelLo), v3 = q8x2_to_f16x2(bh, kSelHi);
        bq[ns] = (f16x8){v0.x, v0.y, v1.x, v1.y, v2.x, v2.y, v3.x, v3.y};
      }
      f32x4 cur[2][2];
#pragma unroll
      for (int ms = 0; ms < 2; ++ms)
#pragma unroll
        for (int ns = 0; ns < 2; ++ns)
          cur[ms][ns] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[ms], bq[ns], zero, 0, 0, 0);
      scale_in();  // block b - 1 (zeros before the first block)
#pragma unroll
      for (int ms = 0; ms < 2; ++ms)
#pragma unroll
        for (int ns = 0; ns < 2; ++ns) prev[ms][ns] = cur[ms][ns];
      prev_sc[0] = sc[0];
      prev_sc[1] = sc[1];
    }
  }
  scale_in();

  // epilogue: lane holds rows 4 g + i, column c16 of each 16 x 16 tile
#pragma unroll
  for (int ms = 0; ms < 2; ++ms) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m0 + 32 * wm + 16 * ms + 4 * g + i;
      if (m >= A.M) continue;
      if constexpr (EPI == kEpiSwiGLU) {
        const int col = 32 * n_tile + 16 * wn + c16;
        A.y[(size_t)m * A.ldy + col] = swiglu_f16(acc[ms][0][i], acc[ms][1][i]);
      } else {
#pragma unroll
        for (int ns = 0; ns < 2; ++ns) {
          const int col = kGemmBN * n_tile + 32 * wn + 16 * ns + c16;
          if constexpr (EPI == kEpiResidual)
            A.y[(size_t)m * A.ldy + col] =
                residual_f16(as_half(A.r[(size_t)m * A.ldr + col]), acc[ms][ns][i]);
          else
            A.y[(size_t)m * A.ldy + col] = f32_to_f16_bits(acc[ms][ns][i]);
        }
      }
    }
  }
}

// ----------------------------------------------------------- attention ----

struct PfAttnLds {
  uint32_t qh[2][64];  // roped q heads 2g, 2g+1 as f16 pairs
  float pbuf[kAttnWaves][2][32];
  float mrg[kAttnWaves][2][2 + kHeadDim];
};

}  // namespace

// h[i] = token_embd[tokens[i]] (qwen3_full.mlir:86-94); an id outside the
// vocabulary reads row 0, as the decode step does.
extern "C" __global__ __launch_bounds__(128) void pf_embed(const int32_t* __restrict__ tokens,
                                                           const uint16_t* __restrict__ emb,
                                                           uint16_t* __restrict__ h) {
  const int i = blockIdx.x;
  int tok = tokens[i];
  tok = (tok < 0 || tok >= kVocab) ? 0 : tok;
  reinterpret_cast<u32x4*>(h + (size_t)i * kHidden)[threadIdx.x] =
      load_global(reinterpret_cast<const u32x4*>(emb + (size_t)tok * kHidden) + threadIdx.x);
}

// out[i] = rms_norm(h[i], w) (qwen3_full.mlir:96-133, the same computation as
// @rms_norm_1x1024): 16 lanes per row, the decode step's lane layout and
// reduction, so a row's result is the decode kernels' bit for bit.
extern "C" __global__ __launch_bounds__(256) void pf_rmsnorm(const uint16_t* __restrict__ h,
                                                             const uint16_t* __restrict__ w,
                                                             uint16_t* __restrict__ out, int n) {
  const int row = blockIdx.x * 16 + (threadIdx.x >> 4);
  const int r = row < n ? row : n - 1;
  u32x4 xr[8];
  rmsnorm_gemv_x<false>(h + (size_t)r * kHidden, w, xr);
  if (row < n) {
    u32x4* o = reinterpret_cast<u32x4*>(out + (size_t)r * kHidden + 64 * (threadIdx.x & 15));
#pragma unroll
    for (int m = 0; m < 8; ++m) o[m] = xr[m];
  }
}

extern "C" __global__ __launch_bounds__(256) void pf_gemm_q8(GemmArgs A) {
  gemm_q8<kEpiStore>(A);
}
extern "C" __global__ __launch_bounds__(256) void pf_gemm_q8_res(GemmArgs A) {
  gemm_q8<kEpiResidual>(A);
}
extern "C" __global__ __launch_bounds__(256) void pf_gemm_q8_swiglu(GemmArgs A) {
  gemm_q8<kEpiSwiGLU>(A);
}

// Token i (position start + i), kv head g = blockIdx.y; waves 0, 1: q heads
// 2g, 2g+1, wave 2: k head g -> per-head rms_norm with q_norm / k_norm
// (qwen3_full.mlir:1812-1879) and RoPE (@position_components.rope,
// :1060-1130, the decode step's formula) -> q_roped[i] / the k cache slot;
// wave 3: v head g -> the v cache slot (the cache scatter of :1979-1983).
// Lane owns dims 2 lane, 2 lane + 1; the same operations as the decode step's
// attention prologue.  k_cache, v_cache: the layer's base ([max_seq, 8, 128]).
extern "C" __global__ __launch_bounds__(256) void pf_qk_rope_cache(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, int start, const uint16_t* __restrict__ qn_w,
    const uint16_t* __restrict__ kn_w, uint16_t* __restrict__ q_roped,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache) {
  const int i = blockIdx.x;
  const int g = blockIdx.y;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int pos = start + i;
  const size_t slot = ((size_t)pos * kKvHeads + g) * kHeadDim;
  if (wave == 3) {
    reinterpret_cast<uint32_t*>(v_cache + slot)[lane] =
        load_global(reinterpret_cast<const uint32_t*>(v + (size_t)i * 1024 + g * kHeadDim) + lane);
    return;
  }
  const uint16_t* src = wave < 2 ? q + (size_t)i * 2048 + (2 * g + wave) * kHeadDim
                                 : k + (size_t)i * 1024 + g * kHeadDim;
  const f16x2 xv = as_f16x2(load_global(reinterpret_cast<const uint32_t*>(src) + lane));
  const f16x2 wv = as_f16x2(
      load_global(reinterpret_cast<const uint32_t*>(wave < 2 ? qn_w : kn_w) + lane));
  float cs[2], sn[2];
  rope_angles(pos, cs, sn);
  const float a = (float)xv.x, b = (float)xv.y;
  float ss = a * a;
  ss = ss + b * b;
  ss = wave_sum(ss);
  const float r = sqrtf(ss / 128.0f + kEps);
  float xs[2];
  xs[0] = (float)to_f16((a / r) * (float)wv.x);
  xs[1] = (float)to_f16((b / r) * (float)wv.y);
  float r2[2];
#pragma unroll
  for (int dd = 0; dd < 2; ++dd) {
    const float other = __shfl_xor(xs[dd], 32, 64);  // dim d + 64 or d - 64
    if (lane < 32) {
      const float u = xs[dd] * cs[dd];
      const float w2 = other * sn[dd];
      r2[dd] = u - w2;
    } else {
      const float u = other * sn[dd];
      const float w2 = xs[dd] * cs[dd];
      r2[dd] = u + w2;
    }
  }
  const uint32_t out = pack_f16x2(r2[0], r2[1]);
  if (wave < 2)
    reinterpret_cast<uint32_t*>(q_roped + (size_t)i * 2048 + (2 * g + wave) * kHeadDim)[lane] = out;
  else
    reinterpret_cast<uint32_t*>(k_cache + slot)[lane] = out;
}

// Causal GQA attention (@attention_prefill, qwen3_full.mlir:1571-1729, with the
// mask j <= i of :1700-1710): token i at position start + i, kv head g =
// blockIdx.y, both query heads 2g, 2g+1, over cache positions [lo, start + i]
// where lo = 0 (the whole cache, as the decode steps of @prefill_all see it)
// or lo = start with chunk_local != 0 (only this call's tokens, as the
// reference's @prefill attends).  Four waves take four near-equal position
// ranges; each runs the decode step's chunk loop (scores of 32 positions,
// online softmax in f32, the weighted v sum in f32), and the four results
// merge in LDS.  out: [n, 2048] f16.
extern "C" __global__ __launch_bounds__(256) void pf_attention(
    const uint16_t* __restrict__ q_roped, const uint16_t* __restrict__ k_cache,
    const uint16_t* __restrict__ v_cache, int start, int chunk_local, uint16_t* __restrict__ out) {
  __shared__ PfAttnLds L;
  const int i = blockIdx.x;
  const int g = blockIdx.y;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int half = lane >> 5;
  const int pl = lane & 31;
  const int pos = start + i;
  const int lo = chunk_local ? start : 0;
  const int n = pos - lo + 1;
  if (t < 128)
    L.qh[t >> 6][t & 63] = load_global(
        reinterpret_cast<const uint32_t*>(q_roped + (size_t)i * 2048 + 2 * g * kHeadDim) + t);
  const int beg = lo + (int)((int64_t)wave * n / kAttnWaves);
  const int end = lo + (int)((int64_t)(wave + 1) * n / kAttnWaves);
  const int n_chunks = ((n + kAttnWaves - 1) / kAttnWaves + 31) / 32;  // workgroup-uniform
  const int last = end - 1 > lo ? end - 1 : lo;
  __syncthreads();

  float m = -__builtin_inff(), l = 0.0f;
  float mB = -__builtin_inff(), lB = 0.0f;
  float accA0 = 0.0f, accA1 = 0.0f, accB0 = 0.0f, accB1 = 0.0f;
  for (int c = 0; c < n_chunks; ++c) {
    const int c0 = beg + 32 * c;
    const int p = c0 + pl;
    const bool valid = p < end;
    const int pr = p < last ? p : last;
    u32x4 kreg[8];
    const u32x4* krow = reinterpret_cast<const u32x4*>(
        k_cache + ((size_t)pr * kKvHeads + g) * kHeadDim + 64 * half);
#pragma unroll
    for (int mm = 0; mm < 8; ++mm) kreg[mm] = load_global(krow + mm);
    uint32_t vreg[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const int pj = c0 + j < last ? c0 + j : last;
      vreg[j] = load_global(
          reinterpret_cast<const uint32_t*>(v_cache + ((size_t)pj * kKvHeads + g) * kHeadDim) + lane);
    }
    float dA = 0.0f, dB = 0.0f;
#pragma unroll
    for (int mm = 0; mm < 8; ++mm) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = 32 * half + 4 * mm + j;
        const f16x2 kv = as_f16x2(kreg[mm][j]);
        dA = __builtin_amdgcn_fdot2(as_f16x2(L.qh[0][d]), kv, dA, false);
        dB = __builtin_amdgcn_fdot2(as_f16x2(L.qh[1][d]), kv, dB, false);
      }
    }
    dA = dA + __shfl_xor(dA, 32, 64);
    dB = dB + __shfl_xor(dB, 32, 64);
    const float sA = valid ? dA * kAttnScale : -__builtin_inff();
    const float sB = valid ? dB * kAttnScale : -__builtin_inff();
    const float mnA = fmaxf(m, max32(sA));
    const float mnB = fmaxf(mB, max32(sB));
    const float cA = mnA == -__builtin_inff() ? 1.0f : expf(m - mnA);
    const float cB = mnB == -__builtin_inff() ? 1.0f : expf(mB - mnB);
    const float pA = valid ? expf(sA - mnA) : 0.0f;
    const float pB = valid ? expf(sB - mnB) : 0.0f;
    l = l * cA + sum32(pA);
    lB = lB * cB + sum32(pB);
    m = mnA;
    mB = mnB;
    if (half == 0) {
      L.pbuf[wave][0][pl] = pA;
      L.pbuf[wave][1][pl] = pB;
    }
    __syncthreads();
    accA0 *= cA;
    accA1 *= cA;
    accB0 *= cB;
    accB1 *= cB;
    const int nv = end - c0 < 32 ? end - c0 : 32;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const uint32_t vw = j < nv ? vreg[j] : 0u;
      const f16x2 vv = as_f16x2(vw);
      const float v0 = (float)vv.x, v1 = (float)vv.y;
      const float wa = L.pbuf[wave][0][j], wb = L.pbuf[wave][1][j];
      accA0 = accA0 + wa * v0;
      accA1 = accA1 + wa * v1;
      accB0 = accB0 + wb * v0;
      accB1 = accB1 + wb * v1;
    }
    __syncthreads();
  }

  if (lane == 0) {
    L.mrg[wave][0][0] = m;
    L.mrg[wave][0][1] = l;
    L.mrg[wave][1][0] = mB;
    L.mrg[wave][1][1] = lB;
  }
  L.mrg[wave][0][2 + 2 * lane] = accA0;
  L.mrg[wave][0][3 + 2 * lane] = accA1;
  L.mrg[wave][1][2 + 2 * lane] = accB0;
  L.mrg[wave][1][3 + 2 * lane] = accB1;
  __syncthreads();
  if (wave < 2) {
    const int hh = wave;
    float M = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, L.mrg[w][hh][0]);
    float Ls = 0.0f, a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) {
      const float mw = L.mrg[w][hh][0];
      const float ww = mw == -__builtin_inff() ? 0.0f : expf(mw - M);
      Ls = Ls + L.mrg[w][hh][1] * ww;
      a0 = a0 + L.mrg[w][hh][2 + 2 * lane] * ww;
      a1 = a1 + L.mrg[w][hh][3 + 2 * lane] * ww;
    }
    reinterpret_cast<uint32_t*>(out + (size_t)i * 2048 + (2 * g + hh) * kHeadDim)[lane] =
        pack_f16x2(a0 / Ls, a1 / Ls);
  }
}

// *pos = v (the position after the prompt, before the head's advance).
extern "C" __global__ void pf_set_pos(int32_t* __restrict__ pos, int v) {
  if (threadIdx.x == 0) *pos = v;
}
