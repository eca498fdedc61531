// gfx950 kernels for batched prompt ingestion: the reference's @prefill
// (model/qwen3_full.mlir:2032-2111, one @transformer_layer_prefill per layer,
// :1731-2030) runs all prompt tokens of a layer together, so the layer
// matrices become GEMMs [n_tokens, K] x [K, N] instead of n_tokens GEMVs.
//
// Per layer (eight launches, nine when an attention query block has several
// position splits):
//   pf_rmsnorm       rms_norm(h, attn_norm) of every token row
//   pf_gemm_q8       q, k and v projections in one launch (MFMA, Q8_0 weights
//                    dequantized to f16 in registers)
//   pf_qk_rope_cache per-head rms_norm of q and k, RoPE at each token's
//                    position, k and v written to their cache slots
//   pf_attention     causal GQA attention of every token over the cache
//   pf_attn_merge    the position splits' partial results combined
//   pf_gemm_q8       attn_o + residual
//   pf_rmsnorm       rms_norm(res, ffn_norm)
//   pf_gemm_q8       gate/up with SwiGLU in the epilogue
//   pf_gemm_q8       ffn_down + residual
// plus pf_embed (token rows) before the first layer.  The vocab GEMV + argmax
// of the last token reuses the decode kernels.  Prompts below 1024 tokens run
// attn_o and ffn_down with K split (pf_gemm_q8_part); their reduce
// (pf_res_reduce_norm) then also forms the rms_norm that follows (ffn_norm of
// the row after attn_o, the next layer's attn_norm after ffn_down), so those
// two pf_rmsnorm launches drop out.
//
// Numerics follow the decode step op for op (f16 tensors between ops, f32 in
// sums, norms and transcendental math): the norms, RoPE, SwiGLU and residual
// adds are the same device functions the decode kernels call.  The GEMMs use
// the weights @prefill itself reads: the f16 layer matrices the reference's
// converter makes from a Q8_0 file, f16(scale * q) with the product exact in
// f32 and rounded once (tools/convert_gguf_to_irpa.py:28-44, 174-199); every
// weight is formed that way in registers (one f16 multiply of the exact
// integer q by the f16 scale) and the MFMA accumulates f16 x * f16 w in f32
// over the whole K.
#include "decode_device.h"
#include "prefill_split.h"

namespace {

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

constexpr int kGemmBN = 64;
constexpr int kStageBlocks = 8;
constexpr int kXRow = 2 * 32 * kStageBlocks + 16;  // 528
constexpr int kWRow = 34 * kStageBlocks;           // 272
constexpr int kWLds = kGemmBN * kWRow;
constexpr int kWPieces = kGemmBN * 17;

enum { kEpiStore = 0, kEpiResidual = 1, kEpiSwiGLU = 2, kEpiPartial = 3 };

struct GemmArgs {
  const uint16_t* x;  // [M, ldx] f16
  const uint8_t* w;   // Q8_0 rows of the layer
  uint16_t* y;        // [M, ldy] f16
  const uint16_t* r;  // residual [M, ldr] (kEpiResidual)
  int M, K;
  int n_tiles;        // output tiles of 64 columns (kEpiSwiGLU: 32 gate + 32 up rows)
  int ldx, ldy, ldr;
  int up_row;         // kEpiSwiGLU: first up row of W (gate rows are 0..up_row-1)
  // Up to three products with the same x in one launch: tiles [seg_tile[0],
  // seg_tile[1]) use w_seg[0] / y_seg[0] / ldy_seg[0], tiles from seg_tile[1]
  // on the second set (tile numbers counted from the set's first tile);
  // seg_tile = n_tiles when unused.
  const uint8_t* w_seg[2];
  uint16_t* y_seg[2];
  int ldy_seg[2];
  int seg_tile[2];
  // kEpiPartial: K in `splits` equal ranges, one per group of workgroups;
  // split s stores its f32 sums at part[(s M + m) N + n], N = 64 n_tiles
  float* part;
  int splits;
};

template <int EPI, int BM>
__device__ __forceinline__ void gemm_q8(const GemmArgs& A) {
  static_assert(BM == 64 || (BM == 32 && EPI != kEpiSwiGLU), "tile shapes");
  constexpr int kXL = BM * kXRow;
  constexpr int kXP = BM * 32;   // 16-byte X pieces per stage
  // waves 2 (m) x 2 (n) of 32 x 32 (SwiGLU: 32 tokens x 16 gate + 16 up
  // columns), else waves 1 x 4 of BM x 16: a wave converts each B fragment
  // once and uses it for all BM / 16 of its m tiles
  constexpr bool kSplitM = EPI == kEpiSwiGLU;
  constexpr int MS = kSplitM ? 2 : BM / 16;  // 16-row tiles per wave
  constexpr int NS = kSplitM ? 2 : 1;        // 16-column tiles per wave
  __shared__ __attribute__((aligned(16))) uint8_t lds[kXL + kWLds];
  uint8_t* xl = lds;
  uint8_t* wl = lds + kXL;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int g = lane >> 4;
  const int c16 = lane & 15;

  // Workgroups are dealt to the 8 XCDs round robin; the m tiles of one n tile
  // go to the same XCD, one after another, so its weight rows are fetched
  // from HBM once and then hit that XCD's L2.
  const int mt = (A.M + BM - 1) / BM;
  const int tiles = mt * A.n_tiles;
  const int split = EPI == kEpiPartial ? (int)blockIdx.x / tiles : 0;
  const int bid = (int)blockIdx.x - split * tiles;
  const int xcd = bid & 7;
  const int slot = bid >> 3;
  int n_tile = (slot / mt) * 8 + xcd;
  const int m0 = (slot % mt) * BM;
  const uint8_t* wb = A.w;
  uint16_t* yb = A.y;
  int ldy = A.ldy;
  if (n_tile >= A.seg_tile[0]) {
    const int sg = n_tile >= A.seg_tile[1] ? 1 : 0;
    wb = A.w_seg[sg];
    yb = A.y_seg[sg];
    ldy = A.ldy_seg[sg];
    n_tile -= A.seg_tile[sg];
  }
  const int row_bytes = A.K / 32 * 34;
  const int stages = A.K / (32 * kStageBlocks) / (EPI == kEpiPartial ? A.splits : 1);
  const int s_base = split * stages;  // this split's first stage

  auto w_row = [&](int r) -> int {
    if constexpr (EPI == kEpiSwiGLU)
      return r < 32 ? 32 * n_tile + r : A.up_row + 32 * n_tile + (r - 32);
    else
      return kGemmBN * n_tile + r;
  };

  u32x4 xp[kXP / 256], wp[(kWPieces + 255) / 256];
  auto gload = [&](int s) {
#pragma unroll
    for (int j = 0; j < kXP / 256; ++j) {
      const int piece = t + 256 * j;
      const int row = piece >> 5;
      const int m = m0 + row < A.M ? m0 + row : A.M - 1;
      xp[j] = load_global(reinterpret_cast<const u32x4*>(
          A.x + (size_t)m * A.ldx + 256 * (s_base + s) + 8 * (piece & 31)));
    }
#pragma unroll
    for (int j = 0; j < (kWPieces + 255) / 256; ++j) {
      const int piece = t + 256 * j;
      if (piece < kWPieces) {
        const int row = piece / 17;
        wp[j] = load_global(reinterpret_cast<const u32x4*>(
            wb + (size_t)w_row(row) * row_bytes + kWRow * (s_base + s) + 16 * (piece - 17 * row)));
      }
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int j = 0; j < kXP / 256; ++j) {
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

  const int wm = kSplitM ? (wave & 1) : 0;
  const int wn = kSplitM ? (wave >> 1) : wave;
  int nrow[NS];  // LDS W rows of this lane's column in the wave's n tiles
  if constexpr (kSplitM) {
    nrow[0] = 16 * wn + c16;       // gate row
    nrow[1] = 32 + 16 * wn + c16;  // the matching up row
  } else {
    nrow[0] = 16 * wn + c16;
  }
  f32x4 acc[MS][NS];
#pragma unroll
  for (int ms = 0; ms < MS; ++ms)
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) acc[ms][ns] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  gload(0);
  for (int s = 0; s < stages; ++s) {
    __syncthreads();  // every wave is done reading the previous stage
    lstore();
    __syncthreads();
    if (s + 1 < stages) gload(s + 1);
#pragma unroll
    for (int b = 0; b < kStageBlocks; ++b) {
      f16x8 a[MS];
#pragma unroll
      for (int ms = 0; ms < MS; ++ms)
        a[ms] = *reinterpret_cast<const f16x8*>(xl + (32 * wm + 16 * ms + c16) * kXRow +
                                                2 * (32 * b + 8 * g));
      f16x8 bq[NS];
#pragma unroll
      for (int ns = 0; ns < NS; ++ns) {
        const uint8_t* wr = wl + nrow[ns] * kWRow + 34 * b;
        const _Float16 sc = *reinterpret_cast<const _Float16*>(wr);
        const f16x2 s2 = {sc, sc};
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
        // exact q in f16, then one rounding of scale * q (contraction is off)
        const f16x2 v0 = q8x2_to_f16x2(bl, kSelLo) * s2, v1 = q8x2_to_f16x2(bl, kSelHi) * s2;
        const f16x2 v2 = q8x2_to_f16x2(bh, kSelLo) * s2, v3 = q8x2_to_f16x2(bh, kSelHi) * s2;
        bq[ns] = (f16x8){v0.x, v0.y, v1.x, v1.y, v2.x, v2.y, v3.x, v3.y};
      }
#pragma unroll
      for (int ms = 0; ms < MS; ++ms)
#pragma unroll
        for (int ns = 0; ns < NS; ++ns)
          acc[ms][ns] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[ms], bq[ns], acc[ms][ns], 0, 0, 0);
    }
  }

  // epilogue: lane holds rows 4 g + i, column c16 of each 16 x 16 tile
#pragma unroll
  for (int ms = 0; ms < MS; ++ms) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m0 + 32 * wm + 16 * ms + 4 * g + i;
      if (m >= A.M) continue;
      if constexpr (EPI == kEpiSwiGLU) {
        const int col = 32 * n_tile + 16 * wn + c16;
        yb[(size_t)m * ldy + col] = swiglu_f16(acc[ms][0][i], acc[ms][1][i]);
      } else {
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) {
          const int col = kGemmBN * n_tile + 16 * wn + c16;
          if constexpr (EPI == kEpiResidual)
            yb[(size_t)m * ldy + col] =
                residual_f16(as_half(A.r[(size_t)m * A.ldr + col]), acc[ms][ns][i]);
          else if constexpr (EPI == kEpiPartial)
            A.part[((size_t)split * A.M + m) * (kGemmBN * A.n_tiles) + col] = acc[ms][ns][i];
          else
            yb[(size_t)m * ldy + col] = f32_to_f16_bits(acc[ms][ns][i]);
        }
      }
    }
  }
}

// ------------------------------------------------------------ f16 GEMM ----
//
// The same products over f16 copies of the layer matrices (pf_expand_q8: every
// weight f16(scale * q), the value gemm_q8 forms in registers), so no
// conversion runs in the loop.  Y[m, n] = sum_k X[m, k] W[n, k], X [M, ldx]
// and W [N, K] both f16 with k contiguous.
//
// Workgroup tile (16 MS WM) x (16 NS WN), WM x WN waves (default 2 x 2) of
// (16 MS) x (16 NS), each 16 x 16 piece one chain of v_mfma_f32_16x16x32_f16
// over K in order: every output sees the instructions gemm_q8 gives it, on
// the same values in the same order, so the two GEMMs' results are the same
// bits.
//
// A stage is KS k: the tile's BM X rows and BN W rows, 2 KS bytes each,
// copied from memory into LDS by the memory system (global_load_lds, 16 bytes
// per lane, 1 KiB per wave instruction) into one of NBUF buffers while the
// waves multiply another: the copies run NBUF - 1 stages ahead.  The buffers
// are separate LDS arrays and the loop is unrolled by NBUF, so the compiler
// sees that a stage's reads do not touch the buffers being filled and lets
// those copies stay in flight.
//
// LDS layout of a stage (f16_lds_off): rows of 256 bytes or more keep row R's
// 16-byte chunk c in slot c ^ (R & 15) of its 256-byte block, so the 16 rows
// one fragment read touches (lanes with the same k chunk) fall in 16 distinct
// slots; 128-byte rows go two to a 256-byte line (line L = R / 2, position
// 8 (R & 1) + c) with position p in slot p ^ (L & 15), the same pattern over
// the same 16 slots.  Measured with SQ_LDS_BANK_CONFLICT: both read without
// bank conflicts, where 128-byte rows with slot c ^ ((R & 7) ^ (R >> 3 & 1))
// took about 4 conflict cycles per ds_read_b128.

struct GemmF16Args {
  const uint16_t* x;  // [M, ldx] f16
  const uint16_t* w;  // [N, K] f16
  uint16_t* y;        // [M, ldy] f16 (output columns [0, seg_col[0]))
  const uint16_t* r;  // residual [M, ldr] (kEpiResidual)
  float* part;        // kEpiPartial: split s's sums at part[(s M + m) N + n]
  int M, K;
  int n_tiles;        // tiles of BN columns of W
  int ldx, ldy, ldr;
  int splits;         // kEpiPartial: K in `splits` equal ranges
  // output columns [seg_col[0], seg_col[1]) go to y_seg[0] (ld ldy_seg[0]),
  // columns from seg_col[1] on to y_seg[1], each counted from its first;
  // seg_col = N when unused
  uint16_t* y_seg[2];
  int ldy_seg[2];
  int seg_col[2];
};

// byte offset of row r's 16-byte chunk c (k 8 c .. 8 c + 7 of the stage) in
// a stage buffer with rows of C chunks
template <int C>
__device__ __forceinline__ int f16_lds_off(int r, int c) {
  if constexpr (C >= 16) {
    return r * 16 * C + 16 * (c ^ (r & 15));
  } else {
    static_assert(C == 8, "row length");
    const int line = r >> 1;
    return 256 * line + 16 * ((((r & 1) << 3) | c) ^ (line & 15));
  }
}

template <int EPI, int MS, int NS, int KS, int NBUF, int WM = 2, int WN = 2>
__device__ __forceinline__ void gemm_f16(const GemmF16Args& A) {
  static_assert(EPI != kEpiSwiGLU || NS % 2 == 0, "gate/up pairs");
  static_assert(KS == 64 || KS == 128 || KS == 256, "stage length");
  static_assert(NBUF >= 2 && NBUF <= 4, "buffers");
  constexpr int kWaves = WM * WN;
  constexpr int BM = 16 * MS * WM, BN = 16 * NS * WN;
  constexpr int kRows = BM + BN;
  constexpr int RB = 2 * KS;               // bytes of a tile row per stage
  constexpr int C = RB / 16;               // 16-byte chunks per row
  constexpr int RPI = 1024 / RB;           // rows per wave instruction
  constexpr int J = kRows / RPI / kWaves;  // copy instructions per wave per stage
  static_assert(kRows % (kWaves * RPI) == 0 && BM % RPI == 0, "copy pieces");
  static_assert(J * (NBUF - 2) < 64, "vmcnt range");
  constexpr int kBuf = kRows * RB;
  __shared__ __attribute__((aligned(1024))) uint8_t lds0[kBuf];
  __shared__ __attribute__((aligned(1024))) uint8_t lds1[kBuf];
  __shared__ __attribute__((aligned(1024))) uint8_t lds2[NBUF > 2 ? kBuf : 16];
  __shared__ __attribute__((aligned(1024))) uint8_t lds3[NBUF > 3 ? kBuf : 16];
  const int t = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lane = t & 63;
  const int g = lane >> 4;
  const int c16 = lane & 15;

  // XCD-aware tile order as in gemm_q8: the m tiles of one n tile run on one
  // XCD one after another, so its W rows come from HBM once
  const int mt = (A.M + BM - 1) / BM;
  const int tiles = mt * A.n_tiles;
  const int split = EPI == kEpiPartial ? (int)blockIdx.x / tiles : 0;
  const int bid = (int)blockIdx.x - split * tiles;
  const int xcd = bid & 7;
  const int slot = bid >> 3;
  const int n_tile = (slot / mt) * 8 + xcd;
  const int m0 = (slot % mt) * BM;
  const int n0 = n_tile * BN;
  const int stages = A.K / KS / (EPI == kEpiPartial ? A.splits : 1);
  const int k0 = split * stages * KS;

  // Copy sources: instruction j of this wave fills the 1 KiB at byte
  // 1024 (J wave + j) of the buffer, tile rows RPI (J wave + j) .. + RPI - 1
  // (X rows first, then W rows); lane l writes its 16 bytes at 16 l of that,
  // so it loads the (row, chunk) f16_lds_off places there.  X rows past M
  // repeat row M - 1 (their products are never stored).
  const uint8_t* src[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    int row, kc;
    if constexpr (C >= 16) {
      row = RPI * (J * wave + j) + lane / C;
      kc = (lane % C) ^ (row & 15);
    } else {
      const int line = 4 * (J * wave + j) + (lane >> 4);
      const int p = (lane & 15) ^ (line & 15);
      row = 2 * line + (p >> 3);
      kc = p & 7;
    }
    if (row < BM) {
      const int m = m0 + row < A.M ? m0 + row : A.M - 1;
      src[j] = reinterpret_cast<const uint8_t*>(A.x + (size_t)m * A.ldx + k0) + 16 * kc;
    } else {
      src[j] = reinterpret_cast<const uint8_t*>(A.w + (size_t)(n0 + row - BM) * A.K + k0) + 16 * kc;
    }
  }
  auto issue = [&](int s, uint8_t* buf) {
#pragma unroll
    for (int j = 0; j < J; ++j)
      __builtin_amdgcn_global_load_lds((const GLOBAL_AS void*)(src[j] + RB * s),
                                       (LDS_AS void*)(buf + 1024 * (J * wave + j)), 16, 0, 0);
  };

  const int wm = wave % WM;
  const int wn = wave / WM;
  // This lane's fragment chunk of k block kb (k chunk 4 kb + g) in the 16-row
  // group at row base b (a multiple of 16) is at 16 C b + off[(b / 16) & 1][kb]:
  // with 128-byte rows the slot key depends on bit 4 of b, which is known for
  // every fragment at compile time (MS and NS even there).
  static_assert(C >= 16 || (MS % 2 == 0 && NS % 2 == 0), "fragment row bases");
  static_assert(BM % 32 == 0, "fragment row bases");
  int off[2][KS / 32];
#pragma unroll
  for (int hb = 0; hb < 2; ++hb)
#pragma unroll
    for (int kb = 0; kb < KS / 32; ++kb)
      off[hb][kb] = f16_lds_off<C>(16 * hb + c16, 4 * kb + g) - 16 * C * 16 * hb;
  f32x4 acc[MS][NS];
#pragma unroll
  for (int ms = 0; ms < MS; ++ms)
#pragma unroll
    for (int ns = 0; ns < NS; ++ns) acc[ms][ns] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  auto compute = [&](const uint8_t* buf) {
#pragma unroll
    for (int kb = 0; kb < KS / 32; ++kb) {
      f16x8 a[MS], b[NS];
#pragma unroll
      for (int ms = 0; ms < MS; ++ms)
        a[ms] = *reinterpret_cast<const f16x8*>(buf + (16 * MS * wm + 16 * ms) * RB +
                                                off[ms & 1][kb]);
#pragma unroll
      for (int ns = 0; ns < NS; ++ns)
        b[ns] = *reinterpret_cast<const f16x8*>(buf + (BM + 16 * NS * wn + 16 * ns) * RB +
                                                off[ns & 1][kb]);
#pragma unroll
      for (int ms = 0; ms < MS; ++ms)
#pragma unroll
        for (int ns = 0; ns < NS; ++ns)
          acc[ms][ns] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[ms], b[ns], acc[ms][ns], 0, 0, 0);
    }
  };

  // Stage s lives in buffer s % NBUF.  Before stage s: this wave's copies of
  // stage s have landed (later stages' copies, up to NBUF - 2 of them, may
  // still be in flight: vmcnt counts in issue order), then a barrier makes
  // every wave's copies visible and shows that all waves are done with
  // stage s - 1, whose buffer then receives stage s + NBUF - 1.
  auto step = [&](int s, uint8_t* cur, uint8_t* refill) {
    if (s + NBUF - 2 < stages)
      wait_vm<J * (NBUF - 2)>();
    else
      wait_vm<0>();
    __syncthreads();
    if (s + NBUF - 1 < stages) issue(s + NBUF - 1, refill);
    compute(cur);
  };
#pragma unroll
  for (int i = 0; i < NBUF - 1; ++i)
    if (i < stages) issue(i, i == 0 ? lds0 : i == 1 ? lds1 : lds2);
  for (int s = 0; s < stages; s += NBUF) {
    if constexpr (NBUF == 2) {
      step(s, lds0, lds1);
      if (s + 1 < stages) step(s + 1, lds1, lds0);
    } else if constexpr (NBUF == 3) {
      step(s, lds0, lds2);
      if (s + 1 < stages) step(s + 1, lds1, lds0);
      if (s + 2 < stages) step(s + 2, lds2, lds1);
    } else {
      step(s, lds0, lds3);
      if (s + 1 < stages) step(s + 1, lds1, lds0);
      if (s + 2 < stages) step(s + 2, lds2, lds1);
      if (s + 3 < stages) step(s + 3, lds3, lds2);
    }
  }

  // epilogue: lane holds rows 4 g + i, column c16 of each 16 x 16 piece
  const int N = BN * A.n_tiles;
  int col0 = n0 + 16 * NS * wn;
  uint16_t* yb = A.y;
  int ldy = A.ldy;
  if constexpr (EPI == kEpiStore) {
    if (n0 >= A.seg_col[0]) {
      const int sg = n0 >= A.seg_col[1] ? 1 : 0;
      yb = A.y_seg[sg];
      ldy = A.ldy_seg[sg];
      col0 -= A.seg_col[sg];
    }
  }
#pragma unroll
  for (int ms = 0; ms < MS; ++ms) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m0 + 16 * MS * wm + 16 * ms + 4 * g + i;
      if (m >= A.M) continue;
      if constexpr (EPI == kEpiSwiGLU) {
        // W rows come in groups of 32: 16 gate rows, then the matching 16 up
        // rows (pf_expand_q8's gate/up order); group G feeds columns 16 G ..
#pragma unroll
        for (int p = 0; p < NS / 2; ++p) {
          const int col = (col0 + 32 * p) / 2 + c16;
          yb[(size_t)m * ldy + col] = swiglu_f16(acc[ms][2 * p][i], acc[ms][2 * p + 1][i]);
        }
      } else {
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) {
          const int col = col0 + 16 * ns + c16;
          if constexpr (EPI == kEpiResidual)
            yb[(size_t)m * ldy + col] =
                residual_f16(as_half(A.r[(size_t)m * A.ldr + col]), acc[ms][ns][i]);
          else if constexpr (EPI == kEpiPartial)
            A.part[((size_t)split * A.M + m) * N + col] = acc[ms][ns][i];
          else
            yb[(size_t)m * ldy + col] = f32_to_f16_bits(acc[ms][ns][i]);
        }
      }
    }
  }
}

}  // namespace

// f16 copies of Q8_0 layer matrices: dst row r' of layer l = f16(scale * q)
// of every weight of src row r (the reference converter's f16 weights,
// tools/convert_gguf_to_irpa.py:28-44: q exact in f16, one rounding of the
// product; the same two operations gemm_q8 does in registers).  gu_half > 0
// (gate/up stack: rows 0 .. gu_half - 1 gate, then as many up rows) orders the
// rows in groups of 32, gate rows 16 G .. 16 G + 15 then up rows 16 G ..
// 16 G + 15, the order gemm_f16's SwiGLU epilogue reads; otherwise r' = r.
// Thread = one Q8_0 block (34 bytes -> 32 f16); grid (ceil(blocks / 256),
// layers).
extern "C" __global__ __launch_bounds__(256) void pf_expand_q8(
    const uint8_t* __restrict__ src, long long src_layer_bytes, int rows, int K, int gu_half,
    uint16_t* __restrict__ dst, long long dst_layer_elems) {
  const int bpr = K / 32;
  const long long blk = (long long)blockIdx.x * 256 + threadIdx.x;
  if (blk >= (long long)rows * bpr) return;
  const int r = (int)(blk / bpr);
  const int b = (int)(blk - (long long)r * bpr);
  const uint8_t* s = src + (size_t)blockIdx.y * src_layer_bytes + (size_t)blk * 34;
  int rd = r;
  if (gu_half > 0) {
    const int up = r >= gu_half ? 1 : 0;
    const int j = r - up * gu_half;
    rd = 32 * (j >> 4) + 16 * up + (j & 15);
  }
  const uint16_t* s16 = reinterpret_cast<const uint16_t*>(s);  // blocks are 2-byte aligned
  const _Float16 sc = as_half(s16[0]);
  const f16x2 s2 = {sc, sc};
  u32x4 out[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // int8 k = 8 i .. 8 i + 7
    const uint32_t lo = (uint32_t)s16[1 + 4 * i] | ((uint32_t)s16[2 + 4 * i] << 16);
    const uint32_t hi = (uint32_t)s16[3 + 4 * i] | ((uint32_t)s16[4 + 4 * i] << 16);
    const uint32_t bl = lo ^ 0x80808080u, bh = hi ^ 0x80808080u;
    const f16x2 v0 = q8x2_to_f16x2(bl, kSelLo) * s2, v1 = q8x2_to_f16x2(bl, kSelHi) * s2;
    const f16x2 v2 = q8x2_to_f16x2(bh, kSelLo) * s2, v3 = q8x2_to_f16x2(bh, kSelHi) * s2;
    out[i] = (u32x4){__builtin_bit_cast(uint32_t, v0), __builtin_bit_cast(uint32_t, v1),
                     __builtin_bit_cast(uint32_t, v2), __builtin_bit_cast(uint32_t, v3)};
  }
  u32x4* d = reinterpret_cast<u32x4*>(dst + (size_t)blockIdx.y * dst_layer_elems +
                                      (size_t)rd * K + 32 * b);
#pragma unroll
  for (int i = 0; i < 4; ++i) d[i] = out[i];
}

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
  gemm_q8<kEpiStore, 64>(A);
}
extern "C" __global__ __launch_bounds__(256) void pf_gemm_q8_m32(GemmArgs A) {
  gemm_q8<kEpiStore, 32>(A);
}
extern "C" __global__ __launch_bounds__(256) void pf_gemm_q8_res(GemmArgs A) {
  gemm_q8<kEpiResidual, 64>(A);
}
extern "C" __global__ __launch_bounds__(256) void pf_gemm_q8_res_m32(GemmArgs A) {
  gemm_q8<kEpiResidual, 32>(A);
}
extern "C" __global__ __launch_bounds__(256) void pf_gemm_q8_part(GemmArgs A) {
  gemm_q8<kEpiPartial, 64>(A);
}
extern "C" __global__ __launch_bounds__(256) void pf_gemm_q8_part_m32(GemmArgs A) {
  gemm_q8<kEpiPartial, 32>(A);
}

// y[m, n] = residual_f16(r[m, n], sum over s in order of part[(s M + m) N + n])
// (the split-K form of pf_gemm_q8_res: the same residual add, the K ranges'
// f32 sums added one after another).
extern "C" __global__ __launch_bounds__(256) void pf_res_reduce(
    const float* __restrict__ part, int splits, int M, int N, const uint16_t* __restrict__ r,
    int ldr, uint16_t* __restrict__ y, int ldy) {
  const int e = (int)(blockIdx.x * 256 + threadIdx.x);
  if (e >= M * N) return;
  const int m = e / N, n = e - m * N;
  float acc = part[e];
  for (int s = 1; s < splits; ++s) acc += part[(size_t)s * M * N + e];
  y[(size_t)m * ldy + n] = residual_f16(as_half(r[(size_t)m * ldr + n]), acc);
}

// pf_res_reduce for N = 1024 (y, r ld 1024) followed by out = rms_norm(y, w)
// of the same row, so no separate pf_rmsnorm launch is needed.  Workgroup =
// one row: every thread reduces 4 columns (all splits' loads issued first,
// then added in split order, as pf_res_reduce adds them), adds the residual
// and normalises its columns with the workgroup (rmsnorm_wg, the same sum
// order as pf_rmsnorm's 16 lanes).  y and out are those two kernels' bits.
// splits <= kPfMaxSplits.
extern "C" __global__ __launch_bounds__(256) void pf_res_reduce_norm(
    const float* __restrict__ part, int splits, int M, const uint16_t* __restrict__ r,
    uint16_t* __restrict__ y, const uint16_t* __restrict__ w, uint16_t* __restrict__ out) {
  __shared__ float red[4];
  const int m = blockIdx.x;
  const int c = 4 * threadIdx.x;
  const size_t e = (size_t)m * kHidden + c;
  const size_t plane = (size_t)M * kHidden;
  const uint2 w4 = norm_weights4(w);
  float4 v[kPfMaxSplits];
#pragma unroll
  for (int s = 0; s < kPfMaxSplits; ++s)
    if (s < splits) v[s] = *reinterpret_cast<const float4*>(part + s * plane + e);
  float4 a = v[0];
#pragma unroll
  for (int s = 1; s < kPfMaxSplits; ++s)
    if (s < splits) {
      a.x += v[s].x;
      a.y += v[s].y;
      a.z += v[s].z;
      a.w += v[s].w;
    }
  const uint2 rv = *reinterpret_cast<const uint2*>(r + e);
  const uint32_t lo = (uint32_t)residual_f16(as_half((uint16_t)(rv.x & 0xffffu)), a.x) |
                      ((uint32_t)residual_f16(as_half((uint16_t)(rv.x >> 16)), a.y) << 16);
  const uint32_t hi = (uint32_t)residual_f16(as_half((uint16_t)(rv.y & 0xffffu)), a.z) |
                      ((uint32_t)residual_f16(as_half((uint16_t)(rv.y >> 16)), a.w) << 16);
  const uint2 o = {lo, hi};
  *reinterpret_cast<uint2*>(y + e) = o;
  *reinterpret_cast<uint2*>(out + e) = rmsnorm_wg(o, w4, red);
}

extern "C" __global__ __launch_bounds__(256) void pf_gemm_q8_swiglu(GemmArgs A) {
  gemm_q8<kEpiSwiGLU, 64>(A);
}

// gemm_f16 instances: pf_gemm_f16[_epilogue]_<MS><NS>[k] covers 32 MS
// tokens x 32 NS columns of W per workgroup (four waves); the stage length and buffer
// count are the fastest measured for where the host uses each (cold weights,
// 512-2048 tokens): 64 k for the 128-column tiles (two workgroups per CU);
// 128 k for the 64 x 64 tiles of q/k/v and attn_o / ffn_down with two
// workgroups per CU, 256 k (the "k" names: 128 KiB of LDS, one workgroup per
// CU) where the grid covers the CUs once; the SwiGLU 64 x 64 tile keeps 64 k.
#define PF_GEMM_F16(name, EPI, MS, NS, KS, NBUF)                          \
  extern "C" __global__ __launch_bounds__(256) void name(GemmF16Args A) { \
    gemm_f16<EPI, MS, NS, KS, NBUF>(A);                                   \
  }
// 256 x 192 over eight waves 4 (m) x 2 (n) of 64 x 96, 112 KiB of LDS: the
// gate/up product of 2048 tokens in one round of 256 workgroups (42.0 ->
// 32.6 us against 128 x 128 tiles, whose 768 workgroups take 1.5 rounds)
extern "C" __global__ __launch_bounds__(512) void pf_gemm_f16_swiglu_46w(GemmF16Args A) {
  gemm_f16<kEpiSwiGLU, 4, 6, 64, 2, 4, 2>(A);
}
PF_GEMM_F16(pf_gemm_f16_44, kEpiStore, 4, 4, 64, 2)
PF_GEMM_F16(pf_gemm_f16_24, kEpiStore, 2, 4, 64, 2)
PF_GEMM_F16(pf_gemm_f16_22, kEpiStore, 2, 2, 128, 2)
PF_GEMM_F16(pf_gemm_f16_swiglu_44, kEpiSwiGLU, 4, 4, 64, 2)
PF_GEMM_F16(pf_gemm_f16_swiglu_24, kEpiSwiGLU, 2, 4, 64, 2)
PF_GEMM_F16(pf_gemm_f16_swiglu_22, kEpiSwiGLU, 2, 2, 64, 2)
PF_GEMM_F16(pf_gemm_f16_res_22, kEpiResidual, 2, 2, 128, 2)
PF_GEMM_F16(pf_gemm_f16_res_22k, kEpiResidual, 2, 2, 256, 2)
PF_GEMM_F16(pf_gemm_f16_res_12k, kEpiResidual, 1, 2, 256, 3)
PF_GEMM_F16(pf_gemm_f16_part_22, kEpiPartial, 2, 2, 128, 2)
PF_GEMM_F16(pf_gemm_f16_part_22k, kEpiPartial, 2, 2, 256, 2)
PF_GEMM_F16(pf_gemm_f16_part_12k, kEpiPartial, 1, 2, 256, 3)
// 128 x 128 for attn_o / ffn_down where two K ranges of such tiles cover the
// CUs once (about 2048 tokens): a 64 x 64 wave tile reads a quarter of the
// LDS bytes per MFMA that the 32 x 32 of the 64 x 64 workgroup tile does
PF_GEMM_F16(pf_gemm_f16_part_44, kEpiPartial, 4, 4, 64, 2)
PF_GEMM_F16(pf_gemm_f16_part_44k, kEpiPartial, 4, 4, 128, 2)
#undef PF_GEMM_F16

// Per-head rms_norm (q_norm / k_norm, qwen3_full.mlir:648-702) and RoPE
// (:324-454) of one head vector: lane owns dims 2 lane, 2 lane + 1 (xw, an
// f16 pair), wv the lane's norm weights, cs / sn its two frequencies' cosines
// and sines; the same operations as the decode step's attention prologue.
__device__ __forceinline__ uint32_t head_norm_rope(uint32_t xw, f16x2 wv, const float (&cs)[2],
                                                   const float (&sn)[2]) {
  const int lane = threadIdx.x & 63;
  const f16x2 xv = as_f16x2(xw);
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
    const float other = xor32(xs[dd]);  // dim d + 64 or d - 64
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
  return pack_f16x2(r2[0], r2[1]);
}

// this lane's two frequencies (2 lane, 2 lane + 1, mod 64) for token m
__device__ __forceinline__ void rope_lane(const float* __restrict__ rope, int m, float (&cs)[2],
                                          float (&sn)[2]) {
  const int lane = threadIdx.x & 63;
  const uint2 c2 = load_global(reinterpret_cast<const uint2*>(rope + (size_t)m * 128 + ((2 * lane) & 63)));
  const uint2 s2 =
      load_global(reinterpret_cast<const uint2*>(rope + (size_t)m * 128 + 64 + ((2 * lane) & 63)));
  cs[0] = __uint_as_float(c2.x);
  cs[1] = __uint_as_float(c2.y);
  sn[0] = __uint_as_float(s2.x);
  sn[1] = __uint_as_float(s2.y);
}

// table[i] = the 64 cosines then the 64 sines of the RoPE angles at position
// start + i (rope_angle: the decode step's values), for every layer of a
// prompt.  One 64-lane workgroup per token.
extern "C" __global__ __launch_bounds__(64) void pf_rope_table(int start, float* __restrict__ table) {
  const int i = blockIdx.x, lane = threadIdx.x;
  float c, s;
  rope_angle(start + i, lane, c, s);
  table[(size_t)i * 128 + lane] = c;
  table[(size_t)i * 128 + 64 + lane] = s;
}

// Token i = blockIdx.x (position start + i): per-head rms_norm with q_norm /
// k_norm (qwen3_full.mlir:1812-1879) and RoPE (@position_components.rope,
// :1060-1130, the decode step's formula) -> q_roped[i] / the k cache slot,
// and v to its cache slot (the cache scatter of :1979-1983).  Wave w takes q
// heads 4w .. 4w + 3, k heads 2w, 2w + 1 and v heads 2w, 2w + 1; the six
// vectors are independent chains in the same wave.  Lane owns dims 2 lane,
// 2 lane + 1; per vector the same operations as the decode step's attention
// prologue; the angles come from pf_rope_table.  k_cache, v_cache: the
// layer's base ([max_seq, 8, 128]).
extern "C" __global__ __launch_bounds__(256) void pf_qk_rope_cache(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, int start, const uint16_t* __restrict__ qn_w,
    const uint16_t* __restrict__ kn_w, const float* __restrict__ rope,
    uint16_t* __restrict__ q_roped, uint16_t* __restrict__ k_cache,
    uint16_t* __restrict__ v_cache) {
  const int i = blockIdx.x;
  const int w = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int pos = start + i;
  constexpr int kVecs = 6;  // 4 q heads, 2 k heads
  f16x2 xv[kVecs];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    xv[j] = as_f16x2(load_global(
        reinterpret_cast<const uint32_t*>(q + (size_t)i * 2048 + (4 * w + j) * kHeadDim) + lane));
#pragma unroll
  for (int j = 0; j < 2; ++j)
    xv[4 + j] = as_f16x2(load_global(
        reinterpret_cast<const uint32_t*>(k + (size_t)i * 1024 + (2 * w + j) * kHeadDim) + lane));
  uint32_t vv[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
    vv[j] = load_global(
        reinterpret_cast<const uint32_t*>(v + (size_t)i * 1024 + (2 * w + j) * kHeadDim) + lane);
  const f16x2 qwv = as_f16x2(load_global(reinterpret_cast<const uint32_t*>(qn_w) + lane));
  const f16x2 kwv = as_f16x2(load_global(reinterpret_cast<const uint32_t*>(kn_w) + lane));
  float cs[2], sn[2];
  rope_lane(rope, i, cs, sn);  // this lane's frequencies at the token's position
  uint32_t out[kVecs];
#pragma unroll
  for (int j = 0; j < kVecs; ++j)
    out[j] = head_norm_rope(__builtin_bit_cast(uint32_t, xv[j]), j < 4 ? qwv : kwv, cs, sn);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    reinterpret_cast<uint32_t*>(q_roped + (size_t)i * 2048 + (4 * w + j) * kHeadDim)[lane] = out[j];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const size_t slot = ((size_t)pos * kKvHeads + 2 * w + j) * kHeadDim;
    reinterpret_cast<uint32_t*>(k_cache + slot)[lane] = out[4 + j];
    reinterpret_cast<uint32_t*>(v_cache + slot)[lane] = vv[j];
  }
}

// Causal GQA attention (@attention_prefill, qwen3_full.mlir:1571-1729, with the
// mask j <= i of :1700-1710): workgroup (query block qb of 32 tokens, kv head
// g) computes both query heads 2g, 2g+1 for tokens 32 qb .. 32 qb + 31 at
// positions start + token over cache positions [lo, position], lo = 0 (the
// whole cache, what the decode steps of @prefill_all see) or lo = start with
// chunk_local != 0 (this call's tokens only, as the reference's @prefill
// attends).  Wave w takes query head 2g + (w >> 1) and tokens 32 qb + 16 (w &
// 1) .. + 15.  Per block of 32 cache positions the K tile and the V tile
// ([32][128] f16 each) are copied into LDS by the memory system
// (global_load_lds, two blocks ahead, three buffers), row r's 16-byte chunk c
// in slot c ^ (r & 15) (K) or c ^ 2 (r & 7) (V) so that the fragment reads
// below hit distinct banks, and each wave works transposed, one query per
// lane column:
//   S^T = K Q^T: 8 v_mfma_f32_16x16x32_f16 (K rows as A, the wave's 16 query
//     rows as B; exact f16 products, f32 sums), so lane (c16, grp) holds the
//     scores of query c16 at positions 4 grp + e and 16 + 4 grp + e (e < 4);
//   online softmax in f32 per query (a lagging reference maximum m, the
//     lane's share of the sum l; the max over a query's four lanes by
//     permlane swaps), scores
//     scaled by rsqrt(128) log2(e) so each weight is one exp2 (v_exp_f32);
//   O^T += V^T P^T: the lane's 8 weights are the B operand as they are, with
//     the MFMA's 32 k slots standing for positions in the order 4 grp + e,
//     16 + 4 grp + e; V^T comes from two transposing LDS reads per 16 dims in
//     that order.  p is split into f16 hi + lo (p - hi), O^T = V^T hi +
//     V^T lo (8 + 8 MFMAs), carrying p to about 2^-22.
// No weight goes through LDS.  Blocks below every query of the wave skip the
// mask; the O rescale is skipped when no lane's reference moved.  out: [n, 2048]
// f16 = O / l.
//
// A query block's positions are divided into splits of split_blocks blocks of
// 32 (prefill_split.h); grid 8 x (pairs of query block and split),
// workgroup 8 pair + g: kv head g = workgroup mod 8 runs on XCD g (workgroups
// go to the 8 XCDs in turn), so each XCD's L2 holds one head's cache rows
// (1 MiB at 2048 positions) instead of all eight.  A query
// block with one split writes its output directly; otherwise each split
// leaves its partial in its slot of `part` and pf_attn_merge, launched next,
// combines them.

// How far (base-2 units) a block's maximum score may exceed the reference
// maximum before the reference moves (the weights' range is [0, 2^kMaxLag]).
constexpr float kMaxLag = 8.0f;

extern "C" __global__ __launch_bounds__(256) void pf_attention(
    const uint16_t* __restrict__ q_roped, const uint16_t* __restrict__ k_cache,
    const uint16_t* __restrict__ v_cache, int n, int start, int chunk_local, int split_blocks,
    float* __restrict__ part, uint16_t* __restrict__ out) {
  // K and V tiles of two blocks: separate arrays so the compiler sees that
  // reading one buffer does not wait for the copies into the other.  (Three,
  // two blocks copied ahead, 48 KiB of LDS against 32: 4.83 against 4.80 ms
  // for 2048 tokens, the same bits.)
  __shared__ __attribute__((aligned(1024))) uint8_t kt0[8192], kt1[8192];
  __shared__ __attribute__((aligned(1024))) uint8_t vt0[8192], vt1[8192];
  const int g = blockIdx.x & 7;
  const int pair = blockIdx.x >> 3;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int c16 = lane & 15;
  const int grp = lane >> 4;
  const int head = 2 * g + (wave >> 1);
  const int lo = chunk_local ? start : 0;
  const PfSplitGeometry G = pf_split_geometry(n, start, lo);
  const PfSplitPair P = pf_split_pair(G, split_blocks, pair);
  const int qb = P.qb;
  const int q0 = 32 * qb + 16 * (wave & 1);  // this wave's first token

  // Q rows as the MFMA B operand: column c16 (query q0 + c16), dims 32 s +
  // 8 grp .. + 7
  f16x8 qf[4];
  {
    const int qi = q0 + c16 < n ? q0 + c16 : n - 1;
    const _Float16* qs = reinterpret_cast<const _Float16*>(q_roped) + (size_t)qi * 2048 + head * 128;
#pragma unroll
    for (int st = 0; st < 4; ++st)
      qf[st] = *reinterpret_cast<const f16x8*>(qs + 32 * st + 8 * grp);
  }
  const int last_tok = 32 * qb + 31 < n ? 32 * qb + 31 : n - 1;
  const int hi = start + last_tok;  // the last position any query here attends
  // this split's positions: [kb_lo, kb_hi]
  const int kb_lo = lo + 32 * split_blocks * P.s;
  const int kb_hi = hi < kb_lo + 32 * split_blocks - 1 ? hi : kb_lo + 32 * split_blocks - 1;
  // this lane's query and its position; the wave's first query position
  const bool qok = q0 + c16 < n;
  const int qpos = start + q0 + c16;
  const bool wave_full = q0 + 15 < n;  // all 16 queries of the wave exist
  float m = -__builtin_inff(), l = 0.0f;
  f32x4 o[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) o[d] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
  const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  // V^T reads: lane j of a 16-lane group addresses row vrow + j / 4, columns
  // 16 d + 4 (j % 4) .. + 3 (chunk 2 d + (j % 4) / 2, 8 (j % 2) bytes in);
  // ds_read_b64_tr_b16 gives lane i element i % 4 of the pieces of lanes
  // i / 4 + 4 r (r = 0..3): V[vrow + r][16 d + i]
  const int vrow = 4 * grp + (c16 >> 2);
  auto v_off = [&](int row, int d) {
    return 256 * row + 16 * ((2 * d + ((c16 & 3) >> 1)) ^ (2 * (row & 7))) + 8 * (c16 & 1);
  };

  // Copies: wave w fills 1 KiB pieces 2 w, 2 w + 1 of each tile (rows 4 p ..
  // 4 p + 3); lane l loads row 4 p + l / 16, the chunk whose slot is l % 16.
  // Positions past kb_hi repeat kb_hi (only ever masked).
  const int prow = lane >> 4;
  auto issue = [&](int kb, uint8_t* kt, uint8_t* vt) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int pc = 2 * wave + j;
      const int row = 4 * pc + prow;
      const int kp = kb + row <= kb_hi ? kb + row : kb_hi;
      const uint16_t* base = k_cache + ((size_t)kp * kKvHeads + g) * kHeadDim;
      const size_t voff = ((size_t)kp * kKvHeads + g) * kHeadDim;
      __builtin_amdgcn_global_load_lds(
          (const GLOBAL_AS void*)(base + 8 * ((lane & 15) ^ (row & 15))),
          (LDS_AS void*)(kt + 1024 * pc), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(
          (const GLOBAL_AS void*)(v_cache + voff + 8 * ((lane & 15) ^ (2 * (row & 7)))),
          (LDS_AS void*)(vt + 1024 * pc), 16, 0, 0);
    }
  };

  // One block: its copies landed, a barrier (every wave's copies visible,
  // every wave done with the previous block, whose buffers then receive
  // block + 1, copied while this one is computed).
  auto block = [&](int kb, const uint8_t* kt, const uint8_t* vt, uint8_t* kn, uint8_t* vn) {
    wait_vm<0>();
    __syncthreads();
    if (kb + 32 <= kb_hi) issue(kb + 32, kn, vn);

    // S^T for positions kb .. kb + 15 (tile 0) and kb + 16 .. kb + 31 (tile 1)
    f32x4 sc[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      sc[nt] = zero;
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int row = 16 * nt + c16;
        const f16x8 kf = *reinterpret_cast<const f16x8*>(kt + 256 * row + 16 * ((4 * st + grp) ^ c16));
        sc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[st], sc[nt], 0, 0, 0);
      }
    }
    // s[4 nt + e]: position kb + 16 nt + 4 grp + e (a split ends on a block
    // edge or at hi, so positions past kb_hi only appear masked)
    float s[8];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int e = 0; e < 4; ++e) s[4 * nt + e] = sc[nt][e];
    const bool masked = !(wave_full && kb + 31 <= start + q0);
    if (masked) {
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int kp = kb + 16 * nt + 4 * grp + e;
          if (!(qok && kp <= qpos)) s[4 * nt + e] = -__builtin_inff();
        }
    }
    // scores in base-2 units (products are canonical floats, so the max below
    // needs no NaN-quieting of its inputs)
#pragma unroll
    for (int i = 0; i < 8; ++i) s[i] *= kScoreScaleLog2;
    float mx = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])),
                     fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
    mx = max_col4(mx);
    // The reference maximum m lags: it moves to the block's maximum only when
    // that exceeds it by more than kMaxLag (base-2 units), or on the first
    // block with a valid score, so weights stay at most 2^kMaxLag and most
    // blocks skip the rescale of o.  o and l share the reference, so o / l is
    // the same quotient.  alpha = 2^(m - mn) where it moves (0 from m = -inf,
    // where o and l are still 0), else 1.
    const bool grow = mx > m + kMaxLag;  // false while both are -inf
    const float mn = grow ? mx : m;
    // v_exp_f32 without the denormal-range fix-up of exp2f: a weight below
    // 2^-126 beside the weight 1 of the score that set m changes no f32 sum
    const float alpha = __builtin_amdgcn_exp2f(grow ? m - mx : 0.0f);
    // A masked score is -inf and its weight 2^(-inf - mn) = 0 while mn is
    // finite; mn is -inf only while every score of the query so far is
    // masked, where the reference 0 gives those weights 2^-inf = 0 as well
    // (instead of 2^NaN).  One form for masked and unmasked blocks.
    const float mref = mn == -__builtin_inff() ? 0.0f : mn;
    float p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) p[i] = __builtin_amdgcn_exp2f(s[i] - mref);
    float ps = p[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) ps += p[i];
    l = l * alpha + ps;
    m = mn;
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
      for (int d = 0; d < 8; ++d) o[d] *= alpha;
    }
    // hi = f16(p) (pairs at a time, v_cvt_pk_f16_f32), lo = f16(p - hi): p -
    // hi is exact in f32, so the fused -hi * 1 + p of v_fma_mixlo_f16 /
    // v_fma_mixhi_f16 (hi's f16 half widened exactly, one rounding to f16 into
    // the low / high half) gives the same pair as subtracting and converting
    f16x8 ph, pl;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      typedef float f32x2_t __attribute__((ext_vector_type(2)));
      const f16x2 h2 = __builtin_convertvector((f32x2_t){p[i], p[i + 1]}, f16x2);
      const uint32_t hb = __builtin_bit_cast(uint32_t, h2);
      uint32_t lb;
      asm("v_fma_mixlo_f16 %0, -%1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(lb) : "v"(hb), "v"(p[i]));
      asm("v_fma_mixhi_f16 %0, -%1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
          : "+v"(lb)
          : "v"(hb), "v"(p[i + 1]));
      const f16x2 l2 = __builtin_bit_cast(f16x2, lb);
      ph[i] = h2.x;
      ph[i + 1] = h2.y;
      pl[i] = l2.x;
      pl[i + 1] = l2.y;
    }
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const v4i16 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (LDS_AS v4i16*)(vt + v_off(vrow, d)));
      const v4i16 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (LDS_AS v4i16*)(vt + v_off(vrow + 16, d)));
      const f16x8 vf = __builtin_bit_cast(
          f16x8, (v8i16){v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w});
      o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, ph, o[d], 0, 0, 0);
      o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pl, o[d], 0, 0, 0);
    }
  };

  // buffer of block i: i % 2 (the loop unrolled by two); block i + 1 is
  // copied while block i is computed.  Measured and not kept (same bits,
  // 2048 tokens, rocprof mean of this kernel): block i + 1's score MFMAs
  // issued before block i's softmax, K two buffers ahead of V (148 VGPRs:
  // 43.2 us against 40.5; capped at 128: 43.3 against 39.7); the (query
  // block, split) pairs launched longest first (40.6 against 40.5).
  issue(kb_lo, kt0, vt0);
  for (int kb = kb_lo; kb <= kb_hi; kb += 64) {
    block(kb, kt0, vt0, kt1, vt1);
    if (kb + 32 > kb_hi) break;
    block(kb + 32, kt1, vt1, kt0, vt0);
  }
  // o[d][e]: dim 16 d + 4 grp + e of query q0 + c16; l over its four lanes
  l = sum_col4(l);

  if (P.ns == 1) {
    if (!qok) return;
    uint16_t* orow = out + (size_t)(q0 + c16) * 2048 + head * 128 + 4 * grp;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const uint2 v = {pack_f16x2(o[d][0] / l, o[d][1] / l), pack_f16x2(o[d][2] / l, o[d][3] / l)};
      *reinterpret_cast<uint2*>(orow + 16 * d) = v;
    }
    return;
  }

  // several splits: (m, l, O) of this split's positions to its slot, row
  // 16 wave + c16; pf_attn_merge combines the slots
  float* slot = part + ((size_t)pair * kKvHeads + g) * kPfAttnSlotFloats;
  const int r = 16 * wave + c16;
#pragma unroll
  for (int d = 0; d < 8; ++d)
    *reinterpret_cast<f32x4*>(slot + r * kHeadDim + 16 * d + 4 * grp) = o[d];
  if (grp == 0) {
    slot[64 * kHeadDim + r] = m;
    slot[64 * kHeadDim + 64 + r] = l;
  }
}

// The splits of query block blockIdx.x / 32, kv head g = blockIdx.x % 8 (on
// the XCD whose L2 saw that head's partials written; nothing to do for a
// block with one split), merged in split order with a running maximum (m in
// base-2 units, as pf_attention keeps it):
//   M' = max(M, m_s),  O' = O 2^(M - M') + O_s 2^(m_s - M'),
//   l' = l 2^(M - M') + l_s 2^(m_s - M'),
// out = O / l.  Four workgroups per query block, one per 32 of the 128
// dimensions; thread t: slot row t >> 2 (wave w = row >> 4 of pf_attention:
// head 2g + (w >> 1), token 32 qb + 16 (w & 1) + (row & 15)), dims
// 32 ((blockIdx.x / 8) % 4) + 8 (t & 3) .. + 7.  The partials of up to 8
// splits are requested before any is used, so a query block with many splits
// waits for memory once per 8 splits.
extern "C" __global__ __launch_bounds__(256) void pf_attn_merge(
    const float* __restrict__ part, int n, int start, int chunk_local, int split_blocks,
    uint16_t* __restrict__ out) {
  const int qb = blockIdx.x >> 5;
  const int quarter = (blockIdx.x >> 3) & 3;
  const int g = blockIdx.x & 7;
  const PfSplitGeometry G = pf_split_geometry(n, start, chunk_local ? start : 0);
  const int nb = qb == G.nqb - 1 ? G.nb_last : qb + G.c;
  const int ns = (nb + split_blocks - 1) / split_blocks;
  if (ns == 1) return;
  const size_t first = (size_t)pf_pairs_before(G, qb, split_blocks) * kKvHeads + g;
  const int t = threadIdx.x;
  const int r = t >> 2;
  const int d0 = 32 * quarter + 8 * (t & 3);
  const int w = r >> 4;
  const int tok = 32 * qb + 16 * (w & 1) + (r & 15);
  if (tok >= n) return;
  constexpr int kGroup = 8;
  float M = -__builtin_inff(), L = 0.0f, acc[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) acc[d] = 0.0f;
  for (int s0 = 0; s0 < ns; s0 += kGroup) {
    float ms[kGroup], ls[kGroup];
    float4 os[kGroup][2];
#pragma unroll
    for (int k = 0; k < kGroup; ++k) {
      const int s = s0 + k < ns ? s0 + k : ns - 1;
      const float* sl = part + (first + (size_t)s * kKvHeads) * kPfAttnSlotFloats;
      ms[k] = sl[64 * kHeadDim + r];
      ls[k] = sl[64 * kHeadDim + 64 + r];
      const float4* orow = reinterpret_cast<const float4*>(sl + r * kHeadDim + d0);
      os[k][0] = orow[0];
      os[k][1] = orow[1];
    }
#pragma unroll
    for (int k = 0; k < kGroup; ++k) {
      if (s0 + k < ns) {
        const float mn = fmaxf(M, ms[k]);
        const float a = M == -__builtin_inff() ? 0.0f : exp2f(M - mn);
        const float b = ms[k] == -__builtin_inff() ? 0.0f : exp2f(ms[k] - mn);
        L = L * a + ls[k] * b;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          acc[4 * j] = acc[4 * j] * a + os[k][j].x * b;
          acc[4 * j + 1] = acc[4 * j + 1] * a + os[k][j].y * b;
          acc[4 * j + 2] = acc[4 * j + 2] * a + os[k][j].z * b;
          acc[4 * j + 3] = acc[4 * j + 3] * a + os[k][j].w * b;
        }
        M = mn;
      }
    }
  }
  const u32x4 v = {pack_f16x2(acc[0] / L, acc[1] / L), pack_f16x2(acc[2] / L, acc[3] / L),
                   pack_f16x2(acc[4] / L, acc[5] / L), pack_f16x2(acc[6] / L, acc[7] / L)};
  *reinterpret_cast<u32x4*>(out + (size_t)tok * 2048 + (2 * g + (w >> 1)) * kHeadDim + d0) = v;
}

// *pos = v (the position after the prompt, before the head's advance).
extern "C" __global__ void pf_set_pos(int32_t* __restrict__ pos, int v) {
  if (threadIdx.x == 0) *pos = v;
}
