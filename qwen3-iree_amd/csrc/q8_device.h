// Device helpers shared by the gfx950 kernel sources (q8gemv_kernels.hip,
// decode_kernels.hip): f16 / Q8_0 arithmetic, wave64 DPP reductions, the Q8_0
// GEMV engine (single quad, batched units) and the vocab GEMV + argmax body.
// Header-only; every helper is internal to the including translation unit.
#ifndef QWEN3_Q8_DEVICE_H
#define QWEN3_Q8_DEVICE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

// Every multiply-add below is written out; the compiler may not contract on
// its own, so the same row computes to the same bits in every kernel that
// inlines the shared helpers (single, fused q/k/v, batched and decode-step
// launches).
#pragma clang fp contract(off)

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace {

// v_perm_b32 selectors: output bytes (b_lo, 0x64, b_hi, 0x64) taking b from
// bytes 0,1 (SEL_LO) or 2,3 (SEL_HI) of the second operand; selector 4 picks
// byte 0 of the first operand, the 0x64646464 constant.
constexpr uint32_t kSelLo = 0x04010400u;
constexpr uint32_t kSelHi = 0x04030402u;

__device__ __forceinline__ f16x2 q8x2_to_f16x2(uint32_t biased, uint32_t sel) {
  const uint32_t v = __builtin_amdgcn_perm(0x64646464u, biased, sel);
  // (1024 + u) - 1152 = u - 128 = q, exact in f16.
  return __builtin_bit_cast(f16x2, v) - (f16x2){(_Float16)1152.0f, (_Float16)1152.0f};
}

__device__ __forceinline__ f16x2 as_f16x2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }

// Load flavour of the weight streams (read once per launch): nontemporal
// loads (global_load ... nt) for the Q8_0 and the vocab matrices.  Plain loads
// let the memory-side cache (MALL, 256 MB) keep part of a matrix from one
// launch to the next: measured on MI355X, the vocab kernel with plain loads
// ran 48.3 us back to back but 56.5 us after a 1 GiB read evicted the MALL,
// with nontemporal loads 50.5 and 51.8 us; the decode step 518.5 -> 513.9 us.
#ifndef Q8_NT_LOADS
#define Q8_NT_LOADS 1
#endif
#ifndef Q8_X_REUSE
#define Q8_X_REUSE 1
#endif
// Register sets of units a wave of the batched launch keeps in flight (2 or
// 3; three measured 1-2 % slower, warm and after a MALL eviction).
#ifndef Q8_SEG_SETS
#define Q8_SEG_SETS 2
#endif
#ifndef VOCAB_NT_LOADS
#define VOCAB_NT_LOADS 1
#endif

// Ablation builds (qwen3-iree_amd/ablation.py) replace one design choice of
// the batched Q8_0 GEMV and of the vocab GEMV with a plain alternative that
// computes the same outputs, so what each choice is worth can be measured;
// the product build takes every default.
//   Q8_LOAD_BYTES 16 | 8 | 4: each lane's 16 bytes of a weight piece read as
//     one 128-bit load, or as two 64-bit / four 32-bit loads
//   Q8_X_LDS 1 | 0: x staged once per workgroup in LDS, or read by the wave
//     from global memory for every unit
//   Q8_DEQUANT_PACKED 1 | 0: int8 pairs made f16 pairs in registers and
//     multiplied by v_dot2, or every int8 converted to f32 and multiplied by
//     f32(x) (same exact products, summed one by one)
//   Q8_REDUCE_DPP 1 | 0: 16-lane row sums by DPP, or by ds_bpermute shuffles
//     through the LDS crossbar (same pairs, same bits)
#ifndef Q8_LOAD_BYTES
#define Q8_LOAD_BYTES 16
#endif
#ifndef Q8_X_LDS
#define Q8_X_LDS 1
#endif
#ifndef Q8_DEQUANT_PACKED
#define Q8_DEQUANT_PACKED 1
#endif
#ifndef Q8_REDUCE_DPP
#define Q8_REDUCE_DPP 1
#endif
static_assert(Q8_LOAD_BYTES == 16 || Q8_LOAD_BYTES == 8 || Q8_LOAD_BYTES == 4, "load width");

// Pointers read from a batch table are generic; accessing them through the
// global address space keeps the loads global_load (counted by vmcnt alone)
// rather than flat_load, whose completion the compiler can only await with a
// full vmcnt(0) lgkmcnt(0) drain.
#define GLOBAL_AS __attribute__((address_space(1)))

// vmcnt(n) with the other counters left alone (gfx9 s_waitcnt encoding)
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0f70);
}
// lgkmcnt(0): every LDS read of the wave has returned its data
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xc07f); }

// The launch's workgroup size and count in x, from the hidden kernel
// arguments (code object v5: block counts at bytes 0, 4, 8, group sizes as
// u16 at 12, 14, 16), with scalar loads.  blockDim.x compiles to a 16-bit
// vector load (it allows for a partial last workgroup, which these launches
// never have) whose wait would come before a kernel's first weight loads.
__device__ __forceinline__ uint32_t launch_wg_size() {
  return reinterpret_cast<const uint32_t*>(__builtin_amdgcn_implicitarg_ptr())[3] & 0xffffu;
}
__device__ __forceinline__ uint32_t launch_wgs() {
  return reinterpret_cast<const uint32_t*>(__builtin_amdgcn_implicitarg_ptr())[0];
}

template <bool NT>
__device__ __forceinline__ u32x4 load_stream(const u32x4* p) {
  const GLOBAL_AS u32x4* g = (const GLOBAL_AS u32x4*)p;
  if constexpr (NT) return __builtin_nontemporal_load(g);
  else return *g;
}

// A weight stream's 16 bytes per lane, as Q8_LOAD_BYTES wide loads.
template <bool NT>
__device__ __forceinline__ u32x4 load_weights16(const u32x4* p) {
  if constexpr (Q8_LOAD_BYTES == 16) {
    return load_stream<NT>(p);
  } else {
    // the next part's offset is hidden from the compiler, which would
    // otherwise merge the parts back into one 128-bit load
    int k = 1;
    asm volatile("" : "+v"(k));
    if constexpr (Q8_LOAD_BYTES == 8) {
      typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
      const GLOBAL_AS u32x2* g = (const GLOBAL_AS u32x2*)p;
      u32x2 a, b;
      if constexpr (NT) {
        a = __builtin_nontemporal_load(g);
        b = __builtin_nontemporal_load(g + k);
      } else {
        a = g[0];
        b = g[k];
      }
      return (u32x4){a.x, a.y, b.x, b.y};
    } else {
      const GLOBAL_AS uint32_t* g = (const GLOBAL_AS uint32_t*)p;
      u32x4 v;
      if constexpr (NT) {
        v.x = __builtin_nontemporal_load(g);
        v.y = __builtin_nontemporal_load(g + k);
        v.z = __builtin_nontemporal_load(g + 2 * k);
        v.w = __builtin_nontemporal_load(g + 3 * k);
      } else {
        v = (u32x4){g[0], g[k], g[2 * k], g[3 * k]};
      }
      return v;
    }
  }
}

__device__ __forceinline__ u32x4 load_global(const u32x4* p) {
  return *(const GLOBAL_AS u32x4*)p;
}

__device__ __forceinline__ uint32_t load_global(const uint32_t* p) {
  return *(const GLOBAL_AS uint32_t*)p;
}

__device__ __forceinline__ uint16_t load_global_u16(const uint16_t* p) {
  return *(const GLOBAL_AS uint16_t*)p;
}

__device__ __forceinline__ void store_global_u16(uint16_t* p, uint16_t v) {
  *(GLOBAL_AS uint16_t*)p = v;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// f32 -> f16, RNE, of the f32 value v itself.  The empty asm makes v opaque:
// otherwise the compiler may fold the multiply or add that produced v into a
// mixed-precision v_fma_mix*_f16 that rounds the exact result to f16 once,
// which differs from rounding the f32 value in rare halfway cases and differs
// between kernels depending on where it folds.
__device__ __forceinline__ _Float16 to_f16(float v) {
  asm volatile("" : "+v"(v));
  return (_Float16)v;  // v_cvt_f16_f32
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
  return __builtin_bit_cast(uint16_t, to_f16(v));
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the 16 lanes of a DPP row; every lane of the row ends with the same
// value (each step adds a lane and its mirror partner, a symmetric pairing).
__device__ __forceinline__ float reduce_row16(float v) {
#if Q8_REDUCE_DPP
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x141>(v);  // row_half_mirror
  v += dpp<0x140>(v);  // row_mirror
#else
  // the same pairs through ds_bpermute (lane ^ 1, ^ 2; then the quads and
  // half rows pair as the mirrors pair them)
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 16; d <<= 1)
    v += __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(4 * (lane ^ d),
                                                                __builtin_bit_cast(int, v)));
#endif
  return v;
}

// Dot product of one 68-byte Q8_0 block pair with 64 x values.
//   d[0..16]: the pair's 17 dwords (pair start is 4-byte aligned)
//     byte 0-1 scale0, 2-33 q0[0..31], 34-35 scale1, 36-67 q1[0..31]
//   xr[0..7]: x for the pair's 64 K positions, 8 f16 per u32x4
// Returns fma(f32(scale1), dot1, f32(scale0)*dot0) with each dot an f32 sum
// of exact int8*f16 products.
__device__ __forceinline__ float q8_pair_dot(const uint32_t (&d)[17], const u32x4 (&xr)[8]) {
#if !Q8_DEQUANT_PACKED
  // every int8 sign-extended, converted to f32 and multiplied by f32(x)
  float dots[2] = {0.0f, 0.0f};
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const int byte = 34 * blk + 2 + j;
      const int q = (int)(int8_t)(uint8_t)(d[byte >> 2] >> (8 * (byte & 3)));
      const uint32_t xw = xr[4 * blk + (j >> 3)][(j >> 1) & 3];
      const float xv = (float)as_f16x2(xw)[j & 1];
      dots[blk] = __builtin_fmaf((float)q, xv, dots[blk]);
    }
  const float s0 = f16_bits_to_f32(d[0] & 0xffffu);
  const float s1 = f16_bits_to_f32(d[8] >> 16);
  return __builtin_fmaf(s1, dots[1], s0 * dots[0]);
#else
  uint32_t e[17];
#pragma unroll
  for (int m = 0; m < 17; ++m) e[m] = d[m] ^ 0x80808080u;  // q -> q+128 per byte
  float dot0 = 0.0f, dot1 = 0.0f;
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    const int b0 = 2 + 2 * t;   // byte of q0[2t] in the pair
    const int b1 = 36 + 2 * t;  // byte of q1[2t]
    const f16x2 q0 = q8x2_to_f16x2(e[b0 >> 2], (b0 & 2) ? kSelHi : kSelLo);
    const f16x2 q1 = q8x2_to_f16x2(e[b1 >> 2], (b1 & 2) ? kSelHi : kSelLo);
    dot0 = __builtin_amdgcn_fdot2(q0, as_f16x2(xr[t >> 2][t & 3]), dot0, false);
    dot1 = __builtin_amdgcn_fdot2(q1, as_f16x2(xr[4 + (t >> 2)][t & 3]), dot1, false);
  }
  const float s0 = f16_bits_to_f32(d[0] & 0xffffu);
  const float s1 = f16_bits_to_f32(d[8] >> 16);
  return __builtin_fmaf(s1, dot1, s0 * dot0);
#endif
}

// ---------------------------------------------------------- Q8_0 GEMV ------
//
// Rows are handled in quads of 4 consecutive rows; a quad's bytes are one
// contiguous span (4 rows x K/32 blocks x 34 B).  A wave reads its span with
// fully coalesced 16-byte loads (lane l takes pieces l, l+64, ...), stages it
// in LDS and reads it back as 68-byte block pairs: lane l works on row (l >> 4)
// of the quad and pair (l & 15) of each 1024-column chunk.  HBM therefore sees
// whole 1 KiB wave requests despite the 34-byte block stride.  A row's partial
// sums stay in the lane across its K/1024 chunks and meet in a 16-lane DPP
// reduction.
//
// Batched launches split their work into units of one 1024-column chunk of a
// quad (32 blocks per row, 4352 bytes, whatever K is); a wave owns a
// contiguous range of units of a GEMV, quad-major and chunk-minor, so it
// finishes every row it starts.

constexpr int kChunkBytes = 1088;                    // 32 Q8_0 blocks
constexpr int kUnitBytes = 4 * kChunkBytes;          // 4352
constexpr int kUnitPieces = kUnitBytes / 16;         // 272
constexpr int kUnitLoads = (kUnitPieces + 63) / 64;  // 5 per lane
constexpr int kMaxP = 3;                             // K <= 3072
constexpr int kSlotBytes = kUnitLoads * 1024;        // 5120: a unit plus spare tail

struct Q8Seg {
  const uint8_t* w;  // first row of the layer
  const uint16_t* x;
  uint16_t* y;
  int n_rows;
  int p;  // K / 1024
};

// Where lane `lane`'s pieces of a unit sit: row within the quad and byte
// offset within that row's 1088-byte chunk.  The last load covers pieces
// 256..319 of which only 272 exist; lanes past the end re-read piece 271 (the
// same 16 bytes lane 15 reads) so that every load is issued by every lane and
// no load sits behind a branch, and they park the copy in the slot's spare
// tail.
struct PieceMap {
  int row[kUnitLoads];
  int off[kUnitLoads];
};

__device__ __forceinline__ PieceMap piece_map(int lane) {
  PieceMap pm;
#pragma unroll
  for (int i = 0; i < kUnitLoads; ++i) {
    int j = i * 64 + lane;
    j = j < kUnitPieces ? j : kUnitPieces - 1;
    pm.row[i] = j / 68;
    pm.off[i] = (j - (j / 68) * 68) * 16;
  }
  return pm;
}

__device__ __forceinline__ void unit_load(const Q8Seg& s, int quad, int c, const PieceMap& pm,
                                          u32x4 (&buf)[kUnitLoads]) {
  const size_t rowb = (size_t)kChunkBytes * s.p;
  const uint8_t* base = s.w + (size_t)c * kChunkBytes;
#pragma unroll
  for (int i = 0; i < kUnitLoads; ++i) {
    int row = quad * 4 + pm.row[i];
    row = row < s.n_rows ? row : s.n_rows - 1;  // ragged last quad: re-read a valid row
    buf[i] = load_weights16<Q8_NT_LOADS>(
        reinterpret_cast<const u32x4*>(base + (size_t)row * rowb + pm.off[i]));
  }
}

// Units [u_begin, u_end) of one GEMV in a batched launch (segment-local
// numbering: quad = u / p, chunk = u % p; u_begin and u_end are multiples of
// p).  Two register sets ping-pong so that while one unit is computed the
// next one is already in flight; every load inside the loop is unconditional,
// so the wait before staging a set covers only that set.
__device__ __forceinline__ void q8_segment(const Q8Seg& s, int u_begin, int u_end,
                                           uint8_t* __restrict__ slot,
                                           uint16_t* __restrict__ xl) {
  const int lane = threadIdx.x;
  const PieceMap pm = piece_map(lane);
  const int p16 = lane & 15;
  const int rsub = lane >> 4;
  u32x4* l4 = reinterpret_cast<u32x4*>(slot);

  int lq = u_begin / s.p, lc = 0;  // next unit to load
  auto load_next = [&](u32x4 (&dst)[kUnitLoads]) {
    unit_load(s, lq, lc, pm, dst);
    if (++lc == s.p) {
      lc = 0;
      ++lq;
    }
  };
  int cq = lq, cc = 0;  // next unit to compute
  float acc = 0.0f;
  u32x4 xr[8];   // x of chunk xr_c for this lane's 64 columns; for K = 1024
  int xr_c = -1;  // every unit of the GEMV reuses it
  auto compute = [&](const u32x4 (&src)[kUnitLoads]) {
#pragma unroll
    for (int i = 0; i < kUnitLoads; ++i) l4[i * 64 + lane] = src[i];
    __syncthreads();
    const uint32_t* pp = reinterpret_cast<const uint32_t*>(slot + rsub * kChunkBytes + 68 * p16);
    uint32_t d[17];
#pragma unroll
    for (int m = 0; m < 17; ++m) d[m] = pp[m];
    if (cc != xr_c || !Q8_X_REUSE) {
#if Q8_X_LDS
      const u32x4* xs = reinterpret_cast<const u32x4*>(xl + 1024 * cc + 64 * p16);
#pragma unroll
      for (int m = 0; m < 8; ++m) xr[m] = xs[m];
#else
      const u32x4* xs = reinterpret_cast<const u32x4*>(s.x + 1024 * cc + 64 * p16);
#pragma unroll
      for (int m = 0; m < 8; ++m) xr[m] = load_global(xs + m);
#endif
      xr_c = cc;
    }
    acc += q8_pair_dot(d, xr);
    if (cc == s.p - 1) {
      const float tot = reduce_row16(acc);
      const int row = cq * 4 + rsub;
      if (p16 == 0 && row < s.n_rows) store_global_u16(s.y + row, f32_to_f16_bits(tot));
      acc = 0.0f;
    }
    if (++cc == s.p) {
      cc = 0;
      ++cq;
    }
    __syncthreads();
  };

  const int n = u_end - u_begin;
#if Q8_SEG_SETS == 3
  // Three register sets: two units in flight while one is computed.  Loads
  // past the segment's last unit re-read that unit (the same lines this wave
  // just requested), so every load in the loop is unconditional.
  int loaded = 0;
  auto load_ring = [&](u32x4 (&dst)[kUnitLoads]) {
    unit_load(s, lq, lc, pm, dst);
    if (++loaded < n && ++lc == s.p) {
      lc = 0;
      ++lq;
    }
  };
  u32x4 A[kUnitLoads], B[kUnitLoads], C[kUnitLoads];
  load_ring(A);
  const u32x4* xg = reinterpret_cast<const u32x4*>(s.x);
  u32x4* xl4 = reinterpret_cast<u32x4*>(xl);
  if (Q8_X_LDS)
    for (int t = lane; t < 128 * s.p; t += 64) xl4[t] = load_global(xg + t);
  load_ring(B);
  int i = 0;
  for (; i + 3 <= n; i += 3) {
    load_ring(C);
    compute(A);
    load_ring(A);
    compute(B);
    load_ring(B);
    compute(C);
  }
  if (n - i >= 1) compute(A);
  if (n - i >= 2) compute(B);
#else
  u32x4 A[kUnitLoads], B[kUnitLoads];
  load_next(A);
  const u32x4* xg = reinterpret_cast<const u32x4*>(s.x);
  u32x4* xl4 = reinterpret_cast<u32x4*>(xl);
  if (Q8_X_LDS)
    for (int t = lane; t < 128 * s.p; t += 64) xl4[t] = load_global(xg + t);
  int i = 0;
  for (; i + 2 < n; i += 2) {
    load_next(B);
    compute(A);
    load_next(A);
    compute(B);
  }
  if (n - i == 2) {
    load_next(B);
    compute(A);
    compute(B);
  } else {
    compute(A);
  }
#endif
}

// Single GEMV: one wave per row quad, the latency-bound shape of a lone
// decode dispatch.  The wave issues all P*5 of its weight loads at once (the
// quad's 4 rows x P chunks are one contiguous span of 4*1088*P bytes), then
// its x loads (64 columns per chunk straight into registers), stages the span
// in LDS and reads it back as block pairs.
// Building blocks of the one-quad GEMV (also used by the decode-step kernels).
template <int P>
struct QuadShape {
  static constexpr int ROWB = kChunkBytes * P;
  static constexpr int PIECES = 4 * ROWB / 16;  // 272 * P
  static constexpr int LOADS = (PIECES + 63) / 64;
  static constexpr int LDS_BYTES = LOADS * 1024;
};

// Issues the loads of row quad `quad` (4 rows of P chunks, one contiguous
// span).  Pieces past the quad's valid bytes (ragged last quad, or the last
// load's spare lanes) re-read the last valid piece and land in rows or LDS
// bytes that are never consumed, so every lane issues every load.
template <int P>
__device__ __forceinline__ void q8_quad_load(const uint8_t* __restrict__ w, int n_rows, int quad,
                                             u32x4 (&buf)[QuadShape<P>::LOADS]) {
  constexpr int ROWB = QuadShape<P>::ROWB;
  const int lane = threadIdx.x & 63;
  const int row0 = quad * 4;
  int rows_here = n_rows - row0;
  rows_here = rows_here < 4 ? rows_here : 4;
  const int last = rows_here * (ROWB / 16) - 1;
  const u32x4* src = reinterpret_cast<const u32x4*>(w + (size_t)row0 * ROWB);
#pragma unroll
  for (int i = 0; i < QuadShape<P>::LOADS; ++i) {
    const int c = i * 64 + lane;
    buf[i] = load_stream<Q8_NT_LOADS>(src + (c < last ? c : last));
  }
}

template <int P>
__device__ __forceinline__ void q8_quad_stage(const u32x4 (&buf)[QuadShape<P>::LOADS],
                                              uint8_t* __restrict__ lds) {
  const int lane = threadIdx.x & 63;
  u32x4* l4 = reinterpret_cast<u32x4*>(lds);
#pragma unroll
  for (int i = 0; i < QuadShape<P>::LOADS; ++i) l4[i * 64 + lane] = buf[i];
}

// This lane's share of its row (lane >> 4) of a staged quad: the block-pair
// dots of chunks 0..P-1 added in chunk order onto 0.
template <int P>
__device__ __forceinline__ float q8_quad_lane_dot(const uint8_t* __restrict__ lds,
                                                  const u32x4 (&xr)[P][8]) {
  const int lane = threadIdx.x & 63;
  const int p16 = lane & 15;
  const int rsub = lane >> 4;
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < P; ++c) {
    const uint32_t* pp = reinterpret_cast<const uint32_t*>(lds + rsub * QuadShape<P>::ROWB +
                                                           kChunkBytes * c + 68 * p16);
    uint32_t d[17];
#pragma unroll
    for (int m = 0; m < 17; ++m) d[m] = pp[m];
    acc += q8_pair_dot(d, xr[c]);
  }
  return acc;
}

// Row sum for this lane's row (lane >> 4) of a staged quad; every lane of the
// row's 16-lane group returns the same value.
template <int P>
__device__ __forceinline__ float q8_quad_dot(const uint8_t* __restrict__ lds,
                                             const u32x4 (&xr)[P][8]) {
  return reduce_row16(q8_quad_lane_dot<P>(lds, xr));
}

// Chunk c (1024 columns) of row quad `quad` of a K = 1024 P matrix, loaded
// for staging in the one-chunk quad layout (QuadShape<1>): 4 rows of 1088
// bytes at a row stride of 1088 P.  Pieces past the last valid row re-read
// the last valid piece, as in q8_quad_load.
template <int P>
__device__ __forceinline__ void q8_chunk_load(const uint8_t* __restrict__ w, int n_rows, int quad,
                                              int c, u32x4 (&buf)[QuadShape<1>::LOADS]) {
  const int lane = threadIdx.x & 63;
  const int row0 = quad * 4;
  int rows_here = n_rows - row0;
  rows_here = rows_here < 4 ? rows_here : 4;
  const int last = rows_here * 68 - 1;
  const uint8_t* base = w + (size_t)row0 * (kChunkBytes * P) + kChunkBytes * c;
#pragma unroll
  for (int i = 0; i < QuadShape<1>::LOADS; ++i) {
    int j = i * 64 + lane;
    j = j < last ? j : last;
    const int r = j / 68;
    buf[i] = load_stream<Q8_NT_LOADS>(
        reinterpret_cast<const u32x4*>(base + (size_t)r * (kChunkBytes * P) + 16 * (j - 68 * r)));
  }
}

// x for this lane's 64 columns of each chunk straight from global memory.
template <int P>
__device__ __forceinline__ void load_x_cols(const uint16_t* __restrict__ x, u32x4 (&xr)[P][8]) {
  const int p16 = threadIdx.x & 15;
#pragma unroll
  for (int c = 0; c < P; ++c) {
    const u32x4* xs = reinterpret_cast<const u32x4*>(x + 1024 * c + 64 * p16);
#pragma unroll
    for (int m = 0; m < 8; ++m) xr[c][m] = load_global(xs + m);
  }
}

// Single GEMV, one wave per row quad: all of the quad's weight loads are in
// flight before XLoad fetches x (xr[c] = this lane's 64 columns of chunk c);
// Epi(row, acc) runs on one lane per valid row.
// Returns the row sum of this lane's row (row quad*4 + lane/16) in all 16
// lanes of its row group.
template <int P, class XLoad>
__device__ __forceinline__ float q8_quad_core_acc(const uint8_t* __restrict__ w, int n_rows,
                                                  int quad, uint8_t* __restrict__ lds,
                                                  XLoad&& xload) {
  u32x4 buf[QuadShape<P>::LOADS];
  q8_quad_load<P>(w, n_rows, quad, buf);
  u32x4 xr[P][8];
  xload(xr);
  q8_quad_stage<P>(buf, lds);
  __syncthreads();
  return q8_quad_dot<P>(lds, xr);
}

template <int P, class XLoad, class Epi>
__device__ __forceinline__ void q8_quad_core(const uint8_t* __restrict__ w, int n_rows, int quad,
                                             uint8_t* __restrict__ lds, XLoad&& xload,
                                             Epi&& epi) {
  const float acc = q8_quad_core_acc<P>(w, n_rows, quad, lds, xload);
  const int lane = threadIdx.x & 63;
  const int row = quad * 4 + (lane >> 4);
  if ((lane & 15) == 0 && row < n_rows) epi(row, acc);
}

template <int P>
__device__ __forceinline__ void q8_quad(const uint8_t* __restrict__ w,
                                        const uint16_t* __restrict__ x,
                                        uint16_t* __restrict__ y, int n_rows, int quad,
                                        uint8_t* __restrict__ lds) {
  q8_quad_core<P>(w, n_rows, quad, lds, [&](u32x4 (&xr)[P][8]) { load_x_cols<P>(x, xr); },
                  [&](int row, float acc) { y[row] = f32_to_f16_bits(acc); });
}

// Device table of a batched launch: a 16-byte header, then one entry per GEMV
// in the order the caller listed them.  unit_begin is the exclusive prefix sum
// of ceil(n_rows / 4) * p.
struct Q8BatchEntry {
  const uint8_t* w;
  const uint16_t* x;
  uint16_t* y;
  int32_t n_rows;
  int32_t p;
  int32_t unit_begin;
  int32_t reserved;
};
static_assert(sizeof(Q8BatchEntry) == 40, "batch entry layout");
constexpr int kBatchHeaderBytes = 16;

// ------------------------------------------------------------ vocab ------

// Workspace: one u64 argmax key (below), zero between launches.  Every
// workgroup folds its best (value, index) into it with a 64-bit atomic max;
// vocab_argmax_finalize turns the key into the token and zeroes it again.
// Atomics on one location need no fences, so no workgroup pays for an L2
// writeback or invalidate.

// Order-preserving key of a candidate (f16 value v at row i >= 0): the high
// word maps the f16 bit pattern to an unsigned order (-0 folded onto +0, so
// the two tie), the low word is ~i so that equal values prefer the lower row.
// Every candidate key is >= 2^42 (its value is > -inf); 0 means "none".
__device__ __forceinline__ uint64_t argmax_key(float v, int i) {
  uint32_t h = f32_to_f16_bits(v);  // exact: v is an f16 value
  if (h == 0x8000u) h = 0u;
  const uint32_t ord = (h & 0x8000u) ? (~h & 0xffffu) : (h | 0x8000u);
  return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
}

// (v, i) beats (bv, bi): a larger value, or an equal value at a lower index.
// Ordered compares, so NaN never wins; -0 == +0 ties.  A candidate whose value
// is -inf always carries index -1 (nothing was selected), so it never beats
// the initial (-inf, -1).
__device__ __forceinline__ bool argmax_better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// acc + sum of the 8 products w[j]*xv[j] (4 x v_dot2_f32_f16; products exact in f32).
__device__ __forceinline__ float f16_row_dot(const u32x4& w, const u32x4& xv, float acc) {
  acc = __builtin_amdgcn_fdot2(as_f16x2(w[0]), as_f16x2(xv[0]), acc, false);
  acc = __builtin_amdgcn_fdot2(as_f16x2(w[1]), as_f16x2(xv[1]), acc, false);
  acc = __builtin_amdgcn_fdot2(as_f16x2(w[2]), as_f16x2(xv[2]), acc, false);
  acc = __builtin_amdgcn_fdot2(as_f16x2(w[3]), as_f16x2(xv[3]), acc, false);
  return acc;
}

// xload(li, xr) of vocab_body_xp; one that returns false (its input never
// arrived) makes the function return without computing or storing a row.
template <class XLoad>
__device__ __forceinline__ bool vocab_xload(XLoad& xload, int li, u32x4 (&xr)[8]) {
  if constexpr (__is_same(decltype(xload(li, xr)), bool)) {
    return xload(li, xr);
  } else {
    xload(li, xr);
    return true;
  }
}

// f16 GEMV rows [0, n_rows) x K=1024 with a fused argmax.
//
// Rows are taken in batches of 4.  Within a wave, DPP row g (lanes 16g..16g+15)
// owns matrix row 4b+g of batch b: lane i of the group reads bytes
// [256m + 16i, 256m + 16i + 16) of that row for m = 0..7, so each wave load
// instruction covers four fully used 256-byte row segments, and the group's
// partial sums meet in a 16-lane DPP reduction (no cross-row exchange).  The
// lane keeps its 64 x values (positions 128m + 8i .. +8) in registers for all
// rows.  Global wave w owns the contiguous batches [w*B/TW, (w+1)*B/TW); the
// next batch's loads are issued unconditionally before the current batch is
// reduced, so every wave keeps 8 KiB of weights in flight.
//
// Argmax: each logit is rounded to f16 first (the reference compares the f16
// logits tensor).  Per group the rows arrive in increasing order, so a
// strictly-greater update keeps the first maximum; the 16 groups of a
// workgroup are merged with argmax_better, and workgroups meet in a 64-bit
// atomic max over argmax_key, whose order is the same rule.
// The workgroup's result reaches publish(key) on thread 0: key =
// argmax_key(best) or 0 when the workgroup saw no candidate.
// The rows are split over workgroups 0 .. groups - 1 (the whole grid unless a
// caller runs the GEMV on only the first `groups` workgroups), evenly unless
// heavy_wgs > 0: then each wave of workgroups 0 .. heavy_wgs - 1 takes
// heavy_w16 / 16 times the share of a wave of the others (for a caller whose
// later workgroups share their CUs with earlier, faster ones).
//
// PRE > 0 (for a caller whose x arrives late): the wave's last PRE batches go
// straight into its LDS area stage + wave * PRE * 8 KiB (global_load_lds; load
// m of batch s lands at + 8 KiB s + 1 KiB m + 16 lane) and its first two into
// registers, all before xload, so 2 + PRE batches stream in while x is
// awaited; the staged batches are consumed last, which keeps every group's
// rows in increasing order.  Every wave must own at least PRE + 2 batches (the
// caller checks its sizes), and the workgroup must not use the stage area
// until the function returns.
template <bool NT, bool ARGMAX, int PRE = 0, class XLoad, class Publish>
__device__ __forceinline__ void vocab_body_xp(const uint16_t* __restrict__ W, XLoad&& xload,
                                              uint16_t* __restrict__ logits, int n_rows,
                                              Publish&& publish, int groups = -1,
                                              uint8_t* stage = nullptr, int heavy_wgs = 0,
                                              int heavy_w16 = 16) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int grp = lane >> 4;
  const int li = lane & 15;
  // full waves of the grid (a partial last wave of an odd-sized workgroup
  // takes no rows)
  const int64_t wpb = launch_wg_size() >> 6;
  const int64_t gw = (int64_t)blockIdx.x * wpb + wave;
  const int64_t tw = (int64_t)(groups > 0 ? groups : (int)launch_wgs()) * wpb;
  const int64_t nbatch = ((int64_t)n_rows + 3) / 4;
  // a wave of workgroups 0 .. heavy_wgs - 1 takes heavy_w16 / 16 times the
  // batches of any other wave
  const int64_t hw = (int64_t)heavy_wgs * wpb;
  auto cum = [&](int64_t w) { return w <= hw ? w * heavy_w16 : hw * heavy_w16 + (w - hw) * 16; };
  const int64_t tot = cum(tw);
  const int b_begin = wave < wpb ? (int)(cum(gw) * nbatch / tot) : 0;
  const int b_end = wave < wpb ? (int)(cum(gw + 1) * nbatch / tot) : 0;

  const u32x4* Wv = reinterpret_cast<const u32x4*>(W);
  u32x4 xr[8];  // this lane's x columns, formed by xload below
  auto load_batch = [&](int b, u32x4 (&dst)[8]) {
    int row = 4 * b + grp;
    row = row < n_rows ? row : n_rows - 1;  // only the grid's last batch can be short
    const u32x4* p = Wv + (size_t)row * 128 + li;
#pragma unroll
    for (int m = 0; m < 8; ++m) dst[m] = load_weights16<NT>(p + 16 * m);
  };

  float best_v = -__builtin_inff();
  int best_i = -1;
  auto consume = [&](int b, const u32x4 (&w)[8]) {
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int m = 0; m < 8; m += 2) {
      a0 = f16_row_dot(w[m], xr[m], a0);
      a1 = f16_row_dot(w[m + 1], xr[m + 1], a1);
    }
    const float acc = reduce_row16(a0 + a1);
    const int row = 4 * b + grp;
    const uint16_t hb = f32_to_f16_bits(acc);
    if (row < n_rows) {
      if (logits != nullptr && li == 0) logits[row] = hb;
      if constexpr (ARGMAX) {
        const float hv = f16_bits_to_f32(hb);
        if (hv > best_v) {
          best_v = hv;
          best_i = row;
        }
      }
    }
  };

  // The first batch is requested before x is formed (x may need loads and
  // a reduction of its own); rows are clamped, so this is safe even for a
  // wave with no batch.  Then ping-pong between two register sets; every
  // load inside the loop is unconditional, so the compiler can wait for
  // exactly the older set.
  u32x4 A[8], B[8];
  const int nb = b_end - b_begin;
  if constexpr (PRE > 0) {
    const int nr = nb - PRE;  // batches read through registers, >= 2
    uint8_t* ws = stage + (size_t)wave * (PRE * 8192);
    load_batch(b_begin, A);
    load_batch(b_begin + 1, B);
#pragma unroll
    for (int s = 0; s < PRE; ++s) {
      int row = 4 * (b_begin + nr + s) + grp;
      row = row < n_rows ? row : n_rows - 1;
      const u32x4* p = Wv + (size_t)row * 128 + li;
#pragma unroll
      for (int m = 0; m < 8; ++m)
        __builtin_amdgcn_global_load_lds((const GLOBAL_AS void*)(p + 16 * m),
                                         (__attribute__((address_space(3))) void*)(ws + 8192 * s +
                                                                                   1024 * m),
                                         16, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (!vocab_xload(xload, li, xr)) {
      wait_vm<0>();  // the staged rows land before the workgroup ends
      return;
    }
    // A holds batch i, B batch i + 1 (loads in flight) at the top of each round
    int i = 0;
    for (; i + 3 < nr; i += 2) {
      consume(b_begin + i, A);
      load_batch(b_begin + i + 2, A);
      consume(b_begin + i + 1, B);
      load_batch(b_begin + i + 3, B);
    }
    if (nr - i == 3) {
      consume(b_begin + i, A);
      load_batch(b_begin + i + 2, A);
      consume(b_begin + i + 1, B);
      consume(b_begin + i + 2, A);
    } else {
      consume(b_begin + i, A);
      consume(b_begin + i + 1, B);
    }
    wait_vm<0>();  // the staged batches have landed in LDS
#pragma unroll
    for (int s = 0; s < PRE; ++s) {
      u32x4 w[8];
#pragma unroll
      for (int m = 0; m < 8; ++m)
        w[m] = *reinterpret_cast<const u32x4*>(ws + 8192 * s + 1024 * m + 16 * lane);
      consume(b_begin + nr + s, w);
    }
  } else {
    load_batch(b_begin, A);
    __builtin_amdgcn_sched_barrier(0);
    if (!vocab_xload(xload, li, xr)) {
      wait_vm<0>();
      return;
    }
    if (nb > 0) {
      int i = 0;
      for (; i + 2 < nb; i += 2) {
        load_batch(b_begin + i + 1, B);
        consume(b_begin + i, A);
        load_batch(b_begin + i + 2, A);
        consume(b_begin + i + 1, B);
      }
      if (nb - i == 2) {
        load_batch(b_begin + i + 1, B);
        consume(b_begin + i, A);
        consume(b_begin + i + 1, B);
      } else {
        consume(b_begin + i, A);
      }
    }
  }

  if constexpr (!ARGMAX) return;

  // ---- workgroup combine: 4 waves x 4 row groups, then one atomic ----
  __shared__ float s_val[16];
  __shared__ int s_idx[16];
  if (li == 0) {
    s_val[wave * 4 + grp] = best_v;
    s_idx[wave * 4 + grp] = best_i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float bv = -__builtin_inff();
    int bi = -1;
    for (int c = 0; c < 16; ++c) {
      if (argmax_better(s_val[c], s_idx[c], bv, bi)) {
        bv = s_val[c];
        bi = s_idx[c];
      }
    }
    publish(bi >= 0 ? argmax_key(bv, bi) : (uint64_t)0);
  }
}

// Workgroups meet in one 64-bit atomic max on ws[0].
template <bool NT, bool ARGMAX, class XLoad>
__device__ __forceinline__ void vocab_body_x(const uint16_t* __restrict__ W, XLoad&& xload,
                                             uint16_t* __restrict__ logits, int n_rows,
                                             uint8_t* __restrict__ ws) {
  vocab_body_xp<NT, ARGMAX>(W, xload, logits, n_rows, [&](uint64_t key) {
    if (key != 0)
      __hip_atomic_fetch_max(reinterpret_cast<uint64_t*>(ws), key, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  });
}

// x for lane i of a row group: positions 128m + 8i .. +8, m = 0..7.
template <bool NT, bool ARGMAX>
__device__ __forceinline__ void vocab_body(const uint16_t* __restrict__ W,
                                           const uint16_t* __restrict__ x,
                                           uint16_t* __restrict__ logits, int n_rows,
                                           uint8_t* __restrict__ ws) {
  vocab_body_x<NT, ARGMAX>(
      W,
      [&](int li, u32x4 (&xr)[8]) {
        const u32x4* xv = reinterpret_cast<const u32x4*>(x);
#pragma unroll
        for (int m = 0; m < 8; ++m) xr[m] = load_global(xv + 16 * m + li);
      },
      logits, n_rows, ws);
}

}  // namespace

#endif
