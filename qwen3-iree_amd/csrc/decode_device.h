// Device code shared by the decode-step kernels (decode_kernels.hip): the
// launch-per-phase kernels and the single-launch (persistent) step call the
// same functions, so both paths compute every value with the same operations
// in the same order.  Header-only, internal to the including translation unit.
#ifndef QWEN3_DECODE_DEVICE_H
#define QWEN3_DECODE_DEVICE_H

#include "q8_device.h"

namespace {

constexpr int kLayers = 28;
constexpr int kHidden = 1024;
constexpr int kHeadDim = 128;
constexpr int kKvHeads = 8;
constexpr int kQHeads = 16;
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
// attention scores in base-2 units: s log2(e), so each weight is one exp2
constexpr float kScoreScaleLog2 = kAttnScale * 1.44269504088896341f;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef short v8i16 __attribute__((ext_vector_type(8)));
#define LDS_AS __attribute__((address_space(3)))

// Lane exchanges through v_permlane16_swap / v_permlane32_swap (VALU, no LDS
// round trip).  With both operands v, permlane16_swap returns {v of rows 0, 0,
// 2, 2; v of rows 1, 1, 3, 3} and permlane32_swap {v of lanes i & 31; v of
// lanes 32 + (i & 31)}: every lane holds its own value and its partner's.
__device__ __forceinline__ float sum_rows2(float v) {  // rows 2k and 2k + 1: r_2k + r_2k+1
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}
__device__ __forceinline__ float sum_halves(float v) {  // lanes i and i ^ 32: v_lo + v_hi
  auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(a[0]) + __uint_as_float(a[1]);
}
__device__ __forceinline__ float xor32(float v) {  // the value of lane i ^ 32
  auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 32) ? a[0] : a[1]);
}

// the sum of v over lanes i, i ^ 16, i ^ 32, i ^ 48: (r0 + r1) + (r2 + r3) for
// the values r of the wave's four DPP rows, in every lane (fp addition is
// commutative, so a lane adding its partner's value to its own or the other
// way round gets the same bits)
__device__ __forceinline__ float sum_col4(float v) { return sum_halves(sum_rows2(v)); }

// the sum over the wave: rows in index order, (r0 + r1) + (r2 + r3)
__device__ __forceinline__ float wave_sum(float v) { return sum_col4(reduce_row16(v)); }

// the max of v over lanes i, i ^ 16, i ^ 32, i ^ 48 (v_permlane16_swap /
// v_permlane32_swap hand each lane the value of its partner row; sum_col4 is
// the sum).  Both results of each swap are used; the generated code was
// checked for that (a swap whose second result is dropped reduces nothing),
// and the attention tests against the oracle would fail on any lane seeing a
// different max.
__device__ __forceinline__ float max_col4(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// f16(a) | f16(b) << 16, each rounded to nearest even (one v_cvt_pk_f16_f32);
// the opaque copy keeps the compiler from folding a preceding multiply into a
// single-rounding mixed-precision op, as to_f16 does
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  asm volatile("" : "+v"(a), "+v"(b));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, f16x2));
}

__device__ __forceinline__ _Float16 as_half(uint16_t b) { return __builtin_bit_cast(_Float16, b); }

__device__ __forceinline__ uint2 load_global(const uint2* p) {
  const uint64_t v = *(const GLOBAL_AS uint64_t*)p;
  return make_uint2((uint32_t)v, (uint32_t)(v >> 32));
}

// rms_norm (qwen3_full.mlir:134-165).  Every kernel sums the 1024 squares in
// one canonical order, a perfect binary tree over the columns in index order
// with the leaves fl(x^2), so a vector normalized by the 16 lanes of a row
// (rmsnorm_apply) or by a whole workgroup (rmsnorm_wg) gives the same bits.

// the tree over columns 4k .. 4k + 3 (two f16 pairs): (q0 + q1) + (q2 + q3)
__device__ __forceinline__ float sq_tree4(uint32_t lo, uint32_t hi) {
  const f16x2 a = as_f16x2(lo), b = as_f16x2(hi);
  const float a0 = (float)a.x, a1 = (float)a.y, b0 = (float)b.x, b1 = (float)b.y;
  return (a0 * a0 + a1 * a1) + (b0 * b0 + b1 * b1);  // contraction is off: each term rounded
}

// x = f16((h inv) w) for an f16 pair of h and of w, packed
__device__ __forceinline__ uint32_t norm_pair(uint32_t h2, uint32_t w2, float inv) {
  const f16x2 hp = as_f16x2(h2), wp = as_f16x2(w2);
  return pack_f16x2(((float)hp.x * inv) * (float)wp.x, ((float)hp.y * inv) * (float)wp.y);
}

__device__ __forceinline__ float rms_inv(float ss) { return 1.0f / sqrtf(ss / 1024.0f + kEps); }

// The 64 columns this lane holds, contiguous (hv: the values, wv: the norm
// weights, 8 per u32x4): the lane's subtree over them, then the 16 lanes of
// its DPP row (reduce_row16 pairs lanes as a perfect tree in index order, fp
// addition being commutative), so the row must hold the vector's columns in
// lane order.
__device__ __forceinline__ void rmsnorm_apply(const u32x4 (&hv)[8], const u32x4 (&wv)[8],
                                              u32x4 (&xr)[8]) {
  float gs[16];
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    gs[2 * m] = sq_tree4(hv[m][0], hv[m][1]);
    gs[2 * m + 1] = sq_tree4(hv[m][2], hv[m][3]);
  }
#pragma unroll
  for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
    for (int i = 0; i < w; ++i) gs[i] = gs[2 * i] + gs[2 * i + 1];
  const float inv = rms_inv(reduce_row16(gs[0]));
#pragma unroll
  for (int m = 0; m < 8; ++m)
#pragma unroll
    for (int j = 0; j < 4; ++j) xr[m][j] = norm_pair(hv[m][j], wv[m][j], inv);
}

// rms_norm of a 1024-vector by a workgroup of 256 threads: thread t holds
// columns 4t .. 4t + 3 (hv: their f16 values, w4: their norm weights) and gets
// their x.  The thread's subtree, its DPP row (64 columns), the wave's four
// rows, then the four waves' sums through red[4] in LDS.  Every thread of the
// workgroup calls it; one barrier.  The caller keeps red from being written
// again before every thread has read it (a barrier between two calls that
// share it).
__device__ __forceinline__ uint2 rmsnorm_wg(uint2 hv, uint2 w4, float* red) {
  const int t = threadIdx.x;
  const float v = sum_col4(reduce_row16(sq_tree4(hv.x, hv.y)));
  if ((t & 63) == 0) red[t >> 6] = v;
  __syncthreads();
  const float inv = rms_inv((red[0] + red[1]) + (red[2] + red[3]));
  return (uint2){norm_pair(hv.x, w4.x, inv), norm_pair(hv.y, w4.y, inv)};
}

// this thread's four norm weights for rmsnorm_wg
__device__ __forceinline__ uint2 norm_weights4(const uint16_t* __restrict__ w) {
  return load_global(reinterpret_cast<const uint2*>(w) + threadIdx.x);
}

// The loads of q8_quad_load<P> / q8_chunk_load<P> as copies from memory
// straight into LDS (global_load_lds, 16 bytes per lane and instruction): load
// i of lane l lands at lds + 1024 i + 16 l, the layout q8_quad_stage writes,
// so q8_quad_lane_dot reads the staged quad from there.  No register holds the
// data while it is in flight; `lds` must be wave-uniform.  The wave may read
// the bytes once its vector memory counter has drained past these loads (the
// compiler waits for that before the wave's next LDS access).  PACE > 0
// sleeps 64 PACE cycles after each 1 KiB piece, so hundreds of workgroups
// prefetching at once spread their requests instead of filling the memory
// queues in one burst (which delays every hand-off in flight at that time).
template <int P, int PACE = 0>
__device__ __forceinline__ void q8_quad_prefetch(const uint8_t* __restrict__ w, int n_rows,
                                                 int quad, uint8_t* lds) {
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
    __builtin_amdgcn_global_load_lds((const GLOBAL_AS void*)(src + (c < last ? c : last)),
                                     (__attribute__((address_space(3))) void*)(lds + 1024 * i),
                                     16, 0, 0);
    if constexpr (PACE > 0) __builtin_amdgcn_s_sleep(PACE);
  }
}

template <int P, int PACE = 0>
__device__ __forceinline__ void q8_chunk_prefetch(const uint8_t* __restrict__ w, int n_rows,
                                                  int quad, int c, uint8_t* lds) {
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
    __builtin_amdgcn_global_load_lds(
        (const GLOBAL_AS void*)(base + (size_t)r * (kChunkBytes * P) + 16 * (j - 68 * r)),
        (__attribute__((address_space(3))) void*)(lds + 1024 * i), 16, 0, 0);
    if constexpr (PACE > 0) __builtin_amdgcn_s_sleep(PACE);
  }
}

// The Q8_0 GEMV lane layout: columns [64 p16, 64 p16 + 64) in 8 pieces of 8.
__device__ __forceinline__ int gemv_col(int m) { return 64 * (threadIdx.x & 15) + 8 * m; }

// rms_norm of the 1024-vector h (global memory, or LDS for H_LDS) by the 16
// lanes of each DPP row, in their GEMV columns: every row gets the whole x.
template <bool H_LDS>
__device__ __forceinline__ void rmsnorm_gemv_x(const uint16_t* __restrict__ h,
                                               const uint16_t* __restrict__ w, u32x4 (&xr)[8]) {
  u32x4 hv[8], wv[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    if constexpr (H_LDS) hv[m] = *reinterpret_cast<const u32x4*>(h + gemv_col(m));
    else hv[m] = load_global(reinterpret_cast<const u32x4*>(h + gemv_col(m)));
    wv[m] = load_global(reinterpret_cast<const u32x4*>(w + gemv_col(m)));
  }
  rmsnorm_apply(hv, wv, xr);
}

// rms_norm by the workgroup (rmsnorm_wg) with x written over the 1024-vector
// in LDS (vec: 512 words of f16 pairs, thread t's h4 the pair of words 2t,
// 2t + 1), then this lane's GEMV columns of x read back.  Ends with the
// barrier that makes x visible; whatever writes vec next must first wait
// for every thread's reads.
__device__ __forceinline__ void norm_to_vec(uint2 h4, uint2 w4, uint32_t* vec, float* red,
                                            u32x4 (&xr)[8]) {
  const uint2 x = rmsnorm_wg(h4, w4, red);
  reinterpret_cast<uint2*>(vec)[threadIdx.x] = x;
  __syncthreads();
  const uint16_t* xs = reinterpret_cast<const uint16_t*>(vec);
#pragma unroll
  for (int m = 0; m < 8; ++m) xr[m] = *reinterpret_cast<const u32x4*>(xs + gemv_col(m));
}

// x for this lane's GEMV columns of chunk c, from an f16 vector in LDS.
template <int P>
__device__ __forceinline__ void lds_x_cols(const uint16_t* __restrict__ x, u32x4 (&xr)[P][8]) {
  const int p16 = threadIdx.x & 15;
#pragma unroll
  for (int c = 0; c < P; ++c) {
    const u32x4* xs4 = reinterpret_cast<const u32x4*>(x + 1024 * c + 64 * p16);
#pragma unroll
    for (int m = 0; m < 8; ++m) xr[c][m] = xs4[m];
  }
}

// SwiGLU of qwen3_full.mlir:829-839, every op in f16: e = exp(-g),
// den = 1 + e, sig = 1 / den, silu = g * sig, out = silu * up (exp and the
// reciprocal evaluated in f32 and rounded once).
__device__ __forceinline__ uint16_t swiglu_f16(float gate_acc, float up_acc) {
  const _Float16 g = to_f16(gate_acc);
  const _Float16 u = to_f16(up_acc);
  const _Float16 e = to_f16(expf(-(float)g));
  const _Float16 den = (_Float16)1.0f + e;
  const _Float16 sig = to_f16(1.0f / (float)den);
  const _Float16 silu = g * sig;
  return __builtin_bit_cast(uint16_t, (_Float16)(silu * u));
}

// f16(base + f16(acc)): the residual adds of qwen3_full.mlir:801-805, 858-862.
__device__ __forceinline__ uint16_t residual_f16(_Float16 base, float acc) {
  return __builtin_bit_cast(uint16_t, (_Float16)(base + to_f16(acc)));
}

// Weights of the 8 split-group partials of one query head: w_g = 2^(m_g -
// max m) (the maxima are in base-2 units; 0 for an empty group), L = sum_g l_g w_g, summed in group order.
__device__ __forceinline__ void merge_weights(const float (&m)[kAttnGroups],
                                              const float (&l)[kAttnGroups],
                                              float (&w)[kAttnGroups], float& L) {
  float M = -__builtin_inff();
#pragma unroll
  for (int g = 0; g < kAttnGroups; ++g) M = fmaxf(M, m[g]);
  L = 0.0f;
#pragma unroll
  for (int g = 0; g < kAttnGroups; ++g) {
    w[g] = m[g] == -__builtin_inff() ? 0.0f : exp2f(m[g] - M);
    L = L + l[g] * w[g];
  }
}

// One merged output dim: sum_g acc_g w_g in group order.
__device__ __forceinline__ float merge_dim(const float (&acc)[kAttnGroups],
                                           const float (&w)[kAttnGroups]) {
  float a = 0.0f;
#pragma unroll
  for (int g = 0; g < kAttnGroups; ++g) a = a + acc[g] * w[g];
  return a;
}

// RoPE angles for this lane's dims 2*lane + dd at position pos
// (qwen3_full.mlir:324-454): theta = pos * (1e6^(-(2i/128)) * 1), i = d mod 64.
// They depend on the position only, so a step computes them once for all
// layers.
// cos and sin of the angle of frequency i (0..63) at position pos.
__device__ __forceinline__ void rope_angle(int pos, int i, float& c, float& s) {
  const float e = -((2.0f * (float)i) / 128.0f);
  const float th = (float)pos * (powf(kRopeBase, e) * 1.0f);
  c = cosf(th);
  s = sinf(th);
}

__device__ __forceinline__ void rope_angles(int pos, float (&cs)[2], float (&sn)[2]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int dd = 0; dd < 2; ++dd) rope_angle(pos, (2 * lane + dd) & 63, cs[dd], sn[dd]);
}

// Position range [start, end) of attention split s (of kAttnSplits) over ctx
// = pos + 1 positions, and the last row a clamped load may touch.
struct SplitRange {
  int start, end, last;
};
__device__ __forceinline__ SplitRange split_range(int s, int pos) {
  const int ctx = pos + 1;
  SplitRange r;
  r.start = (int)((int64_t)s * ctx / kAttnSplits);
  r.end = (int)((int64_t)(s + 1) * ctx / kAttnSplits);
  r.last = r.end - 1 > 0 ? r.end - 1 : 0;
  return r;
}

// Bytes of one wave's staged chunk of 32 cache rows: K (8 KiB) then V (8 KiB).
constexpr int kKvPrefetchBytes = 8 * 1024 + 32 * 256;

// One chunk of a split's cache rows -- positions c0 .. c0 + 31, clamped to
// `last` -- copied into the wave's LDS region kv by the memory system
// (global_load_lds), so no register holds them while they are in flight: K
// row r's 16-byte chunk ch (dims 8 ch .. + 7) lands at kv + 256 r + 16 (ch ^
// (r & 15)), V row r's chunk ch at kv + 8192 + 256 r + 16 (ch ^ 2 (r & 7)) (so
// the score reads and the transposing reads of attention_group hit distinct
// banks): each load covers four whole rows, the lane whose 16 bytes land in
// slot j of row r loading chunk j ^ (r & 15) (K) or j ^ 2 (r & 7) (V).  (K used
// to land at kv + 1024 (ch & 7) + 512 (ch >> 3) + 16 r, each load taking 16
// bytes of every row: 64 lines per load, each touched by all eight.)  The K part
// is 8 loads per lane, the V part 8, in that order; the compiler does not
// track these copies for the LDS reads that follow, so readers wait on the
// vector memory counter themselves (wait_vm) and let every LDS read of the
// region return (wait_lds) before the region is staged again.  PACE > 0
// sleeps 64 PACE cycles after the K pieces and after every V load (four
// rows).  (The V part was 32 loads of 4 bytes per lane, each lane taking the
// four bytes of its slot; the same bytes land in the same places.)
template <int PACE = 0>
__device__ __forceinline__ void kv_stage_k(uint8_t* kv, const uint16_t* __restrict__ k_cache,
                                           int g, int c0, int last) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 4 * i + (lane >> 4);  // this lane's row; its 16 bytes land in slot lane % 16
    const int pr = c0 + r < last ? c0 + r : last;
    const int ch = (lane & 15) ^ (r & 15);
    __builtin_amdgcn_global_load_lds(
        (const GLOBAL_AS void*)(reinterpret_cast<const u32x4*>(
                                    k_cache + ((size_t)pr * kKvHeads + g) * kHeadDim) +
                                ch),
        (__attribute__((address_space(3))) void*)(kv + 1024 * i), 16, 0, 0);
  }
  if constexpr (PACE > 0) __builtin_amdgcn_s_sleep(PACE);
}

template <int PACE = 0>
__device__ __forceinline__ void kv_stage_v(uint8_t* kv, const uint16_t* __restrict__ v_cache,
                                           int g, int c0, int last) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 4 * i + (lane >> 4);  // this lane's row; its 16 bytes land in slot lane % 16
    const int pr = c0 + r < last ? c0 + r : last;
    const int ch = (lane & 15) ^ (2 * (r & 7));
    __builtin_amdgcn_global_load_lds(
        (const GLOBAL_AS void*)(reinterpret_cast<const u32x4*>(
                                    v_cache + ((size_t)pr * kKvHeads + g) * kHeadDim) +
                                ch),
        (__attribute__((address_space(3))) void*)(kv + 8192 + 1024 * i), 16, 0, 0);
    if constexpr (PACE > 0) __builtin_amdgcn_s_sleep(PACE);
  }
}

template <int PACE = 0>
__device__ __forceinline__ void kv_stage(uint8_t* kv, const uint16_t* __restrict__ k_cache,
                                         const uint16_t* __restrict__ v_cache, int g, int c0,
                                         int last) {
  kv_stage_k<PACE>(kv, k_cache, g, c0, last);
  kv_stage_v<PACE>(kv, v_cache, g, c0, last);
}

// One chunk of a split's cache rows (positions c0 .. c0 + 31, clamped to
// last) brought into the caches without being kept: lane l touches 4 bytes of
// the 128-byte half row l % 2 of row l / 2, of K and then of V, by an LDS-DMA
// into the wave's 256-byte region `sink` (never read), so no register waits
// on the loads.
__device__ __forceinline__ void kv_touch(uint8_t* sink, const uint16_t* __restrict__ k_cache,
                                         const uint16_t* __restrict__ v_cache, int g, int c0,
                                         int last) {
  const int lane = threadIdx.x & 63;
  const int r = lane >> 1;
  const int p = c0 + r < last ? c0 + r : last;
  const size_t off = ((size_t)p * kKvHeads + g) * kHeadDim + 64 * (lane & 1);
  __builtin_amdgcn_global_load_lds((const GLOBAL_AS void*)(k_cache + off), (LDS_AS void*)sink, 4,
                                   0, 0);
  __builtin_amdgcn_global_load_lds((const GLOBAL_AS void*)(v_cache + off), (LDS_AS void*)sink, 4,
                                   0, 0);
}

// The first chunk of split r (what attention_group reads first).
template <int PACE = 0>
__device__ __forceinline__ void kv_prefetch(uint8_t* kv, const uint16_t* __restrict__ k_cache,
                                            const uint16_t* __restrict__ v_cache, int g,
                                            const SplitRange& r) {
  kv_stage<PACE>(kv, k_cache, v_cache, g, r.start, r.last);
}

// LDS of one attention workgroup.
struct __attribute__((aligned(16))) AttnLds {
  uint32_t qh[2][64];  // roped q_A, q_B as f16 pairs
  uint32_t kh[64];     // roped new k as f16 pairs
  float mrg[kAttnWaves][2][4 + kHeadDim];  // per wave and q head: m, l, 2 pad, o[128]
};

// Attention for kv head g and split group sg: four waves, wave w taking
// position split s = 4 sg + w of the 32 equal splits of ctx = pos + 1; the
// four results merge in LDS into one partial per query head and group.  Per
// wave:
//  0. the split's cache rows go through the wave's LDS region kv
//     (kKvPrefetchBytes, kv_stage) 32 at a time; the first chunk is staged
//     before q/k/v are fetched (get_qkv), so its latency overlaps that wait
//     and steps 1-2, or was staged by the caller long before (kv_staged:
//     kv_prefetch);
//  1. waves 0, 1, 2 take q head 2g, q head 2g+1 and k head g: per-head
//     rms_norm with q_norm / k_norm (qwen3_full.mlir:648-702), then RoPE
//     (:324-454) at position pos, shared with the other waves through LDS;
//  2. the workgroup whose splits hold position pos writes the roped k (wave
//     2) and the raw v (wave 3) to cache slot pos (k_cache / v_cache: the
//     layer's base; slot layout [max_seq, 8, 128]); split group 0 stores the
//     roped q heads to q_roped when it is not null;
//  3. chunks of 32 positions on the matrix cores, both q heads at once as two
//     columns of the MFMA's B operand: scores S^T = K Q^T in f32 from exact
//     f16 products, s_j = (q . k_j) * rsqrt(128) log2(e) (base-2 units);
//     online softmax; O^T += V^T P^T with p as f16 hi + lo.  A wave runs its
//     chunks without waiting for the others;
//  4. publish(hh, m, l, a0, a1) on waves 0 and 1 (query head 2g + hh): m =
//     max over the 4 waves (base 2), l and this lane's two dims rescaled by
//     2^(m_w - m).  An empty split (ctx < 32) contributes m = -inf, l = 0.
// get_qkv(xw, v_new) fills this lane's words (dims 2*lane, 2*lane+1) of q
// head 2g, q head 2g+1, k head g (xw[0..2]) and v head g; every thread of the
// workgroup calls it once, and pre_qkv() once before any load of this
// function (where get_qkv's requests can start early).
// cs, sn: rope_angles of the clamped position.
// stamp(k) marks points 16-20 for a timestamp build (NoStamp: nothing).
struct NoStamp {
  __device__ void operator()(int) const {}
};
template <class PreQKV, class GetQKV, class Publish, class Stamp = NoStamp>
__device__ __forceinline__ void attention_group(AttnLds& L, int g, int sg, int pos_raw,
                                                const float (&cs)[2], const float (&sn)[2],
                                                int max_seq, const uint16_t* __restrict__ qn_w,
                                                const uint16_t* __restrict__ kn_w,
                                                uint16_t* __restrict__ k_cache,
                                                uint16_t* __restrict__ v_cache,
                                                uint16_t* __restrict__ q_roped,
                                                uint8_t* kv, bool kv_staged, PreQKV&& pre_qkv,
                                                GetQKV&& get_qkv, Publish&& publish,
                                                Stamp stamp = Stamp()) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int s = sg * kAttnWaves + wave;

  pre_qkv();  // a wait's first round goes out ahead of this function's loads
  uint32_t nwv[3];
  nwv[0] = load_global(reinterpret_cast<const uint32_t*>(qn_w) + lane);
  nwv[2] = load_global(reinterpret_cast<const uint32_t*>(kn_w) + lane);
  nwv[1] = nwv[0];

  const int pos = pos_raw < 0 ? 0 : (pos_raw >= max_seq ? max_seq - 1 : pos_raw);
  const int ctx = pos + 1;
  const SplitRange sr = split_range(s, pos);
  const int start = sr.start;
  const int end = sr.end;
  // this workgroup's four splits hold position pos: it writes the new k / v
  const bool owns_pos = split_range(sg * kAttnWaves, pos).start <= pos &&
                        pos < split_range(sg * kAttnWaves + kAttnWaves - 1, pos).end;
  const int n_chunks = ((ctx + kAttnSplits - 1) / kAttnSplits + 31) / 32;  // workgroup-uniform

  // ---- 0. first chunk of the cache (rows clamped into [start, end - 1],
  // row 0 for an empty split), staged into this wave's LDS region unless the
  // caller already did (kv_prefetch) ----
  const int last = sr.last;
  if (!kv_staged) kv_stage(kv, k_cache, v_cache, g, start, last);
  __builtin_amdgcn_sched_barrier(0);

  uint32_t xw[3], v_new;
  get_qkv(xw, v_new);

  // ---- 1. head norms + RoPE: wave t < 3 takes vector t (q head 2g, q head
  // 2g+1, k head g), lane owns dims 2*lane, 2*lane+1; RoPE's partner dims
  // d -+ 64 sit in lane ^ 32 ----
  if (wave < 3) {
    const f16x2 xv = as_f16x2(wave == 0 ? xw[0] : (wave == 1 ? xw[1] : xw[2]));
    const f16x2 wv = as_f16x2(wave == 2 ? nwv[2] : nwv[0]);
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
      const float other = xor32(xs[dd]);
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
    const uint32_t roped = pack_f16x2(r2[0], r2[1]);
    // ---- 2. the roped q heads once, the new position into the cache ----
    if (wave < 2) {
      L.qh[wave][lane] = roped;
      if (q_roped != nullptr && sg == 0)
        reinterpret_cast<uint32_t*>(q_roped + (2 * g + wave) * kHeadDim)[lane] = roped;
    } else {
      L.kh[lane] = roped;
      if (owns_pos)
        reinterpret_cast<uint32_t*>(k_cache + ((size_t)pos * kKvHeads + g) * kHeadDim)[lane] = roped;
    }
  } else if (owns_pos) {
    reinterpret_cast<uint32_t*>(v_cache + ((size_t)pos * kKvHeads + g) * kHeadDim)[lane] = v_new;
  }
  stamp(16);
  __syncthreads();

  // ---- 3. per chunk (this wave's LDS region), transposed on the matrix
  // cores: S^T = K Q^T (K rows as A; B holds q_A and q_B as columns 0 and 1,
  // the other 14 zero), so lane (c16, grp) has query c16's scores at chunk
  // positions 16 nt + 4 grp + e; online softmax per query in base-2 units
  // (running max m, the lane's share of the sum l); O^T += V^T P^T with the
  // lane's 8 weights as B in the order 4 grp + e, 16 + 4 grp + e of the MFMA's
  // k slots, V^T from two transposing LDS reads per 16 dims in that order, p
  // split into f16 hi + lo (p - hi exact), carrying p to about 2^-22.  Lanes
  // with c16 < 2 hold the results. ----
  const int c16 = lane & 15;
  const int grp = lane >> 4;
  f16x8 qf[4];
  {
    const uint8_t* qrow = reinterpret_cast<const uint8_t*>(L.qh[c16 & 1]);
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const f16x8 q8 = *reinterpret_cast<const f16x8*>(qrow + 2 * (32 * st + 8 * grp));
      qf[st] = c16 < 2 ? q8 : (f16x8){};
    }
  }
  float m = -__builtin_inff(), l = 0.0f;
  f32x4 o[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) o[d] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
  const int vrow = 4 * grp + (c16 >> 2);
  const auto v_off = [&](int row, int d) {
    return 8192 + 256 * row + 16 * ((2 * d + ((c16 & 3) >> 1)) ^ (2 * (row & 7))) + 8 * (c16 & 1);
  };
  // Chunk c's copies: K(c) then V(c), issued as kv_stage does for c = 0 and
  // for c > 0 as K(c) after chunk c - 1's score reads and V(c) after its V^T
  // reads; the loads of one wave return in order, so K(c) has landed once at
  // most the 8 V(c) loads are outstanding, V(c) once at most K(c + 1)'s 8.
  for (int c = 0; c < n_chunks; ++c) {
    const int c0 = start + 32 * c;
    // the staged row of position pos predates this step's k and v: replace it
    const bool has_pos = pos >= c0 && pos < c0 + 32;
    const int rp = pos - c0;
    wait_vm<8>();
    if (has_pos && lane < 16)
      *reinterpret_cast<u32x4*>(kv + 256 * rp + 16 * (lane ^ (rp & 15))) =
          *reinterpret_cast<const u32x4*>(&L.kh[4 * lane]);
    f32x4 sc[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      sc[nt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int ch = 4 * st + grp;
        const int kr = 16 * nt + c16;
        const f16x8 kf = *reinterpret_cast<const f16x8*>(kv + 256 * kr + 16 * (ch ^ (kr & 15)));
        sc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[st], sc[nt], 0, 0, 0);
      }
    }
    stamp(17);
    // the K region is free once the score reads have returned (every MFMA
    // above waited for its fragment): the next chunk's K goes out now, under
    // the softmax and the weighted sum
    wait_lds();
    if (c + 1 < n_chunks) kv_stage_k(kv, k_cache, g, c0 + 32, last);
    // s[4 nt + e]: position c0 + 16 nt + 4 grp + e; past the split: -inf
    float s[8];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool ok = c0 + 16 * nt + 4 * grp + e < end;
        s[4 * nt + e] = ok ? sc[nt][e] * kScoreScaleLog2 : -__builtin_inff();
      }
    float mx = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])),
                     fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
    mx = max_col4(mx);
    const float mn = fmaxf(m, mx);
    // mn = -inf only while the split has seen no valid position (o, l = 0)
    const float alpha = mn == -__builtin_inff() ? 1.0f : __builtin_amdgcn_exp2f(m - mn);
    float p[8], ps = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      p[i] = s[i] == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(s[i] - mn);
      ps += p[i];
    }
    l = l * alpha + ps;
    m = mn;
#pragma unroll
    for (int d = 0; d < 8; ++d) o[d] *= alpha;
    stamp(18);
    // V(c) has landed: only K(c + 1)'s 8 copies, issued after it, may be out
    if (c + 1 < n_chunks) wait_vm<8>();
    else wait_vm<0>();
    if (has_pos)
      *reinterpret_cast<uint32_t*>(kv + 8192 + 256 * rp + 16 * ((lane >> 2) ^ (2 * (rp & 7))) +
                                   4 * (lane & 3)) = v_new;
    f16x8 ph, pl;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      typedef float f32x2_t __attribute__((ext_vector_type(2)));
      const f16x2 h2 = __builtin_convertvector((f32x2_t){p[i], p[i + 1]}, f16x2);
      const f16x2 l2 = __builtin_convertvector(
          (f32x2_t){p[i] - (float)h2.x, p[i + 1] - (float)h2.y}, f16x2);
      ph[i] = h2.x;
      ph[i + 1] = h2.y;
      pl[i] = l2.x;
      pl[i + 1] = l2.y;
    }
    // every V^T fragment of the chunk first; once they have returned the
    // region is free and the next chunk's V goes out under the weighted sum
    f16x8 vfs[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const v4i16 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS v4i16*)(kv + v_off(vrow, d)));
      const v4i16 v1 =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS v4i16*)(kv + v_off(vrow + 16, d)));
      vfs[d] = __builtin_bit_cast(f16x8, (v8i16){v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w});
    }
    wait_lds();
    if (c + 1 < n_chunks) kv_stage_v(kv, v_cache, g, c0 + 32, last);
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vfs[d], ph, o[d], 0, 0, 0);
      o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vfs[d], pl, o[d], 0, 0, 0);
    }
  }
  stamp(19);
  l = sum_col4(l);

  // ---- 4. the four waves' results -> one partial per query head ----
  if (c16 < 2) {
    if (grp == 0) {
      L.mrg[wave][c16][0] = m;
      L.mrg[wave][c16][1] = l;
    }
#pragma unroll
    for (int d = 0; d < 8; ++d)
      *reinterpret_cast<f32x4*>(&L.mrg[wave][c16][4 + 16 * d + 4 * grp]) = o[d];
  }
  __syncthreads();
  stamp(20);
  if (wave < 2) {  // wave hh merges query head 2g + hh
    const int hh = wave;
    float M = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, L.mrg[w][hh][0]);
    float Ls = 0.0f, a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) {
      const float mw = L.mrg[w][hh][0];
      const float ww = mw == -__builtin_inff() ? 0.0f : exp2f(mw - M);
      Ls = Ls + L.mrg[w][hh][1] * ww;
      a0 = a0 + L.mrg[w][hh][4 + 2 * lane] * ww;
      a1 = a1 + L.mrg[w][hh][5 + 2 * lane] * ww;
    }
    publish(hh, M, Ls, a0, a1);
  }
}

}  // namespace

#endif
