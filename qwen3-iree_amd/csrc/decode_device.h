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

__device__ __forceinline__ float max32(float v) {  // over the 32 lanes of a wave half
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
}

__device__ __forceinline__ float sum32(float v) { return sum_rows2(reduce_row16(v)); }

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

// Weights of the 8 split-group partials of one query head: w_g = exp(m_g -
// max m) (0 for an empty group), L = sum_g l_g w_g, summed in group order.
__device__ __forceinline__ void merge_weights(const float (&m)[kAttnGroups],
                                              const float (&l)[kAttnGroups],
                                              float (&w)[kAttnGroups], float& L) {
  float M = -__builtin_inff();
#pragma unroll
  for (int g = 0; g < kAttnGroups; ++g) M = fmaxf(M, m[g]);
  L = 0.0f;
#pragma unroll
  for (int g = 0; g < kAttnGroups; ++g) {
    w[g] = m[g] == -__builtin_inff() ? 0.0f : expf(m[g] - M);
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

// Bytes of one wave's prefetched first chunk: K (32 rows x this lane's half
// row, 8 x 1 KiB) then V (32 rows x the lane's two dims, 32 x 256 B).
constexpr int kKvPrefetchBytes = 8 * 1024 + 32 * 256;

// One chunk of a split's cache rows -- positions c0 .. c0 + 31, clamped to
// `last` -- copied into the wave's LDS region kv by the memory system
// (global_load_lds), so no register holds them while they are in flight: lane
// (pl, half)'s K piece m (row c0 + pl, dims 64 half + 8 m .. + 8) lands at kv
// + 1024 m + 16 lane, the V word of row c0 + j (dims 2 lane, 2 lane + 1) at kv
// + 8192 + 256 j + 4 lane.  The wave may read them once its vector memory
// counter has drained past these loads.  PACE > 0 sleeps 64 PACE cycles after
// the K pieces and after every fourth V row.
template <int PACE = 0>
__device__ __forceinline__ void kv_stage(uint8_t* kv, const uint16_t* __restrict__ k_cache,
                                         const uint16_t* __restrict__ v_cache, int g, int c0,
                                         int last) {
  const int lane = threadIdx.x & 63;
  const int half = lane >> 5;
  const int pl = lane & 31;
  const int p = c0 + pl < last ? c0 + pl : last;
  const u32x4* krow = reinterpret_cast<const u32x4*>(
      k_cache + ((size_t)p * kKvHeads + g) * kHeadDim + 64 * half);
#pragma unroll
  for (int m = 0; m < 8; ++m)
    __builtin_amdgcn_global_load_lds((const GLOBAL_AS void*)(krow + m),
                                     (__attribute__((address_space(3))) void*)(kv + 1024 * m), 16,
                                     0, 0);
  if constexpr (PACE > 0) __builtin_amdgcn_s_sleep(PACE);
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    const int pj = c0 + j < last ? c0 + j : last;
    __builtin_amdgcn_global_load_lds(
        (const GLOBAL_AS void*)(reinterpret_cast<const uint32_t*>(
                                    v_cache + ((size_t)pj * kKvHeads + g) * kHeadDim) +
                                lane),
        (__attribute__((address_space(3))) void*)(kv + 8192 + 256 * j), 4, 0, 0);
    if constexpr (PACE > 0)
      if ((j & 3) == 3) __builtin_amdgcn_s_sleep(PACE);
  }
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
  float mrg[kAttnWaves][2][2 + kHeadDim];
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
//  3. chunks of 32 positions: lane (j, half) scores position j of the chunk
//     on dims [64*half, 64*half + 64) for both q heads, the halves meet in one
//     cross-half add; s_j = (q . k_j) * rsqrt(128); online softmax; the
//     weighted sum of v (each lane owns dims 2*lane, 2*lane+1 of both heads).
//     A position's weights reach the lanes holding v as lane reads, so a
//     wave runs its chunks without waiting for the others;
//  4. publish(hh, m, l, a0, a1) on waves 0 and 1 (query head 2g + hh): m =
//     max over the 4 waves, l and this lane's two dims rescaled by
//     exp(m_w - m).  An empty split (ctx < 32) contributes m = -inf, l = 0.
// get_qkv(xw, v_new) fills this lane's words (dims 2*lane, 2*lane+1) of q
// head 2g, q head 2g+1, k head g (xw[0..2]) and v head g; every thread of the
// workgroup calls it once, and pre_qkv() once before any load of this
// function (where get_qkv's requests can start early).
// cs, sn: rope_angles of the clamped position.
template <class PreQKV, class GetQKV, class Publish>
__device__ __forceinline__ void attention_group(AttnLds& L, int g, int sg, int pos_raw,
                                                const float (&cs)[2], const float (&sn)[2],
                                                int max_seq, const uint16_t* __restrict__ qn_w,
                                                const uint16_t* __restrict__ kn_w,
                                                uint16_t* __restrict__ k_cache,
                                                uint16_t* __restrict__ v_cache,
                                                uint16_t* __restrict__ q_roped,
                                                uint8_t* kv, bool kv_staged, PreQKV&& pre_qkv,
                                                GetQKV&& get_qkv, Publish&& publish) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int s = sg * kAttnWaves + wave;
  const int half = lane >> 5;
  const int pl = lane & 31;

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
  __syncthreads();

  // ---- 3. scores, online softmax, weighted v ----
  float m = -__builtin_inff(), l = 0.0f;  // per q head; identical in all lanes
  float mB = -__builtin_inff(), lB = 0.0f;
  float accA0 = 0.0f, accA1 = 0.0f, accB0 = 0.0f, accB1 = 0.0f;
  for (int c = 0; c < n_chunks; ++c) {
    const int c0 = start + 32 * c;
    const int p = c0 + pl;
    const bool valid = p < end;
    u32x4 kreg[8];
#pragma unroll
    for (int mm = 0; mm < 8; ++mm)
      kreg[mm] = *reinterpret_cast<const u32x4*>(kv + 1024 * mm + 16 * lane);
    // the row of position pos is this step's k (in LDS; the cache slot was
    // staged before it was written): one lane takes it over
    if (p == pos) {
#pragma unroll
      for (int mm = 0; mm < 8; ++mm)
        kreg[mm] = *reinterpret_cast<const u32x4*>(&L.kh[32 * half + 4 * mm]);
    }
    // two partial sums per head (dims of even / odd 8-dim groups) halve the
    // dependent chain
    float dA0 = 0.0f, dB0 = 0.0f, dA1 = 0.0f, dB1 = 0.0f;
#pragma unroll
    for (int mm = 0; mm < 8; mm += 2) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = 32 * half + 4 * mm + j;
        const f16x2 k0 = as_f16x2(kreg[mm][j]), k1 = as_f16x2(kreg[mm + 1][j]);
        dA0 = __builtin_amdgcn_fdot2(as_f16x2(L.qh[0][i]), k0, dA0, false);
        dB0 = __builtin_amdgcn_fdot2(as_f16x2(L.qh[1][i]), k0, dB0, false);
        dA1 = __builtin_amdgcn_fdot2(as_f16x2(L.qh[0][i + 4]), k1, dA1, false);
        dB1 = __builtin_amdgcn_fdot2(as_f16x2(L.qh[1][i + 4]), k1, dB1, false);
      }
    }
    float dA = dA0 + dA1, dB = dB0 + dB1;
    dA = sum_halves(dA);
    dB = sum_halves(dB);
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
    accA0 *= cA;
    accA1 *= cA;
    accB0 *= cB;
    accB1 *= cB;
    __builtin_amdgcn_sched_barrier(0);
    // Four positions at a time, the next four's v requested from LDS before
    // this four's products: position j's weights are lane j's p (lanes j and
    // j + 32 hold the same value), read into scalar registers (the scheduling
    // fences keep the compiler from hoisting all 64 reads).  With `fix`,
    // position pos takes this step's v, and positions past the split (weight
    // 0, a clamped valid row) take v = 0, so a non-finite value there cannot
    // leak in; most chunks need neither (a wave-uniform branch).
    const int n = end - c0 < 32 ? end - c0 : 32;
    const auto v_word = [&](int j) {
      return *reinterpret_cast<const uint32_t*>(kv + 8192 + 256 * j + 4 * lane);
    };
    const auto weighted_v = [&](bool fix) {
      uint32_t vbuf[2][4];
#pragma unroll
      for (int j = 0; j < 4; ++j) vbuf[0][j] = v_word(j);
#pragma unroll
      for (int j0 = 0; j0 < 32; j0 += 4) {
        if (j0 + 4 < 32) {
#pragma unroll
          for (int j = 0; j < 4; ++j) vbuf[((j0 >> 2) + 1) & 1][j] = v_word(j0 + 4 + j);
        }
#pragma unroll
        for (int j = j0; j < j0 + 4; ++j) {
          const uint32_t vs = vbuf[(j0 >> 2) & 1][j - j0];
          const uint32_t vw = fix ? (c0 + j == pos ? v_new : (j < n ? vs : 0u)) : vs;
          const f16x2 vv = as_f16x2(vw);
          const float v0 = (float)vv.x, v1 = (float)vv.y;
          const float wa = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pA), j));
          const float wb = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pB), j));
          accA0 = __builtin_fmaf(wa, v0, accA0);
          accA1 = __builtin_fmaf(wa, v1, accA1);
          accB0 = __builtin_fmaf(wb, v0, accB0);
          accB1 = __builtin_fmaf(wb, v1, accB1);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    if (n < 32 || (pos >= c0 && pos < c0 + 32)) weighted_v(true);
    else weighted_v(false);
    __builtin_amdgcn_sched_barrier(0);
    // the next chunk into the same region: every read of this one has
    // returned (its values were used above)
    if (c + 1 < n_chunks) kv_stage(kv, k_cache, v_cache, g, c0 + 32, last);
  }

  // ---- 4. the four waves' results -> one partial per query head ----
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
  if (wave < 2) {  // wave hh merges query head 2g + hh
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
    publish(hh, M, Ls, a0, a1);
  }
}

}  // namespace

#endif
