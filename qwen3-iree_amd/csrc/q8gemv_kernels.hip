// Hand-written gfx950 (CDNA4) kernels for the Qwen3 decode GEMV path.
//
// Built ahead of time into a code object (hipcc --genco) and launched through
// hipModuleLaunchKernel by the C-ABI shim in q8gemv_shim.cpp.
//
//  * q8gemv_p{P}_r{R}: Q8_0 dequant + GEMV, y[N] = W[N,K] . x[K] for
//    K = 1024*P, one layer of a stacked [L, N*K/32*34] byte buffer.  Replaces
//    kernels/mlir/dispatch_{3,4,12,18,20}_gpu.mlir (model/qwen3_full.mlir:536-589).
//  * vocab_gemv_argmax: f16 GEMV over [n_rows, 1024] with the two-phase argmax
//    fused in.  Replaces kernels/mlir/dispatch_24_gpu.mlir plus the tiled argmax
//    at model/qwen3_full.mlir:1469-1511.
//
// Numerics: f16 x, f32 accumulation, round-to-nearest-even f16 outputs.
// int8 -> f16 conversion is exact (0x6400|u encodes 1024+u; u = q+128), so
// every int8 x f16 product formed by v_dot2_f32_f16 is exact in f32.
#include <hip/hip_runtime.h>
#include <stdint.h>

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

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
  return __builtin_bit_cast(uint16_t, (_Float16)v);  // v_cvt_f16_f32, RNE
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the 16 lanes of a DPP row; every lane of the row ends with the same
// value (each step adds a lane and its mirror partner, a symmetric pairing).
__device__ __forceinline__ float reduce_row16(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x141>(v);  // row_half_mirror
  v += dpp<0x140>(v);  // row_mirror
  return v;
}

__device__ __forceinline__ float reduce_wave64(float v) {
  v = reduce_row16(v);
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

// Dot product of one 68-byte Q8_0 block pair with 64 x values.
//   d[0..16]: the pair's 17 dwords (pair start is 4-byte aligned)
//     byte 0-1 scale0, 2-33 q0[0..31], 34-35 scale1, 36-67 q1[0..31]
//   xr[0..7]: x for the pair's 64 K positions, 8 f16 per u32x4
// Returns f32(scale0)*dot0 + f32(scale1)*dot1 with each dot an f32 sum of
// exact int8*f16 products.
__device__ __forceinline__ float q8_pair_dot(const uint32_t (&d)[17], const u32x4 (&xr)[8]) {
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
  return s0 * dot0 + s1 * dot1;
}

// One wave (64 lanes) per workgroup; the wave owns R quads of 4 consecutive
// rows.  Lane l works on row (l >> 4) of each quad and on block pairs
// p, p+16, ..., p+16(P-1) with p = l & 15, i.e. K positions
// [1024c + 64p, 1024c + 64p + 64) for c < P.
//
// The wave's rows are one contiguous byte span (4*R*ROWB bytes).  It is read
// with fully coalesced 16-byte loads (lane l takes bytes 16l, 16l+1024, ...),
// staged through LDS, and read back per lane as 68-byte block pairs, so HBM
// sees whole 1 KiB requests per instruction despite the 34-byte block stride.
// All of a wave's weight loads are issued before its first x load, so the
// weight stream and the x fetch overlap.
template <int P, int R>
__device__ __forceinline__ void q8gemv_body(const uint8_t* __restrict__ w,
                                            const uint16_t* __restrict__ x,
                                            uint16_t* __restrict__ y, int n_rows,
                                            uint8_t* __restrict__ lds) {
  constexpr int ROWB = 1088 * P;      // bytes per row (32*P blocks of 34 B)
  constexpr int SPAN = 4 * R * ROWB;  // bytes per wave
  constexpr int CHUNKS = SPAN / 16;
  constexpr int ITERS = (CHUNKS + 63) / 64;

  const int lane = threadIdx.x;
  const int row0 = blockIdx.x * (4 * R);
  int rows_here = n_rows - row0;
  rows_here = rows_here < 4 * R ? rows_here : 4 * R;
  const int valid = rows_here * (ROWB / 16);
  const u32x4* src = reinterpret_cast<const u32x4*>(w + (size_t)row0 * ROWB);

  u32x4 buf[ITERS];
#pragma unroll
  for (int i = 0; i < ITERS; ++i) {
    const int c = i * 64 + lane;
    if (c < valid) buf[i] = __builtin_nontemporal_load(src + c);
  }

  const int p = lane & 15;
  const int rsub = lane >> 4;
  u32x4 xr[P][8];
#pragma unroll
  for (int c = 0; c < P; ++c) {
    const u32x4* xs = reinterpret_cast<const u32x4*>(x + 1024 * c + 64 * p);
#pragma unroll
    for (int m = 0; m < 8; ++m) xr[c][m] = xs[m];
  }

  u32x4* l4 = reinterpret_cast<u32x4*>(lds);
#pragma unroll
  for (int i = 0; i < ITERS; ++i) {
    const int c = i * 64 + lane;
    if (c < valid) l4[c] = buf[i];
  }
  __syncthreads();

#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int rl = 4 * i + rsub;
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < P; ++c) {
      const uint32_t* pp = reinterpret_cast<const uint32_t*>(lds + rl * ROWB + 68 * (p + 16 * c));
      uint32_t d[17];
#pragma unroll
      for (int m = 0; m < 17; ++m) d[m] = pp[m];
      acc += q8_pair_dot(d, xr[c]);
    }
    acc = reduce_row16(acc);
    const int row = row0 + rl;
    if (p == 0 && row < n_rows) y[row] = f32_to_f16_bits(acc);
  }
}

// ------------------------------------------------------------ vocab ------

struct ArgmaxPartial {
  float value;
  int32_t index;
};

// Workspace layout: [0,16) completion counter (u32), then one 8-byte
// (value, index) partial per workgroup.
constexpr int kWsHeader = 16;

__device__ __forceinline__ float f16_row_dot(const u32x4& w, const u32x4& xv, float acc) {
  acc = __builtin_amdgcn_fdot2(as_f16x2(w[0]), as_f16x2(xv[0]), acc, false);
  acc = __builtin_amdgcn_fdot2(as_f16x2(w[1]), as_f16x2(xv[1]), acc, false);
  acc = __builtin_amdgcn_fdot2(as_f16x2(w[2]), as_f16x2(xv[2]), acc, false);
  acc = __builtin_amdgcn_fdot2(as_f16x2(w[3]), as_f16x2(xv[3]), acc, false);
  return acc;
}

// f16 GEMV rows [0, n_rows) x K=1024 with a fused argmax.
//
// 256 threads = 4 waves per workgroup; global wave g owns the contiguous rows
// [g*n/TW, (g+1)*n/TW).  Per row, lane l reads bytes [16l, 16l+16) and
// [1024+16l, 1024+16l+16) of the 2 KiB row (two fully coalesced 1 KiB wave
// loads) and keeps its 16 x values in registers for every row.  U rows are in
// flight per wave (double buffered).
//
// Argmax: each logit is rounded to f16 first (the reference compares the f16
// logits tensor); a strictly-greater test in increasing row order keeps the
// lowest index among equal maxima, NaN never wins and -inf never replaces the
// initial (-inf, -1).  Waves, then workgroups, are combined in row order with
// the same rule; the last workgroup to finish (device-scope counter) reduces
// the per-workgroup partials and resets the counter for the next launch.
template <int U>
__device__ __forceinline__ void vocab_body(const uint16_t* __restrict__ W,
                                           const uint16_t* __restrict__ x,
                                           uint16_t* __restrict__ logits, int n_rows,
                                           int32_t* __restrict__ token,
                                           uint8_t* __restrict__ ws) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int gw = blockIdx.x * 4 + wave;
  const int64_t tw = (int64_t)gridDim.x * 4;
  const int r_begin = (int)((int64_t)gw * n_rows / tw);
  const int r_end = (int)((int64_t)(gw + 1) * n_rows / tw);

  const u32x4* xv = reinterpret_cast<const u32x4*>(x);
  const u32x4 xa = xv[lane];
  const u32x4 xb = xv[64 + lane];
  const u32x4* Wv = reinterpret_cast<const u32x4*>(W);

  float best_v = -__builtin_inff();
  int best_i = -1;

  auto consume = [&](int row, const u32x4& wa, const u32x4& wb) {
    float acc = f16_row_dot(wa, xa, 0.0f);
    acc = f16_row_dot(wb, xb, acc);
    acc = reduce_wave64(acc);
    const uint16_t hb = f32_to_f16_bits(acc);
    if (logits != nullptr && lane == 0) logits[row] = hb;
    const float hv = f16_bits_to_f32(hb);
    if (hv > best_v) {
      best_v = hv;
      best_i = row;
    }
  };

  int r = r_begin;
  if (r + U <= r_end) {
    u32x4 ca[U], cb[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      ca[u] = __builtin_nontemporal_load(Wv + (size_t)(r + u) * 128 + lane);
      cb[u] = __builtin_nontemporal_load(Wv + (size_t)(r + u) * 128 + 64 + lane);
    }
    for (;;) {
      const int nr = r + U;
      const bool more = nr + U <= r_end;
      u32x4 na[U], nb[U];
      if (more) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          na[u] = __builtin_nontemporal_load(Wv + (size_t)(nr + u) * 128 + lane);
          nb[u] = __builtin_nontemporal_load(Wv + (size_t)(nr + u) * 128 + 64 + lane);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) consume(r + u, ca[u], cb[u]);
      r = nr;
      if (!more) break;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        ca[u] = na[u];
        cb[u] = nb[u];
      }
    }
  }
  for (; r < r_end; ++r) {
    const u32x4 wa = __builtin_nontemporal_load(Wv + (size_t)r * 128 + lane);
    const u32x4 wb = __builtin_nontemporal_load(Wv + (size_t)r * 128 + 64 + lane);
    consume(r, wa, wb);
  }

  // ---- workgroup combine (waves hold increasing row ranges) ----
  __shared__ float s_val[4];
  __shared__ int s_idx[4];
  __shared__ int s_last;
  if (lane == 0) {
    s_val[wave] = best_v;
    s_idx[wave] = best_i;
  }
  __syncthreads();

  uint32_t* counter = reinterpret_cast<uint32_t*>(ws);
  uint64_t* partials = reinterpret_cast<uint64_t*>(ws + kWsHeader);
  if (threadIdx.x == 0) {
    float bv = -__builtin_inff();
    int bi = -1;
#pragma unroll
    for (int w4 = 0; w4 < 4; ++w4) {
      if (s_val[w4] > bv) {
        bv = s_val[w4];
        bi = s_idx[w4];
      }
    }
    const uint64_t packed = (uint64_t)__builtin_bit_cast(uint32_t, bv) |
                            ((uint64_t)(uint32_t)bi << 32);
    __hip_atomic_store(partials + blockIdx.x, packed, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __threadfence();
    const uint32_t prev = atomicAdd(counter, 1u);
    s_last = (prev == gridDim.x - 1) ? 1 : 0;
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  // ---- last workgroup: reduce the partials in workgroup order ----
  const int G = gridDim.x;
  const int t = threadIdx.x;
  const int p_begin = (int)((int64_t)t * G / 256);
  const int p_end = (int)((int64_t)(t + 1) * G / 256);
  float tv = -__builtin_inff();
  int ti = -1;
  for (int g = p_begin; g < p_end; ++g) {
    const uint64_t pk = __hip_atomic_load(partials + g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const float v = __builtin_bit_cast(float, (uint32_t)(pk & 0xffffffffu));
    if (v > tv) {
      tv = v;
      ti = (int32_t)(uint32_t)(pk >> 32);
    }
  }
  __shared__ float f_val[256];
  __shared__ int f_idx[256];
  f_val[t] = tv;
  f_idx[t] = ti;
  __syncthreads();
  if (t == 0) {
    float bv = -__builtin_inff();
    int bi = -1;
    for (int k = 0; k < 256; ++k) {
      if (f_val[k] > bv) {
        bv = f_val[k];
        bi = f_idx[k];
      }
    }
    *token = bi;
    __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace

// ------------------------------------------------------------ exports -----

#define Q8GEMV_KERNEL(P, R)                                                              \
  extern "C" __global__ __launch_bounds__(64) void q8gemv_p##P##_r##R(                   \
      const uint8_t* __restrict__ w, const uint16_t* __restrict__ x,                     \
      uint16_t* __restrict__ y, int n_rows) {                                            \
    __shared__ __attribute__((aligned(16))) uint8_t lds[4 * (R) * 1088 * (P)];           \
    q8gemv_body<P, R>(w, x, y, n_rows, lds);                                             \
  }

Q8GEMV_KERNEL(1, 1)
Q8GEMV_KERNEL(1, 2)
Q8GEMV_KERNEL(1, 3)
Q8GEMV_KERNEL(1, 4)
Q8GEMV_KERNEL(1, 6)
Q8GEMV_KERNEL(2, 1)
Q8GEMV_KERNEL(2, 2)
Q8GEMV_KERNEL(2, 4)
Q8GEMV_KERNEL(3, 1)
Q8GEMV_KERNEL(3, 2)
Q8GEMV_KERNEL(3, 4)

extern "C" __global__ __launch_bounds__(256) void vocab_gemv_argmax_k1024(
    const uint16_t* __restrict__ W, const uint16_t* __restrict__ x,
    uint16_t* __restrict__ logits, int n_rows, int32_t* __restrict__ token,
    uint8_t* __restrict__ ws) {
  vocab_body<4>(W, x, logits, n_rows, token, ws);
}

// Zeroes the workspace completion counter (graph-capture safe: a kernel, not
// a memset node).
extern "C" __global__ void vocab_workspace_reset(uint32_t* __restrict__ ws) {
  if (threadIdx.x < 4) ws[threadIdx.x] = 0u;
}
