// Hand-written gfx950 (CDNA4) kernels for the Qwen3 decode GEMV path.
//
// Built ahead of time into a code object (hipcc --genco) and launched through
// hipModuleLaunchKernel by the C-ABI shim in q8gemv_shim.cpp.
//
//  * q8gemv_p{1,2,3}, q8gemv_qkv_k, q8gemv_batch_k: Q8_0 dequant + GEMV,
//    y[N] = W[N,K] . x[K] for K = 1024*P over one layer of a stacked
//    [L, N*K/32*34] byte buffer -- one GEMV, q/k/v of a layer, or a list of
//    GEMVs per launch.  Replace kernels/mlir/dispatch_{3,4,12,18,20}_gpu.mlir
//    (model/qwen3_full.mlir:536-589).
//  * vocab_gemv_argmax: f16 GEMV over [n_rows, 1024] with the two-phase argmax
//    fused in.  Replaces kernels/mlir/dispatch_24_gpu.mlir plus the tiled argmax
//    at model/qwen3_full.mlir:1469-1511.
//
// Numerics: f16 x, f32 accumulation, round-to-nearest-even f16 outputs.
// int8 -> f16 conversion is exact (0x6400|u encodes 1024+u; u = q+128), so
// every int8 x f16 product formed by v_dot2_f32_f16 is exact in f32.
#include "q8_device.h"

// ------------------------------------------------------------ exports -----

// One GEMV of K = 1024*P: workgroup (one wave) b computes row quad b.
#define Q8GEMV_SINGLE(P)                                                                   \
  extern "C" __global__ __launch_bounds__(64) void q8gemv_p##P(                            \
      const uint8_t* __restrict__ w, const uint16_t* __restrict__ x,                       \
      uint16_t* __restrict__ y, int n_rows) {                                              \
    __shared__ __attribute__((aligned(16))) uint8_t lds[QuadShape<P>::LDS_BYTES];           \
    q8_quad<P>(w, x, y, n_rows, blockIdx.x, lds);                                          \
  }
Q8GEMV_SINGLE(1)
Q8GEMV_SINGLE(2)
Q8GEMV_SINGLE(3)

// q, k and v of one layer in one launch: the three GEMVs read the same x
// (model/qwen3_full.mlir:625-635).  Workgroups 0..511 take the 512 row quads
// of q [2048,1024], 512..767 those of k [1024,1024], 768..1023 those of v.
extern "C" __global__ __launch_bounds__(64) void q8gemv_qkv_k(
    const uint8_t* __restrict__ wq, const uint8_t* __restrict__ wk,
    const uint8_t* __restrict__ wv, const uint16_t* __restrict__ x, uint16_t* __restrict__ yq,
    uint16_t* __restrict__ yk, uint16_t* __restrict__ yv) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[5 * 1024];
  const int b = blockIdx.x;
  if (b < 512) q8_quad<1>(wq, x, yq, 2048, b, lds);
  else if (b < 768) q8_quad<1>(wk, x, yk, 1024, b - 512, lds);
  else q8_quad<1>(wv, x, yv, 1024, b - 768, lds);
}

// Many independent GEMVs in one launch.  The batch's units are split evenly
// over the waves; a wave owns every quad whose first unit falls in its range
// and walks the table entries that range touches.
extern "C" __global__ __launch_bounds__(64) void q8gemv_batch_k(const uint8_t* __restrict__ table,
                                                               int count, int total_units) {
  __shared__ __attribute__((aligned(16))) uint8_t slot[kSlotBytes];
  __shared__ __attribute__((aligned(16))) uint16_t xl[1024 * kMaxP];
  const Q8BatchEntry* e = reinterpret_cast<const Q8BatchEntry*>(table + kBatchHeaderBytes);
  const int64_t W = gridDim.x;
  const int ga = (int)((int64_t)blockIdx.x * total_units / W);
  const int gb = (int)((int64_t)(blockIdx.x + 1) * total_units / W);
  if (ga >= gb) return;
  int lo = 0, hi = count - 1;  // last entry with unit_begin <= ga
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (e[mid].unit_begin <= ga) lo = mid;
    else hi = mid - 1;
  }
  for (int d = lo; d < count && e[d].unit_begin < gb; ++d) {
    const int p = e[d].p;
    const int nq = (e[d].n_rows + 3) / 4;
    const int t0 = ga - e[d].unit_begin;
    const int t1 = gb - e[d].unit_begin;
    const int qa = t0 <= 0 ? 0 : min(nq, (t0 + p - 1) / p);
    const int qb = t1 <= 0 ? 0 : min(nq, (t1 + p - 1) / p);
    if (qa >= qb) continue;
    const Q8Seg s{e[d].w, e[d].x, e[d].y, e[d].n_rows, p};
    q8_segment(s, qa * p, qb * p, slot, xl);
    __syncthreads();
  }
}

extern "C" __global__ __launch_bounds__(256) void vocab_gemv_argmax_k1024(
    const uint16_t* __restrict__ W, const uint16_t* __restrict__ x,
    uint16_t* __restrict__ logits, int n_rows, uint8_t* __restrict__ ws) {
  vocab_body<VOCAB_NT_LOADS != 0, true>(W, x, logits, n_rows, ws);
}

// token = row of the winning key (-1 for none); leaves the key zero for the
// next launch.
extern "C" __global__ void vocab_argmax_finalize(uint64_t* __restrict__ ws,
                                                 int32_t* __restrict__ token) {
  if (threadIdx.x == 0) {
    const uint64_t key = ws[0];
    *token = key == 0 ? -1 : (int32_t)(0xffffffffu - (uint32_t)(key & 0xffffffffu));
    ws[0] = 0;
  }
}

// Argmax of an f16 vector on its own (logits written by an earlier launch,
// e.g. decode_dispatch_24): the tiled argmax as a separate pass, as the
// reference runs it after the vocab matmul (model/qwen3_full.mlir:1469-1511).
// Thread t of workgroup b takes the 8-element pieces b * 256 + t, stepping by
// the grid's thread count, in increasing order, so a strictly-greater update
// keeps its first maximum; keys (argmax_key: value, then the lower index)
// meet in a wave max, then in the same 64-bit atomic max on ws[0] as the
// fused vocab kernel's, which vocab_argmax_finalize turns into the token.
// NaN never wins; -1 when nothing does.
extern "C" __global__ __launch_bounds__(256) void argmax_f16_k(const uint16_t* __restrict__ v,
                                                              int n, uint64_t* __restrict__ ws) {
  const int t = threadIdx.x;
  const int64_t stride = (int64_t)launch_wgs() * 256;
  float bv = -__builtin_inff();
  int bi = -1;
  for (int64_t p = (int64_t)blockIdx.x * 256 + t; 8 * p < n; p += stride) {
    const int i0 = (int)(8 * p);
    if (i0 + 8 <= n) {
      const u32x4 w = load_global(reinterpret_cast<const u32x4*>(v) + p);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float x = (float)as_f16x2(w[k >> 1])[k & 1];
        if (x > bv) {
          bv = x;
          bi = i0 + k;
        }
      }
    } else {
      for (int i = i0; i < n; ++i) {
        const float x = f16_bits_to_f32(v[i]);
        if (x > bv) {
          bv = x;
          bi = i;
        }
      }
    }
  }
  uint64_t key = bi >= 0 ? argmax_key(bv, bi) : (uint64_t)0;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)key, d, 64);
    const uint32_t hi = __shfl_xor((uint32_t)(key >> 32), d, 64);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    key = o > key ? o : key;
  }
  if ((t & 63) == 0 && key != 0)
    __hip_atomic_fetch_max(ws, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Zeroes the 256-byte workspace (graph-capture safe: a kernel, not a memset
// node): the argmax key and, in a decode scratch, the status word and the
// attention merge counters.
extern "C" __global__ void vocab_workspace_reset(uint32_t* __restrict__ ws) {
  if (threadIdx.x < 64) ws[threadIdx.x] = 0u;
}

// Plain device copy of n16 16-byte words (grid-stride): the reference kernel
// of known traffic for calibrating HBM byte counters, and (with n16 = 0) an
// empty launch for measuring dispatch overhead.
extern "C" __global__ __launch_bounds__(256) void stream_copy_b128(const u32x4* __restrict__ src,
                                                                   u32x4* __restrict__ dst,
                                                                   int64_t n16) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
    dst[i] = src[i];
}

// Plain device read of n16 16-byte words (grid-stride), writing nothing
// unless the words' XOR happens to equal `never` (the caller passes a value
// it is not): evicts the memory-side cache (MALL) without leaving dirty lines
// behind, unlike a copy, whose written lines a later kernel would have to
// write back.
extern "C" __global__ __launch_bounds__(256) void stream_read_b128(const u32x4* __restrict__ src,
                                                                   uint32_t* __restrict__ sink,
                                                                   int64_t n16, uint32_t never) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  uint32_t acc = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
    const u32x4 v = load_global(src + i);
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  if (acc == never) sink[threadIdx.x] = acc;
}

// ------------------------------------------------- calibration kernels ----
//
// Measurements the single-launch decode step's design rests on, made by the
// library itself so a benchmark can record them beside the step.

// An empty kernel: the launch cost of a grid shape (its LDS comes from the
// launch's dynamic size, so a shape can hold as many workgroups per CU as
// the decode step does).
extern "C" __global__ void calib_empty() {}

// Arguments of calib_handoff.
struct HandoffArgs {
  uint64_t* words;       // replicas x n_words tagged words, then the start word
  uint32_t* pub;         // [rounds][producers]: clock when each producer's stores were issued
  uint32_t* recv;        // [rounds][consumers]: clock when each consumer had the whole vector
  int producers, consumers, n_words, replicas, rounds;
  uint32_t seq;          // distinguishes calls (tags are seq << 8 | round + 1)
  uint32_t period;       // clock ticks between rounds
  uint32_t spin_limit;   // poll rounds before a wait gives up (then its clock reads stay 0)
};

__device__ __forceinline__ uint32_t realtime() {
  return (uint32_t)__builtin_amdgcn_s_memrealtime();  // 100 MHz, the same counter on every CU
}

// The latency of a tagged-word hand-off (the exchange of the single-launch
// decode step: 8-byte words = 32 data bits + a 32-bit tag, agent-scope
// relaxed atomic stores and polling loads).  Workgroups 0 .. producers - 1
// each own n_words / producers words of a vector, stored in every replica;
// workgroup producers + c polls replica c % replicas until every word carries
// the round's tag.  Round r starts for all producers at the same clock value
// (T0 + r * period, T0 published once by workgroup 0), so recv - max(pub) of a
// round is the hand-off's latency from the last producer's store to a
// consumer holding the vector.  Every wait is bounded; one that gives up
// leaves its clock reads 0.
extern "C" __global__ __launch_bounds__(256) void calib_handoff(HandoffArgs a) {
  const int wg = blockIdx.x;
  const int t = threadIdx.x;
  __shared__ uint32_t s_t0;
  __shared__ int s_ok;
  uint64_t* start = a.words + (size_t)a.replicas * a.n_words;
  const uint32_t tag0 = a.seq << 8;
  if (t == 0) {
    s_ok = 1;
    if (wg == 0)
      __hip_atomic_store(start, ((uint64_t)tag0 << 32) | (realtime() + 2000u), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    uint64_t w = __hip_atomic_load(start, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (uint32_t spins = 0; (uint32_t)(w >> 32) != tag0; ++spins) {
      if (spins > a.spin_limit) {
        s_ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      w = __hip_atomic_load(start, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    s_t0 = (uint32_t)w;
  }
  __syncthreads();
  if (!s_ok) return;
  const uint32_t t0 = s_t0;
  const int per = a.n_words / a.producers;
  for (int r = 0; r < a.rounds; ++r) {
    const uint32_t tag = tag0 | (uint32_t)(r + 1);
    if (wg < a.producers) {
      if (t == 0)
        while ((int32_t)(realtime() - (t0 + (uint32_t)r * a.period)) < 0) __builtin_amdgcn_s_sleep(2);
      __syncthreads();
      for (int i = t; i < per * a.replicas; i += 256) {
        const int rep = i / per;
        const int k = wg * per + i % per;
        __hip_atomic_store(a.words + (size_t)rep * a.n_words + k, ((uint64_t)tag << 32) | (uint32_t)k,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
      if (t == 0) a.pub[r * a.producers + wg] = realtime();
    } else if (wg < a.producers + a.consumers) {
      const int c = wg - a.producers;
      const uint64_t* src = a.words + (size_t)(c % a.replicas) * a.n_words;
      bool ok = true;
      for (int i = t; i < a.n_words && ok; i += 256) {
        uint64_t w = __hip_atomic_load(src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (uint32_t spins = 0; (uint32_t)(w >> 32) != tag; ++spins) {
          if (spins > a.spin_limit) {
            ok = false;
            break;
          }
          __builtin_amdgcn_s_sleep(1);
          w = __hip_atomic_load(src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      if (!ok) s_ok = 0;
      __syncthreads();
      if (t == 0) a.recv[r * a.consumers + c] = s_ok ? realtime() : 0u;
      if (!s_ok) return;
    }
  }
}

// Load-to-use latency of one lane's dependent loads: the lane follows the
// cycle next[] (u32 indices into next, each a different 128-byte line of a
// region of mask + 1 words) for `hops` steps, reading the 100 MHz clock before
// and after, `passes` times over the same cycle (the first pass finds lines
// wherever a previous kernel left them, a later one in this XCD's L2).  The
// workgroup whose XCD id (HW_REG_XCC_ID) is `xcd` runs the chase (xcd < 0:
// workgroup 0); every workgroup records its XCD id in xcd_of[blockIdx.x].
// ticks[p] = clock ticks of pass p (0 where no workgroup ran); ticks[passes] =
// the XCD that ran, ticks[passes + 1] = the last index (keeps the loads live).
extern "C" __global__ __launch_bounds__(64) void calib_chase(const uint32_t* __restrict__ next,
                                                             uint32_t mask, int hops, int passes,
                                                             int xcd, uint32_t* __restrict__ ticks,
                                                             uint32_t* __restrict__ xcd_of) {
  if (threadIdx.x != 0) return;
  uint32_t my;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(my));
  xcd_of[blockIdx.x] = my;
  if (xcd < 0 ? blockIdx.x != 0 : (int)my != xcd) return;
  uint32_t i = 0;
  for (int p = 0; p < passes; ++p) {
    const uint32_t t0 = realtime();
    for (int h = 0; h < hops; ++h) i = next[i] & mask;
    // the clock is read once the last load's value is in a register
    asm volatile("" : "+v"(i) : : "memory");
    ticks[p] = realtime() - t0;
  }
  ticks[passes] = my;
  ticks[passes + 1] = i;
}

// ------------------------------------------------ IREE HAL binding ABI ----
//
// The same kernels under the reference's executable export names and binding
// ABI, for IREE's executable substitution (compile.sh:35-43) with a ROCm HSACO
// object: binding base pointers, then the i32 push constants, with x and y at
// the byte offsets the reference bakes in (kernels/cuda/dispatch_3.cu:8-22,
// dispatch_4.cu:8-22, dispatch_12.cu:19-21, dispatch_18.cu:19-21,
// dispatch_20.cu:19-21, dispatch_24.cu:11-20).  Any launch shape with 64-256
// threads per workgroup computes every row: the reference's own stubs
// (workgroup_size 256, counts N/8 and 18992, kernels/cuda/dispatch_*.mlir:5-9)
// as well as this build's (64 threads, N/4 workgroups, one quad each).  Each
// full wave takes row quads blockIdx.x * waves + wave, stepping by the grid's
// wave count; a partial wave (blockDim.x % 64 != 0) only joins the barriers.
// Workgroups of fewer than 64 threads compute nothing (the shim rejects them).

// Every wave of the workgroup runs the same rounds (the round count depends
// on the workgroup only), so the barriers inside q8_quad_core match; a wave
// without a quad in the last round recomputes the last quad and stores
// nothing.
// waves: full waves per workgroup; wgs: workgroups of the launch.
template <int P>
__device__ __forceinline__ void hal_q8_quads(const uint8_t* __restrict__ w,
                                             const uint16_t* __restrict__ x,
                                             uint16_t* __restrict__ y, int n_rows,
                                             uint8_t* __restrict__ lds, int waves, int wgs) {
  if (waves == 0) return;
  const int wave = threadIdx.x >> 6;
  const int nq = (n_rows + 3) / 4;
  uint8_t* mine = lds + wave * QuadShape<P>::LDS_BYTES;
  const int step = wgs * waves;
  for (int base = (int)blockIdx.x * waves; base < nq; base += step) {
    const int quad = base + wave;
    const bool store = wave < waves && quad < nq;
    q8_quad_core<P>(w, n_rows, quad < nq ? quad : nq - 1, mine,
                    [&](u32x4 (&xr)[P][8]) { load_x_cols<P>(x, xr); },
                    [&](int row, float acc) {
                      if (store) y[row] = f32_to_f16_bits(acc);
                    });
  }
}

#define HAL_Q8_DISPATCH(NAME, P, N, BPL, X_OFF, Y_OFF)                                      \
  extern "C" __global__ __launch_bounds__(256) void NAME(                                     \
      const uint8_t* __restrict__ q8_stacked, const char* __restrict__ b1,                    \
      char* __restrict__ b2, uint32_t c0, uint32_t c1) {                                      \
    __shared__ __attribute__((aligned(16))) uint8_t lds[4 * QuadShape<P>::LDS_BYTES];         \
    const uint64_t layer = (uint64_t)c0 | ((uint64_t)c1 << 32);                               \
    const uint8_t* w = q8_stacked + layer * (BPL);                                            \
    const int waves = (int)(launch_wg_size() >> 6), wgs = (int)launch_wgs();                  \
    /* every argument is loaded before the first branch (one scalar round trip) */            \
    asm volatile("" ::"s"(w), "s"(b1), "s"(b2), "s"(waves), "s"(wgs));                        \
    hal_q8_quads<P>(w, reinterpret_cast<const uint16_t*>(b1 + (X_OFF)),                       \
                    reinterpret_cast<uint16_t*>(b2 + (Y_OFF)), N, lds, waves, wgs);           \
  }

HAL_Q8_DISPATCH(decode_dispatch_3_matmul_2048x1x1024_f16, 1, 2048, 2228224ULL, 2112, 4160)
HAL_Q8_DISPATCH(decode_dispatch_12_matmul_1024x1x2048_f16, 2, 1024, 2228224ULL, 12352, 2048)
HAL_Q8_DISPATCH(decode_dispatch_18_matmul_6144x1x1024_f16, 1, 6144, 6684672ULL, 64, 6144)
HAL_Q8_DISPATCH(decode_dispatch_20_matmul_1024x1x3072_f16, 3, 1024, 3342336ULL, 18432, 0)

// dispatch_4 takes the output byte offset as c0 and the layer as c1 | c2 << 32.
extern "C" __global__ __launch_bounds__(256) void decode_dispatch_4_matmul_1024x1x1024_f16(
    const uint8_t* __restrict__ q8_stacked, const char* __restrict__ b1, char* __restrict__ b2,
    uint32_t c0, uint32_t c1, uint32_t c2) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[4 * QuadShape<1>::LDS_BYTES];
  const uint64_t layer = (uint64_t)c1 | ((uint64_t)c2 << 32);
  const uint8_t* w = q8_stacked + layer * 1114112ULL;
  uint16_t* y = reinterpret_cast<uint16_t*>(b2 + (int)c0);
  const int waves = (int)(launch_wg_size() >> 6), wgs = (int)launch_wgs();
  asm volatile("" ::"s"(w), "s"(b1), "s"(y), "s"(waves), "s"(wgs));  // as in HAL_Q8_DISPATCH
  hal_q8_quads<1>(w, reinterpret_cast<const uint16_t*>(b1 + 2112), y, 1024, lds, waves, wgs);
}

// dispatch_24 takes the output byte offset as c0 (logits only; the reference
// runs its argmax as separate dispatches).  The vocab body spreads the row
// batches over however many full waves the grid has.
extern "C" __global__ __launch_bounds__(256) void decode_dispatch_24_matmul_151936x1x1024_f16(
    const uint16_t* __restrict__ weight, const char* __restrict__ b1, char* __restrict__ b2,
    uint32_t c0) {
  if ((launch_wg_size() >> 6) == 0) return;
  vocab_body<VOCAB_NT_LOADS != 0, false>(weight, reinterpret_cast<const uint16_t*>(b1 + 64),
                                         reinterpret_cast<uint16_t*>(b2 + (int)c0), 151936,
                                         nullptr);
}
