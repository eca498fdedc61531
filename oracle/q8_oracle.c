/*
 * CPU oracle for the Qwen3 decode GEMV path.  TEST INFRASTRUCTURE ONLY: the
 * checker for the HIP kernels, loaded by the tests, the smoke check and the
 * benchmark's CPU-baseline leg, never by the product.
 *
 * Built with -ffp-contract=off so every multiply and add rounds separately,
 * exactly as the reference MLIR kernels write them (arith.mulf, arith.addf).
 */
#include "q8_oracle.h"

#include <math.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- f16 ---- */

static float bits_to_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f32_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float oracle_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t mant = h & 0x3ff;
  if (exp == 0) {
    /* zero or subnormal: mant * 2^-24, exact in f32 */
    float v = (float)mant * 5.9604644775390625e-8f;
    return sign ? -v : v;
  }
  if (exp == 31) return bits_to_f32(sign | 0x7f800000u | (mant << 13));
  return bits_to_f32(sign | ((exp + 112u) << 23) | (mant << 13));
}

uint16_t oracle_f32_to_f16(float f) {
  uint32_t x = f32_to_bits(f);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu)); /* NaN */
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
  if (ax < 0x38800000u) {
    /* below 2^-14: result is subnormal (or zero / rounds up to min normal) */
    uint32_t e = ax >> 23;
    if (e < 102) return sign; /* < 2^-25 rounds to zero */
    uint32_t m = (ax & 0x7fffffu) | 0x800000u; /* value = m * 2^(e-150) */
    uint32_t shift = 126u - e;                 /* result = m * 2^(e-126) */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
  uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++; /* carry may reach inf */
  return (uint16_t)(sign | h);
}

void oracle_f16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_f16_to_f32(in[i]);
}

void oracle_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_f16(in[i]);
}

/* Table for fast f16 -> f32 widening in the GEMV loops. */
static float g_f16_table[65536];
static int g_f16_table_ready = 0;

static void ensure_table(void) {
  if (g_f16_table_ready) return;
#ifdef _OPENMP
#pragma omp critical(oracle_f16_table)
#endif
  {
    if (!g_f16_table_ready) {
      for (uint32_t i = 0; i < 65536u; ++i) g_f16_table[i] = oracle_f16_to_f32((uint16_t)i);
      g_f16_table_ready = 1;
    }
  }
}

/* ----------------------------------------------------------- quantize ---- */

/* tools/create_q8_irpa.py:103-118.  All arithmetic in f32 as numpy does it:
 * scale = max|w| / 127 (f32 division), a zero scale becomes 1.0,
 * q = round-half-even(w / scale) clipped to [-128, 127], scale stored as
 * f16 (RNE) little-endian in bytes 0-1, q as int8 in bytes 2-33. */
int oracle_q8_quantize(const float* w, int64_t n, uint8_t* out) {
  if (n % 32 != 0) return -1;
  int64_t nb = n / 32;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
  for (int64_t b = 0; b < nb; ++b) {
    const float* blk = w + b * 32;
    float maxabs = 0.0f;
    for (int j = 0; j < 32; ++j) {
      float a = fabsf(blk[j]);
      if (a > maxabs) maxabs = a;
    }
    float scale = maxabs / 127.0f;
    if (scale == 0.0f) scale = 1.0f;
    uint16_t sh = oracle_f32_to_f16(scale);
    uint8_t* o = out + b * 34;
    o[0] = (uint8_t)(sh & 0xff);
    o[1] = (uint8_t)(sh >> 8);
    for (int j = 0; j < 32; ++j) {
      float r = nearbyintf(blk[j] / scale); /* default mode: ties to even */
      if (r < -128.0f) r = -128.0f;
      if (r > 127.0f) r = 127.0f;
      o[2 + j] = (uint8_t)(int8_t)r;
    }
  }
  return 0;
}

/* tools/create_q8_irpa.py:121-129 */
void oracle_q8_dequant(const uint8_t* blocks, int64_t nblocks, float* out) {
  for (int64_t b = 0; b < nblocks; ++b) {
    const uint8_t* o = blocks + b * 34;
    float s = oracle_f16_to_f32((uint16_t)(o[0] | (o[1] << 8)));
    for (int j = 0; j < 32; ++j) out[b * 32 + j] = s * (float)(int8_t)o[2 + j];
  }
}

/* --------------------------------------------------------------- GEMV ---- */

/* xor butterfly over 32 lane partials: gpu.shuffle xor 16,8,4,2,1 with
 * r = own + partner at each step (dispatch_3_gpu.mlir:111-120).  Returns the
 * value lane 0 ends with. */
static float butterfly32(float* v) {
  float t[32];
  for (int off = 16; off >= 1; off >>= 1) {
    for (int l = 0; l < 32; ++l) t[l] = v[l] + v[l ^ off];
    memcpy(v, t, sizeof(t));
  }
  return v[0];
}

/* kernels/mlir/dispatch_3_gpu.mlir:79-126 (one block per lane) and
 * dispatch_20_gpu.mlir:116-144 / dispatch_12_gpu.mlir (blocks l, l+32, ...,
 * acc += scale_b * dot_b).  For K = 1024 the single product scale*dot equals
 * 0 + scale*dot, so one loop covers both forms. */
void oracle_q8_gemv(const uint8_t* w_layer, int64_t N, int64_t K,
                    const uint16_t* x, uint16_t* y) {
  ensure_table();
  const int64_t nblk = K / 32;
  const int64_t row_bytes = nblk * 34;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
  for (int64_t n = 0; n < N; ++n) {
    const uint8_t* row = w_layer + n * row_bytes;
    float lanes[32];
    for (int l = 0; l < 32; ++l) {
      float acc = 0.0f;
      for (int64_t b = l; b < nblk; b += 32) {
        const uint8_t* blk = row + b * 34;
        float scale = g_f16_table[(uint16_t)(blk[0] | (blk[1] << 8))];
        float dot = 0.0f;
        for (int j = 0; j < 32; ++j) {
          float p = (float)(int8_t)blk[2 + j] * g_f16_table[x[b * 32 + j]];
          dot = dot + p;
        }
        float scaled = scale * dot;
        acc = acc + scaled;
      }
      lanes[l] = acc;
    }
    y[n] = oracle_f32_to_f16(butterfly32(lanes));
  }
}

void oracle_q8_gemv_f64(const uint8_t* w_layer, int64_t N, int64_t K,
                        const uint16_t* x, double* y, double* sum_abs) {
  ensure_table();
  const int64_t nblk = K / 32;
  const int64_t row_bytes = nblk * 34;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
  for (int64_t n = 0; n < N; ++n) {
    const uint8_t* row = w_layer + n * row_bytes;
    double acc = 0.0, mag = 0.0;
    for (int64_t b = 0; b < nblk; ++b) {
      const uint8_t* blk = row + b * 34;
      double scale = (double)g_f16_table[(uint16_t)(blk[0] | (blk[1] << 8))];
      double dot = 0.0, dabs = 0.0;
      for (int j = 0; j < 32; ++j) {
        double p = (double)(int8_t)blk[2 + j] * (double)g_f16_table[x[b * 32 + j]];
        dot += p;
        dabs += fabs(p);
      }
      acc += scale * dot;
      mag += fabs(scale) * dabs;
    }
    if (y) y[n] = acc;
    if (sum_abs) sum_abs[n] = mag;
  }
}

/* kernels/mlir/dispatch_24_gpu.mlir:75-91: lane l, k = l, l+32, ...;
 * acc = acc + f32(w) * f32(x) sequentially; butterfly; RNE. */
void oracle_f16_gemv(const uint16_t* W, int64_t N, int64_t K,
                     const uint16_t* x, uint16_t* y) {
  ensure_table();
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
  for (int64_t n = 0; n < N; ++n) {
    const uint16_t* row = W + n * K;
    float lanes[32];
    for (int l = 0; l < 32; ++l) {
      float acc = 0.0f;
      for (int64_t k = l; k < K; k += 32) {
        float p = g_f16_table[row[k]] * g_f16_table[x[k]];
        acc = acc + p;
      }
      lanes[l] = acc;
    }
    y[n] = oracle_f32_to_f16(butterfly32(lanes));
  }
}

void oracle_f16_gemv_f64(const uint16_t* W, int64_t N, int64_t K,
                         const uint16_t* x, double* y, double* sum_abs) {
  ensure_table();
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
  for (int64_t n = 0; n < N; ++n) {
    const uint16_t* row = W + n * K;
    double acc = 0.0, mag = 0.0;
    for (int64_t k = 0; k < K; ++k) {
      double p = (double)g_f16_table[row[k]] * (double)g_f16_table[x[k]];
      acc += p;
      mag += fabs(p);
    }
    if (y) y[n] = acc;
    if (sum_abs) sum_abs[n] = mag;
  }
}

/* ------------------------------------------------------------- argmax ---- */

/* model/qwen3_full.mlir:1469-1511.  Padding value 0xFC00 (-inf); the
 * comparison is arith.cmpf ogt on f16 (ordered: false when either side is
 * NaN), so NaN never wins and equal values keep the earlier index. */
int64_t oracle_argmax_tiled(const uint16_t* v, int64_t n, int64_t tile) {
  ensure_table();
  if (tile <= 0) return -1;
  const float NEG_INF = g_f16_table[0xFC00];
  int64_t ntiles = (n + tile - 1) / tile;
  float best_v = NEG_INF;
  int64_t best_i = -1;
  for (int64_t t = 0; t < ntiles; ++t) {
    float tv = NEG_INF;
    int64_t ti = -1;
    for (int64_t j = 0; j < tile; ++j) {
      int64_t g = t * tile + j;
      float in = g < n ? g_f16_table[v[g]] : NEG_INF;
      if (in > tv) { tv = in; ti = g; } /* ogt */
    }
    if (tv > best_v) { best_v = tv; best_i = ti; } /* phase 2, ogt */
  }
  return best_i;
}

/* OpenMP threads of the following calls (n >= 1); the CPU baseline times the
 * oracle at 1 thread and at all host threads. */
void oracle_set_num_threads(int n) {
#ifdef _OPENMP
  if (n >= 1) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
