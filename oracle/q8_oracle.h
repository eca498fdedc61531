/*
 * CPU oracle for the Qwen3 decode GEMV path (Q8_0 GEMVs + f16 vocab GEMV +
 * tiled argmax).
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only the tests,
 * the smoke check and the benchmark's CPU-baseline leg may load it.  The
 * product (the HIP kernels behind libq8gemv.so) never calls into it.
 *
 * Every function restates the reference's arithmetic on the CPU and cites
 * the reference file:line it follows (paths relative to the reference repo).
 * Half-precision values travel as raw IEEE binary16 bit patterns (uint16_t).
 */
#ifndef QWEN3_Q8_ORACLE_H
#define QWEN3_Q8_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* binary16 <-> binary32.  f16->f32 is exact widening; f32->f16 rounds to
 * nearest even (arith.truncf / __float2half semantics). */
float    oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_f16(float f);
void     oracle_f16_to_f32_array(const uint16_t* in, float* out, int64_t n);
void     oracle_f32_to_f16_array(const float* in, uint16_t* out, int64_t n);

/* Q8_0 quantizer: tools/create_q8_irpa.py:103-118.  n % 32 == 0.
 * out receives n/32 blocks of 34 bytes (f16 scale LE, then 32 int8). */
int      oracle_q8_quantize(const float* w, int64_t n, uint8_t* out);

/* Q8_0 dequantizer: tools/create_q8_irpa.py:121-129 (f32 scale * f32 q). */
void     oracle_q8_dequant(const uint8_t* blocks, int64_t nblocks, float* out);

/* Q8_0 GEMV y[N] = W[N,K] . x[K] over one layer's bytes (w_layer points at
 * layer*BPL), in the order of kernels/mlir/dispatch_{3,4,12,18,20}_gpu.mlir:
 * lane l (0..31) sums blocks b = l, l+32, ... as acc += f32(scale_b) * dot_b,
 * dot_b a sequential f32 sum over the block's 32 products; then an xor
 * butterfly 16,8,4,2,1 and round-to-nearest-even to f16.  K % 32 == 0. */
void     oracle_q8_gemv(const uint8_t* w_layer, int64_t N, int64_t K,
                        const uint16_t* x, uint16_t* y);

/* Same GEMV in float64 (near-exact: each block's 32 products sum exactly in
 * f64), plus sum_abs[n] = sum over terms |scale*q*x| (the magnitude that
 * bounds any f32 summation order's rounding error).  Either output may be
 * NULL. */
void     oracle_q8_gemv_f64(const uint8_t* w_layer, int64_t N, int64_t K,
                            const uint16_t* x, double* y, double* sum_abs);

/* f16 GEMV y[N] = W[N,K] . x[K], W row-major f16, in the order of
 * kernels/mlir/dispatch_24_gpu.mlir:75-91: lane l sums k = l, l+32, ...
 * sequentially in f32, then the xor butterfly and RNE to f16. */
void     oracle_f16_gemv(const uint16_t* W, int64_t N, int64_t K,
                         const uint16_t* x, uint16_t* y);
void     oracle_f16_gemv_f64(const uint16_t* W, int64_t N, int64_t K,
                             const uint16_t* x, double* y, double* sum_abs);

/* Two-phase tiled argmax over f16 values: model/qwen3_full.mlir:1469-1511.
 * Pads to a multiple of `tile` with -inf, phase 1 scans each tile in order
 * keeping the first strictly-greater (cmpf ogt) element, phase 2 applies the
 * same rule to the tile partials.  Returns -1 when no element is > -inf. */
int64_t  oracle_argmax_tiled(const uint16_t* v, int64_t n, int64_t tile);

/* Number of OpenMP threads the oracle uses (1 when built without OpenMP). */
int      oracle_num_threads(void);
void     oracle_set_num_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
