/*
 * libq8gemv: C ABI of the MI355X (gfx950) decode-GEMV path of Qwen3-0.6B.
 *
 * The reference substitutes six IREE dispatch executables with hand-written
 * kernels at compile time (compile.sh:35-43, --iree-hal-substitute-executable-
 * source=decode_dispatch_N=FILE).  Each executable's binding ABI is
 *   (binding0 weights RO, binding1 input buffer RO, binding2 output buffer)
 *   + i32 push constants (layer as lo/hi, output byte offset)
 * with the x / y byte offsets baked into each kernel
 * (kernels/cuda/dispatch_3.cu:8-22, dispatch_4.cu:8-22, dispatch_24.cu:11-20;
 * layouts in kernels/cuda/dispatch_*.mlir:5).  This library keeps that ABI's
 * data contract -- GGUF Q8_0 34-byte blocks, [N,K] row-major weights stacked
 * per layer as [28, BPL] bytes, f16 x, f32 accumulation, f16 y -- and takes
 * explicit device pointers instead of baked-in offsets.
 *
 * Conventions
 *   - Every pointer argument of a compute entry point is a device pointer the
 *     caller owns.  Compute entry points only enqueue work on `stream` (a
 *     hipStream_t; NULL = the null stream) and never allocate.
 *   - Every function returns Q8_OK (0) or a Q8_ERR_* code; q8gemv_last_error()
 *     gives the message for the calling thread.  Arguments are validated on
 *     the host before anything is enqueued; nothing aborts the process.
 *   - Compute entry points are safe to call from several host threads, each
 *     with its own stream, once q8gemv_init() has returned.  One exception:
 *     f16_gemv_argmax_rows_noalloc keeps its argmax key in one array per GPU,
 *     so its calls must not overlap on a GPU (streams not ordered with each
 *     other, or a graph replay beside eager calls).
 *   - Setters of tuning knobs (q8gemv_batch_set_workgroups,
 *     vocab_set_workgroups and those of qwen3_decode.h) are process-wide and
 *     may be called from any thread; a launch reads each knob once, so it
 *     sees either the old or the new value.
 *   - Alignment: weights and x 16 bytes, y / logits 2 bytes, token 4 bytes,
 *     workspace 16 bytes.
 */
#ifndef QWEN3_Q8GEMV_H
#define QWEN3_Q8GEMV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---- */
#define Q8_OK                  0
#define Q8_ERR_NOT_INITIALIZED 1  /* q8gemv_init() not called or failed */
#define Q8_ERR_INVALID_KIND    2  /* kind outside enum q8_kind */
#define Q8_ERR_NULL_POINTER    3  /* a required pointer is NULL */
#define Q8_ERR_LAYER_RANGE     4  /* layer outside [0, Q8_NUM_LAYERS) */
#define Q8_ERR_MISALIGNED      5  /* pointer alignment below the contract */
#define Q8_ERR_BAD_SHAPE       6  /* unsupported N / K / row count */
#define Q8_ERR_CODE_OBJECT     7  /* code object missing, unreadable or lacks a kernel */
#define Q8_ERR_HIP             8  /* a HIP runtime call failed (message has details) */
#define Q8_ERR_BAD_ARGUMENT    9  /* other invalid argument (tuning values, sizes) */
#define Q8_ERR_STEP_ABORTED   10  /* a single-launch decode step gave up waiting (qwen3_decode.h) */

/* ---- model constants (model/qwen3_full.mlir:29-64; tools/create_q8_irpa.py:16-25) ---- */
#define Q8_NUM_LAYERS   28
#define Q8_BLOCK_ELEMS  32
#define Q8_BLOCK_BYTES  34
#define Q8_VOCAB_ROWS   151936
#define Q8_HIDDEN       1024

/* The five Q8_0 GEMV kinds, in the per-layer call order of
 * model/qwen3_full.mlir:751-864 (q, k, v, o, gate_up, down). */
enum q8_kind {
  Q8_ATTN_Q   = 0, /* [2048,1024] decode_dispatch_3,  qwen3_full.mlir:625       */
  Q8_ATTN_KV  = 1, /* [1024,1024] decode_dispatch_4,  qwen3_full.mlir:630, 635  */
  Q8_ATTN_O   = 2, /* [1024,2048] decode_dispatch_12, qwen3_full.mlir:739       */
  Q8_GATE_UP  = 3, /* [6144,1024] decode_dispatch_18, qwen3_full.mlir:820       */
  Q8_FFN_DN   = 4  /* [1024,3072] decode_dispatch_20, qwen3_full.mlir:852       */
};

/* ---- lifetime ---- */

/* Loads the gfx950 code object (hipModuleLoad) on the current device and
 * resolves every kernel.  code_object_path NULL = "q8gemv_gfx950.hsaco" in
 * the directory holding this library.  Idempotent.  Replaces the compile-time
 * substitution step of compile.sh:35-43. */
int q8gemv_init(const char* code_object_path);
void q8gemv_shutdown(void);
const char* q8gemv_last_error(void);

/* Shape of a kind: N rows, K columns, bytes per layer N*K/32*34
 * (create_q8_irpa.py:195-197).  Any output pointer may be NULL. */
int q8gemv_kind_shape(int kind, int64_t* n, int64_t* k, int64_t* bytes_per_layer);

/* ---- Q8_0 GEMV ---- */

/* y[N] = W[layer] . x[K] for one kind.  w_stacked points at the [28, BPL]
 * stacked buffer (create_q8_irpa.py:185-224); the layer's rows start at
 * w_stacked + layer*BPL, row n at + n*K/32*34 (dispatch_3.cu:17-32).
 * Replaces the body of @q8_fused_gemv (qwen3_full.mlir:536-589) as executed
 * by decode_dispatch_{3,4,12,18,20}. */
int q8gemv(int kind, const void* w_stacked, int64_t layer, const void* x_f16,
           void* y_f16, void* stream);

/* Generic form over one layer's bytes: n_rows >= 1 rows of K = 1024, 2048 or
 * 3072 columns starting at w_layer. */
int q8gemv_rows(const void* w_layer, int64_t n_rows, int64_t k, const void* x_f16,
                void* y_f16, void* stream);

/* The five Q8 dispatches under the reference's executable names.
 * decode_dispatch_3_matmul_2048x1x1024_f16   kernels/cuda/dispatch_3.cu:8-13
 * decode_dispatch_4_matmul_1024x1x1024_f16   kernels/cuda/dispatch_4.cu:8-13
 * decode_dispatch_12_matmul_1024x1x2048_f16  kernels/cuda/dispatch_12.cu
 * decode_dispatch_18_matmul_6144x1x1024_f16  kernels/cuda/dispatch_18.cu
 * decode_dispatch_20_matmul_1024x1x3072_f16  kernels/cuda/dispatch_20.cu
 * The reference's (binding, push-constant) pairs become (w_stacked, layer,
 * x, y): the layer push constants c0|c1<<32 (dispatch_3.cu:19) are `layer`;
 * dispatch_4's output byte offset c0 (dispatch_4.cu:19-22) is folded into y. */
int decode_dispatch_3_matmul_2048x1x1024_f16(const void* q8_stacked, int64_t layer,
                                             const void* x_f16, void* y_f16, void* stream);
int decode_dispatch_4_matmul_1024x1x1024_f16(const void* q8_stacked, int64_t layer,
                                             const void* x_f16, void* y_f16, void* stream);
int decode_dispatch_12_matmul_1024x1x2048_f16(const void* q8_stacked, int64_t layer,
                                              const void* x_f16, void* y_f16, void* stream);
int decode_dispatch_18_matmul_6144x1x1024_f16(const void* q8_stacked, int64_t layer,
                                              const void* x_f16, void* y_f16, void* stream);
int decode_dispatch_20_matmul_1024x1x3072_f16(const void* q8_stacked, int64_t layer,
                                              const void* x_f16, void* y_f16, void* stream);

/* q, k and v of one layer in one launch (no reference counterpart: the
 * reference runs decode_dispatch_3 once and decode_dispatch_4 twice on the
 * same normed input, model/qwen3_full.mlir:625-635).  wq_stacked is the
 * [28, 2228224] attn_q buffer, wk_stacked / wv_stacked the [28, 1114112]
 * attn_k / attn_v buffers; yq receives 2048 values, yk and yv 1024 each.
 * Each output is bit-identical to the corresponding q8gemv call. */
int q8gemv_qkv(const void* wq_stacked, const void* wk_stacked, const void* wv_stacked,
               int64_t layer, const void* x_f16, void* yq_f16, void* yk_f16, void* yv_f16,
               void* stream);

/* ---- batched Q8_0 GEMVs: several independent GEMVs in one launch (no
 * reference counterpart; the reference issues one dispatch per GEMV) ----
 *
 * For GEMVs that do not depend on each other -- q, k and v of a layer, which
 * read the same x (qwen3_full.mlir:625-635), or any list of independent calls
 * -- one launch replaces one dispatch each: the batch's row quads are spread
 * evenly over the whole GPU, so small GEMVs stop paying a dispatch apiece.
 * Every row is computed exactly as q8gemv_rows computes it (bit-identical).
 * The outputs must not overlap each other or any input. */
typedef struct q8gemv_desc {
  const void* w_layer; /* first row of the layer's Q8_0 bytes, 16-byte aligned */
  const void* x_f16;   /* K f16 values, 16-byte aligned */
  void* y_f16;         /* n_rows f16 outputs, 2-byte aligned */
  int64_t n_rows;      /* 1 .. 2^24 */
  int64_t k;           /* 1024, 2048 or 3072 */
} q8gemv_desc;

/* Fills *out for one kind's layer of a [28, BPL] stacked buffer. */
int q8gemv_desc_for_kind(int kind, const void* w_stacked, int64_t layer, const void* x_f16,
                         void* y_f16, q8gemv_desc* out);
/* Bytes of the device table for `count` descriptors (0 if count is out of
 * range). */
size_t q8gemv_batch_table_bytes(int count);
/* Validates the descriptors (as q8gemv_rows would) and encodes them into a
 * host buffer of q8gemv_batch_table_bytes(count) bytes; *total_units receives
 * the work size to pass to q8gemv_batch.  Host-only: copy the table to device
 * memory (any allocation the caller owns, 16-byte aligned) before launching. */
int q8gemv_batch_encode(const q8gemv_desc* descs, int count, void* host_table,
                        size_t table_bytes, int32_t* total_units);
/* Launches every GEMV of an encoded table that was copied to the device
 * unchanged.  The table is read by the kernel, so it must stay valid until
 * the launch completes; it can be reused by any number of launches. */
int q8gemv_batch(const void* device_table, int count, int32_t total_units, void* stream);

/* ---- f16 vocab GEMV + fused two-phase argmax ---- */

/* Workspace of the fused argmax: a 64-bit (value, index) key that every
 * workgroup folds its best candidate into with an atomic max.  It must be
 * zero before the first launch that uses it (vocab_argmax_workspace_reset, or
 * a zero fill); every launch leaves it zero again.  Two launches must not
 * share a workspace concurrently. */
size_t vocab_argmax_workspace_bytes(void);
int vocab_argmax_workspace_reset(void* workspace, void* stream);

/* logits[151936] = f16(W[151936,1024] . x) and *token = the lowest index of
 * the maximal f16 logit (-1 if none is > -inf; NaN never wins).  Enqueues two
 * kernels: the GEMV with the per-workgroup argmax phase, then a one-thread
 * finalize that writes *token.
 * decode_dispatch_24_matmul_151936x1x1024_f16 (kernels/cuda/dispatch_24.cu:11-46)
 * fused with the tiled argmax of qwen3_full.mlir:1469-1511 (i64 there, int32
 * here).  logits may be NULL to skip writing them. */
int vocab_gemv_argmax(const void* w_f16, const void* x_f16, void* logits_f16,
                      int32_t* token, void* workspace, void* stream);
int decode_dispatch_24_matmul_151936x1x1024_f16(const void* w_f16, const void* x_f16,
                                                void* logits_f16, int32_t* token,
                                                void* workspace, void* stream);

/* Generic form: n_rows in [1, 2^31) rows of K = 1024. */
int f16_gemv_argmax_rows(const void* w_f16, int64_t n_rows, const void* x_f16,
                         void* logits_f16, int32_t* token, void* workspace, void* stream);

/* f16_gemv_argmax_rows without a workspace argument: allocates nothing and
 * takes no caller memory beyond inputs and outputs.  No counterpart in the
 * reference; for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The argmax key lives
 * in a 256-byte device array inside this library, one per GPU, held until the
 * process ends and set up (address lookup, zero fill) by q8gemv_init on its
 * device; the fixed size serves any n_rows in [1, 2^31), and every call leaves
 * the key zero again.  All calls on one GPU share that array: calls that
 * overlap on one GPU (streams not ordered with each other) race on it.
 * Returns Q8_ERR_NOT_INITIALIZED if q8gemv_init has not set it up on the
 * current device.  Outputs are bit-identical to f16_gemv_argmax_rows. */
int f16_gemv_argmax_rows_noalloc(const void* w_f16, int64_t n_rows, const void* x_f16,
                                 void* logits_f16, int32_t* token, void* stream);

/* Argmax of n f16 values already in memory (logits of an earlier launch,
 * such as decode_dispatch_24_matmul_151936x1x1024_f16 through the HAL ABI,
 * which writes logits only): the reference's tiled argmax as its own pass
 * (model/qwen3_full.mlir:1469-1511) -- the lowest index of the maximal value,
 * NaN never winning, -1 if no value wins.  Same workspace rule as
 * vocab_gemv_argmax (256 bytes, zero between calls; the call leaves it
 * zero).  n in [1, 2^31), values 16-byte aligned. */
int f16_argmax(const void* values_f16, int64_t n, int32_t* token, void* workspace,
               void* stream);

/* ---- the reference's own binding ABI ----
 *
 * The code object also exports the six kernels under the reference's
 * executable names with IREE's HAL binding ABI (binding base pointers, then
 * i32 push constants; x / y at the byte offsets the reference bakes in:
 * kernels/cuda/dispatch_3.cu:19-21, dispatch_4.cu:19-22, dispatch_12.cu:19-21,
 * dispatch_18.cu:19-21, dispatch_20.cu:19-21, dispatch_24.cu:19-20), so an
 * IREE ROCm build can substitute them (compile.sh:35-43; stubs in
 * INTEGRATION.md).  This launches one of them exactly as such a stub would:
 * ordinal 3, 4, 12, 18, 20 or 24; push constants as the reference defines them
 * (layer = c0 | c1 << 32; dispatch 4: c0 = output byte offset, layer =
 * c1 | c2 << 32; dispatch 24: c0 = output byte offset, logits only). */
int q8gemv_hal_dispatch(int ordinal, const void* binding0, const void* binding1, void* binding2,
                        const uint32_t* push_constants, int n_constants, void* stream);
/* The same with the stub's launch shape: `workgroups` x `workgroup_size`
 * threads (0 = this build's stub shape: 64 threads and N/4 workgroups, 256
 * threads and 1024 workgroups for ordinal 24).  The kernels compute every
 * output under any shape with 64, 128, 192 or 256 threads per workgroup,
 * including the reference stubs' own (256 threads; 256, 128, 128, 768, 128 and
 * 18992 workgroups, kernels/cuda/dispatch_{3,4,12,18,20,24}.mlir:5-9). */
int q8gemv_hal_dispatch_grid(int ordinal, const void* binding0, const void* binding1,
                             void* binding2, const uint32_t* push_constants, int n_constants,
                             uint32_t workgroups, uint32_t workgroup_size, void* stream);

/* ---- launch-shape tuning (no reference counterpart) ---- */

/* Upper bound on the workgroups (one wave each) of a batched Q8_0 launch;
 * 0 = default (10 per compute unit).  A launch never uses more workgroups than
 * it has work units.  (A single GEMV always runs one wave per row quad.) */
int q8gemv_batch_set_workgroups(int workgroups);
/* Workgroups (256 threads) of the vocab kernel, 1..8192; 0 = default
 * (1 per compute unit). */
int vocab_set_workgroups(int workgroups);
int vocab_get_workgroups(int* workgroups);

/* ---- device runtime helpers (no reference counterpart: the IREE HAL owns
 * allocation, streams and timing there, benchmark.py:34-49).  The copy and
 * memset helpers are set-up tools, fully synchronous with the device: they
 * wait for all prior work on every stream and return after completing. ---- */
int q8rt_device_count(int* count);
int q8rt_set_device(int device);
int q8rt_device_info(char* name, int name_len, int* compute_units, int64_t* total_mem);
int q8rt_malloc(void** ptr, size_t bytes);
int q8rt_free(void* ptr);
int q8rt_memcpy_htod(void* dst_device, const void* src_host, size_t bytes);
int q8rt_memcpy_dtoh(void* dst_host, const void* src_device, size_t bytes);
int q8rt_memcpy_dtod(void* dst_device, const void* src_device, size_t bytes);
int q8rt_memset(void* ptr, int value, size_t bytes);
int q8rt_device_synchronize(void);
int q8rt_stream_create(void** stream);
int q8rt_stream_destroy(void* stream);
int q8rt_stream_synchronize(void* stream);
int q8rt_event_create(void** event);
int q8rt_event_destroy(void* event);
int q8rt_event_record(void* event, void* stream);
int q8rt_event_synchronize(void* event);
int q8rt_event_elapsed_ms(float* ms, void* start, void* stop);
/* Stream capture into a hipGraph and replay. */
int q8rt_graph_begin_capture(void* stream);
int q8rt_graph_end_capture(void* stream, void** graph_exec);
int q8rt_graph_launch(void* graph_exec, void* stream);
int q8rt_graph_destroy(void* graph_exec);
/* Device-to-device copy by a plain streaming kernel (16-byte aligned pointers,
 * bytes % 16 == 0; bytes = 0 launches one empty workgroup).  A kernel of known
 * traffic for calibrating HBM byte counters and dispatch overhead. */
int q8rt_stream_copy(void* dst, const void* src, size_t bytes, void* stream);
/* Reads `bytes` at src (16-byte aligned, bytes % 16 == 0) with a plain
 * streaming kernel and writes nothing (in practice: a word of src only if the
 * XOR of a thread's reads equals a fixed 32-bit value).  Reading more than the
 * 256 MB memory-side cache (MALL) holds evicts it without leaving dirty lines
 * that a following kernel would pay to write back. */
int q8rt_stream_read(const void* src, size_t bytes, void* stream);
/* The calling thread's next kernel launch through this library records
 * `start` / `stop` around that kernel alone (hipExtModuleLaunchKernel
 * events), for per-kernel timing.  One-shot. */
int q8rt_time_next_launch(void* start_event, void* stop_event);

/* ---- measurement tools (allocate their own buffers and synchronize the
 * device; not compute entry points) ---- */
/* Mean time per launch of an empty kernel of `workgroups` x `threads` with
 * `lds_bytes` of LDS each, `launches` of them back to back on a fresh stream,
 * as ordinary launches or (cooperative != 0) cooperative ones: the launch
 * cost the single-launch decode step's grid (448 x 256, 79,360 LDS bytes)
 * pays per step. */
int q8rt_launch_cost(int cooperative, int workgroups, int threads, size_t lds_bytes,
                     int launches, float* us_per_launch);
/* Latency of the single-launch decode step's hand-off (tagged 8-byte words,
 * agent-scope atomic stores and polls): `producers` workgroups each store
 * n_words / producers words of a vector into each of `replicas` copies, all
 * at the same clock tick; `consumers` further workgroups each poll one copy
 * (consumer c: copy c % replicas) until every word carries the round's tag.
 * latency_us[r * consumers + c] (host, rounds x consumers) = when consumer c
 * held the whole vector in round r minus when the last producer's stores were
 * issued, from the 100 MHz device clock (10 ns ticks; a consumer can see
 * the words a few ticks before the last producer's clock read), NaN (and
 * counted in *failed) where a bounded wait gave up.  n_words % producers == 0, producers + consumers <=
 * 512, rounds <= 255; rounds are 20 us apart. */
int q8rt_handoff_latency(int producers, int consumers, int n_words, int replicas, int rounds,
                         float* latency_us, int* failed);
/* Load-to-use latency of one lane's dependent loads (a pointer chase through
 * `hops` distinct 128-byte lines of a 64 MiB buffer, 16 <= hops <= 65536):
 * ns_per_load[0] with every line in HBM only (a 1 GiB read first evicts L2
 * and the 256 MB memory-side cache), [1] from the memory-side cache (the same
 * lines chased again from another XCD, whose L2 never held them), [2] from
 * the chasing XCD's own L2 (the same lines at once again); NaN where a pass
 * could not be placed.  xcds[0], xcds[1]: the XCD ids of the two chasing
 * workgroups.  The single-dispatch GEMVs wait for their first weight bytes
 * about [0] after their start. */
int q8rt_memory_latency(int hops, float* ns_per_load, int* xcds);

#ifdef __cplusplus
}
#endif
#endif
