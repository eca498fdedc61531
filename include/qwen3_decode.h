/*
 * Qwen3-0.6B decode step on MI355X (gfx950): the glue around the Q8_0 GEMVs of
 * q8gemv.h, as one C ABI.  Implemented by libq8gemv.so (kernels in the code
 * object decode_gfx950.hsaco, loaded by q8gemv_init).
 *
 * The reference runs this step inside IREE: @generate's inner loop
 * (model/qwen3_full.mlir:1431-1526) = embedding gather, 28 x
 * @transformer_layer_decode_static (:751-864), final rms_norm, vocab matmul and
 * the tiled argmax.  Here a step is a sequence of kernel launches on one
 * stream that reads the input token and the position from device memory and
 * writes the next token back, so a step captured once in a hipGraph can be
 * replayed token after token (the reference feeds the token back on device
 * and increments the position on device, :1512-1523).
 *
 * Conventions as in q8gemv.h: device pointers owned by the caller, status
 * codes, nothing allocates, arguments validated before anything is enqueued.
 */
#ifndef QWEN3_DECODE_H
#define QWEN3_DECODE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Device pointers to the model's parameters, in the reference's layout
 * (create_q8_irpa.py:149-224; qwen3_full.mlir:66-79, 772-777): all 16-byte
 * aligned. */
typedef struct qwen3_weights {
  const void* token_embd;  /* f16 [151936, 1024] */
  const void* attn_norm;   /* f16 [28, 1024] */
  const void* ffn_norm;    /* f16 [28, 1024] */
  const void* q_norm;      /* f16 [28, 128] */
  const void* k_norm;      /* f16 [28, 128] */
  const void* wq;          /* Q8_0 [28, 2228224] */
  const void* wk;          /* Q8_0 [28, 1114112] */
  const void* wv;          /* Q8_0 [28, 1114112] */
  const void* wo;          /* Q8_0 [28, 2228224] */
  const void* wgu;         /* Q8_0 [28, 6684672] gate rows then up rows */
  const void* wdn;         /* Q8_0 [28, 3342336] */
  const void* output_norm; /* f16 [1024] */
  const void* output_w;    /* f16 [151936, 1024] (output_T.weight) */
  /* Optional (NULL when unused): f16 copies of the six layer matrices, made
   * from the Q8_0 stacks above by qwen3_prefill_matrices_expand (256-byte
   * aligned, qwen3_prefill_matrices_bytes()).  When set, the prompt GEMMs of
   * qwen3_prefill_batched / qwen3_prefill_layer read these instead of the
   * Q8_0 stacks; the decode step never reads them. */
  const void* prefill_f16;
} qwen3_weights;

/* KV cache: two f16 buffers [28 * max_seq, 8, 128] each (K, V), the flat
 * layout of qwen3_full.mlir:213-230: the entry of layer l, position p is slot
 * l * max_seq + p (:782, 795). */

/* Scratch (activations, attention partials, argmax key, status word, the
 * single-launch step's hand-off words): qwen3_scratch_bytes() bytes, 256-byte
 * aligned.  Clear it once with qwen3_scratch_reset (a kernel on `stream`)
 * before the first step; steps keep it consistent.  One scratch serves one
 * stream: concurrent steps need their own. */
size_t qwen3_scratch_bytes(void);
int qwen3_scratch_reset(void* scratch, void* stream);
/* Byte offset in the scratch of the u32 status word: bit 0 = a step asked to
 * advance past the last cache slot (the position then stays); bit 1 = a
 * single-launch step gave up waiting for a hand-off (its results are not
 * valid; it wrote neither token nor position); bit 2 = a single-launch step
 * gave up and qwen3_decode_step_checked, qwen3_prefill or qwen3_generate
 * re-ran it with the per-phase launches (the results are valid: both modes
 * compute the same bits).  A wait gives up after the spin limit, or about a
 * millisecond into a wait when not every workgroup of the launch has started
 * (the grid is not resident at once, e.g. a kernel on another stream holds
 * CUs).  Bit 1 stays set until the host clears it (qwen3_scratch_reset, or
 * the re-run above); while it is set every single-launch step on the scratch
 * returns at its start without touching token, position or cache, and
 * qwen3_generate, qwen3_prefill, qwen3_decode_step_checked and
 * qwen3_prefill_batched refuse to start. */
size_t qwen3_scratch_status_offset(void);
/* Synchronizes `stream`, then *status = the status word; returns
 * Q8_ERR_STEP_ABORTED if bit 1 is set, else Q8_OK. */
int qwen3_check_status(const void* scratch, uint32_t* status, void* stream);

/* One token: h = token_embd[*token]; 28 layers at position *pos (attention
 * over slots 0..*pos of each layer, the new k/v written to slot *pos); final
 * rms_norm; logits (f16 [151936], may be NULL); *token = argmax (lowest index
 * of the maximal f16 logit, -1 if none).  With advance != 0, *pos then moves
 * to *pos + 1 (not past max_seq - 1; see the status word).  A *pos outside
 * [0, max_seq) is clamped into it.  token and pos are device int32. */
int qwen3_decode_step(const qwen3_weights* w, void* k_cache, void* v_cache, int64_t max_seq,
                      int32_t* token, int32_t* pos, void* logits, int advance, void* scratch,
                      void* stream);

/* qwen3_decode_step, then synchronizes `stream` and checks the status word:
 * when the single launch gave up (bit 1), the step is run again with the
 * per-phase launches (the same bits; bit 2 records it, see
 * qwen3_step_fallback_count), so a successful return always means valid
 * outputs.  Fails with Q8_ERR_STEP_ABORTED if the scratch carries bit 1
 * before the call.  Not for graph capture (it synchronizes). */
int qwen3_decode_step_checked(const qwen3_weights* w, void* k_cache, void* v_cache,
                              int64_t max_seq, int32_t* token, int32_t* pos, void* logits,
                              int advance, void* scratch, void* stream);

/* Steps (process-wide, since the library was loaded) that a single launch
 * gave up on and that were re-run with the per-phase launches. */
int qwen3_step_fallback_count(uint64_t* count);

/* Test hook: the single-launch step `after` launches from now (0 = the next;
 * -1 cancels) gives up at its start as a wait that timed out would, so the
 * error and fallback paths can be exercised without a hang or a fault. */
int qwen3_debug_force_step_abort(int64_t after);

/* How qwen3_decode_step, qwen3_prefill and qwen3_generate run a step:
 * mode 1 = one launch per step (dec_step: all phases in one kernel, 448
 * workgroups resident at once handing activations over through tagged
 * words), the default where the device holds them; mode 0 = one launch per
 * phase (143 per step).  Both
 * compute every value with the same operations in the same order (tested bit
 * for bit).  Setting mode 1 on a device that cannot run it fails with
 * Q8_ERR_BAD_ARGUMENT.  Single-launch steps on different streams run one
 * after another (the library orders each launch after the previous one on
 * any other stream with an event), since two grids of 448 resident
 * workgroups do not fit at once; launches recorded under graph capture are
 * not ordered this way, so graphs holding such steps must not be replayed
 * concurrently (a step that cannot get its grid resident gives up, see the
 * status word).  No counterpart in the reference (IREE schedules its
 * dispatches itself). */
int qwen3_set_step_mode(int mode);
int qwen3_get_step_mode(int* mode);
/* Every wait of the single-launch step is bounded: after `polls` poll rounds
 * (0 = the default, 2^20, about a second) the workgroup gives up, sets status
 * bit 1 and makes every other waiter of the step give up too, so the launch
 * always completes.  A small limit forces that path (tests of the error
 * reporting); no counterpart in the reference.
 * This and the other setters of this header (step mode, prefill tiling) are
 * process-wide: they take effect for launches made after they return, on
 * every thread (a call reads each setting once). */
int qwen3_set_step_spin_limit(uint32_t polls);

/* The same step in parts, for tests and for callers that interleave work:
 * embed: h_out = token_embd[*token];
 * layer: h_out = layer `layer` of h_in at position *pos (h_in, h_out f16[1024],
 *        distinct; uses and overwrites the scratch activations);
 * head:  logits / *token / *pos as in qwen3_decode_step from the final h. */
int qwen3_decode_embed(const qwen3_weights* w, const int32_t* token, void* h_out, void* stream);
int qwen3_decode_layer(const qwen3_weights* w, int layer, void* k_cache, void* v_cache,
                       int64_t max_seq, const int32_t* pos, const void* h_in, void* h_out,
                       void* scratch, void* stream);
int qwen3_decode_head(const qwen3_weights* w, const void* h, void* logits, int32_t* token,
                      int32_t* pos, int advance, int64_t max_seq, void* scratch, void* stream);

/* Prompt ingestion as decode steps, the reference's @prefill_all
 * (qwen3_full.mlir:1541-1561): for i in [0, n_prompt) one step at position
 * *pos with input token prompt[i] (device int32 [n_prompt]); logits are only
 * formed after the last prompt token, whose argmax goes to *token.  *pos ends
 * n_prompt slots further (not past max_seq - 1; see the status word).  In
 * step mode 0 it only enqueues: check the status word (qwen3_check_status)
 * before trusting the token.  In step mode 1 it synchronizes `stream` at its
 * start and after the steps: when a single launch gave up, the steps from it
 * on are run again with the per-phase launches (status bit 2), and it fails
 * with Q8_ERR_STEP_ABORTED if the scratch carried bit 1 before the call or
 * the cache filled up (bit 0) in an aborted run. */
int qwen3_prefill(const qwen3_weights* w, void* k_cache, void* v_cache, int64_t max_seq,
                  const int32_t* prompt, int32_t n_prompt, int32_t* token, int32_t* pos,
                  void* scratch, void* stream);

/* Prompt ingestion with every prompt token of a layer processed together, the
 * reference's @prefill (qwen3_full.mlir:2032-2111, layers :1731-2030): the
 * layer matrices become GEMMs over the n_prompt tokens.  Token i (prompt[i],
 * device int32 [n_prompt]) sits at position p0 + i, p0 = *pos (read on the
 * host: the call synchronizes `stream` once); each layer writes the tokens'
 * k/v to those cache slots, and token i attends to slots [lo, p0 + i] with
 * lo = 0 when chunk_local == 0 (the whole cache, what qwen3_prefill's decode
 * steps see) or lo = p0 when chunk_local != 0 (this call's tokens only, the
 * reference's @prefill, whose mask j <= i covers its own tokens, :1700-1710;
 * the same thing when p0 = 0).  Then, as in qwen3_prefill: the last token's
 * logits (f16 [151936], may be NULL), *token = their argmax, *pos = p0 +
 * n_prompt (at p0 + n_prompt = max_seq it stays at max_seq - 1 and status bit
 * 0 is set).  Fails with Q8_ERR_BAD_SHAPE unless p0 + n_prompt <= max_seq.
 * workspace: device memory of qwen3_prefill_workspace_bytes(n_prompt) bytes,
 * 256-byte aligned (activations of all tokens, 30,720 bytes per token, then
 * the attention's split partials, 266,240 bytes per (query block of 32 tokens,
 * split) pair for 2 ceil(n_prompt / 32) + 64 pairs).  The
 * reference reads f16 copies of the layer matrices for this function
 * (@model_params.attn_q_weight etc., :1132-1210), made from a Q8_0 file as
 * f16(scale * q) with the product exact (tools/convert_gguf_to_irpa.py:28-44,
 * 174-199).  With w->prefill_f16 set this function reads such copies
 * (qwen3_prefill_matrices_expand); without it, it reads the decode step's
 * Q8_0 stacks and forms the same f16 weights in registers.  Both routes give
 * the same bits (the same MFMA instructions on the same values in the same
 * order); the f16 one runs no conversion in its GEMM loops.  (The decode
 * GEMVs scale each block's exact dot instead, as the reference's decode
 * kernels do; the two routes' logits differ by about 2e-3 relative.) */
size_t qwen3_prefill_workspace_bytes(int32_t n_prompt);

/* The f16 layer matrices of qwen3_weights.prefill_f16: bytes needed
 * (880,803,840: 28 layers x 15,728,640 f16 weights) and their expansion from
 * w's Q8_0 stacks into `matrices` (device memory, 256-byte aligned, at least
 * that many bytes), enqueued on `stream`.  Each weight becomes f16(scale * q),
 * the f16 value the reference's converter writes for it
 * (tools/convert_gguf_to_irpa.py:28-44, 174-199).  Per layer: q, k and v rows
 * as one [4096, 1024] matrix, attn_o [1024, 2048], gate/up [6144, 1024] with
 * the rows in groups of 32 (16 gate rows, then the 16 up rows of the same
 * SwiGLU outputs), ffn_down [1024, 3072].  Run it again after the Q8_0 stacks
 * change.  No counterpart call in the reference (its converter writes the f16
 * matrices to the parameter file). */
size_t qwen3_prefill_matrices_bytes(void);
int qwen3_prefill_matrices_expand(const qwen3_weights* w, void* matrices, size_t bytes,
                                  void* stream);

int qwen3_prefill_batched(const qwen3_weights* w, void* k_cache, void* v_cache, int64_t max_seq,
                          const int32_t* prompt, int32_t n_prompt, int32_t* token, int32_t* pos,
                          void* logits, int chunk_local, void* workspace, size_t workspace_bytes,
                          void* scratch, void* stream);

/* One layer of qwen3_prefill_batched, for tests and for callers that
 * interleave work (@transformer_layer_prefill, qwen3_full.mlir:1731-2030):
 * the n_tokens hidden rows in the workspace's "h" region (f16 [n_tokens,
 * 1024]) at positions start_pos.. (host int) are replaced by the layer's
 * output; the layer's k/v go to those cache slots; the intermediates stay in
 * the workspace.  qwen3_prefill_workspace_offset(n_tokens, name) = byte
 * offset of a region ("h", "res", "xn", "q", "k", "v", "q_roped", "attn",
 * "act", "fn"; f16 rows of 1024, 1024, 1024, 2048, 1024, 1024, 2048, 2048,
 * 3072, 1024 columns; then "attn_part", the attention's split partials, and
 * "rope", f32 [n_tokens, 128]: the RoPE cosines and sines of each token's
 * position), -1 for an unknown name. */
int qwen3_prefill_layer(const qwen3_weights* w, int layer, void* k_cache, void* v_cache,
                        int64_t max_seq, int32_t n_tokens, int32_t start_pos, int chunk_local,
                        void* workspace, size_t workspace_bytes, void* stream);
int64_t qwen3_prefill_workspace_offset(int32_t n_tokens, const char* name);

/* Work division of qwen3_prefill_batched / qwen3_prefill_layer (0 = the
 * default, for either):
 * gemm_rows: token rows per GEMM workgroup, 32, 64 or 128.  Over the Q8_0
 *   stacks: the q/k/v, attn_o and ffn_down GEMMs (gate/up always uses 64),
 *   32 or 64 (128 = 64); default: 32 where 64 would give fewer than 2
 *   workgroups per CU.  Over the f16 matrices: every GEMM, the tile of that
 *   many rows (the next larger where the GEMM has none); default: per GEMM the
 *   first of its tiles, largest first, whose grid fills the CUs with the
 *   workgroups that tile is built to share a CU with.  Every tile computes
 *   each output with the same operations in the same order (tested bit for
 *   bit).
 * attn_split_blocks: cache positions per attention split, in blocks of 32
 *   (>= 1; raised where the workspace's partial slots would not hold the
 *   splits); default a third of the longest query block's positions, at
 *   least 8 blocks.  Splits change the order of the softmax sums, within
 *   the attention tolerance.
 * Fails with Q8_ERR_BAD_ARGUMENT for other values.  No counterpart in the
 * reference (IREE tiles its dispatches at compile time). */
int qwen3_set_prefill_tiling(int gemm_rows, int attn_split_blocks);

/* The token loop of @generate (qwen3_full.mlir:1396-1534): starting from
 * *token at *pos, steps run in batches of 4 (fewer for the last) with the
 * token fed back and the position advanced on the device; step i's token goes
 * to out_tokens[i] (device int32 [max_new]).  After each batch the host reads
 * the last token and stops if it equals eos_id, so up to 3 tokens past an EOS
 * are produced, as in the reference.  The input token itself is not output.
 * *n_generated (host) = tokens produced.  Blocks until the loop ends; fails
 * with Q8_ERR_BAD_SHAPE unless *pos + max_new <= max_seq, and with
 * Q8_ERR_STEP_ABORTED if the scratch carries status bit 1 before the loop.
 * When a single-launch step gives up, the batch is re-run from that step with
 * the per-phase launches (status bit 2; the same tokens) and the loop goes on
 * in that mode.  The next batch is queued before the host checks the current
 * one; when the current one ends the loop, *token, *pos and the status are
 * restored to their values after it, but out_tokens slots past *n_generated
 * may hold the queued batch's tokens. */
int qwen3_generate(const qwen3_weights* w, void* k_cache, void* v_cache, int64_t max_seq,
                   int32_t* token, int32_t* pos, int32_t max_new, int32_t eos_id,
                   int32_t* out_tokens, int32_t* n_generated, void* scratch, void* stream);

/* Scratch offsets of the intermediates the last qwen3_decode_layer (or head)
 * left behind, all f16: "xn" [1024] rms_norm(h_in, attn_norm); "q" [2048],
 * "k" [1024], "v" [1024] the projections before head norm and RoPE;
 * "q_roped" [2048] q after head norm and RoPE; "attn" [2048] attention
 * output; "res" [1024] residual after attention; "fn" [1024]
 * rms_norm(res, ffn_norm); "act" [3072] SwiGLU output; "on" [1024] the final
 * rms_norm(h, output_norm) of the head; "part" f32 [16][8][132] the attention
 * partials of the per-phase layer (the single-launch step does not use this
 * region; its timestamp build records its clock reads there).  -1 for an
 * unknown name. */
int64_t qwen3_scratch_offset(const char* name);

#ifdef __cplusplus
}
#endif
#endif
