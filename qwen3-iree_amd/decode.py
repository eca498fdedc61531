"""Host side of the Qwen3-0.6B decode step (include/qwen3_decode.h).

The reference runs a token as @generate's inner loop inside IREE
(model/qwen3_full.mlir:1431-1526): embedding gather, 28 x
@transformer_layer_decode_static, final rms_norm, the vocab GEMV and the tiled
argmax, with the token fed back and the position incremented on the device.
Here the same step is one C call that enqueues 143 gfx950 kernel launches on a
stream (libq8gemv.so); this module owns the device buffers it needs (weights,
the flat KV cache, scratch, token and position words), captures the step in a
hipGraph and replays it.

Weights come in the reference's parameter layout (create_q8_irpa.py:149-224):
Q8_0 stacks [28, BPL] bytes, gate and up concatenated by rows, f16 norms and
f16 embedding / output matrices.  No checkpoint is available offline, so
`synthetic_weights` draws them from seeded normal distributions.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, fields

import numpy as np

from . import q8gemv as Q
from . import weights as Wt

LAYERS = 28
HIDDEN = 1024
Q_HEADS, KV_HEADS, HEAD_DIM = 16, 8, 128
Q_DIM, KV_DIM = Q_HEADS * HEAD_DIM, KV_HEADS * HEAD_DIM
FFN = 3072
VOCAB = 151936
WEIGHT_FIELDS = ("token_embd", "attn_norm", "ffn_norm", "q_norm", "k_norm", "wq", "wk", "wv",
                 "wo", "wgu", "wdn", "output_norm", "output_w")
# (rows, cols) of each Q8_0 matrix per layer (qwen3_full.mlir:772-777)
Q8_SHAPES = {"wq": (Q_DIM, HIDDEN), "wk": (KV_DIM, HIDDEN), "wv": (KV_DIM, HIDDEN),
             "wo": (HIDDEN, Q_DIM), "wgu": (2 * FFN, HIDDEN), "wdn": (HIDDEN, FFN)}
# workspace regions of the batched prompt path (name, f16 columns per token)
PREFILL_REGIONS = (("h", HIDDEN), ("res", HIDDEN), ("xn", HIDDEN), ("q", Q_DIM), ("k", KV_DIM),
                   ("v", KV_DIM), ("q_roped", Q_DIM), ("attn", Q_DIM), ("act", FFN),
                   ("fn", HIDDEN))
NORM_STD = 0.1


@dataclass
class HostWeights:
    """numpy copies of every parameter, in the device layout."""
    token_embd: np.ndarray   # f16 [151936, 1024]
    attn_norm: np.ndarray    # f16 [28, 1024]
    ffn_norm: np.ndarray     # f16 [28, 1024]
    q_norm: np.ndarray       # f16 [28, 128]
    k_norm: np.ndarray       # f16 [28, 128]
    wq: np.ndarray           # u8 [28, 2228224]
    wk: np.ndarray           # u8 [28, 1114112]
    wv: np.ndarray           # u8 [28, 1114112]
    wo: np.ndarray           # u8 [28, 2228224]
    wgu: np.ndarray          # u8 [28, 6684672]
    wdn: np.ndarray          # u8 [28, 3342336]
    output_norm: np.ndarray  # f16 [1024]
    output_w: np.ndarray     # f16 [151936, 1024]

    def validate(self) -> None:
        want = {"token_embd": ((VOCAB, HIDDEN), np.float16),
                "attn_norm": ((LAYERS, HIDDEN), np.float16),
                "ffn_norm": ((LAYERS, HIDDEN), np.float16),
                "q_norm": ((LAYERS, HEAD_DIM), np.float16),
                "k_norm": ((LAYERS, HEAD_DIM), np.float16),
                "output_norm": ((HIDDEN,), np.float16),
                "output_w": ((VOCAB, HIDDEN), np.float16)}
        for name, (n, k) in Q8_SHAPES.items():
            want[name] = ((LAYERS, n * k // 32 * 34), np.uint8)
        for name, (shape, dtype) in want.items():
            a = getattr(self, name)
            if a.shape != shape or a.dtype != dtype or not a.flags["C_CONTIGUOUS"]:
                raise ValueError(f"{name}: expected contiguous {np.dtype(dtype)}{shape}, "
                                 f"got {a.dtype}{a.shape}")


def _norm_weights(shape, seed: int, tensor: int) -> np.ndarray:
    r = Wt._rng(seed, tensor, 0).standard_normal(shape, dtype=np.float32)
    return (np.float32(1.0) + np.float32(NORM_STD) * r).astype(np.float16)


def synthetic_weights(seed: int = 0, workers: int = 8) -> HostWeights:
    """Random-init Qwen3-0.6B parameters: matrices N(0, 0.02) (Q8_0 through
    the reference quantizer), norm weights 1 + N(0, 0.1), embedding and output
    matrices f16(N(0, 0.02)).  One PCG64 stream per (seed, tensor, layer)."""
    q8 = {name: Wt.synthetic_q8_stack(n, k, LAYERS, seed, 10 + i, workers)
          for i, (name, (n, k)) in enumerate(Q8_SHAPES.items())}
    hw = HostWeights(
        token_embd=Wt.synthetic_f16_matrix(VOCAB, HIDDEN, seed, 100, workers),
        attn_norm=_norm_weights((LAYERS, HIDDEN), seed, 101),
        ffn_norm=_norm_weights((LAYERS, HIDDEN), seed, 102),
        q_norm=_norm_weights((LAYERS, HEAD_DIM), seed, 103),
        k_norm=_norm_weights((LAYERS, HEAD_DIM), seed, 104),
        output_norm=_norm_weights((HIDDEN,), seed, 105),
        output_w=Wt.synthetic_f16_matrix(VOCAB, HIDDEN, seed, 106, workers),
        **q8)
    hw.validate()
    return hw


class WeightsC(ctypes.Structure):
    """struct qwen3_weights (include/qwen3_decode.h)."""
    _fields_ = [(f, ctypes.c_void_p) for f in WEIGHT_FIELDS] + [("prefill_f16", ctypes.c_void_p)]


def prefill_matrices_bytes() -> int:
    """Bytes of the f16 layer matrices the prompt GEMMs can read."""
    return int(Q.load_library().qwen3_prefill_matrices_bytes())


class DeviceWeights:
    """The parameters resident in device memory, one allocation each.

    prefill_f16: also make the f16 copies of the layer matrices
    (qwen3_prefill_matrices_expand, 0.88 GB) that the batched prompt path
    then reads instead of forming them from Q8_0 in its GEMM loops."""

    def __init__(self, host: HostWeights, prefill_f16: bool = True):
        host.validate()
        self.buffers = {f.name: Q.DeviceBuffer.from_array(getattr(host, f.name))
                        for f in fields(HostWeights)}
        self.struct = WeightsC(*(self.buffers[f].ptr for f in WEIGHT_FIELDS), None)
        self.prefill_matrices: Q.DeviceBuffer | None = None
        if prefill_f16:
            self.expand_prefill_matrices()

    def expand_prefill_matrices(self) -> None:
        """(Re)make the f16 layer matrices from the resident Q8_0 stacks and
        point the struct at them."""
        if self.prefill_matrices is None:
            self.prefill_matrices = Q.DeviceBuffer(prefill_matrices_bytes())
        stream = Q.Stream()
        try:
            self.struct.prefill_f16 = None
            Q._call("qwen3_prefill_matrices_expand", self.ref(), self.prefill_matrices.ptr,
                    self.prefill_matrices.nbytes, stream.handle)
            stream.synchronize()
        finally:
            stream.destroy()
        self.struct.prefill_f16 = self.prefill_matrices.ptr

    def use_prefill_matrices(self, on: bool) -> None:
        """Route the prompt GEMMs through the f16 matrices (on) or the Q8_0
        stacks (off); the matrices stay allocated."""
        if on and self.prefill_matrices is None:
            self.expand_prefill_matrices()
        self.struct.prefill_f16 = self.prefill_matrices.ptr if on else None

    @property
    def nbytes(self) -> int:
        n = sum(b.nbytes for b in self.buffers.values())
        return n + (self.prefill_matrices.nbytes if self.prefill_matrices is not None else 0)

    def ref(self):
        return ctypes.byref(self.struct)

    def free(self) -> None:
        self.struct.prefill_f16 = None
        if self.prefill_matrices is not None:
            self.prefill_matrices.free()
            self.prefill_matrices = None
        for b in self.buffers.values():
            b.free()


def step_mode() -> int:
    """1: each step is one launch (dec_step); 0: one launch per phase."""
    m = ctypes.c_int(0)
    Q._call("qwen3_get_step_mode", ctypes.byref(m))
    return m.value


def set_step_mode(mode: int) -> None:
    Q._call("qwen3_set_step_mode", int(mode))


def set_step_spin_limit(polls: int = 0) -> None:
    """Poll rounds after which a wait of the single-launch step gives up (0 =
    the library default); a small value forces the abort path."""
    Q._call("qwen3_set_step_spin_limit", int(polls))


def step_fallback_count() -> int:
    """Steps (process-wide) that a single launch gave up on and that were re-run
    with the per-phase launches."""
    n = ctypes.c_uint64(0)
    Q._call("qwen3_step_fallback_count", ctypes.byref(n))
    return int(n.value)


def force_step_abort(after: int = 0) -> None:
    """Test hook: the single-launch step `after` launches from now gives up at
    its start (-1 cancels)."""
    Q._call("qwen3_debug_force_step_abort", int(after))


def set_prefill_tiling(gemm_rows: int = 0, attn_split_blocks: int = 0) -> None:
    """Work division of the batched prompt path (0 = by shape): token rows per
    GEMM workgroup (32 or 64) and cache positions per attention split in
    blocks of 32."""
    Q._call("qwen3_set_prefill_tiling", int(gemm_rows), int(attn_split_blocks))


def scratch_bytes() -> int:
    return int(Q.load_library().qwen3_scratch_bytes())


def scratch_offset(name: str) -> int:
    off = int(Q.load_library().qwen3_scratch_offset(name.encode()))
    if off < 0:
        raise KeyError(name)
    return off


class DecodeSession:
    """One sequence: KV cache for max_seq positions, scratch, and the device
    words holding the current token and position.

    step() enqueues one token; capture() records a step in a hipGraph that
    replays with whatever token / position the device words hold, so the
    argmax of one replay is the input of the next (qwen3_full.mlir:1512-1523).
    """

    def __init__(self, model: DeviceWeights, max_seq: int, stream: Q.Stream | None = None):
        if max_seq < 1:
            raise ValueError("max_seq must be >= 1")
        self.model = model
        self.max_seq = int(max_seq)
        self.stream = stream
        cache_bytes = LAYERS * self.max_seq * KV_DIM * 2
        self.k_cache = Q.DeviceBuffer(cache_bytes)
        self.v_cache = Q.DeviceBuffer(cache_bytes)
        self.k_cache.fill(0)
        self.v_cache.fill(0)
        self.scratch = Q.DeviceBuffer(scratch_bytes())
        self.scratch.fill(0)
        self.state = Q.DeviceBuffer(256)  # int32 token at 0, int32 pos at 4
        self.state.fill(0)
        self.logits = Q.DeviceBuffer(VOCAB * 2)
        Q._call("qwen3_scratch_reset", self.scratch.ptr, Q._stream(stream))
        self._graphs: dict[tuple[bool, bool], Q.Graph] = {}

    # device words
    @property
    def token_ptr(self) -> int:
        return self.state.ptr

    @property
    def pos_ptr(self) -> int:
        return self.state.ptr + 4

    def set_state(self, token: int, pos: int) -> None:
        self.state.upload(np.array([token, pos], np.int32))

    def get_state(self) -> tuple[int, int]:
        t, p = self.state.download(np.int32, 2)
        return int(t), int(p)

    def status(self) -> int:
        off = int(Q.load_library().qwen3_scratch_status_offset())
        return int(self.scratch.download(np.uint32, 1, off)[0])

    def check_status(self) -> int:
        """Synchronizes the stream and returns the status word; raises
        Q8GemvError(Q8_ERR_STEP_ABORTED) if a single-launch step gave up."""
        st = ctypes.c_uint32(0)
        Q._call("qwen3_check_status", self.scratch.ptr, ctypes.byref(st), Q._stream(self.stream))
        return int(st.value)

    def reset_scratch(self) -> None:
        """Clears the scratch (status word, sequence number, hand-off words)."""
        Q._call("qwen3_scratch_reset", self.scratch.ptr, Q._stream(self.stream))

    def step(self, advance: bool = True, logits: bool = True) -> None:
        Q._call("qwen3_decode_step", self.model.ref(), self.k_cache.ptr, self.v_cache.ptr,
                self.max_seq, self.token_ptr, self.pos_ptr,
                self.logits.ptr if logits else None, int(bool(advance)), self.scratch.ptr,
                Q._stream(self.stream))

    def step_checked(self, advance: bool = True, logits: bool = True) -> None:
        """One step, synchronized and checked: a single launch that gave up is
        re-run with the per-phase launches (status bit 2), so the outputs are
        valid on return."""
        Q._call("qwen3_decode_step_checked", self.model.ref(), self.k_cache.ptr,
                self.v_cache.ptr, self.max_seq, self.token_ptr, self.pos_ptr,
                self.logits.ptr if logits else None, int(bool(advance)), self.scratch.ptr,
                Q._stream(self.stream))

    def capture(self, advance: bool = True, logits: bool = False) -> Q.Graph:
        """hipGraph of one step (needs a non-null stream)."""
        if self.stream is None:
            raise ValueError("graph capture needs an explicit stream")
        key = (bool(advance), bool(logits))
        if key not in self._graphs:
            self._graphs[key] = Q.Graph(self.stream, lambda: self.step(advance, logits))
        return self._graphs[key]

    def replay(self, advance: bool = True, logits: bool = False) -> None:
        self.capture(advance, logits).launch(self.stream)

    def synchronize(self) -> None:
        if self.stream is not None:
            self.stream.synchronize()
        else:
            Q.synchronize()

    def read_logits(self) -> np.ndarray:
        self.synchronize()
        return self.logits.download(np.float16, VOCAB)

    # prompt ingestion and the generation loop
    def prefill(self, prompt) -> None:
        """Decode steps over the prompt tokens from the current position; the
        token word then holds the argmax after the last prompt token."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32).reshape(-1)
        if prompt.size == 0:
            raise ValueError("empty prompt")
        buf = Q.DeviceBuffer.from_array(prompt)
        try:
            Q._call("qwen3_prefill", self.model.ref(), self.k_cache.ptr, self.v_cache.ptr,
                    self.max_seq, buf.ptr, int(prompt.size), self.token_ptr, self.pos_ptr,
                    self.scratch.ptr, Q._stream(self.stream))
            self.check_status()
        finally:
            buf.free()

    def prefill_batched(self, prompt, chunk_local: bool = False, logits: bool = False) -> None:
        """The prompt's layers as GEMMs over all its tokens (qwen3_prefill_batched,
        the reference's @prefill) from the current position; the token word
        then holds the argmax after the last prompt token and the position has
        moved past the prompt.  chunk_local: attend only to this call's
        tokens, as the reference's @prefill does (the same when starting at
        position 0)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32).reshape(-1)
        if prompt.size == 0:
            raise ValueError("empty prompt")
        nbytes = int(Q.load_library().qwen3_prefill_workspace_bytes(int(prompt.size)))
        if nbytes == 0:
            raise ValueError(f"prompt of {prompt.size} tokens is too long")
        buf = Q.DeviceBuffer.from_array(prompt)
        ws = Q.DeviceBuffer(nbytes)
        try:
            Q._call("qwen3_prefill_batched", self.model.ref(), self.k_cache.ptr, self.v_cache.ptr,
                    self.max_seq, buf.ptr, int(prompt.size), self.token_ptr, self.pos_ptr,
                    self.logits.ptr if logits else None, int(bool(chunk_local)), ws.ptr, nbytes,
                    self.scratch.ptr, Q._stream(self.stream))
            self.synchronize()
        finally:
            ws.free()
            buf.free()

    def prefill_layer(self, layer: int, h_rows, start_pos: int,
                      chunk_local: bool = False) -> dict[str, np.ndarray]:
        """One layer of the batched prompt path on hidden rows h_rows (f16
        [n, 1024]) at positions start_pos..; returns the workspace regions
        (h = the layer's output, and its intermediates) as f16 arrays."""
        h_rows = np.ascontiguousarray(h_rows, dtype=np.float16).reshape(-1, HIDDEN)
        n = h_rows.shape[0]
        lib = Q.load_library()
        nbytes = int(lib.qwen3_prefill_workspace_bytes(n))
        ws = Q.DeviceBuffer(nbytes)
        try:
            ws.upload(h_rows, int(lib.qwen3_prefill_workspace_offset(n, b"h")))
            Q._call("qwen3_prefill_layer", self.model.ref(), int(layer), self.k_cache.ptr,
                    self.v_cache.ptr, self.max_seq, n, int(start_pos), int(bool(chunk_local)),
                    ws.ptr, nbytes, Q._stream(self.stream))
            self.synchronize()
            out = {}
            for name, cols in PREFILL_REGIONS:
                off = int(lib.qwen3_prefill_workspace_offset(n, name.encode()))
                out[name] = ws.download(np.float16, n * cols, off).reshape(n, cols)
            return out
        finally:
            ws.free()

    def generate(self, max_new: int, eos_id: int) -> np.ndarray:
        """@generate's loop from the current token / position: returns the
        produced tokens (int32; the EOS check runs after every 4 tokens)."""
        out = Q.DeviceBuffer(4 * max(int(max_new), 1))
        n = ctypes.c_int32(0)
        try:
            Q._call("qwen3_generate", self.model.ref(), self.k_cache.ptr, self.v_cache.ptr,
                    self.max_seq, self.token_ptr, self.pos_ptr, int(max_new), int(eos_id),
                    out.ptr, ctypes.byref(n), self.scratch.ptr, Q._stream(self.stream))
            return out.download(np.int32, n.value) if n.value else np.zeros(0, np.int32)
        finally:
            out.free()

    # the step in parts
    def embed(self, h_out: Q.DeviceBuffer) -> None:
        Q._call("qwen3_decode_embed", self.model.ref(), self.token_ptr, h_out.ptr,
                Q._stream(self.stream))

    def layer(self, layer: int, h_in: Q.DeviceBuffer, h_out: Q.DeviceBuffer) -> None:
        Q._call("qwen3_decode_layer", self.model.ref(), int(layer), self.k_cache.ptr,
                self.v_cache.ptr, self.max_seq, self.pos_ptr, h_in.ptr, h_out.ptr,
                self.scratch.ptr, Q._stream(self.stream))

    def head(self, h: Q.DeviceBuffer, advance: bool = False, logits: bool = True) -> None:
        Q._call("qwen3_decode_head", self.model.ref(), h.ptr, self.logits.ptr if logits else None,
                self.token_ptr, self.pos_ptr, int(bool(advance)), self.max_seq,
                self.scratch.ptr, Q._stream(self.stream))

    def scratch_f16(self, name: str, count: int) -> np.ndarray:
        self.synchronize()
        return self.scratch.download(np.float16, count, scratch_offset(name))

    def cache_rows(self, layer: int, start: int, stop: int) -> tuple[np.ndarray, np.ndarray]:
        """(K, V) f16 [stop-start, 1024] of one layer's slots."""
        self.synchronize()
        off = (layer * self.max_seq + start) * KV_DIM * 2
        n = (stop - start) * KV_DIM
        k = self.k_cache.download(np.float16, n, off).reshape(-1, KV_DIM)
        v = self.v_cache.download(np.float16, n, off).reshape(-1, KV_DIM)
        return k, v

    def free(self) -> None:
        for g in self._graphs.values():
            g.destroy()
        self._graphs.clear()
        for b in (self.k_cache, self.v_cache, self.scratch, self.state, self.logits):
            b.free()


def run(model: DeviceWeights, prompt, max_gen: int, eos_id: int,
        stream: Q.Stream | None = None, batched: bool = True) -> np.ndarray:
    """The reference's @run (qwen3_full.mlir:2113-2167): a KV cache of
    len(prompt) + max_gen positions, the prompt ingested from position 0 (all
    tokens at once as @prefill does, or as decode steps, @prefill_all, with
    batched=False), its argmax as the first token, then @generate with max_gen
    tokens.  Returns the generated tokens (the first token itself is not among
    them, as there)."""
    prompt = np.asarray(prompt, dtype=np.int32).reshape(-1)
    sess = DecodeSession(model, int(prompt.size) + int(max_gen), stream)
    try:
        sess.set_state(0, 0)
        if batched:
            sess.prefill_batched(prompt)
        else:
            sess.prefill(prompt)
        return sess.generate(max_gen, eos_id)
    finally:
        sess.free()
