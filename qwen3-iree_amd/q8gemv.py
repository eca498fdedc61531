"""ctypes binding of libq8gemv (include/q8gemv.h): the host-side mirror of the
reference's six substituted decode dispatches.

The reference swaps IREE's generated executables `decode_dispatch_{3,4,12,18,
20,24}` for hand-written kernels at compile time (compile.sh:35-43) and runs
them through the IREE runtime (scripts/benchmark.py:34-49).  Here the same six
operators are plain C entry points over device pointers; this module exposes
them to Python with ctypes, plus the small device runtime (allocation, copies,
streams, events, graphs) that the IREE HAL provided there.  No PyTorch: device
memory is owned by DeviceBuffer objects allocated through the library.

Every call raises Q8GemvError with the library's status code and message when
the library reports a failure; nothing falls back to a CPU path.

At interpreter exit (atexit) the module releases what is still alive in an
order the HIP runtime accepts: it waits for the device, destroys graph execs,
events and streams, frees device buffers, then unloads the code objects
(q8gemv_shutdown) -- so no HIP object outlives the runtime's own teardown.
"""
from __future__ import annotations

import atexit
import ctypes
import weakref
from dataclasses import dataclass
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "lib" / "libq8gemv.so"
CODE_OBJECT_PATH = PKG / "lib" / "q8gemv_gfx950.hsaco"

# status codes (include/q8gemv.h)
Q8_OK = 0
Q8_ERR_NOT_INITIALIZED = 1
Q8_ERR_INVALID_KIND = 2
Q8_ERR_NULL_POINTER = 3
Q8_ERR_LAYER_RANGE = 4
Q8_ERR_MISALIGNED = 5
Q8_ERR_BAD_SHAPE = 6
Q8_ERR_CODE_OBJECT = 7
Q8_ERR_HIP = 8
Q8_ERR_BAD_ARGUMENT = 9
Q8_ERR_STEP_ABORTED = 10

NUM_LAYERS = 28
HIDDEN = 1024
VOCAB_ROWS = 151936
BLOCK_ELEMS = 32
BLOCK_BYTES = 34


@dataclass(frozen=True)
class Dispatch:
    """One substituted reference dispatch (kernels/cuda/dispatch_N.mlir)."""
    kind: int            # enum q8_kind, -1 for the vocab dispatch
    name: str            # role in the layer (qwen3_full.mlir:751-864)
    ordinal: int         # decode_dispatch_<ordinal>
    n: int               # output rows
    k: int               # reduction length
    weight: str          # "q8_0" or "f16"

    @property
    def export(self) -> str:
        return f"decode_dispatch_{self.ordinal}_matmul_{self.n}x1x{self.k}_f16"

    @property
    def row_bytes(self) -> int:
        return self.k // BLOCK_ELEMS * BLOCK_BYTES if self.weight == "q8_0" else 2 * self.k

    @property
    def bytes_per_layer(self) -> int:
        return self.n * self.row_bytes


ATTN_Q = Dispatch(0, "attn_q", 3, 2048, 1024, "q8_0")
ATTN_KV = Dispatch(1, "attn_kv", 4, 1024, 1024, "q8_0")
ATTN_O = Dispatch(2, "attn_o", 12, 1024, 2048, "q8_0")
GATE_UP = Dispatch(3, "gate_up", 18, 6144, 1024, "q8_0")
FFN_DN = Dispatch(4, "ffn_dn", 20, 1024, 3072, "q8_0")
VOCAB = Dispatch(-1, "vocab", 24, VOCAB_ROWS, 1024, "f16")

Q8_KINDS = (ATTN_Q, ATTN_KV, ATTN_O, GATE_UP, FFN_DN)
DISPATCHES = {d.ordinal: d for d in (*Q8_KINDS, VOCAB)}
# Per-layer GEMV order of the decode step: q, k, v, o, gate_up, down
# (qwen3_full.mlir:625, 630, 635, 739, 820, 852).
LAYER_ORDER = (ATTN_Q, ATTN_KV, ATTN_KV, ATTN_O, GATE_UP, FFN_DN)


class Q8GemvError(RuntimeError):
    def __init__(self, code: int, message: str, func: str = ""):
        super().__init__(f"{func}: status {code}: {message}" if func else f"status {code}: {message}")
        self.code = code
        self.message = message


_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t

# name -> argtypes (restype is int for all but the listed exceptions)
_SIGNATURES = {
    "q8gemv_init": [ctypes.c_char_p],
    "q8gemv_shutdown": [],
    "q8gemv_last_error": [],
    "q8gemv_kind_shape": [_I, _P, _P, _P],
    "q8gemv": [_I, _P, _I64, _P, _P, _P],
    "q8gemv_rows": [_P, _I64, _I64, _P, _P, _P],
    "decode_dispatch_3_matmul_2048x1x1024_f16": [_P, _I64, _P, _P, _P],
    "decode_dispatch_4_matmul_1024x1x1024_f16": [_P, _I64, _P, _P, _P],
    "decode_dispatch_12_matmul_1024x1x2048_f16": [_P, _I64, _P, _P, _P],
    "decode_dispatch_18_matmul_6144x1x1024_f16": [_P, _I64, _P, _P, _P],
    "decode_dispatch_20_matmul_1024x1x3072_f16": [_P, _I64, _P, _P, _P],
    "vocab_argmax_workspace_bytes": [],
    "vocab_argmax_workspace_reset": [_P, _P],
    "vocab_gemv_argmax": [_P, _P, _P, _P, _P, _P],
    "decode_dispatch_24_matmul_151936x1x1024_f16": [_P, _P, _P, _P, _P, _P],
    "f16_gemv_argmax_rows": [_P, _I64, _P, _P, _P, _P, _P],
    "f16_gemv_argmax_rows_noalloc": [_P, _I64, _P, _P, _P, _P],
    "f16_argmax": [_P, _I64, _P, _P, _P],
    "q8gemv_qkv": [_P, _P, _P, _I64, _P, _P, _P, _P, _P],
    "q8gemv_hal_dispatch": [_I, _P, _P, _P, _P, _I, _P],
    "q8gemv_hal_dispatch_grid": [_I, _P, _P, _P, _P, _I, ctypes.c_uint32, ctypes.c_uint32, _P],
    "q8gemv_desc_for_kind": [_I, _P, _I64, _P, _P, _P],
    "q8gemv_batch_table_bytes": [_I],
    "q8gemv_batch_encode": [_P, _I, _P, _SZ, _P],
    "q8gemv_batch": [_P, _I, ctypes.c_int32, _P],
    "q8gemv_batch_set_workgroups": [_I],
    "vocab_set_workgroups": [_I],
    "vocab_get_workgroups": [_P],
    "q8rt_device_count": [_P],
    "q8rt_set_device": [_I],
    "q8rt_device_info": [_P, _I, _P, _P],
    "q8rt_malloc": [_P, _SZ],
    "q8rt_free": [_P],
    "q8rt_memcpy_htod": [_P, _P, _SZ],
    "q8rt_memcpy_dtoh": [_P, _P, _SZ],
    "q8rt_memcpy_dtod": [_P, _P, _SZ],
    "q8rt_memset": [_P, _I, _SZ],
    "q8rt_device_synchronize": [],
    "q8rt_stream_create": [_P],
    "q8rt_stream_destroy": [_P],
    "q8rt_stream_synchronize": [_P],
    "q8rt_event_create": [_P],
    "q8rt_event_destroy": [_P],
    "q8rt_event_record": [_P, _P],
    "q8rt_event_synchronize": [_P],
    "q8rt_event_elapsed_ms": [_P, _P, _P],
    "q8rt_graph_begin_capture": [_P],
    "q8rt_graph_end_capture": [_P, _P],
    "q8rt_graph_launch": [_P, _P],
    "q8rt_graph_destroy": [_P],
    "q8rt_time_next_launch": [_P, _P],
    "q8rt_stream_copy": [_P, _P, _SZ, _P],
    "q8rt_stream_read": [_P, _SZ, _P],
    "q8rt_launch_cost": [_I, _I, _I, _SZ, _I, _P],
    "q8rt_handoff_latency": [_I, _I, _I, _I, _I, _P, _P],
    "q8rt_memory_latency": [_I, _P, _P],
    # include/qwen3_decode.h
    "qwen3_scratch_bytes": [],
    "qwen3_scratch_reset": [_P, _P],
    "qwen3_scratch_status_offset": [],
    "qwen3_scratch_offset": [ctypes.c_char_p],
    "qwen3_decode_step": [_P, _P, _P, _I64, _P, _P, _P, _I, _P, _P],
    "qwen3_decode_step_checked": [_P, _P, _P, _I64, _P, _P, _P, _I, _P, _P],
    "qwen3_step_fallback_count": [_P],
    "qwen3_debug_force_step_abort": [_I64],
    "qwen3_decode_embed": [_P, _P, _P, _P],
    "qwen3_decode_layer": [_P, _I, _P, _P, _I64, _P, _P, _P, _P, _P],
    "qwen3_decode_head": [_P, _P, _P, _P, _P, _I, _I64, _P, _P],
    "qwen3_prefill": [_P, _P, _P, _I64, _P, ctypes.c_int32, _P, _P, _P, _P],
    "qwen3_generate": [_P, _P, _P, _I64, _P, _P, ctypes.c_int32, ctypes.c_int32, _P, _P, _P, _P],
    "qwen3_prefill_workspace_bytes": [ctypes.c_int32],
    "qwen3_prefill_matrices_bytes": [],
    "qwen3_prefill_matrices_expand": [_P, _P, _SZ, _P],
    "qwen3_prefill_batched": [_P, _P, _P, _I64, _P, ctypes.c_int32, _P, _P, _P, _I, _P, _SZ, _P,
                              _P],
    "qwen3_prefill_layer": [_P, _I, _P, _P, _I64, ctypes.c_int32, ctypes.c_int32, _I, _P, _SZ, _P],
    "qwen3_prefill_workspace_offset": [ctypes.c_int32, ctypes.c_char_p],
    "qwen3_set_step_mode": [_I],
    "qwen3_set_step_spin_limit": [ctypes.c_uint32],
    "qwen3_check_status": [_P, _P, _P],
    "qwen3_set_prefill_tiling": [_I, _I],
    "qwen3_get_step_mode": [_P],
}
_RESTYPES = {
    "q8gemv_shutdown": None,
    "q8gemv_last_error": ctypes.c_char_p,
    "vocab_argmax_workspace_bytes": _SZ,
    "q8gemv_batch_table_bytes": _SZ,
    "qwen3_scratch_bytes": _SZ,
    "qwen3_scratch_status_offset": _SZ,
    "qwen3_scratch_offset": _I64,
    "qwen3_prefill_workspace_bytes": _SZ,
    "qwen3_prefill_matrices_bytes": _SZ,
    "qwen3_prefill_workspace_offset": _I64,
}

_lib: ctypes.CDLL | None = None
# Device objects still alive (DeviceBuffer, Stream, Event, Graph), released in
# order by teardown() at exit.
_live: "weakref.WeakSet" = weakref.WeakSet()


def load_library(path: str | Path | None = None) -> ctypes.CDLL:
    """dlopen libq8gemv.so (no GPU work happens here)."""
    global _lib
    if _lib is None:
        p = Path(path) if path else LIB_PATH
        if not p.exists():
            raise Q8GemvError(Q8_ERR_CODE_OBJECT, f"{p} is not built (run qwen3-iree_amd/build.py)")
        L = ctypes.CDLL(str(p))
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, _I)
        _lib = L
    return _lib


def last_error() -> str:
    msg = load_library().q8gemv_last_error()
    return msg.decode() if msg else ""


def check(rc: int, func: str = "") -> None:
    if rc != Q8_OK:
        raise Q8GemvError(rc, last_error(), func)


def _call(name: str, *args) -> None:
    check(getattr(load_library(), name)(*args), name)


def init(code_object: str | Path | None = None) -> None:
    """Load the gfx950 code object on the current device (idempotent)."""
    path = str(code_object or CODE_OBJECT_PATH).encode()
    _call("q8gemv_init", path)


def shutdown() -> None:
    load_library().q8gemv_shutdown()


def teardown() -> None:
    """Release every live device object, then unload the code objects.

    Order: device synchronize; graph execs; events; streams; device buffers;
    q8gemv_shutdown.  Errors are ignored (this runs at exit).  Registered with
    atexit; safe to call more than once."""
    if _lib is None:
        return
    try:
        _lib.q8rt_device_synchronize()
    except Exception:
        pass
    for kind in (Graph, Event, Stream, DeviceBuffer):
        for obj in [o for o in list(_live) if isinstance(o, kind)]:
            try:
                obj._release()
            except Exception:
                pass
    try:
        _lib.q8gemv_shutdown()
    except Exception:
        pass


atexit.register(teardown)


def device_count() -> int:
    n = ctypes.c_int(0)
    _call("q8rt_device_count", ctypes.byref(n))
    return n.value


def device_info() -> dict:
    name = ctypes.create_string_buffer(256)
    cus = ctypes.c_int(0)
    mem = ctypes.c_int64(0)
    _call("q8rt_device_info", name, 256, ctypes.byref(cus), ctypes.byref(mem))
    return {"name": name.value.decode(), "compute_units": cus.value, "total_mem": mem.value}


def synchronize() -> None:
    _call("q8rt_device_synchronize")


# ---------------------------------------------------------------- memory ----

class DeviceBuffer:
    """A device allocation owned by Python (hipMalloc through the library)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p(0)
        _call("q8rt_malloc", ctypes.byref(p), max(self.nbytes, 1))
        self.ptr = p.value
        _live.add(self)

    @classmethod
    def from_array(cls, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr)
        return buf

    def upload(self, arr: np.ndarray, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        if offset < 0 or offset + arr.nbytes > self.nbytes:
            raise ValueError("upload out of range")
        _call("q8rt_memcpy_htod", self.ptr + offset, arr.ctypes.data, arr.nbytes)

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype)
        if offset < 0 or offset + out.nbytes > self.nbytes:
            raise ValueError("download out of range")
        _call("q8rt_memcpy_dtoh", out.ctypes.data, self.ptr + offset, out.nbytes)
        return out

    def fill(self, value: int = 0) -> None:
        _call("q8rt_memset", self.ptr, int(value), self.nbytes)

    def free(self) -> None:
        if self.ptr:
            _call("q8rt_free", self.ptr)
            self.ptr = None

    def _release(self) -> None:
        if self.ptr and _lib is not None:
            _lib.q8rt_free(self.ptr)
        self.ptr = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.free()

    def __del__(self):
        try:
            if getattr(self, "ptr", None) and _lib is not None:
                _lib.q8rt_free(self.ptr)
        except Exception:
            pass


class Stream:
    def __init__(self):
        p = ctypes.c_void_p(0)
        _call("q8rt_stream_create", ctypes.byref(p))
        self.handle = p.value
        _live.add(self)

    def synchronize(self) -> None:
        _call("q8rt_stream_synchronize", self.handle)

    def destroy(self) -> None:
        if self.handle:
            _call("q8rt_stream_destroy", self.handle)
            self.handle = None

    def _release(self) -> None:
        if self.handle and _lib is not None:
            _lib.q8rt_stream_destroy(self.handle)
        self.handle = None


class Event:
    def __init__(self):
        p = ctypes.c_void_p(0)
        _call("q8rt_event_create", ctypes.byref(p))
        self.handle = p.value
        _live.add(self)

    def record(self, stream: Stream | None = None) -> None:
        _call("q8rt_event_record", self.handle, stream.handle if stream else None)

    def synchronize(self) -> None:
        _call("q8rt_event_synchronize", self.handle)

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float(0.0)
        _call("q8rt_event_elapsed_ms", ctypes.byref(ms), self.handle, end.handle)
        return float(ms.value)

    def destroy(self) -> None:
        if self.handle:
            _call("q8rt_event_destroy", self.handle)
            self.handle = None

    def _release(self) -> None:
        if self.handle and _lib is not None:
            _lib.q8rt_event_destroy(self.handle)
        self.handle = None


class Graph:
    """A captured hipGraph of library launches on one stream."""

    def __init__(self, stream: Stream, record_fn):
        _call("q8rt_graph_begin_capture", stream.handle)
        try:
            record_fn()
        finally:
            p = ctypes.c_void_p(0)
            _call("q8rt_graph_end_capture", stream.handle, ctypes.byref(p))
        self.exec = p.value
        _live.add(self)

    def launch(self, stream: Stream) -> None:
        _call("q8rt_graph_launch", self.exec, stream.handle)

    def destroy(self) -> None:
        if self.exec:
            _call("q8rt_graph_destroy", self.exec)
            self.exec = None

    def _release(self) -> None:
        if self.exec and _lib is not None:
            _lib.q8rt_graph_destroy(self.exec)
        self.exec = None


def stream_copy(dst, src, nbytes: int, stream=None) -> None:
    _call("q8rt_stream_copy", _ptr(dst), _ptr(src), int(nbytes), _stream(stream))


def stream_read(src, nbytes: int, stream=None) -> None:
    _call("q8rt_stream_read", _ptr(src), int(nbytes), _stream(stream))


def time_next_launch(start: Event, stop: Event) -> None:
    _call("q8rt_time_next_launch", start.handle, stop.handle)


def launch_cost(workgroups: int, threads: int, lds_bytes: int, launches: int = 2000,
                cooperative: bool = False) -> float:
    """Mean us per back-to-back launch of an empty kernel of that shape."""
    us = ctypes.c_float(0.0)
    _call("q8rt_launch_cost", int(bool(cooperative)), int(workgroups), int(threads),
          int(lds_bytes), int(launches), ctypes.byref(us))
    return float(us.value)


def handoff_latency(producers: int, consumers: int, n_words: int, replicas: int = 1,
                    rounds: int = 50) -> tuple[np.ndarray, int]:
    """Tagged-word hand-off latencies in us, [rounds, consumers] (NaN where a
    bounded wait gave up), and the count of those."""
    out = np.zeros(rounds * consumers, np.float32)
    failed = ctypes.c_int(0)
    _call("q8rt_handoff_latency", int(producers), int(consumers), int(n_words), int(replicas),
          int(rounds), out.ctypes.data, ctypes.byref(failed))
    return out.reshape(rounds, consumers), int(failed.value)


def memory_latency(hops: int = 4096) -> dict:
    """ns per dependent load from HBM, from the memory-side cache (MALL) and
    from L2, and the XCDs that chased (q8rt_memory_latency)."""
    ns = np.zeros(3, np.float32)
    xcds = np.zeros(2, np.int32)
    _call("q8rt_memory_latency", int(hops), ns.ctypes.data, xcds.ctypes.data)
    return {"hbm_ns": float(ns[0]), "mall_ns": float(ns[1]), "l2_ns": float(ns[2]),
            "xcds": [int(xcds[0]), int(xcds[1])], "hops": int(hops)}


# ------------------------------------------------------------- operators ----

def _ptr(x) -> int | None:
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    return int(x)


def _stream(s) -> int | None:
    if s is None:
        return None
    return s.handle if isinstance(s, Stream) else int(s)


def kind_shape(kind: int) -> tuple[int, int, int]:
    n, k, bpl = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    _call("q8gemv_kind_shape", kind, ctypes.byref(n), ctypes.byref(k), ctypes.byref(bpl))
    return n.value, k.value, bpl.value


def q8gemv(kind: int, w_stacked, layer: int, x, y, stream=None) -> None:
    """y = W[layer] . x for one Q8_0 kind (decode_dispatch_{3,4,12,18,20})."""
    _call("q8gemv", int(kind), _ptr(w_stacked), int(layer), _ptr(x), _ptr(y), _stream(stream))


def q8gemv_qkv(wq_stacked, wk_stacked, wv_stacked, layer: int, x, yq, yk, yv, stream=None) -> None:
    """q, k and v of one layer in one launch (all three read x)."""
    _call("q8gemv_qkv", _ptr(wq_stacked), _ptr(wk_stacked), _ptr(wv_stacked), int(layer), _ptr(x),
          _ptr(yq), _ptr(yk), _ptr(yv), _stream(stream))


def q8gemv_rows(w_layer, n_rows: int, k: int, x, y, stream=None) -> None:
    _call("q8gemv_rows", _ptr(w_layer), int(n_rows), int(k), _ptr(x), _ptr(y), _stream(stream))


def decode_dispatch(ordinal: int, *args, stream=None) -> None:
    """Call a reference dispatch by its ordinal under its reference export name.

    Q8 ordinals (3, 4, 12, 18, 20): args = (w_stacked, layer, x, y).
    Vocab ordinal 24: args = (w_f16, x, logits_or_None, token, workspace).
    """
    d = DISPATCHES[ordinal]
    if d.weight == "q8_0":
        w, layer, x, y = args
        _call(d.export, _ptr(w), int(layer), _ptr(x), _ptr(y), _stream(stream))
    else:
        w, x, logits, token, ws = args
        _call(d.export, _ptr(w), _ptr(x), _ptr(logits), _ptr(token), _ptr(ws), _stream(stream))


def hal_dispatch(ordinal: int, binding0, binding1, binding2, constants, stream=None,
                 workgroups: int = 0, workgroup_size: int = 0) -> None:
    """Launch a reference executable through its IREE HAL binding ABI, with
    this build's stub shape (0, 0) or an explicit one (e.g. the reference
    stubs' 256-thread workgroups)."""
    c = (ctypes.c_uint32 * max(1, len(constants)))(*[int(v) & 0xffffffff for v in constants])
    _call("q8gemv_hal_dispatch_grid", int(ordinal), _ptr(binding0), _ptr(binding1), _ptr(binding2),
          c, len(constants), int(workgroups), int(workgroup_size), _stream(stream))


def vocab_workspace_bytes() -> int:
    return int(load_library().vocab_argmax_workspace_bytes())


def vocab_workspace_reset(workspace, stream=None) -> None:
    _call("vocab_argmax_workspace_reset", _ptr(workspace), _stream(stream))


def vocab_gemv_argmax(w, x, logits, token, workspace, stream=None) -> None:
    _call("vocab_gemv_argmax", _ptr(w), _ptr(x), _ptr(logits), _ptr(token), _ptr(workspace),
          _stream(stream))


def f16_gemv_argmax_rows(w, n_rows: int, x, logits, token, workspace, stream=None) -> None:
    _call("f16_gemv_argmax_rows", _ptr(w), int(n_rows), _ptr(x), _ptr(logits), _ptr(token),
          _ptr(workspace), _stream(stream))


def f16_argmax(values, n: int, token, workspace, stream=None) -> None:
    """Argmax of n f16 values already in device memory (the tiled argmax as
    its own pass; same workspace rule as vocab_gemv_argmax)."""
    _call("f16_argmax", _ptr(values), int(n), _ptr(token), _ptr(workspace), _stream(stream))


def f16_gemv_argmax_rows_noalloc(w, n_rows: int, x, logits, token, stream=None) -> None:
    """f16_gemv_argmax_rows with the argmax key in the library's own device
    scratch (no workspace, nothing allocated)."""
    _call("f16_gemv_argmax_rows_noalloc", _ptr(w), int(n_rows), _ptr(x), _ptr(logits),
          _ptr(token), _stream(stream))


def set_batch_workgroups(n: int) -> None:
    """Cap on workgroups of a batched Q8_0 launch (0 = default)."""
    _call("q8gemv_batch_set_workgroups", int(n))


class Q8Desc(ctypes.Structure):
    """struct q8gemv_desc (include/q8gemv.h)."""
    _fields_ = [("w_layer", ctypes.c_void_p), ("x_f16", ctypes.c_void_p),
                ("y_f16", ctypes.c_void_p), ("n_rows", ctypes.c_int64), ("k", ctypes.c_int64)]


def desc(w_layer, n_rows: int, k: int, x, y) -> Q8Desc:
    return Q8Desc(_ptr(w_layer), _ptr(x), _ptr(y), int(n_rows), int(k))


def desc_for_kind(kind: int, w_stacked, layer: int, x, y) -> Q8Desc:
    d = Q8Desc()
    _call("q8gemv_desc_for_kind", int(kind), _ptr(w_stacked), int(layer), _ptr(x), _ptr(y),
          ctypes.byref(d))
    return d


class Q8Batch:
    """An encoded list of independent Q8_0 GEMVs resident on the device; each
    launch() runs all of them in one kernel launch."""

    def __init__(self, descs: list[Q8Desc]):
        n = len(descs)
        arr = (Q8Desc * n)(*descs)
        nbytes = int(load_library().q8gemv_batch_table_bytes(n))
        if nbytes == 0:
            raise Q8GemvError(Q8_ERR_BAD_ARGUMENT, f"bad batch size {n}")
        host = (ctypes.c_uint8 * nbytes)()
        units = ctypes.c_int32(0)
        _call("q8gemv_batch_encode", arr, n, host, nbytes, ctypes.byref(units))
        self.count = n
        self.total_units = units.value
        self.table = DeviceBuffer(nbytes)
        self.table.upload(np.frombuffer(host, dtype=np.uint8))

    def launch(self, stream=None) -> None:
        _call("q8gemv_batch", self.table.ptr, self.count, self.total_units, _stream(stream))

    def free(self) -> None:
        self.table.free()


def set_vocab_workgroups(n: int) -> None:
    _call("vocab_set_workgroups", int(n))


def get_vocab_workgroups() -> int:
    q = ctypes.c_int(0)
    _call("vocab_get_workgroups", ctypes.byref(q))
    return q.value
