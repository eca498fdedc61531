"""GGUF reading and writing, and Qwen3-0.6B weight ingestion without IREE.

The reference converts a llama.cpp GGUF checkpoint offline into an IREE
parameter archive (tools/create_q8_irpa.py:28-100 reads the GGUF,
:143-224 stacks the tensors; tools/convert_gguf_to_irpa.py:48-150 is the f16
variant).  This module reads the same GGUF (v2/v3) directly, memory-mapped,
and produces the device layout the decode kernels take (decode.HostWeights):

  token_embd.weight        -> f16 [151936, 1024] (Q8_0 / f32 / bf16 converted)
  output_norm.weight       -> f16 [1024]
  output.weight            -> f16 [151936, 1024], the vocab-major layout of
                              the model's output_T.weight (qwen3_full.mlir:76-79);
                              a file without it has tied embeddings and
                              token_embd is used
  blk.L.{attn_norm, ffn_norm, attn_q_norm, attn_k_norm}.weight
                           -> f16 stacks [28, n]
  blk.L.{attn_q, attn_k, attn_v, attn_output, ffn_down}.weight
                           -> Q8_0 stacks [28, BPL], GGUF-native [N, K] rows
  blk.L.ffn_gate / ffn_up  -> one [28, BPL] stack, gate rows then up rows

Q8_0 tensors are copied byte for byte; layer matrices stored as f16 / f32 /
bf16 are quantized with the reference's quantizer (weights.quantize_q8_0).

File layout (GGUF v3, little endian): magic "GGUF", u32 version, u64 tensor
count, u64 metadata count; metadata entries (string key, u32 value type,
value); tensor infos (string name, u32 n_dims, u64 dims[n_dims] fastest
first, u32 ggml type, u64 offset into the data section); padding to the
alignment (metadata "general.alignment", default 32); the data section.
Strings are u64 length + UTF-8 bytes; arrays are u32 element type + u64
count + elements.
"""
from __future__ import annotations

import mmap
import os
import struct
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from . import weights as Wt

GGUF_MAGIC = 0x46554747  # b"GGUF" little endian
DEFAULT_ALIGNMENT = 32

# ggml tensor types this reader converts: name, block elements, block bytes
GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16 = 0, 1, 8, 30
GGML_TYPES = {GGML_F32: ("f32", 1, 4), GGML_F16: ("f16", 1, 2), GGML_Q8_0: ("q8_0", 32, 34),
              GGML_BF16: ("bf16", 1, 2)}

# metadata value types
(T_UINT8, T_INT8, T_UINT16, T_INT16, T_UINT32, T_INT32, T_FLOAT32, T_BOOL, T_STRING, T_ARRAY,
 T_UINT64, T_INT64, T_FLOAT64) = range(13)
_SCALAR = {T_UINT8: "<B", T_INT8: "<b", T_UINT16: "<H", T_INT16: "<h", T_UINT32: "<I",
           T_INT32: "<i", T_FLOAT32: "<f", T_BOOL: "<?", T_UINT64: "<Q", T_INT64: "<q",
           T_FLOAT64: "<d"}
_NUMPY = {T_UINT8: np.uint8, T_INT8: np.int8, T_UINT16: np.uint16, T_INT16: np.int16,
          T_UINT32: np.uint32, T_INT32: np.int32, T_FLOAT32: np.float32, T_BOOL: np.bool_,
          T_UINT64: np.uint64, T_INT64: np.int64, T_FLOAT64: np.float64}


class GGUFError(ValueError):
    pass


@dataclass(frozen=True)
class GGUFTensor:
    name: str
    shape: tuple          # numpy (row-major) order: the GGUF dims reversed
    ggml_type: int
    offset: int           # absolute byte offset in the file
    nbytes: int
    _buf: object          # the file's memory map

    @property
    def type_name(self) -> str:
        return GGML_TYPES[self.ggml_type][0] if self.ggml_type in GGML_TYPES else f"ggml{self.ggml_type}"

    @property
    def n_elements(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1

    def raw(self) -> np.ndarray:
        """The tensor's bytes (a read-only view of the mapping)."""
        return np.frombuffer(self._buf, dtype=np.uint8, count=self.nbytes, offset=self.offset)

    def to_f32(self) -> np.ndarray:
        raw = self.raw()
        if self.ggml_type == GGML_F32:
            a = raw.view(np.float32)
        elif self.ggml_type == GGML_F16:
            a = raw.view(np.float16).astype(np.float32)
        elif self.ggml_type == GGML_BF16:
            a = (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        elif self.ggml_type == GGML_Q8_0:
            a = Wt.dequant_q8_0(raw)  # create_q8_irpa.py:121-129
        else:
            raise GGUFError(f"{self.name}: tensor type {self.type_name} is not supported")
        return a.reshape(self.shape)

    def to_f16(self) -> np.ndarray:
        if self.ggml_type == GGML_F16:
            return self.raw().view(np.float16).reshape(self.shape)
        return self.to_f32().astype(np.float16)


class GGUFReader:
    """Parses a GGUF file's header and maps its data section (nothing is
    copied until a tensor is converted)."""

    def __init__(self, path: str | Path):
        self.path = Path(path)
        self._file = open(self.path, "rb")
        size = self.path.stat().st_size
        if size < 24:
            raise GGUFError(f"{self.path}: {size} bytes is too short for a GGUF header")
        self._map = mmap.mmap(self._file.fileno(), 0, access=mmap.ACCESS_READ)
        self._size = size
        try:
            self._parse()
        except struct.error as e:
            raise GGUFError(f"{self.path}: truncated header ({e})") from None

    # -- parsing helpers
    def _take(self, fmt: str):
        v = struct.unpack_from(fmt, self._map, self._off)
        self._off += struct.calcsize(fmt)
        return v[0]

    def _string(self) -> str:
        n = self._take("<Q")
        if self._off + n > self._size:
            raise GGUFError(f"{self.path}: string runs past the end of the file")
        s = bytes(self._map[self._off:self._off + n]).decode("utf-8")
        self._off += n
        return s

    def _value(self, vtype: int):
        if vtype in _SCALAR:
            return self._take(_SCALAR[vtype])
        if vtype == T_STRING:
            return self._string()
        if vtype == T_ARRAY:
            etype = self._take("<I")
            count = self._take("<Q")
            if etype in _NUMPY:
                dt = np.dtype(_NUMPY[etype]).newbyteorder("<")
                nbytes = count * dt.itemsize
                if self._off + nbytes > self._size:
                    raise GGUFError(f"{self.path}: array runs past the end of the file")
                a = np.frombuffer(self._map, dtype=dt, count=count, offset=self._off).copy()
                self._off += nbytes
                return a
            return [self._value(etype) for _ in range(count)]
        raise GGUFError(f"{self.path}: unknown metadata value type {vtype}")

    def _parse(self) -> None:
        self._off = 0
        magic = self._take("<I")
        if magic != GGUF_MAGIC:
            raise GGUFError(f"{self.path}: not a GGUF file (magic 0x{magic:08x})")
        self.version = self._take("<I")
        if self.version not in (2, 3):
            raise GGUFError(f"{self.path}: GGUF version {self.version} is not supported (2, 3)")
        n_tensors = self._take("<Q")
        n_kv = self._take("<Q")
        self.metadata: dict = {}
        self.metadata_types: dict = {}
        for _ in range(n_kv):
            key = self._string()
            vtype = self._take("<I")
            self.metadata[key] = self._value(vtype)
            self.metadata_types[key] = vtype
        self.alignment = int(self.metadata.get("general.alignment", DEFAULT_ALIGNMENT))
        if self.alignment <= 0 or self.alignment & (self.alignment - 1):
            raise GGUFError(f"{self.path}: alignment {self.alignment} is not a power of two")
        infos = []
        for _ in range(n_tensors):
            name = self._string()
            n_dims = self._take("<I")
            dims = [self._take("<Q") for _ in range(n_dims)]
            gtype = self._take("<I")
            rel = self._take("<Q")
            infos.append((name, tuple(reversed(dims)), gtype, rel))
        a = self.alignment
        self.data_offset = (self._off + a - 1) // a * a
        self.tensors: dict[str, GGUFTensor] = {}
        for name, shape, gtype, rel in infos:
            n = int(np.prod(shape, dtype=np.int64)) if shape else 1
            if gtype in GGML_TYPES:
                _, blk, bsz = GGML_TYPES[gtype]
                if n % blk:
                    raise GGUFError(f"{name}: {n} elements is not a multiple of the block size {blk}")
                nbytes = n // blk * bsz
            else:
                nbytes = 0  # listed, but not convertible
            off = self.data_offset + rel
            if off + nbytes > self._size:
                raise GGUFError(f"{self.path}: tensor {name} runs past the end of the file")
            if name in self.tensors:
                raise GGUFError(f"{self.path}: duplicate tensor {name}")
            self.tensors[name] = GGUFTensor(name, shape, gtype, off, nbytes, self._map)

    def read_raw(self, t: GGUFTensor, out: np.ndarray) -> np.ndarray:
        """Read the tensor's bytes straight into `out` (any contiguous array of
        t.nbytes bytes) with positioned reads: no page-fault-per-page copy
        out of the mapping."""
        dst = memoryview(np.ascontiguousarray(out).reshape(-1).view(np.uint8))
        if dst.nbytes != t.nbytes:
            raise GGUFError(f"{t.name}: {t.nbytes} bytes do not fit a {dst.nbytes}-byte buffer")
        fd, done = self._file.fileno(), 0
        while done < t.nbytes:
            n = os.preadv(fd, [dst[done:]], t.offset + done)
            if n <= 0:
                raise GGUFError(f"{self.path}: short read of {t.name}")
            done += n
        return out

    def tensor(self, name: str) -> GGUFTensor:
        try:
            return self.tensors[name]
        except KeyError:
            raise GGUFError(f"{self.path}: no tensor {name}") from None

    def close(self) -> None:
        self.tensors = {}
        try:
            self._map.close()
        except BufferError:
            pass  # views handed out keep the mapping alive; it closes with them
        self._file.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def _encode_value(vtype: int, value) -> bytes:
    if vtype in _SCALAR:
        return struct.pack(_SCALAR[vtype], value)
    if vtype == T_STRING:
        b = value.encode("utf-8")
        return struct.pack("<Q", len(b)) + b
    if vtype == T_ARRAY:
        etype, items = value
        if isinstance(items, np.ndarray) and etype in _NUMPY:
            arr = np.ascontiguousarray(items, dtype=np.dtype(_NUMPY[etype]).newbyteorder("<"))
            return struct.pack("<IQ", etype, arr.size) + arr.tobytes()
        return struct.pack("<IQ", etype, len(items)) + b"".join(_encode_value(etype, v) for v in items)
    raise GGUFError(f"unknown metadata value type {vtype}")


def write_gguf(path: str | Path, metadata: list, tensors: list,
               alignment: int = DEFAULT_ALIGNMENT) -> None:
    """Write a GGUF v3 file.

    metadata: [(key, value_type, value)], arrays as (T_ARRAY, (elem_type, items)).
    tensors: [(name, ggml_type, shape (row-major), data)] with data a numpy
    array whose bytes are the tensor's (Q8_0: the raw block bytes).
    """
    meta = list(metadata)
    if alignment != DEFAULT_ALIGNMENT and not any(k == "general.alignment" for k, _, _ in meta):
        meta.append(("general.alignment", T_UINT32, alignment))
    head = bytearray(struct.pack("<IIQQ", GGUF_MAGIC, 3, len(tensors), len(meta)))
    for key, vtype, value in meta:
        head += _encode_value(T_STRING, key) + struct.pack("<I", vtype) + _encode_value(vtype, value)
    rel = 0
    blobs = []
    for name, gtype, shape, data in tensors:
        raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        head += _encode_value(T_STRING, name)
        head += struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in reversed(shape))
        head += struct.pack("<IQ", gtype, rel)
        blobs.append((rel, raw))
        rel = (rel + raw.size + alignment - 1) // alignment * alignment
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * pad)
        pos = 0
        for r, raw in blobs:
            f.write(b"\0" * (r - pos))
            f.write(memoryview(raw))
            pos = r + raw.size


# --------------------------------------------------------------- Qwen3-0.6B

# hyper-parameters the kernels are built for (qwen3_full.mlir:29-64)
QWEN3_METADATA = {"qwen3.block_count": 28, "qwen3.embedding_length": 1024,
                  "qwen3.feed_forward_length": 3072, "qwen3.attention.head_count": 16,
                  "qwen3.attention.head_count_kv": 8, "qwen3.attention.key_length": 128,
                  "qwen3.attention.value_length": 128}
QWEN3_FLOAT_METADATA = {"qwen3.rope.freq_base": 1.0e6,
                        "qwen3.attention.layer_norm_rms_epsilon": 1.0e-6}

_Q8_TENSORS = {"wq": "attn_q", "wk": "attn_k", "wv": "attn_v", "wo": "attn_output",
               "wdn": "ffn_down"}
_NORM_TENSORS = {"attn_norm": "attn_norm", "ffn_norm": "ffn_norm", "q_norm": "attn_q_norm",
                 "k_norm": "attn_k_norm"}


def check_qwen3_metadata(reader: GGUFReader) -> None:
    """Reject a file whose declared hyper-parameters differ from the ones the
    kernels are built for (keys that are absent are not checked)."""
    md = reader.metadata
    arch = md.get("general.architecture")
    if arch is not None and arch != "qwen3":
        raise GGUFError(f"{reader.path}: architecture {arch!r}, expected 'qwen3'")
    for k, v in QWEN3_METADATA.items():
        if k in md and int(md[k]) != v:
            raise GGUFError(f"{reader.path}: {k} = {md[k]}, the kernels need {v}")
    for k, v in QWEN3_FLOAT_METADATA.items():
        if k in md and abs(float(md[k]) - v) > 1e-6 * v:
            raise GGUFError(f"{reader.path}: {k} = {md[k]}, the kernels need {v}")


def _q8_into(r: GGUFReader, t: GGUFTensor, shape: tuple, out: np.ndarray) -> None:
    """Q8_0 bytes of a layer matrix into out: copied if the file holds Q8_0,
    else quantized with the reference's quantizer (create_q8_irpa.py:103-118)."""
    if tuple(t.shape) != tuple(shape):
        raise GGUFError(f"{t.name}: shape {t.shape}, expected {shape}")
    if t.ggml_type == GGML_Q8_0:
        r.read_raw(t, out)
    else:
        out[...] = Wt.quantize_q8_0(t.to_f32())


def qwen3_host_weights(path: str | Path, workers: int = 8):
    """Read a Qwen3-0.6B GGUF into decode.HostWeights (the device layout).
    Tensor bytes go straight from the file into the stacked arrays."""
    from . import decode as D

    with GGUFReader(path) as r:
        check_qwen3_metadata(r)
        L = D.LAYERS

        def f16_into(name, shape, out):
            t = r.tensor(name)
            if tuple(t.shape) != tuple(shape):
                raise GGUFError(f"{name}: shape {t.shape}, expected {shape}")
            if t.ggml_type == GGML_F16:
                r.read_raw(t, out)
            else:
                out[...] = t.to_f32().astype(np.float16)

        out = {"token_embd": np.empty((D.VOCAB, D.HIDDEN), np.float16),
               "output_w": np.empty((D.VOCAB, D.HIDDEN), np.float16),
               "output_norm": np.empty(D.HIDDEN, np.float16)}
        jobs = [lambda: f16_into("token_embd.weight", (D.VOCAB, D.HIDDEN), out["token_embd"]),
                lambda: f16_into("output_norm.weight", (D.HIDDEN,), out["output_norm"])]
        tied = "output.weight" not in r.tensors
        if not tied:
            jobs.append(lambda: f16_into("output.weight", (D.VOCAB, D.HIDDEN), out["output_w"]))
        for field, key in _NORM_TENSORS.items():
            n = D.HIDDEN if field in ("attn_norm", "ffn_norm") else D.HEAD_DIM
            out[field] = np.empty((L, n), np.float16)
            for l in range(L):
                jobs.append(lambda f=field, k=key, l=l, n=n:
                            f16_into(f"blk.{l}.{k}.weight", (n,), out[f][l]))
        for field, key in _Q8_TENSORS.items():
            n, k = D.Q8_SHAPES[field]
            out[field] = np.empty((L, n * k // 32 * 34), np.uint8)
            for l in range(L):
                jobs.append(lambda f=field, key=key, l=l, n=n, k=k:
                            _q8_into(r, r.tensor(f"blk.{l}.{key}.weight"), (n, k), out[f][l]))
        # gate rows then up rows (create_q8_irpa.py:209-224)
        half = D.FFN * D.HIDDEN // 32 * 34
        out["wgu"] = np.empty((L, 2 * half), np.uint8)
        for l in range(L):
            for part, key in ((0, "ffn_gate"), (1, "ffn_up")):
                jobs.append(lambda l=l, part=part, key=key:
                            _q8_into(r, r.tensor(f"blk.{l}.{key}.weight"), (D.FFN, D.HIDDEN),
                                     out["wgu"][l][part * half:(part + 1) * half]))
        with ThreadPoolExecutor(max_workers=max(1, workers)) as ex:
            for f in [ex.submit(j) for j in jobs]:
                f.result()
        if tied:  # no output.weight: the embedding is the output matrix
            out["output_w"][...] = out["token_embd"]
        hw = D.HostWeights(**out)
    hw.validate()
    return hw


def write_qwen3_gguf(hw, path: str | Path, tie_embeddings: bool = False) -> None:
    """Write HostWeights as a llama.cpp-style Q8_0 GGUF (tensor names and
    metadata of a Qwen3 checkpoint): the inverse of qwen3_host_weights."""
    from . import decode as D

    hw.validate()
    meta = [("general.architecture", T_STRING, "qwen3"),
            ("general.name", T_STRING, "Qwen3-0.6B (synthetic)")]
    meta += [(k, T_UINT32, v) for k, v in QWEN3_METADATA.items()]
    meta += [(k, T_FLOAT32, v) for k, v in QWEN3_FLOAT_METADATA.items()]
    tensors = [("token_embd.weight", GGML_F16, (D.VOCAB, D.HIDDEN), hw.token_embd),
               ("output_norm.weight", GGML_F32, (D.HIDDEN,), hw.output_norm.astype(np.float32))]
    if not tie_embeddings:
        tensors.append(("output.weight", GGML_F16, (D.VOCAB, D.HIDDEN), hw.output_w))
    half = D.FFN * D.HIDDEN // 32 * 34
    for l in range(D.LAYERS):
        for field, key in _NORM_TENSORS.items():
            a = getattr(hw, field)[l].astype(np.float32)
            tensors.append((f"blk.{l}.{key}.weight", GGML_F32, a.shape, a))
        for field, key in _Q8_TENSORS.items():
            tensors.append((f"blk.{l}.{key}.weight", GGML_Q8_0, D.Q8_SHAPES[field],
                            getattr(hw, field)[l]))
        tensors.append((f"blk.{l}.ffn_gate.weight", GGML_Q8_0, (D.FFN, D.HIDDEN), hw.wgu[l][:half]))
        tensors.append((f"blk.{l}.ffn_up.weight", GGML_Q8_0, (D.FFN, D.HIDDEN), hw.wgu[l][half:]))
    write_gguf(path, meta, tensors)
