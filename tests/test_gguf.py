"""GGUF reading / writing and Qwen3 weight ingestion (CPU only).

The reader is pinned against a file assembled here byte by byte from the
GGUF v3 layout (not with the module's writer), then the writer against the
reader, then the Qwen3 ingestion against the arrays it was written from (a
full-size synthetic checkpoint, bit for bit) and against the reference's
conversion rules (create_q8_irpa.py: Q8_0 bytes kept, f32 layer matrices
quantized, gate rows then up rows, norms stacked as f16).
"""
from __future__ import annotations

import struct

import numpy as np
import pytest


@pytest.fixture(scope="module")
def G():
    from qwen3_iree_amd import gguf

    return gguf


def _s(text: str) -> bytes:
    b = text.encode()
    return struct.pack("<Q", len(b)) + b


def handmade_gguf(alignment: int = 64) -> tuple[bytes, dict]:
    """A GGUF v3 file built directly from the format description."""
    meta = b""
    meta += _s("general.architecture") + struct.pack("<I", 8) + _s("qwen3")
    meta += _s("general.alignment") + struct.pack("<I", 4) + struct.pack("<I", alignment)
    meta += _s("x.i8") + struct.pack("<I", 1) + struct.pack("<b", -5)
    meta += _s("x.bool") + struct.pack("<I", 7) + struct.pack("<?", True)
    meta += _s("x.f64") + struct.pack("<I", 12) + struct.pack("<d", 2.5)
    meta += _s("x.u64") + struct.pack("<I", 10) + struct.pack("<Q", 1 << 40)
    meta += (_s("x.strs") + struct.pack("<I", 9) + struct.pack("<IQ", 8, 2) + _s("ab") + _s("héllo"))
    meta += (_s("x.ints") + struct.pack("<I", 9) + struct.pack("<IQ", 5, 3)
             + struct.pack("<3i", 7, -8, 9))
    meta += (_s("x.nested") + struct.pack("<I", 9) + struct.pack("<IQ", 9, 2)
             + struct.pack("<IQ", 0, 1) + b"\x05" + struct.pack("<IQ", 0, 0))
    f32 = np.arange(6, dtype=np.float32).reshape(2, 3) - 2.5
    f16 = (np.arange(8, dtype=np.float16) / 4).reshape(8)
    q8 = np.zeros(34 * 2, np.uint8)
    q8[0:2] = np.array([0.5], np.float16).view(np.uint8)  # block 0: scale 0.5
    q8[2:34] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    q8[34:36] = np.array([-2.0], np.float16).view(np.uint8)
    q8[36:68] = np.arange(32, dtype=np.int8).view(np.uint8)
    infos = b""
    # dims are written fastest first: the [2, 3] tensor is dims (3, 2)
    infos += _s("a.f32") + struct.pack("<I", 2) + struct.pack("<QQ", 3, 2) + struct.pack("<IQ", 0, 0)
    infos += _s("b.f16") + struct.pack("<I", 1) + struct.pack("<Q", 8) + struct.pack("<IQ", 1, alignment)
    infos += (_s("c.q8") + struct.pack("<I", 2) + struct.pack("<QQ", 32, 2)
              + struct.pack("<IQ", 8, 2 * alignment))
    head = struct.pack("<IIQQ", 0x46554747, 3, 3, 9) + meta + infos
    head += b"\0" * ((-len(head)) % alignment)
    data = bytearray(3 * alignment)
    data[0:24] = f32.tobytes()
    data[alignment:alignment + 16] = f16.tobytes()
    data[2 * alignment:2 * alignment + 68] = q8.tobytes()
    q8_values = np.concatenate([0.5 * np.arange(-16, 16), -2.0 * np.arange(32)]).reshape(2, 32)
    return head + bytes(data), {"f32": f32, "f16": f16, "q8": q8_values, "q8_raw": q8,
                                "data_offset": len(head)}


def test_reader_on_handmade_file(G, tmp_path):
    blob, want = handmade_gguf(64)
    p = tmp_path / "h.gguf"
    p.write_bytes(blob)
    with G.GGUFReader(p) as r:
        assert r.version == 3 and r.alignment == 64 and r.data_offset == want["data_offset"]
        md = r.metadata
        assert md["general.architecture"] == "qwen3" and md["x.i8"] == -5 and md["x.bool"] is True
        assert md["x.f64"] == 2.5 and md["x.u64"] == 1 << 40
        assert md["x.strs"] == ["ab", "héllo"] and md["x.ints"].tolist() == [7, -8, 9]
        assert md["x.nested"][0].tolist() == [5] and md["x.nested"][1].size == 0
        a, b, c = r.tensor("a.f32"), r.tensor("b.f16"), r.tensor("c.q8")
        assert a.shape == (2, 3) and b.shape == (8,) and c.shape == (2, 32)
        assert np.array_equal(a.to_f32(), want["f32"])
        assert np.array_equal(b.to_f16(), want["f16"])
        assert np.array_equal(c.raw(), want["q8_raw"])
        assert np.array_equal(c.to_f32(), want["q8"])
        assert c.offset == want["data_offset"] + 128 and c.nbytes == 68


def test_writer_roundtrip_all_value_types(G, tmp_path):
    rng = np.random.default_rng(4)
    meta = [("general.architecture", G.T_STRING, "qwen3"),
            ("u8", G.T_UINT8, 200), ("i16", G.T_INT16, -300), ("u32", G.T_UINT32, 70000),
            ("f32", G.T_FLOAT32, 0.25), ("b", G.T_BOOL, False), ("i64", G.T_INT64, -(1 << 50)),
            ("arr.f32", G.T_ARRAY, (G.T_FLOAT32, np.array([1.5, -2.0], np.float32))),
            ("arr.str", G.T_ARRAY, (G.T_STRING, ["x", "", "yz"]))]
    bf = (rng.standard_normal(64).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    tensors = [("t.f16", G.GGML_F16, (4, 8), rng.standard_normal((4, 8)).astype(np.float16)),
               ("t.f32", G.GGML_F32, (3,), np.array([1, 2, 3], np.float32)),
               ("t.bf16", G.GGML_BF16, (64,), bf),
               ("t.q8", G.GGML_Q8_0, (2, 64), rng.integers(0, 256, 4 * 34).astype(np.uint8))]
    for alignment in (32, 256):
        p = tmp_path / f"w{alignment}.gguf"
        G.write_gguf(p, meta, tensors, alignment=alignment)
        with G.GGUFReader(p) as r:
            assert r.alignment == alignment and r.data_offset % alignment == 0
            for k, _, v in meta:
                got = r.metadata[k]
                if isinstance(v, tuple):
                    v = v[1]
                    got = list(got) if not isinstance(got, list) else got
                    v = list(v)
                assert got == v, k
            for name, _, shape, data in tensors:
                t = r.tensor(name)
                assert t.shape == shape and (t.offset - r.data_offset) % alignment == 0
                assert np.array_equal(t.raw(), np.ascontiguousarray(data).view(np.uint8).reshape(-1))
            want_bf = (bf.astype(np.uint32) << 16).view(np.float32)
            assert np.array_equal(r.tensor("t.bf16").to_f32(), want_bf)


@pytest.mark.parametrize("mutate,msg", [
    (lambda b: b"GGUX" + b[4:], "not a GGUF"),
    (lambda b: b[:4] + struct.pack("<I", 1) + b[8:], "version 1"),
    (lambda b: b[:40], "truncated|past the end"),
    (lambda b: b[:-10], "past the end"),
])
def test_reader_rejects_bad_files(G, tmp_path, mutate, msg):
    blob, _ = handmade_gguf(64)
    p = tmp_path / "bad.gguf"
    p.write_bytes(mutate(blob))
    with pytest.raises(G.GGUFError, match=msg):
        G.GGUFReader(p)


@pytest.fixture(scope="module")
def qwen3_file(G, model_host, tmp_path_factory):
    p = tmp_path_factory.mktemp("gguf") / "qwen3-synthetic-q8_0.gguf"
    G.write_qwen3_gguf(model_host, p)
    return p


def test_qwen3_roundtrip_full_size(G, model_host, qwen3_file, tmp_path):
    hw = G.qwen3_host_weights(qwen3_file)
    from qwen3_iree_amd import decode as D

    for f in D.WEIGHT_FIELDS:
        a, b = getattr(hw, f), getattr(model_host, f)
        assert a.dtype == b.dtype and a.shape == b.shape, f
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f
    # tied embeddings: no output.weight -> token_embd
    p2 = tmp_path / "tied.gguf"
    G.write_qwen3_gguf(model_host, p2, tie_embeddings=True)
    hw2 = G.qwen3_host_weights(p2)
    assert np.array_equal(hw2.output_w.view(np.uint16), model_host.token_embd.view(np.uint16))


def test_qwen3_float_layer_matrices_are_quantized_like_the_reference(G, model_host, qwen3_file,
                                                                     tmp_path):
    """A layer matrix stored as f32 (an f32 / f16 checkpoint) goes through the
    reference quantizer; gate and up land in that order."""
    from qwen3_iree_amd import decode as D
    from qwen3_iree_amd import weights as Wt

    rng = np.random.default_rng(9)
    q_f32 = (0.02 * rng.standard_normal((2048, 1024))).astype(np.float32)
    up_f32 = (0.02 * rng.standard_normal((3072, 1024))).astype(np.float32)
    # rewrite with blk.3.attn_q and blk.5.ffn_up as f32
    with G.GGUFReader(qwen3_file) as r:
        meta = [(k, r.metadata_types[k], r.metadata[k] if r.metadata_types[k] != G.T_ARRAY else None)
                for k in r.metadata]
        tensors = []
        for name, t in r.tensors.items():
            if name == "blk.3.attn_q.weight":
                tensors.append((name, G.GGML_F32, (2048, 1024), q_f32))
            elif name == "blk.5.ffn_up.weight":
                tensors.append((name, G.GGML_F32, (3072, 1024), up_f32))
            else:
                tensors.append((name, t.ggml_type, t.shape, np.array(t.raw())))
    p2 = tmp_path / "mixed2.gguf"
    G.write_gguf(p2, meta, tensors)
    hw = G.qwen3_host_weights(p2)
    assert np.array_equal(hw.wq[3], Wt.quantize_q8_0(q_f32))
    half = D.FFN * D.HIDDEN // 32 * 34
    assert np.array_equal(hw.wgu[5][:half], model_host.wgu[5][:half])
    assert np.array_equal(hw.wgu[5][half:], Wt.quantize_q8_0(up_f32))
    assert np.array_equal(hw.wq[2], model_host.wq[2])


def test_qwen3_metadata_mismatch_is_rejected(G, tmp_path):
    t = [("token_embd.weight", G.GGML_F16, (2, 1024), np.zeros((2, 1024), np.float16))]
    p = tmp_path / "m.gguf"
    G.write_gguf(p, [("general.architecture", G.T_STRING, "qwen3"),
                     ("qwen3.block_count", G.T_UINT32, 36)], t)
    with pytest.raises(G.GGUFError, match="block_count"):
        G.qwen3_host_weights(p)
    G.write_gguf(p, [("general.architecture", G.T_STRING, "llama")], t)
    with pytest.raises(G.GGUFError, match="architecture"):
        G.qwen3_host_weights(p)
    G.write_gguf(p, [("general.architecture", G.T_STRING, "qwen3")], t)
    with pytest.raises(G.GGUFError, match="shape"):
        G.qwen3_host_weights(p)
