"""CPU-side checks of the C ABI (no GPU): the library loads, exports every
symbol include/q8gemv.h and include/qwen3_decode.h declare, and validates
arguments before touching the device, reporting status codes instead of
aborting."""
from __future__ import annotations

import ctypes
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
HEADERS = (REPO / "include" / "q8gemv.h", REPO / "include" / "qwen3_decode.h")

A16 = 0x10000  # fake, 16-byte aligned "device" addresses: never dereferenced here


def declared_functions() -> list[str]:
    names = []
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names += re.findall(r"^(?:int|int64_t|void|size_t|const char\*)\s+(\w+)\s*\(", text,
                            flags=re.M)
    return names


def test_header_declares_expected_entry_points():
    names = set(declared_functions())
    for required in ("q8gemv_init", "q8gemv", "vocab_gemv_argmax",
                     "vocab_argmax_workspace_bytes", "q8gemv_shutdown",
                     "decode_dispatch_3_matmul_2048x1x1024_f16",
                     "decode_dispatch_24_matmul_151936x1x1024_f16",
                     "qwen3_decode_step", "qwen3_decode_layer", "qwen3_scratch_bytes",
                     "qwen3_prefill_batched", "qwen3_prefill_layer"):
        assert required in names


def test_library_exports_every_declared_symbol(Q):
    lib = Q.load_library()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_header(Q):
    assert set(declared_functions()) == set(Q._SIGNATURES)


def test_kind_shapes_and_bytes_per_layer(Q):
    want = {0: (2048, 1024, 2228224), 1: (1024, 1024, 1114112), 2: (1024, 2048, 2228224),
            3: (6144, 1024, 6684672), 4: (1024, 3072, 3342336)}
    for kind, shape in want.items():
        assert Q.kind_shape(kind) == shape
        d = Q.Q8_KINDS[kind]
        assert (d.n, d.k, d.bytes_per_layer) == shape
    with pytest.raises(Q.Q8GemvError) as e:
        Q.kind_shape(5)
    assert e.value.code == Q.Q8_ERR_INVALID_KIND


def test_dispatch_table_mirrors_reference_exports(Q):
    assert {o: d.export for o, d in Q.DISPATCHES.items()} == {
        3: "decode_dispatch_3_matmul_2048x1x1024_f16",
        4: "decode_dispatch_4_matmul_1024x1x1024_f16",
        12: "decode_dispatch_12_matmul_1024x1x2048_f16",
        18: "decode_dispatch_18_matmul_6144x1x1024_f16",
        20: "decode_dispatch_20_matmul_1024x1x3072_f16",
        24: "decode_dispatch_24_matmul_151936x1x1024_f16",
    }
    assert Q.VOCAB.bytes_per_layer == 151936 * 2048


@pytest.mark.parametrize("call,code", [
    (lambda L: L.q8gemv(7, A16, 0, A16, A16, None), 2),
    (lambda L: L.q8gemv(-1, A16, 0, A16, A16, None), 2),
    (lambda L: L.q8gemv(0, None, 0, A16, A16, None), 3),
    (lambda L: L.q8gemv(0, A16, 0, None, A16, None), 3),
    (lambda L: L.q8gemv(0, A16, 0, A16, None, None), 3),
    (lambda L: L.q8gemv(0, A16, 28, A16, A16, None), 4),
    (lambda L: L.q8gemv(0, A16, -1, A16, A16, None), 4),
    (lambda L: L.q8gemv(0, A16 + 8, 0, A16, A16, None), 5),
    (lambda L: L.q8gemv(0, A16, 0, A16 + 4, A16, None), 5),
    (lambda L: L.q8gemv(0, A16, 0, A16, A16 + 1, None), 5),
    (lambda L: L.q8gemv_rows(A16, 16, 512, A16, A16, None), 6),
    (lambda L: L.q8gemv_rows(A16, 0, 1024, A16, A16, None), 6),
    (lambda L: L.f16_gemv_argmax_rows(A16, 0, A16, A16, A16, A16, None), 6),
    (lambda L: L.f16_gemv_argmax_rows(A16, 10, A16, None, None, A16, None), 3),
    (lambda L: L.vocab_gemv_argmax(A16, A16, A16, A16 + 2, A16, None), 5),
    (lambda L: L.vocab_gemv_argmax(A16, A16, A16 + 1, A16, A16, None), 5),
    (lambda L: L.vocab_gemv_argmax(A16, A16, None, A16, A16 + 8, None), 5),
    (lambda L: L.q8gemv_batch_set_workgroups(70000), 9),
    (lambda L: L.q8gemv_batch_set_workgroups(-2), 9),
    (lambda L: L.vocab_set_workgroups(9000), 9),
    (lambda L: L.q8gemv_batch(A16, 0, 10, None), 9),
    (lambda L: L.q8gemv_batch(A16, 4, 2, None), 9),
    (lambda L: L.q8gemv_batch(None, 4, 8, None), 3),
    (lambda L: L.q8gemv_batch(A16 + 8, 4, 8, None), 5),
    (lambda L: L.q8gemv_desc_for_kind(9, A16, 0, A16, A16, A16), 2),
    (lambda L: L.q8gemv_qkv(A16, A16, A16, 28, A16, A16, A16, A16, None), 4),
    (lambda L: L.q8gemv_qkv(A16, None, A16, 0, A16, A16, A16, A16, None), 3),
    (lambda L: L.q8gemv_qkv(A16, A16, A16 + 4, 0, A16, A16, A16, A16, None), 5),
    (lambda L: L.q8gemv_qkv(A16, A16, A16, 0, A16, A16, A16 + 1, A16, None), 5),
    (lambda L: L.q8gemv_desc_for_kind(0, A16, 28, A16, A16, A16), 4),
    # measurement tools
    (lambda L: L.q8rt_launch_cost(0, 448, 256, 79360, 10, None), 3),
    (lambda L: L.q8rt_launch_cost(0, 0, 256, 0, 10, A16), 9),
    (lambda L: L.q8rt_launch_cost(0, 448, 2048, 0, 10, A16), 9),
    (lambda L: L.q8rt_launch_cost(1, 448, 256, 200 * 1024, 10, A16), 9),
    (lambda L: L.q8rt_handoff_latency(1, 1, 512, 1, 10, None, A16), 3),
    (lambda L: L.q8rt_handoff_latency(3, 1, 512, 1, 10, A16, A16), 9),
    (lambda L: L.q8rt_handoff_latency(128, 400, 512, 4, 10, A16, A16), 9),
    (lambda L: L.q8rt_handoff_latency(1, 1, 512, 1, 300, A16, A16), 9),
    (lambda L: L.q8rt_memory_latency(4096, None, A16), 3),
    (lambda L: L.q8rt_memory_latency(8, A16, A16), 9),
    (lambda L: L.q8rt_memory_latency(1 << 17, A16, A16), 9),
])
def test_argument_validation_before_any_device_work(Q, call, code):
    lib = Q.load_library()
    assert call(lib) == code
    assert Q.last_error()


_NOT_INITIALIZED_CHECK = """
import sys
sys.path.insert(0, sys.argv[1])
from __graft_entry__ import load_package
load_package()
from qwen3_iree_amd import q8gemv as Q
A16 = 0x10000
lib = Q.load_library()
assert lib.q8gemv(0, A16, 0, A16, A16, None) == Q.Q8_ERR_NOT_INITIALIZED
assert lib.vocab_gemv_argmax(A16, A16, None, A16, A16, None) == Q.Q8_ERR_NOT_INITIALIZED
for ordinal in (3, 4, 12, 18, 20):
    export = Q.DISPATCHES[ordinal].export
    assert getattr(lib, export)(A16, 0, A16, A16, None) == Q.Q8_ERR_NOT_INITIALIZED
try:
    Q.init(sys.argv[2])
    raise SystemExit("init of an absent code object succeeded")
except Q.Q8GemvError as e:
    assert e.code == Q.Q8_ERR_CODE_OBJECT, e.code
print("ok")
"""


def test_uninitialized_library_reports_errors(tmp_path):
    # valid arguments (fake addresses), but no code object loaded; then init
    # from an absent code object.  Checked in a fresh process: in one where
    # q8gemv_init has run, these calls would be launched and init would
    # return at once.
    r = subprocess.run([sys.executable, "-c", _NOT_INITIALIZED_CHECK, str(REPO),
                        str(tmp_path / "absent.hsaco")],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout + r.stderr


def test_workspace_size_and_tuning_roundtrip(Q):
    assert Q.vocab_workspace_bytes() == 256
    Q.set_batch_workgroups(64)
    Q.set_batch_workgroups(0)
    Q.set_vocab_workgroups(512)
    assert Q.get_vocab_workgroups() == 512
    Q.set_vocab_workgroups(0)


def test_tuning_knobs_from_two_threads_while_calls_validate(Q):
    """Setters of the process-wide knobs on one thread while another thread
    makes calls that are validated and rejected before any device work (the
    calls release the GIL, so the two really overlap): every call returns its
    status, and the knobs end with a value one of the setters wrote."""
    import threading

    L = Q.load_library()
    errors = []
    stop = threading.Event()

    def setters():
        try:
            for i in range(4000):
                assert L.q8gemv_batch_set_workgroups(64 * (i % 4)) == 0
                assert L.vocab_set_workgroups(256 * (1 + i % 3)) == 0
                assert L.qwen3_set_step_spin_limit(i % 5) == 0
        except AssertionError as e:  # pragma: no cover - reported below
            errors.append(e)
        finally:
            stop.set()

    def callers():
        n = 0
        while not stop.is_set() or n < 1000:
            if L.q8gemv(7, A16, 0, A16, A16, None) != 2:
                errors.append("q8gemv kind 7")
            if L.vocab_gemv_argmax(A16 + 2, A16, None, A16, A16, None) != 5:
                errors.append("vocab misaligned")
            if L.qwen3_step_fallback_count(None) != 3:
                errors.append("fallback count null")
            n += 1

    threads = [threading.Thread(target=setters), threading.Thread(target=callers)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errors, errors[:3]
    assert Q.get_vocab_workgroups() == 256 * (1 + 3999 % 3)  # the last value set
    Q.set_batch_workgroups(0)
    Q.set_vocab_workgroups(0)
    assert L.qwen3_set_step_spin_limit(0) == 0


def test_code_object_targets_gfx950_and_has_every_kernel():
    co = REPO / "qwen3-iree_amd" / "lib" / "q8gemv_gfx950.hsaco"
    data = co.read_bytes()
    assert data[:4] == b"\x7fELF"
    assert b"amdgcn-amd-amdhsa--gfx950" in data
    for name in ("q8gemv_p1", "q8gemv_p2", "q8gemv_p3", "q8gemv_batch_k", "q8gemv_qkv_k", "vocab_gemv_argmax_k1024",
                 "vocab_argmax_finalize", "vocab_workspace_reset", "stream_copy_b128"):
        assert name.encode() in data
    pf = (REPO / "qwen3-iree_amd" / "lib" / "prefill_gfx950.hsaco").read_bytes()
    assert pf[:4] == b"\x7fELF" and b"amdgcn-amd-amdhsa--gfx950" in pf
    for name in ("pf_embed", "pf_rmsnorm", "pf_gemm_q8", "pf_gemm_q8_res", "pf_gemm_q8_swiglu",
                 "pf_gemm_q8_m32", "pf_gemm_q8_res_m32",
                 "pf_qk_rope_cache", "pf_attention", "pf_attn_merge", "pf_set_pos",
                 "pf_gemm_q8_part", "pf_gemm_q8_part_m32", "pf_res_reduce",
                 "pf_res_reduce_norm"):
        assert name.encode() in pf


def test_desc_for_kind_addresses_the_layer(Q):
    base = 0x100000
    for d in Q.Q8_KINDS:
        desc = Q.desc_for_kind(d.kind, base, 5, A16, A16)
        assert desc.w_layer == base + 5 * d.bytes_per_layer
        assert (desc.n_rows, desc.k) == (d.n, d.k)


def _encode(Q, descs):
    import ctypes

    lib = Q.load_library()
    n = len(descs)
    arr = (Q.Q8Desc * n)(*descs)
    nbytes = lib.q8gemv_batch_table_bytes(n)
    host = (ctypes.c_uint8 * nbytes)()
    units = ctypes.c_int32(0)
    rc = lib.q8gemv_batch_encode(arr, n, host, nbytes, ctypes.byref(units))
    return rc, bytes(host), units.value


def test_batch_encode_layout(Q):
    descs = [Q.desc(0x20000, 2048, 1024, 0x30000, 0x40000),
             Q.desc(0x50000, 1023, 3072, 0x60000, 0x70002),
             Q.desc(0x80000, 1, 2048, 0x90000, 0xA0000)]
    rc, table, units = _encode(Q, descs)
    assert rc == 0
    assert units == 512 * 1 + 256 * 3 + 1 * 2
    assert len(table) == 16 + 40 * 3
    hdr = np.frombuffer(table[:16], np.int32)
    assert hdr.tolist() == [3, units, 0, 0]
    ent = np.frombuffer(table[16:], dtype=np.dtype([("w", "<u8"), ("x", "<u8"), ("y", "<u8"),
                                                     ("n", "<i4"), ("p", "<i4"),
                                                     ("ub", "<i4"), ("r", "<i4")]))
    assert ent["w"].tolist() == [0x20000, 0x50000, 0x80000]
    assert ent["y"].tolist() == [0x40000, 0x70002, 0xA0000]
    assert ent["n"].tolist() == [2048, 1023, 1]
    assert ent["p"].tolist() == [1, 3, 2]
    assert ent["ub"].tolist() == [0, 512, 512 + 768]


@pytest.mark.parametrize("bad,code", [
    (dict(w=0x20008), 5), (dict(x=0x30004), 5), (dict(y=0x40001), 5),
    (dict(k=4096), 6), (dict(n=0), 6), (dict(w=0), 3),
])
def test_batch_encode_rejects_bad_descriptors(Q, bad, code):
    f = dict(w=0x20000, n=64, k=1024, x=0x30000, y=0x40000)
    f.update(bad)
    good = Q.desc(0x20000, 64, 1024, 0x30000, 0x40000)
    rc, _, _ = _encode(Q, [good, Q.desc(f["w"], f["n"], f["k"], f["x"], f["y"])])
    assert rc == code
    assert "descriptor 1" in Q.last_error()


@pytest.mark.parametrize("ordinal,consts,code", [
    (5, [0, 0], 2),
    (3, [0], 9),
    (4, [0, 0], 9),
    (24, [0, 0], 9),
    (3, [28, 0], 4),
    (3, [0, 1], 4),
    (4, [0, 28, 0], 4),
    (4, [3, 0, 0], 5),
    (24, [7], 5),
])
def test_hal_dispatch_validation(Q, ordinal, consts, code):
    import ctypes

    lib = Q.load_library()
    c = (ctypes.c_uint32 * len(consts))(*consts)
    assert lib.q8gemv_hal_dispatch(ordinal, A16, A16, A16, c, len(consts), None) == code


@pytest.mark.parametrize("wgs,wgsize", [(256, 32), (256, 100), (256, 320), (1 << 31, 256)])
def test_hal_dispatch_grid_rejects_bad_shapes(Q, wgs, wgsize):
    """Workgroups of 64, 128, 192 or 256 threads only, and a grid that fits."""
    import ctypes

    lib = Q.load_library()
    c = (ctypes.c_uint32 * 2)(0, 0)
    assert lib.q8gemv_hal_dispatch_grid(3, A16, A16, A16, c, 2, wgs, wgsize, None) == \
        Q.Q8_ERR_BAD_ARGUMENT


# ------------------------------------------------------------ decode step ----

def _fake_weights(Q, **override):
    from qwen3_iree_amd import decode

    vals = {f: A16 + 0x100000 * i for i, f in enumerate(decode.WEIGHT_FIELDS)}
    vals.update(override)
    return decode.WeightsC(*(vals[f] for f in decode.WEIGHT_FIELDS))


def test_decode_scratch_layout(Q):
    from qwen3_iree_amd import decode

    L = Q.load_library()
    total = decode.scratch_bytes()
    assert total % 256 == 0 and 0 < total < 1 << 20
    assert L.qwen3_scratch_status_offset() < 256
    names = {"xn": 1024, "q": 2048, "k": 1024, "v": 1024, "q_roped": 2048, "attn": 2048,
             "res": 1024, "fn": 1024, "act": 3072, "on": 1024}
    spans = sorted((decode.scratch_offset(n), decode.scratch_offset(n) + 2 * c) for n, c in
                   names.items())
    assert spans[0][0] >= 256 and spans[-1][1] <= total
    for (a0, a1), (b0, _) in zip(spans, spans[1:]):
        assert a0 % 256 == 0 and a1 <= b0
    assert L.qwen3_scratch_offset(b"nope") == -1


def test_prefill_workspace_layout(Q):
    from qwen3_iree_amd import decode

    L = Q.load_library()
    assert L.qwen3_prefill_workspace_bytes(0) == 0
    assert L.qwen3_prefill_workspace_bytes((1 << 20) + 1) == 0
    for n in (1, 3, 37, 512):
        total = L.qwen3_prefill_workspace_bytes(n)
        assert total >= n * 30720 and total % 256 == 0
        nqb = (n + 31) // 32
        sizes = [(name, 2 * n * cols) for name, cols in decode.PREFILL_REGIONS]
        # attention split partials: 64 x 128 + 2 x 64 f32 per (pair, kv head)
        sizes += [("attn_part", (2 * nqb + 64) * 8 * (64 * 128 + 128) * 4)]
        # RoPE table: per token 64 cosines and 64 sines, f32
        sizes += [("rope", n * 128 * 4)]
        spans = sorted((L.qwen3_prefill_workspace_offset(n, name.encode()),
                        L.qwen3_prefill_workspace_offset(n, name.encode()) + size)
                       for name, size in sizes)
        assert spans[0][0] == 0 and spans[-1][1] <= total
        for (a0, a1), (b0, _) in zip(spans, spans[1:]):
            assert a0 % 256 == 0 and a1 <= b0
    assert L.qwen3_prefill_workspace_offset(4, b"nope") == -1
    assert L.qwen3_prefill_workspace_offset(0, b"h") == -1


@pytest.mark.parametrize("call,code", [
    # layer outside [0, 28)
    (lambda L, w: L.qwen3_decode_layer(w, 28, A16, A16, 8, A16, A16, A16 + 4096, A16, None), 4),
    (lambda L, w: L.qwen3_decode_layer(w, -1, A16, A16, 8, A16, A16, A16 + 4096, A16, None), 4),
    # h_in == h_out
    (lambda L, w: L.qwen3_decode_layer(w, 0, A16, A16, 8, A16, A16, A16, A16, None), 9),
    # max_seq
    (lambda L, w: L.qwen3_decode_step(w, A16, A16, 0, A16, A16, None, 1, A16, None), 6),
    (lambda L, w: L.qwen3_decode_step(w, A16, A16, 1 << 25, A16, A16, None, 1, A16, None), 6),
    # null / misaligned buffers
    (lambda L, w: L.qwen3_decode_step(w, None, A16, 8, A16, A16, None, 1, A16, None), 3),
    (lambda L, w: L.qwen3_decode_step(w, A16, A16, 8, None, A16, None, 1, A16, None), 3),
    (lambda L, w: L.qwen3_decode_step(w, A16, A16, 8, A16, A16, None, 1, A16 + 16, None), 5),
    (lambda L, w: L.qwen3_decode_step(w, A16 + 8, A16, 8, A16, A16, None, 1, A16, None), 5),
    (lambda L, w: L.qwen3_decode_step(w, A16, A16, 8, A16 + 2, A16, None, 1, A16, None), 5),
    (lambda L, w: L.qwen3_decode_head(w, A16, A16 + 1, A16, A16, 1, 8, A16, None), 5),
    (lambda L, w: L.qwen3_decode_embed(w, None, A16, None), 3),
    (lambda L, w: L.qwen3_decode_step_checked(w, A16, A16, 8, None, A16, None, 1, A16, None), 3),
    (lambda L, w: L.qwen3_decode_step_checked(w, A16, A16, 0, A16, A16, None, 1, A16, None), 6),
    (lambda L, w: L.qwen3_decode_step_checked(w, A16, A16, 8, A16, A16, A16 + 1, 1, A16, None),
     5),
    (lambda L, w: L.qwen3_step_fallback_count(None), 3),
    (lambda L, w: L.qwen3_debug_force_step_abort(-2), 9),
    (lambda L, w: L.qwen3_scratch_reset(A16 + 16, None), 5),
    # prompt ingestion and the generation loop
    (lambda L, w: L.qwen3_prefill(w, A16, A16, 8, None, 3, A16, A16, A16, None), 3),
    (lambda L, w: L.qwen3_prefill(w, A16, A16, 8, A16, 0, A16, A16, A16, None), 6),
    (lambda L, w: L.qwen3_prefill(w, A16, A16, 8, A16, 9, A16, A16, A16, None), 6),
    (lambda L, w: L.qwen3_prefill(w, A16, A16, 8, A16 + 2, 3, A16, A16, A16, None), 5),
    (lambda L, w: L.qwen3_generate(w, A16, A16, 8, A16, A16, 4, 0, None, A16, A16, None), 3),
    (lambda L, w: L.qwen3_generate(w, A16, A16, 8, A16, A16, 4, 0, A16, None, A16, None), 3),
    (lambda L, w: L.qwen3_generate(w, A16, A16, 8, A16, A16, -1, 0, A16, A16, A16, None), 6),
    (lambda L, w: L.qwen3_generate(w, A16, A16, 8, A16, A16, 4, 0, A16 + 1, A16, A16, None), 5),
    # batched prompt ingestion (workspace for 3 tokens: 3 * 30720 bytes)
    (lambda L, w: L.qwen3_prefill_batched(w, A16, A16, 8, None, 3, A16, A16, None, 0, A16, 1 << 20,
                                          A16, None), 3),
    (lambda L, w: L.qwen3_prefill_batched(w, A16, A16, 8, A16, 3, A16, A16, None, 0, None, 1 << 20,
                                          A16, None), 3),
    (lambda L, w: L.qwen3_prefill_batched(w, A16, A16, 8, A16, 0, A16, A16, None, 0, A16, 1 << 20,
                                          A16, None), 6),
    (lambda L, w: L.qwen3_prefill_batched(w, A16, A16, 8, A16, 9, A16, A16, None, 0, A16, 1 << 20,
                                          A16, None), 6),
    (lambda L, w: L.qwen3_prefill_batched(w, A16, A16, 8, A16, 3, A16, A16, None, 0, A16 + 16,
                                          1 << 20, A16, None), 5),
    (lambda L, w: L.qwen3_prefill_batched(w, A16, A16, 8, A16, 3, A16, A16, A16 + 2, 0, A16,
                                          1 << 20, A16, None), 5),
    (lambda L, w: L.qwen3_prefill_batched(w, A16, A16, 8, A16, 3, A16, A16, None, 0, A16,
                                          3 * 30720 - 1, A16, None), 6),
    (lambda L, w: L.qwen3_prefill_layer(w, 28, A16, A16, 8, 3, 0, 0, A16, 1 << 20, None), 4),
    (lambda L, w: L.qwen3_prefill_layer(w, 0, A16, A16, 8, 3, 6, 0, A16, 1 << 20, None), 6),
    (lambda L, w: L.qwen3_prefill_layer(w, 0, A16, A16, 8, 3, -1, 0, A16, 1 << 20, None), 6),
    (lambda L, w: L.qwen3_prefill_layer(w, 0, A16, A16, 8, 3, 0, 0, A16 + 128, 1 << 20, None), 5),
])
def test_decode_validation_before_device(Q, call, code):
    L = Q.load_library()
    w = _fake_weights(Q)
    assert call(L, ctypes.byref(w)) == code
    assert Q.last_error()


@pytest.mark.parametrize("field,value,code", [("wq", None, 3), ("output_w", A16 + 4, 5),
                                              ("token_embd", None, 3)])
def test_decode_validates_weight_pointers(Q, field, value, code):
    L = Q.load_library()
    w = _fake_weights(Q, **{field: value})
    assert L.qwen3_decode_step(ctypes.byref(w), A16, A16, 8, A16, A16, None, 1, A16, None) == code


def test_decode_null_weights_struct(Q):
    L = Q.load_library()
    assert L.qwen3_decode_step(None, A16, A16, 8, A16, A16, None, 1, A16, None) == 3
