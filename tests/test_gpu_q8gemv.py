"""GPU parity of the Q8_0 GEMV kernels against the oracle, through the C ABI.

Tolerance (the GEMV bar): |gpu - ref| <= 2 f16 ulp(ref) or <= 1e-3 |ref|, with
ref the oracle in the reference kernels' f32 order; outputs whose reference is
so small that f32 rounding noise (8 * 2^-24 * sum|terms|) exceeds that rule may
pass on that floor, and each test bounds how many do.  One-hot inputs are
compared bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SEED = 4242


def _check(O, got, raw, n, k, x, max_floor=None):
    ref = O.q8_gemv(raw, n, k, x)
    _, mag = O.q8_gemv_f64(raw, n, k, x)
    rep = O.gemv_tolerance_report(got, ref, mag)
    assert rep["fail"] == 0, rep
    assert rep["on_floor"] <= (max_floor if max_floor is not None else max(2, n // 500)), rep
    return rep


@pytest.fixture(scope="module")
def stacks(Wt, Q):
    """Three distinct layers per kind (full shapes)."""
    return {d.kind: Wt.synthetic_q8_stack(d.n, d.k, 3, seed=SEED, tensor=d.kind) for d in Q.Q8_KINDS}


@pytest.mark.parametrize("kind", [0, 1, 2, 3, 4], ids=["attn_q", "attn_kv", "attn_o", "gate_up", "ffn_dn"])
def test_q8gemv_matches_oracle_per_layer(gpu, O, Wt, stacks, kind):
    Q = gpu
    d = Q.Q8_KINDS[kind]
    stack = stacks[kind]
    # the device buffer holds 28 layers' worth of bytes; layers 0, 13, 27 carry data
    full = np.zeros((28, d.bytes_per_layer), np.uint8)
    full[0], full[13], full[27] = stack[0], stack[1], stack[2]
    with Q.DeviceBuffer.from_array(full) as w_dev, Q.DeviceBuffer(2 * d.k) as x_dev, \
            Q.DeviceBuffer(2 * d.n) as y_dev:
        for li, layer in enumerate((0, 13, 27)):
            x = Wt.synthetic_x(d.k, SEED, index=layer)
            x_dev.upload(x)
            y_dev.fill(0xFF)
            Q.q8gemv(kind, w_dev, layer, x_dev, y_dev)
            Q.synchronize()
            _check(O, y_dev.download(np.float16), stack[li], d.n, d.k, x)


@pytest.mark.parametrize("ordinal", [3, 4, 12, 18, 20])
def test_reference_named_dispatch_entry_points(gpu, O, Wt, stacks, ordinal):
    Q = gpu
    d = Q.DISPATCHES[ordinal]
    stack = stacks[d.kind]
    x = Wt.synthetic_x(d.k, SEED + 1)
    with Q.DeviceBuffer.from_array(stack) as w_dev, Q.DeviceBuffer.from_array(x) as x_dev, \
            Q.DeviceBuffer(2 * d.n) as y_dev:
        Q.decode_dispatch(ordinal, w_dev, 2, x_dev, y_dev)
        Q.synchronize()
        _check(O, y_dev.download(np.float16), stack[2], d.n, d.k, x)


@pytest.mark.parametrize("kind", [1, 2, 4], ids=["K1024", "K2048", "K3072"])
def test_one_hot_x_is_bit_exact_every_layer_block_and_row(gpu, O, Wt, kind):
    """x = e_col makes y[n] = f16(scale[n, col/32] * q[n, col]) exactly: pins the
    layer stride, row stride, block order and byte order on the real shapes."""
    Q = gpu
    d = Q.Q8_KINDS[kind]
    layers = 28
    stack = Wt.synthetic_q8_stack(d.n, d.k, layers, seed=SEED + kind, tensor=kind)
    blocks = stack.reshape(layers, d.n, d.k // 32, 34)
    cols = [0, 33, d.k // 2 + 17, d.k - 1]
    with Q.DeviceBuffer.from_array(stack) as w_dev, Q.DeviceBuffer(2 * d.k) as x_dev, \
            Q.DeviceBuffer(2 * d.n) as y_dev:
        for layer in (0, 1, 14, 27):
            for col in cols:
                x = np.zeros(d.k, np.float16)
                x[col] = 1.0
                x_dev.upload(x)
                Q.q8gemv(kind, w_dev, layer, x_dev, y_dev)
                Q.synchronize()
                y = y_dev.download(np.float16)
                blk = blocks[layer, :, col // 32]
                scale = blk[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1)
                q = blk[:, 2 + col % 32].view(np.int8).astype(np.float32)
                want = (scale * q).astype(np.float16)
                assert np.array_equal(y.view(np.uint16), want.view(np.uint16)), (layer, col)


def test_gate_up_concatenation_halves(gpu, O, Wt):
    """gate_up = gate rows then up rows (create_q8_irpa.py:213-221): y[:3072]
    is gate . x and y[3072:] is up . x."""
    Q = gpu
    gate = Wt.synthetic_q8_layer(3072, 1024, SEED, 0, 31)
    up = Wt.synthetic_q8_layer(3072, 1024, SEED, 0, 32)
    gu = Wt.concat_gate_up(gate, up)
    x = Wt.synthetic_x(1024, SEED, 5)
    with Q.DeviceBuffer.from_array(gu) as w_dev, Q.DeviceBuffer.from_array(x) as x_dev, \
            Q.DeviceBuffer(2 * 6144) as y_dev:
        Q.q8gemv(Q.GATE_UP.kind, w_dev, 0, x_dev, y_dev)
        Q.synchronize()
        y = y_dev.download(np.float16)
    _check(O, y[:3072], gate, 3072, 1024, x)
    _check(O, y[3072:], up, 3072, 1024, x)


@pytest.mark.parametrize("k", [1024, 2048, 3072])
@pytest.mark.parametrize("n_rows", [1, 3, 4, 5, 17, 63, 1023])
def test_ragged_row_counts(gpu, O, Wt, k, n_rows):
    Q = gpu
    raw = Wt.synthetic_q8_layer(n_rows, k, SEED, n_rows, 40 + k // 1024)
    x = Wt.synthetic_x(k, SEED, n_rows)
    # sentinel rows after the last real row must stay untouched
    with Q.DeviceBuffer.from_array(raw) as w_dev, Q.DeviceBuffer.from_array(x) as x_dev, \
            Q.DeviceBuffer(2 * n_rows + 64) as y_dev:
        y_dev.fill(0x7B)
        Q.q8gemv_rows(w_dev, n_rows, k, x_dev, y_dev)
        Q.synchronize()
        out = y_dev.download(np.uint8)
    _check(O, out[: 2 * n_rows].view(np.float16), raw, n_rows, k, x)
    assert np.all(out[2 * n_rows:] == 0x7B)


def _batch_case(Q, Wt, stacks):
    """15 full-shape GEMVs (5 kinds x 3 layers) plus ragged ones, each with
    its own x and y."""
    items = []
    for d in Q.Q8_KINDS:
        for layer in range(3):
            items.append((d.n, d.k, stacks[d.kind][layer]))
    for n, k in ((1, 1024), (5, 3072), (1023, 2048), (17, 1024)):
        items.append((n, k, Wt.synthetic_q8_layer(n, k, SEED, n, 90 + k // 1024)))
    bufs = []
    for i, (n, k, raw) in enumerate(items):
        x = Wt.synthetic_x(k, SEED, 300 + i)
        bufs.append((Q.DeviceBuffer.from_array(raw), Q.DeviceBuffer.from_array(x),
                     Q.DeviceBuffer(2 * n + 64), x))
    return items, bufs


@pytest.mark.parametrize("wgs", [0, 1, 7, 300])
def test_batched_launch_matches_single_launches(gpu, O, Wt, stacks, wgs):
    Q = gpu
    items, bufs = _batch_case(Q, Wt, stacks)
    try:
        singles = []
        for (n, k, raw), (w, xb, y, x) in zip(items, bufs):
            Q.q8gemv_rows(w, n, k, xb, y)
        Q.synchronize()
        for (n, k, raw), (w, xb, y, x) in zip(items, bufs):
            singles.append(y.download(np.uint16, n))
            y.fill(0x7B)
        batch = Q.Q8Batch([Q.desc(w, n, k, xb, y) for (n, k, raw), (w, xb, y, x) in zip(items, bufs)])
        Q.set_batch_workgroups(wgs)
        batch.launch()
        Q.synchronize()
        for i, ((n, k, raw), (w, xb, y, x)) in enumerate(zip(items, bufs)):
            out = y.download(np.uint8)
            assert np.array_equal(out[: 2 * n].view(np.uint16), singles[i]), i
            assert np.all(out[2 * n:] == 0x7B), i
            _check(O, singles[i].view(np.float16), raw, n, k, x)
        batch.free()
    finally:
        Q.set_batch_workgroups(0)
        for b in bufs:
            for buf in b[:3]:
                buf.free()


def test_batched_qkv_of_one_layer_share_x(gpu, O, Wt, stacks):
    """q, k and v of a layer read the same x: one batched launch of the three."""
    Q = gpu
    x = Wt.synthetic_x(1024, SEED, 77)
    kv = stacks[Q.ATTN_KV.kind]
    with Q.DeviceBuffer.from_array(stacks[Q.ATTN_Q.kind]) as wq, Q.DeviceBuffer.from_array(kv) as wkv, \
            Q.DeviceBuffer.from_array(x) as xb, Q.DeviceBuffer(2 * 4096) as y:
        descs = [Q.desc_for_kind(Q.ATTN_Q.kind, wq, 1, xb, y.ptr),
                 Q.desc_for_kind(Q.ATTN_KV.kind, wkv, 1, xb, y.ptr + 4096),
                 Q.desc_for_kind(Q.ATTN_KV.kind, wkv, 2, xb, y.ptr + 6144)]
        b = Q.Q8Batch(descs)
        b.launch()
        Q.synchronize()
        out = y.download(np.float16)
        b.free()
    _check(O, out[:2048], stacks[Q.ATTN_Q.kind][1], 2048, 1024, x)
    _check(O, out[2048:3072], kv[1], 1024, 1024, x)
    _check(O, out[3072:], kv[2], 1024, 1024, x)


@pytest.mark.parametrize("layer", [0, 2])
def test_fused_qkv_matches_three_dispatches(gpu, O, Wt, stacks, layer):
    """q8gemv_qkv gives exactly the bits of decode_dispatch_3 + 2 x decode_dispatch_4."""
    Q = gpu
    x = Wt.synthetic_x(1024, SEED, 78 + layer)
    wq_h = stacks[Q.ATTN_Q.kind]
    wk_h = stacks[Q.ATTN_KV.kind]
    wv_h = Wt.synthetic_q8_stack(1024, 1024, 3, seed=SEED, tensor=99)
    with Q.DeviceBuffer.from_array(wq_h) as wq, Q.DeviceBuffer.from_array(wk_h) as wk, \
            Q.DeviceBuffer.from_array(wv_h) as wv, Q.DeviceBuffer.from_array(x) as xb, \
            Q.DeviceBuffer(2 * 4096) as y1, Q.DeviceBuffer(2 * 4096) as y2:
        Q.decode_dispatch(3, wq, layer, xb, y1.ptr)
        Q.decode_dispatch(4, wk, layer, xb, y1.ptr + 4096)
        Q.decode_dispatch(4, wv, layer, xb, y1.ptr + 6144)
        y2.fill(0x7B)
        Q.q8gemv_qkv(wq, wk, wv, layer, xb, y2.ptr, y2.ptr + 4096, y2.ptr + 6144)
        Q.synchronize()
        a, b = y1.download(np.uint16), y2.download(np.uint16)
    assert np.array_equal(a, b)
    _check(O, b[:2048].view(np.float16), wq_h[layer], 2048, 1024, x)
    _check(O, b[2048:3072].view(np.float16), wk_h[layer], 1024, 1024, x)
    _check(O, b[3072:].view(np.float16), wv_h[layer], 1024, 1024, x)


def test_zero_x_and_power_of_two_linearity(gpu, O, Wt):
    Q = gpu
    d = Q.ATTN_O
    raw = Wt.synthetic_q8_layer(d.n, d.k, SEED, 0, 60)
    x = (Wt.synthetic_x(d.k, SEED, 3).astype(np.float32) * 0.25).astype(np.float16)
    x2 = (x.astype(np.float32) * 4).astype(np.float16)
    with Q.DeviceBuffer.from_array(raw) as w_dev, Q.DeviceBuffer(2 * d.k) as x_dev, \
            Q.DeviceBuffer(2 * d.n) as y_dev:
        outs = []
        for xv in (np.zeros(d.k, np.float16), x, x2):
            x_dev.upload(xv)
            Q.q8gemv(d.kind, w_dev, 0, x_dev, y_dev)
            Q.synchronize()
            outs.append(y_dev.download(np.float16))
    assert np.all(outs[0].view(np.uint16) == 0)
    y1, y4 = outs[1].astype(np.float32), outs[2].astype(np.float32)
    normal = (np.abs(y1) >= 2.0 ** -14) & (np.abs(y4) < 60000)
    assert np.array_equal(y4[normal], 4 * y1[normal])


def test_repeatable_and_stream_ordered(gpu, O, Wt):
    Q = gpu
    d = Q.GATE_UP
    stack = Wt.synthetic_q8_stack(d.n, d.k, 2, seed=SEED, tensor=70)
    xs = [Wt.synthetic_x(d.k, SEED, i) for i in range(2)]
    s = Q.Stream()
    try:
        with Q.DeviceBuffer.from_array(stack) as w_dev, Q.DeviceBuffer.from_array(np.stack(xs)) as x_dev, \
                Q.DeviceBuffer(4 * d.n) as y_dev:
            first = None
            for _ in range(3):
                for layer in range(2):
                    Q.q8gemv(d.kind, w_dev, layer, x_dev.ptr + 2 * d.k * layer,
                             y_dev.ptr + 2 * d.n * layer, s)
                s.synchronize()
                got = y_dev.download(np.uint16)
                if first is None:
                    first = got
                assert np.array_equal(got, first)
        for layer in range(2):
            _check(O, first[layer * d.n:(layer + 1) * d.n].view(np.float16), stack[layer], d.n, d.k, xs[layer])
    finally:
        s.destroy()


def test_graph_replay_matches_eager(gpu, O, Wt):
    """A captured hipGraph of one layer's five GEMVs replays identically, with
    eager work and synchronisation between replays."""
    Q = gpu
    kinds = Q.LAYER_ORDER
    stacks = {d.kind: Wt.synthetic_q8_stack(d.n, d.k, 1, seed=SEED + 9, tensor=d.kind) for d in Q.Q8_KINDS}
    bufs = {d.kind: Q.DeviceBuffer.from_array(stacks[d.kind]) for d in Q.Q8_KINDS}
    xs = [Q.DeviceBuffer.from_array(Wt.synthetic_x(d.k, SEED, i)) for i, d in enumerate(kinds)]
    ys = [Q.DeviceBuffer(2 * d.n) for d in kinds]
    s = Q.Stream()

    def record():
        for i, d in enumerate(kinds):
            Q.q8gemv(d.kind, bufs[d.kind], 0, xs[i], ys[i], s)

    try:
        record()
        s.synchronize()
        eager = [y.download(np.uint16) for y in ys]
        g = Q.Graph(s, record)
        for rep in range(3):
            for y in ys:
                y.fill(0)
            g.launch(s)
            s.synchronize()
            assert all(np.array_equal(y.download(np.uint16), e) for y, e in zip(ys, eager)), rep
            Q.q8gemv(kinds[0].kind, bufs[kinds[0].kind], 0, xs[0], ys[0], s)  # eager work between
            s.synchronize()
        g.destroy()
        for i, d in enumerate(kinds):
            _check(O, eager[i].view(np.float16), stacks[d.kind][0], d.n, d.k,
                   xs[i].download(np.float16))
    finally:
        s.destroy()
        for b in (*bufs.values(), *xs, *ys):
            b.free()


def test_device_errors_after_init(gpu):
    Q = gpu
    with Q.DeviceBuffer(4096) as b:
        with pytest.raises(Q.Q8GemvError) as e:
            Q.q8gemv(0, b.ptr + 8, 0, b, b)
        assert e.value.code == Q.Q8_ERR_MISALIGNED
        with pytest.raises(Q.Q8GemvError) as e:
            Q.q8gemv(0, b, 28, b, b)
        assert e.value.code == Q.Q8_ERR_LAYER_RANGE
