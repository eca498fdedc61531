"""The reference's own binding ABI: the code object's decode_dispatch_N kernels
launched as an IREE substitution stub would (binding base pointers, i32 push
constants, x / y at the reference's baked-in byte offsets) produce exactly the
bits of the C-ABI entry points -- under this build's stub shapes and under the
reference stubs' own (256-thread workgroups, N/8 and 18992 of them,
kernels/cuda/dispatch_{3,4,12,18,20,24}.mlir:5-9), plus odd shapes (a grid
smaller than the work, 128- and 192-thread workgroups)."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SEED = 515
# ordinal -> (x byte offset in binding 1, y byte offset in binding 2 or None if c0)
OFFSETS = {3: (2112, 4160), 4: (2112, None), 12: (12352, 2048), 18: (64, 6144), 20: (18432, 0)}
# workgroup count of the reference stubs (kernels/cuda/dispatch_N.mlir:6)
REF_WORKGROUPS = {3: 256, 4: 128, 12: 128, 18: 768, 20: 128, 24: 18992}
# (workgroups, workgroup size): this build's stub, the reference stub, and
# shapes with fewer waves than row quads or partial use of a workgroup
SHAPES = {"own": lambda o: (0, 0), "reference": lambda o: (REF_WORKGROUPS[o], 256),
          "few_waves": lambda o: (7, 192), "wg128": lambda o: (33, 128)}


@pytest.mark.parametrize("shape", list(SHAPES))
@pytest.mark.parametrize("ordinal", [3, 4, 12, 18, 20])
@pytest.mark.parametrize("layer", [0, 27])
def test_hal_q8_dispatch_matches_c_abi(gpu, O, Wt, ordinal, layer, shape):
    Q = gpu
    d = Q.DISPATCHES[ordinal]
    stack = np.zeros((28, d.bytes_per_layer), np.uint8)
    stack[layer] = Wt.synthetic_q8_layer(d.n, d.k, SEED, layer, d.kind)
    x = Wt.synthetic_x(d.k, SEED, ordinal)
    x_off, y_off = OFFSETS[ordinal]
    if y_off is None:
        y_off = 8194  # dispatch 4: output offset comes in c0
    b1 = np.zeros(x_off + 2 * d.k + 64, np.uint8)
    b1[x_off:x_off + 2 * d.k] = x.view(np.uint8)
    with Q.DeviceBuffer.from_array(stack) as w, Q.DeviceBuffer.from_array(b1) as bind1, \
            Q.DeviceBuffer(y_off + 2 * d.n + 64) as bind2, Q.DeviceBuffer.from_array(x) as xd, \
            Q.DeviceBuffer(2 * d.n) as yd:
        bind2.fill(0x7B)
        consts = [layer, 0] if ordinal != 4 else [y_off, layer, 0]
        wgs, wgsize = SHAPES[shape](ordinal)
        print(f"hal dispatch {ordinal} layer {layer} shape {wgs}x{wgsize}", flush=True)
        Q.hal_dispatch(ordinal, w, bind1, bind2, consts, workgroups=wgs, workgroup_size=wgsize)
        Q.q8gemv(d.kind, w, layer, xd, yd)
        Q.synchronize()
        out = bind2.download(np.uint8)
        ref = yd.download(np.uint16)
    assert np.array_equal(out[y_off:y_off + 2 * d.n].view(np.uint16), ref)
    assert np.all(out[:y_off] == 0x7B) and np.all(out[y_off + 2 * d.n:] == 0x7B)
    rep = O.gemv_tolerance_report(ref.view(np.float16), O.q8_gemv(stack[layer], d.n, d.k, x),
                                  O.q8_gemv_f64(stack[layer], d.n, d.k, x)[1])
    assert rep["fail"] == 0, rep


@pytest.mark.parametrize("shape", ["own", "reference", "few_waves"])
def test_hal_vocab_dispatch_matches_c_abi(gpu, Wt, shape):
    Q = gpu
    n, k = Q.VOCAB_ROWS, Q.HIDDEN
    W = Wt.synthetic_f16_matrix(n, k, seed=SEED, tensor=24)
    x = Wt.synthetic_x(k, SEED, 24)
    b1 = np.zeros(64 + 2 * k, np.uint8)
    b1[64:] = x.view(np.uint8)
    out_off = 1024
    with Q.DeviceBuffer.from_array(W) as w, Q.DeviceBuffer.from_array(b1) as bind1, \
            Q.DeviceBuffer(out_off + 2 * n + 64) as bind2, Q.DeviceBuffer.from_array(x) as xd, \
            Q.DeviceBuffer(2 * n) as ld, Q.DeviceBuffer(16) as td, \
            Q.DeviceBuffer(Q.vocab_workspace_bytes()) as ws:
        bind2.fill(0x7B)
        Q.vocab_workspace_reset(ws)
        wgs, wgsize = SHAPES[shape](24)
        print(f"hal dispatch 24 shape {wgs}x{wgsize}", flush=True)
        Q.hal_dispatch(24, w, bind1, bind2, [out_off], workgroups=wgs, workgroup_size=wgsize)
        Q.vocab_gemv_argmax(w, xd, ld, td, ws)
        Q.synchronize()
        out = bind2.download(np.uint8)
        ref = ld.download(np.uint16)
    assert np.array_equal(out[out_off:out_off + 2 * n].view(np.uint16), ref)
    assert np.all(out[:out_off] == 0x7B) and np.all(out[out_off + 2 * n:] == 0x7B)
