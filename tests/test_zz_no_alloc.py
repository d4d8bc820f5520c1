"""aexrt_hip_conv2d_int8_noalloc: the int8 conv command with its amax scratch in a static device
array instead of library-allocated memory.  Its output must equal aexrt_hip_conv2d_int8's bit for
bit (same kernels, same scratch layout) on two calls in a row, the second with a smaller input,
for each of the command's three paths (per-tensor, pg16 strips, dynamic below 4096 elements)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle as O
from aexrt_amd import _lib
from aexrt_amd import kernels as K
from aexrt_amd import packing
from tests.helpers import he_weight, nchw_to_nhwc

pytestmark = pytest.mark.gpu


def _noalloc():
    return _lib.lib().aexrt_hip_conv2d_int8_noalloc


def _run_both(cuda, n, c, h, w, oc, k, s, flags, seed):
    import torch

    rng = np.random.default_rng(seed)
    x = O.round_f16(rng.standard_normal((n, c, h, w)).astype(np.float32))
    x[:, 16:32] *= 5.0
    wt = he_weight(rng, oc, c, k)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, oc).astype(np.float32))
    desc = O.conv_desc(n, c, h, w, oc, k, s, k // 2)
    alg = 51 if k == 1 else (53 if s == 2 else 52)
    pc = K.prepare_conv(desc, alg, K.SRC_LAYOUT_INT8, packing.pack_conv_int8(wt, fp16_engine=True), b, device=cuda)
    xd = torch.from_numpy(nchw_to_nhwc(x.astype(np.float16))).to(cuda)
    _, _, oh, ow = O.out_shape(desc)
    y_ref = torch.full((n, oh, ow, oc), float("nan"), dtype=torch.float16, device=cuda)
    y = torch.full((n, oh, ow, oc), float("nan"), dtype=torch.float16, device=cuda)
    K.conv2d_int8(pc, xd, y_ref, flags=flags)
    d = _lib.ConvDesc.from_params(pc.params)
    xv, yv = K.view(xd), K.view(y)
    ok = _noalloc()(ctypes.byref(d), pc.algorithm, flags, ctypes.byref(xv), pc.weight.data_ptr(),
                    pc.w_scale.data_ptr(), pc.bias.data_ptr(), None, ctypes.byref(yv), None)
    assert ok, _lib.last_error()
    torch.cuda.synchronize()
    return y_ref.cpu().numpy(), y.cpu().numpy()


@pytest.mark.parametrize("flags,first,second", [
    # per-tensor: 2x64x20x20 then 1x64x10x10 (both >= 4096 elements)
    (K.SILU, (2, 64, 20, 20, 64, 3, 1), (1, 64, 10, 10, 32, 3, 1)),
    # pg16 strips: 2x128x12x12 then 1x32x16x16
    (K.SILU | K.INT8_PG16, (2, 128, 12, 12, 64, 3, 1), (1, 32, 16, 16, 16, 1, 1)),
    # below 4096 elements (dynamic kernel, no scratch): 1x128x5x5 then 1x64x5x5
    (K.SILU, (1, 128, 5, 5, 128, 3, 1), (1, 64, 5, 5, 64, 3, 2)),
])
def test_noalloc_equals_the_allocating_command(cuda, flags, first, second):
    for seed, shape in ((51, first), (52, second)):
        ref, got = _run_both(cuda, *shape, flags, seed)
        assert not np.isnan(ref.astype(np.float32)).any()
        np.testing.assert_array_equal(got, ref)


def test_noalloc_refuses_more_channels_than_its_scratch(cuda):
    import torch

    n, c, h, w, oc = 1, 4112, 2, 2, 16
    desc = O.conv_desc(n, c, h, w, oc, 1, 1, 0)
    d = _lib.ConvDesc.from_params(desc)
    x = torch.zeros((n, h, w, c), dtype=torch.float16, device=cuda)
    y = torch.zeros((n, h, w, oc), dtype=torch.float16, device=cuda)
    wq = torch.zeros(16 * 4160, dtype=torch.uint8, device=cuda)
    ws = torch.ones(oc, dtype=torch.float32, device=cuda)
    xv, yv = K.view(x), K.view(y)
    ok = _noalloc()(ctypes.byref(d), 51, K.SILU, ctypes.byref(xv), wq.data_ptr(), ws.data_ptr(), ws.data_ptr(), None,
                    ctypes.byref(yv), None)
    assert not ok
    assert "4096 input channels" in _lib.last_error()


def test_noalloc_replays_under_graph_capture(cuda):
    """The entry recorded inside a HIP graph capture (where a caller cannot allocate) on a shape no
    other test of this file uses, then replayed three times with eager work and synchronizations
    between the replays: every replay equals the allocating command's eager output bit for bit."""
    import torch

    n, c, h, w, oc = 2, 96, 14, 14, 48
    rng = np.random.default_rng(53)
    x = O.round_f16(rng.standard_normal((n, c, h, w)).astype(np.float32))
    x[:, 32:48] *= 3.0
    wt = he_weight(rng, oc, c, 3)
    b = packing.fp16_round(rng.uniform(-0.1, 0.1, oc).astype(np.float32))
    desc = O.conv_desc(n, c, h, w, oc, 3, 1, 1)
    pc = K.prepare_conv(desc, 52, K.SRC_LAYOUT_INT8, packing.pack_conv_int8(wt, fp16_engine=True), b, device=cuda)
    xd = torch.from_numpy(nchw_to_nhwc(x.astype(np.float16))).to(cuda)
    y_ref = torch.empty((n, h, w, oc), dtype=torch.float16, device=cuda)
    y = torch.empty_like(y_ref)
    K.conv2d_int8(pc, xd, y_ref, flags=K.SILU)
    torch.cuda.synchronize()
    ref = y_ref.cpu().numpy()
    d = _lib.ConvDesc.from_params(pc.params)
    xv, yv = K.view(xd), K.view(y)
    args = (ctypes.byref(d), pc.algorithm, K.SILU, ctypes.byref(xv), pc.weight.data_ptr(), pc.w_scale.data_ptr(),
            pc.bias.data_ptr(), None, ctypes.byref(yv))
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):  # the first call on a device looks up the array's address
        assert _noalloc()(*args, ctypes.c_void_p(side.cuda_stream)), _lib.last_error()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        ok = _noalloc()(*args, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert ok, _lib.last_error()
    other = torch.empty_like(y_ref)
    for _ in range(3):
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(y.cpu().numpy(), ref)
        K.conv2d_int8(pc, xd, other, flags=K.SILU)  # eager work between the replays
        torch.cuda.synchronize()
    np.testing.assert_array_equal(other.cpu().numpy(), ref)
