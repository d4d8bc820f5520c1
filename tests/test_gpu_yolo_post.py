"""GPU parity of the YOLO postprocess (decode + filter, class-wise NMS, top-k).

The kernel and the oracle follow the reference's GPU arithmetic one operation
at a time and append candidates in anchor order, so detections must match
bit for bit (boxes, scores, classes, count), ties and the candidate cap
included.  The reference's own known-answer vector comes first.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle as O
from aexrt_amd import engine as E
from aexrt_amd import kernels as K
from aexrt_amd.runtime import NativeHipYoloModel
from aexrt_amd.yolov8 import build_yolov8n

pytestmark = pytest.mark.gpu


def test_yolo_post_reference_kat_on_gpu(cuda):
    import torch

    out = np.zeros((6, 5), dtype="float32")
    out[:4, 0] = [10, 10, 10, 10]
    out[:4, 1] = [11, 10, 10, 10]
    out[:4, 2] = [50, 50, 8, 8]
    out[:4, 3] = [80, 80, 8, 8]
    out[:4, 4] = [70, 70, 8, 8]
    out[4:, 0] = [0.9, 0.1]
    out[4:, 1] = [0.8, 0.1]
    out[4:, 2] = [0.1, 0.7]
    out[4:, 3] = [0.2, 0.1]
    out[4:, 4] = [0.4, 0.2]
    d = K.yolo_decode_nms_topk(torch.from_numpy(out).to(cuda), classes=2, conf=0.25, iou=0.5, max_candidates=8,
                               max_detections=4).cpu().numpy()
    assert [round(float(v), 2) for v in d[:, 4]] == [0.9, 0.7, 0.4]
    assert [int(v) for v in d[:, 5]] == [0, 1, 0]


POST_CASES = [
    # (anchors, classes, layout, objectness, conf, iou, max_cand, max_det, score step)
    (2100, 80, 1, False, 0.25, 0.45, 512, 100, 0.0),     # YOLOv8n-320 output0, capped candidates
    (8400, 80, 1, False, 0.6, 0.45, 512, 300, 0.0),      # 640x640
    (700, 3, 2, True, 0.2, 0.5, 2048, 2048, 0.0),        # channels last, objectness, no cap
    (1500, 4, 1, False, 0.3, 0.45, 1024, 50, 0.05),      # many exact score ties
    (33, 2, 1, False, 0.99, 0.45, 16, 8, 0.0),           # almost nothing passes
    (0, 80, 1, False, 0.25, 0.45, 512, 100, 0.0),        # no anchors
]


@pytest.mark.parametrize("case", POST_CASES)
def test_yolo_post_bit_exact_vs_oracle(cuda, case):
    import torch

    anchors, classes, layout, obj, conf, iou, mc, md, step = case
    rng = np.random.default_rng(anchors + classes)
    ch = 4 + (1 if obj else 0) + classes
    out = np.zeros((ch, anchors), np.float32)
    out[0:2] = rng.uniform(0, 320, (2, anchors))
    out[2:4] = rng.uniform(4, 80, (2, anchors))
    out[4:] = rng.uniform(0, 1, (ch - 4, anchors))
    if step:
        out[4:] = np.round(out[4:] / step) * step
    host = np.ascontiguousarray(out.T) if layout == 2 else out
    d = K.yolo_decode_nms_topk(torch.from_numpy(host).to(cuda), classes=classes, layout=layout, has_objectness=obj,
                               conf=conf, iou=iou, max_candidates=mc, max_detections=md)
    got = d.cpu().numpy()
    want = O.yolo_decode_nms_topk(host, layout=layout, classes=classes, has_objectness=obj, conf=conf, iou=iou,
                                  max_candidates=mc, max_detections=md)
    assert got.shape == want.shape
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_yolo_post_rejects_bad_arguments(cuda):
    import torch

    x = torch.zeros((84, 10), dtype=torch.float32, device=cuda)
    with pytest.raises(RuntimeError, match="max_candidates"):
        K.yolo_decode_nms_topk(x, classes=80, max_candidates=4096)
    with pytest.raises(RuntimeError, match="channels"):
        K.yolo_decode_nms_topk(x, classes=81)


DFL_CASES = [
    # (levels, classes, layout, conf, iou, max_cand, max_det)
    ([(40, 40, 8.0), (20, 20, 16.0), (10, 10, 32.0)], 80, 1, 0.25, 0.45, 512, 100),   # YOLOv8n-320 head
    ([(20, 20, 8.0), (10, 10, 16.0), (5, 5, 32.0)], 80, 2, 0.5, 0.6, 2048, 300),     # channels last, no cap
    ([(7, 9, 8.0), (4, 5, 16.0)], 3, 1, 0.3, 0.3, 64, 10),                          # ragged grids, cap
]


@pytest.mark.parametrize("case", DFL_CASES)
def test_yolo_dfl_post_bit_exact_vs_oracle(cuda, case):
    import torch

    levels, classes, layout, conf, iou, mc, md = case
    a = sum(h * w for h, w, _ in levels)
    rng = np.random.default_rng(a + classes)
    head = rng.normal(0, 2, (64 + classes, a)).astype(np.float32)
    head[64:] -= 1.0
    host = np.ascontiguousarray(head.T) if layout == 2 else head
    d = K.yolo_dfl_decode_nms_topk(torch.from_numpy(host).to(cuda), levels, classes=classes, layout=layout, conf=conf,
                                   iou=iou, max_candidates=mc, max_detections=md)
    got = d.cpu().numpy()
    want = O.yolo_dfl_decode_nms_topk(host, levels, classes=classes, layout=layout, conf=conf, iou=iou,
                                      max_candidates=mc, max_detections=md)
    assert got.shape == want.shape and want.shape[0] > 0
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_model_run_returns_reference_detections(cuda):
    """aexrt_yolo_run's detections == the oracle postprocess (raw-head decode) of the model's own output0."""
    g = build_yolov8n(batch=1, imgsz=160, seed=4)
    data = E.build_aexrt_engine(g, precision="fp16", classes=80, max_candidates=256, max_detections=50,
                                conf_threshold=0.25, iou_threshold=0.45)
    rng = np.random.default_rng(11)
    x = rng.random((1, 3, 160, 160)).astype(np.float32)
    with NativeHipYoloModel(data) as m:
        dets = m.run(x, max_detections=100)
        out0 = m.output().reshape(144, -1)
        levels = [(20, 20, 8.0), (10, 10, 16.0), (5, 5, 32.0)]
        want = O.yolo_dfl_decode_nms_topk(out0, levels, classes=80, conf=0.25, iou=0.45, max_candidates=256,
                                          max_detections=50)
        assert len(dets) == want.shape[0] > 0
        got = np.array([d[:5] + (float(d[5]),) for d in dets], np.float32)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
        # a smaller caller capacity truncates the same list
        few = m.run(x, max_detections=3)
        assert few == dets[:3]
        # device-side postprocess: same buffer contents, no host round trip
        lib = m.lib
        dptr, cptr = ctypes.c_void_p(), ctypes.c_void_p()
        assert lib.aexrt_yolo_postprocess_device(m.model, None, ctypes.byref(dptr), ctypes.byref(cptr))
        import torch

        torch.cuda.synchronize()
        cnt = np.zeros(1, np.uint32)
        buf = np.zeros((50, 6), np.float32)
        # hipMemcpy of the HIP runtime the library itself is linked against
        # (looked up through the library's handle), kind 2 = device to host
        memcpy = lib.hipMemcpy
        memcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        memcpy.restype = ctypes.c_int
        assert memcpy(cnt.ctypes.data_as(ctypes.c_void_p), cptr, 4, 2) == 0
        assert memcpy(buf.ctypes.data_as(ctypes.c_void_p), dptr, buf.nbytes, 2) == 0
        assert int(cnt[0]) == want.shape[0]
        np.testing.assert_array_equal(buf[: want.shape[0]].view(np.uint32), want.view(np.uint32))
