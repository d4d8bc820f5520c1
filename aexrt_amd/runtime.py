"""ctypes shim over the model-level C ABI (the reference's cpp_runtime.py:229-679).

``NativeHipYoloModel`` mirrors ``NativeCppYoloModel``: it creates a device,
loads a ``.aexrt`` engine (path or bytes) and runs it; everything executes in
libaexrt_hip.so.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

from . import _lib
from ._lib import ConvPlanInfo, DeviceCapabilities, RunTiming, YoloDetection


class NativeHipYoloModel:
    def __init__(self, engine, device_index: int = 0) -> None:
        self.lib = _lib.lib()
        self.closed = True
        self.device = self.lib.aexrt_hip_create_device(device_index)
        if not self.device:
            raise RuntimeError(f"failed to create HIP device {device_index}: {_lib.last_error()}")
        if isinstance(engine, (bytes, bytearray, memoryview)):
            buf = bytes(engine)
            self._engine_bytes = ctypes.create_string_buffer(buf, len(buf))
            self.model = self.lib.aexrt_yolo_load_engine_memory(self.device, self._engine_bytes, len(buf))
            self.engine_path = None
        else:
            self.engine_path = os.fspath(engine)
            if not self.engine_path.lower().endswith(".aexrt"):
                self.close()
                raise ValueError("engine path must end in .aexrt")
            self.model = self.lib.aexrt_yolo_load_engine(self.device, os.fsencode(self.engine_path))
        if not self.model:
            err = _lib.last_error()
            self.lib.aexrt_hip_destroy_device(self.device)
            self.device = None
            raise RuntimeError(f"failed to load AEXRT engine: {err}")
        self.closed = False

    # --- queries (cpp_runtime.py:250-330) ---
    @property
    def input_element_count(self) -> int:
        return int(self.lib.aexrt_yolo_input_element_count(self.model))

    @property
    def output_element_count(self) -> int:
        return int(self.lib.aexrt_yolo_output_element_count(self.model))

    @property
    def class_count(self) -> int:
        return int(self.lib.aexrt_yolo_class_count(self.model))

    @property
    def anchor_count(self) -> int:
        return int(self.lib.aexrt_yolo_anchor_count(self.model))

    @property
    def channel_count(self) -> int:
        return int(self.lib.aexrt_yolo_channel_count(self.model))

    @property
    def output_layout(self) -> int:
        return int(self.lib.aexrt_yolo_output_layout(self.model))

    @property
    def executable(self) -> bool:
        return bool(self.lib.aexrt_yolo_is_executable(self.model))

    @property
    def graph_value_count(self) -> int:
        return int(self.lib.aexrt_yolo_graph_value_count(self.model))

    @property
    def prepared_command_count(self) -> int:
        return int(self.lib.aexrt_yolo_prepared_command_count(self.model))

    @property
    def package_mode(self) -> int:
        return int(self.lib.aexrt_yolo_package_mode(self.model))

    def counter(self, name: str) -> int:
        """One of the reference's prepared-plan counters (native/aexrt.h:313-385), by the name
        after ``aexrt_yolo_`` (e.g. ``"tileflow_conv1x1_count"``)."""
        if name not in _lib.PLAN_COUNTERS:
            raise KeyError(name)
        return int(getattr(self.lib, "aexrt_yolo_" + name)(self.model))

    def counters(self) -> dict:
        return {name: self.counter(name) for name in _lib.PLAN_COUNTERS}

    def flush_pipeline(self, max_detections: int = 100) -> list:
        dets = (YoloDetection * max(1, max_detections))()
        count = ctypes.c_uint32(0)
        if not self.lib.aexrt_yolo_flush_pipeline(self.model, dets, max(1, max_detections), ctypes.byref(count)):
            raise RuntimeError(f"flush_pipeline failed: {self.last_error()}")
        return [(d.x1, d.y1, d.x2, d.y2, d.score, int(d.class_id)) for d in dets[: count.value]]

    def pipeline_cache(self) -> bytes:
        n = int(self.lib.aexrt_yolo_pipeline_cache_size(self.model))
        buf = ctypes.create_string_buffer(max(n, 1))
        if n and not self.lib.aexrt_yolo_export_pipeline_cache(self.model, buf, n):
            raise RuntimeError(f"export_pipeline_cache failed: {self.last_error()}")
        return buf.raw[:n]

    @property
    def capabilities(self) -> dict:
        caps = DeviceCapabilities()
        caps.struct_size = ctypes.sizeof(DeviceCapabilities)
        if not self.lib.aexrt_hip_get_capabilities(self.device, ctypes.byref(caps)):
            raise RuntimeError(_lib.last_error())
        return {f[0]: (getattr(caps, f[0]).decode() if f[0] == "arch_name" else int(getattr(caps, f[0])))
                for f in DeviceCapabilities._fields_ if f[0] not in ("struct_size", "reserved")}

    def last_error(self) -> str:
        raw = self.lib.aexrt_yolo_get_last_error(self.model)
        return raw.decode("utf-8", "replace") if raw else ""

    # --- run ---
    def run(self, image: np.ndarray, max_detections: int = 100) -> list:
        """Host fp32 NCHW input -> detections (cpp_runtime.py:400-440)."""
        x = np.ascontiguousarray(image, dtype=np.float32).reshape(-1)
        if x.size < self.input_element_count:
            raise ValueError("input has too few elements")
        dets = (YoloDetection * max(1, max_detections))()
        count = ctypes.c_uint32(0)
        ok = self.lib.aexrt_yolo_run(self.device, self.model, x.ctypes.data_as(ctypes.c_void_p), x.size, dets,
                                     max_detections, ctypes.byref(count))
        if not ok:
            raise RuntimeError(f"aexrt_yolo_run failed: {self.last_error()}")
        return [(d.x1, d.y1, d.x2, d.y2, d.score, int(d.class_id)) for d in dets[: count.value]]

    def run_device(self, input_ptr: Optional[int] = None, stream=None) -> None:
        """Run with the input already in HBM (no host sync)."""
        s = None if stream is None else ctypes.c_void_p(int(getattr(stream, "cuda_stream", stream) or 0))
        ok = self.lib.aexrt_yolo_run_device(self.model, None if input_ptr is None else ctypes.c_void_p(input_ptr),
                                            s, None)
        if not ok:
            raise RuntimeError(f"aexrt_yolo_run_device failed: {self.last_error()}")

    @property
    def input_device_ptr(self) -> int:
        return int(self.lib.aexrt_yolo_input_device_ptr(self.model) or 0)

    def output(self) -> np.ndarray:
        """Raw network output as fp32 in logical order ([N, C, A] or NCHW)."""
        n = self.output_element_count
        out = np.empty(n, dtype=np.float32)
        if not self.lib.aexrt_yolo_debug_output(self.model, out.ctypes.data_as(ctypes.c_void_p), n):
            raise RuntimeError(f"debug_output failed: {self.last_error()}")
        return out

    def value_info(self, value_id: int):
        dims = (ctypes.c_uint32 * 4)()
        rank = self.lib.aexrt_yolo_value_info(self.model, value_id, dims)
        return rank, tuple(int(v) for v in dims)

    def value(self, value_id: int) -> np.ndarray:
        rank, dims = self.value_info(value_id)
        if rank == 0:
            raise ValueError(f"value {value_id} has no device storage")
        n = int(np.prod(dims))
        out = np.empty(n, dtype=np.float32)
        if not self.lib.aexrt_yolo_debug_value(self.model, value_id, out.ctypes.data_as(ctypes.c_void_p), n):
            raise RuntimeError(f"debug_value failed: {self.last_error()}")
        shape = dims if rank == 4 else dims[:3]
        return out.reshape(shape)

    def debug_conv_int8(self, command_index: int, batch: int, out_hw: tuple, out_channels: int,
                        in_channels: int):
        """The int32 accumulators ([N, OH, OW, OC]) of per-tensor int8 conv ``command_index`` as
        the last run computed them, and its input's per-16-channel amax words (uint32)."""
        oh, ow = out_hw
        acc = np.empty((batch, oh, ow, out_channels), dtype=np.int32)
        slots = np.empty(in_channels // 16, dtype=np.uint32)
        if not self.lib.aexrt_yolo_debug_conv_int8(self.model, command_index, acc.ctypes.data_as(ctypes.c_void_p),
                                                   acc.size, slots.ctypes.data_as(ctypes.c_void_p), slots.size):
            raise RuntimeError(f"debug_conv_int8 failed: {self.last_error()}")
        return acc, slots

    def last_run_timing(self) -> Optional[dict]:
        t = RunTiming()
        t.struct_size = ctypes.sizeof(RunTiming)
        if not self.lib.aexrt_yolo_get_last_run_timing(self.model, ctypes.byref(t)) or not t.valid:
            return None
        return dict(memcpy_ms=t.memcpy_ms, submit_ms=t.submit_ms, fence_ms=t.fence_ms, readback_ms=t.readback_ms)

    def set_profiling(self, enabled: bool) -> None:
        self.lib.aexrt_yolo_set_profiling(self.model, int(enabled))

    def set_graph_capture(self, enabled: bool) -> None:
        self.lib.aexrt_yolo_set_graph_capture(self.model, int(enabled))

    def profile_events(self) -> list:
        n = int(self.lib.aexrt_yolo_profile_event_count(self.model))
        out = []
        for i in range(n):
            raw = self.lib.aexrt_yolo_profile_event_label(self.model, i)
            out.append(((raw or b"").decode(), float(self.lib.aexrt_yolo_profile_event_ms(self.model, i))))
        return out

    # --- conv plan (cpp_runtime.py conv_plan_info / override) ---
    def conv_plan(self) -> list:
        out = []
        for i in range(int(self.lib.aexrt_yolo_conv_plan_count(self.model))):
            info = ConvPlanInfo()
            info.struct_size = ctypes.sizeof(ConvPlanInfo)
            if not self.lib.aexrt_yolo_conv_plan_info(self.model, i, ctypes.byref(info)):
                raise RuntimeError(self.last_error())
            out.append(dict(command_index=info.command_index, silu=bool(info.kind_is_silu),
                            desc=info.desc.as_list(), current_algorithm=info.current_algorithm,
                            planned_algorithm=info.planned_algorithm,
                            candidates=[info.candidates[k] for k in range(info.candidate_count)],
                            in_fusion_group=bool(info.in_fusion_group)))
        return out

    def override_conv_algorithm(self, command_index: int, algorithm_id: int) -> None:
        if not self.lib.aexrt_yolo_override_conv_algorithm(self.model, command_index, algorithm_id):
            raise RuntimeError(f"override failed: {self.last_error()}")

    def close(self) -> None:
        if getattr(self, "model", None):
            self.lib.aexrt_yolo_destroy(self.model)
            self.model = None
        if getattr(self, "device", None):
            self.lib.aexrt_hip_destroy_device(self.device)
            self.device = None
        self.closed = True

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
