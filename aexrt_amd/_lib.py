"""Loader of libaexrt_hip.so, the gfx950 backend (C ABI in include/aexrt_hip.h).

The library is built in-tree by ``aexrt_amd/build.py`` (``hipcc
--offload-arch=gfx950``).  There is no fallback: if the library is missing
or a symbol is absent every entry point raises, so nothing can silently run
on a CPU path instead.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, Structure, c_float, c_int, c_int32, c_int64, c_uint32, c_uint64, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libaexrt_hip.so"
# A host-sanitizer build of the same sources (``make -C aexrt_amd/csrc asan``)
# can be loaded instead for CPU runs of the host paths.
if os.environ.get("AEXRT_HIP_LIBRARY"):
    LIB_PATH = Path(os.environ["AEXRT_HIP_LIBRARY"]).resolve()

_lib = None


class NativeLibraryMissing(RuntimeError):
    pass


class ConvDesc(Structure):
    """native/aexrt.h:98-115 AexrtConv2DDesc."""

    _fields_ = [(name, c_uint32) for name in (
        "batch", "in_channels", "in_h", "in_w", "out_channels", "out_h", "out_w", "kernel_h",
        "kernel_w", "stride_h", "stride_w", "pad_top", "pad_left", "dilation_h", "dilation_w",
        "groups")]

    @classmethod
    def from_params(cls, params) -> "ConvDesc":
        vals = [int(v) for v in params]
        if len(vals) != 16:
            raise ValueError("conv params must have 16 values")
        return cls(*vals)

    def as_list(self) -> list[int]:
        return [int(getattr(self, f[0])) for f in self._fields_]


class TensorView(Structure):
    _fields_ = [
        ("data", c_void_p),
        ("n_stride", c_int64),
        ("c_stride", c_int32),
        ("amax_stripes", c_uint32),
        ("amax_slots", c_void_p),
        ("amax_stripe_stride", c_uint64),
    ]


class YoloDetection(Structure):
    _fields_ = [(n, c_float) for n in ("x1", "y1", "x2", "y2", "score", "class_id")]


class ConvPlanInfo(Structure):
    """native/aexrt.h:435-445 AexrtConvPlanInfo."""

    _fields_ = [
        ("struct_size", c_uint32),
        ("command_index", c_uint32),
        ("kind_is_silu", c_uint32),
        ("desc", ConvDesc),
        ("current_algorithm", c_uint32),
        ("candidate_count", c_uint32),
        ("candidates", c_uint32 * 32),
        ("in_fusion_group", c_uint32),
        ("planned_algorithm", c_uint32),
    ]


class RunTiming(Structure):
    """native/aexrt.h:43-51 AexrtYoloRunTiming."""

    _fields_ = [
        ("struct_size", c_uint32),
        ("valid", c_uint32),
        ("memcpy_ms", ctypes.c_double),
        ("submit_ms", ctypes.c_double),
        ("fence_ms", ctypes.c_double),
        ("readback_ms", ctypes.c_double),
        ("reserved", c_uint64 * 4),
    ]


class DeviceCapabilities(Structure):
    _fields_ = [
        ("struct_size", c_uint32),
        ("device_index", c_uint32),
        ("compute_units", c_uint32),
        ("wavefront_size", c_uint32),
        ("lds_bytes_per_block", c_uint32),
        ("int8_mfma", c_uint32),
        ("fp16_mfma", c_uint32),
        ("reserved", c_uint32),
        ("global_mem_bytes", c_uint64),
        ("arch_name", ctypes.c_char * 64),
    ]


_vp = c_void_p
_SIGS = {
    "aexrt_hip_abi_version": (c_uint32, []),
    "aexrt_hip_get_last_error": (ctypes.c_char_p, []),
    "aexrt_hip_amax_slots": (c_int, [POINTER(TensorView), c_uint32, c_uint32, c_uint32, c_uint32, _vp]),
    "aexrt_hip_amax_nchw": (c_int, [_vp, c_uint32, c_uint32, c_uint32, c_uint32, _vp, _vp]),
    "aexrt_hip_quantize": (c_int, [POINTER(TensorView), c_uint32, c_uint32, c_uint32, c_uint32, _vp, _vp]),
    "aexrt_hip_quant_pack_nchw": (c_int, [_vp, c_uint32, c_uint32, c_uint32, c_uint32, _vp, c_uint32, _vp, _vp]),
    "aexrt_hip_yolo_decode_nms_topk": (c_int, [_vp, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32,
                                               ctypes.c_float, ctypes.c_float, c_uint32, c_uint32, _vp, _vp,
                                               _vp]),
    "aexrt_hip_yolo_dfl_decode_nms_topk": (c_int, [_vp, c_uint32, c_uint32, _vp, _vp, c_uint32, ctypes.c_float,
                                                   ctypes.c_float, c_uint32, c_uint32, _vp, _vp, _vp]),
    "aexrt_hip_amax_strips_nhwc": (c_int, [POINTER(TensorView), c_uint32, c_uint32, c_uint32, c_uint32, _vp,
                                           _vp]),
    "aexrt_hip_quant_fused_pg16": (c_int, [_vp, c_uint32, c_uint32, c_uint32, c_uint32, _vp, _vp, _vp]),
    "aexrt_hip_conv2d_int8_pg16": (c_int, [POINTER(ConvDesc), c_uint32, c_uint32, _vp, _vp, _vp, _vp, _vp, _vp,
                                           _vp]),
    "aexrt_hip_conv2d_int8": (c_int, [POINTER(ConvDesc), c_uint32, c_uint32, POINTER(TensorView), _vp, _vp, _vp,
                                      POINTER(TensorView), POINTER(TensorView), _vp]),
    "aexrt_hip_conv2d_int8_noalloc": (c_int, [POINTER(ConvDesc), c_uint32, c_uint32, POINTER(TensorView), _vp, _vp,
                                              _vp, POINTER(TensorView), POINTER(TensorView), _vp]),
    "aexrt_hip_conv2d_f32": (c_int, [POINTER(ConvDesc), c_uint32, _vp, _vp, _vp, _vp, _vp]),
    "aexrt_hip_conv2d_fused_1x1": (c_int, [POINTER(ConvDesc), c_uint32, POINTER(TensorView), _vp, _vp,
                                           POINTER(ConvDesc), c_uint32, _vp, _vp, POINTER(TensorView), _vp]),
    "aexrt_hip_conv_chain3": (c_int, [POINTER(ConvDesc), _vp, _vp, POINTER(ConvDesc), _vp, _vp, POINTER(ConvDesc),
                                      c_uint32, _vp, _vp, POINTER(TensorView), POINTER(TensorView), c_uint32,
                                      c_uint32, _vp]),
    "aexrt_hip_conv_weight_bytes": (c_int, [POINTER(ConvDesc), c_uint32, POINTER(c_uint64)]),
    "aexrt_hip_pack_conv_weight": (c_int, [POINTER(ConvDesc), c_uint32, c_uint32, _vp, c_uint64, _vp,
                                           c_uint64, _vp]),
    "aexrt_hip_conv2d_upsampled_input": (c_int, [POINTER(ConvDesc), c_uint32, c_uint32, POINTER(TensorView),
                                                 POINTER(TensorView), c_uint32, c_uint32, _vp, _vp, _vp,
                                                 POINTER(TensorView), _vp, _vp]),
    "aexrt_hip_conv2d_upsample_copy": (c_int, [POINTER(ConvDesc), c_uint32, c_uint32, POINTER(TensorView), _vp, _vp,
                                               _vp, POINTER(TensorView), POINTER(TensorView), _vp]),
    "aexrt_hip_conv2d": (c_int, [POINTER(ConvDesc), c_uint32, c_uint32, POINTER(TensorView), _vp, _vp, _vp,
                                 POINTER(TensorView), POINTER(TensorView), _vp, _vp]),
    "aexrt_hip_conv_pair": (c_int, [POINTER(ConvDesc), c_uint32, c_uint32, POINTER(TensorView), _vp, _vp, _vp, _vp,
                                    _vp, _vp, POINTER(TensorView), c_uint32, _vp, _vp, _vp, _vp]),
    "aexrt_hip_conv_pair_barrier_timeouts": (c_uint32, []),
    "aexrt_hip_conv_candidates": (c_uint32, [POINTER(ConvDesc), c_uint32, c_uint32, POINTER(TensorView),
                                             POINTER(TensorView), POINTER(TensorView), _vp, c_uint32, c_uint32]),
    "aexrt_hip_can_use_conv_int8": (c_int, [POINTER(ConvDesc), c_uint32]),
    "aexrt_hip_set_conv_tile": (c_int, [c_int32, c_int32, c_int32]),
    "aexrt_hip_set_conv3x3_halo": (c_int, [c_int32, c_int32, c_int32, c_int32, c_int32, c_int32]),
    "aexrt_hip_set_conv_stem": (c_int, [c_int32, c_int32]),
    "aexrt_hip_set_conv1x1_stream": (c_int, [c_int32, c_int32, c_int32]),
    "aexrt_hip_fill_u32": (c_int, [_vp, c_uint64, c_uint32, _vp]),
    "aexrt_hip_nchw_f32_to_nhwc": (c_int, [_vp, c_uint32, c_uint32, c_uint32, POINTER(TensorView), _vp]),
    "aexrt_hip_nhwc_to_nchw_f32": (c_int, [POINTER(TensorView), c_uint32, c_uint32, c_uint32, c_uint32, _vp,
                                           _vp]),
    "aexrt_hip_copy": (c_int, [POINTER(TensorView), POINTER(TensorView), c_uint32, c_uint32, c_uint32, _vp]),
    "aexrt_hip_maxpool": (c_int, [POINTER(TensorView), POINTER(TensorView), c_uint32, c_uint32, c_uint32,
                                  c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, _vp]),
    "aexrt_hip_sppf_maxpool": (c_int, [POINTER(TensorView), POINTER(TensorView), POINTER(TensorView),
                                       POINTER(TensorView), c_uint32, c_uint32, c_uint32, c_uint32, _vp]),
    "aexrt_hip_resize_nearest": (c_int, [POINTER(TensorView), POINTER(TensorView), c_uint32, c_uint32,
                                         c_uint32, c_uint32, c_uint32, c_uint32, _vp]),
    "aexrt_hip_add": (c_int, [POINTER(TensorView), POINTER(TensorView), POINTER(TensorView), c_uint32,
                              c_uint32, c_uint32, _vp]),
}

# Model-level API (native/aexrt.h YOLO entry points), bound when present.
_MODEL_SIGS = {
    "aexrt_hip_create_device": (_vp, [c_uint32]),
    "aexrt_hip_validate_engine": (c_int, [_vp, c_uint64]),
    "aexrt_hip_destroy_device": (None, [_vp]),
    "aexrt_hip_get_capabilities": (c_int, [_vp, POINTER(DeviceCapabilities)]),
    "aexrt_yolo_load_engine": (_vp, [_vp, ctypes.c_char_p]),
    "aexrt_yolo_load_engine_memory": (_vp, [_vp, _vp, c_uint64]),
    "aexrt_yolo_input_element_count": (c_uint64, [_vp]),
    "aexrt_yolo_output_element_count": (c_uint64, [_vp]),
    "aexrt_yolo_class_count": (c_uint32, [_vp]),
    "aexrt_yolo_anchor_count": (c_uint32, [_vp]),
    "aexrt_yolo_channel_count": (c_uint32, [_vp]),
    "aexrt_yolo_output_layout": (c_uint32, [_vp]),
    "aexrt_yolo_graph_value_count": (c_uint32, [_vp]),
    "aexrt_yolo_prepared_command_count": (c_uint32, [_vp]),
    "aexrt_yolo_is_executable": (c_int, [_vp]),
    "aexrt_yolo_run": (c_int, [_vp, _vp, _vp, c_uint64, POINTER(YoloDetection), c_uint32, POINTER(c_uint32)]),
    "aexrt_yolo_run_device": (c_int, [_vp, _vp, _vp, _vp]),
    "aexrt_yolo_postprocess_device": (c_int, [_vp, _vp, POINTER(_vp), POINTER(_vp)]),
    "aexrt_yolo_debug_output": (c_int, [_vp, _vp, c_uint64]),
    "aexrt_yolo_debug_value": (c_int, [_vp, c_uint32, _vp, c_uint64]),
    "aexrt_yolo_value_info": (c_int, [_vp, c_uint32, POINTER(c_uint32)]),
    "aexrt_yolo_debug_conv_int8": (c_int, [_vp, c_uint32, _vp, c_uint64, _vp, c_uint32]),
    "aexrt_yolo_get_last_error": (ctypes.c_char_p, [_vp]),
    "aexrt_yolo_get_last_run_timing": (c_int, [_vp, POINTER(RunTiming)]),
    "aexrt_yolo_profile_event_count": (c_uint32, [_vp]),
    "aexrt_yolo_profile_event_label": (ctypes.c_char_p, [_vp, c_uint32]),
    "aexrt_yolo_profile_event_ms": (ctypes.c_double, [_vp, c_uint32]),
    "aexrt_yolo_conv_plan_count": (c_uint32, [_vp]),
    "aexrt_yolo_conv_plan_info": (c_int, [_vp, c_uint32, POINTER(ConvPlanInfo)]),
    "aexrt_yolo_override_conv_algorithm": (c_int, [_vp, c_uint32, c_uint32]),
    "aexrt_yolo_set_graph_capture": (c_int, [_vp, c_int]),
    "aexrt_yolo_set_profiling": (c_int, [_vp, c_int]),
    "aexrt_yolo_input_device_ptr": (_vp, [_vp]),
    "aexrt_yolo_input_ptr": (_vp, [_vp, POINTER(c_uint64)]),
    "aexrt_yolo_has_objectness": (c_uint32, [_vp]),
    "aexrt_yolo_graph_node_count": (c_uint32, [_vp]),
    "aexrt_yolo_constant_count": (c_uint32, [_vp]),
    "aexrt_yolo_destroy": (None, [_vp]),
    "aexrt_yolo_package_mode": (c_uint32, [_vp]),
    "aexrt_yolo_flush_pipeline": (c_int, [_vp, POINTER(YoloDetection), c_uint32, POINTER(c_uint32)]),
    "aexrt_yolo_pipeline_cache_size": (c_uint64, [_vp]),
    "aexrt_yolo_export_pipeline_cache": (c_int, [_vp, _vp, c_uint64]),
    "aexrt_yolo_debug_page": (c_int, [_vp, c_uint32, _vp, c_uint64]),
    "aexrt_d3d12_probe": (c_int, []),
    "aexrt_d3d12_create_device": (_vp, [c_uint32]),
    "aexrt_d3d12_destroy_device": (None, [_vp]),
    "aexrt_yolo_compile_from_package": (_vp, [_vp, ctypes.c_char_p]),
    "aexrt_yolo_compile_from_onnx": (_vp, [_vp, ctypes.c_char_p]),
}

# The reference's prepared-plan counters (native/aexrt.h:313-385), all
# uint32(model).
PLAN_COUNTERS = (
    "supported_prepared_command_count", "unsupported_prepared_command_count", "prepared_skipped_command_count",
    "late_concat_conv1x1_fusion_count", "concat_residual_conv1x1_fusion_count", "paired_conv3x3_fusion_count",
    "c2f_bottleneck_superblock_count", "c2f_tail_residual_fusion_count", "head_fusion_enabled",
    "head_final_conv_fusion_enabled", "tileflow_conv1x1_count", "tileflow_3x3_spatial_count",
    "tileflow_3x3_pack4_count", "tileflow_3x3_pack8_count", "tileflow_3x3_implicit_gemm_count",
    "tileflow_3x3_implicit_gemm_40x40_count", "tileflow_3x3_implicit_gemm_20x20_count",
    "tileflow_3x3_implicit_gemm_10x10_count", "tileflow_3x3_exact_40x40_64x64_count",
    "tileflow_3x3_exact_20x20_64x64_count", "tileflow_3x3_exact_10x10_128x128_count",
    "tileflow_3x3_exact_20x20_128x64_count", "tileflow_3x3_exact_10x10_256x64_count",
    "tileflow_native_fp16_count", "dxil_cache_hit_count", "shader_cache_hit_count", "pso_cache_hit_count",
)
for _name in PLAN_COUNTERS:
    _MODEL_SIGS["aexrt_yolo_" + _name] = (c_uint32, [_vp])


def lib():
    """The loaded library; raises NativeLibraryMissing when it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise NativeLibraryMissing(
            f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
            "(hipcc --offload-arch=gfx950).  There is no CPU fallback.")
    L = ctypes.CDLL(str(LIB_PATH))
    for table in (_SIGS, _MODEL_SIGS):
        for name, (res, args) in table.items():
            fn = getattr(L, name, None)
            if fn is None:
                if table is _SIGS:
                    raise NativeLibraryMissing(f"{LIB_PATH} lacks {name}")
                continue
            fn.restype = res
            fn.argtypes = args
    _lib = L
    return L


def last_error() -> str:
    raw = lib().aexrt_hip_get_last_error()
    return raw.decode("utf-8", "replace") if raw else ""


def check(ok: int, what: str) -> None:
    if not ok:
        raise RuntimeError(f"{what} failed: {last_error()}")
