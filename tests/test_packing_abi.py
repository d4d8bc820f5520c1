"""CPU checks of the build-time packers and the C ABI's host-side parts.

No GPU is touched: the library is loaded and only host functions (weight
repack, eligibility) are called.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

import oracle as O
from aexrt_amd import _lib, kernels as K, packing

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"


def test_library_exports_every_declared_symbol():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        names.update(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(aexrt_\w+)\s*\(", text, re.M))
    assert len(names) >= 15
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing


def test_library_exports_every_symbol_the_reference_wrapper_binds():
    """NativeCppYoloModel._configure (src/aexrt/cpp_runtime.py:543-662) binds these names; a
    missing one makes the reference's own wrapper fail on load."""
    names = (GOLDEN / "reference_ffi_symbols.txt").read_text().split()
    assert len(names) == 54
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_reference_compile_entry_points_refuse_with_a_diagnostic():
    L = _lib.lib()
    assert L.aexrt_yolo_compile_from_onnx(None, b"model.onnx") is None
    assert "not supported" in _lib.last_error()
    assert L.aexrt_yolo_compile_from_package(None, b"pkg") is None
    assert "aexrt_yolo_load_engine" in _lib.last_error()


def test_model_queries_on_null_model_are_zero():
    """Every counter the reference's wrapper reads answers 0 for a null model, as in RT:30676-30810."""
    L = _lib.lib()
    for name in _lib.PLAN_COUNTERS:
        assert getattr(L, "aexrt_yolo_" + name)(None) == 0, name
    assert L.aexrt_yolo_package_mode(None) == 0
    assert L.aexrt_yolo_pipeline_cache_size(None) == 0
    det = (_lib.YoloDetection * 4)()
    cnt = ctypes.c_uint32(7)
    assert L.aexrt_yolo_flush_pipeline(None, det, 4, ctypes.byref(cnt)) == 0


def test_library_loads_and_reports_abi():
    assert _lib.lib().aexrt_hip_abi_version() == 2


@pytest.mark.parametrize("fp16_engine", [True, False])
@pytest.mark.parametrize("shape", [(256, 128, 1, 1), (64, 16, 3, 3), (32, 48, 3, 3)])
def test_layout8_packer_matches_oracle(shape, fp16_engine):
    rng = np.random.default_rng(sum(shape))
    w = (rng.standard_normal(shape) * 0.3).astype(np.float32)
    w[3] = 0.0  # an all-zero row -> scale 1
    payload = packing.pack_conv_int8(w, fp16_engine=fp16_engine)
    q, s = O.weight_quant(w, fp16_round=fp16_engine)
    assert payload == q.tobytes() + s.astype("<f4").tobytes()
    assert s[3] == 1.0


def test_layout8_half_away_edge_follows_compiler_not_runtime():
    # |p| = 0.5 - 2^-25: the compiler's fp32 floor(|p| + 0.5) gives 1, the
    # runtime's std::round gives 0 (engine.py:2453-2456 vs RT:21736).
    edge = np.float32(0.5) - np.float32(2.0 ** -25)
    w = np.array([[127.0, edge, -edge, 0.0]], np.float32).reshape(1, 4, 1, 1)
    q, s = packing.quantize_conv_int8(w, fp16_engine=False)
    assert s[0] == 1.0 and q.reshape(-1).tolist() == [127, 1, -1, 0]
    oq, _ = O.weight_quant(w, fp16_round=False)
    assert oq.reshape(-1).tolist() == [127, 1, -1, 0]
    # the C ABI's raw-weight fallback repeats the runtime's std::round
    params = O.conv_desc(1, 4, 2, 2, 8, 1, 1, 0)
    w8 = np.zeros((8, 4, 1, 1), np.float32)
    w8[0] = w[0]
    packed, scales = K.pack_conv_weight(params, 51, K.SRC_RAW_F32, w8)
    row = packed.view(np.int8)[: 4]
    assert row.tolist() == [127, 0, 0, 0]


def test_winograd_packers_match_reference_kat():
    g = np.load(GOLDEN / "winograd_f2x2_kat.npz")
    w = (np.arange(32 * 32 * 9, dtype=np.float32).reshape(32, 32, 3, 3) / 4096.0)
    f16 = np.frombuffer(packing.pack_winograd_f2x2_fp16(w), dtype="<u2").reshape(32, 32, 4, 4)
    np.testing.assert_array_equal(f16, g["expected_f16_bits"])
    f32 = np.frombuffer(packing.pack_winograd_f2x2_fp32(w), dtype="<f4").reshape(32, 32, 4, 4)
    np.testing.assert_array_equal(f32, g["expected_f32"])


def test_conv1x1_oc8_packer_matches_reference_kat():
    g = np.load(GOLDEN / "conv1x1_oc8_kat.npz")
    w = (np.arange(64 * 64, dtype=np.float32) / 1024.0).reshape(64, 64, 1, 1)
    got = np.frombuffer(packing.pack_conv1x1_oc8_fp16(w), dtype="<u2").reshape(8, 64, 8)
    np.testing.assert_array_equal(got, g["expected_f16_bits"])


def _kmajor(w: np.ndarray, kp: int, ocp: int) -> np.ndarray:
    oc, ic, kh, kw = w.shape
    out = np.zeros((ocp, kp), w.dtype)
    out[:oc, : ic * kh * kw] = w.transpose(0, 2, 3, 1).reshape(oc, -1)
    return out


@pytest.mark.parametrize("k,s,alg", [(1, 1, 51), (3, 1, 52), (3, 2, 53)])
def test_abi_int8_repack_is_kmajor_tap_then_channel(k, s, alg):
    rng = np.random.default_rng(3)
    oc, ic = 24, 48
    w = rng.standard_normal((oc, ic, k, k)).astype(np.float32)
    params = O.conv_desc(1, ic, 10, 10, oc, k, s, k // 2)
    payload = packing.pack_conv_int8(w, fp16_engine=True)
    packed, scales = K.pack_conv_weight(params, alg, K.SRC_LAYOUT_INT8, payload)
    q, sc = packing.quantize_conv_int8(w, fp16_engine=True)
    kp = (ic * k * k + 63) // 64 * 64
    np.testing.assert_array_equal(packed.view(np.int8).reshape(32, kp), _kmajor(q, kp, 32))
    np.testing.assert_array_equal(scales, sc)


@pytest.mark.parametrize("layout", ["raw32", "raw16", "oc8", "oc4"])
def test_abi_fp16_repack_from_every_source_layout(layout):
    rng = np.random.default_rng(4)
    k = 1 if layout == "oc8" else 3
    oc, ic = 16, 24
    w = rng.standard_normal((oc, ic, k, k)).astype(np.float32)
    params = O.conv_desc(1, ic, 8, 8, oc, k, 2 if layout == "oc4" else 1, k // 2)
    if layout == "raw32":
        src, lay = w, K.SRC_RAW_F32
    elif layout == "raw16":
        src, lay = w.astype("<f2"), K.SRC_RAW_F16
    elif layout == "oc8":
        src, lay = np.frombuffer(packing.pack_conv1x1_oc8_fp16(w), np.uint8), K.SRC_LAYOUT_OC8_F16
    else:
        src, lay = np.frombuffer(packing.pack_conv3x3_oc4_fp16(w), np.uint8), K.SRC_LAYOUT_OC4_F16
    packed, _ = K.pack_conv_weight(params, 5, lay, src)
    kp = (ic * k * k + 63) // 64 * 64
    want = _kmajor(w.astype(np.float16), kp, 16)
    np.testing.assert_array_equal(packed.view(np.float16).reshape(16, kp), want)


def test_abi_winograd_repack_point_major():
    rng = np.random.default_rng(5)
    oc, ic = 20, 40
    w = rng.standard_normal((oc, ic, 3, 3)).astype(np.float32)
    params = O.conv_desc(1, ic, 8, 8, oc, 3, 1, 1)
    u = np.frombuffer(packing.pack_winograd_f2x2_fp16(w), dtype=np.float16).reshape(oc, ic, 16)
    packed, _ = K.pack_conv_weight(params, 40, K.SRC_LAYOUT_WINO_F16, np.frombuffer(u.tobytes(), np.uint8))
    ocp, cp = 32, 64
    got = packed.view(np.float16).reshape(16, ocp, cp)
    want = np.zeros((16, ocp, cp), np.float16)
    want[:, :oc, :ic] = u.transpose(2, 0, 1)
    np.testing.assert_array_equal(got, want)
    # raw weights go through the same transform on the host
    raw, _ = K.pack_conv_weight(params, 40, K.SRC_RAW_F32, w)
    np.testing.assert_allclose(raw.view(np.float16).astype(np.float32), packed.view(np.float16).astype(np.float32),
                               rtol=2e-3, atol=2e-3)


def test_int8_eligibility_follows_reference_plus_c16():
    ok = [O.conv_desc(1, 64, 20, 20, 64, 3, 1, 1), O.conv_desc(1, 64, 40, 40, 128, 3, 2, 1),
          O.conv_desc(1, 128, 40, 40, 256, 1, 1, 0)]
    for d in ok:
        assert K.can_use_conv_int8(d, 1 if d[7] == 1 else 9)
    bad = [
        (O.conv_desc(1, 3, 320, 320, 16, 3, 2, 1), 9),     # cin % 4 (stem)
        (O.conv_desc(1, 24, 20, 20, 32, 3, 1, 1), 9),      # cin % 16 (this backend)
        (O.conv_desc(1, 64, 20, 20, 60, 1, 1, 0), 1),      # 1x1 oc % 8
        (O.conv_desc(1, 64, 20, 20, 64, 3, 1, 0), 9),      # pad 0
        (O.conv_desc(1, 64, 20, 20, 64, 5, 1, 2), 9),      # 5x5
        (O.conv_desc(1, 64, 20, 20, 64, 3, 1, 1, groups=2), 9),
    ]
    for d, kk in bad:
        assert not K.can_use_conv_int8(d, kk)


def test_conv_tile_override_accepts_only_instantiated_tiles():
    for jn, pw, ksw in [(1, 1, False), (2, 4, False), (8, 1, False), (4, 1, True), (8, 1, True)]:
        K.set_conv_tile(jn, pw, ksw)
    try:
        for jn, pw, ksw in [(3, 1, False), (8, 4, False), (1, 8, False), (2, 2, True), (16, 1, False)]:
            with pytest.raises(RuntimeError, match="no kernel instance"):
                K.set_conv_tile(jn, pw, ksw)
    finally:
        K.set_conv_tile(0, 0, False)


def _fastdiv(n: np.ndarray, d: int) -> np.ndarray:
    """The kernels' launch-constant division (kernels.h FastDiv) in uint64 arithmetic."""
    l = 0
    while (1 << l) < d:
        l += 1
    mul = ((1 << 32) * ((1 << l) - d)) // d + 1
    hi = (n.astype(np.uint64) * np.uint64(mul)) >> np.uint64(32)
    return (hi + n.astype(np.uint64)) >> np.uint64(l)


def test_fastdiv_is_exact_division_below_2_31():
    rng = np.random.default_rng(5)
    divisors = [1, 2, 3, 5, 7, 10, 20, 40, 80, 100, 160, 400, 1600, 6400, 25600, 102400, 2100, 144]
    divisors += [int(v) for v in rng.integers(1, 1 << 20, 40)]
    for d in divisors:
        n = np.concatenate([rng.integers(0, 1 << 31, 20000, dtype=np.int64),
                            np.arange(0, 4096, dtype=np.int64) * d + (d - 1),
                            np.arange((1 << 31) - 4096, 1 << 31, dtype=np.int64)])
        np.testing.assert_array_equal(_fastdiv(n, d), n // d)


def test_tensor_view_layout_matches_header():
    """AexrtHipTensorView: data, n_stride, c_stride, amax_stripes, amax_slots, amax_stripe_stride."""
    tv = _lib.TensorView
    assert ctypes.sizeof(tv) == 40
    offs = {name: getattr(tv, name).offset for name, _ in tv._fields_}
    assert offs == {"data": 0, "n_stride": 8, "c_stride": 16, "amax_stripes": 20, "amax_slots": 24,
                    "amax_stripe_stride": 32}
    hdr = (Path(__file__).resolve().parents[1] / "include" / "aexrt_hip.h").read_text()
    body = hdr[hdr.index("typedef struct AexrtHipTensorView"):]
    body = body[:body.index("} AexrtHipTensorView;")]
    names = re.findall(r"\b(\w+);", body)
    assert names == ["data", "n_stride", "c_stride", "amax_stripes", "amax_slots", "amax_stripe_stride"]
