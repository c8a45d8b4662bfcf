"""GPU parity of the FP8 GEMV and FP4 matvec entry points with the oracle's
restatement of the reference AVX2 kernels: bit-exact on the fast paths and
the generic (odd-shape) paths, plus the BASELINE tolerance written out."""
import json
from pathlib import Path

import numpy as np
import pytest

import wohper_amd
from wohper_amd import workloads as wl
from conftest import lcg_bytes, lcg_f32

pytestmark = pytest.mark.gpu
KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def tolerance_ok(y, ref, dense_rows_norm, x):
    """max |diff| <= 1e-5 * ||w_row||_2 * ||x||_2 (fp32 accumulation)."""
    return np.all(np.abs(y.astype(np.float64) - ref) <= 1e-5 * dense_rows_norm * np.linalg.norm(x.astype(np.float64)))


@pytest.mark.parametrize("ue8m0", [False, True])
def test_fp8_gemv_4096_bit_exact(ctx, oracle, ue8m0):
    case = wl.fp8_gemv_case(4096, 4096, seed=0, ue8m0_compatible=ue8m0)
    if ue8m0:
        sbytes = (np.log2(case.scales).astype(np.int32) + 127).astype(np.uint8)
        t = ctx.store_fp8(case.w, 4096, 4096, sbytes, 32, 32, wohper_amd.SCALE_UE8M0)
    else:
        t = ctx.store_fp8(case.w, 4096, 4096, case.scales, 32, 32, wohper_amd.SCALE_F32)
    y, vals = ctx.fp8_gemv(t, case.x, 4096)
    want = oracle.fp8_gemv(case.w, 4096, 4096, case.scales, 32, 32, case.x)
    assert vals == 4096 * 4096
    assert np.array_equal(bits(y), bits(want))
    fp8, _, _, _ = oracle.luts()
    dense_norm = np.sqrt(((fp8[case.w].astype(np.float64) *
                           np.repeat(np.repeat(case.scales, 128, 0), 128, 1)) ** 2).sum(1))
    ref = (fp8[case.w].astype(np.float64) * np.repeat(np.repeat(case.scales, 128, 0), 128, 1)) @ case.x.astype(np.float64)
    assert tolerance_ok(y, ref, dense_norm, case.x)
    ctx.release(t)


@pytest.mark.parametrize("rows,cols", [(1024, 1024), (256, 8192), (128, 3072), (512, 2048)])
def test_fp8_decode_layer_widths_bit_exact(ctx, oracle, rows, cols):
    """Every split-K width of the decode layer's projections (8, 16, 32 and
    64 groups of 128 per row) plus a width that takes the runtime loop."""
    case = wl.fp8_gemv_case(rows, cols, seed=cols)
    t = ctx.store_fp8(case.w, rows, cols, case.scales, rows // 128, cols // 128, wohper_amd.SCALE_F32)
    y, _ = ctx.fp8_gemv(t, case.x, rows)
    want = oracle.fp8_gemv(case.w, rows, cols, case.scales, rows // 128, cols // 128, case.x)
    assert np.array_equal(bits(y), bits(want))
    ctx.release(t)


def test_fp8_row_ranges_and_multi(ctx, oracle):
    """wo_a-style row groups (E/compute.rs:4244-4258) and the T2 multi-input GEMV."""
    rng = np.random.default_rng(5)
    rows, cols = 1024, 2048
    case = wl.fp8_gemv_case(rows, cols, seed=5)
    t = ctx.store_fp8(case.w, rows, cols, case.scales, rows // 128, cols // 128, wohper_amd.SCALE_F32)
    for r0, r1 in ((0, 128), (128, 512), (896, 1024), (3, 77)):
        y, vals = ctx.fp8_gemv(t, case.x, r1 - r0, r0, r1)
        want = oracle.fp8_gemv(case.w, rows, cols, case.scales, rows // 128, cols // 128, case.x, r0, r1)
        assert np.array_equal(bits(y), bits(want)) and vals == (r1 - r0) * cols
    xs = rng.standard_normal((5, cols)).astype(np.float32)
    ys, _ = ctx.fp8_gemv_multi(t, xs, 100, 900)
    for i in range(5):
        single, _ = ctx.fp8_gemv(t, xs[i], 800, 100, 900)
        assert np.array_equal(bits(ys[i]), bits(single))
        want = oracle.fp8_gemv(case.w, rows, cols, case.scales, rows // 128, cols // 128, xs[i], 100, 900)
        assert np.array_equal(bits(ys[i]), bits(want))
    ctx.release(t)


def test_fp8_special_codes_and_generic_tail(ctx, oracle):
    # 0x7F / 0xFF (+-480 in the reference) on the fast path
    rng = np.random.default_rng(6)
    w = rng.integers(0, 256, (256, 512)).astype(np.uint8)
    w[::7, ::5] = 0x7F
    w[1::7, 2::5] = 0xFF
    s = np.exp2(rng.integers(-9, -5, (2, 4))).astype(np.float32)
    x = rng.standard_normal(512).astype(np.float32)
    t = ctx.store_fp8(w, 256, 512, s, 2, 4, wohper_amd.SCALE_F32)
    y, _ = ctx.fp8_gemv(t, x, 256)
    assert np.array_equal(bits(y), bits(oracle.fp8_gemv(w, 256, 512, s, 2, 4, x)))
    ctx.release(t)
    # the reference's own tail case: cols 200 in groups of 50 (compute.rs:7416-7435)
    k = KATS["fp8_dot_row_tail"]
    rows = 3
    w = np.array(lcg_bytes(k["weight_seed"], rows * k["cols"]), np.uint8).reshape(rows, k["cols"])
    x = lcg_f32(k["input_seed"], k["cols"])
    sb = (np.arange(k["groups"]) + k["scale_base"]).astype(np.uint8).reshape(1, -1)
    t = ctx.store_fp8(w, rows, k["cols"], sb, 1, k["groups"], wohper_amd.SCALE_UE8M0)
    y, _ = ctx.fp8_gemv(t, x, rows)
    want = oracle.fp8_gemv(w, rows, k["cols"], oracle.decode_ue8m0(sb), 1, k["groups"], x)
    assert np.array_equal(bits(y), bits(want))
    ctx.release(t)


def test_fp8_nonfinite_and_shape_errors(ctx):
    w = np.full((128, 128), 0x38, np.uint8)
    t = ctx.store_fp8(w, 128, 128, np.array([[255]], np.uint8), 1, 1, wohper_amd.SCALE_UE8M0)
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.fp8_gemv(t, np.ones(128, np.float32), 128)
    assert e.value.name == "NonFiniteOutput"
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.fp8_gemv(t, np.ones(64, np.float32), 128)
    assert e.value.name == "InputTooSmall"
    ctx.release(t)
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.store_fp8(w, 128, 128, np.ones((3, 1), np.float32), 3, 1, wohper_amd.SCALE_F32)
    assert e.value.name == "InvalidShape"


@pytest.mark.parametrize("rows,cols", [(2048, 4096), (4096, 2048), (64, 768)])
def test_fp4_matvec_bit_exact(ctx, oracle, rows, cols):
    rng = np.random.default_rng(rows * 3 + cols)
    packed = rng.integers(0, 256, (rows, cols // 2)).astype(np.uint8)
    scales = rng.integers(110, 135, (rows, cols // 32)).astype(np.uint8)
    x = (rng.standard_normal(cols) * rng.uniform(0.01, 100)).astype(np.float32)
    t = ctx.store_fp4(packed, scales, rows, cols, cols // 32)
    y = ctx.fp4_matvec(t, x, rows)
    want = oracle.fp4_matvec(packed, scales, rows, cols, cols // 32, x)
    assert np.array_equal(bits(y), bits(want))
    ctx.release(t)


@pytest.mark.parametrize("rows,cols,scale_cols", [(3, 32, 4), (2, 4, 1), (5, 96, 3), (4, 7, 7), (7, 130, 5)])
def test_fp4_matvec_generic_shapes_bit_exact(ctx, oracle, rows, cols, scale_cols):
    rng = np.random.default_rng(cols)
    packed = rng.integers(0, 256, (rows, (cols + 1) // 2)).astype(np.uint8)
    scales = rng.integers(115, 130, (rows, scale_cols)).astype(np.uint8)
    x = rng.standard_normal(cols).astype(np.float32)
    t = ctx.store_fp4(packed, scales, rows, cols, scale_cols)
    y = ctx.fp4_matvec(t, x, rows)
    want = oracle.fp4_matvec(packed, scales, rows, cols, scale_cols, x)
    assert np.array_equal(bits(y), bits(want))
    ctx.release(t)


def test_fp4_known_answer_and_slice_api(ctx):
    k = KATS["fp4_low_nibble_first"]
    spec = wohper_amd.Fp4Matvec(np.array(k["packed"], np.uint8), np.array(k["scales"], np.uint8),
                                k["rows"], k["cols"], k["scale_cols"])
    out = np.zeros(2, np.float32)
    wohper_amd.fp4_e2m1_ue8m0_matvec_scalar(spec, np.array(k["input"], np.float32), out, ctx=ctx)
    assert np.all(np.abs(out - np.array(k["expected"])) < k["tol"])


def test_fp4_nonfinite_output(ctx):
    packed = np.full((32, 256), 0x22, np.uint8)
    scales = np.full((32, 16), 127, np.uint8)
    scales[5, 3] = 255
    t = ctx.store_fp4(packed, scales, 32, 512, 16)
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.fp4_matvec(t, np.ones(512, np.float32), 32)
    assert e.value.name == "NonFiniteOutput"
    ctx.release(t)
