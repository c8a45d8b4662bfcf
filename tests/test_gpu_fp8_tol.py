"""GPU parity of the order-free FP8 GEMV (exact numerics off, one input):
gemv_fp8_e4m3_ue8m0_tensorwise / _rows (E/compute.rs:6174-6321) within
max|diff| <= 1e-5 * ||w_row||_2 * ||x||_2 of the oracle's restatement of the
reference's AVX2 kernel, at every width of a decode layer's projections,
with f32 and UE8M0 scales, on a row range starting inside a scale block and
on row groups with their own input (wo_a).  One-hot inputs pin the weight
decode and the column mapping bit for bit (each output is one product);
tensors holding the reference's +-480 codes keep the exact kernel, bit for
bit."""
import numpy as np
import pytest

import wohper_amd
from parity_util import bits
from wohper_amd import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def free_order(ctx):
    ctx.set_exact_numerics(False)
    yield
    ctx.set_exact_numerics(True)


def _dense(oracle, w, scales):
    fp8, _, _, _ = oracle.luts()
    return fp8[w].astype(np.float64) * np.repeat(np.repeat(scales.astype(np.float64), 128, 0), 128, 1)


def _check(oracle, w, rows, cols, scales, x, y, r0=0, r1=None):
    r1 = rows if r1 is None else r1
    want = oracle.fp8_gemv(w, rows, cols, scales, rows // 128, cols // 128, x, r0, r1)
    norms = np.sqrt((_dense(oracle, w, scales)[r0:r1] ** 2).sum(1))
    tol = 1e-5 * norms * np.linalg.norm(x.astype(np.float64))
    diff = np.abs(y.astype(np.float64) - want.astype(np.float64))
    assert np.all(diff <= tol), float((diff / tol).max())
    return float((diff / tol).max())


def _store(ctx, case, rows, cols, ue8m0):
    if ue8m0:
        sb = (np.log2(case.scales).astype(np.int32) + 127).astype(np.uint8)
        return ctx.store_fp8(case.w, rows, cols, sb, rows // 128, cols // 128, wohper_amd.SCALE_UE8M0)
    return ctx.store_fp8(case.w, rows, cols, case.scales, rows // 128, cols // 128, wohper_amd.SCALE_F32)


@pytest.mark.parametrize("rows,cols,ue8m0", [(4096, 4096, False), (4096, 4096, True), (1024, 4096, False),
                                             (512, 4096, True), (32768, 1024, False), (4096, 8192, False),
                                             (2048, 2048, True), (8192, 4096, False)])
def test_fp8_tol_decode_layer_widths(ctx, oracle, rows, cols, ue8m0):
    case = wl.fp8_gemv_case(rows, cols, seed=rows + cols, ue8m0_compatible=ue8m0)
    t = _store(ctx, case, rows, cols, ue8m0)
    y, vals = ctx.fp8_gemv(t, case.x, rows)
    assert vals == rows * cols
    worst = _check(oracle, case.w, rows, cols, case.scales, case.x, y)
    print(f"{rows}x{cols} ue8m0={ue8m0}: worst |diff| / tolerance {worst:.3f}")
    ctx.release(t)


def test_fp8_tol_row_range(ctx, oracle):
    rows, cols = 2048, 4096
    case = wl.fp8_gemv_case(rows, cols, seed=11)
    t = _store(ctx, case, rows, cols, False)
    y, _ = ctx.fp8_gemv(t, case.x, 1600, 208, 1808)
    _check(oracle, case.w, rows, cols, case.scales, case.x, y, 208, 1808)
    ctx.release(t)


def test_fp8_tol_one_hot_exact(ctx, oracle):
    """x = e_k: every output is w[r, k] * scale exactly, for 64 columns k
    spread over every byte position of the resident chunks."""
    rows, cols = 512, 4096
    case = wl.fp8_gemv_case(rows, cols, seed=12)
    t = _store(ctx, case, rows, cols, False)
    fp8, _, _, _ = oracle.luts()
    for k in list(range(0, 128, 3)) + [1023, 1024, 2047, 2048 + 77, 4095]:
        x = np.zeros(cols, np.float32)
        x[k] = 1.0
        y, _ = ctx.fp8_gemv(t, x, rows)
        want = (fp8[case.w[:, k]] * np.repeat(case.scales[:, k // 128], 128)).astype(np.float32)
        assert np.array_equal(bits(y), bits(want)), k
    ctx.release(t)


def test_fp8_tol_special_codes_keep_exact(ctx, oracle):
    rows, cols = 1024, 4096
    case = wl.fp8_gemv_case(rows, cols, seed=13)
    w = case.w.copy()
    w[3, 100] = 0x7F
    w[700, 4000] = 0xFF
    t = ctx.store_fp8(w, rows, cols, case.scales, rows // 128, cols // 128, wohper_amd.SCALE_F32)
    y, _ = ctx.fp8_gemv(t, case.x, rows)
    assert np.array_equal(bits(y), bits(oracle.fp8_gemv(w, rows, cols, case.scales, rows // 128, cols // 128,
                                                         case.x)))
    ctx.release(t)


def test_fp8_tol_row_groups_own_inputs(ctx, oracle):
    """wo_a at batch 1: 8 groups of 1024 rows, group g on its own input."""
    rows, cols, gr = 8192, 4096, 1024
    case = wl.fp8_gemv_case(rows, cols, seed=14)
    t = _store(ctx, case, rows, cols, False)
    xs = np.random.default_rng(15).standard_normal((8, cols)).astype(np.float32)
    xd, yd = ctx.device_alloc(xs.nbytes), ctx.device_alloc(rows * 4)
    ctx.to_device(xd, xs)
    ctx.fp8_gemv_multi_groups_async(t, 0, rows, gr, xd, cols, 1, 8 * cols, yd, rows)
    y = np.empty(rows, np.float32)
    ctx.from_device(y, yd)
    for g in range(8):
        _check(oracle, case.w, rows, cols, case.scales, xs[g], y[g * gr:(g + 1) * gr], g * gr, (g + 1) * gr)
    ctx.device_free(xd)
    ctx.device_free(yd)
    ctx.release(t)
