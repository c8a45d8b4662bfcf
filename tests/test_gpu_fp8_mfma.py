"""GPU parity of the multi-input FP8 GEMV on bf16 MFMA (exact numerics off):
gemv_fp8_e4m3_ue8m0_rows_multi (E/compute.rs:6384-6577) and the grouped
batch wo_a projection (E/compute.rs:4599-4622).

Every output is checked against the oracle's restatement of the reference
kernel on the same input within max|diff| <= 1e-5 * ||w_row||_2 * ||x||_2.
One-hot inputs make each output a single exact product w * scale, which pins
the weight decode (all 256 codes, +-480 included) and the position mapping
bit for bit.  Rows of two +-1 weights against inputs with full 23-bit
significands have exact sums in any order, so they pin that the input split
loses no bits (a two-piece bf16 split would miss the lowest 7)."""
import numpy as np
import pytest

import wohper_amd
from wohper_amd import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def mfma_mode(ctx):
    ctx.set_exact_numerics(False)
    yield
    ctx.set_exact_numerics(True)


def dense(oracle, w, scales, row_group=128, col_group=128):
    fp8, _, _, _ = oracle.luts()
    return fp8[w].astype(np.float64) * np.repeat(np.repeat(scales.astype(np.float64), row_group, 0), col_group, 1)


def check(oracle, w, rows, cols, scales, xs, ys, r0=0, r1=None, wd=None):
    """ys[i] against the oracle GEMV of xs[i] over rows [r0, r1)."""
    r1 = rows if r1 is None else r1
    if wd is None:
        wd = dense(oracle, w, scales)
    norms = np.sqrt((wd[r0:r1] ** 2).sum(1))
    worst = 0.0
    for i, x in enumerate(xs):
        want = oracle.fp8_gemv(w, rows, cols, scales, scales.shape[0], scales.shape[1], x, r0, r1)
        tol = 1e-5 * norms * np.linalg.norm(x.astype(np.float64))
        diff = np.abs(ys[i].astype(np.float64) - want.astype(np.float64))
        assert np.all(diff <= tol), (i, float((diff / tol).max()))
        worst = max(worst, float((diff / tol).max()))
    return worst


def run_multi(ctx, t, xs, r0, r1, cols):
    n = xs.shape[0]
    xd = ctx.device_alloc(xs.nbytes)
    yd = ctx.device_alloc(n * (r1 - r0) * 4)
    ctx.to_device(xd, np.ascontiguousarray(xs, np.float32))
    ctx.fp8_gemv_multi_async(t, r0, r1, xd, n, cols, yd, r1 - r0)
    ys = np.empty((n, r1 - r0), np.float32)
    ctx.from_device(ys, yd)
    assert ctx.lib.wh_stream_status(ctx._h) == 0
    ctx.device_free(xd)
    ctx.device_free(yd)
    return ys


@pytest.mark.parametrize("rows,cols,n", [(4096, 4096, 16), (1024, 4096, 16), (512, 4096, 16), (4096, 8192, 16),
                                         (32768, 1024, 16), (4096, 4096, 5), (1024, 2048, 20)])
def test_fp8_mfma_decode_layer_shapes(ctx, oracle, rows, cols, n):
    """Every projection shape of a decode layer at batch 16, a partial token
    block (5 inputs) and two token blocks (20)."""
    case = wl.fp8_gemv_case(rows, cols, seed=rows + cols + n)
    t = ctx.store_fp8(case.w, rows, cols, case.scales, rows // 128, cols // 128, wohper_amd.SCALE_F32)
    xs = np.random.default_rng(n).standard_normal((n, cols)).astype(np.float32)
    ys = run_multi(ctx, t, xs, 0, rows, cols)
    worst = check(oracle, case.w, rows, cols, case.scales, xs, ys)
    print(f"{rows}x{cols} n={n}: worst |diff| / tolerance {worst:.3f}")
    ctx.release(t)


def test_fp8_mfma_row_range_ue8m0_and_host_slices(ctx, oracle):
    """UE8M0 scales, a row range starting inside a scale block, and the
    host-slice entry point."""
    rows, cols = 2048, 4096
    case = wl.fp8_gemv_case(rows, cols, seed=9, ue8m0_compatible=True)
    sbytes = (np.log2(case.scales).astype(np.int32) + 127).astype(np.uint8)
    t = ctx.store_fp8(case.w, rows, cols, sbytes, rows // 128, cols // 128, wohper_amd.SCALE_UE8M0)
    xs = np.random.default_rng(3).standard_normal((16, cols)).astype(np.float32)
    ys = run_multi(ctx, t, xs, 208, 1808, cols)
    check(oracle, case.w, rows, cols, case.scales, xs, ys, 208, 1808)
    ys2, vals = ctx.fp8_gemv_multi(t, xs[:7], 208, 1808)
    assert vals == 1600 * cols
    check(oracle, case.w, rows, cols, case.scales, xs[:7], ys2, 208, 1808)
    ctx.release(t)


def test_fp8_mfma_grouped_wo_a(ctx, oracle):
    """wo_a at batch 16: 8 row groups of 1024 rows, group g reading its own
    inputs, one call - equal to 8 per-group calls within tolerance."""
    rows, cols, gr, n = 8192, 4096, 1024, 16
    case = wl.fp8_gemv_case(rows, cols, seed=21)
    t = ctx.store_fp8(case.w, rows, cols, case.scales, rows // 128, cols // 128, wohper_amd.SCALE_F32)
    xs = np.random.default_rng(4).standard_normal((n, 8 * cols)).astype(np.float32)  # [pos][group][cols]
    xd = ctx.device_alloc(xs.nbytes)
    yd = ctx.device_alloc(n * rows * 4)
    ctx.to_device(xd, xs)
    ctx.fp8_gemv_multi_groups_async(t, 0, rows, gr, xd, cols, n, 8 * cols, yd, rows)
    ys = np.empty((n, rows), np.float32)
    ctx.from_device(ys, yd)
    wd = dense(oracle, case.w, case.scales)
    for g in range(8):
        check(oracle, case.w, rows, cols, case.scales, xs[:, g * cols:(g + 1) * cols], ys[:, g * gr:(g + 1) * gr],
              g * gr, (g + 1) * gr, wd)
    ctx.device_free(xd)
    ctx.device_free(yd)
    ctx.release(t)


@pytest.mark.parametrize("special", [False, True])
def test_fp8_mfma_one_hot_exact(ctx, oracle, special):
    """One-hot inputs: output i of row r is the single product w[r, k_i] *
    scale, so every weight code (the reference's +-480 for 0x7F/0xFF when
    present) and every column position must come out exactly."""
    rows, cols, n = 256, 1024, 16
    rng = np.random.default_rng(17)
    w = rng.integers(0, 256, (rows, cols)).astype(np.uint8)
    if not special:
        w[(w & 0x7F) == 0x7F] = 0x42
    else:
        w[::5, ::7] = 0x7F
        w[2::5, 3::7] = 0xFF
    w[0, :256] = np.arange(256, dtype=np.uint8) if special else np.where((np.arange(256) & 0x7F) == 0x7F, 0x42,
                                                                         np.arange(256)).astype(np.uint8)
    s = np.exp2(rng.integers(-6, 3, (rows // 128, cols // 128))).astype(np.float32)
    t = ctx.store_fp8(w, rows, cols, s, rows // 128, cols // 128, wohper_amd.SCALE_F32)
    for start in range(0, cols, n):
        ks = np.arange(start, start + n)
        xs = np.zeros((n, cols), np.float32)
        xs[np.arange(n), ks] = 1.0
        ys = run_multi(ctx, t, xs, 0, rows, cols)
        fp8, _, _, _ = oracle.luts()
        want = (fp8[w[:, ks]] * s[:, ks // 128].repeat(128, 0)).T.astype(np.float32)
        assert np.array_equal(ys, want), (start, int(np.count_nonzero(ys != want)))
    ctx.release(t)


def test_fp8_mfma_threshold_keeps_exact_below(ctx, oracle):
    """Below the MFMA threshold each input runs the single-input GEMV: the
    order-free one (within tolerance) with exact numerics off, the reference
    order (bit for bit) with them on."""
    rows, cols = 512, 2048
    case = wl.fp8_gemv_case(rows, cols, seed=2)
    t = ctx.store_fp8(case.w, rows, cols, case.scales, rows // 128, cols // 128, wohper_amd.SCALE_F32)
    xs = np.random.default_rng(8).standard_normal((3, cols)).astype(np.float32)
    ys = run_multi(ctx, t, xs, 0, rows, cols)
    check(oracle, case.w, rows, cols, case.scales, xs, ys)
    ctx.set_exact_numerics(True)
    ys = run_multi(ctx, t, xs, 0, rows, cols)
    for i in range(3):
        want = oracle.fp8_gemv(case.w, rows, cols, case.scales, rows // 128, cols // 128, xs[i])
        assert np.array_equal(ys[i].view(np.uint32), want.view(np.uint32))
    ctx.set_exact_numerics(False)
    ctx.set_fp8_mfma_min(2)
    try:
        ys = run_multi(ctx, t, xs, 0, rows, cols)
        check(oracle, case.w, rows, cols, case.scales, xs, ys)
    finally:
        ctx.set_fp8_mfma_min(4)
    ctx.release(t)


def test_fp8_mfma_full_precision_inputs_exact(ctx, oracle):
    """Each row holds two weights of +-1 (codes 0x38 / 0xB8), unit scales,
    and the inputs are integers below 2^23 times 2^-20: every sum of two
    products is exact in f32, so the MFMA path must equal the reference
    kernel bit for bit whatever its order."""
    rows, cols, n = 512, 2048, 16
    rng = np.random.default_rng(23)
    w = np.zeros((rows, cols), np.uint8)
    for r in range(rows):
        c0, c1 = rng.choice(cols, 2, replace=False) if r % 2 else (rng.integers(0, 64) * 2, rng.integers(0, 64) * 2 + 1)
        w[r, c0] = rng.choice([0x38, 0xB8])
        w[r, c1] = rng.choice([0x38, 0xB8])
    s = np.ones((rows // 128, cols // 128), np.float32)
    t = ctx.store_fp8(w, rows, cols, s, rows // 128, cols // 128, wohper_amd.SCALE_F32)
    xs = (rng.integers(1 << 22, 1 << 23, (n, cols)) * rng.choice([-1, 1], (n, cols))).astype(np.float64)
    xs = (xs * 2.0 ** -20).astype(np.float32)
    ys = run_multi(ctx, t, xs, 0, rows, cols)
    for i in range(n):
        want = oracle.fp8_gemv(w, rows, cols, s, rows // 128, cols // 128, xs[i])
        assert np.array_equal(ys[i].view(np.uint32), want.view(np.uint32)), (i, int(np.count_nonzero(ys[i] != want)))
    ctx.release(t)


@pytest.mark.parametrize("exact", [False, True])
def test_pair_equals_two_multi_calls(ctx, oracle, exact):
    """wq_a (1024 x 4096) and wkv (512 x 4096) on the same 16 inputs through
    wh_fp8_gemv_multi_pair_async (one launch on the MFMA path): bit-identical
    to two wh_fp8_gemv_multi_async calls, and within tolerance of the oracle
    (bit-exact with exact numerics, where the pair is two launches)."""
    rng = np.random.default_rng(71)
    n, cols = 16, 4096
    shapes = [(1024, 3), (512, 4)]
    ts, cases = [], []
    for rows, seed in shapes:
        w = rng.integers(0, 256, (rows, cols), dtype=np.uint8)
        s = rng.uniform(0.5, 2.0, (rows // 128, cols // 128)).astype(np.float32)
        ts.append(ctx.store_fp8(w, rows, cols, s, rows // 128, cols // 128, wohper_amd.SCALE_F32))
        cases.append((w, rows, s))
    xs = rng.standard_normal((n, cols)).astype(np.float32)
    ctx.set_exact_numerics(exact)
    xd = ctx.device_alloc(xs.nbytes)
    y0, y1 = ctx.device_alloc(n * 1024 * 4), ctx.device_alloc(n * 512 * 4)
    ctx.to_device(xd, xs)
    ctx.fp8_gemv_multi_pair_async(ts[0], 0, 1024, y0, 1024, ts[1], 0, 512, y1, 512, xd, n, cols)
    got = [np.empty((n, 1024), np.float32), np.empty((n, 512), np.float32)]
    ctx.from_device(got[0], y0)
    ctx.from_device(got[1], y1)
    assert ctx.lib.wh_stream_status(ctx._h) == 0
    for d in (xd, y0, y1):
        ctx.device_free(d)
    for (w, rows, s), t, g in zip(cases, ts, got):
        sep = run_multi(ctx, t, xs, 0, rows, cols)
        assert np.array_equal(g.view(np.uint32), sep.view(np.uint32)), rows
        if exact:
            for i in range(n):
                want = oracle.fp8_gemv(w, rows, cols, s, s.shape[0], s.shape[1], xs[i], 0, rows)
                assert np.array_equal(g[i].view(np.uint32), want.view(np.uint32)), (rows, i)
        else:
            check(oracle, w, rows, cols, s, xs, g)
    for t in ts:
        ctx.release(t)
