"""GPU parity of the exact multi-input FP8 GEMV (k_fp8_gemv_multi: each
weight byte decoded once for every input, each input's dot in the
single-input kernel's order) against the oracle's restatement of
gemv_fp8_e4m3_ue8m0_rows_multi (E/compute.rs:6384-6577), bit for bit: the
decode layer's shapes at batch 16, partial input blocks (2, 5, 9, 20
inputs), unaligned row ranges, UE8M0 and f32 scales, the +-480 codes, the
pair entry point (wq_a + wkv on one input set) and row groups with their
own inputs (wo_a)."""
import numpy as np
import pytest

import wohper_amd
from parity_util import bits
from wohper_amd import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def exact(ctx):
    ctx.set_exact_numerics(True)
    yield


def _tensor(ctx, rows, cols, seed, ue8m0=False, special=False):
    case = wl.fp8_gemv_case(rows, cols, seed=seed, ue8m0_compatible=ue8m0)
    w = case.w.copy()
    if special:
        rng = np.random.default_rng(seed)
        w[rng.integers(0, rows, 64), rng.integers(0, cols, 64)] = 0x7F
        w[rng.integers(0, rows, 64), rng.integers(0, cols, 64)] = 0xFF
    if ue8m0:
        sb = (np.log2(case.scales).astype(np.int32) + 127).astype(np.uint8)
        t = ctx.store_fp8(w, rows, cols, sb, rows // 128, cols // 128, wohper_amd.SCALE_UE8M0)
    else:
        t = ctx.store_fp8(w, rows, cols, case.scales, rows // 128, cols // 128, wohper_amd.SCALE_F32)
    return t, w, case.scales


def _run(ctx, t, xs, r0, r1):
    n, cols = xs.shape
    xd, yd = ctx.device_alloc(xs.nbytes), ctx.device_alloc(n * (r1 - r0) * 4)
    ctx.to_device(xd, np.ascontiguousarray(xs))
    ctx.fp8_gemv_multi_async(t, r0, r1, xd, n, cols, yd, r1 - r0)
    ys = np.empty((n, r1 - r0), np.float32)
    ctx.synchronize()
    ctx.from_device(ys, yd)
    ctx.device_free(xd)
    ctx.device_free(yd)
    return ys


@pytest.mark.parametrize("rows,cols,n,r0,r1,ue8m0", [
    (4096, 4096, 16, 0, 4096, False), (32768, 1024, 16, 0, 32768, True), (4096, 8192, 16, 0, 4096, False),
    (1024, 2048, 5, 100, 900, True), (512, 4096, 9, 3, 509, False), (1024, 1024, 2, 0, 1024, True),
    (1024, 4096, 20, 64, 1024, False), (4096, 4096, 7, 0, 4096, True), (8192, 2048, 3, 128, 8064, False)])
def test_multi_exact_matches_rows_multi(ctx, oracle, rows, cols, n, r0, r1, ue8m0):
    t, w, scales = _tensor(ctx, rows, cols, rows + cols + n, ue8m0)
    xs = np.random.default_rng(n).standard_normal((n, cols)).astype(np.float32)
    ys = _run(ctx, t, xs, r0, r1)
    want = oracle.fp8_gemv_rows_multi(w, rows, cols, scales, rows // 128, cols // 128, xs, r0, r1)
    for i in range(n):
        assert np.array_equal(bits(ys[i]), bits(want[i])), (i, int(np.count_nonzero(bits(ys[i]) != bits(want[i]))))
    ctx.release(t)


def test_multi_exact_special_codes(ctx, oracle):
    rows, cols, n = 1024, 2048, 16
    t, w, scales = _tensor(ctx, rows, cols, 17, special=True)
    xs = np.random.default_rng(4).standard_normal((n, cols)).astype(np.float32)
    ys = _run(ctx, t, xs, 0, rows)
    want = oracle.fp8_gemv_rows_multi(w, rows, cols, scales, rows // 128, cols // 128, xs)
    assert np.array_equal(bits(ys), bits(want))
    ctx.release(t)


def test_multi_exact_pair_and_groups(ctx, oracle):
    """wq_a + wkv on one set of 16 inputs in one launch, and wo_a's 8 row
    groups of 1024 each on its own 16 inputs."""
    n = 16
    ta, wa, sa = _tensor(ctx, 1024, 4096, 31)
    tk, wk, sk = _tensor(ctx, 512, 4096, 32)
    xs = np.random.default_rng(8).standard_normal((n, 4096)).astype(np.float32)
    xd = ctx.device_alloc(xs.nbytes)
    ctx.to_device(xd, xs)
    ya, yk = ctx.device_alloc(n * 1024 * 4), ctx.device_alloc(n * 512 * 4)
    ctx.fp8_gemv_multi_pair_async(ta, 0, 1024, ya, 1024, tk, 0, 512, yk, 512, xd, n, 4096)
    ctx.synchronize()
    got_a, got_k = np.empty((n, 1024), np.float32), np.empty((n, 512), np.float32)
    ctx.from_device(got_a, ya)
    ctx.from_device(got_k, yk)
    assert np.array_equal(bits(got_a), bits(oracle.fp8_gemv_rows_multi(wa, 1024, 4096, sa, 8, 32, xs)))
    assert np.array_equal(bits(got_k), bits(oracle.fp8_gemv_rows_multi(wk, 512, 4096, sk, 4, 32, xs)))
    for p in (xd, ya, yk):
        ctx.device_free(p)
    # wo_a: 8 groups of 1024 rows, group g reads its own 16 inputs
    to, wo, so = _tensor(ctx, 8192, 4096, 33)
    xg = np.random.default_rng(9).standard_normal((n, 8, 4096)).astype(np.float32)
    xd, yd = ctx.device_alloc(xg.nbytes), ctx.device_alloc(n * 8192 * 4)
    ctx.to_device(xd, xg)
    ctx.fp8_gemv_multi_groups_async(to, 0, 8192, 1024, xd, 4096, n, 8 * 4096, yd, 8192)
    ctx.synchronize()
    got = np.empty((n, 8192), np.float32)
    ctx.from_device(got, yd)
    for g in range(8):
        want = oracle.fp8_gemv_rows_multi(wo, 8192, 4096, so, 64, 32, xg[:, g], 1024 * g, 1024 * (g + 1))
        assert np.array_equal(bits(got[:, 1024 * g:1024 * (g + 1)]), bits(want)), g
    ctx.device_free(xd)
    ctx.device_free(yd)
    for t in (ta, tk, to):
        ctx.release(t)
