"""GPU parity of the decode-layer pieces: device-synthesized FP8 tensors, the
batched FP8 GEMV entry point and the shared + routed expert sum
(E/compute.rs:1872-1946), against the oracle."""
import numpy as np
import pytest

import wohper_amd
from wohper_amd import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def exact_numerics(ctx):
    """These tests pin the kernels that follow the reference's summation
    order, bit for bit."""
    ctx.set_exact_numerics(True)
    yield


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_fp8_synthetic_store_and_batched_gemv(ctx, oracle):
    rows, cols = 1024, 2048
    scales = wl.fp8_block_scales(7, rows, cols)
    t = ctx.store_fp8_synthetic(rows, cols, 11, wl.fp8_stream(0, 3), scales)
    w = wl.synth_fp8_host(ctx.lib, 11, wl.fp8_stream(0, 3), rows, cols)
    assert not np.any((w & 0x7F) == 0x7F)
    fp8, _, _, _ = oracle.luts()
    assert np.array_equal(bits(ctx.dequant(t, rows, cols)), bits(fp8[w]))
    rng = np.random.default_rng(3)
    xs = rng.standard_normal((3, cols)).astype(np.float32)
    x_dev = ctx.device_alloc(xs.nbytes)
    y_dev = ctx.device_alloc(3 * rows * 4)
    ctx.to_device(x_dev, xs)
    ranges = ((0, 1024), (128, 512), (3, 77))
    ctx.fp8_gemv_batch_async([(t, r0, r1, x_dev + i * cols * 4, y_dev + i * rows * 4)
                              for i, (r0, r1) in enumerate(ranges)])
    ctx.synchronize()
    ys = np.empty((3, rows), np.float32)
    ctx.from_device(ys, y_dev)
    for i, (r0, r1) in enumerate(ranges):
        want = oracle.fp8_gemv(w, rows, cols, scales, rows // 128, cols // 128, xs[i], r0, r1)
        assert np.array_equal(bits(ys[i, :r1 - r0]), bits(want)), (r0, r1)
    # wo_a-style row groups with their own inputs (one merged launch)
    xg = rng.standard_normal((4, cols)).astype(np.float32)
    xg_dev = ctx.device_alloc(xg.nbytes)
    ctx.to_device(xg_dev, xg)
    ctx.fp8_gemv_batch_async([(t, 256 * g, 256 * (g + 1), xg_dev + g * cols * 4, y_dev + g * 256 * 4)
                              for g in range(4)])
    ctx.synchronize()
    yg = np.empty(rows, np.float32)
    ctx.from_device(yg, y_dev)
    for g in range(4):
        want = oracle.fp8_gemv(w, rows, cols, scales, rows // 128, cols // 128, xg[g], 256 * g, 256 * (g + 1))
        assert np.array_equal(bits(yg[256 * g:256 * (g + 1)]), bits(want)), g
    ctx.device_free(xg_dev)
    # several inputs through one row range, device pointers
    xm = rng.standard_normal((5, cols + 4)).astype(np.float32)
    xm_dev = ctx.device_alloc(xm.nbytes)
    ym_dev = ctx.device_alloc(5 * 700 * 4)
    ctx.to_device(xm_dev, xm)
    ctx.fp8_gemv_multi_async(t, 100, 700, xm_dev, 5, cols + 4, ym_dev, 700)
    ctx.synchronize()
    ym = np.empty((5, 700), np.float32)
    ctx.from_device(ym, ym_dev)
    for i in range(5):
        want = oracle.fp8_gemv(w, rows, cols, scales, rows // 128, cols // 128, xm[i, :cols], 100, 700)
        assert np.array_equal(bits(ym[i, :600]), bits(want)), i
    ctx.device_free(xm_dev)
    ctx.device_free(ym_dev)
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.fp8_gemv_batch_async([(t, 0, rows + 1, x_dev, y_dev)])
    assert e.value.name == "InvalidShape"
    ctx.device_free(x_dev)
    ctx.device_free(y_dev)


@pytest.mark.parametrize("n_routed", [6, 1, 0])
def test_shared_plus_routed_bit_exact(ctx, oracle, n_routed):
    seed = 4
    idx, w, x = wl.moe_token_case(seed)
    routes = [(5, int(e), float(wt)) for e, wt in zip(idx[:n_routed], w[:n_routed])]
    for _, e, _ in routes:
        ctx.store_expert_synthetic(5, e, wl.HIDDEN, wl.INTER, seed)
    shared = (5, wl.N_ROUTED)
    ctx.store_expert_synthetic(shared[0], shared[1], wl.HIDDEN, wl.INTER, seed)
    got = ctx.routed_and_shared_experts(routes, shared, x)
    sh = oracle.fp4_expert_forward(*wl.synth_expert_host(ctx.lib, seed, *shared), x)
    if n_routed:
        outs = np.stack([oracle.fp4_expert_forward(*wl.synth_expert_host(ctx.lib, seed, 5, e), x)
                         for _, e, _ in routes])
        want = sh + oracle.routed_combine(outs, [wt for _, _, wt in routes])
    else:
        want = sh
    assert np.array_equal(bits(got), bits(want.astype(np.float32)))
