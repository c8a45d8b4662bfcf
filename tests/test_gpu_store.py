"""GPU checks of the weight store's memory reuse and of the FP8 launch
grouping of wh_fp8_gemv_batch_async.

The reference streams each expert block from disk per token and holds no
device memory (E/direct_io.rs:575-681); the HBM store replaces that, so a
long-lived engine that replaces experts, or calls the host-slice entry points
(each stores and releases its weight), must reuse released HBM rather than
grow."""
import numpy as np
import pytest

import wohper_amd
from wohper_amd import workloads as wl

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_replacing_an_expert_keeps_usage_flat(ctx, oracle):
    layer, expert, hidden, inter = 70, 5, 1024, 512
    ctx.store_expert_synthetic(layer, expert, hidden, inter, 1)
    used0, tensors0, experts0 = ctx.usage()
    for seed in range(2, 1002):
        ctx.store_expert_synthetic(layer, expert, hidden, inter, seed)
    assert ctx.usage() == (used0, tensors0, experts0)
    # the last replacement is the one that computes
    ctx.set_exact_numerics(True)
    x = np.random.default_rng(3).standard_normal(hidden).astype(np.float32)
    got = ctx.routed_experts([(layer, expert, 1.0)], x)
    want = oracle.fp4_expert_forward(*wl.synth_expert_host(ctx.lib, 1001, layer, expert, hidden, inter), x)
    assert np.array_equal(bits(got), bits(want))


def test_slice_api_reuses_released_memory(ctx, oracle):
    """gemv_fp8_e4m3_ue8m0_tensorwise stores and releases its weight per call."""
    case = wl.fp8_gemv_case(1024, 1024, seed=9, ue8m0_compatible=True)
    sc8 = (np.log2(case.scales).astype(np.int32) + 127).astype(np.uint8)
    y = np.empty(1024, np.float32)
    wohper_amd.gemv_fp8_e4m3_ue8m0_tensorwise(case.w, 1024, 1024, sc8, 8, 8, case.x, y, ctx=ctx)
    used0 = ctx.usage()
    for _ in range(200):
        wohper_amd.gemv_fp8_e4m3_ue8m0_tensorwise(case.w, 1024, 1024, sc8, 8, 8, case.x, y, ctx=ctx)
    assert ctx.usage() == used0
    want = oracle.fp8_gemv(case.w, 1024, 1024, case.scales, 8, 8, case.x, 0, 1024)
    assert np.array_equal(bits(y), bits(want))


def test_release_then_store_reuses_and_stays_correct(ctx, oracle):
    """Interleaved stores and releases of different sizes: live bytes return
    to their starting value, and tensors stored into reused ranges compute
    bit-exactly."""
    used0 = ctx.usage()[0]
    rng = np.random.default_rng(4)
    handles = []
    for i in range(40):
        rows = 128 * int(rng.integers(1, 9))
        t = ctx.store_fp8_synthetic(rows, 1024, 100 + i, wl.fp8_stream(1, i), wl.fp8_block_scales(i, rows, 1024))
        handles.append((t, rows, i))
        if i % 3 == 2:  # release an older one, leaving holes
            ctx.release(handles.pop(int(rng.integers(0, len(handles))))[0])
    x = rng.standard_normal(1024).astype(np.float32)
    for t, rows, i in handles[-4:]:
        w = wl.synth_fp8_host(ctx.lib, 100 + i, wl.fp8_stream(1, i), rows, 1024)
        got, _ = ctx.fp8_gemv(t, x, rows)
        want = oracle.fp8_gemv(w, rows, 1024, wl.fp8_block_scales(i, rows, 1024), rows // 128, 8, x, 0, rows)
        assert np.array_equal(bits(got), bits(want)), i
    for t, _, _ in handles:
        ctx.release(t)
    assert ctx.usage()[0] == used0


def test_fp8_batch_keeps_order_and_separate_inputs(ctx, oracle):
    """Row-group descriptors are launched as one only when it cannot change
    a result: an output that overlaps a later group's input keeps its own
    launch (in-order semantics), and inputs in separate allocations (a lower
    address, uneven steps) run correctly."""
    rows = cols = 1024
    scales = wl.fp8_block_scales(21, rows, cols)
    t = ctx.store_fp8_synthetic(rows, cols, 21, wl.fp8_stream(2, 0), scales)
    w = wl.synth_fp8_host(ctx.lib, 21, wl.fp8_stream(2, 0), rows, cols)
    rng = np.random.default_rng(21)

    def ref(xv, r0, r1):
        return oracle.fp8_gemv(w, rows, cols, scales, rows // 128, cols // 128, xv, r0, r1)

    # group 0 writes floats [2048, 2304) of buf, which group 1 reads (its
    # input is floats [1536, 2560)); group 1 writes [2304, 2560)
    buf = rng.standard_normal(8192).astype(np.float32)
    b_dev = ctx.device_alloc(buf.nbytes)
    ctx.to_device(b_dev, buf)
    ctx.fp8_gemv_batch_async([(t, 0, 256, b_dev, b_dev + 2048 * 4), (t, 256, 512, b_dev + 1536 * 4, b_dev + 2304 * 4)])
    ctx.synchronize()
    got = np.empty_like(buf)
    ctx.from_device(got, b_dev)
    want = buf.copy()
    want[2048:2304] = ref(want[0:1024], 0, 256)
    want[2304:2560] = ref(want[1536:2560], 256, 512)
    assert np.array_equal(bits(got), bits(want))
    ctx.device_free(b_dev)

    # inputs in separate allocations, the second at a lower address than the
    # first or not: every group must read its own input
    xs = rng.standard_normal((4, cols)).astype(np.float32)
    x_dev = [ctx.device_alloc(cols * 4) for _ in range(4)]
    for i in range(4):
        ctx.to_device(x_dev[i], xs[i])
    order = sorted(range(4), key=lambda i: -x_dev[i])  # descending addresses
    y_dev = ctx.device_alloc(rows * 4)
    descs = [(t, 256 * g, 256 * (g + 1), x_dev[order[g]], y_dev + g * 256 * 4) for g in range(4)]
    ctx.fp8_gemv_batch_async(descs)
    ctx.synchronize()
    y = np.empty(rows, np.float32)
    ctx.from_device(y, y_dev)
    for g in range(4):
        assert np.array_equal(bits(y[256 * g:256 * (g + 1)]), bits(ref(xs[order[g]], 256 * g, 256 * (g + 1)))), g
    # unaligned inputs of the lane-layout kernels are refused before any launch
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.fp8_gemv_batch_async([(t, 0, 256, x_dev[0] + 4, y_dev)])
    assert e.value.name == "InvalidArgument"
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.fp8_gemv_async(t, 0, 256, x_dev[0] + 8, y_dev)
    assert e.value.name == "InvalidArgument"
    for p in x_dev + [y_dev]:
        ctx.device_free(p)
    ctx.release(t)
