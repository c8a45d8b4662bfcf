"""GPU check of the allocation-free routed-expert entry point
(wh_routed_and_shared_experts_noalloc_async, no counterpart in the reference):
through the C ABI it must give the same bits as
wh_routed_and_shared_experts_async, whose kernels it shares, on two calls in a
row (the second with a smaller input), in both numerics modes, and refuse a
call whose working memory exceeds its fixed array before queueing anything."""
import numpy as np
import pytest

import wohper_amd
from wohper_amd import workloads as wl

pytestmark = pytest.mark.gpu

LAYER = 61
SHARED = (62, 0)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def experts(ctx):
    seed = 41
    ids = [3, 17, 40, 77, 128, 200, 255]
    for e in ids:
        ctx.store_expert_synthetic(LAYER, e, wl.HIDDEN, wl.INTER, seed)
    ctx.store_expert_synthetic(SHARED[0], SHARED[1], wl.HIDDEN, wl.INTER, seed)
    return ids


def _run_both(ctx, routes, x, bf16):
    """The allocating entry point, then the allocation-free one, on the same
    device input; returns both outputs."""
    n_tokens = x.shape[0]
    if bf16:
        host = wl.bf16_bits(x)
    else:
        host = np.ascontiguousarray(x, np.float32)
    x_dev = ctx.device_alloc(host.nbytes)
    ya_dev = ctx.device_alloc(n_tokens * wl.HIDDEN * 4)
    yb_dev = ctx.device_alloc(n_tokens * wl.HIDDEN * 4)
    try:
        ctx.to_device(x_dev, host)
        ctx.routed_and_shared_experts_async(routes, SHARED, x_dev, bf16, n_tokens, ya_dev)
        ctx.synchronize()
        ctx.routed_and_shared_experts_noalloc_async(routes, SHARED, x_dev, bf16, n_tokens, yb_dev)
        ctx.synchronize()
        ya = np.empty((n_tokens, wl.HIDDEN), np.float32)
        yb = np.empty((n_tokens, wl.HIDDEN), np.float32)
        ctx.from_device(ya, ya_dev)
        ctx.from_device(yb, yb_dev)
    finally:
        for p in (x_dev, ya_dev, yb_dev):
            ctx.device_free(p)
    return ya, yb


@pytest.mark.parametrize("exact", [True, False])
def test_noalloc_matches_allocating_entry(ctx, experts, exact):
    ctx.set_exact_numerics(exact)
    try:
        rng = np.random.default_rng(5 if exact else 6)
        # call 1: 3 tokens x (6 routed + shared), bf16 input
        routes = [(LAYER, e, float(w)) for e, w in zip(experts[:6], rng.uniform(0.1, 1.0, 6))]
        x = rng.standard_normal((3, wl.HIDDEN)).astype(np.float32)
        ya, yb = _run_both(ctx, routes, x, True)
        assert np.all(np.isfinite(ya))
        assert np.array_equal(bits(ya), bits(yb))
        # call 2, smaller: 1 token x (2 routed + shared), f32 input; the
        # array still holds call 1's contents
        routes = [(LAYER, experts[6], 0.25), (LAYER, experts[1], 0.75)]
        x = rng.standard_normal((1, wl.HIDDEN)).astype(np.float32) * 2.0
        ya, yb = _run_both(ctx, routes, x, False)
        assert np.array_equal(bits(ya), bits(yb))
    finally:
        ctx.set_exact_numerics(True)


def test_noalloc_refuses_oversize_before_queueing(ctx, experts):
    routes = [(LAYER, e, 1.0) for e in experts[:6]]
    # 64 tokens x 7 experts x 4 x (4096 + 2048) bytes > the fixed array
    n_tokens = 64
    x_dev = ctx.device_alloc(n_tokens * wl.HIDDEN * 4)
    y_dev = ctx.device_alloc(n_tokens * wl.HIDDEN * 4)
    try:
        with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
            ctx.routed_and_shared_experts_noalloc_async(routes, SHARED, x_dev, False, n_tokens, y_dev)
        assert e.value.name == "ScratchTooSmall"
        ctx.synchronize()  # nothing was queued, no deferred status
    finally:
        ctx.device_free(x_dev)
        ctx.device_free(y_dev)
