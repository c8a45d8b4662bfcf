"""Captured launch sequences (wh_graph_*): a decode layer's FP8 projection set
and its shared + routed experts recorded once, replayed several times with
the program's own eager work and synchronizations between the replays; every
replay must equal the eager result bit for bit (the same kernels run), and
the eager result equals the oracle in exact numerics."""
import numpy as np
import pytest

import wohper_amd
from parity_util import bits
from wohper_amd import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def restore_numerics(ctx):
    yield
    ctx.set_exact_numerics(True)


def _layer_case(ctx, seed, layer):
    rng = np.random.default_rng(seed)
    hs = {}
    for i, (name, r, c, _) in enumerate(wl.DECODE_LAYER_FP8):
        hs[name] = ctx.store_fp8_synthetic(r, c, seed, wl.fp8_stream(layer, i), wl.fp8_block_scales(seed + i, r, c))
    idx, w, _ = wl.moe_token_case(seed)
    routes = [(layer, int(e), float(wt)) for e, wt in zip(idx, w)]
    for _, e, _ in routes:
        ctx.store_expert_synthetic(layer, e, wl.HIDDEN, wl.INTER, seed)
    ctx.store_expert_synthetic(layer, wl.N_ROUTED, wl.HIDDEN, wl.INTER, seed)
    vecs = {"x": 4096, "qlat": 1024, "oa": 8 * 4096, "ob": 8192}
    dev = {}
    for k, n in vecs.items():
        dev[k] = ctx.device_alloc(n * 4)
        ctx.to_device(dev[k], rng.standard_normal(n).astype(np.float32))
    ny = 1024 + 32768 + 512 + 8192 + 4096
    y = ctx.device_alloc(ny * 4)
    moe_x = ctx.device_alloc(wl.HIDDEN * 2)
    ctx.to_device(moe_x, wl.bf16_bits(rng.standard_normal(wl.HIDDEN).astype(np.float32)))
    moe_out = ctx.device_alloc(wl.HIDDEN * 4)
    o = {"wq_b": 1024, "wkv": 1024 + 32768, "wo_a": 1024 + 32768 + 512, "wo_b": 1024 + 32768 + 512 + 8192}
    descs = [(hs["wq_a"], 0, 1024, dev["x"], y), (hs["wkv"], 0, 512, dev["x"], y + o["wkv"] * 4),
             (hs["wq_b"], 0, 32768, dev["qlat"], y + o["wq_b"] * 4)]
    descs += [(hs["wo_a"], 1024 * g, 1024 * (g + 1), dev["oa"] + g * 4096 * 4, y + (o["wo_a"] + 1024 * g) * 4)
              for g in range(8)]
    descs += [(hs["wo_b"], 0, 4096, dev["ob"], y + o["wo_b"] * 4)]
    arr = ctx.route_array(routes)

    def step():
        ctx.fp8_gemv_batch_async(descs)
        ctx.routed_and_shared_experts_async(arr, (layer, wl.N_ROUTED), moe_x, True, 1, moe_out, n_routes=len(routes))

    def read():
        ctx.synchronize()
        a = np.empty(ny, np.float32)
        b = np.empty(wl.HIDDEN, np.float32)
        ctx.from_device(a, y)
        ctx.from_device(b, moe_out)
        return a, b

    def clear():
        ctx.to_device(y, np.full(ny, np.nan, np.float32))
        ctx.to_device(moe_out, np.full(wl.HIDDEN, np.nan, np.float32))

    def free():
        for p in list(dev.values()) + [y, moe_x, moe_out]:
            ctx.device_free(p)
        for h in hs.values():
            ctx.release(h)

    return step, read, clear, free


@pytest.mark.parametrize("exact", [True, False])
def test_graph_replays_equal_eager(ctx, exact):
    ctx.set_exact_numerics(exact)
    step, read, clear, free = _layer_case(ctx, 71, 31)
    clear()
    step()
    want_y, want_m = read()
    assert np.all(np.isfinite(want_y)) and np.all(np.isfinite(want_m))
    g = ctx.graph_capture(step)
    try:
        for rep in range(4):
            clear()
            ctx.graph_launch(g)
            got_y, got_m = read()
            assert np.array_equal(bits(got_y), bits(want_y)), rep
            assert np.array_equal(bits(got_m), bits(want_m)), rep
            step()  # eager work between replays
            ctx.synchronize()
    finally:
        ctx.graph_release(g)
    clear()
    step()
    y2, m2 = read()
    assert np.array_equal(bits(y2), bits(want_y)) and np.array_equal(bits(m2), bits(want_m))
    free()


def test_graph_capture_rejects_a_synchronizing_call(ctx):
    """A call that synchronizes fails inside a capture, graph_end reports
    it, and the context works normally afterwards."""
    step, read, clear, free = _layer_case(ctx, 72, 32)
    step()
    want_y, want_m = read()
    ctx.graph_begin()
    step()
    with pytest.raises(wohper_amd.DeepSeekV4KernelError):
        ctx.synchronize()
    with pytest.raises(wohper_amd.DeepSeekV4KernelError):
        ctx.graph_end()
    clear()
    step()
    y2, m2 = read()
    assert np.array_equal(bits(y2), bits(want_y)) and np.array_equal(bits(m2), bits(want_m))
    free()
