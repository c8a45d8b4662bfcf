"""A token's experts from a route list in device memory
(wh_routed_and_shared_experts_dev_async): the router on the device
(route_experts_from_dense_block, E/compute.rs:2129-2268) feeds
compute_active_and_shared_experts (E/compute.rs:1872-1946) without a host
round trip.  The same kernels run as for a host route list, so the result
must equal the host-route call on the router's own ids and weights bit for
bit in both numerics modes, and the oracle's expert forward + routed sum in
exact numerics; shorter route lists, unresident ids and bad arguments are
covered too."""
import numpy as np
import pytest

import wohper_amd
from parity_util import bits
from wohper_amd import model_format as mf
from wohper_amd import workloads as wl

pytestmark = pytest.mark.gpu

LAYER, N_EXP, SEED = 41, 32, 81


@pytest.fixture(scope="module")
def layer(ctx):
    """N_EXP routed experts + the shared one (id N_EXP) and a bf16 router of
    N_EXP rows with a selection bias, all resident."""
    for e in range(N_EXP + 1):
        ctx.store_expert_synthetic(LAYER, e, wl.HIDDEN, wl.INTER, SEED)
    rng = np.random.default_rng(SEED)
    gate = ((rng.standard_normal((N_EXP, wl.HIDDEN)).astype(np.float32) * 0.02).view(np.uint32) >> 16)
    bias = (rng.standard_normal(N_EXP) * 0.05).astype(np.float32)
    blk = mf.build_synthetic_quant_block([
        mf.SyntheticTensor(f"layers.{LAYER}.ffn.gate.weight", 9, (N_EXP, wl.HIDDEN), gate.astype(np.uint16).tobytes(),
                           11, 2404),
        mf.SyntheticTensor(f"layers.{LAYER}.ffn.gate.bias", 9, (N_EXP,), bias.tobytes(), 12, 2405)])
    ctx.store_router(LAYER, blk, wl.HIDDEN)
    yield
    ctx.set_exact_numerics(True)


def _bufs(ctx, x):
    xd = ctx.device_alloc(x.nbytes)
    ctx.to_device(xd, x)
    ids, sc, cnt = ctx.device_alloc(64), ctx.device_alloc(64), ctx.device_alloc(16)
    out, out2 = ctx.device_alloc(wl.HIDDEN * 4), ctx.device_alloc(wl.HIDDEN * 4)
    return xd, ids, sc, cnt, out, out2


def _read(ctx, p, n, dtype=np.float32):
    a = np.empty(n, dtype)
    ctx.from_device(a, p)
    return a


@pytest.mark.parametrize("exact", [True, False])
def test_device_routes_equal_host_routes(ctx, oracle, layer, exact):
    ctx.set_exact_numerics(exact)
    rng = np.random.default_rng(3)
    x = rng.standard_normal(wl.HIDDEN).astype(np.float32)
    xd, ids, sc, cnt, out, out2 = _bufs(ctx, x)
    ctx.route_experts_async(LAYER, xd, wl.HIDDEN, 6, 0, 0, ids, sc, cnt, route_scale=1.5)
    ctx.routed_and_shared_experts_dev_async(LAYER, ids, sc, cnt, 6, (LAYER, N_EXP), xd, False, out)
    ctx.synchronize()
    n = int(_read(ctx, cnt, 1, np.uint32)[0])
    rid, rw = _read(ctx, ids, n, np.uint32), _read(ctx, sc, n)
    assert n == 6
    routes = [(LAYER, int(e), float(w)) for e, w in zip(rid, rw)]
    ctx.routed_and_shared_experts_async(routes, (LAYER, N_EXP), xd, False, 1, out2)
    ctx.synchronize()
    got, want = _read(ctx, out, wl.HIDDEN), _read(ctx, out2, wl.HIDDEN)
    assert np.array_equal(bits(got), bits(want))
    if exact:
        sh = oracle.fp4_expert_forward(*wl.synth_expert_host(ctx.lib, SEED, LAYER, N_EXP), x)
        outs = np.stack([oracle.fp4_expert_forward(*wl.synth_expert_host(ctx.lib, SEED, LAYER, int(e)), x)
                         for e in rid])
        assert np.array_equal(bits(got), bits(sh + oracle.routed_combine(outs, rw)))
    for p in (xd, ids, sc, cnt, out, out2):
        ctx.device_free(p)


@pytest.mark.parametrize("exact", [False, True])
@pytest.mark.parametrize("count,shared", [(3, True), (1, True), (0, True), (4, False)])
def test_device_routes_shorter_lists(ctx, layer, count, shared, exact):
    """count below n_slots: only the first count routes are summed (the
    other slots compute a copy of a resident expert that is never added).
    Exact numerics: bit-identical to the host list of count routes.  MFMA
    numerics: the 7-slot launch and the host list's shorter one may take
    down kernels that round an expert's block sums in another order (one
    256-column block per wave for an odd expert count, chained block pairs
    for an even one), so they agree within 1e-5 of the largest output; a
    padded slot added by mistake would move the output by a whole expert."""
    ctx.set_exact_numerics(exact)
    rng = np.random.default_rng(count)
    x = rng.standard_normal(wl.HIDDEN).astype(np.float32)
    xd, ids, sc, cnt, out, out2 = _bufs(ctx, x)
    rid = np.array([5, 17, 2, 30, 9, 11], np.uint32)
    rw = np.array([0.4, 0.3, 0.2, 0.1, 0.25, 0.05], np.float32)
    ctx.to_device(ids, rid)
    ctx.to_device(sc, rw)
    ctx.to_device(cnt, np.array([count], np.uint32))
    key = (LAYER, N_EXP) if shared else None
    ctx.routed_and_shared_experts_dev_async(LAYER, ids, sc, cnt, 6, key, xd, False, out)
    routes = [(LAYER, int(e), float(w)) for e, w in zip(rid[:count], rw[:count])]
    if shared:
        ctx.routed_and_shared_experts_async(routes, key, xd, False, 1, out2)
    else:
        ctx.routed_experts_async(routes, xd, False, 1, out2)
    ctx.synchronize()
    got, want = _read(ctx, out, wl.HIDDEN), _read(ctx, out2, wl.HIDDEN)
    if exact:
        assert np.array_equal(bits(got), bits(want))
    else:
        assert float(np.abs(got - want).max()) <= 1e-5 * float(np.abs(want).max())
    ctx.set_exact_numerics(False)
    for p in (xd, ids, sc, cnt, out, out2):
        ctx.device_free(p)


def test_device_routes_errors(ctx, layer):
    x = np.ones(wl.HIDDEN, np.float32)
    xd, ids, sc, cnt, out, out2 = _bufs(ctx, x)
    ctx.to_device(ids, np.array([3, 200, 4], np.uint32))  # 200: no such expert
    ctx.to_device(sc, np.array([0.5, 0.3, 0.2], np.float32))
    ctx.to_device(cnt, np.array([3], np.uint32))
    ctx.routed_and_shared_experts_dev_async(LAYER, ids, sc, cnt, 3, (LAYER, N_EXP), xd, False, out)
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.synchronize()
    assert e.value.name == "NotResident"
    for n_slots in (0, 16):  # 16 routed slots + the shared one: one slot too many
        with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
            ctx.routed_and_shared_experts_dev_async(LAYER, ids, sc, cnt, n_slots, (LAYER, N_EXP), xd, False, out)
        assert e.value.name == "InvalidArgument"
    for p in (xd, ids, sc, cnt, out, out2):
        ctx.device_free(p)
