"""GPU parity of the mHC hyper-connections (hc_split_sinkhorn_scalar,
hc_pre_into, hc_post_into; E/compute.rs:4945-5092) against the oracle: the
Sinkhorn split and hc_post bit for bit; hc_pre bit for bit under exact
numerics (the reference's serial dot and sum-of-squares order) and within
1e-5 of the largest value with exact numerics off (tree sums), at the
model's shape (hc 4 x hidden 4096, 24 mix rows, 20 rounds) and small
ones."""
import numpy as np
import pytest

from test_gpu_mla import Dev

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture
def dev(ctx):
    d = Dev(ctx)
    yield d
    d.free()
    ctx.set_exact_numerics(True)


def _params(rng, hc, hidden):
    mix_hc = (2 + hc) * hc
    fn = (rng.standard_normal((mix_hc, hc * hidden)) * (1.0 / np.sqrt(hc * hidden))).astype(np.float32)
    scale = (0.5 + rng.random(3)).astype(np.float32)
    base = (rng.standard_normal(mix_hc) * 0.5).astype(np.float32)
    return fn, scale, base


@pytest.mark.parametrize("hc,iters", [(4, 20), (4, 1), (4, 0), (1, 20), (2, 3), (14, 20)])
def test_split_sinkhorn_bit_exact(ctx, oracle, dev, hc, iters):
    rng = np.random.default_rng(hc * 10 + iters)
    mix_hc = (2 + hc) * hc
    mixes = rng.standard_normal(mix_hc).astype(np.float32) * 2
    scale = (0.5 + rng.random(3)).astype(np.float32)
    base = rng.standard_normal(mix_hc).astype(np.float32)
    pp, qp, cp = dev.empty(hc * 4), dev.empty(hc * 4), dev.empty(hc * hc * 4)
    ctx.hc_split_sinkhorn_async(dev.put(mixes), dev.put(scale), dev.put(base), hc, iters, 1e-6, pp, qp, cp)
    ctx.synchronize()
    want = oracle.hc_split_sinkhorn(mixes, scale, base, hc, iters, 1e-6)
    for got, w in zip((dev.get(pp, hc), dev.get(qp, hc), dev.get(cp, hc * hc)), want):
        assert np.array_equal(bits(got), bits(w))


@pytest.mark.parametrize("hc,hidden", [(4, 4096), (2, 3), (3, 1001), (4, 64)])
def test_hc_pre_post_exact(ctx, oracle, dev, hc, hidden):
    rng = np.random.default_rng(hc * 7 + hidden)
    fn, scale, base = _params(rng, hc, hidden)
    x = rng.standard_normal(hc * hidden).astype(np.float32)
    yp, qp, cp, op = dev.empty(hidden * 4), dev.empty(hc * 4), dev.empty(hc * hc * 4), dev.empty(hc * hidden * 4)
    xp = dev.put(x)
    ctx.set_exact_numerics(True)
    ctx.hc_pre_async(dev.put(fn), dev.put(scale), dev.put(base), hc, hidden, 20, 1e-6, xp, yp, qp, cp)
    ctx.synchronize()
    y, pre, post, comb, _ = oracle.hc_pre(fn, scale, base, x, hc, hidden, 20, 1e-6)
    assert np.array_equal(bits(dev.get(yp, hidden)), bits(y))
    assert np.array_equal(bits(dev.get(qp, hc)), bits(post))
    assert np.array_equal(bits(dev.get(cp, hc * hc)), bits(comb))
    # hc_post with a sub-block output of its own
    ys = rng.standard_normal(hidden).astype(np.float32)
    ctx.hc_post_async(dev.put(ys), xp, qp, cp, op, hc, hidden)
    ctx.synchronize()
    assert np.array_equal(bits(dev.get(op, hc * hidden)), bits(oracle.hc_post(ys, x, post, comb, hc, hidden)))


def test_hc_pre_fast_within_tolerance(ctx, oracle, dev):
    hc, hidden = 4, 4096
    rng = np.random.default_rng(44)
    fn, scale, base = _params(rng, hc, hidden)
    x = rng.standard_normal(hc * hidden).astype(np.float32)
    yp, qp, cp = dev.empty(hidden * 4), dev.empty(hc * 4), dev.empty(hc * hc * 4)
    args = (dev.put(fn), dev.put(scale), dev.put(base), hc, hidden, 20, 1e-6, dev.put(x), yp, qp, cp)
    y, pre, post, comb, _ = oracle.hc_pre(fn, scale, base, x, hc, hidden, 20, 1e-6)
    times = {}
    for exact in (True, False):
        ctx.set_exact_numerics(exact)
        ctx.hc_pre_async(*args)
        ctx.synchronize()
        ctx.timer_start()
        for _ in range(20):
            ctx.hc_pre_async(*args)
        times[exact] = ctx.timer_stop() / 20
        ctx.synchronize()
    # the last run is the tree-sum one
    for got, want in ((dev.get(yp, hidden), y), (dev.get(qp, hc), post), (dev.get(cp, hc * hc), comb)):
        assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))
    print(f"hc_pre 4 x 4096: exact {times[True]:.1f} us, tree sums {times[False]:.1f} us")
