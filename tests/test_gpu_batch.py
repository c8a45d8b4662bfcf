"""GPU parity of the ragged batched routed experts (the batch-prefill MoE of
E/server/generation.rs:2487-2569 with accumulate_expert_for_positions,
E/compute.rs:1779-1810) against the oracle.

Exact path (exact numerics, or every expert below the MFMA threshold):
bit-exact - device packing of the per-expert token lists, the per-position
weight rule, ascending-id accumulation, the shared expert, chunking of large
batches and the generic shapes.  MFMA path (exact numerics off, experts at or
above the threshold): every matvec within max|diff| <= 1e-5 * ||w_row||_2 *
||x||_2 of the oracle on the same input, every other stage bit-exact."""
import numpy as np
import pytest

import wohper_amd
from parity_util import check_matvec as _check_matvec
from wohper_amd import workloads as wl

pytestmark = pytest.mark.gpu
DEFAULT_MFMA_MIN = 1


@pytest.fixture(autouse=True)
def exact_path(ctx):
    """Tests compare bit-exactly unless they opt into MFMA groups."""
    ctx.set_exact_numerics(True)
    yield
    ctx.set_exact_numerics(True)
    ctx.set_moe_mfma_min(DEFAULT_MFMA_MIN)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _store(ctx, layer, n, hidden, inter, seed):
    for e in range(n):
        ctx.store_expert_synthetic(layer, e, hidden, inter, seed)


def _host(ctx, layer, ids, seed, hidden, inter):
    return {int(e): wl.synth_expert_host(ctx.lib, seed, layer, int(e), hidden, inter) for e in np.unique(ids)}


def _special_rows(ids, sc):
    """Rows that exercise every branch of the weight rule."""
    sc = sc.copy()
    sc[0, 1] = np.nan                       # non-finite score -> uniform
    sc[1, :] = 0.0                          # zero sum -> uniform
    sc[2, 0] = -0.25                        # negative score, positive sum -> score / sum
    sc[3, :] = -1.0                         # negative sum -> uniform
    ids = ids.copy()
    ids[4, 1] = ids[4, 0]                   # the same expert twice in one position
    return ids, sc


def test_batch_small_shapes_bit_exact(ctx, oracle):
    hidden, inter, n_exp, seed = 512, 256, 24, 31
    _store(ctx, 40, n_exp, hidden, inter, seed)
    ctx.store_expert_synthetic(41, 0, hidden, inter, seed)  # shared
    ids, sc, x = wl.zipf_batch_routes(seed=5, n_tokens=40, n_experts=n_exp, hidden=hidden)
    ids, sc = _special_rows(ids, sc)
    experts = _host(ctx, 40, ids, seed, hidden, inter)
    want = oracle.moe_batch(experts, ids, sc, x)
    got = ctx.moe_batch(40, ids, sc, x)
    assert np.array_equal(bits(got), bits(want))
    shared = wl.synth_expert_host(ctx.lib, seed, 41, 0, hidden, inter)
    want_sh = oracle.moe_batch(experts, ids, sc, x, shared=shared)
    got_sh = ctx.moe_batch(40, ids, sc, x, shared_key=(41, 0))
    assert np.array_equal(bits(got_sh), bits(want_sh))


def test_batch_one_position_one_route(ctx, oracle):
    """A group of one token and a batch of one position."""
    hidden, inter, seed = 512, 256, 31
    _store(ctx, 40, 24, hidden, inter, seed)
    x = np.random.default_rng(8).standard_normal((1, hidden)).astype(np.float32)
    ids = np.array([[17]], np.uint32)
    got = ctx.moe_batch(40, ids, np.array([[0.3]], np.float32), x)
    want = oracle.fp4_expert_forward(*wl.synth_expert_host(ctx.lib, seed, 40, 17, hidden, inter), x[0])
    assert np.array_equal(bits(got[0]), bits(want))


def test_batch_real_shape_bf16_async(ctx, oracle):
    """Expert shapes of the model (4096 x 2048), bf16 input, device pointers."""
    n_exp, seed, npos = 16, 44, 8
    _store(ctx, 42, n_exp, wl.HIDDEN, wl.INTER, seed)
    ids, sc, x = wl.zipf_batch_routes(seed=6, n_tokens=npos, n_experts=n_exp)
    experts = _host(ctx, 42, ids, seed, wl.HIDDEN, wl.INTER)
    want = oracle.moe_batch(experts, ids, sc, x)
    xb = wl.bf16_bits(x)
    x_dev = ctx.device_alloc(xb.nbytes)
    ids_dev = ctx.device_alloc(ids.nbytes)
    sc_dev = ctx.device_alloc(sc.nbytes)
    out_dev = ctx.device_alloc(x.nbytes)
    ctx.to_device(x_dev, xb)
    ctx.to_device(ids_dev, ids)
    ctx.to_device(sc_dev, sc)
    ctx.moe_batch_async(42, ids_dev, sc_dev, npos, ids.shape[1], x_dev, True, out_dev)
    ctx.synchronize()
    got = np.empty_like(x)
    ctx.from_device(got, out_dev)
    assert np.array_equal(bits(got), bits(want))
    # the host-slice variant (f32 input) agrees
    assert np.array_equal(bits(ctx.moe_batch(42, ids, sc, x)), bits(want))
    # a route to an expert id that is not resident is reported by the stream
    bad = ids.copy()
    bad[3, 2] = 200
    ctx.to_device(ids_dev, bad)
    ctx.moe_batch_async(42, ids_dev, sc_dev, npos, ids.shape[1], x_dev, True, out_dev)
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.synchronize()
    assert e.value.name == "NotResident"
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.moe_batch(42, bad, sc, x)
    assert e.value.name == "NotResident"
    for p in (x_dev, ids_dev, sc_dev, out_dev):
        ctx.device_free(p)


def test_batch_chunked_positions(ctx, oracle):
    """More than 4096 slots: the positions are split into chunks."""
    hidden, inter, n_exp, seed = 512, 256, 24, 31
    _store(ctx, 40, n_exp, hidden, inter, seed)
    ctx.store_expert_synthetic(41, 0, hidden, inter, seed)
    ids, sc, x = wl.zipf_batch_routes(seed=9, n_tokens=700, n_experts=n_exp, hidden=hidden)
    experts = _host(ctx, 40, ids, seed, hidden, inter)
    shared = wl.synth_expert_host(ctx.lib, seed, 41, 0, hidden, inter)
    got = ctx.moe_batch(40, ids, sc, x, shared_key=(41, 0))
    want = oracle.moe_batch(experts, ids, sc, x, shared=shared)
    assert np.array_equal(bits(got), bits(want))


def test_batch_generic_shapes(ctx, oracle):
    """Shapes outside the fast layout take the host-built union."""
    rng = np.random.default_rng(12)
    hidden, inter = 96, 40
    experts = {}
    for e in range(5):
        m = []
        for rows, cols in ((inter, hidden), (inter, hidden), (hidden, inter)):
            p = rng.integers(0, 256, (rows, cols // 2)).astype(np.uint8)
            s = rng.integers(118, 130, (rows, cols // 8)).astype(np.uint8)
            m.append((p, s, rows, cols, cols // 8))
        experts[e] = tuple(m)
        ctx.store_fp4_expert(43, e, wohper_amd.DeepSeekV4Fp4Expert(*[wohper_amd.Fp4Matvec(*t) for t in m]))
    ids = np.array([[4, 0, 2], [1, 4, 3], [2, 2, 0], [3, 1, 4], [0, 1, 2]], np.uint32)
    sc = rng.uniform(0.1, 1.0, ids.shape).astype(np.float32)
    sc[1, 0] = np.inf
    x = rng.standard_normal((5, hidden)).astype(np.float32)
    got = ctx.moe_batch(43, ids, sc, x)
    want = oracle.moe_batch(experts, ids, sc, x)
    assert np.array_equal(bits(got), bits(want))


def _mfma_case(ctx, oracle, layer, n_exp, hidden, inter, seed, npos, mfma_min, routes=None):
    """routes: (ids, scores, x) instead of the Zipf routing; returns the
    worst matvec |diff| / tolerance and the count of virtual experts."""
    _store(ctx, layer, n_exp, hidden, inter, seed)
    ids, sc, x = routes if routes is not None else wl.zipf_batch_routes(seed=seed, n_tokens=npos, n_experts=n_exp,
                                                                       hidden=hidden)
    experts = _host(ctx, layer, ids, seed, hidden, inter)
    topk, S = ids.shape[1], ids.size
    ctx.set_exact_numerics(False)
    ctx.set_moe_mfma_min(mfma_min)
    try:
        out = ctx.moe_batch(layer, ids, sc, x)
    finally:
        ctx.set_exact_numerics(True)
    rd = ctx.debug_moe_batch_read
    srt, gate, up = rd(0, S, np.uint32), rd(1, (S, inter), np.float32), rd(2, (S, inter), np.float32)
    y, hq = rd(3, (S, hidden), np.float32), rd(8, (S, inter), np.float32)
    meta, uoff, uexp, uorder = rd(4, 8, np.uint32), rd(5, S + 1, np.uint32), rd(6, S, np.uint32), rd(7, S, np.uint32)
    n_used, n_mfma, n_virtual = int(meta[0]), int(meta[4]), int(meta[7])
    assert 0 < n_mfma <= n_used, (n_used, n_mfma)
    if mfma_min > 1:
        assert n_mfma < n_used, (n_used, n_mfma)  # both paths run
    on_mfma = {int(uexp[j]) for j in uorder[:n_mfma]}
    xq = {p: oracle.act_quant(x[p], 64) for p in range(npos)}
    wts = oracle.batch_route_weights(sc)
    acc = np.zeros_like(x)
    worst = 0.0
    for j in range(n_used):
        e = int(uexp[j])
        w1, w3, w2 = experts[e]
        exact = e not in on_mfma
        slots = range(int(uoff[j]), int(uoff[j + 1]))
        for s in slots:
            p = int(srt[s]) // topk
            # each matvec on the same input as the oracle's
            worst = max(worst, _check_matvec(oracle, w1, xq[p], gate[s], exact, ("gate", e, p)))
            worst = max(worst, _check_matvec(oracle, w3, xq[p], up[s], exact, ("up", e, p)))
            want_hq = oracle.act_quant(oracle.swiglu_array(gate[s], up[s]), 64)
            assert np.array_equal(bits(hq[s]), bits(want_hq)), ("swiglu + act-quant", s)
            worst = max(worst, _check_matvec(oracle, w2, hq[s], y[s], exact, ("down", e, p)))
        pos = [int(srt[s]) // topk for s in slots]
        acc = oracle.accumulate_expert(y[list(slots)], pos, [wts[int(srt[s]) // topk, int(srt[s]) % topk] for s in slots],
                                       acc)
    assert np.array_equal(bits(out), bits(acc))
    # end to end, the act-quant of h may round a near-tie the other way, so
    # the oracle's output is compared in norm only
    want = oracle.moe_batch(experts, ids, sc, x)
    assert np.linalg.norm(out - want) <= 1e-3 * np.linalg.norm(want)
    return worst, n_virtual


def test_batch_mfma_small_shapes(ctx, oracle):
    worst, _ = _mfma_case(ctx, oracle, 44, 12, 512, 256, 33, 48, 8)
    print(f"worst MFMA matvec |diff| / tolerance: {worst:.3f}")


@pytest.mark.parametrize("mfma_min", [16, DEFAULT_MFMA_MIN])
def test_batch_mfma_real_shapes(ctx, oracle, mfma_min):
    worst, _ = _mfma_case(ctx, oracle, 45, 8, wl.HIDDEN, wl.INTER, 34, 24, mfma_min)
    print(f"worst MFMA matvec |diff| / tolerance: {worst:.3f}")


def test_batch_mfma_more_virtual_experts_than_workgroups(ctx, oracle):
    """More than 256 virtual experts (about 300 experts on 300 positions,
    uniform top-6): the persistent MFMA kernels' workgroups each cover more
    than two virtual experts and stage them in phases of two; every matvec
    within tolerance and every other stage bit-exact, as above."""
    hidden = inter = 2048
    n_exp, npos, seed = 300, 300, 36
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(n_exp, 6, replace=False) for _ in range(npos)]).astype(np.uint32)
    sc = rng.uniform(0.05, 1.0, (npos, 6)).astype(np.float32)
    x = rng.standard_normal((npos, hidden)).astype(np.float32)
    worst, n_virtual = _mfma_case(ctx, oracle, 47, n_exp, hidden, inter, seed, npos, DEFAULT_MFMA_MIN,
                                  routes=(ids, sc, x))
    assert n_virtual > 256, n_virtual
    print(f"{n_virtual} virtual experts; worst MFMA matvec |diff| / tolerance: {worst:.3f}")


def test_batch_exact_numerics_override_the_threshold(ctx, oracle):
    """Exact numerics keep every expert on the exact items whatever the
    threshold: bit-exact against the oracle."""
    layer, n_exp, hidden, inter, seed, npos = 44, 12, 512, 256, 33, 48
    _store(ctx, layer, n_exp, hidden, inter, seed)
    ids, sc, x = wl.zipf_batch_routes(seed=seed, n_tokens=npos, n_experts=n_exp, hidden=hidden)
    ctx.set_moe_mfma_min(1)
    got = ctx.moe_batch(layer, ids, sc, x)
    assert int(ctx.debug_moe_batch_read(4, 8, np.uint32)[4]) == 0
    want = oracle.moe_batch(_host(ctx, layer, ids, seed, hidden, inter), ids, sc, x)
    assert np.array_equal(bits(got), bits(want))


def test_batch_nonfinite_inputs_follow_the_reference(ctx, oracle):
    """A NaN input quantizes to -480 x its block scale (E/compute.rs:2504-2545)
    and the batch stays finite and bit-exact against the oracle, with every
    expert kept off MFMA (-480 has no E4M3 code); an inf makes its block's
    scale infinite and the batch ends in NonFiniteOutput.  The next finite
    batch takes MFMA items again."""
    layer, n_exp, hidden, inter, seed, npos = 46, 12, 512, 256, 35, 48
    _store(ctx, layer, n_exp, hidden, inter, seed)
    ids, sc, x = wl.zipf_batch_routes(seed=seed, n_tokens=npos, n_experts=n_exp, hidden=hidden)
    experts = _host(ctx, layer, ids, seed, hidden, inter)
    ctx.set_exact_numerics(False)
    ctx.set_moe_mfma_min(8)
    xn = x.copy()
    xn[3, [0, 70, 71]] = np.nan
    xn[9, 64:128] = np.nan
    got = ctx.moe_batch(layer, ids, sc, xn)
    assert int(ctx.debug_moe_batch_read(4, 8, np.uint32)[4]) == 0  # no MFMA item ran
    assert np.all(np.isfinite(got))
    assert np.array_equal(bits(got), bits(oracle.moe_batch(experts, ids, sc, xn)))
    xi = x.copy()
    xi[5, 200] = np.inf
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.moe_batch(layer, ids, sc, xi)
    assert e.value.name == "NonFiniteOutput"
    ctx.moe_batch(layer, ids, sc, x)
    assert int(ctx.debug_moe_batch_read(4, 8, np.uint32)[4]) > 0


def test_batch_nonfinite_inputs_at_the_default_threshold(ctx, oracle):
    """At threshold 1 every used expert is an MFMA expert and the exact-item
    kernels are not launched; after a NaN input the MFMA kernel's gate/up runs
    in fp32 from the act-quantized inputs (NaN -> -480 x the block scale, as
    E/compute.rs:2504-2545): every matvec within tolerance of the oracle's on
    the same input, SwiGLU + act-quant and the weighted sums bit-exact.  An inf
    input still ends in NonFiniteOutput, and the next finite batch is
    unaffected."""
    layer, n_exp, hidden, inter, seed, npos = 48, 12, 2048, 2048, 36, 24
    ids, sc, x = wl.zipf_batch_routes(seed=seed, n_tokens=npos, n_experts=n_exp, hidden=hidden)
    xn = x.copy()
    xn[3, [0, 70, 71]] = np.nan
    xn[9, 64:128] = np.nan
    worst, _ = _mfma_case(ctx, oracle, layer, n_exp, hidden, inter, seed, npos, DEFAULT_MFMA_MIN,
                          routes=(ids, sc, xn))
    print(f"worst fp32 matvec |diff| / tolerance: {worst:.3f}")
    xi = x.copy()
    xi[5, 200] = np.inf
    ctx.set_exact_numerics(False)
    ctx.set_moe_mfma_min(DEFAULT_MFMA_MIN)
    try:
        with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
            ctx.moe_batch(layer, ids, sc, xi)
        assert e.value.name == "NonFiniteOutput"
    finally:
        ctx.set_exact_numerics(True)
    worst, _ = _mfma_case(ctx, oracle, layer, n_exp, hidden, inter, seed, npos, DEFAULT_MFMA_MIN,
                          routes=(ids, sc, x))
