"""GPU parity of the MFMA routed-expert kernels (set_exact_numerics(False))
of the routed/shared expert entry points (compute_active_experts and
compute_active_and_shared_experts, E/compute.rs:1872-2030, over
deepseek_v4_fp4_expert_forward_scalar, E/deepseek_v4.rs:551-601).

Every matvec (gate, up, down of every expert and token) is checked against
the oracle on the same input within max|diff| <= 1e-5 * ||w_row||_2 *
||x||_2; the act-quant of x is the oracle's; SwiGLU, the act-quant of h and
the route-weighted sum are bit-exact given the GPU's matvec outputs."""
import numpy as np
import pytest

import wohper_amd
from parity_util import bits, check_matvec
from wohper_amd import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def fast_capture(ctx):
    ctx.set_exact_numerics(False)
    ctx.debug_moe_token_capture(True)
    yield
    ctx.debug_moe_token_capture(False)
    ctx.set_exact_numerics(True)


def _check_token(ctx, oracle, experts, weights, x, out, tok, n_tok, has_shared, hidden, inter):
    """experts: host (w1, w3, w2) per slot (routed first, then the shared one)."""
    n = len(experts)
    gu = ctx.debug_moe_token_read(0, (n_tok, n, 2, inter))[tok]
    h = ctx.debug_moe_token_read(1, (n_tok, n, inter))[tok]
    y = ctx.debug_moe_token_read(2, (n_tok, n, hidden))[tok]
    xq = oracle.act_quant(x, 64)
    worst = 0.0
    for i, (w1, w3, w2) in enumerate(experts):
        worst = max(worst, check_matvec(oracle, w1, xq, gu[i, 0], False, ("gate", i)))
        worst = max(worst, check_matvec(oracle, w3, xq, gu[i, 1], False, ("up", i)))
        assert np.array_equal(bits(h[i]), bits(oracle.swiglu_array(gu[i, 0], gu[i, 1]))), ("swiglu", i)
        worst = max(worst, check_matvec(oracle, w2, oracle.act_quant(h[i], 64), y[i], False, ("down", i)))
    nr = n - has_shared
    if nr:
        want = oracle.routed_combine(y[:nr], weights)
        if has_shared:
            want = (y[nr] + want).astype(np.float32)
    else:
        want = y[nr]
    assert np.array_equal(bits(out), bits(want))
    return worst


def _oracle_forward(oracle, experts, weights, x, has_shared):
    outs = np.stack([oracle.fp4_expert_forward(*m, x) for m in experts])
    nr = len(experts) - has_shared
    want = oracle.routed_combine(outs[:nr], weights) if nr else outs[nr]
    if has_shared and nr:
        want = outs[nr] + want
    return want.astype(np.float32)


@pytest.mark.parametrize("kernels", [1, 0, 2, 3])
def test_fast_routed_six_experts(ctx, oracle, kernels):
    """The headline token: 6 routed experts of the model's shapes, on each
    pairing of the LDS-streaming and register-ring gate/up and down kernels
    (mask bit 0: gate/up, bit 1: down; 1 is the default)."""
    ctx.debug_token_kernels(kernels)
    try:
        _routed_six(ctx, oracle)
    finally:
        ctx.debug_token_kernels(1)


def _routed_six(ctx, oracle):
    seed = 2
    idx, w, x = wl.moe_token_case(seed)
    routes = [(13, int(e), float(wt)) for e, wt in zip(idx, w)]
    for _, e, _ in routes:
        ctx.store_expert_synthetic(13, e, wl.HIDDEN, wl.INTER, seed)
    experts = [wl.synth_expert_host(ctx.lib, seed, 13, e) for _, e, _ in routes]
    got = ctx.routed_experts(routes, x)
    worst = _check_token(ctx, oracle, experts, w, x, got, 0, 1, 0, wl.HIDDEN, wl.INTER)
    print(f"worst matvec |diff| / tolerance: {worst:.3f}")
    want = _oracle_forward(oracle, experts, w, x, 0)
    assert np.linalg.norm(got - want) <= 1e-3 * np.linalg.norm(want)


@pytest.mark.parametrize("n_routed", [6, 4, 2, 1, 0])
def test_fast_shared_plus_routed(ctx, oracle, n_routed):
    seed = 4
    idx, w, x = wl.moe_token_case(seed)
    routes = [(15, int(e), float(wt)) for e, wt in zip(idx[:n_routed], w[:n_routed])]
    for _, e, _ in routes:
        ctx.store_expert_synthetic(15, e, wl.HIDDEN, wl.INTER, seed)
    shared = (15, wl.N_ROUTED)
    ctx.store_expert_synthetic(*shared, wl.HIDDEN, wl.INTER, seed)
    experts = [wl.synth_expert_host(ctx.lib, seed, 15, e) for _, e, _ in routes]
    experts.append(wl.synth_expert_host(ctx.lib, seed, *shared))
    got = ctx.routed_and_shared_experts(routes, shared, x)
    _check_token(ctx, oracle, experts, w[:n_routed], x, got, 0, 1, 1, wl.HIDDEN, wl.INTER)


def test_fast_tokens_bf16_async(ctx, oracle):
    """Three bf16 tokens through one route list on device pointers (grid.y =
    token), with the shared expert."""
    seed, n_tok = 6, 3
    idx, w, _ = wl.moe_token_case(seed)
    x = wl.bf16_round(np.random.default_rng(seed).standard_normal((n_tok, wl.HIDDEN)).astype(np.float32))
    routes = [(16, int(e), float(wt)) for e, wt in zip(idx, w)]
    for _, e, _ in routes:
        ctx.store_expert_synthetic(16, e, wl.HIDDEN, wl.INTER, seed)
    shared = (16, wl.N_ROUTED)
    ctx.store_expert_synthetic(*shared, wl.HIDDEN, wl.INTER, seed)
    experts = [wl.synth_expert_host(ctx.lib, seed, 16, e) for _, e, _ in routes]
    experts.append(wl.synth_expert_host(ctx.lib, seed, *shared))
    xb = wl.bf16_bits(x)
    x_dev, out_dev = ctx.device_alloc(xb.nbytes), ctx.device_alloc(x.nbytes)
    ctx.to_device(x_dev, xb)
    ctx.routed_and_shared_experts_async(routes, shared, x_dev, True, n_tok, out_dev)
    ctx.synchronize()
    got = np.empty_like(x)
    ctx.from_device(got, out_dev)
    for t in range(n_tok):
        _check_token(ctx, oracle, experts, w, x[t], got[t], t, n_tok, 1, wl.HIDDEN, wl.INTER)
    ctx.device_free(x_dev)
    ctx.device_free(out_dev)


def test_fast_hidden_2048(ctx, oracle):
    """hidden 2048 (one column slice per row): two routed experts."""
    hidden, inter, seed = 2048, 2048, 8
    x = np.random.default_rng(seed).standard_normal(hidden).astype(np.float32)
    routes = [(17, 3, 0.7), (17, 9, 0.2)]
    for _, e, _ in routes:
        ctx.store_expert_synthetic(17, e, hidden, inter, seed)
    experts = [wl.synth_expert_host(ctx.lib, seed, 17, e, hidden, inter) for _, e, _ in routes]
    got = ctx.routed_experts(routes, x)
    _check_token(ctx, oracle, experts, [0.7, 0.2], x, got, 0, 1, 0, hidden, inter)


def test_fast_single_expert_forward(ctx, oracle):
    """deepseek_v4_fp4_expert_forward_scalar through the same kernels."""
    seed = 21
    ctx.store_expert_synthetic(18, 7, wl.HIDDEN, wl.INTER, seed)
    x = np.random.default_rng(seed).standard_normal(wl.HIDDEN).astype(np.float32) * 3.0
    got = ctx.fp4_expert_forward(18, 7, x, wl.HIDDEN, 2 * wl.INTER)
    _check_token(ctx, oracle, [wl.synth_expert_host(ctx.lib, seed, 18, 7)], [1.0], x, got, 0, 1, 0,
                 wl.HIDDEN, wl.INTER)


def test_fast_wide_scales(ctx, oracle):
    """UE8M0 exponents over [-20, 6] and x over six decades stay within
    tolerance."""
    seed = 23
    ctx.store_expert_synthetic(19, 1, wl.HIDDEN, wl.INTER, seed, 107, 133)
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(wl.HIDDEN) * np.exp(rng.uniform(-7, 7, wl.HIDDEN))).astype(np.float32)
    got = ctx.routed_experts([(19, 1, 1.0)], x)
    ex = [wl.synth_expert_host(ctx.lib, seed, 19, 1, scale_lo=107, scale_hi=133)]
    _check_token(ctx, oracle, ex, [1.0], x, got, 0, 1, 0, wl.HIDDEN, wl.INTER)


@pytest.mark.parametrize("exact", [False, True])
def test_nonfinite_inputs_follow_the_reference(ctx, oracle, exact):
    """fp8_act_quant_dequant_in_place (E/compute.rs:2504-2545) inside the
    expert forward: NaN inputs quantize to -480 x the block scale and the
    token stays finite (checked against the oracle: bit for bit in exact
    mode, per matvec within tolerance in MFMA mode); an inf makes its
    block's scale infinite, and the forward ends in NonFiniteOutput
    (E/deepseek_v4.rs:597-599), as the oracle does."""
    ctx.set_exact_numerics(exact)
    seed = 24
    ctx.store_expert_synthetic(19, 2, wl.HIDDEN, wl.INTER, seed)
    ctx.store_expert_synthetic(19, 3, wl.HIDDEN, wl.INTER, seed)
    ex = [wl.synth_expert_host(ctx.lib, seed, 19, e) for e in (2, 3)]
    routes, w = [(19, 2, 0.6), (19, 3, 0.4)], [0.6, 0.4]
    x = np.random.default_rng(seed).standard_normal(wl.HIDDEN).astype(np.float32)
    x[[5, 64, 700, 701, 4095]] = np.nan   # several blocks, two NaN in one
    x[128:192] = np.nan                   # a block of NaN only: amax 0 -> scale of 1e-4
    got = ctx.routed_experts(routes, x)
    assert np.all(np.isfinite(got))
    want = _oracle_forward(oracle, ex, w, x, 0)
    if exact:
        assert np.array_equal(bits(got), bits(want))
    else:
        _check_token(ctx, oracle, ex, w, x, got, 0, 1, 0, wl.HIDDEN, wl.INTER)
    for bad in (np.inf, -np.inf):
        xi = x.copy()
        xi[300] = bad
        with pytest.raises(oracle.OracleError) as oe:
            oracle.fp4_expert_forward(*ex[0], xi)
        assert oe.value.code == 8  # NonFiniteOutput
        with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
            ctx.routed_experts(routes, xi)
        assert e.value.name == "NonFiniteOutput"
    # the context recovers: the next finite token is exact again
    got = ctx.routed_experts(routes, np.nan_to_num(x))
    assert np.all(np.isfinite(got))


def test_exact_switch_restores_bit_exact(ctx, oracle):
    seed = 2
    idx, w, x = wl.moe_token_case(seed)
    routes = [(13, int(e), float(wt)) for e, wt in zip(idx, w)]
    for _, e, _ in routes:
        ctx.store_expert_synthetic(13, e, wl.HIDDEN, wl.INTER, seed)
    experts = [wl.synth_expert_host(ctx.lib, seed, 13, e) for _, e, _ in routes]
    ctx.set_exact_numerics(True)
    got = ctx.routed_experts(routes, x)
    assert np.array_equal(bits(got), bits(_oracle_forward(oracle, experts, w, x, 0)))
