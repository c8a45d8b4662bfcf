"""GPU parity of the act-quant, the FP4 SwiGLU expert forward and the routed
expert sum with the oracle - bit-exact - plus the known answers of the
reference's expert tests."""
import json
from pathlib import Path

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
KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("block", [64, 128, 4, 7, 1000])
def test_act_quant_bit_exact(ctx, oracle, block):
    rng = np.random.default_rng(block)
    parts = [rng.standard_normal(4096) * s for s in (1e-6, 1e-3, 1.0, 30.0, 1e5)]
    x = np.concatenate(parts).astype(np.float32)
    x[::97] = 0.0
    x[5::101] = -x[5::101]
    got = ctx.act_quant_dequant(x, block)
    want = oracle.act_quant(x, block)
    assert np.array_equal(bits(got), bits(want))


def test_act_quant_midpoints_and_known_answers(ctx, oracle):
    _, _, _, srt = oracle.luts()
    grid = np.unique(srt.astype(np.float64))
    grid = grid[np.abs(grid) <= 448]
    mids = ((grid[1:] + grid[:-1]) / 2).astype(np.float32)
    # blocks of 64 whose amax is exactly 448 (scale 1) so the values stay midpoints
    vals = np.concatenate([mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf))])
    pad = (-vals.size) % 63
    vals = np.concatenate([vals, np.zeros(pad, np.float32)]).reshape(-1, 63)
    x = np.concatenate([np.full((vals.shape[0], 1), 448.0, np.float32), vals], axis=1).reshape(-1)
    assert np.array_equal(bits(ctx.act_quant_dequant(x, 64)), bits(oracle.act_quant(x, 64)))
    k = KATS["act_quant_representable"]
    assert np.all(np.abs(ctx.act_quant_dequant(np.array(k["values"], np.float32), k["block"]) - k["expected"]) < k["tol"])


def test_tiny_expert_known_answer(ctx, oracle):
    k = KATS["tiny_expert"]
    ex = wohper_amd.DeepSeekV4Fp4Expert(*[
        wohper_amd.Fp4Matvec(np.array(k[m]["packed"], np.uint8), np.array(k[m]["scales"], np.uint8),
                             k[m]["rows"], k[m]["cols"], k[m]["scale_cols"]) for m in ("w1", "w3", "w2")])
    out = np.zeros(2, np.float32)
    wohper_amd.deepseek_v4_fp4_expert_forward_scalar(ex, np.array(k["input"], np.float32), out, k["scratch"], ctx=ctx)
    h = np.float32(2.0) / (np.float32(1.0) + np.exp(np.float32(-2.0))) * np.float32(3.0)
    hq = oracle.act_quant([h], 64)[0]
    assert abs(out[0] - hq) < k["tol"] and abs(out[1] - 2 * hq) < k["tol"]
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        wohper_amd.deepseek_v4_fp4_expert_forward_scalar(ex, np.array(k["input"], np.float32), out, 1, ctx=ctx)
    assert e.value.name == "ScratchTooSmall"


def test_single_expert_forward_real_shape_bit_exact(ctx, oracle):
    seed = 21
    ctx.store_expert_synthetic(1, 7, wl.HIDDEN, wl.INTER, seed)
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(wl.HIDDEN).astype(np.float32)
    got = ctx.fp4_expert_forward(1, 7, x, wl.HIDDEN, 2 * wl.INTER)
    w1, w3, w2 = wl.synth_expert_host(ctx.lib, seed, 1, 7)
    want = oracle.fp4_expert_forward(w1, w3, w2, x)
    assert np.array_equal(bits(got), bits(want))


def test_routed_six_experts_bit_exact_and_within_tolerance(ctx, oracle):
    """One token through 6 routed experts (the headline workload's math)."""
    seed = 2
    idx, w, x = wl.moe_token_case(seed)
    routes = [(3, int(e), float(wt)) for e, wt in zip(idx, w)]
    for _, e, _ in routes:
        ctx.store_expert_synthetic(3, e, wl.HIDDEN, wl.INTER, seed)
    got = ctx.routed_experts(routes, x)
    outs = []
    for _, e, _ in routes:
        w1, w3, w2 = wl.synth_expert_host(ctx.lib, seed, 3, e)
        outs.append(oracle.fp4_expert_forward(w1, w3, w2, x))
    want = oracle.routed_combine(np.stack(outs), w)
    assert np.array_equal(bits(got), bits(want))


def test_routed_generic_shapes_and_weight_rules(ctx, oracle):
    """Odd expert shapes take the generic kernels; weights follow
    valid_route_weight_sum (invalid -> uniform, single expert unweighted)."""
    rng = np.random.default_rng(9)
    hidden, inter = 96, 40
    mats = []
    for e in range(3):
        m = []
        for rows, cols in ((inter, hidden), (inter, hidden), (hidden, inter)):
            p = rng.integers(0, 256, (rows, cols // 2)).astype(np.uint8)
            s = rng.integers(118, 130, (rows, cols // 8)).astype(np.uint8)
            m.append((p, s, rows, cols, cols // 8))
        mats.append(m)
        ex = wohper_amd.DeepSeekV4Fp4Expert(*[wohper_amd.Fp4Matvec(*t) for t in m])
        ctx.store_fp4_expert(9, e, ex)
    x = rng.standard_normal(hidden).astype(np.float32)
    outs = np.stack([oracle.fp4_expert_forward(*m, x) for m in mats])
    for weights in ([0.5, 0.3, 0.2], [np.nan, 1.0, 1.0], [0.0, 0.0, 0.0]):
        got = ctx.routed_experts([(9, e, wt) for e, wt in enumerate(weights)], x)
        want = oracle.routed_combine(outs, weights)
        assert np.array_equal(bits(got), bits(want)), weights
    got = ctx.routed_experts([(9, 1, 0.25)], x)
    assert np.array_equal(bits(got), bits(outs[1]))


def test_missing_expert_is_reported(ctx):
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.routed_experts([(99, 99, 1.0)], np.zeros(wl.HIDDEN, np.float32))
    assert e.value.name == "NotResident"
