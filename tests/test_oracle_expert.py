"""Pins the oracle's expert forward and routed sum: the reference's tiny
expert known answers, its error cases, and the weighting rules of
compute_active_experts (E/compute.rs:1948-2030)."""
import json
from pathlib import Path

import numpy as np
import pytest

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def _m(d):
    return (np.array(d["packed"], np.uint8), np.array(d["scales"], np.uint8), d["rows"], d["cols"], d["scale_cols"])


def test_tiny_expert_known_answer(oracle):
    k = KATS["tiny_expert"]
    y = oracle.fp4_expert_forward(_m(k["w1"]), _m(k["w3"]), _m(k["w2"]), k["input"], scratch_len=k["scratch"])
    # silu(2) * 3 through the act-quant of the hidden (deepseek_v4.rs:863-865)
    h = np.float32(2.0) / (np.float32(1.0) + np.exp(np.float32(-2.0))) * np.float32(3.0)
    hq = oracle.act_quant([h], 64)[0]
    assert abs(y[0] - hq) < k["tol"] and abs(y[1] - 2 * hq) < k["tol"]


def test_tiny_expert_rejects_small_scratch(oracle):
    k = KATS["tiny_expert"]
    with pytest.raises(oracle.OracleError) as e:
        oracle.fp4_expert_forward(_m(k["w1"]), _m(k["w3"]), _m(k["w2"]), k["input"],
                                  scratch_len=KATS["tiny_expert_small_scratch"]["scratch"])
    assert e.value.code == 7


def test_swiglu_clamps(oracle):
    # gate clamped from above at 10, up on both sides (E/deepseek_v4.rs:590-594)
    assert oracle.swiglu(50.0, 1.0) == oracle.swiglu(10.0, 1.0)
    assert oracle.swiglu(1.0, 50.0) == oracle.swiglu(1.0, 10.0)
    assert oracle.swiglu(1.0, -50.0) == oracle.swiglu(1.0, -10.0)
    assert oracle.swiglu(-50.0, 1.0) != oracle.swiglu(-10.0, 1.0)
    assert oracle.silu(0.0) == 0.0
    assert abs(oracle.silu(1.0) - 1.0 / (1.0 + np.exp(-1.0))) < 1e-7


def test_routed_weighting_rules(oracle):
    rng = np.random.default_rng(4)
    y = rng.standard_normal((2, 8)).astype(np.float32)
    w = KATS["route_weighted_sum"]["weights"]
    out = oracle.routed_combine(y, w)
    expect = np.zeros(8, np.float32)
    for e in range(2):
        expect = expect + y[e] * np.float32(w[e] / np.float32(sum(w)))
    assert np.array_equal(out, expect)
    # one expert: no weight applied (E/compute.rs:1959-1965)
    assert np.array_equal(oracle.routed_combine(y[:1], [0.1]), y[0])
    # invalid or vanishing weights fall back to uniform (E/compute.rs:2014-2030)
    uni = oracle.routed_combine(y, [np.nan, 1.0])
    assert np.allclose(uni, y[0] * 0.5 + y[1] * 0.5, rtol=0, atol=1e-7)
    assert oracle.route_weight_sum([0.0, 0.0]) is None
    assert oracle.route_weight_sum([-1.0, 2.0]) is None
    assert oracle.route_weight_sum([0.25, 0.5]) == 0.75
    # weights renormalise: scaling them changes nothing
    assert np.array_equal(oracle.routed_combine(y, [0.5, 0.5]), oracle.routed_combine(y, [2.0, 2.0]))


def test_accumulate_expert_for_positions(oracle):
    acc = np.zeros((3, 4), np.float32)
    y = np.ones((2, 4), np.float32)
    out = oracle.accumulate_expert(y, [2, 0], [0.5, 0.25], acc)
    assert np.array_equal(out[2], np.full(4, 0.5, np.float32))
    assert np.array_equal(out[0], np.full(4, 0.25, np.float32))
    assert np.array_equal(out[1], np.zeros(4, np.float32))


def test_batch_route_weights_rules(oracle):
    """The batch union's weights (E/server/generation.rs:2491-2503) differ from
    valid_route_weight_sum: negative scores and tiny sums pass, only a sum
    that is not finite and positive or a non-finite score goes uniform."""
    f = oracle.batch_route_weights
    assert f([[0.75, 0.25]]).tolist() == [[0.75, 0.25]]
    assert f([[-0.5, 1.0]]).tolist() == [[-1.0, 2.0]]
    assert f([[1e-30, 0.0]]).tolist() == [[1.0, 0.0]]
    assert f([[0.3]]).tolist() == [[1.0]]
    for bad in ([np.nan, 1.0], [np.inf, 1.0], [0.0, 0.0], [-1.0, -1.0], [3e38, 3e38], [1.0, -1.0]):
        assert f([bad]).tolist() == [[0.5, 0.5]], bad
    rng = np.random.default_rng(1)
    s = rng.uniform(0.01, 1.0, (64, 6)).astype(np.float32)
    w = f(s)
    assert np.allclose(w.sum(axis=1), 1.0, rtol=0, atol=4e-7)
    ratio = w / s
    assert np.allclose(ratio, ratio[:, :1], rtol=2e-7, atol=0)


def _small_expert(rng, hidden=64, inter=32):
    mats = []
    for rows, cols in ((inter, hidden), (inter, hidden), (hidden, inter)):
        p = rng.integers(0, 256, (rows, cols // 2)).astype(np.uint8)
        s = rng.integers(120, 132, (rows, cols // 32)).astype(np.uint8)
        mats.append((p, s, rows, cols, cols // 32))
    return tuple(mats)


def test_moe_batch_order_and_independence(oracle):
    """Experts are taken in ascending id whatever the route order, positions
    do not mix, and a position's result is its weighted expert sum."""
    rng = np.random.default_rng(5)
    experts = {e: _small_expert(rng) for e in range(8)}
    ids = np.array([[5, 1, 7, 2], [0, 3, 6, 4], [2, 7, 1, 5]], np.uint32)
    sc = rng.uniform(0.1, 1.0, ids.shape).astype(np.float32)
    x = (rng.standard_normal((3, 64)) * 4).astype(np.float32)
    out = oracle.moe_batch(experts, ids, sc, x)
    # the same routes listed in another order give the same bits
    perm = np.array([3, 0, 2, 1])
    assert np.array_equal(oracle.moe_batch(experts, ids[:, perm], sc[:, perm], x).view(np.uint32),
                          out.view(np.uint32))
    # positions are independent
    for p in range(3):
        one = oracle.moe_batch(experts, ids[p:p + 1], sc[p:p + 1], x[p:p + 1])
        assert np.array_equal(one.view(np.uint32), out[p:p + 1].view(np.uint32))
    # ... and each is the weighted sum of its experts' outputs
    w = oracle.batch_route_weights(sc)
    for p in range(3):
        ys = np.stack([oracle.fp4_expert_forward(*experts[int(e)], x[p]) for e in ids[p]]).astype(np.float64)
        want = (ys * w[p][:, None]).sum(axis=0)
        assert np.allclose(out[p], want, rtol=1e-5, atol=1e-5 * np.abs(ys).max())
    # summing in route order instead changes some bits on this case, so the
    # permutation check above is a real constraint
    route_order = np.zeros_like(x)
    for p in range(3):
        for k in range(4):
            y = oracle.fp4_expert_forward(*experts[int(ids[p, k])], x[p])
            route_order[p] = route_order[p] + y * w[p, k]
    assert not np.array_equal(route_order.view(np.uint32), out.view(np.uint32))
    # the shared expert adds after the routed sum
    sh = _small_expert(rng)
    with_sh = oracle.moe_batch(experts, ids, sc, x, shared=sh)
    for p in range(3):
        ys = oracle.fp4_expert_forward(*sh, x[p])
        assert np.array_equal((ys + out[p]).view(np.uint32), with_sh[p].view(np.uint32))


def _fp8_shared_kat():
    """A sparse FP8 shared expert whose output follows in closed form
    (hidden = inter = 128, one 128x128 block, scales 1):
      w1[0,0] = 1, w3[0,0] = 1.5, w2[5,0] = 2 and w1[1,1] = w3[1,1] = w2[6,1] = 1;
      x[0] = 2, x[1] = 0.3.
    act_quant(x) (block 64): scale 2^ceil(log2(2/448)) = 2^-7, so x0 -> 256 * 2^-7
    = 2 and x1 -> 38.4 -> nearest E4M3 40 -> 0.3125.  gate = (2, 0.3125),
    up = (3, 0.3125); h0 = silu(2) * 3 = 5.28478, h1 = silu(0.3125) * 0.3125
    = 0.0563938.  act_quant(h): scale 2^ceil(log2(5.28478/448)) = 2^-6; h0 * 64
    = 338.23 -> 352 (grid step 32) -> 5.5; h1 * 64 = 3.6092 -> 3.5 (step 0.25)
    -> 0.0546875.  y[5] = 2 * 5.5 = 11, y[6] = 0.0546875, every other y is 0."""
    n = 128
    w1 = np.zeros((n, n), np.uint8)
    w3 = np.zeros((n, n), np.uint8)
    w2 = np.zeros((n, n), np.uint8)
    w1[0, 0], w3[0, 0], w2[5, 0] = 0x38, 0x3C, 0x40  # E4M3 1.0, 1.5, 2.0
    w1[1, 1], w3[1, 1], w2[6, 1] = 0x38, 0x38, 0x38
    x = np.zeros(n, np.float32)
    x[0], x[1] = 2.0, 0.3
    want = np.zeros(n, np.float32)
    want[5], want[6] = 11.0, 0.0546875
    return w1, w3, w2, np.ones((1, 1), np.float32), x, want


def test_fp8_shared_expert_closed_form(oracle):
    """Pins the stage order of E/compute.rs:5585-5612: a swapped w1/w3
    (silu(3) * 2), a skipped act-quant of x (x1 stays 0.3) or of h (y5 =
    10.57) each changes the result."""
    w1, w3, w2, s, x, want = _fp8_shared_kat()
    got = oracle.fp8_shared_expert(w1, s, w3, s, w2, s, 128, 128, x)
    assert np.array_equal(got, want)
