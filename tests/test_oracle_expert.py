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
