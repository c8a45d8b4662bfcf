"""Pins the oracle's activation quant-dequant (E/compute.rs:2504-2545): the
reference's known answers, brute-force nearest search over the E4M3 grid with
ties to the lower value, the power-of-two block scale, and idempotence."""
import json
import math
from pathlib import Path

import numpy as np

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def test_known_answers(oracle):
    k = KATS["act_quant_representable"]
    out = oracle.act_quant(k["values"], k["block"])
    assert np.all(np.abs(out - np.array(k["expected"])) < k["tol"])
    k = KATS["act_quant_grid"]
    out = oracle.act_quant(k["values"], k["block"])
    assert abs(out[0] - k["first"]) < 1e-3
    assert any(abs(out[1] - v) < 1e-3 for v in k["second_in"]) and out[1] != 300.0


def brute_nearest(grid64, t):
    d = np.abs(grid64 - t)
    best = d.min()
    return grid64[d == best].min()  # ties -> the lower value


def test_nearest_is_brute_force_argmin_with_ties_low(oracle):
    _, _, _, srt = oracle.luts()
    grid = np.unique(srt.astype(np.float64))
    grid = grid[np.abs(grid) <= 448]
    # every midpoint (the tie cases), every grid point, and random targets
    mids = (grid[1:] + grid[:-1]) / 2
    rng = np.random.default_rng(0)
    targets = np.concatenate([grid, mids, rng.uniform(-448, 448, 4000), rng.uniform(-0.02, 0.02, 2000),
                              np.nextafter(mids.astype(np.float32), np.float32(np.inf)).astype(np.float64),
                              np.nextafter(mids.astype(np.float32), np.float32(-np.inf)).astype(np.float64)])
    targets = targets.astype(np.float32)
    for t in targets:
        got = oracle.nearest_e4m3(float(t))
        assert got == brute_nearest(grid, float(t)), t
    # zero results are +0.0 (the LUT's zeros are +0.0)
    assert not math.copysign(1.0, oracle.nearest_e4m3(-1e-9)) < 0


def test_scale_is_power_of_two_ceiling(oracle):
    rng = np.random.default_rng(1)
    amax = np.concatenate([np.exp(rng.uniform(-12, 12, 5000)), [1e-4, 5e-5, 448.0, 3.5, 2.0, 0.0]]).astype(np.float32)
    for a in amax:
        s = oracle.act_quant_scale(float(a))
        r = np.float32(max(np.float32(a), np.float32(1e-4))) / np.float32(448.0)
        k = math.ceil(math.log2(float(r)))
        # away from exact powers of two the ceiling is unambiguous
        if abs(math.log2(float(r)) - round(math.log2(float(r)))) > 1e-5:
            assert s == math.ldexp(1.0, k), a
        else:
            assert s in (math.ldexp(1.0, round(math.log2(float(r)))), math.ldexp(1.0, round(math.log2(float(r))) + 1))


def test_outputs_on_grid_and_idempotent(oracle):
    fp8, _, _, _ = oracle.luts()
    grid = set(np.float64(v) for v in fp8)
    rng = np.random.default_rng(2)
    for scale in (1e-3, 1.0, 37.0, 1e4):
        x = (rng.standard_normal(512) * scale).astype(np.float32)
        q = oracle.act_quant(x, 64)
        for b in range(0, 512, 64):
            blk = q[b: b + 64]
            s = oracle.act_quant_scale(float(np.max(np.abs(x[b: b + 64]))))
            assert all(np.float64(v) / s in grid for v in blk)
        assert np.array_equal(oracle.act_quant(q, 64), q)
        # the quantisation error is at most half an E4M3 step (relative 1/16) plus the subnormal floor
        assert np.all(np.abs(q - x) <= np.abs(x) / 16 + 2.0 ** -10 * np.max(np.abs(x)) / 448 * 2 + 1e-30)


def test_block_boundaries_are_independent(oracle):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(200).astype(np.float32)
    x[64:128] *= 1000
    q = oracle.act_quant(x, 64)
    assert np.array_equal(q[:64], oracle.act_quant(x[:64], 64))
    assert np.array_equal(q[128:], oracle.act_quant(x[128:], 64))  # ragged last block of 8
