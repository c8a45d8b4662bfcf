"""CPU pinning of the oracle's router restatement (route_experts_from_dense_block,
E/compute.rs:2129-2268, and the bf16 gate GEMV, E/compute.rs:2910-2941, 6116-6172).

* the reference's router tests (compute.rs:8025-8295) as known answers;
* the bf16 dot row against float64 (the reference's own test, compute.rs:7436-7453)
  and against an independent float32 evaluation of the AVX2 lane order;
* sqrt-softplus against float64 within one float ulp, its branch points
  (+-20) exactly, and log1pf against float64 within one ulp;
* selection against a brute-force sort: stable, total order, NaN and -0."""
import json
from pathlib import Path

import numpy as np
import pytest

from conftest import lcg_f32

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def _bf16_bits(values):
    return (np.asarray(values, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def _bf16_values(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def test_router_known_answers(oracle):
    k = KATS["router"]
    logits = oracle.bf16_gemv(_bf16_bits(k["gate"]), k["hidden"])
    assert list(logits) == [1.0, 4.0]
    ids, w = oracle.route_select(logits, k["raw_logits"]["active"], k["available"], math=oracle.ROUTER_RAW_LOGITS)
    assert list(ids) == k["raw_logits"]["ids"]
    ids, w = oracle.route_select(logits, k["sqrt_softplus"]["active"], k["available"], route_scale=k["route_scale"])
    assert list(ids) == k["sqrt_softplus"]["ids"]
    s0, s1 = np.sqrt(np.log1p(np.exp(1.0))), np.sqrt(np.log1p(np.exp(4.0)))
    assert abs(w[0] - s1 / (s0 + s1) * 1.5) < k["tol"] and abs(w[1] - s0 / (s0 + s1) * 1.5) < k["tol"]
    assert abs(float(w.sum()) - k["sqrt_softplus"]["total"]) < k["tol"]
    b = k["bias"]
    ids, w = oracle.route_select(logits, b["active"], k["available"], bias=b["bias"], route_scale=k["route_scale"])
    assert list(ids) == b["ids"] and list(w) == b["weights"]
    h = k["hash"]
    row = h["tid2eid"][h["token"]]
    ids, w = oracle.route_select(logits, h["active"], k["available"], hash_ids=row, route_scale=k["route_scale"])
    assert list(ids) == h["ids"] and abs(float(w.sum()) - h["total"]) < k["tol"]


def test_bf16_dot_row_known_answer_and_lane_order(oracle):
    k = KATS["bf16_dot_row"]
    x = lcg_f32(k["input_seed"], k["count"])
    w = _bf16_bits(lcg_f32(k["values_seed"], k["count"]))
    got = oracle.bf16_gemv(w[None, :], x)[0]
    ref = float(np.sum(_bf16_values(w).astype(np.float64) * x.astype(np.float64)))
    assert abs(got - ref) <= k["tol"] * max(abs(ref), 1.0)
    # the AVX2 order, evaluated independently in float32 with products that
    # are exact (small integers), so only the summation order decides:
    # lane l of acc0/acc1 sums columns 16c+l / 16c+8+l, then
    # ((s0+s1)+(s2+s3))+((s4+s5)+(s6+s7)) of s = acc0+acc1, plus the tail
    rng = np.random.default_rng(3)
    cols = 16 * 5 + 3
    big = rng.integers(-2 ** 12, 2 ** 12, cols).astype(np.float32) * np.float32(2.0 ** 12)
    xs = np.where(rng.random(cols) < 0.5, np.float32(1.0), np.float32(2.0 ** -12)).astype(np.float32)
    wv = _bf16_values(_bf16_bits(big))
    acc = np.zeros((2, 8), np.float32)
    for c in range(cols // 16):
        for a in range(2):
            for l in range(8):
                i = 16 * c + 8 * a + l
                acc[a, l] = np.float32(np.float64(wv[i]) * np.float64(xs[i]) + np.float64(acc[a, l]))
    s = (acc[0] + acc[1]).astype(np.float32)
    want = np.float32(np.float32(np.float32(s[0] + s[1]) + np.float32(s[2] + s[3])) +
                      np.float32(np.float32(s[4] + s[5]) + np.float32(s[6] + s[7])))
    tail = np.float32(0.0)
    for i in range(cols // 16 * 16, cols):
        tail = np.float32(tail + np.float32(wv[i] * xs[i]))
    want = np.float32(want + tail)
    got = oracle.bf16_gemv(_bf16_bits(big)[None, :], xs)[0]
    assert got.view(np.uint32) == want.view(np.uint32)


def test_sqrt_softplus_and_log1pf(oracle):
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.uniform(-25, 25, 200_000), rng.standard_normal(100_000) * 3,
                        [-20.0, 20.0, -20.000002, 20.000002, 0.0, -0.0, 1e-30, -1e-30, 88.0, -104.0, -1e4]])
    x = x.astype(np.float32)
    got = oracle.sqrt_softplus(x).astype(np.float64)
    xd = x.astype(np.float64)
    # below -20 the softplus is expf(v) itself, which underflows in f32
    sp = np.where(xd > 20, xd, np.where(xd < -20, np.exp(xd).astype(np.float32).astype(np.float64),
                                        np.log1p(np.exp(xd))))
    want = np.sqrt(np.maximum(sp, 0))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - want) <= 1.5 * ulp)
    # branch points: v > 20 returns sqrt(v) of v itself
    assert oracle.sqrt_softplus([25.0])[0] == np.float32(5.0)
    assert oracle.sqrt_softplus([np.nan])[0] == 0.0  # max(NaN, 0) = 0
    y = np.abs(rng.standard_normal(300_000) * np.exp(rng.uniform(-20, 20, 300_000))).astype(np.float32)
    l1 = oracle.log1pf(y).astype(np.float64)
    want = np.log1p(y.astype(np.float64))
    assert np.all(np.abs(l1 - want) <= np.spacing(want.astype(np.float32)).astype(np.float64))


def _brute_select(scores, bias, available, active):
    """sort by (score + bias) descending in f32 total order, ties kept in
    available order."""
    def key(v):
        b = np.float32(v).view(np.int32)
        return int(b ^ ((b >> 31) & 0x7FFFFFFF))
    cand = [(key(np.float32(scores[i] + (bias[i] if bias is not None else 0))), pos, i)
            for pos, i in enumerate(available) if i < len(scores)]
    cand.sort(key=lambda t: (-t[0], t[1]))
    return [i for _, _, i in cand[:active]]


@pytest.mark.parametrize("seed", range(6))
def test_selection_brute_force(oracle, seed):
    rng = np.random.default_rng(seed)
    rows = 256
    logits = rng.standard_normal(rows).astype(np.float32) * 3
    logits[rng.integers(0, rows, 20)] = logits[0]  # ties
    if seed % 2:
        logits[5] = np.nan
        logits[6] = -0.0
        logits[7] = 0.0
    bias = rng.standard_normal(rows).astype(np.float32) * 0.1 if seed % 3 else None
    available = rng.permutation(rows + 8)[:200]  # ids past rows are dropped
    active = 6
    ids, w = oracle.route_select(logits, active, available, bias=bias, route_scale=1.5)
    scores = oracle.sqrt_softplus(logits)
    assert list(ids) == _brute_select(scores, bias, available, active)
    sel = scores[ids]
    total = np.float32(0)
    for v in sel:
        total = np.float32(total + v)
    assert np.array_equal(w, (sel / total * np.float32(1.5)).astype(np.float32))
    ids_raw, w_raw = oracle.route_select(logits, active, available, bias=bias, math=oracle.ROUTER_RAW_LOGITS)
    assert list(ids_raw) == _brute_select(logits, None, available, active)  # raw math ignores the bias
    assert np.array_equal(w_raw.view(np.uint32), logits[ids_raw].view(np.uint32))


def test_finalize_uniform_fallback(oracle):
    # all selected scores 0 (logits far below -20 underflow to 0) -> uniform route_scale / n
    ids, w = oracle.route_select(np.full(8, -200.0, np.float32), 3, route_scale=1.5)
    assert list(ids) == [0, 1, 2] and np.all(w == np.float32(0.5))
    ids, w = oracle.route_select(np.zeros(4, np.float32), 0)
    assert ids.size == 0
