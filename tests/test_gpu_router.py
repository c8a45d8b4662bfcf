"""GPU parity of the router (wh_store_router / wh_route_experts[_async]) with
the oracle's restatement of route_experts_from_dense_block
(E/compute.rs:2129-2268): gate GEMV in the AVX2 lane order, sqrt-softplus
with glibc's expf/log1pf and the IEEE sqrt, biased stable top-k, hash layers,
finalized weights - ids and weights bit-exact.  Plus the reference's router
tests as known answers and its error cases."""
import json
from pathlib import Path

import numpy as np
import pytest

import wohper_amd
import zcblk
from parity_util import bits
from wohper_amd import workloads as wl

pytestmark = pytest.mark.gpu

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())
ROLE_ROUTER = 9
SP, RAW = wohper_amd.ROUTER_SQRT_SOFTPLUS, wohper_amd.ROUTER_RAW_LOGITS


def _bf16_bits(values):
    return (np.asarray(values, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def _gate_t(w_bits, name="layers.3.ffn.gate.weight"):
    w = np.ascontiguousarray(w_bits, np.uint16)
    return zcblk.tensor(name, w.shape, w.view(np.uint8).reshape(-1), 2404, ROLE_ROUTER, 11)


def _bias_t(bias, name="layers.3.ffn.gate.bias", dtype=12):
    b = np.asarray(bias, np.float32)
    data = b.view(np.uint8) if dtype == 12 else _bf16_bits(b).view(np.uint8)
    return zcblk.tensor(name, (b.size,), data, 2405, ROLE_ROUTER, dtype)


def _table_t(table, name="layers.0.ffn.gate.tid2eid", dtype=9):
    t = np.asarray(table, np.int64 if dtype == 9 else np.int32)
    return zcblk.tensor(name, t.shape, t.view(np.uint8).reshape(-1), 2406, ROLE_ROUTER, dtype)


def _oracle_routes(oracle, logits, active, available=None, bias=None, math=SP, route_scale=1.5, hash_ids=None):
    return oracle.route_select(logits, active, available, bias=bias, math=math, route_scale=route_scale,
                               hash_ids=hash_ids)


def _same(got, want):
    assert np.array_equal(got[0], want[0]), (got[0], want[0])
    assert np.array_equal(bits(got[1]), bits(want[1])), (got[1], want[1])


def test_router_known_answers(ctx, oracle):
    k = KATS["router"]
    gate = _gate_t(_bf16_bits(k["gate"]))
    # raw logits; a tid2eid table with other cols ahead of the gate is skipped
    blk = zcblk.build_block([_table_t([[1, 1, 1]] * 4, "layers.3.ffn.gate.tid2eid"), gate])
    assert ctx.store_router(50, blk, 2)
    ids, _ = ctx.route_experts(50, k["hidden"], k["raw_logits"]["active"], k["available"], math=RAW)
    assert list(ids) == k["raw_logits"]["ids"]
    # sqrt-softplus weights
    assert ctx.store_router(51, zcblk.build_block([gate]), 2)
    ids, w = ctx.route_experts(51, k["hidden"], 2, k["available"], route_scale=k["route_scale"])
    assert list(ids) == k["sqrt_softplus"]["ids"] and abs(float(w.sum()) - k["sqrt_softplus"]["total"]) < k["tol"]
    _same((ids, w), _oracle_routes(oracle, [1.0, 4.0], 2, k["available"]))
    # the bias moves the selection, not the weights
    assert ctx.store_router(52, zcblk.build_block([gate, _bias_t(k["bias"]["bias"])]), 2)
    ids, w = ctx.route_experts(52, k["hidden"], 1, k["available"], route_scale=k["route_scale"])
    assert list(ids) == k["bias"]["ids"] and list(w) == k["bias"]["weights"]
    # hash layer
    h = k["hash"]
    assert ctx.store_router(53, zcblk.build_block([_table_t(h["tid2eid"]), gate]), 2)
    ids, w = ctx.route_experts(53, k["hidden"], 2, k["available"], route_scale=k["route_scale"], hash_token_id=h["token"])
    assert list(ids) == h["ids"] and abs(float(w.sum()) - h["total"]) < k["tol"]
    # no gate: Ok(None)
    assert not ctx.store_router(54, zcblk.build_block([_bias_t([0.0, 0.0])]), 2)


def _model_router(seed, rows=256, cols=4096, table_rows=0):
    rng = np.random.default_rng(seed)
    gate = _bf16_bits(rng.standard_normal((rows, cols)).astype(np.float32) * 0.02)
    bias = (rng.standard_normal(rows) * 0.05).astype(np.float32)
    ts = [_gate_t(gate), _bias_t(bias)]
    table = None
    if table_rows:
        table = np.stack([rng.permutation(rows)[:6] for _ in range(table_rows)]).astype(np.int64)
        ts.insert(0, _table_t(table))
    return gate, bias, table, zcblk.build_block(ts)


@pytest.mark.parametrize("cols", [4096, 7168, 200])
def test_router_bit_exact_model_shape(ctx, oracle, cols):
    """256 experts, DeepSeek-V4 math (route_scale 1.5, bias), 40 tokens."""
    gate, bias, _, blk = _model_router(7 + cols, 256, cols)
    assert ctx.store_router(60, blk, cols)
    rng = np.random.default_rng(cols)
    for t in range(40):
        x = wl.bf16_round(rng.standard_normal(cols).astype(np.float32) * (4.0 if t % 5 == 0 else 1.0))
        logits = oracle.bf16_gemv(gate, x)
        got = ctx.route_experts(60, x, 6, route_scale=1.5)
        _same(got, _oracle_routes(oracle, logits, 6, bias=bias))
        got = ctx.route_experts(60, x, 8, math=RAW)
        _same(got, _oracle_routes(oracle, logits, 8, math=RAW))


def test_router_hash_layer_and_available_lists(ctx, oracle):
    gate, bias, table, blk = _model_router(11, 256, 4096, table_rows=500)
    assert ctx.store_router(61, blk, 4096)
    rng = np.random.default_rng(12)
    for t in range(20):
        x = rng.standard_normal(4096).astype(np.float32)
        logits = oracle.bf16_gemv(gate, x)
        avail = rng.permutation(300)[:rng.integers(1, 300)]  # ids past 255 have no score
        token = int(rng.integers(0, 500))
        got = ctx.route_experts(61, x, 6, avail, route_scale=1.5, hash_token_id=token)
        _same(got, _oracle_routes(oracle, logits, 6, avail, hash_ids=table[token]))
        got = ctx.route_experts(61, x, 6, avail, route_scale=1.5)
        _same(got, _oracle_routes(oracle, logits, 6, avail, bias=bias))
    assert ctx.route_experts(61, x, 0)[0].size == 0
    assert ctx.route_experts(61, x, 6, np.zeros(0, np.uint32))[0].size == 0


def test_router_ties_nan_and_uniform_fallback(ctx, oracle):
    rows, cols = 64, 128
    rng = np.random.default_rng(3)
    gate = rng.standard_normal((rows, cols)).astype(np.float32)
    gate[10] = gate[3]
    gate[40] = gate[3]  # equal logits: available order decides
    gate[20] = 0.0      # logit exactly 0
    g = _bf16_bits(gate)
    assert ctx.store_router(62, zcblk.build_block([_gate_t(g)]), cols)
    x = rng.standard_normal(cols).astype(np.float32)
    logits = oracle.bf16_gemv(g, x)
    for avail in (None, rng.permutation(rows), np.array([40, 10, 3, 20, 1, 2, 5], np.uint32)):
        for math in (SP, RAW):
            _same(ctx.route_experts(62, x, 5, avail, math=math, route_scale=1.5),
                  _oracle_routes(oracle, logits, 5, avail, math=math))
    x_nan = x.copy()
    x_nan[7] = np.nan  # every logit NaN: sqrt-softplus scores 0, weights uniform
    got = ctx.route_experts(62, x_nan, 4, route_scale=1.5)
    want = _oracle_routes(oracle, oracle.bf16_gemv(g, x_nan), 4)
    _same(got, want)
    assert np.all(got[1] == np.float32(1.5 / 4))


def test_router_one_launch_selection_ties(ctx, oracle):
    """256 rows, no available list: the one-launch selection, which finds
    the selected set by a search for its smallest key and falls back to
    one candidate per round when equal keys straddle that boundary.  Rows
    5, 77 and 200 tie for first (ordered by row inside the set), 9 and 130
    tie for sixth and seventh (the boundary at 6 active)."""
    rows, cols = 256, 128
    rng = np.random.default_rng(21)
    x = wl.bf16_round(rng.standard_normal(cols).astype(np.float32))
    gate = rng.standard_normal((rows, cols)).astype(np.float32) * 0.01
    for r, a in ((200, 1.0), (5, 1.0), (77, 1.0), (33, 0.75), (150, 0.625), (130, 0.5), (9, 0.5)):
        gate[r] = np.sign(x) * a
    g = _bf16_bits(gate)
    assert ctx.store_router(65, zcblk.build_block([_gate_t(g)]), cols)
    logits = oracle.bf16_gemv(g, x)
    order = np.argsort(-logits, kind="stable")
    assert list(order[:7]) == [5, 77, 200, 33, 150, 9, 130] and logits[9] == logits[130] and logits[5] == logits[200]
    for active in (1, 3, 5, 6, 7, 8, 64):
        for math in (SP, RAW):
            _same(ctx.route_experts(65, x, active, math=math, route_scale=1.5),
                  _oracle_routes(oracle, logits, active, math=math))


@pytest.mark.parametrize("exact", [True, False])
def test_router_fp8_gate(ctx, oracle, exact):
    """An FP8 gate: ids and weights bit-exact in both numerics modes (the
    gate GEMV keeps the reference's order even with exact numerics off: a
    top-k has no tolerance)."""
    ctx.set_exact_numerics(exact)
    try:
        _router_fp8_gate(ctx, oracle)
    finally:
        ctx.set_exact_numerics(True)


def _router_fp8_gate(ctx, oracle):
    rows, cols = 256, 4096
    rng = np.random.default_rng(9)
    c = rng.integers(0, 254, (rows, cols))
    w = np.where(c < 127, c, c + 1).astype(np.uint8)  # the finite E4M3 codes (0x7f, 0xff excluded)
    sexp = rng.integers(117, 124, (rows // 128, cols // 128)).astype(np.uint8)
    ts = [zcblk.tensor("layers.9.ffn.gate.weight", (rows, cols), w, 2401, ROLE_ROUTER, 101),
          zcblk.tensor("layers.9.ffn.gate.scale", sexp.shape, sexp, 2403, ROLE_ROUTER, 102)]
    assert ctx.store_router(63, zcblk.build_block(ts), cols)
    x = rng.standard_normal(cols).astype(np.float32)
    s_f32 = oracle.decode_ue8m0(sexp.reshape(-1)).reshape(sexp.shape)
    logits = oracle.fp8_gemv(w, rows, cols, s_f32, rows // 128, cols // 128, x)
    _same(ctx.route_experts(63, x, 6, route_scale=1.5), _oracle_routes(oracle, logits, 6))


def test_router_async_matches_sync(ctx, oracle):
    gate, bias, table, blk = _model_router(21, 256, 4096, table_rows=64)
    assert ctx.store_router(64, blk, 4096)
    x = np.random.default_rng(22).standard_normal(4096).astype(np.float32)
    want = ctx.route_experts(64, x, 6, route_scale=1.5)
    want_h = ctx.route_experts(64, x, 6, route_scale=1.5, hash_token_id=17)
    xd = ctx.device_alloc(x.nbytes)
    out = ctx.device_alloc(6 * 8 + 4)
    ctx.to_device(xd, x)
    for hash_id, ref in ((None, want), (17, want_h)):
        ctx.route_experts_async(64, xd, 4096, 6, 0, 0, out, out + 24, out + 48, route_scale=1.5, hash_token_id=hash_id)
        ctx.synchronize()
        buf = np.zeros(13, np.uint32)
        ctx.from_device(buf, out)
        n = int(buf[12])
        assert n == ref[0].size
        assert np.array_equal(buf[:n], ref[0]) and np.array_equal(buf[6:6 + n], bits(ref[1]))
    ctx.device_free(xd)
    ctx.device_free(out)


def test_router_errors(ctx):
    k = KATS["router"]
    gate = _gate_t(_bf16_bits(k["gate"]))

    def err(fn):
        with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
            fn()
        return e.value.name, e.value.detail

    assert ctx.store_router(70, zcblk.build_block([_table_t([[0, -1], [1, 0]]), gate]), 2)
    assert err(lambda: ctx.route_experts(70, [1.0, 2.0], 2, hash_token_id=0)) == (
        "InvalidShape", "invalid compute shape: tid2eid negative expert id")
    assert err(lambda: ctx.route_experts(70, [1.0, 2.0], 2, hash_token_id=2)) == (
        "InvalidShape", "invalid compute shape: tid2eid token id out of range")
    assert list(ctx.route_experts(70, [1.0, 2.0], 1, hash_token_id=1)[0]) == [1]
    assert err(lambda: ctx.route_experts(70, [1.0], 1)) == ("InvalidShape", "invalid compute shape: router input too small")
    t8 = zcblk.tensor("layers.0.ffn.gate.tid2eid", (2, 2), np.zeros(4, np.uint8), 2406, ROLE_ROUTER, 1)
    assert ctx.store_router(71, zcblk.build_block([t8, gate]), 2)
    assert err(lambda: ctx.route_experts(71, [1.0, 2.0], 1, hash_token_id=0)) == (
        "InvalidShape", "invalid compute shape: tid2eid table has unsupported dtype")
    # a short bias fails the DeepSeek math only
    short = zcblk.tensor("layers.3.ffn.gate.bias", (2,), np.zeros(4, np.uint8), 2405, ROLE_ROUTER, 12)
    assert ctx.store_router(72, zcblk.build_block([gate, short]), 2)
    assert err(lambda: ctx.route_experts(72, [1.0, 2.0], 1)) == ("InvalidShape", "invalid compute shape: router bias out of range")
    assert list(ctx.route_experts(72, [1.0, 2.0], 1, math=RAW)[0]) == [1]
    assert err(lambda: ctx.route_experts(99, [1.0, 2.0], 1))[0] == "NotResident"
    int4 = zcblk.tensor("layers.3.ffn.gate.weight", (2, 2), np.zeros(2, np.uint8), 4, ROLE_ROUTER, 12)
    assert err(lambda: ctx.store_router(73, zcblk.build_block([int4]), 2))[0] == "Unsupported"


def test_router_libm_pieces_bit_exact(ctx, oracle):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.uniform(-30, 30, 2_000_000), rng.standard_normal(1_000_000) * 5,
                        np.linspace(-20.5, 20.5, 1_000_001)]).astype(np.float32)
    x = np.concatenate([x, np.array([-20.0, 20.0, np.nan, np.inf, -np.inf, 0.0, -0.0, -104.5, -88.0], np.float32)])
    assert np.array_equal(bits(ctx.debug_eval(4, x)), bits(oracle.sqrt_softplus(x)))
    y = np.abs(rng.standard_normal(2_000_000) * np.exp(rng.uniform(-25, 25, 2_000_000))).astype(np.float32)
    y = np.concatenate([y, np.array([0.0, 1e-30, 0.41421, 0.41422, 1e30, np.inf], np.float32)])
    assert np.array_equal(bits(ctx.debug_eval(5, y)), bits(oracle.log1pf(y)))
    # expf over the whole line, subnormal results included
    z = np.concatenate([rng.uniform(-110, 90, 2_000_000), rng.uniform(-104, -87, 1_000_000)]).astype(np.float32)
    want = np.empty_like(z)
    oracle.lib().or_expf_array(oracle._pf(z), oracle._pf(want), z.size)
    assert np.array_equal(bits(ctx.debug_eval(6, z)), bits(want))
    # the square root is the IEEE one
    v = np.abs(rng.standard_normal(4_000_000) * np.exp(rng.uniform(-40, 40, 4_000_000))).astype(np.float32)
    sq = ctx.debug_eval(4, np.full(1, 25.0, np.float32))
    assert sq[0] == np.float32(5.0)
    got = ctx.debug_eval(4, v + np.float32(21.0))  # v > 20: sqrt(v)
    assert np.array_equal(bits(got), bits(np.sqrt(v + np.float32(21.0))))
