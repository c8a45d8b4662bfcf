"""GPU parity of the act-quant inside the LDS-streaming token kernels
(moe_tok.h) with the oracle's restatement of fp8_act_quant_dequant_in_place
(E/compute.rs:2504-2545, block 64), bit for bit.

The bf16 path writes E4M3 codes with the hardware conversion (round to
nearest even) of t - |t| 2^-12, which is the reference's nearest value with
ties toward -inf only because a bf16 input has 8 significant bits; these
cases pin it on every finite bf16 value, on every E4M3 midpoint and its
bf16 neighbours, and on the headline's N(0,1) inputs.  The f32 path (used
for h and f32 x) keeps the integer rounding and is pinned on f32 midpoints
and their f32 neighbours."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

BF16_PATH, F32_PATH = 7, 8


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def bf16_values(u16):
    return (np.asarray(u16, np.uint32) << 16).view(np.float32)


def _blocks(vals, lead=None):
    """vals padded with zeros to whole 64-blocks; lead: one value placed
    first in every block (sets the block's amax)."""
    per = 64 if lead is None else 63
    pad = (-vals.size) % per
    v = np.concatenate([vals.astype(np.float32), np.zeros(pad, np.float32)]).reshape(-1, per)
    if lead is not None:
        v = np.concatenate([np.full((v.shape[0], 1), lead, np.float32), v], axis=1)
    return v.reshape(-1)


def _check(ctx, oracle, fn, x):
    got = ctx.debug_eval(fn, x)
    want = oracle.act_quant(x, 64)
    bad = np.nonzero(bits(got) != bits(want))[0]
    assert bad.size == 0, f"{bad.size} values differ, first at {bad[0]}: x={x[bad[0]]!r} got={got[bad[0]]!r} " \
                          f"want={want[bad[0]]!r}"


def _finite_bf16():
    u = np.arange(1 << 16, dtype=np.uint32)
    u = u[((u >> 7) & 0xFF) != 0xFF]
    return bf16_values(u)


def test_bf16_every_finite_value(ctx, oracle):
    v = _finite_bf16()
    _check(ctx, oracle, BF16_PATH, _blocks(v))                     # blocks of neighbouring magnitudes
    _check(ctx, oracle, BF16_PATH, _blocks(np.random.default_rng(7).permutation(v)))  # mixed blocks
    for lead in (448.0, 1.0, 2.0 ** -20, 3.0e4):                   # every value under a fixed block scale
        small = v[np.abs(v) <= lead]
        _check(ctx, oracle, BF16_PATH, _blocks(small, lead))


def test_bf16_midpoints_and_neighbours(ctx, oracle):
    _, _, _, srt = oracle.luts()
    grid = np.unique(srt.astype(np.float64))
    grid = grid[np.abs(grid) <= 448]
    mids = ((grid[1:] + grid[:-1]) / 2).astype(np.float32)
    mb = (bits(mids) >> 16).astype(np.uint32)
    assert np.array_equal(bf16_values(mb), mids)  # E4M3 midpoints are bf16 values
    near = np.concatenate([mb, mb + 1, mb - 1]) & 0xFFFF
    vals = bf16_values(near)
    vals = vals[np.abs(vals) <= 448]
    for scale_exp in (0, -9, 5, -30):  # the same pattern under other block scales
        s = np.float32(2.0 ** scale_exp)
        _check(ctx, oracle, BF16_PATH, _blocks(vals * s, np.float32(448.0) * s))


def test_bf16_headline_inputs(ctx, oracle):
    rng = np.random.default_rng(2)
    for s in (1.0, 1e-3, 37.0):
        x = (rng.standard_normal(4096 * 16) * s).astype(np.float32)
        x = bf16_values(bits(x) >> 16)  # truncate to bf16 values
        x[::101] = 0.0
        x[3::103] = -0.0
        _check(ctx, oracle, BF16_PATH, x)


def test_f32_midpoints_neighbours_and_random(ctx, oracle):
    _, _, _, srt = oracle.luts()
    grid = np.unique(srt.astype(np.float64))
    grid = grid[np.abs(grid) <= 448]
    mids = ((grid[1:] + grid[:-1]) / 2).astype(np.float32)
    vals = np.concatenate([mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf))])
    _check(ctx, oracle, F32_PATH, _blocks(vals, 448.0))
    rng = np.random.default_rng(5)
    parts = [rng.standard_normal(4096) * s for s in (1e-6, 1e-3, 1.0, 30.0, 1e5)]
    x = np.concatenate(parts).astype(np.float32)
    x[::97] = 0.0
    _check(ctx, oracle, F32_PATH, x)
