"""UE8M0 scale bytes 0 and 255 on the MFMA paths.

decode_ue8m0_scale (E/deepseek_v4.rs:166-192) maps byte 0 to 0.0 and byte
255 to inf.  The block-scaled MFMA reads an E8M0 byte 0 as 2^-127 and 255 as
NaN, so FP4 experts with a byte 0 anywhere run on the exact kernels in every
numerics mode (their result is then the oracle's bit for bit, including rows
whose scales are all 0, which must come out exactly 0), while byte 255 makes
the output non-finite on both sides (NonFiniteOutput).  The multi-input FP8
MFMA decodes UE8M0 in software and is checked against the oracle within
tolerance with zero blocks, and for NonFiniteOutput with an infinite one."""
import numpy as np
import pytest

import wohper_amd
from parity_util import bits
from wohper_amd import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def restore_numerics(ctx):
    yield
    ctx.set_exact_numerics(True)
    ctx.debug_moe_token_capture(False)


def _store_host_expert(ctx, layer, e, ex):
    hs = [ctx.store_fp4(p, s, r, c, sc) for p, s, r, c, sc in ex]
    ctx.store_expert(layer, e, *hs)


def _edited(ex, edit):
    """A copy of a host expert ((packed, scales, rows, cols, scale_cols) x 3)
    with edit(m, scales) applied to each matrix's [rows, scale_cols] scales."""
    out = []
    for m, (p, s, r, c, sc) in enumerate(ex):
        s2 = np.array(s, np.uint8).reshape(r, sc).copy()
        edit(m, s2)
        out.append((p, s2.reshape(-1), r, c, sc))
    return tuple(out)


def _oracle_forward(oracle, experts, weights, x):
    outs = np.stack([oracle.fp4_expert_forward(*m, x) for m in experts])
    return oracle.routed_combine(outs, weights)


@pytest.mark.parametrize("exact", [False, True])
def test_fp4_token_scale_byte_zero(ctx, oracle, exact):
    seed, layer = 61, 23
    base = [wl.synth_expert_host(ctx.lib, seed, layer, e) for e in (0, 1)]

    def zero_rows(m, s):
        if m == 0:
            s[5, :] = 0            # gate row 5: every group scale 0 -> exactly 0
            s[::97, 3] = 0         # scattered zero groups
        if m == 2:
            s[::31, ::7] = 0

    experts = [_edited(base[0], zero_rows), _edited(base[1], lambda m, s: s.__setitem__((slice(None), 0), 0))]
    for e, ex in enumerate(experts):
        _store_host_expert(ctx, layer, e, ex)
    ctx.set_exact_numerics(exact)
    ctx.debug_moe_token_capture(True)
    x = wl.bf16_round(np.random.default_rng(seed).standard_normal(wl.HIDDEN).astype(np.float32))
    routes, w = [(layer, 0, 0.7), (layer, 1, 0.3)], [0.7, 0.3]
    got = ctx.routed_experts(routes, x)
    gu = ctx.debug_moe_token_read(0, (1, 2, 2, wl.INTER))[0]
    assert gu[0, 0, 5] == 0.0
    assert np.array_equal(bits(got), bits(_oracle_forward(oracle, [[m for m in ex] for ex in experts], w, x)))


def test_fp4_batch_scale_byte_zero(ctx, oracle):
    """The batch path with an expert holding zero scale bytes: every expert
    of the call on the exact items, bit-exact, in MFMA numerics."""
    seed, layer, n_exp = 62, 24, 12
    for e in range(n_exp):
        ctx.store_expert_synthetic(layer, e, wl.HIDDEN, wl.INTER, seed)
    ex3 = _edited(wl.synth_expert_host(ctx.lib, seed, layer, 3), lambda m, s: s.__setitem__((slice(0, 64), 2), 0))
    _store_host_expert(ctx, layer, 3, ex3)
    ids, sc, x = wl.zipf_batch_routes(seed=7, n_tokens=20, n_experts=n_exp)
    ids[0, 0] = 3
    experts = {int(e): wl.synth_expert_host(ctx.lib, seed, layer, int(e)) for e in np.unique(ids)}
    experts[3] = ex3
    ctx.set_exact_numerics(False)
    got = ctx.moe_batch(layer, ids, sc, x)
    want = oracle.moe_batch(experts, ids, sc, x)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("exact", [False, True])
def test_fp4_token_scale_byte_255(ctx, oracle, exact):
    seed, layer = 63, 25
    ex = _edited(wl.synth_expert_host(ctx.lib, seed, layer, 0), lambda m, s: s.__setitem__((7, 11), 255) if m == 1 else None)
    _store_host_expert(ctx, layer, 0, ex)
    x = wl.bf16_round(np.random.default_rng(seed).standard_normal(wl.HIDDEN).astype(np.float32))
    with pytest.raises(oracle.OracleError) as oe:
        oracle.fp4_expert_forward(*ex, x)
    assert oe.value.code == 8  # NonFiniteOutput
    ctx.set_exact_numerics(exact)
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.routed_experts([(layer, 0, 1.0)], x)
    assert e.value.name == "NonFiniteOutput"


def _ue8m0_f32(b):
    b = np.asarray(b, np.int32)
    return np.where(b == 0, 0.0, np.where(b == 255, np.inf, np.exp2((b - 127).astype(np.float64)))).astype(np.float32)


def test_fp8_mfma_ue8m0_zero_blocks(ctx, oracle):
    rows, cols, n = 512, 4096, 16
    case = wl.fp8_gemv_case(rows, cols, seed=64, ue8m0_compatible=True)
    sb = (np.log2(case.scales).astype(np.int32) + 127).astype(np.uint8)
    sb[2, :] = 0       # output rows 256..383: every block 0 -> exactly 0
    sb[0, 5] = 0
    sb[3, ::3] = 0
    scales = _ue8m0_f32(sb)
    ctx.set_exact_numerics(False)
    t = ctx.store_fp8(case.w, rows, cols, sb, rows // 128, cols // 128, wohper_amd.SCALE_UE8M0)
    xs = np.random.default_rng(5).standard_normal((n, cols)).astype(np.float32)
    ys, _ = ctx.fp8_gemv_multi(t, xs, 0, rows)
    fp8, _, _, _ = oracle.luts()
    wd = fp8[case.w].astype(np.float64) * np.repeat(np.repeat(scales.astype(np.float64), 128, 0), 128, 1)
    norms = np.sqrt((wd ** 2).sum(1))
    for i, x in enumerate(xs):
        want = oracle.fp8_gemv(case.w, rows, cols, scales, rows // 128, cols // 128, x)
        tol = 1e-5 * norms * np.linalg.norm(x.astype(np.float64))
        assert np.all(np.abs(ys[i].astype(np.float64) - want.astype(np.float64)) <= tol), i
        assert np.all(ys[i][256:384] == 0.0)
    ctx.release(t)


def test_fp8_mfma_ue8m0_infinite_block(ctx, oracle):
    rows, cols, n = 256, 4096, 16
    case = wl.fp8_gemv_case(rows, cols, seed=65, ue8m0_compatible=True)
    sb = (np.log2(case.scales).astype(np.int32) + 127).astype(np.uint8)
    sb[1, 7] = 255
    x = np.random.default_rng(6).standard_normal((n, cols)).astype(np.float32)
    with pytest.raises(oracle.OracleError):
        oracle.fp8_gemv(case.w, rows, cols, _ue8m0_f32(sb), rows // 128, cols // 128, x[0])
    ctx.set_exact_numerics(False)
    t = ctx.store_fp8(case.w, rows, cols, sb, rows // 128, cols // 128, wohper_amd.SCALE_UE8M0)
    with pytest.raises(wohper_amd.DeepSeekV4KernelError):
        ctx.fp8_gemv_multi(t, x, 0, rows)
    ctx.release(t)
