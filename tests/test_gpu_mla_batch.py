"""GPU parity of the batched MLA attention of prefill and MTP verify
(wh_mla_attention_decode_batch_async, compute_deepseek_v4_mla_attention_batch,
E/compute.rs:4307-4641).  The reference batches the projections with
gemv_fp8_e4m3_ue8m0_rows_multi, whose every input is bit-identical to the
single-input kernel (E/compute.rs:6447-6452), writes every position's KV row
before the window loop, and reads in each position's window only rows at or
before its own; so with exact numerics the batch must equal the single-token
layer run position by position, bit for bit, and the oracle's single-token
restatement (mla_attention_decode) run the same way: a sliding-window layer
over a cache with earlier rows, a compressed YaRN layer with per-position
compressed rows, and 16 positions in order-free numerics (the projections on
MFMA) within a loose bound of the exact result."""
import numpy as np
import pytest

import wohper_amd
from parity_util import bits
from test_gpu_mla import HEAD_DIM, HEADS, NOPE, ROPE, GROUPS, O_LORA, Dev, _layer, _proj
from wohper_amd import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture
def dev(ctx):
    d = Dev(ctx)
    yield d
    d.free()
    ctx.set_exact_numerics(True)


def _sequential(ctx, dev, L, xs, positions, cache0, ld, comps=None):
    """The single-token layer at each position in order, on its own cache."""
    cap = cache0.shape[0]
    kvp = dev.put(cache0)
    outs = []
    for i, p in enumerate(positions):
        hp = dev.put(xs[i])
        if comps:
            ctx.mla_attention_decode_async(L, p, hp, kvp, ld, cap, comps[i][0], comps[i][1])
        else:
            ctx.mla_attention_decode_async(L, p, hp, kvp, ld, cap)
        ctx.synchronize()
        outs.append(dev.get(hp, wl.HIDDEN))
    return np.stack(outs), dev.get(kvp, (cap, ld))


def _batch(ctx, dev, L, xs, positions, cache0, ld, comps=None):
    cap = cache0.shape[0]
    kvp, hp = dev.put(cache0), dev.put(np.ascontiguousarray(xs))
    ctx.mla_attention_decode_batch_async(L, positions, hp, kvp, ld, cap, comps)
    ctx.synchronize()
    return dev.get(hp, (len(positions), wl.HIDDEN)), dev.get(kvp, (cap, ld))


def test_mla_batch_window_layer(ctx, oracle, dev):
    """Layer 0 (sliding window, theta 10000): positions 5..9 after five
    earlier cache rows, against the single-token layer and the oracle."""
    ctx.set_exact_numerics(True)
    L, host, qn, kn, sink, handles = _layer(ctx, dev, 0)
    proj = _proj(oracle, host)
    cap, ld = 16, HEAD_DIM + 64
    rng = np.random.default_rng(11)
    cache0 = np.zeros((cap, ld), np.float32)
    cache0[:5] = (rng.standard_normal((5, ld)) * 0.3).astype(np.float32)
    positions = [5, 6, 7, 8, 9]
    xs = rng.standard_normal((len(positions), wl.HIDDEN)).astype(np.float32)
    got, got_cache = _batch(ctx, dev, L, xs, positions, cache0, ld)
    want, want_cache = _sequential(ctx, dev, L, xs, positions, cache0, ld)
    assert np.array_equal(bits(got_cache), bits(want_cache))
    assert np.array_equal(bits(got), bits(want)), int(np.count_nonzero(bits(got) != bits(want)))
    cache = cache0.copy()
    for i, p in enumerate(positions):
        w = oracle.mla_attention_decode(xs[i], proj, qn, kn, sink, HEADS, NOPE, ROPE, GROUPS, O_LORA, 0, p, cache)
        assert np.array_equal(bits(got[i]), bits(w)), p
    assert np.array_equal(bits(got_cache), bits(cache))
    for h in handles.values():
        ctx.release(h)


def test_mla_batch_compressed_layer(ctx, oracle, dev):
    """Layer 2 (theta 160000 with YaRN), positions 300..302 with a full
    window and 75, 75, 76 compressed rows of their own, plain norms, no
    sink."""
    ctx.set_exact_numerics(True)
    L, host, qn, kn, sink, handles = _layer(ctx, dev, 2, with_norms=False, with_sink=False)
    proj = _proj(oracle, host)
    cap, ld = 320, HEAD_DIM
    rng = np.random.default_rng(12)
    cache0 = (rng.standard_normal((cap, ld)) * 0.3).astype(np.float32)
    positions = [300, 301, 302]
    comps_h = [(rng.standard_normal((k, HEAD_DIM)) * 0.3).astype(np.float32) for k in (75, 75, 76)]
    comps = [(dev.put(cmp), cmp.shape[0]) for cmp in comps_h]
    xs = rng.standard_normal((len(positions), wl.HIDDEN)).astype(np.float32)
    got, got_cache = _batch(ctx, dev, L, xs, positions, cache0, ld, comps)
    want, want_cache = _sequential(ctx, dev, L, xs, positions, cache0, ld, comps)
    assert np.array_equal(bits(got_cache), bits(want_cache))
    assert np.array_equal(bits(got), bits(want))
    cache = cache0.copy()
    for i, p in enumerate(positions):
        w = oracle.mla_attention_decode(xs[i], proj, None, None, None, HEADS, NOPE, ROPE, GROUPS, O_LORA, 2, p, cache,
                                        comps_h[i])
        assert np.array_equal(bits(got[i]), bits(w)), p
    for h in handles.values():
        ctx.release(h)


def test_mla_batch_order_free_16(ctx, dev):
    """16 positions: with exact numerics the batch equals the single-token
    layer position by position (the decode-once kernels at 16 inputs); with
    exact numerics off (the projections on bf16 MFMA, exact products, fp32
    accumulation order only; the norms' sums as trees) each position stays
    within 1e-2 of the exact output in norm.  The bound is loose because an
    act-quant between the projections can round a near-tie the other way:
    one such element moves a wo_b output by a whole E4M3 step of its input
    (the per-matvec tolerance of the projections is checked in
    test_gpu_fp8_mfma)."""
    L, host, qn, kn, sink, handles = _layer(ctx, dev, 0)
    cap, ld = 32, HEAD_DIM
    rng = np.random.default_rng(13)
    cache0 = (rng.standard_normal((cap, ld)) * 0.3).astype(np.float32)
    positions = list(range(4, 20))
    xs = rng.standard_normal((len(positions), wl.HIDDEN)).astype(np.float32)
    ctx.set_exact_numerics(True)
    want, _ = _batch(ctx, dev, L, xs, positions, cache0, ld)
    seq, _ = _sequential(ctx, dev, L, xs, positions, cache0, ld)
    assert np.array_equal(bits(want), bits(seq))  # exact: 16 inputs through the decode-once kernels
    ctx.set_exact_numerics(False)
    got, _ = _batch(ctx, dev, L, xs, positions, cache0, ld)
    assert np.all(np.isfinite(got))
    rel = np.linalg.norm(got - want, axis=1) / np.linalg.norm(want, axis=1)
    print("per-position ||diff|| / ||value||:", np.array2string(rel, precision=6))
    assert float(rel.max()) <= 1e-2
    for h in handles.values():
        ctx.release(h)


def test_mla_batch_errors(ctx, dev):
    L, host, qn, kn, sink, handles = _layer(ctx, dev, 0)
    cap, ld = 8, HEAD_DIM
    kvp, hp = dev.put(np.zeros((cap, ld), np.float32)), dev.put(np.zeros((2, wl.HIDDEN), np.float32))
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.mla_attention_decode_batch_async(L, [3, 2], hp, kvp, ld, cap)  # positions must ascend
    assert e.value.name == "InvalidArgument"
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.mla_attention_decode_batch_async(L, [], hp, kvp, ld, cap)
    assert e.value.name == "InvalidShape"
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.mla_attention_decode_batch_async(L, [6, cap], hp, kvp, ld, cap)  # past the cache
    assert e.value.name == "InvalidShape"
    for h in handles.values():
        ctx.release(h)
