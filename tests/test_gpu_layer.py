"""GPU parity of the decode-layer pieces: device-synthesized FP8 tensors, the
batched FP8 GEMV entry point and the shared + routed expert sum
(E/compute.rs:1872-1946), against the oracle."""
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


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_fp8_synthetic_store_and_batched_gemv(ctx, oracle):
    rows, cols = 1024, 2048
    scales = wl.fp8_block_scales(7, rows, cols)
    t = ctx.store_fp8_synthetic(rows, cols, 11, wl.fp8_stream(0, 3), scales)
    w = wl.synth_fp8_host(ctx.lib, 11, wl.fp8_stream(0, 3), rows, cols)
    assert not np.any((w & 0x7F) == 0x7F)
    fp8, _, _, _ = oracle.luts()
    assert np.array_equal(bits(ctx.dequant(t, rows, cols)), bits(fp8[w]))
    rng = np.random.default_rng(3)
    xs = rng.standard_normal((3, cols)).astype(np.float32)
    x_dev = ctx.device_alloc(xs.nbytes)
    y_dev = ctx.device_alloc(3 * rows * 4)
    ctx.to_device(x_dev, xs)
    ranges = ((0, 1024), (128, 512), (3, 77))
    ctx.fp8_gemv_batch_async([(t, r0, r1, x_dev + i * cols * 4, y_dev + i * rows * 4)
                              for i, (r0, r1) in enumerate(ranges)])
    ctx.synchronize()
    ys = np.empty((3, rows), np.float32)
    ctx.from_device(ys, y_dev)
    for i, (r0, r1) in enumerate(ranges):
        want = oracle.fp8_gemv(w, rows, cols, scales, rows // 128, cols // 128, xs[i], r0, r1)
        assert np.array_equal(bits(ys[i, :r1 - r0]), bits(want)), (r0, r1)
    # wo_a-style row groups with their own inputs (one merged launch)
    xg = rng.standard_normal((4, cols)).astype(np.float32)
    xg_dev = ctx.device_alloc(xg.nbytes)
    ctx.to_device(xg_dev, xg)
    ctx.fp8_gemv_batch_async([(t, 256 * g, 256 * (g + 1), xg_dev + g * cols * 4, y_dev + g * 256 * 4)
                              for g in range(4)])
    ctx.synchronize()
    yg = np.empty(rows, np.float32)
    ctx.from_device(yg, y_dev)
    for g in range(4):
        want = oracle.fp8_gemv(w, rows, cols, scales, rows // 128, cols // 128, xg[g], 256 * g, 256 * (g + 1))
        assert np.array_equal(bits(yg[256 * g:256 * (g + 1)]), bits(want)), g
    ctx.device_free(xg_dev)
    # several inputs through one row range, device pointers
    xm = rng.standard_normal((5, cols + 4)).astype(np.float32)
    xm_dev = ctx.device_alloc(xm.nbytes)
    ym_dev = ctx.device_alloc(5 * 700 * 4)
    ctx.to_device(xm_dev, xm)
    ctx.fp8_gemv_multi_async(t, 100, 700, xm_dev, 5, cols + 4, ym_dev, 700)
    ctx.synchronize()
    ym = np.empty((5, 700), np.float32)
    ctx.from_device(ym, ym_dev)
    for i in range(5):
        want = oracle.fp8_gemv(w, rows, cols, scales, rows // 128, cols // 128, xm[i, :cols], 100, 700)
        assert np.array_equal(bits(ym[i, :600]), bits(want)), i
    ctx.device_free(xm_dev)
    ctx.device_free(ym_dev)
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.fp8_gemv_batch_async([(t, 0, rows + 1, x_dev, y_dev)])
    assert e.value.name == "InvalidShape"
    ctx.device_free(x_dev)
    ctx.device_free(y_dev)


def test_fp8_row_group_sizes(ctx, oracle):
    """Runs of equal row groups with their own inputs merge into one launch
    when the group is a power of two of at least 8 rows (8, 64), and go out
    one launch per group otherwise (4, 24); every group matches the oracle."""
    rows, cols = 1024, 2048
    scales = wl.fp8_block_scales(9, rows, cols)
    t = ctx.store_fp8_synthetic(rows, cols, 13, wl.fp8_stream(0, 4), scales)
    w = wl.synth_fp8_host(ctx.lib, 13, wl.fp8_stream(0, 4), rows, cols)
    rng = np.random.default_rng(9)
    for gsize, n, r0 in ((8, 6, 40), (64, 3, 128), (24, 5, 8), (4, 7, 3)):
        xg = rng.standard_normal((n, cols)).astype(np.float32)
        x_dev = ctx.device_alloc(xg.nbytes)
        y_dev = ctx.device_alloc(n * gsize * 4)
        ctx.to_device(x_dev, xg)
        ctx.fp8_gemv_batch_async([(t, r0 + gsize * g, r0 + gsize * (g + 1), x_dev + g * cols * 4,
                                   y_dev + g * gsize * 4) for g in range(n)])
        ctx.synchronize()
        y = np.empty(n * gsize, np.float32)
        ctx.from_device(y, y_dev)
        for g in range(n):
            a, b = r0 + gsize * g, r0 + gsize * (g + 1)
            want = oracle.fp8_gemv(w, rows, cols, scales, rows // 128, cols // 128, xg[g], a, b)
            assert np.array_equal(bits(y[gsize * g:gsize * (g + 1)]), bits(want)), (gsize, g)
        ctx.device_free(x_dev)
        ctx.device_free(y_dev)
    ctx.release(t)


@pytest.mark.parametrize("n_routed", [6, 1, 0])
def test_shared_plus_routed_bit_exact(ctx, oracle, n_routed):
    seed = 4
    idx, w, x = wl.moe_token_case(seed)
    routes = [(5, int(e), float(wt)) for e, wt in zip(idx[:n_routed], w[:n_routed])]
    for _, e, _ in routes:
        ctx.store_expert_synthetic(5, e, wl.HIDDEN, wl.INTER, seed)
    shared = (5, wl.N_ROUTED)
    ctx.store_expert_synthetic(shared[0], shared[1], wl.HIDDEN, wl.INTER, seed)
    got = ctx.routed_and_shared_experts(routes, shared, x)
    sh = oracle.fp4_expert_forward(*wl.synth_expert_host(ctx.lib, seed, *shared), x)
    if n_routed:
        outs = np.stack([oracle.fp4_expert_forward(*wl.synth_expert_host(ctx.lib, seed, 5, e), x)
                         for _, e, _ in routes])
        want = sh + oracle.routed_combine(outs, [wt for _, _, wt in routes])
    else:
        want = sh
    assert np.array_equal(bits(got), bits(want.astype(np.float32)))


def test_fp8_batched_decode_layer_set_order_and_formats(ctx, oracle):
    """A decode layer's projection set in one call (one grouped launch),
    bit-exact per projection; a descriptor reading an earlier one's output
    in the same call sees it (in-order semantics); f32 and UE8M0 scales
    mixed in one call."""
    rng = np.random.default_rng(31)
    host, dev, descs, want = {}, [], [], []

    def alloc(arr):
        p = ctx.device_alloc(arr.nbytes)
        ctx.to_device(p, arr)
        dev.append(p)
        return p

    for i, (name, r, c, groups) in enumerate(wl.DECODE_LAYER_FP8):
        sc = wl.fp8_block_scales(40 + i, r, c)
        t = ctx.store_fp8_synthetic(r, c, 5, wl.fp8_stream(90, i), sc)
        host[name] = (t, wl.synth_fp8_host(ctx.lib, 5, wl.fp8_stream(90, i), r, c), sc, r, c)
    y_all = ctx.device_alloc(64 * 1024 * 4)
    dev.append(y_all)
    off = 0
    for name, r, c, groups in wl.DECODE_LAYER_FP8:
        t, w, sc, _, _ = host[name]
        rows = r // groups
        x = rng.standard_normal((groups, c)).astype(np.float32)
        xp = alloc(x)
        for g in range(groups):
            descs.append((t, rows * g, rows * (g + 1), xp + g * c * 4, y_all + (off + rows * g) * 4))
            want.append((off + rows * g, oracle.fp8_gemv(w, r, c, sc, r // 128, c // 128, x[g], rows * g, rows * (g + 1))))
        off += r
    # chained: wq_b reads the output of wq_a within the same call
    t_a, w_a, sc_a, r_a, c_a = host["wq_a"]
    t_b, w_b, sc_b, r_b, c_b = host["wq_b"]
    xa = rng.standard_normal(c_a).astype(np.float32)
    xa_p = alloc(xa)
    mid = ctx.device_alloc(r_a * 4)
    out = ctx.device_alloc(r_b * 4)
    dev += [mid, out]
    descs.append((t_a, 0, r_a, xa_p, mid))
    descs.append((t_b, 0, r_b, mid, out))
    y_mid = oracle.fp8_gemv(w_a, r_a, c_a, sc_a, r_a // 128, c_a // 128, xa)
    y_chain = oracle.fp8_gemv(w_b, r_b, c_b, sc_b, r_b // 128, c_b // 128, y_mid)
    # a UE8M0-scaled tensor between f32-scaled ones
    case = wl.fp8_gemv_case(1024, 2048, seed=3, ue8m0_compatible=True)
    sbytes = (np.log2(case.scales).astype(np.int32) + 127).astype(np.uint8)
    t_u = ctx.store_fp8(case.w, 1024, 2048, sbytes, 8, 16, wohper_amd.SCALE_UE8M0)
    xu_p = alloc(case.x)
    yu = ctx.device_alloc(1024 * 4)
    dev.append(yu)
    descs.insert(3, (t_u, 0, 1024, xu_p, yu))
    ctx.fp8_gemv_batch_async(descs)
    ctx.synchronize()
    got = np.empty(64 * 1024, np.float32)
    ctx.from_device(got, y_all)
    for o, w_ in want:
        assert np.array_equal(bits(got[o:o + w_.size]), bits(w_)), o
    got_chain = np.empty(r_b, np.float32)
    ctx.from_device(got_chain, out)
    assert np.array_equal(bits(got_chain), bits(y_chain))
    got_u = np.empty(1024, np.float32)
    ctx.from_device(got_u, yu)
    assert np.array_equal(bits(got_u), bits(oracle.fp8_gemv(case.w, 1024, 2048, case.scales, 8, 16, case.x)))
    for p in dev:
        ctx.device_free(p)
    for t, *_ in host.values():
        ctx.release(t)
    ctx.release(t_u)


def test_fp8_shared_expert_bit_exact(ctx, oracle):
    """compute_deepseek_fp8_shared_expert_into_hidden (E/compute.rs:5545-5614)
    at the model's shapes, host-slice and in-place device variants, plus the
    closed-form case of the oracle's tests and the reference's shape errors."""
    hidden, inter = 4096, 2048
    cases = [wl.fp8_gemv_case(inter, hidden, seed=61), wl.fp8_gemv_case(inter, hidden, seed=62),
             wl.fp8_gemv_case(hidden, inter, seed=63)]
    t = [ctx.store_fp8(c.w, c.w.shape[0], c.w.shape[1], c.scales, c.scales.shape[0], c.scales.shape[1],
                       wohper_amd.SCALE_F32) for c in cases]
    x = (np.random.default_rng(64).standard_normal(hidden) * 2.0).astype(np.float32)
    want = oracle.fp8_shared_expert(cases[0].w, cases[0].scales, cases[1].w, cases[1].scales, cases[2].w,
                                    cases[2].scales, hidden, inter, x)
    got = ctx.fp8_shared_expert(t[0], t[1], t[2], x, hidden)
    assert np.array_equal(bits(got), bits(want))
    # in place on the device, like the reference's hidden_states
    h_dev = ctx.device_alloc(x.nbytes)
    ctx.to_device(h_dev, x)
    ctx.fp8_shared_expert_async(t[0], t[1], t[2], h_dev, h_dev)
    ctx.synchronize()
    got_dev = np.empty_like(x)
    ctx.from_device(got_dev, h_dev)
    ctx.device_free(h_dev)
    assert np.array_equal(bits(got_dev), bits(want))
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.fp8_shared_expert(t[0], t[2], t[2], x, hidden)  # w3 is 4096 x 2048
    assert e.value.name == "InvalidShape"
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.fp8_shared_expert(t[0], t[1], t[2], x, hidden - 1)
    assert e.value.name == "OutputTooSmall"
    for h in t:
        ctx.release(h)
    # the oracle's closed-form case
    n = 128
    w1, w3, w2 = (np.zeros((n, n), np.uint8) for _ in range(3))
    w1[0, 0], w3[0, 0], w2[5, 0] = 0x38, 0x3C, 0x40
    w1[1, 1], w3[1, 1], w2[6, 1] = 0x38, 0x38, 0x38
    one = np.ones((1, 1), np.float32)
    tk = [ctx.store_fp8(w, n, n, one, 1, 1, wohper_amd.SCALE_F32) for w in (w1, w3, w2)]
    xk = np.zeros(n, np.float32)
    xk[0], xk[1] = 2.0, 0.3
    wk = np.zeros(n, np.float32)
    wk[5], wk[6] = 11.0, 0.0546875
    assert np.array_equal(ctx.fp8_shared_expert(*tk, xk, n), wk)
    for h in tk:
        ctx.release(h)


def test_fp8_pair_of_one_input_bit_exact(ctx, oracle):
    """Two projections of one input (wq_a and wkv of a decode layer, and a
    UE8M0 pair with the reference's +-480 codes) go out as one launch; each
    stays bit-exact."""
    rng = np.random.default_rng(47)
    dev = []

    def alloc(arr):
        p = ctx.device_alloc(arr.nbytes)
        ctx.to_device(p, arr)
        dev.append(p)
        return p

    ta = ctx.store_fp8_synthetic(1024, 4096, 7, wl.fp8_stream(91, 0), wl.fp8_block_scales(60, 1024, 4096))
    tk = ctx.store_fp8_synthetic(512, 4096, 7, wl.fp8_stream(91, 2), wl.fp8_block_scales(61, 512, 4096))
    wa = wl.synth_fp8_host(ctx.lib, 7, wl.fp8_stream(91, 0), 1024, 4096)
    wk = wl.synth_fp8_host(ctx.lib, 7, wl.fp8_stream(91, 2), 512, 4096)
    x = rng.standard_normal(4096).astype(np.float32)
    xp = alloc(x)
    ya, yk = ctx.device_alloc(1024 * 4), ctx.device_alloc(512 * 4)
    dev += [ya, yk]
    # rows 200..1000 of the first, all of the second
    ctx.fp8_gemv_batch_async([(ta, 200, 1000, xp, ya), (tk, 0, 512, xp, yk)])
    ctx.synchronize()
    got_a, got_k = np.empty(800, np.float32), np.empty(512, np.float32)
    ctx.from_device(got_a, ya)
    ctx.from_device(got_k, yk)
    want_a = oracle.fp8_gemv(wa, 1024, 4096, wl.fp8_block_scales(60, 1024, 4096), 8, 32, x, 200, 1000)
    want_k = oracle.fp8_gemv(wk, 512, 4096, wl.fp8_block_scales(61, 512, 4096), 4, 32, x)
    assert np.array_equal(bits(got_a), bits(want_a))
    assert np.array_equal(bits(got_k), bits(want_k))
    # UE8M0 scales and the special codes in both tensors
    cases, ts = [], []
    for seed, rows in ((11, 768), (12, 256)):
        case = wl.fp8_gemv_case(rows, 2048, seed=seed, ue8m0_compatible=True)
        w = case.w.copy()
        w[::7, ::11] = 0x7F
        w[3::7, 5::11] = 0xFF
        sb = (np.log2(case.scales).astype(np.int32) + 127).astype(np.uint8)
        ts.append(ctx.store_fp8(w, rows, 2048, sb, rows // 128, 16, wohper_amd.SCALE_UE8M0))
        cases.append((w, case.scales, rows))
    x2 = rng.standard_normal(2048).astype(np.float32)
    x2p = alloc(x2)
    ys = [ctx.device_alloc(r * 4) for _, _, r in cases]
    dev += ys
    ctx.fp8_gemv_batch_async([(ts[0], 0, 768, x2p, ys[0]), (ts[1], 0, 256, x2p, ys[1])])
    ctx.synchronize()
    for (w, sc, rows), yp in zip(cases, ys):
        got = np.empty(rows, np.float32)
        ctx.from_device(got, yp)
        assert np.array_equal(bits(got), bits(oracle.fp8_gemv(w, rows, 2048, sc, rows // 128, 16, x2)))
    # two tensors writing the same output stay in order: the second's values
    # win, as with two launches
    ctx.fp8_gemv_batch_async([(tk, 0, 512, xp, ya), (ta, 0, 512, xp, ya)])
    ctx.synchronize()
    got = np.empty(512, np.float32)
    ctx.from_device(got, ya)
    want_a0 = oracle.fp8_gemv(wa, 1024, 4096, wl.fp8_block_scales(60, 1024, 4096), 8, 32, x, 0, 512)
    assert np.array_equal(bits(got), bits(want_a0))
    for p in dev:
        ctx.device_free(p)
    for t in [ta, tk] + ts:
        ctx.release(t)
