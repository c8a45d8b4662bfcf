"""GPU parity at the full workloads of the ragged batch and the 43-layer stack.

* Ragged batched MoE: 64 tokens routed top-6 over 256 experts of the model's
  shapes (w1/w3 2048x4096, w2 4096x2048) with Zipf(1.1) popularity, seed 4,
  through wh_moe_batch with exact numerics off at MFMA thresholds 16, 2 and
  the default 1: groups at or above the threshold run on MFMA (every matvec
  within 1e-5 * ||w_row|| * ||x|| of the oracle on the same input), all
  others bit-exact; every later stage bit-exact given the matvec outputs
  (the batch-prefill MoE of E/server/generation.rs:2487-2569,
  accumulate_expert_for_positions, E/compute.rs:1779-1810).
* The full-depth stack: 43 layers of 256 routed + 1 shared FP4 experts and
  one decode layer's FP8 projections each (152 GB resident), seed 5.  On
  three sampled layers: at batch 1 every FP8 projection (the row ranges and
  wo_a groups of E/compute.rs:4005-4265) and the shared + top-6 routed MoE
  (E/compute.rs:1872-1946) bit-exact against the oracle; at batch 16 every
  projection over 16 inputs (gemv_fp8_e4m3_ue8m0_rows_multi,
  E/compute.rs:6384-6577) bit-exact, and the batch MoE of 16 positions with
  the shared expert bit-exact under exact numerics; with exact numerics off
  every expert runs on MFMA and the output is compared in norm."""
import numpy as np
import pytest

import wohper_amd
from test_gpu_batch import _mfma_case
from wohper_amd import workloads as wl

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("mfma_min", [16, 2, 1])
def test_ragged_batch_full_workload(ctx, oracle, mfma_min):
    """64 Zipf-routed tokens over 256 model-shape experts."""
    try:
        worst, _ = _mfma_case(ctx, oracle, 80, wl.N_ROUTED, wl.HIDDEN, wl.INTER, 4, 64, mfma_min)
        print(f"ragged batch, MFMA threshold {mfma_min}: worst MFMA matvec |diff| / tolerance {worst:.3f}")
    finally:
        ctx.set_moe_mfma_min(1)


STACK_SEED = 5
SAMPLED = (0, 21, 42)


@pytest.fixture(scope="module")
def stack():
    """The resident 43-layer stack on its own context (closed afterwards, so
    its 152 GB do not stay resident for the tests that follow)."""
    c = wohper_amd.Context(0)
    layers = []
    for L in range(wl.LAYERS):
        hs = {}
        for i, (name, r, cols, _) in enumerate(wl.DECODE_LAYER_FP8):
            hs[name] = (c.store_fp8_synthetic(r, cols, STACK_SEED, wl.fp8_stream(L, i),
                                              wl.fp8_block_scales(STACK_SEED * 1000 + L * 7 + i, r, cols)), i)
        for e in range(wl.N_ROUTED + 1):  # id N_ROUTED: the layer's shared expert
            c.store_expert_synthetic(L, e, wl.HIDDEN, wl.INTER, STACK_SEED)
        layers.append(hs)
    used, _, n_exp = c.usage()
    assert n_exp == wl.LAYERS * (wl.N_ROUTED + 1)
    assert used >= 150e9
    c.set_exact_numerics(True)
    yield c, layers
    c.close()


def _fp8_host(lib, L, name):
    i = [n for n, *_ in wl.DECODE_LAYER_FP8].index(name)
    _, r, cols, _ = wl.DECODE_LAYER_FP8[i]
    w = wl.synth_fp8_host(lib, STACK_SEED, wl.fp8_stream(L, i), r, cols)
    return w, wl.fp8_block_scales(STACK_SEED * 1000 + L * 7 + i, r, cols), r, cols


@pytest.mark.parametrize("L", SAMPLED)
def test_stack_layer_batch1(stack, oracle, L):
    c, layers = stack
    rng = np.random.default_rng(100 + L)
    ins = {"x": rng.standard_normal(4096), "qlat": rng.standard_normal(1024), "oa": rng.standard_normal(8 * 4096),
           "ob": rng.standard_normal(8192)}
    ins = {k: v.astype(np.float32) for k, v in ins.items()}
    dev = {k: c.device_alloc(v.nbytes) for k, v in ins.items()}
    for k, v in ins.items():
        c.to_device(dev[k], v)
    hs = layers[L]
    outs = {"wq_a": 1024, "wq_b": 32768, "wkv": 512, "wo_a": 8192, "wo_b": 4096}
    ydev = {k: c.device_alloc(n * 4) for k, n in outs.items()}
    d = [(hs["wq_a"][0], 0, 1024, dev["x"], ydev["wq_a"]), (hs["wq_b"][0], 0, 32768, dev["qlat"], ydev["wq_b"]),
         (hs["wkv"][0], 0, 512, dev["x"], ydev["wkv"])]
    d += [(hs["wo_a"][0], 1024 * g, 1024 * (g + 1), dev["oa"] + g * 4096 * 4, ydev["wo_a"] + g * 1024 * 4)
          for g in range(8)]
    d += [(hs["wo_b"][0], 0, 4096, dev["ob"], ydev["wo_b"])]
    c.fp8_gemv_batch_async(d)
    c.synchronize()
    inputs = {"wq_a": ins["x"], "wq_b": ins["qlat"], "wkv": ins["x"], "wo_b": ins["ob"]}
    for name, n in outs.items():
        got = np.empty(n, np.float32)
        c.from_device(got, ydev[name])
        w, sc, r, cols = _fp8_host(c.lib, L, name)
        if name == "wo_a":
            want = np.concatenate([oracle.fp8_gemv(w, r, cols, sc, r // 128, cols // 128,
                                                   ins["oa"][4096 * g:4096 * (g + 1)], 1024 * g, 1024 * (g + 1))
                                   for g in range(8)])
        else:
            want = oracle.fp8_gemv(w, r, cols, sc, r // 128, cols // 128, inputs[name])
        assert np.array_equal(bits(got), bits(want)), (L, name)
    for p in list(dev.values()) + list(ydev.values()):
        c.device_free(p)
    # shared + top-6 routed MoE of the layer
    idx, w = wl.route_topk_sigmoid(rng.standard_normal(wl.N_ROUTED).astype(np.float32))
    x = wl.bf16_round(rng.standard_normal(wl.HIDDEN).astype(np.float32))
    routes = [(L, int(e), float(wt)) for e, wt in zip(idx, w)]
    got = c.routed_and_shared_experts(routes, (L, wl.N_ROUTED), x)
    ex = [wl.synth_expert_host(c.lib, STACK_SEED, L, int(e)) for e in idx]
    routed = oracle.routed_combine(np.stack([oracle.fp4_expert_forward(*m, x) for m in ex]), w)
    shared = oracle.fp4_expert_forward(*wl.synth_expert_host(c.lib, STACK_SEED, L, wl.N_ROUTED), x)
    assert np.array_equal(bits(got), bits((shared + routed).astype(np.float32))), L


@pytest.mark.parametrize("L", SAMPLED)
def test_stack_layer_batch16(stack, oracle, L):
    c, layers = stack
    batch = 16
    rng = np.random.default_rng(200 + L)
    hs = layers[L]
    specs = [("wq_a", 0, 1024, 4096), ("wq_b", 0, 32768, 1024), ("wkv", 0, 512, 4096), ("wo_b", 0, 4096, 8192)]
    specs += [("wo_a", 1024 * g, 1024 * (g + 1), 4096) for g in range(8)]
    for name, r0, r1, cols in specs:
        xs = rng.standard_normal((batch, cols)).astype(np.float32)
        x_dev, y_dev = c.device_alloc(xs.nbytes), c.device_alloc(batch * (r1 - r0) * 4)
        c.to_device(x_dev, xs)
        c.fp8_gemv_multi_async(hs[name][0], r0, r1, x_dev, batch, cols, y_dev, r1 - r0)
        c.synchronize()
        got = np.empty((batch, r1 - r0), np.float32)
        c.from_device(got, y_dev)
        w, sc, r, _ = _fp8_host(c.lib, L, name)
        for b in range(batch):
            want = oracle.fp8_gemv(w, r, cols, sc, r // 128, cols // 128, xs[b], r0, r1)
            assert np.array_equal(bits(got[b]), bits(want)), (L, name, r0, b)
        c.device_free(x_dev)
        c.device_free(y_dev)
    # the MoE of 16 positions: top-6 of 256 sigmoid scores per position,
    # shared expert on all of them
    ids = np.empty((batch, wl.TOPK), np.uint32)
    sc = np.empty((batch, wl.TOPK), np.float32)
    for p in range(batch):
        s_all = (1.0 / (1.0 + np.exp(-rng.standard_normal(wl.N_ROUTED)))).astype(np.float32)
        order = np.argsort(-s_all, kind="stable")[:wl.TOPK]
        ids[p], sc[p] = order, s_all[order]
    x = wl.bf16_round(rng.standard_normal((batch, wl.HIDDEN)).astype(np.float32))
    experts = {int(e): wl.synth_expert_host(c.lib, STACK_SEED, L, int(e)) for e in np.unique(ids)}
    shared = wl.synth_expert_host(c.lib, STACK_SEED, L, wl.N_ROUTED)
    want = oracle.moe_batch(experts, ids, sc, x, shared=shared)
    # exact numerics: every expert on the exact items, bit for bit
    got = c.moe_batch(L, ids, sc, x, shared_key=(L, wl.N_ROUTED))
    assert int(c.debug_moe_batch_read(4, 8, np.uint32)[4]) == 0
    assert np.array_equal(bits(got), bits(want)), L
    try:
        # exact numerics off, default threshold: every expert on MFMA, each
        # matvec within tolerance, so the output is compared in norm
        c.set_exact_numerics(False)
        got = c.moe_batch(L, ids, sc, x, shared_key=(L, wl.N_ROUTED))
        meta = c.debug_moe_batch_read(4, 8, np.uint32)
        assert int(meta[4]) == int(meta[0])
        assert np.linalg.norm(got - want) <= 1e-3 * np.linalg.norm(want), L
    finally:
        c.set_exact_numerics(True)
