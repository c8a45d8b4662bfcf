"""GPU parity of one whole DeepSeek-V4 decode layer on the device
(wh_deepseek_mhc_layer_async): hc_pre -> attention norm -> MLA attention ->
hc_post -> hc_pre -> ffn norm -> router -> shared + routed experts -> hc_post
(compute_layer_deepseek_mhc, E/compute.rs:1448-1480, with the router between
its phases as E/server/generation.rs:719-836 runs it), at the model's shapes
(hc 4 x hidden 4096, 64 heads of 448 + 64, q_lora 1024, 8 output groups,
expert inter 2048) with a 32-expert router, against the oracle's composition
of the same steps.  Exact numerics: bit for bit over three positions, the KV
cache growing.  Exact numerics off: the order-free kernels stay within a
loose relative bound of the exact layer (same routes).  A captured layer
replays to the eager result bit for bit."""
import numpy as np
import pytest

from parity_util import bits
from test_gpu_mla import HEAD_DIM, HEADS, NOPE, ROPE, GROUPS, O_LORA, Dev, _bf16_weights, _layer, _proj
from test_gpu_mhc import _params
import wohper_amd
from wohper_amd import model_format as mf
from wohper_amd import workloads as wl

pytestmark = pytest.mark.gpu

HC, ITERS, EPS = 4, 20, 1e-6
LAYER, N_EXP, SEED, ACTIVE, SCALE = 52, 32, 91, 6, 1.5


@pytest.fixture
def dev(ctx):
    d = Dev(ctx)
    yield d
    d.free()
    ctx.set_exact_numerics(True)


def _setup(ctx, oracle, dev):
    rng = np.random.default_rng(SEED)
    attn_p, ffn_p = _params(rng, HC, wl.HIDDEN), _params(rng, HC, wl.HIDDEN)
    an, fnorm = _bf16_weights(rng, wl.HIDDEN), _bf16_weights(rng, wl.HIDDEN)
    mla_l, host, qn, kn, sink, handles = _layer(ctx, dev, 0)
    for e in range(N_EXP + 1):
        ctx.store_expert_synthetic(LAYER, e, wl.HIDDEN, wl.INTER, SEED)
    gate = ((rng.standard_normal((N_EXP, wl.HIDDEN)).astype(np.float32) * 0.02).view(np.uint32) >> 16)
    gate = gate.astype(np.uint16)
    bias = (rng.standard_normal(N_EXP) * 0.05).astype(np.float32)
    blk = mf.build_synthetic_quant_block([
        mf.SyntheticTensor(f"layers.{LAYER}.ffn.gate.weight", 9, (N_EXP, wl.HIDDEN), gate.tobytes(), 11, 2404),
        mf.SyntheticTensor(f"layers.{LAYER}.ffn.gate.bias", 9, (N_EXP,), bias.tobytes(), 12, 2405)])
    ctx.store_router(LAYER, blk, wl.HIDDEN)
    L = wohper_amd.WhMhcLayer()
    L.hc, L.hidden, L.sinkhorn_iters, L.hc_eps = HC, wl.HIDDEN, ITERS, EPS
    L.hc_attn_fn, L.hc_attn_scale, L.hc_attn_base = (dev.put(a) for a in attn_p)
    L.hc_ffn_fn, L.hc_ffn_scale, L.hc_ffn_base = (dev.put(a) for a in ffn_p)
    L.attn_norm_bf16, L.ffn_norm_bf16 = dev.put(an), dev.put(fnorm)
    L.attn = mla_l
    L.layer_id, L.active, L.available_dev, L.n_available = LAYER, ACTIVE, None, 0
    L.route = wohper_amd.Context.route_options(wohper_amd.ROUTER_SQRT_SOFTPLUS, SCALE)
    L.shared_layer, L.shared_expert = LAYER, N_EXP
    experts = {}

    def expert(e):
        if e not in experts:
            experts[e] = wl.synth_expert_host(ctx.lib, SEED, LAYER, e)
        return experts[e]

    def moe(ids, w, g):
        sh = oracle.fp4_expert_forward(*expert(N_EXP), g)
        outs = np.stack([oracle.fp4_expert_forward(*expert(int(e)), g) for e in ids])
        return (sh + oracle.routed_combine(outs, w)).astype(np.float32)

    mla = dict(proj=_proj(oracle, host), q_norm=qn, kv_norm=kn, sink=sink, heads=HEADS, nope_dim=NOPE,
               rope_dim=ROPE, o_groups=GROUPS, o_lora=O_LORA, physical_layer=0)

    def want(hidden, pos, cache):
        return oracle.mhc_decode_layer(hidden, HC, wl.HIDDEN, attn_p, ffn_p, an, fnorm, mla, gate, bias, ACTIVE,
                                       SCALE, moe, pos, cache, None, ITERS, EPS)

    class Experts:
        def __getitem__(self, e):
            return expert(int(e))

    def want_batch(hiddens, positions, cache):
        return oracle.mhc_decode_layer_batch(hiddens, positions, HC, wl.HIDDEN, attn_p, ffn_p, an, fnorm, mla, gate,
                                             bias, ACTIVE, SCALE, Experts(), expert(N_EXP), cache, None, ITERS, EPS)

    want.batch = want_batch
    return L, want, handles


def test_decode_layer_bit_exact(ctx, oracle, dev):
    ctx.set_exact_numerics(True)
    L, want, handles = _setup(ctx, oracle, dev)
    cap, ld = 8, HEAD_DIM + 64
    kvp = dev.put(np.zeros((cap, ld), np.float32))
    cache = np.zeros((cap, ld), np.float32)
    rng = np.random.default_rng(5)
    h = (rng.standard_normal(HC * wl.HIDDEN) * 0.5).astype(np.float32)
    hp = dev.put(h)
    for pos in range(3):
        ctx.deepseek_mhc_layer_async(L, pos, hp, kvp, ld, cap)
        ctx.synchronize()
        h, ids, w = want(h, pos, cache)
        got = dev.get(hp, HC * wl.HIDDEN)
        assert np.array_equal(bits(dev.get(kvp, (cap, ld))[:pos + 1]), bits(cache[:pos + 1])), pos
        assert np.array_equal(bits(got), bits(h)), (pos, list(ids), int(np.count_nonzero(bits(got) != bits(h))))
    for t in handles.values():
        ctx.release(t)


def test_decode_layer_order_free_and_graph(ctx, oracle, dev):
    """Exact numerics off: within 1e-3 of the largest value of the exact
    layer's output; then the same layer captured once replays to the eager
    result bit for bit (the KV row it writes is the same each time)."""
    L, want, handles = _setup(ctx, oracle, dev)
    cap, ld = 8, HEAD_DIM + 64
    rng = np.random.default_rng(6)
    h0 = (rng.standard_normal(HC * wl.HIDDEN) * 0.5).astype(np.float32)
    kv0 = (rng.standard_normal((cap, ld)) * 0.3).astype(np.float32)
    outs = {}
    for exact in (True, False):
        ctx.set_exact_numerics(exact)
        hp, kvp = dev.put(h0), dev.put(kv0)
        ctx.deepseek_mhc_layer_async(L, 2, hp, kvp, ld, cap)
        ctx.synchronize()
        outs[exact] = dev.get(hp, HC * wl.HIDDEN)
    assert np.all(np.isfinite(outs[False]))
    scale = float(np.abs(outs[True]).max())
    assert float(np.abs(outs[False] - outs[True]).max()) <= 1e-3 * scale
    # graph: eager once from h0, then replays from h0 each time
    hp, kvp = dev.put(h0), dev.put(kv0)
    g = ctx.graph_capture(lambda: ctx.deepseek_mhc_layer_async(L, 2, hp, kvp, ld, cap))
    try:
        for rep in range(3):
            ctx.to_device(hp, h0)
            ctx.graph_launch(g)
            ctx.synchronize()
            assert np.array_equal(bits(dev.get(hp, HC * wl.HIDDEN)), bits(outs[False])), rep
    finally:
        ctx.graph_release(g)
    for t in handles.values():
        ctx.release(t)


def test_decode_layer_route_to_missing_expert(ctx, oracle, dev):
    """A layer whose router selects experts that are not resident reports
    NotResident through the stream, as the device route list does: the
    router's last workgroup resolves the routes (one expert and the shared
    one resident of 32 rows, so at least five of the six routes miss)."""
    ctx.set_exact_numerics(False)
    L, _, handles = _setup(ctx, oracle, dev)
    other = LAYER + 1
    rng = np.random.default_rng(SEED)
    gate = ((rng.standard_normal((N_EXP, wl.HIDDEN)).astype(np.float32) * 0.02).view(np.uint32) >> 16)
    blk = mf.build_synthetic_quant_block([
        mf.SyntheticTensor(f"layers.{other}.ffn.gate.weight", 9, (N_EXP, wl.HIDDEN), gate.astype(np.uint16).tobytes(),
                           11, 2404),
        mf.SyntheticTensor(f"layers.{other}.ffn.gate.bias", 9, (N_EXP,), np.zeros(N_EXP, np.float32).tobytes(), 12,
                           2405)])
    ctx.store_router(other, blk, wl.HIDDEN)
    for e in (0, N_EXP):
        ctx.store_expert_synthetic(other, e, wl.HIDDEN, wl.INTER, SEED)
    L.layer_id, L.shared_layer = other, other
    cap, ld = 8, HEAD_DIM + 64
    hp = dev.put((rng.standard_normal(HC * wl.HIDDEN) * 0.5).astype(np.float32))
    kvp = dev.put(np.zeros((cap, ld), np.float32))
    ctx.deepseek_mhc_layer_async(L, 0, hp, kvp, ld, cap)
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.synchronize()
    assert e.value.name == "NotResident"
    for t in handles.values():
        ctx.release(t)
