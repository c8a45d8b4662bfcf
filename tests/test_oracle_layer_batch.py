"""CPU pinning of the oracle's batched layer (oracle.mhc_decode_layer_batch,
the batch path of E/server/generation.rs:2437-2590) against its single-token
layer (oracle.mhc_decode_layer, E/compute.rs:1448-1480 with the router
between the phases), at small shapes.

The batched layer differs from running the single-token layer at each
position in one respect only: the union MoE divides each position's router
weights by their sum (E/server/generation.rs:2491-2503) and sums the
experts in ascending id (moe_batch). With a MoE callback that does exactly
that for one position, the two compositions must agree bit for bit, the KV
cache included:

* the phases run in order (hc_pre, norm, attention, hc_post, hc_pre, norm,
  router, MoE, hc_post);
* each position reads its own residual;
* every KV row is written, and each window reads only rows at or before its
  position.

A mistake in the batch composition fails it: a swapped norm weight, the
attention residual instead of the post-attention state for hc_post, a
position's routes applied to another, a missing renormalisation. So does
dropping the renormalisation in the callback (the route_scale of 1.5 then
shows)."""
import numpy as np

HIDDEN, HC, HEADS, NOPE, ROPE, Q_LORA, GROUPS, O_LORA = 64, 4, 2, 32, 32, 32, 2, 32
N_EXP, ACTIVE, SCALE = 8, 2, 1.5


def _small_expert(rng, hidden=HIDDEN, inter=32):
    mats = []
    for rows, cols in ((inter, hidden), (inter, hidden), (hidden, inter)):
        p = rng.integers(0, 256, (rows, cols // 2)).astype(np.uint8)
        s = rng.integers(120, 130, (rows, cols // 32)).astype(np.uint8)
        mats.append((p, s, rows, cols, cols // 32))
    return tuple(mats)


def _bf16(rng, n):
    return ((1.0 + 0.1 * rng.standard_normal(n).astype(np.float32)).view(np.uint32) >> 16).astype(np.uint16)


def _setup(oracle, seed):
    rng = np.random.default_rng(seed)
    head_dim = NOPE + ROPE
    q_full = HEADS * head_dim
    mats = {"wq_a": (Q_LORA, HIDDEN), "wq_b": (q_full, Q_LORA), "wkv": (head_dim, HIDDEN),
            "wo_a": (GROUPS * O_LORA, q_full // GROUPS), "wo_b": (HIDDEN, GROUPS * O_LORA)}
    m = {n: rng.standard_normal(s) / np.sqrt(s[1]) for n, s in mats.items()}
    proj = {n: (lambda a: lambda x: (a @ np.asarray(x, np.float64)).astype(np.float32))(m[n])
            for n in ("wq_a", "wq_b", "wkv", "wo_b")}
    proj["wo_a_group"] = lambda g, x: (m["wo_a"][g * O_LORA:(g + 1) * O_LORA] @ np.asarray(x, np.float64)).astype(
        np.float32)
    mla = dict(proj=proj, q_norm=_bf16(rng, Q_LORA), kv_norm=_bf16(rng, head_dim),
               sink=rng.standard_normal(HEADS).astype(np.float32), heads=HEADS, nope_dim=NOPE, rope_dim=ROPE,
               o_groups=GROUPS, o_lora=O_LORA, physical_layer=0)
    mix = (2 + HC) * HC

    def hc_params():
        return ((rng.standard_normal((mix, HC * HIDDEN)) / np.sqrt(HC * HIDDEN)).astype(np.float32),
                (0.5 + rng.random(3)).astype(np.float32), (rng.standard_normal(mix) * 0.5).astype(np.float32))

    hc_attn, hc_ffn = hc_params(), hc_params()
    an, fnorm = _bf16(rng, HIDDEN), _bf16(rng, HIDDEN)
    gate = ((rng.standard_normal((N_EXP, HIDDEN)).astype(np.float32) * 0.3).view(np.uint32) >> 16).astype(np.uint16)
    bias = (rng.standard_normal(N_EXP) * 0.05).astype(np.float32)
    experts = {e: _small_expert(rng) for e in range(N_EXP)}
    shared = _small_expert(rng)
    return rng, mla, hc_attn, hc_ffn, an, fnorm, gate, bias, experts, shared


def test_batch_layer_equals_single_layers_with_the_batch_moe(oracle):
    rng, mla, hc_attn, hc_ffn, an, fnorm, gate, bias, experts, shared = _setup(oracle, 3)
    head_dim = NOPE + ROPE
    cap = 16
    cache0 = np.zeros((cap, head_dim), np.float32)
    cache0[:2] = (rng.standard_normal((2, head_dim)) * 0.3).astype(np.float32)
    positions = [2, 3, 4, 5]
    hs = (rng.standard_normal((len(positions), HC * HIDDEN)) * 0.5).astype(np.float32)

    cache_b = cache0.copy()
    got, ids_b, w_b = oracle.mhc_decode_layer_batch(hs, positions, HC, HIDDEN, hc_attn, hc_ffn, an, fnorm, mla,
                                                     gate, bias, ACTIVE, SCALE, experts, shared, cache_b)

    def moe_one(ids, w, g):  # the batch MoE of one position
        return oracle.moe_batch(experts, np.asarray(ids)[None], np.asarray(w, np.float32)[None],
                                np.asarray(g, np.float32)[None], shared)[0]

    cache_s = cache0.copy()
    for i, p in enumerate(positions):
        want, ids, w = oracle.mhc_decode_layer(hs[i], HC, HIDDEN, hc_attn, hc_ffn, an, fnorm, mla, gate, bias,
                                               ACTIVE, SCALE, moe_one, p, cache_s)
        assert list(ids) == list(ids_b[i]) and np.array_equal(np.asarray(w, np.float32), w_b[i]), p
        assert np.array_equal(got[i].view(np.uint32), want.view(np.uint32)), p
    assert np.array_equal(cache_b.view(np.uint32), cache_s.view(np.uint32))
    # the routes differ between positions, so a position's output is its own
    assert len({tuple(r) for r in ids_b.tolist()}) > 1


def test_batch_layer_renormalises_the_router_weights(oracle):
    """The single-token MoE with the router's weights as they come (summing
    to route_scale) gives another output: the batch path's division by the
    sum is what the first test checks, not an accident of the data."""
    rng, mla, hc_attn, hc_ffn, an, fnorm, gate, bias, experts, shared = _setup(oracle, 4)
    head_dim = NOPE + ROPE
    cache = np.zeros((8, head_dim), np.float32)
    h = (rng.standard_normal(HC * HIDDEN) * 0.5).astype(np.float32)
    got, _, w_b = oracle.mhc_decode_layer_batch(h[None], [0], HC, HIDDEN, hc_attn, hc_ffn, an, fnorm, mla, gate,
                                                 bias, ACTIVE, SCALE, experts, shared, cache.copy())
    assert abs(float(w_b[0].sum()) - SCALE) < 1e-5  # the router's weights carry route_scale

    def moe_scaled(ids, w, g):  # shared + routed with the weights as they come, ascending id
        out = oracle.fp4_expert_forward(*shared, g).astype(np.float32)
        acc = np.zeros(HIDDEN, np.float32)
        for e, wt in sorted(zip(ids, w)):
            acc = (acc + oracle.fp4_expert_forward(*experts[int(e)], g) * np.float32(wt)).astype(np.float32)
        return (out + acc).astype(np.float32)

    other, _, _ = oracle.mhc_decode_layer(h, HC, HIDDEN, hc_attn, hc_ffn, an, fnorm, mla, gate, bias, ACTIVE, SCALE,
                                          moe_scaled, 0, cache.copy())
    assert not np.allclose(got[0], other, rtol=1e-3, atol=0)
