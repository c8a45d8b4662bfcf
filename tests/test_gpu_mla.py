"""GPU parity of the MLA attention glue (compute_deepseek_v4_mla_attention,
E/compute.rs:3924-4293) against the oracle, bit for bit: the RMS norms
(E/compute.rs:7110-7122, 3077-3107), interleaved RoPE with plain and YaRN
frequencies (E/compute.rs:2591-2649), the device act-quant, the window
softmax with sink (E/compute.rs:4106-4197), and whole decode layers at the
model's shapes (64 heads x 512 = 448 nope + 64 rope, q_lora 1024, 8 output
groups of 1024) through resident FP8 projections, on a sliding-window layer
and on a compressed (YaRN) layer with compressed rows and a full window."""
import numpy as np
import pytest

import wohper_amd
from wohper_amd import workloads as wl

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


class Dev:
    """Device copies of host arrays, freed together."""

    def __init__(self, ctx):
        self.ctx, self.ptrs = ctx, []

    def put(self, arr):
        arr = np.ascontiguousarray(arr)
        p = self.ctx.device_alloc(max(arr.nbytes, 4))
        self.ctx.to_device(p, arr)
        self.ptrs.append(p)
        return p

    def empty(self, nbytes):
        p = self.ctx.device_alloc(max(nbytes, 4))
        self.ptrs.append(p)
        return p

    def get(self, p, shape, dtype=np.float32):
        out = np.empty(shape, dtype)
        self.ctx.from_device(out, p)
        return out

    def free(self):
        for p in self.ptrs:
            self.ctx.device_free(p)
        self.ptrs = []


@pytest.fixture
def dev(ctx):
    d = Dev(ctx)
    yield d
    d.free()


def _bf16_weights(rng, n):
    w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    return (w.view(np.uint32) >> 16).astype(np.uint16)


@pytest.mark.parametrize("rows,n,weighted", [(1, 1024, True), (64, 512, False), (1, 512, True), (3, 7, False),
                                             (2, 4096, True)])
def test_rms_norm_bit_exact(ctx, oracle, dev, rows, n, weighted):
    rng = np.random.default_rng(rows * 100 + n)
    x = (rng.standard_normal((rows, n)) * np.exp2(rng.integers(-6, 6, (rows, 1)))).astype(np.float32)
    w = _bf16_weights(rng, n) if weighted else None
    xp, yp = dev.put(x), dev.empty(x.nbytes)
    ctx.rms_norm_async(xp, yp, rows, n, dev.put(w) if weighted else 0)
    ctx.synchronize()
    got = dev.get(yp, (rows, n))
    assert np.array_equal(bits(got), bits(oracle.rms_norm(x, w)))
    # in place
    ctx.rms_norm_async(xp, xp, rows, n, 0)
    ctx.synchronize()
    assert np.array_equal(bits(dev.get(xp, (rows, n))), bits(oracle.rms_norm(x)))


@pytest.mark.parametrize("rows,n", [(1, 4096), (64, 512), (3, 7)])
def test_rms_norm_tree_within_tolerance(ctx, oracle, dev, rows, n):
    """Exact numerics off: the sum of squares in a fixed tree changes only
    its rounding.  Both orders of n positive terms are within (n - 1) u of
    the exact sum (u = 2^-24), the square root halves that, and the two
    products after it add a rounding each: every value stays within
    (0.5 (n + 16) + 4) u relative of the reference's, and runs reproduce each
    other bit for bit."""
    rng = np.random.default_rng(rows + n)
    x = (rng.standard_normal((rows, n)) * np.exp2(rng.integers(-6, 6, (rows, 1)))).astype(np.float32)
    w = _bf16_weights(rng, n)
    xp, yp = dev.put(x), dev.empty(x.nbytes)
    ctx.set_exact_numerics(False)
    try:
        ctx.rms_norm_async(xp, yp, rows, n, dev.put(w))
        ctx.synchronize()
        got = dev.get(yp, (rows, n))
        ctx.rms_norm_async(xp, yp, rows, n, dev.put(w))
        ctx.synchronize()
        assert np.array_equal(bits(got), bits(dev.get(yp, (rows, n))))
    finally:
        ctx.set_exact_numerics(True)
    want = oracle.rms_norm(x, w).astype(np.float64)
    assert np.all(np.abs(got - want) <= (0.5 * (n + 16) + 4) * 2.0 ** -24 * np.abs(want) + 1e-30)


@pytest.mark.parametrize("layer", [0, 2])
def test_rope_bit_exact(ctx, oracle, dev, layer):
    theta, yarn = wohper_amd.deepseek_rope_for_layer(layer)
    inv = wohper_amd.rope_inv_freqs(64, theta, yarn)
    assert np.array_equal(bits(inv), bits(oracle.rope_inv_freqs(64, *oracle.rope_for_layer(layer))))
    ip = dev.put(inv)
    rng = np.random.default_rng(layer)
    heads, hd, nope = 64, 512, 448
    for pos in (0, 1, 127, 128, 1000, 65535, 65536, 1 << 20, (1 << 24) - 1):
        for inverse in (False, True):
            v = rng.standard_normal((heads, hd)).astype(np.float32)
            vp = dev.put(v)
            ctx.rope_async(vp, heads, hd, nope, ip, 32, pos, inverse)
            ctx.synchronize()
            got = dev.get(vp, (heads, hd))
            want = v.copy()
            for h in range(heads):
                want[h, nope:] = oracle.rope_apply(v[h, nope:], pos, inv, inverse)
            assert np.array_equal(bits(got), bits(want)), (pos, inverse)
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.rope_async(vp, heads, hd, 480, ip, 32, 5)
    assert e.value.name == "InvalidShape"


def test_act_quant_async_bit_exact(ctx, oracle, dev):
    rng = np.random.default_rng(9)
    v = (rng.standard_normal(32768 + 37) * np.exp2(rng.integers(-20, 20, 32768 + 37))).astype(np.float32)
    v[100] = np.nan
    p = dev.put(v)
    ctx.act_quant_dequant_async(p, v.size, 64)
    ctx.synchronize()
    assert np.array_equal(bits(dev.get(p, v.shape)), bits(oracle.act_quant(v, 64)))


@pytest.mark.parametrize("n_win,n_comp,sink,pos", [(1, 0, False, 0), (37, 0, True, 36), (128, 0, True, 500),
                                                   (128, 512, True, 2047), (5, 3, False, 4)])
def test_window_attention_bit_exact(ctx, oracle, dev, n_win, n_comp, sink, pos):
    rng = np.random.default_rng(n_win * 7 + n_comp)
    heads, hd, nope, ld = 64, 512, 448, 520
    inv = oracle.rope_inv_freqs(64, 160000.0, oracle.DEEPSEEK_V4_YARN)
    q = oracle.rms_norm(rng.standard_normal((heads, hd)).astype(np.float32))
    win = (rng.standard_normal((n_win, ld)) * 0.5).astype(np.float32)
    comp = (rng.standard_normal((n_comp, hd)) * 0.5).astype(np.float32)
    sk = rng.standard_normal(heads).astype(np.float32) if sink else None
    outp, scp = dev.empty(heads * hd * 4), dev.empty(heads * (n_win + n_comp) * 4)
    ctx.window_attention_async(dev.put(q), heads, hd, nope, dev.put(win), n_win, ld,
                               dev.put(comp) if n_comp else 0, n_comp, dev.put(sk) if sink else 0, dev.put(inv), 32,
                               pos, scp, outp)
    ctx.synchronize()
    got = dev.get(outp, (heads, hd))
    want = oracle.window_attention(q, hd, nope, win, comp if n_comp else None, sk, inv, pos)
    assert np.array_equal(bits(got), bits(want))


# ---------------------------------------------------------------- the layer
HEADS, NOPE, ROPE, Q_LORA, GROUPS, O_LORA = 64, 448, 64, 1024, 8, 1024
HEAD_DIM = NOPE + ROPE
SEED = 21


def _layer(ctx, dev, physical_layer, with_norms=True, with_sink=True):
    """Resident FP8 projections (f32 128x128 block scales) and bf16 norms."""
    shapes = {"wq_a": (Q_LORA, wl.HIDDEN), "wq_b": (HEADS * HEAD_DIM, Q_LORA), "wkv": (HEAD_DIM, wl.HIDDEN),
              "wo_a": (GROUPS * O_LORA, HEADS * HEAD_DIM // GROUPS), "wo_b": (wl.HIDDEN, GROUPS * O_LORA)}
    handles, host = {}, {}
    for i, (name, (r, c)) in enumerate(shapes.items()):
        sc = wl.fp8_block_scales(SEED * 100 + i, r, c)
        handles[name] = ctx.store_fp8_synthetic(r, c, SEED, 1000 + i, sc)
        host[name] = (wl.synth_fp8_host(ctx.lib, SEED, 1000 + i, r, c), sc, r, c)
    rng = np.random.default_rng(SEED)
    qn = _bf16_weights(rng, Q_LORA) if with_norms else None
    kn = _bf16_weights(rng, HEAD_DIM) if with_norms else None
    sink = rng.standard_normal(HEADS).astype(np.float32) if with_sink else None
    L = wohper_amd.WhMlaLayer(physical_layer, HEADS, NOPE, ROPE, GROUPS, O_LORA, handles["wq_a"], handles["wq_b"],
                              handles["wkv"], handles["wo_a"], handles["wo_b"],
                              dev.put(qn) if with_norms else None, dev.put(kn) if with_norms else None,
                              dev.put(sink) if with_sink else None)
    return L, host, qn, kn, sink, handles


def _proj(oracle, host):
    def gemv(name, x, r0=0, r1=None):
        w, sc, r, c = host[name]
        return oracle.fp8_gemv(w, r, c, sc, r // 128, c // 128, x, r0, r1 if r1 is not None else r)
    return {"wq_a": lambda x: gemv("wq_a", x), "wq_b": lambda x: gemv("wq_b", x), "wkv": lambda x: gemv("wkv", x),
            "wo_a_group": lambda g, x: gemv("wo_a", x, g * O_LORA, (g + 1) * O_LORA), "wo_b": lambda x: gemv("wo_b", x)}


def test_mla_decode_layer_window(ctx, oracle, dev):
    """Sliding-window layer 0 (theta 10000, no compressor): positions 0..3 in
    a row, the KV cache growing on both sides."""
    L, host, qn, kn, sink, handles = _layer(ctx, dev, 0)
    proj = _proj(oracle, host)
    cap, ld = 8, HEAD_DIM + 64
    kvp = dev.put(np.zeros((cap, ld), np.float32))
    cache = np.zeros((cap, ld), np.float32)
    rng = np.random.default_rng(1)
    for pos in range(4):
        x = rng.standard_normal(wl.HIDDEN).astype(np.float32)
        hp = dev.put(x)
        ctx.mla_attention_decode_async(L, pos, hp, kvp, ld, cap)
        ctx.synchronize()
        got = dev.get(hp, wl.HIDDEN)
        want = oracle.mla_attention_decode(x, proj, qn, kn, sink, HEADS, NOPE, ROPE, GROUPS, O_LORA, 0, pos, cache)
        assert np.array_equal(bits(dev.get(kvp, (cap, ld))[:pos + 1]), bits(cache[:pos + 1])), pos
        assert np.array_equal(bits(got), bits(want)), pos
    for h in handles.values():
        ctx.release(h)


def test_mla_decode_layer_compressed(ctx, oracle, dev):
    """Compressed layer 2 (theta 160000 with YaRN) at position 300: a full
    128-row window of earlier cache rows, 75 compressed rows from the caller,
    plain RMS norms (no norm tensors), no sink."""
    L, host, qn, kn, sink, handles = _layer(ctx, dev, 2, with_norms=False, with_sink=False)
    proj = _proj(oracle, host)
    cap, ld, pos = 320, HEAD_DIM, 300
    rng = np.random.default_rng(2)
    cache = (rng.standard_normal((cap, ld)) * 0.3).astype(np.float32)
    comp = (rng.standard_normal((75, HEAD_DIM)) * 0.3).astype(np.float32)
    kvp, cp = dev.put(cache), dev.put(comp)
    x = rng.standard_normal(wl.HIDDEN).astype(np.float32)
    hp = dev.put(x)
    ctx.mla_attention_decode_async(L, pos, hp, kvp, ld, cap, cp, comp.shape[0])
    ctx.synchronize()
    want = oracle.mla_attention_decode(x, proj, None, None, None, HEADS, NOPE, ROPE, GROUPS, O_LORA, 2, pos, cache,
                                       comp)
    assert np.array_equal(bits(dev.get(kvp, (cap, ld))), bits(cache))
    assert np.array_equal(bits(dev.get(hp, wl.HIDDEN)), bits(want))
    # shape and capacity errors
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.mla_attention_decode_async(L, cap, hp, kvp, ld, cap)
    assert e.value.name == "InvalidShape"
    bad = wohper_amd.WhMlaLayer.from_buffer_copy(L)
    bad.o_groups = 3
    with pytest.raises(wohper_amd.DeepSeekV4KernelError) as e:
        ctx.mla_attention_decode_async(bad, 0, hp, kvp, ld, cap)
    assert e.value.name == "InvalidShape"
    for h in handles.values():
        ctx.release(h)
