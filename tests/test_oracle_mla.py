"""CPU pinning of the oracle's MLA glue (oracle.c: or_rms_norm,
or_rope_inv_freqs, or_rope_apply, or_window_attention; oracle.py:
mla_attention_decode).

* The reference's own known answers (tests/golden/reference_kats.json):
  RoPE at position 0, per-head RoPE prefixes, forward-then-inverse RoPE,
  the YaRN blend, the per-layer RoPE selection and the single-token MLA
  layer with identity projections (E/compute.rs:7730-7754, 8298-8599).
* Closed forms and float64 references that a plausible slip would fail: a
  dropped eps or weight in the RMS norm, a wrong rotation sign, a missing
  sink term or max shift in the softmax, a wrong key order.
* The summation orders: the RMS norm's sum of squares and the attention
  score dot run in index order; data where a pairwise sum gives other bits
  show that the order is the one checked."""
import json
from pathlib import Path

import numpy as np
import pytest

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())
F32 = np.float32


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def close(a, b, tol=1e-5):
    return abs(float(a) - float(b)) < tol


def test_rope_position_zero_is_identity(oracle):
    k = KATS["rope_position_zero"]
    inv = oracle.rope_inv_freqs(k["rope_dim"], k["theta"])
    got = oracle.rope_apply(k["values"], k["position"], inv)
    assert np.array_equal(got, np.array(k["expected"], np.float32))


def test_rope_rotates_each_head_prefix(oracle):
    k = KATS["rope_heads_prefix"]
    v = np.array(k["values"], np.float32).reshape(k["heads"], k["head_dim"])
    inv = oracle.rope_inv_freqs(k["rope_dim"], k["theta"])
    for h in range(k["heads"]):
        v[h, :k["rope_dim"]] = oracle.rope_apply(v[h, :k["rope_dim"]], k["position"], inv)
    sym = {"c": np.cos(1.0), "s": np.sin(1.0), "-s": -np.sin(1.0)}
    want = [sym[e] if isinstance(e, str) else e for e in k["expected"]]
    assert all(close(a, b) for a, b in zip(v.reshape(-1), want))


@pytest.mark.parametrize("name", ["rope_inverse", "rope_with_freqs"])
def test_rope_inverse_undoes_forward(oracle, name):
    k = KATS[name]
    inv = oracle.rope_inv_freqs(k["rope_dim"], k["theta"])
    fwd = oracle.rope_apply(k["values"], k["position"], inv)
    back = oracle.rope_apply(fwd, k["position"], inv, inverse=True)
    assert all(close(a, b) for a, b in zip(back, k["values"]))
    # rope_interleaved_in_place's per-pair theta^(-2i/dim) is the same table
    plain = np.array([np.float32(k["theta"]) ** np.float32(-(2.0 * i) / k["rope_dim"])
                      for i in range(k["rope_dim"] // 2)], np.float32)
    assert np.allclose(inv, plain, rtol=1e-6)


def test_yarn_blend(oracle):
    k = KATS["yarn_blend"]
    plain = oracle.rope_inv_freqs(k["rope_dim"], k["theta"])
    yarn = oracle.rope_inv_freqs(k["rope_dim"], k["theta"], tuple(k["yarn"]))
    factor = k["yarn"][0]
    assert plain.size == yarn.size == k["rope_dim"] // 2
    assert close(yarn[k["unchanged"]], plain[k["unchanged"]])
    assert close(yarn[k["scaled"]], plain[k["scaled"]] / factor)
    m = k["between"]
    assert plain[m] / factor < yarn[m] < plain[m]
    # float64 restatement of the ramp: low = floor(15.45) = 15, high = ceil(24.71) = 25
    dim, base = k["rope_dim"], np.log(k["theta"])
    cd = [dim * np.log(k["yarn"][3] / (r * 2 * np.pi)) / (2 * base) for r in (k["yarn"][1], k["yarn"][2])]
    low, high = max(np.floor(cd[0]), 0.0), min(np.ceil(cd[1]), dim - 1)
    assert (low, high) == (15.0, 25.0)
    for p in range(plain.size):
        ramp = min(max((p - low) / (high - low), 0.0), 1.0)
        want = plain[p] / factor * ramp + plain[p] * (1 - ramp)
        assert abs(yarn[p] - want) <= 2e-7 * plain[p], p


def test_rope_for_layer(oracle):
    for layer, theta, has_yarn in KATS["rope_for_layer"]["cases"]:
        t, y = oracle.rope_for_layer(layer)
        assert t == theta and (y is not None) == has_yarn


def test_rope_angles_against_float64(oracle):
    """The rotation of pair i by position * inv[i], against float64 sin/cos
    of the same f32 angle (glibc's sinf/cosf are within an ulp)."""
    rng = np.random.default_rng(3)
    inv = oracle.rope_inv_freqs(64, 160000.0, oracle.DEEPSEEK_V4_YARN)
    for pos in (1, 7, 127, 128, 4097, 65535, 1 << 20):
        v = rng.standard_normal(64).astype(np.float32)
        got = oracle.rope_apply(v, pos, inv)
        ang = (np.float32(pos) * inv).astype(np.float64)
        e, o = v[0::2].astype(np.float64), v[1::2].astype(np.float64)
        want = np.empty(64)
        want[0::2] = e * np.cos(ang) - o * np.sin(ang)
        want[1::2] = e * np.sin(ang) + o * np.cos(ang)
        assert np.max(np.abs(got - want)) < 1e-5 * (1 + np.max(np.abs(v))), pos
        # the rotation keeps each pair's length
        n_in = np.hypot(e, o)
        n_out = np.hypot(got[0::2].astype(np.float64), got[1::2].astype(np.float64))
        assert np.allclose(n_in, n_out, rtol=1e-6)


def test_rms_norm_closed_forms(oracle):
    # constant vector c: every output is c / sqrt(c^2 + 1e-6)
    for c in (0.5, -3.0, 1e-3):
        got = oracle.rms_norm(np.full(512, c, np.float32))
        assert np.allclose(got, c / np.sqrt(c * c + 1e-6), rtol=2e-6)
    # the eps matters for tiny inputs: 1e-4 -> 1e-4 / sqrt(1e-8 + 1e-6)
    got = oracle.rms_norm(np.full(8, 1e-4, np.float32))
    assert np.allclose(got, 1e-4 / np.sqrt(1e-8 + 1e-6), rtol=2e-6)
    # the bf16 weight multiplies after the normalisation
    rng = np.random.default_rng(1)
    x = rng.standard_normal(1024).astype(np.float32)
    wb = (np.float32(1.0) + 0.1 * rng.standard_normal(1024).astype(np.float32)).view(np.uint32) >> 16
    w = (wb.astype(np.uint32) << 16).view(np.float32)
    got = oracle.rms_norm(x, wb.astype(np.uint16))
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt(np.mean(x64 * x64) + 1e-6) * w
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)


def test_rms_norm_sums_in_order(oracle):
    """Sum of squares in index order: with one large square first, the
    small ones round away one by one; a pairwise sum keeps them."""
    x = np.full(1024, 1.0, np.float32)
    x[0] = 4096.0  # 2^24 first, then 1023 ones that each round away
    seq = np.float32(0.0)
    for v in x:
        seq = np.float32(seq + np.float32(v * v))
    assert seq == np.float32(2.0 ** 24)
    pairwise = np.sum(x * x, dtype=np.float32)
    assert pairwise != seq
    got = oracle.rms_norm(x)
    inv = np.float32(1.0) / np.sqrt(np.float32(seq / np.float32(1024)) + np.float32(1e-6))
    assert np.array_equal(bits(got), bits(x * inv))


def _attn64(q, keys, sink, nope, inv, pos):
    """float64 window softmax of one head with sink, then inverse RoPE."""
    s = keys @ q / np.sqrt(q.size)
    m = s.max()
    w = np.exp(s - m)
    den = w.sum() + (np.exp(sink - m) if sink is not None else 0.0)
    out = (w @ keys) / den
    ang = np.float32(pos) * inv.astype(np.float32)
    ang = ang.astype(np.float64)
    e, o = out[nope::2].copy(), out[nope + 1::2].copy()
    out[nope::2] = e * np.cos(ang) + o * np.sin(ang)
    out[nope + 1::2] = -e * np.sin(ang) + o * np.cos(ang)
    return out


@pytest.mark.parametrize("sink", [False, True])
def test_window_attention_against_float64(oracle, sink):
    rng = np.random.default_rng(5)
    heads, hd, nope, pos = 4, 128, 96, 300
    inv = oracle.rope_inv_freqs(hd - nope, 10000.0)
    q = rng.standard_normal((heads, hd)).astype(np.float32)
    win = rng.standard_normal((128, hd + 16)).astype(np.float32)  # cache rows wider than head_dim
    comp = rng.standard_normal((9, hd)).astype(np.float32)
    sk = rng.standard_normal(heads).astype(np.float32) if sink else None
    got = oracle.window_attention(q, hd, nope, win, comp, sk, inv, pos)
    keys = np.concatenate([win[:, :hd], comp]).astype(np.float64)
    for h in range(heads):
        want = _attn64(q[h].astype(np.float64), keys, None if sk is None else float(sk[h]), nope, inv, pos)
        assert np.max(np.abs(got[h] - want)) < 2e-5 * np.max(np.abs(want)), h
    # the sink lowers every weight: without it the output differs
    if sink:
        assert not np.allclose(got, oracle.window_attention(q, hd, nope, win, comp, None, inv, pos))


def test_window_attention_single_key_is_the_key(oracle):
    """Position 0: one key, weight exp(0) = 1, denominator 1, inverse RoPE at
    0 the identity, so each head's output is the key itself, bit for bit."""
    rng = np.random.default_rng(6)
    hd, nope = 64, 48
    inv = oracle.rope_inv_freqs(hd - nope, 10000.0)
    key = rng.standard_normal((1, hd)).astype(np.float32)
    q = rng.standard_normal((3, hd)).astype(np.float32)
    got = oracle.window_attention(q, hd, nope, key, None, None, inv, 0)
    assert np.array_equal(bits(got), bits(np.repeat(key, 3, axis=0)))
    # with a sink s: key / (1 + exp(s - score))
    sink = np.array([0.5, -1.0, 2.0], np.float32)
    got = oracle.window_attention(q, hd, nope, key, None, sink, inv, 0)
    for h in range(3):
        s = float(np.dot(q[h].astype(np.float64), key[0].astype(np.float64)) / 8.0)
        want = key[0] / (1.0 + np.exp(sink[h] - s))
        assert np.allclose(got[h], want, rtol=2e-6, atol=1e-7)


def test_mla_single_token_known_answer(oracle):
    k = KATS["mla_single_token"]
    mats = {n: np.array(k[n], np.float64) for n in ("wq_a", "wq_b", "wkv", "wo_a", "wo_b")}
    o_lora = k["o_lora"]
    # the reference runs these bf16 identity projections with gemv_bf16_rows;
    # with 0/1 weights every row picks one input, exactly in any order
    proj = {n: (lambda m: lambda x: (m @ np.asarray(x, np.float64)).astype(np.float32))(mats[n])
            for n in ("wq_a", "wq_b", "wkv", "wo_b")}
    proj["wo_a_group"] = lambda g, x: (mats["wo_a"][g * o_lora:(g + 1) * o_lora] @ x.astype(np.float64)).astype(
        np.float32)
    head_dim = k["nope_dim"] + k["rope_dim"]
    cache = np.zeros((1, head_dim), np.float32)
    got = oracle.mla_attention_decode(np.array(k["hidden"], np.float32), proj, None, None, None, k["heads"],
                                      k["nope_dim"], k["rope_dim"], k["o_groups"], o_lora, k["layer"],
                                      k["token_pos"], cache)
    ms = np.float32((1.0 + 4.0 + 9.0 + 16.0) / 4.0)
    inv_rms = np.float32(1.0) / np.sqrt(ms + np.float32(1e-6))
    kv = np.array([1.0, 2.0, 3.0, 4.0], np.float32) * inv_rms
    kv[:2] = oracle.act_quant(kv[:2], 64)
    want = oracle.act_quant(np.array([kv[0], kv[1], kv[2], kv[0]], np.float32), 64)
    assert all(close(a, b, k["tol"]) for a, b in zip(got, want))
    assert close(cache[0, 0], kv[0]) and close(cache[0, 3], kv[3])
