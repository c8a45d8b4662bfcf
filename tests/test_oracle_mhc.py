"""CPU pinning of the oracle's mHC functions (oracle.c: or_hc_split_sinkhorn,
or_hc_pre, or_hc_post; E/compute.rs:4945-5092).

* The reference's own tests (tests/golden/reference_kats.json): the Sinkhorn
  split gives pre in (0, 1], post in (0, 2) and a doubly normalised comb;
  hc_pre then hc_post reproduce out[hidden] = post[1] y[0] + comb[1] x[0] +
  comb[hc + 1] x[hidden] (E/compute.rs:8457-8520).
* A float64 restatement of the same steps (sigmoids, row softmax, one column
  pass then rows-and-columns rounds, the RMS-scaled mixes, the pre-weighted
  sum) bounds every output; hc = 4 with copies that differ makes comb
  asymmetric, so a transposed comb in hc_post (the mistake the reference's
  own comment at E/compute.rs:5080-5085 warns of) fails it, and so does a
  wrong number of Sinkhorn rounds."""
import json
from pathlib import Path

import numpy as np

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def _sinkhorn64(mixes, scale, base, hc, iters, eps):
    m = np.asarray(mixes, np.float64)
    b = np.asarray(base, np.float64)
    sig = lambda v: 1.0 / (1.0 + np.exp(-v))
    pre = sig(m[:hc] * scale[0] + b[:hc]) + eps
    post = 2.0 * sig(m[hc:2 * hc] * scale[1] + b[hc:2 * hc])
    c = (m[2 * hc:] * scale[2] + b[2 * hc:]).reshape(hc, hc)
    c = np.exp(c - c.max(axis=1, keepdims=True))
    c = c / c.sum(axis=1, keepdims=True) + eps
    c = c / (c.sum(axis=0, keepdims=True) + eps)
    for _ in range(1, iters):
        c = c / (c.sum(axis=1, keepdims=True) + eps)
        c = c / (c.sum(axis=0, keepdims=True) + eps)
    return pre, post, c.reshape(-1)


def test_sinkhorn_known_answer(oracle):
    k = KATS["hc_sinkhorn"]
    hc = k["hc"]
    mix_hc = (2 + hc) * hc
    mixes = np.arange(mix_hc, dtype=np.float32) * np.float32(k["mix_step"]) + np.float32(k["mix_offset"])
    base = np.arange(mix_hc, dtype=np.float32) * np.float32(k["base_step"])
    pre, post, comb = oracle.hc_split_sinkhorn(mixes, k["scale"], base, hc, k["iters"], k["eps"])
    assert np.all((pre > 0) & (pre < k["pre_max"]))
    assert np.all((post > 0) & (post < k["post_max"]))
    c = comb.reshape(hc, hc).astype(np.float64)
    assert np.all(np.abs(c.sum(axis=1) - 1) < k["sum_tol"]) and np.all(np.abs(c.sum(axis=0) - 1) < k["sum_tol"])
    w = _sinkhorn64(mixes, k["scale"], base, hc, k["iters"], k["eps"])
    for got, want in zip((pre, post, comb), w):
        assert np.allclose(got, want, rtol=1e-5, atol=1e-7)


def test_sinkhorn_rounds_are_counted(oracle):
    """iters = 1 is one column pass only: columns sum to 1/(1+eps), rows do
    not; each iters value matches the float64 restatement with that count."""
    rng = np.random.default_rng(2)
    hc = 4
    mixes = rng.standard_normal((2 + hc) * hc).astype(np.float32)
    base = rng.standard_normal((2 + hc) * hc).astype(np.float32)
    scale = [0.7, 1.3, 2.0]
    _, _, c1 = oracle.hc_split_sinkhorn(mixes, scale, base, hc, 1, 1e-6)
    c1 = c1.reshape(hc, hc).astype(np.float64)
    assert np.allclose(c1.sum(axis=0), 1.0, atol=1e-5)
    assert not np.allclose(c1.sum(axis=1), 1.0, atol=1e-3)
    for iters in (1, 2, 3, 20):
        got = oracle.hc_split_sinkhorn(mixes, scale, base, hc, iters, 1e-6)
        want = _sinkhorn64(mixes, scale, base, hc, iters, 1e-6)
        for g, w in zip(got, want):
            assert np.allclose(g, w, rtol=2e-5, atol=1e-7), iters
    # a round fewer is measurably different
    a = oracle.hc_split_sinkhorn(mixes, scale, base, hc, 3, 1e-6)[2]
    b = _sinkhorn64(mixes, scale, base, hc, 2, 1e-6)[2]
    assert not np.allclose(a, b, rtol=1e-5, atol=1e-7)


def test_pre_post_known_answer(oracle):
    k = KATS["hc_pre_post"]
    hc, hidden = k["hc"], k["hidden"]
    hc_dim, mix_hc = hc * hidden, (2 + hc) * hc
    fn = np.array([[(j + d) * k["fn_step"] for d in range(hc_dim)] for j in range(mix_hc)], np.float32)
    base = np.arange(mix_hc, dtype=np.float32) * np.float32(k["base_step"])
    x = np.arange(hc_dim, dtype=np.float32) * np.float32(k["x_step"]) + np.float32(k["x_offset"])
    y, pre, post, comb, _ = oracle.hc_pre(fn, k["scale"], base, x, hc, hidden, k["iters"], k["eps"])
    assert np.all(np.isfinite(y))
    out = oracle.hc_post(y, x, post, comb, hc, hidden)
    assert np.all(np.isfinite(out))
    expected = post[1] * y[0] + comb[1] * x[0] + comb[hc + 1] * x[hidden]
    assert abs(float(out[hidden]) - float(expected)) < k["tol"]


def test_pre_post_against_float64(oracle):
    rng = np.random.default_rng(3)
    hc, hidden, iters, eps = 4, 256, 20, 1e-6
    hc_dim, mix_hc = hc * hidden, (2 + hc) * hc
    fn = (rng.standard_normal((mix_hc, hc_dim)) * 0.05).astype(np.float32)
    scale = [0.5, 0.8, 1.1]
    base = rng.standard_normal(mix_hc).astype(np.float32)
    x = rng.standard_normal(hc_dim).astype(np.float32)  # four copies that differ
    y, pre, post, comb, mixes = oracle.hc_pre(fn, scale, base, x, hc, hidden, iters, eps)
    x64 = x.astype(np.float64)
    inv = 1.0 / np.sqrt(np.mean(x64 * x64) + eps)
    m64 = fn.astype(np.float64) @ x64 * inv
    assert np.allclose(mixes, m64, rtol=1e-4, atol=1e-5)
    p64, q64, c64 = _sinkhorn64(mixes, scale, base, hc, iters, eps)
    assert np.allclose(pre, p64, rtol=1e-5) and np.allclose(post, q64, rtol=1e-5)
    assert np.allclose(comb, c64, rtol=1e-4, atol=1e-6)
    y64 = (pre.astype(np.float64)[:, None] * x64.reshape(hc, hidden)).sum(axis=0)
    assert np.allclose(y, y64, rtol=1e-5, atol=1e-6)
    out = oracle.hc_post(y, x, post, comb, hc, hidden)
    c = comb.reshape(hc, hc).astype(np.float64)
    out64 = post.astype(np.float64)[:, None] * y.astype(np.float64)[None, :] + c @ x64.reshape(hc, hidden)
    assert np.allclose(out, out64.reshape(-1), rtol=1e-5, atol=1e-5)
    # the transposed combination is a different result on these copies
    wrong = post.astype(np.float64)[:, None] * y.astype(np.float64)[None, :] + c.T @ x64.reshape(hc, hidden)
    assert not np.allclose(out, wrong.reshape(-1), rtol=1e-3, atol=1e-3)
