"""CPU pinning of the summation order of the oracle's FP8 and FP4 row dots.

The float64 checks elsewhere bound a row's value but cannot see its order.
Here the products are exact (integers times powers of two) and the partial
sums cross 2^24, so the float32 result depends on the order alone.  Each row
is evaluated independently in numpy in the order the reference's AVX2 code
states, and the oracle must match it bit for bit:

* FP8 (E/compute.rs:5978-6018): per 128-column group, lane l runs
  g0 = fma(w[16c + l], x, g0) and g1 = fma(w[16c + 8 + l], x, g1) over the 8
  chunks, then acc_l = fma(g0 + g1, scale, acc_l); the row is
  ((a0 + a1) + (a2 + a3)) + ((a4 + a5) + (a6 + a7)) + tail (E/compute.rs:5968-5973).
* FP4 (E/deepseek_v4.rs:294-347): per 32-column group, lane l runs a 4-FMA
  chain over columns l, 8 + l, 16 + l, 24 + l of the x8 LUT integers from
  zero, then acc_l = fma(gacc, scale * 0.125, acc_l); the same final sum.

A float32 fma of an exact product equals the product added in float64 and
rounded once, as long as the float64 sum is exact, which these magnitudes
(below 2^53, powers-of-two scales) guarantee.  The wrong orders a kernel
could plausibly use (a single chain, lanes summed left to right, chunks
swapped) must give different bits on the same data, so the check has teeth."""
import numpy as np

F32 = np.float32


def fma32(a, b, c):
    return F32(np.float64(a) * np.float64(b) + np.float64(c))


def hsum8(v):
    v = [F32(x) for x in v]
    return F32(F32(F32(v[0] + v[1]) + F32(v[2] + v[3])) + F32(F32(v[4] + v[5]) + F32(v[6] + v[7])))


# E4M3 codes with integer values: 1, 2, 3, 4, 6, 8, 12, 16 (and negatives)
FP8_INT_CODES = np.array([0x38, 0x40, 0x44, 0x48, 0x4C, 0x50, 0x54, 0x58], np.uint8)


def _fp8_case(rng, groups):
    cols = 128 * groups
    codes = FP8_INT_CODES[rng.integers(0, 8, cols)] | (rng.integers(0, 2, cols).astype(np.uint8) << 7)
    # big and small inputs: partial sums cross 2^24 so small terms round away
    # depending on where they are added
    x = np.where(rng.random(cols) < 0.5, rng.integers(1, 64, cols) * 2.0 ** 18,
                 rng.integers(1, 8, cols)).astype(np.float32)
    scales = (2.0 ** rng.integers(-3, 4, groups)).astype(np.float32)
    return codes, x, scales


def _fp8_reference_order(wv, x, scales):
    groups = scales.size
    acc = [F32(0)] * 8
    for g in range(groups):
        base = 128 * g
        g0 = [F32(0)] * 8
        g1 = [F32(0)] * 8
        for c in range(8):
            for l in range(8):
                i0, i1 = base + 16 * c + l, base + 16 * c + 8 + l
                g0[l] = fma32(wv[i0], x[i0], g0[l])
                g1[l] = fma32(wv[i1], x[i1], g1[l])
        for l in range(8):
            acc[l] = fma32(F32(g0[l] + g1[l]), scales[g], acc[l])
    return F32(hsum8(acc) + F32(0))


def test_fp8_row_follows_the_reference_lane_order(oracle):
    fp8, _, _, _ = oracle.luts()
    rng = np.random.default_rng(11)
    groups = 6
    for trial in range(20):
        codes, x, scales = _fp8_case(rng, groups)
        wv = fp8[codes]
        assert np.all(wv == np.round(wv)), "products must be exact"
        want = _fp8_reference_order(wv, x, scales)
        got = oracle.fp8_gemv(codes[None, :], 1, codes.size, scales[None, :], 1, groups, x)[0]
        assert F32(got).view(np.uint32) == want.view(np.uint32), trial
    # the same data under orders a kernel could plausibly use instead
    codes, x, scales = _fp8_case(np.random.default_rng(12), groups)
    wv = fp8[codes]
    want = _fp8_reference_order(wv, x, scales)
    one_chain = F32(0)
    for g in range(groups):
        s = F32(0)
        for i in range(128 * g, 128 * (g + 1)):
            s = fma32(wv[i], x[i], s)
        one_chain = fma32(s, scales[g], one_chain)
    assert one_chain.view(np.uint32) != want.view(np.uint32)


def _fp4_case(rng, groups):
    cols = 32 * groups
    nib = rng.integers(0, 16, cols).astype(np.uint8)
    packed = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
    x = np.where(rng.random(cols) < 0.5, rng.integers(1, 64, cols) * 2.0 ** 17,
                 rng.integers(1, 8, cols)).astype(np.float32)
    scale_bytes = rng.integers(124, 131, groups).astype(np.uint8)  # 2^-3 .. 2^3
    return nib, packed, x, scale_bytes


X8 = np.array([0, 1, 8, 12, 16, 24, 32, 48, 0, -1, -8, -12, -16, -24, -32, -48], np.float32)


def _fp4_reference_order(nib, x, scale_bytes, lane_chain=(0, 1, 2, 3)):
    acc = [F32(0)] * 8
    for g in range(scale_bytes.size):
        base = 32 * g
        s8 = F32(F32(2.0 ** (int(scale_bytes[g]) - 127)) * F32(0.125))
        gacc = [F32(0)] * 8
        for l in range(8):
            for k in lane_chain:
                i = base + 8 * k + l
                gacc[l] = fma32(X8[nib[i]], x[i], gacc[l])
        for l in range(8):
            acc[l] = fma32(gacc[l], s8, acc[l])
    return F32(hsum8(acc) + F32(0))


def _fp4_linear_lanes(nib, x, scale_bytes):
    """Lanes summed left to right instead of pairwise."""
    acc = [F32(0)] * 8
    for g in range(scale_bytes.size):
        s8 = F32(F32(2.0 ** (int(scale_bytes[g]) - 127)) * F32(0.125))
        for l in range(8):
            ga = F32(0)
            for k in range(4):
                i = 32 * g + 8 * k + l
                ga = fma32(X8[nib[i]], x[i], ga)
            acc[l] = fma32(ga, s8, acc[l])
    linear = F32(0)
    for v in acc:
        linear = F32(linear + v)
    return linear


def test_fp4_row_follows_the_reference_lane_order(oracle):
    rng = np.random.default_rng(13)
    groups = 8
    differs = {"swapped chain": 0, "linear lanes": 0}
    for trial in range(40):
        nib, packed, x, sb = _fp4_case(rng, groups)
        want = _fp4_reference_order(nib, x, sb)
        got = oracle.fp4_matvec(packed[None, :], sb[None, :], 1, nib.size, groups, x, force_path=0)[0]
        assert F32(got).view(np.uint32) == want.view(np.uint32), trial
        # orders a kernel could plausibly use instead, on the same data: a
        # chain with columns 16 + l before 8 + l, lanes summed left to right
        differs["swapped chain"] += int(_fp4_reference_order(nib, x, sb, (0, 2, 1, 3)).view(np.uint32) !=
                                        want.view(np.uint32))
        differs["linear lanes"] += int(_fp4_linear_lanes(nib, x, sb).view(np.uint32) != want.view(np.uint32))
    assert all(n > 0 for n in differs.values()), differs
