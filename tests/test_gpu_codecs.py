"""GPU: bit-exact dequantisation of resident tensors and the device libm
emulation, against the oracle (host glibc) over every code / wide samples."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_fp8_dequant_all_codes_bit_exact(ctx, oracle):
    fp8, _, _, _ = oracle.luts()
    codes = np.arange(256, dtype=np.uint8)
    rng = np.random.default_rng(0)
    w = np.concatenate([codes, rng.permutation(codes), rng.integers(0, 256, 128 * 4, dtype=np.uint8)])
    w = w.reshape(8, 128)
    for special in (False, True):
        ww = w.copy()
        if not special:
            ww[(ww & 0x7F) == 0x7F] = 0x11
        t = ctx.store_fp8(ww, 8, 128, np.ones((1, 1), np.float32), 1, 1, scale_format=1)
        got = ctx.dequant(t, 8, 128)
        want = fp8[ww]
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), special
        ctx.release(t)


def test_fp4_dequant_all_nibbles_and_scales_bit_exact(ctx, oracle):
    _, ue, fp4, _ = oracle.luts()
    rows, cols = 16, 512
    rng = np.random.default_rng(1)
    packed = rng.integers(0, 256, (rows, cols // 2)).astype(np.uint8)
    packed[0, :128] = np.arange(256, dtype=np.uint32).reshape(128, 2)[:, 0].astype(np.uint8)
    packed[1, :256] = np.arange(256, dtype=np.uint8)
    scales = rng.integers(0, 256, (rows, cols // 32)).astype(np.uint8)
    scales[0, :5] = [0, 1, 127, 254, 255]
    t = ctx.store_fp4(packed, scales, rows, cols, cols // 32)
    got = ctx.dequant(t, rows, cols)
    L = oracle.lib()
    want = np.empty((rows, cols), np.float32)
    for r in range(rows):
        for c in range(cols):
            b = packed[r, c // 2]
            nib = (b >> 4) if c & 1 else (b & 15)
            want[r, c] = L.or_decode_fp4_e2m1(int(nib), float(ue[scales[r, c // 32]]))
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all(), np.argwhere(~same)[:5]


def test_device_silu_and_expf_match_glibc(ctx, oracle):
    rng = np.random.default_rng(2)
    # silu's domain is x <= 10 (the gate is clamped first): every float in
    # (-inf, 10] at a stride, plus random and edge values
    neg = np.arange(0x80000000, 0xFF800001, 977, dtype=np.uint64).astype(np.uint32)
    pos = np.arange(0, 0x41200001, 977, dtype=np.uint32)
    x = np.concatenate([neg.view(np.float32), pos.view(np.float32),
                        rng.uniform(-10, 10, 1 << 20).astype(np.float32),
                        np.array([0.0, -0.0, 10.0, -10.0, 1e-38, -1e-38, -88.0, -200.0, 1e-10, -np.inf], np.float32)])
    got = ctx.debug_eval(0, x)
    want = oracle.silu_array(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    e = np.concatenate([-x, np.array([88.7, 88.72283, 88.73, 89.0, 200.0, 3e38, np.inf], np.float32)])
    e = e[e >= -10]
    got = ctx.debug_eval(1, e)
    want = oracle.expf_array(e)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_device_act_quant_scale_matches_glibc(ctx, oracle):
    rng = np.random.default_rng(3)
    a = np.exp(rng.uniform(-20, 30, 1 << 18)).astype(np.float32)
    # values hugging every power of two from 2^-13 to 2^30 times 448
    p = np.float32(448.0) * np.exp2(np.arange(-13, 30)).astype(np.float32)
    near = np.concatenate([(p.view(np.uint32).astype(np.int64) + d).astype(np.uint32)
                           for d in range(-40, 41)]).view(np.float32)
    a = np.concatenate([a, near, np.array([0.0, 1e-4, 5e-5, 448.0], np.float32)])
    got = ctx.debug_eval(2, a)
    want = oracle.act_quant_scale_array(a)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
