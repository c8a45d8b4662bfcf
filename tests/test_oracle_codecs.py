"""Pins the oracle's codecs: closed forms over every code, torch's OCP E4M3
decoder, and the reference's inline known answers."""
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def test_ue8m0_known_answers_and_closed_form(oracle):
    _, ue, _, _ = oracle.luts()
    for byte, want in KATS["ue8m0_decode"]["cases"]:
        assert ue[byte] == np.float32(want)
    for b in range(1, 255):
        assert ue[b] == np.float32(math.ldexp(1.0, b - 127)), b
    assert ue[0] == 0.0 and math.isinf(ue[255]) and ue[255] > 0


def test_fp8_matches_ocp_decoder_except_reference_special_codes(oracle):
    fp8, _, _, _ = oracle.luts()
    ocp = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    for b in range(256):
        if b in (0x7F, 0xFF):
            continue
        if b == 0x80:  # OCP -0, reference early-returns +0.0
            assert fp8[b] == 0.0 and not np.signbit(fp8[b])
            continue
        assert fp8[b].view(np.uint32) == ocp[b].view(np.uint32), hex(b)
    # the reference decodes the OCP NaN codes as +-(1 + 7/8) * 2^8
    assert fp8[0x7F] == 480.0 and fp8[0xFF] == -480.0


def test_fp8_sign_known_answers(oracle):
    fp8, _, _, _ = oracle.luts()
    k = KATS["fp8_sign"]
    assert all(fp8[b] > 0 for b in k["positive"])
    assert all(fp8[b] < 0 for b in k["negative"])
    assert all(fp8[b] == 0 for b in k["zero"])


def test_fp8_decode_with_scale_is_value_times_scale(oracle):
    fp8, _, _, _ = oracle.luts()
    L = oracle.lib()
    for b in range(256):
        for s in (1.0, 0.5, 2.0 ** -10, 3.0):
            assert L.or_decode_fp8_e4m3(b, s) == (np.float32(fp8[b]) * np.float32(s) if fp8[b] != 0 else 0.0)


# OCP MX spec E2M1 magnitudes by 3-bit code; the reference differs only at
# code 1 (its subnormal uses 2^-2 instead of 2^0: (m/2) * 2^-2 = 0.125).
OCP_E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def test_fp4_table_all_nibbles(oracle):
    _, _, fp4, _ = oracle.luts()
    for n in range(16):
        mag = OCP_E2M1[n & 7] if (n & 7) != 1 else 0.125
        want = -mag if (n & 8) and mag != 0 else mag
        assert fp4[n] == np.float32(want), n
    assert fp4[8] == 0.0 and not np.signbit(fp4[8])
    # the AVX2 path's x8 integer LUT (E/deepseek_v4.rs:285-287) is 8x the base values
    x8 = [0, 1, 8, 12, 16, 24, 32, 48, 0, -1, -8, -12, -16, -24, -32, -48]
    assert [int(v * 8) for v in fp4] == x8


def test_fp4_pair_sign_known_answer(oracle):
    k = KATS["fp4_pair_sign"]
    L = oracle.lib()
    lo = L.or_decode_fp4_e2m1(k["byte"] & 15, k["scale"])
    hi = L.or_decode_fp4_e2m1(k["byte"] >> 4, k["scale"])
    assert lo > 0 and hi < 0
    # [0xa2, 0x11] -> positive, negative, positive (deepseek_v4.rs:742-746)
    assert L.or_decode_fp4_e2m1(0x1, 2.0) > 0


def test_sorted_e4m3_lut(oracle):
    fp8, _, _, srt = oracle.luts()
    assert np.all(np.diff(srt.astype(np.float64)) >= 0)
    assert srt[0] == -480 and srt[-1] == 480
    assert np.count_nonzero(srt == 0) == 2
    assert sorted(fp8.tolist()) == srt.tolist()
