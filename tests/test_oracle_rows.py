"""Pins the oracle's FP8 / FP4 row kernels: the reference's known answers,
its own fast-vs-per-element checks, float64 dots, and invariants that a
dropped term, a sign slip or a transposed operand would break."""
import json
from pathlib import Path

import numpy as np
import pytest

from conftest import lcg_bytes, lcg_f32

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def fp4_dense(oracle, packed, scales, rows, cols, scale_cols):
    """float64 dequantised matrix from the oracle's decoder (per element)."""
    _, ue, fp4, _ = oracle.luts()
    p = np.asarray(packed, np.uint8).reshape(rows, -1)
    nib = np.empty((rows, cols), np.uint8)
    nib[:, 0::2] = p[:, : (cols + 1) // 2] & 15
    nib[:, 1::2] = (p[:, : cols // 2] >> 4)
    s = ue[np.asarray(scales, np.uint8).reshape(rows, scale_cols)].astype(np.float64)
    return fp4[nib].astype(np.float64) * np.repeat(s, cols // scale_cols, axis=1)


def test_fp4_low_nibble_first_known_answer(oracle):
    k = KATS["fp4_low_nibble_first"]
    for path in (-1, 1, 2):
        y = oracle.fp4_matvec(k["packed"], k["scales"], k["rows"], k["cols"], k["scale_cols"], k["input"], path)
        assert np.all(np.abs(y - np.array(k["expected"])) < k["tol"])


def test_fp4_fast_path_matches_per_element_reference(oracle):
    k = KATS["fp4_fast_vs_elementwise"]
    rows, cols, sc = k["rows"], k["cols"], k["scale_cols"]
    state = k["seed"]
    seq = []
    for _ in range(rows * cols // 2 + rows * sc + cols):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        seq.append(state)
    packed = [v >> 24 for v in seq[: rows * cols // 2]]
    scales = [120 + (v >> 29) for v in seq[rows * cols // 2: rows * cols // 2 + rows * sc]]
    x = np.array([np.float32(v >> 16) / np.float32(65536.0) - np.float32(0.5) for v in seq[-cols:]], np.float32)
    fast = oracle.fp4_matvec(packed, scales, rows, cols, sc, x, -1)
    elem = oracle.fp4_matvec(packed, scales, rows, cols, sc, x, 2)
    ref64 = fp4_dense(oracle, packed, scales, rows, cols, sc) @ x.astype(np.float64)
    for r in range(rows):
        assert abs(fast[r] - elem[r]) <= k["tol_rel"] * max(abs(elem[r]), 1.0)
        assert abs(fast[r] - ref64[r]) <= 1e-6 * max(abs(ref64[r]), 1.0)


def test_fp8_dot_row_tail_known_answer(oracle):
    k = KATS["fp8_dot_row_tail"]
    cols, groups = k["cols"], k["groups"]
    w = np.array(lcg_bytes(k["weight_seed"], cols), np.uint8)
    x = lcg_f32(k["input_seed"], cols)
    _, ue, _, _ = oracle.luts()
    fp8, _, _, _ = oracle.luts()
    scales = ue[np.arange(groups) + k["scale_base"]]
    fast = oracle.fp8_dot_row(w, scales, cols // groups, x, avx2=True)
    ref = sum(float(fp8[w[c]] * scales[c // (cols // groups)]) * float(x[c]) for c in range(cols))
    assert abs(fast - ref) <= k["tol_rel"] * max(abs(ref), 1.0)
    scalar = oracle.fp8_dot_row(w, scales, cols // groups, x, avx2=False)
    assert abs(scalar - ref) <= k["tol_rel"] * max(abs(ref), 1.0)


@pytest.mark.parametrize("rows,cols,block", [(256, 512, 128), (64, 1024, 128), (96, 384, 48)])
def test_fp8_gemv_against_float64(oracle, rows, cols, block):
    rng = np.random.default_rng(rows + cols)
    finite = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    w = finite[rng.integers(0, finite.size, (rows, cols))]
    sr, sc = rows // block if rows % block == 0 else 1, cols // block
    scales = np.exp2(rng.uniform(-10, -4, (sr, sc))).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    y = oracle.fp8_gemv(w, rows, cols, scales, sr, sc, x)
    fp8, _, _, _ = oracle.luts()
    dense = fp8[w].astype(np.float64) * np.repeat(np.repeat(scales, rows // sr, 0), cols // sc, 1)
    ref = dense @ x.astype(np.float64)
    bound = 1e-5 * np.linalg.norm(dense, axis=1) * np.linalg.norm(x)
    assert np.all(np.abs(y - ref) <= bound)
    # dropping one scale group visibly breaks the bound
    cut = dense.copy()
    cut[:, :block] = 0
    assert not np.all(np.abs(cut @ x.astype(np.float64) - y) <= bound)


def test_fp8_rows_is_a_slice_of_tensorwise(oracle):
    rng = np.random.default_rng(7)
    rows, cols = 512, 512
    w = rng.integers(0, 256, (rows, cols)).astype(np.uint8)
    w[(w & 0x7F) == 0x7F] = 0
    scales = np.exp2(rng.integers(-8, 0, (4, 4))).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    full = oracle.fp8_gemv(w, rows, cols, scales, 4, 4, x)
    part = oracle.fp8_gemv(w, rows, cols, scales, 4, 4, x, row_start=200, row_end=330)
    assert np.array_equal(full[200:330], part)


@pytest.mark.parametrize("rows,cols,block,n", [(256, 1024, 128, 5), (96, 384, 48, 3), (128, 4096, 128, 16)])
def test_fp8_rows_multi_is_the_single_input_kernel(oracle, rows, cols, block, n):
    """rows_multi (decode each row once, then plain loads) against the
    single-input kernel (gathers) input by input: the reference states the
    two are bit-identical, and here they are two separate code paths.  The
    results also stay within the float64 bound, every code included (+-480
    and NaN-free), and a swapped input order is visible."""
    rng = np.random.default_rng(rows + n)
    w = rng.integers(0, 256, (rows, cols)).astype(np.uint8)
    sr, sc = rows // block if rows % block == 0 else 1, cols // block
    scales = np.exp2(rng.uniform(-10, -4, (sr, sc))).astype(np.float32)
    xs = rng.standard_normal((n, cols)).astype(np.float32)
    r0, r1 = 3, rows - 5
    got = oracle.fp8_gemv_rows_multi(w, rows, cols, scales, sr, sc, xs, r0, r1)
    fp8, _, _, _ = oracle.luts()
    dense = fp8[w].astype(np.float64) * np.repeat(np.repeat(scales, rows // sr, 0), cols // sc, 1)
    for i in range(n):
        single = oracle.fp8_gemv(w, rows, cols, scales, sr, sc, xs[i], r0, r1)
        assert np.array_equal(got[i].view(np.uint32), single.view(np.uint32)), i
        ref = dense[r0:r1] @ xs[i].astype(np.float64)
        assert np.all(np.abs(got[i] - ref) <= 1e-5 * np.linalg.norm(dense[r0:r1], axis=1) * np.linalg.norm(xs[i]))
    assert not np.array_equal(got[0], oracle.fp8_gemv(w, rows, cols, scales, sr, sc, xs[1], r0, r1))


@pytest.mark.parametrize("rows,cols", [(64, 4096), (128, 2048)])
def test_fp4_matvec_against_float64(oracle, rows, cols):
    rng = np.random.default_rng(rows)
    packed = rng.integers(0, 256, (rows, cols // 2)).astype(np.uint8)
    scales = rng.integers(119, 128, (rows, cols // 32)).astype(np.uint8)
    x = rng.standard_normal(cols).astype(np.float32)
    y = oracle.fp4_matvec(packed, scales, rows, cols, cols // 32, x)
    dense = fp4_dense(oracle, packed, scales, rows, cols, cols // 32)
    ref = dense @ x.astype(np.float64)
    bound = 1e-5 * np.linalg.norm(dense, axis=1) * np.linalg.norm(x)
    assert np.all(np.abs(y - ref) <= bound)
    # low nibble = even column: swapping nibbles must break the bound
    swapped = ((packed >> 4) | (packed << 4)).astype(np.uint8)
    ys = oracle.fp4_matvec(swapped, scales, rows, cols, cols // 32, x)
    assert not np.all(np.abs(ys - ref) <= bound)


def test_fp4_validation_errors(oracle):
    with pytest.raises(oracle.OracleError) as e:
        oracle.fp4_matvec([0], [127], 0, 2, 1, [1.0, 1.0])
    assert e.value.code == 1
    with pytest.raises(oracle.OracleError) as e:
        oracle.fp4_matvec([0, 0], [127], 1, 4, 3, [1.0] * 4)
    assert e.value.code == 2
    with pytest.raises(oracle.OracleError) as e:
        oracle.fp4_matvec([0], [127], 1, 4, 1, [1.0] * 4)
    assert e.value.code == 3


def test_fp4_nonfinite_output(oracle):
    with pytest.raises(oracle.OracleError) as e:
        oracle.fp4_matvec([0x22], [255], 1, 2, 1, [1.0, 1.0])
    assert e.value.code == 8
