"""Parity helpers shared by the GPU tests: the reference dequantization of an
FP4 matrix and the matvec tolerance of the north-star bar,
max|diff| <= 1e-5 * ||w_row||_2 * ||x||_2 against the oracle on the same
input."""
import numpy as np


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def dequant(oracle, m):
    """Reference dequantized FP4 matrix (float64) of (packed, scales, rows, cols, scale_cols)."""
    packed, scales, rows, cols, scale_cols = m
    _, ue, fp4, _ = oracle.luts()
    packed = np.asarray(packed, np.uint8).reshape(rows, cols // 2)
    nib = np.empty((rows, cols), np.uint8)
    nib[:, 0::2] = packed & 15
    nib[:, 1::2] = packed >> 4
    sc = ue[np.asarray(scales, np.uint8).reshape(rows, scale_cols)].astype(np.float64)
    return fp4[nib].astype(np.float64) * np.repeat(sc, cols // scale_cols, axis=1)


_ROW_NORMS = {}


def row_norms(oracle, m):
    key = (id(m[0]), id(m[1]))
    if key not in _ROW_NORMS:
        w = dequant(oracle, m)
        _ROW_NORMS[key] = (m, np.sqrt((w * w).sum(axis=1)))
    return _ROW_NORMS[key][1]


def check_matvec(oracle, m, x, got, exact, what):
    want = oracle.fp4_matvec(*m, x)
    if exact:
        assert np.array_equal(bits(got), bits(want)), what
        return 0.0
    tol = 1e-5 * row_norms(oracle, m) * np.linalg.norm(np.asarray(x, np.float64))
    diff = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(diff <= tol), (what, float((diff / tol).max()))
    return float((diff / tol).max())
