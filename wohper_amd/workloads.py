"""Seeded synthetic inputs of the decode-path workloads.

Weights are random (there is no checkpoint offline).  Large expert sets are
generated on the device by wh_store_expert_synthetic; wh_synth_fp4_host
reproduces any of them on the host byte for byte.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

HIDDEN = 4096          # E/deepseek_v4.rs:34
INTER = 2048           # E/deepseek_v4.rs:35
N_ROUTED = 256         # E/deepseek_v4.rs:37
TOPK = 6               # E/deepseek_v4.rs:38
LAYERS = 43            # E/deepseek_v4.rs:36
SCALE_LO, SCALE_HI = 119, 127   # UE8M0 exponents -8..0

FP4_EXPERT_BYTES = 3 * (INTER * HIDDEN // 2) + 3 * (INTER * HIDDEN // 32)   # 13,369,344


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), returned as float32."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    return (b.astype(np.uint32) << 16).view(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


@dataclass
class Fp8Gemv:
    w: np.ndarray          # uint8 [rows, cols] e4m3 codes
    scales: np.ndarray     # float32 [rows/128, cols/128]
    x: np.ndarray          # float32 (bf16-valued) [cols]


def fp8_gemv_case(rows=4096, cols=4096, seed=0, ue8m0_compatible=False) -> Fp8Gemv:
    """Uniform over the 254 finite E4M3 codes; block scales 2^U, U ~ U[-10,-4]
    (integer U for the UE8M0-compatible variant); x ~ N(0,1) rounded to bf16."""
    rng = np.random.default_rng(seed)
    finite = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    w = finite[rng.integers(0, finite.size, size=(rows, cols))]
    shape = (rows // 128, cols // 128)
    if ue8m0_compatible:
        u = rng.integers(-10, -3, size=shape)
    else:
        u = rng.uniform(-10.0, -4.0, size=shape)
    scales = np.exp2(u).astype(np.float32)
    x = bf16_round(rng.standard_normal(cols).astype(np.float32))
    return Fp8Gemv(w, scales, x)


def route_topk_sigmoid(logits: np.ndarray, k: int = TOPK):
    """Top-k experts by sigmoid score, weights s / sum(s) (f32)."""
    s = (1.0 / (1.0 + np.exp(-logits.astype(np.float64)))).astype(np.float32)
    idx = np.argsort(-s, kind="stable")[:k]
    w = s[idx]
    return idx.astype(np.int64), (w / np.float32(w.sum(dtype=np.float32))).astype(np.float32)


def moe_token_case(seed=2, n_experts=N_ROUTED):
    """One token: router logits ~ N(0,1) over the experts -> top-6, x ~ N(0,1) bf16."""
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal(n_experts).astype(np.float32)
    idx, w = route_topk_sigmoid(logits)
    x = bf16_round(rng.standard_normal(HIDDEN).astype(np.float32))
    return idx, w, x


def zipf_batch_routes(seed=4, n_tokens=64, n_experts=N_ROUTED, k=TOPK, s=1.1, hidden=HIDDEN):
    """Ragged batch: expert popularity p(perm[r]) proportional to (r + 1)^-s
    over a seeded permutation; each token draws k distinct experts by
    sequential weighted sampling without replacement; router scores are the
    sigmoid of per-token N(0,1) logits (the batch rule normalizes them);
    x ~ N(0,1) rounded to bf16.  Returns (ids [n, k] u32, scores [n, k] f32,
    x [n, hidden] f32)."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(n_experts)
    pop = np.empty(n_experts)
    pop[perm] = np.arange(1, n_experts + 1, dtype=np.float64) ** -s
    ids = np.empty((n_tokens, k), np.uint32)
    for t in range(n_tokens):
        avail = pop.copy()
        for j in range(k):
            e = rng.choice(n_experts, p=avail / avail.sum())
            ids[t, j] = e
            avail[e] = 0.0
    logits = rng.standard_normal((n_tokens, k))
    scores = (1.0 / (1.0 + np.exp(-logits))).astype(np.float32)
    x = bf16_round(rng.standard_normal((n_tokens, hidden)).astype(np.float32))
    return ids, scores, x


def synth_fp4_host(lib, seed: int, layer: int, expert: int, matrix: int, rows: int, cols: int,
                   scale_lo=SCALE_LO, scale_hi=SCALE_HI):
    """Host copy of the bytes wh_store_expert_synthetic writes for matrix 0/1/2
    (w1/w3/w2) of (layer, expert), in the reference layout."""
    stream = (layer << 40) ^ (expert << 8) ^ matrix
    packed = np.empty(rows * cols // 2, np.uint8)
    scales = np.empty(rows * cols // 32, np.uint8)
    u8p = ctypes.POINTER(ctypes.c_uint8)
    lib.wh_synth_fp4_host(seed, stream, packed.ctypes.data_as(u8p), packed.size, scales.ctypes.data_as(u8p),
                          scales.size, scale_lo, scale_hi)
    return packed.reshape(rows, cols // 2), scales.reshape(rows, cols // 32)


def synth_expert_host(lib, seed: int, layer: int, expert: int, hidden=HIDDEN, inter=INTER, scale_lo=SCALE_LO,
                      scale_hi=SCALE_HI):
    w1 = synth_fp4_host(lib, seed, layer, expert, 0, inter, hidden, scale_lo, scale_hi)
    w3 = synth_fp4_host(lib, seed, layer, expert, 1, inter, hidden, scale_lo, scale_hi)
    w2 = synth_fp4_host(lib, seed, layer, expert, 2, hidden, inter, scale_lo, scale_hi)
    return ((w1[0], w1[1], inter, hidden, hidden // 32), (w3[0], w3[1], inter, hidden, hidden // 32),
            (w2[0], w2[1], hidden, inter, inter // 32))


# One decode layer's FP8 projections (the engine's V4-Flash set,
# E/compute.rs:659-684): (name, rows, cols, row groups with distinct inputs).
DECODE_LAYER_FP8 = (
    ("wq_a", 1024, 4096, 1),
    ("wq_b", 32768, 1024, 1),
    ("wkv", 512, 4096, 1),
    ("wo_a", 8192, 4096, 8),     # 8 groups of 1024 rows, E/compute.rs:4244-4258
    ("wo_b", 4096, 8192, 1),
)
DECODE_LAYER_FP8_BYTES = sum(r * c + (r // 128) * (c // 128) * 4 for _, r, c, _ in DECODE_LAYER_FP8)  # 106,980,864


def fp8_block_scales(seed: int, rows: int, cols: int) -> np.ndarray:
    """f32 128x128 block scales 2^U, U ~ U[-10, -4]."""
    rng = np.random.default_rng(seed)
    return np.exp2(rng.uniform(-10.0, -4.0, size=(rows // 128, cols // 128))).astype(np.float32)


def synth_fp8_host(lib, seed: int, stream: int, rows: int, cols: int) -> np.ndarray:
    """Host copy of the bytes wh_store_fp8_synthetic generates, row-major."""
    w = np.empty(rows * cols, np.uint8)
    lib.wh_synth_fp8_host(seed, stream, w.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), w.size)
    return w.reshape(rows, cols)


def fp8_stream(layer: int, index: int) -> int:
    """Generator stream of FP8 projection `index` of `layer`."""
    return (1 << 62) ^ (layer << 16) ^ index
