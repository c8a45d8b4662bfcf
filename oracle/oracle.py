"""ctypes front-end of the CPU oracle (oracle/oracle.c) - test infrastructure.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, as the checker.  Build with `make -C oracle`.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboracle.so"

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


class Fp4Spec(ctypes.Structure):
    _fields_ = [
        ("packed", ctypes.POINTER(ctypes.c_uint8)),
        ("packed_len", ctypes.c_size_t),
        ("scales", ctypes.POINTER(ctypes.c_uint8)),
        ("scales_len", ctypes.c_size_t),
        ("rows", ctypes.c_size_t),
        ("cols", ctypes.c_size_t),
        ("scale_cols", ctypes.c_size_t),
    ]


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        c = ctypes
        f32p, u8p, sz = c.POINTER(c.c_float), c.POINTER(c.c_uint8), c.c_size_t
        sigs = {
            "or_decode_fp8_e4m3": (c.c_float, [c.c_uint8, c.c_float]),
            "or_decode_ue8m0_scale": (c.c_float, [c.c_uint8]),
            "or_decode_fp4_e2m1": (c.c_float, [c.c_uint8, c.c_float]),
            "or_luts": (None, [f32p, f32p, f32p, f32p]),
            "or_set_threads": (None, [c.c_int]),
            "or_thread_count": (c.c_int, []),
            "or_fp8_dot_row_avx2": (c.c_float, [u8p, f32p, sz, sz, f32p]),
            "or_fp8_dot_row_scalar": (c.c_float, [u8p, f32p, sz, sz, f32p]),
            "or_fp8_gemv": (c.c_int, [u8p, sz, sz, f32p, sz, sz, sz, sz, f32p, f32p, c.c_int]),
            "or_fp8_gemv_rows_multi": (c.c_int, [u8p, sz, sz, f32p, sz, sz, sz, sz, f32p, sz, sz, f32p, sz]),
            "or_fp4_dot_row_avx2": (c.c_float, [u8p, u8p, sz, sz, sz, f32p]),
            "or_fp4_matvec": (c.c_int, [u8p, sz, u8p, sz, sz, sz, sz, f32p, sz, f32p, sz, c.c_int]),
            "or_nearest_e4m3": (c.c_float, [c.c_float]),
            "or_act_quant_dequant": (None, [f32p, sz, sz]),
            "or_act_quant_scale": (c.c_float, [c.c_float]),
            "or_silu": (c.c_float, [c.c_float]),
            "or_swiglu": (c.c_float, [c.c_float, c.c_float]),
            "or_batch_route_weights": (None, [f32p, sz, sz, f32p]),
            "or_fp4_expert_forward": (c.c_int, [c.POINTER(Fp4Spec)] * 3 + [f32p, sz, f32p, sz, f32p, sz, c.c_int]),
            "or_route_weight_sum": (c.c_int, [f32p, sz, f32p]),
            "or_routed_combine": (None, [f32p, f32p, sz, sz, f32p]),
            "or_accumulate_expert": (None, [f32p, c.POINTER(c.c_size_t), f32p, sz, sz, f32p]),
            "or_silu_array": (None, [f32p, f32p, sz]),
            "or_swiglu_array": (None, [f32p, f32p, f32p, sz]),
            "or_expf_array": (None, [f32p, f32p, sz]),
            "or_act_quant_scale_array": (None, [f32p, f32p, sz]),
            "or_fp8_shared_expert": (c.c_int, [u8p, f32p, u8p, f32p, u8p, f32p, sz, sz, sz, sz, sz, sz, f32p, f32p]),
            "or_bf16_dot_row_avx2": (c.c_float, [c.POINTER(c.c_uint16), f32p, sz]),
            "or_bf16_gemv": (None, [c.POINTER(c.c_uint16), sz, sz, f32p, f32p]),
            "or_sqrt_softplus": (c.c_float, [c.c_float]),
            "or_sqrt_softplus_array": (None, [f32p, f32p, sz]),
            "or_log1pf_array": (None, [f32p, f32p, sz]),
            "or_rms_norm": (None, [f32p, sz, c.POINTER(c.c_uint16), f32p]),
            "or_rope_inv_freqs": (None, [sz, c.c_float, c.c_int, c.c_float, c.c_float, c.c_float, sz, f32p]),
            "or_rope_apply": (None, [f32p, sz, f32p, sz, c.c_int]),
            "or_window_attention": (None, [f32p, sz, sz, sz, f32p, sz, sz, f32p, sz, f32p, f32p, sz, sz, f32p]),
            "or_hc_split_sinkhorn": (c.c_int, [f32p, f32p, f32p, sz, sz, c.c_float, f32p, f32p, f32p]),
            "or_hc_pre": (c.c_int, [f32p, f32p, f32p, sz, sz, sz, c.c_float, f32p, f32p, f32p, f32p, f32p, f32p]),
            "or_hc_post": (None, [f32p, f32p, f32p, f32p, f32p, sz, sz]),
            "or_route_select": (c.c_int, [f32p, sz, f32p, c.POINTER(c.c_uint32), sz, sz, c.c_int, c.c_float,
                                          c.POINTER(c.c_uint32), sz, c.POINTER(c.c_uint32), f32p,
                                          c.POINTER(sz)]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _f(a):
    return np.ascontiguousarray(a, np.float32)


def _u(a):
    return np.ascontiguousarray(a, np.uint8)


def _pf(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _pu(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8))


class OracleError(RuntimeError):
    def __init__(self, code):
        self.code = code
        super().__init__(f"oracle status {code}")


def luts():
    fp8, ue, fp4, srt = (np.zeros(256, np.float32), np.zeros(256, np.float32),
                         np.zeros(16, np.float32), np.zeros(256, np.float32))
    lib().or_luts(_pf(fp8), _pf(ue), _pf(fp4), _pf(srt))
    return fp8, ue, fp4, srt


def set_threads(n: int):
    lib().or_set_threads(int(n))


def thread_count() -> int:
    return lib().or_thread_count()


def decode_ue8m0(scales_u8) -> np.ndarray:
    _, ue, _, _ = luts()
    return ue[_u(scales_u8)]


def fp8_gemv(w, rows, cols, scales_f32, scale_rows, scale_cols, x, row_start=0, row_end=None, avx2=True):
    w, s, x = _u(w), _f(scales_f32), _f(x)
    row_end = rows if row_end is None else row_end
    y = np.zeros(row_end - row_start, np.float32)
    st = lib().or_fp8_gemv(_pu(w), rows, cols, _pf(s), scale_rows, scale_cols, row_start, row_end, _pf(x),
                           _pf(y), 1 if avx2 else 0)
    if st:
        raise OracleError(st)
    return y


def fp8_gemv_rows_multi(w, rows, cols, scales_f32, scale_rows, scale_cols, xs, row_start=0, row_end=None):
    """gemv_fp8_e4m3_ue8m0_rows_multi (E/compute.rs:6384-6577): each row
    decoded once, then every input of xs [n, cols] dotted in the single-input
    order.  Returns [n, row_end - row_start]."""
    w, s = _u(w), _f(scales_f32)
    xs = np.ascontiguousarray(xs, np.float32)
    n = xs.shape[0]
    row_end = rows if row_end is None else row_end
    y = np.zeros((n, row_end - row_start), np.float32)
    st = lib().or_fp8_gemv_rows_multi(_pu(w), rows, cols, _pf(s), scale_rows, scale_cols, row_start, row_end,
                                      _pf(xs), n, xs.shape[1], _pf(y), y.shape[1])
    if st:
        raise OracleError(st)
    return y


def fp8_dot_row(w_row, scales_f32, col_group, x, avx2=True):
    w, s, x = _u(w_row), _f(scales_f32), _f(x)
    fn = lib().or_fp8_dot_row_avx2 if avx2 else lib().or_fp8_dot_row_scalar
    return fn(_pu(w), _pf(s), s.size, col_group, _pf(x))


def fp4_matvec(packed, scales, rows, cols, scale_cols, x, force_path=-1):
    p, s, x = _u(packed), _u(scales), _f(x)
    y = np.zeros(rows, np.float32)
    st = lib().or_fp4_matvec(_pu(p), p.size, _pu(s), s.size, rows, cols, scale_cols, _pf(x), x.size, _pf(y),
                             y.size, force_path)
    if st:
        raise OracleError(st)
    return y


def act_quant(values, block=64):
    v = _f(values).copy()
    lib().or_act_quant_dequant(_pf(v), v.size, block)
    return v


def act_quant_scale(amax: float) -> float:
    return lib().or_act_quant_scale(amax)


def nearest_e4m3(t: float) -> float:
    return lib().or_nearest_e4m3(t)


def silu(x: float) -> float:
    return lib().or_silu(x)


def swiglu(g: float, u: float) -> float:
    return lib().or_swiglu(g, u)


def _spec(m):
    packed, scales, rows, cols, scale_cols = m
    p, s = _u(packed), _u(scales)
    spec = Fp4Spec(_pu(p), p.size, _pu(s), s.size, rows, cols, scale_cols)
    return spec, (p, s)


def fp4_expert_forward(w1, w3, w2, x, force_path=-1, scratch_len=None):
    """w1/w3/w2 = (packed, scales, rows, cols, scale_cols)."""
    s1, k1 = _spec(w1)
    s3, k3 = _spec(w3)
    s2, k2 = _spec(w2)
    x = _f(x)
    y = np.zeros(w2[2], np.float32)
    n_scratch = 2 * w1[2] if scratch_len is None else scratch_len
    scratch = np.zeros(max(1, n_scratch), np.float32)
    st = lib().or_fp4_expert_forward(ctypes.byref(s1), ctypes.byref(s3), ctypes.byref(s2), _pf(x), x.size,
                                     _pf(y), y.size, _pf(scratch), n_scratch, force_path)
    if st:
        raise OracleError(st)
    return y


def routed_combine(outs, weights):
    outs, w = _f(outs), _f(weights)
    n, hidden = outs.shape
    out = np.zeros(hidden, np.float32)
    lib().or_routed_combine(_pf(outs), _pf(w), n, hidden, _pf(out))
    return out


def route_weight_sum(weights):
    w = _f(weights)
    s = ctypes.c_float()
    ok = lib().or_route_weight_sum(_pf(w), w.size, ctypes.byref(s))
    return s.value if ok else None


def accumulate_expert(y_per_target, positions, weights, routed_acc):
    y, w = _f(y_per_target), _f(weights)
    pos = np.ascontiguousarray(positions, np.uintp)
    acc = _f(routed_acc).copy()
    hidden = acc.shape[-1]
    lib().or_accumulate_expert(_pf(y), pos.ctypes.data_as(ctypes.POINTER(ctypes.c_size_t)), _pf(w), w.size,
                               hidden, _pf(acc))
    return acc


def batch_route_weights(scores):
    """[npos, topk] router scores -> the batch union's weights
    (E/server/generation.rs:2491-2503)."""
    sc = _f(scores)
    w = np.empty_like(sc)
    npos, topk = sc.shape
    lib().or_batch_route_weights(_pf(sc), npos, topk, _pf(w))
    return w


def moe_batch(experts, route_ids, route_scores, x, shared=None):
    """The batch-prefill routed MoE (E/server/generation.rs:2487-2569): union
    of the selected experts keyed by id, each expert's targets in position
    order, experts taken in ascending id (the reference's submission order),
    acc_p += y * w per target (accumulate_expert_for_positions,
    E/compute.rs:1779-1810); with a shared expert out_p = shared(x_p) + acc_p
    (E/compute.rs:1838-1852).  experts: id -> (w1, w3, w2) matrices as taken
    by fp4_expert_forward; shared: one such triple or None."""
    ids = np.asarray(route_ids)
    x = _f(x)
    npos, topk = ids.shape
    w = batch_route_weights(route_scores)
    union = {}
    for p in range(npos):
        for k in range(topk):
            union.setdefault(int(ids[p, k]), []).append((p, w[p, k]))
    acc = np.zeros_like(x)
    for e in sorted(union):
        targets = union[e]
        ys = np.stack([fp4_expert_forward(*experts[e], x[p]) for p, _ in targets])
        acc = accumulate_expert(ys, [p for p, _ in targets], [wt for _, wt in targets], acc)
    if shared is not None:
        sh = np.stack([fp4_expert_forward(*shared, x[p]) for p in range(npos)])
        acc = (sh + acc).astype(np.float32)
    return acc


def fp8_shared_expert(w1, s1, w3, s3, w2, s2, hidden, inter, x):
    """compute_deepseek_fp8_shared_expert_into_hidden (E/compute.rs:5545-5614):
    W* are E4M3 bytes [rows][cols], s* f32 128x128 block scales."""
    w1, w3, w2 = _u(w1), _u(w3), _u(w2)
    s1, s3, s2 = _f(s1), _f(s3), _f(s2)
    x = _f(x)
    y = np.zeros(hidden, np.float32)
    st = lib().or_fp8_shared_expert(_pu(w1), _pf(s1), _pu(w3), _pf(s3), _pu(w2), _pf(s2), hidden, inter,
                                    s1.shape[0], s1.shape[1], s2.shape[0], s2.shape[1], _pf(x), _pf(y))
    if st:
        raise OracleError(st)
    return y


def swiglu_array(g, u):
    """DeepSeek-V4 SwiGLU elementwise (E/deepseek_v4.rs:590-594)."""
    g, u = _f(g), _f(u)
    h = np.empty_like(g)
    lib().or_swiglu_array(_pf(g), _pf(u), _pf(h), g.size)
    return h


def silu_array(x):
    x = _f(x)
    y = np.empty_like(x)
    lib().or_silu_array(_pf(x), _pf(y), x.size)
    return y


def expf_array(x):
    x = _f(x)
    y = np.empty_like(x)
    lib().or_expf_array(_pf(x), _pf(y), x.size)
    return y


def act_quant_scale_array(amax):
    a = _f(amax)
    y = np.empty_like(a)
    lib().or_act_quant_scale_array(_pf(a), _pf(y), a.size)
    return y


# ------------------------------------------------------------------ router
ROUTER_RAW_LOGITS = 0
ROUTER_SQRT_SOFTPLUS = 1


def bf16_gemv(w_bits, x):
    """gemv_bf16_tensorwise (E/compute.rs:6139-6172) on bf16 bit patterns
    [rows, cols] (uint16)."""
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    rows, cols = w.shape
    x = _f(x)
    y = np.zeros(rows, np.float32)
    lib().or_bf16_gemv(w.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), rows, cols, _pf(x), _pf(y))
    return y


def sqrt_softplus(x):
    x = _f(np.atleast_1d(x))
    y = np.empty_like(x)
    lib().or_sqrt_softplus_array(_pf(x), _pf(y), x.size)
    return y


def log1pf(x):
    x = _f(np.atleast_1d(x))
    y = np.empty_like(x)
    lib().or_log1pf_array(_pf(x), _pf(y), x.size)
    return y


def route_select(logits, active, available=None, bias=None, math=ROUTER_SQRT_SOFTPLUS, route_scale=1.5,
                 hash_ids=None):
    """route_experts_from_dense_block after the gate GEMV (E/compute.rs:2129-2268):
    returns (expert ids, weights)."""
    lg = _f(logits)
    rows = lg.size
    av = np.ascontiguousarray(np.arange(rows) if available is None else available, dtype=np.uint32)
    b = None if bias is None else _f(bias)
    h = None if hash_ids is None else np.ascontiguousarray(hash_ids, dtype=np.uint32)
    cap = max(1, int(active))
    ids = np.zeros(cap, np.uint32)
    sc = np.zeros(cap, np.float32)
    n = ctypes.c_size_t()
    u32p = ctypes.POINTER(ctypes.c_uint32)
    lib().or_route_select(_pf(lg), rows, None if b is None else _pf(b), av.ctypes.data_as(u32p), av.size, active,
                          math, route_scale, None if h is None else h.ctypes.data_as(u32p),
                          0 if h is None else h.size, ids.ctypes.data_as(u32p), _pf(sc), ctypes.byref(n))
    return ids[:n.value].copy(), sc[:n.value].copy()


# ----------------------------------------------------------------- MLA glue

DEEPSEEK_V4_YARN = (16.0, 32.0, 1.0, 65536)  # factor, beta_fast, beta_slow, original_seq_len
COMPRESS_RATIOS = [0, 0] + [4, 128] * 20 + [4, 0]  # E/compute.rs:2552-2555


def rope_for_layer(physical_layer: int):
    """deepseek_rope_for_layer, E/compute.rs:2575-2586: (theta, yarn or None)."""
    ratio = COMPRESS_RATIOS[physical_layer] if physical_layer < len(COMPRESS_RATIOS) else 0
    return (160000.0, DEEPSEEK_V4_YARN) if ratio > 0 else (10000.0, None)


def rms_norm(x, w_bf16=None):
    """Rows of x (last axis) through rms_norm_in_place / apply_weighted_rms_norm."""
    x = _f(x)
    out = np.empty_like(x)
    rows = x.reshape(-1, x.shape[-1])
    o = out.reshape(-1, x.shape[-1])
    wp = None
    if w_bf16 is not None:
        w_bf16 = np.ascontiguousarray(w_bf16, np.uint16)
        wp = w_bf16.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))
    for r in range(rows.shape[0]):
        xr = np.ascontiguousarray(rows[r])
        yr = np.empty_like(xr)
        lib().or_rms_norm(_pf(xr), xr.size, wp, _pf(yr))
        o[r] = yr
    return out


def rope_inv_freqs(rope_dim: int, theta: float, yarn=None):
    out = np.zeros(max(rope_dim // 2, 1), np.float32)
    f, bf, bs, n = yarn if yarn is not None else (0.0, 0.0, 0.0, 0)
    lib().or_rope_inv_freqs(rope_dim, theta, 1 if yarn is not None else 0, f, bf, bs, n, _pf(out))
    return out[:rope_dim // 2]


def rope_apply(values, position: int, inv_freqs, inverse=False):
    v = _f(values).copy()
    inv = _f(inv_freqs)
    lib().or_rope_apply(_pf(v), position, _pf(inv), inv.size, 1 if inverse else 0)
    return v


def window_attention(q, head_dim, nope_dim, win, comp, sink, inv_freqs, token_pos):
    """q [heads, head_dim]; win [n_win, >= head_dim] (cache rows); comp
    [n_comp, head_dim]; sink [heads] or None."""
    q = _f(q)
    heads = q.shape[0]
    win = _f(win)
    comp = _f(comp) if comp is not None and len(comp) else np.zeros((0, head_dim), np.float32)
    inv = _f(inv_freqs)
    out = np.zeros((heads, head_dim), np.float32)
    s_arr = _f(sink) if sink is not None else None
    sp = _pf(s_arr) if s_arr is not None else None
    lib().or_window_attention(_pf(q), heads, head_dim, nope_dim, _pf(win), win.shape[0], win.shape[1], _pf(comp),
                              comp.shape[0], sp, _pf(inv), inv.size, token_pos, _pf(out))
    return out


def mla_attention_decode(x, proj, q_norm, kv_norm, sink, heads, nope_dim, rope_dim, o_groups, o_lora,
                         physical_layer, token_pos, kv_cache, comp=None):
    """compute_deepseek_v4_mla_attention (E/compute.rs:3924-4293) for one
    position.  proj: callables name -> (input -> output) for wq_a, wq_b,
    wkv, wo_a_group(g, input) and wo_b; q_norm / kv_norm: bf16 weights or
    None; kv_cache [capacity, >= head_dim] is updated at token_pos.  Returns
    the new hidden state."""
    head_dim = nope_dim + rope_dim
    theta, yarn = rope_for_layer(physical_layer)
    inv = rope_inv_freqs(rope_dim, theta, yarn)
    xq = act_quant(x, 64)
    ql = proj["wq_a"](xq)
    ql = rms_norm(ql, q_norm)
    ql = act_quant(ql, 64)
    q = proj["wq_b"](ql).reshape(heads, head_dim)
    q = rms_norm(q)
    for h in range(heads):
        q[h, nope_dim:] = rope_apply(q[h, nope_dim:], token_pos, inv)
    kv = proj["wkv"](xq)
    kv = rms_norm(kv, kv_norm)
    kv[nope_dim:] = rope_apply(kv[nope_dim:], token_pos, inv)
    kv[:nope_dim] = act_quant(kv[:nope_dim], 64)
    kv_cache[token_pos, :head_dim] = kv
    context = token_pos + 1
    ws = max(0, context - 128)
    att = window_attention(q, head_dim, nope_dim, kv_cache[ws:context], comp, sink, inv, token_pos)
    att = act_quant(att.reshape(-1), 64)
    group_in = heads * head_dim // o_groups
    om = np.concatenate([proj["wo_a_group"](g, att[g * group_in:(g + 1) * group_in]) for g in range(o_groups)])
    om = act_quant(om, 64)
    return proj["wo_b"](om)


# ---------------------------------------------------------------------- mHC

def hc_split_sinkhorn(mixes, scale, base, hc: int, iters: int = 20, eps: float = 1e-6):
    """hc_split_sinkhorn_scalar (E/compute.rs:4945-5014): (pre, post, comb)."""
    m, s, b = _f(mixes), _f(scale), _f(base)
    pre, post, comb = np.zeros(hc, np.float32), np.zeros(hc, np.float32), np.zeros(hc * hc, np.float32)
    lib().or_hc_split_sinkhorn(_pf(m), _pf(s), _pf(b), hc, iters, eps, _pf(pre), _pf(post), _pf(comb))
    return pre, post, comb


def hc_pre(fn, scale, base, x, hc: int, hidden: int, iters: int = 20, eps: float = 1e-6):
    """hc_pre_into (E/compute.rs:5016-5050): (y, pre, post, comb, mixes)."""
    f, s, b, xx = _f(fn), _f(scale), _f(base), _f(x)
    mix_hc = (2 + hc) * hc
    y = np.zeros(hidden, np.float32)
    pre, post, comb = np.zeros(hc, np.float32), np.zeros(hc, np.float32), np.zeros(hc * hc, np.float32)
    mixes = np.zeros(mix_hc, np.float32)
    st = lib().or_hc_pre(_pf(f), _pf(s), _pf(b), hc, hidden, iters, eps, _pf(xx), _pf(y), _pf(pre), _pf(post),
                         _pf(comb), _pf(mixes))
    if st:
        raise OracleError(st)
    return y, pre, post, comb, mixes


def hc_post(y, residual, post, comb, hc: int, hidden: int):
    """hc_post_into (E/compute.rs:5055-5092)."""
    out = np.zeros(hc * hidden, np.float32)
    lib().or_hc_post(_pf(_f(y)), _pf(_f(residual)), _pf(_f(post)), _pf(_f(comb)), _pf(out), hc, hidden)
    return out


# ------------------------------------------------------------ decode layer

def mhc_decode_layer(hidden_hc, hc: int, hidden: int, hc_attn, hc_ffn, attn_norm, ffn_norm, mla: dict, gate_bits,
                     bias, active: int, route_scale: float, moe, token_pos: int, kv_cache, comp=None,
                     iters: int = 20, eps: float = 1e-6):
    """compute_layer_deepseek_mhc (E/compute.rs:1448-1480) for one decode
    position, with the router between its phases as the engine runs them
    (E/server/generation.rs:719-836):
      phase 1 (E/compute.rs:1552-1630): residual = hidden; y = hc_pre(hc_attn);
      y = rms_norm(y, attn_norm); y = MLA(y); hidden = hc_post(y, residual);
      g = rms_norm(hc_pre(hc_ffn, hidden), ffn_norm);
      router (route_experts_from_dense_block, E/compute.rs:2129-2268) on g:
      bf16 gate GEMV, sqrt-softplus, biased top-`active`;
      phase 2 (E/compute.rs:1641-1700): z = moe(ids, weights, g) (shared +
      routed experts); hidden = hc_post(z, hidden after phase 1).
    hc_attn / hc_ffn: (fn, scale, base); mla: the keyword arguments of
    mla_attention_decode besides x, token_pos, kv_cache and comp.  Returns
    (new hidden, ids, weights); kv_cache is updated at token_pos."""
    residual = _f(hidden_hc).copy()
    y, _, post, comb, _ = hc_pre(*hc_attn, residual, hc, hidden, iters, eps)
    y = rms_norm(y, attn_norm)
    y = mla_attention_decode(y, token_pos=token_pos, kv_cache=kv_cache, comp=comp, **mla)
    h = hc_post(y, residual, post, comb, hc, hidden)
    g, _, post2, comb2, _ = hc_pre(*hc_ffn, h, hc, hidden, iters, eps)
    g = rms_norm(g, ffn_norm)
    ids, w = route_select(bf16_gemv(gate_bits, g), active, None, bias, ROUTER_SQRT_SOFTPLUS, route_scale)
    z = moe(ids, w, g)
    return hc_post(z, h, post2, comb2, hc, hidden), ids, w


def mhc_decode_layer_batch(hiddens, positions, hc: int, hidden: int, hc_attn, hc_ffn, attn_norm, ffn_norm, mla: dict,
                           gate_bits, bias, active: int, route_scale: float, experts, shared, kv_cache, comps=None,
                           iters: int = 20, eps: float = 1e-6):
    """The batched layer of prefill and MTP verify (E/server/generation.rs:
    2437-2590) over ascending positions:
      compute_layer_deepseek_mhc_phase1_batch (E/compute.rs:4649-4750): per
      position y = rms_norm(hc_pre(hc_attn, hidden), attn_norm); the batched
      attention (compute_deepseek_v4_mla_attention_batch, E/compute.rs:
      4307-4641), which equals mla_attention_decode at each position in
      order: its multi-input projections give each input the single-input
      result (E/compute.rs:6447-6452), it writes every KV row before the
      window loop and each window reads only rows at or before its own
      position; then per position h = hc_post(y, hidden) and
      g = rms_norm(hc_pre(hc_ffn, h), ffn_norm);
      the router per position (E/server/generation.rs:2462-2480; DeepSeek-V4
      weights are used as the router returns them, 3137-3150);
      the union MoE with each position's weights divided by their sum
      (moe_batch, E/server/generation.rs:2487-2569);
      finish_layer_deepseek_mhc_phase2_batch (E/compute.rs:1817-1870):
      z = shared(g) + routed sum; hidden = hc_post(z, h).
    hiddens [npos, hc * hidden]; experts: id -> (w1, w3, w2) as moe_batch
    takes them; shared: a triple or None; comps: None or one array of
    compressed rows (or None) per position.  Returns (new hiddens, ids,
    weights)."""
    hs = _f(hiddens).reshape(len(positions), hc * hidden)
    states, gs, posts, combs = [], [], [], []
    for i, pos in enumerate(positions):
        y, _, post, comb, _ = hc_pre(*hc_attn, hs[i], hc, hidden, iters, eps)
        y = rms_norm(y, attn_norm)
        y = mla_attention_decode(y, token_pos=pos, kv_cache=kv_cache, comp=comps[i] if comps else None, **mla)
        h = hc_post(y, hs[i], post, comb, hc, hidden)
        g, _, post2, comb2, _ = hc_pre(*hc_ffn, h, hc, hidden, iters, eps)
        states.append(h)
        gs.append(rms_norm(g, ffn_norm))
        posts.append(post2)
        combs.append(comb2)
    routes = [route_select(bf16_gemv(gate_bits, g), active, None, bias, ROUTER_SQRT_SOFTPLUS, route_scale)
              for g in gs]
    ids = np.array([r[0] for r in routes], np.int64)
    w = np.array([r[1] for r in routes], np.float32)
    z = moe_batch(experts, ids, w, np.stack(gs), shared)
    out = np.stack([hc_post(z[i], states[i], posts[i], combs[i], hc, hidden) for i in range(len(positions))])
    return out, ids, w

