#!/usr/bin/env python3
"""Decode hot-path benchmark on one MI355X.

Headline workload: one token's routed MoE FFN in FP4 - 6 of 256 experts
(top-6 of sigmoid scores over N(0,1) router logits, renormalised), each
w1/w3 2048x4096 and w2 4096x2048 E2M1 with a UE8M0 scale per 32 columns,
x ~ N(0,1) in bf16, SwiGLU then down then the ordered weighted sum.  A step
is one token; each step routes a fresh token on one of `--layers` resident
layers of 256 experts (round robin), so no step reuses weights that the
previous ones left in the 256 MB Infinity Cache.  Inputs are resident in
HBM before the timed region.  The K timed tokens are captured into one HIP
graph and replayed by a single library call; value = algorithmic bytes per
token / the device time per token between HIP events around that replay
(the same tokens enqueued one Python call each are reported beside it).

The headline runs the MFMA kernels (each matvec within
1e-5 * ||w_row|| * ||x|| of the reference kernel); --exact runs the
bit-exact kernels (the reference's summation order) instead, and each line
reports the other mode's kernels beside its own.

Also reported: per-kernel mean durations (HIP events on the library stream),
the FP8 dense GEMV (4096x4096, fp32 128x128 block scales) over 40 rotating
copies, the decode layer's FP8 projections at batch 1 and 16, the HBM read
floor of each kernel's byte count, the router, the ragged batch, the
43-layer stack at batch 1 and 16, and the reference's AVX2 algorithm (the
CPU oracle) timed on the host cores at 1 thread, the reference's thread
count and every CPU.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
EXPERT_BYTES = 13_369_344             # 3 x (4 MiB packed + 256 KiB UE8M0)
TOKEN_BYTES = 6 * EXPERT_BYTES + 4096 * 2 + 4096 * 4   # + bf16 x + f32 y = 80,240,640
# algorithmic bytes per launch of the two routed-expert kernels: weights and
# scales once, plus the vectors each kernel must read and write
GATEUP_BYTES = 6 * 2 * (4_194_304 + 262_144) + 4096 * 2 + 6 * 2048 * 4     # 53,534,720
DOWN_BYTES = 6 * (4_194_304 + 262_144) + 6 * 2048 * 4 + 4096 * 4           # 26,804,224
# The routed-expert kernels of each numerics mode (trace names).
KERNELS = {False: ("k_moe_gateup_tok<3, 4, true>", "k_moe_down_px<3>"), True: ("k_moe_gateup<16, 4>", "k_moe_down<8, 4>")}
# HBM bytes per gate/up launch: rocprofv3 FETCH_SIZE and WRITE_SIZE KiB per
# dispatch, scaled by what the same counters read for a 268,435,456-byte copy
# (FETCH x2.00, WRITE x1.00); see profiles/ (moe_routed_fp4_token.md, the
# FETCH_SIZE / WRITE_SIZE table of k_moe_gateup_tok<3, 4, true> and
# k_moe_gateup<16, 4>).  None: not measured.
GATEUP_TRAFFIC_BYTES = {False: round((26_259.7 * 2 + 48.0) * 1024), True: round((26_287.3 * 2 + 49.0) * 1024)}
FP8_BYTES = 4096 * 4096 + 32 * 32 * 4 + 4096 * 4 + 4096 * 4


def log(msg: str):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_host() -> dict:
    """CPU model, physical cores and logical CPUs of this host (from
    /proc/cpuinfo), and the CPUs this process may run on."""
    model, cores = "unknown", set()
    phys = core = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name":
                    model = v
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    core = v
                elif not k and phys is not None:
                    cores.add((phys, core))
                    phys = core = None
        if phys is not None:
            cores.add((phys, core))
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return {"model": model, "physical_cores": len(cores) or None, "logical_cpus": os.cpu_count(),
            "usable_cpus": usable}


def _timed(fn, budget_s: float, min_reps: int = 1):
    """(reps, seconds) of repeating fn until budget_s has passed."""
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s and reps >= min_reps:
            return reps, el


def cpu_baseline(lib, seed: int, budget_s: float):
    """The oracle's AVX2 restatement of the reference kernels on this host's
    cores.  Returns (headline, per-config figures): the headline is config
    2's token at the reference's default thread count (available CPUs - 2,
    E/deepseek_v4.rs:206-277); the others are the token and the FP8 GEMV at
    1 thread, that count and every usable CPU, one decode layer at batch 1,
    the 64-token ragged batch (a sample of its token-expert forwards) and
    the 43-layer stack from the layer figure."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    from wohper_amd import workloads as wl

    oracle.build()
    host = cpu_host()
    usable = host["usable_cpus"]
    ref_threads = max(1, usable - 2)
    idx, w, x = wl.moe_token_case(seed)
    experts = [wl.synth_expert_host(lib, seed, 0, int(e)) for e in idx]

    def token():
        outs = np.stack([oracle.fp4_expert_forward(*ex, x) for ex in experts])
        oracle.routed_combine(outs, w)

    oracle.set_threads(ref_threads)
    tokens, el = _timed(token, budget_s)
    gbs = tokens * TOKEN_BYTES / el / 1e9
    headline = {"value": round(gbs, 3), "unit": "GB/s", "cores": ref_threads, "kind": "port",
                "sample": f"{tokens} tokens x 6 routed FP4 experts (4096/2048 shapes), oracle AVX2 restatement "
                          f"of the reference kernel, {ref_threads} threads (usable CPUs - 2, the reference's "
                          f"default), {el:.1f} s; {el / tokens * 1e3:.1f} ms/token"}
    extra = {"host": host, "token": {}, "fp8_gemv_4096": {}}
    short = max(2.0, budget_s / 4)
    for n in sorted({1, ref_threads, usable}):
        oracle.set_threads(n)
        if n != ref_threads:
            k, e = _timed(token, short)
            extra["token"][f"{n}_threads"] = {"us_per_token": round(e / k * 1e6, 1),
                                              "GBps": round(k * TOKEN_BYTES / e / 1e9, 3)}
        else:
            extra["token"][f"{n}_threads"] = {"us_per_token": round(el / tokens * 1e6, 1), "GBps": round(gbs, 3)}
    case = wl.fp8_gemv_case(4096, 4096, seed=0)
    for n in sorted({1, ref_threads, usable}):
        oracle.set_threads(n)
        k, e = _timed(lambda: oracle.fp8_gemv(case.w, 4096, 4096, case.scales, 32, 32, case.x), short / 2, 3)
        extra["fp8_gemv_4096"][f"{n}_threads"] = {"us_per_gemv": round(e / k * 1e6, 1),
                                                  "GBps": round(k * FP8_BYTES / e / 1e9, 3)}
    oracle.set_threads(ref_threads)
    # one decode layer at batch 1: the FP8 projection set (wo_a as 8 row
    # groups with their own inputs) and the shared + 6 routed experts
    rng = np.random.default_rng(seed)
    projs = []
    for i, (name, r, c, groups) in enumerate(wl.DECODE_LAYER_FP8):
        pc = wl.fp8_gemv_case(r, c, seed=100 + i)
        xs = rng.standard_normal((groups, c)).astype(np.float32)
        projs.append((pc, r, c, groups, xs))
    shared = wl.synth_expert_host(lib, seed, 0, wl.N_ROUTED)

    def layer():
        for pc, r, c, groups, xs in projs:
            rows = r // groups
            for g in range(groups):
                oracle.fp8_gemv(pc.w, r, c, pc.scales, r // 128, c // 128, xs[g], g * rows, (g + 1) * rows)
        oracle.fp4_expert_forward(*shared, x)
        token()

    k, e = _timed(layer, short, 2)
    layer_us = e / k * 1e6
    vec = (4096 + 1024 + 1024 + 32768 + 4096 + 512 + 8 * (4096 + 1024) + 8192 + 4096) * 4 + 4096 * 2 + 4096 * 4
    layer_bytes = wl.DECODE_LAYER_FP8_BYTES + 7 * wl.FP4_EXPERT_BYTES + vec
    extra["decode_layer"] = {"threads": ref_threads, "us_per_layer": round(layer_us, 1),
                             "GBps": round(layer_bytes / (layer_us * 1e-6) / 1e9, 3)}
    extra["decode_stack_43"] = {"threads": ref_threads, "us_per_step": round(43 * layer_us, 1),
                                "note": "43 x the measured layer: the 150 GB stack is not built on the host"}
    # ragged batch: the reference runs one expert forward per (token, expert)
    # target, so a sample of the targets scales by their count
    ids, scores, xb = wl.zipf_batch_routes(seed=4, n_tokens=64)
    sample_tokens = 4
    sub = ids[:sample_tokens]
    sub_experts = {int(e): wl.synth_expert_host(lib, seed, 0, int(e)) for e in np.unique(sub)}
    k, e = _timed(lambda: oracle.moe_batch(sub_experts, sub, scores[:sample_tokens], xb[:sample_tokens]), 0.0, 1)
    per_fwd = e / k / sub.size
    extra["ragged_batch_64"] = {"threads": ref_threads, "us_per_step": round(per_fwd * ids.size * 1e6, 1),
                                "sample": f"{sample_tokens} of 64 tokens ({sub.size} of {ids.size} token-expert "
                                          "forwards), scaled by forwards"}
    # batch 16: the FP8 set through the oracle's rows_multi restatement
    # (each row decoded once for the 16 inputs, as the reference's
    # gemv_fp8_e4m3_ue8m0_rows_multi) and the MoE of 16 positions as the
    # reference's batch path runs it (one expert forward per (position,
    # expert) target, shared expert on every position), timed per forward
    # above and scaled by the 16 x 7 targets
    b16 = 16
    xs16 = [rng.standard_normal((b16, groups, c)).astype(np.float32) for _, _, c, groups in wl.DECODE_LAYER_FP8]

    def fp8_set16():
        for (pc, r, c, groups, _), xg in zip(projs, xs16):
            rows = r // groups
            for g in range(groups):
                oracle.fp8_gemv_rows_multi(pc.w, r, c, pc.scales, r // 128, c // 128, xg[:, g], g * rows,
                                           (g + 1) * rows)

    k, e = _timed(fp8_set16, short, 1)
    fp8_16_us = e / k * 1e6
    moe_16_us = per_fwd * b16 * (wl.TOPK + 1) * 1e6
    layer16_us = fp8_16_us + moe_16_us
    extra["decode_stack_43_batch16"] = {
        "threads": ref_threads, "us_per_step": round(43 * layer16_us, 1), "layer_us": round(layer16_us, 1),
        "fp8_set_us": round(fp8_16_us, 1), "moe_us": round(moe_16_us, 1),
        "tokens_per_s": round(b16 / (43 * layer16_us * 1e-6), 2),
        "sample": "one layer's FP8 set at 16 inputs through the oracle's rows_multi restatement, timed; the MoE "
                  "as 16 x (6 routed + shared) expert forwards at the per-forward time of the ragged sample; "
                  "x 43 layers"}
    return headline, extra


def read_floor(ctx, reps: int = 60):
    """The HBM read floor of this device: the fastest plain streaming read
    (wh_probe_read_floor sweeps grid size and loads in flight) of each
    kernel's byte count as one launch, from rotating windows of a 4 GiB
    buffer so that no launch is served by the 256 MB Infinity Cache."""
    buf_bytes = 4 << 30
    buf = ctx.device_alloc(buf_bytes)
    res = {}
    try:
        for name, nbytes in (("fp8_gemv_4096", FP8_BYTES), ("moe_down", DOWN_BYTES), ("moe_gateup", GATEUP_BYTES),
                             ("token_one_launch", TOKEN_BYTES), ("256MiB", 256 << 20)):
            nb = nbytes // 16 * 16
            us, grid, depth, empty = ctx.probe_read_floor(buf, buf_bytes, nb, reps)
            res[name] = {"bytes": nb, "us": round(us, 2), "GBps": round(nb / (us * 1e-6) / 1e9, 1),
                         "frac_of_hbm_peak": round(nb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                         "grid": grid, "loads_in_flight": depth}
        res["empty_launch_us"] = round(empty, 2)
    finally:
        ctx.device_free(buf)
    return res


def fp8_dense(ctx, steps: int, warmup: int):
    """4096x4096 FP8 GEMV (fp32 block scales) over 40 rotating copies (672
    MB), in both numerics modes: the order-free kernel (exact numerics off,
    within 1e-5 * ||w_row|| * ||x|| of the reference kernel) and the exact
    kernel (the reference's summation order, bit-identical)."""
    import wohper_amd
    from wohper_amd import workloads as wl

    case = wl.fp8_gemv_case(4096, 4096, seed=0)
    copies = 40
    handles = [ctx.store_fp8(case.w, 4096, 4096, case.scales, 32, 32, wohper_amd.SCALE_F32) for _ in range(copies)]
    xd = ctx.device_alloc(4096 * 4)
    yd = ctx.device_alloc(4096 * 4)
    ctx.to_device(xd, case.x)
    # one library call launches every timed GEMV, so the host's per-call
    # Python cost does not pace the device
    timed = ctx.gemv_descs([(handles[i % copies], 0, 4096, xd, yd) for i in range(steps)])
    res = {"workload": "fp8 e4m3 GEMV 4096x4096, fp32 128x128 block scales, bf16 x, batch 1",
           "bytes": FP8_BYTES,
           "note": "back-to-back launches from one wh_fp8_gemv_batch_async call over 40 rotating weight copies; "
                   "wall clock and HIP events on the library stream"}
    for exact, key in ((False, "order_free"), (True, "exact")):
        ctx.set_exact_numerics(exact)
        for i in range(warmup):
            ctx.fp8_gemv_async(handles[i % copies], 0, 4096, xd, yd)
        ctx.synchronize()
        t0 = time.perf_counter()
        ctx.timer_start()
        ctx.fp8_gemv_batch_async(timed)
        dev_us = ctx.timer_stop() / steps
        ctx.synchronize()
        us = (time.perf_counter() - t0) / steps * 1e6
        gbs = FP8_BYTES / (us * 1e-6) / 1e9
        res[key] = {"us_per_gemv": round(us, 3), "GBps": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                    "device_us_per_gemv": round(dev_us, 3), "device_GBps": round(FP8_BYTES / (dev_us * 1e-6) / 1e9, 1),
                    "device_frac_of_hbm_peak": round(FP8_BYTES / (dev_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    ctx.device_free(xd)
    ctx.device_free(yd)
    for h in handles:
        ctx.release(h)
    return res


def fp8_decode_layer(ctx, steps: int):
    """Each FP8 projection of one decode layer on its own (wq_a, wq_b, wkv,
    wo_a as 8 row groups with their own inputs in one launch, wo_b; f32
    128x128 block scales), back to back over 8 rotating weight copies, in
    both numerics modes."""
    out = {}
    for exact, key in ((False, "order_free"), (True, "exact")):
        ctx.set_exact_numerics(exact)
        out[key] = _fp8_decode_layer(ctx, steps)
        out[key]["total_device_us_separate"] = round(sum(v["device_us"] for v in out[key].values()), 2)
        out[key]["wq_a+wkv"] = _fp8_pair(ctx, steps)
        # the layer as the decode step runs it: wq_a and wkv on their shared
        # input in one launch
        out[key]["total_device_us"] = round(sum(out[key][k]["device_us"] for k in ("wq_a+wkv", "wq_b", "wo_a",
                                                                                    "wo_b")), 2)
    return out


def _fp8_pair(ctx, steps: int) -> dict:
    """wq_a (1024x4096) and wkv (512x4096) on one input, as the decode layer
    runs them: one wh_fp8_gemv_batch_async pair per step (merged into one
    launch), back to back over 8 rotating weight copies."""
    copies = 8
    rng = np.random.default_rng(8)
    ha = [ctx.store_fp8_synthetic(1024, 4096, 3, 5000 + k, wl_scales(31 + k, 1024, 4096)) for k in range(copies)]
    hk = [ctx.store_fp8_synthetic(512, 4096, 3, 6000 + k, wl_scales(41 + k, 512, 4096)) for k in range(copies)]
    xd, yd = ctx.device_alloc(4096 * 4), ctx.device_alloc(1536 * 4)
    ctx.to_device(xd, rng.standard_normal(4096).astype(np.float32))
    per_copy = [[(ha[k], 0, 1024, xd, yd), (hk[k], 0, 512, xd, yd + 1024 * 4)] for k in range(copies)]
    descs = [ctx.gemv_descs(d) for d in per_copy]
    timed = ctx.gemv_descs([t for k in range(steps) for t in per_copy[k % copies]])
    for k in range(10):
        ctx.fp8_gemv_batch_async(descs[k % copies])
    ctx.synchronize()
    ctx.timer_start()
    ctx.fp8_gemv_batch_async(timed)
    us = ctx.timer_stop() / steps
    nbytes = 1536 * 4096 + 12 * 32 * 4 + 4096 * 4 + 1536 * 4
    for h in ha + hk:
        ctx.release(h)
    ctx.device_free(xd)
    ctx.device_free(yd)
    return {"shape": "1024x4096 + 512x4096, one input", "bytes": nbytes, "device_us": round(us, 2),
            "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}


def wl_scales(seed: int, r: int, c: int):
    from wohper_amd import workloads as wl

    return wl.fp8_block_scales(seed, r, c)


def _fp8_decode_layer(ctx, steps: int):
    from wohper_amd import workloads as wl

    res = {}
    copies = 8
    rng = np.random.default_rng(7)
    for i, (name, r, c, groups) in enumerate(wl.DECODE_LAYER_FP8):
        hs = [ctx.store_fp8_synthetic(r, c, 3, wl.fp8_stream(1000 + k, i), wl.fp8_block_scales(11 + k, r, c))
              for k in range(copies)]
        xd, yd = ctx.device_alloc(groups * c * 4), ctx.device_alloc(r * 4)
        ctx.to_device(xd, rng.standard_normal(groups * c).astype(np.float32))
        rows = r // groups
        per_copy = [[(h, rows * g, rows * (g + 1), xd + g * c * 4, yd + rows * g * 4) for g in range(groups)]
                    for h in hs]
        descs = [ctx.gemv_descs(d) for d in per_copy]
        # all timed projections in one call (each copy's row groups still
        # merge into one launch)
        timed = ctx.gemv_descs([t for k in range(steps) for t in per_copy[k % copies]])
        for k in range(10):
            ctx.fp8_gemv_batch_async(descs[k % copies])
        ctx.synchronize()
        ctx.timer_start()
        ctx.fp8_gemv_batch_async(timed)
        us = ctx.timer_stop() / steps
        nbytes = r * c + (r // 128) * (c // 128) * 4 + groups * c * 4 + r * 4
        res[name] = {"shape": f"{r}x{c}", "groups": groups, "bytes": nbytes, "device_us": round(us, 2),
                     "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}
        for h in hs:
            ctx.release(h)
        ctx.device_free(xd)
        ctx.device_free(yd)
    return res


def decode_layer(ctx, n_layers: int, steps: int, graph: bool = True) -> dict:
    """The whole device decode layer (wh_deepseek_mhc_layer_async: hc_pre ->
    norm -> MLA -> hc_post -> hc_pre -> norm -> router -> shared + routed
    experts -> hc_post) at the model's shapes (hc 4, hidden 4096, 64 heads of
    448 + 64, q_lora 1024, 8 output groups of 1024; bf16 router of 256
    experts, top-6, route_scale 1.5, + the shared expert), on the n_layers
    resident layers of the headline (their 256 routed experts), each with its
    own MLA tensors, mHC parameters, norms and router.  A step runs every
    layer once at position 127 (a full 128-row window); timed as one HIP
    graph per step replayed back to back, and as a host loop, in both
    numerics modes.  Nothing is read back between the layers: the router's
    output feeds the experts on the device."""
    import wohper_amd
    from wohper_amd import model_format as mf
    from wohper_amd import workloads as wl

    hc, heads, nope, rope, q_lora, groups, o_lora = 4, 64, 448, 64, 1024, 8, 1024
    head_dim, pos, cap = nope + rope, 127, 128
    rng = np.random.default_rng(71)
    keep, handles = [], []

    def put(a):
        a = np.ascontiguousarray(a)
        p = ctx.device_alloc(max(a.nbytes, 4))
        ctx.to_device(p, a)
        keep.append(p)
        return p

    def bf16w(n):
        return ((1.0 + 0.1 * rng.standard_normal(n).astype(np.float32)).view(np.uint32) >> 16).astype(np.uint16)

    shapes = {"wq_a": (q_lora, wl.HIDDEN), "wq_b": (heads * head_dim, q_lora), "wkv": (head_dim, wl.HIDDEN),
              "wo_a": (groups * o_lora, heads * head_dim // groups), "wo_b": (wl.HIDDEN, groups * o_lora)}
    layers, kvs, hs = [], [], []
    mix = (2 + hc) * hc
    for L in range(n_layers):
        ctx.store_expert_synthetic(L, wl.N_ROUTED, wl.HIDDEN, wl.INTER, 2)  # the layer's shared expert
        t = {n: ctx.store_fp8_synthetic(r, c, 5, 100 * L + i, wl.fp8_block_scales(7 + 31 * L + i, r, c))
             for i, (n, (r, c)) in enumerate(shapes.items())}
        handles += list(t.values())
        mla = wohper_amd.WhMlaLayer(L, heads, nope, rope, groups, o_lora, t["wq_a"], t["wq_b"], t["wkv"], t["wo_a"],
                                    t["wo_b"], put(bf16w(q_lora)), put(bf16w(head_dim)),
                                    put(rng.standard_normal(heads).astype(np.float32)))
        gate = ((rng.standard_normal((wl.N_ROUTED, wl.HIDDEN)).astype(np.float32) * 0.02).view(np.uint32) >> 16)
        bias = (rng.standard_normal(wl.N_ROUTED) * 0.05).astype(np.float32)
        blk = mf.build_synthetic_quant_block([
            mf.SyntheticTensor(f"layers.{L}.ffn.gate.weight", 9, (wl.N_ROUTED, wl.HIDDEN),
                               gate.astype(np.uint16).tobytes(), 11, 2404),
            mf.SyntheticTensor(f"layers.{L}.ffn.gate.bias", 9, (wl.N_ROUTED,), bias.tobytes(), 12, 2405)])
        ctx.store_router(L, blk, wl.HIDDEN)
        d = wohper_amd.WhMhcLayer()
        d.hc, d.hidden, d.sinkhorn_iters, d.hc_eps = hc, wl.HIDDEN, 20, 1e-6
        fns = [(rng.standard_normal((mix, hc * wl.HIDDEN)) / np.sqrt(hc * wl.HIDDEN)).astype(np.float32)
               for _ in range(2)]
        d.hc_attn_fn, d.hc_ffn_fn = put(fns[0]), put(fns[1])
        d.hc_attn_scale, d.hc_ffn_scale = (put((0.5 + rng.random(3)).astype(np.float32)) for _ in range(2))
        d.hc_attn_base, d.hc_ffn_base = (put((rng.standard_normal(mix) * 0.5).astype(np.float32)) for _ in range(2))
        d.attn_norm_bf16, d.ffn_norm_bf16 = put(bf16w(wl.HIDDEN)), put(bf16w(wl.HIDDEN))
        d.attn = mla
        d.layer_id, d.active, d.available_dev, d.n_available = L, wl.TOPK, None, 0
        d.route = wohper_amd.Context.route_options(wohper_amd.ROUTER_SQRT_SOFTPLUS, 1.5)
        d.shared_layer, d.shared_expert = L, wl.N_ROUTED
        layers.append(d)
        kvs.append(put((rng.standard_normal((cap, head_dim)) * 0.3).astype(np.float32)))
        hs.append(put((rng.standard_normal(hc * wl.HIDDEN) * 0.5).astype(np.float32)))

    def step():
        for L in range(n_layers):
            ctx.deepseek_mhc_layer_async(layers[L], pos, hs[L], kvs[L], head_dim, cap)

    mla_bytes = sum(r * c + (r // 128) * (c // 128) * 4 for r, c in shapes.values())
    layer_bytes = (mla_bytes + wl.N_ROUTED * wl.HIDDEN * 2 + wl.N_ROUTED * 4 + (wl.TOPK + 1) * wl.FP4_EXPERT_BYTES +
                   2 * mix * hc * wl.HIDDEN * 4 + cap * head_dim * 4)
    res = {"workload": f"{n_layers} decode layers at batch 1, position {pos}: hc_pre, norm, MLA attention (FP8 "
                       "projections, 128-row window), hc_post, hc_pre, norm, bf16 router 256x4096 top-6, shared + "
                       "6 routed FP4 experts read from the router's device output, hc_post",
           "bytes_per_layer": layer_bytes}
    for exact in (False, True):
        ctx.set_exact_numerics(exact)
        step()
        ctx.synchronize()
        ctx.timer_start()
        for _ in range(steps):
            step()
        loop_us = ctx.timer_stop() / steps / n_layers
        ctx.synchronize()
        r = {"host_loop_layer_us": round(loop_us, 2)}
        if graph:
            g = ctx.graph_capture(step)
            ctx.graph_launch(g)
            ctx.synchronize()
            ctx.timer_start()
            for _ in range(steps):
                ctx.graph_launch(g)
            us = ctx.timer_stop() / steps / n_layers
            ctx.synchronize()
            ctx.graph_release(g)
            r["layer_us"] = round(us, 2)
        else:
            us = loop_us
        r["GBps"] = round(layer_bytes / (us * 1e-6) / 1e9, 1)
        r["frac_of_hbm_peak"] = round(layer_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
        res["exact" if exact else "order_free"] = r
    # the batched layer of prefill and MTP verify: 16 positions (112..127,
    # the last with a full window) per layer through
    # wh_deepseek_mhc_layer_batch_async, the experts of the batch as one
    # union MoE; host loop of library calls
    bpos = list(range(cap - 16, cap))
    hbs = [put((rng.standard_normal((len(bpos), hc * wl.HIDDEN)) * 0.5).astype(np.float32)) for _ in range(n_layers)]

    def bstep():
        for L in range(n_layers):
            ctx.deepseek_mhc_layer_batch_async(layers[L], bpos, hbs[L], kvs[L], head_dim, cap)

    bres = {"workload": f"{len(bpos)} positions ({bpos[0]}..{bpos[-1]}) per layer, the same layers"}
    for exact in (False, True):
        ctx.set_exact_numerics(exact)
        bstep()
        ctx.synchronize()
        ctx.timer_start()
        for _ in range(max(2, steps // 4)):
            bstep()
        us = ctx.timer_stop() / max(2, steps // 4) / n_layers
        ctx.synchronize()
        bres["exact" if exact else "order_free"] = {"layer_us": round(us, 1),
                                                    "us_per_position": round(us / len(bpos), 2)}
    res["batch16"] = bres
    ctx.set_exact_numerics(False)
    for p in keep:
        ctx.device_free(p)
    for t in handles:
        ctx.release(t)
    return res


def router(ctx, steps: int):
    """The DeepSeek-V4 router of a layer (bf16 gate 256x4096, f32 bias,
    sqrt-softplus, top-6, route_scale 1.5) on device pointers, over 8
    rotating layers."""
    from wohper_amd import model_format as mf

    rows, cols, layers = 256, 4096, 8
    rng = np.random.default_rng(31)
    for k in range(layers):
        gate = ((rng.standard_normal((rows, cols)).astype(np.float32) * 0.02).view(np.uint32) >> 16).astype(np.uint16)
        bias = (rng.standard_normal(rows) * 0.05).astype(np.float32)
        blk = mf.build_synthetic_quant_block([
            mf.SyntheticTensor(f"layers.{k}.ffn.gate.weight", 9, (rows, cols), gate.tobytes(), 11, 2404),
            mf.SyntheticTensor(f"layers.{k}.ffn.gate.bias", 9, (rows,), bias.tobytes(), 12, 2405)])
        ctx.store_router(1000 + k, blk, cols)
    xd, out = ctx.device_alloc(cols * 4), ctx.device_alloc(256)
    ctx.to_device(xd, rng.standard_normal(cols).astype(np.float32))
    call = lambda i: ctx.route_experts_async(1000 + i % layers, xd, cols, 6, 0, 0, out, out + 64, out + 128,
                                             route_scale=1.5)
    for i in range(20):
        call(i)
    ctx.synchronize()
    ctx.timer_start()
    for i in range(steps):
        call(i)
    us = ctx.timer_stop() / steps
    ctx.synchronize()
    ctx.device_free(xd)
    ctx.device_free(out)
    nbytes = rows * cols * 2 + rows * 4 + cols * 4
    return {"workload": "router: bf16 gate 256x4096 + f32 bias, sqrt-softplus, top-6 (gate GEMV + selection launch)",
            "bytes": nbytes, "us_per_route": round(us, 2), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
            "note": "HIP events around back-to-back asynchronous calls; includes the host's per-call launch cost"}


def expert_pack_load(ctx, n_experts: int = 24):
    """Loads a consolidated experts pack (ZCBLK01 blocks at 2 MiB-aligned
    offsets) into the store with wh_store_expert_pack; the file was just
    written, so it is read from the page cache."""
    import tempfile

    from wohper_amd import model_format as mf
    from wohper_amd import workloads as wl

    with tempfile.TemporaryDirectory(dir="/tmp") as d:
        pack = Path(d) / "m.experts_pack.bin"
        entries, off, payload = [], 0, 0
        with pack.open("wb") as f:
            for e in range(n_experts):
                mats = wl.synth_expert_host(ctx.lib, 41, 2000, e)
                ts = []
                for name, (p, s, r, c, sc), role in zip(("w1", "w3", "w2"), mats, (6, 7, 8)):
                    ts.append(mf.SyntheticTensor(f"layers.2000.ffn.experts.{e}.{name}.weight", role, (r, c // 2),
                                                 p.tobytes(), 12, 2402))
                    ts.append(mf.SyntheticTensor(f"layers.2000.ffn.experts.{e}.{name}.scale", role, (r, sc),
                                                 s.tobytes(), 1, 2403))
                blk = mf.build_synthetic_quant_block(ts)
                disk = (len(blk) + mf.ALIGN_2MB - 1) // mf.ALIGN_2MB * mf.ALIGN_2MB
                f.seek(off)
                f.write(blk)
                entries.append({"layer_id": 2000, "expert_id": e, "offset": off, "disk_bytes": disk,
                                "payload_bytes": len(blk)})
                off += disk
                payload += len(blk)
            f.truncate(off)
        (Path(d) / "m.experts_pack.index.json").write_text(json.dumps(
            {"format": "wohper-experts-pack", "pack_file": pack.name, "entries": entries}))
        info = mf.load_optional_expert_pack(Path(d) / "m.zcinf")
        t0 = time.perf_counter()
        stored = ctx.store_expert_pack(info)
        el = time.perf_counter() - t0
    return {"workload": f"experts pack load: {stored} FP4 experts (ZCBLK01 blocks, 13.4 MB each) from the page cache",
            "payload_bytes": payload, "seconds": round(el, 4), "GBps": round(payload / el / 1e9, 2)}


def ragged_batch(ctx, n_layers: int, steps: int, warmup: int, exact: bool = False, mfma_min: int = 1):
    """Ragged batched MoE: 64 bf16 tokens, each top-6 of 256 FP4 experts under
    Zipf(1.1) popularity over a seeded permutation (seed 4), one launch
    sequence per step (device packing, act-quant, grouped gate/up, grouped
    down, expert-major weighted sum), rotating over the resident layers.
    exact: every expert on the bit-exact items; else experts with at least
    mfma_min tokens on MFMA items."""
    from wohper_amd import workloads as wl

    ctx.set_exact_numerics(exact)
    ctx.set_moe_mfma_min(mfma_min)

    ids, sc, x = wl.zipf_batch_routes(seed=4, n_tokens=64)
    npos, topk = ids.shape
    used, counts = np.unique(ids, return_counts=True)
    n_used = int(used.size)
    nbytes = n_used * EXPERT_BYTES + npos * wl.HIDDEN * (2 + 4)
    xb = wl.bf16_bits(x)
    x_dev = ctx.device_alloc(xb.nbytes)
    ids_dev = ctx.device_alloc(ids.nbytes)
    sc_dev = ctx.device_alloc(sc.nbytes)
    out_dev = ctx.device_alloc(npos * wl.HIDDEN * 4)
    ctx.to_device(x_dev, xb)
    ctx.to_device(ids_dev, ids)
    ctx.to_device(sc_dev, sc)
    for i in range(warmup):
        ctx.moe_batch_async(i % n_layers, ids_dev, sc_dev, npos, topk, x_dev, True, out_dev)
    ctx.synchronize()
    t0 = time.perf_counter()
    ctx.timer_start()
    for i in range(steps):
        ctx.moe_batch_async(i % n_layers, ids_dev, sc_dev, npos, topk, x_dev, True, out_dev)
    dev_us = ctx.timer_stop() / steps
    ctx.synchronize()
    us = (time.perf_counter() - t0) / steps * 1e6
    n_mfma = int(ctx.debug_moe_batch_read(4, 8, np.uint32)[4])
    for p in (x_dev, ids_dev, sc_dev, out_dev):
        ctx.device_free(p)
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"workload": "ragged batched MoE: 64 bf16 tokens x top-6 of 256 FP4 experts, Zipf(1.1) popularity",
            "numerics": "exact" if exact else f"MFMA for experts with >= {mfma_min} tokens", "experts_on_mfma": n_mfma,
            "experts_used": n_used, "largest_group": int(counts.max()),
            "groups_ge_16": int((counts >= 16).sum()), "tokens_in_groups_ge_16": int(counts[counts >= 16].sum()),
            "bytes_per_step": nbytes, "us_per_step": round(us, 2), "GBps": round(gbs, 1),
            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "device_us_per_step": round(dev_us, 2),
            "flops_per_step": npos * topk * 2 * 3 * wl.INTER * wl.HIDDEN,
            "note": "wall clock and HIP events on the library stream; layers rotate so no step reuses cached weights"}


def fp8_decode_layer_batch(ctx, steps: int, batch: int = 16):
    """The decode layer's FP8 projections over `batch` inputs, each on its
    own, back to back over 8 rotating weight copies: exact numerics (every
    input bit-identical to the single-input kernel) against the bf16 MFMA
    path (each weight byte read once for all inputs; each output within
    1e-5 * ||w_row|| * ||x|| of the reference kernel).  wo_a's 8 row groups
    read their own inputs in one call."""
    from wohper_amd import workloads as wl

    res = {}
    copies = 8
    rng = np.random.default_rng(9)
    for i, (name, r, c, groups) in enumerate(wl.DECODE_LAYER_FP8):
        hs = [ctx.store_fp8_synthetic(r, c, 3, wl.fp8_stream(2000 + k, i), wl.fp8_block_scales(21 + k, r, c))
              for k in range(copies)]
        xd, yd = ctx.device_alloc(batch * groups * c * 4), ctx.device_alloc(batch * r * 4)
        ctx.to_device(xd, rng.standard_normal(batch * groups * c).astype(np.float32))
        rows = r // groups

        def call(h):
            if groups > 1:
                ctx.fp8_gemv_multi_groups_async(h, 0, r, rows, xd, c, batch, groups * c, yd, r)
            else:
                ctx.fp8_gemv_multi_async(h, 0, r, xd, batch, c, yd, r)

        nbytes = r * c + (r // 128) * (c // 128) * 4 + batch * (groups * c + r) * 4
        entry = {"shape": f"{r}x{c}", "groups": groups, "inputs": batch, "bytes": nbytes}
        for exact in (True, False):
            ctx.set_exact_numerics(exact)
            n = steps if not exact else max(8, steps // 8)
            for k in range(copies):
                call(hs[k])
            ctx.synchronize()
            ctx.timer_start()
            for k in range(n):
                call(hs[k % copies])
            us = ctx.timer_stop() / n
            entry["exact_us" if exact else "mfma_us"] = round(us, 2)
            entry["exact_GBps" if exact else "mfma_GBps"] = round(nbytes / (us * 1e-6) / 1e9, 1)
        res[name] = entry
        for h in hs:
            ctx.release(h)
        ctx.device_free(xd)
        ctx.device_free(yd)
    return res


def decode_stack(n_layers: int, steps: int, warmup: int, seed: int, batch_steps: int = 0, exact: bool = False,
                 graph: bool = True):
    """Full-depth synthetic stack at batch 1: per layer the FP8 projections
    of one decode layer (wq_a, wq_b, wkv, wo_a in 8 row groups, wo_b; f32
    128x128 block scales) and the MoE FFN (1 shared + top-6 of 256 routed
    FP4 experts), all resident.  A step runs every layer once; the per-layer
    average is the single decode layer's figure."""
    import wohper_amd
    from wohper_amd import workloads as wl

    ctx = wohper_amd.Context(0)
    ctx.set_exact_numerics(exact)
    t0 = time.perf_counter()
    layers = []
    for L in range(n_layers):
        hs = {}
        for i, (name, r, c, _) in enumerate(wl.DECODE_LAYER_FP8):
            hs[name] = ctx.store_fp8_synthetic(r, c, seed, wl.fp8_stream(L, i),
                                               wl.fp8_block_scales(seed * 100003 + L * 7 + i, r, c))
        for e in range(wl.N_ROUTED + 1):  # expert id N_ROUTED is the layer's shared expert
            ctx.store_expert_synthetic(L, e, wl.HIDDEN, wl.INTER, seed)
        layers.append(hs)
    dev_bytes, _, n_exp = ctx.usage()
    log(f"stack: {n_layers} layers, {n_exp} experts, {dev_bytes / 1e9:.1f} GB resident in {time.perf_counter() - t0:.1f} s")
    rng = np.random.default_rng(seed)
    vec = lambda n: rng.standard_normal(n).astype(np.float32)
    bufs = {"x": vec(4096), "qlat": vec(1024), "oa": vec(8 * 4096), "ob": vec(8192)}
    dev = {}
    for k, v in bufs.items():
        dev[k] = ctx.device_alloc(v.nbytes)
        ctx.to_device(dev[k], v)
    y = ctx.device_alloc((1024 + 32768 + 512 + 8192 + 4096) * 4)
    y_off = {"wq_a": 0, "wq_b": 1024, "wkv": 1024 + 32768, "wo_a": 1024 + 32768 + 512, "wo_b": 1024 + 32768 + 512 + 8192}
    moe_x = ctx.device_alloc(4096 * 2)
    ctx.to_device(moe_x, wl.bf16_bits(vec(4096)))
    moe_out = ctx.device_alloc(4096 * 4)
    descs = []
    for hs in layers:
        # wq_a and wkv read the same input: one launch
        d = [(hs["wq_a"], 0, 1024, dev["x"], y), (hs["wkv"], 0, 512, dev["x"], y + y_off["wkv"] * 4),
             (hs["wq_b"], 0, 32768, dev["qlat"], y + y_off["wq_b"] * 4)]
        d += [(hs["wo_a"], 1024 * g, 1024 * (g + 1), dev["oa"] + g * 4096 * 4, y + (y_off["wo_a"] + 1024 * g) * 4)
              for g in range(8)]
        d += [(hs["wo_b"], 0, 4096, dev["ob"], y + y_off["wo_b"] * 4)]
        descs.append(ctx.gemv_descs(d))
    total = warmup + steps
    route_arrays = []
    for s_ in range(total):
        per = []
        for L in range(n_layers):
            idx, w = wl.route_topk_sigmoid(rng.standard_normal(wl.N_ROUTED).astype(np.float32))
            per.append(ctx.route_array([(L, int(e), float(wt)) for e, wt in zip(idx, w)]))
        route_arrays.append(per)

    def step(s_):
        for L in range(n_layers):
            ctx.fp8_gemv_batch_async(descs[L])
            ctx.routed_and_shared_experts_async(route_arrays[s_][L], (L, wl.N_ROUTED), moe_x, True, 1, moe_out,
                                                n_routes=wl.TOPK)

    for s_ in range(warmup):
        step(s_)
    ctx.synchronize()
    # host loop: two library calls per layer
    t1 = time.perf_counter()
    ctx.timer_start()
    for s_ in range(warmup, total):
        step(s_)
    loop_us = ctx.timer_stop()
    ctx.synchronize()
    loop_wall = time.perf_counter() - t1
    # the same steps captured as one HIP graph each (every step keeps its own
    # routes), replayed once untimed, then timed back to back
    graphs = [ctx.graph_capture(lambda s_=s_: step(s_)) for s_ in range(warmup, total)] if graph else []
    for g in graphs:
        ctx.graph_launch(g)
    ctx.synchronize()
    t1 = time.perf_counter()
    ctx.timer_start()
    for g in graphs:
        ctx.graph_launch(g)
    dev_us = ctx.timer_stop()
    ctx.synchronize()
    wall = time.perf_counter() - t1
    for g in graphs:
        ctx.graph_release(g)
    if not graph:
        dev_us, wall = loop_us, loop_wall
    vec_bytes = (4096 + 1024 + 1024 + 32768 + 4096 + 512 + 8 * (4096 + 1024) + 8192 + 4096) * 4 + 4096 * 2 + 4096 * 4
    layer_bytes = wl.DECODE_LAYER_FP8_BYTES + 7 * wl.FP4_EXPERT_BYTES + vec_bytes
    step_us = dev_us / steps
    res = {"workload": f"{n_layers} decode layers at batch 1: FP8 projections (wq_a 1024x4096, wq_b 32768x1024, "
                       "wkv 512x4096, wo_a 8192x4096 in 8 groups, wo_b 4096x8192; f32 block scales) + MoE "
                       "(1 shared + top-6 of 256 routed FP4 experts) per layer",
           "resident_GB": round(dev_bytes / 1e9, 2), "bytes_per_layer": layer_bytes,
           "timed_region": f"each step one HIP graph of its {n_layers} layers' launches (2 library calls per layer "
                           "captured), graphs replayed back to back between HIP events" if graph else
                           "host loop, 2 library calls per layer, between HIP events",
           "step_us": round(step_us, 1), "wall_step_us": round(wall / steps * 1e6, 1),
           "layer_us": round(step_us / n_layers, 2),
           "host_loop": {"step_us": round(loop_us / steps, 1), "wall_step_us": round(loop_wall / steps * 1e6, 1)},
           "GBps": round(layer_bytes * n_layers / (step_us * 1e-6) / 1e9, 1)}
    res["frac_of_hbm_peak"] = round(res["GBps"] / HBM_PEAK_GBS, 4)
    if graph:
        res["with_gpu_router"] = stack_with_router(ctx, descs, moe_x, moe_out, n_layers, steps, seed)
    for k in list(dev.values()) + [y, moe_x, moe_out]:
        ctx.device_free(k)
    if batch_steps > 0:
        res["batch16"] = decode_stack_batch16(ctx, layers, n_layers, batch_steps, seed)
        res["batch16"]["numerics"] = "exact" if exact else "mfma"
        ctx.set_exact_numerics(not exact)
        other = decode_stack_batch16(ctx, layers, n_layers, batch_steps, seed)
        ctx.set_exact_numerics(exact)
        res["batch16_other_numerics"] = {"numerics": "mfma" if exact else "exact",
                                         **{k: other[k] for k in ("step_us", "layer_us", "GBps", "frac_of_hbm_peak",
                                                                  "tokens_per_s")}}
    ctx.close()
    return res


def stack_with_router(ctx, descs, moe_x, moe_out, n_layers: int, steps: int, seed: int) -> dict:
    """The batch-1 stack with each layer's experts chosen on the device: per
    layer the FP8 projections, the layer's bf16 router (256x4096 + bias,
    sqrt-softplus, top-6, route_scale 1.5) on the MoE input, and the shared +
    6 routed experts read from the router's device output (no host round
    trip); each step one HIP graph, replayed back to back."""
    from wohper_amd import model_format as mf
    from wohper_amd import workloads as wl

    rng = np.random.default_rng(seed + 17)
    for L in range(n_layers):
        gate = ((rng.standard_normal((wl.N_ROUTED, wl.HIDDEN)).astype(np.float32) * 0.02).view(np.uint32) >> 16)
        bias = (rng.standard_normal(wl.N_ROUTED) * 0.05).astype(np.float32)
        blk = mf.build_synthetic_quant_block([
            mf.SyntheticTensor(f"layers.{L}.ffn.gate.weight", 9, (wl.N_ROUTED, wl.HIDDEN),
                               gate.astype(np.uint16).tobytes(), 11, 2404),
            mf.SyntheticTensor(f"layers.{L}.ffn.gate.bias", 9, (wl.N_ROUTED,), bias.tobytes(), 12, 2405)])
        ctx.store_router(L, blk, wl.HIDDEN)
    xb = np.empty(wl.HIDDEN, np.uint16)
    ctx.from_device(xb, moe_x)
    rx = ctx.device_alloc(wl.HIDDEN * 4)  # the router reads the same values as f32
    ctx.to_device(rx, (xb.astype(np.uint32) << 16).view(np.float32))
    rout = ctx.device_alloc(256)  # ids (64 B), weights (64 B), count

    def step():
        for L in range(n_layers):
            ctx.fp8_gemv_batch_async(descs[L])
            ctx.route_experts_async(L, rx, wl.HIDDEN, wl.TOPK, 0, 0, rout, rout + 64, rout + 128, route_scale=1.5)
            ctx.routed_and_shared_experts_dev_async(L, rout, rout + 64, rout + 128, wl.TOPK, (L, wl.N_ROUTED), moe_x,
                                                    True, moe_out)

    step()
    ctx.synchronize()
    g = ctx.graph_capture(step)
    ctx.graph_launch(g)
    ctx.synchronize()
    ctx.timer_start()
    for _ in range(steps):
        ctx.graph_launch(g)
    us = ctx.timer_stop() / steps
    ctx.synchronize()
    ctx.graph_release(g)
    ctx.device_free(rx)
    ctx.device_free(rout)
    return {"per_layer": "FP8 projections, bf16 router 256x4096 top-6 on the device, shared + 6 routed experts "
                         "from the router's device output",
            "step_us": round(us, 1), "layer_us": round(us / n_layers, 2)}


def decode_stack_batch16(ctx, layers, n_layers: int, steps: int, seed: int, batch: int = 16):
    """The same resident stack at batch 16: per layer every FP8 projection
    over 16 inputs (each bit-identical to its single-input GEMV) and the MoE
    FFN of 16 positions through the expert-major batch path (shared expert on
    all 16, routed experts grouped on the device; groups of 16 or more tokens
    on MFMA).  Per-layer routing: top-6 of 256 sigmoid scores of N(0,1)
    logits per position."""
    from wohper_amd import workloads as wl

    rng = np.random.default_rng(seed + 16)
    sizes = {"x": 4096, "qlat": 1024, "oa": 8 * 4096, "ob": 8192}
    dev = {}
    for k, n in sizes.items():
        dev[k] = ctx.device_alloc(batch * n * 4)
        ctx.to_device(dev[k], rng.standard_normal((batch, n)).astype(np.float32))
    outs = {"wq_a": 1024, "wq_b": 32768, "wkv": 512, "wo_a": 8192, "wo_b": 4096}
    ydev = {k: ctx.device_alloc(batch * n * 4) for k, n in outs.items()}
    moe_x = ctx.device_alloc(batch * 4096 * 2)
    ctx.to_device(moe_x, wl.bf16_bits(rng.standard_normal((batch, 4096)).astype(np.float32)))
    moe_out = ctx.device_alloc(batch * 4096 * 4)
    total = steps + 1
    ids_dev, sc_dev, used = [], [], []
    for s_ in range(total):
        per_i, per_s = [], []
        for L in range(n_layers):
            ids = np.empty((batch, wl.TOPK), np.uint32)
            sc = np.empty((batch, wl.TOPK), np.float32)
            for p in range(batch):
                logits = rng.standard_normal(wl.N_ROUTED).astype(np.float32)
                s_all = (1.0 / (1.0 + np.exp(-logits.astype(np.float64)))).astype(np.float32)
                idx = np.argsort(-s_all, kind="stable")[:wl.TOPK]
                ids[p], sc[p] = idx, s_all[idx]
            if s_ > 0:
                used.append(len(np.unique(ids)))
            di, ds = ctx.device_alloc(ids.nbytes), ctx.device_alloc(sc.nbytes)
            ctx.to_device(di, ids)
            ctx.to_device(ds, sc)
            per_i.append(di)
            per_s.append(ds)
        ids_dev.append(per_i)
        sc_dev.append(per_s)

    def step(s_):
        for L in range(n_layers):
            hs = layers[L]
            ctx.fp8_gemv_multi_pair_async(hs["wq_a"], 0, 1024, ydev["wq_a"], 1024, hs["wkv"], 0, 512, ydev["wkv"], 512,
                                          dev["x"], batch, 4096)
            ctx.fp8_gemv_multi_async(hs["wq_b"], 0, 32768, dev["qlat"], batch, 1024, ydev["wq_b"], 32768)
            ctx.fp8_gemv_multi_groups_async(hs["wo_a"], 0, 8192, 1024, dev["oa"], 4096, batch, 8 * 4096,
                                            ydev["wo_a"], 8192)
            ctx.fp8_gemv_multi_async(hs["wo_b"], 0, 4096, dev["ob"], batch, 8192, ydev["wo_b"], 4096)
            ctx.moe_batch_async(L, ids_dev[s_][L], sc_dev[s_][L], batch, wl.TOPK, moe_x, True, moe_out,
                                shared_key=(L, wl.N_ROUTED))

    step(0)
    ctx.synchronize()
    t1 = time.perf_counter()
    ctx.timer_start()
    for s_ in range(1, total):
        step(s_)
    dev_us = ctx.timer_stop()
    ctx.synchronize()
    wall = time.perf_counter() - t1
    step_us = dev_us / steps
    mean_used = float(np.mean(used))
    vec_bytes = batch * ((4096 + 1024 + 1024 + 32768 + 4096 + 512 + 8 * (4096 + 1024) + 8192 + 4096) * 4
                         + 4096 * 2 + 4096 * 4)
    step_bytes = n_layers * (wl.DECODE_LAYER_FP8_BYTES + wl.FP4_EXPERT_BYTES + vec_bytes) \
        + sum(used) / steps * wl.FP4_EXPERT_BYTES
    for per in ids_dev + sc_dev:
        for d in per:
            ctx.device_free(d)
    for d in list(dev.values()) + list(ydev.values()) + [moe_x, moe_out]:
        ctx.device_free(d)
    gbs = step_bytes / (step_us * 1e-6) / 1e9
    return {"workload": f"{n_layers} decode layers at batch {batch}: FP8 projections over {batch} inputs, "
                        f"MoE of {batch} positions (shared + top-6 of 256 routed, expert-major batch path)",
            "routed_experts_per_layer": round(mean_used, 1), "bytes_per_step": int(step_bytes),
            "step_us": round(step_us, 1), "wall_step_us": round(wall / steps * 1e6, 1),
            "layer_us": round(step_us / n_layers, 2), "GBps": round(gbs, 1),
            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "tokens_per_s": round(batch / (step_us * 1e-6), 1)}


TIMELINE_POINTS = {
    "token_gateup": ["start", "DMAs issued", "x slice landed", "x slice act-quantized", "B operands loaded",
                     "tile 0 done", "tile 1 done", "tile 2 done", "tile 3 done", None, "tiles summed", "end"],
    "token_down": ["start", "DMAs issued", "h quarters landed", "h act-quantized, B operands loaded", None,
                   "unit 0 done", "unit 1 done", "unit 2 done", "unit 3 done", None, "units summed", "end"],
    "token_gateup_px": ["start", "tables staged", "x in registers", "x act-quantized", "ring issued",
                        "barrier passed", "tile 0 done", "tile 1 done", "tile 2 done", "tile 3 done", "tiles summed",
                        "end"],
    "token_down_px": ["start", "prologue issued", "h in registers", "h act-quantized", "ring issued", "codes written",
                      "unit 0 done", "unit 1 done", "unit 2 done", "unit 3 done", "units summed", "end"],
    "batch_gateup": ["start", "ring issued", "B staged", "wave's last item done", "workgroup end"],
    "batch_down": ["start", "ring issued", "B staged", "wave's last item done", "workgroup end"],
    "router": ["start", "x staged", "gate rows landed", "dot done", "scores published", "arrived",
               "last: scores gathered", "last: selected", "last: keys", "last: rounds done", "last: weight sum"],
}


def timeline(lib_path: str, seed: int = 2) -> dict:
    """Per-wave timelines of the persistent expert kernels from the measuring
    build (python -m wohper_amd.build --timeline PATH): the routed FP4 token
    (MFMA numerics; k_moe_gateup_px, k_moe_down_px) and the batch-16 MoE with
    the shared expert (k_moe_batch_mx gate/up and down).  Each kernel's lane 0
    of every wave of the first 256 workgroups stamps s_memrealtime (100 MHz)
    at fixed points; returned: per point the 0/10/50/90/100th percentiles in
    us from the launch's earliest start stamp, of the last of 12 calls."""
    import ctypes

    import wohper_amd
    from wohper_amd import workloads as wl

    lib = wohper_amd.load_library(lib_path)
    if not hasattr(lib, "wh_debug_timeline"):
        raise SystemExit(f"{lib_path} is not a timeline build (python -m wohper_amd.build --timeline PATH)")
    wohper_amd._lib = lib
    lib.wh_debug_timeline.restype = ctypes.c_int
    lib.wh_debug_timeline.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t]
    ctx = wohper_amd.Context(0)
    ctx.set_exact_numerics(False)
    n_layers = 4
    for layer in range(n_layers):
        for e in range(wl.N_ROUTED + 1):
            ctx.store_expert_synthetic(layer, e, wl.HIDDEN, wl.INTER, seed)
    rng = np.random.default_rng(seed)
    n_points = 16
    n_stamp = 512 * 16 * n_points

    def read(which, names):
        buf = np.zeros(n_stamp, np.uint64)
        assert lib.wh_debug_timeline(which, buf.ctypes.data, n_stamp) == 0
        t = buf.reshape(512, 16, n_points)[:256].astype(np.int64)
        t0 = t[:, :, 0][t[:, :, 0] > 0].min()
        out = {}
        for k, name in enumerate(names):
            if name is None:
                continue
            v = t[:, :, k].ravel()
            v = (v[v > 0] - t0) * 0.01
            if v.size:
                out[name] = [round(float(np.percentile(v, q)), 2) for q in (0, 10, 50, 90, 100)]
        return out

    res = {"percentiles": [0, 10, 50, 90, 100], "unit": "us from the launch's first start stamp"}
    x = wl.bf16_bits(rng.standard_normal((1, wl.HIDDEN)).astype(np.float32))
    x_dev, out_dev = ctx.device_alloc(x.nbytes), ctx.device_alloc(wl.HIDDEN * 4)
    ctx.to_device(x_dev, x)
    for version, tag in ((0, "_px"), (3, "")):
        ctx.debug_token_kernels(version)
        for i in range(12):
            idx, w = wl.route_topk_sigmoid(rng.standard_normal(wl.N_ROUTED).astype(np.float32))
            ctx.routed_experts_async([(i % n_layers, int(e), float(wt)) for e, wt in zip(idx, w)], x_dev, True, 1,
                                     out_dev)
            ctx.synchronize()
        res["token_gateup" + tag] = read(0, TIMELINE_POINTS["token_gateup" + tag])
        res["token_down" + tag] = read(1, TIMELINE_POINTS["token_down" + tag])
    npos = 16
    ids = np.stack([rng.choice(wl.N_ROUTED, wl.TOPK, replace=False) for _ in range(npos)]).astype(np.uint32)
    sc = rng.uniform(0.1, 1.0, (npos, wl.TOPK)).astype(np.float32)
    xb = wl.bf16_bits(rng.standard_normal((npos, wl.HIDDEN)).astype(np.float32))
    xd, idd, scd, od = (ctx.device_alloc(xb.nbytes), ctx.device_alloc(ids.nbytes), ctx.device_alloc(sc.nbytes),
                        ctx.device_alloc(npos * wl.HIDDEN * 4))
    ctx.to_device(xd, xb)
    ctx.to_device(idd, ids)
    ctx.to_device(scd, sc)
    for i in range(12):
        ctx.moe_batch_async(i % n_layers, idd, scd, npos, wl.TOPK, xd, True, od, shared_key=(i % n_layers, wl.N_ROUTED))
        ctx.synchronize()
    res["batch_gateup"] = read(0, TIMELINE_POINTS["batch_gateup"])
    res["batch_down"] = read(1, TIMELINE_POINTS["batch_down"])
    # the bf16 router (one wave per workgroup, 64 workgroups)
    from wohper_amd import model_format as mf
    rows, cols = 256, 4096
    gate = ((rng.standard_normal((rows, cols)).astype(np.float32) * 0.02).view(np.uint32) >> 16).astype(np.uint16)
    bias = (rng.standard_normal(rows) * 0.05).astype(np.float32)
    for k in range(n_layers):
        blk = mf.build_synthetic_quant_block([
            mf.SyntheticTensor(f"layers.{k}.ffn.gate.weight", 9, (rows, cols), gate.tobytes(), 11, 2404),
            mf.SyntheticTensor(f"layers.{k}.ffn.gate.bias", 9, (rows,), bias.tobytes(), 12, 2405)])
        ctx.store_router(1000 + k, blk, cols)
    rx, rout = ctx.device_alloc(cols * 4), ctx.device_alloc(256)
    ctx.to_device(rx, rng.standard_normal(cols).astype(np.float32))
    for i in range(12):
        ctx.synchronize()
        if i == 11:
            # clears the stamps: the "last:" points then hold only the last
            # call's last workgroup (earlier calls' last workgroups differ)
            assert lib.wh_debug_timeline(0, None, 0) == 0
        ctx.route_experts_async(1000 + i % n_layers, rx, cols, 6, 0, 0, rout, rout + 64, rout + 128, route_scale=1.5)
    ctx.synchronize()
    res["router"] = read(0, TIMELINE_POINTS["router"])
    ctx.close()
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--layers", type=int, default=8, help="resident layers of 256 experts")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-fp8", action="store_true")
    ap.add_argument("--no-aux", action="store_true", help="skip the router and experts-pack load legs")
    ap.add_argument("--aux-legs", default="decode_layer,read_floor,router,expert_pack_load",
                    help="which of the auxiliary legs to run (comma-separated)")
    ap.add_argument("--stack-layers", type=int, default=43, help="layers of the full-depth stack leg (0: skip)")
    ap.add_argument("--stack-steps", type=int, default=20)
    ap.add_argument("--batch-steps", type=int, default=20, help="steps of the ragged batch leg (0: skip)")
    ap.add_argument("--stack-batch-steps", type=int, default=3,
                    help="steps of the batch-16 full-depth stack (0: skip)")
    ap.add_argument("--exact", action="store_true",
                    help="headline on the bit-exact kernels (the reference's summation order) instead of the MFMA "
                         "kernels (each matvec within 1e-5 * ||w_row|| * ||x|| of the reference kernel)")
    ap.add_argument("--batch-mfma-sweep", type=str, default="",
                    help="only time the ragged batch leg: exact items, then each MFMA threshold of this "
                         "comma-separated list (one JSON line each)")
    ap.add_argument("--timeline", type=str, default="",
                    help="only print the per-wave timelines of the expert kernels from this measuring build "
                         "(python -m wohper_amd.build --timeline PATH)")
    ap.add_argument("--no-graph", action="store_true",
                    help="time the headline and the stack as host loops of launches instead of HIP graph replays "
                         "(for kernel-trace profiler runs, which do not follow graph launches here)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 256 MiB device copy 5 times (calibrates HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (every box here has one MI355X); --gpus {args.gpus} is not supported",
              file=sys.stderr)
        sys.exit(2)

    if args.timeline:
        print(json.dumps(timeline(args.timeline)), flush=True)
        return

    import wohper_amd
    from wohper_amd import workloads as wl

    seed = 2
    ctx = wohper_amd.Context(0)
    ctx.set_exact_numerics(args.exact)
    if args.copy_calibration:
        buf = np.arange(64 << 20, dtype=np.float32)
        for _ in range(5):
            assert np.array_equal(ctx.debug_eval(3, buf), buf)
        log("copy calibration: 5 x k_copy_f32x4 of 268,435,456 bytes read + 268,435,456 written")
        ctx.close()
        return
    t0 = time.perf_counter()
    for layer in range(args.layers):
        for e in range(wl.N_ROUTED):
            ctx.store_expert_synthetic(layer, e, wl.HIDDEN, wl.INTER, seed)
    dev_bytes, _, n_exp = ctx.usage()
    log(f"resident: {n_exp} experts, {dev_bytes / 1e9:.1f} GB in {time.perf_counter() - t0:.1f} s")
    if args.batch_mfma_sweep:
        modes = [(True, 0)] + [(False, int(m)) for m in args.batch_mfma_sweep.split(",")]
        for exact, m in modes:
            print(json.dumps(ragged_batch(ctx, args.layers, args.batch_steps, 3, exact, m)), flush=True)
        ctx.close()
        return

    total = args.warmup + args.steps
    rng = np.random.default_rng(seed)
    routes = []
    for i in range(total):
        logits = rng.standard_normal(wl.N_ROUTED).astype(np.float32)
        idx, w = wl.route_topk_sigmoid(logits)
        routes.append([(i % args.layers, int(e), float(wt)) for e, wt in zip(idx, w)])
    xs = wl.bf16_bits(rng.standard_normal((total, wl.HIDDEN)).astype(np.float32))
    x_dev = ctx.device_alloc(xs.nbytes)
    out_dev = ctx.device_alloc(total * wl.HIDDEN * 4)
    ctx.to_device(x_dev, xs)

    def step(i):
        ctx.routed_experts_async(routes[i], x_dev + i * wl.HIDDEN * 2, True, 1, out_dev + i * wl.HIDDEN * 4)

    for i in range(args.warmup):
        step(i)
    ctx.synchronize()
    # The timed region: the K timed tokens (token i on its own route list,
    # input row and output row) captured once into a HIP graph of their
    # gate/up and down launches and replayed by one library call, so no
    # per-step Python call paces the device; HIP events on the library stream
    # bracket exactly those K steps (the graph's second replay; the first is
    # untimed).  The host clock around the same call is reported beside it.
    t0 = time.perf_counter()
    launch_us = ctx.profile_token_pipeline(routes[args.warmup:total], x_dev + args.warmup * wl.HIDDEN * 2, True,
                                           wl.HIDDEN * 2, out_dev + args.warmup * wl.HIDDEN * 4, args.steps,
                                           not args.no_graph)
    call_s = time.perf_counter() - t0
    ms_per_step = launch_us * 1e-3
    value = TOKEN_BYTES / (launch_us * 1e-6) / 1e9
    # the same steps enqueued one Python call per token (the entry point a
    # caller uses per token), HIP events around them
    ctx.timer_start()
    for i in range(args.warmup, total):
        step(i)
    py_us = ctx.timer_stop() / args.steps
    ctx.synchronize()
    log(f"routed FP4 MoE: {launch_us:.2f} us/token (graph of {args.steps} tokens), {value:.1f} GB/s; "
        f"one Python call per token {py_us:.2f} us/token")

    # per-kernel launch durations: each stage launched back to back over the
    # timed steps' route lists, between HIP events on the library stream
    gu_us, dn_us = ctx.profile_routed(routes[args.warmup:args.warmup + min(args.steps, 64)], x_dev, True, out_dev,
                                      max(200, args.steps))
    gu_gbs = GATEUP_BYTES / (gu_us * 1e-6) / 1e9
    dn_gbs = DOWN_BYTES / (dn_us * 1e-6) / 1e9
    log(f"kernels: k_moe_gateup {gu_us:.2f} us ({gu_gbs:.0f} GB/s), k_moe_down {dn_us:.2f} us ({dn_gbs:.0f} GB/s)")

    gu_name, dn_name = KERNELS[args.exact]
    extra = {"numerics": "exact (the reference kernel's summation order)" if args.exact else
             "MFMA (each matvec within 1e-5 * ||w_row|| * ||x|| of the reference kernel)",
             "kernels": {gu_name: {"us": round(gu_us, 3), "GBps": round(gu_gbs, 1), "bytes_per_launch": GATEUP_BYTES},
                         dn_name: {"us": round(dn_us, 3), "GBps": round(dn_gbs, 1), "bytes_per_launch": DOWN_BYTES},
                         "token_device_us": round(launch_us, 3)},
             "timed_region": (f"{args.steps} tokens replayed as one HIP graph (one library call, "
                              f"{call_s * 1e3:.1f} ms host time for capture, untimed replay and timed replay)")
                             if not args.no_graph else
                             f"{args.steps} tokens enqueued by one library call as a host loop of launches",
             "token_us_one_python_call_per_token": round(py_us, 3)}
    # the other numerics mode's kernels on the same route lists
    ctx.set_exact_numerics(not args.exact)
    o_gu, o_dn = ctx.profile_routed(routes[args.warmup:args.warmup + min(args.steps, 64)], x_dev, True, out_dev,
                                    max(200, args.steps))
    ctx.set_exact_numerics(args.exact)
    og, od = KERNELS[not args.exact]
    extra["other_numerics_kernels"] = {og: {"us": round(o_gu, 3), "GBps": round(GATEUP_BYTES / (o_gu * 1e-6) / 1e9, 1)},
                                       od: {"us": round(o_dn, 3), "GBps": round(DOWN_BYTES / (o_dn * 1e-6) / 1e9, 1)}}
    log(f"other numerics: {extra['other_numerics_kernels']}")
    if not args.no_fp8:
        extra["fp8_dense_gemv"] = fp8_dense(ctx, max(200, args.steps), 40)
        ctx.set_exact_numerics(args.exact)
        log(f"fp8 dense: {extra['fp8_dense_gemv']}")
        extra["fp8_decode_layer"] = fp8_decode_layer(ctx, 200)
        ctx.set_exact_numerics(args.exact)
        log(f"fp8 decode layer: {extra['fp8_decode_layer']}")
        extra["fp8_decode_layer_batch16"] = fp8_decode_layer_batch(ctx, 200)
        ctx.set_exact_numerics(args.exact)
        log(f"fp8 decode layer, batch 16: {extra['fp8_decode_layer_batch16']}")
    aux = set(args.aux_legs.split(",")) if not args.no_aux else set()
    if "decode_layer" in aux:
        extra["decode_layer"] = decode_layer(ctx, args.layers, 20, not args.no_graph)
        ctx.set_exact_numerics(args.exact)
        log(f"decode layer: {extra['decode_layer']}")
    if "read_floor" in aux:
        extra["read_floor"] = read_floor(ctx)
        log(f"read floor: {extra['read_floor']}")
    if "router" in aux:
        extra["router"] = router(ctx, 400)
        log(f"router: {extra['router']}")
    if "expert_pack_load" in aux:
        extra["expert_pack_load"] = expert_pack_load(ctx)
        log(f"expert pack load: {extra['expert_pack_load']}")
    if args.batch_steps > 0:
        extra["ragged_batch"] = ragged_batch(ctx, args.layers, args.batch_steps, 3, args.exact)
        if not args.exact:
            # the configuration's own wording: MFMA only for experts of at
            # least 16 tokens (the rest on the exact items)
            t16 = ragged_batch(ctx, args.layers, args.batch_steps, 3, False, 16)
            extra["ragged_batch"]["mfma_min_16"] = {k: t16[k] for k in ("numerics", "experts_on_mfma", "us_per_step",
                                                                         "GBps", "frac_of_hbm_peak",
                                                                         "device_us_per_step")}
            ctx.set_moe_mfma_min(1)
        ctx.set_exact_numerics(args.exact)
        log(f"ragged batch: {extra['ragged_batch']}")
    cpu = None
    if not args.no_cpu:
        cpu, extra["cpu_configs"] = cpu_baseline(ctx.lib, seed, args.cpu_seconds)
        log(f"cpu baseline: {cpu}; {extra['cpu_configs']}")

    if args.stack_layers > 0:
        ctx.close()
        ctx = None
        extra["decode_stack"] = decode_stack(args.stack_layers, args.stack_steps, 3, seed, args.stack_batch_steps,
                                             args.exact, not args.no_graph)
        log(f"decode stack: {extra['decode_stack']}")

    line = {
        "metric": "HBM GB/s (% of peak) for FP4 expert + FP8 dense matvec; batch-1 decode step us",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp4-e2m1/fp8-e4m3 weights, f32 accumulate",
        "data": "synthetic (seeded random weights and activations; no checkpoint offline)",
        "config": {"workload": "routed MoE FFN, 1 token, top-6 of 256 FP4 experts (w1/w3 2048x4096, "
                               "w2 4096x2048, UE8M0 per 32), bf16 x",
                   "global_batch": 1, "experts_resident": n_exp, "resident_GB": round(dev_bytes / 1e9, 2),
                   "bytes_per_step": TOKEN_BYTES, "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": GATEUP_TRAFFIC_BYTES[args.exact],
                     "kernel": gu_name, "bytes_per_launch": GATEUP_BYTES,
                     "avg_launch_us": round(gu_us, 3)},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    if ctx is not None:
        ctx.device_free(x_dev)
        ctx.device_free(out_dev)
        ctx.close()


if __name__ == "__main__":
    main()
