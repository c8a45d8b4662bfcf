// DeepSeek-V4 hyper-connections (mHC) on gfx950: hc_pre_into,
// hc_split_sinkhorn_scalar and hc_post_into (E/compute.rs:4945-5092).
//
// The residual stream holds hc copies of the hidden state (hc * hidden f32,
// 4 x 4096 for V4).  hc_pre reduces them to one working stream: mix_hc =
// (2 + hc) hc dots of learned f32 rows with the stream, scaled by the
// stream's inverse RMS, go through sigmoids (pre, post) and a Sinkhorn
// normalisation (comb); y = sum over i of pre[i] * copy i.  hc_post spreads
// a sub-block's output back: out[k] = post[k] y + sum over i of
// comb[k][i] copy i.
//
// The dots and the sum of squares are 16384-term sums.  In the reference's
// order (each term added to a running f32 sum, E/compute.rs:5026-5038) they
// are serial chains: k_hc_chains runs each chain on one lane of a wave (the
// 24 dots and the sum of squares side by side), which is bit-exact and
// bound by the chain's length.  With exact numerics off, k_hc_partials
// spreads the terms over many workgroups and k_hc_finish adds the partial
// sums in a fixed order: the same value up to rounding, reproducible run to
// run.  Everything after the sums (sigmoids, Sinkhorn, y, hc_post) is
// bit-exact in both modes.
#pragma once
#include "kernels.h"

#define WH_HC_MAX_CHAINS 256u  // mix_hc + 1 (hc <= 14)
#define WH_HC_PARTS 16u        // workgroups per chain of k_hc_partials

struct wh_hc_args {
    const float* fn;       // [mix_hc][hc_dim] f32 rows (or null: mixes given)
    const float* scale;    // [3]
    const float* base;     // [mix_hc]
    const float* x;        // [hc_dim] (or null: no y)
    const float* mixes_in; // [mix_hc] given mixes (hc_split_sinkhorn alone), else null
    float* sums;           // [WH_HC_PARTS or 1][mix_hc + 1] chain sums, then pre (scratch)
    float* y;              // [hidden]
    float* pre;            // [hc]
    float* post;           // [hc]
    float* comb;           // [hc * hc]
    uint32_t hc, hidden, hc_dim, mix_hc, iters, parts;
    float eps;
    // several streams at once: stream z (blockIdx.z of the sums, blockIdx.x
    // of k_hc_finish, blockIdx.y of k_hc_y) reads x + z * hc_dim and writes
    // y + z * hidden, sums + z * sums_ld, pre / post + z * hc, comb + z * hc * hc
    uint32_t sums_ld;
};

// The arguments of stream z of a batched launch.
__device__ __forceinline__ wh_hc_args wh_hc_at(wh_hc_args a, uint32_t z) {
    a.x += (size_t)z * a.hc_dim;
    a.y += (size_t)z * a.hidden;
    a.sums += (size_t)z * a.sums_ld;
    a.pre += (size_t)z * a.hc;
    a.post += (size_t)z * a.hc;
    a.comb += (size_t)z * a.hc * a.hc;
    return a;
}

// Sum over a wave in a fixed butterfly (every lane ends with the same bits).
__device__ __forceinline__ float wh_hc_wave_sum(float v) {
    for (int off = 32; off > 0; off >>= 1) v = v + __shfl_xor(v, off, 64);
    return v;
}

// Serial chains: workgroup c (256 threads) runs chain c < mix_hc (fn row
// c . x) or, for c = mix_hc, the sum of squares.  The 192 threads of waves
// 1-3 form the products w * x (each rounded on its own) of a chunk of
// WH_HC_CHUNK terms into an LDS buffer, their loads for the next chunk in
// flight meanwhile, while thread 0 adds the previous chunk's products to
// its running sum in order; two buffers alternate.
#define WH_HC_CHUNK 768u  // 4 terms per producer thread
__global__ void __launch_bounds__(256) k_hc_chains(wh_hc_args a0) {
    const wh_hc_args a = wh_hc_at(a0, blockIdx.z);
    __shared__ __align__(16) float prod[2][WH_HC_CHUNK];
    const uint32_t t = threadIdx.x, c = blockIdx.x;
    const uint32_t n_chunks = (a.hc_dim + WH_HC_CHUNK - 1) / WH_HC_CHUNK;
    const float* row = c < a.mix_hc ? a.fn + (size_t)c * a.hc_dim : a.x;
    const uint32_t u = t - 64;  // producer index (t >= 64)
    float w[4], xv[4];
    auto load = [&](uint32_t k) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t e = k * WH_HC_CHUNK + u + 192 * i;
            const bool on = k < n_chunks && e < a.hc_dim;
            xv[i] = on ? a.x[e] : 0.0f;
            w[i] = on ? row[e] : 0.0f;
        }
    };
    if (t >= 64) load(0);
    float acc = 0.0f;
    for (uint32_t k = 0; k <= n_chunks; ++k) {
        if (t >= 64 && k < n_chunks) {
#pragma unroll
            for (int i = 0; i < 4; ++i) prod[k & 1][u + 192 * i] = w[i] * xv[i];
            load(k + 1);
        }
        if (t == 0 && k > 0) {
            const float* src = prod[(k - 1) & 1];
            const uint32_t len = min(WH_HC_CHUNK, a.hc_dim - (k - 1) * WH_HC_CHUNK);
            acc = wh_ordered_sum_lds(src, len, acc);
        }
        __syncthreads();
    }
    if (t == 0) a.sums[c] = acc;
}

// Partial sums (exact numerics off): grid (WH_HC_PARTS, mix_hc + 1), 256
// threads; workgroup (p, c) sums slice p of chain c's products in a fixed
// tree.
__global__ void __launch_bounds__(256) k_hc_partials(wh_hc_args a0) {
    const wh_hc_args a = wh_hc_at(a0, blockIdx.z);
    __shared__ float red[4];
    const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63, c = blockIdx.y;
    const uint32_t per = (a.hc_dim + a.parts - 1) / a.parts;
    const uint32_t i0 = blockIdx.x * per, i1 = min(i0 + per, a.hc_dim);
    const float* row = c < a.mix_hc ? a.fn + (size_t)c * a.hc_dim : a.x;
    float s = 0.0f;
    uint32_t i = i0 + t;
    // four terms' loads at a time (a load in a loop is waited for before the
    // next is issued)
    for (; i + 3 * 256 < i1; i += 4 * 256) {
        float rv[4], xv[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            rv[k] = row[i + 256 * k];
            xv[k] = a.x[i + 256 * k];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) s = s + rv[k] * xv[k];
    }
    for (; i < i1; i += 256) s = s + row[i] * a.x[i];
    s = wh_hc_wave_sum(s);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    if (t == 0) a.sums[(size_t)blockIdx.x * (a.mix_hc + 1) + c] = (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ float wh_sigmoid(float v) {
    return 1.0f / (1.0f + wh_expf_glibc(-v, kExpTab, kExpfExc, WH_EXPF_EXC_COUNT));
}

// One workgroup of 256 threads: mixes = chain sums * inverse RMS (or the
// given mixes), then hc_split_sinkhorn_scalar.
__global__ void __launch_bounds__(256) k_hc_finish(wh_hc_args a0) {
    const wh_hc_args a = wh_hc_at(a0, blockIdx.x);
    __shared__ float mixes[WH_HC_MAX_CHAINS];
    __shared__ float comb[WH_HC_MAX_CHAINS];
    __shared__ float rsum[16];
    __shared__ float inv_s;
    const uint32_t t = threadIdx.x, hc = a.hc, hh = hc * hc;
    // the parameters this thread uses, requested first (clamped indices:
    // loads under branches would be waited for one at a time)
    const uint32_t last = a.mix_hc - 1;
    const float sc0 = a.scale[0], sc1 = a.scale[1], sc2 = a.scale[2];
    const float bv0 = a.base[t < last ? t : last], bv1 = a.base[t + hc < last ? t + hc : last];
    const float bv2 = a.base[2 * hc + t < last ? 2 * hc + t : last];
    if (a.mixes_in) {
        if (t < a.mix_hc) mixes[t] = a.mixes_in[t];
    } else {
        if (a.parts <= 1) {
            if (t <= a.mix_hc) mixes[t] = a.sums[t];  // slot mix_hc: the sum of squares
        } else {
            // the partial sums through LDS, then each chain's in the order
            // of the parts
            __shared__ float stage[WH_HC_PARTS * WH_HC_MAX_CHAINS];
            const uint32_t n_ch = a.mix_hc + 1, tot = a.parts * n_ch;
            uint32_t i = t;
            for (; i + 256 < tot; i += 512) {
                const float s0 = a.sums[i], s1 = a.sums[i + 256];
                stage[i] = s0;
                stage[i + 256] = s1;
            }
            if (i < tot) stage[i] = a.sums[i];
            __syncthreads();
            if (t < n_ch) {
                float s = 0.0f;
                for (uint32_t p = 0; p < a.parts; ++p) s = s + stage[p * n_ch + t];
                mixes[t] = s;
            }
        }
        __syncthreads();
        if (t == 0) {
            const float ms = mixes[a.mix_hc] / (float)a.hc_dim;
            inv_s = 1.0f / sqrtf(ms + a.eps);
        }
        __syncthreads();
        if (t < a.mix_hc) mixes[t] = mixes[t] * inv_s;
    }
    __syncthreads();
    // hc_split_sinkhorn on wave 0 alone
    const float eps = a.eps;
    if (t >= 64) return;
    if (t < hc) {
        a.pre[t] = wh_sigmoid(mixes[t] * sc0 + bv0) + eps;
        a.post[t] = 2.0f * wh_sigmoid(mixes[t + hc] * sc1 + bv1);
    }
    const uint32_t n_ops = a.iters ? 2 * a.iters - 1 : 1;
    if (hc == 4) {
        // DeepSeek-V4's hc: comb[j][k] in lane 4j + k of each 16-lane row.
        // A lane gathers its row with DPP quad broadcasts and its column
        // with the three row rotations by 4, 8 and 12 lanes; which row each
        // rotation brings is read off the rotated lane index, so the adds
        // keep the reference's order with no assumption on the rotation's
        // direction.
        const uint32_t j = (t >> 2) & 3;
        const uint32_t r1 = ((uint32_t)__builtin_amdgcn_mov_dpp((int)t, 0x124, 0xf, 0xf, false) >> 2) & 3;
        const uint32_t r2 = ((uint32_t)__builtin_amdgcn_mov_dpp((int)t, 0x128, 0xf, 0xf, false) >> 2) & 3;
        auto row_q = [](float x, auto q) {
            constexpr int kQ = decltype(q)::value;
            return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), kQ * 0x55, 0xf, 0xf, false));
        };
        auto row_sum = [&](float x) {
            float r = 0.0f;
            r = r + row_q(x, std::integral_constant<int, 0>());
            r = r + row_q(x, std::integral_constant<int, 1>());
            r = r + row_q(x, std::integral_constant<int, 2>());
            r = r + row_q(x, std::integral_constant<int, 3>());
            return r;
        };
        auto col_sum = [&](float x) {
            const float x1 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x124, 0xf, 0xf, false));
            const float x2 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x128, 0xf, 0xf, false));
            const float x3 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x12C, 0xf, 0xf, false));
            float r = 0.0f;
#pragma unroll
            for (uint32_t q = 0; q < 4; ++q) r = r + (j == q ? x : r1 == q ? x1 : r2 == q ? x2 : x3);
            return r;
        };
        const bool on = t < 16;
        float v = on ? mixes[8 + t] * sc2 + bv2 : 0.0f;  // 2 hc = 8
        float mx = -__uint_as_float(0x7f800000u);
        mx = fmaxf(mx, row_q(v, std::integral_constant<int, 0>()));
        mx = fmaxf(mx, row_q(v, std::integral_constant<int, 1>()));
        mx = fmaxf(mx, row_q(v, std::integral_constant<int, 2>()));
        mx = fmaxf(mx, row_q(v, std::integral_constant<int, 3>()));
        v = wh_expf_glibc(v - mx, kExpTab, kExpfExc, WH_EXPF_EXC_COUNT);
        v = v / row_sum(v) + eps;
        // n_ops is odd: a column step, then (row, column) pairs; no branch
        // on the step's parity inside the loop
        v = v / (col_sum(v) + eps);
#pragma unroll 2
        for (uint32_t it = 1; it < n_ops; it += 2) {
            v = v / (row_sum(v) + eps);
            v = v / (col_sum(v) + eps);
        }
        if (on) a.comb[t] = v;
        return;
    }
    if (hh <= 64) {
        // comb[j][k] in lane j * hc + k; a lane gathers its row or column
        // with shuffles and sums it in order
        const uint32_t j = t / hc, k = t % hc;
        const bool on = t < hh;
        float v = on ? mixes[2 * hc + t] * sc2 + bv2 : 0.0f;
        float mx = -__uint_as_float(0x7f800000u);
        for (uint32_t q = 0; q < hc; ++q) mx = fmaxf(mx, __shfl(v, (int)(j * hc + q), 64));
        v = wh_expf_glibc(v - mx, kExpTab, kExpfExc, WH_EXPF_EXC_COUNT);
        float s = 0.0f;
        for (uint32_t q = 0; q < hc; ++q) s = s + __shfl(v, (int)(j * hc + q), 64);
        v = v / s + eps;
        for (uint32_t it = 0; it < n_ops; ++it) {
            const bool cols = (it & 1) == 0;
            float r = 0.0f;
            for (uint32_t q = 0; q < hc; ++q) r = r + __shfl(v, (int)(cols ? q * hc + k : j * hc + q), 64);
            v = v / (r + eps);
        }
        if (on) a.comb[t] = v;
        return;
    }
    // larger hc: comb in LDS, one row or column per lane, ordered by wave
    // barriers
    auto wave_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    for (uint32_t l = t; l < hh; l += 64) comb[l] = mixes[2 * hc + l] * a.scale[2] + a.base[2 * hc + l];
    wave_sync();
    if (t < hc) {
        float* row = comb + t * hc;
        float mx = -__uint_as_float(0x7f800000u);
        for (uint32_t k = 0; k < hc; ++k) mx = fmaxf(mx, row[k]);
        float s = 0.0f;
        for (uint32_t k = 0; k < hc; ++k) {
            row[k] = wh_expf_glibc(row[k] - mx, kExpTab, kExpfExc, WH_EXPF_EXC_COUNT);
            s = s + row[k];
        }
        rsum[t] = s;
    }
    wave_sync();
    for (uint32_t l = t; l < hh; l += 64) comb[l] = comb[l] / rsum[l / hc] + eps;
    wave_sync();
    for (uint32_t it = 0; it < n_ops; ++it) {
        const bool cols = (it & 1) == 0;
        if (t < hc) {
            float s = 0.0f;
            for (uint32_t k = 0; k < hc; ++k) s = s + (cols ? comb[k * hc + t] : comb[t * hc + k]);
            rsum[t] = s + eps;
        }
        wave_sync();
        for (uint32_t l = t; l < hh; l += 64) comb[l] = comb[l] / rsum[cols ? l % hc : l / hc];
        wave_sync();
    }
    for (uint32_t l = t; l < hh; l += 64) a.comb[l] = comb[l];
}

// y[d] = sum over i, in order, of pre[i] * x[i * hidden + d] (the end of
// hc_pre_into), one output per thread.
__global__ void __launch_bounds__(256) k_hc_y(wh_hc_args a0) {
    const wh_hc_args a = wh_hc_at(a0, blockIdx.y);
    const uint32_t d = blockIdx.x * 256 + threadIdx.x;
    if (d >= a.hidden) return;
    float acc = 0.0f;
    if (a.hc == 4) {
        // DeepSeek-V4's hc: the four copies' loads issued together
        float xv[4], pv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xv[i] = a.x[(size_t)i * a.hidden + d];
            pv[i] = a.pre[i];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) acc = acc + pv[i] * xv[i];
    } else {
        for (uint32_t i = 0; i < a.hc; ++i) acc = acc + a.pre[i] * a.x[(size_t)i * a.hidden + d];
    }
    a.y[d] = acc;
}

// hc_post_into: out[k * hidden + d] = post[k] * y[d], then + comb[k][i] *
// residual[i * hidden + d] for i in order.  Stream z = blockIdx.y of a
// batched launch: y + z * hidden, residual and out + z * hc * hidden,
// post + z * hc, comb + z * hc * hc.
__global__ void __launch_bounds__(256) k_hc_post(const float* __restrict__ y, const float* __restrict__ res,
                                                 const float* __restrict__ post, const float* __restrict__ comb,
                                                 float* __restrict__ out, uint32_t hc, uint32_t hidden) {
    const size_t z = blockIdx.y, hcd = (size_t)hc * hidden;
    y += z * hidden;
    res += z * hcd;
    out += z * hcd;
    post += z * hc;
    comb += z * hc * hc;
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)hc * hidden) return;
    const uint32_t k = (uint32_t)(idx / hidden), d = (uint32_t)(idx % hidden);
    float acc = post[k] * y[d];
    if (hc == 4) {
        // DeepSeek-V4's hc: the four copies' loads issued together
        float rv[4], cv[4];
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            rv[i] = res[(size_t)i * hidden + d];
            cv[i] = comb[k * 4 + i];
        }
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) acc = acc + cv[i] * rv[i];
    } else {
        for (uint32_t i = 0; i < hc; ++i) acc = acc + comb[k * hc + i] * res[(size_t)i * hidden + d];
    }
    out[idx] = acc;
}
