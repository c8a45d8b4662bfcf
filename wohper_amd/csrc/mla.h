// The non-GEMV glue of a DeepSeek-V4 MLA attention layer at decode, on
// gfx950: RMS norms, interleaved RoPE / YaRN, the act-quant between
// projections, and the sliding-window softmax with attention sink
// (compute_deepseek_v4_mla_attention, E/compute.rs:3924-4293).
//
// Every value follows the reference's f32 arithmetic bit for bit: sums run
// in the reference's sequential order (one lane per chain), products and
// sums are separate roundings (the library is built without contraction),
// exp / sin / cos are the glibc-exact restatements of libm_emul.h, and the
// act-quant is the block-64 rule of E/compute.rs:2504-2521.  The data are a
// few hundred KB per token, so these kernels are latency-bound: they keep
// the hidden state on the device between the FP8 projections rather than
// aiming at bandwidth.
#pragma once
#include "kernels.h"

#define WH_ROWPOST_MAX 4096u     // values per row of k_rowpost
#define WH_ATTN_MAX_KEYS 2048u   // window + compressed keys per head
#define WH_ATTN_MAX_HEAD_DIM 1024u
#define WH_POS_BATCH 32u         // positions per batched launch of k_rowpost / the attention

__device__ __forceinline__ float wh_bf16_value(uint16_t raw) { return __uint_as_float((uint32_t)raw << 16); }

// Act-quant (E/compute.rs:2504-2521) of one 64-value block held one value
// per lane of a wave; lanes past the block's end pass valid = false (they
// add nothing to the block maximum, as the reference's shorter tail chunk).
__device__ __forceinline__ float wh_aq64_wave(float x, bool valid) {
    float amax = wh_wave_max(valid ? fabsf(x) : 0.0f);
    amax = fmaxf(amax, 1.0e-4f);
    const bool inf_scale = !(amax <= 3.4028235e38f);
    const int k = inf_scale ? 0 : wh_aq_scale_exp(amax, kLog2Thr);
    const float scale = inf_scale ? __uint_as_float(0x7f800000u) : wh_pow2f(k);
    const float inv = inf_scale ? 0.0f : wh_pow2f(-k);
    const float t = inf_scale ? x / scale : x * inv;
    const float q = t != t ? -480.0f : wh_e4m3_round(wh_clamp448(t));  // NaN -> the lowest LUT entry
    return q * scale;
}

// ------------------------------------------------------------- row glue
// Per row r (one workgroup of 256 threads each), in this order, on
// x + r * ld_in, n values:
//   norm:  rms_norm_in_place (E/compute.rs:7110-7122) when w is null, else
//          apply_weighted_rms_norm (E/compute.rs:3077-3107) with bf16 w:
//          s = sequential sum of v*v, inv = 1 / sqrt(s / n + 1e-6),
//          v = v * inv (* w);
//   rope:  apply_rope_interleaved_with_freqs (E/compute.rs:2623-2649) on
//          [rope_off, rope_off + 2 pairs) at `position`, inverse or not;
//   quant: act-quant, block 64, of [0, aq_len);
// then the row goes to out + r * ld_out (which may be x).
struct wh_rowpost_args {
    const float* x;
    float* out;
    uint32_t rows, n, ld_in, ld_out;
    uint32_t norm;              // 0: no norm
    const uint16_t* w;          // bf16 [n] or null
    const float* inv_freqs;     // [pairs]
    uint32_t pairs, rope_off, position, inverse;
    uint32_t aq_len;            // 0: no act-quant
    uint32_t tree;              // norm: 1 = the sum of squares in a fixed tree (exact numerics off)
    // several positions in one launch: rows_per_pos > 0 puts row r at
    // position bpos[r / rows_per_pos] (in place of `position`); out_at_pos
    // sends row r to out + bpos[r] * ld_out (one row per position: a KV
    // cache row)
    uint32_t rows_per_pos, out_at_pos;
    uint32_t bpos[WH_POS_BATCH];
    // hc > 0: the row is the end of hc_pre_into (E/compute.rs:5044-5050),
    // y[d] = sum over i in order of hc_pre[r * hc + i] * x[i * hc_stride + d]
    // for the hc copies at x + r * ld_in, instead of x itself
    const float* hc_pre;
    uint32_t hc, hc_stride;
};

// kT threads per row (256, or 1024 for a lone row); each thread's values
// and norm weights are loaded up front.
template <int kT>
__global__ void __launch_bounds__(kT) k_rowpost(wh_rowpost_args a) {
    constexpr int kPer = WH_ROWPOST_MAX / kT;  // values per thread at most
    constexpr int kW = kT / 64;                // waves
    __shared__ __align__(16) float v[WH_ROWPOST_MAX];
    __shared__ float inv_s;
    const uint32_t t = threadIdx.x, n = a.n;
    const float* x = a.x + (size_t)blockIdx.x * a.ld_in;
    uint32_t position = a.position;
    size_t orow = blockIdx.x;
    if (a.rows_per_pos) {
        position = a.bpos[blockIdx.x / a.rows_per_pos];
        if (a.out_at_pos) orow = position;
    }
    float xv[kPer], wv[kPer];
    // every load issued before any is used, from clamped indices (a load
    // under a branch is waited for on its own; with no norm weights the
    // row itself stands in as a valid address)
    const bool use_w = a.norm && a.w;
    const uint16_t* wp = use_w ? a.w : (const uint16_t*)x;
    uint32_t wr[kPer];
    if (a.hc == 4) {
        // the four copies' loads issued together, then the reference's sum
        const float* pre = a.hc_pre + (size_t)blockIdx.x * 4;
        const float p0 = pre[0], p1 = pre[1], p2 = pre[2], p3 = pre[3];
        float cv[4][kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const uint32_t i = t + kT * k, ic = i < n ? i : 0u;
#pragma unroll
            for (int j = 0; j < 4; ++j) cv[j][k] = x[(size_t)j * a.hc_stride + ic];
            wr[k] = wp[ic];
        }
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            float acc = 0.0f;
            acc = acc + p0 * cv[0][k];
            acc = acc + p1 * cv[1][k];
            acc = acc + p2 * cv[2][k];
            acc = acc + p3 * cv[3][k];
            xv[k] = acc;
        }
    } else if (a.hc) {
        const float* pre = a.hc_pre + (size_t)blockIdx.x * a.hc;
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const uint32_t i = t + kT * k, ic = i < n ? i : 0u;
            float acc = 0.0f;
            for (uint32_t j = 0; j < a.hc; ++j) acc = acc + pre[j] * x[(size_t)j * a.hc_stride + ic];
            xv[k] = acc;
            wr[k] = wp[ic];
        }
    } else {
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const uint32_t i = t + kT * k, ic = i < n ? i : 0u;
            xv[k] = x[ic];
            wr[k] = wp[ic];
        }
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const uint32_t i = t + kT * k;
        if (i >= n) xv[k] = 0.0f;
        wv[k] = use_w && i < n ? wh_bf16_value((uint16_t)wr[k]) : 1.0f;
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k)
        if (t + kT * k < n) v[t + kT * k] = xv[k];
    __syncthreads();
    if (a.norm) {
        if (a.tree) {
            // each thread its strided terms, then the wave butterfly, then
            // the waves in order: the same value up to rounding
            __shared__ float red[kW];
            float s = 0.0f;
#pragma unroll
            for (int k = 0; k < kPer; ++k) s = s + xv[k] * xv[k];  // zeros past n
            for (int off = 32; off > 0; off >>= 1) s = s + __shfl_xor(s, off, 64);
            if ((t & 63) == 0) red[t >> 6] = s;
            __syncthreads();
            if (t == 0) {
                float r = red[0];
#pragma unroll
                for (int w = 1; w < kW; ++w) r = r + red[w];
                inv_s = 1.0f / sqrtf(r / (float)n + 1.0e-6f);
            }
        } else {
            // the reference's order: every product rounded on its own in
            // parallel, then one lane adds them in sequence
            __shared__ __align__(16) float sq[WH_ROWPOST_MAX];
#pragma unroll
            for (int k = 0; k < kPer; ++k)
                if (t + kT * k < n) sq[t + kT * k] = xv[k] * xv[k];
            __syncthreads();
            if (t == 0) {
                const float s = wh_ordered_sum_lds(sq, n, 0.0f);
                inv_s = 1.0f / sqrtf(s / (float)n + 1.0e-6f);
            }
        }
        __syncthreads();
        const float inv = inv_s;
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const uint32_t i = t + kT * k;
            if (i < n) {
                float y = xv[k] * inv;
                if (a.w) y = y * wv[k];
                v[i] = y;
            }
        }
        __syncthreads();
    }
    if (a.pairs) {
        const float pos = (float)position;
        for (uint32_t p = t; p < a.pairs; p += kT) {
            const float ang = pos * a.inv_freqs[p];
            float sn = wh_sincosf_glibc(ang, 0);
            const float cs = wh_sincosf_glibc(ang, 1);
            if (a.inverse) sn = -sn;
            float* pv = v + a.rope_off + 2 * p;
            const float e = pv[0], o = pv[1];
            pv[0] = e * cs - o * sn;
            pv[1] = e * sn + o * cs;
        }
        __syncthreads();
    }
    if (a.aq_len) {
        const uint32_t wave = t >> 6, lane = t & 63;
        for (uint32_t b = wave; b * 64 < a.aq_len; b += kW) {
            const uint32_t i = b * 64 + lane;
            const bool valid = i < a.aq_len;
            const float q = wh_aq64_wave(valid ? v[i] : 0.0f, valid);
            if (valid) v[i] = q;
        }
        __syncthreads();
    }
    float* out = a.out + orow * a.ld_out;
    for (uint32_t i = t; i < n; i += kT) out[i] = v[i];
}

// --------------------------------------------------------- window softmax
// Keys of one decode position: the window rows (the KV cache at positions
// [window_start, token_pos], row stride win_ld) then the visible compressed
// rows (head_dim apart), E/compute.rs:4106-4160.
struct wh_attn_args {
    const float* q;        // [heads][head_dim]
    const float* win;      // first window row
    const float* comp;     // compressed rows
    const float* sink;     // [heads] or null
    const float* inv_freqs;
    float* scores;         // [heads][n_keys] scratch
    float* out;            // [heads][head_dim]
    uint32_t heads, head_dim, nope_dim, pairs;
    uint32_t n_win, n_comp, win_ld, token_pos;
    float scale;           // head_dim^-0.5 (host powf, as the reference)
    // a batch of positions (nb > 0): slot z = blockIdx.z takes q and out +
    // z * q_ld, scores + z * scores_ld, token_pos = bpos[z], the window of
    // the last wlen cache rows up to that position (win = the cache's row
    // 0), compressed rows bcomp[z] (bncomp[z] of them)
    uint32_t nb, q_ld, scores_ld, wlen;
    uint32_t wts_ld;       // k_attn_combine: floats per head of its dynamic LDS (>= every n_keys)
    uint32_t bpos[WH_POS_BATCH];
    uint32_t bncomp[WH_POS_BATCH];
    const float* bcomp[WH_POS_BATCH];
};

// One position's keys, queries and outputs.
struct wh_attn_pos {
    const float* q;
    const float* win;
    const float* comp;
    float* scores;
    float* out;
    uint32_t n_win, n_comp, token_pos;
};

__device__ __forceinline__ wh_attn_pos wh_attn_resolve(const wh_attn_args& a) {
    wh_attn_pos v{a.q, a.win, a.comp, a.scores, a.out, a.n_win, a.n_comp, a.token_pos};
    if (a.nb) {
        const uint32_t z = blockIdx.z, p = a.bpos[z], context = p + 1;
        const uint32_t ws = context > a.wlen ? context - a.wlen : 0u;
        v.q = a.q + (size_t)z * a.q_ld;
        v.out = a.out + (size_t)z * a.q_ld;
        v.scores = a.scores + (size_t)z * a.scores_ld;
        v.win = a.win + (size_t)ws * a.win_ld;
        v.n_win = context - ws;
        v.comp = a.bcomp[z];
        v.n_comp = a.bncomp[z];
        v.token_pos = p;
    }
    return v;
}

__device__ __forceinline__ const float* wh_attn_key(const wh_attn_args& a, const wh_attn_pos& v, uint32_t j) {
    return j < v.n_win ? v.win + (size_t)j * a.win_ld : v.comp + (size_t)(j - v.n_win) * a.head_dim;
}

// The q rows of heads h0 .. h0 + 3 into LDS (zeros past the last head):
// every thread's float4 loads are issued before the first store (a load
// inside a loop or under a branch would be waited for one at a time).
__device__ __forceinline__ void wh_attn_stage_q(const wh_attn_args& a, const wh_attn_pos& v, uint32_t h0, float* qs) {
    constexpr int kPer = 4 * WH_ATTN_MAX_HEAD_DIM / 4 / 256;  // float4 per thread at most
    const uint32_t hd = a.head_dim, n4 = hd;                   // 4 * hd floats = hd float4
    float4 qv[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const uint32_t i4 = threadIdx.x + 256 * k, ic = i4 < n4 ? i4 : 0u, e = 4 * ic;
        const uint32_t h = h0 + e / hd, hc = h < a.heads ? h : a.heads - 1;
        qv[k] = *(const float4*)(v.q + (size_t)hc * hd + e % hd);
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const uint32_t i4 = threadIdx.x + 256 * k, e = 4 * i4;
        if (i4 < n4) *(float4*)(qs + e) = h0 + e / hd < a.heads ? qv[k] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

// scores[h][j] = (sum over d, in order, of q[h][d] * key_j[d]) * scale.
// Grid (ceil(n_keys / 64), ceil(heads / 4)), 256 threads: wave w takes
// head 4 * blockIdx.y + w, lane L key 64 * blockIdx.x + L.  Every thread
// requests its share of the 64 keys (16 dims of each 64-dim chunk, up to 8
// chunks) at once, so the launch waits for one memory round trip, not one
// per chunk; the chunks then go through LDS 64 dims at a time (row stride
// 65 floats: the lanes' reads of one dim fall in distinct banks), the four
// heads' q rows once.
#define WH_ATTN_PREFETCH 8u  // 64-dim chunks of a key requested together
__global__ void __launch_bounds__(256) k_attn_scores(wh_attn_args a) {
    __shared__ __align__(16) float qs[4 * WH_ATTN_MAX_HEAD_DIM];
    __shared__ float tile[64 * 65];
    const wh_attn_pos v = wh_attn_resolve(a);
    const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const uint32_t h0 = blockIdx.y * 4, j0 = blockIdx.x * 64;
    const uint32_t nk = v.n_win + v.n_comp, hd = a.head_dim, n_ch = hd / 64;
    if (j0 >= nk) return;  // a batched launch's grid covers its longest key list
    // staging: thread t copies 16 dims (t % 4) of key t / 4 of each chunk
    const uint32_t kk = t >> 2, part = t & 3;
    const bool kon = j0 + kk < nk;
    const float* krow = kon ? wh_attn_key(a, v, j0 + kk) : nullptr;
    float4 kv[WH_ATTN_PREFETCH][4];
    auto request = [&](uint32_t c0) {
#pragma unroll
        for (uint32_t c = 0; c < WH_ATTN_PREFETCH; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                kv[c][i] = kon && c0 + c < n_ch ? *(const float4*)(krow + 64 * (c0 + c) + part * 16 + 4 * i)
                                                : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    request(0);
    wh_attn_stage_q(a, v, h0, qs);
    const float* qrow = qs + wave * hd;
    float s = 0.0f;
    for (uint32_t c0 = 0; c0 < n_ch; c0 += WH_ATTN_PREFETCH) {
        if (c0) request(c0);
#pragma unroll
        for (uint32_t c = 0; c < WH_ATTN_PREFETCH; ++c) {
            if (c0 + c < n_ch) {  // uniform
                __syncthreads();  // the previous chunk's reads are done (and q is staged)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float* d = tile + kk * 65 + part * 16 + 4 * i;
                    d[0] = kv[c][i].x;
                    d[1] = kv[c][i].y;
                    d[2] = kv[c][i].z;
                    d[3] = kv[c][i].w;
                }
                __syncthreads();
                const float* kr = tile + lane * 65;
                const float* qc = qrow + 64 * (c0 + c);
                for (uint32_t d = 0; d < 64; ++d) s = s + qc[d] * kr[d];
            }
        }
    }
    const uint32_t h = h0 + wave, j = j0 + lane;
    if (h < a.heads && j < nk) v.scores[(size_t)h * nk + j] = s * a.scale;
}

// The rest of the window loop for 4 heads x 64 dims per workgroup (grid
// (head_dim / 64, ceil(heads / 4)), 256 threads, 4 * wts_ld floats of
// dynamic LDS; wave w = head, lane = dim):
//   max = the largest score (NaN scores never win, E/compute.rs:4125-4127);
//   w_j = expf(score_j - max); denom = expf(sink - max) (if a sink) +
//   (sequential sum of w_j); out_d = sequential sum of w_j * key_j[d] from 0;
//   out_d /= denom when denom > 0; then the inverse RoPE of the output's
//   rope dims at token_pos (E/compute.rs:4160-4197).
// The keys' 64 dims of the workgroup go through LDS 128 keys at a time,
// staged once for the four heads; the first 128 are requested before the
// softmax pass.
#define WH_ATTN_KCHUNK 128u
__global__ void __launch_bounds__(256) k_attn_combine(wh_attn_args a) {
    extern __shared__ __align__(16) float wts[];  // [4][wts_ld], wts_ld a multiple of 4
    __shared__ __align__(16) float tile[WH_ATTN_KCHUNK * 64];
    __shared__ float res[4 * 64];
    __shared__ float denom_s[4];
    const wh_attn_pos v = wh_attn_resolve(a);
    const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const uint32_t h = blockIdx.y * 4 + wave, d = blockIdx.x * 64 + lane;
    const uint32_t nk = v.n_win + v.n_comp;
    const bool hon = h < a.heads;
    // staging: thread t copies dims 32 (t % 2) .. + 31 of key t / 2 of the chunk
    const uint32_t kk = t >> 1, half = t & 1;
    float4 kr[8];
    auto request = [&](uint32_t c0) {
        const bool on = c0 + kk < nk;
        const float* src = on ? wh_attn_key(a, v, c0 + kk) + blockIdx.x * 64 + 32 * half : nullptr;
#pragma unroll
        for (int i = 0; i < 8; ++i) kr[i] = on ? *(const float4*)(src + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    request(0);
    float* w = wts + wave * a.wts_ld;
    const float* sc = v.scores + (size_t)(hon ? h : 0) * nk;
    float mx = -__uint_as_float(0x7f800000u);
    uint32_t j = lane;
    // four scores' loads at a time (sc is a valid row for every wave)
    for (; j + 192 < nk; j += 256) {
        float sv[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) sv[k] = sc[j + 64 * k];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float x = hon ? sv[k] : 0.0f;
            w[j + 64 * k] = x;
            mx = fmaxf(mx, x);
        }
    }
    if (j + 64 < nk) {
        const float s0 = sc[j], s1 = sc[j + 64];
        const float x0 = hon ? s0 : 0.0f, x1 = hon ? s1 : 0.0f;
        w[j] = x0;
        w[j + 64] = x1;
        mx = fmaxf(fmaxf(mx, x0), x1);
        j += 128;
    }
    for (; j < nk; j += 64) {
        const float x = hon ? sc[j] : 0.0f;
        w[j] = x;
        mx = fmaxf(mx, x);
    }
    mx = wh_wave_max(mx);
    for (uint32_t j = lane; j < nk; j += 64) w[j] = wh_expf_glibc(w[j] - mx, kExpTab, kExpfExc, WH_EXPF_EXC_COUNT);
    __syncthreads();
    if (lane == 0) {
        const float ws = wh_ordered_sum_lds(w, nk, 0.0f);
        float den = 0.0f;
        if (a.sink && hon) den = den + wh_expf_glibc(a.sink[h] - mx, kExpTab, kExpfExc, WH_EXPF_EXC_COUNT);
        denom_s[wave] = den + ws;
    }
    float acc = 0.0f;
    for (uint32_t c0 = 0; c0 < nk; c0 += WH_ATTN_KCHUNK) {
        if (c0) {
            __syncthreads();  // the previous chunk's reads are done
            request(c0);
        }
        float* dst = tile + kk * 64 + 32 * half;
#pragma unroll
        for (int i = 0; i < 8; ++i) *(float4*)(dst + 4 * i) = kr[i];
        __syncthreads();
        const uint32_t m = min(WH_ATTN_KCHUNK, nk - c0);
        if (hon) {
            // blocks of 16 keys: the weights (broadcast) and the lane's 16
            // key values of the next block are read while the current block
            // is added; a full chunk is straight-line code, in which the
            // compiler counts the reads in flight exactly
            const float* wc = w + c0;
            float4 wa[2][4];
            float ta[2][16];
            auto rdb = [&](int sl, uint32_t jb) {
#pragma unroll
                for (int i = 0; i < 4; ++i) wa[sl][i] = *(const float4*)(wc + 16 * jb + 4 * i);
#pragma unroll
                for (int i = 0; i < 16; ++i) ta[sl][i] = tile[(16 * jb + i) * 64 + lane];
            };
            auto addb = [&](int sl) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    acc = acc + wa[sl][i].x * ta[sl][4 * i];
                    acc = acc + wa[sl][i].y * ta[sl][4 * i + 1];
                    acc = acc + wa[sl][i].z * ta[sl][4 * i + 2];
                    acc = acc + wa[sl][i].w * ta[sl][4 * i + 3];
                }
            };
            const uint32_t mb = m / 16;
            if (mb == WH_ATTN_KCHUNK / 16) {
                rdb(0, 0);
#pragma unroll
                for (int b = 0; b < (int)(WH_ATTN_KCHUNK / 16); ++b) {
                    if (b + 1 < (int)(WH_ATTN_KCHUNK / 16)) rdb((b + 1) & 1, b + 1);
                    __builtin_amdgcn_sched_barrier(0);
                    addb(b & 1);
                    __builtin_amdgcn_sched_barrier(0);
                }
            } else {
                for (uint32_t b = 0; b < mb; ++b) {
                    rdb(0, b);
                    addb(0);
                }
            }
            for (uint32_t j = 16 * mb; j < m; ++j) acc = acc + wc[j] * tile[j * 64 + lane];
        }
    }
    __syncthreads();
    const float den = denom_s[wave];
    if (den > 0.0f) acc = acc / den;
    res[wave * 64 + lane] = acc;
    __syncthreads();
    // inverse RoPE: the even lane of a pair in [nope_dim, head_dim) rotates it
    if (d >= a.nope_dim && ((d - a.nope_dim) & 1) == 0 && (d - a.nope_dim) / 2 < a.pairs) {
        const uint32_t p = (d - a.nope_dim) / 2;
        const float ang = (float)v.token_pos * a.inv_freqs[p];
        const float sn = -wh_sincosf_glibc(ang, 0);
        const float cs = wh_sincosf_glibc(ang, 1);
        const float e = res[wave * 64 + lane], o = res[wave * 64 + lane + 1];
        res[wave * 64 + lane] = e * cs - o * sn;
        res[wave * 64 + lane + 1] = e * sn + o * cs;
    }
    __syncthreads();
    if (hon) v.out[(size_t)h * a.head_dim + d] = res[wave * 64 + lane];
}
