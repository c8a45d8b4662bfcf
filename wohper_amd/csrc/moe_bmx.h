// Persistent MFMA kernels of the batch path: the experts the pack put on
// MFMA items (E/compute.rs:1779-1810 computes every expert's slots with the
// reference's AVX2 kernel; here the summation order is freed, as in
// moe_px.h, and each matvec stays within 1e-5 * ||w_row||_2 * ||x||_2).
//
// Work: an MFMA expert with T slots is ceil(T / 16) virtual experts of at
// most 16 slots, one MFMA N-tile each.  An item is (virtual expert, 16-row
// tile, matrix): 2 x inter / 16 items per virtual expert for gate/up (w1,
// w3), hidden / 16 for down (w2).  One workgroup of 512 threads per CU takes
// an equal contiguous range of the items (equal weight bytes and equal MFMA
// counts: the balance a work queue would give, without its atomics); wave w
// takes items w, w + 8, ... of it.  An item streams its 16 rows' whole width
// through the wave's register ring (WH_BMX_DEPTH blocks of 256 columns in
// flight, the ring running on across items) and stores its 16 x 16 output
// tile itself: no workgroup barrier inside the stream and no cross-wave
// reduction.  The B operands - the code records of a virtual expert's slots
// (x's act-quant for gate/up, h's for down) - are staged in LDS once per
// workgroup: a range of at most 256 x 256 items touches at most two virtual
// experts, so one staging serves the whole launch unless there are more
// than 256 of them (then the range goes in phases of two).
#pragma once
#include "moe_px.h"

#ifndef WH_BMX_DEPTH
#define WH_BMX_DEPTH 6  // weight blocks of a wave in flight
#endif
#define WH_BMX_TOK 16u                             // slots per virtual expert
#define WH_BMX_MAX_EXPERTS (WH_BATCH_MAX_TABLE + 1)  // used experts of a pack (the shared one included)

// LDS of one staged virtual expert over `cols` input columns: 16 code
// records of cols bytes + 16 of padding (slot n at n * (cols + 16)), then
// the 16 slots' E8M0 bytes (cols / 32 each).
__host__ __device__ constexpr size_t wh_bmx_buf(size_t cols) {
    return WH_BMX_TOK * (cols + 16) + WH_BMX_TOK * (cols / 32);
}
// Two staged virtual experts and the virtual-expert prefix of the MFMA
// experts.
__host__ __device__ constexpr size_t wh_bmx_lds(size_t cols) {
    return 2 * wh_bmx_buf(cols) + 4 * (WH_BMX_MAX_EXPERTS + 1);
}

// Exclusive prefix sum over the workgroup (any multiple of 64 threads up to
// 1024); `tot` holds 16 words.
__device__ __forceinline__ uint32_t wh_wg_scan_any(uint32_t v, uint32_t* tot, uint32_t* total) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    uint32_t incl = v;
    for (uint32_t off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(incl, off, 64);
        if (lane >= off) incl += y;
    }
    if (lane == 63) tot[wave] = incl;
    __syncthreads();
    uint32_t before = 0, all = 0;
    for (uint32_t w = 0; w < nw; ++w) {
        before += w < wave ? tot[w] : 0u;
        all += tot[w];
    }
    *total = all;
    __syncthreads();
    return before + incl - v;
}

// Loads through pointers the compiler cannot place in an address space (read
// back from LDS) come out as flat loads, which count against the LDS counter
// too: every LDS read of the B operands would then wait for the whole weight
// ring.  These take the global address space explicitly.
// (The vector types matter: through HIP's struct uint4 the address space is
// lost again.)
#define WH_GLOBAL __attribute__((address_space(1)))
typedef unsigned int wh_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int wh_u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 wh_ld16_global(const void* p) {
    const wh_u32x4 v = *(const WH_GLOBAL wh_u32x4*)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 wh_ld8_global(const void* p) {
    const wh_u32x2 v = *(const WH_GLOBAL wh_u32x2*)p;
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ void wh_mx_raw_load_global(wh_mx_raw& r, const uint8_t* wlane, const uint8_t* srow,
                                                      uint32_t blk) {
    r.p = wh_ld16_global(wlane + blk * 128);
    r.q = wh_ld16_global(wlane + blk * 128 + 16);
    r.s = wh_ld8_global(srow + blk * 8);
}

// A value every lane of the wave holds alike, moved to scalar registers.
__device__ __forceinline__ uint32_t wh_uni(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ const uint8_t* wh_uni(const uint8_t* p) {
    const uint64_t v = (uint64_t)p;
    return (const uint8_t*)(((uint64_t)wh_uni((uint32_t)(v >> 32)) << 32) | wh_uni((uint32_t)v));
}

// A staged virtual expert: its matrices (gate/up: w1, w3; down: w2 twice),
// its first slot and its slot count (<= 16).
struct wh_bmx_v {
    const uint8_t *wa, *wb;  // matrices 0 and 1
    const uint8_t *sa, *sb;  // their scales
    uint32_t slot0, count;
};

// kGate: gate/up (kCols = hidden, B = x's codes by position, out g / u);
// else down (kCols = inter, B = h's codes by slot, out y).  inter = 2048.
// Grid: one workgroup of 512 threads per CU.
template <int kCols, bool kGate>
__global__ void __launch_bounds__(512, 1) k_moe_batch_mx(wh_batch_args a) {
    extern __shared__ __align__(16) float lds_f[];
    uint8_t* const lds = (uint8_t*)lds_f;
    __shared__ uint32_t tot[16];
    __shared__ wh_bmx_v vm[2];
    __shared__ const uint8_t* srcp[2 * WH_BMX_TOK];  // code record of each staged slot
    __shared__ const uint8_t* srcs[2 * WH_BMX_TOK];  // its E8M0 bytes
    constexpr uint32_t NB = kCols / 256, G = kCols / 32, TS = kCols + 16;
    constexpr uint32_t BUF = (uint32_t)wh_bmx_buf(kCols);
    constexpr uint32_t CPS = kCols / 16;  // 16-byte pieces of a code record
    constexpr int D = WH_BMX_DEPTH;
    static_assert(NB == 8 || NB == 16, "2048 or 4096 columns");
    uint32_t* vstart = (uint32_t*)(lds + 2 * BUF);
    const uint32_t n_mfma = a.meta[4];
    if (n_mfma == 0 || a.meta[1] == 0) return;
    const uint32_t tid = threadIdx.x, wave = tid >> 6, L = tid & 63, g = L >> 4, nl = L & 15;
    const uint32_t tiles = (kGate ? a.inter : a.hidden) >> 4;
    const uint32_t per_v = kGate ? 2 * tiles : tiles;
    // virtual experts: MFMA expert i of the work order (most slots first)
    // is vstart[i] .. vstart[i + 1] - 1
    {
        constexpr uint32_t K = (WH_BMX_MAX_EXPERTS + 511) / 512;
        uint32_t c[K], sum = 0;
#pragma unroll
        for (uint32_t k = 0; k < K; ++k) {
            const uint32_t i = tid * K + k;
            c[k] = 0;
            if (i < n_mfma) {
                const uint32_t ue = a.uorder[i];
                c[k] = (a.uoff[ue + 1] - a.uoff[ue] + WH_BMX_TOK - 1) / WH_BMX_TOK;
            }
            sum += c[k];
        }
        uint32_t total;
        uint32_t pre = wh_wg_scan_any(sum, tot, &total);
#pragma unroll
        for (uint32_t k = 0; k < K; ++k) {
            const uint32_t i = tid * K + k;
            if (i < n_mfma) vstart[i] = pre;
            pre += c[k];
        }
        if (tid == 0) vstart[n_mfma] = total;
        __syncthreads();
    }
    const uint32_t V = vstart[n_mfma];
    const uint64_t W = (uint64_t)V * per_v;
    const uint32_t i0 = (uint32_t)(W * blockIdx.x / gridDim.x), i1 = (uint32_t)(W * (blockIdx.x + 1) / gridDim.x);
    if (i0 >= i1) return;
    const uint32_t lane_off = 64 * (g & 1) + 32 * (g >> 1);
    for (uint32_t vp = i0 / per_v, v_last = (i1 - 1) / per_v; vp <= v_last; vp += 2) {
        const uint32_t nv = v_last - vp + 1 < 2 ? v_last - vp + 1 : 2;
        // the phase's virtual experts
        if (tid < nv) {
            const uint32_t v = vp + tid;
            uint32_t lo = 0, hi = n_mfma - 1;  // the last i with vstart[i] <= v
            while (lo < hi) {
                const uint32_t mid = (lo + hi + 1) >> 1;
                if (vstart[mid] <= v) lo = mid;
                else hi = mid - 1;
            }
            const uint32_t ue = a.uorder[lo];
            const uint32_t s0 = a.uoff[ue] + WH_BMX_TOK * (v - vstart[lo]), end = a.uoff[ue + 1];
            const wh_expert_ptrs ep = wh_batch_expert(a, a.uexp[ue]);
            vm[tid].wa = kGate ? ep.w1 : ep.w2;
            vm[tid].sa = kGate ? ep.s1 : ep.s2;
            vm[tid].wb = kGate ? ep.w3 : ep.w2;
            vm[tid].sb = kGate ? ep.s3 : ep.s2;
            vm[tid].slot0 = s0;
            vm[tid].count = end - s0 < WH_BMX_TOK ? end - s0 : WH_BMX_TOK;
        }
        __syncthreads();
        // where each staged slot's codes come from
        if (tid < nv * WH_BMX_TOK) {
            const uint32_t q = tid / WH_BMX_TOK, n = tid % WH_BMX_TOK;
            const uint32_t s = vm[q].slot0 + (n < vm[q].count ? n : 0);
            size_t r;
            if constexpr (kGate) r = wh_slot_pos(a, a.sorted[s]);
            else r = s;
            srcp[tid] = (kGate ? a.xq8 : a.hq8) + r * kCols;
            srcs[tid] = (kGate ? a.xs8 : a.hs8) + r * G;
        }
        __syncthreads();
        // the two virtual experts in registers, picked field by field (an
        // array indexed at run time would live in scratch memory)
        // (a copy of the struct itself goes through scratch memory)
        const uint32_t x1 = nv > 1 ? 1 : 0;
        const uint8_t *w0a = wh_uni(vm[0].wa), *w0b = wh_uni(vm[0].wb), *s0a = wh_uni(vm[0].sa),
                      *s0b = wh_uni(vm[0].sb);
        const uint8_t *w1a = wh_uni(vm[x1].wa), *w1b = wh_uni(vm[x1].wb), *s1a = wh_uni(vm[x1].sa),
                      *s1b = wh_uni(vm[x1].sb);
        const uint32_t slot0_0 = wh_uni(vm[0].slot0), slot0_1 = wh_uni(vm[x1].slot0), cnt0 = wh_uni(vm[0].count),
                       cnt1 = wh_uni(vm[x1].count);
        // B staging loads (codes: kCols pieces per virtual expert, then the
        // E8M0 bytes: G pieces), issued before this wave's first weight loads
        constexpr uint32_t KB = (2 * WH_BMX_TOK * CPS + 511) / 512, KS = (2 * WH_BMX_TOK * G / 16 + 511) / 512;
        uint4 bst[KB], sst[KS];
#pragma unroll
        for (uint32_t k = 0; k < KB; ++k) {
            const uint32_t f = tid + 512 * k, q = f / (WH_BMX_TOK * CPS), n = (f / CPS) % WH_BMX_TOK, c = f % CPS;
            if (q < nv && n < (q ? cnt1 : cnt0)) bst[k] = wh_ld16_global(srcp[q * WH_BMX_TOK + n] + 16 * c);
        }
#pragma unroll
        for (uint32_t k = 0; k < KS; ++k) {
            const uint32_t f = tid + 512 * k, q = f / (WH_BMX_TOK * G / 16), n = (f / (G / 16)) % WH_BMX_TOK,
                           c = f % (G / 16);
            if (q < nv && n < (q ? cnt1 : cnt0)) sst[k] = wh_ld16_global(srcs[q * WH_BMX_TOK + n] + 16 * c);
        }
        // this wave's items of the phase and their blocks
        const uint32_t ps = i0 > vp * per_v ? i0 : vp * per_v;
        const uint32_t pe = i1 < (vp + nv) * per_v ? i1 : (vp + nv) * per_v;
        const uint32_t it0 = wh_uni(ps + wave);
        const uint32_t n_items = it0 < pe ? (pe - it0 + 7) / 8 : 0;
        const uint32_t J = n_items * NB;
        // block j of the wave: item it0 + 8 (j / NB) = virtual expert vp + q,
        // row tile `tile`, matrix m; column block j % NB
#define WH_BMX_ITEM(j, q, tile, m)                                    \
    const uint32_t it_##q = it0 + 8 * ((j) / NB) - vp * per_v;        \
    const uint32_t q = it_##q >= per_v;                               \
    const uint32_t tile = kGate ? (it_##q - q * per_v) >> 1 : it_##q - q * per_v; \
    const uint32_t m = kGate ? (it_##q - q * per_v) & 1 : 0
#define WH_BMX_ISSUE(rg, j, dep)                                                                          \
    do {                                                                                                  \
        WH_BMX_ITEM(j, iq, itile, im);                                                                    \
        const uint32_t irow = itile * 16 + nl;                                                            \
        const uint8_t* iw = iq ? (im ? w1b : w1a) : (im ? w0b : w0a);                                     \
        const uint8_t* is = iq ? (im ? s1b : s1a) : (im ? s0b : s0a);                                     \
        wh_mx_raw_load_global(rg, iw + (size_t)irow * (kCols / 2) + lane_off + (dep), is + (size_t)irow * G + (dep), \
                              (j) % NB);                                                                  \
    } while (0)
        // every step of the ring issues its loads (past the end it repeats
        // the last block, whose result is not stored), so the count of loads
        // in flight is the same at every step and the compiler's waits are
        // vmcnt(3 (D - 1)), not vmcnt(0)
        const uint32_t Jl = J ? J - 1 : 0;
        wh_mx_raw ring[D];
        if (J) {
#pragma unroll
            for (int d = 0; d < D; ++d) WH_BMX_ISSUE(ring[d], (uint32_t)d < Jl ? (uint32_t)d : Jl, 0u);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (uint32_t k = 0; k < KB; ++k) {
            const uint32_t f = tid + 512 * k, q = f / (WH_BMX_TOK * CPS), n = (f / CPS) % WH_BMX_TOK, c = f % CPS;
            if (q < nv && n < (q ? cnt1 : cnt0)) *(uint4*)(lds + q * BUF + n * TS + 16 * c) = bst[k];
        }
#pragma unroll
        for (uint32_t k = 0; k < KS; ++k) {
            const uint32_t f = tid + 512 * k, q = f / (WH_BMX_TOK * G / 16), n = (f / (G / 16)) % WH_BMX_TOK,
                           c = f % (G / 16);
            if (q < nv && n < (q ? cnt1 : cnt0))
                *(uint4*)(lds + q * BUF + WH_BMX_TOK * TS + n * G + 16 * c) = sst[k];
        }
        __syncthreads();
        uint32_t dep = wh_opaque_zero(__uint_as_float(*(const uint32_t*)lds));
        wh_v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
        bool nf = false;
        for (uint32_t j0 = 0; j0 < J; j0 += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const uint32_t j = j0 + d < Jl ? j0 + d : Jl;
                {
                    WH_BMX_ITEM(j, q, tile, m);
                    const uint32_t blk = j % NB;
                    const uint8_t* buf = lds + q * BUF;
                    wh_mx_bop bo;
                    wh_mx_bop_load(bo, buf + nl * TS + 256 * blk + dep, buf + WH_BMX_TOK * TS + nl * G + 8 * blk + dep, g);
                    wh_px_step(acc, ring[d], dep, bo, g);
                    WH_BMX_ISSUE(ring[d], j + D < Jl ? j + D : Jl, dep);
                    if (blk == NB - 1 && j0 + d < J) {
                        // C[4 (L / 16) + r][L % 16]: rows of the tile, slot nl
                        asm volatile("" : "+v"(acc));
                        if (nl < (q ? cnt1 : cnt0)) {
                            float o[4];
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                o[r] = acc[r] + 0.0f;
                                nf = nf || !(fabsf(o[r]) <= 3.4028235e38f);
                            }
                            float* dst = kGate ? (m ? a.u : a.g) : a.y;
                            const uint32_t ld = kGate ? a.inter : a.hidden;
                            *(float4*)(dst + (size_t)((q ? slot0_1 : slot0_0) + nl) * ld + tile * 16 + 4 * g) =
                                make_float4(o[0], o[1], o[2], o[3]);
                        }
                        acc = wh_v4f{0.0f, 0.0f, 0.0f, 0.0f};
                    }
                }
            }
        }
#undef WH_BMX_ISSUE
#undef WH_BMX_ITEM
        if (nf) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
        __syncthreads();  // the phase's buffers are free
    }
}
