// Persistent MFMA kernels of the batch path: the experts the pack put on
// MFMA items (E/compute.rs:1779-1810 computes every expert's slots with the
// reference's AVX2 kernel; here the summation order is freed, as in
// moe_px.h, and each matvec stays within 1e-5 * ||w_row||_2 * ||x||_2).
//
// Work: an MFMA expert with T slots is ceil(T / 16) virtual experts of at
// most 16 slots, one MFMA N-tile each; the pack lists them (vtab, in work
// order, meta[7] of them) with their matrices, so a workgroup reaches its
// first weight load after two dependent reads.  An item is (virtual expert,
// 16-row tile, matrix): 2 x inter / 16 items per virtual expert for gate/up
// (w1, w3), hidden / 16 for down (w2).  One workgroup of 512 threads per CU
// takes an equal contiguous range of the items (equal weight bytes and
// MFMA counts); its waves take the range's items on demand from an LDS
// counter, so a wave that streams faster takes more of them.  An item
// streams its 16 rows' whole width through the wave's register ring
// (WH_BMX_DEPTH blocks of 256 columns in flight, the ring running on across
// items) and stores its 16 x 16 output tile itself: no workgroup barrier
// inside the stream and no cross-wave reduction.  The B operands - the code
// records of a virtual expert's slots (x's act-quant for gate/up, h's for
// down) - are staged in LDS once per workgroup: a range of at most 256 x 256
// items touches at most two virtual experts, so one staging serves the whole
// launch unless there are more than 256 of them (then the range goes in
// phases of two).
#pragma once
#include "moe_px.h"

#ifndef WH_BMX_DEPTH
#define WH_BMX_DEPTH 5  // weight blocks of a wave in flight
#endif
#define WH_BMX_TOK 16u                             // slots per virtual expert

// LDS of one staged virtual expert over `cols` input columns: 16 code
// records of cols bytes + 16 of padding (slot n at n * (cols + 16)), then
// the 16 slots' E8M0 bytes (cols / 32 each).
__host__ __device__ constexpr size_t wh_bmx_buf(size_t cols) {
    return WH_BMX_TOK * (cols + 16) + WH_BMX_TOK * (cols / 32);
}
// Two staged virtual experts.
__host__ __device__ constexpr size_t wh_bmx_lds(size_t cols) { return 2 * wh_bmx_buf(cols); }

// A value every lane of the wave holds alike, moved to scalar registers.
__device__ __forceinline__ uint32_t wh_uni(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ const uint8_t* wh_uni(const uint8_t* p) {
    const uint64_t v = (uint64_t)p;
    return (const uint8_t*)(((uint64_t)wh_uni((uint32_t)(v >> 32)) << 32) | wh_uni((uint32_t)v));
}

// Loads through pointers the compiler cannot place in an address space (read
// back from LDS) come out as flat loads, which count against the LDS counter
// too: every LDS read of the B operands would then wait for the whole weight
// ring.  These take the global address space explicitly (through vector
// types: through HIP's struct uint4 the address space is lost again).
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

// Gate/up of the MFMA experts in fp32, for a batch with an inf or NaN input
// (-480, a NaN's act-quantized value, has no E4M3 code and an infinite scale
// no E8M0 byte) when no exact-item kernel follows: the workgroup's items
// [i0, i1) from the dequantized inputs, one wave per item and every slot of
// the item's virtual expert in turn (wh_px_rows_fp32).  The products are
// exact in fp32; only the order of the sums differs from the reference's.
template <int kCols>
__device__ void wh_bmx_gate_fp32(const wh_batch_args& a, uint32_t i0, uint32_t i1, uint32_t per_v, uint32_t wave,
                                 uint32_t L) {
    constexpr uint32_t NB = kCols / 256, G = kCols / 32;
#pragma unroll 1
    for (uint32_t it = i0 + wave; it < i1; it += 8) {
        const uint32_t v = it / per_v, rel = it - v * per_v, tile = rel >> 1, m = rel & 1;
        const wh_bmx_vt* vt = a.vtab + v;
        const uint32_t row = tile * 16 + (L & 15);
        const uint8_t* wrow = (m ? vt->w3 : vt->w1) + (size_t)row * (kCols / 2);
        const uint8_t* srow = (m ? vt->s3 : vt->s1) + (size_t)row * G;
        const uint32_t slot0 = vt->slot0, count = vt->count;
        float* dst = m ? a.u : a.g;
#pragma unroll 1
        for (uint32_t n = 0; n < count; ++n) {
            const uint32_t s = slot0 + n;
            const float r = wh_px_rows_fp32(wrow, srow, a.xq + (size_t)a.pos[s] * kCols, 0, NB, L);
            if (L < 16) {
                dst[(size_t)s * a.inter + tile * 16 + L] = r;
                if (!(fabsf(r) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
            }
        }
    }
}

// kGate: gate/up (kCols = hidden, B = x's codes by position, out g / u);
// else down (kCols = inter, B = h's codes by slot, out y).  inter = 2048.
// Grid: one workgroup of 512 threads per CU.
template <int kCols, bool kGate>
__global__ void __launch_bounds__(512, 1) k_moe_batch_mx(wh_batch_args a) {
    extern __shared__ __align__(16) float lds_f[];
    uint8_t* const lds = (uint8_t*)lds_f;
    __shared__ wh_bmx_vt vm[2];
    __shared__ const uint8_t* srcp[2 * WH_BMX_TOK];  // code record of each staged slot
    __shared__ const uint8_t* srcs[2 * WH_BMX_TOK];  // its E8M0 bytes
    __shared__ uint32_t next_item;                   // the phase's next item for a wave
    constexpr uint32_t NB = kCols / 256, G = kCols / 32, TS = kCols + 16;
    constexpr uint32_t BUF = (uint32_t)wh_bmx_buf(kCols);
    constexpr uint32_t CPS = kCols / 16;  // 16-byte pieces of a code record
    constexpr int D = WH_BMX_DEPTH;
    static_assert(NB == 8 || NB == 16, "2048 or 4096 columns");
    static_assert(D < (int)NB, "the ring spans at most two items");
    // timeline points (builds with -DWH_TIMELINE): 0 start, 1 ring issued,
    // 2 B staged, 3 the wave's last item done, 4 the workgroup's end
    WH_TL(kGate ? 0 : 1, 0);
    // an inf or NaN input: every expert on the exact items, or with
    // mx_fallback gate/up in fp32 here (h is then finite, or the batch has
    // already failed with a non-finite g or u, so down stays on MFMA)
    const bool nonfinite = a.meta[6] != 0;
    if (nonfinite && !a.mx_fallback) return;
    const uint32_t V = a.meta[7];
    if (V == 0 || a.meta[1] == 0) return;
    const uint32_t tid = threadIdx.x, wave = tid >> 6, L = tid & 63, g = L >> 4, nl = L & 15;
    const uint32_t tiles = (kGate ? a.inter : a.hidden) >> 4;
    const uint32_t per_v = kGate ? 2 * tiles : tiles;
    const uint64_t W = (uint64_t)V * per_v;
    const uint32_t i0 = (uint32_t)(W * blockIdx.x / gridDim.x), i1 = (uint32_t)(W * (blockIdx.x + 1) / gridDim.x);
    if (i0 >= i1) return;
    if constexpr (kGate) {
        if (nonfinite) {
            wh_bmx_gate_fp32<kCols>(a, i0, i1, per_v, wave, L);
            return;
        }
    }
    const uint32_t lane_off = 64 * (g & 1) + 32 * (g >> 1);
    for (uint32_t vp = i0 / per_v, v_last = (i1 - 1) / per_v; vp <= v_last; vp += 2) {
        const uint32_t nv = v_last - vp + 1 < 2 ? v_last - vp + 1 : 2;
        // the phase's items [ps, pe): virtual experts vp, vp + 1
        const uint32_t ps = i0 > vp * per_v ? i0 : vp * per_v;
        const uint32_t pe = i1 < (vp + nv) * per_v ? i1 : (vp + nv) * per_v;
        if (tid < nv) vm[tid] = a.vtab[vp + tid];
        if (tid == 0) next_item = ps + 8;  // items ps .. ps + 7 start the waves
        __syncthreads();
        // the two virtual experts in scalar registers, field by field (a
        // struct copy or a run-time indexed array would go through scratch)
        const uint32_t x1 = nv > 1 ? 1 : 0;
        const uint8_t* w0a = wh_uni(kGate ? vm[0].w1 : vm[0].w2);
        const uint8_t* w0b = wh_uni(kGate ? vm[0].w3 : vm[0].w2);
        const uint8_t* s0a = wh_uni(kGate ? vm[0].s1 : vm[0].s2);
        const uint8_t* s0b = wh_uni(kGate ? vm[0].s3 : vm[0].s2);
        const uint8_t* w1a = wh_uni(kGate ? vm[x1].w1 : vm[x1].w2);
        const uint8_t* w1b = wh_uni(kGate ? vm[x1].w3 : vm[x1].w2);
        const uint8_t* s1a = wh_uni(kGate ? vm[x1].s1 : vm[x1].s2);
        const uint8_t* s1b = wh_uni(kGate ? vm[x1].s3 : vm[x1].s2);
        const uint32_t slot0_0 = wh_uni(vm[0].slot0), slot0_1 = wh_uni(vm[x1].slot0);
        const uint32_t cnt0 = wh_uni(vm[0].count), cnt1 = wh_uni(vm[x1].count);
        // item it: virtual expert vp + q, row tile `tile`, matrix m
#define WH_BMX_ITEM(it, q, tile, m)                                                \
    const uint32_t rel_##q = (it) - vp * per_v;                                    \
    const uint32_t q = rel_##q >= per_v;                                           \
    const uint32_t tile = kGate ? (rel_##q - q * per_v) >> 1 : rel_##q - q * per_v; \
    const uint32_t m = kGate ? (rel_##q - q * per_v) & 1 : 0
        // issue side of the ring: block iss_blk of item iss_it; past the
        // wave's last item every step repeats the last block issued (its
        // result is not used), so each step issues the same three loads and
        // the waits stay vmcnt(3 (D - 1)) rather than vmcnt(0)
        uint32_t iss_it = wh_uni(ps + wave), iss_blk = 0, nxt_it = iss_it;
        const uint8_t* iw = w0a;
        const uint8_t* is = s0a;
        uint32_t ib = 0;
#define WH_BMX_ISSUE(rg, dep)                                                                            \
    do {                                                                                                 \
        if (iss_it < pe) {                                                                               \
            WH_BMX_ITEM(iss_it, iq, itile, im);                                                          \
            const uint32_t irow = itile * 16 + nl;                                                       \
            iw = (iq ? (im ? w1b : w1a) : (im ? w0b : w0a)) + (size_t)irow * (kCols / 2) + lane_off;      \
            is = (iq ? (im ? s1b : s1a) : (im ? s0b : s0a)) + (size_t)irow * G;                          \
            ib = iss_blk;                                                                                \
            if (++iss_blk == NB) {                                                                       \
                iss_blk = 0;                                                                             \
                uint32_t nx = 0;                                                                         \
                if (L == 0) nx = atomicAdd(&next_item, 1u);                                              \
                iss_it = nxt_it = wh_uni((uint32_t)__shfl(nx, 0, 64));                                   \
            }                                                                                            \
        }                                                                                                \
        wh_mx_raw_load_global(rg, iw + (dep), is + (dep), ib);                                           \
    } while (0)
        wh_mx_raw ring[D];
        if (iss_it < pe) {
#pragma unroll
            for (int d = 0; d < D; ++d) WH_BMX_ISSUE(ring[d], 0u);
        }
        __builtin_amdgcn_sched_barrier(0);
        WH_TL(kGate ? 0 : 1, 1);
        // where each staged slot's codes come from
        if (tid < nv * WH_BMX_TOK) {
            const uint32_t q = tid / WH_BMX_TOK, n = tid % WH_BMX_TOK;
            const uint32_t c = q ? cnt1 : cnt0;
            const uint32_t s = (q ? slot0_1 : slot0_0) + (n < c ? n : 0);
            const size_t r = kGate ? a.pos[s] : s;
            srcp[tid] = (kGate ? a.xq8 : a.hq8) + r * kCols;
            srcs[tid] = (kGate ? a.xs8 : a.hs8) + r * G;
        }
        __syncthreads();
        // B staging (codes: CPS pieces per slot, then the E8M0 bytes: G / 16)
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
        WH_TL(kGate ? 0 : 1, 2);
        // consume side: block cur_blk of item cur_it
        uint32_t cur_it = wh_uni(ps + wave), cur_blk = 0;
        uint32_t dep = wh_opaque_zero(__uint_as_float(*(const uint32_t*)lds));
        wh_v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
        bool nf = false;
        while (cur_it < pe) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                if (cur_it >= pe) break;
                WH_BMX_ITEM(cur_it, q, tile, m);
                const uint8_t* buf = lds + q * BUF;
                wh_mx_bop bo;
                wh_mx_bop_load(bo, buf + nl * TS + 256 * cur_blk + dep,
                               buf + WH_BMX_TOK * TS + nl * G + 8 * cur_blk + dep, g);
                wh_px_step(acc, ring[d], dep, bo, g);
                WH_BMX_ISSUE(ring[d], dep);
                if (++cur_blk == NB) {
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
                    cur_blk = 0;
                    cur_it = nxt_it;
                }
            }
        }
#undef WH_BMX_ISSUE
#undef WH_BMX_ITEM
        WH_TL(kGate ? 0 : 1, 3);
        if (nf) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
        __syncthreads();  // the phase's buffers and counter are free
    }
    WH_TL(kGate ? 0 : 1, 4);
}
