// Routed-expert token kernels that stream their weights straight into LDS
// (gfx950 global_load_lds_dwordx4): the MFMA-numerics path of the token
// entry points for hidden 4096, inter 2048.
//
// Same arithmetic as k_moe_gateup_px / k_moe_down_px (moe_px.h): the FP4
// weights become E4M3 codes of the reference's x8 LUT integers and meet the
// act-quantized input (E/compute.rs:2504-2521) in
// v_mfma_scale_f32_16x16x128_f8f6f4, so only the fp32 summation order
// differs from the CPU kernel (E/deepseek_v4.rs:551-601).  What differs is
// how the bytes arrive:
//   * every global read of the kernels is a direct-to-LDS load issued from
//     inline assembly, and every wait for one is an explicit
//     s_waitcnt vmcnt(N) with N fixed at compile time (the loops are fully
//     unrolled).  The compiler does not see these loads, so none of its own
//     waits can stall on them; its one conservative rule for the builtin
//     form (vmcnt(0) before any LDS read) would empty the ring every block.
//   * each wave keeps kSlots 2 KB weight blocks in flight in its own LDS
//     slots, refilled as it consumes them.  A streaming probe of the
//     token's 53.5 MB (256 workgroups of 8 waves, no arithmetic) took
//     9.8 us this way against 12.5 us for the same blocks through
//     registers, and 9.4 us for 8192 small workgroups of plain loads.
//   * the DMA lanes fetch whole 128-byte lines (8 lanes a row) and land the
//     16-byte chunks with an XOR swizzle (chunk c of row r at unit
//     8 r + (c ^ (r & 7))), so the MFMA lanes' 16-byte LDS reads hit 8
//     distinct bank groups per 8 lanes.
//   * the act-quant of a bf16 input writes the E4M3 codes directly: t = v
//     2^-k is exact (8 significant bits), and the hardware conversion
//     (round to nearest even) of t - |t| 2^-12 is the reference's nearest
//     value with ties toward -inf: a tie moves below itself and no other
//     bf16-derived t lies within |t| 2^-12 of a tie.  f32 inputs keep the
//     integer rounding of wh_e4m3_round.
// Nothing in these kernels stores to global memory before the last weight
// block has landed (the arrival counters are cleared after the stream), so
// each vmcnt counts only the kernel's own DMA loads.
#pragma once
#include "moe_px.h"

#ifndef WH_TOK_SLOTS
#define WH_TOK_SLOTS 4  // gate/up: 2 KB weight blocks in flight per wave
#endif
#ifndef WH_TOKD_SLOTS
#define WH_TOKD_SLOTS 4  // down: the same
#endif
#ifndef WH_TOK_PRO
#define WH_TOK_PRO 2  // gate/up: weight blocks a wave requests before its act-quant
#endif
#ifndef WH_TOKD_PRO
#define WH_TOKD_PRO 2  // down: the same
#endif

// The act-quant thresholds and the expf table in one 2 KB block that two
// waves copy into LDS with one 16-byte DMA per lane each: words 0..253 the
// per-binade log2f thresholds, 256.. the expf table (WH_EXP_TAB_LEN
// doubles), the rest zero.
struct wh_aq_tabs_t {
    uint32_t thr[256];
    uint64_t exp[128];
};
__device__ __align__(16) const wh_aq_tabs_t kAqTabs = {{WH_LOG2F_THR_INIT}, {WH_EXP_TAB_INIT}};
#define WH_TAB_EXP_WORD 256
static_assert(sizeof(wh_aq_tabs_t) == 2048 && WH_EXP_TAB_LEN <= 128, "tables fit the 2 KB staging block");

// LDS byte address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t wh_lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t*)p;
}

// One 16-byte direct-to-LDS load per lane: lane l's 16 bytes from g land at
// LDS byte lds_base + 16 l (lds_base uniform).  M0 is saved and restored
// around it.  The s_waitcnt lgkmcnt(0) first lets an earlier LDS read of the
// same bytes complete before they are overwritten.
__device__ __forceinline__ void wh_dma16(const void* g, uint32_t lds_base) {
    uint32_t saved;
    asm volatile(
        "s_waitcnt lgkmcnt(0)\n\t"
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_base))
        : "memory");
}
// Waits until at most n of this wave's vector memory operations are
// outstanding (n a compile-time constant, <= 63).
template <int n>
__device__ __forceinline__ void wh_vmcnt() {
    static_assert(n >= 0 && n <= 63, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory");
}

// Per-wave timeline for these kernels (-DWH_TIMELINE): stamps stay in
// registers until the end, so no store interleaves with the weight DMAs.
#ifdef WH_TIMELINE
#define WH_TLR_DECL uint64_t wh_tlr[WH_TL_POINTS] = {}
#define WH_TLR(k) wh_tlr[k] = __builtin_amdgcn_s_memrealtime()
#define WH_TLR_FLUSH(kern)                                                                               \
    do {                                                                                                 \
        if ((threadIdx.x & 63) == 0 && blockIdx.x < 512 && blockIdx.y == 0 && (threadIdx.x >> 6) < 16) { \
            for (int k_ = 0; k_ < WH_TL_POINTS; ++k_)                                                    \
                wh_tl_buf[kern][((size_t)blockIdx.x * 16 + (threadIdx.x >> 6)) * WH_TL_POINTS + k_] =      \
                    wh_tlr[k_];                                                                           \
        }                                                                                                \
    } while (0)
#else
#define WH_TLR_DECL \
    do {            \
    } while (0)
#define WH_TLR(k) \
    do {          \
    } while (0)
#define WH_TLR_FLUSH(kern) \
    do {                   \
    } while (0)
#endif

// The two DMAs of one 16-row x 256-col weight block (128 bytes of each row,
// rows 2048 / `row_bytes` apart) into a 2 KB slot: instruction h brings rows
// 8h .. 8h + 7, lane l row 8h + l / 8 and chunk (l % 8) ^ (l / 8) of it.
__device__ __forceinline__ void wh_dma_wblock(const uint8_t* row0, uint32_t row_bytes, uint32_t L, uint32_t slot) {
    const uint32_t r = L >> 3, c = (L & 7) ^ r;
    const uint8_t* p = row0 + (size_t)r * row_bytes + 16 * c;
    wh_dma16(p, slot);
    wh_dma16(p + 8 * (size_t)row_bytes, slot + 1024);
}
// An MFMA lane's two chunks of a swizzled slot (the wh_mx_raw of
// wh_mx_raw_load) and its row's 8 scale bytes.
__device__ __forceinline__ void wh_slot_read(wh_mx_raw& r, const uint8_t* slot, const uint8_t* srow8, uint32_t L) {
    const uint32_t m = L & 15, g = L >> 4;
    const uint32_t c0 = 4 * (g & 1) + 2 * (g >> 1), u0 = 8 * m + (c0 ^ (m & 7));
    r.p = *(const uint4*)(slot + 16 * u0);
    r.q = *(const uint4*)(slot + 16 * (u0 ^ 1));
    r.s = *(const uint2*)srow8;
}
// One block: decode the weights to E4M3 codes, two MFMAs against bo.
__device__ __forceinline__ void wh_tok_step(wh_v4f& acc, const wh_mx_raw& r, const wh_mx_bop& bo, uint32_t g) {
    const wh_mfma_a a = wh_mx_fix(r);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const wh_v8i av = u ? wh_mfma_a_codes<1>(a) : wh_mfma_a_codes<0>(a);
        const uint32_t as = u ? wh_mfma_sbyte<1>(a.s, g) : wh_mfma_sbyte<0>(a.s, g);
        acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bo.v[u], acc, 0, 0, 0, (int)as, 0, (int)bo.s[u]);
    }
}

// Gate/up + SwiGLU, hidden 4096, inter % 16 == 0: grid (ceil(n_experts *
// inter / 16 / kTiles), n_tokens), 512 threads.  Wave w = (matrix m = w / 4,
// 1024-col slice s = w % 4) of the workgroup's kTiles 16-row tiles: 4 blocks
// of 256 cols a tile, kJ = 4 kTiles blocks, kSlots of them in flight.
// Each wave brings in, act-quantizes and reads back only its own slice of x
// (16 values a lane; the w1 and w3 waves of a slice both do it), so no wave
// waits for another before its first MFMA: with a workgroup barrier there,
// every wave waited for the slowest one to get its DMAs issued (issue
// stalls of up to ~4 us while the memory queues are full).
template <int kTiles, int kSlots, bool kBf16>
__global__ void __launch_bounds__(512, 1) k_moe_gateup_tok(wh_moe_args a) {
    constexpr uint32_t kCols = 4096, kG = kCols / 32, kB = 4;
    constexpr int kJ = kB * kTiles, kS = kSlots < kJ ? kSlots : kJ;
    constexpr int kPro = WH_TOK_PRO < kS ? WH_TOK_PRO : kS;  // weight blocks issued before the act-quant
    constexpr int kXd = kBf16 ? 2 : 4;                         // x DMAs per wave (1 KB each)
    constexpr int kSd = (kTiles + 1) / 2;                      // scale DMAs per wave (two tiles each)
    __shared__ __align__(16) uint8_t wslot[8][kS][2048];
    __shared__ __align__(16) uint8_t wsc[8][kTiles][512];  // tile i: 16 rows x the slice's 32 scale bytes
    __shared__ __align__(16) uint8_t xw[8][kXd * 1024];     // the wave's x slice as loaded
    __shared__ __align__(16) uint8_t xcw[8][1024];          // its codes, record layout
    __shared__ __align__(16) uint8_t xsw[8][32];            // its E8M0 bytes
    __shared__ __align__(16) uint64_t expt[WH_EXP_TAB_LEN + 1];
    __shared__ float red[kTiles * 8 * 16];
    WH_TLR_DECL;
    WH_TLR(0);
    const uint32_t tok = blockIdx.y;
    const uint32_t per_e = a.inter >> 4, n_tiles = a.n_experts * per_e;
    const uint32_t tile0 = blockIdx.x * kTiles;
    const uint32_t nt = n_tiles - tile0 < (uint32_t)kTiles ? n_tiles - tile0 : (uint32_t)kTiles;
    // wave-uniform values in SGPRs: the expert table reads below are then
    // scalar loads, not vector loads the DMA counts would have to include
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), L = threadIdx.x & 63, g = L >> 4;
    const uint32_t m = wave >> 2, s = wave & 3;
    const uint8_t* xs = (const uint8_t*)a.x + ((size_t)tok * kCols + 1024 * s) * (kBf16 ? 2 : 4);
    // the rows of the workgroup's tiles (a tile past the end repeats the
    // last one; its results are not stored)
    const uint8_t* wrow[kTiles];
    const uint8_t* srow[kTiles];
#pragma unroll
    for (int i = 0; i < kTiles; ++i) {
        const uint32_t t = tile0 + ((uint32_t)i < nt ? (uint32_t)i : nt - 1);
        const uint32_t e = t / per_e, row = (t - e * per_e) * 16;
        const wh_expert_ptrs ep = wh_moe_ex(a, e);
        wrow[i] = (m ? ep.w3 : ep.w1) + (size_t)row * (kCols / 2) + 512 * s;
        srow[i] = (m ? ep.s3 : ep.s1) + (size_t)row * kG + 32 * s;
    }
    // DMAs, in this order per wave: the expf table (wave 0, lanes 0..18),
    // its x slice (kXd), the scales of the tiles (lanes 0..31 tile 2c, 32..63
    // tile 2c + 1), weight blocks 0 .. kPro - 1
    if (wave == 0 && L * 16 < sizeof(uint64_t) * (WH_EXP_TAB_LEN + 1))
        wh_dma16((const uint8_t*)kAqTabs.exp + 16 * L, wh_lds_addr(expt));
#pragma unroll
    for (int d = 0; d < kXd; ++d) wh_dma16(xs + 1024 * d + 16 * L, wh_lds_addr(xw[wave] + 1024 * d));
#pragma unroll
    for (int c = 0; c < kSd; ++c) {
        const int i = 2 * c + (int)(L >> 5);
        if (i < kTiles) wh_dma16(srow[i] + (size_t)((L & 31) >> 1) * kG + 16 * (L & 1), wh_lds_addr(wsc[wave][2 * c]));
    }
#pragma unroll
    for (int j = 0; j < kPro; ++j) wh_dma_wblock(wrow[j / kB] + 128 * (j % kB), kCols / 2, L, wh_lds_addr(wslot[wave][j]));
    WH_TLR(1);
    wh_vmcnt<kSd + 2 * kPro>();  // this wave's x slice has landed
    WH_TLR(2);
    // act-quant of the slice (E/compute.rs:2504-2521): lane L, half h: record
    // dwords 2q, 2q + 1 of slice group 16 h + L / 4 (q = L % 4)
    float v[2][8];
    bool bad = false;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t G = 16 * h + (L >> 2), q = L & 3;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const uint32_t col = 32 * G + 2 * q + 8 * kk;
            if constexpr (kBf16) {
                const uint32_t w2 = *(const uint32_t*)(xw[wave] + 2 * col);
                v[h][2 * kk] = __uint_as_float(w2 << 16);
                v[h][2 * kk + 1] = __uint_as_float(w2 & 0xffff0000u);
            } else {
                const float2 f2 = *(const float2*)(xw[wave] + 4 * col);
                v[h][2 * kk] = f2.x;
                v[h][2 * kk + 1] = f2.y;
            }
        }
        uint32_t d0, d1;
        int k;
        bool b;
        wh_tok_quant8<kBf16>(v[h], d0, d1, k, b);
        bad |= b;
        *(uint2*)(xcw[wave] + 32 * G + 8 * q) = make_uint2(d0, d1);
        if (q == 0) xsw[wave][G] = (uint8_t)(127 + k - 3);
    }
    WH_TLR(3);
    if (__builtin_amdgcn_ballot_w64(bad) != 0) {
        // -480 (a NaN's value) and an infinite scale have no E4M3 / E8M0
        // code: this wave's slice runs in fp32 from the dequantized x (column
        // order, in its own drained weight slots)
        wh_vmcnt<0>();
        float* xf = (float*)&wslot[wave][0][0];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t G = 16 * h + (L >> 2), q = L & 3;
            float qv[8], sc;
            int kq;
            bool b2;
            wh_aq_vals<8>(v[h], kLog2Thr, qv, kq, sc, b2);
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const uint32_t col = 32 * G + 2 * q + 8 * kk;
                xf[col] = qv[2 * kk] * sc;
                xf[col + 1] = qv[2 * kk + 1] * sc;
            }
        }
#pragma unroll 1
        for (uint32_t i = 0; i < nt; ++i) {
            // lane L runs row L % 16 of the tile; xf is indexed by the full
            // row's column
            const float r = wh_px_rows_fp32(wrow[i] - 512 * s + (size_t)(L & 15) * (kCols / 2),
                                            srow[i] - 32 * s + (size_t)(L & 15) * kG, xf - 1024 * s, kB * s, kB, L);
            if (L < 16) red[(i * 8 + wave) * 16 + L] = r;
        }
    } else {
        // the rest of the ring, then the wave's B operands (one pair of
        // MFMAs per block of its slice)
#pragma unroll
        for (int j = kPro; j < kS; ++j)
            wh_dma_wblock(wrow[j / kB] + 128 * (j % kB), kCols / 2, L, wh_lds_addr(wslot[wave][j]));
        wh_mx_bop bo[kB];
#pragma unroll
        for (int b = 0; b < (int)kB; ++b) wh_mx_bop_load(bo[b], xcw[wave] + 256 * b, xsw[wave] + 8 * b, g);
        WH_TLR(4);
        wh_v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < kJ; ++j) {
            const int b = j % kB, i = j / kB;
            constexpr int kLast = kJ - 1;
            // DMAs issued after block j's: 2 (min(j + kS - 1, kJ - 1) - j)
            if (j + kS - 1 <= kLast) wh_vmcnt<2 * (kS - 1)>();
            else if (kLast - j == 0) wh_vmcnt<0>();
            else if (kLast - j == 1) wh_vmcnt<2>();
            else if (kLast - j == 2) wh_vmcnt<4>();
            else if (kLast - j == 3) wh_vmcnt<6>();
            else if (kLast - j == 4) wh_vmcnt<8>();
            else if (kLast - j == 5) wh_vmcnt<10>();
            else if (kLast - j == 6) wh_vmcnt<12>();
            else wh_vmcnt<14>();
            wh_mx_raw r;
            wh_slot_read(r, wslot[wave][j % kS], wsc[wave][i] + 32 * (L & 15) + 8 * b, L);
            wh_tok_step(acc, r, bo[b], g);
            if (j + kS < kJ)
                wh_dma_wblock(wrow[(j + kS) / kB] + 128 * ((j + kS) % kB), kCols / 2, L,
                              wh_lds_addr(wslot[wave][j % kS]));
            if (b == (int)kB - 1) {
                asm volatile("" : "+v"(acc));
                if ((L & 15) == 0) {  // C[4 (L / 16) + r][0]: column 0 is the token
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) red[(i * 8 + wave) * 16 + 4 * g + rr] = acc[rr];
                }
                acc = wh_v4f{0.0f, 0.0f, 0.0f, 0.0f};
                if (i < 4) WH_TLR(5 + i);
            }
        }
    }
    __syncthreads();
    WH_TLR(10);
    // SwiGLU of the tiles' rows, thread t: tile t / 16, row t % 16
    if (threadIdx.x < nt * 16) {
        const uint32_t i = threadIdx.x >> 4, r = threadIdx.x & 15;
        const float* ri = red + i * 8 * 16 + r;
        const float gv = ((ri[0] + ri[16]) + ri[32]) + ri[48];
        const float uv = ((ri[64] + ri[80]) + ri[96]) + ri[112];
        if (!(fabsf(gv) <= 3.4028235e38f) || !(fabsf(uv) <= 3.4028235e38f)) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
        const uint32_t t = tile0 + i, e = t / per_e, row = (t - e * per_e) * 16 + r;
        const size_t he = ((size_t)tok * a.n_experts + e) * a.inter;
        a.h[he + row] = wh_swiglu(gv, uv, expt, kExpfExc, WH_EXPF_EXC_COUNT);
        if (a.gu) {
            a.gu[2 * he + row] = gv;
            a.gu[2 * he + a.inter + row] = uv;
        }
    }
    WH_TLR(11);
    WH_TLR_FLUSH(0);
}

// Down + routed sum, hidden 4096, inter 2048: grid (hidden / 16, n_tokens),
// 512 threads.  Unit u = (expert u / 4, 512-col quarter u % 4 = blocks
// 2 (u % 4), + 1) of the workgroup's 16 output rows; wave w runs units w,
// w + 8, ... (kU = ceil(n_experts / 2) of them; one past the end repeats the
// last, its result is not stored).  Every expert's slice of the rows is in
// the workgroup, so the routed sum stays local.  Each wave brings in and
// act-quantizes (E/deepseek_v4.rs:595, block 64) the h quarters of its own
// units only: no wave waits for another before its first MFMA.
template <int kU, int kSlots>
__global__ void __launch_bounds__(512, 1) k_moe_down_tok(wh_moe_args a) {
    constexpr uint32_t kIn = 2048, kGi = kIn / 32;
    constexpr int kJ = 2 * kU, kS = kSlots < kJ ? kSlots : kJ;
    constexpr int kPro = WH_TOKD_PRO < kS ? WH_TOKD_PRO : kS;  // weight blocks issued before the act-quant
    static_assert(kU <= 4, "one scale DMA covers four units");
    __shared__ __align__(16) uint8_t wslot[8][kS][2048];
    __shared__ __align__(16) uint8_t wsc[8][kU][256];    // unit k: 16 rows x its 16 scale bytes
    __shared__ __align__(16) uint8_t hw[8][kU][2048];    // unit k's h quarter (f32), then its codes (+E8M0 at 512)
    __shared__ float red[WH_MAX_EXPERTS * 4 * 16];
    WH_TLR_DECL;
    WH_TLR(0);
    const uint32_t tok = blockIdx.y, n = a.n_experts, n_units = 4 * n;
    // wave-uniform in SGPRs: the expert table reads are scalar loads
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), L = threadIdx.x & 63, g = L >> 4;
    const uint32_t row0 = blockIdx.x * 16;
    const float* htok = a.h + (size_t)tok * n * kIn;
    const uint8_t* wl[kU];
    const uint8_t* sl[kU];
    const uint8_t* hl[kU];
#pragma unroll
    for (int k = 0; k < kU; ++k) {
        uint32_t u = wave + 8 * k;
        u = u < n_units ? u : n_units - 1;
        const uint32_t e = u >> 2, qt = u & 3;
        const wh_expert_ptrs ep = wh_moe_ex(a, e);
        wl[k] = ep.w2 + (size_t)row0 * (kIn / 2) + 256 * qt;
        sl[k] = ep.s2 + (size_t)row0 * kGi + 16 * qt;
        hl[k] = (const uint8_t*)(htok + (size_t)e * kIn + 512 * qt);
    }
    // DMAs per wave: the h quarters of its units (2 each), the units'
    // scales in one DMA (lane l: unit l / 16, row l % 16), weight blocks
    // 0 .. kPro - 1
#pragma unroll
    for (int k = 0; k < kU; ++k) {
        wh_dma16(hl[k] + 16 * L, wh_lds_addr(hw[wave][k]));
        wh_dma16(hl[k] + 1024 + 16 * L, wh_lds_addr(hw[wave][k] + 1024));
    }
    {
        const uint32_t k = L >> 4;
        const uint8_t* sp = sl[0];
#pragma unroll
        for (int kk = 1; kk < kU; ++kk) sp = k == (uint32_t)kk ? sl[kk] : sp;
        if (k < (uint32_t)kU) wh_dma16(sp + (size_t)(L & 15) * kGi, wh_lds_addr(wsc[wave][0]));
    }
#pragma unroll
    for (int j = 0; j < kPro; ++j) wh_dma_wblock(wl[j >> 1] + 128 * (j & 1), kIn / 2, L, wh_lds_addr(wslot[wave][j]));
    WH_TLR(1);
    wh_vmcnt<1 + 2 * kPro>();  // this wave's h quarters have landed
    WH_TLR(2);
    // act-quant of each unit's 512 values: lane L, record dwords 2q, 2q + 1
    // of group L / 4; the codes overwrite the quarter's first 512 bytes (all
    // of the wave's reads of the quarter come first), the E8M0 bytes follow
    wh_mx_bop bo[kU][2];
#pragma unroll
    for (int k = 0; k < kU; ++k) {
        const uint32_t G = L >> 2, q = L & 3;
        const float* hv = (const float*)hw[wave][k];
        float v[8];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const float2 f2 = *(const float2*)(hv + 32 * G + 2 * q + 8 * kk);
            v[2 * kk] = f2.x;
            v[2 * kk + 1] = f2.y;
        }
        // h is finite whenever gate/up was (a non-finite gate/up output is
        // already reported); the arithmetic stays in range regardless
        uint32_t d0, d1;
        int ke;
        bool bad;
        wh_tok_quant8<false>(v, d0, d1, ke, bad);
        // every lane's reads of the quarter precede these writes (one wave)
        asm volatile("" ::: "memory");
        *(uint2*)(hw[wave][k] + 32 * G + 8 * q) = make_uint2(d0, d1);
        if (q == 0) hw[wave][k][512 + G] = (uint8_t)(127 + ke - 3);
#pragma unroll
        for (int bb = 0; bb < 2; ++bb) wh_mx_bop_load(bo[k][bb], hw[wave][k] + 256 * bb, hw[wave][k] + 512 + 8 * bb, g);
    }
    WH_TLR(3);
#pragma unroll
    for (int j = kPro; j < kS; ++j) wh_dma_wblock(wl[j >> 1] + 128 * (j & 1), kIn / 2, L, wh_lds_addr(wslot[wave][j]));
    WH_TLR(4);
    wh_v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
        const int bb = j & 1, k = j >> 1;
        constexpr int kLast = kJ - 1;
        if (j + kS - 1 <= kLast) wh_vmcnt<2 * (kS - 1)>();
        else if (kLast - j == 0) wh_vmcnt<0>();
        else if (kLast - j == 1) wh_vmcnt<2>();
        else if (kLast - j == 2) wh_vmcnt<4>();
        else if (kLast - j == 3) wh_vmcnt<6>();
        else if (kLast - j == 4) wh_vmcnt<8>();
        else if (kLast - j == 5) wh_vmcnt<10>();
        else if (kLast - j == 6) wh_vmcnt<12>();
        else wh_vmcnt<14>();
        wh_mx_raw r;
        wh_slot_read(r, wslot[wave][j % kS], wsc[wave][k] + 16 * (L & 15) + 8 * bb, L);
        wh_tok_step(acc, r, bo[k][bb], g);
        if (j + kS < kJ) wh_dma_wblock(wl[(j + kS) >> 1] + 128 * ((j + kS) & 1), kIn / 2, L, wh_lds_addr(wslot[wave][j % kS]));
        if (bb == 1) {
            asm volatile("" : "+v"(acc));
            if ((L & 15) == 0 && wave + 8 * k < n_units) {  // C[4 (L / 16) + r][0]: the token
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) red[(wave + 8 * k) * 16 + 4 * g + rr] = acc[rr];
            }
            acc = wh_v4f{0.0f, 0.0f, 0.0f, 0.0f};
            if (k < 4) WH_TLR(5 + k);
        }
    }
    __syncthreads();
    WH_TLR(10);
    // per-expert outputs (the 4 quarters of each expert), then the ordered
    // routed sum
    if (threadIdx.x < 16) {
        const uint32_t r = threadIdx.x, orow = row0 + r;
        float yv[WH_MAX_EXPERTS];
        bool finite = true;
#pragma unroll
        for (uint32_t e = 0; e < WH_MAX_EXPERTS; ++e) {
            if (e < n) {
                const float* p = red + 4 * e * 16 + r;
                const float y = ((p[0] + p[16]) + p[32]) + p[48];
                finite = finite && fabsf(y) <= 3.4028235e38f;
                yv[e] = y;
                a.y[((size_t)tok * n + e) * a.hidden + orow] = y;
            } else {
                yv[e] = 0.0f;
            }
        }
        if (!finite) atomicOr(a.status, WH_ST_NONFINITE_OUTPUT);
        a.out[(size_t)tok * a.hidden + orow] = wh_route_combine(a, yv);
    }
    WH_TLR(11);
    WH_TLR_FLUSH(1);
}

// Test support: the act-quant of wh_tok_quant8 over n values (n a multiple
// of 64, one 64-block per 8 threads), written back dequantized in column
// order (code value x 2^k; a code of -0, which the MFMA treats as 0, is
// written as +0).  kBf16: the inputs must be bf16 values.
template <bool kBf16>
__global__ void __launch_bounds__(256) k_debug_tok_quant(const float* __restrict__ in, float* __restrict__ out,
                                                        uint32_t n) {
    const uint32_t t = blockIdx.x * 256 + threadIdx.x, blk = t >> 3, G = (t >> 2) & 1, q = t & 3;
    const bool on = blk < n / 64;  // whole 8-lane blocks are on or off together
    const uint32_t base = 64 * (on ? blk : 0) + 32 * G + 2 * q;
    float v[8];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        v[2 * kk] = in[base + 8 * kk];
        v[2 * kk + 1] = in[base + 8 * kk + 1];
    }
    uint32_t d0, d1;
    int k;
    bool bad;
    wh_tok_quant8<kBf16>(v, d0, d1, k, bad);
    if (!on) return;
    const float sc = wh_pow2f(k);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        const float a0 = kk == 0 ? __builtin_amdgcn_cvt_f32_fp8((int)d0, 0)
                         : kk == 1 ? __builtin_amdgcn_cvt_f32_fp8((int)d0, 1)
                         : kk == 2 ? __builtin_amdgcn_cvt_f32_fp8((int)d0, 2)
                                   : __builtin_amdgcn_cvt_f32_fp8((int)d0, 3);
        const float a1 = kk == 0 ? __builtin_amdgcn_cvt_f32_fp8((int)d1, 0)
                         : kk == 1 ? __builtin_amdgcn_cvt_f32_fp8((int)d1, 1)
                         : kk == 2 ? __builtin_amdgcn_cvt_f32_fp8((int)d1, 2)
                                   : __builtin_amdgcn_cvt_f32_fp8((int)d1, 3);
        out[base + 8 * kk] = a0 * sc + 0.0f;
        out[base + 8 * kk + 1] = a1 * sc + 0.0f;
    }
}
