/*
 * pss_device.h - device-side building blocks shared by the sampler kernels:
 * row parameters, the fp32 logit transform, wave64 / block reductions and the
 * LDS radix "select by cumulative weight from the top" used for top-k (weight
 * 1) and top-p (weight = fixed-point mass).
 */
#ifndef PSS_DEVICE_H
#define PSS_DEVICE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pss_math.h"
#include "pumice_sampler.h"

#pragma clang fp contract(off)

#define PSS_WAVE 64

/* threadIdx.x behind an empty volatile asm: the value cannot be hoisted out
 * of a loop, so lane-derived values are recomputed where they are used
 * instead of holding registers across a persistent kernel's item loop. */
__device__ __forceinline__ uint32_t pss_tid() {
    uint32_t t = threadIdx.x;
    __asm__ __volatile__("" : "+v"(t));
    return t;
}

/* Kernel arguments shared by every sampler kernel (passed by value). */
struct pss_args {
    const void* logits;
    uint64_t stride;      /* elements between rows */
    uint32_t V;
    uint32_t dtype;
    uint32_t mode;
    uint32_t do_inc;
    uint32_t pass_idx;
    uint32_t rng_mode;
    const sample_params* params;
    uint32_t* rng;
    uint32_t* step;
    uint32_t* position;
    uint32_t* history;
    uint32_t* result;
    uint32_t* token_ids;
    pss_row_info* info;
    uint32_t* kept_mask;
    uint32_t mask_words;
    float* probs;
    uint64_t probs_stride;
    uint32_t* host_tokens;
    /* per-row workspace of the fast kernel (candidate pools, tickets) */
    void* ws;
    uint32_t vec_ok;      /* rows 16-byte aligned, V * element size a multiple of 16 */
    uint32_t kmax_cov;    /* largest top-k the launched streaming form covers */
    uint32_t wmax_cov;    /* largest window it covers */
    uint32_t* gate;       /* gated passes: the sampler's eos_at word, else NULL */
    uint32_t gate_seq;
    uint32_t eos;
};

/* Global-memory pointers.  Pointers that reach a kernel inside a struct are
 * generic (flat) to the compiler; casting them through address space 1 once at
 * kernel entry lets it emit global_load / global_store / global_atomic, which
 * only touch the vector memory counter and need no aperture checks. */
#define PSS_G __attribute__((address_space(1)))

template <class T>
__device__ __forceinline__ T* pss_glob(T* p) {
    return (T*)(PSS_G T*)p;
}

__device__ __forceinline__ void pss_globalize(pss_args& a) {
    a.logits = pss_glob((const char*)a.logits);
    a.params = (const sample_params*)(const __attribute__((address_space(4))) sample_params*)a.params;
    a.rng = pss_glob(a.rng);
    a.step = pss_glob(a.step);
    a.position = pss_glob(a.position);
    a.history = pss_glob(a.history);
    a.result = pss_glob(a.result);
    a.token_ids = pss_glob(a.token_ids);
    a.info = pss_glob(a.info);
    a.kept_mask = pss_glob(a.kept_mask);
    a.probs = pss_glob(a.probs);
    a.host_tokens = pss_glob(a.host_tokens);
    a.ws = pss_glob((char*)a.ws);
    a.gate = pss_glob(a.gate);
}

/* A gated pass whose decode group follows the one that drew EOS does
 * nothing.  Every workgroup of a launch reads the same answer: the only store
 * to eos_at during a launch lowers it to that launch's own gate_seq. */
__device__ __forceinline__ bool pss_gate_closed(const pss_args& a) {
    return a.gate && __hip_atomic_load(a.gate, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < a.gate_seq;
}

/* Wait until every memory operation this wave issued has completed. */
__device__ __forceinline__ void pss_wait_mem() { __builtin_amdgcn_s_waitcnt(0); }

/* Per-row sampling constants, derived exactly as ArgMax-Reduce.comp:222-230. */
struct pss_rowcfg {
    float invT;
    float rep;
    float pres;
    float minP;
    float topP;
    uint32_t W;       /* clamped penalty window */
    uint32_t K;       /* clamped top-k, 0 = off */
    int doPen;
    int useMinP;
    int useTopP;
};

__device__ inline pss_rowcfg pss_make_rowcfg(const sample_params& sp, uint32_t V) {
    pss_rowcfg c;
    c.invT = 1.0f / sp.temperature;
    c.pres = sp.presencePenalty * c.invT;
    c.rep = sp.repPenalty;
    c.W = sp.penaltyLength < PSS_MAX_PENALTY_LEN ? sp.penaltyLength : PSS_MAX_PENALTY_LEN;
    c.K = sp.topK < V ? sp.topK : V;
    c.doPen = (c.W > 0u) && (c.rep != 1.0f || c.pres != 0.0f);
    c.minP = sp.minP;
    c.useMinP = sp.minP > 0.0f;
    c.topP = sp.topP;
    c.useTopP = (sp.topP > 0.0f) && (sp.topP < 1.0f);
    return c;
}

/* Penalty of an id in the window applied to v = l * invT
 * (ArgMax-Reduce.comp:247-265). */
__device__ __forceinline__ float pss_penalize(float v, const pss_rowcfg& c) {
    if (c.rep != 1.0f) v = (v > 0.0f) ? (v / c.rep) : (v * c.rep);
    return v - c.pres;
}

/* Transformed, canonical logit t (ArgMax-Reduce.comp:246-265). */
__device__ inline float pss_transform(float l, bool member, const pss_rowcfg& c) {
    float v = l * c.invT;
    if (member) v = pss_penalize(v, c);
    return pss_canon(v);
}

__device__ inline float pss_load1(const void* row, uint32_t dtype, uint32_t j) {
    if (dtype == PSS_DTYPE_F16) return (float)(((const _Float16*)row)[j]);
    return ((const float*)row)[j];
}

__device__ inline bool pss_bit(const uint32_t* bits, uint32_t j) {
    return (bits[j >> 5] >> (j & 31u)) & 1u;
}

/* ------------------------------------------------------------------ */
/* VALU-only lane exchanges: DPP within rows of 16 lanes, the gfx950   */
/* permlane swaps across rows.  All 64 lanes must be active.           */
/* ------------------------------------------------------------------ */

#define PSS_DPP_QUAD_XOR1 0xB1  /* quad_perm [1,0,3,2] */
#define PSS_DPP_QUAD_XOR2 0x4E  /* quad_perm [2,3,0,1] */
#define PSS_DPP_ROW_SHL(n) (0x100 + (n)) /* lane i reads lane i + n of its row */
#define PSS_DPP_ROW_SHR(n) (0x110 + (n)) /* lane i reads lane i - n of its row */

/* v of lane (lane ^ J), J in {1, 2, 4, 8, 16, 32}. */
template <int J>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
    if constexpr (J == 1) {
        return __builtin_amdgcn_update_dpp(v, v, PSS_DPP_QUAD_XOR1, 0xF, 0xF, false);
    } else if constexpr (J == 2) {
        return __builtin_amdgcn_update_dpp(v, v, PSS_DPP_QUAD_XOR2, 0xF, 0xF, false);
    } else if constexpr (J == 4 || J == 8) {
        /* lanes with bit J clear read lane + J, the others lane - J; a bank
         * is 4 lanes of a row, so the two halves are bank masks */
        constexpr int lowBanks = J == 4 ? 0x5 : 0x3;
        const uint32_t r = __builtin_amdgcn_update_dpp(v, v, PSS_DPP_ROW_SHL(J), 0xF, lowBanks, false);
        return __builtin_amdgcn_update_dpp(r, v, PSS_DPP_ROW_SHR(J), 0xF, 0xF ^ lowBanks, false);
    } else if constexpr (J == 16) {
        /* swap odd rows of the first operand with even rows of the second */
        const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (pss_tid() & 16u) ? p[0] : p[1];
    } else {
        static_assert(J == 32, "lane_xor: J must be a power of two below 64");
        /* swap the upper half of the first operand with the lower half of the second */
        const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (pss_tid() & 32u) ? p[0] : p[1];
    }
}

template <int J>
__device__ __forceinline__ uint64_t lane_xor64(uint64_t v) {
    return ((uint64_t)lane_xor<J>((uint32_t)(v >> 32)) << 32) | lane_xor<J>((uint32_t)v);
}

__device__ __forceinline__ uint32_t dpp_max_u32(uint32_t v) {
    v = max(v, lane_xor<1>(v));
    v = max(v, lane_xor<2>(v));
    v = max(v, lane_xor<4>(v));
    v = max(v, lane_xor<8>(v));
    v = max(v, lane_xor<16>(v));
    return max(v, lane_xor<32>(v));
}

__device__ __forceinline__ uint32_t dpp_min_u32(uint32_t v) {
    v = min(v, lane_xor<1>(v));
    v = min(v, lane_xor<2>(v));
    v = min(v, lane_xor<4>(v));
    v = min(v, lane_xor<8>(v));
    v = min(v, lane_xor<16>(v));
    return min(v, lane_xor<32>(v));
}

__device__ __forceinline__ uint64_t dpp_sum_u64(uint64_t v) {
    v += lane_xor64<1>(v);
    v += lane_xor64<2>(v);
    v += lane_xor64<4>(v);
    v += lane_xor64<8>(v);
    v += lane_xor64<16>(v);
    return v + lane_xor64<32>(v);
}

__device__ __forceinline__ uint64_t dpp_max_u64(uint64_t v) {
    uint64_t w;
    w = lane_xor64<1>(v); v = w > v ? w : v;
    w = lane_xor64<2>(v); v = w > v ? w : v;
    w = lane_xor64<4>(v); v = w > v ? w : v;
    w = lane_xor64<8>(v); v = w > v ? w : v;
    w = lane_xor64<16>(v); v = w > v ? w : v;
    w = lane_xor64<32>(v); return w > v ? w : v;
}

/* Inclusive prefix sum over lanes: row_shr steps within each row of 16,
 * then the row totals (lanes 15, 31, 47) carried into the rows above. */
__device__ __forceinline__ uint64_t dpp_incl_scan_u64(uint64_t x) {
    uint32_t lo = (uint32_t)x, hi = (uint32_t)(x >> 32);
#define PSS_SCAN_STEP(d)                                                                   \
    {                                                                                      \
        const uint32_t sl = __builtin_amdgcn_update_dpp(0u, lo, PSS_DPP_ROW_SHR(d), 0xF, 0xF, false); \
        const uint32_t sh_ = __builtin_amdgcn_update_dpp(0u, hi, PSS_DPP_ROW_SHR(d), 0xF, 0xF, false); \
        const uint64_t t = (((uint64_t)hi << 32) | lo) + (((uint64_t)sh_ << 32) | sl);      \
        lo = (uint32_t)t;                                                                  \
        hi = (uint32_t)(t >> 32);                                                          \
    }
    PSS_SCAN_STEP(1)
    PSS_SCAN_STEP(2)
    PSS_SCAN_STEP(4)
    PSS_SCAN_STEP(8)
#undef PSS_SCAN_STEP
    const uint64_t v = ((uint64_t)hi << 32) | lo;
    const uint64_t r0 = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(hi, 15) << 32) |
                        (uint32_t)__builtin_amdgcn_readlane(lo, 15);
    const uint64_t r1 = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(hi, 31) << 32) |
                        (uint32_t)__builtin_amdgcn_readlane(lo, 31);
    const uint64_t r2 = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(hi, 47) << 32) |
                        (uint32_t)__builtin_amdgcn_readlane(lo, 47);
    const uint32_t rowi = (pss_tid() >> 4) & 3u;
    return v + (rowi >= 1u ? r0 : 0ull) + (rowi >= 2u ? r1 : 0ull) + (rowi >= 3u ? r2 : 0ull);
}

/* Inclusive prefix sum of one u32 per lane: row_shr steps within each row
 * of 16, then the row totals (lanes 15, 31, 47) carried into the rows above. */
__device__ __forceinline__ uint32_t dpp_incl_scan_u32(uint32_t x) {
    x += __builtin_amdgcn_update_dpp(0u, x, PSS_DPP_ROW_SHR(1), 0xF, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0u, x, PSS_DPP_ROW_SHR(2), 0xF, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0u, x, PSS_DPP_ROW_SHR(4), 0xF, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0u, x, PSS_DPP_ROW_SHR(8), 0xF, 0xF, false);
    const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane(x, 15);
    const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane(x, 31);
    const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane(x, 47);
    const uint32_t rowi = (pss_tid() >> 4) & 3u;
    return x + (rowi >= 1u ? r0 : 0u) + (rowi >= 2u ? r1 : 0u) + (rowi >= 3u ? r2 : 0u);
}

/* One compare-exchange stage (block size KB, distance J) of an ascending
 * bitonic sort of one u32 per lane. */
template <int KB, int J>
__device__ __forceinline__ uint32_t dpp_bitonic_stage_u32(uint32_t x) {
    const uint32_t y = lane_xor<J>(x);
    const uint32_t lane = pss_tid() & 63u;
    const bool lowSide = (lane & (uint32_t)J) == 0u;
    const bool asc = KB == 64 ? true : (lane & (uint32_t)KB) == 0u;
    return lowSide == asc ? min(x, y) : max(x, y);
}

/* Ascending sort of one u32 per lane across the wave. */
__device__ __forceinline__ uint32_t dpp_sort_asc_u32(uint32_t x) {
    x = dpp_bitonic_stage_u32<2, 1>(x);
    x = dpp_bitonic_stage_u32<4, 2>(x);
    x = dpp_bitonic_stage_u32<4, 1>(x);
    x = dpp_bitonic_stage_u32<8, 4>(x);
    x = dpp_bitonic_stage_u32<8, 2>(x);
    x = dpp_bitonic_stage_u32<8, 1>(x);
    x = dpp_bitonic_stage_u32<16, 8>(x);
    x = dpp_bitonic_stage_u32<16, 4>(x);
    x = dpp_bitonic_stage_u32<16, 2>(x);
    x = dpp_bitonic_stage_u32<16, 1>(x);
    x = dpp_bitonic_stage_u32<32, 16>(x);
    x = dpp_bitonic_stage_u32<32, 8>(x);
    x = dpp_bitonic_stage_u32<32, 4>(x);
    x = dpp_bitonic_stage_u32<32, 2>(x);
    x = dpp_bitonic_stage_u32<32, 1>(x);
    x = dpp_bitonic_stage_u32<64, 32>(x);
    x = dpp_bitonic_stage_u32<64, 16>(x);
    x = dpp_bitonic_stage_u32<64, 8>(x);
    x = dpp_bitonic_stage_u32<64, 4>(x);
    x = dpp_bitonic_stage_u32<64, 2>(x);
    return dpp_bitonic_stage_u32<64, 1>(x);
}

/* One compare-exchange stage (block size KB, distance J) of an ascending
 * bitonic sort of one u64 per lane. */
template <int KB, int J>
__device__ __forceinline__ uint64_t dpp_bitonic_stage(uint64_t x) {
    const uint64_t y = lane_xor64<J>(x);
    const uint32_t lane = pss_tid() & 63u;
    const bool lowSide = (lane & (uint32_t)J) == 0u;
    const bool asc = KB == 64 ? true : (lane & (uint32_t)KB) == 0u;
    const uint64_t mn = x < y ? x : y, mx = x < y ? y : x;
    return lowSide == asc ? mn : mx;
}

/* Ascending sort of one u64 per lane across the wave. */
__device__ __forceinline__ uint64_t dpp_sort_asc_u64(uint64_t x) {
    x = dpp_bitonic_stage<2, 1>(x);
    x = dpp_bitonic_stage<4, 2>(x);
    x = dpp_bitonic_stage<4, 1>(x);
    x = dpp_bitonic_stage<8, 4>(x);
    x = dpp_bitonic_stage<8, 2>(x);
    x = dpp_bitonic_stage<8, 1>(x);
    x = dpp_bitonic_stage<16, 8>(x);
    x = dpp_bitonic_stage<16, 4>(x);
    x = dpp_bitonic_stage<16, 2>(x);
    x = dpp_bitonic_stage<16, 1>(x);
    x = dpp_bitonic_stage<32, 16>(x);
    x = dpp_bitonic_stage<32, 8>(x);
    x = dpp_bitonic_stage<32, 4>(x);
    x = dpp_bitonic_stage<32, 2>(x);
    x = dpp_bitonic_stage<32, 1>(x);
    x = dpp_bitonic_stage<64, 32>(x);
    x = dpp_bitonic_stage<64, 16>(x);
    x = dpp_bitonic_stage<64, 8>(x);
    x = dpp_bitonic_stage<64, 4>(x);
    x = dpp_bitonic_stage<64, 2>(x);
    return dpp_bitonic_stage<64, 1>(x);
}

/* ------------------------------------------------------------------ */
/* wave64 reductions and scans (all 64 lanes active)                   */
/* ------------------------------------------------------------------ */

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) { return dpp_max_u32(v); }
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) { return dpp_min_u32(v); }
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) { return dpp_max_u64(v); }
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) { return dpp_sum_u64(v); }
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) { return (uint32_t)dpp_sum_u64(v); }

/* Inclusive prefix sum across the 64 lanes. */
__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t v) { return dpp_incl_scan_u64(v); }
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) { return dpp_incl_scan_u32(v); }

/* Inclusive suffix sum (sum over lanes >= this lane). */
__device__ __forceinline__ uint64_t wave_incl_suffix_u64(uint64_t v) {
    const uint64_t incl = dpp_incl_scan_u64(v);
    const uint64_t total = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((uint32_t)(incl >> 32), 63) << 32) |
                           (uint32_t)__builtin_amdgcn_readlane((uint32_t)incl, 63);
    return total - incl + v;
}

/* ------------------------------------------------------------------ */
/* block reductions (NT threads, NT/64 waves); `red` holds NT/64 slots */
/* ------------------------------------------------------------------ */

template <int NT>
__device__ inline uint64_t block_sum_u64(uint64_t v, uint64_t* red) {
    constexpr int NW = NT / PSS_WAVE;
    v = wave_sum_u64(v);
    const int w = pss_tid() >> 6;
    if ((pss_tid() & 63) == 0) red[w] = v;
    __syncthreads();
    uint64_t s = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) s += red[i];
    __syncthreads();
    return s;
}

template <int NT>
__device__ inline uint64_t block_max_u64(uint64_t v, uint64_t* red) {
    constexpr int NW = NT / PSS_WAVE;
    v = wave_max_u64(v);
    const int w = pss_tid() >> 6;
    if ((pss_tid() & 63) == 0) red[w] = v;
    __syncthreads();
    uint64_t s = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) s = red[i] > s ? red[i] : s;
    __syncthreads();
    return s;
}

/* Exclusive prefix sum over threads in thread order; *total gets the sum. */
template <int NT>
__device__ inline uint64_t block_excl_scan_u64(uint64_t v, uint64_t* red, uint64_t* total) {
    constexpr int NW = NT / PSS_WAVE;
    uint64_t inc = wave_incl_scan_u64(v);
    const int w = pss_tid() >> 6;
    if ((pss_tid() & 63) == 63) red[w] = inc;
    __syncthreads();
    uint64_t off = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        if (i < w) off += red[i];
        tot += red[i];
    }
    __syncthreads();
    *total = tot;
    return off + inc - v;
}

/*
 * One radix level of "select by cumulative weight from the top": given a
 * 256-bin histogram `hist` of weights per digit and `rem` >= 1 (<= the
 * histogram total), find the digit d with sum(hist[>d]) < rem <= sum(hist[>=d])
 * and return it; *rem_out = rem - sum(hist[>d]).  Run by wave 0 only.
 */
__device__ inline void wave0_pick_digit(const uint64_t* hist, uint64_t rem, uint32_t* digit_out,
                                        uint64_t* rem_out) {
    const int lane = pss_tid() & 63;
    uint64_t h0 = hist[4 * lane + 0], h1 = hist[4 * lane + 1];
    uint64_t h2 = hist[4 * lane + 2], h3 = hist[4 * lane + 3];
    uint64_t s = h0 + h1 + h2 + h3;
    uint64_t incl = wave_incl_suffix_u64(s); /* lanes >= lane */
    uint64_t above = incl - s;               /* lanes > lane   */
    if (above < rem && rem <= incl) {
        uint64_t cum = above;
        uint32_t d = 4u * lane;
        uint64_t hs[4] = {h0, h1, h2, h3};
        for (int i = 3; i >= 0; --i) {
            if (cum + hs[i] >= rem) {
                d = 4u * lane + (uint32_t)i;
                break;
            }
            cum += hs[i];
        }
        *digit_out = d;
        *rem_out = rem - cum;
    }
}


/* ------------------------------------------------------------------ */
/* wave-level selection without LDS or barriers                        */
/* ------------------------------------------------------------------ */

/* The K-th largest (K >= 1) of the R * 64 values a wave holds R per lane:
 * the largest x with count(v >= x) >= K, found bit by bit from the top with
 * ballots.  Returns 0 when fewer than K values are nonzero.  Every lane of
 * the wave calls it and gets the same result.  With BITS < 32 only the top
 * BITS bits are resolved and the rest are left 0, which gives a lower bound
 * of the K-th largest (the largest BITS-bit prefix with count >= K). */
template <int R, int BITS = 32>
__device__ inline uint32_t wave_kth_largest(const uint32_t* v, uint32_t K) {
    uint32_t x = 0;
    for (int b = 31; b >= 32 - BITS; --b) {
        const uint32_t y = x | (1u << b);
        uint32_t cnt = 0;
#pragma unroll
        for (int i = 0; i < R; ++i) cnt += (uint32_t)__popcll(__ballot(v[i] >= y));
        if (cnt >= K) x = y;
    }
    return x;
}

/* wave_kth_largest resolving two bits per step (three ballot counts per value
 * and step, independent of each other): bits lo..hi of the result, with the
 * bits above hi taken from x0 (which must be a prefix of the answer with the
 * bits at and below hi clear).  (hi - lo + 1) must be even.  With lo > 0 the
 * result is the lower bound described for wave_kth_largest. */
template <int R>
__device__ inline uint32_t wave_kth_largest_r4(const uint32_t* v, uint32_t K, uint32_t x0, int hi,
                                               int lo) {
    uint32_t x = x0;
    for (int b = hi - 1; b >= lo; b -= 2) {
        const uint32_t y1 = x | (1u << b), y2 = x | (2u << b), y3 = x | (3u << b);
        uint32_t c1 = 0, c2 = 0, c3 = 0;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            c1 += (uint32_t)__popcll(__ballot(v[i] >= y1));
            c2 += (uint32_t)__popcll(__ballot(v[i] >= y2));
            c3 += (uint32_t)__popcll(__ballot(v[i] >= y3));
        }
        x = c3 >= K ? y3 : (c2 >= K ? y2 : (c1 >= K ? y1 : x));
    }
    return x;
}



/* Value of a lane chosen by a wave-uniform index, in every lane. */
__device__ __forceinline__ uint32_t wave_read_u32(uint32_t v, uint32_t lane) {
    return (uint32_t)__builtin_amdgcn_readlane(v, lane);
}
__device__ __forceinline__ uint64_t wave_read_u64(uint64_t v, uint32_t lane) {
    return ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((uint32_t)(v >> 32), lane) << 32) |
           (uint32_t)__builtin_amdgcn_readlane((uint32_t)v, lane);
}

/* Lanes below this one, as a 64-bit mask. */
__device__ __forceinline__ uint64_t wave_lanes_below() {
    const uint32_t lane = pss_tid() & 63u;
    return lane ? (~0ull >> (64u - lane)) : 0ull;
}


#endif /* PSS_DEVICE_H */
