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
    uint32_t vec_ok;      /* rows are 16-byte aligned: vector loads allowed */
};

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

/* Transformed, canonical logit t (ArgMax-Reduce.comp:246-265). */
__device__ inline float pss_transform(float l, bool member, const pss_rowcfg& c) {
    float v = l * c.invT;
    if (member) {
        if (c.rep != 1.0f) v = (v > 0.0f) ? (v / c.rep) : (v * c.rep);
        v = v - c.pres;
    }
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
/* wave64 reductions                                                   */
/* ------------------------------------------------------------------ */

__device__ inline uint32_t wave_max_u32(uint32_t v) {
    for (int o = 32; o > 0; o >>= 1) {
        uint32_t w = __shfl_xor(v, o);
        v = w > v ? w : v;
    }
    return v;
}

__device__ inline uint64_t wave_max_u64(uint64_t v) {
    for (int o = 32; o > 0; o >>= 1) {
        uint64_t w = __shfl_xor(v, o);
        v = w > v ? w : v;
    }
    return v;
}

__device__ inline uint64_t wave_sum_u64(uint64_t v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ inline uint32_t wave_sum_u32(uint32_t v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

/* Inclusive prefix sum across the 64 lanes. */
__device__ inline uint64_t wave_incl_scan_u64(uint64_t v) {
    const int lane = threadIdx.x & 63;
    for (int o = 1; o < 64; o <<= 1) {
        uint64_t w = __shfl_up(v, (unsigned)o);
        if (lane >= o) v += w;
    }
    return v;
}

/* Inclusive suffix sum (sum over lanes >= this lane). */
__device__ inline uint64_t wave_incl_suffix_u64(uint64_t v) {
    const int lane = threadIdx.x & 63;
    for (int o = 1; o < 64; o <<= 1) {
        uint64_t w = __shfl_down(v, (unsigned)o);
        if (lane + o < 64) v += w;
    }
    return v;
}

/* ------------------------------------------------------------------ */
/* block reductions (NT threads, NT/64 waves); `red` holds NT/64 slots */
/* ------------------------------------------------------------------ */

template <int NT>
__device__ inline uint64_t block_sum_u64(uint64_t v, uint64_t* red) {
    constexpr int NW = NT / PSS_WAVE;
    v = wave_sum_u64(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
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
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
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
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 63) red[w] = inc;
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
    const int lane = threadIdx.x & 63;
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

#endif /* PSS_DEVICE_H */
