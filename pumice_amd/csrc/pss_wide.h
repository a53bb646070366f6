/*
 * pss_wide.h - the split-row form for wide rows: top-k up to PSS_WIDE_KMAX,
 * windows up to PSS_MAX_PENALTY_LEN ids, vocabularies up to PSS_MAX_VOCAB,
 * with every row spread over several workgroups so that a small batch of
 * wide rows still occupies the whole chip (64 rows of 248,320 ids: 256
 * workgroups, one per CU, instead of 64).
 *
 * Grid rows x G, G = ceil(V / 65,536).  The row is cut into waves' spans of
 * 4,096 ids (16 loads of 256 ids per wave fp32, 8 of 512 fp16) and these
 * are split evenly over the row's G workgroups, at most 16 each (61 spans
 * at V = 248,320: 15, 15, 15, 16).  Per workgroup:
 *   1. the row's window ids (one per thread) are requested first, then all
 *      16-byte nontemporal loads of each lane (load j of lane l of a wave
 *      holds ids j 64 E + l E + [0, E) of its span, each load instruction
 *      of a wave 1 KiB contiguous; the buffer resource ends with the
 *      segment, so loads beyond it read nothing);
 *   2. the window ids inside the segment go to an LDS bitmap, each distinct
 *      id once (the thread that sets its bit owns it and fetches its logit);
 *   3. as the loads arrive: t = l * (1/T), window ids and ids beyond the segment set
 *       to -inf, each lane's four largest values;
 *   4. two certificates from the lanes' top values: per full wave (all
 *      4,096 ids in the segment; nf of them) the ceil(K / nf)-th and the
 *      ceil(ceil(K / G) / nf)-th largest of its 256 values (24-bit
 *      resolution, lower bounds), each minimized over those waves.  The
 *      first, LK, has at least K elements of the segment at or above it, so
 *      it is at most the row's K-th largest; the second, L2, has
 *      ceil(K / G) of them, so the minimum of L2 over the row's G segments
 *      has at least K elements of the row at or above it and is a lower
 *      bound too;
 *   5. the segment's elements at or above LK, and its penalized window
 *      elements at or above LK, go to the segment's range of the row's pool
 *      in HBM (about K + K/10 entries); the count and L2 to the workspace;
 *   6. the workgroup counts itself on the row's ticket (agent-scope
 *      acquire-release, after its stores have completed); the workgroup
 *      that completes the count resets the ticket and finishes the row: it
 *      gathers the pool entries at or above max(max LK, min L2) into LDS
 *      (about K + K/10 of the G (K + K/10)), and runs the list finisher (the
 *      exact K-th largest, masses, top-p, min-p, the ascending-id draw and
 *      the epilogue).
 * Greedy rows keep each segment's (key, smallest id) best; rows outside the
 * candidate path (top-k off or above PSS_WIDE_KMAX, a segment whose
 * candidates overflow its pool range, no finite bound) run the general
 * algorithm in the finishing workgroup.  One kernel; no workgroup waits for
 * another.
 *
 * Roofline: HBM, one read of each row (V * e + 4 W + 44 bytes per row); the
 * pool adds about G (K + K/10) 8-byte writes and reads per row (35 KiB at
 * K = 1,000, G = 4: 3.5% of a 248,320-id fp32 row).
 */
#ifndef PSS_WIDE_H
#define PSS_WIDE_H

#include "pss_stream.h"

#define PSS_WSP_NW 16
#define PSS_WSP_NT (PSS_WSP_NW * PSS_WAVE)

/* Value e of a load as a transformed float: fp32 loads hold t in place; fp16
 * loads hold the raw halves (excluded elements set to -inf). */
template <int DT>
__device__ __forceinline__ float pss_res_t(const uint4& r, int e, float invT) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
    if (DT == PSS_DTYPE_F16) {
        const uint16_t h = (uint16_t)(w[e >> 1] >> ((e & 1) * 16));
        _Float16 hf;
        __builtin_memcpy(&hf, &h, 2);
        return (float)hf * invT;
    }
    return __uint_as_float(w[e]);
}

/* Element e of a load set to -inf (an excluded id). */
template <int DT>
__device__ __forceinline__ void pss_res_kill(uint4& r, int e) {
    uint32_t w[4] = {r.x, r.y, r.z, r.w};
    if (DT == PSS_DTYPE_F16)
        w[e >> 1] = (w[e >> 1] & ~(0xFFFFu << ((e & 1) * 16))) | (0xFC00u << ((e & 1) * 16));
    else
        w[e] = 0xFF800000u;
    r = make_uint4(w[0], w[1], w[2], w[3]);
}

/* x as a uniform value defined at this point of the instruction stream (the
 * compiler places no use of x, and no wait for the load that produced it,
 * before this point). */
template <class T>
__device__ __forceinline__ void pss_pin_s(T& x) {
    static_assert(sizeof(T) == 4, "32-bit values");
    uint32_t u = __builtin_bit_cast(uint32_t, x);
    __asm__ __volatile__("" : "+v"(u));
    x = __builtin_bit_cast(T, __builtin_amdgcn_readfirstlane(u));
}

template <int DT>
struct pss_wsp_geom {
    static constexpr int E = DT == PSS_DTYPE_F16 ? 8 : 4;
    static constexpr int NL = DT == PSS_DTYPE_F16 ? 8 : 16;   /* loads per lane: 64 elements */
    static constexpr uint32_t LSPAN = (uint32_t)PSS_WAVE * E; /* ids per load instruction of a wave */
    static constexpr uint32_t WSPAN = (uint32_t)NL * LSPAN;   /* ids per wave */
    static constexpr uint32_t SEG = PSS_WSP_NW * WSPAN;       /* ids per workgroup */
    static constexpr uint32_t SBW = SEG / 32u;                /* window bitmap words */
    static_assert(SEG == 65536u, "segment of 65,536 ids");
};

/* ------------------------------------------------------------------------ */
/* histogram finisher: up to 4,096 candidates, top-k up to 1,024             */
/* ------------------------------------------------------------------------ */

#define PSS_HF_N 4096u    /* candidates the histogram finisher takes (four per thread of 1,024) */
#define PSS_HF_R 4        /* entries per thread */
#define PSS_HF_BINS 2048u /* key bins: 11 bits below the common prefix of the bound and the maximum */
#define PSS_HF_GATHER 64u /* entries of one bin resolved exactly by one wave */

struct pss_hfin_shared {
    uint32_t hc[PSS_HF_BINS];            /* entries per bin */
    uint64_t hq[PSS_HF_BINS];            /* mass per bin */
    uint64_t h8[2][512];                 /* the draw: kept mass per 9-bit id digit (two passes) */
    unsigned long long be[2][PSS_HF_GATHER]; /* entries of the K-th bin / the top-p bin */
    uint32_t bn[2];                      /* entries claimed for be */
    uint32_t wsc[PSS_WSP_NW];            /* per wave: counts (scan), then kept counts */
    uint64_t wsq[PSS_WSP_NW];            /* per wave: masses (scan), then kept masses */
    uint32_t wl[PSS_WSP_NW];             /* per wave: largest kept id + 1 */
    uint32_t rK, rP;                     /* first bin (descending) whose count / mass reaches K / the need */
    uint32_t aC;                         /* entries above the K-th bin */
    uint64_t aQK, aQP;                   /* mass above the K-th bin / the top-p bin */
    uint32_t tauK, tauP, d1, tok;
    uint64_t zk, rem;
};

/* One wave (wave 0): the digit of 512 bins (8 per lane, bin 8 l + i) at which
 * the mass suffix from the top reaches rem (1 <= rem <= total), and rem less
 * the mass strictly above that digit. */
__device__ __forceinline__ uint32_t pss_hf_digit512(const uint64_t* h, uint64_t& rem) {
    const uint32_t lane = threadIdx.x & 63u;
    uint64_t v[8], s8 = 0u;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        v[i] = h[8u * lane + (uint32_t)i];
        s8 += v[i];
    }
    const uint64_t incl = wave_incl_suffix_u64(s8); /* lanes >= lane */
    const uint64_t abv = incl - s8;
    const bool hit = abv < rem && rem <= incl;
    uint32_t dg = 8u * lane;
    uint64_t cum = abv;
    if (hit) {
        for (int i = 7; i >= 0; --i) {
            if (cum + v[i] >= rem) {
                dg = 8u * lane + (uint32_t)i;
                break;
            }
            cum += v[i];
        }
    }
    const uint32_t src = (uint32_t)__ffsll((long long)__ballot(hit)) - 1u;
    rem -= wave_read_u64(cum, src);
    return wave_read_u32(dg, src);
}

/*
 * Finisher over n <= PSS_HF_N candidates (list: key << 32 | id, in LDS), all
 * at or above `lo`, a lower bound of the row's K-th largest value, with the
 * row maximum tmaxKey among them; 1,024 threads, four entries each:
 *   1. one pass: each entry's count and mass q = fixq(p) into 2,048 bins of
 *      its key (the 11 bits below the common prefix of lo and tmaxKey, so
 *      bins are in key order); a block scan of the bins from the top;
 *   2. S5: the bin where the count from the top reaches K; its entries (at
 *      most 64) sorted by wave 0 give the exact K-th largest and, with the
 *      mass above the bin, Z_k;
 *   3. S6: the bin where the mass from the top reaches ceil(topP Z_k) (the
 *      K-th bin at the latest); its entries sorted by wave 0, their masses
 *      scanned in key order, give the cut;
 *   4. S7: kept = key >= tau and p >= min-p; Z, the count by block sums;
 *   5. S8: the first id in ascending order whose cumulative kept mass
 *      exceeds the draw target: two passes over 9-bit id digits (ids below
 *      2^18 = PSS_MAX_VOCAB);
 * then the verification outputs and the epilogue.  The same quantities, bit
 * for bit, as pss_list_finish.  Returns false (nothing written) when a bin
 * it must resolve holds more than 64 entries (dense ties).
 */
/* The histogram finisher's bins and counters at their initial values (all
 * threads; a barrier must follow before pss_hist_finish). */
__device__ __forceinline__ void pss_hist_clear(pss_hfin_shared& hs) {
    const uint32_t tid = threadIdx.x;
    for (uint32_t i = tid; i < PSS_HF_BINS; i += PSS_WSP_NT) {
        hs.hc[i] = 0u;
        hs.hq[i] = 0ull;
    }
    for (uint32_t i = tid; i < 2u * 512u; i += PSS_WSP_NT) (&hs.h8[0][0])[i] = 0ull;
    if (tid == 0u) {
        hs.rK = hs.rP = 0xFFFFFFFFu;
        hs.bn[0] = hs.bn[1] = 0u;
    }
}

__device__ __forceinline__ bool pss_hist_finish(const pss_args& a, uint32_t row, const pss_rowcfg& c,
                                                const unsigned long long* list, uint32_t n, uint32_t lo,
                                                uint32_t tmaxKey, const pss_row_pre& pre, pss_hfin_shared& hs,
                                                bool cleared) {
    constexpr int HR = PSS_HF_R;
    constexpr int NT = PSS_WSP_NT;
    static_assert(PSS_MAX_VOCAB <= (1u << 18), "ids of two 9-bit digits");
    const uint32_t tid = threadIdx.x, lane = tid & 63u, w = tid >> 6;
    const float tmax = pss_unkey(tmaxKey);
    const uint32_t d = lo ^ tmaxKey;
    const int hib = d ? 31 - (int)__clz(d) : 0;
    const int sh = hib >= 10 ? hib - 10 : 0;
    auto binof = [&](uint32_t k) -> uint32_t { return (k >> sh) & (PSS_HF_BINS - 1u); };
    unsigned long long e[HR];
    uint32_t k[HR];
    bool v[HR];
    float p[HR];
    uint64_t q[HR];
#pragma unroll
    for (int h = 0; h < HR; ++h) {
        const uint32_t i = tid + (uint32_t)h * NT;
        v[h] = i < n;
        e[h] = v[h] ? list[i] : 0ull;
        k[h] = (uint32_t)(e[h] >> 32);
        p[h] = v[h] ? pss_prob(pss_unkey(k[h]), tmax) : 0.0f;
        q[h] = v[h] ? pss_fixq(p[h]) : 0ull;
    }
    if (!cleared) {
        pss_hist_clear(hs);
        __syncthreads();
    }
    /* 1 */
#pragma unroll
    for (int h = 0; h < HR; ++h)
        if (v[h]) {
            atomicAdd(&hs.hc[binof(k[h])], 1u);
            atomicAdd((unsigned long long*)&hs.hq[binof(k[h])], (unsigned long long)q[h]);
        }
    __syncthreads();
    /* thread t: descending positions r = 2t, 2t + 1 (bins 2047 - r) */
    const uint32_t b0 = PSS_HF_BINS - 1u - 2u * tid, b1 = b0 - 1u;
    const uint32_t c0 = hs.hc[b0], c1 = hs.hc[b1];
    const uint64_t q0 = hs.hq[b0], q1 = hs.hq[b1];
    const uint32_t ic = wave_incl_scan_u32(c0 + c1);
    const uint64_t iq = wave_incl_scan_u64(q0 + q1);
    if (lane == 63u) {
        hs.wsc[w] = ic;
        hs.wsq[w] = iq;
    }
    __syncthreads();
    uint32_t oc = 0u;
    uint64_t oq = 0u;
#pragma unroll
    for (uint32_t x = 0; x < (uint32_t)PSS_WSP_NW; ++x)
        if (x < w) {
            oc += hs.wsc[x];
            oq += hs.wsq[x];
        }
    const uint32_t S1c = oc + ic, S0c = S1c - c1; /* counts from the top through r = 2t + 1 / 2t */
    const uint64_t S1q = oq + iq, S0q = S1q - q1;
    /* 2 */
    const uint32_t Kc = c.K <= n ? c.K : n;
    {
        const uint32_t r = S0c >= Kc ? 2u * tid : (S1c >= Kc ? 2u * tid + 1u : 0xFFFFFFFFu);
        const uint32_t rm = wave_min_u32(r);
        if (lane == 0u && rm != 0xFFFFFFFFu) atomicMin(&hs.rK, rm);
    }
    __syncthreads();
    const uint32_t rK = hs.rK, bK = PSS_HF_BINS - 1u - rK;
    if (rK >> 1 == tid) {
        hs.aC = (rK & 1u) ? S0c : S0c - c0;
        hs.aQK = (rK & 1u) ? S0q : S0q - q0;
    }
#pragma unroll
    for (int h = 0; h < HR; ++h)
        if (v[h] && binof(k[h]) == bK) {
            const uint32_t pos = atomicAdd(&hs.bn[0], 1u);
            if (pos < PSS_HF_GATHER) hs.be[0][pos] = e[h];
        }
    __syncthreads();
    const uint32_t mK = hs.bn[0];
    if (mK > PSS_HF_GATHER) return false;
    if (w == 0u) {
        const bool in = lane < mK;
        const uint32_t kk = in ? (uint32_t)(hs.be[0][lane] >> 32) : 0u;
        const uint32_t sk = ~pss_sort64_asc(in ? ~kk : 0xFFFFFFFFu, lane); /* descending, padding 0 last */
        const uint32_t tauK = wave_read_u32(sk, Kc - hs.aC - 1u);
        const uint64_t qi = (lane < mK && sk >= tauK) ? pss_fixq(pss_prob(pss_unkey(sk), tmax)) : 0ull;
        const uint64_t zk = hs.aQK + wave_sum_u64(qi);
        if (lane == 0u) {
            hs.tauK = tauK;
            hs.zk = zk;
        }
    }
    __syncthreads();
    const uint32_t tauK = hs.tauK;
    const uint64_t zk = hs.zk;
    /* 3 */
    uint32_t tau = tauK;
    if (c.useTopP) {
        const uint64_t need = pss_topp_need(c.topP, zk);
        {
            /* bins strictly above the K-th bin hold entries >= tauK only */
            const uint32_t r = (2u * tid < rK && S0q >= need) ? 2u * tid
                                                              : ((2u * tid + 1u < rK && S1q >= need) ? 2u * tid + 1u : 0xFFFFFFFFu);
            const uint32_t rm = wave_min_u32(r);
            if (lane == 0u && rm != 0xFFFFFFFFu) atomicMin(&hs.rP, rm);
        }
        __syncthreads();
        const uint32_t rP = hs.rP < rK ? hs.rP : rK;
        const uint32_t bP = PSS_HF_BINS - 1u - rP;
        if (rP < rK) {
            if (rP >> 1 == tid) hs.aQP = (rP & 1u) ? S0q : S0q - q0;
#pragma unroll
            for (int h = 0; h < HR; ++h)
                if (v[h] && binof(k[h]) == bP) {
                    const uint32_t pos = atomicAdd(&hs.bn[1], 1u);
                    if (pos < PSS_HF_GATHER) hs.be[1][pos] = e[h];
                }
            __syncthreads();
        }
        const uint32_t m = rP < rK ? hs.bn[1] : mK;
        if (m > PSS_HF_GATHER) return false;
        if (w == 0u) {
            const unsigned long long* src = rP < rK ? hs.be[1] : hs.be[0];
            const uint64_t above = rP < rK ? hs.aQP : hs.aQK;
            const bool in = lane < m;
            const uint32_t kk = in ? (uint32_t)(src[lane] >> 32) : 0u;
            const uint32_t sk = ~pss_sort64_asc(in ? ~kk : 0xFFFFFFFFu, lane);
            const uint64_t qi = (lane < m && sk >= tauK) ? pss_fixq(pss_prob(pss_unkey(sk), tmax)) : 0ull;
            const uint64_t P = above + wave_incl_scan_u64(qi);
            const uint64_t hit = __ballot(lane < m && sk >= tauK && P >= need);
            const uint32_t tp = hit ? wave_read_u32(sk, (uint32_t)__ffsll((long long)hit) - 1u) : tauK;
            if (lane == 0u) hs.tauP = tp;
        }
        __syncthreads();
        tau = hs.tauP > tau ? hs.tauP : tau;
    }
    /* 4 */
    bool kp[HR];
    uint64_t z = 0ull;
    uint32_t cnt = 0u, last = 0u;
#pragma unroll
    for (int h = 0; h < HR; ++h) {
        kp[h] = v[h] && k[h] >= tau && (!c.useMinP || p[h] >= c.minP);
        z += kp[h] ? q[h] : 0ull;
        cnt += kp[h] ? 1u : 0u;
        last = kp[h] && (uint32_t)e[h] + 1u > last ? (uint32_t)e[h] + 1u : last;
    }
    z = wave_sum_u64(z);
    cnt = (uint32_t)wave_sum_u64(cnt);
    last = wave_max_u32(last);
    if (lane == 0u) {
        hs.wsq[w] = z;
        hs.wsc[w] = cnt;
        hs.wl[w] = last;
    }
    /* 5, first pass (kept masses by the upper id digit) */
#pragma unroll
    for (int h = 0; h < HR; ++h)
        if (kp[h]) atomicAdd((unsigned long long*)&hs.h8[0][(uint32_t)e[h] >> 9], (unsigned long long)q[h]);
    __syncthreads();
    uint64_t Z = 0ull;
    uint32_t keptCount = 0u, lastAll = 0u;
#pragma unroll
    for (uint32_t x = 0; x < (uint32_t)PSS_WSP_NW; ++x) {
        Z += hs.wsq[x];
        keptCount += hs.wsc[x];
        lastAll = hs.wl[x] > lastAll ? hs.wl[x] : lastAll;
    }
    uint32_t newRng;
    const uint32_t u24 = pss_draw_u24_pre(a.rng_mode, pre.rng, pre.step, row, &newRng);
    const uint64_t target = pss_draw_target(u24, Z);
    uint32_t tok, flags = 0;
    if (Z > 0) {
        if (w == 0u) {
            uint64_t rem = Z - target;
            const uint32_t d1 = pss_hf_digit512(hs.h8[0], rem);
            if (lane == 0u) {
                hs.d1 = d1;
                hs.rem = rem;
            }
        }
        __syncthreads();
        const uint32_t d1 = hs.d1;
#pragma unroll
        for (int h = 0; h < HR; ++h)
            if (kp[h] && ((uint32_t)e[h] >> 9) == d1)
                atomicAdd((unsigned long long*)&hs.h8[1][(uint32_t)e[h] & 511u], (unsigned long long)q[h]);
        __syncthreads();
        if (w == 0u) {
            uint64_t rem = hs.rem;
            const uint32_t d2 = pss_hf_digit512(hs.h8[1], rem);
            if (lane == 0u) hs.tok = (d1 << 9) | d2;
        }
        __syncthreads();
        tok = hs.tok;
    } else {
        tok = lastAll > 0u ? lastAll - 1u : 0u;
        flags |= PSS_INFO_FALLBACK;
    }

    /* verification outputs: zero-fill, wait for it, then set kept ids */
    if (a.kept_mask || a.probs) {
        if (a.kept_mask)
            for (uint32_t wd = tid; wd < a.mask_words; wd += NT) a.kept_mask[(size_t)row * a.mask_words + wd] = 0u;
        if (a.probs)
            for (uint32_t j = tid; j < a.V; j += NT) a.probs[(size_t)row * a.probs_stride + j] = 0.0f;
        pss_wait_mem();
        __syncthreads();
        const float zf = (float)Z * 0x1.0p-45f;
#pragma unroll
        for (int h = 0; h < HR; ++h)
            if (kp[h]) {
                const uint32_t id = (uint32_t)e[h];
                if (a.kept_mask) atomicOr(&a.kept_mask[(size_t)row * a.mask_words + (id >> 5)], 1u << (id & 31u));
                if (a.probs) a.probs[(size_t)row * a.probs_stride + id] = p[h] / zf;
            }
    }
    if (tid == 0) {
        pss_row_info inf = {};
        inf.token = tok;
        inf.kept_count = keptCount;
        inf.tau_key = tau;
        inf.tmax_key = tmaxKey;
        inf.z_kept = Z;
        inf.z_topk = zk;
        inf.target = target;
        inf.u24 = u24;
        inf.flags = flags;
        pss_epilogue_pre(a, row, tok, false, c.W, newRng, inf, pre.pos, pre.step);
    }
    return true;
}

/* ------------------------------------------------------------------------ */
/* split-row wide kernel                                                     */
/* ------------------------------------------------------------------------ */

#define PSS_WSP_DEPTH 4    /* loads a wave keeps in flight */
#define PSS_WSP_SCAP 2048u /* candidates a segment stages in LDS */

template <int DT>
union pss_wsp_shared {
    struct {
        uint32_t winbits[pss_wsp_geom<DT>::SBW];   /* window ids of the segment */
        unsigned long long stage[PSS_WSP_SCAP];    /* the segment's candidates, in claim order */
        uint32_t lk[PSS_WSP_NW];                   /* per wave: ceil(K / nf)-th largest */
        uint32_t l2[PSS_WSP_NW];                   /* per wave: ceil(ceil(K / G) / nf)-th largest */
        unsigned long long best[PSS_WSP_NW];       /* greedy rows: each wave's (key << 32) | ~id */
        uint32_t ncl;                              /* candidates claimed (may exceed the stage) */
    } s;
    struct {
        pss_fin_shared fs; /* gathered list + finisher scratch */
        union {
            uint32_t bits[PSS_MAX_VOCAB / 32]; /* the general algorithm's penalty bitmap */
            pss_hfin_shared hs;                /* the histogram finisher */
        } u;
    } f;
};

/* Pool entries per segment: an equal share of the row's pool, a multiple of
 * 16 (each range starts on a 128-byte line). */
__host__ __device__ __forceinline__ uint32_t pss_wsp_capg(uint32_t G) { return (PSS_POOL_CAP / G) & ~15u; }

template <int DT>
__global__ void __launch_bounds__(PSS_WSP_NT) pss_wsplit_kernel(pss_args a, uint32_t G,
                                                                const sample_params* __restrict__ params) {
    using Gm = pss_wsp_geom<DT>;
    constexpr int E = Gm::E, NL = Gm::NL, D = PSS_WSP_DEPTH;
    constexpr uint32_t esz = DT == PSS_DTYPE_F16 ? 2u : 4u;
    __shared__ pss_wsp_shared<DT> S;
    __shared__ uint32_t last;
    pss_globalize(a);
    if (pss_gate_closed(a)) return;
    const uint32_t row = blockIdx.x / G, g = blockIdx.x - row * G;
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63u;
    pss_row_ws* ws = (pss_row_ws*)((char*)a.ws + (size_t)row * PSS_WS_ROW_BYTES);
    const uint32_t capg = pss_wsp_capg(G);
    const uint32_t cap = capg < PSS_WSP_SCAP ? capg : PSS_WSP_SCAP;
    unsigned long long* pool = (unsigned long long*)(ws + 1) + (size_t)g * capg;

    /* 1. requests: the window id of this thread (the history row always
     * holds PSS_MAX_PENALTY_LEN slots) and the row's parameters, then the
     * segment's first D loads; one more load is requested before each wait */
    static_assert(PSS_MAX_PENALTY_LEN <= PSS_WSP_NT, "one window slot per thread");
    const uint32_t hid = tid < PSS_MAX_PENALTY_LEN ? a.history[(size_t)row * PSS_MAX_PENALTY_LEN + tid] : PSS_SENTINEL;
    sample_params sp = params[row];
    /* the row state, for the finishing workgroup (written only by its epilogue) */
    pss_row_pre pre;
    pre.rng = a.rng[row];
    pre.step = a.step[row];
    pre.pos = a.position[row];
    __asm__ __volatile__("" ::: "memory");
    /* the row's waves of WSPAN ids, split evenly over the G segments (at
     * most 16 each); the resource covers the segment only, so loads beyond
     * it return 0 without reading memory */
    const uint32_t V = a.V;
    const uint32_t NWV = (V + Gm::WSPAN - 1u) / Gm::WSPAN;
    const uint32_t wa = g * NWV / G, wb = (g + 1u) * NWV / G;
    const uint32_t seg0 = wa * Gm::WSPAN;
    const uint32_t segEnd = wb * Gm::WSPAN < V ? wb * Gm::WSPAN : V;
    const uint32_t nfull = (segEnd - seg0) / Gm::WSPAN; /* waves whose ids are all in the segment */
    const uint32_t idw = seg0 + wave * Gm::WSPAN;
    const __amdgpu_buffer_rsrc_t rrs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((const char*)a.logits + ((size_t)row * a.stride + seg0) * esz), (short)0, (int)((segEnd - seg0) * esz),
        PSS_BUF_DW3);
    const uint32_t vb = wave * Gm::WSPAN * esz + lane * 16u;
    uint4 raw[NL];
    auto ld = [&](int j) {
        raw[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rrs, (int)(vb + 1024u * (uint32_t)j), 0, PSS_NT));
    };
#pragma unroll
    for (int j = 0; j < D; ++j) ld(j);
    pss_pin_s(sp.temperature);
    pss_pin_s(sp.repPenalty);
    pss_pin_s(sp.penaltyLength);
    pss_pin_s(sp.topK);
    pss_pin_s(sp.topP);
    pss_pin_s(sp.minP);
    pss_pin_s(sp.presencePenalty);
    const float NEG_INF = pss_u2f(0xFF800000u);
    pss_rowcfg c = pss_make_rowcfg(sp, V);
    c.invT = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(c.invT)));
    const bool greedy = pss_seg_row_greedy(a, sp);
    const bool cov = !greedy && c.K >= 1u && c.K <= PSS_WIDE_KMAX;
    const bool doPen = cov && c.doPen;
    const float invT = c.invT;

    /* 2. the window bitmap of the segment (while the first loads arrive) */
    if (doPen)
        for (uint32_t i = tid; i < Gm::SBW; i += PSS_WSP_NT) S.s.winbits[i] = 0u;
    if (tid == 0u) S.s.ncl = 0u;
    __syncthreads();
    bool own = false;
    if (doPen && tid < c.W && hid < V && hid - seg0 < segEnd - seg0) {
        const uint32_t bit = 1u << (hid & 31u);
        own = !(atomicOr(&S.s.winbits[(hid - seg0) >> 5], bit) & bit);
    }
    /* every thread requests (uniform wait counts below); owners' values used */
    const uint32_t wraw = __builtin_amdgcn_raw_buffer_load_b32(rrs, (int)(((own ? hid - seg0 : 0u) * esz) & ~3u), 0, 0);
    __syncthreads();

    /* 3. the loads in arrival order */
    float t0 = NEG_INF, t1 = NEG_INF, t2 = NEG_INF, t3 = NEG_INF;
    uint64_t best = 0ull;
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        if (j + D < NL) ld(j + D);
        uint4& r = raw[j];
        const uint32_t id0 = idw + (uint32_t)j * Gm::LSPAN + lane * (uint32_t)E;
        if (id0 + (uint32_t)E > segEnd) {
#pragma unroll
            for (int e = 0; e < E; ++e)
                if (id0 + (uint32_t)e >= segEnd) pss_res_kill<DT>(r, e);
        }
        if (greedy) {
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const uint64_t b = ((uint64_t)pss_key(pss_canon(pss_res_t<DT>(r, e, 1.0f))) << 32) |
                                   (uint64_t)(0xFFFFFFFFu - (id0 + (uint32_t)e));
                best = b > best ? b : best;
            }
        } else if (cov) {
            if (DT == PSS_DTYPE_F32) {
                r.x = __float_as_uint(__uint_as_float(r.x) * invT);
                r.y = __float_as_uint(__uint_as_float(r.y) * invT);
                r.z = __float_as_uint(__uint_as_float(r.z) * invT);
                r.w = __float_as_uint(__uint_as_float(r.w) * invT);
            }
            if (doPen) {
                const uint32_t o = id0 - seg0;
                const uint32_t wb = S.s.winbits[o >> 5] >> (o & 31u);
                if (wb & ((1u << E) - 1u)) {
#pragma unroll
                    for (int e = 0; e < E; ++e)
                        if ((wb >> e) & 1u) pss_res_kill<DT>(r, e);
                }
            }
            /* the lane's four largest (NaN canonicalizes to -inf) */
#pragma unroll
            for (int e = 0; e < E; ++e) {
                float x = fmaxf(pss_res_t<DT>(r, e, invT), NEG_INF), y;
                y = fminf(t0, x);
                t0 = fmaxf(t0, x);
                x = y;
                y = fminf(t1, x);
                t1 = fmaxf(t1, x);
                x = y;
                y = fminf(t2, x);
                t2 = fmaxf(t2, x);
                x = y;
                t3 = fmaxf(t3, x);
            }
        }
    }

    if (greedy) {
        best = wave_max_u64(best);
        if (lane == 0u) S.s.best[wave] = best;
        __syncthreads();
        if (tid == 0u) {
            uint64_t b = S.s.best[0];
#pragma unroll
            for (int v = 1; v < PSS_WSP_NW; ++v) b = S.s.best[v] > b ? S.s.best[v] : b;
            pss_st_agent64(&ws->seg_best[g], b);
        }
    } else if (cov) {
        /* 4. certificates over the segment's full waves (nfull of them, each
         * certifying kq of its 256 values; a wave certifies at most 256).
         * LK resolves 24 bits; L2, only the finisher's filter, 16. */
        const uint32_t k4[4] = {pss_key(pss_canon(t0)), pss_key(pss_canon(t1)), pss_key(pss_canon(t2)),
                                pss_key(pss_canon(t3))};
        const uint32_t nf = nfull ? nfull : 1u;
        const uint32_t kq = (c.K + nf - 1u) / nf;
        const uint32_t kg = (c.K + G - 1u) / G;
        const uint32_t kq2 = (kg + nf - 1u) / nf;
        uint32_t lk = 0xFFFFFFFFu, l2 = 0xFFFFFFFFu;
        if (wave < nfull) {
            lk = kq <= 256u ? wave_kth_largest<4, 24>(k4, kq) : 0u;
            l2 = kq2 <= 256u ? pss_wave_kth16<4>(k4, kq2) : 0u;
        }
        if (nfull == 0u) lk = l2 = 0u;
        if (lane == 0u) {
            S.s.lk[wave] = lk;
            S.s.l2[wave] = l2;
        }
        __syncthreads();
        uint32_t LK = S.s.lk[0], L2 = S.s.l2[0];
#pragma unroll
        for (int v = 1; v < PSS_WSP_NW; ++v) {
            LK = min(LK, S.s.lk[v]);
            L2 = min(L2, S.s.l2[v]);
        }
        LK = __builtin_amdgcn_readfirstlane(LK);
        L2 = __builtin_amdgcn_readfirstlane(L2);
        /* 5. candidates: a pass mask per lane, one claim per wave, the
         * entries staged in LDS, then copied to the pool with coalesced
         * stores.  With no finite bound every element would pass: the
         * segment reports an overflow (general algorithm). */
        uint32_t n = 0xFFFFFFFFu;
        if (LK > PSS_KEY_NEG_INF) {
            if (tid == 0u) (void)__hip_atomic_fetch_max(&ws->bound, LK, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const float thr = pss_unkey(LK);
            static_assert(NL * E == 64, "one mask bit per element of a lane");
            uint64_t pm = 0ull;
#pragma unroll
            for (int j = 0; j < NL; ++j)
#pragma unroll
                for (int e = 0; e < E; ++e)
                    pm |= (pss_res_t<DT>(raw[j], e, invT) >= thr ? 1ull : 0ull) << (j * E + e);
            unsigned long long went = 0ull;
            bool wk = false;
            if (own) {
                float x;
                if (DT == PSS_DTYPE_F16) {
                    const uint16_t h = (uint16_t)(wraw >> ((hid & 1u) * 16u));
                    _Float16 hf;
                    __builtin_memcpy(&hf, &h, 2);
                    x = (float)hf;
                } else {
                    x = __uint_as_float(wraw);
                }
                const uint32_t k = pss_key(pss_canon(pss_penalize(x * invT, c)));
                wk = k >= LK;
                went = ((unsigned long long)k << 32) | hid;
            }
            const uint32_t mine = (uint32_t)__popcll(pm) + (wk ? 1u : 0u);
            const uint32_t incl = wave_incl_scan_u32(mine);
            const uint32_t tot = wave_read_u32(incl, 63u);
            uint32_t b0 = 0u;
            if (lane == 0u && tot) b0 = atomicAdd(&S.s.ncl, tot);
            uint32_t o = __builtin_amdgcn_readfirstlane(b0) + incl - mine;
            if (wk) {
                if (o < PSS_WSP_SCAP) S.s.stage[o] = went;
                ++o;
            }
            /* per load, the lanes' set bits one at a time (a lane rarely
             * has more than one element of a load at or above the bound) */
            const uint32_t lid = idw + lane * (uint32_t)E;
            uint32_t* st32 = (uint32_t*)S.s.stage;
#pragma clang loop unroll(full)
            for (int j = 0; j < NL; ++j) {
                uint32_t lm = (uint32_t)(pm >> (j * E)) & ((1u << E) - 1u);
                const uint32_t w0 = raw[j].x, w1 = raw[j].y, w2 = raw[j].z, w3 = raw[j].w;
                while (__ballot(lm != 0u) != 0ull) {
                    if (lm) {
                        const uint32_t e = (uint32_t)__builtin_ctz(lm);
                        lm &= lm - 1u;
                        /* the word holding element e: a select tree over
                         * the four words (no indexed access) */
                        const uint32_t sb = DT == PSS_DTYPE_F16 ? e >> 1 : e;
                        const uint32_t lo = (sb & 1u) ? w1 : w0, hi = (sb & 1u) ? w3 : w2;
                        const uint32_t wd = (sb & 2u) ? hi : lo;
                        float te;
                        if (DT == PSS_DTYPE_F16) {
                            const uint16_t h = (uint16_t)(wd >> ((e & 1u) * 16u));
                            _Float16 hf;
                            __builtin_memcpy(&hf, &h, 2);
                            te = (float)hf * invT;
                        } else {
                            te = __uint_as_float(wd);
                        }
                        if (o < PSS_WSP_SCAP) {
                            st32[2u * o] = lid + (uint32_t)j * Gm::LSPAN + e;
                            st32[2u * o + 1u] = pss_key(pss_canon(te));
                        }
                        ++o;
                    }
                }
            }
            __syncthreads();
            n = S.s.ncl;
            if (n <= cap)
                for (uint32_t i = tid; i < n; i += PSS_WSP_NT) pss_st_agent64(pool + i, S.s.stage[i]);
        }
        if (tid == 0u) {
            pss_st_agent(&ws->seg_count[g], n <= cap ? n : PSS_SEG_OVERFLOW);
            pss_st_agent64(&ws->seg_best[g], (unsigned long long)L2);
        }
    }

    /* 6. the ticket */
    pss_wait_mem(); /* this wave's pool stores and counts have completed */
    __syncthreads();
    if (tid == 0u) {
        const bool l = __hip_atomic_fetch_add(&ws->ticket, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == G - 1u;
        if (l) pss_st_agent(&ws->ticket, 0u); /* every other workgroup of the row has counted */
        last = l ? 1u : 0u;
    }
    __syncthreads();
    if (!last) return;

    /* the finishing workgroup: its scratch overlays the segment's */
    pss_fin_shared& sh = S.f.fs;
    if (greedy) {
        uint64_t b = 0ull;
        for (uint32_t s = 0; s < G; ++s) {
            const uint64_t v = pss_ld_agent64(&ws->seg_best[s]);
            b = v > b ? v : b;
        }
        pss_greedy_finish<PSS_WSP_NT>(a, row, b);
        return;
    }
    bool general = !cov;
    if (!general) {
        /* counts, bounds and candidates in one round trip: every thread
         * reads the G (<= 4) counts and bounds and its share of each
         * segment's whole staged range (entries beyond a count are dropped) */
        static_assert(PSS_MAX_VOCAB <= 4u * 65536u, "at most 4 segments");
        constexpr int PS = (int)(PSS_WSP_SCAP / PSS_WSP_NT); /* entries per thread and segment */
        constexpr int GR = 4 * PS;
        const unsigned long long* rowpool = (const unsigned long long*)(ws + 1);
        uint32_t ns[4];
        uint32_t L2min = 0xFFFFFFFFu;
#pragma unroll
        for (uint32_t s = 0; s < 4u; ++s) {
            ns[s] = 0u;
            if (s < G) {
                ns[s] = pss_ld_agent(&ws->seg_count[s]);
                const uint32_t l2 = (uint32_t)pss_ld_agent64(&ws->seg_best[s]);
                L2min = l2 < L2min ? l2 : L2min;
            }
        }
        const uint32_t B = pss_ld_agent(&ws->bound);
        unsigned long long ev[GR];
#pragma unroll
        for (int r = 0; r < GR; ++r) {
            const uint32_t sg = (uint32_t)(r / PS), i = (uint32_t)(r % PS) * PSS_WSP_NT + tid;
            ev[r] = (sg < G && i < cap) ? pss_ld_agent64(rowpool + (size_t)sg * capg + i) : 0ull;
        }
        bool over = false;
#pragma unroll
        for (uint32_t s = 0; s < 4u; ++s) over |= s < G && ns[s] == PSS_SEG_OVERFLOW;
        const uint32_t thr2 = B > L2min ? B : L2min;
        if (tid < 256u) sh.f.hist[0][tid] = sh.f.hist[1][tid] = 0u;
        if (tid == 0u) {
            sh.f.nc = 0u;
            sh.f.nk = 0u;
            sh.f.hflag = 0u;
        }
        /* top-k above the fast finisher's: the histogram finisher's bins
         * cleared under the same barrier */
        const bool hf = c.K > PSS_SEG_KMAX;
        if (hf) pss_hist_clear(S.f.u.hs);
        __syncthreads();
        general = over;
        if (!general) {
            uint32_t mk = 0u;
#pragma unroll
            for (int r = 0; r < GR; ++r) {
                const uint32_t sg = (uint32_t)(r / PS), i = (uint32_t)(r % PS) * PSS_WSP_NT + tid;
                if (sg >= G) break;
                const unsigned long long e = ev[r];
                const bool keep = i < ns[sg] && (uint32_t)(e >> 32) >= thr2;
                const uint64_t m = __ballot(keep);
                if (m) {
                    uint32_t b0 = 0u;
                    if (lane == 0u) b0 = atomicAdd(&sh.f.nc, (uint32_t)__popcll(m));
                    const uint32_t pos = __builtin_amdgcn_readfirstlane(b0) +
                                         __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
                    if (keep && pos < PSS_FIN_LIST_CAP) sh.list[pos] = e;
                    const uint32_t k = (uint32_t)(e >> 32);
                    mk = keep && k > mk ? k : mk;
                }
            }
            mk = wave_max_u32(mk);
            if (lane == 0u) sh.f.mx[wave] = mk;
            __syncthreads();
            const uint32_t n = sh.f.nc;
            general = n > PSS_FIN_LIST_CAP || n == 0u;
            if (!general) {
                pss_pin_s(pre.rng);
                pss_pin_s(pre.step);
                pss_pin_s(pre.pos);
                if (!pss_list_finish_fast<PSS_WSP_NT>(a, row, c, sh.list, n, thr2, pre, sh.f, true)) {
                    uint32_t tmaxKey = 0u;
#pragma unroll
                    for (int v = 0; v < PSS_WSP_NW; ++v) tmaxKey = sh.f.mx[v] > tmaxKey ? sh.f.mx[v] : tmaxKey;
                    if (n > PSS_HF_N || !pss_hist_finish(a, row, c, sh.list, n, thr2, tmaxKey, pre, S.f.u.hs, hf))
                        pss_list_finish<PSS_WSP_NT>(a, row, c, sh.list, n, sh.f.g, thr2);
                }
            }
        }
    }
    if (tid == 0u) pss_st_agent(&ws->bound, 0u); /* for the next launch */
    if (general) pss_general_row<PSS_WSP_NT>(a, row, sh.f.g, S.f.u.bits, PSS_MAX_VOCAB / 32);
}

/* Segments per row (0: the row does not fit this form). */
static inline uint32_t pss_wsplit_segments(uint32_t V) {
    return V <= PSS_MAX_VOCAB ? (V + 65535u) / 65536u : 0u;
}

static inline hipError_t pss_wsplit_launch(pss_args a, uint32_t rows, hipStream_t st) {
    const uint32_t G = pss_wsplit_segments(a.V);
    a.kmax_cov = PSS_WIDE_KMAX;
    a.wmax_cov = PSS_MAX_PENALTY_LEN;
    a.vec_ok = 1u;
    const dim3 grid(rows * G), block(PSS_WSP_NT);
    if (a.dtype == PSS_DTYPE_F16)
        pss_wsplit_kernel<PSS_DTYPE_F16><<<grid, block, 0, st>>>(a, G, a.params);
    else
        pss_wsplit_kernel<PSS_DTYPE_F32><<<grid, block, 0, st>>>(a, G, a.params);
    return hipGetLastError();
}

#endif /* PSS_WIDE_H */
