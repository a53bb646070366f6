/*
 * pss_stream.h - the streaming sampler (the HBM-roofline path).
 *
 * The rows are cut into items of 64 * EPT consecutive ids, processed in
 * rounds by workgroups of PSS_SEG_NW independent waves (one item per wave per
 * round): each item is read once with 16-byte buffer loads straight into the
 * wave's LDS staging area, one round ahead of its compute; window ids are
 * applied once per id by the lane that claims them; every element at or
 * above a certified lower bound of the row's K-th largest value (from the
 * waves' running top values, combined across the workgroup through LDS
 * slots) becomes a candidate.  Two forms:
 *
 * pss_row_kernel (default), one workgroup per row: candidates gather in an
 * LDS list and the workgroup finishes the row itself after its last round --
 * exact K-th largest, masses q = trunc(exp(t - tmax) * 2^45), top-p, min-p,
 * the draw as an ascending-id inverse CDF over the kept set, the epilogue
 * (result slot, token, window, rng, position).
 *
 * pss_seg_kernel + pss_fin_kernel (PSS_ENQ_SPLIT): workgroups over any range
 * of items, candidates into per-item slots of a per-row pool in HBM (rows
 * split across workgroups share a row-wide bound through a relaxed atomic
 * max); then one workgroup per row gathers the candidates and runs the same
 * finisher.
 *
 * Rows the candidates cannot finish (top-k off or above PSS_SEG_KMAX, a window
 * above PSS_SEG_WMAX ids, heavy ties, an overflowing list) run the general
 * algorithm in the finishing workgroup, re-reading the row.  Every path
 * computes the same bits as the one-workgroup-per-row general kernel.
 */
#ifndef PSS_STREAM_H
#define PSS_STREAM_H

#include "pss_general.h"

#define PSS_ST_NT 256
#define PSS_SEG_NW 16            /* waves per segment workgroup: one item each per round */
#define PSS_SEG_NT (PSS_SEG_NW * PSS_WAVE)
#define PSS_ROW_LIST_CAP 2048u   /* fused form: candidates a workgroup gathers in LDS */
#define PSS_ROW_BITS 8192u       /* fused form: penalty-bitmap words of the general algorithm */
#define PSS_SEG_KMAX 256u        /* largest top-k the segment kernel covers (running top-4 per lane) */
#define PSS_SEG_WMAX 256u        /* largest window the segment kernel covers (four ids per lane) */
#define PSS_WIDE_KMAX 1024u      /* largest top-k of the wide fused form (running top-4, 16 waves) */
#define PSS_WIDE_LIST_CAP 8192u  /* the wide fused form's LDS candidate list */
#define PSS_SEG_MAX_SLOTS 256u   /* items per row (V <= 262144 at items >= 1024 ids) */
#define PSS_POOL_CAP 16384u      /* pool entries per row, split evenly over its items */
#define PSS_FIN_LIST_CAP 4096u   /* candidates the finisher gathers in LDS */
#define PSS_FAST_N 1024u         /* candidates the fast finisher handles (K <= PSS_SEG_KMAX) */
#define PSS_KEPT_CAP 256u        /* entries at or above the K-th largest the fast finisher handles */
#define PSS_SEG_OVERFLOW 0xFFFFFFFFu
#define PSS_KEY_NEG_INF 0x007FFFFFu /* pss_key(-inf): the smallest key of any element */

/* Per-row workspace: header, then the candidate pool. */
struct pss_row_ws {
    uint32_t bound;  /* row-wide lower bound on the K-th largest key (max over items) */
    uint32_t ticket; /* small-batch form: workgroups of the row done so far */
    uint32_t pad[30];
    uint32_t seg_count[PSS_SEG_MAX_SLOTS];          /* candidates per item, or PSS_SEG_OVERFLOW */
    unsigned long long seg_best[PSS_SEG_MAX_SLOTS]; /* greedy rows: (key << 32) | ~id per item */
};
static_assert(sizeof(pss_row_ws) % 128 == 0, "workspace header is a multiple of 128 bytes");
#define PSS_WS_ROW_BYTES (sizeof(pss_row_ws) + (size_t)PSS_POOL_CAP * 8u)

/* Pool entries per item: an equal share of the pool, a multiple of 16 (each
 * item's range starts on a 128-byte line; at least 64 for NS <= 256). */
__host__ __device__ __forceinline__ uint32_t pss_pool_capw(uint32_t NS) { return (PSS_POOL_CAP / NS) & ~15u; }
#define PSS_FIN_SPEC 16u /* pool entries per item the finisher loads with the counts */

static inline size_t pss_stream_ws_bytes(uint32_t rows) { return (size_t)rows * PSS_WS_ROW_BYTES; }

/* Workspace accesses that other workgroups of the same launch may read:
 * agent-scope (coherent across the XCDs' L2 caches) relaxed atomics, so a
 * store is visible to every workgroup once the storing wave's memory counter
 * has drained, and a load sees it without any cache maintenance. */
__device__ __forceinline__ uint32_t pss_ld_agent(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long pss_ld_agent64(const unsigned long long* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void pss_st_agent(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void pss_st_agent64(unsigned long long* p, unsigned long long v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* ------------------------------------------------------------------------ */
/* finisher: selection over the row's candidate list in LDS                  */
/* ------------------------------------------------------------------------ */

/* Fused form: the workgroup's candidate list and row-level values. */
template <uint32_t CAP>
struct pss_row_lds_t {
    static constexpr uint32_t cap = CAP;
    unsigned long long list[CAP]; /* (key << 32) | id */
    unsigned long long best;      /* greedy rows: (key << 32) | ~id */
    uint32_t n;                   /* entries claimed (may exceed the capacity) */
    uint32_t bound;               /* largest certified bound of the row */
};
using pss_row_lds = pss_row_lds_t<PSS_ROW_LIST_CAP>;

/* Finisher scratch besides the candidate list. */
struct pss_fin_small {
    unsigned long long cl[PSS_FAST_N]; /* fast path: entries at or above the row bound */
    unsigned long long kept[PSS_KEPT_CAP]; /* fast path: entries at or above the K-th largest */
    uint32_t hist[2][256];             /* fast path: radix digit counts (alternate passes) */
    pss_gen_shared g;
    uint32_t mx[PSS_SEG_NW];           /* per-wave largest key */
    uint32_t digit;
    uint32_t rem;
    uint32_t cum;
    uint32_t hd;
    uint32_t nc;
    uint32_t nk;
    uint32_t fail;
    uint64_t gtot; /* finisher gather totals (overflowed, not filtered, entries) */
    uint32_t g2;   /* finisher: the row bound after the small form's per-item maxima */
    /* two-wave tail: the key-order results wave 0 hands to wave 1 (hflag
     * is cleared with nk, before the caller's last barrier) */
    uint32_t hflag;
    uint32_t htau;
    uint32_t htmax;
    uint64_t hzk;
};

struct pss_fin_shared {
    unsigned long long list[PSS_FIN_LIST_CAP]; /* gathered candidates (key << 32 | id) */
    pss_fin_small f;
};

/*
 * Select by cumulative weight from the top over the list: kw(e, key, w) gives
 * entry e's selection key and weight (w = 0 skips it).  Returns the largest
 * key v with sum_{key >= v} w >= rem (1 <= rem <= total weight).  Digits of 8
 * bits from bit top_shift + 7 down; 256-bin LDS histograms.  Every weighted
 * key shares its bits above top_shift + 7 with `above` (the callers start
 * below the common prefix of a lower bound and the maximum, so the first
 * digit spreads over bins instead of piling onto one).
 */
template <int NT, class KW>
__device__ __forceinline__ uint32_t pss_list_select(pss_gen_shared& sh, const unsigned long long* list,
                                                    uint32_t n, uint64_t rem, int top_shift, uint32_t above,
                                                    KW kw) {
    const uint32_t tid = threadIdx.x;
    uint32_t pmask = top_shift + 8 >= 32 ? 0u : ~((1u << (top_shift + 8)) - 1u);
    uint32_t prefix = above & pmask;
    for (int shift = top_shift; shift >= 0; shift -= 8) {
        for (uint32_t i = tid; i < 256u; i += NT) sh.hist[i] = 0;
        __syncthreads();
        for (uint32_t i = tid; i < n; i += NT) {
            uint32_t k;
            uint64_t w;
            kw(list[i], k, w);
            if (w && (k & pmask) == prefix)
                atomicAdd((unsigned long long*)&sh.hist[(k >> shift) & 255u], (unsigned long long)w);
        }
        __syncthreads();
        if (tid < 64) wave0_pick_digit(sh.hist, rem, &sh.digit, &sh.rem);
        __syncthreads();
        prefix |= sh.digit << shift;
        pmask |= 0xFFu << shift;
        rem = sh.rem;
        __syncthreads();
    }
    return prefix;
}

/* First digit shift for a select between lower bound lo and maximum hi
 * (lo <= hi): below their common prefix; -1 when they are equal. */
__device__ __forceinline__ int pss_select_shift(uint32_t lo, uint32_t hi) {
    const uint32_t d = lo ^ hi;
    return d ? ((31 - (int)__clz(d)) / 8) * 8 : -1;
}

/* Finish a sampled row from n candidates (LDS) that contain every element at
 * or above the row's K-th largest value; G is a lower bound on that value
 * with at least K candidates at or above it (0: none known).  Any K, any
 * number of ties. */
template <int NT>
__device__ __forceinline__ void pss_list_finish(const pss_args& a, uint32_t row, const pss_rowcfg& c,
                                                const unsigned long long* list, uint32_t n,
                                                pss_gen_shared& sh, uint32_t G) {
    const uint32_t tid = threadIdx.x;
    uint64_t mk = 0;
    for (uint32_t i = tid; i < n; i += NT) {
        const uint64_t k = list[i] >> 32;
        mk = k > mk ? k : mk;
    }
    const uint32_t tmaxKey = (uint32_t)block_max_u64<NT>(mk, sh.red);
    const float tmax = pss_unkey(tmaxKey);

    /* S5: exact K-th largest, over the candidates at or above G */
    const uint32_t g = G <= tmaxKey ? G : 0u;
    const int shK = pss_select_shift(g, tmaxKey);
    const uint32_t tauK = shK < 0 ? tmaxKey
                                  : pss_list_select<NT>(sh, list, n, c.K, shK, tmaxKey,
                                                        [&](unsigned long long e, uint32_t& k, uint64_t& w) {
                                                            k = (uint32_t)(e >> 32);
                                                            w = k >= g ? 1u : 0u;
                                                        });
    auto qof = [&](uint32_t k) -> uint64_t { return pss_fixq(pss_prob(pss_unkey(k), tmax)); };
    uint64_t zl = 0;
    for (uint32_t i = tid; i < n; i += NT) {
        const uint32_t k = (uint32_t)(list[i] >> 32);
        if (k >= tauK) zl += qof(k);
    }
    const uint64_t zk = block_sum_u64<NT>(zl, sh.red);

    /* S6 */
    uint32_t tau = tauK;
    if (c.useTopP) {
        const uint64_t need = pss_topp_need(c.topP, zk);
        const int shP = pss_select_shift(tauK, tmaxKey);
        const uint32_t tauP = shP < 0 ? tmaxKey
                                      : pss_list_select<NT>(sh, list, n, need, shP, tmaxKey,
                                                            [&](unsigned long long e, uint32_t& k, uint64_t& w) {
                                                                k = (uint32_t)(e >> 32);
                                                                w = k >= tauK ? qof(k) : 0u;
                                                            });
        tau = tauP > tau ? tauP : tau;
    }

    /* S7 */
    auto kept = [&](unsigned long long e, uint64_t* q, float* p) -> bool {
        const uint32_t k = (uint32_t)(e >> 32);
        *p = pss_prob(pss_unkey(k), tmax);
        const bool kp = k >= tau && (!c.useMinP || *p >= c.minP);
        *q = kp ? pss_fixq(*p) : 0u;
        return kp;
    };
    uint64_t zs = 0;
    uint32_t cnt = 0, lastKept = 0;
    for (uint32_t i = tid; i < n; i += NT) {
        const unsigned long long e = list[i];
        uint64_t q;
        float p;
        if (kept(e, &q, &p)) {
            zs += q;
            cnt++;
            const uint32_t id1 = (uint32_t)e + 1u;
            lastKept = id1 > lastKept ? id1 : lastKept;
        }
    }
    const uint64_t Z = block_sum_u64<NT>(zs, sh.red);
    const uint32_t keptCount = (uint32_t)block_sum_u64<NT>(cnt, sh.red);
    const uint32_t lastAll = (uint32_t)block_max_u64<NT>(lastKept, sh.red);

    /* S8: the smallest id whose cumulative kept mass exceeds the target is the
     * largest id v with sum_{id >= v} q >= Z - target. */
    uint32_t newRng;
    const uint32_t u24 = pss_draw_u24(a, row, &newRng);
    const uint64_t target = pss_draw_target(u24, Z);
    uint32_t tok, flags = 0;
    if (Z > 0) {
        tok = pss_list_select<NT>(sh, list, n, Z - target, 16, 0u,
                                  [&](unsigned long long e, uint32_t& k, uint64_t& w) {
                                      float p;
                                      k = (uint32_t)e;
                                      kept(e, &w, &p);
                                  });
    } else {
        tok = lastAll > 0u ? lastAll - 1u : 0u;
        flags |= PSS_INFO_FALLBACK;
    }

    /* verification outputs: zero-fill, wait for it, then set kept ids */
    if (a.kept_mask || a.probs) {
        if (a.kept_mask)
            for (uint32_t w = tid; w < a.mask_words; w += NT) a.kept_mask[(size_t)row * a.mask_words + w] = 0u;
        if (a.probs)
            for (uint32_t j = tid; j < a.V; j += NT) a.probs[(size_t)row * a.probs_stride + j] = 0.0f;
        pss_wait_mem();
        __syncthreads();
        const float zf = (float)Z * 0x1.0p-45f;
        for (uint32_t i = tid; i < n; i += NT) {
            const unsigned long long e = list[i];
            uint64_t q;
            float p;
            if (!kept(e, &q, &p)) continue;
            const uint32_t id = (uint32_t)e;
            if (a.kept_mask) atomicOr(&a.kept_mask[(size_t)row * a.mask_words + (id >> 5)], 1u << (id & 31u));
            if (a.probs) a.probs[(size_t)row * a.probs_stride + id] = p / zf;
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
        pss_epilogue(a, row, tok, false, c.W, newRng, inf);
    }
}

/* Row state the finisher needs, loaded at kernel start together with the
 * candidate counts so that none of it is a separate round trip later. */
struct pss_row_pre {
    uint32_t rng;
    uint32_t step;
    uint32_t pos;
};

/*
 * One wave, no barriers: the largest key v with sum_{key >= v} w >= rem
 * (1 <= rem <= total weight) over the R (key, weight) pairs of each lane.
 * Digits of 8 bits from bit top_shift + 7 down, every weighted key sharing
 * its bits above that with `above`; the histogram is 256 u64 of LDS the wave
 * owns (a wave's LDS operations complete in order, so no wait is needed
 * between clearing, adding and reading).
 */
template <int R>
__device__ __forceinline__ uint32_t pss_wave_wselect(const uint32_t (&k)[R], const uint64_t (&w)[R], uint64_t rem,
                                                     int top_shift, uint32_t above, uint64_t* hist) {
    const uint32_t lane = pss_tid() & 63u;
    uint32_t pmask = top_shift + 8 >= 32 ? 0u : ~((1u << (top_shift + 8)) - 1u);
    uint32_t prefix = above & pmask;
    for (int shift = top_shift; shift >= 0; shift -= 8) {
#pragma unroll
        for (int i = 0; i < 4; ++i) hist[4u * lane + (uint32_t)i] = 0ull;
        __asm__ __volatile__("" ::: "memory");
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (w[r] && (k[r] & pmask) == prefix)
                atomicAdd((unsigned long long*)&hist[(k[r] >> shift) & 255u], (unsigned long long)w[r]);
        __asm__ __volatile__("" ::: "memory");
        const uint64_t h[4] = {hist[4u * lane], hist[4u * lane + 1u], hist[4u * lane + 2u], hist[4u * lane + 3u]};
        const uint64_t s4 = h[0] + h[1] + h[2] + h[3];
        const uint64_t incl = wave_incl_suffix_u64(s4); /* lanes >= lane */
        const uint64_t abv = incl - s4;                  /* lanes > lane */
        const bool hit = abv < rem && rem <= incl;
        uint32_t dg = 0u;
        uint64_t cum = abv;
        if (hit) {
            dg = 4u * lane;
            for (int i = 3; i >= 0; --i) {
                if (cum + h[i] >= rem) {
                    dg = 4u * lane + (uint32_t)i;
                    break;
                }
                cum += h[i];
            }
        }
        const uint32_t src = (uint32_t)__ffsll((long long)__ballot(hit)) - 1u;
        prefix |= wave_read_u32(dg, src) << shift;
        pmask |= 0xFFu << shift;
        rem -= wave_read_u64(cum, src);
    }
    return prefix;
}

/*
 * Finisher tail for 65..256 entries (src) at or above the exact K-th largest
 * key tauK (maximum tmaxKey), run by wave 0 alone, four entries per lane:
 * masses, the top-p cut as a weighted select over keys (the largest key whose
 * mass at or above it reaches the need: the same cut as a scan in key
 * order), min-p, and the draw as a weighted select over ids (the largest id
 * v whose kept mass at or above it reaches Z - target is the first id, in
 * ascending order, whose cumulative mass exceeds the target).
 */
__device__ __forceinline__ void pss_wave_tail4(const pss_args& a, uint32_t row, const pss_rowcfg& c,
                                            const unsigned long long* src, uint32_t cnt, uint32_t tauK,
                                            uint32_t tmaxKey, const pss_row_pre& pre, uint32_t u24,
                                            uint32_t newRng, uint64_t* hist) {
    const uint32_t lane = pss_tid() & 63u;
    const float tmax = pss_unkey(tmaxKey);
    uint32_t key[4], id[4];
    float p[4];
    uint64_t q[4];
    bool v[4];
    uint64_t qs = 0u;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t i = lane + 64u * (uint32_t)r;
        v[r] = i < cnt;
        const unsigned long long e = v[r] ? src[i] : 0ull;
        key[r] = (uint32_t)(e >> 32);
        id[r] = (uint32_t)e;
        p[r] = v[r] ? pss_prob(pss_unkey(key[r]), tmax) : 0.0f;
        q[r] = v[r] ? pss_fixq(p[r]) : 0ull;
        qs += q[r];
    }
    const uint64_t zk = wave_sum_u64(qs);
    uint32_t tau = tauK;
    if (c.useTopP) {
        const uint64_t need = pss_topp_need(c.topP, zk);
        const int sh = pss_select_shift(tauK, tmaxKey);
        const uint32_t tauP = sh < 0 ? tmaxKey : pss_wave_wselect<4>(key, q, need, sh, tmaxKey, hist);
        tau = tauP > tau ? tauP : tau;
    }
    uint64_t kq[4];
    bool kp[4];
    uint64_t zs = 0u;
    uint32_t kc = 0u, last = 0u;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        kp[r] = v[r] && key[r] >= tau && (!c.useMinP || p[r] >= c.minP);
        kq[r] = kp[r] ? q[r] : 0ull;
        zs += kq[r];
        kc += (uint32_t)__popcll(__ballot(kp[r]));
        last = kp[r] && id[r] + 1u > last ? id[r] + 1u : last;
    }
    const uint64_t Z = wave_sum_u64(zs);
    const uint32_t lastAll = wave_max_u32(last);
    const uint64_t target = pss_draw_target(u24, Z);
    uint32_t tok, flags = 0;
    if (Z > 0) {
        tok = pss_wave_wselect<4>(id, kq, Z - target, 16, 0u, hist);
    } else {
        tok = lastAll > 0u ? lastAll - 1u : 0u;
        flags |= PSS_INFO_FALLBACK;
    }
    if (a.kept_mask || a.probs) {
        if (a.kept_mask)
            for (uint32_t w = lane; w < a.mask_words; w += 64u) a.kept_mask[(size_t)row * a.mask_words + w] = 0u;
        if (a.probs)
            for (uint32_t j = lane; j < a.V; j += 64u) a.probs[(size_t)row * a.probs_stride + j] = 0.0f;
        pss_wait_mem();
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (kp[r]) {
                if (a.kept_mask) atomicOr(&a.kept_mask[(size_t)row * a.mask_words + (id[r] >> 5)], 1u << (id[r] & 31u));
                if (a.probs) a.probs[(size_t)row * a.probs_stride + id[r]] = p[r] / ((float)Z * 0x1.0p-45f);
            }
    }
    if (lane == 0) {
        pss_row_info inf = {};
        inf.token = tok;
        inf.kept_count = kc;
        inf.tau_key = tau;
        inf.tmax_key = tmaxKey;
        inf.z_kept = Z;
        inf.z_topk = zk;
        inf.target = target;
        inf.u24 = u24;
        inf.flags = flags;
        pss_epilogue_pre(a, row, tok, false, c.W, newRng, inf, pre.pos, pre.step);
    }
}

/* Ascending sort of one u32 per lane across the wave (bitonic, DPP /
 * permlane exchanges); `lane` is the lane index, computed once by the caller
 * so the per-stage directions are not recomputed. */
template <int KB, int J>
__device__ __forceinline__ uint32_t pss_sort_stage(uint32_t x, uint32_t lane) {
    uint32_t y;
    if constexpr (J <= 8) {
        y = lane_xor<J>(x);
    } else if constexpr (J == 16) {
        const auto p = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        y = (lane & 16u) ? p[0] : p[1];
    } else {
        const auto p = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        y = (lane & 32u) ? p[0] : p[1];
    }
    const bool lowSide = (lane & (uint32_t)J) == 0u;
    const bool asc = KB == 64 ? true : (lane & (uint32_t)KB) == 0u;
    return lowSide == asc ? min(x, y) : max(x, y);
}
__device__ __forceinline__ uint32_t pss_sort64_asc(uint32_t x, uint32_t lane) {
    x = pss_sort_stage<2, 1>(x, lane);
    x = pss_sort_stage<4, 2>(x, lane);
    x = pss_sort_stage<4, 1>(x, lane);
    x = pss_sort_stage<8, 4>(x, lane);
    x = pss_sort_stage<8, 2>(x, lane);
    x = pss_sort_stage<8, 1>(x, lane);
    x = pss_sort_stage<16, 8>(x, lane);
    x = pss_sort_stage<16, 4>(x, lane);
    x = pss_sort_stage<16, 2>(x, lane);
    x = pss_sort_stage<16, 1>(x, lane);
    x = pss_sort_stage<32, 16>(x, lane);
    x = pss_sort_stage<32, 8>(x, lane);
    x = pss_sort_stage<32, 4>(x, lane);
    x = pss_sort_stage<32, 2>(x, lane);
    x = pss_sort_stage<32, 1>(x, lane);
    x = pss_sort_stage<64, 32>(x, lane);
    x = pss_sort_stage<64, 16>(x, lane);
    x = pss_sort_stage<64, 8>(x, lane);
    x = pss_sort_stage<64, 4>(x, lane);
    x = pss_sort_stage<64, 2>(x, lane);
    return pss_sort_stage<64, 1>(x, lane);
}

/*
 * Finisher tail for 1..64 entries (src) that hold every element at or above
 * the K-th largest, run by waves 0 and 1 together (threads 0..127), one entry
 * per lane in each.  The key order and the id order are independent, so the
 * two sorts run on two SIMDs at once:
 *   wave 0: the keys in descending order give the K-th largest (position
 *     K - 1, when `find_k`; otherwise tauK is exact already) and the
 *     key-order mass scan for the top-p cut (every quantity depends on the
 *     key alone, so ties need no order); it hands the cut tau (with the row
 *     maximum and Z_k) to wave 1 through sh and ends;
 *   wave 1: (id << 6) | lane sorted in ascending order, each entry's key by
 *     ds_bpermute, its mass; once tau arrives, min-p and the cut on each
 *     entry, the kept mass in ascending-id order, the first id whose
 *     cumulative mass exceeds the draw target, the verification outputs and
 *     the epilogue.
 * sh.hflag must be zero on entry (cleared before the caller's last barrier).
 */
__device__ __forceinline__ void pss_tail64_2w(const pss_args& a, uint32_t row, const pss_rowcfg& c,
                                              const unsigned long long* src, uint32_t cnt, uint32_t tauK,
                                              bool find_k, const pss_row_pre& pre, uint32_t u24, uint32_t newRng,
                                              pss_fin_small& sh) {
    const uint32_t lane = threadIdx.x & 63u;
    const bool valid = lane < cnt;
    const uint64_t my = valid ? src[lane] : 0ull;
    const uint32_t mkey = (uint32_t)(my >> 32), mid = (uint32_t)my;
    if (threadIdx.x < 64u) {
        /* S5/S6 over the keys in descending order (keys of entries are at
         * least key(-inf) > 0; missing lanes sort last as key 0) */
        const uint32_t skey = ~pss_sort64_asc(valid ? ~mkey : 0xFFFFFFFFu, lane);
        const uint32_t tmaxKey = wave_read_u32(skey, 0u);
        if (find_k) tauK = wave_read_u32(skey, (c.K <= cnt ? c.K : cnt) - 1u);
        const bool sv = valid && skey >= tauK;
        const float tmax = pss_unkey(tmaxKey);
        const uint64_t sq = sv ? pss_fixq(pss_prob(pss_unkey(skey), tmax)) : 0ull;
        const uint64_t P = wave_incl_scan_u64(sq);
        const uint64_t zk = wave_read_u64(P, 63);
        uint32_t tau = tauK;
        if (c.useTopP) {
            const uint64_t need = pss_topp_need(c.topP, zk);
            const uint64_t m = __ballot(sv && P >= need);
            const uint32_t tauP = wave_read_u32(skey, (uint32_t)__ffsll((long long)m) - 1u);
            tau = tauP > tau ? tauP : tau;
        }
        if (lane == 0u) {
            sh.htau = tau;
            sh.htmax = tmaxKey;
            sh.hzk = zk;
            __hip_atomic_store(&sh.hflag, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        return;
    }
    /* wave 1: the entries in id order ((id << 6) | lane: ids < 2^18) with
     * their keys and masses, while wave 0 finds the cut */
    const uint32_t tmaxKey = __builtin_amdgcn_readfirstlane(wave_max_u32(valid ? mkey : 0u));
    const uint32_t ix = pss_sort64_asc(valid ? ((mid << 6) | lane) : 0xFFFFFFFFu, lane);
    const bool iv = ix != 0xFFFFFFFFu;
    const uint32_t ik = (uint32_t)__builtin_amdgcn_ds_bpermute((int)((ix & 63u) << 2), (int)mkey);
    const float tmax = pss_unkey(tmaxKey);
    const float ip = iv ? pss_prob(pss_unkey(ik), tmax) : 0.0f;
    const uint64_t iq = pss_fixq(ip);
    while (__hip_atomic_load(&sh.hflag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) == 0u)
        __builtin_amdgcn_s_sleep(1);
    const uint32_t tau = sh.htau;
    /* S7 on each entry, S8: the kept mass in ascending-id order, the first
     * crossing of the target */
    const bool kp = iv && ik >= tau && (!c.useMinP || ip >= c.minP);
    const uint64_t C = wave_incl_scan_u64(kp ? iq : 0ull);
    const uint64_t Z = wave_read_u64(C, 63);
    const uint64_t km = __ballot(kp);
    const uint32_t keptCount = (uint32_t)__popcll(km);
    const uint64_t target = pss_draw_target(u24, Z);
    const uint64_t hit = __ballot(kp && C > target);
    uint32_t tok, flags = 0;
    if (hit) {
        tok = wave_read_u32(ix, (uint32_t)__ffsll((long long)hit) - 1u) >> 6;
    } else {
        /* the largest kept id (the last kept entry in id order) */
        tok = km ? wave_read_u32(ix, 63u - (uint32_t)__builtin_clzll(km)) >> 6 : 0u;
        flags |= PSS_INFO_FALLBACK;
    }

    /* verification outputs */
    if (a.kept_mask || a.probs) {
        if (a.kept_mask)
            for (uint32_t w = lane; w < a.mask_words; w += 64u) a.kept_mask[(size_t)row * a.mask_words + w] = 0u;
        if (a.probs)
            for (uint32_t j = lane; j < a.V; j += 64u) a.probs[(size_t)row * a.probs_stride + j] = 0.0f;
        pss_wait_mem();
        if (kp) {
            const uint32_t sid = ix >> 6;
            if (a.kept_mask) atomicOr(&a.kept_mask[(size_t)row * a.mask_words + (sid >> 5)], 1u << (sid & 31u));
            if (a.probs) a.probs[(size_t)row * a.probs_stride + sid] = ip / ((float)Z * 0x1.0p-45f);
        }
    }
    if (lane == 0) {
        pss_row_info inf = {};
        inf.token = tok;
        inf.kept_count = keptCount;
        inf.tau_key = tau;
        inf.tmax_key = tmaxKey;
        inf.z_kept = Z;
        inf.z_topk = sh.hzk;
        inf.target = target;
        inf.u24 = u24;
        inf.flags = flags;
        pss_epilogue_pre(a, row, tok, false, c.W, newRng, inf, pre.pos, pre.step);
    }
}

/* One compare-exchange stage (block KB, distance J) of an ascending bitonic
 * sort of 64 R values, R per lane at positions 64 r + lane (r = 0..R-1):
 * distances of 64 and more pair registers of the lane, smaller ones lanes
 * (DPP / permlane exchanges). */
template <int R, uint32_t KB, uint32_t J>
__device__ __forceinline__ void pss_sortr_stage(uint32_t (&x)[R], uint32_t lane) {
    if constexpr (J >= 64u) {
        constexpr uint32_t d = J / 64u;
#pragma unroll
        for (uint32_t r = 0; r < (uint32_t)R; ++r) {
            if (r & d) continue;
            const uint32_t p = 64u * r + lane;
            const bool asc = (p & KB) == 0u;
            const uint32_t lo = min(x[r], x[r | d]), hi = max(x[r], x[r | d]);
            x[r] = asc ? lo : hi;
            x[r | d] = asc ? hi : lo;
        }
    } else {
        const bool low = (lane & J) == 0u;
#pragma unroll
        for (uint32_t r = 0; r < (uint32_t)R; ++r) {
            const uint32_t p = 64u * r + lane;
            const bool asc = (p & KB) == 0u;
            const uint32_t y = lane_xor<(int)J>(x[r]);
            x[r] = (low == asc) ? min(x[r], y) : max(x[r], y);
        }
    }
}
template <int R, uint32_t KB, uint32_t J>
__device__ __forceinline__ void pss_sortr_from(uint32_t (&x)[R], uint32_t lane) {
    pss_sortr_stage<R, KB, J>(x, lane);
    if constexpr (J > 1u)
        pss_sortr_from<R, KB, J / 2u>(x, lane);
    else if constexpr (KB < 64u * (uint32_t)R)
        pss_sortr_from<R, KB * 2u, KB>(x, lane);
}
/* x[r] of position p (p uniform). */
template <int R>
__device__ __forceinline__ uint32_t pss_posr(const uint32_t (&x)[R], uint32_t p) {
    const uint32_t r = p >> 6, l = p & 63u;
    uint32_t v = wave_read_u32(x[0], l);
#pragma unroll
    for (int i = 1; i < R; ++i) {
        const uint32_t vi = wave_read_u32(x[i], l);
        v = r == (uint32_t)i ? vi : v;
    }
    return v;
}

/*
 * Finisher tail for 65..64 R entries (src, in LDS; R = 2 or 4) holding every
 * element at or above the K-th largest, run by waves 0 and 1 together
 * (threads 0..127), R entries per lane in each (positions 64 r + lane), as
 * pss_tail64_2w:
 *   wave 0: the keys sorted in descending order (one 64 R-value bitonic
 *     network in registers and lanes) give the K-th largest at position
 *     K - 1 and the key-order mass scan for the top-p cut; it hands the cut
 *     (with Z_k) to wave 1 through sh and ends;
 *   wave 1: (id << 8) | index sorted in ascending order, each entry's key
 *     from src, its mass; once the cut arrives, min-p and the cut on each
 *     entry, the kept mass in ascending-id order, the first id whose
 *     cumulative mass exceeds the draw target, the verification outputs and
 *     the epilogue.
 * sh.hflag must be zero on entry (cleared before the caller's last barrier).
 */
template <int R>
__device__ __forceinline__ void pss_tailr_2w(const pss_args& a, uint32_t row, const pss_rowcfg& c,
                                             const unsigned long long* src, uint32_t cnt, const pss_row_pre& pre,
                                             uint32_t u24, uint32_t newRng, pss_fin_small& sh) {
    static_assert(PSS_MAX_VOCAB <= (1u << 24), "ids and an 8-bit index in 32 bits");
    const uint32_t lane = threadIdx.x & 63u;
    if (threadIdx.x < 64u) {
        uint32_t x[R];
#pragma unroll
        for (uint32_t r = 0; r < (uint32_t)R; ++r) {
            const uint32_t i = 64u * r + lane;
            x[r] = i < cnt ? ~(uint32_t)(src[i] >> 32) : 0xFFFFFFFFu; /* missing entries sort last as key 0 */
        }
        pss_sortr_from<R, 2u, 1u>(x, lane);
        uint32_t sk[R];
#pragma unroll
        for (uint32_t r = 0; r < (uint32_t)R; ++r) sk[r] = ~x[r];
        const uint32_t tmaxKey = wave_read_u32(sk[0], 0u);
        const uint32_t tauK = pss_posr<R>(sk, (c.K <= cnt ? c.K : cnt) - 1u);
        const float tmax = pss_unkey(tmaxKey);
        uint64_t P[R];
        bool sv[R];
        uint64_t run = 0u;
#pragma unroll
        for (uint32_t r = 0; r < (uint32_t)R; ++r) {
            sv[r] = 64u * r + lane < cnt && sk[r] >= tauK;
            const uint64_t q = sv[r] ? pss_fixq(pss_prob(pss_unkey(sk[r]), tmax)) : 0ull;
            const uint64_t inc = wave_incl_scan_u64(q);
            P[r] = run + inc;
            run += wave_read_u64(inc, 63u);
        }
        const uint64_t zk = run;
        uint32_t tau = tauK;
        if (c.useTopP) {
            const uint64_t need = pss_topp_need(c.topP, zk);
            uint32_t pos = 0xFFFFFFFFu;
#pragma unroll
            for (int r = R - 1; r >= 0; --r) {
                const uint64_t m = __ballot(sv[r] && P[r] >= need);
                if (m) pos = 64u * (uint32_t)r + (uint32_t)__ffsll((long long)m) - 1u;
            }
            const uint32_t tauP = pos != 0xFFFFFFFFu ? pss_posr<R>(sk, pos) : tmaxKey;
            tau = tauP > tau ? tauP : tau;
        }
        if (lane == 0u) {
            sh.htau = tau;
            sh.htmax = tmaxKey;
            sh.hzk = zk;
            __hip_atomic_store(&sh.hflag, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        return;
    }
    /* wave 1: the entries in id order with their keys and masses */
    uint32_t ix[R];
    uint32_t mk = 0u;
#pragma unroll
    for (uint32_t r = 0; r < (uint32_t)R; ++r) {
        const uint32_t i = 64u * r + lane;
        const unsigned long long e = i < cnt ? src[i] : 0ull;
        ix[r] = i < cnt ? (((uint32_t)e << 8) | i) : 0xFFFFFFFFu;
        const uint32_t k = (uint32_t)(e >> 32);
        mk = i < cnt && k > mk ? k : mk;
    }
    const uint32_t tmaxKey = __builtin_amdgcn_readfirstlane(wave_max_u32(mk));
    pss_sortr_from<R, 2u, 1u>(ix, lane);
    const float tmax = pss_unkey(tmaxKey);
    uint32_t ik[R];
    float ip[R];
    uint64_t iq[R];
#pragma unroll
    for (uint32_t r = 0; r < (uint32_t)R; ++r) {
        const bool iv = ix[r] != 0xFFFFFFFFu;
        ik[r] = iv ? (uint32_t)(src[ix[r] & 255u] >> 32) : 0u;
        ip[r] = iv ? pss_prob(pss_unkey(ik[r]), tmax) : 0.0f;
        iq[r] = pss_fixq(ip[r]);
    }
    while (__hip_atomic_load(&sh.hflag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) == 0u)
        __builtin_amdgcn_s_sleep(1);
    const uint32_t tau = sh.htau;
    bool kp[R];
    uint64_t C[R];
    uint64_t run = 0u;
    uint32_t keptCount = 0u;
    uint32_t lastPos = 0xFFFFFFFFu;
#pragma unroll
    for (uint32_t r = 0; r < (uint32_t)R; ++r) {
        kp[r] = ix[r] != 0xFFFFFFFFu && ik[r] >= tau && (!c.useMinP || ip[r] >= c.minP);
        const uint64_t inc = wave_incl_scan_u64(kp[r] ? iq[r] : 0ull);
        C[r] = run + inc;
        run += wave_read_u64(inc, 63u);
        const uint64_t km = __ballot(kp[r]);
        keptCount += (uint32_t)__popcll(km);
        if (km) lastPos = 64u * r + 63u - (uint32_t)__builtin_clzll(km);
    }
    const uint64_t Z = run;
    const uint64_t target = pss_draw_target(u24, Z);
    uint32_t hitPos = 0xFFFFFFFFu;
#pragma unroll
    for (int r = R - 1; r >= 0; --r) {
        const uint64_t m = __ballot(kp[r] && C[r] > target);
        if (m) hitPos = 64u * (uint32_t)r + (uint32_t)__ffsll((long long)m) - 1u;
    }
    uint32_t tok, flags = 0;
    if (hitPos != 0xFFFFFFFFu) {
        tok = pss_posr<R>(ix, hitPos) >> 8;
    } else {
        /* the largest kept id (the last kept entry in id order) */
        tok = lastPos != 0xFFFFFFFFu ? pss_posr<R>(ix, lastPos) >> 8 : 0u;
        flags |= PSS_INFO_FALLBACK;
    }

    /* verification outputs */
    if (a.kept_mask || a.probs) {
        if (a.kept_mask)
            for (uint32_t w = lane; w < a.mask_words; w += 64u) a.kept_mask[(size_t)row * a.mask_words + w] = 0u;
        if (a.probs)
            for (uint32_t j = lane; j < a.V; j += 64u) a.probs[(size_t)row * a.probs_stride + j] = 0.0f;
        pss_wait_mem();
#pragma unroll
        for (uint32_t r = 0; r < (uint32_t)R; ++r)
            if (kp[r]) {
                const uint32_t sid = ix[r] >> 8;
                if (a.kept_mask) atomicOr(&a.kept_mask[(size_t)row * a.mask_words + (sid >> 5)], 1u << (sid & 31u));
                if (a.probs) a.probs[(size_t)row * a.probs_stride + sid] = ip[r] / ((float)Z * 0x1.0p-45f);
            }
    }
    if (lane == 0) {
        pss_row_info inf = {};
        inf.token = tok;
        inf.kept_count = keptCount;
        inf.tau_key = tau;
        inf.tmax_key = tmaxKey;
        inf.z_kept = Z;
        inf.z_topk = sh.hzk;
        inf.target = target;
        inf.u24 = u24;
        inf.flags = flags;
        pss_epilogue_pre(a, row, tok, false, c.W, newRng, inf, pre.pos, pre.step);
    }
}

/*
 * Fast finisher for up to PSS_FAST_N candidates (list), those
 * below the row-wide bound G ignored (G is at most the K-th largest value,
 * so every entry of the top-K is at or above it):
 *   1. the entries at or above G are compacted into sh.cl (unless the
 *      caller gathered only such entries: `compacted`, with sh.nk zeroed
 *      before its last barrier);
 *   2. at most 64 of them (the usual case): one per lane of wave 0, which
 *      sorts their keys in descending order and reads the K-th largest at
 *      position K - 1.  Otherwise an LDS radix select over them (8-bit
 *      digits below the common prefix of G and the maximum), which stops at
 *      the first digit whose floor has at most 64 entries at or above it
 *      (then wave 0's sort finds the K-th largest among them) or ends at
 *      the K-th largest itself; the <= 64 entries at or above the result go
 *      to wave 0;
 *   3. wave 0, one entry per lane: scan the masses in key order for the
 *      top-p cut, apply min-p, sort the kept ids, fetch their masses from
 *      the owning lanes, scan, take the first id whose cumulative mass
 *      exceeds the draw target.  Lane exchanges are DPP / permlane /
 *      bpermute.
 * With 65..PSS_KEPT_CAP entries at or above the exact K-th largest (K > 64,
 * or ties), wave 0 finishes with pss_wave_tail4 instead of step 3.  Returns
 * false (nothing written) for K > PSS_SEG_KMAX, more than PSS_FAST_N
 * candidates, or more than PSS_KEPT_CAP entries at or above the K-th largest
 * (heavy ties).  TS (0, 128 or 256): 65..TS entries after the compaction go
 * to the two-wave sort tail pss_tailr_2w (no radix passes).
 */
template <int NT, int TS = 256>
__device__ __forceinline__ bool pss_list_finish_fast(const pss_args& a, uint32_t row,
                                                     const pss_rowcfg& c, const unsigned long long* list,
                                                     uint32_t n, uint32_t G, const pss_row_pre& pre,
                                                     pss_fin_small& sh, bool compacted = false) {
    constexpr int R = (int)((PSS_FAST_N + NT - 1) / NT);
    static_assert(NT >= 256 && NT <= 1024, "radix bins: the first 256 threads");
    if (c.K > PSS_SEG_KMAX || n > PSS_FAST_N) return false;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    /* the draw depends on the row state only: off the serial tail */
    uint32_t newRng;
    const uint32_t u24 = pss_draw_u24_pre(a.rng_mode, pre.rng, pre.step, row, &newRng);
    uint32_t nc = n;
    const unsigned long long* cl = list;
    if (!compacted) {
        if (tid == 0) {
            sh.nc = 0u;
            sh.nk = 0u;
            sh.hflag = 0u;
        }
        __syncthreads();
        /* 1. compact */
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t i = tid + (uint32_t)r * NT;
            const unsigned long long e = i < n ? list[i] : 0ull;
            const bool keep = i < n && (uint32_t)(e >> 32) >= G;
            const uint64_t m = __ballot(keep);
            if (m) {
                uint32_t b0 = 0u;
                if (lane == 0u) b0 = atomicAdd(&sh.nc, (uint32_t)__popcll(m));
                const uint32_t base = __builtin_amdgcn_readfirstlane(b0);
                if (keep)
                    sh.cl[base + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u))] = e;
            }
        }
        __syncthreads();
        nc = sh.nc;
        cl = sh.cl;
    }
    uint32_t tauK = 0u, cnt = nc;
    bool coarse = false; /* tauK is a floor below the K-th largest (at most 64 entries at or above it) */
    const unsigned long long* src = cl;
    if (TS > 0 && nc > 64u && nc <= (uint32_t)TS) {
        /* 65..TS candidates: two waves sort them all (no radix passes) */
        if (tid < 128) pss_tailr_2w<(TS > 0 ? TS / 64 : 1)>(a, row, c, cl, nc, pre, u24, newRng, sh);
        return true;
    }
    if (nc > 64u) {
        /* 2b. radix select over the compacted entries */
        uint64_t e[R];
        uint32_t k[R];
        uint32_t kmax = 0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t i = tid + (uint32_t)r * NT;
            e[r] = i < nc ? cl[i] : 0ull;
            k[r] = i < nc ? (uint32_t)(e[r] >> 32) : 0u;
            kmax = k[r] > kmax ? k[r] : kmax;
        }
        if (!compacted) {
            /* (the gathering caller published the per-wave maxima and
             * cleared both histograms before its barrier) */
            kmax = wave_max_u32(kmax);
            if (lane == 0) sh.mx[wave] = kmax;
            if (tid < 256u) sh.hist[0][tid] = sh.hist[1][tid] = 0u;
            __syncthreads();
        }
        uint32_t tmaxKey = 0;
#pragma unroll
        for (int w = 0; w < NT / PSS_WAVE; ++w) tmaxKey = sh.mx[w] > tmaxKey ? sh.mx[w] : tmaxKey;
        const uint32_t d = G ^ tmaxKey;
        tauK = tmaxKey;
        if (d) {
            const int hibit = 31 - __clz(d);
            int shift = (hibit / 8) * 8;
            uint32_t pmask = shift + 8 >= 32 ? 0u : ~((1u << (shift + 8)) - 1u);
            uint32_t prefix = tmaxKey & pmask;
            uint32_t rem = c.K, nab = 0u;
            for (int pass = 0; shift >= 0; shift -= 8, ++pass) {
                /* histogram pass & 1; the other one (read two barriers
                 * ago) is cleared for the next pass meanwhile */
                uint32_t* hist = sh.hist[pass & 1];
                if (pass > 0 && tid < 256u) sh.hist[(pass + 1) & 1][tid] = 0u;
#pragma unroll
                for (int r = 0; r < R; ++r)
                    if (k[r] && (k[r] & pmask) == prefix) atomicAdd(&hist[(k[r] >> shift) & 255u], 1u);
                __syncthreads();
                if (tid < 64) {
                    const uint4 h = *(const uint4*)&hist[4u * lane];
                    const uint32_t s4 = h.x + h.y + h.z + h.w;
                    const uint32_t above = (uint32_t)(wave_incl_suffix_u64(s4) - s4); /* lanes > lane */
                    if (above < rem && rem <= above + s4) {
                        uint32_t cum = above, dg = 4u * lane, hd = 0u;
                        const uint32_t hv[4] = {h.x, h.y, h.z, h.w};
                        for (int i = 3; i >= 0; --i) {
                            if (cum + hv[i] >= rem) {
                                dg = 4u * lane + (uint32_t)i;
                                hd = hv[i];
                                break;
                            }
                            cum += hv[i];
                        }
                        sh.digit = dg;
                        sh.rem = rem - cum;
                        sh.cum = cum;
                        sh.hd = hd;
                    }
                }
                __syncthreads();
                prefix |= sh.digit << shift;
                pmask |= 0xFFu << shift;
                rem = sh.rem;
                /* entries at or above the digit's floor: those above the
                 * prefix, the larger digits, the digit's own.  At most 64
                 * (and at least K): they go to wave 0, whose sort gives the
                 * exact K-th largest. */
                const uint32_t nge = nab + sh.cum + sh.hd;
                if (nge <= 64u) {
                    coarse = true;
                    break;
                }
                nab += sh.cum;
            }
            tauK = prefix;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const bool kp = k[r] && k[r] >= tauK;
            const uint64_t m = __ballot(kp);
            if (m) {
                uint32_t b0 = 0u;
                if (lane == 0u) b0 = atomicAdd(&sh.nk, (uint32_t)__popcll(m));
                const uint32_t pos = __builtin_amdgcn_readfirstlane(b0) +
                                     __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
                if (kp && pos < PSS_KEPT_CAP) sh.kept[pos] = e[r];
            }
        }
        __syncthreads();
        cnt = sh.nk;
        if (cnt > PSS_KEPT_CAP) return false;
        src = sh.kept;
        if (cnt > 64u) {
            /* 65..256 entries at or above the exact K-th largest: wave 0,
             * four per lane, weighted selects instead of sorts */
            if (tid < 64) pss_wave_tail4(a, row, c, sh.kept, cnt, tauK, tmaxKey, pre, u24, newRng, sh.g.hist);
            return true;
        }
    }
    if (cnt == 0u) return false;
    if (tid < 128) pss_tail64_2w(a, row, c, src, cnt, tauK, nc <= 64u || coarse, pre, u24, newRng, sh);
    return true;
}

/* ------------------------------------------------------------------------ */
/* segment kernel: independent persistent waves                              */
/* ------------------------------------------------------------------------ */

template <int EPT, int DT>
struct pss_wgeom {
    static constexpr int E = (DT == PSS_DTYPE_F16) ? 8 : 4; /* elements per 16-byte load */
    static constexpr int NL = EPT / E;                      /* loads per lane */
    static constexpr uint32_t ITEM = (uint32_t)PSS_WAVE * EPT; /* ids per item */
    static constexpr int HPT = 4;                            /* window ids per lane held in registers */
    static_assert(EPT % E == 0, "EPT must be a multiple of the load width");
    static_assert(EPT <= 32, "one claim bit per register index in a 32-bit word");
};

/* LDS of one wave: the staging area of its item (lane l's 16-byte load li at
 * stage[li][l], the layout of a wave's load-to-LDS) and the claim bits of
 * window ids (word l = lane l, bit i = its register t[i]). */
template <int EPT, int DT>
struct pss_wave_lds {
    uint4 stage[pss_wgeom<EPT, DT>::NL][PSS_WAVE];
    uint32_t claim[PSS_WAVE];
};

/* Row tests from the raw parameters (no division).  A row is covered when
 * it is greedy, or its top-k is on and at most a.kmax_cov and its window at
 * most a.wmax_cov ids (PSS_SEG_KMAX / PSS_SEG_WMAX, or the wide fused form's
 * PSS_WIDE_KMAX / PSS_MAX_PENALTY_LEN); the finisher runs the general algorithm on the
 * others and the segment kernel skips them. */
__device__ __forceinline__ bool pss_seg_row_greedy(const pss_args& a, const sample_params& sp) {
    return (a.mode == PSS_MODE_GREEDY) || !(sp.temperature > 0.0f);
}
__device__ __forceinline__ bool pss_seg_row_covered(const pss_args& a, const sample_params& sp) {
    const uint32_t K = sp.topK < a.V ? sp.topK : a.V;
    const uint32_t W = sp.penaltyLength < PSS_MAX_PENALTY_LEN ? sp.penaltyLength : PSS_MAX_PENALTY_LEN;
    return pss_seg_row_greedy(a, sp) || (K > 0u && K <= a.kmax_cov && W <= a.wmax_cov);
}

/* Buffer resource word 3 for raw (untyped, stride 0) buffer loads on gfx9
 * CDNA parts: 32-bit data format, no swizzle, no index stride. */
#define PSS_BUF_DW3 0x00020000

__device__ __forceinline__ __amdgpu_buffer_rsrc_t pss_row_rsrc(const pss_args& a, uint32_t row, uint32_t esz) {
    const char* rowp = (const char*)a.logits + (size_t)row * a.stride * esz;
    return __builtin_amdgcn_make_buffer_rsrc((void*)rowp, (short)0, (int)(a.V * esz), PSS_BUF_DW3);
}

/* Buffer-load cache policy of the fused form's logits stream: nontemporal.
 * Every logit is read once per step; at the headline batch (6 x 105 MB
 * rotating, beyond the last-level cache) this takes a step from 30.6 to
 * 28.8 us.  The small-batch and split forms keep the default policy: a
 * batch-1 decode chain over 64 rows (26 MB, within the L2 caches) is 1.9 us
 * slower per step with the hint. */
#define PSS_NT 2

/* Item s of a row into the wave's staging area.  vec_ok (16-byte aligned
 * rows, V * element size a multiple of 16): raw buffer loads straight to LDS
 * (nontemporal), nothing waited for and no registers held; the hardware
 * returns 0 for ids at or beyond V.  Otherwise one buffer load per element into registers,
 * waited for, then copied to the staging area. */
template <int EPT, int DT, int CPOL = 0>
__device__ __forceinline__ void pss_wave_issue(const pss_args& a, uint32_t row, uint32_t s,
                                               pss_wave_lds<EPT, DT>& wl) {
    using Gm = pss_wgeom<EPT, DT>;
    constexpr int E = Gm::E, NL = Gm::NL;
    constexpr uint32_t esz = DT == PSS_DTYPE_F16 ? 2u : 4u;
    const __amdgpu_buffer_rsrc_t rs = pss_row_rsrc(a, row, esz);
    const uint32_t lane = pss_tid() & 63u;
    const uint32_t base = s * Gm::ITEM;
    if (a.vec_ok) {
#pragma unroll
        for (int li = 0; li < NL; ++li)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rs, (__attribute__((address_space(3))) void*)&wl.stage[li][0], 16, (int)(lane * 16u),
                (int)((base + (uint32_t)li * (PSS_WAVE * E)) * esz), 0, CPOL);
    } else {
#pragma unroll
        for (int li = 0; li < NL; ++li) {
            const uint32_t j0 = base + (uint32_t)li * (PSS_WAVE * E) + lane * E;
            uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int e = 0; e < E; ++e) {
                if (DT == PSS_DTYPE_F16)
                    w[e >> 1] |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (int)((j0 + e) * 2u), 0, 0)
                                 << ((e & 1) * 16);
                else
                    w[e] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)((j0 + e) * 4u), 0, 0);
            }
            wl.stage[li][lane] = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
}

/* Per-item values loaded ahead of the item: the row's window ids (at most
 * PSS_SEG_WMAX on covered rows; sampled rows with a window, the compute step
 * decides exactly whether a penalty applies) and the row-wide bound
 * published so far. */
struct pss_wave_side {
    uint32_t hid[4];
    uint32_t G0;
};

__device__ __forceinline__ void pss_wave_side_load(const pss_args& a, uint32_t row, const sample_params& sp,
                                                   pss_wave_side& sd, bool with_bound) {
    const bool greedy = pss_seg_row_greedy(a, sp);
    const uint32_t W = sp.penaltyLength < PSS_MAX_PENALTY_LEN ? sp.penaltyLength : PSS_MAX_PENALTY_LEN;
    const uint32_t* hist_row = a.history + (size_t)row * PSS_MAX_PENALTY_LEN;
    const uint32_t lane = pss_tid() & 63u;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        const uint32_t idx = lane + (uint32_t)h * PSS_WAVE;
        sd.hid[h] = PSS_SENTINEL;
        if (!greedy && W > (uint32_t)h * PSS_WAVE && idx < W) sd.hid[h] = hist_row[idx];
    }
    const pss_row_ws* ws = (const pss_row_ws*)((const char*)a.ws + (size_t)row * PSS_WS_ROW_BYTES);
    /* The lane-varying (zero) offset keeps the value in a vector register:
     * a uniform load would be moved to a scalar register at once, which
     * waits for every load issued before it. */
    uint32_t z = 0u;
    __asm__ __volatile__("" : "+v"(z));
    sd.G0 = (greedy || !with_bound) ? 0u : pss_ld_agent(&ws->bound + z);
}

/* Small-batch form: the side values loaded before the row's parameters are
 * known (the first 4 x 64 ids of the window buffer, which holds
 * PSS_MAX_PENALTY_LEN >= 256 per row), then trimmed to the row's window. */
__device__ __forceinline__ void pss_wave_side_load_all(const pss_args& a, uint32_t row, pss_wave_side& sd) {
    static_assert(PSS_MAX_PENALTY_LEN >= 4u * PSS_WAVE, "window buffer holds the ids a wave loads");
    const uint32_t* hist_row = a.history + (size_t)row * PSS_MAX_PENALTY_LEN;
    const uint32_t lane = pss_tid() & 63u;
#pragma unroll
    for (int h = 0; h < 4; ++h) sd.hid[h] = hist_row[lane + (uint32_t)h * PSS_WAVE];
    const pss_row_ws* ws = (const pss_row_ws*)((const char*)a.ws + (size_t)row * PSS_WS_ROW_BYTES);
    uint32_t z = 0u;
    __asm__ __volatile__("" : "+v"(z));
    sd.G0 = pss_ld_agent(&ws->bound + z);
}
__device__ __forceinline__ void pss_wave_side_trim(const pss_args& a, const sample_params& sp, pss_wave_side& sd) {
    const bool greedy = pss_seg_row_greedy(a, sp);
    const uint32_t W = sp.penaltyLength < PSS_MAX_PENALTY_LEN ? sp.penaltyLength : PSS_MAX_PENALTY_LEN;
    const uint32_t lane = pss_tid() & 63u;
#pragma unroll
    for (int h = 0; h < 4; ++h)
        if (greedy || lane + (uint32_t)h * PSS_WAVE >= W) sd.hid[h] = PSS_SENTINEL;
    if (greedy) sd.G0 = 0u;
}

/* The K-th largest (1 <= K <= 64 R) of the R keys of each of the 64 lanes,
 * to 16 bits: the largest x with at least K keys >= x, one bit per round
 * (ballots; every lane gets the same value). */
template <int R>
__device__ __forceinline__ uint32_t pss_wave_kth16(const uint32_t (&v)[R], uint32_t K) {
    uint32_t x = 0u;
#pragma unroll
    for (int bit = 31; bit >= 16; --bit) {
        const uint32_t y = x | (1u << bit);
        uint32_t n = 0u;
#pragma unroll
        for (int r = 0; r < R; ++r) n += (uint32_t)__popcll(__ballot(v[r] >= y));
        x = n >= K ? y : x;
    }
    return x;
}

/* t[i] for a lane-varying index i (a select tree over the bits of i). */
template <int N>
__device__ __forceinline__ float pss_pick(const float (&t)[N], uint32_t i) {
    static_assert((N & (N - 1)) == 0, "power-of-two array");
    float cur[N];
#pragma unroll
    for (int k = 0; k < N; ++k) cur[k] = t[k];
#pragma unroll
    for (int w = N / 2, bit = 0; w >= 1; w /= 2, ++bit) {
        const bool hi = (i >> bit) & 1u;
#pragma unroll
        for (int k = 0; k < w; ++k) cur[k] = hi ? cur[2 * k + 1] : cur[2 * k];
    }
    return cur[0];
}

/* Running state of a wave over the items of one row: the row's constants
 * and each lane's largest values so far (M1: one; otherwise a sorted top-4). */
struct pss_wave_run {
    uint32_t row;
    pss_rowcfg c;
    float top[4];
};

/*
 * Persistent segment kernel.  Item i = (row i / NS, item i % NS of the row),
 * 64 EPT consecutive ids.  Workgroup b (PSS_SEG_NW waves) takes items
 * [b per_wg, min((b + 1) per_wg, n_items)), normally whole rows, in rounds:
 * in round r wave w processes item b per_wg + r PSS_SEG_NW + w.  Per round
 * and wave:
 *   A  wait for the item's logits (streamed into the wave's staging area
 *      during the previous round), claim its window ids (a returning LDS or
 *      on a claim bit makes exactly one lane the owner of each id: it reads
 *      the raw value, writes -inf in its place and computes the penalized
 *      value itself), move the item to registers, start the next round's
 *      loads, t = l * (1/T), update the lanes' running top values of the
 *      row (distinct elements outside the window), publish (row, the
 *      ceil(K / NW)-th largest of them) in LDS;
 *   -  one barrier;
 *   B  bound: when every wave's slot holds this row, their minimum has at
 *      least K elements of the row at or above it (otherwise the wave's own
 *      K-th largest); raised by the row-wide bound of other workgroups and
 *      published there.  Then the elements at or above it, and the penalized
 *      window elements at or above it, into the item's slot range of the
 *      row's pool (a pass mask per lane, a wave scan of the counts, one
 *      select tree per entry).  Greedy rows store the item's (max key,
 *      smallest id) instead.
 * A slot only rises within a row, and a wave reads other slots after the
 * barrier, so a slot already rewritten in the next round is still a valid
 * certificate (or a different row, which only withholds the joint bound).
 * M1: every row of the launch has K <= 64 (one running value per lane);
 * otherwise a running top-4 per lane (K <= 256).  `params` is a.params as a
 * restrict argument: the kernel's stores cannot alias it, so the row
 * parameters of later items still come through scalar loads.
 */
template <int EPT, int DT, bool M1, bool FUSED, bool SMALL = false, bool WL = false, class RL = pss_row_lds,
          int NWT = PSS_SEG_NW>
__device__ __forceinline__ void pss_seg_rounds(const pss_args& a, uint32_t NS, uint32_t i0, uint32_t i1,
                                               const sample_params* __restrict__ params,
                                               pss_wave_lds<EPT, DT>* lds, unsigned long long* joint,
                                               RL* rl, const uint32_t* win = nullptr, bool top2 = false) {
    using Gm = pss_wgeom<EPT, DT>;
    constexpr int E = Gm::E, NL = Gm::NL;
    constexpr uint32_t ITEM = Gm::ITEM;
    constexpr uint32_t NW = (uint32_t)NWT;
    constexpr uint32_t esz = DT == PSS_DTYPE_F16 ? 2u : 4u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(pss_tid() >> 6);
    const uint32_t lane = pss_tid() & 63u;
    pss_wave_lds<EPT, DT>& wl = lds[wave];
    /* small form: one round over one row; idle waves hold a neutral slot */
    if (lane == 0u)
        joint[wave] = (SMALL && i0 + wave >= i1) ? (((unsigned long long)(i0 / NS) << 32) | 0xFFFFFFFFull) : ~0ull;
    wl.claim[lane] = 0u;
    __syncthreads();
    const uint32_t V = a.V;
    const float NEG_INF = pss_u2f(0xFF800000u);
    const uint32_t R = (i1 - i0 + NW - 1u) / NW;

    pss_wave_run run;
    run.row = 0xFFFFFFFFu;
    const pss_wave_side none = {{PSS_SENTINEL, PSS_SENTINEL, PSS_SENTINEL, PSS_SENTINEL}, 0u};
    pss_wave_side sd = none;
    uint32_t it = i0 + wave;
    bool act = it < i1;
    uint32_t row = act ? it / NS : i0 / NS;
    uint32_t s = act ? it - row * NS : 0u;
    if (SMALL && act) {
        /* loads first, parameters after: the item and window ids are in
         * flight while the row's parameters arrive (an uncovered row's
         * staged item is never read) */
        pss_wave_issue<EPT, DT, FUSED ? PSS_NT : 0>(a, row, s, wl);
        pss_wave_side_load_all(a, row, sd);
    }
    sample_params sp = params[row];
    bool cov = act && pss_seg_row_covered(a, sp);
    if (SMALL) {
        if (act) pss_wave_side_trim(a, sp, sd);
    } else if (cov) {
        pss_wave_issue<EPT, DT, FUSED ? PSS_NT : 0>(a, row, s, wl);
        pss_wave_side_load(a, row, sp, sd, !FUSED);
    }
    for (uint32_t r = 0; r < R; ++r) {
        const uint32_t nit = it + NW;
        const bool nact = !SMALL && nit < i1;
        const uint32_t nrow = nact ? nit / NS : row;
        const uint32_t ns = nact ? nit - nrow * NS : 0u;
        const sample_params nsp = SMALL ? sp : params[nrow];
        const bool ncov = nact && pss_seg_row_covered(a, nsp);
        pss_wave_side nsd = none;

        /* ---- A ---- */
        const bool greedy = pss_seg_row_greedy(a, sp);
        const uint32_t base = s * ITEM;
        float t[EPT];
        float ov[4] = {NEG_INF, NEG_INF, NEG_INF, NEG_INF};
        uint32_t ovid[4] = {0u, 0u, 0u, 0u};
        uint32_t ovn = 0u; /* bit h: hid[h] is this lane's override */
        uint32_t pw = 0u;  /* this lane's claimed register indices */
        float cur = NEG_INF;
        if (cov) {
            if (run.row != row) {
                run.row = row;
                run.c = pss_make_rowcfg(sp, V);
                run.top[0] = run.top[1] = run.top[2] = run.top[3] = NEG_INF;
            }
            const pss_rowcfg& c = run.c;
            const bool doPen = !greedy && c.doPen;
            const float invT = greedy ? 1.0f : c.invT;
            pss_wait_mem(); /* this item's staged loads and side values */
            __asm__ __volatile__("" ::: "memory");
            if (WL && doPen) {
                /* window in LDS (win[0..W), wide fused form): its ids in this
                 * item become -inf in the staging area and claimed (their
                 * penalized values entered the list before the rounds);
                 * duplicates write the same values */
                const uint32_t nh = (c.W + (uint32_t)PSS_WAVE - 1u) / (uint32_t)PSS_WAVE;
                for (uint32_t h = 0; h < nh; ++h) {
                    const uint32_t idx = h * (uint32_t)PSS_WAVE + lane;
                    const uint32_t id = idx < c.W ? win[idx] : PSS_SENTINEL;
                    const bool inr = id >= base && id - base < ITEM && id < V;
                    if (__ballot(inr) != 0ull && inr) {
                        const uint32_t o = id - base;
                        const uint32_t li = o / (uint32_t)(PSS_WAVE * E), rr = o % (uint32_t)(PSS_WAVE * E);
                        const uint32_t owner = rr / (uint32_t)E, e = rr % (uint32_t)E;
                        atomicOr(&wl.claim[owner], 1u << (li * (uint32_t)E + e));
                        char* p = (char*)&wl.stage[li][owner] + e * esz;
                        if (DT == PSS_DTYPE_F16) {
                            const uint16_t ninf = 0xFC00u;
                            __builtin_memcpy(p, &ninf, 2);
                        } else {
                            *(float*)p = NEG_INF;
                        }
                    }
                }
            }
            if (!WL && doPen) {
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const uint32_t id = sd.hid[h];
                    const bool inr = id >= base && id - base < ITEM && id < V;
                    if (c.W > (uint32_t)h * PSS_WAVE && __ballot(inr) != 0ull && inr) {
                        const uint32_t o = id - base;
                        const uint32_t li = o / (uint32_t)(PSS_WAVE * E), rr = o % (uint32_t)(PSS_WAVE * E);
                        const uint32_t owner = rr / (uint32_t)E, e = rr % (uint32_t)E;
                        const uint32_t bit = 1u << (li * (uint32_t)E + e);
                        const uint32_t old = atomicOr(&wl.claim[owner], bit);
                        if (!(old & bit)) {
                            char* p = (char*)&wl.stage[li][owner] + e * esz;
                            float x;
                            if (DT == PSS_DTYPE_F16) {
                                _Float16 hf;
                                __builtin_memcpy(&hf, p, 2);
                                x = (float)hf;
                                const uint16_t ninf = 0xFC00u;
                                __builtin_memcpy(p, &ninf, 2);
                            } else {
                                x = *(float*)p;
                                *(float*)p = NEG_INF;
                            }
                            ov[h] = pss_penalize(x * invT, c);
                            ovid[h] = id;
                            ovn |= 1u << h;
                        }
                    }
                }
            }
            uint4 raw[NL];
#pragma unroll
            for (int li = 0; li < NL; ++li) raw[li] = wl.stage[li][lane];
            if (doPen) {
                pw = wl.claim[lane];
                wl.claim[lane] = 0u;
            }
            pss_wait_mem(); /* the staging area is free again */
            __asm__ __volatile__("" ::: "memory");
            if (ncov) {
                pss_wave_issue<EPT, DT, FUSED ? PSS_NT : 0>(a, nrow, ns, wl);
                pss_wave_side_load(a, nrow, nsp, nsd, !FUSED);
                __asm__ __volatile__("" ::: "memory");
            }
#pragma unroll
            for (int li = 0; li < NL; ++li) {
                float v[E];
                if (DT == PSS_DTYPE_F16) {
                    const uint32_t w[4] = {raw[li].x, raw[li].y, raw[li].z, raw[li].w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const uint16_t h = (uint16_t)(w[e >> 1] >> ((e & 1) * 16));
                        _Float16 hf;
                        __builtin_memcpy(&hf, &h, 2);
                        v[e] = (float)hf;
                    }
                } else {
                    v[0] = __uint_as_float(raw[li].x);
                    v[1] = __uint_as_float(raw[li].y);
                    v[2] = __uint_as_float(raw[li].z);
                    v[3] = __uint_as_float(raw[li].w);
                }
#pragma unroll
                for (int e = 0; e < E; ++e) t[li * E + e] = v[e] * invT;
            }
            /* The row's last item: ids beyond the vocab read 0; they become
             * -inf, which never passes a bound above key(-inf) and never
             * wins an argmax tie against a real id (larger id); where every
             * element passes they are excluded by id. */
            if (base + ITEM > V) {
#pragma unroll
                for (int i = 0; i < EPT; ++i)
                    t[i] = base + (uint32_t)(i / E) * (PSS_WAVE * E) + lane * E + (uint32_t)(i % E) < V ? t[i]
                                                                                                        : NEG_INF;
            }
            if (greedy) {
                /* argmax of the canonical value, smallest id on ties */
                uint64_t best = 0;
#pragma unroll
                for (int i = 0; i < EPT; ++i) {
                    const uint32_t id = base + (uint32_t)(i / E) * (PSS_WAVE * E) + lane * E + (uint32_t)(i % E);
                    const uint64_t b = ((uint64_t)pss_key(pss_canon(t[i])) << 32) | (uint64_t)(0xFFFFFFFFu - id);
                    best = b > best ? b : best;
                }
                best = wave_max_u64(best);
                if (FUSED) {
                    if (lane == 0u) atomicMax(&rl->best, (unsigned long long)best);
                } else {
                    pss_row_ws* ws = (pss_row_ws*)((char*)a.ws + (size_t)row * PSS_WS_ROW_BYTES);
                    if (lane == 0u) pss_st_agent64(&ws->seg_best[s], best);
                }
            } else {
                /* running values; fmaxf ignores NaN, which canonicalizes to
                 * -inf; -inf (window and padding elements, lanes without
                 * elements) never raises a bound above an order statistic */
#pragma unroll
                for (int i = 0; i < EPT; ++i) cur = fmaxf(cur, t[i]);
                uint32_t T;
                /* ceil(K / waves sharing the slots): NW, or the small form's items */
                const uint32_t nj = SMALL ? (i1 - i0 < NW ? i1 - i0 : NW) : NW;
                const uint32_t kq = (c.K + nj - 1u) / nj;
                if (M1) {
                    run.top[0] = fmaxf(run.top[0], cur);
                    const uint32_t k1[1] = {pss_key(pss_canon(run.top[0]))};
                    T = pss_wave_kth16<1>(k1, kq);
                } else {
                    float t0 = run.top[0], t1 = run.top[1], t2 = run.top[2], t3 = run.top[3];
#pragma unroll
                    for (int i = 0; i < EPT; ++i) {
                        float x = fmaxf(t[i], NEG_INF), y;
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
                    run.top[0] = t0, run.top[1] = t1, run.top[2] = t2, run.top[3] = t3;
                    const uint32_t k4[4] = {pss_key(pss_canon(t0)), pss_key(pss_canon(t1)), pss_key(pss_canon(t2)),
                                            pss_key(pss_canon(t3))};
                    T = pss_wave_kth16<4>(k4, kq);
                }
                if (lane == 0u)
                    __hip_atomic_store(&joint[wave], ((unsigned long long)row << 32) | T, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_WORKGROUP);
                if (SMALL && top2) {
                    /* the item's two largest lane maxima (two distinct
                     * elements), for the finishing workgroup's bound */
                    const uint32_t lk = pss_key(pss_canon(run.top[0]));
                    const uint32_t k1 = wave_max_u32(lk);
                    const uint32_t first = (uint32_t)__builtin_ctzll(__ballot(lk == k1));
                    const uint32_t k2 = wave_max_u32(lane == first ? 0u : lk);
                    pss_row_ws* wsi = (pss_row_ws*)((char*)a.ws + (size_t)row * PSS_WS_ROW_BYTES);
                    if (lane == 0u) pss_st_agent64(&wsi->seg_best[s], ((unsigned long long)k1 << 32) | k2);
                }
            }
        } else if (ncov) {
            pss_wave_issue<EPT, DT, FUSED ? PSS_NT : 0>(a, nrow, ns, wl);
            pss_wave_side_load(a, nrow, nsp, nsd, !FUSED);
        }
        /* The joint certificate needs every slot written once (round 0's
         * barrier).  In the fused form every slot belongs to this row, and a
         * slot only ever grows: whatever mix of this round's and earlier
         * rounds' slots a wave reads, each slot still certifies its own
         * ceil(K / 16) elements, so later rounds need no barrier and a wave
         * whose item arrived early does not wait for the slowest one
         * (slot accesses are atomic 64-bit LDS accesses).  The wide form
         * keeps the barrier: at top-k up to 1,024 a certificate one round
         * old lets measurably more candidates into its list. */
        if (!FUSED || WL || r == 0u) __syncthreads();

        /* ---- B ---- */
        if (cov && !greedy) {
            const pss_rowcfg& c = run.c;
            pss_row_ws* ws = (pss_row_ws*)((char*)a.ws + (size_t)row * PSS_WS_ROW_BYTES);
            /* joint certificate: all NW slots on this row */
            const unsigned long long e = __hip_atomic_load(&joint[lane % NW], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            const bool bad = (uint32_t)(e >> 32) != row;
            uint32_t L = 0u;
            if (__ballot(bad) == 0ull) {
                L = (uint32_t)e;
                L = min(L, lane_xor<1>(L));
                L = min(L, lane_xor<2>(L));
                L = min(L, lane_xor<4>(L));
                L = min(L, lane_xor<8>(L));
                L = __builtin_amdgcn_readfirstlane(L);
            } else if (M1) {
                const uint32_t k1[1] = {pss_key(pss_canon(run.top[0]))};
                L = pss_wave_kth16<1>(k1, c.K);
            } else {
                const uint32_t k4[4] = {pss_key(pss_canon(run.top[0])), pss_key(pss_canon(run.top[1])),
                                        pss_key(pss_canon(run.top[2])), pss_key(pss_canon(run.top[3]))};
                L = pss_wave_kth16<4>(k4, c.K);
            }
            uint32_t thr = L;
            if (FUSED) {
                if (lane == 0u && L > PSS_KEY_NEG_INF) atomicMax(&rl->bound, L);
            } else {
                const uint32_t G0 = __builtin_amdgcn_readfirstlane(sd.G0);
                if (lane == 0u && L > G0 && L > PSS_KEY_NEG_INF)
                    (void)__hip_atomic_fetch_max(&ws->bound, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                thr = L > G0 ? L : G0;
            }

            /* candidates (key >= thr) into the item's slot range.  Above
             * key(-inf) the test is a float compare (false for NaN, which
             * canonicalizes to -inf < thr); at or below it every element of
             * the vocab passes (claimed window elements through their
             * overrides).  A wave with no candidate skips the mask. */
            auto id_of = [&](uint32_t i) -> uint32_t {
                return base + (i / E) * (PSS_WAVE * E) + lane * E + (i % E);
            };
            const uint32_t capw = FUSED ? RL::cap : pss_pool_capw(NS);
            uint32_t pm = 0u, ovp = 0u;
            bool any = true;
            if (thr <= PSS_KEY_NEG_INF) {
#pragma unroll
                for (int i = EPT - 1; i >= 0; --i) pm = pm + pm + (id_of((uint32_t)i) < V ? 1u : 0u);
                pm &= ~pw;
                ovp = ovn;
            } else {
                const float thr_f = pss_unkey(thr);
#pragma unroll
                for (int h = 0; h < 4; ++h) ovp |= (((ovn >> h) & 1u) && ov[h] >= thr_f) ? 1u << h : 0u;
                any = __ballot(cur >= thr_f || ovp != 0u) != 0ull;
                if (any) {
#pragma unroll
                    for (int i = EPT - 1; i >= 0; --i) pm = pm + pm + (t[i] >= thr_f ? 1u : 0u);
                }
            }
            uint32_t tot = 0u;
            if (any) {
                const uint32_t mine = (uint32_t)__popc(pm) + (uint32_t)__popc(ovp);
                const uint32_t incl = wave_incl_scan_u32(mine);
                tot = wave_read_u32(incl, 63);
                /* fused: the wave's range of the workgroup's LDS list */
                uint32_t lbase = 0u;
                if (FUSED) {
                    uint32_t b0 = 0u;
                    if (lane == 0u && tot) b0 = atomicAdd(&rl->n, tot);
                    lbase = __builtin_amdgcn_readfirstlane(b0);
                }
                if ((FUSED ? lbase + tot <= capw : tot <= capw) && mine) {
                    unsigned long long* out = FUSED ? rl->list + lbase + (incl - mine)
                                                    : (unsigned long long*)(ws + 1) + (size_t)s * capw + (incl - mine);
                    auto put = [&](unsigned long long v) {
                        if (FUSED)
                            *out = v;
                        else
                            pss_st_agent64(out, v);
                        ++out;
                    };
#pragma unroll
                    for (int h = 0; h < 4; ++h)
                        if ((ovp >> h) & 1u) put(((unsigned long long)pss_key(pss_canon(ov[h])) << 32) | ovid[h]);
                    while (pm) {
                        const uint32_t i = (uint32_t)__builtin_ctz(pm);
                        pm &= pm - 1u;
                        put(((unsigned long long)pss_key(pss_canon(pss_pick(t, i))) << 32) | id_of(i));
                    }
                }
            }
            if (!FUSED && lane == 0u) pss_st_agent(&ws->seg_count[s], tot <= capw ? tot : PSS_SEG_OVERFLOW);
        }
        it = nit;
        row = nrow;
        s = ns;
        sp = nsp;
        cov = ncov;
        sd = nsd;
    }
}


/* Split form: workgroup b takes items [b per_wg, ...) of the launch; the
 * finisher kernel completes the rows from the workspace pools. */
template <int EPT, int DT, bool M1>
__global__ void __launch_bounds__(PSS_SEG_NT) pss_seg_kernel(pss_args a, uint32_t NS, uint32_t n_items,
                                                             uint32_t per_wg,
                                                             const sample_params* __restrict__ params) {
    __shared__ pss_wave_lds<EPT, DT> lds[PSS_SEG_NW];
    __shared__ unsigned long long joint[PSS_SEG_NW]; /* (row << 32) | per-wave certificate */
    pss_globalize(a);
    if (pss_gate_closed(a)) return;
    const uint32_t i0 = blockIdx.x * per_wg;
    const uint32_t i1 = i0 + per_wg < n_items ? i0 + per_wg : n_items;
    if (i0 >= i1) return;
    pss_seg_rounds<EPT, DT, M1, false>(a, NS, i0, i1, params, lds, joint, (pss_row_lds*)nullptr);
}

/*
 * Fused form: workgroup r takes row r whole, gathers its candidates in an LDS
 * list and finishes the row itself after the last round (no workspace, no
 * second kernel).  The finisher's scratch shares the staging area, free by
 * then.  Rows the list cannot finish (top-k off or above PSS_SEG_KMAX, a
 * window above PSS_SEG_WMAX, more candidates than the list holds) run the
 * general algorithm in the same workgroup.
 */
template <int EPT, int DT>
union pss_row_scratch {
    pss_wave_lds<EPT, DT> st[PSS_SEG_NW];
    struct {
        pss_fin_small f;
        uint32_t bits[PSS_ROW_BITS];
    } fin;
    uint32_t hash[2u * PSS_MAX_PENALTY_LEN]; /* wide form: window dedup before the rounds */
};

/*
 * WIDE (top-k up to PSS_WIDE_KMAX, windows up to PSS_MAX_PENALTY_LEN): the
 * row's window goes to LDS before the rounds; each distinct id in it (an LDS
 * hash set with linear probing, load factor <= 1/2) enters the candidate
 * list with its penalized value, unconditionally, and the rounds turn the
 * window's ids to -inf in their staging areas (pss_seg_rounds WL).  The list
 * holds PSS_WIDE_LIST_CAP entries; the items are 1,024 ids (EPT 16) to make
 * room for it, and the lanes keep a running top-4 (the certificate's
 * ceil(K/16)-th largest of 256 values, K <= 1024).
 */
template <int EPT, int DT, bool M1, bool WIDE>
__global__ void __launch_bounds__(PSS_SEG_NT) pss_row_kernel(pss_args a, uint32_t NS,
                                                             const sample_params* __restrict__ params) {
    constexpr int NT = PSS_SEG_NT;
    using RL = pss_row_lds_t<WIDE ? PSS_WIDE_LIST_CAP : PSS_ROW_LIST_CAP>;
    __shared__ pss_row_scratch<EPT, DT> U;
    __shared__ unsigned long long joint[PSS_SEG_NW];
    __shared__ RL rl;
    __shared__ uint32_t win[WIDE ? PSS_MAX_PENALTY_LEN : 1];
    pss_globalize(a);
    if (pss_gate_closed(a)) return;
    const uint32_t row = blockIdx.x, tid = pss_tid();
    const sample_params sp = params[row];
    pss_row_pre pre;
    pre.rng = a.rng[row];
    pre.step = a.step[row];
    pre.pos = a.position[row];
    if (tid == 0u) {
        rl.n = 0u;
        rl.bound = 0u;
        rl.best = 0ull;
    }
    const bool covered = pss_seg_row_covered(a, sp);
    const pss_rowcfg c = pss_make_rowcfg(sp, a.V);
    if (WIDE && covered && !pss_seg_row_greedy(a, sp) && c.doPen) {
        static_assert(PSS_MAX_PENALTY_LEN <= PSS_SEG_NT, "one window id per thread");
        const uint32_t* hist_row = a.history + (size_t)row * PSS_MAX_PENALTY_LEN;
        for (uint32_t i = tid; i < 2u * PSS_MAX_PENALTY_LEN; i += NT) U.hash[i] = PSS_SENTINEL;
        const uint32_t id = tid < c.W ? hist_row[tid] : PSS_SENTINEL;
        if (tid < c.W) win[tid] = id;
        __syncthreads();
        if (id < a.V) {
            uint32_t h = (id * 2654435761u) >> 21; /* 11 bits: 2,048 slots */
            bool owner = false;
            for (uint32_t probe = 0; probe < 2u * PSS_MAX_PENALTY_LEN; ++probe) {
                const uint32_t old = atomicCAS(&U.hash[h], PSS_SENTINEL, id);
                if (old == PSS_SENTINEL) {
                    owner = true;
                    break;
                }
                if (old == id) break;
                h = (h + 1u) & (2u * PSS_MAX_PENALTY_LEN - 1u);
            }
            if (owner) {
                const char* rowp = (const char*)a.logits + (size_t)row * a.stride * (DT == PSS_DTYPE_F16 ? 2u : 4u);
                const float x = pss_load1(rowp, DT, id);
                const float pen = pss_penalize(x * c.invT, c);
                const uint32_t pos = atomicAdd(&rl.n, 1u);
                if (pos < RL::cap) rl.list[pos] = ((unsigned long long)pss_key(pss_canon(pen)) << 32) | id;
            }
        }
        __syncthreads(); /* the hash shares the staging area */
    }
    if (covered)
        pss_seg_rounds<EPT, DT, M1, true, false, WIDE, RL>(a, NS, row * NS, row * NS + NS, params, U.st, joint, &rl,
                                                          win);
    __syncthreads();
    if (pss_seg_row_greedy(a, sp)) {
        pss_greedy_finish<NT>(a, row, rl.best);
        return;
    }
    const uint32_t n = rl.n;
    bool general = !covered || n > RL::cap;
    if (!general && !pss_list_finish_fast<NT>(a, row, c, rl.list, n, rl.bound, pre, U.fin.f))
        pss_list_finish<NT>(a, row, c, rl.list, n, U.fin.f.g, rl.bound);
    if (general) pss_general_row<NT>(a, row, U.fin.f.g, U.fin.bits, PSS_ROW_BITS);
}

/* ------------------------------------------------------------------------ */
/* finisher kernel                                                           */
/* ------------------------------------------------------------------------ */

/* Finish row `row` from its NS items in the workspace (all NT threads of the
 * workgroup; candidates gathered into sh.list).  Everything the finish needs
 * is requested in one round trip before anything is waited for: thread s < NS
 * loads item s's count, its greedy best and the first SPEC (PSS_FIN_SPEC or twice it) entries
 * of its pool range (one 128-byte line; an item rarely has more, the rest
 * follow in a second trip), every thread the row-wide bound G; the row's
 * parameters and state come loaded by the caller.  Of the first PSS_FIN_SPEC
 * entries only
 * those at or above G are gathered; when no item had more, the list is
 * already compacted for the finisher.  Workspace reads are agent-scope
 * (written by other workgroups of the same launch in the small-batch form). */
#define PSS_SC1 16 /* buffer-load cache policy: device-scope coherent (sc1) */

/* The row's parameters (scalar loads: `params` is never written by these
 * kernels) and state (vector loads through a lane-varying zero offset, so
 * that issuing them waits for nothing; pss_fin_row makes them uniform). */
__device__ __forceinline__ void pss_load_row_state(const pss_args& a, const sample_params* __restrict__ params,
                                                   uint32_t row, sample_params& sp, pss_row_pre& pre) {
    uint32_t z = 0u;
    __asm__ __volatile__("" : "+v"(z));
    pre.rng = a.rng[row + z];
    pre.step = a.step[row + z];
    pre.pos = a.position[row + z];
    sp = params[row];
}
template <int NT, uint32_t SPEC = PSS_FIN_SPEC, bool TOP2 = false>
__device__ __forceinline__ void pss_fin_row(const pss_args& a, const sample_params& sp, const pss_row_pre& pre_in,
                                            uint32_t row, uint32_t NS, pss_fin_shared& sh, uint32_t* bits,
                                            uint32_t bit_words) {
    static_assert(NT >= PSS_SEG_MAX_SLOTS, "one thread per item");
    static_assert(SPEC == 16u || SPEC == 32u, "one or two 128-byte lines per item");
    const uint32_t tid = pss_tid();
    pss_row_ws* ws = (pss_row_ws*)((char*)a.ws + (size_t)row * PSS_WS_ROW_BYTES);
    const uint32_t capw = pss_pool_capw(NS);
    const bool slot = tid < NS;
    const unsigned long long* pool = (const unsigned long long*)(ws + 1);
    const __amdgpu_buffer_rsrc_t prs =
        __builtin_amdgcn_make_buffer_rsrc((void*)pool, (short)0, (int)(PSS_POOL_CAP * 8u), PSS_BUF_DW3);
    /* threads without an item read beyond the resource: zeros, no access */
    const uint32_t voff = slot ? tid * capw * 8u : PSS_POOL_CAP * 8u;
    uint32_t ns = 0u;
    uint64_t best = 0u;
    if (slot) {
        ns = pss_ld_agent(&ws->seg_count[tid]);
        best = pss_ld_agent64(&ws->seg_best[tid]);
    }
    unsigned long long v[SPEC];
#pragma unroll
    for (int j = 0; j < (int)SPEC / 2; ++j) {
        const uint4 w = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(prs, (int)(voff + 16u * j), 0, PSS_SC1));
        v[2 * j] = ((unsigned long long)w.y << 32) | w.x;
        v[2 * j + 1] = ((unsigned long long)w.w << 32) | w.z;
    }
    uint32_t z = 0u;
    __asm__ __volatile__("" : "+v"(z));
    const uint32_t G = pss_ld_agent(&ws->bound + z);
    pss_row_pre pre;
    pre.rng = __builtin_amdgcn_readfirstlane(pre_in.rng);
    pre.step = __builtin_amdgcn_readfirstlane(pre_in.step);
    pre.pos = __builtin_amdgcn_readfirstlane(pre_in.pos);
    const uint32_t V = a.V;
    const bool greedy = (a.mode == PSS_MODE_GREEDY) || !(sp.temperature > 0.0f);
    const pss_rowcfg c = pss_make_rowcfg(sp, V);

    if (greedy) {
        best = block_max_u64<NT>(best, sh.f.g.red);
        pss_greedy_finish<NT>(a, row, best);
        return;
    }
    bool general = !pss_seg_row_covered(a, sp);
    if (!general) {
        /* TOP2 (small form, every item in wave 0): each item's slot holds its
         * two largest lane maxima; the K-th largest of these (K <= 2 NS
         * distinct elements) raises the row bound, usually to about the
         * K-th largest itself */
        uint32_t Gf = G;
        if (TOP2 && NS <= (uint32_t)PSS_WAVE && c.K <= 2u * PSS_WAVE && tid < PSS_WAVE) {
            const uint32_t v2[2] = {slot ? (uint32_t)(best >> 32) : 0u, slot ? (uint32_t)best : 0u};
            const uint32_t x = wave_kth_largest<2, 24>(v2, c.K);
            Gf = x > G ? x : G;
        }
        const bool over = ns == PSS_SEG_OVERFLOW;
        const uint32_t n0 = over ? 0u : ns;
        uint32_t keep = 0u;
#pragma unroll
        for (uint32_t u = 0; u < SPEC; ++u)
            keep |= (u < n0 && (uint32_t)(v[u] >> 32) >= Gf) ? 1u << u : 0u;
        const uint32_t extra = n0 > SPEC ? n0 - SPEC : 0u;
        /* (overflowed items << 54) | (entries not filtered << 32) | entries
         * written: sums of at most 256 items stay within their fields */
        const uint64_t mine = over ? (1ull << 54) : (((uint64_t)extra << 32) | (uint64_t)(__popc(keep) + extra));
        uint64_t off64 = 0u, tot64 = 0u;
        if (tid == 0) {
            sh.f.nk = 0u;
            sh.f.hflag = 0u;
        }
        if (NS <= (uint32_t)PSS_WAVE) {
            /* every item in wave 0: a wave scan, no barrier */
            if (tid < PSS_WAVE) {
                const uint64_t incl = wave_incl_scan_u64(mine);
                off64 = incl - mine;
                tot64 = wave_read_u64(incl, 63);
            }
        } else {
            off64 = block_excl_scan_u64<NT>(mine, sh.f.g.red, &tot64);
        }
        const uint32_t off = (uint32_t)off64;
        if (slot && (uint32_t)tot64 <= PSS_FIN_LIST_CAP) {
            uint32_t o = off;
#pragma unroll
            for (uint32_t u = 0; u < SPEC; ++u)
                if ((keep >> u) & 1u) sh.list[o++] = v[u];
            for (uint32_t i0 = SPEC; i0 < n0; i0 += 8u) {
                unsigned long long w[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) w[u] = i0 + u < n0 ? pss_ld_agent64(pool + (size_t)tid * capw + i0 + u) : 0ull;
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (i0 + u < n0) sh.list[o++] = w[u];
            }
        }
        /* for the finisher: per-wave largest gathered key, cleared radix
         * histograms (both before the barrier) */
        uint32_t mk = 0u;
#pragma unroll
        for (uint32_t u = 0; u < SPEC; ++u)
            mk = ((keep >> u) & 1u) && (uint32_t)(v[u] >> 32) > mk ? (uint32_t)(v[u] >> 32) : mk;
        mk = wave_max_u32(mk);
        if ((tid & 63u) == 0u) sh.f.mx[tid >> 6] = mk;
        if (tid < 256u) sh.f.hist[0][tid] = sh.f.hist[1][tid] = 0u;
        if (tid == 0) {
            sh.f.gtot = tot64;
            sh.f.g2 = Gf;
        }
        __syncthreads();
        tot64 = sh.f.gtot;
        Gf = sh.f.g2;
        const uint32_t total = (uint32_t)tot64;
        const bool compacted = ((tot64 >> 32) & 0x3FFFFFu) == 0u;
        general = (tot64 >> 54) != 0u || total > PSS_FIN_LIST_CAP;
        if (!general && !pss_list_finish_fast<NT>(a, row, c, sh.list, total, Gf, pre, sh.f, compacted)) {
            /* slow path: candidates below the row-wide bound may remain in the
             * list; they are below the K-th largest and never selected */
            pss_list_finish<NT>(a, row, c, sh.list, total, sh.f.g, Gf);
        }
        if (tid == 0) pss_st_agent(&ws->bound, 0u); /* for the next launch */
    }
    if (general) pss_general_row<NT>(a, row, sh.f.g, bits, bit_words);
}

/* One workgroup per row; NS items per row were written by pss_seg_kernel. */
__global__ void __launch_bounds__(PSS_ST_NT) pss_fin_kernel(pss_args a, uint32_t NS,
                                                             const sample_params* __restrict__ params) {
    __shared__ pss_fin_shared sh;
    __shared__ uint32_t bits[PSS_MAX_VOCAB / 32];
    pss_globalize(a);
    if (pss_gate_closed(a)) return;
    sample_params sp;
    pss_row_pre pre;
    pss_load_row_state(a, params, blockIdx.x, sp, pre);
    pss_fin_row<PSS_ST_NT>(a, sp, pre, blockIdx.x, NS, sh, bits, PSS_MAX_VOCAB / 32);
}

/*
 * Small-batch form: GW workgroups per row (grid rows x GW), workgroup g of a
 * row takes items [g NS / GW, (g + 1) NS / GW) of that row only, at most
 * NWS (16 waves, or 4 when the grid of four-wave workgroups fits one per CU:
 * the row then spreads over 13 CUs at batch 1 instead of 4), in one round
 * (each wave one item, the joint certificate over the workgroup's items).  Pool entries and counts are agent-scope stores;
 * every wave waits for its stores to complete, then the workgroup counts
 * itself on the row's ticket with an agent-scope acquire-release
 * fetch-add (release: this workgroup's stores happen before its count;
 * acquire: the workgroup that completes the count sees every other
 * workgroup's stores), and that workgroup resets the ticket and finishes the
 * row in place (pss_fin_row, its scratch over the staging area).  One
 * kernel, no workgroup waits for another.
 */
template <int EPT, int DT>
union pss_small_scratch {
    pss_wave_lds<EPT, DT> st[PSS_SEG_NW];
    struct {
        pss_fin_shared fs;
        uint32_t bits[PSS_ROW_BITS];
    } fin;
};

template <int EPT, int DT, bool M1, int NWS = PSS_SEG_NW>
__global__ void __launch_bounds__(NWS * PSS_WAVE) pss_small_kernel(pss_args a, uint32_t NS, uint32_t GW,
                                                                   const sample_params* __restrict__ params) {
    __shared__ pss_small_scratch<EPT, DT> U;
    __shared__ unsigned long long joint[PSS_SEG_NW];
    __shared__ uint32_t last;
    pss_globalize(a);
    if (pss_gate_closed(a)) return;
    const uint32_t row = blockIdx.x / GW, g = blockIdx.x - row * GW;
    const uint32_t s0 = g * NS / GW, s1 = (g + 1u) * NS / GW;
    const uint32_t tid = pss_tid();
    pss_seg_rounds<EPT, DT, M1, false, true, false, pss_row_lds, NWS>(a, NS, row * NS + s0, row * NS + s1, params, U.st,
                                                                      joint, (pss_row_lds*)nullptr, nullptr, true);
    pss_wait_mem(); /* this wave's pool stores, counts and staged loads have completed */
    __syncthreads();
    if (tid == 0u) {
        pss_row_ws* ws = (pss_row_ws*)((char*)a.ws + (size_t)row * PSS_WS_ROW_BYTES);
        const bool l = __hip_atomic_fetch_add(&ws->ticket, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == GW - 1u;
        if (l) pss_st_agent(&ws->ticket, 0u); /* every other workgroup of the row has counted */
        last = l ? 1u : 0u;
    }
    __syncthreads();
    if (!last) return;
    sample_params sp;
    pss_row_pre pre;
    pss_load_row_state(a, params, row, sp, pre);
    /* four-wave workgroups certify over four items, so an item holds more
     * candidates: two lines of each requested in the first round trip */
    pss_fin_row<NWS * PSS_WAVE, NWS < PSS_SEG_NW ? 2u * PSS_FIN_SPEC : PSS_FIN_SPEC, true>(
        a, sp, pre, row, NS, U.fin.fs, U.fin.bits, PSS_ROW_BITS);
}

/* ---------------------------------------------------------------------- */
/* host-side launch                                                        */
/* ---------------------------------------------------------------------- */

/* Elements per lane: 32 (2048-id items); 16 only if a row would otherwise
 * need more than PSS_SEG_MAX_SLOTS items (none at V <= 262,144). */
static inline int pss_stream_pick_ept(uint32_t V, uint32_t rows) {
    (void)rows;
    const uint64_t n32 = (V + (uint64_t)PSS_WAVE * 32u - 1u) / ((uint64_t)PSS_WAVE * 32u);
    return n32 > PSS_SEG_MAX_SLOTS ? 16 : 32;
}

/* Workgroups of a segment kernel instantiation resident on the current
 * device at once (occupancy x CUs), cached per device; 0 if unknown. */
template <int EPT, int DT, bool M1>
static inline uint32_t pss_seg_capacity() {
    static uint32_t cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
    if (dev < 64 && cache[dev]) return cache[dev];
    int cus = 0, nb = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, pss_seg_kernel<EPT, DT, M1>, PSS_SEG_NT, 0) !=
        hipSuccess)
        return 0;
    const uint32_t cap = (uint32_t)(nb > 0 ? nb : 1) * (uint32_t)(cus > 0 ? cus : 1);
    if (dev < 64) cache[dev] = cap;
    return cap;
}

/* Grid: items split evenly over at most the resident workgroups, at least
 * one round (PSS_SEG_NW items) per workgroup. */
template <int EPT, int DT, bool M1>
static inline hipError_t pss_seg_launch(const pss_args& a, uint32_t NS, uint32_t n_items, hipStream_t st) {
    uint32_t cap = pss_seg_capacity<EPT, DT, M1>();
    if (cap == 0) cap = 1;
    uint32_t per_wg = (n_items + cap - 1u) / cap;
    if (per_wg < PSS_SEG_NW) per_wg = PSS_SEG_NW;
    const uint32_t grid = (n_items + per_wg - 1u) / per_wg;
    pss_seg_kernel<EPT, DT, M1><<<dim3(grid), dim3(PSS_SEG_NT), 0, st>>>(a, NS, n_items, per_wg, a.params);
    return hipGetLastError();
}

/* Streaming forms: fused (one workgroup per row), small-batch (each row over
 * ceil(NS / PSS_SEG_NW) workgroups of one round, finished by the last to
 * arrive), split (two kernels). */
enum { PSS_FORM_FUSED = 0, PSS_FORM_SMALL = 1, PSS_FORM_SPLIT = 2, PSS_FORM_RESIDENT = 3 };

static inline uint32_t pss_small_gw(uint32_t NS) { return (NS + PSS_SEG_NW - 1u) / PSS_SEG_NW; }
/* Workgroups of four waves: a row spread over four times as many CUs, for
 * launches whose grid still fits one workgroup per CU (batch 1 to a few rows). */
#define PSS_SMALL4_NW 4
static inline uint32_t pss_small4_gw(uint32_t NS) { return (NS + PSS_SMALL4_NW - 1u) / PSS_SMALL4_NW; }
static inline uint32_t pss_cu_count() {
    static uint32_t cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
    if (dev < 64 && cache[dev]) return cache[dev];
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 0;
    if (dev < 64) cache[dev] = (uint32_t)cus;
    return (uint32_t)cus;
}

template <int EPT>
static inline hipError_t pss_stream_go(const pss_args& a, uint32_t rows, uint32_t max_k, int form,
                                       hipStream_t st, hipEvent_t split_ev) {
    const uint32_t item = (uint32_t)PSS_WAVE * EPT;
    const uint32_t NS = (a.V + item - 1u) / item;
    if (NS > PSS_SEG_MAX_SLOTS || (uint64_t)rows * NS >= (1ull << 31)) return hipErrorInvalidValue;
    const bool m1 = max_k <= (uint32_t)PSS_WAVE;
    hipError_t e;
    if (form == PSS_FORM_SMALL) {
        const uint32_t GW4 = pss_small4_gw(NS);
        if ((uint64_t)rows * GW4 <= (uint64_t)pss_cu_count()) {
            const dim3 grid(rows * GW4), block(PSS_SMALL4_NW * PSS_WAVE);
            if (a.dtype == PSS_DTYPE_F16) {
                if (m1)
                    pss_small_kernel<EPT, PSS_DTYPE_F16, true, PSS_SMALL4_NW><<<grid, block, 0, st>>>(a, NS, GW4, a.params);
                else
                    pss_small_kernel<EPT, PSS_DTYPE_F16, false, PSS_SMALL4_NW><<<grid, block, 0, st>>>(a, NS, GW4, a.params);
            } else {
                if (m1)
                    pss_small_kernel<EPT, PSS_DTYPE_F32, true, PSS_SMALL4_NW><<<grid, block, 0, st>>>(a, NS, GW4, a.params);
                else
                    pss_small_kernel<EPT, PSS_DTYPE_F32, false, PSS_SMALL4_NW><<<grid, block, 0, st>>>(a, NS, GW4, a.params);
            }
            if ((e = hipGetLastError()) != hipSuccess) return e;
            if (split_ev && (e = hipEventRecord(split_ev, st)) != hipSuccess) return e;
            return hipSuccess;
        }
        const uint32_t GW = pss_small_gw(NS);
        if ((uint64_t)rows * GW > 0x7FFFFFFFull) return hipErrorInvalidValue;
        const dim3 grid(rows * GW), block(PSS_SEG_NT);
        if (a.dtype == PSS_DTYPE_F16) {
            if (m1)
                pss_small_kernel<EPT, PSS_DTYPE_F16, true><<<grid, block, 0, st>>>(a, NS, GW, a.params);
            else
                pss_small_kernel<EPT, PSS_DTYPE_F16, false><<<grid, block, 0, st>>>(a, NS, GW, a.params);
        } else {
            if (m1)
                pss_small_kernel<EPT, PSS_DTYPE_F32, true><<<grid, block, 0, st>>>(a, NS, GW, a.params);
            else
                pss_small_kernel<EPT, PSS_DTYPE_F32, false><<<grid, block, 0, st>>>(a, NS, GW, a.params);
        }
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if (split_ev && (e = hipEventRecord(split_ev, st)) != hipSuccess) return e;
        return hipSuccess;
    }
    if (form == PSS_FORM_FUSED) {
        const dim3 grid(rows), block(PSS_SEG_NT);
        if (a.dtype == PSS_DTYPE_F16) {
            if (m1)
                pss_row_kernel<EPT, PSS_DTYPE_F16, true, false><<<grid, block, 0, st>>>(a, NS, a.params);
            else
                pss_row_kernel<EPT, PSS_DTYPE_F16, false, false><<<grid, block, 0, st>>>(a, NS, a.params);
        } else {
            if (m1)
                pss_row_kernel<EPT, PSS_DTYPE_F32, true, false><<<grid, block, 0, st>>>(a, NS, a.params);
            else
                pss_row_kernel<EPT, PSS_DTYPE_F32, false, false><<<grid, block, 0, st>>>(a, NS, a.params);
        }
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if (split_ev && (e = hipEventRecord(split_ev, st)) != hipSuccess) return e;
        return hipSuccess;
    }
    const uint32_t n_items = rows * NS;
    if (a.dtype == PSS_DTYPE_F16)
        e = m1 ? pss_seg_launch<EPT, PSS_DTYPE_F16, true>(a, NS, n_items, st)
               : pss_seg_launch<EPT, PSS_DTYPE_F16, false>(a, NS, n_items, st);
    else
        e = m1 ? pss_seg_launch<EPT, PSS_DTYPE_F32, true>(a, NS, n_items, st)
               : pss_seg_launch<EPT, PSS_DTYPE_F32, false>(a, NS, n_items, st);
    if (e != hipSuccess) return e;
    if (split_ev && (e = hipEventRecord(split_ev, st)) != hipSuccess) return e;
    pss_fin_kernel<<<dim3(rows), dim3(PSS_ST_NT), 0, st>>>(a, NS, a.params);
    return hipGetLastError();
}

/* Resident workgroups of the small-batch kernel on the current device (one
 * per CU at its LDS footprint), cached; 0 if unknown. */
static inline uint32_t pss_small_capacity() {
    static uint32_t cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
    if (dev < 64 && cache[dev]) return cache[dev];
    int cus = 0, nb = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, pss_small_kernel<32, PSS_DTYPE_F32, true>,
                                                     PSS_SEG_NT, 0) != hipSuccess)
        return 0;
    const uint32_t cap = (uint32_t)(nb > 0 ? nb : 1) * (uint32_t)(cus > 0 ? cus : 1);
    if (dev < 64) cache[dev] = cap;
    return cap;
}

/* max_k, max_w: the largest top-k and window of the launched rows (upper
 * bounds are enough).  form: PSS_FORM_*, or -1 to choose: the small-batch
 * form while its grid is at most one pass of resident workgroups (every row
 * spread over several CUs, one round), the fused form above that; rows with a
 * top-k above PSS_SEG_KMAX or a window above PSS_SEG_WMAX take the wide fused
 * form (unless a split or small-batch form is forced, which leaves them to
 * the general algorithm).  All forms compute the same bits. */
static inline hipError_t pss_stream_launch(pss_args a, uint32_t rows, uint32_t max_k, uint32_t max_w, int form,
                                           hipStream_t st, hipEvent_t split_ev) {
    const size_t esz = a.dtype == PSS_DTYPE_F16 ? 2u : 4u;
    a.vec_ok = ((a.stride * esz) % 16u == 0u) && (((uintptr_t)a.logits & 15u) == 0u) &&
               ((a.V * esz) % 16u == 0u);
    if ((max_k > PSS_SEG_KMAX || max_w > PSS_SEG_WMAX) && (form < 0 || form == PSS_FORM_FUSED)) {
        const uint32_t NS = (a.V + (uint32_t)PSS_WAVE * 16u - 1u) / ((uint32_t)PSS_WAVE * 16u);
        if (NS > PSS_SEG_MAX_SLOTS) return hipErrorInvalidValue;
        a.kmax_cov = PSS_WIDE_KMAX;
        a.wmax_cov = PSS_MAX_PENALTY_LEN;
        const dim3 grid(rows), block(PSS_SEG_NT);
        if (a.dtype == PSS_DTYPE_F16)
            pss_row_kernel<16, PSS_DTYPE_F16, false, true><<<grid, block, 0, st>>>(a, NS, a.params);
        else
            pss_row_kernel<16, PSS_DTYPE_F32, false, true><<<grid, block, 0, st>>>(a, NS, a.params);
        hipError_t e = hipGetLastError();
        if (e == hipSuccess && split_ev) e = hipEventRecord(split_ev, st);
        return e;
    }
    const int ept = pss_stream_pick_ept(a.V, rows);
    if (form < 0) {
        const uint64_t item = (uint64_t)PSS_WAVE * ept;
        const uint32_t NS = (uint32_t)((a.V + item - 1u) / item);
        const uint64_t cap = pss_small_capacity();
        form = (cap && (uint64_t)rows * pss_small_gw(NS) <= cap) ? PSS_FORM_SMALL : PSS_FORM_FUSED;
    }
    switch (ept) {
        case 32: return pss_stream_go<32>(a, rows, max_k, form, st, split_ev);
        default: return pss_stream_go<16>(a, rows, max_k, form, st, split_ev);
    }
}

#endif /* PSS_STREAM_H */
