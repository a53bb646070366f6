/*
 * pss_stream.h - the streaming sampler (the HBM-roofline path): two kernels
 * on the sampler's stream.
 *
 * pss_seg_kernel, grid (S, rows) x 256 threads: workgroup (s, r) owns
 * segment s of row r, SEG = 256 * EPT consecutive ids.  It reads the segment
 * once with 16-byte coalesced loads (4 fp32 / 8 fp16 per lane), all issued
 * before anything waits for them, and keeps the transformed logits
 * t = l * (1/T) (penalized for ids in the window, from an LDS bitmap of the
 * segment's ids) in registers.  Then:
 *   bound  every lane's top-m values (m = ceil(K / 256)) go to LDS and every
 *          wave finds the K-th largest of them with ballots.  They are
 *          elements of the segment, so every element at or above the row's
 *          K-th largest value is >= that bound; the bound is also published
 *          row-wide (atomic max, not waited for) and read back by later
 *          segments of the row to tighten theirs.
 *   pool   the elements at or above the bound (a few more than K) are
 *          appended to an LDS list and copied to the segment's own slot range
 *          of the row's pool, with their count.  No returning global atomic,
 *          no cross-workgroup wait.
 *   greedy rows store the segment's (max key, smallest id) instead.
 *
 * pss_fin_kernel, one 256-thread workgroup per row, after it on the stream:
 * gathers the row's candidates (about S * K entries, L2-resident) into LDS
 * and finishes the row: exact K-th largest, masses q = trunc(exp(t - tmax) *
 * 2^45), top-p, min-p and the draw as an ascending-id inverse CDF over the
 * kept set, then the epilogue (result slot, token, window, rng, position).
 * Rows the candidates cannot finish -- top-k off or above 1024, a segment
 * whose candidates overflow its slots (heavy ties) -- run the general
 * algorithm there instead, re-reading the row.  Every path computes the same
 * bits as the one-workgroup-per-row general kernel.
 */
#ifndef PSS_STREAM_H
#define PSS_STREAM_H

#include "pss_general.h"

#define PSS_ST_NT 256
#define PSS_TOPM_MAX 4u          /* per-lane top-m kept for the bound: K <= 1024 */
#define PSS_SEG_MAX_N 64u        /* segments per row (V <= 262144 at SEG >= 4096) */
#define PSS_POOL_CAP 16384u      /* pool entries per row, split evenly over segments */
#define PSS_FIN_LIST_CAP 4096u   /* candidates the finisher gathers in LDS */
#define PSS_FAST_N 1024u         /* candidates the fast finisher handles (K <= 64) */
#define PSS_SEG_WAVES 4u         /* waves per segment workgroup (PSS_ST_NT / 64) */
#define PSS_SEG_OVERFLOW 0xFFFFFFFFu
#define PSS_KEY_NEG_INF 0x007FFFFFu /* pss_key(-inf): the smallest key of any element */

/* Per-row workspace: header, then the candidate pool. */
struct pss_row_ws {
    uint32_t bound; /* row-wide lower bound on the K-th largest key (max over segments) */
    uint32_t pad[15];
    uint32_t seg_count[PSS_SEG_MAX_N * PSS_SEG_WAVES]; /* candidates per (segment, wave), or PSS_SEG_OVERFLOW */
    unsigned long long seg_best[PSS_SEG_MAX_N];  /* greedy rows: (key << 32) | ~id per segment */
};
static_assert(sizeof(pss_row_ws) % 64 == 0, "workspace header is a multiple of 64 bytes");
#define PSS_WS_ROW_BYTES (sizeof(pss_row_ws) + (size_t)PSS_POOL_CAP * 8u)

static inline size_t pss_stream_ws_bytes(uint32_t rows) { return (size_t)rows * PSS_WS_ROW_BYTES; }

/* Pool slots of one (segment, wave) when a row has S segments. */
__host__ __device__ inline uint32_t pss_wave_cap(uint32_t S) { return PSS_POOL_CAP / (S * PSS_SEG_WAVES); }

__device__ __forceinline__ uint32_t pss_ld_agent(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* ------------------------------------------------------------------------ */
/* finisher: selection over the row's candidate list in LDS                  */
/* ------------------------------------------------------------------------ */

struct pss_fin_shared {
    unsigned long long list[PSS_FIN_LIST_CAP]; /* gathered candidates (key << 32 | id) */
    unsigned long long kept[64];               /* fast path: entries >= the K-th largest */
    uint32_t hist[256];                        /* fast path: radix digit counts */
    pss_gen_shared g;
    uint32_t mx[PSS_ST_NT / PSS_WAVE];         /* per-wave largest key */
    uint32_t digit;
    uint32_t rem;
    uint32_t nk;
    uint32_t fail;
};

/*
 * Select by cumulative weight from the top over the list: kw(e, key, w) gives
 * entry e's selection key and weight (w = 0 skips it).  Returns the largest
 * key v with sum_{key >= v} w >= rem (1 <= rem <= total weight).  Digits of 8
 * bits from bit top_shift + 7 down; 256-bin LDS histograms.
 */
template <int NT, class KW>
__device__ __forceinline__ uint32_t pss_list_select(pss_gen_shared& sh, const unsigned long long* list,
                                                    uint32_t n, uint64_t rem, int top_shift, KW kw) {
    const uint32_t tid = threadIdx.x;
    uint32_t prefix = 0, pmask = 0;
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

/* Finish a sampled row from n candidates (LDS) that contain every element at
 * or above the row's K-th largest value.  Any K, any number of ties. */
template <int NT>
__device__ __forceinline__ void pss_list_finish(const pss_args& a, uint32_t row, const pss_rowcfg& c,
                                                const unsigned long long* list, uint32_t n,
                                                pss_gen_shared& sh) {
    const uint32_t tid = threadIdx.x;
    uint64_t mk = 0;
    for (uint32_t i = tid; i < n; i += NT) {
        const uint64_t k = list[i] >> 32;
        mk = k > mk ? k : mk;
    }
    const uint32_t tmaxKey = (uint32_t)block_max_u64<NT>(mk, sh.red);
    const float tmax = pss_unkey(tmaxKey);

    /* S5: exact K-th largest */
    const uint32_t tauK = pss_list_select<NT>(sh, list, n, c.K, 24,
                                              [&](unsigned long long e, uint32_t& k, uint64_t& w) {
                                                  k = (uint32_t)(e >> 32);
                                                  w = 1u;
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
        const uint32_t tauP = pss_list_select<NT>(sh, list, n, need, 24,
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
        tok = pss_list_select<NT>(sh, list, n, Z - target, 16,
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
 * Fast finisher for K <= 64 and up to PSS_FAST_N candidates (sh.list), those
 * below the row-wide bound G ignored:
 *   1. the row's K-th largest by an LDS radix select (8-bit digits), starting
 *      at the first digit below the common prefix of G and the row maximum --
 *      every candidate that matters lies between the two;
 *   2. the <= 64 entries at or above it, one per lane of wave 0: sort by key
 *      (ties by id), scan the masses for the top-p cut, apply min-p, sort the
 *      kept set by id, scan, take the first id whose cumulative mass exceeds
 *      the draw target.  Lane exchanges are DPP / permlane (no LDS).
 * Returns false (nothing written) when more than 64 entries are at or above
 * the K-th largest (heavy ties).
 */
template <int NT>
__device__ __forceinline__ bool pss_list_finish_fast(const pss_args& a, uint32_t row,
                                                     const pss_rowcfg& c, uint32_t n, uint32_t G,
                                                     const pss_row_pre& pre, pss_fin_shared& sh) {
    constexpr int R = (int)(PSS_FAST_N / NT);
    static_assert(NT == 256, "one radix bin per thread");
    if (c.K > 64u || n > PSS_FAST_N) return false;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    uint64_t e[R];
    uint32_t k[R];
    uint32_t kmax = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t i = tid + (uint32_t)r * NT;
        e[r] = i < n ? sh.list[i] : 0ull;
        k[r] = (uint32_t)(e[r] >> 32);
        if (k[r] < G) k[r] = 0u;
        kmax = k[r] > kmax ? k[r] : kmax;
    }
    kmax = wave_max_u32(kmax);
    if (lane == 0) sh.mx[wave] = kmax;
    if (tid == 0) sh.nk = 0;
    __syncthreads();
    uint32_t tmaxKey = 0;
#pragma unroll
    for (int w = 0; w < NT / PSS_WAVE; ++w) tmaxKey = sh.mx[w] > tmaxKey ? sh.mx[w] : tmaxKey;

    /* S5: radix select of the K-th largest below the common prefix */
    const uint32_t d = G ^ tmaxKey;
    uint32_t tauK = tmaxKey;
    if (d) {
        const int hibit = 31 - __clz(d);
        int shift = (hibit / 8) * 8;
        uint32_t pmask = shift + 8 >= 32 ? 0u : ~((1u << (shift + 8)) - 1u);
        uint32_t prefix = tmaxKey & pmask;
        uint32_t rem = c.K;
        for (; shift >= 0; shift -= 8) {
            sh.hist[tid] = 0u;
            __syncthreads();
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (k[r] && (k[r] & pmask) == prefix) atomicAdd(&sh.hist[(k[r] >> shift) & 255u], 1u);
            __syncthreads();
            if (tid < 64) {
                const uint4 h = *(const uint4*)&sh.hist[4u * lane];
                const uint32_t s4 = h.x + h.y + h.z + h.w;
                const uint32_t above = (uint32_t)(wave_incl_suffix_u64(s4) - s4); /* lanes > lane */
                if (above < rem && rem <= above + s4) {
                    uint32_t cum = above, dg = 4u * lane;
                    const uint32_t hv[4] = {h.x, h.y, h.z, h.w};
                    for (int i = 3; i >= 0; --i) {
                        if (cum + hv[i] >= rem) {
                            dg = 4u * lane + (uint32_t)i;
                            break;
                        }
                        cum += hv[i];
                    }
                    sh.digit = dg;
                    sh.rem = rem - cum;
                }
            }
            __syncthreads();
            prefix |= sh.digit << shift;
            pmask |= 0xFFu << shift;
            rem = sh.rem;
        }
        tauK = prefix;
    }

    /* entries at or above the K-th largest, to wave 0 */
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (k[r] && k[r] >= tauK) {
            const uint32_t pos = atomicAdd(&sh.nk, 1u);
            if (pos < 64u) sh.kept[pos] = e[r];
        }
    __syncthreads();
    const uint32_t nK = sh.nk;
    if (nK > 64u) return false;

    if (tid < 64) {
        const bool valid = lane < nK;
        const uint64_t my = valid ? sh.kept[lane] : 0ull;
        const float tmax = pss_unkey(tmaxKey);

        /* S5/S6: descending by key (ties by id), inclusive mass scan */
        const uint64_t sx = dpp_sort_asc_u64(valid ? (((uint64_t)(~(uint32_t)(my >> 32)) << 32) | (uint32_t)my) : ~0ull);
        const bool sv = sx != ~0ull;
        const uint32_t skey = ~(uint32_t)(sx >> 32), sid = (uint32_t)sx;
        const float sp = sv ? pss_prob(pss_unkey(skey), tmax) : 0.0f;
        const uint64_t sq = sv ? pss_fixq(sp) : 0ull;
        const uint64_t P = wave_incl_scan_u64(sq);
        const uint64_t zk = wave_read_u64(P, 63);
        uint32_t tau = tauK;
        if (c.useTopP) {
            const uint64_t need = pss_topp_need(c.topP, zk);
            const uint64_t m = __ballot(sv && P >= need);
            const uint32_t tauP = wave_read_u32(skey, (uint32_t)__ffsll((long long)m) - 1u);
            tau = tauP > tau ? tauP : tau;
        }
        /* S7 */
        const bool kp = sv && skey >= tau && (!c.useMinP || sp >= c.minP);
        const uint64_t kq = kp ? sq : 0ull;
        const uint64_t Z = wave_sum_u64(kq);
        const uint32_t keptCount = (uint32_t)__popcll(__ballot(kp));
        const uint32_t lastAll = wave_max_u32(kp ? sid + 1u : 0u);

        /* S8: kept entries in id order ((id << 46) | q: ids < 2^18, q <= 2^45),
         * cumulative mass, first crossing */
        uint32_t newRng;
        const uint32_t u24 = pss_draw_u24_pre(a.rng_mode, pre.rng, pre.step, row, &newRng);
        const uint64_t target = pss_draw_target(u24, Z);
        const uint64_t ix = dpp_sort_asc_u64(kp ? (((uint64_t)sid << 46) | kq) : ~0ull);
        const bool iv = ix != ~0ull;
        const uint64_t C = wave_incl_scan_u64(iv ? (ix & ((1ull << 46) - 1ull)) : 0ull);
        const uint64_t hit = __ballot(iv && C > target);
        uint32_t tok, flags = 0;
        if (hit) {
            tok = (uint32_t)(wave_read_u64(ix, (uint32_t)__ffsll((long long)hit) - 1u) >> 46);
        } else {
            tok = lastAll > 0u ? lastAll - 1u : 0u;
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
                if (a.kept_mask) atomicOr(&a.kept_mask[(size_t)row * a.mask_words + (sid >> 5)], 1u << (sid & 31u));
                if (a.probs) a.probs[(size_t)row * a.probs_stride + sid] = sp / ((float)Z * 0x1.0p-45f);
            }
        }
        if (lane == 0) {
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
    }
    return true;
}

/* ------------------------------------------------------------------------ */
/* segment kernel                                                            */
/* ------------------------------------------------------------------------ */

template <int EPT, int DT>
struct pss_seg_geom {
    static constexpr int E = (DT == PSS_DTYPE_F16) ? 8 : 4; /* elements per 16-byte load */
    static constexpr int NL = EPT / E;                      /* loads per lane */
    static constexpr uint32_t SEG = (uint32_t)PSS_ST_NT * EPT;
    static constexpr int HPT = (int)((PSS_MAX_PENALTY_LEN + PSS_ST_NT - 1) / PSS_ST_NT);
    static_assert(EPT % E == 0, "EPT must be a multiple of the load width");
};

/* LDS of a segment workgroup.  The penalty bitmap is transposed: word w is
 * thread w's, bit i its register t[i]; it and the per-wave bound exchange
 * are double-buffered (alternating per item that uses them) and cleared by
 * their readers, so an item needs no barrier before it writes them. */
struct pss_seg_shared {
    uint32_t pen[2][PSS_ST_NT];          /* window-id bits per thread */
    uint32_t penOr[2][PSS_SEG_WAVES];    /* OR of the words of each wave */
    uint32_t lb[2][PSS_SEG_WAVES];       /* per-wave bounds (K <= 256) */
    uint32_t topm[PSS_ST_NT * PSS_TOPM_MAX];
    uint64_t red[PSS_ST_NT / PSS_WAVE];
};

/* Lower bound of one segment's K-th largest: the K-th largest of the lanes'
 * top-m keys to 16 bits (R = 4m values per lane of a wave; every wave
 * computes the same value). */
template <int R>
__device__ __forceinline__ uint32_t pss_lane_bound(const uint32_t* topm, uint32_t K) {
    uint32_t v[R];
    const uint32_t lane = pss_tid() & 63u;
#pragma unroll
    for (int i = 0; i < R; ++i) v[i] = topm[lane * R + i];
    return wave_kth_largest_r4<R>(v, K, 0u, 31, 16);
}

/* Row tests from the raw parameters (no division).  A row is covered when
 * it is greedy or its top-k is on and at most 1024 (otherwise the finisher
 * runs the general algorithm on it and the segment kernel skips it). */
__device__ __forceinline__ bool pss_seg_row_greedy(const pss_args& a, const sample_params& sp) {
    return (a.mode == PSS_MODE_GREEDY) || !(sp.temperature > 0.0f);
}
__device__ __forceinline__ bool pss_seg_row_covered(const pss_args& a, const sample_params& sp) {
    const uint32_t K = sp.topK < a.V ? sp.topK : a.V;
    return pss_seg_row_greedy(a, sp) || (K > 0u && K <= (uint32_t)PSS_ST_NT * PSS_TOPM_MAX);
}

/* Buffer resource word 3 for raw (untyped, stride 0) buffer loads on gfx9
 * CDNA parts: 32-bit data format, no swizzle, no index stride. */
#define PSS_BUF_DW3 0x00020000

/* Issue the loads of segment `seg` of `row` into raw[]; nothing here waits
 * for them.  Raw buffer loads over the row (num_records = V * element size):
 * the hardware returns 0 for ids at or beyond V, which the compute step
 * replaces by -inf.  vec_ok (16-byte aligned rows, V a multiple of the
 * elements per 16 bytes): one 16-byte load per 4 fp32 / 8 fp16; otherwise one
 * load per element. */
template <int EPT, int DT>
__device__ __forceinline__ void pss_seg_issue(const pss_args& a, uint32_t row, uint32_t seg,
                                              uint4 (&raw)[pss_seg_geom<EPT, DT>::NL]) {
    using Gm = pss_seg_geom<EPT, DT>;
    constexpr int E = Gm::E, NL = Gm::NL;
    constexpr uint32_t NT = PSS_ST_NT;
    constexpr uint32_t esz = DT == PSS_DTYPE_F16 ? 2u : 4u;
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    const char* rowp = (const char*)a.logits + (size_t)row * a.stride * esz;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)rowp, (short)0, (int)(a.V * esz), PSS_BUF_DW3);
    const uint32_t tid = pss_tid();
    const uint32_t base = seg * Gm::SEG;
    if (a.vec_ok) {
#pragma unroll
        for (int li = 0; li < NL; ++li) {
            const v4u v = __builtin_amdgcn_raw_buffer_load_b128(
                rs, (int)((base + (uint32_t)li * (NT * E) + tid * E) * esz), 0, 0);
            raw[li] = make_uint4(v.x, v.y, v.z, v.w);
        }
    } else {
#pragma unroll
        for (int li = 0; li < NL; ++li) {
            const uint32_t j0 = base + (uint32_t)li * (NT * E) + tid * E;
            uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int e = 0; e < E; ++e) {
                if (DT == PSS_DTYPE_F16)
                    w[e >> 1] |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (int)((j0 + e) * 2u), 0, 0)
                                 << ((e & 1) * 16);
                else
                    w[e] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)((j0 + e) * 4u), 0, 0);
            }
            raw[li] = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
}

/* Per-item values loaded ahead of the item: the row's window ids (sampled
 * rows with a penalty) and the row-wide bound published so far. */
template <int HPT>
struct pss_seg_side {
    uint32_t hid[HPT];
    uint32_t G0;
};

template <int HPT>
__device__ __forceinline__ void pss_seg_side_load(const pss_args& a, uint32_t row, const sample_params& sp,
                                                  pss_seg_side<HPT>& sd) {
    /* the window ids of sampled rows with a window (a superset of the rows
     * that apply a penalty; the compute step decides exactly) */
    const bool greedy = pss_seg_row_greedy(a, sp);
    const uint32_t W = sp.penaltyLength < PSS_MAX_PENALTY_LEN ? sp.penaltyLength : PSS_MAX_PENALTY_LEN;
    const uint32_t* hist_row = a.history + (size_t)row * PSS_MAX_PENALTY_LEN;
#pragma unroll
    for (int h = 0; h < HPT; ++h) {
        const uint32_t idx = pss_tid() + (uint32_t)h * PSS_ST_NT;
        sd.hid[h] = PSS_SENTINEL;
        if (!greedy && idx < W) sd.hid[h] = hist_row[idx];
    }
    const pss_row_ws* ws = (const pss_row_ws*)((const char*)a.ws + (size_t)row * PSS_WS_ROW_BYTES);
    /* The lane-varying (zero) offset keeps the value in a vector register:
     * a uniform load would be moved to a scalar register at once, which
     * waits for every load issued before it. */
    uint32_t z = 0u;
    __asm__ __volatile__("" : "+v"(z));
    sd.G0 = greedy ? 0u : pss_ld_agent(&ws->bound + z);
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

/*
 * One segment (seg, row) whose loads are in raw[].  `carry` is the largest
 * bound this workgroup has established for `carry_row`: every bound is a lower
 * bound of the row's K-th largest, so later segments of the row reuse it
 * instead of deriving their own.
 */
template <int EPT, int DT, bool M1>
__device__ __forceinline__ void pss_seg_compute(const pss_args& a, pss_seg_shared& sh, uint32_t row, uint32_t seg,
                                                uint32_t S, const sample_params& sp,
                                                const uint4 (&raw)[pss_seg_geom<EPT, DT>::NL],
                                                const pss_seg_side<pss_seg_geom<EPT, DT>::HPT>& sd,
                                                uint32_t& carry_row, uint32_t& carry, uint32_t& npen,
                                                uint32_t& nbound) {
    using Gm = pss_seg_geom<EPT, DT>;
    constexpr int NT = PSS_ST_NT;
    constexpr int E = Gm::E, NL = Gm::NL, HPT = Gm::HPT;
    constexpr uint32_t SEG = Gm::SEG;
    static_assert(EPT <= 32, "one bit per register index in a 32-bit word");
    const uint32_t tid = pss_tid();
    const uint32_t V = a.V;
    const uint32_t seg_base = seg * SEG;
    const bool greedy = pss_seg_row_greedy(a, sp);
    const pss_rowcfg c = pss_make_rowcfg(sp, V);
    pss_row_ws* ws = (pss_row_ws*)((char*)a.ws + (size_t)row * PSS_WS_ROW_BYTES);
    const bool doPen = !greedy && c.doPen;

    /* t = l * (1/T) (greedy rows: the raw logit) */
    const float invT = greedy ? 1.0f : c.invT;
    const float NEG_INF = pss_u2f(0xFF800000u);
    float t[EPT];
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

    /* Penalty: every thread holding a window id of this segment sets the
     * owner's bit (element offset o lives in thread (o % (256 E)) / E, register
     * (o / (256 E)) E + o % E) and the owner wave's summary bit; after one
     * barrier each thread reads and clears its word, and the wave penalizes
     * only the register indices some of its lanes hold. */
    if (doPen) {
        const uint32_t b = npen & 1u;
        ++npen;
#pragma unroll
        for (int h = 0; h < HPT; ++h) {
            const uint32_t id = sd.hid[h];
            if (id >= seg_base && id - seg_base < SEG && id < V) {
                const uint32_t o = id - seg_base;
                const uint32_t owner = (o % (uint32_t)(NT * E)) / (uint32_t)E;
                const uint32_t bit = 1u << ((o / (uint32_t)(NT * E)) * (uint32_t)E + o % (uint32_t)E);
                atomicOr(&sh.pen[b][owner], bit);
                atomicOr(&sh.penOr[b][owner >> 6], bit);
            }
        }
        __syncthreads();
        const uint32_t pb = sh.pen[b][tid];
        const uint32_t wor = __builtin_amdgcn_readfirstlane(sh.penOr[b][tid >> 6]);
        sh.pen[b][tid] = 0u;
        if ((tid & 63u) == 0u) sh.penOr[b][tid >> 6] = 0u;
#pragma unroll
        for (int i = 0; i < EPT; ++i)
            if ((wor >> i) & 1u) t[i] = ((pb >> i) & 1u) ? pss_penalize(t[i], c) : t[i];
    }
    auto id_of = [&](uint32_t i) -> uint32_t {
        return seg_base + (i / E) * (NT * E) + tid * E + (i % E);
    };
    /* The row's last segment: ids beyond the vocab read 0; they become -inf,
     * which never passes a bound above key(-inf) and never wins an argmax
     * tie against a real id (larger id); where every element passes they are
     * excluded by id. */
    if (seg_base + SEG > V) {
#pragma unroll
        for (int i = 0; i < EPT; ++i) t[i] = id_of((uint32_t)i) < V ? t[i] : NEG_INF;
    }

    if (greedy) {
        /* argmax of the canonical value, smallest id on ties */
        uint64_t best = 0;
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            const uint64_t b =
                ((uint64_t)pss_key(pss_canon(t[i])) << 32) | (uint64_t)(0xFFFFFFFFu - id_of((uint32_t)i));
            if (b > best) best = b;
        }
        best = block_max_u64<NT>(best, sh.red);
        if (tid == 0) ws->seg_best[seg] = best;
        return;
    }

    /* Bound (first segment of the row in this workgroup).  max() ignores NaN,
     * which canonicalizes to -inf; lanes without elements contribute
     * key(-inf), the smallest key, which never raises the bound above a true
     * order statistic.
     *   M1 (K <= 256): every wave sorts its 64 lane maxima; with K' =
     *   ceil(K / 4), the minimum over the four waves of their K'-th largest
     *   has at least 4 K' >= K distinct elements of the segment at or above
     *   it.  Otherwise every lane's sorted top-4 goes to LDS and every wave
     *   takes the K-th largest of all of them. */
    uint32_t thr = carry_row == row ? carry : 0u;
    if (carry_row != row) {
        uint32_t L;
        if (M1) {
            float mx = NEG_INF;
#pragma unroll
            for (int i = 0; i < EPT; ++i) mx = fmaxf(mx, t[i]);
            const uint32_t srt = dpp_sort_asc_u32(pss_key(pss_canon(mx)));
            const uint32_t kq = (c.K + (uint32_t)PSS_SEG_WAVES - 1u) / (uint32_t)PSS_SEG_WAVES;
            const uint32_t lw = (uint32_t)__builtin_amdgcn_readlane(srt, (int)(64u - kq));
            const uint32_t b = nbound & 1u;
            ++nbound;
            if ((tid & 63u) == 0u) sh.lb[b][tid >> 6] = lw;
            __syncthreads();
            L = min(min(sh.lb[b][0], sh.lb[b][1]), min(sh.lb[b][2], sh.lb[b][3]));
        } else {
            const uint32_t m = (c.K + NT - 1u) / NT;
            uint32_t* topm = sh.topm;
            /* insertion into a sorted top-4 on floats (NaN mapped to -inf
             * first; -0 and +0 order arbitrarily but share one canonical key) */
            float t0 = NEG_INF, t1 = NEG_INF, t2 = NEG_INF, t3 = NEG_INF;
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
            __syncthreads(); /* the previous item's reads of topm are done */
            topm[tid * m + 0] = pss_key(pss_canon(t0));
            if (m > 1u) topm[tid * m + 1] = pss_key(pss_canon(t1));
            if (m > 2u) topm[tid * m + 2] = pss_key(pss_canon(t2));
            if (m > 3u) topm[tid * m + 3] = pss_key(pss_canon(t3));
            __syncthreads();
            if (m == 1u)
                L = pss_lane_bound<4>(topm, c.K);
            else if (m == 2u)
                L = pss_lane_bound<8>(topm, c.K);
            else if (m == 3u)
                L = pss_lane_bound<12>(topm, c.K);
            else
                L = pss_lane_bound<16>(topm, c.K);
        }
        thr = L > thr ? L : thr;
    }
    const uint32_t G0 = __builtin_amdgcn_readfirstlane(sd.G0);
    if (tid == 0 && thr > G0 && thr > PSS_KEY_NEG_INF)
        (void)__hip_atomic_fetch_max(&ws->bound, thr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    thr = G0 > thr ? G0 : thr;
    carry_row = row;
    carry = thr;

    /* Candidates (key >= thr), written by each wave to its own slot range
     * of the pool: a pass mask per lane, a wave scan of the counts, then each
     * lane stores its entries (one select tree per entry).  Above key(-inf)
     * the test is a float compare (t >= unkey(thr) is false for NaN, which
     * canonicalizes to -inf < thr); at or below it every element of the vocab
     * passes. */
    /* bit i of pm: element i passes (built from the top bit down as
     * pm + pm + pass, a shift-in with no per-bit constants) */
    uint32_t pm = 0;
    if (thr <= PSS_KEY_NEG_INF) {
#pragma unroll
        for (int i = EPT - 1; i >= 0; --i) pm = pm + pm + (id_of((uint32_t)i) < V ? 1u : 0u);
    } else {
        const float thr_f = pss_unkey(thr);
#pragma unroll
        for (int i = EPT - 1; i >= 0; --i) pm = pm + pm + (t[i] >= thr_f ? 1u : 0u);
    }
    const uint32_t mine = (uint32_t)__popc(pm);
    const uint32_t incl = wave_incl_scan_u32(mine);
    const uint32_t wtot = wave_read_u32(incl, 63);
    const uint32_t slot = seg * PSS_SEG_WAVES + (tid >> 6);
    const uint32_t capw = pss_wave_cap(S);
    if (wtot <= capw) {
        unsigned long long* out = (unsigned long long*)(ws + 1) + (size_t)slot * capw + (incl - mine);
        while (pm) {
            const uint32_t i = (uint32_t)__builtin_ctz(pm);
            pm &= pm - 1u;
            *out++ = ((unsigned long long)pss_key(pss_canon(pss_pick(t, i))) << 32) | id_of(i);
        }
    }
    if ((tid & 63u) == 0u) ws->seg_count[slot] = wtot <= capw ? wtot : PSS_SEG_OVERFLOW;
}

/* Staging area of one workgroup: each wave's 16-byte loads of one item, lane
 * l of wave w at v[li][w][l] (the layout of a wave's load-to-LDS). */
template <int EPT, int DT>
struct pss_seg_stage {
    uint4 v[pss_seg_geom<EPT, DT>::NL][PSS_SEG_WAVES][PSS_WAVE];
};

/* Issue item (row, seg)'s 16-byte loads straight into the calling wave's part
 * of the staging area (raw buffer loads to LDS: no registers held while they
 * are in flight; 0 for ids at or beyond V).  Requires vec_ok. */
template <int EPT, int DT>
__device__ __forceinline__ void pss_seg_issue_lds(const pss_args& a, uint32_t row, uint32_t seg,
                                                  pss_seg_stage<EPT, DT>& st) {
    using Gm = pss_seg_geom<EPT, DT>;
    constexpr int E = Gm::E, NL = Gm::NL;
    constexpr uint32_t NT = PSS_ST_NT;
    constexpr uint32_t esz = DT == PSS_DTYPE_F16 ? 2u : 4u;
    const char* rowp = (const char*)a.logits + (size_t)row * a.stride * esz;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)rowp, (short)0, (int)(a.V * esz), PSS_BUF_DW3);
    const uint32_t tid = pss_tid();
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t base = seg * Gm::SEG;
#pragma unroll
    for (int li = 0; li < NL; ++li)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, (__attribute__((address_space(3))) void*)&st.v[li][w][0], 16,
            (int)((base + (uint32_t)li * (NT * E) + tid * E) * esz), 0, 0, 0);
}

/*
 * Persistent segment kernel: item i = (row i / S, segment i % S); workgroup b
 * processes items [b * per_wg, min((b + 1) * per_wg, n_items)) in order, and
 * the grid is sized to the resident capacity, so every workgroup runs from
 * the start.  Pipeline (vec_ok): while item j is computed from registers, item
 * j + 1's logits stream into the wave's staging area in LDS and its window
 * ids, row-wide bound and parameters are loaded; at the top of the next
 * iteration the wave waits for them and moves its staged loads to registers.
 * Each wave reads back only what its own loads wrote, so the staging area
 * needs no barrier.  Without vec_ok (unaligned rows, V not a multiple of the
 * elements per 16 bytes) every item loads element-wise at its own start.  M1:
 * every row of the launch has K <= 256 (one top value per lane); the general
 * form keeps a sorted top-4 per lane, which costs registers.  `params` is
 * a.params as a restrict argument: the workgroup's stores cannot alias it, so
 * the row parameters of later items still come through scalar loads.
 */
template <int EPT, int DT, bool M1>
__global__ void __launch_bounds__(PSS_ST_NT) pss_seg_kernel(pss_args a, uint32_t S, uint32_t n_items,
                                                            uint32_t per_wg,
                                                            const sample_params* __restrict__ params) {
    using Gm = pss_seg_geom<EPT, DT>;
    __shared__ pss_seg_shared sh;
    __shared__ pss_seg_stage<EPT, DT> stage;
    pss_globalize(a);
    const uint32_t i0 = blockIdx.x * per_wg;
    const uint32_t i1 = i0 + per_wg < n_items ? i0 + per_wg : n_items;
    if (i0 >= i1) return;
    uint32_t n = i1 - i0; /* items left, the current one included */
    const bool staged = a.vec_ok != 0u;

    uint4 raw[Gm::NL];
    pss_seg_side<Gm::HPT> sd;
    uint32_t carry_row = 0xFFFFFFFFu, carry = 0u, npen = 0u, nbound = 0u;
    auto covered = [&](const sample_params& sp) -> bool { return pss_seg_row_covered(a, sp); };
    {
        const uint32_t tid = pss_tid();
        sh.pen[0][tid] = 0u;
        sh.pen[1][tid] = 0u;
        if (tid < 2u * PSS_SEG_WAVES) (&sh.penOr[0][0])[tid] = 0u;
        __syncthreads();
    }

    /* (row, seg) and parameters of the current item and the next two */
    auto advance = [&](uint32_t& r, uint32_t& g) {
        if (++g == S) {
            g = 0u;
            ++r;
        }
    };
    uint32_t row0 = __builtin_amdgcn_readfirstlane(i0 / S);
    uint32_t seg0 = i0 - row0 * S;
    uint32_t row1 = row0, seg1 = seg0;
    advance(row1, seg1);
    uint32_t row2 = row1, seg2 = seg1;
    advance(row2, seg2);
    sample_params sp0 = params[row0];
    sample_params sp1 = params[n > 1u ? row1 : row0];
    if (staged) {
        pss_seg_issue_lds<EPT, DT>(a, row0, seg0, stage);
        if (covered(sp0)) pss_seg_side_load<Gm::HPT>(a, row0, sp0, sd);
    }
    for (;;) {
        const bool more = n > 1u;
        if (staged) {
            pss_wait_mem(); /* this item's staged loads and side values */
            __asm__ __volatile__("" ::: "memory");
            const uint32_t tid = pss_tid();
            const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
#pragma unroll
            for (int li = 0; li < Gm::NL; ++li) raw[li] = stage.v[li][w][tid & 63u];
            pss_wait_mem(); /* the staging area is free again */
            __asm__ __volatile__("" ::: "memory");
        } else {
            pss_seg_issue<EPT, DT>(a, row0, seg0, raw);
            if (covered(sp0)) pss_seg_side_load<Gm::HPT>(a, row0, sp0, sd);
        }
        const pss_seg_side<Gm::HPT> cur = sd;
        const sample_params sp2 = params[n > 2u ? row2 : row0];
        if (staged && more) {
            pss_seg_issue_lds<EPT, DT>(a, row1, seg1, stage);
            if (covered(sp1)) pss_seg_side_load<Gm::HPT>(a, row1, sp1, sd);
            __asm__ __volatile__("" ::: "memory");
        }
        if (covered(sp0))
            pss_seg_compute<EPT, DT, M1>(a, sh, row0, seg0, S, sp0, raw, cur, carry_row, carry, npen, nbound);
        if (!more) break;
        --n;
        row0 = row1, seg0 = seg1, sp0 = sp1;
        row1 = row2, seg1 = seg2, sp1 = sp2;
        advance(row2, seg2);
    }
}

/* ------------------------------------------------------------------------ */
/* finisher kernel                                                           */
/* ------------------------------------------------------------------------ */

/* One workgroup per row; S segments per row were written by pss_seg_kernel. */
__global__ void __launch_bounds__(PSS_ST_NT) pss_fin_kernel(pss_args a, uint32_t S) {
    constexpr int NT = PSS_ST_NT;
    __shared__ pss_fin_shared sh;
    __shared__ uint32_t bits[PSS_MAX_VOCAB / 32];
    pss_globalize(a);
    const uint32_t row = blockIdx.x, tid = threadIdx.x;
    const uint32_t V = a.V;
    const sample_params sp = a.params[row];
    const bool greedy = (a.mode == PSS_MODE_GREEDY) || !(sp.temperature > 0.0f);
    const pss_rowcfg c = pss_make_rowcfg(sp, V);
    pss_row_ws* ws = (pss_row_ws*)((char*)a.ws + (size_t)row * PSS_WS_ROW_BYTES);
    pss_row_pre pre;
    pre.rng = a.rng[row];
    pre.step = a.step[row];
    pre.pos = a.position[row];

    if (greedy) {
        uint64_t best = 0;
        for (uint32_t s = tid; s < S; s += NT) best = ws->seg_best[s] > best ? ws->seg_best[s] : best;
        best = block_max_u64<NT>(best, sh.g.red);
        pss_greedy_finish<NT>(a, row, best);
        return;
    }
    bool general = !(c.K > 0u && c.K <= (uint32_t)NT * PSS_TOPM_MAX);
    if (!general) {
        /* Gather: slot counts in one round trip, their prefix sums, then each
         * slot's owner thread copies its entries to the LDS list at its
         * offset (the entries in one more round trip). */
        const uint32_t G = ws->bound;
        const uint32_t NS = S * PSS_SEG_WAVES;
        const uint32_t capw = pss_wave_cap(S);
        const uint32_t ns = tid < NS ? ws->seg_count[tid] : 0u;
        const bool over = ns == PSS_SEG_OVERFLOW;
        const uint32_t n0 = over ? 0u : ns;
        if (tid == 0) sh.fail = 0;
        uint64_t total64;
        const uint32_t off = (uint32_t)block_excl_scan_u64<NT>(n0, sh.g.red, &total64);
        if (over) sh.fail = 1u;
        const uint32_t total = (uint32_t)total64;
        if (n0 && total <= PSS_FIN_LIST_CAP) {
            const unsigned long long* src = (const unsigned long long*)(ws + 1) + (size_t)tid * capw;
            for (uint32_t i0 = 0; i0 < n0; i0 += 8u) {
                unsigned long long v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) v[u] = i0 + u < n0 ? src[i0 + u] : 0ull;
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (i0 + u < n0) sh.list[off + i0 + u] = v[u];
            }
        }
        __syncthreads();
        general = sh.fail != 0u || total > PSS_FIN_LIST_CAP;
        if (!general && !pss_list_finish_fast<NT>(a, row, c, total, G, pre, sh)) {
            /* slow path: candidates below the row-wide bound may remain in the
             * list; they are below the K-th largest and never selected */
            pss_list_finish<NT>(a, row, c, sh.list, total, sh.g);
        }
        if (tid == 0) ws->bound = 0u; /* for the next launch */
    }
    if (general) pss_general_row<NT>(a, row, sh.g, bits, PSS_MAX_VOCAB / 32);
}

/* ---------------------------------------------------------------------- */
/* host-side launch                                                        */
/* ---------------------------------------------------------------------- */

/* Elements per lane: 32 (8192-id segments, one pass bit per element in a
 * 32-bit mask), or 16 for vocabularies that would otherwise exceed
 * PSS_SEG_MAX_N segments (none at V <= 262,144) or give fewer than 8 items. */
static inline int pss_stream_pick_ept(uint32_t V, uint32_t rows) {
    const uint64_t S32 = (V + (uint64_t)PSS_ST_NT * 32u - 1u) / ((uint64_t)PSS_ST_NT * 32u);
    if (S32 > PSS_SEG_MAX_N || (uint64_t)rows * S32 < 8u) return 16;
    return 32;
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
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, pss_seg_kernel<EPT, DT, M1>, PSS_ST_NT, 0) !=
        hipSuccess)
        return 0;
    const uint32_t cap = (uint32_t)(nb > 0 ? nb : 1) * (uint32_t)(cus > 0 ? cus : 1);
    if (dev < 64) cache[dev] = cap;
    return cap;
}

template <int EPT, int DT, bool M1>
static inline hipError_t pss_seg_launch(const pss_args& a, uint32_t S, uint32_t n_items, hipStream_t st) {
    uint32_t cap = pss_seg_capacity<EPT, DT, M1>();
    if (cap == 0) cap = n_items;
    const uint32_t per_wg = (n_items + cap - 1u) / cap;
    const uint32_t grid = (n_items + per_wg - 1u) / per_wg;
    pss_seg_kernel<EPT, DT, M1><<<dim3(grid), dim3(PSS_ST_NT), 0, st>>>(a, S, n_items, per_wg, a.params);
    return hipGetLastError();
}

template <int EPT>
static inline hipError_t pss_stream_go(const pss_args& a, uint32_t rows, uint32_t max_k, hipStream_t st,
                                       hipEvent_t split) {
    const uint32_t seg = (uint32_t)PSS_ST_NT * EPT;
    const uint32_t S = (a.V + seg - 1u) / seg;
    if ((uint64_t)rows * S >= (1ull << 31)) return hipErrorInvalidValue;
    const uint32_t n_items = rows * S;
    const bool m1 = max_k <= (uint32_t)PSS_ST_NT;
    hipError_t e;
    if (a.dtype == PSS_DTYPE_F16)
        e = m1 ? pss_seg_launch<EPT, PSS_DTYPE_F16, true>(a, S, n_items, st)
               : pss_seg_launch<EPT, PSS_DTYPE_F16, false>(a, S, n_items, st);
    else
        e = m1 ? pss_seg_launch<EPT, PSS_DTYPE_F32, true>(a, S, n_items, st)
               : pss_seg_launch<EPT, PSS_DTYPE_F32, false>(a, S, n_items, st);
    if (e != hipSuccess) return e;
    if (split && (e = hipEventRecord(split, st)) != hipSuccess) return e;
    pss_fin_kernel<<<dim3(rows), dim3(PSS_ST_NT), 0, st>>>(a, S);
    return hipGetLastError();
}

/* max_k: the largest top-k of the launched rows (an upper bound is enough). */
static inline hipError_t pss_stream_launch(pss_args a, uint32_t rows, uint32_t max_k, hipStream_t st,
                                           hipEvent_t split) {
    const size_t esz = a.dtype == PSS_DTYPE_F16 ? 2u : 4u;
    a.vec_ok = ((a.stride * esz) % 16u == 0u) && (((uintptr_t)a.logits & 15u) == 0u) &&
               ((a.V * esz) % 16u == 0u);
    switch (pss_stream_pick_ept(a.V, rows)) {
        case 32: return pss_stream_go<32>(a, rows, max_k, st, split);
        default: return pss_stream_go<16>(a, rows, max_k, st, split);
    }
}

#endif /* PSS_STREAM_H */
