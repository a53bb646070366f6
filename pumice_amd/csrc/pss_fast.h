/*
 * pss_fast.h - the register-resident sampler kernel.
 *
 * Grid (S, rows): workgroup (s, r) owns segment s of row r, SEG = NT * EPT
 * consecutive ids.  One HBM pass: 16-byte coalesced loads (4 fp32 / 8 fp16 per
 * lane), the fp32 transform (temperature, repetition / presence penalty from
 * an LDS bitmap of the segment's ids in the window), order-preserving keys kept
 * in registers (EPT per lane).  Nothing re-reads the row afterwards:
 *
 *   1. lower bound L on the K-th largest value: the K-th largest of the
 *      per-lane top-m values (m = ceil(K / NT)), a subset of the segment, so
 *      every element at or above the row's K-th largest is >= L;
 *   2. candidates = elements with key >= L, appended to an LDS list
 *      (typically K..2K entries);
 *   3. S == 1: finish the row from the list.  S > 1: each segment appends its
 *      local top-K (and publishes its K-th largest as a row-wide bound with
 *      atomicMax) to a per-row pool in global memory; the last segment to
 *      arrive (atomic ticket, release/acquire fences) loads the pool and
 *      finishes the row, then clears the row's workspace for the next launch;
 *   4. finish: exact K-th largest (LDS radix select, 8-bit digits), masses
 *      q = trunc(exp(t - tmax) * 2^45) of the survivors, top-p by a
 *      mass-weighted radix select, min-p, and the draw as a mass-weighted
 *      radix select over ids (the smallest id whose cumulative kept mass
 *      exceeds floor(u24 * Z / 2^24)).
 *
 * Rows it cannot finish from candidates -- top-k off or above NT * 4,
 * candidate lists over capacity (heavy ties) -- run the general algorithm in
 * the same launch, on the workgroup that finishes the row.  Results are
 * bit-identical to the general kernel.
 */
#ifndef PSS_FAST_H
#define PSS_FAST_H

#include "pss_general.h"

#define PSS_POOL_CAP 8192u   /* candidates per row across segments */
#define PSS_LDS_CAP 8192u    /* candidates one workgroup holds in LDS */
#define PSS_TOPM_MAX 4u
#define PSS_SEG_MAX 102400u  /* largest segment (512 x 200) */
#define PSS_WS_OVERFLOW 1u

/* Per-row workspace header; the row's candidate pool follows it. */
struct pss_row_ws {
    uint32_t ticket;  /* segments arrived */
    uint32_t count;   /* pool entries appended */
    uint32_t maxkey;  /* row maximum key */
    uint32_t bound;   /* published lower bound on the K-th largest key */
    uint32_t flags;
    uint32_t pad[3];
    unsigned long long greedy_best; /* (key << 32) | ~id */
    unsigned long long pad2[3];
};
static_assert(sizeof(pss_row_ws) == 64, "workspace header is 64 bytes");
#define PSS_WS_ROW_BYTES (sizeof(pss_row_ws) + (size_t)PSS_POOL_CAP * 8u)

static inline size_t pss_fast_ws_bytes(uint32_t V, uint32_t rows) {
    (void)V;
    return (size_t)rows * PSS_WS_ROW_BYTES;
}

template <int NT>
struct pss_fast_shared {
    union {
        struct {
            uint32_t ckey[PSS_LDS_CAP];
            uint32_t cid[PSS_LDS_CAP];
            uint32_t penBits[PSS_SEG_MAX / 32];
            uint32_t topm[NT * PSS_TOPM_MAX];
        } f;
        pss_gen_shared<NT> g;
    };
    uint64_t hist[256];
    uint64_t red[NT / PSS_WAVE];
    uint64_t rem;
    uint32_t digit;
    uint32_t count;
    uint32_t count2;
    uint32_t last;
    uint32_t base;
};

/* Agent-scope loads of workspace fields written by other workgroups. */
__device__ inline uint32_t pss_ld_agent(uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline unsigned long long pss_ld_agent64(unsigned long long* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/*
 * Select by cumulative weight from the top over an LDS list: kw(i, &key, &w)
 * gives item i's key and weight (w = 0 skips it).  Returns the largest key v
 * with sum_{key >= v} w >= rem (rem >= 1 and <= the total weight), i.e. the
 * rem-th largest by weight.  Digits of 8 bits from bit top_shift + 7 down.
 */
template <int NT, class KW>
__device__ inline uint32_t pss_lds_select(pss_fast_shared<NT>& sh, uint32_t n, uint64_t rem,
                                          int top_shift, KW kw) {
    const uint32_t tid = threadIdx.x;
    uint32_t prefix = 0, pmask = 0;
    for (int shift = top_shift; shift >= 0; shift -= 8) {
        for (uint32_t i = tid; i < 256u; i += NT) sh.hist[i] = 0;
        __syncthreads();
        for (uint32_t i = tid; i < n; i += NT) {
            uint32_t k;
            uint64_t w;
            kw(i, k, w);
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

/* Finish a sampled row from a candidate list (sh.f.ckey / sh.f.cid, n entries)
 * that contains every element at or above the row's K-th largest value. */
template <int NT>
__device__ void pss_fast_finish(const pss_args& a, uint32_t row, const pss_rowcfg& c,
                                uint32_t tmaxKey, uint32_t n, pss_fast_shared<NT>& sh) {
    const uint32_t tid = threadIdx.x;
    const float tmax = pss_unkey(tmaxKey);
    const uint32_t* ck = sh.f.ckey;
    const uint32_t* ci = sh.f.cid;

    /* S5: exact K-th largest */
    const uint32_t tauK = pss_lds_select<NT>(sh, n, c.K, 24, [&](uint32_t i, uint32_t& k, uint64_t& w) {
        k = ck[i];
        w = 1;
    });
    auto qof = [&](uint32_t i) -> uint64_t { return pss_fixq(pss_prob(pss_unkey(ck[i]), tmax)); };
    uint64_t zl = 0;
    for (uint32_t i = tid; i < n; i += NT)
        if (ck[i] >= tauK) zl += qof(i);
    const uint64_t zk = block_sum_u64<NT>(zl, sh.red);

    /* S6 */
    uint32_t tau = tauK;
    if (c.useTopP) {
        const uint64_t need = pss_topp_need(c.topP, zk);
        const uint32_t tauP = pss_lds_select<NT>(sh, n, need, 24, [&](uint32_t i, uint32_t& k, uint64_t& w) {
            k = ck[i];
            w = k >= tauK ? qof(i) : 0;
        });
        tau = tauP > tau ? tauP : tau;
    }

    /* S7 */
    auto kept = [&](uint32_t i, uint64_t* q, float* p) -> bool {
        *p = pss_prob(pss_unkey(ck[i]), tmax);
        bool k = ck[i] >= tau && (!c.useMinP || *p >= c.minP);
        *q = k ? pss_fixq(*p) : 0;
        return k;
    };
    uint64_t zs = 0;
    uint32_t cnt = 0, lastKept = 0;
    for (uint32_t i = tid; i < n; i += NT) {
        uint64_t q;
        float p;
        if (kept(i, &q, &p)) {
            zs += q;
            cnt++;
            lastKept = ci[i] + 1u > lastKept ? ci[i] + 1u : lastKept;
        }
    }
    const uint64_t Z = block_sum_u64<NT>(zs, sh.red);
    const uint32_t keptCount = (uint32_t)block_sum_u64<NT>(cnt, sh.red);
    const uint32_t lastAll = (uint32_t)block_max_u64<NT>(lastKept, sh.red);

    /* S8: smallest id whose cumulative kept mass exceeds the target, i.e. the
     * largest id v with sum_{id >= v} q >= Z - target. */
    uint32_t newRng;
    const uint32_t u24 = pss_draw_u24(a, row, &newRng);
    const uint64_t target = pss_draw_target(u24, Z);
    uint32_t tok, flags = 0;
    if (Z > 0) {
        tok = pss_lds_select<NT>(sh, n, Z - target, 16, [&](uint32_t i, uint32_t& k, uint64_t& w) {
            float p;
            k = ci[i];
            kept(i, &w, &p);
        });
    } else {
        tok = lastAll > 0u ? lastAll - 1u : 0u;
        flags |= PSS_INFO_FALLBACK;
    }

    /* verification outputs */
    if (a.kept_mask) {
        uint32_t* m = a.kept_mask + (size_t)row * a.mask_words;
        for (uint32_t w = tid; w < a.mask_words; w += NT) m[w] = 0u;
        __syncthreads();
        for (uint32_t i = tid; i < n; i += NT) {
            uint64_t q;
            float p;
            if (kept(i, &q, &p)) atomicOr(&m[ci[i] >> 5], 1u << (ci[i] & 31u));
        }
    }
    if (a.probs) {
        float* pr = a.probs + (size_t)row * a.probs_stride;
        for (uint32_t j = tid; j < a.V; j += NT) pr[j] = 0.0f;
        __syncthreads();
        const float zf = (float)Z * 0x1.0p-45f;
        for (uint32_t i = tid; i < n; i += NT) {
            uint64_t q;
            float p;
            if (kept(i, &q, &p)) pr[ci[i]] = p / zf;
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

/* Release this workgroup's global writes and take a ticket; returns true in
 * every thread of the workgroup that arrives last (S-th) for the row. */
template <int NT>
__device__ inline bool pss_arrive(pss_row_ws* ws, uint32_t S, pss_fast_shared<NT>& sh) {
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) sh.last = (atomicAdd(&ws->ticket, 1u) == S - 1u) ? 1u : 0u;
    __syncthreads();
    const bool last = sh.last != 0u;
    if (last) __threadfence();
    return last;
}

__device__ inline void pss_ws_clear(pss_row_ws* ws) {
    ws->ticket = 0;
    ws->count = 0;
    ws->maxkey = 0;
    ws->bound = 0;
    ws->flags = 0;
    ws->greedy_best = 0;
}

template <int NT, int EPT, int DT>
__global__ void __launch_bounds__(NT) pss_fast_kernel(pss_args a) {
    __shared__ pss_fast_shared<NT> sh;
    constexpr int E = (DT == PSS_DTYPE_F16) ? 8 : 4; /* elements per 16-byte load */
    constexpr int NL = EPT / E;
    constexpr uint32_t SEG = (uint32_t)NT * EPT;
    static_assert(EPT % E == 0, "EPT must be a multiple of the load width");
    static_assert(SEG <= PSS_SEG_MAX, "segment larger than the LDS bitmap");

    const uint32_t seg = blockIdx.x, row = blockIdx.y, S = gridDim.x;
    const uint32_t tid = threadIdx.x;
    const uint32_t V = a.V;
    const uint32_t seg_base = seg * SEG;
    const sample_params sp = a.params[row];
    const bool greedy = (a.mode == PSS_MODE_GREEDY) || !(sp.temperature > 0.0f);
    const pss_rowcfg c = pss_make_rowcfg(sp, V);
    pss_row_ws* ws = (pss_row_ws*)((char*)a.ws + (size_t)row * PSS_WS_ROW_BYTES);
    unsigned long long* pool = (unsigned long long*)(ws + 1);

    /* Rows the candidate path does not cover run the general algorithm on the
     * workgroup that finishes the row. */
    const bool general = !greedy && !(c.K > 0u && c.K <= (uint32_t)NT * PSS_TOPM_MAX);
    if (general) {
        if (S == 1u) {
            pss_general_row<NT>(a, row, sh.g);
        } else if (pss_arrive<NT>(ws, S, sh)) {
            pss_general_row<NT>(a, row, sh.g);
            if (tid == 0) pss_ws_clear(ws);
        }
        return;
    }

    /* Penalty bitmap of this segment's ids. */
    const bool doPen = !greedy && c.doPen;
    if (doPen) {
        for (uint32_t i = tid; i < SEG / 32u; i += NT) sh.f.penBits[i] = 0u;
        __syncthreads();
        const uint32_t* hist_row = a.history + (size_t)row * PSS_MAX_PENALTY_LEN;
        for (uint32_t h = tid; h < c.W; h += NT) {
            uint32_t id = hist_row[h];
            if (id >= seg_base && id < seg_base + SEG && id < V) {
                uint32_t o = id - seg_base;
                atomicOr(&sh.f.penBits[o >> 5], 1u << (o & 31u));
            }
        }
        __syncthreads();
    }

    /* One pass over HBM: keys of the segment in registers (0 = no element). */
    const size_t esz = DT == PSS_DTYPE_F16 ? 2u : 4u;
    const char* rowp = (const char*)a.logits + (size_t)row * a.stride * esz;
    uint32_t keys[EPT];
#pragma unroll
    for (int li = 0; li < NL; ++li) {
        const uint32_t j0 = seg_base + (uint32_t)li * (NT * E) + tid * E;
        float v[E];
        if (a.vec_ok && j0 + E <= V) {
            if (DT == PSS_DTYPE_F16) {
                const uint4 raw = *(const uint4*)(rowp + (size_t)j0 * 2u);
                const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    uint16_t h = (uint16_t)(w[e >> 1] >> ((e & 1) * 16));
                    _Float16 hf;
                    __builtin_memcpy(&hf, &h, 2);
                    v[e] = (float)hf;
                }
            } else {
                const float4 f = *(const float4*)(rowp + (size_t)j0 * 4u);
                v[0] = f.x;
                v[1] = f.y;
                v[2] = f.z;
                v[3] = f.w;
            }
        } else {
#pragma unroll
            for (int e = 0; e < E; ++e) v[e] = (j0 + e < V) ? pss_load1(rowp, DT, j0 + e) : 0.0f;
        }
        uint32_t bits = 0;
        if (doPen) bits = sh.f.penBits[(j0 - seg_base) >> 5] >> ((j0 - seg_base) & 31u);
#pragma unroll
        for (int e = 0; e < E; ++e) {
            uint32_t k;
            if (greedy)
                k = pss_key(pss_canon(v[e]));
            else
                k = pss_key(pss_transform(v[e], (bits >> e) & 1u, c));
            keys[li * E + e] = (j0 + e < V) ? k : 0u;
        }
    }

    if (greedy) {
        uint64_t best = 0;
#pragma unroll
        for (int li = 0; li < NL; ++li)
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const uint32_t j = seg_base + (uint32_t)li * (NT * E) + tid * E + e;
                const uint64_t b = ((uint64_t)keys[li * E + e] << 32) | (uint64_t)(0xFFFFFFFFu - j);
                if (keys[li * E + e] && b > best) best = b;
            }
        best = block_max_u64<NT>(best, sh.red);
        if (S == 1u) {
            pss_greedy_finish<NT>(a, row, best);
            return;
        }
        if (tid == 0) atomicMax(&ws->greedy_best, (unsigned long long)best);
        if (pss_arrive<NT>(ws, S, sh)) {
            pss_greedy_finish<NT>(a, row, pss_ld_agent64(&ws->greedy_best));
            if (tid == 0) pss_ws_clear(ws);
        }
        return;
    }

    /* Per-lane top-m (m = ceil(K/NT)) and the segment maximum. */
    const uint32_t m = (c.K + NT - 1u) / NT;
    uint32_t t0 = 0, t1 = 0, t2 = 0, t3 = 0;
    if (m == 1u) {
#pragma unroll
        for (int i = 0; i < EPT; ++i) t0 = keys[i] > t0 ? keys[i] : t0;
    } else {
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
            uint32_t x = keys[i], y;
            y = t0 < x ? t0 : x;
            t0 = t0 > x ? t0 : x;
            x = y;
            y = t1 < x ? t1 : x;
            t1 = t1 > x ? t1 : x;
            x = y;
            y = t2 < x ? t2 : x;
            t2 = t2 > x ? t2 : x;
            x = y;
            t3 = t3 > x ? t3 : x;
        }
    }
    const uint32_t segMax = (uint32_t)block_max_u64<NT>(t0, sh.red);
    sh.f.topm[tid * m + 0] = t0;
    if (m > 1u) sh.f.topm[tid * m + 1] = t1;
    if (m > 2u) sh.f.topm[tid * m + 2] = t2;
    if (m > 3u) sh.f.topm[tid * m + 3] = t3;
    if (tid == 0) sh.count = 0;
    __syncthreads();
    const uint32_t* topm = sh.f.topm;
    uint32_t L = pss_lds_select<NT>(sh, NT * m, c.K, 24, [&](uint32_t i, uint32_t& k, uint64_t& w) {
        k = topm[i];
        w = 1;
    });
    if (L == 0u) L = 1u; /* fewer than K elements: take every element */

    /* Candidates: every element >= L. */
#pragma unroll
    for (int li = 0; li < NL; ++li)
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const uint32_t k = keys[li * E + e];
            if (k >= L) {
                const uint32_t pos = atomicAdd(&sh.count, 1u);
                if (pos < PSS_LDS_CAP) {
                    sh.f.ckey[pos] = k;
                    sh.f.cid[pos] = seg_base + (uint32_t)li * (NT * E) + tid * E + e;
                }
            }
        }
    __syncthreads();
    const uint32_t n = sh.count;
    const bool overflow = n > PSS_LDS_CAP;

    if (S == 1u) {
        __syncthreads();
        if (overflow)
            pss_general_row<NT>(a, row, sh.g);
        else
            pss_fast_finish<NT>(a, row, c, segMax, n, sh);
        return;
    }

    /* Multi-segment: publish this segment's top-K and arrive. */
    const uint32_t nvalid = V - seg_base < SEG ? V - seg_base : SEG;
    if (!overflow) {
        uint32_t thr = 1u;
        if (nvalid >= c.K) {
            const uint32_t* ck = sh.f.ckey;
            const uint32_t tauS = pss_lds_select<NT>(sh, n, c.K, 24, [&](uint32_t i, uint32_t& k, uint64_t& w) {
                k = ck[i];
                w = 1;
            });
            if (tid == 0) atomicMax(&ws->bound, tauS);
            thr = tauS;
        }
        const uint32_t G = pss_ld_agent(&ws->bound);
        thr = G > thr ? G : thr;
        uint32_t mine = 0;
        for (uint32_t i = tid; i < n; i += NT) mine += sh.f.ckey[i] >= thr ? 1u : 0u;
        const uint32_t tot = (uint32_t)block_sum_u64<NT>(mine, sh.red);
        if (tid == 0) {
            sh.base = atomicAdd(&ws->count, tot);
            sh.count2 = 0;
        }
        __syncthreads();
        const uint32_t base = sh.base;
        for (uint32_t i = tid; i < n; i += NT) {
            if (sh.f.ckey[i] < thr) continue;
            const uint32_t pos = base + atomicAdd(&sh.count2, 1u);
            if (pos < PSS_POOL_CAP)
                pool[pos] = ((unsigned long long)sh.f.ckey[i] << 32) | sh.f.cid[i];
        }
        if (tid == 0) {
            if (base + tot > PSS_POOL_CAP) atomicOr(&ws->flags, PSS_WS_OVERFLOW);
            atomicMax(&ws->maxkey, segMax);
        }
    } else if (tid == 0) {
        atomicOr(&ws->flags, PSS_WS_OVERFLOW);
    }
    if (!pss_arrive<NT>(ws, S, sh)) return;

    /* Last segment of the row: merge the pool and finish. */
    const uint32_t flags = pss_ld_agent(&ws->flags);
    const uint32_t total = pss_ld_agent(&ws->count);
    if ((flags & PSS_WS_OVERFLOW) || total > PSS_POOL_CAP) {
        pss_general_row<NT>(a, row, sh.g);
        if (tid == 0) pss_ws_clear(ws);
        return;
    }
    const uint32_t G = pss_ld_agent(&ws->bound);
    const uint32_t tmaxKey = pss_ld_agent(&ws->maxkey);
    if (tid == 0) sh.count = 0;
    __syncthreads();
    for (uint32_t i = tid; i < total; i += NT) {
        const unsigned long long e = __hip_atomic_load(&pool[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t k = (uint32_t)(e >> 32);
        if (k >= G) {
            const uint32_t pos = atomicAdd(&sh.count, 1u);
            sh.f.ckey[pos] = k;
            sh.f.cid[pos] = (uint32_t)e;
        }
    }
    __syncthreads();
    const uint32_t nm = sh.count;
    __syncthreads();
    pss_fast_finish<NT>(a, row, c, tmaxKey, nm, sh);
    if (tid == 0) pss_ws_clear(ws);
}

/* ---------------------------------------------------------------------- */
/* host-side launch                                                        */
/* ---------------------------------------------------------------------- */

struct pss_fast_cfg {
    int nt;
    int ept;
};

/* Largest per-workgroup segment that still gives >= ~one workgroup per CU;
 * small batches get the smallest segments (most workgroups per row). */
static inline pss_fast_cfg pss_fast_pick(uint32_t V, uint32_t rows) {
    static const pss_fast_cfg cfgs[] = {{512, 200}, {512, 128}, {512, 64}, {256, 32}, {256, 16}};
    for (const pss_fast_cfg& f : cfgs) {
        uint64_t seg = (uint64_t)f.nt * f.ept;
        uint64_t S = (V + seg - 1) / seg;
        if ((uint64_t)rows * S >= 240u) return f;
    }
    return cfgs[4];
}

static inline int pss_fast_supported(uint32_t V, uint32_t dtype, uint32_t rows) {
    (void)dtype;
    (void)rows;
    return V >= 1u && V <= PSS_MAX_VOCAB;
}

template <int NT, int EPT>
static inline hipError_t pss_fast_go(const pss_args& a, uint32_t rows, hipStream_t st) {
    const uint32_t seg = (uint32_t)NT * EPT;
    const uint32_t S = (a.V + seg - 1u) / seg;
    dim3 grid(S, rows), block(NT);
    if (a.dtype == PSS_DTYPE_F16)
        pss_fast_kernel<NT, EPT, PSS_DTYPE_F16><<<grid, block, 0, st>>>(a);
    else
        pss_fast_kernel<NT, EPT, PSS_DTYPE_F32><<<grid, block, 0, st>>>(a);
    return hipGetLastError();
}

static inline hipError_t pss_fast_launch(pss_args a, uint32_t rows, hipStream_t st) {
    const size_t esz = a.dtype == PSS_DTYPE_F16 ? 2u : 4u;
    a.vec_ok = ((a.stride * esz) % 16u == 0u) && (((uintptr_t)a.logits & 15u) == 0u);
    const pss_fast_cfg f = pss_fast_pick(a.V, rows);
    if (f.nt == 512 && f.ept == 200) return pss_fast_go<512, 200>(a, rows, st);
    if (f.nt == 512 && f.ept == 128) return pss_fast_go<512, 128>(a, rows, st);
    if (f.nt == 512 && f.ept == 64) return pss_fast_go<512, 64>(a, rows, st);
    if (f.nt == 256 && f.ept == 32) return pss_fast_go<256, 32>(a, rows, st);
    return pss_fast_go<256, 16>(a, rows, st);
}

#endif /* PSS_FAST_H */
