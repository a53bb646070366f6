/*
 * pss_general.h - the general sampler algorithm for one row, run by one
 * workgroup: exact for every parameter mix and every input distribution
 * (heavy ties, all-equal rows, +-inf, NaN).  It re-reads the row from memory
 * for each radix level (8-bit digits, LDS histograms), so it is the
 * correctness baseline and the in-kernel fallback of the streaming kernel,
 * not the roofline path.
 *
 * The penalty window is an LDS bitmap of `bit_words` words supplied by the
 * caller.  When it covers the whole vocab it is built once; otherwise every
 * pass walks the row in chunks of bit_words * 32 ids and rebuilds the bitmap
 * per chunk, so the fallback fits in a few KB of LDS.
 *
 * Semantics per row (reference: shader/Utility/ArgMax-Reduce.comp):
 *   S0 T <= 0 (or mode GREEDY): argmax of raw logits, smallest id on ties
 *      (:135-167), position += do_inc, no history / rng change.
 *   S1/S2 t = l * (1/T); ids in history[0..W) get t = t>0 ? t/rep : t*rep
 *      (if rep != 1) then t -= pres (:222-265); NaN -> -inf, -0 -> +0.
 *   S3 tmax = max t.  S4 p = exp(t - tmax), q = trunc(p * 2^45).
 *   S5 tau_k = K-th largest t (ties kept).   S6 tau_p = largest v with
 *      sum_{t >= v} q >= ceil(topP * Z_k).   S7 kept: t >= max(tau_k, tau_p)
 *      and p >= minP.   S8 first kept id (ascending) with cumulative q >
 *      floor(u24 * Z / 2^24).   S9 epilogue (:376-385).
 */
#ifndef PSS_GENERAL_H
#define PSS_GENERAL_H

#include "pss_device.h"

#include <type_traits>

#define PSS_GEN_NT 1024
#define PSS_GEN_U 8 /* ids per thread per pass step, loads requested together */
#define PSS_NO_TOKEN 0xFFFFFFFFu

/* Output stores of the epilogue: plain stores.  (Write-through agent-scope
 * stores end a headline step ~0.3 us earlier but slow the 256-id-window fp16
 * workload by ~10 us per step, so they are not used.) */
__device__ __forceinline__ void pss_out(uint32_t* p, uint32_t v) { *p = v; }

/* pss_epilogue with the row's position and Philox step already loaded. */
__device__ __forceinline__ void pss_epilogue_pre(const pss_args& a, uint32_t row, uint32_t tok, bool greedy,
                                                 uint32_t W, uint32_t new_rng, const pss_row_info& inf,
                                                 uint32_t pos, uint32_t step) {
    pss_out(&a.result[row * PSS_RESULT_SLOTS + a.pass_idx], tok);
    pss_out(&a.token_ids[row], tok);
    if (!greedy) {
        if (W > 0u) pss_out(&a.history[row * PSS_MAX_PENALTY_LEN + pos % W], tok);
        if (a.rng_mode == PSS_RNG_PHILOX)
            pss_out(&a.step[row], step + 1u);
        else
            pss_out(&a.rng[row], new_rng);
    }
    if (a.do_inc) pss_out(&a.position[row], pos + 1u);
    if (a.gate && row == 0u && tok == a.eos)
        (void)__hip_atomic_fetch_min(a.gate, a.gate_seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (a.host_tokens) a.host_tokens[row] = tok;
    if (a.info) a.info[row] = inf;
}

/* Row-level epilogue (ArgMax-Reduce.comp:376-385 for sampled rows,
 * :161-165 for greedy rows).  Called by one thread. */
__device__ __forceinline__ void pss_epilogue(const pss_args& a, uint32_t row, uint32_t tok, bool greedy,
                                             uint32_t W, uint32_t new_rng, const pss_row_info& inf) {
    pss_epilogue_pre(a, row, tok, greedy, W, new_rng, inf, a.position[row], a.step[row]);
}

/* Uniform of the draw from the row's rng state s and Philox step, and the
 * rng state after it. */
__device__ __forceinline__ uint32_t pss_draw_u24_pre(uint32_t rng_mode, uint32_t s, uint32_t step,
                                                     uint32_t row, uint32_t* new_rng) {
    if (rng_mode == PSS_RNG_PHILOX) {
        pss_u32x4 c;
        c.v[0] = step;
        c.v[1] = row;
        c.v[2] = 0u;
        c.v[3] = 0u;
        *new_rng = s;
        return pss_philox4x32_10(c, s, 0u).v[0] >> 8;
    }
    if (s == 0u) s = PSS_XORSHIFT_ZERO_SEED;
    *new_rng = pss_xorshift32(s);
    return s >> 8;
}

/* Uniform of the draw and the rng state after it. */
__device__ __forceinline__ uint32_t pss_draw_u24(const pss_args& a, uint32_t row, uint32_t* new_rng) {
    uint32_t s = a.rng[row];
    if (a.rng_mode == PSS_RNG_PHILOX) {
        pss_u32x4 c;
        c.v[0] = a.step[row];
        c.v[1] = row;
        c.v[2] = 0u;
        c.v[3] = 0u;
        *new_rng = s;
        return pss_philox4x32_10(c, s, 0u).v[0] >> 8;
    }
    if (s == 0u) s = PSS_XORSHIFT_ZERO_SEED;
    *new_rng = pss_xorshift32(s);
    return s >> 8;
}

/* Greedy outputs of one row (mask / probs / epilogue), `best` = packed
 * (key << 32) | (0xFFFFFFFF - id) of the argmax. */
template <int NT>
__device__ __forceinline__ void pss_greedy_finish(const pss_args& a, uint32_t row, uint64_t best) {
    const uint32_t tid = threadIdx.x;
    const uint32_t tok = 0xFFFFFFFFu - (uint32_t)best;
    if (a.kept_mask)
        for (uint32_t w = tid; w < a.mask_words; w += NT)
            a.kept_mask[(size_t)row * a.mask_words + w] = (w == (tok >> 5)) ? (1u << (tok & 31u)) : 0u;
    if (a.probs)
        for (uint32_t j = tid; j < a.V; j += NT)
            a.probs[(size_t)row * a.probs_stride + j] = j == tok ? 1.0f : 0.0f;
    if (tid == 0) {
        pss_row_info inf = {};
        inf.token = tok;
        inf.kept_count = 1;
        inf.tau_key = (uint32_t)(best >> 32);
        inf.tmax_key = inf.tau_key;
        inf.flags = PSS_INFO_GREEDY;
        pss_epilogue(a, row, tok, true, 0u, 0u, inf);
    }
}

/* LDS scratch of the general algorithm (besides the penalty bitmap). */
struct pss_gen_shared {
    uint64_t hist[256];
    uint64_t red[PSS_GEN_NT / PSS_WAVE];
    uint64_t rem;
    uint32_t digit;
    uint32_t tok;
};

/* First digit shift of a select over keys in [lo, hi]: below their common
 * prefix; -1 when lo == hi. */
__device__ __forceinline__ int pss_gen_select_shift(uint32_t lo, uint32_t hi) {
    const uint32_t d = lo ^ hi;
    return d ? ((31 - (int)__clz(d)) / 8) * 8 : -1;
}

/* hist[d] += w for every lane with w != 0 (all 64 lanes active): the lanes
 * sharing the first pending lane's digit combine into one atomic (their count
 * when `unit`, else a wave sum), up to four digits while each covers at least
 * 8 lanes; the rest add one by one.  With heavy ties a wave's lanes share one
 * or two digits; with spread keys the plain atomics are cheaper. */
__device__ __forceinline__ void pss_hist_add_wave(uint64_t* hist, uint32_t d, uint64_t w, bool unit) {
    const uint32_t lane = pss_tid() & 63u;
    uint64_t pending = __ballot(w != 0ull);
    for (int it = 0; it < 4 && pending; ++it) {
        const uint32_t leader = (uint32_t)__builtin_ctzll(pending);
        const uint32_t dl = __builtin_amdgcn_readlane(d, leader);
        const bool in = ((pending >> lane) & 1ull) && d == dl;
        const uint64_t m = __ballot(in);
        if (__popcll(m) < 8) break;
        const uint64_t tot = unit ? (uint64_t)__popcll(m) : wave_sum_u64(in ? w : 0ull);
        if (lane == leader) atomicAdd((unsigned long long*)&hist[dl], (unsigned long long)tot);
        pending &= ~m;
    }
    if ((pending >> lane) & 1ull) atomicAdd((unsigned long long*)&hist[d], (unsigned long long)w);
}

template <int NT>
__device__ __forceinline__ void pss_general_row(const pss_args& a, uint32_t row, pss_gen_shared& sh, uint32_t* bits,
                                uint32_t bit_words) {
    const uint32_t tid = threadIdx.x;
    const uint32_t V = a.V;
    const sample_params sp = a.params[row];
    const size_t esz = a.dtype == PSS_DTYPE_F16 ? 2u : 4u;
    const void* rowp = (const char*)a.logits + (size_t)row * a.stride * esz;
    const bool greedy = (a.mode == PSS_MODE_GREEDY) || !(sp.temperature > 0.0f);

    if (greedy) {
        uint64_t best = 0;
        for (uint32_t j = tid; j < V; j += NT) {
            uint64_t c = ((uint64_t)pss_key(pss_canon(pss_load1(rowp, a.dtype, j))) << 32) |
                         (uint64_t)(0xFFFFFFFFu - j);
            best = c > best ? c : best;
        }
        best = block_max_u64<NT>(best, sh.red);
        pss_greedy_finish<NT>(a, row, best);
        return;
    }

    const pss_rowcfg c = pss_make_rowcfg(sp, V);
    const uint32_t* hist_row = a.history + (size_t)row * PSS_MAX_PENALTY_LEN;
    const uint32_t CH = bit_words * 32u;
    const bool chunked = c.doPen && V > CH;

    /* Penalty bitmap of ids [c0, c0 + CH). */
    auto build = [&](uint32_t c0) {
        for (uint32_t i = tid; i < bit_words; i += NT) bits[i] = 0u;
        __syncthreads();
        for (uint32_t h = tid; h < c.W; h += NT) {
            const uint32_t id = hist_row[h];
            if (id < V && id >= c0 && id - c0 < CH) atomicOr(&bits[(id - c0) >> 5], 1u << ((id - c0) & 31u));
        }
        __syncthreads();
    };
    if (c.doPen && !chunked) build(0u);
    auto T = [&](uint32_t j, uint32_t c0) -> float {
        return pss_transform(pss_load1(rowp, a.dtype, j), c.doPen && pss_bit(bits, j - c0), c);
    };
    /* Unchunked passes take PSS_GEN_U ids per thread per step, their loads
     * requested together (one memory round trip per step instead of per id);
     * ids past V come as -inf with valid = false. */
    constexpr int U = PSS_GEN_U;
    auto each_step = [&](auto&& g) {
        for (uint32_t j0 = 0; j0 < V; j0 += NT * (uint32_t)U) {
            float x[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t j = j0 + (uint32_t)u * NT + tid;
                x[u] = j < V ? pss_load1(rowp, a.dtype, j) : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t j = j0 + (uint32_t)u * NT + tid;
                const bool valid = j < V;
                g(j, valid ? pss_transform(x[u], c.doPen && pss_bit(bits, j), c) : pss_u2f(0xFF800000u), valid);
            }
        }
    };
    /* One pass over the row: f(j, t) for every id, ids strided over threads.
     * Every thread of the workgroup calls it. */
    auto pass = [&](auto&& f) {
        if (!chunked) {
            each_step([&](uint32_t j, float t, bool valid) {
                if (valid) f(j, t);
            });
            return;
        }
        for (uint32_t c0 = 0; c0 < V; c0 += CH) {
            build(c0);
            const uint32_t c1 = V - c0 < CH ? V : c0 + CH;
            for (uint32_t j = c0 + tid; j < c1; j += NT) f(j, T(j, c0));
            __syncthreads();
        }
    };

    /* S3, and the smallest key: the radix selects start below the common
     * prefix of the range they search (none at all on an all-equal row) */
    uint64_t mk = 0, nk = 0;
    constexpr uint32_t NWV = NT / PSS_WAVE;
    const uint32_t lane = tid & 63u, wv = tid >> 6;
    const uint32_t nblk = (V + 1023u) / 1024u;
    static_assert(PSS_MAX_VOCAB <= 256u * 1024u, "per-block values fit the histogram");
    static_assert(NT >= PSS_WAVE && 1024 % NT == 0, "whole waves; a block is whole workgroup passes");
    if (!chunked) {
        /* the row in 1,024-id blocks, block b taken by wave b % NW (lane l on
         * ids 1024 b + 64 i + l: coalesced); each block's largest key and
         * how many ids hold it go to sh.hist[b] (key << 32 | count) */
        /* 16-byte aligned rows: the block as 16-byte loads, all in flight
         * at once (4 per lane fp32, 2 fp16; lane l on 4 (8) consecutive ids) */
        const bool vec = a.vec_ok && (V * (uint32_t)esz) % 16u == 0u;
        /* specialized on the element width and on whether the row has a
         * window (V is a multiple of the ids per 16-byte load, so a load is
         * all in the row or all past it) */
        auto blocks = [&](auto PER, auto PEN) {
            constexpr uint32_t per = decltype(PER)::value; /* ids per 16-byte load: 4 fp32, 8 fp16 */
            constexpr bool pen = decltype(PEN)::value;
            constexpr int nq = (int)(1024u / (64u * per)); /* loads per lane: 4 or 2 */
            uint32_t kmin = 0xFFFFFFFFu;
            for (uint32_t b = wv; b < nblk; b += NWV) {
                uint4 r[nq];
#pragma unroll
                for (int q = 0; q < nq; ++q) {
                    const uint32_t j = b * 1024u + (uint32_t)q * 64u * per + lane * per;
                    r[q] = j < V ? *(const uint4*)((const char*)rowp + (size_t)j * esz) : make_uint4(0u, 0u, 0u, 0u);
                }
                uint32_t km = 0u, cm = 0u;
#pragma unroll
                for (int q = 0; q < nq; ++q) {
                    const uint32_t j0 = b * 1024u + (uint32_t)q * 64u * per + lane * per;
                    if (j0 >= V) continue;
                    const uint32_t w[4] = {r[q].x, r[q].y, r[q].z, r[q].w};
#pragma unroll
                    for (uint32_t e = 0; e < per; ++e) {
                        float x;
                        if (per == 8u) {
                            const uint16_t h = (uint16_t)(w[e >> 1] >> ((e & 1u) * 16u));
                            _Float16 hf;
                            __builtin_memcpy(&hf, &h, 2);
                            x = (float)hf;
                        } else {
                            x = __uint_as_float(w[e & 3u]);
                        }
                        const uint32_t k = pss_key(pss_transform(x, pen && pss_bit(bits, j0 + e), c));
                        cm = k > km ? 1u : cm + (k == km ? 1u : 0u);
                        km = k > km ? k : km;
                        kmin = k < kmin ? k : kmin;
                    }
                }
                mk = km > mk ? km : mk;
                const uint32_t M = wave_max_u32(km);
                const uint32_t cnt = wave_sum_u32(km == M ? cm : 0u);
                if (lane == 0u) sh.hist[b] = ((uint64_t)M << 32) | cnt;
            }
            nk = (0xFFFFFFFFull ^ kmin) > nk ? (0xFFFFFFFFull ^ kmin) : nk;
        };
        if (vec) {
            using f16w = std::integral_constant<uint32_t, 8u>;
            using f32w = std::integral_constant<uint32_t, 4u>;
            using penw = std::integral_constant<bool, true>;
            using nopw = std::integral_constant<bool, false>;
            if (a.dtype == PSS_DTYPE_F16)
                c.doPen ? blocks(f16w{}, penw{}) : blocks(f16w{}, nopw{});
            else
                c.doPen ? blocks(f32w{}, penw{}) : blocks(f32w{}, nopw{});
        }
        for (uint32_t b = wv; b < nblk && !vec; b += NWV) {
            uint32_t km = 0u, cm = 0u;
            for (uint32_t i0 = 0; i0 < 16u; i0 += (uint32_t)U) {
                float x[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const uint32_t j = b * 1024u + (i0 + (uint32_t)u) * 64u + lane;
                    x[u] = j < V ? pss_load1(rowp, a.dtype, j) : 0.0f;
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const uint32_t j = b * 1024u + (i0 + (uint32_t)u) * 64u + lane;
                    if (j < V) {
                        const uint32_t k = pss_key(pss_transform(x[u], c.doPen && pss_bit(bits, j), c));
                        cm = k > km ? 1u : cm + (k == km ? 1u : 0u);
                        km = k > km ? k : km;
                        nk = (0xFFFFFFFFull ^ k) > nk ? (0xFFFFFFFFull ^ k) : nk;
                    }
                }
            }
            mk = km > mk ? km : mk;
            const uint32_t M = wave_max_u32(km);
            const uint32_t cnt = wave_sum_u32(km == M ? cm : 0u);
            if (lane == 0u) sh.hist[b] = ((uint64_t)M << 32) | cnt;
        }
    } else {
        pass([&](uint32_t, float t) {
            const uint64_t k = pss_key(t);
            mk = k > mk ? k : mk;
            nk = (0xFFFFFFFFull ^ k) > nk ? (0xFFFFFFFFull ^ k) : nk;
        });
    }
    const uint32_t tmaxKey = (uint32_t)block_max_u64<NT>(mk, sh.red);
    const uint32_t tminKey = (uint32_t)(0xFFFFFFFFull ^ block_max_u64<NT>(nk, sh.red));
    const float tmax = pss_unkey(tmaxKey);
    /* ids holding the row maximum, when at least K of them: then the top-k
     * set is exactly those ids (the K-th largest is the maximum), top-p
     * cannot cut below it, every one has p = 1 (>= minP), so they are the
     * kept set and the draw picks the floor(target / q(1))-th of them in id
     * order; no select and no mass pass */
    uint64_t cntM = 0;
    if (!chunked) {
        uint64_t cl = 0;
        for (uint32_t b = tid; b < nblk; b += NT)
            cl += (uint32_t)(sh.hist[b] >> 32) == tmaxKey ? (uint32_t)sh.hist[b] : 0u;
        cntM = block_sum_u64<NT>(cl, sh.red);
    }
    const bool topTie = !chunked && c.K >= 1u && cntM >= (uint64_t)c.K && (!c.useMinP || 1.0f >= c.minP);
    /* p = exp(t - tmax) depends on the key alone: each thread keeps its last
     * two keys' values (heavy ties then skip the exp; 0xFFFFFFFF is no key
     * of a canonical value) */
    uint32_t pk0 = 0xFFFFFFFFu, pk1 = 0xFFFFFFFFu;
    float pv0 = 0.0f, pv1 = 0.0f;
    auto prob_of = [&](float t, uint32_t k) -> float {
        if (k == pk0) return pv0;
        if (k == pk1) return pv1;
        const float p = pss_prob(t, tmax);
        pk1 = pk0;
        pv1 = pv0;
        pk0 = k;
        pv0 = p;
        return p;
    };

    /* Radix select over the row: digit levels of 8 bits from the top.  weight
     * 0 = count (top-k), 1 = mass restricted to key >= lo (top-p).  Without
     * chunking every lane runs every iteration (ids past V weigh nothing), so
     * the wave can combine its lanes' additions per digit (pss_hist_add_wave:
     * tied values put a whole wave on one bin, where separate LDS atomics to
     * one address serialize). */
    auto select = [&](uint64_t rem, int weight, uint32_t lo) -> uint32_t {
        /* every weighted key lies in [max(lo, tminKey), tmaxKey] */
        const int top = pss_gen_select_shift(lo > tminKey ? lo : tminKey, tmaxKey);
        if (top < 0) return tmaxKey;
        uint32_t pmask = top + 8 >= 32 ? 0u : ~((1u << (top + 8)) - 1u);
        uint32_t prefix = tmaxKey & pmask;
        for (int shift = top; shift >= 0; shift -= 8) {
            for (uint32_t i = tid; i < 256u; i += NT) sh.hist[i] = 0;
            __syncthreads();
            auto wof = [&](float t, uint32_t k) -> uint64_t {
                if ((k & pmask) != prefix) return 0ull;
                if (weight == 0) return 1ull;
                return k >= lo ? pss_fixq(prob_of(t, k)) : 0ull;
            };
            if (!chunked) {
                each_step([&](uint32_t, float t, bool valid) {
                    const uint32_t k = pss_key(t);
                    const uint64_t w = valid ? wof(t, k) : 0ull;
                    pss_hist_add_wave(sh.hist, (k >> shift) & 255u, w, weight == 0);
                });
            } else {
                pass([&](uint32_t, float t) {
                    const uint32_t k = pss_key(t);
                    const uint64_t w = wof(t, k);
                    if (w) atomicAdd((unsigned long long*)&sh.hist[(k >> shift) & 255u], (unsigned long long)w);
                });
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
    };

    /* q of p = 1 (the value of every id at the row maximum) */
    const uint64_t q1 = pss_fixq(pss_prob(tmax, tmax));
    /* S5 */
    uint32_t tauK = tmaxKey, tau = tmaxKey;
    uint64_t zk = cntM * q1;
    if (!topTie) {
        tauK = c.K > 0u ? select(c.K, 0, 0u) : 0u;
        uint64_t zl = 0;
        pass([&](uint32_t, float t) {
            const uint32_t k = pss_key(t);
            if (k >= tauK) zl += pss_fixq(prob_of(t, k));
        });
        zk = block_sum_u64<NT>(zl, sh.red);
        /* S6 */
        tau = tauK;
        if (c.useTopP) {
            const uint32_t tauP = select(pss_topp_need(c.topP, zk), 1, tauK);
            tau = tauP > tau ? tauP : tau;
        }
    }

    /* S7 */
    auto kept_q = [&](float t, uint64_t* q, float* pout) -> bool {
        const uint32_t key = pss_key(t);
        const float p = key >= tau ? prob_of(t, key) : 0.0f;
        const bool k = key >= tau && (!c.useMinP || p >= c.minP);
        *q = k ? pss_fixq(p) : 0;
        *pout = p;
        return k;
    };
    uint32_t newRng;
    const uint32_t u24 = pss_draw_u24(a, row, &newRng);
    uint64_t Z, target;
    uint32_t keptCount, lastAll;
    const uint32_t CW = chunked ? CH : V;
    if (topTie) {
        Z = zk;
        keptCount = (uint32_t)cntM;
        lastAll = 0u;
        target = pss_draw_target(u24, Z);
        const uint64_t nth = target / q1; /* the kept id the draw lands on, counted from 0 */
        /* wave 0: the block holding it (per-block counts of the maximum) */
        if (tid < PSS_WAVE) {
            uint64_t c4[4], s4 = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t b = 4u * lane + (uint32_t)k;
                c4[k] = b < nblk && (uint32_t)(sh.hist[b] >> 32) == tmaxKey ? (uint32_t)sh.hist[b] : 0u;
                s4 += c4[k];
            }
            uint64_t base = wave_incl_scan_u64(s4) - s4;
            if (lane == 0u) {
                sh.tok = PSS_NO_TOKEN;
                sh.digit = PSS_NO_TOKEN;
            }
            if (s4 > 0 && base <= nth && nth < base + s4) {
                uint32_t blk = PSS_NO_TOKEN;
                uint64_t bbase = 0;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (blk == PSS_NO_TOKEN && c4[k] > 0 && nth < base + c4[k]) {
                        blk = 4u * lane + (uint32_t)k;
                        bbase = base;
                    }
                    base += c4[k];
                }
                sh.digit = blk;
                sh.rem = nth - bbase;
            }
        }
        __syncthreads();
        const uint32_t blk = sh.digit;
        if (blk != PSS_NO_TOKEN) {
            /* the block's ids in order: the (rem)-th holding the maximum */
            uint64_t seen = 0;
            const uint64_t want = sh.rem;
            for (uint32_t sub = 0; sub < 1024u; sub += NT) {
                const uint32_t j = blk * 1024u + sub + tid;
                const uint64_t f = j < V && pss_key(T(j, 0u)) == tmaxKey ? 1u : 0u;
                uint64_t tot;
                const uint64_t P = block_excl_scan_u64<NT>(f, sh.red, &tot);
                if (f && seen + P == want) sh.tok = j;
                seen += tot;
                __syncthreads();
            }
        }
        __syncthreads();
    } else if (!chunked) {
        /* S7 and S8 together.  The row in 1,024-id blocks, block b taken by
         * wave b % NW (lane l on ids 1024 b + 64 i + l: coalesced), each
         * block's kept mass recorded in sh.hist (V <= 256 blocks); Z is their
         * sum; the block holding the draw target comes from a scan over the
         * block masses, then the block's ids are scanned in order. */
        uint64_t zs = 0;
        uint32_t cnt = 0, lastKept = 0;
        for (uint32_t b = wv; b < nblk; b += NWV) {
            uint64_t bs = 0;
            for (uint32_t i0 = 0; i0 < 16u; i0 += (uint32_t)U) {
                float x[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const uint32_t j = b * 1024u + (i0 + (uint32_t)u) * 64u + lane;
                    x[u] = j < V ? pss_load1(rowp, a.dtype, j) : 0.0f;
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const uint32_t j = b * 1024u + (i0 + (uint32_t)u) * 64u + lane;
                    uint64_t q;
                    float p;
                    if (j < V && kept_q(pss_transform(x[u], c.doPen && pss_bit(bits, j), c), &q, &p)) {
                        bs += q;
                        cnt++;
                        lastKept = j + 1u;
                    }
                }
            }
            zs += bs;
            bs = wave_sum_u64(bs);
            if (lane == 0u) sh.hist[b] = bs;
        }
        Z = block_sum_u64<NT>(zs, sh.red);
        keptCount = (uint32_t)block_sum_u64<NT>(cnt, sh.red);
        lastAll = (uint32_t)block_max_u64<NT>(lastKept, sh.red);
        target = pss_draw_target(u24, Z);
        /* wave 0: lane l sums blocks 4l..4l+3; the lane whose range holds the
         * target finds the block */
        if (tid < PSS_WAVE) {
            uint64_t m4[4], s4 = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t b = 4u * lane + (uint32_t)k;
                m4[k] = b < nblk ? sh.hist[b] : 0ull;
                s4 += m4[k];
            }
            uint64_t base = wave_incl_scan_u64(s4) - s4;
            uint32_t blk = PSS_NO_TOKEN;
            uint64_t bbase = 0;
            if (s4 > 0 && base <= target && target < base + s4) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if (blk == PSS_NO_TOKEN && m4[k] > 0 && target < base + m4[k]) {
                        blk = 4u * lane + (uint32_t)k;
                        bbase = base;
                    }
                    base += m4[k];
                }
            }
            const uint64_t hit = __ballot(blk != PSS_NO_TOKEN);
            if (lane == 0u) {
                sh.tok = PSS_NO_TOKEN;
                sh.digit = hit ? 0u : PSS_NO_TOKEN;
            }
            if (blk != PSS_NO_TOKEN) {
                sh.digit = blk;
                sh.rem = bbase;
            }
        }
        __syncthreads();
        const uint32_t blk = sh.digit;
        const uint64_t bbase = sh.rem;
        if (blk != PSS_NO_TOKEN) {
            /* the block's ids in order, NT at a time, one per thread */
            uint64_t base = bbase;
            for (uint32_t sub = 0; sub < 1024u; sub += NT) {
                const uint32_t j = blk * 1024u + sub + tid;
                uint64_t q = 0;
                float p;
                if (j < V && !kept_q(T(j, 0u), &q, &p)) q = 0;
                uint64_t tot;
                const uint64_t P = block_excl_scan_u64<NT>(q, sh.red, &tot);
                if (q > 0 && base + P <= target && target < base + P + q) sh.tok = j;
                base += tot;
                __syncthreads();
            }
        }
        __syncthreads();
    } else {
        uint64_t zs = 0;
        uint32_t cnt = 0, lastKept = 0;
        pass([&](uint32_t j, float t) {
            uint64_t q;
            float p;
            if (kept_q(t, &q, &p)) {
                zs += q;
                cnt++;
                lastKept = j + 1u;
            }
        });
        Z = block_sum_u64<NT>(zs, sh.red);
        keptCount = (uint32_t)block_sum_u64<NT>(cnt, sh.red);
        lastAll = (uint32_t)block_max_u64<NT>(lastKept, sh.red);

        /* S8: walk the row in id order, chunk by chunk; within a chunk each
         * thread owns a contiguous id range and a block scan orders the
         * ranges. */
        target = pss_draw_target(u24, Z);
        if (tid == 0) sh.tok = PSS_NO_TOKEN;
        __syncthreads();
        uint64_t base = 0;
        for (uint32_t c0 = 0; c0 < V; c0 += CW) {
            const uint32_t c0b = c0;
            build(c0);
            const uint32_t c1 = V - c0 < CW ? V : c0 + CW;
            const uint32_t per = (c1 - c0 + NT - 1u) / NT;
            const uint32_t j0 = c0 + tid * per < c1 ? c0 + tid * per : c1;
            const uint32_t j1 = j0 + per < c1 ? j0 + per : c1;
            uint64_t S = 0;
            for (uint32_t j = j0; j < j1; ++j) {
                uint64_t q;
                float p;
                if (kept_q(T(j, c0b), &q, &p)) S += q;
            }
            uint64_t tot;
            const uint64_t P = block_excl_scan_u64<NT>(S, sh.red, &tot);
            if (S > 0 && base + P <= target && target < base + P + S) {
                uint64_t acc = base + P;
                for (uint32_t j = j0; j < j1; ++j) {
                    uint64_t q;
                    float p;
                    if (kept_q(T(j, c0b), &q, &p)) {
                        acc += q;
                        if (acc > target) {
                            sh.tok = j;
                            break;
                        }
                    }
                }
            }
            __syncthreads();
            base += tot;
            if (sh.tok != PSS_NO_TOKEN || base > target) break;
        }
    }
    uint32_t tok = sh.tok;
    uint32_t flags = 0;
    if (tok == PSS_NO_TOKEN) {
        tok = lastAll > 0u ? lastAll - 1u : 0u;
        flags |= PSS_INFO_FALLBACK;
    }

    /* verification outputs */
    if (a.kept_mask) {
        uint32_t* m = a.kept_mask + (size_t)row * a.mask_words;
        for (uint32_t c0 = 0; c0 < V; c0 += CW) {
            const uint32_t c0b = chunked ? c0 : 0u;
            if (chunked) build(c0);
            const uint32_t c1 = V - c0 < CW ? V : c0 + CW;
            for (uint32_t w = c0 / 32u + tid; w < (c1 + 31u) / 32u; w += NT) {
                uint32_t bw = 0;
                for (uint32_t b = 0; b < 32u; ++b) {
                    const uint32_t j = w * 32u + b;
                    uint64_t q;
                    float p;
                    if (j < c1 && kept_q(T(j, c0b), &q, &p)) bw |= 1u << b;
                }
                m[w] = bw;
            }
            if (chunked) __syncthreads();
        }
    }
    if (a.probs) {
        const float zf = (float)Z * 0x1.0p-45f;
        float* pr = a.probs + (size_t)row * a.probs_stride;
        pass([&](uint32_t j, float t) {
            uint64_t q;
            float p;
            pr[j] = kept_q(t, &q, &p) ? p / zf : 0.0f;
        });
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

/* One 1024-thread workgroup per row, penalty bitmap over the whole vocab. */
__global__ void __launch_bounds__(PSS_GEN_NT) pss_general_kernel(pss_args a) {
    __shared__ pss_gen_shared sh;
    __shared__ uint32_t bits[PSS_MAX_VOCAB / 32];
    pss_globalize(a);
    if (pss_gate_closed(a)) return;
    pss_general_row<PSS_GEN_NT>(a, blockIdx.x, sh, bits, PSS_MAX_VOCAB / 32);
}

#endif /* PSS_GENERAL_H */
