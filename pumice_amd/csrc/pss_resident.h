/*
 * pss_resident.h - the register-resident row kernel (the batched roofline
 * path: one workgroup per row, V * element size <= 16 KiB * NL).
 *
 * Each lane reads its share of the row with NL 16-byte buffer loads
 * (nontemporal) into registers, 1,024 lanes covering the row: wave w holds
 * ids [w * NL * 64 * E, (w + 1) * NL * 64 * E), load j of lane l is ids
 * (w * NL + j) * 64 * E + l * E + [0, E) (E = 4 fp32 / 8 fp16 values per 16
 * bytes), so each load instruction of a wave reads 1 KiB contiguous.  A wave
 * keeps PSS_RES_DEPTH loads in flight, the next one requested before each
 * wait (loads complete in issue order); no data passes through LDS.
 *
 * The first JC + 1 loads (seven eighths of an fp32 row, three quarters of
 * an fp16 row) stay in registers, processed on arrival: t = l * (1/T), the window ids excluded (their
 * penalized values enter the candidate list separately, once per distinct
 * id), each lane's running maximum.  Then every wave publishes the 8 (or 16)
 * largest of its lanes' maxima; after one barrier the K-th largest of all published values is a
 * certified lower bound G of the row's K-th largest value (K distinct
 * elements at or above it; ties are kept, so the bound is on values, not
 * positions).  From that much of the row G is close to the exact K-th
 * largest: the elements at or above it, from the registers at once and from
 * the rest of the row as it arrives, go straight into the finisher's list
 * (about K + K/3 of them), and the row finishes after one more barrier in
 * one wave (pss_list_finish_fast of pss_stream.h): the exact K-th largest,
 * masses, top-p, min-p, the ascending-id draw and the epilogue.  The later
 * loads pass through a ring of registers in a runtime loop, so the hot code
 * stays small enough for the instruction cache.
 *
 * Greedy rows keep each lane's (key, smallest id) best instead.  Rows outside
 * the candidate path (top-k off or above PSS_SEG_KMAX, a window above
 * PSS_RES_WMAX ids, a list that overflows, no finite bound) run the general
 * algorithm in the same workgroup.
 *
 * Roofline: HBM, one read of each row (V * e + 4 W + 44 bytes per row).
 */
#ifndef PSS_RESIDENT_H
#define PSS_RESIDENT_H

#include "pss_wide.h"

#define PSS_RES_NW 16
#define PSS_RES_NT (PSS_RES_NW * PSS_WAVE)
#define PSS_RES_WMAX 256u /* window ids the kernel dedups (4 waves x 64) */
#ifndef PSS_RES_DEPTH
#define PSS_RES_DEPTH 4
#endif

template <int NL, int DT>
struct pss_res_geom {
    static constexpr int E = DT == PSS_DTYPE_F16 ? 8 : 4;
    static constexpr uint32_t LSPAN = (uint32_t)PSS_WAVE * E; /* ids per load instruction of a wave */
    static constexpr uint32_t WSPAN = (uint32_t)NL * LSPAN;   /* ids per wave */
    static constexpr uint32_t VMAX = PSS_RES_NW * WSPAN;
    static constexpr uint32_t BW = (VMAX + 31u) / 32u;        /* window bitmap words */
    /* loads 0..JC before the bound: seven eighths of an fp32 row (23.9 ->
     * 23.4 us at 256 x 102,400 against three quarters; no spills), three
     * quarters of an fp16 row (seven eighths: 27.2 -> 27.7 us at 256 x
     * 102,400 with top-k up to 100) */
    static constexpr int JC = DT == PSS_DTYPE_F16 ? (3 * NL) / 4 : (7 * NL) / 8;
    /* loads a wave keeps in flight: a CU can have about 50 outstanding, so
     * more would stall the wave at its next request, ahead of the work on
     * the data that has arrived */
    static constexpr int D = PSS_RES_DEPTH;
    static_assert(NL >= 4 && NL <= 32, "load count per lane");
};

template <int NL, int DT>
struct pss_res_shared {
    pss_fin_small f;                                   /* finisher; f.cl is the candidate list */
    uint32_t winbits[pss_res_geom<NL, DT>::BW];        /* window membership (the general fallback's bitmap) */
    uint32_t wid[PSS_RES_NW][2u * PSS_WAVE];           /* per wave: the distinct window ids in its range */
    uint32_t pub[PSS_RES_NW * 16u];                    /* per wave: its lanes' largest maxima, sorted */
    unsigned long long best[PSS_RES_NW];               /* greedy rows: each wave's (key << 32) | ~id */
    uint32_t wl[PSS_RES_NW];                           /* bit j: load j of the wave holds window ids */
    uint32_t ncl;                                      /* candidates claimed (may exceed PSS_FAST_N) */
    uint32_t G;                                        /* the bound */
    uint32_t over;                                     /* a wave's range holds more window ids than it keeps */
};

template <int NL, int DT>
__global__ void __launch_bounds__(PSS_RES_NT) pss_res_kernel(pss_args a, const sample_params* __restrict__ params) {
    using Gm = pss_res_geom<NL, DT>;
    constexpr int E = Gm::E;
    constexpr int RS = Gm::D + 1; /* ring slots of the loads after JC */
    constexpr uint32_t esz = DT == PSS_DTYPE_F16 ? 2u : 4u;
    __shared__ pss_res_shared<NL, DT> S;
    pss_fin_small& f = S.f;
    const uint32_t row = blockIdx.x, tid = threadIdx.x;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63u;

    /* 1. requests in the order they are needed.  The kernel arguments arrive
     * in one round trip; the row's parameters and state (not waited for
     * here; the state is written only by this workgroup's epilogue, after
     * these loads) and the window ids (waves 0..3, the first 256 slots of
     * the ring; trimmed to the row's window below) are requested ahead of
     * the row's first D loads: loads complete in issue order, so nothing the
     * stream needs waits behind the row's traffic. */
    __asm__ __volatile__("" ::"s"(a.logits), "s"(a.stride), "s"(a.V), "s"(params), "s"(a.rng), "s"(a.step),
                         "s"(a.position), "s"(a.history), "s"(a.gate));
    __asm__ __volatile__("" ::"s"(a.mode), "s"(a.do_inc), "s"(a.pass_idx), "s"(a.rng_mode), "s"(a.result),
                         "s"(a.token_ids), "s"(a.info), "s"(a.kept_mask), "s"(a.mask_words), "s"(a.probs),
                         "s"(a.probs_stride), "s"(a.host_tokens), "s"(a.gate_seq), "s"(a.eos));
    pss_globalize(a);
    if (pss_gate_closed(a)) return;
    sample_params sp = params[row];
    pss_row_pre pre;
    pre.rng = ((const __attribute__((address_space(4))) uint32_t*)a.rng)[row];
    pre.step = ((const __attribute__((address_space(4))) uint32_t*)a.step)[row];
    pre.pos = ((const __attribute__((address_space(4))) uint32_t*)a.position)[row];
    uint32_t hid[PSS_RES_WMAX / PSS_WAVE];
#pragma unroll
    for (int h = 0; h < (int)(PSS_RES_WMAX / PSS_WAVE); ++h)
        hid[h] = a.history[(size_t)row * PSS_MAX_PENALTY_LEN + (uint32_t)h * 64u + lane];
    __asm__ __volatile__("" ::: "memory");
    uint4 raw[Gm::JC + 1];
    uint4 ring[RS];
    const __amdgpu_buffer_rsrc_t rrs = pss_row_rsrc(a, row, esz);
    const uint32_t vb = (wave * (uint32_t)NL * 64u + lane) * 16u;
    auto ld = [&](uint32_t j) -> uint4 {
        return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rrs, (int)(vb + 1024u * j), 0, PSS_NT));
    };
    auto issue1 = [&](int j) { /* j known at compile time */
        if (j <= Gm::JC)
            raw[j <= Gm::JC ? j : 0] = ld((uint32_t)j);
        else
            ring[(j - Gm::JC - 1) % RS] = ld((uint32_t)j);
    };
#pragma unroll
    for (int j = 0; j < Gm::D && j < NL; ++j) issue1(j);
    /* the parameters and state are used only from here on, so that no wait
     * for them precedes the row's first loads */
    pss_pin_s(sp.temperature);
    pss_pin_s(sp.repPenalty);
    pss_pin_s(sp.penaltyLength);
    pss_pin_s(sp.topK);
    pss_pin_s(sp.topP);
    pss_pin_s(sp.minP);
    pss_pin_s(sp.presencePenalty);
    pss_pin_s(pre.rng);
    pss_pin_s(pre.step);
    pss_pin_s(pre.pos);
    const uint32_t V = a.V;
    const float NEG_INF = pss_u2f(0xFF800000u);

    /* shared counters, first used after the bound's barrier */
    if (tid < 256u) f.hist[0][tid] = f.hist[1][tid] = 0u;
    if (tid == 0u) {
        S.ncl = 0u;
        S.over = 0u;
        f.nk = 0u;
        f.hflag = 0u;
    }
    pss_rowcfg c = pss_make_rowcfg(sp, V);
    /* the row constants are uniform: scalar registers, not vector ones */
    c.invT = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(c.invT)));
    c.pres = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(c.pres)));
    const bool greedy = pss_seg_row_greedy(a, sp);
    const bool cov = !greedy && c.K >= 1u && c.K <= PSS_SEG_KMAX && c.W <= PSS_RES_WMAX;
    const bool doPen = cov && c.doPen;
    const float invT = c.invT;

    /* 2. window, wave by wave: each wave takes the window ids in its own id
     * range (its own words of the bitmap; no other wave reads or writes
     * them, so no barrier), each distinct id once (the lane that sets its
     * bit owns it), marks its loads holding window ids and gathers the
     * dword holding each id's logit into a register (requested behind the
     * row's first loads, so it arrives with them).  At most 128 distinct
     * ids per wave; a wave with more sends the row to the general path. */
    uint32_t wlm = 0u; /* bit j: load j of this wave holds window ids */
    uint32_t nown = 0u, wraw0 = 0u, wraw1 = 0u;
    const uint32_t idw = wave * Gm::WSPAN;
    if (doPen) {
        constexpr uint32_t WW = Gm::WSPAN / 32u;
        static_assert(Gm::WSPAN % 32u == 0u, "wave ranges start on bitmap words");
        for (uint32_t i = lane; i < WW; i += PSS_WAVE) S.winbits[idw / 32u + i] = 0u;
        uint32_t lm = 0u;
#pragma unroll
        for (int h = 0; h < (int)(PSS_RES_WMAX / PSS_WAVE); ++h) {
            const uint32_t id = (uint32_t)h * 64u + lane < c.W ? hid[h] : PSS_SENTINEL;
            bool own = false;
            if (id < V && id - idw < Gm::WSPAN) {
                const uint32_t bit = 1u << (id & 31u);
                own = !(atomicOr(&S.winbits[id >> 5], bit) & bit);
            }
            const uint64_t om = __ballot(own);
            if (om) {
                const uint32_t pos =
                    nown + __builtin_amdgcn_mbcnt_hi((uint32_t)(om >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)om, 0u));
                if (own && pos < 2u * PSS_WAVE) S.wid[wave][pos] = id;
                if (own) lm |= 1u << ((id - idw) / Gm::LSPAN);
                nown += (uint32_t)__popcll(om);
            }
        }
        /* the wave's mark word: OR of the lanes' marks */
        lm |= lane_xor<1>(lm);
        lm |= lane_xor<2>(lm);
        lm |= lane_xor<4>(lm);
        lm |= lane_xor<8>(lm);
        lm |= lane_xor<16>(lm);
        lm |= lane_xor<32>(lm);
        wlm = __builtin_amdgcn_readfirstlane(lm);
        if (nown > 2u * PSS_WAVE) {
            if (lane == 0u) S.over = 1u;
            nown = 0u;
        }
    }
    {
        /* both gathers always requested (uniform wait counts in the loop) */
        const uint32_t i0 = lane < nown ? S.wid[wave][lane] : 0u;
        const uint32_t i1 = lane + PSS_WAVE < nown ? S.wid[wave][lane + PSS_WAVE] : 0u;
        wraw0 = __builtin_amdgcn_raw_buffer_load_b32(rrs, (int)((i0 * esz) & ~3u), 0, 0);
        wraw1 = __builtin_amdgcn_raw_buffer_load_b32(rrs, (int)((i1 * esz) & ~3u), 0, 0);
    }

    /* 3. the loads in arrival order */
    /* maxima each wave publishes: 16 x 8 for K <= 64, 16 x 16 up to 256 (at
     * least 2 K of them above 64, so that the K-th largest published value
     * stays close to the K-th largest lane maximum) */
    const uint32_t npub = c.K <= 64u ? 8u : 16u;
    float m = NEG_INF, m2 = NEG_INF;
    uint32_t mpos = 0u;
    uint64_t best = 0ull;
    uint32_t G = 0u;
    float Gf = NEG_INF;
    bool fb = !greedy && !cov; /* general algorithm */

    /* the elements of a load at or above G into the candidate list */
    auto extract = [&](const uint4& r, uint32_t id0) {
        uint64_t mk[E];
        uint32_t tot = 0u;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            mk[e] = __ballot(pss_res_t<DT>(r, e, invT) >= Gf);
            tot += (uint32_t)__popcll(mk[e]);
        }
        if (tot == 0u) return;
        uint32_t b0 = 0u;
        if (lane == 0u) b0 = atomicAdd(&S.ncl, tot);
        uint32_t base = __builtin_amdgcn_readfirstlane(b0);
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const uint32_t pos =
                base + __builtin_amdgcn_mbcnt_hi((uint32_t)(mk[e] >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mk[e], 0u));
            if (((mk[e] >> lane) & 1ull) && pos < PSS_FAST_N) {
                const float te = pss_res_t<DT>(r, e, invT);
                f.cl[pos] = ((unsigned long long)pss_key(pss_canon(te)) << 32) | (id0 + (uint32_t)e);
            }
            base += (uint32_t)__popcll(mk[e]);
        }
    };
    auto gmax = [&](const uint4& r) -> float {
        float g = pss_res_t<DT>(r, 0, invT);
#pragma unroll
        for (int e = 1; e < E; ++e) g = fmaxf(g, pss_res_t<DT>(r, e, invT));
        return g;
    };
    /* ids at or beyond V (the buffer returned 0 for them) become -inf */
    auto clip = [&](uint4& r, uint32_t j) {
        if (idw + (j + 1u) * Gm::LSPAN > V) {
            const uint32_t id0 = idw + j * Gm::LSPAN + lane * (uint32_t)E;
#pragma unroll
            for (int e = 0; e < E; ++e)
                if (id0 + (uint32_t)e >= V) pss_res_kill<DT>(r, e);
        }
    };
    auto greedy_upd = [&](uint4& r, uint32_t j) {
        clip(r, j);
        const uint32_t id0 = idw + j * Gm::LSPAN + lane * (uint32_t)E;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const uint64_t b = ((uint64_t)pss_key(pss_canon(pss_res_t<DT>(r, e, 1.0f))) << 32) |
                               (uint64_t)(0xFFFFFFFFu - (id0 + (uint32_t)e));
            best = b > best ? b : best;
        }
    };
    /* t = l * (1/T) in place (fp32; fp16 values are widened where used) */
    auto transform = [&](uint4& r, uint32_t j) {
        if (DT == PSS_DTYPE_F32) {
            r.x = __float_as_uint(__uint_as_float(r.x) * invT);
            r.y = __float_as_uint(__uint_as_float(r.y) * invT);
            r.z = __float_as_uint(__uint_as_float(r.z) * invT);
            r.w = __float_as_uint(__uint_as_float(r.w) * invT);
        }
        clip(r, j);
    };
    /* window ids of load j: out of the bound and the list */
    auto exclude = [&](uint4& r, uint32_t j) {
        if ((wlm >> j) & 1u) {
            const uint32_t i0 = idw + j * Gm::LSPAN + lane * (uint32_t)E;
            const uint32_t wb = S.winbits[i0 >> 5] >> (i0 & 31u);
#pragma unroll
            for (int e = 0; e < E; ++e)
                if ((wb >> e) & 1u) pss_res_kill<DT>(r, e);
        }
    };

    /* 3a. loads 0..JC on arrival (the next load requested before each
     * wait): transformed, window ids excluded, the lane's running maximum */
#pragma unroll
    for (int j = 0; j <= Gm::JC; ++j) {
        if (j + Gm::D < NL) issue1(j + Gm::D);
        if (greedy) {
            greedy_upd(raw[j], (uint32_t)j);
        } else if (!fb) {
            transform(raw[j], (uint32_t)j);
            exclude(raw[j], (uint32_t)j);
            /* the lane's largest (m, at position mpos) and second largest
             * (m2) values; NaN never enters either */
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const float x = pss_res_t<DT>(raw[j], e, invT);
                m2 = fminf(fmaxf(m2, x), m);
                mpos = x > m ? (uint32_t)(j * E + e) : mpos;
                m = fmaxf(m, x);
            }
        }
    }
    /* 3b. the bound: window marks complete, exclusions, lane maxima, each
     * wave's largest published, one barrier, the K-th largest of them all
     * (resolved to 24 bits: a lower bound of it); then the candidates of
     * loads 0..JC and the penalized window values */
    if (!greedy && !fb) {
        const uint32_t sk = ~dpp_sort_asc_u32(~pss_key(pss_canon(m))); /* descending */
        if (lane < npub) S.pub[wave * npub + lane] = sk;
        __syncthreads();
        /* one wave searches (the search is scalar work, and the CU's scalar
         * unit is shared by all its waves) */
        if (wave == 0u) {
            uint32_t g;
            if (npub == 8u) {
                const uint32_t v[2] = {S.pub[2u * lane], S.pub[2u * lane + 1u]};
                g = wave_kth_largest<2, 24>(v, c.K);
            } else {
                const uint32_t v[4] = {S.pub[4u * lane], S.pub[4u * lane + 1u], S.pub[4u * lane + 2u],
                                       S.pub[4u * lane + 3u]};
                g = wave_kth_largest<4, 24>(v, c.K);
            }
            if (lane == 0u) S.G = g;
        }
        __syncthreads();
        G = __builtin_amdgcn_readfirstlane(S.G);
        Gf = pss_unkey(G);
        if (G <= PSS_KEY_NEG_INF || S.over) {
            fb = true; /* no finite bound (every element could be kept), or too many window ids */
        } else {
            /* loads 0..JC: a lane whose second largest value is below G has
             * at most one element at or above it, its largest; only a wave
             * with a lane holding two or more scans its loads */
            if (__ballot(m2 >= Gf)) {
#pragma unroll
                for (int i = 0; i <= Gm::JC; ++i)
                    if (__ballot(gmax(raw[i]) >= Gf))
                        extract(raw[i], idw + (uint32_t)i * Gm::LSPAN + lane * (uint32_t)E);
            } else {
                const bool p = m >= Gf;
                const uint64_t bm = __ballot(p);
                if (bm) {
                    uint32_t b0 = 0u;
                    if (lane == 0u) b0 = atomicAdd(&S.ncl, (uint32_t)__popcll(bm));
                    const uint32_t pos = __builtin_amdgcn_readfirstlane(b0) +
                                         __builtin_amdgcn_mbcnt_hi((uint32_t)(bm >> 32),
                                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)bm, 0u));
                    const uint32_t id = idw + (mpos / (uint32_t)E) * Gm::LSPAN + lane * (uint32_t)E + mpos % (uint32_t)E;
                    if (p && pos < PSS_FAST_N) f.cl[pos] = ((unsigned long long)pss_key(pss_canon(m)) << 32) | id;
                }
            }
            if (nown) {
                /* the penalized window values at or above G (each id once:
                 * the wave's own ids, at most 128) */
                auto win = [&](uint32_t slot, uint32_t w) {
                    bool keep = false;
                    unsigned long long ent = 0ull;
                    if (slot < nown) {
                        const uint32_t id = S.wid[wave][slot];
                        float x;
                        if (DT == PSS_DTYPE_F16) {
                            const uint16_t h = (uint16_t)(w >> ((id & 1u) * 16u));
                            _Float16 hf;
                            __builtin_memcpy(&hf, &h, 2);
                            x = (float)hf;
                        } else {
                            x = __uint_as_float(w);
                        }
                        const uint32_t k = pss_key(pss_canon(pss_penalize(x * invT, c)));
                        keep = k >= G;
                        ent = ((unsigned long long)k << 32) | id;
                    }
                    const uint64_t bm = __ballot(keep);
                    if (bm) {
                        uint32_t b0 = 0u;
                        if (lane == 0u) b0 = atomicAdd(&S.ncl, (uint32_t)__popcll(bm));
                        const uint32_t pos = __builtin_amdgcn_readfirstlane(b0) +
                                             __builtin_amdgcn_mbcnt_hi((uint32_t)(bm >> 32),
                                                                       __builtin_amdgcn_mbcnt_lo((uint32_t)bm, 0u));
                        if (keep && pos < PSS_FAST_N) f.cl[pos] = ent;
                        m = fmaxf(m, keep ? pss_unkey((uint32_t)(ent >> 32)) : NEG_INF);
                    }
                };
                win(lane, wraw0);
                if (nown > PSS_WAVE) win(lane + PSS_WAVE, wraw1);
            }
        }
    }
    /* 3c. loads JC+1..NL-1 through the ring: load j in slot (j - JC - 1) %
     * RS, load j + D requested into the slot freed by load j - 1 */
#pragma unroll 1
    for (uint32_t base = Gm::JC + 1; base < (uint32_t)NL; base += RS) {
#pragma unroll
        for (int s = 0; s < RS; ++s) {
            const uint32_t j = base + (uint32_t)s;
            if (j + Gm::D < (uint32_t)NL) ring[(s + Gm::D) % RS] = ld(j + Gm::D);
            if (j < (uint32_t)NL) {
                uint4& r = ring[s];
                if (greedy) {
                    greedy_upd(r, j);
                } else if (!fb) {
                    transform(r, j);
                    exclude(r, j);
                    const float g = gmax(r);
                    m = fmaxf(m, g);
                    if (__ballot(g >= Gf)) extract(r, idw + j * Gm::LSPAN + lane * (uint32_t)E);
                }
            }
        }
    }

    /* 4. the row finishes from the candidate list */
    if (greedy) {
        best = wave_max_u64(best);
        if (lane == 0u) S.best[wave] = best;
        __syncthreads();
        best = S.best[0];
#pragma unroll
        for (int w = 1; w < PSS_RES_NW; ++w) best = S.best[w] > best ? S.best[w] : best;
        pss_greedy_finish<PSS_RES_NT>(a, row, best);
        return;
    }
    /* each wave's largest list value, for the finisher's radix path (the row
     * maximum is at or above G, so it is in the list) */
    const uint32_t mkey = wave_max_u32(pss_key(pss_canon(m)));
    if (lane == 0u) f.mx[wave] = mkey;
    __syncthreads();
    const uint32_t n = S.ncl;
    if (fb || n > PSS_FAST_N) {
        pss_general_row<PSS_RES_NT>(a, row, f.g, S.winbits, Gm::BW);
        return;
    }
    /* the fp32 kernel sorts at most 128 candidates in its tail and takes the
     * radix passes above: with the 256-entry sort tail inlined, its streaming
     * code compiled differently and the headline step took 1.7 us longer
     * (24.6 -> 26.4 us, measured A/B) */
    if (!pss_list_finish_fast<PSS_RES_NT, DT == PSS_DTYPE_F16 ? 256 : 128>(a, row, c, f.cl, n, G, pre, f, true))
        pss_list_finish<PSS_RES_NT>(a, row, c, f.cl, n, f.g, G);
}

/* Loads per lane for a row of V values of esz bytes; 0 if the row does not
 * fit the register-resident kernel. */
static inline int pss_res_pick_nl(uint32_t V, uint32_t esz) {
    const uint64_t loads = ((uint64_t)V * esz + 16u * PSS_RES_NT - 1u) / (16u * PSS_RES_NT);
    if (esz == 4u) return loads <= 25u ? 25 : 0;
    return loads <= 13u ? 13 : 0;
}

static inline hipError_t pss_res_launch(const pss_args& a, uint32_t rows, hipStream_t st) {
    const dim3 grid(rows), block(PSS_RES_NT);
    if (a.dtype == PSS_DTYPE_F16)
        pss_res_kernel<13, PSS_DTYPE_F16><<<grid, block, 0, st>>>(a, a.params);
    else
        pss_res_kernel<25, PSS_DTYPE_F32><<<grid, block, 0, st>>>(a, a.params);
    return hipGetLastError();
}

/* The streaming forms with the resident kernel: `form` PSS_FORM_* or -1 to
 * choose.  Automatic: launches with a top-k above PSS_SEG_KMAX or a window
 * above PSS_SEG_WMAX take the wide fused form; otherwise the small-batch form
 * while its grid is at most one pass of resident workgroups, then the
 * resident kernel where the row fits it (16-byte aligned rows, V * element
 * size <= 400 KiB fp32 / 208 KiB fp16), the fused form where it does not.
 * PSS_FORM_RESIDENT forces the resident kernel where the row fits it (the
 * fused form otherwise).  All forms compute the same bits. */
static inline hipError_t pss_launch_rows(pss_args a, uint32_t rows, uint32_t max_k, uint32_t max_w, int form,
                                         hipStream_t st, hipEvent_t split_ev) {
    const size_t esz = a.dtype == PSS_DTYPE_F16 ? 2u : 4u;
    const bool vec = ((a.stride * esz) % 16u == 0u) && (((uintptr_t)a.logits & 15u) == 0u) &&
                     ((a.V * esz) % 16u == 0u);
    const bool fits = vec && pss_res_pick_nl(a.V, (uint32_t)esz) != 0;
    /* wide launches (top-k above PSS_SEG_KMAX or a window above
     * PSS_SEG_WMAX ids): the split-row wide form where rows are 16-byte
     * aligned, the wide fused form when asked for or otherwise */
    if (form < 0 && vec && (max_k > PSS_SEG_KMAX || max_w > PSS_SEG_WMAX) && pss_wsplit_segments(a.V))
        return pss_wsplit_launch(a, rows, st);
    if (form == PSS_FORM_RESIDENT || form < 0) {
        bool use = form == PSS_FORM_RESIDENT && fits;
        if (form < 0 && fits && max_k <= PSS_SEG_KMAX && max_w <= PSS_SEG_WMAX) {
            const uint64_t item = (uint64_t)PSS_WAVE * pss_stream_pick_ept(a.V, rows);
            const uint32_t NS = (uint32_t)((a.V + item - 1u) / item);
            const uint64_t cap = pss_small_capacity();
            use = !(cap && (uint64_t)rows * pss_small_gw(NS) <= cap);
        }
        if (use) {
            a.vec_ok = 1u;
            hipError_t e = pss_res_launch(a, rows, st);
            if (e == hipSuccess && split_ev) e = hipEventRecord(split_ev, st);
            return e;
        }
        if (form == PSS_FORM_RESIDENT) form = PSS_FORM_FUSED;
    }
    return pss_stream_launch(a, rows, max_k, max_w, form, st, split_ev);
}

#endif /* PSS_RESIDENT_H */
