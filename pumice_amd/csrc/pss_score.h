/*
 * pss_score.h - scoring mode (ArgMax-Reduce.comp mode 2, :169-214): the
 * negative log-likelihood of a given target token under each row's raw
 * logits, log(Z) + gmax - l[target], for generateScore
 * (src/generate.c:1161-1236).  No temperature, no penalty, no draw; the row
 * state is untouched except token and position.
 *
 * One workgroup per row, two passes over the row with 16-byte buffer loads:
 * the maximum of the canonical values (order-preserving keys), then the exact
 * fixed-point mass Zq = sum fixq(exp(t - gmax)) (so the reduction order does
 * not matter).  Thread 0 evaluates pss_score_nll (binary64 log, one rounding
 * to binary32) and writes result[passIdx] = the NLL's bits, token = target,
 * position + do_increment.  The target of pass p of row r is
 * targets[r * PSS_RESULT_SLOTS + p] (pss_set_score_targets; the shader reads
 * tokenIds[1 + passIdx]); a target >= V scores against l = 0, as the shader's
 * sum over no matching thread.
 */
#ifndef PSS_SCORE_H
#define PSS_SCORE_H

#include "pss_device.h"
#include "pss_stream.h"

#define PSS_SCORE_NT 1024

/* The canonical values of 16-byte chunk c of the row (E of them), ids past V
 * (zeros from the range-checked load) flagged invalid. */
template <int DT>
__device__ __forceinline__ void pss_score_chunk(__amdgpu_buffer_rsrc_t rs, uint32_t c, uint32_t V, float (&x)[8],
                                                bool (&ok)[8]) {
    constexpr int E = DT == PSS_DTYPE_F16 ? 8 : 4;
    const uint4 w = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(c * 16u), 0, 0));
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < E; ++e) {
        float v;
        if (DT == PSS_DTYPE_F16) {
            const uint16_t h = (uint16_t)(ww[e >> 1] >> ((e & 1) * 16));
            _Float16 hf;
            __builtin_memcpy(&hf, &h, 2);
            v = (float)hf;
        } else {
            v = __uint_as_float(ww[e]);
        }
        x[e] = pss_canon(v);
        ok[e] = c * (uint32_t)E + (uint32_t)e < V;
    }
}

template <int DT>
__global__ void __launch_bounds__(PSS_SCORE_NT) pss_score_kernel(pss_args a, const uint32_t* __restrict__ targets) {
    constexpr int NT = PSS_SCORE_NT;
    constexpr int E = DT == PSS_DTYPE_F16 ? 8 : 4;
    constexpr uint32_t esz = DT == PSS_DTYPE_F16 ? 2u : 4u;
    __shared__ uint64_t red[NT / PSS_WAVE];
    pss_globalize(a);
    const uint32_t row = blockIdx.x, tid = pss_tid();
    const uint32_t V = a.V;
    const __amdgpu_buffer_rsrc_t rs = pss_row_rsrc(a, row, esz);
    const uint32_t nch = (V + (uint32_t)E - 1u) / (uint32_t)E;
    const char* rowp = (const char*)a.logits + (size_t)row * a.stride * esz;

    /* gmax (key order: canonical values, NaN already -inf) */
    uint32_t mk = PSS_KEY_NEG_INF;
    if (a.vec_ok) {
        for (uint32_t c = tid; c < nch; c += NT) {
            float x[8];
            bool ok[8];
            pss_score_chunk<DT>(rs, c, V, x, ok);
#pragma unroll
            for (int e = 0; e < E; ++e) mk = ok[e] && pss_key(x[e]) > mk ? pss_key(x[e]) : mk;
        }
    } else {
        for (uint32_t j = tid; j < V; j += NT) {
            const uint32_t k = pss_key(pss_canon(pss_load1(rowp, DT, j)));
            mk = k > mk ? k : mk;
        }
    }
    const uint32_t gk = (uint32_t)block_max_u64<NT>(mk, red);
    const float gmax = pss_unkey(gk);

    /* Zq */
    uint64_t zl = 0;
    if (a.vec_ok) {
        for (uint32_t c = tid; c < nch; c += NT) {
            float x[8];
            bool ok[8];
            pss_score_chunk<DT>(rs, c, V, x, ok);
#pragma unroll
            for (int e = 0; e < E; ++e) zl += ok[e] ? pss_fixq(pss_prob(x[e], gmax)) : 0ull;
        }
    } else {
        for (uint32_t j = tid; j < V; j += NT) zl += pss_fixq(pss_prob(pss_canon(pss_load1(rowp, DT, j)), gmax));
    }
    const uint64_t zq = block_sum_u64<NT>(zl, red);

    if (tid == 0u) {
        const uint32_t target = targets[row * PSS_RESULT_SLOTS + a.pass_idx];
        const float lt = target < V ? pss_canon(pss_load1(rowp, DT, target)) : 0.0f;
        const float nll = pss_score_nll(zq, gmax, lt);
        a.result[row * PSS_RESULT_SLOTS + a.pass_idx] = __float_as_uint(nll);
        a.token_ids[row] = target;
        if (a.do_inc) a.position[row] = a.position[row] + 1u;
        if (a.host_tokens) a.host_tokens[row] = target;
        if (a.info) {
            pss_row_info inf = {};
            inf.token = target;
            inf.tmax_key = gk;
            inf.z_kept = zq;
            inf.flags = PSS_INFO_SCORE;
            a.info[row] = inf;
        }
    }
}

#endif /* PSS_SCORE_H */
