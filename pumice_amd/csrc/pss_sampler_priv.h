/*
 * pss_sampler_priv.h - the sampler object behind the opaque pss_sampler
 * handle, shared by the library's translation units (pss_sampler.hip, and
 * plh_lmhead.hip, whose fused greedy head writes the sampler's token state).
 */
#ifndef PSS_SAMPLER_PRIV_H
#define PSS_SAMPLER_PRIV_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pumice_sampler.h"

struct pss_sampler {
    int device;
    hipStream_t stream;
    int own_stream;
    uint32_t V;
    uint32_t max_rows;
    sample_params* d_params;
    uint32_t* d_rng;
    uint32_t* d_step;
    uint32_t* d_pos;
    uint32_t* d_hist;
    uint32_t* d_result;
    uint32_t* d_tokens;
    uint32_t* d_targets; /* scoring targets [max_rows][PSS_RESULT_SLOTS] */
    uint32_t* d_gate;    /* eos_at of PSS_ENQ_GATED passes (one word, 256-byte allocation) */
    void* d_ws;       /* streaming-kernel workspace: per-row bounds and candidate pools */
    size_t ws_bytes;
    uint32_t* h_topk; /* host copy of each row's topK (picks the kernel variant) */
    uint32_t* h_wlen; /* host copy of each row's penaltyLength (likewise) */
};

#endif /* PSS_SAMPLER_PRIV_H */
