/*
 * pss_sampler.hip - C ABI of the gfx950 sampler (include/pumice_sampler.h).
 *
 * Host side of the drop-in boundary: the sampler object owns the per-row state
 * buffers that the reference keeps in model_state (src/state.c:84-104:
 * position, tokenIds, result, sampleParams, sampleRng, sampleHistory), sized for
 * max_rows independent rows, and enqueues the sampler kernels on one HIP
 * stream.  Allocation happens only in pss_create.
 */
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "pss_general.h"
#include "pss_score.h"
#include "pss_stream.h"
#include "pss_resident.h"
#include "pss_sampler_priv.h"
#include "pumice_sampler.h"

#define HIP_TRY(expr)                            \
    do {                                         \
        if ((expr) != hipSuccess) return PSS_ERR_HIP; \
    } while (0)

extern "C" const char* pss_status_string(pss_status st) {
    switch (st) {
        case PSS_OK: return "ok";
        case PSS_ERR_INVALID_ARG: return "invalid argument";
        case PSS_ERR_ALLOC: return "allocation failed";
        case PSS_ERR_HIP: return "HIP runtime error";
        case PSS_ERR_UNSUPPORTED: return "unsupported";
        case PSS_ERR_NO_DEVICE: return "no gfx950 device";
    }
    return "unknown status";
}

extern "C" uint32_t pss_mask_words(uint32_t vocab) { return (vocab + 31u) / 32u; }

__global__ void pss_fill_u32_kernel(uint32_t* dst, uint64_t n, uint32_t v) {
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) dst[i] = v;
}

static pss_status fill_u32(hipStream_t st, uint32_t* dst, uint64_t n, uint32_t v) {
    if (n == 0) return PSS_OK;
    uint64_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    pss_fill_u32_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(dst, n, v);
    return hipGetLastError() == hipSuccess ? PSS_OK : PSS_ERR_HIP;
}

static void free_all(pss_sampler* s) {
    if (!s) return;
    (void)hipFree(s->d_params);
    (void)hipFree(s->d_rng);
    (void)hipFree(s->d_step);
    (void)hipFree(s->d_pos);
    (void)hipFree(s->d_hist);
    (void)hipFree(s->d_result);
    (void)hipFree(s->d_tokens);
    (void)hipFree(s->d_targets);
    (void)hipFree(s->d_gate);
    (void)hipFree(s->d_ws);
    free(s->h_topk);
    free(s->h_wlen);
    if (s->own_stream && s->stream) (void)hipStreamDestroy(s->stream);
    free(s);
}

extern "C" pss_status pss_create(pss_sampler** out, uint32_t vocab, uint32_t max_rows,
                                 void* hip_stream) {
    if (!out) return PSS_ERR_INVALID_ARG;
    *out = NULL;
    if (vocab == 0 || max_rows == 0) return PSS_ERR_INVALID_ARG;
    if (vocab > PSS_MAX_VOCAB) return PSS_ERR_UNSUPPORTED;
    int dev = 0, ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) return PSS_ERR_NO_DEVICE;
    if (hipGetDevice(&dev) != hipSuccess) return PSS_ERR_NO_DEVICE;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return PSS_ERR_NO_DEVICE;
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return PSS_ERR_NO_DEVICE;

    pss_sampler* s = (pss_sampler*)calloc(1, sizeof(pss_sampler));
    if (!s) return PSS_ERR_ALLOC;
    s->device = dev;
    s->V = vocab;
    s->max_rows = max_rows;
    if (hip_stream) {
        s->stream = (hipStream_t)hip_stream;
    } else {
        if (hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking) != hipSuccess) {
            free(s);
            return PSS_ERR_HIP;
        }
        s->own_stream = 1;
    }
    const size_t R = max_rows;
    s->h_topk = (uint32_t*)calloc(R, sizeof(uint32_t));
    s->h_wlen = (uint32_t*)calloc(R, sizeof(uint32_t));
    if (!s->h_topk || !s->h_wlen) {
        free_all(s);
        return PSS_ERR_ALLOC;
    }
    s->ws_bytes = pss_stream_ws_bytes(max_rows);
    if (hipMalloc((void**)&s->d_params, sizeof(sample_params) * R) != hipSuccess ||
        hipMalloc((void**)&s->d_rng, 4 * R) != hipSuccess ||
        hipMalloc((void**)&s->d_step, 4 * R) != hipSuccess ||
        hipMalloc((void**)&s->d_pos, 4 * R) != hipSuccess ||
        hipMalloc((void**)&s->d_hist, 4 * R * PSS_MAX_PENALTY_LEN) != hipSuccess ||
        hipMalloc((void**)&s->d_result, 4 * R * PSS_RESULT_SLOTS) != hipSuccess ||
        hipMalloc((void**)&s->d_tokens, 4 * R) != hipSuccess ||
        hipMalloc((void**)&s->d_targets, 4 * R * PSS_RESULT_SLOTS) != hipSuccess ||
        hipMalloc((void**)&s->d_gate, 256) != hipSuccess ||
        (s->ws_bytes && hipMalloc(&s->d_ws, s->ws_bytes) != hipSuccess)) {
        free_all(s);
        return PSS_ERR_ALLOC;
    }
    pss_status st = PSS_OK;
    if (st == PSS_OK) st = fill_u32(s->stream, (uint32_t*)s->d_params, R * 7, 0u);
    if (st == PSS_OK) st = fill_u32(s->stream, s->d_rng, R, 0u);
    if (st == PSS_OK) st = fill_u32(s->stream, s->d_step, R, 0u);
    if (st == PSS_OK) st = fill_u32(s->stream, s->d_pos, R, 0u);
    if (st == PSS_OK) st = fill_u32(s->stream, s->d_hist, R * PSS_MAX_PENALTY_LEN, PSS_SENTINEL);
    if (st == PSS_OK) st = fill_u32(s->stream, s->d_result, R * PSS_RESULT_SLOTS, 0u);
    if (st == PSS_OK) st = fill_u32(s->stream, s->d_tokens, R, 0u);
    if (st == PSS_OK) st = fill_u32(s->stream, s->d_targets, R * PSS_RESULT_SLOTS, 0u);
    if (st == PSS_OK) st = fill_u32(s->stream, s->d_gate, 64, 0xFFFFFFFFu);
    if (st == PSS_OK && s->ws_bytes) st = fill_u32(s->stream, (uint32_t*)s->d_ws, s->ws_bytes / 4, 0u);
    if (st == PSS_OK && hipStreamSynchronize(s->stream) != hipSuccess) st = PSS_ERR_HIP;
    if (st != PSS_OK) {
        free_all(s);
        return st;
    }
    *out = s;
    return PSS_OK;
}

extern "C" pss_status pss_destroy(pss_sampler* s) {
    if (!s) return PSS_ERR_INVALID_ARG;
    pss_status st = hipStreamSynchronize(s->stream) == hipSuccess ? PSS_OK : PSS_ERR_HIP;
    free_all(s);
    return st;
}

extern "C" void* pss_stream(pss_sampler* s) { return s ? (void*)s->stream : NULL; }

static int rows_ok(const pss_sampler* s, uint32_t row0, uint32_t rows) {
    return s && rows > 0 && row0 < s->max_rows && rows <= s->max_rows - row0;
}

/* Upload `bytes` from host memory and wait for it, so the caller may reuse
 * the buffer on return (setup path, not the per-step path). */
static pss_status upload_sync(pss_sampler* s, void* dst, const void* src, size_t bytes) {
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s->stream));
    HIP_TRY(hipStreamSynchronize(s->stream));
    return PSS_OK;
}

extern "C" pss_status pss_set_params(pss_sampler* s, uint32_t row0, uint32_t rows,
                                     const sample_params* params, const uint32_t* seeds) {
    if (!rows_ok(s, row0, rows) || !params) return PSS_ERR_INVALID_ARG;
    for (uint32_t i = 0; i < rows; ++i) {
        const sample_params& p = params[i];
        if (isnan(p.topP) || isnan(p.minP) || isnan(p.repPenalty) || isnan(p.presencePenalty))
            return PSS_ERR_INVALID_ARG;
        if (p.minP > 1.0f) return PSS_ERR_INVALID_ARG;
    }
    pss_status st = upload_sync(s, s->d_params + row0, params, sizeof(sample_params) * rows);
    if (st != PSS_OK) return st;
    for (uint32_t i = 0; i < rows; ++i) {
        s->h_topk[row0 + i] = params[i].topK;
        s->h_wlen[row0 + i] = params[i].penaltyLength;
    }
    if (seeds) {
        st = upload_sync(s, s->d_rng + row0, seeds, 4u * rows);
    } else {
        st = fill_u32(s->stream, s->d_rng + row0, rows, 0u);
    }
    if (st != PSS_OK) return st;
    return fill_u32(s->stream, s->d_step + row0, rows, 0u);
}

extern "C" pss_status pss_reset_history(pss_sampler* s, uint32_t row0, uint32_t rows, uint32_t fill) {
    if (!rows_ok(s, row0, rows)) return PSS_ERR_INVALID_ARG;
    return fill_u32(s->stream, s->d_hist + (size_t)row0 * PSS_MAX_PENALTY_LEN,
                    (uint64_t)rows * PSS_MAX_PENALTY_LEN, fill);
}

extern "C" pss_status pss_set_history(pss_sampler* s, uint32_t row0, uint32_t rows,
                                      const uint32_t* hist, uint32_t len) {
    if (!rows_ok(s, row0, rows) || (!hist && len) || len > PSS_MAX_PENALTY_LEN)
        return PSS_ERR_INVALID_ARG;
    size_t n = (size_t)rows * PSS_MAX_PENALTY_LEN;
    uint32_t* tmp = (uint32_t*)malloc(n * 4);
    if (!tmp) return PSS_ERR_ALLOC;
    for (uint32_t r = 0; r < rows; ++r)
        for (uint32_t h = 0; h < PSS_MAX_PENALTY_LEN; ++h)
            tmp[(size_t)r * PSS_MAX_PENALTY_LEN + h] = h < len ? hist[(size_t)r * len + h] : PSS_SENTINEL;
    pss_status st = upload_sync(s, s->d_hist + (size_t)row0 * PSS_MAX_PENALTY_LEN, tmp, n * 4);
    free(tmp);
    return st;
}

extern "C" pss_status pss_set_score_targets(pss_sampler* s, uint32_t row0, uint32_t rows, uint32_t slots,
                                            const uint32_t* ids) {
    if (!rows_ok(s, row0, rows) || !ids || slots == 0 || slots > PSS_RESULT_SLOTS) return PSS_ERR_INVALID_ARG;
    HIP_TRY(hipMemcpy2DAsync(s->d_targets + (size_t)row0 * PSS_RESULT_SLOTS, 4u * PSS_RESULT_SLOTS, ids,
                             4u * slots, 4u * slots, rows, hipMemcpyHostToDevice, s->stream));
    HIP_TRY(hipStreamSynchronize(s->stream));
    return PSS_OK;
}

extern "C" pss_status pss_set_position(pss_sampler* s, uint32_t row0, uint32_t rows,
                                       const uint32_t* pos) {
    if (!rows_ok(s, row0, rows) || !pos) return PSS_ERR_INVALID_ARG;
    return upload_sync(s, s->d_pos + row0, pos, 4u * rows);
}

extern "C" pss_status pss_sanitize_request(sample_params* params, uint32_t* seed) {
    if (!params || !seed) return PSS_ERR_INVALID_ARG;
    if (params->penaltyLength > PSS_MAX_PENALTY_LEN) params->penaltyLength = PSS_MAX_PENALTY_LEN;
    if (*seed == 0u) *seed = 1u;
    return PSS_OK;
}

static pss_args make_args(pss_sampler* s, const void* logits, uint32_t dtype, uint64_t row_stride,
                          uint32_t mode, uint32_t do_increment, uint32_t pass_idx,
                          uint32_t rng_mode, const pss_enqueue_opts* o) {
    pss_args a;
    memset(&a, 0, sizeof a);
    a.logits = logits;
    a.stride = row_stride;
    a.V = s->V;
    a.dtype = dtype;
    a.mode = mode;
    a.do_inc = do_increment ? 1u : 0u;
    a.pass_idx = pass_idx;
    a.rng_mode = rng_mode;
    a.params = s->d_params;
    a.rng = s->d_rng;
    a.step = s->d_step;
    a.position = s->d_pos;
    a.history = s->d_hist;
    a.result = s->d_result;
    a.token_ids = s->d_tokens;
    a.mask_words = pss_mask_words(s->V);
    a.ws = s->d_ws;
    a.kmax_cov = PSS_SEG_KMAX;
    a.wmax_cov = PSS_SEG_WMAX;
    if (o) {
        a.info = o->row_info;
        a.kept_mask = o->kept_mask;
        a.probs = o->probs;
        a.probs_stride = o->probs_stride;
        a.host_tokens = o->host_tokens;
        if (o->flags & PSS_ENQ_GATED) {
            a.gate = s->d_gate;
            a.gate_seq = o->gate_seq;
            a.eos = o->eos;
        }
    }
    return a;
}

extern "C" pss_status pss_reset_gate(pss_sampler* s) {
    if (!s) return PSS_ERR_INVALID_ARG;
    return fill_u32(s->stream, s->d_gate, 1, 0xFFFFFFFFu);
}

extern "C" pss_status pss_enqueue_ex(pss_sampler* s, const void* logits, uint32_t dtype,
                                     uint64_t row_stride, uint32_t rows, uint32_t mode,
                                     uint32_t do_increment, uint32_t pass_idx, uint32_t rng_mode,
                                     const pss_enqueue_opts* opts) {
    if (!s || !logits || rows == 0 || rows > s->max_rows) return PSS_ERR_INVALID_ARG;
    if (dtype != PSS_DTYPE_F32 && dtype != PSS_DTYPE_F16) return PSS_ERR_INVALID_ARG;
    if (mode != PSS_MODE_GREEDY && mode != PSS_MODE_SAMPLE && mode != PSS_MODE_SCORE) return PSS_ERR_INVALID_ARG;
    if (rng_mode != PSS_RNG_XORSHIFT32 && rng_mode != PSS_RNG_PHILOX) return PSS_ERR_INVALID_ARG;
    if (pass_idx >= PSS_RESULT_SLOTS || row_stride < s->V) return PSS_ERR_INVALID_ARG;
    if (opts && (opts->flags & PSS_ENQ_GATED) && (mode == PSS_MODE_SCORE || opts->gate_seq == 0))
        return PSS_ERR_INVALID_ARG;
    if (opts && opts->probs && opts->probs_stride < s->V) return PSS_ERR_INVALID_ARG;
    pss_args a = make_args(s, logits, dtype, row_stride, mode, do_increment, pass_idx, rng_mode, opts);
    if (mode == PSS_MODE_SCORE) {
        const size_t esz = dtype == PSS_DTYPE_F16 ? 2u : 4u;
        a.vec_ok = ((a.stride * esz) % 16u == 0u) && (((uintptr_t)a.logits & 15u) == 0u) &&
                   ((a.V * esz) % 16u == 0u);
        if (dtype == PSS_DTYPE_F16)
            pss_score_kernel<PSS_DTYPE_F16><<<dim3(rows), dim3(PSS_SCORE_NT), 0, s->stream>>>(a, s->d_targets);
        else
            pss_score_kernel<PSS_DTYPE_F32><<<dim3(rows), dim3(PSS_SCORE_NT), 0, s->stream>>>(a, s->d_targets);
        return hipGetLastError() == hipSuccess ? PSS_OK : PSS_ERR_HIP;
    }
    /* The streaming kernel, or the one-workgroup-per-row general kernel when
     * the caller asks for it (both compute identical results). */
    const int general = opts && (opts->flags & PSS_ENQ_GENERAL);
    if (!general) {
        uint32_t max_k = 0, max_w = 0;
        for (uint32_t r = 0; r < rows; ++r) {
            max_k = s->h_topk[r] > max_k ? s->h_topk[r] : max_k;
            max_w = s->h_wlen[r] > max_w ? s->h_wlen[r] : max_w;
        }
        const hipEvent_t split = opts ? (hipEvent_t)opts->split_event : NULL;
        const uint32_t fl = opts ? opts->flags : 0u;
        const int form = (fl & PSS_ENQ_SPLIT)      ? PSS_FORM_SPLIT
                         : (fl & PSS_ENQ_FUSED)    ? PSS_FORM_FUSED
                         : (fl & PSS_ENQ_SMALL)    ? PSS_FORM_SMALL
                         : (fl & PSS_ENQ_RESIDENT) ? PSS_FORM_RESIDENT
                                                   : -1;
        if (pss_launch_rows(a, rows, max_k, max_w, form, s->stream, split) != hipSuccess) return PSS_ERR_HIP;
        return PSS_OK;
    }
    pss_general_kernel<<<dim3(rows), dim3(PSS_GEN_NT), 0, s->stream>>>(a);
    if (hipGetLastError() != hipSuccess) return PSS_ERR_HIP;
    if (opts && opts->split_event && hipEventRecord((hipEvent_t)opts->split_event, s->stream) != hipSuccess)
        return PSS_ERR_HIP;
    return PSS_OK;
}

extern "C" pss_status pss_enqueue(pss_sampler* s, const void* logits, uint32_t dtype,
                                  uint64_t row_stride, uint32_t rows, uint32_t mode,
                                  uint32_t do_increment, uint32_t pass_idx, uint32_t rng_mode) {
    return pss_enqueue_ex(s, logits, dtype, row_stride, rows, mode, do_increment, pass_idx,
                          rng_mode, NULL);
}

extern "C" pss_status pss_read_results(pss_sampler* s, uint32_t rows, uint32_t* results,
                                       uint32_t* tokens) {
    if (!s || rows == 0 || rows > s->max_rows) return PSS_ERR_INVALID_ARG;
    if (results)
        HIP_TRY(hipMemcpyAsync(results, s->d_result, 4u * PSS_RESULT_SLOTS * rows,
                               hipMemcpyDeviceToHost, s->stream));
    if (tokens)
        HIP_TRY(hipMemcpyAsync(tokens, s->d_tokens, 4u * rows, hipMemcpyDeviceToHost, s->stream));
    HIP_TRY(hipStreamSynchronize(s->stream));
    return PSS_OK;
}

extern "C" pss_status pss_read_state(pss_sampler* s, uint32_t rows, uint32_t* history,
                                     uint32_t* position, uint32_t* rng, uint32_t* step) {
    if (!s || rows == 0 || rows > s->max_rows) return PSS_ERR_INVALID_ARG;
    if (history)
        HIP_TRY(hipMemcpyAsync(history, s->d_hist, 4u * PSS_MAX_PENALTY_LEN * (size_t)rows,
                               hipMemcpyDeviceToHost, s->stream));
    if (position) HIP_TRY(hipMemcpyAsync(position, s->d_pos, 4u * rows, hipMemcpyDeviceToHost, s->stream));
    if (rng) HIP_TRY(hipMemcpyAsync(rng, s->d_rng, 4u * rows, hipMemcpyDeviceToHost, s->stream));
    if (step) HIP_TRY(hipMemcpyAsync(step, s->d_step, 4u * rows, hipMemcpyDeviceToHost, s->stream));
    HIP_TRY(hipStreamSynchronize(s->stream));
    return PSS_OK;
}

extern "C" pss_status pss_get_state_ptrs(pss_sampler* s, pss_state_ptrs* out) {
    if (!s || !out) return PSS_ERR_INVALID_ARG;
    out->result = s->d_result;
    out->token_ids = s->d_tokens;
    out->position = s->d_pos;
    out->rng = s->d_rng;
    out->step = s->d_step;
    out->history = s->d_hist;
    return PSS_OK;
}

/* ------------------------------------------------------------------------ */
/* the entry point that allocates nothing                                    */
/* ------------------------------------------------------------------------ */

/* Workspace of the small-batch and two-kernel forms for up to
 * PSS_NOALLOC_MAX_ROWS rows: per-row bound, arrival ticket and candidate
 * pool.  One copy per GPU, held until the process ends.  In host code this
 * name is a host-side stand-in, not a device address: only the pointer from
 * hipGetSymbolAddress (kept per device below) is ever passed to a kernel. */
static __device__ __align__(256) unsigned char scratch[PSS_NOALLOC_MAX_ROWS * PSS_WS_ROW_BYTES];

#define PSS_NOALLOC_DEVICES 64
static void* g_scratch_ptr[PSS_NOALLOC_DEVICES]; /* device address of scratch, per device */
static std::mutex g_scratch_mu;

/* Set-up on the first call on a device (that device current): check it is a
 * gfx950, look up its copy of scratch and clear it once on the caller's
 * stream.  The kernels return every counter they use to zero (the bound and
 * the arrival ticket are reset by the workgroup that finishes the row), so
 * later calls find it clear. */
static pss_status noalloc_scratch(hipStream_t st, void** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return PSS_ERR_NO_DEVICE;
    if (dev >= PSS_NOALLOC_DEVICES) return PSS_ERR_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return PSS_ERR_NO_DEVICE;
        if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return PSS_ERR_NO_DEVICE;
        void* p = NULL;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return PSS_ERR_HIP;
        const pss_status f = fill_u32(st, (uint32_t*)p, sizeof(scratch) / 4u, 0u);
        if (f != PSS_OK) return f;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return PSS_OK;
}

extern "C" pss_status pss_enqueue_noalloc(const sample_params* params, const pss_state_ptrs* state,
                                          uint32_t vocab, const void* logits, uint32_t dtype,
                                          uint64_t row_stride, uint32_t rows, uint32_t mode,
                                          uint32_t do_increment, uint32_t pass_idx, uint32_t rng_mode,
                                          uint32_t max_topk, uint32_t max_window,
                                          const pss_enqueue_opts* opts, void* hip_stream) {
    if (!params || !state || !logits || !state->result || !state->token_ids || !state->position ||
        !state->rng || !state->step || !state->history)
        return PSS_ERR_INVALID_ARG;
    if (rows == 0 || rows > PSS_NOALLOC_MAX_ROWS || vocab == 0) return PSS_ERR_INVALID_ARG;
    if (vocab > PSS_MAX_VOCAB) return PSS_ERR_UNSUPPORTED;
    if (dtype != PSS_DTYPE_F32 && dtype != PSS_DTYPE_F16) return PSS_ERR_INVALID_ARG;
    if (mode != PSS_MODE_GREEDY && mode != PSS_MODE_SAMPLE) return PSS_ERR_INVALID_ARG;
    if (rng_mode != PSS_RNG_XORSHIFT32 && rng_mode != PSS_RNG_PHILOX) return PSS_ERR_INVALID_ARG;
    if (pass_idx >= PSS_RESULT_SLOTS || row_stride < vocab) return PSS_ERR_INVALID_ARG;
    if (opts && (opts->flags != 0u || opts->split_event)) return PSS_ERR_INVALID_ARG;
    if (opts && opts->probs && opts->probs_stride < vocab) return PSS_ERR_INVALID_ARG;
    const hipStream_t st = (hipStream_t)hip_stream;
    void* ws = NULL;
    const pss_status ss = noalloc_scratch(st, &ws);
    if (ss != PSS_OK) return ss;

    pss_args a;
    memset(&a, 0, sizeof a);
    a.logits = logits;
    a.stride = row_stride;
    a.V = vocab;
    a.dtype = dtype;
    a.mode = mode;
    a.do_inc = do_increment ? 1u : 0u;
    a.pass_idx = pass_idx;
    a.rng_mode = rng_mode;
    a.params = params;
    a.rng = state->rng;
    a.step = state->step;
    a.position = state->position;
    a.history = state->history;
    a.result = state->result;
    a.token_ids = state->token_ids;
    a.mask_words = pss_mask_words(vocab);
    a.ws = ws;
    a.kmax_cov = PSS_SEG_KMAX;
    a.wmax_cov = PSS_SEG_WMAX;
    if (opts) {
        a.info = opts->row_info;
        a.kept_mask = opts->kept_mask;
        a.probs = opts->probs;
        a.probs_stride = opts->probs_stride;
        a.host_tokens = opts->host_tokens;
    }
    /* the automatic form choice; rows <= PSS_NOALLOC_MAX_ROWS, so a form
     * that uses the workspace stays inside scratch */
    return pss_launch_rows(a, rows, max_topk, max_window, -1, st, NULL) == hipSuccess ? PSS_OK : PSS_ERR_HIP;
}

/* ------------------------------------------------------------------------ */
/* read ceiling: the stream alone                                            */
/* ------------------------------------------------------------------------ */

/* The resident kernel's access pattern with nothing else: one 1,024-thread
 * workgroup per 400 KiB chunk, each wave reading PSS_READ_NL contiguous KiB
 * with 16-byte nontemporal buffer loads, PSS_RES_DEPTH of them in flight;
 * the values are folded into one word per workgroup so that no load is
 * dropped.  Bytes beyond `bytes` read as 0 (buffer bounds). */
#define PSS_READ_NL 25
__global__ void __launch_bounds__(1024) pss_read_kernel(const char* src, uint64_t bytes, uint32_t* out) {
    constexpr int NL = PSS_READ_NL, D = PSS_RES_DEPTH;
    const uint64_t chunk = (uint64_t)NL * 16u * 1024u;
    const uint64_t off = (uint64_t)blockIdx.x * chunk;
    const uint64_t left = bytes - off;
    const int nrec = (int)(left < chunk ? left : chunk);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)(src + off), (short)0, nrec, PSS_BUF_DW3);
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t vb = (wave * (uint32_t)NL * 64u + lane) * 16u;
    uint4 r[NL];
    uint32_t acc = 0u;
#pragma unroll
    for (int j = 0; j < D; ++j)
        r[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(vb + 1024u * j), 0, PSS_NT));
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        if (j + D < NL)
            r[j + D] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(vb + 1024u * (j + D)), 0, PSS_NT));
        acc ^= r[j].x ^ r[j].y ^ r[j].z ^ r[j].w;
    }
    acc = wave_max_u32(acc);
    __shared__ uint32_t wv[16];
    if (lane == 0u) wv[wave] = acc;
    __syncthreads();
    if (threadIdx.x == 0u) {
        uint32_t x = 0u;
        for (int w = 0; w < 16; ++w) x ^= wv[w];
        out[blockIdx.x] = x;
    }
}

extern "C" uint32_t pss_read_ceiling_blocks(uint64_t bytes) {
    const uint64_t chunk = (uint64_t)PSS_READ_NL * 16u * 1024u;
    return (uint32_t)((bytes + chunk - 1u) / chunk);
}

extern "C" pss_status pss_read_ceiling(const void* src, uint64_t bytes, uint32_t* out, void* hip_stream) {
    if (!src || !out || bytes == 0 || (bytes & 15u) || ((uintptr_t)src & 15u)) return PSS_ERR_INVALID_ARG;
    const uint32_t blocks = pss_read_ceiling_blocks(bytes);
    pss_read_kernel<<<dim3(blocks), dim3(1024), 0, (hipStream_t)hip_stream>>>((const char*)src, bytes, out);
    return hipGetLastError() == hipSuccess ? PSS_OK : PSS_ERR_HIP;
}
