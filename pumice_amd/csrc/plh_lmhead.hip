/*
 * plh_lmhead.hip - the LM head on gfx950 (include/pumice_lmhead.h): the final
 * RMSNorm and the fp16 GEMV over the vocabulary that produce the sampler's
 * logits (LMHead-GEMV-Q16.comp:28-72), and the fused greedy form that reduces
 * them to a token without a logits buffer (LMHead-GEMV-ArgMax-Q16.comp +
 * ArgMax-Reduce.comp:135-166).
 *
 * Two launches per call, both on the head's stream:
 *
 *   plh_norm_kernel   one 256-thread workgroup per row: the sum of squares in
 *                     binary64 (each square exact), inv_rms in binary32, and
 *                     the normalized row a[k] = (x[k] gamma[k]) inv_rms into
 *                     the head's workspace.
 *   plh_gemv_kernel   grid (ceil(V / 64), row groups), 4 waves per workgroup:
 *                     lane l owns column 64 tile + l, wave s the K-slice s, so
 *                     every 16-byte weight load of a wave is one contiguous
 *                     1 KiB run of the block-transposed head; the activations
 *                     are wave-uniform and come through scalar loads, so the
 *                     vector side issues only the weight loads, 8 fp16->fp32
 *                     conversions and 8 R fused multiply-adds per block.  The
 *                     four slice partials meet in LDS and are added in slice
 *                     order.  The head is read once per row group (R = 1, 2,
 *                     4 or 8 rows share each weight load): the kernel is
 *                     bound by HBM, the algorithmic bytes are K V 2 per group.
 *
 * Greedy form: each workgroup reduces its 64 columns to the packed maximum
 * (key(value) << 32) | (0xFFFFFFFF - id) (largest value, then lowest id; NaN
 * maps to -inf) and folds it into one of the row's PLH_WIN_SLOTS slots (tile
 * mod 64, each in its own 128-byte line, so the atomics of 1,600 workgroups
 * of a 102,400-column head, which finish together, queue 25 deep at most) with an agent-scope atomic max and
 * ends: no workgroup waits for its atomic.  plh_greedy_reduce_kernel, next on
 * the stream (the kernel boundary orders the atomics before its loads), reads
 * and clears a row's slots with one wave and writes result / token_ids /
 * position as ArgMax-Reduce mode 0 -- the reference's own two dispatches
 * (src/generate.c:540-546).
 */
#include <hip/hip_runtime.h>
#include <stdlib.h>
#include <string.h>

#include "pss_device.h"
#include "pss_math.h"
#include "pss_sampler_priv.h"
#include "pumice_lmhead.h"

#define PLH_NORM_NT 256
#define PLH_WIN_SLOTS 64u
#define PLH_WIN_STRIDE 16u /* u64 per slot: one 128-byte line */
#define PLH_WIN_ROW (PLH_WIN_SLOTS * PLH_WIN_STRIDE)
#define PLH_NT 256 /* PLH_SLICES waves */
static_assert(PLH_NT == PLH_SLICES * PSS_WAVE, "one wave per K-slice");
static_assert(PLH_TILE == PSS_WAVE, "one column per lane");
static_assert(PLH_WIN_SLOTS == PSS_WAVE, "the final reduction reads a row's slots with one wave");
static_assert(16u * 8u <= PLH_NT, "16 lanes per row of a group");

struct plh_head {
    int device;
    hipStream_t stream;
    int own_stream;
    const uint4* w;
    const float* gamma;
    uint32_t K, V, max_rows, ntiles;
    float* an;               /* [max_rows][K] normalized rows */
    unsigned long long* win; /* [max_rows][PLH_WIN_ROW] greedy maxima, zeroed at the start of each greedy call */
};

struct plh_args {
    const uint4* w;
    float* logits;
    uint64_t lstride;
    unsigned long long* win;
    uint32_t* result;
    uint32_t* token_ids;
    uint32_t* position;
    uint32_t K, V, rows, ntiles, pass_idx, do_inc;
};

/* ---------------------------------------------------------------------- */
/* RMSNorm                                                                 */
/* ---------------------------------------------------------------------- */

/* Sum of squares: thread t adds x[k]^2 for k = t, t + 256, ... in order
 * (binary64; a binary32 square is exact in binary64), each wave combines its
 * lanes by the xor butterfly over 32, 16, ..., 1 (all lanes end equal), and
 * the four wave sums are added in wave order. */
__global__ void __launch_bounds__(PLH_NORM_NT) plh_norm_kernel(const float* __restrict__ x, uint64_t xs,
                                                               const float* __restrict__ gamma,
                                                               float* __restrict__ an, uint32_t K,
                                                               unsigned long long* __restrict__ win) {
    constexpr uint32_t NB = 16;                 /* values per thread held in registers */
    constexpr uint32_t CH = PLH_NORM_NT * NB;   /* K up to CH: one load of x and gamma */
    __shared__ double wsum[PLH_NORM_NT / PSS_WAVE];
    const uint32_t row = blockIdx.x, t = threadIdx.x;
    /* greedy calls: the row's maxima slots start at zero in every call (this
     * kernel precedes the GEMV's atomics in stream order), whatever an
     * earlier call left in them */
    if (win && t < PLH_WIN_SLOTS) win[(size_t)row * PLH_WIN_ROW + t * PLH_WIN_STRIDE] = 0ull;
    const float* xr = x + (size_t)row * xs;
    float v[NB], gv[NB];
    double s = 0.0;
    for (uint32_t k0 = t; k0 < K; k0 += CH) {
#pragma unroll
        for (uint32_t u = 0; u < NB; ++u) {
            const uint32_t k = k0 + u * PLH_NORM_NT;
            v[u] = k < K ? xr[k] : 0.0f;
            gv[u] = k < K ? gamma[k] : 0.0f;
        }
#pragma unroll
        for (uint32_t u = 0; u < NB; ++u) s = s + (double)v[u] * (double)v[u]; /* + 0 past K: exact */
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) s = s + __shfl_xor(s, off);
    if ((t & 63u) == 0u) wsum[t >> 6] = s;
    __syncthreads();
    double tot = wsum[0];
#pragma unroll
    for (int i = 1; i < PLH_NORM_NT / PSS_WAVE; ++i) tot = tot + wsum[i];
    const float inv = 1.0f / sqrtf((float)tot / (float)K + 1e-6f);
    float* ar = an + (size_t)row * K;
    if (K <= CH) { /* the registers hold this thread's whole share of the row */
#pragma unroll
        for (uint32_t u = 0; u < NB; ++u) {
            const uint32_t k = t + u * PLH_NORM_NT;
            if (k < K) ar[k] = (v[u] * gv[u]) * inv;
        }
        return;
    }
    for (uint32_t k0 = t; k0 < K; k0 += CH) {
#pragma unroll
        for (uint32_t u = 0; u < NB; ++u) {
            const uint32_t k = k0 + u * PLH_NORM_NT;
            v[u] = k < K ? xr[k] : 0.0f;
            gv[u] = k < K ? gamma[k] : 0.0f;
        }
#pragma unroll
        for (uint32_t u = 0; u < NB; ++u) {
            const uint32_t k = k0 + u * PLH_NORM_NT;
            if (k < K) ar[k] = (v[u] * gv[u]) * inv;
        }
    }
}

/* ---------------------------------------------------------------------- */
/* GEMV                                                                    */
/* ---------------------------------------------------------------------- */

__device__ __forceinline__ float plh_half(uint32_t w, int hi) {
    const uint16_t b = (uint16_t)(hi ? (w >> 16) : (w & 0xFFFFu));
    return (float)__builtin_bit_cast(_Float16, b);
}

/* N blocks of rows kb.. of this lane's column; wp advances past them.  The
 * head is read once per call and never reused, so the loads are nontemporal:
 * 126 us instead of 152 us per launch for a 839 MB head, measured. */
template <int N>
__device__ __forceinline__ void plh_load(uint4 (&q)[N], const uint4*& wp, uint32_t V) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int u = 0; u < N; ++u) {
        const u32x4 t = __builtin_nontemporal_load((const u32x4*)(wp + (size_t)u * V));
        q[u] = make_uint4(t.x, t.y, t.z, t.w);
    }
    wp += (size_t)N * V;
}

/* acc[r] = fmaf chain over the N blocks kb, kb + 1, ... (ascending k). */
template <int R, int N>
__device__ __forceinline__ void plh_consume(const uint4 (&q)[N], const float* const (&ar)[R], uint32_t kb,
                                            float (&acc)[R]) {
#pragma unroll
    for (int u = 0; u < N; ++u) {
        float h[8];
        h[0] = plh_half(q[u].x, 0);
        h[1] = plh_half(q[u].x, 1);
        h[2] = plh_half(q[u].y, 0);
        h[3] = plh_half(q[u].y, 1);
        h[4] = plh_half(q[u].z, 0);
        h[5] = plh_half(q[u].z, 1);
        h[6] = plh_half(q[u].w, 0);
        h[7] = plh_half(q[u].w, 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float* ap = ar[r] + (size_t)(kb + (uint32_t)u) * 8u;
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[r] = fmaf(ap[j], h[j], acc[r]);
        }
    }
}

template <int R, bool GREEDY>
__global__ void __launch_bounds__(PLH_NT) plh_gemv_kernel(plh_args a, const float* __restrict__ an) {
    __shared__ float part[PLH_SLICES][R][PSS_WAVE];
    const uint32_t tile = blockIdx.x, g = blockIdx.y;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t s = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t V = a.V, K = a.K, KB = K >> 3;
    const uint32_t kb0 = s * KB / PLH_SLICES, kb1 = (s + 1u) * KB / PLH_SLICES;
    const uint32_t n = tile * PLH_TILE + lane;
    const uint32_t nl = n < V ? n : V - 1u;

    const float* ar[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row = min(g * (uint32_t)R + (uint32_t)r, a.rows - 1u);
        ar[r] = an + (size_t)row * K;
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    const uint4* wp = a.w + (size_t)kb0 * V + nl;
#pragma unroll 8
    for (uint32_t kb = kb0; kb < kb1; ++kb) {
        uint4 q[1];
        plh_load<1>(q, wp, V);
        plh_consume<R, 1>(q, ar, kb, acc);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) part[s][r][lane] = acc[r];
    __syncthreads();
    if (s == 0u) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float v = part[0][r][lane];
#pragma unroll
            for (uint32_t i = 1; i < PLH_SLICES; ++i) v = v + part[i][r][lane];
            const uint32_t row = g * (uint32_t)R + (uint32_t)r;
            if (!GREEDY) {
                if (row < a.rows && n < V) a.logits[(size_t)row * a.lstride + n] = v;
            } else {
                const uint64_t pk = n < V ? ((uint64_t)pss_key(pss_canon(v)) << 32) | (0xFFFFFFFFu - n) : 0ull;
                const uint64_t best = wave_max_u64(pk);
                if (lane == 0u && row < a.rows)
                    (void)__hip_atomic_fetch_max(&a.win[(size_t)row * PLH_WIN_ROW + (tile % PLH_WIN_SLOTS) * PLH_WIN_STRIDE],
                                                 (unsigned long long)best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

/* Greedy form, second kernel: one wave per row, lane = slot; the row's token
 * is the lowest id among its largest logits (0xFFFFFFFF - the packed
 * maximum's low half).  Every slot is cleared for the next call. */
__global__ void __launch_bounds__(PSS_WAVE) plh_greedy_reduce_kernel(plh_args a) {
    const uint32_t row = blockIdx.x, lane = threadIdx.x;
    unsigned long long* p = &a.win[(size_t)row * PLH_WIN_ROW + lane * PLH_WIN_STRIDE];
    const uint64_t best = wave_max_u64(*p);
    *p = 0ull;
    if (lane == 0u) {
        const uint32_t tok = 0xFFFFFFFFu - (uint32_t)best;
        a.result[row * PSS_RESULT_SLOTS + a.pass_idx] = tok;
        a.token_ids[row] = tok;
        if (a.do_inc) a.position[row] = a.position[row] + 1u;
    }
}

/* ---------------------------------------------------------------------- */
/* host side                                                               */
/* ---------------------------------------------------------------------- */

static void plh_free(plh_head* h) {
    if (!h) return;
    if (h->an) (void)hipFree(h->an);
    if (h->win) (void)hipFree(h->win);
    if (h->own_stream && h->stream) (void)hipStreamDestroy(h->stream);
    free(h);
}

extern "C" pss_status plh_create(plh_head** out, const void* weight_bt, const float* gamma, uint32_t K, uint32_t V,
                                 uint32_t max_rows, void* hip_stream) {
    if (!out) return PSS_ERR_INVALID_ARG;
    *out = NULL;
    if (!weight_bt || !gamma || max_rows == 0 || V == 0 || K < 8 || K % 8 != 0) return PSS_ERR_INVALID_ARG;
    if (K > PLH_MAX_K || V > PSS_MAX_VOCAB) return PSS_ERR_UNSUPPORTED;
    int dev = 0, ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) return PSS_ERR_NO_DEVICE;
    if (hipGetDevice(&dev) != hipSuccess) return PSS_ERR_NO_DEVICE;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return PSS_ERR_NO_DEVICE;
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return PSS_ERR_NO_DEVICE;

    plh_head* h = (plh_head*)calloc(1, sizeof(plh_head));
    if (!h) return PSS_ERR_ALLOC;
    h->device = dev;
    h->w = (const uint4*)weight_bt;
    h->gamma = gamma;
    h->K = K;
    h->V = V;
    h->max_rows = max_rows;
    h->ntiles = (V + PLH_TILE - 1u) / PLH_TILE;
    if (hip_stream) {
        h->stream = (hipStream_t)hip_stream;
    } else {
        if (hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking) != hipSuccess) {
            free(h);
            return PSS_ERR_HIP;
        }
        h->own_stream = 1;
    }
    if (hipMalloc((void**)&h->an, (size_t)max_rows * K * 4u) != hipSuccess ||
        hipMalloc((void**)&h->win, (size_t)max_rows * PLH_WIN_ROW * 8u) != hipSuccess) {
        plh_free(h);
        return PSS_ERR_ALLOC;
    }
    if (hipMemsetAsync(h->win, 0, (size_t)max_rows * PLH_WIN_ROW * 8u, h->stream) != hipSuccess ||
        hipStreamSynchronize(h->stream) != hipSuccess) {
        plh_free(h);
        return PSS_ERR_HIP;
    }
    *out = h;
    return PSS_OK;
}

extern "C" pss_status plh_destroy(plh_head* h) {
    if (!h) return PSS_ERR_INVALID_ARG;
    (void)hipStreamSynchronize(h->stream);
    plh_free(h);
    return PSS_OK;
}

extern "C" void* plh_stream(plh_head* h) { return h ? (void*)h->stream : NULL; }

/* Rows per weight pass: 1, 2, 4 (3 or 4 rows), or groups of 8 (VALU work per
 * 16-byte block: 8 conversions folded into 8 R fused multiply-adds, still
 * under the block's HBM time at 8 rows; 16 would be VALU-bound). */
static inline int plh_pick_r(uint32_t rows) { return rows == 1u ? 1 : rows == 2u ? 2 : rows <= 4u ? 4 : 8; }

template <bool GREEDY>
static pss_status plh_launch(plh_head* h, const float* x, uint64_t xs, uint32_t rows, plh_args a) {
    hipLaunchKernelGGL(plh_norm_kernel, dim3(rows), dim3(PLH_NORM_NT), 0, h->stream, x, xs, h->gamma, h->an, h->K,
                       GREEDY ? h->win : (unsigned long long*)nullptr);
    const int R = plh_pick_r(rows);
    const dim3 grid(h->ntiles, (rows + (uint32_t)R - 1u) / (uint32_t)R);
    if (R == 1)
        hipLaunchKernelGGL((plh_gemv_kernel<1, GREEDY>), grid, dim3(PLH_NT), 0, h->stream, a, (const float*)h->an);
    else if (R == 2)
        hipLaunchKernelGGL((plh_gemv_kernel<2, GREEDY>), grid, dim3(PLH_NT), 0, h->stream, a, (const float*)h->an);
    else if (R == 4)
        hipLaunchKernelGGL((plh_gemv_kernel<4, GREEDY>), grid, dim3(PLH_NT), 0, h->stream, a, (const float*)h->an);
    else
        hipLaunchKernelGGL((plh_gemv_kernel<8, GREEDY>), grid, dim3(PLH_NT), 0, h->stream, a, (const float*)h->an);
    if (GREEDY) hipLaunchKernelGGL(plh_greedy_reduce_kernel, dim3(rows), dim3(PSS_WAVE), 0, h->stream, a);
    return hipGetLastError() == hipSuccess ? PSS_OK : PSS_ERR_HIP;
}

static plh_args plh_make_args(const plh_head* h, uint32_t rows) {
    plh_args a;
    memset(&a, 0, sizeof(a));
    a.w = h->w;
    a.win = h->win;
    a.K = h->K;
    a.V = h->V;
    a.rows = rows;
    a.ntiles = h->ntiles;
    return a;
}

extern "C" pss_status plh_logits(plh_head* h, const float* x, uint64_t x_stride, uint32_t rows, float* logits,
                                 uint64_t logits_stride) {
    if (!h || !x || !logits || rows == 0 || rows > h->max_rows) return PSS_ERR_INVALID_ARG;
    if (x_stride < h->K || logits_stride < h->V) return PSS_ERR_INVALID_ARG;
    plh_args a = plh_make_args(h, rows);
    a.logits = logits;
    a.lstride = logits_stride;
    return plh_launch<false>(h, x, x_stride, rows, a);
}

extern "C" pss_status plh_greedy(plh_head* h, pss_sampler* s, const float* x, uint64_t x_stride, uint32_t rows,
                                 uint32_t do_increment, uint32_t pass_idx) {
    if (!h || !s || !x || rows == 0 || rows > h->max_rows || rows > s->max_rows) return PSS_ERR_INVALID_ARG;
    if (x_stride < h->K || pass_idx >= PSS_RESULT_SLOTS || s->V != h->V || s->stream != h->stream)
        return PSS_ERR_INVALID_ARG;
    plh_args a = plh_make_args(h, rows);
    a.result = s->d_result;
    a.token_ids = s->d_tokens;
    a.position = s->d_pos;
    a.pass_idx = pass_idx;
    a.do_inc = do_increment ? 1u : 0u;
    return plh_launch<true>(h, x, x_stride, rows, a);
}

extern "C" pss_status plh_transpose_block16(const uint16_t* w_kv, uint16_t* w_bt, uint32_t K, uint32_t V) {
    if (!w_kv || !w_bt || K == 0 || K % 8 != 0 || V == 0) return PSS_ERR_INVALID_ARG;
    for (uint32_t kb = 0; kb < K / 8u; ++kb)
        for (uint32_t n = 0; n < V; ++n)
            for (uint32_t j = 0; j < 8u; ++j)
                w_bt[((size_t)kb * V + n) * 8u + j] = w_kv[(size_t)(8u * kb + j) * V + n];
    return PSS_OK;
}
