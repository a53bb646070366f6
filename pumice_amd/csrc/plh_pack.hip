/*
 * plh_pack.hip - load-time side of the LM head (include/pumice_lmhead.h):
 * the pruned-vocabulary map (pruned-vocab/mapping.npy, read as src/prune.c:32-57
 * loadMapping reads it) and the device kernel that builds the block-transposed
 * fp16 head from the model's lm_head rows, folding into one pass what the
 * reference does on the host in three: the pruning gather of rows mapping[n]
 * (src/prune.c:128-146, fp16 rows re-encoded as bf16), the loader's
 * conversion to fp16 (src/weights.c:520-566, bf16 -> fp32 -> truncating fp16)
 * and transpose_block16 (src/data.c:305-331).
 *
 * plh_pack_kernel: one workgroup per tile of 64 head columns x 32 8-row
 * blocks.  Reads: 32 lanes take 32 consecutive 16-byte blocks of one source
 * row (512 contiguous bytes), converted in registers into an LDS tile; writes:
 * 64 lanes store the 64 columns of one block row (1 KiB contiguous).  HBM-bound
 * byte work: K V 2 bytes read and K V 2 written.
 */
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "pumice_lmhead.h"

#define PLP_TN 64u  /* head columns per tile */
#define PLP_TKB 32u /* 8-row blocks per tile */
#define PLP_NT 256u

enum { PLP_CONV_BF16 = 0, PLP_CONV_FP16_VIA_BF16 = 1, PLP_CONV_FP16 = 2 };

/* Source and head are each touched once: nontemporal loads and stores. */
typedef unsigned int plp_u32x4 __attribute__((ext_vector_type(4)));

/* src/data.c:30-52 float_to_fp16: truncation, no rounding; e < -24 -> signed
 * zero, e <= -15 -> subnormal (mantissa with its hidden bit shifted right by
 * -1 - e), e >= 16 -> signed infinity (NaN included). */
__device__ __forceinline__ uint32_t plp_f2h(float f) {
    const uint32_t b = __float_as_uint(f);
    const uint32_t sign = (b >> 16) & 0x8000u;
    const int e = (int)((b >> 23) & 0xFFu) - 127;
    const uint32_t m = b & 0x7FFFFFu;
    if (e < -24) return sign;
    if (e <= -15) return sign | ((m | 0x800000u) >> (-1 - e));
    if (e >= 16) return sign | 0x7C00u;
    return sign | ((uint32_t)(e + 15) << 10) | (m >> 13);
}

/* src/data.c:194-200 float_to_bf16: add 0x7FFF plus the kept lsb, keep the
 * high half (round to nearest, ties to even; no NaN special case). */
__device__ __forceinline__ uint32_t plp_f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ float plp_bf2f(uint32_t b) { return __uint_as_float(b << 16); }

/* src/data.c:54-81 fp16_to_float: exact, a NaN keeps its payload bits (the
 * hardware conversion would quiet a signalling NaN, and the bf16 rounding
 * that follows in the pruned path depends on every payload bit). */
__device__ __forceinline__ float plp_h2f(uint32_t h) {
    if ((h & 0x7C00u) == 0x7C00u) return __uint_as_float(((h & 0x8000u) << 16) | 0x7F800000u | ((h & 0x3FFu) << 13));
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

__device__ __forceinline__ uint32_t plp_conv(uint32_t raw, int mode) {
    if (mode == PLP_CONV_BF16) return plp_f2h(plp_bf2f(raw));
    if (mode == PLP_CONV_FP16_VIA_BF16) return plp_f2h(plp_bf2f(plp_f2bf(plp_h2f(raw))));
    return plp_f2h(plp_h2f(raw));
}

template <int MODE>
__global__ void __launch_bounds__(PLP_NT) plh_pack_kernel(const uint4* __restrict__ src, uint32_t K,
                                                          const int32_t* __restrict__ map, uint32_t V,
                                                          uint4* __restrict__ out) {
    __shared__ uint4 tile[PLP_TN][PLP_TKB + 1u];
    const uint32_t n0 = blockIdx.x * PLP_TN, kb0 = blockIdx.y * PLP_TKB;
    const uint32_t KB = K >> 3, t = threadIdx.x;
#pragma unroll
    for (uint32_t pass = 0; pass < PLP_TN * PLP_TKB / PLP_NT; ++pass) {
        const uint32_t r = pass * (PLP_NT / PLP_TKB) + t / PLP_TKB, b = t % PLP_TKB;
        const uint32_t n = n0 + r, kb = kb0 + b;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (n < V && kb < KB) {
            const uint32_t row = map ? (uint32_t)map[n] : n;
            const plp_u32x4 q = __builtin_nontemporal_load((const plp_u32x4*)&src[(size_t)row * KB + kb]);
            const uint32_t w[4] = {q.x, q.y, q.z, q.w};
            uint32_t o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                o[i] = plp_conv(w[i] & 0xFFFFu, MODE) | (plp_conv(w[i] >> 16, MODE) << 16);
            v = make_uint4(o[0], o[1], o[2], o[3]);
        }
        tile[r][b] = v;
    }
    __syncthreads();
#pragma unroll
    for (uint32_t pass = 0; pass < PLP_TN * PLP_TKB / PLP_NT; ++pass) {
        const uint32_t b = pass * (PLP_NT / PLP_TN) + t / PLP_TN, r = t % PLP_TN;
        const uint32_t n = n0 + r, kb = kb0 + b;
        if (n < V && kb < KB) {
            const uint4 v = tile[r][b];
            const plp_u32x4 o = {v.x, v.y, v.z, v.w};
            __builtin_nontemporal_store(o, (plp_u32x4*)&out[(size_t)kb * V + n]);
        }
    }
}

extern "C" pss_status plh_pack_head(const void* src, uint32_t src_dtype, uint32_t src_rows, uint32_t K,
                                    const int32_t* mapping, uint32_t V, uint16_t* w_bt, void* hip_stream) {
    if (!src || !w_bt || K < 8 || K % 8 != 0 || V == 0 || src_rows == 0) return PSS_ERR_INVALID_ARG;
    if (src_dtype != PLH_SRC_BF16 && src_dtype != PLH_SRC_FP16) return PSS_ERR_INVALID_ARG;
    if (((uintptr_t)src & 15u) || ((uintptr_t)w_bt & 15u)) return PSS_ERR_INVALID_ARG;
    if (K > PLH_MAX_K || V > PSS_MAX_VOCAB) return PSS_ERR_UNSUPPORTED;
    if (!mapping && src_rows < V) return PSS_ERR_INVALID_ARG;
    if (mapping)
        for (uint32_t i = 0; i < V; ++i) /* src/prune.c:159-161 */
            if (mapping[i] < 0 || (uint32_t)mapping[i] >= src_rows) return PSS_ERR_INVALID_ARG;
    hipStream_t st = (hipStream_t)hip_stream;
    int32_t* dmap = NULL;
    if (mapping) {
        if (hipMalloc((void**)&dmap, (size_t)V * 4u) != hipSuccess) return PSS_ERR_ALLOC;
        if (hipMemcpyAsync(dmap, mapping, (size_t)V * 4u, hipMemcpyHostToDevice, st) != hipSuccess) {
            (void)hipFree(dmap);
            return PSS_ERR_HIP;
        }
    }
    const dim3 grid((V + PLP_TN - 1u) / PLP_TN, (K / 8u + PLP_TKB - 1u) / PLP_TKB);
    const uint4* s4 = (const uint4*)src;
    uint4* o4 = (uint4*)w_bt;
    if (src_dtype == PLH_SRC_BF16)
        hipLaunchKernelGGL(plh_pack_kernel<PLP_CONV_BF16>, grid, dim3(PLP_NT), 0, st, s4, K, dmap, V, o4);
    else if (mapping)
        hipLaunchKernelGGL(plh_pack_kernel<PLP_CONV_FP16_VIA_BF16>, grid, dim3(PLP_NT), 0, st, s4, K, dmap, V, o4);
    else
        hipLaunchKernelGGL(plh_pack_kernel<PLP_CONV_FP16>, grid, dim3(PLP_NT), 0, st, s4, K, dmap, V, o4);
    pss_status r = hipGetLastError() == hipSuccess ? PSS_OK : PSS_ERR_HIP;
    if (hipStreamSynchronize(st) != hipSuccess) r = PSS_ERR_HIP;
    if (dmap) (void)hipFree(dmap);
    return r;
}

/* src/prune.c:32-57: magic "\x93NUMPY", version 1, little-endian 16-bit
 * header length, a header naming '<i4' and 'shape': (count, ...), count ==
 * expected, then count int32 values. */
extern "C" pss_status plh_load_vocab_map(const char* path, uint32_t expected, int32_t* out) {
    if (!path || !out || expected == 0) return PSS_ERR_INVALID_ARG;
    FILE* f = fopen(path, "rb");
    if (!f) return PSS_ERR_INVALID_ARG;
    pss_status r = PSS_ERR_INVALID_ARG;
    unsigned char pre[10];
    char* hdr = NULL;
    do {
        if (fread(pre, 1, 10, f) != 10 || memcmp(pre, "\x93NUMPY", 6) != 0 || pre[6] != 1) break;
        const size_t hl = (size_t)pre[8] | ((size_t)pre[9] << 8);
        hdr = (char*)malloc(hl + 1);
        if (!hdr) {
            r = PSS_ERR_ALLOC;
            break;
        }
        if (fread(hdr, 1, hl, f) != hl) break;
        hdr[hl] = '\0';
        if (!strstr(hdr, "'<i4'")) break;
        const char* shp = strstr(hdr, "'shape':");
        long count = 0;
        if (!shp || sscanf(shp, "'shape': (%ld,", &count) != 1 || count != (long)expected) break;
        if (fread(out, sizeof(int32_t), expected, f) != expected) break;
        r = PSS_OK;
    } while (0);
    free(hdr);
    fclose(f);
    return r;
}
