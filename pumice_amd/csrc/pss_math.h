/*
 * pss_math.h - deterministic arithmetic shared by the HIP sampler kernels and
 * the host-side C code.
 *
 * Every function here is built only from IEEE-754 binary32 operations that are
 * correctly rounded on both x86-64 (SSE, no x87 excess precision) and gfx950
 * (v_mul/v_add/v_fma/v_rndne with f32 denormals enabled): +, -, *, fmaf, rintf,
 * exact power-of-two scaling and integer operations.  Compiled with
 * -ffp-contract=off on both sides, so a value computed by the GPU and by the CPU
 * is bit-identical.  That is what lets token ids and candidate sets match
 * exactly between the GPU sampler and a CPU restatement of it.
 *
 * Contents
 *   pss_exp       exp(x) in binary32: Cody-Waite reduction by ln2 plus the
 *                 degree-7 Taylor polynomial of e^r on |r| <= ln2/2, evaluated
 *                 by Horner with explicit fma.  Error <= 2 ulp for x in
 *                 [-104, 0]; subnormal results are produced (no flush).
 *   pss_key       order-preserving map float -> uint32 (total order equal to
 *                 IEEE order on canonical values).
 *   pss_canon     canonical transformed logit: NaN -> -inf, -0 -> +0.
 *   pss_fixq      fixed-point mass q = trunc(p * 2^45); sums of up to 2^18 such
 *                 masses stay below 2^63, so any reduction order gives the
 *                 same bits.
 *   pss_xorshift32  Marsaglia (2003) "Xorshift RNGs", triple (13, 17, 5); the
 *                 generator the reference sampler advances per draw
 *                 (shader/Utility/ArgMax-Reduce.comp:56-61).
 *   pss_philox4x32_10  Salmon, Moraes, Dror, Shaw, "Parallel random numbers:
 *                 as easy as 1, 2, 3" (SC'11), Philox-4x32 with 10 rounds.
 */
#ifndef PSS_MATH_H
#define PSS_MATH_H

#include <stdint.h>

#if defined(__HIPCC__)
#define PSS_HD __host__ __device__ static inline
#else
#define PSS_HD static inline
#endif

#define PSS_FIX_SHIFT 45
#define PSS_SENTINEL 0xFFFFFFFFu
#define PSS_XORSHIFT_ZERO_SEED 0x9E3779B9u

PSS_HD uint32_t pss_f2u(float f) {
    uint32_t u;
    __builtin_memcpy(&u, &f, sizeof u);
    return u;
}

PSS_HD float pss_u2f(uint32_t u) {
    float f;
    __builtin_memcpy(&f, &u, sizeof f);
    return f;
}

/* 2^n as a binary32 for n in [-126, 127]. */
PSS_HD float pss_pow2i(int n) { return pss_u2f((uint32_t)(n + 127) << 23); }

/*
 * exp(x) for binary32 x.  Range used by the sampler: x = t - tmax <= 0.
 *   n = rint(x * log2e), r = x - n*ln2 (two fma steps, ln2 split hi/lo),
 *   e^r = 1 + r + r^2/2! + ... + r^7/7!   (truncation error < 6e-9 relative),
 *   result = e^r * 2^n, scaled in two exact steps when 2^n is subnormal so the
 *   only rounding of a subnormal result is the final multiply.
 */
/* exp(x + xlo) for a head x and a small tail |xlo| <= ulp(x)/2: the tail is
 * added to the reduced argument, so exp of an exact two-float difference is
 * as accurate as exp of a single float. */
PSS_HD float pss_exp2f(float x, float xlo) {
    if (!(x == x)) return x;                 /* NaN in, NaN out */
    if (x < -104.0f) return 0.0f;            /* below half the smallest subnormal */
    if (x > 88.72283935546875f) return pss_u2f(0x7F800000u);
    const float log2e = 0x1.715476p+0f;
    const float ln2_hi = 0x1.62e430p-1f;
    const float ln2_lo = -0x1.05c610p-29f;
    float n = __builtin_rintf(x * log2e);
    float r = __builtin_fmaf(n, -ln2_hi, x);
    r = __builtin_fmaf(n, -ln2_lo, r);
    r = r + xlo;
    /* e^r = 1 + s, s = r + r^2 * P(r), P(r) = 1/2! + r/3! + ... + r^5/7!.
     * s is accurate to far below ulp(1), so the value is set by the final
     * rounding of 1 + s, which is monotone in s. */
    float P = 0x1.a01a02p-13f;                 /* 1/7! */
    P = __builtin_fmaf(P, r, 0x1.6c16c2p-10f); /* 1/6! */
    P = __builtin_fmaf(P, r, 0x1.111112p-7f);  /* 1/5! */
    P = __builtin_fmaf(P, r, 0x1.555556p-5f);  /* 1/4! */
    P = __builtin_fmaf(P, r, 0x1.555556p-3f);  /* 1/3! */
    P = __builtin_fmaf(P, r, 0x1.0p-1f);       /* 1/2! */
    float s = __builtin_fmaf(r * r, P, r);
    float p = 1.0f + s;
    int ni = (int)n;
    if (ni < -126) {
        /* 2^n subnormal: (p * 2^(n+64)) is exact and normal, then one rounding. */
        return (p * pss_pow2i(ni + 64)) * 0x1.0p-64f;
    }
    if (ni > 127) return (p * pss_pow2i(ni - 1)) * 2.0f;
    return p * pss_pow2i(ni);
}

PSS_HD float pss_exp(float x) { return pss_exp2f(x, 0.0f); }

/* Canonical transformed logit: NaN -> -inf, -0 -> +0 (adding +0 maps -0 to +0
 * under round-to-nearest and leaves every other value unchanged). */
PSS_HD float pss_canon(float t) {
    if (!(t == t)) return pss_u2f(0xFF800000u);
    return t + 0.0f;
}

/* Order-preserving key: a < b (IEEE, canonical values) <=> key(a) < key(b). */
PSS_HD uint32_t pss_key(float t) {
    uint32_t b = pss_f2u(t);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

PSS_HD float pss_unkey(uint32_t k) {
    return pss_u2f((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

/* Probability of a canonical value t given the row maximum tmax:
 * exp(t - tmax) with the difference taken exactly as hi + lo (Knuth's
 * TwoSum), so a far-tail p keeps full binary32 accuracy.  Equal values
 * (including tmax = +-inf) get exactly 1. */
PSS_HD float pss_prob(float t, float tmax) {
    if (t == tmax) return 1.0f;
    const float b = -tmax;
    const float hi = t + b;
    if (!(hi >= -104.0f)) return 0.0f;       /* also t = -inf or tmax = +inf */
    const float a1 = hi - b;
    const float b1 = hi - a1;
    const float lo = (t - a1) + (b - b1);
    return pss_exp2f(hi, lo);
}

/* Fixed-point mass: p in [0, 1] -> trunc(p * 2^45).  p * 2^45 is exact. */
PSS_HD uint64_t pss_fixq(float p) { return (uint64_t)(p * 0x1.0p45f); }

/*
 * Natural log of a finite binary64 x >= 2^-1022 (the scoring mode takes it of
 * Z in [1, 2^18]), the same bits on the CPU and the GPU: plain IEEE adds,
 * multiplies and one division, no fused operations.  The reduction of
 * fdlibm's e_log.c (Sun Microsystems, 1993): x = (1 + f) * 2^k with 1 + f in
 * [sqrt(1/2), sqrt(2)), s = f / (2 + f), log(1 + f) = f - (hfsq - s (hfsq +
 * R)) with hfsq = f^2 / 2 and R = 2 atanh(s) / s - 2 = z (2/3 + 2/5 z + ...)
 * (z = s^2 <= 0.0295), here the Taylor series through z^12 instead of
 * fdlibm's minimax polynomial; ln2 split hi + lo (hi has 36 significant bits,
 * so k * hi is exact for |k| < 2^17).  Under one unit in the last place.
 */
PSS_HD double pss_log64(double x) {
    uint64_t b;
    __builtin_memcpy(&b, &x, sizeof b);
    int k = (int)((b >> 52) & 0x7FFu) - 1022; /* x = m * 2^k, m in [0.5, 1) */
    b = (b & 0x000FFFFFFFFFFFFFull) | 0x3FE0000000000000ull;
    double m;
    __builtin_memcpy(&m, &b, sizeof m);
    if (m < 0x1.6a09e667f3bcdp-1) { /* sqrt(1/2) */
        m = m * 2.0;
        k = k - 1;
    }
    const double f = m - 1.0;
    const double s = f / (2.0 + f);
    const double z = s * s;
    double R = 2.0 / 25.0;
    R = R * z + 2.0 / 23.0;
    R = R * z + 2.0 / 21.0;
    R = R * z + 2.0 / 19.0;
    R = R * z + 2.0 / 17.0;
    R = R * z + 2.0 / 15.0;
    R = R * z + 2.0 / 13.0;
    R = R * z + 2.0 / 11.0;
    R = R * z + 2.0 / 9.0;
    R = R * z + 2.0 / 7.0;
    R = R * z + 2.0 / 5.0;
    R = R * z + 2.0 / 3.0;
    R = R * z;
    const double hfsq = 0.5 * f * f;
    const double ln2_hi = 0x1.62e42fefap-1;      /* 36 significant bits */
    const double ln2_lo = 0x1.cf79abc9e3b3ap-40; /* ln2 - ln2_hi */
    const double dk = (double)k;
    return dk * ln2_hi - ((hfsq - (s * (hfsq + R) + dk * ln2_lo)) - f);
}

/*
 * Scoring (ArgMax-Reduce.comp mode 2, :169-214): the negative log-likelihood
 * of `lt` under the row's raw logits, log(Z) + gmax - lt, from the exact
 * fixed-point mass Zq = sum fixq(exp(t - gmax)) (Z = Zq * 2^-45), evaluated in
 * binary64 and rounded once to binary32.
 */
PSS_HD float pss_score_nll(uint64_t Zq, float gmax, float lt) {
    const double Z = (double)Zq * 0x1.0p-45;
    return (float)((pss_log64(Z) + (double)gmax) - (double)lt);
}

PSS_HD uint32_t pss_xorshift32(uint32_t x) {
    x ^= x << 13;
    x ^= x >> 17;
    x ^= x << 5;
    return x;
}

/* 64x64 -> high 64 bits of the 128-bit product, portable integer code. */
PSS_HD uint64_t pss_mulhi64(uint64_t a, uint64_t b) {
    uint64_t a0 = a & 0xFFFFFFFFu, a1 = a >> 32;
    uint64_t b0 = b & 0xFFFFFFFFu, b1 = b >> 32;
    uint64_t p00 = a0 * b0, p01 = a0 * b1, p10 = a1 * b0, p11 = a1 * b1;
    uint64_t mid = (p00 >> 32) + (p01 & 0xFFFFFFFFu) + (p10 & 0xFFFFFFFFu);
    return p11 + (p01 >> 32) + (p10 >> 32) + (mid >> 32);
}

/*
 * Top-p mass threshold: ceil(topP * zk) computed exactly, for 0 < topP < 1.
 * topP = m * 2^-s with m the 24-bit significand; ceil(m * zk / 2^s) evaluated
 * on the 128-bit product.  A prefix mass `acc` (integer) satisfies
 * acc >= topP * zk  <=>  acc >= pss_topp_need(topP, zk).
 */
PSS_HD uint64_t pss_topp_need(float topP, uint64_t zk) {
    uint32_t b = pss_f2u(topP);
    uint32_t e = (b >> 23) & 0xFFu;
    uint64_t m = (b & 0x7FFFFFu) | (e ? 0x800000u : 0u);
    int s = (e ? (int)(150 - (int)e) : 149);  /* topP = m * 2^-s */
    uint64_t lo = m * zk;                      /* low 64 bits of the product */
    uint64_t hi = pss_mulhi64(m, zk);
    if (s >= 128) return (lo | hi) ? 1u : 0u;
    uint64_t q_lo, q_hi, rem;
    if (s >= 64) {
        q_lo = hi >> (s - 64);
        q_hi = 0;
        rem = lo | (s > 64 ? (hi & ((1ull << (s - 64)) - 1)) : 0);
    } else if (s == 0) {
        return lo; /* not reached for topP < 1 */
    } else {
        q_lo = (lo >> s) | (hi << (64 - s));
        q_hi = hi >> s;
        rem = lo & ((1ull << s) - 1);
    }
    (void)q_hi; /* zero: topP < 1 keeps the quotient below zk < 2^63 */
    return q_lo + (rem ? 1u : 0u);
}

/*
 * Draw target: floor(u24 * z / 2^24) for a 24-bit uniform u24 = k and kept mass
 * z.  The drawn token is the first kept id (ascending) whose cumulative mass c
 * satisfies c > target, which is exactly c > (k / 2^24) * z.
 */
PSS_HD uint64_t pss_draw_target(uint32_t u24, uint64_t z) {
    uint64_t lo = (uint64_t)u24 * z;
    uint64_t hi = pss_mulhi64((uint64_t)u24, z);
    return (lo >> 24) | (hi << 40);
}

typedef struct {
    uint32_t v[4];
} pss_u32x4;

PSS_HD void pss_mulhilo32(uint32_t a, uint32_t b, uint32_t* hi, uint32_t* lo) {
    uint64_t p = (uint64_t)a * (uint64_t)b;
    *hi = (uint32_t)(p >> 32);
    *lo = (uint32_t)p;
}

PSS_HD pss_u32x4 pss_philox4x32_10(pss_u32x4 ctr, uint32_t k0, uint32_t k1) {
    const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
    const uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
    for (int r = 0; r < 10; ++r) {
        uint32_t hi0, lo0, hi1, lo1;
        pss_mulhilo32(M0, ctr.v[0], &hi0, &lo0);
        pss_mulhilo32(M1, ctr.v[2], &hi1, &lo1);
        pss_u32x4 n;
        n.v[0] = hi1 ^ ctr.v[1] ^ k0;
        n.v[1] = lo1;
        n.v[2] = hi0 ^ ctr.v[3] ^ k1;
        n.v[3] = lo0;
        ctr = n;
        k0 += W0;
        k1 += W1;
    }
    return ctr;
}

/* fp16 (IEEE binary16) bits -> binary32, exact (integer-only, subnormals kept). */
PSS_HD float pss_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0x1Fu) return pss_u2f(sign | 0x7F800000u | (m << 13));
    if (e == 0) {
        if (m == 0) return pss_u2f(sign);
        /* subnormal half: m * 2^-24, exact in binary32 */
        float v = (float)m * 0x1.0p-24f;
        return sign ? -v : v;
    }
    return pss_u2f(sign | ((e + 112u) << 23) | (m << 13));
}

#endif /* PSS_MATH_H */
