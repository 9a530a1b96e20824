/* fst_exact_math.h — canonical scalar math shared bit-for-bit by host and device.
 *
 * Every decision on the verify path that depends on a transcendental (router
 * scores feeding top-k, softmax probabilities feeding rejection sampling) is
 * computed with the functions below.  They use only IEEE-754 binary32
 * operations whose results are fully specified (add, mul, fmaf, correctly
 * rounded division and sqrt, integer bit manipulation), so a gcc host build
 * with -ffp-contract=off and a hipcc gfx950 build produce identical bits.
 * Implicit contraction is disabled for clang below; explicit fmaf() is used
 * wherever a fused operation is wanted.
 *
 * Methods:
 *   exp  : Cody & Waite (1980) range reduction x = n*ln2 + r with a two-part
 *          ln2, then the degree-7 Taylor polynomial of e^r on |r| <= ln2/2
 *          (truncation error < 6e-9 relative), scaled by 2^n through the
 *          exponent field.
 *   log  : x = m*2^e with m in [sqrt(1/2), sqrt(2)), log m = 2*atanh(s),
 *          s = (m-1)/(m+1), odd series to s^13 (error < 1e-10 for |s|<0.172).
 *   Philox-4x32-10 : Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
 *          easy as 1, 2, 3", SC'11 (multipliers 0xD2511F53/0xCD9E8D57, Weyl
 *          key increments 0x9E3779B9/0xBB67AE85, 10 rounds).
 *   bf16 : round-to-nearest-even from binary32, NaN kept quiet.
 */
#ifndef FST_EXACT_MATH_H
#define FST_EXACT_MATH_H

#include <stdint.h>
#include <math.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define FST_HD __host__ __device__ inline
#else
#define FST_HD static inline
#endif

#if defined(__clang__)
#pragma clang fp contract(off)
#endif

FST_HD float fst_bits_f32(uint32_t u) {
    union { uint32_t u; float f; } c; c.u = u; return c.f;
}
FST_HD uint32_t fst_f32_bits(float f) {
    union { uint32_t u; float f; } c; c.f = f; return c.u;
}

/* binary16 -> binary32, exact for every code including subnormals, inf, NaN. */
FST_HD float fst_fp16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0x1fu) return fst_bits_f32(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        /* subnormal: value = m * 2^-24, exact in binary32 */
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return fst_bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

/* binary32 -> bfloat16 bits, round to nearest even. */
FST_HD uint16_t fst_f32_to_bf16(float f) {
    uint32_t u = fst_f32_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t r = 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)((u + r) >> 16);
}
FST_HD float fst_bf16_to_f32(uint16_t b) { return fst_bits_f32((uint32_t)b << 16); }

/* 2^n for integer n in [-126, 127]. */
FST_HD float fst_pow2i(int n) { return fst_bits_f32((uint32_t)(n + 127) << 23); }

/* Written without early returns so that a GPU build evaluates it with
 * selects (no divergent branches); the arithmetic is the same for every x. */
FST_HD float fst_expf(float x) {
    const float HI = 88.72283935546875f, LO = -87.33654022216797f; /* LO: below 2^-126 -> flushed */
    const float LOG2E = 1.44269502162933349609f;
    const float LN2_HI = 0.693145751953125f;       /* 0x3f317200 */
    const float LN2_LO = 1.42860676533018704504e-06f; /* 0x35bfbe8e */
    const float SHIFT = 12582912.0f;               /* 1.5 * 2^23 */
    const float xc = (x > HI) ? HI : ((x < LO) ? LO : x);  /* NaN passes through */
    float t = fmaf(xc, LOG2E, SHIFT);
    float n = t - SHIFT;                           /* round(x*log2e) */
    float r = fmaf(-n, LN2_HI, xc);
    r = fmaf(-n, LN2_LO, r);
    float p = 1.98412698412698412526e-04f;         /* 1/5040 */
    p = fmaf(p, r, 1.38888888888888894189e-03f);   /* 1/720  */
    p = fmaf(p, r, 8.33333333333333321769e-03f);   /* 1/120  */
    p = fmaf(p, r, 4.16666666666666643537e-02f);   /* 1/24   */
    p = fmaf(p, r, 1.66666666666666657415e-01f);   /* 1/6    */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int ni = (n == n) ? (int)n : 0;
    ni = ni > 128 ? 128 : (ni < -127 ? -127 : ni);
    const float big = (p * 2.0f) * fst_pow2i(127);
    const float small = (p * 0.5f) * fst_pow2i(-126);
    const float mid = p * fst_pow2i(ni > 127 ? 127 : (ni < -126 ? -126 : ni));
    float res = (ni > 127) ? big : ((ni < -126) ? small : mid);
    res = (x > HI) ? fst_bits_f32(0x7f800000u) : res;
    res = (x < LO) ? 0.0f : res;
    return (x != x) ? x : res;
}

/* e^x for x <= 0 (a logit minus its row's maximum): fst_expf's operations
 * without its overflow path, so for every x <= 0 (and -inf, and NaN) the
 * result is fst_expf(x) bit for bit: x below LO gives 0, otherwise the
 * exponent n = round(x*log2e) lies in [-126, 0] and the scaling is fst_expf's
 * "mid" product. */
FST_HD float fst_exp_nonpos(float x) {
    const float LO = -87.33654022216797f;
    const float LOG2E = 1.44269502162933349609f;
    const float LN2_HI = 0.693145751953125f;
    const float LN2_LO = 1.42860676533018704504e-06f;
    const float SHIFT = 12582912.0f;
    const float xc = x < LO ? LO : x;  /* NaN passes through */
    float t = fmaf(xc, LOG2E, SHIFT);
    float n = t - SHIFT;
    float r = fmaf(-n, LN2_HI, xc);
    r = fmaf(-n, LN2_LO, r);
    float p = 1.98412698412698412526e-04f;
    p = fmaf(p, r, 1.38888888888888894189e-03f);
    p = fmaf(p, r, 8.33333333333333321769e-03f);
    p = fmaf(p, r, 4.16666666666666643537e-02f);
    p = fmaf(p, r, 1.66666666666666657415e-01f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const int ni = (n == n) ? (int)n : 0;
    const float res = p * fst_pow2i(ni);
    return (x != x) ? x : (x < LO ? 0.0f : res);
}

FST_HD float fst_logf(float x) {
    if (x != x) return x;
    if (x < 0.0f) return fst_bits_f32(0x7fc00000u);
    if (x == 0.0f) return fst_bits_f32(0xff800000u);
    if (x == fst_bits_f32(0x7f800000u)) return x;
    int e = 0;
    if (x < 1.17549435e-38f) { x = x * 16777216.0f; e = -24; }  /* scale subnormals */
    uint32_t u = fst_f32_bits(x);
    e += (int)((u >> 23) & 0xffu) - 127;
    float m = fst_bits_f32((u & 0x007fffffu) | 0x3f800000u);   /* [1,2) */
    if (m > 1.41421353816986083984f) { m = m * 0.5f; e += 1; }
    float s = (m - 1.0f) / (m + 1.0f);
    float z = s * s;
    float q = 0.07692307692307692f;                /* 1/13 */
    q = fmaf(q, z, 0.09090909090909091f);          /* 1/11 */
    q = fmaf(q, z, 0.1111111111111111f);           /* 1/9  */
    q = fmaf(q, z, 0.14285714285714285f);          /* 1/7  */
    q = fmaf(q, z, 0.2f);
    q = fmaf(q, z, 0.3333333333333333f);
    float lm = 2.0f * fmaf(s * z, q, s);            /* 2*(s + s^3*q) */
    const float LN2_HI = 0.693145751953125f;
    const float LN2_LO = 1.42860676533018704504e-06f;
    float fe = (float)e;
    return fmaf(fe, LN2_HI, fmaf(fe, LN2_LO, lm));
}

/* Router score functions.  sigmoid(x) = 1/(1+e^-x).  sqrtsoftplus follows
 * src/fst_engine.cpp:976-983: sp = x > 20 ? x : log(1+e^x), score = sqrt(sp). */
FST_HD float fst_sigmoidf(float x) { return 1.0f / (1.0f + fst_expf(-x)); }
FST_HD float fst_sqrtsoftplusf(float x) {
    float sp = (x > 20.0f) ? x : fst_logf(1.0f + fst_expf(x));
    return sqrtf(sp);
}

/* ---- Philox-4x32-10 ---- */
typedef struct { uint32_t v[4]; } fst_philox_ctr;

FST_HD void fst_mulhilo32(uint32_t a, uint32_t b, uint32_t* hi, uint32_t* lo) {
    uint64_t p = (uint64_t)a * (uint64_t)b;
    *hi = (uint32_t)(p >> 32);
    *lo = (uint32_t)p;
}

FST_HD fst_philox_ctr fst_philox4x32_10(fst_philox_ctr c, uint32_t k0, uint32_t k1) {
    for (int i = 0; i < 10; ++i) {
        uint32_t hi0, lo0, hi1, lo1;
        fst_mulhilo32(0xD2511F53u, c.v[0], &hi0, &lo0);
        fst_mulhilo32(0xCD9E8D57u, c.v[2], &hi1, &lo1);
        fst_philox_ctr n;
        n.v[0] = hi1 ^ c.v[1] ^ k0;
        n.v[1] = lo1;
        n.v[2] = hi0 ^ c.v[3] ^ k1;
        n.v[3] = lo0;
        c = n;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return c;
}

/* 24-bit uniform integer U (u = U / 2^24 in [0,1)) for acceptance sampling.
 * Counter = (position, stream, seq_lo, seq_hi), key = (seed_lo, seed_hi).
 * stream 0: the accept/reject uniform u_i; stream 2: sample_token's draw. */
FST_HD uint32_t fst_uniform24(uint64_t seed, uint64_t seq, uint32_t pos, uint32_t stream) {
    fst_philox_ctr c;
    c.v[0] = pos; c.v[1] = stream; c.v[2] = (uint32_t)seq; c.v[3] = (uint32_t)(seq >> 32);
    fst_philox_ctr r = fst_philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    return r.v[0] >> 8;
}

/* ---- rejection sampling: softmax partials and the exponential race ----
 * e(x | m): the softmax weight of x relative to a maximum m: 0 for x = -inf,
 * exactly 1 at the maximum, fst_expf(x - m) otherwise (callers skip NaN). */
FST_HD float fst_rel_exp(float x, float m) {
    const float ninf = fst_bits_f32(0xff800000u);
    return x == ninf ? 0.0f : (x == m ? 1.0f : fst_exp_nonpos(x - m));
}
/* Merge of two softmax partials (m = maximum, s = sum of e(x | m)):
 * M = max(m1, m2), S = s1*e(m1 | M) + s2*e(m2 | M), two rounded products
 * and one rounded sum (symmetric in its arguments, bit for bit); both
 * empty (-inf) stays (-inf, 0). */
FST_HD void fst_softmax_merge(float* m1, float* s1, float m2, float s2) {
    const float ninf = fst_bits_f32(0xff800000u);
    const float M = *m1 > m2 ? *m1 : m2;
    if (M == ninf) {
        *m1 = ninf;
        *s1 = 0.0f;
        return;
    }
    const float w1 = *m1 == M ? 1.0f : fst_exp_nonpos(*m1 - M);
    const float w2 = m2 == M ? 1.0f : fst_exp_nonpos(m2 - M);
    const float a = *s1 * w1, b = s2 * w2;
    *m1 = M;
    *s1 = a + b;
}
/* Uniform in (0, 1) for element v of the exponential race at position pos:
 * Philox counter (v, 0x52430000 ^ pos, seq_lo, seq_hi), key (seed_lo,
 * seed_hi), first word w; u = (2*(w >> 9) + 1) * 2^-24, exact in binary32
 * (distinct from fst_uniform24's counters, whose second word is < 3). */
FST_HD float fst_race_uniform(uint64_t seed, uint64_t seq, uint32_t pos, uint32_t v) {
    fst_philox_ctr c;
    c.v[0] = v; c.v[1] = 0x52430000u ^ pos; c.v[2] = (uint32_t)seq; c.v[3] = (uint32_t)(seq >> 32);
    fst_philox_ctr r = fst_philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    return (float)(2u * (r.v[0] >> 9) + 1u) * 5.9604644775390625e-8f;
}

/* Fixed-point probability mass: E = floor(exp(l - max) * 2^32), l - max <= 0.
 * exp() <= 1 so E <= 2^32; products with 2^32 are exact (power of two). */
FST_HD uint64_t fst_prob_fixed(float l_minus_max) {
    float e = fst_expf(l_minus_max);
    return (uint64_t)(e * 4294967296.0f);
}

#endif
