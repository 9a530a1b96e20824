/* fst_cpu_baseline.c — the CPU baseline of the benchmark (not the checker).
 *
 * The reference engine has no CPU expert path (include/fst_engine.h:326-327:
 * the FFN runs on the NPU only), so the CPU figure next to the GPU one is this
 * port of the same block-verify MoE layer, written for speed on host cores:
 *   router logits h . W_r (src/fst_engine.cpp:936-1061 semantics: sigmoid,
 *   top-k by score, weights renormalised), then per distinct routed expert
 *   and the shared expert the Q4_K SwiGLU FFN (kernels/fst_dequant_q4k_kernel.cc
 *   decode, src/fst_engine.cpp:4160-4194 FFN), then the weighted combine
 *   (:4196-4201, :2851-2852).
 * fp32 throughout: each weight row is decoded once into a float buffer and
 * dotted with every token of its expert (vectorised fp32 reductions), rows
 * spread over OpenMP threads.  Built by the benchmark on the machine it runs
 * on with -O3 -march=native -fopenmp (oracle/build_cpu_baseline.sh).  Its
 * outputs are compared with the fp64 oracle only for sanity (tests); the
 * oracle in fst_oracle.c stays the parity checker.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static float cb_half(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
    uint32_t u;
    if (e == 0) {
        float f = (float)m * (1.0f / 16777216.0f); /* m * 2^-24 */
        return (h >> 15) ? -f : f;
    }
    if (e == 31) u = s | 0x7f800000u | (m << 13);
    else u = s | ((e + 112) << 23) | (m << 13);
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static float cb_bf16(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint16_t cb_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

/* One Q4_K row of K weights (K/256 blocks of 144 B) decoded to floats. */
static void cb_decode_row(const uint8_t* blk, int nb, float* w) {
    for (int b = 0; b < nb; ++b, blk += 144, w += 256) {
        const float d = cb_half((uint16_t)(blk[0] | (blk[1] << 8)));
        const float dmin = cb_half((uint16_t)(blk[2] | (blk[3] << 8)));
        const uint8_t* q = blk + 4;
        const uint8_t* qs = blk + 16;
        for (int j = 0; j < 8; ++j) {
            int sc, m;
            if (j < 4) {
                sc = q[j] & 63;
                m = q[j + 4] & 63;
            } else {
                sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);
                m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
            }
            const float d1 = d * (float)sc, m1 = dmin * (float)m;
            const uint8_t* src = qs + 32 * (j >> 1);
            const int sh = (j & 1) * 4;
            float* dst = w + 32 * j;
#pragma omp simd
            for (int i = 0; i < 32; ++i) dst[i] = d1 * (float)((src[i] >> sh) & 15) - m1;
        }
    }
}

static float cb_dot(const float* a, const float* b, int n) {
    float acc = 0.0f;
#pragma omp simd reduction(+ : acc)
    for (int i = 0; i < n; ++i) acc += a[i] * b[i];
    return acc;
}

/* One expert over Mt token rows x [Mt][hd]: y [Mt][hd] (fp32).  Q4_K packed
 * expert gate|up|down, each [N][K/256] blocks. */
static void cb_expert(const uint8_t* ex, int hd, int inter, const float* x, int Mt, float* act, float* y) {
    const size_t proj = (size_t)inter * (hd / 256) * 144;
    const uint8_t* wg = ex;
    const uint8_t* wu = ex + proj;
    const uint8_t* wd = ex + 2 * proj;
#pragma omp parallel
    {
        float* row = (float*)malloc(sizeof(float) * (size_t)(hd > inter ? hd : inter) * 2);
        float* row2 = row + (hd > inter ? hd : inter);
#pragma omp for schedule(static)
        for (int n = 0; n < inter; ++n) {
            cb_decode_row(wg + (size_t)n * (hd / 256) * 144, hd / 256, row);
            cb_decode_row(wu + (size_t)n * (hd / 256) * 144, hd / 256, row2);
            for (int t = 0; t < Mt; ++t) {
                const float g = cb_dot(row, x + (size_t)t * hd, hd);
                const float u = cb_dot(row2, x + (size_t)t * hd, hd);
                act[(size_t)t * inter + n] = g / (1.0f + expf(-g)) * u;
            }
        }
#pragma omp for schedule(static)
        for (int n = 0; n < hd; ++n) {
            cb_decode_row(wd + (size_t)n * (inter / 256) * 144, inter / 256, row);
            for (int t = 0; t < Mt; ++t) y[(size_t)t * hd + n] = cb_dot(row, act + (size_t)t * inter, inter);
        }
        free(row);
    }
}

void fcb_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* One MoE-layer verify: h [M][hd] bf16, router w_kn [hd][E] bf16, experts[e]
 * the packed Q4_K expert e (e == E: shared).  out [M][hd] bf16, eids [M][tk].
 * Returns the number of distinct routed experts. */
int fcb_moe_step(const uint16_t* h, int M, const uint16_t* w_kn, int E, int tk, const uint8_t* const* experts,
                 int hd, int inter, uint16_t* out, int32_t* eids) {
    float* x = (float*)malloc(sizeof(float) * (size_t)M * hd);
    float* lg = (float*)malloc(sizeof(float) * (size_t)M * E);
    float* wt = (float*)malloc(sizeof(float) * (size_t)M * tk);
    float* acc = (float*)calloc((size_t)M * hd, sizeof(float));
    float* xs = (float*)malloc(sizeof(float) * (size_t)M * hd);
    float* act = (float*)malloc(sizeof(float) * (size_t)M * inter);
    float* y = (float*)malloc(sizeof(float) * (size_t)M * hd);
    for (size_t i = 0; i < (size_t)M * hd; ++i) x[i] = cb_bf16(h[i]);
    /* router: logits[m][e] = sum_k x[m][k] w[k][e], sigmoid scores */
#pragma omp parallel for schedule(static)
    for (int e = 0; e < E; ++e) {
        float col[8192];
        for (int k = 0; k < hd; ++k) col[k] = cb_bf16(w_kn[(size_t)k * E + e]);
        for (int m = 0; m < M; ++m) {
            const float v = cb_dot(col, x + (size_t)m * hd, hd);
            lg[(size_t)m * E + e] = 1.0f / (1.0f + expf(-v));
        }
    }
    for (int m = 0; m < M; ++m) {
        float* row = lg + (size_t)m * E;
        float sum = 0.0f;
        for (int j = 0; j < tk; ++j) {
            int best = -1;
            for (int e = 0; e < E; ++e)
                if (row[e] >= 0.0f && (best < 0 || row[e] > row[best])) best = e;
            eids[m * tk + j] = best;
            wt[m * tk + j] = row[best];
            sum += row[best];
            row[best] = -1.0f;
        }
        for (int j = 0; j < tk; ++j) wt[m * tk + j] *= 1.0f / (sum + 1e-12f);
    }
    /* routed experts, each over the tokens that chose it */
    int distinct = 0;
    for (int e = 0; e <= E; ++e) {
        int toks[64], slot[64], n = 0;
        for (int m = 0; m < M; ++m) {
            if (e == E) {
                toks[n] = m;
                slot[n++] = -1;
                continue;
            }
            for (int j = 0; j < tk; ++j)
                if (eids[m * tk + j] == e) {
                    toks[n] = m;
                    slot[n++] = j;
                    break;
                }
        }
        if (!n) continue;
        if (e < E) ++distinct;
        for (int i = 0; i < n; ++i) memcpy(xs + (size_t)i * hd, x + (size_t)toks[i] * hd, sizeof(float) * hd);
        cb_expert(experts[e], hd, inter, xs, n, act, y);
        for (int i = 0; i < n; ++i) {
            const float w = slot[i] < 0 ? 1.0f : wt[toks[i] * tk + slot[i]];
            float* a = acc + (size_t)toks[i] * hd;
            const float* yy = y + (size_t)i * hd;
            for (int k = 0; k < hd; ++k) a[k] += w * yy[k];
        }
    }
    for (size_t i = 0; i < (size_t)M * hd; ++i) out[i] = cb_to_bf16(acc[i]);
    free(x);
    free(lg);
    free(wt);
    free(acc);
    free(xs);
    free(act);
    free(y);
    return distinct;
}
