/* fst_oracle.c — CPU oracle for the DSpark verify hot path.
 *
 * TEST INFRASTRUCTURE ONLY: this is the checker used by tests/, smoke() and
 * the cpu_baseline leg of bench.py.  The product library never links it.
 *
 * Built with: gcc -O2 -fopenmp -ffp-contract=off -shared -fPIC (oracle/build.sh).
 * -ffp-contract=off matters: the canonical router sum and the exact-math
 * functions must not be re-associated or fused by the compiler.
 *
 * Pins (what fixes each function independently of this code; see tests/):
 *   fo_fp16_to_f32      exhaustive over all 65,536 codes vs numpy.float16.
 *   fo_q4k_dequant      hand-built blocks (impulses, all scale/min patterns)
 *                       vs closed form d*sc*q - dmin*m; ggml layout known
 *                       answers; random blocks vs an independent numpy decode.
 *   fo_mxfp4_dequant    closed form LUT[nib]*2^(e-127), e in {0,255} -> 0.
 *   fo_expert_ffn       ones@ones = K and A@I known answers through the
 *                       projections; wrong-transpose discrimination; numpy
 *                       float64 restatement on small shapes.
 *   fo_router           brute-force tie/bias/hash cases; logits vs float64 sum
 *                       (within fp32 error); top-k vs numpy lexsort.
 *   fo_accept_greedy    planted accepted lengths 0..k, argmax ties and NaN.
 *   fo_accept_stochastic closed forms (p = q accepts every draft; q(x) = 0
 *                       accepts iff p(x) > 0; p(x) = 0 always rejects; a
 *                       residual with one positive entry draws it), row
 *                       statistics vs float64 softmax, the decision against
 *                       a float64 u < p/q away from ties, and chi-square tests
 *                       of the accept rate min(1, p/q) and of the drawn
 *                       tokens against norm(max(0, p - q)) and p; Philox
 *                       known-answer vectors from Salmon et al.
 */
#include "fst_oracle.h"
#include "../include/fst_exact_math.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 0;
void fo_set_threads(int n) { g_threads = n; }
int fo_get_threads(void) {
#ifdef _OPENMP
    return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
    return 1;
#endif
}
#ifdef _OPENMP
#define FO_NT fo_get_threads()
#endif

float fo_fp16_to_f32(uint16_t h) { return fst_fp16_to_f32(h); }
uint16_t fo_f32_to_bf16(float f) { return fst_f32_to_bf16(f); }
float fo_expf(float x) { return fst_expf(x); }
/* fst_exp_nonpos over n values (for the bit-for-bit check against fst_expf). */
void fo_exp_nonpos_n(const float* x, int n, float* out) {
    for (int i = 0; i < n; ++i) out[i] = fst_exp_nonpos(x[i]);
}
void fo_expf_n(const float* x, int n, float* out) {
    for (int i = 0; i < n; ++i) out[i] = fst_expf(x[i]);
}
float fo_logf(float x) { return fst_logf(x); }
float fo_sigmoidf(float x) { return fst_sigmoidf(x); }
float fo_sqrtsoftplusf(float x) { return fst_sqrtsoftplusf(x); }
void fo_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    fst_philox_ctr c;
    for (int i = 0; i < 4; ++i) c.v[i] = ctr[i];
    fst_philox_ctr r = fst_philox4x32_10(c, key[0], key[1]);
    for (int i = 0; i < 4; ++i) out[i] = r.v[i];
}
uint32_t fo_uniform24(uint64_t seed, uint64_t seq, uint32_t pos, uint32_t stream) {
    return fst_uniform24(seed, seq, pos, stream);
}

/* ------------------------------------------------------------------ codecs */

/* kernels/fst_dequant_q4k_kernel.cc:12-20 (get_scale_min_k4). */
void fo_q4k_scale_min(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* kernels/fst_dequant_q4k_kernel.cc:40-100 (dequant_q4k_block): block of 144 B,
 * d = fp16 @0, dmin = fp16 @2, scales[12] @4, qs[128] @16.  qs[32g+i] low
 * nibble -> element 64g+i (sub-block 2g), high nibble -> 64g+32+i (2g+1).
 * Value = d*sc*q - dmin*m computed in binary32 (d*sc, (d*sc)*q and dmin*m are
 * exact products; one rounding in the subtraction).  The fp16 decode is the
 * correct IEEE one (the reference's decoder at :22-38 mis-decodes subnormals). */
int fo_q4k_dequant(const uint8_t* blocks, size_t nblocks, float* out) {
#pragma omp parallel for num_threads(FO_NT) schedule(static)
    for (long long b = 0; b < (long long)nblocks; ++b) {
        const uint8_t* blk = blocks + (size_t)b * 144;
        float* dst = out + (size_t)b * 256;
        float d = fst_fp16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        float dmin = fst_fp16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
        const uint8_t* sc = blk + 4;
        const uint8_t* qs = blk + 16;
        for (int j = 0; j < 8; ++j) {
            uint8_t s, m;
            fo_q4k_scale_min(j, sc, &s, &m);
            float d1 = d * (float)s;
            float m1 = dmin * (float)m;
            int g = j >> 1, hi = j & 1;
            for (int i = 0; i < 32; ++i) {
                uint8_t byte = qs[32 * g + i];
                int q = hi ? (byte >> 4) : (byte & 0x0F);
                dst[32 * j + i] = d1 * (float)q - m1;
            }
        }
    }
    return 0;
}

/* kernels/fst_dequant_v4_vectorized_kernel.cc:19-37,60-80 and
 * scripts/fst_converter.py:449-482: 17-byte block = e8m0 scale byte + 16
 * bytes of nibbles (low nibble = even element).  Value = LUT[nib]*2^(e-127);
 * e = 0 or 255 decode to 0 as in the kernel (the converter's python decode
 * maps them differently; the engine runs the kernel). */
static const float FO_FP4_LUT[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                                     0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};
int fo_mxfp4_dequant(const uint8_t* blocks, size_t nblocks, float* out) {
#pragma omp parallel for num_threads(FO_NT) schedule(static)
    for (long long b = 0; b < (long long)nblocks; ++b) {
        const uint8_t* blk = blocks + (size_t)b * 17;
        float* dst = out + (size_t)b * 32;
        int e = blk[0];
        float s = (e == 0 || e == 255) ? 0.0f : ldexpf(1.0f, e - 127);
        for (int i = 0; i < 16; ++i) {
            uint8_t byte = blk[1 + i];
            dst[2 * i] = FO_FP4_LUT[byte & 15] * s;
            dst[2 * i + 1] = FO_FP4_LUT[byte >> 4] * s;
        }
    }
    return 0;
}

/* --------------------------------------------------------------------- FFN */

/* src/fst_engine.cpp:4160-4194 (FST_FFN_AUDIT fp32 reference):
 * g = h.Wg^T, u = h.Wu^T accumulated in double, act = (g/(1+exp(-g)))*u in
 * float, y = act.Wd^T accumulated in double.  Orientation A.B^T with B[N][K]
 * (scripts/fst_validate_gemms.py:174).  Optional SwiGLU clamp as in
 * scripts/hf_gen_ref.py:475-484 (gate <= lim, up in [-lim, lim]). */
void fo_expert_ffn_f32(const float* wg, const float* wu, const float* wd, int hd, int inter,
                       const uint16_t* h, int M, float swiglu_limit, float* y) {
    float* act = (float*)malloc(sizeof(float) * (size_t)M * inter);
    float* hf = (float*)malloc(sizeof(float) * (size_t)M * hd);
    for (size_t i = 0; i < (size_t)M * hd; ++i) hf[i] = fst_bf16_to_f32(h[i]);
#pragma omp parallel for num_threads(FO_NT) schedule(static)
    for (int n = 0; n < inter; ++n) {
        const float* rg = wg + (size_t)n * hd;
        const float* ru = wu + (size_t)n * hd;
        for (int m = 0; m < M; ++m) {
            const float* x = hf + (size_t)m * hd;
            double g = 0.0, u = 0.0;
            for (int k = 0; k < hd; ++k) {
                g += (double)x[k] * (double)rg[k];
                u += (double)x[k] * (double)ru[k];
            }
            float gf = (float)g, uf = (float)u;
            if (swiglu_limit > 0.0f) {
                if (gf > swiglu_limit) gf = swiglu_limit;
                if (uf > swiglu_limit) uf = swiglu_limit;
                if (uf < -swiglu_limit) uf = -swiglu_limit;
            }
            act[(size_t)m * inter + n] = (gf / (1.0f + expf(-gf))) * uf;
        }
    }
#pragma omp parallel for num_threads(FO_NT) schedule(static)
    for (int d = 0; d < hd; ++d) {
        const float* rd = wd + (size_t)d * inter;
        for (int m = 0; m < M; ++m) {
            const float* a = act + (size_t)m * inter;
            double s = 0.0;
            for (int k = 0; k < inter; ++k) s += (double)a[k] * (double)rd[k];
            y[(size_t)m * hd + d] = (float)s;
        }
    }
    free(act);
    free(hf);
}

int fo_expert_ffn(int codec, const uint8_t* expert, int hd, int inter,
                  const uint16_t* h, int M, float swiglu_limit, float* y) {
    size_t n_gu = (size_t)inter * hd;
    float* wg = (float*)malloc(sizeof(float) * n_gu);
    float* wu = (float*)malloc(sizeof(float) * n_gu);
    float* wd = (float*)malloc(sizeof(float) * n_gu);
    if (!wg || !wu || !wd) { free(wg); free(wu); free(wd); return 2; }
    if (codec == 0) {
        if (hd % 256 || inter % 256) { free(wg); free(wu); free(wd); return 1; }
        size_t nb = n_gu / 256, bytes = nb * 144;
        fo_q4k_dequant(expert, nb, wg);
        fo_q4k_dequant(expert + bytes, nb, wu);
        fo_q4k_dequant(expert + 2 * bytes, nb, wd);
    } else if (codec == 1) {
        if (hd % 32 || inter % 32) { free(wg); free(wu); free(wd); return 1; }
        size_t nb = n_gu / 32, bytes = nb * 17;
        fo_mxfp4_dequant(expert, nb, wg);
        fo_mxfp4_dequant(expert + bytes, nb, wu);
        fo_mxfp4_dequant(expert + 2 * bytes, nb, wd);
    } else {
        free(wg); free(wu); free(wd);
        return 1;
    }
    fo_expert_ffn_f32(wg, wu, wd, hd, inter, h, M, swiglu_limit, y);
    free(wg); free(wu); free(wd);
    return 0;
}

/* ------------------------------------------------------------------ router */

/* Logits of src/fst_engine.cpp:936-960 (h[M,K] . W[K,N], bf16 inputs).  The
 * reference leaves the fp32 summation order to the NPU; this build fixes one:
 * bf16*bf16 products are exact in fp32, each of 64 partials is a sequential
 * fmaf chain over a contiguous K/64 chunk, and the partials are combined by a
 * halving tree p[j] += p[j+off] for off = 32,16,8,4,2,1. */
void fo_router_logits(const uint16_t* h, const uint16_t* w_kn, int M, int K, int N, float* logits) {
    int chunk = K / 64;
#pragma omp parallel for num_threads(FO_NT) schedule(static)
    for (int e = 0; e < N; ++e) {
        for (int m = 0; m < M; ++m) {
            float p[64];
            for (int j = 0; j < 64; ++j) {
                float acc = 0.0f;
                for (int i = 0; i < chunk; ++i) {
                    int k = j * chunk + i;
                    acc = fmaf(fst_bf16_to_f32(h[(size_t)m * K + k]),
                               fst_bf16_to_f32(w_kn[(size_t)k * N + e]), acc);
                }
                p[j] = acc;
            }
            for (int off = 32; off >= 1; off >>= 1)
                for (int j = 0; j < off; ++j) p[j] = p[j] + p[j + off];
            logits[(size_t)m * N + e] = p[0];
        }
    }
}

/* Selection and weights: src/fst_engine.cpp:974-1061.  score = sigmoid or
 * sqrt(softplus) of the logit (optionally rounded to bf16 first, as the NPU
 * GEMM returns bf16), top-k by score + bias with ties broken toward the lower
 * expert id (partial_sort leaves ties unspecified), weights = unbiased scores
 * of the chosen experts, w = v * (1/(sum+1e-12)) * route_scale.  NaN scores
 * are never selected ahead of a number.  Hash rows (tid2eid, :1015-1021)
 * replace the selection when given. */
int fo_router(const uint16_t* h, const uint16_t* w_kn, const float* bias, int M, int K, int N,
              int top_k, int score_func, float route_scale, int round_logits_bf16,
              const int32_t* hash_row_eids, int32_t* eids, float* wts, float* logits_out) {
    if (K % 64 || top_k <= 0 || top_k > N || top_k > 64) return 1;
    float* lg = (float*)malloc(sizeof(float) * (size_t)M * N);
    fo_router_logits(h, w_kn, M, K, N, lg);
    for (int m = 0; m < M; ++m) {
        float* row = lg + (size_t)m * N;
        float score[1024], sel[1024];
        char used[1024];
        if (N > 1024) { free(lg); return 1; }
        for (int e = 0; e < N; ++e) {
            float x = row[e];
            if (round_logits_bf16) x = fst_bf16_to_f32(fst_f32_to_bf16(x));
            row[e] = x;
            score[e] = score_func == 0 ? fst_sigmoidf(x) : fst_sqrtsoftplusf(x);
            sel[e] = score[e] + (bias ? bias[e] : 0.0f);
            used[e] = 0;
        }
        int idx[64];
        if (hash_row_eids) {
            for (int k = 0; k < top_k; ++k) idx[k] = hash_row_eids[(size_t)m * top_k + k];
        } else {
            for (int k = 0; k < top_k; ++k) {
                int best = -1;
                for (int e = 0; e < N; ++e) {
                    if (used[e]) continue;
                    if (best < 0) { best = e; continue; }
                    float a = sel[e], b = sel[best];
                    int better;
                    if (a != a) better = 0;
                    else if (b != b) better = 1;
                    else better = a > b;
                    if (better) best = e;
                }
                used[best] = 1;
                idx[k] = best;
            }
        }
        float sum = 0.0f;
        for (int k = 0; k < top_k; ++k) {
            if (idx[k] < 0 || idx[k] >= N) { free(lg); return 1; }
            sum += score[idx[k]];
        }
        float inv = 1.0f / (sum + 1e-12f);
        for (int k = 0; k < top_k; ++k) {
            eids[(size_t)m * top_k + k] = idx[k];
            wts[(size_t)m * top_k + k] = score[idx[k]] * inv * route_scale;
        }
    }
    if (logits_out) memcpy(logits_out, lg, sizeof(float) * (size_t)M * N);
    free(lg);
    return 0;
}

/* ----------------------------------------------------------------- combine */

/* src/fst_engine.cpp:4196-4201 (acc += w * down_out, fp32) and :2851-2852
 * (routed + shared).  The reference truncates each stage to bf16; this build
 * keeps fp32 to the end and rounds once (RNE). */
void fo_combine(const float* y_routed, const float* y_shared, const float* wts,
                int M, int tk, int hd, uint16_t* out, float* out_f32) {
    for (int m = 0; m < M; ++m)
        for (int d = 0; d < hd; ++d) {
            float acc = 0.0f;
            for (int j = 0; j < tk; ++j)
                acc = acc + wts[(size_t)m * tk + j] * y_routed[((size_t)m * tk + j) * hd + d];
            if (y_shared) acc = acc + y_shared[(size_t)m * hd + d];
            if (out) out[(size_t)m * hd + d] = fst_f32_to_bf16(acc);
            if (out_f32) out_f32[(size_t)m * hd + d] = acc;
        }
}

/* -------------------------------------------------------------- acceptance */

/* src/fst_engine.cpp:6039-6042: int argmax = 0; for v>=1: if (l[v] > max)
 * update.  First maximum wins; NaN never compares greater, so a NaN at index
 * 0 pins the result to 0 and NaNs elsewhere are skipped. */
int fo_argmax(const float* l, int V) {
    int best = 0;
    float mx = l[0];
    for (int v = 1; v < V; ++v)
        if (l[v] > mx) { mx = l[v]; best = v; }
    return best;
}

/* src/fst_engine.cpp:6021-6063: n_acc = longest prefix with pred[i]==draft[i]
 * (i < k), bonus = pred[n_acc]; emitted = draft[0..n_acc) + bonus. */
int fo_accept_greedy(const float* target, int k, int V, const int32_t* draft,
                     int32_t* n_acc, int32_t* tokens) {
    int n = 0;
    while (n < k && fo_argmax(target + (size_t)n * V, V) == draft[n]) ++n;
    for (int i = 0; i < n; ++i) tokens[i] = draft[i];
    tokens[n] = fo_argmax(target + (size_t)n * V, V);
    *n_acc = n;
    return 0;
}

typedef unsigned __int128 u128;

/* Fixed-point softmax row: E[v] = floor(exp(l[v]*inv_t - max)*2^32). */
static uint64_t fo_softmax_fixed(const float* row, int V, float inv_t, uint64_t* E) {
    float mx = -INFINITY;
    int any = 0;
    for (int v = 0; v < V; ++v) {
        float l = row[v] * inv_t;
        if (l != l) continue;
        if (!any || l > mx) { mx = l; any = 1; }
    }
    uint64_t s = 0;
    for (int v = 0; v < V; ++v) {
        float l = row[v] * inv_t;
        uint64_t e;
        if (!any || l != l) e = 0;
        else if (l == mx) e = 4294967296ull;
        else {
            float dlt = l - mx;
            e = (dlt != dlt) ? 0 : fst_prob_fixed(dlt);
        }
        if (E) E[v] = e;
        s += e;
    }
    return s;
}

/* Speculative rejection sampling (Leviathan et al. 2023; Chen et al. 2023).
 * The reference has no stochastic acceptance (its only sampler draws from an
 * unseeded mt19937, src/fst_engine.cpp:4522-4523), so this build defines it:
 *   p_i = softmax(t_i/T), q_i = softmax(d_i/T) in 2^-32 fixed point
 *   (E = floor(exp(l-max)*2^32), S = sum E, exact integers);
 *   u_i = U_i/2^24 from Philox(seed, seq, pos=i, stream=0);
 *   accept x_i iff U_i*Q(x_i)*S_p < P(x_i)*S_q*2^24   (u < p/q);
 *   on the first reject, sample from max(0, P*S_q - Q*S_p) (exact 128-bit)
 *   by inverse CDF with target = (U'_i * sum) >> 24, U'_i from stream 1
 *   (if that residual is all zero, sample from p_i instead);
 *   if all k accepted, the bonus is sampled from p_k with U'_k. */
/* Rejection-sampling softmax statistics of one row of logits l (x = l*inv_t),
 * in the device's fixed order: the row is cut into FO_RS_CHUNKS = 64 chunks of
 * L = ceil(V/64) rounded up to a multiple of 4 elements; a chunk's maximum
 * m_c (NaN skipped) and s_c = sum e(x | m_c), summed by 256 "threads" (thread
 * t adds elements b0 + 4t + 1024i + {0,1,2,3}, i = 0, 1, ..., in that order),
 * the 64 partials of each group of 64 threads by the halving tree p[j] +=
 * p[j+off] (off = 32..1), then the four group sums left to right; the row's
 * (M, S) merges the 64 chunk partials (fst_softmax_merge) by the same
 * halving tree. */
#define FO_RS_CHUNKS 64
static int fo_rs_chunk_len(int V) { return ((V + FO_RS_CHUNKS - 1) / FO_RS_CHUNKS + 3) & ~3; }

static void fo_rs_chunk(const float* row, int V, float inv_t, int c, float* m_out, float* s_out) {
    const int L = fo_rs_chunk_len(V);
    const int b0 = c * L < V ? c * L : V, b1 = b0 + L < V ? b0 + L : V;
    float m = -INFINITY;
    for (int v = b0; v < b1; ++v) {
        const float x = row[v] * inv_t;
        if (x == x && x > m) m = x;
    }
    float part[256];
    for (int t = 0; t < 256; ++t) {
        float acc = 0.0f;
        for (int base = b0 + 4 * t; base < b1; base += 1024)
            for (int e = 0; e < 4; ++e) {
                const int v = base + e;
                if (v >= b1) break;
                const float x = row[v] * inv_t;
                if (x == x) acc = acc + fst_rel_exp(x, m);
            }
        part[t] = acc;
    }
    float ws[4];
    for (int w = 0; w < 4; ++w) {
        float a[64];
        for (int j = 0; j < 64; ++j) a[j] = part[64 * w + j];
        for (int off = 32; off >= 1; off >>= 1)
            for (int j = 0; j < off; ++j) a[j] = a[j] + a[j + off];
        ws[w] = a[0];
    }
    *m_out = m;
    *s_out = ((ws[0] + ws[1]) + ws[2]) + ws[3];
}

void fo_rs_row_stats(const float* row, int V, float inv_t, float* M, float* S) {
    float lm[FO_RS_CHUNKS], ls[FO_RS_CHUNKS];
    for (int c = 0; c < FO_RS_CHUNKS; ++c) fo_rs_chunk(row, V, inv_t, c, &lm[c], &ls[c]);
    for (int off = 32; off >= 1; off >>= 1)
        for (int j = 0; j < off; ++j) fst_softmax_merge(&lm[j], &ls[j], lm[j + off], ls[j + off]);
    *M = lm[0];
    *S = ls[0];
}

/* e(x | M) of a scaled logit (0 for NaN, -inf, or a row with no number):
 * the softmax numerator, p(x) = e / S. */
static float fo_rs_e(float x, float M) {
    if (x != x || M == -INFINITY) return 0.0f;
    return fst_rel_exp(x, M);
}

float fo_race_uniform(uint64_t seed, uint64_t seq, uint32_t pos, uint32_t v) {
    return fst_race_uniform(seed, seq, pos, v);
}

/* The exponential race at position pos over the residual in numerator form,
 * r_v = e_t(v)*S_d - e_d(v)*S_t = (p_v - q_v)*S_t*S_d (two rounded products,
 * one rounded difference; for the bonus position r_v = e_t(v)): the token is
 * the v minimising E_v / r_v over r_v > 0 (E_v = -log u_v, u_v =
 * fst_race_uniform(seed, seq, pos, v); ties to the lower index), i.e. a draw
 * from norm(max(0, p - q)); with no r_v > 0, the race over e_t(v) > 0 (a draw
 * from p); with neither, token 0.  Keys compare as (float bits << 32 | v),
 * which orders non-negative floats, then indices. */
int fo_rs_race(const float* trow, const float* drow, int V, float inv_t, float Mt, float St, float Md, float Sd,
               uint64_t seed, uint64_t seq, uint32_t pos) {
    uint64_t best_r = ~0ull, best_p = ~0ull;
    for (int v = 0; v < V; ++v) {
        const float et = fo_rs_e(trow[v] * inv_t, Mt);
        float r = et;
        if (drow) {
            const float ed = fo_rs_e(drow[v] * inv_t, Md);
            const float a = et * Sd, b = ed * St;
            r = a - b;
        }
        const float E = -fst_logf(fst_race_uniform(seed, seq, pos, (uint32_t)v));
        if (r > 0.0f) {
            const uint64_t key = ((uint64_t)fst_f32_bits(E / r) << 32) | (uint32_t)v;
            if (key < best_r) best_r = key;
        }
        if (et > 0.0f) {
            const uint64_t key = ((uint64_t)fst_f32_bits(E / et) << 32) | (uint32_t)v;
            if (key < best_p) best_p = key;
        }
    }
    if (best_r != ~0ull) return (int)(uint32_t)best_r;
    if (best_p != ~0ull) return (int)(uint32_t)best_p;
    return 0;
}

/* Speculative rejection sampling (Leviathan et al. 2023; Chen et al. 2023).
 * The reference has no stochastic acceptance (its only sampler draws from an
 * unseeded mt19937, src/fst_engine.cpp:4522-4523; its HF script samples by
 * Gumbel-max, scripts/hf_gen_ref.py:632-639), so this build defines it:
 *   p_i = softmax(t_i/T), q_i = softmax(d_i/T) from the rows' (M, S)
 *   (fo_rs_row_stats) and numerators e(x | M);
 *   u_i = U_i / 2^24, U_i = fst_uniform24(seed, seq, i, 0);
 *   accept x_i iff (u_i * e_d(x_i)) * S_t < e_t(x_i) * S_d, i.e. u < p/q
 *   with both sides multiplied by S_t*S_d (a draft row with no number
 *   rejects);
 *   on the first reject at i, the token is drawn from norm(max(0, p_i - q_i))
 *   by the exponential race fo_rs_race(pos = i) (from p_i if that residual is
 *   all zero); if all k are accepted, the bonus is the race over p_k. */
int fo_accept_stochastic(const float* target, const float* draft_logits, int k, int V,
                         const int32_t* draft, float temperature, uint64_t seed, uint64_t seq,
                         int32_t* n_acc, int32_t* tokens) {
    if (!(temperature > 0.0f)) return 1;
    const float inv_t = 1.0f / temperature;
    int n = 0;
    for (; n < k; ++n) {
        const int x = draft[n];
        if (x < 0 || x >= V) return 1;
        float Mt, St, Md, Sd;
        fo_rs_row_stats(target + (size_t)n * V, V, inv_t, &Mt, &St);
        fo_rs_row_stats(draft_logits + (size_t)n * V, V, inv_t, &Md, &Sd);
        const float et = fo_rs_e(target[(size_t)n * V + x] * inv_t, Mt);
        const float ed = fo_rs_e(draft_logits[(size_t)n * V + x] * inv_t, Md);
        const float u = (float)fst_uniform24(seed, seq, (uint32_t)n, 0) * 5.9604644775390625e-8f;
        const float lhs = (u * ed) * St, rhs = et * Sd;
        if (lhs < rhs) {
            tokens[n] = x;
            continue;
        }
        tokens[n] = fo_rs_race(target + (size_t)n * V, draft_logits + (size_t)n * V, V, inv_t, Mt, St, Md, Sd,
                               seed, seq, (uint32_t)n);
        *n_acc = n;
        return 0;
    }
    float Mt, St;
    fo_rs_row_stats(target + (size_t)k * V, V, inv_t, &Mt, &St);
    tokens[k] = fo_rs_race(target + (size_t)k * V, NULL, V, inv_t, Mt, St, 0.0f, 0.0f, seed, seq, (uint32_t)k);
    *n_acc = k;
    return 0;
}

/* ------------------------------------------------------------ sample_token */

/* src/fst_engine.cpp:4491-4528 (FSTEngine::sample_token): temperature <= 0
 * gives the plain argmax (:4495-4500, the rule of fo_argmax); otherwise the
 * softmax of logits/T, the top-p set (tokens by descending probability,
 * :4511-4517, kept until the cumulative mass reaches top_p), renormalised,
 * and one draw by inverse CDF over the kept tokens in that order (:4519-4527).
 * The reference draws from an unseeded std::mt19937, so this build defines
 * a reproducible form with the fixed-point machinery of the acceptance:
 *   E[v] = floor(exp(x_v*(1/T) - max)*2^32) (fo_softmax_fixed), S = sum E;
 *   order: E descending, ties by lower index (the reference's partial_sort
 *   leaves tie order unspecified);
 *   kept = shortest prefix (at least one token) whose mass C satisfies
 *   C*2^32 >= q*S, q = floor(top_p*2^32) clamped to [0, 2^32];
 *   U = fst_uniform24(seed, seq, 0, 2); target = (U*C_kept) >> 24; the token
 *   is the first of the kept prefix whose running mass exceeds target.
 * Restated here with an explicit sort (the device kernel searches by radix
 * histograms instead). */
typedef struct { uint64_t e; int v; } fo_ev;
static int fo_ev_cmp(const void* a, const void* b) {
    const fo_ev* x = (const fo_ev*)a;
    const fo_ev* y = (const fo_ev*)b;
    if (x->e != y->e) return x->e > y->e ? -1 : 1;
    return x->v < y->v ? -1 : (x->v > y->v ? 1 : 0);
}

uint64_t fo_top_p_fixed(float top_p) {
    if (!(top_p > 0.0f)) return 0;
    if (top_p >= 1.0f) return 4294967296ull;
    return (uint64_t)floor((double)top_p * 4294967296.0);
}

int fo_sample_token(const float* logits, int V, float temperature, float top_p, uint64_t seed, uint64_t seq,
                    int* n_kept) {
    if (n_kept) *n_kept = 1;
    if (!(temperature > 0.0f)) return fo_argmax(logits, V);
    const float inv_t = 1.0f / temperature;
    uint64_t* E = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)V);
    fo_ev* ord = (fo_ev*)malloc(sizeof(fo_ev) * (size_t)V);
    const uint64_t S = fo_softmax_fixed(logits, V, inv_t, E);
    if (S == 0) { free(E); free(ord); return 0; }
    for (int v = 0; v < V; ++v) { ord[v].e = E[v]; ord[v].v = v; }
    qsort(ord, (size_t)V, sizeof(fo_ev), fo_ev_cmp);
    const u128 need = (u128)fo_top_p_fixed(top_p) * S;
    uint64_t C = 0;
    int n = 0;
    while (n < V) {
        C += ord[n].e;
        ++n;
        if (((u128)C << 32) >= need) break;
    }
    const uint32_t U = fst_uniform24(seed, seq, 0u, 2u);
    const uint64_t tgt = (uint64_t)(((u128)U * C) >> 24);
    uint64_t c = 0;
    int tok = ord[n - 1].v;
    for (int i = 0; i < n; ++i) {
        c += ord[i].e;
        if (c > tgt) { tok = ord[i].v; break; }
    }
    if (n_kept) *n_kept = n;
    free(E);
    free(ord);
    return tok;
}

/* ----------------------------------------------------------------- RMSNorm */

/* src/fst_engine.cpp:89-91 (rms_cpu): r = 1/sqrt(mean(x^2)+eps), out =
 * bf16(x*r*w); this build rounds RNE and accumulates the mean in double. */
void fo_rmsnorm(const float* x, const uint16_t* w, int M, int d, float eps, uint16_t* out) {
    /* src/fst_engine.cpp:89-90 (rms_cpu) with RNE output and a fixed order
     * for the sum of squares: in double, 64 partials over contiguous d/64
     * chunks summed sequentially, then p[j] += p[j+off] for off = 32..1. */
    const int C = d / 64;
    for (int m = 0; m < M; ++m) {
        const float* xr = x + (size_t)m * d;
        double p[64];
        for (int j = 0; j < 64; ++j) {
            double a = 0.0;
            for (int i = 0; i < C; ++i) {
                const double v = (double)xr[j * C + i];
                a = a + v * v;
            }
            p[j] = a;
        }
        for (int off = 32; off >= 1; off >>= 1)
            for (int j = 0; j < off; ++j) p[j] = p[j] + p[j + off];
        const float r = (float)(1.0 / sqrt(p[0] / (double)d + (double)eps));
        for (int j = 0; j < d; ++j)
            out[(size_t)m * d + j] = fst_f32_to_bf16((xr[j] * r) * fst_bf16_to_f32(w[j]));
    }
}

/* Dense Q4_K linear (the LM head, src/fst_engine.cpp:2115-2160 with a Q4_K
 * head): y[m][n] = sum_k W[n][k] x[m][k], W dequantised per
 * kernels/fst_dequant_q4k_kernel.cc, double accumulation.  blocks: [N][K/256]. */
int fo_q4k_linear(const uint8_t* blocks, int N, int K, const uint16_t* x, int M, float* y) {
    if (K % 256) return 1;
    float* xf = (float*)malloc(sizeof(float) * (size_t)M * K);
    if (!xf) return 2;
    for (size_t i = 0; i < (size_t)M * K; ++i) xf[i] = fst_bf16_to_f32(x[i]);
    const size_t row_bytes = (size_t)(K / 256) * 144;
#pragma omp parallel num_threads(FO_NT)
    {
        float* wr = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
        for (int n = 0; n < N; ++n) {
            fo_q4k_dequant(blocks + (size_t)n * row_bytes, (size_t)(K / 256), wr);
            for (int m = 0; m < M; ++m) {
                const float* xr = xf + (size_t)m * K;
                double acc = 0.0;
                for (int k = 0; k < K; ++k) acc += (double)xr[k] * (double)wr[k];
                y[(size_t)m * N + n] = (float)acc;
            }
        }
        free(wr);
    }
    free(xf);
    return 0;
}

/* ------------------------------------------------- Hyper-Connections (HC) */

/* src/fst_engine.cpp:2286-2459 (hc_split_sinkhorn, hc_rmsnorm_no_weight,
 * hc_pre, hc_post, output_hc_head) and :694-742 (npu_gemm_hc) for N = 4
 * streams of width d, with fixed orders where the reference leaves them to
 * the NPU or to libm:
 *  - sum of squares over the 4d values: double, 64 partials over contiguous
 *    chunks, then p[j] += p[j+off] (off = 32..1); inv = 1/sqrtf((float)(ss/n) + eps);
 *  - the control matvec mix[n] = flat . fn[n]: per 1024-wide K chunk, 16
 *    partials of 64 consecutive products (sequential fmaf), a halving tree,
 *    the chunk sum rounded to bf16 (the NPU tile output), chunk sums added
 *    in order in float, the total rounded to bf16;
 *  - exp is fst_expf; bf16 rounding is RNE; no contraction. */
static float fo_hc_inv_rms(const float* v, int n, float eps) {
    const int C = n / 64;
    double p[64];
    for (int j = 0; j < 64; ++j) {
        double a = 0.0;
        for (int i = 0; i < C; ++i) {
            const double x = (double)v[j * C + i];
            a = a + x * x;
        }
        p[j] = a;
    }
    for (int off = 32; off >= 1; off >>= 1)
        for (int j = 0; j < off; ++j) p[j] = p[j] + p[j + off];
    return 1.0f / sqrtf((float)(p[0] / (double)n) + eps);
}

void fo_hc_mix(const uint16_t* flat_bf, const uint16_t* fnT, int K, int nout, float* mix) {
    for (int n = 0; n < nout; ++n) {
        const uint16_t* w = fnT + (size_t)n * K;
        float acc = 0.0f;
        for (int c0 = 0; c0 < K; c0 += 1024) {
            float p[16];
            for (int l = 0; l < 16; ++l) {
                float a = 0.0f;
                for (int i = 0; i < 64; ++i) {
                    const int k = c0 + l * 64 + i;
                    a = fmaf(fst_bf16_to_f32(flat_bf[k]), fst_bf16_to_f32(w[k]), a);
                }
                p[l] = a;
            }
            for (int off = 8; off >= 1; off >>= 1)
                for (int l = 0; l < off; ++l) p[l] = p[l] + p[l + off];
            acc = acc + fst_bf16_to_f32(fst_f32_to_bf16(p[0]));
        }
        mix[n] = fst_bf16_to_f32(fst_f32_to_bf16(acc));
    }
}

void fo_hc_split(const float* mix, const float* scale, const float* base, int n, int iters, float eps,
                 float* split) {
    const float pre_scale = scale[0], post_scale = scale[1], comb_scale = scale[2];
    for (int i = 0; i < n; ++i) {
        const float z = mix[i] * pre_scale + base[i];
        split[i] = 1.0f / (1.0f + fst_expf(-z)) + eps;
    }
    for (int i = 0; i < n; ++i) {
        const int off = n + i;
        const float z = mix[off] * post_scale + base[off];
        split[off] = 2.0f / (1.0f + fst_expf(-z));
    }
    float c[16];
    for (int dst = 0; dst < n; ++dst) {
        float row_max = -1e30f;
        for (int src = 0; src < n; ++src) {
            const int idx = src + dst * n;
            const float v = mix[2 * n + idx] * comb_scale + base[2 * n + idx];
            c[idx] = v;
            if (v > row_max) row_max = v;
        }
        float row_sum = 0.0f;
        for (int src = 0; src < n; ++src) {
            const int idx = src + dst * n;
            c[idx] = fst_expf(c[idx] - row_max);
            row_sum += c[idx];
        }
        const float inv = 1.0f / row_sum;
        for (int src = 0; src < n; ++src) c[src + dst * n] = c[src + dst * n] * inv + eps;
    }
    for (int src = 0; src < n; ++src) {
        float sum = 0.0f;
        for (int dst = 0; dst < n; ++dst) sum += c[src + dst * n];
        const float inv = 1.0f / (sum + eps);
        for (int dst = 0; dst < n; ++dst) c[src + dst * n] *= inv;
    }
    for (int it = 1; it < iters; ++it) {
        for (int dst = 0; dst < n; ++dst) {
            float sum = 0.0f;
            for (int src = 0; src < n; ++src) sum += c[src + dst * n];
            const float inv = 1.0f / (sum + eps);
            for (int src = 0; src < n; ++src) c[src + dst * n] *= inv;
        }
        for (int src = 0; src < n; ++src) {
            float sum = 0.0f;
            for (int dst = 0; dst < n; ++dst) sum += c[src + dst * n];
            const float inv = 1.0f / (sum + eps);
            for (int dst = 0; dst < n; ++dst) c[src + dst * n] *= inv;
        }
    }
    for (int i = 0; i < n * n; ++i) split[2 * n + i] = c[i];
}

static void fo_hc_flat(const uint16_t* r, int n, float eps, uint16_t* flat_bf) {
    float* v = (float*)malloc(sizeof(float) * (size_t)n);
    if (!v) return;
    for (int i = 0; i < n; ++i) v[i] = fst_bf16_to_f32(r[i]);
    const float inv = fo_hc_inv_rms(v, n, eps);
    for (int i = 0; i < n; ++i) flat_bf[i] = fst_f32_to_bf16(v[i] * inv);
    free(v);
}

void fo_hc_pre(const uint16_t* h_hc, const uint16_t* fnT, const float* scale, const float* base, int M, int d,
               int iters, float eps, uint16_t* cur, float* post, float* comb) {
    const int N = 4, K = N * d, NM = 2 * N + N * N;
    uint16_t* flat = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)K);
    for (int m = 0; m < M; ++m) {
        const uint16_t* r = h_hc + (size_t)m * K;
        fo_hc_flat(r, K, eps, flat);
        float mix[24], split[24];
        fo_hc_mix(flat, fnT, K, NM, mix);
        fo_hc_split(mix, scale, base, N, iters, eps, split);
        for (int i = 0; i < N; ++i) post[(size_t)m * N + i] = split[N + i];
        for (int i = 0; i < N * N; ++i) comb[(size_t)m * N * N + i] = split[2 * N + i];
        for (int j = 0; j < d; ++j) {
            float acc = 0.0f;
            for (int h = 0; h < N; ++h) acc = acc + split[h] * fst_bf16_to_f32(r[(size_t)h * d + j]);
            cur[(size_t)m * d + j] = fst_f32_to_bf16(acc);
        }
    }
    free(flat);
}

void fo_hc_post(const uint16_t* bo, const uint16_t* h_hc, const float* post, const float* comb, int M, int d,
                uint16_t* out_hc) {
    const int N = 4;
    for (int m = 0; m < M; ++m)
        for (int dst = 0; dst < N; ++dst)
            for (int j = 0; j < d; ++j) {
                float acc = fst_bf16_to_f32(bo[(size_t)m * d + j]) * post[(size_t)m * N + dst];
                for (int src = 0; src < N; ++src)
                    acc = acc + comb[(size_t)m * N * N + dst + src * N] *
                                    fst_bf16_to_f32(h_hc[(size_t)m * N * d + (size_t)src * d + j]);
                out_hc[(size_t)m * N * d + (size_t)dst * d + j] = fst_f32_to_bf16(acc);
            }
}

void fo_hc_head(const uint16_t* h_hc, const uint16_t* fnT, float scale, const float* base, int M, int d, float eps,
                uint16_t* plain) {
    const int N = 4, K = N * d;
    uint16_t* flat = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)K);
    for (int m = 0; m < M; ++m) {
        const uint16_t* r = h_hc + (size_t)m * K;
        fo_hc_flat(r, K, eps, flat);
        float mix[4], w[4];
        fo_hc_mix(flat, fnT, K, N, mix);
        for (int h = 0; h < N; ++h) {
            const float z = mix[h] * scale + (base ? base[h] : 0.0f);
            w[h] = 1.0f / (1.0f + fst_expf(-z)) + eps;
        }
        for (int j = 0; j < d; ++j) {
            float acc = 0.0f;
            for (int h = 0; h < N; ++h) acc = acc + w[h] * fst_bf16_to_f32(r[(size_t)h * d + j]);
            plain[(size_t)m * d + j] = fst_f32_to_bf16(acc);
        }
    }
    free(flat);
}
