/* fst_oracle.h — CPU restatement of the reference's verify-path semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this code.  It is used by tests/ (as the checker), by
 * __graft_entry__.smoke() (as the checker) and by bench.py's cpu_baseline
 * leg (as the timed CPU baseline).  Each function cites the reference
 * file:line it restates; see fst_oracle.c for the per-function pins.
 */
#ifndef FST_ORACLE_H
#define FST_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* codecs */
int fo_q4k_dequant(const uint8_t* blocks, size_t nblocks, float* out);     /* 256 per block */
int fo_mxfp4_dequant(const uint8_t* blocks, size_t nblocks, float* out);   /* 32 per block  */
void fo_q4k_scale_min(int j, const uint8_t* q, uint8_t* sc, uint8_t* m);
float fo_fp16_to_f32(uint16_t h);
uint16_t fo_f32_to_bf16(float f);

/* Expert SwiGLU FFN, fp32 weights, fp64 accumulation.
 * codec 0 = Q4_K, 1 = MXFP4.  h: bf16 [M][hd], y: fp32 [M][hd]. */
int fo_expert_ffn(int codec, const uint8_t* expert, int hd, int inter,
                  const uint16_t* h, int M, float swiglu_limit, float* y);

/* Same, with pre-dequantised fp32 matrices gate/up [inter][hd], down [hd][inter]. */
void fo_expert_ffn_f32(const float* wg, const float* wu, const float* wd, int hd, int inter,
                       const uint16_t* h, int M, float swiglu_limit, float* y);

/* Router.  w_kn: bf16 [K][N] (K = hd, N = n_experts).  Canonical logit order:
 * 64 partials over contiguous K/64 chunks (sequential fmaf), then a halving
 * tree (offsets 32,16,8,4,2,1).  score_func 0 = sigmoid, 1 = sqrtsoftplus. */
void fo_router_logits(const uint16_t* h, const uint16_t* w_kn, int M, int K, int N, float* logits);
int fo_router(const uint16_t* h, const uint16_t* w_kn, const float* bias, int M, int K, int N,
              int top_k, int score_func, float route_scale, int round_logits_bf16,
              const int32_t* hash_row_eids /* [M][top_k] or NULL */,
              int32_t* eids, float* wts, float* logits_out /* nullable */);

/* Combine: out[m] = bf16( sum_j wts[m][j] * y_routed[m][j][:] + y_shared[m][:] ). */
void fo_combine(const float* y_routed /* [M][tk][hd] */, const float* y_shared /* [M][hd] or NULL */,
                const float* wts, int M, int tk, int hd, uint16_t* out, float* out_f32);

/* Acceptance (one sequence).  target: [k+1][V], draft_logits: [k][V]. */
int fo_argmax(const float* logits, int V);
/* sample_token (src/fst_engine.cpp:4491-4528) in the build's reproducible
 * fixed-point form; n_kept (nullable) gets the size of the top-p set. */
uint64_t fo_top_p_fixed(float top_p);
int fo_sample_token(const float* logits, int V, float temperature, float top_p, uint64_t seed, uint64_t seq,
                    int* n_kept);
int fo_accept_greedy(const float* target, int k, int V, const int32_t* draft,
                     int32_t* n_acc, int32_t* tokens);
int fo_accept_stochastic(const float* target, const float* draft_logits, int k, int V,
                         const int32_t* draft, float temperature, uint64_t seed, uint64_t seq,
                         int32_t* n_acc, int32_t* tokens);
/* Rejection sampling's pieces, for pinning tests: a row's softmax (M, S) in the
 * device's fixed order, and the exponential race of one position. */
void fo_rs_row_stats(const float* row, int V, float inv_t, float* M, float* S);
int fo_rs_race(const float* trow, const float* drow /* nullable */, int V, float inv_t, float Mt, float St,
               float Md, float Sd, uint64_t seed, uint64_t seq, uint32_t pos);
float fo_race_uniform(uint64_t seed, uint64_t seq, uint32_t pos, uint32_t v);

/* RMSNorm (src/fst_engine.cpp:89-91 with RNE): out = bf16((x * r) * w),
 * r = (float)(1/sqrt(ss/d + eps)), ss in double in the fixed order of fst_oracle.c. */
void fo_rmsnorm(const float* x, const uint16_t* w, int M, int d, float eps, uint16_t* out);

/* Dense Q4_K linear (LM head): y[M][N] = x[M][K] . W^T, W = blocks [N][K/256]. */
int fo_q4k_linear(const uint8_t* blocks, int N, int K, const uint16_t* x, int M, float* y);

/* Hyper-Connections with 4 streams of width d (residual h_hc [M][4][d] bf16).
 * fnT: the control matrices transposed to [outputs][4d] bf16 (24 outputs for
 * pre/post/comb, 4 for the head).  iters = Sinkhorn iterations (20), eps 1e-6. */
void fo_hc_mix(const uint16_t* flat_bf, const uint16_t* fnT, int K, int nout, float* mix);
void fo_hc_split(const float* mix, const float* scale, const float* base, int n, int iters, float eps,
                 float* split);
void fo_hc_pre(const uint16_t* h_hc, const uint16_t* fnT, const float* scale, const float* base, int M, int d,
               int iters, float eps, uint16_t* cur, float* post, float* comb);
void fo_hc_post(const uint16_t* bo, const uint16_t* h_hc, const float* post, const float* comb, int M, int d,
                uint16_t* out_hc);
void fo_hc_head(const uint16_t* h_hc, const uint16_t* fnT, float scale, const float* base, int M, int d, float eps,
                uint16_t* plain);

/* exact-math passthroughs for pinning tests */
float fo_expf(float x);
void fo_exp_nonpos_n(const float* x, int n, float* out);
void fo_expf_n(const float* x, int n, float* out);
float fo_logf(float x);
float fo_sigmoidf(float x);
float fo_sqrtsoftplusf(float x);
void fo_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
uint32_t fo_uniform24(uint64_t seed, uint64_t seq, uint32_t pos, uint32_t stream);

void fo_set_threads(int n);
int fo_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
