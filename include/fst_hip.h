/* fst_hip.h — C-ABI of the MI355X (gfx950) DSpark verify hot path.
 *
 * This library replaces, for one GPU, the four pieces of the reference
 * engine's block-verification path:
 *
 *   FSTEngine::npu_router           include/fst_engine.h:413, src/fst_engine.cpp:936-1076
 *   FSTEngine::process_expert_ffn   include/fst_engine.h:318, src/fst_engine.cpp:4068-4371
 *   FSTEngine::process_shared_expert include/fst_engine.h:319, src/fst_engine.cpp:4373-4489
 *   routed + shared combine         src/fst_engine.cpp:2848-2852
 *   greedy accept/reject            src/fst_engine.cpp:6021-6063 (inline in generate_dspark)
 *
 * plus the expert residency the engine gets from get_expert_bo
 * (src/fst_engine.cpp:3892-3926): all routed and shared experts of a layer
 * are uploaded once and stay in HBM.
 *
 * Conventions: plain pointers and sizes only; bf16 values are uint16_t bit
 * patterns (as bf16_t in include/fst_engine.h:16); activations are row-major
 * [M][hidden]; eids/wts are token-major [M][top_k].  Functions return an
 * FST_* status code; fst_last_error() gives the message of the last failure
 * on the calling thread.  Host-pointer entry points are synchronous.  The
 * *_dev entry points take device pointers and are asynchronous on the
 * context's stream (fst_stream()); fst_sync() waits for them.  Their
 * activation and logits buffers must be 16-byte aligned (hipMalloc and
 * fst_device_alloc give 256; FST_EINVAL otherwise), as the kernels read them
 * with 16-byte loads.  A context is not re-entrant: calls on one context
 * must not overlap.
 */
#ifndef FST_HIP_H
#define FST_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FST_ABI_VERSION 1

enum fst_status {
    FST_OK = 0,
    FST_EINVAL = 1,    /* bad argument, shape or state */
    FST_ENOMEM = 2,    /* device or host allocation failed */
    FST_EHIP = 3,      /* HIP runtime error (message says which call) */
    FST_ENODEV = 4,    /* no usable gfx950 device */
    FST_ENOTREADY = 5  /* weights for this layer/expert were never uploaded */
};

enum fst_codec { FST_CODEC_Q4K = 0, FST_CODEC_MXFP4 = 1 };
enum fst_score { FST_SCORE_SIGMOID = 0, FST_SCORE_SQRTSOFTPLUS = 1 };

typedef struct fst_ctx fst_ctx;

/* Layer geometry and routing semantics (ModelConfig, include/fst_engine.h:127-149). */
typedef struct fst_config {
    int hidden_dim;        /* 4096 */
    int inter_dim;         /* 2048 (INTER_DIM, include/fst_engine.h:92) */
    int n_experts;         /* routed experts per layer, 256 */
    int top_k;             /* 6 */
    int n_layers;          /* layers with resident weights */
    int max_tokens;        /* largest M per call, <= 64 */
    int codec;             /* enum fst_codec */
    int has_shared;        /* 1: one shared expert per layer */
    int score_func;        /* enum fst_score */
    float route_scale;     /* routed_scaling_factor: 1.0 (sigmoid configs) or 1.5 (V4) */
    int round_logits_bf16; /* 1: round router logits to bf16 before scoring, as the NPU GEMM does */
    int n_hash_layers;     /* layers < this use tid2eid hash routing when a table is uploaded */
    int vocab_size;        /* 129280; used by hash tables, LM head and acceptance */
    float swiglu_limit;    /* 0: no clamp (engine default); >0: HF clamp */
    int device;            /* HIP device ordinal */
} fst_config;

/* Fills the DeepSeek-V4-Flash-like defaults used by the benchmark configs. */
void fst_config_default(fst_config* cfg);

const char* fst_last_error(void);
int fst_abi_version(void);

/* Bytes of one packed expert (gate|up|down, each [N rows][K/block] blocks):
 * Q4_K 14,155,776 B, MXFP4 13,369,344 B at 4096/2048. */
size_t fst_expert_bytes(const fst_config* cfg);

int fst_create(const fst_config* cfg, fst_ctx** out);
/* The configuration the context was created with. */
int fst_get_config(const fst_ctx* ctx, fst_config* out);
void fst_destroy(fst_ctx* ctx);
void* fst_stream(fst_ctx* ctx);       /* hipStream_t of the context */
int fst_sync(fst_ctx* ctx);

/* ---- device buffers for the *_dev entry points (hipMalloc / hipMemcpy on the context stream) ---- */
void* fst_device_alloc(fst_ctx* ctx, size_t bytes);
void fst_device_free(fst_ctx* ctx, void* p);
int fst_copy_to_device(fst_ctx* ctx, void* dst, const void* src, size_t bytes);
int fst_copy_to_host(fst_ctx* ctx, void* dst, const void* src, size_t bytes);

/* ---- weight residency (replaces get_expert_bo / ExpertPager for the timed path) ---- */
/* eid in [0, n_experts) uploads a routed expert; eid == n_experts the shared one. */
int fst_upload_expert(fst_ctx* ctx, int lid, int eid, const void* packed, size_t bytes);
/* Router weight W[K=hidden][N=n_experts] in bf16 or fp32
 * (the reference's npu_router argument, converted with RNE).  bias may be NULL. */
int fst_upload_router_bf16(fst_ctx* ctx, int lid, const uint16_t* w_kn, const float* bias);
int fst_upload_router_f32(fst_ctx* ctx, int lid, const float* w_kn, const float* bias);
/* tid2eid hash table [vocab][top_k] for lid < n_hash_layers (src/fst_engine.cpp:1015-1021). */
int fst_upload_hash_table(fst_ctx* ctx, int lid, const int32_t* tid2eid);
/* The shared expert in bf16, as the reference keeps it (TID_SHARED_GATE/UP/DOWN,
 * process_shared_expert src/fst_engine.cpp:4373-4489): gate, up [inter][hidden]
 * and down [hidden][inter], row-major.  Once uploaded, the layer's shared expert
 * runs from these matrices (bf16 MFMA, h rounded to bf16) instead of expert
 * slot n_experts of the codec bank. */
int fst_upload_shared_bf16(fst_ctx* ctx, int lid, const uint16_t* gate, const uint16_t* up, const uint16_t* down);
/* Device address of a resident expert (for in-place generation/inspection). */
void* fst_expert_device_ptr(fst_ctx* ctx, int lid, int eid);

/* ---- router: npu_router (include/fst_engine.h:413) ---- */
int fst_router(fst_ctx* ctx, int lid, const uint16_t* h, int M, const int32_t* input_ids,
               int32_t* eids, float* wts);

/* ---- expert FFN: process_expert_ffn / process_shared_expert (include/fst_engine.h:318-319) ---- */
/* out = bf16( sum_j wts[m][j] * FFN_{eids[m][j]}(h[m]) ) */
int fst_expert_ffn(fst_ctx* ctx, int lid, const uint16_t* h, uint16_t* out, int M,
                   const int32_t* eids, int tk, const float* wts);
/* out = bf16( FFN_shared(h[m]) ) */
int fst_shared_expert(fst_ctx* ctx, int lid, const uint16_t* h, uint16_t* out, int M);

/* ---- fused MoE layer: router -> routed -> shared -> combine, all on device ---- */
/* out = bf16( routed + shared ); eids/wts outputs may be NULL. */
int fst_moe_layer(fst_ctx* ctx, int lid, const uint16_t* h, int M, const int32_t* input_ids,
                  uint16_t* out, int32_t* eids, float* wts);
/* Device-pointer, stream-ordered variants.  eids/wts are written (device). */
int fst_moe_layer_dev(fst_ctx* ctx, int lid, const uint16_t* d_h, int M, const int32_t* d_input_ids,
                      uint16_t* d_out, int32_t* d_eids, float* d_wts);
/* Given routing (device eids/wts), with optional routed-only / shared-only outputs. */
int fst_moe_ffn_dev(fst_ctx* ctx, int lid, const uint16_t* d_h, int M, const int32_t* d_eids,
                    const float* d_wts, int use_shared, uint16_t* d_out,
                    uint16_t* d_out_routed, uint16_t* d_out_shared);
/* Errors of the asynchronous MoE calls (fst_moe_layer_dev, fst_moe_ffn_dev,
 * fst_verify_forward_dev).  The reference raises a failed or stuck NPU
 * dispatch as an exception per dispatch (npu_run_wait, flush_pending_runs,
 * src/fst_engine.cpp:200-223).  Here every MoE launch ORs what it detects on
 * the device into a sticky error word of the context: an expert id out of
 * range (FST_EINVAL), an input id out of the vocabulary for hash routing
 * (FST_EINVAL), a cross-workgroup hand-off wait that gave up at the spin
 * limit (FST_EHIP; that call's output rows are wrong).  Kernels only set
 * bits; fst_moe_check waits for the context's stream, returns the status of
 * the bits set since the last check (FST_OK when none), and clears them.
 * The host-pointer entry points (fst_moe_layer, fst_router, fst_expert_ffn,
 * fst_shared_expert, fst_verify_forward) run the same check before they
 * return, so an error of any layer of a verify forward is reported. */
int fst_moe_check(fst_ctx* ctx);
/* The status fst_moe_check returns for a given word of sticky bits (1: expert
 * id, 2: hash input id, 4: hand-off timeout), for callers that read the word
 * themselves; sets fst_last_error like any failing call. */
int fst_device_error_status(int flags);

/* ---- acceptance (src/fst_engine.cpp:6021-6063) ---- */
/* target: [n_seq][k+1][V] fp32, draft: [n_seq][k] int32,
 * n_acc: [n_seq], tokens: [n_seq][k+1] (first n_acc[s]+1 valid). */
int fst_accept_greedy(fst_ctx* ctx, const float* target, int n_seq, int k, int V,
                      const int32_t* draft, int32_t* n_acc, int32_t* tokens);
/* Rejection sampling (defined by this build; the reference is greedy-only):
 * draft_logits [n_seq][k][V]; p = softmax(target/T), q = softmax(draft/T)
 * from each row's (max, sum) in binary32 in a fixed order; draft x_i is
 * accepted iff u_i*q(x_i) < p(x_i) (compared as (u*e_q)*S_p < e_p*S_q); the
 * first rejected position draws from norm(max(0, p - q)), and the bonus
 * position from p, by an exponential race (argmin of -log(u_v)/r_v, Gumbel-max
 * sampling); Philox uniforms keyed by (seed, seq_base + s, position). */
int fst_accept_stochastic(fst_ctx* ctx, const float* target, const float* draft_logits,
                          int n_seq, int k, int V, const int32_t* draft, float temperature,
                          uint64_t seed, uint64_t seq_base, int32_t* n_acc, int32_t* tokens);
int fst_accept_greedy_dev(fst_ctx* ctx, const float* d_target, int n_seq, int k, int V,
                          const int32_t* d_draft, int32_t* d_n_acc, int32_t* d_tokens);
int fst_accept_stochastic_dev(fst_ctx* ctx, const float* d_target, const float* d_draft_logits,
                              int n_seq, int k, int V, const int32_t* d_draft, float temperature,
                              uint64_t seed, uint64_t seq_base, int32_t* d_n_acc, int32_t* d_tokens);
/* Limits: V <= 1,048,574 and n_seq*(2k+1) within the device's grid rows.
 * The greedy launch hands chunk results between workgroups; the collecting
 * workgroup's wait is bounded (fst_set_wait_limit polls, default 2^20).  A
 * wait that gives up writes n_acc[s] = -1 and tokens -1 for its sequence
 * (the host-pointer entry points then return FST_EHIP); after an asynchronous
 * *_dev call, fst_accept_check on the copied-back n_acc does the same. */
int fst_set_wait_limit(fst_ctx* ctx, int spins);  /* 0: the default; also bounds the MoE launches' waits (fst_moe_check) */
/* MoE calls of at most 32 tokens and 256 routed pairs over 4096 -> 2048 ->
 * 4096 experts (router-driven or caller-routed) run gate||up and down as one
 * persistent launch (default); on = 0 selects the
 * separate launch chain.  Both give the same results (bit for bit where the
 * chain does not split the gate||up sums over K).  A fused launch whose
 * hand-off wait exceeds the spin limit sets the sticky timeout bit
 * (fst_moe_check and the host-pointer entry points return FST_EHIP). */
int fst_set_fused(fst_ctx* ctx, int on);
/* Caller-routed calls (fst_moe_ffn_dev, fst_expert_ffn, fst_shared_expert) of
 * one or two tokens over Q4_K experts (hidden and intermediate sizes <= 4096)
 * run as one launch (default): gate||up and down as fp16 MFMA tiles over the
 * exact fp16 decode of the weights, with each token's activations prescaled
 * by a power of two per 256-element super-block and rounded to fp16.  on = 0
 * selects the launch chain, whose prescale is per row: the two agree within
 * the fp16 operand rounding, not bit for bit.  Its hand-off wait is bounded
 * like the fused launch's. */
int fst_set_small_m(fst_ctx* ctx, int on);
int fst_accept_check(const int32_t* n_acc, int n_seq);  /* host memory; FST_EHIP if any n_acc < 0 */
/* fst_accept_greedy_dev without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The workgroups' hand-off words live in a fixed per-device array of the
 * library (256 KiB, n_seq*(k+1) <= 2048 rows; larger calls get FST_EINVAL)
 * instead of the context's workspace.  All calls on one GPU share that array:
 * calls that overlap on one GPU race.  Same results as fst_accept_greedy_dev. */
int fst_accept_greedy_dev_noalloc(fst_ctx* ctx, const float* d_target, int n_seq, int k, int V,
                                  const int32_t* d_draft, int32_t* d_n_acc, int32_t* d_tokens);

/* ---- sample_token (include/fst_engine.h:277, src/fst_engine.cpp:4491-4528) ----
 * temperature <= 0: the plain argmax (first maximum wins, NaN skipped, a NaN
 * at index 0 pins 0).  Otherwise a reproducible form of the reference's
 * softmax(logits/T) -> top-p -> one draw (the reference draws from an unseeded
 * std::mt19937): probabilities in 2^-32 fixed point E = floor(exp(x/T - max)
 * * 2^32), tokens by E descending then lower index, the kept set the shortest
 * prefix whose mass reaches floor(top_p * 2^32) / 2^32 of the total (at
 * least one token), and the token the first of the kept prefix whose running
 * mass exceeds (U * kept mass) >> 24 with U = 24-bit Philox-4x32-10 uniform of
 * (seed, seq, position 0, stream 2).  The logits are not modified.
 * _dev: n_rows rows [n_rows][V] on the device, row r with seq = seq_base + r,
 * tokens [n_rows] int32 on the device. */
int fst_sample_token(fst_ctx* ctx, const float* logits, int V, float temperature, float top_p, uint64_t seed,
                     uint64_t seq, int32_t* token);
int fst_sample_token_dev(fst_ctx* ctx, const float* d_logits, int n_rows, int V, float temperature, float top_p,
                         uint64_t seed, uint64_t seq_base, int32_t* d_tokens);

/* ---- standalone dequant (bit-exact check of the codec; kernels/fst_dequant_q4k_kernel.cc) ---- */
/* codec blocks (host) -> fp32 and/or bf16 (host); either output may be NULL. */
int fst_dequant(fst_ctx* ctx, int codec, const void* blocks, size_t nblocks,
                float* out_f32, uint16_t* out_bf16);

/* ---- instrumentation ---- */
typedef struct fst_timings {
    int n;                  /* kernels recorded in the last call */
    const char* name[16];
    float ms[16];           /* per-kernel duration from HIP events on the context stream */
} fst_timings;
int fst_set_profiling(fst_ctx* ctx, int on);
int fst_last_timings(fst_ctx* ctx, fst_timings* out);
/* Kernel ring: with capacity > 0, the next `capacity` fused MoE launches
 * (router-driven calls of at most 8 tokens) record their dispatch's start and
 * end times in HIP events, with no synchronisation between calls; 0 turns it
 * off.  fst_kernel_ring_read synchronises the stream, writes up to max_n
 * kernel durations in microseconds, sets *n and empties the ring. */
int fst_kernel_ring(fst_ctx* ctx, int capacity);
int fst_kernel_ring_read(fst_ctx* ctx, float* us, int max_n, int* n);
/* Plain streaming copy kernel (16-byte vector loads/stores) used to calibrate
 * hardware byte counters against a known traffic volume.  Asynchronous. */
int fst_device_copy(fst_ctx* ctx, void* d_dst, const void* d_src, size_t bytes);
/* Number of distinct routed experts touched by the last MoE call (device -> host copy). */
int fst_last_active_experts(fst_ctx* ctx, int* n_routed_active);

/* ---- verify forward: residual stream, norms, LM head ----
 * The non-HC layer of process_layer (src/fst_engine.cpp:2738-2741 RMSNorm with
 * moe_norm, :2826-2852 MoE, :2913-2917 residual h = bf16(h + ffn_out)) and
 * apply_final_norm_and_lm_head (:2115-2160; final norm, Q4_K LM head
 * [vocab][hidden/256] blocks instead of the reference's bf16 head).
 * RMSNorm: eps 1e-6, sum of squares in double in a fixed order, out =
 * bf16((x * r) * w) (see resid_norm_kernel). */
/* lid in [0, n_layers): the layer's moe_norm; lid == n_layers: the final norm. */
int fst_upload_norm(fst_ctx* ctx, int lid, const uint16_t* w_bf16);
/* Bytes of a packed Q4_K LM head: vocab_size * hidden_dim/256 * 144. */
size_t fst_lm_head_bytes(const fst_config* cfg);
/* vocab_size must be a multiple of 128. */
int fst_upload_lm_head(fst_ctx* ctx, const void* packed, size_t bytes);
/* The reference's own bf16 head [vocab][hidden] (TID_LM_HEAD, row-major as
 * stored; src/fst_engine.cpp:2115-2160).  The head uploaded last is the one
 * fst_lm_head_dev / fst_verify_forward use. */
int fst_upload_lm_head_bf16(fst_ctx* ctx, const uint16_t* w);
/* d_h_out (nullable) = d_y ? bf16(d_h + d_y) : d_h;  d_normed = RMSNorm_lid(that). */
int fst_rmsnorm_dev(fst_ctx* ctx, int lid, const uint16_t* d_h, const uint16_t* d_y, int M, uint16_t* d_h_out,
                    uint16_t* d_normed);
/* d_logits[M][vocab] fp32 = LMHead(RMSNorm_final(d_h)). */
int fst_lm_head_dev(fst_ctx* ctx, const uint16_t* d_h, int M, float* d_logits);
/* apply_final_norm_and_lm_head (include/fst_engine.h:276, src/fst_engine.cpp:2115-2160)
 * with host buffers: logits[M][vocab] fp32.  When the HC head is uploaded
 * (fst_upload_hc_head), hs is the reference's 4-stream residual [M][4][hidden]
 * and is collapsed by output_hc_head first (:2120-2128); otherwise hs is a
 * plain [M][hidden].  The device buffers are the context's own (the logits
 * buffer is allocated on the first call and kept). */
int fst_final_head(fst_ctx* ctx, const uint16_t* hs, int M, float* logits);
/* For l in 0..n_layers-1: h = h + MoE_l(RMSNorm_l(h)); then logits =
 * LMHead(RMSNorm_final(h)).  d_h [M][hidden] bf16 is updated in place. */
int fst_verify_forward_dev(fst_ctx* ctx, uint16_t* d_h, int M, const int32_t* d_input_ids, float* d_logits);
int fst_verify_forward(fst_ctx* ctx, uint16_t* h, int M, const int32_t* input_ids, float* logits);

/* ---- Hyper-Connections: 4 residual streams of width hidden_dim ----
 * hc_pre / hc_post / output_hc_head (src/fst_engine.cpp:2286-2459) with the
 * control matvec of npu_gemm_hc (:694-742); fixed orders as in fst_hc.hip.
 * fn is the checkpoint's bf16 [24][4*hidden] (TID_HC_FFN_FN) with scale f32[3]
 * and base f32[24]; the head fn is bf16 [4][4*hidden] (TID_HC_HEAD_FN), scale
 * and base f32[4] (nullable: zeros).  When every layer's HC and the head are
 * uploaded, fst_verify_forward[_dev] runs in HC mode: h is [M][4][hidden],
 * each layer is h = hc_post(MoE(RMSNorm(hc_pre(h))), h), and the head input
 * is output_hc_head(h). */
int fst_upload_hc(fst_ctx* ctx, int lid, const uint16_t* fn, const float* scale, const float* base);
int fst_upload_hc_head(fst_ctx* ctx, const uint16_t* fn, float scale, const float* base);
/* d_cur [M][hidden] bf16, d_post [M][4], d_comb [M][16] (comb[dst + 4*src]). */
int fst_hc_pre_dev(fst_ctx* ctx, int lid, const uint16_t* d_h_hc, int M, uint16_t* d_cur, float* d_post,
                   float* d_comb);
/* In place on d_h_hc [M][4][hidden]. */
int fst_hc_post_dev(fst_ctx* ctx, const uint16_t* d_block_out, uint16_t* d_h_hc, const float* d_post,
                    const float* d_comb, int M);
int fst_hc_head_dev(fst_ctx* ctx, const uint16_t* d_h_hc, int M, uint16_t* d_plain);

/* ---- synthetic inputs (deterministic from a seed) ---- */
/* One Q4_K expert (gate|up|down in the packed ABI layout): uniform nibbles and
 * 6-bit scales/mins, d,dmin = fp16(|z|*sigma) with z ~ N(0,1) (Irwin-Hall). */
int fst_synth_q4k_expert(uint64_t seed, uint64_t expert_id, int hd, int inter, float d_sigma,
                         uint8_t* out);
/* nblocks consecutive 144-byte Q4_K blocks of matrix `id` (the expert above is
 * id = expert_id, 3*hd*inter/256 blocks). */
int fst_synth_q4k_blocks(uint64_t seed, uint64_t id, size_t nblocks, float d_sigma, uint8_t* out);
/* The same bytes generated on the device straight into the resident layout:
 * experts e_first..e_first+e_count-1 of layer lid (e == n_experts: shared)
 * from generator id id_base + e (= fst_synth_q4k_expert(seed, id_base + e)),
 * and the LM head from generator id `id` (= fst_synth_q4k_blocks(seed, id,
 * vocab*hidden/256)).  For an MXFP4 context the experts are those of
 * fst_synth_mxfp4_expert(seed, id_base + e, ..., e_lo = 108, e_hi = 128)
 * (d_sigma unused).  Synchronous. */
int fst_synth_experts_dev(fst_ctx* ctx, uint64_t seed, int lid, int e_first, int e_count, uint64_t id_base,
                          float d_sigma);
int fst_synth_lm_head_dev(fst_ctx* ctx, uint64_t seed, uint64_t id, float d_sigma);
int fst_synth_mxfp4_expert(uint64_t seed, uint64_t expert_id, int hd, int inter, int e_lo,
                           int e_hi, uint8_t* out);
/* n values ~ N(mean, std) rounded to bf16 / kept fp32. */
int fst_synth_normal_bf16(uint64_t seed, uint64_t stream, size_t n, float mean, float std,
                          uint16_t* out);
int fst_synth_normal_f32(uint64_t seed, uint64_t stream, size_t n, float mean, float std, float* out);

/* ---- on-disk .fst model file (expert bank + shared tensors) ----
 * Reader for the file written by scripts/fst_converter.py (convert_to_fst,
 * :718-776) and read by ExpertPager (src/expert_pager.cpp:88-130, :265-290)
 * and FSTEngine::load_shared_weights (src/fst_engine.cpp:1500-1760).
 * Layout (little-endian): a 128-byte header (fst_bank_header fields in file
 * order, HEADER_FMT "<4sIIIIIIIIIIIQffQQQQQQQQ", :169), a directory of 64-byte
 * tensor entries (SHARED_ENTRY_FMT "<IHHHHIQQQQQQ"), page-aligned tensor data,
 * and the expert bank: expert (l, e) at expert_bank_offset +
 * (l * n_experts + e) * expert_block_stride, expert_block_bytes long, dense
 * MXFP4 gate|up|down (17-byte blocks; the fst_upload_expert MXFP4 layout).
 * The bank functions need no GPU. */
typedef struct fst_bank fst_bank;
typedef struct fst_bank_header {
    char magic[4];                 /* "FST\0" */
    uint32_t version, hidden_dim, n_layers, n_experts, top_k, n_q_heads, n_kv_heads, head_dim, inter_dim,
        n_shared, reserved0;
    uint64_t vocab_size;
    float rms_eps, rope_freq_base;
    uint64_t shared_dir_offset, shared_dir_count, expert_bank_offset, expert_block_bytes, expert_block_stride,
        expert_count;
    uint64_t dspark; /* block_size | markov_rank << 16 */
    uint64_t dspark_noise_token_id;
} fst_bank_header;
typedef struct fst_bank_tensor {
    uint32_t tid;                  /* TID_* of scripts/fst_converter.py:116-160 */
    uint16_t lid;                  /* layer, 0xFFFF = global */
    uint16_t sid, qtype, ndim;     /* qtype: 1 Q8_0, 2 BF16, 3 F32 */
    uint64_t shape[3];             /* padded with 1 */
    uint64_t offset, size;         /* bytes in the file */
} fst_bank_tensor;
enum {
    FST_TID_OUTPUT_NORM = 1, FST_TID_LM_HEAD = 2, FST_TID_INPUT_NORM = 3, FST_TID_POST_ATTN_NORM = 4,
    FST_TID_ROUTER = 9, FST_TID_ROUTER_BIAS = 10, FST_TID_SHARED_GATE = 11, FST_TID_SHARED_UP = 12,
    FST_TID_SHARED_DOWN = 13, FST_TID_HC_FFN_FN = 26, FST_TID_HC_FFN_SCALE = 27, FST_TID_HC_FFN_BASE = 28,
    FST_TID_HC_HEAD_FN = 29, FST_TID_HC_HEAD_SCALE = 30, FST_TID_HC_HEAD_BASE = 31
};
/* Opens and validates the file: magic, directory and every tensor and expert
 * inside the file. */
int fst_bank_open(const char* path, fst_bank** out);
void fst_bank_close(fst_bank* b);
int fst_bank_get_header(const fst_bank* b, fst_bank_header* out);
int fst_bank_n_tensors(const fst_bank* b);
int fst_bank_tensor_at(const fst_bank* b, int i, fst_bank_tensor* out);
/* The entry with this tid and layer (lid = -1: the first entry with the tid);
 * FST_ENOTREADY if absent. */
int fst_bank_find(const fst_bank* b, uint32_t tid, int lid, fst_bank_tensor* out);
/* Raw bytes of a tensor (bytes == t->size). */
int fst_bank_read_tensor(const fst_bank* b, const fst_bank_tensor* t, void* dst, size_t bytes);
/* Expert (lid, eid) as stored (bytes == expert_block_bytes); ExpertPager::load_from_disk. */
int fst_bank_read_expert(const fst_bank* b, int lid, int eid, void* dst, size_t bytes);
/* A context configuration for the file: geometry from the header, MXFP4
 * codec, and the engine's fixed DeepSeek-V4 router settings
 * (src/fst_engine.cpp:1506-1526, include/fst_engine.h:138-144): sqrt(softplus)
 * scores, route_scale 1.5, 3 hash layers, bf16-rounded logits, no SwiGLU clamp
 * (the NPU FFN applies none). */
int fst_bank_config(const fst_bank* b, fst_config* cfg);
enum {
    FST_BANK_EXPERTS = 1,   /* routed experts -> fst_upload_expert */
    FST_BANK_ROUTER = 2,    /* TID 9 [E][hidden] (+ TID 10 bias) -> router */
    FST_BANK_NORM = 4,      /* TID 4 moe norm (absent: ones, as the engine) */
    FST_BANK_SHARED = 8,    /* TID 11-13 -> fst_upload_shared_bf16 */
    FST_BANK_HC = 16,       /* TID 26-28 -> fst_upload_hc (when present) */
    FST_BANK_HASH = 32,     /* <path>.tid2eid sidecar rows of the layer (when present, lid < n_hash_layers) */
    FST_BANK_LAYER_ALL = 63,
    FST_BANK_BIAS_AS_FP16 = 256  /* read a 2-byte bias as fp16, as the engine does (:1626-1630) */
};
/* Loads layer lid of the file into the context (flags above). */
int fst_bank_load_layer(fst_ctx* ctx, const fst_bank* b, int lid, int flags);
enum { FST_BANK_HEAD_NORM = 1, FST_BANK_HEAD_LM = 2, FST_BANK_HEAD_HC = 4, FST_BANK_HEAD_ALL = 7 };
/* Output norm (TID 1), bf16 LM head (TID 2), HC head (TID 29-31, when present). */
int fst_bank_load_head(fst_ctx* ctx, const fst_bank* b, int flags);

#ifdef __cplusplus
}
#endif
#endif
