// fst_engine_hip.h — FSTEngine-shaped C++ adapter over the C-ABI in fst_hip.h.
//
// The reference engine's verify path is driven through four private members
// of FSTEngine (include/fst_engine.h) and an inline acceptance block:
//
//   npu_router            include/fst_engine.h:413   src/fst_engine.cpp:936-1076
//   process_expert_ffn    include/fst_engine.h:318   src/fst_engine.cpp:4068-4371
//   process_shared_expert include/fst_engine.h:319   src/fst_engine.cpp:4373-4489
//   accept/reject         src/fst_engine.cpp:6021-6063 (inline in generate_dspark)
//   apply_final_norm_and_lm_head include/fst_engine.h:276 src/fst_engine.cpp:2115-2160
//   sample_token          include/fst_engine.h:277   src/fst_engine.cpp:4491-4528
//   process_layer (FFN half, non-HC residual) include/fst_engine.h:308
//                         src/fst_engine.cpp:2734-2917
//
// FSTEngineHip keeps those member signatures, argument meanings and buffer
// layouts (bf16_t = uint16_t host buffers, row-major [M][hidden], token-major
// eids/wts) so process_layer / generate_dspark can call it unchanged, and
// reports failures the way the reference does: by throwing
// std::runtime_error.  Weights are uploaded once per (layer, expert) and stay
// resident in HBM; there is no per-call paging or host accumulation.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "fst_hip.h"

using bf16_t = uint16_t;

namespace fst_hip {

class FSTEngineHip {
public:
    explicit FSTEngineHip(const fst_config& cfg) : cfg_(cfg) {
        check(fst_create(&cfg_, &ctx_), "fst_create");
        router_src_.assign(cfg_.n_layers, nullptr);
        bias_src_.assign(cfg_.n_layers, nullptr);
    }
    ~FSTEngineHip() { fst_destroy(ctx_); }
    FSTEngineHip(const FSTEngineHip&) = delete;
    FSTEngineHip& operator=(const FSTEngineHip&) = delete;

    fst_ctx* handle() const { return ctx_; }
    const fst_config& config() const { return cfg_; }

    // Residency (replaces get_expert_bo / ExpertPager, src/fst_engine.cpp:3892-3926).
    // eid == n_experts uploads the layer's shared expert.
    void upload_expert(int lid, int eid, const void* packed, size_t bytes) {
        check(fst_upload_expert(ctx_, lid, eid, packed, bytes), "fst_upload_expert");
    }
    void upload_router(int lid, const float* router_weights, const float* router_bias) {
        check(fst_upload_router_f32(ctx_, lid, router_weights, router_bias), "fst_upload_router_f32");
        router_src_[lid] = router_weights;
        bias_src_[lid] = router_bias;
    }
    void upload_hash_table(int lid, const int32_t* tid2eid) {
        check(fst_upload_hash_table(ctx_, lid, tid2eid), "fst_upload_hash_table");
    }

    // include/fst_engine.h:413.  router_weights is [hd][n_experts] fp32 as in
    // the reference; it is converted to bf16 (RNE) and kept resident the first
    // time a layer sees a given weight pointer instead of on every call
    // (src/fst_engine.cpp:944-945 converts per call).
    void npu_router(int* eids, float* wts, const bf16_t* hidden, const float* router_weights,
                    const float* router_bias, int M, int n_experts, int top_k, int hd, int lid,
                    const int* input_ids) {
        if (n_experts != cfg_.n_experts || top_k != cfg_.top_k || hd != cfg_.hidden_dim)
            throw std::runtime_error("npu_router: shape does not match the engine configuration");
        if (lid < 0 || lid >= cfg_.n_layers) throw std::runtime_error("npu_router: layer id out of range");
        if (router_weights != router_src_[lid] || router_bias != bias_src_[lid])
            upload_router(lid, router_weights, router_bias);
        check(fst_router(ctx_, lid, hidden, M, input_ids, eids, wts), "fst_router");
    }

    // include/fst_engine.h:318: out = bf16( sum_j r_weights[m][j] * FFN_{eids[m][j]}(h[m]) ).
    void process_expert_ffn(int lid, const bf16_t* h, bf16_t* out, int M, const int* eids, int tk,
                            const float* r_weights) {
        check(fst_expert_ffn(ctx_, lid, h, out, M, eids, tk, r_weights), "fst_expert_ffn");
    }

    // include/fst_engine.h:319: out = bf16( FFN_shared(h[m]) ).
    void process_shared_expert(int lid, const bf16_t* h, bf16_t* out, int M) {
        check(fst_shared_expert(ctx_, lid, h, out, M), "fst_shared_expert");
    }

    // src/fst_engine.cpp:2826-2852 as one device chain: router -> routed ->
    // shared -> combine (mn = bf16(routed + shared)), eids/wts optional.
    void moe_layer(int lid, const bf16_t* mn, bf16_t* out, int M, const int* input_ids, int* eids = nullptr,
                   float* wts = nullptr) {
        check(fst_moe_layer(ctx_, lid, mn, M, input_ids, out, eids, wts), "fst_moe_layer");
    }

    // src/fst_engine.cpp:6021-6063 extracted: target_logits [k+1][V] (row m =
    // main-model logits after verify position m), draft [k].  Writes the
    // emitted tokens (accepted drafts then the bonus) and returns n_accepted.
    int accept_block(const float* target_logits, int k, int V, const int* draft, std::vector<int>* emitted) {
        int32_t n_acc = 0;
        std::vector<int32_t> tok(k + 1);
        check(fst_accept_greedy(ctx_, target_logits, 1, k, V, draft, &n_acc, tok.data()), "fst_accept_greedy");
        if (emitted) emitted->assign(tok.begin(), tok.begin() + n_acc + 1);
        return n_acc;
    }

    // include/fst_engine.h:276 (src/fst_engine.cpp:2115-2160): logits[M][vocab]
    // = LMHead(RMSNorm_final(plain)).  As in the reference, hidden_state is the
    // 4-stream HC residual [M][4][hidden] once the HC head is uploaded
    // (upload_hc_head), collapsed by output_hc_head first (:2120-2128); without
    // an HC head it is a plain [M][hidden].  The final norm weights go in with
    // upload_norm(n_layers, w), the head with upload_lm_head.  The device
    // buffers belong to the context: nothing is allocated per call.
    void apply_final_norm_and_lm_head(bf16_t* hidden_state, int M, float* logits) {
        check(fst_final_head(ctx_, hidden_state, M, logits), "apply_final_norm_and_lm_head");
    }
    void upload_hc_head(const bf16_t* fn, float scale, const float* base) {
        check(fst_upload_hc_head(ctx_, fn, scale, base), "fst_upload_hc_head");
    }

    // include/fst_engine.h:277 (src/fst_engine.cpp:4491-4528): temperature <= 0
    // is the argmax; otherwise softmax(logits/T), top-p, one draw.  The draw is
    // reproducible: Philox keyed by (sample seed, call number) instead of the
    // reference's unseeded std::mt19937 (fst_sample_token gives the exact
    // fixed-point definition).  logits are left unchanged (the reference
    // overwrites them with probabilities; its callers do not read them again).
    int sample_token(float* logits, int vocab_size, float temperature, float top_p) {
        int32_t tok = 0;
        check(fst_sample_token(ctx_, logits, vocab_size, temperature, top_p, sample_seed_, sample_calls_++, &tok),
              "fst_sample_token");
        return tok;
    }
    void set_sample_seed(uint64_t seed) {
        sample_seed_ = seed;
        sample_calls_ = 0;
    }

    // The FFN half of process_layer without HC (src/fst_engine.cpp:2738-2741,
    // :2826-2852, :2913-2917) for every layer, then the final norm and head:
    // h = h + MoE_l(RMSNorm_l(h)) for l < n_layers; logits = LMHead(RMSNorm(h)).
    void verify_forward(bf16_t* h, int M, const int* input_ids, float* logits) {
        check(fst_verify_forward(ctx_, h, M, input_ids, logits), "fst_verify_forward");
    }
    void upload_norm(int lid, const bf16_t* w) { check(fst_upload_norm(ctx_, lid, w), "fst_upload_norm"); }
    void upload_lm_head(const void* packed, size_t bytes) {
        check(fst_upload_lm_head(ctx_, packed, bytes), "fst_upload_lm_head");
    }

    // Rejection-sampling variant (no counterpart in the reference, which only
    // accepts greedily); draft_logits [k][V], deterministic in (seed, seq).
    int accept_block_stochastic(const float* target_logits, const float* draft_logits, int k, int V,
                                const int* draft, float temperature, uint64_t seed, uint64_t seq,
                                std::vector<int>* emitted) {
        int32_t n_acc = 0;
        std::vector<int32_t> tok(k + 1);
        check(fst_accept_stochastic(ctx_, target_logits, draft_logits, 1, k, V, draft, temperature, seed, seq,
                                    &n_acc, tok.data()),
              "fst_accept_stochastic");
        if (emitted) emitted->assign(tok.begin(), tok.begin() + n_acc + 1);
        return n_acc;
    }

private:
    static void check(int rc, const char* what) {
        if (rc != FST_OK) throw std::runtime_error(std::string(what) + ": " + fst_last_error());
    }

    fst_config cfg_;
    fst_ctx* ctx_ = nullptr;
    std::vector<const float*> router_src_, bias_src_;
    uint64_t sample_seed_ = 0x5eed5eedull, sample_calls_ = 0;
};

}  // namespace fst_hip
