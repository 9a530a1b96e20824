// Drives the FSTEngine-shaped adapter (include/fst_engine_hip.h) the way the
// reference's process_layer / generate_dspark call the engine members.
//   adapter_check cpu : no GPU visible -> construction must throw runtime_error
//   adapter_check gpu : small layer end to end, cross-checked between members
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "fst_engine_hip.h"

static float bf(uint16_t v) {
    uint32_t b = (uint32_t)v << 16;
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

int main(int argc, char** argv) {
    const bool gpu = argc > 1 && std::strcmp(argv[1], "gpu") == 0;
    fst_config cfg;
    fst_config_default(&cfg);
    cfg.n_experts = 4;
    cfg.top_k = 2;
    cfg.max_tokens = 16;
    if (!gpu) {
        try {
            fst_hip::FSTEngineHip eng(cfg);
            std::printf("unexpected: engine constructed without a GPU\n");
            return 1;
        } catch (const std::runtime_error& e) {
            std::printf("ADAPTER CPU OK: %s\n", e.what());
            return std::strstr(e.what(), "fst_create") ? 0 : 1;
        }
    }
    fst_hip::FSTEngineHip eng(cfg);
    const int hd = cfg.hidden_dim, E = cfg.n_experts, tk = cfg.top_k, M = 4;
    std::vector<uint8_t> expert(fst_expert_bytes(&cfg));
    for (int e = 0; e <= E; ++e) {
        fst_synth_q4k_expert(99, e, hd, cfg.inter_dim, 0.01f, expert.data());
        eng.upload_expert(0, e, expert.data(), expert.size());
    }
    std::vector<float> rw((size_t)hd * E);
    fst_synth_normal_f32(99, 7, rw.size(), 0.0f, 0.02f, rw.data());
    std::vector<uint16_t> h((size_t)M * hd), routed(h.size()), shared(h.size()), fused(h.size());
    fst_synth_normal_bf16(99, 8, h.size(), 0.0f, 1.0f, h.data());
    std::vector<int> eids(M * tk), eids2(M * tk);
    std::vector<float> wts(M * tk), wts2(M * tk);
    // src/fst_engine.cpp:2826-2852 call order
    eng.npu_router(eids.data(), wts.data(), h.data(), rw.data(), nullptr, M, E, tk, hd, 0, nullptr);
    eng.process_expert_ffn(0, h.data(), routed.data(), M, eids.data(), tk, wts.data());
    eng.process_shared_expert(0, h.data(), shared.data(), M);
    eng.moe_layer(0, h.data(), fused.data(), M, nullptr, eids2.data(), wts2.data());
    if (eids != eids2 || wts != wts2) {
        std::printf("router mismatch between npu_router and moe_layer\n");
        return 1;
    }
    double num = 0, den = 0;
    for (size_t i = 0; i < h.size(); ++i) {
        const double ref = (double)bf(routed[i]) + (double)bf(shared[i]);
        num += (bf(fused[i]) - ref) * (bf(fused[i]) - ref);
        den += ref * ref;
    }
    const double rel = std::sqrt(num / den);
    // accept_block on planted logits: rows 0..2 match the draft, row 3 does not
    const int k = 5, V = 1000;
    std::vector<float> logits((size_t)(k + 1) * V, 0.0f);
    std::vector<int> draft = {11, 22, 33, 44, 55};
    for (int i = 0; i <= k; ++i) logits[(size_t)i * V + (i < 3 ? draft[i] : 700 + i)] = 5.0f;
    std::vector<int> emitted;
    const int n = eng.accept_block(logits.data(), k, V, draft.data(), &emitted);
    const bool acc_ok = n == 3 && emitted.size() == 4 && emitted[0] == 11 && emitted[2] == 33 && emitted[3] == 703;
    bool threw = false;
    try {
        eng.npu_router(eids.data(), wts.data(), h.data(), rw.data(), nullptr, M, E + 1, tk, hd, 0, nullptr);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    // apply_final_norm_and_lm_head (include/fst_engine.h:276) on a small head:
    // one logit row recomputed here from the GPU dequant of the same blocks
    // and a double-precision RMSNorm must agree to 1e-2
    double head_rel = 1.0;
    bool hc_equal = false, sample_ok = false;
    {
        fst_config c2 = cfg;
        c2.vocab_size = 256;
        fst_hip::FSTEngineHip head(c2);
        std::vector<uint16_t> nw(hd);
        fst_synth_normal_bf16(99, 9, nw.size(), 1.0f, 0.1f, nw.data());
        head.upload_norm(c2.n_layers, nw.data());
        std::vector<uint8_t> lm(fst_lm_head_bytes(&c2));
        fst_synth_q4k_blocks(99, 12345, lm.size() / 144, 0.01f, lm.data());
        head.upload_lm_head(lm.data(), lm.size());
        std::vector<float> lg((size_t)M * c2.vocab_size);
        head.apply_final_norm_and_lm_head(h.data(), M, lg.data());
        std::vector<float> wf(lm.size() / 144 * 256);
        if (fst_dequant(head.handle(), FST_CODEC_Q4K, lm.data(), lm.size() / 144, wf.data(), nullptr) != FST_OK)
            return 1;
        double ss = 0;
        for (int j = 0; j < hd; ++j) ss += (double)bf(h[j]) * bf(h[j]);
        const double r = 1.0 / std::sqrt(ss / hd + 1e-6);
        double hn = 0, hd2 = 0;
        for (int v = 0; v < c2.vocab_size; ++v) {
            double acc = 0;
            for (int j = 0; j < hd; ++j) acc += bf(h[j]) * r * bf(nw[j]) * wf[(size_t)v * hd + j];
            hn += (lg[v] - acc) * (lg[v] - acc);
            hd2 += acc * acc;
        }
        head_rel = std::sqrt(hn / hd2);

        // with the HC head uploaded the input is the 4-stream residual
        // [M][4][hd] (src/fst_engine.cpp:2120-2128): the logits must equal
        // output_hc_head -> final norm -> head run piece by piece on the device
        std::vector<uint16_t> fn((size_t)4 * 4 * hd), hs((size_t)M * 4 * hd);
        fst_synth_normal_bf16(99, 13, fn.size(), 0.0f, 0.02f, fn.data());
        fst_synth_normal_bf16(99, 14, hs.size(), 0.0f, 1.0f, hs.data());
        const float base[4] = {0.1f, -0.2f, 0.3f, 0.0f};
        head.upload_hc_head(fn.data(), 0.5f, base);
        std::vector<float> lg_hc((size_t)M * c2.vocab_size), lg_ref(lg_hc.size());
        head.apply_final_norm_and_lm_head(hs.data(), M, lg_hc.data());
        fst_ctx* hc = head.handle();
        void* d_hs = fst_device_alloc(hc, hs.size() * 2);
        void* d_plain = fst_device_alloc(hc, (size_t)M * hd * 2);
        void* d_lg = fst_device_alloc(hc, lg_ref.size() * 4);
        int rc = fst_copy_to_device(hc, d_hs, hs.data(), hs.size() * 2);
        if (!rc) rc = fst_hc_head_dev(hc, (const uint16_t*)d_hs, M, (uint16_t*)d_plain);
        if (!rc) rc = fst_lm_head_dev(hc, (const uint16_t*)d_plain, M, (float*)d_lg);
        if (!rc) rc = fst_copy_to_host(hc, lg_ref.data(), d_lg, lg_ref.size() * 4);
        fst_device_free(hc, d_hs);
        fst_device_free(hc, d_plain);
        fst_device_free(hc, d_lg);
        hc_equal = rc == FST_OK && std::memcmp(lg_hc.data(), lg_ref.data(), lg_ref.size() * 4) == 0;

        // sample_token (include/fst_engine.h:277): argmax at temperature 0,
        // and the seeded draw equals fst_sample_token with (seed, call number)
        std::vector<float> row(lg_hc.begin(), lg_hc.begin() + c2.vocab_size);
        int am = 0;
        for (int v = 1; v < c2.vocab_size; ++v)
            if (row[v] > row[am]) am = v;
        head.set_sample_seed(4242);
        const int t0 = head.sample_token(row.data(), c2.vocab_size, 0.0f, 0.9f);
        const int t1 = head.sample_token(row.data(), c2.vocab_size, 1.0f, 0.9f);
        int32_t r1 = -1;
        if (fst_sample_token(hc, row.data(), c2.vocab_size, 1.0f, 0.9f, 4242, 1, &r1) != FST_OK) return 1;
        sample_ok = t0 == am && t1 == r1 && t1 >= 0 && t1 < c2.vocab_size;
    }
    const bool ok = rel < 1e-2 && acc_ok && threw && head_rel < 1e-2 && hc_equal && sample_ok;
    std::printf("ADAPTER GPU %s: combine rel=%.3e accept n=%d threw_on_bad_shape=%d lm_head rel=%.3e "
                "hc_head_equal=%d sample_ok=%d\n",
                ok ? "OK" : "FAIL", rel, n, (int)threw, head_rel, (int)hc_equal, (int)sample_ok);
    return ok ? 0 : 1;
}
