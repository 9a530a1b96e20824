// fst_api.cpp — host runtime behind include/fst_hip.h.
//
// A context owns one HIP stream, the resident expert banks of every layer,
// the router weights, and device scratch sized for max_tokens.  Every MoE call
// is a fixed chain of launches on that stream (router -> bucket -> prep ->
// gate/up -> prep -> down -> combine) with no host synchronisation inside;
// host-pointer entry points add one H2D copy, one D2H copy and one sync.
#include <cstdlib>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/fst_exact_math.h"
#include "../../include/fst_hip.h"
#include "fst_internal.h"

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

#define FST_HIP_TRY(expr)                                                                         \
    do {                                                                                          \
        hipError_t e_ = (expr);                                                                   \
        if (e_ != hipSuccess)                                                                     \
            return fail(FST_EHIP, std::string(#expr " failed: ") + hipGetErrorString(e_));       \
    } while (0)

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

}  // namespace

struct fst_ctx {
    fst_config cfg{};
    hipStream_t st = nullptr;
    fst::Geometry geo{};
    size_t expert_bytes = 0, expert_stride = 0;
    uint8_t* bank = nullptr;                 // [L][E+1] experts
    std::vector<std::vector<char>> uploaded; // [L][E+1]
    std::vector<int> n_uploaded;             // [L]
    uint16_t* router = nullptr;              // [L][E][hd]
    float* bias = nullptr;                   // [L][E]
    std::vector<char> has_router, has_bias;
    std::vector<int32_t*> hash;              // [L] (lid < n_hash_layers)
    uint16_t* norms = nullptr;               // [L+1][hd] bf16 (moe norms, then the final norm)
    std::vector<char> has_norm;              // [L+1]
    uint8_t* lm_head = nullptr;              // [vocab][hd/256] Q4_K, device layout
    uint16_t* lm_head16 = nullptr;           // [vocab][hd] bf16 (checkpoint layout)
    int lm_kind = 0;                         // LM head in use: 0 none, 1 Q4_K, 2 bf16
    std::vector<uint16_t*> shared16;         // [L] bf16 shared expert: gate [inter][hd], up, down [hd][inter]
    int* lm_tab = nullptr;                   // one-slot table for the dense LM-head call
    uint16_t* mn = nullptr;                  // [T][hd] normed layer input
    // Hyper-Connections (4-stream residual)
    uint16_t* hc_fn = nullptr;               // [L][24][4 hd] bf16 (checkpoint layout)
    float* hc_sb = nullptr;                  // [L][3 + 24] scale, base
    std::vector<char> has_hc;                // [L]
    uint16_t* hc_head_fn = nullptr;          // [4][4 hd]
    float* hc_head_base = nullptr;           // [4]
    float hc_head_scale = 1.0f;
    bool has_hc_head = false;
    uint16_t* hc_cur = nullptr;              // [T][hd]
    float* hc_post = nullptr;                // [T][4]
    float* hc_comb = nullptr;                // [T][16]
    uint16_t* hc_h = nullptr;                // [T][4][hd] host-call staging
    bool nested = false;                     // inside verify_forward: no per-kernel marks
    fst::Scratch s{};
    uint32_t fused_epoch = 0;                // fused MoE launches issued (tags of their h words)
    // verify forward: the next layer's residual + RMSNorm folded into this
    // layer's combine (run_moe sets folded when it did so)
    uint16_t* fold_h = nullptr;
    const uint16_t* fold_w = nullptr;
    uint16_t* fold_mn = nullptr;
    bool folded = false;
    bool fused = true;                       // use the fused launch where it applies
    bool gemv = true;                        // use the small-M launch where it applies
    std::vector<void*> allocs;
    std::vector<uint8_t> staging;            // host repack buffer for expert uploads
    // acceptance staging (grown on demand)
    void* acc_ws = nullptr;
    size_t acc_ws_cap = 0;
    int acc_ws_nseq = -1, acc_ws_k = -1;  // shape whose counter layout the workspace holds
    uint32_t acc_epoch = 0;                  // greedy words of acc_ws: epoch of the last call
    int spin_limit = fst::kDefaultSpinLimit; // polls before a cross-workgroup wait gives up
    int max_grid_y = 65535;                  // device grid limit (acceptance rows)
    float* acc_logits = nullptr;
    size_t acc_logits_cap = 0;
    int32_t* acc_io = nullptr;
    size_t acc_io_cap = 0;
    float* head_logits = nullptr;            // [T][vocab] logits of the host-pointer final head
    size_t head_logits_cap = 0;
    void* samp_ws = nullptr;                 // sample_token: fixed-point masses [rows][V]
    size_t samp_ws_cap = 0;
    // profiling
    bool profiling = false;
    std::vector<hipEvent_t> ev;
    std::vector<const char*> ev_names;
    int n_ev = 0;
    fst_timings last{};
    // kernel ring: start/stop event pairs taken by the dominant launch of
    // consecutive calls (no synchronisation until read)
    std::vector<hipEvent_t> kev;
    int kev_n = 0;
    int kev_cap = 0;  // launches the ring records (its events may be more)
    bool kring = false;

    ~fst_ctx() {
        if (st) (void)hipStreamSynchronize(st);
        for (void* p : allocs) (void)hipFree(p);
        for (int32_t* p : hash)
            if (p) (void)hipFree(p);
        if (lm_head) (void)hipFree(lm_head);
        if (lm_head16) (void)hipFree(lm_head16);
        for (uint16_t* p : shared16)
            if (p) (void)hipFree(p);
        if (acc_ws) (void)hipFree(acc_ws);
        if (acc_logits) (void)hipFree(acc_logits);
        if (acc_io) (void)hipFree(acc_io);
        if (samp_ws) (void)hipFree(samp_ws);
        if (head_logits) (void)hipFree(head_logits);
        for (hipEvent_t e : ev) (void)hipEventDestroy(e);
        for (hipEvent_t e : kev) (void)hipEventDestroy(e);
        if (st) (void)hipStreamDestroy(st);
    }

    template <typename T>
    int dalloc(T** p, size_t count) {
        void* q = nullptr;
        size_t bytes = std::max<size_t>(256, count * sizeof(T));
        hipError_t e = hipMalloc(&q, bytes);
        if (e != hipSuccess)
            return fail(FST_ENOMEM, "hipMalloc(" + std::to_string(bytes) + ") failed: " + hipGetErrorString(e));
        allocs.push_back(q);
        *p = static_cast<T*>(q);
        return FST_OK;
    }

    fst::LayerView layer(int lid) const {
        fst::LayerView L;
        L.bank = bank + (size_t)lid * (cfg.n_experts + 1) * expert_stride;
        L.expert_stride = expert_stride;
        L.router_nk = router + (size_t)lid * cfg.n_experts * cfg.hidden_dim;
        L.router_bias = has_bias[lid] ? bias + (size_t)lid * cfg.n_experts : nullptr;
        L.hash = hash[lid];
        return L;
    }

    // profiling marks: mark(name) after a launch closes the interval opened by the previous mark
    void mark_begin() {
        if (nested) return;
        n_ev = 0;
        if (!profiling) return;
        (void)hipEventRecord(ev[0], st);
        n_ev = 1;
    }
    void mark(const char* name, bool outer = false) {
        if ((nested && !outer) || !profiling || n_ev >= (int)ev.size()) return;
        (void)hipEventRecord(ev[n_ev], st);
        ev_names[n_ev] = name;
        ++n_ev;
    }
    void collect() {
        last.n = 0;
        if (!profiling || n_ev < 2) return;
        (void)hipEventSynchronize(ev[n_ev - 1]);
        for (int i = 1; i < n_ev && last.n < 16; ++i) {
            float ms = 0.0f;
            (void)hipEventElapsedTime(&ms, ev[i - 1], ev[i]);
            last.name[last.n] = ev_names[i];
            last.ms[last.n] = ms;
            ++last.n;
        }
    }
};

namespace fst {
int set_error(int code, const char* msg) { return fail(code, msg); }
}  // namespace fst

extern "C" {

void fst_config_default(fst_config* c) {
    if (!c) return;
    std::memset(c, 0, sizeof(*c));
    c->hidden_dim = 4096;
    c->inter_dim = 2048;
    c->n_experts = 256;
    c->top_k = 6;
    c->n_layers = 1;
    c->max_tokens = 64;
    c->codec = FST_CODEC_Q4K;
    c->has_shared = 1;
    c->score_func = FST_SCORE_SIGMOID;
    c->route_scale = 1.0f;
    c->round_logits_bf16 = 0;
    c->n_hash_layers = 0;
    c->vocab_size = 129280;
    c->swiglu_limit = 0.0f;
    c->device = 0;
}

const char* fst_last_error(void) { return g_err.c_str(); }
int fst_abi_version(void) { return FST_ABI_VERSION; }

size_t fst_expert_bytes(const fst_config* c) {
    if (!c) return 0;
    const size_t w = (size_t)c->hidden_dim * c->inter_dim;
    if (c->codec == FST_CODEC_Q4K) return 3 * (w / 256) * 144;
    if (c->codec == FST_CODEC_MXFP4) return 3 * (w / 32) * 17;
    return 0;
}

int fst_create(const fst_config* cfg, fst_ctx** out) {
    if (!cfg || !out) return fail(FST_EINVAL, "fst_create: null argument");
    *out = nullptr;
    const fst_config& c = *cfg;
    if (c.codec != FST_CODEC_Q4K && c.codec != FST_CODEC_MXFP4)
        return fail(FST_EINVAL, "fst_create: codec must be FST_CODEC_Q4K or FST_CODEC_MXFP4");
    if (c.hidden_dim <= 0 || c.hidden_dim % 512 || c.inter_dim <= 0 || c.inter_dim % 512)
        return fail(FST_EINVAL, "fst_create: hidden_dim and inter_dim must be multiples of 512");
    if (c.hidden_dim > 8192 || c.inter_dim > 8192)
        return fail(FST_EINVAL, "fst_create: hidden_dim and inter_dim must be <= 8192");

    if (c.n_experts <= 0 || c.n_experts > 1024)
        return fail(FST_EINVAL, "fst_create: n_experts must be in [1, 1024]");
    if (c.top_k <= 0 || c.top_k > fst::kMaxTopK || c.top_k > c.n_experts)
        return fail(FST_EINVAL, "fst_create: top_k must be in [1, min(16, n_experts)]");
    if (c.max_tokens <= 0 || c.max_tokens > fst::kMaxTokens)
        return fail(FST_EINVAL, "fst_create: max_tokens must be in [1, 64]");
    if (c.n_layers <= 0) return fail(FST_EINVAL, "fst_create: n_layers must be >= 1");
    if (c.score_func != FST_SCORE_SIGMOID && c.score_func != FST_SCORE_SQRTSOFTPLUS)
        return fail(FST_EINVAL, "fst_create: unknown score_func");
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
        return fail(FST_ENODEV, "fst_create: no HIP device");
    if (c.device < 0 || c.device >= ndev) return fail(FST_ENODEV, "fst_create: device ordinal out of range");
    FST_HIP_TRY(hipSetDevice(c.device));
    hipDeviceProp_t prop;
    FST_HIP_TRY(hipGetDeviceProperties(&prop, c.device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(FST_ENODEV, std::string("fst_create: device is ") + prop.gcnArchName + ", need gfx950");

    // the allocation-free greedy entry point's scratch address on this device
    if (int rc0 = fst::accept_scratch_init(c.device)) return rc0;

    fst_ctx* x = new fst_ctx();
    x->cfg = c;
    x->max_grid_y = prop.maxGridSize[1] > 0 ? prop.maxGridSize[1] : 65535;
    int rc = FST_OK;
    auto bail = [&](int code) {
        delete x;
        return code;
    };
    if (hipStreamCreateWithFlags(&x->st, hipStreamNonBlocking) != hipSuccess)
        return bail(fail(FST_EHIP, "hipStreamCreate failed"));
    x->geo.hd = c.hidden_dim;
    x->geo.inter = c.inter_dim;
    x->geo.E = c.n_experts;
    x->geo.tk = c.top_k;
    x->geo.codec = c.codec;
    x->geo.score_func = c.score_func;
    x->geo.round_logits_bf16 = c.round_logits_bf16;
    x->geo.route_scale = c.route_scale;
    x->geo.swiglu_limit = c.swiglu_limit;
    x->geo.vocab = c.vocab_size;
    x->expert_bytes = fst_expert_bytes(&c);
    x->expert_stride = align_up(x->expert_bytes, 4096);
    const int L = c.n_layers, E = c.n_experts, hd = c.hidden_dim, inter = c.inter_dim;
    if ((rc = x->dalloc(&x->bank, (size_t)L * (E + 1) * x->expert_stride))) return bail(rc);
    if ((rc = x->dalloc(&x->router, (size_t)L * E * hd))) return bail(rc);
    if ((rc = x->dalloc(&x->bias, (size_t)L * E))) return bail(rc);
    x->uploaded.assign(L, std::vector<char>(E + 1, 0));
    x->n_uploaded.assign(L, 0);
    x->has_router.assign(L, 0);
    x->has_bias.assign(L, 0);
    x->hash.assign(L, nullptr);
    if ((rc = x->dalloc(&x->norms, (size_t)(L + 1) * hd))) return bail(rc);
    x->has_norm.assign(L + 1, 0);
    if ((rc = x->dalloc(&x->lm_tab, fst::META_WORDS + 4))) return bail(rc);
    if ((rc = x->dalloc(&x->mn, (size_t)c.max_tokens * hd))) return bail(rc);
    if ((rc = x->dalloc(&x->hc_fn, (size_t)L * 24 * 4 * hd)) || (rc = x->dalloc(&x->hc_sb, (size_t)L * 27)) ||
        (rc = x->dalloc(&x->hc_head_fn, (size_t)4 * 4 * hd)) || (rc = x->dalloc(&x->hc_head_base, 4)) ||
        (rc = x->dalloc(&x->hc_cur, (size_t)c.max_tokens * hd)) || (rc = x->dalloc(&x->hc_post, (size_t)c.max_tokens * 4)) ||
        (rc = x->dalloc(&x->hc_comb, (size_t)c.max_tokens * 16)) ||
        (rc = x->dalloc(&x->hc_h, (size_t)c.max_tokens * 4 * hd)))
        return bail(rc);
    x->has_hc.assign(L, 0);
    x->shared16.assign(L, nullptr);

    fst::Scratch& s = x->s;
    const int T = c.max_tokens, tk = c.top_k;
    s.max_tokens = T;
    s.n_cu = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    // the fused launch's down items wait for gate||up items of other
    // workgroups, so its grid is only as large as the device holds at once
    s.fused_per_cu = fst::moe_fused_occupancy(c.codec);
    if (s.fused_per_cu < 1) x->fused = false;
    s.max_pairs = T * tk + T;
    s.max_slots = std::min(E, T * tk) + 1;
    const int P = s.max_pairs, S = s.max_slots;
    if ((rc = x->dalloc(&s.h, (size_t)T * hd)) || (rc = x->dalloc(&s.out, (size_t)T * hd)) ||
        (rc = x->dalloc(&s.out_routed, (size_t)T * hd)) || (rc = x->dalloc(&s.out_shared, (size_t)T * hd)) ||
        (rc = x->dalloc(&s.ids, T)) || (rc = x->dalloc(&s.logits, (size_t)T * E)) ||
        (rc = x->dalloc(&s.eids, (size_t)T * tk)) || (rc = x->dalloc(&s.wts, (size_t)T * tk)) ||
        (rc = x->dalloc(&s.meta, fst::META_WORDS)) || (rc = x->dalloc(&s.slot_eid, S)) ||
        (rc = x->dalloc(&s.slot_M, S)) || (rc = x->dalloc(&s.slot_off, S)) ||
        (rc = x->dalloc(&s.pair_tok, P)) || (rc = x->dalloc(&s.pair_of, (size_t)T * tk)) ||
        (rc = x->dalloc(&s.pair_shared, T)) || (rc = x->dalloc(&s.x16p, (size_t)T * hd)) ||
        (rc = x->dalloc(&s.sxp, (size_t)T * (hd / 256) * 4)) || (rc = x->dalloc(&s.xs, T)) ||
        (rc = x->dalloc(&s.act, (size_t)P * inter)) || (rc = x->dalloc(&s.a16p, (size_t)P * inter)) ||
        (rc = x->dalloc(&s.sx2p, (size_t)P * (inter / 256) * 4)) || (rc = x->dalloc(&s.xs2, P)) ||
        (rc = x->dalloc(&s.y, (size_t)P * hd)) ||
        (rc = x->dalloc(&s.sh_h16, (size_t)T * c.inter_dim)) || (rc = x->dalloc(&s.ys, (size_t)T * hd)) ||
        (rc = x->dalloc(&s.hbuf, (size_t)2 * P * inter)) ||
        (rc = x->dalloc(&s.amaxw, (size_t)P * (inter / 16))) || (rc = x->dalloc(&s.fused_claim, 64)) ||
        (rc = x->dalloc(&s.gemv_cnt, hd / 16 + 1)) || (rc = x->dalloc(&s.norm_part, (size_t)T * 64)) ||
        (rc = x->dalloc(&s.norm_cnt, T)))
        return bail(rc);
    if (hipMemsetAsync(s.hbuf, 0, sizeof(unsigned long long) * (size_t)2 * P * inter, x->st) != hipSuccess ||
        hipMemsetAsync(s.amaxw, 0, sizeof(unsigned long long) * (size_t)P * (inter / 16), x->st) != hipSuccess)
        return bail(fail(FST_EHIP, "hipMemsetAsync(hand-off words) failed"));
    if (hipMemsetAsync(s.meta, 0, sizeof(int) * fst::META_WORDS, x->st) != hipSuccess ||
        hipMemsetAsync(s.gemv_cnt, 0, sizeof(int) * (hd / 16 + 1), x->st) != hipSuccess ||
        hipMemsetAsync(s.norm_cnt, 0, sizeof(int) * T, x->st) != hipSuccess)
        return bail(fail(FST_EHIP, "hipMemsetAsync(meta) failed"));
    x->ev.resize(17);
    x->ev_names.assign(17, "");
    for (auto& e : x->ev)
        if (hipEventCreate(&e) != hipSuccess) return bail(fail(FST_EHIP, "hipEventCreate failed"));
    if (hipStreamSynchronize(x->st) != hipSuccess) return bail(fail(FST_EHIP, "hipStreamSynchronize failed"));
    *out = x;
    return FST_OK;
}

void fst_destroy(fst_ctx* ctx) { delete ctx; }

int fst_get_config(const fst_ctx* ctx, fst_config* out) {
    if (!ctx || !out) return fail(FST_EINVAL, "null argument");
    *out = ctx->cfg;
    return FST_OK;
}
void* fst_stream(fst_ctx* ctx) { return ctx ? (void*)ctx->st : nullptr; }

int fst_sync(fst_ctx* ctx) {
    if (!ctx) return fail(FST_EINVAL, "fst_sync: null context");
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    return FST_OK;
}

int fst_set_profiling(fst_ctx* ctx, int on) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    ctx->profiling = on != 0;
    return FST_OK;
}

int fst_last_timings(fst_ctx* ctx, fst_timings* out) {
    if (!ctx || !out) return fail(FST_EINVAL, "null argument");
    ctx->collect();
    *out = ctx->last;
    return FST_OK;
}

int fst_kernel_ring(fst_ctx* ctx, int capacity) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (capacity < 0 || capacity > 65536) return fail(FST_EINVAL, "capacity must be in [0, 65536]");
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    while ((int)ctx->kev.size() < 2 * capacity) {
        hipEvent_t e;
        FST_HIP_TRY(hipEventCreate(&e));
        ctx->kev.push_back(e);
    }
    ctx->kring = capacity > 0;
    ctx->kev_cap = capacity;
    ctx->kev_n = 0;
    return FST_OK;
}

int fst_kernel_ring_read(fst_ctx* ctx, float* us, int max_n, int* n) {
    if (!ctx || !n || (max_n > 0 && !us)) return fail(FST_EINVAL, "null argument");
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    const int cnt = std::min(ctx->kev_n, std::max(max_n, 0));
    for (int i = 0; i < cnt; ++i) {
        float ms = 0.0f;
        FST_HIP_TRY(hipEventElapsedTime(&ms, ctx->kev[2 * i], ctx->kev[2 * i + 1]));
        us[i] = ms * 1e3f;
    }
    *n = cnt;
    ctx->kev_n = 0;
    return FST_OK;
}

int fst_device_copy(fst_ctx* ctx, void* d_dst, const void* d_src, size_t bytes) {
    if (!ctx || !d_dst || !d_src) return fail(FST_EINVAL, "null argument");
    if (bytes % 16) return fail(FST_EINVAL, "bytes must be a multiple of 16");
    fst::launch_copy(ctx->st, d_dst, d_src, bytes);
    FST_HIP_TRY(hipGetLastError());
    return FST_OK;
}

int fst_last_active_experts(fst_ctx* ctx, int* n) {
    if (!ctx || !n) return fail(FST_EINVAL, "null argument");
    int m[fst::META_WORDS];
    FST_HIP_TRY(hipMemcpyAsync(m, ctx->s.meta, sizeof(m), hipMemcpyDeviceToHost, ctx->st));
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    *n = m[fst::META_N_ROUTED];
    return FST_OK;
}

void* fst_device_alloc(fst_ctx* ctx, size_t bytes) {
    if (!ctx) {
        fail(FST_EINVAL, "null context");
        return nullptr;
    }
    void* p = nullptr;
    if (hipMalloc(&p, std::max<size_t>(bytes, 256)) != hipSuccess) {
        fail(FST_ENOMEM, "hipMalloc(" + std::to_string(bytes) + ") failed");
        return nullptr;
    }
    return p;
}

void fst_device_free(fst_ctx* ctx, void* p) {
    if (ctx) (void)hipStreamSynchronize(ctx->st);
    if (p) (void)hipFree(p);
}

int fst_copy_to_device(fst_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx || !dst || !src) return fail(FST_EINVAL, "null argument");
    FST_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->st));
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    return FST_OK;
}

int fst_copy_to_host(fst_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx || !dst || !src) return fail(FST_EINVAL, "null argument");
    FST_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->st));
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    return FST_OK;
}

// ------------------------------------------------------------- residency

static int check_lid(fst_ctx* ctx, int lid) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (lid < 0 || lid >= ctx->cfg.n_layers) return fail(FST_EINVAL, "layer id out of range");
    return FST_OK;
}

int fst_upload_expert(fst_ctx* ctx, int lid, int eid, const void* packed, size_t bytes) {
    if (int rc = check_lid(ctx, lid)) return rc;
    if (eid < 0 || eid > ctx->cfg.n_experts) return fail(FST_EINVAL, "expert id out of range");
    if (eid == ctx->cfg.n_experts && !ctx->cfg.has_shared)
        return fail(FST_EINVAL, "config has no shared expert");
    if (!packed || bytes != ctx->expert_bytes)
        return fail(FST_EINVAL, "expert size mismatch: got " + std::to_string(bytes) + ", expected " +
                                    std::to_string(ctx->expert_bytes));
    uint8_t* dst = ctx->bank + ((size_t)lid * (ctx->cfg.n_experts + 1) + eid) * ctx->expert_stride;
    ctx->staging.resize(bytes);
    if (ctx->cfg.codec == FST_CODEC_MXFP4)
        fst::repack_mx_expert(static_cast<const uint8_t*>(packed), ctx->staging.data(), ctx->cfg.hidden_dim,
                              ctx->cfg.inter_dim);
    else
        fst::repack_q4k_expert(static_cast<const uint8_t*>(packed), ctx->staging.data(), ctx->cfg.hidden_dim,
                               ctx->cfg.inter_dim);
    FST_HIP_TRY(hipMemcpyAsync(dst, ctx->staging.data(), bytes, hipMemcpyHostToDevice, ctx->st));
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    if (!ctx->uploaded[lid][eid]) {
        ctx->uploaded[lid][eid] = 1;
        ctx->n_uploaded[lid]++;
    }
    return FST_OK;
}

void* fst_expert_device_ptr(fst_ctx* ctx, int lid, int eid) {
    if (!ctx || lid < 0 || lid >= ctx->cfg.n_layers || eid < 0 || eid > ctx->cfg.n_experts) return nullptr;
    return ctx->bank + ((size_t)lid * (ctx->cfg.n_experts + 1) + eid) * ctx->expert_stride;
}

// Device layout of one layer's router: per expert, the hd bf16 weights
// in 16-byte pieces, piece i of lane j's K/64 chunk (elements
// [j*hd/64 + 8i, +8)) at piece index 64 i + j, so that the router kernel's
// per-lane chunk loads are contiguous across the wave.
static std::vector<uint16_t> router_interleave(const std::vector<uint16_t>& nk, int E, int hd) {
    const int nv = hd / 512;
    std::vector<uint16_t> il(nk.size());
    for (int e = 0; e < E; ++e) {
        const uint16_t* src = nk.data() + (size_t)e * hd;
        uint16_t* dst = il.data() + (size_t)e * hd;
        for (int j = 0; j < 64; ++j)
            for (int i = 0; i < nv; ++i)
                std::memcpy(dst + (size_t)(i * 64 + j) * 8, src + (size_t)(j * nv + i) * 8, 16);
    }
    return il;
}

static int upload_router_common(fst_ctx* ctx, int lid, const std::vector<uint16_t>& nk_rows, const float* bias) {
    const int E = ctx->cfg.n_experts, hd = ctx->cfg.hidden_dim;
    const std::vector<uint16_t> nk = router_interleave(nk_rows, E, hd);
    FST_HIP_TRY(hipMemcpyAsync(ctx->router + (size_t)lid * E * hd, nk.data(), nk.size() * 2,
                               hipMemcpyHostToDevice, ctx->st));
    if (bias)
        FST_HIP_TRY(hipMemcpyAsync(ctx->bias + (size_t)lid * E, bias, sizeof(float) * E, hipMemcpyHostToDevice,
                                   ctx->st));
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    ctx->has_router[lid] = 1;
    ctx->has_bias[lid] = bias != nullptr;
    return FST_OK;
}

int fst_upload_router_bf16(fst_ctx* ctx, int lid, const uint16_t* w_kn, const float* bias) {
    if (int rc = check_lid(ctx, lid)) return rc;
    if (!w_kn) return fail(FST_EINVAL, "null router weights");
    const int E = ctx->cfg.n_experts, hd = ctx->cfg.hidden_dim;
    std::vector<uint16_t> nk((size_t)E * hd);
    for (int k = 0; k < hd; ++k)
        for (int e = 0; e < E; ++e) nk[(size_t)e * hd + k] = w_kn[(size_t)k * E + e];
    return upload_router_common(ctx, lid, nk, bias);
}

int fst_upload_router_f32(fst_ctx* ctx, int lid, const float* w_kn, const float* bias) {
    if (int rc = check_lid(ctx, lid)) return rc;
    if (!w_kn) return fail(FST_EINVAL, "null router weights");
    const int E = ctx->cfg.n_experts, hd = ctx->cfg.hidden_dim;
    std::vector<uint16_t> nk((size_t)E * hd);
    for (int k = 0; k < hd; ++k)
        for (int e = 0; e < E; ++e) nk[(size_t)e * hd + k] = fst_f32_to_bf16(w_kn[(size_t)k * E + e]);
    return upload_router_common(ctx, lid, nk, bias);
}

int fst_upload_hash_table(fst_ctx* ctx, int lid, const int32_t* tid2eid) {
    if (int rc = check_lid(ctx, lid)) return rc;
    if (lid >= ctx->cfg.n_hash_layers) return fail(FST_EINVAL, "layer is not a hash-routing layer");
    if (!tid2eid || ctx->cfg.vocab_size <= 0) return fail(FST_EINVAL, "null table or vocab_size <= 0");
    const size_t n = (size_t)ctx->cfg.vocab_size * ctx->cfg.top_k;
    for (size_t i = 0; i < n; ++i)
        if (tid2eid[i] < 0 || tid2eid[i] >= ctx->cfg.n_experts)
            return fail(FST_EINVAL, "hash table entry out of range at " + std::to_string(i));
    if (!ctx->hash[lid]) {
        void* p = nullptr;
        if (hipMalloc(&p, n * sizeof(int32_t)) != hipSuccess) return fail(FST_ENOMEM, "hipMalloc(hash) failed");
        ctx->hash[lid] = (int32_t*)p;
    }
    FST_HIP_TRY(hipMemcpyAsync(ctx->hash[lid], tid2eid, n * sizeof(int32_t), hipMemcpyHostToDevice, ctx->st));
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    return FST_OK;
}

// ------------------------------------------------------------ MoE chain

static constexpr float kNormEps = 1e-6f;  // rms_cpu default and the NPU rmsnorm (src/fst_engine.cpp:89)

static int run_moe(fst_ctx* ctx, int lid, const uint16_t* d_h, int M, const int32_t* d_ids, int do_router,
                   int32_t* d_eids, float* d_wts, int tk, int use_routed, int use_shared, uint16_t* d_out,
                   uint16_t* d_out_routed, uint16_t* d_out_shared) {
    if (int rc = check_lid(ctx, lid)) return rc;
    const fst_config& c = ctx->cfg;
    if (M <= 0 || M > c.max_tokens) return fail(FST_EINVAL, "M must be in [1, max_tokens]");
    if (use_shared && !c.has_shared) return fail(FST_EINVAL, "config has no shared expert");
    if (use_routed && ctx->n_uploaded[lid] - (ctx->uploaded[lid][c.n_experts] ? 1 : 0) < c.n_experts)
        return fail(FST_ENOTREADY, "not all routed experts of layer " + std::to_string(lid) + " are uploaded");
    const bool sh16 = use_shared && ctx->shared16[lid];  // bf16 shared expert: its own launches
    if (use_shared && !sh16 && !ctx->uploaded[lid][c.n_experts])
        return fail(FST_ENOTREADY, "shared expert of layer " + std::to_string(lid) + " is not uploaded");
    if (do_router && !ctx->has_router[lid])
        return fail(FST_ENOTREADY, "router of layer " + std::to_string(lid) + " is not uploaded");
    if (tk < 0 || tk > c.top_k) return fail(FST_EINVAL, "tk must be in [0, top_k]");
    fst::Geometry g = ctx->geo;
    g.tk = use_routed ? tk : 0;
    fst::LayerView L = ctx->layer(lid);
    const int use_hash = do_router && lid < c.n_hash_layers && L.hash && d_ids;
    hipStream_t st = ctx->st;
    ctx->mark_begin();
    const bool mx = c.codec == FST_CODEC_MXFP4;  // bf16 operands: no fp16 operand prep
    // top-k + bucketing run inside the gate||up launch when the expert count allows
    const bool fuse_topk = do_router && c.n_experts <= fst::kFusedRouteMaxExperts;
    const fst::RouteReq rq{d_ids, use_hash, use_shared && !sh16, d_eids, d_wts, do_router ? 0 : 1};
    if (do_router) {
        // logits and operand prep (Q4_K) in one launch, then (unless fused) top-k + bucketing
        fst::launch_route(st, g, L, d_h, M, mx ? 0 : 1, d_ids, use_hash, use_shared && !sh16, d_eids, d_wts,
                          ctx->s, fuse_topk ? 0 : 1);
        ctx->mark("route");
    }
    if (sh16) {
        // process_shared_expert (src/fst_engine.cpp:4373-4489) over bf16 weights; its fp32
        // output joins the combine of the routed down projection (or is the result)
        const int hd = c.hidden_dim, inter = c.inter_dim;
        const uint16_t* W = ctx->shared16[lid];
        fst::launch_bf16_gate_up(st, W, hd, inter, d_h, M, c.swiglu_limit, ctx->s.sh_h16);
        fst::launch_bf16_linear(st, W + (size_t)2 * inter * hd, inter, hd, ctx->s.sh_h16, M,
                                use_routed ? ctx->s.ys : nullptr, use_routed ? nullptr : d_out,
                                use_routed ? nullptr : d_out_shared);
        ctx->mark("shared_bf16");
        if (!use_routed) {
            FST_HIP_TRY(hipGetLastError());
            return FST_OK;
        }
    }
    if (!do_router && !mx && !sh16 && ctx->gemv && fst::gemv_supported(g, M, g.tk, use_shared, ctx->s)) {
        // at one or two tokens: one launch from the caller's routing to the
        // combined rows (every workgroup finds the slots)
        ctx->fused_epoch = ctx->fused_epoch == 0xffffffffu ? 1u : ctx->fused_epoch + 1u;
        fst::launch_expert_gemv(st, g, L, M, g.tk, d_eids, d_wts, use_shared, d_h, ctx->s, ctx->fused_epoch,
                                ctx->spin_limit, d_out, d_out_routed, d_out_shared);
        ctx->mark("expert_gemv");
        FST_HIP_TRY(hipGetLastError());
        return FST_OK;
    }
    // one routed pair per token and no shared expert: the down launch writes
    // the bf16 result itself (the combine of one term), no combine launch
    const bool direct = use_routed && g.tk == 1 && !use_shared;
    // gate||up and down as one persistent launch (which routes or buckets the
    // call itself), or the launch chain
    const bool fused_path =
        (fuse_topk || !do_router) && !direct && ctx->fused && use_routed && fst::moe_fused_supported(g, M);
    if (!do_router && fused_path) {
        // the fused launch buckets the given ids itself (and streams the
        // shared expert first): only the token rows' operand (Q4_K) and the
        // launch's claim counter are prepared
        fst::launch_bucket_prep(st, g, M, 0, d_eids, ctx->s, mx ? nullptr : d_h, nullptr, nullptr, nullptr, 0, false);
        ctx->mark("prep");
    } else if (!do_router) {
        // the shared expert's gate||up weights (Q4_K) are read into the
        // device-wide cache during this latency-bound launch
        const size_t gu_bytes = (size_t)2 * c.inter_dim * (c.hidden_dim / 256) * 144;
        const bool pf = !mx && use_shared && !sh16;
        fst::launch_bucket_prep(st, g, M, use_shared && !sh16, d_eids, ctx->s, mx ? nullptr : d_h,
                                direct ? d_out : nullptr, direct ? d_out_routed : nullptr,
                                pf ? L.bank + (size_t)c.n_experts * L.expert_stride : nullptr, pf ? gu_bytes : 0);
        ctx->mark("bucket_prep");
    }
    const int sh_q = use_shared && !sh16 ? 1 : 0;  // the shared expert runs as slot 0
    if (fused_path) {
        // gate||up and down in one persistent launch, then the combine
        ctx->fused_epoch = ctx->fused_epoch == 0xffffffffu ? 1u : ctx->fused_epoch + 1u;
        hipEvent_t k0 = nullptr, k1 = nullptr;
        if (ctx->kring && ctx->kev_n < ctx->kev_cap) {
            k0 = ctx->kev[2 * ctx->kev_n];
            k1 = ctx->kev[2 * ctx->kev_n + 1];
            ++ctx->kev_n;
        }
        fst::launch_moe_fused(st, g, L, M, ctx->s, rq, ctx->fused_epoch, ctx->spin_limit, d_h, k0, k1);
        ctx->mark("moe_fused");
        // (a bf16 shared expert ran above; its fp32 rows are the combine's
        // shared term).  Router-driven calls: y rows by (token, j); caller
        // routing: y rows by pair, through the pair tables
        if (do_router && ctx->fold_w && !d_out_routed && !d_out_shared && fst::combine_norm_supported(g)) {
            // the verify forward's next residual add + RMSNorm in the same launch
            fst::launch_combine_norm_tj(st, g, M, use_shared, ctx->s, d_wts, sh16 ? ctx->s.ys : nullptr, ctx->fold_h,
                                        ctx->fold_w, kNormEps, ctx->fold_mn);
            ctx->folded = true;
        } else if (do_router)
            fst::launch_combine_tj(st, g, M, use_shared, ctx->s, d_wts, sh16 ? ctx->s.ys : nullptr, d_out,
                                   d_out_routed, d_out_shared);
        else
            fst::launch_combine(st, g, M, use_shared, ctx->s, d_wts, sh16 ? ctx->s.ys : nullptr, d_out,
                                d_out_routed, d_out_shared);
        ctx->mark("combine");
        FST_HIP_TRY(hipGetLastError());
        return FST_OK;
    }
    const int ksplit = fst::launch_q4k_gate_up(st, g, L, M, ctx->s, d_h, fuse_topk ? &rq : nullptr,
                                               std::min(c.n_experts, M * g.tk) + sh_q, M * (g.tk + sh_q));
    ctx->mark("q4k_gate_up");
    if (!mx) {
        // the shared expert's down matrix (slot 0 of the down launch) is read
        // into the device-wide cache during the prep launch
        const size_t proj = (size_t)c.inter_dim * (c.hidden_dim / 256) * 144;
        const void* pf = sh_q ? L.bank + (size_t)c.n_experts * L.expert_stride + 2 * proj : nullptr;
        if (ksplit > 1)
            fst::launch_prep_act_split(st, ctx->s.act, ksplit, M * (g.tk + sh_q), c.swiglu_limit, ctx->s.meta,
                                       c.inter_dim, ctx->s.a16p, ctx->s.sx2p, ctx->s.xs2, pf, proj);
        else
            fst::launch_prep_act(st, ctx->s.act, ctx->s.meta, ctx->s.max_pairs, c.inter_dim, ctx->s.a16p,
                                 ctx->s.sx2p, ctx->s.xs2, pf, proj);
        ctx->mark("prep_h");
    }
    if (direct) {
        fst::launch_q4k_down(st, g, L, M, ctx->s, d_wts, d_out, d_out_routed);
        ctx->mark("q4k_down");
    } else {
        fst::launch_q4k_down(st, g, L, M, ctx->s);
        ctx->mark("q4k_down");
        fst::launch_combine(st, g, M, use_shared, ctx->s, d_wts, sh16 ? ctx->s.ys : nullptr, d_out, d_out_routed,
                            d_out_shared);
        ctx->mark("combine");
    }
    FST_HIP_TRY(hipGetLastError());
    return FST_OK;
}

// Status of the sticky error bits of the MoE path (meta[META_STICKY]).
static int sticky_status(int flags) {
    // (an input id out of range also leaves its token without valid experts:
    // the hash message names the cause)
    if (flags & fst::STICKY_HASH_ID) return fail(FST_EINVAL, "input id out of vocabulary range for hash routing");
    if (flags & fst::STICKY_EXPERT_ID) return fail(FST_EINVAL, "expert id out of range in routing");
    if (flags & fst::STICKY_TIMEOUT)
        return fail(FST_EHIP, "a cross-workgroup hand-off of the MoE launch exceeded its spin limit");
    return FST_OK;
}

// Waits for the context's stream, reads the sticky error bits every MoE
// launch since the last read ORed in, clears them, and turns them into a
// status.
static int check_meta_error(fst_ctx* ctx) {
    int flags = 0;
    FST_HIP_TRY(hipMemcpyAsync(&flags, ctx->s.meta + fst::META_STICKY, sizeof(int), hipMemcpyDeviceToHost, ctx->st));
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    if (flags) {
        const int zero = 0;
        FST_HIP_TRY(hipMemcpyAsync(ctx->s.meta + fst::META_STICKY, &zero, sizeof(int), hipMemcpyHostToDevice, ctx->st));
        FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    }
    return sticky_status(flags);
}

int fst_moe_check(fst_ctx* ctx) {
    if (!ctx) return fail(FST_EINVAL, "fst_moe_check: null context");
    return check_meta_error(ctx);
}

int fst_device_error_status(int flags) { return sticky_status(flags); }

// Device activation / logits buffers are read with 16-byte loads (null
// pointers, i.e. absent optional buffers, pass).
static bool misaligned(const void* a, const void* b = nullptr, const void* c = nullptr, const void* d = nullptr) {
    return (((uintptr_t)a | (uintptr_t)b | (uintptr_t)c | (uintptr_t)d) & 15u) != 0;
}

int fst_moe_layer_dev(fst_ctx* ctx, int lid, const uint16_t* d_h, int M, const int32_t* d_input_ids,
                      uint16_t* d_out, int32_t* d_eids, float* d_wts) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (!d_h || !d_out) return fail(FST_EINVAL, "null device buffer");
    if (misaligned(d_h, d_out)) return fail(FST_EINVAL, "device buffers must be 16-byte aligned");
    int32_t* e = d_eids ? d_eids : ctx->s.eids;
    float* w = d_wts ? d_wts : ctx->s.wts;
    return run_moe(ctx, lid, d_h, M, d_input_ids, 1, e, w, ctx->cfg.top_k, 1, ctx->cfg.has_shared, d_out,
                   nullptr, nullptr);
}

int fst_moe_ffn_dev(fst_ctx* ctx, int lid, const uint16_t* d_h, int M, const int32_t* d_eids,
                    const float* d_wts, int use_shared, uint16_t* d_out, uint16_t* d_out_routed,
                    uint16_t* d_out_shared) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (!d_h || !d_eids || !d_wts) return fail(FST_EINVAL, "null device buffer");
    if (misaligned(d_h, d_out, d_out_routed, d_out_shared))
        return fail(FST_EINVAL, "device buffers must be 16-byte aligned");
    return run_moe(ctx, lid, d_h, M, nullptr, 0, const_cast<int32_t*>(d_eids), const_cast<float*>(d_wts),
                   ctx->cfg.top_k, 1, use_shared, d_out, d_out_routed, d_out_shared);
}

int fst_moe_layer(fst_ctx* ctx, int lid, const uint16_t* h, int M, const int32_t* input_ids, uint16_t* out,
                  int32_t* eids, float* wts) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (!h || !out) return fail(FST_EINVAL, "null host buffer");
    if (M <= 0 || M > ctx->cfg.max_tokens) return fail(FST_EINVAL, "M must be in [1, max_tokens]");
    const int hd = ctx->cfg.hidden_dim, tk = ctx->cfg.top_k;
    FST_HIP_TRY(hipMemcpyAsync(ctx->s.h, h, (size_t)M * hd * 2, hipMemcpyHostToDevice, ctx->st));
    if (input_ids) FST_HIP_TRY(hipMemcpyAsync(ctx->s.ids, input_ids, M * 4, hipMemcpyHostToDevice, ctx->st));
    if (int rc = run_moe(ctx, lid, ctx->s.h, M, input_ids ? ctx->s.ids : nullptr, 1, ctx->s.eids, ctx->s.wts,
                         tk, 1, ctx->cfg.has_shared, ctx->s.out, nullptr, nullptr))
        return rc;
    FST_HIP_TRY(hipMemcpyAsync(out, ctx->s.out, (size_t)M * hd * 2, hipMemcpyDeviceToHost, ctx->st));
    if (eids) FST_HIP_TRY(hipMemcpyAsync(eids, ctx->s.eids, (size_t)M * tk * 4, hipMemcpyDeviceToHost, ctx->st));
    if (wts) FST_HIP_TRY(hipMemcpyAsync(wts, ctx->s.wts, (size_t)M * tk * 4, hipMemcpyDeviceToHost, ctx->st));
    return check_meta_error(ctx);
}

int fst_router(fst_ctx* ctx, int lid, const uint16_t* h, int M, const int32_t* input_ids, int32_t* eids,
               float* wts) {
    if (int rc = check_lid(ctx, lid)) return rc;
    if (!h || !eids || !wts) return fail(FST_EINVAL, "null host buffer");
    const fst_config& c = ctx->cfg;
    if (M <= 0 || M > c.max_tokens) return fail(FST_EINVAL, "M must be in [1, max_tokens]");
    if (!ctx->has_router[lid]) return fail(FST_ENOTREADY, "router not uploaded");
    fst::LayerView L = ctx->layer(lid);
    const int use_hash = lid < c.n_hash_layers && L.hash && input_ids;
    FST_HIP_TRY(hipMemcpyAsync(ctx->s.h, h, (size_t)M * c.hidden_dim * 2, hipMemcpyHostToDevice, ctx->st));
    if (input_ids) FST_HIP_TRY(hipMemcpyAsync(ctx->s.ids, input_ids, M * 4, hipMemcpyHostToDevice, ctx->st));
    ctx->mark_begin();
    fst::launch_route(ctx->st, ctx->geo, L, ctx->s.h, M, 0, input_ids ? ctx->s.ids : nullptr, use_hash, 0,
                      ctx->s.eids, ctx->s.wts, ctx->s);
    ctx->mark("route");
    FST_HIP_TRY(hipGetLastError());
    FST_HIP_TRY(hipMemcpyAsync(eids, ctx->s.eids, (size_t)M * c.top_k * 4, hipMemcpyDeviceToHost, ctx->st));
    FST_HIP_TRY(hipMemcpyAsync(wts, ctx->s.wts, (size_t)M * c.top_k * 4, hipMemcpyDeviceToHost, ctx->st));
    return check_meta_error(ctx);
}

static int host_ffn(fst_ctx* ctx, int lid, const uint16_t* h, uint16_t* out, int M, const int32_t* eids, int tk,
                    const float* wts, int routed, int shared) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (!h || !out) return fail(FST_EINVAL, "null host buffer");
    const fst_config& c = ctx->cfg;
    if (M <= 0 || M > c.max_tokens) return fail(FST_EINVAL, "M must be in [1, max_tokens]");
    if (routed) {
        if (!eids || !wts) return fail(FST_EINVAL, "null eids/wts");
        if (tk <= 0 || tk > c.top_k) return fail(FST_EINVAL, "tk must be in [1, top_k]");
        for (int i = 0; i < M * tk; ++i)
            if (eids[i] < 0 || eids[i] >= c.n_experts)
                return fail(FST_EINVAL, "expert id out of range at " + std::to_string(i));
    }
    const int hd = c.hidden_dim;
    FST_HIP_TRY(hipMemcpyAsync(ctx->s.h, h, (size_t)M * hd * 2, hipMemcpyHostToDevice, ctx->st));
    if (routed) {
        FST_HIP_TRY(hipMemcpyAsync(ctx->s.eids, eids, (size_t)M * tk * 4, hipMemcpyHostToDevice, ctx->st));
        FST_HIP_TRY(hipMemcpyAsync(ctx->s.wts, wts, (size_t)M * tk * 4, hipMemcpyHostToDevice, ctx->st));
    }
    if (int rc = run_moe(ctx, lid, ctx->s.h, M, nullptr, 0, ctx->s.eids, ctx->s.wts, routed ? tk : 0, routed,
                         shared, ctx->s.out, nullptr, nullptr))
        return rc;
    FST_HIP_TRY(hipMemcpyAsync(out, ctx->s.out, (size_t)M * hd * 2, hipMemcpyDeviceToHost, ctx->st));
    return check_meta_error(ctx);
}

int fst_expert_ffn(fst_ctx* ctx, int lid, const uint16_t* h, uint16_t* out, int M, const int32_t* eids, int tk,
                   const float* wts) {
    return host_ffn(ctx, lid, h, out, M, eids, tk, wts, 1, 0);
}

int fst_shared_expert(fst_ctx* ctx, int lid, const uint16_t* h, uint16_t* out, int M) {
    return host_ffn(ctx, lid, h, out, M, nullptr, 0, nullptr, 0, 1);
}

// ------------------------------------------------------------ acceptance

// Grows a device buffer; a fresh buffer is zero-filled (the acceptance
// workspace starts with its completion counters at zero).
static int grow(hipStream_t st, void** p, size_t* cap, size_t need) {
    if (*cap >= need) return FST_OK;
    if (*p) {
        (void)hipStreamSynchronize(st);
        (void)hipFree(*p);
    }
    *p = nullptr;
    *cap = 0;
    if (hipMalloc(p, need) != hipSuccess) return fail(FST_ENOMEM, "hipMalloc(acceptance staging) failed");
    if (hipMemsetAsync(*p, 0, need, st) != hipSuccess) return fail(FST_EHIP, "hipMemsetAsync failed");
    *cap = need;
    return FST_OK;
}

// The acceptance workspace carries completion counters that the kernels leave
// at zero; its layout depends on (n_seq, k), so a shape change re-zeroes it.
static int accept_ws(fst_ctx* ctx, int n_seq, int k, int V) {
    if (int rc = grow(ctx->st, &ctx->acc_ws, &ctx->acc_ws_cap, fst::accept_ws_bytes(n_seq, k, V))) return rc;
    if (ctx->acc_ws_nseq != n_seq || ctx->acc_ws_k != k) {
        FST_HIP_TRY(hipMemsetAsync(ctx->acc_ws, 0, ctx->acc_ws_cap, ctx->st));
        ctx->acc_ws_nseq = n_seq;
        ctx->acc_ws_k = k;
    }
    return FST_OK;
}

static int check_accept_args(fst_ctx* ctx, int n_seq, int k, int V) {
    if (n_seq <= 0 || n_seq > 4096) return fail(FST_EINVAL, "n_seq must be in [1, 4096]");
    if (k < 0 || k > 63) return fail(FST_EINVAL, "k must be in [0, 63]");
    if (V <= 0 || V > fst::kMaxAcceptVocab)
        return fail(FST_EINVAL, "V must be in [1, " + std::to_string(fst::kMaxAcceptVocab) + "]");
    // the launches put one row of logits per grid row: n_seq*(2k+1) rows
    // (target and draft) for rejection sampling, n_seq*(k+1) for greedy
    if ((long)n_seq * (2 * k + 1) > (long)ctx->max_grid_y)
        return fail(FST_EINVAL, "n_seq*(2k+1) exceeds the device grid limit " + std::to_string(ctx->max_grid_y));
    return FST_OK;
}

static uint32_t next_epoch(uint32_t* e) {
    *e = *e % 4095u + 1u;  // 1..4095
    return *e;
}

int fst_accept_greedy_dev(fst_ctx* ctx, const float* d_target, int n_seq, int k, int V, const int32_t* d_draft,
                          int32_t* d_n_acc, int32_t* d_tokens) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (int rc = check_accept_args(ctx, n_seq, k, V)) return rc;
    if (misaligned(d_target)) return fail(FST_EINVAL, "device buffers must be 16-byte aligned");
    if (int rc = accept_ws(ctx, n_seq, k, V)) return rc;
    ctx->mark_begin();
    fst::launch_accept_greedy(ctx->st, d_target, n_seq, k, V, d_draft, d_n_acc, d_tokens,
                              fst::accept_greedy_words(ctx->acc_ws, n_seq, k), next_epoch(&ctx->acc_epoch),
                              ctx->spin_limit);
    ctx->mark("accept_greedy");
    FST_HIP_TRY(hipGetLastError());
    return FST_OK;
}

int fst_accept_greedy_dev_noalloc(fst_ctx* ctx, const float* d_target, int n_seq, int k, int V,
                                  const int32_t* d_draft, int32_t* d_n_acc, int32_t* d_tokens) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (int rc = check_accept_args(ctx, n_seq, k, V)) return rc;
    if ((long)n_seq * (k + 1) > fst::kStaticGreedyRows)
        return fail(FST_EINVAL, "n_seq*(k+1) exceeds the fixed scratch of " + std::to_string(fst::kStaticGreedyRows) +
                                    " rows");
    if (!d_target || !d_n_acc || !d_tokens || (k > 0 && !d_draft)) return fail(FST_EINVAL, "null device buffer");
    if (misaligned(d_target)) return fail(FST_EINVAL, "device buffers must be 16-byte aligned");
    void* words = fst::accept_scratch_ptr(ctx->cfg.device);
    if (!words) return fail(FST_EHIP, "scratch address of the device was not set up");
    ctx->mark_begin();
    const uint32_t epoch = fst::accept_scratch_epoch(ctx->cfg.device);
    if (epoch == 1) fst::accept_scratch_clear(ctx->st, words);
    fst::launch_accept_greedy(ctx->st, d_target, n_seq, k, V, d_draft, d_n_acc, d_tokens, words, epoch,
                              ctx->spin_limit);
    ctx->mark("accept_greedy");
    FST_HIP_TRY(hipGetLastError());
    return FST_OK;
}

int fst_set_fused(fst_ctx* ctx, int on) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    ctx->fused = on != 0 && ctx->s.fused_per_cu > 0;
    return FST_OK;
}

int fst_set_small_m(fst_ctx* ctx, int on) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    ctx->gemv = on != 0;
    return FST_OK;
}

int fst_set_wait_limit(fst_ctx* ctx, int spins) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (spins < 0) return fail(FST_EINVAL, "spins must be >= 0");
    ctx->spin_limit = spins == 0 ? fst::kDefaultSpinLimit : spins;
    return FST_OK;
}

int fst_accept_check(const int32_t* n_acc, int n_seq) {
    if (!n_acc || n_seq <= 0) return fail(FST_EINVAL, "fst_accept_check: null n_acc or n_seq <= 0");
    for (int s = 0; s < n_seq; ++s)
        if (n_acc[s] < 0)
            return fail(FST_EHIP, "acceptance of sequence " + std::to_string(s) +
                                      " abandoned: its cross-workgroup wait exceeded the spin limit");
    return FST_OK;
}

int fst_accept_stochastic_dev(fst_ctx* ctx, const float* d_target, const float* d_draft_logits, int n_seq, int k,
                              int V, const int32_t* d_draft, float temperature, uint64_t seed, uint64_t seq_base,
                              int32_t* d_n_acc, int32_t* d_tokens) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (int rc = check_accept_args(ctx, n_seq, k, V)) return rc;
    if (!(temperature > 0.0f)) return fail(FST_EINVAL, "temperature must be > 0");
    if (int rc = accept_ws(ctx, n_seq, k, V)) return rc;
    const float inv_t = 1.0f / temperature;
    ctx->mark_begin();
    fst::launch_accept_stochastic(ctx->st, d_target, d_draft_logits, n_seq, k, V, d_draft, inv_t, seed, seq_base,
                                  d_n_acc, d_tokens, ctx->acc_ws);
    ctx->mark("accept_stochastic");
    FST_HIP_TRY(hipGetLastError());
    return FST_OK;
}

static int accept_host(fst_ctx* ctx, const float* target, const float* draft_logits, int n_seq, int k, int V,
                       const int32_t* draft, float temperature, uint64_t seed, uint64_t seq_base, int32_t* n_acc,
                       int32_t* tokens, int stochastic) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (int rc = check_accept_args(ctx, n_seq, k, V)) return rc;
    if (!target || !n_acc || !tokens || (k > 0 && !draft) || (stochastic && k > 0 && !draft_logits))
        return fail(FST_EINVAL, "null host buffer");
    for (int i = 0; i < n_seq * k; ++i)
        if (draft[i] < 0 || draft[i] >= V) return fail(FST_EINVAL, "draft token out of range");
    const size_t nt = (size_t)n_seq * (k + 1) * V, nd = stochastic ? (size_t)n_seq * k * V : 0;
    if (int rc = grow(ctx->st, (void**)&ctx->acc_logits, &ctx->acc_logits_cap, (nt + nd) * sizeof(float) + 256)) return rc;
    const size_t io = (size_t)n_seq * k + n_seq + (size_t)n_seq * (k + 1);
    if (int rc = grow(ctx->st, (void**)&ctx->acc_io, &ctx->acc_io_cap, io * 4 + 256)) return rc;
    int32_t* d_draft = ctx->acc_io;
    int32_t* d_nacc = d_draft + (size_t)n_seq * k;
    int32_t* d_tok = d_nacc + n_seq;
    FST_HIP_TRY(hipMemcpyAsync(ctx->acc_logits, target, nt * 4, hipMemcpyHostToDevice, ctx->st));
    if (nd)
        FST_HIP_TRY(hipMemcpyAsync(ctx->acc_logits + nt, draft_logits, nd * 4, hipMemcpyHostToDevice, ctx->st));
    if (k > 0) FST_HIP_TRY(hipMemcpyAsync(d_draft, draft, (size_t)n_seq * k * 4, hipMemcpyHostToDevice, ctx->st));
    int rc = stochastic ? fst_accept_stochastic_dev(ctx, ctx->acc_logits, ctx->acc_logits + nt, n_seq, k, V, d_draft,
                                                    temperature, seed, seq_base, d_nacc, d_tok)
                        : fst_accept_greedy_dev(ctx, ctx->acc_logits, n_seq, k, V, d_draft, d_nacc, d_tok);
    if (rc) return rc;
    FST_HIP_TRY(hipMemcpyAsync(n_acc, d_nacc, n_seq * 4, hipMemcpyDeviceToHost, ctx->st));
    FST_HIP_TRY(hipMemcpyAsync(tokens, d_tok, (size_t)n_seq * (k + 1) * 4, hipMemcpyDeviceToHost, ctx->st));
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    return fst_accept_check(n_acc, n_seq);
}

int fst_accept_greedy(fst_ctx* ctx, const float* target, int n_seq, int k, int V, const int32_t* draft,
                      int32_t* n_acc, int32_t* tokens) {
    return accept_host(ctx, target, nullptr, n_seq, k, V, draft, 1.0f, 0, 0, n_acc, tokens, 0);
}

int fst_accept_stochastic(fst_ctx* ctx, const float* target, const float* draft_logits, int n_seq, int k, int V,
                          const int32_t* draft, float temperature, uint64_t seed, uint64_t seq_base, int32_t* n_acc,
                          int32_t* tokens) {
    if (!(temperature > 0.0f)) return fail(FST_EINVAL, "temperature must be > 0");
    return accept_host(ctx, target, draft_logits, n_seq, k, V, draft, temperature, seed, seq_base, n_acc, tokens, 1);
}


// ------------------------------------------------------------ sample_token

int fst_sample_token_dev(fst_ctx* ctx, const float* d_logits, int n_rows, int V, float temperature, float top_p,
                         uint64_t seed, uint64_t seq_base, int32_t* d_tokens) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (!d_logits || !d_tokens) return fail(FST_EINVAL, "null device buffer");
    if (n_rows <= 0 || n_rows > ctx->max_grid_y) return fail(FST_EINVAL, "n_rows out of range");
    if (V <= 0 || V > fst::kMaxAcceptVocab)
        return fail(FST_EINVAL, "V must be in [1, " + std::to_string(fst::kMaxAcceptVocab) + "]");
    if (temperature != temperature || top_p != top_p) return fail(FST_EINVAL, "temperature/top_p is NaN");
    if (temperature > 0.0f)
        if (int rc = grow(ctx->st, &ctx->samp_ws, &ctx->samp_ws_cap, fst::sample_ws_bytes(n_rows, V))) return rc;
    ctx->mark_begin();
    fst::launch_sample_token(ctx->st, d_logits, n_rows, V, temperature, top_p, seed, seq_base, ctx->samp_ws,
                             d_tokens);
    ctx->mark("sample_token");
    FST_HIP_TRY(hipGetLastError());
    return FST_OK;
}

int fst_sample_token(fst_ctx* ctx, const float* logits, int V, float temperature, float top_p, uint64_t seed,
                     uint64_t seq, int32_t* token) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (!logits || !token) return fail(FST_EINVAL, "null host buffer");
    if (V <= 0 || V > fst::kMaxAcceptVocab)
        return fail(FST_EINVAL, "V must be in [1, " + std::to_string(fst::kMaxAcceptVocab) + "]");
    if (int rc = grow(ctx->st, (void**)&ctx->acc_logits, &ctx->acc_logits_cap, (size_t)V * 4 + 256)) return rc;
    if (int rc = grow(ctx->st, (void**)&ctx->acc_io, &ctx->acc_io_cap, 256)) return rc;
    FST_HIP_TRY(hipMemcpyAsync(ctx->acc_logits, logits, (size_t)V * 4, hipMemcpyHostToDevice, ctx->st));
    if (int rc = fst_sample_token_dev(ctx, ctx->acc_logits, 1, V, temperature, top_p, seed, seq, ctx->acc_io))
        return rc;
    FST_HIP_TRY(hipMemcpyAsync(token, ctx->acc_io, 4, hipMemcpyDeviceToHost, ctx->st));
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    return FST_OK;
}

// ------------------------------------------------------------ dequant

int fst_dequant(fst_ctx* ctx, int codec, const void* blocks, size_t nblocks, float* out_f32, uint16_t* out_bf16) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (codec != FST_CODEC_Q4K && codec != FST_CODEC_MXFP4) return fail(FST_EINVAL, "unknown codec");
    if (!blocks || nblocks == 0) return fail(FST_EINVAL, "no blocks");
    if (nblocks > (1u << 24)) return fail(FST_EINVAL, "too many blocks for one call");
    const size_t bb = codec == FST_CODEC_Q4K ? 144 : 17, be = codec == FST_CODEC_Q4K ? 256 : 32;
    void *din = nullptr, *df = nullptr, *db = nullptr;
    auto cleanup = [&]() {
        if (din) (void)hipFree(din);
        if (df) (void)hipFree(df);
        if (db) (void)hipFree(db);
    };
    if (hipMalloc(&din, nblocks * bb) != hipSuccess || (out_f32 && hipMalloc(&df, nblocks * be * 4) != hipSuccess) ||
        (out_bf16 && hipMalloc(&db, nblocks * be * 2) != hipSuccess)) {
        cleanup();
        return fail(FST_ENOMEM, "hipMalloc(dequant) failed");
    }
    int rc = FST_OK;
    if (hipMemcpyAsync(din, blocks, nblocks * bb, hipMemcpyHostToDevice, ctx->st) != hipSuccess)
        rc = fail(FST_EHIP, "dequant upload failed");
    if (!rc) {
        fst::launch_dequant(ctx->st, codec, (const uint8_t*)din, nblocks, (float*)df, (uint16_t*)db);
        if (hipGetLastError() != hipSuccess) rc = fail(FST_EHIP, "dequant launch failed");
    }
    if (!rc && out_f32 && hipMemcpyAsync(out_f32, df, nblocks * be * 4, hipMemcpyDeviceToHost, ctx->st) != hipSuccess)
        rc = fail(FST_EHIP, "dequant download failed");
    if (!rc && out_bf16 && hipMemcpyAsync(out_bf16, db, nblocks * be * 2, hipMemcpyDeviceToHost, ctx->st) != hipSuccess)
        rc = fail(FST_EHIP, "dequant download failed");
    if (hipStreamSynchronize(ctx->st) != hipSuccess && !rc) rc = fail(FST_EHIP, "dequant sync failed");
    cleanup();
    return rc;
}


// ------------------------------------------------ verify forward (C5 path)


int fst_upload_norm(fst_ctx* ctx, int lid, const uint16_t* w) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (lid < 0 || lid > ctx->cfg.n_layers) return fail(FST_EINVAL, "norm id must be in [0, n_layers]");
    if (!w) return fail(FST_EINVAL, "null norm weights");
    const int hd = ctx->cfg.hidden_dim;
    FST_HIP_TRY(hipMemcpyAsync(ctx->norms + (size_t)lid * hd, w, (size_t)hd * 2, hipMemcpyHostToDevice, ctx->st));
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    ctx->has_norm[lid] = 1;
    return FST_OK;
}

size_t fst_lm_head_bytes(const fst_config* c) {
    if (!c || c->hidden_dim <= 0 || c->vocab_size <= 0) return 0;
    return (size_t)c->vocab_size * (c->hidden_dim / 256) * 144;
}

static int lm_head_alloc(fst_ctx* ctx) {
    const fst_config& c = ctx->cfg;
    if (c.vocab_size % 128) return fail(FST_EINVAL, "vocab_size must be a multiple of 128 for the LM head");
    if (!ctx->lm_head) {
        void* p = nullptr;
        if (hipMalloc(&p, fst_lm_head_bytes(&c)) != hipSuccess) return fail(FST_ENOMEM, "hipMalloc(lm_head) failed");
        ctx->lm_head = static_cast<uint8_t*>(p);
    }
    return FST_OK;
}

int fst_upload_lm_head(fst_ctx* ctx, const void* packed, size_t bytes) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    const size_t need = fst_lm_head_bytes(&ctx->cfg);
    if (!packed || bytes != need)
        return fail(FST_EINVAL, "LM head size mismatch: got " + std::to_string(bytes) + ", expected " +
                                    std::to_string(need));
    if (int rc = lm_head_alloc(ctx)) return rc;
    std::vector<uint8_t> tiled(bytes);
    fst::repack_q4k_matrix(static_cast<const uint8_t*>(packed), tiled.data(), ctx->cfg.vocab_size,
                           ctx->cfg.hidden_dim);
    FST_HIP_TRY(hipMemcpyAsync(ctx->lm_head, tiled.data(), bytes, hipMemcpyHostToDevice, ctx->st));
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    ctx->lm_kind = 1;
    return FST_OK;
}

int fst_upload_lm_head_bf16(fst_ctx* ctx, const uint16_t* w) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (!w) return fail(FST_EINVAL, "null LM head");
    const fst_config& c = ctx->cfg;
    if (c.vocab_size % 128) return fail(FST_EINVAL, "vocab_size must be a multiple of 128 for the LM head");
    const size_t bytes = (size_t)c.vocab_size * c.hidden_dim * 2;
    if (!ctx->lm_head16) {
        void* p = nullptr;
        if (hipMalloc(&p, bytes) != hipSuccess) return fail(FST_ENOMEM, "hipMalloc(lm_head bf16) failed");
        ctx->lm_head16 = static_cast<uint16_t*>(p);
    }
    FST_HIP_TRY(hipMemcpyAsync(ctx->lm_head16, w, bytes, hipMemcpyHostToDevice, ctx->st));
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    ctx->lm_kind = 2;
    return FST_OK;
}

int fst_upload_shared_bf16(fst_ctx* ctx, int lid, const uint16_t* gate, const uint16_t* up, const uint16_t* down) {
    if (int rc = check_lid(ctx, lid)) return rc;
    const fst_config& c = ctx->cfg;
    if (!c.has_shared) return fail(FST_EINVAL, "config has no shared expert");
    if (!gate || !up || !down) return fail(FST_EINVAL, "null shared-expert matrix");
    const size_t n = (size_t)c.inter_dim * c.hidden_dim;
    if (!ctx->shared16[lid]) {
        void* p = nullptr;
        if (hipMalloc(&p, 3 * n * 2) != hipSuccess) return fail(FST_ENOMEM, "hipMalloc(shared expert bf16) failed");
        ctx->shared16[lid] = static_cast<uint16_t*>(p);
    }
    uint16_t* d = ctx->shared16[lid];
    FST_HIP_TRY(hipMemcpyAsync(d, gate, n * 2, hipMemcpyHostToDevice, ctx->st));
    FST_HIP_TRY(hipMemcpyAsync(d + n, up, n * 2, hipMemcpyHostToDevice, ctx->st));
    FST_HIP_TRY(hipMemcpyAsync(d + 2 * n, down, n * 2, hipMemcpyHostToDevice, ctx->st));
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    return FST_OK;
}

int fst_synth_experts_dev(fst_ctx* ctx, uint64_t seed, int lid, int e_first, int e_count, uint64_t id_base,
                          float d_sigma) {
    if (int rc = check_lid(ctx, lid)) return rc;
    const fst_config& c = ctx->cfg;
    if (e_first < 0 || e_count < 0 || e_first + e_count > c.n_experts + 1)
        return fail(FST_EINVAL, "expert range out of [0, n_experts]");
    if (e_first + e_count == c.n_experts + 1 && !c.has_shared) return fail(FST_EINVAL, "config has no shared expert");
    const int hd = c.hidden_dim, inter = c.inter_dim;
    const uint64_t gate_blocks = (uint64_t)inter * (hd / 256);
    const size_t proj = gate_blocks * 144;
    for (int e = e_first; e < e_first + e_count; ++e) {
        uint8_t* dst = ctx->bank + ((size_t)lid * (c.n_experts + 1) + e) * ctx->expert_stride;
        const uint64_t id = id_base + (uint64_t)e;
        if (c.codec == FST_CODEC_MXFP4) {
            // d_sigma is unused; scales e in [108, 128) as fst_synth_mxfp4_expert's defaults
            const uint64_t mb = (uint64_t)inter * (hd / 32);
            const size_t mp = mb * 17;
            fst::launch_synth_mx_tiled(ctx->st, seed, id, 0, inter, hd, 108, 128, dst);
            fst::launch_synth_mx_tiled(ctx->st, seed, id, mb, inter, hd, 108, 128, dst + mp);
            fst::launch_synth_mx_tiled(ctx->st, seed, id, 2 * mb, hd, inter, 108, 128, dst + 2 * mp);
            continue;
        }
        fst::launch_synth_q4k_tiled(ctx->st, seed, id, 0, inter, hd, d_sigma, dst);
        fst::launch_synth_q4k_tiled(ctx->st, seed, id, gate_blocks, inter, hd, d_sigma, dst + proj);
        fst::launch_synth_q4k_tiled(ctx->st, seed, id, 2 * gate_blocks, hd, inter, d_sigma, dst + 2 * proj);
    }
    FST_HIP_TRY(hipGetLastError());
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    for (int e = e_first; e < e_first + e_count; ++e)
        if (!ctx->uploaded[lid][e]) {
            ctx->uploaded[lid][e] = 1;
            ctx->n_uploaded[lid]++;
        }
    return FST_OK;
}

int fst_synth_lm_head_dev(fst_ctx* ctx, uint64_t seed, uint64_t id, float d_sigma) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (int rc = lm_head_alloc(ctx)) return rc;
    fst::launch_synth_q4k_tiled(ctx->st, seed, id, 0, ctx->cfg.vocab_size, ctx->cfg.hidden_dim, d_sigma,
                                ctx->lm_head);
    FST_HIP_TRY(hipGetLastError());
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    ctx->lm_kind = 1;
    return FST_OK;
}

int fst_rmsnorm_dev(fst_ctx* ctx, int lid, const uint16_t* d_h, const uint16_t* d_y, int M, uint16_t* d_h_out,
                    uint16_t* d_normed) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (lid < 0 || lid > ctx->cfg.n_layers) return fail(FST_EINVAL, "norm id must be in [0, n_layers]");
    if (!ctx->has_norm[lid]) return fail(FST_ENOTREADY, "norm weights not uploaded");
    if (!d_h || !d_normed) return fail(FST_EINVAL, "null device buffer");
    if (misaligned(d_h, d_y, d_h_out, d_normed)) return fail(FST_EINVAL, "device buffers must be 16-byte aligned");
    if (M <= 0 || M > ctx->cfg.max_tokens) return fail(FST_EINVAL, "M must be in [1, max_tokens]");
    const int hd = ctx->cfg.hidden_dim;
    fst::launch_resid_norm(ctx->st, d_h, d_y, ctx->norms + (size_t)lid * hd, M, hd, kNormEps, d_h_out, d_normed,
                           nullptr, nullptr);
    FST_HIP_TRY(hipGetLastError());
    return FST_OK;
}

// final norm (optionally after adding d_y to the residual d_h) + LM head
static int final_head(fst_ctx* ctx, uint16_t* d_h, const uint16_t* d_y, int M, float* d_logits) {
    const fst_config& c = ctx->cfg;
    if (!ctx->lm_kind) return fail(FST_ENOTREADY, "LM head not uploaded");
    if (!ctx->has_norm[c.n_layers]) return fail(FST_ENOTREADY, "final norm weights not uploaded");
    const int hd = c.hidden_dim;
    if (ctx->lm_kind == 2) {
        // bf16 head as the reference keeps it: normed rows in bf16, then Y = W x
        fst::launch_resid_norm(ctx->st, d_h, d_y, ctx->norms + (size_t)c.n_layers * hd, M, hd, kNormEps,
                               d_y ? d_h : nullptr, ctx->mn, nullptr, nullptr);
        fst::launch_bf16_linear(ctx->st, ctx->lm_head16, hd, c.vocab_size, ctx->mn, M, d_logits, nullptr, nullptr);
        FST_HIP_TRY(hipGetLastError());
        return FST_OK;
    }
    fst::launch_resid_norm(ctx->st, d_h, d_y, ctx->norms + (size_t)c.n_layers * hd, M, hd, kNormEps,
                           d_y ? d_h : nullptr, nullptr, &ctx->s, ctx->lm_tab);
    fst::launch_q4k_dense(ctx->st, ctx->lm_head, M, hd, c.vocab_size, ctx->s, ctx->lm_tab, d_logits);
    FST_HIP_TRY(hipGetLastError());
    return FST_OK;
}

int fst_lm_head_dev(fst_ctx* ctx, const uint16_t* d_h, int M, float* d_logits) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (!d_h || !d_logits) return fail(FST_EINVAL, "null device buffer");
    if (misaligned(d_h, d_logits)) return fail(FST_EINVAL, "device buffers must be 16-byte aligned");
    if (M <= 0 || M > ctx->cfg.max_tokens) return fail(FST_EINVAL, "M must be in [1, max_tokens]");
    ctx->mark_begin();
    if (int rc = final_head(ctx, const_cast<uint16_t*>(d_h), nullptr, M, d_logits)) return rc;
    ctx->mark("lm_head");
    return FST_OK;
}

// HC mode: the FFN control of every layer and the output head are uploaded.
static bool hc_ready(fst_ctx* ctx) {
    if (!ctx->has_hc_head) return false;
    for (int l = 0; l < ctx->cfg.n_layers; ++l)
        if (!ctx->has_hc[l]) return false;
    return true;
}

int fst_upload_hc(fst_ctx* ctx, int lid, const uint16_t* fn, const float* scale, const float* base) {
    if (int rc = check_lid(ctx, lid)) return rc;
    if (!fn || !scale || !base) return fail(FST_EINVAL, "null HC tensor");
    if (ctx->cfg.hidden_dim > 8192) return fail(FST_EINVAL, "HC needs hidden_dim <= 8192");
    const size_t n = (size_t)24 * 4 * ctx->cfg.hidden_dim;
    FST_HIP_TRY(hipMemcpyAsync(ctx->hc_fn + (size_t)lid * n, fn, n * 2, hipMemcpyHostToDevice, ctx->st));
    FST_HIP_TRY(hipMemcpyAsync(ctx->hc_sb + (size_t)lid * 27, scale, 3 * sizeof(float), hipMemcpyHostToDevice, ctx->st));
    FST_HIP_TRY(hipMemcpyAsync(ctx->hc_sb + (size_t)lid * 27 + 3, base, 24 * sizeof(float), hipMemcpyHostToDevice,
                               ctx->st));
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    ctx->has_hc[lid] = 1;
    return FST_OK;
}

int fst_upload_hc_head(fst_ctx* ctx, const uint16_t* fn, float scale, const float* base) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (!fn) return fail(FST_EINVAL, "null HC head tensor");
    if (ctx->cfg.hidden_dim > 8192) return fail(FST_EINVAL, "HC needs hidden_dim <= 8192");
    const size_t n = (size_t)4 * 4 * ctx->cfg.hidden_dim;
    float b[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (base) std::memcpy(b, base, sizeof(b));
    FST_HIP_TRY(hipMemcpyAsync(ctx->hc_head_fn, fn, n * 2, hipMemcpyHostToDevice, ctx->st));
    FST_HIP_TRY(hipMemcpyAsync(ctx->hc_head_base, b, sizeof(b), hipMemcpyHostToDevice, ctx->st));
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    ctx->hc_head_scale = scale;
    ctx->has_hc_head = true;
    return FST_OK;
}

int fst_hc_pre_dev(fst_ctx* ctx, int lid, const uint16_t* d_h_hc, int M, uint16_t* d_cur, float* d_post,
                   float* d_comb) {
    if (int rc = check_lid(ctx, lid)) return rc;
    if (!ctx->has_hc[lid]) return fail(FST_ENOTREADY, "HC tensors of the layer not uploaded");
    if (!d_h_hc || !d_cur || !d_post || !d_comb) return fail(FST_EINVAL, "null device buffer");
    if (M <= 0 || M > ctx->cfg.max_tokens) return fail(FST_EINVAL, "M must be in [1, max_tokens]");
    const int hd = ctx->cfg.hidden_dim;
    fst::launch_hc_pre(ctx->st, d_h_hc, ctx->hc_fn + (size_t)lid * 24 * 4 * hd, ctx->hc_sb + (size_t)lid * 27,
                       ctx->hc_sb + (size_t)lid * 27 + 3, M, hd, d_cur, d_post, d_comb);
    FST_HIP_TRY(hipGetLastError());
    return FST_OK;
}

int fst_hc_post_dev(fst_ctx* ctx, const uint16_t* d_block_out, uint16_t* d_h_hc, const float* d_post,
                    const float* d_comb, int M) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (!d_block_out || !d_h_hc || !d_post || !d_comb) return fail(FST_EINVAL, "null device buffer");
    if (M <= 0 || M > ctx->cfg.max_tokens) return fail(FST_EINVAL, "M must be in [1, max_tokens]");
    fst::launch_hc_post(ctx->st, d_block_out, d_h_hc, d_post, d_comb, M, ctx->cfg.hidden_dim);
    FST_HIP_TRY(hipGetLastError());
    return FST_OK;
}

int fst_hc_head_dev(fst_ctx* ctx, const uint16_t* d_h_hc, int M, uint16_t* d_plain) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (!ctx->has_hc_head) return fail(FST_ENOTREADY, "HC head tensors not uploaded");
    if (!d_h_hc || !d_plain) return fail(FST_EINVAL, "null device buffer");
    if (M <= 0 || M > ctx->cfg.max_tokens) return fail(FST_EINVAL, "M must be in [1, max_tokens]");
    fst::launch_hc_head(ctx->st, d_h_hc, ctx->hc_head_fn, ctx->hc_head_scale, ctx->hc_head_base, M,
                        ctx->cfg.hidden_dim, d_plain);
    FST_HIP_TRY(hipGetLastError());
    return FST_OK;
}

int fst_final_head(fst_ctx* ctx, const uint16_t* hs, int M, float* logits) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (!hs || !logits) return fail(FST_EINVAL, "null host buffer");
    const fst_config& c = ctx->cfg;
    if (M <= 0 || M > c.max_tokens) return fail(FST_EINVAL, "M must be in [1, max_tokens]");
    if (!ctx->lm_kind) return fail(FST_ENOTREADY, "LM head not uploaded");
    // one logits buffer for the context's largest call, kept across calls
    const size_t lbytes = (size_t)c.max_tokens * c.vocab_size * sizeof(float);
    if (int rc = grow(ctx->st, (void**)&ctx->head_logits, &ctx->head_logits_cap, lbytes)) return rc;
    const int hd = c.hidden_dim;
    uint16_t* plain = ctx->s.h;
    ctx->mark_begin();
    if (ctx->has_hc_head) {
        // the 4-stream residual [M][4][hd] collapses through output_hc_head
        // before the final norm and the head (src/fst_engine.cpp:2120-2128)
        FST_HIP_TRY(hipMemcpyAsync(ctx->hc_h, hs, (size_t)M * 4 * hd * 2, hipMemcpyHostToDevice, ctx->st));
        fst::launch_hc_head(ctx->st, ctx->hc_h, ctx->hc_head_fn, ctx->hc_head_scale, ctx->hc_head_base, M, hd,
                            ctx->hc_cur);
        plain = ctx->hc_cur;
        ctx->mark("hc_head");
    } else {
        FST_HIP_TRY(hipMemcpyAsync(plain, hs, (size_t)M * hd * 2, hipMemcpyHostToDevice, ctx->st));
    }
    if (int rc = final_head(ctx, plain, nullptr, M, ctx->head_logits)) return rc;
    ctx->mark("lm_head");
    FST_HIP_TRY(hipMemcpyAsync(logits, ctx->head_logits, (size_t)M * c.vocab_size * 4, hipMemcpyDeviceToHost,
                               ctx->st));
    FST_HIP_TRY(hipStreamSynchronize(ctx->st));
    return FST_OK;
}

int fst_verify_forward_dev(fst_ctx* ctx, uint16_t* d_h, int M, const int32_t* d_input_ids, float* d_logits) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (!d_h || !d_logits) return fail(FST_EINVAL, "null device buffer");
    if (misaligned(d_h, d_logits)) return fail(FST_EINVAL, "device buffers must be 16-byte aligned");
    const fst_config& c = ctx->cfg;
    if (M <= 0 || M > c.max_tokens) return fail(FST_EINVAL, "M must be in [1, max_tokens]");
    for (int l = 0; l < c.n_layers; ++l)
        if (!ctx->has_norm[l]) return fail(FST_ENOTREADY, "norm weights of layer " + std::to_string(l) + " not uploaded");
    const int hd = c.hidden_dim;
    const bool hc = hc_ready(ctx);
    ctx->mark_begin();
    ctx->nested = true;
    int rc = FST_OK;
    for (int l = 0; l < c.n_layers && rc == FST_OK; ++l) {
        if (hc) {
            // cur = hc_pre(h); mn = RMSNorm_l(cur); y = MoE_l(mn); h = hc_post(y, h)
            fst::launch_hc_pre(ctx->st, d_h, ctx->hc_fn + (size_t)l * 24 * 4 * hd, ctx->hc_sb + (size_t)l * 27,
                               ctx->hc_sb + (size_t)l * 27 + 3, M, hd, ctx->hc_cur, ctx->hc_post, ctx->hc_comb);
            fst::launch_resid_norm(ctx->st, ctx->hc_cur, nullptr, ctx->norms + (size_t)l * hd, M, hd, kNormEps,
                                   nullptr, ctx->mn, nullptr, nullptr);
        } else if (!ctx->folded) {
            // h += y (previous layer), mn = RMSNorm_l(h); y = MoE_l(mn)
            fst::launch_resid_norm(ctx->st, d_h, l > 0 ? ctx->s.out : nullptr, ctx->norms + (size_t)l * hd, M, hd,
                                   kNormEps, l > 0 ? d_h : nullptr, ctx->mn, nullptr, nullptr);
        }
        // (the previous layer's combine did this layer's h += y and norm when folded)
        ctx->folded = false;
        if (!hc && l + 1 < c.n_layers) {
            ctx->fold_h = d_h;
            ctx->fold_w = ctx->norms + (size_t)(l + 1) * hd;
            ctx->fold_mn = ctx->mn;
        }
        rc = run_moe(ctx, l, ctx->mn, M, d_input_ids, 1, ctx->s.eids, ctx->s.wts, c.top_k, 1, c.has_shared,
                     ctx->s.out, nullptr, nullptr);
        ctx->fold_h = nullptr;
        ctx->fold_w = nullptr;
        ctx->fold_mn = nullptr;
        if (hc && rc == FST_OK) fst::launch_hc_post(ctx->st, ctx->s.out, d_h, ctx->hc_post, ctx->hc_comb, M, hd);
    }
    ctx->nested = false;
    ctx->folded = false;
    ctx->fold_h = nullptr;
    ctx->fold_w = nullptr;
    ctx->fold_mn = nullptr;
    if (rc) return rc;
    ctx->mark("layers", true);
    if (hc) {
        fst::launch_hc_head(ctx->st, d_h, ctx->hc_head_fn, ctx->hc_head_scale, ctx->hc_head_base, M, hd, ctx->hc_cur);
        rc = final_head(ctx, ctx->hc_cur, nullptr, M, d_logits);
    } else {
        rc = final_head(ctx, d_h, ctx->s.out, M, d_logits);
    }
    if (rc) return rc;
    ctx->mark("lm_head", true);
    return FST_OK;
}

int fst_verify_forward(fst_ctx* ctx, uint16_t* h, int M, const int32_t* input_ids, float* logits) {
    if (!ctx) return fail(FST_EINVAL, "null context");
    if (!h || !logits) return fail(FST_EINVAL, "null host buffer");
    const fst_config& c = ctx->cfg;
    if (M <= 0 || M > c.max_tokens) return fail(FST_EINVAL, "M must be in [1, max_tokens]");
    const int hd = c.hidden_dim;
    const bool hc = hc_ready(ctx);
    const size_t hbytes = (size_t)M * (hc ? 4 : 1) * hd * 2;
    uint16_t* d_res = hc ? ctx->hc_h : ctx->s.h;
    const size_t nlog = (size_t)M * c.vocab_size;
    // the context's logits buffer (grown once, shared with fst_final_head)
    if (int rc = grow(ctx->st, (void**)&ctx->head_logits, &ctx->head_logits_cap, nlog * sizeof(float))) return rc;
    float* d_logits = ctx->head_logits;
    int rc = FST_OK;
    do {
        if (hipMemcpyAsync(d_res, h, hbytes, hipMemcpyHostToDevice, ctx->st) != hipSuccess ||
            (input_ids &&
             hipMemcpyAsync(ctx->s.ids, input_ids, M * 4, hipMemcpyHostToDevice, ctx->st) != hipSuccess)) {
            rc = fail(FST_EHIP, "host-to-device copy failed");
            break;
        }
        if ((rc = fst_verify_forward_dev(ctx, d_res, M, input_ids ? ctx->s.ids : nullptr, d_logits))) break;
        if (hipMemcpyAsync(logits, d_logits, nlog * sizeof(float), hipMemcpyDeviceToHost, ctx->st) != hipSuccess ||
            hipMemcpyAsync(h, d_res, hbytes, hipMemcpyDeviceToHost, ctx->st) != hipSuccess) {
            rc = fail(FST_EHIP, "device-to-host copy failed");
            break;
        }
        rc = check_meta_error(ctx);
    } while (0);
    (void)hipStreamSynchronize(ctx->st);  // (the error, if any, is already in rc)
    return rc;
}

}  // extern "C"
