// fst_bank.cpp — reader for the .fst model file and its upload into a context.
//
// Format (scripts/fst_converter.py:50-92, :169-176, :685-776): a 128-byte
// header, a directory of 64-byte tensor entries at shared_dir_offset, page
// aligned tensor data, and the expert bank of n_layers * n_experts blocks of
// expert_block_bytes at a page-aligned stride.  Readers in the reference:
// ExpertPager::parse_header / load_from_disk (src/expert_pager.cpp:88-130,
// :265-290) for experts, FSTEngine::load_shared_weights
// (src/fst_engine.cpp:1500-1760) for the rest.
//
// Differences from the reference readers, on purpose:
//  - tensors are found by (TID, layer) — the engine finds most by shape
//    ("256x4096x1", :1556-1605) and takes the moe norm as the second
//    4096-vector of the layer; the TID says which tensor it is;
//  - a 2-byte router bias is decoded by its qtype (the converter writes BF16,
//    :638-639); the engine reads it as fp16 (:1626-1630) — FST_BANK_BIAS_AS_FP16
//    reproduces that;
//  - fp16 scales of Q8_0 tensors are decoded as IEEE fp16 (subnormals
//    included; the engine's decoder mishandles them).
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/fst_exact_math.h"
#include "../../include/fst_hip.h"
#include "fst_internal.h"

struct fst_bank {
    int fd = -1;
    std::string path;
    uint64_t file_size = 0;
    fst_bank_header hdr{};
    std::vector<fst_bank_tensor> dir;
    ~fst_bank() {
        if (fd >= 0) ::close(fd);
    }
};

namespace {

constexpr size_t kHeaderBytes = 128;
constexpr size_t kEntryBytes = 64;
enum { QT_Q8_0 = 1, QT_BF16 = 2, QT_F32 = 3 };

int err(int code, const std::string& m) { return fst::set_error(code, m.c_str()); }

template <typename T>
T rd(const uint8_t* p) {
    T v;
    std::memcpy(&v, p, sizeof(T));
    return v;
}

bool pread_all(int fd, void* dst, size_t n, uint64_t off) {
    uint8_t* d = static_cast<uint8_t*>(dst);
    while (n) {
        const ssize_t r = ::pread(fd, d, n, (off_t)off);
        if (r <= 0) return false;
        d += r;
        n -= (size_t)r;
        off += (uint64_t)r;
    }
    return true;
}

bool in_file(const fst_bank* b, uint64_t off, uint64_t n) { return off <= b->file_size && n <= b->file_size - off; }

// Element count; 0 when a dimension alone exceeds the data size (every qtype
// stores at least one byte per element), so a corrupt shape cannot overflow.
uint64_t numel(const fst_bank_tensor& t) {
    for (uint64_t s : t.shape)
        if (s == 0 || s > t.size) return 0;
    const uint64_t a = t.shape[0] * t.shape[1];
    if (t.shape[1] && a / t.shape[1] != t.shape[0]) return 0;
    const uint64_t n = a * t.shape[2];
    return (t.shape[2] && n / t.shape[2] == a && n <= t.size) ? n : 0;
}

// A tensor as floats: BF16, F32, or Q8_0 (all fp16 block scales first, then
// the int8 values, scripts/fst_converter.py:518-536; a scale below 1e-12
// reads as 1, src/fst_engine.cpp:1596).
int read_f32(const fst_bank* b, const fst_bank_tensor& t, std::vector<float>& out) {
    const uint64_t n = numel(t);
    if (n == 0) return err(FST_EINVAL, "tensor shape does not fit its data size");
    std::vector<uint8_t> raw(t.size);
    if (!pread_all(b->fd, raw.data(), raw.size(), t.offset)) return err(FST_EINVAL, "short read of tensor data");
    out.resize(n);
    if (t.qtype == QT_BF16) {
        if (t.size != n * 2) return err(FST_EINVAL, "BF16 tensor size does not match its shape");
        for (uint64_t i = 0; i < n; ++i) out[i] = fst_bf16_to_f32(rd<uint16_t>(&raw[2 * i]));
    } else if (t.qtype == QT_F32) {
        if (t.size != n * 4) return err(FST_EINVAL, "F32 tensor size does not match its shape");
        std::memcpy(out.data(), raw.data(), n * 4);
    } else if (t.qtype == QT_Q8_0) {
        const uint64_t nb = (n + 31) / 32;
        if (t.size != nb * 2 + nb * 32) return err(FST_EINVAL, "Q8_0 tensor size does not match its shape");
        for (uint64_t blk = 0; blk < nb; ++blk) {
            float sf = fst_fp16_to_f32(rd<uint16_t>(&raw[2 * blk]));
            if (std::fabs(sf) < 1e-12f) sf = 1.0f;
            for (uint64_t j = 0; j < 32 && blk * 32 + j < n; ++j)
                out[blk * 32 + j] = (float)(int8_t)raw[nb * 2 + blk * 32 + j] * sf;
        }
    } else {
        return err(FST_EINVAL, "unknown tensor qtype " + std::to_string(t.qtype));
    }
    return FST_OK;
}

// A tensor as bf16: BF16 as stored, the other types rounded (RNE).
int read_bf16(const fst_bank* b, const fst_bank_tensor& t, std::vector<uint16_t>& out) {
    if (t.qtype == QT_BF16) {
        if (t.size != numel(t) * 2) return err(FST_EINVAL, "BF16 tensor size does not match its shape");
        out.resize(numel(t));
        if (!pread_all(b->fd, out.data(), t.size, t.offset)) return err(FST_EINVAL, "short read of tensor data");
        return FST_OK;
    }
    std::vector<float> f;
    if (int rc = read_f32(b, t, f)) return rc;
    out.resize(f.size());
    for (size_t i = 0; i < f.size(); ++i) out[i] = fst_f32_to_bf16(f[i]);
    return FST_OK;
}

int find_exact(const fst_bank* b, uint32_t tid, int lid, fst_bank_tensor* out) {
    for (const fst_bank_tensor& t : b->dir)
        if (t.tid == tid && (lid < 0 || (int)t.lid == lid)) {
            *out = t;
            return FST_OK;
        }
    return FST_ENOTREADY;
}

int need_shape(const fst_bank_tensor& t, uint64_t s0, uint64_t s1, const char* what) {
    if (t.shape[0] != s0 || t.shape[1] != s1 || t.shape[2] != 1)
        return err(FST_EINVAL, std::string(what) + ": shape " + std::to_string(t.shape[0]) + "x" +
                                   std::to_string(t.shape[1]) + "x" + std::to_string(t.shape[2]) + ", expected " +
                                   std::to_string(s0) + "x" + std::to_string(s1));
    return FST_OK;
}

}  // namespace

extern "C" {

int fst_bank_open(const char* path, fst_bank** out) {
    if (!path || !out) return err(FST_EINVAL, "fst_bank_open: null argument");
    *out = nullptr;
    auto* b = new fst_bank();
    b->path = path;
    auto bail = [&](int rc) {
        delete b;
        return rc;
    };
    b->fd = ::open(path, O_RDONLY);
    if (b->fd < 0) return bail(err(FST_EINVAL, std::string("cannot open ") + path));
    struct stat sb;
    if (fstat(b->fd, &sb) != 0) return bail(err(FST_EINVAL, "fstat failed"));
    b->file_size = (uint64_t)sb.st_size;
    uint8_t h[kHeaderBytes];
    if (b->file_size < kHeaderBytes || !pread_all(b->fd, h, kHeaderBytes, 0))
        return bail(err(FST_EINVAL, "file shorter than the 128-byte header"));
    if (std::memcmp(h, "FST\0", 4) != 0) return bail(err(FST_EINVAL, "bad magic (not an .fst file)"));
    fst_bank_header& H = b->hdr;
    std::memcpy(H.magic, h, 4);
    uint32_t* u32[] = {&H.version, &H.hidden_dim, &H.n_layers, &H.n_experts, &H.top_k, &H.n_q_heads,
                       &H.n_kv_heads, &H.head_dim, &H.inter_dim, &H.n_shared, &H.reserved0};
    for (int i = 0; i < 11; ++i) *u32[i] = rd<uint32_t>(h + 4 + 4 * i);
    H.vocab_size = rd<uint64_t>(h + 48);
    H.rms_eps = rd<float>(h + 56);
    H.rope_freq_base = rd<float>(h + 60);
    uint64_t* u64[] = {&H.shared_dir_offset, &H.shared_dir_count, &H.expert_bank_offset, &H.expert_block_bytes,
                       &H.expert_block_stride, &H.expert_count, &H.dspark, &H.dspark_noise_token_id};
    for (int i = 0; i < 8; ++i) *u64[i] = rd<uint64_t>(h + 64 + 8 * i);

    // directory
    if (H.shared_dir_count > (b->file_size / kEntryBytes) ||
        !in_file(b, H.shared_dir_offset, H.shared_dir_count * kEntryBytes))
        return bail(err(FST_EINVAL, "tensor directory outside the file"));
    std::vector<uint8_t> d(H.shared_dir_count * kEntryBytes);
    if (!d.empty() && !pread_all(b->fd, d.data(), d.size(), H.shared_dir_offset))
        return bail(err(FST_EINVAL, "short read of the tensor directory"));
    b->dir.resize(H.shared_dir_count);
    for (uint64_t i = 0; i < H.shared_dir_count; ++i) {
        const uint8_t* e = &d[i * kEntryBytes];
        fst_bank_tensor& t = b->dir[i];
        t.tid = rd<uint32_t>(e);
        t.lid = rd<uint16_t>(e + 4);
        t.sid = rd<uint16_t>(e + 6);
        t.qtype = rd<uint16_t>(e + 8);
        t.ndim = rd<uint16_t>(e + 10);
        for (int k = 0; k < 3; ++k) t.shape[k] = rd<uint64_t>(e + 16 + 8 * k);
        t.offset = rd<uint64_t>(e + 40);
        t.size = rd<uint64_t>(e + 48);
        if (!in_file(b, t.offset, t.size))
            return bail(err(FST_EINVAL, "tensor " + std::to_string(i) + " (tid " + std::to_string(t.tid) +
                                            ") outside the file"));
    }
    // expert bank
    const uint64_t n_exp = (uint64_t)H.n_layers * H.n_experts;
    if (n_exp) {
        if (H.expert_block_stride < H.expert_block_bytes)
            return bail(err(FST_EINVAL, "expert stride smaller than the expert block"));
        if (H.n_experts && H.expert_block_stride &&
            (n_exp - 1) > (b->file_size / H.expert_block_stride))
            return bail(err(FST_EINVAL, "expert bank outside the file"));
        if (!in_file(b, H.expert_bank_offset, (n_exp - 1) * H.expert_block_stride) ||
            !in_file(b, H.expert_bank_offset + (n_exp - 1) * H.expert_block_stride, H.expert_block_bytes))
            return bail(err(FST_EINVAL, "expert bank outside the file"));
    }
    *out = b;
    return FST_OK;
}

void fst_bank_close(fst_bank* b) { delete b; }

int fst_bank_get_header(const fst_bank* b, fst_bank_header* out) {
    if (!b || !out) return err(FST_EINVAL, "null argument");
    *out = b->hdr;
    return FST_OK;
}

int fst_bank_n_tensors(const fst_bank* b) { return b ? (int)b->dir.size() : -1; }

int fst_bank_tensor_at(const fst_bank* b, int i, fst_bank_tensor* out) {
    if (!b || !out) return err(FST_EINVAL, "null argument");
    if (i < 0 || i >= (int)b->dir.size()) return err(FST_EINVAL, "tensor index out of range");
    *out = b->dir[i];
    return FST_OK;
}

int fst_bank_find(const fst_bank* b, uint32_t tid, int lid, fst_bank_tensor* out) {
    if (!b || !out) return err(FST_EINVAL, "null argument");
    if (find_exact(b, tid, lid, out) == FST_OK) return FST_OK;
    return err(FST_ENOTREADY, "tensor tid " + std::to_string(tid) + " layer " + std::to_string(lid) + " not in file");
}

int fst_bank_read_tensor(const fst_bank* b, const fst_bank_tensor* t, void* dst, size_t bytes) {
    if (!b || !t || !dst) return err(FST_EINVAL, "null argument");
    if (bytes != t->size) return err(FST_EINVAL, "buffer size does not match the tensor size");
    if (!in_file(b, t->offset, t->size)) return err(FST_EINVAL, "tensor outside the file");
    if (!pread_all(b->fd, dst, bytes, t->offset)) return err(FST_EINVAL, "short read of tensor data");
    return FST_OK;
}

int fst_bank_read_expert(const fst_bank* b, int lid, int eid, void* dst, size_t bytes) {
    if (!b || !dst) return err(FST_EINVAL, "null argument");
    const fst_bank_header& H = b->hdr;
    if (lid < 0 || lid >= (int)H.n_layers || eid < 0 || eid >= (int)H.n_experts)
        return err(FST_EINVAL, "expert (" + std::to_string(lid) + ", " + std::to_string(eid) + ") out of range");
    if (bytes != H.expert_block_bytes) return err(FST_EINVAL, "buffer size does not match expert_block_bytes");
    const uint64_t off = H.expert_bank_offset + ((uint64_t)lid * H.n_experts + eid) * H.expert_block_stride;
    if (!pread_all(b->fd, dst, bytes, off)) return err(FST_EINVAL, "short read of expert block");
    return FST_OK;
}

int fst_bank_config(const fst_bank* b, fst_config* cfg) {
    if (!b || !cfg) return err(FST_EINVAL, "null argument");
    const fst_bank_header& H = b->hdr;
    fst_config_default(cfg);
    cfg->hidden_dim = (int)H.hidden_dim;
    cfg->inter_dim = (int)H.inter_dim;
    cfg->n_experts = (int)H.n_experts;
    cfg->top_k = (int)H.top_k;
    cfg->n_layers = (int)H.n_layers;
    cfg->vocab_size = (int)H.vocab_size;
    cfg->codec = FST_CODEC_MXFP4;
    cfg->has_shared = H.n_shared > 0 ? 1 : 0;
    cfg->score_func = FST_SCORE_SQRTSOFTPLUS;
    cfg->route_scale = 1.5f;
    cfg->n_hash_layers = 3;
    cfg->round_logits_bf16 = 1;
    cfg->swiglu_limit = 0.0f;
    if (fst_expert_bytes(cfg) != H.expert_block_bytes)
        return err(FST_EINVAL, "expert_block_bytes " + std::to_string(H.expert_block_bytes) +
                                   " is not an MXFP4 expert of hidden " + std::to_string(H.hidden_dim) +
                                   ", inter " + std::to_string(H.inter_dim));
    return FST_OK;
}

int fst_bank_load_layer(fst_ctx* ctx, const fst_bank* b, int lid, int flags) {
    if (!ctx || !b) return err(FST_EINVAL, "null argument");
    const fst_bank_header& H = b->hdr;
    if (lid < 0 || lid >= (int)H.n_layers) return err(FST_EINVAL, "layer out of the file's range");
    fst_config cfg;
    fst_get_config(ctx, &cfg);
    if (lid >= cfg.n_layers) return err(FST_EINVAL, "layer out of the context's range");
    if (cfg.hidden_dim != (int)H.hidden_dim || cfg.inter_dim != (int)H.inter_dim ||
        cfg.n_experts != (int)H.n_experts)
        return err(FST_EINVAL, "context geometry differs from the file's");
    const int hd = cfg.hidden_dim, inter = cfg.inter_dim, E = cfg.n_experts;
    fst_bank_tensor t;
    int rc = FST_OK;

    if (flags & FST_BANK_EXPERTS) {
        if (cfg.codec != FST_CODEC_MXFP4) return err(FST_EINVAL, "the expert bank is MXFP4: use an MXFP4 context");
        if (fst_expert_bytes(&cfg) != H.expert_block_bytes) return err(FST_EINVAL, "expert size mismatch");
        std::vector<uint8_t> blk(H.expert_block_bytes);
        for (int e = 0; e < E; ++e) {
            if ((rc = fst_bank_read_expert(b, lid, e, blk.data(), blk.size()))) return rc;
            if ((rc = fst_upload_expert(ctx, lid, e, blk.data(), blk.size()))) return rc;
        }
    }
    if (flags & FST_BANK_ROUTER) {
        if (find_exact(b, FST_TID_ROUTER, lid, &t)) return err(FST_ENOTREADY, "router (TID 9) missing for the layer");
        if ((rc = need_shape(t, (uint64_t)E, (uint64_t)hd, "router"))) return rc;
        std::vector<uint16_t> w;
        if ((rc = read_bf16(b, t, w))) return rc;
        std::vector<uint16_t> kn((size_t)hd * E);  // [E][hd] -> [hd][E] (src/fst_engine.cpp:1617)
        for (int e = 0; e < E; ++e)
            for (int k = 0; k < hd; ++k) kn[(size_t)k * E + e] = w[(size_t)e * hd + k];
        std::vector<float> bias;
        if (find_exact(b, FST_TID_ROUTER_BIAS, lid, &t) == FST_OK) {
            if (numel(t) != (uint64_t)E) return err(FST_EINVAL, "router bias: size is not n_experts");
            if ((flags & FST_BANK_BIAS_AS_FP16) && t.size == (uint64_t)E * 2) {
                std::vector<uint16_t> raw(E);
                if (!pread_all(b->fd, raw.data(), t.size, t.offset)) return err(FST_EINVAL, "short read of bias");
                bias.resize(E);
                for (int e = 0; e < E; ++e) bias[e] = fst_fp16_to_f32(raw[e]);
            } else if ((rc = read_f32(b, t, bias))) {
                return rc;
            }
        }
        if ((rc = fst_upload_router_bf16(ctx, lid, kn.data(), bias.empty() ? nullptr : bias.data()))) return rc;
    }
    if (flags & FST_BANK_NORM) {
        std::vector<uint16_t> w;
        if (find_exact(b, FST_TID_POST_ATTN_NORM, lid, &t) == FST_OK) {
            if ((rc = need_shape(t, (uint64_t)hd, 1, "moe norm"))) return rc;
            if ((rc = read_bf16(b, t, w))) return rc;
        } else {
            w.assign(hd, fst_f32_to_bf16(1.0f));  // src/fst_engine.cpp:1724
        }
        if ((rc = fst_upload_norm(ctx, lid, w.data()))) return rc;
    }
    if ((flags & FST_BANK_SHARED) && cfg.has_shared) {
        fst_bank_tensor tg, tu, td;
        if (find_exact(b, FST_TID_SHARED_GATE, lid, &tg) || find_exact(b, FST_TID_SHARED_UP, lid, &tu) ||
            find_exact(b, FST_TID_SHARED_DOWN, lid, &td))
            return err(FST_ENOTREADY, "shared expert (TID 11-13) missing for the layer");
        if ((rc = need_shape(tg, inter, hd, "shared gate")) || (rc = need_shape(tu, inter, hd, "shared up")) ||
            (rc = need_shape(td, hd, inter, "shared down")))
            return rc;
        std::vector<uint16_t> g, u, dn;
        if ((rc = read_bf16(b, tg, g)) || (rc = read_bf16(b, tu, u)) || (rc = read_bf16(b, td, dn))) return rc;
        if ((rc = fst_upload_shared_bf16(ctx, lid, g.data(), u.data(), dn.data()))) return rc;
    }
    if ((flags & FST_BANK_HC) && find_exact(b, FST_TID_HC_FFN_FN, lid, &t) == FST_OK) {
        fst_bank_tensor ts, tb;
        if (find_exact(b, FST_TID_HC_FFN_SCALE, lid, &ts) || find_exact(b, FST_TID_HC_FFN_BASE, lid, &tb))
            return err(FST_ENOTREADY, "HC scale/base (TID 27/28) missing for the layer");
        if ((rc = need_shape(t, 24, (uint64_t)4 * hd, "HC fn"))) return rc;
        std::vector<uint16_t> fn;
        std::vector<float> sc, bs;
        if ((rc = read_bf16(b, t, fn)) || (rc = read_f32(b, ts, sc)) || (rc = read_f32(b, tb, bs))) return rc;
        if (sc.size() != 3 || bs.size() != 24) return err(FST_EINVAL, "HC scale/base sizes are not 3/24");
        if ((rc = fst_upload_hc(ctx, lid, fn.data(), sc.data(), bs.data()))) return rc;
    }
    if ((flags & FST_BANK_HASH) && lid < cfg.n_hash_layers && cfg.vocab_size > 0) {
        // <model>.fst.tid2eid: int32 [n_hash_layers][vocab][top_k] (src/fst_engine.cpp:1527-1549)
        const std::string sp = b->path + ".tid2eid";
        const int fd = ::open(sp.c_str(), O_RDONLY);
        if (fd >= 0) {
            const size_t per = (size_t)cfg.vocab_size * cfg.top_k;
            std::vector<int32_t> tab(per);
            const bool ok = pread_all(fd, tab.data(), per * 4, (uint64_t)lid * per * 4);
            ::close(fd);
            if (!ok) return err(FST_EINVAL, "short read of the tid2eid sidecar");
            if ((rc = fst_upload_hash_table(ctx, lid, tab.data()))) return rc;
        }
    }
    return FST_OK;
}

int fst_bank_load_head(fst_ctx* ctx, const fst_bank* b, int flags) {
    if (!ctx || !b) return err(FST_EINVAL, "null argument");
    fst_config cfg;
    fst_get_config(ctx, &cfg);
    const int hd = cfg.hidden_dim;
    if (cfg.hidden_dim != (int)b->hdr.hidden_dim) return err(FST_EINVAL, "context geometry differs from the file's");
    fst_bank_tensor t;
    int rc = FST_OK;
    if (flags & FST_BANK_HEAD_NORM) {
        if (find_exact(b, FST_TID_OUTPUT_NORM, -1, &t)) return err(FST_ENOTREADY, "output norm (TID 1) missing");
        if ((rc = need_shape(t, (uint64_t)hd, 1, "output norm"))) return rc;
        std::vector<uint16_t> w;
        if ((rc = read_bf16(b, t, w))) return rc;
        if ((rc = fst_upload_norm(ctx, cfg.n_layers, w.data()))) return rc;
    }
    if (flags & FST_BANK_HEAD_LM) {
        if (find_exact(b, FST_TID_LM_HEAD, -1, &t)) return err(FST_ENOTREADY, "LM head (TID 2) missing");
        if ((rc = need_shape(t, (uint64_t)cfg.vocab_size, (uint64_t)hd, "LM head"))) return rc;
        std::vector<uint16_t> w;
        if ((rc = read_bf16(b, t, w))) return rc;
        if ((rc = fst_upload_lm_head_bf16(ctx, w.data()))) return rc;
    }
    if ((flags & FST_BANK_HEAD_HC) && find_exact(b, FST_TID_HC_HEAD_FN, -1, &t) == FST_OK) {
        fst_bank_tensor ts, tb;
        if ((rc = need_shape(t, 4, (uint64_t)4 * hd, "HC head fn"))) return rc;
        std::vector<uint16_t> fn;
        std::vector<float> sc(1, 1.0f), bs;
        if ((rc = read_bf16(b, t, fn))) return rc;
        if (find_exact(b, FST_TID_HC_HEAD_SCALE, -1, &ts) == FST_OK && (rc = read_f32(b, ts, sc))) return rc;
        if (find_exact(b, FST_TID_HC_HEAD_BASE, -1, &tb) == FST_OK && (rc = read_f32(b, tb, bs))) return rc;
        if (sc.empty() || (!bs.empty() && bs.size() != 4)) return err(FST_EINVAL, "HC head scale/base sizes");
        if ((rc = fst_upload_hc_head(ctx, fn.data(), sc[0], bs.empty() ? nullptr : bs.data()))) return rc;
    }
    return FST_OK;
}

}  // extern "C"
