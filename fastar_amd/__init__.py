"""fastar_amd — MI355X (gfx950) DSpark block-verification hot path.

Python bindings over the C-ABI in include/fst_hip.h (libfst_hip.so, built
in-tree by fastar_amd.build).  The product path is the HIP library; these
bindings only move numpy buffers across the ABI.  Loading fails loudly if
the library has not been built; there is no CPU fallback.
"""
import ctypes as C
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "lib", "libfst_hip.so")
HEADERS = [os.path.join(ROOT, "include", "fst_hip.h")]

FST_OK, FST_EINVAL, FST_ENOMEM, FST_EHIP, FST_ENODEV, FST_ENOTREADY = range(6)
CODEC_Q4K, CODEC_MXFP4 = 0, 1
SCORE_SIGMOID, SCORE_SQRTSOFTPLUS = 0, 1


class FstError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("fst error %d: %s" % (code, msg))
        self.code = code


class fst_config(C.Structure):
    _fields_ = [
        ("hidden_dim", C.c_int), ("inter_dim", C.c_int), ("n_experts", C.c_int), ("top_k", C.c_int),
        ("n_layers", C.c_int), ("max_tokens", C.c_int), ("codec", C.c_int), ("has_shared", C.c_int),
        ("score_func", C.c_int), ("route_scale", C.c_float), ("round_logits_bf16", C.c_int),
        ("n_hash_layers", C.c_int), ("vocab_size", C.c_int), ("swiglu_limit", C.c_float),
        ("device", C.c_int),
    ]


class fst_timings(C.Structure):
    _fields_ = [("n", C.c_int), ("name", C.c_char_p * 16), ("ms", C.c_float * 16)]


_lib = None

P = C.c_void_p
I32 = C.c_int32
U64 = C.c_uint64
SZ = C.c_size_t

_SIGS = {
    "fst_config_default": (None, [P]),
    "fst_last_error": (C.c_char_p, []),
    "fst_abi_version": (C.c_int, []),
    "fst_expert_bytes": (SZ, [P]),
    "fst_create": (C.c_int, [P, P]),
    "fst_destroy": (None, [P]),
    "fst_stream": (P, [P]),
    "fst_sync": (C.c_int, [P]),
    "fst_device_alloc": (P, [P, SZ]),
    "fst_device_free": (None, [P, P]),
    "fst_copy_to_device": (C.c_int, [P, P, P, SZ]),
    "fst_copy_to_host": (C.c_int, [P, P, P, SZ]),
    "fst_upload_expert": (C.c_int, [P, C.c_int, C.c_int, P, SZ]),
    "fst_upload_router_bf16": (C.c_int, [P, C.c_int, P, P]),
    "fst_upload_router_f32": (C.c_int, [P, C.c_int, P, P]),
    "fst_upload_hash_table": (C.c_int, [P, C.c_int, P]),
    "fst_expert_device_ptr": (P, [P, C.c_int, C.c_int]),
    "fst_router": (C.c_int, [P, C.c_int, P, C.c_int, P, P, P]),
    "fst_expert_ffn": (C.c_int, [P, C.c_int, P, P, C.c_int, P, C.c_int, P]),
    "fst_shared_expert": (C.c_int, [P, C.c_int, P, P, C.c_int]),
    "fst_moe_layer": (C.c_int, [P, C.c_int, P, C.c_int, P, P, P, P]),
    "fst_moe_layer_dev": (C.c_int, [P, C.c_int, P, C.c_int, P, P, P, P]),
    "fst_moe_ffn_dev": (C.c_int, [P, C.c_int, P, C.c_int, P, P, C.c_int, P, P, P]),
    "fst_accept_greedy": (C.c_int, [P, P, C.c_int, C.c_int, C.c_int, P, P, P]),
    "fst_accept_stochastic": (C.c_int, [P, P, P, C.c_int, C.c_int, C.c_int, P, C.c_float, U64, U64, P, P]),
    "fst_accept_greedy_dev": (C.c_int, [P, P, C.c_int, C.c_int, C.c_int, P, P, P]),
    "fst_accept_stochastic_dev": (C.c_int, [P, P, P, C.c_int, C.c_int, C.c_int, P, C.c_float, U64, U64, P, P]),
    "fst_set_wait_limit": (C.c_int, [P, C.c_int]),
    "fst_set_fused": (C.c_int, [P, C.c_int]),
    "fst_set_small_m": (C.c_int, [P, C.c_int]),
    "fst_final_head": (C.c_int, [P, P, C.c_int, P]),
    "fst_sample_token": (C.c_int, [P, P, C.c_int, C.c_float, C.c_float, U64, U64, P]),
    "fst_sample_token_dev": (C.c_int, [P, P, C.c_int, C.c_int, C.c_float, C.c_float, U64, U64, P]),
    "fst_accept_check": (C.c_int, [P, C.c_int]),
    "fst_moe_check": (C.c_int, [P]),
    "fst_device_error_status": (C.c_int, [C.c_int]),
    "fst_accept_greedy_dev_noalloc": (C.c_int, [P, P, C.c_int, C.c_int, C.c_int, P, P, P]),
    "fst_dequant": (C.c_int, [P, C.c_int, P, SZ, P, P]),
    "fst_set_profiling": (C.c_int, [P, C.c_int]),
    "fst_last_timings": (C.c_int, [P, P]),
    "fst_kernel_ring": (C.c_int, [P, C.c_int]),
    "fst_kernel_ring_read": (C.c_int, [P, P, C.c_int, P]),
    "fst_last_active_experts": (C.c_int, [P, P]),
    "fst_device_copy": (C.c_int, [P, P, P, SZ]),
    "fst_upload_norm": (C.c_int, [P, C.c_int, P]),
    "fst_lm_head_bytes": (SZ, [P]),
    "fst_upload_lm_head": (C.c_int, [P, P, SZ]),
    "fst_rmsnorm_dev": (C.c_int, [P, C.c_int, P, P, C.c_int, P, P]),
    "fst_lm_head_dev": (C.c_int, [P, P, C.c_int, P]),
    "fst_verify_forward_dev": (C.c_int, [P, P, C.c_int, P, P]),
    "fst_verify_forward": (C.c_int, [P, P, C.c_int, P, P]),
    "fst_upload_shared_bf16": (C.c_int, [P, C.c_int, P, P, P]),
    "fst_get_config": (C.c_int, [P, P]),
    "fst_bank_open": (C.c_int, [C.c_char_p, P]),
    "fst_bank_close": (None, [P]),
    "fst_bank_get_header": (C.c_int, [P, P]),
    "fst_bank_n_tensors": (C.c_int, [P]),
    "fst_bank_tensor_at": (C.c_int, [P, C.c_int, P]),
    "fst_bank_find": (C.c_int, [P, C.c_uint32, C.c_int, P]),
    "fst_bank_read_tensor": (C.c_int, [P, P, P, SZ]),
    "fst_bank_read_expert": (C.c_int, [P, C.c_int, C.c_int, P, SZ]),
    "fst_bank_config": (C.c_int, [P, P]),
    "fst_bank_load_layer": (C.c_int, [P, P, C.c_int, C.c_int]),
    "fst_bank_load_head": (C.c_int, [P, P, C.c_int]),
    "fst_upload_lm_head_bf16": (C.c_int, [P, P]),
    "fst_upload_hc": (C.c_int, [P, C.c_int, P, P, P]),
    "fst_upload_hc_head": (C.c_int, [P, P, C.c_float, P]),
    "fst_hc_pre_dev": (C.c_int, [P, C.c_int, P, C.c_int, P, P, P]),
    "fst_hc_post_dev": (C.c_int, [P, P, P, P, P, C.c_int]),
    "fst_hc_head_dev": (C.c_int, [P, P, C.c_int, P]),
    "fst_synth_experts_dev": (C.c_int, [P, U64, C.c_int, C.c_int, C.c_int, U64, C.c_float]),
    "fst_synth_lm_head_dev": (C.c_int, [P, U64, U64, C.c_float]),
    "fst_synth_q4k_blocks": (C.c_int, [U64, U64, SZ, C.c_float, P]),
    "fst_synth_q4k_expert": (C.c_int, [U64, U64, C.c_int, C.c_int, C.c_float, P]),
    "fst_synth_mxfp4_expert": (C.c_int, [U64, U64, C.c_int, C.c_int, C.c_int, C.c_int, P]),
    "fst_synth_normal_bf16": (C.c_int, [U64, U64, SZ, C.c_float, C.c_float, P]),
    "fst_synth_normal_f32": (C.c_int, [U64, U64, SZ, C.c_float, C.c_float, P]),
}


def header_symbols():
    """Function names declared in include/*.h (the ABI contract)."""
    names = []
    for h in HEADERS:
        txt = open(h).read()
        txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
        for m in re.finditer(r"^\s*[A-Za-z_][\w\s\*]*?\b(fst_\w+)\s*\(", txt, flags=re.M):
            names.append(m.group(1))
    return sorted(set(names))


def lib():
    """Loads libfst_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError("libfst_hip.so not built: run `python -m fastar_amd.build` (%s)" % LIB_PATH)
    L = C.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def _check(rc):
    if rc != FST_OK:
        raise FstError(rc, lib().fst_last_error().decode(errors="replace"))


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def default_config(**kw):
    c = fst_config()
    lib().fst_config_default(C.byref(c))
    for k, v in kw.items():
        if not hasattr(c, k):
            raise TypeError("unknown config field %s" % k)
        setattr(c, k, v)
    return c


def expert_bytes(cfg):
    return lib().fst_expert_bytes(C.byref(cfg))


# --------------------------------------------------------------- synthetic data

def synth_q4k_expert(seed, expert_id, hd=4096, inter=2048, d_sigma=0.01):
    out = np.empty(3 * hd * inter // 256 * 144, dtype=np.uint8)
    _check(lib().fst_synth_q4k_expert(seed, expert_id, hd, inter, d_sigma, _ptr(out)))
    return out


def synth_q4k_blocks(seed, matrix_id, nblocks, d_sigma=0.01):
    out = np.empty(nblocks * 144, dtype=np.uint8)
    _check(lib().fst_synth_q4k_blocks(seed, matrix_id, nblocks, d_sigma, _ptr(out)))
    return out


def lm_head_bytes(cfg):
    return lib().fst_lm_head_bytes(C.byref(cfg))


def synth_mxfp4_expert(seed, expert_id, hd=4096, inter=2048, e_lo=108, e_hi=128):
    out = np.empty(3 * hd * inter // 32 * 17, dtype=np.uint8)
    _check(lib().fst_synth_mxfp4_expert(seed, expert_id, hd, inter, e_lo, e_hi, _ptr(out)))
    return out


def synth_normal_bf16(seed, stream, shape, mean=0.0, std=1.0):
    out = np.empty(shape, dtype=np.uint16)
    _check(lib().fst_synth_normal_bf16(seed, stream, out.size, mean, std, _ptr(out)))
    return out


def synth_normal_f32(seed, stream, shape, mean=0.0, std=1.0):
    out = np.empty(shape, dtype=np.float32)
    _check(lib().fst_synth_normal_f32(seed, stream, out.size, mean, std, _ptr(out)))
    return out


def bf16_to_f32(a):
    return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a):
    """Round-to-nearest-even float32 -> bf16 bits (NaN kept quiet)."""
    a = np.asarray(a, dtype=np.float32)
    u = np.atleast_1d(a).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r.reshape(a.shape)


# --------------------------------------------------------------------- context

class Context:
    """One GPU context (stream + resident experts + scratch)."""

    def __init__(self, cfg=None, **kw):
        self.cfg = cfg if cfg is not None else default_config(**kw)
        h = C.c_void_p()
        _check(lib().fst_create(C.byref(self.cfg), C.byref(h)))
        self.h = h
        self.expert_bytes = expert_bytes(self.cfg)

    def close(self):
        if getattr(self, "h", None):
            lib().fst_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    # residency
    def upload_expert(self, lid, eid, packed):
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        _check(lib().fst_upload_expert(self.h, lid, eid, _ptr(packed), packed.nbytes))

    def upload_router_bf16(self, lid, w_kn, bias=None):
        w = np.ascontiguousarray(w_kn, dtype=np.uint16)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        _check(lib().fst_upload_router_bf16(self.h, lid, _ptr(w), _ptr(b)))

    def upload_router_f32(self, lid, w_kn, bias=None):
        w = np.ascontiguousarray(w_kn, dtype=np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        _check(lib().fst_upload_router_f32(self.h, lid, _ptr(w), _ptr(b)))

    def upload_hash_table(self, lid, table):
        t = np.ascontiguousarray(table, dtype=np.int32)
        _check(lib().fst_upload_hash_table(self.h, lid, _ptr(t)))

    # path pieces
    def router(self, lid, h, input_ids=None):
        h = np.ascontiguousarray(h, dtype=np.uint16)
        M = h.shape[0]
        tk = self.cfg.top_k
        e = np.empty((M, tk), np.int32)
        w = np.empty((M, tk), np.float32)
        ids = None if input_ids is None else np.ascontiguousarray(input_ids, dtype=np.int32)
        _check(lib().fst_router(self.h, lid, _ptr(h), M, _ptr(ids), _ptr(e), _ptr(w)))
        return e, w

    def expert_ffn(self, lid, h, eids, wts):
        h = np.ascontiguousarray(h, dtype=np.uint16)
        eids = np.ascontiguousarray(eids, dtype=np.int32)
        wts = np.ascontiguousarray(wts, dtype=np.float32)
        M = h.shape[0]
        out = np.empty_like(h)
        _check(lib().fst_expert_ffn(self.h, lid, _ptr(h), _ptr(out), M, _ptr(eids), eids.shape[1], _ptr(wts)))
        return out

    def shared_expert(self, lid, h):
        h = np.ascontiguousarray(h, dtype=np.uint16)
        out = np.empty_like(h)
        _check(lib().fst_shared_expert(self.h, lid, _ptr(h), _ptr(out), h.shape[0]))
        return out

    def moe_layer(self, lid, h, input_ids=None):
        h = np.ascontiguousarray(h, dtype=np.uint16)
        M = h.shape[0]
        tk = self.cfg.top_k
        out = np.empty_like(h)
        e = np.empty((M, tk), np.int32)
        w = np.empty((M, tk), np.float32)
        ids = None if input_ids is None else np.ascontiguousarray(input_ids, dtype=np.int32)
        _check(lib().fst_moe_layer(self.h, lid, _ptr(h), M, _ptr(ids), _ptr(out), _ptr(e), _ptr(w)))
        return out, e, w

    def accept_greedy(self, target, draft):
        target = np.ascontiguousarray(target, dtype=np.float32)
        draft = np.ascontiguousarray(draft, dtype=np.int32)
        n_seq, kp1, V = target.shape
        k = kp1 - 1
        n_acc = np.empty(n_seq, np.int32)
        tok = np.empty((n_seq, kp1), np.int32)
        _check(lib().fst_accept_greedy(self.h, _ptr(target), n_seq, k, V, _ptr(draft), _ptr(n_acc), _ptr(tok)))
        return n_acc, tok

    def accept_stochastic(self, target, draft_logits, draft, temperature, seed, seq_base=0):
        target = np.ascontiguousarray(target, dtype=np.float32)
        dl = np.ascontiguousarray(draft_logits, dtype=np.float32)
        draft = np.ascontiguousarray(draft, dtype=np.int32)
        n_seq, kp1, V = target.shape
        k = kp1 - 1
        n_acc = np.empty(n_seq, np.int32)
        tok = np.empty((n_seq, kp1), np.int32)
        _check(lib().fst_accept_stochastic(self.h, _ptr(target), _ptr(dl), n_seq, k, V, _ptr(draft),
                                           temperature, seed, seq_base, _ptr(n_acc), _ptr(tok)))
        return n_acc, tok

    def set_fused(self, on):
        _check(lib().fst_set_fused(self.h, 1 if on else 0))

    def moe_check(self):
        """Sticky errors of the stream-ordered MoE calls since the last check
        (raises FstError; clears them)."""
        _check(lib().fst_moe_check(self.h))

    def set_wait_limit(self, spins):
        _check(lib().fst_set_wait_limit(self.h, spins))

    def set_small_m(self, on):
        _check(lib().fst_set_small_m(self.h, 1 if on else 0))

    def final_head(self, hs):
        """apply_final_norm_and_lm_head: hs [M][4][hidden] with the HC head
        uploaded, else [M][hidden] -> fp32 logits [M][vocab]."""
        hs = np.ascontiguousarray(hs, dtype=np.uint16)
        M = hs.shape[0]
        out = np.empty((M, self.cfg.vocab_size), np.float32)
        _check(lib().fst_final_head(self.h, _ptr(hs), M, _ptr(out)))
        return out

    def sample_token(self, logits, temperature, top_p, seed, seq=0):
        x = np.ascontiguousarray(logits, dtype=np.float32)
        t = C.c_int32()
        _check(lib().fst_sample_token(self.h, _ptr(x), x.shape[-1], temperature, top_p, seed, seq, C.byref(t)))
        return t.value

    # verify forward (norms, residual stream, LM head)
    def upload_norm(self, lid, w_bf16):
        w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
        _check(lib().fst_upload_norm(self.h, lid, _ptr(w)))

    def upload_lm_head(self, packed):
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        _check(lib().fst_upload_lm_head(self.h, _ptr(packed), packed.nbytes))

    def synth_experts(self, seed, lid, e_first, e_count, id_base, d_sigma=0.01):
        _check(lib().fst_synth_experts_dev(self.h, seed, lid, e_first, e_count, id_base, d_sigma))

    def synth_lm_head(self, seed, matrix_id, d_sigma=0.01):
        _check(lib().fst_synth_lm_head_dev(self.h, seed, matrix_id, d_sigma))

    def upload_shared_bf16(self, lid, gate, up, down):
        """bf16 shared expert: gate, up [inter][hidden], down [hidden][inter]."""
        g, u, d = (np.ascontiguousarray(t, dtype=np.uint16) for t in (gate, up, down))
        _check(lib().fst_upload_shared_bf16(self.h, lid, _ptr(g), _ptr(u), _ptr(d)))

    def upload_lm_head_bf16(self, w):
        w = np.ascontiguousarray(w, dtype=np.uint16)
        _check(lib().fst_upload_lm_head_bf16(self.h, _ptr(w)))

    # Hyper-Connections (4 residual streams)
    def upload_hc(self, lid, fn_bf16, scale, base):
        """fn: bf16 [24][4*hidden]; scale f32[3]; base f32[24]."""
        fn = np.ascontiguousarray(fn_bf16, dtype=np.uint16)
        sc = np.ascontiguousarray(scale, dtype=np.float32)
        b = np.ascontiguousarray(base, dtype=np.float32)
        _check(lib().fst_upload_hc(self.h, lid, _ptr(fn), _ptr(sc), _ptr(b)))

    def upload_hc_head(self, fn_bf16, scale, base=None):
        fn = np.ascontiguousarray(fn_bf16, dtype=np.uint16)
        b = None if base is None else np.ascontiguousarray(base, dtype=np.float32)
        _check(lib().fst_upload_hc_head(self.h, _ptr(fn), float(scale), _ptr(b)))

    def hc_pre(self, lid, h_hc):
        """h_hc [M][4][hidden] bf16 -> (cur [M][hidden] bf16, post [M][4], comb [M][16])."""
        h_hc = np.ascontiguousarray(h_hc, dtype=np.uint16)
        M, d = h_hc.shape[0], h_hc.shape[2]
        dh = self.to_device(h_hc)
        dc, dp, dm = self.dev_alloc(M * d * 2), self.dev_alloc(M * 16), self.dev_alloc(M * 64)
        try:
            _check(lib().fst_hc_pre_dev(self.h, lid, dh, M, dc, dp, dm))
            self.sync()
            return (self.to_host(dc, (M, d), np.uint16), self.to_host(dp, (M, 4), np.float32),
                    self.to_host(dm, (M, 16), np.float32))
        finally:
            for p in (dh, dc, dp, dm):
                self.dev_free(p)

    def hc_post(self, block_out, h_hc, post, comb):
        """Returns the updated [M][4][hidden] streams."""
        h_hc = np.ascontiguousarray(h_hc, dtype=np.uint16)
        M = h_hc.shape[0]
        ptrs = [self.to_device(np.ascontiguousarray(block_out, dtype=np.uint16)), self.to_device(h_hc),
                self.to_device(np.ascontiguousarray(post, dtype=np.float32)),
                self.to_device(np.ascontiguousarray(comb, dtype=np.float32))]
        try:
            _check(lib().fst_hc_post_dev(self.h, ptrs[0], ptrs[1], ptrs[2], ptrs[3], M))
            self.sync()
            return self.to_host(ptrs[1], h_hc.shape, np.uint16)
        finally:
            for p in ptrs:
                self.dev_free(p)

    def hc_head(self, h_hc):
        h_hc = np.ascontiguousarray(h_hc, dtype=np.uint16)
        M, d = h_hc.shape[0], h_hc.shape[2]
        dh, do = self.to_device(h_hc), self.dev_alloc(M * d * 2)
        try:
            _check(lib().fst_hc_head_dev(self.h, dh, M, do))
            self.sync()
            return self.to_host(do, (M, d), np.uint16)
        finally:
            self.dev_free(dh)
            self.dev_free(do)

    def verify_forward(self, h, input_ids=None):
        """h: [M][hidden] bf16, or [M][4][hidden] once HC is uploaded (updated
        copy returned); returns (logits [M][vocab], h_out)."""
        h = np.array(h, dtype=np.uint16, copy=True, order="C")
        M = h.shape[0]
        logits = np.empty((M, self.cfg.vocab_size), np.float32)
        ids = None if input_ids is None else np.ascontiguousarray(input_ids, dtype=np.int32)
        _check(lib().fst_verify_forward(self.h, _ptr(h), M, _ptr(ids), _ptr(logits)))
        return logits, h

    def dequant(self, codec, blocks):
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        bb, be = (144, 256) if codec == CODEC_Q4K else (17, 32)
        nb = blocks.nbytes // bb
        f = np.empty(nb * be, np.float32)
        b = np.empty(nb * be, np.uint16)
        _check(lib().fst_dequant(self.h, codec, _ptr(blocks), nb, _ptr(f), _ptr(b)))
        return f, b

    def set_profiling(self, on):
        _check(lib().fst_set_profiling(self.h, 1 if on else 0))

    def last_timings(self):
        t = fst_timings()
        _check(lib().fst_last_timings(self.h, C.byref(t)))
        return [(t.name[i].decode(), t.ms[i]) for i in range(t.n)]

    def kernel_ring(self, capacity):
        _check(lib().fst_kernel_ring(self.h, int(capacity)))

    def kernel_ring_read(self, max_n=65536):
        buf = np.zeros(max_n, np.float32)
        n = C.c_int()
        _check(lib().fst_kernel_ring_read(self.h, _ptr(buf), max_n, C.byref(n)))
        return buf[: n.value].copy()

    def last_active_experts(self):
        n = C.c_int()
        _check(lib().fst_last_active_experts(self.h, C.byref(n)))
        return n.value

    # device buffers
    def dev_alloc(self, nbytes):
        p = lib().fst_device_alloc(self.h, nbytes)
        if not p:
            raise FstError(FST_ENOMEM, lib().fst_last_error().decode(errors="replace"))
        return p

    def dev_free(self, p):
        lib().fst_device_free(self.h, p)

    def to_device(self, arr, dptr=None):
        arr = np.ascontiguousarray(arr)
        if dptr is None:
            dptr = self.dev_alloc(arr.nbytes)
        _check(lib().fst_copy_to_device(self.h, dptr, _ptr(arr), arr.nbytes))
        return dptr

    def to_host(self, dptr, shape, dtype):
        out = np.empty(shape, dtype)
        _check(lib().fst_copy_to_host(self.h, _ptr(out), dptr, out.nbytes))
        return out

    def sync(self):
        _check(lib().fst_sync(self.h))

    # .fst model file
    def load_bank_layer(self, bank, lid, flags=None):
        _check(lib().fst_bank_load_layer(self.h, bank.h, lid, BANK_LAYER_ALL if flags is None else flags))

    def load_bank_head(self, bank, flags=None):
        _check(lib().fst_bank_load_head(self.h, bank.h, BANK_HEAD_ALL if flags is None else flags))

    def config(self):
        c = fst_config()
        _check(lib().fst_get_config(self.h, C.byref(c)))
        return c


# ---------------------------------------------------------------- .fst files

(BANK_EXPERTS, BANK_ROUTER, BANK_NORM, BANK_SHARED, BANK_HC, BANK_HASH) = (1, 2, 4, 8, 16, 32)
BANK_LAYER_ALL, BANK_BIAS_AS_FP16 = 63, 256
BANK_HEAD_NORM, BANK_HEAD_LM, BANK_HEAD_HC, BANK_HEAD_ALL = 1, 2, 4, 7


class fst_bank_header(C.Structure):
    _fields_ = ([("magic", C.c_char * 4)] +
                [(n, C.c_uint32) for n in ("version", "hidden_dim", "n_layers", "n_experts", "top_k", "n_q_heads",
                                           "n_kv_heads", "head_dim", "inter_dim", "n_shared", "reserved0")] +
                [("vocab_size", C.c_uint64), ("rms_eps", C.c_float), ("rope_freq_base", C.c_float)] +
                [(n, C.c_uint64) for n in ("shared_dir_offset", "shared_dir_count", "expert_bank_offset",
                                           "expert_block_bytes", "expert_block_stride", "expert_count", "dspark",
                                           "dspark_noise_token_id")])


class fst_bank_tensor(C.Structure):
    _fields_ = [("tid", C.c_uint32), ("lid", C.c_uint16), ("sid", C.c_uint16), ("qtype", C.c_uint16),
                ("ndim", C.c_uint16), ("shape", C.c_uint64 * 3), ("offset", C.c_uint64), ("size", C.c_uint64)]


class Bank:
    """An opened .fst model file (fst_bank_open); needs no GPU."""

    def __init__(self, path):
        h = C.c_void_p()
        _check(lib().fst_bank_open(str(path).encode(), C.byref(h)))
        self.h = h
        self.header = fst_bank_header()
        _check(lib().fst_bank_get_header(self.h, C.byref(self.header)))

    def close(self):
        if self.h:
            lib().fst_bank_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def tensors(self):
        out = []
        for i in range(lib().fst_bank_n_tensors(self.h)):
            t = fst_bank_tensor()
            _check(lib().fst_bank_tensor_at(self.h, i, C.byref(t)))
            out.append(t)
        return out

    def find(self, tid, lid=-1):
        t = fst_bank_tensor()
        _check(lib().fst_bank_find(self.h, tid, lid, C.byref(t)))
        return t

    def read_tensor(self, t):
        out = np.empty(t.size, np.uint8)
        _check(lib().fst_bank_read_tensor(self.h, C.byref(t), _ptr(out), out.nbytes))
        return out

    def read_expert(self, lid, eid):
        out = np.empty(self.header.expert_block_bytes, np.uint8)
        _check(lib().fst_bank_read_expert(self.h, lid, eid, _ptr(out), out.nbytes))
        return out

    def config(self, **kw):
        c = fst_config()
        _check(lib().fst_bank_config(self.h, C.byref(c)))
        for k, v in kw.items():
            if not hasattr(c, k):
                raise TypeError("unknown config field %s" % k)
            setattr(c, k, v)
        return c
