"""ctypes bindings for the CPU oracle (oracle/_build/libfst_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU
baseline, never as part of the product path.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libfst_oracle.so")

P = C.c_void_p
_o = None


def build():
    import subprocess
    subprocess.run(["bash", os.path.join(HERE, "build.sh")], check=True)


def lib():
    global _o
    if _o is not None:
        return _o
    if not os.path.exists(LIB_PATH):
        build()
    L = C.CDLL(LIB_PATH)
    sig = {
        "fo_q4k_dequant": (C.c_int, [P, C.c_size_t, P]),
        "fo_mxfp4_dequant": (C.c_int, [P, C.c_size_t, P]),
        "fo_q4k_scale_min": (None, [C.c_int, P, P, P]),
        "fo_fp16_to_f32": (C.c_float, [C.c_uint16]),
        "fo_f32_to_bf16": (C.c_uint16, [C.c_float]),
        "fo_expert_ffn": (C.c_int, [C.c_int, P, C.c_int, C.c_int, P, C.c_int, C.c_float, P]),
        "fo_expert_ffn_f32": (None, [P, P, P, C.c_int, C.c_int, P, C.c_int, C.c_float, P]),
        "fo_router_logits": (None, [P, P, C.c_int, C.c_int, C.c_int, P]),
        "fo_router": (C.c_int, [P, P, P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int,
                                P, P, P, P]),
        "fo_combine": (None, [P, P, P, C.c_int, C.c_int, C.c_int, P, P]),
        "fo_argmax": (C.c_int, [P, C.c_int]),
        "fo_top_p_fixed": (C.c_uint64, [C.c_float]),
        "fo_sample_token": (C.c_int, [P, C.c_int, C.c_float, C.c_float, C.c_uint64, C.c_uint64, P]),
        "fo_accept_greedy": (C.c_int, [P, C.c_int, C.c_int, P, P, P]),
        "fo_accept_stochastic": (C.c_int, [P, P, C.c_int, C.c_int, P, C.c_float, C.c_uint64, C.c_uint64, P, P]),
        "fo_rs_row_stats": (None, [P, C.c_int, C.c_float, P, P]),
        "fo_rs_race": (C.c_int, [P, P, C.c_int, C.c_float, C.c_float, C.c_float, C.c_float, C.c_float,
                                 C.c_uint64, C.c_uint64, C.c_uint32]),
        "fo_race_uniform": (C.c_float, [C.c_uint64, C.c_uint64, C.c_uint32, C.c_uint32]),
        "fo_rmsnorm": (None, [P, P, C.c_int, C.c_int, C.c_float, P]),
        "fo_q4k_linear": (C.c_int, [P, C.c_int, C.c_int, P, C.c_int, P]),
        "fo_hc_mix": (None, [P, P, C.c_int, C.c_int, P]),
        "fo_hc_split": (None, [P, P, P, C.c_int, C.c_int, C.c_float, P]),
        "fo_hc_pre": (None, [P, P, P, P, C.c_int, C.c_int, C.c_int, C.c_float, P, P, P]),
        "fo_hc_post": (None, [P, P, P, P, C.c_int, C.c_int, P]),
        "fo_hc_head": (None, [P, P, C.c_float, P, C.c_int, C.c_int, C.c_float, P]),
        "fo_expf": (C.c_float, [C.c_float]),
        "fo_exp_nonpos_n": (None, [P, C.c_int, P]),
        "fo_expf_n": (None, [P, C.c_int, P]),
        "fo_logf": (C.c_float, [C.c_float]),
        "fo_sigmoidf": (C.c_float, [C.c_float]),
        "fo_sqrtsoftplusf": (C.c_float, [C.c_float]),
        "fo_philox4x32_10": (None, [P, P, P]),
        "fo_uniform24": (C.c_uint32, [C.c_uint64, C.c_uint64, C.c_uint32, C.c_uint32]),
        "fo_set_threads": (None, [C.c_int]),
        "fo_get_threads": (C.c_int, []),
    }
    for n, (r, a) in sig.items():
        f = getattr(L, n)
        f.restype = r
        f.argtypes = a
    _o = L
    return L


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def set_threads(n):
    lib().fo_set_threads(int(n))


def q4k_dequant(blocks):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    nb = blocks.nbytes // 144
    out = np.empty(nb * 256, np.float32)
    lib().fo_q4k_dequant(_p(blocks), nb, _p(out))
    return out


def mxfp4_dequant(blocks):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    nb = blocks.nbytes // 17
    out = np.empty(nb * 32, np.float32)
    lib().fo_mxfp4_dequant(_p(blocks), nb, _p(out))
    return out


def expert_ffn(codec, expert, h, hd=4096, inter=2048, swiglu_limit=0.0):
    expert = np.ascontiguousarray(expert, dtype=np.uint8)
    h = np.ascontiguousarray(h, dtype=np.uint16)
    M = h.shape[0]
    y = np.empty((M, hd), np.float32)
    rc = lib().fo_expert_ffn(codec, _p(expert), hd, inter, _p(h), M, swiglu_limit, _p(y))
    assert rc == 0
    return y


def expert_ffn_f32(wg, wu, wd, h, swiglu_limit=0.0):
    inter, hd = wg.shape
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty((h.shape[0], hd), np.float32)
    lib().fo_expert_ffn_f32(_p(np.ascontiguousarray(wg, np.float32)), _p(np.ascontiguousarray(wu, np.float32)),
                            _p(np.ascontiguousarray(wd, np.float32)), hd, inter, _p(h), h.shape[0],
                            swiglu_limit, _p(y))
    return y


def router_logits(h, w_kn):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    w_kn = np.ascontiguousarray(w_kn, dtype=np.uint16)
    M, K = h.shape
    N = w_kn.shape[1]
    out = np.empty((M, N), np.float32)
    lib().fo_router_logits(_p(h), _p(w_kn), M, K, N, _p(out))
    return out


def router(h, w_kn, bias=None, top_k=6, score_func=0, route_scale=1.0, round_logits_bf16=0, hash_rows=None):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    w_kn = np.ascontiguousarray(w_kn, dtype=np.uint16)
    M, K = h.shape
    N = w_kn.shape[1]
    e = np.empty((M, top_k), np.int32)
    w = np.empty((M, top_k), np.float32)
    lg = np.empty((M, N), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    hr = None if hash_rows is None else np.ascontiguousarray(hash_rows, np.int32)
    rc = lib().fo_router(_p(h), _p(w_kn), _p(b), M, K, N, top_k, score_func, route_scale, round_logits_bf16,
                         _p(hr), _p(e), _p(w), _p(lg))
    assert rc == 0
    return e, w, lg


def combine(y_routed, y_shared, wts):
    M, tk, hd = y_routed.shape
    out = np.empty((M, hd), np.uint16)
    of = np.empty((M, hd), np.float32)
    lib().fo_combine(_p(np.ascontiguousarray(y_routed, np.float32)),
                     _p(None if y_shared is None else np.ascontiguousarray(y_shared, np.float32)),
                     _p(np.ascontiguousarray(wts, np.float32)), M, tk, hd, _p(out), _p(of))
    return out, of


def argmax(row):
    row = np.ascontiguousarray(row, np.float32)
    return lib().fo_argmax(_p(row), row.size)


def accept_greedy(target, draft):
    target = np.ascontiguousarray(target, np.float32)
    kp1, V = target.shape
    draft = np.ascontiguousarray(draft, np.int32)
    n = C.c_int32()
    tok = np.full(kp1, -1, np.int32)
    lib().fo_accept_greedy(_p(target), kp1 - 1, V, _p(draft), C.byref(n), _p(tok))
    return n.value, tok[: n.value + 1]


def sample_token(logits, temperature, top_p, seed, seq):
    """fo_sample_token: (token, size of the top-p set)."""
    logits = np.ascontiguousarray(logits, np.float32)
    n = C.c_int()
    t = lib().fo_sample_token(_p(logits), logits.shape[-1], temperature, top_p, seed, seq, C.byref(n))
    return t, n.value


def accept_stochastic(target, draft_logits, draft, temperature, seed, seq):
    target = np.ascontiguousarray(target, np.float32)
    kp1, V = target.shape
    dl = np.ascontiguousarray(draft_logits, np.float32)
    draft = np.ascontiguousarray(draft, np.int32)
    n = C.c_int32()
    tok = np.full(kp1, -1, np.int32)
    rc = lib().fo_accept_stochastic(_p(target), _p(dl), kp1 - 1, V, _p(draft), temperature, seed, seq,
                                    C.byref(n), _p(tok))
    assert rc == 0
    return n.value, tok[: n.value + 1]


def rs_row_stats(row, inv_t=1.0):
    """fo_rs_row_stats: a row's softmax (max, sum) in the device's fixed order."""
    row = np.ascontiguousarray(row, np.float32)
    M, S = C.c_float(), C.c_float()
    lib().fo_rs_row_stats(_p(row), row.shape[-1], inv_t, C.byref(M), C.byref(S))
    return M.value, S.value


def rs_race(trow, drow, inv_t, seed, seq, pos):
    """fo_rs_race with the rows' statistics computed by rs_row_stats (drow None: the bonus race)."""
    trow = np.ascontiguousarray(trow, np.float32)
    Mt, St = rs_row_stats(trow, inv_t)
    if drow is None:
        return lib().fo_rs_race(_p(trow), None, trow.shape[-1], inv_t, Mt, St, 0.0, 0.0, seed, seq, pos)
    drow = np.ascontiguousarray(drow, np.float32)
    Md, Sd = rs_row_stats(drow, inv_t)
    return lib().fo_rs_race(_p(trow), _p(drow), trow.shape[-1], inv_t, Mt, St, Md, Sd, seed, seq, pos)


def rmsnorm(x, w, eps=1e-6):
    x = np.ascontiguousarray(x, np.float32)
    M, d = x.shape
    out = np.empty((M, d), np.uint16)
    lib().fo_rmsnorm(_p(x), _p(np.ascontiguousarray(w, np.uint16)), M, d, eps, _p(out))
    return out


def q4k_linear(blocks, x, N, K):
    """y[M][N] = x . W^T for a packed Q4_K matrix W [N][K/256] (LM head)."""
    x = np.ascontiguousarray(x, np.uint16)
    M = x.shape[0]
    y = np.empty((M, N), np.float32)
    rc = lib().fo_q4k_linear(_p(np.ascontiguousarray(blocks, np.uint8)), N, K, _p(x), M, _p(y))
    if rc:
        raise ValueError("fo_q4k_linear failed (%d)" % rc)
    return y


def resid_norm(h, y, w, eps=1e-6):
    """Residual add then RMSNorm: x = bf16(h + y) (or h), returns (x bf16, RMSNorm(x) bf16)."""
    from fastar_amd import bf16_to_f32, f32_to_bf16  # bit helpers only (numpy)
    x = np.ascontiguousarray(h, np.uint16)
    if y is not None:
        x = f32_to_bf16(bf16_to_f32(x) + bf16_to_f32(np.ascontiguousarray(y, np.uint16))).reshape(x.shape)
    return x, rmsnorm(bf16_to_f32(x).reshape(x.shape), w, eps)


HC_ITERS, HC_EPS = 20, 1e-6


def hc_mix(flat_bf, fnT):
    fnT = np.ascontiguousarray(fnT, np.uint16)
    nout, K = fnT.shape
    mix = np.empty(nout, np.float32)
    lib().fo_hc_mix(_p(np.ascontiguousarray(flat_bf, np.uint16)), _p(fnT), K, nout, _p(mix))
    return mix


def hc_split(mix, scale, base, n=4, iters=HC_ITERS, eps=HC_EPS):
    out = np.empty(2 * n + n * n, np.float32)
    lib().fo_hc_split(_p(np.ascontiguousarray(mix, np.float32)), _p(np.ascontiguousarray(scale, np.float32)),
                      _p(np.ascontiguousarray(base, np.float32)), n, iters, eps, _p(out))
    return out


def hc_pre(h_hc, fnT, scale, base, iters=HC_ITERS, eps=HC_EPS):
    """h_hc [M][4][d] bf16, fnT [24][4d] bf16 -> (cur [M][d] bf16, post [M][4], comb [M][16])."""
    h_hc = np.ascontiguousarray(h_hc, np.uint16)
    M, _, d = h_hc.shape
    cur = np.empty((M, d), np.uint16)
    post = np.empty((M, 4), np.float32)
    comb = np.empty((M, 16), np.float32)
    lib().fo_hc_pre(_p(h_hc), _p(np.ascontiguousarray(fnT, np.uint16)), _p(np.ascontiguousarray(scale, np.float32)),
                    _p(np.ascontiguousarray(base, np.float32)), M, d, iters, eps, _p(cur), _p(post), _p(comb))
    return cur, post, comb


def hc_post(bo, h_hc, post, comb):
    h_hc = np.ascontiguousarray(h_hc, np.uint16)
    M, _, d = h_hc.shape
    out = np.empty_like(h_hc)
    lib().fo_hc_post(_p(np.ascontiguousarray(bo, np.uint16)), _p(h_hc), _p(np.ascontiguousarray(post, np.float32)),
                     _p(np.ascontiguousarray(comb, np.float32)), M, d, _p(out))
    return out


def hc_head(h_hc, fnT, scale, base, eps=HC_EPS):
    h_hc = np.ascontiguousarray(h_hc, np.uint16)
    M, _, d = h_hc.shape
    out = np.empty((M, d), np.uint16)
    b = None if base is None else np.ascontiguousarray(base, np.float32)
    lib().fo_hc_head(_p(h_hc), _p(np.ascontiguousarray(fnT, np.uint16)), float(scale), _p(b), M, d, eps, _p(out))
    return out


def philox(ctr, key):
    c = np.ascontiguousarray(ctr, np.uint32)
    k = np.ascontiguousarray(key, np.uint32)
    o = np.empty(4, np.uint32)
    lib().fo_philox4x32_10(_p(c), _p(k), _p(o))
    return o


def uniform24(seed, seq, pos, stream):
    return lib().fo_uniform24(seed, seq, pos, stream)
