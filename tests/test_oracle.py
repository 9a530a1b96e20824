"""CPU tests pinning the oracle (oracle/fst_oracle.c) against golden fixtures,
closed forms, independent implementations and brute force.  No GPU needed."""
import json
import math
import os
from fractions import Fraction

import numpy as np
import pytest

from tests.helpers import bf16_to_f32, make_q4k_block, pack_scale_min, q4k_closed_form

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ------------------------------------------------------------------ numerics

def test_fp16_decode_exhaustive(oracle):
    """All 65,536 fp16 codes against numpy's IEEE binary16 conversion."""
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = codes.view(np.float16).astype(np.float32)
    got = np.array([oracle.lib().fo_fp16_to_f32(int(c)) for c in codes], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_bf16_rne_matches_torch(oracle):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.normal(0, 1, 20000), rng.normal(0, 1e-30, 1000), rng.normal(0, 1e30, 1000),
                        [0.0, -0.0, 1.0, 65504.0, 3.3895314e38]]).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([oracle.lib().fo_f32_to_bf16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, ref)


def _ulps(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


def test_expf_within_2ulp(oracle):
    xs = np.concatenate([np.linspace(-87.0, 88.5, 200001), [-1e-7, 0.0, 1e-7, 0.693147, -0.693147]])
    xs = xs.astype(np.float32)
    got = np.array([oracle.lib().fo_expf(float(v)) for v in xs], np.float32)
    ref = np.exp(xs.astype(np.float64)).astype(np.float32)
    assert oracle.lib().fo_expf(0.0) == 1.0
    assert _ulps(got, ref).max() <= 2
    assert oracle.lib().fo_expf(-100.0) == 0.0
    assert math.isinf(oracle.lib().fo_expf(100.0))


def test_logf_within_2ulp(oracle):
    xs = np.concatenate([np.geomspace(1e-38, 3e38, 100001), np.linspace(0.5, 2.0, 20001)]).astype(np.float32)
    got = np.array([oracle.lib().fo_logf(float(v)) for v in xs], np.float32)
    ref = np.log(xs.astype(np.float64)).astype(np.float32)
    assert _ulps(got, ref).max() <= 2
    assert oracle.lib().fo_logf(1.0) == 0.0


def test_score_functions(oracle):
    xs = np.linspace(-30, 30, 20001).astype(np.float32)
    sg = np.array([oracle.lib().fo_sigmoidf(float(v)) for v in xs], np.float32)
    sp = np.array([oracle.lib().fo_sqrtsoftplusf(float(v)) for v in xs], np.float32)
    x64 = xs.astype(np.float64)
    ref_sg = (1.0 / (1.0 + np.exp(-x64))).astype(np.float32)
    assert _ulps(sg, ref_sg).max() <= 3
    # src/fst_engine.cpp:976-983 evaluates log(1 + exp(x)) in binary32, so
    # 1 + exp(x) is rounded to a multiple of 2^-23 first: compare the squares
    # (softplus) against float64 with that absolute granularity.
    ref_spl = np.where(x64 > 20, x64, np.log1p(np.exp(x64)))
    got_spl = sp.astype(np.float64) ** 2
    assert np.all(np.abs(got_spl - ref_spl) <= 2.5e-7 + 2e-6 * ref_spl)


def test_philox_known_answers(oracle):
    with open(os.path.join(GOLDEN, "philox_kat.json")) as f:
        kat = json.load(f)
    for v in kat:
        assert list(oracle.philox(v["ctr"], v["key"])) == v["out"]


def test_uniform24_range_and_balance(oracle):
    u = np.array([oracle.uniform24(7, 3, i, s) for i in range(4000) for s in (0, 1)], np.float64)
    assert u.min() >= 0 and u.max() < 2 ** 24
    assert abs(u.mean() / 2 ** 24 - 0.5) < 0.02


# -------------------------------------------------------------------- codecs

def test_q4k_golden_blocks(oracle):
    g = np.load(os.path.join(GOLDEN, "q4k_known.npz"))
    got = oracle.q4k_dequant(g["blocks"].reshape(-1)).reshape(g["values"].shape)
    assert np.array_equal(got.view(np.uint32), g["values"].view(np.uint32))


def test_mxfp4_golden_blocks(oracle):
    g = np.load(os.path.join(GOLDEN, "mxfp4_known.npz"))
    got = oracle.mxfp4_dequant(g["blocks"].reshape(-1)).reshape(g["values"].shape)
    same = (got.view(np.uint32) == g["values"].view(np.uint32)) | (np.isinf(got) & np.isinf(g["values"]))
    assert same.all()


def test_q4k_scale_packing_roundtrip(oracle):
    """get_scale_min_k4 (kernels/fst_dequant_q4k_kernel.cc:12-20) inverts the ggml packer."""
    import ctypes as C
    rng = np.random.default_rng(3)
    for _ in range(500):
        sc = rng.integers(0, 64, 8)
        m = rng.integers(0, 64, 8)
        q = pack_scale_min(sc, m)
        for j in range(8):
            a, b = C.c_uint8(), C.c_uint8()
            oracle.lib().fo_q4k_scale_min(j, q.ctypes.data_as(C.c_void_p), C.byref(a), C.byref(b))
            assert (a.value, b.value) == (sc[j], m[j])


def test_q4k_random_blocks_vs_closed_form(oracle):
    rng = np.random.default_rng(11)
    blocks, refs = [], []
    for _ in range(300):
        d16 = np.float16(abs(rng.normal(0, 0.01))).view(np.uint16)
        m16 = np.float16(abs(rng.normal(0, 0.01))).view(np.uint16)
        sc, m, q = rng.integers(0, 64, 8), rng.integers(0, 64, 8), rng.integers(0, 16, 256)
        blocks.append(make_q4k_block(d16, m16, sc, m, q))
        refs.append(q4k_closed_form(float(d16.view(np.float16)), float(m16.view(np.float16)), sc, m, q)
                    .astype(np.float32))
    got = oracle.q4k_dequant(np.concatenate(blocks)).reshape(len(blocks), 256)
    assert np.array_equal(got.view(np.uint32), np.stack(refs).view(np.uint32))


# ----------------------------------------------------------------------- FFN

def _q4k_matrix(rows, cols, fn):
    """Q4_K matrix [rows][cols/256] whose weights are the small integers fn(r, k)
    in [0, 15] (d = 1, sc = 1, dmin = 0), so the weights are exact."""
    out = []
    for r in range(rows):
        for b in range(cols // 256):
            q = np.array([fn(r, b * 256 + i) for i in range(256)], np.int64)
            out.append(make_q4k_block(0x3C00, 0, [1] * 8, [0] * 8, q))
    return np.concatenate(out)


def test_ffn_ones_known_answer(oracle):
    hd, inter = 512, 256
    ones = _q4k_matrix(inter, hd, lambda r, k: 1)
    down = _q4k_matrix(hd, inter, lambda r, k: 1)
    expert = np.concatenate([ones, ones, down])
    h = np.full((2, hd), 0x3F80, np.uint16)
    y = oracle.expert_ffn(0, expert, h, hd, inter)
    act = hd * hd / (1.0 + math.exp(-hd))
    assert np.allclose(y, inter * act, rtol=1e-6)


def test_ffn_selector_known_answer(oracle):
    """gate = up = selector (row n picks input n), down = selector^T: y[n] =
    silu(x[n]) * x[n] for n < inter and 0 above."""
    hd, inter = 512, 256
    sel = _q4k_matrix(inter, hd, lambda r, k: 1 if k == r else 0)
    down = _q4k_matrix(hd, inter, lambda r, k: 1 if k == r else 0)
    expert = np.concatenate([sel, sel, down])
    rng = np.random.default_rng(2)
    x = rng.normal(0, 1, (3, hd)).astype(np.float32)
    h = (x.view(np.uint32) >> 16).astype(np.uint16)
    xf = bf16_to_f32(h).astype(np.float64)
    y = oracle.expert_ffn(0, expert, h, hd, inter)
    ref = np.zeros((3, hd))
    ref[:, :inter] = xf[:, :inter] / (1 + np.exp(-xf[:, :inter])) * xf[:, :inter]
    assert np.allclose(y, ref, rtol=1e-6, atol=1e-7)


def test_ffn_orientation_and_float64(oracle):
    """A.B^T with B[N][K] (scripts/fst_validate_gemms.py:173-186): the oracle
    matches a float64 A.B^T restatement and is far from the transposed product."""
    hd, inter = 512, 512
    rng = np.random.default_rng(4)
    wg = rng.normal(0, 0.05, (inter, hd))
    wu = rng.normal(0, 0.05, (inter, hd))
    wd = rng.normal(0, 0.05, (hd, inter))
    h = ((rng.normal(0, 1, (4, hd)).astype(np.float32).view(np.uint32)) >> 16).astype(np.uint16)
    x = bf16_to_f32(h).astype(np.float64)
    y = oracle.expert_ffn_f32(wg, wu, wd, h)
    g, u = x @ wg.T, x @ wu.T
    ref = (g / (1 + np.exp(-g)) * u) @ wd.T
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) < 1e-5
    g2, u2 = x @ wg, x @ wu  # wrong transpose (square matrices so it is defined)
    wrong = (g2 / (1 + np.exp(-g2)) * u2) @ wd
    assert np.linalg.norm(y - wrong) > 10 * np.linalg.norm(y - ref)


# -------------------------------------------------------------------- router

def _router_inputs(seed, M=5, K=512, N=64):
    rng = np.random.default_rng(seed)
    h = ((rng.normal(0, 1, (M, K)).astype(np.float32).view(np.uint32)) >> 16).astype(np.uint16)
    w = ((rng.normal(0, 0.05, (K, N)).astype(np.float32).view(np.uint32)) >> 16).astype(np.uint16)
    return h, w


def test_router_logits_close_to_float64(oracle):
    h, w = _router_inputs(1)
    lg = oracle.router_logits(h, w)
    ref = bf16_to_f32(h).astype(np.float64) @ bf16_to_f32(w).astype(np.float64)
    assert np.max(np.abs(lg - ref)) < 1e-5 * np.max(np.abs(ref)) + 1e-6


@pytest.mark.parametrize("score_func", [0, 1])
def test_router_topk_matches_sorted_scores(oracle, score_func):
    h, w = _router_inputs(7)
    bias = np.random.default_rng(8).normal(0, 0.1, 64).astype(np.float32)
    e, wt, lg = oracle.router(h, w, bias, 6, score_func, 1.5, 0)
    f = oracle.lib().fo_sigmoidf if score_func == 0 else oracle.lib().fo_sqrtsoftplusf
    for m in range(h.shape[0]):
        sc = np.array([f(float(v)) for v in lg[m]], np.float32)
        sel = (sc + bias).astype(np.float32)
        order = np.lexsort((np.arange(64), -sel.astype(np.float64)))[:6]
        assert list(e[m]) == list(order)
        ref_w = sc[order].astype(np.float64) / float(np.float32(sc[order].sum()) + np.float32(1e-12)) * 1.5
        assert np.allclose(wt[m], ref_w, rtol=1e-6)
        assert abs(float(wt[m].sum()) - 1.5) < 1e-5


def test_router_ties_prefer_lower_id(oracle):
    h, w = _router_inputs(9)
    for a, b in [(3, 40), (7, 2), (10, 11)]:
        w[:, b] = w[:, a]
    e, _, lg = oracle.router(h, w, None, 6, 0, 1.0, 0)
    for m in range(h.shape[0]):
        for a, b in [(3, 40), (7, 2), (10, 11)]:
            lo, hi = min(a, b), max(a, b)
            if hi in e[m]:
                assert lo in e[m] and list(e[m]).index(lo) < list(e[m]).index(hi)


def test_router_hash_rows_and_bf16_rounding(oracle):
    h, w = _router_inputs(12)
    rows = np.array([[1, 2, 3, 4, 5, 6], [60, 50, 40, 30, 20, 10]] * 2 + [[0, 1, 2, 3, 4, 5]], np.int32)
    e, wt, lg = oracle.router(h, w, None, 6, 1, 1.5, 1, hash_rows=rows)
    assert np.array_equal(e, rows)
    assert np.array_equal(lg, bf16_to_f32((lg.view(np.uint32) >> 16).astype(np.uint16)))  # already bf16


# ------------------------------------------------------------------ combine

def test_combine_matches_float64(oracle):
    rng = np.random.default_rng(1)
    yr = rng.normal(0, 1, (3, 6, 256)).astype(np.float32)
    ys = rng.normal(0, 1, (3, 256)).astype(np.float32)
    wt = rng.random((3, 6)).astype(np.float32)
    out, of = oracle.combine(yr, ys, wt)
    ref = np.einsum("mj,mjd->md", wt.astype(np.float64), yr.astype(np.float64)) + ys
    assert np.allclose(of, ref, rtol=1e-5, atol=1e-6)
    assert np.array_equal(out, ((of.view(np.uint32) + 0x7FFF + ((of.view(np.uint32) >> 16) & 1)) >> 16)
                          .astype(np.uint16))


# ---------------------------------------------------------------- acceptance

def test_greedy_golden_planted(oracle):
    g = np.load(os.path.join(GOLDEN, "accept_planted.npz"))
    for t, d, n, tok in zip(g["target"], g["draft"], g["n_acc"], g["tokens"]):
        rn, rt = oracle.accept_greedy(t, d)
        assert rn == n
        assert np.array_equal(rt, tok[: n + 1])


def test_argmax_reference_semantics(oracle):
    x = np.array([1.0, 3.0, 3.0, 2.0], np.float32)
    assert oracle.argmax(x) == 1                        # first maximum wins
    assert oracle.argmax(np.array([np.nan, 5.0, 6.0], np.float32)) == 0   # NaN at 0 pins
    assert oracle.argmax(np.array([1.0, np.nan, 6.0], np.float32)) == 2   # NaN skipped
    assert oracle.argmax(np.array([-np.inf, -np.inf], np.float32)) == 0


def _fixed_probs(oracle, row, inv_t):
    l = (row.astype(np.float32) * np.float32(inv_t)).astype(np.float32)
    mx = np.max(l)
    E = []
    for v in l:
        if v == mx:
            E.append(2 ** 32)
        else:
            e = np.float32(oracle.lib().fo_expf(float(np.float32(v - mx))))
            E.append(int(np.float32(e * np.float32(4294967296.0))))
    return E


@pytest.mark.parametrize("seed", range(40))
def test_stochastic_bruteforce_small_vocab(oracle, seed):
    """Rational-arithmetic restatement of the decision and the residual draw."""
    rng = np.random.default_rng(seed)
    k, V = 3, 5
    t = rng.normal(0, 1.5, (k + 1, V)).astype(np.float32)
    d = rng.normal(0, 1.5, (k, V)).astype(np.float32)
    draft = rng.integers(0, V, k).astype(np.int32)
    n, tok = oracle.accept_stochastic(t, d, draft, 1.0, seed, 5)
    emitted = []
    for i in range(k + 1):
        P = _fixed_probs(oracle, t[i], 1.0)
        Sp = sum(P)
        if i == k:
            u2 = oracle.uniform24(seed, 5, i, 1)
            target = (u2 * Sp) >> 24
            c = 0
            for v in range(V):
                c += P[v]
                if c > target:
                    emitted.append(v)
                    break
            break
        Q = _fixed_probs(oracle, d[i], 1.0)
        Sq = sum(Q)
        x = int(draft[i])
        u = Fraction(oracle.uniform24(seed, 5, i, 0), 2 ** 24)
        if u * Fraction(Q[x], Sq) < Fraction(P[x], Sp):
            emitted.append(x)
            continue
        R = [max(0, P[v] * Sq - Q[v] * Sp) for v in range(V)]
        u2 = oracle.uniform24(seed, 5, i, 1)
        tot = sum(R) if sum(R) > 0 else Sp
        vals = R if sum(R) > 0 else P
        target = (u2 * tot) >> 24
        c = 0
        for v in range(V):
            c += vals[v]
            if c > target:
                emitted.append(v)
                break
        break
    assert n == len(emitted) - 1
    assert list(tok) == emitted


def test_speculative_sampling_preserves_target_distribution(oracle):
    """Leviathan et al. 2023: with x ~ q the first emitted token is distributed
    as p.  Checked on V=4 over 6000 draws (chi-square, generous bound)."""
    V = 4
    p_log = np.log(np.array([0.1, 0.2, 0.3, 0.4])).astype(np.float32)
    q_log = np.log(np.array([0.4, 0.3, 0.2, 0.1])).astype(np.float32)
    t = np.stack([p_log, p_log])
    d = q_log[None, :]
    q = np.array([0.4, 0.3, 0.2, 0.1])
    counts = np.zeros(V)
    rng = np.random.default_rng(0)
    for s in range(6000):
        x = int(rng.choice(V, p=q))
        n, tok = oracle.accept_stochastic(t, d, np.array([x], np.int32), 1.0, 1000 + s, 0)
        counts[tok[0]] += 1
    exp = 6000 * np.array([0.1, 0.2, 0.3, 0.4])
    chi2 = float(((counts - exp) ** 2 / exp).sum())
    assert chi2 < 20.0, (counts, chi2)


def test_rmsnorm(oracle):
    rng = np.random.default_rng(3)
    x = rng.normal(0, 2, (3, 256)).astype(np.float32)
    w = ((rng.normal(1, 0.1, 256).astype(np.float32).view(np.uint32)) >> 16).astype(np.uint16)
    out = bf16_to_f32(oracle.rmsnorm(x, w))
    r = 1 / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6)
    ref = x * r * bf16_to_f32(w)
    assert np.allclose(out, ref, rtol=1e-2)
