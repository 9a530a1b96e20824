"""CPU tests pinning the oracle (oracle/fst_oracle.c) against golden fixtures,
closed forms, independent implementations and brute force.  No GPU needed."""
import json
import math
import os

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


def test_exp_nonpos_equals_expf_bit_for_bit(oracle):
    """fst_exp_nonpos (the softmax weights of rejection sampling) is fst_expf
    without its overflow path: identical bits for every x <= 0, checked on
    every float in [-2^-20, 0], around the flush boundary -87.3365 and the
    2^-126 results, on 4M random values in [-100, 0], and on -0, -inf, NaN."""
    import ctypes as C
    rng = np.random.default_rng(11)
    lo = np.float32(-87.33654022216797)
    parts = [
        -rng.random(4_000_000, dtype=np.float32) * np.float32(100.0),
        np.arange(0x80000000, 0x80000000 + (1 << 20) + 1, dtype=np.uint64).astype(np.uint32).view(np.float32)[:-1],
        (lo.view(np.uint32) + np.arange(-50000, 50000).astype(np.int64)).astype(np.uint32).view(np.float32),
        np.linspace(-88.0, -86.5, 200_000, dtype=np.float32),
        np.array([0.0, -0.0, -np.inf, np.nan, -1e-45, -1e-30, -103.0], np.float32),
    ]
    x = np.ascontiguousarray(np.concatenate(parts).astype(np.float32))
    x = x[(x <= 0) | np.isnan(x)]
    a = np.empty_like(x)
    b = np.empty_like(x)
    P = C.c_void_p
    oracle.lib().fo_exp_nonpos_n(x.ctypes.data_as(P), x.size, a.ctypes.data_as(P))
    oracle.lib().fo_expf_n(x.ctypes.data_as(P), x.size, b.ctypes.data_as(P))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


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


def _softmax64(row, inv_t=1.0):
    x = (np.asarray(row, np.float32) * np.float32(inv_t)).astype(np.float64)
    x = np.where(np.isnan(x), -np.inf, x)
    e = np.exp(x - x.max())
    return e / e.sum()


@pytest.mark.parametrize("V", [1, 5, 1000, 129280, 262147])
def test_rs_row_stats_vs_float64(oracle, V):
    """(M, S): M is the row's exact maximum, S = sum exp(x - M) within fp32
    summation error of the float64 sum, at vocabularies that leave chunks
    empty (V < 256), partial (V % 4 != 0) and several float4s long."""
    rng = np.random.default_rng(V)
    row = rng.normal(0, 2, V).astype(np.float32)
    for inv_t in (1.0, 0.5):
        M, S = oracle.rs_row_stats(row, inv_t)
        x = (row * np.float32(inv_t)).astype(np.float32)
        assert M == float(x.max())
        ref = np.exp(x.astype(np.float64) - float(x.max())).sum()
        assert abs(S - ref) <= 2e-6 * ref, (S, ref)


def test_rs_row_stats_special_values(oracle):
    row = np.array([1.0, np.nan, -np.inf, 2.0, np.nan], np.float32)
    M, S = oracle.rs_row_stats(row)
    assert M == 2.0 and abs(S - (1.0 + math.exp(-1.0))) < 1e-6
    M, S = oracle.rs_row_stats(np.full(7, np.nan, np.float32))
    assert M == -math.inf and S == 0.0
    M, S = oracle.rs_row_stats(np.array([0.0, np.inf, 3.0, np.inf], np.float32))
    assert M == math.inf and S == 2.0                  # each +inf weighs 1, the rest 0
    M, S = oracle.rs_row_stats(np.zeros(1000, np.float32))
    assert M == 0.0 and S == 1000.0                    # exact: 1000 ones in any order


def test_race_uniform_range_and_mean(oracle):
    u = np.array([oracle.lib().fo_race_uniform(9, 3, 2, v) for v in range(20000)])
    assert u.min() > 0.0 and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 0.01
    # a different position or sequence gives other uniforms
    assert oracle.lib().fo_race_uniform(9, 3, 2, 5) != oracle.lib().fo_race_uniform(9, 3, 3, 5)
    assert oracle.lib().fo_race_uniform(9, 3, 2, 5) != oracle.lib().fo_race_uniform(9, 4, 2, 5)


@pytest.mark.parametrize("seed", range(20))
def test_stochastic_closed_forms(oracle, seed):
    rng = np.random.default_rng(seed)
    k, V = 5, 300
    t = rng.normal(0, 2, (k + 1, V)).astype(np.float32)
    draft = rng.integers(0, V, k).astype(np.int32)
    # p == q: u < 1 = p/q accepts every draft; the bonus is the race over p_k
    n, tok = oracle.accept_stochastic(t, t[:k], draft, 1.0, seed, 3)
    assert n == k and list(tok[:k]) == list(draft)
    assert tok[k] == oracle.rs_race(t[k], None, 1.0, seed, 3, k)
    # q(x) = 0 (draft logit -inf at x): accepted whenever p(x) > 0
    d = t[:k].copy()
    d[np.arange(k), draft] = -np.inf
    n, tok = oracle.accept_stochastic(t, d, draft, 1.0, seed, 4)
    assert n == k
    # p(x) = 0 at position 2 (target logit -inf): rejected there, and the
    # resampled token has p > q
    d = rng.normal(0, 2, (k, V)).astype(np.float32)
    t2 = t.copy()
    t2[:2] = d[:2]                                    # positions 0, 1: p == q, accepted
    t2[2, draft[2]] = -np.inf
    n, tok = oracle.accept_stochastic(t2, d, draft, 1.0, seed, 5)
    assert n == 2 and tok[2] != draft[2]
    p, q = _softmax64(t2[2]), _softmax64(d[2])
    assert p[tok[2]] > q[tok[2]]


@pytest.mark.parametrize("seed", range(10))
def test_race_single_positive_residual(oracle, seed):
    """Only v* has p > q (the target raises one logit of the draft row), so
    norm(max(0, p - q)) is the point mass at v*, whatever the uniforms."""
    rng = np.random.default_rng(100 + seed)
    V = 1000
    d = rng.normal(0, 2, V).astype(np.float32)
    vs = int(rng.integers(0, V))
    t = d.copy()
    t[vs] += 3.0
    for pos in range(4):
        assert oracle.rs_race(t, d, 1.0, seed, 7, pos) == vs
    # an identically zero residual falls back to the race over p
    assert oracle.rs_race(d, d, 1.0, seed, 7, 1) == oracle.rs_race(d, None, 1.0, seed, 7, 1)


def test_stochastic_decision_vs_float64(oracle):
    """The accept decision u*q(x) < p(x) agrees with float64 u < p/q wherever
    the two sides are not within float rounding of each other."""
    rng = np.random.default_rng(5)
    V, checked = 2000, 0
    for s in range(300):
        t = rng.normal(0, 1, (2, V)).astype(np.float32)
        d = rng.normal(0, 1, (1, V)).astype(np.float32)
        x = int(rng.integers(0, V))
        n, tok = oracle.accept_stochastic(t, d, np.array([x], np.int32), 1.0, s, 0)
        p, q = _softmax64(t[0])[x], _softmax64(d[0])[x]
        u = oracle.uniform24(s, 0, 0, 0) / 2 ** 24
        if abs(u * q - p) <= 1e-5 * p:
            continue
        checked += 1
        assert (n == 1) == (u * q < p)
    assert checked > 250


def test_race_draws_the_normalized_residual(oracle):
    """Chi-square of 6000 races (different sequence numbers) against
    norm(max(0, p - q)) on V = 6."""
    p = np.array([0.30, 0.05, 0.25, 0.10, 0.20, 0.10])
    q = np.array([0.10, 0.20, 0.10, 0.30, 0.05, 0.25])
    t, d = np.log(p).astype(np.float32), np.log(q).astype(np.float32)
    r = np.maximum(p - q, 0)
    r /= r.sum()
    counts = np.zeros(6)
    for s in range(6000):
        counts[oracle.rs_race(t, d, 1.0, 11, s, 0)] += 1
    assert counts[r == 0].sum() == 0
    exp = 6000 * r[r > 0]
    chi2 = float(((counts[r > 0] - exp) ** 2 / exp).sum())
    assert chi2 < 16.0, (counts, chi2)        # 2 degrees of freedom


def test_accept_rate_is_sum_of_min(oracle):
    """With x ~ q the first draft is accepted with probability sum_x min(p, q)."""
    V = 5
    p = np.array([0.35, 0.05, 0.2, 0.3, 0.1])
    q = np.array([0.1, 0.3, 0.2, 0.15, 0.25])
    t = np.log(np.stack([p, p])).astype(np.float32)
    d = np.log(q)[None, :].astype(np.float32)
    rng = np.random.default_rng(1)
    n_acc = 0
    N = 6000
    for s in range(N):
        x = int(rng.choice(V, p=q))
        n, _ = oracle.accept_stochastic(t, d, np.array([x], np.int32), 1.0, 500 + s, 0)
        n_acc += n
    a = float(np.minimum(p, q).sum())
    assert abs(n_acc / N - a) < 4 * math.sqrt(a * (1 - a) / N), (n_acc / N, a)


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
