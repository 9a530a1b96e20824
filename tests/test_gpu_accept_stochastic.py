"""GPU tests of rejection sampling (two launches: every row's chunk softmax
partials, then the decisions, the exponential race and the token, the last
workgroup of a sequence to arrive picking it) against the CPU oracle: the
accepted lengths and the emitted tokens must be identical, including rows
with NaN and -inf logits, a draft row without a finite logit, k = 0 up to the
largest k (63), vocabularies that leave chunks empty or end mid-vector, and
the largest vocabulary the launches take."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def note(*a):
    print("[gpu-test]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def acc_ctx(fa):
    """A context for acceptance calls only (no experts needed)."""
    note("create acceptance ctx")
    ctx = fa.Context(n_experts=4, top_k=2, max_tokens=64)
    yield ctx
    ctx.close()


def case(fa, seed, n_seq, k, V, special=False):
    t = fa.synth_normal_f32(seed, 1, (n_seq, k + 1, V), 0.0, 2.0)
    d = fa.synth_normal_f32(seed, 2, (n_seq, max(k, 1), V), 0.0, 2.0)[:, :k]
    d = np.ascontiguousarray(0.6 * d + 0.4 * t[:, :k]).astype(np.float32)
    rng = np.random.default_rng(seed)
    draft = np.zeros((n_seq, k), np.int32)
    for s in range(n_seq):
        for i in range(k):
            draft[s, i] = int(np.argmax(t[s, i])) if rng.random() < 0.6 else int(rng.integers(V))
    if special:
        t[0, 0, ::97] = np.nan          # NaNs are no tokens
        t[0, -1, 5:50] = -np.inf         # zero mass
        if k:
            d[0, 0, 1::13] = np.nan
            d[-1, -1, :] = -np.inf       # a draft row with no finite logit but one
            d[-1, -1, 7] = 3.0
    return t, np.ascontiguousarray(d), draft


def check(oracle, t, d, draft, temp, seed, base, na, ta):
    for s in range(t.shape[0]):
        rn, rt = oracle.accept_stochastic(t[s], d[s], draft[s], temp, seed, base + s)
        assert rn == na[s], (seed, s, rn, na[s])
        assert np.array_equal(ta[s, : rn + 1], rt), (seed, s, ta[s, : rn + 1], rt)
        assert np.all(ta[s, rn + 1:] == -1)


@pytest.mark.parametrize("n_seq,k,V", [(1, 7, 129280), (4, 7, 129280), (2, 3, 1000), (1, 8, 262144),
                                       (3, 1, 4099), (1, 0, 5000), (2, 2, 5), (1, 4, 131072), (1, 4, 131073),
                                       (2, 15, 3000), (1, 63, 301), (1, 2, (1 << 20) - 2), (64, 7, 5000),
                                       (16, 31, 777)])
def test_rejection_sampling_matches_oracle(fa, oracle, acc_ctx, n_seq, k, V):
    ctx = acc_ctx
    t, d, draft = case(fa, 500 + V % 97 + k, n_seq, k, V, special=(V > 4000))
    for seed in range(4 if V <= 262144 else 1):
        temp = (1.0, 0.7, 1.3, 0.25)[seed]
        note("rejection sampling n_seq=%d k=%d V=%d seed=%d T=%g" % (n_seq, k, V, seed, temp))
        na, ta = ctx.accept_stochastic(t, d, draft, temp, seed, 40)
        check(oracle, t, d, draft, temp, seed, 40, na, ta)


def test_rejection_sampling_planted_lengths(fa, oracle, acc_ctx):
    """Draft rows equal to the target rows accept every draft (p = q), and a
    draft token of zero target mass is rejected: planting one at position j
    gives n_acc = j exactly, with the rejected token redrawn."""
    ctx = acc_ctx
    k, V = 7, 129280
    t, _, draft = case(fa, 1234, 1, k, V)
    for j in range(k + 1):
        d = np.ascontiguousarray(t[:, :k].copy())
        tj = t.copy()
        if j < k:
            tj[0, j, draft[0, j]] = -np.inf
        note("planted n_acc=%d" % j)
        na, ta = ctx.accept_stochastic(tj, d, draft, 1.0, 3, 9)
        assert na[0] == j
        check(oracle, tj, d, draft, 1.0, 3, 9, na, ta)


def test_rejection_sampling_repeated_calls(fa, oracle, acc_ctx):
    """Back-to-back calls with changing shapes: the per-sequence arrival
    counters end every call at zero, and each call equals the oracle."""
    ctx = acc_ctx
    shapes = [(1, 7, 129280), (2, 2, 3000), (1, 7, 129280), (4, 5, 60000), (1, 1, 70)]
    for i, (n_seq, k, V) in enumerate(shapes):
        t, d, draft = case(fa, 800 + i, n_seq, k, V)
        note("repeated call %d: n_seq=%d k=%d V=%d" % (i, n_seq, k, V))
        na, ta = ctx.accept_stochastic(t, d, draft, 1.0, 11 + i, 0)
        check(oracle, t, d, draft, 1.0, 11 + i, 0, na, ta)


@pytest.mark.parametrize("V", [129280, 777])
def test_rejection_sampling_zero_residual(fa, oracle, acc_ctx, V):
    """Draft rows equal to the target rows and a draft token of zero mass: the
    first position is rejected and the residual is identically zero, so the
    token is drawn from the target row instead."""
    ctx = acc_ctx
    k = 3
    t, _, _ = case(fa, 900 + V % 13, 1, k, V)
    t[0, 0, 11] = -np.inf
    d = np.ascontiguousarray(t[:, :k].copy())
    draft = np.array([[11, 2, 3]], np.int32)
    for seed in range(3):
        note("zero residual V=%d seed=%d" % (V, seed))
        na, ta = ctx.accept_stochastic(t, d, draft, 1.0, seed, 7)
        rn, rt = oracle.accept_stochastic(t[0], d[0], draft[0], 1.0, seed, 7)
        assert rn == 0 and na[0] == 0
        assert np.array_equal(ta[0, :1], rt)
        assert ta[0, 0] == oracle.rs_race(t[0, 0], None, 1.0, seed, 7, 0)
