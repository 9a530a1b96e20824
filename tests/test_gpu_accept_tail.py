"""GPU tests of rejection sampling with its last three steps in one launch
(decisions, residual chunk sums and the pick; the last workgroup of a
sequence to arrive picks the token) against the five-launch chain and the
CPU oracle: the accept decisions and the resampled token must be identical,
including rows with NaN and -inf logits, k = 0 and k = 8, and vocabularies up
to the largest the launch takes (V = 262144)."""
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
            d[-1, -1, :] = -np.inf       # a draft row with no finite logit
            d[-1, -1, 7] = 3.0
    return t, np.ascontiguousarray(d), draft


def run_both(fa, ctx, t, d, draft, temp, seed, base):
    ctx.set_fused(True)
    a = ctx.accept_stochastic(t, d, draft, temp, seed, base)
    ctx.set_fused(False)
    try:
        b = ctx.accept_stochastic(t, d, draft, temp, seed, base)
    finally:
        ctx.set_fused(True)
    return a, b


@pytest.mark.parametrize("n_seq,k,V", [(1, 7, 129280), (4, 7, 129280), (2, 3, 1000), (1, 8, 262144),
                                       (3, 1, 4099), (1, 0, 5000), (2, 2, 5), (1, 4, 131072), (1, 4, 131073)])
def test_fused_rejection_sampling_matches_chain_and_oracle(fa, oracle, acc_ctx, n_seq, k, V):
    ctx = acc_ctx
    t, d, draft = case(fa, 500 + V % 97 + k, n_seq, k, V, special=(V > 4000))
    for seed in range(4):
        temp = (1.0, 0.7, 1.3, 0.25)[seed]
        note("fused rejection sampling n_seq=%d k=%d V=%d seed=%d T=%g" % (n_seq, k, V, seed, temp))
        (na, ta), (nb, tb) = run_both(fa, ctx, t, d, draft, temp, seed, 40)
        assert np.array_equal(na, nb), (seed, na, nb)
        for s in range(n_seq):
            assert np.array_equal(ta[s, : na[s] + 1], tb[s, : nb[s] + 1]), (seed, s)
        if V <= 5000 or seed == 0:
            for s in range(n_seq):
                rn, rt = oracle.accept_stochastic(t[s], d[s], draft[s], temp, seed, 40 + s)
                assert rn == na[s], (seed, s)
                assert np.array_equal(ta[s, : rn + 1], rt), (seed, s)


def test_fused_rejection_sampling_repeated_calls(fa, acc_ctx):
    """Back-to-back calls with changing shapes: the per-sequence arrival
    counters end every call at zero."""
    ctx = acc_ctx
    shapes = [(1, 7, 129280), (2, 2, 3000), (1, 7, 129280), (4, 5, 60000), (1, 1, 70)]
    for i, (n_seq, k, V) in enumerate(shapes):
        t, d, draft = case(fa, 800 + i, n_seq, k, V)
        note("repeated fused call %d: n_seq=%d k=%d V=%d" % (i, n_seq, k, V))
        (na, ta), (nb, tb) = run_both(fa, ctx, t, d, draft, 1.0, 11 + i, 0)
        assert np.array_equal(na, nb)
        for s in range(n_seq):
            assert np.array_equal(ta[s, : na[s] + 1], tb[s, : nb[s] + 1])


@pytest.mark.parametrize("V", [129280, 777])
def test_fused_rejection_sampling_zero_residual(fa, oracle, acc_ctx, V):
    """Draft rows equal to the target rows and a draft token of zero mass: the
    first position is rejected and the residual is identically zero, so the
    token is drawn from the target row instead (both paths and the oracle)."""
    ctx = acc_ctx
    k = 3
    t, _, _ = case(fa, 900 + V % 13, 1, k, V)
    t[0, 0, 11] = -np.inf
    d = np.ascontiguousarray(t[:, :k].copy())
    draft = np.array([[11, 2, 3]], np.int32)
    for seed in range(3):
        note("zero residual V=%d seed=%d" % (V, seed))
        (na, ta), (nb, tb) = run_both(fa, ctx, t, d, draft, 1.0, seed, 7)
        rn, rt = oracle.accept_stochastic(t[0], d[0], draft[0], 1.0, seed, 7)
        assert rn == 0 and na[0] == 0 and nb[0] == 0
        assert np.array_equal(ta[0, :1], rt) and np.array_equal(tb[0, :1], rt)
