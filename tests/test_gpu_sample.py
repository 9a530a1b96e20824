"""sample_token on the GPU (fst_sample_token[_dev], src/fst_engine.cpp:4491-4528)
against the oracle, bit-exact on the token for identical logits and seed, at
the full vocabulary and on edge cases: argmax path with NaNs, ties, top_p at
0 and 1, duplicated maxima, rows of one value."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

V = 129280


@pytest.fixture(scope="module")
def sctx(fa):
    print("[gpu-test] sample_token context", flush=True)
    ctx = fa.Context(n_experts=8, top_k=1, max_tokens=16)
    yield ctx
    ctx.close()


@pytest.mark.parametrize("T,top_p", [(1.0, 0.9), (0.7, 0.5), (1.0, 1.0), (1.5, 0.99), (0.3, 0.0), (0.0, 0.9),
                                     (-1.0, 0.5), (1.0, 1e-7)])
def test_sample_token_bit_exact_full_vocab(fa, oracle, sctx, T, top_p):
    print("[gpu-test] sample T=%g top_p=%g" % (T, top_p), flush=True)
    rng = np.random.default_rng(int(T * 100) + int(top_p * 1000))
    for s in range(4):
        x = rng.normal(0, 2, V).astype(np.float32)
        got = sctx.sample_token(x, T, top_p, 1234, s)
        ref, _ = oracle.sample_token(x, T, top_p, 1234, s)
        assert got == ref, (s, got, ref)


def test_sample_token_edge_rows(fa, oracle, sctx):
    print("[gpu-test] sample edge rows", flush=True)
    rng = np.random.default_rng(5)
    rows = []
    x = rng.normal(0, 2, V).astype(np.float32)
    x[[10, 99999]] = 30.0                       # two maxima
    rows.append(x)
    y = np.full(V, 0.5, np.float32)             # one value everywhere: ties only
    rows.append(y)
    z = rng.normal(0, 1, V).astype(np.float32)
    z[rng.integers(0, V, 500)] = np.nan         # NaNs get no mass
    rows.append(z)
    w = rng.normal(0, 1, V).astype(np.float32)
    w[0] = np.nan                               # argmax path: NaN at 0 pins 0
    rows.append(w)
    q = np.round(rng.normal(0, 2, V)).astype(np.float32)  # many equal values
    rows.append(q)
    for i, r in enumerate(rows):
        for T, tp in ((1.0, 0.9), (0.0, 0.9), (2.0, 0.3), (1.0, 1.0)):
            for s in range(3):
                got = sctx.sample_token(r, T, tp, 77, 10 * i + s)
                ref, _ = oracle.sample_token(r, T, tp, 77, 10 * i + s)
                assert got == ref, (i, T, tp, s, got, ref)


def test_sample_token_dev_rows_use_seq_base(fa, oracle, sctx):
    print("[gpu-test] sample dev rows", flush=True)
    L = fa.lib()
    rng = np.random.default_rng(9)
    n = 6
    x = rng.normal(0, 2, (n, V)).astype(np.float32)
    dx = sctx.to_device(x)
    dt = sctx.dev_alloc(4 * n)
    fa._check(L.fst_sample_token_dev(sctx.h, dx, n, V, 0.9, 0.95, 31, 500, dt))
    sctx.sync()
    got = sctx.to_host(dt, (n,), np.int32)
    for r in range(n):
        assert got[r] == oracle.sample_token(x[r], 0.9, 0.95, 31, 500 + r)[0]
    sctx.dev_free(dx)
    sctx.dev_free(dt)
