"""CPU tests pinning the Hyper-Connection (HC) pieces of the oracle
(src/fst_engine.cpp:2286-2459, :694-742): Sinkhorn split, the control matvec,
hc_pre / hc_post / output_hc_head, against float64 restatements, closed forms
and invariants."""
import numpy as np

from tests.helpers import bf16_to_f32, f32_to_bf16, rel_l2


def _bf16(rng, shape, mean=0.0, std=1.0):
    return f32_to_bf16(rng.normal(mean, std, shape).astype(np.float32)).reshape(shape)


def _split64(mix, scale, base, n=4, iters=20, eps=1e-6):
    """float64 restatement of hc_split_sinkhorn."""
    mix = np.asarray(mix, np.float64)
    out = np.zeros(2 * n + n * n)
    sig = lambda z: 1.0 / (1.0 + np.exp(-z))
    out[:n] = sig(mix[:n] * scale[0] + base[:n]) + eps
    out[n:2 * n] = 2.0 * sig(mix[n:2 * n] * scale[1] + base[n:2 * n])
    c = (mix[2 * n:] * scale[2] + base[2 * n:]).reshape(n, n)  # [dst][src]
    c = np.exp(c - c.max(1, keepdims=True))
    c = c / c.sum(1, keepdims=True) + eps
    c = c / (c.sum(0, keepdims=True) + eps)
    for _ in range(1, iters):
        c = c / (c.sum(1, keepdims=True) + eps)
        c = c / (c.sum(0, keepdims=True) + eps)
    out[2 * n:] = c.ravel()
    return out


def test_hc_split_closed_form_at_zero(oracle):
    s = oracle.hc_split(np.zeros(24), [1.0, 1.0, 1.0], np.zeros(24))
    assert np.allclose(s[:4], 0.5 + 1e-6, atol=1e-7)
    assert np.allclose(s[4:8], 1.0, atol=1e-7)
    assert np.allclose(s[8:], 0.25, atol=1e-5)


def test_hc_split_vs_float64_and_doubly_stochastic(oracle):
    rng = np.random.default_rng(21)
    for _ in range(20):
        mix = rng.normal(0, 2, 24).astype(np.float32)
        scale = rng.uniform(0.2, 2.0, 3).astype(np.float32)
        base = rng.normal(0, 1, 24).astype(np.float32)
        got = oracle.hc_split(mix, scale, base)
        ref = _split64(mix, scale, base)
        assert np.allclose(got, ref, rtol=2e-5, atol=2e-6)
        c = got[8:].reshape(4, 4)
        assert np.allclose(c.sum(0), 1.0, atol=1e-5)   # last step normalises columns (over dst)
        assert np.allclose(c.sum(1), 1.0, atol=0.1)   # rows: 20 iterations need not have converged


def test_hc_mix_vs_float64(oracle):
    rng = np.random.default_rng(22)
    K = 4 * 4096
    flat = _bf16(rng, (K,))
    fnT = _bf16(rng, (24, K), 0.0, 0.05)
    got = oracle.hc_mix(flat, fnT)
    ref = bf16_to_f32(fnT).astype(np.float64) @ bf16_to_f32(flat).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 2 ** -7 * np.abs(ref) + 0.05)
    # the result is bf16-representable
    assert np.array_equal(f32_to_bf16(got), f32_to_bf16(got.astype(np.float32)))
    assert np.array_equal(bf16_to_f32(f32_to_bf16(got)), got)


def test_hc_pre_equal_streams_and_vs_float64(oracle):
    rng = np.random.default_rng(23)
    d, M = 4096, 3
    h = _bf16(rng, (M, 4, d))
    fnT = _bf16(rng, (24, 4 * d), 0.0, 0.02)
    scale = np.array([1.0, 0.5, 2.0], np.float32)
    base = rng.normal(0, 0.5, 24).astype(np.float32)
    cur, post, comb = oracle.hc_pre(h, fnT, scale, base)
    for m in range(M):
        r = bf16_to_f32(h[m]).astype(np.float64)
        flat = r.ravel() / np.sqrt((r.ravel() ** 2).mean() + 1e-6)
        mix = bf16_to_f32(fnT).astype(np.float64) @ flat
        s = _split64(mix, scale, base)
        assert np.allclose(post[m], s[4:8], rtol=2e-2, atol=1e-3)
        ref_cur = (s[:4, None] * r).sum(0)
        assert rel_l2(bf16_to_f32(cur[m]), ref_cur) < 2e-2
    # four equal streams: cur = bf16((sum of pre) * r0) exactly as the sequential float sum
    h2 = np.repeat(h[:, :1], 4, axis=1)
    cur2, _, _ = oracle.hc_pre(h2, fnT, scale, base)
    assert cur2.shape == (M, d) and np.isfinite(bf16_to_f32(cur2)).all()


def test_hc_post_identity_comb(oracle):
    """post = 1 and comb = identity give out[dst] = bf16(bo + r[dst])."""
    rng = np.random.default_rng(24)
    d, M = 512, 2
    h = _bf16(rng, (M, 4, d))
    bo = _bf16(rng, (M, d))
    post = np.ones((M, 4), np.float32)
    comb = np.tile(np.eye(4, dtype=np.float32).ravel(), (M, 1))
    out = oracle.hc_post(bo, h, post, comb)
    ref = f32_to_bf16(bf16_to_f32(bo)[:, None, :] + bf16_to_f32(h)).reshape(h.shape)
    assert np.array_equal(out, ref)


def test_hc_head_uniform_weights(oracle):
    """A zero control matrix and zero base: w = sigmoid(0) + eps for every
    stream, out = bf16(sum_h w r_h)."""
    rng = np.random.default_rng(25)
    d, M = 4096, 2
    h = _bf16(rng, (M, 4, d))
    fnT = np.zeros((4, 4 * d), np.uint16)
    out = oracle.hc_head(h, fnT, 1.0, np.zeros(4, np.float32))
    w = np.float32(0.5) + np.float32(1e-6)
    acc = np.zeros((M, d), np.float32)
    for k in range(4):
        acc = acc + w * bf16_to_f32(h[:, k])
    assert np.array_equal(out, f32_to_bf16(acc).reshape(M, d))


def test_hc_post_vs_float64_detects_transposed_comb(oracle):
    """out[dst] = bo post[dst] + sum_src comb[dst + 4 src] r[src]
    (src/fst_engine.cpp:2394-2414); using comb transposed must not match."""
    rng = np.random.default_rng(26)
    d, M = 1024, 3
    h = _bf16(rng, (M, 4, d))
    bo = _bf16(rng, (M, d))
    post = rng.uniform(0, 2, (M, 4)).astype(np.float32)
    comb = rng.uniform(0, 1, (M, 16)).astype(np.float32)
    out = bf16_to_f32(oracle.hc_post(bo, h, post, comb)).reshape(M, 4, d).astype(np.float64)
    r = bf16_to_f32(h).reshape(M, 4, d).astype(np.float64)
    b = bf16_to_f32(bo).reshape(M, d).astype(np.float64)
    c = comb.reshape(M, 4, 4).astype(np.float64)  # [m][src][dst]
    ref = b[:, None, :] * post[:, :, None] + np.einsum("msd,msj->mdj", c, r)
    assert rel_l2(out, ref) < 5e-3
    bad = b[:, None, :] * post[:, :, None] + np.einsum("mds,msj->mdj", c, r)
    assert rel_l2(out, bad) > 0.1


def test_hc_head_vs_float64(oracle):
    rng = np.random.default_rng(27)
    d, M = 4096, 2
    h = _bf16(rng, (M, 4, d))
    fnT = _bf16(rng, (4, 4 * d), 0.0, 0.02)
    base = rng.normal(0, 1, 4).astype(np.float32)
    out = bf16_to_f32(oracle.hc_head(h, fnT, 0.7, base)).reshape(M, d)
    for m in range(M):
        r = bf16_to_f32(h[m]).astype(np.float64)
        flat = r.ravel() / np.sqrt((r.ravel() ** 2).mean() + 1e-6)
        z = bf16_to_f32(fnT).astype(np.float64) @ flat * 0.7 + base
        w = 1.0 / (1.0 + np.exp(-z)) + 1e-6
        assert rel_l2(out[m], (w[:, None] * r).sum(0)) < 2e-2
