"""GPU parity tests: the HIP path (through the C-ABI) against the CPU oracle.

Bars: dequantised weights, router indices (and weights), accepted lengths and
emitted tokens are bit-exact; FFN / MoE outputs within 1e-2 relative L2 of the
fp32 (fp64-accumulated) oracle.
"""
import sys

import numpy as np
import pytest

from tests.helpers import bf16_to_f32, make_q4k_block, rel_l2

pytestmark = pytest.mark.gpu

HD, INTER = 4096, 2048
FFN_TOL = 1e-2


def note(*a):
    print("[gpu-test]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def small_ctx(fa):
    """4 routed + 1 shared experts at the real 4096/2048 shape."""
    note("create small ctx")
    ctx = fa.Context(n_experts=4, top_k=2, max_tokens=64)
    experts = [fa.synth_q4k_expert(11, e) for e in range(5)]
    for e in range(5):
        ctx.upload_expert(0, e, experts[e])
    yield ctx, experts
    ctx.close()


def test_dequant_q4k_bit_exact(fa, oracle, small_ctx):
    ctx, experts = small_ctx
    blocks = experts[0][: 144 * 4096].copy()
    # plant subnormal / zero / negative-zero / max scales
    blocks[0:2] = [0x01, 0x00]
    blocks[144 + 2: 144 + 4] = [0xFF, 0x03]
    blocks[288: 290] = [0x00, 0x80]
    blocks[432: 434] = [0xFF, 0x7B]
    note("dequant q4k", blocks.size // 144, "blocks")
    f, b = ctx.dequant(fa.CODEC_Q4K, blocks)
    ref = oracle.q4k_dequant(blocks)
    assert np.array_equal(f.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(b, fa.f32_to_bf16(ref))


def test_dequant_mxfp4_bit_exact(fa, oracle, small_ctx):
    ctx, _ = small_ctx
    blk = fa.synth_mxfp4_expert(5, 0, 512, 256, 100, 140)[: 17 * 2048].copy()
    blk[0] = 0
    blk[17] = 255
    blk[34] = 1
    note("dequant mxfp4")
    f, b = ctx.dequant(fa.CODEC_MXFP4, blk)
    ref = oracle.mxfp4_dequant(blk)
    assert np.array_equal(f.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(b, fa.f32_to_bf16(ref))


@pytest.mark.parametrize("M", [1, 3, 8, 16, 17, 32, 64])
def test_single_expert_ffn(fa, oracle, small_ctx, M):
    ctx, experts = small_ctx
    h = fa.synth_normal_bf16(100 + M, 1, (M, HD))
    eids = np.zeros((M, 2), np.int32)
    eids[:, 1] = 1
    wts = np.zeros((M, 2), np.float32)
    wts[:, 0] = 1.0
    note("expert_ffn M=%d" % M)
    out = ctx.expert_ffn(0, h, eids, wts)
    ref = oracle.expert_ffn(0, experts[0], h)
    err = rel_l2(bf16_to_f32(out), ref)
    note("rel_l2 =", err)
    assert err < FFN_TOL


def test_shared_expert(fa, oracle, small_ctx):
    ctx, experts = small_ctx
    h = fa.synth_normal_bf16(7, 2, (8, HD))
    note("shared_expert M=8")
    out = ctx.shared_expert(0, h)
    ref = oracle.expert_ffn(0, experts[4], h)
    assert rel_l2(bf16_to_f32(out), ref) < FFN_TOL


def test_weighted_multi_expert(fa, oracle, small_ctx):
    ctx, experts = small_ctx
    M = 5
    h = fa.synth_normal_bf16(9, 3, (M, HD))
    eids = np.array([[0, 1], [1, 2], [3, 0], [2, 2], [1, 3]], np.int32)
    wts = np.array([[0.7, 0.3], [0.5, 0.25], [1.5, -0.5], [0.4, 0.6], [0.9, 0.1]], np.float32)
    note("weighted expert_ffn M=5 with duplicate expert")
    out = ctx.expert_ffn(0, h, eids, wts)
    ys = [oracle.expert_ffn(0, experts[e], h) for e in range(4)]
    ref = np.zeros((M, HD), np.float64)
    for m in range(M):
        for j in range(2):
            ref[m] += wts[m, j] * ys[eids[m, j]][m]
    assert rel_l2(bf16_to_f32(out), ref) < FFN_TOL


def test_single_pair_per_token(fa, oracle, small_ctx):
    """tk = 1 and no shared expert: the down launch writes bf16(w * y) itself
    instead of a separate combine.  Checked against the oracle, and bit for
    bit against the combine path (the same tokens at tk = 2 with a second
    pair of weight 0)."""
    ctx, experts = small_ctx
    M = 6
    h = fa.synth_normal_bf16(9, 4, (M, HD))
    eids = np.array([[0], [1], [2], [3], [1], [0]], np.int32)
    wts = np.array([[0.7], [1.0], [-0.5], [2.0], [0.25], [1.5]], np.float32)
    note("expert_ffn tk=1 M=6 (direct down output)")
    out = ctx.expert_ffn(0, h, eids, wts)
    note("expert_ffn tk=2 M=6 (combine)")
    out2 = ctx.expert_ffn(0, h, np.concatenate([eids, (eids + 1) % 4], 1),
                          np.concatenate([wts, np.zeros_like(wts)], 1))
    assert np.array_equal(out, out2)
    ys = [oracle.expert_ffn(0, experts[e], h) for e in range(4)]
    ref = np.stack([wts[m, 0] * ys[eids[m, 0]][m] for m in range(M)])
    assert rel_l2(bf16_to_f32(out), ref) < FFN_TOL
    with pytest.raises(fa.FstError) as ei:
        ctx.expert_ffn(0, h[:2], np.array([[0], [7]], np.int32), np.ones((2, 1), np.float32))
    assert ei.value.code == fa.FST_EINVAL


def test_invalid_expert_rejected(fa, small_ctx):
    ctx, _ = small_ctx
    h = np.zeros((2, HD), np.uint16)
    with pytest.raises(fa.FstError) as ei:
        ctx.expert_ffn(0, h, np.array([[0, 9], [0, 1]], np.int32), np.ones((2, 2), np.float32))
    assert ei.value.code == fa.FST_EINVAL


def test_token_count_bounds(fa, oracle, small_ctx):
    """M = 0 and M = max_tokens + 1 are argument errors (the reference's
    process_expert_ffn divides by M, src/fst_engine.cpp:4070), and a valid
    call right after them is unaffected."""
    ctx, experts = small_ctx
    for M in (0, 65):
        h = np.zeros((M, HD), np.uint16)
        note("token bound M", M)
        with pytest.raises(fa.FstError) as ei:
            ctx.expert_ffn(0, h, np.zeros((M, 1), np.int32), np.ones((M, 1), np.float32))
        assert ei.value.code == fa.FST_EINVAL
        with pytest.raises(fa.FstError) as ei:
            ctx.shared_expert(0, h)
        assert ei.value.code == fa.FST_EINVAL
    h = fa.synth_normal_bf16(5, 1, (1, HD))
    got = bf16_to_f32(ctx.expert_ffn(0, h, np.array([[2]], np.int32), np.ones((1, 1), np.float32)))
    ref = oracle.expert_ffn(0, experts[2], h)
    assert rel_l2(got, ref) < FFN_TOL


def test_known_answer_ones(fa, oracle):
    """ones@ones: every weight 1.0 (d=1, sc=1, q=1, dmin=0) and h = 1 gives
    g = u = 4096, act = silu(4096)*4096, y = 2048*act for every output."""
    blk = make_q4k_block(0x3C00, 0x0000, [1] * 8, [0] * 8, [1] * 256)
    nblk = 3 * HD * INTER // 256
    expert = np.tile(blk, nblk)
    ctx = fa.Context(n_experts=1, top_k=1, max_tokens=16, has_shared=0)
    try:
        ctx.upload_expert(0, 0, expert)
        h = np.full((2, HD), 0x3F80, np.uint16)
        note("ones@ones")
        out = ctx.expert_ffn(0, h, np.zeros((2, 1), np.int32), np.ones((2, 1), np.float32))
    finally:
        ctx.close()
    act = 4096.0 * 4096.0 / (1.0 + np.exp(-4096.0))
    expect = bf16_to_f32(fa.f32_to_bf16(np.float32(2048.0 * act)))
    assert np.all(bf16_to_f32(out) == expect)


# ------------------------------------------------------------------ router

@pytest.fixture(scope="module")
def router_ctx(fa):
    note("create router ctx")
    ctx = fa.Context(n_experts=256, top_k=6, max_tokens=64, n_layers=4, n_hash_layers=1,
                     vocab_size=1000)
    yield ctx
    ctx.close()


@pytest.mark.parametrize("mode", ["sigmoid", "sqrtsoftplus_bias", "bf16_logits"])
@pytest.mark.parametrize("M", [1, 8, 32, 64])
def test_router_bit_exact(fa, oracle, router_ctx, mode, M):
    ctx = router_ctx
    lid = {"sigmoid": 1, "sqrtsoftplus_bias": 2, "bf16_logits": 3}[mode]
    w = fa.synth_normal_bf16(21, lid, (HD, 256), 0.0, 0.02)
    bias = fa.synth_normal_f32(22, lid, (256,), 0.0, 0.05) if mode == "sqrtsoftplus_bias" else None
    sf = 1 if mode == "sqrtsoftplus_bias" else 0
    rs = 1.5 if mode == "sqrtsoftplus_bias" else 1.0
    rb = 1 if mode == "bf16_logits" else 0
    # the context's scoring mode is global; use per-mode contexts through cfg fields
    c2 = fa.Context(n_experts=256, top_k=6, max_tokens=64, score_func=sf, route_scale=rs,
                    round_logits_bf16=rb)
    try:
        c2.upload_router_bf16(0, w, bias)
        h = fa.synth_normal_bf16(23 + M, lid, (M, HD))
        note("router mode=%s M=%d" % (mode, M))
        e, wt = c2.router(0, h)
    finally:
        c2.close()
    re_, rw, _ = oracle.router(h, w, bias, 6, sf, rs, rb)
    assert np.array_equal(e, re_)
    assert np.array_equal(wt.view(np.uint32), rw.view(np.uint32))


@pytest.mark.parametrize("hd", [512, 1536, 3072, 7168, 8192])
def test_router_hidden_sizes(fa, oracle, hd):
    """Every legal hidden size (a multiple of 512 up to 8192) gets the
    canonical K/64-chunk sum: sizes other than powers of two included."""
    w = fa.synth_normal_bf16(51, hd, (hd, 64), 0.0, 0.02)
    h = fa.synth_normal_bf16(52, hd, (8, hd))
    note("router hidden=%d" % hd)
    with fa.Context(n_experts=64, top_k=4, max_tokens=16, hidden_dim=hd, inter_dim=512) as c:
        c.upload_router_bf16(0, w)
        e, wt = c.router(0, h)
    re_, rw, _ = oracle.router(h, w, None, 4)
    assert np.array_equal(e, re_)
    assert np.array_equal(wt.view(np.uint32), rw.view(np.uint32))


def test_router_ties_and_hash(fa, oracle, router_ctx):
    ctx = router_ctx
    w = fa.synth_normal_bf16(31, 0, (HD, 256), 0.0, 0.02)
    # duplicate columns -> exactly tied logits; lower expert id must win
    for a, b in [(5, 200), (17, 3), (64, 65), (128, 0)]:
        w[:, b] = w[:, a]
    table = (np.arange(1000 * 6, dtype=np.int32).reshape(1000, 6) * 37) % 256
    ctx.upload_router_bf16(0, w)
    ctx.upload_hash_table(0, table)
    h = fa.synth_normal_bf16(32, 0, (16, HD))
    ids = np.arange(16, dtype=np.int32) * 61 % 1000
    note("router hash layer")
    e, wt = ctx.router(0, h, ids)
    re_, rw, _ = oracle.router(h, w, None, 6, 0, 1.0, 0, hash_rows=table[ids])
    assert np.array_equal(e, re_)
    assert np.array_equal(wt.view(np.uint32), rw.view(np.uint32))
    ctx.upload_router_bf16(1, w)
    note("router ties (non-hash layer)")
    e, wt = ctx.router(1, h, ids)
    re_, rw, _ = oracle.router(h, w, None, 6)
    assert np.array_equal(e, re_)
    assert np.array_equal(wt.view(np.uint32), rw.view(np.uint32))


def test_router_tie_heavy(fa, oracle, router_ctx):
    """Groups of 8 exactly tied experts (identical router columns, spread
    over lanes and per-lane slots by a permutation), all 256 tied, and E not
    a multiple of 64: the selection must return the lowest ids of a tied
    group in id order, as the oracle's (score desc, id asc) order does."""
    ctx = router_ctx
    base = fa.synth_normal_bf16(41, 0, (HD, 32), 0.0, 0.02)
    w = np.ascontiguousarray(np.repeat(base, 8, axis=1)[:, np.random.default_rng(5).permutation(256)])
    h = fa.synth_normal_bf16(42, 0, (16, HD))
    note("router tie-heavy")
    ctx.upload_router_bf16(3, w)
    e, wt = ctx.router(3, h)
    re_, rw, _ = oracle.router(h, w, None, 6)
    assert np.array_equal(e, re_)
    assert np.array_equal(wt.view(np.uint32), rw.view(np.uint32))
    wall = np.ascontiguousarray(np.repeat(base[:, :1], 256, axis=1))
    ctx.upload_router_bf16(3, wall)
    e, wt = ctx.router(3, h)
    assert (e == np.arange(6, dtype=np.int32)[None, :]).all()
    re_, rw, _ = oracle.router(h, wall, None, 6)
    assert np.array_equal(e, re_) and np.array_equal(wt.view(np.uint32), rw.view(np.uint32))
    with fa.Context(n_experts=200, top_k=8, max_tokens=16) as c2:
        w2 = fa.synth_normal_bf16(43, 0, (HD, 200), 0.0, 0.02)
        w2[:, 150:200] = w2[:, 0:50]
        c2.upload_router_bf16(0, w2)
        e, wt = c2.router(0, h)
        re_, rw, _ = oracle.router(h, w2, None, 8)
        assert np.array_equal(e, re_) and np.array_equal(wt.view(np.uint32), rw.view(np.uint32))


# ------------------------------------------------------------ MoE layer (C2)

@pytest.mark.parametrize("M", [8, 32])
def test_moe_layer_c2(fa, oracle, c2_layer, M):
    ctx, seed, w = c2_layer
    h = fa.synth_normal_bf16(seed, 2000 + M, (M, HD))
    note("moe_layer M=%d" % M)
    out, e, wt = ctx.moe_layer(0, h)
    re_, rw, _ = oracle.router(h, w, None, 6)
    assert np.array_equal(e, re_)
    assert np.array_equal(wt.view(np.uint32), rw.view(np.uint32))
    experts = {}
    y = np.zeros((M, 6, HD), np.float32)
    for m in range(M):
        for j in range(6):
            ex = int(e[m, j])
            if ex not in experts:
                experts[ex] = oracle.expert_ffn(0, fa.synth_q4k_expert(seed, ex), h)
            y[m, j] = experts[ex][m]
    ys = oracle.expert_ffn(0, fa.synth_q4k_expert(seed, 256), h)
    _, ref = oracle.combine(y, ys, rw)
    err = rel_l2(bf16_to_f32(out), ref)
    note("moe rel_l2 =", err, "distinct experts =", len(experts), ctx.last_active_experts())
    assert ctx.last_active_experts() == len(experts)
    assert err < FFN_TOL


# ---------------------------------------------------------------- acceptance

def planted_logits(fa, seed, n_seq, k, V, n_acc_list):
    t = fa.synth_normal_f32(seed, 0, (n_seq, k + 1, V), 0.0, 2.0)
    draft = np.zeros((n_seq, k), np.int32)
    rng = np.random.default_rng(seed)
    for s in range(n_seq):
        for i in range(k):
            tok = int(rng.integers(V))
            draft[s, i] = tok
            if i < n_acc_list[s]:
                t[s, i, tok] = 50.0
            elif i == n_acc_list[s]:
                t[s, i, tok] = -50.0
    return t, draft


def test_accept_greedy_planted(fa, oracle, small_ctx):
    ctx, _ = small_ctx
    k, V = 7, 129280
    n_acc_list = list(range(8))
    t, draft = planted_logits(fa, 77, 8, k, V, n_acc_list)
    note("accept greedy planted 0..7")
    n_acc, tok = ctx.accept_greedy(t, draft)
    assert list(n_acc) == n_acc_list
    for s in range(8):
        rn, rt = oracle.accept_greedy(t[s], draft[s])
        assert rn == n_acc[s]
        assert np.array_equal(tok[s, : rn + 1], rt)


def test_accept_greedy_nan_ties(fa, oracle, small_ctx):
    ctx, _ = small_ctx
    k, V = 3, 5000
    t = fa.synth_normal_f32(5, 0, (4, k + 1, V), 0.0, 1.0)
    t[0, 0, 0] = np.nan          # NaN at index 0 pins argmax to 0
    t[1, 0, 10] = 9.0
    t[1, 0, 4000] = 9.0          # tie: first index wins
    t[2, 1, :] = -np.inf
    t[3, 0, 17] = np.nan         # NaN elsewhere is skipped
    draft = np.array([[0, 1, 2], [10, 3, 4], [1, 2, 3], [5, 6, 7]], np.int32)
    note("accept greedy nan/ties")
    n_acc, tok = ctx.accept_greedy(t, draft)
    for s in range(4):
        rn, rt = oracle.accept_greedy(t[s], draft[s])
        assert rn == n_acc[s]
        assert np.array_equal(tok[s, : rn + 1], rt)


@pytest.mark.parametrize("temp", [1.0, 0.7])
def test_accept_stochastic_bit_exact(fa, oracle, small_ctx, temp):
    ctx, _ = small_ctx
    k, V, n_seq = 7, 129280, 4
    t = fa.synth_normal_f32(91, 1, (n_seq, k + 1, V), 0.0, 2.0)
    d = fa.synth_normal_f32(91, 2, (n_seq, k, V), 0.0, 2.0)
    # make drafts plausible: draft token = argmax of target half the time
    draft = np.zeros((n_seq, k), np.int32)
    for s in range(n_seq):
        for i in range(k):
            draft[s, i] = int(np.argmax(t[s, i])) if (s + i) % 2 == 0 else int(np.argmax(d[s, i]))
        d[s, :, :] = 0.5 * d[s] + 0.5 * t[s, :k]
    for seed in range(6):
        note("accept stochastic temp=%g seed=%d" % (temp, seed))
        n_acc, tok = ctx.accept_stochastic(t, d, draft, temp, seed, 100)
        for s in range(n_seq):
            rn, rt = oracle.accept_stochastic(t[s], d[s], draft[s], temp, seed, 100 + s)
            assert rn == n_acc[s], (seed, s)
            assert np.array_equal(tok[s, : rn + 1], rt), (seed, s)


def test_accept_stochastic_small_vocab(fa, oracle, small_ctx):
    ctx, _ = small_ctx
    k, V, n_seq = 5, 37, 16
    t = fa.synth_normal_f32(3, 1, (n_seq, k + 1, V), 0.0, 1.5)
    d = fa.synth_normal_f32(3, 2, (n_seq, k, V), 0.0, 1.5)
    draft = (np.arange(n_seq * k, dtype=np.int32).reshape(n_seq, k) * 7) % V
    d[0] = t[0, :k]  # identical distributions: always accept
    note("accept stochastic small vocab")
    n_acc, tok = ctx.accept_stochastic(t, d, draft, 1.0, 42, 0)
    assert n_acc[0] == k
    for s in range(n_seq):
        rn, rt = oracle.accept_stochastic(t[s], d[s], draft[s], 1.0, 42, s)
        assert rn == n_acc[s]
        assert np.array_equal(tok[s, : rn + 1], rt)
