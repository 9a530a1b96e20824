"""GPU tests of the Hyper-Connection kernels (hc_pre / hc_post /
output_hc_head, src/fst_engine.cpp:2350-2459 with the control matvec of
:694-742) through the C-ABI, bit-exact against the CPU oracle, and of the HC
mode of the verify forward against the composition of its public pieces."""
import numpy as np
import pytest

from tests.helpers import bf16_to_f32, rel_l2

pytestmark = pytest.mark.gpu

HD = 4096
SEED = 808


def _log(*a):
    print("[gpu-test]", *a, flush=True)


def _hc_tensors(fa, seed, lid):
    fn = fa.synth_normal_bf16(seed, 5000 + lid, (24, 4 * HD), 0.0, 0.02)
    rng = np.random.default_rng(seed + lid)
    scale = rng.uniform(0.2, 1.5, 3).astype(np.float32)
    base = rng.normal(0.0, 1.0, 24).astype(np.float32)
    return fn, scale, base


def _head_tensors(fa, seed):
    fn = fa.synth_normal_bf16(seed, 6000, (4, 4 * HD), 0.0, 0.02)
    base = np.random.default_rng(seed).normal(0.0, 1.0, 4).astype(np.float32)
    return fn, np.float32(0.7), base


@pytest.mark.parametrize("M", [1, 8, 32])
def test_hc_kernels_bit_exact(fa, oracle, M):
    _log("hc_pre/post/head M=%d" % M)
    fn, scale, base = _hc_tensors(fa, SEED, 0)
    hfn, hscale, hbase = _head_tensors(fa, SEED)
    with fa.Context(n_experts=4, top_k=1, max_tokens=64, n_layers=1) as ctx:
        ctx.upload_hc(0, fn, scale, base)
        ctx.upload_hc_head(hfn, hscale, hbase)
        h = fa.synth_normal_bf16(SEED, 7000 + M, (M, 4, HD), 0.0, 1.5)
        cur, post, comb = ctx.hc_pre(0, h)
        c_ref, p_ref, m_ref = oracle.hc_pre(h, fn, scale, base)
        assert np.array_equal(post, p_ref)
        assert np.array_equal(comb, m_ref)
        assert np.array_equal(cur, c_ref)
        bo = fa.synth_normal_bf16(SEED, 7100 + M, (M, HD), 0.0, 0.5)
        out = ctx.hc_post(bo, h, post, comb)
        assert np.array_equal(out, oracle.hc_post(bo, h, p_ref, m_ref))
        plain = ctx.hc_head(h)
        assert np.array_equal(plain, oracle.hc_head(h, hfn, hscale, hbase))
        ctx.upload_hc_head(hfn, hscale, None)
        plain0 = ctx.hc_head(h)
        assert np.array_equal(plain0, oracle.hc_head(h, hfn, hscale, None))


def test_hc_pre_not_ready(fa):
    with fa.Context(n_experts=4, top_k=1, max_tokens=8, n_layers=2) as ctx:
        with pytest.raises(fa.FstError):
            ctx.hc_pre(1, np.zeros((1, 4, HD), np.uint16))


def test_verify_forward_hc_mode_matches_composition(fa, oracle):
    """With HC uploaded for every layer and the head, fst_verify_forward runs
    h = hc_post(MoE(RMSNorm(hc_pre(h))), h) per layer and
    lm_head(output_hc_head(h)); it equals the composition of the public
    entry points bit for bit, and the HC steps of that composition equal the
    oracle bit for bit."""
    L, E, tk, V, M, seed = 2, 8, 2, 1280, 16, 91
    _log("verify_forward HC mode L=%d M=%d" % (L, M))
    ctx = fa.Context(n_experts=E, top_k=tk, max_tokens=64, n_layers=L, vocab_size=V)
    with ctx:
        hcs = []
        for l in range(L):
            ctx.synth_experts(seed, l, 0, E + 1, l * 1000)
            ctx.upload_router_bf16(l, fa.synth_normal_bf16(seed, 1000 + l, (HD, E), 0.0, 0.02))
            ctx.upload_norm(l, fa.synth_normal_bf16(seed, 2000 + l, (HD,), 1.0, 0.1))
            hcs.append(_hc_tensors(fa, seed, l))
            ctx.upload_hc(l, *hcs[l])
        fnorm = fa.synth_normal_bf16(seed, 2000 + L, (HD,), 1.0, 0.1)
        ctx.upload_norm(L, fnorm)
        ctx.synth_lm_head(seed, 999999)
        hfn, hscale, hbase = _head_tensors(fa, seed)
        ctx.upload_hc_head(hfn, hscale, hbase)

        h0 = fa.synth_normal_bf16(seed, 3000, (M, 4, HD))
        logits, h_fin = ctx.verify_forward(h0)
        assert h_fin.shape == (M, 4, HD)

        h = h0
        for l in range(L):
            cur, post, comb = ctx.hc_pre(l, h)
            c_ref, p_ref, m_ref = oracle.hc_pre(h, *hcs[l])
            assert np.array_equal(cur, c_ref) and np.array_equal(post, p_ref) and np.array_equal(comb, m_ref)
            dc = ctx.to_device(cur)
            dn = ctx.dev_alloc(cur.nbytes)
            fa._check(fa.lib().fst_rmsnorm_dev(ctx.h, l, dc, None, M, None, dn))
            ctx.sync()
            mn = ctx.to_host(dn, cur.shape, np.uint16)
            ctx.dev_free(dc)
            ctx.dev_free(dn)
            out, _, _ = ctx.moe_layer(l, mn)
            h_new = ctx.hc_post(out, h, post, comb)
            assert np.array_equal(h_new, oracle.hc_post(out, h, p_ref, m_ref))
            h = h_new
        assert np.array_equal(h, h_fin)
        plain = ctx.hc_head(h)
        assert np.array_equal(plain, oracle.hc_head(h, hfn, hscale, hbase))
        dp = ctx.to_device(plain)
        dl = ctx.dev_alloc(M * V * 4)
        fa._check(fa.lib().fst_lm_head_dev(ctx.h, dp, M, dl))
        ctx.sync()
        manual = ctx.to_host(dl, (M, V), np.float32)
        ctx.dev_free(dp)
        ctx.dev_free(dl)
        assert np.array_equal(manual, logits)
        blocks = fa.synth_q4k_blocks(seed, 999999, V * HD // 256)
        ref = oracle.q4k_linear(blocks, oracle.rmsnorm(bf16_to_f32(plain).reshape(M, HD), fnorm), V, HD)
        assert rel_l2(logits, ref) < 1e-2


@pytest.mark.parametrize("M", [1, 8])
def test_final_head_collapses_hc_residual(fa, oracle, M):
    # apply_final_norm_and_lm_head (src/fst_engine.cpp:2115-2160): with the HC
    # head uploaded the input is the 4-stream residual, collapsed by
    # output_hc_head before the final norm and the LM head (:2120-2128)
    _log("final_head HC M=%d" % M)
    V = 4096
    hfn, hscale, hbase = _head_tensors(fa, SEED)
    with fa.Context(n_experts=4, top_k=1, max_tokens=16, n_layers=1, vocab_size=V) as ctx:
        nw = fa.synth_normal_bf16(SEED, 7300, (HD,), 1.0, 0.1)
        ctx.upload_norm(1, nw)
        head = fa.synth_q4k_blocks(SEED, 7301, V * HD // 256)
        ctx.upload_lm_head(head)
        h_hc = fa.synth_normal_bf16(SEED, 7200 + M, (M, 4, HD), 0.0, 1.5)
        # plain mode first: only stream 0's shape [M][HD] is read
        plain_in = np.ascontiguousarray(h_hc[:, 0, :])
        lg_plain = ctx.final_head(plain_in)
        ref_plain = oracle.q4k_linear(head, oracle.rmsnorm(bf16_to_f32(plain_in), nw), V, HD)
        assert rel_l2(lg_plain, ref_plain) < 1e-2
        ctx.upload_hc_head(hfn, hscale, hbase)
        lg = ctx.final_head(h_hc)
        # the composition of the public device pieces, bit for bit
        L = fa.lib()
        d_hs = ctx.to_device(h_hc)
        d_pl = ctx.dev_alloc(M * HD * 2)
        d_lg = ctx.dev_alloc(M * V * 4)
        fa._check(L.fst_hc_head_dev(ctx.h, d_hs, M, d_pl))
        fa._check(L.fst_lm_head_dev(ctx.h, d_pl, M, d_lg))
        ctx.sync()
        comp = ctx.to_host(d_lg, (M, V), np.float32)
        assert np.array_equal(lg.view(np.uint32), comp.view(np.uint32))
        # and the oracle: hc_head (bit-exact pieces) -> RMSNorm -> Q4_K head
        plain = oracle.hc_head(h_hc, hfn, hscale, hbase)
        ref = oracle.q4k_linear(head, oracle.rmsnorm(bf16_to_f32(plain), nw), V, HD)
        assert rel_l2(lg, ref) < 1e-2
        # reading the residual as plain rows instead gives different logits
        assert rel_l2(lg, lg_plain) > 0.1
        for p in (d_hs, d_pl, d_lg):
            ctx.dev_free(p)
