"""GPU tests of the bf16-weight linear kernels (fst_dense.hip): the shared
expert kept in bf16 as the reference keeps it (process_shared_expert,
src/fst_engine.cpp:4373-4489) inside the MoE chain, and the bf16 LM head
(apply_final_norm_and_lm_head, :2115-2160), against the CPU oracle."""
import numpy as np
import pytest

from tests.helpers import bf16_to_f32, rel_l2

pytestmark = pytest.mark.gpu

SEED = 909
TOL = 1e-2


def _log(*a):
    print("[gpu-test]", *a, flush=True)


def _shared16(fa, seed, hd, inter, lid=0):
    g = fa.synth_normal_bf16(seed, 8000 + 3 * lid, (inter, hd), 0.0, 0.02)
    u = fa.synth_normal_bf16(seed, 8001 + 3 * lid, (inter, hd), 0.0, 0.02)
    d = fa.synth_normal_bf16(seed, 8002 + 3 * lid, (hd, inter), 0.0, 0.02)
    return g, u, d


def _shared_ref(oracle, sh, h):
    g, u, d = (bf16_to_f32(t).reshape(t.shape) for t in sh)
    return oracle.expert_ffn_f32(g, u, d, h)


@pytest.mark.parametrize("hd,inter", [(4096, 2048), (1024, 512), (2048, 1536)])
@pytest.mark.parametrize("M", [1, 8, 17, 64])
def test_shared_bf16_alone(fa, oracle, hd, inter, M):
    """fst_shared_expert runs only the bf16 kernels; covers every K split
    (K/256 divisible by 8, by 4, and only by 2) and all token-group counts."""
    _log("shared bf16 alone hd=%d inter=%d M=%d" % (hd, inter, M))
    with fa.Context(n_experts=4, top_k=1, max_tokens=64, hidden_dim=hd, inter_dim=inter) as ctx:
        sh = _shared16(fa, SEED, hd, inter)
        ctx.upload_shared_bf16(0, *sh)
        h = fa.synth_normal_bf16(SEED, 100 + M, (M, hd))
        out = ctx.shared_expert(0, h)
        assert rel_l2(bf16_to_f32(out), _shared_ref(oracle, sh, h)) < TOL


@pytest.mark.parametrize("codec", ["mxfp4", "q4k"])
@pytest.mark.parametrize("M", [1, 8, 32])
def test_moe_layer_with_bf16_shared(fa, oracle, codec, M):
    """Routed experts in the codec bank plus the bf16 shared expert, combined
    in the routed down projection's epilogue: out = bf16(sum_j w_j y_j + y_sh)."""
    E, TK, HD = 8, 2, 4096
    _log("moe_layer %s + bf16 shared M=%d" % (codec, M))
    mx = codec == "mxfp4"
    ctx = fa.Context(n_experts=E, top_k=TK, max_tokens=64, codec=fa.CODEC_MXFP4 if mx else fa.CODEC_Q4K)
    with ctx:
        experts = [(fa.synth_mxfp4_expert if mx else fa.synth_q4k_expert)(SEED, e) for e in range(E)]
        for e in range(E):
            ctx.upload_expert(0, e, experts[e])
        sh = _shared16(fa, SEED, HD, 2048)
        ctx.upload_shared_bf16(0, *sh)
        w = fa.synth_normal_bf16(SEED, 11, (HD, E), 0.0, 0.02)
        ctx.upload_router_bf16(0, w)
        h = fa.synth_normal_bf16(SEED, 200 + M, (M, HD))
        out, eids, wts = ctx.moe_layer(0, h)
        e_ref, w_ref, _ = oracle.router(h, w, None, TK)
        assert np.array_equal(eids, e_ref) and np.array_equal(wts, w_ref)
        y = np.zeros((M, TK, HD), np.float32)
        for ex in sorted(set(int(v) for v in e_ref.ravel())):
            rows = [m for m in range(M) if ex in e_ref[m]]
            ye = oracle.expert_ffn(1 if mx else 0, experts[ex], h[rows])
            for r, m in enumerate(rows):
                y[m, list(e_ref[m]).index(ex)] = ye[r]
        _, ref = oracle.combine(y, _shared_ref(oracle, sh, h), w_ref)
        err = rel_l2(bf16_to_f32(out), ref)
        _log("rel_l2", err)
        assert err < TOL


@pytest.mark.parametrize("M", [1, 8, 32, 64])
def test_lm_head_bf16(fa, oracle, M):
    """Final RMSNorm (bit-exact path) then logits = W x over the bf16 head,
    vs float64 on the same normed bf16 rows."""
    HD, V = 4096, 2560
    _log("lm_head bf16 M=%d" % M)
    with fa.Context(n_experts=4, top_k=1, max_tokens=64, n_layers=1, vocab_size=V) as ctx:
        norm = fa.synth_normal_bf16(SEED, 12, (HD,), 1.0, 0.1)
        ctx.upload_norm(1, norm)
        W = fa.synth_normal_bf16(SEED, 13, (V, HD), 0.0, 0.02)
        ctx.upload_lm_head_bf16(W)
        h = fa.synth_normal_bf16(SEED, 300 + M, (M, HD))
        dh = ctx.to_device(h)
        dl = ctx.dev_alloc(M * V * 4)
        fa._check(fa.lib().fst_lm_head_dev(ctx.h, dh, M, dl))
        ctx.sync()
        got = ctx.to_host(dl, (M, V), np.float32)
        ctx.dev_free(dh)
        ctx.dev_free(dl)
    xn = bf16_to_f32(oracle.rmsnorm(bf16_to_f32(h).reshape(M, HD), norm)).reshape(M, HD).astype(np.float64)
    ref = xn @ bf16_to_f32(W).reshape(V, HD).astype(np.float64).T
    for m in range(M):
        assert rel_l2(got[m], ref[m]) < 1e-5
