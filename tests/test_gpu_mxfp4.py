"""GPU tests of the MXFP4 expert path (the format the reference engine runs its experts in):
fused FP4 decode with the block scale (hardware E2M1 -> bf16 conversion) +
bf16 MFMA, through the same MoE chain and C-ABI, against the CPU oracle
(dequantise per kernels/fst_dequant_v4_vectorized_kernel.cc:19-37,60-80, fp64
accumulation)."""
import numpy as np
import pytest

from tests.helpers import bf16_to_f32, rel_l2

pytestmark = pytest.mark.gpu

HD, INTER, E, TK = 4096, 2048, 8, 2
SEED = 707
TOL = 1e-2


def _log(*a):
    print("[gpu-test]", *a, flush=True)


@pytest.fixture(scope="module")
def mx_layer(fa):
    _log("MXFP4 layer: %d routed + 1 shared experts" % E)
    ctx = fa.Context(n_experts=E, top_k=TK, max_tokens=64, codec=fa.CODEC_MXFP4)
    experts = [fa.synth_mxfp4_expert(SEED, e) for e in range(E + 1)]
    # special scales in expert 3: e = 0 and e = 255 decode to 0 (reference kernel)
    x = experts[3].reshape(-1, 17).copy()
    x[0::97, 0] = 0
    x[5::89, 0] = 255
    experts[3] = x.ravel()
    for e in range(E + 1):
        ctx.upload_expert(0, e, experts[e])
    w = fa.synth_normal_bf16(SEED, 11, (HD, E), 0.0, 0.02)
    ctx.upload_router_bf16(0, w)
    yield ctx, experts, w
    ctx.close()


def _routed_ref(oracle, experts, h, eids, wts, shared):
    M = h.shape[0]
    y = np.zeros((M, TK, HD), np.float32)
    for ex in sorted(set(int(v) for v in eids.ravel())):
        rows = [m for m in range(M) if ex in eids[m]]
        ye = oracle.expert_ffn(1, experts[ex], h[rows])
        for r, m in enumerate(rows):
            for j in range(TK):
                if eids[m, j] == ex:
                    y[m, j] = ye[r]
    ys = oracle.expert_ffn(1, experts[E], h) if shared else None
    _, ref = oracle.combine(y, ys, wts)
    return ref


@pytest.mark.parametrize("M", [1, 8, 32])
def test_mxfp4_moe_layer_vs_oracle(fa, oracle, mx_layer, M):
    ctx, experts, w = mx_layer
    _log("mxfp4 moe_layer M=%d" % M)
    h = fa.synth_normal_bf16(SEED, 100 + M, (M, HD))
    out, eids, wts = ctx.moe_layer(0, h)
    e_ref, w_ref, _ = oracle.router(h, w, None, TK)
    assert np.array_equal(eids, e_ref) and np.array_equal(wts, w_ref)
    err = rel_l2(bf16_to_f32(out), _routed_ref(oracle, experts, h, e_ref, w_ref, True))
    _log("rel_l2", err)
    assert err < TOL


def test_mxfp4_special_scales_and_single_expert(fa, oracle, mx_layer):
    """Every token routed to expert 3 (blocks with e = 0 and e = 255) and the
    shared expert alone, each against the oracle."""
    ctx, experts, _ = mx_layer
    M = 16
    h = fa.synth_normal_bf16(SEED, 300, (M, HD))
    eids = np.stack([np.array([3, 5], np.int32)] * M)
    wts = np.full((M, TK), 0.5, np.float32)
    out = ctx.expert_ffn(0, h, eids, wts)
    assert rel_l2(bf16_to_f32(out), _routed_ref(oracle, experts, h, eids, wts, False)) < TOL
    sh = ctx.shared_expert(0, h)
    ref = oracle.expert_ffn(1, experts[E], h)
    assert rel_l2(bf16_to_f32(sh), ref) < TOL


def test_mxfp4_device_synth_matches_host(fa):
    """fst_synth_experts_dev on an MXFP4 context writes the bytes of
    fst_synth_mxfp4_expert: the uploaded expert and its device-generated twin
    give bit-identical outputs."""
    with fa.Context(n_experts=4, top_k=1, max_tokens=16, codec=fa.CODEC_MXFP4) as ctx:
        ctx.upload_expert(0, 0, fa.synth_mxfp4_expert(SEED, 50))
        ctx.synth_experts(SEED, 0, 1, 1, 49)  # expert 1 <- generator id 50
        ctx.synth_experts(SEED, 0, 2, 3, 0)
        h = fa.synth_normal_bf16(SEED, 400, (8, HD))
        w = np.ones((8, 1), np.float32)
        a = ctx.expert_ffn(0, h, np.zeros((8, 1), np.int32), w)
        b = ctx.expert_ffn(0, h, np.ones((8, 1), np.int32), w)
        assert np.array_equal(a, b)


@pytest.mark.parametrize("M", [1, 2, 5, 8])
def test_mxfp4_fused_launch_matches_chain(fa, mx_layer, M):
    """Router-driven MXFP4 calls of at most 8 tokens run gate||up and down in
    the fused launch (bf16 operands, h rounded to bf16 as the chain's
    gate||up epilogue does): the same bits as the launch chain, on several
    batches in a row (the epoch tags of one call must not leak into the
    next), with the e = 0 / e = 255 blocks of expert 3 in play."""
    ctx, experts, _ = mx_layer
    try:
        for b in range(3):
            _log("mxfp4 fused vs chain M=%d batch %d" % (M, b))
            h = fa.synth_normal_bf16(SEED, 500 + 10 * M + b, (M, HD))
            ctx.set_fused(True)
            out_f, e_f, w_f = ctx.moe_layer(0, h)
            ctx.set_fused(False)
            out_c, e_c, w_c = ctx.moe_layer(0, h)
            assert np.array_equal(e_f, e_c) and np.array_equal(w_f.view(np.uint32), w_c.view(np.uint32))
            assert np.array_equal(out_f, out_c)
    finally:
        ctx.set_fused(True)


def test_mxfp4_c2_layer_fused_vs_chain_and_oracle(fa, oracle):
    """The C2 shape with MXFP4 experts (256 routed + 1 shared, top-6, 8
    tokens): the fused launch equals the chain bit for bit over 8 batches in a
    row, and the first batch matches the oracle."""
    E2, TK2, M = 256, 6, 8
    with fa.Context(n_experts=E2, top_k=TK2, max_tokens=64, codec=fa.CODEC_MXFP4) as ctx:
        ctx.synth_experts(SEED, 0, 0, E2 + 1, 0)
        w = fa.synth_normal_bf16(SEED, 12, (HD, E2), 0.0, 0.02)
        ctx.upload_router_bf16(0, w)
        for b in range(8):
            _log("mxfp4 C2 fused vs chain batch %d" % b)
            h = fa.synth_normal_bf16(SEED, 600 + b, (M, HD))
            ctx.set_fused(True)
            out_f, e_f, w_f = ctx.moe_layer(0, h)
            ctx.set_fused(False)
            out_c, _, _ = ctx.moe_layer(0, h)
            ctx.set_fused(True)
            assert np.array_equal(out_f, out_c)
            if b == 0:
                e_ref, w_ref, _ = oracle.router(h, w, None, TK2)
                assert np.array_equal(e_f, e_ref)
                y = np.zeros((M, TK2, HD), np.float32)
                for ex in sorted(set(int(v) for v in e_ref.ravel())):
                    ye = oracle.expert_ffn(1, fa.synth_mxfp4_expert(SEED, ex), h)
                    for m in range(M):
                        for j in range(TK2):
                            if e_ref[m, j] == ex:
                                y[m, j] = ye[m]
                ys = oracle.expert_ffn(1, fa.synth_mxfp4_expert(SEED, E2), h)
                _, ref = oracle.combine(y, ys, w_ref)
                err = rel_l2(bf16_to_f32(out_f), ref)
                _log("rel_l2", err)
                assert err < TOL
