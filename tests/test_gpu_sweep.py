"""GPU sweep of the router-driven fused MoE launch against the launch chain
over layer shapes the other tests do not cover: 8, 64, 200 and 256 experts,
top-k 1 to 8, with and without the shared expert, 1 to 32 tokens, Q4_K and
MXFP4.  Routing (ids and weights) must agree bit for bit.  MXFP4 outputs must
agree bit for bit; Q4_K outputs bit for bit except where the chain splits the
gate||up sums over K (calls with few slot x tile items), there within 2e-3
relative L2 and finite."""
import numpy as np
import pytest

from tests.helpers import bf16_to_f32, rel_l2

pytestmark = pytest.mark.gpu

HD, SEED = 4096, 99
SHAPES = [(8, 1), (8, 2), (64, 4), (64, 8), (200, 6), (256, 6)]


@pytest.mark.parametrize("codec", [0, 1])
@pytest.mark.parametrize("E,tk", SHAPES)
@pytest.mark.parametrize("shared", [1, 0])
def test_fused_matches_chain_sweep(fa, codec, E, tk, shared):
    print("[gpu-test] sweep codec=%d E=%d tk=%d shared=%d" % (codec, E, tk, shared), flush=True)
    with fa.Context(n_experts=E, top_k=tk, max_tokens=64, codec=codec, has_shared=shared) as ctx:
        ctx.synth_experts(SEED, 0, 0, E + shared, 0)
        ctx.upload_router_bf16(0, fa.synth_normal_bf16(SEED, 11 + E + tk, (HD, E), 0.0, 0.02))
        try:
            for M in (1, 2, 3, 5, 7, 8, 12, 16, 24, 32):
                if M * tk > 256:
                    continue
                h = fa.synth_normal_bf16(SEED, 1000 + M + 10 * E + tk, (M, HD))
                ctx.set_fused(True)
                of, ef, wf = ctx.moe_layer(0, h)
                ctx.set_fused(False)
                oc, ec, wc = ctx.moe_layer(0, h)
                assert np.array_equal(ef, ec) and np.array_equal(wf.view(np.uint32), wc.view(np.uint32)), M
                if codec == 1 or np.array_equal(of, oc):
                    assert np.array_equal(of, oc), M
                else:
                    a, b = bf16_to_f32(of), bf16_to_f32(oc)
                    assert np.isfinite(a).all() and rel_l2(a, b) < 2e-3, M
        finally:
            ctx.set_fused(True)


@pytest.mark.parametrize("codec", [0, 1])
@pytest.mark.parametrize("M", [17, 32])
def test_fused_split_slots_match_chain(fa, codec, M):
    """Hash routing that sends every token to the same two experts: slots of
    more than 16 tokens run as several 16-token slots of the fused launch (the
    expert streamed once per group).  Same bits as the launch chain (Q4_K:
    within 2e-3 where the chain splits K), and the routing is the table's."""
    E, tk, V = 8, 2, 512
    print("[gpu-test] split slots codec=%d M=%d" % (codec, M), flush=True)
    with fa.Context(n_experts=E, top_k=tk, max_tokens=64, codec=codec, n_hash_layers=1, vocab_size=V) as ctx:
        ctx.synth_experts(SEED, 0, 0, E + 1, 0)
        ctx.upload_router_bf16(0, fa.synth_normal_bf16(SEED, 77, (HD, E), 0.0, 0.02))
        table = np.tile(np.array([[3, 5]], np.int32), (V, 1))
        table[7] = [5, 1]
        ctx.upload_hash_table(0, table)
        ids = (np.arange(M, dtype=np.int32) * 13) % V
        ids[1] = 7
        h = fa.synth_normal_bf16(SEED, 4000 + M, (M, HD))
        try:
            ctx.set_fused(True)
            of, ef, wf = ctx.moe_layer(0, h, ids)
            ctx.set_fused(False)
            oc, ec, wc = ctx.moe_layer(0, h, ids)
        finally:
            ctx.set_fused(True)
        assert np.array_equal(ef, table[ids]) and np.array_equal(ef, ec)
        assert np.array_equal(wf.view(np.uint32), wc.view(np.uint32))
        if codec == 1 or np.array_equal(of, oc):
            assert np.array_equal(of, oc)
        else:
            a, b = bf16_to_f32(of), bf16_to_f32(oc)
            assert np.isfinite(a).all() and rel_l2(a, b) < 2e-3
