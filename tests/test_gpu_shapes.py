"""MoE layer (router -> routed + shared experts -> combine) at shapes the
C2-based tests do not reach, against the oracle:

- 300 experts: more than the gate||up launch routes in-launch, so the top-k
  runs as its own launch; at hidden 1024 an M = 1 call splits K (few slots);
- hidden 1536 / inter 1024: super-block counts that are not powers of two
  (router chunks of 24 elements, 6 and 4 super-blocks per row);
- M from 1 to 32: every token capacity of the linear kernel."""
import sys

import numpy as np
import pytest

from tests.helpers import bf16_to_f32, rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-2
TK = 4
SEED = 61


def note(*a):
    print("[gpu-test]", *a, flush=True)
    sys.stdout.flush()


def reference(fa, oracle, h, eids, wts, E, hd, inter):
    M = h.shape[0]
    y = np.zeros((M, TK, hd), np.float32)
    for ex in sorted(set(int(x) for x in eids.ravel())):
        rows = [m for m in range(M) if ex in eids[m]]
        ye = oracle.expert_ffn(0, fa.synth_q4k_expert(SEED, ex, hd, inter), h[rows], hd, inter)
        for r, m in enumerate(rows):
            for j in range(TK):
                if eids[m, j] == ex:
                    y[m, j] = ye[r]
    ys = oracle.expert_ffn(0, fa.synth_q4k_expert(SEED, E, hd, inter), h, hd, inter)
    _, ref = oracle.combine(y, ys, wts)
    return ref


@pytest.mark.parametrize("E,hd,inter,Ms", [(300, 1024, 512, (1, 8, 20)), (64, 1536, 1024, (1, 5, 32))])
def test_moe_layer_shapes(fa, oracle, E, hd, inter, Ms):
    note("create ctx E=%d hd=%d inter=%d" % (E, hd, inter))
    with fa.Context(n_experts=E, top_k=TK, max_tokens=64, hidden_dim=hd, inter_dim=inter) as ctx:
        for ex in range(E + 1):
            ctx.upload_expert(0, ex, fa.synth_q4k_expert(SEED, ex, hd, inter))
        w = fa.synth_normal_bf16(SEED, 1000, (hd, E), 0.0, 0.02)
        ctx.upload_router_bf16(0, w)
        for M in Ms:
            h = fa.synth_normal_bf16(SEED, 2000 + M, (M, hd))
            note("moe_layer E=%d hd=%d M=%d" % (E, hd, M))
            out, e, wt = ctx.moe_layer(0, h)
            re_, rw, _ = oracle.router(h, w, None, TK)
            assert np.array_equal(e, re_)
            assert np.array_equal(wt.view(np.uint32), rw.view(np.uint32))
            ref = reference(fa, oracle, h, e, wt, E, hd, inter)
            assert rel_l2(bf16_to_f32(out), ref) < TOL
