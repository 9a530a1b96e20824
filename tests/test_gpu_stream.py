"""GPU tests of the one-launch paths run back to back on the stream, as a
serving loop (and bench.py) runs them: many calls with no host
synchronisation in between, each checked afterwards against the launch chain
on the same input.  The fused MoE launch and the small-M launch hand results
between workgroups through epoch-tagged words; here each call's words follow
the previous call's on the device with no gap, so a word of one call taken
for the next one's, or a late store, would show as a mismatch."""
import numpy as np
import pytest

from tests.test_gpu_moe import HD, TK, E
from tests.test_gpu_small_m import CHAIN_TOL
from tests.helpers import bf16_to_f32, rel_l2

pytestmark = pytest.mark.gpu

NB = 16      # distinct inputs
CALLS = 192  # back-to-back calls


def note(*a):
    print("[gpu-test]", *a, flush=True)


def test_fused_moe_back_to_back_matches_chain(fa, c2_layer):
    """192 router-driven MoE calls of 1-8 tokens back to back through the
    fused launch, bit-identical to the launch chain on every call (M >= 2;
    at M = 1 the chain splits K, so within tolerance)."""
    ctx, seed, _ = c2_layer
    L = fa.lib()
    Ms = [8, 3, 8, 5, 8, 2, 7, 8, 4, 8, 6, 1, 8, 8, 2, 8]
    hs = [fa.synth_normal_bf16(seed, 7300 + b, (Ms[b], HD)) for b in range(NB)]
    dh = [ctx.to_device(h) for h in hs]
    ref = []
    ctx.set_fused(False)
    try:
        for b in range(NB):
            out, _, _ = ctx.moe_layer(0, hs[b])
            ref.append(out)
    finally:
        ctx.set_fused(True)
    douts = [ctx.dev_alloc(8 * HD * 2) for _ in range(CALLS)]
    de, dw = ctx.dev_alloc(8 * TK * 4), ctx.dev_alloc(8 * TK * 4)
    note("fused back to back: %d calls" % CALLS)
    try:
        for i in range(CALLS):
            b = i % NB
            fa._check(L.fst_moe_layer_dev(ctx.h, 0, dh[b], Ms[b], None, douts[i], de, dw))
        ctx.sync()
        bad = []
        for i in range(CALLS):
            b = i % NB
            got = ctx.to_host(douts[i], (Ms[b], HD), np.uint16)
            if Ms[b] == 1:
                ok = rel_l2(bf16_to_f32(got), bf16_to_f32(ref[b])) < 2e-3
            else:
                ok = np.array_equal(got, ref[b])
            if not ok:
                bad.append(i)
        assert not bad, "calls differing from the chain: %s" % bad[:10]
    finally:
        for p in douts + dh + [de, dw]:
            ctx.dev_free(p)


def test_small_m_back_to_back_matches_chain(fa, c2_layer):
    """192 caller-routed one- and two-token calls back to back through the
    small-M launch (different experts, with and without the shared expert),
    each within the chain tolerance of the launch chain and bit-identical to
    the same call made alone."""
    ctx, seed, _ = c2_layer
    L = fa.lib()
    rng = np.random.default_rng(41)
    cases = []
    for b in range(NB):
        M = 1 + (b % 2)
        eids = np.stack([rng.choice(E, TK, replace=False) for _ in range(M)]).astype(np.int32)
        w = (rng.random((M, TK)) + 0.05).astype(np.float32)
        w /= w.sum(1, keepdims=True)
        cases.append((fa.synth_normal_bf16(seed, 7400 + b, (M, HD)), eids, w.astype(np.float32), b % 3 != 0))
    dev = [(ctx.to_device(h), ctx.to_device(e), ctx.to_device(w)) for h, e, w, _ in cases]
    alone, chain = [], []
    for small_m, store in ((True, alone), (False, chain)):
        ctx.set_small_m(small_m)
        try:
            for (h, e, w, sh), (dh, de, dw) in zip(cases, dev):
                do = ctx.dev_alloc(2 * HD * 2)
                fa._check(L.fst_moe_ffn_dev(ctx.h, 0, dh, h.shape[0], de, dw, int(sh), do, None, None))
                ctx.sync()
                store.append(ctx.to_host(do, h.shape, np.uint16))
                ctx.dev_free(do)
        finally:
            ctx.set_small_m(True)
    for b in range(NB):
        assert rel_l2(bf16_to_f32(alone[b]), bf16_to_f32(chain[b])) < CHAIN_TOL
    douts = [ctx.dev_alloc(2 * HD * 2) for _ in range(CALLS)]
    note("small-M back to back: %d calls" % CALLS)
    try:
        for i in range(CALLS):
            b = i % NB
            h, _, _, sh = cases[b]
            dh, de, dw = dev[b]
            fa._check(L.fst_moe_ffn_dev(ctx.h, 0, dh, h.shape[0], de, dw, int(sh), douts[i], None, None))
        ctx.sync()
        bad = [i for i in range(CALLS)
               if not np.array_equal(ctx.to_host(douts[i], cases[i % NB][0].shape, np.uint16), alone[i % NB])]
        assert not bad, "calls differing from the same call made alone: %s" % bad[:10]
    finally:
        for p in douts:
            ctx.dev_free(p)
        for t in dev:
            for p in t:
                ctx.dev_free(p)


@pytest.mark.parametrize("mode", ["greedy", "stochastic"])
def test_acceptance_back_to_back_matches_single_calls(fa, mode):
    """192 acceptance calls back to back at k = 7, V = 129,280 (greedy:
    chunk words handed to the owner workgroup; stochastic: the tail launch's
    arrival counters, left at zero by each call), on 16 different inputs of
    one or two sequences, each identical to the same call made alone."""
    from tests.test_gpu_parity import planted_logits
    with fa.Context(n_experts=4, top_k=1, max_tokens=64) as ctx:
        _acceptance_back_to_back(fa, ctx, mode)


def _acceptance_back_to_back(fa, ctx, mode):
    from tests.test_gpu_parity import planted_logits
    L = fa.lib()
    k, V = 7, 129280
    ins = []
    for b in range(NB):
        n_seq = 1 + (b % 2)
        t, d = planted_logits(fa, 500 + b, n_seq, k, V, [(b + s) % (k + 1) for s in range(n_seq)])
        q = fa.synth_normal_f32(600 + b, 0, (n_seq, k, V), 0.0, 2.0)
        ins.append((n_seq, ctx.to_device(t), ctx.to_device(q), ctx.to_device(d)))
    outs = [(ctx.dev_alloc(8), ctx.dev_alloc(2 * (k + 1) * 4)) for _ in range(CALLS)]

    def call(i, dn, dk):
        n_seq, dt, dq, dd = ins[i % NB]
        if mode == "greedy":
            fa._check(L.fst_accept_greedy_dev(ctx.h, dt, n_seq, k, V, dd, dn, dk))
        else:
            fa._check(L.fst_accept_stochastic_dev(ctx.h, dt, dq, n_seq, k, V, dd, 1.0, 99, 1000 * (i % NB), dn, dk))

    def read(i, dn, dk):
        n_seq = ins[i % NB][0]
        return ctx.to_host(dn, (n_seq,), np.int32), ctx.to_host(dk, (n_seq, k + 1), np.int32)

    try:
        alone = []
        for b in range(NB):
            call(b, *outs[b])
            ctx.sync()
            alone.append(read(b, *outs[b]))
        note("%s acceptance back to back: %d calls" % (mode, CALLS))
        for i in range(CALLS):
            call(i, *outs[i])
        ctx.sync()
        bad = []
        for i in range(CALLS):
            n, t = read(i, *outs[i])
            a_n, a_t = alone[i % NB]
            if not (np.array_equal(n, a_n) and np.array_equal(t, a_t)):
                bad.append(i)
        assert not bad, "calls differing from the same call made alone: %s" % bad[:10]
        assert all((a[0] >= 0).all() for a in alone)
    finally:
        for p in outs:
            ctx.dev_free(p[0])
            ctx.dev_free(p[1])
        for _, dt, dq, dd in ins:
            ctx.dev_free(dt)
            ctx.dev_free(dq)
            ctx.dev_free(dd)
