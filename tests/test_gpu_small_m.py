"""GPU tests of the small-M launch (caller-given routing, one or two tokens,
Q4_K): one launch from the eids to the combined rows, fp32 VALU dot products.
Checked against the fp64 oracle (process_expert_ffn / process_shared_expert and
the combine, src/fst_engine.cpp:4068-4489, :4196-4201) and against the MFMA
launch chain on the same inputs, including duplicate experts, invalid ids,
shared-only calls and repeated calls whose slot counts change (the per-tile
arrival counters must re-arm)."""
import sys

import numpy as np
import pytest

from tests.helpers import bf16_to_f32, rel_l2
from tests.test_gpu_moe import E, HD, TK, TOL

pytestmark = pytest.mark.gpu

CHAIN_TOL = 4e-3   # both paths are within 1e-2 of the oracle; to each other closer


def note(*a):
    print("[gpu-test]", *a, flush=True)
    sys.stdout.flush()


def run_dev(fa, ctx, h, eids, wts, use_shared, small_m=True):
    """fst_moe_ffn_dev (routing width = the context's top_k) with the
    combined, routed-only and shared-only outputs."""
    L = fa.lib()
    M = h.shape[0]
    dh, de, dw = ctx.to_device(h), ctx.to_device(eids), ctx.to_device(wts)
    do, dr, ds = ctx.dev_alloc(M * HD * 2), ctx.dev_alloc(M * HD * 2), ctx.dev_alloc(M * HD * 2)
    ctx.set_small_m(small_m)
    try:
        fa._check(L.fst_moe_ffn_dev(ctx.h, 0, dh, M, de, dw, use_shared, do, dr, ds))
        ctx.sync()
        outs = [ctx.to_host(p, (M, HD), np.uint16) for p in (do, dr, ds)]
    finally:
        ctx.set_small_m(True)
        for p in (dh, de, dw, do, dr, ds):
            ctx.dev_free(p)
    return outs


def run(fa, ctx, h, eids, wts, use_shared, small_m=True):
    """Full-width routing through the device entry, narrower routing (tk <
    top_k, no shared expert) through fst_expert_ffn."""
    if eids.shape[1] == TK:
        return run_dev(fa, ctx, h, eids, wts, use_shared, small_m)
    assert not use_shared
    ctx.set_small_m(small_m)
    try:
        return [ctx.expert_ffn(0, h, eids, wts), None, None]
    finally:
        ctx.set_small_m(True)


def reference_any_tk(fa, oracle, seed, h, eids, wts, shared):
    """The oracle's expert FFNs and combine for any routing width."""
    M, tk = eids.shape
    y = np.zeros((M, tk, HD), np.float32)
    for ex in sorted(set(int(x) for x in eids.ravel())):
        rows = [m for m in range(M) if ex in eids[m]]
        ye = oracle.expert_ffn(0, fa.synth_q4k_expert(seed, ex), h[rows])
        for r, m in enumerate(rows):
            for j in range(tk):
                if eids[m, j] == ex:
                    y[m, j] = ye[r]
    ys = oracle.expert_ffn(0, fa.synth_q4k_expert(seed, E), h) if shared else None
    _, ref = oracle.combine(y, ys, wts)
    return ref, y, ys


def routing(seed, M, tk):
    rng = np.random.default_rng(seed)
    eids = np.stack([rng.choice(E, tk, replace=False) for _ in range(M)]).astype(np.int32)
    w = rng.random((M, tk)).astype(np.float32) + 0.05
    return eids, (w / w.sum(1, keepdims=True)).astype(np.float32)


@pytest.mark.parametrize("M,tk,shared", [(1, 1, 0), (1, 6, 1), (2, 1, 0), (2, 6, 1), (2, 3, 0), (1, 6, 0)])
def test_small_m_matches_oracle_and_chain(fa, oracle, c2_layer, M, tk, shared):
    ctx, seed, _ = c2_layer
    eids, wts = routing(900 + 10 * M + tk, M, tk)
    h = fa.synth_normal_bf16(seed, 9000 + M * 10 + tk, (M, HD))
    note("small-M M=%d tk=%d shared=%d" % (M, tk, shared))
    out, outr, outs = run(fa, ctx, h, eids, wts, shared)
    ref, y, ys = reference_any_tk(fa, oracle, seed, h, eids, wts, bool(shared))
    e_out = rel_l2(bf16_to_f32(out), ref)
    note("rel_l2 out %.2e" % e_out)
    assert e_out < TOL
    if outr is not None:
        routed = np.einsum("mj,mjd->md", wts.astype(np.float64), y.astype(np.float64))
        assert rel_l2(bf16_to_f32(outr), routed) < TOL
    if shared:
        assert rel_l2(bf16_to_f32(outs), ys) < TOL
    note("chain")
    c_out, c_outr, c_outs = run(fa, ctx, h, eids, wts, shared, small_m=False)
    assert rel_l2(bf16_to_f32(out), bf16_to_f32(c_out)) < CHAIN_TOL
    if outr is not None:
        assert rel_l2(bf16_to_f32(outr), bf16_to_f32(c_outr)) < CHAIN_TOL
    if shared:
        assert rel_l2(bf16_to_f32(outs), bf16_to_f32(c_outs)) < CHAIN_TOL


def test_small_m_duplicates_and_shared_slots(fa, oracle, c2_layer):
    """Both tokens on the same experts, and one expert twice within a token:
    each distinct expert is read once, every (token, j) pair is summed."""
    ctx, seed, _ = c2_layer
    eids = np.array([[5, 9, 5, 17, 2, 3], [9, 5, 40, 41, 42, 5]], np.int32)
    wts = np.array([[0.3, 0.2, 0.1, 0.2, 0.1, 0.1], [0.25, 0.25, 0.2, 0.1, 0.1, 0.1]], np.float32)
    h = fa.synth_normal_bf16(seed, 9100, (2, HD))
    note("small-M duplicates")
    out, _, _ = run_dev(fa, ctx, h, eids, wts, 1)
    ref, _, _ = reference_any_tk(fa, oracle, seed, h, eids, wts, True)
    assert rel_l2(bf16_to_f32(out), ref) < TOL


def test_small_m_invalid_expert_id(fa, oracle, c2_layer):
    """An out-of-range id: the host entry fails with FST_EINVAL (both paths);
    on the device entry the pair contributes zero, as in the chain."""
    ctx, seed, _ = c2_layer
    h = fa.synth_normal_bf16(seed, 9200, (1, HD))
    eids = np.array([[3, E, 7, -1, 8, 9]], np.int32)
    wts = np.full((1, TK), 1.0 / TK, np.float32)
    for small in (True, False):
        ctx.set_small_m(small)
        try:
            with pytest.raises(fa.FstError) as ei:
                ctx.expert_ffn(0, h, eids, wts)
            assert ei.value.code == fa.FST_EINVAL
        finally:
            ctx.set_small_m(True)
    note("small-M invalid id, device entry")
    out, _, _ = run_dev(fa, ctx, h, eids, wts, 0)
    c_out, _, _ = run_dev(fa, ctx, h, eids, wts, 0, small_m=False)
    # both device calls left the sticky expert-id bit; one check reports it
    with pytest.raises(fa.FstError) as ei:
        ctx.moe_check()
    assert ei.value.code == fa.FST_EINVAL
    ctx.moe_check()
    assert rel_l2(bf16_to_f32(out), bf16_to_f32(c_out)) < CHAIN_TOL
    valid = eids.copy()
    keep = (eids >= 0) & (eids < E)
    valid[~keep] = 3
    w0 = np.where(keep, wts, 0.0).astype(np.float32)
    ref, _, _ = reference_any_tk(fa, oracle, seed, h, valid, w0, False)
    assert rel_l2(bf16_to_f32(out), ref) < TOL


def test_small_m_shared_only(fa, oracle, c2_layer):
    ctx, seed, _ = c2_layer
    for M in (1, 2):
        h = fa.synth_normal_bf16(seed, 9300 + M, (M, HD))
        note("small-M shared only M=%d" % M)
        out = ctx.shared_expert(0, h)
        ref = oracle.expert_ffn(0, fa.synth_q4k_expert(seed, E), h)
        assert rel_l2(bf16_to_f32(out), ref) < TOL


def test_small_m_repeated_calls_changing_slots(fa, c2_layer):
    """Slot counts 1, 7, 2, 13, 1 in a row (about; random experts may
    coincide): the per-tile counters of the
    multi-slot combine end every call at zero."""
    ctx, seed, _ = c2_layer
    cases = [(1, 1, 0), (1, 6, 1), (2, 1, 0), (2, 6, 1), (1, 1, 0)]
    for i, (M, tk, shared) in enumerate(cases):
        eids, wts = routing(950 + i, M, tk)
        h = fa.synth_normal_bf16(seed, 9400 + i, (M, HD))
        note("repeated call %d: M=%d tk=%d shared=%d" % (i, M, tk, shared))
        a = run(fa, ctx, h, eids, wts, shared)[0]
        b = run(fa, ctx, h, eids, wts, shared, small_m=False)[0]
        assert rel_l2(bf16_to_f32(a), bf16_to_f32(b)) < CHAIN_TOL
