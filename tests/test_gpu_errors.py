"""GPU tests of the error channel of the stream-ordered MoE path.

The reference raises a failed NPU dispatch as an exception per dispatch
(npu_run_wait / flush_pending_runs, src/fst_engine.cpp:200-223).  Here each
MoE launch ORs what it detects into a sticky word that only the host clears
(fst_moe_check, and the host-pointer entry points before they return).  An
error raised in a middle layer of an 8-layer verify forward must survive the
layers after it.  The timeout path is forced from the host with a spin limit
of one poll: the kernels' bounded waits give up and every kernel still exits
normally."""
import ctypes as C

import numpy as np
import pytest

from tests.helpers import bf16_to_f32, rel_l2

pytestmark = pytest.mark.gpu

HD = 4096


def _log(*a):
    print("[gpu-test]", *a, flush=True)


def _stack(fa, L, E, tk, V, seed, n_hash_layers=0):
    ctx = fa.Context(n_experts=E, top_k=tk, max_tokens=64, n_layers=L, vocab_size=V, n_hash_layers=n_hash_layers)
    for l in range(L):
        ctx.synth_experts(seed, l, 0, E + 1, l * 1000)
        ctx.upload_router_bf16(l, fa.synth_normal_bf16(seed, 1000 + l, (HD, E), 0.0, 0.02))
    for l in range(L + 1):
        ctx.upload_norm(l, fa.synth_normal_bf16(seed, 2000 + l, (HD,), 1.0, 0.1))
    ctx.synth_lm_head(seed, 999999)
    return ctx


@pytest.mark.parametrize("M", [8, 16])
def test_hash_id_error_in_layer_2_of_8_is_reported(fa, M):
    """Layer 2 (the only layer with a hash table) sees an input id outside the
    vocabulary; layers 3..7 route normally afterwards.  The host-pointer
    verify forward returns FST_EINVAL, and so does fst_moe_check after the
    device-pointer forward.  M = 8 runs the fused launch (top-k inside it), M =
    16 the launch chain (top-k inside its gate||up launch)."""
    L, E, tk, V, seed = 8, 8, 2, 1280, 71
    _log("hash-id error in layer 2 of 8, M=%d" % M)
    with _stack(fa, L, E, tk, V, seed, n_hash_layers=3) as ctx:
        table = np.random.default_rng(3).integers(0, E, (V, tk)).astype(np.int32)
        ctx.upload_hash_table(2, table)
        h0 = fa.synth_normal_bf16(seed, 3000, (M, HD))
        good = np.arange(M, dtype=np.int32) * 7
        bad = good.copy()
        bad[M // 2] = V + 5
        logits, _ = ctx.verify_forward(h0, good)
        assert np.isfinite(logits).all()
        with pytest.raises(fa.FstError) as ei:
            ctx.verify_forward(h0, bad)
        assert ei.value.code == fa.FST_EINVAL
        assert b"hash" in fa.lib().fst_last_error()
        # the check cleared the word: the next good call is clean and gives
        # the same logits as before
        logits2, _ = ctx.verify_forward(h0, good)
        assert np.array_equal(logits, logits2)

        # device-pointer forward: FST_OK at issue, the error at fst_moe_check
        lib = fa.lib()
        dh = ctx.to_device(h0)
        di = ctx.to_device(bad)
        dl = ctx.dev_alloc(M * V * 4)
        try:
            assert lib.fst_verify_forward_dev(ctx.h, dh, M, di, dl) == fa.FST_OK
            assert lib.fst_moe_check(ctx.h) == fa.FST_EINVAL
            assert lib.fst_moe_check(ctx.h) == fa.FST_OK
            dg = ctx.to_device(good)
            assert lib.fst_verify_forward_dev(ctx.h, ctx.to_device(h0), M, dg, dl) == fa.FST_OK
            assert lib.fst_moe_check(ctx.h) == fa.FST_OK
        finally:
            for p in (dh, di, dl):
                ctx.dev_free(p)


def test_expert_id_error_of_dev_call_is_sticky(fa):
    """An out-of-range expert id given to fst_moe_ffn_dev is reported by
    fst_moe_check even after later good calls on the same stream."""
    E, tk, seed, M = 8, 2, 72, 4
    with fa.Context(n_experts=E, top_k=tk, max_tokens=16) as ctx:
        ctx.synth_experts(seed, 0, 0, E + 1, 0)
        lib = fa.lib()
        h = fa.synth_normal_bf16(seed, 1, (M, HD))
        eids = np.array([[0, 1], [2, 3], [4, E + 3], [6, 7]], np.int32)
        wts = np.full((M, tk), 0.5, np.float32)
        good = np.array([[0, 1], [2, 3], [4, 5], [6, 7]], np.int32)
        dh, de, dg, dw = ctx.to_device(h), ctx.to_device(eids), ctx.to_device(good), ctx.to_device(wts)
        do = ctx.dev_alloc(M * HD * 2)
        try:
            assert lib.fst_moe_ffn_dev(ctx.h, 0, dh, M, de, dw, 1, do, None, None) == fa.FST_OK
            for _ in range(3):
                assert lib.fst_moe_ffn_dev(ctx.h, 0, dh, M, dg, dw, 1, do, None, None) == fa.FST_OK
            assert lib.fst_moe_check(ctx.h) == fa.FST_EINVAL
            assert b"expert id" in lib.fst_last_error()
            assert lib.fst_moe_check(ctx.h) == fa.FST_OK
        finally:
            for p in (dh, de, dg, dw, do):
                ctx.dev_free(p)


def test_recovery_after_forced_wait_give_up(fa, c2_layer):
    """With a spin limit of one poll the fused launch's and the small-M
    launch's hand-off waits may give up (the host forces it; the kernels exit
    normally).  The call then returns FST_OK with a correct result, or
    FST_EHIP.  With the default limit restored the next calls match the
    launch chain bit for bit (fused) and within the FFN tolerance (small-M)."""
    ctx, seed, _ = c2_layer
    M = 8
    h = fa.synth_normal_bf16(seed, 9100, (M, HD))
    ctx.set_fused(False)
    ref, e_ref, w_ref = ctx.moe_layer(0, h)
    ctx.set_fused(True)
    h1 = h[:1].copy()
    eids = e_ref[:1].copy()
    wts = w_ref[:1].copy()
    ctx.set_small_m(False)
    ref1 = ctx.expert_ffn(0, h1, eids, wts)
    ctx.set_small_m(True)
    outcomes = []
    try:
        ctx.set_wait_limit(1)
        for _ in range(3):
            _log("fused launch at spin limit 1")
            try:
                out, _, _ = ctx.moe_layer(0, h)
                outcomes.append("ok")
                assert np.array_equal(out, ref)
            except fa.FstError as e:
                assert e.code == fa.FST_EHIP
                outcomes.append("ehip")
            _log("small-M launch at spin limit 1")
            try:
                o1 = ctx.expert_ffn(0, h1, eids, wts)
                outcomes.append("ok1")
                assert rel_l2(bf16_to_f32(o1), bf16_to_f32(ref1)) < 4e-3
            except fa.FstError as e:
                assert e.code == fa.FST_EHIP
                outcomes.append("ehip1")
    finally:
        ctx.set_wait_limit(0)
    _log("outcomes at spin limit 1: %s" % outcomes)
    for _ in range(2):
        out, e, w = ctx.moe_layer(0, h)
        assert np.array_equal(e, e_ref) and np.array_equal(out, ref)
        o1 = ctx.expert_ffn(0, h1, eids, wts)
        assert rel_l2(bf16_to_f32(o1), bf16_to_f32(ref1)) < 4e-3
    ctx.moe_check()
