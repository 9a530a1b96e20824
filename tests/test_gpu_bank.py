"""GPU tests of loading an .fst model file into a context (fst_bank_load_*):
a model loaded from the file computes exactly what the same tensors uploaded
through the individual entry points compute, and its routing (sqrt(softplus)
scores, bias, route_scale 1.5, bf16 logits, tid2eid hash layers) matches the
oracle bit for bit."""
import numpy as np
import pytest

from tests import fst_file
from tests.helpers import bf16_to_f32

pytestmark = pytest.mark.gpu

HD, INTER, L, E, TK, V, SEED = 4096, 2048, 2, 8, 2, 1280, 12


def _log(*a):
    print("[gpu-test]", *a, flush=True)


@pytest.fixture(scope="module")
def model(fa, tmp_path_factory):
    path = tmp_path_factory.mktemp("fst") / "model.fst"
    _log("writing", path)
    m = fst_file.build_model(fa, path, hd=HD, inter=INTER, L=L, E=E, tk=TK, V=V, seed=SEED, hash_layers=3)
    m["path"] = path
    return m


def _manual_ctx(fa, cfg, m, bias_decode):
    ctx = fa.Context(cfg)
    for l in range(L):
        for e in range(E):
            ctx.upload_expert(l, e, m["experts"][(l, e)])
        ctx.upload_router_bf16(l, np.ascontiguousarray(m["router"][l].T), bias_decode(m["bias"][l]))
        ctx.upload_norm(l, m["norm"][l])
        ctx.upload_shared_bf16(l, *m["shared"][l])
        ctx.upload_hc(l, *m["hc"][l])
        if l < cfg.n_hash_layers:
            ctx.upload_hash_table(l, m["tid2eid"][l])
    ctx.upload_norm(L, m["out_norm"])
    ctx.upload_lm_head_bf16(m["lm_head"])
    ctx.upload_hc_head(*m["hc_head"])
    return ctx


def test_loaded_model_equals_manual_upload(fa, model):
    _log("load .fst vs manual upload, verify forward in HC mode")
    with fa.Bank(model["path"]) as b:
        cfg = b.config(max_tokens=64)
        ctx = fa.Context(cfg)
        with ctx:
            for l in range(L):
                ctx.load_bank_layer(b, l)
            ctx.load_bank_head(b)
            with _manual_ctx(fa, cfg, model, lambda x: bf16_to_f32(x)) as ref:
                M = 16
                h0 = fa.synth_normal_bf16(SEED, 50, (M, 4, HD))
                ids = np.random.default_rng(1).integers(0, V, M).astype(np.int32)
                la, ha = ctx.verify_forward(h0, ids)
                lb, hb = ref.verify_forward(h0, ids)
                assert np.isfinite(la).all()
                assert np.array_equal(la, lb) and np.array_equal(ha, hb)


def test_loaded_routing_vs_oracle(fa, oracle, model):
    """Layer 0 is a hash layer (rows of the tid2eid sidecar), layer 1 scores
    with sqrt(softplus) + bias; weights and indices bit-exact vs the oracle."""
    _log("routing of the loaded model vs oracle")
    M = 8
    h = fa.synth_normal_bf16(SEED, 60, (M, HD))
    ids = np.random.default_rng(2).integers(0, V, M).astype(np.int32)
    kw = dict(score_func=1, route_scale=1.5, round_logits_bf16=1)
    with fa.Bank(model["path"]) as b:
        with fa.Context(b.config(max_tokens=64)) as ctx:
            for l in range(L):
                ctx.load_bank_layer(b, l, fa.BANK_ROUTER | fa.BANK_HASH)
            w0 = np.ascontiguousarray(model["router"][0].T)
            e, w = ctx.router(0, h, ids)
            er, wr, _ = oracle.router(h, w0, bf16_to_f32(model["bias"][0]), TK,
                                      hash_rows=model["tid2eid"][0][ids], **kw)
            assert np.array_equal(e, er) and np.array_equal(w, wr)
            w1 = np.ascontiguousarray(model["router"][1].T)
            e, w = ctx.router(1, h)
            er, wr, _ = oracle.router(h, w1, bf16_to_f32(model["bias"][1]), TK, **kw)
            assert np.array_equal(e, er) and np.array_equal(w, wr)
        # the engine's fp16 reading of the 2-byte bias (src/fst_engine.cpp:1626-1630)
        with fa.Context(b.config(max_tokens=64)) as ctx:
            ctx.load_bank_layer(b, 1, fa.BANK_ROUTER | fa.BANK_BIAS_AS_FP16)
            e, w = ctx.router(1, h)
            b16 = model["bias"][1].view(np.float16).astype(np.float32)
            er, wr, _ = oracle.router(h, w1, b16, TK, **kw)
            assert np.array_equal(e, er) and np.array_equal(w, wr)


def test_loaded_moe_layer_vs_oracle(fa, oracle, model):
    """One layer of the loaded model against the oracle: MXFP4 routed experts
    from the bank, the bf16 shared expert, combine with the loaded weights."""
    from tests.helpers import rel_l2
    _log("moe layer of the loaded model vs oracle")
    M = 8
    h = fa.synth_normal_bf16(SEED, 70, (M, HD))
    with fa.Bank(model["path"]) as b:
        with fa.Context(b.config(max_tokens=64)) as ctx:
            ctx.load_bank_layer(b, 1)
            out, eids, wts = ctx.moe_layer(1, h)
    y = np.zeros((M, TK, HD), np.float32)
    for ex in sorted(set(int(v) for v in eids.ravel())):
        rows = [m for m in range(M) if ex in eids[m]]
        ye = oracle.expert_ffn(1, model["experts"][(1, ex)], h[rows])
        for r, m in enumerate(rows):
            y[m, list(eids[m]).index(ex)] = ye[r]
    g, u, d = (bf16_to_f32(t).reshape(t.shape) for t in model["shared"][1])
    _, ref = oracle.combine(y, oracle.expert_ffn_f32(g, u, d, h), wts)
    assert rel_l2(bf16_to_f32(out), ref) < 1e-2
