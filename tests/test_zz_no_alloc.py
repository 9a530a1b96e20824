"""The allocation-free greedy acceptance entry point
(fst_accept_greedy_dev_noalloc, fixed per-device scratch) against
fst_accept_greedy_dev through the C-ABI: two calls in a row, the second with
a smaller input, each bit-exact against the workspace entry point and the
oracle.  Collected last: it must also pass alone in a fresh process."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _planted(fa, seed, n_seq, k, V, prefixes):
    t = fa.synth_normal_f32(seed, 1, (n_seq, k + 1, V), 0.0, 2.0)
    draft = np.zeros((n_seq, k), np.int32)
    for s in range(n_seq):
        for i in range(k):
            am = int(np.argmax(t[s, i]))
            draft[s, i] = am if i < prefixes[s] else (am + 1 + i) % V
    return t, draft


@pytest.mark.parametrize("shapes", [((4, 7, 129280, [0, 3, 7, 5]), (2, 3, 50000, [3, 1]))])
def test_noalloc_greedy_matches_workspace_entry(fa, oracle, shapes):
    L = fa.lib()
    ctx = fa.Context(n_experts=8, top_k=1, max_tokens=16)
    try:
        for call, (n_seq, k, V, pre) in enumerate(shapes):
            print("[gpu-test] noalloc greedy call %d: n_seq=%d k=%d V=%d" % (call, n_seq, k, V), flush=True)
            t, draft = _planted(fa, 11 + call, n_seq, k, V, pre)
            dt, dd = ctx.to_device(t), ctx.to_device(draft)
            outs = []
            for fn in (L.fst_accept_greedy_dev_noalloc, L.fst_accept_greedy_dev):
                dn = ctx.dev_alloc(4 * n_seq)
                dk = ctx.dev_alloc(4 * n_seq * (k + 1))
                fa._check(fn(ctx.h, dt, n_seq, k, V, dd, dn, dk))
                ctx.sync()
                n_acc = ctx.to_host(dn, (n_seq,), np.int32)
                tok = ctx.to_host(dk, (n_seq, k + 1), np.int32)
                assert L.fst_accept_check(fa._ptr(n_acc), n_seq) == fa.FST_OK
                outs.append((n_acc, tok))
                ctx.dev_free(dn)
                ctx.dev_free(dk)
            (na, ta), (nb, tb) = outs
            assert np.array_equal(na, nb) and np.array_equal(ta, tb)
            for s in range(n_seq):
                rn, rt = oracle.accept_greedy(t[s], draft[s])
                assert na[s] == rn == pre[s]
                assert np.array_equal(ta[s, :rn + 1], rt)
            ctx.dev_free(dt)
            ctx.dev_free(dd)
    finally:
        ctx.close()


def test_noalloc_rejects_oversized_call(fa):
    L = fa.lib()
    ctx = fa.Context(n_experts=8, top_k=1, max_tokens=16)
    try:
        # 300 sequences x 8 rows > the 2048-row scratch: rejected before any launch
        rc = L.fst_accept_greedy_dev_noalloc(ctx.h, None, 300, 7, 1000, None, None, None)
        assert rc == fa.FST_EINVAL
    finally:
        ctx.close()
