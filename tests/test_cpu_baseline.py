"""The benchmark's CPU baseline port (oracle/fst_cpu_baseline.c, fp32) computes
the same MoE-layer verify as the fp64 oracle: same routing, outputs within
the FFN tolerance.  Small shapes; built here with the benchmark's recipe."""
import ctypes as C
import os
import subprocess

import numpy as np

from tests.helpers import bf16_to_f32, rel_l2

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_cpu_baseline_matches_oracle(fa, oracle, tmp_path):
    out = str(tmp_path / "libcb.so")
    subprocess.run(["bash", os.path.join(ROOT, "oracle", "build_cpu_baseline.sh"), out], check=True)
    L = C.CDLL(out)
    P = C.c_void_p
    L.fcb_moe_step.argtypes = [P, C.c_int, P, C.c_int, C.c_int, P, C.c_int, C.c_int, P, P]
    L.fcb_moe_step.restype = C.c_int
    hd, inter, E, tk, M, seed = 512, 256, 8, 2, 5, 77
    experts = [fa.synth_q4k_expert(seed, e, hd, inter) for e in range(E + 1)]
    ptrs = (C.c_void_p * (E + 1))(*[x.ctypes.data for x in experts])
    w = fa.synth_normal_bf16(seed, 1, (hd, E), 0.0, 0.2)
    h = fa.synth_normal_bf16(seed, 2, (M, hd))
    out_ = np.empty((M, hd), np.uint16)
    eids = np.empty((M, tk), np.int32)
    L.fcb_set_threads.argtypes = [C.c_int]
    L.fcb_set_threads(2)
    n = L.fcb_moe_step(h.ctypes.data, M, w.ctypes.data, E, tk, ptrs, hd, inter, out_.ctypes.data, eids.ctypes.data)
    re_, rw, _ = oracle.router(h, w, None, tk)
    assert np.array_equal(eids, re_)
    assert n == len(set(re_.ravel().tolist()))
    y = np.zeros((M, tk, hd), np.float32)
    for m in range(M):
        for j in range(tk):
            y[m, j] = oracle.expert_ffn(0, experts[int(re_[m, j])], h[m:m + 1], hd, inter)[0]
    ys = oracle.expert_ffn(0, experts[E], h, hd, inter)
    _, ref = oracle.combine(y, ys, rw)
    assert rel_l2(bf16_to_f32(out_), ref) < 1e-2
