"""CPU tests of the C-ABI library: it loads, exports every symbol the public
header declares, reports its geometry, and its host-only synthetic input
generators are deterministic.  No GPU compute is issued."""
import ctypes as C
import os

import numpy as np
import pytest


def test_library_loads_and_exports_header_symbols(fa):
    # RTLD_NOW: every undefined symbol must resolve at load time
    lib = C.CDLL(fa.LIB_PATH, mode=os.RTLD_NOW)
    names = fa.header_symbols()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_header_declares_every_bound_function(fa):
    names = set(fa.header_symbols())
    bound = set(fa._SIGS)
    assert bound <= names, bound - names


def test_abi_version_and_defaults(fa):
    L = fa.lib()
    assert L.fst_abi_version() == 1
    c = fa.default_config()
    assert (c.hidden_dim, c.inter_dim, c.n_experts, c.top_k, c.vocab_size) == (4096, 2048, 256, 6, 129280)
    assert fa.expert_bytes(c) == 14155776
    c.codec = fa.CODEC_MXFP4
    assert fa.expert_bytes(c) == 13369344


def test_create_rejects_bad_config(fa):
    L = fa.lib()
    h = C.c_void_p()
    c = fa.default_config(top_k=0)
    assert L.fst_create(C.byref(c), C.byref(h)) == fa.FST_EINVAL
    c = fa.default_config(hidden_dim=1000)
    assert L.fst_create(C.byref(c), C.byref(h)) == fa.FST_EINVAL
    c = fa.default_config(max_tokens=65)
    assert L.fst_create(C.byref(c), C.byref(h)) == fa.FST_EINVAL
    assert b"max_tokens" in L.fst_last_error()


def test_create_without_gpu_fails_loudly(fa):
    if os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK | os.W_OK):
        pytest.skip("a GPU is visible")
    with pytest.raises(fa.FstError) as ei:
        fa.Context()
    assert ei.value.code == fa.FST_ENODEV


def test_synth_q4k_deterministic_and_distributed(fa):
    a = fa.synth_q4k_expert(5, 3, 512, 256)
    b = fa.synth_q4k_expert(5, 3, 512, 256)
    c = fa.synth_q4k_expert(5, 4, 512, 256)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    big = fa.synth_q4k_expert(9, 0)
    blocks = big.reshape(-1, 144)
    d = blocks[:, 0:2].copy().view(np.uint16).ravel().view(np.float16).astype(np.float64)
    assert np.all(d >= 0)
    assert abs(d.mean() - 0.01 * np.sqrt(2 / np.pi)) < 0.02 * 0.01 * np.sqrt(2 / np.pi) * 10
    sub = np.mean(blocks[:, 0:2].copy().view(np.uint16).ravel() < 0x0400)
    assert 0.002 < sub < 0.01            # ~0.5% of |N(0,0.01)| values are fp16 subnormals
    qs = blocks[:, 16:]
    assert abs(qs.mean() - 127.5) < 0.5  # uniform nibble bytes


def test_synth_normal(fa):
    x = fa.bf16_to_f32(fa.synth_normal_bf16(1, 2, (200000,)))
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01
    y = fa.synth_normal_f32(1, 2, (1001,), 3.0, 0.5)
    assert y.shape == (1001,) and abs(y.mean() - 3) < 0.1
    assert np.array_equal(fa.synth_normal_f32(1, 2, (1001,), 3.0, 0.5), y)


def test_f32_to_bf16_helper(fa):
    torch = pytest.importorskip("torch")
    x = np.random.default_rng(0).normal(0, 10, 5000).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(fa.f32_to_bf16(x), ref)


def test_accept_check_flags_abandoned_sequences(fa):
    # host-side handling of the greedy launch's bounded wait: a sequence
    # whose owner gave up reports n_acc = -1, which becomes FST_EHIP
    L = fa.lib()
    ok = np.array([0, 7, 3], np.int32)
    assert L.fst_accept_check(fa._ptr(ok), 3) == fa.FST_OK
    bad = np.array([2, -1, 0], np.int32)
    assert L.fst_accept_check(fa._ptr(bad), 3) == fa.FST_EHIP
    assert b"sequence 1" in L.fst_last_error()
    assert L.fst_accept_check(None, 3) == fa.FST_EINVAL
    assert L.fst_accept_check(fa._ptr(ok), 0) == fa.FST_EINVAL


def test_device_error_status_decoding(fa):
    # the sticky error bits of the MoE launches and the status each maps to
    L = fa.lib()
    assert L.fst_device_error_status(0) == fa.FST_OK
    assert L.fst_device_error_status(1) == fa.FST_EINVAL
    assert b"expert id" in L.fst_last_error()
    assert L.fst_device_error_status(2) == fa.FST_EINVAL
    assert b"hash" in L.fst_last_error()
    assert L.fst_device_error_status(4) == fa.FST_EHIP
    assert b"spin limit" in L.fst_last_error()
    # an id error outranks a timeout seen in the same calls
    assert L.fst_device_error_status(4 | 2) == fa.FST_EINVAL
    assert L.fst_device_error_status(1 | 2) == fa.FST_EINVAL
    assert b"hash" in L.fst_last_error()
    assert L.fst_moe_check(None) == fa.FST_EINVAL
