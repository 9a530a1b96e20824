"""CPU tests pinning the verify-forward pieces of the oracle (RMSNorm with its
fixed summation order, the dense Q4_K linear used for the LM head) and the
shared synthetic-weight generator.  No GPU needed."""
import numpy as np
import pytest

from tests.helpers import bf16_to_f32, f32_to_bf16, make_q4k_block, rel_l2


def _bf16(rng, shape, mean=0.0, std=1.0):
    return f32_to_bf16(rng.normal(mean, std, shape).astype(np.float32)).reshape(shape)


# ------------------------------------------------------------------ RMSNorm

def test_rmsnorm_constant_row_closed_form(oracle):
    """x = c everywhere: ss = d c^2 exactly, r = 1/sqrt(c^2 + eps)."""
    d = 4096
    for c in (1.0, -3.5, 0.015625, 200.0):
        x = np.full((1, d), c, np.float32)
        w = f32_to_bf16(np.linspace(0.5, 1.5, d).astype(np.float32))
        r = np.float32(1.0 / np.sqrt(c * c + 1e-6))
        ref = f32_to_bf16((np.float32(c) * r) * bf16_to_f32(w))
        assert np.array_equal(oracle.rmsnorm(x, w)[0], ref)


def test_rmsnorm_vs_float64(oracle):
    """Within one bf16 rounding of the float64 formula (rms_cpu semantics)."""
    rng = np.random.default_rng(11)
    x = bf16_to_f32(_bf16(rng, (6, 4096), 0.0, 3.0))
    w = _bf16(rng, (4096,), 1.0, 0.1)
    out = bf16_to_f32(oracle.rmsnorm(x, w)).astype(np.float64)
    r = 1.0 / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6)
    ref = x * r * bf16_to_f32(w)
    assert np.all(np.abs(out - ref) <= 2.0 ** -7 * np.abs(ref) + 1e-30)


def test_rmsnorm_power_of_two_invariance(oracle):
    """With eps = 0, scaling x by 2^k leaves every output bit unchanged (the
    sum of squares scales exactly in double, r by 2^-k exactly)."""
    rng = np.random.default_rng(12)
    x = bf16_to_f32(_bf16(rng, (4, 4096)))
    w = _bf16(rng, (4096,), 1.0, 0.1)
    a = oracle.rmsnorm(x, w, eps=0.0)
    for k in (-20, -3, 5, 30):
        assert np.array_equal(oracle.rmsnorm(x * np.float32(2.0 ** k), w, eps=0.0), a)


def test_resid_norm_adds_in_bf16(oracle):
    rng = np.random.default_rng(13)
    h = _bf16(rng, (2, 4096))
    y = _bf16(rng, (2, 4096), 0.0, 0.5)
    w = _bf16(rng, (4096,), 1.0, 0.1)
    x, n = oracle.resid_norm(h, y, w)
    assert np.array_equal(x, f32_to_bf16(bf16_to_f32(h) + bf16_to_f32(y)).reshape(h.shape))
    assert np.array_equal(n, oracle.rmsnorm(bf16_to_f32(x).reshape(x.shape), w))


# ------------------------------------------------------- dense Q4_K linear

def test_q4k_linear_ones_known_answer(oracle):
    """All weights 1 (d = 1, sc = 1, q = 1, m = 0): y[m][n] = sum_k x[m][k]
    (ones@ones of src/fst_engine.cpp:5755-5794 generalised to any x)."""
    blk = make_q4k_block(0x3C00, 0x0000, [1] * 8, [0] * 8, [1] * 256)
    N, K = 32, 512
    blocks = np.tile(blk, N * (K // 256))
    rng = np.random.default_rng(14)
    x = _bf16(rng, (3, K))
    y = oracle.q4k_linear(blocks, x, N, K)
    ref = bf16_to_f32(x).astype(np.float64).sum(1)
    assert np.allclose(y, ref[:, None], rtol=0, atol=1e-4)


def test_q4k_linear_vs_dequant_matmul(oracle):
    """Against dequantise-then-matmul in float64, and the transposed product
    must not match (orientation A.B^T, scripts/fst_validate_gemms.py:173-186)."""
    from fastar_amd import synth_q4k_blocks
    N, K = 96, 1024
    blocks = synth_q4k_blocks(77, 5, N * K // 256)
    W = oracle.q4k_dequant(blocks).reshape(N, K).astype(np.float64)
    rng = np.random.default_rng(15)
    x = _bf16(rng, (4, K))
    y = oracle.q4k_linear(blocks, x, N, K)
    ref = bf16_to_f32(x).astype(np.float64) @ W.T
    assert rel_l2(y, ref) < 1e-6
    # a wrong block order (row-major over K instead of N) must be detected
    Wt = oracle.q4k_dequant(blocks).reshape(K // 256, N, 256).transpose(1, 0, 2).reshape(N, K)
    assert rel_l2(bf16_to_f32(x).astype(np.float64) @ Wt.T, ref) > 0.5


# ------------------------------------------------------ synthetic generator

def test_synth_q4k_expert_is_block_stream(fa):
    """An expert is blocks 0..3*hd*inter/256-1 of its generator stream."""
    e = fa.synth_q4k_expert(3, 9, hd=512, inter=256)
    b = fa.synth_q4k_blocks(3, 9, 3 * 512 * 256 // 256)
    assert np.array_equal(e, b)
    assert not np.array_equal(e, fa.synth_q4k_expert(3, 10, hd=512, inter=256))


def test_synth_q4k_scale_statistics(fa):
    """d, dmin = fp16(|z| sigma) with z Irwin-Hall N(0,1): |z| <= 6 and the
    half-normal mean sigma*sqrt(2/pi)."""
    b = fa.synth_q4k_blocks(21, 1, 20000, d_sigma=0.01).reshape(-1, 144)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float64).ravel()
    dm = b[:, 2:4].copy().view(np.float16).astype(np.float64).ravel()
    for v in (d, dm):
        assert np.all(v >= 0) and np.all(v <= 0.06 + 1e-6)
        assert abs(v.mean() - 0.01 * np.sqrt(2 / np.pi)) < 3e-4
    # the nibble and scale bytes are uniform
    assert abs(b[:, 16:].astype(np.float64).mean() - 127.5) < 1.0
