"""GPU tests of the measurement hooks bench.py relies on: the kernel ring
(HIP events attached to the fused MoE launch's dispatch) records one duration
per fused call, none for calls that take the launch chain, and empties on
read; recording does not change the layer's output."""
import numpy as np
import pytest

from tests.test_gpu_moe import HD

pytestmark = pytest.mark.gpu


def test_kernel_ring_records_fused_launches(fa, c2_layer):
    ctx, seed, _ = c2_layer
    h = fa.synth_normal_bf16(seed, 7100, (8, HD))
    print("[gpu-test] kernel ring", flush=True)
    ref, _, _ = ctx.moe_layer(0, h)
    ctx.kernel_ring(4)
    try:
        outs = [ctx.moe_layer(0, h)[0] for _ in range(6)]  # two more calls than the ring holds
        us = ctx.kernel_ring_read()
    finally:
        ctx.kernel_ring(0)
    assert len(us) == 4
    assert np.all(us > 1.0) and np.all(us < 10000.0)
    for o in outs:
        assert np.array_equal(o, ref)
    assert len(ctx.kernel_ring_read()) == 0  # emptied by the read
    # the launch chain (fused launch off) records nothing
    ctx.kernel_ring(4)
    ctx.set_fused(False)
    try:
        o, _, _ = ctx.moe_layer(0, h)
        assert len(ctx.kernel_ring_read()) == 0
    finally:
        ctx.set_fused(True)
        ctx.kernel_ring(0)
    assert np.array_equal(o, ref)  # the two paths agree bit for bit
    # a smaller capacity after a larger one records only that many launches
    ctx.kernel_ring(8)
    ctx.kernel_ring(2)
    try:
        for _ in range(4):
            ctx.moe_layer(0, h)
        assert len(ctx.kernel_ring_read()) == 2
    finally:
        ctx.kernel_ring(0)
