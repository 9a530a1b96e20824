import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle import pyoracle
    pyoracle.lib()
    return pyoracle


@pytest.fixture(scope="session")
def fa():
    import fastar_amd
    fastar_amd.lib()
    return fastar_amd


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


HD, INTER = 4096, 2048
C2_SEED = 2024


@pytest.fixture(scope="session")
def c2_layer(fa):
    """One resident MoE layer: 256 routed + 1 shared Q4_K experts (3.64 GB) and
    a bf16 router ~N(0, 0.02), all generated from C2_SEED."""
    print("[gpu-test] create C2 ctx: 256 routed + 1 shared Q4_K experts", flush=True)
    ctx = fa.Context(n_experts=256, top_k=6, max_tokens=64)
    # generated on the device; byte-identical to fa.synth_q4k_expert(C2_SEED, e)
    ctx.synth_experts(C2_SEED, 0, 0, 257, 0)
    w = fa.synth_normal_bf16(C2_SEED, 1000, (HD, 256), 0.0, 0.02)
    ctx.upload_router_bf16(0, w)
    yield ctx, C2_SEED, w
    ctx.close()
