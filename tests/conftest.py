import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mojo-gemma4-cpu_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def O():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def gpu():
    """The HIP library on cuda:0.  A GPU test must never fall back to CPU:
    if the device or libbq.so is missing this fails loudly."""
    import torch
    assert torch.cuda.is_available(), "GPU test collected on a machine without a GPU"
    import bq
    bq.init(0)
    return bq


@pytest.fixture
def tune_env(gpu):
    """Set BQ_* tuning switches for one test: libbq reads them at bq_init,
    so each change re-runs it, and the old values are restored (and re-read)
    after the test."""
    saved = {}

    def set_(**kv):
        for k, v in kv.items():
            saved.setdefault(k, os.environ.get(k))
            os.environ[k] = str(v)
        gpu.init(0)

    yield set_
    for k, v in saved.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v
    gpu.init(0)


@pytest.fixture(scope="session")
def moe_model(gpu, O):
    """128-expert Gemma-4-26B-A4B expert weights (bf16 N(0, 0.02), numpy RNG),
    quantized with the oracle's reference recipe, re-tiled on the GPU once."""
    import numpy as np

    from test_gpu_parity import dev
    E, H, I = 128, 2816, 704
    rng = np.random.default_rng(0)
    gu = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((E * 2 * I, H), np.float32) * np.float32(0.02)))
    gq, gs = O.rotate_and_quant(gu, 128)
    del gu
    dn = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((E * H, I), np.float32) * np.float32(0.02)))
    dq, ds = O.rotate_and_quant(dn, 64)
    del dn
    Wgu = gpu.ButterquantWeight(gpu.retile(dev(gq.reshape(-1)), E * 2 * I, H), dev(gs), E * 2 * I, H)
    Wd = gpu.ButterquantWeight(gpu.retile(dev(dq.reshape(-1)), E * H, I), dev(ds), E * H, I)
    gp, gcs = O.pack_and_colsum(gq)
    dp, dcs = O.pack_and_colsum(dq, 64, False)
    return dict(E=E, H=H, I=I, gs=gs, ds=ds, gp=gp, gcs=gcs, dp=dp, dcs=dcs, Wgu=Wgu, Wd=Wd)

# the CPU port's OpenMP team (oracle/cpu_baseline.c) sleeps between parallel
# regions: spinning threads on a CPU share no larger than the team throttle
# the process (read when the port's libgomp loads, after this module)
os.environ.setdefault("OMP_WAIT_POLICY", "PASSIVE")
