import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "boa-constrictor_amd")
ORACLE = os.path.join(ROOT, "oracle")
for p in (PKG, ORACLE, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs the HIP library)")


@pytest.fixture(scope="session")
def oracle():
    import refcpu
    refcpu.lib()
    return refcpu


@pytest.fixture(scope="session")
def weights_dir(tmp_path_factory):
    return tmp_path_factory.mktemp("weights")


def _weights(weights_dir, d, L, ds=16, seed=0, fp16=False):
    import synth
    p = weights_dir / f"w_d{d}_L{L}_s{ds}_seed{seed}{'_fp16' if fp16 else ''}.bin"
    if not p.exists():
        synth.write_random_weights(str(p), d, L, ds, seed=seed, fp16=fp16)
    return p


@pytest.fixture(scope="session")
def w_c1(weights_dir):
    """BASELINE config 1 model: d_model=64, 2 layers, d_state=16, seed 0."""
    return _weights(weights_dir, 64, 2)


@pytest.fixture(scope="session")
def make_weights(weights_dir):
    def f(d, L, ds=16, seed=0, fp16=False):
        return _weights(weights_dir, d, L, ds, seed, fp16)
    return f
