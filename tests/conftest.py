import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libc2h.so on the device)")
    config.addinivalue_line("markers", "slow: full-size model (minutes on the CPU oracle)")


@pytest.fixture(scope="session")
def tiny_model_path(tmp_path_factory):
    """2-layer model with the real per-layer shapes (E=896, FF=4864, 14/2
    heads) and a 4096-token vocabulary: every kernel shape of the decode path
    at a size the oracle runs in well under a second per token."""
    from c2slm_amd import gguf as G
    p = str(tmp_path_factory.mktemp("models") / "tiny.gguf")
    shape = G.ModelShape(n_layers=2, n_vocab=4096)
    G.write_synthetic_model(p, shape, seed=1234)
    return p


@pytest.fixture(scope="session")
def full_model_path(tmp_path_factory):
    """The Qwen2.5-0.5B-shaped synthetic model (24 layers, vocab 151936)."""
    from c2slm_amd import gguf as G
    p = str(tmp_path_factory.mktemp("models") / "qwen05b_synth.gguf")
    G.write_synthetic_model(p, G.QWEN05B, seed=20261201)
    return p
