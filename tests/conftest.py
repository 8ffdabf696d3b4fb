import os
import sys
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mac-gpu-compiler_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

import qe  # noqa: E402

# Small Qwen3-shaped config for fast parity runs: head_dim 128 and 2 q heads per KV head like
# the real model, everything else shrunk.
TINY = qe.Config(256, 512, 2, 4, 2, 128, 1000, 1e-6, 1e6, 999)
TINY_SEED = 1234
REAL_SEED = 20260101          # seed of the random-init Qwen3-0.6B-architecture checkpoint
PROMPT_SEED = 7               # seed of the 130-token random prompt
PROMPT_LEN = 130
DECODE_STEPS = 128


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libqe.so")
    config.addinivalue_line("markers", "slow: takes more than ~20 s")


@pytest.fixture(scope="session")
def workdir():
    d = os.environ.get("QE_TEST_DIR") or tempfile.mkdtemp(prefix="qe_tests_")
    os.makedirs(d, exist_ok=True)
    return d


@pytest.fixture(scope="session")
def tiny_ckpt(workdir):
    return qe.write_random_checkpoint(os.path.join(workdir, "tiny"), TINY_SEED, TINY)


@pytest.fixture(scope="session")
def real_ckpt(workdir):
    d = os.path.join(workdir, "qwen3_0_6b")
    path = os.path.join(d, "model.safetensors")
    if not os.path.exists(path):
        qe.write_random_checkpoint(d, REAL_SEED, qe.QWEN3_0_6B)
    return path


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
