import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "fish-s2pro_amd"), ROOT, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

from s2hip import synth  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device")


def make_prompt(shape, n_tokens, seed):
    """Time-major flat prompt of uniform random text ids (codebook rows 0)."""
    return synth.synthetic_prompt(shape, n_tokens, seed)


@pytest.fixture(scope="session")
def model_dir(tmp_path_factory):
    return str(tmp_path_factory.mktemp("models"))


@pytest.fixture(scope="session")
def tiny_gguf(model_dir):
    return synth.ensure_gguf(synth.TINY, model_dir)


@pytest.fixture(scope="session")
def tiny_q8_gguf(model_dir):
    return synth.ensure_gguf(synth.TINY.with_(linear_type=synth.GGML_Q8_0), model_dir)


@pytest.fixture(scope="session")
def tiny_q4_gguf(model_dir):
    return synth.ensure_gguf(synth.TINY.with_(linear_type=synth.GGML_Q4_0), model_dir)
