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


@pytest.fixture(scope="session")
def codec_gguf(model_dir):
    return synth.ensure_codec_gguf(model_dir)


def random_codes(n_frames, seed):
    """Codebook-major codes [10][n_frames]: row 0 semantic in [0, 4096), rows
    1..9 residual in [0, 1024) (rvq_lookup_codes, codec.rs:2536-2596)."""
    import numpy as np

    rng = np.random.default_rng(seed)
    sem = rng.integers(0, 4096, (1, n_frames))
    res = rng.integers(0, 1024, (9, n_frames))
    return np.concatenate([sem, res]).astype(np.int32)
