"""Q8_0 / Q4_0 decode on 2560-wide rows (the S2-Pro model dimension).

The tiny test model has 512-wide rows; this small model (d = 2560, 4 + 2
layers) sends wqkv, the fused w1 / w3 + SwiGLU and the heads through the
decode GEMVs at the S2-Pro row width, where the repacked-block kernel takes
w1 / w3 as one block list.  Greedy codes must equal the oracle's bit for bit,
and eval hidden states / logits agree to 1e-4 relative.
"""

import numpy as np
import pytest

from conftest import make_prompt
from oracle import oracle as O
from s2hip import synth

pytestmark = pytest.mark.gpu

WIDE = synth.TINY.with_(name="tinywide", dim=2560, ffn=1536, fast_ffn=1536)


@pytest.fixture(scope="module", params=["q8_0", "q4_0"])
def wide(request, model_dir):
    shape = WIDE.with_(linear_type={"q8_0": synth.GGML_Q8_0, "q4_0": synth.GGML_Q4_0}[request.param])
    return shape, synth.ensure_gguf(shape, model_dir)


def _rel(a, b):
    return float(np.max(np.abs(a - b)) / max(1e-30, float(np.max(np.abs(b)))))


def test_wide_eval_matches_oracle(wide):
    from s2hip import Engine

    shape, path = wide
    e, o = Engine(path, 64, shape.im_end_id), O.OracleModel(path, 64, shape.im_end_id)
    prompt = make_prompt(shape, 16, seed=3)
    hg, lg = e.eval(prompt)
    ho, lo = o.eval(prompt)
    assert _rel(hg, ho) < 1e-4 and _rel(lg, lo) < 1e-4
    tok = np.zeros(11, np.int32)
    tok[0] = shape.semantic_begin + 7
    tok[1:] = np.arange(10) * 5
    hg, lg = e.step(tok)
    ho, lo = o.eval(tok)
    assert _rel(hg, ho) < 1e-4 and _rel(lg, lo) < 1e-4


def test_wide_greedy_codes_bit_exact(wide):
    from s2hip import Engine

    shape, path = wide
    prompt = make_prompt(shape, 24, seed=4)
    rg = Engine(path, 64, shape.im_end_id).generate_codes(prompt, 16, min_tokens_before_end=100)
    ro = O.OracleModel(path, 64, shape.im_end_id).generate_codes(prompt, 16, min_tokens_before_end=100)
    assert rg["n_frames"] == ro["n_frames"] == 16
    assert np.array_equal(rg["codes"], ro["codes"]) and rg["rng_state"] == ro["rng_state"]
