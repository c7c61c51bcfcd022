"""Full-size parity: the HIP engine at the benchmark shapes against the CPU
oracle's committed fixtures (tests/golden/full/*.json, written by
tests/golden/make_full_fixtures.py in the build container).

Each test rebuilds the fixture's seeded synthetic GGUF (checked by sha256)
and prompt (checked by sha256), then:

* cfg2 (S2-Pro shape, f16, 256-token prompt, KV 768) and cfg4 (Q4_0, KV 1280):
  the prompt's post-final-norm hidden within 1e-4 relative, and 64 greedy
  frames bit-exact with the final RNG state (generate.rs:117-221);
* cfg3 (Q8_0, T 0.7, top-p 0.9, SeededRng 1): 32 sampled frames equal, or the
  first differing draw sits at a boundary of the oracle's own probabilities
  (tests/loop_util.py: a draw target or top-p sum within 1e-4, or a logit
  tie within 1e-4 relative) -- after it the trajectories may part;
* cfg5 (8 voice-clone requests of 1500 positions, batch 8, KV 2560):
  requests 0 and 1 of the batch bit-exact over 16 greedy frames, with every
  request's frame count.
"""

import hashlib
import json
import os

import numpy as np
import pytest

from loop_util import at_boundary
from s2hip import synth

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
FIX = os.path.join(HERE, "golden", "full")
MODEL_DIR = os.environ.get("S2HIP_MODEL_DIR", "/tmp/s2hip_models")
_verified = {}


def _fixture(name):
    with open(os.path.join(FIX, name + ".json")) as f:
        return json.load(f)


def _sha256(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        while True:
            b = f.read(1 << 24)
            if not b:
                return h.hexdigest()
            h.update(b)


def _model(fx):
    shape = synth.SHAPES[fx["shape"]]
    path = synth.ensure_gguf(shape, MODEL_DIR, threads=min(16, os.cpu_count() or 1))
    if path not in _verified:
        _verified[path] = _sha256(path)
    assert _verified[path] == fx["gguf_sha256"], f"{path} differs from the fixture's model"
    return shape, path


def _prompt(shape, fx, request):
    recipe = fx["prompt_recipe"]
    if recipe[0] == "synthetic":
        p = synth.synthetic_prompt(shape, recipe[1], seed=shape.seed)
    else:
        p = synth.voice_clone_prompt(shape, recipe[1], recipe[2], seed=shape.seed + 100 * request)
    return p


def _check_prompt(p, req):
    assert hashlib.sha256(np.ascontiguousarray(p, np.int32).tobytes()).hexdigest() == req["prompt_sha256"]


def _rel(a, b):
    return float(np.max(np.abs(a - b)) / max(1e-30, float(np.max(np.abs(b)))))


def _draw_order(codes):
    """(frame, codebook) in draw order: semantic code, then codebooks 1..9."""
    ncb, n = codes.shape
    return [(t, cb) for t in range(n) for cb in range(ncb)]


def _first_difference(got, want):
    for t, cb in _draw_order(want):
        if got[cb, t] != want[cb, t]:
            return t, cb
    return None


def _margins(req, t, cb):
    for d in req["draws"]:
        if d[0] == t and d[1] == cb:
            return d[3], d[4], d[5]
    raise KeyError((t, cb))


def _engine(path, fx):
    from s2hip import Engine

    return Engine(path, fx["max_seq"], fx["im_end_id"])


@pytest.mark.parametrize("name", ["cfg2", "cfg4"])
def test_full_size_greedy_codes_bit_exact(name):
    fx = _fixture(name)
    shape, path = _model(fx)
    req = fx["requests"][0]
    prompt = _prompt(shape, fx, 0)
    _check_prompt(prompt, req)
    want = np.array(req["codes"], np.int32)
    with _engine(path, fx) as e:
        hidden, _ = e.eval(prompt, want_logits=False)
        assert _rel(hidden, np.array(req["hidden_prefill"], np.float32)) < 1e-4
        e.reset()
        r = e.generate_codes(prompt, fx["frames"], fx["temperature"], fx["top_p"], fx["top_k"],
                             fx["min_tokens_before_end"], req["rng_seed"])
    assert r["n_frames"] == fx["frames"]
    diff = _first_difference(r["codes"], want)
    assert diff is None, (f"{name}: first differing draw at frame {diff[0]} codebook {diff[1]}; "
                          f"oracle margins (draw, cut, tie) {_margins(req, *diff)}")
    assert r["rng_state"] == req["rng_state"]


def test_full_size_q8_sampled_codes_match():
    fx = _fixture("cfg3")
    shape, path = _model(fx)
    req = fx["requests"][0]
    prompt = _prompt(shape, fx, 0)
    _check_prompt(prompt, req)
    want = np.array(req["codes"], np.int32)
    with _engine(path, fx) as e:
        hidden, _ = e.eval(prompt, want_logits=False)
        assert _rel(hidden, np.array(req["hidden_prefill"], np.float32)) < 2e-2  # quantized path
        e.reset()
        r = e.generate_codes(prompt, fx["frames"], fx["temperature"], fx["top_p"], fx["top_k"],
                             fx["min_tokens_before_end"], req["rng_seed"])
    assert r["n_frames"] == fx["frames"]
    diff = _first_difference(r["codes"], want)
    if diff is None:
        assert r["rng_state"] == req["rng_state"]
        return
    t, cb = diff
    mg = _margins(req, t, cb)
    chosen = want[cb, t]
    # the logit scale of a Fast-AR codebook logit or a semantic logit is O(1)
    # here; at_boundary takes max(1, |logit|) for the tie test
    assert at_boundary(1.0, mg), (f"cfg3: draw at frame {t} codebook {cb} differs (oracle token {chosen}) "
                                  f"away from any boundary: margins {mg}")


def test_full_size_voice_clone_batch_of_8_bit_exact():
    fx = _fixture("cfg5")
    shape, path = _model(fx)
    n = fx["n_requests"]
    prompts = [_prompt(shape, fx, b) for b in range(n)]
    for req in fx["requests"]:
        _check_prompt(prompts[req["index"]], req)
    with _engine(path, fx) as e:
        rb = e.generate_codes_batch(prompts, fx["frames"], fx["temperature"], fx["top_p"], fx["top_k"],
                                    fx["min_tokens_before_end"], [1 + b for b in range(n)])
    assert [q["n_frames"] for q in rb["requests"]] == [fx["frames"]] * n
    for req in fx["requests"]:
        got = rb["requests"][req["index"]]
        want = np.array(req["codes"], np.int32)
        diff = _first_difference(got["codes"], want)
        assert diff is None, (f"request {req['index']}: first differing draw at frame {diff[0]} codebook "
                              f"{diff[1]}; oracle margins {_margins(req, *diff)}")
        assert got["rng_state"] == req["rng_state"]
