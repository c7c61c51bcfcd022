"""Writes tests/golden/*.json from the CPU oracle on the seeded tiny model.

Run from the repository root after building (python tests/golden/make_golden.py).
The fixtures pin (a) the synthetic-model writer (sha256 of the GGUF), and
(b) the oracle's greedy code ids for the tiny dual-AR shape: 32-token prompt
of uniform random text ids (seed 0), 16 frames, im_end blocked.
"""

import hashlib
import json
import os
import sys
import tempfile

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [os.path.join(ROOT, "fish-s2pro_amd"), ROOT, os.path.join(ROOT, "tests")]

from conftest import make_prompt  # noqa: E402
from oracle import oracle as O  # noqa: E402
from s2hip import synth  # noqa: E402


def sha256(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for blk in iter(lambda: f.read(1 << 20), b""):
            h.update(blk)
    return h.hexdigest()


def main():
    out_dir = os.path.dirname(os.path.abspath(__file__))
    with tempfile.TemporaryDirectory() as d:
        sums = {}
        for key, shape in (("tiny_f16", synth.TINY),
                           ("tiny_q8_0", synth.TINY.with_(linear_type=synth.GGML_Q8_0)),
                           ("tiny_q4_0", synth.TINY.with_(linear_type=synth.GGML_Q4_0))):
            sums[key] = sha256(synth.write_gguf(shape, os.path.join(d, shape.file_name())))
        path = os.path.join(d, synth.TINY.file_name())
        prompt = make_prompt(synth.TINY, 32, seed=0)
        m = O.OracleModel(path, 64, synth.TINY.im_end_id)
        r = m.generate_codes(prompt, 16, 0.0, 1.0, 0, 1000, 0)
        gold = {
            "shape": "tiny", "gguf_sha256": sums, "prompt_flat": prompt.tolist(), "max_new_tokens": 16,
            "min_tokens_before_end": 1000, "temperature": 0.0, "top_p": 1.0, "top_k": 0, "rng_seed": 0,
            "n_frames": r["n_frames"], "rng_state": r["rng_state"], "codes": r["codes"].tolist(),
        }
        with open(os.path.join(out_dir, "tiny_greedy_codes.json"), "w") as f:
            json.dump(gold, f)
        print("wrote", os.path.join(out_dir, "tiny_greedy_codes.json"), r["n_frames"], "frames")


if __name__ == "__main__":
    main()
