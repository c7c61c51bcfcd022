"""Writes the full-size parity fixtures: the CPU oracle's outputs at the
benchmark shapes, for the GPU tests in tests/test_gpu_full.py.

Run in the build container (the oracle at full size takes minutes per
config; the GPU box only reads the committed JSON):

    python tests/golden/make_full_fixtures.py [--configs cfg2,cfg3,cfg4,cfg5]

Each config writes tests/golden/full/<name>.json with the seeded synthetic
GGUF it used (file name + sha256), the prompt recipe (+ sha256 of its int32
ids), the post-final-norm hidden of the prompt's last token, and the
oracle's own generation: codebook-major codes, the final SeededRng state and
every draw with its margins (sample_token_margins: distance of the draw target
from the cumulative-probability boundaries, of the top-p sums from top_p, and
the chosen logit's gap to its sort-order neighbours).

The loop restates generate_codes (crates/fish_s2_infer/src/generate.rs:117-221)
with im_end blocked for every frame (min_tokens_before_end >= frames), so each
run yields exactly `frames` frames: semantic draw -> codebook 0 = main -
semantic_begin -> nine Fast-AR draws (fast_ar.rs:440-470) -> Slow step on
[main, codes] -> next semantic draw.  The draw order and RNG steps are the
ones tests/loop_util.py replays.
"""

import argparse
import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "fish-s2pro_amd"), ROOT, os.path.dirname(HERE)]

from oracle import oracle as O  # noqa: E402
from s2hip import synth  # noqa: E402

OUT = os.path.join(HERE, "full")
NEVER_END = 1 << 30

# name: shape, prompt recipe, KV capacity, frames, sampler, rng seed, requests
CONFIGS = {
    "cfg2": dict(shape="full", prompt=("synthetic", 256), max_seq=768, frames=64,
                 sampler=(0.0, 1.0, 0), rng=1,
                 what="full S2-Pro shape, f16, seed 1, 256-token prompt, greedy, KV 768"),
    "cfg3": dict(shape="full_q8", prompt=("synthetic", 256), max_seq=768, frames=64,
                 sampler=(0.7, 0.9, 0), rng=1,
                 what="full shape, Q8_0 linears, 256-token prompt, T 0.7 top-p 0.9 top-k 0, SeededRng seed 1"),
    "cfg4": dict(shape="full_q4", prompt=("synthetic", 256), max_seq=1280, frames=64,
                 sampler=(0.0, 1.0, 0), rng=1,
                 what="full shape, Q4_0 linears, 256-token prompt, greedy, KV 1280"),
    "cfg5": dict(shape="full", prompt=("voice_clone", 500, 1000), max_seq=2560, frames=16,
                 sampler=(0.0, 1.0, 0), rng=1, requests=8, oracle_requests=(0, 1, 2, 3),
                 what="full shape, f16, 8 requests of 500 text ids + 1000 reference frames "
                      "(1500 positions), greedy, batch 8, KV 2560; requests 0 to 3 run on the oracle"),
}


def sha256_file(path, chunk=1 << 24):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        while True:
            b = f.read(chunk)
            if not b:
                return h.hexdigest()
            h.update(b)


def prompt_for(shape, recipe, request=0):
    """The prompt of a config's request (the recipes bench.py uses)."""
    if recipe[0] == "synthetic":
        return synth.synthetic_prompt(shape, recipe[1], seed=shape.seed)
    n_text, n_frames = recipe[1], recipe[2]
    return synth.voice_clone_prompt(shape, n_text, n_frames, seed=shape.seed + 100 * request)


def prompt_sha(prompt):
    return hashlib.sha256(np.ascontiguousarray(prompt, np.int32).tobytes()).hexdigest()


def oracle_generation(m, prompt, frames, sampler, rng):
    spec = m.spec
    T, top_p, top_k = sampler
    ncb = spec.num_codebooks
    m.reset()
    hidden, logits = m.eval(prompt)
    hidden_prefill = hidden.copy()
    codes = np.zeros((ncb, frames), np.int32)
    draws = []

    def semantic(lg, st):
        b = O.semantic_bias(lg, spec.semantic_begin, spec.semantic_end, m.im_end_id, True)
        tok, st, mg = O.sample_token_margins(b, T, top_p, top_k, None, st)
        return tok, st, mg

    main, rng, mg = semantic(logits, rng)
    for t in range(frames):
        if not spec.semantic_begin <= main <= spec.semantic_end:
            raise RuntimeError(f"frame {t}: main token {main} outside the semantic range")
        codes[0, t] = min(main - spec.semantic_begin, spec.codebook_size - 1)
        draws.append([t, 0, int(main)] + [float(v) for v in mg])
        for cb in range(1, ncb):
            lg = m.fast_logits(hidden, codes[:cb, t].astype(np.uint32))
            tok, rng, mgf = O.sample_token_margins(lg, T, top_p, top_k, None, rng)
            codes[cb, t] = tok
            draws.append([t, cb, int(tok)] + [float(v) for v in mgf])
        step = np.zeros(ncb + 1, np.int32)
        step[0] = main
        step[1:] = codes[:, t]
        hidden, logits = m.eval(step)
        main, rng, mg = semantic(logits, rng)
    return hidden_prefill, codes, rng, draws


def run_config(name, model_dir, threads):
    c = CONFIGS[name]
    shape = synth.SHAPES[c["shape"]]
    t0 = time.time()
    path = synth.ensure_gguf(shape, model_dir, threads=threads)
    sha = sha256_file(path)
    print(f"[{name}] {os.path.basename(path)} sha256 {sha[:16]} ({time.time() - t0:.0f}s)", flush=True)
    m = O.OracleModel(path, c["max_seq"], shape.im_end_id, threads=threads)
    out = {
        "config": name, "what": c["what"], "shape": c["shape"], "gguf": os.path.basename(path), "gguf_sha256": sha,
        "im_end_id": shape.im_end_id, "max_seq": c["max_seq"], "frames": c["frames"],
        "temperature": c["sampler"][0], "top_p": c["sampler"][1], "top_k": c["sampler"][2],
        "min_tokens_before_end": NEVER_END, "n_requests": c.get("requests", 1),
        "prompt_recipe": list(c["prompt"]), "requests": [],
        "draw_fields": ["frame", "codebook", "token", "draw_margin", "cut_margin", "tie_margin"],
    }
    for b in c.get("oracle_requests", (0,)):
        prompt = prompt_for(shape, c["prompt"], b)
        rng0 = c["rng"] + b
        t0 = time.time()
        hidden, codes, rng, draws = oracle_generation(m, prompt, c["frames"], c["sampler"], rng0)
        print(f"[{name}] request {b}: {c['frames']} frames in {time.time() - t0:.0f}s; "
              f"min draw/cut margin {min(min(d[3], d[4]) for d in draws):.3g}, "
              f"min tie {min(d[5] for d in draws):.3g}", flush=True)
        out["requests"].append({
            "index": b, "prompt_tokens": len(prompt) // (shape.num_codebooks + 1), "prompt_sha256": prompt_sha(prompt),
            "rng_seed": rng0, "rng_state": int(rng), "hidden_prefill": [float(v) for v in hidden],
            "codes": codes.tolist(), "draws": draws,
        })
    m.close()
    os.makedirs(OUT, exist_ok=True)
    with open(os.path.join(OUT, f"{name}.json"), "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print(f"[{name}] wrote {os.path.join(OUT, name + '.json')}", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--configs", default="cfg2,cfg3,cfg4,cfg5")
    ap.add_argument("--model-dir", default=os.environ.get("S2HIP_MODEL_DIR", "/tmp/s2hip_models"))
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 1)
    args = ap.parse_args()
    for name in args.configs.split(","):
        run_config(name, args.model_dir, args.threads)


if __name__ == "__main__":
    main()
