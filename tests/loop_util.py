"""Teacher-forced replay of a generated code trajectory on the oracle.

A seeded sampled trajectory is chaotic: one draw that lands within ~1e-6 of
a probability boundary changes every later frame, and f32 sums in another
order (GPU reductions vs the reference's sequential sums) move boundaries by
that much.  So sampled trajectories are checked draw by draw: the oracle
re-derives every draw of the GPU trajectory from the GPU's own previous
codes and the RNG state at that draw (each sample consumes exactly one LCG
step, sampling.rs:120-241), as generate_codes (generate.rs:117-221) and
generate_codebooks_for_semantic (fast_ar.rs:440-470) order them.
"""

import numpy as np

from oracle import oracle as O


# A draw may differ from the oracle's only where the oracle's own sampler
# puts it within reordering noise of a boundary (GPU logits follow the
# oracle's to ~1e-5 relative; the exp and the sequential sums are bit-exact):
# the draw target within BOUNDARY_EPS of a cumulative-probability boundary
# around the chosen item, the top-p sums within BOUNDARY_EPS of top_p at the
# cut, or the chosen logit within TIE_EPS (relative) of a neighbour's.
BOUNDARY_EPS = 1e-4
TIE_EPS = 1e-4


def at_boundary(logit, margins):
    draw, cut, tie = margins
    return min(draw, cut) < BOUNDARY_EPS or tie < TIE_EPS * max(1.0, abs(logit))


def _semantic_draw(logits, spec, im_end, generated, min_tokens_before_end, T, top_p, top_k, rng):
    """sample_semantic_token (generate.rs:284-298) on the oracle sampler, with
    the oracle's semantic bias (sampling.rs:54-100).  Returns (token, rng,
    margins, chosen logit)."""
    block = generated < min_tokens_before_end
    lg = O.semantic_bias(logits, spec.semantic_begin, spec.semantic_end, im_end, block)
    tok, rng, mg = O.sample_token_margins(lg, T, top_p, top_k, None if block else im_end, rng)
    return tok, rng, mg, float(lg[tok])


def teacher_forced_mismatches(oracle, prompt, codes, n_frames, temperature, top_p, top_k,
                              min_tokens_before_end, rng_state, im_end):
    """Returns (mismatching draws, total draws) of a codebook-major
    [num_codebooks][n_frames] trajectory; each mismatch is (frame, codebook,
    oracle token, gpu token, oracle margins, at_boundary)."""
    spec = oracle.spec
    ncb = spec.num_codebooks
    cols = len(prompt) // (ncb + 1)
    oracle.reset()
    hidden, logits = oracle.eval(prompt)
    rng = rng_state
    main, rng, mg, lv = _semantic_draw(logits, spec, im_end, 0, min_tokens_before_end, temperature, top_p,
                                       top_k, rng)
    mism = []
    total = 0
    for t in range(n_frames):
        gpu_main = spec.semantic_begin + int(codes[0, t])
        total += 1
        if main != gpu_main:
            mism.append((t, 0, main, gpu_main, mg, at_boundary(lv, mg)))
        for cb in range(1, ncb):
            lg = oracle.fast_logits(hidden, codes[:cb, t].astype(np.uint32))
            tok, rng, mgf = O.sample_token_margins(lg, temperature, top_p, top_k, None, rng)
            total += 1
            if tok != int(codes[cb, t]):
                mism.append((t, cb, tok, int(codes[cb, t]), mgf, at_boundary(float(lg[tok]), mgf)))
        step_in = np.zeros(ncb + 1, np.int32)
        step_in[0] = gpu_main
        step_in[1:] = codes[:, t]
        hidden, logits = oracle.eval(step_in)
        generated = (oracle.n_past - cols) + (t + 1)
        main, rng, mg, lv = _semantic_draw(logits, spec, im_end, generated, min_tokens_before_end, temperature,
                                           top_p, top_k, rng)
    return mism, total


def assert_draws_match(mism, total, expected_total):
    """Every mismatching draw must sit at a boundary of the oracle's own
    probabilities (see BOUNDARY_EPS); otherwise the samplers disagree."""
    assert total == expected_total, (total, expected_total)
    off = [m for m in mism if not m[5]]
    assert not off, off[:5]
