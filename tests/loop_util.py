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


def _semantic_draw(logits, spec, im_end, generated, min_tokens_before_end, T, top_p, top_k, rng):
    """sample_semantic_token (generate.rs:284-298) on the oracle sampler."""
    lg = np.full_like(logits, -np.inf)
    lo, hi = spec.semantic_begin, spec.semantic_end
    lg[lo:hi + 1] = logits[lo:hi + 1]
    block = generated < min_tokens_before_end
    if not block and im_end < lg.size:
        lg[im_end] = logits[im_end]
    return O.sample_token(lg, T, top_p, top_k, None if block else im_end, rng)


def teacher_forced_mismatches(oracle, prompt, codes, n_frames, temperature, top_p, top_k,
                              min_tokens_before_end, rng_state, im_end):
    """Returns (mismatching draws, total draws) of a codebook-major
    [num_codebooks][n_frames] trajectory."""
    spec = oracle.spec
    ncb = spec.num_codebooks
    cols = len(prompt) // (ncb + 1)
    oracle.reset()
    hidden, logits = oracle.eval(prompt)
    rng = rng_state
    main, rng = _semantic_draw(logits, spec, im_end, 0, min_tokens_before_end, temperature, top_p, top_k, rng)
    mism = total = 0
    for t in range(n_frames):
        gpu_main = spec.semantic_begin + int(codes[0, t])
        total += 1
        mism += int(main != gpu_main)
        for cb in range(1, ncb):
            lg = oracle.fast_logits(hidden, codes[:cb, t].astype(np.uint32))
            tok, rng = O.sample_token(lg, temperature, top_p, top_k, None, rng)
            total += 1
            mism += int(tok != int(codes[cb, t]))
        step_in = np.zeros(ncb + 1, np.int32)
        step_in[0] = gpu_main
        step_in[1:] = codes[:, t]
        hidden, logits = oracle.eval(step_in)
        generated = (oracle.n_past - cols) + (t + 1)
        main, rng = _semantic_draw(logits, spec, im_end, generated, min_tokens_before_end, temperature, top_p,
                                   top_k, rng)
    return mism, total
