"""Batched decode: several generate_codes requests in one engine call.

Each request owns a KV slot; every frame kernel runs once for the whole batch
(weights read once per step).  The reference has no batch API (one
SlowArState), so the oracle runs each request alone with generate_codes
(generate.rs:117-221): per request, greedy codes and the final RNG state must
be bit-exact, and sampled trajectories are checked draw by draw (teacher
forcing) as for single requests.
"""

import numpy as np
import pytest

from conftest import make_prompt
from loop_util import assert_draws_match, teacher_forced_mismatches
from oracle import oracle as O
from s2hip import synth

pytestmark = pytest.mark.gpu



def _engine(path, max_seq=96, im_end=None, graph=True):
    from s2hip import Engine

    return Engine(path, max_seq, synth.TINY.im_end_id if im_end is None else im_end, use_graph=graph)


def _oracle(path, max_seq=96, im_end=None):
    return O.OracleModel(path, max_seq, synth.TINY.im_end_id if im_end is None else im_end)


def _prompts(n, seed, lengths=None):
    lengths = lengths or [8 + (7 * i) % 33 for i in range(n)]
    return [make_prompt(synth.TINY, lengths[i], seed=seed + i) for i in range(n)]


@pytest.mark.parametrize("nb", [1, 2, 3, 5, 9])
def test_batch_greedy_codes_match_oracle_per_request(tiny_gguf, nb):
    """nb = 1, 2: GEMV kernels; 3 and 5: skinny MFMA products; 9: the first
    Fast-AR pass has 18 columns, two skinny launches per linear."""
    prompts = _prompts(nb, seed=100 + nb)
    e, o = _engine(tiny_gguf), _oracle(tiny_gguf)
    rb = e.generate_codes_batch(prompts, 14, min_tokens_before_end=100, rng_states=list(range(nb)))
    assert rb["graph_used"] and rb["total_frames"] == 14 * nb
    for b, pr in enumerate(prompts):
        ro = o.generate_codes(pr, 14, 0.0, 1.0, 0, 100, b)
        got = rb["requests"][b]
        assert got["n_frames"] == ro["n_frames"] == 14
        assert np.array_equal(got["codes"], ro["codes"]), b
        assert got["rng_state"] == ro["rng_state"]


def test_batch_of_one_equals_single_call(tiny_gguf):
    prompt = make_prompt(synth.TINY, 20, seed=120)
    e = _engine(tiny_gguf)
    single = e.generate_codes(prompt, 10, 0.7, 0.9, 0, 100, 3)
    batch = e.generate_codes_batch([prompt], 10, 0.7, 0.9, 0, 100, [3])["requests"][0]
    assert np.array_equal(single["codes"], batch["codes"]) and single["rng_state"] == batch["rng_state"]


def test_batch_sampled_codes_match_oracle_teacher_forced(tiny_gguf):
    nb = 4
    prompts = _prompts(nb, seed=130)
    seeds = [11, 12, 13, 14]
    kw = dict(temperature=0.7, top_p=0.9, top_k=0, min_tokens_before_end=100)
    rg = _engine(tiny_gguf, graph=True).generate_codes_batch(prompts, 16, rng_states=seeds, **kw)
    rn = _engine(tiny_gguf, graph=False).generate_codes_batch(prompts, 16, rng_states=seeds, **kw)
    assert rg["graph_used"] and not rn["graph_used"]
    o = _oracle(tiny_gguf)
    for b in range(nb):
        g, n = rg["requests"][b], rn["requests"][b]
        # graph replay and direct launches run the same kernels
        assert np.array_equal(g["codes"], n["codes"]) and g["rng_state"] == n["rng_state"]
        assert g["n_frames"] == 16
        mism, total = teacher_forced_mismatches(o, prompts[b], g["codes"], 16, 0.7, 0.9, 0, 100, seeds[b],
                                                synth.TINY.im_end_id)
        assert_draws_match(mism, total, 160)


def test_batch_requests_stop_independently(tiny_gguf):
    """im_end chosen from request 0's greedy trajectory: request 0 stops
    early while the others run on (or stop at their own frame)."""
    prompts = _prompts(4, seed=140)
    o = _oracle(tiny_gguf)
    ref = o.generate_codes(prompts[0], 12, 0.0, 1.0, 0, 0, 0)
    stop_id = synth.TINY.semantic_begin + int(ref["codes"][0, 5])
    e2, o2 = _engine(tiny_gguf, im_end=stop_id), _oracle(tiny_gguf, im_end=stop_id)
    for mtbe in (0, 3):
        rb = e2.generate_codes_batch(prompts, 12, min_tokens_before_end=mtbe, rng_states=[0, 1, 2, 3])
        frames = []
        for b, pr in enumerate(prompts):
            ro = o2.generate_codes(pr, 12, 0.0, 1.0, 0, mtbe, b)
            got = rb["requests"][b]
            assert got["n_frames"] == ro["n_frames"], (b, mtbe)
            assert np.array_equal(got["codes"], ro["codes"]) and got["rng_state"] == ro["rng_state"]
            frames.append(got["n_frames"])
        assert frames[0] < 12
        assert rb["total_frames"] == sum(frames)


@pytest.mark.parametrize("which", ["q8", "q4"])
def test_batch_quantized_greedy_codes(request, which):
    path = request.getfixturevalue(f"tiny_{which}_gguf")
    prompts = _prompts(4, seed=150)
    e, o = _engine(path), _oracle(path)
    rb = e.generate_codes_batch(prompts, 12, min_tokens_before_end=100)
    for b, pr in enumerate(prompts):
        ro = o.generate_codes(pr, 12, 0.0, 1.0, 0, 100, 0)
        assert np.array_equal(rb["requests"][b]["codes"], ro["codes"]), b


def test_batch_errors_and_recovery(tiny_gguf):
    from s2hip import S2HipError

    e = _engine(tiny_gguf, max_seq=40)
    ok = make_prompt(synth.TINY, 8, seed=160)
    with pytest.raises(S2HipError, match="requests"):
        e.generate_codes_batch([ok] * 17, 4)
    # request 2 runs out of KV positions (30 + 16 > 40)
    long = make_prompt(synth.TINY, 30, seed=161)
    with pytest.raises(S2HipError, match=r"KV cache overflow \(request 2\)"):
        e.generate_codes_batch([ok, ok, long], 16, min_tokens_before_end=100)
    bad = ok.copy()
    bad[0] = synth.TINY.vocab + 1
    with pytest.raises(S2HipError, match="out of range"):
        e.generate_codes_batch([ok, bad], 4)
    # the engine still works, in batches and alone
    r = e.generate_codes_batch([ok, ok], 4, min_tokens_before_end=100)
    assert [q["n_frames"] for q in r["requests"]] == [4, 4]
    assert np.array_equal(r["requests"][0]["codes"], r["requests"][1]["codes"])
    assert e.generate_codes(ok, 4, min_tokens_before_end=100)["n_frames"] == 4


def test_batch_kv_f16_greedy_codes_match_oracle(tiny_gguf):
    from s2hip import Engine

    prompts = _prompts(3, seed=170)
    e = Engine(tiny_gguf, 96, synth.TINY.im_end_id, kv_f16=True)
    o = O.OracleModel(tiny_gguf, 96, synth.TINY.im_end_id, flags=O.KV_F16)
    rb = e.generate_codes_batch(prompts, 12, min_tokens_before_end=100)
    for b, pr in enumerate(prompts):
        ro = o.generate_codes(pr, 12, 0.0, 1.0, 0, 100, 0)
        assert np.array_equal(rb["requests"][b]["codes"], ro["codes"]), b


def test_batch_with_an_outlier_channel_matches_oracle(model_dir, tmp_path):
    """SwiGLU output channel 300 of every layer is ~1e4-1e5 times the others
    (rows 300 of w1 and w3 scaled by 300): it lies past the first 256
    elements of its wave's k range in the batched w2 product, beyond the
    per-wave scale's headroom.  The call then runs again on the per-column
    paths (whole-row scale) and every request's greedy codes match the
    oracle."""
    import shutil

    import gguf_util

    src = synth.ensure_gguf(synth.TINY, model_dir)
    path = str(tmp_path / "tiny_outlier.gguf")
    shutil.copyfile(src, path)
    for pre, n in (("layers", synth.TINY.slow_layers), ("fast_layers", synth.TINY.fast_layers)):
        for l in range(n):
            for w in ("w1", "w3"):
                gguf_util.scale_rows(path, f"{pre}.{l}.feed_forward.{w}.weight", [300], 300.0)
    prompts = _prompts(3, seed=150)
    e, o = _engine(path), _oracle(path)
    rb = e.generate_codes_batch(prompts, 12, min_tokens_before_end=100, rng_states=[0, 1, 2])
    assert rb["per_column_rerun"]
    for b, pr in enumerate(prompts):
        ro = o.generate_codes(pr, 12, 0.0, 1.0, 0, 100, b)
        got = rb["requests"][b]
        assert got["n_frames"] == ro["n_frames"] == 12
        assert np.array_equal(got["codes"], ro["codes"]), b
    # the engine keeps working on the batched product afterwards
    rb2 = e.generate_codes_batch(prompts[:2], 4, min_tokens_before_end=100, rng_states=[0, 1])
    for b in range(2):
        ro = o.generate_codes(prompts[b], 4, 0.0, 1.0, 0, 100, b)
        assert np.array_equal(rb2["requests"][b]["codes"], ro["codes"]), b


def test_batch_with_large_norm_gains_matches_oracle(model_dir):
    """Every Slow and Fast linear of a 3-request batch runs the batched MFMA
    product; with RMSNorm gains of 100 the raw residual times the gain reaches
    ~1e6-1e7, which the per-wave power-of-two scale brings into the f16 hi / lo
    split's range, and codes stay bit-exact."""
    path = synth.ensure_gguf(synth.TINY.with_(norm_gain=100.0), model_dir)
    prompts = _prompts(3, seed=140)
    e, o = _engine(path), _oracle(path)
    rb = e.generate_codes_batch(prompts, 12, min_tokens_before_end=100, rng_states=[0, 1, 2])
    for b, pr in enumerate(prompts):
        ro = o.generate_codes(pr, 12, 0.0, 1.0, 0, 100, b)
        got = rb["requests"][b]
        assert got["n_frames"] == ro["n_frames"] == 12
        assert np.array_equal(got["codes"], ro["codes"]), b
