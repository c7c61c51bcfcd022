"""Parity dumps written from the GPU path against the same dumps built from
the oracle, judged by the restated comparators (`s2hip.parity`, after
crates/fish_s2_parity/src/lib.rs) and, for the per-op Slow-AR statistics,
also by a tighter 1e-4 relative bound.

The oracle side restates the reference's dump loops here: generate_codes,
generate_semantic_tokens (generate.rs:56-114) and
generate_fast_ar_first_frame (generate.rs:224-271) with the semantic mask
applied to the full vocabulary (sampling.rs:54-100), and the Slow-AR block
(slow_ar.rs:558-617,980-1039) on the oracle's per-op functions.
"""

import json

import numpy as np
import pytest

from conftest import make_prompt
from oracle import oracle as O
from s2hip import dumps, parity, synth
from s2hip.gguf import GgufFile

pytestmark = pytest.mark.gpu

IM_END = synth.TINY.im_end_id


def _engine(path, max_seq=96):
    from s2hip import Engine

    return Engine(path, max_seq, IM_END)


def _oracle(path, max_seq=96):
    return O.OracleModel(path, max_seq, IM_END)


def _masked_sample(om, logits, gap, mtbe, T, top_p, top_k, rng):
    """sample_semantic_token over the full vocabulary (generate.rs:284-298)."""
    s = om.spec
    l = np.full(s.vocab, -np.inf, np.float32)
    l[s.semantic_begin:s.semantic_end + 1] = logits[s.semantic_begin:s.semantic_end + 1]
    block = gap < mtbe
    if not block:
        l[IM_END] = logits[IM_END]
    return O.sample_token(l, T, top_p, top_k, None if block else IM_END, rng)


def _oracle_semantic_dump(om, prompt, max_new, T, top_p, top_k, mtbe, seed):
    s = om.spec
    width = s.num_codebooks + 1
    cols = prompt.size // width
    om.reset()
    _, logits = om.eval(prompt)
    main, rng = _masked_sample(om, logits, 0, mtbe, T, top_p, top_k, seed)
    tokens, generated = [main], 0
    while main != IM_END and generated < max_new:
        step = np.zeros(width, np.int32)
        step[0] = main
        if s.semantic_begin <= main <= s.semantic_end:
            step[1] = main - s.semantic_begin
        _, logits = om.eval(step)
        generated += 1
        gap = max(om.n_past - cols, 0) + len(tokens) - 1
        main, rng = _masked_sample(om, logits, gap, mtbe, T, top_p, top_k, rng)
        tokens.append(main)
    return {"backend": "oracle", "text": "hi", "temperature": T, "top_p": top_p, "top_k": top_k,
            "max_new_tokens": max_new, "min_tokens_before_end": mtbe, "prompt_cols": cols,
            "main_token_ids": tokens}


def _oracle_fast_frame_dump(om, prompt, T, top_p, top_k, mtbe, seed):
    s = om.spec
    om.reset()
    hidden, logits = om.eval(prompt)
    main, rng = _masked_sample(om, logits, 0, mtbe, T, top_p, top_k, seed)
    code = min(main - s.semantic_begin, s.codebook_size - 1) if s.semantic_begin <= main <= s.semantic_end else 0
    codes, _ = om.fast_codebooks(hidden, code, T, top_p, top_k, rng)
    return {"backend": "oracle", "text": "hi", "temperature": T, "top_p": top_p, "top_k": top_k,
            "min_tokens_before_end": mtbe, "prompt_cols": prompt.size // (s.num_codebooks + 1),
            "main_token_id": main, "slow_hidden": [float(x) for x in hidden],
            "codebook_ids": [int(c) for c in codes]}


def _oracle_codes_dump(om, prompt, max_new, T, top_p, top_k, mtbe, seed):
    r = om.generate_codes(prompt, max_new, T, top_p, top_k, mtbe, seed)
    s = om.spec
    return {"backend": "oracle", "text": "hi", "temperature": T, "top_p": top_p, "top_k": top_k,
            "max_new_tokens": max_new, "min_tokens_before_end": mtbe,
            "prompt_cols": prompt.size // (s.num_codebooks + 1), "num_codebooks": s.num_codebooks,
            "n_frames": r["n_frames"], "codes": [int(c) for c in r["codes"].ravel()]}


@pytest.mark.parametrize("mtbe", [100, 0])
def test_generated_codes_dump_matches_oracle(tiny_gguf, mtbe):
    prompt = make_prompt(synth.TINY, 24, seed=200)
    e, om = _engine(tiny_gguf), _oracle(tiny_gguf)
    got = dumps.generated_codes_dump(e, prompt, max_new_tokens=6, min_tokens_before_end=mtbe)
    ref = _oracle_codes_dump(om, prompt, 6, 0.0, 1.0, 0, mtbe, 0)
    r = parity.compare_generated_codes_dumps(ref, got)
    assert r.passed, r.failures


@pytest.mark.parametrize("T,top_p,top_k,seed", [(0.0, 1.0, 0, 0), (0.7, 0.9, 0, 5), (1.0, 1.0, 30, 11)])
def test_semantic_token_dump_matches_oracle(tiny_gguf, T, top_p, top_k, seed):
    prompt = make_prompt(synth.TINY, 20, seed=210)
    e, om = _engine(tiny_gguf), _oracle(tiny_gguf)
    got = dumps.semantic_token_dump(e, prompt, max_new_tokens=6, temperature=T, top_p=top_p, top_k=top_k,
                                    min_tokens_before_end=2, seed=seed)
    ref = _oracle_semantic_dump(om, prompt, 6, T, top_p, top_k, 2, seed)
    r = parity.compare_semantic_token_dumps(ref, got)
    assert r.passed, r.failures
    assert len(got["main_token_ids"]) >= 2


@pytest.mark.parametrize("T,top_p,seed", [(0.0, 1.0, 0), (0.7, 0.9, 3)])
def test_fast_ar_frame_dump_matches_oracle(tiny_gguf, T, top_p, seed):
    prompt = make_prompt(synth.TINY, 16, seed=220)
    e, om = _engine(tiny_gguf), _oracle(tiny_gguf)
    got = dumps.fast_ar_frame_dump(e, prompt, temperature=T, top_p=top_p, min_tokens_before_end=1, seed=seed)
    ref = _oracle_fast_frame_dump(om, prompt, T, top_p, 0, 1, seed)
    r = parity.compare_fast_ar_frame_dumps(ref, got)
    assert r.passed, r.failures
    assert len(got["codebook_ids"]) == synth.TINY.num_codebooks


class OracleOps:
    """slow_ar_dump's primitives on the oracle (test side only)."""

    def rms_norm(self, x, w, eps):
        return O.rms_norm(x, w, eps)

    def linear(self, w_raw, ggml_type, in_dim, out_dim, x):
        return O.linear(x, w_raw, ggml_type, in_dim, out_dim)

    def qk_rope(self, qkv, heads, kv_heads, head_dim, position, base, q_norm, k_norm, eps):
        q = qkv[:heads * head_dim]
        k = qkv[heads * head_dim:(heads + kv_heads) * head_dim]
        v = qkv[(heads + kv_heads) * head_dim:].copy()
        if q_norm is not None:
            q = O.rms_norm_heads(q, q_norm, head_dim, eps)
        if k_norm is not None:
            k = O.rms_norm_heads(k, k_norm, head_dim, eps)
        return O.rope_normal(q, head_dim, position, base), O.rope_normal(k, head_dim, position, base), v

    def attention(self, q, keys, values, heads, kv_heads, head_dim, tokens, scale):
        return O.gqa_attention(q, keys, values, heads, kv_heads, head_dim, tokens, float(scale))

    def swiglu(self, gate, up):
        return O.swiglu(gate, up, False)


def _stats_close(a, b, rtol):
    for k in ("l2", "mean_abs", "max_abs"):
        assert abs(a[k] - b[k]) <= rtol * max(1e-6, abs(b[k])), (k, a[k], b[k])
    scale = max(1e-6, max(abs(x) for x in b["first8"]) if b["first8"] else 1.0)
    assert all(abs(x - y) <= rtol * scale for x, y in zip(a["first8"], b["first8"]))


@pytest.mark.parametrize("which", ["f16", "q8"])
def test_slow_ar_dump_matches_oracle(request, which):
    path = request.getfixturevalue("tiny_gguf" if which == "f16" else "tiny_q8_gguf")
    e = _engine(path)
    g = GgufFile(path)
    kw = dict(layer=1, layers=2, position=3, tokens=3, logits=True, top_k=8)
    got = dumps.slow_ar_dump(dumps.EngineOps(e), g, e.spec, "tiny.gguf", **kw)
    ref = dumps.slow_ar_dump(OracleOps(), g, e.spec, "tiny.gguf", **kw)
    r = parity.compare_slow_ar_dumps(ref, got)
    assert r.passed, r.failures
    assert len(r.tensor_deltas) == 3 * 13 + 2
    assert [t["token_id"] for t in got["top_logits"]] == [t["token_id"] for t in ref["top_logits"]]
    for i in range(3):
        for name in dumps._TOKEN_FIELDS:
            _stats_close(got["sequence"][i][name], ref["sequence"][i][name], 1e-4)
    _stats_close(got["logits"], ref["logits"], 1e-4)
    g.close()


def test_dump_and_parity_command_lines(tiny_gguf, tmp_path, capsys):
    prompt = make_prompt(synth.TINY, 12, seed=230)
    pf = tmp_path / "prompt.json"
    pf.write_text(json.dumps({"flat_time_major": [int(x) for x in prompt]}))
    out = tmp_path / "codes_hip.json"
    assert dumps.main(["codes", "--transformer", tiny_gguf, "--prompt-ids", str(pf), "--output", str(out),
                       "--im-end-id", str(IM_END), "--max-new-tokens", "3", "--min-tokens-before-end", "100"]) == 0
    ref = tmp_path / "codes_oracle.json"
    ref.write_text(json.dumps(_oracle_codes_dump(_oracle(tiny_gguf), prompt, 3, 0.0, 1.0, 0, 100, 0)))
    assert parity.main(["compare-generated-codes", str(ref), str(out)]) == 0
    slow = tmp_path / "slow.json"
    assert dumps.main(["slow-ar", "--transformer", tiny_gguf, "--output", str(slow), "--tokens", "2",
                       "--logits"]) == 0
    d = json.loads(slow.read_text())
    assert d["token_count"] == 2 and len(d["sequence"]) == 2 and len(d["top_logits"]) == 8
    assert parity.main(["compare-slow-ar", str(slow), str(slow)]) == 0
    assert "passed=true" in capsys.readouterr().out


def test_semantic_sample_keeps_the_reference_masked_tail(tiny_gguf):
    """sample_discrete's fall-through (sampling.rs:227-241) returns the last
    entry of the reference's list, which is a masked id when the top-p loop
    runs past the finite candidates: the dump sampler must return that id too.
    The RNG state is chosen so the draw target is the largest one (0.99999988),
    and the cases where the oracle falls through are checked along with
    ordinary ones."""
    from s2hip import Engine
    from s2hip.dumps import semantic_sample

    sp = synth.TINY
    a = 6364136223846793005
    s0 = ((0xFFFFFFFFFFFFF800 - 1) * pow(a, -1, 1 << 64)) % (1 << 64)  # next unit value 1 - 2^-53
    rng = np.random.default_rng(1)
    fall = 0
    with Engine(tiny_gguf, 64, sp.im_end_id) as e:
        for trial in range(240):
            logits = (rng.standard_normal(sp.vocab) * rng.uniform(0.5, 3)).astype(np.float32)
            block = trial % 2 == 0
            st = s0 if trial % 3 else int(rng.integers(1, 1 << 62))
            lg = O.semantic_bias(logits, sp.semantic_begin, sp.semantic_end, sp.im_end_id, block)
            want = O.sample_token(lg, 1.0, 1.0, 0, None if block else sp.im_end_id, st)
            got = semantic_sample(e, logits, 0 if block else 10, 5, 1.0, 1.0, 0, st)
            assert got == want, (trial, got, want)
            fall += not (sp.semantic_begin <= want[0] <= sp.semantic_end or want[0] == sp.im_end_id)
    assert fall >= 3
