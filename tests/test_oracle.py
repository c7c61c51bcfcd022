"""Pins the CPU oracle (oracle/s2_oracle.cpp) before it is trusted as the checker.

Sources of truth, in order:
* the reference's own known-answer tests (values copied from its #[test]s);
* closed forms / textbook routines (IEEE half via numpy, sequential f32 sums
  via np.add.accumulate, float64 softmax attention, the LCG in Python ints);
* invariants the reference itself asserts (decode == prefill, Fast-AR
  recompute == incremental).
"""

import math
import os

import numpy as np
import pytest

from oracle import oracle as O
import gguf_util
from conftest import make_prompt
from s2hip import synth


# ---------------------------------------------------------------- f16 ----
def test_f16_decode_kat():
    # crates/fish_s2_infer/src/tensor.rs:339-345
    assert [O.f16_to_f32(b) for b in (0x3C00, 0xC000, 0x3800, 0x4400)] == [1.0, -2.0, 0.5, 4.0]


def test_f16_round_kat():
    # tensor.rs:356-364
    for v in (1.0, -2.0, 0.5):
        assert O.f16_to_f32(O.f32_to_f16(v)) == v
    assert O.f32_to_f16(float("inf")) == 0x7C00
    assert O.f32_to_f16(float("-inf")) == 0xFC00
    assert O.f32_to_f16(float("nan")) & 0x7C00 == 0x7C00


def test_f16_decode_exhaustive_matches_ieee():
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(int(b)) for b in bits], np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(want))


def test_f16_round_matches_numpy_rne():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 0.02,
        (rng.standard_normal(5000) * 1e-6).astype(np.float32),  # f16 subnormals
        rng.uniform(-70000, 70000, 5000).astype(np.float32),    # overflow region
        np.array([65504, 65519.99, 65520, 2.0 ** -25, 2.0 ** -24, 1.5 * 2.0 ** -24], np.float32),
    ])
    want = x.astype(np.float16).view(np.uint16)
    got = np.array([O.f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, want)


# --------------------------------------------------------- Q blocks ------
def _q8_block(d, q):
    return np.frombuffer(np.float16(d).tobytes(), np.uint8).tobytes() + np.asarray(q, np.int8).tobytes()


def _q4_block(d, nib):
    nib = np.asarray(nib, np.uint8)
    qs = (nib[:16] | (nib[16:] << 4)).astype(np.uint8)
    return np.frombuffer(np.float16(d).tobytes(), np.uint8).tobytes() + qs.tobytes()


def test_q8_0_dequant_closed_form():
    rng = np.random.default_rng(1)
    raw, want = b"", []
    for _ in range(8):
        d = np.float16(rng.uniform(-0.01, 0.01))
        q = rng.integers(-128, 128, 32)
        raw += _q8_block(d, q)
        want.append(np.float32(d) * q.astype(np.float32))
    got = O.dequant_row(raw, 8, 256)
    assert np.array_equal(got, np.concatenate(want).astype(np.float32))


def test_q4_0_dequant_closed_form():
    rng = np.random.default_rng(2)
    raw, want = b"", []
    for _ in range(8):
        d = np.float16(rng.uniform(-0.01, 0.01))
        nib = rng.integers(0, 16, 32)
        raw += _q4_block(d, nib)
        want.append(np.float32(d) * (nib.astype(np.float32) - 8.0))
    got = O.dequant_row(raw, 2, 256)
    assert np.array_equal(got, np.concatenate(want).astype(np.float32))


# ------------------------------------------------------------- ops -------
def test_rms_norm_kat():
    # tensor.rs:366-371
    out = O.rms_norm([1.0, 2.0, 3.0, 4.0], [1.0, 0.5, 2.0, -1.0], 1e-6)
    s = np.float32(1.0) / np.sqrt(np.float32(7.5) + np.float32(1e-6))
    np.testing.assert_allclose(out, [s, s, 6 * s, -4 * s], atol=1e-6)


def test_rms_norm_sequential_order():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(2560).astype(np.float32)
    w = rng.standard_normal(2560).astype(np.float32)
    ss = np.add.accumulate(x * x, dtype=np.float32)[-1]
    scale = np.float32(1.0) / np.sqrt(ss / np.float32(2560) + np.float32(1e-6))
    assert np.array_equal(O.rms_norm(x, w, 1e-6), (x * scale) * w)


def test_linear_kat_f32_and_f16():
    # backend.rs:208-215 and tensor.rs:373-391 ([out][in] layout)
    w = np.array([1, 2, 3, 4, 5, 6], np.float32)
    assert np.array_equal(O.linear([2.0, -1.0], w.view(np.uint8), 0, 2, 3), [0.0, 2.0, 4.0])
    assert np.array_equal(O.linear([2.0, -1.0], w.astype(np.float16).view(np.uint8), 1, 2, 3), [0.0, 2.0, 4.0])


@pytest.mark.parametrize("gtype", [1, 8, 2])
def test_linear_is_sequential_dot_over_dequantised_rows(gtype):
    rng = np.random.default_rng(4)
    in_dim, out_dim = 512, 48
    wf = (rng.standard_normal((out_dim, in_dim)) * 0.02).astype(np.float32)
    if gtype == 1:
        raw = wf.astype(np.float16).view(np.uint8).ravel()
    else:
        raw = np.frombuffer(b"".join(synth.quantize_block(gtype, blk) for blk in wf.reshape(-1, 32)), np.uint8)
    rows = O.dequant_row(raw.tobytes(), gtype, in_dim * out_dim).reshape(out_dim, in_dim)
    x = rng.standard_normal(in_dim).astype(np.float32)
    want = np.array([np.add.accumulate(x * r, dtype=np.float32)[-1] for r in rows], np.float32)
    assert np.array_equal(O.linear(x, raw, gtype, in_dim, out_dim), want)


def test_rope_kat():
    # crates/fish_s2_infer/src/attention.rs:337-343
    out = O.rope_normal([1.0, 0.0, 0.0, 1.0], 4, 1, 10000.0)
    np.testing.assert_allclose(out, [math.cos(1), math.sin(1), -math.sin(0.01), math.cos(0.01)], atol=1e-5)


def test_rope_closed_form_float64():
    rng = np.random.default_rng(5)
    hd, pos, base = 128, 37, 1.0e6
    v = rng.standard_normal(4 * hd).astype(np.float32)
    got = O.rope_normal(v, hd, pos, base)
    x = v.astype(np.float64).reshape(4, hd // 2, 2)
    th = pos / base ** (np.arange(0, hd, 2) / hd)
    want = np.stack([x[..., 0] * np.cos(th) - x[..., 1] * np.sin(th),
                     x[..., 0] * np.sin(th) + x[..., 1] * np.cos(th)], -1).ravel()
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5)


def test_gqa_attention_kat():
    # attention.rs:362-406
    q = [1.0, 0.0, 0.0, 1.0, 1.0, 0.0, 0.0, 1.0]
    k = [1.0, 0.0, 0.0, 1.0, 0.0, 1.0, 1.0, 0.0]
    v = [10.0, 0.0, 0.0, 10.0, 20.0, 0.0, 0.0, 20.0]
    out = O.gqa_attention(q, k, v, 4, 2, 2, 2, 1.0)
    ph = math.e / (math.e + 1)
    pl = 1 - ph
    np.testing.assert_allclose(out, [10 * ph + 20 * pl, 0, 10 * pl + 20 * ph, 0, 0, 10 * pl + 20 * ph, 0,
                                     10 * ph + 20 * pl], atol=1e-5)


def test_cached_attention_kat():
    # attention.rs:408-428
    out = O.gqa_attention([1.0, 0.0, 0.0, 1.0], [1.0, 0.0, 0.0, 1.0], [2.0, 0.0, 4.0, 0.0], 2, 1, 2, 2, 1.0)
    ph = math.e / (math.e + 1)
    pl = 1 - ph
    np.testing.assert_allclose(out, [2 * ph + 4 * pl, 0, 2 * pl + 4 * ph, 0], atol=1e-5)


def test_attention_matches_float64_softmax():
    rng = np.random.default_rng(6)
    H, Hkv, hd, T = 8, 2, 64, 37
    q = rng.standard_normal(H * hd).astype(np.float32)
    k = rng.standard_normal(T * Hkv * hd).astype(np.float32)
    v = rng.standard_normal(T * Hkv * hd).astype(np.float32)
    got = O.gqa_attention(q, k, v, H, Hkv, hd, T, 1 / math.sqrt(hd))
    q64, k64, v64 = q.reshape(H, hd), k.reshape(T, Hkv, hd), v.reshape(T, Hkv, hd)
    want = []
    for h in range(H):
        g = h // (H // Hkv)
        s = k64[:, g, :].astype(np.float64) @ q64[h] / math.sqrt(hd)
        p = np.exp(s - s.max())
        want.append((p / p.sum()) @ v64[:, g, :])
    np.testing.assert_allclose(got, np.concatenate(want), atol=1e-5)


def test_swiglu_kat_and_closed_form():
    # slow_ar.rs:1518-1521
    np.testing.assert_allclose(O.swiglu([0.0, 1.0], [2.0, 3.0]), [0.0, 3.0 / (1.0 + math.exp(-1.0))], atol=1e-6)
    rng = np.random.default_rng(7)
    g = rng.standard_normal(1000).astype(np.float32) * 4
    u = rng.standard_normal(1000).astype(np.float32)
    want = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    np.testing.assert_allclose(O.swiglu(g, u), want, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(O.swiglu(g, u, fast=True), want, rtol=1e-6, atol=1e-6)


# --------------------------------------------------------- sampling ------
def test_lcg_closed_form():
    # SeededRng (sampling.rs:34-52) in Python integers
    s = 42
    st = 42
    for _ in range(100):
        s = (s * 6364136223846793005 + 1) % (1 << 64)
        want = ((s >> 11) & ((1 << 53) - 1)) / float(1 << 53)
        got, st = O.next_unit(st)
        assert got == want and st == s


def test_sampler_kats():
    # sampling.rs:276-328
    assert O.sample_token([0.1, 5.0, 3.0, 2.0], 0.0, 1.0, 0, rng_state=1)[0] == 1
    assert O.sample_token([10.0, 9.0, 8.0, 0.0], 0.0, 1.0, 2, rng_state=99)[0] <= 1
    ninf = float("-inf")
    assert O.sample_token([ninf] * 4 + [5.0], 0.0, 1.0, 1, always_include=4, rng_state=1)[0] == 4
    a = O.sample_token([1.0, 3.0, 2.0, 0.5, 4.0], 0.8, 0.9, 3, rng_state=42)
    b = O.sample_token([1.0, 3.0, 2.0, 0.5, 4.0], 0.8, 0.9, 3, rng_state=42)
    assert a == b


def test_greedy_tie_uses_the_draw():
    # T=0 gives every value within 1e-6 of the max probability 1, so two
    # tied maxima are chosen by the draw: u < 0.5 -> first (lower id).
    for seed in range(20):
        u, _ = O.next_unit(seed)
        tok, st = O.sample_token([1.0, 5.0, 5.0, 2.0], 0.0, 1.0, 0, rng_state=seed)
        assert tok == (1 if u < 0.5 else 2)
        assert st == O.next_unit(seed)[1]


def test_sampler_frequencies_follow_softmax():
    logits = np.array([2.0, 1.0, 0.5, -1.0, 0.0], np.float32)
    T = 0.7
    p = np.exp((logits - logits.max()) / T)
    p /= p.sum()
    st = 7
    counts = np.zeros(5)
    n = 20000
    for _ in range(n):
        tok, st = O.sample_token(logits, T, 1.0, 0, rng_state=st)
        counts[tok] += 1
    np.testing.assert_allclose(counts / n, p, atol=0.015)


def test_top_p_truncates_the_tail():
    logits = np.array([3.0, 2.0, 1.0, 0.0, -1.0], np.float32)
    st = 11
    seen = set()
    for _ in range(2000):
        tok, st = O.sample_token(logits, 1.0, 0.5, 0, rng_state=st)
        seen.add(tok)
    # softmax(3,2,1,0,-1) = .636 .234 ..: top-p 0.5 keeps only the first item
    assert seen == {0}


def test_compact_and_transpose_kats():
    # generate.rs:410-415, prompt.rs:289-303
    assert O.compact_codes([10, 11, 0, 20, 21, 0], 2, 3, 2).tolist() == [10, 11, 20, 21]
    assert O.transpose_to_time_major([10, 20, 1, 2, 3, 4], 3, 2).tolist() == [10, 1, 3, 20, 2, 4]


# ----------------------------------------------------- model level -------
TOY_WQKV = [[1, 0, 0, 0], [0, 0, 0, 0], [0, 0, 0, 0], [1, 0, 0, 0], [1, 0, 0, 0], [0, 0, 0, 0], [3, 0, 0, 0],
            [0, 0, 0, 0]]
TOY_WO = [[1, 0, 0, 0], [0, 0, 2, 0], [0, 0, 0, 0], [0, 0, 0, 0]]


@pytest.fixture(scope="module")
def toy_gguf(tmp_path_factory):
    p = str(tmp_path_factory.mktemp("toy") / "toy.gguf")
    gguf_util.toy_dual_ar(p, TOY_WQKV, TOY_WO, [0.5, 1, 1, 1], [1 / math.sqrt(2)] * 2)
    return p


def test_toy_layer_decode_kat(toy_gguf):
    # slow_ar.rs:1283-1349: token [1,0,0,0] -> layer hidden [4,6,0,0]; the FFN
    # is zero, and eval returns the final-RMSNorm'd hidden (eps 0, gains 1).
    m = O.OracleModel(toy_gguf, 4, im_end_id=3)
    hidden, logits = m.eval([0, 0])
    np.testing.assert_allclose(hidden, np.array([4, 6, 0, 0]) / math.sqrt(13.0), atol=1e-6)
    np.testing.assert_allclose(logits, [hidden[0], hidden[0] + hidden[1], 0, 0], atol=1e-6)


def test_toy_decode_equals_prefill(toy_gguf):
    # slow_ar.rs:1455-1493: a two-token prefill equals two single-token steps
    a = O.OracleModel(toy_gguf, 4, im_end_id=3)
    h_pre, l_pre = a.eval([0, 0, 1, 0])
    b = O.OracleModel(toy_gguf, 4, im_end_id=3)
    b.eval([0, 0])
    h_dec, l_dec = b.eval([1, 0])
    assert np.array_equal(h_pre, h_dec) and np.array_equal(l_pre, l_dec)
    assert a.n_past == b.n_past == 2


def test_kv_overflow_and_bad_token_errors(toy_gguf):
    m = O.OracleModel(toy_gguf, 2, im_end_id=3)
    with pytest.raises(RuntimeError, match="KV cache overflow"):
        m.eval([0, 0, 1, 0, 0, 0])
    with pytest.raises(RuntimeError, match="out of range"):
        m.eval([9, 0])


def test_tiny_fast_incremental_equals_recompute(tiny_gguf):
    # Fast-AR without KV cache (fast_ar.rs:417-424) vs. the incremental form
    prompt = make_prompt(synth.TINY, 8, seed=3)
    inc = O.OracleModel(tiny_gguf, 64, synth.TINY.im_end_id)
    rec = O.OracleModel(tiny_gguf, 64, synth.TINY.im_end_id, flags=O.FAITHFUL_FAST_RECOMPUTE)
    h, _ = inc.eval(prompt)
    for T, top_p, seed in ((0.0, 1.0, 0), (0.7, 0.9, 5)):
        ci, si = inc.fast_codebooks(h, 17, T, top_p, 0, seed)
        cr, sr = rec.fast_codebooks(h, 17, T, top_p, 0, seed)
        assert np.array_equal(ci, cr) and si == sr
    # the logits themselves, bit for bit, at every prefix length
    rng = np.random.default_rng(8)
    for plen in range(synth.TINY.num_codebooks):
        prefix = rng.integers(0, synth.TINY.codebook_size, plen).tolist()
        li = np.asarray(inc.fast_logits(h, prefix), np.float32)
        lr = np.asarray(rec.fast_logits(h, prefix), np.float32)
        assert np.array_equal(li.view(np.uint32), lr.view(np.uint32)), plen


def test_tiny_faithful_modes_give_identical_codes(tiny_gguf):
    prompt = make_prompt(synth.TINY, 12, seed=4)
    fast = O.OracleModel(tiny_gguf, 64, synth.TINY.im_end_id)
    faithful = O.OracleModel(tiny_gguf, 64, synth.TINY.im_end_id,
                             flags=O.FAITHFUL_FAST_RECOMPUTE | O.FAITHFUL_SLOW_RELOAD)
    a = fast.generate_codes(prompt, 6, min_tokens_before_end=100)
    b = faithful.generate_codes(prompt, 6, min_tokens_before_end=100)
    assert np.array_equal(a["codes"], b["codes"]) and a["rng_state"] == b["rng_state"]
    assert a["n_frames"] == 6


def test_tiny_prefill_chunking_is_exact(tiny_gguf):
    # one 10-token prefill == 10 single-token evals (the decode path)
    prompt = make_prompt(synth.TINY, 10, seed=6)
    a = O.OracleModel(tiny_gguf, 64, synth.TINY.im_end_id)
    ha, la = a.eval(prompt)
    b = O.OracleModel(tiny_gguf, 64, synth.TINY.im_end_id)
    for t in range(10):
        hb, lb = b.eval(prompt[t * 11:(t + 1) * 11])
    assert np.array_equal(ha, hb) and np.array_equal(la, lb)


def test_kv_f16_mode_rounds_the_cache_only(tiny_gguf):
    """ORC_KV_F16: K and V are stored as their f16 roundings, so the hidden
    state moves by about f16 precision (nonzero, below 2e-2), and prefill
    chunking stays exact."""
    prompt = make_prompt(synth.TINY, 10, seed=6)
    a = O.OracleModel(tiny_gguf, 64, synth.TINY.im_end_id)
    f = O.OracleModel(tiny_gguf, 64, synth.TINY.im_end_id, flags=O.KV_F16)
    ha, _ = a.eval(prompt)
    hf, _ = f.eval(prompt)
    rel = float(np.max(np.abs(ha - hf)) / np.max(np.abs(ha)))
    assert 0 < rel < 2e-2
    b = O.OracleModel(tiny_gguf, 64, synth.TINY.im_end_id, flags=O.KV_F16)
    for t in range(10):
        hb, _ = b.eval(prompt[t * 11:(t + 1) * 11])
    assert np.array_equal(hf, hb)


def test_im_end_blocking_yields_exact_frame_count(tiny_gguf):
    prompt = make_prompt(synth.TINY, 8, seed=9)
    m = O.OracleModel(tiny_gguf, 64, synth.TINY.im_end_id)
    r = m.generate_codes(prompt, 5, min_tokens_before_end=10)
    assert r["n_frames"] == 5 and r["codes"].shape == (10, 5)
    # codebook 0 is the semantic code of each frame's main token
    assert (r["codes"] >= 0).all() and (r["codes"] < synth.TINY.codebook_size).all()


def test_teacher_forced_replay_of_oracle_trajectory_is_exact(tiny_gguf):
    """The draw-by-draw replay used for sampled GPU trajectories reproduces
    the oracle's own sampled trajectory with zero mismatches (same draw order
    and RNG steps as generate_codes)."""
    from loop_util import teacher_forced_mismatches

    o = O.OracleModel(tiny_gguf, 64, synth.TINY.im_end_id)
    prompt = make_prompt(synth.TINY, 16, seed=21)
    r = o.generate_codes(prompt, 8, temperature=0.7, top_p=0.9, top_k=0, min_tokens_before_end=4, rng_state=3)
    assert r["n_frames"] >= 1
    mism, total = teacher_forced_mismatches(o, prompt, r["codes"], r["n_frames"], 0.7, 0.9, 0, 4, 3,
                                            synth.TINY.im_end_id)
    assert mism == [] and total == 10 * r["n_frames"]
    # a planted wrong code is caught, and is not excused as a boundary draw
    bad = r["codes"].copy()
    bad[3, 0] = (bad[3, 0] + 1) % synth.TINY.codebook_size
    mism2, _ = teacher_forced_mismatches(o, prompt, bad, r["n_frames"], 0.7, 0.9, 0, 4, 3, synth.TINY.im_end_id)
    assert len(mism2) >= 1 and not all(m[5] for m in mism2)


# ------------------------------------------- hand-derived model KATs ------
def test_rms_norm_heads_kat():
    # rms_norm_heads_f32 (backend.rs:104-121): each head normalised on its own
    # with the shared per-head gain.  Head 0 = [3, 4]: ms 12.5; head 1 = [0, 2]:
    # ms 2; gain [1, 0.5], eps 0.
    got = O.rms_norm_heads(np.array([3, 4, 0, 2], np.float32), np.array([1, 0.5], np.float32), 2, 0.0)
    want = [3 / math.sqrt(12.5), 4 / math.sqrt(12.5) * 0.5, 0.0, 2 / math.sqrt(2.0) * 0.5]
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)
    # a whole-vector norm would give ms = 7.25 for every element
    assert abs(got[0] - 3 / math.sqrt(7.25)) > 1e-2


def test_semantic_mask_kats():
    # sampling.rs:248-274 (semantic_mask_leaves_only_allowed_ids_finite,
    # semantic_mask_can_block_im_end, apply_semantic_bias_zeros_disallowed_logits)
    m = O.semantic_bias([1.0, 2.0, 3.0, 4.0, 5.0], 1, 2, im_end=4, block_im_end=False)
    assert np.isneginf(m[0]) and m[1] == 2.0 and m[2] == 3.0 and np.isneginf(m[3]) and m[4] == 5.0
    m = O.semantic_bias([0.1, 0.2, 0.3, 0.4, 0.5], 1, 2, im_end=4, block_im_end=True)
    assert np.isneginf(m[4]) and np.isneginf(m[0]) and np.float32(m[1]) == np.float32(0.2)
    m = O.semantic_bias([0.1, 0.2, 0.3, 0.4, 0.5], 1, 2, im_end=4, block_im_end=False)
    assert np.isinf(m[0]) and m[1] == np.float32(0.2) and m[4] == np.float32(0.5)
    # None: nothing outside the semantic range survives
    m = O.semantic_bias([0.1, 0.2, 0.3, 0.4, 0.5], 1, 2)
    assert np.isneginf(m[[0, 3, 4]]).all() and np.isfinite(m[[1, 2]]).all()


@pytest.fixture(scope="module")
def embed_toy_gguf(tmp_path_factory):
    # width 4, vocab 8, semantic ids [4, 6], 2 codebooks of 3 codes; every
    # Slow-layer weight zero (the layer passes the embedding through), eps 1
    # so the final RMSNorm keeps the embedding's scale visible.
    emb = np.zeros((8, 4), np.float32)
    emb[0] = [2, 0, 0, 0]  # a text id
    emb[5] = [1, 0, 0, 0]  # a semantic id
    cb = np.zeros((6, 4), np.float32)
    cb[:, 1] = np.arange(6)  # codebook row r = [0, r, 0, 0]
    p = str(tmp_path_factory.mktemp("embtoy") / "embed_toy.gguf")
    gguf_util.toy_model(p, 4, 8, emb=emb, cb_emb=cb, eps=1.0, num_codebooks=2, codebook_size=3,
                        semantic=(4, 6))
    return p


def test_semantic_token_embedding_kat(embed_toy_gguf):
    # embed_slow_ar_time_major (slow_ar.rs:1041-1133) by hand: token [5 | 2, 1]
    # is semantic, so h = emb[5] + (cb[0*3 + 2] + cb[1*3 + 1]) = [1, 6, 0, 0],
    # scaled by 1/sqrt(2 + 1); final RMSNorm with eps 1: ms = 37/12, so
    # hidden = [1, 6, 0, 0] / sqrt(3) / sqrt(49/12) = [2/7, 12/7, 0, 0].
    m = O.OracleModel(embed_toy_gguf, 4, im_end_id=7)
    hidden, logits = m.eval([5, 2, 1])
    np.testing.assert_allclose(hidden, [2 / 7, 12 / 7, 0, 0], rtol=1e-6, atol=1e-7)
    # tied head: logits[i] = emb[i] . hidden
    np.testing.assert_allclose(logits, [4 / 7, 0, 0, 0, 0, 2 / 7, 0, 0], rtol=1e-6, atol=1e-7)
    # the embedding itself, before any layer: [1, 6, 0, 0] / sqrt(3) and [2, 0, 0, 0]
    np.testing.assert_allclose(m.embed([5, 2, 1, 0, 0, 0]), [[1 / math.sqrt(3), 6 / math.sqrt(3), 0, 0],
                                                             [2, 0, 0, 0]], rtol=1e-6)
    # a text id takes no codebook rows and no scale: [2, 0, 0, 0] / sqrt(1 + 1)
    m.reset()
    hidden, _ = m.eval([0, 2, 1])
    np.testing.assert_allclose(hidden, [math.sqrt(2), 0, 0, 0], rtol=1e-6)
    # the mistakes this pins: no cb * codebook_size offset would sum rows 2 and
    # 1 ([1, 3, 0, 0]); 1/sqrt(num_codebooks) would give [1, 6, 0, 0] / sqrt(45/4)
    assert abs(2 / 7 - 1 / math.sqrt(3) / math.sqrt(10 / 12 / 1 + 1)) > 1e-3
    assert abs(2 / 7 - 1 / math.sqrt(45 / 4)) > 1e-3


FAST_TOY = dict(
    # one Fast layer, width 4, 1 q head / 1 kv head of head_dim 4, FFN zero
    # (it passes through), Wo = I.  q[2] = 1.5 n[0]; k[2] = n[1]; v[0] = n[3],
    # v[1] = 0.5 n[0], where n is the RMS-normalised input (eps 0, gain 1).
    wqkv=[[0, 0, 0, 0], [0, 0, 0, 0], [1.5, 0, 0, 0], [0, 0, 0, 0],
          [0, 0, 0, 0], [0, 0, 0, 0], [0, 1, 0, 0], [0, 0, 0, 0],
          [0, 0, 0, 1], [0.5, 0, 0, 0], [0, 0, 0, 0], [0, 0, 0, 0]],
    fast_emb=[[1, 1, 1, 1], [2, 0, 0, 0], [0, 0, 0, 2], [0, 2, 0, 0]],
    out=[[1, 0, 0, 0], [0, 1, 0, 0], [0, 0, 1, 0], [1, 1, 0, 0]],
)


@pytest.fixture(scope="module")
def fast_toy_gguf(tmp_path_factory):
    # Fast RoPE base 4 (Slow: 1e6), so position 1 rotates the second pair of a
    # head_dim-4 head by 1 / 4^(2/4) = 0.5 rad
    p = str(tmp_path_factory.mktemp("fasttoy") / "fast_toy.gguf")
    gguf_util.toy_model(p, 4, 8, fast={"attention.wqkv.weight": FAST_TOY["wqkv"],
                                       "attention.wo.weight": np.eye(4)},
                        fast_emb=FAST_TOY["fast_emb"], fast_output=FAST_TOY["out"], num_codebooks=3,
                        codebook_size=4, semantic=(4, 7), fast_heads=(1, 1, 4), fast_rope_base=4.0,
                        rope_base=1e6)
    return p


def _fast_toy_logits(h):
    # fast_output . rmsnorm(h) with rows [1,0,0,0], [0,1,0,0], [0,0,1,0], [1,1,0,0]
    n = np.asarray(h, np.float64) / math.sqrt(float(np.mean(np.square(h))))
    return np.array([n[0], n[1], n[2], n[0] + n[1]])


@pytest.mark.parametrize("flags", [0, O.FAITHFUL_FAST_RECOMPUTE])
def test_fast_ar_toy_layer_kat(fast_toy_gguf, flags):
    """forward_codebook_prefix (fast_ar.rs:360-437) on a one-layer toy, derived
    by hand.  Slow hidden h0 = [1,1,1,1] (rms 1): q0 = [0,0,1.5,0], k0 =
    [0,0,1,0], v0 = [1,0.5,0,0]."""
    m = O.OracleModel(fast_toy_gguf, 4, im_end_id=7, flags=flags)
    h0 = np.ones(4, np.float32)
    # no prefix: one position attends to itself, out = h0 + v0 = [2, 1.5, 1, 1]
    np.testing.assert_allclose(m.fast_logits(h0, []), _fast_toy_logits([2, 1.5, 1, 1]), rtol=1e-6, atol=1e-6)
    # prefix [1]: position 1 holds fast_emb[1] = [2,0,0,0] (no codebook offset,
    # fast_ar.rs:396-401): q1 = [0,0,3,0] rotated at position 1 with the FAST
    # base 4 -> pair (2,3) = 3 (cos .5, sin .5); k1 = 0, v1 = [0,1,0,0]; no
    # QK-norm on the Fast path.  Scores (scale 1/sqrt(4)): s0 = 1.5 cos(.5),
    # s1 = 0 -> p0 = 1 / (1 + e^-s0); out = [2 + p0, 0.5 p0 + p1, 0, 0].
    s0 = 1.5 * math.cos(0.5)
    p0 = 1.0 / (1.0 + math.exp(-s0))
    p1 = 1.0 - p0
    want = _fast_toy_logits([2 + p0, 0.5 * p0 + p1, 0, 0])
    np.testing.assert_allclose(m.fast_logits(h0, [1]), want, rtol=1e-6, atol=1e-6)
    # prefix [1, 2]: position 2 holds fast_emb[2] = [0,0,0,2]: q2 = 0, so the
    # three causal positions get weight 1/3 each: attn = (v0 + v1 + v2) / 3 with
    # v2 = [2,0,0,0] -> [1, 0.5, 0, 0]; out = [1, 0.5, 0, 2]
    np.testing.assert_allclose(m.fast_logits(h0, [1, 2]), _fast_toy_logits([1, 0.5, 0, 2]), rtol=1e-6, atol=1e-6)
    # what the case at prefix [1] separates: a QK-norm'd Fast path (s0 = 2 cos .5)
    # and the Slow RoPE base (s0 = 1.5 cos 1e-3) both move the logits by > 1e-2
    for s_bad in (2 * math.cos(0.5), 1.5 * math.cos(1e-3)):
        pb = 1.0 / (1.0 + math.exp(-s_bad))
        assert np.abs(_fast_toy_logits([2 + pb, 0.5 * pb + 1 - pb, 0, 0]) - want).max() > 1e-2


def test_sampler_margins_kat():
    # two equal logits at T = 1: probabilities [0.5, 0.5]; the draw target t
    # (the LCG's first unit value) picks item 0 iff t < 0.5, and its margin is
    # the distance to 0 or 0.5 (or 0.5 and 1); top_p 1 never cuts before the end
    u, _ = O.next_unit(7)
    t = np.float32(u)
    tok, _, (draw, cut, tie) = O.sample_token_margins([1.0, 1.0], 1.0, 1.0, 0, None, 7)
    assert tok == (0 if t < 0.5 else 1)
    want = min(t, 0.5 - t) if t < 0.5 else min(t - 0.5, 1.0 - t)
    assert abs(draw - want) < 1e-7 and tie == 0.0
    assert abs(cut - 0.0) < 1e-7  # cumsum reaches exactly 1.0 = top_p at the last item
    # top_p 0.6 over [0.5, 0.5]: the cut falls after item 1 with sums 0.5 / 1.0
    _, _, (_, cut, _) = O.sample_token_margins([1.0, 1.0], 1.0, 0.6, 0, None, 7)
    assert abs(cut - 0.1) < 1e-6


# ------------------------------------------------- FFN sublayer KATs ------
# forward_feed_forward (Slow: slow_ar.rs:659-710, swiglu_split :1215-1232;
# Fast: fast_ar.rs:325-353, swiglu_split :472-485), derived by hand on d = 4,
# ffn = 2 toys whose attention sublayer is zero (wqkv = 0, so v = 0 and the
# attention adds nothing): the residual entering the FFN is the input x =
# [2, 2, 2, 2] (rms 2).  ffn_norm gains g = [0.5, 1, 2, 1.5], eps 0, so the
# normalised input is n = x / 2 * g = g exactly.
#   w1 rows [0, 0, -1.5, 0], [0, -2.5, 0, 0]  -> gate = [-3, -2.5]
#   w3 rows [2, 0, 0, 0],    [0, 2, 0, 0]     -> up   = [1, 2]
#   a_i = SwiGLU(gate_i, up_i)
#   w2 rows [1, 0], [0, 1], [1, 1], [0, 0]    -> proj = [a0, a1, a0 + a1, 0]
#   out = x + proj, then the final RMSNorm (gain 1, eps 0).
# Each planted mistake moves the output by far more than the 1e-6 tolerance:
# w1 <-> w3 (gate [1, 2], up [-3, -2.5]), ffn_norm dropped (n = x) or its
# gain dropped (n = [1, 1, 1, 1]), the FFN residual dropped (out[3] = 0).
# The Slow and Fast SwiGLU forms, g * sigmoid(g) * u and g / (1 + e^-g) * u,
# differ only in rounding; at gate -2.5, up 2 they differ by one f32 ulp, and
# the bit-level checks below see it in the output.
FFN_GAIN = [0.5, 1.0, 2.0, 1.5]
FFN_W1 = [[0, 0, -1.5, 0], [0, -2.5, 0, 0]]
FFN_W3 = [[2, 0, 0, 0], [0, 2, 0, 0]]
FFN_W2 = [[1, 0], [0, 1], [1, 1], [0, 0]]
FFN_X = [2.0, 2.0, 2.0, 2.0]


def _libm_expf():
    import ctypes
    import ctypes.util

    libm = ctypes.CDLL(ctypes.util.find_library("m") or "libm.so.6")
    fn = libm.expf
    fn.restype, fn.argtypes = ctypes.c_float, [ctypes.c_float]
    return lambda v: np.float32(fn(np.float32(v)))


def _ffn_closed_form():
    """float64: the toy's normalised output vector from the formulas above."""
    sig = lambda v: 1.0 / (1.0 + math.exp(-v))
    a0, a1 = -3.0 * sig(-3.0) * 1.0, -2.5 * sig(-2.5) * 2.0
    out = np.array([2 + a0, 2 + a1, 2 + a0 + a1, 2.0])
    return out / math.sqrt(float(np.mean(out * out)))


def _ffn_f32(fast_form):
    """The same toy in f32 with the reference's operation order: sequential
    sums (`Iterator::sum`, no fused multiply-add), RMSNorm as
    (x * (ms + eps).sqrt().recip()) * w (backend.rs:95-101), glibc expf (what
    Rust's f32::exp calls on Linux)."""
    f = np.float32
    expf = _libm_expf()

    def dot(x, w):
        s = f(0)
        for a, b in zip(x, w):
            s = f(s + f(f(a) * f(b)))
        return s

    def rms(x, w):
        ss = f(0)
        for v in x:
            ss = f(ss + f(v * v))
        sc = f(f(1) / f(np.sqrt(f(f(ss / f(len(x))) + f(0)))))
        return [f(f(v * sc) * f(g)) for v, g in zip(x, w)]

    def swiglu(g, u):
        if fast_form:  # fast_ar.rs:484
            return f(f(g / f(f(1) + expf(-g))) * u)
        return f(f(g * f(f(1) / f(f(1) + expf(-g)))) * u)  # slow_ar.rs:1229,1234

    x = [f(v) for v in FFN_X]
    n = rms(x, FFN_GAIN)
    act = [swiglu(dot(n, r1), dot(n, r3)) for r1, r3 in zip(FFN_W1, FFN_W3)]
    out = [f(a + dot(act, r)) for a, r in zip(x, FFN_W2)]
    return np.array(rms(out, [1.0] * 4), np.float32)


def _ffn_layer(**extra):
    return {"ffn_norm.weight": FFN_GAIN, "feed_forward.w1.weight": FFN_W1,
            "feed_forward.w3.weight": FFN_W3, "feed_forward.w2.weight": FFN_W2, **extra}


def test_swiglu_rounding_orders_bit_exact():
    # gate -2.5, up 2: the Slow form rounds g * sigmoid(g) first, the Fast form
    # g / (1 + e^-g); the two f32 results differ by one ulp here, and -3 / 1 too
    f = np.float32
    expf = _libm_expf()
    g = np.array([-2.5, -3.0], np.float32)
    u = np.array([2.0, 1.0], np.float32)
    slow = np.array([f(f(a * f(f(1) / f(f(1) + expf(-a)))) * b) for a, b in zip(g, u)], np.float32)
    fast = np.array([f(f(a / f(f(1) + expf(-a))) * b) for a, b in zip(g, u)], np.float32)
    assert (slow.view(np.uint32) != fast.view(np.uint32)).all()
    assert np.array_equal(np.asarray(O.swiglu(g, u), np.float32).view(np.uint32), slow.view(np.uint32))
    assert np.array_equal(np.asarray(O.swiglu(g, u, fast=True), np.float32).view(np.uint32), fast.view(np.uint32))


@pytest.fixture(scope="module")
def ffn_toy_gguf(tmp_path_factory):
    # token 0 embeds to x; rows 1..4 of the tied head are unit vectors, so
    # logits[1..4] read the hidden state back; no QK-norm (q = k = 0)
    emb = np.zeros((8, 4), np.float32)
    emb[0] = FFN_X
    emb[1:5] = np.eye(4)
    p = str(tmp_path_factory.mktemp("ffntoy") / "ffn_toy.gguf")
    gguf_util.toy_model(p, 4, 8, slow=_ffn_layer(), emb=emb, qk_norm=False, semantic=(3, 6),
                        codebook_size=4, fast=_ffn_layer(), fast_output=np.eye(4), fast_ffn=2)
    return p


def test_slow_ffn_sublayer_kat(ffn_toy_gguf):
    m = O.OracleModel(ffn_toy_gguf, 4, im_end_id=7)
    hidden, logits = m.eval([0, 0])
    want = _ffn_closed_form()
    np.testing.assert_allclose(hidden, want, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(logits, [2 * want.sum(), *want, 0, 0, 0], rtol=1e-6, atol=1e-6)
    # the Slow rounding order, bit for bit; the Fast form gives other bits
    bits = _ffn_f32(fast_form=False).view(np.uint32)
    assert np.array_equal(hidden.view(np.uint32), bits)
    assert not np.array_equal(_ffn_f32(fast_form=True).view(np.uint32), bits)


@pytest.mark.parametrize("flags", [0, O.FAITHFUL_FAST_RECOMPUTE])
def test_fast_ffn_sublayer_kat(ffn_toy_gguf, flags):
    # fast_logits with no prefix: the one position is the Slow hidden x;
    # logits = fast_output . rmsnorm(out) with unit-vector rows
    m = O.OracleModel(ffn_toy_gguf, 4, im_end_id=7, flags=flags)
    logits = np.asarray(m.fast_logits(np.asarray(FFN_X, np.float32), []), np.float32)
    np.testing.assert_allclose(logits, _ffn_closed_form(), rtol=1e-6, atol=1e-6)
    bits = _ffn_f32(fast_form=True).view(np.uint32)
    assert np.array_equal(logits.view(np.uint32), bits)
    assert not np.array_equal(_ffn_f32(fast_form=False).view(np.uint32), bits)
