"""Parity-dump schemas and the restated comparators (no GPU).

The comparator cases are the reference's own unit tests
(crates/fish_s2_parity/src/lib.rs:1971-2129) run against `s2hip.parity`, on
the JSON fixtures those tests hold (tests/golden/parity_dumps).
"""

import copy
import json
import os

import numpy as np
import pytest

import gguf_util
from s2hip import dumps, parity, synth
from s2hip.gguf import GGML_F16, GGML_F32, GGML_Q4_0, GGML_Q8_0, GgufFile, row_bytes

HERE = os.path.dirname(os.path.abspath(__file__))


def _fixture(name):
    with open(os.path.join(HERE, "golden", "parity_dumps", name)) as f:
        return json.load(f)


# -- compare_slow_ar_dumps (lib.rs:1971-2056) ----------------------------------
def test_identical_slow_ar_dumps_pass():
    d = _fixture("slow_ar_single.json")
    r = parity.compare_slow_ar_dumps(d, d)
    assert r.passed and not r.failures
    assert len(r.tensor_deltas) == 7 and r.tensor_deltas[0].name == "token0.normalized"


def test_slow_ar_tensor_delta_failure():
    e = _fixture("slow_ar_single.json")
    a = copy.deepcopy(e)
    a["query"]["l2"] += 0.1
    r = parity.compare_slow_ar_dumps(e, a)
    assert not r.passed and any("token0.query.l2" in f for f in r.failures)


def test_slow_ar_sequence_dumps():
    e = _fixture("slow_ar_sequence.json")
    a = copy.deepcopy(e)
    a["sequence"][1]["hidden"]["l2"] += 0.1
    r = parity.compare_slow_ar_dumps(e, a)
    assert not r.passed and len(r.tensor_deltas) == 14
    assert any("token1.hidden.l2" in f for f in r.failures)


def test_slow_ar_full_block_dumps():
    e = _fixture("slow_ar_full_block.json")
    a = copy.deepcopy(e)
    a["block_hidden"]["l2"] += 0.1
    r = parity.compare_slow_ar_dumps(e, a)
    assert not r.passed and len(r.tensor_deltas) == 13
    assert any("token0.block_hidden.l2" in f for f in r.failures)


def test_slow_ar_layer_count_mismatch():
    e = _fixture("slow_ar_full_block.json")
    e["layer_count"] = 2
    a = copy.deepcopy(e)
    a["layer_count"] = 3
    r = parity.compare_slow_ar_dumps(e, a)
    assert not r.passed and any("layer_count mismatch" in f for f in r.failures)


def test_full_stack_tolerance_only_for_36_layers():
    e = _fixture("slow_ar_full_block.json")
    e["layer_count"] = 36
    a = copy.deepcopy(e)
    a["block_hidden"]["max_abs"] += 0.9
    assert parity.compare_slow_ar_dumps(e, a).passed
    e["layer_count"] = a["layer_count"] = 2
    r = parity.compare_slow_ar_dumps(e, a)
    assert not r.passed and any("token0.block_hidden.max_abs" in f for f in r.failures)


def test_slow_ar_logits_and_top_logits_checks():
    e = _fixture("slow_ar_single.json")
    e["logits"] = {"len": 3, "l2": 10.0, "mean_abs": 2.0, "max_abs": 5.0, "first8": [1.0, 2.0, 5.0]}
    e["top_logits"] = [{"token_id": 2, "value": 5.0}, {"token_id": 1, "value": 2.0}]
    a = copy.deepcopy(e)
    a["logits"]["l2"] += 2.0  # the logits bound on l2 is 2.5
    assert parity.compare_slow_ar_dumps(e, a).passed
    a["top_logits"][1]["token_id"] = 0
    r = parity.compare_slow_ar_dumps(e, a)
    assert not r.passed and any("top_logits[1].token_id" in f for f in r.failures)
    del a["logits"]
    r = parity.compare_slow_ar_dumps(e, a)
    assert any("logits missing from actual dump" in f for f in r.failures)


# -- loop-level dumps (lib.rs:2057-2113) ----------------------------------------
FAST = {"backend": "rust", "text": "hi", "temperature": 0.0, "top_p": 1.0, "top_k": 0,
        "min_tokens_before_end": 0, "prompt_cols": 42, "main_token_id": 155666,
        "slow_hidden": [0.1, -0.2, 0.3], "codebook_ids": [100, 200, 300]}
SEMANTIC = {"backend": "rust", "text": "hi", "temperature": 0.0, "top_p": 1.0, "top_k": 0,
            "max_new_tokens": 4, "min_tokens_before_end": 0, "prompt_cols": 42,
            "main_token_ids": [151678, 151679]}
CODES = {"backend": "rust", "text": "hi", "temperature": 0.0, "top_p": 1.0, "top_k": 0,
         "max_new_tokens": 2, "min_tokens_before_end": 0, "prompt_cols": 42, "num_codebooks": 2,
         "n_frames": 2, "codes": [10, 11, 20, 21]}


def test_loop_dumps_exact_match():
    assert parity.compare_fast_ar_frame_dumps(FAST, FAST).passed
    assert parity.compare_semantic_token_dumps(SEMANTIC, SEMANTIC).passed
    assert parity.compare_generated_codes_dumps(CODES, CODES).passed


def test_loop_dump_mismatches():
    a = dict(CODES, codes=[10, 11, 20, 22])
    assert any("codes mismatch" in f for f in parity.compare_generated_codes_dumps(CODES, a).failures)
    a = dict(CODES, n_frames=3)
    r = parity.compare_generated_codes_dumps(CODES, a)
    assert any("n_frames mismatch" in f for f in r.failures)
    assert any("actual codes length 4 does not match" in f for f in r.failures)
    a = dict(FAST, slow_hidden=[0.1, -0.2, 0.3 + 0.011])
    assert any("slow_hidden mismatch" in f for f in parity.compare_fast_ar_frame_dumps(FAST, a).failures)
    a = dict(FAST, slow_hidden=[0.1, -0.2, 0.309])  # within max_abs 1e-2
    assert parity.compare_fast_ar_frame_dumps(FAST, a).passed
    a = dict(SEMANTIC, temperature=0.5)
    assert any("temperature mismatch" in f for f in parity.compare_semantic_token_dumps(SEMANTIC, a).failures)


def test_parity_cli(tmp_path, capsys):
    p = tmp_path / "a.json"
    p.write_text(json.dumps(CODES))
    assert parity.main(["compare-generated-codes", str(p), str(p)]) == 0
    assert "passed=true" in capsys.readouterr().out
    q = tmp_path / "b.json"
    q.write_text(json.dumps(dict(CODES, codes=[1, 2, 3, 4])))
    assert parity.main(["compare-generated-codes", str(p), str(q)]) == 1
    assert parity.main(["compare-nothing", str(p), str(q)]) == 2


# -- dump contents -----------------------------------------------------------------
def test_tensor_stats_definition():
    s = dumps.tensor_stats([3.0, -4.0])
    assert s == {"len": 2, "l2": 5.0, "mean_abs": 3.5, "max_abs": 4.0, "first8": [3.0, -4.0]}
    assert dumps.tensor_stats([]) == {"len": 0, "l2": 0.0, "mean_abs": 0.0, "max_abs": 0.0, "first8": []}
    # sequential f32 sums: each 0.5625 added to 2^24 rounds away (a pairwise
    # or multi-accumulator sum would keep 7.875 of them)
    s = dumps.tensor_stats([4096.0] + [0.75] * 15)
    assert s["l2"] == 4096.0 and s["max_abs"] == 4096.0 and len(s["first8"]) == 8
    # f32 values are written with their shortest f32 repr
    assert json.dumps(dumps.tensor_stats([0.1])["first8"]) == "[0.1]"


def test_top_logits_order():
    t = dumps.top_logits([1.0, 5.0, 5.0, -2.0, 3.0], 4)
    assert [x["token_id"] for x in t] == [1, 2, 4, 0]


def test_hidden_fixture():
    h = dumps.hidden_fixture(8, 2)
    assert h[0] == 1.0 and h[1] == 1.5 and h[7] == 0.5 and not h[2:7].any()


class FakeEngine:
    """Stands in for s2hip.Engine in the host-side dump loops: the logits
    put im_end first, then a scripted semantic id; the sampler is argmax
    over the candidates it is given and counts its calls in the RNG state."""

    spec = {"semantic_begin": 10, "semantic_end": 19, "vocab": 32, "codebook_size": 10,
            "num_codebooks": 2, "dim": 4}
    im_end_id = 5
    codebook_dim = 3

    def __init__(self, script):
        self.script, self.calls, self.steps, self.n_past = list(script), 0, [], 0

    def reset(self):
        self.n_past = 0

    def eval(self, flat):
        flat = np.asarray(flat).ravel()
        self.n_past += flat.size // self.codebook_dim
        if self.n_past > flat.size // self.codebook_dim:
            self.steps.append(flat.tolist())
        logits = np.full(32, -1.0, np.float32)
        logits[self.script[min(self.calls, len(self.script) - 1)]] = 2.0
        logits[self.im_end_id] = 3.0
        self.calls += 1
        return np.arange(4, dtype=np.float32) / 3, logits

    step = eval

    def sample(self, sub, temperature, top_p, top_k, force, rng):
        return int(np.argmax(sub)), rng + 1

    def fast_codebooks(self, hidden, code, temperature, top_p, top_k, rng):
        return np.array([code, 7], np.uint32), rng + 1

    def generate_codes(self, flat, max_new, temperature, top_p, top_k, min_before_end, rng):
        return {"codes": np.array([[1, 2], [3, 4]]), "n_frames": 2, "rng_state": rng}


def test_semantic_dump_loop_blocks_im_end_then_stops():
    """generate.rs:56-114: im_end is masked while generated_after_prefill
    (n_past - prompt_cols + tokens so far - 1: 0, 1, 3, ...) is below
    min_tokens_before_end; each step feeds [main, semantic code, 0]."""
    e = FakeEngine([12, 13, 14])
    d = dumps.semantic_token_dump(e, np.zeros(6, np.int32), max_new_tokens=8, min_tokens_before_end=3)
    assert d["main_token_ids"] == [12, 13, 5] and d["prompt_cols"] == 2
    assert e.steps == [[12, 2, 0], [13, 3, 0]]
    assert list(d) == ["backend", "text", "temperature", "top_p", "top_k", "max_new_tokens",
                       "min_tokens_before_end", "prompt_cols", "main_token_ids"]
    d = dumps.semantic_token_dump(FakeEngine([12]), np.zeros(6, np.int32), max_new_tokens=2,
                                  min_tokens_before_end=100)
    assert d["main_token_ids"] == [12, 12, 12]  # max_new_tokens steps, then stop


def test_loop_dump_fields_follow_reference_structs():
    """serde writes struct fields in declaration order
    (fish_s2_codes_dump.rs:10-26, fish_s2_fast_ar_dump.rs:10-22)."""
    e = FakeEngine([12])
    d = dumps.generated_codes_dump(e, np.zeros(6, np.int32), prompt_text="ref", prompt_code_cols=4)
    assert list(d) == ["backend", "prompt_text", "prompt_code_cols", "text", "temperature", "top_p", "top_k",
                       "max_new_tokens", "min_tokens_before_end", "prompt_cols", "num_codebooks", "n_frames",
                       "codes"]
    assert d["codes"] == [1, 2, 3, 4] and d["backend"] == "rust-hip"
    d = dumps.fast_ar_frame_dump(FakeEngine([13]), np.zeros(6, np.int32), min_tokens_before_end=1)
    assert list(d) == ["backend", "text", "temperature", "top_p", "top_k", "min_tokens_before_end", "prompt_cols",
                       "main_token_id", "slow_hidden", "codebook_ids"]
    assert d["main_token_id"] == 13 and d["codebook_ids"] == [3, 7]
    with pytest.raises(Exception, match="multiple"):
        dumps.generated_codes_dump(e, np.zeros(5, np.int32))


# -- GGUF reader ----------------------------------------------------------------------
def test_gguf_reader_roundtrip(tmp_path):
    path = str(tmp_path / "t.gguf")
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    b = (np.arange(8, dtype=np.float32) / 3).astype(np.float16)
    gguf_util.write(path, [("x.count", gguf_util.U32, 7), ("x.name", gguf_util.STR, "tiny"),
                           ("x.eps", gguf_util.F32, 1e-6)],
                    [("a", [4, 3], a), ("b", [8], b)])
    g = GgufFile(path)
    assert g.metadata["x.count"] == 7 and g.metadata["x.name"] == "tiny"
    ta, tb = g.tensor("a"), g.tensor("b")
    assert ta.dims == [4, 3] and ta.ggml_type == GGML_F32 and ta.rows == 3 and ta.row_len == 4
    assert np.array_equal(ta.f32(), a.ravel())
    assert tb.ggml_type == GGML_F16 and np.array_equal(tb.f32(), b.astype(np.float32))
    with pytest.raises(KeyError):
        g.tensor("missing")
    g.close()


def test_gguf_reader_on_synthetic_model(tiny_gguf):
    g = GgufFile(tiny_gguf)
    sh = synth.TINY
    w = g.tensor("layers.0.attention.wqkv.weight")
    q, kv = sh.heads * sh.head_dim, sh.kv_heads * sh.head_dim
    assert w.dims == [sh.dim, q + 2 * kv] and w.data.size == (q + 2 * kv) * sh.dim * 2
    assert g.tensor("embeddings.weight").rows == sh.vocab
    assert g.tensor("layers.0.attention_norm.weight").f32().shape == (sh.dim,)
    assert row_bytes(GGML_Q8_0, 64) == 68 and row_bytes(GGML_Q4_0, 64) == 36
    with pytest.raises(ValueError):
        row_bytes(GGML_Q8_0, 40)
    g.close()


# -- codec-stage dumps (fish_s2_parity lib.rs:268-403, 564-707, 855-1122) ---------------

def _stage_dump(kind, prefix, **over):
    d = {"backend": "rust", "text": "hi", "num_codebooks": 10}
    if kind in ("rvq", "post"):
        dim = "latent_dim" if kind == "rvq" else "hidden_dim"
        d.update({"n_frames": 2, dim: 1024, f"{prefix}_len": 2048})
    elif kind == "decode":
        d.update({"input_frames": 2, "output_frames": 8, "hidden_dim": 1024, "hidden_len": 8192})
    else:
        d.update({"input_frames": 2, "latent_frames": 8, "sample_rate": 44100, "num_samples": 4096})
    d.update({f"{prefix}_l2": 10.0, f"{prefix}_mean_abs": 0.25, f"{prefix}_max_abs": 1.5,
              f"{prefix}_first8": [0.1 * i for i in range(8)]})
    d.update(over)
    return d


STAGES = [("rvq", "latent", parity.compare_rvq_lookup_dumps, parity.RVQ_LOOKUP_TOLERANCE),
          ("post", "hidden", parity.compare_post_module_dumps, parity.POST_MODULE_TOLERANCE),
          ("decode", "hidden", parity.compare_decode_stage_dumps, parity.DECODE_STAGE_TOLERANCE),
          ("wave", "samples", parity.compare_waveform_dumps, parity.WAVEFORM_TOLERANCE)]


@pytest.mark.parametrize("kind,prefix,fn,tol", STAGES)
def test_codec_stage_comparators(kind, prefix, fn, tol):
    e = _stage_dump(kind, prefix)
    r = fn(e, copy.deepcopy(e))
    assert r.passed and r.failures == []
    # each statistic just inside, then just past its tolerance (the reference's texts)
    for key, limit, label in ((f"{prefix}_l2", tol.max_l2_delta, f"{prefix}_l2 delta"),
                              (f"{prefix}_mean_abs", tol.max_mean_abs_delta, f"{prefix}_mean_abs delta"),
                              (f"{prefix}_max_abs", tol.max_max_abs_delta, f"{prefix}_max_abs delta")):
        assert fn(e, _stage_dump(kind, prefix, **{key: e[key] + 0.9 * limit})).passed
        r = fn(e, _stage_dump(kind, prefix, **{key: e[key] + 1.5 * limit}))
        assert not r.passed and r.failures == [f"{label} {1.5 * limit:.8f} exceeds {limit:.8f}"], r.failures
    f8 = [x + 2 * tol.max_first8_mae for x in e[f"{prefix}_first8"]]
    r = fn(e, _stage_dump(kind, prefix, **{f"{prefix}_first8": f8}))
    assert r.failures == [f"{prefix}_first8 MAE {2 * tol.max_first8_mae:.8f} exceeds {tol.max_first8_mae:.8f}"]
    r = fn(e, _stage_dump(kind, prefix, text="hello"))
    assert r.failures == ['text mismatch: expected Some("hi"), actual Some("hello")']
    r = fn(e, _stage_dump(kind, prefix, num_codebooks=9))
    assert r.failures == ["num_codebooks mismatch: expected 10, actual 9"]


def test_codec_stage_length_and_sample_checks():
    e = _stage_dump("rvq", "latent")
    r = parity.compare_rvq_lookup_dumps(e, _stage_dump("rvq", "latent", latent_len=2047))
    assert r.failures == ["latent_len mismatch: expected 2048, actual 2047",
                          "actual latent_len 2047 does not match n_frames*latent_dim 2048"]
    e = _stage_dump("decode", "hidden")
    r = parity.compare_decode_stage_dumps(e, _stage_dump("decode", "hidden", output_frames=9))
    assert "output_frames mismatch: expected 8, actual 9" in r.failures
    assert "actual hidden_len 8192 does not match output_frames*hidden_dim 9216" in r.failures
    e = _stage_dump("wave", "samples")
    r = parity.compare_waveform_dumps(e, _stage_dump("wave", "samples", num_samples=4095))
    assert r.failures == ["num_samples delta 1 exceeds 0"]
    # latent_frames is not compared (serde default field in the reference)
    assert parity.compare_waveform_dumps(e, _stage_dump("wave", "samples", latent_frames=0)).passed


def test_codec_stage_stats_definition():
    v = np.array([3.0, -4.0, 0.5, 1e-3, -2.5, 7.0, 0.0, 1.0, 9.0], np.float32)
    s = dumps.f64_stats("x", v)
    x = v.astype(np.float64)
    assert s["x_l2"] == pytest.approx(np.sqrt(np.sum(x * x)), rel=1e-15)
    assert s["x_mean_abs"] == pytest.approx(np.mean(np.abs(x)), rel=1e-15)
    assert s["x_max_abs"] == 9.0 and s["x_first8"] == [float(a) for a in x[:8]]
    assert dumps.f64_stats("y", np.zeros(0, np.float32)) == {"y_l2": 0.0, "y_mean_abs": 0.0, "y_max_abs": 0.0,
                                                             "y_first8": []}


def test_codec_stage_cli(tmp_path, capsys):
    e = _stage_dump("wave", "samples")
    a = _stage_dump("wave", "samples", samples_max_abs=1.9)
    pe, pa = tmp_path / "e.json", tmp_path / "a.json"
    pe.write_text(json.dumps(e))
    pa.write_text(json.dumps(a))
    assert parity.main(["compare-waveform", str(pe), str(pe)]) == 0
    assert "samples_l2_delta=0.00000000" in capsys.readouterr().out
    assert parity.main(["compare-waveform", str(pe), str(pa)]) == 1
    out = capsys.readouterr()
    assert "failure=samples_max_abs delta 0.40000000 exceeds 0.20000000" in out.out
    assert "waveform parity failed" in out.err


# -- WAV output and WAV parity (wav.rs:7-39; fish_s2_parity lib.rs:1712-1944) --------------

def test_pcm_to_wav_layout_and_reference_roundtrip():
    from s2hip import wav
    samples = np.array([-1.0, -0.25, 0.0, 0.25, 0.999], np.float32)  # wav.rs:201-210
    b = wav.pcm_to_wav(samples, 44100)
    assert len(b) == 44 + 10 and b[:4] == b"RIFF" and b[8:16] == b"WAVEfmt " and b[36:40] == b"data"
    riff, fmt_size, fmt, ch, sr, br, ba, bits, dsz = (
        *np.frombuffer(b[4:8], "<u4"), *np.frombuffer(b[16:20], "<u4"), *np.frombuffer(b[20:24], "<u2"),
        *np.frombuffer(b[24:32], "<u4"), *np.frombuffer(b[32:36], "<u2"), *np.frombuffer(b[40:44], "<u4"))
    assert (riff, fmt_size, fmt, ch, sr, br, ba, bits, dsz) == (54, 16, 1, 1, 44100, 88200, 2, 16, 10)
    pcm = np.frombuffer(b[44:], "<i2")
    # clamp, x 32767 in f32, truncation toward zero
    assert pcm.tolist() == [-32767, -8191, 0, 8191, 32734]
    decoded = pcm / 32768.0
    assert np.all(np.abs(decoded - samples) <= 2.0 / 32768.0)
    assert np.frombuffer(wav.pcm_to_wav(np.array([3.0, -7.0], np.float32), 8000)[44:], "<i2").tolist() == [32767, -32767]


def test_wav_metrics_reference_cases():
    from s2hip import wav

    def pcm16(values, rate):
        return wav.pcm_to_wav(np.zeros(0, np.float32), rate)[:40] + np.uint32(2 * len(values)).tobytes() + \
            np.asarray(values, "<i2").tobytes()

    m = wav.metrics_from_wav_bytes(pcm16([0, 16384, -16384, 0], 24000))  # lib.rs:1950-1958
    assert (m.sample_rate, m.channels, m.bits_per_sample) == (24000, 1, 16)
    assert abs(m.duration_seconds - 4 / 24000) < 1e-6 and 0.35 < m.rms < 0.36
    a = wav.metrics_from_wav_bytes(pcm16([0] * 24000, 24000))  # lib.rs:1960-1967
    b = wav.metrics_from_wav_bytes(pcm16([0] * 12000, 24000))
    r = wav.compare_metrics(a, b)
    assert not r.passed and r.failures == ["duration delta 0.5000s exceeds 0.1000s"]
    assert wav.compare_metrics(a, a).passed
    with pytest.raises(wav.WavError, match="not a RIFF/WAVE file"):
        wav.metrics_from_wav_bytes(b"RIFX" + bytes(40))
    with pytest.raises(wav.WavError, match="WAV contains no samples"):
        wav.metrics_from_wav_bytes(pcm16([], 24000))
    # envelope: 50 ms frames of RMS, compared after resampling both to a common length
    x = np.concatenate([np.full(1200, 8000, np.int16), np.zeros(1200, np.int16)])
    m = wav.metrics_from_wav_bytes(pcm16(x, 24000))
    assert len(m.envelope_rms) == 2 and abs(m.envelope_rms[0] - 8000 / 32768) < 1e-12 and m.envelope_rms[1] == 0
    assert wav.envelope_mae([1.0, 0.0], [1.0, 0.5, 0.0]) == pytest.approx(0.0)


def test_wav_parity_cli(tmp_path, capsys):
    from s2hip import wav
    p = tmp_path / "a.wav"
    p.write_bytes(wav.pcm_to_wav(np.sin(np.arange(4410, dtype=np.float32) / 7.0) * 0.5, 44100))
    assert parity.main(["metrics", str(p)]) == 0
    out = capsys.readouterr().out
    assert "sample_rate=44100" in out and "duration_seconds=0.100000" in out and "envelope_frames=2" in out
    assert parity.main(["compare", str(p), str(p)]) == 0
    assert "passed=true" in capsys.readouterr().out
