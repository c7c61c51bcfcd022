"""The reference's dump comparators, restated (crates/fish_s2_parity/src/lib.rs).

Same checks, tolerances and failure texts as compare_generated_codes_dumps
(:709-804), compare_fast_ar_frame_dumps (:1211-1289),
compare_semantic_token_dumps (:1291-1348), compare_slow_ar_dumps
(:1365-1710) and the codec-stage comparators compare_rvq_lookup_dumps
(:855-941), compare_post_module_dumps (:943-1029),
compare_decode_stage_dumps (:1031-1122) and compare_waveform_dumps
(:626-707), over the JSON files that `s2hip.dumps` and the reference's dump
tools write.  Command line as `fish_s2_parity`'s subcommands:

    python -m s2hip.parity compare-generated-codes expected.json actual.json
    python -m s2hip.parity compare-semantic-tokens expected.json actual.json
    python -m s2hip.parity compare-fast-ar-frame expected.json actual.json
    python -m s2hip.parity compare-slow-ar expected.json actual.json
    python -m s2hip.parity compare-rvq-lookup expected.json actual.json
    python -m s2hip.parity compare-post-module expected.json actual.json
    python -m s2hip.parity compare-decode-stage expected.json actual.json
    python -m s2hip.parity compare-waveform expected.json actual.json
    python -m s2hip.parity metrics file.wav
    python -m s2hip.parity compare golden.wav candidate.wav
"""

import json
import math
import sys
from dataclasses import dataclass, field, replace
from typing import List, Optional


@dataclass
class Report:
    passed: bool
    failures: List[str]
    tensor_deltas: list = field(default_factory=list)


@dataclass(frozen=True)
class SlowArTensorTolerance:
    """SlowArTensorTolerance::default (lib.rs:155-172)."""
    max_l2_delta: float = 6e-2
    max_mean_abs_delta: float = 5e-4
    max_max_abs_delta: float = 1.5e-2
    max_first8_mae: float = 8e-4


@dataclass
class TensorDelta:
    name: str
    l2_delta: float
    mean_abs_delta: float
    max_abs_delta: float
    first8_mae: float


def _f32(x) -> float:
    """f32 fields compare after an f32 round trip, as serde reads them."""
    import numpy as np
    return float(np.float32(x))


def _meta(failures, name, expected, actual, close=False):
    if close:
        if abs(_f32(expected) - _f32(actual)) > 1e-6:
            failures.append(f"{name} mismatch: expected {expected}, actual {actual}")
    elif expected != actual:
        failures.append(f"{name} mismatch: expected {expected!r}, actual {actual!r}")


def compare_generated_codes_dumps(expected: dict, actual: dict) -> Report:
    f = []
    _meta(f, "text", expected["text"], actual["text"])
    _meta(f, "prompt_text", expected.get("prompt_text"), actual.get("prompt_text"))
    _meta(f, "prompt_code_cols", expected.get("prompt_code_cols"), actual.get("prompt_code_cols"))
    _meta(f, "temperature", expected["temperature"], actual["temperature"], close=True)
    _meta(f, "top_p", expected["top_p"], actual["top_p"], close=True)
    for k in ("top_k", "max_new_tokens", "min_tokens_before_end", "prompt_cols", "num_codebooks", "n_frames"):
        _meta(f, k, expected[k], actual[k])
    for side, d in (("expected", expected), ("actual", actual)):
        n = d["num_codebooks"] * d["n_frames"]
        if len(d["codes"]) != n:
            f.append(f"{side} codes length {len(d['codes'])} does not match num_codebooks*n_frames {n}")
    if expected["codes"] != actual["codes"]:
        f.append(f"codes mismatch: expected {expected['codes']}, actual {actual['codes']}")
    return Report(not f, f)


def compare_fast_ar_frame_dumps(expected: dict, actual: dict) -> Report:
    f = []
    _meta(f, "text", expected["text"], actual["text"])
    _meta(f, "temperature", expected["temperature"], actual["temperature"], close=True)
    _meta(f, "top_p", expected["top_p"], actual["top_p"], close=True)
    for k in ("top_k", "min_tokens_before_end", "prompt_cols", "main_token_id"):
        _meta(f, k, expected[k], actual[k])
    e, a = expected["slow_hidden"], actual["slow_hidden"]
    if len(e) != len(a):
        f.append(f"slow_hidden length mismatch: expected {len(e)}, actual {len(a)}")
    else:
        max_abs, l2 = 0.0, 0.0
        for x, y in zip(e, a):
            d = _f32(x) - _f32(y)
            max_abs = max(max_abs, abs(d))
            l2 += d * d
        l2 = math.sqrt(l2)
        if max_abs > 1e-2 or l2 > 0.5:
            f.append(f"slow_hidden mismatch: max_abs={max_abs:.8f} l2={l2:.8f}")
    if expected["codebook_ids"] != actual["codebook_ids"]:
        f.append(f"codebook_ids mismatch: expected {expected['codebook_ids']}, actual {actual['codebook_ids']}")
    return Report(not f, f)


def compare_semantic_token_dumps(expected: dict, actual: dict) -> Report:
    f = []
    _meta(f, "text", expected["text"], actual["text"])
    _meta(f, "temperature", expected["temperature"], actual["temperature"], close=True)
    _meta(f, "top_p", expected["top_p"], actual["top_p"], close=True)
    for k in ("top_k", "max_new_tokens", "min_tokens_before_end", "prompt_cols", "main_token_ids"):
        _meta(f, k, expected[k], actual[k])
    return Report(not f, f)


# -- Slow-AR tensor statistics ---------------------------------------------------
_REQUIRED = ("normalized", "query", "key", "value", "attention", "projected", "hidden")
_OPTIONAL = ("ffn_normalized", "ffn_gate", "ffn_up", "ffn_activated", "ffn_projected", "block_hidden")


def _effective_tolerance(expected: dict, actual: dict, tol: SlowArTensorTolerance) -> SlowArTensorTolerance:
    """Looser bounds for full 36-layer stacks (lib.rs:1516-1534)."""
    layers = max(expected.get("layer_count") or 1, actual.get("layer_count") or 1)
    if layers < 36:
        return tol
    return SlowArTensorTolerance(max(tol.max_l2_delta, 0.75), max(tol.max_mean_abs_delta, 6e-3),
                                 max(tol.max_max_abs_delta, 1.0), max(tol.max_first8_mae, 0.20))


def _tokens(dump: dict, side: str, failures: list):
    """normalized_slow_ar_tokens (lib.rs:1536-1592)."""
    seq = dump.get("sequence") or []
    if seq:
        tc = dump.get("token_count")
        if tc is not None and tc != len(seq):
            failures.append(f"{side}.token_count mismatch: declared {tc}, sequence has {len(seq)}")
        return seq
    if all(dump.get(k) is not None for k in _REQUIRED):
        tok = {"position": dump["position"]}
        for k in _REQUIRED + _OPTIONAL:
            tok[k] = dump.get(k)
        return [tok]
    failures.append(f"{side} Slow-AR dump has no top-level stats or sequence")
    return []


def _first8_mae(e, a) -> float:
    n = max(len(e), len(a))
    if n == 0:
        return 0.0
    return sum(abs((e[i] if i < len(e) else 0.0) - (a[i] if i < len(a) else 0.0)) for i in range(n)) / n


def _compare_stats(name, e, a, tol, failures) -> TensorDelta:
    if e["len"] != a["len"]:
        failures.append(f"{name}.len mismatch: expected {e['len']}, actual {a['len']}")
    d = TensorDelta(name, abs(e["l2"] - a["l2"]), abs(e["mean_abs"] - a["mean_abs"]),
                    abs(e["max_abs"] - a["max_abs"]), _first8_mae(e["first8"], a["first8"]))
    if d.l2_delta > tol.max_l2_delta:
        failures.append(f"{name}.l2 delta {d.l2_delta:.8f} exceeds {tol.max_l2_delta:.8f}")
    if d.mean_abs_delta > tol.max_mean_abs_delta:
        failures.append(f"{name}.mean_abs delta {d.mean_abs_delta:.8f} exceeds {tol.max_mean_abs_delta:.8f}")
    if d.max_abs_delta > tol.max_max_abs_delta:
        failures.append(f"{name}.max_abs delta {d.max_abs_delta:.8f} exceeds {tol.max_max_abs_delta:.8f}")
    if d.first8_mae > tol.max_first8_mae:
        failures.append(f"{name}.first8 MAE {d.first8_mae:.8f} exceeds {tol.max_first8_mae:.8f}")
    return d


def _compare_optional(name, e, a, tol, failures) -> Optional[TensorDelta]:
    if e is not None and a is not None:
        return _compare_stats(name, e, a, tol, failures)
    if e is not None:
        failures.append(f"{name} missing from actual dump")
    elif a is not None:
        failures.append(f"{name} missing from expected dump")
    return None


def compare_slow_ar_dumps(expected: dict, actual: dict, tolerance: SlowArTensorTolerance = None) -> Report:
    tol = tolerance or SlowArTensorTolerance()
    f = []
    for k in ("layer", "position", "hidden_size", "head_count", "head_count_kv", "head_dim"):
        if expected[k] != actual[k]:
            f.append(f"{k} mismatch: expected {expected[k]}, actual {actual[k]}")
    el, al = expected.get("layer_count"), actual.get("layer_count")
    if el is not None and al is not None and el != al:
        f.append(f"layer_count mismatch: expected {el}, actual {al}")
    elif el is not None and al is None:
        f.append("layer_count missing from actual dump")
    elif el is None and al is not None:
        f.append("layer_count missing from expected dump")
    tol = _effective_tolerance(expected, actual, tol)
    et, at = _tokens(expected, "expected", f), _tokens(actual, "actual", f)
    if len(et) != len(at):
        f.append(f"token count mismatch: expected {len(et)}, actual {len(at)}")
    deltas = []
    for i, (e, a) in enumerate(zip(et, at)):
        if e["position"] != a["position"]:
            f.append(f"token{i}.position mismatch: expected {e['position']}, actual {a['position']}")
        for k in _REQUIRED:
            deltas.append(_compare_stats(f"token{i}.{k}", e[k], a[k], tol, f))
        for k in _OPTIONAL:
            d = _compare_optional(f"token{i}.{k}", e.get(k), a.get(k), tol, f)
            if d:
                deltas.append(d)
    d = _compare_optional("final_normalized", expected.get("final_normalized"), actual.get("final_normalized"),
                          tol, f)
    if d:
        deltas.append(d)
    d = _compare_optional("logits", expected.get("logits"), actual.get("logits"),
                          replace(tol, max_l2_delta=max(tol.max_l2_delta, 2.5)), f)
    if d:
        deltas.append(d)
    et_top, at_top = expected.get("top_logits") or [], actual.get("top_logits") or []
    if et_top or at_top:
        if len(et_top) != len(at_top):
            f.append(f"top_logits length mismatch: expected {len(et_top)}, actual {len(at_top)}")
        for i, (e, a) in enumerate(zip(et_top, at_top)):
            if e["token_id"] != a["token_id"]:
                f.append(f"top_logits[{i}].token_id mismatch: expected {e['token_id']}, actual {a['token_id']}")
            dv = abs(e["value"] - a["value"])
            if dv > tol.max_max_abs_delta:
                f.append(f"top_logits[{i}].value delta {dv:.8f} exceeds {tol.max_max_abs_delta:.8f}")
    return Report(not f, f, deltas)


# -- codec stages -----------------------------------------------------------------

@dataclass(frozen=True)
class StageTolerance:
    max_l2_delta: float
    max_mean_abs_delta: float
    max_max_abs_delta: float
    max_first8_mae: float
    max_num_samples_delta: int = 0


# RvqLookupTolerance / PostModuleTolerance / DecodeStageTolerance /
# WaveformTolerance ::default (lib.rs:290-300, 334-344, 378-391, 584-595)
RVQ_LOOKUP_TOLERANCE = StageTolerance(5e-4, 5e-6, 5e-5, 5e-5)
POST_MODULE_TOLERANCE = StageTolerance(5e-4, 5e-6, 5e-5, 5e-5)
DECODE_STAGE_TOLERANCE = StageTolerance(5e-3, 5e-5, 3e-3, 2e-3)
WAVEFORM_TOLERANCE = StageTolerance(50.0, 0.05, 0.2, 0.15, 0)


@dataclass
class StageReport:
    passed: bool
    failures: List[str]
    l2_delta: float
    mean_abs_delta: float
    max_abs_delta: float
    first8_mae: float
    prefix: str = ""

    @property
    def tensor_deltas(self):
        return []


def _stage_common(expected, actual, checks, failures):
    if expected.get("text") != actual.get("text"):
        failures.append(f"text mismatch: expected {_opt(expected.get('text'))}, actual {_opt(actual.get('text'))}")
    for name in checks:
        if int(expected[name]) != int(actual[name]):
            failures.append(f"{name} mismatch: expected {int(expected[name])}, actual {int(actual[name])}")


def _opt(text):
    """Rust's {:?} of an Option<String>."""
    return "None" if text is None else f"Some({json.dumps(text)})"


def _stage_stats(expected, actual, prefix, tol, failures):
    l2 = abs(expected[f"{prefix}_l2"] - actual[f"{prefix}_l2"])
    mean = abs(expected[f"{prefix}_mean_abs"] - actual[f"{prefix}_mean_abs"])
    mx = abs(expected[f"{prefix}_max_abs"] - actual[f"{prefix}_max_abs"])
    f8 = _first8_mae(expected[f"{prefix}_first8"], actual[f"{prefix}_first8"])
    if l2 > tol.max_l2_delta:
        failures.append(f"{prefix}_l2 delta {l2:.8f} exceeds {tol.max_l2_delta:.8f}")
    if mean > tol.max_mean_abs_delta:
        failures.append(f"{prefix}_mean_abs delta {mean:.8f} exceeds {tol.max_mean_abs_delta:.8f}")
    if mx > tol.max_max_abs_delta:
        failures.append(f"{prefix}_max_abs delta {mx:.8f} exceeds {tol.max_max_abs_delta:.8f}")
    if f8 > tol.max_first8_mae:
        failures.append(f"{prefix}_first8 MAE {f8:.8f} exceeds {tol.max_first8_mae:.8f}")
    return StageReport(not failures, failures, l2, mean, mx, f8, prefix)


def _len_check(dump, side, len_key, frames_key, dim_key, failures):
    want = int(dump[frames_key]) * int(dump[dim_key])
    if int(dump[len_key]) != want:
        failures.append(f"{side} {len_key} {int(dump[len_key])} does not match {frames_key}*{dim_key} {want}")


def compare_rvq_lookup_dumps(expected: dict, actual: dict, tolerance: StageTolerance = RVQ_LOOKUP_TOLERANCE):
    f = []
    _stage_common(expected, actual, ("num_codebooks", "n_frames", "latent_dim", "latent_len"), f)
    _len_check(expected, "expected", "latent_len", "n_frames", "latent_dim", f)
    _len_check(actual, "actual", "latent_len", "n_frames", "latent_dim", f)
    return _stage_stats(expected, actual, "latent", tolerance, f)


def compare_post_module_dumps(expected: dict, actual: dict, tolerance: StageTolerance = POST_MODULE_TOLERANCE):
    f = []
    _stage_common(expected, actual, ("num_codebooks", "n_frames", "hidden_dim", "hidden_len"), f)
    _len_check(expected, "expected", "hidden_len", "n_frames", "hidden_dim", f)
    _len_check(actual, "actual", "hidden_len", "n_frames", "hidden_dim", f)
    return _stage_stats(expected, actual, "hidden", tolerance, f)


def compare_decode_stage_dumps(expected: dict, actual: dict, tolerance: StageTolerance = DECODE_STAGE_TOLERANCE):
    f = []
    _stage_common(expected, actual, ("num_codebooks", "input_frames", "output_frames", "hidden_dim", "hidden_len"), f)
    _len_check(expected, "expected", "hidden_len", "output_frames", "hidden_dim", f)
    _len_check(actual, "actual", "hidden_len", "output_frames", "hidden_dim", f)
    return _stage_stats(expected, actual, "hidden", tolerance, f)


def compare_waveform_dumps(expected: dict, actual: dict, tolerance: StageTolerance = WAVEFORM_TOLERANCE):
    f = []
    _stage_common(expected, actual, ("num_codebooks", "input_frames", "sample_rate"), f)
    d = abs(int(expected["num_samples"]) - int(actual["num_samples"]))
    if d > tolerance.max_num_samples_delta:
        f.append(f"num_samples delta {d} exceeds {tolerance.max_num_samples_delta}")
    return _stage_stats(expected, actual, "samples", tolerance, f)


_COMMANDS = {
    "compare-generated-codes": (compare_generated_codes_dumps, "generated codebook parity failed"),
    "compare-semantic-tokens": (compare_semantic_token_dumps, "semantic token parity failed"),
    "compare-fast-ar-frame": (compare_fast_ar_frame_dumps, "Fast-AR frame parity failed"),
    "compare-slow-ar": (compare_slow_ar_dumps, "Slow-AR tensor parity failed"),
    "compare-rvq-lookup": (compare_rvq_lookup_dumps, "RVQ lookup parity failed"),
    "compare-post-module": (compare_post_module_dumps, "post-module parity failed"),
    "compare-decode-stage": (compare_decode_stage_dumps, "decode-stage parity failed"),
    "compare-waveform": (compare_waveform_dumps, "waveform parity failed"),
}


def _wav_main(argv) -> int:
    from .wav import WavError, compare_metrics, metrics_from_wav_bytes

    def load(p):
        with open(p, "rb") as f:
            return metrics_from_wav_bytes(f.read(), 50)
    try:
        if argv[0] == "metrics":
            m = load(argv[1])
            print(f"sample_rate={m.sample_rate}\nchannels={m.channels}\nbits_per_sample={m.bits_per_sample}\n"
                  f"duration_seconds={m.duration_seconds:.6f}\nrms={m.rms:.8f}\npeak={m.peak:.8f}\n"
                  f"envelope_frames={len(m.envelope_rms)}")
            return 0
        r = compare_metrics(load(argv[1]), load(argv[2]))
    except (WavError, OSError) as e:
        print(f"error: {e}", file=sys.stderr)
        return 1
    print(f"passed={'true' if r.passed else 'false'}\nduration_delta_seconds={r.duration_delta_seconds:.6f}\n"
          f"rms_delta={r.rms_delta:.8f}\nenvelope_mae={r.envelope_mae:.8f}")
    for x in r.failures:
        print(f"failure={x}")
    if not r.passed:
        print("error: WAV parity failed", file=sys.stderr)
        return 1
    return 0


def main(argv=None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    if (len(argv) == 2 and argv[0] == "metrics") or (len(argv) == 3 and argv[0] == "compare"):
        return _wav_main(argv)
    if len(argv) != 3 or argv[0] not in _COMMANDS:
        print("usage:\n" + "\n".join(f"  python -m s2hip.parity {c} <expected.json> <actual.json>"
                                     for c in _COMMANDS), file=sys.stderr)
        return 2
    fn, msg = _COMMANDS[argv[0]]
    with open(argv[1]) as fe, open(argv[2]) as fa:
        report = fn(json.load(fe), json.load(fa))
    print(f"passed={'true' if report.passed else 'false'}")
    if isinstance(report, StageReport):
        for key, v in (("l2_delta", report.l2_delta), ("mean_abs_delta", report.mean_abs_delta),
                       ("max_abs_delta", report.max_abs_delta), ("first8_mae", report.first8_mae)):
            print(f"{report.prefix}_{key}={v:.8f}")
    for d in report.tensor_deltas:
        print(f"tensor={d.name} l2_delta={d.l2_delta:.8f} mean_abs_delta={d.mean_abs_delta:.8f} "
              f"max_abs_delta={d.max_abs_delta:.8f} first8_mae={d.first8_mae:.8f}")
    for x in report.failures:
        print(f"failure={x}")
    if not report.passed:
        print(msg, file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
