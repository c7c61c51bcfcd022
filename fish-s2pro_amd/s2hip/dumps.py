"""Parity dumps in the JSON schemas of the reference's dump tools.

The reference's comparator (`fish_s2_parity compare-*`,
crates/fish_s2_parity/src/lib.rs:67-260,709-804,1211-1534) reads these files,
and so does `s2hip.parity`, its restatement here:

* `generated_codes_dump`  GeneratedCodesDump (fish_s2_codes_dump.rs:10-26):
  generate_codes (generate.rs:117-221), codebook-major codes.
* `semantic_token_dump`   SemanticTokenDump (fish_s2_semantic_dump.rs:8-19):
  generate_semantic_tokens (generate.rs:56-114), the Slow-AR-only loop whose
  step input is [main, semantic code, 0, ...].
* `fast_ar_frame_dump`    FastArFrameDump (fish_s2_fast_ar_dump.rs:10-22):
  generate_fast_ar_first_frame (generate.rs:224-271).
* `slow_ar_dump`          SlowArDump with TensorStats
  (fish_s2_slow_ar_dump.rs:9-74,110-226): every intermediate of a block of
  Slow-AR layers (forward_slow_ar_block_prefill_layers, slow_ar.rs:980-1039)
  over the tool's fixed hidden inputs, computed with the op-level kernels.
* codec stages over a GeneratedCodesDump, computed by the GPU codec
  (`s2hip.Codec`): `rvq_lookup_dump` RvqLookupDump
  (fish_s2_rvq_lookup_dump.rs:16-27), `post_module_dump` PostModuleDump
  (fish_s2_post_module_dump.rs:17-28), `decode_stage_dump` DecodeStageDump
  (fish_s2_decode_stage_dump.rs:19-31, rvq_decode_latents' output) and
  `waveform_dump` WaveformDump (fish_s2_waveform_dump.rs:19-31).

The reference's tools build the prompt from text with tokenizer.json; here
the caller passes the prompt as time-major token ids and `text` is carried
into the dump as a label (the comparator checks it like any metadata field).
The loops and samplers run on the GPU through the engine; nothing here
computes model math on the host except the per-tensor statistics.
"""

import argparse
import json
import sys

import numpy as np

from .engine import Engine, S2HipError
from .gguf import GgufFile

BACKEND = "rust-hip"


def f32_json(x) -> float:
    """The value of an f32 as a float whose shortest repr is the f32's
    shortest repr (serde_json writes f32 fields that way)."""
    return float(str(np.float32(x)))


def tensor_stats(values) -> dict:
    """TensorStats (fish_s2_slow_ar_dump.rs:208-226): len, l2 = sqrt of the
    sequential f32 sum of squares, mean_abs = sequential f32 sum of |x| / len,
    max_abs, first8."""
    v = np.ascontiguousarray(values, np.float32).ravel()
    n = v.size
    if n:
        l2 = np.sqrt(np.cumsum(v * v, dtype=np.float32)[-1])
        mean_abs = np.cumsum(np.abs(v), dtype=np.float32)[-1] / np.float32(n)
        max_abs = max(np.float32(0.0), np.max(np.abs(v)))
    else:
        l2 = mean_abs = max_abs = np.float32(0.0)
    return {
        "len": int(n),
        "l2": f32_json(l2),
        "mean_abs": f32_json(mean_abs),
        "max_abs": f32_json(max_abs),
        "first8": [f32_json(x) for x in v[:8]],
    }


def f64_stats(prefix: str, values) -> dict:
    """The codec dump tools' statistics (fish_s2_rvq_lookup_dump.rs:123-150):
    l2 = sqrt of the sequential f64 sum of squares, mean_abs = sequential f64
    sum of |x| / len, max_abs = fold(0, max) over |x|, first8 as f64."""
    v = np.ascontiguousarray(values, np.float32).ravel().astype(np.float64)
    n = v.size
    return {
        f"{prefix}_l2": float(np.sqrt(np.cumsum(v * v)[-1])) if n else 0.0,
        f"{prefix}_mean_abs": float(np.cumsum(np.abs(v))[-1] / n) if n else 0.0,
        f"{prefix}_max_abs": float(max(0.0, np.max(np.abs(v)))) if n else 0.0,
        f"{prefix}_first8": [float(x) for x in v[:8]],
    }


def write_json(path: str, dump: dict):
    with open(path, "w") as f:
        json.dump(dump, f, indent=2)


# -- Slow-AR sampling over the semantic candidates ---------------------------
def semantic_sample(engine: Engine, logits, generated_after_prefill: int, min_tokens_before_end: int,
                    temperature: float, top_p: float, top_k: int, rng_state: int):
    """sample_semantic_token (generate.rs:284-298) on the device sampler.

    build_semantic_bias / apply_semantic_bias (sampling.rs:54-100) leave the
    semantic ids and im_end finite and every other logit -inf; im_end is
    masked too while generated_after_prefill < min_tokens_before_end, and is
    the force-included id otherwise.  The sampler runs on the finite
    candidates in ascending-id order (the stable descending sort, top-k,
    softmax and top-p see the same finite values in the same order) plus, when
    the reference's list reaches into the masked ids, the one masked id its
    list would end with: the -inf entries sort last in ascending-id order and
    add nothing to any sum, so the only way one is drawn is the fall-through
    of sample_discrete (sampling.rs:227-241), which returns the list's last
    entry.  Returns (token id, new RNG state)."""
    sp = engine.spec
    im_end = engine.im_end_id
    vocab = sp["vocab"]
    block = generated_after_prefill < min_tokens_before_end
    ids = np.arange(sp["semantic_begin"], sp["semantic_end"] + 1, dtype=np.int64)
    if block:
        ids = ids[ids != im_end]
    elif im_end < vocab:
        ids = np.union1d(ids, np.array([im_end], np.int64))
    force = None
    if not block and im_end < vocab:
        force = int(np.searchsorted(ids, im_end))
    sub = np.asarray(logits, np.float32)[ids]
    n_fin = int(np.isfinite(sub).sum())
    n_list = min(top_k, vocab) if top_k > 0 else vocab  # entries after top-k (before force-include)
    if n_list > n_fin and n_fin == ids.size:
        # the masked entry at the end of the reference's list: the
        # (n_list - n_fin)-th masked id in ascending order
        k = n_list - n_fin - 1
        masked = np.setdiff1d(np.arange(vocab, dtype=np.int64), ids, assume_unique=True)
        ids = np.append(ids, masked[k])
        sub = np.append(sub, np.float32(-np.inf))
    sub = np.ascontiguousarray(sub, np.float32)
    idx, rng = engine.sample(sub, temperature, top_p, top_k, force, rng_state)
    return int(ids[idx]), rng


def semantic_to_codebook_id(spec: dict, token: int) -> int:
    """generate.rs:273-282."""
    if token < spec["semantic_begin"] or token > spec["semantic_end"]:
        return 0
    code = token - spec["semantic_begin"]
    return min(code, spec["codebook_size"] - 1)


def _prompt(engine: Engine, prompt_flat):
    flat = np.ascontiguousarray(prompt_flat, np.int32).ravel()
    if flat.size == 0 or flat.size % engine.codebook_dim:
        raise S2HipError(f"prompt length {flat.size} is not a positive multiple of {engine.codebook_dim}")
    return flat, flat.size // engine.codebook_dim


# -- loop-level dumps ----------------------------------------------------------
def generated_codes_dump(engine: Engine, prompt_flat, text: str = "hi", max_new_tokens: int = 2,
                         temperature: float = 0.0, top_p: float = 1.0, top_k: int = 0,
                         min_tokens_before_end: int = 0, seed: int = 0, prompt_text=None,
                         prompt_code_cols=None) -> dict:
    """fish_s2_codes_dump (defaults as its flags: 2 frames, greedy, seed 0)."""
    flat, cols = _prompt(engine, prompt_flat)
    r = engine.generate_codes(flat, max_new_tokens, temperature, top_p, top_k, min_tokens_before_end, seed)
    dump = {"backend": BACKEND}
    if prompt_text is not None:
        dump["prompt_text"] = prompt_text
    if prompt_code_cols is not None:
        dump["prompt_code_cols"] = int(prompt_code_cols)
    dump.update({
        "text": text,
        "temperature": f32_json(temperature),
        "top_p": f32_json(top_p),
        "top_k": int(top_k),
        "max_new_tokens": int(max_new_tokens),
        "min_tokens_before_end": int(min_tokens_before_end),
        "prompt_cols": int(cols),
        "num_codebooks": int(engine.spec["num_codebooks"]),
        "n_frames": int(r["n_frames"]),
        "codes": [int(c) for c in np.asarray(r["codes"]).ravel()],
    })
    return dump


def semantic_token_dump(engine: Engine, prompt_flat, text: str = "hi", max_new_tokens: int = 4,
                        temperature: float = 0.0, top_p: float = 1.0, top_k: int = 0,
                        min_tokens_before_end: int = 0, seed: int = 0) -> dict:
    """fish_s2_semantic_dump: prefill, then Slow-AR steps on
    [main, semantic code, 0, ...] (build_step_input without codebooks,
    generate.rs:300-344) until im_end or max_new_tokens steps."""
    sp = engine.spec
    flat, cols = _prompt(engine, prompt_flat)
    engine.reset()
    _, logits = engine.eval(flat)
    rng = seed
    main, rng = semantic_sample(engine, logits, 0, min_tokens_before_end, temperature, top_p, top_k, rng)
    tokens = [main]
    generated = 0
    while main != engine.im_end_id and generated < max_new_tokens:
        step = np.zeros(engine.codebook_dim, np.int32)
        step[0] = main
        if sp["semantic_begin"] <= main <= sp["semantic_end"]:
            code = main - sp["semantic_begin"]
            if code >= sp["codebook_size"]:
                raise S2HipError(f"semantic token {main} maps outside codebook_size {sp['codebook_size']}")
            step[1] = code
        _, logits = engine.step(step)
        generated += 1
        gap = max(engine.n_past - cols, 0) + (len(tokens) - 1)  # generate.rs:97-100
        main, rng = semantic_sample(engine, logits, gap, min_tokens_before_end, temperature, top_p, top_k, rng)
        tokens.append(main)
    return {
        "backend": BACKEND,
        "text": text,
        "temperature": f32_json(temperature),
        "top_p": f32_json(top_p),
        "top_k": int(top_k),
        "max_new_tokens": int(max_new_tokens),
        "min_tokens_before_end": int(min_tokens_before_end),
        "prompt_cols": int(cols),
        "main_token_ids": [int(t) for t in tokens],
    }


def fast_ar_frame_dump(engine: Engine, prompt_flat, text: str = "hi", temperature: float = 0.0,
                       top_p: float = 1.0, top_k: int = 0, min_tokens_before_end: int = 0,
                       seed: int = 0) -> dict:
    """fish_s2_fast_ar_dump: prefill, the first main token, and the Fast-AR
    codebooks of that frame from the post-norm hidden."""
    flat, cols = _prompt(engine, prompt_flat)
    engine.reset()
    hidden, logits = engine.eval(flat)
    main, rng = semantic_sample(engine, logits, 0, min_tokens_before_end, temperature, top_p, top_k, seed)
    code = semantic_to_codebook_id(engine.spec, main)
    codes, _ = engine.fast_codebooks(hidden, code, temperature, top_p, top_k, rng)
    return {
        "backend": BACKEND,
        "text": text,
        "temperature": f32_json(temperature),
        "top_p": f32_json(top_p),
        "top_k": int(top_k),
        "min_tokens_before_end": int(min_tokens_before_end),
        "prompt_cols": int(cols),
        "main_token_id": int(main),
        "slow_hidden": [f32_json(x) for x in hidden],
        "codebook_ids": [int(c) for c in codes],
    }


# -- Slow-AR per-op dump ---------------------------------------------------------
class EngineOps:
    """The per-op primitives slow_ar_dump composes, on the engine's kernels."""

    def __init__(self, engine: Engine):
        self.e = engine

    def rms_norm(self, x, w, eps):
        return self.e.rms_norm(x, w, eps).ravel()

    def linear(self, w_raw, ggml_type, in_dim, out_dim, x):
        return self.e.linear(w_raw, ggml_type, in_dim, out_dim, x).ravel()

    def qk_rope(self, qkv, heads, kv_heads, head_dim, position, base, q_norm, k_norm, eps):
        return self.e.qk_rope(qkv, heads, kv_heads, head_dim, position, base, q_norm, k_norm, eps)

    def attention(self, q, keys, values, heads, kv_heads, head_dim, tokens, scale):
        return self.e.attention(q, keys, values, heads, kv_heads, head_dim, tokens, scale)

    def swiglu(self, gate, up):
        return self.e.swiglu(gate, up, fast=False)


def hidden_fixture(hidden_size: int, token_index: int) -> np.ndarray:
    """The dump tool's input row (fish_s2_slow_ar_dump.rs:200-206)."""
    h = np.zeros(hidden_size, np.float32)
    h[0] = 1.0
    h[1] = np.float32(-0.5) + np.float32(token_index)
    h[hidden_size - 1] = np.float32(0.25) + np.float32(token_index) * np.float32(0.125)
    return h


def _layer_weights(g: GgufFile, layer: int):
    def t(suffix):
        return g.tensor(f"layers.{layer}.{suffix}")
    return {
        "attn_norm": t("attention_norm.weight").f32(),
        "ffn_norm": t("ffn_norm.weight").f32(),
        "q_norm": t("attention.q_norm.weight").f32() if f"layers.{layer}.attention.q_norm.weight" in g.tensors else None,
        "k_norm": t("attention.k_norm.weight").f32() if f"layers.{layer}.attention.k_norm.weight" in g.tensors else None,
        "wqkv": t("attention.wqkv.weight"),
        "wo": t("attention.wo.weight"),
        "w1": t("feed_forward.w1.weight"),
        "w2": t("feed_forward.w2.weight"),
        "w3": t("feed_forward.w3.weight"),
    }


def _block_prefill_layer(ops, W, spec, hidden_tokens, cache_k, cache_v, start):
    """forward_block_prefill_sequence (slow_ar.rs:558-617) for one layer:
    every token prepared (norm, wqkv, QK-norm, RoPE), every K/V written, then
    attention over positions [0, position] of the cache (entries below
    `start` stay zero, as in a fresh SlowArKvCache), wo + residual, and the
    feed-forward block."""
    d, H, Hkv, hd, ffn = spec["dim"], spec["heads"], spec["kv_heads"], spec["head_dim"], spec["ffn"]
    eps, base = spec["eps"], spec["rope_base"]
    q_size, kv_size = H * hd, Hkv * hd
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    prepared = []
    for off, h in enumerate(hidden_tokens):
        normalized = ops.rms_norm(h, W["attn_norm"], eps)
        qkv = ops.linear(W["wqkv"].data, W["wqkv"].ggml_type, d, q_size + 2 * kv_size, normalized)
        q, k, v = ops.qk_rope(qkv, H, Hkv, hd, start + off, base, W["q_norm"], W["k_norm"], eps)
        prepared.append((normalized, q, k, v))
    for off, (_, _, k, v) in enumerate(prepared):
        cache_k[start + off] = k
        cache_v[start + off] = v
    outs = []
    for off, (h, (normalized, q, k, v)) in enumerate(zip(hidden_tokens, prepared)):
        visible = start + off + 1
        att = ops.attention(q, cache_k[:visible], cache_v[:visible], H, Hkv, hd, visible, scale)
        projected = ops.linear(W["wo"].data, W["wo"].ggml_type, q_size, d, att)
        hidden = (h + projected).astype(np.float32)
        f_norm = ops.rms_norm(hidden, W["ffn_norm"], eps)
        gate = ops.linear(W["w1"].data, W["w1"].ggml_type, d, ffn, f_norm)
        up = ops.linear(W["w3"].data, W["w3"].ggml_type, d, ffn, f_norm)
        act = ops.swiglu(gate, up)
        f_proj = ops.linear(W["w2"].data, W["w2"].ggml_type, ffn, d, act)
        block = (hidden + f_proj).astype(np.float32)
        outs.append({
            "normalized": normalized, "query": q, "key": k, "value": v, "attention": att,
            "projected": projected, "hidden": hidden, "ffn_normalized": f_norm, "ffn_gate": gate,
            "ffn_up": up, "ffn_activated": act, "ffn_projected": f_proj, "block_hidden": block,
        })
    return outs


_TOKEN_FIELDS = ("normalized", "query", "key", "value", "attention", "projected", "hidden", "ffn_normalized",
                 "ffn_gate", "ffn_up", "ffn_activated", "ffn_projected", "block_hidden")


def top_logits(logits, count: int):
    """Descending by value, ties by ascending id (fish_s2_slow_ar_dump.rs:228-246)."""
    v = np.asarray(logits, np.float32)
    order = np.lexsort((np.arange(v.size), -v.astype(np.float64)))[: min(count, v.size)]
    return [{"token_id": int(i), "value": f32_json(v[i])} for i in order]


def slow_ar_dump(ops, gguf: GgufFile, spec: dict, transformer: str, layer: int = 0, layers: int = 1,
                 position: int = 0, tokens: int = 1, logits: bool = False, top_k: int = 8) -> dict:
    """fish_s2_slow_ar_dump: layers [layer, layer + layers) over `tokens`
    fixture rows at positions position..; the statistics are those of the
    block's last layer, the first token at the top level and every token
    under "sequence" when tokens > 1.  With `logits`, the head
    (SlowArOutputHeadF16Weights::forward_logits, slow_ar.rs:943-955) on the
    last token's output: final_normalized, logits and top_logits."""
    if layers < 1 or tokens < 1 or top_k < 1:
        raise S2HipError("layers, tokens and top_k must be greater than zero")
    if layer + layers > spec["slow_layers"]:
        raise S2HipError(f"slow layer range out of bounds: start={layer} count={layers} "
                         f"available={spec['slow_layers']}")
    kv = spec["kv_heads"] * spec["head_dim"]
    cache_k = np.zeros((position + tokens, kv), np.float32)
    cache_v = np.zeros((position + tokens, kv), np.float32)
    hs = [hidden_fixture(spec["dim"], i) for i in range(tokens)]
    outs = None
    for li in range(layer, layer + layers):
        cache_k[:] = 0.0  # each layer has its own cache rows
        cache_v[:] = 0.0
        outs = _block_prefill_layer(ops, _layer_weights(gguf, li), spec, hs, cache_k, cache_v, position)
        hs = [o["block_hidden"] for o in outs]
    stats = [{name: tensor_stats(o[name]) for name in _TOKEN_FIELDS} for o in outs]
    dump = {
        "transformer": transformer,
        "layer": int(layer),
        "layer_count": int(layers),
        "position": int(position),
        "token_count": int(tokens),
        "hidden_size": int(spec["dim"]),
        "head_count": int(spec["heads"]),
        "head_count_kv": int(spec["kv_heads"]),
        "head_dim": int(spec["head_dim"]),
    }
    dump.update(stats[0])
    if logits:
        emb = gguf.tensor("embeddings.weight")
        normalized = ops.rms_norm(hs[-1], gguf.tensor("norm.weight").f32(), spec["eps"])
        lg = ops.linear(emb.data, emb.ggml_type, spec["dim"], emb.rows, normalized)
        dump["final_normalized"] = tensor_stats(normalized)
        dump["logits"] = tensor_stats(lg)
        dump["top_logits"] = top_logits(lg, top_k)
    if tokens > 1:
        dump["sequence"] = [dict({"position": int(position + i)}, **s) for i, s in enumerate(stats)]
    return dump


# -- command line ------------------------------------------------------------------
def _load_prompt(path: str):
    with open(path) as f:
        obj = json.load(f)
    if isinstance(obj, dict):
        obj = obj.get("flat_time_major", obj.get("flat"))
    return np.asarray(obj, np.int32)


# -- codec stages ---------------------------------------------------------------

def _codes(codes_dump: dict):
    return (np.asarray(codes_dump["codes"], np.int32), int(codes_dump["num_codebooks"]),
            int(codes_dump["n_frames"]))


def rvq_lookup_dump(codec, codes_dump: dict) -> dict:
    """RvqLookupDump of rvq_lookup_codes (codec.rs:2536-2596) on the codes."""
    codes, ncb, n = _codes(codes_dump)
    lat = codec.rvq_lookup(codes, ncb, n)
    return {"backend": BACKEND, "text": codes_dump.get("text"), "num_codebooks": ncb, "n_frames": n,
            "latent_dim": int(lat.shape[1]), "latent_len": int(lat.size), **f64_stats("latent", lat)}


def post_module_dump(codec, codes_dump: dict) -> dict:
    """PostModuleDump of forward_codec_post_module (codec.rs:986-1018) after the lookup."""
    codes, ncb, n = _codes(codes_dump)
    hid = codec.post_module(codec.rvq_lookup(codes, ncb, n))
    return {"backend": BACKEND, "text": codes_dump.get("text"), "num_codebooks": ncb, "n_frames": n,
            "hidden_dim": int(hid.shape[1]), "hidden_len": int(hid.size), **f64_stats("hidden", hid)}


def decode_stage_dump(codec, codes_dump: dict) -> dict:
    """DecodeStageDump of rvq_decode_latents (codec.rs:1282-1297) after the lookup."""
    codes, ncb, n = _codes(codes_dump)
    out = codec.decode_latents(codec.rvq_lookup(codes, ncb, n))
    return {"backend": BACKEND, "text": codes_dump.get("text"), "num_codebooks": ncb, "input_frames": n,
            "output_frames": int(out.shape[0]), "hidden_dim": int(out.shape[1]), "hidden_len": int(out.size),
            **f64_stats("hidden", out)}


def waveform_dump(codec, codes_dump: dict) -> dict:
    """WaveformDump of decode_waveform (codec.rs:1690-1714)."""
    codes, ncb, n = _codes(codes_dump)
    w = codec.decode_waveform(codes, ncb, n)
    return {"backend": BACKEND, "text": codes_dump.get("text"), "num_codebooks": ncb,
            "input_frames": int(w.input_frames), "latent_frames": int(w.latent_frames),
            "sample_rate": int(w.sample_rate), "num_samples": int(w.num_samples),
            **f64_stats("samples", w.samples[: w.num_samples])}


_CODEC_DUMPS = {"rvq-lookup": rvq_lookup_dump, "post-module": post_module_dump,
                "decode-stage": decode_stage_dump, "waveform": waveform_dump}


def main(argv=None):
    ap = argparse.ArgumentParser(prog="python -m s2hip.dumps",
                                 description="Write parity dumps in the reference's JSON schemas.")
    sub = ap.add_subparsers(dest="kind", required=True)
    for kind in ("codes", "semantic", "fast-ar-frame"):
        p = sub.add_parser(kind)
        p.add_argument("--transformer", required=True)
        p.add_argument("--prompt-ids", required=True,
                       help="JSON: time-major flat prompt ids (a list, or {'flat_time_major': [...]})")
        p.add_argument("--output", required=True)
        p.add_argument("--text", default="hi")
        p.add_argument("--im-end-id", type=int, required=True)
        p.add_argument("--temperature", type=float, default=0.0)
        p.add_argument("--top-p", type=float, default=1.0)
        p.add_argument("--top-k", type=int, default=0)
        p.add_argument("--min-tokens-before-end", type=int, default=0)
        p.add_argument("--seed", type=int, default=0)
        if kind != "fast-ar-frame":
            p.add_argument("--max-new-tokens", type=int, default=2 if kind == "codes" else 4)
    p = sub.add_parser("slow-ar")
    p.add_argument("--transformer", required=True)
    p.add_argument("--output", required=True)
    p.add_argument("--layer", type=int, default=0)
    p.add_argument("--layers", type=int, default=1)
    p.add_argument("--position", type=int, default=0)
    p.add_argument("--tokens", type=int, default=1)
    p.add_argument("--logits", action="store_true")
    p.add_argument("--top-k", type=int, default=8)
    for kind in _CODEC_DUMPS:
        p = sub.add_parser(kind)
        p.add_argument("--codec", required=True, help="codec GGUF (fish-speech-codec)")
        p.add_argument("--codes", required=True, help="GeneratedCodesDump JSON (the `codes` dump)")
        p.add_argument("--output", required=True)
    a = ap.parse_args(argv)

    if a.kind in _CODEC_DUMPS:
        from .codec import Codec

        with open(a.codes) as f:
            codes_dump = json.load(f)
        with Codec(a.codec, max(1, int(codes_dump["n_frames"]))) as c:
            dump = _CODEC_DUMPS[a.kind](c, codes_dump)
        write_json(a.output, dump)
        print(f"wrote {a.output}")
        return 0

    if a.kind == "slow-ar":
        g = GgufFile(a.transformer)
        with Engine(a.transformer, max(2, a.position + a.tokens), 0) as e:
            dump = slow_ar_dump(EngineOps(e), g, e.spec, a.transformer, a.layer, a.layers, a.position,
                                a.tokens, a.logits, a.top_k)
    else:
        prompt = _load_prompt(a.prompt_ids)
        max_new = getattr(a, "max_new_tokens", 0)
        with Engine(a.transformer, prompt.size + max_new + 2, a.im_end_id) as e:
            kw = dict(text=a.text, temperature=a.temperature, top_p=a.top_p, top_k=a.top_k,
                      min_tokens_before_end=a.min_tokens_before_end, seed=a.seed)
            if a.kind == "codes":
                dump = generated_codes_dump(e, prompt, max_new_tokens=max_new, **kw)
            elif a.kind == "semantic":
                dump = semantic_token_dump(e, prompt, max_new_tokens=max_new, **kw)
            else:
                dump = fast_ar_frame_dump(e, prompt, **kw)
    write_json(a.output, dump)
    print(f"wrote {a.output}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
