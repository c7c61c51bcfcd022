"""Seeded synthetic dual-AR GGUF models.

The named shapes are the workloads this library is measured and checked on:

* ``tiny``  -- 4 Slow layers, d=512, 8 q / 2 kv heads, head_dim 64, FFN 1536,
  vocab 8192 (semantic ids 7168..8191), 2 Fast layers, 10 codebooks x 1024,
  seed 0.
* ``full``  -- the S2-Pro shape: 36 Slow layers, d=2560, 32 q / 8 kv heads,
  head_dim 128, FFN 9728, vocab 155776 (semantic ids 151678..155773),
  4 Fast layers, 10 codebooks x 4096, seed 1.  f16 weights.
* ``full_q8`` / ``full_q4`` -- the same shape with every linear weight in
  GGML Q8_0 / Q4_0 blocks (norms and embeddings stay f16).

Weights are N(0, 0.02) rounded to f16 (round to nearest even); RMSNorm gains
are 1 (``norm_gain`` sets the residual-stream gains -- attention, FFN and final
norms -- to another value; QK-norm gains stay 1).  Tensor names, shapes and metadata keys follow the reference's
registry (crates/fish_s2_infer/src/registry.rs:45-99, 360-496, 625-650).
``im_end_id`` comes from the tokenizer in the reference
(crates/fish_s2_infer/src/tokenizer.rs:36-62); here it is a fixed
non-semantic id per shape.
"""

from __future__ import annotations

import ctypes
import dataclasses
import os

from . import _paths

GGML_F16 = 1
GGML_Q4_0 = 2
GGML_Q8_0 = 8


class _SynthConfig(ctypes.Structure):
    _fields_ = [
        (name, ctypes.c_uint32)
        for name in (
            "slow_layers", "dim", "ffn", "heads", "kv_heads", "head_dim",
            "fast_layers", "fast_ffn", "fast_heads", "fast_kv_heads", "fast_head_dim",
            "vocab", "codebook_size", "num_codebooks", "semantic_begin", "semantic_end",
            "context_length", "linear_type",
        )
    ] + [
        ("rope_base", ctypes.c_float),
        ("fast_rope_base", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("fast_eps", ctypes.c_float),
        ("init_std", ctypes.c_float),
        ("norm_gain", ctypes.c_float),
        ("seed", ctypes.c_uint64),
    ]


@dataclasses.dataclass(frozen=True)
class ModelShape:
    name: str
    slow_layers: int
    dim: int
    ffn: int
    heads: int
    kv_heads: int
    head_dim: int
    fast_layers: int
    fast_ffn: int
    fast_heads: int
    fast_kv_heads: int
    fast_head_dim: int
    vocab: int
    codebook_size: int
    num_codebooks: int
    semantic_begin: int
    semantic_end: int
    im_end_id: int
    seed: int
    linear_type: int = GGML_F16
    rope_base: float = 1.0e6
    fast_rope_base: float = 1.0e6
    eps: float = 1.0e-6
    fast_eps: float = 1.0e-6
    init_std: float = 0.02
    norm_gain: float = 1.0
    context_length: int = 32768

    def with_(self, **kw) -> "ModelShape":
        return dataclasses.replace(self, **kw)

    def linear_params_per_slow_layer(self) -> int:
        q, kv = self.heads * self.head_dim, self.kv_heads * self.head_dim
        return self.dim * (q + 2 * kv) + q * self.dim + 3 * self.dim * self.ffn

    def linear_params_per_fast_layer(self) -> int:
        q, kv = self.fast_heads * self.fast_head_dim, self.fast_kv_heads * self.fast_head_dim
        return self.dim * (q + 2 * kv) + q * self.dim + 3 * self.dim * self.fast_ffn

    def file_name(self) -> str:
        tag = {GGML_F16: "f16", GGML_Q8_0: "q8_0", GGML_Q4_0: "q4_0"}[self.linear_type]
        gain = "" if self.norm_gain == 1.0 else f"-gain{self.norm_gain:g}"
        return f"s2synth-{self.name}-{tag}{gain}-seed{self.seed}.gguf"


TINY = ModelShape(
    name="tiny", slow_layers=4, dim=512, ffn=1536, heads=8, kv_heads=2, head_dim=64,
    fast_layers=2, fast_ffn=1536, fast_heads=8, fast_kv_heads=2, fast_head_dim=64,
    vocab=8192, codebook_size=1024, num_codebooks=10, semantic_begin=7168,
    semantic_end=8191, im_end_id=7000, seed=0,
)

FULL = ModelShape(
    name="full", slow_layers=36, dim=2560, ffn=9728, heads=32, kv_heads=8, head_dim=128,
    fast_layers=4, fast_ffn=9728, fast_heads=32, fast_kv_heads=8, fast_head_dim=128,
    vocab=155776, codebook_size=4096, num_codebooks=10, semantic_begin=151678,
    semantic_end=155773, im_end_id=151645, seed=1,
)

FULL_Q8 = FULL.with_(name="full", linear_type=GGML_Q8_0)
FULL_Q4 = FULL.with_(name="full", linear_type=GGML_Q4_0)

SHAPES = {"tiny": TINY, "full": FULL, "full_q8": FULL_Q8, "full_q4": FULL_Q4}

_lib = None


def _load():
    global _lib
    if _lib is None:
        path = _paths.synth_library()
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: run __graft_entry__.build() first")
        lib = ctypes.CDLL(path)
        lib.s2synth_write_gguf.argtypes = [
            ctypes.c_char_p, ctypes.POINTER(_SynthConfig), ctypes.c_uint32,
            ctypes.c_char_p, ctypes.c_size_t,
        ]
        lib.s2synth_write_gguf.restype = ctypes.c_int32
        lib.s2synth_write_codec_gguf.argtypes = [
            ctypes.c_char_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_char_p, ctypes.c_size_t,
        ]
        lib.s2synth_write_codec_gguf.restype = ctypes.c_int32
        lib.s2synth_f32_to_f16.argtypes = [ctypes.c_float]
        lib.s2synth_f32_to_f16.restype = ctypes.c_uint16
        lib.s2synth_quantize_block.argtypes = [ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p]
        lib.s2synth_quantize_block.restype = ctypes.c_int32
        _lib = lib
    return _lib


def write_gguf(shape: ModelShape, path: str, threads: int = 0) -> str:
    """Write ``shape`` as a GGUF file at ``path`` and return the path."""
    cfg = _SynthConfig()
    for f in _SynthConfig._fields_:
        key = f[0]
        setattr(cfg, key, getattr(shape, "init_std" if key == "init_std" else key))
    err = ctypes.create_string_buffer(512)
    tmp = path + ".tmp"
    if not _load().s2synth_write_gguf(tmp.encode(), ctypes.byref(cfg), threads, err, len(err)):
        raise RuntimeError(err.value.decode())
    os.replace(tmp, path)
    return path


def ensure_gguf(shape: ModelShape, directory: str, threads: int = 0) -> str:
    """Return a cached GGUF for ``shape`` under ``directory``, writing it once."""
    os.makedirs(directory, exist_ok=True)
    path = os.path.join(directory, shape.file_name())
    if not os.path.exists(path):
        write_gguf(shape, path, threads)
    return path


CODEC_SEED = 3


def codec_file_name(seed: int = CODEC_SEED) -> str:
    return f"s2synth-codec-f16-seed{seed}.gguf"


def write_codec_gguf(path: str, seed: int = CODEC_SEED, threads: int = 0) -> str:
    """Write the decode-side tensors of a seeded synthetic RVQ codec GGUF
    (architecture ``fish-speech-codec``; quantizers, post_module, upsample and
    decoder, all F16, about 370 MB) at ``path`` and return the path."""
    err = ctypes.create_string_buffer(512)
    tmp = path + ".tmp"
    if not _load().s2synth_write_codec_gguf(tmp.encode(), seed, threads, err, len(err)):
        raise RuntimeError(err.value.decode())
    os.replace(tmp, path)
    return path


def ensure_codec_gguf(directory: str, seed: int = CODEC_SEED, threads: int = 0) -> str:
    """Return a cached synthetic codec GGUF under ``directory``, writing it once."""
    os.makedirs(directory, exist_ok=True)
    path = os.path.join(directory, codec_file_name(seed))
    if not os.path.exists(path):
        write_codec_gguf(path, seed, threads)
    return path


def quantize_block(ggml_type: int, values) -> bytes:
    import numpy as np

    x = np.ascontiguousarray(values, dtype=np.float32)
    assert x.size == 32
    out = np.zeros(34 if ggml_type == GGML_Q8_0 else 18, dtype=np.uint8)
    if not _load().s2synth_quantize_block(ggml_type, x.ctypes.data, out.ctypes.data):
        raise ValueError(f"unsupported block type {ggml_type}")
    return out.tobytes()


def voice_clone_prompt(shape: ModelShape, n_text: int, n_frames: int, seed: int):
    """Time-major flat voice-clone prompt in the layout of build_prompt's
    reference-audio branch (prompt.rs:105-192): n_text // 2 text ids, then
    n_frames reference frames (row 0 = semantic_begin + code0, rows 1..ncb =
    the frame's codes, uniform in [0, codebook_size)), then the remaining text
    ids.  Text ids are uniform in [0, semantic_begin)."""
    import numpy as np

    rng = np.random.default_rng(seed)
    ncb = shape.num_codebooks
    pre, post = n_text // 2, n_text - n_text // 2
    flat = np.zeros((pre + n_frames + post, ncb + 1), np.int32)
    flat[:pre, 0] = rng.integers(0, shape.semantic_begin, pre)
    codes = rng.integers(0, shape.codebook_size, (n_frames, ncb))
    flat[pre:pre + n_frames, 0] = shape.semantic_begin + codes[:, 0]
    flat[pre:pre + n_frames, 1:] = codes
    flat[pre + n_frames:, 0] = rng.integers(0, shape.semantic_begin, post)
    return flat.ravel()


def synthetic_prompt(shape: ModelShape, n_tokens: int, seed: int):
    """Time-major flat prompt ([n_tokens][num_codebooks + 1], prompt.rs:77-103)
    of uniform random text ids in [0, semantic_begin) with codebook rows 0."""
    import numpy as np

    rng = np.random.default_rng(seed)
    flat = np.zeros((n_tokens, shape.num_codebooks + 1), np.int32)
    flat[:, 0] = rng.integers(0, shape.semantic_begin, n_tokens)
    return flat.ravel()
