"""ctypes binding of the CPU oracle (oracle/s2_oracle.cpp).

TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker / CPU baseline, never by the
product path.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libs2oracle.so")

FAITHFUL_SLOW_RELOAD = 1
FAITHFUL_FAST_RECOMPUTE = 2
KV_F16 = 4  # Slow-AR K/V rounded to f16 when cached

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u64p = ctypes.POINTER(ctypes.c_uint64)


class Spec(ctypes.Structure):
    _fields_ = [
        (n, ctypes.c_uint32)
        for n in (
            "slow_layers", "fast_layers", "dim", "ffn", "heads", "kv_heads", "head_dim",
            "fast_dim", "fast_ffn", "fast_heads", "fast_kv_heads", "fast_head_dim",
            "vocab", "codebook_size", "num_codebooks", "semantic_begin", "semantic_end",
            "slow_qk_norm", "scale_codebook_embeddings", "linear_type",
        )
    ] + [(n, ctypes.c_float) for n in ("rope_base", "fast_rope_base", "eps", "fast_eps")]


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} missing: build it with `make -C oracle`")
    L = ctypes.CDLL(LIB_PATH)
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    L.orc_f32_to_f16.argtypes = [ctypes.c_float]
    L.orc_f32_to_f16.restype = ctypes.c_uint16
    L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_f16_to_f32.restype = ctypes.c_float
    L.orc_dequant_row.argtypes = [vp, ctypes.c_uint32, sz, vp]
    L.orc_rms_norm.argtypes = [vp, vp, sz, ctypes.c_float, vp]
    L.orc_rms_norm_heads.argtypes = [vp, vp, sz, sz, ctypes.c_float, vp]
    L.orc_linear.argtypes = [vp, vp, ctypes.c_uint32, sz, sz, vp]
    L.orc_rope_normal.argtypes = [vp, sz, sz, sz, ctypes.c_float]
    L.orc_gqa_attention.argtypes = [vp, vp, vp, sz, sz, sz, sz, ctypes.c_float, vp]
    L.orc_swiglu_slow.argtypes = [vp, vp, sz, vp]
    L.orc_swiglu_slow.restype = None
    L.orc_swiglu_fast.argtypes = [vp, vp, sz, vp]
    L.orc_swiglu_fast.restype = None
    L.orc_rng_next_unit.argtypes = [_u64p]
    L.orc_rng_next_unit.restype = ctypes.c_double
    L.orc_sample_token.argtypes = [vp, sz, ctypes.c_float, ctypes.c_float, ctypes.c_int32,
                                   ctypes.c_int64, _u64p, _u32p]
    L.orc_sample_token_margins.argtypes = [vp, sz, ctypes.c_float, ctypes.c_float, ctypes.c_int32,
                                           ctypes.c_int64, _u64p, _u32p, vp]
    L.orc_semantic_bias.argtypes = [vp, sz, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int64, ctypes.c_int32]
    L.orc_semantic_bias.restype = None
    L.orc_expf.argtypes = [vp, sz, vp]
    L.orc_expf.restype = None
    L.orc_transpose_to_time_major.argtypes = [vp, ctypes.c_uint32, sz, vp]
    L.orc_compact_codes.argtypes = [vp, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]
    L.orc_compact_codes.restype = sz
    L.orc_open.argtypes = [ctypes.c_char_p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                           ctypes.c_uint32, ctypes.c_char_p, sz]
    L.orc_open.restype = vp
    L.orc_close.argtypes = [vp]
    L.orc_close.restype = None
    L.orc_get_spec.argtypes = [vp, ctypes.POINTER(Spec)]
    L.orc_reset.argtypes = [vp]
    L.orc_reset.restype = None
    L.orc_n_past.argtypes = [vp]
    L.orc_n_past.restype = ctypes.c_uint32
    L.orc_eval.argtypes = [vp, vp, sz, vp, vp, ctypes.c_char_p, sz]
    L.orc_fast_logits.argtypes = [vp, vp, vp, sz, vp, ctypes.c_char_p, sz]
    L.orc_embed.argtypes = [vp, vp, sz, vp, ctypes.c_char_p, sz]
    L.orc_fast_codebooks.argtypes = [vp, vp, ctypes.c_uint32, ctypes.c_float, ctypes.c_float,
                                     ctypes.c_int32, _u64p, vp, ctypes.c_char_p, sz]
    L.orc_generate_codes.argtypes = [vp, vp, sz, ctypes.c_uint32, ctypes.c_float, ctypes.c_float,
                                     ctypes.c_int32, ctypes.c_uint32, _u64p, vp, _u32p,
                                     ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
                                     ctypes.c_char_p, sz]
    cp, u32 = ctypes.c_char_p, ctypes.c_uint32
    L.orc_codec_open.argtypes = [cp, u32, cp, sz]
    L.orc_codec_open.restype = vp
    L.orc_codec_close.argtypes = [vp]
    L.orc_codec_close.restype = None
    L.orc_codec_rvq_lookup.argtypes = [vp, vp, u32, u32, vp, cp, sz]
    L.orc_codec_post_module.argtypes = [vp, vp, u32, vp, cp, sz]
    L.orc_codec_upsample.argtypes = [vp, vp, u32, vp, cp, sz]
    L.orc_codec_decoder.argtypes = [vp, vp, u32, u32, u32, vp, cp, sz]
    L.orc_codec_decode_waveform.argtypes = [vp, vp, u32, u32, vp, cp, sz]
    L.orc_codec_snake.argtypes = [vp, sz, sz, vp, vp]
    L.orc_codec_snake.restype = None
    L.orc_codec_conv1d.argtypes = [vp, sz, sz, sz, sz, vp, sz, vp, vp, cp, sz]
    L.orc_codec_conv_transpose.argtypes = [vp, sz, sz, sz, sz, vp, sz, vp, vp, cp, sz]
    L.orc_codec_depthwise.argtypes = [vp, sz, sz, sz, vp, vp, vp]
    L.orc_codec_depthwise.restype = None
    L.orc_codec_layer_norm.argtypes = [vp, sz, sz, vp, vp, ctypes.c_float]
    L.orc_codec_layer_norm.restype = None
    L.orc_codec_erf.argtypes = [ctypes.c_float]
    L.orc_codec_erf.restype = ctypes.c_float
    L.orc_codec_gelu.argtypes = [ctypes.c_float]
    L.orc_codec_gelu.restype = ctypes.c_float
    for name in ("orc_codec_rvq_lookup", "orc_codec_post_module", "orc_codec_upsample", "orc_codec_decoder",
                 "orc_codec_decode_waveform", "orc_codec_conv1d", "orc_codec_conv_transpose"):
        getattr(L, name).restype = ctypes.c_int32
    for name in ("orc_dequant_row", "orc_rms_norm", "orc_rms_norm_heads", "orc_linear",
                 "orc_rope_normal", "orc_gqa_attention", "orc_sample_token", "orc_sample_token_margins",
                 "orc_transpose_to_time_major", "orc_get_spec", "orc_eval", "orc_fast_logits", "orc_embed",
                 "orc_fast_codebooks", "orc_generate_codes"):
        getattr(L, name).restype = ctypes.c_int32
    _lib = L
    return L


def _p(a):
    return a.ctypes.data


def f32_to_f16(v: float) -> int:
    return lib().orc_f32_to_f16(v)


def f16_to_f32(b: int) -> float:
    return lib().orc_f16_to_f32(b)


def dequant_row(raw: bytes, ggml_type: int, n: int) -> np.ndarray:
    src = np.frombuffer(raw, dtype=np.uint8).copy()
    out = np.zeros(n, np.float32)
    if not lib().orc_dequant_row(_p(src), ggml_type, n, _p(out)):
        raise ValueError("dequant failed")
    return out


def rms_norm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.zeros_like(x)
    if not lib().orc_rms_norm(_p(x), _p(w), x.size, eps, _p(out)):
        raise ValueError("rms_norm failed")
    return out


def rms_norm_heads(x, w, head_dim, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.zeros_like(x)
    if not lib().orc_rms_norm_heads(_p(x), _p(w), x.size, head_dim, eps, _p(out)):
        raise ValueError("rms_norm_heads failed")
    return out


def linear(x, w_raw: np.ndarray, ggml_type: int, in_dim: int, out_dim: int):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w_raw)
    y = np.zeros(out_dim, np.float32)
    if not lib().orc_linear(_p(x), _p(w), ggml_type, in_dim, out_dim, _p(y)):
        raise ValueError("linear failed")
    return y


def rope_normal(values, head_dim, position, base):
    v = np.array(values, np.float32)
    if not lib().orc_rope_normal(_p(v), v.size, head_dim, position, base):
        raise ValueError("rope failed")
    return v


def gqa_attention(q, k, v, heads, kv_heads, head_dim, tokens, scale):
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    out = np.zeros(heads * head_dim, np.float32)
    if not lib().orc_gqa_attention(_p(q), _p(k), _p(v), heads, kv_heads, head_dim, tokens, scale, _p(out)):
        raise ValueError("attention failed")
    return out


def swiglu(gate, up, fast=False):
    g = np.ascontiguousarray(gate, np.float32)
    u = np.ascontiguousarray(up, np.float32)
    out = np.zeros_like(g)
    (lib().orc_swiglu_fast if fast else lib().orc_swiglu_slow)(_p(g), _p(u), g.size, _p(out))
    return out


def sample_token(logits, temperature, top_p, top_k, always_include=None, rng_state=0):
    """Returns (token, new_rng_state)."""
    x = np.ascontiguousarray(logits, np.float32)
    st = ctypes.c_uint64(rng_state)
    tok = ctypes.c_uint32(0)
    lib().orc_sample_token(_p(x), x.size, temperature, top_p, top_k,
                           -1 if always_include is None else always_include,
                           ctypes.byref(st), ctypes.byref(tok))
    return tok.value, st.value


def sample_token_margins(logits, temperature, top_p, top_k, always_include=None, rng_state=0):
    """sample_token plus its margins: returns (token, new_rng_state, (draw, cut, tie))
    -- the distance of the draw target from the cumulative-sum boundaries
    around the chosen item, of the top-p sums from top_p around the cut, and
    the logit gap between the chosen item and its sort-order neighbours."""
    x = np.ascontiguousarray(logits, np.float32)
    st = ctypes.c_uint64(rng_state)
    tok = ctypes.c_uint32(0)
    mg = np.zeros(3, np.float32)
    lib().orc_sample_token_margins(_p(x), x.size, temperature, top_p, top_k,
                                   -1 if always_include is None else always_include,
                                   ctypes.byref(st), ctypes.byref(tok), _p(mg))
    return tok.value, st.value, tuple(float(v) for v in mg)


def semantic_bias(logits, sem_begin, sem_end, im_end=None, block_im_end=False):
    """build_semantic_bias + apply_semantic_bias on a copy of `logits`."""
    x = np.array(logits, np.float32)
    lib().orc_semantic_bias(_p(x), x.size, sem_begin, sem_end, -1 if im_end is None else im_end,
                            1 if block_im_end else 0)
    return x


def expf(x):
    """The C library's expf (what Rust's f32::exp calls) over an array."""
    a = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(a)
    lib().orc_expf(_p(a), a.size, _p(out))
    return out


def next_unit(rng_state):
    st = ctypes.c_uint64(rng_state)
    v = lib().orc_rng_next_unit(ctypes.byref(st))
    return v, st.value


def transpose_to_time_major(data, rows, cols):
    d = np.ascontiguousarray(data, np.uint32)
    out = np.zeros(rows * cols, np.int32)
    if not lib().orc_transpose_to_time_major(_p(d), rows, cols, _p(out)):
        raise ValueError("rows must be non-zero")
    return out


def compact_codes(codes, num_codebooks, max_new, n_frames):
    c = np.array(codes, np.int32)
    n = lib().orc_compact_codes(_p(c), num_codebooks, max_new, n_frames)
    return c[:n]


class OracleModel:
    """The restated SlowArState + FastArWeights + generate_codes."""

    def __init__(self, gguf_path: str, max_seq_len: int, im_end_id: int, flags: int = 0,
                 threads: int = 0):
        err = ctypes.create_string_buffer(1024)
        h = lib().orc_open(gguf_path.encode(), max_seq_len, im_end_id, flags, threads, err, len(err))
        if not h:
            raise RuntimeError(err.value.decode())
        self._h = h
        self.im_end_id = im_end_id
        sp = Spec()
        lib().orc_get_spec(h, ctypes.byref(sp))
        self.spec = sp

    def close(self):
        if self._h:
            lib().orc_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        lib().orc_reset(self._h)

    @property
    def n_past(self):
        return lib().orc_n_past(self._h)

    def eval(self, flat_tokens, want_logits=True):
        flat = np.ascontiguousarray(flat_tokens, np.int32)
        width = self.spec.num_codebooks + 1
        hidden = np.zeros(self.spec.dim, np.float32)
        logits = np.zeros(self.spec.vocab, np.float32) if want_logits else None
        err = ctypes.create_string_buffer(1024)
        ok = lib().orc_eval(self._h, _p(flat), flat.size // width, _p(hidden),
                            _p(logits) if want_logits else None, err, len(err))
        if not ok:
            raise RuntimeError(err.value.decode())
        return hidden, logits

    def embed(self, flat_tokens):
        """embed_slow_ar_time_major alone: [n_tokens][dim]."""
        flat = np.ascontiguousarray(flat_tokens, np.int32)
        n = flat.size // (self.spec.num_codebooks + 1)
        out = np.zeros((n, self.spec.dim), np.float32)
        err = ctypes.create_string_buffer(1024)
        if not lib().orc_embed(self._h, _p(flat), n, _p(out), err, len(err)):
            raise RuntimeError(err.value.decode())
        return out

    def fast_logits(self, hidden, prefix):
        h = np.ascontiguousarray(hidden, np.float32)
        p = np.ascontiguousarray(prefix, np.uint32)
        out = np.zeros(self.spec.codebook_size, np.float32)
        err = ctypes.create_string_buffer(1024)
        if not lib().orc_fast_logits(self._h, _p(h), _p(p), p.size, _p(out), err, len(err)):
            raise RuntimeError(err.value.decode())
        return out

    def fast_codebooks(self, hidden, sem_code, temperature, top_p, top_k, rng_state):
        h = np.ascontiguousarray(hidden, np.float32)
        codes = np.zeros(self.spec.num_codebooks, np.uint32)
        st = ctypes.c_uint64(rng_state)
        err = ctypes.create_string_buffer(1024)
        if not lib().orc_fast_codebooks(self._h, _p(h), sem_code, temperature, top_p, top_k,
                                        ctypes.byref(st), _p(codes), err, len(err)):
            raise RuntimeError(err.value.decode())
        return codes, st.value

    def generate_codes(self, prompt_flat, max_new, temperature=0.0, top_p=1.0, top_k=0,
                       min_tokens_before_end=0, rng_state=0):
        flat = np.ascontiguousarray(prompt_flat, np.int32)
        width = self.spec.num_codebooks + 1
        codes = np.zeros(self.spec.num_codebooks * max_new, np.int32)
        st = ctypes.c_uint64(rng_state)
        nf = ctypes.c_uint32(0)
        tp, td = ctypes.c_double(0), ctypes.c_double(0)
        err = ctypes.create_string_buffer(1024)
        if not lib().orc_generate_codes(self._h, _p(flat), flat.size // width, max_new, temperature,
                                        top_p, top_k, min_tokens_before_end, ctypes.byref(st),
                                        _p(codes), ctypes.byref(nf), ctypes.byref(tp),
                                        ctypes.byref(td), err, len(err)):
            raise RuntimeError(err.value.decode())
        n = nf.value
        return {
            "codes": codes[: self.spec.num_codebooks * n].reshape(self.spec.num_codebooks, n),
            "n_frames": n,
            "rng_state": st.value,
            "prefill_seconds": tp.value,
            "decode_seconds": td.value,
        }


# ---------------------------------------------------------------------------
# RVQ codec decode (crates/fish_s2_infer/src/codec.rs:1690-1714)
# ---------------------------------------------------------------------------
CODEC_HIDDEN = 1024
CODEC_SAMPLES_PER_LATENT = 512  # decoder rates 8 * 8 * 4 * 2


def _f32(a):
    return np.ascontiguousarray(a, np.float32)


def _check(ok, err):
    if not ok:
        raise RuntimeError(err.value.decode())


def codec_snake(x, alpha):
    x, alpha = _f32(x), _f32(alpha)
    out = np.empty_like(x)
    lib().orc_codec_snake(_p(x), x.shape[0], x.shape[1], _p(alpha), _p(out))
    return out


def codec_conv1d(x, weight, bias, dilation=1):
    """x [frames][in]; weight in ggml order [out][in][k] (numpy shape (out, in, k))."""
    x, w, b = _f32(x), _f32(weight), _f32(bias)
    out = np.empty((x.shape[0], w.shape[0]), np.float32)
    err = ctypes.create_string_buffer(512)
    _check(lib().orc_codec_conv1d(_p(x), x.shape[0], x.shape[1], w.shape[0], dilation, _p(w), w.size, _p(b),
                                  _p(out), err, len(err)), err)
    return out


def codec_conv_transpose(x, weight, bias, stride):
    """x [frames][in]; weight in ggml order [in][out][k] (numpy shape (in, out, k))."""
    x, w, b = _f32(x), _f32(weight), _f32(bias)
    out = np.empty((x.shape[0] * stride, w.shape[1]), np.float32)
    err = ctypes.create_string_buffer(512)
    _check(lib().orc_codec_conv_transpose(_p(x), x.shape[0], x.shape[1], w.shape[1], stride, _p(w), w.size,
                                          _p(b), _p(out), err, len(err)), err)
    return out


def codec_depthwise(x, weight, bias):
    """x [frames][ch]; weight numpy shape (ch, k)."""
    x, w, b = _f32(x), _f32(weight), _f32(bias)
    out = np.empty_like(x)
    lib().orc_codec_depthwise(_p(x), x.shape[0], x.shape[1], w.shape[1], _p(w), _p(b), _p(out))
    return out


def codec_layer_norm(x, weight, bias, eps):
    x = _f32(x).copy()
    w, b = _f32(weight), _f32(bias)
    lib().orc_codec_layer_norm(_p(x), x.shape[0], x.shape[1], _p(w), _p(b), eps)
    return x


def codec_erf(v):
    return float(lib().orc_codec_erf(v))


def codec_gelu(v):
    return float(lib().orc_codec_gelu(v))


class OracleCodec:
    """CPU decode_waveform and its stages over a codec GGUF."""

    def __init__(self, gguf_path: str, threads: int = 0):
        err = ctypes.create_string_buffer(1024)
        self._h = lib().orc_codec_open(gguf_path.encode(), threads, err, len(err))
        if not self._h:
            raise RuntimeError(err.value.decode())

    def close(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.orc_codec_close(self._h)
        self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def rvq_lookup(self, codes, num_codebooks, n_frames):
        c = np.ascontiguousarray(codes, np.int32).ravel()
        out = np.empty((n_frames, CODEC_HIDDEN), np.float32)
        err = ctypes.create_string_buffer(512)
        _check(lib().orc_codec_rvq_lookup(self._h, _p(c), num_codebooks, n_frames, _p(out), err, len(err)), err)
        return out

    def post_module(self, latents):
        x = _f32(latents)
        out = np.empty_like(x)
        err = ctypes.create_string_buffer(512)
        _check(lib().orc_codec_post_module(self._h, _p(x), x.shape[0], _p(out), err, len(err)), err)
        return out

    def upsample(self, hidden):
        x = _f32(hidden)
        out = np.empty((4 * x.shape[0], CODEC_HIDDEN), np.float32)
        err = ctypes.create_string_buffer(512)
        _check(lib().orc_codec_upsample(self._h, _p(x), x.shape[0], _p(out), err, len(err)), err)
        return out

    def decoder(self, hidden, stop_block=5):
        """Samples (stop_block 5), or the residual stream after stop_block
        (0..4) decoder blocks."""
        x = _f32(hidden)
        rates, ch = (8, 8, 4, 2), (1536, 768, 384, 192, 96)
        if stop_block >= 5:
            out = np.empty(x.shape[0] * CODEC_SAMPLES_PER_LATENT, np.float32)
        else:
            out = np.empty((x.shape[0] * int(np.prod(rates[:stop_block])), ch[stop_block]), np.float32)
        err = ctypes.create_string_buffer(512)
        _check(lib().orc_codec_decoder(self._h, _p(x), x.shape[0], x.shape[1], stop_block, _p(out), err,
                                       len(err)), err)
        return out

    def decode_waveform(self, codes, num_codebooks, n_frames):
        c = np.ascontiguousarray(codes, np.int32).ravel()
        out = np.empty(n_frames * 4 * CODEC_SAMPLES_PER_LATENT, np.float32)
        err = ctypes.create_string_buffer(512)
        _check(lib().orc_codec_decode_waveform(self._h, _p(c), num_codebooks, n_frames, _p(out), err, len(err)),
               err)
        return out
