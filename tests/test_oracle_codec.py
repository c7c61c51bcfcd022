"""Pins of the CPU oracle's RVQ codec decode (crates/fish_s2_infer/src/codec.rs).

Each oracle function is checked against an independent formulation: torch's
float64 conv1d / conv_transpose1d / layer_norm / linear (library routines with
PyTorch's weight layouts, which match the ggml orders [out][in][k] and
[in][out][k] the reference indexes), math.erf (the Abramowitz-Stegun bound of
erf_approx), closed forms, and the causal-prefix invariant of the whole
decode.  A transposed weight, a flipped or mis-padded tap, a wrong dilation,
a window off by one or a dropped bias fails one of them.

The reference's own codec tests need a real codec GGUF (ignored in its tree,
codec.rs:3974-4060) and hold no numeric vectors; their invariants (shapes,
finiteness, non-zero outputs, 2 code frames -> 8 latent frames) are checked
here on the synthetic codec.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import random_codes
from oracle import oracle as O
from s2hip.gguf import GgufFile

torch.set_default_dtype(torch.float64)


def _f16v(rng, shape, scale=1.0):
    """Random values that are exactly representable in f16 (like F16 weights)."""
    return (rng.standard_normal(shape) * scale).astype(np.float16).astype(np.float32)


def _t(a):
    return torch.from_numpy(np.asarray(a, np.float64))


def _round16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float64)


def _close(got, ref, tol):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    err = np.max(np.abs(got - ref)) / max(1e-30, np.max(np.abs(ref)))
    assert err < tol, f"relative max error {err:.3e} >= {tol:.1e}"


# --- op level ---------------------------------------------------------------------------

@pytest.mark.parametrize("k,dil", [(7, 1), (7, 3), (7, 9), (1, 1), (3, 2)])
def test_conv1d_matches_torch(k, dil):
    rng = np.random.default_rng(k * 10 + dil)
    T, cin, cout = 41, 24, 20
    x = rng.standard_normal((T, cin)).astype(np.float32) * 1.7
    w = _f16v(rng, (cout, cin, k), 0.2)
    b = _f16v(rng, (cout,), 0.1)
    got = O.codec_conv1d(x, w, b, dil)
    # causal: left-pad (k-1)*dil frames; the reference rounds its padded input to f16
    xin = F.pad(_t(_round16(x)).T[None], ((k - 1) * dil, 0))
    ref = F.conv1d(xin, _t(w), _t(b), dilation=dil)[0].T
    assert got.shape == (T, cout)
    _close(got, ref.numpy(), 2e-6)


def test_conv1d_rounds_input_to_f16():
    # an input halfway between two f16 values rounds to even before the product
    x = np.array([[1.0 + 2.0 ** -11]], np.float32)  # halfway between 1 and 1 + 2^-10
    got = O.codec_conv1d(x, np.ones((1, 1, 1), np.float32), np.zeros(1, np.float32))
    assert got[0, 0] == 1.0


@pytest.mark.parametrize("stride,k", [(2, 2), (8, 16), (4, 8), (2, 4), (3, 5)])
def test_conv_transpose_matches_torch(stride, k):
    rng = np.random.default_rng(stride * 100 + k)
    T, cin, cout = 13, 18, 22
    x = rng.standard_normal((T, cin)).astype(np.float32)
    w = _f16v(rng, (cin, cout, k), 0.2)
    b = _f16v(rng, (cout,), 0.1)
    got = O.codec_conv_transpose(x, w, b, stride)
    full = F.conv_transpose1d(_t(x).T[None], _t(w), _t(b), stride=stride)[0].T
    # crop to frames * stride: taps past the last output frame are dropped
    assert got.shape == (T * stride, cout)
    _close(got, full[: T * stride].numpy(), 2e-6)


def test_depthwise_matches_torch():
    rng = np.random.default_rng(5)
    T, C, k = 33, 16, 7
    x = rng.standard_normal((T, C)).astype(np.float32)
    w = _f16v(rng, (C, k), 0.3)
    b = _f16v(rng, (C,), 0.1)
    got = O.codec_depthwise(x, w, b)
    ref = F.conv1d(F.pad(_t(x).T[None], (k - 1, 0)), _t(w)[:, None, :], _t(b), groups=C)[0].T
    _close(got, ref.numpy(), 2e-6)


def test_layer_norm_matches_torch():
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((9, 1024)) * 3 + 0.7).astype(np.float32)
    w, b = _f16v(rng, (1024,), 1.0), _f16v(rng, (1024,), 0.5)
    got = O.codec_layer_norm(x, w, b, 1e-6)
    ref = F.layer_norm(_t(x), (1024,), _t(w), _t(b), eps=1e-6)
    _close(got, ref.numpy(), 2e-6)


def test_erf_and_gelu_within_abramowitz_stegun_bound():
    # 7.1.26: |error| <= 1.5e-7; f32 evaluation adds a few ulp of 1
    for v in np.linspace(-6, 6, 2401):
        v = float(np.float32(v))
        assert abs(O.codec_erf(v) - math.erf(v)) < 1.5e-7 + 3e-7, v
        exact = 0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0)))
        assert abs(O.codec_gelu(v) - exact) < 4e-7 * max(1.0, abs(v)), v
    assert O.codec_erf(0.0) == pytest.approx(0.0, abs=1e-7)
    assert O.codec_erf(-1.0) == -O.codec_erf(1.0)


def test_snake_closed_form_and_zero_alpha_guard():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((5, 6)).astype(np.float32) * 2
    alpha = np.array([1.0, 0.5, -0.7, 0.0, 1e-9, 2.0], np.float32)
    got = O.codec_snake(x, alpha)
    a = np.where(np.abs(alpha) < 1e-8, np.float32(1e-8), alpha).astype(np.float64)
    ref = x + np.sin(a * x) ** 2 / a
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=1e-6)
    # alpha 0 behaves as alpha 1e-8: x + 1e-8 x^2 (to f32 rounding)
    np.testing.assert_allclose(got[:, 3], x[:, 3] + 1e-8 * x[:, 3].astype(np.float64) ** 2, rtol=1e-6)


# --- stage level over the synthetic codec -----------------------------------------------

@pytest.fixture(scope="module")
def codec(codec_gguf):
    with O.OracleCodec(codec_gguf, 8) as c:
        yield c


@pytest.fixture(scope="module")
def gg(codec_gguf):
    g = GgufFile(codec_gguf)
    yield g
    g.close()


def _w(gg, name):
    t = gg.tensor(name)
    return t.f32().reshape(tuple(reversed(t.dims))).astype(np.float64)


def test_rvq_lookup_closed_form(codec, gg):
    codes = random_codes(6, seed=1)
    got = codec.rvq_lookup(codes, 10, 6)
    ref = np.zeros((6, 1024))
    for q in range(10):
        p = ("quantizer.semantic_quantizer.quantizers.0" if q == 0
             else f"quantizer.quantizer.quantizers.{q - 1}")
        cb = _w(gg, p + ".codebook.weight")          # [size][8]
        wp = _w(gg, p + ".out_proj.weight")          # [1024][8]
        bp = _w(gg, p + ".out_proj.bias")
        ref += cb[codes[q]] @ wp.T + bp
    _close(got, ref, 1e-6)


def test_rvq_lookup_errors(codec):
    codes = random_codes(2, seed=2)
    with pytest.raises(RuntimeError, match="codec codebook count mismatch: expected 10, got 9"):
        codec.rvq_lookup(codes[:9], 9, 2)
    bad = codes.copy()
    bad[3, 1] = -1
    with pytest.raises(RuntimeError, match="codec code must be non-negative, got -1"):
        codec.rvq_lookup(bad, 10, 2)
    bad = codes.copy()
    bad[0, 0] = 4096
    with pytest.raises(RuntimeError, match="embedding index 4096 out of range for vocab_dim 4096"):
        codec.rvq_lookup(bad, 10, 2)
    bad = codes.copy()
    bad[5, 1] = 1024
    with pytest.raises(RuntimeError, match="embedding index 1024 out of range for vocab_dim 1024"):
        codec.rvq_lookup(bad, 10, 2)


def _rms(x, w, eps):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w


def _rope(x, pos, hd=64, base=1e4):
    # adjacent pairs (x0, x1) rotated by pos / base^(2i/hd), as complex numbers
    T = x.shape[0]
    z = x.reshape(T, -1, hd // 2, 2)
    zc = z[..., 0] + 1j * z[..., 1]
    ang = pos[:, None, None] / base ** (np.arange(0, hd, 2) / hd)[None, None, :]
    r = zc * np.exp(1j * ang)
    return np.stack([r.real, r.imag], -1).reshape(x.shape)


def _post_module_ref(gg, lat, window=128):
    T = lat.shape[0]
    x = lat.astype(np.float64)
    pos = np.arange(T, dtype=np.float64)
    idx = np.arange(T)
    band = (idx[None, :] <= idx[:, None]) & (idx[None, :] > idx[:, None] - window)
    for l in range(8):
        p = f"quantizer.post_module.layers.{l}"
        h = _rms(x, _w(gg, p + ".attention_norm.weight"), 1e-5)
        qkv = h @ _w(gg, p + ".attention.wqkv.weight").T
        q, k, v = _rope(qkv[:, :1024], pos), _rope(qkv[:, 1024:2048], pos), qkv[:, 2048:]
        q, k, v = (a.reshape(T, 16, 64).transpose(1, 0, 2) for a in (q, k, v))
        s = q @ k.transpose(0, 2, 1) / 8.0
        s = np.where(band[None], s, -np.inf)
        pr = np.exp(s - s.max(-1, keepdims=True))
        pr /= pr.sum(-1, keepdims=True)
        att = (pr @ v).transpose(1, 0, 2).reshape(T, 1024)
        x = x + (att @ _w(gg, p + ".attention.wo.weight").T) * _w(gg, p + ".attention_layer_scale.gamma")
        h = _rms(x, _w(gg, p + ".ffn_norm.weight"), 1e-5)
        g, u = h @ _w(gg, p + ".feed_forward.w1.weight").T, h @ _w(gg, p + ".feed_forward.w3.weight").T
        a = g / (1 + np.exp(-g)) * u
        x = x + (a @ _w(gg, p + ".feed_forward.w2.weight").T) * _w(gg, p + ".ffn_layer_scale.gamma")
    return _rms(x, _w(gg, "quantizer.post_module.norm.weight"), 1e-5)


def test_post_module_matches_float64_with_window(codec, gg):
    # 133 frames: the 128-frame window drops the oldest keys of the last 5 queries
    lat = codec.rvq_lookup(random_codes(133, seed=3), 10, 133)
    got = codec.post_module(lat)
    _close(got, _post_module_ref(gg, lat), 2e-5)
    # a 129-frame window is measurably different (the check sees the window)
    assert np.max(np.abs(_post_module_ref(gg, lat, 129) - got)) > 1e-3


def test_post_module_needs_a_frame(codec):
    with pytest.raises(RuntimeError, match="codec transformer requires at least one frame"):
        codec.post_module(np.zeros((0, 1024), np.float32))


def _upsample_ref(gg, x):
    x = _t(x)
    for st in range(2):
        p = f"quantizer.upsample.{st}"
        y = F.conv_transpose1d(x.T[None], _t(_w(gg, p + ".0.conv.weight")), _t(_w(gg, p + ".0.conv.bias")),
                               stride=2)[0].T[: 2 * x.shape[0]]
        dw = _t(_w(gg, p + ".1.dwconv.conv.weight"))  # (1024, 1, 7)
        h = F.conv1d(F.pad(y.T[None], (6, 0)), dw, _t(_w(gg, p + ".1.dwconv.conv.bias")), groups=1024)[0].T
        h = F.layer_norm(h, (1024,), _t(_w(gg, p + ".1.norm.weight")), _t(_w(gg, p + ".1.norm.bias")), eps=1e-6)
        h = F.gelu(F.linear(h, _t(_w(gg, p + ".1.pwconv1.weight")), _t(_w(gg, p + ".1.pwconv1.bias"))))
        h = F.linear(h, _t(_w(gg, p + ".1.pwconv2.weight")), _t(_w(gg, p + ".1.pwconv2.bias")))
        x = y + h * _t(_w(gg, p + ".1.gamma"))
    return x.numpy()


def test_upsample_matches_torch(codec, gg):
    rng = np.random.default_rng(8)
    hid = rng.standard_normal((5, 1024)).astype(np.float32)
    got = codec.upsample(hid)
    assert got.shape == (20, 1024)
    _close(got, _upsample_ref(gg, hid), 2e-5)


def _snake_t(x, alpha):
    a = torch.where(alpha.abs() < 1e-8, torch.full_like(alpha, float(np.float32(1e-8))), alpha)
    return x + torch.sin(a * x) ** 2 / a


def _conv_t(x, w, b, dil=1):
    # causal conv over f16-rounded input (the reference rounds its padded input)
    k = w.shape[2]
    xin = _t(_round16(x.numpy()))
    return F.conv1d(F.pad(xin.T[None], ((k - 1) * dil, 0)), w, b, dilation=dil)[0].T


def _entry_ref(gg, hidden):
    return _conv_t(_t(hidden), _t(_w(gg, "decoder.model.0.conv.weight")),
                   _t(_w(gg, "decoder.model.0.conv.bias"))).numpy()


def _block_ref(gg, x, b):
    """forward_codec_decoder_block b (0-based) on the residual stream x."""
    rates = (8, 8, 4, 2)
    p = f"decoder.model.{b + 1}.block"
    x = _snake_t(_t(x), _t(_w(gg, p + ".0.alpha")).reshape(-1))
    n = x.shape[0]
    x = F.conv_transpose1d(x.T[None], _t(_w(gg, p + ".1.conv.weight")), _t(_w(gg, p + ".1.conv.bias")),
                           stride=rates[b])[0].T[: n * rates[b]]
    for r, dil in zip(range(3), (1, 3, 9)):
        q = f"{p}.{r + 2}.block"
        y = _snake_t(x, _t(_w(gg, q + ".0.alpha")).reshape(-1))
        y = _conv_t(y, _t(_w(gg, q + ".1.conv.weight")), _t(_w(gg, q + ".1.conv.bias")), dil)
        y = _snake_t(y, _t(_w(gg, q + ".2.alpha")).reshape(-1))
        y = _conv_t(y, _t(_w(gg, q + ".3.conv.weight")), _t(_w(gg, q + ".3.conv.bias")))
        x = x + y
    return x.numpy()


def _tail_ref(gg, x):
    x = _snake_t(_t(x), _t(_w(gg, "decoder.model.5.alpha")).reshape(-1))
    x = _conv_t(x, _t(_w(gg, "decoder.model.6.conv.weight")), _t(_w(gg, "decoder.model.6.conv.bias")))
    return torch.tanh(x).reshape(-1).numpy()


def test_decoder_matches_torch_stage_by_stage(codec, gg):
    """Each decoder stage in float64 from the oracle's previous checkpoint, so
    the check is per stage: a rounding-boundary flip of one f16 conv input
    (f32 vs f64 operands) cannot compound across the 13 convolutions."""
    rng = np.random.default_rng(9)
    hid = rng.standard_normal((2, 1024)).astype(np.float32)
    prev = codec.decoder(hid, 0)
    _close(prev, _entry_ref(gg, hid), 2e-5)
    for b in range(4):
        cur = codec.decoder(hid, b + 1)
        assert cur.shape == (prev.shape[0] * (8, 8, 4, 2)[b], (768, 384, 192, 96)[b])
        # per block (6 convolutions), rounding-boundary flips of f16 inputs
        # leave ~2e-4 of the block's largest value; a layout mistake is O(1)
        _close(cur, _block_ref(gg, prev, b), 1e-3)
        prev = cur
    wav = codec.decoder(hid)
    assert wav.shape == (1024,)
    _close(wav, _tail_ref(gg, prev), 2e-5)


def test_decoder_rejects_wrong_hidden_dim(codec):
    with pytest.raises(RuntimeError, match="decoder expects latent dim 1024, got 512"):
        codec.decoder(np.zeros((2, 512), np.float32))


def test_decode_waveform_composes_stages_and_is_causal(codec):
    codes = random_codes(5, seed=4)
    wav = codec.decode_waveform(codes, 10, 5)
    assert wav.shape == (5 * 2048,)
    assert np.all(np.isfinite(wav)) and np.all(np.abs(wav) <= 1.0) and np.any(wav != 0)
    lat = codec.rvq_lookup(codes, 10, 5)
    up = codec.upsample(codec.post_module(lat))
    assert up.shape == (20, 1024)  # 2 code frames -> 8 latent frames in the reference's test
    np.testing.assert_array_equal(wav, codec.decoder(up))
    # every stage is causal: the first 3 frames decode to the same leading samples
    head = codec.decode_waveform(np.ascontiguousarray(codes[:, :3]), 10, 3)
    np.testing.assert_array_equal(head, wav[: 3 * 2048])
