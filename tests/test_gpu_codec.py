"""GPU RVQ codec decode (s2hip_codec_*) against the CPU oracle.

Bars: the RVQ lookup is bit-exact (every sum in the reference's order);
the post-module transformer and the upsample stage agree to ~1e-4 of the
largest value (split-f16 MFMA products are f32-accurate, sums in another
order); the decoder's convolutions take f16-rounded inputs as the reference
does, so a value that lands on the other side of an f16 rounding boundary
moves one input by one f16 ulp, and such moves compound over the decoder's
13 convolutions (measured: 1.7e-4, 3.8e-4, 7.7e-4, 1.1e-3 of the largest
value after blocks 1-4) -- checkpoints after each decoder block agree to
5e-3 of the largest value, inside the 1e-2 relative tolerance stated for f16
accumulation paths, while a layout or indexing mistake is O(1).
The waveform itself (tanh output in [-1, 1]) agrees to 1e-2 absolute at
worst and 1e-3 on average.  The full 512-frame decode (the bench workload) is
tied to the oracle-checked short decode by the causal-prefix property.
"""

import numpy as np
import pytest

from conftest import random_codes
from oracle import oracle as O
from s2hip import Codec, S2HipError

pytestmark = pytest.mark.gpu


def _rel(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / max(1e-30, np.max(np.abs(ref))))


@pytest.fixture(scope="module")
def codec(codec_gguf):
    print(f"[codec] open {codec_gguf} max_frames 64", flush=True)
    with Codec(codec_gguf, max_frames=64, device=0) as c:
        yield c


@pytest.fixture(scope="module")
def oracle(codec_gguf):
    with O.OracleCodec(codec_gguf) as c:
        yield c


def test_rvq_lookup_bit_exact(codec, oracle):
    for n in (1, 37, 64):
        codes = random_codes(n, seed=n)
        np.testing.assert_array_equal(codec.rvq_lookup(codes, 10, n), oracle.rvq_lookup(codes, 10, n))


def test_rvq_lookup_errors_match_reference_texts(codec):
    codes = random_codes(3, seed=5)
    with pytest.raises(S2HipError, match="codec codebook count mismatch: expected 10, got 9"):
        codec.rvq_lookup(codes[:9], 9, 3)
    bad = codes.copy()
    bad[2, 1] = -3
    with pytest.raises(S2HipError, match="codec code must be non-negative, got -3"):
        codec.rvq_lookup(bad, 10, 3)
    bad = codes.copy()
    bad[0, 2] = 4096
    with pytest.raises(S2HipError, match="embedding index 4096 out of range for vocab_dim 4096"):
        codec.decode_waveform(bad, 10, 3)
    with pytest.raises(S2HipError, match="codec transformer requires at least one frame"):
        codec.decode_waveform(np.zeros((10, 0), np.int32), 10, 0)
    with pytest.raises(S2HipError, match="exceeds the configured max_frames 64"):
        codec.rvq_lookup(random_codes(65, seed=6), 10, 65)
    with pytest.raises(S2HipError, match="decoder expects latent dim 1024, got 512"):
        codec.decoder(np.zeros((4, 512), np.float32))
    # the handle stays usable after errors
    codes = random_codes(2, seed=7)
    assert np.all(np.isfinite(codec.rvq_lookup(codes, 10, 2)))


def test_post_module_matches_oracle(codec, oracle):
    # 61 frames: more than one 64-query attention tile is not needed for the
    # window (128); the 133-frame case needs max_frames >= 133 (below)
    lat = oracle.rvq_lookup(random_codes(61, seed=8), 10, 61)
    got, ref = codec.post_module(lat), oracle.post_module(lat)
    assert _rel(got, ref) < 2e-4, _rel(got, ref)


def test_post_module_window_matches_oracle(codec_gguf, oracle):
    with Codec(codec_gguf, max_frames=140, device=0) as c:
        lat = oracle.rvq_lookup(random_codes(140, seed=9), 10, 140)
        got, ref = c.post_module(lat), oracle.post_module(lat)
    assert _rel(got, ref) < 2e-4, _rel(got, ref)


def test_upsample_matches_oracle(codec, oracle):
    rng = np.random.default_rng(10)
    for n in (1, 5, 64):
        hid = rng.standard_normal((n, 1024)).astype(np.float32)
        got, ref = codec.upsample(hid), oracle.upsample(hid)
        assert got.shape == (4 * n, 1024)
        assert _rel(got, ref) < 2e-4, (n, _rel(got, ref))


def test_decode_latents_composes_post_module_and_upsample(codec, oracle):
    lat = oracle.rvq_lookup(random_codes(6, seed=11), 10, 6)
    got = codec.decode_latents(lat)
    ref = oracle.upsample(oracle.post_module(lat))
    assert _rel(got, ref) < 3e-4, _rel(got, ref)


@pytest.mark.parametrize("frames", [3, 20])
def test_decoder_checkpoints_match_oracle(codec, oracle, frames):
    rng = np.random.default_rng(12 + frames)
    hid = rng.standard_normal((frames, 1024)).astype(np.float32)
    for stop in range(5):
        got, ref = codec.decoder(hid, stop), oracle.decoder(hid, stop)
        print(f"[codec] decoder frames {frames} stop_block {stop}: rel max err {_rel(got, ref):.2e}", flush=True)
        assert got.shape == ref.shape
        assert _rel(got, ref) < 5e-3, (stop, _rel(got, ref))
    got, ref = codec.decoder(hid), oracle.decoder(hid)
    err = np.abs(got - ref)
    print(f"[codec] decoder frames {frames} samples: max err {err.max():.2e}, mean {err.mean():.2e}", flush=True)
    assert got.shape == (frames * 512,)
    # samples lie in [-1, 1]: absolute bounds
    assert err.max() < 1e-2 and err.mean() < 1e-3, (err.max(), err.mean())


def test_decode_waveform_matches_oracle(codec, oracle):
    n = 16
    codes = random_codes(n, seed=13)
    res = codec.decode_waveform(codes, 10, n)
    assert (res.sample_rate, res.input_frames, res.latent_frames, res.num_samples) == (44100, n, 4 * n, n * 2048)
    ref = oracle.decode_waveform(codes, 10, n)
    err = np.abs(res.samples - ref)
    print(f"[codec] decode_waveform {n} frames: max err {err.max():.2e}, mean {err.mean():.2e}", flush=True)
    assert np.max(err) < 1e-2 and np.mean(err) < 1e-3, (np.max(err), np.mean(err))
    assert np.all(np.abs(res.samples) <= 1.0)


class _DeviceBuffer:
    """Device memory through the HIP runtime the library itself uses
    (libamdhip64, already loaded in the process by libs2hip.so)."""

    _hip = None

    def __init__(self, nbytes):
        import ctypes

        if _DeviceBuffer._hip is None:
            hip = ctypes.CDLL("libamdhip64.so")
            hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
            hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
            hip.hipFree.argtypes = [ctypes.c_void_p]
            hip.hipDeviceSynchronize.argtypes = []
            _DeviceBuffer._hip = hip
        self.ptr = ctypes.c_void_p()
        assert self._hip.hipMalloc(ctypes.byref(self.ptr), nbytes) == 0
        self.nbytes = nbytes

    def put(self, a):
        assert a.nbytes <= self.nbytes
        assert self._hip.hipMemcpy(self.ptr, a.ctypes.data, a.nbytes, 1) == 0  # host to device

    def get(self, a):
        assert self._hip.hipDeviceSynchronize() == 0
        assert self._hip.hipMemcpy(a.ctypes.data, self.ptr, a.nbytes, 2) == 0  # device to host
        return a

    def free(self):
        self._hip.hipFree(self.ptr)


def test_decode_waveform_device_equals_host_path(codec):
    n = 9
    codes = np.ascontiguousarray(random_codes(n, seed=14))
    host = codec.decode_waveform(codes, 10, n).samples
    d_codes, d_out = _DeviceBuffer(codes.nbytes), _DeviceBuffer(n * 2048 * 4)
    try:
        d_codes.put(codes)
        codec.decode_waveform_device(d_codes.ptr.value, 10, n, d_out.ptr.value)
        got = d_out.get(np.empty(n * 2048, np.float32))
        np.testing.assert_array_equal(got, host)
        bad = codes.copy()
        bad[4, 3] = 1024
        d_codes.put(bad)
        with pytest.raises(S2HipError, match="out of range"):
            codec.decode_waveform_device(d_codes.ptr.value, 10, n, d_out.ptr.value)
    finally:
        d_codes.free()
        d_out.free()


def test_full_size_decode_is_causal_extension_of_short_decode(codec_gguf, codec):
    """512 code frames (23.8 s of audio at 44.1 kHz, the bench workload): the
    first 16 frames' samples equal the 16-frame decode (checked against the
    oracle above) up to the post-module products' K split, which depends on
    the frame count."""
    codes = random_codes(512, seed=15)
    with Codec(codec_gguf, max_frames=512, device=0) as big:
        full = big.decode_waveform(codes, 10, 512).samples
    assert full.shape == (512 * 2048,)
    assert np.all(np.isfinite(full)) and np.all(np.abs(full) <= 1.0)
    head = codec.decode_waveform(np.ascontiguousarray(codes[:, :16]), 10, 16).samples
    d = np.abs(full[: 16 * 2048] - head)
    print(f"[codec] 512-frame decode vs 16-frame decode, shared samples: max diff {d.max():.2e}", flush=True)
    assert d.max() < 1e-2 and d.mean() < 1e-3, (d.max(), d.mean())
    # the signal is not degenerate over the whole length
    assert np.std(full[-2048 * 16:]) > 0.05


def test_codec_stage_dumps_pass_the_reference_comparators(codec, oracle):
    """The GPU codec's stage dumps (s2hip.dumps, the reference dump tools'
    schemas) against the same dumps of the oracle, under the reference
    comparators' default tolerances (s2hip.parity; fish_s2_parity
    compare-rvq-lookup / -post-module / -decode-stage / -waveform)."""
    from s2hip import dumps, parity

    n = 12
    codes = random_codes(n, seed=21)
    codes_dump = {"text": "hi", "num_codebooks": 10, "n_frames": n, "codes": codes.ravel().tolist()}
    lat = oracle.rvq_lookup(codes, 10, n)
    hid = oracle.post_module(lat)
    up = oracle.upsample(hid)
    wav = oracle.decode_waveform(codes, 10, n)
    base = {"backend": "rust", "text": "hi", "num_codebooks": 10}
    expect = {
        "rvq": {**base, "n_frames": n, "latent_dim": 1024, "latent_len": lat.size, **dumps.f64_stats("latent", lat)},
        "post": {**base, "n_frames": n, "hidden_dim": 1024, "hidden_len": hid.size, **dumps.f64_stats("hidden", hid)},
        "decode": {**base, "input_frames": n, "output_frames": 4 * n, "hidden_dim": 1024, "hidden_len": up.size,
                   **dumps.f64_stats("hidden", up)},
        "wave": {**base, "input_frames": n, "latent_frames": 4 * n, "sample_rate": 44100, "num_samples": wav.size,
                 **dumps.f64_stats("samples", wav)},
    }
    got = {"rvq": dumps.rvq_lookup_dump(codec, codes_dump), "post": dumps.post_module_dump(codec, codes_dump),
           "decode": dumps.decode_stage_dump(codec, codes_dump), "wave": dumps.waveform_dump(codec, codes_dump)}
    cmp = {"rvq": parity.compare_rvq_lookup_dumps, "post": parity.compare_post_module_dumps,
           "decode": parity.compare_decode_stage_dumps, "wave": parity.compare_waveform_dumps}
    for k in cmp:
        assert got[k]["backend"] == "rust-hip"
        r = cmp[k](expect[k], got[k])
        print(f"[codec] {k} dump: l2 {r.l2_delta:.2e} mean_abs {r.mean_abs_delta:.2e} max_abs {r.max_abs_delta:.2e} "
              f"first8 {r.first8_mae:.2e}", flush=True)
        assert r.passed, (k, r.failures)
    # the lookup is bit-exact, so its statistics are identical
    assert got["rvq"] == {**expect["rvq"], "backend": "rust-hip"}


def test_decode_waveform_to_wav_passes_the_reference_wav_parity(codec, oracle):
    """decode_waveform_to_wav (codec.rs:1716-1738): the GPU decode packed by
    pcm_to_wav against the oracle's samples packed the same way, under the
    reference's WAV comparator (fish_s2_parity compare)."""
    from s2hip import wav

    n = 20
    codes = random_codes(n, seed=22)
    got = codec.decode_waveform_to_wav(codes, 10, n)
    ref = wav.pcm_to_wav(oracle.decode_waveform(codes, 10, n), 44100)
    assert len(got) == len(ref) == 44 + 2 * n * 2048 and got[:44] == ref[:44]
    r = wav.compare_metrics(wav.metrics_from_wav_bytes(ref), wav.metrics_from_wav_bytes(got))
    d = np.abs(np.frombuffer(got[44:], "<i2").astype(np.int32) - np.frombuffer(ref[44:], "<i2"))
    print(f"[codec] wav: rms delta {r.rms_delta:.2e}, envelope MAE {r.envelope_mae:.2e}, "
          f"PCM LSB diff max {d.max()} mean {d.mean():.3f}", flush=True)
    assert r.passed, r.failures
    assert d.max() <= 330  # the waveform bound (1e-2) in 16-bit steps
