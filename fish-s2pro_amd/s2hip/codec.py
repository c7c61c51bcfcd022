"""Host-side mirror of the reference's RVQ codec decode over the s2hip C ABI.

``Codec`` plays the part of the codec weights plus the decode functions of
crates/fish_s2_infer/src/codec.rs -- ``decode_waveform`` (:1690-1714),
``rvq_lookup_codes`` (:2536-2596), ``rvq_decode_latents`` (:1282-1297),
``forward_codec_post_module`` (:986-1018), ``forward_codec_upsample``
(:2302-2325) and ``forward_codec_decoder`` (:1941-2001) -- with the same
argument meaning and error texts; failures raise ``S2HipError``.  Arrays are
frame-major float32; codes are codebook-major int32 [num_codebooks][n_frames].
The computation runs in libs2hip.so on the GPU; there is no CPU fallback.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from .engine import S2HipError

HIDDEN = 1024
SAMPLE_RATE = 44100
SAMPLES_PER_CODE_FRAME = 2048
SAMPLES_PER_LATENT_FRAME = 512


@dataclass
class CodecWaveformResult:
    """codec.rs:1681-1688"""
    sample_rate: int
    input_frames: int
    latent_frames: int
    num_samples: int
    samples: np.ndarray


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class Codec:
    def __init__(self, gguf_path: str, max_frames: int, device: int = 0):
        """max_frames: the most code frames one call decodes (buffers are
        sized for it once)."""
        L = _lib.load()
        err = ctypes.create_string_buffer(_lib.ERR_CAP)
        h = L.s2hip_codec_open(gguf_path.encode(), max_frames, device, err, len(err))
        if not h:
            raise S2HipError(err.value.decode())
        self._h, self._L, self.max_frames = h, L, max_frames

    def close(self):
        if getattr(self, "_h", None):
            self._L.s2hip_codec_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _call(self, fn, *args):
        err = ctypes.create_string_buffer(_lib.ERR_CAP)
        if not fn(self._h, *args, err, len(err)):
            raise S2HipError(err.value.decode())

    @staticmethod
    def _codes(codes, num_codebooks, n_frames):
        c = np.ascontiguousarray(codes, dtype=np.int32).ravel()
        if c.size != num_codebooks * n_frames:
            raise S2HipError(f"codec codes length mismatch: expected {num_codebooks * n_frames}, got {c.size}")
        return c

    def rvq_lookup(self, codes, num_codebooks: int, n_frames: int) -> np.ndarray:
        c = self._codes(codes, num_codebooks, n_frames)
        out = np.empty((n_frames, HIDDEN), np.float32)
        self._call(self._L.s2hip_codec_rvq_lookup, c.ctypes.data, num_codebooks, n_frames, out.ctypes.data)
        return out

    def post_module(self, latents) -> np.ndarray:
        x = _f32(latents)
        out = np.empty_like(x)
        self._call(self._L.s2hip_codec_post_module, x.ctypes.data, x.shape[0], out.ctypes.data)
        return out

    def upsample(self, hidden) -> np.ndarray:
        x = _f32(hidden)
        out = np.empty((4 * x.shape[0], HIDDEN), np.float32)
        self._call(self._L.s2hip_codec_upsample, x.ctypes.data, x.shape[0], out.ctypes.data)
        return out

    def decode_latents(self, latents) -> np.ndarray:
        x = _f32(latents)
        out = np.empty((4 * x.shape[0], HIDDEN), np.float32)
        self._call(self._L.s2hip_codec_decode_latents, x.ctypes.data, x.shape[0], out.ctypes.data)
        return out

    def decoder(self, hidden, stop_block: int = 5) -> np.ndarray:
        """Samples (stop_block 5), or the residual stream after stop_block
        (0..4) decoder blocks."""
        x = _f32(hidden)
        rates, ch = (8, 8, 4, 2), (1536, 768, 384, 192, 96)
        if stop_block >= 5:
            shape = (x.shape[0] * SAMPLES_PER_LATENT_FRAME,)
        else:
            shape = (x.shape[0] * int(np.prod(rates[:stop_block])), ch[stop_block])
        out = np.empty(shape, np.float32)
        n = ctypes.c_size_t(0)
        self._call(self._L.s2hip_codec_decoder, x.ctypes.data, x.shape[0], x.shape[1] if x.ndim == 2 else 0,
                   stop_block, out.ctypes.data, out.size, ctypes.byref(n))
        return out

    def decode_waveform(self, codes, num_codebooks: int, n_frames: int) -> CodecWaveformResult:
        c = self._codes(codes, num_codebooks, n_frames)
        out = np.empty(max(n_frames, 0) * SAMPLES_PER_CODE_FRAME, np.float32)
        info = _lib.WaveformInfo()
        self._call(self._L.s2hip_codec_decode_waveform, c.ctypes.data, num_codebooks, n_frames,
                   out.ctypes.data, out.size, ctypes.byref(info))
        return CodecWaveformResult(info.sample_rate, info.input_frames, info.latent_frames, info.num_samples, out)

    def decode_waveform_to_wav(self, codes, num_codebooks: int, n_frames: int) -> bytes:
        """decode_waveform_to_wav (codec.rs:1716-1738): the decode, then
        pcm_to_wav (wav.rs:7-39) on the host."""
        from .wav import pcm_to_wav

        w = self.decode_waveform(codes, num_codebooks, n_frames)
        return pcm_to_wav(w.samples[: w.num_samples], w.sample_rate)

    def decode_waveform_device(self, codes_ptr: int, num_codebooks: int, n_frames: int, samples_ptr: int):
        """Device pointers (e.g. torch tensors' data_ptr() on the codec's device)."""
        self._call(self._L.s2hip_codec_decode_waveform_device, ctypes.c_void_p(codes_ptr), num_codebooks,
                   n_frames, ctypes.c_void_p(samples_ptr))

    def time(self, what: str, n_frames: int, reps: int):
        """(average microseconds per launch, flops per launch) of `what`
        ("decode" or a convolution's name), timed with HIP events."""
        us, fl = ctypes.c_double(0), ctypes.c_double(0)
        self._call(self._L.s2hip_codec_time, what.encode(), n_frames, reps, ctypes.byref(us), ctypes.byref(fl))
        return us.value, fl.value
