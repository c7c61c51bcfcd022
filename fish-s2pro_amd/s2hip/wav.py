"""WAV output of the decoded waveform and the reference's WAV parity metrics.

* `pcm_to_wav` restates crates/fish_s2_infer/src/wav.rs:7-39: a 44-byte
  RIFF/WAVE header (PCM, mono, 16 bits), then each sample clamped to [-1, 1],
  multiplied by 32767 in f32 and truncated toward zero to i16.
* `metrics_from_wav_bytes` / `compare_metrics` restate the WAV parity of
  crates/fish_s2_parity/src/lib.rs:1712-1944 (chunk parser, PCM 8/16/24/32 and
  float32 decode, RMS, peak, duration, 50 ms RMS envelope, envelope MAE over
  a common resampling), with the same tolerances and failure texts;
  `python -m s2hip.parity metrics|compare` prints them like `fish_s2_parity`.
"""

from __future__ import annotations

import math
import struct
from dataclasses import dataclass, field
from typing import List

import numpy as np


def pcm_to_wav(samples, sample_rate: int) -> bytes:
    s = np.ascontiguousarray(samples, np.float32).ravel()
    clamped = np.clip(np.nan_to_num(s, nan=0.0), np.float32(-1.0), np.float32(1.0))
    pcm = (clamped * np.float32(32767.0)).astype(np.int16)  # truncation toward zero, as `as i16`
    data_size = pcm.size * 2
    header = b"RIFF" + struct.pack("<I", 44 + data_size) + b"WAVE" + b"fmt " + struct.pack(
        "<IHHIIHH", 16, 1, 1, sample_rate, sample_rate * 2, 2, 16) + b"data" + struct.pack("<I", data_size)
    return header + pcm.astype("<i2").tobytes()


class WavError(ValueError):
    pass


@dataclass
class WavMetrics:
    sample_rate: int
    channels: int
    bits_per_sample: int
    duration_seconds: float
    rms: float
    peak: float
    envelope_rms: List[float] = field(default_factory=list)


@dataclass(frozen=True)
class WavTolerance:
    """ParityTolerance::default (lib.rs:28-36)."""
    max_duration_delta_seconds: float = 0.10
    max_rms_delta: float = 0.03
    max_envelope_mae: float = 0.04


@dataclass
class WavReport:
    passed: bool
    duration_delta_seconds: float
    rms_delta: float
    envelope_mae: float
    failures: List[str]


def _parse(b: bytes):
    if len(b) < 12 or b[0:4] != b"RIFF" or b[8:12] != b"WAVE":
        raise WavError("not a RIFF/WAVE file")
    pos, fmt, data = 12, None, None
    while pos + 8 <= len(b):
        cid = b[pos:pos + 4]
        size = struct.unpack_from("<I", b, pos + 4)[0]
        pos += 8
        if pos + size > len(b):
            raise WavError("truncated WAV chunk")
        chunk = b[pos:pos + size]
        if cid == b"fmt ":
            if len(chunk) < 16:
                raise WavError("fmt chunk too short")
            fmt = struct.unpack_from("<HHI", chunk, 0) + struct.unpack_from("<HH", chunk, 12)
        elif cid == b"data":
            data = chunk
        pos += size + (size % 2)
    if fmt is None:
        raise WavError("missing fmt chunk")
    if data is None:
        raise WavError("missing data chunk")
    audio_format, channels, sample_rate, block_align, bits = fmt
    if channels == 0 or sample_rate == 0 or block_align == 0:
        raise WavError("invalid WAV format values")
    return audio_format, channels, sample_rate, block_align, bits, data


def _decode(audio_format, bits, data) -> np.ndarray:
    def aligned(width):
        if len(data) % width:
            raise WavError("WAV data is not sample-aligned")
    if (audio_format, bits) == (1, 8):
        return (np.frombuffer(data, np.uint8).astype(np.float32) - np.float32(128.0)) / np.float32(128.0)
    if (audio_format, bits) == (1, 16):
        aligned(2)
        return np.frombuffer(data, "<i2").astype(np.float32) / np.float32(32768.0)
    if (audio_format, bits) == (1, 24):
        aligned(3)
        a = np.frombuffer(data, np.uint8).reshape(-1, 3).astype(np.int32)
        v = a[:, 0] | (a[:, 1] << 8) | (a[:, 2] << 16)
        v = np.where(v & 0x800000, v - (1 << 24), v)
        return v.astype(np.float32) / np.float32(8388608.0)
    if (audio_format, bits) == (1, 32):
        aligned(4)
        return np.frombuffer(data, "<i4").astype(np.float32) / np.float32(2147483648.0)
    if (audio_format, bits) == (3, 32):
        aligned(4)
        return np.clip(np.frombuffer(data, "<f4"), np.float32(-1.0), np.float32(1.0))
    raise WavError(f"unsupported WAV format: audio_format={audio_format}, bits_per_sample={bits}")


def metrics_from_wav_bytes(b: bytes, frame_ms: int = 50) -> WavMetrics:
    audio_format, channels, sample_rate, block_align, bits, data = _parse(b)
    s = _decode(audio_format, bits, data)
    if s.size == 0:
        raise WavError("WAV contains no samples")
    x = s.astype(np.float64)
    rms = math.sqrt(float(np.cumsum(x * x)[-1]) / s.size)
    peak = float(max(np.float32(0.0), np.max(np.abs(s))))
    duration = (len(data) / block_align) / sample_rate
    per = max(1, (sample_rate * channels * frame_ms) // 1000)
    env = [math.sqrt(float(np.cumsum(x[i:i + per] * x[i:i + per])[-1]) / len(x[i:i + per]))
           for i in range(0, x.size, per)]
    return WavMetrics(sample_rate, channels, bits, duration, rms, peak, env)


def _sample_envelope(values, pos):
    if not values:
        return 0.0
    if len(values) == 1:
        return values[0]
    scaled = min(max(pos, 0.0), 1.0) * (len(values) - 1)
    lo, hi = math.floor(scaled), math.ceil(scaled)
    if lo == hi:
        return values[lo]
    t = scaled - lo
    return values[lo] * (1.0 - t) + values[hi] * t


def envelope_mae(expected, actual) -> float:
    n = max(len(expected), len(actual))
    if n == 0:
        return 0.0
    total = 0.0
    for i in range(n):
        pos = 0.0 if n == 1 else i / (n - 1)
        total += abs(_sample_envelope(expected, pos) - _sample_envelope(actual, pos))
    return total / n


def compare_metrics(expected: WavMetrics, actual: WavMetrics, tolerance: WavTolerance = WavTolerance()) -> WavReport:
    dd = abs(expected.duration_seconds - actual.duration_seconds)
    rd = abs(expected.rms - actual.rms)
    em = envelope_mae(expected.envelope_rms, actual.envelope_rms)
    f = []
    if expected.sample_rate != actual.sample_rate:
        f.append(f"sample rate mismatch: expected {expected.sample_rate}, actual {actual.sample_rate}")
    if expected.channels != actual.channels:
        f.append(f"channel count mismatch: expected {expected.channels}, actual {actual.channels}")
    if dd > tolerance.max_duration_delta_seconds:
        f.append(f"duration delta {dd:.4f}s exceeds {tolerance.max_duration_delta_seconds:.4f}s")
    if rd > tolerance.max_rms_delta:
        f.append(f"RMS delta {rd:.6f} exceeds {tolerance.max_rms_delta:.6f}")
    if em > tolerance.max_envelope_mae:
        f.append(f"envelope MAE {em:.6f} exceeds {tolerance.max_envelope_mae:.6f}")
    return WavReport(not f, dd, rd, em, f)
