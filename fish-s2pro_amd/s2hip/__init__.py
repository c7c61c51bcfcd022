"""s2hip -- MI355X-native dual-AR (Slow-AR + Fast-AR) token loop and RVQ codec decode.

The compute path is libs2hip.so (HIP kernels for gfx950 behind the C ABI in
include/s2hip.h); this package is its host-side binding plus the seeded
synthetic-model writers.
"""

from .engine import Engine, S2HipError, transpose_to_time_major, version  # noqa: F401
from .codec import Codec, CodecWaveformResult  # noqa: F401
from . import synth  # noqa: F401
