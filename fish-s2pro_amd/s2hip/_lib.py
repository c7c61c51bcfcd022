"""ctypes binding of libs2hip.so (the C ABI declared in include/s2hip.h).

There is no fallback: if the HIP library is missing or fails to load, every
entry point raises.  The product path never imports the CPU oracle.
"""

from __future__ import annotations

import ctypes
import os
import re

from . import _paths

ERR_CAP = 2048


class Config(ctypes.Structure):
    _fields_ = [
        ("gguf_path", ctypes.c_char_p),
        ("max_seq_len", ctypes.c_uint32),
        ("im_end_id", ctypes.c_uint32),
        ("device", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
    ]


class Spec(ctypes.Structure):
    _fields_ = [
        (n, ctypes.c_uint32)
        for n in (
            "slow_layers", "fast_layers", "dim", "ffn", "heads", "kv_heads", "head_dim",
            "fast_ffn", "fast_heads", "fast_kv_heads", "fast_head_dim", "vocab",
            "codebook_size", "num_codebooks", "semantic_begin", "semantic_end", "slow_qk_norm",
            "scale_codebook_embeddings", "linear_type", "max_seq_len",
        )
    ] + [(n, ctypes.c_float) for n in ("rope_base", "fast_rope_base", "eps", "fast_eps")] + [
        ("weight_bytes", ctypes.c_uint64)
    ]


class Sampler(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_p", ctypes.c_float), ("top_k", ctypes.c_int32)]


class GenParams(ctypes.Structure):
    _fields_ = [
        ("max_new_tokens", ctypes.c_uint32),
        ("temperature", ctypes.c_float),
        ("top_p", ctypes.c_float),
        ("top_k", ctypes.c_int32),
        ("min_tokens_before_end", ctypes.c_uint32),
    ]


class GenStats(ctypes.Structure):
    _fields_ = [
        ("prefill_ms", ctypes.c_double),
        ("decode_ms", ctypes.c_double),
        ("n_frames", ctypes.c_uint32),
        ("graph_used", ctypes.c_uint32),
        ("per_column_rerun", ctypes.c_uint32),
        ("greedy_rerun", ctypes.c_uint32),
    ]


FLAG_NO_GRAPH = 1
FLAG_KV_F16 = 2
FLAG_PROFILE = 4


class WaveformInfo(ctypes.Structure):
    _fields_ = [("sample_rate", ctypes.c_uint32), ("input_frames", ctypes.c_uint32),
                ("latent_frames", ctypes.c_uint32), ("num_samples", ctypes.c_size_t)]


class SlowProfile(ctypes.Structure):
    _fields_ = [(n, ctypes.c_double) for n in ("rms_norm_ms", "linear_ms", "gqa_attention_ms", "rope_ms",
                                               "kv_write_ms", "swiglu_ms", "output_head_ms")] + [
        ("steps", ctypes.c_uint32)]

_lib = None


def declared_functions():
    """Names of the functions include/s2hip.h declares."""
    text = open(os.path.join(_paths.INCLUDE_DIR, "s2hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(s2hip_[a-z0-9_]+)\s*\(", text)))


def load():
    global _lib
    if _lib is not None:
        return _lib
    path = _paths.hip_library()
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: the HIP extension must be built (__graft_entry__.build())")
    L = ctypes.CDLL(path)
    vp, sz, cp = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_char_p
    u32, i32, f32 = ctypes.c_uint32, ctypes.c_int32, ctypes.c_float
    u64p = ctypes.POINTER(ctypes.c_uint64)
    L.s2hip_version.argtypes = []
    L.s2hip_version.restype = cp
    L.s2hip_create.argtypes = [ctypes.POINTER(Config), cp, sz]
    L.s2hip_create.restype = vp
    L.s2hip_destroy.argtypes = [vp]
    L.s2hip_destroy.restype = None
    L.s2hip_get_spec.argtypes = [vp, ctypes.POINTER(Spec)]
    L.s2hip_reset.argtypes = [vp, cp, sz]
    L.s2hip_n_past.argtypes = [vp]
    L.s2hip_n_past.restype = u32
    L.s2hip_eval.argtypes = [vp, vp, sz, vp, vp, cp, sz]
    L.s2hip_fast_logits.argtypes = [vp, vp, vp, sz, vp, cp, sz]
    L.s2hip_fast_codebooks.argtypes = [vp, vp, u32, ctypes.POINTER(Sampler), u64p, vp, cp, sz]
    L.s2hip_generate_codes.argtypes = [vp, vp, sz, ctypes.POINTER(GenParams), u64p, vp,
                                       ctypes.POINTER(u32), ctypes.POINTER(GenStats), cp, sz]
    L.s2hip_generate_codes_batch.argtypes = [vp, u32, ctypes.POINTER(vp), ctypes.POINTER(sz),
                                             ctypes.POINTER(GenParams), u64p, ctypes.POINTER(vp),
                                             ctypes.POINTER(u32), ctypes.POINTER(GenStats), cp, sz]
    L.s2hip_op_linear.argtypes = [vp, vp, u32, sz, sz, vp, sz, vp, cp, sz]
    L.s2hip_op_rms_norm.argtypes = [vp, vp, vp, sz, sz, f32, vp, cp, sz]
    L.s2hip_op_dequant_rows.argtypes = [vp, vp, u32, sz, sz, vp, cp, sz]
    L.s2hip_op_qk_rope.argtypes = [vp, vp, u32, u32, u32, u32, f32, vp, vp, f32, vp, vp, vp, cp, sz]
    L.s2hip_op_attention.argtypes = [vp, vp, vp, vp, u32, u32, u32, u32, f32, vp, cp, sz]
    L.s2hip_op_swiglu.argtypes = [vp, vp, vp, sz, i32, vp, cp, sz]
    L.s2hip_op_sample.argtypes = [vp, vp, sz, ctypes.POINTER(Sampler), ctypes.c_int64, u64p,
                                  ctypes.POINTER(u32), cp, sz]
    L.s2hip_op_running_sums.argtypes = [vp, vp, sz, vp, ctypes.POINTER(f32), cp, sz]
    L.s2hip_op_running_cut.argtypes = [vp, vp, sz, f32, ctypes.c_int32, sz, ctypes.POINTER(sz), ctypes.POINTER(f32),
                                       ctypes.POINTER(f32), cp, sz]
    L.s2hip_op_sample_noalloc.argtypes = [vp, vp, sz, ctypes.POINTER(Sampler), ctypes.c_int64, u64p,
                                          ctypes.POINTER(u32), cp, sz]
    L.s2hip_device_allocations.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
    L.s2hip_device_allocations.restype = None
    L.s2hip_op_expf.argtypes = [vp, vp, sz, vp, cp, sz]
    L.s2hip_op_embed.argtypes = [vp, vp, sz, vp, cp, sz]
    L.s2hip_last_slow_profile.argtypes = [vp, ctypes.POINTER(SlowProfile)]
    L.s2hip_last_slow_profile.restype = i32
    L.s2hip_reset_slot.argtypes = [vp, u32, cp, sz]
    L.s2hip_n_past_slot.argtypes = [vp, u32]
    L.s2hip_n_past_slot.restype = u32
    L.s2hip_eval_slot.argtypes = [vp, u32, vp, sz, vp, vp, cp, sz]
    L.s2hip_transpose_to_time_major.argtypes = [vp, sz, u32, sz, vp, cp, sz]
    L.s2hip_expf_host.argtypes = [vp, sz, vp]
    L.s2hip_expf_host.restype = None
    L.s2hip_time_kernel.argtypes = [vp, cp, u32, ctypes.POINTER(ctypes.c_double),
                                    ctypes.POINTER(ctypes.c_double), cp, sz]
    for name in ("s2hip_get_spec", "s2hip_reset", "s2hip_eval", "s2hip_fast_logits",
                 "s2hip_fast_codebooks", "s2hip_generate_codes", "s2hip_generate_codes_batch",
                 "s2hip_op_linear",
                 "s2hip_op_rms_norm", "s2hip_op_dequant_rows", "s2hip_op_qk_rope",
                 "s2hip_op_attention", "s2hip_op_swiglu", "s2hip_op_sample", "s2hip_op_sample_noalloc",
                 "s2hip_op_running_sums",
                 "s2hip_op_running_cut",
                 "s2hip_op_expf", "s2hip_op_embed", "s2hip_reset_slot", "s2hip_eval_slot",
                 "s2hip_transpose_to_time_major", "s2hip_time_kernel"):
        getattr(L, name).restype = i32
    L.s2hip_codec_open.argtypes = [cp, u32, i32, cp, sz]
    L.s2hip_codec_open.restype = vp
    L.s2hip_codec_close.argtypes = [vp]
    L.s2hip_codec_close.restype = None
    L.s2hip_codec_rvq_lookup.argtypes = [vp, vp, u32, u32, vp, cp, sz]
    L.s2hip_codec_post_module.argtypes = [vp, vp, u32, vp, cp, sz]
    L.s2hip_codec_upsample.argtypes = [vp, vp, u32, vp, cp, sz]
    L.s2hip_codec_decode_latents.argtypes = [vp, vp, u32, vp, cp, sz]
    L.s2hip_codec_decoder.argtypes = [vp, vp, u32, u32, u32, vp, sz, ctypes.POINTER(sz), cp, sz]
    L.s2hip_codec_decode_waveform.argtypes = [vp, vp, u32, u32, vp, sz, ctypes.POINTER(WaveformInfo), cp, sz]
    L.s2hip_codec_decode_waveform_device.argtypes = [vp, vp, u32, u32, vp, cp, sz]
    L.s2hip_codec_snake_host.argtypes = [vp, sz, vp, vp]
    L.s2hip_codec_snake_host.restype = None
    L.s2hip_codec_time.argtypes = [vp, cp, u32, u32, ctypes.POINTER(ctypes.c_double),
                                   ctypes.POINTER(ctypes.c_double), cp, sz]
    for name in ("s2hip_codec_rvq_lookup", "s2hip_codec_post_module", "s2hip_codec_upsample",
                 "s2hip_codec_decode_latents", "s2hip_codec_decoder", "s2hip_codec_decode_waveform",
                 "s2hip_codec_decode_waveform_device", "s2hip_codec_time"):
        getattr(L, name).restype = i32
    _lib = L
    return L
