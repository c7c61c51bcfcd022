"""CPU-only checks: golden fixtures, the synthetic GGUF writer, and that the
C-ABI library loads and exports every symbol include/s2hip.h declares (no
compute call is made: there is no GPU here)."""

import ctypes
import hashlib
import json
import os

import numpy as np
import pytest

from oracle import oracle as O
from s2hip import _lib, _paths, synth

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = json.load(open(os.path.join(HERE, "golden", "tiny_greedy_codes.json")))


def _sha(path):
    return hashlib.sha256(open(path, "rb").read()).hexdigest()


def test_synthetic_writer_is_deterministic(tiny_gguf, tiny_q8_gguf, tiny_q4_gguf):
    assert _sha(tiny_gguf) == GOLD["gguf_sha256"]["tiny_f16"]
    assert _sha(tiny_q8_gguf) == GOLD["gguf_sha256"]["tiny_q8_0"]
    assert _sha(tiny_q4_gguf) == GOLD["gguf_sha256"]["tiny_q4_0"]


def test_oracle_reproduces_golden_codes(tiny_gguf):
    m = O.OracleModel(tiny_gguf, 64, synth.TINY.im_end_id)
    r = m.generate_codes(np.array(GOLD["prompt_flat"], np.int32), GOLD["max_new_tokens"], 0.0, 1.0, 0,
                         GOLD["min_tokens_before_end"], GOLD["rng_seed"])
    assert r["codes"].tolist() == GOLD["codes"] and r["rng_state"] == GOLD["rng_state"]


def test_synthetic_weights_statistics(tiny_gguf):
    import gguf_util

    t = gguf_util.read_tensors(tiny_gguf)
    emb = t["embeddings.weight"]
    assert emb.shape == (8192, 512) and emb.dtype == np.float16
    assert abs(float(emb.astype(np.float64).std()) - 0.02) < 2e-4
    assert abs(float(emb.astype(np.float64).mean())) < 2e-4
    assert (t["norm.weight"] == 1).all() and (t["layers.0.attention.q_norm.weight"] == 1).all()
    w = t["layers.3.feed_forward.w2.weight"]
    assert w.shape == (512, 1536) and abs(float(w.astype(np.float64).std()) - 0.02) < 4e-4


@pytest.mark.parametrize("gtype", [synth.GGML_Q8_0, synth.GGML_Q4_0])
def test_quantizer_error_bound(gtype):
    rng = np.random.default_rng(0)
    for _ in range(200):
        x = (rng.standard_normal(32) * 0.02).astype(np.float32)
        blk = synth.quantize_block(gtype, x)
        y = O.dequant_row(blk, gtype, 32)
        amax = np.abs(x).max()
        if gtype == synth.GGML_Q8_0:
            step = amax / 127.0  # rounding to nearest + f16 rounding of d (rel 2^-11) on |q| <= 127
            bound = 0.5 * step + 127 * step * 2.0 ** -10
        else:
            step = amax / 8.0  # the clamp at 15 costs one step on the side opposite the max
            bound = 1.0 * step + 8 * step * 2.0 ** -10
        assert np.max(np.abs(x - y)) <= bound


def test_f16_writer_matches_numpy():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(5000) * 0.02, rng.standard_normal(500) * 1e-6]).astype(np.float32)
    got = np.array([synth._load().s2synth_f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, x.astype(np.float16).view(np.uint16))


def test_library_exports_every_declared_symbol():
    L = _lib.load()
    declared = _lib.declared_functions()
    assert len(declared) >= 17
    missing = [f for f in declared if not hasattr(L, f)]
    assert not missing
    assert L.s2hip_version().decode().startswith("s2hip")


def test_library_has_gfx950_code_object():
    # the fat binary embedded in the library names its offload target
    assert b"amdgcn-amd-amdhsa--gfx950" in open(_paths.hip_library(), "rb").read()


def test_create_rejects_bad_config_without_gpu():
    L = _lib.load()
    err = ctypes.create_string_buffer(256)
    assert not L.s2hip_create(None, err, len(err))
    assert b"NULL" in err.value
    # a NULL engine fails with a message, not a silent 0
    err2 = ctypes.create_string_buffer(256)
    assert L.s2hip_reset(None, err2, len(err2)) == 0 and b"NULL" in err2.value
    # the allocation counter answers without a device
    c = ctypes.c_uint64(123)
    L.s2hip_device_allocations(ctypes.byref(c))
    assert c.value == 0


# Algorithmic HBM bytes per launch of each profiled w13 kernel: w1 and w3
# rows (9728 x 2560 weights each, at 2 B, 34/32 B or 2 B per weight), plus
# the f32 input and output columns.
_W13_ALGO_BYTES = {
    ("slow_w13", "full"): 2 * 9728 * 2560 * 2 + 2560 * 4 + 9728 * 4,
    ("slow_w13", "full_q8"): 2 * 9728 * 80 * 34 + 2560 * 4 + 9728 * 4,
    ("slow_w13_b8", "full_b8"): 2 * 9728 * 2560 * 2 + 8 * (2560 + 9728) * 4,
}


@pytest.mark.parametrize("kernel,workload", sorted(_W13_ALGO_BYTES))
def test_committed_counter_summaries_parse_and_match_algorithmic_bytes(kernel, workload):
    # bench.py reports FETCH_SIZE + WRITE_SIZE from these summaries as
    # roofline.traffic; a kernel streaming its weights once reads within a few
    # percent of its algorithmic bytes
    import bench

    traffic = bench.counter_traffic(kernel, workload)
    assert traffic is not None, f"profiles/counters_{kernel}_{workload}.txt missing or malformed"
    algo = _W13_ALGO_BYTES[(kernel, workload)]
    assert 0.99 * algo <= traffic <= 1.05 * algo, (traffic, algo)


def _create_err(path):
    L = _lib.load()
    err = ctypes.create_string_buffer(512)
    cfg = _lib.Config(path.encode(), 16, 0, 0, 0)
    h = L.s2hip_create(ctypes.byref(cfg), err, len(err))
    assert not h
    return err.value.decode()


def test_malformed_gguf_headers_fail_by_name(tmp_path):
    """The GGUF header is validated on the host before any device call:
    element counts and offsets that would wrap 64 bits fail with the tensor's
    name (the reference's checked_mul / checked_add, gguf.rs:161,254,351)."""
    import struct

    import gguf_util

    base = str(tmp_path / "ok.gguf")
    gguf_util.write(base, [("general.architecture", gguf_util.STR, "fish-speech")],
                    [("a.weight", (4, 2), np.zeros((2, 4), np.float32))])
    raw = bytearray(open(base, "rb").read())
    name = b"a.weight"
    at = raw.index(name) + len(name)  # then n_dims u32, dims u64 x2, type u32, offset u64
    # dims whose product wraps to a small number: 2^33 x 2^31 = 2^64 -> 0
    bad = bytearray(raw)
    struct.pack_into("<QQ", bad, at + 4, 1 << 33, 1 << 31)
    p = str(tmp_path / "dims.gguf")
    open(p, "wb").write(bad)
    assert "a.weight" in _create_err(p) and "overflow" in _create_err(p)
    # an offset that wraps past the end of the address space
    bad = bytearray(raw)
    struct.pack_into("<Q", bad, at + 4 + 16 + 4, (1 << 64) - 16)
    p = str(tmp_path / "offset.gguf")
    open(p, "wb").write(bad)
    assert "a.weight extends past file end" in _create_err(p)
    # an offset just past the data
    bad = bytearray(raw)
    struct.pack_into("<Q", bad, at + 4 + 16 + 4, 64)
    p = str(tmp_path / "past.gguf")
    open(p, "wb").write(bad)
    assert "a.weight extends past file end" in _create_err(p)


def test_transpose_to_time_major_matches_reference_kat_and_oracle():
    from s2hip import S2HipError, transpose_to_time_major

    # prompt.rs:289-303 (transpose_matches_time_major_layout)
    assert transpose_to_time_major([10, 20, 1, 2, 3, 4], 3, 2).tolist() == [10, 1, 3, 20, 2, 4]
    # against the oracle's restatement on a prompt-shaped tensor (11 x 61)
    rng = np.random.default_rng(3)
    data = rng.integers(0, 155776, (11, 61)).astype(np.uint32)
    got = transpose_to_time_major(data, 11, 61)
    assert np.array_equal(got, O.transpose_to_time_major(data.ravel(), 11, 61))
    assert np.array_equal(got.reshape(61, 11), data.T.astype(np.int32))
    # the reference's errors
    with pytest.raises(S2HipError, match="prompt rows must be non-zero"):
        transpose_to_time_major([], 0, 0)
    with pytest.raises(S2HipError, match="prompt data length mismatch: expected 6, got 5"):
        transpose_to_time_major([1, 2, 3, 4, 5], 3, 2)
    with pytest.raises(S2HipError, match="does not fit i32"):
        transpose_to_time_major([1, 2 ** 31], 1, 2)
    assert transpose_to_time_major([], 3, 0).size == 0


def test_codec_snake_routine_matches_glibc_snake():
    """The device snake (sin^2 by Cody-Waite reduction + minimax polynomials,
    csrc/sin_cw.h), built for the host, against the oracle's snake (glibc
    sinf, snake_activation_frame_major codec.rs:2162-2186): mostly the same
    bits, never more than 4 ulp of the larger of x and sin^2(a x) / a."""
    L = _lib.load()
    rng = np.random.default_rng(0)
    x = np.concatenate([np.linspace(-1024, 1024, 400_001), rng.standard_normal(200_000) * 30]).astype(np.float32)
    a = np.where(rng.random(x.size) < 0.5, rng.uniform(0.5, 1.5, x.size), rng.uniform(-2, 2, x.size)).astype(np.float32)
    a[::97] = 0.0  # the |a| < 1e-8 guard
    y = np.empty_like(x)
    L.s2hip_codec_snake_host(x.ctypes.data, x.size, a.ctypes.data, y.ctypes.data)
    ref = O.codec_snake(x.reshape(1, -1), a).reshape(-1)
    ae = np.where(np.abs(a) < 1e-8, 1e-8, a).astype(np.float64)
    scale = np.maximum(np.abs(x), np.sin(ae * x) ** 2 / np.abs(ae)).astype(np.float32)
    err = np.abs(y.astype(np.float64) - ref) / np.spacing(scale)
    assert np.max(err) <= 4.0, np.max(err)
    assert np.mean(y == ref) > 0.98
