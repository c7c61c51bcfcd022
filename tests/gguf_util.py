"""Minimal GGUF v3 writer for hand-built test models (F32 / F16 tensors).

Independent of the package's synthetic writer, like the reference's in-test
writer (crates/fish_s2_core/src/gguf.rs:678-705).
"""

import struct

import numpy as np

U32, F32, BOOL, STR = 4, 6, 7, 8


def _s(b: bytearray, text: str):
    raw = text.encode()
    b += struct.pack("<Q", len(raw)) + raw


def write(path, metadata, tensors):
    """metadata: list of (key, type, value); tensors: list of (name, dims(ne0 first), np.array)."""
    out = bytearray(b"GGUF")
    out += struct.pack("<IQQ", 3, len(tensors), len(metadata))
    for key, typ, val in metadata:
        _s(out, key)
        out += struct.pack("<I", typ)
        if typ == U32:
            out += struct.pack("<I", val)
        elif typ == F32:
            out += struct.pack("<f", val)
        elif typ == BOOL:
            out += struct.pack("<B", 1 if val else 0)
        elif typ == STR:
            _s(out, val)
    blobs, off = [], 0
    for name, dims, arr in tensors:
        arr = np.ascontiguousarray(arr)
        gtype = {np.dtype(np.float32): 0, np.dtype(np.float16): 1}[arr.dtype]
        _s(out, name)
        out += struct.pack("<I", len(dims))
        for d in dims:
            out += struct.pack("<Q", d)
        out += struct.pack("<IQ", gtype, off)
        raw = arr.tobytes()
        blobs.append(raw)
        off = (off + len(raw) + 31) // 32 * 32
    out += b"\0" * ((32 - len(out) % 32) % 32)
    for raw in blobs:
        out += raw
        out += b"\0" * ((32 - len(raw) % 32) % 32)
    with open(path, "wb") as f:
        f.write(out)


def toy_dual_ar(path, wqkv_rows, wo_rows, attention_norm, head_norm, eps=0.0):
    """One Slow layer with the reference's toy layer weights
    (crates/fish_s2_infer/src/slow_ar.rs:1283-1349, 1633-1680): hidden 4,
    2 q heads / 1 kv head, head_dim 2, FFN 2 (zero weights), RoPE base 1e4.
    Token 0 embeds to [1,0,0,0], token 1 to [1,1,0,0]."""
    d, ffn = 4, 2
    emb = np.zeros((4, d), np.float16)
    emb[0] = [1, 0, 0, 0]
    emb[1] = [1, 1, 0, 0]
    f32 = np.float32
    meta = [
        ("general.architecture", STR, "fish-speech"),
        ("fish-speech.context_length", U32, 16),
        ("fish-speech.embedding_length", U32, d),
        ("fish-speech.feed_forward_length", U32, ffn),
        ("fish-speech.block_count", U32, 1),
        ("fish-speech.attention.head_count", U32, 2),
        ("fish-speech.attention.head_count_kv", U32, 1),
        ("fish-speech.rope.freq_base", F32, 10000.0),
        ("fish-speech.attention.layer_norm_rms_epsilon", F32, eps),
        ("fish_speech.attention_qk_norm", BOOL, True),
        ("fish_speech.fast_context_length", U32, 2),
        ("fish_speech.fast_embedding_length", U32, d),
        ("fish_speech.fast_feed_forward_length", U32, ffn),
        ("fish_speech.fast_block_count", U32, 0),
        ("fish_speech.fast_head_count", U32, 2),
        ("fish_speech.fast_head_count_kv", U32, 1),
        ("fish_speech.fast_head_dim", U32, 2),
        ("fish_speech.fast_rope_freq_base", F32, 10000.0),
        ("fish_speech.fast_layer_norm_rms_eps", F32, eps),
        ("fish_speech.fast_attention_qk_norm", BOOL, False),
        ("fish_speech.codebook_size", U32, 1),
        ("fish_speech.num_codebooks", U32, 1),
        ("fish_speech.semantic_begin_id", U32, 2),
        ("fish_speech.semantic_end_id", U32, 3),
        ("fish_speech.scale_codebook_embeddings", BOOL, True),
        ("fish_speech.tie_word_embeddings", BOOL, True),
        ("fish_speech.fast_project_in", BOOL, False),
    ]
    tensors = [
        ("embeddings.weight", (d, 4), emb),
        ("codebook_embeddings.weight", (d, 1), np.zeros((1, d), np.float16)),
        ("norm.weight", (d,), np.ones(d, f32)),
        ("fast_embeddings.weight", (d, 1), np.zeros((1, d), np.float16)),
        ("fast_norm.weight", (d,), np.ones(d, f32)),
        ("fast_output.weight", (d, 1), np.zeros((1, d), f32)),
        ("layers.0.attention_norm.weight", (d,), np.asarray(attention_norm, f32)),
        ("layers.0.attention.q_norm.weight", (2,), np.asarray(head_norm, f32)),
        ("layers.0.attention.k_norm.weight", (2,), np.asarray(head_norm, f32)),
        ("layers.0.attention.wqkv.weight", (d, 8), np.asarray(wqkv_rows, f32)),
        ("layers.0.attention.wo.weight", (4, d), np.asarray(wo_rows, f32)),
        ("layers.0.ffn_norm.weight", (d,), np.ones(d, f32)),
        ("layers.0.feed_forward.w1.weight", (d, ffn), np.zeros((ffn, d), f32)),
        ("layers.0.feed_forward.w2.weight", (ffn, d), np.zeros((d, ffn), f32)),
        ("layers.0.feed_forward.w3.weight", (d, ffn), np.zeros((ffn, d), f32)),
    ]
    write(path, meta, tensors)


def toy_model(path, d, vocab, slow=None, fast=None, emb=None, cb_emb=None, fast_emb=None, fast_output=None,
              eps=0.0, fast_eps=0.0, rope_base=1e6, fast_rope_base=1e6, num_codebooks=1, codebook_size=1,
              semantic=(2, 3), heads=(2, 1, 2), fast_heads=(2, 1, 2), ffn=2, fast_ffn=2, qk_norm=True):
    """A hand-built dual-AR GGUF of width d with at most one Slow and one
    Fast layer.  slow / fast: dicts of the layer's tensors by suffix
    ("attention.wqkv.weight" [rows][d], "attention.wo.weight", "feed_forward.w1/w2/w3.weight",
    "attention_norm.weight", "ffn_norm.weight", and for Slow "attention.q_norm.weight" /
    "attention.k_norm.weight"); missing ones are zero (gains: one).  heads =
    (q heads, kv heads, head_dim)."""
    f32 = np.float32
    H, Hkv, hd = heads
    fH, fHkv, fhd = fast_heads

    def layer(prefix, spec, H, Hkv, hd, ffn, qk):
        spec = dict(spec or {})
        q, kv = H * hd, Hkv * hd
        shapes = {
            "attention_norm.weight": (d,), "ffn_norm.weight": (d,),
            "attention.wqkv.weight": (q + 2 * kv, d), "attention.wo.weight": (d, q),
            "feed_forward.w1.weight": (ffn, d), "feed_forward.w3.weight": (ffn, d),
            "feed_forward.w2.weight": (d, ffn),
        }
        if qk:
            shapes["attention.q_norm.weight"] = (hd,)
            shapes["attention.k_norm.weight"] = (hd,)
        out = []
        for suf, shp in shapes.items():
            if suf in spec:
                arr = np.asarray(spec[suf], f32).reshape(shp)
            elif len(shp) == 1:
                arr = np.ones(shp, f32)
            else:
                arr = np.zeros(shp, f32)
            out.append((f"{prefix}.0.{suf}", tuple(reversed(shp)), arr))
        return out

    meta = [
        ("general.architecture", STR, "fish-speech"),
        ("fish-speech.context_length", U32, 16),
        ("fish-speech.embedding_length", U32, d),
        ("fish-speech.feed_forward_length", U32, ffn),
        ("fish-speech.block_count", U32, 1),
        ("fish-speech.attention.head_count", U32, H),
        ("fish-speech.attention.head_count_kv", U32, Hkv),
        ("fish-speech.rope.freq_base", F32, rope_base),
        ("fish-speech.attention.layer_norm_rms_epsilon", F32, eps),
        ("fish_speech.attention_qk_norm", BOOL, qk_norm),
        ("fish_speech.fast_context_length", U32, num_codebooks + 1),
        ("fish_speech.fast_embedding_length", U32, d),
        ("fish_speech.fast_feed_forward_length", U32, fast_ffn),
        ("fish_speech.fast_block_count", U32, 1 if fast is not None else 0),
        ("fish_speech.fast_head_count", U32, fH),
        ("fish_speech.fast_head_count_kv", U32, fHkv),
        ("fish_speech.fast_head_dim", U32, fhd),
        ("fish_speech.fast_rope_freq_base", F32, fast_rope_base),
        ("fish_speech.fast_layer_norm_rms_eps", F32, fast_eps),
        ("fish_speech.fast_attention_qk_norm", BOOL, False),
        ("fish_speech.codebook_size", U32, codebook_size),
        ("fish_speech.num_codebooks", U32, num_codebooks),
        ("fish_speech.semantic_begin_id", U32, semantic[0]),
        ("fish_speech.semantic_end_id", U32, semantic[1]),
        ("fish_speech.scale_codebook_embeddings", BOOL, True),
        ("fish_speech.tie_word_embeddings", BOOL, True),
        ("fish_speech.fast_project_in", BOOL, False),
    ]

    def table(arr, rows):
        a = np.zeros((rows, d), np.float16) if arr is None else np.asarray(arr, np.float16).reshape(rows, d)
        return (tuple(reversed(a.shape)), a)

    cb_rows = num_codebooks * codebook_size
    tensors = [
        ("embeddings.weight",) + table(emb, vocab),
        ("codebook_embeddings.weight",) + table(cb_emb, cb_rows),
        ("norm.weight", (d,), np.ones(d, f32)),
        ("fast_embeddings.weight",) + table(fast_emb, codebook_size),
        ("fast_norm.weight", (d,), np.ones(d, f32)),
        ("fast_output.weight", (d, codebook_size),
         np.zeros((codebook_size, d), f32) if fast_output is None else np.asarray(fast_output, f32)),
    ]
    tensors += layer("layers", slow, H, Hkv, hd, ffn, qk_norm)
    if fast is not None:
        tensors += layer("fast_layers", fast, fH, fHkv, fhd, fast_ffn, False)
    write(path, meta, tensors)


def scale_rows(path, name, rows, factor):
    """Multiplies rows `rows` of the F16 matrix `name` ([ne1][ne0]) by
    `factor`, in place in the GGUF file."""
    raw = bytearray(open(path, "rb").read())
    off, dims, typ = _locate(raw, name)
    assert typ == 1 and len(dims) == 2, (name, typ, dims)
    ne0 = dims[0]
    mat = np.frombuffer(raw, np.float16, ne0 * dims[1], off).reshape(dims[1], ne0).copy()
    mat[rows] = (mat[rows].astype(np.float32) * factor).astype(np.float16)
    raw[off:off + mat.nbytes] = mat.tobytes()
    with open(path, "wb") as f:
        f.write(raw)


def copy_row(path, name, src, dst):
    """Row dst of the F16 matrix `name` := row src, in place in the GGUF file."""
    raw = bytearray(open(path, "rb").read())
    off, dims, typ = _locate(raw, name)
    assert typ == 1 and len(dims) == 2, (name, typ, dims)
    rb = dims[0] * 2
    raw[off + dst * rb:off + (dst + 1) * rb] = raw[off + src * rb:off + (src + 1) * rb]
    with open(path, "wb") as f:
        f.write(raw)


def _locate(raw, want):
    """(absolute data offset, dims ne0 first, ggml type) of tensor `want`."""
    pos = 4

    def get(fmt):
        nonlocal pos
        v = struct.unpack_from(fmt, raw, pos)
        pos += struct.calcsize(fmt)
        return v[0]

    def gstr():
        n = get("<Q")
        nonlocal pos
        s = bytes(raw[pos:pos + n]).decode()
        pos += n
        return s

    sizes = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}

    def skip(t):
        nonlocal pos
        if t == 8:
            gstr()
        elif t == 9:
            et, n = get("<I"), get("<Q")
            for _ in range(n):
                skip(et)
        else:
            pos += sizes[t]

    _ver, n_t, n_kv = get("<I"), get("<Q"), get("<Q")
    for _ in range(n_kv):
        gstr()
        skip(get("<I"))
    found = None
    for _ in range(n_t):
        name = gstr()
        nd = get("<I")
        dims = [get("<Q") for _ in range(nd)]
        typ, off = get("<I"), get("<Q")
        if name == want:
            found = (off, dims, typ)
    start = (pos + 31) // 32 * 32
    assert found is not None, want
    return start + found[0], found[1], found[2]


def read_tensors(path):
    """name -> numpy array ([ne1][ne0] for matrices) for F32 / F16 tensors."""
    raw = open(path, "rb").read()
    pos = 4

    def get(fmt):
        nonlocal pos
        v = struct.unpack_from(fmt, raw, pos)
        pos += struct.calcsize(fmt)
        return v[0]

    def gstr():
        n = get("<Q")
        nonlocal pos
        s = raw[pos:pos + n].decode()
        pos += n
        return s

    sizes = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}

    def skip(t):
        nonlocal pos
        if t == 8:
            gstr()
        elif t == 9:
            et, n = get("<I"), get("<Q")
            for _ in range(n):
                skip(et)
        else:
            pos += sizes[t]

    _ver, n_t, n_kv = get("<I"), get("<Q"), get("<Q")
    for _ in range(n_kv):
        gstr()
        skip(get("<I"))
    infos = []
    for _ in range(n_t):
        name = gstr()
        nd = get("<I")
        dims = [get("<Q") for _ in range(nd)]
        infos.append((name, dims, get("<I"), get("<Q")))
    start = (pos + 31) // 32 * 32
    out = {}
    for name, dims, typ, off in infos:
        if typ not in (0, 1):
            continue
        dt = np.float32 if typ == 0 else np.float16
        n = int(np.prod(dims))
        arr = np.frombuffer(raw, dt, n, start + off)
        out[name] = arr.reshape(list(reversed(dims))) if len(dims) > 1 else arr
    return out
