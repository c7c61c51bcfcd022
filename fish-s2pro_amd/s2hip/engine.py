"""Host-side mirror of the reference's dual-AR interface over the s2hip C ABI.

``Engine`` plays the part of the reference's ``SlowArState`` +
``FastArWeights`` + ``generate_codes`` (crates/fish_s2_infer/src/slow_ar.rs:372-528,
fast_ar.rs:195-470, generate.rs:117-221) with the same argument meaning and
error behaviour: invalid shapes, out-of-range ids and KV overflow raise
``S2HipError`` carrying the library's message.  The op-level methods mirror the
``MatmulBackend`` seam (crates/fish_s2_infer/src/backend.rs:5-39).
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib


class S2HipError(RuntimeError):
    pass


def _p(a: np.ndarray):
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class Engine:
    def __init__(self, gguf_path: str, max_seq_len: int, im_end_id: int, device: int = 0,
                 use_graph: bool = True, kv_f16: bool = False, profile: bool = False):
        """kv_f16: store the Slow-AR KV cache as f16 (S2HIP_FLAG_KV_F16).
        profile: collect the SlowArDecodeProfile counterpart of each generate
        call (S2HIP_FLAG_PROFILE; frames then run without graph replay)."""
        L = _lib.load()
        flags = ((0 if use_graph else _lib.FLAG_NO_GRAPH) | (_lib.FLAG_KV_F16 if kv_f16 else 0) |
                 (_lib.FLAG_PROFILE if profile else 0))
        cfg = _lib.Config(gguf_path.encode(), max_seq_len, im_end_id, device, flags)
        err = ctypes.create_string_buffer(_lib.ERR_CAP)
        h = L.s2hip_create(ctypes.byref(cfg), err, len(err))
        if not h:
            raise S2HipError(err.value.decode())
        self._h = h
        self._L = L
        self.im_end_id = im_end_id
        sp = _lib.Spec()
        L.s2hip_get_spec(h, ctypes.byref(sp))
        self.spec = {f[0]: getattr(sp, f[0]) for f in _lib.Spec._fields_}
        self.codebook_dim = self.spec["num_codebooks"] + 1

    # -- lifetime -----------------------------------------------------------
    def close(self):
        if getattr(self, "_h", None):
            self._L.s2hip_destroy(self._h)
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

    # -- SlowArState ----------------------------------------------------------
    def reset(self, slot: int = 0):
        """SlowArState::reset (slow_ar.rs:434-438) of KV slot `slot`."""
        if slot == 0:
            self._call(self._L.s2hip_reset)
        else:
            self._call(self._L.s2hip_reset_slot, slot)

    @property
    def n_past(self) -> int:
        return int(self._L.s2hip_n_past(self._h))

    def last_slow_profile(self) -> dict:
        """SlowArDecodeProfile (slow_ar.rs:248-319) of the last generate call, in
        milliseconds per operation (all zero without profile=True)."""
        p = _lib.SlowProfile()
        self._L.s2hip_last_slow_profile(self._h, ctypes.byref(p))
        return {f[0]: getattr(p, f[0]) for f in _lib.SlowProfile._fields_}

    def n_past_slot(self, slot: int) -> int:
        return int(self._L.s2hip_n_past_slot(self._h, slot))

    def eval_slot(self, slot: int, flat_tokens, want_logits: bool = True):
        """eval on KV slot `slot` (0..15); slot 0 is the state eval uses."""
        flat = np.ascontiguousarray(flat_tokens, dtype=np.int32).ravel()
        if flat.size % self.codebook_dim:
            raise S2HipError(
                f"flat token length {flat.size} is not a multiple of codebook_dim {self.codebook_dim}")
        hidden = np.zeros(self.spec["dim"], np.float32)
        logits = np.zeros(self.spec["vocab"], np.float32) if want_logits else None
        self._call(self._L.s2hip_eval_slot, slot, _p(flat), flat.size // self.codebook_dim, _p(hidden),
                   _p(logits) if want_logits else None)
        return hidden, logits

    def embed(self, flat_tokens):
        """embed_slow_ar_time_major (slow_ar.rs:1041-1133) on the device:
        [n_tokens][dim] f32 for time-major flat ids."""
        flat = np.ascontiguousarray(flat_tokens, dtype=np.int32).ravel()
        if flat.size % self.codebook_dim:
            raise S2HipError(
                f"flat token length {flat.size} is not a multiple of codebook_dim {self.codebook_dim}")
        n = flat.size // self.codebook_dim
        out = np.zeros((n, self.spec["dim"]), np.float32)
        self._call(self._L.s2hip_op_embed, _p(flat), n, _p(out))
        return out

    def eval(self, flat_tokens, want_logits: bool = True):
        flat = np.ascontiguousarray(flat_tokens, dtype=np.int32).ravel()
        if flat.size % self.codebook_dim:
            raise S2HipError(
                f"flat token length {flat.size} is not a multiple of codebook_dim {self.codebook_dim}")
        hidden = np.zeros(self.spec["dim"], np.float32)
        logits = np.zeros(self.spec["vocab"], np.float32) if want_logits else None
        self._call(self._L.s2hip_eval, _p(flat), flat.size // self.codebook_dim, _p(hidden),
                   _p(logits) if want_logits else None)
        return hidden, logits

    prefill = eval

    def step(self, flat_token, want_logits: bool = True):
        flat = np.ascontiguousarray(flat_token, dtype=np.int32).ravel()
        if flat.size != self.codebook_dim:
            raise S2HipError(f"step token width mismatch: expected {self.codebook_dim}, got {flat.size}")
        return self.eval(flat, want_logits)

    # -- Fast-AR --------------------------------------------------------------
    def fast_logits(self, slow_hidden, prefix_codes):
        h = _f32(slow_hidden)
        pre = np.ascontiguousarray(prefix_codes, dtype=np.uint32)
        out = np.zeros(self.spec["codebook_size"], np.float32)
        self._call(self._L.s2hip_fast_logits, _p(h), _p(pre) if pre.size else None, pre.size, _p(out))
        return out

    def fast_codebooks(self, slow_hidden, semantic_code, temperature=0.0, top_p=1.0, top_k=0,
                       rng_state=0):
        h = _f32(slow_hidden)
        codes = np.zeros(self.spec["num_codebooks"], np.uint32)
        st = ctypes.c_uint64(rng_state)
        smp = _lib.Sampler(temperature, top_p, top_k)
        self._call(self._L.s2hip_fast_codebooks, _p(h), semantic_code, ctypes.byref(smp),
                   ctypes.byref(st), _p(codes))
        return codes, st.value

    # -- generate_codes ---------------------------------------------------------
    def generate_codes(self, prompt_flat, max_new_tokens, temperature=0.0, top_p=1.0, top_k=0,
                       min_tokens_before_end=0, rng_state=0):
        flat = np.ascontiguousarray(prompt_flat, dtype=np.int32).ravel()
        if flat.size % self.codebook_dim:
            raise S2HipError("prompt length is not a multiple of codebook_dim")
        ncb = self.spec["num_codebooks"]
        codes = np.zeros(max(1, ncb * max_new_tokens), np.int32)
        params = _lib.GenParams(max_new_tokens, temperature, top_p, top_k, min_tokens_before_end)
        st = ctypes.c_uint64(rng_state)
        nf = ctypes.c_uint32(0)
        stats = _lib.GenStats()
        self._call(self._L.s2hip_generate_codes, _p(flat), flat.size // self.codebook_dim,
                   ctypes.byref(params), ctypes.byref(st), _p(codes), ctypes.byref(nf),
                   ctypes.byref(stats))
        n = nf.value
        return {
            "codes": codes[: ncb * n].reshape(ncb, n).copy(),
            "n_frames": n,
            "rng_state": st.value,
            "prefill_ms": stats.prefill_ms,
            "decode_ms": stats.decode_ms,
            "graph_used": bool(stats.graph_used),
            "per_column_rerun": bool(stats.per_column_rerun),
            "greedy_rerun": bool(stats.greedy_rerun),
        }

    def generate_codes_batch(self, prompts, max_new_tokens, temperature=0.0, top_p=1.0, top_k=0,
                             min_tokens_before_end=0, rng_states=None):
        """Several independent generate_codes requests decoded together (one KV
        slot each).  Returns one result dict per request, as generate_codes
        does, plus the batch's prefill / decode times and total frames."""
        flats = []
        for pr in prompts:
            flat = np.ascontiguousarray(pr, dtype=np.int32).ravel()
            if flat.size % self.codebook_dim:
                raise S2HipError("prompt length is not a multiple of codebook_dim")
            flats.append(flat)
        nb = len(flats)
        if nb == 0:
            raise S2HipError("expected at least one request")
        ncb = self.spec["num_codebooks"]
        if rng_states is None:
            rng_states = [0] * nb
        if len(rng_states) != nb:
            raise S2HipError("one rng state per request expected")
        codes = [np.zeros(max(1, ncb * max_new_tokens), np.int32) for _ in range(nb)]
        prompt_ptrs = (ctypes.c_void_p * nb)(*[f.ctypes.data for f in flats])
        cols = (ctypes.c_size_t * nb)(*[f.size // self.codebook_dim for f in flats])
        code_ptrs = (ctypes.c_void_p * nb)(*[c.ctypes.data for c in codes])
        states = (ctypes.c_uint64 * nb)(*[int(r) for r in rng_states])
        nf = (ctypes.c_uint32 * nb)()
        params = _lib.GenParams(max_new_tokens, temperature, top_p, top_k, min_tokens_before_end)
        stats = _lib.GenStats()
        self._call(self._L.s2hip_generate_codes_batch, nb, prompt_ptrs, cols, ctypes.byref(params), states,
                   code_ptrs, nf, ctypes.byref(stats))
        out = []
        for b in range(nb):
            n = nf[b]
            out.append({
                "codes": codes[b][: ncb * n].reshape(ncb, n).copy(),
                "n_frames": n,
                "rng_state": states[b],
            })
        return {
            "requests": out,
            "prefill_ms": stats.prefill_ms,
            "decode_ms": stats.decode_ms,
            "total_frames": stats.n_frames,
            "graph_used": bool(stats.graph_used),
            "per_column_rerun": bool(stats.per_column_rerun),
            "greedy_rerun": bool(stats.greedy_rerun),
        }

    # -- op level -------------------------------------------------------------
    def linear(self, weight_rows: np.ndarray, ggml_type: int, in_dim: int, out_dim: int, x):
        w = np.ascontiguousarray(weight_rows)
        xs = _f32(x).reshape(-1, in_dim)
        y = np.zeros((xs.shape[0], out_dim), np.float32)
        self._call(self._L.s2hip_op_linear, _p(w), ggml_type, in_dim, out_dim, _p(xs), xs.shape[0], _p(y))
        return y

    def rms_norm(self, x, weight, eps):
        w = _f32(weight)
        xs = _f32(x).reshape(-1, w.size)
        y = np.zeros_like(xs)
        self._call(self._L.s2hip_op_rms_norm, _p(xs), _p(w), w.size, xs.shape[0], eps, _p(y))
        return y

    def dequant_rows(self, weight_rows: np.ndarray, ggml_type: int, in_dim: int, rows: int):
        w = np.ascontiguousarray(weight_rows)
        out = np.zeros((rows, in_dim), np.float32)
        self._call(self._L.s2hip_op_dequant_rows, _p(w), ggml_type, in_dim, rows, _p(out))
        return out

    def qk_rope(self, qkv, heads, kv_heads, head_dim, position, rope_base, q_norm=None, k_norm=None,
                eps=1e-6):
        v_in = _f32(qkv)
        qn = None if q_norm is None else _f32(q_norm)
        kn = None if k_norm is None else _f32(k_norm)
        q = np.zeros(heads * head_dim, np.float32)
        k = np.zeros(kv_heads * head_dim, np.float32)
        v = np.zeros(kv_heads * head_dim, np.float32)
        self._call(self._L.s2hip_op_qk_rope, _p(v_in), heads, kv_heads, head_dim, position, rope_base,
                   None if qn is None else _p(qn), None if kn is None else _p(kn), eps, _p(q), _p(k),
                   _p(v))
        return q, k, v

    def attention(self, q, keys, values, heads, kv_heads, head_dim, tokens, scale):
        qa, ka, va = _f32(q), _f32(keys), _f32(values)
        out = np.zeros(heads * head_dim, np.float32)
        self._call(self._L.s2hip_op_attention, _p(qa), _p(ka), _p(va), heads, kv_heads, head_dim,
                   tokens, scale, _p(out))
        return out

    def swiglu(self, gate, up, fast=False):
        g, u = _f32(gate), _f32(up)
        out = np.zeros_like(g)
        self._call(self._L.s2hip_op_swiglu, _p(g), _p(u), g.size, 1 if fast else 0, _p(out))
        return out

    def running_sums(self, terms):
        """Sequential f32 running sums of `terms` on the device (the samplers'
        summation routine): returns (prefix sums, total)."""
        t = _f32(terms)
        out = np.zeros_like(t)
        total = ctypes.c_float(0)
        self._call(self._L.s2hip_op_running_sums, _p(t), t.size, _p(out), ctypes.byref(total))
        return out, total.value

    def running_cut(self, terms, threshold, absorb=False, at=None):
        """The samplers' cut search on the device: (first index whose running
        sum reaches `threshold` or len(terms), the running sum there or the
        total, the running sum at index `at` or 0.0)."""
        t = _f32(terms)
        cut = ctypes.c_size_t(0)
        s, s_at = ctypes.c_float(0), ctypes.c_float(0)
        at_v = t.size if at is None else int(at)
        self._call(self._L.s2hip_op_running_cut, _p(t), t.size, float(threshold), 1 if absorb else 0, at_v,
                   ctypes.byref(cut), ctypes.byref(s), ctypes.byref(s_at))
        return cut.value, s.value, s_at.value

    def expf(self, x):
        """The device exp of the samplers and SwiGLU epilogues over an array."""
        a = _f32(x)
        out = np.empty_like(a)
        self._call(self._L.s2hip_op_expf, _p(a), a.size, _p(out))
        return out

    def sample(self, logits, temperature, top_p, top_k, always_include=None, rng_state=0):
        x = _f32(logits)
        smp = _lib.Sampler(temperature, top_p, top_k)
        st = ctypes.c_uint64(rng_state)
        tok = ctypes.c_uint32(0)
        self._call(self._L.s2hip_op_sample, _p(x), x.size, ctypes.byref(smp),
                   -1 if always_include is None else always_include, ctypes.byref(st),
                   ctypes.byref(tok))
        return tok.value, st.value

    def sample_noalloc(self, logits, temperature, top_p, top_k, always_include=None, rng_state=0):
        """sample() through the allocation-free entry point (at most 8191 logits)."""
        x = _f32(logits)
        smp = _lib.Sampler(temperature, top_p, top_k)
        st = ctypes.c_uint64(rng_state)
        tok = ctypes.c_uint32(0)
        self._call(self._L.s2hip_op_sample_noalloc, _p(x), x.size, ctypes.byref(smp),
                   -1 if always_include is None else always_include, ctypes.byref(st), ctypes.byref(tok))
        return tok.value, st.value

    def time_kernel(self, name: str, reps: int = 10):
        avg = ctypes.c_double(0)
        nbytes = ctypes.c_double(0)
        self._call(self._L.s2hip_time_kernel, name.encode(), reps, ctypes.byref(avg), ctypes.byref(nbytes))
        return avg.value, nbytes.value


def transpose_to_time_major(data, rows: int, cols: int) -> np.ndarray:
    """transpose_to_time_major (crates/fish_s2_infer/src/prompt.rs:79-103):
    the codebook-major (rows x cols) prompt tensor of build_prompt to the
    time-major flat i32 layout the engine takes, flat[t * rows + r] =
    data[r * cols + t].  Raises S2HipError with the reference's messages."""
    d = np.ascontiguousarray(data, dtype=np.uint32).ravel()
    out = np.zeros(max(1, d.size), np.int32)
    err = ctypes.create_string_buffer(_lib.ERR_CAP)
    if not _lib.load().s2hip_transpose_to_time_major(_p(d) if d.size else None, d.size, rows, cols, _p(out), err,
                                                     len(err)):
        raise S2HipError(err.value.decode())
    return out[: d.size]


def expf_host(x) -> np.ndarray:
    """The device exp routine compiled for the host (no device needed)."""
    a = _f32(x)
    out = np.empty_like(a)
    _lib.load().s2hip_expf_host(_p(a), a.size, _p(out))
    return out


def version() -> str:
    return _lib.load().s2hip_version().decode()
