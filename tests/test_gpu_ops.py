"""Per-op parity of the HIP kernels against the CPU oracle (through the C ABI).

Tolerances are the north-star bars: 1e-2 relative for f16-weight paths and
2e-2 for quantised ones (the kernels accumulate in f32, so actual errors are
~1e-6); dequantisation and sampling must be bit-exact.
"""

import math

import numpy as np
import pytest

from oracle import oracle as O
from s2hip import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng(tiny_gguf):
    from s2hip import Engine

    e = Engine(tiny_gguf, 64, synth.TINY.im_end_id)
    yield e
    e.close()


def _rows(gtype, wf):
    if gtype == 1:
        return wf.astype(np.float16).view(np.uint8).ravel()
    return np.frombuffer(b"".join(synth.quantize_block(gtype, b) for b in wf.reshape(-1, 32)), np.uint8)


def _rel(a, b):
    return float(np.max(np.abs(a - b)) / max(1e-30, float(np.max(np.abs(b)))))


@pytest.mark.parametrize("gtype", [1, 8, 2])
def test_dequant_bit_exact(eng, gtype):
    rng = np.random.default_rng(10 + gtype)
    in_dim, rows = 2560, 24
    wf = (rng.standard_normal((rows, in_dim)) * 0.02).astype(np.float32)
    raw = _rows(gtype, wf)
    got = eng.dequant_rows(raw, gtype, in_dim, rows)
    want = O.dequant_row(raw.tobytes(), gtype, in_dim * rows).reshape(rows, in_dim)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("gtype,tol", [(1, 1e-2), (8, 2e-2), (2, 2e-2)])
@pytest.mark.parametrize("in_dim,out_dim,ncol", [(512, 768, 1), (2560, 6144, 1), (9728, 2560, 1), (4096, 2560, 1),
                                                 (4096, 2560, 2), (2560, 9728, 4), (1536, 100, 3),
                                                 (9728, 2560, 8), (4096, 2560, 16), (512, 1029, 11),
                                                 (1056, 64, 5), (9728, 103, 1), (9728, 2561, 1)])
def test_linear_matches_oracle(eng, gtype, tol, in_dim, out_dim, ncol):
    rng = np.random.default_rng(in_dim + out_dim + ncol)
    wf = (rng.standard_normal((out_dim, in_dim)) * 0.02).astype(np.float32)
    raw = _rows(gtype, wf)
    x = rng.standard_normal((ncol, in_dim)).astype(np.float32)
    got = eng.linear(raw, gtype, in_dim, out_dim, x)
    for c in range(ncol):
        want = O.linear(x[c], raw, gtype, in_dim, out_dim)
        assert _rel(got[c], want) < min(tol, 1e-4), c


@pytest.mark.parametrize("in_dim,out_dim", [(2560, 6144), (4096, 2560), (9728, 2560), (512, 1029)])
def test_batched_product_column_bits_independent_of_batch_width(eng, in_dim, out_dim):
    """Up to 8 columns take the packed batched product (the 8 columns' hi and
    lo parts in one MFMA's 16 columns, split where they are staged), 9-16
    columns the 16-column product (hi and lo in two MFMAs, split in the MFMA
    lanes).  Both take the same per-column scale, split and sums in the same
    order, so each column's result has the same bits whichever product serves
    it (a swapped hi / lo half, a wrong scale lane or a misplaced fragment
    row would break this)."""
    rng = np.random.default_rng(in_dim * 7 + out_dim)
    wf = (rng.standard_normal((out_dim, in_dim)) * 0.02).astype(np.float32)
    raw = _rows(1, wf)
    x = rng.standard_normal((9, in_dim)).astype(np.float32)
    x *= (10.0 ** rng.uniform(-3, 3, (9, in_dim))).astype(np.float32)
    y9 = eng.linear(raw, 1, in_dim, out_dim, x)
    for n in (8, 5, 3):
        yn = eng.linear(raw, 1, in_dim, out_dim, x[:n])
        assert np.array_equal(yn.view(np.uint32), y9[:n].view(np.uint32)), n


@pytest.mark.parametrize("ncol", [2, 8])
def test_batched_linear_activation_range(eng, ncol):
    """Batched F16 columns go through the MFMA product with activations scaled
    per wave by a power of two and split into f16 hi and lo parts: columns
    whose values span 1e-6 .. 1e6 (and single entries up to 1e8) match the
    oracle to 1e-4, a spike beyond the per-wave headroom is taken on the
    per-column path, and a non-finite value makes the call fail instead of
    returning a wrong result."""
    from s2hip import S2HipError

    rng = np.random.default_rng(31 + ncol)
    in_dim, out_dim = 2560, 256
    wf = (rng.standard_normal((out_dim, in_dim)) * 0.02).astype(np.float32)
    raw = _rows(1, wf)
    for lo_exp, hi_exp in ((-6, 6), (-6, -5), (5, 6), (-1, 1)):
        x = rng.standard_normal((ncol, in_dim)).astype(np.float32)
        x *= (10.0 ** rng.uniform(lo_exp, hi_exp, (ncol, in_dim))).astype(np.float32)
        x[0, 7] = 6.0e4 * 10.0 ** (hi_exp - 1)
        x[-1, 100] = -1.0e8 if hi_exp == 6 else x[-1, 100]
        got = eng.linear(raw, 1, in_dim, out_dim, x)
        for c in range(ncol):
            want = O.linear(x[c], raw, 1, in_dim, out_dim)
            assert _rel(got[c], want) < 1e-4, (lo_exp, hi_exp, c, _rel(got[c], want))
    # one column of tiny values next to one of huge values
    x = rng.standard_normal((ncol, in_dim)).astype(np.float32)
    x[0] *= 1e-6
    x[-1] *= 1e6
    got = eng.linear(raw, 1, in_dim, out_dim, x)
    for c in range(ncol):
        assert _rel(got[c], O.linear(x[c], raw, 1, in_dim, out_dim)) < 1e-4, c
    # one channel 1e6 / 1e5 times the rest, past the first 256 elements of its
    # wave's k range (beyond the per-wave scale's 2^15 headroom): the product
    # is taken on the per-column path and still matches
    for spike in (1e6, -1e5):
        xs = rng.standard_normal((ncol, in_dim)).astype(np.float32)
        xs[0, 300] = spike
        xs[-1, 2000] = spike
        got = eng.linear(raw, 1, in_dim, out_dim, xs)
        for c in range(ncol):
            assert _rel(got[c], O.linear(xs[c], raw, 1, in_dim, out_dim)) < 1e-4, (spike, c)
    for bad in (np.nan, np.inf):
        x[0, 5] = bad
        with pytest.raises(S2HipError, match="batched product"):
            eng.linear(raw, 1, in_dim, out_dim, x)
    # the engine still works
    x[0, 5] = 1.0
    got = eng.linear(raw, 1, in_dim, out_dim, x)
    assert _rel(got[0], O.linear(x[0], raw, 1, in_dim, out_dim)) < 1e-4


def test_rms_norm_matches_oracle(eng):
    rng = np.random.default_rng(20)
    x = rng.standard_normal((3, 2560)).astype(np.float32) * 3
    w = rng.standard_normal(2560).astype(np.float32)
    got = eng.rms_norm(x, w, 1e-6)
    for c in range(3):
        np.testing.assert_allclose(got[c], O.rms_norm(x[c], w, 1e-6), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("hd,H,Hkv,qk", [(128, 32, 8, True), (64, 8, 2, True), (128, 32, 8, False)])
@pytest.mark.parametrize("pos", [0, 1, 255, 767])
def test_qk_norm_rope_matches_oracle(eng, hd, H, Hkv, qk, pos):
    rng = np.random.default_rng(hd + pos)
    qkv = rng.standard_normal((H + 2 * Hkv) * hd).astype(np.float32)
    qn = rng.uniform(0.5, 1.5, hd).astype(np.float32) if qk else None
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32) if qk else None
    q, k, v = eng.qk_rope(qkv, H, Hkv, hd, pos, 1.0e6, qn, kn, 1e-6)
    q_raw, k_raw, v_raw = qkv[:H * hd], qkv[H * hd:(H + Hkv) * hd], qkv[(H + Hkv) * hd:]
    if qk:
        q_raw = O.rms_norm_heads(q_raw, qn, hd, 1e-6)
        k_raw = O.rms_norm_heads(k_raw, kn, hd, 1e-6)
    np.testing.assert_allclose(q, O.rope_normal(q_raw, hd, pos, 1.0e6), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(k, O.rope_normal(k_raw, hd, pos, 1.0e6), rtol=1e-5, atol=1e-5)
    assert np.array_equal(v, v_raw)


@pytest.mark.parametrize("H,Hkv,hd,T", [(32, 8, 128, 1), (32, 8, 128, 200), (32, 8, 128, 768), (8, 2, 64, 37),
                                        (32, 8, 128, 10), (32, 8, 128, 2000), (32, 8, 128, 2560), (8, 2, 64, 4100)])
def test_attention_matches_oracle(eng, H, Hkv, hd, T):
    rng = np.random.default_rng(T + hd)
    q = rng.standard_normal(H * hd).astype(np.float32)
    k = rng.standard_normal(T * Hkv * hd).astype(np.float32)
    v = rng.standard_normal(T * Hkv * hd).astype(np.float32)
    sc = 1 / math.sqrt(hd)
    got = eng.attention(q, k, v, H, Hkv, hd, T, sc)
    want = O.gqa_attention(q, k, v, H, Hkv, hd, T, sc)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("fast", [False, True])
def test_swiglu_matches_oracle(eng, fast):
    # same operation order and the same expf bits as the reference: bit-exact
    rng = np.random.default_rng(30)
    g = (rng.standard_normal(97280) * 4).astype(np.float32)
    u = rng.standard_normal(97280).astype(np.float32)
    got, want = eng.swiglu(g, u, fast), O.swiglu(g, u, fast)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_expf_bit_exact_on_device(eng):
    # the device exp of the samplers and SwiGLU sigmoids reproduces the C
    # library's expf (what Rust's f32::exp calls) bit for bit: every 397th
    # float bit pattern (10.8 M inputs over all binades, inf, NaN) plus 4 M
    # softmax arguments in [-104, 0]
    u = np.arange(0, 1 << 32, 397, dtype=np.uint64).astype(np.uint32)
    rng = np.random.default_rng(8)
    x = np.concatenate([u.view(np.float32), -rng.exponential(4.0, 2_000_000).astype(np.float32),
                        -rng.uniform(0, 104, 2_000_000).astype(np.float32)])
    got, want = eng.expf(x), O.expf(x)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert x.size >= 10_000_000 and same.all(), x[~same][:5]


def _running_sum_cases():
    rng = np.random.default_rng(77)
    cases = []
    for n in (1, 37, 255, 256, 257, 4096, 8192):
        lg = rng.standard_normal(n).astype(np.float32)
        p = np.exp((lg - lg.max()) / np.float32(0.7)).astype(np.float32)
        cases.append(("softmax_sorted", np.sort(p / p.sum())[::-1].astype(np.float32)))
        cases.append(("uniform", rng.random(n).astype(np.float32)))
        cases.append(("wide_exponents", (rng.random(n) * 2.0 ** rng.integers(-149, 20, n)).astype(np.float32)))
        t = (rng.integers(0, 8, n) * 2.0 ** -25).astype(np.float32)
        t[0] = 1.0
        cases.append(("half_ulp_ties", t))
        z = np.zeros(n, np.float32)
        z[rng.integers(0, n, 3)] = rng.random(3).astype(np.float32)
        cases.append(("mostly_zero", z))
        cases.append(("subnormal", (rng.integers(0, 1 << 20, n) * 2.0 ** -149).astype(np.float32)))
        cases.append(("growing", (2.0 ** (np.arange(n) % 40) * 1e-30).astype(np.float32)))
        cases.append(("mixed_sign", rng.standard_normal(n).astype(np.float32)))
    cases.append(("overflow", np.array([3e38, 3e38, 1.0, 2.0], np.float32)))
    cases.append(("equal_terms", np.full(8192, 1.0 / 3.0, np.float32)))
    return cases


@pytest.mark.parametrize("name,terms", _running_sum_cases(), ids=lambda v: v if isinstance(v, str) else str(len(v)))
def test_running_sums_bit_exact(eng, name, terms):
    # The samplers' sums (sampling.rs:202-241) add term by term in index
    # order; numpy's add.accumulate in float32 is that sequential loop.
    want = np.add.accumulate(terms, dtype=np.float32)
    got, total = eng.running_sums(terms)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (
        name, int(np.argmax(got.view(np.uint32) != want.view(np.uint32))))
    assert np.float32(total).view(np.uint32) == want[-1].view(np.uint32)



def _cut_terms(n, rng):
    lg = rng.standard_normal(n).astype(np.float32)
    top = lg.max() if n else np.float32(0)
    soft = np.exp((lg - top) / np.float32(0.7)).astype(np.float32)
    steep = np.exp((lg - top) / np.float32(0.02)).astype(np.float32)
    soft /= soft.sum() if n else np.float32(1)
    steep /= steep.sum() if n else np.float32(1)
    return [
        ("uniform", np.full(n, np.float32(1.0) / np.float32(max(n, 1)), np.float32), True),
        ("softmax", np.sort(soft)[::-1].astype(np.float32), True),
        ("steep", np.sort(steep)[::-1].astype(np.float32), True),  # absorbed early
        ("unsorted", rng.random(n).astype(np.float32), False),
    ]


@pytest.mark.parametrize("n", [0, 1, 31, 32, 33, 63, 64, 65, 100, 4096, 4100, 8192])
def test_running_cut_matches_sequential_loop(eng, n):
    # The top-p loop (sampling.rs:226-233) stops at the first item whose
    # running sum reaches top_p, the draw (:235-240) at the first whose running
    # sum exceeds the target; numpy's float32 add.accumulate is the loop.
    # Thresholds hit running sums exactly (ties), fall just above one (the
    # crossing is the next index), sit at batch edges and in the tail, and
    # never match (NaN, above the total).
    rng = np.random.default_rng(1000 + n)
    for kind, terms, absorb in _cut_terms(n, rng):
        pref = np.add.accumulate(terms, dtype=np.float32)
        total = pref[-1] if n else np.float32(0)
        thrs = [np.float32(np.nan), np.float32(0.0), np.float32(total) * np.float32(0.9),
                np.nextafter(np.float32(total), np.float32(np.inf)), np.float32(total) + np.float32(1.0)]
        for k in sorted({0, 30, 31, 32, 33, 64, n // 2, n - 2, n - 1}):
            if 0 <= k < n:
                thrs += [pref[k], np.nextafter(pref[k], np.float32(np.inf))]
        for thr in thrs:
            for at in (None, 0, 31, 32, n // 3, n - 1):
                if at is not None and not 0 <= at < n:
                    continue
                hit = np.nonzero(pref >= thr)[0]
                cut = int(hit[0]) if hit.size else n
                want_s = pref[cut] if cut < n else np.float32(total)
                want_at = pref[at] if at is not None else np.float32(0)
                got_cut, got_s, got_at = eng.running_cut(terms, thr, absorb=absorb, at=at)
                ctx = (kind, n, float(thr), at)
                assert got_cut == cut, ctx
                assert np.float32(got_s).view(np.uint32) == np.float32(want_s).view(np.uint32), ctx
                assert np.float32(got_at).view(np.uint32) == np.float32(want_at).view(np.uint32), ctx


def test_running_cut_rejects_bad_terms(eng):
    with pytest.raises(Exception, match="non-negative"):
        eng.running_cut(np.array([0.5, -0.1], np.float32), 0.3)
    with pytest.raises(Exception, match="non-increasing"):
        eng.running_cut(np.array([0.1, 0.5], np.float32), 0.3, absorb=True)

SAMPLER_CASES = [
    (0.0, 1.0, 0), (0.0, 0.9, 0), (0.0, 1.0, 30), (0.7, 0.9, 0), (0.7, 0.7, 30), (1.0, 1.0, 0),
    (0.3, 0.5, 5), (0.7, 1.0, 4096), (1.5, 0.95, 1),
]


@pytest.mark.parametrize("T,top_p,top_k", SAMPLER_CASES)
@pytest.mark.parametrize("n", [4096, 1024, 4097, 37])
def test_sampler_bit_exact(eng, T, top_p, top_k, n):
    rng = np.random.default_rng(n * 7 + int(T * 10) + top_k)
    st_o = st_g = 12345 + n
    for trial in range(12):
        logits = rng.standard_normal(n).astype(np.float32)
        if trial % 4 == 1:
            logits[rng.integers(0, n, 3)] = logits.max()  # exact ties at the max
        if trial % 4 == 2:
            logits[rng.integers(0, n, n // 3)] = -np.inf  # masked entries
        if trial % 4 == 3:
            logits = np.round(logits * 4) / 4  # many equal values
        always = int(rng.integers(0, n)) if trial % 3 == 0 else None
        to, st_o = O.sample_token(logits, T, top_p, top_k, always, st_o)
        tg, st_g = eng.sample(logits, T, top_p, top_k, always, st_g)
        assert (tg, st_g) == (to, st_o), (trial, tg, to)



@pytest.mark.parametrize("n", [4096, 4097, 37])
def test_sampler_greedy_uniqueness_threshold(eng, n):
    # The greedy path needs exactly one value within 1e-6 of the max
    # (sampling.rs:120-140); the device decides it from the largest and the
    # second largest value.  Second values one ulp below the max, at about
    # 1e-6 below it on either side of the threshold, masked (-inf) entries
    # and a +inf max (inf - inf is NaN: no value passes, so the reference
    # leaves the greedy path) must give the oracle's token and RNG state.
    rng = np.random.default_rng(900 + n)
    st_o = st_g = 777 + n
    one = np.float32(1.0)
    seconds = [np.nextafter(one, np.float32(0)), one - np.float32(1e-6), one - np.float32(9e-7),
               one - np.float32(1.1e-6), one - np.float32(2e-6), np.float32(0.5)]
    for trial in range(2 * len(seconds) + 4):
        logits = (rng.standard_normal(n) * 0.1).astype(np.float32)
        i, j = rng.choice(n, 2, replace=False)
        logits[i] = one
        if trial < 2 * len(seconds):
            logits[j] = seconds[trial % len(seconds)]
            if trial >= len(seconds):  # a masked (-inf) entry above them: ignored
                logits[rng.integers(0, n)] = -np.inf
        elif trial % 2 == 0:
            logits[j] = np.float32(np.inf)
        else:
            logits[i] = logits[j] = np.float32(np.inf)
        to, st_o = O.sample_token(logits, 0.0, 1.0, 0, None, st_o)
        tg, st_g = eng.sample(logits, 0.0, 1.0, 0, None, st_g)
        assert (tg, st_g) == (to, st_o), (trial, tg, to)


@pytest.mark.parametrize("T,top_p,top_k", [(0.7, 0.9, 0), (0.7, 0.7, 30), (1.0, 1.0, 0)])
def test_sampler_infinite_logits(eng, T, top_p, top_k):
    # +inf logits make the softmax numerators NaN ((inf - inf) / T); the
    # reference's sums, cut and draw then compare against NaN, and the
    # device must end on the same item and RNG state.
    rng = np.random.default_rng(31)
    st_o = st_g = 4242
    for trial in range(6):
        n = (4096, 37, 4097)[trial % 3]
        logits = rng.standard_normal(n).astype(np.float32)
        logits[rng.choice(n, 1 + trial % 2, replace=False)] = np.inf
        to, st_o = O.sample_token(logits, T, top_p, top_k, None, st_o)
        tg, st_g = eng.sample(logits, T, top_p, top_k, None, st_g)
        assert (tg, st_g) == (to, st_o), (trial, tg, to)

def test_sampler_exact_on_the_draws_nearest_a_boundary(eng):
    # Draws whose target lies closest to a cumulative-probability boundary (or
    # whose top-p sums lie closest to top_p) are the ones a probability that is
    # off by one ulp would flip.  Pick the 64 most sensitive of 3000 seeded
    # cases with the oracle's own margins and require identical draws.
    rng = np.random.default_rng(404)
    cases = []
    for i in range(3000):
        n = 4096
        logits = (rng.standard_normal(n) * 2).astype(np.float32)
        T, top_p, top_k = [(0.7, 0.9, 0), (0.7, 0.7, 30), (1.0, 0.95, 0)][i % 3]
        st = int(rng.integers(1, 1 << 62))
        tok, st_after, (draw, cut, tie) = O.sample_token_margins(logits, T, top_p, top_k, None, st)
        cases.append((min(draw, cut), logits, T, top_p, top_k, st, tok, st_after))
    cases.sort(key=lambda c: c[0])
    for margin, logits, T, top_p, top_k, st, tok, st_after in cases[:64]:
        assert margin < 1e-4
        assert eng.sample(logits, T, top_p, top_k, None, st) == (tok, st_after), margin
