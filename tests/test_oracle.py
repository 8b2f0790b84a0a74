"""Pinning the CPU oracle (oracle/qtts_oracle.c) before trusting it.

Each oracle function is checked against something other than a retyping of
its own formula: the reference's differential tests (gemv.rs:756-861),
numpy float64 recomputations, closed forms and invariants, and the
reference's sampler known-answer tests (generate_new.rs:918-955).
"""
import numpy as np
import pytest

import oracle as O
import refgen
from qtts import hostdesc, synth


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ---- Q4 GEMV (gemv.rs:249-346, simd.rs:76-153) ---------------------------

@pytest.mark.parametrize("k,n,seed", refgen.SHAPE_CASES)
def test_avx2_matches_scalar_shapes(k, n, seed):
    x, w = refgen.case(k, n, seed)
    ya = O.gemv_avx2(x, w)
    if ya is None:
        pytest.skip("host has no AVX2")
    assert np.array_equal(bits(ya), bits(O.gemv_scalar(x, w)))


@pytest.mark.parametrize("k,n,seed,iz,sz", refgen.SPARSE_CASES)
def test_avx2_matches_scalar_sparse(k, n, seed, iz, sz):
    x, w = refgen.case(k, n, seed, iz, sz)
    ya = O.gemv_avx2(x, w)
    if ya is None:
        pytest.skip("host has no AVX2")
    assert np.array_equal(bits(ya), bits(O.gemv_scalar(x, w)))


@pytest.mark.parametrize("k,n,seed", refgen.SHAPE_CASES)
def test_avx512_matches_scalar_shapes(k, n, seed):
    # simd.rs:203-269 is bit-identical to the scalar kernel, as its AVX2 sibling
    x, w = refgen.case(k, n, seed)
    ya = O.gemv_avx512(x, w)
    if ya is None:
        pytest.skip("host has no AVX-512")
    assert np.array_equal(bits(ya), bits(O.gemv_scalar(x, w)))


@pytest.mark.parametrize("k,n,seed,iz,sz", refgen.SPARSE_CASES)
def test_avx512_matches_scalar_sparse(k, n, seed, iz, sz):
    x, w = refgen.case(k, n, seed, iz, sz)
    ya = O.gemv_avx512(x, w)
    if ya is None:
        pytest.skip("host has no AVX-512")
    assert np.array_equal(bits(ya), bits(O.gemv_scalar(x, w)))


def test_avx512_interleave_order():
    # one-hot rows: column j of the output is exactly (nibble_j - 8) * s, so a
    # wrong lane of the interleave (lo/hi or first/second half) moves a value
    rng = np.random.Generator(np.random.PCG64(5))
    w = synth.q4_random(rng, 3, 96)
    for r in range(3):
        x = np.zeros(3, np.float32)
        x[r] = 1.0
        ya = O.gemv_avx512(x, w)
        if ya is None:
            pytest.skip("host has no AVX-512")
        nib = np.empty(96, np.int64)
        nib[0::2] = w.packed[r] & 15
        nib[1::2] = w.packed[r] >> 4
        sc = np.repeat(np.ascontiguousarray(w.scales[r]).view(np.float16).astype(np.float32), 32)
        assert np.array_equal(bits(ya), bits((nib - 8).astype(np.float32) * sc))


def test_isa_dispatch_and_chunked_gemv_agree():
    # gemv.rs:230-243 picks AVX-512 first; every ISA gives the chunked GEMV
    # the same bits (the kernels are bit-identical per k-range)
    rng = np.random.Generator(np.random.PCG64(6))
    w = synth.q4_random(rng, 2048, 1024)
    x = rng.standard_normal(2048).astype(np.float32)
    O.set_workers(8, 8)
    try:
        default = O.set_isa(None)
        assert default == ("avx512f" if O.gemv_avx512(x[:1], synth.q4_random(rng, 1, 32)) is not None
                           else "avx2" if O.gemv_avx2(x[:1], synth.q4_random(rng, 1, 32)) is not None else "scalar")
        ref = O.gemv(x, w)
        for isa in ("scalar", "avx2", "avx512f"):
            if O.set_isa(isa) is None:
                continue
            assert np.array_equal(bits(O.gemv(x, w)), bits(ref)), isa
    finally:
        O.set_isa(None)


def test_subrange_chunks():
    # gemv.rs:777-810: chunked AVX2 == chunked scalar exactly, ~ full within 1e-3
    st = refgen.XRng(21)
    k, n = 64, 1024
    g = n // 32
    packed = refgen.rbytes(st, k * g * 16).reshape(k, g * 16)
    scales = refgen.rscales(st, k * g, 0.1).reshape(k, g)
    x = refgen.rinput(st, k, 0.1)
    w = synth.Q4(packed, scales, k, n)
    full = O.gemv_scalar(x, w)
    acc = np.zeros(n, np.float32)
    acc_ref = np.zeros(n, np.float32)
    for a, b in [(0, 16), (16, 48), (48, 64)]:
        pa = O.gemv_avx2(x, w, a, b)
        if pa is None:
            pytest.skip("host has no AVX2")
        acc += pa
        acc_ref += O.gemv_scalar(x, w, a, b)
    assert np.array_equal(bits(acc), bits(acc_ref))
    assert np.abs(acc - full).max() < 1e-3


def test_many_chunks_tolerance():
    # gemv.rs:814-842: 32-chunk over-decomposition within 1e-3 of one pass
    st = refgen.XRng(77)
    k, n = 128, 1024
    g = n // 32
    w = synth.Q4(refgen.rbytes(st, k * g * 16).reshape(k, g * 16), refgen.rscales(st, k * g, 0.1).reshape(k, g), k, n)
    x = refgen.rinput(st, k, 0.1)
    full = O.gemv_scalar(x, w)
    ck = (k + 31) // 32
    acc = np.zeros(n, np.float32)
    for t in range(32):
        a, b = t * ck, min((t + 1) * ck, k)
        if a < b:
            acc += O.gemv_scalar(x, w, a, b)
    assert np.abs(acc - full).max() < 1e-3


def test_tail_columns_stay_zero():
    # gemv.rs:846-861: n = 100 -> 3 full groups, columns 96..99 stay zero
    x, w = refgen.case(16, 100, 31)
    y = O.gemv_scalar(x, w)
    assert np.all(y[96:] == 0.0)
    ya = O.gemv_avx2(x, w)
    if ya is not None:
        assert np.array_equal(bits(ya), bits(y))


def test_gemv_matches_float64_dense():
    # the numeric definition: y = x . dequant(W), against a float64 product
    rng = np.random.Generator(np.random.PCG64(5))
    w = synth.q4_random(rng, 2048, 6144)
    x = rng.standard_normal(2048).astype(np.float32)
    ref = x.astype(np.float64) @ w.dequant().astype(np.float64)
    y = O.gemv_scalar(x, w)
    assert np.abs(y - ref).max() <= 1e-5 * np.sqrt((ref ** 2).mean())


def test_one_hot_returns_dequantised_row():
    rng = np.random.Generator(np.random.PCG64(6))
    w = synth.q4_random(rng, 64, 512)
    for r in (0, 17, 63):
        x = np.zeros(64, np.float32)
        x[r] = 1.0
        assert np.array_equal(bits(O.gemv_scalar(x, w)), bits(w.dequant()[r]))
        assert np.array_equal(bits(O.embed_lookup(w, r)), bits(w.dequant()[r]))


def _policy_chunks(k, n, workers):
    # gemv.rs:302-315, written out independently
    nt = max(1, min(k * n // 500_000, workers))
    if k * n < 500_000:
        nt = 1
    if nt <= 1:
        return [(0, k)]
    nc = max(min(nt * 4, k), nt)
    ck = (k + nc - 1) // nc
    return [(min(t * ck, k), min((t + 1) * ck, k)) for t in range(nc)]


@pytest.mark.parametrize("k,n,workers", [(2048, 6144, 16), (2048, 1024, 16), (6144, 2048, 16), (1024, 1024, 4),
                                         (1024, 2048, 1), (300, 1024, 16)])
def test_chunk_policy(k, n, workers):
    rng = np.random.Generator(np.random.PCG64(k + n))
    w = synth.q4_random(rng, k, n)
    x = rng.standard_normal(k).astype(np.float32)
    acc = np.zeros(n, np.float32)
    for a, b in _policy_chunks(k, n, workers):
        acc += O.gemv_scalar(x, w, a, b)
    O.set_workers(workers, 0)
    try:
        assert np.array_equal(bits(O.gemv(x, w)), bits(acc))
        O.set_workers(workers, 4)
        assert np.array_equal(bits(O.gemv(x, w)), bits(acc))
    finally:
        O.set_workers(16, 0)


def test_gemm_rows_are_full_k():
    rng = np.random.Generator(np.random.PCG64(8))
    w = synth.q4_random(rng, 1024, 2048)
    X = rng.standard_normal((3, 1024)).astype(np.float32)
    Y = O.gemm(X, w)
    for r in range(3):
        assert np.array_equal(bits(Y[r]), bits(O.gemv_scalar(X[r], w)))


# ---- conversions, RNG -------------------------------------------------------

def test_f16_to_f32_exhaustive():
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(int(v)) for v in h], np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(bits(got[finite]), bits(ref[finite]))
    assert np.all(np.isnan(got[np.isnan(ref)]))
    assert np.array_equal(got[np.isinf(ref)], ref[np.isinf(ref)])


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.Generator(np.random.PCG64(9))
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(0.05),
        rng.standard_normal(1000).astype(np.float32) * np.float32(1e4),
        (rng.standard_normal(1000) * 1e-6).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65520.0, 1e9, -1e9, 6e-8, 3e-8, 2.98e-8], np.float32),
    ])
    with np.errstate(over="ignore"):                # 65520 and +-1e9 round to +-inf on purpose
        ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([O.f32_to_f16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, ref)


def test_simple_rand_sequence():
    # generate_new.rs:17-22 written out with Python integers
    s = 42
    st = 42
    for _ in range(1000):
        s ^= (s << 13) & refgen.M64
        s ^= s >> 7
        s ^= (s << 17) & refgen.M64
        r, st = O.simple_rand(st)
        assert st == s
        assert r == np.float32(np.float32(s) / np.float32(2.0 ** 64))
        assert 0.0 <= r <= 1.0


# ---- elementwise ---------------------------------------------------------------

def test_rms_norm_against_float64():
    rng = np.random.Generator(np.random.PCG64(10))
    x = (rng.standard_normal(2048) * 7).astype(np.float32)
    g = synth.gamma(rng, 2048)
    ref = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-6) * g.view(np.float16).astype(np.float64)
    assert np.abs(O.rms_norm(x, g) - ref).max() <= 1e-5 * np.abs(ref).max()


def test_rms_norm_eps_is_1e_6():
    # rows with mean(x^2) = 1e-6: the eps doubles the variance term, so the
    # output is x / sqrt(2e-6) * gamma; eps 1e-5 would give x / sqrt(1.1e-5)
    x = np.full(1024, 1e-3, np.float32)
    x[1::2] = -1e-3
    g = np.full(1024, np.float16(1.0)).view(np.uint16)
    out = O.rms_norm(x, g).astype(np.float64)
    ref = x.astype(np.float64) / np.sqrt(2e-6)
    assert np.abs(out - ref).max() <= 1e-5 * np.abs(ref).max()


def test_rms_norm_constant_vector():
    # closed form: rms of c*ones is |c|, so out = sign(c) * gamma (eps aside)
    g = np.full(1024, np.float16(1.0)).view(np.uint16)
    out = O.rms_norm(np.full(1024, -3.0, np.float32), g)
    assert np.allclose(out, -1.0, atol=1e-6)


def test_softmax_raw():
    rng = np.random.Generator(np.random.PCG64(11))
    s = (rng.standard_normal(513) * 4).astype(np.float32)
    p = O.softmax_raw(s)
    e = np.exp(s.astype(np.float64) - s.max())
    assert np.abs(p - e / e.sum()).max() < 1e-7
    assert abs(float(p.astype(np.float64).sum()) - 1.0) < 1e-5
    assert O.softmax_raw(np.array([3.5], np.float32))[0] == 1.0


def test_silu():
    for x in (-20.0, -1.5, 0.0, 0.3, 4.0, 30.0):
        assert abs(O.silu(x) - x / (1 + np.exp(-x))) <= 1e-6 * max(1.0, abs(x))


def test_qk_norm_per_head():
    rng = np.random.Generator(np.random.PCG64(12))
    d = rng.standard_normal(16 * 128).astype(np.float32) * 3
    g = synth.gamma(rng, 128)
    out = O.qk_norm(d, 16, 128, g)
    for h in range(16):
        v = d[h * 128:(h + 1) * 128].astype(np.float64)
        ref = v / np.sqrt((v ** 2).mean() + 1e-6) * g.view(np.float16).astype(np.float64)
        assert np.abs(out[h * 128:(h + 1) * 128] - ref).max() < 1e-5


def test_rope_table_and_rotation():
    c, s = O.rope_table(128, 2048)
    # f64 angles rounded to f32 (rope.rs:26-38): compare with numpy in f64
    i = np.arange(64, dtype=np.float64)
    ang = np.arange(2048, dtype=np.float64)[:, None] / np.power(1e6, 2 * i / 128)[None, :]
    assert np.abs(c - np.cos(ang)).max() < 1e-7 and np.abs(s - np.sin(ang)).max() < 1e-7
    assert np.array_equal(c[0], np.ones(64, np.float32)) and np.array_equal(s[0], np.zeros(64, np.float32))
    rng = np.random.Generator(np.random.PCG64(13))
    d = rng.standard_normal(8 * 128).astype(np.float32)
    assert np.array_equal(O.rope_apply(d, 8, 128, 0, c, s), d)          # pos 0: identity
    for pos in (1, 77, 2047):
        r = O.rope_apply(d, 8, 128, pos, c, s)
        for h in range(8):
            a, b = d[h * 128:h * 128 + 64], d[h * 128 + 64:(h + 1) * 128]
            ra, rb = r[h * 128:h * 128 + 64], r[h * 128 + 64:(h + 1) * 128]
            # rotate-half == complex multiply of (a + ib) by e^{i angle}
            z = (a.astype(np.float64) + 1j * b) * np.exp(1j * ang[pos])
            assert np.abs(ra - z.real).max() < 1e-5 and np.abs(rb - z.imag).max() < 1e-5
    # predictor guard (code_predictor.rs:107): no row -> untouched
    assert np.array_equal(O.rope_apply(d, 8, 128, 5000, c, s), d)


def test_quantizer_round_trip():
    rng = np.random.Generator(np.random.PCG64(14))
    data = rng.standard_normal((8, 256)).astype(np.float32)
    packed, scales = O.quantize(data, 8, 256)
    w = synth.Q4(packed, scales, 8, 256)
    nib = np.concatenate([(packed & 0xF).ravel(), (packed >> 4).ravel()])
    assert nib.min() >= 1                              # never emits nibble 0 (F1c)
    err = np.abs(w.dequant() - data)
    s = scales.view(np.float16).astype(np.float32).repeat(32, axis=1)
    assert np.all(err <= 0.5 * s + 1e-3 * np.abs(data) + 1e-6)


# ---- argmax / sampler (code_predictor.rs:335-341, generate_new.rs:771-862) ----

def test_argmax_last_on_ties():
    assert O.argmax_last(np.array([1, 3, 2, 3, 0], np.float32)) == 3
    assert O.argmax_last(np.array([5.0], np.float32)) == 0
    assert O.argmax_last(np.array([-1, -1, -1], np.float32)) == 2
    assert O.argmax_last(np.array([0.0, -0.0], np.float32)) == 1


def _params(top_p, top_k=0):
    return hostdesc.sample_params(temperature=1.0, top_k=top_k, top_p=top_p, repetition_penalty=1.0)


def test_top_p_off_by_default():
    lg = np.array([2.0, 1.0, 0.5, 0.1], np.float32)
    for tp in (1.0, 0.0, -0.5, 2.0):
        seen = set()
        rng = 12345
        for _ in range(200):
            t, rng = O.sample_token(lg, _params(tp), [], rng, 1.0)
            seen.add(t)
        assert seen == {0, 1, 2, 3}


def test_top_p_cuts_tail():
    rng = 999
    for _ in range(50):
        t, rng = O.sample_token(np.array([5.0, 1.0, 1.0, 1.0], np.float32), _params(0.5), [], rng, 1.0)
        assert t == 0


def test_top_p_keeps_argmax_always():
    rng = 7
    for _ in range(20):
        t, rng = O.sample_token(np.array([3.0, 2.9, 2.8], np.float32), _params(0.01), [], rng, 1.0)
        assert t == 0


def test_top_k_one_is_greedy_with_lowest_index_ties():
    p = hostdesc.sample_params(temperature=0.9, top_k=1, repetition_penalty=1.0)
    rng = 5
    lg = np.array([0.5, 2.0, 1.0, 2.0], np.float32)
    for _ in range(20):
        t, rng = O.sample_token(lg, p, [], rng, 0.9)
        assert t == 1


def test_repetition_penalty_applies_per_history_entry():
    # index 0 appears 16 times in the zeroed history: penalised 16 times
    p = hostdesc.sample_params(temperature=1.0, top_k=1, repetition_penalty=1.05)
    lg = np.array([2.0, 1.7], np.float32)
    t, _ = O.sample_token(lg, p, [0] * 16, 1, 1.0)
    assert t == 1                          # 2.0 / 1.05**16 = 0.916 < 1.7
    t, _ = O.sample_token(lg, p, [0] * 2, 1, 1.0)
    assert t == 0                          # 2.0 / 1.05**2 = 1.81 > 1.7


def test_sampler_distribution_matches_softmax():
    # empirical frequencies of top-k 50 / T 0.9 sampling follow the renormalised softmax
    rng_np = np.random.Generator(np.random.PCG64(15))
    lg = (rng_np.standard_normal(3072) * 2).astype(np.float32)
    p = hostdesc.sample_params(temperature=0.9, top_k=50, repetition_penalty=1.0)
    s = lg.astype(np.float64) / 0.9
    e = np.exp(s - s.max())
    pr = e / e.sum()
    keep = np.argsort(-pr, kind="stable")[:50]
    q = np.zeros_like(pr)
    q[keep] = pr[keep]
    q /= q.sum()
    counts = np.zeros(3072)
    rng = 42
    N = 20000
    for _ in range(N):
        t, rng = O.sample_token(lg, p, [], rng, 0.9)
        counts[t] += 1
    assert set(np.nonzero(counts)[0]) <= set(keep)
    top = keep[:5]
    assert np.all(np.abs(counts[top] / N - q[top]) < 5 * np.sqrt(q[top] / N) + 1e-3)
