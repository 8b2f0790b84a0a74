"""The oracle's speech decoder (oracle/qtts_decoder.c) pinned against an
independent float64 model (tests/f64decoder.py) and the reference's own
known answers (warmup_trim_len, decoder.rs:692-703).  CPU only."""
import numpy as np
import pytest

import f64decoder as F
import oracle as O
from qtts import synth


def small_decoder(seed=11):
    return synth.make_decoder(seed=seed, latent=64, hidden=64, n_heads=4, head_dim=16, inter=128, n_tf_layers=2,
                              codebook_size=64, codebook_dim=32, vq_dim=32, vocos=(48, 32, 24, 16, 8),
                              rope_max_pos=512)


def rel(a, b):
    b = np.asarray(b, np.float64)
    return np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-30)


def test_warmup_trim_len_known_answers():
    assert O.warmup_trim_len(141, 175, 175 * 1920) == 141 * 1920
    assert O.warmup_trim_len(1, 3, 100) == 33
    assert O.warmup_trim_len(0, 10, 100) == 0
    assert O.warmup_trim_len(5, 0, 100) == 0
    assert O.warmup_trim_len(10, 10, 50) == 50


def bits32(v):
    return int(np.float32(v).view(np.uint32))


def test_reference_transpose_dw_goldens():
    """The reference's own bit-exact goldens (test_transpose_dw_golden,
    conv.rs:772-823): a 192 -> 96 transposed conv (kernel 4, stride 3,
    padding 1) over 3000 positions and a 96-channel depthwise conv (kernel
    7, causal) over 20000, inputs from its xorshift generator (seed 777):
    sums, three sampled output bits each and the 64-point sweep hash."""
    from refgen import XRng, rvec
    st = XRng(777)
    inp = rvec(st, 192 * 3000, 1.0).reshape(192, 3000)
    w = rvec(st, 192 * 96 * 4, 0.2).reshape(192, 96, 4)
    b = rvec(st, 96, 0.1)
    y = O.conv_transpose1d(inp, synth.ConvT1d(w, b, 192, 96, 4, 3, 1)).reshape(-1)
    assert y.size == 96 * ((3000 - 1) * 3 - 2 + 4)
    assert abs(float(y.sum(dtype=np.float64)) - 10309.475586) < 1.0
    assert bits32(y[0]) == bits32(0.11413957)
    assert bits32(y[12345]) == bits32(0.30676275)
    assert bits32(y[-1]) == bits32(0.7365111)
    step = y.size // 64
    acc = 0
    for n in range(0, 64 * step, step):
        acc = (acc + bits32(y[n]) * (n + 1)) % (1 << 64)
    assert acc == 59818250823433361
    inp2 = rvec(st, 96 * 20000, 1.0).reshape(96, 20000)
    w2 = rvec(st, 96 * 7, 0.2).reshape(96, 7)
    b2 = rvec(st, 96, 0.1)
    y2 = O.depthwise_conv1d(inp2, synth.DwConv(w2, b2, 96, 7, 6)).reshape(-1)
    assert abs(float(y2.sum(dtype=np.float64)) - -3754.235596) < 1.0
    assert bits32(y2[0]) == bits32(0.030722003)
    assert bits32(y2[765432]) == bits32(-0.250796)
    assert bits32(y2[-1]) == bits32(-0.10229)


def test_reference_gemm_bitexact_cases():
    """test_f32_gemm_bitexact (conv.rs:713-757): f32_gemm_bias equals the
    reference's naive same-order loop (bias first, k ascending, exact zeros
    of A skipped so a -0.0 bias keeps its sign) bit for bit, on its three
    shapes and xorshift inputs (seed 4242), with its planted zeros."""
    from refgen import XRng, rvec
    st = XRng(4242)
    for m, n, k in ((7, 13, 11), (64, 97, 48), (128, 482, 256)):
        a = rvec(st, m * k, 1.0)
        b = rvec(st, k * n, 0.5).reshape(k, n)
        bias = rvec(st, m, 0.1)
        a[0] = 0.0
        a[1] = -0.0
        bias[0] = -0.0
        a = a.reshape(m, k)
        expect = np.repeat(bias[:, None], n, axis=1).astype(np.float32)
        for kk in range(k):
            col = a[:, kk:kk + 1]
            expect = np.where(col == 0.0, expect, expect + col * b[kk][None, :]).astype(np.float32)
        got = O.gemm_bias(a, b, bias)
        assert np.array_equal(got.view(np.uint32), expect.view(np.uint32)), (m, n, k)
    # the -0.0 bias survives a row whose A entries are all zero
    z = O.gemm_bias(np.zeros((1, 3), np.float32), np.ones((3, 2), np.float32), np.array([-0.0], np.float32))
    assert np.signbit(z).all()


def test_conv_kernels_vs_f64():
    rng = np.random.Generator(np.random.PCG64(5))
    x = rng.standard_normal((24, 50)).astype(np.float32)
    for k, d in ((7, 1), (7, 3), (7, 9), (1, 1), (3, 1)):
        c = synth._conv(rng, 24, 20, k, d)
        assert rel(O.causal_conv1d(x, c), F.causal_conv(x, c)) < 1e-5, (k, d)
    # delta input: a causal conv returns its taps in time order, delayed
    delta = np.zeros((24, 50), np.float32)
    delta[3, 10] = 1.0
    c = synth._conv(rng, 24, 20, 7, 3)
    y = O.causal_conv1d(delta, c) - c.bias[:, None]
    for k in range(7):
        np.testing.assert_allclose(y[:, 10 + (6 - k) * 3], c.weight[:, 3, k], rtol=0, atol=1e-7)
    for k, s in ((16, 8), (10, 5), (6, 3), (2, 2)):
        c = synth._convt(rng, 24, 12, k, s)
        assert rel(O.conv_transpose1d(x, c), F.conv_t(x, c)) < 1e-5, (k, s)
    dw = synth.DwConv(rng.standard_normal((24, 7)).astype(np.float32), synth._vec(rng, 24), 24, 7, 3)
    assert rel(O.depthwise_conv1d(x, dw), F.depthwise(x, dw)) < 1e-5
    a, b, bias = rng.standard_normal((9, 24)), x, rng.standard_normal(9)
    assert rel(O.gemm_bias(a, b, bias), a @ b.astype(np.float64) + bias[:, None]) < 1e-5


def test_activations_and_norm_vs_f64():
    rng = np.random.Generator(np.random.PCG64(6))
    x = (2 * rng.standard_normal((16, 40))).astype(np.float32)
    al, be = synth._vec(rng, 16, 0, 0.3), synth._vec(rng, 16, 0, 0.3)
    assert rel(O.snake_beta(x, al, be), F.snake(x.astype(np.float64), al, be)) < 1e-5
    for v in (-3.0, -0.5, 0.0, 0.7, 4.0):
        assert abs(O.gelu(v) - F.gelu(v)) < 1e-6
    assert O.gelu(0.0) == 0.0
    g, b = synth._vec(rng, 16, 1, 0.1), synth._vec(rng, 16)
    assert rel(O.layer_norm_cf(x, g, b), F.layer_norm_cf(x.astype(np.float64), g, b)) < 1e-5
    # a constant channel column normalises to beta
    xc = np.ones((16, 3), np.float32)
    np.testing.assert_allclose(O.layer_norm_cf(xc, g, b), np.repeat(b[:, None], 3, axis=1), atol=1e-6)


@pytest.mark.parametrize("T,warm", [(5, 0), (80, 0), (30, 12)])
def test_decode_vs_f64(T, warm):
    """Whole decoder: T = 80 frames passes the 72-position attention window;
    a warmup prefix is decoded and trimmed as decode_to_audio does."""
    d = small_decoder()
    rng = np.random.Generator(np.random.PCG64(100 + T))
    codes = rng.integers(0, d.codebook_size, (16, T))
    warmup = rng.integers(0, d.codebook_size, (16, warm)) if warm else None
    got = O.decode_to_audio(d, codes, warmup)
    ref = F.decode(d, codes, warmup)
    assert got.shape == ref.shape == (T * d.upsample_factor,)
    assert rel(got, ref) < 1e-4
    assert 0.02 < np.abs(ref).mean() < 0.9          # not silent, not saturated
