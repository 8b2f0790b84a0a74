"""Numeric range of the device paths against the oracle.

The reference computes in f32 on any finite input (gemm_q4, gemv.rs:349-412;
f32_gemm_bias, conv.rs:434-526).  The device's matrix-core paths hold each
operand as f16 hi + lo:
- the prefill / API GEMM stages each row times a power of two that takes its
  largest |value| into [2^14, 2^15) (rows without a norm, from their
  measured maxima) or below a static bound (normed rows, the attention's
  q, k and v), and scales the sums back exactly;
- the speech decoder's convolutions check their inputs' range while staging
  and the decode is repeated on the f32 matrix path when a tile leaves it
  (a weight matrix outside it sends the decoder to the f32 path at upload).
The decode GEMV sums nib * a over nib in [0, 15] and subtracts 8 * sum(a)
once per column (a cancellation on shifted inputs), so it is tested on
shifted inputs and outliers too.

Bars: each GEMM row within 1e-3 of its own largest |reference output| (rows
are independent, so a tiny row is held to its own scale); model outputs
within 1e-3 of the oracle's as elsewhere; a decode whose inputs leave the
split's range equals the f32-path decode bit for bit (the repeat ran).
"""
import numpy as np
import pytest

import oracle as O
import qtts
from qtts import synth

pytestmark = pytest.mark.gpu

TOL = 1e-3


def close(got, ref, rel=TOL):
    ref = np.asarray(ref, np.float64)
    scale = max(np.abs(ref).max(), np.sqrt((ref ** 2).mean()), 1e-300)
    err = np.abs(np.asarray(got, np.float64) - ref).max()
    return err <= rel * scale, err / scale


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def scale_q4(w, e):
    """Scales times 2^e, in place (exact while the f16 results stay normal)."""
    s = w.scales.view(np.float16).astype(np.float32) * np.float32(2.0 ** e)
    w.scales[...] = s.astype(np.float16).view(np.uint16)


def scale_gamma(g, e):
    g[...] = (g.view(np.float16).astype(np.float32) * np.float32(2.0 ** e)).astype(np.float16).view(np.uint16)


@pytest.fixture(scope="module")
def ctx(ctx_factory):
    return ctx_factory(1024)


def extreme_rows(rng, k, n_rows=20):
    X = rng.standard_normal((n_rows, k)).astype(np.float32)
    X[0] *= 1e5                                   # every entry near or past the f16 maximum
    X[1] *= 1e-6                                  # every entry below the f16 normals
    X[2, 17] = 1e5                                # one outlier channel
    X[3] += 50.0                                  # shifted
    X[4] = np.abs(X[4]) + 8.0
    X[5] *= 1e-30                                 # near the f32 normals
    X[6] = 0.0
    X[7, ::2] *= 1e5                              # mixed magnitudes in one row
    X[7, 1::2] *= 1e-6
    X[8] *= 3e4
    return X


@pytest.mark.parametrize("k,n", [(2048, 4096), (6144, 2048), (3072, 1000)])
def test_gemm_mfma_extreme_rows(ctx, k, n):
    """qtts_gemm_q4 on the matrix cores (the reference's gemm) over rows of
    +-1e5, +-1e-6, 1e-30, zeros, an outlier channel, shifted and mixed
    entries: every row within 1e-3 of its own scale."""
    rng = np.random.Generator(np.random.PCG64(9100 + k))
    w = synth.q4_random(rng, k, n)
    X = extreme_rows(rng, k)
    dw = ctx.upload(w)
    Y = ctx.gemm(dw, X, path="mfma")
    dw.free()
    R = O.gemm(X, w)
    assert np.all(np.isfinite(Y))
    for r in range(X.shape[0]):
        if not np.any(R[r]):
            assert not np.any(Y[r]), f"row {r}: zero input, nonzero output"
            continue
        ok, e = close(Y[r], R[r])
        assert ok, f"row {r}: rel err {e}"


@pytest.mark.parametrize("cfg", range(len(qtts.TILE_SHAPES)))
def test_gemv_shifted_and_outlier_inputs(ctx, cfg, monkeypatch):
    """The decode GEMV's per-column -8 * sum(a) correction on non-zero-mean
    inputs (|N(0,1)| + 8, N(0,1) + 50) and one 1e4 outlier, every tile shape,
    against gemv_q4_scalar (gemv.rs:249-287)."""
    monkeypatch.setenv("QTTS_TILE_GEMV", str(cfg))
    rng = np.random.Generator(np.random.PCG64(9200 + cfg))
    for k, n in ((2048, 6144), (3072, 1000)):
        w = synth.q4_random(rng, k, n)
        xs = [np.abs(rng.standard_normal(k)).astype(np.float32) + 8.0,
              rng.standard_normal(k).astype(np.float32) + 50.0]
        xo = np.abs(rng.standard_normal(k)).astype(np.float32) + 8.0
        xo[k // 3] = 1e4
        xs.append(xo)
        dw = ctx.upload(w)
        for i, x in enumerate(xs):
            ok, e = close(ctx.gemv(dw, x), O.gemv_scalar(x, w))
            assert ok, f"cfg {cfg} {qtts.TILE_SHAPES[cfg]} k={k} n={n} input {i}: rel err {e}"
        dw.free()


def test_model_steps_on_shifted_inputs(ctx_factory):
    """A talker step (its gate|up + down launch keeps the byte-convert loop)
    and the predictor chain on shifted inputs with an outlier, against the
    oracle."""
    t = synth.make_talker(seed=9301, n_layers=2, text_vocab=256, rope_max_pos=512)
    p = synth.make_predictor(seed=9302, n_layers=5)
    c = ctx_factory(256)
    c.upload_model(t, p)
    om = O.Model(t, p, kv_cap=256)
    rng = np.random.Generator(np.random.PCG64(9303))
    K = rng.standard_normal((2, 100, 8, 128)).astype(np.float32)
    V = rng.standard_normal((2, 100, 8, 128)).astype(np.float32)
    c.kv_load(K, V)
    om.kv_load(K, V)
    emb = np.abs(rng.standard_normal(t.hidden)).astype(np.float32) + 8.0
    emb[123] = 1e4
    ok, e = close(c.forward_with_embedding(emb, 100), om.forward_with_embedding(emb, 100))
    assert ok, f"talker step rel err {e}"
    th = np.abs(rng.standard_normal(t.hidden)).astype(np.float32) + 8.0
    th[7] = 1e4
    sem = om.embed_codec_token(99)
    got, ref = c.generate_acoustic_codes(th, sem), om.predictor_chain(th, sem)
    assert (got == ref).mean() >= 14 / 15, f"codes {got} vs {ref}"
    om.close()


def scaled_talker(seed, case):
    t = synth.make_talker(seed=seed, n_layers=2, text_vocab=256, rope_max_pos=1024)
    for L in t.layers:
        if case == "huge":
            # v past the f16 maximum (attention v and the o-projection's
            # input), silu(gate) * up near 1e7 (the down projection's input)
            scale_q4(L.v_proj, 15)
            scale_q4(L.gate_proj, 10)
            scale_q4(L.up_proj, 10)
        else:
            # v near 1e-6 (input gamma and v_proj scaled down), the
            # o-projection scaled up so that the tiny attention rows decide
            # the residual; q / k gammas far from 1
            scale_gamma(L.input_norm, -11)
            scale_q4(L.v_proj, -11)
            scale_q4(L.o_proj, 15)
            scale_gamma(L.q_norm, 9)
            scale_gamma(L.k_norm, -9)
    return t


@pytest.mark.parametrize("case", ["huge", "tiny"])
def test_prefill_mfma_out_of_f16_range(ctx_factory, case):
    """The 2-layer matrix-core prefill (100 rows) with activations past the
    f16 maximum or below its normals inside the layer (attention v, the
    o-projection's and the down projection's inputs, normed rows with
    gammas far from 1): hidden and every cached K / V row against the
    oracle."""
    t = scaled_talker(9400 + (case == "tiny"), case)
    p = synth.make_predictor(seed=9402, n_layers=1)
    c = ctx_factory(256)
    c.upload_model(t, p)
    om = O.Model(t, p, kv_cap=256)
    X = np.random.Generator(np.random.PCG64(9403)).standard_normal((100, t.hidden)).astype(np.float32)
    if case == "tiny":
        X *= np.float32(1e-3)                     # the attention path, not the input, decides the residual
    ref = om.prefill(X, 0)
    got = c.prefill_talker_raw_from(X, 0, path="mfma")
    ok, e = close(got, ref)
    assert ok, f"{case}: hidden rel err {e}"
    for l in range(2):
        k, v = c.kv_gather(l)
        rk, rv = om.kv_layer(l)
        for pos in range(0, 100, 9):
            ok_k, ek = close(k[pos], rk[pos])
            ok_v, ev = close(v[pos], rv[pos])
            assert ok_k and ok_v, f"{case}: layer {l} position {pos}: K rel err {ek}, V {ev}"
    om.close()


@pytest.mark.parametrize("e", [17, -14])
def test_text_projection_out_of_f16_range(ctx_factory, e):
    """The text projection on the matrix cores (fc1 + bias, SiLU, fc2 +
    bias, talker.rs:105-116) with table rows past the f16 maximum or below
    its normals: each row against the oracle's embed_text_token."""
    t = synth.make_talker(seed=9500, n_layers=1, text_vocab=256, rope_max_pos=64)
    scale_q4(t.text_embedding, e)
    p = synth.make_predictor(seed=9501, n_layers=1)
    c = ctx_factory(64)
    c.upload_model(t, p)
    om = O.Model(t, p, kv_cap=64)
    ids = np.arange(0, 256, 11)
    rows = c.embed_text_tokens(ids)
    for i, tok in enumerate(ids):
        ok, err = close(rows[i], om.embed_text_token(int(tok)))
        assert ok, f"2^{e}: id {tok}: rel err {err}"
    om.close()


def small_decoder(seed, **kw):
    return synth.make_decoder(seed=seed, latent=64, hidden=64, n_heads=4, head_dim=16, inter=128, n_tf_layers=2,
                              codebook_size=64, codebook_dim=32, vq_dim=32, vocos=(48, 32, 24, 16, 8),
                              rope_max_pos=512, **kw)


@pytest.mark.parametrize("case", ["codebooks_1e5", "codebooks_1e-7", "weights_1e6", "plain"])
def test_decoder_out_of_f16_range(ctx_factory, monkeypatch, case):
    """The speech decoder with convolution inputs past the f16 maximum or
    below its normals (codebooks scaled), or a weight matrix past it: the
    decode equals the f32-path decode bit for bit (the range check sent it
    there) and the oracle's within 1e-3 of the peak; the plain decoder stays
    on the split-f16 path (other bits than the f32 path)."""
    d = small_decoder(9600)
    if case == "codebooks_1e5":
        d.first_codebook *= np.float32(1e5)
        for cb in d.rest_codebooks:
            cb *= np.float32(1e5)
    elif case == "codebooks_1e-7":
        d.first_codebook *= np.float32(1e-7)
        for cb in d.rest_codebooks:
            cb *= np.float32(1e-7)
    elif case == "weights_1e6":
        # a ConvNeXt pointwise pair scaled by 1e6 and 1e-6: its inner rows
        # (after GELU) near 1e6 and the second matrix's weights near 1e-7,
        # both outside the split's range; the product keeps its scale
        U = d.upsample[0]
        U.pw1_w *= np.float32(1e6)
        U.pw1_b *= np.float32(1e6)
        U.pw2_w *= np.float32(1e-6)
    c = ctx_factory(64)
    c.upload_decoder(d)
    codes = np.random.Generator(np.random.PCG64(9601)).integers(0, 64, (16, 24)).astype(np.uint32)
    got = c.decode_to_audio(codes)
    monkeypatch.setenv("QTTS_DEC_F32", "1")
    f32 = c.decode_to_audio(codes)
    monkeypatch.delenv("QTTS_DEC_F32")
    ref = O.decode_to_audio(d, codes, threads=16)
    scale = max(np.abs(ref).max(), 1e-30)
    assert np.abs(got.astype(np.float64) - ref).max() <= TOL * scale
    if case == "plain":
        assert not np.array_equal(bits(got), bits(f32))
    else:
        assert np.array_equal(bits(got), bits(f32))
