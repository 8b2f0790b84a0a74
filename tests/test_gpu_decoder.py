"""The speech decoder on the device (decode_to_audio, decoder.rs:395-584)
against the oracle's C restatement (oracle/qtts_decoder.c, itself pinned
against a float64 model and the reference's warmup-trim answers).

Bar: the waveform within 1e-3 of the oracle's peak amplitude (f32
matrix-core sums in another order than the reference's loops; the clamp to
[-1, 1] is the same).  Size-independent checks: warmup trimming equals
decoding the concatenation and dropping `warmup_trim_len` samples (bit for
bit, same kernels and sizes), and a decoder is causal, so a prefix of the
frames decodes to a prefix of the samples (within 1e-5).
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
    scale = max(np.abs(ref).max(), 1e-30)
    err = np.abs(np.asarray(got, np.float64) - ref).max()
    return err <= rel * scale, err / scale


def small_decoder(seed=11):
    return synth.make_decoder(seed=seed, latent=64, hidden=64, n_heads=4, head_dim=16, inter=128, n_tf_layers=2,
                              codebook_size=64, codebook_dim=32, vq_dim=32, vocos=(48, 32, 24, 16, 8),
                              rope_max_pos=512)


def codes_for(d, T, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.integers(0, d.codebook_size, (len(d.rest_codebooks) + 1, T)).astype(np.uint32)


@pytest.fixture(scope="module")
def small():
    return small_decoder()


@pytest.fixture(scope="module")
def ctx(ctx_factory, small):
    c = ctx_factory(64)
    c.upload_decoder(small)
    return c


@pytest.mark.parametrize("T", [1, 5, 80])
def test_decode_small_vs_oracle(ctx, small, T):
    codes = codes_for(small, T, 4000 + T)
    ref = O.decode_to_audio(small, codes, threads=16)
    got = ctx.decode_to_audio(codes)
    assert got.shape == ref.shape == (T * small.upsample_factor,)
    ok, e = close(got, ref)
    assert ok, f"T={T}: rel err {e}"


def test_decode_f32_instructions_vs_oracle(ctx, small, monkeypatch):
    """The f32-instruction convolutions (QTTS_DEC_F32=1) kept beside the
    split-f16 ones: against the oracle, and against the default path."""
    codes = codes_for(small, 40, 4050)
    ref = O.decode_to_audio(small, codes, threads=16)
    default = ctx.decode_to_audio(codes)
    monkeypatch.setenv("QTTS_DEC_F32", "1")
    got = ctx.decode_to_audio(codes)
    ok, e = close(got, ref)
    assert ok, f"rel err {e}"
    assert close(got, default)[0]


def test_decode_small_warmup_vs_oracle(ctx, small):
    codes, warm = codes_for(small, 30, 4100), codes_for(small, 12, 4101)
    ref = O.decode_to_audio(small, codes, warmup=warm, threads=16)
    got = ctx.decode_to_audio(codes, warmup=warm)
    total = 42 * small.upsample_factor
    assert got.size == ref.size == total - O.warmup_trim_len(12, 42, total)
    ok, e = close(got, ref)
    assert ok, f"rel err {e}"


def test_warmup_is_trimmed_concatenation(ctx, small):
    codes, warm = codes_for(small, 17, 4200), codes_for(small, 9, 4201)
    full = ctx.decode_to_audio(np.concatenate([warm, codes], axis=1))
    got = ctx.decode_to_audio(codes, warmup=warm)
    cut = O.warmup_trim_len(9, 26, full.size)
    assert np.array_equal(got.view(np.uint32), full[cut:].view(np.uint32))


CAUSAL_TOL = 1e-5


def test_decode_is_causal(ctx, small):
    """Every stage is causal (causal convs, left-looking attention window,
    right-cropped transposed convs), so frames past t leave samples up to t
    unchanged.  Within 1e-5 of the peak rather than bitwise: how a short
    stage splits its contraction across workgroups depends on the launch
    size, so two lengths may add the same products in another order."""
    codes = codes_for(small, 64, 4300)
    full = ctx.decode_to_audio(codes)
    head = ctx.decode_to_audio(codes[:, :40])
    ok, e = close(head, full[:head.size], rel=CAUSAL_TOL)
    assert ok, f"rel err {e}"


def test_decode_edges(ctx, small):
    ncb = len(small.rest_codebooks) + 1
    assert ctx.decode_to_audio(np.zeros((ncb, 0), np.uint32)).size == 0
    bad = codes_for(small, 4, 4400)
    bad[3, 2] = small.codebook_size
    with pytest.raises(qtts.QttsError) as e:
        ctx.decode_to_audio(bad)
    assert e.value.code == qtts.ERR_INVALID
    # sizes past the first workspace reuse / regrow it
    for T in (3, 120, 7):
        codes = codes_for(small, T, 4500 + T)
        ok, e = close(ctx.decode_to_audio(codes), O.decode_to_audio(small, codes, threads=16))
        assert ok, f"T={T}: rel err {e}"


def test_decode_without_decoder(ctx_factory):
    c = ctx_factory(64)
    with pytest.raises(qtts.QttsError) as e:
        c.decode_to_audio(np.zeros((16, 2), np.uint32))
    assert e.value.code == qtts.ERR_STATE


@pytest.mark.parametrize("f32", [False, True])
def test_snake_wide_arguments_vs_oracle(ctx_factory, monkeypatch, f32):
    """SnakeBeta arguments e^alpha * x past 2^14 take the epilogues'
    out-of-line sinf call (qtts_snake.h): with e^alpha = 1.2e6 every
    |x| >= 0.014 does, in the same waves whose smaller values take the
    series.  e^-beta = 1.1e-7 keeps sin^2's sensitivity to the rounding of
    x below the bar, so the comparison sees what the call could break
    around it: the epilogue's other values and registers (sin^2 itself is
    pinned on the host, test_snake_sin2.py)."""
    d = small_decoder(seed=23)
    for b in d.vocos_blocks:
        for r in b.residuals:
            r.act2_alpha = np.full_like(r.act2_alpha, 14.0)
            r.act2_beta = np.full_like(r.act2_beta, 16.0)
    c = ctx_factory(64)
    c.upload_decoder(d)
    if f32:
        monkeypatch.setenv("QTTS_DEC_F32", "1")
    codes = codes_for(d, 40, 4900)
    ref = O.decode_to_audio(d, codes, threads=16)
    got = c.decode_to_audio(codes)
    assert np.all(np.isfinite(got))
    ok, e = close(got, ref)
    assert ok, f"rel err {e}"


@pytest.fixture(scope="module")
def full():
    return synth.make_decoder(seed=7)


@pytest.fixture(scope="module")
def full_ctx(ctx_factory, full):
    c = ctx_factory(64)
    c.upload_decoder(full)
    return c


def test_decode_full_dims_vs_oracle(full_ctx, full):
    """The 12 Hz tokenizer's decoder shapes (16 codebooks of 2048 x 256, an
    8-layer 512-wide transformer, 1024-channel upsamplers, Vocos 1536 -> 96,
    1920 samples per frame) on 6 frames after 3 warmup frames."""
    d, c = full, full_ctx
    codes, warm = codes_for(d, 6, 4600), codes_for(d, 3, 4601)
    ref = O.decode_to_audio(d, codes, warmup=warm, threads=16)
    got = c.decode_to_audio(codes, warmup=warm)
    assert got.size == ref.size == 6 * 1920
    ok, e = close(got, ref)
    assert ok, f"rel err {e}"
    assert np.abs(ref).max() > 0.05            # a live signal, not a clamp or zeros


def test_decode_full_dims_longer_vs_oracle(full_ctx, full):
    """80 frames at the full shapes: the transformer (one position per
    frame) runs past its 72-position window, and the short stages split
    their contraction differently than at 9 frames."""
    d, c = full, full_ctx
    codes = codes_for(d, 80, 4700)
    ref = O.decode_to_audio(d, codes, threads=16)
    got = c.decode_to_audio(codes)
    ok, e = close(got, ref)
    assert ok, f"rel err {e}"


def test_fused_vocos_unit_bit_identical(full_ctx, full, monkeypatch):
    """The last Vocos block's residual units (96 channels: one row tile)
    run as one launch each at 80 frames -- the k 7 conv's snake output kept
    in LDS as the 1x1 conv's operand -- with the same bits as the two
    launches (QTTS_DEC_FUSE_VOC=0)."""
    codes = codes_for(full, 80, 5100)
    fused = full_ctx.decode_to_audio(codes)
    monkeypatch.setenv("QTTS_DEC_FUSE_VOC", "0")
    apart = full_ctx.decode_to_audio(codes)
    assert np.array_equal(fused.view(np.uint32), apart.view(np.uint32))


def test_fused_vocos_unit_column_tail(ctx_factory, monkeypatch):
    """The fused Vocos residual unit where the last column tile is partial:
    a small decoder whose one Vocos block keeps 96 channels at rate 8, 2049
    frames -> 65,568 positions = 512 whole 128-column tiles + 32 columns
    (the 12 Hz shapes always give whole tiles: 1920 samples a frame).
    Against the oracle, and bit-identical to the two launches."""
    d = synth.make_decoder(seed=29, latent=64, hidden=64, n_heads=4, head_dim=16, inter=128, n_tf_layers=2,
                           codebook_size=64, codebook_dim=32, vq_dim=32, vocos=(96, 96), rates=(8,),
                           rope_max_pos=4096)
    c = ctx_factory(64)
    c.upload_decoder(d)
    codes = codes_for(d, 2049, 5200)
    ref = O.decode_to_audio(d, codes, threads=16)
    got = c.decode_to_audio(codes)
    assert got.size == ref.size == 65568
    ok, e = close(got, ref)
    assert ok, f"rel err {e}"
    monkeypatch.setenv("QTTS_DEC_FUSE_VOC", "0")
    apart = c.decode_to_audio(codes)
    assert np.array_equal(got.view(np.uint32), apart.view(np.uint32))


def test_decode_full_dims_properties(full_ctx, full):
    """Warmup trim (bit-identical: same length, same kernels) and causality
    (within 1e-5, see test_decode_is_causal) at the full shapes, at lengths
    past the attention window (120 and 80 frames)."""
    d, c = full, full_ctx
    codes, warm = codes_for(d, 100, 4800), codes_for(d, 20, 4801)
    whole = c.decode_to_audio(np.concatenate([warm, codes], axis=1))
    got = c.decode_to_audio(codes, warmup=warm)
    cut = O.warmup_trim_len(20, 120, whole.size)
    assert np.array_equal(got.view(np.uint32), whole[cut:].view(np.uint32))
    head = c.decode_to_audio(np.concatenate([warm, codes], axis=1)[:, :80])
    ok, e = close(head, whole[:head.size], rel=CAUSAL_TOL)
    assert ok, f"rel err {e}"
