"""The frame's trailing-text fusion on the device against the oracle.

Every frame adds one text row to the talker's next input: trailing_text[f]
while f < len(trailing_text), tts_pad after (generate_new.rs:645-654).
trailing_text is the text after the first token plus TTS_EOS
(build_trailing_text, generate_new.rs:756-767), or the ICL block's
remainder (generate_new.rs:567-574).  The device takes the rows through
qtts_gen_set_text and picks the row of frame f inside the frame graph
(k_combine), from the frame counter kept in device state across calls.

Bars: code 0 exact and >= 99% of the other codes on teacher-forced greedy
frames, logits and hidden within 1e-3 of the oracle's after the last
frame; free-running frames equal to the oracle's up to their first
divergence, which must lie past the switch from text rows to pad.  Layer
0's cached V row of a frame is a function of that frame's input alone, so
those rows pin each frame's text row (a pad-only oracle run leaves other V
rows: the check tells text rows from pad).  The chunk test runs one generate_speech chunk (generate_new.rs:
479-722) end to end: prompt, trailing text, sampled frames, decode_to_audio.
"""
import numpy as np
import pytest

import oracle as O
import qtts
from qtts import synth

pytestmark = pytest.mark.gpu

TOL = 1e-3
TTS_PAD = 151671


def close(got, ref, rel=TOL):
    ref = np.asarray(ref, np.float64)
    scale = max(np.abs(ref).max(), np.sqrt((ref ** 2).mean()), 1e-30)
    err = np.abs(np.asarray(got, np.float64) - ref).max()
    return err <= rel * scale, err / scale


@pytest.fixture(scope="module")
def model():
    t = synth.make_talker(seed=601, n_layers=4, rope_max_pos=2048)
    p = synth.make_predictor(seed=602, n_layers=5)
    return t, p


@pytest.fixture(scope="module")
def ctx(ctx_factory, model):
    c = ctx_factory(1024)
    c.upload_model(*model)
    return c


@pytest.fixture(scope="module")
def om(model):
    O.set_workers(16, 8)
    m = O.Model(*model, kv_cap=1024)
    yield m
    m.close()


def start(ctx, om, t, seed, n=16):
    """The same prefilled prompt of n random rows on both sides:
    (hidden, logits) after it."""
    rng = np.random.Generator(np.random.PCG64(seed))
    X = rng.standard_normal((n, t.hidden)).astype(np.float32)
    ctx.kv_reset()
    om.kv_reset()
    hid = om.prefill(X, 0)
    ctx.prefill_talker_raw_from(X, 0)
    return X, hid, om.codec_head(hid)


def text_rows(ctx, seed, n):
    rng = np.random.Generator(np.random.PCG64(seed))
    return ctx.embed_text_tokens(rng.integers(0, 151936, n)), ctx.embed_text_token(TTS_PAD)


def oracle_frames(om, params, rows, pad, n):
    """n oracle frames fed rows[f] while f < len(rows), pad after."""
    return np.stack([om.frame(params, rows[f] if f < len(rows) else pad)[0] for f in range(n)])


def first_divergence(a, b):
    same = np.all(a == b, axis=1)
    return int(np.argmin(same)) if not same.all() else len(same)


def test_text_rows_teacher_forced_split(ctx, om, model):
    """Five text rows then pad, nine greedy frames teacher-forced in two
    calls (3 + 6): the row index carries across the split.  Layer 0's
    cached V row of frame f is v_proj(norm(input of frame f)), so the V rows
    at positions 16..24 pin each frame's input row; the same frames fed
    pad only leave other V rows at positions 16..20, so the check tells the
    text rows from pad."""
    t, _ = model
    params = qtts.sample_params(top_k=1, eos_enabled=False)
    X, hid, logits = start(ctx, om, t, 7001)
    rows, pad = text_rows(ctx, 7002, 5)
    om.gen_begin(logits, hid, 16, 42)
    ref = oracle_frames(om, params, rows, pad, 9)
    ref_lg, ref_hd = om.g_logits.copy(), om.g_hidden.copy()
    ref_k, ref_v = om.kv_layer(0)
    om.kv_reset()
    om.prefill(X, 0)
    om.gen_begin(logits, hid, 16, 42)
    for f in range(9):
        om.frame(params, pad, forced=ref[f])
    _, pad_v = om.kv_layer(0)
    for f in range(5):
        assert not close(pad_v[16 + f], ref_v[16 + f], 1e-2)[0], f"frame {f}: text row and pad alike"

    ctx.gen_set_text(rows, pad)
    ctx.gen_begin(logits, hid, 16, 42, params)
    pred = np.concatenate([ctx.gen_frames_forced(ref[:3]), ctx.gen_frames_forced(ref[3:])])
    assert np.array_equal(pred[:, 0], ref[:, 0]), f"code 0: {pred[:, 0]} vs {ref[:, 0]}"
    assert (pred[:, 1:] == ref[:, 1:]).mean() >= 0.99
    lg, hd, pos, _ = ctx.gen_state()
    assert pos == 16 + 9
    k0, v0 = ctx.kv_gather(0)
    for f in range(9):
        ok_k, ek = close(k0[16 + f], ref_k[16 + f])
        ok_v, ev = close(v0[16 + f], ref_v[16 + f])
        assert ok_k and ok_v, f"frame {f}: layer-0 K rel err {ek}, V {ev}"
    ok_l, el = close(lg, ref_lg)
    ok_h, eh = close(hd, ref_hd)
    assert ok_l and ok_h, f"logits rel err {el}, hidden {eh}"


def test_text_rows_forced_prefix_then_free_running(ctx, om, model):
    """Three teacher-forced frames, then free-running greedy frames in two
    more calls (graph replays): the rows continue at frame 3 and switch to
    pad at frame 5."""
    t, _ = model
    params = qtts.sample_params(top_k=1, eos_enabled=False)
    _, hid, logits = start(ctx, om, t, 7011)
    rows, pad = text_rows(ctx, 7012, 5)
    om.gen_begin(logits, hid, 16, 42)
    ref = oracle_frames(om, params, rows, pad, 10)
    ctx.gen_set_text(rows, pad)
    ctx.gen_begin(logits, hid, 16, 42, params)
    head = ctx.gen_frames_forced(ref[:3])
    assert np.array_equal(head[:, 0], ref[:3, 0])
    got = np.concatenate([ctx.gen_frames(3)[0], ctx.gen_frames(4)[0]])
    assert got.shape == (7, 16)
    d = first_divergence(got, ref[3:])
    assert d >= 3, f"free-running frames diverge at frame {3 + d}: {got[:, 0]} vs {ref[3:, 0]}"
    if d == 7:
        lg, hd, _, _ = ctx.gen_state()
        assert close(lg, om.g_logits)[0] and close(hd, om.g_hidden)[0]


def test_text_rows_sampled(ctx, om, model):
    """The default sampler (top-k 50, T 0.9, penalty 1.05, seed 42) over six
    text rows then pad: the free-running frames and the RNG follow the
    oracle's draw for draw."""
    t, _ = model
    params = qtts.sample_params(eos_enabled=False)
    _, hid, logits = start(ctx, om, t, 7021)
    rows, pad = text_rows(ctx, 7022, 6)
    om.gen_begin(logits, hid, 16, 42)
    ref = oracle_frames(om, params, rows, pad, 9)
    ctx.gen_set_text(rows, pad)
    ctx.gen_begin(logits, hid, 16, 42, params)
    got, eos = ctx.gen_frames(9)
    assert not eos and got.shape == (9, 16)
    d = first_divergence(got, ref)
    assert d >= 6, f"sampled frames diverge at frame {d}: {got[:, 0]} vs {ref[:, 0]}"
    if d == 9:
        lg, hd, _, rng_state = ctx.gen_state()
        assert rng_state == om.gen.rng
        assert close(lg, om.g_logits)[0] and close(hd, om.g_hidden)[0]


def test_icl_remainder_rows(ctx, om, model):
    """ICL prompt (voice clone): build_icl_block's remainder rows are the
    trailing text (generate_new.rs:567-570).  Prompt prefilled on both
    sides, then 32 teacher-forced greedy frames; the remainder (30 rows)
    runs out at frame 30."""
    t, _ = model
    rng = np.random.Generator(np.random.PCG64(7031))
    voice = rng.standard_normal(t.hidden).astype(np.float32)
    ref_tokens = rng.integers(0, 151936, 10)
    text = rng.integers(0, 151936, 40)
    codes = rng.integers(0, 2048, (16, 20))
    icl, rem = ctx.build_icl_block(ref_tokens, text, codes)
    assert rem.shape[0] == 30
    ctx.kv_reset()
    om.kv_reset()
    hid, lg, pos = ctx.prefill_custom_voice(text, 0, 2055, voice, icl)
    ohid, olg, opos, _ = om.prefill_custom_voice(text, 0, 2055, voice, icl)
    assert pos == opos
    pad = ctx.embed_text_token(TTS_PAD)
    params = qtts.sample_params(top_k=1, eos_enabled=False)
    om.gen_begin(olg, ohid, opos, 42)
    ref = oracle_frames(om, params, rem, pad, 32)
    ctx.gen_set_text(rem, pad)
    ctx.gen_begin(olg, ohid, opos, 42, params)
    pred = np.concatenate([ctx.gen_frames_forced(ref[:29]), ctx.gen_frames_forced(ref[29:])])
    assert np.array_equal(pred[:, 0], ref[:, 0]), f"code 0: {pred[:, 0]} vs {ref[:, 0]}"
    assert (pred[:, 1:] == ref[:, 1:]).mean() >= 0.99
    glg, ghd, gpos, _ = ctx.gen_state()
    assert gpos == opos + 32
    assert close(glg, om.g_logits)[0] and close(ghd, om.g_hidden)[0]
    _, v0 = ctx.kv_gather(0)
    _, ref_v = om.kv_layer(0)
    for f in range(32):
        ok, e = close(v0[opos + f], ref_v[opos + f])
        assert ok, f"frame {f}: layer-0 V rel err {e}"


def test_chunk_end_to_end(ctx, om, model):
    """One generate_speech chunk (generate_new.rs:479-722), built-in
    speaker: the prompt (prefill_custom_voice), the trailing text
    (build_trailing_text), sampled frames and decode_to_audio, on the
    device against the oracle's chain.  The frames match up to their first
    divergence; the decoder is causal, so the audio of the common frames is
    compared (within 1e-3 of the oracle's peak)."""
    t, _ = model
    rng = np.random.Generator(np.random.PCG64(7041))
    text = rng.integers(0, 151936, 7)
    ctx.kv_reset()
    om.kv_reset()
    hid, lg, pos = ctx.prefill_custom_voice(text, 3000, 2055)
    ohid, olg, opos, _ = om.prefill_custom_voice(text, 3000, 2055)
    assert pos == opos == 10
    assert close(hid, ohid)[0] and close(lg, olg)[0]
    trail = ctx.build_trailing_text(text)
    assert trail.shape[0] == 7 and close(trail, om.build_trailing_text(text))[0]
    pad = ctx.embed_text_token(TTS_PAD)
    params = qtts.sample_params(eos_enabled=False)
    n = 12
    # both sides sample from their own prompt; the oracle's rows for its own
    # trailing text
    om.gen_begin(olg, ohid, opos, 42)
    ref = oracle_frames(om, params, om.build_trailing_text(text), pad, n)
    ctx.gen_set_text(trail, pad)
    ctx.gen_begin(lg, hid, pos, 42, params)
    got, eos = ctx.gen_frames(n)
    assert not eos and got.shape == (n, 16)
    d = first_divergence(got, ref)
    assert d >= 8, f"chunk frames diverge at frame {d}: {got[:, 0]} vs {ref[:, 0]}"
    dec = synth.make_decoder(seed=7042, latent=64, hidden=64, n_heads=4, head_dim=16, inter=128, n_tf_layers=2,
                             codebook_size=3072, codebook_dim=32, vq_dim=32, vocos=(48, 32, 24, 16, 8),
                             rope_max_pos=512)
    ctx.upload_decoder(dec)
    audio = ctx.decode_to_audio(got.T.copy())
    ref_audio = O.decode_to_audio(dec, ref.T.copy(), threads=16)
    spf = dec.upsample_factor
    assert audio.shape == ref_audio.shape == (n * spf,)
    ok, e = close(audio[:d * spf], ref_audio[:d * spf])
    assert ok, f"audio of the first {d} frames: rel err {e}"
    ctx.kv_reset()
    om.kv_reset()
