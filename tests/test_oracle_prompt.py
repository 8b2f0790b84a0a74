"""Pinning the oracle's prompt construction (generate_new.rs:82-476).

- frame_temperature and icl_block_layout against the reference's own unit
  tests (generate_new.rs:869-900, 966-976);
- build_icl_prefix is the first R rows of build_icl_block, bit for bit: the
  reference's prefix cache depends on it (generate_new.rs:240-243, the
  suffix path of :537-551);
- build_prefill_head (the prefix cache's head) and the rows that
  prefill_custom_voice assembles on its own are two restatements of two
  reference code paths that must agree row for row (the cached prefix plus a
  suffix prefill equals a full prefill, README:182), on both the voice and
  the built-in speaker paths;
- rows against the pinned primitives (embed_text_token, embed_codec_token,
  the Q4 row lookup), including the voice row's zero tail past a short
  embedding and the ICL block's codec-side sum order.
"""
import numpy as np
import pytest

import oracle as O
import qtts
from qtts import synth

IM_START, ASSISTANT, NEWLINE = 151644, 77091, 198
TTS_PAD, TTS_BOS, TTS_EOS = 151671, 151672, 151673
THINK, THINK_BOS, THINK_EOS, CODEC_PAD, CODEC_BOS = 2154, 2156, 2157, 2148, 2149


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def om():
    t = synth.make_talker(seed=601, n_layers=1, rope_max_pos=512)
    p = synth.make_predictor(seed=602, n_layers=1)
    O.set_workers(8, 8)
    m = O.Model(t, p, kv_cap=512)
    yield m
    m.close()


def test_frame_temperature_known_answers():
    # generate_new.rs:966-976
    p = qtts.sample_params(temperature=0.8, onset_frames=8, onset_temperature=0.3)
    assert O.frame_temperature(p, 0) == np.float32(0.3)
    assert O.frame_temperature(p, 7) == np.float32(0.3)
    assert O.frame_temperature(p, 8) == np.float32(0.8)
    assert O.frame_temperature(p, 500) == np.float32(0.8)
    p0 = qtts.sample_params(temperature=0.8, onset_frames=0, onset_temperature=0.3)
    assert O.frame_temperature(p0, 0) == np.float32(0.8)


@pytest.mark.parametrize("r,t,tv,icl,rem", [(8, 8, 23, 24, 0), (30, 30, 23, 24, 37), (11, 11, 22, 23, 0),
                                            (1, 1, 23, 24, 0)])
def test_icl_layout_known_answers(r, t, tv, icl, rem):
    # generate_new.rs:869-900
    assert O.icl_layout(r, t, tv) == (icl, rem)


def codec_rows(om, codes):
    """codec_full (generate_new.rs:159-172) from the pinned row lookups."""
    t, p = om.t, om.p
    rows = [om.embed_codec_token(CODEC_BOS)]
    for f in range(codes.shape[1]):
        s = om.embed_codec_token(int(codes[0, f]))
        for g in range(1, 16):
            s = s + O.embed_lookup(p.codec_embeddings[g - 1], int(codes[g, f])).astype(np.float32)
        rows.append(s.astype(np.float32))
    return np.stack(rows)


@pytest.mark.parametrize("n_ref,n_text,n_frames", [(5, 4, 12), (9, 20, 12), (3, 3, 6)])
def test_icl_block_from_primitives(om, n_ref, n_text, n_frames):
    rng = np.random.Generator(np.random.PCG64(610 + n_ref))
    ref = rng.integers(0, 151936, n_ref)
    text = rng.integers(0, 151936, n_text)
    codes = rng.integers(0, 2048, (16, n_frames))
    icl, rem = om.build_icl_block(ref, text, codes)
    text_full = np.stack([om.embed_text_token(int(x)) for x in list(ref) + list(text) + [TTS_EOS]])
    cod = codec_rows(om, codes)
    pad = om.embed_text_token(TTS_PAD)
    side = np.stack([text_full[i] if i < len(text_full) else pad for i in range(len(cod))])
    assert np.array_equal(bits(icl), bits(side + cod))
    assert np.array_equal(bits(rem), bits(text_full[len(cod):].reshape(-1, om.t.hidden)))


@pytest.mark.parametrize("n_ref,n_text,n_frames", [(5, 4, 12), (9, 20, 12), (12, 2, 12)])
def test_icl_prefix_is_the_blocks_head(om, n_ref, n_text, n_frames):
    """build_icl_prefix == build_icl_block[:R] bit for bit (pad branch,
    remainder branch, and R = Tv: the prefix reaches the last frame)."""
    rng = np.random.Generator(np.random.PCG64(620 + n_ref))
    ref = rng.integers(0, 151936, n_ref)
    text = rng.integers(0, 151936, n_text)
    codes = rng.integers(0, 2048, (16, n_frames))
    icl, _ = om.build_icl_block(ref, text, codes)
    pre = om.build_icl_prefix(ref, codes)
    assert pre.shape == (n_ref, om.t.hidden)
    assert np.array_equal(bits(pre), bits(icl[:n_ref]))


def test_icl_prefix_past_the_frames_is_codec_pad(om):
    # generate_new.rs:262-276: a ref token past the last frame meets CODEC_PAD
    rng = np.random.Generator(np.random.PCG64(630))
    ref = rng.integers(0, 151936, 6)
    codes = rng.integers(0, 2048, (16, 3))
    pre = om.build_icl_prefix(ref, codes)
    for i in (4, 5):
        assert np.array_equal(bits(pre[i]), bits(om.embed_text_token(int(ref[i])) + om.embed_codec_token(CODEC_PAD)))


@pytest.mark.parametrize("voice_len", [None, 2048, 1000])
def test_prefill_head_agrees_with_prefill_custom_voice(om, voice_len):
    rng = np.random.Generator(np.random.PCG64(640))
    voice = None if voice_len is None else rng.standard_normal(voice_len).astype(np.float32)
    spk, lang = 3000, 2055
    head = om.build_prefill_head(spk, lang, voice)
    text = rng.integers(0, 151936, 7)
    hid, lg, pos, rows = om.prefill_custom_voice(text, spk, lang, voice)
    assert pos == 10 and rows.shape[0] == 10
    assert np.array_equal(bits(rows[:9]), bits(head))
    # role prefix, then the rows from the primitives
    for i, tok in enumerate((IM_START, ASSISTANT, NEWLINE)):
        assert np.array_equal(bits(head[i]), bits(om.embed_text_token(tok)))
    pad, bos = om.embed_text_token(TTS_PAD), om.embed_text_token(TTS_BOS)
    c = om.embed_codec_token
    codec = [THINK, THINK_BOS, lang, THINK_EOS] + ([spk, CODEC_PAD] if voice is None else [])
    for i, tok in enumerate(codec):
        assert np.array_equal(bits(head[3 + i]), bits(c(tok) + (bos if i == 5 else pad)))
    if voice is not None:
        m = min(voice_len, om.t.hidden)
        v4 = np.zeros(om.t.hidden, np.float32)
        v4[:m] = voice[:m] + pad[:m]
        assert np.array_equal(bits(head[7]), bits(v4))
        assert np.array_equal(bits(head[8]), bits(c(CODEC_PAD) + bos))
    # BOS + first text token closes the non-ICL prompt
    assert np.array_equal(bits(rows[9]), bits(c(CODEC_BOS) + om.embed_text_token(int(text[0]))))
    # the prefill and codec head of those rows
    om.kv_reset()
    h2 = om.prefill(rows, 0)
    assert np.array_equal(bits(h2), bits(hid))
    assert np.array_equal(bits(om.codec_head(h2)), bits(lg))


def test_prefill_custom_voice_positions(om):
    # generate_new.rs:560-565: ICL 9 + block, else 10, or 9 with no text
    rng = np.random.Generator(np.random.PCG64(650))
    voice = rng.standard_normal(2048).astype(np.float32)
    ref = rng.integers(0, 151936, 4)
    text = rng.integers(0, 151936, 5)
    codes = rng.integers(0, 2048, (16, 8))
    icl, _ = om.build_icl_block(ref, text, codes)
    _, _, pos, rows = om.prefill_custom_voice(text, 0, 2055, voice, icl_rows=icl)
    assert pos == 9 + icl.shape[0] and np.array_equal(bits(rows[9:]), bits(icl))
    assert om.prefill_custom_voice([], 3000, 2055)[2] == 9
    # the prefix-cache split (generate_new.rs:307-316): prefix = head + icl prefix
    pre = om.build_icl_prefix(ref, codes)
    head = om.build_prefill_head(0, 2055, voice)
    assert np.array_equal(bits(np.concatenate([head, pre])), bits(rows[:9 + len(ref)]))


def test_trailing_text(om):
    # generate_new.rs:756-767
    rng = np.random.Generator(np.random.PCG64(660))
    toks = rng.integers(0, 151936, 4)
    tr = om.build_trailing_text(toks)
    assert tr.shape[0] == 4
    for i in range(3):
        assert np.array_equal(bits(tr[i]), bits(om.embed_text_token(int(toks[i + 1]))))
    assert np.array_equal(bits(tr[3]), bits(om.embed_text_token(TTS_EOS)))
    assert np.array_equal(bits(om.build_trailing_text([])), bits(om.embed_text_token(TTS_EOS)[None]))
