"""Prompt construction on the device and the talker prefix cache.

- embed_text_token over a batch (talker.rs:105-116): within the GEMV bar of
  the oracle, and bit-identical for an id wherever it sits in a batch (the
  prefix cache depends on it);
- build_icl_block (generate_new.rs:140-195): codec side bit-exact (rows are
  exact Q4 values summed in the reference's order), text side as above, on
  the three layouts of the reference's own tests;
- prefix capture / attach (TalkerPrefixCache, generate_new.rs:317-355,
  537-551): prefix + suffix prefill is bit-identical to one full prefill,
  hidden and every layer's cache, and the prefix survives the sequence
  rewriting its cache (copy-on-write);
- the prompt head (build_prefill_head, build_icl_prefix,
  build_trailing_text, prefill_custom_voice; generate_new.rs:91-476): rows
  bit-identical to the device's text rows plus the exact codec rows in the
  reference's arrangement, within the bar of the oracle, and the reference's
  prefix-cache path (head + ICL prefix kept, block suffix prefilled) equal
  to prefill_custom_voice over the whole prompt bit for bit.
"""
import numpy as np
import pytest

import oracle as O
import qtts
from qtts import synth

pytestmark = pytest.mark.gpu

TOL = 1e-3
TTS_PAD, TTS_EOS, CODEC_BOS = 151671, 151673, 2149


def close(got, ref, rel=TOL):
    ref = np.asarray(ref, np.float64)
    scale = max(np.abs(ref).max(), np.sqrt((ref ** 2).mean()), 1e-30)
    err = np.abs(np.asarray(got, np.float64) - ref).max()
    return err <= rel * scale, err / scale


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def model():
    t = synth.make_talker(seed=501, n_layers=2, rope_max_pos=2048)
    p = synth.make_predictor(seed=502, n_layers=5)
    return t, p


@pytest.fixture(scope="module")
def ctx(ctx_factory, model):
    c = ctx_factory(1024)
    c.upload_model(*model)
    return c


@pytest.fixture(scope="module")
def om(model):
    O.set_workers(16, 8)
    m = O.Model(*model, kv_cap=64)
    yield m
    m.close()


def test_embed_text_tokens_batch(ctx, om):
    rng = np.random.Generator(np.random.PCG64(3001))
    ids = rng.integers(0, 151936, 37)
    rows = ctx.embed_text_tokens(ids)
    for i, tok in enumerate(ids[:12]):
        ok, e = close(rows[i], om.embed_text_token(int(tok)))
        assert ok, f"id {tok}: rel err {e}"
    # the same id gives the same bits alone, first or last in a batch
    one = ctx.embed_text_tokens(ids[5:6])
    assert np.array_equal(bits(one[0]), bits(rows[5]))
    tail = ctx.embed_text_tokens(np.concatenate([ids[:3], ids[5:6]]))
    assert np.array_equal(bits(tail[3]), bits(rows[5]))


def codec_side(t, p, codes):
    """Codec side of the ICL block in f32, the reference's order
    (generate_new.rs:161-172)."""
    rows = [O.embed_lookup(t.codec_embedding, CODEC_BOS)]
    for f in range(codes.shape[1]):
        s = O.embed_lookup(t.codec_embedding, int(codes[0, f])).astype(np.float32)
        for g in range(1, 16):
            s = s + O.embed_lookup(p.codec_embeddings[g - 1], int(codes[g, f])).astype(np.float32)
        rows.append(s)
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("n_ref,n_text,n_frames", [(8, 8, 23), (30, 30, 23), (11, 11, 22), (1, 1, 23)])
def test_icl_block(ctx, model, om, n_ref, n_text, n_frames):
    t, p = model
    rng = np.random.Generator(np.random.PCG64(3100 + n_ref))
    ref = rng.integers(0, 151936, n_ref)
    text = rng.integers(0, 151936, n_text)
    codes = rng.integers(0, 2048, (16, n_frames))
    icl, rem = ctx.build_icl_block(ref, text, codes)
    icl_len, rem_len = qtts.icl_layout(n_ref, n_text, n_frames)
    assert icl.shape == (icl_len, t.hidden) and rem.shape == (rem_len, t.hidden)
    # text side through the same batched projection
    text_full = ctx.embed_text_tokens(np.concatenate([ref, text, [TTS_EOS]]))
    pad = ctx.embed_text_tokens([TTS_PAD])[0]
    side = np.stack([text_full[i] if i < len(text_full) else pad for i in range(icl_len)])
    expect = (side + codec_side(t, p, codes)).astype(np.float32)
    assert np.array_equal(bits(icl), bits(expect))
    assert np.array_equal(bits(rem), bits(text_full[icl_len:]))
    # text side against the oracle's per-token projection
    ok, e = close(text_full[-1], om.embed_text_token(TTS_EOS))
    assert ok, f"tts_eos rel err {e}"


def test_prefix_attach_bit_identical(ctx, model):
    """A 109-position prefix (9 head rows + 100 reference rows) kept once;
    two chunks attach it and prefill their suffixes; each equals a full
    prefill of the same rows bit for bit, and the prefix outlives a reset
    and a rewrite of the sequence's cache."""
    t, p = model
    rng = np.random.Generator(np.random.PCG64(3200))
    P = 109
    head = rng.standard_normal((P, t.hidden)).astype(np.float32)
    suf_a = rng.standard_normal((291, t.hidden)).astype(np.float32)
    suf_b = rng.standard_normal((150, t.hidden)).astype(np.float32)

    def full(X):
        ctx.kv_reset()
        h = ctx.prefill_talker_raw_from(X, 0, path="mfma")
        return h, [ctx.kv_gather(l) for l in range(len(t.layers))]

    ha, kva = full(np.concatenate([head, suf_a]))
    hb, kvb = full(np.concatenate([head, suf_b]))

    ctx.kv_reset()
    ctx.prefill_talker_raw_from(head, 0, path="mfma")
    pfx = ctx.prefix_capture()
    assert pfx.len == P
    for suffix, h_ref, kv_ref in ((suf_a, ha, kva), (suf_b, hb, kvb), (suf_a, ha, kva)):
        ctx.prefix_attach(pfx)
        assert ctx.kv_len() == P
        h = ctx.prefill_talker_raw_from(suffix, P, path="mfma")
        assert np.array_equal(bits(h), bits(h_ref))
        for l in range(len(t.layers)):
            k, v = ctx.kv_gather(l)
            assert np.array_equal(bits(k), bits(kv_ref[l][0])) and np.array_equal(bits(v), bits(kv_ref[l][1]))
        # the sequence rewrites positions inside the shared pages
        ctx.kv_reset()
        ctx.prefill_talker_raw_from(suf_b[:100], 0, path="mfma")
    pfx.free()
    ctx.kv_reset()


def test_prefix_then_frames(ctx, model):
    """Greedy frames after attach + suffix equal the frames after a full
    prefill (same cache bits, same kernels)."""
    t, p = model
    rng = np.random.Generator(np.random.PCG64(3300))
    X = rng.standard_normal((140, t.hidden)).astype(np.float32)
    params = qtts.sample_params(top_k=1, eos_enabled=False)
    pad = ctx.embed_text_tokens([TTS_PAD])[0]
    ctx.gen_set_text(None, pad)

    def frames(h):
        ctx.gen_begin(ctx.apply_codec_head(h), h, 140, 42, params)
        return ctx.gen_frames(12)[0]

    ctx.kv_reset()
    ref = frames(ctx.prefill_talker_raw_from(X, 0, path="mfma"))
    ctx.kv_reset()
    ctx.prefill_talker_raw_from(X[:70], 0, path="mfma")
    pfx = ctx.prefix_capture()
    ctx.prefix_attach(pfx)
    got = frames(ctx.prefill_talker_raw_from(X[70:], 70, path="mfma"))
    assert np.array_equal(got, ref)
    pfx.free()
    ctx.kv_reset()


def test_shorter_prefix_over_longer(ctx, model):
    """Attach a 200-position prefix A, then a 64-position prefix B: the
    sequence's pages past B's end were A's.  Steps and frames after B write
    positions 64..150 into private pages, so A is untouched: attaching A
    again and prefilling a suffix equals one full prefill bit for bit."""
    t, p = model
    rng = np.random.Generator(np.random.PCG64(3350))
    XA = rng.standard_normal((200, t.hidden)).astype(np.float32)
    XB = rng.standard_normal((64, t.hidden)).astype(np.float32)
    suf = rng.standard_normal((50, t.hidden)).astype(np.float32)
    ctx.kv_reset()
    h_ref = ctx.prefill_talker_raw_from(np.concatenate([XA, suf]), 0, path="mfma")
    kv_ref = [ctx.kv_gather(l) for l in range(len(t.layers))]
    ctx.kv_reset()
    ctx.prefill_talker_raw_from(XA, 0, path="mfma")
    a = ctx.prefix_capture()
    ctx.kv_reset()
    hb = ctx.prefill_talker_raw_from(XB, 0, path="mfma")
    b = ctx.prefix_capture()
    ctx.prefix_attach(a)
    ctx.prefix_attach(b)
    assert ctx.kv_len() == 64
    for i in range(3):
        ctx.forward_with_embedding(rng.standard_normal(t.hidden).astype(np.float32), 64 + i)
    pad = ctx.embed_text_tokens([TTS_PAD])[0]
    ctx.gen_set_text(None, pad)
    ctx.gen_begin(ctx.apply_codec_head(hb), hb, 67, 42, qtts.sample_params(eos_enabled=False))
    codes, _ = ctx.gen_frames(84)
    assert codes.shape[0] == 84 and ctx.kv_len() == 151
    ctx.prefix_attach(a)
    h = ctx.prefill_talker_raw_from(suf, 200, path="mfma")
    assert np.array_equal(bits(h), bits(h_ref))
    for l in range(len(t.layers)):
        k, v = ctx.kv_gather(l)
        assert np.array_equal(bits(k), bits(kv_ref[l][0])) and np.array_equal(bits(v), bits(kv_ref[l][1]))
    a.free()
    b.free()
    ctx.kv_reset()


def test_prefix_pool_capacity(ctx_factory, model):
    """kv_capacity 256: 4 sequence pages + 4 spare.  A kept prefix pins its
    pages; once the sequence has unshared them the pool is exhausted and a
    second capture fails cleanly until the first prefix is freed."""
    c = ctx_factory(256)
    c.upload_model(*model)
    rng = np.random.Generator(np.random.PCG64(3400))
    X = rng.standard_normal((200, model[0].hidden)).astype(np.float32)
    c.prefill_talker_raw_from(X, 0, path="mfma")
    a = c.prefix_capture()                         # 3 shared pages + 1 copied
    c.kv_reset()                                   # unshares 3 pages: pool empty
    c.prefill_talker_raw_from(X[:100], 0, path="mfma")
    with pytest.raises(qtts.QttsError) as e:
        c.prefix_capture()
    assert e.value.code == qtts.ERR_CAPACITY
    a.free()
    b = c.prefix_capture()
    assert b.len == 100
    c.prefix_attach(b)
    assert c.kv_len() == 100
    b.free()
    c.close()


IM_START, ASSISTANT, NEWLINE, TTS_BOS = 151644, 77091, 198, 151672
THINK, THINK_BOS, THINK_EOS, CODEC_PAD = 2154, 2156, 2157, 2148


@pytest.mark.parametrize("voice_len", [None, 2048, 1000])
def test_prefill_head(ctx, model, om, voice_len):
    """build_prefill_head (generate_new.rs:222-237) on the device: bit for
    bit the device's own text rows plus the exact codec rows in the
    reference's arrangement, and within the bar of the oracle's head."""
    t, p = model
    rng = np.random.Generator(np.random.PCG64(3500))
    voice = None if voice_len is None else rng.standard_normal(voice_len).astype(np.float32)
    spk, lang = 3000, 2055
    head = ctx.build_prefill_head(spk, lang, voice)
    T = ctx.embed_text_tokens([IM_START, ASSISTANT, NEWLINE, TTS_PAD, TTS_BOS])
    c = om.embed_codec_token
    exp = [T[0], T[1], T[2]]
    codec = [THINK, THINK_BOS, lang, THINK_EOS]
    exp += [c(k) + T[3] for k in codec]
    if voice is None:
        exp += [c(spk) + T[3], c(CODEC_PAD) + T[4]]
    else:
        m = min(voice_len, t.hidden)
        v4 = np.zeros(t.hidden, np.float32)
        v4[:m] = voice[:m] + T[3][:m]
        exp += [v4, c(CODEC_PAD) + T[4]]
    assert np.array_equal(bits(head), bits(np.stack(exp)))
    ref = om.build_prefill_head(spk, lang, voice)
    for i in range(9):
        ok, e = close(head[i], ref[i])
        assert ok, f"row {i}: rel err {e}"


@pytest.mark.parametrize("n_ref,n_text,n_frames", [(8, 8, 23), (30, 30, 23), (5, 3, 3)])
def test_icl_prefix_is_the_blocks_head(ctx, n_ref, n_text, n_frames):
    """build_icl_prefix on the device is bit-identical to the ICL block's
    first n_ref rows (the prefix cache depends on it); with more ref tokens
    than frames the tail pairs meet CODEC_PAD."""
    rng = np.random.Generator(np.random.PCG64(3600 + n_ref))
    ref = rng.integers(0, 151936, n_ref)
    text = rng.integers(0, 151936, n_text)
    codes = rng.integers(0, 2048, (16, n_frames))
    icl, _ = ctx.build_icl_block(ref, text, codes)
    pre = ctx.build_icl_prefix(ref, codes)
    k = min(n_ref, icl.shape[0])
    assert np.array_equal(bits(pre[:k]), bits(icl[:k]))
    if n_ref > n_frames + 1:
        T = ctx.embed_text_tokens(ref)
        pad = ctx.embed_codec_token(CODEC_PAD)
        for i in range(n_frames + 1, n_ref):
            assert np.array_equal(bits(pre[i]), bits(T[i] + pad))


def test_trailing_text(ctx):
    rng = np.random.Generator(np.random.PCG64(3700))
    toks = rng.integers(0, 151936, 6)
    tr = ctx.build_trailing_text(toks)
    assert np.array_equal(bits(tr), bits(ctx.embed_text_tokens(list(toks[1:]) + [TTS_EOS])))
    assert np.array_equal(bits(ctx.build_trailing_text([])), bits(ctx.embed_text_tokens([TTS_EOS])))


@pytest.mark.parametrize("case", ["voice_icl", "voice_text", "builtin_text", "builtin_empty"])
def test_prefill_custom_voice(ctx, model, case):
    """prefill_custom_voice (generate_new.rs:361-476) on the device against
    the oracle: hidden and logits within the bar, the same start position."""
    t, p = model
    rng = np.random.Generator(np.random.PCG64(3800))
    voice = rng.standard_normal(t.hidden).astype(np.float32) if case.startswith("voice") else None
    text = [] if case == "builtin_empty" else rng.integers(0, 151936, 12)
    icl = None
    if case == "voice_icl":
        ref = rng.integers(0, 151936, 20)
        codes = rng.integers(0, 2048, (16, 30))
        icl, _ = ctx.build_icl_block(ref, text, codes)
    om = O.Model(t, p, kv_cap=128)
    try:
        hid, lg, pos = ctx.prefill_custom_voice(text, 3000, 2055, voice, icl)
        ohid, olg, opos, _ = om.prefill_custom_voice(text, 3000, 2055, voice, icl)
    finally:
        om.close()
    assert pos == opos and ctx.kv_len() == pos
    ok_h, eh = close(hid, ohid)
    ok_l, el = close(lg, olg)
    assert ok_h and ok_l, f"{case}: hidden rel err {eh}, logits {el}"
    ctx.kv_reset()


def test_prefix_cache_path_bit_identical(ctx, model):
    """The reference's prefix cache (build_talker_prefix, generate_new.rs:
    330-355, then the suffix path :537-551): head + ICL prefix prefilled and
    kept, then attached and the block's rows past the prefix prefilled, gives
    the hidden, logits and cache of prefill_custom_voice over the whole
    prompt bit for bit."""
    t, p = model
    rng = np.random.Generator(np.random.PCG64(3900))
    voice = rng.standard_normal(t.hidden).astype(np.float32)
    ref = rng.integers(0, 151936, 25)
    text = rng.integers(0, 151936, 40)
    codes = rng.integers(0, 2048, (16, 50))
    icl, rem = ctx.build_icl_block(ref, text, codes)
    hid, lg, pos = ctx.prefill_custom_voice(text, 0, 2055, voice, icl, path="mfma")
    kv_full = [ctx.kv_gather(l) for l in range(len(t.layers))]
    head = ctx.build_prefill_head(0, 2055, voice)
    pre = ctx.build_icl_prefix(ref, codes)
    assert qtts.prefix_suffix_split(icl.shape[0], len(ref), 9 + len(ref)) == icl.shape[0] - len(ref)
    ctx.kv_reset()
    ctx.prefill_talker_raw_from(np.concatenate([head, pre]), 0, path="mfma")
    pfx = ctx.prefix_capture()
    ctx.kv_reset()
    ctx.prefix_attach(pfx)
    h2 = ctx.prefill_talker_raw_from(icl[len(ref):], pfx.len, path="mfma")
    assert ctx.kv_len() == pos == 9 + icl.shape[0]
    assert np.array_equal(bits(h2), bits(hid))
    assert np.array_equal(bits(ctx.apply_codec_head(h2)), bits(lg))
    for l in range(len(t.layers)):
        k, v = ctx.kv_gather(l)
        assert np.array_equal(bits(k), bits(kv_full[l][0])) and np.array_equal(bits(v), bits(kv_full[l][1]))
    pfx.free()
    ctx.kv_reset()
