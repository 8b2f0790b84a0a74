"""The legacy generation loop's pieces (generate.rs:107-250) on the device,
against the oracle: prefill_talker over (id, is_text) tokens
(talker.rs:487-508), predict_codes with its cache kept across calls
(code_predictor.rs:126-216), the legacy sampler (generate.rs:50-98), and a
short teacher-forced loop composed from them.  Bars as in the other parity
tests: hidden and logits within 1e-3 of the scale, sampled tokens <= 1
mismatch in 60 draws (expf bits), greedy codes >= 99%."""
import numpy as np
import pytest

import oracle as O
import qtts
from qtts import synth

pytestmark = pytest.mark.gpu

TOL = 1e-3


def close(got, ref, rel=TOL):
    ref = np.asarray(ref, np.float64)
    scale = max(np.abs(ref).max(), np.sqrt((ref ** 2).mean()), 1e-30)
    err = np.abs(np.asarray(got, np.float64) - ref).max()
    return err <= rel * scale, err / scale


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def model():
    t = synth.make_talker(seed=601, n_layers=2, text_vocab=512, rope_max_pos=1024)
    p = synth.make_predictor(seed=602, n_layers=5, rope_max_pos=1024)
    return t, p


@pytest.fixture(scope="module")
def ctx(ctx_factory, model):
    c = ctx_factory(512)
    c.upload_model(*model)
    return c


@pytest.fixture(scope="module")
def om(model):
    O.set_workers(16, 8)
    m = O.Model(*model, kv_cap=512)
    yield m
    m.close()


@pytest.mark.parametrize("temp,top_k,penalty", [(0.9, 50, 1.05), (0.7, 5, 1.3), (1.0, 3072, 1.0), (0.0, 50, 1.2)])
def test_sample_top_k_matches_oracle(ctx, temp, top_k, penalty):
    rng = np.random.Generator(np.random.PCG64(61))
    s_gpu = s_cpu = 1234
    mismatch = 0
    for i in range(60):
        lg = (rng.standard_normal(3072) * 3).astype(np.float32)
        prev = rng.integers(0, 3072, 40 + i).astype(np.uint32)
        a, s_gpu = ctx.sample_top_k(lg, temp, top_k, prev, penalty, s_gpu)
        b, s_cpu = O.sample_top_k(lg, temp, top_k, prev, penalty, s_cpu)
        assert s_gpu == s_cpu
        mismatch += a != b
    assert mismatch <= (0 if temp <= 0 else 1)


def test_sample_top_k_edges(ctx):
    assert ctx.sample_top_k([1.0, 3.0, 3.0, 2.0], 0.0, 50, [], 1.0, 7) == (2, 7)
    assert ctx.sample_top_k([2.0, 1.7], 0.0, 2, [0, 0], 1.1, 1)[0] == 1
    assert ctx.sample_top_k([-1.0, -1.5], 0.0, 2, [0], 2.0, 1)[0] == 1
    tok, rng = ctx.sample_top_k([0.5, 4.0, 1.0], 0.9, 1, [], 1.0, 7)
    assert tok == 1 and rng == O.simple_rand(7)[1]
    with pytest.raises(qtts.QttsError) as e:
        ctx.sample_top_k([1.0, 2.0], 1.0, 0, [], 1.0, 1)
    assert e.value.code == qtts.ERR_INVALID
    with pytest.raises(qtts.QttsError) as e:
        ctx.sample_top_k([1.0, float("nan")], 1.0, 2, [], 1.0, 1)
    assert e.value.code == qtts.ERR_NAN


def test_prefill_tokens(ctx, model, om):
    """Mixed text / codec tokens (the legacy prompt: 3 text, 7 codec, then
    text); against the oracle's embeddings + prefill, and bit-identical to
    the device's own embed + prefill_talker_raw_from."""
    t, p = model
    rng = np.random.Generator(np.random.PCG64(62))
    n = 22
    is_text = np.array([1] * 3 + [0] * 7 + [1] * (n - 10), np.uint8)
    ids = np.where(is_text == 1, rng.integers(0, 512, n), rng.integers(0, 3072, n)).astype(np.uint32)
    hid = ctx.prefill_tokens(ids, is_text)
    assert ctx.kv_len() == n
    X = np.stack([om.embed_text_token(int(i)) if tt else om.embed_codec_token(int(i)) for i, tt in zip(ids, is_text)])
    om.kv_reset()
    ok, e = close(hid, om.prefill(X, 0))
    assert ok, f"rel err {e}"
    om.kv_reset()
    rows = np.stack([ctx.embed_text_tokens([int(i)])[0] if tt else ctx.embed_codec_token(int(i))
                     for i, tt in zip(ids, is_text)])
    ctx.kv_reset()
    assert np.array_equal(bits(ctx.prefill_talker_raw_from(rows, 0)), bits(hid))
    ctx.kv_reset()


def test_predict_codes_matches_oracle(ctx, model, om):
    """Eight calls with the cache growing 1 -> 8, all 15 heads; a reset
    starts over with the first call's bits."""
    t, p = model
    rng = np.random.Generator(np.random.PCG64(63))
    hs = [rng.standard_normal(t.hidden).astype(np.float32) for _ in range(8)]
    ctx.predict_codes_reset()
    om.predict_codes_reset()
    first = None
    for i, h in enumerate(hs):
        got, ref = ctx.predict_codes(h), om.predict_codes(h)
        if i == 0:
            first = got.copy()
        for g in range(len(p.lm_heads)):
            ok, e = close(got[g], ref[g])
            assert ok, f"call {i} head {g}: rel err {e}"
    ctx.predict_codes_reset()
    assert np.array_equal(bits(ctx.predict_codes(hs[0])), bits(first))
    ctx.predict_codes_reset()
    om.predict_codes_reset()


def test_legacy_loop_teacher_forced(ctx, model, om):
    """generate.rs:185-235 greedy: codec head -> code 0, predict_codes ->
    codes 1..15 (argmax of each head), forward_talker_decode(code 0); the
    oracle's code 0 fed to both sides each step; >= 99% of codes agree."""
    t, p = model
    rng = np.random.Generator(np.random.PCG64(64))
    is_text = np.array([1] * 3 + [0] * 7 + [1] * 6, np.uint8)
    ids = np.where(is_text == 1, rng.integers(0, 512, 16), rng.integers(0, 3072, 16)).astype(np.uint32)
    hid = ctx.prefill_tokens(ids, is_text)
    X = np.stack([om.embed_text_token(int(i)) if tt else om.embed_codec_token(int(i)) for i, tt in zip(ids, is_text)])
    om.kv_reset()
    ohid = om.prefill(X, 0)
    ctx.predict_codes_reset()
    om.predict_codes_reset()
    agree = total = 0
    pos = 16
    for step in range(12):
        c0_ref, _ = O.sample_top_k(om.codec_head(ohid), 0.0, 50, [], 1.0, 1)
        c0_got, _ = ctx.sample_top_k(ctx.apply_codec_head(hid), 0.0, 50, [], 1.0, 1)
        ref = [c0_ref] + [O.argmax_last(l) for l in om.predict_codes(ohid)]
        got = [c0_got] + [O.argmax_last(l) for l in ctx.predict_codes(hid)]
        agree += sum(int(a == b) for a, b in zip(got, ref))
        total += len(ref)
        ohid = om.forward_with_embedding(om.embed_codec_token(c0_ref), pos)[: t.hidden]
        hid = ctx.forward_talker_decode(c0_ref, False, pos)
        pos += 1
    assert agree >= 0.99 * total, f"{agree}/{total}"
    ctx.kv_reset()
    om.kv_reset()
