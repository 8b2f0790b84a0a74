"""The frame loop's stops and errors (generate_new.rs:583-675).  EOS ends
generation before the EOS frame is emitted: the reference breaks before
pushing it (generate_new.rs:617-621).  A full KV cache, NaN logits and calls
out of order return their statuses and leave the context usable."""
import numpy as np
import pytest

import oracle as O
import qtts
from qtts import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model():
    t = synth.make_talker(seed=701, n_layers=2, text_vocab=256, rope_max_pos=1024)
    p = synth.make_predictor(seed=702, n_layers=5, rope_max_pos=64)
    return t, p


def begin(ctx, t, n, params, edit_logits=None, seed=42):
    X = np.random.Generator(np.random.PCG64(71)).standard_normal((n, t.hidden)).astype(np.float32)
    ctx.kv_reset()
    hid = ctx.prefill_talker_raw_from(X, 0)
    lg = ctx.apply_codec_head(hid)
    if edit_logits is not None:
        lg = edit_logits(lg.copy())
    ctx.gen_set_text(None, ctx.embed_text_token(3))
    ctx.gen_begin(lg, hid, n, seed, params)
    return X, hid, lg


def test_eos_on_the_first_frame(ctx_factory, model):
    t, p = model
    c = ctx_factory(256)
    c.upload_model(t, p)

    def eos_wins(lg):
        lg[2150] = 1e4
        return lg
    params = qtts.sample_params(eos_enabled=True)
    X, hid, lg = begin(c, t, 16, params, eos_wins)
    codes, eos = c.gen_frames(10)
    assert eos and codes.shape[0] == 0 and c.kv_len() == 16
    codes, eos = c.gen_frames(10)                  # stays stopped
    assert eos and codes.shape[0] == 0
    om = O.Model(t, p, kv_cap=256)
    om.prefill(X, 0)
    om.gen_begin(lg, hid, 16, 42)
    _, oeos = om.frame(params, c.embed_text_token(3))
    om.close()
    assert oeos


def test_eos_mid_run_stops_before_the_frame(ctx_factory, model):
    """Frames sampled without EOS, then the same run with the EOS id set to
    the first code 0 that frame k introduces: exactly frames 0..k-1 come
    back, identical, and the flag is set."""
    t, p = model
    c = ctx_factory(256)
    c.upload_model(t, p)
    begin(c, t, 16, qtts.sample_params(eos_enabled=False))
    free, eos = c.gen_frames(24)
    assert not eos and free.shape[0] == 24
    first = {}
    for f, code in enumerate(free[:, 0]):
        first.setdefault(int(code), f)
    k, x = max((f, code) for code, f in first.items() if f > 0)
    begin(c, t, 16, qtts.sample_params(eos_enabled=True, codec_eos_id=x))
    got, eos = c.gen_frames(24)
    assert eos and got.shape[0] == k
    assert np.array_equal(got, free[:k])
    assert c.kv_len() == 16 + k


def test_kv_capacity(ctx_factory, model):
    """A batch that would overflow the cache is refused before it runs; the
    frames that fit still run afterwards; the next one is refused."""
    t, p = model
    c = ctx_factory(128)
    c.upload_model(t, p)
    begin(c, t, 100, qtts.sample_params(eos_enabled=False))
    with pytest.raises(qtts.QttsError) as e:
        c.gen_frames(64)
    assert e.value.code == qtts.ERR_CAPACITY
    assert c.kv_len() == 100
    codes, eos = c.gen_frames(28)
    assert codes.shape[0] == 28 and not eos and c.kv_len() == 128
    with pytest.raises(qtts.QttsError) as e:
        c.gen_frames(1)
    assert e.value.code == qtts.ERR_CAPACITY


def test_nan_logits_and_order(ctx_factory, model):
    t, p = model
    c = ctx_factory(256)
    c.upload_model(t, p)
    with pytest.raises(qtts.QttsError) as e:
        c.gen_frames(4)                            # before gen_begin
    assert e.value.code == qtts.ERR_STATE

    def poison(lg):
        lg[7] = np.nan
        return lg
    begin(c, t, 16, qtts.sample_params(eos_enabled=False), poison)
    with pytest.raises(qtts.QttsError) as e:
        c.gen_frames(4)
    assert e.value.code == qtts.ERR_NAN
    # a fresh start on the same context works
    begin(c, t, 16, qtts.sample_params(eos_enabled=False))
    codes, eos = c.gen_frames(3)
    assert codes.shape[0] == 3 and not eos
    assert c.gen_frames(0)[0].shape[0] == 0


def test_frame_half_timing_between_frames(ctx_factory, model):
    """qtts_time_kernel kinds 5 and 6 (each half of the frame replayed alone)
    called in the middle of a generation leave it as it was: the frames that
    follow are the ones an undisturbed run produces."""
    t, p = model
    c = ctx_factory(256)
    c.upload_model(t, p)
    params = qtts.sample_params(eos_enabled=False)
    begin(c, t, 16, params)
    ref, _ = c.gen_frames(8)
    begin(c, t, 16, params)
    a, _ = c.gen_frames(4)
    c.time_kernel(5, 3)
    c.time_kernel(6, 3)
    b, _ = c.gen_frames(4)
    assert np.array_equal(np.concatenate([a, b]), ref)
    assert c.kv_len() == 16 + 8


def test_wait_give_up_reported_then_recovers(ctx_factory, model):
    """The give-up path of the fused launches' bounded waits, forced from the
    host (qtts_debug_force_sync_err: the next call starts with the flag a
    wait sets when it runs out, so every workgroup skips its polls and each
    kernel exits normally).  The talker step, a frame batch, the predictor
    chain and the legacy predictor step each return QTTS_ERR_HIP, and the
    same call repeated is correct: against the oracle, or bit-identical to
    an undisturbed run."""
    t, p = model
    c = ctx_factory(256)
    c.upload_model(t, p)
    om = O.Model(t, p, kv_cap=256)
    rng = np.random.Generator(np.random.PCG64(7100))
    K = rng.standard_normal((len(t.layers), 40, 8, 128)).astype(np.float32)
    V = rng.standard_normal((len(t.layers), 40, 8, 128)).astype(np.float32)
    c.kv_load(K, V)
    om.kv_load(K, V)
    emb = rng.standard_normal(t.hidden).astype(np.float32)
    c.debug_force_sync_err()
    with pytest.raises(qtts.QttsError) as e:
        c.forward_with_embedding(emb, 40)
    assert e.value.code == qtts.ERR_HIP
    assert c.kv_len() == 40
    got, ref = c.forward_with_embedding(emb, 40), om.forward_with_embedding(emb, 40)
    scale = max(np.abs(ref).max(), 1e-30)
    assert np.abs(got.astype(np.float64) - ref).max() <= 1e-3 * scale
    assert c.kv_len() == 41
    om.close()

    th = rng.standard_normal(t.hidden).astype(np.float32)
    sem = c.embed_codec_token(77)
    codes = c.generate_acoustic_codes(th, sem)
    c.debug_force_sync_err()
    with pytest.raises(qtts.QttsError) as e:
        c.generate_acoustic_codes(th, sem)
    assert e.value.code == qtts.ERR_HIP
    assert np.array_equal(c.generate_acoustic_codes(th, sem), codes)

    c.predict_codes_reset()
    lg = c.predict_codes(th)
    c.predict_codes_reset()
    c.debug_force_sync_err()
    with pytest.raises(qtts.QttsError) as e:
        c.predict_codes(th)
    assert e.value.code == qtts.ERR_HIP
    assert np.array_equal(c.predict_codes(th).view(np.uint32), lg.view(np.uint32))

    params = qtts.sample_params(eos_enabled=False)
    begin(c, t, 16, params)
    ref_frames, _ = c.gen_frames(6)
    begin(c, t, 16, params)
    c.debug_force_sync_err()
    with pytest.raises(qtts.QttsError) as e:
        c.gen_frames(6)
    assert e.value.code == qtts.ERR_HIP
    begin(c, t, 16, params)                        # truncate and begin again
    assert c.kv_len() == 16
    got, _ = c.gen_frames(6)
    assert np.array_equal(got, ref_frames)


def test_codec_vocab_not_whole_groups_refused(ctx_factory):
    """A codec vocabulary that does not fill whole 32-column groups is refused
    at upload with QTTS_ERR_UNSUPPORTED: the step end, the sampler and the
    predictor's argmax read whole groups of the heads' partial sums, and the
    12 Hz model's vocabularies (3072, 2048) are whole groups.  The context
    takes a supported model afterwards."""
    c = ctx_factory(64)
    p = synth.make_predictor(seed=704, n_layers=1, rope_max_pos=64)
    t = synth.make_talker(seed=703, n_layers=1, vocab=3000, text_vocab=256, rope_max_pos=128)
    with pytest.raises(qtts.QttsError) as e:
        c.upload_model(t, p)
    assert e.value.code == qtts.ERR_UNSUPPORTED
    t = synth.make_talker(seed=703, n_layers=1, text_vocab=256, rope_max_pos=128)
    p2 = synth.make_predictor(seed=704, n_layers=1, vocab=2000, rope_max_pos=64)
    with pytest.raises(qtts.QttsError) as e:
        c.upload_model(t, p2)
    assert e.value.code == qtts.ERR_UNSUPPORTED
    c.upload_model(t, p)
    X = np.random.Generator(np.random.PCG64(705)).standard_normal((4, t.hidden)).astype(np.float32)
    lg = c.apply_codec_head(c.prefill_talker_raw_from(X, 0))
    assert lg.shape == (3072,) and np.isfinite(lg).all()
