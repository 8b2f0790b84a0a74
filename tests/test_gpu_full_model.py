"""The 1.7B shapes end to end against the oracle: a 28-layer talker and the
5-layer predictor (random Q4 weights; the text vocabulary cut to 256 rows,
which the frame loop does not read), a 16-row prompt, then 200 greedy frames
fed the oracle's codes (teacher forcing).  Bars: prefill hidden and codec
logits within 1e-3 of the scale; >= 99% of the 16 x 200 codes equal."""
import numpy as np
import pytest

import oracle as O
import qtts
from qtts import synth

pytestmark = pytest.mark.gpu

FRAMES = 200


def close(got, ref, rel=1e-3):
    ref = np.asarray(ref, np.float64)
    scale = max(np.abs(ref).max(), np.sqrt((ref ** 2).mean()))
    err = np.abs(np.asarray(got, np.float64) - ref).max()
    return err <= rel * scale, err / scale


@pytest.fixture(scope="module")
def full(ctx_factory):
    t = synth.make_talker(seed=801, text_vocab=256, rope_max_pos=4096)
    p = synth.make_predictor(seed=802, rope_max_pos=64)
    assert len(t.layers) == 28 and t.hidden == 2048 and len(p.layers) == 5 and p.hidden == 1024
    c = ctx_factory(4096)
    c.upload_model(t, p)
    O.set_workers(16, 8)
    om = O.Model(t, p, kv_cap=4096)
    yield c, om, t, p
    om.close()


def test_full_model_prefill_and_frames(full):
    c, om, t, p = full
    X = np.random.Generator(np.random.PCG64(81)).standard_normal((16, t.hidden)).astype(np.float32)
    c.kv_reset()
    om.kv_reset()
    hid = c.prefill_talker_raw_from(X, 0)
    ohid = om.prefill(X, 0)
    ok, e = close(hid, ohid)
    assert ok, f"prefill hidden rel err {e}"
    logits = om.codec_head(ohid)
    ok, e = close(c.apply_codec_head(ohid), logits)
    assert ok, f"codec head rel err {e}"
    pad = om.embed_text_token(3)
    params = qtts.sample_params(top_k=1, eos_enabled=False)
    c.gen_set_text(None, pad)
    om.gen_begin(logits, ohid, 16, 42)
    c.gen_begin(logits, ohid, 16, 42, params)
    ref = np.stack([om.frame(params, pad)[0] for _ in range(FRAMES)])
    pred = c.gen_frames_forced(ref)
    agree = (pred == ref).mean()
    assert agree >= 0.99, f"agreement {agree:.4f}"
    assert c.kv_len() == 16 + FRAMES


def test_full_model_sampled_frames_kv2048(full):
    c, om, t, p = full
    L, n_frames = 2048, 16
    print(f"28-layer frames from KV {L}", flush=True)
    rng = np.random.Generator(np.random.PCG64(82))
    n = len(t.layers)
    K = rng.standard_normal((n, L, 8, 128), dtype=np.float32)
    V = rng.standard_normal((n, L, 8, 128), dtype=np.float32)
    c.kv_load(K, V)
    om.kv_load(K, V)
    del K, V
    hid = rng.standard_normal(t.hidden).astype(np.float32)
    logits = om.codec_head(hid)
    pad = om.embed_text_token(3)
    params = qtts.sample_params(eos_enabled=False)    # top-k 50, T 0.9, penalty 1.05
    c.gen_set_text(None, pad)
    om.gen_begin(logits, hid, L, 42)
    c.gen_begin(logits, hid, L, 42, params)
    ref = np.stack([om.frame(params, pad)[0] for _ in range(n_frames)])
    pred = c.gen_frames_forced(ref)
    assert np.array_equal(pred[:, 0], ref[:, 0]), f"sampled codes {pred[:, 0]} vs {ref[:, 0]}"
    agree = (pred[:, 1:] == ref[:, 1:]).mean()
    assert agree >= 0.99, f"predictor codes agree {agree:.4f}"
    lg, hd, pos, rng_state = c.gen_state()
    assert pos == L + n_frames and c.kv_len() == L + n_frames
    assert rng_state == om.gen.rng
    ok_h, eh = close(hd, om.g_hidden)
    ok_l, el = close(lg, om.g_logits)
    assert ok_h and ok_l, f"after {n_frames} frames: hidden rel err {eh}, logits {el}"
    c.kv_reset()
    om.kv_reset()
