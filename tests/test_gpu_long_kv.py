"""The talker step at long context against the oracle (talker.rs:263-360,
attention talker.rs:304-331): a 2-layer talker at the 1.7B layer shapes, the
KV cache loaded with N(0,1) rows to L positions, one step appending at L and
attending over L + 1.

The lengths straddle every boundary of the device's attention and page
merge: KV 1024, where the attention switches from one page (64 positions) per
work item to two (128-position chunks); 20 chunks (the chunks fetched ahead of
the o-proj's weights, KV 2560) and 21 (the first 22-chunk block after them);
42-43 (the second block, KV 5376); KV 2048 and 2112 (the headline KV and the
frame loop's last); 8192 positions (the largest cache).  A frame loop crosses
the KV-1024 switch inside one batch of frames.

By default the q|k|v GEMV and the attention run as one launch, two pages
per work item at every length; a q|k|v tile other than the fused kernel's
(QTTS_TILE_TQKV) keeps them apart, with one page per work item below
KV 1024.  Both paths are checked.

Bars: hidden, logits and the appended K/V row within 1e-3 of the scale
(f32 accumulation in another order); the L loaded rows bit-exact.
"""
import numpy as np
import pytest

import oracle as O
import qtts
from qtts import synth

pytestmark = pytest.mark.gpu

TOL = 1e-3
CAP = 8192


def close(got, ref, rel=TOL):
    ref = np.asarray(ref, np.float64)
    scale = max(np.abs(ref).max(), np.sqrt((ref ** 2).mean()), 1e-30)
    err = np.abs(np.asarray(got, np.float64) - ref).max()
    return err <= rel * scale, err / scale


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# q|k|v tiles: the fused launch's (the default) and one the unfused kernels take
FUSED, UNFUSED = "15", "13"


@pytest.fixture(scope="module", params=[FUSED, UNFUSED], ids=["fused", "unfused"])
def long_model(ctx_factory, request):
    t = synth.make_talker(seed=131, n_layers=2, text_vocab=256, rope_max_pos=CAP)
    p = synth.make_predictor(seed=132, n_layers=2)
    c = ctx_factory(CAP)
    with pytest.MonkeyPatch.context() as mp:
        mp.setenv("QTTS_TILE_TQKV", request.param)
        c.upload_model(t, p)
    O.set_workers(16, 8)
    om = O.Model(t, p, kv_cap=CAP)
    yield c, om, t
    om.close()


@pytest.mark.parametrize("L", [1022, 1023, 1024, 1100, 2047, 2048, 2111, 2559, 2560, 2561, 4096, 5375, 5376, 8191])
def test_talker_step_long_kv(long_model, L):
    c, om, t = long_model
    print(f"talker step at KV {L} -> {L + 1}", flush=True)
    rng = np.random.Generator(np.random.PCG64(1300 + L))
    n = len(t.layers)
    K = rng.standard_normal((n, L, 8, 128), dtype=np.float32)
    V = rng.standard_normal((n, L, 8, 128), dtype=np.float32)
    c.kv_load(K, V)
    om.kv_load(K, V)
    emb = rng.standard_normal(t.hidden).astype(np.float32)
    out = c.forward_with_embedding(emb, L)
    ref = om.forward_with_embedding(emb, L)
    ok_h, eh = close(out[: t.hidden], ref[: t.hidden])
    ok_l, el = close(out[t.hidden:], ref[t.hidden:])
    assert ok_h and ok_l, f"KV {L}: hidden rel err {eh}, logits {el}"
    assert c.kv_len() == L + 1
    for l in range(n):
        k, v = c.kv_gather(l)
        ko, vo = om.kv_layer(l)
        assert np.array_equal(bits(k[:L]), bits(K[l])) and np.array_equal(bits(v[:L]), bits(V[l]))
        ok_k, ek = close(k[L], ko[L])
        ok_v, ev = close(v[L], vo[L])
        assert ok_k and ok_v, f"KV {L} layer {l}: new K rel err {ek}, V {ev}"
    c.kv_reset()
    om.kv_reset()


def test_steps_across_page_boundary(long_model):
    """Four steps from KV 2046 (pages 32 -> 33, the 33rd page starting at
    the step that writes position 2048), each against the oracle."""
    c, om, t = long_model
    rng = np.random.Generator(np.random.PCG64(1399))
    n, L = len(t.layers), 2046
    K = rng.standard_normal((n, L, 8, 128), dtype=np.float32)
    V = rng.standard_normal((n, L, 8, 128), dtype=np.float32)
    c.kv_load(K, V)
    om.kv_load(K, V)
    for step in range(4):
        emb = rng.standard_normal(t.hidden).astype(np.float32)
        ok, e = close(c.forward_with_embedding(emb, L + step), om.forward_with_embedding(emb, L + step))
        assert ok, f"step at KV {L + step}: rel err {e}"
    c.kv_reset()
    om.kv_reset()


def test_frames_across_attention_switch(long_model):
    """Sampled frames teacher-forced from KV 1018 to 1030 in one batch: when
    the launches are apart, the frames before KV 1024 replay the one-page
    attention graph and those after the two-page one (fused, every frame
    replays the two-page graph); codes, generator state and the final
    hidden/logits against the oracle's frame loop (generate_new.rs:606-675)."""
    c, om, t = long_model
    L, n_frames = 1018, 12
    rng = np.random.Generator(np.random.PCG64(1401))
    n = len(t.layers)
    K = rng.standard_normal((n, L, 8, 128), dtype=np.float32)
    V = rng.standard_normal((n, L, 8, 128), dtype=np.float32)
    c.kv_load(K, V)
    om.kv_load(K, V)
    hid = rng.standard_normal(t.hidden).astype(np.float32)
    logits = om.codec_head(hid)
    pad = om.embed_text_token(3)
    params = qtts.sample_params(eos_enabled=False)
    c.gen_set_text(None, pad)
    om.gen_begin(logits, hid, L, 42)
    c.gen_begin(logits, hid, L, 42, params)
    ref = np.stack([om.frame(params, pad)[0] for _ in range(n_frames)])
    pred = c.gen_frames_forced(ref)
    assert np.array_equal(pred[:, 0], ref[:, 0]), f"sampled codes {pred[:, 0]} vs {ref[:, 0]}"
    assert (pred[:, 1:] == ref[:, 1:]).mean() >= 0.99
    lg, hd, pos, rng_state = c.gen_state()
    assert pos == L + n_frames and c.kv_len() == L + n_frames
    assert rng_state == om.gen.rng
    ok_h, eh = close(hd, om.g_hidden)
    ok_l, el = close(lg, om.g_logits)
    assert ok_h and ok_l, f"after {n_frames} frames: hidden rel err {eh}, logits {el}"
    for l in range(n):
        k, v = c.kv_gather(l)
        ko, vo = om.kv_layer(l)
        ok_k, ek = close(k[L:L + n_frames], ko[L:L + n_frames])
        ok_v, ev = close(v[L:L + n_frames], vo[L:L + n_frames])
        assert ok_k and ok_v, f"layer {l}: appended K rel err {ek}, V {ev}"
    c.kv_reset()
    om.kv_reset()
