"""The talker step at long context against the oracle (talker.rs:263-360,
attention talker.rs:304-331): a 2-layer talker at the 1.7B layer shapes, the
KV cache loaded with N(0,1) rows to L positions, one step appending at L and
attending over L + 1.

The lengths straddle every boundary of the device's page merge: 16 pages
(the pages fetched ahead of the o-proj's weights), 17 (the first 24-page
block after them), 33-34 (BASELINE's KV 2048 and the frame loop's last KV
2112), 64-65 (the second lane of pages in the merge) and 128 (the largest
cache, 8192 positions).

Bars: hidden, logits and the appended K/V row within 1e-3 of the scale
(f32 accumulation in another order); the L loaded rows bit-exact.
"""
import numpy as np
import pytest

import oracle as O
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


@pytest.fixture(scope="module")
def long_model(ctx_factory):
    t = synth.make_talker(seed=131, n_layers=2, text_vocab=256, rope_max_pos=CAP)
    p = synth.make_predictor(seed=132, n_layers=2)
    c = ctx_factory(CAP)
    c.upload_model(t, p)
    O.set_workers(16, 8)
    om = O.Model(t, p, kv_cap=CAP)
    yield c, om, t
    om.close()


@pytest.mark.parametrize("L", [1023, 1024, 1100, 2047, 2048, 2111, 4095, 4096, 4160, 8191])
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
