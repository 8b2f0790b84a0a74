"""Pinning the oracle's composed model functions against a float64 numpy
model written independently in matrix form (tests/f64model.py).

Reduced-width synthetic models (talker hidden 512, FFN 1024; predictor
hidden 256, FFN 512; the real head layout 16 / 8 x 128 and codec vocab 3072)
keep the float64 matrices small.  f32-vs-f64 differences here are ~1e-6 of
the output scale; the bar REL = 1e-4 leaves room for that and fails on any
structural mistake (a dropped term, a wrong sign, index or operand order),
each of which moves outputs by O(1e-2) or more — see
test_pinning_detects_planted_mistakes for such mistakes planted on the CPU.
"""
import numpy as np
import pytest

import f64model as F
import oracle as O
import qtts
from qtts import synth

REL = 1e-4


def rel_err(got, ref):
    ref = np.asarray(ref, np.float64)
    scale = max(np.abs(ref).max(), np.sqrt((ref ** 2).mean()), 1e-30)
    return np.abs(np.asarray(got, np.float64) - ref).max() / scale


@pytest.fixture(scope="module")
def models():
    t = synth.make_talker(seed=201, n_layers=2, hidden=512, inter=1024, vocab=3072, text_vocab=64,
                          text_hidden=512, rope_max_pos=4096)
    p = synth.make_predictor(seed=202, n_layers=5, hidden=256, inter=512, talker_hidden=512)
    O.set_workers(8, 8)
    om = O.Model(t, p, kv_cap=512)
    return t, p, om, F.Talker64(t), F.Predictor64(p)


def test_talker_step_and_kv_append(models):
    t, p, om, ft, fp = models
    rng = np.random.Generator(np.random.PCG64(1))
    L = 37
    K = rng.standard_normal((2, L, 8, 128)).astype(np.float32)
    V = rng.standard_normal((2, L, 8, 128)).astype(np.float32)
    om.kv_reset()
    om.kv_load(K, V)
    ft.load_kv(K, V)
    emb = rng.standard_normal(512).astype(np.float32)
    out = om.forward_with_embedding(emb, 1000)
    ref = ft.step(emb, 1000)
    assert rel_err(out[:512], ref[:512]) <= REL
    assert rel_err(out[512:], ref[512:]) <= REL
    for l in range(2):
        k, v = om.kv_layer(l)
        assert np.array_equal(k[:L], K[l]) and np.array_equal(v[:L], V[l])
        assert rel_err(k[L], ft.K[l][L]) <= REL and rel_err(v[L], ft.V[l][L]) <= REL
    om.kv_reset()


def test_prefill_from_nonzero_start(models):
    t, p, om, ft, fp = models
    rng = np.random.Generator(np.random.PCG64(2))
    X0 = rng.standard_normal((5, 512)).astype(np.float32)
    X1 = rng.standard_normal((9, 512)).astype(np.float32)
    om.kv_reset()
    ft.load_kv([[], []], [[], []])
    om.prefill(X0, 0)
    ft.prefill(X0, 0)
    h = om.prefill(X1, 5)                     # suffix prefill at start_pos 5
    r = ft.prefill(X1, 5)
    assert rel_err(h, r) <= REL
    assert om.kv_len() == 14
    for l in range(2):
        k, v = om.kv_layer(l)
        assert rel_err(k, np.stack(ft.K[l])) <= REL and rel_err(v, np.stack(ft.V[l])) <= REL
    om.kv_reset()


def test_codec_head_and_text_embedding(models):
    t, p, om, ft, fp = models
    h = np.random.Generator(np.random.PCG64(3)).standard_normal(512).astype(np.float32)
    assert rel_err(om.codec_head(h), ft.codec_head(h)) <= REL
    for tok in (0, 17, 63):
        assert rel_err(om.embed_text_token(tok), ft.embed_text(tok)) <= REL
    for tok in (0, 2150, 3071):
        assert np.array_equal(om.embed_codec_token(tok), F.row(t.codec_embedding, tok).astype(np.float32))


def _consistent_argmax(code, logits64):
    """The f32 chain's code is the float64 argmax, or within f32 noise of it."""
    top = logits64.max()
    return int(np.argmax(logits64)) == code or top - logits64[code] <= 1e-5 * np.abs(logits64).max()


def test_predictor_chain_teacher_forced(models):
    t, p, om, ft, fp = models
    rng = np.random.Generator(np.random.PCG64(4))
    for trial in range(3):
        th = rng.standard_normal(512).astype(np.float32)
        sem = F.row(t.codec_embedding, int(rng.integers(0, 2048))).astype(np.float32)
        codes = om.predictor_chain(th, sem)
        logits = fp.chain_logits(th, sem, codes)
        for g in range(15):
            assert _consistent_argmax(int(codes[g]), logits[g]), f"trial {trial} group {g}"
        # forced inputs: the chain consumes the forced codes, not its own
        forced = rng.integers(0, 2048, 15).astype(np.uint32)
        codes_f = om.predictor_chain(th, sem, forced)
        logits_f = fp.chain_logits(th, sem, forced)
        for g in range(15):
            assert _consistent_argmax(int(codes_f[g]), logits_f[g]), f"forced trial {trial} group {g}"


def test_predict_codes_legacy(models):
    """predict_codes (code_predictor.rs:126-216): four successive calls, the
    cache carried from call to call (RoPE at the cache length), all 15
    heads' logits against the float64 model; a reset starts over."""
    t, p, om, ft, fp = models
    rng = np.random.Generator(np.random.PCG64(41))
    hs = [rng.standard_normal(512).astype(np.float32) for _ in range(4)]
    om.predict_codes_reset()
    got = [om.predict_codes(h) for h in hs]
    ref = fp.predict_logits(hs)
    for i in range(4):
        for g in range(15):
            assert rel_err(got[i][g], ref[i][g]) <= REL, f"call {i} head {g}"
    # the first call's logits depend on position 0 only: after a reset, equal
    om.predict_codes_reset()
    assert np.array_equal(om.predict_codes(hs[0]), got[0])
    om.predict_codes_reset()


def test_sample_top_k_legacy_known_answers():
    """sample_top_k and apply_repetition_penalty (generate.rs:50-98): the
    answers the definitions fix."""
    # temperature <= 0: the last of equal maxima (max_by), one draw not taken
    assert O.sample_top_k([1.0, 3.0, 3.0, 2.0], 0.0, 50, [], 1.0, 7) == (2, 7)
    # top_k 1: the maximum whatever the draw; the generator advances once
    tok, rng = O.sample_top_k([0.5, 4.0, 1.0], 0.9, 1, [], 1.0, 7)
    assert tok == 1 and rng == O.simple_rand(7)[1]
    # penalty > 1 divides a positive logit, multiplies a negative one, once per
    # occurrence; penalty <= 1 is not applied (generate.rs:188-190)
    assert O.sample_top_k([2.0, 1.5], 0.0, 2, [0], 2.0, 1)[0] == 1
    assert O.sample_top_k([2.0, 1.7], 0.0, 2, [0], 1.1, 1)[0] == 0
    assert O.sample_top_k([2.0, 1.7], 0.0, 2, [0, 0], 1.1, 1)[0] == 1
    assert O.sample_top_k([-1.0, -1.5], 0.0, 2, [1], 2.0, 1)[0] == 0
    assert O.sample_top_k([-1.0, -1.5], 0.0, 2, [0], 2.0, 1)[0] == 1
    assert O.sample_top_k([2.0, 1.5], 0.0, 2, [0], 0.5, 1)[0] == 0
    with pytest.raises(RuntimeError):
        O.sample_top_k([1.0, 2.0], 1.0, 0, [], 1.0, 1)     # top_k 0: the reference indexes an empty list


def test_sample_top_k_legacy_distribution():
    """Draws follow the top-k softmax at temperature T: only the k largest
    logits are drawn, with frequencies exp((l - max) / T) normalised
    (4000 draws, 5-sigma bands)."""
    logits = np.array([2.0, 0.5, 1.2, -1.0, 1.9, 0.0], np.float32)
    T, k, n = 0.8, 3, 4000
    top = np.argsort(-logits, kind="stable")[:k]
    p = np.exp((logits[top].astype(np.float64) - logits[top].max()) / T)
    p /= p.sum()
    counts = np.zeros(len(logits))
    rng = 12345
    for _ in range(n):
        tok, rng = O.sample_top_k(logits, T, k, [], 1.0, rng)
        counts[tok] += 1
    assert counts[np.setdiff1d(np.arange(len(logits)), top)].sum() == 0
    for j, pj in zip(top, p):
        assert abs(counts[j] / n - pj) <= 5 * np.sqrt(pj * (1 - pj) / n), (j, counts[j] / n, pj)


def test_acoustic_embed_sum(models):
    t, p, om, ft, fp = models
    codes = np.random.Generator(np.random.PCG64(5)).integers(0, 2048, 15).astype(np.uint32)
    assert rel_err(om.acoustic_embed_sum(codes), fp.embed_sum(codes)) <= 1e-6


def test_frame_composition_greedy(models):
    """Two greedy frames (top-k 1): code 0 is the penalised argmax of the
    previous logits, codes 1..15 follow the predictor chain, and the next
    hidden/logits are the talker step on semantic + sum of code embeddings +
    text row at the next position."""
    t, p, om, ft, fp = models
    rng = np.random.Generator(np.random.PCG64(6))
    X = rng.standard_normal((6, 512)).astype(np.float32)
    om.kv_reset()
    ft.load_kv([[], []], [[], []])
    hid = om.prefill(X, 0)
    ft.prefill(X, 0)
    logits = om.codec_head(hid)
    text = rng.standard_normal(512).astype(np.float32)
    params = qtts.sample_params(top_k=1, eos_enabled=False)
    om.gen_begin(logits, hid, 6, 42)
    prev = np.zeros(16, np.uint32)
    for f in range(2):
        lg_before = om.g_logits.astype(np.float64).copy()
        hid_before = om.g_hidden.copy()
        codes, eos = om.frame(params, text)
        assert not eos
        pen = lg_before.copy()
        for c in prev:                                  # penalty once per history entry
            pen[c] = pen[c] / 1.05 if pen[c] > 0 else pen[c] * 1.05
        assert codes[0] == int(np.argmax(pen))          # lowest index on ties, as argmax
        sem = F.row(t.codec_embedding, int(codes[0]))
        chain = fp.chain_logits(hid_before, sem.astype(np.float32), codes[1:])
        for g in range(15):
            assert _consistent_argmax(int(codes[g + 1]), chain[g])
        comb = sem + fp.embed_sum(codes[1:]) + text.astype(np.float64)
        ref = ft.step(comb, 6 + f)
        assert rel_err(om.g_hidden, ref[:512]) <= REL
        assert rel_err(om.g_logits, ref[512:]) <= REL
        prev = codes.copy()
    om.kv_reset()


def test_pinning_detects_planted_mistakes(models):
    """The bar separates f32 rounding from structural mistakes: each planted
    mistake (applied to the float64 model on the CPU) moves the talker step
    by far more than REL."""
    t, p, om, ft, fp = models
    rng = np.random.Generator(np.random.PCG64(7))
    L = 20
    K = rng.standard_normal((2, L, 8, 128)).astype(np.float32)
    V = rng.standard_normal((2, L, 8, 128)).astype(np.float32)
    emb = rng.standard_normal(512).astype(np.float32)
    om.kv_reset()
    om.kv_load(K, V)
    out = om.forward_with_embedding(emb, 300)
    om.kv_reset()

    def run(**patch):
        saved = {k: getattr(F, k) for k in patch}
        for k, v in patch.items():
            setattr(F, k, v)
        try:
            m = F.Talker64(t)
            m.load_kv(K, V)
            return m.step(emb, 300)
        finally:
            for k, v in saved.items():
                setattr(F, k, v)

    base = run()
    assert rel_err(out, base) <= REL
    good_rope = F.rope
    mistakes = {
        "rope sign": dict(rope=lambda x, pos, theta=1e6: good_rope(x, -pos, theta)),
        "rope pairs (2i, 2i+1)": dict(rope=lambda x, pos, theta=1e6: good_rope(
            x.reshape(*x.shape[:-1], 64, 2).swapaxes(-1, -2).reshape(x.shape), pos, theta)
            .reshape(*x.shape[:-1], 2, 64).swapaxes(-1, -2).reshape(x.shape)),
        "GQA h % n_kv": dict(kv_head_map=lambda nh, nkv: np.arange(nh) % nkv),
        "no gamma": dict(rms=lambda x, g: x / np.sqrt(np.mean(x * x, -1, keepdims=True) + 1e-6)),
        "silu -> sigmoid": dict(silu=lambda x: 1.0 / (1.0 + np.exp(-x))),
    }
    for name, patch in mistakes.items():
        e = rel_err(out, run(**patch))
        assert e > 100 * REL, f"{name}: only {e:.2e}"
