"""The HIP path against the committed golden fixtures (tests/golden/, the
oracle's outputs on seeded inputs; inputs regenerated here from the seeds in
manifest.json and checked against their recorded digests).  Bars as in the
other parity tests: GEMV, step and decoder outputs within 1e-3 of the
reference's scale; codes exact on the first predictor input and >= 99%
overall; greedy frames >= 99% teacher-forced."""
import json
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_golden as G  # noqa: E402
import qtts  # noqa: E402
from qtts import synth  # noqa: E402

pytestmark = pytest.mark.gpu

MANIFEST = json.load(open(os.path.join(HERE, "golden", "manifest.json")))
TOL = 1e-3


def fixture(name):
    return np.load(os.path.join(HERE, "golden", name + ".npz"))


def close(got, ref, rel=TOL):
    ref = np.asarray(ref, np.float64)
    scale = max(np.abs(ref).max(), np.sqrt((ref ** 2).mean()), 1e-30)
    err = np.abs(np.asarray(got, np.float64) - ref).max()
    return err <= rel * scale, err / scale


@pytest.fixture(scope="module")
def loaded(ctx_factory):
    t, p = G.models()
    assert G.digest((t, p)) == MANIFEST["fixtures"]["talker_step"]["model"], "synthetic model generator drifted"
    c = ctx_factory(1024)
    c.upload_model(t, p)
    return c, t


def test_gemv_golden(ctx_factory):
    c = ctx_factory(64)
    w, x, cases = G.gemv_inputs()
    f = fixture("gemv")
    assert G.digest((w, x)) == MANIFEST["fixtures"]["gemv"]["inputs"]["gemv_2048x6144"]
    dw = c.upload(w)
    ok, e = close(c.gemv(dw, x), f["gemv_2048x6144_y"])
    dw.free()
    assert ok, f"config 1: rel err {e}"
    for name, (cx, cw) in cases.items():
        dw = c.upload(cw)
        ok, e = close(c.gemv(dw, cx), f[name + "_y"])
        dw.free()
        assert ok, f"{name}: rel err {e}"


def test_talker_step_golden(loaded):
    c, t = loaded
    K, V, emb = G.talker_step_inputs(t)
    f = fixture("talker_step")
    c.kv_reset()
    c.kv_load(K, V)
    out = c.forward_with_embedding(emb, 512)
    k, v = c.kv_gather(0)
    c.kv_reset()
    for name, got in (("hidden", out[: t.hidden]), ("logits", out[t.hidden:]), ("k_new", k[512]), ("v_new", v[512])):
        ok, e = close(got, f[name])
        assert ok, f"{name}: rel err {e}"


def test_predictor_golden(loaded):
    c, t = loaded
    ref = fixture("predictor")["codes"]
    got = np.stack([c.generate_acoustic_codes(th, c.embed_codec_token(sem)) for th, sem in G.predictor_inputs(t)])
    assert np.array_equal(got[0], ref[0]), f"{got[0]} vs {ref[0]}"
    assert (got == ref).mean() >= 0.99


def test_greedy_frames_golden(loaded):
    """200 greedy frames, each fed the recorded codes of the frame before."""
    c, t = loaded
    ref = fixture("greedy_frames")["codes"]
    X = G.greedy_prompt(t)
    c.kv_reset()
    hid = c.prefill_talker_raw_from(X, 0)
    logits = c.apply_codec_head(hid)
    c.gen_set_text(None, c.embed_text_token(3))
    c.gen_begin(logits, hid, 16, 42, qtts.sample_params(top_k=1, eos_enabled=False))
    pred = c.gen_frames_forced(ref)
    c.kv_reset()
    agree = (pred == ref).mean()
    assert agree >= 0.99, f"agreement {agree:.4f}"


def test_decoder_golden(ctx_factory):
    d = synth.make_decoder(**G.DECODER)
    assert G.digest(d) == MANIFEST["fixtures"]["decoder"]["model"]
    codes, warm = G.decoder_inputs(d)
    c = ctx_factory(64)
    c.upload_decoder(d)
    ok, e = close(c.decode_to_audio(codes, warm), fixture("decoder")["audio"])
    assert ok, f"rel err {e}"


def test_icl28_golden(ctx_factory):
    """The ICL workload at full depth against the oracle's fixture: the
    voice-clone prompt built on the device (build_icl_block, the prompt head,
    prefill_custom_voice on the matrix cores through all 28 layers), the
    last hidden and logits and cached K/V rows of layers 0, 13 and 27, then
    32 greedy frames fed the block's remainder rows as trailing text and
    teacher-forced on the fixture's codes (talker.rs:379-482,
    generate_new.rs:552-654)."""
    m = MANIFEST["fixtures"]["icl28"]
    t, p = G.icl28_models()
    assert G.digest((t, p)) == m["model"], "synthetic model generator drifted"
    ref_tok, text, codes, voice = G.icl28_inputs()
    assert G.digest((ref_tok, text, codes, voice)) == m["inputs"]
    f = fixture("icl28")
    c = ctx_factory(1024)
    c.upload_model(t, p)
    del t, p
    icl, rem = c.build_icl_block(ref_tok, text, codes)
    assert icl.shape[0] == 400 and rem.shape[0] == int(f["remainder_rows"])
    hid, lg, pos = c.prefill_custom_voice(text, m["speaker"], m["language"], voice, icl)
    assert pos == int(f["position"]) == 409
    for name, got in (("hidden", hid), ("logits", lg)):
        ok, e = close(got, f[name])
        assert ok, f"prompt {name}: rel err {e}"
    for l in m["kv"]["layers"]:
        k, v = c.kv_gather(l)
        for name, got in ((f"k_l{l}", k[m["kv"]["positions"]]), (f"v_l{l}", v[m["kv"]["positions"]])):
            for i, pos_i in enumerate(m["kv"]["positions"]):
                ok, e = close(got[i], f[name][i])
                assert ok, f"{name} position {pos_i}: rel err {e}"
    ref = f["codes"]
    c.gen_set_text(rem, c.embed_text_token(G.TTS_PAD))
    c.gen_begin(lg, hid, pos, m["seed"], qtts.sample_params(top_k=1, eos_enabled=False))
    pred = np.concatenate([c.gen_frames_forced(ref[:20]), c.gen_frames_forced(ref[20:])])
    assert np.array_equal(pred[:, 0], ref[:, 0]), f"code 0: {pred[:, 0]} vs {ref[:, 0]}"
    assert (pred[:, 1:] == ref[:, 1:]).mean() >= 0.99
    lg2, hd2, pos2, _ = c.gen_state()
    assert pos2 == 409 + ref.shape[0]
    for name, got, want in (("logits", lg2, f["final_logits"]), ("hidden", hd2, f["final_hidden"])):
        ok, e = close(got, want)
        assert ok, f"after the frames, {name}: rel err {e}"
    c.close()
