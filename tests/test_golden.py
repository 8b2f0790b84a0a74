"""The committed golden fixtures (tests/golden/, written by make_golden.py)
against the oracle, on the CPU: the seeded generators still produce the
recorded inputs (SHA-256 prefixes), and the oracle still produces the
recorded outputs bit for bit -- so the fixtures the GPU tests read and the
oracle they were made with cannot drift apart unnoticed."""
import json
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_golden as G  # noqa: E402
import oracle as O  # noqa: E402
from qtts import synth  # noqa: E402

MANIFEST = json.load(open(os.path.join(HERE, "golden", "manifest.json")))


def fixture(name):
    return np.load(os.path.join(HERE, "golden", name + ".npz"))


def same_bits(a, b):
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    return a.shape == b.shape and a.tobytes() == b.tobytes()


@pytest.fixture(scope="module")
def oracle_model():
    O.set_workers(MANIFEST["oracle_workers"], MANIFEST["oracle_threads"])
    t, p = G.models()
    assert G.digest((t, p)) == MANIFEST["fixtures"]["talker_step"]["model"], "synthetic model generator drifted"
    om = O.Model(t, p, kv_cap=1024)
    yield om, t
    om.close()


def test_gemv_fixture():
    O.set_workers(MANIFEST["oracle_workers"], MANIFEST["oracle_threads"])
    w, x, cases = G.gemv_inputs()
    rec = MANIFEST["fixtures"]["gemv"]["inputs"]
    assert G.digest((w, x)) == rec["gemv_2048x6144"]
    f = fixture("gemv")
    assert same_bits(O.gemv_scalar(x, w), f["gemv_2048x6144_y"])
    for name, (cx, cw) in cases.items():
        assert G.digest((cx, cw)) == rec[name], name
        assert same_bits(O.gemv_scalar(cx, cw), f[name + "_y"]), name


def test_talker_step_fixture(oracle_model):
    om, t = oracle_model
    assert G.digest(G.talker_step_inputs(t)) == MANIFEST["fixtures"]["talker_step"]["inputs"]
    got, f = G.run_talker_step(om, t), fixture("talker_step")
    for k in ("hidden", "logits", "k_new", "v_new"):
        assert same_bits(got[k], f[k]), k


def test_predictor_fixture(oracle_model):
    om, t = oracle_model
    assert same_bits(G.run_predictor(om)["codes"], fixture("predictor")["codes"])


def test_greedy_frames_fixture_prefix(oracle_model):
    """The first 40 of the 200 recorded frames (frames are sequential, so a
    prefix regenerates exactly)."""
    om, t = oracle_model
    assert G.digest(G.greedy_prompt(t)) == MANIFEST["fixtures"]["greedy_frames"]["inputs"]
    got = G.run_greedy(om, 40)["codes"]
    assert same_bits(got, fixture("greedy_frames")["codes"][:40])


def test_decoder_fixture():
    d = synth.make_decoder(**G.DECODER)
    rec = MANIFEST["fixtures"]["decoder"]
    assert G.digest(d) == rec["model"]
    codes, warm = G.decoder_inputs(d)
    assert G.digest((codes, warm)) == rec["inputs"]
    got = O.decode_to_audio(d, codes, warmup=warm, threads=MANIFEST["oracle_threads"])
    assert same_bits(got, fixture("decoder")["audio"])


def test_icl28_fixture_inputs():
    """The 28-layer ICL fixture: its seeded inputs still regenerate
    (digest), and it holds what the GPU test reads.  Regenerating its
    outputs takes the oracle about three minutes (make_golden.py icl28), so
    this CPU check stops at the inputs."""
    rec = MANIFEST["fixtures"]["icl28"]
    assert G.digest(G.icl28_inputs()) == rec["inputs"]
    f = fixture("icl28")
    assert int(f["position"]) == 409 and int(f["remainder_rows"]) == 20
    assert f["codes"].shape == (rec["frames"], 16) and f["hidden"].shape == (2048,) and f["logits"].shape == (3072,)
    for l in rec["kv"]["layers"]:
        assert f[f"k_l{l}"].shape == f[f"v_l{l}"].shape == (len(rec["kv"]["positions"]), 8, 128)
    assert np.all(np.isfinite(f["final_logits"])) and np.all(np.isfinite(f["final_hidden"]))
