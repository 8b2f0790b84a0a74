"""Writes the golden fixtures of this directory with the oracle (the C
restatement of the reference's CPU path), on the CPU:

    python tests/golden/make_golden.py

Each fixture holds outputs only; its inputs are regenerated from the seeds
recorded in manifest.json (numpy PCG64 through qtts.synth and
tests/refgen.py), and a SHA-256 prefix of every input array is recorded so a
drift of the generators is caught before any comparison.

  gemv.npz            the GEMV k 2048 -> n 6144 (seed 1) and the
                      reference's own differential cases (gemv.rs:756-861),
                      gemv_q4_scalar order
  talker_step.npz     one talker layer at the 1.7B shapes, KV N(0,1) to 512,
                      one appended position: hidden, logits, the new K/V row
  predictor.npz       the 15-codebook chain for 4 inputs (greedy argmax)
  greedy_frames.npz   200 greedy frames (top-k 1) after a 16-row prefill
  decoder.npz         the speech decoder (reduced widths) on 12 frames
                      after 4 warmup frames
  icl28.npz           the ICL workload at full depth (28-layer talker):
                      a voice-clone prompt of 9 + 400 rows (build_icl_block
                      of 150 reference tokens, 269 text tokens and 399
                      reference frames, prefill_custom_voice), then 32
                      greedy frames fed the block's 20 remainder rows, then
                      tts_pad: hidden, logits, K/V rows of layers 0, 13, 27,
                      the frames' codes, the last frame's logits and hidden

    python tests/golden/make_golden.py            every fixture
    python tests/golden/make_golden.py icl28      icl28.npz only (minutes)
"""
import hashlib
import json
import os
import sys
from dataclasses import fields, is_dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (os.path.join(ROOT, "qora-tts-12hz-1.7b_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

import oracle as O  # noqa: E402
import qtts  # noqa: E402
import refgen  # noqa: E402
from qtts import synth  # noqa: E402

WORKERS, THREADS = 16, 8       # oracle GEMV chunking (the bits depend on it)
TALKER = dict(seed=201, n_layers=1, text_vocab=256, rope_max_pos=1024)
PREDICTOR = dict(seed=202, n_layers=5)
DECODER = dict(seed=211, latent=64, hidden=64, n_heads=4, head_dim=16, inter=128, n_tf_layers=2, codebook_size=64,
               codebook_dim=32, vq_dim=32, vocos=(48, 32, 24, 16, 8), rope_max_pos=512)
GREEDY_FRAMES = 200
ICL28 = dict(talker=dict(seed=221, n_layers=28, rope_max_pos=2048), predictor=dict(seed=222, n_layers=5))
ICL28_FRAMES = 32
ICL28_KV = dict(layers=[0, 13, 27], positions=[0, 204, 408])
TTS_PAD = 151671


def digest(obj):
    """SHA-256 prefix over every array reachable from obj, in field order."""
    h = hashlib.sha256()

    def walk(o):
        if isinstance(o, np.ndarray):
            h.update(np.ascontiguousarray(o).tobytes())
        elif is_dataclass(o):
            for f in fields(o):
                walk(getattr(o, f.name))
        elif isinstance(o, (list, tuple)):
            for x in o:
                walk(x)
    walk(obj)
    return h.hexdigest()[:16]


def gemv_inputs():
    rng = np.random.Generator(np.random.PCG64(1))
    w = synth.q4_random(rng, 2048, 6144)
    x = rng.standard_normal(2048).astype(np.float32)
    cases = {}
    for c in [c + (0.0, 0.0) for c in refgen.SHAPE_CASES] + refgen.SPARSE_CASES:
        k, n, seed, iz, sz = c
        cases[f"case_{k}x{n}_s{seed}"] = refgen.case(k, n, seed, iz, sz)
    return w, x, cases


def models():
    return synth.make_talker(**TALKER), synth.make_predictor(**PREDICTOR)


def talker_step_inputs(t):
    rng = np.random.Generator(np.random.PCG64(6))
    L = 512
    K = rng.standard_normal((len(t.layers), L, 8, 128)).astype(np.float32)
    V = rng.standard_normal((len(t.layers), L, 8, 128)).astype(np.float32)
    emb = rng.standard_normal(t.hidden).astype(np.float32)
    return K, V, emb


def predictor_inputs(t):
    out = []
    for seed in range(4):
        rng = np.random.Generator(np.random.PCG64(100 + seed))
        th = rng.standard_normal(t.hidden).astype(np.float32)
        out.append((th, int(rng.integers(0, 2048))))
    return out


def greedy_prompt(t):
    return np.random.Generator(np.random.PCG64(11)).standard_normal((16, t.hidden)).astype(np.float32)


def decoder_inputs(d):
    rng = np.random.Generator(np.random.PCG64(4900))
    codes = rng.integers(0, d.codebook_size, (16, 12)).astype(np.uint32)
    warm = rng.integers(0, d.codebook_size, (16, 4)).astype(np.uint32)
    return codes, warm


def icl28_models():
    return synth.make_talker(**ICL28["talker"]), synth.make_predictor(**ICL28["predictor"])


def icl28_inputs():
    """Reference tokens, text tokens, reference codes [16][399] and a voice
    embedding: 150 + 269 + 1 text rows against 399 + 1 codec rows, so the
    ICL block holds 400 rows and leaves 20 text rows as the remainder
    (icl_block_layout, generate_new.rs:120-128)."""
    rng = np.random.Generator(np.random.PCG64(2210))
    ref = rng.integers(0, 151936, 150).astype(np.uint32)
    text = rng.integers(0, 151936, 269).astype(np.uint32)
    codes = rng.integers(0, 2048, (16, 399)).astype(np.uint32)
    voice = rng.standard_normal(2048).astype(np.float32)
    return ref, text, codes, voice


def run_icl28(om):
    """generate_speech's ICL path (generate_new.rs:479-675) on the oracle."""
    ref, text, codes, voice = icl28_inputs()
    om.kv_reset()
    icl, rem = om.build_icl_block(ref, text, codes)
    hid, lg, pos, _ = om.prefill_custom_voice(text, 0, 2055, voice, icl)
    out = {"hidden": hid, "logits": lg, "position": np.int64(pos), "remainder_rows": np.int64(rem.shape[0])}
    for l in ICL28_KV["layers"]:
        k, v = om.kv_layer(l)
        out[f"k_l{l}"] = k[ICL28_KV["positions"]]
        out[f"v_l{l}"] = v[ICL28_KV["positions"]]
    pad = om.embed_text_token(TTS_PAD)
    om.gen_begin(lg, hid, pos, 42)
    params = qtts.sample_params(top_k=1, eos_enabled=False)
    out["codes"] = np.stack([om.frame(params, rem[f] if f < rem.shape[0] else pad)[0] for f in range(ICL28_FRAMES)])
    out["final_logits"] = om.g_logits.copy()
    out["final_hidden"] = om.g_hidden.copy()
    om.kv_reset()
    return out


def write_icl28(manifest):
    t, p = icl28_models()
    om = O.Model(t, p, kv_cap=1024)
    np.savez_compressed(os.path.join(HERE, "icl28.npz"), **run_icl28(om))
    om.close()
    manifest["fixtures"]["icl28"] = {"talker": ICL28["talker"], "predictor": ICL28["predictor"],
                                     "model": digest((t, p)), "inputs": digest(icl28_inputs()),
                                     "frames": ICL28_FRAMES, "seed": 42, "kv": ICL28_KV,
                                     "speaker": 0, "language": 2055,
                                     "bar": "hidden, logits, K/V rows and the last frame's logits and hidden within "
                                            "1e-3 * max(max|ref|, rms(ref)); code 0 exact and >= 99% of the "
                                            "codes, teacher-forced"}


def run_talker_step(om, t):
    K, V, emb = talker_step_inputs(t)
    om.kv_reset()
    om.kv_load(K, V)
    out = om.forward_with_embedding(emb, 512)
    k, v = om.kv_layer(0)
    om.kv_reset()
    return {"hidden": out[: t.hidden], "logits": out[t.hidden:], "k_new": k[512], "v_new": v[512]}


def run_predictor(om):
    t = om.t
    codes = [om.predictor_chain(th, om.embed_codec_token(sem)) for th, sem in predictor_inputs(t)]
    return {"codes": np.stack(codes)}


def run_greedy(om, n_frames):
    t = om.t
    X = greedy_prompt(t)
    om.kv_reset()
    hid = om.prefill(X, 0)
    logits = om.codec_head(hid)
    pad = om.embed_text_token(3)
    om.gen_begin(logits, hid, 16, 42)
    params = qtts.sample_params(top_k=1, eos_enabled=False)
    codes = np.stack([om.frame(params, pad)[0] for _ in range(n_frames)])
    om.kv_reset()
    return {"codes": codes}


def main(which=None):
    O.set_workers(WORKERS, THREADS)
    if which == "icl28":
        path = os.path.join(HERE, "manifest.json")
        manifest = json.load(open(path))
        write_icl28(manifest)
        with open(path, "w") as f:
            json.dump(manifest, f, indent=1, sort_keys=True)
            f.write("\n")
        return
    manifest = {"oracle_workers": WORKERS, "oracle_threads": THREADS, "fixtures": {}}

    w, x, cases = gemv_inputs()
    out = {"gemv_2048x6144_y": O.gemv_scalar(x, w)}
    for name, (cx, cw) in cases.items():
        out[name + "_y"] = O.gemv_scalar(cx, cw)
    np.savez(os.path.join(HERE, "gemv.npz"), **out)
    manifest["fixtures"]["gemv"] = {
        "inputs": {"gemv_2048x6144": digest((w, x)), **{k: digest(v) for k, v in cases.items()}},
        "tolerance": "1e-3 * max(max|ref|, rms(ref))"}

    t, p = models()
    om = O.Model(t, p, kv_cap=1024)
    md = digest((t, p))
    np.savez(os.path.join(HERE, "talker_step.npz"), **run_talker_step(om, t))
    manifest["fixtures"]["talker_step"] = {"talker": TALKER, "predictor": PREDICTOR, "model": md,
                                           "inputs": digest(talker_step_inputs(t)),
                                           "tolerance": "1e-3 * max(max|ref|, rms(ref))"}
    np.savez(os.path.join(HERE, "predictor.npz"), **run_predictor(om))
    manifest["fixtures"]["predictor"] = {"model": md, "inputs": digest([a for a, _ in predictor_inputs(t)]),
                                         "semantic_codes": [s for _, s in predictor_inputs(t)],
                                         "bar": "first input exact, >= 99% of codes"}
    np.savez(os.path.join(HERE, "greedy_frames.npz"), **run_greedy(om, GREEDY_FRAMES))
    manifest["fixtures"]["greedy_frames"] = {"model": md, "inputs": digest(greedy_prompt(t)), "frames": GREEDY_FRAMES,
                                             "seed": 42, "text_add": "embed_text_token(3)",
                                             "bar": ">= 99% of codes, teacher-forced"}
    om.close()

    d = synth.make_decoder(**DECODER)
    codes, warm = decoder_inputs(d)
    np.savez(os.path.join(HERE, "decoder.npz"), audio=O.decode_to_audio(d, codes, warmup=warm, threads=THREADS))
    manifest["fixtures"]["decoder"] = {"decoder": {k: list(v) if isinstance(v, tuple) else v for k, v in DECODER.items()},
                                       "model": digest(d), "inputs": digest((codes, warm)),
                                       "tolerance": "1e-3 * max|ref|"}
    write_icl28(manifest)
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
        f.write("\n")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else None)
