"""`.qora-tts` loading (save.rs:262-552 -> qtts_model_load_qtts): a model
written in the reference's stream layout by tests/qtts_writer.py and loaded
from the file behaves bit-for-bit like the same weights uploaded from
memory -- talker, predictor and speech decoder -- and malformed files fail
with the documented status before anything is uploaded."""
import os

import numpy as np
import pytest

import oracle as O
import qtts
from qtts import synth
from qtts_writer import write_qora_q4, write_qtts

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def model_file(tmp_path_factory):
    t = synth.make_talker(seed=301, n_layers=2, text_vocab=256, rope_max_pos=2048)
    p = synth.make_predictor(seed=302, n_layers=5, rope_max_pos=64)
    path = str(tmp_path_factory.mktemp("qtts") / "model.qora-tts")
    write_qtts(path, t, p)
    return path, t, p


def test_loaded_model_matches_upload(ctx_factory, model_file):
    path, t, p = model_file
    a, b = ctx_factory(1024), ctx_factory(1024)
    a.upload_model(t, p)
    b.load_qtts(path)
    assert b.dims() == a.dims() == (t.hidden, t.vocab, len(t.layers), p.hidden, p.vocab, len(p.lm_heads))
    rng = np.random.Generator(np.random.PCG64(31))
    X = rng.standard_normal((12, t.hidden)).astype(np.float32)
    ha = a.prefill_talker_raw_from(X, 0)
    hb = b.prefill_talker_raw_from(X, 0)
    assert np.array_equal(bits(ha), bits(hb))
    emb = rng.standard_normal(t.hidden).astype(np.float32)
    assert np.array_equal(bits(a.forward_with_embedding(emb, 12)), bits(b.forward_with_embedding(emb, 12)))
    for tok in (0, 100, 255):
        assert np.array_equal(bits(a.embed_text_token(tok)), bits(b.embed_text_token(tok)))
    sem = a.embed_codec_token(2000)
    assert np.array_equal(a.generate_acoustic_codes(ha, sem), b.generate_acoustic_codes(hb, sem))
    # and the loaded model against the oracle
    om = O.Model(t, p, kv_cap=64)
    ref = om.prefill(X, 0)
    scale = max(np.abs(ref).max(), np.sqrt((ref ** 2).mean()))
    assert np.abs(hb - ref).max() <= 1e-3 * scale
    om.close()


def test_malformed_files(ctx_factory, model_file, tmp_path):
    path, t, p = model_file
    c = ctx_factory(256)
    data = open(path, "rb").read()
    cases = {
        "bad_magic": (b"QTTX" + data[4:], qtts.ERR_IO),
        "bad_version": (data[:4] + (2).to_bytes(4, "little") + data[8:], qtts.ERR_IO),
        "truncated": (data[: len(data) // 2], qtts.ERR_IO),
        "f16_format": (data[:8] + bytes([0]) + data[9:], qtts.ERR_UNSUPPORTED),
        "empty": (b"", qtts.ERR_IO),
    }
    # talker head_dim (u32 at byte 29: magic, version, format, then n_layers,
    # hidden, text_hidden, n_heads, n_kv_heads): 1 once divided by zero in
    # the RoPE table check; every width but 128 is refused with a status
    for hd in (0, 1, 2, 64, 256):
        cases[f"head_dim_{hd}"] = (data[:29] + hd.to_bytes(4, "little") + data[33:], qtts.ERR_IO)
    for name, (blob, code) in cases.items():
        f = tmp_path / f"{name}.qora-tts"
        f.write_bytes(blob)
        with pytest.raises(qtts.QttsError) as e:
            c.load_qtts(str(f))
        assert e.value.code == code, f"{name}: status {e.value.code}"
    with pytest.raises(qtts.QttsError) as e:
        c.load_qtts(str(tmp_path / "missing.qora-tts"))
    assert e.value.code == qtts.ERR_IO


def small_decoder():
    return synth.make_decoder(seed=41, latent=64, hidden=64, n_heads=4, head_dim=16, inter=128, n_tf_layers=2,
                              codebook_size=64, codebook_dim=32, vq_dim=32, vocos=(48, 32, 24, 16, 8),
                              rope_max_pos=512)


@pytest.fixture(scope="module")
def full_file(tmp_path_factory):
    t = synth.make_talker(seed=311, n_layers=1, text_vocab=256, rope_max_pos=256)
    p = synth.make_predictor(seed=312, n_layers=5, rope_max_pos=64)
    d = small_decoder()
    path = str(tmp_path_factory.mktemp("qtts") / "full.qora-tts")
    write_qtts(path, t, p, decoder=d)
    return path, t, p, d


def test_loaded_decoder_matches_upload(ctx_factory, full_file):
    path, t, p, d = full_file
    a, b = ctx_factory(256), ctx_factory(256)
    a.upload_decoder(d)
    b.load_qtts(path)
    assert b.decoder_dims() == a.decoder_dims() == (16, d.codebook_size, d.upsample_factor)
    rng = np.random.Generator(np.random.PCG64(32))
    codes = rng.integers(0, d.codebook_size, (16, 25))
    warm = rng.integers(0, d.codebook_size, (16, 7))
    assert np.array_equal(bits(a.decode_to_audio(codes, warm)), bits(b.decode_to_audio(codes, warm)))
    # the talker and predictor of the same file still load as before
    emb = rng.standard_normal(t.hidden).astype(np.float32)
    a.upload_model(t, p)
    assert np.array_equal(bits(a.forward_with_embedding(emb, 0)), bits(b.forward_with_embedding(emb, 0)))


def test_malformed_decoder_section(ctx_factory, full_file, tmp_path):
    path, t, p, d = full_file
    data = open(path, "rb").read()
    write_qtts(str(tmp_path / "head.qora-tts"), t, p)
    head = len(open(tmp_path / "head.qora-tts", "rb").read())   # where the decoder section starts
    assert data[:head] == open(tmp_path / "head.qora-tts", "rb").read()
    c = ctx_factory(256)
    for name, blob in (("cut_config", data[:head + 10]), ("cut_middle", data[:(head + len(data)) // 2]),
                       ("cut_rope", data[:len(data) - 3])):
        f = tmp_path / f"{name}.qora-tts"
        f.write_bytes(blob)
        with pytest.raises(qtts.QttsError) as e:
            c.load_qtts(str(f))
        assert e.value.code == qtts.ERR_IO, name
        assert not c.has_decoder(), name


def test_qora_q4_container(ctx_factory, tmp_path):
    """The older named-tensor container (loader.rs:47-127 read, 724-882
    mapped): the same weights, biases rounded to f16 as the container stores
    them, behave bit for bit like an upload; a bad header, a truncated file,
    a missing lm head and an F16 linear weight fail with their statuses."""
    from dataclasses import replace
    r16 = lambda v: np.asarray(v, np.float32).astype(np.float16).astype(np.float32)
    t = synth.make_talker(seed=321, n_layers=2, text_vocab=256, rope_max_pos=512)
    p = synth.make_predictor(seed=322, n_layers=5, rope_max_pos=64)
    t = replace(t, text_fc1_bias=r16(t.text_fc1_bias), text_fc2_bias=r16(t.text_fc2_bias))
    p = replace(p, input_proj_bias=r16(p.input_proj_bias))
    path = str(tmp_path / "legacy.qora-tts")
    write_qora_q4(path, t, p)
    ropes = ((t.rope_cos, t.rope_sin), (p.rope_cos, p.rope_sin))
    a, b = ctx_factory(512), ctx_factory(512)
    a.upload_model(t, p)
    b.load_qora_q4(path, *ropes)
    assert b.dims() == a.dims() == (t.hidden, t.vocab, len(t.layers), p.hidden, p.vocab, len(p.lm_heads))
    rng = np.random.Generator(np.random.PCG64(33))
    X = rng.standard_normal((12, t.hidden)).astype(np.float32)
    ha, hb = a.prefill_talker_raw_from(X, 0), b.prefill_talker_raw_from(X, 0)
    assert np.array_equal(bits(ha), bits(hb))
    emb = rng.standard_normal(t.hidden).astype(np.float32)
    assert np.array_equal(bits(a.forward_with_embedding(emb, 12)), bits(b.forward_with_embedding(emb, 12)))
    for tok in (0, 200):
        assert np.array_equal(bits(a.embed_text_token(tok)), bits(b.embed_text_token(tok)))
    sem = a.embed_codec_token(1500)
    assert np.array_equal(a.generate_acoustic_codes(ha, sem), b.generate_acoustic_codes(hb, sem))

    data = open(path, "rb").read()
    c = ctx_factory(256)
    bad = {"bad_header": (b"QORA-TTS-Q5" + data[11:], qtts.ERR_IO),
           "truncated": (data[: len(data) // 2], qtts.ERR_IO),
           "empty": (b"", qtts.ERR_IO)}
    for name, (blob, code) in bad.items():
        f = tmp_path / f"{name}.qora-tts"
        f.write_bytes(blob)
        with pytest.raises(qtts.QttsError) as e:
            c.load_qora_q4(str(f), *ropes)
        assert e.value.code == code, name
    write_qora_q4(str(tmp_path / "short.qora-tts"), t, replace(p, lm_heads=p.lm_heads[:-1]))
    with pytest.raises(qtts.QttsError) as e:
        c.load_qora_q4(str(tmp_path / "short.qora-tts"), *ropes)
    assert e.value.code == qtts.ERR_IO
    write_qora_q4(str(tmp_path / "f16.qora-tts"), t, p, f16_weights={"talker.codec_head.weight"})
    with pytest.raises(qtts.QttsError) as e:
        c.load_qora_q4(str(tmp_path / "f16.qora-tts"), *ropes)
    assert e.value.code == qtts.ERR_UNSUPPORTED


def test_device_bytes_report(ctx_factory):
    """qtts_device_bytes: each part from the shapes of what was uploaded."""
    t = synth.make_talker(seed=171, n_layers=2, text_vocab=256)
    p = synth.make_predictor(seed=172, n_layers=2)
    c = ctx_factory(256)
    c.upload_model(t, p)
    r = c.device_bytes()
    q4 = lambda w: w.nbytes                 # nibbles + an f16 scale per 32 columns
    talker = sum(q4(w) for L in t.layers for w in (L.q_proj, L.k_proj, L.v_proj, L.o_proj, L.gate_proj,
                                                   L.up_proj, L.down_proj))
    talker += q4(t.codec_head) + q4(t.text_fc1) + q4(t.text_fc2)
    pred = sum(q4(w) for L in p.layers for w in (L.q_proj, L.k_proj, L.v_proj, L.o_proj, L.gate_proj,
                                                 L.up_proj, L.down_proj))
    pred += sum(q4(h) for h in p.lm_heads) + q4(p.input_proj)
    # tiles pad k to whole slices and n to whole groups, never below the weights
    assert talker <= r["talker_q4"] <= 1.25 * talker
    assert pred <= r["predictor_q4"] <= 1.25 * pred
    ntab, rows = len(p.lm_heads) - 1, p.codec_embeddings[0].k
    assert r["predictor_row_tables"] == ntab * rows * p.hidden * 4
    assert r["predictor_qkv_tables"] >= ntab * rows * 4096 * 4
    emb = q4(t.codec_embedding) + q4(t.text_embedding) + sum(q4(e) for e in p.codec_embeddings)
    assert r["embedding_rows"] == emb
    assert r["kv_pool"] == len(t.layers) * 2 * (256 // 64) * 2 * 8 * 64 * 128 * 4
    parts = sum(v for k, v in r.items() if k != "device_used")
    assert r["device_used"] >= parts
