"""Matrix-core prefill: the MFMA Q4 GEMM (`gemm_q4`, gemv.rs:349-412) and the
batched talker prefill (`prefill_talker_raw_from`, talker.rs:379-482)
against the oracle, with the same bars as the decode path: outputs within
|d| <= 1e-3 * max(max|ref|, rms(ref)), the KV cache within the same bar per
layer, greedy codes after an ICL-length prefill agreeing at >= 99%.
"""
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


@pytest.fixture(scope="module")
def ctx(ctx_factory):
    return ctx_factory(4096)


@pytest.fixture(scope="module")
def model2():
    t = synth.make_talker(seed=401, n_layers=2, text_vocab=512, rope_max_pos=4096)
    p = synth.make_predictor(seed=402, n_layers=5)
    return t, p


@pytest.fixture(scope="module")
def loaded(ctx, model2):
    t, p = model2
    ctx.upload_model(t, p)
    O.set_workers(16, 8)
    om = O.Model(t, p, kv_cap=4096)
    yield ctx, om, t, p
    om.close()


# ---- GEMM ---------------------------------------------------------------

@pytest.mark.parametrize("cfg", [None, 0, 1, 5, 8, 9, 13, 17])
def test_gemm_mfma_every_layout(ctx, cfg, monkeypatch):
    """The matrix-core GEMM reads the weight through the tiled layout's
    address map: every tile family (one group per wave, groups interleaved
    by thread, 1-8 groups, 2-8 rows per thread); row counts on and off the
    64-row block; n not a multiple of 32 (tail columns stay zero)."""
    if cfg is not None:
        monkeypatch.setenv("QTTS_TILE_GEMV", str(cfg))
    rng = np.random.Generator(np.random.PCG64(2000 + (cfg or 0)))
    for k, n, rows in ((2048, 3072, 65), (6144, 2048, 17), (1024, 96, 1), (2048, 1000, 64), (512, 4096, 130)):
        w = synth.q4_random(rng, k, n)
        X = rng.standard_normal((rows, k)).astype(np.float32)
        dw = ctx.upload(w)
        Y = ctx.gemm(dw, X, path="mfma")
        dw.free()
        R = O.gemm(X, w)
        for r in range(rows):
            ok, e = close(Y[r], R[r])
            assert ok, f"cfg {cfg} k={k} n={n} rows={rows} row {r} rel err {e}"
        assert not Y[:, (n // 32) * 32:].any()


def test_gemm_paths_agree(ctx):
    """Default choice by row count: 16+ rows on the matrix cores, fewer row
    by row; both against the oracle on the same input."""
    rng = np.random.Generator(np.random.PCG64(2100))
    w = synth.q4_random(rng, 2048, 6144)
    X = rng.standard_normal((40, 2048)).astype(np.float32)
    dw = ctx.upload(w)
    Ym, Yr, Yd = ctx.gemm(dw, X, path="mfma"), ctx.gemm(dw, X, path="rowwise"), ctx.gemm(dw, X)
    dw.free()
    R = O.gemm(X, w)
    for r in range(40):
        assert close(Ym[r], R[r])[0] and close(Yr[r], R[r])[0]
    assert np.array_equal(Yd, Ym)


# ---- talker prefill ---------------------------------------------------------

def check_kv(ctx, om, n_layers, upto):
    for l in range(n_layers):
        k, v = ctx.kv_gather(l)
        ko, vo = om.kv_layer(l)
        assert k.shape[0] == upto == ko.shape[0]
        ok_k, ek = close(k, ko)
        ok_v, ev = close(v, vo)
        assert ok_k and ok_v, f"layer {l}: K rel err {ek}, V rel err {ev}"


def test_prefill_mfma_matches_oracle(loaded):
    ctx, om, t, p = loaded
    rng = np.random.Generator(np.random.PCG64(2200))
    X = rng.standard_normal((100, t.hidden)).astype(np.float32)
    ctx.kv_reset()
    om.kv_reset()
    h = ctx.prefill_talker_raw_from(X, 0, path="mfma")
    ok, e = close(h, om.prefill(X, 0))
    assert ok, f"prefill rel err {e}"
    assert ctx.kv_len() == 100
    check_kv(ctx, om, len(t.layers), 100)
    # decode steps on top of the batched prefill
    for step in range(2):
        emb = rng.standard_normal(t.hidden).astype(np.float32)
        ok, e = close(ctx.forward_with_embedding(emb, 100 + step), om.forward_with_embedding(emb, 100 + step))
        assert ok, f"step {step} rel err {e}"
    ctx.kv_reset()
    om.kv_reset()


def test_prefill_mfma_on_prefix(loaded):
    """A suffix prefilled on top of a cached prefix (prefill_talker_raw_from
    with start_pos > 0, talker.rs:419-430): the suffix attends to the prefix
    and its own earlier rows."""
    ctx, om, t, p = loaded
    rng = np.random.Generator(np.random.PCG64(2300))
    A = rng.standard_normal((37, t.hidden)).astype(np.float32)
    B = rng.standard_normal((90, t.hidden)).astype(np.float32)
    ctx.kv_reset()
    om.kv_reset()
    ok, e = close(ctx.prefill_talker_raw_from(A, 0, path="mfma"), om.prefill(A, 0))
    assert ok, f"prefix rel err {e}"
    ok, e = close(ctx.prefill_talker_raw_from(B, 37, path="mfma"), om.prefill(B, 37))
    assert ok, f"suffix rel err {e}"
    check_kv(ctx, om, len(t.layers), 127)
    ctx.kv_reset()
    om.kv_reset()


def test_prefill_mfma_single_row_and_paths(loaded):
    """One row forced onto the matrix cores; the row-by-row path on the same
    input gives the same hidden within the bar."""
    ctx, om, t, p = loaded
    rng = np.random.Generator(np.random.PCG64(2400))
    X = rng.standard_normal((1, t.hidden)).astype(np.float32)
    ctx.kv_reset()
    om.kv_reset()
    ref = om.prefill(X, 0)
    assert close(ctx.prefill_talker_raw_from(X, 0, path="mfma"), ref)[0]
    ctx.kv_reset()
    assert close(ctx.prefill_talker_raw_from(X, 0, path="rowwise"), ref)[0]
    ctx.kv_reset()
    om.kv_reset()


def test_prefill_pieces_bit_identical_across_groups(loaded):
    """Each row's attention walks its pages, and each wave its fixed position
    quarter of a page, in the same order whatever rows share the launch: a
    500-row prompt prefilled whole and as 300 + 200 rows (and as 37 + 463)
    gives the same last hidden and the same cache, bit for bit, and matches
    the oracle."""
    ctx, om, t, p = loaded
    rng = np.random.Generator(np.random.PCG64(2360))
    X = rng.standard_normal((500, t.hidden)).astype(np.float32)
    ctx.kv_reset()
    whole = ctx.prefill_talker_raw_from(X, 0, path="mfma")
    kv_whole = [ctx.kv_gather(l) for l in range(len(t.layers))]
    om.kv_reset()
    ok, e = close(whole, om.prefill(X, 0))
    assert ok, f"rel err {e}"
    om.kv_reset()
    for cut in (300, 37):
        ctx.kv_reset()
        ctx.prefill_talker_raw_from(X[:cut], 0, path="mfma")
        h = ctx.prefill_talker_raw_from(X[cut:], cut, path="mfma")
        assert np.array_equal(h.view(np.uint32), whole.view(np.uint32)), f"cut {cut}: hidden differs"
        for l in range(len(t.layers)):
            k, v = ctx.kv_gather(l)
            assert np.array_equal(k.view(np.uint32), kv_whole[l][0].view(np.uint32)), f"cut {cut} layer {l} K"
            assert np.array_equal(v.view(np.uint32), kv_whole[l][1].view(np.uint32)), f"cut {cut} layer {l} V"
    ctx.kv_reset()


@pytest.mark.parametrize("env", ["QTTS_GEMM_F32", "QTTS_PREFILL_ATTN_VALU"])
def test_prefill_fallback_paths(loaded, env, monkeypatch):
    """The f32-instruction GEMM (QTTS_GEMM_F32=1) and the VALU attention
    (QTTS_PREFILL_ATTN_VALU=1) kept beside the split-f16 matrix-core kernels:
    each against the oracle on a prefill over a cached prefix, and against
    the default path within the same bar."""
    ctx, om, t, p = loaded
    rng = np.random.Generator(np.random.PCG64(2350))
    A = rng.standard_normal((70, t.hidden)).astype(np.float32)
    B = rng.standard_normal((90, t.hidden)).astype(np.float32)
    ctx.kv_reset()
    om.kv_reset()
    ref_a, ref_b = om.prefill(A, 0), om.prefill(B, 70)
    ctx.prefill_talker_raw_from(A, 0, path="mfma")
    default = ctx.prefill_talker_raw_from(B, 70, path="mfma")
    ctx.kv_reset()
    monkeypatch.setenv(env, "1")
    ok, e = close(ctx.prefill_talker_raw_from(A, 0, path="mfma"), ref_a)
    assert ok, f"{env}: prefix rel err {e}"
    got = ctx.prefill_talker_raw_from(B, 70, path="mfma")
    ok, e = close(got, ref_b)
    assert ok, f"{env}: suffix rel err {e}"
    assert close(got, default)[0]
    check_kv(ctx, om, len(t.layers), 160)
    if env == "QTTS_GEMM_F32":
        w = synth.q4_random(rng, 2048, 4096)
        X = rng.standard_normal((40, 2048)).astype(np.float32)
        dw = ctx.upload(w)
        Y = ctx.gemm(dw, X, path="mfma")
        dw.free()
        R = O.gemm(X, w)
        for r in range(40):
            assert close(Y[r], R[r])[0], f"f32 GEMM row {r}"
    ctx.kv_reset()
    om.kv_reset()


def test_prefill_chunked(ctx_factory):
    """More rows than one prefill chunk (1024): the second chunk attends to
    the first through the cache."""
    t = synth.make_talker(seed=411, n_layers=1, text_vocab=256, rope_max_pos=2048)
    p = synth.make_predictor(seed=412, n_layers=5)
    c = ctx_factory(2048)
    c.upload_model(t, p)
    om = O.Model(t, p, kv_cap=2048)
    rng = np.random.Generator(np.random.PCG64(2500))
    X = rng.standard_normal((1100, t.hidden)).astype(np.float32)
    ok, e = close(c.prefill_talker_raw_from(X, 0), om.prefill(X, 0))
    assert ok, f"rel err {e}"
    check_kv(c, om, 1, 1100)
    om.close()
    c.close()


def test_prefill_28_layers_paths_agree(ctx_factory):
    """Full depth (28 layers of the 1.7B shapes), 400 rows: the matrix-core
    prefill against the row-by-row decode kernels (each pinned to the oracle
    above) on the hidden and on every layer's cache."""
    t = synth.make_talker(seed=421, n_layers=28, text_vocab=256, rope_max_pos=1024)
    p = synth.make_predictor(seed=422, n_layers=5)
    c = ctx_factory(1024)
    c.upload_model(t, p)
    rng = np.random.Generator(np.random.PCG64(2600))
    X = rng.standard_normal((400, t.hidden)).astype(np.float32)
    hm = c.prefill_talker_raw_from(X, 0, path="mfma")
    km = [c.kv_gather(l) for l in range(28)]
    c.kv_reset()
    hr = c.prefill_talker_raw_from(X, 0, path="rowwise")
    ok, e = close(hm, hr)
    assert ok, f"hidden rel err {e}"
    for l in range(28):
        k, v = c.kv_gather(l)
        assert close(km[l][0], k)[0] and close(km[l][1], v)[0], f"layer {l}"
    c.close()


def test_icl_prefill_then_greedy_frames(ctx_factory):
    """ICL-style prompt: 400 positions (text rows of ids uniform in
    [0, 151936) and rows of 16-codebook reference codes uniform in
    [0, 2048)), prefilled on the matrix cores, then 100 greedy frames
    teacher-forced on the oracle's codes: >= 99% of the codes agree."""
    t = synth.make_talker(seed=431, n_layers=4, rope_max_pos=1024)
    p = synth.make_predictor(seed=432, n_layers=5)
    c = ctx_factory(1024)
    c.upload_model(t, p)
    O.set_workers(16, 8)
    om = O.Model(t, p, kv_cap=1024)
    rng = np.random.Generator(np.random.PCG64(2700))
    n_text, n_ref = 200, 200
    rows = [om.embed_text_token(int(tok)) for tok in rng.integers(0, 151936, n_text)]
    for codes in rng.integers(0, 2048, (n_ref, 16)):
        sem = om.embed_codec_token(int(codes[0]))
        rows.append(sem + om.acoustic_embed_sum(codes[1:]))
    X = np.stack(rows).astype(np.float32)
    hid = om.prefill(X, 0)
    h = c.prefill_talker_raw_from(X, 0)
    ok, e = close(h, hid)
    assert ok, f"prefill rel err {e}"
    params = qtts.sample_params(top_k=1, eos_enabled=False)
    logits = om.codec_head(hid)
    pad = om.embed_text_token(3)
    c.gen_set_text(None, pad)
    om.gen_begin(logits, hid, 400, 42)
    c.gen_begin(logits, hid, 400, 42, params)
    ref = np.stack([om.frame(params, pad)[0] for _ in range(100)])
    pred = c.gen_frames_forced(ref)
    agree = (pred == ref).mean()
    assert agree >= 0.99, f"agreement {agree:.4f}"
    om.close()
    c.close()
