"""Parity of the HIP path (libqtts_hip.so via the C ABI) with the oracle.

Bars (from the decode path's contract): KV append/gather, embedding rows and
sums, argmax indices are bit-exact; GEMV, attention and whole-step outputs
agree within |d| <= 1e-3 * max(max|ref|, rms(ref)) (f32 accumulation in a
different order); predicted codes agree.
"""
import numpy as np
import pytest

import oracle as O
import qtts
import refgen
from qtts import synth

pytestmark = pytest.mark.gpu

TOL = 1e-3


def close(got, ref, rel=TOL):
    ref = np.asarray(ref, np.float64)
    scale = max(np.abs(ref).max(), np.sqrt((ref ** 2).mean()), 1e-30)
    err = np.abs(np.asarray(got, np.float64) - ref).max()
    return err <= rel * scale, err / scale


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def ctx(ctx_factory):
    return ctx_factory(4096)


@pytest.fixture(scope="module")
def small_model():
    t = synth.make_talker(seed=101, n_layers=2, text_vocab=512, rope_max_pos=4096)
    p = synth.make_predictor(seed=102, n_layers=5)
    return t, p


@pytest.fixture(scope="module")
def loaded(ctx, small_model):
    t, p = small_model
    ctx.upload_model(t, p)
    O.set_workers(16, 8)
    om = O.Model(t, p, kv_cap=4096)
    return ctx, om, t, p


# ---- operator level ------------------------------------------------------

def test_gemv_2048x6144(ctx):
    # one Q4 GEMV, k=2048 -> n=6144, nibbles uniform, scales |N(0,0.02)|, x ~ N(0,1)
    rng = np.random.Generator(np.random.PCG64(1))
    w = synth.q4_random(rng, 2048, 6144)
    x = rng.standard_normal(2048).astype(np.float32)
    dw = ctx.upload(w)
    y = ctx.gemv(dw, x)
    ok, e = close(y, O.gemv_scalar(x, w))
    dw.free()
    assert ok, f"rel err {e}"


@pytest.mark.parametrize("k,n,seed,iz,sz", [c + (0.0, 0.0) for c in refgen.SHAPE_CASES] + refgen.SPARSE_CASES
                         + [(16, 100, 31, 0.0, 0.0)])
def test_gemv_reference_cases(ctx, k, n, seed, iz, sz):
    x, w = refgen.case(k, n, seed, iz, sz)
    dw = ctx.upload(w)
    y = ctx.gemv(dw, x)
    dw.free()
    ref = O.gemv_scalar(x, w)
    ok, e = close(y, ref)
    assert ok, f"rel err {e}"
    assert np.all(y[(n // 32) * 32:] == 0.0)


@pytest.mark.parametrize("k,n", [(1024, 2048), (2048, 1024), (3072, 1024), (6144, 2048), (2048, 12288)])
def test_gemv_model_shapes(ctx, k, n):
    rng = np.random.Generator(np.random.PCG64(k * 7 + n))
    w = synth.q4_random(rng, k, n)
    x = (rng.standard_normal(k) * 3).astype(np.float32)
    dw = ctx.upload(w)
    y = ctx.gemv(dw, x)
    dw.free()
    ok, e = close(y, O.gemv_scalar(x, w))
    assert ok, f"rel err {e}"


@pytest.mark.parametrize("cfg", range(len(qtts.TILE_SHAPES)))
def test_gemv_every_tile_config(ctx, cfg, monkeypatch):
    """Each tile shape (QTTS_TILE_GEMV override) on ragged shapes: k not a
    multiple of the slice height, n not a multiple of 32, k % 4 != 0; one
    row (NB 1) and three rows (NB 2 + NB 1)."""
    monkeypatch.setenv("QTTS_TILE_GEMV", str(cfg))
    rng = np.random.Generator(np.random.PCG64(1000 + cfg))
    for k, n in ((3072, 1000), (2048, 4096), (100, 96)):
        w = synth.q4_random(rng, k, n)
        X = rng.standard_normal((3, k)).astype(np.float32)
        dw = ctx.upload(w)
        y = ctx.gemv(dw, X[0])
        Y = ctx.gemm(dw, X)
        dw.free()
        R = O.gemm(X, w)
        ok, e = close(y, R[0])
        assert ok, f"cfg {cfg} {qtts.TILE_SHAPES[cfg]} k={k} n={n} gemv rel err {e}"
        for r in range(3):
            ok, e = close(Y[r], R[r])
            assert ok, f"cfg {cfg} k={k} n={n} gemm row {r} rel err {e}"


def test_gemm_rows(ctx):
    rng = np.random.Generator(np.random.PCG64(3))
    w = synth.q4_random(rng, 2048, 3072)
    X = rng.standard_normal((5, 2048)).astype(np.float32)
    dw = ctx.upload(w)
    Y = ctx.gemm(dw, X)
    dw.free()
    R = O.gemm(X, w)
    for r in range(5):
        ok, e = close(Y[r], R[r])
        assert ok, f"row {r} rel err {e}"


def test_embed_lookup_exact(ctx):
    rng = np.random.Generator(np.random.PCG64(4))
    w = synth.q4_random(rng, 3072, 2048)
    dw = ctx.upload(w)
    for row in (0, 1, 2150, 3071):
        assert np.array_equal(bits(ctx.embed_lookup(dw, row)), bits(O.embed_lookup(w, row)))
    dw.free()


# ---- model level ----------------------------------------------------------

def test_kv_load_gather_bit_exact(loaded):
    ctx, om, t, p = loaded
    rng = np.random.Generator(np.random.PCG64(5))
    L = 200
    K = rng.standard_normal((len(t.layers), L, 8, 128)).astype(np.float32)
    V = rng.standard_normal((len(t.layers), L, 8, 128)).astype(np.float32)
    ctx.kv_load(K, V)
    assert ctx.kv_len() == L
    for l in range(len(t.layers)):
        k, v = ctx.kv_gather(l)
        assert np.array_equal(bits(k), bits(K[l])) and np.array_equal(bits(v), bits(V[l]))
    ctx.kv_reset()
    assert ctx.kv_len() == 0


def test_talker_step_kv512(loaded):
    # 1.7B layer shapes on a 2-layer talker: KV prefilled N(0,1) to 512, append one, attend 513
    ctx, om, t, p = loaded
    rng = np.random.Generator(np.random.PCG64(6))
    L = 512
    K = rng.standard_normal((len(t.layers), L, 8, 128)).astype(np.float32)
    V = rng.standard_normal((len(t.layers), L, 8, 128)).astype(np.float32)
    ctx.kv_load(K, V)
    om.kv_load(K, V)
    emb = rng.standard_normal(t.hidden).astype(np.float32)
    out = ctx.forward_with_embedding(emb, L)
    ref = om.forward_with_embedding(emb, L)
    ok_h, eh = close(out[: t.hidden], ref[: t.hidden])
    ok_l, el = close(out[t.hidden:], ref[t.hidden:])
    assert ok_h and ok_l, f"hidden {eh} logits {el}"
    assert ctx.kv_len() == L + 1
    for l in range(len(t.layers)):
        k, v = ctx.kv_gather(l)
        ko, vo = om.kv_layer(l)
        assert np.array_equal(bits(k[:L]), bits(K[l])) and np.array_equal(bits(v[:L]), bits(V[l]))
        assert close(k[L], ko[L])[0] and close(v[L], vo[L])[0]
    ctx.kv_reset()
    om.kv_reset()


def test_prefill_then_steps(loaded):
    ctx, om, t, p = loaded
    rng = np.random.Generator(np.random.PCG64(7))
    X = rng.standard_normal((70, t.hidden)).astype(np.float32)
    ctx.kv_reset()
    om.kv_reset()
    h = ctx.prefill_talker_raw_from(X, 0)
    hr = om.prefill(X, 0)
    ok, e = close(h, hr)
    assert ok, f"prefill rel err {e}"
    for step in range(3):
        emb = rng.standard_normal(t.hidden).astype(np.float32)
        out = ctx.forward_with_embedding(emb, 70 + step)
        ref = om.forward_with_embedding(emb, 70 + step)
        ok, e = close(out, ref)
        assert ok, f"step {step} rel err {e}"
    ctx.kv_reset()
    om.kv_reset()


def test_forward_talker_decode_legacy(loaded):
    """Legacy forward_talker_decode (talker.rs:161-258): token embedded on the
    device, then one step; bit-identical to a step on the embedding API's
    row, within the bar of the oracle."""
    ctx, om, t, p = loaded
    rng = np.random.Generator(np.random.PCG64(71))
    X = rng.standard_normal((20, t.hidden)).astype(np.float32)
    ctx.kv_reset()
    om.kv_reset()
    ctx.prefill_talker_raw_from(X, 0)
    om.prefill(X, 0)
    for pos, (tok, is_text) in enumerate(((2149, False), (300, True), (17, False)), start=20):
        h = ctx.forward_talker_decode(tok, is_text, pos)
        emb = om.embed_text_token(tok) if is_text else om.embed_codec_token(tok)
        ok, e = close(h, om.forward_with_embedding(emb, pos)[: t.hidden])
        assert ok, f"token {tok}: rel err {e}"
        ctx.kv_truncate(pos)
        dev_emb = ctx.embed_text_token(tok) if is_text else ctx.embed_codec_token(tok)
        h2 = ctx.forward_with_embedding(dev_emb, pos)[: t.hidden]
        assert np.array_equal(bits(h), bits(h2))
    ctx.kv_reset()
    om.kv_reset()


def test_text_and_codec_embeddings(loaded):
    ctx, om, t, p = loaded
    for tok in (0, 7, 511):
        ok, e = close(ctx.embed_text_token(tok), om.embed_text_token(tok))
        assert ok, f"text token {tok} rel err {e}"
    for tok in (0, 2150, 3071):
        assert np.array_equal(bits(ctx.embed_codec_token(tok)), bits(om.embed_codec_token(tok)))


def test_codec_head(loaded):
    ctx, om, t, p = loaded
    h = np.random.Generator(np.random.PCG64(8)).standard_normal(t.hidden).astype(np.float32)
    ok, e = close(ctx.apply_codec_head(h), om.codec_head(h))
    assert ok, f"rel err {e}"


def test_predictor_chain_codes(loaded):
    # predictor chain: 5 layers, 15 codebooks, KV 2 -> 16, greedy argmax
    ctx, om, t, p = loaded
    agree = total = 0
    for seed in range(4):
        rng = np.random.Generator(np.random.PCG64(100 + seed))
        th = rng.standard_normal(t.hidden).astype(np.float32)
        sem = om.embed_codec_token(int(rng.integers(0, 2048)))
        got = ctx.generate_acoustic_codes(th, sem)
        ref = om.predictor_chain(th, sem)
        if seed == 0:
            assert np.array_equal(got, ref), f"{got} vs {ref}"
        agree += int((got == ref).sum())
        total += ref.size
    assert agree >= 0.99 * total


def test_acoustic_embed_sum_exact(loaded):
    ctx, om, t, p = loaded
    codes = np.random.Generator(np.random.PCG64(9)).integers(0, 2048, 15).astype(np.uint32)
    assert np.array_equal(bits(ctx.get_acoustic_embeddings_sum(codes)), bits(om.acoustic_embed_sum(codes)))


@pytest.mark.parametrize("top_k,top_p,temp,rep", [(50, 1.0, 0.9, 1.05), (1, 1.0, 0.9, 1.05), (0, 0.8, 1.0, 1.0),
                                                  (50, 0.9, 0.7, 1.2)])
def test_sampler_matches_oracle(ctx, top_k, top_p, temp, rep):
    rng = np.random.Generator(np.random.PCG64(10))
    params = qtts.sample_params(temperature=temp, top_k=top_k, top_p=top_p, repetition_penalty=rep)
    mismatch = 0
    s_gpu = s_cpu = 42
    for i in range(60):
        lg = (rng.standard_normal(3072) * 3).astype(np.float32)
        prev = rng.integers(0, 3072, 16).astype(np.uint32)
        prev[:4] = 0
        a, s_gpu = ctx.sample_token(lg, params, prev, s_gpu, temp)
        b, s_cpu = O.sample_token(lg, params, prev, s_cpu, temp)
        assert s_gpu == s_cpu
        mismatch += a != b
    assert mismatch <= 1


@pytest.mark.parametrize("n,top_k,top_p,temp,rep,n_prev,ties", [
    (37, 5, 1.0, 0.9, 1.05, 16, False),       # ragged n: one thread holds a partial range
    (4096, 4095, 1.0, 0.8, 1.3, 16, False),   # the largest n, top-k of all but one
    (3072, 50, 1.0, 0.9, 1.2, 1000, False),   # long history, many repeats per token
    (3072, 20, 0.9, 1.0, 1.0, 0, True),       # heavy ties: 8 distinct logits
    (3072, 1, 1.0, 0.9, 1.05, 16, True),      # greedy among ties: the lowest index
    (1000, 0, 1.0, 0.0, 1.05, 16, False),     # T <= 0 is softmax at T = 1, no top-k
])
def test_sampler_edges_match_oracle(ctx, n, top_k, top_p, temp, rep, n_prev, ties):
    """The sampler on the edges of its layout (entries per thread, the
    radix select's ties and early exit, the history count) against the
    oracle; selections are exact, a draw may differ where the CDF's float
    rounding differs (expf bits), at most once per 20 draws."""
    rng = np.random.Generator(np.random.PCG64(1000 + n + top_k))
    params = qtts.sample_params(temperature=temp, top_k=top_k, top_p=top_p, repetition_penalty=rep)
    mismatch = 0
    s_gpu = s_cpu = 7
    for i in range(20):
        if ties:
            lg = (rng.integers(0, 8, n) * 0.5).astype(np.float32)
        else:
            lg = (rng.standard_normal(n) * 3).astype(np.float32)
        prev = rng.integers(0, min(n, 64) if n_prev > 16 else n, n_prev).astype(np.uint32)
        a, s_gpu = ctx.sample_token(lg, params, prev, s_gpu, temp)
        b, s_cpu = O.sample_token(lg, params, prev, s_cpu, temp)
        assert s_gpu == s_cpu
        mismatch += a != b
    assert mismatch <= (0 if top_k == 1 else 1)


def test_frames_teacher_forced_greedy(loaded):
    """200 greedy frames (top_k 1), each fed the oracle's previous codes;
    >= 99% of the 16 x 200 codes agree."""
    ctx, om, t, p = loaded
    n_frames = 200
    params = qtts.sample_params(top_k=1, eos_enabled=False)
    rng = np.random.Generator(np.random.PCG64(11))
    X = rng.standard_normal((16, t.hidden)).astype(np.float32)
    ctx.kv_reset()
    om.kv_reset()
    hid = om.prefill(X, 0)
    ctx.prefill_talker_raw_from(X, 0)
    logits = om.codec_head(hid)
    pad = om.embed_text_token(3)
    ctx.gen_set_text(None, pad)
    om.gen_begin(logits, hid, 16, 42)
    ctx.gen_begin(logits, hid, 16, 42, params)
    ref = np.stack([om.frame(params, pad)[0] for _ in range(n_frames)])
    pred = ctx.gen_frames_forced(ref)
    agree = (pred == ref).mean()
    assert agree >= 0.99, f"agreement {agree:.4f}"
    ctx.kv_reset()
    om.kv_reset()


def test_frames_free_running_sampled(loaded):
    """Default sampling (top-k 50, T 0.9, penalty 1.05, seed 42): free-running
    frames track the oracle; report the first divergence."""
    ctx, om, t, p = loaded
    params = qtts.sample_params(eos_enabled=False)
    rng = np.random.Generator(np.random.PCG64(12))
    X = rng.standard_normal((16, t.hidden)).astype(np.float32)
    ctx.kv_reset()
    om.kv_reset()
    hid = om.prefill(X, 0)
    ctx.prefill_talker_raw_from(X, 0)
    logits = om.codec_head(hid)
    pad = om.embed_text_token(3)
    ctx.gen_set_text(None, pad)
    om.gen_begin(logits, hid, 16, 42)
    ctx.gen_begin(logits, hid, 16, 42, params)
    n = 20
    ref = np.stack([om.frame(params, pad)[0] for _ in range(n)])
    got, eos = ctx.gen_frames(n)
    assert not eos and got.shape == (n, 16)
    same = np.all(got == ref, axis=1)
    first_div = int(np.argmin(same)) if not same.all() else n
    assert first_div >= 5, f"free-running frames diverge at frame {first_div}"
    ctx.kv_reset()
    om.kv_reset()


def test_predictor_row_tables_bit_identical(ctx_factory, small_model, monkeypatch):
    """Layer 0 of predictor steps 1..14 from the tables built at upload --
    the projected embedding rows, and their layer-0 q|k|v read inside the
    attention prologue -- carries the same bits as the per-step projection
    and q|k|v GEMVs: contexts with both tables, with the row tables only
    (QTTS_PRED_QKV_ROWS=0) and with neither (QTTS_PRED_ROWS=0) give identical
    chain codes, free-running and teacher-forced frames, and final
    logits/hidden."""
    t, p = small_model
    ctxs = []
    for env in ({}, {"QTTS_PRED_QKV_ROWS": "0"}, {"QTTS_PRED_ROWS": "0"}):
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        c = ctx_factory(256)
        c.upload_model(t, p)
        ctxs.append(c)
        for k in env:
            monkeypatch.delenv(k)
    rng = np.random.Generator(np.random.PCG64(81))
    for _ in range(3):
        th = rng.standard_normal(t.hidden).astype(np.float32)
        sem = ctxs[0].embed_codec_token(int(rng.integers(0, 3072)))
        ref = ctxs[2].generate_acoustic_codes(th, sem)
        for c in ctxs[:2]:
            assert np.array_equal(c.generate_acoustic_codes(th, sem), ref)
    X = rng.standard_normal((16, t.hidden)).astype(np.float32)
    params = qtts.sample_params(eos_enabled=False)
    outs = []
    for c in ctxs:
        h = c.prefill_talker_raw_from(X, 0)
        c.gen_set_text(None, c.embed_text_token(3))
        c.gen_begin(c.apply_codec_head(h), h, 16, 42, params)
        codes, _ = c.gen_frames(24)
        lg, hd, pos, rng_state = c.gen_state()
        c.kv_truncate(16)
        c.gen_begin(c.apply_codec_head(h), h, 16, 42, params)
        forced = c.gen_frames_forced(codes[::-1].copy())
        outs.append((codes, forced, lg, hd, pos, rng_state))
    for o in outs[:2]:
        assert np.array_equal(o[0], outs[2][0]) and np.array_equal(o[1], outs[2][1])
        assert np.array_equal(bits(o[2]), bits(outs[2][2])) and np.array_equal(bits(o[3]), bits(outs[2][3]))
        assert o[4:] == outs[2][4:]
    for c in ctxs:
        c.close()


@pytest.mark.parametrize("tiles", [{"TGU": "14", "PGU": "16"}, {"TGU": "11", "PGU": "12", "PO": "11"},
                                   {"TQKV": "3", "TDOWN": "12", "PQKV": "2", "PDOWN": "3"},
                                   {"TQKV": "9", "HEAD": "7", "PQKV": "7"},
                                   {"PGU": "14", "PDOWN": "15"}, {"PGU": "15", "PDOWN": "15"},
                                   {"TGU": "15", "TDOWN": "15"}, {"PHEAD": "12", "HEAD": "0"}])
def test_alternative_tiles_step_and_chain(ctx_factory, small_model, tiles, monkeypatch):
    """Other tile shapes per role (QTTS_TILE_<ROLE>): split-K gate|up with the
    SwiGLU prologue in the down projection, the unfused predictor attention,
    multi-slice q|k|v, the RMSNorm prologue's register rows on two- and
    four-group tiles, the predictor's gate|up + down launch on paired
    gate|up tiles (SwiGLU in their epilogue) and on 512-thread one-group
    tiles, and the talker's on one-group tiles; two-slice predictor heads
    (argmax over the summed partials instead of per-tile candidates) and an
    eight-slice codec head (the step end's loop past its four unrolled
    slices); a talker step at KV 100 and the predictor codes match the
    oracle."""
    for role, cfg in tiles.items():
        monkeypatch.setenv(f"QTTS_TILE_{role}", cfg)
    t, p = small_model
    c = ctx_factory(1024)
    c.upload_model(t, p)
    om = O.Model(t, p, kv_cap=1024)
    rng = np.random.Generator(np.random.PCG64(21))
    K = rng.standard_normal((len(t.layers), 100, 8, 128)).astype(np.float32)
    V = rng.standard_normal((len(t.layers), 100, 8, 128)).astype(np.float32)
    c.kv_load(K, V)
    om.kv_load(K, V)
    emb = rng.standard_normal(t.hidden).astype(np.float32)
    ok, e = close(c.forward_with_embedding(emb, 100), om.forward_with_embedding(emb, 100))
    assert ok, f"{tiles}: talker step rel err {e}"
    th = rng.standard_normal(t.hidden).astype(np.float32)
    sem = om.embed_codec_token(77)
    got, ref = c.generate_acoustic_codes(th, sem), om.predictor_chain(th, sem)
    assert (got == ref).mean() >= 14 / 15, f"{tiles}: codes {got} vs {ref}"
    om.close()
    c.close()


def test_onset_temperature_schedule(loaded):
    """frame_temperature (generate_new.rs:82-88): frames 0..2 sample at the
    onset temperature 0.3, later frames at 0.9.  Eight teacher-forced frames
    in two calls (2 + 6, the boundary inside the onset window) sample the
    oracle's code 0 draw for draw, so the frame count carries across calls;
    the same seed without the onset samples other codes (the test can tell
    the schedule from its absence)."""
    ctx, om, t, p = loaded
    params = qtts.sample_params(eos_enabled=False, onset_frames=3, onset_temperature=0.3)
    plain = qtts.sample_params(eos_enabled=False)
    rng = np.random.Generator(np.random.PCG64(13))
    X = rng.standard_normal((16, t.hidden)).astype(np.float32)
    ctx.kv_reset()
    om.kv_reset()
    hid = om.prefill(X, 0)
    ctx.prefill_talker_raw_from(X, 0)
    logits = om.codec_head(hid)
    pad = om.embed_text_token(3)
    ctx.gen_set_text(None, pad)

    def oracle_frames(prm, n=8):
        om.kv_reset()
        om.prefill(X, 0)
        om.gen_begin(logits, hid, 16, 42)
        return np.stack([om.frame(prm, pad)[0] for _ in range(n)])

    ref_plain = oracle_frames(plain)
    ref = oracle_frames(params)
    assert not np.array_equal(ref[:3, 0], ref_plain[:3, 0])
    ctx.gen_begin(logits, hid, 16, 42, params)
    pred = np.concatenate([ctx.gen_frames_forced(ref[:2]), ctx.gen_frames_forced(ref[2:])])
    assert np.array_equal(pred[:, 0], ref[:, 0]), f"code 0: {pred[:, 0]} vs {ref[:, 0]}"
    assert (pred[:, 1:] == ref[:, 1:]).mean() >= 0.99
    # free-running, also split inside the onset window: the first frames
    # match the oracle's onset run
    ctx.kv_truncate(16)
    ctx.gen_begin(logits, hid, 16, 42, params)
    got = np.concatenate([ctx.gen_frames(2)[0], ctx.gen_frames(2)[0]])
    assert np.array_equal(got, ref[:4]), f"{got[:, 0]} vs {ref[:4, 0]}"
    ctx.kv_reset()
    om.kv_reset()
