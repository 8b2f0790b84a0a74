"""Python binding of libqtts_hip.so (include/qtts.h) for the MI355X decode path.

The functions mirror the reference crate's forward-call surface:

    gemv / gemm / embed_lookup        gemv.rs:149, 157, 165
    forward_with_embedding            talker.rs:263
    prefill_talker_raw_from           talker.rs:379
    apply_codec_head                  talker.rs:647
    embed_text_token / codec_token    talker.rs:105, 152
    generate_acoustic_codes           code_predictor.rs:218
    get_acoustic_embeddings_sum       code_predictor.rs:287
    sample_token                      generate_new.rs:771
    frame loop                        generate_new.rs:606-675

Every call goes through the C ABI; there is no CPU fallback.  A missing or
unloadable library raises QttsError.
"""
import ctypes
import os
from ctypes import POINTER, byref, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_uint32, c_uint64, c_void_p

import numpy as np

from . import hostdesc
from .hostdesc import DecoderHost, PredictorHost, Q4Host, SampleParams, TalkerHost, decoder_host, ptr, sample_params


class RopeTables(ctypes.Structure):
    """qtts_rope_tables (include/qtts.h)."""
    _fields_ = [("talker_cos", c_void_p), ("talker_sin", c_void_p), ("talker_max_pos", c_int64),
                ("pred_cos", c_void_p), ("pred_sin", c_void_p), ("pred_max_pos", c_int64)]


PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "libqtts_hip.so")

# GEMV tile shapes (T threads, GB 32-column groups, R rows per thread), indexed
# by the TileCfg value that QTTS_TILE_<ROLE> environment overrides take
# (csrc/qtts_device.h, tile_shape()).
TILE_SHAPES = [(256, 8, 8), (128, 8, 8), (64, 1, 8), (128, 1, 8), (256, 1, 8), (384, 1, 8), (768, 1, 8),
               (256, 2, 8), (512, 2, 8), (256, 4, 8), (512, 1, 8), (256, 1, 4), (256, 1, 2), (512, 1, 4),
               (512, 2, 4), (512, 1, 2), (256, 2, 4), (1024, 1, 2), (1024, 2, 4)]

OK, ERR_INVALID, ERR_HIP, ERR_OOM, ERR_CAPACITY, ERR_STATE, ERR_IO, ERR_NAN, ERR_UNSUPPORTED = 0, -1, -2, -3, -4, -5, -6, -7, -8
DEVICE_PTRS = 1
PATH_ROWWISE, PATH_MFMA = 2, 4
_PATH_FLAGS = {None: 0, "rowwise": PATH_ROWWISE, "mfma": PATH_MFMA}

# Exported symbols and their signatures (argtypes, restype), in header order.
SIGNATURES = {
    "qtts_ctx_create": ([c_int, c_int64, POINTER(c_void_p)], c_int),
    "qtts_ctx_destroy": ([c_void_p], None),
    "qtts_last_error": ([c_void_p], c_char_p),
    "qtts_sync": ([c_void_p], c_int),
    "qtts_stream": ([c_void_p], c_void_p),
    "qtts_q4_upload": ([c_void_p, POINTER(Q4Host), POINTER(c_void_p)], c_int),
    "qtts_q4_free": ([c_void_p, c_void_p], c_int),
    "qtts_gemv_q4": ([c_void_p, c_void_p, c_void_p, c_void_p, c_int], c_int),
    "qtts_gemm_q4": ([c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int], c_int),
    "qtts_gemm_q4_noalloc": ([c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int], c_int),
    "qtts_embed_lookup_q4": ([c_void_p, c_void_p, c_int64, c_void_p, c_int], c_int),
    "qtts_model_upload": ([c_void_p, POINTER(TalkerHost), POINTER(PredictorHost)], c_int),
    "qtts_model_load_qtts": ([c_void_p, c_char_p], c_int),
    "qtts_model_load_qora_q4": ([c_void_p, c_char_p, c_void_p], c_int),
    "qtts_model_dims": ([c_void_p] + [POINTER(c_int32)] * 6, c_int),
    "qtts_talker_step": ([c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_int], c_int),
    "qtts_talker_decode_token": ([c_void_p, c_uint32, c_int, c_int64, c_void_p, c_int], c_int),
    "qtts_talker_prefill": ([c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int], c_int),
    "qtts_codec_head": ([c_void_p, c_void_p, c_void_p, c_int], c_int),
    "qtts_embed_text_token": ([c_void_p, c_uint32, c_void_p, c_int], c_int),
    "qtts_embed_codec_token": ([c_void_p, c_uint32, c_void_p, c_int], c_int),
    "qtts_kv_reset": ([c_void_p], c_int),
    "qtts_kv_len": ([c_void_p, POINTER(c_int64)], c_int),
    "qtts_kv_gather": ([c_void_p, c_int32, c_void_p, c_void_p], c_int),
    "qtts_kv_load": ([c_void_p, c_void_p, c_void_p, c_int64], c_int),
    "qtts_kv_truncate": ([c_void_p, c_int64], c_int),
    "qtts_prefix_capture": ([c_void_p, POINTER(c_void_p)], c_int),
    "qtts_prefix_attach": ([c_void_p, c_void_p], c_int),
    "qtts_prefix_len": ([c_void_p, POINTER(c_int64)], c_int),
    "qtts_prefix_free": ([c_void_p, c_void_p], c_int),
    "qtts_prefix_suffix_split": ([c_int64, c_int64, c_int64, POINTER(c_int64)], c_int),
    "qtts_icl_layout": ([c_int64, c_int64, c_int64, POINTER(c_int64), POINTER(c_int64)], c_int),
    "qtts_embed_text_tokens": ([c_void_p, c_void_p, c_int64, c_void_p, c_int], c_int),
    "qtts_build_icl_block": ([c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                              c_void_p, c_int], c_int),
    "qtts_build_prefill_head": ([c_void_p, c_uint32, c_uint32, c_void_p, c_int64, c_void_p, c_int], c_int),
    "qtts_build_icl_prefix": ([c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int], c_int),
    "qtts_build_trailing_text": ([c_void_p, c_void_p, c_int64, c_void_p, c_int], c_int),
    "qtts_prefill_custom_voice": ([c_void_p, c_void_p, c_int64, c_uint32, c_uint32, c_void_p, c_int64, c_void_p,
                                   c_int64, c_void_p, c_void_p, POINTER(c_int64), c_int], c_int),
    "qtts_decoder_upload": ([c_void_p, POINTER(DecoderHost)], c_int),
    "qtts_decoder_dims": ([c_void_p, POINTER(c_int32), POINTER(c_int32), POINTER(c_int64)], c_int),
    "qtts_decode_to_audio": ([c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, POINTER(c_int64),
                              c_int], c_int),
    "qtts_predictor_chain": ([c_void_p, c_void_p, c_void_p, c_void_p, c_int], c_int),
    "qtts_acoustic_embed_sum": ([c_void_p, c_void_p, c_void_p, c_int], c_int),
    "qtts_sample_token": ([c_void_p, c_void_p, c_int64, POINTER(SampleParams), c_void_p, c_int64,
                           POINTER(c_uint64), c_float, POINTER(c_uint32)], c_int),
    "qtts_prefill_tokens": ([c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int], c_int),
    "qtts_predict_codes": ([c_void_p, c_void_p, c_void_p, c_int], c_int),
    "qtts_predict_codes_reset": ([c_void_p], c_int),
    "qtts_sample_top_k": ([c_void_p, c_void_p, c_int64, c_float, c_int32, c_void_p, c_int64, c_float,
                           POINTER(c_uint64), POINTER(c_uint32)], c_int),
    "qtts_gen_begin": ([c_void_p, c_void_p, c_void_p, c_int64, c_uint64, POINTER(SampleParams)], c_int),
    "qtts_gen_set_text": ([c_void_p, c_void_p, c_int64, c_void_p], c_int),
    "qtts_gen_frames": ([c_void_p, c_int64, c_void_p, POINTER(c_int64), POINTER(c_int32)], c_int),
    "qtts_gen_frames_forced": ([c_void_p, c_int64, c_void_p, c_void_p], c_int),
    "qtts_gen_state": ([c_void_p, c_void_p, c_void_p, POINTER(c_int64), POINTER(c_uint64)], c_int),
    "qtts_debug_force_sync_err": ([c_void_p], c_int),
    "qtts_time_kernel": ([c_void_p, c_int32, c_int32, POINTER(c_double), POINTER(c_double)], c_int),
    "qtts_device_bytes": ([c_void_p, c_void_p], c_int),
    "qtts_time_graph": ([c_void_p, c_int32], c_int),
    "qtts_time_gemv": ([c_void_p, POINTER(c_void_p), c_int32, c_int32, POINTER(c_double), POINTER(c_double)], c_int),
    "qtts_time_prefill": ([c_void_p, c_int64, c_int32, c_int32, POINTER(c_double), POINTER(c_double)], c_int),
    "qtts_time_decode": ([c_void_p, c_int64, c_int32, POINTER(c_double), POINTER(c_double)], c_int),
}


class QttsError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"qtts error {code}: {msg}")
        self.code = code


_lib = None


def load_library(path=None):
    """Load libqtts_hip.so (built by __graft_entry__.build()).  Raises
    QttsError when it is missing: the device path has no fallback."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or os.environ.get("QTTS_LIB", LIB_PATH)
    if not os.path.exists(p):
        raise QttsError(ERR_STATE, f"{p} not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(p)
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    if path is None:
        _lib = lib
    return lib


def _f32(a, n=None):
    a = np.ascontiguousarray(a, dtype=np.float32)
    if n is not None and a.size != n:
        raise ValueError(f"expected {n} floats, got {a.size}")
    return a


class Weight:
    """A Q4 weight uploaded for the operator-level calls."""

    def __init__(self, ctx, w):
        self.ctx, self.k, self.n = ctx, w.k, w.n
        self._src = w
        h = c_void_p()
        ctx._check(ctx.lib.qtts_q4_upload(ctx.h, byref(hostdesc.q4_host(w)), byref(h)))
        self.h = h

    def free(self):
        if self.h:
            self.ctx.lib.qtts_q4_free(self.ctx.h, self.h)
            self.h = None


class Context:
    """One device context (qtts_ctx): model, paged talker KV cache, stream."""

    def __init__(self, device=0, kv_capacity=0, lib=None):
        self.lib = lib or load_library()
        h = c_void_p()
        rc = self.lib.qtts_ctx_create(device, kv_capacity, byref(h))
        if rc != OK:
            raise QttsError(rc, "qtts_ctx_create failed (no HIP device?)")
        self.h = h
        self._keep = []
        self.dec_codebooks = 16

    def close(self):
        if self.h:
            self.lib.qtts_ctx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _check(self, rc):
        if rc != OK:
            raise QttsError(rc, (self.lib.qtts_last_error(self.h) or b"").decode())
        return rc

    # ---- operator level -------------------------------------------------
    def upload(self, w):
        return Weight(self, w)

    def gemv(self, w, x):
        """`gemv` (gemv.rs:149) for an uploaded weight."""
        x = _f32(x, w.k)
        y = np.empty(w.n, np.float32)
        self._check(self.lib.qtts_gemv_q4(self.h, w.h, ptr(x), ptr(y), 0))
        return y

    def gemm(self, w, X, path=None):
        """`gemm` (gemv.rs:157): rows of X times W.  path: None (by row
        count), "rowwise" (GEMV per row) or "mfma" (matrix cores)."""
        X = _f32(X).reshape(-1, w.k)
        Y = np.empty((X.shape[0], w.n), np.float32)
        self._check(self.lib.qtts_gemm_q4(self.h, w.h, ptr(X), X.shape[0], ptr(Y), _PATH_FLAGS[path]))
        return Y

    def gemm_noalloc(self, w, X_dev, rows, Y_dev, path=None):
        """`gemm` on device addresses X_dev [rows][k] and Y_dev [rows][n]
        with nothing allocated (qtts_gemm_q4_noalloc); enqueues only, call
        sync() before reading Y."""
        self._check(self.lib.qtts_gemm_q4_noalloc(self.h, w.h, c_void_p(X_dev), rows, c_void_p(Y_dev),
                                                  _PATH_FLAGS[path]))

    def sync(self):
        self._check(self.lib.qtts_sync(self.h))

    def embed_lookup(self, w, row):
        """`embed_lookup_q4` (gemv.rs:415)."""
        out = np.empty(w.n, np.float32)
        self._check(self.lib.qtts_embed_lookup_q4(self.h, w.h, row, ptr(out), 0))
        return out

    # ---- model -----------------------------------------------------------
    def upload_model(self, talker, predictor):
        th, keep_t = hostdesc.talker_host(talker)
        ph, keep_p = hostdesc.predictor_host(predictor)
        self._check(self.lib.qtts_model_upload(self.h, byref(th), byref(ph)))
        self.dims()

    def load_qtts(self, path):
        self._check(self.lib.qtts_model_load_qtts(self.h, os.fsencode(path)))
        if self.has_decoder():
            self.dec_codebooks = self.decoder_dims()[0]
        self.dims()

    def load_qora_q4(self, path, talker_rope, pred_rope):
        """The older "QORA-TTS-Q4" container (loader.rs:724-882); the RoPE
        tables come from the caller as (cos, sin) pairs [max_pos][head_dim/2]."""
        tc, ts = (np.ascontiguousarray(a, np.float32) for a in talker_rope)
        pc, ps = (np.ascontiguousarray(a, np.float32) for a in pred_rope)
        rt = RopeTables(tc.ctypes.data, ts.ctypes.data, tc.shape[0], pc.ctypes.data, ps.ctypes.data, pc.shape[0])
        self._check(self.lib.qtts_model_load_qora_q4(self.h, os.fsencode(path), byref(rt)))
        self.dims()

    def dims(self):
        v = [c_int32() for _ in range(6)]
        self._check(self.lib.qtts_model_dims(self.h, *[byref(x) for x in v]))
        (self.hidden, self.vocab, self.n_layers, self.p_hidden, self.p_vocab, self.n_groups) = [x.value for x in v]
        return self.hidden, self.vocab, self.n_layers, self.p_hidden, self.p_vocab, self.n_groups

    def forward_with_embedding(self, embedding, position):
        """`forward_with_embedding` (talker.rs:263-360): [hidden | logits]."""
        e = _f32(embedding, self.hidden)
        hid = np.empty(self.hidden, np.float32)
        lg = np.empty(self.vocab, np.float32)
        self._check(self.lib.qtts_talker_step(self.h, ptr(e), position, ptr(hid), ptr(lg), 0))
        return np.concatenate([hid, lg])

    def forward_talker_decode(self, token, is_text, position):
        """Legacy `forward_talker_decode` (talker.rs:161-258): final-normed hidden."""
        hid = np.empty(self.hidden, np.float32)
        self._check(self.lib.qtts_talker_decode_token(self.h, token, 1 if is_text else 0, position, ptr(hid), 0))
        return hid

    def prefill_talker_raw_from(self, X, start_pos, path=None):
        """`prefill_talker_raw_from` (talker.rs:379-482): last row's normed
        hidden.  path as for gemm()."""
        X = _f32(X).reshape(-1, self.hidden)
        out = np.empty(self.hidden, np.float32)
        self._check(self.lib.qtts_talker_prefill(self.h, ptr(X), X.shape[0], start_pos, ptr(out),
                                                 _PATH_FLAGS[path]))
        return out

    def apply_codec_head(self, hidden):
        h = _f32(hidden, self.hidden)
        out = np.empty(self.vocab, np.float32)
        self._check(self.lib.qtts_codec_head(self.h, ptr(h), ptr(out), 0))
        return out

    def embed_text_token(self, token):
        out = np.empty(self.hidden, np.float32)
        self._check(self.lib.qtts_embed_text_token(self.h, token, ptr(out), 0))
        return out

    def embed_codec_token(self, token):
        out = np.empty(self.hidden, np.float32)
        self._check(self.lib.qtts_embed_codec_token(self.h, token, ptr(out), 0))
        return out

    # ---- KV -----------------------------------------------------------------
    def kv_reset(self):
        self._check(self.lib.qtts_kv_reset(self.h))

    def kv_len(self):
        n = c_int64()
        self._check(self.lib.qtts_kv_len(self.h, byref(n)))
        return n.value

    def kv_gather(self, layer):
        n = self.kv_len()
        K = np.empty((n, 8, 128), np.float32)
        V = np.empty((n, 8, 128), np.float32)
        self._check(self.lib.qtts_kv_gather(self.h, layer, ptr(K), ptr(V)))
        return K, V

    def kv_load(self, K, V):
        """K, V: [n_layers][len][8][128] f32."""
        K = _f32(K)
        V = _f32(V)
        self._check(self.lib.qtts_kv_load(self.h, ptr(K), ptr(V), K.shape[1]))

    def kv_truncate(self, n):
        self._check(self.lib.qtts_kv_truncate(self.h, n))

    # ---- predictor / sampler -----------------------------------------------
    # ---- prefix cache --------------------------------------------------------
    def prefix_capture(self):
        """Keep the cached positions as a prefix (TalkerPrefixCache,
        generate_new.rs:317-355)."""
        h = c_void_p()
        self._check(self.lib.qtts_prefix_capture(self.h, byref(h)))
        return Prefix(self, h)

    def prefix_attach(self, prefix):
        """Start the cache from a kept prefix (pfx.kv.clone(), generate_new.rs:541)."""
        self._check(self.lib.qtts_prefix_attach(self.h, prefix.h))

    # ---- prompt construction ------------------------------------------------
    def embed_text_tokens(self, ids):
        """embed_text_token (talker.rs:105-116) over a batch of ids."""
        ids = np.ascontiguousarray(ids, np.uint32).reshape(-1)
        out = np.empty((ids.size, self.hidden), np.float32)
        self._check(self.lib.qtts_embed_text_tokens(self.h, ptr(ids), ids.size, ptr(out), 0))
        return out

    def build_icl_block(self, ref_tokens, text_tokens, ref_codes):
        """build_icl_block (generate_new.rs:140-195): (icl rows, remainder rows).
        ref_codes is [16][n_frames]."""
        r = np.ascontiguousarray(ref_tokens, np.uint32).reshape(-1)
        t = np.ascontiguousarray(text_tokens, np.uint32).reshape(-1)
        codes = np.ascontiguousarray(ref_codes, np.uint32).reshape(16, -1)
        icl_len, rem_len = icl_layout(r.size, t.size, codes.shape[1], self.lib)
        icl = np.empty((icl_len, self.hidden), np.float32)
        rem = np.empty((rem_len, self.hidden), np.float32)
        self._check(self.lib.qtts_build_icl_block(self.h, ptr(r) if r.size else None, r.size,
                                                  ptr(t) if t.size else None, t.size, ptr(codes), codes.shape[1],
                                                  ptr(icl), ptr(rem) if rem_len else None, 0))
        return icl, rem

    def build_prefill_head(self, speaker_id, language_id, voice=None):
        """build_prefill_head (generate_new.rs:222-237): [9][hidden]."""
        v = None if voice is None else _f32(voice)
        out = np.empty((9, self.hidden), np.float32)
        self._check(self.lib.qtts_build_prefill_head(self.h, speaker_id, language_id, ptr(v) if v is not None else None,
                                                     0 if v is None else v.size, ptr(out), 0))
        return out

    def build_icl_prefix(self, ref_tokens, ref_codes):
        """build_icl_prefix (generate_new.rs:244-280): [len(ref_tokens)][hidden]."""
        r = np.ascontiguousarray(ref_tokens, np.uint32).reshape(-1)
        codes = np.ascontiguousarray(ref_codes, np.uint32).reshape(16, -1)
        out = np.empty((r.size, self.hidden), np.float32)
        self._check(self.lib.qtts_build_icl_prefix(self.h, ptr(r) if r.size else None, r.size, ptr(codes),
                                                   codes.shape[1], ptr(out), 0))
        return out

    def build_trailing_text(self, tokens):
        """build_trailing_text (generate_new.rs:756-767)."""
        t = np.ascontiguousarray(tokens, np.uint32).reshape(-1)
        out = np.empty((max(t.size - 1, 0) + 1, self.hidden), np.float32)
        self._check(self.lib.qtts_build_trailing_text(self.h, ptr(t) if t.size else None, t.size, ptr(out), 0))
        return out

    def prefill_custom_voice(self, text_tokens, speaker_id, language_id, voice=None, icl_rows=None, path=None):
        """prefill_custom_voice (generate_new.rs:361-476) from position 0:
        (hidden, logits, position)."""
        t = np.ascontiguousarray(text_tokens, np.uint32).reshape(-1)
        v = None if voice is None else _f32(voice)
        icl = None if icl_rows is None else _f32(icl_rows).reshape(-1, self.hidden)
        hid = np.empty(self.hidden, np.float32)
        lg = np.empty(self.vocab, np.float32)
        pos = c_int64()
        self._check(self.lib.qtts_prefill_custom_voice(
            self.h, ptr(t) if t.size else None, t.size, speaker_id, language_id, ptr(v) if v is not None else None,
            0 if v is None else v.size, ptr(icl) if icl is not None else None, 0 if icl is None else icl.shape[0],
            ptr(hid), ptr(lg), byref(pos), _PATH_FLAGS[path]))
        return hid, lg, pos.value

    # ---- speech decoder -----------------------------------------------------
    def upload_decoder(self, decoder):
        """Upload a SpeechDecoderWeights-shaped decoder (synth.Decoder)."""
        h, keep = decoder_host(decoder)
        self._check(self.lib.qtts_decoder_upload(self.h, ctypes.byref(h)))
        self.dec_codebooks = len(decoder.rest_codebooks) + 1

    def decoder_dims(self):
        """(codebooks per frame, codes per codebook, samples per frame)."""
        n, cs, spf = c_int32(), c_int32(), c_int64()
        self._check(self.lib.qtts_decoder_dims(self.h, byref(n), byref(cs), byref(spf)))
        return n.value, cs.value, spf.value

    def has_decoder(self):
        n, cs, spf = c_int32(), c_int32(), c_int64()
        return self.lib.qtts_decoder_dims(self.h, byref(n), byref(cs), byref(spf)) == OK

    def decode_to_audio(self, codes, warmup=None):
        """decode_to_audio (decoder.rs:395-574): codes [n_codebooks][T],
        optional warmup codes [n_codebooks][Tv] prepended and trimmed."""
        c = np.ascontiguousarray(codes, np.uint32).reshape(self.dec_codebooks, -1)
        w = None if warmup is None else np.ascontiguousarray(warmup, np.uint32).reshape(self.dec_codebooks, -1)
        nw = 0 if w is None else w.shape[1]
        n = c_int64(0)
        rc = self.lib.qtts_decode_to_audio(self.h, ptr(c), c.shape[1], ptr(w) if nw else None, nw, None, 0,
                                           ctypes.byref(n), 0)
        if rc == OK:
            return np.empty(0, np.float32)
        if rc != ERR_CAPACITY:
            self._check(rc)
        out = np.empty(n.value, np.float32)
        self._check(self.lib.qtts_decode_to_audio(self.h, ptr(c), c.shape[1], ptr(w) if nw else None, nw, ptr(out),
                                                  out.size, ctypes.byref(n), 0))
        return out[:n.value]

    # ---- legacy loop (generate.rs) ----------------------------------------------
    def prefill_tokens(self, ids, is_text):
        """prefill_talker (talker.rs:487-508) over a fresh cache."""
        ids = np.ascontiguousarray(ids, np.uint32).reshape(-1)
        it = np.ascontiguousarray(is_text, np.uint8).reshape(-1)
        out = np.empty(self.hidden, np.float32)
        self._check(self.lib.qtts_prefill_tokens(self.h, ptr(ids), ptr(it), ids.size, ptr(out), 0))
        return out

    def predict_codes(self, talker_hidden):
        """predict_codes (code_predictor.rs:126-216): [n_groups][vocab] logits."""
        th = _f32(talker_hidden, self.hidden)
        out = np.empty((self.n_groups, self.p_vocab), np.float32)
        self._check(self.lib.qtts_predict_codes(self.h, ptr(th), ptr(out), 0))
        return out

    def predict_codes_reset(self):
        self._check(self.lib.qtts_predict_codes_reset(self.h))

    def sample_top_k(self, logits, temperature, top_k, prev, penalty, rng):
        """The legacy sampler (generate.rs:185-217): (token, rng)."""
        lg = _f32(logits)
        pv = np.ascontiguousarray(prev, np.uint32).reshape(-1)
        s, out = c_uint64(rng), c_uint32()
        self._check(self.lib.qtts_sample_top_k(self.h, ptr(lg), lg.size, temperature, top_k, ptr(pv) if pv.size else None,
                                               pv.size, penalty, byref(s), byref(out)))
        return out.value, s.value

    def generate_acoustic_codes(self, talker_hidden, semantic_embed):
        th = _f32(talker_hidden, self.hidden)
        se = _f32(semantic_embed, self.hidden)
        codes = np.empty(self.n_groups, np.uint32)
        self._check(self.lib.qtts_predictor_chain(self.h, ptr(th), ptr(se), ptr(codes), 0))
        return codes

    def get_acoustic_embeddings_sum(self, codes):
        c = np.ascontiguousarray(codes, dtype=np.uint32)
        out = np.empty(self.hidden, np.float32)
        self._check(self.lib.qtts_acoustic_embed_sum(self.h, ptr(c), ptr(out), 0))
        return out

    def sample_token(self, logits, params, prev_tokens, rng_state, temperature):
        """`sample_token` (generate_new.rs:771-862): returns (token, rng_state)."""
        lg = _f32(logits)
        prev = np.ascontiguousarray(prev_tokens, dtype=np.uint32)
        rng = c_uint64(rng_state)
        out = c_uint32()
        self._check(self.lib.qtts_sample_token(self.h, ptr(lg), lg.size, byref(params), ptr(prev) if prev.size else None,
                                               prev.size, byref(rng), temperature, byref(out)))
        return out.value, rng.value

    # ---- frame loop -----------------------------------------------------------
    def gen_begin(self, logits, hidden, position, seed, params):
        lg = _f32(logits, self.vocab)
        hd = _f32(hidden, self.hidden)
        self._check(self.lib.qtts_gen_begin(self.h, ptr(lg), ptr(hd), position, seed, byref(params)))

    def gen_set_text(self, text_rows, pad):
        t = None if text_rows is None or len(text_rows) == 0 else _f32(text_rows).reshape(-1, self.hidden)
        p = _f32(pad, self.hidden)
        self._check(self.lib.qtts_gen_set_text(self.h, ptr(t) if t is not None else None,
                                               0 if t is None else t.shape[0], ptr(p)))

    def gen_frames(self, max_frames):
        """Frames until EOS or max_frames: (codes [frames][16], eos)."""
        out = np.empty((max(max_frames, 1), 16), np.uint32)
        done, eos = c_int64(), c_int32()
        self._check(self.lib.qtts_gen_frames(self.h, max_frames, ptr(out), byref(done), byref(eos)))
        return out[: done.value].copy(), bool(eos.value)

    def gen_frames_forced(self, forced):
        f = np.ascontiguousarray(forced, dtype=np.uint32).reshape(-1, 16)
        pred = np.empty_like(f)
        self._check(self.lib.qtts_gen_frames_forced(self.h, f.shape[0], ptr(f), ptr(pred)))
        return pred

    def gen_state(self):
        lg = np.empty(self.vocab, np.float32)
        hd = np.empty(self.hidden, np.float32)
        pos, rng = c_int64(), c_uint64()
        self._check(self.lib.qtts_gen_state(self.h, ptr(lg), ptr(hd), byref(pos), byref(rng)))
        return lg, hd, pos.value, rng.value

    def debug_force_sync_err(self):
        """Leave the state of a cross-workgroup wait that ran out: the next
        step / frame batch / chain call returns QTTS_ERR_HIP once."""
        self._check(self.lib.qtts_debug_force_sync_err(self.h))

    # ---- measurement ----------------------------------------------------------
    MEM_FIELDS = ("talker_q4", "predictor_q4", "predictor_row_tables", "predictor_qkv_tables", "embedding_rows",
                  "kv_pool", "device_used")

    def device_bytes(self):
        """The device memory the uploaded model holds, bytes per part
        (qtts_mem_report)."""
        out = (c_int64 * len(self.MEM_FIELDS))()
        self._check(self.lib.qtts_device_bytes(self.h, out))
        return dict(zip(self.MEM_FIELDS, (int(v) for v in out)))

    def time_kernel(self, kind, iters):
        us, b = c_double(), c_double()
        self._check(self.lib.qtts_time_kernel(self.h, kind, iters, byref(us), byref(b)))
        return us.value, b.value

    def time_graph(self, on):
        """Timing calls launch from a replayed graph (True) or from the
        stream (False, the default)."""
        self._check(self.lib.qtts_time_graph(self.h, 1 if on else 0))

    def time_gemv(self, weights, iters):
        arr = (c_void_p * len(weights))(*[w.h for w in weights])
        us, b = c_double(), c_double()
        self._check(self.lib.qtts_time_gemv(self.h, arr, len(weights), iters, byref(us), byref(b)))
        return us.value, b.value

    def time_prefill(self, rows, what, iters):
        """(avg us, flops) of the matrix-core prefill over `rows` synthetic
        rows: what 0 the gate|up GEMM, 1 the whole prefill."""
        us, fl = c_double(), c_double()
        self._check(self.lib.qtts_time_prefill(self.h, rows, what, iters, byref(us), byref(fl)))
        return us.value, fl.value

    def time_decode(self, n_frames, iters):
        """(avg us, flops) of one device decode_to_audio over `n_frames`
        synthetic frames."""
        us, fl = c_double(), c_double()
        self._check(self.lib.qtts_time_decode(self.h, n_frames, iters, byref(us), byref(fl)))
        return us.value, fl.value


class Prefix:
    """A kept talker KV prefix (qtts_prefix); free() returns its pages."""

    def __init__(self, ctx, h):
        self.ctx, self.h = ctx, h
        n = c_int64()
        ctx._check(ctx.lib.qtts_prefix_len(h, byref(n)))
        self.len = n.value

    def free(self):
        if self.h:
            self.ctx._check(self.ctx.lib.qtts_prefix_free(self.ctx.h, self.h))
            self.h = None


def icl_layout(n_ref, n_text, n_frames, lib=None):
    """icl_block_layout (generate_new.rs:120-128): (icl_len, remainder_len)."""
    lib = lib or load_library()
    a, b = c_int64(), c_int64()
    rc = lib.qtts_icl_layout(n_ref, n_text, n_frames, byref(a), byref(b))
    if rc != OK:
        raise QttsError(rc, "invalid ICL layout arguments")
    return a.value, b.value


def prefix_suffix_split(block_len, n_ref, prefix_len, lib=None):
    """prefix_suffix_split (generate_new.rs:307-316): suffix length or None."""
    lib = lib or load_library()
    n = c_int64()
    rc = lib.qtts_prefix_suffix_split(block_len, n_ref, prefix_len, byref(n))
    if rc < 0:
        raise QttsError(rc, "invalid prefix split arguments")
    return n.value if rc == 1 else None


def header_symbols(header_path=None):
    """Function names declared in include/qtts.h."""
    import re
    hp = header_path or os.path.join(os.path.dirname(PKG_DIR), "include", "qtts.h")
    text = open(hp).read()
    return sorted(set(re.findall(r"\b(qtts_[a-z0-9_]+)\s*\(", text)))
