"""ctypes binding of the CPU oracle (oracle/liboqtts_oracle.so).

TEST INFRASTRUCTURE: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use this module.  It restates the reference's CPU decode
path (see qtts_oracle.c) and is the oracle the HIP path is tested
against, never part of it.
"""
import ctypes
import os
import subprocess
import sys
from ctypes import POINTER, byref, c_double, c_float, c_int, c_int32, c_int64, c_uint16, c_uint32, c_uint64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, os.path.join(ROOT, "qora-tts-12hz-1.7b_amd"))
from qtts import hostdesc  # noqa: E402  (descriptor structs only)
from qtts.hostdesc import (Conv1dHost, ConvT1dHost, DecoderHost, DwConvHost, LayerHost,  # noqa: E402
                           PredictorHost, Q4Host, SampleParams, TalkerHost, ptr)

LIB = os.path.join(HERE, "liboqtts_oracle.so")


class OqKv(ctypes.Structure):
    _fields_ = [("n_layers", c_int32), ("n_kv", c_int32), ("hd", c_int32), ("cap", c_int64),
                ("len", POINTER(c_int64)), ("K", POINTER(POINTER(c_float))), ("V", POINTER(POINTER(c_float)))]


class OqGen(ctypes.Structure):
    _fields_ = [("logits", c_void_p), ("hidden", c_void_p), ("prev", c_uint32 * 16), ("rng", c_uint64),
                ("position", c_int64), ("frame_idx", c_int64)]


_SIG = {
    "oq_f16_to_f32": ([c_uint16], c_float),
    "oq_f32_to_f16": ([c_float], c_uint16),
    "oq_xorshift": ([POINTER(c_uint64)], c_uint64),
    "oq_simple_rand": ([POINTER(c_uint64)], c_float),
    "oq_gemv_q4_scalar": ([c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p], None),
    "oq_gemv_q4_avx2": ([c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p], c_int),
    "oq_gemv_q4_avx512": ([c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p], c_int),
    "oq_set_isa": ([c_int], c_int),
    "oq_get_isa": ([], c_int),
    "oq_set_workers": ([c_int, c_int], None),
    "oq_get_workers": ([], c_int),
    "oq_gemv_q4": ([c_void_p, POINTER(Q4Host), c_void_p], None),
    "oq_gemm_q4": ([c_void_p, c_int64, POINTER(Q4Host), c_void_p], None),
    "oq_embed_lookup_q4": ([POINTER(Q4Host), c_int64, c_int64, c_void_p], None),
    "oq_quantize_q4": ([c_void_p, c_int64, c_int64, c_void_p, c_void_p], None),
    "oq_rms_norm_f16": ([c_void_p, c_void_p, c_int64, c_void_p], None),
    "oq_softmax_raw": ([c_void_p, c_int64], None),
    "oq_silu": ([c_float], c_float),
    "oq_qk_norm": ([c_void_p, c_int64, c_int64, c_void_p], None),
    "oq_rope_table": ([c_int64, c_int64, c_double, c_void_p, c_void_p], None),
    "oq_rope_apply": ([c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_int64], None),
    "oq_kv_new": ([c_int32, c_int32, c_int32, c_int64], POINTER(OqKv)),
    "oq_kv_free": ([POINTER(OqKv)], None),
    "oq_kv_reset": ([POINTER(OqKv)], None),
    "oq_kv_k": ([POINTER(OqKv), c_int32], POINTER(c_float)),
    "oq_kv_v": ([POINTER(OqKv), c_int32], POINTER(c_float)),
    "oq_kv_len": ([POINTER(OqKv), c_int32], c_int64),
    "oq_kv_set_len": ([POINTER(OqKv), c_int64], None),
    "oq_talker_step": ([POINTER(TalkerHost), c_void_p, POINTER(OqKv), c_int64, c_void_p], c_int),
    "oq_talker_prefill": ([POINTER(TalkerHost), c_void_p, c_int64, POINTER(OqKv), c_int64, c_void_p], c_int),
    "oq_codec_head": ([POINTER(TalkerHost), c_void_p, c_void_p], None),
    "oq_embed_text_token": ([POINTER(TalkerHost), c_uint32, c_void_p], None),
    "oq_embed_codec_token": ([POINTER(TalkerHost), c_uint32, c_void_p], None),
    "oq_predictor_chain": ([POINTER(PredictorHost), c_void_p, c_void_p, POINTER(OqKv), c_void_p, c_void_p], c_int),
    "oq_acoustic_embed_sum": ([POINTER(PredictorHost), c_void_p, c_int32, c_void_p], None),
    "oq_argmax_last": ([c_void_p, c_int64], c_uint32),
    "oq_sample_token": ([c_void_p, c_int64, POINTER(SampleParams), c_void_p, c_int64, POINTER(c_uint64), c_float,
                         POINTER(c_uint32)], c_int),
    "oq_predict_codes": ([POINTER(PredictorHost), c_void_p, POINTER(OqKv), c_void_p], c_int),
    "oq_sample_top_k": ([c_void_p, c_int64, c_float, c_int64, c_void_p, c_int64, c_float, POINTER(c_uint64),
                         POINTER(c_uint32)], c_int),
    "oq_frame": ([POINTER(TalkerHost), POINTER(PredictorHost), POINTER(OqKv), POINTER(OqKv), POINTER(OqGen),
                  POINTER(SampleParams), c_void_p, c_void_p, POINTER(c_int32), c_void_p], c_int),
    "oq_frame_temperature": ([POINTER(SampleParams), c_int64], c_float),
    "oq_build_prefill_head": ([POINTER(TalkerHost), c_uint32, c_uint32, c_void_p, c_int64, c_void_p], None),
    "oq_icl_layout": ([c_int64, c_int64, c_int64, POINTER(c_int64), POINTER(c_int64)], None),
    "oq_build_icl_block": ([POINTER(TalkerHost), POINTER(PredictorHost), c_void_p, c_int64, c_void_p, c_int64,
                            c_void_p, c_int64, c_void_p, c_void_p], None),
    "oq_build_icl_prefix": ([POINTER(TalkerHost), POINTER(PredictorHost), c_void_p, c_int64, c_void_p, c_int64,
                             c_void_p], None),
    "oq_build_trailing_text": ([POINTER(TalkerHost), c_void_p, c_int64, c_void_p], None),
    "oq_prefill_custom_voice": ([POINTER(TalkerHost), c_void_p, c_int64, c_uint32, c_uint32, c_void_p, c_int64,
                                 c_void_p, c_int64, POINTER(OqKv), c_void_p, c_void_p, c_void_p], c_int64),
    "od_set_threads": ([c_int], None),
    "od_causal_conv1d": ([c_void_p, c_int64, POINTER(Conv1dHost), c_void_p], None),
    "od_conv_transpose1d": ([c_void_p, c_int64, POINTER(ConvT1dHost), c_void_p], c_int64),
    "od_depthwise_conv1d": ([c_void_p, c_int64, POINTER(DwConvHost), c_void_p], None),
    "od_gemm_bias": ([c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p], None),
    "od_snake_beta": ([c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p], None),
    "od_gelu": ([c_float], c_float),
    "od_layer_norm_cf": ([c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_float, c_void_p], None),
    "od_warmup_trim_len": ([c_int64, c_int64, c_int64], c_int64),
    "od_decode_to_audio": ([POINTER(DecoderHost), c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                            POINTER(c_int64)], c_int),
}

_lib = None


def build():
    """Compile the oracle with its Makefile (gcc, strict IEEE)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        _lib = ctypes.CDLL(LIB)
        for k, (a, r) in _SIG.items():
            f = getattr(_lib, k)
            f.argtypes = a
            f.restype = r
    return _lib


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------------------
# numeric kernels
# ---------------------------------------------------------------------------

def gemv_scalar(x, w, k0=0, k1=None):
    """gemv_q4_scalar (gemv.rs:249-287) over rows k0..k1."""
    x = f32(x)
    out = np.empty(w.n, np.float32)
    lib().oq_gemv_q4_scalar(ptr(x), ptr(w.packed), ptr(w.scales), w.n, k0, w.k if k1 is None else k1, ptr(out))
    return out


def gemv_avx2(x, w, k0=0, k1=None):
    """gemv_q4_avx2 (simd.rs:76-153); None when the host lacks AVX2."""
    x = f32(x)
    out = np.empty(w.n, np.float32)
    ok = lib().oq_gemv_q4_avx2(ptr(x), ptr(w.packed), ptr(w.scales), w.n, k0, w.k if k1 is None else k1, ptr(out))
    return out if ok else None


def gemv_avx512(x, w, k0=0, k1=None):
    """gemv_q4_avx512 (simd.rs:203-269); None when the host lacks AVX-512."""
    x = f32(x)
    out = np.empty(w.n, np.float32)
    ok = lib().oq_gemv_q4_avx512(ptr(x), ptr(w.packed), ptr(w.scales), w.n, k0, w.k if k1 is None else k1, ptr(out))
    return out if ok else None


ISA_NAMES = {0: "scalar", 1: "avx2", 2: "avx512f"}


def set_isa(isa=None):
    """Inner GEMV kernel of the chunked GEMV: None for the reference's own
    choice (gemv.rs:230-243: AVX-512, else AVX2, else scalar), or "scalar",
    "avx2", "avx512f".  Returns the ISA in use, None if the host lacks it."""
    code = -1 if isa is None else {v: k for k, v in ISA_NAMES.items()}[isa]
    r = lib().oq_set_isa(code)
    return None if r < 0 else ISA_NAMES[r]


def get_isa():
    return ISA_NAMES[lib().oq_get_isa()]


def frame_temperature(params, frame_idx):
    """frame_temperature (generate_new.rs:82-88)."""
    return lib().oq_frame_temperature(byref(params), frame_idx)


def icl_layout(n_ref, n_text, n_frames):
    """icl_block_layout (generate_new.rs:120-128): (icl_len, remainder_len)."""
    a, b = c_int64(), c_int64()
    lib().oq_icl_layout(n_ref, n_text, n_frames, byref(a), byref(b))
    return a.value, b.value


def set_workers(workers=16, threads=0):
    lib().oq_set_workers(workers, threads)


def gemv(x, w):
    """gemv_q4 chunk policy (gemv.rs:290-346)."""
    x = f32(x)
    out = np.empty(w.n, np.float32)
    lib().oq_gemv_q4(ptr(x), byref(hostdesc.q4_host(w)), ptr(out))
    return out


def gemm(X, w):
    X = f32(X).reshape(-1, w.k)
    Y = np.empty((X.shape[0], w.n), np.float32)
    lib().oq_gemm_q4(ptr(X), X.shape[0], byref(hostdesc.q4_host(w)), ptr(Y))
    return Y


def embed_lookup(w, row, width=None):
    width = w.n if width is None else width
    out = np.empty(width, np.float32)
    lib().oq_embed_lookup_q4(byref(hostdesc.q4_host(w)), row, width, ptr(out))
    return out


def quantize(data, k, n):
    d = f32(data)
    packed = np.empty((k, n // 32 * 16), np.uint8)
    scales = np.empty((k, n // 32), np.uint16)
    lib().oq_quantize_q4(ptr(d), k, n, ptr(packed), ptr(scales))
    return packed, scales


def rms_norm(x, gamma):
    x = f32(x)
    out = np.empty_like(x)
    lib().oq_rms_norm_f16(ptr(x), ptr(gamma), x.size, ptr(out))
    return out


def softmax_raw(s):
    s = f32(s).copy()
    lib().oq_softmax_raw(ptr(s), s.size)
    return s


def silu(x):
    return lib().oq_silu(x)


def qk_norm(d, heads, hd, gamma):
    d = f32(d).copy()
    lib().oq_qk_norm(ptr(d), heads, hd, ptr(gamma))
    return d


def rope_table(head_dim, max_pos, theta=1_000_000.0):
    half = head_dim // 2
    c = np.empty((max_pos, half), np.float32)
    s = np.empty((max_pos, half), np.float32)
    lib().oq_rope_table(head_dim, max_pos, theta, ptr(c), ptr(s))
    return c, s


def rope_apply(d, heads, hd, pos, cos_t, sin_t):
    d = f32(d).copy()
    lib().oq_rope_apply(ptr(d), heads, hd, pos, ptr(cos_t), ptr(sin_t), cos_t.shape[0])
    return d


def f16_to_f32(h):
    return lib().oq_f16_to_f32(h)


def f32_to_f16(f):
    return lib().oq_f32_to_f16(f)


def simple_rand(state):
    s = c_uint64(state)
    r = lib().oq_simple_rand(byref(s))
    return r, s.value


def argmax_last(v):
    v = f32(v)
    return lib().oq_argmax_last(ptr(v), v.size)


def sample_token(logits, params, prev, rng, temperature):
    lg = f32(logits)
    pv = np.ascontiguousarray(prev, dtype=np.uint32)
    s = c_uint64(rng)
    out = c_uint32()
    rc = lib().oq_sample_token(ptr(lg), lg.size, byref(params), ptr(pv) if pv.size else None, pv.size, byref(s),
                               temperature, byref(out))
    if rc != 0:
        raise RuntimeError(f"oracle sample_token rc={rc}")
    return out.value, s.value


def sample_top_k(logits, temperature, top_k, prev, penalty, rng):
    """The legacy loop's sampler (generate.rs:185-217): (token, rng) or
    raises with the status (QTTS_ERR_INVALID for top_k 0, _NAN)."""
    lg = f32(logits)
    pv = np.ascontiguousarray(prev, dtype=np.uint32)
    s = c_uint64(rng)
    out = c_uint32()
    rc = lib().oq_sample_top_k(ptr(lg), lg.size, temperature, top_k, ptr(pv) if pv.size else None, pv.size, penalty,
                               byref(s), byref(out))
    if rc != 0:
        raise RuntimeError(f"oracle sample_top_k rc={rc}")
    return out.value, s.value


# ---------------------------------------------------------------------------
# model-level oracle
# ---------------------------------------------------------------------------

class Model:
    """Talker + predictor held by the oracle, with its own KV caches."""

    def __init__(self, talker, predictor, kv_cap=4096):
        self.t, self.p = talker, predictor
        self.th, self._kt = hostdesc.talker_host(talker)
        self.ph, self._kp = hostdesc.predictor_host(predictor)
        self.tkv = lib().oq_kv_new(len(talker.layers), talker.n_kv_heads, talker.head_dim, kv_cap)
        self.pkv = lib().oq_kv_new(len(predictor.layers), predictor.n_kv_heads, predictor.head_dim, 16)
        # the legacy predictor's cache, kept across predict_codes calls
        self.lkv = lib().oq_kv_new(len(predictor.layers), predictor.n_kv_heads, predictor.head_dim, kv_cap)

    def close(self):
        if self.tkv:
            lib().oq_kv_free(self.tkv)
            lib().oq_kv_free(self.pkv)
            lib().oq_kv_free(self.lkv)
            self.tkv = self.pkv = self.lkv = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def kv_len(self):
        return lib().oq_kv_len(self.tkv, 0)

    def kv_layer(self, layer):
        n = self.kv_len()
        cnt = n * self.t.n_kv_heads * self.t.head_dim
        K = np.ctypeslib.as_array(lib().oq_kv_k(self.tkv, layer), shape=(cnt,)).reshape(n, 8, 128).copy()
        V = np.ctypeslib.as_array(lib().oq_kv_v(self.tkv, layer), shape=(cnt,)).reshape(n, 8, 128).copy()
        return K, V

    def kv_load(self, K, V):
        """K, V: [n_layers][len][8][128]."""
        n = K.shape[1]
        for l in range(len(self.t.layers)):
            cnt = n * 8 * 128
            ctypes.memmove(lib().oq_kv_k(self.tkv, l), f32(K[l]).ctypes.data, cnt * 4)
            ctypes.memmove(lib().oq_kv_v(self.tkv, l), f32(V[l]).ctypes.data, cnt * 4)
        lib().oq_kv_set_len(self.tkv, n)

    def kv_reset(self):
        lib().oq_kv_reset(self.tkv)

    def forward_with_embedding(self, emb, position):
        e = f32(emb)
        out = np.empty(self.t.hidden + self.t.vocab, np.float32)
        rc = lib().oq_talker_step(byref(self.th), ptr(e), self.tkv, position, ptr(out))
        if rc:
            raise RuntimeError(f"oracle talker step rc={rc}")
        return out

    def prefill(self, X, start_pos):
        X = f32(X).reshape(-1, self.t.hidden)
        out = np.empty(self.t.hidden, np.float32)
        rc = lib().oq_talker_prefill(byref(self.th), ptr(X), X.shape[0], self.tkv, start_pos, ptr(out))
        if rc:
            raise RuntimeError(f"oracle prefill rc={rc}")
        return out

    def codec_head(self, hidden):
        h = f32(hidden)
        out = np.empty(self.t.vocab, np.float32)
        lib().oq_codec_head(byref(self.th), ptr(h), ptr(out))
        return out

    def embed_text_token(self, tok):
        out = np.empty(self.t.hidden, np.float32)
        lib().oq_embed_text_token(byref(self.th), tok, ptr(out))
        return out

    def embed_codec_token(self, tok):
        out = np.empty(self.t.hidden, np.float32)
        lib().oq_embed_codec_token(byref(self.th), tok, ptr(out))
        return out

    def predictor_chain(self, th, sem, forced=None):
        a, b = f32(th), f32(sem)
        codes = np.empty(len(self.p.lm_heads), np.uint32)
        fc = None if forced is None else np.ascontiguousarray(forced, dtype=np.uint32)
        rc = lib().oq_predictor_chain(byref(self.ph), ptr(a), ptr(b), self.pkv, ptr(codes), ptr(fc) if fc is not None else None)
        if rc:
            raise RuntimeError(f"oracle predictor rc={rc}")
        return codes

    def predict_codes(self, th):
        """predict_codes (code_predictor.rs:126-216): logits [n_groups][vocab]."""
        out = np.empty((len(self.p.lm_heads), self.p.vocab), np.float32)
        rc = lib().oq_predict_codes(byref(self.ph), ptr(f32(th)), self.lkv, ptr(out))
        if rc:
            raise RuntimeError(f"oracle predict_codes rc={rc}")
        return out

    def predict_codes_reset(self):
        lib().oq_kv_reset(self.lkv)

    def acoustic_embed_sum(self, codes):
        c = np.ascontiguousarray(codes, dtype=np.uint32)
        out = np.empty(self.t.hidden, np.float32)
        lib().oq_acoustic_embed_sum(byref(self.ph), ptr(c), c.size, ptr(out))
        return out

    # prompt construction (generate_new.rs:82-476) ----------------------------
    def build_prefill_head(self, speaker_id, language_id, voice=None):
        """build_prefill_head (generate_new.rs:222-237): [9][hidden]."""
        out = np.empty((9, self.t.hidden), np.float32)
        v = None if voice is None else f32(voice)
        lib().oq_build_prefill_head(byref(self.th), speaker_id, language_id, ptr(v) if v is not None else None,
                                    0 if v is None else v.size, ptr(out))
        return out

    def build_icl_block(self, ref_tokens, text_tokens, ref_codes):
        """build_icl_block (generate_new.rs:140-195): (icl, remainder)."""
        rt = np.ascontiguousarray(ref_tokens, np.uint32)
        tt = np.ascontiguousarray(text_tokens, np.uint32)
        codes = np.ascontiguousarray(ref_codes, np.uint32).reshape(16, -1)
        icl_len, rem_len = icl_layout(rt.size, tt.size, codes.shape[1])
        icl = np.empty((icl_len, self.t.hidden), np.float32)
        rem = np.empty((rem_len, self.t.hidden), np.float32)
        lib().oq_build_icl_block(byref(self.th), byref(self.ph), ptr(rt) if rt.size else None, rt.size,
                                 ptr(tt) if tt.size else None, tt.size, ptr(codes), codes.shape[1], ptr(icl),
                                 ptr(rem) if rem_len else None)
        return icl, rem

    def build_icl_prefix(self, ref_tokens, ref_codes):
        """build_icl_prefix (generate_new.rs:244-280): [len(ref_tokens)][hidden]."""
        rt = np.ascontiguousarray(ref_tokens, np.uint32)
        codes = np.ascontiguousarray(ref_codes, np.uint32).reshape(16, -1)
        out = np.empty((rt.size, self.t.hidden), np.float32)
        lib().oq_build_icl_prefix(byref(self.th), byref(self.ph), ptr(rt), rt.size, ptr(codes), codes.shape[1],
                                  ptr(out))
        return out

    def build_trailing_text(self, tokens):
        """build_trailing_text (generate_new.rs:756-767)."""
        tk = np.ascontiguousarray(tokens, np.uint32)
        out = np.empty((max(tk.size - 1, 0) + 1, self.t.hidden), np.float32)
        lib().oq_build_trailing_text(byref(self.th), ptr(tk) if tk.size else None, tk.size, ptr(out))
        return out

    def prefill_custom_voice(self, text_tokens, speaker_id, language_id, voice=None, icl_rows=None):
        """prefill_custom_voice (generate_new.rs:361-476) from position 0:
        (hidden, logits, position, prompt rows)."""
        tt = np.ascontiguousarray(text_tokens, np.uint32)
        v = None if voice is None else f32(voice)
        icl = None if icl_rows is None else f32(icl_rows).reshape(-1, self.t.hidden)
        n = 9 + (icl.shape[0] if icl is not None else int(tt.size > 0))
        rows = np.empty((n, self.t.hidden), np.float32)
        hid = np.empty(self.t.hidden, np.float32)
        lg = np.empty(self.t.vocab, np.float32)
        pos = lib().oq_prefill_custom_voice(byref(self.th), ptr(tt) if tt.size else None, tt.size, speaker_id,
                                            language_id, ptr(v) if v is not None else None,
                                            0 if v is None else v.size, ptr(icl) if icl is not None else None,
                                            0 if icl is None else icl.shape[0], self.tkv, ptr(hid), ptr(lg), ptr(rows))
        if pos < 0:
            raise RuntimeError(f"oracle prefill_custom_voice rc={pos}")
        return hid, lg, int(pos), rows

    # frame loop ---------------------------------------------------------------
    def gen_begin(self, logits, hidden, position, seed):
        self.g_logits = f32(logits).copy()
        self.g_hidden = f32(hidden).copy()
        self.gen = OqGen(self.g_logits.ctypes.data, self.g_hidden.ctypes.data, (c_uint32 * 16)(), seed, position, 0)

    def frame(self, params, text_add, forced=None):
        """One frame: (codes[16] predicted, eos)."""
        codes = np.empty(16, np.uint32)
        eos = c_int32()
        ta = f32(text_add)
        fc = None if forced is None else np.ascontiguousarray(forced, dtype=np.uint32)
        rc = lib().oq_frame(byref(self.th), byref(self.ph), self.tkv, self.pkv, byref(self.gen), byref(params), ptr(ta),
                            ptr(codes), byref(eos), ptr(fc) if fc is not None else None)
        if rc:
            raise RuntimeError(f"oracle frame rc={rc}")
        return codes, bool(eos.value)


# ---------------------------------------------------------------------------
# speech decoder (qtts_decoder.c)
# ---------------------------------------------------------------------------

def causal_conv1d(x, c):
    """causal_conv1d (conv.rs:114-228): x [in][len] -> [out][len]."""
    x = f32(x)
    out = np.empty((c.out_channels, x.shape[1]), np.float32)
    lib().od_causal_conv1d(ptr(x), x.shape[1], byref(hostdesc.conv1d_host(c)), ptr(out))
    return out


def conv_transpose1d(x, c):
    """conv_transpose1d (conv.rs:247-349), uncropped."""
    x = f32(x)
    n = (x.shape[1] - 1) * c.stride - 2 * c.padding + c.kernel_size
    out = np.empty((c.out_channels, n), np.float32)
    lib().od_conv_transpose1d(ptr(x), x.shape[1], byref(hostdesc.convt1d_host(c)), ptr(out))
    return out


def depthwise_conv1d(x, c):
    x = f32(x)
    out = np.empty_like(x)
    lib().od_depthwise_conv1d(ptr(x), x.shape[1], byref(DwConvHost(ptr(c.weight), ptr(c.bias), c.channels,
                                                                      c.kernel_size, c.padding, 0)), ptr(out))
    return out


def gemm_bias(a, b, bias):
    a, b, bias = f32(a), f32(b), f32(bias)
    out = np.empty((a.shape[0], b.shape[1]), np.float32)
    lib().od_gemm_bias(ptr(a), ptr(b), ptr(bias), a.shape[0], b.shape[1], a.shape[1], ptr(out))
    return out


def snake_beta(x, alpha, beta):
    x, alpha, beta = f32(x), f32(alpha), f32(beta)
    out = np.empty_like(x)
    lib().od_snake_beta(ptr(x), ptr(alpha), ptr(beta), x.shape[0], x.shape[1], ptr(out))
    return out


def gelu(x):
    return lib().od_gelu(x)


def layer_norm_cf(x, gamma, beta, eps=1e-5):
    x = f32(x)
    out = np.empty_like(x)
    lib().od_layer_norm_cf(ptr(x), ptr(f32(gamma)), ptr(f32(beta)), x.shape[0], x.shape[1], eps, ptr(out))
    return out


def warmup_trim_len(tv, total, n):
    return lib().od_warmup_trim_len(tv, total, n)


def decode_to_audio(d, codes, warmup=None, threads=8):
    """decode_to_audio (decoder.rs:395-584): codes [16][T] -> samples."""
    codes = np.ascontiguousarray(codes, np.uint32)
    T = codes.shape[1]
    Tv = 0 if warmup is None else warmup.shape[1]
    if warmup is not None:
        warmup = np.ascontiguousarray(warmup, np.uint32)
    cap = (T + Tv) * d.upsample_factor
    out = np.empty(cap, np.float32)
    n = c_int64()
    h, keep = hostdesc.decoder_host(d)
    lib().od_set_threads(threads)
    rc = lib().od_decode_to_audio(byref(h), ptr(codes), T, ptr(warmup) if warmup is not None else None, Tv,
                                  ptr(out), cap, byref(n))
    assert rc == 0, "oracle decode failed"
    return out[: n.value].copy()
