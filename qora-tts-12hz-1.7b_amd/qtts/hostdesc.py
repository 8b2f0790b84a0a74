"""ctypes mirrors of the host-side descriptor structs in include/qtts.h.

These describe weights that live in caller (host) memory: plain pointers and
sizes, the layout of the reference's `Q4Weight` (gemv.rs:26-31),
`TalkerWeights` (talker.rs:33-56) and `CodePredictorWeights`
(code_predictor.rs:28-46).
"""
import ctypes
from ctypes import c_float, c_int32, c_int64, c_uint32, c_void_p


class Q4Host(ctypes.Structure):
    _fields_ = [("packed", c_void_p), ("scales", c_void_p), ("k", c_int64), ("n", c_int64)]


class LayerHost(ctypes.Structure):
    _fields_ = [
        ("q_proj", Q4Host), ("k_proj", Q4Host), ("v_proj", Q4Host), ("o_proj", Q4Host),
        ("q_norm", c_void_p), ("k_norm", c_void_p),
        ("gate_proj", Q4Host), ("up_proj", Q4Host), ("down_proj", Q4Host),
        ("input_norm", c_void_p), ("post_attn_norm", c_void_p),
    ]


class TalkerHost(ctypes.Structure):
    _fields_ = [
        ("n_layers", c_int32), ("hidden", c_int32), ("text_hidden", c_int32),
        ("n_heads", c_int32), ("n_kv_heads", c_int32), ("head_dim", c_int32),
        ("inter", c_int32), ("vocab", c_int32),
        ("layers", ctypes.POINTER(LayerHost)),
        ("codec_embedding", Q4Host), ("text_embedding", Q4Host),
        ("text_fc1", Q4Host), ("text_fc2", Q4Host),
        ("text_fc1_bias", c_void_p), ("text_fc2_bias", c_void_p),
        ("codec_head", Q4Host),
        ("final_norm", c_void_p),
        ("rope_cos", c_void_p), ("rope_sin", c_void_p),
        ("rope_max_pos", c_int64),
    ]


class PredictorHost(ctypes.Structure):
    _fields_ = [
        ("n_layers", c_int32), ("hidden", c_int32), ("n_heads", c_int32),
        ("n_kv_heads", c_int32), ("head_dim", c_int32), ("inter", c_int32),
        ("vocab", c_int32), ("n_groups", c_int32), ("has_input_proj", c_int32),
        ("input_proj", Q4Host), ("input_proj_bias", c_void_p),
        ("codec_embeddings", ctypes.POINTER(Q4Host)),
        ("layers", ctypes.POINTER(LayerHost)),
        ("lm_heads", ctypes.POINTER(Q4Host)),
        ("final_norm", c_void_p),
        ("rope_cos", c_void_p), ("rope_sin", c_void_p),
        ("rope_max_pos", c_int64),
    ]


class SampleParams(ctypes.Structure):
    """`TTSParams` fields read by `sample_token` (generate_new.rs:38-79)."""
    _fields_ = [
        ("temperature", c_float), ("top_k", c_int32), ("top_p", c_float),
        ("repetition_penalty", c_float), ("codec_eos_id", c_uint32),
        ("eos_enabled", c_int32), ("onset_frames", c_int32),
        ("onset_temperature", c_float),
    ]


def sample_params(temperature=0.9, top_k=50, top_p=1.0, repetition_penalty=1.05,
                  codec_eos_id=2150, eos_enabled=True, onset_frames=0,
                  onset_temperature=0.3):
    """Defaults of `TTSParams::default()` (generate_new.rs:63-79)."""
    return SampleParams(temperature, top_k, top_p, repetition_penalty, codec_eos_id,
                        1 if eos_enabled else 0, onset_frames, onset_temperature)


def ptr(a):
    """Address of a C-contiguous numpy array (None for None)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "arrays passed to the C ABI must be contiguous"
    return a.ctypes.data


def q4_host(w):
    """Q4Host for a `Q4` (packed uint8 [k, n/32*16], scales uint16 [k, n/32])."""
    return Q4Host(ptr(w.packed), ptr(w.scales), w.k, w.n)


def layer_host(L):
    return LayerHost(
        q4_host(L.q_proj), q4_host(L.k_proj), q4_host(L.v_proj), q4_host(L.o_proj),
        ptr(L.q_norm), ptr(L.k_norm),
        q4_host(L.gate_proj), q4_host(L.up_proj), q4_host(L.down_proj),
        ptr(L.input_norm), ptr(L.post_attn_norm))


def talker_host(t):
    """Build a TalkerHost; the returned tuple keeps the layer array alive."""
    layers = (LayerHost * len(t.layers))(*[layer_host(L) for L in t.layers])
    h = TalkerHost(
        len(t.layers), t.hidden, t.text_hidden, t.n_heads, t.n_kv_heads, t.head_dim,
        t.inter, t.vocab, layers,
        q4_host(t.codec_embedding), q4_host(t.text_embedding),
        q4_host(t.text_fc1), q4_host(t.text_fc2),
        ptr(t.text_fc1_bias), ptr(t.text_fc2_bias),
        q4_host(t.codec_head), ptr(t.final_norm),
        ptr(t.rope_cos), ptr(t.rope_sin), t.rope_cos.shape[0])
    return h, layers


def predictor_host(p):
    layers = (LayerHost * len(p.layers))(*[layer_host(L) for L in p.layers])
    embs = (Q4Host * len(p.codec_embeddings))(*[q4_host(e) for e in p.codec_embeddings])
    heads = (Q4Host * len(p.lm_heads))(*[q4_host(h) for h in p.lm_heads])
    h = PredictorHost(
        len(p.layers), p.hidden, p.n_heads, p.n_kv_heads, p.head_dim, p.inter,
        p.vocab, len(p.lm_heads), 1,
        q4_host(p.input_proj), ptr(p.input_proj_bias),
        embs, layers, heads, ptr(p.final_norm),
        ptr(p.rope_cos), ptr(p.rope_sin), p.rope_cos.shape[0])
    return h, (layers, embs, heads)
