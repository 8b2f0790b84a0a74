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


class Conv1dHost(ctypes.Structure):
    """`Conv1dWeight` (conv.rs:29-38)."""
    _fields_ = [("weight", c_void_p), ("bias", c_void_p), ("in_channels", c_int32), ("out_channels", c_int32),
                ("kernel_size", c_int32), ("stride", c_int32), ("padding", c_int32), ("dilation", c_int32)]


class ConvT1dHost(ctypes.Structure):
    """`ConvTranspose1dWeight` (conv.rs:235-243)."""
    _fields_ = [("weight", c_void_p), ("bias", c_void_p), ("in_channels", c_int32), ("out_channels", c_int32),
                ("kernel_size", c_int32), ("stride", c_int32), ("padding", c_int32), ("reserved", c_int32)]


class DwConvHost(ctypes.Structure):
    """`DepthwiseConv1dWeight` (conv.rs:351-357)."""
    _fields_ = [("weight", c_void_p), ("bias", c_void_p), ("channels", c_int32), ("kernel_size", c_int32),
                ("padding", c_int32), ("reserved", c_int32)]


class DecLayerHost(ctypes.Structure):
    """`DecoderTfLayer` (decoder.rs:68-80)."""
    _fields_ = [(n, c_void_p) for n in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj",
                                        "down_proj", "input_norm", "post_attn_norm", "attn_scale", "mlp_scale")]


class UpsampleHost(ctypes.Structure):
    """`UpsampleStage` (decoder.rs:82-93)."""
    _fields_ = [("conv_t", ConvT1dHost), ("dw_conv", DwConvHost)] + \
        [(n, c_void_p) for n in ("norm_w", "norm_b", "pw1_w", "pw1_b", "pw2_w", "pw2_b", "gamma")] + \
        [("channels", c_int32), ("inner", c_int32)]


class VocosResHost(ctypes.Structure):
    """`VocosResidual` (decoder.rs:102-109)."""
    _fields_ = [("act1_alpha", c_void_p), ("act1_beta", c_void_p), ("conv1", Conv1dHost),
                ("act2_alpha", c_void_p), ("act2_beta", c_void_p), ("conv2", Conv1dHost)]


class VocosBlockHost(ctypes.Structure):
    """`VocosBlock` (decoder.rs:95-100)."""
    _fields_ = [("pre_snake_alpha", c_void_p), ("pre_snake_beta", c_void_p), ("upsample", ConvT1dHost),
                ("residuals", ctypes.POINTER(VocosResHost)), ("n_residuals", c_int32), ("reserved", c_int32)]


class DecoderHost(ctypes.Structure):
    """`SpeechDecoderWeights` (decoder.rs:22-66)."""
    _fields_ = [
        ("hidden", c_int32), ("n_heads", c_int32), ("head_dim", c_int32), ("inter", c_int32),
        ("sliding_window", c_int32), ("codebook_dim", c_int32), ("codebook_size", c_int32), ("vq_dim", c_int32),
        ("first_codebook", c_void_p), ("first_output_proj", c_void_p),
        ("rest_codebooks", ctypes.POINTER(c_void_p)), ("rest_output_proj", c_void_p),
        ("n_rest", c_int32), ("latent", c_int32),
        ("pre_conv", Conv1dHost),
        ("tf_input_w", c_void_p), ("tf_input_b", c_void_p),
        ("tf_layers", ctypes.POINTER(DecLayerHost)),
        ("tf_norm", c_void_p), ("tf_output_w", c_void_p), ("tf_output_b", c_void_p),
        ("n_tf_layers", c_int32), ("n_upsample", c_int32),
        ("upsample", ctypes.POINTER(UpsampleHost)),
        ("vocos_init", Conv1dHost),
        ("vocos_blocks", ctypes.POINTER(VocosBlockHost)),
        ("n_vocos_blocks", c_int32), ("reserved", c_int32),
        ("final_snake_alpha", c_void_p), ("final_snake_beta", c_void_p),
        ("output_conv", Conv1dHost),
        ("rope_cos", c_void_p), ("rope_sin", c_void_p), ("rope_max_pos", c_int64),
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


def conv1d_host(c):
    return Conv1dHost(ptr(c.weight), ptr(c.bias), c.in_channels, c.out_channels, c.kernel_size, c.stride,
                      c.padding, c.dilation)


def convt1d_host(c):
    return ConvT1dHost(ptr(c.weight), ptr(c.bias), c.in_channels, c.out_channels, c.kernel_size, c.stride,
                       c.padding, 0)


def decoder_host(d):
    """Build a DecoderHost; the returned tuple keeps the nested arrays alive."""
    rest = (c_void_p * len(d.rest_codebooks))(*[ptr(c) for c in d.rest_codebooks])
    layers = (DecLayerHost * len(d.tf_layers))(*[
        DecLayerHost(*[ptr(getattr(L, n)) for n, _ in DecLayerHost._fields_]) for L in d.tf_layers])
    ups = (UpsampleHost * max(1, len(d.upsample)))(*[
        UpsampleHost(convt1d_host(u.conv_t),
                     DwConvHost(ptr(u.dw_conv.weight), ptr(u.dw_conv.bias), u.dw_conv.channels,
                                u.dw_conv.kernel_size, u.dw_conv.padding, 0),
                     ptr(u.norm_w), ptr(u.norm_b), ptr(u.pw1_w), ptr(u.pw1_b), ptr(u.pw2_w), ptr(u.pw2_b),
                     ptr(u.gamma), u.channels, u.inner) for u in d.upsample])
    res_arrays = []
    blocks = []
    for b in d.vocos_blocks:
        ra = (VocosResHost * len(b.residuals))(*[
            VocosResHost(ptr(r.act1_alpha), ptr(r.act1_beta), conv1d_host(r.conv1), ptr(r.act2_alpha),
                         ptr(r.act2_beta), conv1d_host(r.conv2)) for r in b.residuals])
        res_arrays.append(ra)
        blocks.append(VocosBlockHost(ptr(b.pre_snake_alpha), ptr(b.pre_snake_beta), convt1d_host(b.upsample),
                                     ra, len(b.residuals), 0))
    vb = (VocosBlockHost * max(1, len(blocks)))(*blocks)
    h = DecoderHost(
        d.hidden, d.n_heads, d.head_dim, d.inter, d.sliding_window, d.codebook_dim, d.codebook_size, d.vq_dim,
        ptr(d.first_codebook), ptr(d.first_output_proj), rest, ptr(d.rest_output_proj),
        len(d.rest_codebooks), d.latent, conv1d_host(d.pre_conv),
        ptr(d.tf_input_w), ptr(d.tf_input_b), layers, ptr(d.tf_norm), ptr(d.tf_output_w), ptr(d.tf_output_b),
        len(d.tf_layers), len(d.upsample), ups, conv1d_host(d.vocos_init), vb, len(d.vocos_blocks), 0,
        ptr(d.final_snake_alpha), ptr(d.final_snake_beta), conv1d_host(d.output_conv),
        ptr(d.rope_cos), ptr(d.rope_sin), d.rope_cos.shape[0])
    return h, (rest, layers, ups, res_arrays, vb)
