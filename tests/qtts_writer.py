"""Writer of the `.qora-tts` stream's header, talker and predictor sections
(save.rs:23-137, field order of save_model / save_talker / save_predictor;
weight and vector encodings of gemv.rs:645-687), for round-trip tests of
qtts_model_load_qtts.  Little-endian throughout:

    "QTTS", u32 version = 1, u8 format (1 = Q4, 0 = F16)
    talker:    u32 n_layers, hidden, text_hidden, n_heads, n_kv_heads, head_dim,
               n_kv_groups, u32 n_sections, u32 sections[n]
               per layer: W q k v o, f16v q_norm k_norm, W gate up down,
                          f16v input_norm post_norm
               W codec_emb, W text_emb, W fc1, f32v fc1_bias, W fc2, f32v fc2_bias,
               W codec_head, f16v final_norm, f32v rope_cos, f32v rope_sin
    predictor: u32 n_layers, hidden, n_heads, n_kv_heads, head_dim, n_kv_groups,
               u8 has_proj [W proj, f32v bias], u32 n_emb, W emb[n],
               layers as above, u32 n_heads_lm, W heads[n], f16v final_norm,
               f32v rope_cos, f32v rope_sin
    W    = u64 k, u64 n, u64 len + packed bytes, u64 len + len f16 scales
    f16v = u64 len + len * 2 bytes;  f32v = u64 len + len * 4 bytes

With `decoder`, the speech-decoder section follows (save.rs:139-260:
config u32s, codebooks, pre-conv, transformer, upsamplers, Vocos, output
conv, RoPE tables; convolutions as u32 shape fields then f32v weight and
bias).  The speaker-encoder section of a real file is not written.
"""
import struct

import numpy as np


def _u32(f, v):
    f.write(struct.pack("<I", v))


def _u64(f, v):
    f.write(struct.pack("<Q", v))


def _bytes(f, b):
    b = np.ascontiguousarray(b, np.uint8)
    _u64(f, b.size)
    f.write(b.tobytes())


def _f16v(f, bits):
    bits = np.ascontiguousarray(bits, np.uint16)
    _u64(f, bits.size)
    f.write(bits.tobytes())


def _f32v(f, v):
    v = np.ascontiguousarray(v, np.float32)
    _u64(f, v.size)
    f.write(v.tobytes())


def _weight(f, w):
    _u64(f, w.k)
    _u64(f, w.n)
    _bytes(f, w.packed.reshape(-1))
    _f16v(f, w.scales.reshape(-1))


def _layer(f, L):
    for w in (L.q_proj, L.k_proj, L.v_proj, L.o_proj):
        _weight(f, w)
    _f16v(f, L.q_norm)
    _f16v(f, L.k_norm)
    for w in (L.gate_proj, L.up_proj, L.down_proj):
        _weight(f, w)
    _f16v(f, L.input_norm)
    _f16v(f, L.post_attn_norm)


def _conv(f, c):
    for v in (c.in_channels, c.out_channels, c.kernel_size, c.stride, c.padding, c.dilation):
        _u32(f, v)
    _f32v(f, c.weight.reshape(-1))
    _f32v(f, c.bias)


def _convt(f, c):
    for v in (c.in_channels, c.out_channels, c.kernel_size, c.stride, c.padding):
        _u32(f, v)
    _f32v(f, c.weight.reshape(-1))
    _f32v(f, c.bias)


def _dw(f, c):
    for v in (c.channels, c.kernel_size, c.padding):
        _u32(f, v)
    _f32v(f, c.weight.reshape(-1))
    _f32v(f, c.bias)


def _decoder(f, d):
    for v in (d.hidden, d.n_heads, d.head_dim, d.inter, d.sliding_window, d.codebook_dim):
        _u32(f, v)
    _f32v(f, d.first_codebook.reshape(-1))
    _f32v(f, d.first_output_proj.reshape(-1))
    _u32(f, len(d.rest_codebooks))
    for cb in d.rest_codebooks:
        _f32v(f, cb.reshape(-1))
    _f32v(f, d.rest_output_proj.reshape(-1))
    _conv(f, d.pre_conv)
    _f32v(f, d.tf_input_w.reshape(-1))
    _f32v(f, d.tf_input_b)
    _u32(f, len(d.tf_layers))
    for L in d.tf_layers:
        for v in (L.q_proj, L.k_proj, L.v_proj, L.o_proj, L.gate_proj, L.up_proj, L.down_proj, L.input_norm,
                  L.post_attn_norm, L.attn_scale, L.mlp_scale):
            _f32v(f, v.reshape(-1))
    _f32v(f, d.tf_norm)
    _f32v(f, d.tf_output_w.reshape(-1))
    _f32v(f, d.tf_output_b)
    _u32(f, len(d.upsample))
    for u in d.upsample:
        _u32(f, u.channels)
        _convt(f, u.conv_t)
        _dw(f, u.dw_conv)
        for v in (u.norm_w, u.norm_b, u.pw1_w, u.pw1_b, u.pw2_w, u.pw2_b, u.gamma):
            _f32v(f, v.reshape(-1))
    _conv(f, d.vocos_init)
    _u32(f, len(d.vocos_blocks))
    for b in d.vocos_blocks:
        _f32v(f, b.pre_snake_alpha)
        _f32v(f, b.pre_snake_beta)
        _convt(f, b.upsample)
        _u32(f, len(b.residuals))
        for r in b.residuals:
            _f32v(f, r.act1_alpha)
            _f32v(f, r.act1_beta)
            _conv(f, r.conv1)
            _f32v(f, r.act2_alpha)
            _f32v(f, r.act2_beta)
            _conv(f, r.conv2)
    _f32v(f, d.final_snake_alpha)
    _f32v(f, d.final_snake_beta)
    _conv(f, d.output_conv)
    _f32v(f, d.rope_cos.reshape(-1))
    _f32v(f, d.rope_sin.reshape(-1))


def write_qtts(path, talker, predictor, format_id=1, mrope_section=(24, 20, 20), decoder=None):
    t, p = talker, predictor
    with open(path, "wb") as f:
        f.write(b"QTTS")
        _u32(f, 1)
        f.write(bytes([format_id]))
        for v in (len(t.layers), t.hidden, t.text_hidden, t.n_heads, t.n_kv_heads, t.head_dim,
                  t.n_heads // t.n_kv_heads, len(mrope_section)):
            _u32(f, v)
        for v in mrope_section:
            _u32(f, v)
        for L in t.layers:
            _layer(f, L)
        _weight(f, t.codec_embedding)
        _weight(f, t.text_embedding)
        _weight(f, t.text_fc1)
        _f32v(f, t.text_fc1_bias)
        _weight(f, t.text_fc2)
        _f32v(f, t.text_fc2_bias)
        _weight(f, t.codec_head)
        _f16v(f, t.final_norm)
        _f32v(f, t.rope_cos.reshape(-1))
        _f32v(f, t.rope_sin.reshape(-1))
        for v in (len(p.layers), p.hidden, p.n_heads, p.n_kv_heads, p.head_dim, p.n_heads // p.n_kv_heads):
            _u32(f, v)
        f.write(bytes([1]))
        _weight(f, p.input_proj)
        _f32v(f, p.input_proj_bias)
        _u32(f, len(p.codec_embeddings))
        for w in p.codec_embeddings:
            _weight(f, w)
        for L in p.layers:
            _layer(f, L)
        _u32(f, len(p.lm_heads))
        for w in p.lm_heads:
            _weight(f, w)
        _f16v(f, p.final_norm)
        _f32v(f, p.rope_cos.reshape(-1))
        _f32v(f, p.rope_sin.reshape(-1))
        if decoder is not None:
            _decoder(f, decoder)


def _f16_bits(v):
    return np.ascontiguousarray(np.asarray(v, np.float32).astype(np.float16)).view(np.uint16)


def write_qora_q4(path, talker, predictor, f16_weights=()):
    """The older "QORA-TTS-Q4" named-tensor container (loader.rs:47-127),
    with the tensor names load_talker_binary / load_code_predictor_binary
    map (loader.rs:724-882).  Biases are stored as F16, as the container
    holds them; names in `f16_weights` are written in the F16 format (which
    the device path refuses)."""
    t, p = talker, predictor
    items = []

    def q4(name, w):
        items.append((name, [w.k, w.n], w))

    def f16(name, v):
        items.append((name, [len(v)], _f16_bits(v) if np.asarray(v).dtype != np.uint16 else np.asarray(v, np.uint16)))

    def layer(pre, L):
        for nm, w in (("self_attn.q_proj", L.q_proj), ("self_attn.k_proj", L.k_proj), ("self_attn.v_proj", L.v_proj),
                      ("self_attn.o_proj", L.o_proj), ("mlp.gate_proj", L.gate_proj), ("mlp.up_proj", L.up_proj),
                      ("mlp.down_proj", L.down_proj)):
            q4(f"{pre}.{nm}.weight", w)
        f16(f"{pre}.self_attn.q_norm.weight", L.q_norm)
        f16(f"{pre}.self_attn.k_norm.weight", L.k_norm)
        f16(f"{pre}.input_layernorm.weight", L.input_norm)
        f16(f"{pre}.post_attention_layernorm.weight", L.post_attn_norm)

    for i, L in enumerate(t.layers):
        layer(f"talker.model.layers.{i}", L)
    q4("talker.model.codec_embedding.weight", t.codec_embedding)
    q4("talker.model.text_embedding.weight", t.text_embedding)
    q4("talker.text_projection.linear_fc1.weight", t.text_fc1)
    f16("talker.text_projection.linear_fc1.bias", t.text_fc1_bias)
    q4("talker.text_projection.linear_fc2.weight", t.text_fc2)
    f16("talker.text_projection.linear_fc2.bias", t.text_fc2_bias)
    q4("talker.codec_head.weight", t.codec_head)
    f16("talker.model.norm.weight", t.final_norm)
    q4("talker.code_predictor.small_to_mtp_projection.weight", p.input_proj)
    f16("talker.code_predictor.small_to_mtp_projection.bias", p.input_proj_bias)
    for g, w in enumerate(p.codec_embeddings):
        q4(f"talker.code_predictor.model.codec_embedding.{g}.weight", w)
    for i, L in enumerate(p.layers):
        layer(f"talker.code_predictor.model.layers.{i}", L)
    for g, w in enumerate(p.lm_heads):
        q4(f"talker.code_predictor.lm_head.{g}.weight", w)
    f16("talker.code_predictor.model.norm.weight", p.final_norm)
    with open(path, "wb") as f:
        f.write(b"QORA-TTS-Q4" + bytes(5))
        f.write(struct.pack("<II", 1, len(items)))
        for name, shape, data in items:
            nb = name.encode()
            f.write(struct.pack("<I", len(nb)) + nb)
            f.write(struct.pack("<I", len(shape)) + b"".join(struct.pack("<I", d) for d in shape))
            if hasattr(data, "packed") and name not in f16_weights:
                sc = np.ascontiguousarray(data.scales, np.uint16).reshape(-1)
                pk = np.ascontiguousarray(data.packed, np.uint8).reshape(-1)
                f.write(bytes([1]) + struct.pack("<I", sc.size) + sc.tobytes() + struct.pack("<I", pk.size) + pk.tobytes())
            elif hasattr(data, "packed"):
                vals = _f16_bits(np.zeros(data.k * data.n, np.float32))
                f.write(bytes([0]) + struct.pack("<I", vals.size) + vals.tobytes())
            else:
                f.write(bytes([0]) + struct.pack("<I", data.size) + data.tobytes())
