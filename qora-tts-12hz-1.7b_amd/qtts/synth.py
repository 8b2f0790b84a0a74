"""Seeded synthetic models in the reference's Q4 layout.

Real weights are not available, so every workload runs on random Q4
weights of the real architecture (Qwen3-TTS-12Hz-1.7B shapes,
model/1.7B/config.json): nibbles uniform over 0..15, per-group scales
|N(0, 0.02)| rounded to f16, RMSNorm gammas N(1, 0.05) in f16, biases
N(0, 0.02).  All draws come from numpy's PCG64 with an explicit seed, so
the device path and the oracle see identical bytes.
"""
from dataclasses import dataclass, field
from typing import List

import numpy as np

GROUP = 32   # Q4_GROUP_SIZE (gemv.rs:18)


@dataclass
class Q4:
    """`Q4Weight` (gemv.rs:26-31): packed[k][n/32*16] u8, scales[k][n/32] f16 bits."""
    packed: np.ndarray
    scales: np.ndarray
    k: int
    n: int

    def dequant(self) -> np.ndarray:
        """Dense f32 [k][n] (columns past (n/32)*32 are zero)."""
        g = self.n // GROUP
        lo = (self.packed & 0x0F).astype(np.int32) - 8
        hi = (self.packed >> 4).astype(np.int32) - 8
        q = np.empty((self.k, g * 16 * 2), np.int32)
        q[:, 0::2] = lo
        q[:, 1::2] = hi
        s = self.scales.view(np.float16).astype(np.float32)
        out = np.zeros((self.k, self.n), np.float32)
        out[:, : g * GROUP] = (q.reshape(self.k, g, GROUP) * s[:, :, None]).reshape(self.k, g * GROUP)
        return out

    @property
    def nbytes(self) -> int:
        return self.packed.nbytes + self.scales.nbytes


def q4_random(rng, k, n, scale_sigma=0.02):
    g = n // GROUP
    packed = rng.integers(0, 256, size=(k, g * 16), dtype=np.uint8)
    s = np.abs(rng.standard_normal((k, g), dtype=np.float32)) * np.float32(scale_sigma)
    return Q4(packed, s.astype(np.float16).view(np.uint16), k, n)


def gamma(rng, n):
    return (1.0 + 0.05 * rng.standard_normal(n)).astype(np.float16).view(np.uint16)


def bias(rng, n):
    return (0.02 * rng.standard_normal(n)).astype(np.float32)


def rope_table(head_dim, max_pos, theta=1_000_000.0):
    """`build_mrope_tables` (rope.rs:11-41) / loader.rs:393-408: f64 angles
    pos * theta^(-2i/head_dim), cos/sin rounded to f32, [max_pos][head_dim/2]."""
    half = head_dim // 2
    i = np.arange(half, dtype=np.float64)
    freq = 1.0 / np.power(theta, (2.0 * i) / head_dim)
    ang = np.arange(max_pos, dtype=np.float64)[:, None] * freq[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


@dataclass
class Layer:
    q_proj: Q4
    k_proj: Q4
    v_proj: Q4
    o_proj: Q4
    q_norm: np.ndarray
    k_norm: np.ndarray
    gate_proj: Q4
    up_proj: Q4
    down_proj: Q4
    input_norm: np.ndarray
    post_attn_norm: np.ndarray


def make_layer(rng, hidden, n_heads=16, n_kv=8, head_dim=128, inter=6144):
    qd, kd = n_heads * head_dim, n_kv * head_dim
    return Layer(
        q4_random(rng, hidden, qd), q4_random(rng, hidden, kd), q4_random(rng, hidden, kd),
        q4_random(rng, qd, hidden), gamma(rng, head_dim), gamma(rng, head_dim),
        q4_random(rng, hidden, inter), q4_random(rng, hidden, inter), q4_random(rng, inter, hidden),
        gamma(rng, hidden), gamma(rng, hidden))


@dataclass
class Talker:
    layers: List[Layer]
    codec_embedding: Q4
    text_embedding: Q4
    text_fc1: Q4
    text_fc2: Q4
    text_fc1_bias: np.ndarray
    text_fc2_bias: np.ndarray
    codec_head: Q4
    final_norm: np.ndarray
    rope_cos: np.ndarray
    rope_sin: np.ndarray
    hidden: int = 2048
    text_hidden: int = 2048
    n_heads: int = 16
    n_kv_heads: int = 8
    head_dim: int = 128
    inter: int = 6144
    vocab: int = 3072

    @property
    def weight_bytes(self) -> int:
        """Q4 bytes one decode step streams (layers + codec head)."""
        b = sum(w.nbytes for L in self.layers for w in
                (L.q_proj, L.k_proj, L.v_proj, L.o_proj, L.gate_proj, L.up_proj, L.down_proj))
        return b + self.codec_head.nbytes


@dataclass
class Predictor:
    layers: List[Layer]
    input_proj: Q4
    input_proj_bias: np.ndarray
    codec_embeddings: List[Q4]
    lm_heads: List[Q4]
    final_norm: np.ndarray
    rope_cos: np.ndarray
    rope_sin: np.ndarray
    hidden: int = 1024
    n_heads: int = 16
    n_kv_heads: int = 8
    head_dim: int = 128
    inter: int = 3072
    vocab: int = 2048


def make_talker(seed=1, n_layers=28, hidden=2048, inter=6144, vocab=3072, text_vocab=151936,
                text_hidden=2048, rope_max_pos=32768):
    """Talker of the 1.7B shape (model/1.7B/config.json: 28 layers, hidden
    2048, 16/8 heads of 128, FFN 6144, codec vocab 3072, text vocab 151936)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    layers = [make_layer(rng, hidden, inter=inter) for _ in range(n_layers)]
    cos, sin = rope_table(128, rope_max_pos)
    return Talker(
        layers=layers,
        codec_embedding=q4_random(rng, vocab, hidden),
        text_embedding=q4_random(rng, text_vocab, text_hidden),
        text_fc1=q4_random(rng, text_hidden, hidden),
        text_fc2=q4_random(rng, hidden, hidden),
        text_fc1_bias=bias(rng, hidden), text_fc2_bias=bias(rng, hidden),
        codec_head=q4_random(rng, hidden, vocab),
        final_norm=gamma(rng, hidden), rope_cos=cos, rope_sin=sin,
        hidden=hidden, text_hidden=text_hidden, inter=inter, vocab=vocab)


def make_predictor(seed=2, n_layers=5, hidden=1024, inter=3072, vocab=2048, n_groups=15,
                   talker_hidden=2048, rope_max_pos=65536):
    """Code predictor of the 1.7B shape (model/1.7B/config.json: 5 layers,
    hidden 1024, FFN 3072, 2048 codes, 15 codebooks, input projection from
    the talker's 2048)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    layers = [make_layer(rng, hidden, inter=inter) for _ in range(n_layers)]
    cos, sin = rope_table(128, rope_max_pos)
    return Predictor(
        layers=layers,
        input_proj=q4_random(rng, talker_hidden, hidden),
        input_proj_bias=bias(rng, hidden),
        codec_embeddings=[q4_random(rng, vocab, talker_hidden) for _ in range(n_groups)],
        lm_heads=[q4_random(rng, hidden, vocab) for _ in range(n_groups)],
        final_norm=gamma(rng, hidden), rope_cos=cos, rope_sin=sin,
        hidden=hidden, inter=inter, vocab=vocab)


# ---------------------------------------------------------------------------
# speech decoder (SpeechDecoderWeights, decoder.rs:22-66): f32 weights
# ---------------------------------------------------------------------------

@dataclass
class Conv1d:
    """`Conv1dWeight` (conv.rs:29-38): weight [out][in][k]."""
    weight: np.ndarray
    bias: np.ndarray
    in_channels: int
    out_channels: int
    kernel_size: int
    stride: int = 1
    padding: int = 0
    dilation: int = 1


@dataclass
class ConvT1d:
    """`ConvTranspose1dWeight` (conv.rs:235-243): weight [in][out][k]."""
    weight: np.ndarray
    bias: np.ndarray
    in_channels: int
    out_channels: int
    kernel_size: int
    stride: int
    padding: int = 0


@dataclass
class DwConv:
    """`DepthwiseConv1dWeight` (conv.rs:351-357): weight [c][k]."""
    weight: np.ndarray
    bias: np.ndarray
    channels: int
    kernel_size: int
    padding: int


@dataclass
class DecLayer:
    q_proj: np.ndarray
    k_proj: np.ndarray
    v_proj: np.ndarray
    o_proj: np.ndarray
    gate_proj: np.ndarray
    up_proj: np.ndarray
    down_proj: np.ndarray
    input_norm: np.ndarray
    post_attn_norm: np.ndarray
    attn_scale: np.ndarray
    mlp_scale: np.ndarray


@dataclass
class Upsample:
    conv_t: ConvT1d
    dw_conv: DwConv
    norm_w: np.ndarray
    norm_b: np.ndarray
    pw1_w: np.ndarray      # [channels][inner]
    pw1_b: np.ndarray
    pw2_w: np.ndarray      # [inner][channels]
    pw2_b: np.ndarray
    gamma: np.ndarray
    channels: int
    inner: int


@dataclass
class VocosRes:
    act1_alpha: np.ndarray
    act1_beta: np.ndarray
    conv1: Conv1d
    act2_alpha: np.ndarray
    act2_beta: np.ndarray
    conv2: Conv1d


@dataclass
class VocosBlock:
    pre_snake_alpha: np.ndarray
    pre_snake_beta: np.ndarray
    upsample: ConvT1d
    residuals: List[VocosRes]


@dataclass
class Decoder:
    first_codebook: np.ndarray       # [codebook_size][codebook_dim]
    first_output_proj: np.ndarray    # [codebook_dim][vq_dim]
    rest_codebooks: List[np.ndarray]
    rest_output_proj: np.ndarray
    pre_conv: Conv1d
    tf_input_w: np.ndarray           # [latent][hidden]
    tf_input_b: np.ndarray
    tf_layers: List[DecLayer]
    tf_norm: np.ndarray
    tf_output_w: np.ndarray          # [hidden][latent]
    tf_output_b: np.ndarray
    upsample: List[Upsample]
    vocos_init: Conv1d
    vocos_blocks: List[VocosBlock]
    final_snake_alpha: np.ndarray
    final_snake_beta: np.ndarray
    output_conv: Conv1d
    rope_cos: np.ndarray             # [max_pos][head_dim/2]
    rope_sin: np.ndarray
    hidden: int = 512
    n_heads: int = 16
    head_dim: int = 64
    inter: int = 1024
    sliding_window: int = 72
    codebook_dim: int = 256
    codebook_size: int = 2048
    vq_dim: int = 512
    latent: int = 1024

    @property
    def upsample_factor(self) -> int:
        f = 1
        for u in self.upsample:
            f *= u.conv_t.stride
        for b in self.vocos_blocks:
            f *= b.upsample.stride
        return f


def _mat(rng, k, n, gain=1.0):
    return (rng.standard_normal((k, n), dtype=np.float32) * np.float32(gain / np.sqrt(k))).astype(np.float32)


def _vec(rng, n, mean=0.0, sigma=0.02):
    return (mean + sigma * rng.standard_normal(n)).astype(np.float32)


def _conv(rng, ic, oc, k, dilation=1, gain=1.0):
    w = (rng.standard_normal((oc, ic, k), dtype=np.float32) * np.float32(gain / np.sqrt(ic * k))).astype(np.float32)
    return Conv1d(w, _vec(rng, oc), ic, oc, k, 1, 0, dilation)


def _convt(rng, ic, oc, k, s, gain=1.0):
    w = (rng.standard_normal((ic, oc, k), dtype=np.float32) * np.float32(gain / np.sqrt(ic * k / s))).astype(np.float32)
    return ConvT1d(w, _vec(rng, oc), ic, oc, k, s, 0)


def make_decoder(seed=7, latent=1024, hidden=512, n_heads=16, head_dim=64, inter=1024, n_tf_layers=8,
                 sliding_window=72, codebook_size=2048, codebook_dim=256, vq_dim=512, n_rest=15, n_upsample=2,
                 vocos=(1536, 768, 384, 192, 96), rates=(8, 5, 4, 3), dilations=(1, 3, 9), rope_max_pos=8000):
    """Random decoder of the 12 Hz speech tokenizer's shapes (loader.rs:540-720):
    16 VQ codebooks -> 512, pre-conv to 1024, an 8-layer transformer (512
    hidden, 16 x 64 heads, sliding window 72), two 2x ConvTranspose +
    ConvNeXt upsamplers, Vocos (1536 -> 96 channels, rates 8, 5, 4, 3),
    1920 samples per frame.  Scales keep every stage's activations O(1)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    A = n_heads * head_dim
    layers = []
    for _ in range(n_tf_layers):
        layers.append(DecLayer(
            _mat(rng, hidden, A), _mat(rng, hidden, A), _mat(rng, hidden, A), _mat(rng, A, hidden),
            _mat(rng, hidden, inter), _mat(rng, hidden, inter), _mat(rng, inter, hidden),
            _vec(rng, hidden, 1.0, 0.05), _vec(rng, hidden, 1.0, 0.05),
            _vec(rng, hidden, 0.1, 0.02), _vec(rng, hidden, 0.1, 0.02)))
    ups = []
    for _ in range(n_upsample):
        inner = 4 * latent
        ups.append(Upsample(
            _convt(rng, latent, latent, 2, 2),
            DwConv((rng.standard_normal((latent, 7), dtype=np.float32) / np.float32(np.sqrt(7))).astype(np.float32),
                   _vec(rng, latent), latent, 7, 3),
            _vec(rng, latent, 1.0, 0.05), _vec(rng, latent), _mat(rng, latent, inner), _vec(rng, inner),
            _mat(rng, inner, latent), _vec(rng, latent), _vec(rng, latent, 0.1, 0.02), latent, inner))
    blocks = []
    for b, r in enumerate(rates[:len(vocos) - 1]):
        ic, oc = vocos[b], vocos[b + 1]
        res = [VocosRes(_vec(rng, oc, 0.0, 0.1), _vec(rng, oc, 0.0, 0.1), _conv(rng, oc, oc, 7, d, 0.5),
                        _vec(rng, oc, 0.0, 0.1), _vec(rng, oc, 0.0, 0.1), _conv(rng, oc, oc, 1, 1, 0.5))
               for d in dilations]
        blocks.append(VocosBlock(_vec(rng, ic, 0.0, 0.1), _vec(rng, ic, 0.0, 0.1), _convt(rng, ic, oc, 2 * r, r), res))
    last = vocos[len(blocks)]
    cos, sin = rope_table(head_dim, rope_max_pos, theta=10000.0)
    return Decoder(
        first_codebook=(0.5 * rng.standard_normal((codebook_size, codebook_dim))).astype(np.float32),
        first_output_proj=_mat(rng, codebook_dim, vq_dim),
        rest_codebooks=[(0.15 * rng.standard_normal((codebook_size, codebook_dim))).astype(np.float32)
                        for _ in range(n_rest)],
        rest_output_proj=_mat(rng, codebook_dim, vq_dim),
        pre_conv=_conv(rng, vq_dim, latent, 3),
        tf_input_w=_mat(rng, latent, hidden), tf_input_b=_vec(rng, hidden),
        tf_layers=layers, tf_norm=_vec(rng, hidden, 1.0, 0.05),
        tf_output_w=_mat(rng, hidden, latent), tf_output_b=_vec(rng, latent),
        upsample=ups, vocos_init=_conv(rng, latent, vocos[0], 7),
        vocos_blocks=blocks,
        final_snake_alpha=_vec(rng, last, 0.0, 0.1), final_snake_beta=_vec(rng, last, 0.0, 0.1),
        output_conv=_conv(rng, last, 1, 7, 1, 0.15),
        rope_cos=cos, rope_sin=sin,
        hidden=hidden, n_heads=n_heads, head_dim=head_dim, inter=inter, sliding_window=sliding_window,
        codebook_dim=codebook_dim, codebook_size=codebook_size, vq_dim=vq_dim, latent=latent)
