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
