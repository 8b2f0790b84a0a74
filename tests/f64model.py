"""Float64 numpy model of the decode path, used to pin the oracle's composed
functions (talker step, prefill, codec head, text embedding, predictor
chain, frame) beyond its own restatement.

Written in matrix form from the model's mathematics, not from the oracle's
loops: a dropped residual or bias, a wrong RoPE pairing or sign, a wrong
GQA head mapping or a transposed weight in the oracle shows up as an O(1)
difference against this model, while f32 rounding stays near 1e-6.

Reference semantics followed (file:line in the reference crate):
  Q4 layout input-major, low nibble = even column      gemv.rs:26-31, 249-287
  RMSNorm x / sqrt(mean(x^2) + 1e-6) * gamma           gemv.rs:445-454
  QK-norm per head, shared [128] gamma                 talker.rs:89-99
  rotate-half RoPE, pairs (i, i + 64), theta 1e6      rope.rs:26-38, 79-92
  K cached after norm + RoPE, V raw                     talker.rs:299-302
  decode attention, kv head = q head / 2, no mask      talker.rs:304-331
  SwiGLU silu(g) * u                                    talker.rs:338-349
  final norm hidden -> codec head                       talker.rs:352-359, 647
  text embedding -> fc1 + b -> SiLU -> fc2 + b           talker.rs:105-116
  predictor: proj(h) = h W + b, 2-row prefill, 14 steps,
  head g, argmax with last-max ties                    code_predictor.rs:51-61, 218-273, 335-341
  frame: semantic + sum of 15 code embeddings + text    generate_new.rs:606-675
"""
import numpy as np


def dense(w):
    """Q4 weight -> float64 [k][n]: byte j of group g holds column 32g + 2j
    in its low nibble and 32g + 2j + 1 in its high nibble; value
    (nibble - 8) * scale(row, group)."""
    g = w.n // 32
    p = w.packed.reshape(w.k, g, 16).astype(np.int64)
    q = np.stack([(p & 0xF) - 8, (p >> 4) - 8], axis=-1).reshape(w.k, g, 32)
    s = w.scales.view(np.float16).astype(np.float64).reshape(w.k, g, 1)
    out = np.zeros((w.k, w.n))
    out[:, : g * 32] = (q * s).reshape(w.k, g * 32)
    return out


def row(w, r):
    """One dequantised row of a Q4 table (an embedding lookup)."""
    return dense_rows(w, [r])[0]


def dense_rows(w, rows):
    g = w.n // 32
    p = w.packed[rows].reshape(len(rows), g, 16).astype(np.int64)
    q = np.stack([(p & 0xF) - 8, (p >> 4) - 8], axis=-1).reshape(len(rows), g, 32)
    s = w.scales[rows].view(np.float16).astype(np.float64).reshape(len(rows), g, 1)
    out = np.zeros((len(rows), w.n))
    out[:, : g * 32] = (q * s).reshape(len(rows), g * 32)
    return out


def gam(g):
    return g.view(np.float16).astype(np.float64)


def rms(x, g):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + 1e-6) * gam(g)


def silu(x):
    return x / (1.0 + np.exp(-x))


def rope(x, pos, theta=1_000_000.0):
    """x [..., heads, 128] at integer position pos; pairs (i, i + 64)."""
    half = x.shape[-1] // 2
    freq = theta ** (-2.0 * np.arange(half) / x.shape[-1])
    c, s = np.cos(pos * freq), np.sin(pos * freq)
    a, b = x[..., :half], x[..., half:]
    return np.concatenate([a * c - b * s, b * c + a * s], axis=-1)


def kv_head_map(nh, nkv):
    """GQA: q head h reads kv head h / (nh / nkv)."""
    return np.arange(nh) * nkv // nh


def softmax(v):
    e = np.exp(v - v.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


class Layer64:
    def __init__(self, L, n_heads, n_kv, hd):
        self.wq, self.wk, self.wv, self.wo = dense(L.q_proj), dense(L.k_proj), dense(L.v_proj), dense(L.o_proj)
        self.wg, self.wu, self.wd = dense(L.gate_proj), dense(L.up_proj), dense(L.down_proj)
        self.L = L
        self.nh, self.nkv, self.hd = n_heads, n_kv, hd

    def step(self, x, pos, K, V):
        """One position through the layer; K, V: lists of [n_kv][hd] the
        position's K (normed, rotated) and V are appended to."""
        L, nh, nkv, hd = self.L, self.nh, self.nkv, self.hd
        h = rms(x, L.input_norm)
        q = rope(rms((h @ self.wq).reshape(nh, hd), L.q_norm), pos)
        k = rope(rms((h @ self.wk).reshape(nkv, hd), L.k_norm), pos)
        v = (h @ self.wv).reshape(nkv, hd)
        K.append(k)
        V.append(v)
        Ks, Vs = np.stack(K), np.stack(V)              # [len][nkv][hd]
        kvh = kv_head_map(nh, nkv)
        scores = np.einsum("hd,lhd->hl", q, Ks[:, kvh, :]) / np.sqrt(hd)
        att = np.einsum("hl,lhd->hd", softmax(scores), Vs[:, kvh, :]).reshape(nh * hd)
        x = x + att @ self.wo
        h = rms(x, L.post_attn_norm)
        return x + (silu(h @ self.wg) * (h @ self.wu)) @ self.wd


class Talker64:
    def __init__(self, t):
        self.t = t
        self.layers = [Layer64(L, t.n_heads, t.n_kv_heads, t.head_dim) for L in t.layers]
        self.head = dense(t.codec_head)
        self.K = [[] for _ in t.layers]
        self.V = [[] for _ in t.layers]

    def load_kv(self, K, V):
        """K, V [layers][len][n_kv][hd] (any float type)."""
        for l in range(len(self.layers)):
            self.K[l] = [np.asarray(k, np.float64) for k in K[l]]
            self.V[l] = [np.asarray(v, np.float64) for v in V[l]]

    def hidden_at(self, x, pos):
        x = np.asarray(x, np.float64)
        for l, L in enumerate(self.layers):
            x = L.step(x, pos, self.K[l], self.V[l])
        return rms(x, self.t.final_norm)

    def step(self, emb, pos):
        """forward_with_embedding: [normed hidden | codec logits]."""
        h = self.hidden_at(emb, pos)
        return np.concatenate([h, h @ self.head])

    def prefill(self, X, start):
        """Causal prefill of rows X at positions start.. ; normed hidden of the
        last row (row-by-row through all layers equals layer-by-layer)."""
        h = None
        for i, x in enumerate(np.asarray(X, np.float64)):
            h = self.hidden_at(x, start + i)
        return h

    def codec_head(self, h):
        return np.asarray(h, np.float64) @ self.head

    def embed_text(self, tok):
        t = self.t
        e = row(t.text_embedding, tok)
        h1 = e @ dense(t.text_fc1) + t.text_fc1_bias.astype(np.float64)
        return silu(h1) @ dense(t.text_fc2) + t.text_fc2_bias.astype(np.float64)


class Predictor64:
    def __init__(self, p):
        self.p = p
        self.layers = [Layer64(L, p.n_heads, p.n_kv_heads, p.head_dim) for L in p.layers]
        self.proj = dense(p.input_proj)
        self.bias = p.input_proj_bias.astype(np.float64)
        self.heads = [dense(w) for w in p.lm_heads]

    def project(self, v):
        return np.asarray(v, np.float64) @ self.proj + self.bias

    def _hidden(self, x, pos, K, V):
        for l, L in enumerate(self.layers):
            x = L.step(x, pos, K[l], V[l])
        return rms(x, self.p.final_norm)

    def chain_logits(self, talker_hidden, semantic, codes):
        """Teacher-forced chain: step g's input embeds codes[g-1] (the chain's
        own code for step g-1).  Returns the 15 logit vectors."""
        K = [[] for _ in self.layers]
        V = [[] for _ in self.layers]
        self._hidden(self.project(talker_hidden), 0, K, V)
        h = self._hidden(self.project(semantic), 1, K, V)
        out = [h @ self.heads[0]]
        for g in range(1, len(self.heads)):
            e = row(self.p.codec_embeddings[g - 1], int(codes[g - 1]))
            h = self._hidden(self.project(e), g + 1, K, V)
            out.append(h @ self.heads[g])
        return out

    def predict_logits(self, talker_hiddens):
        """predict_codes (code_predictor.rs:126-216) over successive calls:
        call t projects hidden t, runs the layers at position t against the
        cache the earlier calls left, and returns every head's logits."""
        K = [[] for _ in self.layers]
        V = [[] for _ in self.layers]
        out = []
        for t, th in enumerate(talker_hiddens):
            h = self._hidden(self.project(th), t, K, V)
            out.append([h @ w for w in self.heads])
        return out

    def embed_sum(self, codes):
        return sum(row(self.p.codec_embeddings[g], int(c)) for g, c in enumerate(codes))
