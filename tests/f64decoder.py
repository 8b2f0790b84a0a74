"""Float64 numpy model of the speech decoder (decode_to_audio,
decoder.rs:395-584; conv.rs kernels), written in array form from the
network's definition, not from the oracle's loops.  It pins the oracle's
decoder: a wrong tap offset, crop side, RoPE pairing, window bound, norm
axis or activation form moves the output by far more than f32 rounding.
"""
import numpy as np


def causal_conv(x, c):
    """out[oc][t] = b[oc] + sum_ic,k W[oc][ic][k] x[ic][t + k*d - (K-1)*d]."""
    x = np.asarray(x, np.float64)
    K, d = c.kernel_size, c.dilation
    pad = (K - 1) * d
    xp = np.concatenate([np.zeros((x.shape[0], pad)), x], axis=1)
    W = c.weight.astype(np.float64)
    L = x.shape[1]
    out = np.repeat(c.bias.astype(np.float64)[:, None], L, axis=1)
    for k in range(K):
        out += W[:, :, k] @ xp[:, k * d: k * d + L]
    return out


def conv_t(x, c):
    """out[oc][i*s + k - p] += sum_ic x[ic][i] W[ic][oc][k] (+ bias), uncropped."""
    x = np.asarray(x, np.float64)
    L = x.shape[1]
    n = (L - 1) * c.stride - 2 * c.padding + c.kernel_size
    out = np.repeat(c.bias.astype(np.float64)[:, None], n, axis=1)
    W = c.weight.astype(np.float64)
    for k in range(c.kernel_size):
        contrib = W[:, :, k].T @ x                      # [oc][L]
        pos = np.arange(L) * c.stride + k - c.padding
        ok = (pos >= 0) & (pos < n)
        out[:, pos[ok]] += contrib[:, ok]
    return out


def conv_t_crop(x, c):
    y = conv_t(x, c)
    crop = c.kernel_size - c.stride
    return y[:, : y.shape[1] - crop] if crop > 0 else y


def depthwise(x, c):
    x = np.asarray(x, np.float64)
    K = c.kernel_size
    xp = np.concatenate([np.zeros((x.shape[0], K - 1)), x], axis=1)
    W = c.weight.astype(np.float64)
    out = np.repeat(c.bias.astype(np.float64)[:, None], x.shape[1], axis=1)
    for k in range(K):
        out += W[:, k: k + 1] * xp[:, k: k + x.shape[1]]
    return out


def snake(x, alpha, beta):
    a = np.exp(alpha.astype(np.float64))[:, None]
    ib = np.exp(-beta.astype(np.float64))[:, None]
    return x + ib * np.sin(a * x) ** 2


def gelu(x):
    return x * 0.5 * (1.0 + np.tanh(x * 0.7071067811865476))


def rms_rows(x, g, eps=1e-5):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * g.astype(np.float64)


def layer_norm_cf(x, g, b, eps=1e-5):
    mu = x.mean(axis=0, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=0, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * g.astype(np.float64)[:, None] + b.astype(np.float64)[:, None]


def rope(x, heads, hd, cos, sin):
    """x [T][heads*hd]; rotate-half pairs (i, i + hd/2) at position t."""
    T = x.shape[0]
    half = hd // 2
    x = x.reshape(T, heads, hd).copy()
    c = cos[:T].astype(np.float64)[:, None, :]
    s = sin[:T].astype(np.float64)[:, None, :]
    a, b = x[..., :half].copy(), x[..., half:].copy()
    x[..., :half] = a * c - b * s
    x[..., half:] = b * c + a * s
    return x.reshape(T, heads * hd)


def transformer(d, x_ch):
    """x_ch [latent][T] -> [latent][T]"""
    x = x_ch.T @ d.tf_input_w.astype(np.float64) + d.tf_input_b.astype(np.float64)   # [T][hidden]
    T = x.shape[0]
    nh, hd, W = d.n_heads, d.head_dim, d.sliding_window
    t = np.arange(T)
    mask = (t[None, :] <= t[:, None]) & (t[None, :] > t[:, None] - W)
    for L in d.tf_layers:
        h = rms_rows(x, L.input_norm)
        q = rope(h @ L.q_proj.astype(np.float64), nh, hd, d.rope_cos, d.rope_sin).reshape(T, nh, hd)
        k = rope(h @ L.k_proj.astype(np.float64), nh, hd, d.rope_cos, d.rope_sin).reshape(T, nh, hd)
        v = (h @ L.v_proj.astype(np.float64)).reshape(T, nh, hd)
        s = np.einsum("thd,shd->hts", q, k) / np.sqrt(hd)
        s = np.where(mask[None], s, -np.inf)
        p = np.exp(s - s.max(axis=-1, keepdims=True))
        p /= p.sum(axis=-1, keepdims=True)
        att = np.einsum("hts,shd->thd", p, v).reshape(T, nh * hd)
        x = x + (att @ L.o_proj.astype(np.float64)) * L.attn_scale.astype(np.float64)
        h = rms_rows(x, L.post_attn_norm)
        g = h @ L.gate_proj.astype(np.float64)
        u = h @ L.up_proj.astype(np.float64)
        x = x + ((g / (1.0 + np.exp(-g)) * u) @ L.down_proj.astype(np.float64)) * L.mlp_scale.astype(np.float64)
    x = rms_rows(x, d.tf_norm)
    return (x @ d.tf_output_w.astype(np.float64) + d.tf_output_b.astype(np.float64)).T


def convnext(u, x):
    h = layer_norm_cf(depthwise(x, u.dw_conv), u.norm_w, u.norm_b)
    h = gelu(u.pw1_w.astype(np.float64).T @ h + u.pw1_b.astype(np.float64)[:, None])
    h = u.pw2_w.astype(np.float64).T @ h + u.pw2_b.astype(np.float64)[:, None]
    return x + u.gamma.astype(np.float64)[:, None] * h


def vq(d, codes):
    e0 = d.first_codebook[codes[0]].astype(np.float64)               # [T][D]
    rest = sum(d.rest_codebooks[g][codes[g + 1]].astype(np.float64) for g in range(len(d.rest_codebooks)))
    return (e0 @ d.first_output_proj.astype(np.float64) + rest @ d.rest_output_proj.astype(np.float64)).T


def decode(d, codes, warmup=None, clamp=True):
    codes = np.asarray(codes)
    tv = 0
    if warmup is not None:
        tv = warmup.shape[1]
        codes = np.concatenate([warmup, codes], axis=1)
    x = causal_conv(vq(d, codes), d.pre_conv)
    x = transformer(d, x)
    for u in d.upsample:
        x = convnext(u, conv_t_crop(x, u.conv_t))
    x = causal_conv(x, d.vocos_init)
    for b in d.vocos_blocks:
        x = conv_t_crop(snake(x, b.pre_snake_alpha, b.pre_snake_beta), b.upsample)
        for r in b.residuals:
            y = causal_conv(snake(x, r.act1_alpha, r.act1_beta), r.conv1)
            x = x + causal_conv(snake(y, r.act2_alpha, r.act2_beta), r.conv2)
    y = causal_conv(snake(x, d.final_snake_alpha, d.final_snake_beta), d.output_conv)[0]
    if clamp:
        y = np.clip(y, -1.0, 1.0)
    if tv:
        y = y[tv * len(y) // codes.shape[1]:]
    return y
