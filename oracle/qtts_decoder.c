/*
 * qtts_decoder.c — CPU restatement of the reference's speech decoder
 * (decode_to_audio, decoder.rs:395-584, with the conv.rs kernels), test
 * infrastructure only: the oracle the HIP decoder is tested against.
 *
 * Each function follows the cited Rust function's floating-point operation
 * order for every output element (bias first, then the taps in the
 * reference's loop order), compiled with -ffp-contract=off.  Loops over
 * independent output rows are spread over threads; that never changes an
 * element's operation order.
 */
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "qtts_oracle.h"

/* ---- a small parallel-for over independent rows --------------------------- */

typedef void (*od_row_fn)(void *ctx, int64_t r0, int64_t r1);
struct od_job { od_row_fn fn; void *ctx; int64_t r0, r1; };

static void *od_run(void *p)
{
    struct od_job *j = (struct od_job *)p;
    j->fn(j->ctx, j->r0, j->r1);
    return NULL;
}

static int od_threads = 8;
void od_set_threads(int n) { od_threads = n < 1 ? 1 : (n > 64 ? 64 : n); }

static void od_parallel(int64_t rows, od_row_fn fn, void *ctx)
{
    int nt = od_threads;
    if (rows < 2 * nt) nt = rows < 1 ? 1 : (int)(rows < nt ? rows : nt);
    if (nt <= 1) {
        fn(ctx, 0, rows);
        return;
    }
    pthread_t th[64];
    struct od_job jobs[64];
    const int64_t per = (rows + nt - 1) / nt;
    int started = 0;
    for (int i = 0; i < nt; i++) {
        jobs[i].fn = fn;
        jobs[i].ctx = ctx;
        jobs[i].r0 = i * per;
        jobs[i].r1 = (i + 1) * per < rows ? (i + 1) * per : rows;
        if (jobs[i].r0 >= jobs[i].r1) break;
        if (pthread_create(&th[started], NULL, od_run, &jobs[i]) != 0) {
            od_run(&jobs[i]);
            continue;
        }
        started++;
    }
    for (int i = 0; i < started; i++) pthread_join(th[i], NULL);
}

/* ---- conv.rs kernels -------------------------------------------------------- */

struct conv_ctx { const float *in; int64_t in_len, out_len; const qtts_conv1d_host *w; float *out; };

/* causal_conv1d_range_scalar (conv.rs:191-228): pad = (k-1)*dilation on the
 * left; sum = bias, then ic ascending, k ascending. */
static void conv_rows(void *p, int64_t oc0, int64_t oc1)
{
    const struct conv_ctx *c = (const struct conv_ctx *)p;
    const qtts_conv1d_host *w = c->w;
    const int64_t K = w->kernel_size, dil = w->dilation, pad = (K - 1) * dil, IC = w->in_channels;
    for (int64_t oc = oc0; oc < oc1; oc++)
        for (int64_t o = 0; o < c->out_len; o++) {
            float sum = w->bias[oc];
            for (int64_t ic = 0; ic < IC; ic++) {
                const float *in_row = c->in + ic * c->in_len;
                const float *w_row = w->weight + (oc * IC + ic) * K;
                for (int64_t k = 0; k < K; k++) {
                    const int64_t in_pos = o + k * dil;
                    if (in_pos >= pad) {
                        const int64_t idx = in_pos - pad;
                        if (idx < c->in_len) sum += in_row[idx] * w_row[k];
                    }
                }
            }
            c->out[oc * c->out_len + o] = sum;
        }
}

void od_causal_conv1d(const float *in, int64_t in_len, const qtts_conv1d_host *w, float *out)
{
    struct conv_ctx c = {in, in_len, in_len, w, out};
    od_parallel(w->out_channels, conv_rows, &c);
}

struct convt_ctx { const float *in; int64_t in_len, out_len; const qtts_convt1d_host *w; float *out; };

/* conv_transpose1d_range_scalar (conv.rs:320-349) after the bias fill
 * (conv.rs:291-300): per output channel, ic ascending, input position
 * ascending, k ascending; zero inputs skipped. */
static void convt_rows(void *p, int64_t oc0, int64_t oc1)
{
    const struct convt_ctx *c = (const struct convt_ctx *)p;
    const qtts_convt1d_host *w = c->w;
    const int64_t K = w->kernel_size, S = w->stride, P = w->padding, OC = w->out_channels;
    for (int64_t oc = oc0; oc < oc1; oc++) {
        float *out_row = c->out + oc * c->out_len;
        for (int64_t o = 0; o < c->out_len; o++) out_row[o] = w->bias[oc];
        for (int64_t ic = 0; ic < w->in_channels; ic++) {
            const float *in_row = c->in + ic * c->in_len;
            const float *wb = w->weight + (ic * OC + oc) * K;
            for (int64_t i = 0; i < c->in_len; i++) {
                const float val = in_row[i];
                if (val == 0.0f) continue;
                for (int64_t k = 0; k < K; k++) {
                    const int64_t o = i * S + k - P;
                    if (o >= 0 && o < c->out_len) out_row[o] += val * wb[k];
                }
            }
        }
    }
}

/* conv_transpose1d (conv.rs:247-289): out_len = (in_len-1)*stride -
 * 2*padding + kernel. */
int64_t od_conv_transpose1d(const float *in, int64_t in_len, const qtts_convt1d_host *w, float *out)
{
    const int64_t out_len = (in_len - 1) * w->stride - 2 * (int64_t)w->padding + w->kernel_size;
    struct convt_ctx c = {in, in_len, out_len, w, out};
    od_parallel(w->out_channels, convt_rows, &c);
    return out_len;
}

/* dw_conv1d_range (conv.rs:398-432): causal pad kernel-1 whatever the
 * stored padding. */
void od_depthwise_conv1d(const float *in, int64_t len, const qtts_dwconv_host *w, float *out)
{
    const int64_t K = w->kernel_size, pad = K - 1;
    for (int64_t c = 0; c < w->channels; c++)
        for (int64_t o = 0; o < len; o++) {
            float sum = w->bias[c];
            for (int64_t k = 0; k < K; k++) {
                const int64_t in_pos = o + k;
                if (in_pos >= pad) {
                    const int64_t idx = in_pos - pad;
                    if (idx < len) sum += in[c * len + idx] * w->weight[c * K + k];
                }
            }
            out[c * len + o] = sum;
        }
}

struct gemm_ctx { const float *a, *b, *bias; int64_t n, k; float *c; };

/* f32_gemm_block_scalar (conv.rs:501-526) after the bias prefill: row m of
 * C = bias[m] + sum over kk ascending of a[m][kk] * b[kk][:], zero a skipped. */
static void gemm_rows(void *p, int64_t m0, int64_t m1)
{
    const struct gemm_ctx *g = (const struct gemm_ctx *)p;
    for (int64_t m = m0; m < m1; m++) {
        float *crow = g->c + m * g->n;
        for (int64_t j = 0; j < g->n; j++) crow[j] = g->bias[m];
        for (int64_t kk = 0; kk < g->k; kk++) {
            const float av = g->a[m * g->k + kk];
            if (av == 0.0f) continue;
            const float *brow = g->b + kk * g->n;
            for (int64_t j = 0; j < g->n; j++) crow[j] += av * brow[j];
        }
    }
}

/* f32_gemm_bias (conv.rs:434-499): C[m][n] = bias[m] + A[m][k] B[k][n]. */
void od_gemm_bias(const float *a, const float *b, const float *bias, int64_t m, int64_t n, int64_t k, float *c)
{
    struct gemm_ctx g = {a, b, bias, n, k, c};
    od_parallel(m, gemm_rows, &g);
}

/* snake_beta_range (conv.rs:620-640): x + exp(-beta) * sin(exp(alpha) x)^2. */
void od_snake_beta(const float *in, const float *alpha, const float *beta, int64_t channels, int64_t len, float *out)
{
    for (int64_t c = 0; c < channels; c++) {
        const float a = expf(alpha[c]);
        const float inv_b = expf(-beta[c]);
        for (int64_t t = 0; t < len; t++) {
            const float x = in[c * len + t];
            const float s = sinf(a * x);
            out[c * len + t] = x + inv_b * s * s;
        }
    }
}

/* gelu (conv.rs:692-694): x * 0.5 * (1 + tanh(x * 0.7071067811865476)). */
float od_gelu(float x) { return x * 0.5f * (1.0f + tanhf(x * 0.7071067811865476f)); }

/* ---- decoder.rs helpers ------------------------------------------------------ */

/* rms_norm_f32 (decoder.rs:589-598). */
static void rms_norm_f32(const float *x, const float *gamma, int64_t n, float eps, float *out)
{
    float ss = 0.0f;
    for (int64_t i = 0; i < n; i++) ss += x[i] * x[i];
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int64_t i = 0; i < n; i++) out[i] = x[i] * inv * gamma[i];
}

/* f32_gemv / f32_gemv_bias (decoder.rs:601-627): w is [k][n]. */
static void gemv_f32(const float *x, const float *w, int64_t k, int64_t n, const float *bias, float *out)
{
    for (int64_t j = 0; j < n; j++) out[j] = bias ? bias[j] : 0.0f;
    for (int64_t i = 0; i < k; i++) {
        const float v = x[i];
        if (v == 0.0f) continue;
        const float *row = w + i * n;
        for (int64_t j = 0; j < n; j++) out[j] += v * row[j];
    }
}

/* apply_rope_split_half (decoder.rs:631-655): positions past the table are
 * left unrotated. */
static void rope_split_half(float *d, int64_t heads, int64_t hd, int64_t pos, const float *cs, const float *sn,
                            int64_t table_len)
{
    const int64_t half = hd / 2, off = pos * half;
    if (off + half > table_len) return;
    for (int64_t h = 0; h < heads; h++) {
        float *b = d + h * hd;
        for (int64_t i = 0; i < half; i++) {
            const float x0 = b[i], x1 = b[half + i], c = cs[off + i], s = sn[off + i];
            b[i] = x0 * c - x1 * s;
            b[half + i] = x1 * c + x0 * s;
        }
    }
}

/* warmup_trim_len (decoder.rs:661-666). */
int64_t od_warmup_trim_len(int64_t tv, int64_t total, int64_t out_len)
{
    if (total == 0) return 0;
    const int64_t cut = tv * out_len / total;
    return cut < out_len ? cut : out_len;
}

/* layer_norm_channel_first (decoder.rs:668-690). */
void od_layer_norm_cf(const float *in, const float *gamma, const float *beta, int64_t channels, int64_t len,
                      float eps, float *out)
{
    for (int64_t t = 0; t < len; t++) {
        float mean = 0.0f;
        for (int64_t c = 0; c < channels; c++) mean += in[c * len + t];
        mean /= (float)channels;
        float var = 0.0f;
        for (int64_t c = 0; c < channels; c++) {
            const float d = in[c * len + t] - mean;
            var += d * d;
        }
        const float inv_std = 1.0f / sqrtf(var / (float)channels + eps);
        for (int64_t c = 0; c < channels; c++) out[c * len + t] = (in[c * len + t] - mean) * inv_std * gamma[c] + beta[c];
    }
}

/* codebook_lookup (decoder.rs:147-191): [vq_dim][T] channel-first. */
static void codebook_lookup(const qtts_decoder_host *w, const uint32_t *codes, int64_t T, float *out)
{
    const int64_t D = w->codebook_dim, V = w->vq_dim;
    float *proj = malloc(sizeof(float) * V), *sum = malloc(sizeof(float) * D);
    memset(out, 0, sizeof(float) * V * T);
    for (int64_t s = 0; s < T; s++) {
        gemv_f32(w->first_codebook + (int64_t)codes[s] * D, w->first_output_proj, D, V, NULL, proj);
        for (int64_t c = 0; c < V; c++) out[c * T + s] += proj[c];
    }
    for (int64_t s = 0; s < T; s++) {
        for (int64_t d = 0; d < D; d++) sum[d] = 0.0f;
        for (int g = 0; g < w->n_rest; g++) {
            const float *e = w->rest_codebooks[g] + (int64_t)codes[(int64_t)(g + 1) * T + s] * D;
            for (int64_t d = 0; d < D; d++) sum[d] += e[d];
        }
        gemv_f32(sum, w->rest_output_proj, D, V, NULL, proj);
        for (int64_t c = 0; c < V; c++) out[c * T + s] += proj[c];
    }
    free(proj);
    free(sum);
}

struct tf_ctx {
    const qtts_decoder_host *w;
    const qtts_dec_layer_host *L;
    int64_t T;
    float *x, *q, *k, *v;
};

/* one position's attention + o-proj + layer scale (decoder.rs:264-297) */
static void tf_attn_rows(void *p, int64_t t0, int64_t t1)
{
    const struct tf_ctx *c = (const struct tf_ctx *)p;
    const qtts_decoder_host *w = c->w;
    const int64_t H = w->hidden, A = (int64_t)w->n_heads * w->head_dim, hd = w->head_dim;
    const float scale = 1.0f / sqrtf((float)hd);
    float *out = malloc(sizeof(float) * A), *o = malloc(sizeof(float) * H), *sc = malloc(sizeof(float) * (c->T + 1));
    for (int64_t t = t0; t < t1; t++) {
        const int64_t start = t + 1 > w->sliding_window ? t + 1 - w->sliding_window : 0;
        const int64_t n = t + 1 - start;
        for (int64_t i = 0; i < A; i++) out[i] = 0.0f;
        for (int64_t h = 0; h < w->n_heads; h++) {
            const float *qv = c->q + t * A + h * hd;
            for (int64_t s = 0; s < n; s++) {
                const float *kv = c->k + (start + s) * A + h * hd;
                float dot = 0.0f;
                for (int64_t d = 0; d < hd; d++) dot += qv[d] * kv[d];
                sc[s] = dot * scale;
            }
            oq_softmax_raw(sc, n);
            for (int64_t s = 0; s < n; s++) {
                const float *vv = c->v + (start + s) * A + h * hd;
                for (int64_t d = 0; d < hd; d++) out[h * hd + d] += sc[s] * vv[d];
            }
        }
        /* the new x rows are written after every position's attention */
        gemv_f32(out, c->L->o_proj, A, H, NULL, o);
        for (int64_t j = 0; j < H; j++) c->q[t * A + j] = o[j];   /* park o in q's row (q is done) */
    }
    free(out);
    free(o);
    free(sc);
}

/* decoder_transformer (decoder.rs:198-340): x_ch [latent][T] -> [latent][T] */
static void decoder_transformer(const qtts_decoder_host *w, const float *x_ch, int64_t T, float *out_ch)
{
    const int64_t in_dim = w->latent, H = w->hidden, A = (int64_t)w->n_heads * w->head_dim, I = w->inter;
    float *xr = malloc(sizeof(float) * T * in_dim), *x = malloc(sizeof(float) * T * H);
    float *q = malloc(sizeof(float) * T * (A > H ? A : H)), *k = malloc(sizeof(float) * T * A);
    float *v = malloc(sizeof(float) * T * A), *xn = malloc(sizeof(float) * H);
    float *g = malloc(sizeof(float) * I), *u = malloc(sizeof(float) * I), *m = malloc(sizeof(float) * H);
    float *orow = malloc(sizeof(float) * in_dim);
    const int64_t rope_len = w->rope_max_pos * (w->head_dim / 2);
    for (int64_t c = 0; c < in_dim; c++)
        for (int64_t t = 0; t < T; t++) xr[t * in_dim + c] = x_ch[c * T + t];
    for (int64_t t = 0; t < T; t++) gemv_f32(xr + t * in_dim, w->tf_input_w, in_dim, H, w->tf_input_b, x + t * H);
    for (int li = 0; li < w->n_tf_layers; li++) {
        const qtts_dec_layer_host *L = &w->tf_layers[li];
        for (int64_t t = 0; t < T; t++) {
            rms_norm_f32(x + t * H, L->input_norm, H, 1e-5f, xn);
            gemv_f32(xn, L->q_proj, H, A, NULL, q + t * A);
            gemv_f32(xn, L->k_proj, H, A, NULL, k + t * A);
            gemv_f32(xn, L->v_proj, H, A, NULL, v + t * A);
        }
        for (int64_t t = 0; t < T; t++) {
            rope_split_half(q + t * A, w->n_heads, w->head_dim, t, w->rope_cos, w->rope_sin, rope_len);
            rope_split_half(k + t * A, w->n_heads, w->head_dim, t, w->rope_cos, w->rope_sin, rope_len);
        }
        /* attention reads q/k/v only; each position's o-proj output lands in
         * q's row t after that row's attention is done */
        struct tf_ctx c = {w, L, T, x, q, k, v};
        od_parallel(T, tf_attn_rows, &c);
        for (int64_t t = 0; t < T; t++)
            for (int64_t j = 0; j < H; j++) x[t * H + j] += q[t * A + j] * L->attn_scale[j];
        for (int64_t t = 0; t < T; t++) {
            rms_norm_f32(x + t * H, L->post_attn_norm, H, 1e-5f, xn);
            gemv_f32(xn, L->gate_proj, H, I, NULL, g);
            gemv_f32(xn, L->up_proj, H, I, NULL, u);
            for (int64_t j = 0; j < I; j++) {
                const float gv = g[j];
                g[j] = (gv / (1.0f + expf(-gv))) * u[j];
            }
            gemv_f32(g, L->down_proj, I, H, NULL, m);
            for (int64_t j = 0; j < H; j++) x[t * H + j] += m[j] * L->mlp_scale[j];
        }
    }
    for (int64_t t = 0; t < T; t++) {
        rms_norm_f32(x + t * H, w->tf_norm, H, 1e-5f, xn);
        gemv_f32(xn, w->tf_output_w, H, in_dim, w->tf_output_b, orow);
        for (int64_t c = 0; c < in_dim; c++) out_ch[c * T + t] = orow[c];
    }
    free(xr); free(x); free(q); free(k); free(v); free(xn); free(g); free(u); free(m); free(orow);
}

/* convnext_forward (decoder.rs:346-388) on [ch][len] in place */
static void convnext(const qtts_upsample_host *u, float *sig, int64_t len)
{
    const int64_t ch = u->channels, inner = u->inner;
    float *dw = malloc(sizeof(float) * ch * len), *nm = malloc(sizeof(float) * ch * len);
    float *w1t = malloc(sizeof(float) * ch * inner), *w2t = malloc(sizeof(float) * ch * inner);
    float *h = malloc(sizeof(float) * inner * len), *o = malloc(sizeof(float) * ch * len);
    od_depthwise_conv1d(sig, len, &u->dw_conv, dw);
    od_layer_norm_cf(dw, u->norm_w, u->norm_b, ch, len, 1e-5f, nm);
    for (int64_t r = 0; r < ch; r++)            /* transpose2d(pw1_w, ch, inner) */
        for (int64_t c = 0; c < inner; c++) w1t[c * ch + r] = u->pw1_w[r * inner + c];
    od_gemm_bias(w1t, nm, u->pw1_b, inner, len, ch, h);
    for (int64_t i = 0; i < inner * len; i++) h[i] = od_gelu(h[i]);
    for (int64_t r = 0; r < inner; r++)         /* transpose2d(pw2_w, inner, ch) */
        for (int64_t c = 0; c < ch; c++) w2t[c * inner + r] = u->pw2_w[r * ch + c];
    od_gemm_bias(w2t, h, u->pw2_b, ch, len, inner, o);
    for (int64_t c = 0; c < ch; c++) {
        const float gm = u->gamma[c];
        for (int64_t t = 0; t < len; t++) sig[c * len + t] = sig[c * len + t] + gm * o[c * len + t];
    }
    free(dw); free(nm); free(w1t); free(w2t); free(h); free(o);
}

/* conv_transpose1d then the causal right crop of kernel - stride
 * (decoder.rs:472-486, 512-525): [out][in_len*stride...] */
static float *convt_crop(const float *in, int64_t in_len, const qtts_convt1d_host *w, int64_t *len_out)
{
    const int64_t full = (in_len - 1) * w->stride - 2 * (int64_t)w->padding + w->kernel_size;
    float *o = malloc(sizeof(float) * w->out_channels * full);
    od_conv_transpose1d(in, in_len, w, o);
    const int64_t crop = w->kernel_size - w->stride;
    int64_t len = full;
    if (crop > 0) {
        len = full - crop;
        for (int64_t c = 0; c < w->out_channels; c++) memmove(o + c * len, o + c * full, sizeof(float) * len);
    }
    *len_out = len;
    return o;
}

/* decode_to_audio (decoder.rs:395-584).  codes and warmup are [16][T] /
 * [16][Tv] codebook-major.  Writes *n_out samples to out (capacity cap);
 * returns 0, or -1 when cap is too small / the input is empty. */
int od_decode_to_audio(const qtts_decoder_host *w, const uint32_t *codes, int64_t T, const uint32_t *warmup,
                       int64_t Tv, float *out, int64_t cap, int64_t *n_out)
{
    *n_out = 0;
    if (T < 1) return 0;
    const int64_t n_cb = 1 + (int64_t)w->n_rest;
    const int use_warm = warmup && Tv > 0;
    const int64_t TT = use_warm ? Tv + T : T;
    uint32_t *work = malloc(sizeof(uint32_t) * n_cb * TT);
    for (int64_t g = 0; g < n_cb; g++) {
        if (use_warm) {
            memcpy(work + g * TT, warmup + g * Tv, sizeof(uint32_t) * Tv);
            memcpy(work + g * TT + Tv, codes + g * T, sizeof(uint32_t) * T);
        } else {
            memcpy(work + g * TT, codes + g * T, sizeof(uint32_t) * T);
        }
    }
    float *vq = malloc(sizeof(float) * w->vq_dim * TT);
    codebook_lookup(w, work, TT, vq);
    free(work);
    float *pre = malloc(sizeof(float) * w->pre_conv.out_channels * TT);
    od_causal_conv1d(vq, TT, &w->pre_conv, pre);
    free(vq);
    float *sig = malloc(sizeof(float) * w->latent * TT);
    decoder_transformer(w, pre, TT, sig);
    free(pre);
    int64_t len = TT;
    for (int i = 0; i < w->n_upsample; i++) {
        int64_t nl;
        float *o = convt_crop(sig, len, &w->upsample[i].conv_t, &nl);
        free(sig);
        sig = o;
        len = nl;
        convnext(&w->upsample[i], sig, len);
    }
    float *v = malloc(sizeof(float) * w->vocos_init.out_channels * len);
    od_causal_conv1d(sig, len, &w->vocos_init, v);
    free(sig);
    sig = v;
    int64_t ch = w->vocos_init.out_channels;
    for (int b = 0; b < w->n_vocos_blocks; b++) {
        const qtts_vocos_block_host *vb = &w->vocos_blocks[b];
        float *sn = malloc(sizeof(float) * ch * len);
        od_snake_beta(sig, vb->pre_snake_alpha, vb->pre_snake_beta, ch, len, sn);
        free(sig);
        int64_t nl;
        sig = convt_crop(sn, len, &vb->upsample, &nl);
        free(sn);
        len = nl;
        ch = vb->upsample.out_channels;
        float *res = malloc(sizeof(float) * ch * len), *t1 = malloc(sizeof(float) * ch * len);
        float *t2 = malloc(sizeof(float) * ch * len);
        for (int r = 0; r < vb->n_residuals; r++) {
            const qtts_vocos_res_host *ru = &vb->residuals[r];
            memcpy(res, sig, sizeof(float) * ch * len);
            od_snake_beta(sig, ru->act1_alpha, ru->act1_beta, ch, len, t1);
            od_causal_conv1d(t1, len, &ru->conv1, t2);
            od_snake_beta(t2, ru->act2_alpha, ru->act2_beta, ch, len, t1);
            od_causal_conv1d(t1, len, &ru->conv2, sig);
            for (int64_t j = 0; j < ch * len; j++) sig[j] += res[j];
        }
        free(res); free(t1); free(t2);
    }
    float *sn = malloc(sizeof(float) * ch * len);
    od_snake_beta(sig, w->final_snake_alpha, w->final_snake_beta, ch, len, sn);
    float *audio = malloc(sizeof(float) * len);
    od_causal_conv1d(sn, len, &w->output_conv, audio);
    free(sn);
    free(sig);
    for (int64_t i = 0; i < len; i++) {
        const float s = audio[i];
        audio[i] = s < -1.0f ? -1.0f : (s > 1.0f ? 1.0f : s);
    }
    int64_t cut = use_warm ? od_warmup_trim_len(Tv, TT, len) : 0;
    const int64_t n = len - cut;
    int rc = 0;
    if (n > cap) rc = -1;
    else {
        memcpy(out, audio + cut, sizeof(float) * n);
        *n_out = n;
    }
    free(audio);
    return rc;
}
