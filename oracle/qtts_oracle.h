/*
 * qtts_oracle.h — CPU restatement of the QORA-TTS decode path (test
 * infrastructure only).
 *
 * This library is the oracle the HIP path is tested against, and the timed
 * CPU baseline.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it; the product library never links or calls it.
 *
 * Every function restates one Rust function of the reference crate
 * (swordreforge/QORA-TTS-12Hz-1.7B, src/...) in the same floating-point
 * operation order, compiled with -ffp-contract=off and without fast-math so
 * each f32 operation rounds once, as Rust's do.  Citations are file:line.
 *
 * Parity pinning (what checks each function beyond the restatement itself)
 * is listed per function in tests/test_oracle.py; functions with no such
 * check are marked "parity unpinned" there.
 */
#ifndef QTTS_ORACLE_H
#define QTTS_ORACLE_H

#include <stdint.h>
#include "../include/qtts.h"

#ifdef __cplusplus
extern "C" {
#endif

/* -- conversions and RNG -------------------------------------------------- */
float    oq_f16_to_f32(uint16_t h);              /* half::f16::to_f32         */
uint16_t oq_f32_to_f16(float f);                 /* half::f16::from_f32 (RNE) */
uint64_t oq_xorshift(uint64_t *state);           /* gemv.rs:693-698           */
float    oq_simple_rand(uint64_t *state);        /* generate_new.rs:17-22     */

/* -- Q4 kernels ---------------------------------------------------------- */
/* gemv.rs:249-287.  out[n] is overwritten (zeroed, then accumulated). */
void oq_gemv_q4_scalar(const float *x, const uint8_t *packed,
                       const uint16_t *scales, int64_t n, int64_t k0,
                       int64_t k1, float *out);
/* simd.rs:76-153 (AVX2), bit-identical to the scalar kernel per k-range.
 * Returns 0 if the host has no AVX2 (out untouched). */
int  oq_gemv_q4_avx2(const float *x, const uint8_t *packed,
                     const uint16_t *scales, int64_t n, int64_t k0,
                     int64_t k1, float *out);
/* gemv_q4_avx512 (simd.rs:203-269); 0 when the host lacks AVX-512. */
int  oq_gemv_q4_avx512(const float *x, const uint8_t *packed,
                       const uint16_t *scales, int64_t n, int64_t k0, int64_t k1,
                       float *out);
/* Inner-kernel ISA of the chunked GEMV (gemv.rs:230-243). */
enum { OQ_ISA_SCALAR = 0, OQ_ISA_AVX2 = 1, OQ_ISA_AVX512 = 2 };
int  oq_set_isa(int isa);     /* -1 restores the reference's choice; returns the ISA in use or -1 */
int  oq_get_isa(void);
/* gemv.rs:290-346 chunk policy.  `workers` is the pool size the policy
 * assumes (the reference's gpool::num_workers(), gpool.rs:29-34) and
 * `threads` the OS threads that execute chunks (0/1 = run in this thread).
 * Output bits depend on `workers` only. */
void oq_set_workers(int workers, int threads);
int  oq_get_workers(void);
void oq_gemv_q4(const float *x, const qtts_q4_host *w, float *out);
/* gemv.rs:349-412: each row is a full-k single-chunk GEMV. */
void oq_gemm_q4(const float *X, int64_t rows, const qtts_q4_host *w,
                float *Y);
/* gemv.rs:415-437 / talker.rs:119-150: dequantise row `row` (width
 * `width` columns, 32-column groups). */
void oq_embed_lookup_q4(const qtts_q4_host *w, int64_t row, int64_t width,
                        float *out);
/* gemv.rs:92-130 (used to build fixtures; never emits nibble 0). */
void oq_quantize_q4(const float *data, int64_t k, int64_t n, uint8_t *packed,
                    uint16_t *scales);

/* -- elementwise --------------------------------------------------------- */
void  oq_rms_norm_f16(const float *x, const uint16_t *gamma, int64_t n,
                      float *out);                         /* gemv.rs:445-454 */
void  oq_softmax_raw(float *s, int64_t n);                 /* gemv.rs:471-482 */
float oq_silu(float x);                                    /* gemv.rs:486-488 */
void  oq_qk_norm(float *data, int64_t heads, int64_t hd,
                 const uint16_t *gamma);                   /* talker.rs:89-99 */
/* rope.rs:11-41 (sections concatenated) == loader.rs:393-408. */
void  oq_rope_table(int64_t head_dim, int64_t max_pos, double theta,
                    float *cos_t, float *sin_t);
/* rope.rs:79-92 / code_predictor.rs:97-121 (rotate-half).  Skips (like
 * code_predictor.rs:107) when the table has no row `pos`. */
void  oq_rope_apply(float *data, int64_t heads, int64_t hd, int64_t pos,
                    const float *cos_t, const float *sin_t,
                    int64_t table_rows);

/* -- KV cache (gemv.rs:75-86: per layer [len][n_kv][hd] f32) ------------- */
typedef struct oq_kv {
    int32_t n_layers, n_kv, hd;
    int64_t cap;
    int64_t *len;          /* [n_layers]                 */
    float  **K, **V;       /* [n_layers][cap*n_kv*hd]    */
} oq_kv;
oq_kv *oq_kv_new(int32_t n_layers, int32_t n_kv, int32_t hd, int64_t cap);
void   oq_kv_free(oq_kv *kv);
void   oq_kv_reset(oq_kv *kv);
float *oq_kv_k(oq_kv *kv, int32_t layer);
float *oq_kv_v(oq_kv *kv, int32_t layer);
int64_t oq_kv_len(oq_kv *kv, int32_t layer);
void   oq_kv_set_len(oq_kv *kv, int64_t len);

/* -- talker -------------------------------------------------------------- */
/* talker.rs:263-360.  out = [hidden (normed) | logits]. */
int oq_talker_step(const qtts_talker_host *t, const float *emb, oq_kv *kv,
                   int64_t position, float *out);
/* talker.rs:379-482. */
int oq_talker_prefill(const qtts_talker_host *t, const float *X, int64_t seq,
                      oq_kv *kv, int64_t start_pos, float *hidden_out);
void oq_codec_head(const qtts_talker_host *t, const float *hidden,
                   float *logits);                       /* talker.rs:647 */
void oq_embed_text_token(const qtts_talker_host *t, uint32_t id,
                         float *out);                    /* talker.rs:105 */
void oq_embed_codec_token(const qtts_talker_host *t, uint32_t id,
                          float *out);                   /* talker.rs:152 */

/* -- code predictor ------------------------------------------------------ */
/* code_predictor.rs:218-273.  forced (NULL or [15]): when given, step g
 * (g = 1..14) embeds forced[g-1] instead of its own previous prediction;
 * codes_out always receives the predictions. */
int  oq_predictor_chain(const qtts_predictor_host *p, const float *th,
                        const float *sem, oq_kv *kv, uint32_t *codes_out,
                        const uint32_t *forced);
void oq_acoustic_embed_sum(const qtts_predictor_host *p,
                           const uint32_t *codes, int32_t n,
                           float *out);          /* code_predictor.rs:287-300 */
uint32_t oq_argmax_last(const float *v, int64_t n); /* code_predictor.rs:335 */

/* -- sampler ------------------------------------------------------------- */
/* generate_new.rs:771-862.  Returns QTTS_ERR_NAN where Rust would panic
 * (partial_cmp().unwrap() on NaN). */
int  oq_predict_codes(const qtts_predictor_host *p, const float *th, oq_kv *kv, float *logits);
int oq_sample_top_k(const float *logits, int64_t n, float temperature, int64_t top_k,
                    const uint32_t *prev, int64_t n_prev, float penalty, uint64_t *rng,
                    uint32_t *out);
int oq_sample_token(const float *logits, int64_t n,
                    const qtts_sample_params *p, const uint32_t *prev,
                    int64_t n_prev, uint64_t *rng, float temperature,
                    uint32_t *out);

/* -- frame loop body (generate_new.rs:606-675) --------------------------- */
typedef struct oq_gen {
    float   *logits;        /* [talker vocab], in/out        */
    float   *hidden;        /* [talker hidden], in/out       */
    uint32_t prev[16];      /* generate_new.rs:583           */
    uint64_t rng;
    int64_t  position;
    int64_t  frame_idx;
} oq_gen;
/* One frame.  text_add: the row added to the talker input.  forced (NULL or
 * [16]) feeds those codes downstream instead of the predictions; codes_out
 * receives the predictions.  *eos = 1 (and nothing else changes) when the
 * sampled code 0 is the EOS id and EOS is enabled. */
int oq_frame(const qtts_talker_host *t, const qtts_predictor_host *p,
             oq_kv *tkv, oq_kv *pkv, oq_gen *st, const qtts_sample_params *sp,
             const float *text_add, uint32_t *codes_out, int32_t *eos,
             const uint32_t *forced);

/* -- prompt construction (generate_new.rs:82-476) ------------------------ */
float oq_frame_temperature(const qtts_sample_params *sp, int64_t frame_idx);   /* :82-88 */
/* build_prefill_head (:222-237): role prefix + codec header, [9][hidden];
 * voice NULL -> the built-in speaker's header. */
void oq_build_prefill_head(const qtts_talker_host *t, uint32_t speaker_id, uint32_t language_id,
                           const float *voice, int64_t voice_len, float *out);
void oq_icl_layout(int64_t n_ref, int64_t n_text, int64_t n_frames, int64_t *icl_len,
                   int64_t *rem_len);                                          /* :120-128 */
/* build_icl_block (:140-195): codes [16][n_frames]. */
void oq_build_icl_block(const qtts_talker_host *t, const qtts_predictor_host *p, const uint32_t *ref_tokens,
                        int64_t n_ref, const uint32_t *text_tokens, int64_t n_text, const uint32_t *codes,
                        int64_t n_frames, float *icl, float *rem);
/* build_icl_prefix (:244-280): [n_ref][hidden]. */
void oq_build_icl_prefix(const qtts_talker_host *t, const qtts_predictor_host *p, const uint32_t *ref_tokens,
                         int64_t n_ref, const uint32_t *codes, int64_t n_frames, float *out);
/* build_trailing_text (:756-767): [max(n-1, 0) + 1][hidden]. */
void oq_build_trailing_text(const qtts_talker_host *t, const uint32_t *tokens, int64_t n, float *out);
/* prefill_custom_voice (:361-476) into kv from position 0; returns the
 * frame loop's start position (:560-565) or a negative status.  rows_out
 * (NULL or [position rows][hidden]) receives the prompt rows. */
int64_t oq_prefill_custom_voice(const qtts_talker_host *t, const uint32_t *text_tokens, int64_t n_text,
                                uint32_t speaker_id, uint32_t language_id, const float *voice, int64_t voice_len,
                                const float *icl_rows, int64_t n_icl, oq_kv *kv, float *hidden_out,
                                float *logits_out, float *rows_out);

/* -- speech decoder (qtts_decoder.c; decoder.rs, conv.rs) -------------------- */
void    od_set_threads(int n);
void    od_causal_conv1d(const float *in, int64_t in_len, const qtts_conv1d_host *w,
                         float *out);                                  /* conv.rs:114-228 */
int64_t od_conv_transpose1d(const float *in, int64_t in_len, const qtts_convt1d_host *w,
                            float *out);                               /* conv.rs:247-349 */
void    od_depthwise_conv1d(const float *in, int64_t len, const qtts_dwconv_host *w,
                            float *out);                               /* conv.rs:361-432 */
void    od_gemm_bias(const float *a, const float *b, const float *bias, int64_t m,
                     int64_t n, int64_t k, float *c);                  /* conv.rs:434-526 */
void    od_snake_beta(const float *in, const float *alpha, const float *beta,
                      int64_t channels, int64_t len, float *out);      /* conv.rs:545-640 */
float   od_gelu(float x);                                              /* conv.rs:692-694 */
void    od_layer_norm_cf(const float *in, const float *gamma, const float *beta,
                         int64_t channels, int64_t len, float eps, float *out); /* decoder.rs:668-690 */
int64_t od_warmup_trim_len(int64_t tv, int64_t total, int64_t out_len);  /* decoder.rs:661-666 */
/* decode_to_audio (decoder.rs:395-584): codes [n_rest+1][T] (+ warmup
 * [n_rest+1][Tv] or NULL) -> clamped samples, warmup portion trimmed. */
int     od_decode_to_audio(const qtts_decoder_host *w, const uint32_t *codes, int64_t T,
                           const uint32_t *warmup, int64_t Tv, float *out, int64_t cap,
                           int64_t *n_out);

#ifdef __cplusplus
}
#endif
#endif
