/*
 * qtts.h — C ABI of the MI355X (gfx950) decode path for QORA-TTS 12 Hz 1.7B.
 *
 * The path covered is the per-frame autoregressive decode: the 28-layer
 * Talker step and the 5-layer code predictor's 15-codebook chain, with the
 * talker sampler between them.  Every entry point below replaces one Rust
 * function of the reference crate (cited as file:line).
 *
 * Conventions (mirroring the reference's borrow/own rules):
 *  - Every call returns an int status: QTTS_OK (0) or a negative QTTS_ERR_*.
 *    qtts_last_error(ctx) returns a message for the last failure.
 *  - Inputs are borrowed; uploads copy (and repack) into device memory owned
 *    by the context.  Output buffers are caller-owned.
 *  - Host pointers are the default.  Where a call takes `flags`,
 *    QTTS_DEVICE_PTRS says the float buffers are device pointers instead.
 *  - One context per host thread; a context is not re-entrant.
 *  - Weights are the reference's Q4 layout (gemv.rs:26-31): a linear map
 *    in -> out is stored input-major as `packed[k=in][n/2]` (two 4-bit codes
 *    per byte, low nibble = even output column) and `scales[k][n/32]` f16;
 *    value = (nibble - 8) * scale.
 */
#ifndef QTTS_H
#define QTTS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QTTS_OK             0
#define QTTS_ERR_INVALID   -1   /* bad argument, shape or handle           */
#define QTTS_ERR_HIP       -2   /* HIP runtime error                       */
#define QTTS_ERR_OOM       -3   /* device allocation failed                */
#define QTTS_ERR_CAPACITY  -4   /* KV cache or workspace capacity exceeded */
#define QTTS_ERR_STATE     -5   /* call out of order (no model, no begin)  */
#define QTTS_ERR_IO        -6   /* model file missing, truncated or bad    */
#define QTTS_ERR_NAN       -7   /* non-finite logits reached a sampler     */
#define QTTS_ERR_UNSUPPORTED -8 /* format the device path does not run     */

#define QTTS_DEVICE_PTRS   1    /* flags: float buffers are device memory  */
/* Path choice for qtts_gemm_q4 and qtts_talker_prefill (default: by row
 * count, the matrix cores from 16 rows up). */
#define QTTS_PATH_ROWWISE  2    /* flags: one GEMV pass per row            */
#define QTTS_PATH_MFMA     4    /* flags: matrix-core GEMM at any row count */

typedef struct qtts_ctx qtts_ctx;
typedef struct qtts_w   qtts_w;      /* one uploaded Q4 weight             */
typedef struct qtts_prefix qtts_prefix; /* a kept talker KV prefix          */

/* ---- host-side weight descriptors (plain pointers into caller memory) ---- */

/* One Q4 weight, layout of `Q4Weight` (gemv.rs:26-31). */
typedef struct qtts_q4_host {
    const uint8_t  *packed;   /* k * (n/32) * 16 bytes                    */
    const uint16_t *scales;   /* k * (n/32) f16 bit patterns              */
    int64_t k;                /* input dim  (rows)                        */
    int64_t n;                /* output dim (columns)                     */
} qtts_q4_host;

/* One decoder layer: `TalkerLayerWeights` (talker.rs:19-31) and
 * `PredictorLayerWeights` (code_predictor.rs:14-26) share this shape. */
typedef struct qtts_layer_host {
    qtts_q4_host q_proj, k_proj, v_proj, o_proj;
    const uint16_t *q_norm, *k_norm;             /* [head_dim] f16         */
    qtts_q4_host gate_proj, up_proj, down_proj;
    const uint16_t *input_norm, *post_attn_norm; /* [hidden] f16           */
} qtts_layer_host;

/* `TalkerWeights` (talker.rs:33-56). */
typedef struct qtts_talker_host {
    int32_t n_layers, hidden, text_hidden, n_heads, n_kv_heads, head_dim;
    int32_t inter, vocab;
    const qtts_layer_host *layers;               /* [n_layers]             */
    qtts_q4_host codec_embedding;                /* [vocab x hidden]       */
    qtts_q4_host text_embedding;                 /* [text_vocab x text_hidden] */
    qtts_q4_host text_fc1, text_fc2;
    const float *text_fc1_bias, *text_fc2_bias;
    qtts_q4_host codec_head;                     /* hidden -> vocab        */
    const uint16_t *final_norm;                  /* [hidden] f16           */
    const float *rope_cos, *rope_sin;            /* [rope_max_pos][head_dim/2] */
    int64_t rope_max_pos;
} qtts_talker_host;

/* `CodePredictorWeights` (code_predictor.rs:28-46). */
typedef struct qtts_predictor_host {
    int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, inter;
    int32_t vocab;                               /* codes per codebook (2048) */
    int32_t n_groups;                            /* acoustic codebooks (15)   */
    int32_t has_input_proj;
    qtts_q4_host input_proj;                     /* talker hidden -> hidden */
    const float *input_proj_bias;
    const qtts_q4_host *codec_embeddings;        /* [n_groups]              */
    const qtts_layer_host *layers;               /* [n_layers]              */
    const qtts_q4_host *lm_heads;                /* [n_groups]              */
    const uint16_t *final_norm;
    const float *rope_cos, *rope_sin;
    int64_t rope_max_pos;
} qtts_predictor_host;

/* ---- speech decoder (codes -> 24 kHz audio) ---------------------------- */

/* `Conv1dWeight` (conv.rs:29-38): weight [out][in][kernel] f32. */
typedef struct qtts_conv1d_host {
    const float *weight, *bias;
    int32_t in_channels, out_channels, kernel_size, stride;
    int32_t padding, dilation;
} qtts_conv1d_host;

/* `ConvTranspose1dWeight` (conv.rs:235-243): weight [in][out][kernel]. */
typedef struct qtts_convt1d_host {
    const float *weight, *bias;
    int32_t in_channels, out_channels, kernel_size, stride;
    int32_t padding, reserved;
} qtts_convt1d_host;

/* `DepthwiseConv1dWeight` (conv.rs:351-357): weight [channels][kernel]. */
typedef struct qtts_dwconv_host {
    const float *weight, *bias;
    int32_t channels, kernel_size, padding, reserved;
} qtts_dwconv_host;

/* `DecoderTfLayer` (decoder.rs:68-80): matrices input-major [k][n]. */
typedef struct qtts_dec_layer_host {
    const float *q_proj, *k_proj, *v_proj;     /* [hidden][heads*head_dim] */
    const float *o_proj;                       /* [heads*head_dim][hidden] */
    const float *gate_proj, *up_proj;          /* [hidden][inter]          */
    const float *down_proj;                    /* [inter][hidden]          */
    const float *input_norm, *post_attn_norm;  /* [hidden]                 */
    const float *attn_scale, *mlp_scale;       /* [hidden] layer scales    */
} qtts_dec_layer_host;

/* `UpsampleStage` (decoder.rs:82-93): ConvTranspose1d + ConvNeXt. */
typedef struct qtts_upsample_host {
    qtts_convt1d_host conv_t;
    qtts_dwconv_host dw_conv;
    const float *norm_w, *norm_b;              /* [channels]               */
    const float *pw1_w, *pw1_b;                /* [channels][inner], [inner] */
    const float *pw2_w, *pw2_b;                /* [inner][channels], [channels] */
    const float *gamma;                        /* [channels]               */
    int32_t channels, inner;
} qtts_upsample_host;

/* `VocosResidual` (decoder.rs:102-109). */
typedef struct qtts_vocos_res_host {
    const float *act1_alpha, *act1_beta;
    qtts_conv1d_host conv1;                    /* k 7, dilation 1 / 3 / 9  */
    const float *act2_alpha, *act2_beta;
    qtts_conv1d_host conv2;                    /* k 1                      */
} qtts_vocos_res_host;

/* `VocosBlock` (decoder.rs:95-100). */
typedef struct qtts_vocos_block_host {
    const float *pre_snake_alpha, *pre_snake_beta;
    qtts_convt1d_host upsample;
    const qtts_vocos_res_host *residuals;
    int32_t n_residuals, reserved;
} qtts_vocos_block_host;

/* `SpeechDecoderWeights` (decoder.rs:22-66). */
typedef struct qtts_decoder_host {
    int32_t hidden, n_heads, head_dim, inter;  /* transformer: 512, 16, 64, 1024 */
    int32_t sliding_window, codebook_dim;      /* 72, 256                  */
    int32_t codebook_size, vq_dim;             /* 2048 entries, 512        */
    const float *first_codebook;               /* [codebook_size][codebook_dim] */
    const float *first_output_proj;            /* [codebook_dim][vq_dim]   */
    const float *const *rest_codebooks;        /* n_rest x [codebook_size][codebook_dim] */
    const float *rest_output_proj;             /* [codebook_dim][vq_dim]   */
    int32_t n_rest, latent;                    /* 15, 1024                 */
    qtts_conv1d_host pre_conv;                 /* vq_dim -> latent, k 3    */
    const float *tf_input_w, *tf_input_b;      /* [latent][hidden], [hidden] */
    const qtts_dec_layer_host *tf_layers;
    const float *tf_norm;                      /* [hidden]                 */
    const float *tf_output_w, *tf_output_b;    /* [hidden][latent], [latent] */
    int32_t n_tf_layers, n_upsample;
    const qtts_upsample_host *upsample;
    qtts_conv1d_host vocos_init;
    const qtts_vocos_block_host *vocos_blocks;
    int32_t n_vocos_blocks, reserved;
    const float *final_snake_alpha, *final_snake_beta;
    qtts_conv1d_host output_conv;              /* -> 1 channel, k 7        */
    const float *rope_cos, *rope_sin;          /* [rope_max_pos][head_dim/2] */
    int64_t rope_max_pos;
} qtts_decoder_host;

/* Sampler parameters: the fields of `TTSParams` (generate_new.rs:38-61)
 * that `sample_token` and the frame loop read. */
typedef struct qtts_sample_params {
    float    temperature;          /* generate_new.rs:82-88 (after onset)    */
    int32_t  top_k;                /* 0 = off                                */
    float    top_p;                /* >=1 or <=0 = off                       */
    float    repetition_penalty;   /* 1.0 = off                              */
    uint32_t codec_eos_id;         /* 2150; stop when sampled                */
    int32_t  eos_enabled;          /* 0: never stop (throughput runs)        */
    int32_t  onset_frames;         /* frames using onset_temperature         */
    float    onset_temperature;
} qtts_sample_params;

/* ---- context ---------------------------------------------------------- */

/* Create a context on HIP device `device` with room for `kv_capacity`
 * talker positions (0 = 4096).  No reference counterpart: the reference
 * keeps all state in host Vecs. */
int  qtts_ctx_create(int device, int64_t kv_capacity, qtts_ctx **out);
void qtts_ctx_destroy(qtts_ctx *ctx);
const char *qtts_last_error(const qtts_ctx *ctx);
/* Wait for all work queued on the context's stream. */
int  qtts_sync(qtts_ctx *ctx);
/* The HIP stream (hipStream_t) the context launches on. */
void *qtts_stream(qtts_ctx *ctx);

/* ---- operator level --------------------------------------------------- */

/* Upload one Q4 weight (repacked for the device).  Replaces building a
 * `Weight::Q4` (gemv.rs:26-36) for the device path. */
int qtts_q4_upload(qtts_ctx *ctx, const qtts_q4_host *w, qtts_w **out);
int qtts_q4_free(qtts_ctx *ctx, qtts_w *w);

/* y[n] = x[k] * W.  Replaces `gemv` (gemv.rs:149-154) -> `gemv_q4`
 * (gemv.rs:290-346).  Output columns past (n/32)*32 are left zero, as in
 * `gemv_q4_scalar` (gemv.rs:249-287). */
int qtts_gemv_q4(qtts_ctx *ctx, const qtts_w *w, const float *x, float *y,
                 int flags);

/* Y[rows][n] = X[rows][k] * W.  Replaces `gemm` (gemv.rs:157-162) ->
 * `gemm_q4` (gemv.rs:349-412).  From 16 rows (k a multiple of 32, at least
 * 64) an f32 matrix-core GEMM; fewer rows run the GEMV, two rows per pass
 * over W.  flags may force either path (QTTS_PATH_*). */
int qtts_gemm_q4(qtts_ctx *ctx, const qtts_w *w, const float *X, int64_t rows,
                 float *Y, int flags);

/* qtts_gemm_q4 on DEVICE pointers X [rows][k] and Y [rows][n] that
 * allocates nothing: no reference counterpart.  For callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops).  The GEMV passes' split-K partial sums use a 4 MiB device array
 * held by the library on each GPU until the process ends; a weight whose
 * passes need more (S * 2 * npad floats, S = ceil(k / 2048) for the
 * default tile) is refused with QTTS_ERR_CAPACITY.  Only enqueues on the
 * context stream (no synchronisation; qtts_sync or the stream from
 * qtts_stream orders the results).  Calls that overlap on one GPU share
 * that array and race.  At most 2^20 rows per call (QTTS_ERR_CAPACITY
 * beyond).  flags: QTTS_PATH_* as for qtts_gemm_q4. */
int qtts_gemm_q4_noalloc(qtts_ctx *ctx, const qtts_w *w, const float *X,
                         int64_t rows, float *Y, int flags);

/* out[n] = dequantised row `row`.  Replaces `embed_lookup_q4`
 * (gemv.rs:415-437); exact in f32. */
int qtts_embed_lookup_q4(qtts_ctx *ctx, const qtts_w *w, int64_t row,
                         float *out, int flags);

/* ---- model level ------------------------------------------------------ */

/* Upload talker + predictor.  Replaces holding `TalkerWeights` /
 * `CodePredictorWeights` (talker.rs:33-56, code_predictor.rs:28-46).
 * QTTS_ERR_UNSUPPORTED for shapes other than the 12 Hz model's layout:
 * 16 query / 8 KV heads of 128, hidden sizes multiples of 32 up to 2048,
 * codec vocabularies multiples of 32 (talker at most 4096). */
int qtts_model_upload(qtts_ctx *ctx, const qtts_talker_host *talker,
                      const qtts_predictor_host *predictor);

/* Read a `.qora-tts` file (QTTS v1, Q4 format byte) straight into the
 * context: talker and predictor, then the speech decoder when the file goes
 * on past the predictor.  Replaces `save::load_model` (save.rs:262-298) ->
 * `load_talker` / `load_predictor` / `load_decoder_weights`
 * (save.rs:300-552); the speaker-encoder section after them is not read.
 * A malformed section fails with QTTS_ERR_IO before anything is uploaded. */
int qtts_model_load_qtts(qtts_ctx *ctx, const char *path);

/* RoPE tables for a container that does not hold them: the talker's
 * multimodal tables (rope::build_mrope_tables, rope.rs:11-41) and the
 * predictor's standard ones (loader.rs:869-881), [max_pos][head_dim/2]. */
typedef struct qtts_rope_tables {
    const float *talker_cos, *talker_sin;
    int64_t talker_max_pos;
    const float *pred_cos, *pred_sin;
    int64_t pred_max_pos;
} qtts_rope_tables;

/* Read the older "QORA-TTS-Q4" named-tensor container straight into the
 * context: talker and predictor.  Replaces `load_talker_binary` /
 * `load_code_predictor_binary` (loader.rs:724-882, container read by
 * loader.rs:47-127).  Shapes come from the tensors (layer and codebook
 * counts from the names present); the RoPE tables from `rope`.  A missing
 * or malformed tensor fails with QTTS_ERR_IO, an F16 linear weight with
 * QTTS_ERR_UNSUPPORTED, before anything is uploaded. */
int qtts_model_load_qora_q4(qtts_ctx *ctx, const char *path, const qtts_rope_tables *rope);

/* Shapes of the uploaded model (hidden, vocab, ...); 0 on success. */
int qtts_model_dims(qtts_ctx *ctx, int32_t *talker_hidden,
                    int32_t *talker_vocab, int32_t *talker_layers,
                    int32_t *pred_hidden, int32_t *pred_vocab,
                    int32_t *pred_groups);

/* ---- talker ------------------------------------------------------------ */

/* One decode step: `forward_with_embedding` (talker.rs:263-360).  Appends
 * one position to the talker KV cache (RoPE at `position`) and writes the
 * final-normed hidden [hidden] and the codec-head logits [vocab]. */
int qtts_talker_step(qtts_ctx *ctx, const float *embedding, int64_t position,
                     float *hidden_out, float *logits_out, int flags);

/* Legacy `forward_talker_decode` (talker.rs:161-258, the loop of
 * generate.rs:185-235): embeds `token` itself (text projection when
 * is_text, else the codec table), runs one step at `position` and writes
 * the final-normed hidden (no codec head). */
int qtts_talker_decode_token(qtts_ctx *ctx, uint32_t token, int is_text,
                             int64_t position, float *hidden_out, int flags);

/* Prefill `seq` rows of pre-built embeddings at positions
 * start_pos..start_pos+seq-1 on top of the cached prefix:
 * `prefill_talker_raw_from` (talker.rs:379-482).  Requires
 * kv_len == start_pos.  Writes the last row's final-normed hidden.  From
 * 16 rows the layers run as batched matrix-core GEMMs (chunks of up to
 * 1024 rows); fewer rows go one by one through the decode kernels.  flags
 * may force either path (QTTS_PATH_*). */
int qtts_talker_prefill(qtts_ctx *ctx, const float *X, int64_t seq,
                        int64_t start_pos, float *hidden_out, int flags);

/* logits = hidden * codec_head: `apply_codec_head` (talker.rs:647-649). */
int qtts_codec_head(qtts_ctx *ctx, const float *hidden, float *logits,
                    int flags);

/* `embed_text_token` (talker.rs:105-116): text row + fc1/SiLU/fc2. */
int qtts_embed_text_token(qtts_ctx *ctx, uint32_t token, float *out,
                          int flags);
/* `embed_codec_token` (talker.rs:152-154). */
int qtts_embed_codec_token(qtts_ctx *ctx, uint32_t token, float *out,
                           int flags);

/* ---- talker KV cache (paged, device resident) ------------------------- */

/* Drop every cached position (`empty_kv_cache`, gemv.rs:79-86). */
int qtts_kv_reset(qtts_ctx *ctx);
int qtts_kv_len(qtts_ctx *ctx, int64_t *len);
/* Copy layer `layer`'s cache out in the reference layout
 * `[len][n_kv_heads][head_dim]` f32 (gemv.rs:75-77).  Bit-exact. */
int qtts_kv_gather(qtts_ctx *ctx, int32_t layer, float *K, float *V);
/* Overwrite the cache with `len` positions per layer, reference layout,
 * K and V each [n_layers][len][n_kv_heads][head_dim] (test and bench
 * set-up).  Bit-exact. */
int qtts_kv_load(qtts_ctx *ctx, const float *K, const float *V, int64_t len);
/* Keep the first `len` positions and drop the rest (prefix reuse,
 * generate_new.rs:537-551: the cached prefix is kept, the suffix redone). */
int qtts_kv_truncate(qtts_ctx *ctx, int64_t len);

/* ---- talker prefix cache (page-table fork) ---------------------------- */

/* Keep cached positions 0..kv_len-1 as a reusable prefix: the
 * `TalkerPrefixCache` built once per run (generate_new.rs:317-355).  The
 * full 64-position pages are shared with the running sequence, not copied
 * (copy-on-write if the sequence rewrites them); the last partial page is
 * copied.  The context's page pool holds 2 * kv_capacity / 64 pages. */
int qtts_prefix_capture(qtts_ctx *ctx, qtts_prefix **out);
/* Start the cache from a kept prefix: `pfx.kv.clone()` then a suffix
 * prefill at start_pos = prefix length (generate_new.rs:537-551).  The full
 * pages are mapped into the page table; the partial page is copied.  Sets
 * kv_len and position to the prefix length. */
int qtts_prefix_attach(qtts_ctx *ctx, const qtts_prefix *prefix);
int qtts_prefix_len(const qtts_prefix *prefix, int64_t *len);
/* Release a prefix (its pages return to the pool once no sequence holds
 * them).  Prefixes die with their model: after a new upload this only
 * frees the handle. */
int qtts_prefix_free(qtts_ctx *ctx, qtts_prefix *prefix);
/* `prefix_suffix_split` (generate_new.rs:307-316): 1 and *suffix_len =
 * block_len - n_ref when a prefix of 9 + n_ref positions covers the
 * chunk-independent part of an ICL block, else 0 (full prefill needed).
 * Host only; needs no device. */
int qtts_prefix_suffix_split(int64_t block_len, int64_t n_ref, int64_t prefix_len,
                             int64_t *suffix_len);

/* ---- prompt construction on the device -------------------------------- */

/* `icl_block_layout` (generate_new.rs:120-128): rows of the ICL block
 * (n_frames + 1) and of the trailing-text remainder.  Host only. */
int qtts_icl_layout(int64_t n_ref, int64_t n_text, int64_t n_frames,
                    int64_t *icl_len, int64_t *remainder_len);
/* `embed_text_token` (talker.rs:105-116) over `n` ids in one batch (ids in
 * host memory): the table rows, then fc1 + bias, SiLU, fc2 + bias on the
 * matrix cores.  out [n][hidden]. */
int qtts_embed_text_tokens(qtts_ctx *ctx, const uint32_t *ids, int64_t n,
                           float *out, int flags);
/* `build_icl_block` (generate_new.rs:140-195) on the device.  ref_codes is
 * [16][n_frames] (codebook-major, values < 2048), ids and codes in host
 * memory.  icl_out gets [n_frames + 1][hidden]: text side (ref_tokens ++
 * text_tokens, then tts_eos; tts_pad past its end) + codec side (codec_bos,
 * then per frame the talker codec row of code 0 plus the predictor rows of
 * codes 1..15, added in that order).  remainder_out gets the text rows past
 * the block, [remainder_len][hidden] (may be null when that is 0). */
int qtts_build_icl_block(qtts_ctx *ctx, const uint32_t *ref_tokens, int64_t n_ref,
                         const uint32_t *text_tokens, int64_t n_text,
                         const uint32_t *ref_codes, int64_t n_frames,
                         float *icl_out, float *remainder_out, int flags);
/* `build_prefill_head` (generate_new.rs:222-237) on the device: the
 * chunk-independent head, out [9][hidden].  Rows 0-2 are the text rows of
 * IM_START, ASSISTANT, NEWLINE (`build_role_prefix`, :91-97).  With a
 * voice embedding (`build_codec_prefix_voice`, :200-223): codec rows of
 * THINK, THINK_BOS, language_id, THINK_EOS + the TTS_PAD text row, then
 * voice[j] + TTS_PAD[j] for j < min(voice_len, hidden) (zero past it),
 * then CODEC_PAD + TTS_BOS.  With voice null (`build_codec_prefix_builtin`,
 * :226-238): codec rows of THINK, THINK_BOS, language_id, THINK_EOS,
 * speaker_id, CODEC_PAD under the overlay [TTS_PAD x5, TTS_BOS].  voice is
 * a host or device float buffer as flags say. */
int qtts_build_prefill_head(qtts_ctx *ctx, uint32_t speaker_id, uint32_t language_id,
                            const float *voice, int64_t voice_len, float *out, int flags);
/* `build_icl_prefix` (generate_new.rs:244-280) on the device: the first
 * n_ref pairs of the ICL block, out [n_ref][hidden], bit-identical to those
 * rows of qtts_build_icl_block; a ref token past the last frame meets
 * CODEC_PAD.  ref_codes [16][n_frames], ids and codes in host memory. */
int qtts_build_icl_prefix(qtts_ctx *ctx, const uint32_t *ref_tokens, int64_t n_ref,
                          const uint32_t *ref_codes, int64_t n_frames, float *out, int flags);
/* `build_trailing_text` (generate_new.rs:756-767): the text rows of
 * tokens[1..n) then TTS_EOS, out [max(n - 1, 0) + 1][hidden]. */
int qtts_build_trailing_text(qtts_ctx *ctx, const uint32_t *tokens, int64_t n, float *out, int flags);
/* `prefill_custom_voice` (generate_new.rs:361-476) on the device: the
 * prompt is the 9 head rows (qtts_build_prefill_head), then the ICL rows
 * (icl_rows [n_icl][hidden], voice-cloning head only) or, without them and
 * with text, CODEC_BOS + the first text token's row.  The KV cache is reset
 * and the prompt prefilled from position 0, then the codec head: hidden_out
 * [hidden], logits_out [vocab], and *position_out the frame loop's first
 * position (9 + n_icl, else 10, or 9 with no text; generate_new.rs:560-565).
 * flags: QTTS_DEVICE_PTRS for the float buffers, QTTS_PATH_* for the
 * prefill. */
int qtts_prefill_custom_voice(qtts_ctx *ctx, const uint32_t *text_tokens, int64_t n_text,
                              uint32_t speaker_id, uint32_t language_id,
                              const float *voice, int64_t voice_len,
                              const float *icl_rows, int64_t n_icl,
                              float *hidden_out, float *logits_out, int64_t *position_out,
                              int flags);

/* ---- speech decoder --------------------------------------------------- */

/* Upload the speech decoder (codes -> 24 kHz waveform).  Replaces holding
 * `SpeechDecoderWeights` (decoder.rs:22-66).  Matrices are repacked for
 * the matrix-core convolutions; transposed convolutions must have
 * kernel = stride or 2 * stride and padding 0 (the model's 2x / 8,5,4,3x
 * stages), head_dim 64 or 16.  Replaces a previously uploaded decoder. */
int qtts_decoder_upload(qtts_ctx *ctx, const qtts_decoder_host *decoder);

/* Shape of the uploaded decoder: codebooks per frame (n_rest + 1), codes
 * per codebook, and output samples per frame (the product of the upsampling
 * strides: 1920 for the 12 Hz tokenizer).  QTTS_ERR_STATE without one.  No
 * reference counterpart (the reference reads these off its Vecs). */
int qtts_decoder_dims(qtts_ctx *ctx, int32_t *n_codebooks, int32_t *codebook_size,
                      int64_t *samples_per_frame);

/* `decode_to_audio` (decoder.rs:395-574): codes [n_codebooks][n_frames]
 * (codebook-major, n_codebooks = n_rest + 1), optional warmup codes
 * [n_codebooks][n_warmup] prepended and trimmed off the output
 * (`warmup_trim_len`, decoder.rs:651-656).  audio gets *n_samples
 * samples in [-1, 1]; with too small a capacity it fails with
 * QTTS_ERR_CAPACITY and *n_samples holds the size needed.  n_frames 0
 * gives no samples.  Codes and audio in host memory, or device memory
 * with QTTS_DEVICE_PTRS for audio. */
int qtts_decode_to_audio(qtts_ctx *ctx, const uint32_t *codes, int64_t n_frames,
                         const uint32_t *warmup, int64_t n_warmup,
                         float *audio, int64_t capacity, int64_t *n_samples,
                         int flags);

/* ---- code predictor --------------------------------------------------- */

/* `generate_acoustic_codes` (code_predictor.rs:218-273): 2-token prefill,
 * 14 autoregressive steps, greedy argmax (last index on ties). */
int qtts_predictor_chain(qtts_ctx *ctx, const float *talker_hidden,
                         const float *semantic_embed, uint32_t *codes_out,
                         int flags);

/* `get_acoustic_embeddings_sum` (code_predictor.rs:287-300). */
int qtts_acoustic_embed_sum(qtts_ctx *ctx, const uint32_t *codes, float *out,
                            int flags);

/* ---- sampler ---------------------------------------------------------- */

/* `sample_token` (generate_new.rs:771-862) with `simple_rand`
 * (generate_new.rs:17-22) advancing *rng by one draw.  `prev` holds
 * `n_prev` previous tokens for the repetition penalty. */
int qtts_sample_token(qtts_ctx *ctx, const float *logits, int64_t n,
                      const qtts_sample_params *p, const uint32_t *prev,
                      int64_t n_prev, uint64_t *rng, float temperature,
                      uint32_t *out);

/* ---- legacy loop (generate.rs:107-250) -------------------------------- */

/* `prefill_talker` (talker.rs:487-508): each id embedded as a text token
 * (is_text != 0: the text projection) or a codec token, then
 * prefill_talker_raw over a fresh cache (positions 0..n-1).  hidden_out
 * gets the final-normed hidden of the last row. */
int qtts_prefill_tokens(qtts_ctx *ctx, const uint32_t *ids, const uint8_t *is_text,
                        int64_t n, float *hidden_out, int flags);

/* `predict_codes` (code_predictor.rs:126-216): the legacy, non-autoregressive
 * predictor step -- project the talker hidden, run the predictor's layers
 * over a cache kept across calls (the new row sits at the cache length),
 * final norm, then every lm head: logits [n_groups][vocab].
 * qtts_predict_codes_reset empties that cache (a new utterance; the
 * reference allocates a fresh one, generate.rs:129). */
int qtts_predict_codes(qtts_ctx *ctx, const float *talker_hidden, float *logits,
                       int flags);
int qtts_predict_codes_reset(qtts_ctx *ctx);

/* The legacy loop's sampler (generate.rs:185-217): apply_repetition_penalty
 * over the n_prev previous tokens when repetition_penalty > 1
 * (generate.rs:87-98), then sample_top_k (generate.rs:50-84): temperature
 * <= 0 takes the last maximum; otherwise the top_k logits in descending
 * order, exp((l - max) / T) normalised, one `simple_rand` draw.  Equal
 * logits keep index order (the reference's unstable sort leaves it open).
 * QTTS_ERR_INVALID for top_k < 1 with temperature > 0, QTTS_ERR_NAN for a
 * NaN logit.  Host buffers; n <= 4096. */
int qtts_sample_top_k(qtts_ctx *ctx, const float *logits, int64_t n, float temperature,
                      int32_t top_k, const uint32_t *prev, int64_t n_prev,
                      float repetition_penalty, uint64_t *rng, uint32_t *out);

/* ---- frame loop (generate_new.rs:606-675) ----------------------------- */

/* Start a generation: the prefill's logits [vocab] and final-normed hidden
 * [hidden], the next RoPE position, the RNG seed and the sampler settings.
 * prev_tokens start at zero (generate_new.rs:583). */
int qtts_gen_begin(qtts_ctx *ctx, const float *logits, const float *hidden,
                   int64_t position, uint64_t seed,
                   const qtts_sample_params *p);

/* Trailing text rows added to frames 0..n_text-1, then `pad` for every
 * later frame (generate_new.rs:645-654).  text may be NULL when n_text=0. */
int qtts_gen_set_text(qtts_ctx *ctx, const float *text, int64_t n_text,
                      const float *pad);

/* Run up to `max_frames` frames.  codes_out is [max_frames][16]
 * (code 0 = talker sample, 1..15 = predictor).  Stops after the frame whose
 * sampled code 0 is the EOS id (that frame's codes are not emitted, as in
 * generate_new.rs:611-614).  *frames_done counts emitted frames, *eos is 1
 * when EOS stopped the run.  One host synchronisation per call batch. */
int qtts_gen_frames(qtts_ctx *ctx, int64_t max_frames, uint32_t *codes_out,
                    int64_t *frames_done, int32_t *eos);

/* Teacher-forced frames for parity checks: frame f predicts 16 codes into
 * pred_out[f] but feeds forced[f] downstream (talker input, predictor chain
 * steps, repetition history).  No EOS stop. */
int qtts_gen_frames_forced(qtts_ctx *ctx, int64_t n_frames,
                           const uint32_t *forced, uint32_t *pred_out);

/* Current generation state: logits [vocab], hidden [hidden], position and
 * RNG state (host copies). */
int qtts_gen_state(qtts_ctx *ctx, float *logits, float *hidden,
                   int64_t *position, uint64_t *rng);

/* Test hook, no reference counterpart (the reference has no device waits):
 * the next call that runs fused launches (talker step or row prefill, frame
 * batch, predictor chain, legacy predictor step) starts from the state a
 * bounded cross-workgroup wait leaves when it runs out.  Its fused launches
 * skip their waits (every kernel exits normally, outputs invalid) and the
 * call returns QTTS_ERR_HIP; the one after it runs normally.  A talker step
 * that fails so keeps its cache length and position; a frame batch has
 * counted and cached the frames it ran, so the caller truncates the cache
 * (qtts_kv_truncate) and begins again (qtts_gen_begin), as after a real
 * timeout. */
int qtts_debug_force_sync_err(qtts_ctx *ctx);

/* ---- measurement ------------------------------------------------------ */

/* Average device time (us) of one kernel launch: one HIP event pair around
 * `iters` back-to-back launches on the context stream (after one warm-up
 * launch), divided by `iters`; *bytes gets the
 * algorithmic bytes one launch moves.  No reference counterpart (the
 * reference times phases with Instant, generate_new.rs:600-678).
 *   kind 0: talker gate|up GEMV (RMSNorm prologue), cycling the layers;
 *   kind 1: talker decode attention over the cached positions, cycling
 *           the layers;
 *   kind 2: plain float4 copy of 256 MiB (no model needed), the HBM
 *           calibration point for byte counters;
 *   kind 3: predictor attention + o-proj, one row at position 8;
 *   kind 4: one whole predictor layer step, one row at position 8;
 *   kind 5: the frame without its talker step (sampler, predictor chain,
 *           combine), captured alone and replayed; *bytes = the predictor's
 *           Q4 weight bytes;
 *   kind 6: the talker step alone (28 layers + codec head), captured and
 *           replayed from the current KV length (QTTS_ERR_CAPACITY without
 *           room for iters + 1 positions); *bytes = its Q4 weight bytes;
 *   kind 7: a streaming read of 7,110,656 B (the Q4 GEMV k=2048 -> n=6144's
 *           bytes) in one launch, cycling 64 buffers (455 MB, beyond the
 *           last-level cache; no model needed): the attainable time of a
 *           single launch that moves those bytes;
 *   kind 8: one talker layer as the frame's step runs it (q|k|v + attention
 *           in one launch, the o-proj, gate|up + down in one launch) at the
 *           current length, appending at the free slot, cycling the layers;
 *           *bytes = the layer's Q4 weights + the K/V read and appended;
 *   kind 9: one predictor layer step as the chain runs it (q|k|v +
 *           attention + o-proj in one launch, gate|up + down in the next),
 *           one row at position 8, cycling the layers; *bytes = the layer's
 *           Q4 weights + the cached K/V.
 * Kinds 5 and 6 restore the generation state afterwards (counters, the
 * next frame's logits and hidden), so frames generated after the call are
 * those that would have followed without it. */
int qtts_time_kernel(qtts_ctx *ctx, int32_t kind, int32_t iters,
                     double *avg_us, double *bytes);

/* Launch mode of the timing calls above and below: 0 (default) launches
 * each timed kernel from the context stream; 1 captures the `iters`
 * launches once into a graph and replays it (one warm-up replay, then four
 * between the events; the average is over all replayed launches), which
 * is how the frame loop runs its kernels.  Kinds 5 and 6 replay their own
 * graph either way; the whole-prefill and speech-decoder timings always
 * launch from the stream.  No reference counterpart. */
int qtts_time_graph(qtts_ctx *ctx, int32_t on);

/* Same for the standalone Q4 GEMV, cycling through `n_w` uploaded weights
 * of one shape (a pool larger than the 256 MB last-level cache measures
 * HBM, not cache). */
int qtts_time_gemv(qtts_ctx *ctx, const qtts_w *const *ws, int32_t n_w,
                   int32_t iters, double *avg_us, double *bytes);

/* Average device time (us) of the matrix-core prefill over `rows`
 * synthetic rows (same event scheme); *flops gets the algorithmic
 * floating-point operations of one launch.  No reference counterpart.
 *   what 0: the talker gate|up GEMM with its SwiGLU epilogue
 *           ([rows x hidden] x [hidden x 2 inter]), cycling the layers;
 *   what 1: the whole prefill_talker_raw_from over positions 0..rows-1
 *           (every layer, attention included, input rows restaged per
 *           launch).  Overwrites cached positions 0..rows-1 and leaves
 *           the cache length at 0. */
int qtts_time_prefill(qtts_ctx *ctx, int64_t rows, int32_t what, int32_t iters,
                      double *avg_us, double *flops);

/* Average device time (us) of one whole decode_to_audio on the device over
 * `n_frames` synthetic frames (codes from a fixed generator, already
 * resident; no warmup trim), same event scheme; *flops gets the
 * algorithmic floating-point operations of one decode (every projection
 * and convolution at its true kernel size, attention q.k and p.v).  No
 * reference counterpart (the reference prints phase times,
 * decoder.rs:572-574). */
int qtts_time_decode(qtts_ctx *ctx, int64_t n_frames, int32_t iters,
                     double *avg_us, double *flops);

/* Device memory the uploaded model holds, in bytes.  No reference
 * counterpart (the reference keeps its weights in host memory): a
 * measurement helper so a caller can see what the upload-time tables cost
 * against the weights they stand in for. */
typedef struct {
    int64_t talker_q4;            /* talker Q4 tiles: layers, codec head, text projection */
    int64_t predictor_q4;         /* predictor Q4 tiles: layers, lm heads, input projection */
    int64_t predictor_row_tables; /* projected code-embedding rows of steps 1..14 (f32), 0 if off */
    int64_t predictor_qkv_tables; /* their layer-0 q|k|v rows (f32), 0 if off */
    int64_t embedding_rows;       /* Q4 embedding tables kept row-major (text, codec, predictor) */
    int64_t kv_pool;              /* talker KV page pool (f32), 2 x capacity */
    int64_t device_used;          /* total minus free device memory (hipMemGetInfo) */
} qtts_mem_report;

int qtts_device_bytes(qtts_ctx *ctx, qtts_mem_report *out);

#ifdef __cplusplus
}
#endif
#endif /* QTTS_H */
