// qtts_kernels.h — model/workspace descriptors and the enqueue functions the
// runtime calls.  Everything here lives in device memory except the
// descriptor structs themselves (host copies passed by value to kernels).
#pragma once
#include "qtts_device.h"

namespace qtts {

constexpr int MAX_CHUNKS = 128;          // KV pages per sequence (8192 positions)
// Talker decode attention: pages per workgroup (four waves per page), the
// unit of the page merge in the o-proj's prologue.  One page per workgroup
// below ATTN_LONG_KV cached positions, two from there on (fewer, longer
// work items, and half the partials for the merge to read).
constexpr int ATTN_LONG_KV = 1024;
inline int attn_pages(int64_t kv_len) { return kv_len >= ATTN_LONG_KV ? 2 : 1; }
constexpr int RING_FRAMES = 64;          // frames per host synchronisation, max
constexpr int MAX_CAND = 64;             // lm-head column tiles reduced by one wave

// Epoch counters of the fused launches.  A launch of one kind reads its
// counter at its start and stamps its words with counter + 1; a launch that
// always runs between two launches of that kind, and never reads that
// counter, advances it: the talker o-proj advances LL_TQKV and LL_TMLP, the
// predictor's attention + o-proj launches advance LL_PMLP, the predictor's
// MLP launch (fused or its gate|up) advances LL_PQKV.
enum LlKind { LL_TQKV = 0, LL_PQKV = 1, LL_PMLP = 2, LL_TMLP = 3, LL_KINDS = 4 };

struct KvPaged {
    float *base;           // [layers][n_phys][2 (K,V)][8 heads][64 pos][128]
    const int32_t *ptab;   // logical page -> physical page
    int32_t n_phys;
};

// One decoder layer on the device.  q|k|v and gate|up are fused along the
// output dimension (columns [q | k | v], [gate | up]).
struct LayerDev {
    Q4Tiled qkv, o, gate_up, down;
    const uint16_t *q_norm, *k_norm, *input_norm, *post_norm;
    // matrix-core prefill: the staging powers of two (shift = 14 -
    // ceil(log2(bound))) of the normed rows (bound sqrt(hidden) * max|gamma|
    // of the input / post norm) and of the attention's q and k (after
    // QK-norm and RoPE: sqrt(128) * max|gamma|) and v (sqrt(hidden) *
    // max|input gamma| * the largest column 2-norm of v_proj); the
    // attention's are 0 while the bound lies in [2^-4, 2^14]
    int in_shift, post_shift, q_shift, k_shift, v_shift;
};

struct TalkerDev {
    int n_layers, hidden, text_hidden, n_heads, n_kv_heads, inter, vocab;
    const LayerDev *layers;              // host array [n_layers]
    Q4Tiled codec_head, text_fc1, text_fc2;
    const float *text_fc1_bias, *text_fc2_bias;
    Q4Rows codec_rows, text_rows;        // embedding tables, reference layout
    const uint16_t *final_norm;
    const float *rope_cos, *rope_sin;
    int64_t rope_rows;
    KvPaged kv;
};

struct PredictorDev {
    int n_layers, hidden, n_heads, n_kv_heads, inter, vocab, n_groups;
    const LayerDev *layers;              // host array
    Q4Tiled proj;
    const float *proj_bias;
    const float *proj_rows;              // [n_groups-1][emb rows][hidden] projected embedding rows, or null
    const float *qkv_rows;               // [n_groups-1][emb rows][layers[0].qkv.npad] their layer-0 q|k|v, or null
    const Q4Tiled *heads;                // host array [n_groups]
    Q4Rows emb_rows;                     // [n_groups][rows][...] contiguous
    const uint16_t *final_norm;
    const float *rope_cos, *rope_sin;
    int64_t rope_rows;
};

struct Workspace {
    float *x;          // talker step input [hidden]
    float *xa, *xb;    // talker residual stream, ping-pong [hidden]
    float *pxa, *pxb;  // predictor residual rows, ping-pong [2][p.hidden]
    float *pin;        // predictor API input rows [2][t.hidden]
    float *am, *al;    // attention chunk max / sum [16][MAX_CHUNKS], a chunk = 1 or 2 pages
    float *aacc;       // attention chunk P.V [MAX_CHUNKS][16][128]
    float *attn;       // talker attention output [16*128]
    float *pattn;      // predictor attention output [2][16*128]
    float *pk, *pv;    // predictor KV [layers][16][8][128]
    float *h;          // silu(gate)*up [2][max inter]
    // split-K partial sums, one buffer per producer role
    float *part_qkv, *part_o, *part_gu, *part_down, *part_head, *part_proj;
    float *hid_work;   // final-normed hidden of the running step
    float *hidden;     // last_hidden kept across frames
    float *logits;     // logits kept across frames
    float *text;       // trailing text rows [n][hidden]
    float *pad;        // tts_pad row [hidden]
    uint32_t *ring_pred, *ring_used;      // [RING_FRAMES][16]
    float2 *cand;      // lm-head argmax candidates [16 heads][MAX_CAND] (value, index bits)
    int attn_grid;     // attention workgroups at one page each (8 per page of the capacity)
    // (epoch, value) words handed between the two halves of a fused launch,
    // one buffer per kind of launch, and the epoch counter of each kind
    uint64_t *ll_qkv;  // talker q|k|v [S][npad] (q|k|v GEMV + attention)
    uint64_t *ll_pqkv; // predictor q|k|v [S][npad] (q|k|v GEMV + attention + o-proj)
    uint64_t *ll_th;   // talker silu(gate)*up [inter] (gate|up + down)
    uint64_t *ll_ph;   // predictor silu(gate)*up [inter] (gate|up + down)
    uint32_t *ll_seq;  // [LL_KINDS] epoch counters, indexed by LlKind
};

// Buffers of the batched prefill, rows of one prompt chunk.
struct PrefillWs {
    float *x;          // residual rows [cap_rows][hidden]
    float *q;          // normed + roped q rows [cap_rows][16*128]
    float *attn;       // attention rows [cap_rows][16*128]
    float *h;          // silu(gate)*up rows [cap_rows][inter]
    float *part;       // k-slice partial sums of a projection [cap_rows * prefill_part_floats]
    float *inv;        // per-row 1/rms [cap_rows]
    float *rmax;       // per-row largest |x| of a GEMM input by column slots [cap_rows][prefill_rmax_slots]
    int cap_rows;
};

// Speech decoder on the device (qtts_decoder.hip).  Matrices are stored as
// the GEMM's A operand, [output channels][input channels x taps].
// Decoder convolution weights are stored tap-major ([out][kernel][in])
// when this holds (K = 1, or the input channels a multiple of the GEMM's
// 32-wide contraction chunk), else as [out][in][kernel].
inline bool conv_tap_major(int ic, int k) { return k == 1 || ic % 32 == 0; }

struct DecConv {
    const float *w, *b;      // w [oc][k][ic] when conv_tap_major(ic, k), else [oc][ic][k]
    int ic, oc, k, dil;
};
struct DecConvT {            // kernel == stride (1 tap) or 2*stride (2 taps), padding 0
    const float *phases, *b; // [stride][oc] rows of ic x taps (tap-major as DecConv); 2 taps: x[i-1] (kernel tap r+stride), x[i] (tap r)
    int ic, oc, stride, taps;
};
struct DecLayer {
    const float *qkv;        // [3A][hidden] rows q, k, v
    const float *o;          // [hidden][A]
    const float *gate_up;    // [2 inter][hidden] rows gate_j, up_j interleaved
    const float *down;       // [hidden][inter]
    const float *in_norm, *post_norm, *attn_scale, *mlp_scale;
};
struct DecUpsample {
    DecConvT conv_t;
    const float *dw_w, *dw_b;
    int dw_k;
    const float *norm_w, *norm_b;
    const float *pw1, *pw1_b;   // [inner][ch]
    const float *pw2, *pw2_b;   // [ch][inner]
    const float *gamma;
    int ch, inner;
};
struct DecVocosRes {
    const float *a1_alpha, *a1_beta, *a2_alpha, *a2_beta;
    DecConv c1, c2;
};
struct DecVocos {
    const float *pre_alpha, *pre_beta;
    DecConvT up;
    const DecVocosRes *res;  // host array
    int n_res;
};
struct DecoderDev {
    int hidden, n_heads, head_dim, inter, window, codebook_dim, codebook_size, vq_dim, latent, n_rest;
    const float *first_codebook;
    const float *const *rest_codebooks;   // device array of n_rest device pointers
    const float *vq_proj;                 // [vq_dim][2 codebook_dim]: first | rest output projections
    DecConv pre_conv;
    const float *tf_in_w, *tf_in_b;       // [hidden][latent]
    const DecLayer *tf;                   // host array
    int n_tf;
    const float *tf_norm, *tf_out_w, *tf_out_b;   // tf_out_w [latent][hidden]
    const DecUpsample *up;                // host array
    int n_up;
    DecConv voc_init;
    const DecVocos *voc;                  // host array
    int n_voc;
    const float *final_alpha, *final_beta;
    const float *out_w;                   // [ch][k], one output channel
    float out_b;
    int out_k, out_dil;
    const float *rope_cos, *rope_sin;
    int64_t rope_rows;
    bool weights_f32;                     // a weight matrix outside the split-f16 range: f32 matrix path
};
struct DecoderWs {
    float *a, *b, *c, *d, *e;             // each floats_per_frame * cap_frames
    float *part;                          // split-K partial sums
    size_t part_cap;                      // floats in part
    uint32_t *codes;                      // [n_rest + 1][cap_frames]
    int32_t *range_flag;                  // set by a split-f16 convolution whose inputs left its range
    int cap_frames;
    bool f32;                             // this decode on the f32 matrix path
};

struct SampleArgsHost {
    float temperature, top_p, rep;
    int top_k;
    const uint32_t *prev;   // device
    int n_prev;
};

hipError_t enqueue_gemv_plain(const Q4Tiled &w, const float *x, int NB, int ld, float *part, hipStream_t st);
hipError_t enqueue_gemv_store(const Q4Tiled &w, const float *x, float *y, const float *bias, float *part,
                              hipStream_t st);
hipError_t enqueue_gemv_rows(const Q4Tiled &w, const float *X, int rows, float *Y, float *part, hipStream_t st);
hipError_t enqueue_embed_row(const Q4Rows &e, const uint32_t *code_dev, uint32_t code, float *out,
                             hipStream_t st);
hipError_t enqueue_embed_sum(const Q4Rows &cp, int n_groups, const uint32_t *codes, float *out, hipStream_t st);
hipError_t enqueue_silu(float *x, int n, hipStream_t st);
hipError_t enqueue_zero_cols(float *Y, int rows, int ld, int c0, int c1, hipStream_t st);

// True when every talker layer runs its q|k|v GEMV and decode attention as
// one launch (two pages per attention work item at every length); the
// caller then passes attn_pg = 2 for every step.
bool talker_fused_attn(const TalkerDev &m);
// True unless QTTS_FUSED_MLP=0: gate|up and down run as one launch where the
// tiles allow (single-slice gate|up); the predictor's gate|up then takes a
// single-slice tile.
bool fused_mlp_enabled();
hipError_t enqueue_talker_step(const TalkerDev &m, const Workspace &ws, DevState *st, int frame_mode, int attn_pg,
                               hipStream_t s);
hipError_t enqueue_talker_row(const TalkerDev &m, const Workspace &ws, const DevState *st, int64_t pos,
                              int slot, int attn_pg, hipStream_t s);
hipError_t enqueue_final_norm(const TalkerDev &m, const Workspace &ws, float *hidden_out, hipStream_t s);
hipError_t enqueue_codec_head(const TalkerDev &m, const Workspace &ws, const float *hidden, float *logits,
                              hipStream_t s);
hipError_t enqueue_predictor_chain(const PredictorDev &p, const TalkerDev &m, const Workspace &ws,
                                   DevState *st, const float *hidden, const float *sem,
                                   const uint32_t *forced, uint32_t *codes_api, hipStream_t s);
// The frame up to the talker step: sampler, predictor chain, combine.
hipError_t enqueue_frame_codes(const TalkerDev &m, const PredictorDev &p, const Workspace &ws, DevState *st,
                               const uint32_t *forced, hipStream_t s);
hipError_t enqueue_frame(const TalkerDev &m, const PredictorDev &p, const Workspace &ws, DevState *st,
                         const uint32_t *forced, int attn_pg, hipStream_t s);
hipError_t enqueue_sample_top_k(const float *logits, int n, float temperature, int top_k, const uint32_t *prev,
                                int n_prev, float penalty, uint64_t *rng, uint32_t *out, int *status, hipStream_t s);
hipError_t enqueue_sample_api(const float *logits, int n, const SampleArgsHost &a, uint64_t *rng_dev,
                              uint32_t *out_dev, DevState *st, hipStream_t s);
hipError_t enqueue_kv_gather(const KvPaged &kv, int layer, int len, float *K, float *V, hipStream_t s);
hipError_t enqueue_kv_scatter(const KvPaged &kv, int layer, int len, const float *K, const float *V,
                              hipStream_t s);
hipError_t enqueue_pred_attn_o_timing(const PredictorDev &p, const Workspace &ws, int l, int pos0, hipStream_t s);
hipError_t enqueue_pred_layer_timing(const PredictorDev &p, const Workspace &ws, int l, int pos0, hipStream_t s);
hipError_t enqueue_pred_layer_fused_timing(const PredictorDev &p, const Workspace &ws, int l, int pos0, DevState *st,
                                           hipStream_t s);
hipError_t enqueue_talker_layer_timing(const TalkerDev &m, const Workspace &ws, int l, int slot, int64_t pos,
                                       const DevState *st, hipStream_t s);
hipError_t enqueue_copy(const float *src, float *dst, int64_t n, hipStream_t s);
hipError_t enqueue_read(const float *src, int64_t n, uint32_t never, uint32_t *sink, hipStream_t s);
hipError_t enqueue_pred_row_tables(const PredictorDev &p, int n_tables, float *X, float *part, float *out,
                                   hipStream_t s);
bool pred_qkv_tables_supported(const PredictorDev &p);
hipError_t enqueue_pred_qkv_tables(const PredictorDev &p, int n_tables, float *part, float *out, hipStream_t s);
bool gemm_supported(const Q4Tiled &w);
hipError_t enqueue_gemm_rows(const Q4Tiled &w, const float *X, int rows, float *Y, int ldy, float *rmax,
                             hipStream_t s);
hipError_t enqueue_gemm_bias(const Q4Tiled &w, const float *X, int rows, const float *bias, bool silu, float *Y,
                             int ldy, float *rmax, hipStream_t s);
bool prefill_supported(const TalkerDev &m);
int64_t prefill_part_floats(const TalkerDev &m);
int64_t prefill_rmax_slots(const TalkerDev &m);
int norm_shift(const uint16_t *gamma_host, int n);
int bound_shift(double bound);
int attn_shift(double bound);
double f16_max_abs(const uint16_t *h, int n);
hipError_t enqueue_gather_rows(const Q4Rows &e, const uint32_t *ids, int n, float *out, int ld, hipStream_t s);
hipError_t enqueue_codec_frame_rows(const Q4Rows &tcodec, const Q4Rows &pemb, int n_groups, const uint32_t *codes,
                                    int n_frames, float *out, int ld, hipStream_t s);
hipError_t enqueue_add_rows(const float *a, int lda, const float *b, int ldb, float *out, int ldo, int rows, int n,
                            hipStream_t s);
hipError_t enqueue_fill_rows(float *x, int64_t n, uint32_t seed, hipStream_t s);
hipError_t enqueue_row_inv(const float *X, int ld, int M, int K, float *inv, hipStream_t s);
hipError_t enqueue_gemm_gateup(const TalkerDev &m, const PrefillWs &pw, int l, int M, hipStream_t s);
hipError_t enqueue_talker_prefill(const TalkerDev &m, const PrefillWs &pw, int M, int64_t start,
                                  float *hidden_out, hipStream_t s);
hipError_t enqueue_decode(const DecoderDev &d, const DecoderWs &ws, const uint32_t *codes, int T, int64_t cut,
                          float *audio, hipStream_t s);
double decode_flops(const DecoderDev &d, int T);
hipError_t enqueue_gateup_timing(const TalkerDev &m, const Workspace &ws, int l, hipStream_t s);
hipError_t enqueue_attn_timing(const TalkerDev &m, const Workspace &ws, int l, int slot, int64_t pos,
                               const DevState *st, int attn_pg, hipStream_t s);

}  // namespace qtts
