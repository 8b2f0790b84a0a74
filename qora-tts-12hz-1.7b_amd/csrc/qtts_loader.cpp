// qtts_loader.cpp — reads the talker, predictor and speech-decoder sections
// of a `.qora-tts` model file straight into a context.
//
// Stream layout (save.rs:23-137, gemv.rs:595-687), all little-endian:
//   "QTTS" u32 version=1 u8 format (1 = Q4)
//   talker:  u32 n_layers hidden text_hidden n_heads n_kv_heads head_dim
//            n_kv_groups, u32 n_sections, u32 sections[n]
//            per layer: W q k v o, f16v q_norm k_norm, W gate up down,
//                       f16v input_norm post_norm
//            W codec_emb text_emb fc1, f32v fc1_bias, W fc2, f32v fc2_bias,
//            W codec_head, f16v final_norm, f32v rope_cos rope_sin
//   predictor: u32 n_layers hidden n_heads n_kv_heads head_dim n_kv_groups,
//            u8 has_proj [W proj, f32v bias], u32 n_emb, W emb[n],
//            layers as above, u32 n_heads_lm, W heads[n], f16v final_norm,
//            f32v rope_cos rope_sin
//   W    = u64 k, u64 n, u64 len + bytes (packed), u64 len + len*2 (f16 scales)
//   f16v = u64 len + len*2 bytes;  f32v = u64 len + len*4 bytes
//   speech decoder (save.rs:171-260; read when bytes follow the predictor):
//            u32 hidden n_heads head_dim inter sliding_window codebook_dim,
//            f32v first_codebook first_output_proj, u32 n_rest,
//            f32v rest[n_rest], f32v rest_output_proj, C pre_conv,
//            f32v tf_input_w tf_input_b, u32 n_tf, per layer f32v q k v o
//            gate up down input_norm post_norm attn_scale mlp_scale,
//            f32v tf_norm tf_output_w tf_output_b, u32 n_up, per stage
//            u32 channels, CT conv_t, DW dw_conv, f32v norm_w norm_b pw1_w
//            pw1_b pw2_w pw2_b gamma, C vocos_init, u32 n_blocks, per block
//            f32v pre_alpha pre_beta, CT upsample, u32 n_res, per residual
//            f32v a1_alpha a1_beta, C conv1, f32v a2_alpha a2_beta, C conv2;
//            f32v final_alpha final_beta, C output_conv, f32v rope_cos rope_sin
//   C  = u32 in out kernel stride padding dilation, f32v weight bias
//   CT = u32 in out kernel stride padding, f32v weight bias
//   DW = u32 channels kernel padding, f32v weight bias
// The speaker-encoder section that may follow is not read.
#include "../../include/qtts.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <vector>

namespace {

struct Reader {
    const uint8_t *p, *end;
    bool ok = true;
    template <class T>
    T get()
    {
        T v{};
        if ((size_t)(end - p) < sizeof(T)) { ok = false; return v; }
        memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    const uint8_t *bytes(uint64_t n)
    {
        if ((uint64_t)(end - p) < n) { ok = false; return nullptr; }
        const uint8_t *r = p;
        p += n;
        return r;
    }
    // read_f16_vec_io / read_f32_vec_io / read_bytes_io (gemv.rs:645-670)
    const uint8_t *vec(uint64_t elem, uint64_t *len)
    {
        const uint64_t n = get<uint64_t>();
        if (!ok || n > (uint64_t)(end - p) / elem) { ok = false; return nullptr; }
        *len = n;
        return bytes(n * elem);
    }
    // read_weight_io, format 1 (gemv.rs:672-687)
    qtts_q4_host weight()
    {
        qtts_q4_host w{};
        w.k = (int64_t)get<uint64_t>();
        w.n = (int64_t)get<uint64_t>();
        uint64_t pl = 0, sl = 0;
        w.packed = vec(1, &pl);
        w.scales = (const uint16_t *)vec(2, &sl);
        if (ok && (w.k <= 0 || w.n <= 0 || pl != (uint64_t)(w.k * (w.n / 32) * 16) ||
                   sl != (uint64_t)(w.k * (w.n / 32))))
            ok = false;
        return w;
    }
    const uint16_t *f16v(uint64_t expect)
    {
        uint64_t n = 0;
        const uint8_t *d = vec(2, &n);
        if (ok && expect && n != expect) ok = false;
        return (const uint16_t *)d;
    }
    const float *f32v(uint64_t expect, uint64_t *got = nullptr)
    {
        uint64_t n = 0;
        const uint8_t *d = vec(4, &n);
        if (ok && expect && n != expect) ok = false;
        if (got) *got = n;
        return (const float *)d;
    }
};

// f32 vectors of the decoder section, copied out of the mapping into
// 4-byte-aligned storage (the stream has no alignment).
struct F32Store {
    std::vector<std::vector<float>> bufs;
    const float *take(Reader &r, uint64_t expect, uint64_t *got = nullptr)
    {
        uint64_t n = 0;
        const uint8_t *d = r.vec(4, &n);
        if (!r.ok || (expect && n != expect) || n == 0) {
            r.ok = false;
            return nullptr;
        }
        if (got) *got = n;
        bufs.emplace_back(n);
        memcpy(bufs.back().data(), d, n * 4);
        return bufs.back().data();
    }
};

uint64_t u32v(Reader &r) { return r.get<uint32_t>(); }

void read_conv(Reader &r, F32Store &st, qtts_conv1d_host &c)
{
    c.in_channels = (int32_t)u32v(r);
    c.out_channels = (int32_t)u32v(r);
    c.kernel_size = (int32_t)u32v(r);
    c.stride = (int32_t)u32v(r);
    c.padding = (int32_t)u32v(r);
    c.dilation = (int32_t)u32v(r);
    if (!r.ok || c.in_channels < 1 || c.out_channels < 1 || c.kernel_size < 1 || c.in_channels > (1 << 16) ||
        c.out_channels > (1 << 16) || c.kernel_size > 64) {
        r.ok = false;
        return;
    }
    c.weight = st.take(r, (uint64_t)c.out_channels * c.in_channels * c.kernel_size);
    c.bias = st.take(r, (uint64_t)c.out_channels);
}

void read_convt(Reader &r, F32Store &st, qtts_convt1d_host &c)
{
    c.in_channels = (int32_t)u32v(r);
    c.out_channels = (int32_t)u32v(r);
    c.kernel_size = (int32_t)u32v(r);
    c.stride = (int32_t)u32v(r);
    c.padding = (int32_t)u32v(r);
    if (!r.ok || c.in_channels < 1 || c.out_channels < 1 || c.kernel_size < 1 || c.in_channels > (1 << 16) ||
        c.out_channels > (1 << 16) || c.kernel_size > 64) {
        r.ok = false;
        return;
    }
    c.weight = st.take(r, (uint64_t)c.in_channels * c.out_channels * c.kernel_size);
    c.bias = st.take(r, (uint64_t)c.out_channels);
}

void read_dw(Reader &r, F32Store &st, qtts_dwconv_host &c)
{
    c.channels = (int32_t)u32v(r);
    c.kernel_size = (int32_t)u32v(r);
    c.padding = (int32_t)u32v(r);
    if (!r.ok || c.channels < 1 || c.kernel_size < 1 || c.channels > (1 << 16) || c.kernel_size > 64) {
        r.ok = false;
        return;
    }
    c.weight = st.take(r, (uint64_t)c.channels * c.kernel_size);
    c.bias = st.take(r, (uint64_t)c.channels);
}

// Everything a decoder host descriptor points at.
struct DecoderParts {
    F32Store st;
    std::vector<const float *> rest;
    std::vector<qtts_dec_layer_host> layers;
    std::vector<qtts_upsample_host> ups;
    std::vector<std::vector<qtts_vocos_res_host>> res;
    std::vector<qtts_vocos_block_host> blocks;
};

// load_decoder_weights (save.rs:446-552); sizes the reference derives from
// vector lengths (codebook size, vq dim, ConvNeXt width) are derived the
// same way and every vector's length is checked against them.
bool read_decoder(Reader &r, DecoderParts &P, qtts_decoder_host &d)
{
    F32Store &st = P.st;
    d.hidden = (int32_t)u32v(r);
    d.n_heads = (int32_t)u32v(r);
    d.head_dim = (int32_t)u32v(r);
    d.inter = (int32_t)u32v(r);
    d.sliding_window = (int32_t)u32v(r);
    d.codebook_dim = (int32_t)u32v(r);
    if (!r.ok || d.hidden < 1 || d.hidden > 65536 || d.n_heads < 1 || d.n_heads > 1024 || d.head_dim < 2 ||
        d.head_dim > 1024 || d.inter < 1 || d.inter > (1 << 20) || d.codebook_dim < 1 || d.codebook_dim > 65536)
        return false;
    const uint64_t D = (uint64_t)d.codebook_dim, H = (uint64_t)d.hidden, A = (uint64_t)d.n_heads * d.head_dim;
    const uint64_t I = (uint64_t)d.inter;
    uint64_t cbl = 0, pl = 0;
    d.first_codebook = st.take(r, 0, &cbl);
    d.first_output_proj = st.take(r, 0, &pl);
    if (!r.ok || cbl % D || pl % D) return false;
    d.codebook_size = (int32_t)(cbl / D);
    d.vq_dim = (int32_t)(pl / D);
    const uint32_t n_rest = r.get<uint32_t>();
    if (!r.ok || n_rest > 15) return false;
    P.rest.resize(n_rest);
    for (auto &c : P.rest) c = st.take(r, cbl);
    d.rest_codebooks = P.rest.data();
    d.n_rest = (int32_t)n_rest;
    d.rest_output_proj = st.take(r, pl);
    read_conv(r, st, d.pre_conv);
    if (!r.ok) return false;
    d.latent = d.pre_conv.out_channels;
    const uint64_t LAT = (uint64_t)d.latent;
    d.tf_input_w = st.take(r, LAT * H);
    d.tf_input_b = st.take(r, H);
    const uint32_t n_tf = r.get<uint32_t>();
    if (!r.ok || n_tf > 256) return false;
    P.layers.resize(n_tf);
    for (auto &L : P.layers) {
        L.q_proj = st.take(r, H * A);
        L.k_proj = st.take(r, H * A);
        L.v_proj = st.take(r, H * A);
        L.o_proj = st.take(r, A * H);
        L.gate_proj = st.take(r, H * I);
        L.up_proj = st.take(r, H * I);
        L.down_proj = st.take(r, I * H);
        L.input_norm = st.take(r, H);
        L.post_attn_norm = st.take(r, H);
        L.attn_scale = st.take(r, H);
        L.mlp_scale = st.take(r, H);
    }
    d.tf_layers = P.layers.data();
    d.n_tf_layers = (int32_t)n_tf;
    d.tf_norm = st.take(r, H);
    d.tf_output_w = st.take(r, H * LAT);
    d.tf_output_b = st.take(r, LAT);
    const uint32_t n_up = r.get<uint32_t>();
    if (!r.ok || n_up > 16) return false;
    P.ups.resize(n_up);
    for (auto &U : P.ups) {
        U.channels = (int32_t)u32v(r);
        if (!r.ok || U.channels < 1 || U.channels > 65536) return false;
        const uint64_t ch = (uint64_t)U.channels;
        read_convt(r, st, U.conv_t);
        read_dw(r, st, U.dw_conv);
        U.norm_w = st.take(r, ch);
        U.norm_b = st.take(r, ch);
        uint64_t w1 = 0;
        U.pw1_w = st.take(r, 0, &w1);
        if (!r.ok || w1 % ch) return false;
        U.inner = (int32_t)(w1 / ch);
        U.pw1_b = st.take(r, (uint64_t)U.inner);
        U.pw2_w = st.take(r, (uint64_t)U.inner * ch);
        U.pw2_b = st.take(r, ch);
        U.gamma = st.take(r, ch);
    }
    d.upsample = P.ups.data();
    d.n_upsample = (int32_t)n_up;
    read_conv(r, st, d.vocos_init);
    const uint32_t n_vb = r.get<uint32_t>();
    if (!r.ok || n_vb > 16) return false;
    P.blocks.resize(n_vb);
    P.res.resize(n_vb);
    int32_t ch = d.vocos_init.out_channels;
    for (uint32_t b = 0; b < n_vb; b++) {
        qtts_vocos_block_host &B = P.blocks[b];
        B.pre_snake_alpha = st.take(r, (uint64_t)ch);
        B.pre_snake_beta = st.take(r, (uint64_t)ch);
        read_convt(r, st, B.upsample);
        if (!r.ok) return false;
        ch = B.upsample.out_channels;
        const uint32_t n_res = r.get<uint32_t>();
        if (!r.ok || n_res > 16) return false;
        P.res[b].resize(n_res);
        for (auto &R : P.res[b]) {
            R.act1_alpha = st.take(r, (uint64_t)ch);
            R.act1_beta = st.take(r, (uint64_t)ch);
            read_conv(r, st, R.conv1);
            R.act2_alpha = st.take(r, (uint64_t)ch);
            R.act2_beta = st.take(r, (uint64_t)ch);
            read_conv(r, st, R.conv2);
        }
        B.residuals = P.res[b].data();
        B.n_residuals = (int32_t)n_res;
    }
    d.vocos_blocks = P.blocks.data();
    d.n_vocos_blocks = (int32_t)n_vb;
    d.final_snake_alpha = st.take(r, (uint64_t)ch);
    d.final_snake_beta = st.take(r, (uint64_t)ch);
    read_conv(r, st, d.output_conv);
    uint64_t nc = 0, ns = 0;
    d.rope_cos = st.take(r, 0, &nc);
    d.rope_sin = st.take(r, 0, &ns);
    if (!r.ok || nc != ns || nc % (uint64_t)(d.head_dim / 2)) return false;
    d.rope_max_pos = (int64_t)(nc / (d.head_dim / 2));
    return true;
}

void read_layer(Reader &r, qtts_layer_host &L, uint64_t head_dim, uint64_t hidden)
{
    L.q_proj = r.weight();
    L.k_proj = r.weight();
    L.v_proj = r.weight();
    L.o_proj = r.weight();
    L.q_norm = r.f16v(head_dim);
    L.k_norm = r.f16v(head_dim);
    L.gate_proj = r.weight();
    L.up_proj = r.weight();
    L.down_proj = r.weight();
    L.input_norm = r.f16v(hidden);
    L.post_attn_norm = r.f16v(hidden);
}

}  // namespace

extern "C" int qtts_model_load_qtts(qtts_ctx *ctx, const char *path)
{
    if (!ctx || !path) return QTTS_ERR_INVALID;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return QTTS_ERR_IO;
    struct stat sb;
    if (fstat(fd, &sb) != 0 || sb.st_size < 9) {
        close(fd);
        return QTTS_ERR_IO;
    }
    void *map = mmap(nullptr, (size_t)sb.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return QTTS_ERR_IO;
    Reader r{(const uint8_t *)map, (const uint8_t *)map + sb.st_size};

    int rc = QTTS_ERR_IO;
    std::vector<qtts_layer_host> tl, pl;
    std::vector<qtts_q4_host> emb, heads;
    qtts_talker_host t{};
    qtts_predictor_host p{};
    DecoderParts dparts;
    qtts_decoder_host dec{};
    do {
        const uint8_t *magic = r.bytes(4);                       // save.rs:265-269
        if (!r.ok || memcmp(magic, "QTTS", 4) != 0) break;
        if (r.get<uint32_t>() != 1u) break;                      // save.rs:270-273
        const uint8_t fmt = r.get<uint8_t>();                    // save.rs:274
        if (!r.ok) break;
        if (fmt != 1) { rc = QTTS_ERR_UNSUPPORTED; break; }      // F16 weights: not on the device path

        // talker (save.rs:300-351)
        t.n_layers = (int32_t)r.get<uint32_t>();
        t.hidden = (int32_t)r.get<uint32_t>();
        t.text_hidden = (int32_t)r.get<uint32_t>();
        t.n_heads = (int32_t)r.get<uint32_t>();
        t.n_kv_heads = (int32_t)r.get<uint32_t>();
        t.head_dim = (int32_t)r.get<uint32_t>();
        (void)r.get<uint32_t>();                                 // n_kv_groups
        const uint32_t nsec = r.get<uint32_t>();
        // the device kernels are built for 128-wide heads (both models' head_dim);
        // anything else is refused before the layers are read
        if (!r.ok || nsec > 16 || t.n_layers <= 0 || t.n_layers > 256 || t.head_dim != 128) break;
        for (uint32_t i = 0; i < nsec; i++) (void)r.get<uint32_t>();
        tl.resize(t.n_layers);
        for (auto &L : tl) read_layer(r, L, t.head_dim, t.hidden);
        t.layers = tl.data();
        t.codec_embedding = r.weight();
        t.text_embedding = r.weight();
        t.text_fc1 = r.weight();
        t.text_fc1_bias = r.f32v((uint64_t)t.text_fc1.n);
        t.text_fc2 = r.weight();
        t.text_fc2_bias = r.f32v((uint64_t)t.text_fc2.n);
        t.codec_head = r.weight();
        t.final_norm = r.f16v(t.hidden);
        uint64_t nc = 0, ns = 0;
        t.rope_cos = r.f32v(0, &nc);
        t.rope_sin = r.f32v(0, &ns);
        if (!r.ok || nc != ns || nc % (uint64_t)(t.head_dim / 2)) break;
        t.rope_max_pos = (int64_t)(nc / (t.head_dim / 2));
        t.inter = (int32_t)tl[0].gate_proj.n;
        t.vocab = (int32_t)t.codec_head.n;

        // predictor (save.rs:353-409)
        p.n_layers = (int32_t)r.get<uint32_t>();
        p.hidden = (int32_t)r.get<uint32_t>();
        p.n_heads = (int32_t)r.get<uint32_t>();
        p.n_kv_heads = (int32_t)r.get<uint32_t>();
        p.head_dim = (int32_t)r.get<uint32_t>();
        (void)r.get<uint32_t>();
        const uint8_t has_proj = r.get<uint8_t>();
        if (!r.ok || p.n_layers <= 0 || p.n_layers > 64 || p.head_dim != 128) break;
        p.has_input_proj = has_proj == 1;
        if (p.has_input_proj) {
            p.input_proj = r.weight();
            p.input_proj_bias = r.f32v((uint64_t)p.input_proj.n);
        }
        const uint32_t nemb = r.get<uint32_t>();
        if (!r.ok || nemb == 0 || nemb > 64) break;
        emb.resize(nemb);
        for (auto &e : emb) e = r.weight();
        pl.resize(p.n_layers);
        for (auto &L : pl) read_layer(r, L, p.head_dim, p.hidden);
        const uint32_t nheads = r.get<uint32_t>();
        if (!r.ok || nheads != nemb) break;
        heads.resize(nheads);
        for (auto &h : heads) h = r.weight();
        p.final_norm = r.f16v(p.hidden);
        uint64_t pc = 0, ps = 0;
        p.rope_cos = r.f32v(0, &pc);
        p.rope_sin = r.f32v(0, &ps);
        if (!r.ok || pc != ps || pc % (uint64_t)(p.head_dim / 2)) break;
        p.rope_max_pos = (int64_t)(pc / (p.head_dim / 2));
        p.layers = pl.data();
        p.codec_embeddings = emb.data();
        p.lm_heads = heads.data();
        p.n_groups = (int32_t)nemb;
        p.inter = (int32_t)pl[0].gate_proj.n;
        p.vocab = (int32_t)heads[0].n;
        // speech decoder, when the file goes on (a malformed section fails
        // the load before anything is uploaded)
        const bool has_decoder = r.p < r.end;
        if (has_decoder && !read_decoder(r, dparts, dec)) break;
        rc = qtts_model_upload(ctx, &t, &p);
        if (rc == QTTS_OK && has_decoder) rc = qtts_decoder_upload(ctx, &dec);
    } while (0);
    munmap(map, (size_t)sb.st_size);
    return rc;
}

// ---------------------------------------------------------------------------
// The older "QORA-TTS-Q4" container (loader.rs:47-127 read, 724-882 mapped):
//   16-byte header starting "QORA-TTS-Q4", u32 version, u32 n_tensors, then
//   per tensor: u32 name_len + name, u32 rank + u32 dims[rank], u8 format,
//     format 1 (Q4): u32 n_scales + f16 scales, u32 n_packed + bytes
//     format 0 (F16): u32 n_values + f16 values
//   little-endian.  Linear weights and embeddings are stored [in][out]
//   (shape [k, n]) in the F1 layout; norms and biases are F16 vectors.
// The file holds no configuration or RoPE tables: the shapes come from the
// tensors, and the tables from the caller (the reference builds them from
// config.json, loader.rs:770-775 and 869-881).
// ---------------------------------------------------------------------------

#include <map>
#include <string>

namespace {

struct LegacyTensor {
    std::vector<uint32_t> shape;
    uint8_t format = 0;
    const uint16_t *f16 = nullptr;   // scales (Q4) or values (F16)
    uint64_t n16 = 0;
    const uint8_t *packed = nullptr;
    uint64_t npacked = 0;
};

bool read_legacy_tensors(Reader &r, std::map<std::string, LegacyTensor> &m)
{
    const uint8_t *hdr = r.bytes(16);
    if (!r.ok || memcmp(hdr, "QORA-TTS-Q4", 11) != 0) return false;
    (void)r.get<uint32_t>();                                   // version
    const uint32_t nt = r.get<uint32_t>();
    if (!r.ok || nt > (1u << 20)) return false;
    for (uint32_t i = 0; i < nt; i++) {
        const uint32_t nl = r.get<uint32_t>();
        const uint8_t *nm = r.bytes(nl);
        const uint32_t rank = r.get<uint32_t>();
        if (!r.ok || rank > 8) return false;
        LegacyTensor t;
        for (uint32_t d = 0; d < rank; d++) t.shape.push_back(r.get<uint32_t>());
        t.format = r.get<uint8_t>();
        t.n16 = r.get<uint32_t>();
        t.f16 = (const uint16_t *)r.bytes(t.n16 * 2);
        if (t.format == 1) {
            t.npacked = r.get<uint32_t>();
            t.packed = r.bytes(t.npacked);
        } else if (t.format != 0) {
            return false;
        }
        if (!r.ok) return false;
        m[std::string((const char *)nm, nl)] = std::move(t);
    }
    return true;
}

struct LegacyModel {
    std::map<std::string, LegacyTensor> m;
    std::vector<std::vector<float>> f32;   // F16 biases widened to f32
    int status = QTTS_OK;                  // first problem met
    void fail(int s) { if (status == QTTS_OK) status = s; }
    const LegacyTensor *find(const std::string &k)
    {
        auto it = m.find(k);
        if (it == m.end()) { fail(QTTS_ERR_IO); return nullptr; }
        return &it->second;
    }
    // binary_to_weight (loader.rs:148-170); F16 weights are not on the device path
    qtts_q4_host weight(const std::string &k)
    {
        qtts_q4_host w{};
        const LegacyTensor *t = find(k);
        if (!t) return w;
        if (t->shape.size() != 2) { fail(QTTS_ERR_IO); return w; }
        if (t->format != 1) { fail(QTTS_ERR_UNSUPPORTED); return w; }
        w.k = t->shape[0];
        w.n = t->shape[1];
        if (w.k <= 0 || w.n <= 0 || w.n % 32 || t->npacked != (uint64_t)(w.k * (w.n / 2)) ||
            t->n16 != (uint64_t)(w.k * (w.n / 32))) {
            fail(QTTS_ERR_IO);
            return w;
        }
        w.packed = t->packed;
        w.scales = t->f16;
        return w;
    }
    // binary_to_f16 (loader.rs:139-145)
    const uint16_t *f16v(const std::string &k, uint64_t expect)
    {
        const LegacyTensor *t = find(k);
        if (!t) return nullptr;
        if (t->format != 0 || t->n16 != expect) { fail(QTTS_ERR_IO); return nullptr; }
        return t->f16;
    }
    // binary_to_f32 (loader.rs:130-136): f16 -> f32 is exact
    const float *f32v(const std::string &k, uint64_t expect)
    {
        const uint16_t *h = f16v(k, expect);
        if (!h) return nullptr;
        f32.emplace_back(expect);
        for (uint64_t i = 0; i < expect; i++) {
            uint16_t b;
            memcpy(&b, h + i, 2);
            f32.back()[i] = half_to_float(b);
        }
        return f32.back().data();
    }
    static float half_to_float(uint16_t h)
    {
        const uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1F, f = h & 0x3FF;
        uint32_t bits;
        if (e == 0) {
            if (f == 0) {
                bits = s;
            } else {                               // subnormal: renormalise
                int sh = 0;
                uint32_t ff = f;
                while (!(ff & 0x400)) { ff <<= 1; sh++; }
                bits = s | ((uint32_t)(113 - sh) << 23) | ((ff & 0x3FF) << 13);
            }
        } else if (e == 31) {
            bits = s | 0x7F800000u | (f << 13);
        } else {
            bits = s | ((e + 112) << 23) | (f << 13);
        }
        float v;
        memcpy(&v, &bits, 4);
        return v;
    }
    void layer(const std::string &pre, qtts_layer_host &L, int64_t hidden)
    {
        L.q_proj = weight(pre + ".self_attn.q_proj.weight");
        L.k_proj = weight(pre + ".self_attn.k_proj.weight");
        L.v_proj = weight(pre + ".self_attn.v_proj.weight");
        L.o_proj = weight(pre + ".self_attn.o_proj.weight");
        const LegacyTensor *qn = find(pre + ".self_attn.q_norm.weight");
        const uint64_t hd = qn ? qn->n16 : 0;
        L.q_norm = f16v(pre + ".self_attn.q_norm.weight", hd);
        L.k_norm = f16v(pre + ".self_attn.k_norm.weight", hd);
        L.gate_proj = weight(pre + ".mlp.gate_proj.weight");
        L.up_proj = weight(pre + ".mlp.up_proj.weight");
        L.down_proj = weight(pre + ".mlp.down_proj.weight");
        L.input_norm = f16v(pre + ".input_layernorm.weight", (uint64_t)hidden);
        L.post_attn_norm = f16v(pre + ".post_attention_layernorm.weight", (uint64_t)hidden);
    }
    int count(const std::string &pre, const std::string &post, int max)
    {
        int n = 0;
        while (n < max && m.count(pre + std::to_string(n) + post)) n++;
        return n;
    }
};

}  // namespace

extern "C" int qtts_model_load_qora_q4(qtts_ctx *ctx, const char *path, const qtts_rope_tables *rope)
{
    if (!ctx || !path || !rope || !rope->talker_cos || !rope->talker_sin || !rope->pred_cos || !rope->pred_sin ||
        rope->talker_max_pos <= 0 || rope->pred_max_pos <= 0)
        return QTTS_ERR_INVALID;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return QTTS_ERR_IO;
    struct stat sb;
    if (fstat(fd, &sb) != 0 || sb.st_size < 24) {
        close(fd);
        return QTTS_ERR_IO;
    }
    void *map = mmap(nullptr, (size_t)sb.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return QTTS_ERR_IO;
    Reader r{(const uint8_t *)map, (const uint8_t *)map + sb.st_size};
    LegacyModel M;
    int rc = QTTS_ERR_IO;
    std::vector<qtts_layer_host> tl, pl;
    std::vector<qtts_q4_host> emb, heads;
    qtts_talker_host t{};
    qtts_predictor_host p{};
    do {
        if (!read_legacy_tensors(r, M.m)) break;
        // talker (load_talker_binary, loader.rs:724-799)
        const std::string tp = "talker.model.layers.";
        t.n_layers = M.count(tp, ".self_attn.q_proj.weight", 256);
        if (t.n_layers == 0) break;
        const qtts_q4_host q0 = M.weight(tp + "0.self_attn.q_proj.weight");
        const qtts_q4_host k0 = M.weight(tp + "0.self_attn.k_proj.weight");
        const LegacyTensor *qn0 = M.find(tp + "0.self_attn.q_norm.weight");
        if (M.status != QTTS_OK || !qn0 || qn0->n16 == 0) break;
        t.hidden = (int32_t)q0.k;
        t.head_dim = (int32_t)qn0->n16;
        t.n_heads = (int32_t)(q0.n / t.head_dim);
        t.n_kv_heads = (int32_t)(k0.n / t.head_dim);
        tl.resize(t.n_layers);
        for (int i = 0; i < t.n_layers; i++) M.layer(tp + std::to_string(i), tl[i], t.hidden);
        t.layers = tl.data();
        t.codec_embedding = M.weight("talker.model.codec_embedding.weight");
        t.text_embedding = M.weight("talker.model.text_embedding.weight");
        t.text_fc1 = M.weight("talker.text_projection.linear_fc1.weight");
        t.text_fc1_bias = M.f32v("talker.text_projection.linear_fc1.bias", (uint64_t)t.text_fc1.n);
        t.text_fc2 = M.weight("talker.text_projection.linear_fc2.weight");
        t.text_fc2_bias = M.f32v("talker.text_projection.linear_fc2.bias", (uint64_t)t.text_fc2.n);
        t.codec_head = M.weight("talker.codec_head.weight");
        t.final_norm = M.f16v("talker.model.norm.weight", (uint64_t)t.hidden);
        t.text_hidden = (int32_t)t.text_embedding.n;
        t.inter = (int32_t)tl[0].gate_proj.n;
        t.vocab = (int32_t)t.codec_head.n;
        t.rope_cos = rope->talker_cos;
        t.rope_sin = rope->talker_sin;
        t.rope_max_pos = rope->talker_max_pos;
        // code predictor (load_code_predictor_binary, loader.rs:801-882)
        const std::string cp = "talker.code_predictor.";
        p.n_layers = M.count(cp + "model.layers.", ".self_attn.q_proj.weight", 64);
        p.n_groups = M.count(cp + "model.codec_embedding.", ".weight", 64);
        if (M.status != QTTS_OK || p.n_layers == 0 || p.n_groups == 0 ||
            M.count(cp + "lm_head.", ".weight", 64) != p.n_groups)
            break;
        if (M.m.count(cp + "small_to_mtp_projection.weight")) {
            p.has_input_proj = 1;
            p.input_proj = M.weight(cp + "small_to_mtp_projection.weight");
            p.input_proj_bias = M.f32v(cp + "small_to_mtp_projection.bias", (uint64_t)p.input_proj.n);
        }
        const qtts_q4_host pq0 = M.weight(cp + "model.layers.0.self_attn.q_proj.weight");
        const qtts_q4_host pk0 = M.weight(cp + "model.layers.0.self_attn.k_proj.weight");
        const LegacyTensor *pqn0 = M.find(cp + "model.layers.0.self_attn.q_norm.weight");
        if (M.status != QTTS_OK || !pqn0 || pqn0->n16 == 0) break;
        p.hidden = (int32_t)pq0.k;
        p.head_dim = (int32_t)pqn0->n16;
        p.n_heads = (int32_t)(pq0.n / p.head_dim);
        p.n_kv_heads = (int32_t)(pk0.n / p.head_dim);
        emb.resize(p.n_groups);
        heads.resize(p.n_groups);
        for (int g = 0; g < p.n_groups; g++) {
            emb[g] = M.weight(cp + "model.codec_embedding." + std::to_string(g) + ".weight");
            heads[g] = M.weight(cp + "lm_head." + std::to_string(g) + ".weight");
        }
        pl.resize(p.n_layers);
        for (int i = 0; i < p.n_layers; i++) M.layer(cp + "model.layers." + std::to_string(i), pl[i], p.hidden);
        p.final_norm = M.f16v(cp + "model.norm.weight", (uint64_t)p.hidden);
        p.layers = pl.data();
        p.codec_embeddings = emb.data();
        p.lm_heads = heads.data();
        p.inter = (int32_t)pl[0].gate_proj.n;
        p.vocab = (int32_t)heads[0].n;
        p.rope_cos = rope->pred_cos;
        p.rope_sin = rope->pred_sin;
        p.rope_max_pos = rope->pred_max_pos;
        if (M.status != QTTS_OK) break;
        rc = qtts_model_upload(ctx, &t, &p);
    } while (0);
    if (rc == QTTS_ERR_IO && M.status != QTTS_OK) rc = M.status;
    munmap(map, (size_t)sb.st_size);
    return rc;
}
