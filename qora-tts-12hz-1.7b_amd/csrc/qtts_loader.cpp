// qtts_loader.cpp — reads the talker and predictor sections of a
// `.qora-tts` model file straight into a context.
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
// The decoder and speaker-encoder sections that follow are not read.
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
        if (!r.ok || nsec > 16 || t.n_layers <= 0 || t.n_layers > 256 || t.head_dim <= 0) break;
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
        if (!r.ok || p.n_layers <= 0 || p.n_layers > 64 || p.head_dim <= 0) break;
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
        rc = qtts_model_upload(ctx, &t, &p);
    } while (0);
    munmap(map, (size_t)sb.st_size);
    return rc;
}
