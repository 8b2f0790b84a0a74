// qtts_runtime.cpp — context, weight upload (repack into device tiles),
// KV-cache management, frame graphs and the C ABI declared in
// include/qtts.h.
#include "../../include/qtts.h"
#include "qtts_device.h"
#include "qtts_kernels.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

using namespace qtts;

struct qtts_w {
    Q4Tiled t;
    Q4Rows rows;
    float *x = nullptr, *y = nullptr, *part = nullptr;
    std::vector<void *> allocs;
};

struct qtts_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string err;
    int64_t kv_cap = 4096;

    bool has_model = false;
    TalkerDev tm{};
    PredictorDev pm{};
    std::vector<LayerDev> tlayers, players;
    std::vector<Q4Tiled> pheads;
    std::vector<void *> model_allocs;
    Workspace ws{};
    std::vector<void *> ws_allocs;
    int64_t text_cap = 0;

    DevState *st_gen = nullptr, *st_api = nullptr;   // device
    DevState *h_st = nullptr;                        // pinned host mirror
    uint32_t *h_ring = nullptr;                      // pinned [RING_FRAMES][16]
    uint32_t *d_forced = nullptr;                    // forced codes
    int64_t forced_cap = 0;
    uint32_t *d_codes_api = nullptr;                 // [16]
    uint64_t *d_rng_api = nullptr;
    uint32_t *d_prev_api = nullptr;                  // [4096]

    // legacy loop (generate.rs): the predictor's cache kept across
    // predict_codes calls, and small device buffers
    float *lkv = nullptr;                            // model allocation: [layers][pages][2][8][64][128]
    int32_t *lkv_ptab = nullptr;                     // identity page table
    float *leg_buf = nullptr;                        // side row + logits
    int *d_status = nullptr;
    int64_t lkv_len = 0;
    float *d_io = nullptr;                           // API staging, 2 rows of max(hidden,vocab,4096)
    float *d_io2 = nullptr;
    int64_t io_floats = 0;
    float *d_rmax = nullptr;                         // per-row largest |x| of a GEMM's rows (staging range)
    int64_t rmax_rows = 0;

    hipGraphExec_t frame_exec[2] = {nullptr, nullptr};   // one and two attention pages per workgroup
    bool gen_started = false;
    bool force_sync_err = false;                     // qtts_debug_force_sync_err: armed for the next call

    float *scratch = nullptr;                        // this device's copy of `scratch` (qtts_gemm_q4_noalloc)

    float *d_copy = nullptr;                         // copy-calibration buffers, 2 x copy_floats
    int64_t copy_floats = 0;
    float *d_read = nullptr;                         // streaming-read bound: READ_POOL buffers of READ_BYTES
    uint32_t *d_sink = nullptr;
    bool time_graph = false;                         // qtts_time_*: launches captured in a graph and replayed

    PrefillWs pf{};                                  // batched-prefill rows (allocated on first use)
    void *pf_mem = nullptr;

    // speech decoder (independent of the talker / predictor model)
    bool has_decoder = false;
    DecoderDev dec{};
    std::vector<DecLayer> dec_layers;
    std::vector<DecUpsample> dec_up;
    std::vector<DecVocos> dec_voc;
    std::vector<std::vector<DecVocosRes>> dec_res;
    std::vector<void *> dec_allocs;
    int64_t dec_floats_per_frame = 0;                // largest stage, [channels][positions] per frame
    DecoderWs dws{};
    void *dws_mem = nullptr;

    // Talker KV page pool: 2 * kv_cap/64 physical pages shared by the running
    // sequence and captured prefixes.  seq_ptab is the host copy of the
    // sequence's page table (d_ptab on the device), page_ref counts the
    // holders of each physical page (the sequence, prefixes).
    std::vector<int32_t> seq_ptab, page_ref, free_pages;
    int32_t *d_ptab = nullptr;
    uint64_t model_gen = 0;                          // bumped by every model upload
};

// A kept talker prefix (TalkerPrefixCache, generate_new.rs:317-325; built by
// build_talker_prefix, generate_new.rs:330-355): the
// physical pages holding positions 0..len-1 of every layer.  Full pages are
// shared with the sequences that attach it; the last partial page is its
// own copy.
struct qtts_prefix {
    const qtts_ctx *owner = nullptr;
    uint64_t model_gen = 0;
    int64_t len = 0;
    std::vector<int32_t> pages;
};

// Prompts at least this long take the matrix-core prefill; shorter ones run
// row by row through the decode kernels.  Same for qtts_gemm_q4 rows.
constexpr int64_t MFMA_MIN_ROWS = 16;
constexpr int PREFILL_MAX_ROWS = 1024;   // rows per prefill chunk

// special ids of the prompt layout (generate_new.rs:25-36)
constexpr uint32_t TTS_PAD_ID = 151671, TTS_EOS_ID = 151673, CODEC_BOS_ID = 2149;
constexpr uint32_t IM_START_ID = 151644, ASSISTANT_ID = 77091, NEWLINE_ID = 198, TTS_BOS_ID = 151672;
constexpr uint32_t CODEC_THINK_ID = 2154, CODEC_THINK_BOS_ID = 2156, CODEC_THINK_EOS_ID = 2157, CODEC_PAD_ID = 2148;

// ---------------------------------------------------------------------------
// error helpers
// ---------------------------------------------------------------------------

static int fail(qtts_ctx *c, int code, const char *fmt, ...)
{
    if (c) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        c->err = buf;
    }
    return code;
}

#define HIPCHK(c, x)                                                                       \
    do {                                                                                   \
        hipError_t e_ = (x);                                                               \
        if (e_ != hipSuccess)                                                              \
            return fail((c), e_ == hipErrorOutOfMemory ? QTTS_ERR_OOM : QTTS_ERR_HIP,      \
                        "%s: %s (%s:%d)", #x, hipGetErrorString(e_), __FILE__, __LINE__);  \
    } while (0)

#define RCHK(x)                          \
    do {                                 \
        int r_ = (x);                    \
        if (r_ != QTTS_OK) return r_;    \
    } while (0)

template <class T>
static int dev_alloc(qtts_ctx *c, std::vector<void *> &list, T **p, size_t count)
{
    void *m = nullptr;
    HIPCHK(c, hipMalloc(&m, std::max<size_t>(count * sizeof(T), 256)));
    list.push_back(m);
    *p = (T *)m;
    return QTTS_OK;
}

// ---------------------------------------------------------------------------
// repacking a (column-concatenated) Q4 weight into device tiles
// ---------------------------------------------------------------------------

struct SrcW {
    const uint8_t *packed;
    const uint16_t *scales;
    int64_t k, n;
};

static int env_tile(const char *name, int dflt)
{
    char key[64];
    snprintf(key, sizeof key, "QTTS_TILE_%s", name);
    const char *v = getenv(key);
    if (!v || !*v) return dflt;
    const int x = atoi(v);
    return (x >= 0 && x < TILE_COUNT) ? x : dflt;
}

// Default tile of each weight role (QTTS_TILE_<ROLE> overrides it), chosen by
// a per-role sweep of frames/s on MI355X at the 1.7B shapes.  Wide
// workgroups with few rows per thread (R 2-4) win on the small predictor
// and attention-side weights: more waves share each tile, so the per-lane
// dequant chain and the cross-wave reduction are shorter.
static int default_cfg(const char *role, int64_t k)
{
    const std::string r(role);
    if (r == "TQKV") return TILE_G1_T512_R2;                                    // KC 1024
    if (r == "TO" || r == "PQKV" || r == "PO" || r == "PPROJ") return TILE_G1_T256_R2;   // KC 512
    if (r == "HEAD" || r == "PHEAD") return TILE_G1_T256_R4;                    // KC 1024
    if (r == "TGU") return k <= 2048 ? TILE_G2_T512 : TILE_G2_T256;            // one slice, SiLU epilogue
    if (r == "PGU") {
        if (k <= 1024 && fused_mlp_enabled()) return TILE_G1_T256_R4;           // one slice, one group per tile: gate|up + down in one launch
        return k <= 1024 ? TILE_G2_T256_R4 : TILE_G2_T512;                      // 2 slices, SwiGLU in the down prologue
    }
    if (r == "TDOWN") return TILE_G1_T512_R4;                                   // KC 2048
    if (r == "PDOWN") return fused_mlp_enabled() ? TILE_G1_T256_R2 : TILE_G1_T512_R2;   // KC 512 (6 slices) / 1024
    if (r == "GEMV") return TILE_G1_T256;                                       // standalone Q4 GEMV
    return k <= 2048 ? TILE_G1_T256 : TILE_G8_T256;                             // text fc
}

static int role_cfg(const char *role, int64_t k) { return env_tile(role, default_cfg(role, k)); }

static void parallel_for(int64_t n, const std::function<void(int64_t, int64_t)> &fn);

static float f16_to_f32(uint16_t h)
{
    _Float16 v;
    memcpy(&v, &h, sizeof v);
    return (float)v;
}

// interleave = true (two sources of equal width): groups alternate a0 b0 a1
// b1 ..., so a tile of an even number of groups holds matching pairs.
static int build_tiled(qtts_ctx *c, std::vector<void *> &allocs, const std::vector<SrcW> &srcs, int cfg,
                       Q4Tiled *out, void **mem_out, bool interleave = false)
{
    if (interleave && (srcs.size() != 2 || srcs[0].n != srcs[1].n))
        return fail(c, QTTS_ERR_INVALID, "interleaved weights must be two of equal width");
    if (srcs.empty()) return fail(c, QTTS_ERR_INVALID, "empty weight list");
    const int64_t k = srcs[0].k;
    std::vector<int64_t> g0;   // first group of each source
    int64_t Gt = 0;
    for (const SrcW &s : srcs) {
        if (s.k != k) return fail(c, QTTS_ERR_INVALID, "fused weights disagree on k");
        if (!s.packed || !s.scales || s.k <= 0 || s.n <= 0)
            return fail(c, QTTS_ERR_INVALID, "weight with null data or bad shape (k=%lld n=%lld)",
                        (long long)s.k, (long long)s.n);
        if (srcs.size() > 1 && s.n % 32) return fail(c, QTTS_ERR_INVALID, "fused weight n %% 32 != 0");
        g0.push_back(Gt);
        Gt += s.n / 32;
    }
    if (Gt == 0) return fail(c, QTTS_ERR_INVALID, "weight narrower than one 32-column group");
    const TileShape ts = tile_shape(cfg);
    const int P = ts.T / ts.GB, KC = ts.R * P;
    const int64_t G = (Gt + ts.GB - 1) / ts.GB * ts.GB;
    const int64_t S = (k + KC - 1) / KC, CT = G / ts.GB;
    const int64_t tile_bytes = (int64_t)ts.R * ts.T * 16 + (int64_t)ts.T * ts.R * 2;
    const size_t total = (size_t)(S * CT * tile_bytes);
    std::vector<uint8_t> host(total);
    parallel_for(S * CT, [&](int64_t i0, int64_t i1) {
        for (int64_t item = i0; item < i1; item++) {
            const int64_t s = item / CT, ct = item % CT;
            uint8_t *tile = host.data() + item * tile_bytes;
            uint16_t *scl = (uint16_t *)(tile + (size_t)ts.R * ts.T * 16);
            // thread t -> (group, row offset): one group per wave when the
            // wave count is a multiple of GB, else interleaved by thread
            const bool wave_groups = (ts.T / 64) % ts.GB == 0;
            for (int t = 0; t < ts.T; t++) {
                const int gt = wave_groups ? (t / 64) % ts.GB : t % ts.GB;
                const int pt = wave_groups ? (t / 64) / ts.GB * 64 + t % 64 : t / ts.GB;
                const int64_t g = ct * ts.GB + gt;
                int si = -1;
                int64_t lg = 0;
                if (g < Gt) {
                    if (interleave) {
                        si = (int)(g & 1);
                        lg = g >> 1;
                    } else {
                        si = (int)(std::upper_bound(g0.begin(), g0.end(), g) - g0.begin()) - 1;
                        lg = g - g0[si];
                    }
                }
                for (int r = 0; r < ts.R; r++) {
                    const int64_t row = s * KC + (int64_t)r * P + pt;
                    uint8_t *dst = tile + ((size_t)r * ts.T + t) * 16;
                    uint16_t sc = 0;
                    if (si >= 0 && row < k) {
                        const SrcW &w = srcs[si];
                        const int64_t Gw = w.n / 32;
                        memcpy(dst, w.packed + (size_t)row * Gw * 16 + lg * 16, 16);
                        sc = w.scales[(size_t)row * Gw + lg];
                    } else {
                        memset(dst, 0x88, 16);
                    }
                    scl[(size_t)t * ts.R + r] = sc;
                }
            }
        }
    });
    void *mem = nullptr;
    HIPCHK(c, hipMalloc(&mem, total));
    allocs.push_back(mem);
    HIPCHK(c, hipMemcpy(mem, host.data(), total, hipMemcpyHostToDevice));
    Q4Tiled d{};
    d.data = (const uint8_t *)mem;
    d.k = (int32_t)k;
    int64_t n_all = 0;
    for (const SrcW &s : srcs) n_all += s.n;
    d.n = (int32_t)(srcs.size() > 1 ? Gt * 32 : n_all);
    d.G = (int32_t)G;
    d.S = (int32_t)S;
    d.CT = (int32_t)CT;
    d.KC = KC;
    d.cfg = cfg;
    d.tile_bytes = (int32_t)tile_bytes;
    d.npad = (int32_t)(G * 32);
    d.interleave = interleave ? 1 : 0;
    // The split-f16 matrix path scales the dequantised weights by 2^bshift so
    // that the low half of each split stays a normal f16: the largest
    // |(nibble - 8) * scale| * 2^bshift must stay below 2^15.
    float smax = 0.0f;
    for (const SrcW &w : srcs)
        for (int64_t i = 0; i < w.k * (w.n / 32); i++) smax = std::max(smax, std::fabs(f16_to_f32(w.scales[i])));
    d.bshift = -1;
    for (int b = 12; b >= 0; b--)
        if (8.0f * smax * std::ldexp(1.0f, b) < 32768.0f) {
            d.bshift = b;
            break;
        }
    *out = d;
    if (mem_out) *mem_out = mem;
    return QTTS_OK;
}

static void parallel_for(int64_t n, const std::function<void(int64_t, int64_t)> &fn)
{
    int nt = (int)std::min<int64_t>(std::max(1u, std::thread::hardware_concurrency()), 16);
    if (n < 64 || nt <= 1) { fn(0, n); return; }
    std::vector<std::thread> th;
    const int64_t per = (n + nt - 1) / nt;
    for (int i = 0; i < nt; i++) {
        const int64_t a = i * per, b = std::min(n, a + per);
        if (a >= b) break;
        th.emplace_back([&fn, a, b] { fn(a, b); });
    }
    for (auto &t : th) t.join();
}

// Reference-layout copy of row-indexed tables (embeddings).
static int upload_rows(qtts_ctx *c, std::vector<void *> &allocs, const std::vector<qtts_q4_host> &ws,
                       Q4Rows *out)
{
    const int64_t rows = ws[0].k, n = ws[0].n, G = n / 32;
    for (const auto &w : ws)
        if (w.k != rows || w.n != n || !w.packed || !w.scales)
            return fail(c, QTTS_ERR_INVALID, "embedding tables disagree in shape");
    const size_t pb = (size_t)rows * G * 16, sb = (size_t)rows * G * 2;
    uint8_t *pm = nullptr;
    uint16_t *sm = nullptr;
    RCHK(dev_alloc(c, allocs, &pm, pb * ws.size()));
    RCHK(dev_alloc(c, allocs, &sm, (sb / 2) * ws.size()));
    for (size_t i = 0; i < ws.size(); i++) {
        HIPCHK(c, hipMemcpy(pm + i * pb, ws[i].packed, pb, hipMemcpyHostToDevice));
        HIPCHK(c, hipMemcpy((uint8_t *)sm + i * sb, ws[i].scales, sb, hipMemcpyHostToDevice));
    }
    out->packed = pm;
    out->scales = sm;
    out->rows = (int32_t)rows;
    out->n = (int32_t)n;
    out->G = (int32_t)G;
    return QTTS_OK;
}

template <class T>
static int upload_vec(qtts_ctx *c, std::vector<void *> &allocs, const T *src, size_t count, const T **out)
{
    if (!src) return fail(c, QTTS_ERR_INVALID, "null vector in model descriptor");
    T *d = nullptr;
    RCHK(dev_alloc(c, allocs, &d, count));
    HIPCHK(c, hipMemcpy(d, src, count * sizeof(T), hipMemcpyHostToDevice));
    *out = d;
    return QTTS_OK;
}

static SrcW src_of(const qtts_q4_host &w) { return SrcW{w.packed, w.scales, w.k, w.n}; }

// Largest 2-norm of a column of a Q4 weight (dequantised, in double).
static double q4_max_col_norm(const qtts_q4_host &w)
{
    if (!w.packed || !w.scales || w.n < 32) return 0.0;
    const int64_t G = w.n / 32;
    std::vector<double> ss((size_t)G * 32, 0.0);
    for (int64_t k = 0; k < w.k; k++)
        for (int64_t g = 0; g < G; g++) {
            const double sc = f16_max_abs(&w.scales[k * G + g], 1);   // |scale|: only squares are summed
            const uint8_t *p = w.packed + (k * G + g) * 16;
            for (int j = 0; j < 32; j++) {
                const double v = (double)((int)((p[j >> 1] >> (4 * (j & 1))) & 15) - 8) * sc;
                ss[(size_t)g * 32 + j] += v * v;
            }
        }
    double m = 0.0;
    for (double v : ss) m = std::max(m, v);
    return std::sqrt(m);
}

static int upload_layer(qtts_ctx *c, const qtts_layer_host &L, int hidden, int head_dim, LayerDev *out,
                        bool predictor)
{
    auto &A = c->model_allocs;
    const char *pfx = predictor ? "P" : "T";
    char name[32];
    snprintf(name, sizeof name, "%sQKV", pfx);
    RCHK(build_tiled(c, A, {src_of(L.q_proj), src_of(L.k_proj), src_of(L.v_proj)}, role_cfg(name, L.q_proj.k),
                     &out->qkv, nullptr));
    snprintf(name, sizeof name, "%sO", pfx);
    RCHK(build_tiled(c, A, {src_of(L.o_proj)}, role_cfg(name, L.o_proj.k), &out->o, nullptr));
    snprintf(name, sizeof name, "%sGU", pfx);
    RCHK(build_tiled(c, A, {src_of(L.gate_proj), src_of(L.up_proj)}, role_cfg(name, L.gate_proj.k),
                     &out->gate_up, nullptr, true));
    snprintf(name, sizeof name, "%sDOWN", pfx);
    RCHK(build_tiled(c, A, {src_of(L.down_proj)}, role_cfg(name, L.down_proj.k), &out->down, nullptr));
    RCHK(upload_vec(c, A, L.q_norm, head_dim, &out->q_norm));
    RCHK(upload_vec(c, A, L.k_norm, head_dim, &out->k_norm));
    RCHK(upload_vec(c, A, L.input_norm, hidden, &out->input_norm));
    RCHK(upload_vec(c, A, L.post_attn_norm, hidden, &out->post_norm));
    out->in_shift = norm_shift(L.input_norm, hidden);
    out->post_shift = norm_shift(L.post_attn_norm, hidden);
    out->q_shift = attn_shift(std::sqrt((double)head_dim) * f16_max_abs(L.q_norm, head_dim));
    out->k_shift = attn_shift(std::sqrt((double)head_dim) * f16_max_abs(L.k_norm, head_dim));
    out->v_shift = attn_shift(std::sqrt((double)hidden) * f16_max_abs(L.input_norm, hidden) *
                              q4_max_col_norm(L.v_proj));
    if (L.q_proj.n != 16 * HEAD_DIM || L.k_proj.n != 8 * HEAD_DIM || L.v_proj.n != 8 * HEAD_DIM)
        return fail(c, QTTS_ERR_UNSUPPORTED, "device path expects 16 q heads / 8 kv heads of 128");
    if (L.o_proj.n != hidden || L.down_proj.n != hidden || L.q_proj.k != hidden)
        return fail(c, QTTS_ERR_INVALID, "layer shapes disagree with hidden size %d", hidden);
    return QTTS_OK;
}

// ---------------------------------------------------------------------------
// context
// ---------------------------------------------------------------------------

static void free_list(std::vector<void *> &l)
{
    for (void *p : l) hipFree(p);
    l.clear();
}

static void drop_graph(qtts_ctx *c)
{
    for (auto &e : c->frame_exec) {
        if (e) hipGraphExecDestroy(e);
        e = nullptr;
    }
}

// ---------------------------------------------------------------------------
// scratch of the allocation-free entry point (qtts_gemm_q4_noalloc): the
// split-K partial sums of its GEMV passes live in this file-scope device
// array, one copy per GPU, held until the process ends.  Host code never
// passes the array's name to a kernel (on the host it is only a stand-in):
// its device address is looked up once per device, with that device
// current, when the first context on the device is created.
// ---------------------------------------------------------------------------

constexpr size_t SCRATCH_FLOATS = (size_t)1 << 20;    // 4 MiB
constexpr int SCRATCH_MAX_DEVICES = 64;
static __device__ __align__(256) float scratch[SCRATCH_FLOATS];
static std::mutex g_scratch_mu;
static float *g_scratch_dev[SCRATCH_MAX_DEVICES];      // device address of `scratch` per device

static hipError_t scratch_address(int device, float **out)
{
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (device < 0 || device >= SCRATCH_MAX_DEVICES) return hipErrorInvalidDevice;
    if (!g_scratch_dev[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_dev[device] = (float *)p;
    }
    *out = g_scratch_dev[device];
    return hipSuccess;
}

extern "C" int qtts_ctx_create(int device, int64_t kv_capacity, qtts_ctx **out)
{
    if (!out) return QTTS_ERR_INVALID;
    *out = nullptr;
    qtts_ctx *c = new qtts_ctx();
    c->device = device;
    c->kv_cap = kv_capacity <= 0 ? 4096 : kv_capacity;
    if (c->kv_cap > (int64_t)MAX_CHUNKS * KV_PAGE || c->kv_cap % KV_PAGE) {
        delete c;
        return QTTS_ERR_CAPACITY;
    }
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) {
        delete c;
        return QTTS_ERR_HIP;
    }
    if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return QTTS_ERR_HIP;
    }
    if (scratch_address(device, &c->scratch) != hipSuccess) {
        hipStreamDestroy(c->stream);
        delete c;
        return QTTS_ERR_HIP;
    }
    bool ok = hipMalloc(&c->st_gen, sizeof(DevState)) == hipSuccess &&
              hipMalloc(&c->st_api, sizeof(DevState)) == hipSuccess &&
              hipHostMalloc(&c->h_st, sizeof(DevState), hipHostMallocDefault) == hipSuccess &&
              hipHostMalloc(&c->h_ring, sizeof(uint32_t) * RING_FRAMES * 16 * 2, hipHostMallocDefault) == hipSuccess &&
              hipMalloc(&c->d_codes_api, sizeof(uint32_t) * 16) == hipSuccess &&
              hipMalloc(&c->d_rng_api, sizeof(uint64_t)) == hipSuccess &&
              hipMalloc(&c->d_prev_api, sizeof(uint32_t) * 4096) == hipSuccess &&
              hipMalloc(&c->d_status, sizeof(int) * 2) == hipSuccess;
    if (!ok) {
        qtts_ctx_destroy(c);
        return QTTS_ERR_OOM;
    }
    memset(c->h_st, 0, sizeof(DevState));
    hipMemcpy(c->st_gen, c->h_st, sizeof(DevState), hipMemcpyHostToDevice);
    hipMemcpy(c->st_api, c->h_st, sizeof(DevState), hipMemcpyHostToDevice);
    *out = c;
    return QTTS_OK;
}

static void free_model(qtts_ctx *c)
{
    drop_graph(c);
    free_list(c->model_allocs);
    c->lkv = c->leg_buf = nullptr;                   // were model allocations
    c->lkv_ptab = nullptr;
    c->lkv_len = 0;
    free_list(c->ws_allocs);
    if (c->pf_mem) hipFree(c->pf_mem);   // sized for the model's hidden / inter
    c->pf_mem = nullptr;
    c->pf = PrefillWs{};
    c->has_model = false;
    c->gen_started = false;
    c->text_cap = 0;
}

extern "C" void qtts_ctx_destroy(qtts_ctx *c)
{
    if (!c) return;
    hipSetDevice(c->device);
    if (c->stream) hipStreamSynchronize(c->stream);
    free_model(c);
    if (c->d_forced) hipFree(c->d_forced);
    if (c->d_io) hipFree(c->d_io);
    if (c->d_io2) hipFree(c->d_io2);
    if (c->d_rmax) hipFree(c->d_rmax);
    if (c->d_copy) hipFree(c->d_copy);
    if (c->d_read) hipFree(c->d_read);
    if (c->d_sink) hipFree(c->d_sink);
    free_list(c->dec_allocs);
    if (c->dws_mem) hipFree(c->dws_mem);
    if (c->st_gen) hipFree(c->st_gen);
    if (c->st_api) hipFree(c->st_api);
    if (c->h_st) hipHostFree(c->h_st);
    if (c->h_ring) hipHostFree(c->h_ring);
    if (c->d_codes_api) hipFree(c->d_codes_api);
    if (c->d_rng_api) hipFree(c->d_rng_api);
    if (c->d_status) hipFree(c->d_status);
    if (c->d_prev_api) hipFree(c->d_prev_api);
    if (c->stream) hipStreamDestroy(c->stream);
    delete c;
}

extern "C" const char *qtts_last_error(const qtts_ctx *c) { return c ? c->err.c_str() : "null context"; }

extern "C" int qtts_sync(qtts_ctx *c)
{
    if (!c) return QTTS_ERR_INVALID;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return QTTS_OK;
}

extern "C" void *qtts_stream(qtts_ctx *c) { return c ? (void *)c->stream : nullptr; }

static int ensure_io(qtts_ctx *c, int64_t floats)
{
    if (floats <= c->io_floats) return QTTS_OK;
    if (c->d_io) hipFree(c->d_io);
    if (c->d_io2) hipFree(c->d_io2);
    c->d_io = c->d_io2 = nullptr;
    HIPCHK(c, hipMalloc(&c->d_io, floats * sizeof(float)));
    HIPCHK(c, hipMalloc(&c->d_io2, floats * sizeof(float)));
    c->io_floats = floats;
    return QTTS_OK;
}

// One float per GEMM row for the rows' largest |x| (grown on demand).
static int ensure_rmax(qtts_ctx *c, int64_t rows)
{
    if (rows <= c->rmax_rows) return QTTS_OK;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    if (c->d_rmax) hipFree(c->d_rmax);
    c->d_rmax = nullptr;
    c->rmax_rows = 0;
    HIPCHK(c, hipMalloc(&c->d_rmax, (size_t)rows * sizeof(float)));
    c->rmax_rows = rows;
    return QTTS_OK;
}

// Row buffers of the batched prefill for `rows` rows (grown on demand).
static int ensure_prefill(qtts_ctx *c, int rows)
{
    if (rows <= c->pf.cap_rows) return QTTS_OK;
    if (c->pf_mem) hipFree(c->pf_mem);
    c->pf_mem = nullptr;
    c->pf = PrefillWs{};
    const int64_t H = c->tm.hidden, A = 16 * HEAD_DIM, I = c->tm.inter, P = prefill_part_floats(c->tm);
    const int64_t RS = prefill_rmax_slots(c->tm);
    const int64_t per_row = H + A + A + I + P + 1 + RS;
    float *base = nullptr;
    HIPCHK(c, hipMalloc(&base, (size_t)rows * per_row * sizeof(float)));
    c->pf_mem = base;
    c->pf.x = base;
    c->pf.q = c->pf.x + rows * H;
    c->pf.attn = c->pf.q + rows * A;
    c->pf.h = c->pf.attn + rows * A;
    c->pf.part = c->pf.h + rows * I;
    c->pf.rmax = c->pf.part + rows * P;   // 16-byte aligned: every width before it is a multiple of 4
    c->pf.inv = c->pf.rmax + rows * RS;
    c->pf.cap_rows = rows;
    return QTTS_OK;
}

static bool use_mfma(int flags, int64_t rows)
{
    if (flags & QTTS_PATH_ROWWISE) return false;
    return (flags & QTTS_PATH_MFMA) || rows >= MFMA_MIN_ROWS;
}

// Copy n floats in (host or device source) to a device buffer.
static int stage_in(qtts_ctx *c, const float *src, int64_t n, float *dst, int flags)
{
    HIPCHK(c, hipMemcpyAsync(dst, src, n * sizeof(float),
                             (flags & QTTS_DEVICE_PTRS) ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                             c->stream));
    return QTTS_OK;
}

static int stage_out(qtts_ctx *c, const float *src, int64_t n, float *dst, int flags)
{
    if (!dst) return QTTS_OK;
    HIPCHK(c, hipMemcpyAsync(dst, src, n * sizeof(float),
                             (flags & QTTS_DEVICE_PTRS) ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost,
                             c->stream));
    return QTTS_OK;
}

// ---------------------------------------------------------------------------
// operator level
// ---------------------------------------------------------------------------

extern "C" int qtts_q4_upload(qtts_ctx *c, const qtts_q4_host *w, qtts_w **out)
{
    if (!c || !w || !out) return QTTS_ERR_INVALID;
    *out = nullptr;
    hipSetDevice(c->device);
    qtts_w *h = new qtts_w();
    const int64_t G = w->n / 32;
    (void)G;
    int r = build_tiled(c, h->allocs, {src_of(*w)}, role_cfg("GEMV", w->k), &h->t, nullptr);
    if (r == QTTS_OK) r = upload_rows(c, h->allocs, {*w}, &h->rows);
    if (r == QTTS_OK) r = dev_alloc(c, h->allocs, &h->x, (size_t)w->k * 2);
    if (r == QTTS_OK) r = dev_alloc(c, h->allocs, &h->y, (size_t)std::max<int64_t>(w->n, h->t.npad) * 2);
    if (r == QTTS_OK) r = dev_alloc(c, h->allocs, &h->part, (size_t)h->t.S * 2 * h->t.npad);
    if (r != QTTS_OK) {
        free_list(h->allocs);
        delete h;
        return r;
    }
    *out = h;
    return QTTS_OK;
}

extern "C" int qtts_q4_free(qtts_ctx *c, qtts_w *w)
{
    if (!c || !w) return QTTS_ERR_INVALID;
    hipStreamSynchronize(c->stream);
    free_list(w->allocs);
    delete w;
    return QTTS_OK;
}

extern "C" int qtts_gemv_q4(qtts_ctx *c, const qtts_w *w, const float *x, float *y, int flags)
{
    if (!c || !w || !x || !y) return QTTS_ERR_INVALID;
    RCHK(stage_in(c, x, w->t.k, w->x, flags));
    HIPCHK(c, enqueue_gemv_store(w->t, w->x, w->y, nullptr, w->part, c->stream));
    // columns past the last full group stay zero (gemv.rs:255 starts from
    // vec![0.0; n] and only full groups are accumulated)
    const int64_t full = (int64_t)(w->t.n / 32) * 32;
    if (full < w->t.n) HIPCHK(c, hipMemsetAsync(w->y + full, 0, (w->t.n - full) * sizeof(float), c->stream));
    RCHK(stage_out(c, w->y, w->t.n, y, flags));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return QTTS_OK;
}

extern "C" int qtts_gemm_q4(qtts_ctx *c, const qtts_w *w, const float *X, int64_t rows, float *Y, int flags)
{
    if (!c || !w || !X || !Y || rows < 0) return QTTS_ERR_INVALID;
    if (rows == 0) return QTTS_OK;
    RCHK(ensure_io(c, std::max<int64_t>(rows * w->t.k, rows * w->t.npad)));
    RCHK(stage_in(c, X, rows * w->t.k, c->d_io, flags));
    HIPCHK(c, hipMemsetAsync(c->d_io2, 0, rows * w->t.n * sizeof(float), c->stream));
    if (use_mfma(flags, rows) && gemm_supported(w->t)) {
        RCHK(ensure_rmax(c, rows));
        HIPCHK(c, enqueue_gemm_rows(w->t, c->d_io, (int)rows, c->d_io2, w->t.n, c->d_rmax, c->stream));
    }
    else
        HIPCHK(c, enqueue_gemv_rows(w->t, c->d_io, (int)rows, c->d_io2, w->part, c->stream));
    RCHK(stage_out(c, c->d_io2, rows * w->t.n, Y, flags));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return QTTS_OK;
}

// qtts_gemm_q4 on device rows, allocating nothing: the GEMV passes' partial
// sums go to this device's `scratch` (its address looked up when the
// context was created), the ragged columns are cleared by a fill kernel,
// and nothing is staged, so the call only enqueues kernels on the context
// stream and returns.  Calls that overlap on one GPU (other contexts,
// other host threads) share the array and race.
extern "C" int qtts_gemm_q4_noalloc(qtts_ctx *c, const qtts_w *w, const float *X, int64_t rows, float *Y,
                                    int flags)
{
    if (!c || !w || !X || !Y || rows < 0) return QTTS_ERR_INVALID;
    if (rows == 0) return QTTS_OK;
    // 2^20 rows keep every launch's grid within the device's limits (the
    // matrix-core GEMM's row tiles x column tiles x 256 threads below 2^32)
    static_assert((size_t)1 << 20 <= SCRATCH_FLOATS, "one float of scratch per row for the rows' ranges");
    if (rows > (1 << 20)) return fail(c, QTTS_ERR_CAPACITY, "at most %d rows", 1 << 20);
    if (!c->scratch) return fail(c, QTTS_ERR_STATE, "no scratch address for device %d", c->device);
    hipSetDevice(c->device);
    const Q4Tiled &t = w->t;
    if (use_mfma(flags, rows) && gemm_supported(t)) {
        // the rows' largest |x| (the staging range) in the scratch array:
        // rows <= 2^20 = its size
        HIPCHK(c, enqueue_gemm_rows(t, X, (int)rows, Y, t.n, c->scratch, c->stream));
    } else {
        const size_t need = (size_t)t.S * 2 * t.npad;
        if (need > SCRATCH_FLOATS)
            return fail(c, QTTS_ERR_CAPACITY, "this weight's GEMV passes need %zu floats of scratch; the maximum is %zu",
                        need, SCRATCH_FLOATS);
        HIPCHK(c, enqueue_gemv_rows(t, X, (int)rows, Y, c->scratch, c->stream));
    }
    // columns past the last full group are zero (gemv.rs:255)
    const int full = (t.n / 32) * 32;
    HIPCHK(c, enqueue_zero_cols(Y, (int)rows, t.n, full, t.n, c->stream));
    return QTTS_OK;
}

extern "C" int qtts_embed_lookup_q4(qtts_ctx *c, const qtts_w *w, int64_t row, float *out, int flags)
{
    if (!c || !w || !out) return QTTS_ERR_INVALID;
    if (row < 0 || row >= w->rows.rows) return fail(c, QTTS_ERR_INVALID, "row %lld out of range", (long long)row);
    HIPCHK(c, hipMemsetAsync(w->y, 0, w->rows.n * sizeof(float), c->stream));
    Q4Rows e = w->rows;
    e.n = e.G * 32;
    HIPCHK(c, enqueue_embed_row(e, nullptr, (uint32_t)row, w->y, c->stream));
    RCHK(stage_out(c, w->y, w->rows.n, out, flags));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return QTTS_OK;
}

// ---------------------------------------------------------------------------
// model upload
// ---------------------------------------------------------------------------

static int alloc_workspace(qtts_ctx *c)
{
    auto &A = c->ws_allocs;
    Workspace &w = c->ws;
    const TalkerDev &m = c->tm;
    const PredictorDev &p = c->pm;
    const int H = m.hidden, h = p.hidden;
    // split-K partial buffers: S * NB * npad per producer role
    size_t pq = 0, po = 0, pg = 0, pd = 0, ph = 0, pp = 0;
    auto upd = [](size_t &v, const Q4Tiled &t, int nb) { v = std::max(v, (size_t)t.S * nb * t.npad); };
    for (const LayerDev &L : c->tlayers) { upd(pq, L.qkv, 1); upd(po, L.o, 1); upd(pg, L.gate_up, 1); upd(pd, L.down, 1); }
    for (const LayerDev &L : c->players) { upd(pq, L.qkv, 2); upd(po, L.o, 2); upd(pg, L.gate_up, 2); upd(pd, L.down, 2); }
    upd(ph, m.codec_head, 1);
    for (const Q4Tiled &t : c->pheads) upd(ph, t, 1);
    upd(pp, p.proj, 2);
    upd(pp, m.text_fc1, 1);
    upd(pp, m.text_fc2, 1);
    RCHK(dev_alloc(c, A, &w.x, 2 * (size_t)std::max(H, m.text_hidden)));
    RCHK(dev_alloc(c, A, &w.xa, H));
    RCHK(dev_alloc(c, A, &w.xb, H));
    RCHK(dev_alloc(c, A, &w.pxa, 2 * (size_t)h));
    RCHK(dev_alloc(c, A, &w.pxb, 2 * (size_t)h));
    RCHK(dev_alloc(c, A, &w.pin, 2 * (size_t)H));
    RCHK(dev_alloc(c, A, &w.am, MAX_CHUNKS * 16));
    RCHK(dev_alloc(c, A, &w.al, MAX_CHUNKS * 16));
    RCHK(dev_alloc(c, A, &w.aacc, (size_t)MAX_CHUNKS * 16 * HEAD_DIM));
    RCHK(dev_alloc(c, A, &w.attn, 16 * HEAD_DIM));
    RCHK(dev_alloc(c, A, &w.pattn, 2 * 16 * HEAD_DIM));
    RCHK(dev_alloc(c, A, &w.pk, (size_t)p.n_layers * PRED_KV_CAP * 8 * HEAD_DIM));
    RCHK(dev_alloc(c, A, &w.pv, (size_t)p.n_layers * PRED_KV_CAP * 8 * HEAD_DIM));
    RCHK(dev_alloc(c, A, &w.h, 2 * (size_t)std::max(m.inter, p.inter)));
    RCHK(dev_alloc(c, A, &w.part_qkv, pq));
    size_t lq = 0, lpq = 0;
    for (const LayerDev &L : c->tlayers) upd(lq, L.qkv, 1);
    for (const LayerDev &L : c->players) upd(lpq, L.qkv, 2);
    // silu(gate) * up words, or the raw gate|up column sums (twice as many)
    // when a one-group gate|up tile feeds the down tiles (the predictor's
    // default, any role's tile override); the predictor's for up to 2 rows
    const size_t lth = 2 * (size_t)m.inter, lph = 2 * 2 * (size_t)p.inter;
    RCHK(dev_alloc(c, A, &w.ll_qkv, lq));
    RCHK(dev_alloc(c, A, &w.ll_pqkv, lpq));
    RCHK(dev_alloc(c, A, &w.ll_th, lth));
    RCHK(dev_alloc(c, A, &w.ll_ph, lph));
    RCHK(dev_alloc(c, A, &w.ll_seq, LL_KINDS));
    HIPCHK(c, hipMemset(w.ll_qkv, 0, sizeof(uint64_t) * std::max<size_t>(lq, 32)));
    HIPCHK(c, hipMemset(w.ll_pqkv, 0, sizeof(uint64_t) * std::max<size_t>(lpq, 32)));
    HIPCHK(c, hipMemset(w.ll_th, 0, sizeof(uint64_t) * std::max<size_t>(lth, 32)));
    HIPCHK(c, hipMemset(w.ll_ph, 0, sizeof(uint64_t) * std::max<size_t>(lph, 32)));
    HIPCHK(c, hipMemset(w.ll_seq, 0, sizeof(uint32_t) * LL_KINDS));
    RCHK(dev_alloc(c, A, &w.part_o, po));
    RCHK(dev_alloc(c, A, &w.part_gu, pg));
    RCHK(dev_alloc(c, A, &w.part_down, pd));
    RCHK(dev_alloc(c, A, &w.part_head, ph));
    RCHK(dev_alloc(c, A, &w.part_proj, pp));
    RCHK(dev_alloc(c, A, &w.hid_work, H));
    RCHK(dev_alloc(c, A, &w.hidden, H));
    RCHK(dev_alloc(c, A, &w.logits, std::max(m.vocab, 4096)));
    RCHK(dev_alloc(c, A, &w.pad, H));
    RCHK(dev_alloc(c, A, &w.ring_pred, RING_FRAMES * 16));
    RCHK(dev_alloc(c, A, &w.ring_used, RING_FRAMES * 16));
    RCHK(dev_alloc(c, A, &w.cand, 16 * MAX_CAND));
    c->text_cap = 256;
    RCHK(dev_alloc(c, A, &w.text, (size_t)c->text_cap * H));
    HIPCHK(c, hipMemset(w.pad, 0, sizeof(float) * H));
    w.attn_grid = 8 * (int)(c->kv_cap / KV_PAGE);
    RCHK(ensure_io(c, std::max<int64_t>(8192, 4 * (int64_t)std::max(H, m.vocab))));
    return QTTS_OK;
}

static int build_pred_rows(qtts_ctx *c);

static int upload_model(qtts_ctx *c, const qtts_talker_host *t, const qtts_predictor_host *p)
{
    auto &A = c->model_allocs;
    if (t->n_layers <= 0 || !t->layers || t->head_dim != HEAD_DIM || t->n_heads != 16 || t->n_kv_heads != 8)
        return fail(c, QTTS_ERR_UNSUPPORTED, "talker shape not supported (heads %d/%d, head_dim %d)",
                    t->n_heads, t->n_kv_heads, t->head_dim);
    if (p->n_layers <= 0 || !p->layers || p->head_dim != HEAD_DIM || p->n_heads != 16 || p->n_kv_heads != 8)
        return fail(c, QTTS_ERR_UNSUPPORTED, "predictor shape not supported");
    if (!p->has_input_proj)
        return fail(c, QTTS_ERR_UNSUPPORTED, "predictor without input projection not supported");
    if (p->n_groups < 1 || p->n_groups > 15 || !p->lm_heads || !p->codec_embeddings)
        return fail(c, QTTS_ERR_INVALID, "predictor needs 1..15 heads and embeddings");
    if (t->vocab > 4096 || t->vocab <= 0) return fail(c, QTTS_ERR_UNSUPPORTED, "talker vocab must be <= 4096");
    // the step end, the sampler and the predictor's argmax read whole 32-column
    // groups of the heads' partial sums (the 12 Hz model's 3072 and 2048 are)
    if (t->vocab % 32 || p->vocab <= 0 || p->vocab % 32)
        return fail(c, QTTS_ERR_UNSUPPORTED, "codec vocab sizes must be multiples of 32 (talker %d, predictor %d)",
                    t->vocab, p->vocab);
    if (t->hidden > 2048 || p->hidden > 2048 || t->hidden % 32 || p->hidden % 32)
        return fail(c, QTTS_ERR_UNSUPPORTED, "hidden sizes must be multiples of 32 and <= 2048");
    if (t->rope_max_pos < 1 || !t->rope_cos || !t->rope_sin || p->rope_max_pos < PRED_KV_CAP)
        return fail(c, QTTS_ERR_INVALID, "rope tables missing");

    TalkerDev &m = c->tm;
    m.n_layers = t->n_layers; m.hidden = t->hidden; m.text_hidden = t->text_hidden;
    m.n_heads = t->n_heads; m.n_kv_heads = t->n_kv_heads; m.inter = t->inter; m.vocab = t->vocab;
    c->tlayers.assign(t->n_layers, LayerDev{});
    for (int l = 0; l < t->n_layers; l++) RCHK(upload_layer(c, t->layers[l], t->hidden, t->head_dim, &c->tlayers[l], false));
    m.layers = c->tlayers.data();
    RCHK(build_tiled(c, A, {src_of(t->codec_head)}, role_cfg("HEAD", t->hidden), &m.codec_head, nullptr));
    RCHK(build_tiled(c, A, {src_of(t->text_fc1)}, role_cfg("TEXT", t->text_fc1.k), &m.text_fc1, nullptr));
    RCHK(build_tiled(c, A, {src_of(t->text_fc2)}, role_cfg("TEXT", t->text_fc2.k), &m.text_fc2, nullptr));
    RCHK(upload_vec(c, A, t->text_fc1_bias, t->text_fc1.n, &m.text_fc1_bias));
    RCHK(upload_vec(c, A, t->text_fc2_bias, t->text_fc2.n, &m.text_fc2_bias));
    RCHK(upload_rows(c, A, {t->codec_embedding}, &m.codec_rows));
    RCHK(upload_rows(c, A, {t->text_embedding}, &m.text_rows));
    RCHK(upload_vec(c, A, t->final_norm, t->hidden, &m.final_norm));
    RCHK(upload_vec(c, A, t->rope_cos, (size_t)t->rope_max_pos * 64, &m.rope_cos));
    RCHK(upload_vec(c, A, t->rope_sin, (size_t)t->rope_max_pos * 64, &m.rope_sin));
    m.rope_rows = t->rope_max_pos;
    if (m.codec_rows.n != m.hidden) return fail(c, QTTS_ERR_INVALID, "codec embedding width != hidden");

    // paged KV pool: the sequence starts on pages 0..kv_cap/64-1, the other
    // half of the pool is free for prefixes and copy-on-write
    const int n_seq = (int)(c->kv_cap / KV_PAGE), n_pool = 2 * n_seq;
    float *kvb = nullptr;
    RCHK(dev_alloc(c, A, &kvb, (size_t)t->n_layers * n_pool * 2 * 8 * KV_PAGE * HEAD_DIM));
    c->seq_ptab.assign(MAX_CHUNKS, 0);
    c->page_ref.assign(n_pool, 0);
    c->free_pages.clear();
    for (int i = 0; i < n_seq; i++) {
        c->seq_ptab[i] = i;
        c->page_ref[i] = 1;
    }
    for (int i = n_pool - 1; i >= n_seq; i--) c->free_pages.push_back(i);
    const int32_t *dptab = nullptr;
    RCHK(upload_vec(c, A, c->seq_ptab.data(), c->seq_ptab.size(), &dptab));
    c->d_ptab = const_cast<int32_t *>(dptab);
    m.kv = KvPaged{kvb, dptab, n_pool};
    c->model_gen++;

    PredictorDev &q = c->pm;
    q.n_layers = p->n_layers; q.hidden = p->hidden; q.n_heads = p->n_heads; q.n_kv_heads = p->n_kv_heads;
    q.inter = p->inter; q.vocab = p->vocab; q.n_groups = p->n_groups;
    c->players.assign(p->n_layers, LayerDev{});
    for (int l = 0; l < p->n_layers; l++) RCHK(upload_layer(c, p->layers[l], p->hidden, p->head_dim, &c->players[l], true));
    q.layers = c->players.data();
    RCHK(build_tiled(c, A, {src_of(p->input_proj)}, role_cfg("PPROJ", p->input_proj.k), &q.proj, nullptr));
    if (q.proj.n != q.hidden || p->input_proj.k != t->hidden)
        return fail(c, QTTS_ERR_INVALID, "predictor input projection shape");
    RCHK(upload_vec(c, A, p->input_proj_bias, p->input_proj.n, &q.proj_bias));
    c->pheads.assign(p->n_groups, Q4Tiled{});
    for (int g = 0; g < p->n_groups; g++) {
        RCHK(build_tiled(c, A, {src_of(p->lm_heads[g])}, role_cfg("PHEAD", p->lm_heads[g].k), &c->pheads[g], nullptr));
        if (c->pheads[g].n != p->vocab) return fail(c, QTTS_ERR_INVALID, "lm_head %d width != vocab", g);
    }
    q.heads = c->pheads.data();
    std::vector<qtts_q4_host> embs(p->codec_embeddings, p->codec_embeddings + p->n_groups);
    RCHK(upload_rows(c, A, embs, &q.emb_rows));
    if (q.emb_rows.n != t->hidden) return fail(c, QTTS_ERR_INVALID, "predictor embedding width != talker hidden");
    RCHK(upload_vec(c, A, p->final_norm, p->hidden, &q.final_norm));
    RCHK(upload_vec(c, A, p->rope_cos, (size_t)p->rope_max_pos * 64, &q.rope_cos));
    RCHK(upload_vec(c, A, p->rope_sin, (size_t)p->rope_max_pos * 64, &q.rope_sin));
    q.rope_rows = p->rope_max_pos;
    RCHK(alloc_workspace(c));
    RCHK(build_pred_rows(c));
    return QTTS_OK;
}

// Projected embedding rows of the predictor's steps 1..n_groups-1 (layer 0's
// input is a function of the step's code alone): 2048 x 1024 floats per
// codebook, 117 MB for the 1.7B predictor.  QTTS_PRED_ROWS=0 keeps the
// per-step projection GEMV instead.
static int build_pred_rows(qtts_ctx *c)
{
    PredictorDev &q = c->pm;
    q.proj_rows = nullptr;
    q.qkv_rows = nullptr;
    const char *env = getenv("QTTS_PRED_ROWS");
    if (q.n_groups < 2 || q.hidden > 1024 || q.emb_rows.n != q.proj.k || (env && env[0] == '0')) return QTTS_OK;
    const int ntab = q.n_groups - 1, rows = q.emb_rows.rows;
    float *tab = nullptr;
    RCHK(dev_alloc(c, c->model_allocs, &tab, (size_t)ntab * rows * q.hidden));
    float *X = nullptr, *part = nullptr;
    HIPCHK(c, hipMalloc(&X, (size_t)rows * q.proj.k * sizeof(float)));
    if (hipMalloc(&part, (size_t)rows * q.proj.S * q.proj.npad * sizeof(float)) != hipSuccess) {
        hipFree(X);
        return fail(c, QTTS_ERR_OOM, "predictor row tables: scratch allocation failed");
    }
    hipError_t e = enqueue_pred_row_tables(q, ntab, X, part, tab, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    hipFree(X);
    hipFree(part);
    if (e != hipSuccess) return fail(c, QTTS_ERR_HIP, "predictor row tables: %s", hipGetErrorString(e));
    q.proj_rows = tab;
    // layer 0's q|k|v of every table row (14 x 2048 x 4096 floats, 470 MB for
    // the 1.7B predictor); QTTS_PRED_QKV_ROWS=0 keeps the per-step GEMV
    q.qkv_rows = nullptr;
    const char *qenv = getenv("QTTS_PRED_QKV_ROWS");
    if ((qenv && qenv[0] == '0') || !pred_qkv_tables_supported(q)) return QTTS_OK;
    const LayerDev &L0 = q.layers[0];
    float *qtab = nullptr;
    RCHK(dev_alloc(c, c->model_allocs, &qtab, (size_t)ntab * rows * L0.qkv.npad));
    HIPCHK(c, hipMalloc(&part, (size_t)rows * L0.qkv.S * L0.qkv.npad * sizeof(float)));
    e = enqueue_pred_qkv_tables(q, ntab, part, qtab, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    hipFree(part);
    if (e != hipSuccess) return fail(c, QTTS_ERR_HIP, "predictor q|k|v tables: %s", hipGetErrorString(e));
    q.qkv_rows = qtab;
    return QTTS_OK;
}

static int write_state(qtts_ctx *c)
{
    HIPCHK(c, hipMemcpyAsync(c->st_gen, c->h_st, sizeof(DevState), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return QTTS_OK;
}

// ---------------------------------------------------------------------------
// KV page pool
// ---------------------------------------------------------------------------

static int push_ptab(qtts_ctx *c)
{
    HIPCHK(c, hipMemcpyAsync(c->d_ptab, c->seq_ptab.data(), c->seq_ptab.size() * sizeof(int32_t),
                             hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return QTTS_OK;
}

static int page_take(qtts_ctx *c, int32_t *page)
{
    if (c->free_pages.empty())
        return fail(c, QTTS_ERR_CAPACITY, "KV page pool exhausted (free unused prefixes)");
    *page = c->free_pages.back();
    c->free_pages.pop_back();
    c->page_ref[*page] = 1;
    return QTTS_OK;
}

static void page_drop(qtts_ctx *c, int32_t page)
{
    if (--c->page_ref[page] == 0) c->free_pages.push_back(page);
}

// Copy one physical page (all layers, K and V) to another.
static int page_copy(qtts_ctx *c, int32_t src, int32_t dst)
{
    const size_t blk = (size_t)2 * 8 * KV_PAGE * HEAD_DIM;
    for (int l = 0; l < c->tm.n_layers; l++) {
        float *b = c->tm.kv.base + (size_t)l * c->tm.kv.n_phys * blk;
        HIPCHK(c, hipMemcpyAsync(b + (size_t)dst * blk, b + (size_t)src * blk, blk * sizeof(float),
                                 hipMemcpyDeviceToDevice, c->stream));
    }
    return QTTS_OK;
}

// Before the sequence writes positions from `pos` on: every logical page from
// the one holding `pos` that is shared with a prefix gets a private page
// (copy-on-write, keeping the positions below `pos`).
static int seq_unshare_from(qtts_ctx *c, int64_t pos)
{
    const int n_seq = (int)(c->kv_cap / KV_PAGE);
    bool changed = false;
    for (int i = (int)(pos / KV_PAGE); i < n_seq; i++) {
        const int32_t old = c->seq_ptab[i];
        if (c->page_ref[old] <= 1) continue;
        int32_t p;
        RCHK(page_take(c, &p));
        if ((int64_t)i * KV_PAGE < pos) {
            const int r = page_copy(c, old, p);
            if (r != QTTS_OK) {
                page_drop(c, p);
                return r;
            }
        }
        page_drop(c, old);
        c->seq_ptab[i] = p;
        changed = true;
    }
    return changed ? push_ptab(c) : QTTS_OK;
}

static int read_state(qtts_ctx *c)
{
    HIPCHK(c, hipMemcpyAsync(c->h_st, c->st_gen, sizeof(DevState), hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return QTTS_OK;
}

extern "C" int qtts_model_upload(qtts_ctx *c, const qtts_talker_host *t, const qtts_predictor_host *p)
{
    if (!c || !t || !p) return QTTS_ERR_INVALID;
    hipSetDevice(c->device);
    HIPCHK(c, hipStreamSynchronize(c->stream));
    free_model(c);
    const int r = upload_model(c, t, p);
    if (r != QTTS_OK) {
        free_model(c);
        return r;
    }
    memset(c->h_st, 0, sizeof(DevState));
    RCHK(write_state(c));
    c->has_model = true;
    return QTTS_OK;
}

extern "C" int qtts_model_dims(qtts_ctx *c, int32_t *th, int32_t *tv, int32_t *tl, int32_t *ph, int32_t *pv,
                               int32_t *pg)
{
    if (!c) return QTTS_ERR_INVALID;
    if (!c->has_model) return fail(c, QTTS_ERR_STATE, "no model uploaded");
    if (th) *th = c->tm.hidden;
    if (tv) *tv = c->tm.vocab;
    if (tl) *tl = c->tm.n_layers;
    if (ph) *ph = c->pm.hidden;
    if (pv) *pv = c->pm.vocab;
    if (pg) *pg = c->pm.n_groups;
    return QTTS_OK;
}

#define NEED_MODEL(c)                                                                \
    do {                                                                             \
        if (!(c)) return QTTS_ERR_INVALID;                                           \
        if (!(c)->has_model) return fail((c), QTTS_ERR_STATE, "no model uploaded");  \
        hipSetDevice((c)->device);                                                   \
    } while (0)

// ---------------------------------------------------------------------------
// talker
// ---------------------------------------------------------------------------

// A bounded cross-workgroup wait that ran out (a fused launch: q|k|v +
// attention, gate|up + down) leaves sync_err set in the device state:
// reported once, then cleared.  The launches after it skipped their waits,
// so the outputs of the call are invalid.
static int check_sync(qtts_ctx *c)
{
    int32_t e = 0;
    HIPCHK(c, hipMemcpyAsync(&e, &c->st_gen->sync_err, sizeof e, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    if (!e) return QTTS_OK;
    const int32_t z = 0;
    HIPCHK(c, hipMemcpy(&c->st_gen->sync_err, &z, sizeof z, hipMemcpyHostToDevice));
    c->h_st->sync_err = 0;
    return fail(c, QTTS_ERR_HIP, "a cross-workgroup wait timed out (fused launch): outputs of this call are invalid");
}

// qtts_debug_force_sync_err armed: the state `st` of the call about to
// launch gets the flag a wait that ran out leaves (the call's fused
// launches then skip their waits).
static int arm_sync_err(qtts_ctx *c, DevState *st)
{
    if (!c->force_sync_err) return QTTS_OK;
    c->force_sync_err = false;
    if (st == c->st_gen) c->h_st->sync_err = 1;
    const int32_t one = 1;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    HIPCHK(c, hipMemcpy(&st->sync_err, &one, sizeof one, hipMemcpyHostToDevice));
    return QTTS_OK;
}

// Pages per attention work item for a talker step at cached length kv.
static int step_pages(const qtts_ctx *c, int64_t kv) { return talker_fused_attn(c->tm) ? 2 : attn_pages(kv); }

// One talker step on the input already in ws.x.  A step whose waits ran
// out reports QTTS_ERR_HIP and leaves the cache length and position where
// they were (the device's counters are rolled back; the row it appended
// lies past the length and is overwritten by the next step).
static int talker_step_staged(qtts_ctx *c, int64_t position, float *hidden_out, float *logits_out, int flags)
{
    c->h_st->position = position;
    HIPCHK(c, hipMemcpyAsync(&c->st_gen->position, &c->h_st->position, sizeof(int64_t), hipMemcpyHostToDevice, c->stream));
    RCHK(arm_sync_err(c, c->st_gen));
    HIPCHK(c, enqueue_talker_step(c->tm, c->ws, c->st_gen, 0, step_pages(c, c->h_st->kv_len), c->stream));
    RCHK(stage_out(c, c->ws.hidden, c->tm.hidden, hidden_out, flags));
    RCHK(stage_out(c, c->ws.logits, c->tm.vocab, logits_out, flags));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    const int rs = check_sync(c);
    if (rs != QTTS_OK) {
        const std::string msg = c->err;
        RCHK(write_state(c));
        c->err = msg;
        return rs;
    }
    c->h_st->kv_len += 1;
    c->h_st->position = position + 1;
    return QTTS_OK;
}

static int step_checks(qtts_ctx *c, int64_t position)
{
    if (position < 0) return QTTS_ERR_INVALID;
    if (position >= c->tm.rope_rows) return fail(c, QTTS_ERR_CAPACITY, "position beyond the RoPE table");
    if (c->h_st->kv_len + 1 > c->kv_cap) return fail(c, QTTS_ERR_CAPACITY, "talker KV cache full");
    c->gen_started = false;
    return QTTS_OK;
}

extern "C" int qtts_talker_step(qtts_ctx *c, const float *emb, int64_t position, float *hidden_out,
                                float *logits_out, int flags)
{
    NEED_MODEL(c);
    if (!emb) return QTTS_ERR_INVALID;
    RCHK(step_checks(c, position));
    RCHK(stage_in(c, emb, c->tm.hidden, c->ws.x, flags));
    return talker_step_staged(c, position, hidden_out, logits_out, flags);
}

// embed_text_token (talker.rs:105-116) of one id into a device row, one
// GEMV pass per projection.
static int text_token_row(qtts_ctx *c, uint32_t token, float *out_dev)
{
    const TalkerDev &m = c->tm;
    if ((int64_t)token >= m.text_rows.rows) return fail(c, QTTS_ERR_INVALID, "text token %u out of range", token);
    float *raw = c->d_io, *h1 = c->d_io + 2 * std::max(m.text_hidden, m.hidden);
    Q4Rows e = m.text_rows;
    e.n = m.text_hidden;
    HIPCHK(c, enqueue_embed_row(e, nullptr, token, raw, c->stream));
    HIPCHK(c, enqueue_gemv_store(m.text_fc1, raw, h1, m.text_fc1_bias, c->ws.part_proj, c->stream));
    HIPCHK(c, enqueue_silu(h1, m.text_fc1.n, c->stream));
    HIPCHK(c, enqueue_gemv_store(m.text_fc2, h1, out_dev, m.text_fc2_bias, c->ws.part_proj, c->stream));
    return QTTS_OK;
}

extern "C" int qtts_talker_decode_token(qtts_ctx *c, uint32_t token, int is_text, int64_t position,
                                        float *hidden_out, int flags)
{
    NEED_MODEL(c);
    RCHK(step_checks(c, position));
    if (is_text) {
        RCHK(text_token_row(c, token, c->ws.x));
    } else {
        if ((int64_t)token >= c->tm.codec_rows.rows) return fail(c, QTTS_ERR_INVALID, "codec token %u out of range", token);
        HIPCHK(c, enqueue_embed_row(c->tm.codec_rows, nullptr, token, c->ws.x, c->stream));
    }
    return talker_step_staged(c, position, hidden_out, nullptr, flags);
}

extern "C" int qtts_talker_prefill(qtts_ctx *c, const float *X, int64_t seq, int64_t start_pos, float *hidden_out,
                                   int flags)
{
    NEED_MODEL(c);
    if (!X || seq < 1 || start_pos < 0) return QTTS_ERR_INVALID;
    if (c->h_st->kv_len != start_pos)
        return fail(c, QTTS_ERR_STATE, "prefill at %lld but %d positions cached", (long long)start_pos, c->h_st->kv_len);
    if (start_pos + seq > c->kv_cap) return fail(c, QTTS_ERR_CAPACITY, "talker KV cache full");
    if (start_pos + seq > c->tm.rope_rows) return fail(c, QTTS_ERR_CAPACITY, "position beyond the RoPE table");
    RCHK(seq_unshare_from(c, start_pos));
    c->gen_started = false;
    const int H = c->tm.hidden;
    if (use_mfma(flags, seq) && prefill_supported(c->tm)) {
        RCHK(ensure_prefill(c, (int)std::min<int64_t>(seq, PREFILL_MAX_ROWS)));
        for (int64_t r0 = 0; r0 < seq; r0 += c->pf.cap_rows) {
            const int rows = (int)std::min<int64_t>(c->pf.cap_rows, seq - r0);
            RCHK(stage_in(c, X + r0 * H, (int64_t)rows * H, c->pf.x, flags));
            HIPCHK(c, enqueue_talker_prefill(c->tm, c->pf, rows, start_pos + r0, c->ws.hid_work, c->stream));
        }
    } else {
        RCHK(arm_sync_err(c, c->st_gen));
        for (int64_t t = 0; t < seq; t++) {
            RCHK(stage_in(c, X + t * H, H, c->ws.x, flags));
            HIPCHK(c, enqueue_talker_row(c->tm, c->ws, c->st_gen, start_pos + t, (int)(start_pos + t),
                                         step_pages(c, start_pos + t), c->stream));
        }
        HIPCHK(c, enqueue_final_norm(c->tm, c->ws, c->ws.hid_work, c->stream));
        RCHK(check_sync(c));
    }
    RCHK(stage_out(c, c->ws.hid_work, H, hidden_out, flags));
    c->h_st->kv_len = (int32_t)(start_pos + seq);
    c->h_st->position = start_pos + seq;
    HIPCHK(c, hipMemcpyAsync(c->st_gen, c->h_st, sizeof(DevState), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return QTTS_OK;
}

extern "C" int qtts_codec_head(qtts_ctx *c, const float *hidden, float *logits, int flags)
{
    NEED_MODEL(c);
    if (!hidden || !logits) return QTTS_ERR_INVALID;
    RCHK(stage_in(c, hidden, c->tm.hidden, c->d_io, flags));
    HIPCHK(c, enqueue_codec_head(c->tm, c->ws, c->d_io, c->d_io2, c->stream));
    RCHK(stage_out(c, c->d_io2, c->tm.vocab, logits, flags));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return QTTS_OK;
}

extern "C" int qtts_embed_text_token(qtts_ctx *c, uint32_t token, float *out, int flags)
{
    NEED_MODEL(c);
    if (!out) return QTTS_ERR_INVALID;
    RCHK(text_token_row(c, token, c->d_io2));
    RCHK(stage_out(c, c->d_io2, c->tm.text_fc2.n, out, flags));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return QTTS_OK;
}

extern "C" int qtts_embed_codec_token(qtts_ctx *c, uint32_t token, float *out, int flags)
{
    NEED_MODEL(c);
    if (!out) return QTTS_ERR_INVALID;
    if ((int64_t)token >= c->tm.codec_rows.rows) return fail(c, QTTS_ERR_INVALID, "codec token %u out of range", token);
    HIPCHK(c, enqueue_embed_row(c->tm.codec_rows, nullptr, token, c->d_io, c->stream));
    RCHK(stage_out(c, c->d_io, c->tm.hidden, out, flags));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return QTTS_OK;
}

// ---------------------------------------------------------------------------
// KV cache
// ---------------------------------------------------------------------------

extern "C" int qtts_kv_reset(qtts_ctx *c)
{
    NEED_MODEL(c);
    RCHK(seq_unshare_from(c, 0));
    c->gen_started = false;
    c->h_st->kv_len = 0;
    c->h_st->position = 0;
    return write_state(c);
}

extern "C" int qtts_kv_len(qtts_ctx *c, int64_t *len)
{
    NEED_MODEL(c);
    if (!len) return QTTS_ERR_INVALID;
    *len = c->h_st->kv_len;
    return QTTS_OK;
}

extern "C" int qtts_kv_truncate(qtts_ctx *c, int64_t len)
{
    NEED_MODEL(c);
    if (len < 0 || len > c->h_st->kv_len) return QTTS_ERR_INVALID;
    RCHK(seq_unshare_from(c, len));
    c->gen_started = false;
    c->h_st->kv_len = (int32_t)len;
    return write_state(c);
}

extern "C" int qtts_kv_gather(qtts_ctx *c, int32_t layer, float *K, float *V)
{
    NEED_MODEL(c);
    if (layer < 0 || layer >= c->tm.n_layers || !K || !V) return QTTS_ERR_INVALID;
    const int len = c->h_st->kv_len;
    const size_t n = (size_t)len * 8 * HEAD_DIM;
    if (n == 0) return QTTS_OK;
    float *dk = nullptr, *dv = nullptr;
    HIPCHK(c, hipMalloc(&dk, n * sizeof(float)));
    HIPCHK(c, hipMalloc(&dv, n * sizeof(float)));
    int r = QTTS_OK;
    if (enqueue_kv_gather(c->tm.kv, layer, len, dk, dv, c->stream) != hipSuccess ||
        hipMemcpyAsync(K, dk, n * sizeof(float), hipMemcpyDeviceToHost, c->stream) != hipSuccess ||
        hipMemcpyAsync(V, dv, n * sizeof(float), hipMemcpyDeviceToHost, c->stream) != hipSuccess ||
        hipStreamSynchronize(c->stream) != hipSuccess)
        r = fail(c, QTTS_ERR_HIP, "kv gather failed");
    hipFree(dk);
    hipFree(dv);
    return r;
}

extern "C" int qtts_kv_load(qtts_ctx *c, const float *K, const float *V, int64_t len)
{
    NEED_MODEL(c);
    if (!K || !V || len < 0) return QTTS_ERR_INVALID;
    if (len > c->kv_cap) return fail(c, QTTS_ERR_CAPACITY, "kv_load of %lld > capacity", (long long)len);
    RCHK(seq_unshare_from(c, 0));
    c->gen_started = false;
    const size_t n = (size_t)len * 8 * HEAD_DIM;
    if (n) {
        float *dk = nullptr, *dv = nullptr;
        HIPCHK(c, hipMalloc(&dk, n * sizeof(float)));
        HIPCHK(c, hipMalloc(&dv, n * sizeof(float)));
        int r = QTTS_OK;
        for (int l = 0; l < c->tm.n_layers && r == QTTS_OK; l++) {
            if (hipMemcpyAsync(dk, K + (size_t)l * n, n * sizeof(float), hipMemcpyHostToDevice, c->stream) != hipSuccess ||
                hipMemcpyAsync(dv, V + (size_t)l * n, n * sizeof(float), hipMemcpyHostToDevice, c->stream) != hipSuccess ||
                enqueue_kv_scatter(c->tm.kv, l, (int)len, dk, dv, c->stream) != hipSuccess)
                r = fail(c, QTTS_ERR_HIP, "kv load failed");
        }
        hipStreamSynchronize(c->stream);
        hipFree(dk);
        hipFree(dv);
        if (r != QTTS_OK) return r;
    }
    c->h_st->kv_len = (int32_t)len;
    return write_state(c);
}

// ---------------------------------------------------------------------------
// talker prefix cache on the page pool
// ---------------------------------------------------------------------------

extern "C" int qtts_prefix_capture(qtts_ctx *c, qtts_prefix **out)
{
    NEED_MODEL(c);
    if (!out) return QTTS_ERR_INVALID;
    *out = nullptr;
    const int64_t len = c->h_st->kv_len;
    if (len < 1) return fail(c, QTTS_ERR_STATE, "no cached positions to keep as a prefix");
    const int full = (int)(len / KV_PAGE);
    int32_t tail = -1;
    if (len % KV_PAGE) {
        RCHK(page_take(c, &tail));
        const int r = page_copy(c, c->seq_ptab[full], tail);
        if (r == QTTS_OK) HIPCHK(c, hipStreamSynchronize(c->stream));
        if (r != QTTS_OK) {
            page_drop(c, tail);
            return r;
        }
    }
    qtts_prefix *p = new qtts_prefix();
    p->owner = c;
    p->model_gen = c->model_gen;
    p->len = len;
    for (int i = 0; i < full; i++) {
        p->pages.push_back(c->seq_ptab[i]);
        c->page_ref[c->seq_ptab[i]]++;
    }
    if (tail >= 0) p->pages.push_back(tail);
    *out = p;
    return QTTS_OK;
}

extern "C" int qtts_prefix_attach(qtts_ctx *c, const qtts_prefix *p)
{
    NEED_MODEL(c);
    if (!p) return QTTS_ERR_INVALID;
    if (p->owner != c || p->model_gen != c->model_gen)
        return fail(c, QTTS_ERR_STATE, "prefix kept by another context or for another model");
    const int full = (int)(p->len / KV_PAGE);
    if (p->len % KV_PAGE) {
        // the partial page is copied: the sequence appends into it
        int32_t cur = c->seq_ptab[full];
        if (c->page_ref[cur] > 1) {
            int32_t q;
            RCHK(page_take(c, &q));
            page_drop(c, cur);
            c->seq_ptab[full] = q;
            cur = q;
        }
        RCHK(page_copy(c, p->pages[full], cur));
    }
    for (int i = 0; i < full; i++) {
        const int32_t pg = p->pages[i];
        if (c->seq_ptab[i] == pg) continue;
        c->page_ref[pg]++;
        page_drop(c, c->seq_ptab[i]);
        c->seq_ptab[i] = pg;
    }
    // Pages past the prefix may still be shared with another kept prefix
    // (attaching a shorter prefix over a longer one's pages): the steps and
    // frames that follow append there without a copy-on-write check, so
    // they get private pages now.
    RCHK(seq_unshare_from(c, p->len));
    RCHK(push_ptab(c));
    c->gen_started = false;
    c->h_st->kv_len = (int32_t)p->len;
    c->h_st->position = p->len;
    return write_state(c);
}

extern "C" int qtts_prefix_len(const qtts_prefix *p, int64_t *len)
{
    if (!p || !len) return QTTS_ERR_INVALID;
    *len = p->len;
    return QTTS_OK;
}

extern "C" int qtts_prefix_free(qtts_ctx *c, qtts_prefix *p)
{
    if (!c || !p || p->owner != c) return QTTS_ERR_INVALID;
    if (c->has_model && p->model_gen == c->model_gen)
        for (int32_t pg : p->pages) page_drop(c, pg);
    delete p;
    return QTTS_OK;
}

extern "C" int qtts_prefix_suffix_split(int64_t block_len, int64_t n_ref, int64_t prefix_len, int64_t *suffix_len)
{
    if (!suffix_len || block_len < 0 || n_ref < 0 || prefix_len < 0) return QTTS_ERR_INVALID;
    *suffix_len = 0;
    if (prefix_len != 9 + n_ref || n_ref >= block_len) return 0;
    *suffix_len = block_len - n_ref;
    return 1;
}

// ---------------------------------------------------------------------------
// prompt construction
// ---------------------------------------------------------------------------

extern "C" int qtts_icl_layout(int64_t n_ref, int64_t n_text, int64_t n_frames, int64_t *icl_len,
                               int64_t *remainder_len)
{
    if (!icl_len || !remainder_len || n_ref < 0 || n_text < 0 || n_frames < 1) return QTTS_ERR_INVALID;
    const int64_t text_len = n_ref + n_text + 1, codec_len = n_frames + 1;
    *icl_len = codec_len;
    *remainder_len = text_len > codec_len ? text_len - codec_len : 0;
    return QTTS_OK;
}

// Text projection of n ids into device rows out[n][hidden]: table rows, then
// fc1 + bias and SiLU, fc2 + bias on the matrix cores.  `scratch` holds
// n * (text_hidden + hidden) floats.
static int text_rows(qtts_ctx *c, const uint32_t *d_ids, int n, float *out, float *scratch)
{
    const TalkerDev &m = c->tm;
    if (!gemm_supported(m.text_fc1) || !gemm_supported(m.text_fc2))
        return fail(c, QTTS_ERR_UNSUPPORTED, "text projection widths outside the matrix-core GEMM");
    Q4Rows e = m.text_rows;
    e.n = m.text_hidden;
    float *raw = scratch, *h1 = scratch + (size_t)n * m.text_hidden;
    RCHK(ensure_rmax(c, n));
    HIPCHK(c, enqueue_gather_rows(e, d_ids, n, raw, m.text_hidden, c->stream));
    HIPCHK(c, enqueue_gemm_bias(m.text_fc1, raw, n, m.text_fc1_bias, true, h1, m.text_fc1.n, c->d_rmax, c->stream));
    HIPCHK(c, enqueue_gemm_bias(m.text_fc2, h1, n, m.text_fc2_bias, false, out, m.hidden, c->d_rmax, c->stream));
    return QTTS_OK;
}

// Device scratch for one prompt call, freed on every exit.
struct DevScratch {
    void *p = nullptr;
    ~DevScratch() { if (p) hipFree(p); }
};

extern "C" int qtts_embed_text_tokens(qtts_ctx *c, const uint32_t *ids, int64_t n, float *out, int flags)
{
    NEED_MODEL(c);
    if (!ids || !out || n < 0) return QTTS_ERR_INVALID;
    if (n == 0) return QTTS_OK;
    const TalkerDev &m = c->tm;
    for (int64_t i = 0; i < n; i++)
        if ((int64_t)ids[i] >= m.text_rows.rows) return fail(c, QTTS_ERR_INVALID, "text token %u out of range", ids[i]);
    const size_t n_out = (size_t)n * m.hidden;
    DevScratch buf;
    HIPCHK(c, hipMalloc(&buf.p, n * sizeof(uint32_t) + ((size_t)n * (m.text_hidden + m.text_fc1.n) + n_out) * sizeof(float)));
    float *rows = (float *)buf.p, *scratch = rows + n_out;
    uint32_t *d_ids = (uint32_t *)(scratch + (size_t)n * (m.text_hidden + m.text_fc1.n));
    HIPCHK(c, hipMemcpyAsync(d_ids, ids, n * sizeof(uint32_t), hipMemcpyHostToDevice, c->stream));
    RCHK(text_rows(c, d_ids, (int)n, rows, scratch));
    RCHK(stage_out(c, rows, (int64_t)n_out, out, flags));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return QTTS_OK;
}

extern "C" int qtts_build_icl_block(qtts_ctx *c, const uint32_t *ref_tokens, int64_t n_ref,
                                    const uint32_t *text_tokens, int64_t n_text, const uint32_t *ref_codes,
                                    int64_t n_frames, float *icl_out, float *remainder_out, int flags)
{
    NEED_MODEL(c);
    int64_t icl_len, rem_len;
    if ((n_ref && !ref_tokens) || (n_text && !text_tokens) || !ref_codes || !icl_out ||
        qtts_icl_layout(n_ref, n_text, n_frames, &icl_len, &rem_len) != QTTS_OK)
        return QTTS_ERR_INVALID;
    if (rem_len && !remainder_out) return QTTS_ERR_INVALID;
    const TalkerDev &m = c->tm;
    const PredictorDev &p = c->pm;
    if (p.n_groups != 15 || p.emb_rows.n != m.hidden)
        return fail(c, QTTS_ERR_UNSUPPORTED, "ICL block needs 15 predictor tables of the talker width");
    const int64_t text_len = n_ref + n_text + 1;
    // ids: ref ++ text ++ [TTS_EOS, TTS_PAD]; codes [16][n_frames]
    std::vector<uint32_t> ids;
    ids.insert(ids.end(), ref_tokens, ref_tokens + n_ref);
    ids.insert(ids.end(), text_tokens, text_tokens + n_text);
    ids.push_back(TTS_EOS_ID);
    ids.push_back(TTS_PAD_ID);
    for (uint32_t t : ids)
        if ((int64_t)t >= m.text_rows.rows) return fail(c, QTTS_ERR_INVALID, "text token %u out of range", t);
    for (int64_t i = 0; i < 16 * n_frames; i++)
        if (ref_codes[i] >= (uint32_t)p.emb_rows.rows || (i < n_frames && ref_codes[i] >= (uint32_t)m.codec_rows.rows))
            return fail(c, QTTS_ERR_INVALID, "reference code %u out of range", ref_codes[i]);
    const int nt = (int)ids.size();
    const size_t H = m.hidden;
    DevScratch buf;
    const size_t f_text = (size_t)nt * H, f_codec = (size_t)(n_frames + 1) * H, f_icl = (size_t)icl_len * H;
    const size_t f_scr = (size_t)nt * (m.text_hidden + m.text_fc1.n);
    HIPCHK(c, hipMalloc(&buf.p, (f_text + f_codec + f_icl + f_scr) * sizeof(float) +
                                    (nt + 16 * n_frames + 1) * sizeof(uint32_t)));
    float *text = (float *)buf.p, *codec = text + f_text, *icl = codec + f_codec, *scr = icl + f_icl;
    uint32_t *d_ids = (uint32_t *)(scr + f_scr), *d_codes = d_ids + nt;
    const uint32_t bos = CODEC_BOS_ID;
    HIPCHK(c, hipMemcpyAsync(d_ids, ids.data(), nt * sizeof(uint32_t), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(d_codes, ref_codes, 16 * n_frames * sizeof(uint32_t), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(d_codes + 16 * n_frames, &bos, sizeof(uint32_t), hipMemcpyHostToDevice, c->stream));
    // text side: rows 0..text_len-1 (tts_eos last), row text_len = tts_pad
    RCHK(text_rows(c, d_ids, nt, text, scr));
    // codec side: codec_bos, then the per-frame sums (generate_new.rs:161-172)
    HIPCHK(c, enqueue_gather_rows(m.codec_rows, d_codes + 16 * n_frames, 1, codec, (int)H, c->stream));
    HIPCHK(c, enqueue_codec_frame_rows(m.codec_rows, p.emb_rows, 15, d_codes, (int)n_frames, codec + H, (int)H,
                                       c->stream));
    // pairs (generate_new.rs:174-189): text row (tts_pad past the text) + codec row
    const int64_t paired = std::min(text_len, icl_len);
    HIPCHK(c, enqueue_add_rows(text, (int)H, codec, (int)H, icl, (int)H, (int)paired, (int)H, c->stream));
    if (icl_len > paired)
        HIPCHK(c, enqueue_add_rows(text + (size_t)text_len * H, 0, codec + paired * H, (int)H, icl + paired * H, (int)H,
                                   (int)(icl_len - paired), (int)H, c->stream));
    RCHK(stage_out(c, icl, (int64_t)f_icl, icl_out, flags));
    if (rem_len) RCHK(stage_out(c, text + (size_t)icl_len * H, rem_len * (int64_t)H, remainder_out, flags));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return QTTS_OK;
}

// Floats of device scratch text_rows needs for n text ids.
static size_t text_scratch_floats(const TalkerDev &m, int64_t n) { return (size_t)n * (m.text_hidden + m.text_fc1.n); }

static int check_text_ids(qtts_ctx *c, const uint32_t *ids, int64_t n)
{
    for (int64_t i = 0; i < n; i++)
        if ((int64_t)ids[i] >= c->tm.text_rows.rows) return fail(c, QTTS_ERR_INVALID, "text token %u out of range", ids[i]);
    return QTTS_OK;
}

// The 9 head rows of the prompt into out [9][H] (device): build_role_prefix
// (generate_new.rs:91-97), then build_codec_prefix_voice (:200-223) when a
// voice embedding is given, else build_codec_prefix_builtin (:226-238, the
// overlay of build_tts_pad_bos :100-108).  Each row is one two-operand sum
// (codec row + text row, or the voice row + TTS_PAD) or a text row.
// voice: device, voice_len floats (rows past min(voice_len, H) stay zero in
// the voice row, as generate_new.rs:211-214 leaves them).
static int head_rows(qtts_ctx *c, uint32_t speaker_id, uint32_t language_id, const float *voice, int64_t voice_len,
                     float *out)
{
    const TalkerDev &m = c->tm;
    const size_t H = m.hidden;
    const uint32_t tids[5] = {IM_START_ID, ASSISTANT_ID, NEWLINE_ID, TTS_PAD_ID, TTS_BOS_ID};
    const uint32_t cids[6] = {CODEC_THINK_ID, CODEC_THINK_BOS_ID, language_id, CODEC_THINK_EOS_ID,
                              voice ? CODEC_PAD_ID : speaker_id, CODEC_PAD_ID};
    RCHK(check_text_ids(c, tids, 5));
    for (uint32_t t : cids)
        if ((int64_t)t >= m.codec_rows.rows) return fail(c, QTTS_ERR_INVALID, "codec token %u out of range", t);
    DevScratch buf;
    HIPCHK(c, hipMalloc(&buf.p, (11 * H + text_scratch_floats(m, 5)) * sizeof(float) + 11 * sizeof(uint32_t)));
    float *T = (float *)buf.p, *C = T + 5 * H, *scr = C + 6 * H;
    uint32_t *d_ids = (uint32_t *)(scr + text_scratch_floats(m, 5));
    HIPCHK(c, hipMemcpyAsync(d_ids, tids, sizeof tids, hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(d_ids + 5, cids, sizeof cids, hipMemcpyHostToDevice, c->stream));
    RCHK(text_rows(c, d_ids, 5, T, scr));
    HIPCHK(c, enqueue_gather_rows(m.codec_rows, d_ids + 5, 6, C, (int)H, c->stream));
    const int64_t vm = voice ? std::min<int64_t>(voice_len, (int64_t)H) : 0;
    if (voice && vm > 0)
        HIPCHK(c, hipMemcpyAsync(C + 4 * H, voice, vm * sizeof(float), hipMemcpyDeviceToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(out, T, 3 * H * sizeof(float), hipMemcpyDeviceToDevice, c->stream));
    // rows 3..7: codec (or voice) row + TTS_PAD; row 8: CODEC_PAD + TTS_BOS
    HIPCHK(c, enqueue_add_rows(T + 3 * H, 0, C, (int)H, out + 3 * H, (int)H, 5, (int)H, c->stream));
    HIPCHK(c, enqueue_add_rows(T + 4 * H, 0, C + 5 * H, (int)H, out + 8 * H, (int)H, 1, (int)H, c->stream));
    if (voice) HIPCHK(c, enqueue_zero_cols(out + 7 * H, 1, (int)H, (int)vm, (int)H, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return QTTS_OK;
}

extern "C" int qtts_build_prefill_head(qtts_ctx *c, uint32_t speaker_id, uint32_t language_id, const float *voice,
                                       int64_t voice_len, float *out, int flags)
{
    NEED_MODEL(c);
    if (!out || voice_len < 0) return QTTS_ERR_INVALID;
    const size_t H = c->tm.hidden;
    DevScratch buf;
    HIPCHK(c, hipMalloc(&buf.p, (9 * H + (voice ? (size_t)voice_len : 0) + 1) * sizeof(float)));
    float *rows = (float *)buf.p, *v = rows + 9 * H;
    if (voice && voice_len) RCHK(stage_in(c, voice, voice_len, v, flags));
    RCHK(head_rows(c, speaker_id, language_id, voice ? v : nullptr, voice_len, rows));
    RCHK(stage_out(c, rows, (int64_t)(9 * H), out, flags));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return QTTS_OK;
}

extern "C" int qtts_build_icl_prefix(qtts_ctx *c, const uint32_t *ref_tokens, int64_t n_ref,
                                     const uint32_t *ref_codes, int64_t n_frames, float *out, int flags)
{
    NEED_MODEL(c);
    if (n_ref < 0 || n_frames < 1 || (n_ref && (!ref_tokens || !out)) || !ref_codes) return QTTS_ERR_INVALID;
    if (n_ref == 0) return QTTS_OK;
    const TalkerDev &m = c->tm;
    const PredictorDev &p = c->pm;
    if (p.n_groups != 15 || p.emb_rows.n != m.hidden)
        return fail(c, QTTS_ERR_UNSUPPORTED, "ICL rows need 15 predictor tables of the talker width");
    RCHK(check_text_ids(c, ref_tokens, n_ref));
    for (int64_t i = 0; i < 16 * n_frames; i++)
        if (ref_codes[i] >= (uint32_t)p.emb_rows.rows || (i < n_frames && ref_codes[i] >= (uint32_t)m.codec_rows.rows))
            return fail(c, QTTS_ERR_INVALID, "reference code %u out of range", ref_codes[i]);
    const size_t H = m.hidden;
    // codec side of pair i: CODEC_BOS, frames 0.. (generate_new.rs:255-275),
    // CODEC_PAD for a ref token past the last frame
    const int64_t nf = std::min<int64_t>(n_ref - 1, n_frames), npad = n_ref - 1 - nf;
    DevScratch buf;
    HIPCHK(c, hipMalloc(&buf.p, (3 * (size_t)n_ref * H + text_scratch_floats(m, n_ref)) * sizeof(float) +
                                    (n_ref + 16 * n_frames + 2) * sizeof(uint32_t)));
    float *text = (float *)buf.p, *codec = text + n_ref * H, *rows = codec + n_ref * H, *scr = rows + n_ref * H;
    uint32_t *d_ids = (uint32_t *)(scr + text_scratch_floats(m, n_ref)), *d_codes = d_ids + n_ref;
    const uint32_t special[2] = {CODEC_BOS_ID, CODEC_PAD_ID};
    HIPCHK(c, hipMemcpyAsync(d_ids, ref_tokens, n_ref * sizeof(uint32_t), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(d_codes, ref_codes, 16 * n_frames * sizeof(uint32_t), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(d_codes + 16 * n_frames, special, sizeof special, hipMemcpyHostToDevice, c->stream));
    RCHK(text_rows(c, d_ids, (int)n_ref, text, scr));
    HIPCHK(c, enqueue_gather_rows(m.codec_rows, d_codes + 16 * n_frames, 1, codec, (int)H, c->stream));
    if (nf > 0)
        HIPCHK(c, enqueue_codec_frame_rows(m.codec_rows, p.emb_rows, 15, d_codes, (int)n_frames, codec + H, (int)H,
                                           c->stream));
    for (int64_t i = 0; i < npad; i++)
        HIPCHK(c, enqueue_gather_rows(m.codec_rows, d_codes + 16 * n_frames + 1, 1, codec + (1 + nf + i) * H, (int)H,
                                      c->stream));
    HIPCHK(c, enqueue_add_rows(text, (int)H, codec, (int)H, rows, (int)H, (int)n_ref, (int)H, c->stream));
    RCHK(stage_out(c, rows, n_ref * (int64_t)H, out, flags));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return QTTS_OK;
}

extern "C" int qtts_build_trailing_text(qtts_ctx *c, const uint32_t *tokens, int64_t n, float *out, int flags)
{
    NEED_MODEL(c);
    if (n < 0 || (n && !tokens) || !out) return QTTS_ERR_INVALID;
    std::vector<uint32_t> ids(tokens + std::min<int64_t>(n, 1), tokens + n);
    ids.push_back(TTS_EOS_ID);
    return qtts_embed_text_tokens(c, ids.data(), (int64_t)ids.size(), out, flags);
}

extern "C" int qtts_prefill_custom_voice(qtts_ctx *c, const uint32_t *text_tokens, int64_t n_text,
                                         uint32_t speaker_id, uint32_t language_id, const float *voice,
                                         int64_t voice_len, const float *icl_rows, int64_t n_icl, float *hidden_out,
                                         float *logits_out, int64_t *position_out, int flags)
{
    NEED_MODEL(c);
    if (n_text < 0 || (n_text && !text_tokens) || voice_len < 0 || n_icl < 0 || (n_icl && !icl_rows) ||
        !hidden_out || !logits_out || !position_out)
        return QTTS_ERR_INVALID;
    if (icl_rows && !voice)
        return fail(c, QTTS_ERR_INVALID, "ICL rows follow the voice-cloning head only (generate_new.rs:413-431)");
    const TalkerDev &m = c->tm;
    const size_t H = m.hidden;
    const bool first = !icl_rows && n_text > 0;
    const int64_t n = 9 + (icl_rows ? n_icl : (first ? 1 : 0));
    if (first) RCHK(check_text_ids(c, text_tokens, 1));
    if (first && (int64_t)CODEC_BOS_ID >= m.codec_rows.rows) return fail(c, QTTS_ERR_INVALID, "no CODEC_BOS row");
    if (n > c->kv_cap) return fail(c, QTTS_ERR_CAPACITY, "prompt of %lld rows beyond the KV cache", (long long)n);
    DevScratch buf;
    HIPCHK(c, hipMalloc(&buf.p, ((size_t)(n + 2) * H + (voice ? (size_t)voice_len : 0) + m.vocab +
                                 text_scratch_floats(m, 1)) * sizeof(float) + 2 * sizeof(uint32_t)));
    float *X = (float *)buf.p, *row = X + (size_t)n * H, *v = row + 2 * H, *lg = v + (voice ? voice_len : 0);
    float *scr = lg + m.vocab;
    uint32_t *d_ids = (uint32_t *)(scr + text_scratch_floats(m, 1));
    if (voice && voice_len) RCHK(stage_in(c, voice, voice_len, v, flags));
    RCHK(head_rows(c, speaker_id, language_id, voice ? v : nullptr, voice_len, X));
    if (icl_rows) {
        RCHK(stage_in(c, icl_rows, n_icl * (int64_t)H, X + 9 * H, flags));
    } else if (first) {
        // CODEC_BOS + the first text token (generate_new.rs:423-431, 453-461)
        const uint32_t ids[2] = {text_tokens[0], CODEC_BOS_ID};
        HIPCHK(c, hipMemcpyAsync(d_ids, ids, sizeof ids, hipMemcpyHostToDevice, c->stream));
        RCHK(text_rows(c, d_ids, 1, row, scr));
        HIPCHK(c, enqueue_gather_rows(m.codec_rows, d_ids + 1, 1, row + H, (int)H, c->stream));
        HIPCHK(c, enqueue_add_rows(row + H, (int)H, row, (int)H, X + 9 * H, (int)H, 1, (int)H, c->stream));
    }
    RCHK(qtts_kv_reset(c));
    RCHK(qtts_talker_prefill(c, X, n, 0, row, flags | QTTS_DEVICE_PTRS));
    HIPCHK(c, enqueue_codec_head(m, c->ws, row, lg, c->stream));
    RCHK(stage_out(c, row, (int64_t)H, hidden_out, flags));
    RCHK(stage_out(c, lg, m.vocab, logits_out, flags));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    *position_out = icl_rows ? 9 + n_icl : (n_text > 0 ? 10 : 9);
    return QTTS_OK;
}

// ---------------------------------------------------------------------------
// speech decoder
// ---------------------------------------------------------------------------

// The split-f16 convolutions hold a weight as f16 hi + lo: f32-accurate for
// every |w| below the f16 maximum, and (through lo) to 2^-25 absolute
// below 2^-14.  A matrix outside that (any |w| >= 65504, or all of it below
// 2^-14 but not zero) sends the whole decoder to the f32 matrix path.
static void note_gemm_weights(qtts_ctx *c, const float *w, size_t n)
{
    float mx = 0.0f;
    for (size_t i = 0; i < n; i++) mx = std::max(mx, std::fabs(w[i]));
    if (!(mx < 65504.0f) || (mx > 0.0f && mx < 0x1p-14f)) c->dec.weights_f32 = true;
}

// Host matrix [k][n] (input-major) -> device [n][k] (the GEMM's A operand).
static int upload_t(qtts_ctx *c, const float *src, int k, int n, const float **out)
{
    if (!src) return fail(c, QTTS_ERR_INVALID, "null matrix in decoder descriptor");
    note_gemm_weights(c, src, (size_t)k * n);
    std::vector<float> t((size_t)k * n);
    for (int i = 0; i < k; i++)
        for (int j = 0; j < n; j++) t[(size_t)j * k + i] = src[(size_t)i * n + j];
    return upload_vec(c, c->dec_allocs, t.data(), t.size(), out);
}

static int upload_conv(qtts_ctx *c, const qtts_conv1d_host &h, DecConv *d)
{
    if (!h.weight || !h.bias || h.in_channels < 1 || h.out_channels < 1 || h.kernel_size < 1 || h.dilation < 1)
        return fail(c, QTTS_ERR_INVALID, "bad conv1d descriptor");
    if (h.stride != 1) return fail(c, QTTS_ERR_UNSUPPORTED, "strided conv1d not used by the decoder");
    const int IC = h.in_channels, OC = h.out_channels, K = h.kernel_size;
    if ((IC * K) % 4) return fail(c, QTTS_ERR_UNSUPPORTED, "conv1d in_channels*kernel %d not a multiple of 4", IC * K);
    d->ic = IC;
    d->oc = OC;
    d->k = K;
    d->dil = h.dilation;
    note_gemm_weights(c, h.weight, (size_t)OC * IC * K);
    if (K > 1 && conv_tap_major(IC, K)) {   // [out][in][k] -> [out][k][in]
        std::vector<float> w((size_t)OC * IC * K);
        for (int o = 0; o < OC; o++)
            for (int i = 0; i < IC; i++)
                for (int k = 0; k < K; k++) w[((size_t)o * K + k) * IC + i] = h.weight[((size_t)o * IC + i) * K + k];
        RCHK(upload_vec(c, c->dec_allocs, w.data(), w.size(), &d->w));
    } else {
        RCHK(upload_vec(c, c->dec_allocs, h.weight, (size_t)OC * IC * K, &d->w));
    }
    return upload_vec(c, c->dec_allocs, h.bias, (size_t)OC, &d->b);
}

// Transposed conv [in][out][k] -> per stride phase r: [oc][ic*taps] with
// taps (k = 2*stride) x[i-1] <- tap r + stride, x[i] <- tap r.
static int upload_convt(qtts_ctx *c, const qtts_convt1d_host &h, DecConvT *d)
{
    if (!h.weight || !h.bias || h.in_channels < 1 || h.out_channels < 1 || h.stride < 1)
        return fail(c, QTTS_ERR_INVALID, "bad conv_transpose1d descriptor");
    if (h.padding != 0 || (h.kernel_size != h.stride && h.kernel_size != 2 * h.stride))
        return fail(c, QTTS_ERR_UNSUPPORTED, "conv_transpose1d needs kernel = stride or 2*stride, padding 0");
    const int IC = h.in_channels, OC = h.out_channels, K = h.kernel_size, S = h.stride;
    const int taps = K / S;
    if ((IC * taps) % 4) return fail(c, QTTS_ERR_UNSUPPORTED, "conv_transpose1d in_channels*taps not a multiple of 4");
    const bool tm = conv_tap_major(IC, taps);
    std::vector<float> p((size_t)S * OC * IC * taps);
    for (int r = 0; r < S; r++)
        for (int oc = 0; oc < OC; oc++)
            for (int ic = 0; ic < IC; ic++) {
                const float *w = h.weight + ((size_t)ic * OC + oc) * K;
                const size_t row = ((size_t)r * OC + oc) * IC * taps;
                for (int j = 0; j < taps; j++) {
                    const float v = (taps == 2 && j == 0) ? w[r + S] : w[r];
                    p[row + (tm ? (size_t)j * IC + ic : (size_t)ic * taps + j)] = v;
                }
            }
    d->ic = IC;
    d->oc = OC;
    d->stride = S;
    d->taps = taps;
    note_gemm_weights(c, p.data(), p.size());
    RCHK(upload_vec(c, c->dec_allocs, p.data(), p.size(), &d->phases));
    return upload_vec(c, c->dec_allocs, h.bias, (size_t)OC, &d->b);
}

static int upload_decoder(qtts_ctx *c, const qtts_decoder_host *h)
{
    DecoderDev &d = c->dec;
    auto &A = c->dec_allocs;
    const int H = h->hidden, NH = h->n_heads, HD = h->head_dim, I = h->inter, D = h->codebook_dim, V = h->vq_dim;
    const int LAT = h->latent, AD = NH * HD;
    if (H < 1 || NH < 1 || (HD != 64 && HD != 16) || I < 1 || D < 1 || V < 1 || LAT < 1 || h->sliding_window < 1)
        return fail(c, QTTS_ERR_UNSUPPORTED, "decoder shape not supported (head_dim %d)", HD);
    if (H % 4 || I % 4 || D % 2 || LAT % 4)   // matrix-core contractions run in quads
        return fail(c, QTTS_ERR_UNSUPPORTED, "decoder widths must be multiples of 4");
    if (h->n_rest < 0 || h->n_rest > 15 || h->codebook_size < 1 || !h->first_codebook || !h->first_output_proj ||
        (h->n_rest && (!h->rest_codebooks || !h->rest_output_proj)))
        return fail(c, QTTS_ERR_INVALID, "decoder codebooks");
    if (h->output_conv.out_channels != 1 || h->pre_conv.in_channels != V || h->pre_conv.out_channels != LAT)
        return fail(c, QTTS_ERR_INVALID, "decoder conv shapes");
    d.weights_f32 = false;
    d.hidden = H; d.n_heads = NH; d.head_dim = HD; d.inter = I; d.window = h->sliding_window;
    d.codebook_dim = D; d.codebook_size = h->codebook_size; d.vq_dim = V; d.latent = LAT; d.n_rest = h->n_rest;
    const size_t cb = (size_t)h->codebook_size * D;
    RCHK(upload_vec(c, A, h->first_codebook, cb, &d.first_codebook));
    std::vector<const float *> rest(std::max(1, h->n_rest));
    for (int g = 0; g < h->n_rest; g++) RCHK(upload_vec(c, A, h->rest_codebooks[g], cb, &rest[g]));
    if (!h->n_rest) rest[0] = d.first_codebook;
    const float *const *drest = nullptr;
    RCHK(upload_vec(c, A, rest.data(), rest.size(), (const float *const **)&drest));
    d.rest_codebooks = drest;
    {   // [V][2D]: first | rest output projections, transposed
        std::vector<float> vp((size_t)V * 2 * D, 0.0f);
        for (int k = 0; k < D; k++)
            for (int v = 0; v < V; v++) {
                vp[(size_t)v * 2 * D + k] = h->first_output_proj[(size_t)k * V + v];
                if (h->n_rest) vp[(size_t)v * 2 * D + D + k] = h->rest_output_proj[(size_t)k * V + v];
            }
        note_gemm_weights(c, vp.data(), vp.size());
        RCHK(upload_vec(c, A, vp.data(), vp.size(), &d.vq_proj));
    }
    RCHK(upload_conv(c, h->pre_conv, &d.pre_conv));
    RCHK(upload_t(c, h->tf_input_w, LAT, H, &d.tf_in_w));
    RCHK(upload_vec(c, A, h->tf_input_b, (size_t)H, &d.tf_in_b));
    c->dec_layers.assign(h->n_tf_layers, DecLayer{});
    for (int l = 0; l < h->n_tf_layers; l++) {
        const qtts_dec_layer_host &L = h->tf_layers[l];
        DecLayer &o = c->dec_layers[l];
        if (!L.q_proj || !L.k_proj || !L.v_proj || !L.gate_proj || !L.up_proj)
            return fail(c, QTTS_ERR_INVALID, "decoder layer %d: null matrix", l);
        std::vector<float> qkv((size_t)3 * AD * H), gu((size_t)2 * I * H);
        for (int k = 0; k < H; k++) {
            for (int j = 0; j < AD; j++) {
                qkv[(size_t)j * H + k] = L.q_proj[(size_t)k * AD + j];
                qkv[(size_t)(AD + j) * H + k] = L.k_proj[(size_t)k * AD + j];
                qkv[(size_t)(2 * AD + j) * H + k] = L.v_proj[(size_t)k * AD + j];
            }
            for (int j = 0; j < I; j++) {
                gu[(size_t)(2 * j) * H + k] = L.gate_proj[(size_t)k * I + j];
                gu[(size_t)(2 * j + 1) * H + k] = L.up_proj[(size_t)k * I + j];
            }
        }
        note_gemm_weights(c, qkv.data(), qkv.size());
        note_gemm_weights(c, gu.data(), gu.size());
        RCHK(upload_vec(c, A, qkv.data(), qkv.size(), &o.qkv));
        RCHK(upload_vec(c, A, gu.data(), gu.size(), &o.gate_up));
        RCHK(upload_t(c, L.o_proj, AD, H, &o.o));
        RCHK(upload_t(c, L.down_proj, I, H, &o.down));
        RCHK(upload_vec(c, A, L.input_norm, (size_t)H, &o.in_norm));
        RCHK(upload_vec(c, A, L.post_attn_norm, (size_t)H, &o.post_norm));
        RCHK(upload_vec(c, A, L.attn_scale, (size_t)H, &o.attn_scale));
        RCHK(upload_vec(c, A, L.mlp_scale, (size_t)H, &o.mlp_scale));
    }
    d.tf = c->dec_layers.data();
    d.n_tf = h->n_tf_layers;
    RCHK(upload_vec(c, A, h->tf_norm, (size_t)H, &d.tf_norm));
    RCHK(upload_t(c, h->tf_output_w, H, LAT, &d.tf_out_w));
    RCHK(upload_vec(c, A, h->tf_output_b, (size_t)LAT, &d.tf_out_b));
    // per-frame sizes of every stage, for the workspace
    int64_t fpf = std::max<int64_t>({(int64_t)2 * D, V, LAT, H, 3 * AD, I, AD});
    int64_t factor = 1;
    c->dec_up.assign(h->n_upsample, DecUpsample{});
    int ch = LAT;
    for (int u = 0; u < h->n_upsample; u++) {
        const qtts_upsample_host &U = h->upsample[u];
        DecUpsample &o = c->dec_up[u];
        if (U.channels != ch || U.conv_t.in_channels != ch || U.conv_t.out_channels != ch ||
            U.dw_conv.channels != ch || U.inner < 1 || U.inner % 4)
            return fail(c, QTTS_ERR_INVALID, "upsample stage %d shapes", u);
        RCHK(upload_convt(c, U.conv_t, &o.conv_t));
        RCHK(upload_vec(c, A, U.dw_conv.weight, (size_t)ch * U.dw_conv.kernel_size, &o.dw_w));
        RCHK(upload_vec(c, A, U.dw_conv.bias, (size_t)ch, &o.dw_b));
        o.dw_k = U.dw_conv.kernel_size;
        RCHK(upload_vec(c, A, U.norm_w, (size_t)ch, &o.norm_w));
        RCHK(upload_vec(c, A, U.norm_b, (size_t)ch, &o.norm_b));
        RCHK(upload_t(c, U.pw1_w, ch, U.inner, &o.pw1));
        RCHK(upload_vec(c, A, U.pw1_b, (size_t)U.inner, &o.pw1_b));
        RCHK(upload_t(c, U.pw2_w, U.inner, ch, &o.pw2));
        RCHK(upload_vec(c, A, U.pw2_b, (size_t)ch, &o.pw2_b));
        RCHK(upload_vec(c, A, U.gamma, (size_t)ch, &o.gamma));
        o.ch = ch;
        o.inner = U.inner;
        factor *= U.conv_t.stride;
        fpf = std::max<int64_t>(fpf, (int64_t)std::max(U.inner, ch) * factor);
    }
    d.up = c->dec_up.data();
    d.n_up = h->n_upsample;
    if (h->vocos_init.in_channels != ch) return fail(c, QTTS_ERR_INVALID, "vocos init input channels");
    RCHK(upload_conv(c, h->vocos_init, &d.voc_init));
    ch = h->vocos_init.out_channels;
    fpf = std::max<int64_t>(fpf, (int64_t)ch * factor);
    c->dec_voc.assign(h->n_vocos_blocks, DecVocos{});
    c->dec_res.assign(h->n_vocos_blocks, {});
    for (int b = 0; b < h->n_vocos_blocks; b++) {
        const qtts_vocos_block_host &B = h->vocos_blocks[b];
        DecVocos &o = c->dec_voc[b];
        if (B.upsample.in_channels != ch) return fail(c, QTTS_ERR_INVALID, "vocos block %d input channels", b);
        RCHK(upload_vec(c, A, B.pre_snake_alpha, (size_t)ch, &o.pre_alpha));
        RCHK(upload_vec(c, A, B.pre_snake_beta, (size_t)ch, &o.pre_beta));
        RCHK(upload_convt(c, B.upsample, &o.up));
        ch = B.upsample.out_channels;
        factor *= B.upsample.stride;
        fpf = std::max<int64_t>(fpf, (int64_t)ch * factor);
        c->dec_res[b].assign(B.n_residuals, DecVocosRes{});
        for (int r = 0; r < B.n_residuals; r++) {
            const qtts_vocos_res_host &R = B.residuals[r];
            DecVocosRes &q = c->dec_res[b][r];
            if (R.conv1.in_channels != ch || R.conv1.out_channels != ch || R.conv2.in_channels != ch ||
                R.conv2.out_channels != ch)
                return fail(c, QTTS_ERR_INVALID, "vocos residual %d.%d shapes", b, r);
            RCHK(upload_vec(c, A, R.act1_alpha, (size_t)ch, &q.a1_alpha));
            RCHK(upload_vec(c, A, R.act1_beta, (size_t)ch, &q.a1_beta));
            RCHK(upload_vec(c, A, R.act2_alpha, (size_t)ch, &q.a2_alpha));
            RCHK(upload_vec(c, A, R.act2_beta, (size_t)ch, &q.a2_beta));
            RCHK(upload_conv(c, R.conv1, &q.c1));
            RCHK(upload_conv(c, R.conv2, &q.c2));
        }
        o.res = c->dec_res[b].data();
        o.n_res = B.n_residuals;
    }
    d.voc = c->dec_voc.data();
    d.n_voc = h->n_vocos_blocks;
    if (h->output_conv.in_channels != ch) return fail(c, QTTS_ERR_INVALID, "output conv input channels");
    if ((h->output_conv.kernel_size - 1) * h->output_conv.dilation > 64)
        return fail(c, QTTS_ERR_UNSUPPORTED, "output conv reach (kernel-1)*dilation above 64");
    RCHK(upload_vec(c, A, h->final_snake_alpha, (size_t)ch, &d.final_alpha));
    RCHK(upload_vec(c, A, h->final_snake_beta, (size_t)ch, &d.final_beta));
    RCHK(upload_vec(c, A, h->output_conv.weight, (size_t)ch * h->output_conv.kernel_size, &d.out_w));
    d.out_b = h->output_conv.bias[0];
    d.out_k = h->output_conv.kernel_size;
    d.out_dil = h->output_conv.dilation;
    if (!h->rope_cos || !h->rope_sin || h->rope_max_pos < 1) return fail(c, QTTS_ERR_INVALID, "decoder rope tables");
    RCHK(upload_vec(c, A, h->rope_cos, (size_t)h->rope_max_pos * (HD / 2), &d.rope_cos));
    RCHK(upload_vec(c, A, h->rope_sin, (size_t)h->rope_max_pos * (HD / 2), &d.rope_sin));
    d.rope_rows = h->rope_max_pos;
    c->dec_floats_per_frame = fpf;
    return QTTS_OK;
}

static void free_decoder(qtts_ctx *c)
{
    free_list(c->dec_allocs);
    if (c->dws_mem) hipFree(c->dws_mem);
    c->dws_mem = nullptr;
    c->dws = DecoderWs{};
    c->has_decoder = false;
}

extern "C" int qtts_decoder_upload(qtts_ctx *c, const qtts_decoder_host *d)
{
    if (!c || !d) return QTTS_ERR_INVALID;
    hipSetDevice(c->device);
    free_decoder(c);
    const int r = upload_decoder(c, d);
    if (r != QTTS_OK) {
        free_decoder(c);
        return r;
    }
    c->has_decoder = true;
    return QTTS_OK;
}

// Split-K partial sums of the decoder's convolutions (64 MiB): enough to
// split every stage of short utterances, where the launches are too small
// to fill the GPU; long ones have columns enough and do not split.
static constexpr size_t DEC_PART_FLOATS = (size_t)16 << 20;

extern "C" int qtts_decoder_dims(qtts_ctx *c, int32_t *n_codebooks, int32_t *codebook_size,
                                 int64_t *samples_per_frame)
{
    if (!c || !n_codebooks || !codebook_size || !samples_per_frame) return QTTS_ERR_INVALID;
    if (!c->has_decoder) return fail(c, QTTS_ERR_STATE, "no speech decoder uploaded");
    const DecoderDev &d = c->dec;
    int64_t factor = 1;
    for (int u = 0; u < d.n_up; u++) factor *= d.up[u].conv_t.stride;
    for (int b = 0; b < d.n_voc; b++) factor *= d.voc[b].up.stride;
    *n_codebooks = d.n_rest + 1;
    *codebook_size = d.codebook_size;
    *samples_per_frame = factor;
    return QTTS_OK;
}

static int ensure_dec_ws(qtts_ctx *c, int frames)
{
    if (frames <= c->dws.cap_frames) return QTTS_OK;
    if (c->dws_mem) hipFree(c->dws_mem);
    c->dws_mem = nullptr;
    c->dws = DecoderWs{};
    const size_t per = (size_t)c->dec_floats_per_frame * frames;
    const size_t part = DEC_PART_FLOATS;
    void *m = nullptr;
    HIPCHK(c, hipMalloc(&m, (5 * per + part) * sizeof(float) + (size_t)16 * frames * sizeof(uint32_t) + 256));
    c->dws_mem = m;
    float *f = (float *)m;
    c->dws.a = f;
    c->dws.b = f + per;
    c->dws.c = f + 2 * per;
    c->dws.d = f + 3 * per;
    c->dws.e = f + 4 * per;
    c->dws.part = f + 5 * per;
    c->dws.part_cap = part;
    c->dws.codes = (uint32_t *)(f + 5 * per + part);
    c->dws.range_flag = (int32_t *)(c->dws.codes + (size_t)16 * frames);
    c->dws.cap_frames = frames;
    return QTTS_OK;
}

extern "C" int qtts_decode_to_audio(qtts_ctx *c, const uint32_t *codes, int64_t n_frames, const uint32_t *warmup,
                                    int64_t n_warmup, float *audio, int64_t capacity, int64_t *n_samples, int flags)
{
    if (!c || !n_samples) return QTTS_ERR_INVALID;
    *n_samples = 0;
    if (!c->has_decoder) return fail(c, QTTS_ERR_STATE, "no speech decoder uploaded");
    if (n_frames < 0 || n_warmup < 0 || (n_frames && !codes) || (n_warmup && !warmup)) return QTTS_ERR_INVALID;
    if (n_frames == 0) return QTTS_OK;   // decode_to_audio returns no samples for no codes
    const DecoderDev &d = c->dec;
    const int ncb = d.n_rest + 1;
    const int64_t T = n_frames + n_warmup;
    if (T > (1 << 20)) return fail(c, QTTS_ERR_CAPACITY, "too many frames");
    for (int64_t i = 0; i < (int64_t)ncb * n_frames; i++)
        if (codes[i] >= (uint32_t)d.codebook_size) return fail(c, QTTS_ERR_INVALID, "code %u out of range", codes[i]);
    for (int64_t i = 0; i < (int64_t)ncb * n_warmup; i++)
        if (warmup[i] >= (uint32_t)d.codebook_size) return fail(c, QTTS_ERR_INVALID, "warmup code out of range");
    int64_t factor = 1;
    for (int u = 0; u < d.n_up; u++) factor *= d.up[u].conv_t.stride;
    for (int b = 0; b < d.n_voc; b++) factor *= d.voc[b].up.stride;
    const int64_t len = T * factor;
    if (len > INT32_MAX) return fail(c, QTTS_ERR_CAPACITY, "%lld samples exceed one decode", (long long)len);
    // warmup_trim_len (decoder.rs:651-656)
    const int64_t cut = n_warmup ? std::min<int64_t>(n_warmup * len / T, len) : 0;
    const int64_t n = len - cut;
    if (!audio || capacity < n) {
        *n_samples = n;
        return fail(c, QTTS_ERR_CAPACITY, "audio buffer holds %lld samples, %lld needed", (long long)capacity,
                    (long long)n);
    }
    hipSetDevice(c->device);
    RCHK(ensure_dec_ws(c, (int)T));
    // codes of warmup ++ frames, codebook-major [ncb][T]
    std::vector<uint32_t> all((size_t)ncb * T);
    for (int g = 0; g < ncb; g++) {
        if (n_warmup) memcpy(&all[(size_t)g * T], warmup + (size_t)g * n_warmup, n_warmup * sizeof(uint32_t));
        memcpy(&all[(size_t)g * T + n_warmup], codes + (size_t)g * n_frames, n_frames * sizeof(uint32_t));
    }
    HIPCHK(c, hipMemcpyAsync(c->dws.codes, all.data(), all.size() * sizeof(uint32_t), hipMemcpyHostToDevice,
                             c->stream));
    float *out = audio;
    if (!(flags & QTTS_DEVICE_PTRS)) {   // stage the samples in the context's I/O buffer
        RCHK(ensure_io(c, n));
        out = c->d_io;
    }
    // on the split-f16 convolutions unless a weight matrix is outside their
    // range; inputs outside it (flagged by the convolutions) repeat the
    // decode on the f32 matrix path
    c->dws.f32 = d.weights_f32;
    HIPCHK(c, enqueue_decode(d, c->dws, c->dws.codes, (int)T, cut, out, c->stream));
    int32_t range = 0;
    HIPCHK(c, hipMemcpyAsync(&range, c->dws.range_flag, sizeof range, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    if (range && !c->dws.f32) {
        c->dws.f32 = true;
        const hipError_t e = enqueue_decode(d, c->dws, c->dws.codes, (int)T, cut, out, c->stream);
        c->dws.f32 = false;
        HIPCHK(c, e);
    }
    if (!(flags & QTTS_DEVICE_PTRS))
        HIPCHK(c, hipMemcpyAsync(audio, out, (size_t)n * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    *n_samples = n;
    return QTTS_OK;
}

// ---------------------------------------------------------------------------
// predictor and sampler (operator level)
// ---------------------------------------------------------------------------

extern "C" int qtts_predictor_chain(qtts_ctx *c, const float *th, const float *sem, uint32_t *codes_out, int flags)
{
    NEED_MODEL(c);
    if (!th || !sem || !codes_out) return QTTS_ERR_INVALID;
    const int H = c->tm.hidden;
    RCHK(stage_in(c, th, H, c->d_io, flags));
    RCHK(stage_in(c, sem, H, c->d_io2, flags));
    DevState z{};
    HIPCHK(c, hipMemcpyAsync(c->st_api, &z, sizeof(DevState), hipMemcpyHostToDevice, c->stream));
    RCHK(arm_sync_err(c, c->st_api));
    HIPCHK(c, enqueue_predictor_chain(c->pm, c->tm, c->ws, c->st_api, c->d_io, c->d_io2, nullptr, c->d_codes_api,
                                      c->stream));
    HIPCHK(c, hipMemcpyAsync(codes_out, c->d_codes_api, sizeof(uint32_t) * c->pm.n_groups, hipMemcpyDeviceToHost,
                             c->stream));
    DevState back{};
    HIPCHK(c, hipMemcpyAsync(&back, c->st_api, sizeof(DevState), hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    if (back.nan_flag) return fail(c, QTTS_ERR_NAN, "NaN logits in the predictor");
    if (back.sync_err) return fail(c, QTTS_ERR_HIP, "a cross-workgroup wait timed out (predictor q|k|v + attention launch)");
    return QTTS_OK;
}

extern "C" int qtts_acoustic_embed_sum(qtts_ctx *c, const uint32_t *codes, float *out, int flags)
{
    NEED_MODEL(c);
    if (!codes || !out) return QTTS_ERR_INVALID;
    for (int g = 0; g < c->pm.n_groups; g++)
        if ((int64_t)codes[g] >= c->pm.emb_rows.rows) return fail(c, QTTS_ERR_INVALID, "code %u out of range", codes[g]);
    HIPCHK(c, hipMemcpyAsync(c->d_codes_api, codes, sizeof(uint32_t) * c->pm.n_groups, hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, enqueue_embed_sum(c->pm.emb_rows, c->pm.n_groups, c->d_codes_api, c->d_io, c->stream));
    RCHK(stage_out(c, c->d_io, c->pm.emb_rows.n, out, flags));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return QTTS_OK;
}

extern "C" int qtts_sample_token(qtts_ctx *c, const float *logits, int64_t n, const qtts_sample_params *p,
                                 const uint32_t *prev, int64_t n_prev, uint64_t *rng, float temperature,
                                 uint32_t *out)
{
    if (!c || !logits || !p || !rng || !out || n <= 0 || n_prev < 0 || (n_prev > 0 && !prev)) return QTTS_ERR_INVALID;
    if (n > 4096 || n_prev > 4096) return fail(c, QTTS_ERR_UNSUPPORTED, "sampler supports n <= 4096");
    hipSetDevice(c->device);
    RCHK(ensure_io(c, 8192));
    HIPCHK(c, hipMemcpyAsync(c->d_io, logits, n * sizeof(float), hipMemcpyHostToDevice, c->stream));
    if (n_prev) HIPCHK(c, hipMemcpyAsync(c->d_prev_api, prev, n_prev * sizeof(uint32_t), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(c->d_rng_api, rng, sizeof(uint64_t), hipMemcpyHostToDevice, c->stream));
    DevState z{};
    HIPCHK(c, hipMemcpyAsync(c->st_api, &z, sizeof(DevState), hipMemcpyHostToDevice, c->stream));
    SampleArgsHost a{temperature, p->top_p, p->repetition_penalty, p->top_k, c->d_prev_api, (int)n_prev};
    HIPCHK(c, enqueue_sample_api(c->d_io, (int)n, a, c->d_rng_api, c->d_codes_api, c->st_api, c->stream));
    DevState back{};
    HIPCHK(c, hipMemcpyAsync(&back, c->st_api, sizeof(DevState), hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipMemcpyAsync(rng, c->d_rng_api, sizeof(uint64_t), hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipMemcpyAsync(out, c->d_codes_api, sizeof(uint32_t), hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    if (back.nan_flag) return fail(c, QTTS_ERR_NAN, "NaN in sampler input");
    return QTTS_OK;
}

// ---------------------------------------------------------------------------
// legacy loop (generate.rs:107-250)
// ---------------------------------------------------------------------------

extern "C" int qtts_sample_top_k(qtts_ctx *c, const float *logits, int64_t n, float temperature, int32_t top_k,
                                 const uint32_t *prev, int64_t n_prev, float repetition_penalty, uint64_t *rng,
                                 uint32_t *out)
{
    if (!c || !logits || !rng || !out || n <= 0 || n_prev < 0 || (n_prev > 0 && !prev)) return QTTS_ERR_INVALID;
    if (n > 4096) return fail(c, QTTS_ERR_UNSUPPORTED, "sampler supports n <= 4096");
    hipSetDevice(c->device);
    RCHK(ensure_io(c, std::max<int64_t>(8192, n_prev)));
    HIPCHK(c, hipMemcpyAsync(c->d_io, logits, n * sizeof(float), hipMemcpyHostToDevice, c->stream));
    uint32_t *d_prev = (uint32_t *)c->d_io2;
    if (n_prev) HIPCHK(c, hipMemcpyAsync(d_prev, prev, n_prev * sizeof(uint32_t), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(c->d_rng_api, rng, sizeof(uint64_t), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, enqueue_sample_top_k(c->d_io, (int)n, temperature, top_k, d_prev, (int)n_prev, repetition_penalty,
                                   c->d_rng_api, c->d_codes_api, c->d_status, c->stream));
    int status = 0;
    HIPCHK(c, hipMemcpyAsync(&status, c->d_status, sizeof(int), hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipMemcpyAsync(rng, c->d_rng_api, sizeof(uint64_t), hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipMemcpyAsync(out, c->d_codes_api, sizeof(uint32_t), hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    if (status == -7) return fail(c, QTTS_ERR_NAN, "NaN in sampler input");
    if (status == -1) return fail(c, QTTS_ERR_INVALID, "top_k must be at least 1 when temperature > 0");
    return QTTS_OK;
}

// The legacy predictor's cache: the talker step's paged layout for the
// predictor's layers, pages in identity order (no prefix sharing here).
static int ensure_legacy(qtts_ctx *c)
{
    if (c->lkv) return QTTS_OK;
    const PredictorDev &p = c->pm;
    const int n_pages = (int)(c->kv_cap / KV_PAGE);
    float *kv = nullptr, *buf = nullptr;
    RCHK(dev_alloc(c, c->model_allocs, &kv, (size_t)p.n_layers * n_pages * 2 * 8 * KV_PAGE * HEAD_DIM));
    RCHK(dev_alloc(c, c->model_allocs, &buf, (size_t)p.hidden + (size_t)p.n_groups * p.vocab));
    std::vector<int32_t> id(MAX_CHUNKS);
    for (int i = 0; i < MAX_CHUNKS; i++) id[i] = i;
    const int32_t *pt = nullptr;
    RCHK(upload_vec(c, c->model_allocs, id.data(), id.size(), &pt));
    c->lkv = kv;
    c->leg_buf = buf;
    c->lkv_ptab = const_cast<int32_t *>(pt);
    c->lkv_len = 0;
    return QTTS_OK;
}

extern "C" int qtts_predict_codes_reset(qtts_ctx *c)
{
    NEED_MODEL(c);
    c->lkv_len = 0;
    return QTTS_OK;
}

extern "C" int qtts_predict_codes(qtts_ctx *c, const float *talker_hidden, float *logits, int flags)
{
    NEED_MODEL(c);
    if (!talker_hidden || !logits) return QTTS_ERR_INVALID;
    hipSetDevice(c->device);
    RCHK(ensure_legacy(c));
    const TalkerDev &m = c->tm;
    const PredictorDev &p = c->pm;
    const int64_t pos = c->lkv_len;
    if (pos >= c->kv_cap) return fail(c, QTTS_ERR_CAPACITY, "legacy predictor cache full (%lld)", (long long)pos);
    if (pos >= p.rope_rows) return fail(c, QTTS_ERR_CAPACITY, "position beyond the predictor's RoPE table");
    // project_input (code_predictor.rs:135) into the step input row
    RCHK(ensure_io(c, m.hidden));
    RCHK(stage_in(c, talker_hidden, m.hidden, c->d_io, flags));
    HIPCHK(c, enqueue_gemv_store(p.proj, c->d_io, c->ws.x, p.proj_bias, c->ws.part_proj, c->stream));
    // the layers through the talker step's kernels: a view of the predictor
    TalkerDev v = m;
    v.n_layers = p.n_layers;
    v.hidden = p.hidden;
    v.inter = p.inter;
    v.vocab = p.vocab;
    v.layers = p.layers;
    v.final_norm = p.final_norm;
    v.rope_cos = p.rope_cos;
    v.rope_sin = p.rope_sin;
    v.rope_rows = p.rope_rows;
    v.kv = KvPaged{c->lkv, c->lkv_ptab, (int32_t)(c->kv_cap / KV_PAGE)};
    RCHK(arm_sync_err(c, c->st_gen));
    HIPCHK(c, enqueue_talker_row(v, c->ws, c->st_gen, pos, (int)pos, attn_pages(pos), c->stream));
    // final norm (code_predictor.rs:202) into `side`, then every head
    float *side = c->leg_buf, *out = c->leg_buf + p.hidden;
    v.codec_head = p.heads[0];
    HIPCHK(c, enqueue_final_norm(v, c->ws, side, c->stream));
    for (int g = 0; g < p.n_groups; g++) {
        v.codec_head = p.heads[g];
        HIPCHK(c, enqueue_codec_head(v, c->ws, side, out + (size_t)g * p.vocab, c->stream));
    }
    RCHK(stage_out(c, out, (int64_t)p.n_groups * p.vocab, logits, flags));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    RCHK(check_sync(c));   // a wait that ran out: the cache keeps its length
    c->lkv_len = pos + 1;
    return QTTS_OK;
}

extern "C" int qtts_prefill_tokens(qtts_ctx *c, const uint32_t *ids, const uint8_t *is_text, int64_t n,
                                   float *hidden_out, int flags)
{
    NEED_MODEL(c);
    if (!ids || !is_text || n < 1 || !hidden_out) return QTTS_ERR_INVALID;
    const TalkerDev &m = c->tm;
    std::vector<uint32_t> tid, cid;
    std::vector<int64_t> tpos, cpos;
    for (int64_t i = 0; i < n; i++) {
        if (is_text[i]) {
            if ((int64_t)ids[i] >= m.text_rows.rows) return fail(c, QTTS_ERR_INVALID, "text token %u out of range", ids[i]);
            tid.push_back(ids[i]);
            tpos.push_back(i);
        } else {
            if ((int64_t)ids[i] >= m.codec_rows.rows) return fail(c, QTTS_ERR_INVALID, "codec token %u out of range", ids[i]);
            cid.push_back(ids[i]);
            cpos.push_back(i);
        }
    }
    hipSetDevice(c->device);
    const int H = m.hidden;
    const int64_t nt = (int64_t)tid.size(), nc = (int64_t)cid.size();
    DevScratch buf;
    const size_t rows_f = (size_t)(n + nt + nc + 1) * H, scr_f = (size_t)nt * (m.text_hidden + m.text_fc1.n);
    HIPCHK(c, hipMalloc(&buf.p, (rows_f + scr_f) * sizeof(float) + (size_t)n * sizeof(uint32_t)));
    float *X = (float *)buf.p, *trows = X + (size_t)n * H, *crows = trows + (size_t)nt * H;
    float *hid = crows + (size_t)nc * H, *scratch = hid + H;
    uint32_t *d_tid = (uint32_t *)(scratch + scr_f), *d_cid = d_tid + nt;
    // embed_text_token / embed_codec_token per position (talker.rs:497-504)
    if (nt) {
        HIPCHK(c, hipMemcpyAsync(d_tid, tid.data(), nt * sizeof(uint32_t), hipMemcpyHostToDevice, c->stream));
        RCHK(text_rows(c, d_tid, (int)nt, trows, scratch));
    }
    if (nc) {
        HIPCHK(c, hipMemcpyAsync(d_cid, cid.data(), nc * sizeof(uint32_t), hipMemcpyHostToDevice, c->stream));
        HIPCHK(c, enqueue_gather_rows(m.codec_rows, d_cid, (int)nc, crows, H, c->stream));
    }
    for (int64_t i = 0; i < nt; i++)
        HIPCHK(c, hipMemcpyAsync(X + tpos[i] * H, trows + i * H, H * sizeof(float), hipMemcpyDeviceToDevice, c->stream));
    for (int64_t i = 0; i < nc; i++)
        HIPCHK(c, hipMemcpyAsync(X + cpos[i] * H, crows + i * H, H * sizeof(float), hipMemcpyDeviceToDevice, c->stream));
    // prefill_talker_raw over a fresh cache (talker.rs:506-507)
    RCHK(qtts_kv_reset(c));
    RCHK(qtts_talker_prefill(c, X, n, 0, hid, flags | QTTS_DEVICE_PTRS));
    RCHK(stage_out(c, hid, H, hidden_out, flags));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return QTTS_OK;
}

// ---------------------------------------------------------------------------
// frame loop
// ---------------------------------------------------------------------------

// The frame graph of the attention variant `pg` (pages per workgroup),
// captured on first use.
static int build_frame_graph(qtts_ctx *c, int pg)
{
    hipGraphExec_t &exec = c->frame_exec[pg - 1];
    if (exec) return QTTS_OK;
    hipGraph_t g = nullptr;
    HIPCHK(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    const hipError_t e = enqueue_frame(c->tm, c->pm, c->ws, c->st_gen, c->d_forced, pg, c->stream);
    const hipError_t e2 = hipStreamEndCapture(c->stream, &g);
    if (e != hipSuccess || e2 != hipSuccess) {
        if (g) hipGraphDestroy(g);
        return fail(c, QTTS_ERR_HIP, "frame capture failed: %s / %s", hipGetErrorString(e), hipGetErrorString(e2));
    }
    const hipError_t e3 = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e3 != hipSuccess) {
        exec = nullptr;
        return fail(c, QTTS_ERR_HIP, "graph instantiate: %s", hipGetErrorString(e3));
    }
    return QTTS_OK;
}

extern "C" int qtts_gen_begin(qtts_ctx *c, const float *logits, const float *hidden, int64_t position, uint64_t seed,
                              const qtts_sample_params *p)
{
    NEED_MODEL(c);
    if (!logits || !hidden || !p || position < 0) return QTTS_ERR_INVALID;
    HIPCHK(c, hipMemcpyAsync(c->ws.logits, logits, sizeof(float) * c->tm.vocab, hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(c->ws.hidden, hidden, sizeof(float) * c->tm.hidden, hipMemcpyHostToDevice, c->stream));
    DevState &s = *c->h_st;
    const int32_t kv = s.kv_len;
    const int32_t n_text = s.n_text;
    memset(&s, 0, sizeof s);
    s.kv_len = kv;
    s.n_text = n_text;
    s.position = position;
    s.rng = seed;
    s.temperature = p->temperature;
    s.top_k = p->top_k;
    s.top_p = p->top_p;
    s.rep_penalty = p->repetition_penalty;
    s.eos_id = p->codec_eos_id;
    s.eos_enabled = p->eos_enabled;
    s.onset_frames = p->onset_frames;
    s.onset_temperature = p->onset_temperature;
    RCHK(write_state(c));
    c->gen_started = true;
    return QTTS_OK;
}

extern "C" int qtts_gen_set_text(qtts_ctx *c, const float *text, int64_t n_text, const float *pad)
{
    NEED_MODEL(c);
    if (n_text < 0 || (n_text > 0 && !text) || !pad) return QTTS_ERR_INVALID;
    const int H = c->tm.hidden;
    if (n_text > c->text_cap) {
        drop_graph(c);
        float *nt = nullptr;
        HIPCHK(c, hipMalloc(&nt, (size_t)n_text * H * sizeof(float)));
        for (auto &p : c->ws_allocs)
            if (p == c->ws.text) { hipFree(p); p = nt; }
        c->ws.text = nt;
        c->text_cap = n_text;
    }
    if (n_text) HIPCHK(c, hipMemcpyAsync(c->ws.text, text, (size_t)n_text * H * sizeof(float), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(c->ws.pad, pad, (size_t)H * sizeof(float), hipMemcpyHostToDevice, c->stream));
    c->h_st->n_text = (int32_t)n_text;
    HIPCHK(c, hipMemcpyAsync(&c->st_gen->n_text, &c->h_st->n_text, sizeof(int32_t), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return QTTS_OK;
}

// Run frames in batches of up to RING_FRAMES graph launches per host sync.
// QTTS_NO_GRAPH=1 enqueues each frame's kernels directly instead of
// replaying the captured graph (same kernels; used under profilers).
static bool use_graph()
{
    const char *v = getenv("QTTS_NO_GRAPH");
    return !(v && *v && *v != '0');
}

static int run_frames(qtts_ctx *c, int64_t n, uint32_t *pred_out, int64_t *done, int32_t *eos, bool forced)
{
    const bool graph = use_graph();
    int64_t emitted = 0;
    *eos = 0;
    while (emitted < n) {
        // direct launches (QTTS_NO_GRAPH=1) synchronise after every frame
        // (a profiled process once crashed on the host queueing 64 frames of
        // direct launches, ~28k dispatches, between synchronisations; no
        // cause was found in this code)
        const int64_t batch = std::min<int64_t>(n - emitted, graph ? RING_FRAMES : 1);
        if (c->h_st->kv_len + batch > c->kv_cap)
            return fail(c, QTTS_ERR_CAPACITY, "talker KV cache full at %d positions", c->h_st->kv_len);
        if (c->h_st->position + batch > c->tm.rope_rows)
            return fail(c, QTTS_ERR_CAPACITY, "position beyond the RoPE table");
        c->h_st->ring_base = c->h_st->frame_idx;
        HIPCHK(c, hipMemcpyAsync(&c->st_gen->ring_base, &c->h_st->ring_base, sizeof(int32_t), hipMemcpyHostToDevice,
                                 c->stream));
        // frame f's talker step attends kv_len + f + 1 positions (frames after
        // a stop are no-ops whichever variant runs them); the batch's graphs
        // are captured before its first launch
        if (graph) {
            RCHK(build_frame_graph(c, step_pages(c, c->h_st->kv_len)));
            RCHK(build_frame_graph(c, step_pages(c, c->h_st->kv_len + batch - 1)));
        }
        RCHK(arm_sync_err(c, c->st_gen));
        for (int64_t f = 0; f < batch; f++) {
            const int pg = step_pages(c, c->h_st->kv_len + f);
            if (graph) {
                HIPCHK(c, hipGraphLaunch(c->frame_exec[pg - 1], c->stream));
            } else {
                HIPCHK(c, enqueue_frame(c->tm, c->pm, c->ws, c->st_gen, c->d_forced, pg, c->stream));
            }
        }
        HIPCHK(c, hipMemcpyAsync(c->h_ring, c->ws.ring_pred, sizeof(uint32_t) * batch * 16, hipMemcpyDeviceToHost,
                                 c->stream));
        const int32_t base = c->h_st->ring_base;
        HIPCHK(c, hipMemcpyAsync(c->h_st, c->st_gen, sizeof(DevState), hipMemcpyDeviceToHost, c->stream));
        HIPCHK(c, hipStreamSynchronize(c->stream));
        const int64_t got = c->h_st->frame_idx - base;
        if (got < 0 || got > batch) return fail(c, QTTS_ERR_STATE, "frame counter out of step");
        if (pred_out) memcpy(pred_out + emitted * 16, c->h_ring, sizeof(uint32_t) * got * 16);
        emitted += got;
        if (c->h_st->sync_err) {
            *done = emitted;
            RCHK(check_sync(c));
        }
        if (c->h_st->nan_flag) {
            *done = emitted;
            return fail(c, QTTS_ERR_NAN, "NaN logits during generation");
        }
        if (!forced && c->h_st->stop) {
            *eos = c->h_st->eos;
            break;
        }
        if (got < batch) break;
    }
    *done = emitted;
    return QTTS_OK;
}

extern "C" int qtts_gen_frames(qtts_ctx *c, int64_t max_frames, uint32_t *codes_out, int64_t *frames_done,
                               int32_t *eos)
{
    NEED_MODEL(c);
    if (max_frames < 0 || !frames_done || !eos) return QTTS_ERR_INVALID;
    if (!c->gen_started) return fail(c, QTTS_ERR_STATE, "qtts_gen_begin first");
    *frames_done = 0;
    *eos = c->h_st->eos;
    if (c->h_st->stop) return QTTS_OK;
    return run_frames(c, max_frames, codes_out, frames_done, eos, false);
}

extern "C" int qtts_gen_frames_forced(qtts_ctx *c, int64_t n_frames, const uint32_t *forced, uint32_t *pred_out)
{
    NEED_MODEL(c);
    if (n_frames < 0 || (n_frames > 0 && !forced)) return QTTS_ERR_INVALID;
    if (!c->gen_started) return fail(c, QTTS_ERR_STATE, "qtts_gen_begin first");
    // forced codes index embedding tables on the device: validate them here
    for (int64_t f = 0; f < n_frames; f++) {
        if ((int64_t)forced[f * 16] >= c->tm.codec_rows.rows)
            return fail(c, QTTS_ERR_INVALID, "forced code 0 of frame %lld out of range", (long long)f);
        for (int g = 1; g <= c->pm.n_groups; g++)
            if ((int64_t)forced[f * 16 + g] >= c->pm.emb_rows.rows)
                return fail(c, QTTS_ERR_INVALID, "forced code %d of frame %lld out of range", g, (long long)f);
    }
    if (n_frames > c->forced_cap) {
        drop_graph(c);
        if (c->d_forced) hipFree(c->d_forced);
        c->d_forced = nullptr;
        HIPCHK(c, hipMalloc(&c->d_forced, sizeof(uint32_t) * 16 * n_frames));
        c->forced_cap = n_frames;
    }
    if (!c->d_forced) {
        HIPCHK(c, hipMalloc(&c->d_forced, sizeof(uint32_t) * 16));
        c->forced_cap = 1;
    }
    if (n_frames) HIPCHK(c, hipMemcpyAsync(c->d_forced, forced, sizeof(uint32_t) * 16 * n_frames, hipMemcpyHostToDevice, c->stream));
    c->h_st->force = 1;
    c->h_st->forced_base = c->h_st->frame_idx;
    HIPCHK(c, hipMemcpyAsync(&c->st_gen->force, &c->h_st->force, sizeof(int32_t), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(&c->st_gen->forced_base, &c->h_st->forced_base, sizeof(int32_t), hipMemcpyHostToDevice,
                             c->stream));
    int64_t done = 0;
    int32_t eos = 0;
    const int r = run_frames(c, n_frames, pred_out, &done, &eos, true);
    c->h_st->force = 0;
    HIPCHK(c, hipMemcpyAsync(&c->st_gen->force, &c->h_st->force, sizeof(int32_t), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    if (r == QTTS_OK && done != n_frames) return fail(c, QTTS_ERR_STATE, "forced run stopped early");
    return r;
}

extern "C" int qtts_gen_state(qtts_ctx *c, float *logits, float *hidden, int64_t *position, uint64_t *rng)
{
    NEED_MODEL(c);
    RCHK(read_state(c));
    if (logits) HIPCHK(c, hipMemcpy(logits, c->ws.logits, sizeof(float) * c->tm.vocab, hipMemcpyDeviceToHost));
    if (hidden) HIPCHK(c, hipMemcpy(hidden, c->ws.hidden, sizeof(float) * c->tm.hidden, hipMemcpyDeviceToHost));
    if (position) *position = c->h_st->position;
    if (rng) *rng = c->h_st->rng;
    return QTTS_OK;
}

// Test hook: the next call that runs fused launches (talker step or row
// prefill, frame batch, predictor chain, legacy predictor step) starts from
// the state a bounded wait leaves when it runs out, so its fused launches
// take no wait at all (each workgroup reads the flag at its start and skips
// its polls: every kernel exits normally) and it reports QTTS_ERR_HIP once.
extern "C" int qtts_debug_force_sync_err(qtts_ctx *c)
{
    NEED_MODEL(c);
    c->force_sync_err = true;
    return QTTS_OK;
}

// ---------------------------------------------------------------------------
// measurement
// ---------------------------------------------------------------------------

// Average launch duration: one event pair around `iters` back-to-back
// launches on the context stream (a warm-up launch first), so the figure is
// the kernel plus the dispatch gap, without per-event overhead.
//
// In graph mode (qtts_time_graph) the `iters` launches are captured once into
// a graph, which is replayed once to warm up and then GRAPH_REPLAYS times
// between the events: the launches then run as the frame loop runs its
// kernels, from a replayed graph.  Launchers that replay a graph themselves
// pass allow_graph = false.
static int time_launches(qtts_ctx *c, int32_t iters, const std::function<hipError_t(int)> &launch, double *avg_us,
                         bool allow_graph = true)
{
    constexpr int GRAPH_REPLAYS = 4;
    const bool graph = allow_graph && c->time_graph;
    hipEvent_t e0, e1;
    HIPCHK(c, hipEventCreate(&e0));
    HIPCHK(c, hipEventCreate(&e1));
    int rc = QTTS_OK;
    hipError_t err = hipSuccess;
    hipGraphExec_t ge = nullptr;
    if (graph) {
        hipGraph_t g = nullptr;
        err = hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal);
        if (err == hipSuccess) {
            for (int i = 0; i < iters && err == hipSuccess; i++) err = launch(i);
            const hipError_t e2 = hipStreamEndCapture(c->stream, &g);
            if (err == hipSuccess) err = e2;
        }
        if (err == hipSuccess) err = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
        if (g) hipGraphDestroy(g);
        if (err == hipSuccess) err = hipGraphLaunch(ge, c->stream);
        if (err == hipSuccess) err = hipEventRecord(e0, c->stream);
        for (int r = 0; r < GRAPH_REPLAYS && err == hipSuccess; r++) err = hipGraphLaunch(ge, c->stream);
    } else {
        err = launch(0);
        if (err == hipSuccess) err = hipEventRecord(e0, c->stream);
        for (int i = 0; i < iters && err == hipSuccess; i++) err = launch(i);
    }
    if (err == hipSuccess) err = hipEventRecord(e1, c->stream);
    if (err == hipSuccess) err = hipEventSynchronize(e1);
    float ms = 0.0f;
    if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
    if (err != hipSuccess) rc = fail(c, QTTS_ERR_HIP, "kernel timing: %s", hipGetErrorString(err));
    if (ge) hipGraphExecDestroy(ge);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    *avg_us = ms * 1000.0 / ((double)iters * (graph ? GRAPH_REPLAYS : 1));
    return rc;
}

extern "C" int qtts_time_graph(qtts_ctx *c, int32_t on)
{
    if (!c || (on != 0 && on != 1)) return QTTS_ERR_INVALID;
    c->time_graph = on != 0;
    return QTTS_OK;
}

extern "C" int qtts_time_kernel(qtts_ctx *c, int32_t kind, int32_t iters, double *avg_us, double *bytes)
{
    if (!c || iters < 1 || !avg_us || !bytes) return QTTS_ERR_INVALID;
    if (kind == 2) {
        // plain float4 copy of 256 MiB (read + write), the HBM calibration
        // point for byte counters and for achievable bandwidth
        hipSetDevice(c->device);
        const int64_t n = 64ll << 20;
        if (!c->d_copy) {
            HIPCHK(c, hipMalloc(&c->d_copy, 2 * n * sizeof(float)));
            HIPCHK(c, hipMemsetAsync(c->d_copy, 0, 2 * n * sizeof(float), c->stream));
            c->copy_floats = n;
        }
        *bytes = 2.0 * n * sizeof(float);
        return time_launches(c, iters, [&](int) { return enqueue_copy(c->d_copy, c->d_copy + n, n, c->stream); },
                             avg_us);
    }
    if (kind == 7) {
        // streaming read of the Q4 GEMV's bytes (k=2048 -> n=6144: 7,110,656 B)
        // in one launch, cycling 64 buffers (455 MB, beyond the 256 MB
        // last-level cache): the attainable time of a launch that moves the
        // GEMV's bytes and nothing else
        constexpr int64_t READ_BYTES = 7110656, READ_POOL = 64;
        hipSetDevice(c->device);
        if (!c->d_read) {
            HIPCHK(c, hipMalloc(&c->d_read, READ_BYTES * READ_POOL));
            HIPCHK(c, hipMalloc(&c->d_sink, sizeof(uint32_t)));
            HIPCHK(c, hipMemsetAsync(c->d_read, 0, READ_BYTES * READ_POOL, c->stream));
        }
        *bytes = (double)READ_BYTES;
        // zero words fold to 0, never to 1: the sink is never written
        return time_launches(c, iters, [&](int i) {
            return enqueue_read(c->d_read + (i % READ_POOL) * (READ_BYTES / 4), READ_BYTES / 4, 1u, c->d_sink, c->stream);
        }, avg_us);
    }
    NEED_MODEL(c);
    const TalkerDev &m = c->tm;
    if (kind == 0) {
        const LayerDev &L = m.layers[0];
        *bytes = (double)L.gate_up.k * (L.gate_up.n) * 0.5625 + 4.0 * L.gate_up.k + 4.0 * L.gate_up.n;
        return time_launches(c, iters, [&](int i) { return enqueue_gateup_timing(m, c->ws, i % m.n_layers, c->stream); },
                             avg_us);
    }
    if (kind == 1) {
        // one decode step's attention at the current length: appends at the
        // free slot kv_len (cached positions untouched), attends kv_len + 1
        const int slot = c->h_st->kv_len;
        if (slot + 1 > c->kv_cap) return fail(c, QTTS_ERR_CAPACITY, "no free KV slot to time attention");
        const int64_t pos = std::min<int64_t>(c->h_st->position, m.rope_rows - 1);
        *bytes = (double)(slot + 1) * 8 * HEAD_DIM * 4 * 2 + 16.0 * HEAD_DIM * 4 * 3;
        // pages per work item: the step's choice, or QTTS_ATTN_PAGES (1, 2)
        const char *pe = getenv("QTTS_ATTN_PAGES");
        const int pg = (pe && (atoi(pe) == 1 || atoi(pe) == 2)) ? atoi(pe) : attn_pages(slot);
        return time_launches(c, iters,
                             [&](int i) {
                                 return enqueue_attn_timing(m, c->ws, i % m.n_layers, slot, pos, c->st_api, pg,
                                                            c->stream);
                             },
                             avg_us);
    }
    if (kind == 5 || kind == 6) {
        // the frame's two halves, each captured alone and replayed back to
        // back: 5 = sampler + predictor chain + combine (the predictor's
        // weights stay warm in the last-level cache between replays), 6 =
        // the talker step (KV appended from the current length).  The
        // generation state is restored afterwards.
        const PredictorDev &p = c->pm;
        const int64_t n = (int64_t)iters + 1;
        if (kind == 6 && (c->h_st->kv_len + n > c->kv_cap || c->h_st->position + n > m.rope_rows))
            return fail(c, QTTS_ERR_CAPACITY, "no room in the KV cache to time %d talker steps", iters);
        hipSetDevice(c->device);
        // the generation state: counters, the next frame's logits and hidden
        DevState saved;
        std::vector<float> lg(m.vocab), hd(m.hidden);
        HIPCHK(c, hipMemcpyAsync(&saved, c->st_gen, sizeof saved, hipMemcpyDeviceToHost, c->stream));
        HIPCHK(c, hipMemcpyAsync(lg.data(), c->ws.logits, lg.size() * sizeof(float), hipMemcpyDeviceToHost, c->stream));
        HIPCHK(c, hipMemcpyAsync(hd.data(), c->ws.hidden, hd.size() * sizeof(float), hipMemcpyDeviceToHost, c->stream));
        HIPCHK(c, hipStreamSynchronize(c->stream));
        double w = 0.0;
        if (kind == 5) {
            for (int l = 0; l < p.n_layers; l++) {
                const LayerDev &L = p.layers[l];
                w += (double)(L.qkv.k * L.qkv.n + L.o.k * L.o.n + L.gate_up.k * L.gate_up.n + L.down.k * L.down.n);
            }
            for (int g = 0; g < p.n_groups; g++) w += (double)p.heads[g].k * p.heads[g].n;
            w += (double)p.proj.k * p.proj.n;
        } else {
            for (int l = 0; l < m.n_layers; l++) {
                const LayerDev &L = m.layers[l];
                w += (double)(L.qkv.k * L.qkv.n + L.o.k * L.o.n + L.gate_up.k * L.gate_up.n + L.down.k * L.down.n);
            }
            w += (double)m.codec_head.k * m.codec_head.n;
        }
        *bytes = w * 0.5625;
        hipGraph_t g = nullptr;
        hipGraphExec_t ge = nullptr;
        HIPCHK(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
        const hipError_t e = kind == 5 ? enqueue_frame_codes(m, p, c->ws, c->st_gen, c->d_forced, c->stream)
                                       : enqueue_talker_step(m, c->ws, c->st_gen, 0, step_pages(c, c->h_st->kv_len),
                                                             c->stream);
        const hipError_t e2 = hipStreamEndCapture(c->stream, &g);
        if (e != hipSuccess || e2 != hipSuccess) {
            if (g) hipGraphDestroy(g);
            return fail(c, QTTS_ERR_HIP, "capture failed: %s / %s", hipGetErrorString(e), hipGetErrorString(e2));
        }
        const hipError_t e3 = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
        hipGraphDestroy(g);
        if (e3 != hipSuccess) return fail(c, QTTS_ERR_HIP, "graph instantiate: %s", hipGetErrorString(e3));
        const int rc = time_launches(c, iters, [&](int) { return hipGraphLaunch(ge, c->stream); }, avg_us, false);
        hipGraphExecDestroy(ge);
        HIPCHK(c, hipMemcpyAsync(c->st_gen, &saved, sizeof saved, hipMemcpyHostToDevice, c->stream));
        HIPCHK(c, hipMemcpyAsync(c->ws.logits, lg.data(), lg.size() * sizeof(float), hipMemcpyHostToDevice, c->stream));
        HIPCHK(c, hipMemcpyAsync(c->ws.hidden, hd.data(), hd.size() * sizeof(float), hipMemcpyHostToDevice, c->stream));
        HIPCHK(c, hipStreamSynchronize(c->stream));
        return rc;
    }
    if (kind == 8 || kind == 9) {
        // the fused launches as the frame runs them, cycling the layers: 8 =
        // one talker layer (q|k|v + attention, o-proj, gate|up + down) at the
        // current length, appending at the free slot kv_len; 9 = one
        // predictor layer step (q|k|v + attention + o-proj, gate|up + down),
        // one row at position 8.  The waits read the API state (cleared
        // first); one that ran out is reported.
        DevState z{};
        HIPCHK(c, hipMemcpyAsync(c->st_api, &z, sizeof z, hipMemcpyHostToDevice, c->stream));
        int rc;
        if (kind == 8) {
            const int slot = c->h_st->kv_len;
            if (slot + 1 > c->kv_cap) return fail(c, QTTS_ERR_CAPACITY, "no free KV slot to time the talker layer");
            if (!talker_fused_attn(m)) return fail(c, QTTS_ERR_UNSUPPORTED, "the talker's q|k|v tile is not the fused one");
            const int64_t pos = std::min<int64_t>(c->h_st->position, m.rope_rows - 1);
            const LayerDev &L = m.layers[0];
            *bytes = (double)(L.qkv.k * L.qkv.n + L.o.k * L.o.n + L.gate_up.k * L.gate_up.n + L.down.k * L.down.n) *
                         0.5625 + (double)(slot + 2) * 8 * HEAD_DIM * 4 * 2;
            rc = time_launches(c, iters, [&](int i) {
                return enqueue_talker_layer_timing(m, c->ws, i % m.n_layers, slot, pos, c->st_api, c->stream);
            }, avg_us);
        } else {
            const PredictorDev &p = c->pm;
            const LayerDev &L = p.layers[0];
            *bytes = (double)(L.qkv.k * L.qkv.n + L.o.k * L.o.n + L.gate_up.k * L.gate_up.n + L.down.k * L.down.n) *
                         0.5625 + 9.0 * 8 * HEAD_DIM * 4 * 2;
            rc = time_launches(c, iters, [&](int i) {
                return enqueue_pred_layer_fused_timing(p, c->ws, i % p.n_layers, 8, c->st_api, c->stream);
            }, avg_us);
        }
        if (rc != QTTS_OK) return rc;
        DevState back{};
        HIPCHK(c, hipMemcpyAsync(&back, c->st_api, sizeof back, hipMemcpyDeviceToHost, c->stream));
        HIPCHK(c, hipStreamSynchronize(c->stream));
        if (back.sync_err) return fail(c, QTTS_ERR_HIP, "a cross-workgroup wait timed out while timing");
        return QTTS_OK;
    }
    if (kind == 3 || kind == 4) {
        // predictor, one row at position 8 (a mid-chain step), cycling the layers
        const PredictorDev &p = c->pm;
        const LayerDev &L = p.layers[0];
        const double w = kind == 3 ? (double)L.o.k * L.o.n * 0.5625
                                   : (double)(L.qkv.k * L.qkv.n + L.o.k * L.o.n + L.gate_up.k * L.gate_up.n +
                                              L.down.k * L.down.n) * 0.5625;
        *bytes = w + 9.0 * 8 * HEAD_DIM * 4 * 2;
        if (kind == 3)
            return time_launches(c, iters, [&](int i) { return enqueue_pred_attn_o_timing(p, c->ws, i % p.n_layers, 8, c->stream); },
                                 avg_us);
        return time_launches(c, iters, [&](int i) { return enqueue_pred_layer_timing(p, c->ws, i % p.n_layers, 8, c->stream); },
                             avg_us);
    }
    return QTTS_ERR_INVALID;
}

extern "C" int qtts_time_prefill(qtts_ctx *c, int64_t rows, int32_t what, int32_t iters, double *avg_us,
                                 double *flops)
{
    if (!c || iters < 1 || !avg_us || !flops || rows < 1 || (what != 0 && what != 1)) return QTTS_ERR_INVALID;
    NEED_MODEL(c);
    const TalkerDev &m = c->tm;
    if (!prefill_supported(m)) return fail(c, QTTS_ERR_UNSUPPORTED, "model shapes outside the matrix-core prefill");
    if (rows > PREFILL_MAX_ROWS) return fail(c, QTTS_ERR_CAPACITY, "at most %d rows per prefill chunk", PREFILL_MAX_ROWS);
    if (rows > c->kv_cap || rows > m.rope_rows) return fail(c, QTTS_ERR_CAPACITY, "rows beyond the KV cache");
    hipSetDevice(c->device);
    RCHK(ensure_prefill(c, (int)rows));
    RCHK(seq_unshare_from(c, 0));
    c->gen_started = false;
    const int M = (int)rows, H = m.hidden;
    if (what == 0) {
        HIPCHK(c, enqueue_fill_rows(c->pf.x, (int64_t)M * H, 7u, c->stream));
        HIPCHK(c, enqueue_row_inv(c->pf.x, H, M, H, c->pf.inv, c->stream));
        *flops = 2.0 * M * H * 2.0 * m.inter;
        return time_launches(c, iters, [&](int i) { return enqueue_gemm_gateup(m, c->pf, i % m.n_layers, M, c->stream); },
                             avg_us);
    }
    double f = 0.0;
    for (int l = 0; l < m.n_layers; l++) {
        const LayerDev &L = m.layers[l];
        f += 2.0 * M * ((double)L.qkv.k * 32 * HEAD_DIM + (double)L.o.k * H + (double)H * 2 * m.inter +
                        (double)m.inter * H);
        f += 4.0 * 16 * HEAD_DIM * ((double)M * (M + 1) / 2);   // QK and PV of the causal attention
    }
    *flops = f;
    // synthetic input rows, restaged into pf.x before each launch
    RCHK(ensure_io(c, (int64_t)M * H));
    float *src = c->d_io;
    HIPCHK(c, enqueue_fill_rows(src, (int64_t)M * H, 11u, c->stream));
    const int rc = time_launches(c, iters, [&](int) {
        hipError_t e = hipMemcpyAsync(c->pf.x, src, (size_t)M * H * sizeof(float), hipMemcpyDeviceToDevice, c->stream);
        if (e != hipSuccess) return e;
        return enqueue_talker_prefill(m, c->pf, M, 0, c->ws.hid_work, c->stream);
    }, avg_us, false);
    c->h_st->kv_len = 0;
    c->h_st->position = 0;
    HIPCHK(c, hipMemcpyAsync(c->st_gen, c->h_st, sizeof(DevState), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return rc;
}

extern "C" int qtts_time_decode(qtts_ctx *c, int64_t n_frames, int32_t iters, double *avg_us, double *flops)
{
    if (!c || iters < 1 || !avg_us || !flops || n_frames < 1) return QTTS_ERR_INVALID;
    if (!c->has_decoder) return fail(c, QTTS_ERR_STATE, "no speech decoder uploaded");
    if (n_frames > (1 << 16)) return fail(c, QTTS_ERR_CAPACITY, "too many frames");
    hipSetDevice(c->device);
    const DecoderDev &d = c->dec;
    const int T = (int)n_frames, ncb = d.n_rest + 1;
    RCHK(ensure_dec_ws(c, T));
    c->dws.f32 = d.weights_f32;
    // synthetic codes from a fixed LCG, uniform over the codebook
    std::vector<uint32_t> codes((size_t)ncb * T);
    uint64_t x = 0x9E3779B97F4A7C15ull;
    for (auto &v : codes) {
        x = x * 6364136223846793005ull + 1442695040888963407ull;
        v = (uint32_t)((x >> 33) % (uint64_t)d.codebook_size);
    }
    HIPCHK(c, hipMemcpyAsync(c->dws.codes, codes.data(), codes.size() * sizeof(uint32_t), hipMemcpyHostToDevice,
                             c->stream));
    int64_t factor = 1;
    for (int u = 0; u < d.n_up; u++) factor *= d.up[u].conv_t.stride;
    for (int b = 0; b < d.n_voc; b++) factor *= d.voc[b].up.stride;
    RCHK(ensure_io(c, (int64_t)T * factor));
    *flops = decode_flops(d, T);
    return time_launches(c, iters, [&](int) { return enqueue_decode(d, c->dws, c->dws.codes, T, 0, c->d_io, c->stream); },
                         avg_us, false);
}

extern "C" int qtts_time_gemv(qtts_ctx *c, const qtts_w *const *ws, int32_t n_w, int32_t iters, double *avg_us,
                              double *bytes)
{
    if (!c || !ws || n_w < 1 || iters < 1 || !avg_us || !bytes) return QTTS_ERR_INVALID;
    hipSetDevice(c->device);
    const Q4Tiled &t0 = ws[0]->t;
    *bytes = (double)t0.k * (t0.n / 32) * 32 * 0.5625 + 4.0 * t0.k + 4.0 * t0.n;
    return time_launches(
        c, iters,
        [&](int i) {
            const qtts_w *w = ws[i % n_w];
            return enqueue_gemv_plain(w->t, w->x, 1, w->t.k, w->part, c->stream);
        },
        avg_us);
}

// ---------------------------------------------------------------------------
// device memory of the uploaded model
// ---------------------------------------------------------------------------

static int64_t tiled_bytes(const Q4Tiled &w) { return (int64_t)w.S * w.CT * w.tile_bytes; }
static int64_t rows_bytes(const Q4Rows &e) { return (int64_t)e.rows * e.G * (16 + 2); }

extern "C" int qtts_device_bytes(qtts_ctx *c, qtts_mem_report *out)
{
    NEED_MODEL(c);
    if (!out) return QTTS_ERR_INVALID;
    memset(out, 0, sizeof *out);
    const TalkerDev &m = c->tm;
    const PredictorDev &p = c->pm;
    for (int l = 0; l < m.n_layers; l++) {
        const LayerDev &L = m.layers[l];
        out->talker_q4 += tiled_bytes(L.qkv) + tiled_bytes(L.o) + tiled_bytes(L.gate_up) + tiled_bytes(L.down);
    }
    out->talker_q4 += tiled_bytes(m.codec_head) + tiled_bytes(m.text_fc1) + tiled_bytes(m.text_fc2);
    for (int l = 0; l < p.n_layers; l++) {
        const LayerDev &L = p.layers[l];
        out->predictor_q4 += tiled_bytes(L.qkv) + tiled_bytes(L.o) + tiled_bytes(L.gate_up) + tiled_bytes(L.down);
    }
    for (int g = 0; g < p.n_groups; g++) out->predictor_q4 += tiled_bytes(p.heads[g]);
    out->predictor_q4 += tiled_bytes(p.proj);
    const int64_t ntab = p.n_groups - 1, rows = p.emb_rows.rows;
    if (p.proj_rows) out->predictor_row_tables = ntab * rows * p.hidden * (int64_t)sizeof(float);
    if (p.qkv_rows) out->predictor_qkv_tables = ntab * rows * p.layers[0].qkv.npad * (int64_t)sizeof(float);
    out->embedding_rows = rows_bytes(m.codec_rows) + rows_bytes(m.text_rows) + p.n_groups * rows_bytes(p.emb_rows);
    out->kv_pool = (int64_t)m.n_layers * m.kv.n_phys * 2 * 8 * KV_PAGE * HEAD_DIM * (int64_t)sizeof(float);
    size_t fr = 0, tot = 0;
    HIPCHK(c, hipMemGetInfo(&fr, &tot));
    out->device_used = (int64_t)(tot - fr);
    return QTTS_OK;
}
