// qtts_kernels.hip — hand-written gfx950 kernels for the QORA-TTS decode
// path, and the host functions that enqueue one talker step, one predictor
// chain and one frame on a stream.
//
// Reference functions restated (src/ of the reference crate):
//   Q4 GEMV            gemv.rs:249-346      (k_gemv; split-K partials)
//   RMSNorm + residual gemv.rs:445-454, talker.rs:334-349 (ProResidRms)
//   QK-norm + RoPE     talker.rs:286-297, rope.rs:79-92 (k_talker_attn prologue)
//   KV append          talker.rs:299-302    (k_talker_attn, paged)
//   decode attention   talker.rs:304-331    (k_talker_attn + the o-proj's ProAttnCombine)
//   SwiGLU             talker.rs:338-349    (EpiSwiglu / ProSwiglu)
//   predictor layers   code_predictor.rs:345-513 (k_pred_attn et al.)
//   argmax             code_predictor.rs:335-341 (EpiArgmax candidates, k_argmax)
//   sample_token       generate_new.rs:771-862   (k_sampler)
//   frame fusion       generate_new.rs:638-654   (k_combine)
//
// A frame is 264 dependent launches replayed from a HIP graph.  Launches
// hand partial sums (one row per k-slice) to the next launch, whose
// prologue reduces them in slice order.  Inside the fused launches
// (k_talker_qkv_attn, k_pred_qkv_attn_o, k_mlp, k_mlp1) the first stage's
// workgroups hand their column sums to the second stage's as (epoch, value)
// words, stored and polled with system-scope relaxed atomics and bounded
// waits; no kernel uses a device-wide fence or a read-modify-write atomic
// on global memory.
#include "qtts_device.h"
#include "qtts_kernels.h"
#include "qtts_devutil.h"

#include <algorithm>
#include <math.h>

#include <type_traits>

namespace qtts {




typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// AND kept opaque to the optimiser: with a visible mask the compiler splits
// the masked word into per-field extracts (one v_bfe_u32 each), while an
// opaque masked word is consumed whole (its bytes by v_cvt_f32_ubyte{0..3},
// its 16-bit halves by v_fma_mix_f32's half selects).
__device__ __forceinline__ uint32_t and_opaque(uint32_t w, uint32_t m)
{
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "s"(m), "v"(w));
    return r;
}

// Bound on the polls of a workgroup waiting for (epoch, value) words from
// another workgroup of the same launch: past it (milliseconds, against the
// few microseconds a producer takes) the workgroup records sync_err in the
// device state and finishes with whatever it read; once sync_err is set,
// later launches do not wait at all.
constexpr int LL_SPIN_MAX = 1 << 14;

// A second-stage workgroup of some fused launches holds back its own loads
// for a fixed time so that the first stage's weight stream, which its
// inputs depend on, is served first: HBM serves requests roughly in arrival
// order, and weights a waiting tile fetched at once would only delay the
// words it waits for.  Times are ticks of the 100 MHz real-time counter,
// tuned on frames/s (MI355X, KV 64 and 2048): the talker's down tiles 2.5 us
// (1.5-4 us swept), the predictor's o-proj tiles 1.0 us (0.2-2.2 us swept),
// the predictor's down tiles behind one-group gate|up tiles 0.8 us (0.3-3 us
// swept; behind paired gate|up tiles a hold did not help).  Holding the
// talker's attention items back did not help either (their page reads are
// the larger stream).
constexpr uint32_t HOLD_TALKER_DOWN = 250;
constexpr uint32_t HOLD_PRED_O = 100;
constexpr uint32_t HOLD_PRED_DOWN = 80;

// Waits `ticks` of the real-time counter (bounded by the clock).
__device__ __forceinline__ void stage_hold(uint32_t ticks)
{
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (__builtin_amdgcn_s_memrealtime() - t0 < ticks) __builtin_amdgcn_s_sleep(2);
}

// ---------------------------------------------------------------------------
// wave-wide sum (deterministic butterfly order)
// ---------------------------------------------------------------------------

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}

template <int CTRL>
__device__ __forceinline__ int dpp_mov_i(int v)
{
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}

// (v, i) pairs: the larger value wins, equal values go to the larger index
// (the last maximum, as Iterator::max_by in code_predictor.rs:335-341).
__device__ __forceinline__ void argmax_merge(float &v, int &i, float ov, int oi)
{
    if (ov > v || (ov == v && oi > i)) { v = ov; i = oi; }
}

template <int CTRL>
__device__ __forceinline__ void argmax_dpp_step(float &v, int &i)
{
    const float ov = dpp_mov<CTRL>(v);
    const int oi = dpp_mov_i<CTRL>(i);
    argmax_merge(v, i, ov, oi);
}

// Wave-wide argmax of one (value, index) per lane; uniform result.
__device__ __forceinline__ void wave_argmax_last(float &v, int &i)
{
    argmax_dpp_step<0xB1>(v, i);
    argmax_dpp_step<0x4E>(v, i);
    argmax_dpp_step<0x141>(v, i);
    argmax_dpp_step<0x140>(v, i);
    float bv = lane_value(v, 0);
    int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
    for (int r = 16; r < 64; r += 16) argmax_merge(bv, bi, lane_value(v, r), __builtin_amdgcn_readlane(i, r));
    v = bv;
    i = bi;
}

// Code chosen from the per-tile argmax candidates of one lm head (one per
// lane, ncand <= 64): the last maximum; any NaN tile -> code 0 and nan.
__device__ __forceinline__ uint32_t cand_argmax(const float2 *cand, int ncand, bool &nan)
{
    const int lane = threadIdx.x & 63;
    const float2 cv = cand[min(lane, ncand - 1)];
    float v = lane < ncand ? cv.x : -INFINITY;
    int i = lane < ncand ? __builtin_bit_cast(int, cv.y) : -2;
    nan = __ballot(i == -1) != 0;
    wave_argmax_last(v, i);
    return (nan || i < 0) ? 0u : (uint32_t)i;
}

// ---------------------------------------------------------------------------
// GEMV prologues.  A prologue fills xs[b*KC + i] with input row b, rows
// k0 + i, in two stages:
//   fetch<T, KC>(f, k0, ctile): every global load the prologue needs, into
//     the registers of f, issued before the tile's weight loads and without
//     a barrier.  Vector loads retire in issue order, so a load issued after
//     the weights could only be waited on by also waiting for the weights.
//   load<T, KC>(f, xs, k0, ctile): the arithmetic, LDS writes and barriers;
//     its waits cover the prologue's loads while the weights stay in flight.
// Loads use clamped (always valid) addresses and are masked afterwards, so no
// load sits behind a branch.
// ---------------------------------------------------------------------------



template <int NB>
struct ProPlain {
    const float *x;
    int ld, k;
    template <int T, int KC>
    struct Fetch {
        f32x4 v[(NB * KC / 4 + T - 1) / T];
    };
    template <int T, int KC>
    __device__ void fetch(Fetch<T, KC> &f, int k0, int ctile) const
    {
        constexpr int N4 = NB * KC / 4, U = (N4 + T - 1) / T;
        const bool vec = !((k & 3) | (ld & 3));
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = min((int)threadIdx.x + u * T, N4 - 1);
            const int b = i / (KC / 4), r = k0 + 4 * (i - b * (KC / 4));
            const float *row = x + (size_t)b * ld;
            if (vec)
                f.v[u] = ld4(row + min(r, k - 4));
            else
                f.v[u] = f32x4{row[min(r, k - 1)], row[min(r + 1, k - 1)], row[min(r + 2, k - 1)],
                               row[min(r + 3, k - 1)]};
        }
    }
    template <int T, int KC>
    __device__ void load(const Fetch<T, KC> &f, float *xs, int k0, int ctile) const
    {
        constexpr int N4 = NB * KC / 4, U = (N4 + T - 1) / T;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = threadIdx.x + u * T;
            if (i < N4) {
                const int b = i / (KC / 4), r = k0 + 4 * (i - b * (KC / 4));
                f32x4 v = f.v[u];
                v.x = r < k ? v.x : 0.0f;
                v.y = r + 1 < k ? v.y : 0.0f;
                v.z = r + 2 < k ? v.z : 0.0f;
                v.w = r + 3 < k ? v.w : 0.0f;
                *(f32x4 *)(xs + 4 * i) = v;
            }
        }
    }
    __device__ void finish(int s, int c, int nct) const {}
};

// The talker o-proj's input rows from the per-page attention partials of
// k_talker_attn (flash-decoding): row h*128 + d of the attention output is
//   sum_c w_c acc[c][h][d] / sum_c w_c l[c][h],  w_c = exp(m[c][h] - max m),
// the reference's softmax over the whole row (talker.rs:304-331, softmax_raw
// gemv.rs:471-482) regrouped by page.  Thread t owns rows t + e*T of the
// tile's k-slice; the rows of a wave share one head, so the page maxima and
// sums are wave-uniform loads.  The cache length is read in the fetch stage
// (a scalar load) and the pages after the weights are in flight.
template <int PG>
struct ProAttnCombine {
    // chunks of P.V fetched ahead of the weights: 16 one-page chunks (KV 1024,
    // where two-page chunks take over), 20 two-page chunks (KV 2560)
    static constexpr int PF = PG == 1 ? 16 : 20;
    static constexpr int PB = (64 - PF) / 2;  // chunks loaded together after them (PF + k*PB never straddles 64)
    const float *am, *al;    // [16 heads][MAX_CHUNKS] chunk max / exp-sum (a chunk: PG pages)
    const float *aacc;       // [MAX_CHUNKS][16][128] chunk P.V
    const DevState *st;
    int slot_ovr;            // >= 0: the row's KV slot (prefill rows), else st->kv_len
    uint32_t *seq;           // the epoch counters: LL_TQKV and LL_TMLP advanced once per launch
    template <int T, int KC>
    struct Fetch {
        int L;
        float m[KC / T][2], l[KC / T][2], a[KC / T][PF];
    };
    // every load here is in bounds whatever the cache length (pages past it
    // are masked in load), so all are issued before the weights
    template <int T, int KC>
    __device__ void fetch(Fetch<T, KC> &f, int k0, int ctile) const
    {
        static_assert(KC % T == 0 && KC % HEAD_DIM == 0 && MAX_CHUNKS == 128, "rows per thread, pages per lane");
        static_assert(PF + 2 * PB == 64, "a block of pages never straddles page 64");
        const int lane = threadIdx.x & 63;
        f.L = (slot_ovr >= 0 ? slot_ovr : st->kv_len) + 1;
#pragma unroll
        for (int e = 0; e < KC / T; e++) {
            const int row = k0 + threadIdx.x + e * T;   // rows past the 16 heads (a slice's tail) read head 15
            const int h = __builtin_amdgcn_readfirstlane(min(row / HEAD_DIM, 15)), d = row & (HEAD_DIM - 1);
            f.m[e][0] = am[h * MAX_CHUNKS + lane];
            f.m[e][1] = am[h * MAX_CHUNKS + 64 + lane];
            f.l[e][0] = al[h * MAX_CHUNKS + lane];
            f.l[e][1] = al[h * MAX_CHUNKS + 64 + lane];
#pragma unroll
            for (int j = 0; j < PF; j++) f.a[e][j] = aacc[((size_t)j * 16 + h) * HEAD_DIM + d];
        }
    }
    template <int T, int KC>
    __device__ void load(const Fetch<T, KC> &f, float *xs, int k0, int ctile) const
    {
        merge<T, KC>(f, k0, [&](int e, int i, float v) { xs[i] = v; });
    }
    // Thread t merges rows k0 + t + e * T, which on a one-group tile are its
    // own GEMV rows: they go straight into its registers (no LDS, no barrier).
    static constexpr bool kOwnRows = true;
    template <int T, int KC, int R>
    __device__ void load_own(const Fetch<T, KC> &f, float (&xv)[R][1], int k0) const
    {
        static_assert(KC / T == R, "one group per tile");
        merge<T, KC>(f, k0, [&](int e, int i, float v) { xv[e][0] = v; });
    }
    template <int T, int KC, class Put>
    __device__ void merge(const Fetch<T, KC> &f, int k0, const Put &put) const
    {
        const int lane = threadIdx.x & 63;
        const int C = (f.L + KV_PAGE * PG - 1) / (KV_PAGE * PG);
        const bool v0 = lane < C, v1 = lane + 64 < C;
#pragma unroll
        for (int e = 0; e < KC / T; e++) {
            const int i = threadIdx.x + e * T, row = k0 + i;
            const int h = __builtin_amdgcn_readfirstlane(min(row / HEAD_DIM, 15)), d = row & (HEAD_DIM - 1);
            // lane j holds chunks j and j + 64
            const float m0 = v0 ? f.m[e][0] : -INFINITY, m1 = v1 ? f.m[e][1] : -INFINITY;
            const float M = wave_max_dpp(fmaxf(m0, m1));
            const float w0 = v0 ? expf(m0 - M) : 0.0f, w1 = v1 ? expf(m1 - M) : 0.0f;
            const float Ls = wave_sum_dpp(w0 * (v0 ? f.l[e][0] : 0.0f) + w1 * (v1 ? f.l[e][1] : 0.0f));
            float o = 0.0f;
#pragma unroll
            for (int j = 0; j < PF; j++) {
                const float wc = lane_value(w0, j);
                o = j < C ? fmaf(wc, f.a[e][j], o) : o;
            }
            const float *ah = aacc + (size_t)h * HEAD_DIM + d;
            for (int c0 = PF; c0 < C; c0 += PB) {
                float av[PB];
#pragma unroll
                for (int j = 0; j < PB; j++) av[j] = ah[(size_t)min(c0 + j, C - 1) * 16 * HEAD_DIM];
                const float wb = c0 < 64 ? w0 : w1;
#pragma unroll
                for (int j = 0; j < PB; j++) {
                    const int c = c0 + j;
                    o = c < C ? fmaf(lane_value(wb, c & 63), av[j], o) : o;
                }
            }
            put(e, i, row < 16 * HEAD_DIM ? o / Ls : 0.0f);
        }
    }
    __device__ void finish(int s, int c, int nct) const
    {
        if (seq && s == 0 && c == 0 && threadIdx.x == 0) {
            seq[LL_TQKV] = seq[LL_TQKV] + 1;
            seq[LL_TMLP] = seq[LL_TMLP] + 1;
        }
    }
};

// Residual update + RMSNorm (gemv.rs:445-454):
//   x = base + sum_s parts[s]   (+ bias)        -- the producer's k-slices in order
//   xs = x * (1/sqrt(mean(x^2) + 1e-6)) * gamma  -- this tile's rows
// Every workgroup rebuilds x in LDS; after the tile's GEMV, the slice-0
// workgroups store x (the residual stream) to x_out and the normed vector to
// side, each a share of the columns.  Consumer row b reads producer row
// prow + b of NBP rows.  Needs k % 4 == 0 and k <= KMAX.  Up to MS producer
// slices are fetched ahead (RES_MAX_S, or 6 at the predictor's width, whose
// down projection leaves 6); more are read in the load stage.
constexpr int RES_MAX_S = 4;

template <int NB, int KMAX>
struct ProResidRms {
    static constexpr int MS = KMAX <= 1024 ? 6 : RES_MAX_S;
    const float *base;
    int ldb;
    const float *parts;
    int S, NBP, prow, npad;
    const float *bias;
    const uint16_t *gamma;
    int k;
    float *x_out;
    float *side;
    uint32_t *seq;           // when set: advanced once per launch (the epoch of a fused launch before it)
    __device__ static float *xf_lds()
    {
        __shared__ float xf[NB * KMAX];
        return xf;
    }
    __device__ static float *inv_lds()
    {
        __shared__ float inv[NB];
        return inv;
    }
    template <int T, int KC>
    struct Fetch {
        static constexpr int U = (KMAX / 4 + T - 1) / T;   // float4 of a row per thread
        static constexpr int UG = (KC + T - 1) / T;         // gamma values per thread
        f32x4 base[NB][U];
        f32x4 part[NB][MS][U];
        f32x4 bias[U];
        uint32_t g[4 * UG];   // UG for the LDS tile; a thread's own R rows (R = GB * UG, GB <= 4)
    };
    template <int T, int KC>
    __device__ void fetch(Fetch<T, KC> &f, int k0, int ctile) const
    {
        constexpr int UG = Fetch<T, KC>::UG;
#pragma unroll
        for (int u = 0; u < UG; u++) f.g[u] = gamma[min(k0 + (int)threadIdx.x + u * T, k - 1)];
        fetch_rows<T, KC>(f);
    }
    // The gammas of the thread's own GEMV rows k0 + r * P + ph instead.
    template <int T, int KC, int R, int P>
    __device__ void fetch_own(Fetch<T, KC> &f, int k0, int ph) const
    {
        static_assert(R <= 4 * Fetch<T, KC>::UG, "own-row gammas");
#pragma unroll
        for (int r = 0; r < R; r++) f.g[r] = gamma[min(k0 + r * P + ph, k - 1)];
        fetch_rows<T, KC>(f);
    }
    template <int T, int KC>
    __device__ void fetch_rows(Fetch<T, KC> &f) const
    {
        constexpr int U = Fetch<T, KC>::U;
        const int k4 = k >> 2, t = threadIdx.x;
#pragma unroll
        for (int b = 0; b < NB; b++) {
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int i = min(t + u * T, k4 - 1);
                if (base) f.base[b][u] = ld4(base + (size_t)b * ldb + 4 * i);
                if (parts) {
#pragma unroll
                    for (int s = 0; s < MS; s++)
                        f.part[b][s][u] = ld4(parts + ((size_t)min(s, S - 1) * NBP + prow + b) * npad + 4 * i);
                }
            }
        }
        if (bias) {
#pragma unroll
            for (int u = 0; u < U; u++) f.bias[u] = ld4(bias + 4 * min(t + u * T, k4 - 1));
        }
    }
    template <int T, int KC>
    __device__ void load(const Fetch<T, KC> &f, float *xs, int k0, int ctile) const
    {
        constexpr int UG = Fetch<T, KC>::UG;
        float iv[NB];
        stage<T, KC>(f, iv);
        const float *xf = xf_lds();
        const int t = threadIdx.x;
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int u = 0; u < UG; u++) {
                const int r = t + u * T;
                if (r < KC) xs[b * KC + r] = (k0 + r < k) ? xf[b * KMAX + k0 + r] * iv[b] * h2f(f.g[u]) : 0.0f;
            }
    }
    // Each thread normalises its own GEMV rows k0 + r * P + ph straight from
    // the staged row into its registers: no LDS tile, no second barrier.
    static constexpr bool kOwnRowsAny = true;
    template <int T, int KC, int R, int P>
    __device__ void load_own(const Fetch<T, KC> &f, float (&xv)[R][NB], int k0, int ph) const
    {
        float iv[NB];
        stage<T, KC>(f, iv);
        const float *xf = xf_lds();
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = k0 + r * P + ph;
                xv[r][b] = row < k ? xf[b * KMAX + row] * iv[b] * h2f(f.g[r]) : 0.0f;
            }
    }
    // The residual row(s) summed and staged in LDS, and 1 / rms of each.
    template <int T, int KC>
    __device__ void stage(const Fetch<T, KC> &f, float (&ivs)[NB]) const
    {
        constexpr int NW = T / 64;
        __shared__ float wss[NB][NW];
        constexpr int U = Fetch<T, KC>::U;
        float *xf = xf_lds();
        const int k4 = k >> 2, t = threadIdx.x;
        float ssb[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            float ss = 0.0f;
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int i = t + u * T;
                f32x4 x = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                if (parts) {
                    f32x4 a = f.part[b][0][u];
#pragma unroll
                    for (int s = 1; s < MS; s++)
                        if (s < S) a += f.part[b][s][u];
                    for (int s = MS; s < S; s++)
                        a += ld4(parts + ((size_t)s * NBP + prow + b) * npad + 4 * min(i, k4 - 1));
                    x = base ? f.base[b][u] + a : a;
                } else if (base) {
                    x = f.base[b][u];
                }
                if (bias) x += f.bias[u];
                if (i < k4) {
                    *(f32x4 *)(xf + b * KMAX + 4 * i) = x;
                    ss += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
                }
            }
            ssb[b] = ss;
        }
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const float w = wave_sum_dpp(ssb[b]);
            if ((t & 63) == 0) wss[b][t >> 6] = w;
        }
        __syncthreads();
#pragma unroll
        for (int b = 0; b < NB; b++) {
            float tot = 0.0f;
#pragma unroll
            for (int i = 0; i < NW; i++) tot += wss[b][i];
            const float iv = 1.0f / sqrtf(tot / (float)k + 1e-6f);
            if (t == 0) inv_lds()[b] = iv;
            ivs[b] = iv;
        }
    }
    // after the tile: slice-0 workgroups store their share of x / normed x
    __device__ void finish(int s, int c, int nct) const
    {
        if (seq && s == 0 && c == 0 && threadIdx.x == 0) *seq = *seq + 1;
        if (s != 0 || (!x_out && !side)) return;
        const float *xf = xf_lds();
        const int per = (k + nct - 1) / nct;
        const int j0 = c * per, j1 = min(j0 + per, k);
        for (int b = 0; b < NB; b++) {
            const float iv = inv_lds()[b];
            for (int j = j0 + threadIdx.x; j < j1; j += blockDim.x) {
                const float x = xf[b * KMAX + j];
                if (x_out) x_out[(size_t)b * k + j] = x;
                if (side) side[(size_t)b * k + j] = x * iv * h2f(gamma[j]);
            }
        }
    }
};

// silu(gate) * up from gate|up partial sums (talker.rs:343-345).  The fused
// weight interleaves 32-column groups: gate group j at columns 64j..64j+31,
// up group j at 64j+32..64j+63.  Used only when gate|up runs in more than one
// k-slice (the SiLU epilogue covers the single-slice case).
template <int NB>
struct ProSwiglu {
    const float *part;
    int S, npad, inter;
    template <int T, int KC>
    struct Fetch {
        static constexpr int U = (NB * KC + T - 1) / T;
        float g[U][RES_MAX_S], u[U][RES_MAX_S];
    };
    template <int T, int KC>
    __device__ void fetch(Fetch<T, KC> &f, int k0, int ctile) const
    {
        constexpr int U = Fetch<T, KC>::U;
#pragma unroll
        for (int q = 0; q < U; q++) {
            const int i = min((int)threadIdx.x + q * T, NB * KC - 1);
            const int b = i / KC, r = min(k0 + (i - b * KC), inter - 1);
            const int gc = (r >> 5) * 64 + (r & 31);
#pragma unroll
            for (int s = 0; s < RES_MAX_S; s++) {
                const float *p = part + ((size_t)min(s, S - 1) * NB + b) * npad;
                f.g[q][s] = p[gc];
                f.u[q][s] = p[gc + 32];
            }
        }
    }
    template <int T, int KC>
    __device__ void load(const Fetch<T, KC> &f, float *xs, int k0, int ctile) const
    {
        constexpr int U = Fetch<T, KC>::U;
#pragma unroll
        for (int q = 0; q < U; q++) {
            const int i = threadIdx.x + q * T;
            if (i < NB * KC) {
                const int b = i / KC, r = k0 + (i - b * KC);
                float g = f.g[q][0], u = f.u[q][0];
#pragma unroll
                for (int s = 1; s < RES_MAX_S; s++) {
                    g = s < S ? g + f.g[q][s] : g;
                    u = s < S ? u + f.u[q][s] : u;
                }
                const int gc = (min(r, inter - 1) >> 5) * 64 + (min(r, inter - 1) & 31);
                for (int s = RES_MAX_S; s < S; s++) {
                    const float *p = part + ((size_t)s * NB + b) * npad;
                    g += p[gc];
                    u += p[gc + 32];
                }
                xs[i] = r < inter ? silu_f(g) * u : 0.0f;
            }
        }
    }
    __device__ void finish(int s, int c, int nct) const {}
};

// Raw Q4 element of a reference-layout row: the packed byte and the scale.
struct Q4Elem {
    uint32_t byte, scale;
};

__device__ __forceinline__ Q4Elem q4_row_fetch(const Q4Rows &e, uint32_t row, int col)
{
    const int g = col >> 5, j = col & 31;
    return Q4Elem{e.packed[(size_t)row * e.G * 16 + g * 16 + (j >> 1)], e.scales[(size_t)row * e.G + g]};
}

__device__ __forceinline__ float q4_elem_value(Q4Elem v, int col)
{
    const int q = (int)((col & 1) ? (v.byte >> 4) : (v.byte & 0x0F)) - 8;
    return h2f(v.scale) * (float)q;
}

// One dequantised embedding row (embed_lookup_q4, gemv.rs:415-437); the row
// index is read from device memory.
struct ProEmbed {
    Q4Rows emb;
    const uint32_t *code;
    template <int T, int KC>
    struct Fetch {
        Q4Elem e[(KC + T - 1) / T];
    };
    template <int T, int KC>
    __device__ void fetch(Fetch<T, KC> &f, int k0, int ctile) const
    {
        const uint32_t row = *code;
#pragma unroll
        for (int u = 0; u < (KC + T - 1) / T; u++)
            f.e[u] = q4_row_fetch(emb, row, min(k0 + (int)threadIdx.x + u * T, emb.n - 1));
    }
    template <int T, int KC>
    __device__ void load(const Fetch<T, KC> &f, float *xs, int k0, int ctile) const
    {
#pragma unroll
        for (int u = 0; u < (KC + T - 1) / T; u++) {
            const int i = threadIdx.x + u * T, r = k0 + i;
            if (i < KC) xs[i] = r < emb.n ? q4_elem_value(f.e[u], r) : 0.0f;
        }
    }
    __device__ void finish(int s, int c, int nct) const {}
};

// Predictor step input: the previous head's code chosen from its argmax
// candidates (code_predictor.rs:253-260; the teacher-forced code when forcing),
// then that code's embedding row.  The wave argmax runs in every wave, so
// the row loads need no barrier; workgroup (0, 0) records the code.
// Layer 0's input at predictor steps 1..14: the projected embedding row of
// the step's code (project_input(get_acoustic_embedding(g-1, code)) + bias,
// code_predictor.rs:51-61, 255-260), read from a table built at upload with
// the same GEMV, then RMSNorm as in ProResidRms.  The code is the argmax of
// the previous head's candidates, or the teacher-forced code, or (no
// candidates) the code already recorded in DevState; with candidates
// workgroup (0, 0) records it.  Slice-0 workgroups store the row (the
// layer's residual input) to x_out.
template <int KMAX>
struct ProCodeRowRms {
    const float *table;      // [rows][k]
    int rows;
    const float2 *cand;      // null: the code is st->used[slot]
    int ncand;
    DevState *st;
    int slot;
    uint32_t *codes_api;
    const uint16_t *gamma;
    int k;
    float *x_out;
    __device__ static float *xf_lds()
    {
        __shared__ float xf[KMAX];
        return xf;
    }
    template <int T, int KC>
    struct Fetch {
        static constexpr int U = (KMAX / 4 + T - 1) / T;
        static constexpr int UG = (KC + T - 1) / T;
        f32x4 x[U];
        uint32_t g[UG];
        uint32_t pred, used;
        bool nan;
    };
    template <int T, int KC>
    __device__ void fetch(Fetch<T, KC> &f, int k0, int ctile) const
    {
        constexpr int U = Fetch<T, KC>::U, UG = Fetch<T, KC>::UG;
        const int k4 = k >> 2, t = threadIdx.x;
#pragma unroll
        for (int u = 0; u < UG; u++) f.g[u] = gamma[min(k0 + t + u * T, k - 1)];
        f.nan = false;
        if (cand) {
            const int force = st->force;
            const uint32_t fc = st->fcode[slot];
            f.pred = cand_argmax(cand, ncand, f.nan);
            f.used = force ? fc : f.pred;
        } else if (st) {
            f.pred = f.used = st->used[slot];
        } else {
            f.pred = f.used = blockIdx.y;   // table build: one row per grid row
        }
        const float *row = table + (size_t)min(f.used, (uint32_t)(rows - 1)) * k;
#pragma unroll
        for (int u = 0; u < U; u++) f.x[u] = ld4(row + 4 * min(t + u * T, k4 - 1));
    }
    template <int T, int KC>
    __device__ void load(const Fetch<T, KC> &f, float *xs, int k0, int ctile) const
    {
        constexpr int NW = T / 64;
        __shared__ float wss[NW];
        constexpr int U = Fetch<T, KC>::U, UG = Fetch<T, KC>::UG;
        float *xf = xf_lds();
        const int k4 = k >> 2, t = threadIdx.x;
        float ss = 0.0f;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = t + u * T;
            const f32x4 x = f.x[u];
            if (i < k4) {
                *(f32x4 *)(xf + 4 * i) = x;
                ss += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
            }
        }
        const float w = wave_sum_dpp(ss);
        if ((t & 63) == 0) wss[t >> 6] = w;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int i = 0; i < NW; i++) tot += wss[i];
        const float iv = 1.0f / sqrtf(tot / (float)k + 1e-6f);
#pragma unroll
        for (int u = 0; u < UG; u++) {
            const int r = t + u * T;
            if (r < KC) xs[r] = (k0 + r < k) ? xf[k0 + r] * iv * h2f(f.g[u]) : 0.0f;
        }
        if (cand && k0 == 0 && ctile == 0 && t == 0) {
            st->pred[slot] = f.pred;
            st->used[slot] = f.used;
            st->prev[slot] = f.used;
            if (f.nan) st->nan_flag = 1;
            if (codes_api) codes_api[slot - 1] = f.pred;
        }
    }
    __device__ void finish(int s, int c, int nct) const
    {
        if (s != 0 || !x_out) return;
        const float *xf = xf_lds();
        const int per = (k + nct - 1) / nct;
        const int j0 = c * per, j1 = min(j0 + per, k);
        for (int j = j0 + threadIdx.x; j < j1; j += blockDim.x) x_out[j] = xf[j];
    }
};

// Every row of a Q4 table dequantised: out[r][j], grid (column blocks, rows).
__global__ void k_dequant_rows(Q4Rows e, float *out)
{
    const int j = blockIdx.x * blockDim.x + threadIdx.x, r = blockIdx.y;
    if (j < e.n) out[(size_t)r * e.n + j] = q4_row_value(e, r, j);
}

// x[r][j] = (sum over slices s of part[r][s][j], in slice order) + bias[j]:
// the order of ProResidRms's residual-free sum, so a table row feeds the
// same bits into layer 0 as the projection partials would.
__global__ void k_rows_from_parts(const float *part, int S, int npad, const float *bias, int n, float *out)
{
    const int j = blockIdx.x * blockDim.x + threadIdx.x, r = blockIdx.y;
    if (j >= n) return;
    const float *pr = part + (size_t)r * S * npad + j;
    float a = pr[0];
    for (int s2 = 1; s2 < S; s2++) a += pr[(size_t)s2 * npad];
    out[(size_t)r * n + j] = bias ? a + bias[j] : a;
}

struct ProArgmaxEmbed {
    Q4Rows emb;
    const float2 *cand;
    int ncand;
    DevState *st;
    int slot;
    uint32_t *codes_api;
    template <int T, int KC>
    struct Fetch {
        Q4Elem e[(KC + T - 1) / T];
        uint32_t pred, used;
        bool nan;
    };
    template <int T, int KC>
    __device__ void fetch(Fetch<T, KC> &f, int k0, int ctile) const
    {
        const int force = st->force;
        const uint32_t fc = st->fcode[slot];
        f.pred = cand_argmax(cand, ncand, f.nan);
        f.used = force ? fc : f.pred;
#pragma unroll
        for (int u = 0; u < (KC + T - 1) / T; u++)
            f.e[u] = q4_row_fetch(emb, f.used, min(k0 + (int)threadIdx.x + u * T, emb.n - 1));
    }
    template <int T, int KC>
    __device__ void load(const Fetch<T, KC> &f, float *xs, int k0, int ctile) const
    {
#pragma unroll
        for (int u = 0; u < (KC + T - 1) / T; u++) {
            const int i = threadIdx.x + u * T, r = k0 + i;
            if (i < KC) xs[i] = r < emb.n ? q4_elem_value(f.e[u], r) : 0.0f;
        }
        if (k0 == 0 && ctile == 0 && threadIdx.x == 0) {
            st->pred[slot] = f.pred;
            st->used[slot] = f.used;
            st->prev[slot] = f.used;
            if (f.nan) st->nan_flag = 1;
            if (codes_api) codes_api[slot - 1] = f.pred;
        }
    }
    __device__ void finish(int s, int c, int nct) const {}
};

// Predictor prefill input: row 0 = talker hidden, row 1 = codec embedding
// of the semantic code (code_predictor.rs:235-241, generate_new.rs:620).
struct ProHidEmbed {
    const float *hidden;
    Q4Rows emb;
    const uint32_t *code;
    int k;
    template <int T, int KC>
    struct Fetch {
        float h[(KC + T - 1) / T];
        Q4Elem e[(KC + T - 1) / T];
    };
    template <int T, int KC>
    __device__ void fetch(Fetch<T, KC> &f, int k0, int ctile) const
    {
        const uint32_t row = *code;
#pragma unroll
        for (int u = 0; u < (KC + T - 1) / T; u++) {
            const int rc = min(k0 + (int)threadIdx.x + u * T, k - 1);
            f.h[u] = hidden[rc];
            f.e[u] = q4_row_fetch(emb, row, rc);
        }
    }
    template <int T, int KC>
    __device__ void load(const Fetch<T, KC> &f, float *xs, int k0, int ctile) const
    {
#pragma unroll
        for (int u = 0; u < (KC + T - 1) / T; u++) {
            const int i = threadIdx.x + u * T, r = k0 + i;
            if (i < KC) {
                xs[i] = r < k ? f.h[u] : 0.0f;
                xs[KC + i] = r < k ? q4_elem_value(f.e[u], r) : 0.0f;
            }
        }
    }
    __device__ void finish(int s, int c, int nct) const {}
};

// ---------------------------------------------------------------------------
// GEMV epilogues: (slice s, row b, column tile c, column cc in the tile,
// tile width C, this row's tile outputs yb[0..C))
// ---------------------------------------------------------------------------

template <int NB>
struct EpiPart {
    float *part;
    int npad;
    template <class Y>
    __device__ void operator()(int s, int b, int c, int cc, int C, const Y &y) const
    {
        part[((size_t)s * NB + b) * npad + c * C + cc] = y(cc);
    }
};

// Column sums stored as (epoch, value) words for a consumer in the same
// launch (k_talker_qkv_attn): one 8-byte system-scope store per column, the
// epoch (*seq + 1) in the high half, so a word and its epoch arrive
// together and no fence is needed.
template <int NB = 1>
struct EpiLL {
    uint64_t *ll;            // [S][NB][npad]
    int npad;
    const uint32_t *seq;
    uint32_t epoch;          // *seq + 1, read by the kernel at its start
    template <class Y>
    __device__ void operator()(int s, int b, int c, int cc, int C, const Y &y) const
    {
        __hip_atomic_store(ll + ((size_t)s * NB + b) * npad + c * C + cc,
                           ((uint64_t)epoch << 32) | __float_as_uint(y(cc)), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
    }
};

// silu(gate) * up of an interleaved single-slice gate|up tile (EpiSwiglu)
// stored as (epoch, value) words for the down projection's tiles in the
// same launch (k_mlp).
template <int NB = 1>
struct EpiSwigluLL {
    uint64_t *ll;            // [NB][ld]
    int ld;                  // inter
    const uint32_t *seq;
    uint32_t epoch;          // *seq + 1, read by the kernel at its start
    template <class Y>
    __device__ void operator()(int s, int b, int c, int cc, int C, const Y &y) const
    {
        if ((cc & 63) < 32) {
            const int j = (c * C + cc) >> 6;
            const float h = silu_f(y(cc)) * y(cc + 32);
            __hip_atomic_store(ll + (size_t)b * ld + j * 32 + (cc & 31), ((uint64_t)epoch << 32) | __float_as_uint(h),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
};

// GEMV input rows k0.. from (epoch, value) words that producer tiles of the
// same launch store (k_mlp's down projection): fetch reads the epoch, load
// polls the slice's words (bounded, as every such wait) once the weights are
// in flight.  Rows past n read as 0.
template <int NB = 1>
struct ProLL {
    const uint64_t *ll;      // [NB][n]
    int n;
    const uint32_t *seq;
    DevState *st;
    template <int T, int KC>
    struct Fetch {
        uint32_t epoch;
        int give_up;
    };
    template <int T, int KC>
    __device__ void fetch(Fetch<T, KC> &f, int k0, int ctile) const
    {
        f.epoch = *seq + 1;
        f.give_up = st->sync_err;
    }
    template <int T, int KC>
    __device__ void load(const Fetch<T, KC> &f, float *xs, int k0, int ctile) const
    {
        constexpr int U = (NB * KC + T - 1) / T;
        float v[U];
        for (int it = 0;; it++) {
            bool ok = true;
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int i = min((int)threadIdx.x + u * T, NB * KC - 1);
                const int b = i / KC, r = k0 + (i - b * KC);
                const uint64_t w = __hip_atomic_load(ll + (size_t)b * n + min(r, n - 1), __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_SYSTEM);
                ok = ok && (r >= n || (uint32_t)(w >> 32) == f.epoch);
                v[u] = r < n ? __uint_as_float((uint32_t)w) : 0.0f;
            }
            if (__all(ok) || f.give_up) break;
            if (it >= LL_SPIN_MAX) {
                if ((threadIdx.x & 63) == 0) st->sync_err = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = threadIdx.x + u * T;
            if (i < NB * KC) xs[i] = v[u];
        }
    }
    __device__ void finish(int s, int c, int nct) const {}
};

// silu(gate) * up of the GEMV input rows k0.. from the raw gate|up column
// sums that one-group producer tiles of the same launch store as (epoch,
// value) words (EpiLL over the interleaved gate|up weight: group 2j holds
// gate columns 32j..32j+31, group 2j + 1 the matching up columns).  The
// product is formed as EpiSwigluLL and ProSwiglu form it.  Rows past n read
// as 0.
template <int NB = 1>
struct ProSwigluLL {
    const uint64_t *ll;      // [NB][npad] gate|up words
    int npad, n;             // words per row, rows of h (inter)
    const uint32_t *seq;
    DevState *st;
    template <int T, int KC>
    struct Fetch {
        uint32_t epoch;
        int give_up;
    };
    template <int T, int KC>
    __device__ void fetch(Fetch<T, KC> &f, int k0, int ctile) const
    {
        f.epoch = *seq + 1;
        f.give_up = st->sync_err;
    }
    template <int T, int KC>
    __device__ void load(const Fetch<T, KC> &f, float *xs, int k0, int ctile) const
    {
        constexpr int U = (NB * KC + T - 1) / T;
        float g[U], u[U];
        for (int it = 0;; it++) {
            bool ok = true;
#pragma unroll
            for (int q = 0; q < U; q++) {
                const int i = min((int)threadIdx.x + q * T, NB * KC - 1);
                const int b = i / KC, r = k0 + (i - b * KC), rr = min(r, n - 1);
                const uint64_t *p = ll + (size_t)b * npad + (rr >> 5) * 64 + (rr & 31);
                const uint64_t wg = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                const uint64_t wu = __hip_atomic_load(p + 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                ok = ok && (r >= n || ((uint32_t)(wg >> 32) == f.epoch && (uint32_t)(wu >> 32) == f.epoch));
                g[q] = __uint_as_float((uint32_t)wg);
                u[q] = __uint_as_float((uint32_t)wu);
            }
            if (__all(ok) || f.give_up) break;
            if (it >= LL_SPIN_MAX) {
                if ((threadIdx.x & 63) == 0) st->sync_err = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
#pragma unroll
        for (int q = 0; q < U; q++) {
            const int i = threadIdx.x + q * T;
            if (i < NB * KC) {
                const int b = i / KC, r = k0 + (i - b * KC);
                xs[i] = r < n ? silu_f(g[q]) * u[q] : 0.0f;
            }
        }
    }
    __device__ void finish(int s, int c, int nct) const {}
};

// Row blockIdx.y of a batch of single rows: the per-row arithmetic of NB = 1
// (used to build the predictor's projected-row tables at upload).
struct ProPlainY {
    const float *x;
    int ld, k;
    template <int T, int KC>
    using Fetch = typename ProPlain<1>::template Fetch<T, KC>;
    template <int T, int KC>
    __device__ void fetch(Fetch<T, KC> &f, int k0, int ctile) const
    {
        ProPlain<1>{x + (size_t)blockIdx.y * ld, ld, k}.template fetch<T, KC>(f, k0, ctile);
    }
    template <int T, int KC>
    __device__ void load(const Fetch<T, KC> &f, float *xs, int k0, int ctile) const
    {
        ProPlain<1>{x + (size_t)blockIdx.y * ld, ld, k}.template load<T, KC>(f, xs, k0, ctile);
    }
    __device__ void finish(int s, int c, int nct) const {}
};

struct EpiPartY {
    float *part;             // [rows][S][npad]
    int npad, S;
    template <class Y>
    __device__ void operator()(int s, int b, int c, int cc, int C, const Y &y) const
    {
        part[((size_t)blockIdx.y * S + s) * npad + c * C + cc] = y(cc);
    }
};

template <int NB>
struct EpiStore {
    float *y;
    int ld, n;
    const float *bias;
    template <class Y>
    __device__ void operator()(int s, int b, int c, int cc, int C, const Y &yv) const
    {
        const int col = c * C + cc;
        if (col < n) y[(size_t)b * ld + col] = bias ? yv(cc) + bias[col] : yv(cc);
    }
};

// Single-slice interleaved gate|up: h = silu(gate) * up, straight from the
// tile (the tile holds whole gate/up group pairs).
template <int NB>
struct EpiSwiglu {
    float *h;
    int ld;
    template <class Y>
    __device__ void operator()(int s, int b, int c, int cc, int C, const Y &y) const
    {
        if ((cc & 63) < 32) {
            const int j = (c * C + cc) >> 6;
            h[(size_t)b * ld + j * 32 + (cc & 31)] = silu_f(y(cc)) * y(cc + 32);
        }
    }
};

// Single-slice lm head: the tile's argmax candidate (value, index) with the
// last maximum among its columns below n; index -1 marks a NaN in the tile.
// Runs on wave 0 (lane l takes columns l, l + 64, ...) instead of per column.
struct EpiArgmax {
    static constexpr bool kWave = true;
    float2 *cand;
    int n;
    template <class Y>
    __device__ void wave(int s, int c, int C, const Y &y, int lane) const
    {
        float v = -INFINITY;
        int i = -2;
        bool nanl = false;
        for (int j0 = 0; j0 < C; j0 += 64) {
            const int col = j0 + lane;
            const bool ok = col < C && c * C + col < n;
            const float yv = y(min(col, C - 1));
            nanl |= ok && isnan(yv);
            argmax_merge(v, i, ok ? yv : -INFINITY, ok ? c * C + col : -2);
        }
        const bool nan = __ballot(nanl) != 0;
        wave_argmax_last(v, i);
        if (lane == 0) cand[c] = make_float2(v, __builtin_bit_cast(float, nan ? -1 : i));
    }
    template <class Y>
    __device__ void operator()(int, int, int, int, int, const Y &) const {}
};

template <class E, class = void>
struct WaveEpi { static constexpr bool v = false; };
template <class E>
struct WaveEpi<E, std::void_t<decltype(E::kWave)>> { static constexpr bool v = E::kWave; };

// ---------------------------------------------------------------------------
// The split-K Q4 GEMV.
//
// Thread t of a T-thread workgroup owns one 32-column group gl of the tile
// and rows r*P + ph (P = T/GB, r < R) of its k-slice.  When the number of
// waves NW is a multiple of GB, whole waves share a group: wave w holds group
// w % GB and ph = (w / GB) * 64 + lane; otherwise gl = t % GB, ph = t / GB.
// Per row a thread loads one 16-byte block of 32 nibbles and computes
//     acc[j] += a * nib_j,   a = f32(scale) * x[row]
// with each 32-bit word masked into f16 halves that hold one nibble each as
// an exact subnormal (nib * 2^-24 or nib * 2^-20), multiplied by a * 2^24 or
// a * 2^20 in one v_fma_mix_f32 per output (the product is exactly
// a * nib); 1.625 VALU operations per weight.  The -8 offset is applied
// once as acc[j] -= 8 * sum(a).  The lanes of a group are folded by a
// reduce-scatter (DPP lane exchanges in the one-group-per-wave layout),
// the waves through LDS, in fixed order.
// ---------------------------------------------------------------------------

// One halving step of the in-wave reduce-scatter: the lane keeps half H of
// its values (the upper half when `sel`) and adds the partner lane's copy
// of that half; CTRL is the DPP lane exchange with the partner.
template <int H, int CTRL, int NB>
__device__ __forceinline__ void rs_dpp_step(float (&v)[NB][32], bool sel)
{
    // both halves summed with the partner (DPP operands are values from the
    // previous step, so no VALU -> DPP hazard waits), then the lane's half
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int j = 0; j < H; j++) {
            const float lo = v[b][j] + dpp_mov<CTRL>(v[b][j]);
            const float hi = v[b][j + H] + dpp_mov<CTRL>(v[b][j + H]);
            v[b][j] = sel ? hi : lo;
        }
}

// Reduce-scatter of 32 column sums held by all 64 lanes of a wave.  Partner
// masks in order: lane^15 (row_mirror), ^7 (row_half_mirror), ^3 and ^1
// (quad permutes), ^16 (row swap), then ^32 adds the last value; each mask
// leaves the bits chosen by earlier steps unchanged, so partners always hold
// the same columns.  Lanes l and l^32 end with column wave_rs_col(l).
template <int NB>
__device__ __forceinline__ void wave_rs32(float (&v)[NB][32], int lane)
{
    rs_dpp_step<16, 0x140, NB>(v, lane & 8);
    rs_dpp_step<8, 0x141, NB>(v, lane & 4);
    rs_dpp_step<4, 0x1B, NB>(v, lane & 2);
    rs_dpp_step<2, 0xB1, NB>(v, lane & 1);
#pragma unroll
    for (int b = 0; b < NB; b++) v[b][0] = add_xor32(add_xor16_split(v[b][0], v[b][1]));
}

__device__ __forceinline__ int wave_rs_col(int lane)
{
    return ((lane >> 3) & 1) * 16 + ((lane >> 2) & 1) * 8 + ((lane >> 1) & 1) * 4 + (lane & 1) * 2 + ((lane >> 4) & 1);
}

template <int M, int CNT, int NB>
__device__ __forceinline__ void rs_steps(float (&v)[NB][32], int lane, int &base)
{
    if constexpr (M < 64) {
        if constexpr (CNT > 1) {
            constexpr int H = CNT / 2;
            const bool hi = (lane & M) != 0;
#pragma unroll
            for (int b = 0; b < NB; b++) {
#pragma unroll
                for (int i = 0; i < H; i++) {
                    const float send = hi ? v[b][i] : v[b][i + H];
                    const float keep = hi ? v[b][i + H] : v[b][i];
                    v[b][i] = keep + __shfl_xor(send, M);
                }
            }
            if (hi) base += H;
            rs_steps<M * 2, H, NB>(v, lane, base);
        } else {
#pragma unroll
            for (int b = 0; b < NB; b++) v[b][0] += __shfl_xor(v[b][0], M);
            rs_steps<M * 2, 1, NB>(v, lane, base);
        }
    }
}

// A prologue that can leave each thread's own rows in its registers when
// the tile has one group (P == T) declares `kOwnRows` and load_own.
template <class P, class = void>
struct OwnRows { static constexpr bool v = false; };
template <class P>
struct OwnRows<P, std::void_t<decltype(P::kOwnRows)>> { static constexpr bool v = P::kOwnRows; };

// A prologue that can leave each thread's own rows k0 + r * P + ph in its
// registers on any tile with one group per wave declares `kOwnRowsAny` and
// fetch_own / load_own<T, KC, R, P>.
template <class P, class = void>
struct OwnRowsAny { static constexpr bool v = false; };
template <class P>
struct OwnRowsAny<P, std::void_t<decltype(P::kOwnRowsAny)>> { static constexpr bool v = P::kOwnRowsAny; };

// One tile of the GEMV on workgroup `item` (one workgroup per tile): the
// body of k_gemv, and of the fused launches that host GEMV tiles beside
// other work.  MIX picks the inner loop: v_fma_mix_f32 on f16-subnormal
// nibbles (1.625 VALU operations per weight) or byte converts and FMAs
// (2.25); both give the same bits.
template <int T, int GB, int R, int NB, bool MIX = true, class Pro, class Epi>
__device__ __forceinline__ void gemv_tile(const Q4Tiled &w, const Pro &pro, const Epi &epi, int item)
{
    constexpr int P = T / GB;
    constexpr int KC = R * P;
    constexpr int NW = T / 64;
    constexpr int C = GB * 32;
    constexpr int NL = 64 / GB;
    constexpr int CNTF = (32 / NL) > 0 ? (32 / NL) : 1;
    constexpr int DUP = (GB == 1) ? 32 : 0;     // lanes holding duplicates
    static_assert(R == 2 || R == 4 || R == 8, "scale block is one 4/8/16-byte load");
    __shared__ float xs[NB * KC];
    __shared__ float red[NW * NB * C];
    __shared__ float ybuf[(NW % GB == 0) ? 1 : NB * C];

    constexpr bool WAVE_GROUPS = NW % GB == 0;   // one group per wave
    const int t = threadIdx.x;
    const int lane = t & 63, wv = t >> 6;
    const int gl = WAVE_GROUPS ? wv % GB : t % GB;
    const int ph = WAVE_GROUPS ? (wv / GB) * 64 + lane : t / GB;
    const int items = w.S * w.CT;

    {
        // launch_gemv starts exactly one workgroup per tile
        if (item >= items) return;
        const int s = item / w.CT, c = item - s * w.CT;
        const uint8_t *tile = w.data + (size_t)item * w.tile_bytes;
        // the prologue's loads first, then the weight stream: the prologue's
        // waits then leave the weights in flight
        constexpr bool OWN_ANY = OwnRowsAny<Pro>::v && WAVE_GROUPS;
        typename Pro::template Fetch<T, KC> pf;
        if constexpr (OWN_ANY)
            pro.template fetch_own<T, KC, R, P>(pf, s * KC, ph);
        else
            pro.template fetch<T, KC>(pf, s * KC, c);
        asm volatile("" ::: "memory");
        // the scales before the nibble rows: loads retire in issue order, so
        // row r's arithmetic then waits for rows 0..r only, not the whole tile
        uint32_t sc[R / 2];
        {
            const uint8_t *sp = tile + (size_t)R * T * 16 + (size_t)t * (2 * R);
            if constexpr (R == 8) {
                const u32x4 v = __builtin_nontemporal_load((const u32x4 *)sp);
                sc[0] = v[0]; sc[1] = v[1]; sc[2] = v[2]; sc[3] = v[3];
            } else if constexpr (R == 4) {
                typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
                const u32x2 v = __builtin_nontemporal_load((const u32x2 *)sp);
                sc[0] = v[0]; sc[1] = v[1];
            } else {
                sc[0] = __builtin_nontemporal_load((const uint32_t *)sp);
            }
        }
        u32x4 q[R];
#pragma unroll
        for (int r = 0; r < R; r++)
            q[r] = __builtin_nontemporal_load((const u32x4 *)(tile + ((size_t)r * T + t) * 16));

        constexpr bool OWN = OWN_ANY || (OwnRows<Pro>::v && GB == 1 && WAVE_GROUPS);   // GB == 1: ph == t, P == T
        float xv[R][NB];
        if constexpr (OWN_ANY) {
            pro.template load_own<T, KC, R, P>(pf, xv, s * KC, ph);
        } else if constexpr (OWN) {
            pro.template load_own<T, KC, R>(pf, xv, s * KC);
        } else {
            pro.template load<T, KC>(pf, xs, s * KC, c);
            __syncthreads();
        }

        float acc[NB][32];
        float asum[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            asum[b] = 0.0f;
#pragma unroll
            for (int j = 0; j < 32; j++) acc[b][j] = 0.0f;
        }
        // the inputs of every row read from LDS before the first row waits
        if constexpr (!OWN) {
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int b = 0; b < NB; b++) xv[r][b] = xs[b * KC + r * P + ph];
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t sw = sc[r >> 1];
            const float scl = h2f((r & 1) ? (sw >> 16) : (sw & 0xFFFFu));
            if constexpr (MIX) {
                float a[NB], a24[NB], a20[NB];
#pragma unroll
                for (int b = 0; b < NB; b++) {
                    a[b] = scl * xv[r][b];
                    a24[b] = a[b] * 16777216.0f;   // 2^24
                    a20[b] = a[b] * 1048576.0f;    // 2^20
                    asum[b] += a[b];
                }
#pragma unroll
                for (int wi = 0; wi < 4; wi++) {
                    // Each 16-bit half of a masked word is an f16 subnormal
                    // nib * 2^-24 (nibble in bits 0-3) or nib * 2^-20 (bits
                    // 4-7), exact, and v_fma_mix_f32 takes it straight from
                    // the half: acc + (nib * 2^-24) * (a * 2^24) rounds once,
                    // like acc + nib * a.  Bytes 1 and 3 are shifted down
                    // first (bits 8-15 of a half would reach the exponent).
                    const uint32_t wd = q[r][wi];
                    const uint32_t w8 = wd >> 8;
                    const half2v m0 = __builtin_bit_cast(half2v, and_opaque(wd, 0x000F000Fu));   // columns 0, 4
                    const half2v m1 = __builtin_bit_cast(half2v, and_opaque(wd, 0x00F000F0u));   // 1, 5
                    const half2v m2 = __builtin_bit_cast(half2v, and_opaque(w8, 0x000F000Fu));   // 2, 6
                    const half2v m3 = __builtin_bit_cast(half2v, and_opaque(w8, 0x00F000F0u));   // 3, 7
#pragma unroll
                    for (int b = 0; b < NB; b++) {
                        float *ac = &acc[b][wi * 8];
                        ac[0] = fmaf((float)m0[0], a24[b], ac[0]);
                        ac[4] = fmaf((float)m0[1], a24[b], ac[4]);
                        ac[1] = fmaf((float)m1[0], a20[b], ac[1]);
                        ac[5] = fmaf((float)m1[1], a20[b], ac[5]);
                        ac[2] = fmaf((float)m2[0], a24[b], ac[2]);
                        ac[6] = fmaf((float)m2[1], a24[b], ac[6]);
                        ac[3] = fmaf((float)m3[0], a20[b], ac[3]);
                        ac[7] = fmaf((float)m3[1], a20[b], ac[7]);
                    }
                }
            } else {
                // byte lanes: & 0x0F0F0F0F (even columns) and & 0xF0F0F0F0
                // (odd ones, times a/16), one v_cvt_f32_ubyte and one FMA
                // per weight; the same sums bit for bit
                float a[NB], a16[NB];
#pragma unroll
                for (int b = 0; b < NB; b++) {
                    a[b] = scl * xv[r][b];
                    a16[b] = a[b] * 0.0625f;
                    asum[b] += a[b];
                }
#pragma unroll
                for (int wi = 0; wi < 4; wi++) {
                    const uint32_t wd = q[r][wi];
                    const uint32_t lo = and_opaque(wd, 0x0F0F0F0Fu);
                    const uint32_t hi = and_opaque(wd, 0xF0F0F0F0u);
#pragma unroll
                    for (int bb = 0; bb < 4; bb++) {
                        const float fl = (float)((lo >> (8 * bb)) & 0xFFu);
                        const float fh = (float)((hi >> (8 * bb)) & 0xFFu);
#pragma unroll
                        for (int b = 0; b < NB; b++) {
                            acc[b][wi * 8 + bb * 2] = fmaf(a[b], fl, acc[b][wi * 8 + bb * 2]);
                            acc[b][wi * 8 + bb * 2 + 1] = fmaf(a16[b], fh, acc[b][wi * 8 + bb * 2 + 1]);
                        }
                    }
                }
            }
            // keep each row's arithmetic behind its own load: the compiler
            // would otherwise hoist later rows' work and wait for their loads
            // too (2048 x 6144: 4.48 -> 4.20 us).  With two rows per thread
            // the lost interleaving costs more than the earlier start.
            if constexpr (R >= 4) __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (!WAVE_GROUPS) {
#pragma unroll
            for (int b = 0; b < NB; b++) {
                const float off = -8.0f * asum[b];
#pragma unroll
                for (int j = 0; j < 32; j++) acc[b][j] += off;
            }
        }

        if constexpr (WAVE_GROUPS) {
            // the whole wave holds one group: its -8 * sum(a) offset is added
            // once to each column sum, not to every lane's 32 partials
            float off[NB];
#pragma unroll
            for (int b = 0; b < NB; b++) off[b] = -8.0f * wave_sum_dpp(asum[b]);
            wave_rs32<NB>(acc, lane);
            if (lane < 32) {
                const int col = wave_rs_col(lane);
#pragma unroll
                for (int b = 0; b < NB; b++) red[(wv * NB + b) * 32 + col] = acc[b][0] + off[b];
            }
            __syncthreads();
            // column sums straight from the per-wave partials, waves in fixed order
            if constexpr (WaveEpi<Epi>::v) {
                static_assert(NB == 1, "wave epilogue: one row");
                if (wv == 0) {
                    const auto y = [&](int cc) {
                        float v = 0.0f;
#pragma unroll
                        for (int i = 0; i < NW / GB; i++) v += red[(i * GB + (cc >> 5)) * 32 + (cc & 31)];
                        return v;
                    };
                    epi.wave(s, c, C, y, lane);
                }
            } else {
                for (int col = t; col < NB * C; col += T) {
                    const int b = col / C, cc = col - b * C;
                    const auto y = [&](int j) {
                        float v = 0.0f;
#pragma unroll
                        for (int i = 0; i < NW / GB; i++) v += red[((i * GB + (j >> 5)) * NB + b) * 32 + (j & 31)];
                        return v;
                    };
                    epi(s, b, c, cc, C, y);
                }
            }
        } else {
            int base = 0;
            rs_steps<GB, 32, NB>(acc, lane, base);
            if ((lane & DUP) == 0) {
#pragma unroll
                for (int b = 0; b < NB; b++)
#pragma unroll
                    for (int i = 0; i < CNTF; i++)
                        red[(wv * NB + b) * C + gl * 32 + base + i] = acc[b][i];
            }
            __syncthreads();
            for (int col = t; col < NB * C; col += T) {
                const int b = col / C, cc = col - b * C;
                float y = 0.0f;
#pragma unroll
                for (int i = 0; i < NW; i++) y += red[(i * NB + b) * C + cc];
                ybuf[col] = y;
            }
            __syncthreads();
            if constexpr (WaveEpi<Epi>::v) {
                static_assert(NB == 1, "wave epilogue: one row");
                if (wv == 0) epi.wave(s, c, C, [&](int j) { return ybuf[j]; }, lane);
            } else {
                for (int col = t; col < NB * C; col += T) {
                    const int b = col / C, cc = col - b * C;
                    epi(s, b, c, cc, C, [&](int j) { return ybuf[b * C + j]; });
                }
            }
        }
        pro.finish(s, c, w.CT);
    }
}

template <int T, int GB, int R, int NB, class Pro, class Epi>
__global__ void __launch_bounds__(T) k_gemv(Q4Tiled w, Pro pro, Epi epi)
{
    gemv_tile<T, GB, R, NB>(w, pro, epi, blockIdx.x);
}

// A prologue that only supports one workgroup size declares it as
// `static constexpr int kOnlyT`; other tile shapes are then rejected.
template <class P, class = void>
struct OnlyT { static constexpr int v = 0; };
template <class P>
struct OnlyT<P, std::void_t<decltype(P::kOnlyT)>> { static constexpr int v = P::kOnlyT; };

template <int NB, class Pro, class Epi>
static hipError_t launch_gemv(const Q4Tiled &w, const Pro &pro, const Epi &epi, hipStream_t st, int rows = 1)
{
    const dim3 grid(w.S * w.CT, rows);
#define QTTS_GEMV_CASE(CFG)                                                                     \
    case CFG: {                                                                                 \
        constexpr TileShape ts = tile_shape(CFG);                                               \
        if constexpr (OnlyT<Pro>::v == 0 || OnlyT<Pro>::v == ts.T) {                            \
            hipLaunchKernelGGL((k_gemv<ts.T, ts.GB, ts.R, NB, Pro, Epi>), grid, dim3(ts.T), 0, st, w, pro, epi); \
        } else {                                                                                \
            return hipErrorInvalidValue;                                                        \
        }                                                                                       \
        break;                                                                                  \
    }
    switch (w.cfg) {
        QTTS_GEMV_CASE(TILE_G8_T256)
        QTTS_GEMV_CASE(TILE_G8_T128)
        QTTS_GEMV_CASE(TILE_G1_T64)
        QTTS_GEMV_CASE(TILE_G1_T128)
        QTTS_GEMV_CASE(TILE_G1_T256)
        QTTS_GEMV_CASE(TILE_G1_T384)
        QTTS_GEMV_CASE(TILE_G1_T768)
        QTTS_GEMV_CASE(TILE_G2_T256)
        QTTS_GEMV_CASE(TILE_G2_T512)
        QTTS_GEMV_CASE(TILE_G4_T256)
        QTTS_GEMV_CASE(TILE_G1_T512)
        QTTS_GEMV_CASE(TILE_G1_T256_R4)
        QTTS_GEMV_CASE(TILE_G1_T256_R2)
        QTTS_GEMV_CASE(TILE_G1_T512_R4)
        QTTS_GEMV_CASE(TILE_G2_T512_R4)
        QTTS_GEMV_CASE(TILE_G1_T512_R2)
        QTTS_GEMV_CASE(TILE_G2_T256_R4)
        QTTS_GEMV_CASE(TILE_G1_T1024_R2)
        QTTS_GEMV_CASE(TILE_G2_T1024_R4)
    default: return hipErrorInvalidValue;
    }
#undef QTTS_GEMV_CASE
    return hipGetLastError();
}

// y[b][j] = (resid ? y : 0) + sum_s part[s][b][j] (+ bias[j]); summation in
// slice order, then the residual/bias add, as gemv.rs:340-345 then the
// caller's `+=` (talker.rs:110, code_predictor.rs:55).
__global__ void k_reduce_parts(const float *part, int S, int NB, int npad, int n,
                               float *y, int ld, const float *bias, int resid)
{
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    const int b = blockIdx.y;
    if (j >= n) return;
    // columns past the last whole 32-column group (j >= npad) have no
    // partials and stay zero, as gemv.rs:255 leaves them
    float v = 0.0f;
    if (j < npad) {
#pragma unroll 8
        for (int s = 0; s < S; s++) v += part[((size_t)s * NB + b) * npad + j];
    }
    float *o = y + (size_t)b * ld + j;
    if (resid) v = *o + v;
    if (bias) v += bias[j];
    *o = v;
}

static hipError_t reduce_parts(const float *part, int S, int NB, int npad, int n, float *y,
                               int ld, const float *bias, int resid, hipStream_t st)
{
    hipLaunchKernelGGL(k_reduce_parts, dim3((n + 255) / 256, NB), dim3(256), 0, st, part, S, NB,
                       npad, n, y, ld, bias, resid);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// paged talker KV cache and RoPE
// ---------------------------------------------------------------------------


// rotate-half pair (i, i+64) of one head held in buf (rope.rs:79-92)
__device__ __forceinline__ float rope_rotate(const float *buf, int d, const float *cs, const float *sn)
{
    if (d < 64) return buf[d] * cs[d] - buf[d + 64] * sn[d];
    return buf[d] * cs[d - 64] + buf[d - 64] * sn[d - 64];
}

// q heads 2h, 2h+1 and k, v of KV head h from the fused q|k|v partials:
// sums over slices, QK-norm (talker.rs:89-99), RoPE at the table row cs/sn.
// Thread t: d = t & 127; threads 0..127 own q(2h) and k, 128..255 q(2h+1)
// and v.  Leaves the roped q in qr[upper][d]; returns k (normed, roped) or
// v (raw).
__device__ __forceinline__ float qkv_head_prologue(const float *part, int S, int NBP, int b, int npad,
                                                   const uint16_t *qn_g, const uint16_t *kn_g,
                                                   const float *cs, const float *sn, int h,
                                                   float (*qr)[HEAD_DIM], float (*vb)[HEAD_DIM],
                                                   float *scratch)
{
    const int t = threadIdx.x, d = t & 127, upper = t >> 7;
    const int wv = t >> 6, lane = t & 63;
    const int qcol = (2 * h + upper) * HEAD_DIM + d;
    const int kvcol = 16 * HEAD_DIM + upper * 8 * HEAD_DIM + h * HEAD_DIM + d;   // k | v
    float qv = 0.0f, kvv = 0.0f;
#pragma unroll 4
    for (int s = 0; s < S; s++) {
        const float *p = part + ((size_t)s * NBP + b) * npad;
        qv += p[qcol];
        kvv += p[kvcol];
    }
    const float qsq = wave_sum(qv * qv);
    const float ksq = wave_sum(kvv * kvv);
    __syncthreads();
    if (lane == 0) { scratch[wv] = qsq; scratch[4 + wv] = ksq; }
    __syncthreads();
    const float ssq = upper ? scratch[2] + scratch[3] : scratch[0] + scratch[1];
    const float ssk = scratch[4] + scratch[5];
    const float qn = qv * (1.0f / sqrtf(ssq / 128.0f + 1e-6f)) * h2f(qn_g[d]);
    vb[upper][d] = qn;
    if (!upper) vb[2][d] = kvv * (1.0f / sqrtf(ssk / 128.0f + 1e-6f)) * h2f(kn_g[d]);
    __syncthreads();
    qr[upper][d] = rope_rotate(vb[upper], d, cs, sn);
    return upper ? kvv : rope_rotate(vb[2], d, cs, sn);
}

// ---------------------------------------------------------------------------
// talker decode attention, split over 64-position pages (flash-decoding).
// Work item (chunk g of PG pages, kv head h): both query heads 2h, 2h+1
// share one pass over the pages' K and V (GQA, talker.rs:310).  All global
// loads are issued first (q/k/v partial sums, then the pages' K and V as
// 16-byte loads), so the q/k/v prologue (QK-norm, RoPE) runs while the pages
// stream in.  The item owning the newest position appends K (normed, roped)
// and V (raw) (talker.rs:299-302) and patches that row in its registers (the
// page was read before the append).  Writes per (chunk, query head) the max
// score, the exp-sum and the unnormalised P.V.
//
// Four waves per page: wave w takes page PG*g + w/4 and its rows
// 16(w%4)..+15; lane l holds dims 4(l%32)..+4 of rows 16(w%4) + 8(l/32) + i,
// i = 0..7, of both K and V, so every load instruction reads two whole
// 512-byte rows.  A row's score is the sum of 32 lanes' 4-dim partial dot
// products: a reduce-scatter over those lanes leaves the score of (head
// (l>>3)&1, row i = l&7) in lanes l and l^16.  Each wave forms its own
// softmax pieces (max, exp, sum, P.V over its 16 rows); one barrier then
// merges the waves, rescaled to the chunk maximum.  A wave whose page is past
// the cache's end re-reads the rows of the chunk's first page (same lines,
// no extra HBM traffic) and masks every row.
// ---------------------------------------------------------------------------

// One halving step of a reduce-scatter of N values across lanes: keep the
// upper half when `sel`, adding the partner's copy (DPP exchange CTRL).
template <int H, int CTRL, int N>
__device__ __forceinline__ void rs_step_n(float (&v)[N], bool sel)
{
#pragma unroll
    for (int j = 0; j < H; j++) {
        const float lo = v[j] + dpp_mov<CTRL>(v[j]);
        const float hi = v[j + H] + dpp_mov<CTRL>(v[j + H]);
        v[j] = sel ? hi : lo;
    }
}

// The q|k|v of the step arrive either as the q|k|v GEMV's k-slice partials
// (`part`, written by an earlier launch) or, when the GEMV runs in the same
// launch (LL), as (epoch, value) words `ll[s][col]` that its tiles store
// with system-scope atomics: the attention workgroups poll their words
// after issuing the page loads, so the pages stream in while the GEMV is
// still running.  A word is current when its epoch is *seq + 1; the o-proj
// launch that follows advances *seq, so words of an earlier launch never
// match.  Polls are bounded (LL_SPIN_MAX).

template <int PG, bool LL>
__device__ __forceinline__ void
talker_attn_body(const float *part, int S, int npad, const uint16_t *qn_g, const uint16_t *kn_g,
                 const float *rope_cos, const float *rope_sin, const DevState *st, int64_t pos_ovr,
                 int slot_ovr, int layer, KvPaged kv, float *am, float *al, float *aacc,
                 const uint64_t *ll, const uint32_t *seq, int bid)
{
    static_assert(PG == 1 || PG == 2, "one or two pages per workgroup");
    constexpr int NWV = 4 * PG;
    __shared__ __attribute__((aligned(16))) float qr[2][HEAD_DIM];
    __shared__ __attribute__((aligned(16))) float knew[HEAD_DIM];
    __shared__ __attribute__((aligned(16))) float vnew[HEAD_DIM];
    __shared__ __attribute__((aligned(16))) float pw[NWV][2][2][8];   // [wave][head][half][row] probabilities
    __shared__ float wml[NWV][2][2];                                   // [wave][head][max, sum]
    __shared__ __attribute__((aligned(16))) float ored[NWV][2][HEAD_DIM];
    const int t = threadIdx.x, lane = t & 63, wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wp = wv >> 2, wq = wv & 3;           // page of the chunk, row block of the page
    const int half = lane >> 5, dl = lane & 31, d4 = 4 * dl;
    const int row0 = 16 * wq + 8 * half;           // this lane's rows row0 + i, i = 0..7
    // the page-table entries of this workgroup's chunk (the wave's page and
    // the chunk's first page; the grid never exceeds the table) are read
    // beside the sequence length; the pages themselves only once the length
    // shows which are in use
    const int g = bid >> 3, h = bid & 7;
    const int c = PG * g + wp;                     // this wave's page
    const int pgw = kv.ptab[min(c, MAX_CHUNKS - 1)];
    const int pgf = kv.ptab[min(PG * g, MAX_CHUNKS - 1)];
    asm volatile("" ::: "memory");               // keeps the loads above the length's
    // position and length in one load (the device state's first 16 bytes),
    // so the RoPE values do not wait a second round trip
    const u32x4 sv = *(const u32x4 *)st;
    // the other arguments now, not after the length's wait
    asm volatile("" ::"s"(part), "s"(qn_g), "s"(kn_g), "s"(rope_cos), "s"(rope_sin), "s"(kv.base), "s"(aacc),
                 "s"(am), "s"(al), "s"(S), "s"(npad), "s"(layer), "s"(kv.n_phys));
    uint32_t epoch = 0;
    bool give_up = false;
    if constexpr (LL) {
        epoch = *seq + 1;
        give_up = st->sync_err != 0;
    }
    const int slot = slot_ovr >= 0 ? slot_ovr : (int)sv[2];
    const int64_t pos = pos_ovr >= 0 ? pos_ovr : (int64_t)(((uint64_t)sv[1] << 32) | sv[0]);
    const int L = slot + 1;
    const int C = (L + KV_PAGE - 1) / KV_PAGE;     // pages in use
    // the grid covers the capacity: chunks past the length exit (the whole
    // workgroup, before any barrier)
    if (PG * g >= C) return;
    const float scale = 1.0f / sqrtf(128.0f);
    {
        const bool live = c < C;
        const int ntok = live ? min(KV_PAGE, L - c * KV_PAGE) : 0;
        const bool last = g == (C - 1) / PG;       // the chunk holding the newest position
        // ---- loads: the vector of the step (waves w%4 = 0, 1: q heads 2h,
        // 2h+1; 2: k head h; 3: v head h; waves past the first page load the
        // same and only read LDS), lane l holding dims l and l+64 (a
        // rotate-half pair), its gammas and RoPE values, then the page
        const int base = (wq < 2 ? 2 * h + wq : 16 + 8 * (wq - 2) + h) * HEAD_DIM + lane;
        float xa[RES_MAX_S], xb[RES_MAX_S];
        if constexpr (!LL) {
#pragma unroll
            for (int s = 0; s < RES_MAX_S; s++) {
                const float *p = part + (size_t)min(s, S - 1) * npad + base;
                xa[s] = p[0];
                xb[s] = p[64];
            }
        }
        const uint16_t *gam = wq < 2 ? qn_g : kn_g;
        const uint32_t ga = gam[lane], gb = gam[lane + 64];
        const float cs = rope_cos[pos * 64 + lane], sn = rope_sin[pos * 64 + lane];
        const int pg = live ? pgw : pgf;
        const float *Kp = kv_page_ptr(kv, layer, pg, row0, h, 0) + d4;
        const float *Vp = kv_page_ptr(kv, layer, pg, row0, h, 1) + d4;
        f32x4 kk[8], vv[8];
#pragma unroll
        for (int i = 0; i < 8; i++) kk[i] = ld4nt(Kp + i * HEAD_DIM);
#pragma unroll
        for (int i = 0; i < 8; i++) vv[i] = ld4nt(Vp + i * HEAD_DIM);
        // nothing below may be scheduled above the page loads: a wait for the
        // step's vectors there would hold the pages back a round trip
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (LL) {
            // the step's vector from the GEMV tiles of this launch: waves of
            // the second page only read LDS and skip the wait
            for (int s = 0; s < RES_MAX_S; s++) { xa[s] = 0.0f; xb[s] = 0.0f; }
            if (wv < 4) {
                for (int it = 0;; it++) {
                    bool ok = true;
#pragma unroll
                    for (int s = 0; s < RES_MAX_S; s++) {
                        if (s < S) {
                            const uint64_t *p = ll + (size_t)s * npad + base;
                            const uint64_t wa = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                            const uint64_t wb = __hip_atomic_load(p + 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                            ok = ok && (uint32_t)(wa >> 32) == epoch && (uint32_t)(wb >> 32) == epoch;
                            xa[s] = __uint_as_float((uint32_t)wa);
                            xb[s] = __uint_as_float((uint32_t)wb);
                        }
                    }
                    if (__all(ok) || give_up) break;
                    if (it >= LL_SPIN_MAX) {
                        if (lane == 0) const_cast<DevState *>(st)->sync_err = 1;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                }
            }
        }
        // ---- QK-norm (talker.rs:286-297) and RoPE (rope.rs:79-92) in
        // registers: the sum of squares is the dims 0..63 wave sum plus the
        // dims 64..127 wave sum, in that order
        float a = xa[0], b = xb[0];
#pragma unroll
        for (int s = 1; s < RES_MAX_S; s++) {
            a = s < S ? a + xa[s] : a;
            b = s < S ? b + xb[s] : b;
        }
        if constexpr (!LL) {
            for (int s = RES_MAX_S; s < S; s++) {
                const float *p = part + (size_t)s * npad + base;
                a += p[0];
                b += p[64];
            }
        }
        if (wq < 3) {
            const float ss = wave_sum_dpp(a * a) + wave_sum_dpp(b * b);
            const float r = 1.0f / sqrtf(ss / 128.0f + 1e-6f);
            const float na = a * r * h2f(ga), nb = b * r * h2f(gb);
            a = na * cs - nb * sn;
            b = nb * cs + na * sn;
        }
        if (wv < 4) {
            float *dst = wq < 2 ? qr[wq] : wq == 2 ? knew : vnew;
            dst[lane] = a;
            dst[lane + 64] = b;
            if (last && wv >= 2) {
                // append (talker.rs:299-302): K normed and roped, V raw
                float *row = kv_ptr(kv, layer, slot, h, wv - 2);
                row[lane] = a;
                row[lane + 64] = b;
            }
        }
        __syncthreads();
        if (c == C - 1) {
            // patch the stale row in registers (the page was read before the append)
            const int ts = slot - c * KV_PAGE;
            const f32x4 kn = *(const f32x4 *)&knew[d4], vn = *(const f32x4 *)&vnew[d4];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                kk[i] = row0 + i == ts ? kn : kk[i];
                vv[i] = row0 + i == ts ? vn : vv[i];
            }
        }
        // ---- 4-dim partial scores of the lane's 8 rows, both query heads,
        // then the reduce-scatter over the half's 32 lanes (partner masks 15,
        // 7, 3, 1 by DPP, then 16 by a row swap)
        const f32x4 q0 = *(const f32x4 *)&qr[0][d4], q1 = *(const f32x4 *)&qr[1][d4];
        float sc[16];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const f32x4 k = kk[i];
            sc[i] = fmaf(q0.x, k.x, fmaf(q0.y, k.y, fmaf(q0.z, k.z, q0.w * k.w)));
            sc[8 + i] = fmaf(q1.x, k.x, fmaf(q1.y, k.y, fmaf(q1.z, k.z, q1.w * k.w)));
        }
        rs_step_n<8, 0x140, 16>(sc, lane & 8);
        rs_step_n<4, 0x141, 16>(sc, lane & 4);
        rs_step_n<2, 0x1B, 16>(sc, lane & 2);
        rs_step_n<1, 0xB1, 16>(sc, lane & 1);
        const float dot = add_xor16_split(sc[0], sc[0]);
        const int hh = (lane >> 3) & 1, ri = lane & 7, row = row0 + ri;
        const bool valid = row < ntok;
        const float sv = valid ? dot * scale : -INFINITY;
        // ---- softmax_raw pieces over the wave's rows (gemv.rs:471-482)
        const float m0 = wave_max_dpp(hh == 0 ? sv : -INFINITY), m1 = wave_max_dpp(hh == 1 ? sv : -INFINITY);
        const float e = valid ? expf(sv - (hh ? m1 : m0)) : 0.0f;
        const bool first = (lane & 16) == 0;       // one of the two lanes holding each value
        const float l0 = wave_sum_dpp(first && hh == 0 ? e : 0.0f), l1 = wave_sum_dpp(first && hh == 1 ? e : 0.0f);
        if (first) pw[wv][hh][half][ri] = e;
        if (lane == 0) { wml[wv][0][0] = m0; wml[wv][0][1] = l0; wml[wv][1][0] = m1; wml[wv][1][1] = l1; }
        __builtin_amdgcn_wave_barrier();
        // ---- P.V over the lane's 8 rows and 4 dims, both heads
        const f32x4 pa0 = *(const f32x4 *)&pw[wv][0][half][0], pa1 = *(const f32x4 *)&pw[wv][0][half][4];
        const f32x4 pb0 = *(const f32x4 *)&pw[wv][1][half][0], pb1 = *(const f32x4 *)&pw[wv][1][half][4];
        const float p0[8] = {pa0.x, pa0.y, pa0.z, pa0.w, pa1.x, pa1.y, pa1.z, pa1.w};
        const float p1[8] = {pb0.x, pb0.y, pb0.z, pb0.w, pb1.x, pb1.y, pb1.z, pb1.w};
        f32x4 a0 = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, a1 = a0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const bool ok = row0 + i < ntok;             // rows past the page's end may hold anything
            const f32x4 v = vv[i];
            a0.x = ok ? fmaf(p0[i], v.x, a0.x) : a0.x; a0.y = ok ? fmaf(p0[i], v.y, a0.y) : a0.y;
            a0.z = ok ? fmaf(p0[i], v.z, a0.z) : a0.z; a0.w = ok ? fmaf(p0[i], v.w, a0.w) : a0.w;
            a1.x = ok ? fmaf(p1[i], v.x, a1.x) : a1.x; a1.y = ok ? fmaf(p1[i], v.y, a1.y) : a1.y;
            a1.z = ok ? fmaf(p1[i], v.z, a1.z) : a1.z; a1.w = ok ? fmaf(p1[i], v.w, a1.w) : a1.w;
        }
        // the two halves hold the same dims of rows 8 apart
        a0.x = add_xor32(a0.x); a0.y = add_xor32(a0.y); a0.z = add_xor32(a0.z); a0.w = add_xor32(a0.w);
        a1.x = add_xor32(a1.x); a1.y = add_xor32(a1.y); a1.z = add_xor32(a1.z); a1.w = add_xor32(a1.w);
        if (lane < 32) {
            *(f32x4 *)&ored[wv][0][d4] = a0;
            *(f32x4 *)&ored[wv][1][d4] = a1;
        }
        __syncthreads();
        if (t < 2 * HEAD_DIM) {
            // the waves merged at the chunk maximum, in wave order
            const int oh = t >> 7, d = t & 127;
            float M = wml[0][oh][0];
#pragma unroll
            for (int w = 1; w < NWV; w++) M = fmaxf(M, wml[w][oh][0]);
            float o = 0.0f, ls = 0.0f;
#pragma unroll
            for (int w = 0; w < NWV; w++) {
                const float f = expf(wml[w][oh][0] - M);   // 0 for a wave with no valid row
                o = fmaf(f, ored[w][oh][d], o);
                ls = fmaf(f, wml[w][oh][1], ls);
            }
            aacc[((size_t)g * 16 + 2 * h + oh) * HEAD_DIM + d] = o;
            if (d == 0) {
                am[(2 * h + oh) * MAX_CHUNKS + g] = M;
                al[(2 * h + oh) * MAX_CHUNKS + g] = ls;
            }
        }
    }
}

// q|k|v GEMV and decode attention in one launch (two pages per attention
// workgroup): workgroups [0, nq) are the GEMV's tiles, storing their column
// sums as (epoch, value) words; the rest are the attention's work items,
// which issue their page loads at once and then wait for their words.  The
// GEMV tiles come first in the grid, and workgroups are dispatched in index
// order, so every tile an attention workgroup waits for has been dispatched
// before it and never waits itself.
template <int T, int GB, int R>
__global__ void __launch_bounds__(512, 1)
k_talker_qkv_attn(Q4Tiled wq, ProResidRms<1, 2048> pro, EpiLL<1> epi, int nq, const uint16_t *qn_g,
                  const uint16_t *kn_g, const float *rope_cos, const float *rope_sin, const DevState *st,
                  int64_t pos_ovr, int slot_ovr, int layer, KvPaged kv, float *am, float *al, float *aacc)
{
    static_assert(T == 512, "the attention side runs 512 threads (two pages)");
    if ((int)blockIdx.x < nq) {
        // the epoch loaded now, waited for only by the epilogue
        EpiLL<1> e = epi;
        e.epoch = *epi.seq + 1;
        gemv_tile<T, GB, R, 1>(wq, pro, e, blockIdx.x);
        return;
    }
    talker_attn_body<2, true>(nullptr, wq.S, epi.npad, qn_g, kn_g, rope_cos, rope_sin, st, pos_ovr, slot_ovr,
                              layer, kv, am, al, aacc, epi.ll, epi.seq, blockIdx.x - nq);
}

template <int PG>
__global__ void __launch_bounds__(256 * PG, 2 / PG)
k_talker_attn(const float *part, int S, int npad, const uint16_t *qn_g, const uint16_t *kn_g,
              const float *rope_cos, const float *rope_sin, const DevState *st, int64_t pos_ovr,
              int slot_ovr, int layer, KvPaged kv, float *am, float *al, float *aacc)
{
    talker_attn_body<PG, false>(part, S, npad, qn_g, kn_g, rope_cos, rope_sin, st, pos_ovr, slot_ovr, layer, kv, am,
                                al, aacc, nullptr, nullptr, blockIdx.x);
}

// ---------------------------------------------------------------------------
// predictor: q|k|v partial sums -> QK-norm -> RoPE -> KV append -> causal
// attention over <= 16 positions, fused (code_predictor.rs:369-414,
// 457-498).  Grid: one workgroup per KV head; NB tokens at positions
// pos0..pos0+NB-1.  Output: attn[b][16*128] (final, normalised).
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(256)
k_pred_attn(const float *part, int S, int NB, int npad, const uint16_t *qn_g, const uint16_t *kn_g,
            const float *rope_cos, const float *rope_sin, int pos0, float *Kc, float *Vc,
            float *attn)
{
    __shared__ float scratch[16];
    __shared__ float vb[3][HEAD_DIM];
    __shared__ float qr[2][2][HEAD_DIM];          // [token][head][d]
    __shared__ float Ks[PRED_KV_CAP][HEAD_DIM], Vs[PRED_KV_CAP][HEAD_DIM];
    __shared__ float prob[2][2][PRED_KV_CAP];
    const int h = blockIdx.x, t = threadIdx.x;
    const int d = t & 127, upper = t >> 7;
    const size_t kvrow = 8 * HEAD_DIM;
    // earlier positions of this head, written by previous launches
    for (int i = t; i < pos0 * HEAD_DIM; i += blockDim.x) {
        const int p = i / HEAD_DIM, dd = i - p * HEAD_DIM;
        Ks[p][dd] = Kc[p * kvrow + h * HEAD_DIM + dd];
        Vs[p][dd] = Vc[p * kvrow + h * HEAD_DIM + dd];
    }
    for (int b = 0; b < NB; b++) {
        const int pos = pos0 + b;
        const float *cs = rope_cos + (size_t)pos * 64, *sn = rope_sin + (size_t)pos * 64;
        const float kvnew = qkv_head_prologue(part, S, NB, b, npad, qn_g, kn_g, cs, sn, h, qr[b], vb, scratch);
        if (!upper) {
            Ks[pos][d] = kvnew;
            Kc[pos * kvrow + h * HEAD_DIM + d] = kvnew;
        } else {
            Vs[pos][d] = kvnew;
            Vc[pos * kvrow + h * HEAD_DIM + d] = kvnew;
        }
    }
    __syncthreads();
    const float scale = 1.0f / sqrtf(128.0f);
    for (int b = 0; b < NB; b++) {
        const int len = pos0 + b + 1;
        // scores: thread -> (head hh, position p, 16-dim part j) = 2 x 16 x 8
        {
            const int hh = t >> 7, p = (t >> 3) & 15, j = t & 7;
            float dot = 0.0f;
            if (p < len) {
#pragma unroll
                for (int i = 0; i < 16; i++) dot = fmaf(qr[b][hh][j * 16 + i], Ks[p][j * 16 + i], dot);
            }
#pragma unroll
            for (int m = 4; m >= 1; m >>= 1) dot += __shfl_xor(dot, m);
            if (j == 0) prob[b][hh][p] = p < len ? dot * scale : -INFINITY;
        }
        __syncthreads();
        // softmax_raw (gemv.rs:471-482), sequential per head
        if (t < 2) {
            float *sv = prob[b][t];
            float m = -INFINITY;
            for (int p = 0; p < len; p++) m = fmaxf(m, sv[p]);
            float sum = 0.0f;
            for (int p = 0; p < len; p++) { sv[p] = expf(sv[p] - m); sum += sv[p]; }
            const float inv = 1.0f / sum;
            for (int p = 0; p < len; p++) sv[p] *= inv;
        }
        __syncthreads();
        {
            const int hh = t >> 7;
            float o = 0.0f;
            for (int p = 0; p < len; p++) o += prob[b][hh][p] * Vs[p][d];
            attn[(size_t)b * 16 * HEAD_DIM + (2 * h + hh) * HEAD_DIM + d] = o;
        }
    }
}

// Predictor o-proj prologue with the attention fused in (code_predictor.rs:
// 369-414, 457-498).  The workgroup owning o-proj input rows k0..k0+511
// (query heads 4s..4s+3, kv heads h0 = 2s, h0 + 1) rebuilds those heads'
// q, k, v from the qkv partial sums, attends over the cached positions plus
// the new ones (causal among the NB new rows) and leaves the normalised
// attention output in xs.  Wave w owns query head 4s + w and one more head
// vector (w = 0, 1: k of kv head h0 + w; w = 2, 3: v of kv head h0 + w - 2);
// lane l holds dims l and l + 64, the two halves of a rotate-half RoPE pair,
// so QK-norm is a wave sum and RoPE stays in registers.  Column tile 0
// appends the new K (normed, roped) and V (raw) to the cache; no workgroup
// of the same launch reads those entries back from memory.
// Needs T == 256, KC == 512 and exactly MS qkv k-slices.
//
// TAB (layer 0 of steps 1..14): q|k|v come from a table row instead of the
// partial sums, chosen by the code the previous head's argmax candidates
// give (or the forced code), the table holding layer 0's q|k|v of every code
// (slice sums, so MS = 1 reads the bits the partials would give); the
// workgroup then records the code as the skipped q|k|v launch's prologue did
// and the slice-0 workgroups write the layer's residual input row to x_out.
//
// LL (q|k|v GEMV in the same launch, k_pred_qkv_attn_o): q|k|v arrive as the
// GEMV tiles' (epoch, value) words ll[s][col] instead of partial sums; the
// fetch issues everything else, and the load stage polls the words (bounded,
// as in the talker's fused launch) once the weights are in flight.
template <int NB, int MS, bool TAB = false, bool LL = false>
struct ProPredAttn {
    static_assert(!TAB || (NB == 1 && MS == 1), "table rows: one row, slice sums");
    static_assert(!LL || !TAB, "words or a table row, not both");
    static constexpr int kOnlyT = 256;   // launch_gemv instantiates 256-thread tiles only
    static constexpr int HPW = 2;        // kv heads per workgroup
    static constexpr int NC4 = HPW * PRED_KV_CAP * (HEAD_DIM / 4) / 256;   // cached float4 per thread
    const float *part;       // qkv partial sums [S][NB][npad]
    int S, npad;
    const uint16_t *qn_g, *kn_g;
    const float *rope_cos, *rope_sin;
    int pos0;                // position of row 0
    float *Kc, *Vc;          // this layer's cache [PRED_KV_CAP][8][HEAD_DIM]
    // TAB only
    const float *tab;        // [rows][npad] q|k|v of each code
    int rows;
    const float2 *cand;      // previous head's argmax candidates
    int ncand;
    DevState *st;
    int slot;
    uint32_t *codes_api;
    const float *xtab;       // [rows][xk] the layer's input row of each code
    float *x_out;
    int xk;
    // LL only (st above takes sync_err)
    const uint64_t *ll;      // [S][npad] q|k|v words
    const uint32_t *seq;
    uint32_t *adv;           // an epoch counter advanced once per launch (the MLP launch's), or null

    __device__ static uint32_t *code_lds()
    {
        __shared__ uint32_t code;
        return &code;
    }

    template <int T, int KC>
    struct Fetch {
        float q[NB][MS][2], kv[NB][MS][2];
        uint32_t gq[2], gk[2];
        float cs[NB], sn[NB];
        f32x4 kc[NC4], vc[NC4];
        uint32_t pred, used;
        bool nan;
        uint32_t epoch;
        int give_up;
    };
    template <int T, int KC>
    __device__ void fetch(Fetch<T, KC> &f, int k0, int ctile) const
    {
        const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
        const int h0 = k0 / (2 * HEAD_DIM);
        const int plast = pos0 > 0 ? pos0 - 1 : 0;
        // cached positions 0..pos0-1 of both kv heads: float4 i -> (head j, position p, dims 4*d4..)
#pragma unroll
        for (int u = 0; u < NC4; u++) {
            const int i = t + u * 256, j = i >> 9, p = (i >> 5) & 15, d4 = i & 31;
            const int off = min(p, plast) * (8 * HEAD_DIM) + (h0 + j) * HEAD_DIM + d4 * 4;
            f.kc[u] = ld4(Kc + off);
            f.vc[u] = ld4(Vc + off);
        }
        const int qcol = (2 * h0 + wv) * HEAD_DIM + lane;
        const int kvcol = 16 * HEAD_DIM + (wv >> 1) * 8 * HEAD_DIM + (h0 + (wv & 1)) * HEAD_DIM + lane;
        const float *pbase = part;
        if constexpr (TAB) {
            f.nan = false;
            if (cand) {
                const int force = st->force;
                const uint32_t fc = st->fcode[slot];
                f.pred = cand_argmax(cand, ncand, f.nan);
                f.used = force ? fc : f.pred;
            } else {
                f.pred = f.used = st->used[slot];
            }
            pbase = tab + (size_t)min(f.used, (uint32_t)(rows - 1)) * npad;
        }
        if constexpr (LL) {
            f.epoch = *seq + 1;
            f.give_up = st->sync_err;
        } else {
#pragma unroll
            for (int s = 0; s < MS; s++)
#pragma unroll
                for (int b = 0; b < NB; b++) {
                    const float *pp = pbase + (s * NB + b) * npad;
                    f.q[b][s][0] = pp[qcol];
                    f.q[b][s][1] = pp[qcol + 64];
                    f.kv[b][s][0] = pp[kvcol];
                    f.kv[b][s][1] = pp[kvcol + 64];
                }
        }
        f.gq[0] = qn_g[lane];
        f.gq[1] = qn_g[lane + 64];
        f.gk[0] = kn_g[lane];
        f.gk[1] = kn_g[lane + 64];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            f.cs[b] = rope_cos[(pos0 + b) * 64 + lane];
            f.sn[b] = rope_sin[(pos0 + b) * 64 + lane];
        }
    }
    template <int T, int KC>
    __device__ void load(const Fetch<T, KC> &f, float *xs, int k0, int ctile) const
    {
        __shared__ float Ks[HPW * PRED_KV_CAP * HEAD_DIM], Vs[HPW * PRED_KV_CAP * HEAD_DIM];
        __shared__ float qr[NB * 4 * HEAD_DIM];
        const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
        const int h0 = k0 / (2 * HEAD_DIM);
        const bool isk = wv < 2;
        const int jn = wv & 1;                       // kv head offset of this wave's k / v vector
        if constexpr (TAB) {
            if (t == 0) {
                *code_lds() = f.used;                // read by finish, after the GEMV's barriers
                if (cand && k0 == 0 && ctile == 0) {
                    st->pred[slot] = f.pred;
                    st->used[slot] = f.used;
                    st->prev[slot] = f.used;
                    if (f.nan) st->nan_flag = 1;
                    if (codes_api) codes_api[slot - 1] = f.pred;
                }
            }
        }
        // cached K / V rows into LDS
#pragma unroll
        for (int u = 0; u < NC4; u++) {
            const int i = t + u * 256, j = i >> 9, p = (i >> 5) & 15, d4 = i & 31;
            if (p < pos0) {
                *(f32x4 *)(Ks + (j * PRED_KV_CAP + p) * HEAD_DIM + d4 * 4) = f.kc[u];
                *(f32x4 *)(Vs + (j * PRED_KV_CAP + p) * HEAD_DIM + d4 * 4) = f.vc[u];
            }
        }
        const float gq0 = h2f(f.gq[0]), gq1 = h2f(f.gq[1]), gk0 = h2f(f.gk[0]), gk1 = h2f(f.gk[1]);
        float wq[NB][MS][2], wkv[NB][MS][2];
        if constexpr (LL) {
            const int qcol = (2 * h0 + wv) * HEAD_DIM + lane;
            const int kvcol = 16 * HEAD_DIM + (wv >> 1) * 8 * HEAD_DIM + (h0 + (wv & 1)) * HEAD_DIM + lane;
            for (int it = 0;; it++) {
                bool ok = true;
#pragma unroll
                for (int s = 0; s < MS; s++)
#pragma unroll
                    for (int b = 0; b < NB; b++) {
                        const uint64_t *pp = ll + ((size_t)s * NB + b) * npad;
                        const uint64_t w0 = __hip_atomic_load(pp + qcol, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                        const uint64_t w1 =
                            __hip_atomic_load(pp + qcol + 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                        const uint64_t w2 = __hip_atomic_load(pp + kvcol, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                        const uint64_t w3 =
                            __hip_atomic_load(pp + kvcol + 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                        ok = ok && (uint32_t)(w0 >> 32) == f.epoch && (uint32_t)(w1 >> 32) == f.epoch &&
                             (uint32_t)(w2 >> 32) == f.epoch && (uint32_t)(w3 >> 32) == f.epoch;
                        wq[b][s][0] = __uint_as_float((uint32_t)w0);
                        wq[b][s][1] = __uint_as_float((uint32_t)w1);
                        wkv[b][s][0] = __uint_as_float((uint32_t)w2);
                        wkv[b][s][1] = __uint_as_float((uint32_t)w3);
                    }
                if (__all(ok) || f.give_up) break;
                if (it >= LL_SPIN_MAX) {
                    if (lane == 0) st->sync_err = 1;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
        } else {
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int s = 0; s < MS; s++) {
                    wq[b][s][0] = f.q[b][s][0]; wq[b][s][1] = f.q[b][s][1];
                    wkv[b][s][0] = f.kv[b][s][0]; wkv[b][s][1] = f.kv[b][s][1];
                }
        }
#pragma unroll
        for (int b = 0; b < NB; b++) {
            // k-slice sums in slice order
            float q0 = wq[b][0][0], q1 = wq[b][0][1], v0 = wkv[b][0][0], v1 = wkv[b][0][1];
#pragma unroll
            for (int s = 1; s < MS; s++) {
                q0 += wq[b][s][0]; q1 += wq[b][s][1];
                v0 += wkv[b][s][0]; v1 += wkv[b][s][1];
            }
            // QK-norm over the head's 128 dims (talker.rs:89-99; code_predictor.rs:84-93)
            const float iq = 1.0f / sqrtf(wave_sum_dpp(q0 * q0 + q1 * q1) / 128.0f + 1e-6f);
            const float ik = 1.0f / sqrtf(wave_sum_dpp(v0 * v0 + v1 * v1) / 128.0f + 1e-6f);
            const float a0 = q0 * iq * gq0, a1 = q1 * iq * gq1;
            // rotate-half RoPE (rope.rs:79-92): pair (l, l + 64)
            const float cs = f.cs[b], sn = f.sn[b];
            qr[(b * 4 + wv) * HEAD_DIM + lane] = a0 * cs - a1 * sn;
            qr[(b * 4 + wv) * HEAD_DIM + lane + 64] = a1 * cs + a0 * sn;
            float n0 = v0, n1 = v1;                  // V stays raw
            if (isk) {
                const float c0 = v0 * ik * gk0, c1 = v1 * ik * gk1;
                n0 = c0 * cs - c1 * sn;
                n1 = c1 * cs + c0 * sn;
            }
            float *row = (isk ? Ks : Vs) + (jn * PRED_KV_CAP + pos0 + b) * HEAD_DIM;
            row[lane] = n0;
            row[lane + 64] = n1;
            if (ctile == 0) {
                float *cache = (isk ? Kc : Vc) + (pos0 + b) * (8 * HEAD_DIM) + (h0 + jn) * HEAD_DIM;
                cache[lane] = n0;
                cache[lane + 64] = n1;
            }
        }
        __syncthreads();
        // wave w = query head 4s + w (kv head h0 + w/2): lane -> position
        // p = lane/4 and a quarter of the head dims; softmax_raw
        // (gemv.rs:471-482) over the positions 0..len-1
        const int jw = wv >> 1, p = lane >> 2, q4i = lane & 3;
        const float scale = 1.0f / sqrtf(128.0f);
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const int len = pos0 + b + 1;
            const float *qrow = qr + (b * 4 + wv) * HEAD_DIM + q4i * 32;
            const float *krow = Ks + (jw * PRED_KV_CAP + p) * HEAD_DIM + q4i * 32;
            float dot = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; i += 4) {
                const f32x4 a = *(const f32x4 *)(qrow + i), c = *(const f32x4 *)(krow + i);
                dot = fmaf(a.x, c.x, dot);
                dot = fmaf(a.y, c.y, dot);
                dot = fmaf(a.z, c.z, dot);
                dot = fmaf(a.w, c.w, dot);
            }
            dot += dpp_mov<0xB1>(dot);
            dot += dpp_mov<0x4E>(dot);
            const float sc = p < len ? dot * scale : -INFINITY;
            const float m = wave_max_dpp(sc);
            const float e = p < len ? expf(sc - m) : 0.0f;
            const float prob = e * (1.0f / wave_sum_dpp(q4i == 0 ? e : 0.0f));
            float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
            for (int pp = 0; pp < PRED_KV_CAP; pp++) {
                const float w = lane_value(prob, 4 * pp);
                const float *vrow = Vs + (jw * PRED_KV_CAP + pp) * HEAD_DIM;
                const float x0 = vrow[lane], x1 = vrow[lane + 64];
                o0 = pp < len ? fmaf(w, x0, o0) : o0;
                o1 = pp < len ? fmaf(w, x1, o1) : o1;
            }
            xs[b * KC + wv * HEAD_DIM + lane] = o0;
            xs[b * KC + wv * HEAD_DIM + lane + 64] = o1;
        }
    }
    __device__ void finish(int s, int c, int nct) const
    {
        if (adv && s == 0 && c == 0 && threadIdx.x == 0) *adv = *adv + 1;
        if constexpr (TAB) {
            if (s != 0 || !x_out) return;
            const float *row = xtab + (size_t)min(*code_lds(), (uint32_t)(rows - 1)) * xk;
            const int per = (xk + nct - 1) / nct;
            const int j0 = c * per, j1 = min(j0 + per, xk);
            for (int j = j0 + threadIdx.x; j < j1; j += blockDim.x) x_out[j] = row[j];
        }
    }
};

// ---------------------------------------------------------------------------
// argmax over the lm-head logits (sample_argmax, code_predictor.rs:335-341):
// the LAST index among equal maxima.  Writes pred[slot]/used[slot]/prev.
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(1024)
k_argmax(const float *part, int S, int npad, int n, DevState *st, int slot,
         const uint32_t *forced, uint32_t *codes_api)
{
    __shared__ float bv[16];
    __shared__ int bi[16];
    __shared__ int nanf;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    if (t == 0) nanf = 0;
    __syncthreads();
    float best = -INFINITY;
    int bidx = -1;
    for (int j = t; j < n; j += blockDim.x) {
        float v = 0.0f;
#pragma unroll 4
        for (int s = 0; s < S; s++) v += part[(size_t)s * npad + j];
        if (isnan(v)) nanf = 1;
        if (bidx < 0 || v >= best) { best = v; bidx = j; }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = __shfl_xor(best, m);
        const int oi = __shfl_xor(bidx, m);
        if (oi >= 0 && (bidx < 0 || ov > best || (ov == best && oi > bidx))) { best = ov; bidx = oi; }
    }
    if (lane == 0) { bv[wv] = best; bi[wv] = bidx; }
    __syncthreads();
    if (t == 0) {
        float b = bv[0];
        int i0 = bi[0];
        for (int w = 1; w < (int)(blockDim.x >> 6); w++) {
            if (bi[w] >= 0 && (i0 < 0 || bv[w] > b || (bv[w] == b && bi[w] > i0))) { b = bv[w]; i0 = bi[w]; }
        }
        uint32_t code = i0 < 0 ? 0u : (uint32_t)i0;
        if (nanf) { st->nan_flag = 1; code = 0; }
        st->pred[slot] = code;
        uint32_t used = code;
        if (st->force && forced) used = forced[(size_t)(st->frame_idx - st->forced_base) * 16 + slot];
        st->used[slot] = used;
        st->prev[slot] = used;
        if (codes_api) codes_api[slot - 1] = code;
    }
}

// ---------------------------------------------------------------------------
// talker input for the next step (generate_new.rs:638-654), bit-exact:
// sum = 0; sum += e_g (g = 0..14); x = semantic + sum; x += text.
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(256)
k_combine(Q4Rows tcodec, Q4Rows cpemb, int n_groups, DevState *st, const float *text,
          const float *pad, float *x, int H, const float2 *cand_last, int ncand)
{
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    // the last code straight from the last head's argmax candidates (every
    // wave chooses it; workgroup 0 records it)
    uint32_t last = 0;
    if (cand_last) {
        bool nan;
        const uint32_t pred = cand_argmax(cand_last, ncand, nan);
        last = st->force ? st->fcode[n_groups] : pred;
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            st->pred[n_groups] = pred;
            st->used[n_groups] = last;
            st->prev[n_groups] = last;
            if (nan) st->nan_flag = 1;
        }
    }
    if (j >= H) return;
    // n_groups is 1..15 (checked at upload).  Every code and row value is
    // loaded first, then summed in group order: the 16 codes as eight 8-byte
    // loads, group g's code u[g + 1] for g < n_groups - 1 and the last
    // group's from the candidates (or u[n_groups]); groups past n_groups
    // repeat the last group's row (loaded, never summed).  No load sits
    // behind a branch, so none waits for another.
    constexpr int MAXG = 15;
    static_assert(offsetof(DevState, used) % 8 == 0, "codes as 8-byte loads");
    uint32_t u[16];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint2 w = ((const uint2 *)st->used)[i];
        u[2 * i] = w.x;
        u[2 * i + 1] = w.y;
    }
    uint32_t lastc = u[1];
#pragma unroll
    for (int i = 2; i < 16; i++) lastc = i == n_groups ? u[i] : lastc;
    if (cand_last) lastc = last;
    uint32_t code[MAXG];
#pragma unroll
    for (int g = 0; g < MAXG; g++) code[g] = g < n_groups - 1 ? u[g + 1] : lastc;
    const int f = st->frame_idx, n_text = st->n_text;
    const float sem = q4_row_value(tcodec, u[0], j);
    float val[MAXG];
#pragma unroll
    for (int g = 0; g < MAXG; g++) {
        const int gg = min(g, n_groups - 1);
        Q4Rows e = cpemb;
        e.packed += (size_t)gg * e.rows * e.G * 16;
        e.scales += (size_t)gg * e.rows * e.G;
        val[g] = q4_row_value(e, code[g], j);
    }
    float sum = 0.0f;
#pragma unroll
    for (int g = 0; g < MAXG; g++)
        if (g < n_groups) sum += val[g];
    float v = sem + sum;
    const float *tr = (f < n_text) ? text + (size_t)f * H : pad;
    v += tr[j];
    x[j] = v;
}

// The code of `slot` from an lm head's argmax candidates (API calls, where
// no frame combine follows the chain).
__global__ void __launch_bounds__(64)
k_cand_final(const float2 *cand, int ncand, DevState *st, int slot, uint32_t *codes_api)
{
    bool nan;
    const uint32_t pred = cand_argmax(cand, ncand, nan);
    if (threadIdx.x == 0) {
        const uint32_t used = st->force ? st->fcode[slot] : pred;
        st->pred[slot] = pred;
        st->used[slot] = used;
        st->prev[slot] = used;
        if (nan) st->nan_flag = 1;
        if (codes_api) codes_api[slot - 1] = pred;
    }
}

// code_predictor.rs:287-300 for the operator-level API.
__global__ void k_embed_sum(Q4Rows cpemb, int n_groups, const uint32_t *codes, float *out, int n)
{
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n) return;
    float sum = 0.0f;
    for (int g = 0; g < n_groups; g++) {
        Q4Rows e = cpemb;
        e.packed += (size_t)g * e.rows * e.G * 16;
        e.scales += (size_t)g * e.rows * e.G;
        sum += q4_row_value(e, codes[g], j);
    }
    out[j] = sum;
}

__global__ void k_embed_row(Q4Rows e, const uint32_t *code, uint32_t code_imm, float *out, int n)
{
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= n) return;
    out[j] = q4_row_value(e, code ? *code : code_imm, j);
}

__global__ void k_silu(float *x, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = silu_f(x[i]);
}

// ---------------------------------------------------------------------------
// sampler (sample_token, generate_new.rs:771-862) in one workgroup of four
// waves.  Thread t holds entries 16t..16t+15 in registers, so "index order"
// is thread order then register order.  The repetition penalty is applied
// per history entry (a count per token, the same division repeated); top-k
// keeps the k largest probabilities with ties broken by lower index (Rust's
// stable sort): a radix select over the probability bits (8 bits a pass,
// per-wave histograms, the bin scan on one wave) finds the k-th largest,
// then equal values are admitted in index order.  Top-p sorts the kept
// entries (bitonic, rank = (p desc, index asc)).  The draw walks nonzero
// probabilities in index order.
// ---------------------------------------------------------------------------

constexpr int SAMP_MAX = 4096;
constexpr int SAMP_T = 256;
constexpr int SAMP_E = SAMP_MAX / SAMP_T;        // entries per thread
static_assert(SAMP_MAX % 16 == 0, "the draw reads blocks of 16");

__device__ __forceinline__ bool rank_before(float pa, int ia, float pb, int ib)
{
    return pa > pb || (pa == pb && ia < ib);
}

__device__ void bitonic_sort_desc(float *kp, int *ki, int N)
{
    for (int k = 2; k <= N; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < N; i += blockDim.x) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const bool up = (i & k) == 0;
                    const float pa = kp[i], pb = kp[ixj];
                    const int ia = ki[i], ib = ki[ixj];
                    const bool swap = up ? rank_before(pb, ib, pa, ia) : rank_before(pa, ia, pb, ib);
                    if (swap) { kp[i] = pb; kp[ixj] = pa; ki[i] = ib; ki[ixj] = ia; }
                }
            }
            __syncthreads();
        }
    }
}

__device__ __forceinline__ float simple_rand_dev(uint64_t &s)
{
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    return (float)s / 18446744073709551616.0f;   // (state as f32) / (u64::MAX as f32)
}

struct SampleArgs {
    float temperature, top_p, rep;
    int top_k;
    const uint32_t *prev;
    int n_prev;
};

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_int(int v)
{
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xF, false);
}

// Exclusive prefix sum of one int per lane in lane order; *total = the
// wave's sum.  On the VALU: row shifts by 1, 2, 4 and 8 scan each 16-lane
// row (lanes without a source add 0), then row_bcast:15 adds row r's total
// to row r + 1 (rows 1 and 3) and row_bcast:31 adds lane 31 to rows 2 and 3.
__device__ __forceinline__ int wave_excl_scan(int v, int *total)
{
    int x = v;
    x += dpp_int<0x111, 0xF>(x);
    x += dpp_int<0x112, 0xF>(x);
    x += dpp_int<0x114, 0xF>(x);
    x += dpp_int<0x118, 0xF>(x);
    x += dpp_int<0x142, 0xA>(x);
    x += dpp_int<0x143, 0xC>(x);
    *total = __builtin_amdgcn_readlane(x, 63);
    return x - v;
}

// Four-wave block helpers, one barrier each.  Every call site passes its own
// 4-slot scratch, so no barrier is needed before the scratch is reused.
__device__ __forceinline__ int blk4_excl_scan(int v, int *wsum, int *total)
{
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    int wt;
    const int x = wave_excl_scan(v, &wt);
    if (lane == 0) wsum[wv] = wt;
    __syncthreads();
    int base = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int s = wsum[i];
        base += i < wv ? s : 0;
        tot += s;
    }
    if (total) *total = tot;
    return base + x;
}

__device__ __forceinline__ float blk4_sum(float v, float *red)
{
    v = wave_sum_dpp(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ float blk4_max(float v, float *red)
{
    v = wave_max_dpp(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__global__ void __launch_bounds__(SAMP_T)
k_sampler(const float *logits, int n, DevState *st, int mode, SampleArgs api, uint64_t *rng_api,
          uint32_t *out_api, const uint32_t *forced)
{
    __shared__ __align__(16) float kp[SAMP_MAX];
    __shared__ __align__(16) int ki[SAMP_MAX];
    __shared__ __align__(16) int hist[2][4][256];
    __shared__ float redf[4][4];
    __shared__ int redi[4][4];
    __shared__ uint32_t sel_prefix, sel_mask;
    __shared__ int sel_need, sel_done, cutoff_s;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    // the logits and every state word the kernel reads are loaded up front
    // (the logits buffer is valid whatever the state holds)
    const int i0 = t * SAMP_E;
    float v[SAMP_E];
    if (i0 + SAMP_E <= n && ((uintptr_t)logits & 15) == 0) {
#pragma unroll
        for (int q = 0; q < SAMP_E / 4; q++) {
            const f32x4 a = ld4(logits + i0 + 4 * q);
            v[4 * q] = a.x; v[4 * q + 1] = a.y; v[4 * q + 2] = a.z; v[4 * q + 3] = a.w;
        }
    } else {
#pragma unroll
        for (int e = 0; e < SAMP_E; e++) {
            const float x = logits[min(i0 + e, n - 1)];
            v[e] = i0 + e < n ? x : -INFINITY;
        }
    }
    float temp, top_p, rep;
    int top_k, n_prev;
    const uint32_t *prev;
    uint64_t rs0;
    uint32_t tok0;   // history entry t, for t < min(n_prev, SAMP_T)
    int force = 0, eos_en = 0, fidx = 0, fbase = 0;
    uint32_t eos_id = 0;
    if (mode == 0) {
        if (st->stop) return;
        temp = st->frame_idx < st->onset_frames ? st->onset_temperature : st->temperature;
        top_p = st->top_p; rep = st->rep_penalty; top_k = st->top_k;
        prev = st->prev; n_prev = 16;
        tok0 = st->prev[min(t, 15)];
        rs0 = st->rng;
        force = st->force; eos_en = st->eos_enabled; eos_id = st->eos_id;
        fidx = st->frame_idx; fbase = st->forced_base;
    } else {
        temp = api.temperature; top_p = api.top_p; rep = api.rep; top_k = api.top_k;
        prev = api.prev; n_prev = api.n_prev;
        tok0 = n_prev > 0 ? prev[min(t, n_prev - 1)] : 0u;
        rs0 = *rng_api;
    }
    // repetition penalty (generate_new.rs:776-785): once per history entry
    if (rep != 1.0f && n_prev > 0) {
        for (int i = t; i < n; i += SAMP_T) ki[i] = 0;
        __syncthreads();
        for (int j = t; j < n_prev; j += SAMP_T) {
            const uint32_t tok = j < SAMP_T ? tok0 : prev[j];
            if (tok < (uint32_t)n) atomicAdd(&ki[tok], 1);
        }
        __syncthreads();
#pragma unroll
        for (int e = 0; e < SAMP_E; e++) {
            const int c = i0 + e < n ? ki[i0 + e] : 0;
            for (int k = 0; k < c; k++) v[e] = v[e] > 0.0f ? v[e] / rep : v[e] * rep;
        }
    }
    // temperature, softmax
    const bool use_t = temp != 1.0f && temp > 0.0f;
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < SAMP_E; e++) {
        if (use_t) v[e] = v[e] / temp;
        mx = fmaxf(mx, v[e]);
    }
    mx = blk4_max(mx, redf[0]);
    float sum = 0.0f;
#pragma unroll
    for (int e = 0; e < SAMP_E; e++) {
        const float ex = i0 + e < n ? expf(v[e] - mx) : 0.0f;
        v[e] = ex;
        sum += ex;
    }
    sum = blk4_sum(sum, redf[1]);
    int nan_l = 0;
#pragma unroll
    for (int e = 0; e < SAMP_E; e++) {
        const float q = v[e] / sum;
        nan_l |= (i0 + e < n) && isnan(q);
        v[e] = i0 + e < n ? q : 0.0f;
    }

    const bool do_k = top_k > 0 && top_k < n;
    const bool do_p = top_p > 0.0f && top_p < 1.0f;
    if (__syncthreads_or(nan_l) && (do_k || do_p)) {   // Rust panics in partial_cmp().unwrap()
        if (t == 0) {
            st->nan_flag = 1;
            if (mode == 0) st->stop = 1; else *out_api = 0;
        }
        return;
    }
    if (do_k) {
        uint32_t key[SAMP_E];
#pragma unroll
        for (int e = 0; e < SAMP_E; e++) key[e] = __float_as_uint(v[e]);
        for (int i = t; i < 4 * 256; i += SAMP_T) (&hist[0][0][0])[i] = 0;
        if (t == 0) { sel_prefix = 0; sel_mask = 0; sel_need = top_k; sel_done = 0; }
        __syncthreads();
        for (int pass = 0; pass < 4; pass++) {
            const int shift = 24 - 8 * pass;
            const uint32_t prefix = sel_prefix, mask = sel_mask;
            int *h = &hist[pass & 1][wv][0];
#pragma unroll
            for (int e = 0; e < SAMP_E; e++)
                if (i0 + e < n && (key[e] & mask) == prefix) atomicAdd(&h[(key[e] >> shift) & 0xFF], 1);
            for (int i = t; i < 4 * 256; i += SAMP_T) (&hist[(pass + 1) & 1][0][0])[i] = 0;
            __syncthreads();
            if (wv == 0) {
                // lane l scans bins 255-4l down to 252-4l; the bin holding
                // the need-th largest is where the running count crosses need
                const int b0 = 252 - 4 * lane;
                int c[4] = {0, 0, 0, 0};
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    const int4 q = *(const int4 *)&hist[pass & 1][w][b0];
                    c[0] += q.w; c[1] += q.z; c[2] += q.y; c[3] += q.x;
                }
                int wt;
                int above = wave_excl_scan((c[0] + c[1]) + (c[2] + c[3]), &wt);
                const int need = sel_need;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    if (above < need && above + c[q] >= need) {
                        sel_prefix = prefix | ((uint32_t)(b0 + 3 - q) << shift);
                        sel_mask = mask | (0xFFu << shift);
                        sel_need = need - above;
                        sel_done = above + c[q] == need;
                    }
                    above += c[q];
                }
            }
            __syncthreads();
            if (sel_done) break;
        }
        // keep entries above the selected bits, and the first sel_need equal
        // to them in index order
        const uint32_t prefix = sel_prefix, mask = sel_mask;
        const int need = sel_need;
        int eq = 0;
#pragma unroll
        for (int e = 0; e < SAMP_E; e++) eq += (i0 + e < n) && (key[e] & mask) == prefix;
        int before = blk4_excl_scan(eq, redi[0], nullptr);
        float s2 = 0.0f;
#pragma unroll
        for (int e = 0; e < SAMP_E; e++) {
            bool keep = false;
            if (i0 + e < n) {
                const uint32_t km = key[e] & mask;
                keep = km > prefix;
                if (km == prefix) keep = before++ < need;
            }
            if (!keep) v[e] = 0.0f;
            s2 += v[e];
        }
        s2 = blk4_sum(s2, redf[2]);
        if (s2 > 0.0f)
#pragma unroll
            for (int e = 0; e < SAMP_E; e++) v[e] = v[e] / s2;
    }
    if (do_p) {
        // rank the nonzero entries (after top-k at most top_k of them)
        uint8_t *drop = (uint8_t *)&hist[0][0][0];
        int c = 0;
#pragma unroll
        for (int e = 0; e < SAMP_E; e++) c += v[e] != 0.0f;
        int tot = 0;
        int o = blk4_excl_scan(c, redi[1], &tot);
#pragma unroll
        for (int e = 0; e < SAMP_E; e++)
            if (v[e] != 0.0f) { kp[o] = v[e]; ki[o] = i0 + e; o++; }
        int N = 1;
        while (N < tot) N <<= 1;
        for (int i = tot + t; i < N; i += SAMP_T) { kp[i] = -1.0f; ki[i] = 0x7fffffff; }
        for (int i = t; i < n; i += SAMP_T) drop[i] = 0;
        __syncthreads();
        bitonic_sort_desc(kp, ki, N);
        if (t == 0) {
            float cum = 0.0f;
            int cutoff = n;
            for (int r = 0; r < tot; r++) {
                cum += kp[r];
                if (cum >= top_p) { cutoff = r + 1; break; }
            }
            cutoff_s = cutoff < 1 ? 1 : cutoff;
        }
        __syncthreads();
        for (int r = cutoff_s + t; r < tot; r += SAMP_T) drop[ki[r]] = 1;
        __syncthreads();
        float s3 = 0.0f;
#pragma unroll
        for (int e = 0; e < SAMP_E; e++) {
            if (i0 + e < n && drop[i0 + e]) v[e] = 0.0f;
            s3 += v[e];
        }
        s3 = blk4_sum(s3, redf[3]);
        if (s3 > 0.0f)
#pragma unroll
            for (int e = 0; e < SAMP_E; e++) v[e] = v[e] / s3;
    }
    // compact nonzero probabilities in index order, then the cumulative draw
    int c = 0;
#pragma unroll
    for (int e = 0; e < SAMP_E; e++) c += v[e] != 0.0f;
    int total = 0;
    int o = blk4_excl_scan(c, redi[2], &total);
#pragma unroll
    for (int e = 0; e < SAMP_E; e++)
        if (v[e] != 0.0f) { kp[o] = v[e]; ki[o] = i0 + e; o++; }
    __syncthreads();
    if (t == 0) {
        uint64_t rs = rs0;
        const float r = simple_rand_dev(rs);
        float cs = 0.0f;
        uint32_t res = 0;
        bool found = false;
        // blocks of 16 read together, then summed in index order without
        // branches (entries past `total` are read, never summed: total <=
        // SAMP_MAX, a multiple of 16)
        for (int k = 0; k < total && !found; k += 16) {
            f32x4 q[4];
            int4 qi[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                q[j] = *(const f32x4 *)&kp[k + 4 * j];
                qi[j] = *(const int4 *)&ki[k + 4 * j];
            }
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const bool live = !found && k + j < total;
                const float c2 = cs + q[j >> 2][j & 3];
                const bool hit = live && r < c2;
                cs = live ? c2 : cs;
                res = hit ? (uint32_t)qi[j >> 2][j & 3] : res;
                found = found || hit;
            }
        }
        if (mode == 0) {
            st->rng = rs;
            st->pred[0] = res;
            uint32_t used = res;
            if (force && forced) {
                // this frame's forced codes, staged for the predictor chain
                const uint32_t *fr = forced + (size_t)(fidx - fbase) * 16;
                for (int i = 0; i < 16; i++) st->fcode[i] = fr[i];
                used = fr[0];
            }
            st->used[0] = used;
            st->prev[0] = used;
            if (eos_en && !force && res == eos_id) { st->stop = 1; st->eos = 1; }
        } else {
            *rng_api = rs;
            *out_api = res;
        }
    }
}

// ---------------------------------------------------------------------------
// end of a talker step: logits from the codec-head partials, the normed
// hidden kept, position and KV length advanced; in frame mode also the
// frame's codes recorded.
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(1024)
k_step_end(const float *part, int S, int npad, int V, const float *hid_work, int H, float *logits,
           float *hidden, DevState *st, int frame_mode, uint32_t *ring_pred, uint32_t *ring_used)
{
    const int t = threadIdx.x;
    if (frame_mode && st->stop) return;
    // V and npad are whole 32-column groups (checked at upload), V <= 4096.
    // The common case (up to four columns per thread, up to four slices,
    // up to two hidden values) issues every load before its first wait;
    // the loops below take the rest.
    constexpr int JV = 4, SV = 4, HV = 2;
    float pv[JV][SV], hv[HV];
#pragma unroll
    for (int q = 0; q < JV; q++)
#pragma unroll
        for (int s = 0; s < SV; s++)
            pv[q][s] = part[(size_t)min(s, S - 1) * npad + min(t + q * 1024, V - 1)];
#pragma unroll
    for (int q = 0; q < HV; q++) hv[q] = hid_work[min(t + q * 1024, H - 1)];
#pragma unroll
    for (int q = 0; q < JV; q++) {
        const int j = t + q * 1024;
        float v = pv[q][0];
#pragma unroll
        for (int s = 1; s < SV; s++)
            if (s < S) v += pv[q][s];
        for (int s = SV; s < S; s++) v += part[(size_t)s * npad + j];
        if (j < V) logits[j] = v;
    }
#pragma unroll
    for (int q = 0; q < HV; q++)
        if (t + q * 1024 < H) hidden[t + q * 1024] = hv[q];
    for (int j = t + HV * 1024; j < H; j += 1024) hidden[j] = hid_work[j];
    const int f = st->frame_idx;
    if (frame_mode && t < 16) {
        ring_pred[(size_t)(f - st->ring_base) * 16 + t] = st->pred[t];
        ring_used[(size_t)(f - st->ring_base) * 16 + t] = st->used[t];
    }
    __syncthreads();
    if (t == 0) {
        st->position += 1;
        st->kv_len += 1;
        if (frame_mode) st->frame_idx = f + 1;
    }
}

// ---------------------------------------------------------------------------
// KV cache copies between the paged layout and the reference layout
// [len][8][128] (gemv.rs:75-77).  Pure copies: bit-exact.
// ---------------------------------------------------------------------------

__global__ void k_kv_gather(KvPaged kv, int layer, int len, float *K, float *V)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)len * 8 * HEAD_DIM) return;
    const int pos = (int)(i / (8 * HEAD_DIM));
    const int rem = (int)(i - (size_t)pos * 8 * HEAD_DIM);
    const int h = rem / HEAD_DIM, d = rem % HEAD_DIM;
    K[i] = kv_ptr(kv, layer, pos, h, 0)[d];
    V[i] = kv_ptr(kv, layer, pos, h, 1)[d];
}

__global__ void k_kv_scatter(KvPaged kv, int layer, int len, const float *K, const float *V)
{
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)len * 8 * HEAD_DIM) return;
    const int pos = (int)(i / (8 * HEAD_DIM));
    const int rem = (int)(i - (size_t)pos * 8 * HEAD_DIM);
    const int h = rem / HEAD_DIM, d = rem % HEAD_DIM;
    kv_ptr(kv, layer, pos, h, 0)[d] = K[i];
    kv_ptr(kv, layer, pos, h, 1)[d] = V[i];
}

// ===========================================================================
// host-side enqueue functions
// ===========================================================================

#define QCHK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) return e_; } while (0)

hipError_t enqueue_gemv_plain(const Q4Tiled &w, const float *x, int NB, int ld, float *part,
                              hipStream_t st)
{
    if (NB == 1) return launch_gemv<1>(w, ProPlain<1>{x, ld, w.k}, EpiPart<1>{part, w.npad}, st);
    if (NB == 2) return launch_gemv<2>(w, ProPlain<2>{x, ld, w.k}, EpiPart<2>{part, w.npad}, st);
    return hipErrorInvalidValue;
}

hipError_t enqueue_gemv_store(const Q4Tiled &w, const float *x, float *y, const float *bias,
                              float *part, hipStream_t st)
{
    if (w.S == 1)
        return launch_gemv<1>(w, ProPlain<1>{x, w.k, w.k}, EpiStore<1>{y, w.n, w.n, bias}, st);
    QCHK(launch_gemv<1>(w, ProPlain<1>{x, w.k, w.k}, EpiPart<1>{part, w.npad}, st));
    return reduce_parts(part, w.S, 1, w.npad, w.n, y, w.n, bias, 0, st);
}

hipError_t enqueue_gemv_rows(const Q4Tiled &w, const float *X, int rows, float *Y, float *part,
                             hipStream_t st)
{
    for (int r = 0; r < rows; r += 2) {
        const int nb = rows - r >= 2 ? 2 : 1;
        QCHK(enqueue_gemv_plain(w, X + (size_t)r * w.k, nb, w.k, part, st));
        QCHK(reduce_parts(part, w.S, nb, w.npad, w.n, Y + (size_t)r * w.n, w.n, nullptr, 0, st));
    }
    return hipSuccess;
}

hipError_t enqueue_embed_row(const Q4Rows &e, const uint32_t *code_dev, uint32_t code, float *out,
                             hipStream_t st)
{
    hipLaunchKernelGGL(k_embed_row, dim3((e.n + 255) / 256), dim3(256), 0, st, e, code_dev, code, out, e.n);
    return hipGetLastError();
}

hipError_t enqueue_silu(float *x, int n, hipStream_t st)
{
    hipLaunchKernelGGL(k_silu, dim3((n + 255) / 256), dim3(256), 0, st, x, n);
    return hipGetLastError();
}

// Columns c0..c1-1 of rows [rows][ld] set to zero (a fill kernel rather than
// a memset node, so the call can sit in a captured graph).
__global__ void k_zero_cols(float *Y, int rows, int ld, int c0, int c1)
{
    const int j = c0 + blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= c1) return;
    for (int r = blockIdx.y; r < rows; r += gridDim.y) Y[(size_t)r * ld + j] = 0.0f;
}

hipError_t enqueue_zero_cols(float *Y, int rows, int ld, int c0, int c1, hipStream_t st)
{
    if (rows <= 0 || c1 <= c0) return hipSuccess;
    // rows beyond the grid's y limit are taken by a row loop
    const int gy = std::min(rows, 65535);
    hipLaunchKernelGGL(k_zero_cols, dim3((c1 - c0 + 255) / 256, gy), dim3(256), 0, st, Y, rows, ld, c0, c1);
    return hipGetLastError();
}

hipError_t enqueue_embed_sum(const Q4Rows &cp, int n_groups, const uint32_t *codes, float *out,
                             hipStream_t st)
{
    hipLaunchKernelGGL(k_embed_sum, dim3((cp.n + 255) / 256), dim3(256), 0, st, cp, n_groups, codes, out, cp.n);
    return hipGetLastError();
}

// gate|up and down in one launch (one row): workgroups [0, ng) are the
// gate|up tiles (single slice, interleaved groups), storing silu(gate) * up
// as (epoch, value) words; the rest are the down projection's tiles, which
// issue their weight loads (after HOLD ticks) and take their k-slice of the
// words when they arrive.  The gate|up tiles come first in the grid, so
// every tile a down workgroup waits for has been dispatched before it and
// never waits.
template <int GBG, int RG, int RD, int KMAX, int NB, uint32_t HOLD>
__global__ void __launch_bounds__(512)
k_mlp(Q4Tiled wg, ProResidRms<NB, KMAX> pg, EpiSwigluLL<NB> eg, int ng, Q4Tiled wd, ProLL<NB> pd, EpiPart<NB> ed)
{
    // the down tiles on the byte-convert inner loop, the gate|up tiles on
    // v_fma_mix (same bits either way): frames at KV 2048 586.9 against
    // 585.7 frames/s with both on byte converts and 584.7 with the down
    // tiles on v_fma_mix too (the same split measured for k_mlp1)
    if ((int)blockIdx.x < ng) {
        EpiSwigluLL<NB> e = eg;
        e.epoch = *eg.seq + 1;
        gemv_tile<512, GBG, RG, NB, true>(wg, pg, e, blockIdx.x);
        return;
    }
    if constexpr (HOLD > 0) stage_hold(HOLD);
    gemv_tile<512, 1, RD, NB, false>(wd, pd, ed, blockIdx.x - ng);
}

// The same on one-group gate|up tiles: a gate or an up group per tile, twice
// the tiles of the paired layout, so twice the CUs stream the gate|up weight
// (a 1024 x 6144 gate|up GEMV: 3.0 us on 192 one-group tiles, 3.6 us on 96
// paired ones).  The tiles store their raw column sums as words and the
// down tiles form silu(gate) * up from them (ProSwigluLL).
template <int T, int RG, int RD, int KMAX, int NB, uint32_t HOLD>
__global__ void __launch_bounds__(T)
k_mlp1(Q4Tiled wg, ProResidRms<NB, KMAX> pg, EpiLL<NB> eg, int ng, Q4Tiled wd, ProSwigluLL<NB> pd, EpiPart<NB> ed)
{
    if ((int)blockIdx.x < ng) {
        EpiLL<NB> e = eg;
        e.epoch = *eg.seq + 1;
        gemv_tile<T, 1, RG, NB, true>(wg, pg, e, blockIdx.x);
        return;
    }
    if constexpr (HOLD > 0) stage_hold(HOLD);
    gemv_tile<T, 1, RD, NB, false>(wd, pd, ed, blockIdx.x - ng);
}

// The words and epoch of a fused gate|up + down launch.
struct MlpFuse {
    uint64_t *ll;
    uint32_t *seq;
    DevState *st;
};

// QTTS_FUSED_MLP=0 keeps gate|up and down apart.
static bool fused_mlp_on()
{
    static const bool on = [] {
        const char *v = getenv("QTTS_FUSED_MLP");
        return !(v && *v == '0');
    }();
    return on;
}

bool fused_mlp_enabled() { return fused_mlp_on(); }

// Tile pairs k_mlp is built for: the talker's (gate|up 2 groups x 2048 rows,
// down 4 rows per thread) and the predictor's (2 groups x 1024 rows, down 2
// rows per thread), 512 threads each.
template <int NB, int KMAX>
static hipError_t launch_mlp(const LayerDev &L, const Workspace &ws, const ProResidRms<NB, KMAX> &pro_gu, int inter,
                             const MlpFuse &fz, hipStream_t s)
{
    const int ng = L.gate_up.S * L.gate_up.CT, nd = L.down.S * L.down.CT;
    const EpiSwigluLL<NB> eg{fz.ll, inter, fz.seq, 0};
    const ProLL<NB> pd{fz.ll, inter, fz.seq, fz.st};
    const EpiPart<NB> ed{ws.part_down, L.down.npad};
    constexpr uint32_t hold = KMAX == 2048 ? HOLD_TALKER_DOWN : 0;   // the talker's hidden size
    if (L.gate_up.cfg == TILE_G2_T512 && L.down.cfg == TILE_G1_T512_R4)
        hipLaunchKernelGGL((k_mlp<2, 8, 4, KMAX, NB, hold>), dim3(ng + nd), dim3(512), 0, s, L.gate_up, pro_gu, eg, ng,
                           L.down, pd, ed);
    else if (L.gate_up.cfg == TILE_G2_T512_R4 && L.down.cfg == TILE_G1_T512_R2)
        hipLaunchKernelGGL((k_mlp<2, 4, 2, KMAX, NB, hold>), dim3(ng + nd), dim3(512), 0, s, L.gate_up, pro_gu, eg, ng,
                           L.down, pd, ed);
    else if (L.gate_up.cfg == TILE_G1_T512_R2 && L.down.cfg == TILE_G1_T512_R2 && L.gate_up.interleave)
        hipLaunchKernelGGL((k_mlp1<512, 2, 2, KMAX, NB, KMAX == 2048 ? HOLD_TALKER_DOWN : HOLD_PRED_DOWN>),
                           dim3(ng + nd), dim3(512), 0, s, L.gate_up, pro_gu,
                           EpiLL<NB>{fz.ll, L.gate_up.npad, fz.seq, 0}, ng, L.down,
                           ProSwigluLL<NB>{fz.ll, L.gate_up.npad, inter, fz.seq, fz.st}, ed);
    else if (L.gate_up.cfg == TILE_G1_T256_R4 && L.down.cfg == TILE_G1_T256_R2 && L.gate_up.interleave)
        hipLaunchKernelGGL((k_mlp1<256, 4, 2, KMAX, NB, KMAX == 2048 ? HOLD_TALKER_DOWN : HOLD_PRED_DOWN>),
                           dim3(ng + nd), dim3(256), 0, s, L.gate_up, pro_gu,
                           EpiLL<NB>{fz.ll, L.gate_up.npad, fz.seq, 0}, ng, L.down,
                           ProSwigluLL<NB>{fz.ll, L.gate_up.npad, inter, fz.seq, fz.st}, ed);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

static bool mlp_fusable(const LayerDev &L)
{
    if (!fused_mlp_on() || L.gate_up.S != 1) return false;
    return (L.gate_up.cfg == TILE_G2_T512 && L.down.cfg == TILE_G1_T512_R4) ||
           (L.gate_up.cfg == TILE_G2_T512_R4 && L.down.cfg == TILE_G1_T512_R2) ||
           (L.gate_up.cfg == TILE_G1_T512_R2 && L.down.cfg == TILE_G1_T512_R2 && L.gate_up.interleave) ||
           (L.gate_up.cfg == TILE_G1_T256_R4 && L.down.cfg == TILE_G1_T256_R2 && L.gate_up.interleave);
}

// gate|up then down: h = silu(gate) * up written by the gate|up epilogue when
// the gate|up weight is one slice, else formed in the down prologue; with
// `fz` and tiles k_mlp is built for, both in one launch.
template <int NB, class ProGU>
static hipError_t swiglu_down(const LayerDev &L, const Workspace &ws, const ProGU &pro_gu, int inter,
                              hipStream_t s, const MlpFuse *fz = nullptr)
{
    if constexpr (std::is_same<ProGU, ProResidRms<NB, 1024>>::value) {
        if (fz && mlp_fusable(L)) return launch_mlp<NB, 1024>(L, ws, pro_gu, inter, *fz, s);
    }
    if constexpr (NB == 1 && std::is_same<ProGU, ProResidRms<1, 2048>>::value) {
        if (fz && mlp_fusable(L)) return launch_mlp<1, 2048>(L, ws, pro_gu, inter, *fz, s);
    }
    if (L.gate_up.S == 1 && tile_shape(L.gate_up.cfg).GB % 2 == 0) {
        QCHK(launch_gemv<NB>(L.gate_up, pro_gu, EpiSwiglu<NB>{ws.h, inter}, s));
        return launch_gemv<NB>(L.down, ProPlain<NB>{ws.h, inter, inter}, EpiPart<NB>{ws.part_down, L.down.npad}, s);
    }
    QCHK(launch_gemv<NB>(L.gate_up, pro_gu, EpiPart<NB>{ws.part_gu, L.gate_up.npad}, s));
    return launch_gemv<NB>(L.down, ProSwiglu<NB>{ws.part_gu, L.gate_up.S, L.gate_up.npad, inter},
                           EpiPart<NB>{ws.part_down, L.down.npad}, s);
}

// One talker layer, decode (talker.rs:274-350).  The residual stream enters
// as base (+ the previous layer's down partials) and leaves as ws.xa plus
// this layer's down partials.
// The decode attention over one or two pages per workgroup, and the o-proj
// that merges its chunks.
template <int PG>
static hipError_t talker_attn_o(const TalkerDev &m, const Workspace &ws, const LayerDev &L, int l,
                                const DevState *st, int64_t pos_ovr, int slot_ovr, bool fused, hipStream_t s)
{
    if (!fused) {
        const int grid = 8 * ((ws.attn_grid / 8 + PG - 1) / PG);
        hipLaunchKernelGGL(k_talker_attn<PG>, dim3(grid), dim3(256 * PG), 0, s, ws.part_qkv, L.qkv.S, L.qkv.npad,
                           L.q_norm, L.k_norm, m.rope_cos, m.rope_sin, st, pos_ovr, slot_ovr, l, m.kv, ws.am,
                           ws.al, ws.aacc);
        QCHK(hipGetLastError());
    }
    return launch_gemv<1>(L.o, ProAttnCombine<PG>{ws.am, ws.al, ws.aacc, st, slot_ovr, ws.ll_seq},
                          EpiPart<1>{ws.part_o, L.o.npad}, s);
}

// The q|k|v GEMV and the two-page attention share one launch when the q|k|v
// weight has the tile the fused kernel is built for (QTTS_FUSED_ATTN=0
// keeps them apart).  Fused, two pages per work item is faster at every
// length (KV 80-336: 507 frames/s unfused with one page, 517 fused with
// two; KV 2064-2320: 492 unfused, 510 fused).
static bool fused_attn_on()
{
    static const bool on = [] {
        const char *v = getenv("QTTS_FUSED_ATTN");
        return !(v && *v == '0');
    }();
    return on;
}

static bool qkv_attn_fusable(const LayerDev &L)
{
    return L.qkv.cfg == TILE_G1_T512_R2 && L.qkv.S <= RES_MAX_S && L.qkv.npad >= 32 * HEAD_DIM && fused_attn_on();
}

bool talker_fused_attn(const TalkerDev &m)
{
    for (int l = 0; l < m.n_layers; l++)
        if (!qkv_attn_fusable(m.layers[l])) return false;
    return m.n_layers > 0;
}

static hipError_t talker_layer(const TalkerDev &m, const Workspace &ws, int l, const float *x_in,
                               const DevState *st, int64_t pos_ovr, int slot_ovr, int attn_pg, hipStream_t s)
{
    const LayerDev &L = m.layers[l];
    const LayerDev *P = l > 0 ? &m.layers[l - 1] : nullptr;
    const int H = m.hidden;
    // 1. residual + RMSNorm + fused q|k|v GEMV -> partials
    const ProResidRms<1, 2048> pre_attn{l == 0 ? x_in : ws.xa, H, P ? ws.part_down : nullptr, P ? P->down.S : 0, 1, 0,
                                  P ? P->down.npad : 0, nullptr, L.input_norm, H, ws.xb, nullptr};
    const bool fused = attn_pg == 2 && qkv_attn_fusable(L);
    if (fused) {
        // 1-2 in one launch: the GEMV's tiles, then the attention's work items
        constexpr TileShape ts = tile_shape(TILE_G1_T512_R2);
        const int nq = L.qkv.S * L.qkv.CT;
        const int na = 8 * ((ws.attn_grid / 8 + 1) / 2);
        hipLaunchKernelGGL((k_talker_qkv_attn<ts.T, ts.GB, ts.R>), dim3(nq + na), dim3(ts.T), 0, s, L.qkv, pre_attn,
                           EpiLL<1>{ws.ll_qkv, L.qkv.npad, ws.ll_seq + LL_TQKV, 0}, nq, L.q_norm, L.k_norm, m.rope_cos, m.rope_sin,
                           st, pos_ovr, slot_ovr, l, m.kv, ws.am, ws.al, ws.aacc);
        QCHK(hipGetLastError());
    } else {
        QCHK(launch_gemv<1>(L.qkv, pre_attn, EpiPart<1>{ws.part_qkv, L.qkv.npad}, s));
    }
    // 2. QK-norm, RoPE, KV append, split-K attention over the pages
    // 3. o_proj -> partials, the pages merged in its prologue
    QCHK(attn_pg == 2 ? talker_attn_o<2>(m, ws, L, l, st, pos_ovr, slot_ovr, fused, s)
                      : talker_attn_o<1>(m, ws, L, l, st, pos_ovr, slot_ovr, fused, s));
    // 5-6. residual + RMSNorm + gate|up, SiLU * up, down -> partials
    const ProResidRms<1, 2048> pre_mlp{ws.xb, H, ws.part_o, L.o.S, 1, 0, L.o.npad, nullptr, L.post_norm, H, ws.xa, nullptr};
    const MlpFuse fz{ws.ll_th, ws.ll_seq + LL_TMLP, const_cast<DevState *>(st)};
    return swiglu_down<1>(L, ws, pre_mlp, m.inter, s, st ? &fz : nullptr);
}

// Final norm of the residual (talker.rs:352-353) into `side` + codec-head
// partials.
static hipError_t talker_head(const TalkerDev &m, const Workspace &ws, float *side, hipStream_t s)
{
    const LayerDev &P = m.layers[m.n_layers - 1];
    const ProResidRms<1, 2048> pre{ws.xa, m.hidden, ws.part_down, P.down.S, 1, 0, P.down.npad, nullptr, m.final_norm,
                             m.hidden, nullptr, side};
    return launch_gemv<1>(m.codec_head, pre, EpiPart<1>{ws.part_head, m.codec_head.npad}, s);
}

// forward_with_embedding (talker.rs:263-360) on the input ws.x: 28 layers,
// final norm (hidden -> ws.hid_work), codec head, then k_step_end.
hipError_t enqueue_talker_step(const TalkerDev &m, const Workspace &ws, DevState *st, int frame_mode, int attn_pg,
                               hipStream_t s)
{
    for (int l = 0; l < m.n_layers; l++) QCHK(talker_layer(m, ws, l, ws.x, st, -1, -1, attn_pg, s));
    QCHK(talker_head(m, ws, ws.hid_work, s));
    hipLaunchKernelGGL(k_step_end, dim3(1), dim3(1024), 0, s, ws.part_head, m.codec_head.S,
                       m.codec_head.npad, m.vocab, ws.hid_work, m.hidden, ws.logits, ws.hidden, st,
                       frame_mode, ws.ring_pred, ws.ring_used);
    return hipGetLastError();
}

// One prefill row: RoPE at pos, KV slot `slot`, no codec head.
hipError_t enqueue_talker_row(const TalkerDev &m, const Workspace &ws, const DevState *st, int64_t pos,
                              int slot, int attn_pg, hipStream_t s)
{
    for (int l = 0; l < m.n_layers; l++) QCHK(talker_layer(m, ws, l, ws.x, st, pos, slot, attn_pg, s));
    return hipSuccess;
}

hipError_t enqueue_final_norm(const TalkerDev &m, const Workspace &ws, float *hidden_out, hipStream_t s)
{
    return talker_head(m, ws, hidden_out, s);
}

hipError_t enqueue_codec_head(const TalkerDev &m, const Workspace &ws, const float *hidden, float *logits,
                              hipStream_t s)
{
    QCHK(launch_gemv<1>(m.codec_head, ProPlain<1>{hidden, m.hidden, m.hidden},
                        EpiPart<1>{ws.part_head, m.codec_head.npad}, s));
    return reduce_parts(ws.part_head, m.codec_head.S, 1, m.codec_head.npad, m.vocab, logits, m.vocab,
                        nullptr, 0, s);
}

// One predictor layer over NB tokens at positions pos0.. (code_predictor.rs:
// 354-432 for NB=2, 450-510 for NB=1).  Layer 0 starts from the input
// projection partials + bias.
template <int NB, class Pro>
static hipError_t launch_gemv_then_mlp(const PredictorDev &p, const LayerDev &L, const Workspace &ws,
                                       const Pro &pro, hipStream_t s, DevState *st = nullptr);

// The fused attention prologue covers 2 kv heads per workgroup of 256
// threads: o-proj tiles of 256 threads and 512 rows, 16 / 8 heads of 128.
static bool pred_attn_fusable(const PredictorDev &p, const LayerDev &L)
{
    return tile_shape(L.o.cfg).T == 256 && L.o.KC == 512 && p.n_heads == 16 && p.n_kv_heads == 8 &&
           L.qkv.npad >= 32 * HEAD_DIM && L.qkv.S <= RES_MAX_S;
}

template <int NB, int MS>
static ProPredAttn<NB, MS> pred_attn_pro(const PredictorDev &p, const LayerDev &L, const Workspace &ws, int pos0,
                                         float *Kc, float *Vc)
{
    return ProPredAttn<NB, MS>{ws.part_qkv, L.qkv.S, L.qkv.npad, L.q_norm, L.k_norm, p.rope_cos, p.rope_sin,
                               pos0, Kc, Vc, nullptr, 0, nullptr, 0, nullptr, 0, nullptr, nullptr, nullptr, 0,
                               nullptr, nullptr, ws.ll_seq + LL_PMLP};
}

// The predictor MLP after the attention + o-proj: residual + RMSNorm,
// gate|up, down (one launch when fusable and `st` takes the wait errors).
// Its gate|up advances the LL_PQKV epoch.
template <int NB>
static hipError_t pred_mlp(const PredictorDev &p, const LayerDev &L, const Workspace &ws, hipStream_t s,
                           DevState *st)
{
    const int h = p.hidden;
    ProResidRms<NB, 1024> pre_mlp{ws.pxb, h, ws.part_o, L.o.S, NB, 0, L.o.npad, nullptr, L.post_norm, h, ws.pxa, nullptr};
    pre_mlp.seq = ws.ll_seq + LL_PQKV;
    const MlpFuse fz{ws.ll_ph, ws.ll_seq + LL_PMLP, st};
    return swiglu_down<NB>(L, ws, pre_mlp, p.inter, s, st ? &fz : nullptr);
}

// Predictor q|k|v GEMV and attention + o-proj in one launch (one row):
// workgroups [0, nq) are the q|k|v tiles, storing (epoch, value) words; the
// rest are the o-proj tiles, whose prologue issues its cache, gamma and
// weight loads (after HOLD_PRED_O ticks) and attends when its words arrive.  The q|k|v tiles
// come first in the grid, so every tile an o-proj workgroup waits for has
// been dispatched before it and never waits itself.  The gate|up launch that
// follows advances the epoch.
template <int MS, int NB>
__global__ void __launch_bounds__(256)
k_pred_qkv_attn_o(Q4Tiled wq, ProResidRms<NB, 1024> pq, EpiLL<NB> eq, int nq, Q4Tiled wo,
                  ProPredAttn<NB, MS, false, true> po, EpiPart<NB> eo)
{
    if ((int)blockIdx.x < nq) {
        EpiLL<NB> e = eq;
        e.epoch = *eq.seq + 1;
        gemv_tile<256, 1, 2, NB>(wq, pq, e, blockIdx.x);
        return;
    }
    stage_hold(HOLD_PRED_O);
    gemv_tile<256, 1, 2, NB>(wo, po, eo, blockIdx.x - nq);
}

// QTTS_FUSED_PRED=0 keeps the predictor's q|k|v and attention + o-proj apart.
static bool fused_pred_on()
{
    static const bool on = [] {
        const char *v = getenv("QTTS_FUSED_PRED");
        return !(v && *v == '0');
    }();
    return on;
}

static bool pred_qkv_attn_fusable(const PredictorDev &p, const LayerDev &L)
{
    return fused_pred_on() && pred_attn_fusable(p, L) && L.qkv.cfg == TILE_G1_T256_R2 &&
           L.o.cfg == TILE_G1_T256_R2 && L.qkv.S == 2;
}

template <int NB>
static hipError_t pred_layer(const PredictorDev &p, const Workspace &ws, int l, int pos0, hipStream_t s,
                             const ProCodeRowRms<1024> *row_in = nullptr, const float *qkv_tab = nullptr,
                             DevState *st = nullptr)
{
    const LayerDev &L = p.layers[l];
    const int h = p.hidden;
    if constexpr (NB == 1) {
        if (row_in && qkv_tab) {
            // layer 0's q|k|v read from the table inside the attention prologue
            float *Kc = ws.pk + (size_t)l * PRED_KV_CAP * 8 * HEAD_DIM;
            float *Vc = ws.pv + (size_t)l * PRED_KV_CAP * 8 * HEAD_DIM;
            ProPredAttn<1, 1, true> pro{nullptr, 1, L.qkv.npad, L.q_norm, L.k_norm, p.rope_cos, p.rope_sin, pos0,
                                        Kc, Vc, qkv_tab, row_in->rows, row_in->cand, row_in->ncand, row_in->st,
                                        row_in->slot, row_in->codes_api, row_in->table, row_in->x_out, row_in->k,
                                        nullptr, nullptr, ws.ll_seq + LL_PMLP};
            return launch_gemv_then_mlp<1>(p, L, ws, pro, s, row_in->st);
        }
    }
    float *Kc = ws.pk + (size_t)l * PRED_KV_CAP * 8 * HEAD_DIM;
    float *Vc = ws.pv + (size_t)l * PRED_KV_CAP * 8 * HEAD_DIM;
    if (NB == 1 && row_in) {
        QCHK(launch_gemv<1>(L.qkv, *row_in, EpiPart<1>{ws.part_qkv, L.qkv.npad}, s));
    } else {
        const ProResidRms<NB, 1024> pre_attn =
            l == 0 ? ProResidRms<NB, 1024>{nullptr, h, ws.part_proj, p.proj.S, NB, 0, p.proj.npad, p.proj_bias,
                                           L.input_norm, h, ws.pxb, nullptr}
                   : ProResidRms<NB, 1024>{ws.pxa, h, ws.part_down, p.layers[l - 1].down.S, NB, 0,
                                           p.layers[l - 1].down.npad, nullptr, L.input_norm, h, ws.pxb, nullptr};
        if (st && pred_qkv_attn_fusable(p, L)) {
            // q|k|v and attention + o-proj in one launch; the gate|up launch advances the epoch
            const ProPredAttn<NB, 2, false, true> po{nullptr, L.qkv.S, L.qkv.npad, L.q_norm, L.k_norm,
                                                     p.rope_cos, p.rope_sin, pos0, Kc, Vc, nullptr, 0, nullptr,
                                                     0, st, 0, nullptr, nullptr, nullptr, 0, ws.ll_pqkv,
                                                     ws.ll_seq + LL_PQKV, ws.ll_seq + LL_PMLP};
            const int nq = L.qkv.S * L.qkv.CT, no = L.o.S * L.o.CT;
            hipLaunchKernelGGL((k_pred_qkv_attn_o<2, NB>), dim3(nq + no), dim3(256), 0, s, L.qkv, pre_attn,
                               EpiLL<NB>{ws.ll_pqkv, L.qkv.npad, ws.ll_seq + LL_PQKV, 0}, nq, L.o, po,
                               EpiPart<NB>{ws.part_o, L.o.npad});
            QCHK(hipGetLastError());
            return pred_mlp<NB>(p, L, ws, s, st);
        }
        QCHK(launch_gemv<NB>(L.qkv, pre_attn, EpiPart<NB>{ws.part_qkv, L.qkv.npad}, s));
    }
    if (pred_attn_fusable(p, L)) {
        // attention inside the o-proj prologue
        switch (L.qkv.S) {
        case 1: return launch_gemv_then_mlp<NB>(p, L, ws, pred_attn_pro<NB, 1>(p, L, ws, pos0, Kc, Vc), s, st);
        case 2: return launch_gemv_then_mlp<NB>(p, L, ws, pred_attn_pro<NB, 2>(p, L, ws, pos0, Kc, Vc), s, st);
        case 3: return launch_gemv_then_mlp<NB>(p, L, ws, pred_attn_pro<NB, 3>(p, L, ws, pos0, Kc, Vc), s, st);
        default: return launch_gemv_then_mlp<NB>(p, L, ws, pred_attn_pro<NB, 4>(p, L, ws, pos0, Kc, Vc), s, st);
        }
    }
    hipLaunchKernelGGL(k_pred_attn, dim3(p.n_kv_heads), dim3(256), 0, s, ws.part_qkv, L.qkv.S, NB, L.qkv.npad,
                       L.q_norm, L.k_norm, p.rope_cos, p.rope_sin, pos0, Kc, Vc, ws.pattn);
    QCHK(hipGetLastError());
    // this o-proj does not advance the MLP epoch: the MLP stays two launches
    const int qd = p.n_heads * HEAD_DIM;
    return launch_gemv_then_mlp<NB>(p, L, ws, ProPlain<NB>{ws.pattn, qd, qd}, s, nullptr);
}

template <int NB, class Pro>
static hipError_t launch_gemv_then_mlp(const PredictorDev &p, const LayerDev &L, const Workspace &ws,
                                       const Pro &pro, hipStream_t s, DevState *st)
{
    QCHK(launch_gemv<NB>(L.o, pro, EpiPart<NB>{ws.part_o, L.o.npad}, s));
    return pred_mlp<NB>(p, L, ws, s, st);
}

// A single-slice lm head whose column tiles fit one wave writes per-tile
// argmax candidates; the consumer of the code chooses among them.
static bool head_cand(const PredictorDev &p, int g) { return p.heads[g].S == 1 && p.heads[g].CT <= MAX_CAND; }

// final norm of row `row` of the last layer's output + lm_head[g] + argmax
static hipError_t pred_head(const PredictorDev &p, const Workspace &ws, DevState *st, int g, int NBP, int row,
                            const uint32_t *forced, uint32_t *codes_api, hipStream_t s)
{
    const LayerDev &P = p.layers[p.n_layers - 1];
    const ProResidRms<1, 1024> pre{ws.pxa + (size_t)row * p.hidden, p.hidden, ws.part_down, P.down.S, NBP, row,
                             P.down.npad, nullptr, p.final_norm, p.hidden, nullptr, nullptr};
    if (head_cand(p, g)) return launch_gemv<1>(p.heads[g], pre, EpiArgmax{ws.cand + g * MAX_CAND, p.vocab}, s);
    QCHK(launch_gemv<1>(p.heads[g], pre, EpiPart<1>{ws.part_head, p.heads[g].npad}, s));
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, s, ws.part_head, p.heads[g].S, p.heads[g].npad, p.vocab,
                       st, g + 1, forced, codes_api);
    return hipGetLastError();
}

// generate_acoustic_codes (code_predictor.rs:218-273).  Inputs: talker
// hidden and either the semantic code in st->used[0] (frame mode, sem ==
// nullptr) or an explicit semantic embedding `sem` (API mode).  Codes go to
// st->pred[1..15] / st->used[1..15] (and codes_api when given).
hipError_t enqueue_predictor_chain(const PredictorDev &p, const TalkerDev &m, const Workspace &ws,
                                   DevState *st, const float *hidden, const float *sem,
                                   const uint32_t *forced, uint32_t *codes_api, hipStream_t s)
{
    // projections of [talker hidden, semantic embedding] (:235-241)
    if (sem) {
        QCHK(hipMemcpyAsync(ws.pin, hidden, sizeof(float) * m.hidden, hipMemcpyDeviceToDevice, s));
        QCHK(hipMemcpyAsync(ws.pin + m.hidden, sem, sizeof(float) * m.hidden, hipMemcpyDeviceToDevice, s));
        QCHK(launch_gemv<2>(p.proj, ProPlain<2>{ws.pin, m.hidden, m.hidden}, EpiPart<2>{ws.part_proj, p.proj.npad}, s));
    } else {
        QCHK(launch_gemv<2>(p.proj, ProHidEmbed{hidden, m.codec_rows, &st->used[0], m.hidden},
                            EpiPart<2>{ws.part_proj, p.proj.npad}, s));
    }
    for (int l = 0; l < p.n_layers; l++) QCHK(pred_layer<2>(p, ws, l, 0, s, nullptr, nullptr, st));
    QCHK(pred_head(p, ws, st, 0, 2, 1, forced, codes_api, s));           // :247-248
    for (int g = 1; g < p.n_groups; g++) {
        if (p.proj_rows) {
            // the projected embedding row of the previous code, looked up (:255-260)
            const float2 *cand = head_cand(p, g - 1) ? ws.cand + (g - 1) * MAX_CAND : nullptr;
            const ProCodeRowRms<1024> row_in{p.proj_rows + (size_t)(g - 1) * p.emb_rows.rows * p.hidden,
                                             p.emb_rows.rows, cand, p.heads[g - 1].CT, st, g, codes_api,
                                             p.layers[0].input_norm, p.hidden, ws.pxb};
            QCHK(pred_layer<1>(p, ws, 0, 1 + g, s, &row_in,
                               p.qkv_rows ? p.qkv_rows + (size_t)(g - 1) * p.emb_rows.rows * p.layers[0].qkv.npad
                                          : nullptr));
            for (int l = 1; l < p.n_layers; l++) QCHK(pred_layer<1>(p, ws, l, 1 + g, s, nullptr, nullptr, st));
            QCHK(pred_head(p, ws, st, g, 1, 0, forced, codes_api, s));
            continue;
        }
        // embed the previous code with codebook g-1, project (:255-260)
        Q4Rows e = p.emb_rows;
        e.packed += (size_t)(g - 1) * e.rows * e.G * 16;
        e.scales += (size_t)(g - 1) * e.rows * e.G;
        if (head_cand(p, g - 1))
            QCHK(launch_gemv<1>(p.proj, ProArgmaxEmbed{e, ws.cand + (g - 1) * MAX_CAND, p.heads[g - 1].CT, st, g, codes_api},
                                EpiPart<1>{ws.part_proj, p.proj.npad}, s));
        else
            QCHK(launch_gemv<1>(p.proj, ProEmbed{e, &st->used[g]}, EpiPart<1>{ws.part_proj, p.proj.npad}, s));
        for (int l = 0; l < p.n_layers; l++) QCHK(pred_layer<1>(p, ws, l, 1 + g, s, nullptr, nullptr, st));
        QCHK(pred_head(p, ws, st, g, 1, 0, forced, codes_api, s));
    }
    // API calls resolve the last code here; a frame's combine does it itself
    const int gl = p.n_groups - 1;
    if (sem && head_cand(p, gl)) {
        hipLaunchKernelGGL(k_cand_final, dim3(1), dim3(64), 0, s, ws.cand + gl * MAX_CAND, p.heads[gl].CT, st,
                           p.n_groups, codes_api);
        QCHK(hipGetLastError());
    }
    return hipSuccess;
}

// The predictor's projected rows proj(E_g[c]) + bias for every code c of
// codebooks g = 0..n_tables-1 (the layer-0 inputs of steps 1..n_tables),
// with the step's own GEMV instance so the rows carry the same bits.
// Scratch: X [rows][proj.k], part [rows][proj.S][proj.npad].
hipError_t enqueue_pred_row_tables(const PredictorDev &p, int n_tables, float *X, float *part, float *out,
                                   hipStream_t s)
{
    const int rows = p.emb_rows.rows, kin = p.proj.k;
    if (p.emb_rows.n != kin) return hipErrorInvalidValue;
    for (int g = 0; g < n_tables; g++) {
        Q4Rows e = p.emb_rows;
        e.packed += (size_t)g * e.rows * e.G * 16;
        e.scales += (size_t)g * e.rows * e.G;
        hipLaunchKernelGGL(k_dequant_rows, dim3((kin + 255) / 256, rows), dim3(256), 0, s, e, X);
        QCHK(hipGetLastError());
        QCHK(launch_gemv<1>(p.proj, ProPlainY{X, kin, kin}, EpiPartY{part, p.proj.npad, p.proj.S}, s, rows));
        hipLaunchKernelGGL(k_rows_from_parts, dim3((p.hidden + 255) / 256, rows), dim3(256), 0, s, part, p.proj.S,
                           p.proj.npad, p.proj_bias, p.hidden, out + (size_t)g * rows * p.hidden);
        QCHK(hipGetLastError());
    }
    return hipSuccess;
}

// Layer 0's q|k|v of every row of the projected tables (rows of proj_rows
// through the input RMSNorm and the q|k|v GEMV, the step's own prologue and
// GEMV instance, slices summed in slice order as the attention prologue
// sums them).  Scratch: part [rows][qkv.S][qkv.npad].
bool pred_qkv_tables_supported(const PredictorDev &p)
{
    return p.proj_rows && pred_attn_fusable(p, p.layers[0]) && p.hidden <= 1024;
}

hipError_t enqueue_pred_qkv_tables(const PredictorDev &p, int n_tables, float *part, float *out, hipStream_t s)
{
    if (!pred_qkv_tables_supported(p)) return hipErrorInvalidValue;
    const LayerDev &L = p.layers[0];
    const int rows = p.emb_rows.rows;
    for (int g = 0; g < n_tables; g++) {
        const ProCodeRowRms<1024> pro{p.proj_rows + (size_t)g * rows * p.hidden, rows, nullptr, 0, nullptr, 0,
                                      nullptr, L.input_norm, p.hidden, nullptr};
        QCHK(launch_gemv<1>(L.qkv, pro, EpiPartY{part, L.qkv.npad, L.qkv.S}, s, rows));
        hipLaunchKernelGGL(k_rows_from_parts, dim3((L.qkv.npad + 255) / 256, rows), dim3(256), 0, s, part, L.qkv.S,
                           L.qkv.npad, (const float *)nullptr, L.qkv.npad, out + (size_t)g * rows * L.qkv.npad);
        QCHK(hipGetLastError());
    }
    return hipSuccess;
}

// One frame (generate_new.rs:606-675): sample code 0, predictor chain,
// fuse embeddings + text, talker step, record.
hipError_t enqueue_frame_codes(const TalkerDev &m, const PredictorDev &p, const Workspace &ws, DevState *st,
                               const uint32_t *forced, hipStream_t s)
{
    SampleArgs none{};
    hipLaunchKernelGGL(k_sampler, dim3(1), dim3(SAMP_T), 0, s, ws.logits, m.vocab, st, 0, none,
                       (uint64_t *)nullptr, (uint32_t *)nullptr, forced);
    QCHK(hipGetLastError());
    QCHK(enqueue_predictor_chain(p, m, ws, st, ws.hidden, nullptr, forced, nullptr, s));
    const int gl = p.n_groups - 1;
    hipLaunchKernelGGL(k_combine, dim3((m.hidden + 255) / 256), dim3(256), 0, s, m.codec_rows,
                       p.emb_rows, p.n_groups, st, ws.text, ws.pad, ws.x, m.hidden,
                       head_cand(p, gl) ? (const float2 *)(ws.cand + gl * MAX_CAND) : (const float2 *)nullptr,
                       p.heads[gl].CT);
    return hipGetLastError();
}

hipError_t enqueue_frame(const TalkerDev &m, const PredictorDev &p, const Workspace &ws, DevState *st,
                         const uint32_t *forced, int attn_pg, hipStream_t s)
{
    QCHK(enqueue_frame_codes(m, p, ws, st, forced, s));
    return enqueue_talker_step(m, ws, st, 1, attn_pg, s);
}

// The legacy loop's sampler (generate.rs:185-217): apply_repetition_penalty
// (generate.rs:87-98, every previous token in order, when penalty > 1), then
// sample_top_k (generate.rs:50-84).  One workgroup: temperature <= 0 takes
// the last maximum; otherwise a bitonic sort of (logit desc, index asc) in
// LDS (the reference's unstable sort leaves the order of equal logits
// open), then thread 0 forms exp((l - max) / T) over the top k, their
// sequential sum, the normalised running sum and the draw.  status: 0,
// -1 (top_k < 1: the reference indexes an empty list), -7 (NaN).
constexpr int LEG_N = 4096;

__global__ void __launch_bounds__(1024)
k_sample_top_k(const float *logits, int n, float temperature, int top_k, const uint32_t *prev, int n_prev,
               float penalty, uint64_t *rng, uint32_t *out, int *status)
{
    __shared__ float v[LEG_N];
    __shared__ int ix[LEG_N];
    __shared__ int nanf;
    __shared__ float bv[32];
    __shared__ int bi[32];
    const int t = threadIdx.x;
    if (t == 0) nanf = 0;
    for (int i = t; i < LEG_N; i += 1024) {
        v[i] = i < n ? logits[i] : -INFINITY;
        ix[i] = i;
    }
    __syncthreads();
    if (t == 0 && penalty > 1.0f) {
        for (int i = 0; i < n_prev; i++) {
            const uint32_t tok = prev[i];
            if (tok < (uint32_t)n) {
                const float x = v[tok];
                v[tok] = x > 0.0f ? x / penalty : x * penalty;
            }
        }
    }
    __syncthreads();
    bool mynan = false;
    for (int i = t; i < n; i += 1024) mynan |= isnan(v[i]);
    if (mynan) nanf = 1;
    __syncthreads();
    if (nanf) {
        if (t == 0) *status = -7;
        return;
    }
    if (temperature <= 0.0f) {
        // max_by: the last index among equal maxima
        float best = -INFINITY;
        int bidx = -1;
        for (int i = t; i < n; i += 1024)
            if (bidx < 0 || !(best > v[i])) { best = v[i]; bidx = i; }
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(best, o);
            const int oi = __shfl_xor(bidx, o);
            if (oi >= 0 && (bidx < 0 || ov > best || (ov == best && oi > bidx))) { best = ov; bidx = oi; }
        }
        if ((t & 63) == 0) { bv[t >> 6] = best; bi[t >> 6] = bidx; }
        __syncthreads();
        if (t == 0) {
            float b = bv[0];
            int j = bi[0];
            for (int w = 1; w < 16; w++)
                if (bi[w] >= 0 && (j < 0 || bv[w] > b || (bv[w] == b && bi[w] > j))) { b = bv[w]; j = bi[w]; }
            *out = (uint32_t)j;
            *status = 0;
        }
        return;
    }
    // bitonic sort of all LEG_N slots into (value desc, index asc)
    for (int size = 2; size <= LEG_N; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = t; i < LEG_N; i += 1024) {
                const int j = i ^ stride;
                if (j > i) {
                    const float a = v[i], b = v[j];
                    const int ia = ix[i], ib = ix[j];
                    const bool a_first = a > b || (a == b && ia < ib);
                    const bool up = (i & size) == 0;
                    if (up != a_first) {
                        v[i] = b; v[j] = a;
                        ix[i] = ib; ix[j] = ia;
                    }
                }
            }
            __syncthreads();
        }
    }
    if (t == 0) {
        const int k = top_k < n ? top_k : n;
        if (k < 1) {
            *status = -1;
            return;
        }
        // probabilities over the top k reuse the sorted values' slots
        const float mx = v[0];
        for (int i = 0; i < k; i++) v[i] = expf((v[i] - mx) / temperature);
        float sum = 0.0f;
        for (int i = 0; i < k; i++) sum += v[i];
        for (int i = 0; i < k; i++) v[i] /= sum;
        uint64_t rs = *rng;
        const float r = simple_rand_dev(rs);
        *rng = rs;
        float cs = 0.0f;
        int res = ix[k - 1];
        for (int i = 0; i < k; i++) {
            cs += v[i];
            if (r < cs) {
                res = ix[i];
                break;
            }
        }
        *out = (uint32_t)res;
        *status = 0;
    }
}

hipError_t enqueue_sample_top_k(const float *logits, int n, float temperature, int top_k, const uint32_t *prev,
                                int n_prev, float penalty, uint64_t *rng, uint32_t *out, int *status, hipStream_t s)
{
    if (n < 1 || n > LEG_N) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_sample_top_k, dim3(1), dim3(1024), 0, s, logits, n, temperature, top_k, prev, n_prev,
                       penalty, rng, out, status);
    return hipGetLastError();
}

hipError_t enqueue_sample_api(const float *logits, int n, const SampleArgsHost &a, uint64_t *rng_dev,
                              uint32_t *out_dev, DevState *st, hipStream_t s)
{
    SampleArgs sa{a.temperature, a.top_p, a.rep, a.top_k, a.prev, a.n_prev};
    hipLaunchKernelGGL(k_sampler, dim3(1), dim3(SAMP_T), 0, s, logits, n, st, 1, sa, rng_dev, out_dev,
                       (const uint32_t *)nullptr);
    return hipGetLastError();
}

hipError_t enqueue_kv_gather(const KvPaged &kv, int layer, int len, float *K, float *V, hipStream_t s)
{
    const size_t n = (size_t)len * 8 * HEAD_DIM;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_kv_gather, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, kv, layer, len, K, V);
    return hipGetLastError();
}

hipError_t enqueue_kv_scatter(const KvPaged &kv, int layer, int len, const float *K, const float *V,
                              hipStream_t s)
{
    const size_t n = (size_t)len * 8 * HEAD_DIM;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_kv_scatter, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, kv, layer, len, K, V);
    return hipGetLastError();
}

// Timing helpers: the gate|up GEMV of layer l with its real prologue, and the
// decode attention of layer l over `len` positions.
// Predictor timing: attention + o-proj of layer l for one row at position
// pos0 (the path pred_layer takes), or the whole layer step.
hipError_t enqueue_pred_attn_o_timing(const PredictorDev &p, const Workspace &ws, int l, int pos0, hipStream_t s)
{
    const LayerDev &L = p.layers[l];
    float *Kc = ws.pk + (size_t)l * PRED_KV_CAP * 8 * HEAD_DIM;
    float *Vc = ws.pv + (size_t)l * PRED_KV_CAP * 8 * HEAD_DIM;
    if (pred_attn_fusable(p, L)) {
        const EpiPart<1> epi{ws.part_o, L.o.npad};
        switch (L.qkv.S) {
        case 1: return launch_gemv<1>(L.o, pred_attn_pro<1, 1>(p, L, ws, pos0, Kc, Vc), epi, s);
        case 2: return launch_gemv<1>(L.o, pred_attn_pro<1, 2>(p, L, ws, pos0, Kc, Vc), epi, s);
        case 3: return launch_gemv<1>(L.o, pred_attn_pro<1, 3>(p, L, ws, pos0, Kc, Vc), epi, s);
        default: return launch_gemv<1>(L.o, pred_attn_pro<1, 4>(p, L, ws, pos0, Kc, Vc), epi, s);
        }
    }
    hipLaunchKernelGGL(k_pred_attn, dim3(p.n_kv_heads), dim3(256), 0, s, ws.part_qkv, L.qkv.S, 1, L.qkv.npad,
                       L.q_norm, L.k_norm, p.rope_cos, p.rope_sin, pos0, Kc, Vc, ws.pattn);
    QCHK(hipGetLastError());
    const int qd = p.n_heads * HEAD_DIM;
    return launch_gemv<1>(L.o, ProPlain<1>{ws.pattn, qd, qd}, EpiPart<1>{ws.part_o, L.o.npad}, s);
}

hipError_t enqueue_pred_layer_timing(const PredictorDev &p, const Workspace &ws, int l, int pos0, hipStream_t s)
{
    return pred_layer<1>(p, ws, l, pos0, s);
}

// One predictor layer step as the chain runs it (one row at pos0): q|k|v +
// attention + o-proj in one launch, gate|up + down in the next, the bounded
// waits reading st.
hipError_t enqueue_pred_layer_fused_timing(const PredictorDev &p, const Workspace &ws, int l, int pos0, DevState *st,
                                           hipStream_t s)
{
    return pred_layer<1>(p, ws, l, pos0, s, nullptr, nullptr, st);
}

// One talker layer as the frame's step runs it (q|k|v + attention in one
// launch at two pages per work item, the o-proj with the page merge,
// gate|up + down in one launch), appending at `slot` (past the cached
// length: cached positions untouched) and attending slot + 1 positions.
hipError_t enqueue_talker_layer_timing(const TalkerDev &m, const Workspace &ws, int l, int slot, int64_t pos,
                                       const DevState *st, hipStream_t s)
{
    return talker_layer(m, ws, l, ws.x, st, pos, slot, 2, s);
}

// Plain 16-byte-per-lane copy, 8 loads per thread in flight; n % 4 == 0.
__global__ void __launch_bounds__(256) k_copy_f4(const u32x4 *__restrict__ src, u32x4 *__restrict__ dst, int64_t n4)
{
    constexpr int U = 8;
    const int64_t base = (int64_t)blockIdx.x * 256 * U + threadIdx.x;
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int64_t i = base + (int64_t)u * 256;
        v[u] = __builtin_nontemporal_load(src + (i < n4 ? i : n4 - 1));
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int64_t i = base + (int64_t)u * 256;
        if (i < n4) __builtin_nontemporal_store(v[u], dst + i);
    }
}

hipError_t enqueue_copy(const float *src, float *dst, int64_t n, hipStream_t s)
{
    if (n <= 0 || n % 4) return hipErrorInvalidValue;
    const int64_t n4 = n / 4;
    const int64_t grid = (n4 + 256 * 8 - 1) / (256 * 8);
    hipLaunchKernelGGL(k_copy_f4, dim3((unsigned)grid), dim3(256), 0, s, (const u32x4 *)src, (u32x4 *)dst, n4);
    return hipGetLastError();
}

// Streaming read of n4 16-byte words, 8 loads per thread in flight, as the
// GEMV issues its weight tile: the attainable time of one launch that only
// has to move the same bytes.  The loaded words are folded into one value
// that is stored only if it equals `never` (the host passes a value the
// data cannot fold to), so the loads stay and nothing is written.
__global__ void __launch_bounds__(256) k_read_f4(const u32x4 *__restrict__ src, int64_t n4, uint32_t never,
                                                 uint32_t *sink)
{
    constexpr int U = 8;
    const int64_t base = (int64_t)blockIdx.x * 256 * U + threadIdx.x;
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int64_t i = base + (int64_t)u * 256;
        v[u] = __builtin_nontemporal_load(src + (i < n4 ? i : n4 - 1));
    }
    // every load issued before the first wait (the default schedule
    // otherwise waits after every second load: 3.04 against 2.57 us for a
    // 7.1 MB read)
    __builtin_amdgcn_sched_barrier(0);
    uint32_t acc = 0;
#pragma unroll
    for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (acc == never) sink[0] = acc;
}

hipError_t enqueue_read(const float *src, int64_t n, uint32_t never, uint32_t *sink, hipStream_t s)
{
    if (n <= 0 || n % 4) return hipErrorInvalidValue;
    const int64_t n4 = n / 4;
    const int64_t grid = (n4 + 256 * 8 - 1) / (256 * 8);
    hipLaunchKernelGGL(k_read_f4, dim3((unsigned)grid), dim3(256), 0, s, (const u32x4 *)src, n4, never, sink);
    return hipGetLastError();
}

hipError_t enqueue_gateup_timing(const TalkerDev &m, const Workspace &ws, int l, hipStream_t s)
{
    const LayerDev &L = m.layers[l];
    const ProResidRms<1, 2048> pre{ws.xb, m.hidden, ws.part_o, L.o.S, 1, 0, L.o.npad, nullptr, L.post_norm, m.hidden,
                             nullptr, nullptr};
    if (L.gate_up.S == 1 && tile_shape(L.gate_up.cfg).GB % 2 == 0)
        return launch_gemv<1>(L.gate_up, pre, EpiSwiglu<1>{ws.h, m.inter}, s);
    return launch_gemv<1>(L.gate_up, pre, EpiPart<1>{ws.part_gu, L.gate_up.npad}, s);
}

hipError_t enqueue_attn_timing(const TalkerDev &m, const Workspace &ws, int l, int slot, int64_t pos,
                               const DevState *st, int attn_pg, hipStream_t s)
{
    const LayerDev &L = m.layers[l];
    // a decode step's attention: appends at the free slot `slot` (beyond the
    // cached length, so cached positions are untouched) and attends slot+1
    if (attn_pg == 2) {
        hipLaunchKernelGGL(k_talker_attn<2>, dim3(8 * ((ws.attn_grid / 8 + 1) / 2)), dim3(512), 0, s, ws.part_qkv,
                           L.qkv.S, L.qkv.npad, L.q_norm, L.k_norm, m.rope_cos, m.rope_sin, st, pos, slot, l, m.kv,
                           ws.am, ws.al, ws.aacc);
    } else {
        hipLaunchKernelGGL(k_talker_attn<1>, dim3(ws.attn_grid), dim3(256), 0, s, ws.part_qkv, L.qkv.S, L.qkv.npad,
                           L.q_norm, L.k_norm, m.rope_cos, m.rope_sin, st, pos, slot, l, m.kv, ws.am, ws.al, ws.aacc);
    }
    return hipGetLastError();
}

}  // namespace qtts
