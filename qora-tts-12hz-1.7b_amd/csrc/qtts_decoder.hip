// qtts_decoder.hip — the speech decoder (decode_to_audio, decoder.rs:395-584)
// on the device: 16 codebook indices per frame -> 24 kHz samples.
//
// Activations stay channel-first [channels][positions] as in the reference.
// Every convolution, projection and pointwise layer is one implicit GEMM on
// the matrix cores (k_conv_gemm; f32-accurate: operands split into f16 hi +
// lo, three f16 products per pair, f32 accumulation; f32 matrix
// instructions with QTTS_DEC_F32=1): rows = output channels, columns =
// positions, contraction = input channels x taps, with the im2col gather
// done while staging the activation tile:
//   causal_conv1d        conv.rs:114-228   taps at t + j*dil - (K-1)*dil
//   conv_transpose1d     conv.rs:247-349   stride phases, 1 or 2 taps each
//   ConvNeXt pw1 / pw2   decoder.rs:346-388, GELU / gamma-residual epilogues
//   transformer          decoder.rs:198-340, q|k|v, o (+ layer scale),
//                        gate|up rows interleaved (SwiGLU epilogue), down
// Epilogues fuse the bias, SnakeBeta (conv.rs:620-640) of the next stage,
// the residual adds and the layer scales.  Small kernels do the VQ gather,
// the column RMSNorm, RoPE, sliding-window attention, depthwise conv +
// LayerNorm and the one-channel output conv with its clamp.

#include "qtts_device.h"
#include "qtts_kernels.h"
#include "qtts_devutil.h"
#include "qtts_mfma.h"
#include "qtts_snake.h"

#include <algorithm>

namespace qtts {

// ---------------------------------------------------------------------------
// implicit-GEMM convolution
// ---------------------------------------------------------------------------

constexpr int CGN = MFMA_N, CGK = MFMA_K, CLD = MFMA_LD;

// Read (never written) in place of out-of-range taps; a plain global
// (not const) so that selecting between it and an activation pointer
// stays in the global address space.
__device__ __attribute__((aligned(16))) float k_zero[4] = {0.0f, 0.0f, 0.0f, 0.0f};

enum ConvEpi : int {
    CE_STORE = 0,        // y = acc + bias
    CE_SNAKE = 1,        // y = snake(acc + bias)
    CE_STORE_SNAKE = 2,  // x = acc + bias (+ res); y = snake(x)
    CE_GELU = 3,         // y = gelu(acc + bias)
    CE_SCALE_RES = 4,    // y += scale * (acc + bias)
    CE_SWIGLU = 5,       // rows (2j, 2j+1) = (gate, up): y[j] = silu(gate) * up
};

struct ConvIn {
    const float *x;      // [IC][L_in] (row stride ldx)
    int ldx, L_in;
    int IC, K, dil, pad; // tap j of channel ic reads x[ic][t + j*dil - pad]
};

struct ConvOut {
    float *y;            // y[oc * ldy + t * os + oo]
    int ldy, os, oo;
    const float *bias;   // [M] or null
    const float *res;    // CE_STORE_SNAKE: residual added to x (same indexing), or null
    float *x;            // CE_STORE_SNAKE: pre-activation output
    const float *alpha, *beta;   // snake parameters [M]
    const float *scale;  // CE_SCALE_RES: [M]
};

// Per-row constants of an epilogue and the element operation, shared by the
// GEMM's own epilogue and the split-K reduction.
struct RowPar {
    float bias, a, ib, scale;
};

template <int EPI>
__device__ __forceinline__ RowPar row_par(const ConvOut &o, int m)
{
    RowPar r;
    r.bias = o.bias ? o.bias[m] : 0.0f;
    r.a = (EPI == CE_SNAKE || EPI == CE_STORE_SNAKE) ? expf(o.alpha[m]) : 0.0f;
    r.ib = (EPI == CE_SNAKE || EPI == CE_STORE_SNAKE) ? expf(-o.beta[m]) : 0.0f;
    r.scale = EPI == CE_SCALE_RES ? o.scale[m] : 0.0f;
    return r;
}

// The element the epilogue reads at idx before storing there: y of
// CE_SCALE_RES, the residual of CE_STORE_SNAKE (none when o.res is null).
template <int EPI>
constexpr bool epi_reads() { return EPI == CE_SCALE_RES || EPI == CE_STORE_SNAKE; }

template <int EPI>
__device__ __forceinline__ const float *epi_src(const ConvOut &o)
{
    return EPI == CE_SCALE_RES ? o.y : EPI == CE_STORE_SNAKE ? o.res : nullptr;
}

// ext: the element epi_src() holds at idx (read by the caller).
template <int EPI>
__device__ __forceinline__ void epi_store(const ConvOut &o, const RowPar &r, size_t idx, float acc, float ext)
{
    const float v = acc + r.bias;
    if (EPI == CE_STORE) {
        o.y[idx] = v;
    } else if (EPI == CE_GELU) {
        o.y[idx] = v * 0.5f * (1.0f + tanhf(v * 0.7071067811865476f));
    } else if (EPI == CE_SCALE_RES) {
        o.y[idx] = ext + r.scale * v;
    } else {
        const float xv = (EPI == CE_STORE_SNAKE && o.res) ? v + ext : v;
        if (EPI == CE_STORE_SNAKE) o.x[idx] = xv;
        o.y[idx] = xv + r.ib * snake_sin2(r.a * xv);
    }
}

// SwiGLU rows (2j, 2j + 1) = (gate, up) -> y[j]; bg, bu: their biases (0
// without)
__device__ __forceinline__ void epi_swiglu(const ConvOut &o, int m, size_t col, float g, float u, float bg, float bu)
{
    g += bg;
    u += bu;
    o.y[(size_t)(m >> 1) * o.ldy + col] = silu_f(g) * u;
}

// Contraction order: general, k = ic * K + tap (the [out][in][kernel]
// weight rows as they are); tap-major (TM), k = tap * IC + ic, for K = 1
// or IC a multiple of the 32-wide chunk, so that a chunk has one tap and
// the im2col gather needs no division per element (weights repacked to
// [out][kernel][in] at upload, conv_tap_major()).
//
// Launch geometry (GemmGeo): tm x tn output tiles, times nph stride phases
// of a transposed conv (phase ph uses A + ph * M * Kd and writes columns
// n * os + ph), times ks contraction slices.  With ks > 1 each slice writes
// its raw sums to part[slice][ph][M][N] and k_conv_reduce adds the slices
// in order and applies the epilogue.
struct GemmGeo {
    int tm, tn, nph, ks, cps;   // cps: 32-wide chunks per slice
    float *part;
    int32_t *range_flag;        // X3: set when a workgroup's staged inputs leave the split's range
};

// The second half of a Vocos residual unit, fused behind its k 7 conv
// (FUSE): the 1x1 conv [BM][BM] weights, and its output (x += conv + bias,
// y = the next snake of x, CE_STORE_SNAKE with the residual x).
struct ConvFuse {
    const float *A2;
    ConvOut o2;
};

// X3: the split-f16 contraction (qtts_mfma.h): weights and gathered inputs
// staged as f16 hi + lo, three f16 matrix products per pair, f32
// accumulation; otherwise v_mfma_f32_16x16x4_f32 on f32 operands.  On X3
// a B lane stages 16 consecutive k of its column (quads 4bq..4bq+3, two
// 16-byte writes per half: 16 columns 20 dwords apart cover the 64 banks
// once), and the A rows of each 16-row block are staged in 4 x 4
// transposed order (the 4 rows of a half-wave write 80 dwords apart,
// disjoint bank ranges).

template <int MB, int EPI, bool TM, bool X3, bool FUSE = false>
__global__ void __launch_bounds__(256, 2)
k_conv_gemm(const float *A, int M, int Kd, ConvIn in, ConvOut o, int N, GemmGeo g, ConvFuse fz)
{
    constexpr int BM = 16 * MB;
    constexpr int NA = (BM * CGK / 4 + 255) / 256;
    constexpr int XSTRIDE = (BM + CGN) * MFMA_HLD;   // halves per (buffer, half) on X3
    constexpr int F32_BYTES = 2 * (BM + CGN) * CLD * 4, X3_BYTES = 2 * 2 * XSTRIDE * 2;
    constexpr int TILE_BYTES = X3 ? X3_BYTES : F32_BYTES;
    // FUSE: the 1x1 conv's B operand, BM channels in BM / 32 chunks of hi and
    // lo [CGN][HLD] tiles, then one A tile pair [BM][HLD]
    constexpr int B2_HALVES = CGN * MFMA_HLD;
    constexpr int FUSE_BYTES = (2 * (BM / CGK) * B2_HALVES + 2 * BM * MFMA_HLD) * 2;
    constexpr int REGION = FUSE && FUSE_BYTES > TILE_BYTES ? FUSE_BYTES : TILE_BYTES;
    constexpr int WMX_BYTES = FUSE ? 32 : 16;
    static_assert(!FUSE || (X3 && TM && EPI == CE_SNAKE && BM % CGK == 0),
                  "the fused 1x1 conv takes a split-f16 k 7 conv");
    // the staging tiles first (their bank layout assumes the block's base),
    // then the range check's per-wave maxima and the epilogue's row constants
    __shared__ __attribute__((aligned(16))) unsigned char lds[REGION + WMX_BYTES + 16 * BM];
    // f32: As[2][BM*CLD], Bs[2][CGN*CLD]; X3: per buffer Ah, Al [BM*HLD] and Bh, Bl [CGN*HLD]
    float(*As)[BM * CLD] = (float(*)[BM * CLD])lds;
    float(*Bs)[CGN * CLD] = (float(*)[CGN * CLD])(lds + 2 * BM * CLD * 4);
    const auto ha = [&](int buf, int hl) { return (_Float16 *)lds + (size_t)(buf * 2 + hl) * XSTRIDE; };
    const auto hb = [&](int buf, int hl) { return ha(buf, hl) + (size_t)BM * MFMA_HLD; };
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int tiles = g.tm * g.tn;
    int tile, ph, slice;
    if (g.nph > 1 && g.ks == 1 && tiles % 8 == 0) {
        // The stride phases of a tile 8 workgroup indices apart: workgroup i
        // runs on XCD i mod 8, so they share an XCD and are dispatched
        // together, and the output lines they interleave into (column
        // n * nph + ph) are completed in that XCD's L2 instead of from
        // several, one phase at a time.
        const int k = blockIdx.x >> 3;
        ph = k % g.nph;
        tile = (k / g.nph) * 8 + (blockIdx.x & 7);
        slice = 0;
    } else {
        tile = blockIdx.x % tiles;
        const int rest = blockIdx.x / tiles;
        ph = rest % g.nph;
        slice = rest / g.nph;
    }
    const int mt = tile % g.tm, nt = tile / g.tm;
    const int m0 = mt * BM, n0 = nt * CGN;
    A += (size_t)ph * M * Kd;
    if (g.nph > 1) o.oo = ph;
    const int c0 = slice * g.cps;
    const int nch = min(g.cps, (Kd + CGK - 1) / CGK - c0);
    const int kb = c0 * CGK;

    // A slots: row slot/8, k 4*(slot%8)
    const float *arow[NA];
    int aoff[NA], akk[NA];
    bool aok[NA];
#pragma unroll
    for (int j = 0; j < NA; j++) {
        const int slot = min(t + 256 * j, BM * CGK / 4 - 1);
        const int rr = slot >> 3;
        const int r = X3 ? (rr & ~15) | ((rr & 3) << 2) | ((rr >> 2) & 3) : rr, m = m0 + r;
        aok[j] = m < M;
        arow[j] = A + (size_t)min(m, M - 1) * Kd;
        aoff[j] = r * CLD + 4 * (slot & 7);
        akk[j] = 4 * (slot & 7);
    }
    // B: column n0 + (t & 127); k quads bq, bq + 2, bq + 4, bq + 6 of the chunk (X3: 4bq..4bq+3)
    const int bcol = t & 127, bq = t >> 7;
    const int pos0 = n0 + bcol;
    const bool bcok = pos0 < N;
    const float *xb = in.x;

    // Interior chunks (tap-major): every row, k, tap position and column of
    // the tile in range, decided per chunk from wave-uniform values.  Each
    // load is then a wave-uniform base (scalar registers) plus a per-lane
    // byte offset fixed for the whole contraction: no per-lane address
    // arithmetic, compare or select per load.
    const int bqu = __builtin_amdgcn_readfirstlane(bq);   // t >> 7: one value per wave
    const bool tile_in = m0 + BM <= M && n0 + CGN <= N && (size_t)M * Kd < (size_t{1} << 30);
    const unsigned b_vo = 4u * (unsigned)pos0;
    unsigned a_vo[NA];
#pragma unroll
    for (int j = 0; j < NA; j++) a_vo[j] = 4u * (unsigned)((arow[j] - A) + akk[j]);

    struct Fetch {
        f32x4 a[NA];
        f32x4 b[4];
    };
    auto fetch = [&](Fetch &f, int k0) {
        if (TM) {
            const int tap = k0 / in.IC, icb = k0 - tap * in.IC;
            const int pofs = tap * in.dil - in.pad;
            if (tile_in && k0 + CGK <= Kd && icb + CGK <= in.IC && n0 + pofs >= 0 && n0 + CGN + pofs <= in.L_in) {
                const char *ab = (const char *)(A + k0);
#pragma unroll
                for (int j = 0; j < NA; j++) f.a[j] = ld4((const float *)(ab + a_vo[j]));
                const size_t ldx4 = (size_t)in.ldx * 4;
                const char *xr = (const char *)(xb + (size_t)icb * in.ldx + pofs);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const char *row = xr + (size_t)(4 * (X3 ? 4 * bqu + i : bqu + 2 * i)) * ldx4;
                    float v[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) v[e] = *(const float *)(row + e * ldx4 + b_vo);
                    f.b[i] = f32x4{v[0], v[1], v[2], v[3]};
                }
                return;
            }
        }
        // Out-of-range rows, chunk tails and taps read k_zero: selecting the
        // address rather than the value keeps every load unconditional (a
        // select on the value lets the compiler sink each load into a
        // branch of its own, or compute both sides, and wait on it there).
        // Kd is a multiple of 4 (conv_gemm checks), so a quad is in or out.
#pragma unroll
        for (int j = 0; j < NA; j++) {
            const int kk = k0 + akk[j];
            f.a[j] = ld4((aok[j] && kk < Kd) ? arow[j] + kk : k_zero);
        }
        if (TM) {
            const int tap = k0 / in.IC, icb = k0 - tap * in.IC;
            const int p = pos0 + tap * in.dil - in.pad;
            const bool pok = bcok && p >= 0 && p < in.L_in;
            const float *xp = xb + min(max(p, 0), in.L_in - 1);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int ic = icb + 4 * (X3 ? 4 * bq + i : bq + 2 * i);
                const float *row = xp + (size_t)ic * in.ldx;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float *src = (pok && ic + e < in.IC) ? row + (size_t)e * in.ldx : k_zero;
                    v[e] = *src;
                }
                f.b[i] = f32x4{v[0], v[1], v[2], v[3]};
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int kq = X3 ? 4 * bq + i : bq + 2 * i;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int kk = k0 + 4 * kq + e;
                    const int ic = kk / in.K, tap = kk - ic * in.K;
                    const int p = pos0 + tap * in.dil - in.pad;
                    const bool ok = bcok && kk < Kd && p >= 0 && p < in.L_in;
                    v[e] = *(ok ? xb + (size_t)ic * in.ldx + p : k_zero);
                }
                f.b[i] = f32x4{v[0], v[1], v[2], v[3]};
            }
        }
    };
    // X3: largest |input| this thread stages (the range check below)
    float bmax = 0.0f;
    auto stage = [&](const Fetch &f, int buf) {
        if constexpr (X3) {
            // a chain, two values per step: one v_max3 with |.| modifiers each
#pragma unroll
            for (int i = 0; i < 4; i++) {
                bmax = fmaxf(fmaxf(bmax, fabsf(f.b[i].x)), fabsf(f.b[i].y));
                bmax = fmaxf(fmaxf(bmax, fabsf(f.b[i].z)), fabsf(f.b[i].w));
            }
#pragma unroll
            for (int j = 0; j < NA; j++) {
                const int r = aoff[j] / CLD, kk = aoff[j] - r * CLD;
                uint32_t h01, l01, h23, l23;
                split_f16_pair(f.a[j].x, f.a[j].y, h01, l01);
                split_f16_pair(f.a[j].z, f.a[j].w, h23, l23);
                *(uint2 *)&ha(buf, 0)[r * MFMA_HLD + kk] = uint2{h01, h23};
                *(uint2 *)&ha(buf, 1)[r * MFMA_HLD + kk] = uint2{l01, l23};
            }
#pragma unroll
            for (int i = 0; i < 4; i += 2) {
                uint32_t h[4], l[4];
                split_f16_pair(f.b[i].x, f.b[i].y, h[0], l[0]);
                split_f16_pair(f.b[i].z, f.b[i].w, h[1], l[1]);
                split_f16_pair(f.b[i + 1].x, f.b[i + 1].y, h[2], l[2]);
                split_f16_pair(f.b[i + 1].z, f.b[i + 1].w, h[3], l[3]);
                *(uint4 *)&hb(buf, 0)[bcol * MFMA_HLD + 4 * (4 * bq + i)] = uint4{h[0], h[1], h[2], h[3]};
                *(uint4 *)&hb(buf, 1)[bcol * MFMA_HLD + 4 * (4 * bq + i)] = uint4{l[0], l[1], l[2], l[3]};
            }
        } else {
#pragma unroll
            for (int j = 0; j < NA; j++) *(f32x4 *)&As[buf][aoff[j]] = f.a[j];
#pragma unroll
            for (int i = 0; i < 4; i++) *(f32x4 *)&Bs[buf][bcol * CLD + 4 * (bq + 2 * i)] = f.b[i];
        }
    };

    const int r16 = lane & 15, q = lane >> 4;
    const int cb[2] = {2 * wv, 2 * wv + 1};      // wave w owns 16-column blocks 2w, 2w + 1
    f32x4 acc[MB][2];
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    mfma_pipeline<Fetch>(
        nch, [&](Fetch &f, int c) { fetch(f, kb + c * CGK); }, stage,
        [&](int buf) {
            if constexpr (X3)
                mfma_chunk_x3<MB>(acc, ha(buf, 0), ha(buf, 1), hb(buf, 0), hb(buf, 1), cb, lane);
            else
                mfma_chunk<MB>(acc, As[buf], Bs[buf], cb, lane);
        });

    // What the epilogue reads (the residual, or y of y += ...) at this
    // thread's outputs, loaded together once the contraction is done (its
    // registers are free then).  Read by the epilogue one element at a
    // time, between its stores to the same buffers, each load would wait
    // out a memory round trip of its own.
    float ext[epi_reads<EPI>() ? MB : 1][4][2];
    const float *esrc = epi_src<EPI>(o);
    if (epi_reads<EPI>() && g.ks == 1 && esrc) {
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + 16 * i + 4 * q + e;
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int n = n0 + 16 * (2 * wv + j) + r16;
                    ext[i][e][j] = *((m < M && n < N) ? esrc + (size_t)m * o.ldy + (size_t)n * o.os + o.oo : k_zero);
                }
            }
    }
    // The tile's per-row epilogue constants (bias, snake or scale), one row
    // per thread into LDS, for the same reason; the barrier below (the
    // range check's on X3) publishes them.
    float *rp = (float *)(lds + REGION + WMX_BYTES);   // [4][BM]: bias, a, ib, scale
    if (g.ks == 1 && t < BM) {
        const RowPar r = row_par<EPI>(o, min(m0 + t, M - 1));
        rp[t] = r.bias;
        rp[BM + t] = r.a;
        rp[2 * BM + t] = r.ib;
        rp[3 * BM + t] = r.scale;
    }
    // The split holds an input as f16 hi + lo: f32-accurate below the f16
    // maximum and, through lo, to 2^-25 absolute.  A workgroup whose inputs
    // reach 65504, or are all below 2^-14 but not zero, flags the decode,
    // which the host then repeats on the f32 matrix path.
    if constexpr (X3) {
        float *wmx = (float *)(lds + REGION);
        const float m = wave_max_dpp(bmax);
        if (lane == 0) wmx[wv] = m;
        __syncthreads();
        const float mx = fmaxf(fmaxf(wmx[0], wmx[1]), fmaxf(wmx[2], wmx[3]));
        if (t == 0 && g.range_flag && (!(mx < 65504.0f) || (mx > 0.0f && mx < 0x1p-14f))) *g.range_flag = 1;
    } else {
        if (g.ks == 1) __syncthreads();
    }
    if constexpr (FUSE) {
        // The rest of the Vocos residual unit in this workgroup (one row
        // tile holds all BM channels; no split): the k 7 conv's output
        // t1 = snake(acc + bias), formed as its epilogue would form it, goes
        // into LDS as f16 hi + lo -- the values the 1x1 conv's staging would
        // split after a round trip through memory (zero past column N, as it
        // would read there) -- then the 1x1 contraction over BM / 32 chunks
        // and its epilogue (x += conv + bias; y = the next snake of x).
        // Same operations in the same order as the two launches.
        _Float16 *b2 = (_Float16 *)lds;
        _Float16 *a2h = b2 + 2 * (BM / CGK) * B2_HALVES, *a2l = a2h + BM * MFMA_HLD;
        float *wmx = (float *)(lds + REGION);
        f32x4 av[BM / CGK][NA];   // the 1x1 weights, every chunk loaded first
#pragma unroll
        for (int c = 0; c < BM / CGK; c++)
#pragma unroll
            for (int j = 0; j < NA; j++) av[c][j] = ld4(fz.A2 + (size_t)(aoff[j] / CLD) * BM + c * CGK + akk[j]);
        float xr[MB][4][2];       // the residual x at this thread's outputs
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int m = 16 * i + 4 * q + e, n = n0 + 16 * (2 * wv + j) + r16;
                    xr[i][e][j] = *(n < N ? fz.o2.res + (size_t)m * fz.o2.ldy + n : k_zero);
                }
        float tmax = 0.0f;
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int cl = 16 * (2 * wv + j) + r16;
                const bool nok = n0 + cl < N;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int lr = 16 * i + 4 * q + e;
                    const float xv = acc[i][j][e] + rp[lr];
                    v[e] = nok ? xv + rp[2 * BM + lr] * snake_sin2(rp[BM + lr] * xv) : 0.0f;
                }
                tmax = fmaxf(fmaxf(tmax, fabsf(v[0])), fabsf(v[1]));
                tmax = fmaxf(fmaxf(tmax, fabsf(v[2])), fabsf(v[3]));
                uint32_t h01, l01, h23, l23;
                split_f16_pair(v[0], v[1], h01, l01);
                split_f16_pair(v[2], v[3], h23, l23);
                const int c = i >> 1, kk = 16 * (i & 1) + 4 * q;
                *(uint2 *)&b2[(2 * c) * B2_HALVES + cl * MFMA_HLD + kk] = uint2{h01, h23};
                *(uint2 *)&b2[(2 * c + 1) * B2_HALVES + cl * MFMA_HLD + kk] = uint2{l01, l23};
            }
        {
            const float m = wave_max_dpp(tmax);
            if (lane == 0) wmx[4 + wv] = m;
        }
        __syncthreads();   // t1 staged; every read of the k 7 conv's row constants done
        {
            const float mx = fmaxf(fmaxf(wmx[4], wmx[5]), fmaxf(wmx[6], wmx[7]));
            if (t == 0 && g.range_flag && (!(mx < 65504.0f) || (mx > 0.0f && mx < 0x1p-14f))) *g.range_flag = 1;
        }
        if (t < BM) {
            const RowPar r = row_par<CE_STORE_SNAKE>(fz.o2, t);
            rp[t] = r.bias;
            rp[BM + t] = r.a;
            rp[2 * BM + t] = r.ib;
        }
        f32x4 acc2[MB][2];
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) acc2[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < BM / CGK; c++) {
#pragma unroll
            for (int j = 0; j < NA; j++) {
                const int r = aoff[j] / CLD, kk = aoff[j] - r * CLD;
                uint32_t h01, l01, h23, l23;
                split_f16_pair(av[c][j].x, av[c][j].y, h01, l01);
                split_f16_pair(av[c][j].z, av[c][j].w, h23, l23);
                *(uint2 *)&a2h[r * MFMA_HLD + kk] = uint2{h01, h23};
                *(uint2 *)&a2l[r * MFMA_HLD + kk] = uint2{l01, l23};
            }
            __syncthreads();
            mfma_chunk_x3<MB>(acc2, a2h, a2l, b2 + (2 * c) * B2_HALVES, b2 + (2 * c + 1) * B2_HALVES, cb, lane);
            __syncthreads();
        }
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = 16 * i + 4 * q + e;
                const RowPar r = {rp[m], rp[BM + m], rp[2 * BM + m], 0.0f};
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int n = n0 + 16 * (2 * wv + j) + r16;
                    if (n < N)
                        epi_store<CE_STORE_SNAKE>(fz.o2, r, (size_t)m * fz.o2.ldy + n, acc2[i][j][e], xr[i][e][j]);
                }
            }
        return;
    }
    // element e of acc[i][j]: row 16i + 4q + e, column 16(2wv + j) + r16
    if (g.ks > 1) {
        float *pp = g.part + ((size_t)slice * g.nph + ph) * M * N;
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + 16 * i + 4 * q + e;
                if (m >= M) continue;
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int n = n0 + 16 * (2 * wv + j) + r16;
                    if (n < N) pp[(size_t)m * N + n] = acc[i][j][e];
                }
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < MB; i++) {
        if (EPI == CE_SWIGLU) {
#pragma unroll
            for (int e = 0; e < 4; e += 2) {
                const int m = m0 + 16 * i + 4 * q + e;   // even: gate row, m + 1: up row
                if (m + 1 >= M) continue;
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int n = n0 + 16 * (2 * wv + j) + r16;
                    if (n < N)
                        epi_swiglu(o, m, (size_t)n * o.os + o.oo, acc[i][j][e], acc[i][j][e + 1], rp[m - m0],
                                   rp[m - m0 + 1]);
                }
            }
            continue;
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int m = m0 + 16 * i + 4 * q + e;
            if (m >= M) continue;
            const int lr = m - m0;
            const RowPar r = {rp[lr], rp[BM + lr], rp[2 * BM + lr], rp[3 * BM + lr]};
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int n = n0 + 16 * (2 * wv + j) + r16;
                if (n < N)
                    epi_store<EPI>(o, r, (size_t)m * o.ldy + (size_t)n * o.os + o.oo, acc[i][j][e],
                                   epi_reads<EPI>() && esrc ? ext[epi_reads<EPI>() ? i : 0][e][j] : 0.0f);
            }
        }
    }
}

// Split-K reduction: thread per (phase, row, column) (row pairs for
// SwiGLU); slices added in slice order, then the epilogue.  The phase is
// the fastest index, so that consecutive threads store consecutive output
// columns n * nph + ph.  KS: the slice count when fixed at compile time (0:
// ks at run time), so that a thread's slice loads are all issued before the
// first addition instead of one round trip each.
template <int EPI, int KS>
__global__ void __launch_bounds__(256)
k_conv_reduce(const float *part, int ks_arg, int nph, int M, int N, ConvOut o)
{
    const int ks = KS ? KS : ks_arg;
    const int rows = EPI == CE_SWIGLU ? M / 2 : M;
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= (int64_t)nph * rows * N) return;
    const int ph = (int)(id % nph);
    const int64_t r2 = id / nph;
    const int n = (int)(r2 % N), mr = (int)(r2 / N);
    const size_t plane = (size_t)M * N;
    const size_t col = (size_t)n * o.os + (nph > 1 ? ph : o.oo);
    if (EPI == CE_SWIGLU) {
        const int m = 2 * mr;
        float gs = 0.0f, us = 0.0f;
        if constexpr (KS > 0) {
            float gv[KS > 0 ? KS : 1], uv[KS > 0 ? KS : 1];
#pragma unroll
            for (int sl = 0; sl < KS; sl++) {
                const float *pp = part + ((size_t)sl * nph + ph) * plane;
                gv[sl] = pp[(size_t)m * N + n];
                uv[sl] = pp[(size_t)(m + 1) * N + n];
            }
#pragma unroll
            for (int sl = 0; sl < KS; sl++) {
                gs += gv[sl];
                us += uv[sl];
            }
        } else {
            for (int sl = 0; sl < ks; sl++) {
                const float *pp = part + ((size_t)sl * nph + ph) * plane;
                gs += pp[(size_t)m * N + n];
                us += pp[(size_t)(m + 1) * N + n];
            }
        }
        epi_swiglu(o, m, col, gs, us, o.bias ? o.bias[m] : 0.0f, o.bias ? o.bias[m + 1] : 0.0f);
        return;
    }
    float sum = 0.0f;
    if constexpr (KS > 0) {
        float pv[KS > 0 ? KS : 1];
#pragma unroll
        for (int sl = 0; sl < KS; sl++) pv[sl] = part[((size_t)sl * nph + ph) * plane + (size_t)mr * N + n];
#pragma unroll
        for (int sl = 0; sl < KS; sl++) sum += pv[sl];
    } else {
        for (int sl = 0; sl < ks; sl++) sum += part[((size_t)sl * nph + ph) * plane + (size_t)mr * N + n];
    }
    const size_t idx = (size_t)mr * o.ldy + col;
    const float *esrc = epi_src<EPI>(o);
    epi_store<EPI>(o, row_par<EPI>(o, mr), idx, sum, esrc ? esrc[idx] : 0.0f);
}

// ---------------------------------------------------------------------------
// small kernels
// ---------------------------------------------------------------------------

// VQ inputs (codebook_lookup, decoder.rs:147-191) as one contraction of
// 2*D rows: rows 0..D-1 = first codebook row of code 0, rows D..2D-1 = the
// sum of the other codebooks' rows (added in codebook order).  codes
// [n_cb][T]; out [2D][T].  NR: the number of other codebooks when fixed at
// compile time (0: n_rest at run time); with it every code, row pointer and
// row value is loaded before the sum, not one dependent chain per codebook.
template <int NR>
__global__ void k_vq_gather(const float *first, const float *const *rest, int n_rest, int D, const uint32_t *codes,
                            int T, int rows_cb, float *out)
{
    const int d = blockIdx.y, t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= T) return;
    const uint32_t c0 = min(codes[t], (uint32_t)(rows_cb - 1));
    const float f = first[(size_t)c0 * D + d];
    float s = 0.0f;
    if constexpr (NR > 0) {
        uint32_t c[NR];
        const float *row[NR];
        float v[NR];
#pragma unroll
        for (int g = 0; g < NR; g++) c[g] = min(codes[(size_t)(g + 1) * T + t], (uint32_t)(rows_cb - 1));
#pragma unroll
        for (int g = 0; g < NR; g++) row[g] = rest[g];
#pragma unroll
        for (int g = 0; g < NR; g++) v[g] = row[g][(size_t)c[g] * D + d];
#pragma unroll
        for (int g = 0; g < NR; g++) s += v[g];
    } else {
        for (int g = 0; g < n_rest; g++) {
            const uint32_t c = min(codes[(size_t)(g + 1) * T + t], (uint32_t)(rows_cb - 1));
            s += rest[g][(size_t)c * D + d];
        }
    }
    out[(size_t)d * T + t] = f;
    out[(size_t)(D + d) * T + t] = s;
}

// Column RMSNorm (rms_norm_f32, decoder.rs:589-598) of x [H][T]:
// workgroup of 16 positions x COLRMS_CG channel groups; the sum of squares
// is the group partials added in group order.  At the 12 Hz shapes (512
// channels, 160 positions per decode) the grid is 10 workgroups, so each
// takes 16 waves.
constexpr int COLRMS_CG = 64;
__global__ void __launch_bounds__(16 * COLRMS_CG)
k_col_rms(const float *x, const float *gamma, int H, int T, float eps, float *out)
{
    __shared__ float red[COLRMS_CG][17];
    const int tl = threadIdx.x & 15, cg = threadIdx.x >> 4;
    const int t = blockIdx.x * 16 + tl;
    const bool ok = t < T;
    const float *xc = x + min(t, T - 1);
    float ss = 0.0f;
#pragma unroll 8
    for (int h = cg; h < H; h += COLRMS_CG) {
        const float v = xc[(size_t)h * T];
        ss = fmaf(v, v, ss);
    }
    red[cg][tl] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll 8
    for (int g = 0; g < COLRMS_CG; g++) tot += red[g][tl];
    const float inv = 1.0f / sqrtf(tot / (float)H + eps);
    if (!ok) return;
#pragma unroll 8
    for (int h = cg; h < H; h += COLRMS_CG) out[(size_t)h * T + t] = xc[(size_t)h * T] * inv * gamma[h];
}

// A column sum over the 1024 threads of a workgroup of 4 positions x 256
// channel groups (thread 4g + tl: group g, position tl): over the 16 groups
// of a wave by lane exchanges, then over the 16 waves in order.
__device__ __forceinline__ float col_sum_tp4(float v, float (*wred)[4], int tl)
{
#pragma unroll
    for (int m = 4; m < 64; m *= 2) v += __shfl_xor(v, m);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    if (lane < 4) wred[wv][lane] = v;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; q++) tot += wred[q][tl];
    return tot;
}

// The same on a grid four times wider, for H <= 1024: workgroups of 4
// positions x 256 channel groups (40 workgroups at 160 positions, where 16
// positions gave 10), each thread's values kept in registers between the
// two passes (the reload of x and the store of out no longer alternate:
// each reload after a store that may alias it waited out a round trip).
constexpr int COLRMS_NV = 4;
__global__ void __launch_bounds__(1024)
k_col_rms_r(const float *x, const float *gamma, int H, int T, float eps, float *out)
{
    __shared__ float wred[16][4];
    const int tl = threadIdx.x & 3, cg = threadIdx.x >> 2;
    const int t = blockIdx.x * 4 + tl;
    const bool ok = t < T;
    const float *xc = x + min(t, T - 1);
    float xv[COLRMS_NV], gv[COLRMS_NV];
#pragma unroll
    for (int u = 0; u < COLRMS_NV; u++) {
        const int h = min(cg + 256 * u, H - 1);
        xv[u] = xc[(size_t)h * T];
        gv[u] = gamma[h];
    }
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < COLRMS_NV; u++)
        if (cg + 256 * u < H) ss = fmaf(xv[u], xv[u], ss);
    const float inv = 1.0f / sqrtf(col_sum_tp4(ss, wred, tl) / (float)H + eps);
    if (!ok) return;
#pragma unroll
    for (int u = 0; u < COLRMS_NV; u++) {
        const int h = cg + 256 * u;
        if (h < H) out[(size_t)h * T + t] = xv[u] * inv * gv[u];
    }
}

// Rotate-half RoPE (apply_rope_split_half, decoder.rs:631-655) of the q and
// k rows of qkv [3A][T] in place; positions past the table stay unrotated.
__global__ void k_rope_cf(float *qkv, int heads, int hd, int T, const float *cs, const float *sn, int64_t rope_rows)
{
    const int t = blockIdx.x * blockDim.x + threadIdx.x, hi = blockIdx.y;   // hi: q heads then k heads
    const int half = hd / 2;
    if (t >= T || t >= rope_rows) return;
    float *b = qkv + (size_t)hi * hd * T;
    for (int i = 0; i < half; i++) {
        const float x0 = b[(size_t)i * T + t], x1 = b[(size_t)(half + i) * T + t];
        const float c = cs[(size_t)t * half + i], s = sn[(size_t)t * half + i];
        b[(size_t)i * T + t] = x0 * c - x1 * s;
        b[(size_t)(half + i) * T + t] = x1 * c + x0 * s;
    }
}

// Causal sliding-window attention (decoder.rs:264-291): thread per (head,
// query position); keys t-W+1..t; online softmax; out [A][T].
template <int HD>
__global__ void __launch_bounds__(64)
k_dec_attn(const float *qkv, int heads, int T, int W, float *out)
{
    const int t = blockIdx.x * blockDim.x + threadIdx.x, h = blockIdx.y;
    if (t >= T) return;
    const size_t A = (size_t)heads * HD;
    const float *q = qkv + (size_t)h * HD * T, *k = qkv + (A + (size_t)h * HD) * T, *v = qkv + (2 * A + (size_t)h * HD) * T;
    const float scale = 1.0f / sqrtf((float)HD);
    float qr[HD], acc[HD];
#pragma unroll
    for (int d = 0; d < HD; d++) {
        qr[d] = q[(size_t)d * T + t];
        acc[d] = 0.0f;
    }
    const int start = t + 1 > W ? t + 1 - W : 0;
    float m = -INFINITY, l = 0.0f;
    for (int s = start; s <= t; s++) {
        float dot = 0.0f;
#pragma unroll
        for (int d = 0; d < HD; d++) dot = fmaf(qr[d], k[(size_t)d * T + s], dot);
        const float sc = dot * scale;
        const float mn = fmaxf(m, sc);
        const float f = expf(m - mn), p = expf(sc - mn);
        l = l * f + p;
#pragma unroll
        for (int d = 0; d < HD; d++) acc[d] = fmaf(p, v[(size_t)d * T + s], acc[d] * f);
        m = mn;
    }
    const float il = 1.0f / l;
#pragma unroll
    for (int d = 0; d < HD; d++) out[((size_t)h * HD + d) * T + t] = acc[d] * il;
}

// Sliding-window attention, workgroup per (head, 16 queries): the key and
// value rows those queries see (positions t0-W+1 .. t0+15, zero before
// position 0) and the 16 query rows staged in LDS position-major, HD + 4
// floats a row (every global load issued first), q and k then rotated
// (RoPE) in place.  Scores: lane (query qi, key slot kl) holds keys
// kl + 16i, its query row in registers and each key row read as 16-byte
// vectors (rows 68 floats apart: 16 rows cover the 64 banks once), the dot
// product in dimension order; softmax max and sum over the 16 lanes of the
// query's row (DPP); then lane (qi, dim group kl) sums p.v for dims
// 4kl..4kl+3 over the query's W keys in position order (keys before
// position 0 have p = 0 and v = 0).  Needs W + 15 <= 16 * ATT_SLOTS.
constexpr int ATT_QB = 16, ATT_SLOTS = 7;

static inline size_t attn_tile_lds(int hd, int W)
{
    const int nk = ATT_QB + W - 1, kp = hd + 4;
    return (size_t)(2 * nk * kp + ATT_QB * kp + ATT_QB * (nk + 1)) * sizeof(float);
}

template <int HD>
__global__ void __launch_bounds__(256)
k_dec_attn_tile(const float *qkv, int heads, int T, int W, const float *cs, const float *sn, int64_t rope_rows,
                float *out)
{
    static_assert(HD % 4 == 0 && HD / 4 <= 16, "a lane's p.v takes 4 consecutive dims of 16 groups");
    extern __shared__ float sm[];
    constexpr int KP = HD + 4;                 // floats per staged row
    const int NK = ATT_QB + W - 1, NKP = NK + 1;
    const int h = blockIdx.y, t0 = blockIdx.x * ATT_QB, kb = t0 - (W - 1);
    const int tid = threadIdx.x;
    const size_t A = (size_t)heads * HD;
    const float *q = qkv + (size_t)h * HD * T, *k = qkv + (A + (size_t)h * HD) * T,
                *v = qkv + (2 * A + (size_t)h * HD) * T;
    float *Ks = sm, *Vs = Ks + NK * KP, *Qs = Vs + NK * KP, *Ps = Qs + ATT_QB * KP;
    // Every global load of the tile first (K and V of the window, Q of the
    // block, the RoPE values of the pairs this thread rotates; clamped, so
    // none is conditional), then the raw rows into LDS, then rotate-half
    // RoPE in place: the partner of dim d is dim d +- HD/2 of the same row.
    constexpr int half = HD / 2;
    constexpr int KE = (HD * 16 * ATT_SLOTS + 255) / 256;        // K / V elements per thread, at most
    constexpr int QE = (HD * ATT_QB + 255) / 256;                // Q elements per thread
    constexpr int KR = (half * 16 * ATT_SLOTS + 255) / 256;      // K pairs per thread, at most
    constexpr int QR = (half * ATT_QB + 255) / 256;              // Q pairs per thread
    float kraw[KE], vraw[KE], qraw[QE], kc[KR], ks[KR], qc[QR], qs[QR];
#pragma unroll
    for (int u = 0; u < KE; u++) {
        const int i = min(tid + u * 256, HD * NK - 1);
        const int d = i / NK, j = i - d * NK, pc = min(max(kb + j, 0), T - 1);
        kraw[u] = k[(size_t)d * T + pc];
        vraw[u] = v[(size_t)d * T + pc];
    }
#pragma unroll
    for (int u = 0; u < QE; u++) {
        const int i = min(tid + u * 256, HD * ATT_QB - 1);
        const int d = i / ATT_QB, j = i - d * ATT_QB;
        qraw[u] = q[(size_t)d * T + min(t0 + j, T - 1)];
    }
    const int64_t rmax = rope_rows - 1;
#pragma unroll
    for (int u = 0; u < KR; u++) {
        const int i = min(tid + u * 256, half * NK - 1);
        const int d = i / NK, j = i - d * NK;
        const int64_t pr = min((int64_t)min(max(kb + j, 0), T - 1), rmax);
        kc[u] = cs[pr * half + d];
        ks[u] = sn[pr * half + d];
    }
#pragma unroll
    for (int u = 0; u < QR; u++) {
        const int i = min(tid + u * 256, half * ATT_QB - 1);
        const int d = i / ATT_QB, j = i - d * ATT_QB;
        const int64_t pr = min((int64_t)min(t0 + j, T - 1), rmax);
        qc[u] = cs[pr * half + d];
        qs[u] = sn[pr * half + d];
    }
#pragma unroll
    for (int u = 0; u < KE; u++) {
        const int i = tid + u * 256;
        if (i < HD * NK) {
            const int d = i / NK, j = i - d * NK, p = kb + j;
            const bool ok = p >= 0 && p < T;
            Ks[j * KP + d] = ok ? kraw[u] : 0.0f;
            Vs[j * KP + d] = ok ? vraw[u] : 0.0f;
        }
    }
#pragma unroll
    for (int u = 0; u < QE; u++) {
        const int i = tid + u * 256;
        if (i < HD * ATT_QB) {
            const int d = i / ATT_QB, j = i - d * ATT_QB;
            Qs[j * KP + d] = t0 + j < T ? qraw[u] : 0.0f;
        }
    }
    __syncthreads();
    // positions past the table stay unrotated, as k_rope_cf leaves them;
    // positions outside the sequence hold zeros
#pragma unroll
    for (int u = 0; u < KR; u++) {
        const int i = tid + u * 256;
        if (i < half * NK) {
            const int d = i / NK, j = i - d * NK, p = kb + j;
            if (p >= 0 && p < T && p < rope_rows) {
                float *row = Ks + j * KP;
                const float x = row[d], xp = row[d + half];
                row[d] = x * kc[u] - xp * ks[u];
                row[d + half] = xp * kc[u] + x * ks[u];
            }
        }
    }
#pragma unroll
    for (int u = 0; u < QR; u++) {
        const int i = tid + u * 256;
        if (i < half * ATT_QB) {
            const int d = i / ATT_QB, j = i - d * ATT_QB, p = t0 + j;
            if (p < T && p < rope_rows) {
                float *row = Qs + j * KP;
                const float x = row[d], xp = row[d + half];
                row[d] = x * qc[u] - xp * qs[u];
                row[d + half] = xp * qc[u] + x * qs[u];
            }
        }
    }
    __syncthreads();
    const int qi = tid >> 4, kl = tid & 15;
    const float scale = 1.0f / sqrtf((float)HD);
    f32x4 qv[HD / 4];
#pragma unroll
    for (int e = 0; e < HD / 4; e++) qv[e] = *(const f32x4 *)(Qs + qi * KP + 4 * e);
    float sc[ATT_SLOTS];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < ATT_SLOTS; i++) {
        const int j = kl + 16 * i;
        const bool ok = j < NK && j >= qi && j <= qi + W - 1 && kb + j >= 0;
        float dot = 0.0f;
        if (ok) {
            const float *kr = Ks + j * KP;
#pragma unroll
            for (int e = 0; e < HD / 4; e++) {
                const f32x4 k4 = *(const f32x4 *)(kr + 4 * e);
                dot = fmaf(qv[e].x, k4.x, dot);
                dot = fmaf(qv[e].y, k4.y, dot);
                dot = fmaf(qv[e].z, k4.z, dot);
                dot = fmaf(qv[e].w, k4.w, dot);
            }
        }
        sc[i] = ok ? dot * scale : -INFINITY;
        m = fmaxf(m, sc[i]);
    }
    m = row_max16(m);
    float l = 0.0f;
#pragma unroll
    for (int i = 0; i < ATT_SLOTS; i++) {
        sc[i] = expf(sc[i] - m);
        l += sc[i];
    }
    l = row_sum16(l);
    const float il = 1.0f / l;
#pragma unroll
    for (int i = 0; i < ATT_SLOTS; i++) {
        const int j = kl + 16 * i;
        if (j < NK) Ps[qi * NKP + j] = sc[i] * il;
    }
    __syncthreads();
    const int t = t0 + qi;
    if (4 * kl >= HD) return;
    f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
    const float *pr = Ps + qi * NKP + qi;
    const float *vr = Vs + qi * KP + 4 * kl;
    for (int r = 0; r < W; r++) {
        const float pv = pr[r];
        const f32x4 v4 = *(const f32x4 *)(vr + r * KP);
        o.x = fmaf(pv, v4.x, o.x);
        o.y = fmaf(pv, v4.y, o.y);
        o.z = fmaf(pv, v4.z, o.z);
        o.w = fmaf(pv, v4.w, o.w);
    }
    if (t >= T) return;
    float *op = out + ((size_t)h * HD + 4 * kl) * T + t;
    op[0] = o.x;
    op[(size_t)T] = o.y;
    op[2 * (size_t)T] = o.z;
    op[3 * (size_t)T] = o.w;
}

// ConvNeXt front (decoder.rs:346-352): causal depthwise conv then LayerNorm
// over channels per position (layer_norm_channel_first, decoder.rs:668-690).
// Workgroup of 16 positions x DWLN_CG channel groups: thread (cg, tl) takes
// position 16*blockIdx.x + tl and channels cg, cg + DWLN_CG, ...; the conv
// values go to the output buffer, then the column statistics (group
// partials summed in group order).  At the 12 Hz shapes (1024 channels,
// 320 and 640 positions) the grid is 20-40 workgroups, so each takes 16
// waves: a thread walks 16 channels, not 64.
constexpr int DWLN_CG = 64;
__global__ void __launch_bounds__(16 * DWLN_CG)
k_dw_ln(const float *x, int C, int L, const float *dw_w, const float *dw_b, int K, const float *g, const float *b,
        float eps, float *out)
{
    __shared__ float red[2][DWLN_CG][17];
    const int tl = threadIdx.x & 15, cg = threadIdx.x >> 4;
    const int t = blockIdx.x * 16 + tl;
    const bool ok = t < L;
    const int tc = min(t, L - 1);
    float s1 = 0.0f;
#pragma unroll 4
    for (int c = cg; c < C; c += DWLN_CG) {
        const float *xr = x + (size_t)c * L;
        const float *wr = dw_w + (size_t)c * K;
        float v = dw_b[c];
#pragma unroll 7
        for (int k = 0; k < K; k++) {
            const int p = tc + k - (K - 1);
            v += p >= 0 ? xr[max(p, 0)] * wr[k] : 0.0f;
        }
        if (ok) out[(size_t)c * L + t] = v;
        s1 += v;
    }
    red[0][cg][tl] = s1;
    __syncthreads();
    float mean = 0.0f;
#pragma unroll 8
    for (int q = 0; q < DWLN_CG; q++) mean += red[0][q][tl];
    mean /= (float)C;
    float s2 = 0.0f;
#pragma unroll 8
    for (int c = cg; c < C; c += DWLN_CG) {
        const float d = ok ? out[(size_t)c * L + t] - mean : 0.0f;
        s2 += d * d;
    }
    red[1][cg][tl] = s2;
    __syncthreads();
    float var = 0.0f;
#pragma unroll 8
    for (int q = 0; q < DWLN_CG; q++) var += red[1][q][tl];
    var /= (float)C;
    const float inv = 1.0f / sqrtf(var + eps);
    if (!ok) return;
#pragma unroll 8
    for (int c = cg; c < C; c += DWLN_CG) out[(size_t)c * L + t] = (out[(size_t)c * L + t] - mean) * inv * g[c] + b[c];
}

// The same for the ConvNeXt kernel of 7 taps and C <= DWLN_CMAX, on a grid
// four times wider: workgroups of DWLN_TP = 4 positions x 256 channel
// groups (80-160 workgroups at the 12 Hz shapes, where 16 positions gave
// 20-40).  The conv values and the affine parameters are kept in LDS (a
// store there cannot alias the next channel's global loads); a column's
// sums are taken over the 16 groups of a wave by lane exchanges, then over
// the 16 waves in order.
constexpr int DWLN_CMAX = 1024, DWLN_K = 7, DWLN_TP = 4, DWLN_G = 1024 / DWLN_TP;
static_assert(DWLN_TP == 4, "col_sum_tp4 sums columns of 4 positions");
__global__ void __launch_bounds__(1024)
k_dw_ln_r(const float *x, int C, int L, const float *dw_w, const float *dw_b, const float *g, const float *b, float eps,
          float *out)
{
    __shared__ float wred[2][16][DWLN_TP];
    __shared__ float vs[DWLN_CMAX][DWLN_TP + 1];
    __shared__ float gs[DWLN_CMAX], bs[DWLN_CMAX];
    const int tl = threadIdx.x & (DWLN_TP - 1), cg = threadIdx.x / DWLN_TP;
    const int t = blockIdx.x * DWLN_TP + tl;
    const bool ok = t < L;
    const int tc = min(t, L - 1);
    float s1 = 0.0f;
#pragma unroll 4
    for (int c = cg; c < C; c += DWLN_G) {
        const float *xr = x + (size_t)c * L;
        const float *wr = dw_w + (size_t)c * DWLN_K;
        float v = dw_b[c];
#pragma unroll
        for (int k = 0; k < DWLN_K; k++) {
            const int p = tc + k - (DWLN_K - 1);
            v += p >= 0 ? xr[max(p, 0)] * wr[k] : 0.0f;
        }
        vs[c][tl] = v;
        s1 += v;
        if (tl == 0) {
            gs[c] = g[c];
            bs[c] = b[c];
        }
    }
    const float mean = col_sum_tp4(s1, wred[0], tl) / (float)C;
    float s2 = 0.0f;
#pragma unroll 4
    for (int c = cg; c < C; c += DWLN_G) {
        const float d = ok ? vs[c][tl] - mean : 0.0f;
        s2 += d * d;
    }
    const float var = col_sum_tp4(s2, wred[1], tl) / (float)C;
    const float inv = 1.0f / sqrtf(var + eps);
    if (!ok) return;
#pragma unroll 4
    for (int c = cg; c < C; c += DWLN_G) out[(size_t)c * L + t] = (vs[c][tl] - mean) * inv * gs[c] + bs[c];
}

// Output conv (one channel, causal, conv.rs:191-228) on the snake input,
// clamp to [-1, 1] (decoder.rs:567-570), written from sample `cut` on.
// Workgroup per 256 samples; 16-channel slabs of the input with the
// (K-1)*dil left halo (at most OUT_HALO, zero before position 0) staged in
// LDS through registers, the next slab's loads in flight while the current
// one is summed; each thread sums channel by channel, taps in order.
constexpr int OUT_HALO = 64;

__global__ void __launch_bounds__(256)
k_out_conv(const float *x, int C, int L, const float *w, float bias, int K, int dil, int64_t cut, float *out)
{
    constexpr int W = 256 + OUT_HALO;
    constexpr int PER = 16 * W / 256;             // slab values per thread
    static_assert(16 * W % 256 == 0, "whole slabs per thread");
    __shared__ float xs[16][W];
    const int tl = threadIdx.x, t0 = blockIdx.x * 256, t = t0 + tl;
    const int pad = (K - 1) * dil;
    // a slab's values in registers: all PER loads issued together, the next
    // slab's while the current one is summed (the last slab loads itself
    // again, in bounds, rather than branch around the loads)
    float v[PER];
    const auto fetch = [&](int c0) {
        const int nc = min(16, C - c0);
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int idx = tl + i * 256, cc = idx / W, j = idx - cc * W, p = t0 - pad + j;
            const bool ok = cc < nc && p >= 0 && p < L;
            v[i] = *(ok ? x + (size_t)(c0 + cc) * L + p : k_zero);
        }
    };
    fetch(0);
    float s = bias;
    for (int c0 = 0; c0 < C; c0 += 16) {
        const int nc = min(16, C - c0);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int idx = tl + i * 256, cc = idx / W, j = idx - cc * W;
            xs[cc][j] = v[i];
        }
        __syncthreads();
        fetch(c0 + 16 < C ? c0 + 16 : c0);
        for (int cc = 0; cc < nc; cc++) {
            const float *wr = w + (size_t)(c0 + cc) * K;
            for (int k = 0; k < K; k++) s += xs[cc][tl + k * dil] * wr[k];
        }
    }
    if (t >= L || t < cut) return;
    out[t - cut] = s < -1.0f ? -1.0f : (s > 1.0f ? 1.0f : s);
}

// SnakeBeta over [C][L] (snake_beta, conv.rs:545-640), out-of-place.
__global__ void k_snake(const float *x, int C, int L, const float *alpha, const float *beta, float *out)
{
    const int t = blockIdx.x * blockDim.x + threadIdx.x, c = blockIdx.y;
    if (t >= L) return;
    const float a = expf(alpha[c]), ib = expf(-beta[c]);
    const float v = x[(size_t)c * L + t];
    out[(size_t)c * L + t] = v + ib * snake_sin2(a * v);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

#define DCHK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) return e_; } while (0)

// Row-tile height 16 * MB: 96 rows when they divide M (the Vocos channel
// counts 1536 ... 96), else 64 / 32 / 16.  The 96-row tile is built for
// the tap-major path only (every large conv); 128 rows would spill at two
// workgroups per CU.
static int conv_mb(int M, bool tm)
{
    if (tm && M % 96 == 0) return 6;
    return M >= 64 ? 4 : (M >= 32 ? 2 : 1);
}

// Vocos residual units fused where they fit (vocos_res_fused) unless
// QTTS_DEC_FUSE_VOC=0 (read at every launch, as dec_x3)
static bool dec_fuse_voc()
{
    const char *v = getenv("QTTS_DEC_FUSE_VOC");
    return !(v && *v == '0');
}

// the split-f16 contraction unless QTTS_DEC_F32=1
static bool dec_x3()
{
    // read at every launch (a few hundred ns), so a caller or test can switch
    // paths between calls
    const char *v = getenv("QTTS_DEC_F32");
    return !(v && *v && *v != '0');
}

template <int EPI, bool TM, bool X3>
static void conv_launch_x(int mb, dim3 grid, const float *A, int M, int Kd, const ConvIn &in, const ConvOut &o, int N,
                          const GemmGeo &g, hipStream_t s)
{
    switch (mb) {
    case 6:
        if constexpr (TM)
            hipLaunchKernelGGL((k_conv_gemm<6, EPI, TM, X3>), grid, dim3(256), 0, s, A, M, Kd, in, o, N, g, ConvFuse{});
        break;
    case 4:
        hipLaunchKernelGGL((k_conv_gemm<4, EPI, TM, X3>), grid, dim3(256), 0, s, A, M, Kd, in, o, N, g, ConvFuse{});
        break;
    case 2:
        hipLaunchKernelGGL((k_conv_gemm<2, EPI, TM, X3>), grid, dim3(256), 0, s, A, M, Kd, in, o, N, g, ConvFuse{});
        break;
    default:
        hipLaunchKernelGGL((k_conv_gemm<1, EPI, TM, X3>), grid, dim3(256), 0, s, A, M, Kd, in, o, N, g, ConvFuse{});
        break;
    }
}

template <int EPI, bool TM>
static void conv_launch(int mb, dim3 grid, const float *A, int M, int Kd, const ConvIn &in, const ConvOut &o, int N,
                        const GemmGeo &g, bool f32, hipStream_t s)
{
    if (!f32 && dec_x3())
        conv_launch_x<EPI, TM, true>(mb, grid, A, M, Kd, in, o, N, g, s);
    else
        conv_launch_x<EPI, TM, false>(mb, grid, A, M, Kd, in, o, N, g, s);
}

// Contraction slices: split K while the launch has fewer than 2 workgroups
// per CU and each slice keeps at least 4 chunks, within the partial buffer.
static int pick_ks(int blocks, int nch, size_t plane_floats, const DecoderWs &ws)
{
    int ks = 1;
    while (blocks * ks < 512 && nch / (2 * ks) >= 4 && (size_t)(2 * ks) * plane_floats <= ws.part_cap) ks *= 2;
    return ks;
}

// One implicit-GEMM convolution (nph > 1: the stride phases of a
// transposed conv, A holding nph consecutive [M][Kd] matrices).  A's rows
// are tap-major exactly when conv_tap_major(IC, K) (upload repacks by the
// same predicate).
template <int EPI>
static hipError_t conv_gemm(const float *A, int M, const ConvIn &in, const ConvOut &o, int N, const DecoderWs &ws,
                            hipStream_t s, int nph = 1)
{
    const int Kd = in.IC * in.K;
    if (M < 1 || N < 1 || Kd < 1 || (Kd & 3) || nph < 1 || (EPI == CE_SWIGLU && (M & 1))) return hipErrorInvalidValue;
    const bool tm = conv_tap_major(in.IC, in.K);
    const int mb = conv_mb(M, tm);
    GemmGeo g{};
    g.tm = (M + 16 * mb - 1) / (16 * mb);
    g.tn = (N + CGN - 1) / CGN;
    g.nph = nph;
    const int nch = (Kd + CGK - 1) / CGK;
    g.ks = pick_ks(g.tm * g.tn * nph, nch, (size_t)nph * M * N, ws);
    g.cps = (nch + g.ks - 1) / g.ks;
    g.ks = (nch + g.cps - 1) / g.cps;   // no empty slice
    g.part = ws.part;
    g.range_flag = ws.range_flag;
    const dim3 grid(g.tm * g.tn * nph * g.ks);
    if (tm)
        conv_launch<EPI, true>(mb, grid, A, M, Kd, in, o, N, g, ws.f32, s);
    else
        conv_launch<EPI, false>(mb, grid, A, M, Kd, in, o, N, g, ws.f32, s);
    DCHK(hipGetLastError());
    if (g.ks > 1) {
        const int64_t n = (int64_t)nph * (EPI == CE_SWIGLU ? M / 2 : M) * N;
        const dim3 rg((unsigned)((n + 255) / 256));
        if (g.ks == 2)
            hipLaunchKernelGGL((k_conv_reduce<EPI, 2>), rg, dim3(256), 0, s, ws.part, g.ks, nph, M, N, o);
        else if (g.ks == 4)
            hipLaunchKernelGGL((k_conv_reduce<EPI, 4>), rg, dim3(256), 0, s, ws.part, g.ks, nph, M, N, o);
        else if (g.ks == 8)
            hipLaunchKernelGGL((k_conv_reduce<EPI, 8>), rg, dim3(256), 0, s, ws.part, g.ks, nph, M, N, o);
        else
            hipLaunchKernelGGL((k_conv_reduce<EPI, 0>), rg, dim3(256), 0, s, ws.part, g.ks, nph, M, N, o);
        DCHK(hipGetLastError());
    }
    return hipSuccess;
}

static ConvIn causal_in(const float *x, int IC, int L, int K, int dil)
{
    return ConvIn{x, L, L, IC, K, dil, (K - 1) * dil};
}

static ConvOut plain_out(float *y, int ld, const float *bias);

// A Vocos residual unit -- conv1 (k, dilation) + snake, then the 1x1
// conv2 + residual + the next snake (conv.rs, decoder.rs:515-540) -- as one
// launch (k_conv_gemm's FUSE form) where its channels fill one 96-row tile
// and conv1 needs no split of its contraction.  sn: conv1's input; the next
// snake goes to out_sn (conv1's neighbouring tiles still read sn); x: the
// residual, updated in place.  *done = false: nothing launched, the caller
// runs the two convs.
static hipError_t vocos_res_fused(const DecVocosRes &R, int ch, const float *sn, float *out_sn, float *x, int L,
                                  const float *next_alpha, const float *next_beta, const DecoderWs &ws, hipStream_t s,
                                  bool *done)
{
    *done = false;
    if (ch != 96 || ws.f32 || !dec_fuse_voc() || R.c2.k != 1 || !conv_tap_major(ch, R.c1.k) || conv_mb(ch, true) != 6)
        return hipSuccess;
    const int Kd = ch * R.c1.k, nch = (Kd + CGK - 1) / CGK, tn = (L + CGN - 1) / CGN;
    if (Kd & 3 || pick_ks(tn, nch, (size_t)ch * L, ws) != 1) return hipSuccess;
    GemmGeo g{};
    g.tm = 1;
    g.tn = tn;
    g.nph = 1;
    g.ks = 1;
    g.cps = nch;
    g.part = ws.part;
    g.range_flag = ws.range_flag;
    ConvOut c1 = plain_out(nullptr, L, R.c1.b);
    c1.alpha = R.a2_alpha;
    c1.beta = R.a2_beta;
    ConvFuse fz{};
    fz.A2 = R.c2.w;
    fz.o2 = plain_out(out_sn, L, R.c2.b);
    fz.o2.x = x;
    fz.o2.res = x;
    fz.o2.alpha = next_alpha;
    fz.o2.beta = next_beta;
    hipLaunchKernelGGL((k_conv_gemm<6, CE_SNAKE, true, true, true>), dim3(tn), dim3(256), 0, s, R.c1.w, ch, Kd,
                       causal_in(sn, ch, L, R.c1.k, R.c1.dil), c1, L, g, fz);
    *done = true;
    return hipGetLastError();
}

static ConvOut plain_out(float *y, int ld, const float *bias)
{
    ConvOut o{};
    o.y = y;
    o.ldy = ld;
    o.os = 1;
    o.bias = bias;
    return o;
}

// Transposed conv with kernel 2*stride or stride (padding 0), cropped to
// L_in * stride positions (decoder.rs:472-486, 512-525), as `stride` phase
// GEMMs.  Phase r's weights (repacked at upload) are [OC][IC*taps]: taps =
// 2 reads x[i-1] (kernel tap r + stride) then x[i] (tap r); taps = 1 reads
// x[i] (tap r).
template <int EPI>
static hipError_t conv_t_phases(const DecConvT &w, const float *x, int L_in, ConvOut o, const DecoderWs &ws,
                                hipStream_t s)
{
    const int taps = w.taps;
    ConvIn in{x, L_in, L_in, w.ic, taps, 1, taps - 1};
    o.os = w.stride;
    o.oo = 0;
    return conv_gemm<EPI>(w.phases, w.oc, in, o, L_in, ws, s, w.stride);
}

// Column RMSNorm of x [H][T]: the register-resident kernel where H fits it
static void col_rms(const float *x, const float *gamma, int H, int T, float *out, hipStream_t s)
{
    if (H <= 256 * COLRMS_NV)
        hipLaunchKernelGGL(k_col_rms_r, dim3((T + 3) / 4), dim3(1024), 0, s, x, gamma, H, T, 1e-5f, out);
    else
        hipLaunchKernelGGL(k_col_rms, dim3((T + 15) / 16), dim3(16 * COLRMS_CG), 0, s, x, gamma, H, T, 1e-5f, out);
}

hipError_t enqueue_decode(const DecoderDev &d, const DecoderWs &ws, const uint32_t *codes, int T, int64_t cut,
                          float *audio, hipStream_t s)
{
    if (T < 1 || T > ws.cap_frames) return hipErrorInvalidValue;
    if (ws.range_flag) DCHK(hipMemsetAsync(ws.range_flag, 0, sizeof(int32_t), s));
    const int D = d.codebook_dim, V = d.vq_dim, H = d.hidden, A = d.n_heads * d.head_dim, I = d.inter;
    const int LAT = d.latent;
    // 1. VQ -> [V][T]
    if (d.n_rest == 15)
        hipLaunchKernelGGL(k_vq_gather<15>, dim3((T + 63) / 64, D), dim3(64), 0, s, d.first_codebook, d.rest_codebooks,
                           d.n_rest, D, codes, T, d.codebook_size, ws.a);
    else
        hipLaunchKernelGGL(k_vq_gather<0>, dim3((T + 63) / 64, D), dim3(64), 0, s, d.first_codebook, d.rest_codebooks,
                           d.n_rest, D, codes, T, d.codebook_size, ws.a);
    DCHK(hipGetLastError());
    DCHK(conv_gemm<CE_STORE>(d.vq_proj, V, causal_in(ws.a, 2 * D, T, 1, 1), plain_out(ws.b, T, nullptr), T, ws, s));
    // 2. pre-conv -> [LAT][T]
    DCHK(conv_gemm<CE_STORE>(d.pre_conv.w, d.pre_conv.oc, causal_in(ws.b, V, T, d.pre_conv.k, d.pre_conv.dil),
                             plain_out(ws.a, T, d.pre_conv.b), T, ws, s));
    // 3. transformer on [H][T]: x in ws.b, normed in ws.c, q|k|v in ws.d, attention in ws.e
    DCHK(conv_gemm<CE_STORE>(d.tf_in_w, H, causal_in(ws.a, LAT, T, 1, 1), plain_out(ws.b, T, d.tf_in_b), T, ws, s));
    const size_t att_lds = attn_tile_lds(d.head_dim, d.window);
    const bool att_tile = d.window + ATT_QB - 1 <= 16 * ATT_SLOTS && att_lds <= 65536;
    for (int l = 0; l < d.n_tf; l++) {
        const DecLayer &L = d.tf[l];
        col_rms(ws.b, L.in_norm, H, T, ws.c, s);
        DCHK(hipGetLastError());
        DCHK(conv_gemm<CE_STORE>(L.qkv, 3 * A, causal_in(ws.c, H, T, 1, 1), plain_out(ws.d, T, nullptr), T, ws, s));
        if (!att_tile) {   // the tiled kernel applies RoPE while staging
            hipLaunchKernelGGL(k_rope_cf, dim3((T + 63) / 64, 2 * d.n_heads), dim3(64), 0, s, ws.d, d.n_heads,
                               d.head_dim, T, d.rope_cos, d.rope_sin, d.rope_rows);
            DCHK(hipGetLastError());
        }
        const dim3 ag((T + ATT_QB - 1) / ATT_QB, d.n_heads);
        if (att_tile && d.head_dim == 64)
            hipLaunchKernelGGL(k_dec_attn_tile<64>, ag, dim3(256), att_lds, s, ws.d, d.n_heads, T, d.window,
                               d.rope_cos, d.rope_sin, d.rope_rows, ws.e);
        else if (att_tile)
            hipLaunchKernelGGL(k_dec_attn_tile<16>, ag, dim3(256), att_lds, s, ws.d, d.n_heads, T, d.window,
                               d.rope_cos, d.rope_sin, d.rope_rows, ws.e);
        else if (d.head_dim == 64)
            hipLaunchKernelGGL(k_dec_attn<64>, dim3((T + 63) / 64, d.n_heads), dim3(64), 0, s, ws.d, d.n_heads, T,
                               d.window, ws.e);
        else
            hipLaunchKernelGGL(k_dec_attn<16>, dim3((T + 63) / 64, d.n_heads), dim3(64), 0, s, ws.d, d.n_heads, T,
                               d.window, ws.e);
        DCHK(hipGetLastError());
        ConvOut ro = plain_out(ws.b, T, nullptr);
        ro.scale = L.attn_scale;
        DCHK(conv_gemm<CE_SCALE_RES>(L.o, H, causal_in(ws.e, A, T, 1, 1), ro, T, ws, s));
        col_rms(ws.b, L.post_norm, H, T, ws.c, s);
        DCHK(hipGetLastError());
        DCHK(conv_gemm<CE_SWIGLU>(L.gate_up, 2 * I, causal_in(ws.c, H, T, 1, 1), plain_out(ws.d, T, nullptr), T, ws, s));
        ConvOut mo = plain_out(ws.b, T, nullptr);
        mo.scale = L.mlp_scale;
        DCHK(conv_gemm<CE_SCALE_RES>(L.down, H, causal_in(ws.d, I, T, 1, 1), mo, T, ws, s));
    }
    col_rms(ws.b, d.tf_norm, H, T, ws.c, s);
    DCHK(hipGetLastError());
    DCHK(conv_gemm<CE_STORE>(d.tf_out_w, LAT, causal_in(ws.c, H, T, 1, 1), plain_out(ws.a, T, d.tf_out_b), T, ws, s));
    // 4. upsample stages: ConvT (phases) then ConvNeXt; the signal moves
    // between ws.a and ws.b
    int L = T;
    float *sig = ws.a, *other = ws.b;
    for (int u = 0; u < d.n_up; u++) {
        const DecUpsample &U = d.up[u];
        const int Lo = L * U.conv_t.stride;
        DCHK(conv_t_phases<CE_STORE>(U.conv_t, sig, L, plain_out(other, Lo, U.conv_t.b), ws, s));
        L = Lo;
        if (U.dw_k == DWLN_K && U.ch <= DWLN_CMAX)
            hipLaunchKernelGGL(k_dw_ln_r, dim3((L + DWLN_TP - 1) / DWLN_TP), dim3(1024), 0, s, other, U.ch, L, U.dw_w,
                               U.dw_b, U.norm_w, U.norm_b, 1e-5f, ws.c);
        else
            hipLaunchKernelGGL(k_dw_ln, dim3((L + 15) / 16), dim3(16 * DWLN_CG), 0, s, other, U.ch, L, U.dw_w, U.dw_b,
                               U.dw_k, U.norm_w, U.norm_b, 1e-5f, ws.c);
        DCHK(hipGetLastError());
        DCHK(conv_gemm<CE_GELU>(U.pw1, U.inner, causal_in(ws.c, U.ch, L, 1, 1), plain_out(ws.d, L, U.pw1_b), L, ws, s));
        ConvOut po = plain_out(other, L, U.pw2_b);
        po.scale = U.gamma;
        DCHK(conv_gemm<CE_SCALE_RES>(U.pw2, U.ch, causal_in(ws.d, U.inner, L, 1, 1), po, L, ws, s));
        std::swap(sig, other);
    }
    // 5. Vocos: init conv with the first block's pre-snake (or the final
    // snake) fused
    const float *na = d.n_voc ? d.voc[0].pre_alpha : d.final_alpha;
    const float *nb = d.n_voc ? d.voc[0].pre_beta : d.final_beta;
    {
        ConvOut so = plain_out(ws.c, L, d.voc_init.b);
        so.alpha = na;
        so.beta = nb;
        DCHK(conv_gemm<CE_SNAKE>(d.voc_init.w, d.voc_init.oc,
                                 causal_in(sig, d.voc_init.ic, L, d.voc_init.k, d.voc_init.dil), so, L, ws, s));
    }
    int ch = d.voc_init.oc;
    float *sn = ws.c, *x = sig, *t1 = other;   // snake(x) / x / scratch
    for (int b = 0; b < d.n_voc; b++) {
        const DecVocos &B = d.voc[b];
        const int Lo = L * B.up.stride;
        ch = B.up.oc;
        // ConvT phases: x = convT(snake); sn = snake of the first residual's act1
        const bool has_res = B.n_res > 0;
        ConvOut xo = plain_out(x, Lo, B.up.b);
        xo.x = x;
        xo.y = t1;
        xo.alpha = has_res ? B.res[0].a1_alpha : (b + 1 < d.n_voc ? d.voc[b + 1].pre_alpha : d.final_alpha);
        xo.beta = has_res ? B.res[0].a1_beta : (b + 1 < d.n_voc ? d.voc[b + 1].pre_beta : d.final_beta);
        DCHK(conv_t_phases<CE_STORE_SNAKE>(B.up, sn, L, xo, ws, s));
        L = Lo;
        std::swap(sn, t1);   // sn = snake(x)
        for (int r = 0; r < B.n_res; r++) {
            const DecVocosRes &R = B.res[r];
            const float *nal = r + 1 < B.n_res ? B.res[r + 1].a1_alpha
                                               : (b + 1 < d.n_voc ? d.voc[b + 1].pre_alpha : d.final_alpha);
            const float *nbe = r + 1 < B.n_res ? B.res[r + 1].a1_beta
                                               : (b + 1 < d.n_voc ? d.voc[b + 1].pre_beta : d.final_beta);
            bool fused;
            DCHK(vocos_res_fused(R, ch, sn, t1, x, L, nal, nbe, ws, s, &fused));
            if (fused) {
                std::swap(sn, t1);   // sn = the next snake of x
                continue;
            }
            // conv1 (k 7, dilation) with act2 fused: t1 = snake2(conv1(sn))
            ConvOut c1 = plain_out(t1, L, R.c1.b);
            c1.alpha = R.a2_alpha;
            c1.beta = R.a2_beta;
            DCHK(conv_gemm<CE_SNAKE>(R.c1.w, ch, causal_in(sn, ch, L, R.c1.k, R.c1.dil), c1, L, ws, s));
            // conv2 (k 1) + residual: x += conv2(t1); sn = next snake(x)
            ConvOut c2 = plain_out(sn, L, R.c2.b);
            c2.x = x;
            c2.res = x;
            c2.alpha = nal;
            c2.beta = nbe;
            DCHK(conv_gemm<CE_STORE_SNAKE>(R.c2.w, ch, causal_in(t1, ch, L, R.c2.k, R.c2.dil), c2, L, ws, s));
        }
    }
    // 6. output conv on snake(x) + clamp, first `cut` samples dropped
    hipLaunchKernelGGL(k_out_conv, dim3((L + 255) / 256), dim3(256), 0, s, sn, ch, L, d.out_w, d.out_b, d.out_k,
                       d.out_dil, cut, audio);
    return hipGetLastError();
}

// Algorithmic floating-point operations of enqueue_decode over T frames:
// 2 per multiply-add of every projection and convolution at its true
// kernel size (transposed convs: 2 * ic * oc * kernel per input position),
// plus q.k and p.v of the windowed attention.
double decode_flops(const DecoderDev &d, int T)
{
    const double t = T;
    const double D = d.codebook_dim, V = d.vq_dim, H = d.hidden, A = (double)d.n_heads * d.head_dim, I = d.inter;
    const double LAT = d.latent;
    double f = 2.0 * V * 2 * D * t + 2.0 * LAT * V * d.pre_conv.k * t + 2.0 * H * LAT * t + 2.0 * LAT * H * t;
    double keys = 0.0;
    for (int i = 0; i < T; i++) keys += std::min(i + 1, d.window);
    f += d.n_tf * (2.0 * t * (3 * A * H + H * A + 2 * I * H + H * I) + 4.0 * A * keys);
    double L = t;
    for (int u = 0; u < d.n_up; u++) {
        const DecUpsample &U = d.up[u];
        f += 2.0 * U.ch * U.ch * U.conv_t.taps * U.conv_t.stride * L;
        L *= U.conv_t.stride;
        f += 2.0 * L * (2.0 * U.inner * U.ch + U.dw_k * U.ch);
    }
    f += 2.0 * d.voc_init.oc * d.voc_init.ic * d.voc_init.k * L;
    for (int b = 0; b < d.n_voc; b++) {
        const DecVocos &B = d.voc[b];
        f += 2.0 * B.up.oc * B.up.ic * B.up.taps * B.up.stride * L;
        L *= B.up.stride;
        for (int r = 0; r < B.n_res; r++)
            f += 2.0 * L * ((double)B.res[r].c1.oc * B.res[r].c1.ic * B.res[r].c1.k +
                            (double)B.res[r].c2.oc * B.res[r].c2.ic * B.res[r].c2.k);
    }
    const int ch = d.n_voc ? d.voc[d.n_voc - 1].up.oc : d.voc_init.oc;
    f += 2.0 * ch * d.out_k * L;
    return f;
}

}  // namespace qtts
