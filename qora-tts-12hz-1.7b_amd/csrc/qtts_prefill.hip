// qtts_prefill.hip — batched talker prefill for long prompts on the matrix
// cores (prefill_talker_raw_from, talker.rs:379-482).
//
// A prompt of M rows runs layer by layer (k_row_inv first: 1/rms of every
// input row, gemv.rs:445-454): per layer
//   k_gemm_q4 (parts)    [M x 2048] x [2048 x 4096] q|k|v,   talker.rs:392-400
//                        input norm fused, 3 k-slices
//   k_prefill_qkv_post   slices summed, QK-norm, RoPE,       talker.rs:402-425
//                        K/V append
//   k_prefill_attn_mx    causal attention over the cache     talker.rs:427-458
//   k_gemm_q4 (parts)    attn x o_proj, 6 k-slices           talker.rs:460
//   k_resid_add_inv      x += slices; post-attention 1/rms   talker.rs:461-468
//   k_gemm_q4 (swiglu)   silu(gate) * up, gate|up fused,     talker.rs:470-474
//                        post-attention norm fused
//   k_gemm_q4 (parts)    h x down_proj, 6 k-slices           talker.rs:475
//   k_resid_add_inv      x += slices; next layer's 1/rms     talker.rs:476
// then k_final_rms on the last row (talker.rs:477-481).
//
// k_gemm_q4 contracts f32 operands with f32 accumulation, the arithmetic
// the reference's gemm_q4 (gemv.rs:349-412) does on the CPU: by default on
// the f16 matrix cores with every operand split into f16 hi + lo (three
// products, f32-accurate; see X3 below), or on v_mfma_f32_16x16x4_f32
// (QTTS_GEMM_F32=1).  The weight is read from the same tiled Q4 layout the
// decode GEMV streams (no second copy in HBM) and dequantised into LDS once
// per row tile of the prompt.

#include "qtts_device.h"
#include "qtts_kernels.h"
#include "qtts_devutil.h"
#include "qtts_mfma.h"

#include <algorithm>
#include <cmath>

namespace qtts {

// ---------------------------------------------------------------------------
// per-row 1/rms (rms_norm_f16, gemv.rs:445-454): inv = 1 / sqrt(sum x^2 / K
// + 1e-6).  One wave per row.
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(256)
k_row_inv(const float *X, int ld, int M, int K, float *inv)
{
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= M) return;
    const float *x = X + (size_t)m * ld;
    float s = 0.0f;
    for (int k = lane * 4; k < K; k += 256) {
        const f32x4 v = ld4(x + k);
        s = fmaf(v.x, v.x, s);
        s = fmaf(v.y, v.y, s);
        s = fmaf(v.z, v.z, s);
        s = fmaf(v.w, v.w, s);
    }
    s = wave_sum_dpp(s);
    if (lane == 0) inv[m] = 1.0f / sqrtf(s / (float)K + 1e-6f);
}

// ---------------------------------------------------------------------------
// Q4 GEMM on the matrix cores: Y[M][n] (op)= A'[M][K] x W[K][n], with
// A' = A * inv[row] * gamma[k] when a norm is fused (the reference's
// x * inv_rms * gamma order) and W dequantised as (nibble - 8) * scale,
// exact in f32.
//
// Workgroup tile: 16*MB rows x 128 columns (four 32-column groups), K in
// chunks of 32 through double-buffered LDS; a weight with S k-slices runs S
// workgroups per tile, each writing its partial sums (GEMM_PART) for the
// consumer kernel to add in slice order.  All four waves cover every row
// of the tile; wave w owns the 16-column blocks c = (w&1) + 4*(w>>1) and
// c + 2, so for the gate|up weight (groups interleaved gate, up, gate, up)
// a lane holds gate and up of the same output column and the SwiGLU
// epilogue stays in registers.
//
// v_mfma_f32_16x16x4_f32 lane layout: A operand lane l = A[l%16][l/16],
// B operand B[l/16][l%16], result element i = D[4*(l/16)+i][l%16].  The
// contraction index of lane group q = l/16 at sub-step e is k = 4q + e of a
// 16-wide slice, so each lane reads its A row and B column as one 16-byte
// LDS load (As is [row][k], Bs is [column][k]).
// ---------------------------------------------------------------------------

constexpr int GN = MFMA_N, GK = MFMA_K, GLD = MFMA_LD;

enum GemmEpi : int { GEMM_STORE = 0, GEMM_PART = 1, GEMM_SWIGLU = 2, GEMM_BIAS = 3, GEMM_BIAS_SILU = 4 };

struct GemmA {
    const float *A;
    int lda;
    const float *inv;        // per-row 1/rms, or null
    const uint16_t *gamma;   // [K] f16, or null
    int M;
    // The range of the split-f16 staging (X3).  Rows without a norm: rmax
    // [M][rslots] holds the largest |A| of each row over slots of rw columns
    // (slot s: k in [s rw, (s+1) rw)), or is null (rows staged as they are).
    // Rows with a norm: nshift, a power of two that takes the bound of
    // |x * inv * gamma| (sqrt(K) * max|gamma|) into [2^13, 2^14].
    const float *rmax;
    int rslots, rw;
    int nshift;
};

struct GemmOut {
    float *Y;
    int ldy, ncols;
    const float *bias;       // GEMM_BIAS*: [ncols]
    size_t slice_stride;     // GEMM_PART: floats between the slices' blocks
    float *rmax;             // GEMM_SWIGLU: largest |output| per (row, 64-column tile) [rows][rslots], or null
    int rslots;
};

// Address of the 16-byte word and the scale of (row k, group g) in the
// tiled layout built by the runtime (qtts_device.h).
__device__ __forceinline__ void tiled_word(const Q4Tiled &w, TileShape ts, int k, int g, const uint8_t *&word,
                                           const uint16_t *&scale)
{
    const int P = ts.T / ts.GB;
    const int s = k / w.KC, rr = k - s * w.KC, r = rr / P, pt = rr - r * P;
    const int ct = g / ts.GB, gt = g - ct * ts.GB;
    const bool wave_groups = (ts.T / 64) % ts.GB == 0;
    const int t = wave_groups ? ((pt >> 6) * ts.GB + gt) * 64 + (pt & 63) : pt * ts.GB + gt;
    const uint8_t *tile = w.data + (size_t)(s * w.CT + ct) * w.tile_bytes;
    word = tile + ((size_t)r * ts.T + t) * 16;
    scale = (const uint16_t *)(tile + (size_t)ts.R * ts.T * 16) + t * ts.R + r;
}

// X3: the contraction on v_mfma_f32_16x16x32_f16 in three products per
// pair of operands.  Each staged value v is split into hi = f16(v) and
// lo = f16(v - hi): hi + lo carries 22 bits of v's 24, and a dequantised
// weight (a 4-bit integer times an f16 scale, 15 significant bits) is
// exactly hi + lo.  acc += Ahi Bhi + Ahi Blo + Alo Bhi (f32 accumulation,
// the products exact); the dropped Alo Blo is below 2^-22 of each term.
// Per chunk of 32 that is 3 matrix instructions of 8192 multiply-adds
// where the f32 path issues 8 of 1024.  The staged tiles are f16 rows of
// HLD halves (80 bytes: a lane's 16-byte read of 8 halves at 16q bytes).
constexpr int HLD = MFMA_HLD;
// word 3 of a raw buffer descriptor on this GPU family (untyped dword
// access, no swizzle, offsets checked against the record count in bytes)
constexpr int BUF_RSRC_W3 = 0x00020000;
// The B tile's 16-column blocks are BPAD halves apart beyond their rows, so
// the four 8-column groups a wave writes at once (8 rows = 160 dwords apart
// otherwise: the same banks two by two) start on banks 0, 32, 16, 48.
constexpr int BPAD = 32;

// (w & m) | o, kept opaque so the masked word is consumed as two f16 halves
__device__ __forceinline__ uint32_t and_or_opaque(uint32_t w, uint32_t m, uint32_t o)
{
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(w), "v"(m), "s"(o));   // one scalar operand (VOP3)
    return r;
}

// x * g with g the low (HI = 0) or high f16 half of a register: one
// v_fma_mix_f32 with a -0 addend, the product rounded once to f32 as a
// multiply rounds it (sign of a zero product kept)
template <int HI>
__device__ __forceinline__ float mul_f16_half(uint32_t g, float x, float nz)
{
    float r;
    if constexpr (HI)
        asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(g), "v"(x), "v"(nz));
    else
        asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(g), "v"(x), "v"(nz));
    return r;
}

template <int MB, int EPI, bool NORM, bool X3>
__global__ void __launch_bounds__(256, 2)
k_gemm_q4(GemmA a, Q4Tiled w, GemmOut o, int tm, int S)
{
    constexpr int BM = 16 * MB;
    constexpr int NA = (BM * GK / 4 + 255) / 256;   // 16-byte A slots per thread
    constexpr int XSTRIDE = BM * HLD + GN * HLD + (GN / 16) * BPAD;   // halves per (buffer, half) on X3
    constexpr int F32_BYTES = 2 * (BM + GN) * GLD * 4, X3_BYTES = 2 * 2 * XSTRIDE * 2;
    constexpr int TILE_BYTES = X3 ? X3_BYTES : F32_BYTES;
    // one LDS block: the staging tiles first (their bank layout assumes the
    // block's base), then the per-row factors that undo the staging scales
    // (X3) and the SwiGLU epilogue's per-wave row maxima
    __shared__ __attribute__((aligned(16))) unsigned char lds[TILE_BYTES + BM * 4 + 4 * BM * 4];
    float *rsc = (float *)(lds + TILE_BYTES);
    float(*wmx)[BM] = (float(*)[BM])(lds + TILE_BYTES + BM * 4);
    // f32: As[2][BM*GLD], Bs[2][GN*GLD]; X3: per buffer Ah, Al [BM*HLD] and Bh, Bl [GN*HLD]
    float(*As)[BM * GLD] = (float(*)[BM * GLD])lds;
    float(*Bs)[GN * GLD] = (float(*)[GN * GLD])(lds + 2 * BM * GLD * 4);
    const auto xa = [&](int buf, int hl) { return (_Float16 *)lds + (size_t)(buf * 2 + hl) * XSTRIDE; };
    const auto xb = [&](int buf, int hl) { return xa(buf, hl) + (size_t)BM * HLD; };
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    // Workgroups are dealt round-robin to the 8 XCDs: give each XCD a
    // contiguous run of tiles (row blocks fastest) so the row blocks that
    // share a weight tile share that XCD's L2.
    const int nwg = gridDim.x, id = blockIdx.x;
    const int xcd = id & 7, qq = nwg >> 3, rem = nwg & 7;
    const int logical = xcd * qq + min(xcd, rem) + (id >> 3);
    const int mt = logical % tm, rest = logical / tm;
    const int sl = rest % S, nt = rest / S;
    const int m0 = mt * BM;
    const int nch = w.k / GK, c0 = sl * nch / S, c1 = (sl + 1) * nch / S;
    const TileShape ts = tile_shape(w.cfg);
    const int P = ts.T / ts.GB;
    const bool wave_groups = (ts.T / 64) % ts.GB == 0;

    // A staging: slot i = t + 256 j (clamped: spare threads repeat the last
    // slot) covers row i / 8, floats 4 (i % 8)..+4 of the chunk.  Rows past
    // M load row M-1 and stage zeros.  On X3 the rows of each 16-row block
    // are taken in 4 x 4 transposed order, so the 4 rows of one 32-lane
    // half of a write are 4 apart (80 dwords: disjoint bank ranges).
    // aoffg: byte offset of the slot in A, unsigned 32 bits, so each load
    // takes the chunk's wave-uniform base in scalar registers plus this
    // X3 range: row r is staged times 2^sh(r), sh chosen so that the row's
    // largest |value| over this slice's columns lies in [2^14, 2^15) (from
    // rmax) or below the norm's static bound (nshift); the f16 halves then
    // neither overflow nor go subnormal where the value is not tiny against
    // the row.  The sums are scaled back by 2^-(sh + bshift) per row in the
    // epilogue.  Both scalings are exact.  The loads the staging factors need
    // (1/rms, the rows' slots) are issued here and used in `pre`, after the
    // first chunk's loads are issued: waiting for them does not hold those
    // back.
    uint32_t aoffg[NA];
    int aoff[NA], akk[NA], arow[NA];
    float amul[NA], ainv[NA];
    float arv[NA][2];               // two of the row's slots over this slice (rows without a norm, X3)
    const int s0 = a.rmax ? (c0 * GK) / a.rw : 0, s1 = a.rmax ? (c1 * GK - 1) / a.rw : 0;
    // A row's 8 slots of a chunk sit in 8 consecutive lanes (8 | 256, and the
    // clamped slots fill whole groups of 8): lane e8 of the group reads the
    // row's slots s0 + 2 e8 and s0 + 2 e8 + 1 (the launcher checks that a
    // slice spans at most 16), and the group takes their maximum by DPP
    const int e8 = t & 7;
#pragma unroll
    for (int j = 0; j < NA; j++) {
        const int slot = min(t + 256 * j, BM * GK / 4 - 1);
        const int rr = slot >> 3;
        const int r = X3 ? (rr & ~15) | ((rr & 3) << 2) | ((rr >> 2) & 3) : rr, m = m0 + r;
        aoffg[j] = (uint32_t)(min(m, a.M - 1) * a.lda + 4 * (slot & 7)) * 4u;
        aoff[j] = r * GLD + 4 * (slot & 7);
        akk[j] = 4 * (slot & 7);
        arow[j] = (slot & 7) == 0 ? r : -1;      // the thread that records the row's factor
        ainv[j] = NORM ? a.inv[min(m, a.M - 1)] : 1.0f;
        if constexpr (X3 && !NORM) {
            if (a.rmax) {
                const float *rp = a.rmax + (size_t)min(m, a.M - 1) * a.rslots;
#pragma unroll
                for (int u = 0; u < 2; u++) {
                    const int sl = s0 + 2 * e8 + u;
                    const float v = rp[min(sl, s1)];
                    arv[j][u] = sl <= s1 ? v : 0.0f;
                }
            }
        }
    }
    auto pre = [&]() {
#pragma unroll
        for (int j = 0; j < NA; j++) {
            const int m = m0 + (aoff[j] / GLD);
            int sh = 0;
            if constexpr (X3) {
                if (NORM) {
                    sh = a.nshift;
                } else if (a.rmax) {
                    float mx = fmaxf(arv[j][0], arv[j][1]);
                    mx = fmaxf(mx, dpp_mov<0xB1>(mx));    // lane ^ 1
                    mx = fmaxf(mx, dpp_mov<0x4E>(mx));    // lane ^ 2
                    mx = fmaxf(mx, dpp_mov<0x141>(mx));   // the other quad of the 8 (half-row mirror)
                    sh = range_shift(mx);
                }
            }
            const float p2 = __builtin_ldexpf(1.0f, sh);
            amul[j] = m < a.M ? (NORM ? ainv[j] * p2 : p2) : 0.0f;
            if (arow[j] >= 0) rsc[arow[j]] = __builtin_ldexpf(1.0f, -(sh + (X3 ? w.bshift : 0)));
        }
    };
    // B staging: bytes 4*qw..+4 (8 columns) of the tiled rows; groups past
    // G stage zeros.  f32: row kr of groups 4*nt + gi and + 2.  X3: rows kr
    // and kr + 1 of group 4*nt + gi (one wave per group), so the two rows'
    // values of a column leave as one 4-byte LDS write.
    const int kr = X3 ? 2 * (t & 15) : (t & 31);
    const int qw = X3 ? (t >> 4) & 3 : (t >> 5) & 3;
    // gi is the same across a wave: read it as a scalar, so the tile
    // addresses below come from the scalar unit
    const int gi = __builtin_amdgcn_readfirstlane(X3 ? t >> 6 : t >> 7);
    int gt[2], gct[2];
    bool gok[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int g = 4 * nt + gi + (X3 ? 0 : 2 * h);
        gok[h] = g < w.G;
        const int gc = min(g, w.G - 1);
        gct[h] = gc / ts.GB;
        gt[h] = gc - gct[h] * ts.GB;
    }

    // X3: the weights are staged times 2^bshift (their split's low half a
    // normal f16) and the sums scaled back by 2^-bshift (both exact)
    const float bscale = X3 ? __builtin_ldexpf(1.0f, w.bshift) : 1.0f;

    // tile position of (pt, group): one group per wave when wave_groups,
    // else groups interleaved by thread -- one formula for both
    const int tA = wave_groups ? 1 : ts.GB, tB = wave_groups ? 64 : 1;
    // With P >= 32 (every tile but 8 groups x 128 threads) a chunk's 32 rows
    // lie in one tile row r0 and one 64-position block (pt0 is a multiple of
    // 32), so tt = ttu(k0) + (kr [+ h]) * tA + gt * tB: a wave-uniform part
    // per chunk and this constant thread part.
    uint32_t thr_w[2], thr_s[2];   // byte offsets of the word and the scale from the chunk's base
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t tt = (uint32_t)((kr + (X3 ? h : 0)) * tA + gt[h] * tB);
        thr_w[h] = tt * 16u + 4u * (uint32_t)qw;
        thr_s[h] = tt * (uint32_t)ts.R * 2u;
    }
    // A and the tiled weight are read through buffer descriptors: the
    // chunk's wave-uniform offset goes in a scalar register (soffset), the
    // thread's byte offset is a constant vector register, so a chunk's loads
    // need no per-chunk vector address arithmetic
    const __amdgpu_buffer_rsrc_t rsA =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.A, (short)0, (int)((size_t)a.M * a.lda * 4), BUF_RSRC_W3);
    const __amdgpu_buffer_rsrc_t rsW =
        __builtin_amdgcn_make_buffer_rsrc((void *)w.data, (short)0, (int)((size_t)w.S * w.CT * w.tile_bytes), BUF_RSRC_W3);
    struct Fetch {
        f32x4 ra[NA];
        uint32_t rg[NA][2];
        uint32_t rb[2], rs[2];
    };
    auto fetch = [&](Fetch &f, int k0) {
#pragma unroll
        for (int j = 0; j < NA; j++) {
            f.ra[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsA, aoffg[j], k0 * 4, 0));
            if (NORM) {
                const uint2 gv = *(const uint2 *)(a.gamma + k0 + akk[j]);
                f.rg[j][0] = gv.x;
                f.rg[j][1] = gv.y;
            }
        }
        // k = k0 + kr (+ h on X3): slice s, row r, position pt of the tiled
        // layout; k0 is a multiple of 32, so only P = 16 splits a chunk over
        // rows
        const int s = k0 / w.KC, rr0 = k0 - s * w.KC, r0 = rr0 / P, pt0 = rr0 - r0 * P;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            uint32_t word;
            uint16_t sc;
            if (P >= 32) {
                const int ttu = (pt0 >> 6) * 64 * ts.GB + (pt0 & 63) * tA;
                const int tb = (s * w.CT + gct[h]) * w.tile_bytes;
                word = __builtin_amdgcn_raw_buffer_load_b32(rsW, thr_w[h], tb + (r0 * ts.T + ttu) * 16, 0);
                sc = __builtin_amdgcn_raw_buffer_load_b16(rsW, thr_s[h], tb + ts.R * ts.T * 16 + (ttu * ts.R + r0) * 2, 0);
            } else {
                const uint8_t *tile = w.data + (size_t)(s * w.CT + gct[h]) * w.tile_bytes;
                const int ptk = pt0 + kr + (X3 ? h : 0);
                const int r = r0 + (ptk >> 4), pt = ptk & 15;
                const int tt = (pt >> 6) * 64 * ts.GB + (pt & 63) * tA + gt[h] * tB;
                word = *(const uint32_t *)(tile + ((size_t)r * ts.T + tt) * 16 + 4 * qw);
                sc = *((const uint16_t *)(tile + (size_t)ts.R * ts.T * 16) + tt * ts.R + r);
            }
            f.rb[h] = gok[h] ? word : 0x88888888u;
            f.rs[h] = gok[h] ? (uint32_t)sc : 0u;
        }
    };
    auto stage = [&](const Fetch &f, int buf) {
#pragma unroll
        for (int j = 0; j < NA; j++) {
            f32x4 x = f.ra[j] * amul[j];
            if constexpr (X3) {
                if (NORM) {
                    // (x * inv) * gamma, gamma read as f16 from its register
                    const float nz = -0.0f;
                    x.x = mul_f16_half<0>(f.rg[j][0], x.x, nz);
                    x.y = mul_f16_half<1>(f.rg[j][0], x.y, nz);
                    x.z = mul_f16_half<0>(f.rg[j][1], x.z, nz);
                    x.w = mul_f16_half<1>(f.rg[j][1], x.w, nz);
                }
                // row aoff / GLD, halves 4 (slot % 8)..+3
                const int r = aoff[j] / GLD, kk = aoff[j] - r * GLD;
                uint32_t h01, l01, h23, l23;
                split_f16_pair(x.x, x.y, h01, l01);
                split_f16_pair(x.z, x.w, h23, l23);
                *(uint2 *)&xa(buf, 0)[r * HLD + kk] = uint2{h01, h23};
                *(uint2 *)&xa(buf, 1)[r * HLD + kk] = uint2{l01, l23};
            } else {
                if (NORM) {
                    x.x *= h2f(f.rg[j][0] & 0xFFFFu);
                    x.y *= h2f(f.rg[j][0] >> 16);
                    x.z *= h2f(f.rg[j][1] & 0xFFFFu);
                    x.w *= h2f(f.rg[j][1] >> 16);
                }
                *(f32x4 *)&As[buf][aoff[j]] = x;
            }
        }
        // 8 columns 32*g + 8*qw + c, c = 0..7: byte c/2, low nibble even c
        if constexpr (X3) {
            // Rows kr, kr + 1 interleaved by bytes: p01 = [r0.b0, r0.b1,
            // r1.b0, r1.b1], p23 likewise, so (p >> 4c') & 0x000F000F
            // holds column c's nibble of both rows.  Two values per packed
            // f16 operation: | 0x64006400 gives 1024 + nib, adding -1032
            // leaves nib - 8 exactly; hi = f16(n8 * s) is the f16 rounding
            // of the exact product (4 + 11 significant bits), as
            // f16(f32(n8) * s) is, and lo = f16(n8 * s - hi) in one fused
            // operation is the rounding of the exact remainder, as
            // f16(f32 product - hi) is.
            const uint32_t p01 = __builtin_amdgcn_perm(f.rb[1], f.rb[0], 0x05040100u);
            const uint32_t p23 = __builtin_amdgcn_perm(f.rb[1], f.rb[0], 0x07060302u);
            // the rows' scales times 2^bshift: exact (a power-of-two multiple)
            const h16x2 sp = {(_Float16)(h2f(f.rs[0]) * bscale), (_Float16)(h2f(f.rs[1]) * bscale)};
            const h16x2 off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const uint32_t pw = (c < 4 ? p01 : p23) >> (4 * (c & 3));
                const h16x2 n8 = __builtin_bit_cast(h16x2, and_or_opaque(pw, 0x000F000Fu, 0x64006400u)) + off;
                const h16x2 hi = n8 * sp;
                const h16x2 lo = __builtin_elementwise_fma(n8, sp, -hi);
                const int col = 32 * gi + 8 * qw + c;
                *(h16x2 *)&xb(buf, 0)[col * HLD + (col >> 4) * BPAD + kr] = hi;
                *(h16x2 *)&xb(buf, 1)[col * HLD + (col >> 4) * BPAD + kr] = lo;
            }
        } else {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const float sc = h2f(f.rs[h]);
#pragma unroll
                for (int c = 0; c < 8; c++) {
                    const float v = (float)((int)((f.rb[h] >> (4 * c)) & 15u) - 8) * sc;
                    Bs[buf][(32 * gi + 8 * qw + 64 * h + c) * GLD + kr] = v;
                }
            }
        }
    };

    // compute roles: wave w owns 16-column blocks cb0 and cb0 + 2
    const int r16 = lane & 15, q = lane >> 4;
    const int cb0 = (wv & 1) + 4 * (wv >> 1);
    const int cb[2] = {cb0, cb0 + 2};
    f32x4 acc[MB][2];
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    mfma_pipeline<Fetch>(
        c1 - c0, [&](Fetch &f, int c) { fetch(f, (c0 + c) * GK); }, stage, pre, [&](int buf) {
            if constexpr (X3)
                mfma_chunk_x3<MB, BPAD>(acc, xa(buf, 0), xa(buf, 1), xb(buf, 0), xb(buf, 1), cb, lane);
            else
                mfma_chunk<MB>(acc, As[buf], Bs[buf], cb, lane);
        });

    if constexpr (X3) {
        // rsc was written before the pipeline's first barrier
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float u = rsc[16 * i + 4 * q + e];
#pragma unroll
                for (int j = 0; j < 2; j++) acc[i][j][e] *= u;
            }
    }
    // epilogue: element e of acc[i][j] is row 16i + 4q + e of the tile,
    // column 128nt + 16(cb0 + 2j) + r16
    float *Y = o.Y + (EPI == GEMM_PART ? (size_t)sl * o.slice_stride : 0);
    if constexpr (EPI == GEMM_SWIGLU) {
        // groups (4nt, 4nt+1) and (4nt+2, 4nt+3) are (gate, up) pairs
        const int col = 32 * (2 * nt + (wv >> 1)) + 16 * (wv & 1) + r16;
        float vmax[MB][4];
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + 16 * i + 4 * q + e;
                const float v = silu_f(acc[i][0][e]) * acc[i][1][e];
                if (m < a.M && col < o.ncols) Y[(size_t)m * o.ldy + col] = v;
                vmax[i][e] = col < o.ncols ? fabsf(v) : 0.0f;
            }
        // largest |silu(g) u| of each row over this tile's 64 output columns
        // (the range of the down projection's staging): over a wave's 16
        // columns by DPP, then over the four waves through LDS
        if (o.rmax) {
#pragma unroll
            for (int i = 0; i < MB; i++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float v = row_max16(vmax[i][e]);   // the 16 lanes r16 of this q form one DPP row
                    if (r16 == 0) wmx[wv][16 * i + 4 * q + e] = v;
                }
            __syncthreads();
            if (t < BM && m0 + t < a.M)
                o.rmax[(size_t)(m0 + t) * o.rslots + nt] =
                    fmaxf(fmaxf(wmx[0][t], wmx[1][t]), fmaxf(wmx[2][t], wmx[3][t]));
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < MB; i++) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int m = m0 + 16 * i + 4 * q + e;
            if (m >= a.M) continue;
            float *yr = Y + (size_t)m * o.ldy;
            {
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int col = GN * nt + 16 * (cb0 + 2 * j) + r16;
                    if (col >= o.ncols) continue;
                    const float v = acc[i][j][e];
                    if (EPI == GEMM_BIAS) yr[col] = v + o.bias[col];
                    else if (EPI == GEMM_BIAS_SILU) yr[col] = silu_f(v + o.bias[col]);
                    else yr[col] = v;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// q|k|v partial rows (S k-slices, added in slice order) -> QK-norm
// (talker.rs:89-99), RoPE at start + row (rope.rs:79-92), q rows out, K
// (normed, roped) and V (raw) appended to the paged cache at the same
// position (talker.rs:419-425).  One wave per (row, head): heads 0..15 q,
// 16..23 k, 24..31 v; lane holds dims (l, l+64).
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(256)
k_prefill_qkv_post(const float *part, int S, size_t slice_stride, int ldp, int M, int64_t start,
                   const uint16_t *qn_g, const uint16_t *kn_g, const float *rope_cos, const float *rope_sin,
                   KvPaged kv, int layer, float *q, int ldq)
{
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x, hh = blockIdx.y * 4 + (threadIdx.x >> 6);
    if (m >= M) return;
    const int64_t pos = start + m;
    const float *row = part + (size_t)m * ldp + hh * HEAD_DIM;
    float x0 = row[lane], x1 = row[lane + 64];
    for (int s = 1; s < S; s++) {
        x0 += row[s * slice_stride + lane];
        x1 += row[s * slice_stride + lane + 64];
    }
    if (hh >= 24) {
        float *vp = kv_ptr(kv, layer, (int)pos, hh - 24, 1);
        vp[lane] = x0;
        vp[lane + 64] = x1;
        return;
    }
    const uint16_t *gam = hh < 16 ? qn_g : kn_g;
    const float ss = wave_sum_dpp(x0 * x0 + x1 * x1);
    const float inv = 1.0f / sqrtf(ss / 128.0f + 1e-6f);
    const float n0 = x0 * inv * h2f(gam[lane]), n1 = x1 * inv * h2f(gam[lane + 64]);
    const float cs = rope_cos[pos * 64 + lane], sn = rope_sin[pos * 64 + lane];
    const float r0 = n0 * cs - n1 * sn, r1 = n1 * cs + n0 * sn;
    float *out = hh < 16 ? q + (size_t)m * ldq + hh * HEAD_DIM : kv_ptr(kv, layer, (int)pos, hh - 16, 0);
    out[lane] = r0;
    out[lane + 64] = r1;
}

// ---------------------------------------------------------------------------
// Residual add of a projection's k-slice partials (x += sum over slices, in
// slice order: talker.rs:461, 474) fused with the next RMSNorm's 1/rms of
// the updated row (gemv.rs:445-454).  One workgroup per row.
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(256)
k_resid_add_inv(float *x, int ldx, const float *part, int S, size_t slice_stride, int ldp, int H, float *inv)
{
    __shared__ float red[4];
    const int t = threadIdx.x, m = blockIdx.x;
    float *xr = x + (size_t)m * ldx;
    const float *pr = part + (size_t)m * ldp;
    float ss = 0.0f;
    for (int j = 4 * t; j < H; j += 1024) {
        f32x4 p = ld4(pr + j);
        for (int s = 1; s < S; s++) p += ld4(pr + s * slice_stride + j);
        const f32x4 v = ld4(xr + j) + p;
        *(f32x4 *)(xr + j) = v;
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
    }
    ss = wave_sum_dpp(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    if (t == 0) inv[m] = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)H + 1e-6f);
}

// ---------------------------------------------------------------------------
// Causal prefill attention (talker.rs:427-458): query row m (position
// start + m) attends to cached positions 0..start+m.  Workgroup (block of
// QB rows, kv head h) serves q heads 2h and 2h+1 of its rows -- 2*QB
// queries -- with one pass over the K/V pages they need and an online
// softmax across pages (the reference's softmax_raw over the whole row,
// regrouped).  Thread t keeps K row t/4 of the page (dims 32*(t%4)..+32)
// and V dims 4*(t%32)..+4 of page rows 8*(t/32)..+8 in registers, reused
// by every query of the block; the next page's K/V loads are issued before
// the current page's probabilities are formed.
// ---------------------------------------------------------------------------

template <int QB>
__global__ void __launch_bounds__(256)
k_prefill_attn(const float *q, int ldq, int M, int64_t start, KvPaged kv, int layer, float *out, int ldo)
{
    constexpr int NQ = 2 * QB;                    // query j: row j/2, head 2h + j%2
    __shared__ __attribute__((aligned(16))) float qs[NQ][HEAD_DIM];
    __shared__ float pr[NQ][KV_PAGE];
    __shared__ float wmax[4][NQ], wsum[4][NQ];
    __shared__ __attribute__((aligned(16))) float ored[4][NQ][HEAD_DIM];
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int m0 = blockIdx.x * QB, h = blockIdx.y;
    const int nq = min(QB, M - m0);
    const int Lmax = (int)(start + m0 + nq);      // positions the block's last row attends
    const int C = (Lmax + KV_PAGE - 1) / KV_PAGE;
    const float scale = 1.0f / sqrtf(128.0f);
    const int tk = t >> 2, kq = t & 3;
    const int vd = (t & 31) * 4, vt0 = (t >> 5) * 8;
    for (int i = t; i < NQ * HEAD_DIM; i += 256) {
        const int j = i / HEAD_DIM, d = i - j * HEAD_DIM, r = j >> 1;
        qs[j][d] = r < nq ? q[(size_t)(m0 + r) * ldq + (2 * h + (j & 1)) * HEAD_DIM + d] : 0.0f;
    }
    float mrun[NQ], lrun[NQ];
    f32x4 acc[NQ];
#pragma unroll
    for (int j = 0; j < NQ; j++) {
        mrun[j] = -INFINITY;
        lrun[j] = 0.0f;
        acc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    f32x4 kk[8], vv[8];
    {
        const float *Kp = kv_ptr(kv, layer, 0, h, 0), *Vp = kv_ptr(kv, layer, 0, h, 1);
#pragma unroll
        for (int i = 0; i < 8; i++) kk[i] = ld4(Kp + tk * HEAD_DIM + kq * 32 + 4 * i);
#pragma unroll
        for (int i = 0; i < 8; i++) vv[i] = ld4(Vp + (vt0 + i) * HEAD_DIM + vd);
    }
    __syncthreads();
    for (int c = 0; c < C; c++) {
        const int pos = c * KV_PAGE + tk;
        // scores of K row tk against every query of the block
        float sc[NQ];
#pragma unroll
        for (int j = 0; j < NQ; j++) {
            float d = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const f32x4 qa = *(const f32x4 *)&qs[j][kq * 32 + 4 * i];
                const f32x4 k = kk[i];
                d = fmaf(qa.x, k.x, fmaf(qa.y, k.y, fmaf(qa.z, k.z, fmaf(qa.w, k.w, d))));
            }
            d += dpp_mov<0xB1>(d);
            d += dpp_mov<0x4E>(d);
            const bool valid = (j >> 1) < nq && pos <= (int)start + m0 + (j >> 1);
            sc[j] = valid ? d * scale : -INFINITY;
        }
        // this page's V rows stay in registers; the next page's K is free to load
        f32x4 vcur[8];
#pragma unroll
        for (int i = 0; i < 8; i++) vcur[i] = vv[i];
        if (c + 1 < C) {
            const float *Kp = kv_ptr(kv, layer, (c + 1) * KV_PAGE, h, 0), *Vp = kv_ptr(kv, layer, (c + 1) * KV_PAGE, h, 1);
#pragma unroll
            for (int i = 0; i < 8; i++) kk[i] = ld4(Kp + tk * HEAD_DIM + kq * 32 + 4 * i);
#pragma unroll
            for (int i = 0; i < 8; i++) vv[i] = ld4(Vp + (vt0 + i) * HEAD_DIM + vd);
        }
#pragma unroll
        for (int j = 0; j < NQ; j++) {
            const float mw = wave_max_dpp(sc[j]);
            if (lane == 0) wmax[wv][j] = mw;
        }
        __syncthreads();
        float f[NQ];
#pragma unroll
        for (int j = 0; j < NQ; j++) {
            const float pm = fmaxf(fmaxf(wmax[0][j], wmax[1][j]), fmaxf(wmax[2][j], wmax[3][j]));
            const float mn = fmaxf(mrun[j], pm);
            f[j] = mn == -INFINITY ? 0.0f : expf(mrun[j] - mn);   // 0 before the row's first position
            const float e = sc[j] == -INFINITY ? 0.0f : expf(sc[j] - mn);
            if (kq == 0) pr[j][tk] = e;
            const float lw = wave_sum_dpp(kq == 0 ? e : 0.0f);
            if (lane == 0) wsum[wv][j] = lw;
            mrun[j] = mn;
        }
        __syncthreads();
        // P.V over this thread's 8 rows and 4 dims (rows past the written
        // cache may hold anything and are skipped)
#pragma unroll
        for (int j = 0; j < NQ; j++) {
            f32x4 a = acc[j] * f[j];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const bool ok = c * KV_PAGE + vt0 + i < Lmax;
                const float p = pr[j][vt0 + i];
                const f32x4 v = vcur[i];
                a.x = ok ? fmaf(p, v.x, a.x) : a.x; a.y = ok ? fmaf(p, v.y, a.y) : a.y;
                a.z = ok ? fmaf(p, v.z, a.z) : a.z; a.w = ok ? fmaf(p, v.w, a.w) : a.w;
            }
            acc[j] = a;
            lrun[j] = lrun[j] * f[j] + ((wsum[0][j] + wsum[1][j]) + (wsum[2][j] + wsum[3][j]));
        }
        __syncthreads();                             // wmax, wsum and pr are reused by the next page
    }
    // rows 8*(t/32): lanes l and l^32 of a wave hold the same dims
#pragma unroll
    for (int j = 0; j < NQ; j++) {
        f32x4 a = acc[j];
        a.x += __shfl_xor(a.x, 32); a.y += __shfl_xor(a.y, 32);
        a.z += __shfl_xor(a.z, 32); a.w += __shfl_xor(a.w, 32);
        if (lane < 32) *(f32x4 *)&ored[wv][j][vd] = a;
    }
    __syncthreads();
    for (int i = t; i < NQ * HEAD_DIM; i += 256) {
        const int j = i / HEAD_DIM, d = i - j * HEAD_DIM, r = j >> 1;
        if (r < nq) {
            const float o = (ored[0][j][d] + ored[1][j][d]) + (ored[2][j][d] + ored[3][j][d]);
            float l = 0.0f;
#pragma unroll
            for (int jj = 0; jj < NQ; jj++) l = jj == j ? lrun[jj] : l;
            out[(size_t)(m0 + r) * ldo + (2 * h + (j & 1)) * HEAD_DIM + d] = o / l;
        }
    }
}

// rows per workgroup: at 400 rows x 28 layers, 1 / 2 / 4 / 8 rows measured
// 75 / 62 / 76 / 140 us per layer (the per-page chain and the occupancy bind)
constexpr int PREFILL_ATTN_QB = 2;

// ---------------------------------------------------------------------------
// The same causal attention on the matrix cores.  Workgroup (block of 8
// rows, kv head h): 16 queries, query i = (row i/2, head 2h + i%2).  Wave w
// takes positions 16w..16w+15 of every 64-position page and keeps its own
// online softmax (max, sum, output) per query; the four waves are merged
// once at the end, in wave order.  Per page and wave:
//   S^T = K Q^T on v_mfma_f32_16x16x32_f16: A = the wave's 16 K rows, B = the
//        16 queries; lane l then holds query l%16 at positions 4(l/16)..+3,
//   which is the B operand of
//   O^T += V^T P^T on v_mfma_f32_16x16x16_f16 (A = V^T: dims 16t + l%16 at
//        the same 4 positions), so the probabilities never leave the lane
//        and the softmax statistics of a query stay in its lanes.
// Every product is split f16 (hi*hi + hi*lo + lo*hi, f32 accumulation), as
// in the GEMM.  Cache rows at or past the block's length may hold anything:
// their scores are replaced by -inf and their V values by 0 (selects).  A
// query's result depends only on its own row and position, not on the
// block it shares, so a prompt prefilled in pieces matches one prefilled
// whole bit for bit.
// ---------------------------------------------------------------------------

// (results straight into matrix instructions: the register form of the split)
__device__ __forceinline__ void split8(const f32x4 &a, const f32x4 &b, half8 &hi, half8 &lo)
{
    uint32_t h[4], l[4];
    split_f16_pair<true>(a.x, a.y, h[0], l[0]);
    split_f16_pair<true>(a.z, a.w, h[1], l[1]);
    split_f16_pair<true>(b.x, b.y, h[2], l[2]);
    split_f16_pair<true>(b.z, b.w, h[3], l[3]);
    hi = __builtin_bit_cast(half8, uint4{h[0], h[1], h[2], h[3]});
    lo = __builtin_bit_cast(half8, uint4{l[0], l[1], l[2], l[3]});
}

__device__ __forceinline__ void split4(float a, float b, float c, float d, half4 &hi, half4 &lo)
{
    uint32_t h[2], l[2];
    split_f16_pair<true>(a, b, h[0], l[0]);
    split_f16_pair<true>(c, d, h[1], l[1]);
    hi = __builtin_bit_cast(half4, uint2{h[0], h[1]});
    lo = __builtin_bit_cast(half4, uint2{l[0], l[1]});
}

// Split range: with SC, q, K and V are staged times 2^sq, 2^sk, 2^sv, static
// powers of two from the layer's bounds (the QK-norm gammas, the input norm
// and v_proj) for a layer whose bounds leave [2^-4, 2^14], so their f16
// halves neither overflow nor go subnormal; the scores are scaled back by
// 2^-(sq + sk), the output by 2^-sv (exact).  Layers within that band run
// without the scalings (SC false).
template <bool SC>
__global__ void __launch_bounds__(256)
k_prefill_attn_mx(const float *q, int ldq, int M, int64_t start, KvPaged kv, int layer, float *out, int ldo,
                  float *rmax, int rslots, int sq, int sk, int sv)
{
    constexpr int QR = 8;
    __shared__ float smax[4][16], ssum[4][16];
    __shared__ __attribute__((aligned(16))) float so[4][16][HEAD_DIM + 4];
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6, r16 = lane & 15, qd = lane >> 4;
    const int m0 = blockIdx.x * QR, h = blockIdx.y;
    const int nq = min(QR, M - m0);
    const int Lmax = (int)(start + m0 + nq);     // positions 0..Lmax-1 hold the block's keys
    const int C = (Lmax + KV_PAGE - 1) / KV_PAGE;
    const float scale = 1.0f / sqrtf(128.0f);
    // this lane's query: row r16/2 of the block, head 2h + r16%2
    const int qrow = r16 >> 1;
    const int qpos = (int)start + m0 + qrow;

    // Q as the B operand of S^T: dims 32c + 8qd..+7 of the lane's query
    half8 qh[4], ql[4];
    {
        const bool ok = qrow < nq;
        const float *qp = q + (size_t)(m0 + min(qrow, nq - 1)) * ldq + (2 * h + (r16 & 1)) * HEAD_DIM + 8 * qd;
        const float pq = __builtin_ldexpf(1.0f, sq);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            f32x4 a = ld4(qp + 32 * c), b = ld4(qp + 32 * c + 4);
            if constexpr (SC) {
                a *= pq;
                b *= pq;
            }
            const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
            split8(ok ? a : z, ok ? b : z, qh[c], ql[c]);
        }
    }
    const float pk = __builtin_ldexpf(1.0f, sk), pv = __builtin_ldexpf(1.0f, sv);
    const float uqk = __builtin_ldexpf(1.0f, -(sq + sk)), uv = __builtin_ldexpf(1.0f, -sv);
    // K rows p0 + r16 (dims 32c + 8qd..+7) and V rows p0 + 4qd + kk (dims
    // 16t + r16) of page c, p0 = 64c + 16w
    auto load_kv = [&](int c, f32x4 (&kr)[8], float (&vr)[32]) {
        const float *Kp = kv_ptr(kv, layer, c * KV_PAGE, h, 0) + (16 * wv + r16) * HEAD_DIM + 8 * qd;
        const float *Vp = kv_ptr(kv, layer, c * KV_PAGE, h, 1) + (16 * wv + 4 * qd) * HEAD_DIM + r16;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            kr[2 * i] = ld4(Kp + 32 * i);
            kr[2 * i + 1] = ld4(Kp + 32 * i + 4);
        }
#pragma unroll
        for (int tt = 0; tt < 8; tt++)
#pragma unroll
            for (int kk = 0; kk < 4; kk++) vr[tt * 4 + kk] = Vp[kk * HEAD_DIM + 16 * tt];
    };
    float mrun = -INFINITY, lrun = 0.0f;
    f32x4 o[8];
#pragma unroll
    for (int tt = 0; tt < 8; tt++) o[tt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 kn[8];
    float vn[32];
    load_kv(0, kn, vn);
    for (int c = 0; c < C; c++) {
        f32x4 kr[8];
        float vr[32];
#pragma unroll
        for (int i = 0; i < 8; i++) kr[i] = kn[i];
#pragma unroll
        for (int i = 0; i < 32; i++) vr[i] = vn[i];
        if (c + 1 < C) load_kv(c + 1, kn, vn);
        const int p0 = c * KV_PAGE + 16 * wv;
        // scores S^T[position p0 + 4qd + e][query r16]
        f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            half8 kh, kl;
            if constexpr (SC)
                split8(kr[2 * i] * pk, kr[2 * i + 1] * pk, kh, kl);
            else
                split8(kr[2 * i], kr[2 * i + 1], kh, kl);
            s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kl, qh[i], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[i], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[i], s, 0, 0, 0);
        }
        // causal mask, the wave's online softmax for query r16 (its four
        // lanes r16 + 16j combine by lane swaps, in a fixed order)
        float sc[4];
#pragma unroll
        for (int e = 0; e < 4; e++) sc[e] = p0 + 4 * qd + e <= qpos ? (SC ? s[e] * uqk : s[e]) * scale : -INFINITY;
        float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(mrun, mx);
        const float alpha = mn == -INFINITY ? 1.0f : expf(mrun - mn);
        float p[4];
#pragma unroll
        for (int e = 0; e < 4; e++) p[e] = sc[e] == -INFINITY ? 0.0f : expf(sc[e] - mn);
        float ps = (p[0] + p[1]) + (p[2] + p[3]);
        ps += __shfl_xor(ps, 16);
        ps += __shfl_xor(ps, 32);
        lrun = lrun * alpha + ps;
        mrun = mn;
        half4 ph, pl;
        split4(p[0], p[1], p[2], p[3], ph, pl);
        // O^T[dim 16t + 4qd + e][query r16] += V^T P^T
#pragma unroll
        for (int tt = 0; tt < 8; tt++) {
            float v[4];
#pragma unroll
            for (int kk = 0; kk < 4; kk++) v[kk] = p0 + 4 * qd + kk < Lmax ? (SC ? vr[tt * 4 + kk] * pv : vr[tt * 4 + kk]) : 0.0f;
            half4 vh, vl;
            split4(v[0], v[1], v[2], v[3], vh, vl);
            f32x4 a = o[tt] * alpha;
            a = __builtin_amdgcn_mfma_f32_16x16x16f16(vl, ph, a, 0, 0, 0);
            a = __builtin_amdgcn_mfma_f32_16x16x16f16(vh, pl, a, 0, 0, 0);
            o[tt] = __builtin_amdgcn_mfma_f32_16x16x16f16(vh, ph, a, 0, 0, 0);
        }
    }
    // merge the waves: weights exp(m_w - max_w m_w), in wave order
    if (qd == 0) {
        smax[wv][r16] = mrun;
        ssum[wv][r16] = lrun;
    }
#pragma unroll
    for (int tt = 0; tt < 8; tt++) *(f32x4 *)&so[wv][r16][16 * tt + 4 * qd] = o[tt];
    __syncthreads();
    const int qi = t >> 4, d0 = 8 * (t & 15), row = qi >> 1;
    if (row < nq) {
        const float mm = fmaxf(fmaxf(smax[0][qi], smax[1][qi]), fmaxf(smax[2][qi], smax[3][qi]));
        float wgt[4], l = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            wgt[w] = smax[w][qi] == -INFINITY ? 0.0f : expf(smax[w][qi] - mm);
            l = fmaf(wgt[w], ssum[w][qi], l);
        }
        const float inv = 1.0f / l;
        float *op = out + (size_t)(m0 + row) * ldo + (2 * h + (qi & 1)) * HEAD_DIM + d0;
        float mx = 0.0f;
        // (the sums of P V times 2^sv, merged, divided by l, scaled back)
#pragma unroll
        for (int j = 0; j < 8; j += 4) {
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int w = 0; w < 4; w++) acc += wgt[w] * *(const f32x4 *)&so[w][qi][d0 + j];
            acc = SC ? (acc * inv) * uv : acc * inv;
            *(f32x4 *)(op + j) = acc;
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(acc.x), fabsf(acc.y)), fmaxf(fabsf(acc.z), fabsf(acc.w))));
        }
        // the largest |output| of the row over its two heads (the range of
        // the o-projection's staging): the row's 32 lanes are one half-wave
        mx = fmaxf(mx, __shfl_xor(mx, 1));
        mx = fmaxf(mx, __shfl_xor(mx, 2));
        mx = fmaxf(mx, __shfl_xor(mx, 4));
        mx = fmaxf(mx, __shfl_xor(mx, 8));
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        if (rmax && (t & 31) == 0) rmax[(size_t)(m0 + row) * rslots + h] = mx;
    }
}

// ---------------------------------------------------------------------------
// Largest |x| of each row over slots of rw columns: out[m][s] = max over k in
// [s rw, min((s+1) rw, K)) of |X[m][k]|.  One wave per (row, slot).  The
// range of the split-f16 staging for GEMM rows no kernel of the chain
// measured on the way out.
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(256)
k_row_absmax(const float *X, int ld, int M, int K, int rw, int rslots, float *out)
{
    const int lane = threadIdx.x & 63;
    const int id = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (id >= M * rslots) return;
    const int m = id / rslots, sl = id - m * rslots;
    const float *x = X + (size_t)m * ld;
    const int k1 = min((sl + 1) * rw, K);
    float mx = 0.0f;
    for (int k = sl * rw + lane; k < k1; k += 64) mx = fmaxf(mx, fabsf(x[k]));
    mx = fmaxf(mx, __shfl_xor(mx, 1));
    mx = fmaxf(mx, __shfl_xor(mx, 2));
    mx = fmaxf(mx, __shfl_xor(mx, 4));
    mx = fmaxf(mx, __shfl_xor(mx, 8));
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    if (lane == 0) out[(size_t)m * rslots + sl] = mx;
}

// the matrix-core attention unless QTTS_PREFILL_ATTN_VALU=1
static bool prefill_attn_mx()
{
    // read at every launch (a few hundred ns), so a caller or test can switch
    // paths between calls
    const char *v = getenv("QTTS_PREFILL_ATTN_VALU");
    return !(v && *v && *v != '0');
}

// final-normed hidden of one row (talker.rs:477-481)
__global__ void __launch_bounds__(256)
k_final_rms(const float *x, const uint16_t *gamma, int H, float *out)
{
    __shared__ float red[4];
    const int t = threadIdx.x, lane = t & 63;
    float s = 0.0f;
    for (int k = t; k < H; k += 256) s = fmaf(x[k], x[k], s);
    s = wave_sum_dpp(s);
    if (lane == 0) red[t >> 6] = s;
    __syncthreads();
    const float inv = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)H + 1e-6f);
    for (int k = t; k < H; k += 256) out[k] = x[k] * inv * h2f(gamma[k]);
}

// Synthetic rows for timing: x[i] uniform in [-1, 1) from a hash of (seed, i).
__global__ void k_fill_rows(float *x, int64_t n, uint32_t seed)
{
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        uint32_t h = (uint32_t)i * 0x9E3779B1u ^ seed * 0x85EBCA77u;
        h ^= h >> 15;
        h *= 0x2C1B3C6Du;
        h ^= h >> 12;
        x[i] = (float)(h >> 8) * (1.0f / 8388608.0f) - 1.0f;
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

#define PCHK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) return e_; } while (0)

static bool gemm_shape_ok(const Q4Tiled &w, int K)
{
    return K == w.k && K % GK == 0 && K >= 2 * GK;   // two chunks at least per k-slice
}

// Rows per tile, 16 * MB: one tile when M <= 80; else MB in 3..5 with the
// least padding (larger MB on ties: each weight tile is dequantised once per
// row tile).
static int pick_mb(int M)
{
    if (M <= 80) return (M + 15) / 16;
    int best = 5, pad = 1 << 30;
    for (int mb = 5; mb >= 3; mb--) {
        const int p = (M + 16 * mb - 1) / (16 * mb) * 16 * mb;
        if (p < pad) {
            pad = p;
            best = mb;
        }
    }
    return best;
}

// k-slices of a weight for the prefill projections whose consumer adds
// partials (q|k|v, o, down): about 96 workgroups per row tile.  A function
// of the weight alone, so a row's sums do not depend on the prompt length
// (prefix + suffix prefill stays bit-identical to one full prefill).
static int part_slices(const Q4Tiled &w)
{
    const int tn = (w.G * 32 + GN - 1) / GN, nch = w.k / GK;
    int S = std::max(1, (96 + tn / 2) / tn);
    S = std::min(S, 8);
    while (S > 1 && nch / S < 8) S--;
    return S;
}

// The split-f16 contraction unless QTTS_GEMM_F32=1 (f32 matrix instructions).
static bool gemm_x3()
{
    // read at every launch (a few hundred ns), so a caller or test can switch
    // paths between calls
    const char *v = getenv("QTTS_GEMM_F32");
    return !(v && *v && *v != '0');
}

template <int MB, int EPI>
static hipError_t launch_gemm_mb(const GemmA &a, const Q4Tiled &w, const GemmOut &o, int S, hipStream_t s)
{
    const int tm = (a.M + 16 * MB - 1) / (16 * MB), tn = (w.G * 32 + GN - 1) / GN;
    const dim3 grid(tm * tn * S);
    if (gemm_x3() && w.bshift >= 0) {
        if (a.inv)
            hipLaunchKernelGGL((k_gemm_q4<MB, EPI, true, true>), grid, dim3(256), 0, s, a, w, o, tm, S);
        else
            hipLaunchKernelGGL((k_gemm_q4<MB, EPI, false, true>), grid, dim3(256), 0, s, a, w, o, tm, S);
    } else {
        if (a.inv)
            hipLaunchKernelGGL((k_gemm_q4<MB, EPI, true, false>), grid, dim3(256), 0, s, a, w, o, tm, S);
        else
            hipLaunchKernelGGL((k_gemm_q4<MB, EPI, false, false>), grid, dim3(256), 0, s, a, w, o, tm, S);
    }
    return hipGetLastError();
}

// The staging-range slots of every k-slice fit the GEMM's reads: at most 16
// slots per slice (two per lane of a row's 8), all within the row.
static bool rmax_fits(const GemmA &a, int K, int S)
{
    if (!a.rmax) return true;
    if (a.rslots < 1 || a.rw < 1 || (int64_t)a.rslots * a.rw < K) return false;
    const int nch = K / GK;
    for (int sl = 0; sl < S; sl++) {
        const int c0 = sl * nch / S, c1 = (sl + 1) * nch / S;
        if ((c1 * GK - 1) / a.rw - (c0 * GK) / a.rw >= 16) return false;
    }
    return true;
}

template <int EPI>
static hipError_t launch_gemm(const GemmA &a, const Q4Tiled &w, const GemmOut &o, int S, hipStream_t s)
{
    if (!gemm_shape_ok(w, w.k) || a.M < 1 || a.lda % 4 || S < 1 || S > w.k / (2 * GK)) return hipErrorInvalidValue;
    if (!rmax_fits(a, w.k, S) || (o.rmax && o.rslots < (w.G * 32 + GN - 1) / GN)) return hipErrorInvalidValue;
    if (EPI == GEMM_SWIGLU && (!w.interleave || w.G % 4)) return hipErrorInvalidValue;
    if ((EPI == GEMM_BIAS || EPI == GEMM_BIAS_SILU) && !o.bias) return hipErrorInvalidValue;
    if (EPI != GEMM_PART && S != 1) return hipErrorInvalidValue;
    if (!a.inv != !a.gamma) return hipErrorInvalidValue;   // a fused norm has both
    switch (pick_mb(a.M)) {
    case 1: return launch_gemm_mb<1, EPI>(a, w, o, S, s);
    case 2: return launch_gemm_mb<2, EPI>(a, w, o, S, s);
    case 3: return launch_gemm_mb<3, EPI>(a, w, o, S, s);
    case 4: return launch_gemm_mb<4, EPI>(a, w, o, S, s);
    default: return launch_gemm_mb<5, EPI>(a, w, o, S, s);
    }
}

bool gemm_supported(const Q4Tiled &w)
{
    return gemm_shape_ok(w, w.k);
}

static hipError_t row_absmax(const float *X, int ld, int M, int K, int rw, int rslots, float *out, hipStream_t s)
{
    const int n = M * rslots;
    hipLaunchKernelGGL(k_row_absmax, dim3((n + 3) / 4), dim3(256), 0, s, X, ld, M, K, rw, rslots, out);
    return hipGetLastError();
}

// Rows of any magnitude (gemm_q4 takes any finite input, gemv.rs:349-412):
// each row's largest |x| first (rmax, rows floats), for the staging's range.
hipError_t enqueue_gemm_rows(const Q4Tiled &w, const float *X, int rows, float *Y, int ldy, float *rmax,
                             hipStream_t s)
{
    if (gemm_x3()) PCHK(row_absmax(X, w.k, rows, w.k, w.k, 1, rmax, s));
    const GemmA a{X, w.k, nullptr, nullptr, rows, rmax, 1, w.k, 0};
    return launch_gemm<GEMM_STORE>(a, w, GemmOut{Y, ldy, std::min(ldy, w.G * 32), nullptr, 0}, 1, s);
}

// Y = X W + bias, optionally through SiLU (the text projection's fc1 / fc2,
// talker.rs:105-116, over a batch of rows).  rmax: rows floats, as above.
hipError_t enqueue_gemm_bias(const Q4Tiled &w, const float *X, int rows, const float *bias, bool silu, float *Y,
                             int ldy, float *rmax, hipStream_t s)
{
    if (gemm_x3()) PCHK(row_absmax(X, w.k, rows, w.k, w.k, 1, rmax, s));
    const GemmA a{X, w.k, nullptr, nullptr, rows, rmax, 1, w.k, 0};
    const GemmOut o{Y, ldy, std::min(ldy, w.n), bias, 0};
    return silu ? launch_gemm<GEMM_BIAS_SILU>(a, w, o, 1, s) : launch_gemm<GEMM_BIAS>(a, w, o, 1, s);
}

// Slots of the down projection's input range: one per 64 output columns of
// the gate|up GEMM (one column tile).
static int down_rslots(const TalkerDev &m) { return ((m.inter + 63) / 64 + 3) & ~3; }

bool prefill_supported(const TalkerDev &m)
{
    if (m.n_heads != 16 || m.n_kv_heads != 8 || m.hidden % GK) return false;
    for (int l = 0; l < m.n_layers; l++) {
        const LayerDev &L = m.layers[l];
        if (!gemm_shape_ok(L.qkv, m.hidden) || !gemm_shape_ok(L.o, 16 * HEAD_DIM) ||
            !gemm_shape_ok(L.gate_up, m.hidden) || !gemm_shape_ok(L.down, m.inter) || !L.gate_up.interleave ||
            L.gate_up.G % 4 || L.qkv.G * 32 < 32 * HEAD_DIM || L.gate_up.G * 16 < m.inter ||
            L.o.G * 32 < m.hidden || L.down.G * 32 < m.hidden)
            return false;
    }
    return true;
}

// Column slots per prompt row of the staging-range buffer (PrefillWs.rmax):
// 8 for the o-projection's input (one per kv head), one per 64 columns for
// the down projection's.
int64_t prefill_rmax_slots(const TalkerDev &m) { return std::max<int64_t>(8, down_rslots(m)); }

// The staging power of two of rows normed with this gamma (f16 bit
// patterns, on the host): |x * inv * gamma| <= sqrt(n) * max|gamma|, since
// |x_k| * inv <= sqrt(n); the shift takes that bound into [2^13, 2^14].
// Largest finite |value| of n f16 bit patterns (inf / NaN skipped: they
// give no finite bound and propagate as in f32).
double f16_max_abs(const uint16_t *h, int n)
{
    double g = 0.0;
    for (int k = 0; k < n; k++) {
        const uint16_t a = h[k] & 0x7FFFu;
        if (a >= 0x7C00u) continue;
        const int e = a >> 10, f = a & 0x3FF;
        g = std::max(g, e ? std::ldexp(1024.0 + f, e - 25) : std::ldexp((double)f, -24));
    }
    return g;
}

// The power of two that takes a bound on |values| into [2^13, 2^14].
int bound_shift(double bound)
{
    if (!(bound > 0.0) || !std::isfinite(bound)) return 0;
    return std::max(-100, std::min(100, 14 - (int)std::ceil(std::log2(bound))));
}

// The attention's staging shifts: none while the bound lies in [2^-4, 2^14]
// (the values' f16 halves then neither overflow nor lose precision against
// the bound), else the shift that takes it into [2^13, 2^14].
int attn_shift(double bound)
{
    if (bound >= 0x1p-4 && bound <= 0x1p14) return 0;
    return bound_shift(bound);
}

int norm_shift(const uint16_t *gamma_host, int n)
{
    return bound_shift(std::sqrt((double)n) * f16_max_abs(gamma_host, n));
}

// Floats per prompt row of the k-slice partials buffer.
int64_t prefill_part_floats(const TalkerDev &m)
{
    int64_t f = 0;
    for (int l = 0; l < m.n_layers; l++) {
        const LayerDev &L = m.layers[l];
        f = std::max<int64_t>(f, (int64_t)part_slices(L.qkv) * L.qkv.G * 32);
        f = std::max<int64_t>(f, (int64_t)part_slices(L.o) * L.o.G * 32);
        f = std::max<int64_t>(f, (int64_t)part_slices(L.down) * L.down.G * 32);
    }
    return f;
}

hipError_t enqueue_fill_rows(float *x, int64_t n, uint32_t seed, hipStream_t s)
{
    hipLaunchKernelGGL(k_fill_rows, dim3(1024), dim3(256), 0, s, x, n, seed);
    return hipGetLastError();
}

hipError_t enqueue_row_inv(const float *X, int ld, int M, int K, float *inv, hipStream_t s)
{
    if (K % 4 || ld % 4) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_row_inv, dim3((M + 3) / 4), dim3(256), 0, s, X, ld, M, K, inv);
    return hipGetLastError();
}

// The prefill's gate|up GEMM of layer l alone (pw.x rows and pw.inv set).
hipError_t enqueue_gemm_gateup(const TalkerDev &m, const PrefillWs &pw, int l, int M, hipStream_t s)
{
    const LayerDev &L = m.layers[l];
    return launch_gemm<GEMM_SWIGLU>(GemmA{pw.x, m.hidden, pw.inv, L.post_norm, M, nullptr, 0, 0, L.post_shift},
                                    L.gate_up, GemmOut{pw.h, m.inter, m.inter, nullptr, 0, pw.rmax, down_rslots(m)},
                                    1, s);
}

// A projection into k-slice partials: slice s of row m at part[s * M * ld +
// m * ld], ld = the weight's padded width.
static hipError_t gemm_parts(const GemmA &a, const Q4Tiled &w, const PrefillWs &pw, int *S, int *ld, hipStream_t s)
{
    *S = part_slices(w);
    *ld = w.G * 32;
    return launch_gemm<GEMM_PART>(a, w, GemmOut{pw.part, *ld, *ld, nullptr, (size_t)a.M * *ld}, *S, s);
}

// Rows pw.x[0..M) at positions start..start+M-1 through every layer; the
// last row's final-normed hidden goes to hidden_out.  Positions
// start..start+M-1 must be backed by the page table.
hipError_t enqueue_talker_prefill(const TalkerDev &m, const PrefillWs &pw, int M, int64_t start, float *hidden_out,
                                  hipStream_t s)
{
    if (M < 1 || M > pw.cap_rows) return hipErrorInvalidValue;
    const int H = m.hidden, A = 16 * HEAD_DIM;
    int S, ld;
    PCHK(enqueue_row_inv(pw.x, H, M, H, pw.inv, s));
    for (int l = 0; l < m.n_layers; l++) {
        const LayerDev &L = m.layers[l];
        // q|k|v (input norm fused), QK-norm + RoPE + KV append, attention
        PCHK(gemm_parts(GemmA{pw.x, H, pw.inv, L.input_norm, M, nullptr, 0, 0, L.in_shift}, L.qkv, pw, &S, &ld, s));
        hipLaunchKernelGGL(k_prefill_qkv_post, dim3(M, 8), dim3(256), 0, s, pw.part, S, (size_t)M * ld, ld, M, start,
                           L.q_norm, L.k_norm, m.rope_cos, m.rope_sin, m.kv, l, pw.q, A);
        PCHK(hipGetLastError());
        // attention rows, and each row's largest |value| per kv head's two
        // q heads (the o-projection's staging range: 8 slots of 256)
        if (prefill_attn_mx()) {
            if (L.q_shift || L.k_shift || L.v_shift)
                hipLaunchKernelGGL(k_prefill_attn_mx<true>, dim3((M + 7) / 8, 8), dim3(256), 0, s, pw.q, A, M, start,
                                   m.kv, l, pw.attn, A, pw.rmax, 8, L.q_shift, L.k_shift, L.v_shift);
            else
                hipLaunchKernelGGL(k_prefill_attn_mx<false>, dim3((M + 7) / 8, 8), dim3(256), 0, s, pw.q, A, M, start,
                                   m.kv, l, pw.attn, A, pw.rmax, 8, 0, 0, 0);
        } else {
            hipLaunchKernelGGL(k_prefill_attn<PREFILL_ATTN_QB>, dim3((M + PREFILL_ATTN_QB - 1) / PREFILL_ATTN_QB, 8),
                               dim3(256), 0, s, pw.q, A, M, start, m.kv, l, pw.attn, A);
            PCHK(hipGetLastError());
            PCHK(row_absmax(pw.attn, A, M, A, 2 * HEAD_DIM, 8, pw.rmax, s));
        }
        PCHK(hipGetLastError());
        // o-proj, residual, post-attention norm
        PCHK(gemm_parts(GemmA{pw.attn, A, nullptr, nullptr, M, pw.rmax, 8, 2 * HEAD_DIM, 0}, L.o, pw, &S, &ld, s));
        hipLaunchKernelGGL(k_resid_add_inv, dim3(M), dim3(256), 0, s, pw.x, H, pw.part, S, (size_t)M * ld, ld, H,
                           pw.inv);
        PCHK(hipGetLastError());
        // gate|up with SwiGLU (and the down projection's staging range per
        // 64 columns), down, residual, next layer's input norm
        PCHK(enqueue_gemm_gateup(m, pw, l, M, s));
        PCHK(gemm_parts(GemmA{pw.h, m.inter, nullptr, nullptr, M, pw.rmax, down_rslots(m), 64, 0}, L.down, pw, &S,
                        &ld, s));
        hipLaunchKernelGGL(k_resid_add_inv, dim3(M), dim3(256), 0, s, pw.x, H, pw.part, S, (size_t)M * ld, ld, H,
                           pw.inv);
        PCHK(hipGetLastError());
    }
    hipLaunchKernelGGL(k_final_rms, dim3(1), dim3(256), 0, s, pw.x + (size_t)(M - 1) * H, m.final_norm, H,
                       hidden_out);
    return hipGetLastError();
}

}  // namespace qtts
