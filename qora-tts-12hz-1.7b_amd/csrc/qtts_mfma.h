// qtts_mfma.h — the matrix-core main loop shared by the prefill GEMM
// (qtts_prefill.hip, k_gemm_q4) and the speech decoder's implicit-GEMM
// convolutions (qtts_decoder.hip, k_conv_gemm).
//
// A workgroup of four waves computes a (16*MB)-row x 128-column tile over
// the contraction in chunks of MFMA_K.  Each chunk is staged in LDS as
// As[row][k] and Bs[column][k], rows MFMA_LD floats apart (MFMA_K + 4: the
// padding spreads a lane group's 16-byte reads over the banks).
#pragma once
#include "qtts_devutil.h"

namespace qtts {

constexpr int MFMA_N = 128, MFMA_K = 32, MFMA_LD = MFMA_K + 4;

// acc[i][j] += A rows 16i..16i+15 x B columns 16*cb[j]..+15 over one staged
// chunk, on v_mfma_f32_16x16x4_f32 (f32 operands, f32 accumulation).  Lane
// (r16 = lane % 16, q = lane / 16) reads its A row and B column as one
// 16-byte LDS load per 16-wide slice (k = 4q..4q+3).  Element e of
// acc[i][j] is then row 16i + 4q + e, column 16*cb[j] + r16.
template <int MB>
__device__ __forceinline__ void mfma_chunk(f32x4 (&acc)[MB][2], const float *As, const float *Bs, const int (&cb)[2],
                                           int lane)
{
    const int r16 = lane & 15, q = lane >> 4;
#pragma unroll
    for (int kk = 0; kk < MFMA_K / 16; kk++) {
        f32x4 av[MB], bv[2];
#pragma unroll
        for (int i = 0; i < MB; i++) av[i] = *(const f32x4 *)&As[(16 * i + r16) * MFMA_LD + 16 * kk + 4 * q];
#pragma unroll
        for (int j = 0; j < 2; j++) bv[j] = *(const f32x4 *)&Bs[(16 * cb[j] + r16) * MFMA_LD + 16 * kk + 4 * q];
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
            for (int i = 0; i < MB; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i][e], bv[j][e], acc[i][j], 0, 0, 0);
    }
}

// The split-f16 form of the contraction (f32-accurate on the f16 matrix
// cores): each staged value v is stored as hi = f16(v) and lo = f16(v - hi)
// in rows of MFMA_HLD halves (80 bytes: a lane's 16-byte read of 8 halves
// at 16q bytes), and acc += Ahi Bhi + Ahi Blo + Alo Bhi on
// v_mfma_f32_16x16x32_f16 with f32 accumulation (the dropped Alo Blo is
// below 2^-22 of each term).
constexpr int MFMA_HLD = MFMA_K + 8;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));

// hi = f16(v), lo = f16(v - hi) of two values, as packed pairs: hi by
// v_cvt_pk_f16_f32 (RNE), lo by v_fma_mixlo/mixhi_f16 (hi * -1 + v, the
// exact remainder rounded once to f16).  v is made opaque first: otherwise
// the compiler folds a product feeding the conversion into one
// mixed-precision FMA (v_fma_mix) for hi, rounding the exact product once,
// while lo is formed from the f32-rounded product, and the two disagree by
// an f16 ulp.
//
// The compiler's hazard checks do not see through inline asm: a matrix
// instruction may read lo too soon after the asm wrote it (a VALU write read
// as an MFMA source needs wait states on this GPU, which nothing inserts for
// an asm write).  REG = true, for results that feed a matrix instruction
// straight from registers, forms lo in plain code instead: v - f32(hi) is
// exact in f32 (v and hi agree in all but their last 13 bits), so its one
// rounding to f16 gives the bits of the fused form, and the compiler sees
// every write.  Staged through LDS (REG = false), the LDS write and the
// barrier lie between the asm and any matrix instruction.
template <bool REG = false>
__device__ __forceinline__ void split_f16_pair(float v0, float v1, uint32_t &hi, uint32_t &lo)
{
    asm volatile("" : "+v"(v0), "+v"(v1));
    const h16x2 h = {(_Float16)v0, (_Float16)v1};
    hi = __builtin_bit_cast(uint32_t, h);
    if constexpr (REG) {
        const h16x2 l = {(_Float16)(v0 - (float)h.x), (_Float16)(v1 - (float)h.y)};
        lo = __builtin_bit_cast(uint32_t, l);
    } else {
        uint32_t r;
        asm("" : "=v"(r));   // both halves are written below: no initial value needed
        asm("v_fma_mixlo_f16 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "+v"(r) : "v"(hi), "v"(v0));
        asm("v_fma_mixhi_f16 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(r) : "v"(hi), "v"(v1));
        lo = r;
    }
}

// acc[i][j] += the split-f16 products over one staged chunk: A rows
// 16i..16i+15 (Ah, Al), B columns 16*cb[j]..+15 (Bh, Bl; the column block
// cb at BP extra halves per block).  Element e of acc[i][j] is row
// 16i + 4q + e, column 16*cb[j] + r16, as with mfma_chunk.
template <int MB, int BP = 0>
__device__ __forceinline__ void mfma_chunk_x3(f32x4 (&acc)[MB][2], const _Float16 *Ah, const _Float16 *Al,
                                              const _Float16 *Bh, const _Float16 *Bl, const int (&cb)[2], int lane)
{
    // v_mfma_f32_16x16x32_f16: lane l holds A row l%16 and B column l%16 at
    // k = 8(l/16)..+7; result element e is row 4(l/16) + e, column l%16
    const int r16 = lane & 15, q = lane >> 4;
    half8 ah[MB], al[MB], bh[2], bl[2];
#pragma unroll
    for (int i = 0; i < MB; i++) {
        ah[i] = *(const half8 *)&Ah[(16 * i + r16) * MFMA_HLD + 8 * q];
        al[i] = *(const half8 *)&Al[(16 * i + r16) * MFMA_HLD + 8 * q];
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
        bh[j] = *(const half8 *)&Bh[(16 * cb[j] + r16) * MFMA_HLD + cb[j] * BP + 8 * q];
        bl[j] = *(const half8 *)&Bl[(16 * cb[j] + r16) * MFMA_HLD + cb[j] * BP + 8 * q];
    }
    // the small terms first, then the leading one; each pass over all
    // 2*MB accumulators, so consecutive instructions never share one
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bh[j], acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bl[j], acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bh[j], acc[i][j], 0, 0, 0);
}

// The power of two 2^s that takes a largest magnitude mx into [2^14, 2^15).
// Staged times 2^s, no value of a row reaches the f16 maximum, values above
// 2^-17 of mx keep 22 bits in hi + lo, and smaller ones are off by at most
// 2^-39 of mx (lo's subnormal step).  0 for zero, inf and NaN (those
// propagate as in f32); |s| <= 100, so 2^s and 2^-s are normal floats.
__device__ __forceinline__ int range_shift(float mx)
{
    if (!(mx > 0.0f) || mx == __builtin_huge_valf()) return 0;
    int e;
    (void)__builtin_frexpf(mx, &e);              // mx in [2^(e-1), 2^e)
    return max(-100, min(100, 15 - e));
}

// The double-buffered schedule over nch >= 1 chunks.  fetch(f, c) issues
// chunk c's global loads into register set f, stage(f, buf) writes a
// register set into LDS buffer buf, mma(buf) runs the MFMAs of buffer buf.
// Two register sets alternate, so chunk c's loads are issued two chunks
// before its MFMAs and one before its staging, and no wait on memory sits
// between MFMAs; chunks alternate LDS buffers 0 and 1.
//
// pre() runs once after chunk 0's loads are issued and before chunk 1's:
// per-tile set-up that waits on loads issued before the pipeline (they are
// older than chunk 0's, so the wait leaves chunk 0 in flight).
template <class F, class FetchFn, class StageFn, class PreFn, class MmaFn>
__device__ __forceinline__ void mfma_pipeline(int nch, FetchFn &&fetch, StageFn &&stage, PreFn &&pre, MmaFn &&mma)
{
    F fa, fb;
    fetch(fa, 0);
    pre();
    if (nch > 1) fetch(fb, 1);
    stage(fa, 0);
    __syncthreads();
    int c = 0;
    for (; c + 3 < nch; c += 2) {
        fetch(fa, c + 2);
        mma(0);
        stage(fb, 1);
        __syncthreads();
        fetch(fb, c + 3);
        mma(1);
        stage(fa, 0);
        __syncthreads();
    }
    if (c + 2 < nch) {
        fetch(fa, c + 2);
        mma(0);
        stage(fb, 1);
        __syncthreads();
        mma(1);
        stage(fa, 0);
        __syncthreads();
        mma(0);
    } else if (c + 1 < nch) {
        mma(0);
        stage(fb, 1);
        __syncthreads();
        mma(1);
    } else {
        mma(0);
    }
}

template <class F, class FetchFn, class StageFn, class MmaFn>
__device__ __forceinline__ void mfma_pipeline(int nch, FetchFn &&fetch, StageFn &&stage, MmaFn &&mma)
{
    mfma_pipeline<F>(nch, fetch, stage, [] {}, mma);
}

}  // namespace qtts
