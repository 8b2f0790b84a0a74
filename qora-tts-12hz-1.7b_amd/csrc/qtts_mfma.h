// qtts_mfma.h — the f32 matrix-core main loop shared by the prefill GEMM
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

// The double-buffered schedule over nch >= 1 chunks.  fetch(f, c) issues
// chunk c's global loads into register set f, stage(f, buf) writes a
// register set into LDS buffer buf, mma(buf) runs the MFMAs of buffer buf.
// Two register sets alternate, so chunk c's loads are issued two chunks
// before its MFMAs and one before its staging, and no wait on memory sits
// between MFMAs; chunks alternate LDS buffers 0 and 1.
template <class F, class FetchFn, class StageFn, class MmaFn>
__device__ __forceinline__ void mfma_pipeline(int nch, FetchFn &&fetch, StageFn &&stage, MmaFn &&mma)
{
    F fa, fb;
    fetch(fa, 0);
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

}  // namespace qtts
