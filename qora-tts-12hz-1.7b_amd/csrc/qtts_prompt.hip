// qtts_prompt.hip — prompt rows built on the device: embedding-table rows
// for a batch of ids, the codec side of the ICL block, and row sums.
//
//   k_gather_rows        text_embedding rows of a batch of ids    talker.rs:107
//   k_codec_frame_rows   codec row of code 0 + predictor rows of
//                        codes 1..15 per reference frame          generate_new.rs:161-172
//   k_add_rows           text side + codec side                    generate_new.rs:130-132, 174-189
//
// Every value is an exact Q4 dequantisation (s * (nib - 8)) or a sum taken
// in the reference's order, so these rows are bit-identical to the
// reference's.  The text projection between them (fc1, SiLU, fc2) runs on
// the matrix-core GEMM (qtts_prefill.hip).

#include "qtts_device.h"
#include "qtts_kernels.h"
#include "qtts_devutil.h"

namespace qtts {

// out[i][j] = row ids[i] of e, j < e.n.  Grid (column blocks, rows).
__global__ void __launch_bounds__(256)
k_gather_rows(Q4Rows e, const uint32_t *ids, int n, float *out, int ld)
{
    const int j = blockIdx.x * 256 + threadIdx.x, i = blockIdx.y;
    if (j >= e.n || i >= n) return;
    out[(size_t)i * ld + j] = q4_row_value(e, ids[i], j);
}

// Frame t: talker codec row of codes[0][t], then += predictor table g-1 row
// codes[g][t] for g = 1..n_groups, one f32 add at a time in that order.
// codes is [n_groups + 1][n_frames].  Grid (column blocks, frames).
__global__ void __launch_bounds__(256)
k_codec_frame_rows(Q4Rows tcodec, Q4Rows pemb, int n_groups, const uint32_t *codes, int n_frames, float *out,
                   int ld)
{
    const int j = blockIdx.x * 256 + threadIdx.x, t = blockIdx.y;
    if (j >= tcodec.n || t >= n_frames) return;
    float sum = q4_row_value(tcodec, codes[t], j);
    for (int g = 1; g <= n_groups; g++) {
        Q4Rows e = pemb;
        e.packed += (size_t)(g - 1) * e.rows * e.G * 16;
        e.scales += (size_t)(g - 1) * e.rows * e.G;
        sum += q4_row_value(e, codes[(size_t)g * n_frames + t], j);
    }
    out[(size_t)t * ld + j] = sum;
}

__global__ void __launch_bounds__(256)
k_add_rows(const float *a, int lda, const float *b, int ldb, float *out, int ldo, int n)
{
    const int j = blockIdx.x * 256 + threadIdx.x, i = blockIdx.y;
    if (j >= n) return;
    out[(size_t)i * ldo + j] = a[(size_t)i * lda + j] + b[(size_t)i * ldb + j];
}

hipError_t enqueue_gather_rows(const Q4Rows &e, const uint32_t *ids, int n, float *out, int ld, hipStream_t s)
{
    if (n < 1) return hipSuccess;
    hipLaunchKernelGGL(k_gather_rows, dim3((e.n + 255) / 256, n), dim3(256), 0, s, e, ids, n, out, ld);
    return hipGetLastError();
}

hipError_t enqueue_codec_frame_rows(const Q4Rows &tcodec, const Q4Rows &pemb, int n_groups, const uint32_t *codes,
                                    int n_frames, float *out, int ld, hipStream_t s)
{
    if (n_frames < 1) return hipSuccess;
    hipLaunchKernelGGL(k_codec_frame_rows, dim3((tcodec.n + 255) / 256, n_frames), dim3(256), 0, s, tcodec, pemb,
                       n_groups, codes, n_frames, out, ld);
    return hipGetLastError();
}

hipError_t enqueue_add_rows(const float *a, int lda, const float *b, int ldb, float *out, int ldo, int rows, int n,
                            hipStream_t s)
{
    if (rows < 1) return hipSuccess;
    hipLaunchKernelGGL(k_add_rows, dim3((n + 255) / 256, rows), dim3(256), 0, s, a, lda, b, ldb, out, ldo, n);
    return hipGetLastError();
}

}  // namespace qtts
