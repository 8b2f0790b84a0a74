// qtts_snake.h — sin^2 for SnakeBeta (snake_beta, conv.rs:620-640:
// x + e^-beta * sin^2(e^alpha * x)), shared by the speech decoder's
// epilogues and compiled for the host too, so that it can be checked on
// its own against a float64 sin^2.
#pragma once

#include <math.h>

#if defined(__HIPCC__)
#define QTTS_HD __host__ __device__ __forceinline__
#else
#define QTTS_HD static inline
#endif

namespace qtts {

// sin^2(t) for SnakeBeta.  t is reduced by the multiple k of pi/2 nearest
// to it (Cody-Waite: pi/2 as three f32 parts, one fma each), sin r on
// [-pi/4, pi/4] is its Taylor series to r^9 (truncation below 2^-28 of r),
// and an odd k swaps sin^2 for cos^2 = 1 - sin^2 (at least 1/2 there, so
// no cancellation).  Over |t| < 2^14 the largest error is that of squaring
// a correctly rounded sin in f32 (1.2e-7 absolute); larger |t|, inf and NaN
// take sinf.  No branch on the common path.
#if defined(__HIPCC__)
__host__ __device__ __attribute__((noinline))
#else
static
#endif
float snake_sin2_wide(float t)
{
    const float s = sinf(t);
    return s * s;
}

QTTS_HD float snake_sin2(float t)
{
    // out of line: inlined, sinf's wide-argument reduction would be copied
    // into every epilogue element
    if (!(fabsf(t) < 16384.0f)) return snake_sin2_wide(t);
    const float k = __builtin_rintf(t * 0x1.45f306p-1f);   // 2/pi
    float r = __builtin_fmaf(-k, 0x1.921fb6p+0f, t);
    r = __builtin_fmaf(-k, -0x1.777a5cp-25f, r);
    r = __builtin_fmaf(-k, -0x1.ee59dap-50f, r);
    const float r2 = r * r;
    float p = __builtin_fmaf(r2, 0x1.71de3ap-19f, -0x1.a01a02p-13f);   // 1/9!, -1/7!
    p = __builtin_fmaf(r2, p, 0x1.111112p-7f);                         // 1/5!
    p = __builtin_fmaf(r2, p, -0x1.555556p-3f);                        // -1/3!
    const float s = __builtin_fmaf(r * r2, p, r);
    const float s2 = s * s;
    return ((int)k & 1) ? 1.0f - s2 : s2;
}

}  // namespace qtts
