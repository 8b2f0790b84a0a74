// qtts_devutil.h — device helpers shared by the decode kernels
// (qtts_kernels.hip) and the prefill kernels (qtts_prefill.hip).
#pragma once
#include "qtts_kernels.h"

#include <math.h>

namespace qtts {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint32_t h16)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

// ---------------------------------------------------------------------------
// DPP wave reductions: lane exchanges on the VALU (quad permutes, half-row
// and row mirrors), then the four row totals read as uniform values.  Every
// lane gets the same result.
// ---------------------------------------------------------------------------

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

__device__ __forceinline__ float lane_value(float v, int lane)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

__device__ __forceinline__ float row_sum16(float v)
{
    v += dpp_mov<0xB1>(v);    // quad_perm [1,0,3,2]: lane ^ 1
    v += dpp_mov<0x4E>(v);    // quad_perm [2,3,0,1]: lane ^ 2
    v += dpp_mov<0x141>(v);   // row_half_mirror: the other quad of the half row
    v += dpp_mov<0x140>(v);   // row_mirror: the other half of the row
    return v;
}

__device__ __forceinline__ float row_max16(float v)
{
    v = fmaxf(v, dpp_mov<0xB1>(v));
    v = fmaxf(v, dpp_mov<0x4E>(v));
    v = fmaxf(v, dpp_mov<0x141>(v));
    v = fmaxf(v, dpp_mov<0x140>(v));
    return v;
}

__device__ __forceinline__ float wave_sum_dpp(float v)
{
    v = row_sum16(v);
    return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

__device__ __forceinline__ float wave_max_dpp(float v)
{
    v = fmaxf(v, dpp_mov<0xB1>(v));
    v = fmaxf(v, dpp_mov<0x4E>(v));
    v = fmaxf(v, dpp_mov<0x141>(v));
    v = fmaxf(v, dpp_mov<0x140>(v));
    return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

// ---------------------------------------------------------------------------
// gfx950 lane swaps on the VALU (no LDS crossbar round trip).  Of the
// builtins' two results, the first holds operand a's even 16-lane rows
// (32-lane halves) and b's even rows in the odd positions, the second a's
// odd rows in the even positions and b's odd rows.
// ---------------------------------------------------------------------------

// Sum of the swap's two results.  Both pass through an empty register
// constraint first: used directly in one add, the compiler reads the first
// result twice.
__device__ __forceinline__ float swap_pair_sum(unsigned a, unsigned b)
{
    asm volatile("" : "+v"(a), "+v"(b));
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}

// v + (v of lane ^ 32).  The second operand is the same value passed through
// an empty register copy, so the compiler cannot fold the two operands.
__device__ __forceinline__ float add_xor32(float v)
{
    const unsigned u = __builtin_bit_cast(unsigned, v);
    unsigned w;
    asm volatile("" : "=v"(w) : "0"(u));
    const auto r = __builtin_amdgcn_permlane32_swap(u, w, false, false);
    return swap_pair_sum(r[0], r[1]);
}

// Lanes in even 16-lane rows return lo + (lo of lane ^ 16), lanes in odd
// rows hi + (hi of lane ^ 16): one halving step of a reduce-scatter.
__device__ __forceinline__ float add_xor16_split(float lo, float hi)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, lo),
                                                    __builtin_bit_cast(unsigned, hi), false, false);
    return swap_pair_sum(r[0], r[1]);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 ld4(const float *p) { return *(const f32x4 *)p; }
// streaming read (no reuse within the frame): the non-temporal hint evicts
// less of the last-level cache than an ordinary load
__device__ __forceinline__ f32x4 ld4nt(const float *p) { return __builtin_nontemporal_load((const f32x4 *)p); }

// row `row` of physical page `pg`
__device__ __forceinline__ float *kv_page_ptr(const KvPaged &kv, int layer, int pg, int row, int h, int isv)
{
    const size_t blk = ((size_t)layer * kv.n_phys + pg) * 2 + isv;
    return kv.base + ((blk * 8 + h) * KV_PAGE + row) * HEAD_DIM;
}

__device__ __forceinline__ float *kv_ptr(const KvPaged &kv, int layer, int pos, int h, int isv)
{
    return kv_page_ptr(kv, layer, kv.ptab[pos / KV_PAGE], pos % KV_PAGE, h, isv);
}

// ---------------------------------------------------------------------------
// Q4 dequantisation of one reference-layout row element (exact in f32)
// ---------------------------------------------------------------------------

__device__ __forceinline__ float q4_row_value(const Q4Rows &e, uint32_t row, int col)
{
    const int g = col >> 5, j = col & 31;
    const uint8_t b = e.packed[(size_t)row * e.G * 16 + g * 16 + (j >> 1)];
    const int q = (int)((j & 1) ? (b >> 4) : (b & 0x0F)) - 8;
    return h2f(e.scales[(size_t)row * e.G + g]) * (float)q;
}

}  // namespace qtts
