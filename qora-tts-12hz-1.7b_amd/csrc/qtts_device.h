// qtts_device.h — device-side data structures shared by the kernels and the
// host runtime of the MI355X decode path.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace qtts {

// Tiling of one Q4 weight for the split-K GEMV (see qtts_kernels.hip).
// A tile covers GB 32-column groups x KC rows, KC = R * T / GB, and is
// stored contiguously: nibble block [R][T] x 16 B, then scale block [T] x
// R f16 (R = 2, 4 or 8 rows per thread).  Thread t of a workgroup owns one
// group gl and rows r * (T/GB) + ph, r = 0..R-1, of the tile: with NW = T/64
// waves, gl = (t/64) % GB and ph = (t/64)/GB * 64 + t % 64 when NW % GB == 0
// (one group per wave), else gl = t % GB and ph = t / GB.  A weight with
// S = ceil(k / KC) k-slices writes S partial sums per output; S = 1 is a
// full-k pass.
enum TileCfg : int32_t {
    TILE_G8_T256 = 0,       // KC = 256
    TILE_G8_T128 = 1,       // KC = 128
    TILE_G1_T64 = 2,        // KC = 512
    TILE_G1_T128 = 3,       // KC = 1024
    TILE_G1_T256 = 4,       // KC = 2048
    TILE_G1_T384 = 5,       // KC = 3072
    TILE_G1_T768 = 6,       // KC = 6144
    TILE_G2_T256 = 7,       // KC = 1024
    TILE_G2_T512 = 8,       // KC = 2048
    TILE_G4_T256 = 9,       // KC = 512
    TILE_G1_T512 = 10,      // KC = 4096
    TILE_G1_T256_R4 = 11,   // KC = 1024
    TILE_G1_T256_R2 = 12,   // KC = 512
    TILE_G1_T512_R4 = 13,   // KC = 2048
    TILE_G2_T512_R4 = 14,   // KC = 1024
    TILE_G1_T512_R2 = 15,   // KC = 1024
    TILE_G2_T256_R4 = 16,   // KC = 512
    TILE_G1_T1024_R2 = 17,  // KC = 2048
    TILE_G2_T1024_R4 = 18,  // KC = 2048
    TILE_COUNT
};

struct TileShape { int T, GB, R; };
__host__ __device__ constexpr TileShape tile_shape(int cfg)
{
    constexpr TileShape tab[TILE_COUNT] = {
        {256, 8, 8}, {128, 8, 8}, {64, 1, 8}, {128, 1, 8}, {256, 1, 8}, {384, 1, 8}, {768, 1, 8},
        {256, 2, 8}, {512, 2, 8}, {256, 4, 8}, {512, 1, 8}, {256, 1, 4}, {256, 1, 2}, {512, 1, 4},
        {512, 2, 4}, {512, 1, 2}, {256, 2, 4}, {1024, 1, 2}, {1024, 2, 4}};
    return tab[cfg];
}

struct Q4Tiled {
    const uint8_t *data;   // S*CT tiles, tile (s, c) at index s*CT + c
    int32_t k, n;          // logical shape (in, out)
    int32_t G;             // 32-column groups, padded to a multiple of GB
    int32_t S, CT;         // k-slices, column tiles
    int32_t KC;            // rows per slice
    int32_t cfg;           // TileCfg
    int32_t tile_bytes;
    int32_t npad;          // G * 32
    int32_t interleave;    // 1: two fused weights alternate by group (a0 b0 a1 b1 ...)
    int32_t bshift;        // split-f16 matrix path: dequantised weights scaled by 2^bshift (-1: not usable)
};

// Row-major Q4 (the reference layout) kept for embedding lookups.
struct Q4Rows {
    const uint8_t *packed;   // [rows][G*16]
    const uint16_t *scales;  // [rows][G]
    int32_t rows, n, G;
};

// Per-context generation state, resident in device memory so one captured
// graph replays every frame.
struct DevState {
    int64_t position;        // RoPE position of the next talker step
    int32_t kv_len;          // talker positions cached
    int32_t frame_idx;       // frames emitted so far
    uint64_t rng;            // xorshift64 state
    uint32_t prev[16];       // repetition-penalty history
    uint32_t used[16];       // codes fed downstream this frame
    uint32_t pred[16];       // codes predicted this frame
    uint32_t fcode[16];      // teacher-forced codes of this frame (force on)
    int32_t stop;            // 1 after EOS: frame kernels become no-ops
    int32_t eos;             // sticky EOS flag
    int32_t nan_flag;        // a sampler met a NaN
    int32_t force;           // teacher forcing on
    int32_t n_text;          // trailing text rows
    int32_t ring_base;       // frame_idx of ring slot 0
    int32_t forced_base;     // frame_idx of forced row 0
    int32_t sync_err;        // a bounded cross-workgroup wait ran out (results invalid)
    // sampler parameters
    float temperature, top_p, rep_penalty, onset_temperature;
    int32_t top_k, onset_frames, eos_enabled;
    uint32_t eos_id;
};
// the decode attention reads position and kv_len as one 16-byte load
static_assert(offsetof(DevState, position) == 0 && offsetof(DevState, kv_len) == 8, "DevState head");

constexpr int KV_PAGE = 64;          // talker KV positions per page
constexpr int HEAD_DIM = 128;
constexpr int PRED_KV_CAP = 16;      // predictor positions (2 + 14)

}  // namespace qtts
