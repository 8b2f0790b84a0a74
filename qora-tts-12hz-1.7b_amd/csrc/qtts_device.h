// qtts_device.h — device-side data structures shared by the kernels and the
// host runtime of the MI355X decode path.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qtts {

// Tiling of one Q4 weight for the split-K GEMV (see qtts_kernels.hip).
// A tile covers GB 32-column groups x KC rows, KC = R * T / GB, and is
// stored contiguously: nibble block [R][T] x 16 B, then scale block [T] x
// R f16.  Thread t of a workgroup owns group (t % GB) and rows
// r * (T/GB) + t / GB, r = 0..R-1, of the tile.
enum TileCfg : int32_t {
    TILE_S256 = 0,   // T=256, GB=8,  R=8  -> KC = 256   (split-K)
    TILE_S128 = 1,   // T=128, GB=8,  R=8  -> KC = 128   (split-K)
    TILE_D256 = 2,   // T=256, GB=1,  R=8  -> KC = 2048  (one slice for k <= 2048)
    TILE_D384 = 3,   // T=384, GB=1,  R=8  -> KC = 3072
    TILE_D768 = 4,   // T=768, GB=1,  R=8  -> KC = 6144
    TILE_COUNT
};

struct TileShape { int T, GB, R; };
__host__ __device__ constexpr TileShape tile_shape(int cfg)
{
    return cfg == TILE_S256 ? TileShape{256, 8, 8}
         : cfg == TILE_S128 ? TileShape{128, 8, 8}
         : cfg == TILE_D256 ? TileShape{256, 1, 8}
         : cfg == TILE_D384 ? TileShape{384, 1, 8}
                            : TileShape{768, 1, 8};
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
    int32_t stop;            // 1 after EOS: frame kernels become no-ops
    int32_t eos;             // sticky EOS flag
    int32_t nan_flag;        // a sampler met a NaN
    int32_t force;           // teacher forcing on
    int32_t n_text;          // trailing text rows
    int32_t ring_base;       // frame_idx of ring slot 0
    int32_t forced_base;     // frame_idx of forced row 0
    int32_t pad0;
    // sampler parameters
    float temperature, top_p, rep_penalty, onset_temperature;
    int32_t top_k, onset_frames, eos_enabled;
    uint32_t eos_id;
};

constexpr int KV_PAGE = 64;          // talker KV positions per page
constexpr int HEAD_DIM = 128;
constexpr int PRED_KV_CAP = 16;      // predictor positions (2 + 14)

}  // namespace qtts
