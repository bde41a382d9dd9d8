// Process-wide kernel-variant overrides: the planners' choices can be forced
// per call (tests that cover every tile shape, tuning sweeps). Each knob
// starts from its environment variable, read once when the library first
// needs it, and can be changed at any time through rpx_set_tuning(); a
// change applies to the calls that start after it.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>

namespace rpx {

enum TuneKnob : int {
  kTuneInt4Tile = 0,    // INT4 fused GEMM tile (0: planner)        RPX_GEMM_TILE
  kTuneBf16Tile = 1,    // bf16 GEMM tile (0: planner)              RPX_GEMM_TILE
  kTuneFp8Tile = 2,     // fp8 GEMM tile (0: planner)               RPX_FP8_TILE
  kTuneSkinnyTile = 3,  // one-launch skinny tile (0: planner)      RPX_SKINNY_TILE
  kTuneSkinny2 = 4,     // two-launch skinny: -1 planner, 0 never, 1 for M <= 16   RPX_SKINNY2
  kTuneSkinny2One = 5,  // M <= 4 form: -1 planner, 0 two launches, 1 one launch  RPX_SKINNY2_ONE
  kTuneSpinLimit = 6,   // polls of the skinny kernels' bounded waits (0: default)
  kTuneBand = 7,        // row-blocks per band of the GEMM tile order (0: planner)  RPX_GEMM_BAND
  kTuneDxPacked = 8,    // INT4 + LoRA input gradient's weight operand: -1 planner (bf16
                        // W_b^T), 0 bf16 W_b^T, 1 packed where allowed    RPX_DX_PACKED
  kTuneRankBlocks = 9,  // workgroups a token-reduction product (dA, dB) aims for (0: planner)
  kTuneRankNtU = 10,    // rank_nt 128-column steps in flight per wave (0: planner; 4, 8, 16)
  kTuneFp8Splits = 11,  // fp8 GEMM split-K count (0: planner; else forced where it divides K)
  kTuneFp8Pair = 12,    // fp8 backward's two products in one launch: -1 planner, 0 never  RPX_FP8_PAIR
  kTuneCount = 13
};

// Current value of a knob.
int tune(int knob);
// Sets a knob; false if the knob or the value is unknown.
bool tune_set(int knob, int value);

// Tile ids of the GEMM planners (the values kTuneInt4Tile / kTuneBf16Tile take).
enum GemmTile : int {
  kTileAuto = 0,
  kTileI4_256x128 = 1,     // INT4 256 x 128, three stages, one workgroup per CU
  kTileI4_128x128 = 2,     // INT4 128 x 128, stages chosen by the scale footprint
  kTileI4_64x128 = 3,      // INT4 64 x 128, three stages
  kTileBf_256x128 = 4,     // bf16 256 x 128, two stages
  kTileBf_128x128 = 5,     // bf16 128 x 128, two stages
  kTileBf_64x128 = 6,      // bf16 64 x 128, three stages
  kTileI4_256x256 = 7,     // INT4 256 x 256 (sweeps; no activation epilogues)
  kTileBf_256x256 = 8,     // bf16 256 x 256 (sweeps; no activation epilogues)
  kTileBf_128x96 = 9,      // bf16 128 x 96, three stages
  kTileI4_128x128s2 = 10,  // INT4 128 x 128, two stages, three workgroups per CU
  kTileI4_128x128s3 = 11,  // INT4 128 x 128, three stages, two workgroups per CU
  kTileI4_256x128s2 = 12,  // INT4 256 x 128, two stages, two workgroups per CU
  kTileBf_256x128s3 = 13,  // bf16 256 x 128, three stages, one workgroup per CU
  kTileT4_256x128 = 14,    // packed-weight input gradient 256 x 128, one workgroup per CU
  kTileT4_128x128 = 15,    // packed-weight input gradient 128 x 128, one workgroup per CU
  kTileT4_64x128 = 16,     // packed-weight input gradient 64 x 128, two workgroups per CU
  kTileI4L_256x192 = 17,   // INT4 256 x 192, B dequantized once per workgroup into LDS
};

// Sets the dynamic-LDS limit of a kernel once per device (idempotent, so
// concurrent first calls are harmless).
hipError_t ensure_lds_limit(const void* kernel, int bytes, std::atomic<unsigned>& done_devices);

}  // namespace rpx
