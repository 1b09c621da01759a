#pragma once

// Compile-time tuning knobs and CDNA4 hardware constants. Every knob can be
// overridden on the hipcc line, e.g. -DOPWORKS_THREADS=512. They stay
// compile-time because block and tile shapes size LDS arrays and unroll loops.
// Mirrors the knob set of the reference's include/core/config.cuh:15-77.

#include <cfloat>
#include <cmath>

#ifndef OPWORKS_THREADS
#define OPWORKS_THREADS 256
#endif

#ifndef OPWORKS_NUM_WAVES
#define OPWORKS_NUM_WAVES 32
#endif

#ifndef OPWORKS_PACK_SIZE
#define OPWORKS_PACK_SIZE 4
#endif

// Tile knobs of the reference's SIMT GEMM (its include/core/config.cuh:27-37,
// 61-63). They are accepted and checked for source compatibility, but the
// MFMA GEMMs here take their tile shapes from the matrix-core layout
// (ops/gemm_f32.hpp, ops/gemm_bf16.hpp), so these values select nothing.
#ifndef OPWORKS_MATMUL_TILE
#define OPWORKS_MATMUL_TILE 64
#endif

#ifndef OPWORKS_MATMUL_BLOCK
#define OPWORKS_MATMUL_BLOCK 16
#endif

#ifndef OPWORKS_MATMUL_SUBTILE
#define OPWORKS_MATMUL_SUBTILE 4
#endif

#ifndef OPWORKS_LAYERNORM_EPS
#define OPWORKS_LAYERNORM_EPS 1e-5f
#endif

namespace opworks {

// gfx950 hardware constants (not tunable).
constexpr int kWaveSize = 64;                     // lanes per wavefront
constexpr int kWarpSize = kWaveSize;              // the reference's name for the same quantity
constexpr int kMaxThreadsPerBlock = 1024;         // workgroup size limit
constexpr unsigned long long kFullWaveMask = ~0ull;
constexpr int kMaxWavesPerBlock = kMaxThreadsPerBlock / kWaveSize;

constexpr float kInf = INFINITY;
constexpr float kNegInf = -INFINITY;
constexpr float kFloatMax = FLT_MAX;
constexpr float kFloatLowest = -FLT_MAX;

constexpr int kThreads = OPWORKS_THREADS;    // default workgroup size for op launches
constexpr int kNumWaves = OPWORKS_NUM_WAVES; // grid cap: resident workgroups per CU times this
constexpr int kPackSize = OPWORKS_PACK_SIZE; // floats per 16-byte pack in map/reduce kernels
constexpr float kLayerNormEps = OPWORKS_LAYERNORM_EPS;
constexpr int kMatmulTile = OPWORKS_MATMUL_TILE;   // reference SIMT GEMM output tile edge (inert here)
constexpr int kMatmulBlock = OPWORKS_MATMUL_BLOCK; // reference SIMT GEMM K slice (inert here)
constexpr int kMatmulSub = OPWORKS_MATMUL_SUBTILE; // reference SIMT GEMM per-lane sub-tile (inert here)

// The reference's block_reduce contract requires whole multiples of 32 threads;
// it is kept (a 32-lane tail wave is handled through LDS).
constexpr int kBlockGranule = 32;

static_assert(kThreads > 0 && kThreads % kWaveSize == 0 && kThreads <= kMaxThreadsPerBlock,
              "kThreads must be a positive multiple of the 64-lane wavefront and fit in a workgroup");
static_assert(kNumWaves > 0, "kNumWaves must be positive");
static_assert(kPackSize == 1 || kPackSize == 2 || kPackSize == 4, "kPackSize must be 1, 2 or 4");
static_assert(kMatmulTile == kMatmulBlock * kMatmulSub, "kMatmulTile must equal kMatmulBlock * kMatmulSub");
static_assert(kMatmulBlock > 0 && kMatmulSub > 0 && kMatmulBlock * kMatmulBlock <= kMaxThreadsPerBlock,
              "matmul knobs must be positive and describe a workgroup of at most 1024 lanes");
static_assert(kLayerNormEps > 0 && kLayerNormEps <= FLT_MAX, "layer norm epsilon must be finite and positive");

} // namespace opworks
