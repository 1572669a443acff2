// Launch descriptors and launchers shared by the host runtime and the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace satori {

// Formats: BlockQuantization values (src/Satori.Core/BlockQuantization.cs:3) plus Ternary2.
enum Format : int { kQ8_0 = 0, kQ4_0 = 1, kQ4_K = 2, kQ6_K = 3, kTernary2 = 16 };

// Bytes of one Q8_K activation block (src/Satori.Core/Q8KCodec.cs:31).
constexpr int kQ8KBlockBytes = 292;

// One matrix of a launch. Row-major payload: row r starts at w + r * row_bytes.
struct MatDesc {
    const uint8_t* w;   // packed payload (device)
    const float* x;     // FP32 activations [positions][columns] (float products)
    const uint8_t* a;   // Q8_K activations [positions][blocks * 292] (integer products)
    float* y;           // output [positions][rows]
    int rows;
    int pad_;
};

// Shape shared by every member of a launch.
struct LaunchShape {
    int format;         // Format
    int columns;        // C
    int block_size;     // Ternary2 B, else the format's block elements
    int blocks;         // blocks per row
    int64_t row_bytes;  // payload bytes per row
    int positions;      // activation vectors per call
    int rows_max;       // largest member row count (grid extent)
    int rows_per_wg;    // rows one workgroup owns (launcher-chosen)
};

// FP32-activation MatVec for every format (Ternary2, Q8_0, Q4_0, Q4_K, Q6_K). `group` is a device array
// of `count` descriptors or nullptr, in which case `one` is used and count must be 1.
hipError_t launch_gemv_float(const MatDesc& one, const MatDesc* group, int count, LaunchShape shape,
                             hipStream_t stream);

// Q8_K quantization of `positions` rows of `columns` floats (columns a multiple of 256), bit-exact with
// Q8KCodec.QuantizeRow. Output [positions][columns / 256 * 292].
hipError_t launch_q8k_quantize(const float* x, int columns, int positions, uint8_t* out, hipStream_t stream);

// Integer K-format product against Q8_K activations (Q4_K or Q6_K), bit-exact with the reference's
// ExecuteQuantizedTiled composition.
hipError_t launch_gemv_kint(const MatDesc& one, const MatDesc* group, int count, LaunchShape shape,
                            hipStream_t stream);

// Rows one workgroup of the integer product owns (its LDS holds that many rows of block terms).
int kint_tile_rows();

}  // namespace satori
