// Host-only (CPU) entry points: weight quantizers, payload lengths and payload validation.
//
// satori_hip_ternary2_quantize restates Ternary2Matrix.Quantize (src/Satori.Core/Ternary2Matrix.cs:38-71),
// a public reference API (setup only; excluded from timing, docs/benchmark-method.md).
//
// satori_hip_quantize_weights writes Q8_0 / Q4_0 / Q4_K / Q6_K payloads from FP32 weights. The reference
// has no quantizer for these formats (it only decodes GGUF files), so these are this library's own
// simple round-to-nearest quantizers, used to build seeded synthetic matrices. Their only contract is
// that the result is a valid payload whose decode is close to the input; the packing is the exact
// inverse of the reference decoders (Q4KCodec.GetScaleMin / DecodeBlock, Q6KCodec.DecodeBlock,
// QuantizedRow.DecodeQ8Block / DecodeQ4Block).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>

#include "../../include/satori_hip.h"
#include "host_shapes.hpp"

namespace satori {
namespace {

// binary32 -> binary16, round to nearest even (as the (Half) cast).
uint16_t float_to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t abs = x & 0x7FFFFFFFu;
    if (abs >= 0x7F800000u) return static_cast<uint16_t>(sign | 0x7C00u | (abs > 0x7F800000u ? 0x200u : 0u));
    if (abs >= 0x477FF000u) return static_cast<uint16_t>(sign | 0x7C00u);  // rounds to >= 65520: infinity
    if (abs < 0x38800000u) {                                                 // result is subnormal or zero
        if (abs < 0x33000000u) return static_cast<uint16_t>(sign);           // < 2^-25: rounds to zero
        const uint32_t exponent = abs >> 23;
        const uint32_t mantissa = (abs & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126 - exponent;                               // 14..24
        uint32_t half = mantissa >> shift;
        const uint32_t rest = mantissa & ((1u << shift) - 1);
        const uint32_t midpoint = 1u << (shift - 1);
        if (rest > midpoint || (rest == midpoint && (half & 1))) half++;
        return static_cast<uint16_t>(sign | half);
    }
    uint32_t half = ((abs >> 13) - (112u << 10));
    const uint32_t rest = abs & 0x1FFFu;
    if (rest > 0x1000u || (rest == 0x1000u && (half & 1))) half++;
    return static_cast<uint16_t>(sign | half);
}

void put16(uint8_t* p, uint16_t v) {
    p[0] = static_cast<uint8_t>(v);
    p[1] = static_cast<uint8_t>(v >> 8);
}

int nearest(float v) { return static_cast<int>(std::lrintf(v)); }

void quantize_q8_0(const float* x, uint8_t* block) {
    float amax = 0;
    for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(x[j]));
    const float d = amax / 127.0f;
    const uint16_t dh = float_to_half(d);
    const float dq = half_to_float(dh);
    put16(block, dh);
    for (int j = 0; j < 32; ++j) {
        const int q = dq > 0 ? std::clamp(nearest(x[j] / dq), -127, 127) : 0;
        block[2 + j] = static_cast<uint8_t>(static_cast<int8_t>(q));
    }
}

void quantize_q4_0(const float* x, uint8_t* block) {
    float amax = 0, max = 0;
    for (int j = 0; j < 32; ++j)
        if (std::fabs(x[j]) > amax) {
            amax = std::fabs(x[j]);
            max = x[j];
        }
    const float d = max / -8.0f;
    const uint16_t dh = float_to_half(d);
    const float dq = half_to_float(dh);
    put16(block, dh);
    for (int j = 0; j < 16; ++j) {
        const int lo = dq != 0 ? std::clamp(nearest(x[j] / dq) + 8, 0, 15) : 8;
        const int hi = dq != 0 ? std::clamp(nearest(x[j + 16] / dq) + 8, 0, 15) : 8;
        block[2 + j] = static_cast<uint8_t>(lo | (hi << 4));
    }
}

// Inverse of Q4KCodec.GetScaleMin (src/Satori.Core/Q4KCodec.cs:24-36) for 6-bit scale/min pairs.
void pack_q4k_scales(const int* sc, const int* mn, uint8_t* s) {
    std::memset(s, 0, 12);
    for (int j = 0; j < 4; ++j) {
        s[j] = static_cast<uint8_t>((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = static_cast<uint8_t>((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        s[j + 8] = static_cast<uint8_t>((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
    }
}

void quantize_q4_k(const float* x, uint8_t* block) {
    float scale[8], minimum[8];
    for (int j = 0; j < 8; ++j) {
        float lo = x[32 * j], hi = x[32 * j];
        for (int i = 1; i < 32; ++i) {
            lo = std::min(lo, x[32 * j + i]);
            hi = std::max(hi, x[32 * j + i]);
        }
        lo = std::min(lo, 0.0f);
        scale[j] = (hi - lo) / 15.0f;
        minimum[j] = -lo;
    }
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
        max_scale = std::max(max_scale, scale[j]);
        max_min = std::max(max_min, minimum[j]);
    }
    const uint16_t dh = float_to_half(max_scale / 63.0f), mh = float_to_half(max_min / 63.0f);
    const float d = half_to_float(dh), dmin = half_to_float(mh);
    int sc[8], mn[8];
    for (int j = 0; j < 8; ++j) {
        sc[j] = d > 0 ? std::clamp(nearest(scale[j] / d), 0, 63) : 0;
        mn[j] = dmin > 0 ? std::clamp(nearest(minimum[j] / dmin), 0, 63) : 0;
    }
    put16(block, dh);
    put16(block + 2, mh);
    pack_q4k_scales(sc, mn, block + 4);
    uint8_t* qs = block + 16;
    std::memset(qs, 0, 128);
    for (int j = 0; j < 8; ++j) {
        const float step = d * sc[j], offset = dmin * mn[j];
        for (int i = 0; i < 32; ++i) {
            const int q = step > 0 ? std::clamp(nearest((x[32 * j + i] + offset) / step), 0, 15) : 0;
            // Sub-block j: group g = j / 2; low nibble for even j, high nibble for odd j (Q4KCodec.cs:84-85).
            uint8_t& byte = qs[32 * (j / 2) + i];
            byte = static_cast<uint8_t>(byte | (j % 2 == 0 ? q : q << 4));
        }
    }
}

void quantize_q6_k(const float* x, uint8_t* block) {
    float scale[16];
    float max_abs_scale = 0;
    for (int j = 0; j < 16; ++j) {
        float amax = 0;
        for (int i = 0; i < 16; ++i) amax = std::max(amax, std::fabs(x[16 * j + i]));
        scale[j] = amax / 31.0f;
        max_abs_scale = std::max(max_abs_scale, scale[j]);
    }
    const uint16_t dh = float_to_half(max_abs_scale / 127.0f);
    const float d = half_to_float(dh);
    int8_t sc[16];
    for (int j = 0; j < 16; ++j) sc[j] = static_cast<int8_t>(d > 0 ? std::clamp(nearest(scale[j] / d), -128, 127) : 0);
    int q[256];
    for (int j = 0; j < 16; ++j) {
        const float step = d * sc[j];
        for (int i = 0; i < 16; ++i)
            q[16 * j + i] = step != 0 ? std::clamp(nearest(x[16 * j + i] / step) + 32, 0, 63) : 32;
    }
    uint8_t* ql = block;
    uint8_t* qh = block + 128;
    std::memset(block, 0, 208);
    // Inverse of Q6KCodec.DecodeBlock (src/Satori.Core/Q6KCodec.cs:62-80): weight 128h + 32k + l.
    for (int h = 0; h < 2; ++h)
        for (int l = 0; l < 32; ++l) {
            const int q1 = q[128 * h + l], q2 = q[128 * h + 32 + l], q3 = q[128 * h + 64 + l], q4 = q[128 * h + 96 + l];
            ql[64 * h + l] = static_cast<uint8_t>((q1 & 0xF) | ((q3 & 0xF) << 4));
            ql[64 * h + 32 + l] = static_cast<uint8_t>((q2 & 0xF) | ((q4 & 0xF) << 4));
            qh[32 * h + l] = static_cast<uint8_t>((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
        }
    std::memcpy(block + 192, sc, 16);
    put16(block + 208, dh);
}

}  // namespace
}  // namespace satori

using namespace satori;

extern "C" int satori_hip_ternary2_quantize(const float* weights, int rows, int columns, int block_size,
                                            void* payload, size_t payload_length) {
    try {
        const Shape s = ternary2_shape(rows, columns, block_size);
        if (!weights || !payload) fail(SATORI_HIP_E_ARGUMENT_NULL, "Value cannot be null.");
        if (static_cast<int64_t>(payload_length) != s.byte_length)
            fail(SATORI_HIP_E_ARGUMENT, "Payload length must match matrix dimensions.");
        const int64_t n = static_cast<int64_t>(rows) * columns;
        for (int64_t i = 0; i < n; ++i)
            if (!std::isfinite(weights[i])) fail(SATORI_HIP_E_ARGUMENT, "Weights must be finite.");
        uint8_t* out = static_cast<uint8_t*>(payload);
        std::memset(out, 0, static_cast<size_t>(s.byte_length));
        for (int row = 0; row < rows; ++row)
            for (int block = 0; block < s.blocks; ++block) {
                const int column = block * block_size;
                const int count = std::min(block_size, columns - column);
                const float* source = weights + static_cast<int64_t>(row) * columns + column;
                double magnitude = 0;  // FP64 accumulation in order (Ternary2Matrix.cs:55-57)
                for (int i = 0; i < count; ++i) magnitude += std::fabs(static_cast<double>(source[i]));
                const float scale = static_cast<float>(magnitude / count);
                uint8_t* target = out + row * s.row_bytes + static_cast<int64_t>(block) * s.block_bytes;
                std::memcpy(target, &scale, 4);
                if (scale == 0) continue;
                const double threshold = static_cast<double>(scale) / 2;  // FP64 threshold (:63)
                for (int i = 0; i < count; ++i) {
                    const double v = source[i];
                    const int code = v > threshold ? 1 : v < -threshold ? 2 : 0;
                    target[4 + i / 4] = static_cast<uint8_t>(target[4 + i / 4] | (code << (2 * (i % 4))));
                }
            }
        return SATORI_HIP_OK;
    } catch (const Failure& f) {
        record_error(f.message);
        return f.status;
    }
}

extern "C" int satori_hip_quantize_weights(int format, const float* weights, int rows, int columns, void* payload,
                                           size_t payload_length) {
    try {
        const Shape s = quantized_shape(rows, columns, format);
        if (!weights || !payload) fail(SATORI_HIP_E_ARGUMENT_NULL, "Value cannot be null.");
        if (static_cast<int64_t>(payload_length) != s.byte_length)
            fail(SATORI_HIP_E_ARGUMENT, "Incorrect quantized payload length.");
        const int64_t n = static_cast<int64_t>(rows) * columns;
        for (int64_t i = 0; i < n; ++i)
            if (!std::isfinite(weights[i])) fail(SATORI_HIP_E_ARGUMENT, "Weights must be finite.");
        uint8_t* out = static_cast<uint8_t*>(payload);
        for (int row = 0; row < rows; ++row)
            for (int b = 0; b < s.blocks; ++b) {
                const float* x = weights + static_cast<int64_t>(row) * columns + static_cast<int64_t>(b) * s.block_size;
                uint8_t* block = out + row * s.row_bytes + static_cast<int64_t>(b) * s.block_bytes;
                switch (format) {
                    case SATORI_HIP_Q8_0: quantize_q8_0(x, block); break;
                    case SATORI_HIP_Q4_0: quantize_q4_0(x, block); break;
                    case SATORI_HIP_Q4_K: quantize_q4_k(x, block); break;
                    default: quantize_q6_k(x, block); break;
                }
            }
        return SATORI_HIP_OK;
    } catch (const Failure& f) {
        record_error(f.message);
        return f.status;
    }
}

// Ternary2Shape.ByteLength / QuantizedMatrixShape.ByteLength with the reference's argument checks.
extern "C" int satori_hip_payload_length(int format, int rows, int columns, int block_size, int64_t* length) {
    try {
        if (!length) fail(SATORI_HIP_E_ARGUMENT_NULL, "Value cannot be null.");
        const Shape s = format == SATORI_HIP_TERNARY2 ? ternary2_shape(rows, columns, block_size)
                                                      : quantized_shape(rows, columns, format);
        *length = s.byte_length;
        return SATORI_HIP_OK;
    } catch (const Failure& f) {
        record_error(f.message);
        return f.status;
    }
}

// Ternary2Matrix.FromPacked checks (src/Satori.Core/Ternary2Matrix.cs:73-101), on the host.
extern "C" int satori_hip_ternary2_validate(int rows, int columns, int block_size, const void* payload,
                                            size_t payload_length) {
    try {
        const Shape s = ternary2_shape(rows, columns, block_size);
        if (!payload) fail(SATORI_HIP_E_ARGUMENT_NULL, "Value cannot be null.");
        if (static_cast<int64_t>(payload_length) != s.byte_length)
            fail(SATORI_HIP_E_ARGUMENT, "Payload length must match matrix dimensions.");
        validate_ternary2(s, static_cast<const uint8_t*>(payload));
        return SATORI_HIP_OK;
    } catch (const Failure& f) {
        record_error(f.message);
        return f.status;
    }
}

// QuantizedMatrix ctor checks (src/Satori.Core/QuantizedMatrix.cs:8-13 -> QuantizedMatVec.ValidatePayload).
extern "C" int satori_hip_quantized_validate(int rows, int columns, int format, const void* payload,
                                             size_t payload_length) {
    try {
        const Shape s = quantized_shape(rows, columns, format);
        if (!payload) fail(SATORI_HIP_E_ARGUMENT_NULL, "Value cannot be null.");
        if (static_cast<int64_t>(payload_length) != s.byte_length)
            fail(SATORI_HIP_E_ARGUMENT, "Incorrect quantized payload length.");
        validate_quantized(s, static_cast<const uint8_t*>(payload));
        return SATORI_HIP_OK;
    } catch (const Failure& f) {
        record_error(f.message);
        return f.status;
    }
}

// ---- Ternary bitplane host utilities (src/Satori.Core/TernaryBitplaneMatrix.cs) ----

extern "C" int satori_hip_bitplane_validate(int rows, int columns, int block_size, const void* payload,
                                            size_t payload_length) {
    try {
        const Shape s = ternary2_shape(rows, columns, block_size);
        if (!payload) fail(SATORI_HIP_E_ARGUMENT_NULL, "Value cannot be null.");
        if (static_cast<int64_t>(payload_length) != s.byte_length)
            fail(SATORI_HIP_E_ARGUMENT, "Incorrect bitplane payload length. (Parameter 'payload')");
        validate_bitplane(s, static_cast<const uint8_t*>(payload));
        return SATORI_HIP_OK;
    } catch (const Failure& f) {
        record_error(f.message);
        return f.status;
    }
}

extern "C" int satori_hip_bitplane_from_ternary2(int rows, int columns, int block_size, const void* ternary2,
                                                 size_t ternary2_length, void* bitplane, size_t bitplane_length) {
    try {
        const Shape s = ternary2_shape(rows, columns, block_size);
        if (!ternary2 || !bitplane) fail(SATORI_HIP_E_ARGUMENT_NULL, "Value cannot be null.");
        if (static_cast<int64_t>(ternary2_length) != s.byte_length || static_cast<int64_t>(bitplane_length) != s.byte_length)
            fail(SATORI_HIP_E_ARGUMENT, "Payload length must match matrix dimensions.");
        validate_ternary2(s, static_cast<const uint8_t*>(ternary2));
        bitplane_from_ternary2(s, static_cast<const uint8_t*>(ternary2), static_cast<uint8_t*>(bitplane));
        return SATORI_HIP_OK;
    } catch (const Failure& f) {
        record_error(f.message);
        return f.status;
    }
}

extern "C" int satori_hip_bitplane_to_ternary2(int rows, int columns, int block_size, const void* bitplane,
                                               size_t bitplane_length, void* ternary2, size_t ternary2_length) {
    try {
        const Shape s = ternary2_shape(rows, columns, block_size);
        if (!ternary2 || !bitplane) fail(SATORI_HIP_E_ARGUMENT_NULL, "Value cannot be null.");
        if (static_cast<int64_t>(ternary2_length) != s.byte_length || static_cast<int64_t>(bitplane_length) != s.byte_length)
            fail(SATORI_HIP_E_ARGUMENT, "Payload length must match matrix dimensions.");
        validate_bitplane(s, static_cast<const uint8_t*>(bitplane));
        bitplane_to_ternary2(s, static_cast<const uint8_t*>(bitplane), static_cast<uint8_t*>(ternary2));
        return SATORI_HIP_OK;
    } catch (const Failure& f) {
        record_error(f.message);
        return f.status;
    }
}
