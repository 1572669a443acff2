// Host-side shape and payload rules of the reference, restated in C++ for the library's own use
// (validation before upload). Failures throw satori::Failure carrying the status that maps to the
// exception the reference throws.
#pragma once

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>

#include "../../include/satori_hip.h"

namespace satori {

struct Failure {
    int status;
    std::string message;
};

[[noreturn]] inline void fail(int status, std::string message) { throw Failure{status, std::move(message)}; }

// Sets the calling thread's satori_hip_last_error() message (defined with the runtime).
void record_error(const std::string& message);

inline float f32_at(const uint8_t* p) {
    float f;
    std::memcpy(&f, p, 4);
    return f;
}

inline uint16_t u16_at(const uint8_t* p) { return static_cast<uint16_t>(p[0] | (p[1] << 8)); }

// binary16 -> binary32 (System.Half conversion), exact.
inline float half_to_float(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h >> 15) << 31;
    uint32_t exponent = (h >> 10) & 0x1F, mantissa = h & 0x3FF, bits;
    if (exponent == 0x1F) {
        bits = sign | 0x7F800000u | (mantissa << 13);
    } else if (exponent != 0) {
        bits = sign | ((exponent + 112) << 23) | (mantissa << 13);
    } else if (mantissa == 0) {
        bits = sign;
    } else {
        int shift = 0;
        while ((mantissa & 0x400) == 0) {
            mantissa <<= 1;
            ++shift;
        }
        bits = sign | (static_cast<uint32_t>(113 - shift) << 23) | ((mantissa & 0x3FF) << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// Geometry of one matrix.
struct Shape {
    int format = 0;      // satori_hip_format
    int rows = 0;
    int columns = 0;
    int block_size = 0;  // Ternary2 B, else block elements
    int block_bytes = 0;
    int blocks = 0;      // blocks per row
    int64_t row_bytes = 0;
    int64_t byte_length = 0;
};

// Ternary2Shape (src/Satori.Core/Ternary2Shape.cs:5-22).
inline Shape ternary2_shape(int rows, int columns, int block_size) {
    if (rows <= 0) fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "rows must be positive.");
    if (columns <= 0) fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "columns must be positive.");
    if (block_size != 64 && block_size != 128 && block_size != 256)
        fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "Supported block sizes: 64, 128, 256.");
    Shape s;
    s.format = SATORI_HIP_TERNARY2;
    s.rows = rows;
    s.columns = columns;
    s.block_size = block_size;
    s.block_bytes = 4 + block_size / 4;
    s.blocks = static_cast<int>((static_cast<int64_t>(columns) + block_size - 1) / block_size);
    s.row_bytes = static_cast<int64_t>(s.blocks) * s.block_bytes;
    s.byte_length = static_cast<int64_t>(rows) * s.row_bytes;
    if (s.byte_length > INT32_MAX) fail(SATORI_HIP_E_OVERFLOW, "Arithmetic operation resulted in an overflow.");
    return s;
}

// Ternary bitplane blocks (src/Satori.Core/TernaryBitplaneMatrix.cs): the FP32 scale, then B/8 bytes of
// positive-plane bits and B/8 bytes of negative-plane bits (bit i % 8 of byte i / 8 is weight i). Same shape
// and byte length as Ternary2.

// TernaryBitplaneMatrix.Validate (TernaryBitplaneMatrix.cs:64-85).
inline void validate_bitplane(const Shape& s, const uint8_t* data) {
    const int plane = s.block_size / 8;
    for (int row = 0; row < s.rows; ++row)
        for (int block = 0; block < s.blocks; ++block) {
            const uint8_t* bytes = data + row * s.row_bytes + static_cast<int64_t>(block) * s.block_bytes;
            float scale;
            std::memcpy(&scale, bytes, 4);
            uint32_t bits;
            std::memcpy(&bits, bytes, 4);
            if (!std::isfinite(scale) || scale < 0 || bits == 0x80000000u)
                fail(SATORI_HIP_E_ARGUMENT, "Invalid bitplane scale. (Parameter 'data')");
            const int count = std::min(s.block_size, s.columns - block * s.block_size);
            if (scale != 0 && count == s.block_size) {
                // A whole block with a positive scale: only a weight in both planes is invalid (planes of 8, 16
                // or 32 bytes: whole 8-byte words).
                uint64_t overlap = 0;
                for (int i = 0; i < plane; i += 8) {
                    uint64_t p, n;
                    std::memcpy(&p, bytes + 4 + i, 8);
                    std::memcpy(&n, bytes + 4 + plane + i, 8);
                    overlap |= p & n;
                }
                if (overlap)
                    fail(SATORI_HIP_E_ARGUMENT,
                         "Overlapping bits, invalid padding or noncanonical zero. (Parameter 'data')");
                continue;
            }
            for (int i = 0; i < plane; ++i) {
                const int positive = bytes[4 + i], negative = bytes[4 + plane + i];
                const int valid = std::clamp(count - i * 8, 0, 8);
                const int padding = ~((1 << valid) - 1);
                if ((positive & negative) != 0 || ((positive | negative) & padding) != 0 ||
                    (scale == 0 && (positive | negative) != 0))
                    fail(SATORI_HIP_E_ARGUMENT,
                         "Overlapping bits, invalid padding or noncanonical zero. (Parameter 'data')");
            }
        }
}

// Bit (de)interleaving of four 2-bit codes and their plane bits, a byte at a time: code i of a Ternary2
// byte is bits 2i (positive) and 2i + 1 (negative); plane bit i of a nibble is weight i.
struct CodeTables {
    uint8_t even[256];    // bits 0, 2, 4, 6 of a byte -> bits 0..3
    uint16_t spread[256]; // bits 0..7 -> bits 0, 2, ..., 14
    constexpr CodeTables() : even(), spread() {
        for (int v = 0; v < 256; ++v) {
            even[v] = static_cast<uint8_t>((v & 1) | ((v >> 1) & 2) | ((v >> 2) & 4) | ((v >> 3) & 8));
            uint16_t w = 0;
            for (int b = 0; b < 8; ++b) w = static_cast<uint16_t>(w | (((v >> b) & 1) << (2 * b)));
            spread[v] = w;
        }
    }
};
inline constexpr CodeTables kCodeTables{};
inline uint8_t even_bits(uint8_t v) { return kCodeTables.even[v]; }

// TernaryBitplaneMatrix.FromTernary2 (TernaryBitplaneMatrix.cs:19-36), on a validated Ternary2 payload:
// code 1 sets the positive plane bit, code 2 the negative one (code 3 does not occur).
inline void bitplane_from_ternary2(const Shape& s, const uint8_t* t2, uint8_t* out) {
    const int plane = s.block_size / 8;
    for (int64_t offset = 0; offset < s.byte_length; offset += s.block_bytes) {
        std::memcpy(out + offset, t2 + offset, 4);
        const uint8_t* codes = t2 + offset + 4;
        uint8_t* positive = out + offset + 4;
        uint8_t* negative = positive + plane;
        for (int j = 0; j < plane; ++j) {  // weights 8j .. 8j + 7: code bytes 2j and 2j + 1
            const uint8_t lo = codes[2 * j], hi = codes[2 * j + 1];
            positive[j] = static_cast<uint8_t>(even_bits(lo) | (even_bits(hi) << 4));
            negative[j] = static_cast<uint8_t>(even_bits(lo >> 1) | (even_bits(hi >> 1) << 4));
        }
    }
}

// TernaryBitplaneMatrix.ToTernary2 (TernaryBitplaneMatrix.cs:38-54), on a validated bitplane payload.
inline void bitplane_to_ternary2(const Shape& s, const uint8_t* tb, uint8_t* out) {
    const int plane = s.block_size / 8;
    for (int64_t offset = 0; offset < s.byte_length; offset += s.block_bytes) {
        std::memcpy(out + offset, tb + offset, 4);
        const uint8_t* positive = tb + offset + 4;
        const uint8_t* negative = positive + plane;
        uint8_t* codes = out + offset + 4;
        for (int j = 0; j < plane; ++j) {
            const uint16_t w = static_cast<uint16_t>(kCodeTables.spread[positive[j]] | (kCodeTables.spread[negative[j]] << 1));
            codes[2 * j] = static_cast<uint8_t>(w);
            codes[2 * j + 1] = static_cast<uint8_t>(w >> 8);
        }
    }
}

// QuantizedMatrixShape (src/Satori.Core/QuantizedMatrixShape.cs:5-22).
inline Shape quantized_shape(int rows, int columns, int format) {
    Shape s;
    switch (format) {
        case SATORI_HIP_Q8_0: s.block_size = 32; s.block_bytes = 34; break;
        case SATORI_HIP_Q4_0: s.block_size = 32; s.block_bytes = 18; break;
        case SATORI_HIP_Q4_K: s.block_size = 256; s.block_bytes = 144; break;
        case SATORI_HIP_Q6_K: s.block_size = 256; s.block_bytes = 210; break;
        default: fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE, "format is not a BlockQuantization value.");
    }
    if (rows <= 0 || columns <= 0 || columns % s.block_size != 0)
        fail(SATORI_HIP_E_ARGUMENT_OUT_OF_RANGE,
             "Positive dimensions and complete " + std::to_string(s.block_size) + "-weight rows required.");
    s.format = format;
    s.rows = rows;
    s.columns = columns;
    s.blocks = columns / s.block_size;
    const int64_t blocks_total = static_cast<int64_t>(rows) * s.blocks;
    if (blocks_total > INT32_MAX || blocks_total * s.block_bytes > INT32_MAX)
        fail(SATORI_HIP_E_OVERFLOW, "Arithmetic operation resulted in an overflow.");
    s.row_bytes = static_cast<int64_t>(s.blocks) * s.block_bytes;
    s.byte_length = blocks_total * s.block_bytes;
    return s;
}

// Ternary2Matrix.ValidatePayload (src/Satori.Core/Ternary2Matrix.cs:83-101).
inline void validate_ternary2(const Shape& s, const uint8_t* data) {
    const int code_bytes = s.block_size / 4;  // 16, 32 or 64: whole 8-byte words
    for (int row = 0; row < s.rows; ++row)
        for (int block = 0; block < s.blocks; ++block) {
            const uint8_t* bytes = data + row * s.row_bytes + static_cast<int64_t>(block) * s.block_bytes;
            const float scale = f32_at(bytes);
            uint32_t bits;
            std::memcpy(&bits, bytes, 4);
            if (!std::isfinite(scale) || scale < 0 || bits == 0x80000000u)
                fail(SATORI_HIP_E_ARGUMENT, "Invalid block scale.");
            const int count = std::min(s.block_size, s.columns - block * s.block_size);
            if (scale != 0 && count == s.block_size) {
                // A whole block with a positive scale: only code 3 (both bits of a field set) is invalid.
                uint64_t bad = 0;
                for (int i = 0; i < code_bytes; i += 8) {
                    uint64_t w;
                    std::memcpy(&w, bytes + 4 + i, 8);
                    bad |= w & (w >> 1) & 0x5555555555555555ull;
                }
                if (bad) fail(SATORI_HIP_E_ARGUMENT, "Invalid weight code or padding.");
                continue;
            }
            for (int i = 0; i < s.block_size; ++i) {
                const int code = (bytes[4 + i / 4] >> (2 * (i % 4))) & 3;
                if (code == 3 || ((i >= count || scale == 0) && code != 0))
                    fail(SATORI_HIP_E_ARGUMENT, "Invalid weight code or padding.");
            }
        }
}

// QuantizedMatVec.ValidatePayload (src/Satori.Core/QuantizedMatVec.cs:28-42) with the K codecs'
// AreScalesFinite (Q4KCodec.cs:91-93, Q6KCodec.cs:84-85).
inline void validate_quantized(const Shape& s, const uint8_t* data) {
    for (int64_t offset = 0; offset < s.byte_length; offset += s.block_bytes) {
        const uint8_t* block = data + offset;
        bool finite;
        if (s.format == SATORI_HIP_Q4_K)
            finite = std::isfinite(half_to_float(u16_at(block))) && std::isfinite(half_to_float(u16_at(block + 2)));
        else if (s.format == SATORI_HIP_Q6_K)
            finite = std::isfinite(half_to_float(u16_at(block + 208)));
        else
            finite = std::isfinite(half_to_float(u16_at(block)));
        if (!finite) fail(SATORI_HIP_E_INVALID_DATA, "Nonfinite block scale at " + std::to_string(offset) + ".");
    }
}

}  // namespace satori
