/*
 * CPU oracle: scalar restatement of the reference's quantized MatVec hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see satori_oracle.h). Built with -O2 -ffp-contract=off so every
 * floating-point operation is rounded exactly where the C# source rounds it.
 */
#include "satori_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* System.Half -> float conversion used by QuantizedMatVec.Scale
 * (src/Satori.Core/QuantizedMatVec.cs:369). Exact for every binary16 value. */
float or_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exponent = (h >> 10) & 0x1F;
    uint32_t mantissa = h & 0x3FF;
    uint32_t bits;
    if (exponent == 0x1F) {
        bits = sign | 0x7F800000u | (mantissa << 13);
    } else if (exponent != 0) {
        bits = sign | ((exponent + 112) << 23) | (mantissa << 13);
    } else if (mantissa == 0) {
        bits = sign;
    } else {
        /* subnormal binary16: value = mantissa * 2^-24, representable exactly in binary32 */
        int shift = 0;
        while ((mantissa & 0x400) == 0) { mantissa <<= 1; shift++; }
        mantissa &= 0x3FF;
        bits = sign | ((uint32_t)(113 - shift) << 23) | (mantissa << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static int16_t rds16(const uint8_t* p) { return (int16_t)rd16(p); }
static int32_t rd32(const uint8_t* p) { return (int32_t)((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24)); }
static int64_t rd64(const uint8_t* p) { return (int64_t)((uint64_t)(uint32_t)rd32(p) | ((uint64_t)(uint32_t)rd32(p + 4) << 32)); }
static float rdf32(const uint8_t* p) { uint32_t b = (uint32_t)rd32(p); float f; memcpy(&f, &b, 4); return f; }
static void wr32(uint8_t* p, uint32_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); p[2] = (uint8_t)(v >> 16); p[3] = (uint8_t)(v >> 24); }
static void wrf32(uint8_t* p, float f) { uint32_t b; memcpy(&b, &f, 4); wr32(p, b); }
static float half_at(const uint8_t* p) { return or_half_to_float(rd16(p)); }

/* ======================================================================================
 * Ternary2
 * ====================================================================================== */

/* Ternary2Shape ctor (src/Satori.Core/Ternary2Shape.cs:5-15): positive dims, block in {64,128,256},
 * ByteLength = checked((int)(rows * ceil(cols/B) * (4 + B/4))). Returns -code on failure. */
int64_t or_t2_byte_length(int rows, int columns, int block_size) {
    if (rows <= 0 || columns <= 0) return -OR_OUT_OF_RANGE;
    if (block_size != 64 && block_size != 128 && block_size != 256) return -OR_OUT_OF_RANGE;
    int64_t blocks = ((int64_t)columns + block_size - 1) / block_size;
    int64_t bytes = (int64_t)rows * blocks * (4 + block_size / 4);
    if (bytes > 2147483647LL) return -OR_OVERFLOW;
    return bytes;
}

/* Ternary2Matrix.Quantize (src/Satori.Core/Ternary2Matrix.cs:38-71). */
int or_t2_quantize(const float* weights, int rows, int columns, int block_size, uint8_t* out, size_t out_len) {
    int64_t length = or_t2_byte_length(rows, columns, block_size);
    if (length < 0) return (int)-length;
    if ((int64_t)out_len != length) return OR_ARGUMENT;
    int64_t count_all = (int64_t)rows * columns;
    for (int64_t i = 0; i < count_all; i++)
        if (!isfinite(weights[i])) return OR_ARGUMENT; /* :43-45 */
    memset(out, 0, (size_t)length);
    int blocks = (int)(((int64_t)columns + block_size - 1) / block_size);
    int stride = 4 + block_size / 4;
    for (int row = 0; row < rows; row++)
        for (int block = 0; block < blocks; block++) {
            int column = block * block_size;
            int count = block_size < columns - column ? block_size : columns - column;
            const float* source = weights + (int64_t)row * columns + column;
            double magnitude = 0; /* :55-57, FP64 accumulation in order */
            for (int i = 0; i < count; i++) magnitude += fabs((double)source[i]);
            float scale = (float)(magnitude / count); /* :58 */
            uint8_t* target = out + ((int64_t)row * blocks + block) * stride;
            wrf32(target, scale);
            if (scale == 0) continue; /* :61-62 */
            double threshold = (double)scale / 2; /* :63 */
            for (int i = 0; i < count; i++) {
                int code = (double)source[i] > threshold ? 1 : (double)source[i] < -threshold ? 2 : 0; /* :66 */
                target[4 + i / 4] |= (uint8_t)(code << (2 * (i % 4))); /* :67 */
            }
        }
    return OR_OK;
}

/* Ternary2Matrix.ValidatePayload (src/Satori.Core/Ternary2Matrix.cs:83-101) + the length check of
 * FromPacked (:75-76). */
int or_t2_validate(const uint8_t* data, size_t len, int rows, int columns, int block_size) {
    int64_t length = or_t2_byte_length(rows, columns, block_size);
    if (length < 0) return (int)-length;
    if ((int64_t)len != length) return OR_ARGUMENT;
    int blocks = (int)(((int64_t)columns + block_size - 1) / block_size);
    int stride = 4 + block_size / 4;
    for (int row = 0; row < rows; row++)
        for (int block = 0; block < blocks; block++) {
            const uint8_t* bytes = data + ((int64_t)row * blocks + block) * stride;
            float scale = rdf32(bytes);
            uint32_t bits = (uint32_t)rd32(bytes);
            if (!isfinite(scale) || scale < 0 || bits == 0x80000000u) return OR_ARGUMENT; /* :91-92 */
            int count = block_size < columns - block * block_size ? block_size : columns - block * block_size;
            for (int i = 0; i < block_size; i++) {
                int code = (bytes[4 + i / 4] >> (2 * (i % 4))) & 3;
                if (code == 3 || ((i >= count || scale == 0) && code != 0)) return OR_ARGUMENT; /* :97-98 */
            }
        }
    return OR_OK;
}

/* TernaryBitplaneMatrix.Validate (src/Satori.Core/TernaryBitplaneMatrix.cs:64-85): scale finite, >= 0 and
 * not -0; no weight in both planes; no bit past the last column; no bit in a zero-scale block. */
int or_tb_validate(const uint8_t* data, size_t len, int rows, int columns, int block_size) {
    int64_t length = or_t2_byte_length(rows, columns, block_size);
    if (length < 0) return (int)-length;
    if ((int64_t)len != length) return OR_ARGUMENT;
    int blocks = (int)(((int64_t)columns + block_size - 1) / block_size);
    int stride = 4 + block_size / 4, plane = block_size / 8;
    for (int row = 0; row < rows; row++)
        for (int block = 0; block < blocks; block++) {
            const uint8_t* bytes = data + ((int64_t)row * blocks + block) * stride;
            float scale = rdf32(bytes);
            uint32_t bits = (uint32_t)rd32(bytes);
            if (!isfinite(scale) || scale < 0 || bits == 0x80000000u) return OR_ARGUMENT;
            int count = block_size < columns - block * block_size ? block_size : columns - block * block_size;
            for (int i = 0; i < plane; i++) {
                int positive = bytes[4 + i], negative = bytes[4 + plane + i];
                int valid = count - i * 8;
                valid = valid < 0 ? 0 : valid > 8 ? 8 : valid;
                int padding = ~((1 << valid) - 1);
                if ((positive & negative) != 0 || ((positive | negative) & padding) != 0 ||
                    (scale == 0 && (positive | negative) != 0))
                    return OR_ARGUMENT;
            }
        }
    return OR_OK;
}

/* TernaryBitplaneMatrix.FromTernary2 (TernaryBitplaneMatrix.cs:19-36): code 1 sets the positive bit, code 2
 * the negative bit. */
void or_tb_from_t2(const uint8_t* t2, int rows, int columns, int block_size, uint8_t* out) {
    int64_t length = or_t2_byte_length(rows, columns, block_size);
    int stride = 4 + block_size / 4, plane = block_size / 8;
    memset(out, 0, (size_t)length);
    for (int64_t offset = 0; offset < length; offset += stride) {
        memcpy(out + offset, t2 + offset, 4);
        for (int i = 0; i < block_size; i++) {
            int code = (t2[offset + 4 + i / 4] >> (2 * (i % 4))) & 3;
            if (code != 0) out[offset + 4 + (code == 2 ? plane : 0) + i / 8] |= (uint8_t)(1 << (i % 8));
        }
    }
}

/* TernaryBitplaneMatrix.ToTernary2 (TernaryBitplaneMatrix.cs:38-54). */
void or_tb_to_t2(const uint8_t* tb, int rows, int columns, int block_size, uint8_t* out) {
    int64_t length = or_t2_byte_length(rows, columns, block_size);
    int stride = 4 + block_size / 4, plane = block_size / 8;
    memset(out, 0, (size_t)length);
    for (int64_t offset = 0; offset < length; offset += stride) {
        memcpy(out + offset, tb + offset, 4);
        for (int i = 0; i < block_size; i++) {
            int positive = (tb[offset + 4 + i / 8] >> (i % 8)) & 1;
            int negative = (tb[offset + 4 + plane + i / 8] >> (i % 8)) & 1;
            out[offset + 4 + i / 4] |= (uint8_t)((positive | negative << 1) << (2 * (i % 4)));
        }
    }
}

/* TernaryBitplaneMatVec.ExecuteScalar (src/Satori.Core/TernaryBitplaneMatVec.cs:24-46): per block a sequential
 * FP32 sum of +x (positive bit) or -x (negative bit), then total += scale * sum. */
void or_tb_matvec_scalar(const uint8_t* data, int rows, int columns, int block_size, const float* x, float* y) {
    int blocks = (int)(((int64_t)columns + block_size - 1) / block_size);
    int stride = 4 + block_size / 4, plane = block_size / 8;
    for (int row = 0; row < rows; row++) {
        float total = 0;
        for (int block = 0; block < blocks; block++) {
            const uint8_t* bytes = data + ((int64_t)row * blocks + block) * stride;
            int column = block * block_size;
            int count = block_size < columns - column ? block_size : columns - column;
            float sum = 0;
            for (int i = 0; i < count; i++) {
                int mask = 1 << (i % 8);
                if (bytes[4 + i / 8] & mask) sum += x[column + i];
                else if (bytes[4 + plane + i / 8] & mask) sum -= x[column + i];
            }
            total += rdf32(bytes) * sum;
        }
        y[row] = total;
    }
}

/* Ternary2Matrix.Dequantize (src/Satori.Core/Ternary2Matrix.cs:103-120). */
void or_t2_dequantize(const uint8_t* data, int rows, int columns, int block_size, float* out) {
    int blocks = (int)(((int64_t)columns + block_size - 1) / block_size);
    int stride = 4 + block_size / 4;
    for (int row = 0; row < rows; row++)
        for (int block = 0; block < blocks; block++) {
            const uint8_t* bytes = data + ((int64_t)row * blocks + block) * stride;
            float scale = rdf32(bytes);
            int column = block * block_size;
            int count = block_size < columns - column ? block_size : columns - column;
            for (int i = 0; i < count; i++) {
                int code = (bytes[4 + i / 4] >> (2 * (i % 4))) & 3;
                out[(int64_t)row * columns + column + i] = code == 1 ? scale : code == 2 ? -scale : 0;
            }
        }
}

/* Ternary2MatVec.ExecuteScalarCore (src/Satori.Core/Ternary2MatVec.cs:52-76): the scalar reference. */
void or_t2_matvec_scalar(const uint8_t* data, int rows, int columns, int block_size, const float* x, float* y) {
    int blocks = (int)(((int64_t)columns + block_size - 1) / block_size);
    int stride = 4 + block_size / 4;
    for (int row = 0; row < rows; row++) {
        float sum = 0;
        for (int block = 0; block < blocks; block++) {
            const uint8_t* bytes = data + ((int64_t)row * blocks + block) * stride;
            float scale = rdf32(bytes);
            int column = block * block_size;
            int count = block_size < columns - column ? block_size : columns - column;
            float partial = 0;
            for (int i = 0; i < count; i++) {
                int code = (bytes[4 + i / 4] >> (2 * (i % 4))) & 3;
                if (code == 1) partial += x[column + i];
                else if (code == 2) partial -= x[column + i];
            }
            sum += partial * scale;
        }
        y[row] = sum;
    }
}

/* Ternary2FileFormat.WriteHeader (src/Satori.Core/Ternary2FileFormat.cs:9-19). */
void or_stq2_write_header(uint8_t header[32], int rows, int columns, int block_size) {
    memset(header, 0, 32);
    memcpy(header, "STQ2", 4);
    header[4] = 1; header[5] = 0;
    header[6] = 32; header[7] = 0;
    wr32(header + 8, (uint32_t)rows);
    wr32(header + 12, (uint32_t)columns);
    wr32(header + 16, (uint32_t)block_size);
    int64_t bytes = or_t2_byte_length(rows, columns, block_size);
    wr32(header + 24, (uint32_t)(uint64_t)bytes);
    wr32(header + 28, (uint32_t)((uint64_t)bytes >> 32));
}

/* Ternary2FileFormat.ReadHeader (src/Satori.Core/Ternary2FileFormat.cs:21-35), with the shape
 * failures mapped to InvalidDataException as MappedTernary2Matrix does (MappedTernary2Matrix.cs:25-28). */
int or_stq2_read_header(const uint8_t header[32], int* rows, int* columns, int* block_size) {
    if (memcmp(header, "STQ2", 4) != 0 || rd16(header + 4) != 1 || rd16(header + 6) != 32 || rd32(header + 20) != 0)
        return OR_INVALID_DATA;
    int r = rd32(header + 8), c = rd32(header + 12), b = rd32(header + 16);
    int64_t length = or_t2_byte_length(r, c, b);
    if (length < 0) return OR_INVALID_DATA;
    if (rd64(header + 24) != length) return OR_INVALID_DATA;
    *rows = r; *columns = c; *block_size = b;
    return OR_OK;
}

/* ======================================================================================
 * GGUF block formats
 * ====================================================================================== */

static int q_geometry(int format, int* elements, int* bytes) {
    switch (format) { /* QuantizedMatrixShape ctor (src/Satori.Core/QuantizedMatrixShape.cs:7-14) */
        case OR_Q8_0: *elements = 32; *bytes = 34; return 1;
        case OR_Q4_0: *elements = 32; *bytes = 18; return 1;
        case OR_Q4_K: *elements = 256; *bytes = 144; return 1;
        case OR_Q6_K: *elements = 256; *bytes = 210; return 1;
        default: return 0;
    }
}

/* QuantizedMatrixShape (src/Satori.Core/QuantizedMatrixShape.cs:5-22). */
int64_t or_q_byte_length(int rows, int columns, int format) {
    int e = 0, b = 0;
    if (!q_geometry(format, &e, &b)) return -OR_OUT_OF_RANGE;
    if (rows <= 0 || columns <= 0 || columns % e != 0) return -OR_OUT_OF_RANGE;
    int64_t bytes = (int64_t)rows * (columns / e);
    if (bytes > 2147483647LL) return -OR_OVERFLOW; /* checked(rows * (columns/E)) */
    bytes *= b;
    if (bytes > 2147483647LL) return -OR_OVERFLOW; /* checked(... * BlockBytes) */
    return bytes;
}

/* QuantizedMatVec.ValidatePayload (src/Satori.Core/QuantizedMatVec.cs:28-42) with
 * Q4KCodec.AreScalesFinite (Q4KCodec.cs:91-93) and Q6KCodec.AreScalesFinite (Q6KCodec.cs:84-85). */
int or_q_validate(const uint8_t* data, size_t len, int rows, int columns, int format) {
    int64_t length = or_q_byte_length(rows, columns, format);
    if (length < 0) return (int)-length;
    if ((int64_t)len != length) return OR_ARGUMENT;
    int e = 0, b = 0;
    q_geometry(format, &e, &b);
    for (int64_t offset = 0; offset < length; offset += b) {
        const uint8_t* block = data + offset;
        int finite;
        if (format == OR_Q4_K) finite = isfinite(half_at(block)) && isfinite(half_at(block + 2));
        else if (format == OR_Q6_K) finite = isfinite(half_at(block + 208));
        else finite = isfinite(half_at(block));
        if (!finite) return OR_INVALID_DATA;
    }
    return OR_OK;
}

/* Q4KCodec.GetScaleMin (src/Satori.Core/Q4KCodec.cs:24-36). */
void or_q4k_get_scale_min(int j, const uint8_t* scales, int* scale, int* min) {
    if (j < 4) {
        *scale = scales[j] & 63;
        *min = scales[j + 4] & 63;
    } else {
        *scale = (scales[j + 4] & 0xF) | ((scales[j - 4] >> 6) << 4);
        *min = (scales[j + 4] >> 4) | ((scales[j] >> 6) << 4);
    }
}

/* Q4KCodec.DotBlock (src/Satori.Core/Q4KCodec.cs:39-65). */
float or_q4k_dot_block(const uint8_t* block, const float* input) {
    float d = half_at(block), dmin = half_at(block + 2);
    const uint8_t* scales = block + 4;
    const uint8_t* quants = block + 16;
    float total = 0;
    for (int group = 0; group < 4; group++) {
        const uint8_t* qs = quants + group * 32;
        const float* low = input + group * 64;
        const float* high = input + group * 64 + 32;
        int s0, n0, s1, n1;
        or_q4k_get_scale_min(group * 2, scales, &s0, &n0);
        or_q4k_get_scale_min(group * 2 + 1, scales, &s1, &n1);
        float dl = d * (float)s0, ml = dmin * (float)n0, dh = d * (float)s1, mh = dmin * (float)n1;
        float acc_low = 0, acc_high = 0;
        for (int l = 0; l < 32; l++) {
            acc_low += (dl * (float)(qs[l] & 0xF) - ml) * low[l];
            acc_high += (dh * (float)(qs[l] >> 4) - mh) * high[l];
        }
        total += acc_low + acc_high;
    }
    return total;
}

/* Q4KCodec.DecodeBlock (src/Satori.Core/Q4KCodec.cs:68-88). */
void or_q4k_decode_block(const uint8_t* block, float* weights) {
    float d = half_at(block), dmin = half_at(block + 2);
    const uint8_t* scales = block + 4;
    const uint8_t* quants = block + 16;
    for (int group = 0; group < 4; group++) {
        const uint8_t* qs = quants + group * 32;
        int s0, n0, s1, n1;
        or_q4k_get_scale_min(group * 2, scales, &s0, &n0);
        or_q4k_get_scale_min(group * 2 + 1, scales, &s1, &n1);
        float dl = d * (float)s0, ml = dmin * (float)n0, dh = d * (float)s1, mh = dmin * (float)n1;
        for (int l = 0; l < 32; l++) {
            weights[group * 64 + l] = dl * (float)(qs[l] & 0xF) - ml;
            weights[group * 64 + 32 + l] = dh * (float)(qs[l] >> 4) - mh;
        }
    }
}

/* Q8KCodec accessors (src/Satori.Core/Q8KCodec.cs:79, 104-112). */
static float q8k_scale(const uint8_t* activation) { return rdf32(activation); }
static int q8k_is_zero(const uint8_t* activation) { return q8k_scale(activation) == 0; }
static const int8_t* q8k_codes(const uint8_t* activation) { return (const int8_t*)(activation + 4); }
static int16_t q8k_sum(const uint8_t* activation, int g) { return rds16(activation + 260 + 2 * g); }

/* Q4KCodec.DotProduct (src/Satori.Core/Q4KCodec.cs:117-137). */
int32_t or_q4k_dot_product(const uint8_t* block, const uint8_t* activation) {
    const int8_t* codes = q8k_codes(activation);
    const uint8_t* scales = block + 4;
    const uint8_t* quants = block + 16;
    int32_t total = 0;
    for (int group = 0; group < 4; group++) {
        const uint8_t* qs = quants + group * 32;
        int low_scale, high_scale, unused;
        or_q4k_get_scale_min(group * 2, scales, &low_scale, &unused);
        or_q4k_get_scale_min(group * 2 + 1, scales, &high_scale, &unused);
        int32_t low = 0, high = 0;
        for (int l = 0; l < 32; l++) {
            low += (qs[l] & 0xF) * codes[group * 64 + l];
            high += (qs[l] >> 4) * codes[group * 64 + 32 + l];
        }
        total += low_scale * low + high_scale * high;
    }
    return total;
}

/* Q4KCodec.MinProduct (src/Satori.Core/Q4KCodec.cs:140-153). */
int32_t or_q4k_min_product(const uint8_t* block, const uint8_t* activation) {
    const uint8_t* scales = block + 4;
    int32_t total = 0;
    for (int group = 0; group < 4; group++) {
        int unused, low_min, high_min;
        or_q4k_get_scale_min(group * 2, scales, &unused, &low_min);
        or_q4k_get_scale_min(group * 2 + 1, scales, &unused, &high_min);
        total += low_min * (q8k_sum(activation, group * 4) + q8k_sum(activation, group * 4 + 1));
        total += high_min * (q8k_sum(activation, group * 4 + 2) + q8k_sum(activation, group * 4 + 3));
    }
    return total;
}

/* Q4KCodec.DotBlockQuantized (src/Satori.Core/Q4KCodec.cs:105-114). */
float or_q4k_dot_block_quantized(const uint8_t* block, const uint8_t* activation) {
    if (q8k_is_zero(activation)) return 0;
    float activation_scale = q8k_scale(activation);
    float d = activation_scale * half_at(block);
    float dmin = activation_scale * half_at(block + 2);
    return d * (float)or_q4k_dot_product(block, activation) - dmin * (float)or_q4k_min_product(block, activation);
}

/* Q6K code of weight (h, l, k): the decoder's index expressions (src/Satori.Core/Q6KCodec.cs:70-74). */
static void q6k_codes(const uint8_t* lql, const uint8_t* lqh, int l, int q[4]) {
    q[0] = ((lql[l] & 0xF) | (((lqh[l] >> 0) & 3) << 4)) - 32;
    q[1] = ((lql[l + 32] & 0xF) | (((lqh[l] >> 2) & 3) << 4)) - 32;
    q[2] = ((lql[l] >> 4) | (((lqh[l] >> 4) & 3) << 4)) - 32;
    q[3] = ((lql[l + 32] >> 4) | (((lqh[l] >> 6) & 3) << 4)) - 32;
}

/* Q6KCodec.DotBlock (src/Satori.Core/Q6KCodec.cs:22-51). */
float or_q6k_dot_block(const uint8_t* block, const float* input) {
    float d = half_at(block + 208);
    const uint8_t* ql = block;
    const uint8_t* qh = block + 128;
    const int8_t* scales = (const int8_t*)(block + 192);
    float total = 0;
    for (int half = 0; half < 2; half++) {
        const uint8_t* lql = ql + half * 64;
        const uint8_t* lqh = qh + half * 32;
        const int8_t* lsc = scales + half * 8;
        int base = half * 128;
        for (int l = 0; l < 32; l++) {
            int sub = l / 16, q[4];
            q6k_codes(lql, lqh, l, q);
            total += d * (float)lsc[sub + 0] * (float)q[0] * input[base + l + 0];
            total += d * (float)lsc[sub + 2] * (float)q[1] * input[base + l + 32];
            total += d * (float)lsc[sub + 4] * (float)q[2] * input[base + l + 64];
            total += d * (float)lsc[sub + 6] * (float)q[3] * input[base + l + 96];
        }
    }
    return total;
}

/* Q6KCodec.DecodeBlock (src/Satori.Core/Q6KCodec.cs:54-81). */
void or_q6k_decode_block(const uint8_t* block, float* weights) {
    float d = half_at(block + 208);
    const uint8_t* ql = block;
    const uint8_t* qh = block + 128;
    const int8_t* scales = (const int8_t*)(block + 192);
    for (int half = 0; half < 2; half++) {
        const uint8_t* lql = ql + half * 64;
        const uint8_t* lqh = qh + half * 32;
        const int8_t* lsc = scales + half * 8;
        int base = half * 128;
        for (int l = 0; l < 32; l++) {
            int sub = l / 16, q[4];
            q6k_codes(lql, lqh, l, q);
            weights[base + l + 0] = d * (float)lsc[sub + 0] * (float)q[0];
            weights[base + l + 32] = d * (float)lsc[sub + 2] * (float)q[1];
            weights[base + l + 64] = d * (float)lsc[sub + 4] * (float)q[2];
            weights[base + l + 96] = d * (float)lsc[sub + 6] * (float)q[3];
        }
    }
}

/* Q6KCodec.DotProduct (src/Satori.Core/Q6KCodec.cs:114-146). */
int32_t or_q6k_dot_product(const uint8_t* block, const uint8_t* activation) {
    const int8_t* codes = q8k_codes(activation);
    const uint8_t* ql = block;
    const uint8_t* qh = block + 128;
    const int8_t* scales = (const int8_t*)(block + 192);
    int32_t total = 0;
    for (int half = 0; half < 2; half++) {
        const uint8_t* lql = ql + half * 64;
        const uint8_t* lqh = qh + half * 32;
        const int8_t* lsc = scales + half * 8;
        int base = half * 128;
        for (int l = 0; l < 32; l++) {
            int sub = l / 16, q[4];
            q6k_codes(lql, lqh, l, q);
            total += lsc[sub + 0] * q[0] * codes[base + l + 0];
            total += lsc[sub + 2] * q[1] * codes[base + l + 32];
            total += lsc[sub + 4] * q[2] * codes[base + l + 64];
            total += lsc[sub + 6] * q[3] * codes[base + l + 96];
        }
    }
    return total;
}

/* Q6KCodec.DotBlockQuantized (src/Satori.Core/Q6KCodec.cs:99-107). */
float or_q6k_dot_block_quantized(const uint8_t* block, const uint8_t* activation) {
    if (q8k_is_zero(activation)) return 0;
    float d = q8k_scale(activation) * half_at(block + 208);
    return d * (float)or_q6k_dot_product(block, activation);
}

/* Q8KCodec.NearestInteger (src/Satori.Core/Q8KCodec.cs:120-125). */
static int q8k_nearest_integer(float value) {
    volatile float shifted = value + 12582912.0f; /* one rounded single-precision add */
    float s = shifted;
    uint32_t bits;
    memcpy(&bits, &s, 4);
    return (int)(bits & 0x007fffff) - 0x00400000;
}

/* Q8KCodec.QuantizeBlock (src/Satori.Core/Q8KCodec.cs:44-76). */
void or_q8k_quantize_block(const float* input, uint8_t* block) {
    float max = 0, magnitude = 0;
    for (int j = 0; j < 256; j++) {
        float value = input[j];
        float absolute = fabsf(value);
        if (absolute > magnitude) { magnitude = absolute; max = value; }
    }
    if (magnitude == 0) { memset(block, 0, 292); return; }
    volatile float inverse_v = -127.0f / max;
    float inverse = inverse_v;
    int8_t* codes = (int8_t*)(block + 4);
    for (int j = 0; j < 256; j++) {
        volatile float product = inverse * input[j]; /* rounded product, then the add inside */
        int n = q8k_nearest_integer(product);
        codes[j] = (int8_t)(n < 127 ? n : 127); /* (sbyte)Math.Min(127, ...), unchecked */
    }
    for (int group = 0; group < 16; group++) {
        int total = 0;
        for (int j = 0; j < 16; j++) total += codes[group * 16 + j];
        int16_t s = (int16_t)total;
        block[260 + 2 * group] = (uint8_t)(uint16_t)s;
        block[261 + 2 * group] = (uint8_t)((uint16_t)s >> 8);
    }
    wrf32(block, 1.0f / inverse);
}

/* Q8KCodec.QuantizeRow (src/Satori.Core/Q8KCodec.cs:85-93). */
int or_q8k_quantize_row(const float* input, int columns, uint8_t* output, size_t out_len) {
    if (columns < 0 || columns % 256 != 0) return OR_ARGUMENT;
    int blocks = columns / 256;
    if ((int64_t)out_len != (int64_t)blocks * 292) return OR_ARGUMENT;
    for (int block = 0; block < blocks; block++) or_q8k_quantize_block(input + block * 256, output + block * 292);
    return OR_OK;
}

/* QuantizedRow.DecodeBlock (src/Satori.Core/QuantizedRow.cs:20-54). */
void or_q_decode_block(const uint8_t* block, int format, float* out) {
    switch (format) {
        case OR_Q8_0: {
            float scale = half_at(block); /* QuantizedRow.cs:23-24 */
            for (int j = 0; j < 32; j++) out[j] = scale * (float)(int8_t)block[2 + j];
            break;
        }
        case OR_Q4_0: {
            float scale = half_at(block); /* QuantizedRow.cs:31-36 */
            for (int j = 0; j < 16; j++) {
                out[j] = scale * (float)((block[2 + j] & 15) - 8);
                out[j + 16] = scale * (float)((block[2 + j] >> 4) - 8);
            }
            break;
        }
        case OR_Q4_K: or_q4k_decode_block(block, out); break;
        case OR_Q6_K: or_q6k_decode_block(block, out); break;
    }
}

/* QuantizedMatVec.ExecuteScalar (src/Satori.Core/QuantizedMatVec.cs:45-78): the scalar reference
 * for every format with FP32 activations. */
void or_q_matvec_scalar(const uint8_t* data, int rows, int columns, int format, const float* input, float* output) {
    int e = 0, b = 0;
    q_geometry(format, &e, &b);
    int blocks = columns / e;
    for (int row = 0; row < rows; row++) {
        float total = 0;
        for (int column = 0; column < columns; column += e) {
            const uint8_t* block = data + ((int64_t)row * blocks + column / e) * b;
            if (format == OR_Q4_K) { total += or_q4k_dot_block(block, input + column); continue; }
            if (format == OR_Q6_K) { total += or_q6k_dot_block(block, input + column); continue; }
            float sum = 0;
            if (format == OR_Q8_0) {
                for (int j = 0; j < 32; j++) sum += (float)(int8_t)block[2 + j] * input[column + j];
            } else {
                for (int j = 0; j < 16; j++) sum += (float)((block[2 + j] & 15) - 8) * input[column + j];
                for (int j = 0; j < 16; j++) sum += (float)((block[2 + j] >> 4) - 8) * input[column + 16 + j];
            }
            total += half_at(block) * sum;
        }
        output[row] = total;
    }
}

/* Eight-lane vector sum as QuantizedKAvx2Kernel.HorizontalSum (QuantizedKAvx2Kernel.cs:341-347):
 * h[k] = a[k] + a[k+4]; then (h0 + h2) + (h1 + h3). */
static float hsum8(const float a[8]) {
    float h0 = a[0] + a[4], h1 = a[1] + a[5], h2 = a[2] + a[6], h3 = a[3] + a[7];
    float g0 = h0 + h2, g1 = h1 + h3;
    return g0 + g1;
}

/* QuantizedMatVec.Dot with FMA (src/Satori.Core/QuantizedMatVec.cs:350-365): eight FMA lanes, the
 * horizontal sum, then the scalar tail. */
static float fma_dot(const float* weights, const float* input, int length) {
    float lanes[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int j = 0;
    for (; j + 8 <= length; j += 8)
        for (int k = 0; k < 8; k++) lanes[k] = fmaf(weights[j + k], input[j + k], lanes[k]);
    float total = hsum8(lanes);
    for (; j < length; j++) total += weights[j] * input[j];
    return total;
}

/* QuantizedMatVec.ExecuteBatch (src/Satori.Core/QuantizedMatVec.cs:104-120) on an AVX2 host:
 * K formats -> ExecuteBatchQuantized (:136-219) -> QuantizedKAvx2Kernel.ExecuteQuantizedTiled
 * (QuantizedKAvx2Kernel.cs:47-99); Q8_0/Q4_0 -> ExecuteBatchFloat -> ExecuteBatchRows (:308-347).
 * The row split does not change the result (:93-94), so rows run in order here. */
int or_q_matvec_batch(const uint8_t* data, int rows, int columns, int format, const float* input, int positions,
                      float* output) {
    int e = 0, b = 0;
    if (!q_geometry(format, &e, &b)) return OR_OUT_OF_RANGE;
    if (positions <= 0) return OR_OUT_OF_RANGE;
    int blocks = columns / e;
    if (format == OR_Q4_K || format == OR_Q6_K) {
        if (positions > 256) return OR_OUT_OF_RANGE; /* QuantizedKAvx2Kernel.cs:50-51 */
        int row_bytes = blocks * 292;
        uint8_t* quantized = (uint8_t*)malloc((size_t)positions * row_bytes);
        if (!quantized) return OR_ARGUMENT;
        for (int p = 0; p < positions; p++)
            or_q8k_quantize_row(input + (int64_t)p * columns, columns, quantized + (int64_t)p * row_bytes, row_bytes);
        int q4 = format == OR_Q4_K;
        for (int row = 0; row < rows; row++) {
            for (int p = 0; p < positions; p++) {
                float acc = 0;
                for (int block = 0; block < blocks; block++) {
                    const uint8_t* w = data + ((int64_t)row * blocks + block) * b;
                    const uint8_t* a = quantized + (int64_t)p * row_bytes + (int64_t)block * 292;
                    if (q8k_is_zero(a)) continue;
                    float as = q8k_scale(a);
                    if (q4) {
                        float d = half_at(w) * as, dmin = half_at(w + 2) * as;
                        acc += d * (float)or_q4k_dot_product(w, a) - dmin * (float)or_q4k_min_product(w, a);
                    } else {
                        float d = half_at(w + 208);
                        acc += as * d * (float)or_q6k_dot_product(w, a);
                    }
                }
                output[(int64_t)p * rows + row] = acc;
            }
        }
        free(quantized);
        return OR_OK;
    }
    float weights[32];
    for (int row = 0; row < rows; row++)
        for (int p = 0; p < positions; p++) {
            float acc = 0;
            for (int block = 0; block < blocks; block++) {
                or_q_decode_block(data + ((int64_t)row * blocks + block) * b, format, weights);
                acc += fma_dot(weights, input + (int64_t)p * columns + block * e, e);
            }
            output[(int64_t)p * rows + row] = acc;
        }
    return OR_OK;
}

/* NumericalCorpus.RandomMatrix (validation/Satori.Validation/NumericalCorpus.cs:8-16, 41-47): xorshift32
 * from seed 1729 with the fixed 24-bit conversion; weights are drawn first, then the input. */
static float corpus_next(uint32_t* state) {
    *state ^= *state << 13;
    *state ^= *state >> 17;
    *state ^= *state << 5;
    return (float)(*state >> 8) * (1.0f / 8388608.0f) - 1.0f;
}

void or_corpus_random_matrix(int rows, int columns, float* weights, float* input) {
    uint32_t state = 1729;
    int64_t n = (int64_t)rows * columns;
    for (int64_t i = 0; i < n; i++) weights[i] = corpus_next(&state) * 2;
    for (int i = 0; i < columns; i++) input[i] = corpus_next(&state);
}

/* ---- TransformerOps (src/Satori.Core/TransformerOps.cs) ---- */

/* RmsNorm (TransformerOps.cs:13-21). */
void or_rms_norm(const float* input, const float* weights, float epsilon, int length, float* output) {
    double sum = 0;
    for (int i = 0; i < length; i++) sum += (double)input[i] * input[i];
    double scale = 1 / sqrt(sum / length + epsilon);
    for (int i = 0; i < length; i++) output[i] = (float)(input[i] * scale * weights[i]);
}

/* RmsNormHeads (TransformerOps.cs:117-130). */
void or_rms_norm_heads(float* vector, const float* weights, float epsilon, int head_dim, int length) {
    for (int start = 0; start < length; start += head_dim) {
        double sum = 0;
        for (int i = 0; i < head_dim; i++) sum += (double)vector[start + i] * vector[start + i];
        double scale = 1 / sqrt(sum / head_dim + epsilon);
        for (int i = 0; i < head_dim; i++) vector[start + i] = (float)(vector[start + i] * scale * weights[i]);
    }
}

/* Rope (TransformerOps.cs:23-38): interleaved pairs (j, j + 1). */
void or_rope(float* vector, int length, int head_dim, int position) {
    for (int j = 0; j < head_dim; j += 2) {
        double angle = position / pow(10000, (double)j / head_dim);
        double sn = sin(angle), cs = cos(angle);
        for (int start = 0; start < length; start += head_dim) {
            double x = vector[start + j], y = vector[start + j + 1];
            vector[start + j] = (float)(x * cs - y * sn);
            vector[start + j + 1] = (float)(x * sn + y * cs);
        }
    }
}

/* RopeHalf (TransformerOps.cs:94-114): pairs (k, k + half) of the first `rotary` lanes of each head. */
void or_rope_half(float* vector, int length, int head_dim, int position, double base, int rotary) {
    int half = rotary / 2;
    for (int k = 0; k < half; k++) {
        double angle = position / pow(base, 2.0 * k / rotary);
        double sn = sin(angle), cs = cos(angle);
        for (int start = 0; start < length; start += head_dim) {
            double x = vector[start + k], y = vector[start + k + half];
            vector[start + k] = (float)(x * cs - y * sn);
            vector[start + k + half] = (float)(x * sn + y * cs);
        }
    }
}

/* SwiGlu (TransformerOps.cs:40-50): the sigmoid branch keeps exp's argument non-positive. */
void or_swiglu(const float* gate, const float* up, int length, float* output) {
    for (int i = 0; i < length; i++) {
        double x = gate[i];
        double sigmoid = x >= 0 ? 1 / (1 + exp(-x)) : exp(x) / (1 + exp(x));
        output[i] = (float)(x * sigmoid * up[i]);
    }
}

/* Add (TransformerOps.cs:52-57): FP32 sums. */
void or_add(const float* left, const float* right, int length, float* output) {
    for (int i = 0; i < length; i++) output[i] = left[i] + right[i];
}

/* GroupedAttention (TransformerOps.cs:135-179); Attention (:61-91) is the case query_heads == kv_heads. */
void or_grouped_attention(const float* query, const float* keys, const float* values, int query_heads,
                          int kv_heads, int head_dim, int tokens, double* scores, float* output) {
    int kv_width = kv_heads * head_dim, group = query_heads / kv_heads;
    double scale = 1 / sqrt(head_dim);
    for (int head = 0; head < query_heads; head++) {
        int kv_head = head / group, q_offset = head * head_dim;
        double max = -INFINITY;
        for (int token = 0; token < tokens; token++) {
            int k_offset = token * kv_width + kv_head * head_dim;
            double dot = 0;
            for (int j = 0; j < head_dim; j++) dot += (double)query[q_offset + j] * keys[k_offset + j];
            scores[token] = dot * scale;
            max = max > scores[token] ? max : scores[token];
        }
        double total = 0;
        for (int token = 0; token < tokens; token++) total += scores[token] = exp(scores[token] - max);
        for (int j = 0; j < head_dim; j++) {
            double sum = 0;
            for (int token = 0; token < tokens; token++)
                sum += scores[token] / total * values[token * kv_width + kv_head * head_dim + j];
            output[q_offset + j] = (float)sum;
        }
    }
}

/* QuantizedRow.DecodeRow (src/Satori.Core/QuantizedRow.cs:59-70) through the block decoders. */
void or_q_decode_row(const uint8_t* row, int columns, int format, float* output) {
    int elements = format == 2 || format == 3 ? 256 : 32;
    int bytes = format == 0 ? 34 : format == 1 ? 18 : format == 2 ? 144 : 210;
    for (int b = 0; b < columns / elements; b++) or_q_decode_block(row + (int64_t)b * bytes, format, output + (int64_t)b * elements);
}
