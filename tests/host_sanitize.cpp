// Host code of the library under AddressSanitizer and UndefinedBehaviorSanitizer (built and run by
// tests/test_host_sanitize.py with g++; any sanitizer report aborts the run):
//  * the GGUF catalogue parser (satori_amd/csrc/gguf.cpp) over seed files, every truncation of each, every
//    single-byte mutation of their first 1,024 bytes and 64-bit extreme values written at every offset
//    there: each parse either succeeds, with every tensor and metadata window inside the file, or throws
//    satori::Failure with a status;
//  * the host validation, quantizer and bitplane entry points (satori_amd/csrc/host_cpu.cpp) on payloads
//    allocated at exactly the length the shape gives (so any read past the end is reported), valid and
//    corrupted, with wrong lengths and with shapes whose byte length overflows.
// Usage: host_sanitize WORK_DIR SEED.gguf...
#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <climits>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <random>
#include <string>
#include <vector>

#include "../include/satori_hip.h"
#include "../satori_amd/csrc/gguf.hpp"
#include "../satori_amd/csrc/host_shapes.hpp"

namespace satori {
void record_error(const std::string&) {}  // the runtime keeps the message per thread; not needed here
}  // namespace satori

namespace {

int failures = 0;

void expect(bool ok, const std::string& what) {
    if (!ok) {
        std::fprintf(stderr, "FAILED: %s\n", what.c_str());
        ++failures;
    }
}

std::vector<uint8_t> read_file(const std::string& path) {
    std::vector<uint8_t> bytes;
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return bytes;
    uint8_t buffer[4096];
    size_t n;
    while ((n = std::fread(buffer, 1, sizeof buffer, f)) > 0) bytes.insert(bytes.end(), buffer, buffer + n);
    std::fclose(f);
    return bytes;
}

void write_file(const std::string& path, const uint8_t* data, size_t n) {
    const int fd = ::open(path.c_str(), O_WRONLY | O_CREAT | O_TRUNC, 0600);
    if (fd < 0) {
        std::perror("open");
        std::exit(2);
    }
    size_t done = 0;
    while (done < n) {
        const ssize_t w = ::write(fd, data + done, n - done);
        if (w <= 0) {
            std::perror("write");
            std::exit(2);
        }
        done += static_cast<size_t>(w);
    }
    ::close(fd);
}

struct ParseCounts {
    long parsed = 0, rejected = 0;
};

// One parse of `bytes`; a success must publish only windows inside the file, whose bytes are then read.
void parse_case(const std::string& path, const std::vector<uint8_t>& bytes, const std::string& label,
                ParseCounts& counts) {
    write_file(path, bytes.data(), bytes.size());
    try {
        satori::GgufFile file(path);
        ++counts.parsed;
        const int64_t n = file.length();
        expect(n == static_cast<int64_t>(bytes.size()), label + ": length");
        expect(file.data_offset() >= 0 && file.data_offset() <= n, label + ": data offset inside the file");
        unsigned sum = 0;
        for (const auto& t : file.tensors()) {
            const bool inside = t.offset >= 0 && t.byte_length >= 0 && t.offset <= n && t.byte_length <= n - t.offset;
            expect(inside, label + ": tensor window of " + t.name);
            if (inside)
                for (int64_t i = 0; i < t.byte_length; ++i) sum += file.bytes()[t.offset + i];
            expect(file.find_tensor(t.name) >= 0, label + ": tensor index of " + t.name);
        }
        for (const auto& m : file.metadata()) {
            const bool inside = m.offset >= 0 && m.byte_length >= 0 && m.offset <= n && m.byte_length <= n - m.offset;
            expect(inside, label + ": metadata window of " + m.key);
            if (inside)
                for (int64_t i = 0; i < m.byte_length; ++i) sum += file.bytes()[m.offset + i];
            expect(file.find_metadata(m.key) >= 0, label + ": metadata index of " + m.key);
        }
        if (sum == 0xFFFFFFFFu) std::fprintf(stderr, " ");  // keeps the reads
    } catch (const satori::Failure& f) {
        ++counts.rejected;
        expect(f.status != SATORI_HIP_OK && !f.message.empty(), label + ": failure carries a status and message");
    } catch (...) {
        expect(false, label + ": exception other than satori::Failure");
    }
}

void fuzz_gguf(const std::string& work, const std::string& seed_path) {
    const std::vector<uint8_t> seed = read_file(seed_path);
    expect(!seed.empty(), "seed " + seed_path + " readable");
    if (seed.empty()) return;
    const std::string path = work + "/case.gguf";
    ParseCounts counts;
    parse_case(path, seed, seed_path, counts);
    expect(counts.parsed == 1, seed_path + ": the seed itself parses");
    for (size_t length = 0; length < seed.size(); ++length) {
        const std::vector<uint8_t> cut(seed.begin(), seed.begin() + static_cast<long>(length));
        parse_case(path, cut, seed_path + " truncated to " + std::to_string(length), counts);
    }
    const size_t span = std::min<size_t>(seed.size(), 1024);
    for (size_t i = 0; i < span; ++i)
        for (uint8_t value : {uint8_t(0x00), uint8_t(0xFF), uint8_t(seed[i] ^ 0x01), uint8_t(seed[i] ^ 0x80)}) {
            if (value == seed[i]) continue;
            std::vector<uint8_t> m = seed;
            m[i] = value;
            parse_case(path, m, seed_path + " byte " + std::to_string(i) + " = " + std::to_string(value), counts);
        }
    const uint64_t extremes[] = {0, 1, 0x7FFFFFFFull, 0xFFFFFFFFull, 0x8000000000000000ull, 0x7FFFFFFFFFFFFFFFull,
                                 ~0ull};
    for (size_t i = 0; i + 8 <= span; ++i)
        for (uint64_t value : extremes) {
            std::vector<uint8_t> m = seed;
            std::memcpy(m.data() + i, &value, 8);  // little-endian, as GGUF stores it
            parse_case(path, m, seed_path + " u64 at " + std::to_string(i), counts);
        }
    std::printf("gguf %s: %zu bytes, %ld parsed, %ld rejected\n", seed_path.c_str(), seed.size(), counts.parsed,
                counts.rejected);
}

// ---- Host payload entry points ----

struct Case {
    int format, rows, columns, block;  // block: Ternary2 block size (ignored for the other formats)
};

std::vector<uint8_t*> owned;

uint8_t* exact(size_t n) {  // heap block of exactly n bytes (at least one, so it has an address)
    uint8_t* p = new uint8_t[n ? n : 1];
    owned.push_back(p);
    return p;
}

std::string name(const Case& c) {
    return "format " + std::to_string(c.format) + " " + std::to_string(c.rows) + "x" + std::to_string(c.columns) +
           " block " + std::to_string(c.block);
}

int validate(const Case& c, const void* p, size_t n) {
    return c.format == SATORI_HIP_TERNARY2 ? satori_hip_ternary2_validate(c.rows, c.columns, c.block, p, n)
                                           : satori_hip_quantized_validate(c.rows, c.columns, c.format, p, n);
}

void fuzz_payloads() {
    std::mt19937_64 rng(2031);
    const Case cases[] = {
        {SATORI_HIP_TERNARY2, 1, 1, 64},    {SATORI_HIP_TERNARY2, 3, 65, 64},   {SATORI_HIP_TERNARY2, 2, 300, 128},
        {SATORI_HIP_TERNARY2, 2, 513, 256}, {SATORI_HIP_TERNARY2, 5, 64, 128},  {SATORI_HIP_Q8_0, 1, 32, 0},
        {SATORI_HIP_Q8_0, 3, 96, 0},        {SATORI_HIP_Q4_0, 2, 64, 0},        {SATORI_HIP_Q4_K, 1, 256, 0},
        {SATORI_HIP_Q4_K, 3, 512, 0},       {SATORI_HIP_Q6_K, 2, 256, 0},       {SATORI_HIP_Q6_K, 1, 768, 0},
    };
    long valid_random = 0;
    for (const Case& c : cases) {
        int64_t length = -1;
        expect(satori_hip_payload_length(c.format, c.rows, c.columns, c.block, &length) == SATORI_HIP_OK && length > 0,
               name(c) + ": payload length");
        if (length <= 0) continue;
        const size_t n = static_cast<size_t>(length);
        // Quantized from finite weights: valid, and (Ternary2) a lossless bitplane round trip.
        std::normal_distribution<float> normal(0.0f, 1.0f);
        std::vector<float> weights(static_cast<size_t>(c.rows) * c.columns);
        for (float& w : weights) w = normal(rng);
        uint8_t* payload = exact(n);
        const int q = c.format == SATORI_HIP_TERNARY2
                          ? satori_hip_ternary2_quantize(weights.data(), c.rows, c.columns, c.block, payload, n)
                          : satori_hip_quantize_weights(c.format, weights.data(), c.rows, c.columns, payload, n);
        expect(q == SATORI_HIP_OK, name(c) + ": quantize");
        expect(validate(c, payload, n) == SATORI_HIP_OK, name(c) + ": quantized payload validates");
        if (c.format == SATORI_HIP_TERNARY2) {
            uint8_t* planes = exact(n);
            uint8_t* back = exact(n);
            expect(satori_hip_bitplane_from_ternary2(c.rows, c.columns, c.block, payload, n, planes, n) == SATORI_HIP_OK,
                   name(c) + ": to bitplanes");
            expect(satori_hip_bitplane_validate(c.rows, c.columns, c.block, planes, n) == SATORI_HIP_OK,
                   name(c) + ": bitplanes validate");
            expect(satori_hip_bitplane_to_ternary2(c.rows, c.columns, c.block, planes, n, back, n) == SATORI_HIP_OK &&
                       std::memcmp(back, payload, n) == 0,
                   name(c) + ": bitplane round trip");
            // Lengths one short and one long never read or write past the buffers they are given.
            if (n > 1) {
                expect(satori_hip_bitplane_from_ternary2(c.rows, c.columns, c.block, payload, n - 1, planes, n) != 0,
                       name(c) + ": short Ternary2 length rejected");
                expect(satori_hip_bitplane_to_ternary2(c.rows, c.columns, c.block, planes, n, back, n - 1) != 0,
                       name(c) + ": short output length rejected");
            }
        }
        // Wrong lengths are rejected before anything is read.
        expect(validate(c, payload, n - 1) != SATORI_HIP_OK, name(c) + ": short length rejected");
        uint8_t* longer = exact(n + 1);
        std::memcpy(longer, payload, n);
        expect(validate(c, longer, n + 1) != SATORI_HIP_OK, name(c) + ": long length rejected");
        // Random and corrupted payloads: any status, no report.
        for (int trial = 0; trial < 200; ++trial) {
            uint8_t* random = exact(n);
            for (size_t i = 0; i < n; ++i) random[i] = static_cast<uint8_t>(rng());
            if (validate(c, random, n) == SATORI_HIP_OK) {
                ++valid_random;
                if (c.format == SATORI_HIP_TERNARY2) {
                    uint8_t* planes = exact(n);
                    (void)satori_hip_bitplane_from_ternary2(c.rows, c.columns, c.block, random, n, planes, n);
                }
            }
            if (c.format == SATORI_HIP_TERNARY2) (void)satori_hip_bitplane_validate(c.rows, c.columns, c.block, random, n);
            uint8_t* flipped = exact(n);
            std::memcpy(flipped, payload, n);
            flipped[rng() % n] ^= static_cast<uint8_t>(1u << (rng() % 8));
            (void)validate(c, flipped, n);
        }
        // Non-finite weights are rejected.
        weights[weights.size() / 2] = std::numeric_limits<float>::infinity();
        const int bad = c.format == SATORI_HIP_TERNARY2
                            ? satori_hip_ternary2_quantize(weights.data(), c.rows, c.columns, c.block, payload, n)
                            : satori_hip_quantize_weights(c.format, weights.data(), c.rows, c.columns, payload, n);
        expect(bad != SATORI_HIP_OK, name(c) + ": non-finite weight rejected");
    }
    // Shapes whose checks must fail without overflowing: zero, negative, ragged and huge dimensions.
    const int formats[] = {SATORI_HIP_TERNARY2, SATORI_HIP_Q8_0, SATORI_HIP_Q4_0, SATORI_HIP_Q4_K, SATORI_HIP_Q6_K};
    const int dims[] = {INT_MIN, -1, 0, 1, 31, 33, 255, 257, 65536, 1 << 30, INT_MAX};
    const int blocks[] = {0, 63, 64, 128, 256, 512};
    long shapes = 0;
    for (int format : formats)
        for (int rows : dims)
            for (int columns : dims)
                for (int block : blocks) {
                    int64_t length = -1;
                    const int s = satori_hip_payload_length(format, rows, columns, block, &length);
                    expect(s != SATORI_HIP_OK || length > 0, "payload length positive when accepted");
                    uint8_t byte = 0;
                    if (format == SATORI_HIP_TERNARY2)
                        (void)satori_hip_ternary2_validate(rows, columns, block, &byte, 1);
                    else
                        (void)satori_hip_quantized_validate(rows, columns, format, &byte, 1);
                    ++shapes;
                    if (format != SATORI_HIP_TERNARY2) break;  // the block size only matters for Ternary2
                }
    expect(satori_hip_payload_length(SATORI_HIP_TERNARY2, 1, 64, 128, nullptr) != SATORI_HIP_OK,
           "null length pointer rejected");
    expect(satori_hip_ternary2_validate(1, 64, 64, nullptr, 20) != SATORI_HIP_OK, "null payload rejected");
    std::printf("payloads: %zu shapes quantized and round-tripped, %ld random payloads valid, %ld shape checks\n",
                sizeof(cases) / sizeof(cases[0]), valid_random, shapes);
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 2) {
        std::fprintf(stderr, "usage: %s WORK_DIR SEED.gguf...\n", argv[0]);
        return 2;
    }
    for (int i = 2; i < argc; ++i) fuzz_gguf(argv[1], argv[i]);
    fuzz_payloads();
    for (uint8_t* p : owned) delete[] p;
    if (failures) {
        std::fprintf(stderr, "%d checks failed\n", failures);
        return 1;
    }
    std::printf("ok\n");
    return 0;
}
