// GGUF v3 catalogue parse (see gguf.hpp). The checks run in the order GgufFile.Parse runs them
// (src/Satori.Formats.Gguf/GgufFile.cs:78-176), so a file with several defects fails with the same kind.
#include "gguf.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <limits>

#include "host_shapes.hpp"

namespace satori {
namespace {

constexpr int64_t kFileLimit = int64_t(1) << 40;        // GgufFile.cs:21-22
constexpr int64_t kHeaderLimit = int64_t(256) << 20;    // GgufCursor.cs:17-18
constexpr int64_t kCatalogueLimit = 100000;             // GgufFile.cs:86
constexpr int64_t kArrayLimit = 1048576;                // GgufFile.cs:98
constexpr int64_t kMetadataStringLimit = 16 << 20;      // GgufFile.cs:193
constexpr int64_t kKeyLimit = 65535;                    // GgufFile.cs:89
constexpr int64_t kTensorNameLimit = 63;                // GgufFile.cs:127

// Checked Int64 arithmetic fails as the reference's OverflowException, which its constructor reports as
// InvalidDataException (GgufFile.cs:30-34).
struct Overflow {};

int64_t checked_add(int64_t a, int64_t b) {
    int64_t r;
    if (__builtin_add_overflow(a, b, &r)) throw Overflow{};
    return r;
}

int64_t checked_mul(int64_t a, int64_t b) {
    int64_t r;
    if (__builtin_mul_overflow(a, b, &r)) throw Overflow{};
    return r;
}

int64_t align_up(int64_t value, uint32_t alignment) {  // GgufFile.cs:205
    return checked_add(value, static_cast<int64_t>(alignment) - 1) & ~(static_cast<int64_t>(alignment) - 1);
}

class Cursor {  // GgufCursor.cs
public:
    Cursor(const uint8_t* base, int64_t length) : base_(base), length_(length) {}
    int64_t position() const { return pos_; }

    void skip(int64_t n) {
        if (n < 0 || n > length_ - pos_) fail(SATORI_HIP_E_INVALID_DATA, at("Truncated value"));
        if (n > kHeaderLimit - pos_) fail(SATORI_HIP_E_NOT_SUPPORTED, "Header limit: 256 MiB.");
        pos_ += n;
    }

    uint64_t unsigned_value(int size) {
        const int64_t start = pos_;
        skip(size);
        uint64_t v = 0;
        for (int i = size - 1; i >= 0; --i) v = (v << 8) | base_[start + i];
        return v;
    }

    int64_t count(uint64_t v) {
        if (v > static_cast<uint64_t>(std::numeric_limits<int64_t>::max()))
            fail(SATORI_HIP_E_INVALID_DATA, at("Integer exceeds Int64"));
        return static_cast<int64_t>(v);
    }

    std::string string(int64_t limit) {
        const int64_t n = count(unsigned_value(8));
        if (n > limit)
            fail(SATORI_HIP_E_NOT_SUPPORTED,
                 "String byte limit: " + std::to_string(limit) + " at " + std::to_string(pos_) + ".");
        const int64_t start = pos_;
        skip(n);
        if (!valid_utf8(base_ + start, n)) fail(SATORI_HIP_E_INVALID_DATA, at("Invalid UTF-8"));
        return std::string(reinterpret_cast<const char*>(base_ + start), static_cast<size_t>(n));
    }

    std::string at(const std::string& message) const {
        return "GGUF at byte " + std::to_string(pos_) + ": " + message + ".";
    }

private:
    const uint8_t* base_;
    int64_t length_;
    int64_t pos_ = 0;
};

void check_scalar_type(uint32_t type) {  // GgufFile.cs:185-188
    if (type > 12 || type == 9)
        fail(SATORI_HIP_E_NOT_SUPPORTED, "Metadata scalar type " + std::to_string(type) + " is unsupported.");
}

void skip_scalar(Cursor& cursor, uint32_t type) {  // GgufFile.cs:190-200
    check_scalar_type(type);
    if (type == 8) {
        (void)cursor.string(kMetadataStringLimit);
        return;
    }
    if (type == 7) {
        if (cursor.unsigned_value(1) > 1) fail(SATORI_HIP_E_INVALID_DATA, cursor.at("Invalid Boolean"));
        return;
    }
    cursor.skip(type <= 1 ? 1 : type <= 3 ? 2 : type <= 6 ? 4 : 8);
}

bool valid_key(const std::string& key) {  // GgufFile.cs:182-183
    if (key.empty()) return false;
    size_t part = 0;
    for (size_t i = 0; i <= key.size(); ++i) {
        if (i == key.size() || key[i] == '.') {
            if (i == part) return false;
            part = i + 1;
            continue;
        }
        const char c = key[i];
        if (!((c >= 'a' && c <= 'z') || (c >= '0' && c <= '9') || c == '_')) return false;
    }
    return true;
}

}  // namespace

bool valid_utf8(const uint8_t* p, int64_t n) {
    int64_t i = 0;
    while (i < n) {
        const uint8_t b = p[i];
        if (b < 0x80) {
            ++i;
            continue;
        }
        int extra;
        uint8_t lo = 0x80, hi = 0xBF;  // allowed range of the first continuation byte
        if (b >= 0xC2 && b <= 0xDF) {
            extra = 1;
        } else if (b == 0xE0) {
            extra = 2, lo = 0xA0;
        } else if ((b >= 0xE1 && b <= 0xEC) || b == 0xEE || b == 0xEF) {
            extra = 2;
        } else if (b == 0xED) {
            extra = 2, hi = 0x9F;  // no UTF-16 surrogates
        } else if (b == 0xF0) {
            extra = 3, lo = 0x90;
        } else if (b >= 0xF1 && b <= 0xF3) {
            extra = 3;
        } else if (b == 0xF4) {
            extra = 3, hi = 0x8F;  // nothing above U+10FFFF
        } else {
            return false;
        }
        if (n - i <= extra) return false;
        if (p[i + 1] < lo || p[i + 1] > hi) return false;
        for (int k = 2; k <= extra; ++k)
            if ((p[i + k] & 0xC0) != 0x80) return false;
        i += extra + 1;
    }
    return true;
}

GgufFile::GgufFile(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) fail(SATORI_HIP_E_ARGUMENT, "Cannot open " + path + ".");
    struct stat st;
    if (::fstat(fd, &st) != 0) {
        ::close(fd);
        fail(SATORI_HIP_E_ARGUMENT, "Cannot stat " + path + ".");
    }
    const int64_t length = static_cast<int64_t>(st.st_size);
    if (length == 0) {
        ::close(fd);
        fail(SATORI_HIP_E_INVALID_DATA, "GGUF at byte 0: empty file.");
    }
    if (length > kFileLimit) {
        ::close(fd);
        fail(SATORI_HIP_E_NOT_SUPPORTED, "File limit: 1 TiB.");
    }
    void* map = ::mmap(nullptr, static_cast<size_t>(length), PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (map == MAP_FAILED) fail(SATORI_HIP_E_ARGUMENT, "Cannot map " + path + ".");
    map_ = static_cast<const uint8_t*>(map);
    length_ = length;
    try {
        parse();
    } catch (const Overflow&) {
        ::munmap(const_cast<uint8_t*>(map_), static_cast<size_t>(length_));
        fail(SATORI_HIP_E_INVALID_DATA, "GGUF: offset or dimension overflow.");
    } catch (...) {
        ::munmap(const_cast<uint8_t*>(map_), static_cast<size_t>(length_));
        throw;
    }
}

GgufFile::~GgufFile() {
    if (map_) ::munmap(const_cast<uint8_t*>(map_), static_cast<size_t>(length_));
}

int64_t GgufFile::find_tensor(const std::string& name) const {
    const auto it = tensor_index_.find(name);
    return it == tensor_index_.end() ? -1 : it->second;
}

int64_t GgufFile::find_metadata(const std::string& key) const {
    const auto it = metadata_index_.find(key);
    return it == metadata_index_.end() ? -1 : it->second;
}

void GgufFile::parse() {
    Cursor cursor(map_, length_);
    if (cursor.unsigned_value(4) != 0x46554747u) fail(SATORI_HIP_E_INVALID_DATA, cursor.at("Invalid magic"));
    if (cursor.unsigned_value(4) != 3) fail(SATORI_HIP_E_NOT_SUPPORTED, "Only little-endian GGUF v3 is supported.");
    const int64_t tensor_count = cursor.count(cursor.unsigned_value(8));
    const int64_t metadata_count = cursor.count(cursor.unsigned_value(8));
    if (tensor_count == 0) fail(SATORI_HIP_E_NOT_SUPPORTED, "Tensor count zero is outside the profile.");
    if (tensor_count > kCatalogueLimit || metadata_count > kCatalogueLimit)
        fail(SATORI_HIP_E_NOT_SUPPORTED, "Catalogue count limit: 100000.");

    for (int64_t i = 0; i < metadata_count; ++i) {
        GgufMetadataInfo entry;
        entry.key = cursor.string(kKeyLimit);
        if (!valid_key(entry.key)) fail(SATORI_HIP_E_INVALID_DATA, cursor.at("Invalid metadata key"));
        entry.type = static_cast<uint32_t>(cursor.unsigned_value(4));
        const int64_t start = cursor.position();
        if (entry.type == 9) {
            const uint32_t element_type = static_cast<uint32_t>(cursor.unsigned_value(4));
            const int64_t count = cursor.count(cursor.unsigned_value(8));
            if (count > kArrayLimit) fail(SATORI_HIP_E_NOT_SUPPORTED, "Array count limit: 1048576.");
            check_scalar_type(element_type);
            for (int64_t j = 0; j < count; ++j) skip_scalar(cursor, element_type);
            entry.element_type = element_type;
            entry.element_count = count;
        } else {
            skip_scalar(cursor, entry.type);
        }
        entry.offset = start;
        entry.byte_length = cursor.position() - start;
        if (metadata_index_.count(entry.key)) fail(SATORI_HIP_E_INVALID_DATA, cursor.at("Duplicate metadata key"));
        metadata_index_.emplace(entry.key, static_cast<int64_t>(metadata_.size()));
        metadata_.push_back(std::move(entry));
    }

    // Typed lookups with a fallback (GgufFile.cs:176-181): a present key of another type is corrupt.
    auto entry_of = [&](const char* key, uint32_t type) -> const GgufMetadataInfo* {
        const int64_t k = find_metadata(key);
        if (k < 0) return nullptr;
        const GgufMetadataInfo& e = metadata_[static_cast<size_t>(k)];
        if (e.type != type)
            fail(SATORI_HIP_E_INVALID_DATA,
                 "GGUF at byte " + std::to_string(e.offset) + ": wrong type for " + key + ".");
        return &e;
    };
    auto get_u32 = [&](const char* key, uint32_t fallback) -> uint32_t {
        const GgufMetadataInfo* e = entry_of(key, 4);
        if (!e) return fallback;
        uint32_t v;
        std::memcpy(&v, map_ + e->offset, 4);
        return v;
    };
    auto get_u16 = [&](const char* key, uint16_t fallback) -> uint16_t {
        const GgufMetadataInfo* e = entry_of(key, 2);
        return e ? u16_at(map_ + e->offset) : fallback;
    };
    auto get_i32 = [&](const char* key, int32_t fallback) -> int32_t {
        const GgufMetadataInfo* e = entry_of(key, 5);
        if (!e) return fallback;
        int32_t v;
        std::memcpy(&v, map_ + e->offset, 4);
        return v;
    };
    auto get_string = [&](const char* key, const char* fallback) -> std::string {
        const GgufMetadataInfo* e = entry_of(key, 8);
        if (!e) return fallback;
        return std::string(reinterpret_cast<const char*>(map_ + e->offset + 8), static_cast<size_t>(e->byte_length - 8));
    };

    const uint32_t alignment = get_u32("general.alignment", 32);
    if (alignment == 0 || (alignment & (alignment - 1)) != 0) fail(SATORI_HIP_E_INVALID_DATA, cursor.at("Invalid alignment"));
    if (alignment < 8 || alignment > 4096) fail(SATORI_HIP_E_NOT_SUPPORTED, "Alignment range: 8 to 4096.");
    const std::string architecture = get_string("general.architecture", "");
    const bool arch_ok = !architecture.empty() && std::all_of(architecture.begin(), architecture.end(), [](char c) {
        return (c >= 'a' && c <= 'z') || (c >= '0' && c <= '9');
    });
    if (!arch_ok) fail(SATORI_HIP_E_INVALID_DATA, cursor.at("Missing or invalid general.architecture"));
    if (get_string("general.type", "model") != "model") fail(SATORI_HIP_E_NOT_SUPPORTED, "Only model files are supported.");
    (void)get_u32("general.file_type", 0);
    // A single unsharded file may declare split.count 0 or 1 (GgufFile.cs:112-115).
    const uint16_t split_count = get_u16("split.count", 1);
    if (!(split_count == 0 || split_count == 1) || get_u16("split.no", 0) != 0)
        fail(SATORI_HIP_E_NOT_SUPPORTED, "Sharded GGUF is unsupported.");
    if (get_i32("split.tensors.count", static_cast<int32_t>(tensor_count)) != tensor_count)
        fail(SATORI_HIP_E_INVALID_DATA, cursor.at("Invalid split.tensors.count"));

    bool quantized = false;
    std::vector<GgufTensorInfo> relative;
    for (int64_t i = 0; i < tensor_count; ++i) {
        GgufTensorInfo t;
        t.name = cursor.string(kTensorNameLimit);
        if (t.name.empty() || t.name.find('\0') != std::string::npos)
            fail(SATORI_HIP_E_INVALID_DATA, cursor.at("Invalid tensor name"));
        const uint32_t rank = static_cast<uint32_t>(cursor.unsigned_value(4));
        if (rank == 0) fail(SATORI_HIP_E_INVALID_DATA, cursor.at("Zero rank"));
        if (rank > 4) fail(SATORI_HIP_E_NOT_SUPPORTED, "Tensor rank limit: 4.");
        t.rank = static_cast<int>(rank);
        int64_t elements = 1;
        for (int d = 0; d < t.rank; ++d) {
            t.dims[d] = cursor.count(cursor.unsigned_value(8));
            if (t.dims[d] == 0) fail(SATORI_HIP_E_INVALID_DATA, cursor.at("Zero dimension"));
            elements = checked_mul(elements, t.dims[d]);
        }
        t.type = static_cast<uint32_t>(cursor.unsigned_value(4));
        int block, bytes;
        switch (t.type) {  // GgufFile.cs:139-146
            case 0: block = 1, bytes = 4; break;
            case 1: block = 1, bytes = 2; break;
            case 2: block = 32, bytes = 18; break;
            case 8: block = 32, bytes = 34; break;
            case 12: block = 256, bytes = 144; break;
            case 14: block = 256, bytes = 210; break;
            default: fail(SATORI_HIP_E_NOT_SUPPORTED, "Tensor type " + std::to_string(t.type) + " is unsupported.");
        }
        quantized |= block != 1;
        if (t.dims[0] % block != 0)
            fail(SATORI_HIP_E_INVALID_DATA, cursor.at("Quantized row is not a multiple of " + std::to_string(block)));
        t.byte_length = checked_mul(elements / block, bytes);
        t.offset = cursor.count(cursor.unsigned_value(8));
        if (t.offset % alignment != 0) fail(SATORI_HIP_E_INVALID_DATA, cursor.at("Unaligned tensor offset"));
        (void)checked_add(t.offset, align_up(t.byte_length, alignment));
        if (tensor_index_.count(t.name)) fail(SATORI_HIP_E_INVALID_DATA, cursor.at("Duplicate tensor name"));
        tensor_index_.emplace(t.name, static_cast<int64_t>(relative.size()));
        relative.push_back(std::move(t));
    }
    if (quantized && find_metadata("general.quantization_version") < 0)
        fail(SATORI_HIP_E_INVALID_DATA, cursor.at("Missing quantization version"));
    if (get_u32("general.quantization_version", 2) != 2)
        fail(SATORI_HIP_E_NOT_SUPPORTED, "Quantization version must be 2.");
    data_offset_ = align_up(cursor.position(), alignment);
    cursor.skip(data_offset_ - cursor.position());

    // Physical extents in offset order (a stable sort, as OrderBy): inside the file, no overlap.
    std::vector<size_t> order(relative.size());
    for (size_t i = 0; i < order.size(); ++i) order[i] = i;
    std::stable_sort(order.begin(), order.end(),
                     [&](size_t a, size_t b) { return relative[a].offset < relative[b].offset; });
    int64_t previous_end = 0;
    for (size_t i : order) {
        const int64_t end = checked_add(relative[i].offset, align_up(relative[i].byte_length, alignment));
        if (end > length_ - data_offset_) fail(SATORI_HIP_E_INVALID_DATA, cursor.at("Tensor data or final padding exceeds file"));
        if (relative[i].offset < previous_end) fail(SATORI_HIP_E_INVALID_DATA, cursor.at("Overlapping tensor ranges"));
        previous_end = end;
    }
    // Canonical layout: tensors packed in declaration order, each padded to the alignment.
    int64_t expected = 0;
    for (const GgufTensorInfo& t : relative) {
        if (t.offset != expected) fail(SATORI_HIP_E_NOT_SUPPORTED, "Noncanonical tensor gap/order.");
        expected = checked_add(t.offset, align_up(t.byte_length, alignment));
    }
    for (GgufTensorInfo& t : relative) t.offset = checked_add(data_offset_, t.offset);
    tensors_ = std::move(relative);
}

}  // namespace satori
