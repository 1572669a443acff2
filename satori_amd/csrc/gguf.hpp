// GGUF v3 container: strict parse of the catalogue over a read-only file mapping, with the limits, checks and
// failure kinds of GgufFile (src/Satori.Formats.Gguf/GgufFile.cs:17-176) and GgufCursor
// (src/Satori.Formats.Gguf/GgufCursor.cs:7-56). Failures throw satori::Failure with the status of the
// exception the reference throws (InvalidData, NotSupported, ...).
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace satori {

struct GgufTensorInfo {
    std::string name;
    int rank = 0;
    int64_t dims[4] = {0, 0, 0, 0};  // dims[0] is the contiguous (column) dimension
    uint32_t type = 0;
    int64_t offset = 0;              // absolute file offset of the payload
    int64_t byte_length = 0;
};

struct GgufMetadataInfo {
    std::string key;
    uint32_t type = 0;
    int64_t offset = 0;              // absolute file offset of the value (after the type field)
    int64_t byte_length = 0;
    int64_t element_type = -1;       // arrays only
    int64_t element_count = -1;      // arrays only
};

class GgufFile {
public:
    // Maps and parses `path`; throws Failure. The mapping lives until the object is destroyed.
    explicit GgufFile(const std::string& path);
    ~GgufFile();
    GgufFile(const GgufFile&) = delete;
    GgufFile& operator=(const GgufFile&) = delete;

    const std::vector<GgufTensorInfo>& tensors() const { return tensors_; }
    const std::vector<GgufMetadataInfo>& metadata() const { return metadata_; }
    int64_t data_offset() const { return data_offset_; }
    int64_t length() const { return length_; }
    const uint8_t* bytes() const { return map_; }
    // Index of a tensor / key, or -1.
    int64_t find_tensor(const std::string& name) const;
    int64_t find_metadata(const std::string& key) const;

private:
    void parse();

    const uint8_t* map_ = nullptr;
    int64_t length_ = 0;
    int64_t data_offset_ = 0;
    std::vector<GgufTensorInfo> tensors_;
    std::vector<GgufMetadataInfo> metadata_;
    std::unordered_map<std::string, int64_t> tensor_index_, metadata_index_;
};

// Strict UTF-8 (RFC 3629: no overlong forms, no surrogates, nothing above U+10FFFF), the acceptance rule of
// a throwing UTF8Encoding.
bool valid_utf8(const uint8_t* p, int64_t n);

}  // namespace satori
