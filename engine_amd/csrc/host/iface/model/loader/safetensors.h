// Read-only, validated safetensors file, restated with the reference's API
// (model/loader/safetensors.h:21-79): the hip backend's Load reads its
// weights through exactly these calls. Implementation: safetensors.cpp.
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <string_view>
#include <vector>

#include "core/engine/error.h"

namespace lykuro::nie {

// kU8 / kI8 extend the reference's allowlist (safetensors.h:21) for
// offline-quantized artifacts: packed int4 codes (U8) and int8 codes (I8).
enum class Dtype { kBf16, kF16, kF32, kU8, kI8 };

size_t DtypeSize(Dtype dtype);
std::string_view DtypeName(Dtype dtype);

struct TensorInfo {
    Dtype dtype = Dtype::kF32;
    std::vector<uint64_t> shape;
    uint64_t data_offset = 0;
    uint64_t data_size = 0;
    uint64_t element_count = 0;
};

struct SafetensorsHeader {
    std::map<std::string, TensorInfo> tensors;
    std::map<std::string, std::string> metadata;
};

struct HeaderParseResult {
    Status status;
    SafetensorsHeader header;
};

HeaderParseResult ParseSafetensorsHeader(std::string_view header_json, uint64_t data_section_size);

class SafetensorsFile {
public:
    SafetensorsFile() = default;
    ~SafetensorsFile();
    SafetensorsFile(const SafetensorsFile&) = delete;
    SafetensorsFile& operator=(const SafetensorsFile&) = delete;
    SafetensorsFile(SafetensorsFile&& other) noexcept;
    SafetensorsFile& operator=(SafetensorsFile&& other) noexcept;

    Status Open(const std::string& path, uint64_t max_header_bytes = 16ull << 20);

    bool is_open() const { return data_ != nullptr; }
    const SafetensorsHeader& header() const { return header_; }

    const uint8_t* TensorData(const std::string& name) const;
    const TensorInfo* FindTensor(const std::string& name) const;

    void Close();

private:
    SafetensorsHeader header_;
    void* map_base_ = nullptr;
    size_t map_size_ = 0;
    const uint8_t* data_ = nullptr;
    uint64_t data_size_ = 0;
};

}  // namespace lykuro::nie
