// Minimal read-only safetensors reader (8-byte little-endian header length, JSON
// header of {name: {dtype, shape, data_offsets}}, then the raw bytes). The reference
// reads the same files through mx::load_safetensors (weights_loader.cc:96-101).
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace hyperion::model {

struct TensorInfo {
    std::string dtype;              // "U32", "BF16", "F32", ...
    std::vector<int64_t> shape;
    uint64_t begin = 0;             // offsets relative to the data section
    uint64_t end = 0;
};

// A memory-mapped shard. Throws NativeError(IO) if the file cannot be read and
// NativeError(INVALID_ARGUMENT) if the header is malformed or inconsistent.
class SafetensorsFile {
  public:
    explicit SafetensorsFile(const std::string& path);
    ~SafetensorsFile();
    SafetensorsFile(const SafetensorsFile&) = delete;
    SafetensorsFile& operator=(const SafetensorsFile&) = delete;

    [[nodiscard]] const std::map<std::string, TensorInfo>& tensors() const noexcept { return tensors_; }
    [[nodiscard]] const uint8_t* data(const TensorInfo& t) const noexcept { return data_ + t.begin; }
    [[nodiscard]] const std::string& path() const noexcept { return path_; }

  private:
    std::string path_;
    void* map_ = nullptr;
    size_t map_bytes_ = 0;
    const uint8_t* data_ = nullptr;
    std::map<std::string, TensorInfo> tensors_;
};

// Parse a safetensors JSON header (exposed for tests of malformed input).
std::map<std::string, TensorInfo> parse_safetensors_header(const std::string& json, uint64_t data_bytes);

size_t dtype_bytes(const std::string& dtype);

}  // namespace hyperion::model
