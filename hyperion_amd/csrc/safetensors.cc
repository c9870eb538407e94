#include "safetensors.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>

#include "common.h"

namespace hyperion::model {

using hip::NativeError;

namespace {

[[noreturn]] void malformed(const std::string& why) {
    throw NativeError(HYP_STATUS_INVALID_ARGUMENT, "malformed safetensors header: " + why);
}

// Recursive-descent JSON reader covering what safetensors headers contain.
class Json {
  public:
    explicit Json(const std::string& s) : s_(s) {}

    void ws() {
        while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t')) ++i_;
    }
    bool peek(char c) {
        ws();
        return i_ < s_.size() && s_[i_] == c;
    }
    void expect(char c) {
        ws();
        if (i_ >= s_.size() || s_[i_] != c) malformed(std::string("expected '") + c + "'");
        ++i_;
    }
    bool at_end() {
        ws();
        return i_ >= s_.size();
    }

    std::string string() {
        expect('"');
        std::string out;
        while (true) {
            if (i_ >= s_.size()) malformed("unterminated string");
            const char c = s_[i_++];
            if (c == '"') break;
            if (c == '\\') {
                if (i_ >= s_.size()) malformed("bad escape");
                const char e = s_[i_++];
                switch (e) {
                    case '"': out += '"'; break;
                    case '\\': out += '\\'; break;
                    case '/': out += '/'; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'n': out += '\n'; break;
                    case 'r': out += '\r'; break;
                    case 't': out += '\t'; break;
                    case 'u': {
                        if (i_ + 4 > s_.size()) malformed("bad \\u escape");
                        const unsigned cp = static_cast<unsigned>(std::stoul(s_.substr(i_, 4), nullptr, 16));
                        i_ += 4;
                        if (cp < 0x80) {
                            out += static_cast<char>(cp);
                        } else if (cp < 0x800) {
                            out += static_cast<char>(0xC0 | (cp >> 6));
                            out += static_cast<char>(0x80 | (cp & 0x3F));
                        } else {
                            out += static_cast<char>(0xE0 | (cp >> 12));
                            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
                            out += static_cast<char>(0x80 | (cp & 0x3F));
                        }
                        break;
                    }
                    default: malformed("bad escape");
                }
            } else {
                out += c;
            }
        }
        return out;
    }

    int64_t integer() {
        ws();
        size_t start = i_;
        if (i_ < s_.size() && s_[i_] == '-') ++i_;
        while (i_ < s_.size() && s_[i_] >= '0' && s_[i_] <= '9') ++i_;
        if (i_ == start || (s_[start] == '-' && i_ == start + 1)) malformed("expected an integer");
        if (i_ < s_.size() && (s_[i_] == '.' || s_[i_] == 'e' || s_[i_] == 'E')) malformed("expected an integer");
        if (i_ - start > 18) malformed("integer out of range");
        return std::stoll(s_.substr(start, i_ - start));
    }

    std::vector<int64_t> int_array() {
        std::vector<int64_t> out;
        expect('[');
        if (peek(']')) {
            ++i_;
            return out;
        }
        while (true) {
            out.push_back(integer());
            if (peek(',')) {
                ++i_;
                continue;
            }
            expect(']');
            return out;
        }
    }

    // Skip any JSON value (used for __metadata__ and unknown keys).
    void skip_value(int depth = 0) {
        if (depth > 64) malformed("nesting too deep");
        ws();
        if (i_ >= s_.size()) malformed("unexpected end");
        const char c = s_[i_];
        if (c == '"') {
            (void)string();
        } else if (c == '{') {
            ++i_;
            if (peek('}')) {
                ++i_;
                return;
            }
            while (true) {
                (void)string();
                expect(':');
                skip_value(depth + 1);
                if (peek(',')) {
                    ++i_;
                    continue;
                }
                expect('}');
                return;
            }
        } else if (c == '[') {
            ++i_;
            if (peek(']')) {
                ++i_;
                return;
            }
            while (true) {
                skip_value(depth + 1);
                if (peek(',')) {
                    ++i_;
                    continue;
                }
                expect(']');
                return;
            }
        } else {
            // number / true / false / null
            const size_t start = i_;
            while (i_ < s_.size() && s_[i_] != ',' && s_[i_] != '}' && s_[i_] != ']' && s_[i_] != ' ' &&
                   s_[i_] != '\n' && s_[i_] != '\r' && s_[i_] != '\t')
                ++i_;
            if (i_ == start) malformed("expected a value");
        }
    }

    size_t i_ = 0;

  private:
    const std::string& s_;
};

}  // namespace

size_t dtype_bytes(const std::string& dtype) {
    if (dtype == "U32" || dtype == "I32" || dtype == "F32") return 4;
    if (dtype == "BF16" || dtype == "F16" || dtype == "U16" || dtype == "I16") return 2;
    if (dtype == "U8" || dtype == "I8" || dtype == "BOOL") return 1;
    if (dtype == "F64" || dtype == "I64" || dtype == "U64") return 8;
    return 0;
}

std::map<std::string, TensorInfo> parse_safetensors_header(const std::string& json, uint64_t data_bytes) {
    std::map<std::string, TensorInfo> out;
    Json p(json);
    p.expect('{');
    if (p.peek('}')) {
        ++p.i_;
        return out;
    }
    while (true) {
        const std::string name = p.string();
        p.expect(':');
        if (name == "__metadata__") {
            p.skip_value();
        } else {
            TensorInfo t;
            bool have_dtype = false, have_shape = false, have_offsets = false;
            p.expect('{');
            while (true) {
                const std::string key = p.string();
                p.expect(':');
                if (key == "dtype") {
                    t.dtype = p.string();
                    have_dtype = true;
                } else if (key == "shape") {
                    t.shape = p.int_array();
                    have_shape = true;
                } else if (key == "data_offsets") {
                    const auto off = p.int_array();
                    if (off.size() != 2 || off[0] < 0 || off[1] < off[0]) malformed("bad data_offsets for " + name);
                    t.begin = static_cast<uint64_t>(off[0]);
                    t.end = static_cast<uint64_t>(off[1]);
                    have_offsets = true;
                } else {
                    p.skip_value();
                }
                if (p.peek(',')) {
                    ++p.i_;
                    continue;
                }
                p.expect('}');
                break;
            }
            if (!have_dtype || !have_shape || !have_offsets) malformed("incomplete entry for " + name);
            const size_t eb = dtype_bytes(t.dtype);
            if (eb == 0) malformed("unknown dtype " + t.dtype + " for " + name);
            uint64_t count = 1;
            for (int64_t d : t.shape) {
                if (d < 0) malformed("negative dimension for " + name);
                count *= static_cast<uint64_t>(d);
            }
            if (t.end > data_bytes) malformed("data_offsets past the end of the file for " + name);
            if (t.end - t.begin != count * eb) malformed("byte length does not match shape for " + name);
            if (!out.emplace(name, std::move(t)).second) malformed("duplicate tensor " + name);
        }
        if (p.peek(',')) {
            ++p.i_;
            continue;
        }
        p.expect('}');
        break;
    }
    if (!p.at_end()) malformed("trailing bytes after header");
    return out;
}

SafetensorsFile::SafetensorsFile(const std::string& path) : path_(path) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) throw NativeError(HYP_STATUS_IO, "cannot open " + path + ": " + std::strerror(errno));
    struct stat st {};
    if (::fstat(fd, &st) != 0) {
        const int e = errno;
        ::close(fd);
        throw NativeError(HYP_STATUS_IO, "cannot stat " + path + ": " + std::strerror(e));
    }
    map_bytes_ = static_cast<size_t>(st.st_size);
    if (map_bytes_ < 8) {
        ::close(fd);
        throw NativeError(HYP_STATUS_INVALID_ARGUMENT, "safetensors file too short: " + path);
    }
    map_ = ::mmap(nullptr, map_bytes_, PROT_READ, MAP_PRIVATE, fd, 0);
    const int e = errno;
    ::close(fd);
    if (map_ == MAP_FAILED) {
        map_ = nullptr;
        throw NativeError(HYP_STATUS_IO, "cannot map " + path + ": " + std::strerror(e));
    }
    const auto* bytes = static_cast<const uint8_t*>(map_);
    uint64_t header_len = 0;
    for (int i = 7; i >= 0; --i) header_len = (header_len << 8) | bytes[i];
    if (header_len > map_bytes_ - 8) {
        ::munmap(map_, map_bytes_);
        map_ = nullptr;
        throw NativeError(HYP_STATUS_INVALID_ARGUMENT, "safetensors header length exceeds file: " + path);
    }
    const std::string json(reinterpret_cast<const char*>(bytes + 8), static_cast<size_t>(header_len));
    data_ = bytes + 8 + header_len;
    try {
        tensors_ = parse_safetensors_header(json, map_bytes_ - 8 - header_len);
    } catch (...) {
        ::munmap(map_, map_bytes_);
        map_ = nullptr;
        throw;
    }
}

SafetensorsFile::~SafetensorsFile() {
    if (map_ != nullptr) ::munmap(map_, map_bytes_);
}

}  // namespace hyperion::model
