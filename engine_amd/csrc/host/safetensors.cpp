// Safetensors reader for the hip backend's loader. The file is untrusted
// input: 8-byte little-endian header length with a cap, a strict JSON header
// (only the constructs safetensors uses), dtype allow-list BF16/F16/F32,
// offsets that tile the data section exactly, shape products that match the
// byte sizes (overflow-checked), and a read-only mapping. Same checks as the
// reference reader (model/loader/safetensors.cpp:1-297), written here from
// that contract.
#include "model/loader/safetensors.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>

#include "core/engine/error.h"

namespace lykuro::nie {

namespace {

constexpr const char kComponent[] = "safetensors";

Status Bad(const char* msg) { return Status(ErrorCode::kArtifactVerificationFailed, msg, kComponent); }

// Limits on untrusted headers: tensor rank, tensor count, name length.
constexpr size_t kRankLimit = 8;
constexpr size_t kTensorLimit = 100000;
constexpr size_t kNameLimit = 512;

// Minimal JSON reader over the header: objects, arrays, strings (with the
// escapes JSON allows) and non-negative integers.
class Json {
public:
    explicit Json(std::string_view s) : s_(s) {}

    bool Ws() {
        while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\t' || s_[i_] == '\r')) ++i_;
        return i_ < s_.size();
    }
    bool Eat(char c) {
        if (!Ws() || s_[i_] != c) return false;
        ++i_;
        return true;
    }
    bool Peek(char c) { return Ws() && s_[i_] == c; }
    bool End() {
        Ws();
        return i_ == s_.size();
    }

    bool String(std::string& out) {
        out.clear();
        if (!Eat('"')) return false;
        while (i_ < s_.size()) {
            char c = s_[i_++];
            if (c == '"') return true;
            if (static_cast<unsigned char>(c) < 0x20) return false;
            if (c != '\\') {
                out.push_back(c);
                continue;
            }
            if (i_ >= s_.size()) return false;
            char e = s_[i_++];
            switch (e) {
                case '"': out.push_back('"'); break;
                case '\\': out.push_back('\\'); break;
                case '/': out.push_back('/'); break;
                case 'b': out.push_back('\b'); break;
                case 'f': out.push_back('\f'); break;
                case 'n': out.push_back('\n'); break;
                case 'r': out.push_back('\r'); break;
                case 't': out.push_back('\t'); break;
                case 'u': {
                    if (i_ + 4 > s_.size()) return false;
                    unsigned v = 0;
                    for (int k = 0; k < 4; ++k) {
                        char h = s_[i_++];
                        v <<= 4;
                        if (h >= '0' && h <= '9') v |= unsigned(h - '0');
                        else if (h >= 'a' && h <= 'f') v |= unsigned(h - 'a' + 10);
                        else if (h >= 'A' && h <= 'F') v |= unsigned(h - 'A' + 10);
                        else return false;
                    }
                    if (v >= 0xD800 && v <= 0xDFFF) return false;  // no surrogates in names
                    if (v < 0x80) out.push_back(char(v));
                    else if (v < 0x800) {
                        out.push_back(char(0xC0 | (v >> 6)));
                        out.push_back(char(0x80 | (v & 0x3F)));
                    } else {
                        out.push_back(char(0xE0 | (v >> 12)));
                        out.push_back(char(0x80 | ((v >> 6) & 0x3F)));
                        out.push_back(char(0x80 | (v & 0x3F)));
                    }
                    break;
                }
                default: return false;
            }
        }
        return false;
    }

    bool Uint(uint64_t& out) {
        if (!Ws() || s_[i_] < '0' || s_[i_] > '9') return false;
        if (s_[i_] == '0' && i_ + 1 < s_.size() && s_[i_ + 1] >= '0' && s_[i_ + 1] <= '9') return false;
        out = 0;
        while (i_ < s_.size() && s_[i_] >= '0' && s_[i_] <= '9') {
            const uint64_t d = uint64_t(s_[i_++] - '0');
            if (out > (UINT64_MAX - d) / 10) return false;
            out = out * 10 + d;
        }
        return true;
    }

    bool UintArray(std::vector<uint64_t>& out) {
        out.clear();
        if (!Eat('[')) return false;
        if (Eat(']')) return true;
        do {
            uint64_t v;
            if (!Uint(v)) return false;
            out.push_back(v);
        } while (Eat(','));
        return Eat(']');
    }

private:
    std::string_view s_;
    size_t i_ = 0;
};

bool ParseDtype(const std::string& s, Dtype& d) {
    if (s == "BF16") d = Dtype::kBf16;
    else if (s == "F16") d = Dtype::kF16;
    else if (s == "F32") d = Dtype::kF32;
    else if (s == "U8") d = Dtype::kU8;
    else if (s == "I8") d = Dtype::kI8;
    else return false;
    return true;
}

}  // namespace

size_t DtypeSize(Dtype dtype) {
    switch (dtype) {
        case Dtype::kF32: return 4;
        case Dtype::kU8:
        case Dtype::kI8: return 1;
        default: return 2;
    }
}

std::string_view DtypeName(Dtype dtype) {
    switch (dtype) {
        case Dtype::kBf16: return "BF16";
        case Dtype::kF16: return "F16";
        case Dtype::kF32: return "F32";
        case Dtype::kU8: return "U8";
        case Dtype::kI8: return "I8";
    }
    return "?";
}

HeaderParseResult ParseSafetensorsHeader(std::string_view text, uint64_t data_section_size) {
    HeaderParseResult r;
    Json j(text);
    if (!j.Eat('{')) {
        r.status = Bad("safetensors header is not a JSON object");
        return r;
    }
    std::vector<std::pair<uint64_t, uint64_t>> spans;
    if (!j.Eat('}')) {
        do {
            std::string name;
            if (!j.String(name) || !j.Eat(':')) {
                r.status = Bad("malformed safetensors header");
                return r;
            }
            if (name == "__metadata__") {
                if (!j.Eat('{')) {
                    r.status = Bad("malformed safetensors metadata");
                    return r;
                }
                if (!j.Eat('}')) {
                    do {
                        std::string k, v;
                        if (!j.String(k) || !j.Eat(':') || !j.String(v)) {
                            r.status = Bad("malformed safetensors metadata");
                            return r;
                        }
                        r.header.metadata[k] = v;
                    } while (j.Eat(','));
                    if (!j.Eat('}')) {
                        r.status = Bad("malformed safetensors metadata");
                        return r;
                    }
                }
                continue;
            }
            if (r.header.tensors.count(name)) {
                r.status = Bad("duplicate tensor name");
                return r;
            }
            if (name.empty() || name.size() > kNameLimit || r.header.tensors.size() >= kTensorLimit) {
                r.status = Bad("tensor name or count out of range");
                return r;
            }
            TensorInfo info;
            bool have_dtype = false, have_shape = false, have_offsets = false;
            std::vector<uint64_t> offsets;
            if (!j.Eat('{')) {
                r.status = Bad("malformed tensor entry");
                return r;
            }
            do {
                std::string key;
                if (!j.String(key) || !j.Eat(':')) {
                    r.status = Bad("malformed tensor entry");
                    return r;
                }
                if (key == "dtype" && !have_dtype) {
                    std::string d;
                    if (!j.String(d) || !ParseDtype(d, info.dtype)) {
                        r.status = Bad("unsupported tensor dtype");
                        return r;
                    }
                    have_dtype = true;
                } else if (key == "shape" && !have_shape) {
                    if (!j.UintArray(info.shape) || info.shape.size() > kRankLimit) {
                        r.status = Bad("malformed tensor shape");
                        return r;
                    }
                    have_shape = true;
                } else if (key == "data_offsets" && !have_offsets) {
                    if (!j.UintArray(offsets) || offsets.size() != 2 || offsets[0] > offsets[1]) {
                        r.status = Bad("malformed tensor offsets");
                        return r;
                    }
                    have_offsets = true;
                } else {
                    r.status = Bad("unexpected tensor entry field");
                    return r;
                }
            } while (j.Eat(','));
            if (!j.Eat('}') || !have_dtype || !have_shape || !have_offsets) {
                r.status = Bad("incomplete tensor entry");
                return r;
            }
            uint64_t count = 1;
            for (uint64_t d : info.shape) {
                if (d != 0 && count > UINT64_MAX / d) {
                    r.status = Bad("tensor shape overflows");
                    return r;
                }
                count *= d;
            }
            info.element_count = count;
            info.data_offset = offsets[0];
            info.data_size = offsets[1] - offsets[0];
            if (count > UINT64_MAX / DtypeSize(info.dtype) || count * DtypeSize(info.dtype) != info.data_size) {
                r.status = Bad("tensor byte size does not match shape");
                return r;
            }
            spans.emplace_back(offsets[0], offsets[1]);
            r.header.tensors.emplace(std::move(name), std::move(info));
        } while (j.Eat(','));
        if (!j.Eat('}')) {
            r.status = Bad("malformed safetensors header");
            return r;
        }
    }
    if (!j.End()) {
        r.status = Bad("trailing bytes after safetensors header");
        return r;
    }
    if (r.header.tensors.empty()) {
        r.status = Bad("safetensors file holds no tensors");
        return r;
    }
    std::sort(spans.begin(), spans.end());
    uint64_t at = 0;
    for (const auto& [b, e] : spans) {
        if (b != at) {
            r.status = Bad("tensor data offsets are not contiguous");
            return r;
        }
        at = e;
    }
    if (at != data_section_size) {
        r.status = Bad("tensor data does not cover the data section");
        return r;
    }
    return r;
}

SafetensorsFile::~SafetensorsFile() { Close(); }

SafetensorsFile::SafetensorsFile(SafetensorsFile&& o) noexcept { *this = std::move(o); }

SafetensorsFile& SafetensorsFile::operator=(SafetensorsFile&& o) noexcept {
    if (this != &o) {
        Close();
        header_ = std::move(o.header_);
        map_base_ = o.map_base_;
        map_size_ = o.map_size_;
        data_ = o.data_;
        data_size_ = o.data_size_;
        o.map_base_ = nullptr;
        o.map_size_ = 0;
        o.data_ = nullptr;
        o.data_size_ = 0;
    }
    return *this;
}

void SafetensorsFile::Close() {
    if (map_base_ != nullptr) munmap(map_base_, map_size_);
    map_base_ = nullptr;
    map_size_ = 0;
    data_ = nullptr;
    data_size_ = 0;
    header_ = SafetensorsHeader{};
}

Status SafetensorsFile::Open(const std::string& path, uint64_t max_header_bytes) {
    Close();
    // A symlink is refused (O_NOFOLLOW), and so is anything but a regular
    // file (a FIFO or device would block or lie about its size).
    const int fd = ::open(path.c_str(), O_RDONLY | O_NOFOLLOW | O_CLOEXEC | O_NONBLOCK);
    if (fd < 0) return Status(ErrorCode::kArtifactVerificationFailed, "cannot open weight file", kComponent);
    struct stat st;
    if (fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        ::close(fd);
        return Bad("weight file is not a regular file");
    }
    if (st.st_size < 8) {
        ::close(fd);
        return Bad("weight file too small");
    }
    const size_t size = size_t(st.st_size);
    void* base = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (base == MAP_FAILED) return Status(ErrorCode::kArtifactVerificationFailed, "cannot map weight file", kComponent);
    const uint8_t* p = static_cast<const uint8_t*>(base);
    uint64_t hlen = 0;
    for (int i = 0; i < 8; ++i) hlen |= uint64_t(p[i]) << (8 * i);
    if (hlen > max_header_bytes || hlen > size - 8) {
        munmap(base, size);
        return Bad("safetensors header length out of range");
    }
    HeaderParseResult r = ParseSafetensorsHeader(
        std::string_view(reinterpret_cast<const char*>(p + 8), size_t(hlen)), size - 8 - hlen);
    if (!r.status.ok()) {
        munmap(base, size);
        return r.status;
    }
    header_ = std::move(r.header);
    map_base_ = base;
    map_size_ = size;
    data_ = p + 8 + hlen;
    data_size_ = size - 8 - hlen;
    return Status::Ok();
}

const TensorInfo* SafetensorsFile::FindTensor(const std::string& name) const {
    auto it = header_.tensors.find(name);
    return it == header_.tensors.end() ? nullptr : &it->second;
}

const uint8_t* SafetensorsFile::TensorData(const std::string& name) const {
    const TensorInfo* info = FindTensor(name);
    return info == nullptr || data_ == nullptr ? nullptr : data_ + info->data_offset;
}

}  // namespace lykuro::nie
