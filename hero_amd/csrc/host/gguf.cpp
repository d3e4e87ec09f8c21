// gguf.cpp -- GGUF v3 parsing for the host loader (see hero/gguf.hpp).
#include "hero/gguf.hpp"

#include <cstring>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "hero/errors.hpp"
#include "hero_kernels.h"

namespace hero {

namespace {
[[noreturn]] void fail(const std::string& what) { throw Error(HERO_EIO, "GGUF: " + what); }

struct Reader {
    const uint8_t* p;
    const uint8_t* end;
    template <class T>
    T get() {
        if (uint64_t(end - p) < sizeof(T)) fail("truncated file");
        T v;
        std::memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string text() {
        const uint64_t n = get<uint64_t>();
        if (uint64_t(end - p) < n) fail("truncated file");
        std::string s(reinterpret_cast<const char*>(p), size_t(n));
        p += n;
        return s;
    }
    double number(uint32_t t) {
        switch (t) {
            case 0: return get<uint8_t>();
            case 1: return get<int8_t>();
            case 2: return get<uint16_t>();
            case 3: return get<int16_t>();
            case 4: return get<uint32_t>();
            case 5: return get<int32_t>();
            case 6: return get<float>();
            case 7: return get<uint8_t>() != 0;
            case 10: return double(get<uint64_t>());
            case 11: return double(get<int64_t>());
            case 12: return get<double>();
            default: fail("bad value type");
        }
    }
};

uint64_t tensor_bytes(uint32_t type, uint64_t n, const std::string& name) {
    switch (type) {
        case 0: return n * 4;
        case 1: return n * 2;
        case 8:
            if (n % 32) fail("tensor '" + name + "' has a partial quant block");
            return n / 32 * 34;
        case 12:  // Q4_K, Q5_K, Q6_K: super-blocks of 256 (nm/src/quant.hpp:52-86)
        case 13:
        case 14:
            if (n % 256) fail("tensor '" + name + "' has a partial quant block");
            return n / 256 * (type == 12 ? 144 : type == 13 ? 176 : 210);
        default: fail("tensor '" + name + "' has ggml type " + std::to_string(type) + "; this path reads F32, F16, Q8_0, Q4_K, Q5_K and Q6_K");
    }
}
}  // namespace

GgufFile::~GgufFile() {
    if (map_) ::munmap(map_, map_size_);
    if (fd_ >= 0) ::close(fd_);
}

void GgufFile::open(const std::string& path) {
    fd_ = ::open(path.c_str(), O_RDONLY);
    if (fd_ < 0) fail("cannot open " + path);
    struct stat st{};
    if (::fstat(fd_, &st) != 0) fail("fstat failed");
    map_size_ = uint64_t(st.st_size);
    map_ = ::mmap(nullptr, map_size_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (map_ == MAP_FAILED) {
        map_ = nullptr;
        fail("mmap failed");
    }
    parse(static_cast<const uint8_t*>(map_), map_size_);
}

void GgufFile::parse(const uint8_t* image, uint64_t size) {
    Reader r{image, image + size};
    if (r.get<uint32_t>() != 0x46554747u) fail("bad magic (not a GGUF file)");
    const uint32_t version = r.get<uint32_t>();
    if (version != 3) fail("unsupported version " + std::to_string(version) + " (expect 3)");
    const uint64_t n_tensors = r.get<uint64_t>();
    const uint64_t n_kv = r.get<uint64_t>();
    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key = r.text();
        Value v;
        v.type = r.get<uint32_t>();
        if (v.type == 8) {
            v.str = r.text();
        } else if (v.type == 9) {
            const uint32_t et = r.get<uint32_t>();
            const uint64_t n = r.get<uint64_t>();
            for (uint64_t j = 0; j < n; ++j) {
                if (et == 8)
                    v.arr_str.push_back(r.text());
                else
                    v.arr_num.push_back(r.number(et));
            }
        } else {
            v.num = r.number(v.type);
        }
        meta_[key] = std::move(v);
    }
    uint64_t align = has("general.alignment") ? uint64_t(num("general.alignment")) : 32;
    if (align == 0) align = 32;
    if (align & (align - 1)) fail("general.alignment is not a power of two");
    for (uint64_t i = 0; i < n_tensors; ++i) {
        Tensor t;
        t.name = r.text();
        const uint32_t nd = r.get<uint32_t>();
        if (nd == 0 || nd > 4) fail("tensor '" + t.name + "' has " + std::to_string(nd) + " dims");
        t.nelem = 1;
        for (uint32_t d = 0; d < nd; ++d) {
            t.dims.push_back(r.get<uint64_t>());
            t.nelem *= t.dims.back();
        }
        t.type = r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
        t.nbytes = tensor_bytes(t.type, t.nelem, t.name);
        tensors_.push_back(std::move(t));
    }
    const uint64_t header_end = uint64_t(r.p - image);
    const uint64_t data_start = (header_end + align - 1) & ~(align - 1);
    if (!tensors_.empty() && data_start > size) fail("data section starts past end of file");
    for (Tensor& t : tensors_) {
        if (t.offset % align) fail("tensor '" + t.name + "' offset is misaligned");
        if (t.offset > size - data_start || t.nbytes > size - data_start - t.offset) fail("tensor '" + t.name + "' data out of range");
        t.data = image + data_start + t.offset;
    }
}

const GgufFile::Value& GgufFile::get(const std::string& key) const {
    auto it = meta_.find(key);
    if (it == meta_.end()) throw Error(HERO_EIO, "qwen35 loader: missing metadata key " + key);
    return it->second;
}

const GgufFile::Tensor* GgufFile::find(const std::string& name) const {
    for (const Tensor& t : tensors_)
        if (t.name == name) return &t;
    return nullptr;
}

const GgufFile::Tensor& GgufFile::require(const std::string& name) const {
    const Tensor* t = find(name);
    if (!t) throw Error(HERO_EIO, "GGUF: required tensor '" + name + "' not found");
    return *t;
}

}  // namespace hero
