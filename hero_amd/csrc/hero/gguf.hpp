// gguf.hpp -- GGUF v3 reader for the host side of the model (the loader stays
// on the host). Restates the checks of nm/src/gguf.cpp:130-230: magic and
// version, typed metadata, tensor table, the aligned data start, per-tensor
// alignment and bounds. Tensor data are pointers into the mapped file or the
// caller's image; nothing is copied here.
#pragma once
#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace hero {

class GgufFile {
public:
    struct Value {
        uint32_t type = 0;
        double num = 0;
        std::string str;
        std::vector<double> arr_num;
        std::vector<std::string> arr_str;
    };
    struct Tensor {
        std::string name;
        std::vector<uint64_t> dims;  // ggml order: dims[0] is contiguous
        uint32_t type = 0;           // 0 F32, 1 F16, 8 Q8_0
        uint64_t offset = 0, nelem = 0, nbytes = 0;
        const uint8_t* data = nullptr;
    };

    GgufFile() = default;
    ~GgufFile();
    GgufFile(const GgufFile&) = delete;
    GgufFile& operator=(const GgufFile&) = delete;

    void open(const std::string& path);
    void parse(const uint8_t* image, uint64_t size);

    bool has(const std::string& key) const { return meta_.count(key) != 0; }
    const Value& get(const std::string& key) const;
    double num(const std::string& key) const { return get(key).num; }
    std::string str(const std::string& key) const { return has(key) ? get(key).str : std::string(); }
    const Tensor* find(const std::string& name) const;
    const Tensor& require(const std::string& name) const;

private:
    std::map<std::string, Value> meta_;
    std::vector<Tensor> tensors_;
    void* map_ = nullptr;
    uint64_t map_size_ = 0;
    int fd_ = -1;
};

}  // namespace hero
