// oracle_gguf.hpp -- GGUF v3 reader + Qwen 3.5 loader for the oracle.
// TEST INFRASTRUCTURE ONLY (see oracle.hpp).
#pragma once
#include "oracle.hpp"

#include <map>
#include <string>
#include <vector>

namespace oracle {

class Gguf {
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
        std::vector<uint64_t> dims;
        uint32_t type = 0;
        uint64_t offset = 0, nelem = 0;
        const uint8_t* data = nullptr;
    };

    Gguf() = default;
    ~Gguf();
    Gguf(const Gguf&) = delete;
    Gguf& operator=(const Gguf&) = delete;

    void open(const std::string& path);                // mmap a file
    void parse(const uint8_t* base, size_t size);      // a caller-owned image

    bool has(const std::string& k) const { return meta_.count(k) != 0; }
    double num(const std::string& k) const;
    std::string str(const std::string& k) const {
        auto it = meta_.find(k);
        return it == meta_.end() ? std::string("?") : it->second.str;
    }
    const std::map<std::string, Value>& meta() const { return meta_; }
    const Tensor* find(const std::string& name) const;
    const Tensor& require(const std::string& name) const;

private:
    const uint8_t* base_ = nullptr;
    size_t size_ = 0;
    void* map_ = nullptr;
    size_t map_size_ = 0;
    int fd_ = -1;
    std::map<std::string, Value> meta_;
    std::vector<Tensor> tensors_;
};

Model load_qwen35(const Gguf& g);
// gemma4_loader::load_e4b_text (gemma4_loader.hpp:31-52, 105-130)
Gemma4Model load_gemma4(const Gguf& g);

}  // namespace oracle
