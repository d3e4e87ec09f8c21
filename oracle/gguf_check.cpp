// gguf_check.cpp -- TEST INFRASTRUCTURE: parses one GGUF file with the
// product's host reader (hero_amd/csrc/host/gguf.cpp, hero::GgufFile) and with
// the oracle's reader and model loader, and prints what each reported. Built
// by `make -C oracle sanitize` with AddressSanitizer and UndefinedBehavior-
// Sanitizer (any finding aborts), so tests/test_sanitize.py can feed it
// malformed files: both readers take untrusted files and must turn every
// defect into an error, never into an out-of-bounds access.
//
//   gguf_check FILE    exit 0 whatever the file holds (errors are printed);
//                      a sanitizer finding exits non-zero
#include <cstdio>
#include <exception>
#include <string>

#include "hero/gguf.hpp"
#include "oracle_gguf.hpp"

extern "C" {
void* oracle_model_open(const char* path);
void oracle_model_close(void* h);
const char* oracle_last_error();
}

int main(int argc, char** argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: gguf_check FILE\n");
        return 2;
    }
    const std::string path = argv[1];
    try {
        hero::GgufFile g;
        g.open(path);
        // the loader's first queries (qwen35 schema)
        const std::string arch = g.str("general.architecture");
        const hero::GgufFile::Tensor* emb = g.find("token_embd.weight");
        std::printf("hero: ok (%s, token_embd %s)\n", arch.c_str(), emb ? "present" : "absent");
    } catch (const std::exception& e) {
        std::printf("hero: error: %s\n", e.what());
    }
    try {
        oracle::Gguf g;
        g.open(path);
        std::printf("oracle gguf: ok\n");
    } catch (const std::exception& e) {
        std::printf("oracle gguf: error: %s\n", e.what());
    }
    void* m = oracle_model_open(path.c_str());
    if (m) {
        std::printf("oracle model: ok\n");
        oracle_model_close(m);
    } else {
        std::printf("oracle model: error: %s\n", oracle_last_error());
    }
    return 0;
}
