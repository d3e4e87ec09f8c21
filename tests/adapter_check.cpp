// adapter_check.cpp -- compiles include/qwen35_gpu.hpp against the reference's
// own headers (nm/src) and instantiates it where the reference's code would:
// the TransformerModel concept, the adapter class and PrefixCache over it.
// Built and run by tests/test_adapter.py in a container that holds the
// reference tree; the binary goes to oracle/_ref/ and is never shipped.
//
//   adapter_check            no GPU needed: the error paths map HERO_* codes
//                            to the reference's exception types
#include "qwen35_gpu.hpp"

#include <cstdio>

#include "transformer.hpp"

// the tiny synthetic shape (the reference ships no such config; its fields
// follow nm/src/qwen35.hpp:26-57)
struct TinyConfig {
    static constexpr size_t V = 32000, D = 1024, L = 4, CTX = 4096;
    static constexpr size_t Hq = 8, Hkv = 2, HEAD_DIM = 128;
    static constexpr size_t ROPE_BASE = 1000000, ROTARY_NUM = 1, ROTARY_DEN = 4;
    static constexpr size_t KEY_HEAD_DIM = 128, VALUE_HEAD_DIM = 128, KEY_HEADS = 8, VALUE_HEADS = 8, CONV_WIDTH = 4;
    static constexpr size_t FF = 2816;
    static constexpr Scalar RMS_EPS = 1e-6f;
    static constexpr size_t FULL_ATTENTION_INTERVAL = 4;
    using OutputWeight = std::monostate;
    static constexpr bool is_recurrent(size_t layer) { return (layer + 1) % FULL_ATTENTION_INTERVAL != 0; }
};

using Model = GpuQwen35Model<TinyConfig>;
static_assert(TransformerModel<Model>, "GpuQwen35Model models the reference's model contract");
static_assert(TransformerModel<GpuQwen35Model<Qwen35_9BConfig>>, "and does so for the reference's own configs");
static_assert(std::is_default_constructible_v<Model::PrefixState> && std::is_move_assignable_v<Model::PrefixState>);
template class GpuQwen35Model<TinyConfig>;
template class PrefixCache<Model>;

int main() {
    int failures = 0;
    try {
        Model m("/nonexistent/model.gguf");
        std::puts("FAIL: opening a missing file did not throw");
        ++failures;
    } catch (const std::runtime_error& e) {
        std::printf("missing file -> std::runtime_error: %s\n", e.what());
    }
    try {
        Model m("/nonexistent/model.gguf", TinyConfig::CTX + 1);
        std::puts("FAIL: a context above the config's did not throw");
        ++failures;
    } catch (const std::invalid_argument& e) {
        std::printf("max_tokens above CTX -> std::invalid_argument: %s\n", e.what());
    }
    try {
        hero_throw(HERO_ERANGE);
        ++failures;
    } catch (const std::length_error&) {
        std::puts("HERO_ERANGE -> std::length_error");
    }
    Model::PrefixState empty;
    if (empty.tokens() != 0) ++failures;
    std::printf("%s\n", failures ? "FAILED" : "OK");
    return failures;
}
