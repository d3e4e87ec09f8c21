// synth.hpp -- seeded random-init Qwen 3.5-style hybrid models and Gemma 4
// text models as GGUF images.
#pragma once
#include <cstdint>
#include <string>

namespace hero {

struct SynthConfig {
    uint64_t V = 32000, D = 1024, L = 4, FF = 2816;
    uint64_t Hq = 8, Hkv = 2, head_dim = 128;
    uint64_t Dk = 128, Dv = 128, Hk = 8, Hv = 8, conv_width = 4;
    uint64_t ctx = 4096;
    double rope_base = 1e6;
    bool tied = true;
    uint64_t seed = 1;
    uint32_t weight_mix = 0;  // 0: Q8_0 2-D weights; 1: a Q4_K_M-style mix of Q4_K, Q5_K, Q6_K and Q8_0; 2: Q8_0 projections with K-quant embedding, down and output projections
};

// Gemma 4 text models in the E4B schema (defaults: the E4B shape itself)
struct Gemma4SynthConfig {
    uint64_t V = 262144, D = 2560, L = 42, FF = 10240;
    uint64_t Hq = 8, Hkv = 2, local_dim = 256, full_dim = 512;
    uint64_t ple = 256, window = 512, shared_kv_layers = 18;
    uint64_t ctx = 131072;
    uint64_t seed = 1;
};

uint64_t synth_qwen35_size(const SynthConfig& c);
void synth_qwen35_image(const SynthConfig& c, uint8_t* image, uint64_t capacity);
void synth_qwen35_file(const SynthConfig& c, const std::string& path);
uint64_t synth_gemma4_size(const Gemma4SynthConfig& c);
void synth_gemma4_image(const Gemma4SynthConfig& c, uint8_t* image, uint64_t capacity);
void synth_gemma4_file(const Gemma4SynthConfig& c, const std::string& path);

}  // namespace hero
