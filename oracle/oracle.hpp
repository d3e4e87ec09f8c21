// oracle.hpp -- CPU restatement of the reference engine's Q8_0 Qwen 3.5 hybrid
// forward pass (flywithfang/hero, engine `nm/`), with runtime dimensions.
//
// TEST INFRASTRUCTURE ONLY. This library is the parity checker and the timed
// CPU baseline. It is never linked into, loaded by, or called from the product
// path (hero_amd/): only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg may use it, and only as the checker.
//
// Every function restates one reference function with the SAME fp32 operation
// order (no FMA contraction: build with -ffp-contract=off), so that a pinned
// result from the reference compiled with the same flags matches bit for bit.
// Citations are file:line into nm/src of the reference.
//
// Parity status per function (what pins it; tests/test_oracle_golden.py holds
// the golden-vector checks, tests/test_oracle_properties.py the closed forms):
//   fp16 codec            exhaustive 2^16 decode check + nearest-ties-away encode sweep + golden vectors
//   quantize_row_q8_0     golden vectors from the compiled reference
//   quantize_q8_0         golden vectors + round trip within one quantum, |q| <= 127, zero block
//   vec_dot_q8_0_q8_0     golden vectors; int32 block sums by brute force
//   rmsnorm / l2 / silu   golden vectors + scale invariance, row = batch, float64 closed form
//   conv_step             golden vectors + closed form 100/210/321
//   gated_delta_step      golden vectors + associative-memory identities + float64 brute force
//                         (tiled key heads h % Hk, Hk != Hv)
//   rope                  golden vectors (8 positions to 65535) + offset identity, position 0
//   attention             golden vectors (scale 1/sqrt(128) and 1) + the reference's own
//                         Full / Local (ring, width 3 and 1024) caches at 12 probes + hand-worked
//                         causal / window-of-one cases + float64 brute force (grouped K/V heads)
//   Q4_K / Q6_K dots      golden vectors from the compiled reference
//   dot_block_q5_K        golden vectors from the compiled reference + float64 dequant-dot
//   dequant_row (K-quants) golden rows from the compiled reference + integer decode of the
//                         packed fields written independently in the test
//   Qwen35 forward        golden logits and greedy ids of the tiny Q8_0 model, of its variant
//                         with 4 key heads over 8 value heads and an untied output.weight, of
//                         the tiny model with Q4_K/Q5_K/Q6_K/Q8_0 tensors (a Q4_K_M mix), and
//                         the greedy ids of the ~8B model (600-token prompt, 32 passes)
#pragma once
#include <cstddef>
#include <cstdint>
#include <vector>

namespace oracle {

// ---- fp16 codec (nm/src/core.hpp:34-79) ------------------------------------
float fp16_to_fp32(uint16_t h);
uint16_t fp32_to_fp16(float f);

// ---- K-quant blocks (nm/src/quant.hpp:52,63-86; nm/src/quant_i8.hpp:22-28) -----
// Super-blocks of 256 weights. Q4_K: fp16 d, dmin, 12 bytes of packed 6-bit
// scales/mins, 128 bytes of nibbles (144). Q6_K: 128 bytes low nibbles, 64
// bytes of 2-bit high parts, 16 int8 scales, fp16 d (210). Activations go to
// Q8_K: fp32 d, 256 int8, 16 int16 sums of 16 (292).
#pragma pack(push, 1)
struct BlockQ4K {
    uint16_t d, dmin;
    uint8_t scales[12];
    uint8_t qs[128];
};
struct BlockQ6K {
    uint8_t ql[128];
    uint8_t qh[64];
    int8_t scales[16];
    uint16_t d;
};
struct BlockQ8K {
    float d;
    int8_t qs[256];
    int16_t bsums[16];
};
// Q5_K (nm/src/quant.hpp:70-76): Q4_K's scales plus a fifth bit per weight in
// qh (bit j of qh[l] for element l of 32-element sub-block j): 176 bytes
struct BlockQ5K {
    uint16_t d, dmin;
    uint8_t scales[12];
    uint8_t qh[32];
    uint8_t qs[128];
};
#pragma pack(pop)
static_assert(sizeof(BlockQ4K) == 144 && sizeof(BlockQ5K) == 176 && sizeof(BlockQ6K) == 210 && sizeof(BlockQ8K) == 292, "K-quant block sizes");

// activation quantizer for K-quant weights (nm/src/quant_i8.hpp:31-64)
void quantize_row_q8_K(const float* x, BlockQ8K* y, size_t k);
// the x86 (scalar) dots (nm/src/quant_i8.hpp:146-191, 239-278)
float vec_dot_q4_K_q8_K(size_t n, const BlockQ4K* w, const BlockQ8K* x);
float vec_dot_q6_K_q8_K(size_t n, const BlockQ6K* w, const BlockQ8K* x);
// Weight::matvec / ::matmul for Q4_K (type 12) and Q6_K (type 14): T rows of
// X quantized to Q8_K, each output = the dot above (nm/src/quant_i8.hpp:352-383,430-474)
void matmul_kquant(int type, const void* W, size_t N, size_t K, const float* X, size_t T, float* Y);
// Q5_K has no integer-activation kernel (has_i8_kernel, nm/src/quant_i8.hpp:325):
// the fp32-activation dequant-in-dot of one block (nm/src/quant.hpp:207-229)
// and its row sum over blocks in order (nm/src/quant_i8.hpp:403-407)
float dot_block_q5_K(const BlockQ5K& b, const float* x);
void matmul_q5_K(const BlockQ5K* W, size_t N, size_t K, const float* X, size_t T, float* Y);
// one row of a Q4_K (12) / Q5_K (13) / Q6_K (14) / Q8_0 (8) tensor as fp32
// (dequant_to_f32, nm/src/quant.hpp:291-400)
void dequant_row(int type, const void* row, float* out, size_t k);
// bytes of one row of k elements of a ggml type (8, 12, 13, 14)
size_t row_bytes(int type, size_t k);

// ---- sampling (nm/src/logits.hpp:71-105) -----------------------------------------
// Logits::sample with temp > 0, given u = the uniform draw the caller's RNG
// makes for std::uniform_real_distribution<float>(0, s2) (libstdc++:
// r = u * (s2 - 0) + 0 with u = generate_canonical<float, 24>(rng)).
// Candidates are ordered by logit, descending; equal logits by ascending id.
int32_t sample_topk(const float* logits, size_t V, size_t top_k, float temp, float top_p, float u);

// ---- Q8_0 block (nm/src/quant.hpp:59-62): fp16 d + 32 int8, 34 bytes ------
#pragma pack(push, 1)
struct BlockQ8 {
    uint16_t d;
    int8_t qs[32];
};
#pragma pack(pop)
static_assert(sizeof(BlockQ8) == 34, "Q8_0 block is 34 bytes");

// activation quantizer, roundf (nm/src/quant_i8.hpp:70-80)
void quantize_row_q8_0(const float* x, BlockQ8* y, size_t k);
// weight quantizer, lround (nm/src/quant.hpp:404-413)
void quantize_q8_0(const float* x, BlockQ8* y, size_t n);
// integer dot, sequential fp32 block combination (nm/src/quant_i8.hpp:85-100)
float vec_dot_q8_0_q8_0(size_t n, const BlockQ8* w, const BlockQ8* x);
// d*q row dequant (nm/src/quant.hpp:306-313)
void dequant_row_q8_0(const BlockQ8* row, float* out, size_t k);

// ---- the row-parallel pool (nm/src/core.cpp:22-117) -----------------------
// Persistent pool of N-1 workers plus the caller; chunk = n/(threads*16);
// nested calls run serially. Threads default to hardware_concurrency and can
// be set with set_threads() (the reference reads NM_THREADS).
void par_for(size_t n, void (*fn)(size_t, void*), void* ctx);
size_t num_threads();
void set_threads(size_t n);

// y[N] = W[N,K] x (nm/src/quant_i8.hpp:352-383): x quantized once, serially.
void matvec_q8_0(const BlockQ8* W, size_t N, size_t K, const float* x, float* y);
// Y[T,N] = X[T,K] W^T (nm/src/quant_i8.hpp:430-474)
void matmul_q8_0(const BlockQ8* W, size_t N, size_t K, const float* X, size_t T, float* Y);

// ---- elementwise / small reductions ----------------------------------------
float dot(const float* a, const float* b, size_t n);          // core.hpp:496-500
float sigmoid(float x);                                         // core.hpp:579
float silu(float x);                                            // components.hpp:105
float softplus(float x);                                        // recurrent.hpp:35
void rmsnorm(float* x, const float* gamma, size_t n, float eps);  // components.hpp:176-181
void l2_normalize(const float* x, float* out, size_t n, float eps);  // recurrent.hpp:40-48
void softmax(float* v, size_t n);                               // components.hpp:132-141

// depthwise causal conv step (recurrent.hpp:75-106). history holds the last
// (width-1) inputs, oldest first, [width-1][channels]; taps are [channels][width].
void conv_step(const float* input, const float* taps, float* history, float* out, size_t channels, size_t width);

// one head, one token, in place (recurrent.hpp:146-177)
void gated_delta_step(float* state, const float* q, const float* k, const float* v, float gate, float beta, float* out, size_t dk, size_t dv);

// RoPE inv_freq table (attention.hpp:76-80) and one head rotation (:82-91)
std::vector<float> rope_inv_freq(size_t head_dim, double base, size_t rotary_dims);
void rope_apply(float* head, const float* inv_freq, size_t head_dim, size_t position);

// GQA decode/prefill reduction for one (query row, head):
// softmax(scale * q.k_j) over rows [first, end), then sum alpha_j v_j
// (qwen35.hpp:366-380 with scale 1/sqrt(Dh); gemma4.hpp:597-610 with scale 1).
// keys/values are [rows][kv_width] with the head at offset kv_head*head_dim.
void attend_one(const float* q, const float* keys, const float* values, size_t kv_width, size_t kv_head, size_t head_dim, size_t first, size_t end, float scale, float* out);

// ---- the Qwen 3.5 hybrid model (qwen35.hpp:26-463) --------------------------
struct Config {
    size_t V = 0, D = 0, L = 0, CTX = 0;
    size_t Hq = 0, Hkv = 0, head_dim = 0, rotary_dims = 0;
    double rope_base = 0;
    size_t Dk = 0, Dv = 0, Hk = 0, Hv = 0, conv_width = 0;
    size_t FF = 0;
    float eps = 0;
    size_t full_attention_interval = 4;
    bool tied = true;
    bool is_recurrent(size_t layer) const { return (layer + 1) % full_attention_interval != 0; }
    size_t conv_channels() const { return 2 * Hk * Dk + Hv * Dv; }
};

// A linear weight as stored in the GGUF, row-major by output: N rows of K
// elements of ggml type `type` (8 Q8_0, 12 Q4_K, 13 Q5_K, 14 Q6_K).
struct Linear {
    const void* w = nullptr;
    int type = 8;
    size_t N = 0, K = 0;
};
// Weight::matmul (nm/src/quant_i8.hpp:415-495): the integer-activation form
// for Q8_0 / Q4_K / Q6_K, the fp32-activation form for Q5_K
void linear_rows(const Linear& lin, const float* X, size_t T, float* Y);

struct Layer {
    std::vector<float> mixer_norm, channel_norm;  // [D]
    Linear gate, up, down;
    // attention mixer
    Linear wqg, wk, wv, wo;
    std::vector<float> q_norm, k_norm;  // [head_dim]
    // delta-net mixer
    Linear wqkv, wz, wbeta, walpha, wout;
    std::vector<float> conv;         // [conv_channels][conv_width]
    std::vector<float> dt_bias;      // [Hv]
    std::vector<float> decay_scale;  // [Hv], -exp(A_log)
    std::vector<float> ssm_norm;     // [Dv]
};

struct Model {
    Config c;
    Linear embedding;  // [V rows of D]
    Linear output;     // untied head, or embedding when tied
    std::vector<Layer> layers;
    std::vector<float> final_norm;
    std::vector<float> inv_freq;
};

struct State {
    size_t tokens = 0;
    // diagnosis switch (not in the reference, whose cache is fp32): store the
    // attention keys and values rounded to IEEE fp16, nearest-even, as the
    // GPU's fp16 paged cache does; reset() keeps it
    bool kv_fp16 = false;
    // the same for Q8_0 storage (the reference's plan, nm/INFERENCE_PLAN.md:235-236):
    // each appended K and V row goes through quantize_row_q8_0 (the activation
    // quantizer) and is kept as its dequantized values d * q; reset() keeps it
    bool kv_q8 = false;
    // attention layers: fp32 K/V rows [tokens][Hkv*head_dim]
    std::vector<std::vector<float>> keys, values;
    // recurrent layers: conv history [(W-1)][CC] oldest first, delta state [Hv][Dk][Dv]
    std::vector<std::vector<float>> conv_hist, delta;
    void reset(const Config& c);
};

// IEEE binary16 rounding (nearest even) of fp32 values, returned as fp32:
// the storage of the fp16 attention cache. Not the reference's fp16 encoder,
// whose ties go away from zero (core.hpp:61-79).
float round_fp16_rne(float x);

// gather_rows / dequant_row (quant.hpp:464-480)
void embed(const Model& m, const int32_t* ids, size_t n, float* out);
// Qwen35Model::forward (qwen35.hpp:288-303): rows [T][D] at state.tokens(),
// writes logits [V] of the last row. Throws on context exhaustion.
void forward(const Model& m, State& s, const float* rows, size_t T, float* logits);
// Logits::argmax: ties go to the lowest id (logits.hpp:61-66)
int32_t argmax(const float* logits, size_t n);

// ---- Gemma 4 text, E4B schema (gemma4.hpp:19-482, gemma4_loader.hpp:31-130) ----
// Dimensions from the GGUF; the schedule is the reference's: layer l attends
// over the whole context when l % 6 == 5, over a sliding window otherwise; the
// last `shared` layers read the caches of the last earlier layer of their kind.
struct Gemma4Config {
    size_t V = 0, D = 0, L = 0, CTX = 0, FF = 0;
    size_t Hq = 0, Hkv = 0, Dl = 0, Df = 0, P = 0;
    size_t window = 0, shared = 0, local_rot = 0, full_rot = 0;
    double local_base = 0, full_base = 0;
    float eps = 0, softcap = 0;
    bool full(size_t l) const { return l % 6 == 5; }                    // gemma4.hpp:37
    bool shares_kv(size_t l) const { return l >= L - shared; }          // gemma4.hpp:38
    size_t head_dim(size_t l) const { return full(l) ? Df : Dl; }
    size_t kv_source(size_t l) const;                                   // gemma4.hpp:41-47, 370-373
};

struct Gemma4Layer {
    std::vector<float> attn_norm, q_norm, k_norm, post_attn_norm, ffn_norm, post_ffn_norm, post_norm;
    Linear wq, wk, wv, wo, gate, up, down, pgate, proj;
    float out_scale = 1.f;  // layer_output_scale (gemma4_loader.hpp:56-63: 1 when absent)
};

struct Gemma4Model {
    Gemma4Config c;
    Linear embedding;  // [V rows of D], also the tied LM head
    Linear ple_table;  // [V rows of P*L]
    Linear ple_proj;   // [P*L rows of D]
    std::vector<float> ple_norm, final_norm;
    std::vector<Gemma4Layer> layers;
    std::vector<float> inv_local, inv_full;
};

struct Gemma4State {
    size_t tokens = 0;
    // per layer that owns K/V: rows [tokens][Hkv*dh] (the window layers' rings
    // hold the same rows; visibility is the window rule)
    std::vector<std::vector<float>> keys, values;
    void reset(const Gemma4Config& c);
};

// gelu_pytorch_tanh (components.hpp:73-81)
float gelu_tanh(float v);
// cap * tanh(v / cap) (gemma4.hpp:79)
float gemma_softcap(float v, float cap);
// Gemma4E4BModel::embed (gemma4.hpp:415-419): dequant_row * sqrt(D)
void gemma4_embed(const Gemma4Model& m, const int32_t* ids, size_t n, float* out);
// Gemma4E4BModel::forward (gemma4.hpp:424-445) over T token ids at
// state.tokens: the batched form (every layer over all T rows); writes the
// soft-capped logits [V] of the last row. Throws on context exhaustion.
void gemma4_forward(const Gemma4Model& m, Gemma4State& s, const int32_t* ids, size_t T, float* logits);

}  // namespace oracle
