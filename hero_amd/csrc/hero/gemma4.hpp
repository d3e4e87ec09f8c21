// gemma4.hpp -- the GPU Gemma 4 text model (E4B schema): the C++ side of
// include/hero_gemma4.h.
//
// Mirrors the reference's model contract (nm/src/transformer.hpp:70-78) for
// Gemma4E4BModel (nm/src/gemma4.hpp:386-482):
//   Gemma4Model::open(gguf)      <- gemma4_loader::load_e4b_text (gemma4_loader.hpp:105-130)
//   model.new_state(max_tokens)  <- Gemma4E4BCache (gemma4.hpp:343-378)
//   model.embed(ids, n, rows)    <- Gemma4E4BModel::embed (gemma4.hpp:415-419)
//   model.forward(state, ids)    <- Gemma4E4BModel::forward (gemma4.hpp:424-445)
// Dimensions come from the GGUF metadata, validated the way
// validate_e4b_text_metadata (gemma4_loader.hpp:31-52) checks them against its
// compiled configuration. Rows are run one token at a time; every row attends
// over exactly the positions the reference's batched prefill lets it see, so
// results equal the reference's bit for bit.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "hero/model.hpp"

namespace hero {

class GgufFile;

struct Gemma4Config {
    int64_t V = 0, D = 0, L = 0, CTX = 0, FF = 0;
    int64_t Hq = 0, Hkv = 0, Dl = 0, Df = 0;  // local / full head widths
    int64_t P = 0;                            // per-layer input width
    int64_t window = 0, shared = 0;           // sliding window; layers reusing K/V
    int64_t local_rot = 0, full_rot = 0;      // rotated dims per head
    double local_base = 0, full_base = 0;
    float eps = 0, softcap = 0;
    // nm/src/gemma4.hpp:36-57: every sixth layer attends over the whole
    // context; the last `shared` layers reuse the caches of the last earlier
    // layer of their kind
    bool full(int64_t l) const { return l % 6 == 5; }
    bool shares_kv(int64_t l) const { return l >= L - shared; }
    int64_t head_dim(int64_t l) const { return full(l) ? Df : Dl; }
    int64_t kv_source(int64_t l) const;
};

struct Gemma4Layer {
    bool full = false, shared = false;
    int64_t dh = 0, src = 0;  // head width; the layer whose cache it reads
    DeviceBuffer attn_norm, q_norm, k_norm, post_attn_norm, ffn_norm, post_ffn_norm, post_norm;  // fp32
    DeviceBuffer w_qkv;      // packed Q8_0 [q Hq*dh | k Hkv*dh | v Hkv*dh][D] (q only when shared)
    int64_t n_qkv = 0;
    DeviceBuffer w_o;        // [D][Hq*dh]
    DeviceBuffer w_gate_up;  // [gate FF | up FF][D]
    DeviceBuffer w_down;     // [D][FF]
    DeviceBuffer w_pgate;    // [P][D]   PLE gate
    DeviceBuffer w_proj;     // [D][P]   PLE projection
    float out_scale = 1.f;   // layer_output_scale
};

class Gemma4Model {
public:
    class State;

    static std::unique_ptr<Gemma4Model> open(const std::string& gguf_path);
    static std::unique_ptr<Gemma4Model> open_image(const uint8_t* image, uint64_t size);
    ~Gemma4Model();
    Gemma4Model(const Gemma4Model&) = delete;
    Gemma4Model& operator=(const Gemma4Model&) = delete;

    const Gemma4Config& config() const { return c_; }
    int64_t device_bytes() const { return device_bytes_; }
    std::unique_ptr<State> new_state(int64_t max_tokens) const;
    // host rows out[n][D]
    void embed(const int32_t* ids, int64_t n, float* out) const;
    // T token ids at the state's position; logits / greedy id of the last row
    void forward(State& s, const int32_t* ids, int64_t T, float* logits, int32_t* next_id) const;
    // greedy loop from first_id; out_ids[steps] on the host
    void decode_greedy(State& s, int32_t first_id, int64_t steps, int32_t* out_ids, float* logits) const;
    double last_decode_seconds() const { return last_decode_seconds_; }

private:
    Gemma4Model() = default;
    void load(const GgufFile& g);
    // one token (position and id in the state's step scalars): embedding,
    // per-layer inputs, the layers, then the final norm, tied head, soft-cap
    // and argmax (into the step's id)
    void enqueue_step(State& s) const;

    Gemma4Config c_;
    std::vector<Gemma4Layer> layers_;
    DeviceBuffer embedding_;   // packed Q8_0 [V][D]; also the LM head (tied)
    DeviceBuffer ple_table_;   // packed Q8_0 [V][P*L]
    DeviceBuffer ple_proj_;    // packed Q8_0 [P*L][D]
    DeviceBuffer ple_norm_, final_norm_;
    DeviceBuffer rope_local_, rope_full_;  // [positions][dh/2][2]
    float embed_scale_ = 0, token_scale_ = 0, proj_scale_ = 0, comb_scale_ = 0;
    int64_t rope_positions_ = 0;
    int64_t device_bytes_ = 0;
    hipStream_t stream_ = nullptr;
    hipEvent_t ev_start_ = nullptr, ev_stop_ = nullptr;
    mutable double last_decode_seconds_ = 0;
};

class Gemma4Model::State {
public:
    ~State();
    int64_t tokens() const { return tokens_; }
    int64_t max_tokens() const { return max_tokens_; }
    void reset();

private:
    friend class Gemma4Model;
    State(const Gemma4Model& m, int64_t max_tokens);

    const Gemma4Model& m_;
    int64_t max_tokens_ = 0, tokens_ = 0;
    DeviceBuffer step_;  // [0] position, [1] token id, [2] greedy step counter
    DeviceBuffer x_, h_, h2_, a_, act_, tok_, ctx_, ple_, proj_, q_rot_, scores_, act_o_, gu_, act_ff_, pg_, act_p_;
    DeviceBuffer logits_, argmax_scratch_, out_ids_;
    int64_t out_ids_capacity_ = 0;
    std::vector<DeviceBuffer> k_cache_, v_cache_;  // per layer; empty for layers that reuse another's
    std::vector<int64_t> slots_;
    hipGraphExec_t graph_ = nullptr;  // one greedy step, replayed
};

}  // namespace hero
