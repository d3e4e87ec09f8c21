// model.hpp -- the GPU Qwen 3.5 hybrid model: the C++ side of the drop-in.
//
// Mirrors the reference's model contract (nm/src/transformer.hpp:70-78):
//   Qwen35Model::open(gguf)        <- qwen35_loader::load<C> (qwen35_loader.hpp:141-155)
//   model.new_state(max_tokens)    <- Qwen35State<C> (qwen35.hpp:206-241)
//   state.tokens()                 <- PrefixState::tokens()
//   model.embed(ids, n, rows)      <- Qwen35Model::embed (qwen35.hpp:285)
//   model.forward(state, rows|ids) <- Qwen35Model::forward (qwen35.hpp:288-303)
// Dimensions are read from the GGUF metadata at run time (the reference fixes
// them at compile time) and validated the way validate_metadata does.
// The model is immutable after load and non-copyable; a State belongs to one
// sequence and one caller thread.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "hero/kernels.hpp"

namespace hero {

class GgufFile;
struct WeightPacker;

struct ModelConfig {
    int64_t V = 0, D = 0, L = 0, CTX = 0;
    int64_t Hq = 0, Hkv = 0, Dh = 0, rotary_dims = 0;
    int64_t Dk = 0, Dv = 0, Hk = 0, Hv = 0, W = 0;
    int64_t FF = 0;
    double rope_base = 0;
    float eps = 0;
    bool tied = true;
    bool is_recurrent(int64_t layer) const { return (layer + 1) % 4 != 0; }
    int64_t conv_channels() const { return 2 * Hk * Dk + Hv * Dv; }
    int64_t q_width() const { return Hq * Dh; }
    int64_t kv_width() const { return Hkv * Dh; }
    int64_t v_width() const { return Hv * Dv; }
};

// Owning device allocation.
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t bytes);
    ~DeviceBuffer();
    DeviceBuffer(DeviceBuffer&& o) noexcept : p_(o.p_), bytes_(o.bytes_) {
        o.p_ = nullptr;
        o.bytes_ = 0;
    }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept;
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    template <class T = void>
    T* get() const {
        return static_cast<T*>(p_);
    }
    size_t bytes() const { return bytes_; }

private:
    void* p_ = nullptr;
    size_t bytes_ = 0;
};

// One linear weight of a model with K-quant tensors, kept in the tensor's
// own type: packed Q8_0 (type 8), packed Q4_K (12) / Q6_K (14), or Q5_K (13).
struct TypedLinear {
    DeviceBuffer w;
    int type = 8;
    int64_t N = 0, K = 0;
};

struct LayerWeights {
    bool recurrent = true;
    DeviceBuffer mixer_norm, channel_norm;  // [D] fp32
    DeviceBuffer w_in;                      // packed Q8_0, K = D
    int64_t n_in = 0;
    DeviceBuffer w_out;                     // packed Q8_0 [D][Hv*Dv or Hq*Dh]
    DeviceBuffer w_gate_up;                 // packed Q8_0 [2FF][D]: gate rows then up rows
    DeviceBuffer w_down;                    // packed Q8_0 [D][FF]
    // recurrent: w_in rows = [qkv CC | z Hv*Dv | beta Hv | alpha Hv]
    DeviceBuffer conv, dt_bias, decay, ssm_norm;
    int64_t z_off = 0, beta_off = 0, alpha_off = 0;
    // attention: w_in rows = [q|gate pairs 2*Hq*Dh | k Hkv*Dh | v Hkv*Dh]
    DeviceBuffer q_norm, k_norm;
    int64_t k_off = 0, v_off = 0;
    // K-quant models: every linear in its own type (the packed Q8_0 buffers
    // above stay empty). tin[i] writes proj columns [tin_off[i], + tin[i].N):
    // recurrent qkv, z, beta, alpha; attention q|gate, k, v
    std::vector<TypedLinear> tin;
    std::vector<int64_t> tin_off;
    TypedLinear tout, tgate, tup, tdown;
};

class Qwen35Model {
public:
    class State;
    static constexpr int64_t kMaxBatch = 16;    // sequences per state (the skinny GEMM's rows)
    static constexpr int64_t kPageTokens = 64;  // positions per page of the paged attention cache
    // attention cache formats: the reference's fp32 rows (exact), fp16 pages
    // or Q8_0 pages (split-K attention over either)
    enum KvFormat : int { kKvF32 = 0, kKvF16 = 1, kKvQ8 = 2 };

    static std::unique_ptr<Qwen35Model> open(const std::string& gguf_path);
    static std::unique_ptr<Qwen35Model> open_image(const uint8_t* image, uint64_t size);
    ~Qwen35Model();
    Qwen35Model(const Qwen35Model&) = delete;
    Qwen35Model& operator=(const Qwen35Model&) = delete;

    const ModelConfig& config() const { return c_; }
    int64_t device_bytes() const { return device_bytes_; }
    hipStream_t stream() const { return stream_; }

    // `batch` independent sequences of up to `max_tokens` each; `kv_format`
    // keeps the attention cache as the reference's fp32 rows, or as fp16 /
    // Q8_0 pages (split-K attention); gdn_chunked runs the delta-net prefill
    // in its chunked form (tolerance-equal to the token-serial recurrence
    // instead of bit-equal)
    std::unique_ptr<State> new_state(int64_t max_tokens, int64_t batch = 1, int kv_format = kKvF32, bool gdn_chunked = false) const;
    // host rows out[n][D]
    void embed(const int32_t* ids, int64_t n, float* out) const;
    // T rows from host `rows` or from `ids`; logits / greedy id of the last row
    void forward(State& s, const float* rows, const int32_t* ids, int64_t T, float* logits, int32_t* next_id) const;
    // the same for sequence `seq` of a batch state
    void forward_seq(State& s, int64_t seq, const float* rows, const int32_t* ids, int64_t T, float* logits, int32_t* next_id) const;
    // greedy loop from `first_id`; out_ids[steps] on the host
    void decode_greedy(State& s, int32_t first_id, int64_t steps, int32_t* out_ids, float* logits) const;
    // greedy loop of every sequence of a batch state at once, each from its own
    // position: first_ids[B]; out_ids[steps][B]; logits [B][V] of the last pass
    void decode_batch(State& s, const int32_t* first_ids, int64_t steps, int32_t* out_ids, float* logits) const;
    double last_decode_seconds() const { return last_decode_seconds_; }
    // true when some linear weight is not Q8_0 (Q4_K / Q5_K / Q6_K): every
    // linear then runs in its own type, one product per tensor
    bool typed() const { return typed_; }
    // Every Q8_0 matvec of one decode step (all layers + LM head), `reps`
    // times back to back, between two events on the model's stream.
    // Returns seconds; *launches and *bytes are per repetition (algorithmic
    // bytes: weights + scales, activation, outputs, residual reads).
    double time_gemvs(State& s, int reps, int64_t* launches, int64_t* bytes) const;

private:
    Qwen35Model() = default;
    void load(const GgufFile& g);
    void load_typed(const GgufFile& g, WeightPacker& pk);
    void build_rope_table(int64_t positions);
    // one token at the state's device position; `with_head` adds the final
    // norm, LM head and argmax (the reference computes logits for the last row only)
    void enqueue_step(State& s, bool from_ids, bool with_head) const;
    // T rows of one sequence at positions pos0 .. pos0+T-1, already in the
    // state's chunk input rows: each layer as batched GEMMs around the
    // token-serial delta-net and the causal attention; `with_head` adds the
    // final norm, LM head and argmax of the last row
    void enqueue_chunk(State& s, int64_t seq, int64_t pos0, int64_t T, bool with_head) const;
    // one token of every sequence of a batch state (positions and ids on the
    // device): the matvecs as skinny GEMMs over the B rows
    void enqueue_batch_step(State& s) const;
    // attention of rows a.B (their positions in a.positions): fp32 rows, or
    // the fp16 pages of the sequences whose page-table rows start at `pt`
    void attention(State& s, size_t layer, AttnDecodeArgs a, const int32_t* pt, float* work, hipStream_t stream) const;
    // rows per prefill chunk: at most 512, and the chunk's attention scores
    // (rows x query heads x max_tokens fp32) within 256 MiB
    int64_t chunk_rows(const State& s) const;
    // ---- models with K-quant tensors ----
    struct TypedScratch;
    // y[m * ldy + n] (+ resid, same stride) = the M fp32 rows x [M][K] times
    // W^T, in the reference's arithmetic for W's type
    void typed_linear(const TypedLinear& w, const float* x, int64_t M, float* y, int64_t ldy, const float* resid, TypedScratch& ts,
                      hipStream_t s) const;
    // the layers over M rows in x: one token of one sequence (chunk = false,
    // position positions[0]) or M consecutive tokens of sequence `seq` (chunk)
    void typed_layers(State& st, TypedScratch& ts, float* x, float* h, float* proj, float* gate_up, int64_t M, const int32_t* positions, int64_t seq,
                      bool chunk, hipStream_t s) const;
    void typed_head(State& st, TypedScratch& ts, const float* x_last, hipStream_t s) const;
    void embed_rows(const int32_t* ids, int64_t n, float* out, hipStream_t s) const;

    ModelConfig c_;
    std::vector<LayerWeights> layers_;
    DeviceBuffer embedding_, output_, final_norm_, rope_cs_;
    // d_model 4096: gate and up packed in alternating 32-row chunks, so the
    // gate/up GEMV ends in SwiGLU and writes the down projection's input
    bool ffn_fused_ = false;
    bool typed_ = false;
    TypedLinear t_embedding_, t_output_;  // typed models; t_output_ empty when tied
    int64_t rope_positions_ = 0;
    int64_t device_bytes_ = 0;
    hipStream_t stream_ = nullptr;
    hipEvent_t ev_start_ = nullptr, ev_stop_ = nullptr;
    mutable double last_decode_seconds_ = 0;
};

class Qwen35Model::State {
public:
    ~State();
    int64_t tokens() const { return seq_tokens_[0]; }
    int64_t tokens(int64_t seq) const { return seq_tokens_.at(size_t(seq)); }
    int64_t max_tokens() const { return max_tokens_; }
    int64_t batch() const { return batch_; }
    void reset();

private:
    friend class Qwen35Model;
    explicit State(const Qwen35Model& m, int64_t max_tokens, int64_t batch, int kv_format);

    const Qwen35Model& m_;
    int64_t max_tokens_ = 0, batch_ = 1;
    // paged attention cache (fp16 or Q8_0 rows): per attention layer a pool
    // of batch x max_pages pages; page_table_ [batch][max_pages] (sequence b
    // owns pages b * max_pages ...); attn_work_ the split-K partials of a step
    bool kv_paged_ = false, kv_q8_ = false, gdn_chunked_ = false;
    int64_t max_pages_ = 0;
    std::vector<DeviceBuffer> kv_pages_;
    DeviceBuffer page_table_, attn_work_;
    std::vector<int64_t> seq_tokens_;
    // batch step scalars: [0, B) positions, [B, 2B) token ids, [2B] step counter
    DeviceBuffer bstep_;
    hipGraphExec_t bgraph_ = nullptr;  // one batch greedy step, replayed
    // per-step device scalars: [0] position, [1] token id, [2] step counter
    DeviceBuffer step_;
    DeviceBuffer x_, h_, proj_, act_d_, act_mix_, act_ff_, gate_up_, logits_, argmax_scratch_, out_ids_, q_rot_;
    DeviceBuffer o_raw_;  // [B][Hv*Dv] raw delta-net outputs of a decode step (before the head norm)
    DeviceBuffer g_raw_;  // [B][Hv*Dv] its output gates silu(z)
    DeviceBuffer gemv_scratch_;  // [D] output of the GEMV timing runs
    int64_t out_ids_capacity_ = 0;
    // prefill chunk buffers (row-major, chunk_capacity_ rows), made on first use
    DeviceBuffer cx_, ch_, cproj_, cact_d_, cact_mix_, cgate_up_, cact_ff_, cq_rot_, cscores_, cpos_, cids_, cgdn_work_, cattn_work_;
    int64_t chunk_capacity_ = 0;
    void ensure_chunk(int64_t rows);
    // per layer, every sequence's: [B][...]
    std::vector<DeviceBuffer> k_cache_, v_cache_, scores_, conv_hist_, delta_;
    // models with K-quant tensors: fp32 intermediates and activation scratch
    // of a decode step and of a prefill chunk
    std::unique_ptr<TypedScratch> tstep_, tchunk_;
    hipGraphExec_t graph_ = nullptr;  // one greedy decode step, replayed
};

}  // namespace hero
