// model.cpp -- load, state and the per-token schedule of the GPU model.
//
// Per token and layer the device runs (all on the model's stream):
//   rmsnorm_quant(x)                       mixer norm + Q8_0 quantize
//   gemv(w_in)                             all input projections of the layer in one matvec
//   gdn_decode | attn_decode               token mixer, emits the quantized W_o input
//   gemv(w_out, residual x)   -> h         h = x + mix(norm(x))      (qwen35.hpp:319-321)
//   rmsnorm_quant(h)                       channel norm
//   gemv(w_gate_up)                        gate and up in one matvec
//   swiglu_quant                           silu(gate)*up, quantized
//   gemv(w_down, residual h)  -> x         out = h + mlp(norm(h))    (qwen35.hpp:324-326)
// then, for the last row only, the final norm, the LM head matvec and the
// argmax (qwen35.hpp:296-302, logits.hpp:61-66). The position and the token
// id of a step live in device memory and are advanced by the device, so a
// greedy decode step has no host input and is replayed as one hipGraph.
//
// A forward of T > 1 rows (prefill) runs in chunks of rows. Per chunk and layer
// the matvecs become int8-MFMA GEMMs over all the chunk's rows (one weight read
// per chunk), the norms and the SwiGLU work row-wise, the delta-net runs its
// tokens in order with the state in shared memory, and attention appends the
// chunk's keys and values before every row attends causally -- the same
// per-row arithmetic as T single steps, so the two agree bit for bit.
#include "hero/model.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

#include "hero/errors.hpp"
#include "hero/fp16.hpp"
#include "hero/gguf.hpp"
#include "hero/kernels.hpp"
#include "hero/weights.hpp"
#include "hero_kernels.h"

namespace hero {

// ---- small device helpers for the step scalars --------------------------------
// step[0] = position, step[1] = token id, step[2] = greedy step counter
__global__ void set_step_kernel(int32_t* step, int32_t position, int32_t token, int32_t counter) {
    if (position >= 0) step[0] = position;
    if (token >= 0) step[1] = token;
    if (counter >= 0) step[2] = counter;
}
__global__ void positions_kernel(int32_t* pos, int32_t pos0, int32_t n) {
    const int32_t i = int32_t(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n) pos[i] = pos0 + i;
}
// batch: bstep[0, B) positions, [B, 2B) token ids, [2B] step counter
__global__ void advance_batch_kernel(int32_t* bstep, int32_t* out_ids, int32_t B) {
    int32_t* pos = bstep;
    const int32_t* ids = bstep + B;
    int32_t* counter = bstep + 2 * B;
    for (int32_t b = 0; b < B; ++b) {
        pos[b] += 1;
        out_ids[int64_t(*counter) * B + b] = ids[b];
    }
    *counter += 1;
}
__global__ void advance_step_kernel(int32_t* step, int32_t* out_ids, int32_t record) {
    step[0] += 1;
    if (record) {
        out_ids[step[2]] = step[1];
        step[2] += 1;
    }
}

// ---- DeviceBuffer -----------------------------------------------------------------
DeviceBuffer::DeviceBuffer(size_t bytes) : bytes_(bytes) {
    if (bytes == 0) return;
    hip_check(hipMalloc(&p_, bytes), "hipMalloc");
}
DeviceBuffer::~DeviceBuffer() {
    if (p_) (void)hipFree(p_);
}
DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& o) noexcept {
    if (this != &o) {
        if (p_) (void)hipFree(p_);
        p_ = o.p_;
        bytes_ = o.bytes_;
        o.p_ = nullptr;
        o.bytes_ = 0;
    }
    return *this;
}

namespace {

void expect(bool ok, const std::string& what) {
    if (!ok) throw Error(HERO_EIO, "qwen35 loader: " + what);
}
std::string blk(int64_t l, const char* s) { return "blk." + std::to_string(l) + "." + s; }
int64_t meta_int(const GgufFile& g, const std::string& k) { return int64_t(g.num(k)); }

}  // namespace

namespace {

// The linear weights of a layer, by GGUF name, with their (In, Out).
std::vector<std::pair<std::string, std::pair<int64_t, int64_t>>> layer_linears(const ModelConfig& c, int64_t l) {
    const int64_t CC = c.conv_channels(), VW = c.v_width(), QW = c.q_width(), KW = c.kv_width();
    std::vector<std::pair<std::string, std::pair<int64_t, int64_t>>> v = {
        {blk(l, "ffn_gate.weight"), {c.D, c.FF}}, {blk(l, "ffn_up.weight"), {c.D, c.FF}}, {blk(l, "ffn_down.weight"), {c.FF, c.D}}};
    if (c.is_recurrent(l)) {
        v.push_back({blk(l, "attn_qkv.weight"), {c.D, CC}});
        v.push_back({blk(l, "attn_gate.weight"), {c.D, VW}});
        v.push_back({blk(l, "ssm_beta.weight"), {c.D, c.Hv}});
        v.push_back({blk(l, "ssm_alpha.weight"), {c.D, c.Hv}});
        v.push_back({blk(l, "ssm_out.weight"), {VW, c.D}});
    } else {
        v.push_back({blk(l, "attn_q.weight"), {c.D, 2 * QW}});
        v.push_back({blk(l, "attn_k.weight"), {c.D, KW}});
        v.push_back({blk(l, "attn_v.weight"), {c.D, KW}});
        v.push_back({blk(l, "attn_output.weight"), {QW, c.D}});
    }
    return v;
}

}  // namespace

// ---- load ---------------------------------------------------------------------------
std::unique_ptr<Qwen35Model> Qwen35Model::open(const std::string& path) {
    GgufFile g;
    g.open(path);
    std::unique_ptr<Qwen35Model> m(new Qwen35Model());
    m->load(g);
    return m;
}

std::unique_ptr<Qwen35Model> Qwen35Model::open_image(const uint8_t* image, uint64_t size) {
    GgufFile g;
    g.parse(image, size);
    std::unique_ptr<Qwen35Model> m(new Qwen35Model());
    m->load(g);
    return m;
}

Qwen35Model::~Qwen35Model() {
    if (ev_start_) (void)hipEventDestroy(ev_start_);
    if (ev_stop_) (void)hipEventDestroy(ev_stop_);
    if (stream_) (void)hipStreamDestroy(stream_);
}

// Schema validation restates nm/src/qwen35_loader.hpp:30-75 with the
// dimensions read from the file instead of compared to a compiled config.
void Qwen35Model::load(const GgufFile& g) {
    expect(g.str("general.architecture") == "qwen35", "general.architecture is not 'qwen35'");
    ModelConfig& c = c_;
    c.L = meta_int(g, "qwen35.block_count");
    c.D = meta_int(g, "qwen35.embedding_length");
    c.FF = meta_int(g, "qwen35.feed_forward_length");
    c.Hq = meta_int(g, "qwen35.attention.head_count");
    c.Hkv = meta_int(g, "qwen35.attention.head_count_kv");
    c.Dh = meta_int(g, "qwen35.attention.key_length");
    expect(meta_int(g, "qwen35.attention.value_length") == c.Dh, "attention value_length != key_length");
    c.eps = float(g.num("qwen35.attention.layer_norm_rms_epsilon"));
    c.rope_base = double(float(g.num("qwen35.rope.freq_base")));
    c.rotary_dims = meta_int(g, "qwen35.rope.dimension_count");
    c.W = meta_int(g, "qwen35.ssm.conv_kernel");
    c.Dk = meta_int(g, "qwen35.ssm.state_size");
    c.Hk = meta_int(g, "qwen35.ssm.group_count");
    c.Hv = meta_int(g, "qwen35.ssm.time_step_rank");
    const int64_t inner = meta_int(g, "qwen35.ssm.inner_size");
    expect(c.Hv > 0 && inner % c.Hv == 0, "ssm.inner_size is not a whole number of value heads");
    c.Dv = inner / c.Hv;
    c.CTX = g.has("qwen35.context_length") ? meta_int(g, "qwen35.context_length") : 262144;
    if (g.has("qwen35.full_attention_interval")) expect(meta_int(g, "qwen35.full_attention_interval") == 4, "full_attention_interval must be 4");
    if (g.has("qwen35.attention.recurrent_layers")) {
        const auto& a = g.get("qwen35.attention.recurrent_layers").arr_num;
        expect(int64_t(a.size()) >= c.L, "qwen35.attention.recurrent_layers is shorter than block_count");
        for (int64_t l = 0; l < c.L; ++l) expect((a[size_t(l)] != 0) == c.is_recurrent(l), "layer " + std::to_string(l) + " disagrees with the hybrid schedule");
    }
    expect(c.L > 0 && c.L % 4 == 0, "block_count must be a positive multiple of 4 (3 delta-net : 1 attention)");
    expect(c.Hkv > 0 && c.Hq % c.Hkv == 0, "query heads must be a multiple of K/V heads");
    expect(c.Hk > 0 && c.Hv % c.Hk == 0, "value heads must be a multiple of key heads");
    expect(c.Dk == 128 && c.Dv == 128, "this build runs 128x128 delta-net heads");
    expect(c.Dh == 128 || c.Dh == 256, "this build runs 128- or 256-wide attention heads");
    expect(c.rotary_dims % 2 == 0 && c.rotary_dims <= c.Dh, "rope.dimension_count out of range");
    expect(c.W >= 1 && c.W <= 8, "ssm.conv_kernel must be 1..8");
    expect(c.D % 256 == 0 && c.FF % 32 == 0, "embedding_length must be a multiple of 256 and feed_forward_length of 32");
    const GgufFile::Tensor& emb = g.require("token_embd.weight");
    expect(emb.dims.size() == 2 && int64_t(emb.dims[0]) == c.D, "token_embd.weight has the wrong shape");
    c.V = int64_t(emb.dims[1]);
    c.tied = g.find("output.weight") == nullptr;

    hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "stream");
    (void)argmax_noalloc_scratch();  // resolve the static key array's address outside any capture
    hip_check(hipEventCreate(&ev_start_), "event");
    hip_check(hipEventCreate(&ev_stop_), "event");

    WeightPacker pk{DeviceBuffer(), stream_, &device_bytes_};
    // any linear weight not in Q8_0: every linear runs in its own type
    auto type_of = [&](const std::string& name) { return g.require(name).type; };
    typed_ = type_of("token_embd.weight") != 8 || (!c.tied && type_of("output.weight") != 8);
    for (int64_t l = 0; l < c.L && !typed_; ++l)
        for (const auto& lin : layer_linears(c, l)) typed_ = typed_ || type_of(lin.first) != 8;
    if (typed_) {
        load_typed(g, pk);
        hip_check(hipStreamSynchronize(stream_), "load sync");
        build_rope_table(c.CTX);
        return;
    }
    embedding_ = pk.alloc(c.V, c.D);
    pk.put(g, "token_embd.weight", embedding_, c.V, c.D, 0, c.V);
    if (!c.tied) {
        output_ = pk.alloc(c.V, c.D);
        pk.put(g, "output.weight", output_, c.V, c.D, 0, c.V);
    }
    final_norm_ = upload(host_vector(g, "output_norm.weight", c.D));

    const int64_t CC = c.conv_channels(), VW = c.v_width(), QW = c.q_width(), KW = c.kv_width();
    ffn_fused_ = c.D == 4096 && c.FF % 32 == 0;
    for (int64_t l = 0; l < c.L; ++l) {
        LayerWeights L;
        L.recurrent = c.is_recurrent(l);
        L.mixer_norm = upload(host_vector(g, blk(l, "attn_norm.weight"), c.D));
        L.channel_norm = upload(host_vector(g, blk(l, "post_attention_norm.weight"), c.D));
        L.w_gate_up = pk.alloc(2 * c.FF, c.D);
        if (ffn_fused_) {  // [gate 0..31 | up 0..31 | gate 32..63 | ...]
            pk.put(g, blk(l, "ffn_gate.weight"), L.w_gate_up, 2 * c.FF, c.D, 0, c.FF, 32);
            pk.put(g, blk(l, "ffn_up.weight"), L.w_gate_up, 2 * c.FF, c.D, 32, c.FF, 32);
        } else {
            pk.put(g, blk(l, "ffn_gate.weight"), L.w_gate_up, 2 * c.FF, c.D, 0, c.FF);
            pk.put(g, blk(l, "ffn_up.weight"), L.w_gate_up, 2 * c.FF, c.D, c.FF, c.FF);
        }
        L.w_down = pk.alloc(c.D, c.FF);
        pk.put(g, blk(l, "ffn_down.weight"), L.w_down, c.D, c.FF, 0, c.D);
        if (L.recurrent) {
            L.n_in = CC + VW + 2 * c.Hv;
            L.z_off = CC;
            L.beta_off = CC + VW;
            L.alpha_off = CC + VW + c.Hv;
            L.w_in = pk.alloc(L.n_in, c.D);
            pk.put(g, blk(l, "attn_qkv.weight"), L.w_in, L.n_in, c.D, 0, CC);
            pk.put(g, blk(l, "attn_gate.weight"), L.w_in, L.n_in, c.D, L.z_off, VW);
            pk.put(g, blk(l, "ssm_beta.weight"), L.w_in, L.n_in, c.D, L.beta_off, c.Hv);
            pk.put(g, blk(l, "ssm_alpha.weight"), L.w_in, L.n_in, c.D, L.alpha_off, c.Hv);
            L.w_out = pk.alloc(c.D, VW);
            pk.put(g, blk(l, "ssm_out.weight"), L.w_out, c.D, VW, 0, c.D);
            const GgufFile::Tensor& conv = g.require(blk(l, "ssm_conv1d.weight"));
            expect(conv.dims.size() == 2 && int64_t(conv.dims[0]) == c.W && int64_t(conv.dims[1]) == CC, blk(l, "ssm_conv1d.weight") + " has the wrong shape");
            L.conv = upload(host_vector(g, blk(l, "ssm_conv1d.weight"), CC * c.W));
            L.dt_bias = upload(host_vector(g, blk(l, "ssm_dt.bias"), c.Hv));
            std::vector<float> a = host_vector(g, blk(l, "ssm_a"), c.Hv);
            for (float& x : a) {  // nm/src/qwen35_loader.hpp:108-119
                if (x > 0.f) x = -std::exp(x);
                expect(x <= 0.f, blk(l, "ssm_a") + ": decay scale must be <= 0 (-exp(A_log))");
            }
            L.decay = upload(a);
            L.ssm_norm = upload(host_vector(g, blk(l, "ssm_norm.weight"), c.Dv));
        } else {
            L.n_in = 2 * QW + 2 * KW;
            L.k_off = 2 * QW;
            L.v_off = 2 * QW + KW;
            L.w_in = pk.alloc(L.n_in, c.D);
            pk.put(g, blk(l, "attn_q.weight"), L.w_in, L.n_in, c.D, 0, 2 * QW);
            pk.put(g, blk(l, "attn_k.weight"), L.w_in, L.n_in, c.D, L.k_off, KW);
            pk.put(g, blk(l, "attn_v.weight"), L.w_in, L.n_in, c.D, L.v_off, KW);
            L.w_out = pk.alloc(c.D, QW);
            pk.put(g, blk(l, "attn_output.weight"), L.w_out, c.D, QW, 0, c.D);
            L.q_norm = upload(host_vector(g, blk(l, "attn_q_norm.weight"), c.Dh));
            L.k_norm = upload(host_vector(g, blk(l, "attn_k_norm.weight"), c.Dh));
        }
        layers_.push_back(std::move(L));
    }
    hip_check(hipStreamSynchronize(stream_), "load sync");
    build_rope_table(c.CTX);
}

// The same schema as load() with every linear kept in its own type
// (tensor_loader::load_weight, nm/src/tensor_loader.hpp:17-35).
void Qwen35Model::load_typed(const GgufFile& g, WeightPacker& pk) {
    const ModelConfig& c = c_;
    expect(c.D % 256 == 0, "embedding_length must be a multiple of 256");
    t_embedding_ = pk.typed(g, "token_embd.weight", c.D, c.V);
    if (!c.tied) t_output_ = pk.typed(g, "output.weight", c.D, c.V);
    final_norm_ = upload(host_vector(g, "output_norm.weight", c.D));
    const int64_t CC = c.conv_channels(), VW = c.v_width(), QW = c.q_width(), KW = c.kv_width();
    for (int64_t l = 0; l < c.L; ++l) {
        LayerWeights L;
        L.recurrent = c.is_recurrent(l);
        L.mixer_norm = upload(host_vector(g, blk(l, "attn_norm.weight"), c.D));
        L.channel_norm = upload(host_vector(g, blk(l, "post_attention_norm.weight"), c.D));
        L.tgate = pk.typed(g, blk(l, "ffn_gate.weight"), c.D, c.FF);
        L.tup = pk.typed(g, blk(l, "ffn_up.weight"), c.D, c.FF);
        L.tdown = pk.typed(g, blk(l, "ffn_down.weight"), c.FF, c.D);
        if (L.recurrent) {
            L.n_in = CC + VW + 2 * c.Hv;
            L.z_off = CC;
            L.beta_off = CC + VW;
            L.alpha_off = CC + VW + c.Hv;
            L.tin.push_back(pk.typed(g, blk(l, "attn_qkv.weight"), c.D, CC));
            L.tin.push_back(pk.typed(g, blk(l, "attn_gate.weight"), c.D, VW));
            L.tin.push_back(pk.typed(g, blk(l, "ssm_beta.weight"), c.D, c.Hv));
            L.tin.push_back(pk.typed(g, blk(l, "ssm_alpha.weight"), c.D, c.Hv));
            L.tin_off = {0, L.z_off, L.beta_off, L.alpha_off};
            L.tout = pk.typed(g, blk(l, "ssm_out.weight"), VW, c.D);
            const GgufFile::Tensor& conv = g.require(blk(l, "ssm_conv1d.weight"));
            expect(conv.dims.size() == 2 && int64_t(conv.dims[0]) == c.W && int64_t(conv.dims[1]) == CC, blk(l, "ssm_conv1d.weight") + " has the wrong shape");
            L.conv = upload(host_vector(g, blk(l, "ssm_conv1d.weight"), CC * c.W));
            L.dt_bias = upload(host_vector(g, blk(l, "ssm_dt.bias"), c.Hv));
            std::vector<float> a = host_vector(g, blk(l, "ssm_a"), c.Hv);
            for (float& x : a) {  // nm/src/qwen35_loader.hpp:108-119
                if (x > 0.f) x = -std::exp(x);
                expect(x <= 0.f, blk(l, "ssm_a") + ": decay scale must be <= 0 (-exp(A_log))");
            }
            L.decay = upload(a);
            L.ssm_norm = upload(host_vector(g, blk(l, "ssm_norm.weight"), c.Dv));
        } else {
            L.n_in = 2 * QW + 2 * KW;
            L.k_off = 2 * QW;
            L.v_off = 2 * QW + KW;
            L.tin.push_back(pk.typed(g, blk(l, "attn_q.weight"), c.D, 2 * QW));
            L.tin.push_back(pk.typed(g, blk(l, "attn_k.weight"), c.D, KW));
            L.tin.push_back(pk.typed(g, blk(l, "attn_v.weight"), c.D, KW));
            L.tin_off = {0, L.k_off, L.v_off};
            L.tout = pk.typed(g, blk(l, "attn_output.weight"), QW, c.D);
            L.q_norm = upload(host_vector(g, blk(l, "attn_q_norm.weight"), c.Dh));
            L.k_norm = upload(host_vector(g, blk(l, "attn_k_norm.weight"), c.Dh));
        }
        layers_.push_back(std::move(L));
    }
}

// cos/sin per (position, plane) with the reference's float expressions
// (nm/src/attention.hpp:76-91): inv_freq = float(pow(double base, -2i/Dh)) for
// the rotary planes and 0 otherwise; angle = float(pos) * inv_freq.
void Qwen35Model::build_rope_table(int64_t positions) {
    const int64_t planes = c_.Dh / 2, rotary = c_.rotary_dims / 2;
    std::vector<float> inv(size_t(planes), 0.f);
    for (int64_t i = 0; i < planes; ++i) inv[size_t(i)] = i < rotary ? float(std::pow(c_.rope_base, -double(2 * i) / double(c_.Dh))) : 0.f;
    std::vector<float> cs(size_t(positions * planes * 2));
    for (int64_t p = 0; p < positions; ++p)
        for (int64_t i = 0; i < planes; ++i) {
            const float angle = float(p) * inv[size_t(i)];
            cs[size_t((p * planes + i) * 2)] = std::cos(angle);
            cs[size_t((p * planes + i) * 2 + 1)] = std::sin(angle);
        }
    rope_cs_ = upload(cs);
    rope_positions_ = positions;
}

// ---- state --------------------------------------------------------------------------
std::unique_ptr<Qwen35Model::State> Qwen35Model::new_state(int64_t max_tokens, int64_t batch, int kv_format, bool gdn_chunked) const {
    if (max_tokens <= 0 || max_tokens > c_.CTX || max_tokens > rope_positions_) throw Error(HERO_ERANGE, "state: max_tokens must be in 1.." + std::to_string(std::min(c_.CTX, rope_positions_)));
    if (batch < 1 || batch > kMaxBatch) throw Error(HERO_EINVAL, "state: batch must be in 1.." + std::to_string(kMaxBatch));
    if (kv_format != kKvF32 && kv_format != kKvF16 && kv_format != kKvQ8) throw Error(HERO_EINVAL, "state: unknown attention cache format");
    if (kv_format != kKvF32 && c_.Hq / c_.Hkv > kAttnMaxGroup) throw Error(HERO_EINVAL, "state: the paged cache takes at most 8 query heads per KV head");
    std::unique_ptr<State> st(new State(*this, max_tokens, batch, kv_format));
    st->gdn_chunked_ = gdn_chunked;
    return st;
}

Qwen35Model::State::State(const Qwen35Model& m, int64_t max_tokens, int64_t batch, int kv_format)
    : m_(m), max_tokens_(max_tokens), batch_(batch), kv_paged_(kv_format != kKvF32), kv_q8_(kv_format == kKvQ8), seq_tokens_(size_t(batch), 0) {
    const bool kv_paged = kv_paged_;
    const ModelConfig& c = m.c_;
    expect(!kv_q8_ || c.Dh == 128, "the Q8_0 K/V cache holds 128-wide heads; 256-wide heads use the fp32 or fp16 cache");
    const int64_t B = batch;
    int64_t n_in_max = 0;
    for (const LayerWeights& L : m.layers_) n_in_max = std::max(n_in_max, L.n_in);
    step_ = DeviceBuffer(16);
    bstep_ = DeviceBuffer(size_t(2 * B + 4) * 4);
    x_ = DeviceBuffer(size_t(B * c.D) * 4);
    h_ = DeviceBuffer(size_t(B * c.D) * 4);
    gemv_scratch_ = DeviceBuffer(size_t(c.D) * 4);
    proj_ = DeviceBuffer(size_t(B * n_in_max) * 4);
    act_d_ = DeviceBuffer(size_t(act_q8_bytes(B, c.D)));
    act_mix_ = DeviceBuffer(size_t(act_q8_bytes(B, std::max(c.q_width(), c.v_width()))));
    act_ff_ = DeviceBuffer(size_t(act_q8_bytes(B, c.FF)));
    gate_up_ = DeviceBuffer(size_t(B * 2 * c.FF) * 4);
    logits_ = DeviceBuffer(size_t(B * c.V) * 4);
    argmax_scratch_ = DeviceBuffer(size_t(B) * 128 * 8);
    out_ids_ = DeviceBuffer(size_t(max_tokens * B) * 4);
    q_rot_ = DeviceBuffer(size_t(B * c.q_width()) * 4);
    o_raw_ = DeviceBuffer(size_t(B * c.v_width()) * 4);
    g_raw_ = DeviceBuffer(size_t(B * c.v_width()) * 4);
    out_ids_capacity_ = max_tokens;
    if (m.typed_) tstep_ = std::make_unique<TypedScratch>(m, B);
    for (int64_t l = 0; l < c.L; ++l) {
        if (c.is_recurrent(l)) {
            k_cache_.emplace_back();
            v_cache_.emplace_back();
            scores_.emplace_back();
            conv_hist_.emplace_back(size_t(B * c.W * c.conv_channels()) * 4);
            delta_.emplace_back(size_t(B * c.Hv * c.Dk * c.Dv) * 4);
        } else if (kv_paged) {
            k_cache_.emplace_back();
            v_cache_.emplace_back();
            scores_.emplace_back();
            conv_hist_.emplace_back();
            delta_.emplace_back();
        } else {
            k_cache_.emplace_back(size_t(B * max_tokens * c.kv_width()) * 4);
            v_cache_.emplace_back(size_t(B * max_tokens * c.kv_width()) * 4);
            scores_.emplace_back(size_t(B * max_tokens * c.Hq) * 4);
            conv_hist_.emplace_back();
            delta_.emplace_back();
        }
    }
    kv_pages_.resize(size_t(c.L));
    if (kv_paged) {
        max_pages_ = (max_tokens + kPageTokens - 1) / kPageTokens;
        const int64_t page_bytes = attn_page_bytes(c.Hkv, c.Dh, kPageTokens, kv_q8_);
        for (int64_t l = 0; l < c.L; ++l)
            if (!c.is_recurrent(l)) kv_pages_[size_t(l)] = DeviceBuffer(size_t(B * max_pages_ * page_bytes));
        // sequence b owns pool pages b * max_pages ... (a server would map pages on demand)
        std::vector<int32_t> table(size_t(B * max_pages_));
        for (size_t i = 0; i < table.size(); ++i) table[i] = int32_t(i);
        page_table_ = DeviceBuffer(table.size() * 4);
        hip_check(hipMemcpy(page_table_.get(), table.data(), table.size() * 4, hipMemcpyHostToDevice), "page table");
        int split = 0, nsplit = 0;
        attn_paged_plan(max_pages_ * kPageTokens, 0, int(B), int(c.Hkv), &split, &nsplit);
        attn_work_ = DeviceBuffer(size_t(attn_paged_work_floats(int(B), int(c.Hq), nsplit, int(c.Dh))) * 4);
    }
    reset();
}

Qwen35Model::State::~State() {
    if (graph_) (void)hipGraphExecDestroy(graph_);
    if (bgraph_) (void)hipGraphExecDestroy(bgraph_);
}

void Qwen35Model::State::reset() {
    hipStream_t s = m_.stream_;
    auto zero = [&](DeviceBuffer& b) {
        if (b.bytes()) hip_check(hipMemsetAsync(b.get(), 0, b.bytes(), s), "state reset");
    };
    for (auto& b : k_cache_) zero(b);
    for (auto& b : v_cache_) zero(b);
    for (auto& b : conv_hist_) zero(b);
    for (auto& b : delta_) zero(b);
    for (auto& b : kv_pages_) zero(b);
    zero(step_);
    zero(bstep_);
    hip_check(hipStreamSynchronize(s), "state reset");
    std::fill(seq_tokens_.begin(), seq_tokens_.end(), 0);
}

int64_t Qwen35Model::chunk_rows(const State& st) const {
    const int64_t per_row = c_.Hq * st.max_tokens_ * 4;  // attention scores of one row
    // up to 1024 rows (512 MiB of scores): taller GEMM tiles over the chunk
    // (2048-token prefill 15.2k -> 16.1k tok/s against 512-row chunks)
    return std::max<int64_t>(1, std::min<int64_t>(1024, (int64_t(512) << 20) / per_row));
}

void Qwen35Model::State::ensure_chunk(int64_t rows) {
    if (rows <= chunk_capacity_) return;
    const ModelConfig& c = m_.c_;
    int64_t n_in_max = 0;
    for (const LayerWeights& L : m_.layers_) n_in_max = std::max(n_in_max, L.n_in);
    hip_check(hipStreamSynchronize(m_.stream_), "chunk buffers");
    cx_ = DeviceBuffer(size_t(rows * c.D) * 4);
    ch_ = DeviceBuffer(size_t(rows * c.D) * 4);
    cproj_ = DeviceBuffer(size_t(rows * n_in_max) * 4);
    cact_d_ = DeviceBuffer(size_t(act_q8_bytes(rows, c.D)));
    cact_mix_ = DeviceBuffer(size_t(act_q8_bytes(rows, std::max(c.q_width(), c.v_width()))));
    cgate_up_ = DeviceBuffer(size_t(rows * 2 * c.FF) * 4);
    cact_ff_ = DeviceBuffer(size_t(act_q8_bytes(rows, c.FF)));
    cq_rot_ = DeviceBuffer(size_t(rows * c.q_width()) * 4);
    if (!kv_paged_) cscores_ = DeviceBuffer(size_t(rows * c.Hq * max_tokens_) * 4);
    cpos_ = DeviceBuffer(size_t(rows) * 4);
    cids_ = DeviceBuffer(size_t(rows) * 4);
    cgdn_work_ = DeviceBuffer(size_t(gdn_prefill_work_bytes(rows, c.Hk, c.Hv)));
    if (m_.typed_) tchunk_ = std::make_unique<TypedScratch>(m_, rows);
    if (kv_paged_) {
        int split = 0, nsplit = 0;
        attn_paged_plan(max_pages_ * kPageTokens, 0, int(rows), int(c.Hkv), &split, &nsplit);
        cattn_work_ = DeviceBuffer(size_t(attn_paged_work_floats(int(rows), int(c.Hq), nsplit, int(c.Dh))) * 4);
    }
    chunk_capacity_ = rows;
}

// ---- the step -------------------------------------------------------------------------
namespace {

// The three GEMV forms of a layer; each returns its algorithmic bytes (weights
// and scales, inputs as read, outputs, residual reads).
//  norm:   y = W quantize(RMSNorm(x)) (+ r), one launch when K == 4096
//  swiglu: y = W quantize(silu(gate) up) (+ r), one launch when K streams
//  act:    y = W act (+ r), act already quantized
int64_t gemv_norm(const void* w, const float* x, const float* gamma, float eps, void* act_scratch, float* y, const float* r, int64_t N, int64_t K, hipStream_t s, int epi_swiglu = 0) {
    const int epi = epi_swiglu ? kEpiSwigluQuant : r ? kEpiResidual : kEpiStore;
    if (K == 4096) {
        GemvInput in{};
        in.mode = kInRmsNorm;
        in.x = x;
        in.gamma = gamma;
        in.eps = eps;
        launch_gemv_q8_in(w, in, y, r, N, K, epi, s);
    } else {
        launch_rmsnorm_quant(x, gamma, eps, nullptr, act_scratch, 1, K, s);
        launch_gemv_q8(w, act_scratch, y, r, N, K, epi, s);
    }
    return packed_q8_bytes(N, K) + 2 * K * 4 + (epi_swiglu ? act_q8_bytes(1, N / 2) : N * 4) + (r ? N * 4 : 0);
}

int64_t gemv_swiglu(const void* w, const float* gate_up, void* act_scratch, float* y, const float* r, int64_t N, int64_t K, hipStream_t s) {
    const int epi = r ? kEpiResidual : kEpiStore;
    if (gemv_streams(K)) {
        GemvInput in{};
        in.mode = kInSwiglu;
        in.gate_up = gate_up;
        launch_gemv_q8_in(w, in, y, r, N, K, epi, s);
    } else {
        launch_swiglu_quant(gate_up, act_scratch, 1, K, s);
        launch_gemv_q8(w, act_scratch, y, r, N, K, epi, s);
    }
    return packed_q8_bytes(N, K) + 2 * K * 4 + N * 4 + (r ? N * 4 : 0);
}

int64_t gemv_act(const void* w, const void* act, float* y, const float* r, int64_t N, int64_t K, hipStream_t s) {
    launch_gemv_q8(w, act, y, r, N, K, r ? kEpiResidual : kEpiStore, s);
    return packed_q8_bytes(N, K) + act_q8_bytes(1, K) + N * 4 + (r ? N * 4 : 0);
}

}  // namespace

void Qwen35Model::attention(State& st, size_t layer, AttnDecodeArgs a, const int32_t* pt, float* work, hipStream_t s) const {
    if (!st.kv_paged_) {
        launch_attn_decode(a, s);
        return;
    }
    AttnPagedArgs p{};
    p.a = a;
    p.pages = st.kv_pages_[layer].get<uint16_t>();
    p.q8 = st.kv_q8_ ? 1 : 0;
    p.page_table = pt;
    p.page_size = int(kPageTokens);
    p.max_pages = int(st.max_pages_);
    attn_paged_plan(st.max_pages_ * kPageTokens, a.window, a.B, a.Hkv, &p.split, &p.nsplit);
    p.work = work;
    launch_attn_paged(p, s);
}

// ---- models with K-quant tensors -------------------------------------------------------
// fp32 intermediates of `rows` rows and the activation scratch of each type;
// k_for / q_for remember which input rows the Q8_K / Q8_0 scratch holds, so
// linears sharing an input quantize it once (new_input() forgets)
struct Qwen35Model::TypedScratch {
    int64_t rows = 0;
    int64_t qtmp_floats = 0;
    DeviceBuffer xn, mix, ff, kact, qact, qtmp, act_mix;
    const float* k_for = nullptr;
    const float* q_for = nullptr;
    int64_t k_rows = 0, k_k = 0, q_rows = 0, q_k = 0;
    void new_input() { k_for = q_for = nullptr; }
    TypedScratch(const Qwen35Model& m, int64_t n) : rows(n) {
        const ModelConfig& c = m.c_;
        const int64_t kmax = std::max({c.D, c.FF, c.q_width(), c.v_width()});
        // every linear whose output is strided (ldy != N) goes through qtmp:
        // the input projections (ldy = n_in) and gate / up (ldy = 2 FF)
        int64_t nmax = 0;
        for (const LayerWeights& L : m.layers_) {
            for (const TypedLinear& t : L.tin) nmax = std::max(nmax, t.N);
            nmax = std::max({nmax, L.tgate.N, L.tup.N});
        }
        qtmp_floats = n * nmax;
        xn = DeviceBuffer(size_t(n * c.D) * 4);
        mix = DeviceBuffer(size_t(n * std::max(c.q_width(), c.v_width())) * 4);
        ff = DeviceBuffer(size_t(n * c.FF) * 4);
        kact = DeviceBuffer(size_t(act_q8_K_bytes(n, (kmax + 255) / 256 * 256)));
        qact = DeviceBuffer(size_t(act_q8_bytes(n, kmax)));
        qtmp = DeviceBuffer(size_t(n * nmax) * 4);
        act_mix = DeviceBuffer(size_t(act_q8_bytes(n, std::max(c.q_width(), c.v_width()))));
    }
};

void Qwen35Model::typed_linear(const TypedLinear& w, const float* x, int64_t M, float* y, int64_t ldy, const float* resid, TypedScratch& ts,
                               hipStream_t s) const {
    const int64_t N = w.N, K = w.K;
    if (w.type == 13) {  // Q5_K: fp32 activations (quant_i8.hpp:325)
        launch_q5k_gemm(w.w.get(), x, K, y, resid, M, N, K, ldy, s);
        return;
    }
    if (w.type == 12 || w.type == 14) {  // Q8_K activations (quant_i8.hpp:332-336)
        if (ts.k_for != x || ts.k_rows != M || ts.k_k != K) {
            launch_quantize_q8_K(x, ts.kact.get(), M, K, s);
            ts.k_for = x, ts.k_rows = M, ts.k_k = K;
        }
        launch_kquant_gemm_ld(w.type, w.w.get(), ts.kact.get(), y, resid, M, N, K, ldy, s);
        return;
    }
    // Q8_0 (quant_i8.hpp:338-339)
    if (ts.q_for != x || ts.q_rows != M || ts.q_k != K) {
        launch_quantize_act(x, ts.qact.get(), M, K, s);
        ts.q_for = x, ts.q_rows = M, ts.q_k = K;
    }
    const int epi = resid ? kEpiResidual : kEpiStore;
    if (ldy == N) {
        if (M == 1)
            launch_gemv_q8(w.w.get(), ts.qact.get(), y, resid, N, K, epi, s);
        else
            launch_gemm_q8(w.w.get(), ts.qact.get(), y, resid, M, N, K, epi, s);
        return;
    }
    if (resid) throw Error(HERO_EINVAL, "typed_linear: a strided Q8_0 output takes no residual");
    if (M * N > ts.qtmp_floats) throw Error(HERO_EINVAL, "typed_linear: a strided Q8_0 output larger than its scratch");
    float* tmp = ts.qtmp.get<float>();
    if (M == 1)
        launch_gemv_q8(w.w.get(), ts.qact.get(), tmp, nullptr, N, K, kEpiStore, s);
    else
        launch_gemm_q8(w.w.get(), ts.qact.get(), tmp, nullptr, M, N, K, kEpiStore, s);
    hip_check(hipMemcpy2DAsync(y, size_t(ldy) * 4, tmp, size_t(N) * 4, size_t(N) * 4, size_t(M), hipMemcpyDeviceToDevice, s), "strided copy");
}

// nm/src/qwen35.hpp:318-327 for every layer, each linear in its own type:
// U = rms(X); mix(U) from its input projections; H = X + W_o mix;
// Z = rms(H); X' = H + W_down (silu(W_gate Z) * W_up Z)
void Qwen35Model::typed_layers(State& st, TypedScratch& ts, float* x, float* h, float* proj, float* gate_up, int64_t M, const int32_t* positions,
                               int64_t seq, bool chunk, hipStream_t s) const {
    const ModelConfig& c = c_;
    float* xn = ts.xn.get<float>();
    float* mix = ts.mix.get<float>();
    for (int64_t l = 0; l < c.L; ++l) {
        const LayerWeights& L = layers_[size_t(l)];
        launch_rmsnorm_quant(x, L.mixer_norm.get<float>(), c.eps, xn, nullptr, M, c.D, s);
        ts.new_input();
        for (size_t i = 0; i < L.tin.size(); ++i) typed_linear(L.tin[i], xn, M, proj + L.tin_off[i], L.n_in, nullptr, ts, s);
        if (L.recurrent) {
            GdnDecodeArgs a{};
            a.proj = proj;
            a.proj_stride = L.n_in;
            a.z_off = L.z_off;
            a.beta_off = L.beta_off;
            a.alpha_off = L.alpha_off;
            a.conv_taps = L.conv.get<float>();
            a.conv_hist = st.conv_hist_[size_t(l)].get<float>() + seq * c.W * c.conv_channels();
            a.state = st.delta_[size_t(l)].get<float>() + seq * c.Hv * c.Dk * c.Dv;
            a.dt_bias = L.dt_bias.get<float>();
            a.decay = L.decay.get<float>();
            a.norm_gamma = L.ssm_norm.get<float>();
            a.eps = c.eps;
            a.positions = positions;
            a.act_out = ts.act_mix.get();  // the kernels' Q8_0 copy, unused here
            a.out_f32 = mix;
            a.B = int(M);
            a.Hk = int(c.Hk);
            a.Hv = int(c.Hv);
            a.Dk = int(c.Dk);
            a.Dv = int(c.Dv);
            a.W = int(c.W);
            if (chunk) {
                launch_gdn_prefill(a, st.cgdn_work_.get(), s, st.gdn_chunked_);
            } else if (M == 1) {  // one row: the step split over value columns, then the head norm and gate
                launch_gdn_decode_cols(a, st.o_raw_.get<float>(), nullptr, s);
                launch_gdn_norm_gate(st.o_raw_.get<float>(), a, s);
            } else {  // many sequences fill the GPU with the fused kernel
                launch_gdn_decode(a, s);
            }
        } else {
            AttnDecodeArgs a{};
            a.proj = proj;
            a.proj_stride = L.n_in;
            a.k_off = L.k_off;
            a.v_off = L.v_off;
            a.q_gamma = L.q_norm.get<float>();
            a.k_gamma = L.k_norm.get<float>();
            a.eps = c.eps;
            a.rope_cs = rope_cs_.get<float>();
            if (!st.kv_paged_) {
                a.k_cache = st.k_cache_[size_t(l)].get<float>() + seq * st.max_tokens_ * c.kv_width();
                a.v_cache = st.v_cache_[size_t(l)].get<float>() + seq * st.max_tokens_ * c.kv_width();
            }
            a.max_ctx = st.max_tokens_;
            a.positions = positions;
            a.shared_cache = chunk ? 1 : 0;
            a.scores = chunk ? st.cscores_.get<float>() : st.scores_[size_t(l)].get<float>() + seq * st.max_tokens_ * c.Hq;
            a.q_rot = chunk ? st.cq_rot_.get<float>() : st.q_rot_.get<float>();
            a.score_scale = 1.f / std::sqrt(float(c.Dh));  // qwen35.hpp:359
            a.window = 0;
            a.act_out = ts.act_mix.get();
            a.out_f32 = mix;
            a.B = int(M);
            a.Hq = int(c.Hq);
            a.Hkv = int(c.Hkv);
            a.Dh = int(c.Dh);
            attention(st, size_t(l), a, st.page_table_.get<int32_t>() + seq * st.max_pages_, chunk ? st.cattn_work_.get<float>() : st.attn_work_.get<float>(), s);
        }
        ts.new_input();
        typed_linear(L.tout, mix, M, h, c.D, x, ts, s);
        launch_rmsnorm_quant(h, L.channel_norm.get<float>(), c.eps, xn, nullptr, M, c.D, s);
        ts.new_input();
        typed_linear(L.tgate, xn, M, gate_up, 2 * c.FF, nullptr, ts, s);
        typed_linear(L.tup, xn, M, gate_up + c.FF, 2 * c.FF, nullptr, ts, s);
        launch_swiglu_f32(gate_up, ts.ff.get<float>(), M, c.FF, s);
        ts.new_input();
        typed_linear(L.tdown, ts.ff.get<float>(), M, x, c.D, h, ts, s);
    }
}

// the final norm, the LM head and the argmax of one row (qwen35.hpp:296-302)
void Qwen35Model::typed_head(State& st, TypedScratch& ts, const float* x_last, hipStream_t s) const {
    const ModelConfig& c = c_;
    launch_rmsnorm_quant(x_last, final_norm_.get<float>(), c.eps, ts.xn.get<float>(), nullptr, 1, c.D, s);
    ts.new_input();
    typed_linear(c.tied ? t_embedding_ : t_output_, ts.xn.get<float>(), 1, st.logits_.get<float>(), c.V, nullptr, ts, s);
    launch_argmax(st.logits_.get<float>(), 1, c.V, st.step_.get<int32_t>() + 1, st.argmax_scratch_.get<uint64_t>(), s);
}

// gather_rows (quant.hpp:464-480) of device ids
void Qwen35Model::embed_rows(const int32_t* ids, int64_t n, float* out, hipStream_t s) const {
    if (!typed_ || t_embedding_.type == 8)
        launch_embed_q8(typed_ ? t_embedding_.w.get() : embedding_.get(), c_.V, c_.D, ids, n, out, s);
    else
        launch_kquant_dequant_rows(t_embedding_.type, t_embedding_.w.get(), c_.V, c_.D, ids, n, out, s);
}

void Qwen35Model::enqueue_step(State& st, bool from_ids, bool with_head) const {
    const ModelConfig& c = c_;
    hipStream_t s = stream_;
    int32_t* step = st.step_.get<int32_t>();
    float* x = st.x_.get<float>();
    float* h = st.h_.get<float>();
    float* proj = st.proj_.get<float>();
    if (typed_) {
        if (from_ids) embed_rows(step + 1, 1, x, s);
        typed_layers(st, *st.tstep_, x, h, proj, st.gate_up_.get<float>(), 1, step, 0, false, s);
        if (with_head) typed_head(st, *st.tstep_, x, s);
        hipLaunchKernelGGL(advance_step_kernel, dim3(1), dim3(1), 0, s, step, st.out_ids_.get<int32_t>(), int32_t(with_head && from_ids));
        check_launch("decode step");
        return;
    }
    if (from_ids) launch_embed_q8(embedding_.get(), c.V, c.D, step + 1, 1, x, s);
    for (int64_t l = 0; l < c.L; ++l) {
        const LayerWeights& L = layers_[size_t(l)];
        // h = x + mix(rms(x)); x' = h + mlp(rms(h))  (nm/src/qwen35.hpp:318-327)
        gemv_norm(L.w_in.get(), x, L.mixer_norm.get<float>(), c.eps, st.act_d_.get(), proj, nullptr, L.n_in, c.D, s);
        if (L.recurrent) {
            GdnDecodeArgs a{};
            a.proj = proj;
            a.proj_stride = L.n_in;
            a.z_off = L.z_off;
            a.beta_off = L.beta_off;
            a.alpha_off = L.alpha_off;
            a.conv_taps = L.conv.get<float>();
            a.conv_hist = st.conv_hist_[size_t(l)].get<float>();
            a.state = st.delta_[size_t(l)].get<float>();
            a.dt_bias = L.dt_bias.get<float>();
            a.decay = L.decay.get<float>();
            a.norm_gamma = L.ssm_norm.get<float>();
            a.eps = c.eps;
            a.positions = step;
            a.act_out = st.act_mix_.get();
            a.out_f32 = nullptr;
            a.B = 1;
            a.Hk = int(c.Hk);
            a.Hv = int(c.Hv);
            a.Dk = int(c.Dk);
            a.Dv = int(c.Dv);
            a.W = int(c.W);
            // the step split over value columns; the head norm, SiLU(z) gate and
            // quantization then run in the output projection's prologue
            // (K = 4096) or in their own kernel
            float* o_raw = st.o_raw_.get<float>();
            const bool fused = c.v_width() == 4096;
            launch_gdn_decode_cols(a, o_raw, fused ? st.g_raw_.get<float>() : nullptr, s);
            if (fused) {
                GemvInput in{};
                in.mode = kInHeadGate;
                in.x = o_raw;
                in.z = st.g_raw_.get<float>();
                in.gamma = L.ssm_norm.get<float>();
                in.eps = c.eps;
                launch_gemv_q8_in(L.w_out.get(), in, h, x, c.D, c.v_width(), kEpiResidual, s);
            } else {
                launch_gdn_norm_gate(o_raw, a, s);
                gemv_act(L.w_out.get(), st.act_mix_.get(), h, x, c.D, c.v_width(), s);
            }
        } else {
            AttnDecodeArgs a{};
            a.proj = proj;
            a.proj_stride = L.n_in;
            a.k_off = L.k_off;
            a.v_off = L.v_off;
            a.q_gamma = L.q_norm.get<float>();
            a.k_gamma = L.k_norm.get<float>();
            a.eps = c.eps;
            a.rope_cs = rope_cs_.get<float>();
            a.k_cache = st.k_cache_[size_t(l)].get<float>();
            a.v_cache = st.v_cache_[size_t(l)].get<float>();
            a.max_ctx = st.max_tokens_;
            a.positions = step;
            a.scores = st.scores_[size_t(l)].get<float>();
            a.q_rot = st.q_rot_.get<float>();
            a.score_scale = 1.f / std::sqrt(float(c.Dh));  // qwen35.hpp:359
            a.window = 0;
            a.act_out = st.act_mix_.get();
            a.out_f32 = nullptr;
            a.B = 1;
            a.Hq = int(c.Hq);
            a.Hkv = int(c.Hkv);
            a.Dh = int(c.Dh);
            attention(st, size_t(l), a, st.page_table_.get<int32_t>(), st.attn_work_.get<float>(), s);
            gemv_act(L.w_out.get(), st.act_mix_.get(), h, x, c.D, c.q_width(), s);
        }
        if (ffn_fused_) {
            gemv_norm(L.w_gate_up.get(), h, L.channel_norm.get<float>(), c.eps, st.act_d_.get(), static_cast<float*>(st.act_ff_.get()), nullptr, 2 * c.FF, c.D, s, 1);
            gemv_act(L.w_down.get(), st.act_ff_.get(), x, h, c.D, c.FF, s);
        } else {
            gemv_norm(L.w_gate_up.get(), h, L.channel_norm.get<float>(), c.eps, st.act_d_.get(), st.gate_up_.get<float>(), nullptr, 2 * c.FF, c.D, s);
            gemv_swiglu(L.w_down.get(), st.gate_up_.get<float>(), st.act_ff_.get(), x, h, c.D, c.FF, s);
        }
    }
    if (with_head) {
        gemv_norm(c.tied ? embedding_.get() : output_.get(), x, final_norm_.get<float>(), c.eps, st.act_d_.get(), st.logits_.get<float>(), nullptr, c.V, c.D, s);
        launch_argmax(st.logits_.get<float>(), 1, c.V, step + 1, st.argmax_scratch_.get<uint64_t>(), s);
    }
    hipLaunchKernelGGL(advance_step_kernel, dim3(1), dim3(1), 0, s, step, st.out_ids_.get<int32_t>(), int32_t(with_head && from_ids));
    check_launch("decode step");
}

void Qwen35Model::enqueue_chunk(State& st, int64_t seq, int64_t pos0, int64_t T, bool with_head) const {
    const ModelConfig& c = c_;
    hipStream_t s = stream_;
    float* x = st.cx_.get<float>();
    float* h = st.ch_.get<float>();
    float* proj = st.cproj_.get<float>();
    int32_t* pos = st.cpos_.get<int32_t>();
    hipLaunchKernelGGL(positions_kernel, dim3(unsigned((T + 255) / 256)), dim3(256), 0, s, pos, int32_t(pos0), int32_t(T));
    if (typed_) {
        typed_layers(st, *st.tchunk_, x, h, proj, st.cgate_up_.get<float>(), T, pos, seq, true, s);
        if (with_head) typed_head(st, *st.tchunk_, x + (T - 1) * c.D, s);
        check_launch("prefill chunk");
        return;
    }
    for (int64_t l = 0; l < c.L; ++l) {
        const LayerWeights& L = layers_[size_t(l)];
        // H = X + mix(rms(X)); X' = H + mlp(rms(H))  (nm/src/qwen35.hpp:318-327)
        launch_rmsnorm_quant(x, L.mixer_norm.get<float>(), c.eps, nullptr, st.cact_d_.get(), T, c.D, s);
        launch_gemm_q8(L.w_in.get(), st.cact_d_.get(), proj, nullptr, T, L.n_in, c.D, kEpiStore, s);
        int64_t k_mix;
        if (L.recurrent) {
            GdnDecodeArgs a{};
            a.proj = proj;
            a.proj_stride = L.n_in;
            a.z_off = L.z_off;
            a.beta_off = L.beta_off;
            a.alpha_off = L.alpha_off;
            a.conv_taps = L.conv.get<float>();
            a.conv_hist = st.conv_hist_[size_t(l)].get<float>() + seq * c.W * c.conv_channels();
            a.state = st.delta_[size_t(l)].get<float>() + seq * c.Hv * c.Dk * c.Dv;
            a.dt_bias = L.dt_bias.get<float>();
            a.decay = L.decay.get<float>();
            a.norm_gamma = L.ssm_norm.get<float>();
            a.eps = c.eps;
            a.positions = pos;
            a.act_out = st.cact_mix_.get();
            a.out_f32 = nullptr;
            a.B = int(T);
            a.Hk = int(c.Hk);
            a.Hv = int(c.Hv);
            a.Dk = int(c.Dk);
            a.Dv = int(c.Dv);
            a.W = int(c.W);
            launch_gdn_prefill(a, st.cgdn_work_.get(), s, st.gdn_chunked_);
            k_mix = c.v_width();
        } else {
            AttnDecodeArgs a{};
            a.proj = proj;
            a.proj_stride = L.n_in;
            a.k_off = L.k_off;
            a.v_off = L.v_off;
            a.q_gamma = L.q_norm.get<float>();
            a.k_gamma = L.k_norm.get<float>();
            a.eps = c.eps;
            a.rope_cs = rope_cs_.get<float>();
            if (!st.kv_paged_) {  // the fp16 pages are found through the page table
                a.k_cache = st.k_cache_[size_t(l)].get<float>() + seq * st.max_tokens_ * c.kv_width();
                a.v_cache = st.v_cache_[size_t(l)].get<float>() + seq * st.max_tokens_ * c.kv_width();
            }
            a.max_ctx = st.max_tokens_;
            a.positions = pos;
            a.shared_cache = 1;
            a.scores = st.cscores_.get<float>();
            a.q_rot = st.cq_rot_.get<float>();
            a.score_scale = 1.f / std::sqrt(float(c.Dh));  // qwen35.hpp:359
            a.window = 0;
            a.act_out = st.cact_mix_.get();
            a.out_f32 = nullptr;
            a.B = int(T);
            a.Hq = int(c.Hq);
            a.Hkv = int(c.Hkv);
            a.Dh = int(c.Dh);
            attention(st, size_t(l), a, st.page_table_.get<int32_t>() + seq * st.max_pages_, st.cattn_work_.get<float>(), s);
            k_mix = c.q_width();
        }
        launch_gemm_q8(L.w_out.get(), st.cact_mix_.get(), h, x, T, c.D, k_mix, kEpiResidual, s);
        launch_rmsnorm_quant(h, L.channel_norm.get<float>(), c.eps, nullptr, st.cact_d_.get(), T, c.D, s);
        launch_gemm_q8(L.w_gate_up.get(), st.cact_d_.get(), st.cgate_up_.get<float>(), nullptr, T, 2 * c.FF, c.D, kEpiStore, s);
        launch_swiglu_quant(st.cgate_up_.get<float>(), st.cact_ff_.get(), T, c.FF, s, ffn_fused_ ? 32 : 0);
        launch_gemm_q8(L.w_down.get(), st.cact_ff_.get(), x, h, T, c.D, c.FF, kEpiResidual, s);
    }
    if (with_head) {
        int32_t* step = st.step_.get<int32_t>();
        gemv_norm(c.tied ? embedding_.get() : output_.get(), x + (T - 1) * c.D, final_norm_.get<float>(), c.eps, st.act_d_.get(), st.logits_.get<float>(), nullptr, c.V, c.D, s);
        launch_argmax(st.logits_.get<float>(), 1, c.V, step + 1, st.argmax_scratch_.get<uint64_t>(), s);
    }
    check_launch("prefill chunk");
}

void Qwen35Model::forward(State& st, const float* rows, const int32_t* ids, int64_t T, float* logits, int32_t* next_id) const {
    if (st.batch_ != 1) throw Error(HERO_EINVAL, "forward: a batch state takes forward_seq");
    forward_seq(st, 0, rows, ids, T, logits, next_id);
}

void Qwen35Model::forward_seq(State& st, int64_t seq, const float* rows, const int32_t* ids, int64_t T, float* logits, int32_t* next_id) const {
    const ModelConfig& c = c_;
    if (&st.m_ != this) throw Error(HERO_EINVAL, "forward: state belongs to another model");
    if (seq < 0 || seq >= st.batch_) throw Error(HERO_EINVAL, "forward: sequence index out of range");
    if (T <= 0) throw Error(HERO_EINVAL, "forward: empty input");
    if (!rows && !ids) throw Error(HERO_EINVAL, "forward: need rows or ids");
    const int64_t pos0 = st.seq_tokens_[size_t(seq)];
    if (T > st.max_tokens_ - pos0) throw Error(HERO_ERANGE, "Qwen35Model: context exhausted");
    if (ids)
        for (int64_t t = 0; t < T; ++t)
            if (ids[t] < 0 || ids[t] >= c.V) throw Error(HERO_EINVAL, "forward: token id out of range");
    hipStream_t s = stream_;
    try {
        if (T == 1 && st.batch_ == 1) {
            hipLaunchKernelGGL(set_step_kernel, dim3(1), dim3(1), 0, s, st.step_.get<int32_t>(), int32_t(pos0), ids ? ids[0] : -1, 0);
            if (rows) hip_check(hipMemcpyAsync(st.x_.get(), rows, size_t(c.D) * 4, hipMemcpyHostToDevice, s), "row upload");
            enqueue_step(st, rows == nullptr, true);
        } else {
            const int64_t cap = chunk_rows(st);
            st.ensure_chunk(std::min(cap, T));
            for (int64_t t0 = 0; t0 < T; t0 += cap) {
                const int64_t n = std::min(cap, T - t0);
                if (rows) {
                    hip_check(hipMemcpyAsync(st.cx_.get(), rows + t0 * c.D, size_t(n * c.D) * 4, hipMemcpyHostToDevice, s), "rows upload");
                } else {
                    hip_check(hipMemcpyAsync(st.cids_.get(), ids + t0, size_t(n) * 4, hipMemcpyHostToDevice, s), "ids upload");
                    embed_rows(st.cids_.get<int32_t>(), n, st.cx_.get<float>(), s);
                }
                enqueue_chunk(st, seq, pos0 + t0, n, t0 + n == T);
            }
            // the position of the next single step
            if (st.batch_ == 1) hipLaunchKernelGGL(set_step_kernel, dim3(1), dim3(1), 0, s, st.step_.get<int32_t>(), int32_t(pos0 + T), -1, -1);
        }
        if (logits) hip_check(hipMemcpyAsync(logits, st.logits_.get(), size_t(c.V) * 4, hipMemcpyDeviceToHost, s), "logits download");
        int32_t scalars[4] = {0, 0, 0, 0};
        hip_check(hipMemcpyAsync(scalars, st.step_.get(), 16, hipMemcpyDeviceToHost, s), "step download");
        hip_check(hipStreamSynchronize(s), "forward");
        if (next_id) *next_id = scalars[1];
        st.seq_tokens_[size_t(seq)] += T;
    } catch (...) {
        // the carried state is now unknown: forget it (transformer.hpp:139-142)
        (void)hipStreamSynchronize(s);
        st.reset();
        throw;
    }
}

void Qwen35Model::decode_greedy(State& st, int32_t first_id, int64_t steps, int32_t* out_ids, float* logits) const {
    const ModelConfig& c = c_;
    if (&st.m_ != this) throw Error(HERO_EINVAL, "decode: state belongs to another model");
    if (steps <= 0) throw Error(HERO_EINVAL, "decode: steps must be positive");
    if (first_id < 0 || first_id >= c.V) throw Error(HERO_EINVAL, "decode: token id out of range");
    if (st.batch_ != 1) throw Error(HERO_EINVAL, "decode: a batch state takes decode_batch");
    if (steps > st.max_tokens_ - st.seq_tokens_[0]) throw Error(HERO_ERANGE, "Qwen35Model: context exhausted");
    hipStream_t s = stream_;
    try {
        if (!st.graph_) {
            hipGraph_t graph = nullptr;
            hip_check(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "capture begin");
            enqueue_step(st, true, true);
            hip_check(hipStreamEndCapture(s, &graph), "capture end");
            hip_check(hipGraphInstantiate(&st.graph_, graph, nullptr, nullptr, 0), "graph instantiate");
            (void)hipGraphDestroy(graph);
        }
        hipLaunchKernelGGL(set_step_kernel, dim3(1), dim3(1), 0, s, st.step_.get<int32_t>(), int32_t(st.seq_tokens_[0]), first_id, 0);
        hip_check(hipEventRecord(ev_start_, s), "event");
        for (int64_t i = 0; i < steps; ++i) hip_check(hipGraphLaunch(st.graph_, s), "graph launch");
        hip_check(hipEventRecord(ev_stop_, s), "event");
        hip_check(hipMemcpyAsync(out_ids, st.out_ids_.get(), size_t(steps) * 4, hipMemcpyDeviceToHost, s), "ids download");
        if (logits) hip_check(hipMemcpyAsync(logits, st.logits_.get(), size_t(c.V) * 4, hipMemcpyDeviceToHost, s), "logits download");
        hip_check(hipStreamSynchronize(s), "decode");
        float ms = 0.f;
        hip_check(hipEventElapsedTime(&ms, ev_start_, ev_stop_), "event time");
        last_decode_seconds_ = double(ms) * 1e-3;
        st.seq_tokens_[0] += steps;
    } catch (...) {
        (void)hipStreamSynchronize(s);
        st.reset();
        throw;
    }
}

void Qwen35Model::enqueue_batch_step(State& st) const {
    const ModelConfig& c = c_;
    hipStream_t s = stream_;
    const int64_t B = st.batch_;
    int32_t* pos = st.bstep_.get<int32_t>();
    int32_t* ids = pos + B;
    float* x = st.x_.get<float>();
    float* h = st.h_.get<float>();
    float* proj = st.proj_.get<float>();
    if (typed_) {  // row b is sequence b: the decode forms of the mixers over B rows
        TypedScratch& ts = *st.tstep_;
        embed_rows(ids, B, x, s);
        typed_layers(st, ts, x, h, proj, st.gate_up_.get<float>(), B, pos, 0, false, s);
        launch_rmsnorm_quant(x, final_norm_.get<float>(), c.eps, ts.xn.get<float>(), nullptr, B, c.D, s);
        ts.new_input();
        typed_linear(c.tied ? t_embedding_ : t_output_, ts.xn.get<float>(), B, st.logits_.get<float>(), c.V, nullptr, ts, s);
        launch_argmax(st.logits_.get<float>(), B, c.V, ids, st.argmax_scratch_.get<uint64_t>(), s);
        hipLaunchKernelGGL(advance_batch_kernel, dim3(1), dim3(1), 0, s, pos, st.out_ids_.get<int32_t>(), int32_t(B));
        check_launch("batch decode step");
        return;
    }
    launch_embed_q8(embedding_.get(), c.V, c.D, ids, B, x, s);
    for (int64_t l = 0; l < c.L; ++l) {
        const LayerWeights& L = layers_[size_t(l)];
        // per row the arithmetic of enqueue_step (nm/src/qwen35.hpp:318-327)
        launch_rmsnorm_quant(x, L.mixer_norm.get<float>(), c.eps, nullptr, st.act_d_.get(), B, c.D, s);
        launch_gemm_q8(L.w_in.get(), st.act_d_.get(), proj, nullptr, B, L.n_in, c.D, kEpiStore, s);
        int64_t k_mix;
        if (L.recurrent) {
            GdnDecodeArgs a{};
            a.proj = proj;
            a.proj_stride = L.n_in;
            a.z_off = L.z_off;
            a.beta_off = L.beta_off;
            a.alpha_off = L.alpha_off;
            a.conv_taps = L.conv.get<float>();
            a.conv_hist = st.conv_hist_[size_t(l)].get<float>();
            a.state = st.delta_[size_t(l)].get<float>();
            a.dt_bias = L.dt_bias.get<float>();
            a.decay = L.decay.get<float>();
            a.norm_gamma = L.ssm_norm.get<float>();
            a.eps = c.eps;
            a.positions = pos;
            a.act_out = st.act_mix_.get();
            a.out_f32 = nullptr;
            a.B = int(B);
            a.Hk = int(c.Hk);
            a.Hv = int(c.Hv);
            a.Dk = int(c.Dk);
            a.Dv = int(c.Dv);
            a.W = int(c.W);
            launch_gdn_decode(a, s);
            k_mix = c.v_width();
        } else {
            AttnDecodeArgs a{};
            a.proj = proj;
            a.proj_stride = L.n_in;
            a.k_off = L.k_off;
            a.v_off = L.v_off;
            a.q_gamma = L.q_norm.get<float>();
            a.k_gamma = L.k_norm.get<float>();
            a.eps = c.eps;
            a.rope_cs = rope_cs_.get<float>();
            a.k_cache = st.k_cache_[size_t(l)].get<float>();
            a.v_cache = st.v_cache_[size_t(l)].get<float>();
            a.max_ctx = st.max_tokens_;
            a.positions = pos;
            a.shared_cache = 0;
            a.scores = st.scores_[size_t(l)].get<float>();
            a.q_rot = st.q_rot_.get<float>();
            a.score_scale = 1.f / std::sqrt(float(c.Dh));  // qwen35.hpp:359
            a.window = 0;
            a.act_out = st.act_mix_.get();
            a.out_f32 = nullptr;
            a.B = int(B);
            a.Hq = int(c.Hq);
            a.Hkv = int(c.Hkv);
            a.Dh = int(c.Dh);
            attention(st, size_t(l), a, st.page_table_.get<int32_t>(), st.attn_work_.get<float>(), s);
            k_mix = c.q_width();
        }
        launch_gemm_q8(L.w_out.get(), st.act_mix_.get(), h, x, B, c.D, k_mix, kEpiResidual, s);
        launch_rmsnorm_quant(h, L.channel_norm.get<float>(), c.eps, nullptr, st.act_d_.get(), B, c.D, s);
        // interleaved gate/up rows: SwiGLU and its quantization in the GEMM's epilogue
        if (!ffn_fused_ || !launch_gemm_q8_swiglu(L.w_gate_up.get(), st.act_d_.get(), st.act_ff_.get(), B, 2 * c.FF, c.D, s)) {
            launch_gemm_q8(L.w_gate_up.get(), st.act_d_.get(), st.gate_up_.get<float>(), nullptr, B, 2 * c.FF, c.D, kEpiStore, s);
            launch_swiglu_quant(st.gate_up_.get<float>(), st.act_ff_.get(), B, c.FF, s, ffn_fused_ ? 32 : 0);
        }
        launch_gemm_q8(L.w_down.get(), st.act_ff_.get(), x, h, B, c.D, c.FF, kEpiResidual, s);
    }
    launch_rmsnorm_quant(x, final_norm_.get<float>(), c.eps, nullptr, st.act_d_.get(), B, c.D, s);
    launch_gemm_q8(c.tied ? embedding_.get() : output_.get(), st.act_d_.get(), st.logits_.get<float>(), nullptr, B, c.V, c.D, kEpiStore, s);
    launch_argmax(st.logits_.get<float>(), B, c.V, ids, st.argmax_scratch_.get<uint64_t>(), s);
    hipLaunchKernelGGL(advance_batch_kernel, dim3(1), dim3(1), 0, s, pos, st.out_ids_.get<int32_t>(), int32_t(B));
    check_launch("batch decode step");
}

void Qwen35Model::decode_batch(State& st, const int32_t* first_ids, int64_t steps, int32_t* out_ids, float* logits) const {
    const ModelConfig& c = c_;
    const int64_t B = st.batch_;
    if (&st.m_ != this) throw Error(HERO_EINVAL, "decode: state belongs to another model");
    if (steps <= 0) throw Error(HERO_EINVAL, "decode: steps must be positive");
    if (!first_ids) throw Error(HERO_EINVAL, "decode: need the first ids");
    std::vector<int32_t> init(size_t(2 * B + 4), 0);
    for (int64_t b = 0; b < B; ++b) {
        if (first_ids[b] < 0 || first_ids[b] >= c.V) throw Error(HERO_EINVAL, "decode: token id out of range");
        if (steps > st.max_tokens_ - st.seq_tokens_[size_t(b)]) throw Error(HERO_ERANGE, "Qwen35Model: context exhausted");
        init[size_t(b)] = int32_t(st.seq_tokens_[size_t(b)]);
        init[size_t(B + b)] = first_ids[b];
    }
    hipStream_t s = stream_;
    try {
        if (!st.bgraph_) {
            hipGraph_t graph = nullptr;
            hip_check(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "capture begin");
            enqueue_batch_step(st);
            hip_check(hipStreamEndCapture(s, &graph), "capture end");
            hip_check(hipGraphInstantiate(&st.bgraph_, graph, nullptr, nullptr, 0), "graph instantiate");
            (void)hipGraphDestroy(graph);
        }
        hip_check(hipMemcpyAsync(st.bstep_.get(), init.data(), init.size() * 4, hipMemcpyHostToDevice, s), "batch step upload");
        hip_check(hipEventRecord(ev_start_, s), "event");
        for (int64_t i = 0; i < steps; ++i) hip_check(hipGraphLaunch(st.bgraph_, s), "graph launch");
        hip_check(hipEventRecord(ev_stop_, s), "event");
        hip_check(hipMemcpyAsync(out_ids, st.out_ids_.get(), size_t(steps * B) * 4, hipMemcpyDeviceToHost, s), "ids download");
        if (logits) hip_check(hipMemcpyAsync(logits, st.logits_.get(), size_t(B * c.V) * 4, hipMemcpyDeviceToHost, s), "logits download");
        hip_check(hipStreamSynchronize(s), "decode");
        float ms = 0.f;
        hip_check(hipEventElapsedTime(&ms, ev_start_, ev_stop_), "event time");
        last_decode_seconds_ = double(ms) * 1e-3;
        for (int64_t b = 0; b < B; ++b) st.seq_tokens_[size_t(b)] += steps;
    } catch (...) {
        (void)hipStreamSynchronize(s);
        st.reset();
        throw;
    }
}

double Qwen35Model::time_gemvs(State& st, int reps, int64_t* launches, int64_t* bytes) const {
    const ModelConfig& c = c_;
    if (typed_) throw Error(HERO_EINVAL, "time_gemvs: the Q8_0 matvec timing takes a model whose linears are all Q8_0");
    hipStream_t s = stream_;
    int64_t n_launch = 0, n_bytes = 0;
    // the GEMVs exactly as a decode step launches them (fused input forms
    // included), on scratch outputs: x and h are read, never written
    float* x = st.x_.get<float>();
    float* h = st.h_.get<float>();
    float* y_d = st.gemv_scratch_.get<float>();
    auto one_step = [&] {
        for (const LayerWeights& L : layers_) {
            const int64_t k_mix = L.recurrent ? c.v_width() : c.q_width();
            n_bytes += gemv_norm(L.w_in.get(), x, L.mixer_norm.get<float>(), c.eps, st.act_d_.get(), st.proj_.get<float>(), nullptr, L.n_in, c.D, s);
            if (L.recurrent && c.v_width() == 4096) {  // the head-norm-gated input form
                GemvInput in{};
                in.mode = kInHeadGate;
                in.x = st.o_raw_.get<float>();
                in.z = st.g_raw_.get<float>();
                in.gamma = L.ssm_norm.get<float>();
                in.eps = c.eps;
                launch_gemv_q8_in(L.w_out.get(), in, y_d, x, c.D, k_mix, kEpiResidual, s);
                n_bytes += packed_q8_bytes(c.D, k_mix) + 2 * k_mix * 4 + c.Dv * 4 + 2 * c.D * 4;
            } else {
                n_bytes += gemv_act(L.w_out.get(), st.act_mix_.get(), y_d, x, c.D, k_mix, s);
            }
            if (ffn_fused_) {
                n_bytes += gemv_norm(L.w_gate_up.get(), h, L.channel_norm.get<float>(), c.eps, st.act_d_.get(), static_cast<float*>(st.act_ff_.get()), nullptr, 2 * c.FF, c.D, s, 1);
                n_bytes += gemv_act(L.w_down.get(), st.act_ff_.get(), y_d, h, c.D, c.FF, s);
            } else {
                n_bytes += gemv_norm(L.w_gate_up.get(), h, L.channel_norm.get<float>(), c.eps, st.act_d_.get(), st.gate_up_.get<float>(), nullptr, 2 * c.FF, c.D, s);
                n_bytes += gemv_swiglu(L.w_down.get(), st.gate_up_.get<float>(), st.act_ff_.get(), y_d, h, c.D, c.FF, s);
            }
            n_launch += 4;
        }
        n_bytes += gemv_norm(c.tied ? embedding_.get() : output_.get(), x, final_norm_.get<float>(), c.eps, st.act_d_.get(), st.logits_.get<float>(), nullptr, c.V, c.D, s);
        n_launch += 1;
    };
    one_step();  // warm the instruction cache and the launch path
    hip_check(hipStreamSynchronize(s), "gemv warmup");
    n_launch = n_bytes = 0;
    hip_check(hipEventRecord(ev_start_, s), "event");
    for (int r = 0; r < reps; ++r) one_step();
    hip_check(hipEventRecord(ev_stop_, s), "event");
    hip_check(hipStreamSynchronize(s), "gemv timing");
    check_launch("gemv timing");
    float ms = 0.f;
    hip_check(hipEventElapsedTime(&ms, ev_start_, ev_stop_), "event time");
    *launches = n_launch / std::max(reps, 1);
    *bytes = n_bytes / std::max(reps, 1);
    return double(ms) * 1e-3;
}

void Qwen35Model::embed(const int32_t* ids, int64_t n, float* out) const {
    if (n <= 0) throw Error(HERO_EINVAL, "embed: empty input");
    for (int64_t i = 0; i < n; ++i)
        if (ids[i] < 0 || ids[i] >= c_.V) throw Error(HERO_EINVAL, "embed: token id out of range");
    DeviceBuffer d_ids(size_t(n) * 4), d_out(size_t(n * c_.D) * 4);
    hip_check(hipMemcpyAsync(d_ids.get(), ids, size_t(n) * 4, hipMemcpyHostToDevice, stream_), "ids upload");
    embed_rows(d_ids.get<int32_t>(), n, d_out.get<float>(), stream_);
    check_launch("embed");
    hip_check(hipMemcpyAsync(out, d_out.get(), size_t(n * c_.D) * 4, hipMemcpyDeviceToHost, stream_), "rows download");
    hip_check(hipStreamSynchronize(stream_), "embed");
}

}  // namespace hero
