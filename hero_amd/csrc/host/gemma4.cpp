// gemma4.cpp -- load, state and the per-token schedule of the GPU Gemma 4
// text model (E4B schema).
//
// Per token (all on the model's stream; position and id in device memory, so
// a greedy step is replayed as one hipGraph):
//   gemma_embed                 x = emb[id] * sqrt(D), act = Q8_0(x), tok = ple_table[id] * sqrt(P)
//   gemv(ple_proj)              ctx = W_ple x                         (gemma4.hpp:132-134)
//   gemma_ple_inputs            ple = (RMSNorm_P(ctx / sqrt(D)) + tok) / sqrt(2), per layer slice
//   rmsnorm_quant(x)            layer 0's attn_norm
// per layer (GemmaE4BLayer::forward, gemma4.hpp:258-272):
//   gemv(w_qkv)                 q | k | v (q only on layers that reuse K/V)
//   gemma_attention             norms, RoPE, append, softmax(q.k) v, Q8_0 of the W_o input
//   gemv(w_o)                   a
//   gemma_post_norm             h = x + post_attn_norm(a); act = Q8_0(ffn_norm(h))
//   gemv(w_gate_up)             gelu(gate) | up
//   gemv(w_down)                a, over Q8_0(gelu(gate) * up)
//   gemma_post_norm             h2 = h + post_ffw_norm(a); act = Q8_0(h2)
//   gemv(w_pgate)               gelu(pg)
//   gemv(w_proj)                a, over Q8_0(gelu(pg) * ple[l])       (gemma4.hpp:100-105)
//   gemma_post_norm             x = (h2 + post_norm(a)) * layer_output_scale; act = Q8_0(next norm(x))
// then the tied LM head over act (the final norm's output), the soft-cap and
// the argmax (gemma4.hpp:440-444).
// The GELU is applied to each gate row in the producing GEMV's epilogue (once
// per value) and the product formed and quantized in the consuming GEMV's
// prologue; at row lengths without a streaming GEMV a gemma_gelu_mul_quant
// does both between two plain GEMVs. At d_model 2560 each post-norm runs in
// the prologue of the GEMV that reads its act (w_gate_up, w_pgate, the next
// layer's w_qkv, after the last layer the LM head): every workgroup forms the
// row itself and workgroup 0 writes h, h2 or x.
#include "hero/gemma4.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

#include "hero/errors.hpp"
#include "hero/gguf.hpp"
#include "hero/kernels.hpp"
#include "hero/weights.hpp"
#include "hero_kernels.h"

namespace hero {

// step[0] = position, step[1] = token id, step[2] = greedy step counter
__global__ void gemma_set_step_kernel(int32_t* step, int32_t position, int32_t token, int32_t counter) {
    if (position >= 0) step[0] = position;
    if (token >= 0) step[1] = token;
    if (counter >= 0) step[2] = counter;
}
__global__ void gemma_advance_step_kernel(int32_t* step, int32_t* out_ids, int32_t record) {
    step[0] += 1;
    if (record) {
        out_ids[step[2]] = step[1];
        step[2] += 1;
    }
}

namespace {

void expect(bool ok, const std::string& what) {
    if (!ok) throw Error(HERO_EIO, "gemma4 loader: " + what);
}
std::string blk(int64_t l, const char* s) { return "blk." + std::to_string(l) + "." + s; }

int64_t meta_int(const GgufFile& g, const std::string& k) {
    expect(g.has(k), "missing metadata key " + k);
    const GgufFile::Value& v = g.get(k);
    if (!v.arr_num.empty()) {  // per-layer arrays must be uniform here
        for (double x : v.arr_num) expect(x == v.arr_num[0], k + " differs between layers");
        return int64_t(v.arr_num[0]);
    }
    return int64_t(v.num);
}
double meta_num_or(const GgufFile& g, const std::string& k, double fallback) { return g.has(k) ? g.num(k) : fallback; }

}  // namespace

int64_t Gemma4Config::kv_source(int64_t l) const {
    if (!shares_kv(l)) return l;
    for (int64_t s = L - shared - 1; s >= 0; --s)
        if (full(s) == full(l)) return s;
    return -1;
}

// ---- load ---------------------------------------------------------------------------
std::unique_ptr<Gemma4Model> Gemma4Model::open(const std::string& path) {
    GgufFile g;
    g.open(path);
    std::unique_ptr<Gemma4Model> m(new Gemma4Model());
    m->load(g);
    return m;
}

std::unique_ptr<Gemma4Model> Gemma4Model::open_image(const uint8_t* image, uint64_t size) {
    GgufFile g;
    g.parse(image, size);
    std::unique_ptr<Gemma4Model> m(new Gemma4Model());
    m->load(g);
    return m;
}

Gemma4Model::~Gemma4Model() {
    if (ev_start_) (void)hipEventDestroy(ev_start_);
    if (ev_stop_) (void)hipEventDestroy(ev_stop_);
    if (stream_) (void)hipStreamDestroy(stream_);
}

// validate_e4b_text_metadata (nm/src/gemma4_loader.hpp:31-52) with the
// dimensions read from the file, then load_e4b_text (:105-130).
void Gemma4Model::load(const GgufFile& g) {
    expect(g.str("general.architecture") == "gemma4", "general.architecture is not 'gemma4'");
    Gemma4Config& c = c_;
    c.L = meta_int(g, "gemma4.block_count");
    c.D = meta_int(g, "gemma4.embedding_length");
    c.FF = meta_int(g, "gemma4.feed_forward_length");
    c.Hq = meta_int(g, "gemma4.attention.head_count");
    c.Hkv = meta_int(g, "gemma4.attention.head_count_kv");
    c.Df = meta_int(g, "gemma4.attention.key_length");
    expect(meta_int(g, "gemma4.attention.value_length") == c.Df, "attention.value_length != key_length");
    c.Dl = meta_int(g, "gemma4.attention.key_length_swa");
    expect(meta_int(g, "gemma4.attention.value_length_swa") == c.Dl, "attention.value_length_swa != key_length_swa");
    c.window = meta_int(g, "gemma4.attention.sliding_window");
    c.shared = meta_int(g, "gemma4.attention.shared_kv_layers");
    c.P = meta_int(g, "gemma4.embedding_length_per_layer_input");
    expect(g.has("gemma4.attention.layer_norm_rms_epsilon"), "missing gemma4.attention.layer_norm_rms_epsilon");
    expect(g.has("gemma4.final_logit_softcapping"), "missing gemma4.final_logit_softcapping");
    c.eps = float(g.num("gemma4.attention.layer_norm_rms_epsilon"));
    c.softcap = float(g.num("gemma4.final_logit_softcapping"));
    c.CTX = g.has("gemma4.context_length") ? meta_int(g, "gemma4.context_length") : 131072;
    // the reference's RoPE tables (gemma4.hpp:396-397): local heads rotate every
    // plane with base 1e4, full heads their first quarter with base 1e6
    c.local_base = double(float(meta_num_or(g, "gemma4.rope.freq_base_swa", 1e4)));
    c.full_base = double(float(meta_num_or(g, "gemma4.rope.freq_base", 1e6)));
    c.local_rot = g.has("gemma4.rope.dimension_count_swa") ? meta_int(g, "gemma4.rope.dimension_count_swa") : c.Dl;
    c.full_rot = g.has("gemma4.rope.dimension_count") ? meta_int(g, "gemma4.rope.dimension_count") : c.Df / 4;
    const GgufFile::Tensor& emb = g.require("token_embd.weight");
    expect(emb.dims.size() == 2 && int64_t(emb.dims[0]) == c.D, "token_embd.weight has the wrong shape");
    c.V = int64_t(emb.dims[1]);

    expect(c.L >= 6 && c.shared >= 0 && c.shared < c.L, "block_count / shared_kv_layers out of range");
    expect(c.D > 0 && c.D <= 4096 && c.D % 32 == 0, "embedding_length must be a multiple of 32 up to 4096");
    expect(c.FF > 0 && c.FF % 32 == 0, "feed_forward_length must be a positive multiple of 32");
    expect(c.P > 0 && c.P <= 4096 && c.P % 32 == 0, "embedding_length_per_layer_input must be a multiple of 32 up to 4096");
    expect(c.Hkv > 0 && c.Hq > 0 && c.Hq % c.Hkv == 0 && c.Hq / c.Hkv <= kAttnMaxGroup, "head_count must be a multiple of head_count_kv, at most 8 per KV head");
    expect((c.Dl == 256 || c.Dl == 512) && (c.Df == 256 || c.Df == 512), "this build runs heads of 256 or 512");
    expect(c.Hq * std::max(c.Dl, c.Df) <= 65536, "too many query channels");
    expect(c.local_rot > 0 && c.local_rot <= c.Dl && c.local_rot % 2 == 0 && c.full_rot > 0 && c.full_rot <= c.Df && c.full_rot % 2 == 0, "rope dimension counts out of range");
    expect(c.window > 0 && c.CTX > 0 && c.V > 0 && c.V < (int64_t(1) << 31), "sliding_window / context_length / vocabulary out of range");
    expect(c.eps > 0.f && c.softcap > 0.f, "epsilon and soft-cap must be positive");
    for (int64_t l = 0; l < c.L; ++l) expect(c.kv_source(l) >= 0, "a layer that reuses K/V has no earlier layer of its kind");

    hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "stream");
    hip_check(hipEventCreate(&ev_start_), "event");
    hip_check(hipEventCreate(&ev_stop_), "event");
    (void)argmax_noalloc_scratch();  // resolve the no-alloc argmax's array outside any capture

    WeightPacker pk{DeviceBuffer(), stream_, &device_bytes_};
    const int64_t PL = c.P * c.L;
    embedding_ = pk.alloc(c.V, c.D);
    pk.put(g, "token_embd.weight", embedding_, c.V, c.D, 0, c.V);
    ple_table_ = pk.alloc(c.V, PL);
    pk.put(g, "per_layer_token_embd.weight", ple_table_, c.V, PL, 0, c.V);
    ple_proj_ = pk.alloc(PL, c.D);
    pk.put(g, "per_layer_model_proj.weight", ple_proj_, PL, c.D, 0, PL);
    ple_norm_ = upload(host_vector(g, "per_layer_proj_norm.weight", c.P));
    final_norm_ = upload(host_vector(g, "output_norm.weight", c.D));
    // nm/src/gemma4.hpp:417 and gemma4_loader.hpp:112: sqrt(D), sqrt(P),
    // 1/sqrt(D), 1/sqrt(2) in fp32
    embed_scale_ = std::sqrt(float(c.D));
    token_scale_ = std::sqrt(float(c.P));
    proj_scale_ = 1.f / std::sqrt(float(c.D));
    comb_scale_ = 1.f / std::sqrt(2.f);

    for (int64_t l = 0; l < c.L; ++l) {
        Gemma4Layer L;
        L.full = c.full(l);
        L.shared = c.shares_kv(l);
        L.dh = c.head_dim(l);
        L.src = c.kv_source(l);
        const int64_t QW = c.Hq * L.dh, KW = c.Hkv * L.dh;
        L.attn_norm = upload(host_vector(g, blk(l, "attn_norm.weight"), c.D));
        L.q_norm = upload(host_vector(g, blk(l, "attn_q_norm.weight"), L.dh));
        L.post_attn_norm = upload(host_vector(g, blk(l, "post_attention_norm.weight"), c.D));
        L.ffn_norm = upload(host_vector(g, blk(l, "ffn_norm.weight"), c.D));
        L.post_ffn_norm = upload(host_vector(g, blk(l, "post_ffw_norm.weight"), c.D));
        L.post_norm = upload(host_vector(g, blk(l, "post_norm.weight"), c.D));
        L.n_qkv = L.shared ? QW : QW + 2 * KW;
        L.w_qkv = pk.alloc(L.n_qkv, c.D);
        pk.put(g, blk(l, "attn_q.weight"), L.w_qkv, L.n_qkv, c.D, 0, QW);
        if (!L.shared) {  // layers that reuse K/V load no K/V tensors (gemma4_loader.hpp:95-103)
            L.k_norm = upload(host_vector(g, blk(l, "attn_k_norm.weight"), L.dh));
            pk.put(g, blk(l, "attn_k.weight"), L.w_qkv, L.n_qkv, c.D, QW, KW);
            pk.put(g, blk(l, "attn_v.weight"), L.w_qkv, L.n_qkv, c.D, QW + KW, KW);
        }
        L.w_o = pk.alloc(c.D, QW);
        pk.put(g, blk(l, "attn_output.weight"), L.w_o, c.D, QW, 0, c.D);
        L.w_gate_up = pk.alloc(2 * c.FF, c.D);
        pk.put(g, blk(l, "ffn_gate.weight"), L.w_gate_up, 2 * c.FF, c.D, 0, c.FF);
        pk.put(g, blk(l, "ffn_up.weight"), L.w_gate_up, 2 * c.FF, c.D, c.FF, c.FF);
        L.w_down = pk.alloc(c.D, c.FF);
        pk.put(g, blk(l, "ffn_down.weight"), L.w_down, c.D, c.FF, 0, c.D);
        L.w_pgate = pk.alloc(c.P, c.D);
        pk.put(g, blk(l, "inp_gate.weight"), L.w_pgate, c.P, c.D, 0, c.P);
        L.w_proj = pk.alloc(c.D, c.P);
        pk.put(g, blk(l, "proj.weight"), L.w_proj, c.D, c.P, 0, c.D);
        // optional_scalar (gemma4_loader.hpp:56-63): 1 when absent
        if (g.find(blk(l, "layer_output_scale.weight"))) L.out_scale = host_vector(g, blk(l, "layer_output_scale.weight"), 1)[0];
        layers_.push_back(std::move(L));
    }
    hip_check(hipStreamSynchronize(stream_), "weight packing");

    // RoPE tables (RotaryEmbedding, nm/src/attention.hpp:76-91): inv_freq_i =
    // base^(-2i/Dh) for the rotated planes, 0 for the rest; angle = p * inv_i in
    // fp32, then cos and sin
    rope_positions_ = c.CTX;
    auto table = [&](int64_t dh, int64_t rot, double base) {
        const int64_t planes = dh / 2, rotary = rot / 2;
        std::vector<float> inv(size_t(planes), 0.f);
        for (int64_t i = 0; i < planes; ++i) inv[size_t(i)] = i < rotary ? float(std::pow(base, -double(2 * i) / double(dh))) : 0.f;
        std::vector<float> cs(size_t(rope_positions_ * planes * 2));
        for (int64_t p = 0; p < rope_positions_; ++p)
            for (int64_t i = 0; i < planes; ++i) {
                const float angle = float(p) * inv[size_t(i)];
                cs[size_t((p * planes + i) * 2)] = std::cos(angle);
                cs[size_t((p * planes + i) * 2 + 1)] = std::sin(angle);
            }
        return upload(cs);
    };
    rope_local_ = table(c.Dl, c.local_rot, c.local_base);
    rope_full_ = table(c.Df, c.full_rot, c.full_base);
}

// ---- state --------------------------------------------------------------------------
std::unique_ptr<Gemma4Model::State> Gemma4Model::new_state(int64_t max_tokens) const {
    if (max_tokens <= 0 || max_tokens > c_.CTX || max_tokens > rope_positions_) throw Error(HERO_ERANGE, "state: max_tokens must be in 1.." + std::to_string(c_.CTX));
    return std::unique_ptr<State>(new State(*this, max_tokens));
}

Gemma4Model::State::State(const Gemma4Model& m, int64_t max_tokens) : m_(m), max_tokens_(max_tokens) {
    const Gemma4Config& c = m.c_;
    const int64_t PL = c.P * c.L, dmax = std::max(c.Dl, c.Df);
    int64_t nq = 0;
    for (const Gemma4Layer& L : m.layers_) nq = std::max(nq, L.n_qkv);
    const int64_t act_k = std::max({c.D, c.FF, c.P, c.Hq * dmax});
    step_ = DeviceBuffer(16);
    x_ = DeviceBuffer(size_t(c.D) * 4);
    h_ = DeviceBuffer(size_t(c.D) * 4);
    h2_ = DeviceBuffer(size_t(c.D) * 4);
    a_ = DeviceBuffer(size_t(c.D) * 4);
    act_ = DeviceBuffer(size_t(act_q8_bytes(1, c.D)));
    tok_ = DeviceBuffer(size_t(PL) * 4);
    ctx_ = DeviceBuffer(size_t(PL) * 4);
    ple_ = DeviceBuffer(size_t(PL) * 4);
    proj_ = DeviceBuffer(size_t(nq) * 4);
    q_rot_ = DeviceBuffer(size_t(c.Hq * dmax) * 4);
    scores_ = DeviceBuffer(size_t(c.Hq * max_tokens) * 4);
    act_o_ = DeviceBuffer(size_t(act_q8_bytes(1, act_k)));
    gu_ = DeviceBuffer(size_t(2 * c.FF) * 4);
    act_ff_ = DeviceBuffer(size_t(act_q8_bytes(1, c.FF)));
    pg_ = DeviceBuffer(size_t(c.P) * 4);
    act_p_ = DeviceBuffer(size_t(act_q8_bytes(1, c.P)));
    logits_ = DeviceBuffer(size_t(c.V) * 4);
    argmax_scratch_ = DeviceBuffer(size_t(kArgmaxGroups) * 8);
    k_cache_.resize(size_t(c.L));
    v_cache_.resize(size_t(c.L));
    slots_.assign(size_t(c.L), 0);
    for (int64_t l = 0; l < c.L; ++l) {
        const Gemma4Layer& L = m.layers_[size_t(l)];
        if (L.shared) continue;
        // Gemma4E4BCache (gemma4.hpp:350-358): window layers keep a ring of
        // `window` rows, full layers every position
        const int64_t slots = L.full ? max_tokens : std::min(c.window, max_tokens);
        slots_[size_t(l)] = slots;
        k_cache_[size_t(l)] = DeviceBuffer(size_t(c.Hkv * L.dh * slots) * 4);
        v_cache_[size_t(l)] = DeviceBuffer(size_t(c.Hkv * L.dh * slots) * 4);
    }
    reset();
}

Gemma4Model::State::~State() {
    if (graph_) (void)hipGraphExecDestroy(graph_);
}

void Gemma4Model::State::reset() {
    tokens_ = 0;
    hipLaunchKernelGGL(gemma_set_step_kernel, dim3(1), dim3(1), 0, m_.stream_, step_.get<int32_t>(), 0, 0, 0);
    check_launch("state reset");
    hip_check(hipStreamSynchronize(m_.stream_), "state reset");
}

// ---- the step ------------------------------------------------------------------------
namespace {
// GELU gate, then a projection over it: g[G] = W_g x (its first `gated` rows
// through the GELU when `fused`), then y[N] = W Q8_0(gelu(g[0..K)) * up[0..K))
// (K = `gated`). fused: both row lengths stream, the GELU is in the first
// GEMV's epilogue and the product in the second's prologue.
bool gelu_fusable(int64_t Kx, int64_t K) { return gemv_streams_act(Kx) && gemv_streams_act(K); }

// the quantized row act [K] as a GEMV input
GemvInput act_input(const DeviceBuffer& act, int64_t K) {
    GemvInput in{};
    in.mode = kInAct;
    in.xq = act.get<int8_t>();
    in.xd = reinterpret_cast<const float*>(act.get<int8_t>() + K);
    return in;
}

// The end of a sub-block, out = (RMSNorm(a) * gamma + res) * scale, and the
// next GEMV's input Q8_0(next_gamma ? RMSNorm(out) * next_gamma : out): formed
// in that GEMV's prologue where its width allows, else by a post-norm launch
// into act.
struct SubBlockEnd {
    const float* a;
    const float* gamma;
    const float* res;
    float scale;
    float* out;
    const float* next_gamma;
};
GemvInput sub_block_end(const SubBlockEnd& e, float eps, const DeviceBuffer& act, int64_t D, hipStream_t s) {
    if (!gemv_post_norm_fusable(D)) {
        launch_gemma_post_norm(e.a, e.gamma, e.res, e.scale, eps, e.out, e.next_gamma, act.get(), D, s);
        return act_input(act, D);
    }
    GemvInput in{};
    in.mode = kInPostNorm;
    in.x = e.a;
    in.gamma = e.gamma;
    in.res = e.res;
    in.scale = e.scale;
    in.out = e.out;
    in.next_gamma = e.next_gamma;
    in.eps = eps;
    return in;
}

// y[N] = W over the input in (the quantized row act when in is kInAct)
void gemv_in(const DeviceBuffer& w, const GemvInput& in, const DeviceBuffer& act, float* y, int64_t N, int64_t K, hipStream_t s) {
    if (in.mode == kInAct)
        launch_gemv_q8(w.get(), act.get(), y, nullptr, N, K, kEpiStore, s);
    else
        launch_gemv_q8_in(w.get(), in, y, nullptr, N, K, kEpiStore, s);
}

void gelu_gated_pair(const DeviceBuffer& wg, const GemvInput& in0, const DeviceBuffer& act_in, float* g, int64_t G, int64_t Kx, const float* up, const DeviceBuffer& w,
                     const DeviceBuffer& act_mid, float* y, int64_t N, int64_t K, hipStream_t s) {
    if (gelu_fusable(Kx, K)) {
        GemvInput in = in0;
        in.act_rows = int(K);
        launch_gemv_q8_in(wg.get(), in, g, nullptr, G, Kx, kEpiGelu, s);
        GemvInput pin{};
        pin.mode = kInMul;
        pin.gate_up = g;
        pin.up = up;
        launch_gemv_q8_in(w.get(), pin, y, nullptr, N, K, kEpiStore, s);
    } else {
        gemv_in(wg, in0, act_in, g, G, Kx, s);
        launch_gemma_gelu_mul_quant(g, up, act_mid.get(), K, s);
        launch_gemv_q8(w.get(), act_mid.get(), y, nullptr, N, K, kEpiStore, s);
    }
}
}  // namespace

void Gemma4Model::enqueue_step(State& st) const {
    const Gemma4Config& c = c_;
    hipStream_t s = stream_;
    int32_t* step = st.step_.get<int32_t>();
    float* x = st.x_.get<float>();
    const int64_t PL = c.P * c.L;
    // the input embedding and the per-layer inputs (GemmaPerLayerInputs, gemma4.hpp:127-135)
    launch_gemma_embed(embedding_.get(), c.V, c.D, ple_table_.get(), PL, step + 1, embed_scale_, token_scale_, x, st.act_.get(), st.tok_.get<float>(), s);
    launch_gemv_q8(ple_proj_.get(), st.act_.get(), st.ctx_.get<float>(), nullptr, PL, c.D, kEpiStore, s);
    launch_gemma_ple_inputs(st.ctx_.get<float>(), st.tok_.get<float>(), ple_norm_.get<float>(), c.eps, proj_scale_, comb_scale_, st.ple_.get<float>(), c.L, c.P, s);
    launch_rmsnorm_quant(x, layers_[0].attn_norm.get<float>(), c.eps, nullptr, st.act_.get(), 1, c.D, s);
    GemvInput qkv_in = act_input(st.act_, c.D);  // after layer 0: the previous layer's end
    for (int64_t l = 0; l < c.L; ++l) {
        const Gemma4Layer& L = layers_[size_t(l)];
        const int64_t QW = c.Hq * L.dh, KW = c.Hkv * L.dh;
        gemv_in(L.w_qkv, qkv_in, st.act_, st.proj_.get<float>(), L.n_qkv, c.D, s);
        GemmaAttnArgs a{};
        a.proj = st.proj_.get<float>();
        a.k_off = QW;
        a.v_off = QW + KW;
        a.q_gamma = L.q_norm.get<float>();
        a.k_gamma = L.shared ? nullptr : L.k_norm.get<float>();
        a.eps = c.eps;
        a.rope_cs = (L.full ? rope_full_ : rope_local_).get<float>();
        a.pos = step;
        a.k_cache = st.k_cache_[size_t(L.src)].get<float>();
        a.v_cache = st.v_cache_[size_t(L.src)].get<float>();
        a.slots = st.slots_[size_t(L.src)];
        a.window = L.full ? 0 : int(c.window);
        a.append = L.shared ? 0 : 1;
        a.q_rot = st.q_rot_.get<float>();
        a.scores = st.scores_.get<float>();
        a.max_ctx = st.max_tokens_;
        a.act_out = st.act_o_.get();
        a.Hq = int(c.Hq);
        a.Hkv = int(c.Hkv);
        a.Dh = int(L.dh);
        launch_gemma_attention(a, s);
        launch_gemv_q8(L.w_o.get(), st.act_o_.get(), st.a_.get<float>(), nullptr, c.D, QW, kEpiStore, s);
        // the sub-block ends: H = X + post_attn_norm(attn), H = H + post_ffn_norm(ffn),
        // then the PLE branch and layer_output_scale (gemma4.hpp:102-104, 258-272)
        const GemvInput ffn_in = sub_block_end({st.a_.get<float>(), L.post_attn_norm.get<float>(), x, 1.f, st.h_.get<float>(), L.ffn_norm.get<float>()}, c.eps, st.act_, c.D, s);
        gelu_gated_pair(L.w_gate_up, ffn_in, st.act_, st.gu_.get<float>(), 2 * c.FF, c.D, st.gu_.get<float>() + c.FF, L.w_down, st.act_ff_, st.a_.get<float>(), c.D, c.FF, s);
        const GemvInput ple_in = sub_block_end({st.a_.get<float>(), L.post_ffn_norm.get<float>(), st.h_.get<float>(), 1.f, st.h2_.get<float>(), nullptr}, c.eps, st.act_, c.D, s);
        gelu_gated_pair(L.w_pgate, ple_in, st.act_, st.pg_.get<float>(), c.P, c.D, st.ple_.get<float>() + l * c.P, L.w_proj, st.act_p_, st.a_.get<float>(), c.D, c.P, s);
        // the next layer's attention norm, or after the last layer the final norm
        const float* next = l + 1 < c.L ? layers_[size_t(l + 1)].attn_norm.get<float>() : final_norm_.get<float>();
        qkv_in = sub_block_end({st.a_.get<float>(), L.post_norm.get<float>(), st.h2_.get<float>(), L.out_scale, x, next}, c.eps, st.act_, c.D, s);
    }
    // tied head over the final norm's output, soft-cap, argmax into the step's id
    gemv_in(embedding_, qkv_in, st.act_, st.logits_.get<float>(), c.V, c.D, s);
    launch_gemma_softcap(st.logits_.get<float>(), c.V, c.softcap, s);
    launch_argmax(st.logits_.get<float>(), 1, c.V, step + 1, st.argmax_scratch_.get<uint64_t>(), s);
    check_launch("gemma4 step");
}

void Gemma4Model::embed(const int32_t* ids, int64_t n, float* out) const {
    const Gemma4Config& c = c_;
    if (n <= 0) throw Error(HERO_EINVAL, "embed: empty input");
    for (int64_t t = 0; t < n; ++t)
        if (ids[t] < 0 || ids[t] >= c.V) throw Error(HERO_EINVAL, "embed: token id out of range");
    DeviceBuffer id(4), x(size_t(c.D) * 4), act(size_t(act_q8_bytes(1, c.D))), tok(size_t(c.P * c.L) * 4);
    for (int64_t t = 0; t < n; ++t) {
        hip_check(hipMemcpyAsync(id.get(), ids + t, 4, hipMemcpyHostToDevice, stream_), "id upload");
        launch_gemma_embed(embedding_.get(), c.V, c.D, ple_table_.get(), c.P * c.L, id.get<int32_t>(), embed_scale_, token_scale_, x.get<float>(), act.get(),
                           tok.get<float>(), stream_);
        hip_check(hipMemcpyAsync(out + t * c.D, x.get(), size_t(c.D) * 4, hipMemcpyDeviceToHost, stream_), "rows download");
    }
    hip_check(hipStreamSynchronize(stream_), "embed");
}

void Gemma4Model::forward(State& st, const int32_t* ids, int64_t T, float* logits, int32_t* next_id) const {
    const Gemma4Config& c = c_;
    if (&st.m_ != this) throw Error(HERO_EINVAL, "forward: state belongs to another model");
    if (T <= 0) throw Error(HERO_EINVAL, "forward: empty input");
    if (T > st.max_tokens_ - st.tokens_) throw Error(HERO_ERANGE, "Gemma4Model: context exhausted");
    for (int64_t t = 0; t < T; ++t)
        if (ids[t] < 0 || ids[t] >= c.V) throw Error(HERO_EINVAL, "forward: token id out of range");
    hipStream_t s = stream_;
    try {
        for (int64_t t = 0; t < T; ++t) {
            hipLaunchKernelGGL(gemma_set_step_kernel, dim3(1), dim3(1), 0, s, st.step_.get<int32_t>(), int32_t(st.tokens_ + t), ids[t], -1);
            enqueue_step(st);
        }
        if (logits) hip_check(hipMemcpyAsync(logits, st.logits_.get(), size_t(c.V) * 4, hipMemcpyDeviceToHost, s), "logits download");
        int32_t scalars[4] = {0, 0, 0, 0};
        hip_check(hipMemcpyAsync(scalars, st.step_.get(), 16, hipMemcpyDeviceToHost, s), "step download");
        hip_check(hipStreamSynchronize(s), "forward");
        if (next_id) *next_id = scalars[1];
        st.tokens_ += T;
        hipLaunchKernelGGL(gemma_set_step_kernel, dim3(1), dim3(1), 0, s, st.step_.get<int32_t>(), int32_t(st.tokens_), -1, -1);
    } catch (...) {
        // the carried state is now unknown: forget it (transformer.hpp:139-142)
        (void)hipStreamSynchronize(s);
        st.reset();
        throw;
    }
}

void Gemma4Model::decode_greedy(State& st, int32_t first_id, int64_t steps, int32_t* out_ids, float* logits) const {
    const Gemma4Config& c = c_;
    if (&st.m_ != this) throw Error(HERO_EINVAL, "decode: state belongs to another model");
    if (steps <= 0) throw Error(HERO_EINVAL, "decode: steps must be positive");
    if (first_id < 0 || first_id >= c.V) throw Error(HERO_EINVAL, "decode: token id out of range");
    if (steps > st.max_tokens_ - st.tokens_) throw Error(HERO_ERANGE, "Gemma4Model: context exhausted");
    hipStream_t s = stream_;
    try {
        if (st.out_ids_capacity_ < steps) {
            st.out_ids_ = DeviceBuffer(size_t(steps) * 4);
            st.out_ids_capacity_ = steps;
            if (st.graph_) {  // the graph records the old buffer's address
                (void)hipGraphExecDestroy(st.graph_);
                st.graph_ = nullptr;
            }
        }
        if (!st.graph_) {
            hipGraph_t graph = nullptr;
            hip_check(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "capture begin");
            enqueue_step(st);
            hipLaunchKernelGGL(gemma_advance_step_kernel, dim3(1), dim3(1), 0, s, st.step_.get<int32_t>(), st.out_ids_.get<int32_t>(), 1);
            hip_check(hipStreamEndCapture(s, &graph), "capture end");
            hip_check(hipGraphInstantiate(&st.graph_, graph, nullptr, nullptr, 0), "graph instantiate");
            (void)hipGraphDestroy(graph);
        }
        hipLaunchKernelGGL(gemma_set_step_kernel, dim3(1), dim3(1), 0, s, st.step_.get<int32_t>(), int32_t(st.tokens_), first_id, 0);
        hip_check(hipEventRecord(ev_start_, s), "event");
        for (int64_t i = 0; i < steps; ++i) hip_check(hipGraphLaunch(st.graph_, s), "graph launch");
        hip_check(hipEventRecord(ev_stop_, s), "event");
        hip_check(hipMemcpyAsync(out_ids, st.out_ids_.get(), size_t(steps) * 4, hipMemcpyDeviceToHost, s), "ids download");
        if (logits) hip_check(hipMemcpyAsync(logits, st.logits_.get(), size_t(c.V) * 4, hipMemcpyDeviceToHost, s), "logits download");
        hip_check(hipStreamSynchronize(s), "decode");
        float ms = 0.f;
        hip_check(hipEventElapsedTime(&ms, ev_start_, ev_stop_), "event time");
        last_decode_seconds_ = double(ms) * 1e-3;
        st.tokens_ += steps;
    } catch (...) {
        (void)hipStreamSynchronize(s);
        st.reset();
        throw;
    }
}

}  // namespace hero
