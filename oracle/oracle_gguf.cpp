// oracle_gguf.cpp -- GGUF v3 reader, Qwen 3.5 and Gemma 4 loaders for the oracle.
// TEST INFRASTRUCTURE ONLY. Restates nm/src/gguf.cpp:130-230 (header,
// metadata, tensor table, aligned data start, per-tensor bounds checks) and
// nm/src/qwen35_loader.hpp:30-155 (schema validation, ssm_a sign
// normalisation), with dimensions read from the metadata instead of a
// compile-time config.
#include "oracle_gguf.hpp"

#include <cmath>
#include <cstring>
#include <fcntl.h>
#include <stdexcept>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

namespace oracle {

namespace {
struct Cursor {
    const uint8_t* p;
    const uint8_t* end;
    void need(size_t n) const {
        if (size_t(end - p) < n) throw std::runtime_error("GGUF: truncated file");
    }
    template <class T>
    T read() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = read<uint64_t>();
        need(n);
        std::string s(reinterpret_cast<const char*>(p), n);
        p += n;
        return s;
    }
};

double read_number(Cursor& c, uint32_t type) {
    switch (type) {
        case 0: return c.read<uint8_t>();
        case 1: return c.read<int8_t>();
        case 2: return c.read<uint16_t>();
        case 3: return c.read<int16_t>();
        case 4: return c.read<uint32_t>();
        case 5: return c.read<int32_t>();
        case 6: return c.read<float>();
        case 7: return c.read<uint8_t>() != 0;
        case 10: return double(c.read<uint64_t>());
        case 11: return double(c.read<int64_t>());
        case 12: return c.read<double>();
        default: throw std::runtime_error("GGUF: bad value type");
    }
}

size_t type_bytes(uint32_t type, uint64_t nelem) {
    switch (type) {
        case 0: return nelem * 4;            // F32
        case 1: return nelem * 2;            // F16
        case 8: return nelem / 32 * 34;      // Q8_0
        case 12: return nelem / 256 * 144;   // Q4_K
        case 13: return nelem / 256 * 176;   // Q5_K
        case 14: return nelem / 256 * 210;   // Q6_K
        default: throw std::runtime_error("GGUF: tensor type " + std::to_string(type) + " is not supported by this path (F32/F16/Q8_0/Q4_K/Q5_K/Q6_K)");
    }
}
size_t type_block(uint32_t type) { return type == 8 ? 32 : type >= 12 && type <= 14 ? 256 : 1; }
}  // namespace

void Gguf::parse(const uint8_t* base, size_t size) {
    base_ = base;
    size_ = size;
    Cursor c{base, base + size};
    if (c.read<uint32_t>() != 0x46554747u) throw std::runtime_error("GGUF: bad magic (not a GGUF file)");
    const uint32_t version = c.read<uint32_t>();
    if (version != 3) throw std::runtime_error("GGUF: unsupported version " + std::to_string(version) + " (expect 3)");
    const uint64_t tensor_count = c.read<uint64_t>();
    const uint64_t kv_count = c.read<uint64_t>();
    for (uint64_t i = 0; i < kv_count; ++i) {
        const std::string key = c.str();
        Value v;
        v.type = c.read<uint32_t>();
        if (v.type == 8) {
            v.str = c.str();
        } else if (v.type == 9) {
            const uint32_t et = c.read<uint32_t>();
            const uint64_t n = c.read<uint64_t>();
            for (uint64_t j = 0; j < n; ++j) {
                if (et == 8) v.arr_str.push_back(c.str());
                else v.arr_num.push_back(read_number(c, et));
            }
        } else {
            v.num = read_number(c, v.type);
        }
        meta_[key] = std::move(v);
    }
    uint64_t alignment = has("general.alignment") ? uint64_t(meta_.at("general.alignment").num) : 32;
    if (alignment == 0) alignment = 32;
    if ((alignment & (alignment - 1)) != 0) throw std::runtime_error("GGUF: general.alignment is not a power of two");
    for (uint64_t i = 0; i < tensor_count; ++i) {
        Tensor t;
        t.name = c.str();
        const uint32_t nd = c.read<uint32_t>();
        for (uint32_t d = 0; d < nd; ++d) t.dims.push_back(c.read<uint64_t>());
        t.type = c.read<uint32_t>();
        t.offset = c.read<uint64_t>();
        tensors_.push_back(std::move(t));
    }
    const uint64_t header_end = uint64_t(c.p - base);
    const uint64_t data_start = (header_end + alignment - 1) & ~(alignment - 1);
    if (!tensors_.empty() && data_start > size) throw std::runtime_error("GGUF: data section starts past end of file");
    for (Tensor& t : tensors_) {
        if (t.offset % alignment != 0) throw std::runtime_error("GGUF: tensor '" + t.name + "' offset is misaligned");
        if (t.offset > size - data_start) throw std::runtime_error("GGUF: tensor '" + t.name + "' data out of range");
        uint64_t n = 1;
        for (uint64_t d : t.dims) n *= d;
        if (n % type_block(t.type) != 0) throw std::runtime_error("GGUF: tensor '" + t.name + "' has a partial quant block");
        const uint64_t bytes = type_bytes(t.type, n);
        const uint64_t abs = data_start + t.offset;
        if (bytes > size - abs) throw std::runtime_error("GGUF: tensor '" + t.name + "' data out of range");
        t.data = base + abs;
        t.nelem = n;
    }
}

void Gguf::open(const std::string& path) {
    fd_ = ::open(path.c_str(), O_RDONLY);
    if (fd_ < 0) throw std::runtime_error("GGUF: cannot open " + path);
    struct stat st{};
    if (::fstat(fd_, &st) != 0) throw std::runtime_error("GGUF: fstat failed");
    map_size_ = size_t(st.st_size);
    map_ = ::mmap(nullptr, map_size_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (map_ == MAP_FAILED) {
        map_ = nullptr;
        throw std::runtime_error("GGUF: mmap failed");
    }
    parse(static_cast<const uint8_t*>(map_), map_size_);
}

Gguf::~Gguf() {
    if (map_) ::munmap(map_, map_size_);
    if (fd_ >= 0) ::close(fd_);
}

const Gguf::Tensor* Gguf::find(const std::string& name) const {
    for (const Tensor& t : tensors_)
        if (t.name == name) return &t;
    return nullptr;
}
const Gguf::Tensor& Gguf::require(const std::string& name) const {
    const Tensor* t = find(name);
    if (!t) throw std::runtime_error("GGUF: required tensor '" + name + "' not found");
    return *t;
}
double Gguf::num(const std::string& key) const {
    auto it = meta_.find(key);
    if (it == meta_.end()) throw std::runtime_error("qwen35 loader: missing metadata key " + key);
    return it->second.num;
}

// ---- loader ----------------------------------------------------------------
namespace {
void expect(bool ok, const std::string& msg) {
    if (!ok) throw std::runtime_error("qwen35 loader: " + msg);
}
std::string blk(size_t l, const char* s) { return "blk." + std::to_string(l) + "." + s; }

Linear load_linear(const Gguf& g, const std::string& name, size_t in, size_t out) {
    const Gguf::Tensor& t = g.require(name);
    expect(t.dims.size() == 2 && t.dims[0] == in && t.dims[1] == out, name + " has the wrong shape");
    // tensor_loader::load_weight (tensor_loader.hpp:17-35) for the quantized types
    expect(t.type == 8 || t.type == 12 || t.type == 13 || t.type == 14, name + " is not Q8_0, Q4_K, Q5_K or Q6_K");
    expect(in % type_block(t.type) == 0, name + " In not divisible by its block length");
    return Linear{t.data, int(t.type), out, in};
}

std::vector<float> load_vector(const Gguf& g, const std::string& name, size_t n) {
    const Gguf::Tensor& t = g.require(name);
    expect(t.nelem == n, name + " has the wrong length");
    std::vector<float> v(n);
    if (t.type == 0) {
        std::memcpy(v.data(), t.data, n * 4);
    } else if (t.type == 1) {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(t.data);
        for (size_t i = 0; i < n; ++i) v[i] = fp16_to_fp32(h[i]);
    } else {
        throw std::runtime_error("qwen35 loader: " + name + " must be F32 or F16");
    }
    return v;
}
}  // namespace

Model load_qwen35(const Gguf& g) {
    expect(g.str("general.architecture") == "qwen35", "general.architecture is not 'qwen35'");
    Config c;
    c.L = size_t(g.num("qwen35.block_count"));
    c.D = size_t(g.num("qwen35.embedding_length"));
    c.FF = size_t(g.num("qwen35.feed_forward_length"));
    c.Hq = size_t(g.num("qwen35.attention.head_count"));
    c.Hkv = size_t(g.num("qwen35.attention.head_count_kv"));
    c.head_dim = size_t(g.num("qwen35.attention.key_length"));
    expect(size_t(g.num("qwen35.attention.value_length")) == c.head_dim, "attention value_length != key_length");
    c.eps = float(g.num("qwen35.attention.layer_norm_rms_epsilon"));
    c.rope_base = double(float(g.num("qwen35.rope.freq_base")));
    c.rotary_dims = size_t(g.num("qwen35.rope.dimension_count"));
    c.conv_width = size_t(g.num("qwen35.ssm.conv_kernel"));
    c.Dk = size_t(g.num("qwen35.ssm.state_size"));
    c.Hk = size_t(g.num("qwen35.ssm.group_count"));
    c.Hv = size_t(g.num("qwen35.ssm.time_step_rank"));
    const size_t inner = size_t(g.num("qwen35.ssm.inner_size"));
    expect(c.Hv != 0 && inner % c.Hv == 0, "ssm.inner_size is not a whole number of value heads");
    c.Dv = inner / c.Hv;
    expect(c.Dk == c.Dv, "the delta rule requires Dk == Dv");
    expect(c.Hk != 0 && c.Hv % c.Hk == 0, "value heads must be a multiple of key heads");
    expect(c.Hkv != 0 && c.Hq % c.Hkv == 0, "query heads must be a multiple of K/V heads");
    expect(c.rotary_dims <= c.head_dim && c.rotary_dims % 2 == 0, "rope.dimension_count out of range");
    c.full_attention_interval = g.has("qwen35.full_attention_interval") ? size_t(g.num("qwen35.full_attention_interval")) : 4;
    expect(c.full_attention_interval == 4, "full_attention_interval must be 4");
    if (g.has("qwen35.attention.recurrent_layers")) {
        const auto& arr = g.meta().at("qwen35.attention.recurrent_layers").arr_num;
        expect(arr.size() >= c.L, "qwen35.attention.recurrent_layers is shorter than block_count");
        for (size_t l = 0; l < c.L; ++l) expect((arr[l] != 0) == c.is_recurrent(l), "layer " + std::to_string(l) + " disagrees with the hybrid schedule");
    }
    c.CTX = g.has("qwen35.context_length") ? size_t(g.num("qwen35.context_length")) : 262144;
    expect(c.L % 4 == 0, "block_count must be a multiple of the 4-layer schedule");

    const Gguf::Tensor& emb = g.require("token_embd.weight");
    expect(emb.dims.size() == 2 && emb.dims[0] == c.D, "token_embd.weight has the wrong shape");
    c.V = size_t(emb.dims[1]);
    c.tied = g.find("output.weight") == nullptr;

    Model m;
    m.c = c;
    m.embedding = load_linear(g, "token_embd.weight", c.D, c.V);
    m.output = c.tied ? m.embedding : load_linear(g, "output.weight", c.D, c.V);
    m.final_norm = load_vector(g, "output_norm.weight", c.D);
    m.inv_freq = rope_inv_freq(c.head_dim, c.rope_base, c.rotary_dims);
    const size_t CC = c.conv_channels();
    for (size_t l = 0; l < c.L; ++l) {
        Layer L;
        L.mixer_norm = load_vector(g, blk(l, "attn_norm.weight"), c.D);
        L.channel_norm = load_vector(g, blk(l, "post_attention_norm.weight"), c.D);
        L.gate = load_linear(g, blk(l, "ffn_gate.weight"), c.D, c.FF);
        L.up = load_linear(g, blk(l, "ffn_up.weight"), c.D, c.FF);
        L.down = load_linear(g, blk(l, "ffn_down.weight"), c.FF, c.D);
        if (c.is_recurrent(l)) {
            L.wqkv = load_linear(g, blk(l, "attn_qkv.weight"), c.D, CC);
            L.wz = load_linear(g, blk(l, "attn_gate.weight"), c.D, c.Hv * c.Dv);
            L.wbeta = load_linear(g, blk(l, "ssm_beta.weight"), c.D, c.Hv);
            L.walpha = load_linear(g, blk(l, "ssm_alpha.weight"), c.D, c.Hv);
            L.wout = load_linear(g, blk(l, "ssm_out.weight"), c.Hv * c.Dv, c.D);
            const Gguf::Tensor& conv = g.require(blk(l, "ssm_conv1d.weight"));
            expect(conv.dims.size() == 2 && conv.dims[0] == c.conv_width && conv.dims[1] == CC, blk(l, "ssm_conv1d.weight") + " has the wrong shape");
            L.conv = load_vector(g, blk(l, "ssm_conv1d.weight"), CC * c.conv_width);
            L.dt_bias = load_vector(g, blk(l, "ssm_dt.bias"), c.Hv);
            L.decay_scale = load_vector(g, blk(l, "ssm_a"), c.Hv);
            for (float& a : L.decay_scale) {  // qwen35_loader.hpp:108-119
                if (a > 0.f) a = -std::exp(a);
                expect(a <= 0.f, blk(l, "ssm_a") + ": decay scale must be <= 0 (-exp(A_log))");
            }
            L.ssm_norm = load_vector(g, blk(l, "ssm_norm.weight"), c.Dv);
        } else {
            L.wqg = load_linear(g, blk(l, "attn_q.weight"), c.D, 2 * c.Hq * c.head_dim);
            L.q_norm = load_vector(g, blk(l, "attn_q_norm.weight"), c.head_dim);
            L.wk = load_linear(g, blk(l, "attn_k.weight"), c.D, c.Hkv * c.head_dim);
            L.k_norm = load_vector(g, blk(l, "attn_k_norm.weight"), c.head_dim);
            L.wv = load_linear(g, blk(l, "attn_v.weight"), c.D, c.Hkv * c.head_dim);
            L.wo = load_linear(g, blk(l, "attn_output.weight"), c.Hq * c.head_dim, c.D);
        }
        m.layers.push_back(std::move(L));
    }
    return m;
}

// validate_e4b_text_metadata (gemma4_loader.hpp:31-52) with the dimensions
// read from the metadata, then load_e4b_text (:105-130). Layers that reuse
// K/V load no K/V tensors (:95-103).
Gemma4Model load_gemma4(const Gguf& g) {
    expect(g.str("general.architecture") == "gemma4", "general.architecture is not 'gemma4'");
    Gemma4Config c;
    c.L = size_t(g.num("gemma4.block_count"));
    c.D = size_t(g.num("gemma4.embedding_length"));
    c.FF = size_t(g.num("gemma4.feed_forward_length"));
    c.Hq = size_t(g.num("gemma4.attention.head_count"));
    c.Hkv = size_t(g.num("gemma4.attention.head_count_kv"));
    c.Df = size_t(g.num("gemma4.attention.key_length"));
    expect(size_t(g.num("gemma4.attention.value_length")) == c.Df, "attention.value_length != key_length");
    c.Dl = size_t(g.num("gemma4.attention.key_length_swa"));
    expect(size_t(g.num("gemma4.attention.value_length_swa")) == c.Dl, "attention.value_length_swa != key_length_swa");
    c.window = size_t(g.num("gemma4.attention.sliding_window"));
    c.shared = size_t(g.num("gemma4.attention.shared_kv_layers"));
    c.P = size_t(g.num("gemma4.embedding_length_per_layer_input"));
    c.eps = float(g.num("gemma4.attention.layer_norm_rms_epsilon"));
    c.softcap = float(g.num("gemma4.final_logit_softcapping"));
    c.CTX = g.has("gemma4.context_length") ? size_t(g.num("gemma4.context_length")) : 131072;
    // gemma4.hpp:396-397: local heads rotate every plane (base 1e4), full
    // heads their first quarter (base 1e6)
    c.local_base = g.has("gemma4.rope.freq_base_swa") ? double(float(g.num("gemma4.rope.freq_base_swa"))) : 1e4;
    c.full_base = g.has("gemma4.rope.freq_base") ? double(float(g.num("gemma4.rope.freq_base"))) : 1e6;
    c.local_rot = g.has("gemma4.rope.dimension_count_swa") ? size_t(g.num("gemma4.rope.dimension_count_swa")) : c.Dl;
    c.full_rot = g.has("gemma4.rope.dimension_count") ? size_t(g.num("gemma4.rope.dimension_count")) : c.Df / 4;
    expect(c.Hkv != 0 && c.Hq % c.Hkv == 0, "query heads must be a multiple of K/V heads");
    expect(c.L >= 1 && c.shared < c.L && c.window > 0 && c.P > 0, "block_count / shared_kv_layers / sliding_window / per-layer width out of range");
    expect(c.local_rot <= c.Dl && c.full_rot <= c.Df, "rope dimension counts out of range");
    const Gguf::Tensor& emb = g.require("token_embd.weight");
    expect(emb.dims.size() == 2 && emb.dims[0] == c.D, "token_embd.weight has the wrong shape");
    c.V = size_t(emb.dims[1]);
    for (size_t l = 0; l < c.L; ++l) (void)c.kv_source(l);

    Gemma4Model m;
    m.c = c;
    const size_t PL = c.P * c.L;
    m.embedding = load_linear(g, "token_embd.weight", c.D, c.V);
    m.ple_table = load_linear(g, "per_layer_token_embd.weight", PL, c.V);
    m.ple_proj = load_linear(g, "per_layer_model_proj.weight", c.D, PL);
    m.ple_norm = load_vector(g, "per_layer_proj_norm.weight", c.P);
    m.final_norm = load_vector(g, "output_norm.weight", c.D);
    m.inv_local = rope_inv_freq(c.Dl, c.local_base, c.local_rot);
    m.inv_full = rope_inv_freq(c.Df, c.full_base, c.full_rot);
    for (size_t l = 0; l < c.L; ++l) {
        Gemma4Layer L;
        const size_t dh = c.head_dim(l);
        L.attn_norm = load_vector(g, blk(l, "attn_norm.weight"), c.D);
        L.wq = load_linear(g, blk(l, "attn_q.weight"), c.D, c.Hq * dh);
        L.q_norm = load_vector(g, blk(l, "attn_q_norm.weight"), dh);
        if (!c.shares_kv(l)) {
            L.wk = load_linear(g, blk(l, "attn_k.weight"), c.D, c.Hkv * dh);
            L.k_norm = load_vector(g, blk(l, "attn_k_norm.weight"), dh);
            L.wv = load_linear(g, blk(l, "attn_v.weight"), c.D, c.Hkv * dh);
        }
        L.wo = load_linear(g, blk(l, "attn_output.weight"), c.Hq * dh, c.D);
        L.post_attn_norm = load_vector(g, blk(l, "post_attention_norm.weight"), c.D);
        L.ffn_norm = load_vector(g, blk(l, "ffn_norm.weight"), c.D);
        L.gate = load_linear(g, blk(l, "ffn_gate.weight"), c.D, c.FF);
        L.up = load_linear(g, blk(l, "ffn_up.weight"), c.D, c.FF);
        L.down = load_linear(g, blk(l, "ffn_down.weight"), c.FF, c.D);
        L.post_ffn_norm = load_vector(g, blk(l, "post_ffw_norm.weight"), c.D);
        L.pgate = load_linear(g, blk(l, "inp_gate.weight"), c.D, c.P);
        L.proj = load_linear(g, blk(l, "proj.weight"), c.P, c.D);
        L.post_norm = load_vector(g, blk(l, "post_norm.weight"), c.D);
        if (g.find(blk(l, "layer_output_scale.weight"))) L.out_scale = load_vector(g, blk(l, "layer_output_scale.weight"), 1)[0];
        m.layers.push_back(std::move(L));
    }
    return m;
}

}  // namespace oracle
