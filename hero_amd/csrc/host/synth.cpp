// synth.cpp -- seeded random-init Qwen 3.5-style hybrid models written as
// GGUF v3 images with Q8_0 weights, in the `qwen35` schema that
// nm/src/qwen35_loader.hpp:30-155 reads.
//
// Every element is a pure function of (seed, tensor index, element index):
// a splitmix64 counter hash of the element pair gives two 24-bit uniforms,
// Box-Muller (in fp32) gives the pair of standard normals, and the value is
// scale*normal in fp32. 2-D tensors are then quantized to Q8_0 with the reference weight quantizer
// (nm/src/quant.hpp:404-413: d = amax/127, q = lround(x/d), d stored through
// the reference fp16 encoder). Rows are generated in parallel; the bytes do
// not depend on the thread count.
//
// Fixed choices the workload description leaves open:
//   2-D weights N(0, 0.02); RMSNorm / q_norm / k_norm / ssm_norm gamma = 1;
//   conv taps N(0, 0.5); ssm_a = -exp(N(0, 0.5)); ssm_dt.bias = 0;
//   rope.dimension_count = head_dim/4 (Qwen 3.5's partial rotary factor).
#include "hero/synth.hpp"

#include "hero/fp16.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

namespace hero {

namespace {

inline uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// Standard normals for elements 2p and 2p+1 of a stream: one counter hash
// gives two 24-bit uniforms, Box-Muller (in fp32) gives the pair.
inline void normal_pair(uint64_t stream, uint64_t p, float* z0, float* z1) {
    const uint64_t h = splitmix64(stream ^ splitmix64(p));
    const float u1 = (float(uint32_t(h >> 40)) + 0.5f) * (1.f / 16777216.f);            // (0,1)
    const float u2 = float(uint32_t(h >> 8) & 0xFFFFFFu) * (1.f / 16777216.f);          // [0,1)
    const float r = std::sqrt(-2.f * std::log(u1));
    const float a = 6.2831853f * u2;
    *z0 = r * std::cos(a);
    *z1 = r * std::sin(a);
}
inline float normal_at(uint64_t stream, uint64_t i) {
    float z0, z1;
    normal_pair(stream, i >> 1, &z0, &z1);
    return (i & 1) ? z1 : z0;
}

inline uint64_t stream_of(uint64_t seed, uint64_t tensor_index) { return splitmix64(seed * 0x632BE59BD9B4E019ull + tensor_index + 1); }

// Reference weight quantizer for one 32-block.
void quantize_block_lround(const float* x, uint8_t* out34) {
    float amax = 0.f;
    for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(x[j]));
    const float d = amax / 127.f;
    const float id = d != 0.f ? 1.f / d : 0.f;
    const uint16_t dh = fp32_to_fp16_ref(d);
    std::memcpy(out34, &dh, 2);
    for (int j = 0; j < 32; ++j) out34[2 + j] = uint8_t(int8_t(std::lround(x[j] * id)));
}

// ---- K-quant blocks of 256 weights (GGUF types 12, 13, 14) -------------------
// A plain min/max quantizer per 32 (Q4_K, Q5_K) or 16 (Q6_K) weights, with the
// sub-block scales and mins quantized against the block's largest ones; the
// byte layouts are ggml's (the ones nm/src/quant.hpp:153-300 decodes). These
// synthetic fixtures only need to be valid blocks whose decoded weights follow
// the floats roughly; both the reference and this build decode the bytes.
inline int nearest(float v) { return int(std::lround(v)); }

// 6-bit scale / min j (0..7) into the 12-byte packing get_scale_min_k4 reads
void put_scale_min_k4(uint8_t* q, int j, int sc, int m) {
    if (j < 4) {
        q[j] = uint8_t((q[j] & 0xC0) | sc);
        q[j + 4] = uint8_t((q[j + 4] & 0xC0) | m);
    } else {
        q[j + 4] = uint8_t((sc & 0xF) | ((m & 0xF) << 4));
        q[j - 4] = uint8_t(q[j - 4] | ((sc >> 4) << 6));
        q[j] = uint8_t(q[j] | ((m >> 4) << 6));
    }
}

// Q4_K (bits = 4, 144 bytes) or Q5_K (bits = 5, 176 bytes): weight i of
// sub-block j (32 weights) = d*sc_j*q - dmin*m_j, q in [0, 2^bits - 1]
void quantize_block_q45_k(const float* x, uint8_t* out, int bits) {
    const int qmax = (1 << bits) - 1;
    float scale[8], minv[8];
    for (int j = 0; j < 8; ++j) {
        float lo = x[32 * j], hi = x[32 * j];
        for (int i = 1; i < 32; ++i) lo = std::min(lo, x[32 * j + i]), hi = std::max(hi, x[32 * j + i]);
        lo = std::min(lo, 0.f);  // the min term subtracts: keep it >= 0
        scale[j] = (hi - lo) / float(qmax);
        minv[j] = -lo;
    }
    const float max_scale = *std::max_element(scale, scale + 8), max_min = *std::max_element(minv, minv + 8);
    const uint16_t dh = fp32_to_fp16_ref(max_scale / 63.f), mh = fp32_to_fp16_ref(max_min / 63.f);
    const float d = fp16_to_fp32_ref(dh), dmin = fp16_to_fp32_ref(mh);
    uint8_t scales[12] = {0};
    int sc[8], mn[8];
    for (int j = 0; j < 8; ++j) {
        sc[j] = d > 0.f ? std::min(63, std::max(0, nearest(scale[j] / d))) : 0;
        mn[j] = dmin > 0.f ? std::min(63, std::max(0, nearest(minv[j] / dmin))) : 0;
        put_scale_min_k4(scales, j, sc[j], mn[j]);
    }
    uint8_t qs[128] = {0}, qh[32] = {0};
    for (int j = 0; j < 8; ++j) {
        const float step = d * float(sc[j]), off = dmin * float(mn[j]);
        for (int i = 0; i < 32; ++i) {
            const int q = step > 0.f ? std::min(qmax, std::max(0, nearest((x[32 * j + i] + off) / step))) : 0;
            // sub-blocks 2p and 2p+1 share qs[32p .. 32p+31]: low and high nibbles
            qs[32 * (j / 2) + i] = uint8_t(qs[32 * (j / 2) + i] | ((q & 0xF) << (4 * (j & 1))));
            if (bits == 5 && (q & 16)) qh[i] = uint8_t(qh[i] | (1 << j));  // bit j of qh[i]
        }
    }
    std::memcpy(out, &dh, 2);
    std::memcpy(out + 2, &mh, 2);
    std::memcpy(out + 4, scales, 12);
    if (bits == 5) {
        std::memcpy(out + 16, qh, 32);
        std::memcpy(out + 48, qs, 128);
    } else {
        std::memcpy(out + 16, qs, 128);
    }
}

// Q6_K (210 bytes): weight = d*sc_g*q, q in [-32, 31], an int8 scale per 16
void quantize_block_q6_k(const float* x, uint8_t* out) {
    float scale[16];
    for (int g = 0; g < 16; ++g) {
        float amax = 0.f;
        for (int i = 0; i < 16; ++i) amax = std::max(amax, std::fabs(x[16 * g + i]));
        scale[g] = amax / 31.f;
    }
    const float max_scale = *std::max_element(scale, scale + 16);
    const uint16_t dh = fp32_to_fp16_ref(max_scale / 127.f);
    const float d = fp16_to_fp32_ref(dh);
    int8_t sc[16];
    for (int g = 0; g < 16; ++g) sc[g] = int8_t(d > 0.f ? std::min(127, nearest(scale[g] / d)) : 0);
    uint8_t ql[128] = {0}, qh[64] = {0};
    for (int p = 0; p < 256; ++p) {
        const float step = d * float(sc[p / 16]);
        const int q = (step > 0.f ? std::min(31, std::max(-32, nearest(x[p] / step))) : 0) + 32;  // 0..63
        // half h (128 weights): element e lives in ql[64h + e % 64] (low nibble for
        // e < 64, high for e >= 64) and qh[32h + e % 32] at bit 2 (e / 32)
        const int h = p / 128, e = p % 128;
        ql[64 * h + e % 64] = uint8_t(ql[64 * h + e % 64] | ((q & 0xF) << (e < 64 ? 0 : 4)));
        qh[32 * h + e % 32] = uint8_t(qh[32 * h + e % 32] | ((q >> 4) << (2 * (e / 32))));
    }
    std::memcpy(out, ql, 128);
    std::memcpy(out + 128, qh, 64);
    std::memcpy(out + 192, sc, 16);
    std::memcpy(out + 208, &dh, 2);
}

template <class F>
void parallel_rows(size_t rows, F&& f) {
    size_t threads = std::max<size_t>(1, std::min<size_t>(std::thread::hardware_concurrency(), 16));
    if (const char* env = std::getenv("HERO_SYNTH_THREADS")) threads = std::max<long>(1, std::atol(env));
    threads = std::min(threads, std::max<size_t>(1, rows / 64));
    if (threads <= 1) {
        for (size_t r = 0; r < rows; ++r) f(r);
        return;
    }
    std::vector<std::thread> pool;
    for (size_t t = 0; t < threads; ++t)
        pool.emplace_back([&, t] {
            for (size_t r = t; r < rows; r += threads) f(r);
        });
    for (auto& th : pool) th.join();
}

// ---- GGUF image builder ------------------------------------------------------
enum : uint32_t { GGUF_U32 = 4, GGUF_F32 = 6, GGUF_STRING = 8, GGUF_ARRAY = 9 };
enum : uint32_t { T_F32 = 0, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14 };

uint64_t type_bytes(uint32_t type, uint64_t n) {
    switch (type) {
        case T_Q8_0: return n / 32 * 34;
        case T_Q4_K: return n / 256 * 144;
        case T_Q5_K: return n / 256 * 176;
        case T_Q6_K: return n / 256 * 210;
        default: return n * 4;
    }
}

struct TensorSpec {
    std::string name;
    uint64_t in = 0, out = 1;  // ggml dims [in, out]; a vector has out == 1 and one dim
    bool matrix = false;
    uint32_t type = T_F32;
    enum Kind { Normal, Ones, Zeros, NegExpNormal, Affine } kind = Normal;
    double scale = 0.02;
    double mean = 0.0;  // Affine: mean + scale * normal
    uint64_t offset = 0, bytes = 0;
};

struct Writer {
    std::vector<uint8_t> buf;
    void raw(const void* p, size_t n) {
        const uint8_t* b = static_cast<const uint8_t*>(p);
        buf.insert(buf.end(), b, b + n);
    }
    void u32(uint32_t v) { raw(&v, 4); }
    void u64(uint64_t v) { raw(&v, 8); }
    void f32(float v) { raw(&v, 4); }
    void str(const std::string& s) {
        u64(s.size());
        raw(s.data(), s.size());
    }
    void kv_u32(const std::string& k, uint32_t v) {
        str(k);
        u32(GGUF_U32);
        u32(v);
    }
    void kv_f32(const std::string& k, float v) {
        str(k);
        u32(GGUF_F32);
        f32(v);
    }
    void kv_str(const std::string& k, const std::string& v) {
        str(k);
        u32(GGUF_STRING);
        str(v);
    }
    void kv_u32_array(const std::string& k, const std::vector<uint32_t>& v) {
        str(k);
        u32(GGUF_ARRAY);
        u32(GGUF_U32);
        u64(v.size());
        for (uint32_t x : v) u32(x);
    }
};

std::vector<TensorSpec> tensor_specs(const SynthConfig& c) {
    std::vector<TensorSpec> t;
    // weight_mix 1: the tensor types of a Q4_K_M checkpoint (Q4_K for most
    // projections, Q5_K and Q6_K for some, Q8_0 for the small gate
    // projections); 2: Q8_0 projections (the in-projections, gate and up)
    // beside a Q6_K embedding, a Q6_K down projection and Q4_K output
    // projections; 0: Q8_0 everywhere
    auto mat = [&](const std::string& name, uint64_t in, uint64_t out, uint32_t mix1_type = T_Q8_0, uint32_t mix2_type = T_Q8_0) {
        TensorSpec s;
        s.name = name;
        s.in = in;
        s.out = out;
        s.matrix = true;
        s.type = c.weight_mix == 1 ? mix1_type : c.weight_mix == 2 ? mix2_type : T_Q8_0;
        t.push_back(s);
    };
    auto vec = [&](const std::string& name, uint64_t n, TensorSpec::Kind kind, double scale = 0.0) {
        TensorSpec s;
        s.name = name;
        s.in = n;
        s.kind = kind;
        s.scale = scale;
        t.push_back(s);
    };
    const uint64_t D = c.D, CC = 2 * c.Hk * c.Dk + c.Hv * c.Dv;
    mat("token_embd.weight", D, c.V, T_Q6_K, T_Q6_K);
    vec("output_norm.weight", D, TensorSpec::Ones);
    if (!c.tied) mat("output.weight", D, c.V, T_Q6_K);
    for (uint64_t l = 0; l < c.L; ++l) {
        const std::string b = "blk." + std::to_string(l) + ".";
        vec(b + "attn_norm.weight", D, TensorSpec::Ones);
        vec(b + "post_attention_norm.weight", D, TensorSpec::Ones);
        mat(b + "ffn_gate.weight", D, c.FF, T_Q4_K);
        mat(b + "ffn_up.weight", D, c.FF, T_Q4_K);
        mat(b + "ffn_down.weight", c.FF, D, T_Q6_K, T_Q6_K);
        if ((l + 1) % 4 != 0) {
            mat(b + "attn_qkv.weight", D, CC, T_Q5_K);
            mat(b + "attn_gate.weight", D, c.Hv * c.Dv, T_Q4_K);
            TensorSpec conv;
            conv.name = b + "ssm_conv1d.weight";
            conv.in = c.conv_width;
            conv.out = CC;
            conv.matrix = true;  // 2-D F32 [conv_width, CC]
            conv.type = T_F32;
            conv.scale = 0.5;
            t.push_back(conv);
            vec(b + "ssm_a", c.Hv, TensorSpec::NegExpNormal, 0.5);
            mat(b + "ssm_beta.weight", D, c.Hv);
            mat(b + "ssm_alpha.weight", D, c.Hv);
            vec(b + "ssm_dt.bias", c.Hv, TensorSpec::Zeros);
            vec(b + "ssm_norm.weight", c.Dv, TensorSpec::Ones);
            mat(b + "ssm_out.weight", c.Hv * c.Dv, D, T_Q4_K, T_Q4_K);
        } else {
            mat(b + "attn_q.weight", D, 2 * c.Hq * c.head_dim, T_Q4_K);
            vec(b + "attn_q_norm.weight", c.head_dim, TensorSpec::Ones);
            mat(b + "attn_k.weight", D, c.Hkv * c.head_dim, T_Q4_K);
            vec(b + "attn_k_norm.weight", c.head_dim, TensorSpec::Ones);
            mat(b + "attn_v.weight", D, c.Hkv * c.head_dim, T_Q6_K);
            mat(b + "attn_output.weight", c.Hq * c.head_dim, D, T_Q5_K, T_Q4_K);
        }
    }
    return t;
}

// magic, version, counts, the metadata `meta` writes (kv_count pairs), the
// tensor table and the aligned data start; fills each spec's offset and size
template <class Meta>
std::vector<uint8_t> gguf_header(std::vector<TensorSpec>& specs, uint64_t kv_count, Meta&& meta, uint64_t& data_start, uint64_t& total) {
    Writer w;
    w.u32(0x46554747u);
    w.u32(3);
    w.u64(specs.size());
    w.u64(kv_count);
    meta(w);
    uint64_t offset = 0;
    for (TensorSpec& s : specs) {
        const uint64_t n = s.in * s.out;
        s.bytes = type_bytes(s.type, n);
        s.offset = offset;
        offset = (offset + s.bytes + 31) & ~uint64_t(31);
        w.str(s.name);
        if (s.matrix) {
            w.u32(2);
            w.u64(s.in);
            w.u64(s.out);
        } else {
            w.u32(1);
            w.u64(s.in);
        }
        w.u32(s.type);
        w.u64(s.offset);
    }
    data_start = (w.buf.size() + 31) & ~uint64_t(31);
    total = data_start + offset;
    w.buf.resize(data_start, 0);
    return std::move(w.buf);
}

std::vector<uint8_t> header_bytes(const SynthConfig& c, std::vector<TensorSpec>& specs, uint64_t& data_start, uint64_t& total) {
    return gguf_header(specs, 20, [&](Writer& w) {
        w.kv_str("general.architecture", "qwen35");
        w.kv_u32("general.alignment", 32);
        w.kv_u32("qwen35.block_count", uint32_t(c.L));
        w.kv_u32("qwen35.context_length", uint32_t(c.ctx));
        w.kv_u32("qwen35.embedding_length", uint32_t(c.D));
        w.kv_u32("qwen35.feed_forward_length", uint32_t(c.FF));
        w.kv_u32("qwen35.attention.head_count", uint32_t(c.Hq));
        w.kv_u32("qwen35.attention.head_count_kv", uint32_t(c.Hkv));
        w.kv_u32("qwen35.attention.key_length", uint32_t(c.head_dim));
        w.kv_u32("qwen35.attention.value_length", uint32_t(c.head_dim));
        w.kv_f32("qwen35.attention.layer_norm_rms_epsilon", 1e-6f);
        w.kv_f32("qwen35.rope.freq_base", float(c.rope_base));
        w.kv_u32("qwen35.rope.dimension_count", uint32_t(c.head_dim / 4));
        w.kv_u32("qwen35.ssm.conv_kernel", uint32_t(c.conv_width));
        w.kv_u32("qwen35.ssm.state_size", uint32_t(c.Dk));
        w.kv_u32("qwen35.ssm.group_count", uint32_t(c.Hk));
        w.kv_u32("qwen35.ssm.time_step_rank", uint32_t(c.Hv));
        w.kv_u32("qwen35.ssm.inner_size", uint32_t(c.Hv * c.Dv));
        w.kv_u32("qwen35.full_attention_interval", 4);
        std::vector<uint32_t> recurrent(c.L);
        for (uint64_t l = 0; l < c.L; ++l) recurrent[l] = (l + 1) % 4 != 0;
        w.kv_u32_array("qwen35.attention.recurrent_layers", recurrent);
    }, data_start, total);
}

void fill_tensor(uint64_t seed, const TensorSpec& s, uint64_t tensor_index, uint8_t* dst) {
    const uint64_t stream = stream_of(seed, tensor_index);
    if (s.type == T_Q4_K || s.type == T_Q5_K || s.type == T_Q6_K) {
        const uint64_t in = s.in, blocks = in / 256, bb = type_bytes(s.type, 256);
        parallel_rows(s.out, [&](size_t r) {
            std::vector<float> row(in);
            const uint64_t base = uint64_t(r) * in;
            for (uint64_t i = 0; i < in; i += 2) {
                float z0, z1;
                normal_pair(stream, (base + i) >> 1, &z0, &z1);
                row[i] = 0.02f * z0;
                row[i + 1] = 0.02f * z1;
            }
            for (uint64_t b = 0; b < blocks; ++b) {
                uint8_t* o = dst + (uint64_t(r) * blocks + b) * bb;
                if (s.type == T_Q6_K)
                    quantize_block_q6_k(row.data() + b * 256, o);
                else
                    quantize_block_q45_k(row.data() + b * 256, o, s.type == T_Q5_K ? 5 : 4);
            }
        });
        return;
    }
    if (s.type == T_Q8_0) {
        const uint64_t in = s.in, blocks = in / 32;
        parallel_rows(s.out, [&](size_t r) {
            std::vector<float> row(in);
            const uint64_t base = uint64_t(r) * in;  // in is even: pairs never straddle rows
            for (uint64_t i = 0; i < in; i += 2) {
                float z0, z1;
                normal_pair(stream, (base + i) >> 1, &z0, &z1);
                row[i] = 0.02f * z0;
                row[i + 1] = 0.02f * z1;
            }
            for (uint64_t b = 0; b < blocks; ++b) quantize_block_lround(row.data() + b * 32, dst + (uint64_t(r) * blocks + b) * 34);
        });
        return;
    }
    const uint64_t n = s.in * s.out;
    float* f = reinterpret_cast<float*>(dst);
    for (uint64_t i = 0; i < n; ++i) {
        switch (s.kind) {
            case TensorSpec::Ones: f[i] = 1.f; break;
            case TensorSpec::Zeros: f[i] = 0.f; break;
            case TensorSpec::Normal: f[i] = float(s.scale) * normal_at(stream, i); break;
            case TensorSpec::NegExpNormal: f[i] = -std::exp(float(s.scale) * normal_at(stream, i)); break;
            case TensorSpec::Affine: f[i] = float(s.mean) + float(s.scale) * normal_at(stream, i); break;
        }
    }
}

void check_config(const SynthConfig& c) {
    if (c.L == 0 || c.L % 4 != 0) throw std::invalid_argument("synth: L must be a positive multiple of 4");
    if (c.D % 32 || c.FF % 32 || (c.Hv * c.Dv) % 32 || (c.Hq * c.head_dim) % 32) throw std::invalid_argument("synth: every Q8_0 input width must be a multiple of 32");
    if (c.weight_mix > 2) throw std::invalid_argument("synth: weight_mix must be 0 (Q8_0), 1 (K-quant mix) or 2 (Q8_0 projections with K-quant down and output projections)");
    if (c.weight_mix >= 1 && (c.D % 256 || c.FF % 256 || (c.Hv * c.Dv) % 256 || (c.Hq * c.head_dim) % 256))
        throw std::invalid_argument("synth: K-quant input widths must be multiples of 256");
    if (c.Hkv == 0 || c.Hq % c.Hkv || c.Hk == 0 || c.Hv % c.Hk || c.Dk != c.Dv || c.head_dim % 8) throw std::invalid_argument("synth: inconsistent head shapes");
}

}  // namespace

uint64_t synth_qwen35_size(const SynthConfig& c) {
    check_config(c);
    std::vector<TensorSpec> specs = tensor_specs(c);
    uint64_t data_start = 0, total = 0;
    header_bytes(c, specs, data_start, total);
    return total;
}

void synth_qwen35_image(const SynthConfig& c, uint8_t* image, uint64_t capacity) {
    check_config(c);
    std::vector<TensorSpec> specs = tensor_specs(c);
    uint64_t data_start = 0, total = 0;
    const std::vector<uint8_t> header = header_bytes(c, specs, data_start, total);
    if (capacity < total) throw std::invalid_argument("synth: image buffer too small");
    std::memcpy(image, header.data(), header.size());
    std::memset(image + header.size(), 0, size_t(total - header.size()));
    for (size_t i = 0; i < specs.size(); ++i) fill_tensor(c.seed, specs[i], i, image + data_start + specs[i].offset);
}

namespace {
void write_file(const std::vector<uint8_t>& image, const std::string& path) {
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) throw std::runtime_error("synth: cannot write " + path);
    const size_t wrote = std::fwrite(image.data(), 1, image.size(), f);
    std::fclose(f);
    if (wrote != image.size()) throw std::runtime_error("synth: short write to " + path);
}
}  // namespace

void synth_qwen35_file(const SynthConfig& c, const std::string& path) {
    const uint64_t total = synth_qwen35_size(c);
    std::vector<uint8_t> image(total);
    synth_qwen35_image(c, image.data(), total);
    write_file(image, path);
}

// ---- Gemma 4 (E4B text schema, nm/src/gemma4_loader.hpp:31-52,104-155) ---------
// Fixed choices: 2-D weights N(0, 0.02) in Q8_0; norm weights 1 + N(0, 0.1);
// q_norm 0.125 + N(0, 0.02) (Gemma folds the score scale into it); the final
// norm 8 + N(0, 1), so the logits reach the soft-cap's curved range;
// layer_output_scale 0.8 + N(0, 0.1), a 1-element F32 tensor on every layer.
// Layers from L - shared_kv_layers on carry no attn_k / attn_v.
namespace {

bool gemma_full(uint64_t l) { return l % 6 == 5; }

std::vector<TensorSpec> gemma4_specs(const Gemma4SynthConfig& c) {
    std::vector<TensorSpec> t;
    auto mat = [&](const std::string& name, uint64_t in, uint64_t out) {
        TensorSpec s;
        s.name = name;
        s.in = in;
        s.out = out;
        s.matrix = true;
        s.type = T_Q8_0;
        t.push_back(s);
    };
    auto vec = [&](const std::string& name, uint64_t n, double mean, double scale) {
        TensorSpec s;
        s.name = name;
        s.in = n;
        s.kind = TensorSpec::Affine;
        s.mean = mean;
        s.scale = scale;
        t.push_back(s);
    };
    const uint64_t D = c.D, P = c.ple;
    mat("token_embd.weight", D, c.V);
    mat("per_layer_token_embd.weight", P * c.L, c.V);
    mat("per_layer_model_proj.weight", D, P * c.L);
    vec("per_layer_proj_norm.weight", P, 1.0, 0.1);
    vec("output_norm.weight", D, 8.0, 1.0);
    for (uint64_t l = 0; l < c.L; ++l) {
        const std::string b = "blk." + std::to_string(l) + ".";
        const uint64_t dh = gemma_full(l) ? c.full_dim : c.local_dim;
        const bool shared = l >= c.L - c.shared_kv_layers;
        vec(b + "attn_norm.weight", D, 1.0, 0.1);
        mat(b + "attn_q.weight", D, c.Hq * dh);
        vec(b + "attn_q_norm.weight", dh, 0.125, 0.02);
        if (!shared) {
            mat(b + "attn_k.weight", D, c.Hkv * dh);
            vec(b + "attn_k_norm.weight", dh, 1.0, 0.1);
            mat(b + "attn_v.weight", D, c.Hkv * dh);
        }
        mat(b + "attn_output.weight", c.Hq * dh, D);
        vec(b + "post_attention_norm.weight", D, 1.0, 0.1);
        vec(b + "ffn_norm.weight", D, 1.0, 0.1);
        mat(b + "ffn_gate.weight", D, c.FF);
        mat(b + "ffn_up.weight", D, c.FF);
        mat(b + "ffn_down.weight", c.FF, D);
        vec(b + "post_ffw_norm.weight", D, 1.0, 0.1);
        mat(b + "inp_gate.weight", D, P);
        mat(b + "proj.weight", P, D);
        vec(b + "post_norm.weight", D, 1.0, 0.1);
        vec(b + "layer_output_scale.weight", 1, 0.8, 0.1);
    }
    return t;
}

std::vector<uint8_t> gemma4_header(const Gemma4SynthConfig& c, std::vector<TensorSpec>& specs, uint64_t& data_start, uint64_t& total) {
    return gguf_header(specs, 21, [&](Writer& w) {
        w.kv_str("general.architecture", "gemma4");
        w.kv_u32("general.alignment", 32);
        w.kv_u32("gemma4.block_count", uint32_t(c.L));
        w.kv_u32("gemma4.context_length", uint32_t(c.ctx));
        w.kv_u32("gemma4.embedding_length", uint32_t(c.D));
        w.kv_u32("gemma4.feed_forward_length", uint32_t(c.FF));
        w.kv_u32("gemma4.attention.head_count", uint32_t(c.Hq));
        w.kv_u32("gemma4.attention.head_count_kv", uint32_t(c.Hkv));
        w.kv_u32("gemma4.attention.key_length", uint32_t(c.full_dim));
        w.kv_u32("gemma4.attention.value_length", uint32_t(c.full_dim));
        w.kv_u32("gemma4.attention.key_length_swa", uint32_t(c.local_dim));
        w.kv_u32("gemma4.attention.value_length_swa", uint32_t(c.local_dim));
        w.kv_u32("gemma4.attention.sliding_window", uint32_t(c.window));
        w.kv_u32("gemma4.attention.shared_kv_layers", uint32_t(c.shared_kv_layers));
        w.kv_u32("gemma4.embedding_length_per_layer_input", uint32_t(c.ple));
        w.kv_f32("gemma4.attention.layer_norm_rms_epsilon", 1e-6f);
        w.kv_f32("gemma4.final_logit_softcapping", 30.f);
        w.kv_f32("gemma4.rope.freq_base", 1e6f);
        w.kv_f32("gemma4.rope.freq_base_swa", 1e4f);
        w.kv_u32("gemma4.rope.dimension_count", uint32_t(c.full_dim / 4));
        w.kv_u32("gemma4.rope.dimension_count_swa", uint32_t(c.local_dim));
    }, data_start, total);
}

void check_gemma4(const Gemma4SynthConfig& c) {
    if (c.L < 6 || c.shared_kv_layers >= c.L) throw std::invalid_argument("synth gemma4: need at least 6 layers and fewer shared-KV layers than layers");
    if (c.D % 32 || c.FF % 32 || c.ple % 32 || c.local_dim % 32 || c.full_dim % 32) throw std::invalid_argument("synth gemma4: every Q8_0 input width must be a multiple of 32");
    if (c.Hkv == 0 || c.Hq % c.Hkv || c.V == 0 || c.window == 0 || c.ctx == 0) throw std::invalid_argument("synth gemma4: inconsistent shapes");
}

}  // namespace

uint64_t synth_gemma4_size(const Gemma4SynthConfig& c) {
    check_gemma4(c);
    std::vector<TensorSpec> specs = gemma4_specs(c);
    uint64_t data_start = 0, total = 0;
    gemma4_header(c, specs, data_start, total);
    return total;
}

void synth_gemma4_image(const Gemma4SynthConfig& c, uint8_t* image, uint64_t capacity) {
    check_gemma4(c);
    std::vector<TensorSpec> specs = gemma4_specs(c);
    uint64_t data_start = 0, total = 0;
    const std::vector<uint8_t> header = gemma4_header(c, specs, data_start, total);
    if (capacity < total) throw std::invalid_argument("synth: image buffer too small");
    std::memcpy(image, header.data(), header.size());
    std::memset(image + header.size(), 0, size_t(total - header.size()));
    for (size_t i = 0; i < specs.size(); ++i) fill_tensor(c.seed, specs[i], i, image + data_start + specs[i].offset);
}

void synth_gemma4_file(const Gemma4SynthConfig& c, const std::string& path) {
    const uint64_t total = synth_gemma4_size(c);
    std::vector<uint8_t> image(total);
    synth_gemma4_image(c, image.data(), total);
    write_file(image, path);
}

}  // namespace hero
