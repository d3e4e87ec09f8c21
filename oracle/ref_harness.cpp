// ref_harness.cpp -- drives the REFERENCE engine (flywithfang/hero, nm/src),
// compiled from its own sources where they lie, to write golden vectors.
// TEST INFRASTRUCTURE ONLY: built by oracle/Makefile into oracle/_ref/ (not
// committed); it needs the reference tree at build time only.
//
//   ref_harness kernels DIR          read DIR/*.in.bin, write DIR/*.out.bin
//   ref_harness window DIR           causal / sliding-window attention cases
//   ref_harness model CFG GGUF PROMPT STEPS OUTDIR
//        CFG = tiny | tiny_hk4u | tiny_dh256 | tiny_ff3584 | 8b | gemma4_e4b.
//        Prefill the int32 ids in PROMPT through PrefixCache::evaluate, then
//        STEPS greedy decode passes, exactly as tools/qwen35_check.cpp:43-70
//        and tools/gemma4_text.cpp:16-52 do (minus the tokenizer).
//
// Each kernel case instantiates the reference template at a fixed size and
// applies it to the inputs the golden script wrote.
#include "src/gemma4_loader.hpp"
#include "src/qwen35_loader.hpp"
#include "src/logits.hpp"

#include <limits>
#include <random>

#include <chrono>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

template <class T>
std::vector<T> read_bin(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot read " + path);
    f.seekg(0, std::ios::end);
    const size_t bytes = size_t(f.tellg());
    f.seekg(0);
    std::vector<T> v(bytes / sizeof(T));
    f.read(reinterpret_cast<char*>(v.data()), std::streamsize(bytes));
    return v;
}
template <class T>
void write_bin(const std::string& path, const T* data, size_t n) {
    std::ofstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot write " + path);
    f.write(reinterpret_cast<const char*>(data), std::streamsize(n * sizeof(T)));
}
template <size_t N>
Vec<N> vec_from(const float* p) {
    Vec<N> v;
    for (size_t i = 0; i < N; ++i) v[i] = p[i];
    return v;
}

// ---- model configurations (runtime GGUF dims must equal these) --------------
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
// the tiny shape with 4 key heads tiled over 8 value heads in the delta-net
// (nm/src/qwen35.hpp:164-172) and a separate output.weight (untied head,
// nm/src/qwen35_loader.hpp:132-139)
struct TinyHk4UntiedConfig {
    static constexpr size_t V = 32000, D = 1024, L = 4, CTX = 4096;
    static constexpr size_t Hq = 8, Hkv = 2, HEAD_DIM = 128;
    static constexpr size_t ROPE_BASE = 1000000, ROTARY_NUM = 1, ROTARY_DEN = 4;
    static constexpr size_t KEY_HEAD_DIM = 128, VALUE_HEAD_DIM = 128, KEY_HEADS = 4, VALUE_HEADS = 8, CONV_WIDTH = 4;
    static constexpr size_t FF = 2816;
    static constexpr Scalar RMS_EPS = 1e-6f;
    static constexpr size_t FULL_ATTENTION_INTERVAL = 4;
    using OutputWeight = Weight<D, V>;
    static constexpr bool is_recurrent(size_t layer) { return (layer + 1) % FULL_ATTENTION_INTERVAL != 0; }
};
// the attention geometry of the reference's Qwen 3.5 4B / 9B (nm/src/qwen35.hpp:25-88):
// 256-wide heads (Hq * HEAD_DIM = 2048 != D), a quarter of them rotating, RoPE
// base 1e7, 4 key heads over 8 value heads, untied head -- at tiny width
struct TinyDh256Config {
    static constexpr size_t V = 32000, D = 1024, L = 4, CTX = 4096;
    static constexpr size_t Hq = 8, Hkv = 2, HEAD_DIM = 256;
    static constexpr size_t ROPE_BASE = 10000000, ROTARY_NUM = 1, ROTARY_DEN = 4;
    static constexpr size_t KEY_HEAD_DIM = 128, VALUE_HEAD_DIM = 128, KEY_HEADS = 4, VALUE_HEADS = 8, CONV_WIDTH = 4;
    static constexpr size_t FF = 2816;
    static constexpr Scalar RMS_EPS = 1e-6f;
    static constexpr size_t FULL_ATTENTION_INTERVAL = 4;
    using OutputWeight = Weight<D, V>;
    static constexpr bool is_recurrent(size_t layer) { return (layer + 1) % FULL_ATTENTION_INTERVAL != 0; }
};
// the tiny shape with a SwiGLU width (3584) above every input projection's
// width (3072), the model of the Q8_0-gate/up mix beside K-quant tensors
struct TinyFf3584Config {
    static constexpr size_t V = 32000, D = 1024, L = 4, CTX = 4096;
    static constexpr size_t Hq = 8, Hkv = 2, HEAD_DIM = 128;
    static constexpr size_t ROPE_BASE = 1000000, ROTARY_NUM = 1, ROTARY_DEN = 4;
    static constexpr size_t KEY_HEAD_DIM = 128, VALUE_HEAD_DIM = 128, KEY_HEADS = 8, VALUE_HEADS = 8, CONV_WIDTH = 4;
    static constexpr size_t FF = 3584;
    static constexpr Scalar RMS_EPS = 1e-6f;
    static constexpr size_t FULL_ATTENTION_INTERVAL = 4;
    using OutputWeight = std::monostate;
    static constexpr bool is_recurrent(size_t layer) { return (layer + 1) % FULL_ATTENTION_INTERVAL != 0; }
};
struct Hybrid8BConfig {
    static constexpr size_t V = 151936, D = 4096, L = 32, CTX = 65536;
    static constexpr size_t Hq = 32, Hkv = 8, HEAD_DIM = 128;
    static constexpr size_t ROPE_BASE = 1000000, ROTARY_NUM = 1, ROTARY_DEN = 4;
    static constexpr size_t KEY_HEAD_DIM = 128, VALUE_HEAD_DIM = 128, KEY_HEADS = 32, VALUE_HEADS = 32, CONV_WIDTH = 4;
    static constexpr size_t FF = 12288;
    static constexpr Scalar RMS_EPS = 1e-6f;
    static constexpr size_t FULL_ATTENTION_INTERVAL = 4;
    using OutputWeight = std::monostate;
    static constexpr bool is_recurrent(size_t layer) { return (layer + 1) % FULL_ATTENTION_INTERVAL != 0; }
};

template <class Model>
int run_loaded(const Model& model, const char* prompt_path, size_t steps, const std::string& out) {
    constexpr size_t D = Model::D, V = Model::V;
    const std::vector<int32_t> prompt_ids = read_bin<int32_t>(prompt_path);
    std::vector<TokenId> tokens;
    for (int32_t id : prompt_ids) tokens.push_back(TokenId{id});

    EmbeddedSequence<D> sequence;
    sequence.append(model.embed(tokens), tokens);
    PrefixCache<Model> memo(model);
    const auto t0 = std::chrono::steady_clock::now();
    Logits<V> logits = memo.evaluate(sequence);
    const auto t1 = std::chrono::steady_clock::now();
    write_bin(out + "/logits_prefill.f32", &logits[0], V);

    // per step: the greedy id, and the top-5 (ids, logits)
    std::vector<int32_t> ids, top_ids;
    std::vector<float> top_logits;
    for (size_t i = 0;; ++i) {
        const TokenId token = logits.argmax();
        ids.push_back(int32_t(token));
        for (const ScoredToken& s : logits.top(5)) {
            top_ids.push_back(int32_t(s.id));
            top_logits.push_back(s.logit);
        }
        if (i == steps) break;
        const std::span<const TokenId> next(&token, 1);
        sequence.append(model.embed(next), next);
        logits = memo.evaluate(sequence);
        if (i + 1 == steps / 2) write_bin(out + "/logits_mid.f32", &logits[0], V);
    }
    const auto t2 = std::chrono::steady_clock::now();
    write_bin(out + "/logits_last.f32", &logits[0], V);
    write_bin(out + "/ids.i32", ids.data(), ids.size());
    write_bin(out + "/top5_ids.i32", top_ids.data(), top_ids.size());
    write_bin(out + "/top5_logits.f32", top_logits.data(), top_logits.size());
    const double prefill = std::chrono::duration<double>(t1 - t0).count();
    const double decode = std::chrono::duration<double>(t2 - t1).count();
    std::FILE* f = std::fopen((out + "/times.txt").c_str(), "w");
    std::fprintf(f, "threads %zu\nprefill_seconds %.6f\nprompt_tokens %zu\ndecode_seconds %.6f\ndecode_passes %zu\n", nm_num_threads(), prefill, prompt_ids.size(), decode, steps);
    std::fclose(f);
    std::printf("reference %s: prefill %zu tokens %.3fs, %zu decode passes %.3fs (%.3f passes/s, %zu threads)\n", out.c_str(), prompt_ids.size(), prefill, steps, decode, steps / decode, nm_num_threads());
    return 0;
}

template <class C>
int run_model(const char* gguf_path, const char* prompt_path, size_t steps, const std::string& out) {
    const GGUF gguf(gguf_path);
    const auto model = qwen35_loader::load<C>(gguf);
    return run_loaded(model, prompt_path, steps, out);
}

// Gemma 4 E4B text (its classes are fixed to the E4B configuration): the
// loop of tools/gemma4_text.cpp:16-52 minus the tokenizer
int run_gemma4(const char* gguf_path, const char* prompt_path, size_t steps, const std::string& out) {
    const GGUF gguf(gguf_path);
    const Gemma4E4BModel model = gemma4_loader::load_e4b_text(gguf);
    return run_loaded(model, prompt_path, steps, out);
}

// ---- kernel-level golden vectors ------------------------------------------------
int run_kernels(const std::string& dir) {
    auto in = [&](const char* name) { return read_bin<float>(dir + "/" + name + ".in.bin"); };
    auto out = [&](const char* name, const std::vector<float>& v) { write_bin(dir + "/" + name + ".out.bin", v.data(), v.size()); };

    {  // fp16 encoder over arbitrary fp32 bit patterns
        const std::vector<float> x = in("fp16_encode");
        std::vector<uint16_t> h(x.size());
        for (size_t i = 0; i < x.size(); ++i) h[i] = fp32_to_fp16(x[i]);
        write_bin(dir + "/fp16_encode.out.bin", h.data(), h.size());
    }
    {  // activation quantizer (roundf) and weight quantizer (lround), K = 4096
        const std::vector<float> x = in("quant");
        std::vector<block_q8_0> a(x.size() / 32), w(x.size() / 32);
        quantize_row_q8_0(x.data(), a.data(), x.size());
        quantize_q8_0(x.data(), w.data(), x.size());
        write_bin(dir + "/quant_act.out.bin", a.data(), a.size());
        write_bin(dir + "/quant_weight.out.bin", w.data(), w.size());
    }
    {  // Weight<4096,64>::matvec and ::matmul over 8 rows (int8-activation path)
        const std::vector<float> wf = in("gemv_w");  // [64][4096] fp32, quantized here
        const std::vector<float> x = in("gemv_x");   // [8][4096]
        constexpr size_t K = 4096, N = 64;
        auto blocks = std::make_shared<std::vector<block_q8_0>>(N * K / 32);
        quantize_q8_0(wf.data(), blocks->data(), N * K);
        write_bin(dir + "/gemv_wq.out.bin", blocks->data(), blocks->size());
        const Weight<K, N> weight(GT::Q8_0, blocks->data(), blocks);
        const Vec<N> y = weight.matvec(vec_from<K>(x.data()));
        out("gemv_y", std::vector<float>(y.p.get(), y.p.get() + N));
        Matrix<K> X;
        for (size_t r = 0; r < 8; ++r) X.append(vec_from<K>(x.data() + r * K));
        const Matrix<N> Y = weight.matmul(X.view());
        std::vector<float> yy;
        for (size_t r = 0; r < 8; ++r)
            for (size_t n = 0; n < N; ++n) yy.push_back(Y.row(r)[n]);
        out("gemm_y", yy);
    }
    {  // K-quants: Q8_K activation quantizer and Weight<4096,64>::matvec /
       // ::matmul over raw Q4_K and Q6_K blocks (int8-activation, x86 scalar dots)
        const std::vector<float> x = in("kq_x");  // [4][4096]
        constexpr size_t K = 4096, N = 64, T = 4;
        std::vector<block_q8_K> act(T * K / QK_K);
        for (size_t r = 0; r < T; ++r) quantize_row_q8_K(x.data() + r * K, act.data() + r * K / QK_K, K);
        write_bin(dir + "/kq_act.out.bin", act.data(), act.size());
        auto run = [&](const char* wname, GT type, const char* yname) {
            auto raw = std::make_shared<std::vector<uint8_t>>(read_bin<uint8_t>(dir + "/" + wname + ".in.bin"));
            if (raw->size() != type_size_bytes(type, N * K)) throw std::runtime_error(std::string("bad size for ") + wname);
            const Weight<K, N> weight(type, raw->data(), raw);
            std::vector<float> yy;
            const Vec<N> y = weight.matvec(vec_from<K>(x.data()));
            yy.insert(yy.end(), y.p.get(), y.p.get() + N);
            Matrix<K> X;
            for (size_t r = 0; r < T; ++r) X.append(vec_from<K>(x.data() + r * K));
            const Matrix<N> Y = weight.matmul(X.view());
            for (size_t r = 0; r < T; ++r)
                for (size_t n = 0; n < N; ++n) yy.push_back(Y.row(r)[n]);
            out(yname, yy);
        };
        run("kq_w4", GT::Q4_K, "kq_y4");
        run("kq_w6", GT::Q6_K, "kq_y6");
        // Q5_K: no integer-activation kernel, so matvec / matmul take the
        // fp32-activation dequant-in-dot form
        run("kq_w5", GT::Q5_K, "kq_y5");
        // Weight::dequant_row (the embedding gather) of rows 0 and 37
        auto dequant = [&](const char* wname, GT type, const char* yname) {
            auto raw = std::make_shared<std::vector<uint8_t>>(read_bin<uint8_t>(dir + "/" + wname + ".in.bin"));
            const Weight<K, N> weight(type, raw->data(), raw);
            std::vector<float> yy;
            for (size_t row : {size_t(0), size_t(37)}) {
                const Vec<K> r = weight.dequant_row(row);
                yy.insert(yy.end(), r.p.get(), r.p.get() + K);
            }
            out(yname, yy);
        };
        dequant("kq_w4", GT::Q4_K, "kq_dq4");
        dequant("kq_w5", GT::Q5_K, "kq_dq5");
        dequant("kq_w6", GT::Q6_K, "kq_dq6");
    }
    {  // Logits<32000>::sample over 8 logit rows x 6 configurations; the
       // uniform draw it makes is recorded from a copy of the generator
        const std::vector<float> lg = in("sample_logits");  // [8][32000]
        constexpr size_t V = 32000;
        const SamplerCfg cfgs[6] = {{0.7f, 40, 0.9f, 1}, {1.0f, 1, 1.0f, 2}, {1.3f, 1000, 0.95f, 3}, {0.5f, 0, 1.0f, 4}, {2.0f, 200, 0.5f, 5}, {0.9f, 64, 0.0f, 6}};
        std::vector<float> res;  // per (row, cfg): token, u
        for (size_t r = 0; r < 8; ++r) {
            Vec<V> v;
            for (size_t i = 0; i < V; ++i) v[i] = lg[r * V + i];
            const Logits<V> logits(std::move(v));
            for (const SamplerCfg& c : cfgs) {
                std::mt19937_64 rng(c.seed * 1000 + r);
                std::mt19937_64 copy = rng;
                const float u = std::generate_canonical<float, std::numeric_limits<float>::digits>(copy);
                const TokenId t = logits.sample(c, rng);
                res.push_back(float(int32_t(t)));
                res.push_back(u);
            }
        }
        out("sample", res);
    }
    {  // RMSNorm at the three widths the path uses; gamma is [width] after x
        auto norm = [&]<size_t N>(const char* name, std::integral_constant<size_t, N>) {
            const std::vector<float> v = in(name);  // [x | gamma]
            const RMSNorm<N> rn(vec_from<N>(v.data() + N), 1e-6f);
            const Vec<N> y = rn(vec_from<N>(v.data()));
            out(name, std::vector<float>(y.p.get(), y.p.get() + N));
        };
        norm("rms128", std::integral_constant<size_t, 128>{});
        norm("rms1024", std::integral_constant<size_t, 1024>{});
        norm("rms4096", std::integral_constant<size_t, 4096>{});
    }
    {  // l2 normalize over 16 heads of 128
        const std::vector<float> x = in("l2");
        std::vector<float> y;
        for (size_t h = 0; h < x.size() / 128; ++h) {
            const Vec<128> r = l2_normalize<128>(vec_from<128>(x.data() + h * 128));
            y.insert(y.end(), r.p.get(), r.p.get() + 128);
        }
        out("l2", y);
    }
    {  // scalar activations
        const std::vector<float> x = in("act");
        std::vector<float> s(x.size()), g(x.size()), p(x.size());
        for (size_t i = 0; i < x.size(); ++i) {
            Vec<1> v;
            v[0] = x[i];
            v = Silu{}(std::move(v));
            s[i] = v[0];
            g[i] = sigmoid(x[i]);
            p[i] = softplus(x[i]);
        }
        out("silu", s);
        out("sigmoid", g);
        out("softplus", p);
    }
    {  // causal conv, 256 channels, width 4, 6 steps
        const std::vector<float> taps = in("conv_taps");  // [256][4]
        const std::vector<float> xs = in("conv_x");       // [6][256]
        Matrix<4> w;
        for (size_t c = 0; c < 256; ++c) w.append(vec_from<4>(taps.data() + c * 4));
        CausalConv1dState<256, 4> conv;
        std::vector<float> y;
        for (size_t t = 0; t < 6; ++t) {
            const Vec<256> r = conv.step(vec_from<256>(xs.data() + t * 256), w);
            y.insert(y.end(), r.p.get(), r.p.get() + 256);
        }
        out("conv", y);
    }
    {  // gated delta rule, one head 128x128, 4 consecutive tokens
        std::vector<float> state = in("delta_state");  // [128*128]
        const std::vector<float> tok = in("delta_tok");  // 4 x [q 128 | k 128 | v 128 | gate | beta]
        std::vector<float> y;
        const size_t stride = 3 * 128 + 2;
        for (size_t t = 0; t < 4; ++t) {
            const float* p = tok.data() + t * stride;
            const Vec<128> o = gated_delta_step<128, 128>(state.data(), vec_from<128>(p), vec_from<128>(p + 128), vec_from<128>(p + 256), p[384], p[385]);
            y.insert(y.end(), o.p.get(), o.p.get() + 128);
        }
        out("delta_out", y);
        out("delta_state", state);
    }
    {  // RoPE, head 128, base 1e6, rotary 1/4, at several positions
        const std::vector<float> x = in("rope");  // [P][128]
        static const size_t positions[] = {0, 1, 2, 7, 100, 1023, 4095, 65535};
        const RotaryEmbedding<128, 1000000, 1, 4> rope;
        std::vector<float> y;
        for (size_t i = 0; i < 8; ++i) {
            Vec<128> v = vec_from<128>(x.data() + i * 128);
            rope(slice_mut<128>(v, 0), Position{positions[i]});
            y.insert(y.end(), v.p.get(), v.p.get() + 128);
        }
        out("rope", y);
    }
    {  // attention reduction: one query over ctx keys (the decode case), at
       // scale 1/sqrt(128) and at scale 1; scaled_dot_product_attention is
       // the same dot / Softmax / scaled_add reduction as qwen35.hpp:366-380
        const std::vector<float> q = in("attn_q");  // [128]
        const std::vector<float> k = in("attn_k");  // [ctx][128]
        const std::vector<float> v = in("attn_v");  // [ctx][128]
        const size_t ctx = k.size() / 128;
        Matrix<128> Q, K, V;
        Q.append(vec_from<128>(q.data()));
        for (size_t j = 0; j < ctx; ++j) {
            K.append(vec_from<128>(k.data() + j * 128));
            V.append(vec_from<128>(v.data() + j * 128));
        }
        for (const float scale : {1.f / std::sqrt(128.f), 1.f}) {
            const Matrix<128> A = scaled_dot_product_attention<1, 128, 128>(Q.view(), K.view(), V.view(), scale);
            out(scale == 1.f ? "attn_unit" : "attn_scaled", std::vector<float>(A.row(0).begin(), A.row(0).end()));
        }
    }
    std::printf("kernel golden vectors written to %s\n", dir.c_str());
    return 0;
}

// ---- causal and sliding-window attention over the reference's own caches ------
// Keys and values of `ctx` consecutive positions are appended one at a time to
// a FullAttentionCache (width 0) or a LocalAttentionCache ring (widths 3 and
// 1024, evicting); at each probe position the query of that position attends
// over cache.visible_rows(), the reduction of nm/src/gemma4.hpp:586-606
// (score = scale * dot, Softmax, sum of alpha * value, K/V head = head / group).
// Four query heads over two K/V heads of 128.
int run_window(const std::string& dir) {
    constexpr size_t Hq = 4, Hkv = 2, Dh = 128, KW = Hkv * Dh, QW = Hq * Dh;
    const std::vector<float> k = read_bin<float>(dir + "/window_k.in.bin");  // [ctx][KW]
    const std::vector<float> v = read_bin<float>(dir + "/window_v.in.bin");  // [ctx][KW]
    const std::vector<float> q = read_bin<float>(dir + "/window_q.in.bin");  // [ctx][QW]
    const std::vector<float> probes_f = read_bin<float>(dir + "/window_probes.in.bin");
    const size_t ctx = k.size() / KW;
    std::vector<size_t> probes;
    for (float p : probes_f) probes.push_back(size_t(p));
    Matrix<KW> K, V;
    Matrix<QW> Q;
    for (size_t t = 0; t < ctx; ++t) {
        K.append(vec_from<KW>(k.data() + t * KW));
        V.append(vec_from<KW>(v.data() + t * KW));
        Q.append(vec_from<QW>(q.data() + t * QW));
    }
    auto attend = [&](auto& cache, size_t t, float scale, std::vector<float>& outv) {
        const VisibleRows rows = cache.visible_rows(Position{t});
        for (size_t head = 0; head < Hq; ++head) {
            const VecView<Dh> query = slice<Dh>(Q.row(t), head);
            const KVHead group{head / (Hq / Hkv)};
            std::vector<Scalar> alpha;
            for (size_t j = rows.first; j < rows.end; ++j) alpha.push_back(scale * dot(query, cache.key(j, group)));
            alpha = Softmax{}(std::move(alpha));
            Vec<Dh> o;
            for (size_t n = 0; n < alpha.size(); ++n) o.scaled_add(cache.value(rows.first + n, group), alpha[n]);
            outv.insert(outv.end(), o.p.get(), o.p.get() + Dh);
        }
        outv.push_back(float(rows.first));
        outv.push_back(float(rows.end));
    };
    auto run = [&](auto& cache, float scale, const char* name) {
        std::vector<float> outv;
        size_t next = 0;
        for (size_t t = 0; t < ctx; ++t) {
            cache.append(Position{t}, K.row(t), V.row(t));
            if (next < probes.size() && probes[next] == t) {
                attend(cache, t, scale, outv);
                ++next;
            }
        }
        write_bin(dir + "/" + name + ".out.bin", outv.data(), outv.size());
    };
    {
        FullAttentionCache<Hkv, Dh> cache;
        run(cache, 1.f / std::sqrt(128.f), "window_full");
    }
    {
        LocalAttentionCache<Hkv, Dh> cache(3);
        run(cache, 1.f, "window_w3");
    }
    {
        LocalAttentionCache<Hkv, Dh> cache(1024);
        run(cache, 1.f, "window_w1024");
    }
    std::printf("window golden vectors written to %s\n", dir.c_str());
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        if (argc == 3 && std::strcmp(argv[1], "kernels") == 0) return run_kernels(argv[2]);
        if (argc == 3 && std::strcmp(argv[1], "window") == 0) return run_window(argv[2]);
        if (argc == 7 && std::strcmp(argv[1], "model") == 0) {
            const size_t steps = std::strtoull(argv[5], nullptr, 10);
            if (std::strcmp(argv[2], "tiny") == 0) return run_model<TinyConfig>(argv[3], argv[4], steps, argv[6]);
            if (std::strcmp(argv[2], "tiny_hk4u") == 0) return run_model<TinyHk4UntiedConfig>(argv[3], argv[4], steps, argv[6]);
            if (std::strcmp(argv[2], "tiny_dh256") == 0) return run_model<TinyDh256Config>(argv[3], argv[4], steps, argv[6]);
            if (std::strcmp(argv[2], "tiny_ff3584") == 0) return run_model<TinyFf3584Config>(argv[3], argv[4], steps, argv[6]);
            if (std::strcmp(argv[2], "8b") == 0) return run_model<Hybrid8BConfig>(argv[3], argv[4], steps, argv[6]);
            if (std::strcmp(argv[2], "gemma4_e4b") == 0) return run_gemma4(argv[3], argv[4], steps, argv[6]);
        }
        std::fprintf(stderr, "usage: %s kernels DIR | window DIR | model {tiny|tiny_hk4u|tiny_dh256|tiny_ff3584|8b|gemma4_e4b} GGUF PROMPT STEPS OUTDIR\n", argv[0]);
        return 2;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "ref_harness: %s\n", e.what());
        return 1;
    }
}
