// oracle_capi.cpp -- extern "C" surface of the oracle for the Python tests
// and the CPU-baseline leg of bench.py. TEST INFRASTRUCTURE ONLY.
// Every entry returns 0 on success, or -1 with a message in oracle_last_error().
#include "oracle.hpp"
#include "oracle_gguf.hpp"

#include <chrono>
#include <cmath>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>

using namespace oracle;

namespace {
thread_local std::string g_error;

template <class F>
int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return -1;
    }
}

struct Session {
    Gguf gguf;
    Model model;
    State state;
};
struct Gemma4Session {
    Gguf gguf;
    Gemma4Model model;
    Gemma4State state;
};
}  // namespace

extern "C" {

const char* oracle_last_error() { return g_error.c_str(); }
void oracle_set_threads(size_t n) { set_threads(n); }
size_t oracle_threads() { return num_threads(); }

void oracle_fp16_to_fp32(const uint16_t* h, float* f, size_t n) {
    for (size_t i = 0; i < n; ++i) f[i] = fp16_to_fp32(h[i]);
}
void oracle_fp32_to_fp16(const float* f, uint16_t* h, size_t n) {
    for (size_t i = 0; i < n; ++i) h[i] = fp32_to_fp16(f[i]);
}
void oracle_quantize_row_q8_0(const float* x, void* blocks, size_t k) { quantize_row_q8_0(x, static_cast<BlockQ8*>(blocks), k); }
void oracle_quantize_q8_0(const float* x, void* blocks, size_t k) { quantize_q8_0(x, static_cast<BlockQ8*>(blocks), k); }
float oracle_vec_dot_q8_0(size_t k, const void* w, const void* x) { return vec_dot_q8_0_q8_0(k, static_cast<const BlockQ8*>(w), static_cast<const BlockQ8*>(x)); }

// int32 block sums (the bit-exact part of the dot): out[n*(K/32)+b]
void oracle_block_sums_q8_0(const void* W, size_t N, size_t K, const void* xq, int32_t* out) {
    const BlockQ8* w = static_cast<const BlockQ8*>(W);
    const BlockQ8* x = static_cast<const BlockQ8*>(xq);
    const size_t nb = K / 32;
    for (size_t n = 0; n < N; ++n)
        for (size_t b = 0; b < nb; ++b) {
            int s = 0;
            for (size_t j = 0; j < 32; ++j) s += int(w[n * nb + b].qs[j]) * int(x[b].qs[j]);
            out[n * nb + b] = s;
        }
}

int32_t oracle_sample_topk(const float* logits, size_t V, size_t top_k, float temp, float top_p, float u) { return sample_topk(logits, V, top_k, temp, top_p, u); }
void oracle_quantize_row_q8_K(const float* x, void* blocks, size_t k) { quantize_row_q8_K(x, static_cast<BlockQ8K*>(blocks), k); }
float oracle_vec_dot_kquant(int type, const void* w, const void* x, size_t k) {
    return type == 12 ? vec_dot_q4_K_q8_K(k, static_cast<const BlockQ4K*>(w), static_cast<const BlockQ8K*>(x))
                      : vec_dot_q6_K_q8_K(k, static_cast<const BlockQ6K*>(w), static_cast<const BlockQ8K*>(x));
}
void oracle_matmul_kquant(int type, const void* W, size_t N, size_t K, const float* X, size_t T, float* Y) { matmul_kquant(type, W, N, K, X, T, Y); }
float oracle_dot_block_q5_K(const void* block, const float* x) { return dot_block_q5_K(*static_cast<const BlockQ5K*>(block), x); }
// any linear weight type (8, 12, 13, 14): the Weight::matmul the model calls
int oracle_linear_rows(int type, const void* W, size_t N, size_t K, const float* X, size_t T, float* Y) {
    try {
        linear_rows(Linear{W, type, N, K}, X, T, Y);
        return 0;
    } catch (...) {
        return 1;
    }
}
// `rows` rows of a tensor of `type`, k elements each, dequantized to fp32
int oracle_dequant_rows(int type, const void* W, size_t rows, size_t k, float* out) {
    try {
        const size_t rb = row_bytes(type, k);
        for (size_t r = 0; r < rows; ++r) dequant_row(type, static_cast<const uint8_t*>(W) + r * rb, out + r * k, k);
        return 0;
    } catch (...) {
        return 1;
    }
}
void oracle_matvec_q8_0(const void* W, size_t N, size_t K, const float* x, float* y) { matvec_q8_0(static_cast<const BlockQ8*>(W), N, K, x, y); }
void oracle_matmul_q8_0(const void* W, size_t N, size_t K, const float* X, size_t T, float* Y) { matmul_q8_0(static_cast<const BlockQ8*>(W), N, K, X, T, Y); }

void oracle_rmsnorm_rows(float* x, const float* gamma, size_t rows, size_t n, float eps) {
    for (size_t r = 0; r < rows; ++r) rmsnorm(x + r * n, gamma, n, eps);
}
void oracle_l2_normalize(const float* x, float* out, size_t n, float eps) { l2_normalize(x, out, n, eps); }
void oracle_silu(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = silu(x[i]);
}
void oracle_sigmoid(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = sigmoid(x[i]);
}
void oracle_softplus(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = softplus(x[i]);
}
void oracle_softmax(float* v, size_t n) { softmax(v, n); }
// glibc's expf and log1pf as the reference calls them (std::exp / std::log1p on float)
void oracle_expf(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = std::exp(x[i]);
}
void oracle_log1pf(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = std::log1p(x[i]);
}
void oracle_conv_step(const float* input, const float* taps, float* history, float* out, size_t channels, size_t width) { conv_step(input, taps, history, out, channels, width); }

// H heads of one token; head h reads key head h % Hk (qwen35.hpp:172)
void oracle_gated_delta_step(float* state, const float* q, const float* k, const float* v, const float* gate, const float* beta, float* out, size_t heads, size_t key_heads, size_t dk, size_t dv) {
    for (size_t h = 0; h < heads; ++h) {
        const size_t hk = h % key_heads;
        gated_delta_step(state + h * dk * dv, q + hk * dk, k + hk * dk, v + h * dv, gate[h], beta[h], out + h * dv, dk, dv);
    }
}

void oracle_rope_inv_freq(size_t head_dim, double base, size_t rotary_dims, float* out) {
    const std::vector<float> t = rope_inv_freq(head_dim, base, rotary_dims);
    std::memcpy(out, t.data(), t.size() * sizeof(float));
}
void oracle_rope_apply(float* heads, size_t n_heads, const float* inv_freq, size_t head_dim, size_t position) {
    for (size_t h = 0; h < n_heads; ++h) rope_apply(heads + h * head_dim, inv_freq, head_dim, position);
}

// cos/sin per (position, plane) with the reference's float expressions
// (attention.hpp:84-85): angle = float(pos) * inv_freq[i]. out [positions][planes][2]
void oracle_rope_table(size_t head_dim, double base, size_t rotary_dims, size_t positions, float* out) {
    const std::vector<float> inv = rope_inv_freq(head_dim, base, rotary_dims);
    const size_t planes = head_dim / 2;
    for (size_t p = 0; p < positions; ++p)
        for (size_t i = 0; i < planes; ++i) {
            const float angle = float(p) * inv[i];
            out[(p * planes + i) * 2] = std::cos(angle);
            out[(p * planes + i) * 2 + 1] = std::sin(angle);
        }
}

// GQA decode over a [ctx][Hkv*Dh] fp32 cache: q [Hq][Dh] -> out [Hq][Dh].
// window == 0 is full causal; otherwise keys with q_pos - k_pos < window.
int oracle_attend_decode(const float* q, const float* keys, const float* values, size_t ctx, size_t hq, size_t hkv, size_t head_dim, size_t window, float scale, float* out) {
    return guarded([&] {
        const size_t group = hq / hkv;
        const size_t first = (window == 0 || ctx <= window) ? 0 : ctx - window;
        for (size_t h = 0; h < hq; ++h) attend_one(q + h * head_dim, keys, values, hkv * head_dim, h / group, head_dim, first, ctx, scale, out + h * head_dim);
    });
}

// ---- whole model -------------------------------------------------------------
void* oracle_model_open(const char* path) {
    try {
        auto s = std::make_unique<Session>();
        s->gguf.open(path);
        s->model = load_qwen35(s->gguf);
        s->state.reset(s->model.c);
        return s.release();
    } catch (const std::exception& e) {
        g_error = e.what();
        return nullptr;
    }
}
// A GGUF image already in memory (owned by the caller for the session's life).
void* oracle_model_open_image(const void* base, size_t size) {
    try {
        auto s = std::make_unique<Session>();
        s->gguf.parse(static_cast<const uint8_t*>(base), size);
        s->model = load_qwen35(s->gguf);
        s->state.reset(s->model.c);
        return s.release();
    } catch (const std::exception& e) {
        g_error = e.what();
        return nullptr;
    }
}
void oracle_model_close(void* h) { delete static_cast<Session*>(h); }

// dims: V D L CTX Hq Hkv head_dim rotary_dims Dk Dv Hk Hv conv_width FF tied
void oracle_model_dims(void* h, size_t* out) {
    const Config& c = static_cast<Session*>(h)->model.c;
    const size_t v[] = {c.V, c.D, c.L, c.CTX, c.Hq, c.Hkv, c.head_dim, c.rotary_dims, c.Dk, c.Dv, c.Hk, c.Hv, c.conv_width, c.FF, size_t(c.tied)};
    std::memcpy(out, v, sizeof(v));
}
void oracle_model_reset(void* h) {
    Session* s = static_cast<Session*>(h);
    s->state.reset(s->model.c);
}
void oracle_model_set_kv_fp16(void* h, int on) { static_cast<Session*>(h)->state.kv_fp16 = on != 0; }
void oracle_model_set_kv_q8(void* h, int on) { static_cast<Session*>(h)->state.kv_q8 = on != 0; }
void oracle_round_fp16(const float* x, size_t n, float* out) {
    for (size_t i = 0; i < n; ++i) out[i] = round_fp16_rne(x[i]);
}
size_t oracle_model_tokens(void* h) { return static_cast<Session*>(h)->state.tokens; }
int oracle_model_embed(void* h, const int32_t* ids, size_t n, float* out) {
    return guarded([&] { embed(static_cast<Session*>(h)->model, ids, n, out); });
}
int oracle_model_forward(void* h, const float* rows, size_t T, float* logits) {
    return guarded([&] {
        Session* s = static_cast<Session*>(h);
        forward(s->model, s->state, rows, T, logits);
    });
}
// ids -> embed -> forward, the common case
int oracle_model_forward_ids(void* h, const int32_t* ids, size_t T, float* logits) {
    return guarded([&] {
        Session* s = static_cast<Session*>(h);
        std::vector<float> rows(T * s->model.c.D);
        embed(s->model, ids, T, rows.data());
        forward(s->model, s->state, rows.data(), T, logits);
    });
}
int32_t oracle_argmax(const float* logits, size_t n) { return argmax(logits, n); }

// Greedy loop (tools/qwen35_check.cpp:54-70 pattern): prefill `prompt`, then
// `steps` decode passes. out_ids receives steps+1 greedy ids (the first from
// the prefill logits). Times are wall seconds for prefill and for the decode
// passes; decode tok/s = steps / decode_seconds (passes over time).
int oracle_model_greedy(void* h, const int32_t* prompt, size_t n_prompt, size_t steps, int32_t* out_ids, float* last_logits, double* prefill_seconds, double* decode_seconds) {
    return guarded([&] {
        Session* s = static_cast<Session*>(h);
        const size_t V = s->model.c.V;
        std::vector<float> logits(V);
        const auto t0 = std::chrono::steady_clock::now();
        std::vector<float> rows(n_prompt * s->model.c.D);
        embed(s->model, prompt, n_prompt, rows.data());
        forward(s->model, s->state, rows.data(), n_prompt, logits.data());
        const auto t1 = std::chrono::steady_clock::now();
        int32_t next = argmax(logits.data(), V);
        out_ids[0] = next;
        std::vector<float> row(s->model.c.D);
        for (size_t i = 0; i < steps; ++i) {
            embed(s->model, &next, 1, row.data());
            forward(s->model, s->state, row.data(), 1, logits.data());
            next = argmax(logits.data(), V);
            out_ids[i + 1] = next;
        }
        const auto t2 = std::chrono::steady_clock::now();
        if (last_logits) std::memcpy(last_logits, logits.data(), V * sizeof(float));
        if (prefill_seconds) *prefill_seconds = std::chrono::duration<double>(t1 - t0).count();
        if (decode_seconds) *decode_seconds = std::chrono::duration<double>(t2 - t1).count();
    });
}

// ---- Gemma 4 (oracle_gemma4.cpp) ----
void* oracle_gemma4_open(const char* path) {
    Gemma4Session* out = nullptr;
    guarded([&] {
        auto sess = std::make_unique<Gemma4Session>();
        sess->gguf.open(path);
        sess->model = load_gemma4(sess->gguf);
        sess->state.reset(sess->model.c);
        out = sess.release();
    });
    return out;
}
void* oracle_gemma4_open_image(const void* image, size_t size) {
    Gemma4Session* out = nullptr;
    guarded([&] {
        auto sess = std::make_unique<Gemma4Session>();
        sess->gguf.parse(static_cast<const uint8_t*>(image), size);
        sess->model = load_gemma4(sess->gguf);
        sess->state.reset(sess->model.c);
        out = sess.release();
    });
    return out;
}
void oracle_gemma4_close(void* h) { delete static_cast<Gemma4Session*>(h); }
// V, D, L, window, shared, P
void oracle_gemma4_dims(void* h, size_t* out) {
    const Gemma4Config& c = static_cast<Gemma4Session*>(h)->model.c;
    out[0] = c.V, out[1] = c.D, out[2] = c.L, out[3] = c.window, out[4] = c.shared, out[5] = c.P;
}
void oracle_gemma4_reset(void* h) {
    Gemma4Session* s = static_cast<Gemma4Session*>(h);
    s->state.reset(s->model.c);
}
size_t oracle_gemma4_tokens(void* h) { return static_cast<Gemma4Session*>(h)->state.tokens; }
size_t oracle_gemma4_kv_source(void* h, size_t layer) { return static_cast<Gemma4Session*>(h)->model.c.kv_source(layer); }
int oracle_gemma4_embed(void* h, const int32_t* ids, size_t n, float* out) {
    return guarded([&] { gemma4_embed(static_cast<Gemma4Session*>(h)->model, ids, n, out); });
}
int oracle_gemma4_forward(void* h, const int32_t* ids, size_t T, float* logits) {
    Gemma4Session* s = static_cast<Gemma4Session*>(h);
    return guarded([&] { gemma4_forward(s->model, s->state, ids, T, logits); });
}
void oracle_gemma_math(const float* x, float* out, size_t n, float cap) {
    for (size_t i = 0; i < n; ++i) {
        out[2 * i] = gelu_tanh(x[i]);
        out[2 * i + 1] = gemma_softcap(x[i], cap);
    }
}

}  // extern "C"
