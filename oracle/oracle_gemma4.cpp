// oracle_gemma4.cpp -- CPU restatement of the reference's Gemma 4 E4B text
// model (nm/src/gemma4.hpp) and its loader (nm/src/gemma4_loader.hpp).
// TEST INFRASTRUCTURE ONLY (see oracle.hpp). Same fp32 operation order as the
// reference; every Linear goes through the oracle's Weight::matmul
// restatement (linear_rows), so T rows give the same per-row results as T
// single-row passes.
#include "oracle.hpp"
#include "oracle_gguf.hpp"

#include <cmath>
#include <stdexcept>
#include <string>

namespace oracle {

// gemma4.hpp:41-47 and Gemma4E4BCache::local / full (:370-373): a layer that
// reuses K/V reads the last earlier owning layer of its attention kind
size_t Gemma4Config::kv_source(size_t l) const {
    if (!shares_kv(l)) return l;
    for (size_t s = L - shared; s-- > 0;)
        if (full(s) == full(l)) return s;
    throw std::invalid_argument("gemma4: a layer that reuses K/V has no earlier layer of its kind");
}

void Gemma4State::reset(const Gemma4Config& c) {
    tokens = 0;
    keys.assign(c.L, {});
    values.assign(c.L, {});
}

// components.hpp:73-81
float gelu_tanh(float v) { return 0.5f * v * (1.f + std::tanh(0.7978845608f * (v + 0.044715f * v * v * v))); }
// gemma4.hpp:79
float gemma_softcap(float v, float cap) { return cap * std::tanh(v / cap); }

void gemma4_embed(const Gemma4Model& m, const int32_t* ids, size_t n, float* out) {
    const size_t D = m.c.D;
    const float scale = std::sqrt(float(D));  // gemma4.hpp:417
    for (size_t i = 0; i < n; ++i) {
        if (ids[i] < 0 || size_t(ids[i]) >= m.c.V) throw std::out_of_range("gemma4 embed: token id out of range");
        dequant_row(m.embedding.type, static_cast<const uint8_t*>(m.embedding.w) + size_t(ids[i]) * row_bytes(m.embedding.type, D), out + i * D, D);
        for (size_t j = 0; j < D; ++j) out[i * D + j] *= scale;
    }
}

namespace {

std::vector<float> rows_through(const Linear& lin, const float* X, size_t T) {
    std::vector<float> Y(T * lin.N);
    linear_rows(lin, X, T, Y.data());
    return Y;
}

// RMSNorm (components.hpp:176-181) of each of T rows of n
std::vector<float> normed(const float* X, size_t T, size_t n, const std::vector<float>& gamma, float eps) {
    std::vector<float> Y(X, X + T * n);
    for (size_t t = 0; t < T; ++t) rmsnorm(Y.data() + t * n, gamma.data(), n, eps);
    return Y;
}

// RMSNormNoScale (components.hpp:210-215)
void rmsnorm_noscale(float* x, size_t n, float eps) {
    const float inv = 1.f / std::sqrt(dot(x, x, n) / float(n) + eps);
    for (size_t c = 0; c < n; ++c) x[c] *= inv;
}

// GemmaE4BLayer / GemmaE4BSharedLayer::attention (gemma4.hpp:203-255, 300-324):
// Q = rope(q_norm(WQ x)); an owning layer appends K = rope(k_norm(WK x)) and
// V = v_norm(WV x) for all T rows, then every row attends over the rows its
// window leaves visible, score scale 1
std::vector<float> gemma_attention(const Gemma4Model& m, size_t l, Gemma4State& s, const float* U, size_t T) {
    const Gemma4Config& c = m.c;
    const Gemma4Layer& L = m.layers[l];
    const size_t dh = c.head_dim(l), QW = c.Hq * dh, KW = c.Hkv * dh;
    const std::vector<float>& inv = c.full(l) ? m.inv_full : m.inv_local;
    std::vector<float> Q = rows_through(L.wq, U, T);
    for (size_t t = 0; t < T; ++t)
        for (size_t h = 0; h < c.Hq; ++h) {
            rmsnorm(Q.data() + t * QW + h * dh, L.q_norm.data(), dh, c.eps);
            rope_apply(Q.data() + t * QW + h * dh, inv.data(), dh, s.tokens + t);
        }
    if (!c.shares_kv(l)) {
        std::vector<float> K = rows_through(L.wk, U, T);
        std::vector<float> V = rows_through(L.wv, U, T);
        for (size_t t = 0; t < T; ++t)
            for (size_t h = 0; h < c.Hkv; ++h) {
                rmsnorm(K.data() + t * KW + h * dh, L.k_norm.data(), dh, c.eps);
                rope_apply(K.data() + t * KW + h * dh, inv.data(), dh, s.tokens + t);
                rmsnorm_noscale(V.data() + t * KW + h * dh, dh, c.eps);
            }
        s.keys[l].insert(s.keys[l].end(), K.begin(), K.end());
        s.values[l].insert(s.values[l].end(), V.begin(), V.end());
    }
    const size_t src = c.kv_source(l), group = c.Hq / c.Hkv;
    std::vector<float> A(T * QW);
    for (size_t t = 0; t < T; ++t) {
        const size_t pos = s.tokens + t;
        // CausalWindow::visible_rows (attention.hpp:170-176)
        const size_t first = c.full(l) || pos + 1 <= c.window ? 0 : pos + 1 - c.window;
        for (size_t h = 0; h < c.Hq; ++h)
            attend_one(Q.data() + t * QW + h * dh, s.keys[src].data(), s.values[src].data(), KW, h / group, dh, first, pos + 1, 1.f, A.data() + t * QW + h * dh);
    }
    return rows_through(L.wo, A.data(), T);
}

}  // namespace

void gemma4_forward(const Gemma4Model& m, Gemma4State& s, const int32_t* ids, size_t T, float* logits) {
    const Gemma4Config& c = m.c;
    if (T == 0) throw std::invalid_argument("gemma4 forward: empty input");
    if (T > c.CTX - s.tokens) throw std::length_error("gemma4 forward: context exhausted");
    const size_t D = c.D, P = c.P, PL = c.P * c.L;
    std::vector<float> X(T * D);
    gemma4_embed(m, ids, T, X.data());
    // GemmaPerLayerInputs (gemma4.hpp:127-135): the token part from the packed
    // table times sqrt(P), the context part W X / sqrt(D) normalized per
    // P-wide slice, then (context + token) / sqrt(2)
    const float token_scale = std::sqrt(float(P)), proj_scale = 1.f / std::sqrt(float(D)), comb = 1.f / std::sqrt(2.f);
    std::vector<float> tok(T * PL);
    for (size_t t = 0; t < T; ++t) {
        dequant_row(m.ple_table.type, static_cast<const uint8_t*>(m.ple_table.w) + size_t(ids[t]) * row_bytes(m.ple_table.type, PL), tok.data() + t * PL, PL);
        for (size_t i = 0; i < PL; ++i) tok[t * PL + i] *= token_scale;
    }
    std::vector<float> ple = rows_through(m.ple_proj, X.data(), T);
    for (float& v : ple) v *= proj_scale;
    for (size_t t = 0; t < T; ++t)
        for (size_t l = 0; l < c.L; ++l) rmsnorm(ple.data() + t * PL + l * P, m.ple_norm.data(), P, c.eps);
    for (size_t i = 0; i < T * PL; ++i) ple[i] = (ple[i] + tok[i]) * comb;

    for (size_t l = 0; l < c.L; ++l) {
        const Gemma4Layer& L = m.layers[l];
        // GemmaE4BLayer::forward (gemma4.hpp:258-272)
        const std::vector<float> U = normed(X.data(), T, D, L.attn_norm, c.eps);
        const std::vector<float> A = normed(gemma_attention(m, l, s, U.data(), T).data(), T, D, L.post_attn_norm, c.eps);
        std::vector<float> H(T * D);
        for (size_t i = 0; i < T * D; ++i) H[i] = X[i] + A[i];
        const std::vector<float> Z = normed(H.data(), T, D, L.ffn_norm, c.eps);
        std::vector<float> g = rows_through(L.gate, Z.data(), T);
        const std::vector<float> u = rows_through(L.up, Z.data(), T);
        for (size_t i = 0; i < g.size(); ++i) g[i] = gelu_tanh(g[i]) * u[i];  // GatedMLP (components.hpp:300-304)
        const std::vector<float> F = normed(rows_through(L.down, g.data(), T).data(), T, D, L.post_ffn_norm, c.eps);
        for (size_t i = 0; i < T * D; ++i) H[i] = H[i] + F[i];
        // GemmaPerLayerResidual (gemma4.hpp:98-104): gelu(W_gate h) * ple_l,
        // projected, post-normed, plus h
        std::vector<float> pg = rows_through(L.pgate, H.data(), T);
        for (size_t t = 0; t < T; ++t)
            for (size_t i = 0; i < P; ++i) pg[t * P + i] = gelu_tanh(pg[t * P + i]) * ple[t * PL + l * P + i];
        const std::vector<float> B = normed(rows_through(L.proj, pg.data(), T).data(), T, D, L.post_norm, c.eps);
        for (size_t i = 0; i < T * D; ++i) X[i] = (B[i] + H[i]) * L.out_scale;
    }
    s.tokens += T;
    // gemma4.hpp:440-444: final norm of the last row, tied head, soft-cap
    std::vector<float> last(X.begin() + (T - 1) * D, X.begin() + T * D);
    rmsnorm(last.data(), m.final_norm.data(), D, c.eps);
    linear_rows(m.embedding, last.data(), 1, logits);
    for (size_t v = 0; v < c.V; ++v) logits[v] = gemma_softcap(logits[v], c.softcap);
}

}  // namespace oracle
