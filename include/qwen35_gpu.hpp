// qwen35_gpu.hpp -- the reference engine's model contract over this build's
// C ABI: GpuQwen35Model<C> models TransformerModel (nm/src/transformer.hpp:70-78),
// so PrefixCache<GpuQwen35Model<C>> (transformer.hpp:97-169) and the tools that
// drive it (tools/qwen35_check.cpp:45-67) use the GPU path unchanged.
//
// This header belongs next to nm/src/qwen35.hpp: it includes the reference's
// own headers (compile with -I<reference>/nm/src -I<this repo>/include and link
// -lhero_amd). C is a Qwen 3.5 config type of the reference's shape
// (qwen35.hpp:26-88); the GPU loader accepts 128- or 256-wide attention heads
// (the published Qwen 3.5 4B / 9B shapes have 256) and 128-wide delta-net heads.
#pragma once

#include <hero_model.h>

#include <algorithm>
#include <cstdint>
#include <memory>
#include <span>
#include <stdexcept>
#include <string>
#include <vector>

#include "logits.hpp"
#include "multimodal.hpp"
#include "qwen35.hpp"

// HERO_* status -> the reference's exception types: running out of context is
// std::length_error (qwen35.hpp:289, transformer.hpp:115), bad arguments
// std::invalid_argument, everything else (HIP, I/O, memory) std::runtime_error.
inline void hero_throw(int status) {
    if (status == HERO_OK) return;
    const std::string message = hero_last_error();
    if (status == HERO_ERANGE) throw std::length_error(message);
    if (status == HERO_EINVAL) throw std::invalid_argument(message);
    throw std::runtime_error(message);
}

template <class C>
class GpuQwen35Model {
public:
    static constexpr size_t D = C::D, V = C::V, CTX = C::CTX;
    // positions of a device state when the caller names none (the K/V caches
    // are sized to a state's positions when it is created; any count up to
    // C::CTX may be asked for)
    static constexpr size_t kDefaultStateTokens = 65536;

    // The carried state. PrefixCache owns it by value and forgets it by
    // assigning a fresh one (transformer.hpp:155), so it is
    // default-constructible and move-assignable, and frees its device memory
    // when destroyed. The device state is created by the first forward().
    class PrefixState {
    public:
        PrefixState() = default;
        PrefixState(PrefixState&&) noexcept = default;
        PrefixState& operator=(PrefixState&&) noexcept = default;
        size_t tokens() const { return state_ ? size_t(hero_state_tokens(state_.get())) : 0; }

    private:
        friend class GpuQwen35Model;
        struct Destroy {
            void operator()(hero_state* s) const { hero_state_destroy(s); }
        };
        std::unique_ptr<hero_state, Destroy> state_;
    };

    // max_tokens: the context of the states this model creates, at most
    // C::CTX; 0 takes min(C::CTX, kDefaultStateTokens).
    explicit GpuQwen35Model(const std::string& gguf_path, size_t max_tokens = 0)
        : max_tokens_(max_tokens ? max_tokens : std::min(CTX, kDefaultStateTokens)) {
        if (max_tokens_ > CTX) throw std::invalid_argument("GpuQwen35Model: max_tokens above the model's context");
        hero_model* m = nullptr;
        hero_throw(hero_model_open(gguf_path.c_str(), &m));
        model_.reset(m);
        hero_model_dims dims{};
        hero_throw(hero_model_dims_get(model_.get(), &dims));
        if (size_t(dims.d_model) != D || size_t(dims.vocab) != V) throw std::invalid_argument("GpuQwen35Model: checkpoint dimensions differ from the config");
    }
    GpuQwen35Model(const GpuQwen35Model&) = delete;  // weights are immutable and never copied
    GpuQwen35Model& operator=(const GpuQwen35Model&) = delete;

    Matrix<D> embed(std::span<const TokenId> ids) const {
        std::vector<Scalar> rows(ids.size() * D);
        if (!ids.empty()) {
            std::vector<int32_t> raw(ids.size());
            for (size_t i = 0; i < ids.size(); ++i) raw[i] = int32_t(ids[i]);
            hero_throw(hero_model_embed(model_.get(), raw.data(), int64_t(raw.size()), rows.data()));
        }
        return Matrix<D>::from_row_major(std::move(rows));
    }

    Logits<V> forward(PrefixState& prefix_state, EmbeddedRows<D> input) const {
        if (input.tokens() == 0) throw std::invalid_argument("forward: no rows");
        if (!prefix_state.state_) {
            hero_state* s = nullptr;
            hero_throw(hero_state_create(model_.get(), int64_t(max_tokens_), &s));
            prefix_state.state_.reset(s);
        }
        // the rows must continue the carried state (attention.hpp:215-220)
        if (input.conversation_position() != Position{prefix_state.tokens()}) throw std::invalid_argument("forward: rows do not continue the state");
        // the view hides its buffer: stage it row by row
        std::vector<Scalar> rows;
        rows.reserve(input.tokens() * D);
        for (size_t i = 0; i < input.tokens(); ++i) {
            const VecView<D> row = input.embedding(i);
            rows.insert(rows.end(), row.begin(), row.end());
        }
        Vec<V> logits;
        hero_throw(hero_model_forward(model_.get(), prefix_state.state_.get(), rows.data(), nullptr, int64_t(input.tokens()), logits.begin(), nullptr));
        return Logits<V>(std::move(logits));
    }

    size_t max_tokens() const { return max_tokens_; }

private:
    struct Close {
        void operator()(hero_model* m) const { hero_model_close(m); }
    };
    std::unique_ptr<hero_model, Close> model_;
    size_t max_tokens_;
};
