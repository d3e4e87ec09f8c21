// capi_model.cpp -- extern "C" surface of include/hero_model.h over the C++
// model (hero/model.hpp) and the synthetic model writer (hero/synth.hpp).
#include "hero_model.h"

#include "hero/errors.hpp"
#include "hero/model.hpp"
#include "hero/synth.hpp"

using namespace hero;

struct hero_model {
    std::unique_ptr<Qwen35Model> impl;
};
struct hero_state {
    std::unique_ptr<Qwen35Model::State> impl;
};

namespace {
void need(bool ok, const char* what) {
    if (!ok) throw Error(HERO_EINVAL, what);
}
SynthConfig to_synth(const hero_synth_config* c) {
    need(c != nullptr, "null synth config");
    SynthConfig s;
    s.V = uint64_t(c->vocab);
    s.D = uint64_t(c->d_model);
    s.L = uint64_t(c->layers);
    s.FF = uint64_t(c->ffn);
    s.Hq = uint64_t(c->q_heads);
    s.Hkv = uint64_t(c->kv_heads);
    s.head_dim = uint64_t(c->head_dim);
    s.Dk = uint64_t(c->key_head_dim);
    s.Dv = uint64_t(c->value_head_dim);
    s.Hk = uint64_t(c->key_heads);
    s.Hv = uint64_t(c->value_heads);
    s.conv_width = uint64_t(c->conv_width);
    s.ctx = uint64_t(c->ctx);
    s.rope_base = c->rope_base;
    s.tied = c->tied != 0;
    s.seed = c->seed;
    s.weight_mix = uint32_t(c->weight_mix);
    need(c->vocab > 0 && c->d_model > 0 && c->layers > 0 && c->ffn > 0 && c->q_heads > 0 && c->kv_heads > 0 && c->head_dim > 0, "synth: dimensions must be positive");
    need(c->key_head_dim > 0 && c->value_head_dim > 0 && c->key_heads > 0 && c->value_heads > 0 && c->conv_width > 0 && c->ctx > 0, "synth: dimensions must be positive");
    return s;
}
}  // namespace

extern "C" {

int hero_model_open(const char* path, hero_model** out) {
    return guard([&] {
        need(path && out, "null argument");
        auto m = std::make_unique<hero_model>();
        m->impl = Qwen35Model::open(path);
        *out = m.release();
    });
}

int hero_model_open_image(const void* image, size_t size, hero_model** out) {
    return guard([&] {
        need(image && out && size > 0, "null argument");
        auto m = std::make_unique<hero_model>();
        m->impl = Qwen35Model::open_image(static_cast<const uint8_t*>(image), size);
        *out = m.release();
    });
}

void hero_model_close(hero_model* model) { delete model; }

int hero_model_dims_get(const hero_model* model, hero_model_dims* out) {
    return guard([&] {
        need(model && out, "null argument");
        const ModelConfig& c = model->impl->config();
        out->vocab = c.V;
        out->d_model = c.D;
        out->layers = c.L;
        out->ctx = c.CTX;
        out->q_heads = c.Hq;
        out->kv_heads = c.Hkv;
        out->head_dim = c.Dh;
        out->rotary_dims = c.rotary_dims;
        out->key_head_dim = c.Dk;
        out->value_head_dim = c.Dv;
        out->key_heads = c.Hk;
        out->value_heads = c.Hv;
        out->conv_width = c.W;
        out->ffn = c.FF;
        out->tied = c.tied ? 1 : 0;
        out->rope_base = c.rope_base;
        out->rms_eps = c.eps;
        out->device_bytes = model->impl->device_bytes();
    });
}

int hero_state_create(const hero_model* model, int64_t max_tokens, hero_state** out) {
    return guard([&] {
        need(model && out, "null argument");
        auto s = std::make_unique<hero_state>();
        s->impl = model->impl->new_state(max_tokens);
        *out = s.release();
    });
}

int hero_batch_state_create(const hero_model* model, int64_t max_tokens, int32_t batch, uint32_t flags, hero_state** out) {
    return guard([&] {
        need(model && out, "null argument");
        need((flags & ~(HERO_STATE_KV_FP16 | HERO_STATE_KV_Q8_0 | HERO_STATE_GDN_CHUNKED)) == 0, "unknown state flags");
        need((flags & HERO_STATE_KV_FP16) == 0 || (flags & HERO_STATE_KV_Q8_0) == 0, "choose one attention cache format");
        auto s = std::make_unique<hero_state>();
        const int kv = (flags & HERO_STATE_KV_Q8_0) ? Qwen35Model::kKvQ8 : (flags & HERO_STATE_KV_FP16) ? Qwen35Model::kKvF16 : Qwen35Model::kKvF32;
        s->impl = model->impl->new_state(max_tokens, batch, kv, (flags & HERO_STATE_GDN_CHUNKED) != 0);
        *out = s.release();
    });
}

int64_t hero_state_batch(const hero_state* state) { return state ? state->impl->batch() : -1; }

int64_t hero_state_seq_tokens(const hero_state* state, int32_t seq) {
    if (!state || seq < 0 || seq >= state->impl->batch()) return -1;
    return state->impl->tokens(seq);
}

void hero_state_destroy(hero_state* state) { delete state; }

int hero_state_reset(hero_state* state) {
    return guard([&] {
        need(state, "null state");
        state->impl->reset();
    });
}

int64_t hero_state_tokens(const hero_state* state) { return state ? state->impl->tokens() : -1; }

int hero_model_embed(const hero_model* model, const int32_t* ids, int64_t n, float* out) {
    return guard([&] {
        need(model && ids && out, "null argument");
        model->impl->embed(ids, n, out);
    });
}

int hero_model_forward(const hero_model* model, hero_state* state, const float* rows, const int32_t* ids, int64_t t, float* logits, int32_t* next_id) {
    return guard([&] {
        need(model && state, "null argument");
        model->impl->forward(*state->impl, rows, ids, t, logits, next_id);
    });
}

int hero_model_forward_seq(const hero_model* model, hero_state* state, int32_t seq, const float* rows, const int32_t* ids, int64_t t, float* logits, int32_t* next_id) {
    return guard([&] {
        need(model && state, "null argument");
        model->impl->forward_seq(*state->impl, seq, rows, ids, t, logits, next_id);
    });
}

int hero_model_decode_batch(const hero_model* model, hero_state* state, const int32_t* first_ids, int64_t steps, int32_t* out_ids, float* logits) {
    return guard([&] {
        need(model && state && first_ids && out_ids, "null argument");
        model->impl->decode_batch(*state->impl, first_ids, steps, out_ids, logits);
    });
}

int hero_model_decode_greedy(const hero_model* model, hero_state* state, int32_t first_id, int64_t steps, int32_t* out_ids, float* logits) {
    return guard([&] {
        need(model && state && out_ids, "null argument");
        model->impl->decode_greedy(*state->impl, first_id, steps, out_ids, logits);
    });
}

double hero_model_last_decode_seconds(const hero_model* model) { return model ? model->impl->last_decode_seconds() : 0.0; }

int hero_model_time_gemvs(const hero_model* model, hero_state* state, int32_t reps, double* seconds, int64_t* launches, int64_t* bytes) {
    return guard([&] {
        need(model && state && seconds && launches && bytes && reps > 0, "bad argument");
        *seconds = model->impl->time_gemvs(*state->impl, reps, launches, bytes);
    });
}

int64_t hero_synth_qwen35_size(const hero_synth_config* config) {
    int64_t size = -1;
    const int rc = guard([&] { size = int64_t(synth_qwen35_size(to_synth(config))); });
    return rc == 0 ? size : -1;
}

int hero_synth_qwen35_image(const hero_synth_config* config, void* image, size_t capacity) {
    return guard([&] {
        need(image != nullptr, "null image");
        synth_qwen35_image(to_synth(config), static_cast<uint8_t*>(image), capacity);
    });
}

int hero_synth_qwen35_file(const hero_synth_config* config, const char* path) {
    return guard([&] {
        need(path != nullptr, "null path");
        synth_qwen35_file(to_synth(config), path);
    });
}

}  // extern "C"
