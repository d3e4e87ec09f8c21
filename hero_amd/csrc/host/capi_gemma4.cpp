// capi_gemma4.cpp -- extern "C" surface of include/hero_gemma4.h over the C++
// Gemma 4 model (hero/gemma4.hpp) and the synthetic model writer (hero/synth.hpp).
#include "hero_gemma4.h"

#include "hero/errors.hpp"
#include "hero/gemma4.hpp"
#include "hero/synth.hpp"

using namespace hero;

struct hero_gemma4 {
    std::unique_ptr<Gemma4Model> impl;
};
struct hero_gemma4_state {
    std::unique_ptr<Gemma4Model::State> impl;
};

namespace {
void need(bool ok, const char* what) {
    if (!ok) throw Error(HERO_EINVAL, what);
}
Gemma4SynthConfig to_synth(const hero_synth_gemma4_config* c) {
    need(c != nullptr, "null synth config");
    need(c->vocab > 0 && c->d_model > 0 && c->layers > 0 && c->ffn > 0 && c->q_heads > 0 && c->kv_heads > 0, "synth: dimensions must be positive");
    need(c->local_head_dim > 0 && c->full_head_dim > 0 && c->per_layer_input > 0 && c->window > 0 && c->shared_kv_layers >= 0 && c->ctx > 0,
         "synth: dimensions must be positive");
    Gemma4SynthConfig s;
    s.V = uint64_t(c->vocab);
    s.D = uint64_t(c->d_model);
    s.L = uint64_t(c->layers);
    s.FF = uint64_t(c->ffn);
    s.Hq = uint64_t(c->q_heads);
    s.Hkv = uint64_t(c->kv_heads);
    s.local_dim = uint64_t(c->local_head_dim);
    s.full_dim = uint64_t(c->full_head_dim);
    s.ple = uint64_t(c->per_layer_input);
    s.window = uint64_t(c->window);
    s.shared_kv_layers = uint64_t(c->shared_kv_layers);
    s.ctx = uint64_t(c->ctx);
    s.seed = c->seed;
    return s;
}
}  // namespace

extern "C" {

int hero_gemma4_open(const char* path, hero_gemma4** out) {
    return guard([&] {
        need(path && out, "null argument");
        auto m = std::make_unique<hero_gemma4>();
        m->impl = Gemma4Model::open(path);
        *out = m.release();
    });
}

int hero_gemma4_open_image(const void* image, size_t size, hero_gemma4** out) {
    return guard([&] {
        need(image && out && size > 0, "null argument");
        auto m = std::make_unique<hero_gemma4>();
        m->impl = Gemma4Model::open_image(static_cast<const uint8_t*>(image), size);
        *out = m.release();
    });
}

void hero_gemma4_close(hero_gemma4* model) { delete model; }

int hero_gemma4_dims_get(const hero_gemma4* model, hero_gemma4_dims* out) {
    return guard([&] {
        need(model && out, "null argument");
        const Gemma4Config& c = model->impl->config();
        out->vocab = c.V;
        out->d_model = c.D;
        out->layers = c.L;
        out->ctx = c.CTX;
        out->ffn = c.FF;
        out->q_heads = c.Hq;
        out->kv_heads = c.Hkv;
        out->local_head_dim = c.Dl;
        out->full_head_dim = c.Df;
        out->per_layer_input = c.P;
        out->window = c.window;
        out->shared_kv_layers = c.shared;
        out->rms_eps = c.eps;
        out->logit_softcap = c.softcap;
        out->device_bytes = model->impl->device_bytes();
    });
}

int hero_gemma4_state_create(const hero_gemma4* model, int64_t max_tokens, hero_gemma4_state** out) {
    return guard([&] {
        need(model && out, "null argument");
        auto s = std::make_unique<hero_gemma4_state>();
        s->impl = model->impl->new_state(max_tokens);
        *out = s.release();
    });
}

void hero_gemma4_state_destroy(hero_gemma4_state* state) { delete state; }

int hero_gemma4_state_reset(hero_gemma4_state* state) {
    return guard([&] {
        need(state, "null state");
        state->impl->reset();
    });
}

int64_t hero_gemma4_state_tokens(const hero_gemma4_state* state) { return state ? state->impl->tokens() : -1; }

int hero_gemma4_embed(const hero_gemma4* model, const int32_t* ids, int64_t n, float* out) {
    return guard([&] {
        need(model && ids && out, "null argument");
        model->impl->embed(ids, n, out);
    });
}

int hero_gemma4_forward(const hero_gemma4* model, hero_gemma4_state* state, const int32_t* ids, int64_t t, float* logits, int32_t* next_id) {
    return guard([&] {
        need(model && state && ids, "null argument");
        model->impl->forward(*state->impl, ids, t, logits, next_id);
    });
}

int hero_gemma4_decode_greedy(const hero_gemma4* model, hero_gemma4_state* state, int32_t first_id, int64_t steps, int32_t* out_ids, float* logits) {
    return guard([&] {
        need(model && state && out_ids, "null argument");
        model->impl->decode_greedy(*state->impl, first_id, steps, out_ids, logits);
    });
}

double hero_gemma4_last_decode_seconds(const hero_gemma4* model) { return model ? model->impl->last_decode_seconds() : 0.0; }

int64_t hero_synth_gemma4_size(const hero_synth_gemma4_config* config) {
    int64_t size = -1;
    const int rc = guard([&] { size = int64_t(synth_gemma4_size(to_synth(config))); });
    return rc == 0 ? size : -1;
}

int hero_synth_gemma4_image(const hero_synth_gemma4_config* config, void* image, size_t capacity) {
    return guard([&] {
        need(image != nullptr, "null image");
        synth_gemma4_image(to_synth(config), static_cast<uint8_t*>(image), capacity);
    });
}

int hero_synth_gemma4_file(const hero_synth_gemma4_config* config, const char* path) {
    return guard([&] {
        need(path != nullptr, "null path");
        synth_gemma4_file(to_synth(config), path);
    });
}

}  // extern "C"
