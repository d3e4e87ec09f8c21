/* hero_gemma4.h -- C ABI of the GPU Gemma 4 text model (E4B schema, Q8_0 GGUF).
 *
 * The model-forward boundary of the reference's Gemma 4 E4B text model,
 * flattened to C:
 *   hero_gemma4_open / hero_gemma4_open_image  <- gemma4_loader::load_e4b_text
 *                                                (nm/src/gemma4_loader.hpp:31-52, 105-130)
 *   hero_gemma4_state_create / reset / tokens  <- Gemma4E4BCache (nm/src/gemma4.hpp:343-378)
 *   hero_gemma4_embed                          <- Gemma4E4BModel::embed (nm/src/gemma4.hpp:415-419)
 *   hero_gemma4_forward                        <- Gemma4E4BModel::forward (nm/src/gemma4.hpp:424-445)
 *   hero_gemma4_decode_greedy                  <- the greedy loop of tools/gemma4_text.cpp:38-52
 * Dimensions are read from the GGUF metadata (the reference fixes them to the
 * E4B configuration at compile time); the layer schedule is the reference's:
 * layer l attends over the whole context when l % 6 == 5 and over a sliding
 * window otherwise, and the last shared_kv_layers layers reuse the caches of
 * the last earlier layer of their kind (nm/src/gemma4.hpp:36-57, 343-378).
 *
 * Input rows are token ids only: the per-layer inputs (PLE) read a table row
 * per token id, so rows without an id (multimodal soft tokens) are outside
 * this boundary. Host pointers are host memory. All calls return 0 or a
 * HERO_E* code (message in hero_last_error()); context exhaustion is
 * HERO_ERANGE, matching the reference's std::length_error.
 */
#ifndef HERO_GEMMA4_H
#define HERO_GEMMA4_H

#include <stddef.h>
#include <stdint.h>

#include "hero_kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct hero_gemma4 hero_gemma4;
typedef struct hero_gemma4_state hero_gemma4_state;

typedef struct hero_gemma4_dims {
    int64_t vocab, d_model, layers, ctx, ffn;
    int64_t q_heads, kv_heads, local_head_dim, full_head_dim;
    int64_t per_layer_input, window, shared_kv_layers;
    float rms_eps, logit_softcap;
    int64_t device_bytes; /* weights resident on the device */
} hero_gemma4_dims;

/* Load a GGUF file (mmap) / an in-memory image, validate the gemma4 schema,
 * upload and repack the weights (every 2-D weight Q8_0). */
int hero_gemma4_open(const char* gguf_path, hero_gemma4** out);
int hero_gemma4_open_image(const void* image, size_t size, hero_gemma4** out);
void hero_gemma4_close(hero_gemma4* model);
int hero_gemma4_dims_get(const hero_gemma4* model, hero_gemma4_dims* out);

/* One sequence's K/V caches (fp32; the window layers' caches are rings of
 * `window` rows) for up to `max_tokens` positions (<= the model's ctx). */
int hero_gemma4_state_create(const hero_gemma4* model, int64_t max_tokens, hero_gemma4_state** out);
void hero_gemma4_state_destroy(hero_gemma4_state* state);
int hero_gemma4_state_reset(hero_gemma4_state* state);
int64_t hero_gemma4_state_tokens(const hero_gemma4_state* state);

/* Input embeddings (the token row times sqrt(d_model)) for n ids: out[n][D]. */
int hero_gemma4_embed(const hero_gemma4* model, const int32_t* ids, int64_t n, float* out);

/* Run `t` token ids (host) at the state's position, one token after another
 * (each row's results equal the reference's batched prefill row, which
 * attends over the same visible keys). Writes the last row's soft-capped
 * logits (host, [V]) if non-NULL and its greedy id if non-NULL; advances the
 * state by t. */
int hero_gemma4_forward(const hero_gemma4* model, hero_gemma4_state* state, const int32_t* ids, int64_t t, float* logits, int32_t* next_id);

/* Greedy decode from `first_id`: `steps` passes, each feeding the previous
 * greedy id; out_ids[i] = the greedy id after pass i; logits of the final
 * pass if non-NULL. The step is one HIP graph replayed. */
int hero_gemma4_decode_greedy(const hero_gemma4* model, hero_gemma4_state* state, int32_t first_id, int64_t steps, int32_t* out_ids, float* logits);
/* Device seconds of the last hero_gemma4_decode_greedy call. */
double hero_gemma4_last_decode_seconds(const hero_gemma4* model);

/* ---- synthetic models (host) -------------------------------------------- */
typedef struct hero_synth_gemma4_config {
    int64_t vocab, d_model, layers, ffn;
    int64_t q_heads, kv_heads, local_head_dim, full_head_dim;
    int64_t per_layer_input, window, shared_kv_layers, ctx;
    uint64_t seed;
} hero_synth_gemma4_config;

/* Seeded random-init gemma4 GGUF in the E4B schema: Q8_0 2-D weights
 * (N(0, 0.02) before quantization), F32 norm weights and per-layer
 * layer_output_scale scalars. size -> bytes of the image; image -> fill a
 * caller buffer; file -> write to a path. */
int64_t hero_synth_gemma4_size(const hero_synth_gemma4_config* config);
int hero_synth_gemma4_image(const hero_synth_gemma4_config* config, void* image, size_t capacity);
int hero_synth_gemma4_file(const hero_synth_gemma4_config* config, const char* path);

#ifdef __cplusplus
}
#endif
#endif /* HERO_GEMMA4_H */
