/* hero_model.h -- C ABI of the GPU Qwen 3.5 hybrid model (Q8_0 GGUF).
 *
 * This is the model-forward boundary of the reference engine, flattened to C:
 *   hero_model_open / hero_model_open_image   <- qwen35_loader::load<C>
 *                                               (nm/src/qwen35_loader.hpp:141-155)
 *   hero_state_create / reset / tokens         <- Qwen35State<C> (nm/src/qwen35.hpp:206-241),
 *                                               PrefixState::tokens() (nm/src/transformer.hpp:74)
 *   hero_model_embed                           <- Qwen35Model::embed (nm/src/qwen35.hpp:285)
 *   hero_model_forward                         <- Qwen35Model::forward (nm/src/qwen35.hpp:288-303)
 *   hero_model_argmax / greedy id outputs      <- Logits::argmax (nm/src/logits.hpp:61-66)
 * Weights stay immutable after load; a state is owned by one caller and is
 * not re-entrant (the reference's single-caller threading model).
 *
 * Host pointers are host memory; everything else lives on the device. All
 * calls return 0 or a HERO_E* code from hero_kernels.h (message in
 * hero_last_error()). Context exhaustion is HERO_ERANGE, matching the
 * reference's std::length_error.
 */
#ifndef HERO_MODEL_H
#define HERO_MODEL_H

#include <stddef.h>
#include <stdint.h>

#include "hero_kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct hero_model hero_model;
typedef struct hero_state hero_state;

typedef struct hero_model_dims {
    int64_t vocab, d_model, layers, ctx;
    int64_t q_heads, kv_heads, head_dim, rotary_dims;
    int64_t key_head_dim, value_head_dim, key_heads, value_heads, conv_width;
    int64_t ffn;
    int64_t tied;            /* 1 if the LM head is the embedding */
    double rope_base;
    float rms_eps;
    int64_t device_bytes;    /* weights resident on the device */
} hero_model_dims;

/* Load a GGUF file (mmap) / an in-memory GGUF image, validate the qwen35
 * schema (nm/src/qwen35_loader.hpp:30-75), upload and repack the weights. */
int hero_model_open(const char* gguf_path, hero_model** out);
int hero_model_open_image(const void* image, size_t size, hero_model** out);
void hero_model_close(hero_model* model);
int hero_model_dims_get(const hero_model* model, hero_model_dims* out);

/* Per-sequence carried state: K/V caches (fp32) for the attention layers,
 * conv history and fp32 delta state for the recurrent layers. `max_tokens`
 * bounds the context this state can hold (<= the model's ctx). */
int hero_state_create(const hero_model* model, int64_t max_tokens, hero_state** out);
void hero_state_destroy(hero_state* state);
int hero_state_reset(hero_state* state);
int64_t hero_state_tokens(const hero_state* state);

/* Embedding rows for `n` token ids into host memory out[n][D]. */
int hero_model_embed(const hero_model* model, const int32_t* ids, int64_t n, float* out);

/* Run T new rows at the state's position: `rows` (host, [T][D]) if non-NULL,
 * else the embeddings of `ids` (host, [T]) gathered on the device. Writes the
 * last row's logits to `logits` (host, [V]) if non-NULL and its greedy id to
 * *next_id if non-NULL. Advances the state by T. */
int hero_model_forward(const hero_model* model, hero_state* state, const float* rows, const int32_t* ids, int64_t t, float* logits, int32_t* next_id);

/* Greedy decode: starting from token `first_id` at the state's position, run
 * `steps` forward passes feeding each greedy id back in (the loop of
 * tools/qwen35_check.cpp:54-70). out_ids[i] = greedy id after pass i.
 * Logits of the final pass are written to `logits` if non-NULL. */
int hero_model_decode_greedy(const hero_model* model, hero_state* state, int32_t first_id, int64_t steps, int32_t* out_ids, float* logits);

/* ---- batched decode --------------------------------------------------------
 * No counterpart in the reference, whose model contract carries one sequence
 * per state (nm/src/transformer.hpp:70-78). For callers that decode several
 * independent sequences at once: a batch state holds `batch` (1..16)
 * sequences, each with its own caches and position; every sequence's results
 * equal those of its own single-sequence state, bit for bit. */
int hero_batch_state_create(const hero_model* model, int64_t max_tokens, int32_t batch, uint32_t flags, hero_state** out);
/* flags: keep the attention cache as fp16 pages with split-K attention (the
 * north-star cache format; the reference's cache is fp32). Results then equal
 * the reference over fp16-rounded keys and values to a few ulp. */
#define HERO_STATE_KV_FP16 1u
/* flags: run the delta-net prefill in its chunked form (chunks of 64 tokens,
 * matrix products instead of the token-serial chain; equal to the reference
 * to fp32 rounding order instead of bit for bit). */
#define HERO_STATE_GDN_CHUNKED 2u
/* flags: keep the attention cache as Q8_0 pages (int8 rows with an fp16 scale
 * per 32, 1.0625 bytes per value) with split-K attention. The reference has
 * no such cache, only a plan line for one (nm/INFERENCE_PLAN.md:235-236); here
 * each appended row is quantized by the reference's activation quantizer
 * (quant_i8.hpp:70-80) and read back as d * q (quant.hpp:306-313). Results
 * are checked against the oracle's own Q8_0-cache switch (equal to a few ulp:
 * the split-K sums), not against reference outputs: parity with the
 * reference is unpinned for this format. Exclusive with HERO_STATE_KV_FP16. */
#define HERO_STATE_KV_Q8_0 4u
int64_t hero_state_batch(const hero_state* state);
int64_t hero_state_seq_tokens(const hero_state* state, int32_t seq);
/* hero_model_forward for sequence `seq` of a batch state. */
int hero_model_forward_seq(const hero_model* model, hero_state* state, int32_t seq, const float* rows, const int32_t* ids, int64_t t, float* logits, int32_t* next_id);
/* Greedy decode of every sequence at once, each from its own position:
 * first_ids[B]; out_ids[steps][B] (row i = the greedy ids after pass i);
 * logits [B][V] of the final pass if non-NULL. */
int hero_model_decode_batch(const hero_model* model, hero_state* state, const int32_t* first_ids, int64_t steps, int32_t* out_ids, float* logits);

/* Seconds of device time of the last hero_model_decode_greedy or
 * hero_model_decode_batch call (HIP
 * events around the decode passes on the model's stream). */
double hero_model_last_decode_seconds(const hero_model* model);

/* Measurement: every Q8_0 matvec of one decode step (all layers and the LM
 * head, the real weights, in step order) launched `reps` times back to back
 * between HIP events on the model's stream. Returns the elapsed seconds in
 * *seconds; *launches and *bytes are per repetition, bytes being algorithmic
 * (weights + fp16 scales, quantized activation, outputs, residual reads).
 * Touches only the state's scratch buffers; the carried state is unchanged. */
int hero_model_time_gemvs(const hero_model* model, hero_state* state, int32_t reps, double* seconds, int64_t* launches, int64_t* bytes);

/* ---- synthetic models (host) -------------------------------------------- */
typedef struct hero_synth_config {
    int64_t vocab, d_model, layers, ffn;
    int64_t q_heads, kv_heads, head_dim;
    int64_t key_head_dim, value_head_dim, key_heads, value_heads, conv_width;
    int64_t ctx;
    double rope_base;
    int32_t tied;
    uint64_t seed;
    int32_t weight_mix;
} hero_synth_config;

/* Seeded random-init qwen35 GGUF, N(0,0.02) weights before quantization.
 * weight_mix 0: every 2-D weight Q8_0; 1: the tensor types of a Q4_K_M
 * checkpoint (Q6_K embedding, LM head, ffn_down and attn_v; Q5_K attn_qkv and
 * attn_output; Q4_K the other projections; Q8_0 ssm_alpha/ssm_beta); 2: Q8_0
 * in-projections, gate and up beside a Q6_K embedding and ffn_down and Q4_K
 * ssm_out / attn_output. Mixes 1 and 2 need every K-quant input width a
 * multiple of 256. size -> bytes of the image; image -> fill a
 * caller buffer; file -> write to a path. */
int64_t hero_synth_qwen35_size(const hero_synth_config* config);
int hero_synth_qwen35_image(const hero_synth_config* config, void* image, size_t capacity);
int hero_synth_qwen35_file(const hero_synth_config* config, const char* path);

#ifdef __cplusplus
}
#endif
#endif /* HERO_MODEL_H */
