// kernels.hpp -- host-side launchers of the gfx950 kernels (internal API).
// Pointers are device pointers; every launcher enqueues on `s` and returns
// immediately. Shape validation happens in the C ABI layer (capi.cpp).
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>
#include <cstdint>

#include "hero/prefetch.hpp"

namespace hero {

// GEMV epilogues: y = Wx; y = r + Wx; for a [gate|up] matrix packed in
// alternating 32-row chunks (K = 4096, N % 64 == 0), y <- the quantized
// activation of silu(gate) * up ([N/2] int8 + [N/64] fp32 scales); and
// (streaming GEMV, quantized input) y = gelu(Wx) on the rows below
// GemvInput::act_rows, Wx past them
enum : int { kEpiStore = 0, kEpiResidual = 1, kEpiSwigluQuant = 2, kEpiGelu = 3 };

// packed Q8_0 weight: [N][K] int8, then the fp16 scales by 8-row group,
// [Npad/8][K/32][8] with Npad = N rounded up to 8 (rows past N unused): the
// scales of 8 consecutive rows of one block are one 16-byte load, and those of
// one 8-row group for every block are contiguous (one sweep per sub-batch)
inline int64_t packed_rows_pad(int64_t N) { return (N + 7) / 8 * 8; }
int device_cus();  // compute units of the current device (cached per device)
// index of the scale of (row, block) among the fp16 scales; nb = K/32
__host__ __device__ inline int64_t scale_index(int64_t row, int64_t block, int64_t nb) { return ((row >> 3) * nb + block) * 8 + (row & 7); }
inline int64_t packed_q8_bytes(int64_t N, int64_t K) { return N * K + packed_rows_pad(N) * (K / 32) * 2; }
inline int64_t act_q8_bytes(int64_t M, int64_t K) { return M * K + M * (K / 32) * 4; }
// K-quants (kquant.hip): Q8_K activations (292 bytes per 256 plus the
// residue-regrouped int8), the Q4_K (type 12) / Q6_K (type 14) products over
// packed weights, the Q5_K (type 13) product over fp32 rows, and the
// embedding gather. Packed: Q4_K / Q6_K residue-regrouped (launch_kquant_pack),
// Q5_K as in the GGUF; the same bytes as the GGUF tensor.
int64_t act_q8_K_bytes(int64_t m, int64_t k);
int64_t kquant_packed_bytes(int type, int64_t N, int64_t K);
int kquant_max_k(int type);  // 65536 (Q4_K, Q6_K), 16384 (Q5_K)
void launch_kquant_pack(int type, const void* gguf, void* packed, int64_t N, int64_t K, hipStream_t s);
void launch_quantize_q8_K(const float* x, void* act, int64_t M, int64_t K, hipStream_t s);
// y[m * ldy + n] (+= resid[m * ldy + n], added after the product)
void launch_kquant_gemm_ld(int type, const void* w, const void* act, float* y, const float* resid, int64_t M, int64_t N, int64_t K, int64_t ldy,
                           hipStream_t s);
void launch_kquant_gemm(int type, const void* w, const void* act, float* y, int64_t M, int64_t N, int64_t K, hipStream_t s);
void launch_q5k_gemm(const void* w, const float* x, int64_t ldx, float* y, const float* resid, int64_t M, int64_t N, int64_t K, int64_t ldy, hipStream_t s);
// out[t][K] = row ids[t] of a packed K-quant tensor [N][K] as fp32
void launch_kquant_dequant_rows(int type, const void* w, int64_t N, int64_t K, const int32_t* ids, int64_t n, float* out, hipStream_t s);
// top-k / top-p sampling of one logits row (sample.hip); top_k in 1 .. sample_max_top_k()
int sample_max_top_k();
void launch_sample_topk(const float* logits, int64_t V, int top_k, float temp, float top_p, float u, int32_t* out, hipStream_t s);
// any top_k (0 = the whole vocabulary) over a sorted copy; work: sample_full_work_bytes(V)
int64_t sample_full_work_bytes(int64_t V);
void launch_sample_full(const float* logits, int64_t V, int top_k, float temp, float top_p, float u, void* work, int32_t* out, hipStream_t s);

// q8.hip
void launch_quantize_act(const float* x, void* act, int64_t M, int64_t K, hipStream_t s);
void launch_pack_q8(const void* gguf_blocks, void* packed, int64_t N_total, int64_t K, int64_t row0, int64_t rows, hipStream_t s, int64_t interleave = 0);
void launch_gemv_q8(const void* packed, const void* act, float* y, const float* resid, int64_t N, int64_t K, int epi, hipStream_t s);
// The streaming GEMV with its input formed in the prologue from one of six
// sources (kInRmsNorm and kInHeadGate at K == 4096, kInSwiglu at K a multiple
// of 4096, kInAct and kInMul at every K of gemv_streams_act, kInPostNorm at
// the K of gemv_post_norm_fusable).
enum : int { kInAct = 0, kInRmsNorm = 1, kInSwiglu = 2, kInHeadGate = 3, kInMul = 4, kInPostNorm = 5 };
struct GemvInput {
    int mode;
    const int8_t* xq;        // kInAct: quantized activation [K] + fp32 scales [K/32]
    const float* xd;
    const float* x;          // kInRmsNorm: residual row [K] (K == 4096), RMSNorm weight, eps
    const float* gamma;      // kInHeadGate: raw delta-net outputs [K] (K == 4096) in x, the
    float eps;               //   head norm's weight [128] in gamma, eps, and the gates silu(z) [K] in z
    const float* gate_up;    // kInSwiglu: [gate K | up K]; kInMul: a [K]
    const float* z;
    const float* up;         // kInMul: b [K]; the input is Q8_0(a * b)
    int act_rows;            // kEpiGelu: rows [0, act_rows) take the GELU
    // kInPostNorm: the end of a Gemma sub-block (launch_gemma_post_norm's
    // arithmetic) formed by every workgroup: o = (RMSNorm(x) * gamma + res) *
    // scale, written to out by workgroup 0; the input is Q8_0 of
    // RMSNorm(o) * next_gamma, or of o when next_gamma is null. out must not
    // alias x or res.
    const float* res;
    float scale;
    float* out;
    const float* next_gamma;
};
bool gemv_streams(int64_t K);
// the row lengths the streaming GEMV takes with the plain quantized input (and
// the GELU input): 256, 1024, 2048, 2560, 2816, 4096, 8192, 10240, 12288
bool gemv_streams_act(int64_t K);
// the row lengths the streaming GEMV takes with the post-norm input: 2560
bool gemv_post_norm_fusable(int64_t K);
// workgroups of the streaming GEMV's launch for N rows under epilogue epi
int gemv_stream_grid(int64_t N, int epi);
// what another kernel's workgroups read ahead of the streaming GEMV over a
// packed N x K matrix (epilogue epi): of each GEMV workgroup's rows the first
// part / 8; .packed == nullptr where the GEMV does not stream (K not a
// multiple of 4096 up to 12288)
GemvPrefetch gemv_prefetch_of(const void* packed, int64_t N, int64_t K, int epi, int part = 8);
// G workgroups of 64 lanes, workgroup g reading what GEMV workgroup g reads (measurement)
void launch_gemv_prefetch(const GemvPrefetch& p, hipStream_t s);
void launch_gemv_q8_in(const void* packed, const GemvInput& in, float* y, const float* resid, int64_t N, int64_t K, int epi, hipStream_t s);
// Y[M][N] (+ R) = the M quantized activation rows (act_q8 layout, M rows)
// times W^T, each element in the reference's block order; int8 MFMA.
void launch_gemm_q8(const void* packed, const void* act, float* y, const float* resid, int64_t M, int64_t N, int64_t K, int epi, hipStream_t s);
// The gate/up GEMM of rows interleaved as 64-row units [32 gate | 32 up] with
// silu(gate) * up and its Q8_0 formed in the epilogue (out: the down
// projection's act [M][N/2] + scales); false (nothing launched) where the
// shape does not take the shared-memory skinny form
bool launch_gemm_q8_swiglu(const void* packed, const void* act, void* out, int64_t M, int64_t N, int64_t K, hipStream_t s);
// Which kernel launch_gemm_q8 runs for a shape: one of the two skinny forms
// (M <= 16) or the tiled kernel's row-tile height BM (16, 32, 64, 128).
enum : int { kGemmPlanSkinnyWave = 1, kGemmPlanSkinnyShared = 2, kGemmPlanSkinnyLds = 3, kGemmPlanSkinnyWave4 = 4 };
int gemm_q8_plan(int64_t M, int64_t N, int64_t K);
void launch_block_sums(const void* packed, const void* act, int32_t* out, int64_t N, int64_t K, hipStream_t s);

// norm.hip: rows x [M][D] -> RMSNorm (gamma, eps) -> quantized act; y (fp32) optional
void launch_rmsnorm_quant(const float* x, const float* gamma, float eps, float* y, void* act, int64_t M, int64_t D, hipStream_t s);

// ew.hip
// gate_up rows [M][2FF]: gate then up, or with interleave > 0 alternating
// chunks [gate il | up il | gate il | ...]
void launch_swiglu_quant(const float* gate_up, void* act, int64_t M, int64_t FF, hipStream_t s, int64_t interleave = 0);
// the same products as fp32 rows y [M][FF] (gate_up [M][gate FF | up FF])
void launch_swiglu_f32(const float* gate_up, float* y, int64_t M, int64_t FF, hipStream_t s);
void launch_embed_q8(const void* packed_embedding, int64_t V, int64_t D, const int32_t* ids, int64_t n, float* out, hipStream_t s);
// argmax over n logits per row (ties -> lowest index); out_index[M]
void launch_argmax(const float* logits, int64_t M, int64_t n, int32_t* out_index, uint64_t* scratch_keys, hipStream_t s);
// the same with the keys in a static device array (no allocation); M <= 64
constexpr int kArgmaxGroups = 128, kArgmaxNoallocRows = 64;
void launch_argmax_noalloc(const float* logits, int64_t M, int64_t n, int32_t* out_index, hipStream_t s);
// the current device's address of hero_argmax_noalloc's static key array (looked up once per device)
uint64_t* argmax_noalloc_scratch();

// a plain read of `bytes` (a multiple of 16) by `workgroups` workgroups of
// 256 lanes (measurement: the read bandwidth ceiling)
void launch_read_probe(const void* p, int64_t bytes, int workgroups, uint32_t* out, hipStream_t s);
// exp, log1p, silu, sigmoid, softplus of x[n] -> out[5][n] (parity export)
void launch_math_eval(const float* x, float* out, int64_t n, hipStream_t s);

// gdn.hip: gated delta-net decode for B sequences x Hv heads (one token each)
struct GdnDecodeArgs {
    const float* proj;      // [B][proj_stride]: qkv at 0, z at z_off, beta at beta_off, alpha at alpha_off
    int64_t proj_stride, z_off, beta_off, alpha_off;
    const float* conv_taps; // [CC][W]
    float* conv_hist;       // [B][W][CC], ring: slot p % W holds the input at position p
    float* state;           // [B][Hv][Dk][Dv]
    const float* dt_bias;   // [Hv]
    const float* decay;     // [Hv], -exp(A_log)
    const float* norm_gamma;// [Dv]
    float eps;
    const int32_t* positions; // [B] position of this token
    void* act_out;          // quantized WO input [B][Hv*Dv]
    float* out_f32;         // optional [B][Hv*Dv], the gated output before quantization
    int B, Hk, Hv, Dk, Dv, W;
};
void launch_gdn_decode(const GdnDecodeArgs& a, hipStream_t s);
// The same step split over value columns (8 workgroups of one wave per head):
// writes the raw delta-rule outputs o_raw [B][Hv*128] (before the head norm),
// the gates silu(z) into g_raw [B][Hv*128] if non-null, and the new state and
// ring; a.act_out / a.out_f32 are not written.
void launch_gdn_decode_cols(const GdnDecodeArgs& a, float* o_raw, float* g_raw, hipStream_t s);
// head RMSNorm, SiLU(z) gate and quantization of o_raw into a.act_out (and
// a.out_f32 if set), for a.B rows
void launch_gdn_norm_gate(const float* o_raw, const GdnDecodeArgs& a, hipStream_t s);
// The same for T = a.B consecutive tokens of ONE sequence at positions
// a.positions[0] + t (proj and act_out have T rows; state and ring are that
// sequence's), then the ring update. `work` holds gdn_prefill_work_bytes.
struct GdnPrefillWork {
    float* q;   // [T][Hk][128] normalised, query-scaled
    float* k;   // [T][Hk][128] normalised
    float* v;   // [T][Hv][128]
    float* o;   // [T][Hv][128] delta-rule outputs before the head norm
    float* bd;  // [T][Hv][2] beta, decay
    float* g;   // [T][Hv] log of the decay (decay = exp(g))
    // the chunked form only (chunks of 64 tokens, c = t / 64):
    float* u;   // [T][Hv][128] (I + L)^-1 beta v
    float* wm;  // [T][Hv][128] (I + L)^-1 beta gamma k
    float* p;   // [c][Hv][64][64] exp(G_t - G_s) q_t . k_s, s <= t
    float* G;   // [T][Hv] cumulative log-decay within the chunk
};
int64_t gdn_prefill_work_bytes(int64_t T, int64_t Hk, int64_t Hv);
// chunked = false: the token-serial scan, bit-exact with T decode steps.
// chunked = true: the chunked (WY) form of the same recurrence over chunks of
// 64 tokens -- matrix products instead of a 128-long chain per token; equal to
// the serial form up to fp32 rounding order, not bit for bit.
void launch_gdn_prefill(const GdnDecodeArgs& a, void* work, hipStream_t s, bool chunked = false);

// attn.hip: gated GQA decode over an fp32 K/V cache (one token per sequence)
struct AttnDecodeArgs {
    const float* proj;       // [B][proj_stride]: q|gate pairs at 0, k at k_off, v at v_off
    int64_t proj_stride, k_off, v_off;
    const float* q_gamma;    // [Dh]
    const float* k_gamma;    // [Dh]
    float eps;
    const float* rope_cs;    // [max_pos][Dh/2][2] (cos, sin) per position and plane
    float* k_cache;          // [B][Hkv][Dh][max_ctx] (channel-major)
    float* v_cache;          // [B][max_ctx][Hkv*Dh]
    int64_t max_ctx;
    const int32_t* positions;// [B]
    // 0: row b is sequence b (its own cache). 1: all B rows are consecutive
    // tokens of ONE sequence (prefill): they share cache 0, every row's k/v is
    // appended before any row's scores, and row b sees positions <= positions[b].
    int shared_cache;
    float* scores;           // scratch [B][Hq][max_ctx]
    float* q_rot;            // scratch [B][Hq][Dh]
    float score_scale;
    int window;              // 0 = full causal
    void* act_out;           // quantized WO input [B][Hq*Dh]
    float* out_f32;          // optional [B][Hq*Dh]
    int B, Hq, Hkv, Dh;
};
void launch_attn_decode(const AttnDecodeArgs& a, hipStream_t s);

// attn.hip, paged fp16 form: the same gated attention over a paged fp16 K/V
// cache, the visible keys of each (row, KV head) split across workgroups
// (split-K: per-split max, exp-sum and weighted V sum, merged per head).
// Fields of `a` used: proj, proj_stride, k_off, v_off, q_gamma, k_gamma, eps,
// rope_cs, positions, shared_cache, q_rot, score_scale, window, act_out,
// out_f32, B, Hq, Hkv, Dh (k_cache, v_cache, scores and max_ctx are not).
struct AttnPagedArgs {
    AttnDecodeArgs a;
    // fp16 pool [page][2 = K, V][Hkv][page_size][Dh]; with q8 set the pool is
    // bytes, each page [2][Hkv][page_size][Dh] int8 then [2][Hkv][page_size][Dh/32]
    // fp16 scales (Q8_0 rows: the reference's activation quantizer at append)
    uint16_t* pages;
    int q8;
    const int32_t* page_table;  // [B][max_pages] pool page of each page_size tokens (row 0 for all rows when shared_cache)
    int page_size;              // tokens per page
    int max_pages;              // pages per sequence: positions < max_pages * page_size
    int split;                  // keys per split, a multiple of 64, at most kAttnMaxSplit
    int nsplit;                 // splits per (row, KV head): ceil(visible keys at most / split)
    float* work;                // [B][Hq][nsplit][2 + Dh]: max, exp-sum, weighted V sum
};
constexpr int kAttnMaxSplit = 512;
// bytes of one page of the pool
// bytes of one page of page_size positions: fp16 K and V rows of Dh, or (q8,
// Dh 128) int8 rows and their four fp16 scales
inline int64_t attn_page_bytes(int64_t Hkv, int64_t Dh, int64_t page_size, bool q8) { return q8 ? 2 * Hkv * page_size * (Dh + Dh / 32 * 2) : 2 * Hkv * page_size * Dh * 2; }
constexpr int kAttnMaxGroup = 8;  // query heads per KV head
// split and nsplit for B rows over at most max_ctx positions (window 0 = full)
void attn_paged_plan(int64_t max_ctx, int window, int B, int Hkv, int* split, int* nsplit);
int64_t attn_paged_work_floats(int B, int Hq, int nsplit, int Dh);
void launch_attn_paged(const AttnPagedArgs& p, hipStream_t s);

// gemma.hip: the Gemma 4 text model's own kernels (one row: a decode step)
// x[D] = the embedding row of *id times embed_scale, act = its Q8_0 row, and
// tok[PL] = the per-layer table's row of *id times token_scale
void launch_gemma_embed(const void* emb, int64_t V, int64_t D, const void* ple_table, int64_t PL, const int32_t* id, float embed_scale, float token_scale, float* x,
                        void* act, float* tok, hipStream_t s);
// ple[l][:] = (RMSNorm_P(ctx[l][:] * proj_scale) * gamma + tok[l][:]) * comb, l < L
void launch_gemma_ple_inputs(const float* ctx, const float* tok, const float* gamma, float eps, float proj_scale, float comb, float* ple, int64_t L, int64_t P,
                             hipStream_t s);
// attention of one row over a K/V cache: K and V [Hkv][slots][Dh] (row-major);
// position p lives in slot p % slots (window > 0: a ring of `window` slots)
// or slot p (full)
struct GemmaAttnArgs {
    const float* proj;        // [q Hq*Dh | k Hkv*Dh at k_off | v Hkv*Dh at v_off]
    int64_t k_off, v_off;
    const float* q_gamma;     // [Dh]
    const float* k_gamma;     // [Dh]
    float eps;
    const float* rope_cs;     // [positions][Dh/2][2] (cos, sin)
    const int32_t* pos;       // device position of the row
    float* k_cache;
    float* v_cache;
    int64_t slots;
    int window;               // 0: every earlier position is visible
    int append;               // 1: form this row's k and v and append them
    float* q_rot;             // scratch [Hq][Dh]
    float* scores;            // scratch [Hq][max_ctx]
    int64_t max_ctx;
    void* act_out;            // Q8_0 W_o input [Hq*Dh]
    int Hq, Hkv, Dh;          // Dh 256 or 512
};
void launch_gemma_attention(const GemmaAttnArgs& a, hipStream_t s);
// out = (RMSNorm(a) * gamma + res) * scale; act = Q8_0 of next_gamma ?
// RMSNorm(out) * next_gamma : out (D <= 4096, D % 32 == 0)
void launch_gemma_post_norm(const float* a, const float* gamma, const float* res, float scale, float eps, float* out, const float* next_gamma, void* act, int64_t D,
                            hipStream_t s);
// act = Q8_0 of gelu_tanh(gate[i]) * mul[i], N % 32 == 0
void launch_gemma_gelu_mul_quant(const float* gate, const float* mul, void* act, int64_t N, hipStream_t s);
// logits[i] = cap * tanh(logits[i] / cap)
void launch_gemma_softcap(float* logits, int64_t n, float cap, hipStream_t s);
// out[2i] = gelu_tanh(x[i]), out[2i+1] = cap * tanh(x[i] / cap) (tests)
void launch_gemma_math_eval(const float* x, float* out, int64_t n, float cap, hipStream_t s);

}  // namespace hero
