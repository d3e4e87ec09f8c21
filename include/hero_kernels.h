/* hero_kernels.h -- C ABI of the gfx950 kernels under the Q8_0 Qwen 3.5 hybrid
 * forward pass. Plain pointers and sizes only: every buffer argument is a
 * DEVICE pointer (hipMalloc'd or a view into one), every `stream` is a
 * hipStream_t passed as void* (NULL = the default stream). Calls enqueue work
 * and return; they do not synchronize.
 *
 * Return value: 0 on success, otherwise a HERO_E* code; hero_last_error()
 * then describes the failure (thread-local). Shapes are validated before
 * anything is enqueued.
 *
 * Layouts
 *   Q8_0 GGUF blocks   [N][K/32] x 34 bytes {fp16 d; int8 q[32]}, row-major by
 *                      output row (the GGUF / ggml tensor layout).
 *   packed weight      [N*K int8 q, row-major][(Npad/8) x (K/32) x 8 fp16 d]
 *                      Npad = N rounded up to 8 (rows past N unused); the scale
 *                      of (row n, block b) at ((n/8)*(K/32) + b)*8 + n%8;
 *                      hero_q8_0_packed_bytes()
 *   quantized act      [M*K int8 q][M*(K/32) fp32 d]        hero_q8_0_act_bytes()
 *                      (d is the fp16-rounded scale, decoded exactly)
 */
#ifndef HERO_KERNELS_H
#define HERO_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    HERO_OK = 0,
    HERO_EINVAL = 1,  /* bad shape, null or misaligned pointer */
    HERO_EHIP = 2,    /* a HIP runtime call failed */
    HERO_ERANGE = 3,  /* context or position out of range */
    HERO_ENOMEM = 4,  /* device allocation failed */
    HERO_EIO = 5      /* file / GGUF format error */
};

const char* hero_last_error(void);
const char* hero_version(void);

int64_t hero_q8_0_packed_bytes(int64_t n, int64_t k);
int64_t hero_q8_0_act_bytes(int64_t m, int64_t k);

/* GGUF Q8_0 blocks -> packed layout. Replaces the zero-copy Weight view of
 * nm/src/quant.hpp:448-451 (weights are uploaded once, then repacked).
 * `row0` places the rows at an offset inside a packed buffer of `n_total`
 * rows, so several GGUF tensors with the same K can share one packed matrix. */
int hero_q8_0_pack(const void* gguf_blocks, void* packed, int64_t n_total, int64_t k, int64_t row0, int64_t rows, void* stream);

/* quantize_row_q8_0 on M rows (nm/src/quant_i8.hpp:70-80; ActQ::from,
 * :329-341). x: [M][K] fp32. Bit-exact. K % 32 == 0. */
int hero_q8_0_quantize(const float* x, void* act, int64_t m, int64_t k, void* stream);

/* y[N] = W[N,K] x for one quantized activation row: Weight::matvec
 * (nm/src/quant_i8.hpp:352-383), per-row block order preserved (bit-exact).
 * If `residual` is non-NULL, y = residual + W x (the residual add of
 * nm/src/qwen35.hpp:321,326). */
int hero_q8_0_gemv(const void* packed, const void* act, float* y, const float* residual, int64_t n, int64_t k, void* stream);

/* y = W * quantize(RMSNorm(x)) (+ residual): RMSNorm
 * (nm/src/components.hpp:176-181), quantize_row_q8_0 and Weight::matvec
 * (nm/src/quant_i8.hpp:70-80,352-383) in one launch when K == 4096, the norm
 * formed in the GEMV's prologue while its first weights load; otherwise as
 * two launches through `act_scratch` (hero_q8_0_act_bytes(1, K) bytes).
 * x, gamma: [K] fp32. Bit-exact. */
int hero_rmsnorm_q8_0_gemv(const void* packed, const float* x, const float* gamma, float eps, float* y, const float* residual, int64_t n, int64_t k, void* act_scratch, void* stream);

/* y = W * quantize(silu(gate) * up) (+ residual): the SwiGLU of
 * nm/src/components.hpp:300-304 followed by the down projection, in one
 * launch when K (= FF) is 4096, 8192 or 12288, else through `act_scratch`.
 * gate_up: [gate K | up K] fp32. Bit-exact. */
int hero_swiglu_q8_0_gemv(const void* packed, const float* gate_up, float* y, const float* residual, int64_t n, int64_t k, void* act_scratch, void* stream);

/* Pack two [rows][K] GGUF Q8_0 tensors into one matrix in alternating
 * `interleave`-row chunks: source row r lands on row
 * row0 + (r / interleave) * 2 * interleave + r % interleave. Used for the
 * SwiGLU gate (row0 = 0) and up (row0 = interleave) projections, interleave 32. */
int hero_q8_0_pack_interleaved(const void* gguf_blocks, void* packed, int64_t n_total, int64_t k, int64_t row0, int64_t rows, int64_t interleave, void* stream);

/* RMSNorm, the gate and up projections and SwiGLU in one launch: act_out =
 * quantize(silu(W_gate x') * (W_up x')), x' = quantize(RMSNorm(x)), i.e.
 * nm/src/components.hpp:176-181 and :300-304 up to the down projection's
 * input. `packed` is [2*ff][k] from hero_q8_0_pack_interleaved with
 * interleave 32; k == 4096; act_out: hero_q8_0_act_bytes(1, ff). Bit-exact. */
int hero_rmsnorm_q8_0_gemv_swiglu(const void* packed, const float* x, const float* gamma, float eps, void* act_out, int64_t ff, int64_t k, void* stream);

/* Y[M][N] = X W^T for M quantized activation rows (hero_q8_0_quantize with
 * m = M): Weight::matmul (nm/src/quant_i8.hpp:430-474), every element equal
 * to the single-row vec_dot_q8_0_q8_0 (block order kept, bit-exact). The int32
 * block sums come from int8 MFMA. If `residual` is non-NULL, Y = R + X W^T
 * ([M][N]). For prefill and batched decode. */
int hero_q8_0_gemm(const void* packed, const void* act, float* y, const float* residual, int64_t m, int64_t n, int64_t k, void* stream);

/* Which kernel hero_q8_0_gemm runs for an (m, n, k) on the current device,
 * without running it: *kernel = 1 (skinny, one wave per range of 16-row
 * groups), 2 (skinny, sixteen waves sharing each group), 3 (skinny, waves
 * per range of 16-row groups with the activation rows in shared memory), 4
 * (skinny, two or four waves per range of 16-row groups, one per 16
 * activation rows: 16 < m <= 64) or the tiled kernel's rows per tile (16, 32,
 * 64, 128). The choice depends on the
 * device's compute-unit count. No counterpart in the reference (its matmul
 * has one form, nm/src/quant_i8.hpp:430-474); lets tests show that every
 * form was checked. */
int hero_q8_0_gemm_plan(int64_t m, int64_t n, int64_t k, int32_t* kernel);

/* Exact int32 block dot products out[N][K/32] of one activation row: the
 * `sumi` of nm/src/quant_i8.hpp:94-95, exported for parity checks. */
int hero_q8_0_block_sums(const void* packed, const void* act, int32_t* out, int64_t n, int64_t k, void* stream);

/* RMSNorm over each of M rows of D, then Q8_0 quantization
 * (nm/src/components.hpp:176-181 followed by quant_i8.hpp:70-80).
 * y (fp32 normalized rows) and act may each be NULL. D % 32 == 0. */
int hero_rmsnorm_quant(const float* x, const float* gamma, float eps, float* y, void* act, int64_t m, int64_t d, void* stream);

/* SwiGLU + quantize: g = silu(gate) * up over rows [gate FF | up FF]
 * (nm/src/components.hpp:300-304), quantized for the down projection. */
int hero_swiglu_quant(const float* gate_up, void* act, int64_t m, int64_t ff, void* stream);

/* Embedding gather from a packed Q8_0 table [V][D]: out[i] = d*q
 * (Weight::gather_rows, nm/src/quant.hpp:464-480). */
int hero_q8_0_embed(const void* packed, int64_t v, int64_t d, const int32_t* ids, int64_t n, float* out, void* stream);

/* Greedy argmax of M rows of n logits, ties to the lowest index
 * (Logits::argmax, nm/src/logits.hpp:61-66). scratch: M*128 uint64. */
int hero_argmax(const float* logits, int64_t m, int64_t n, int32_t* out, uint64_t* scratch, void* stream);

/* hero_argmax without the scratch argument and without any allocation: the
 * partial keys live in a static device array of 64 rows x 128 keys (64 KiB
 * per GPU, kept until the process ends). No counterpart in the reference; for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops that forbid hipMalloc). m <= 64, else HERO_EINVAL. Every call
 * on one GPU shares the array: calls that overlap on one GPU (on two streams
 * at once) race. Results equal hero_argmax's. The array's device address is
 * looked up once per device, with the current device, on the first call or
 * when a model is opened on that device: make that first call (or open a
 * model) outside graph capture, and pass a stream of the current device. */
int hero_argmax_noalloc(const float* logits, int64_t m, int64_t n, int32_t* out, void* stream);

/* ---- K-quant weights (GGUF Q4_K = 12, Q5_K = 13, Q6_K = 14) ----------------
 * Weights are used in a packed form of hero_kquant_packed_bytes(type, n, k)
 * bytes (the GGUF tensor's bytes, its blocks in slots of a tiled layout with
 * each wave's loads contiguous, padded to whole waves): hero_kquant_pack
 * copies a device GGUF tensor (n rows of k/256 super-blocks of 144 / 176 / 210
 * bytes) into it (Q4_K and Q6_K also regroup their quant bytes by sub-block
 * and residue within each block).
 * hero_kquant_gemm replaces the int8-activation branch of Weight<In,Out>::matvec
 * / ::matmul (nm/src/quant_i8.hpp:352-383, 430-474) for Q4_K / Q6_K: the
 * activation rows are quantized to Q8_K (quantize_row_q8_K,
 * nm/src/quant_i8.hpp:31-64), then y[m][n] = vec_dot_q{4,6}_K_q8_K(k, W row n,
 * act row m) (the x86 scalar forms, nm/src/quant_i8.hpp:146-191, 239-278), bit
 * for bit. act holds hero_q8_K_act_bytes(m, k) bytes: the m rows of GGUF Q8_K
 * blocks (fp32 d, 256 int8, 16 int16 sums), then, 16-byte aligned, a copy of
 * each block's int8 regrouped for 4-way dots (256 bytes per block).
 * hero_q5_K_gemm is the fp32-activation branch for Q5_K, which has no integer
 * kernel (has_i8_kernel, nm/src/quant_i8.hpp:325): y[m][n] = sum over blocks in
 * order of dot_block_q5_K (nm/src/quant.hpp:207-229) on the fp32 rows x [m][k].
 * hero_kquant_dequant_rows is Weight::dequant_row / gather_rows
 * (nm/src/quant.hpp:464-480) on a packed tensor: out[t][k] = row ids[t] (device
 * ids; an id outside [0, n) gives a row of zeros).
 * k: a multiple of 256, at most 65536 (16384 for Q5_K). */
int64_t hero_q8_K_act_bytes(int64_t m, int64_t k);
int hero_q8_K_quantize(const float* x, void* act, int64_t m, int64_t k, void* stream);
int64_t hero_kquant_packed_bytes(int32_t type, int64_t n, int64_t k);
int hero_kquant_pack(int32_t type, const void* gguf, void* packed, int64_t n, int64_t k, void* stream);
int hero_kquant_gemm(int32_t type, const void* w, const void* act, float* y, int64_t m, int64_t n, int64_t k, void* stream);
int hero_q5_K_gemm(const void* w, const float* x, float* y, int64_t m, int64_t n, int64_t k, void* stream);
int hero_kquant_dequant_rows(int32_t type, const void* w, int64_t n, int64_t k, const int32_t* ids, int64_t n_ids, float* out, void* stream);

/* Logits::sample with temp > 0 (nm/src/logits.hpp:71-105) on one row of v
 * logits: the top_k candidates (1 <= top_k <= 1024; top_k > v means v), sorted
 * by logit descending with equal logits by ascending id, p = expf((l - max) /
 * temp), the top_p prefix, and the draw. u in [0, 1) is the value the caller's
 * generator gives std::generate_canonical<float, 24> (what the reference's
 * uniform_real_distribution<float>(0, s2) scales by s2). out: two int32 of
 * device memory; the token id goes to out[0], out[1] is used as a flag between
 * the two kernels of the call. temp <= 0 is greedy: use hero_argmax. */
int hero_sample_topk(const float* logits, int64_t v, int32_t top_k, float temp, float top_p, float u, int32_t* out, void* stream);

/* The same Logits::sample for any top_k: 0 (the whole vocabulary,
 * nm/src/logits.hpp:76 with k = V) or any k >= 1 (1 .. 1024 take
 * hero_sample_topk's kernels and need no workspace). The logits are sorted on
 * the device (logit descending, equal logits by ascending id), then the
 * reference's sum, top_p prefix, s2 and draw run over the first k as exact
 * sequential sums. work: hero_sample_work_bytes(v) bytes of device memory
 * (256-byte aligned); out as for hero_sample_topk. */
int64_t hero_sample_work_bytes(int64_t v);
int hero_sample(const float* logits, int64_t v, int32_t top_k, float temp, float top_p, float u, void* work, int64_t work_bytes, int32_t* out, void* stream);

/* The scalar functions of the path evaluated on the device, for parity
 * checks: out[0..n) = expf, [n..2n) = log1pf, then silu
 * (nm/src/components.hpp:105), sigmoid (nm/src/core.hpp:579), softplus
 * (nm/src/recurrent.hpp:35). expf and log1pf return exactly glibc's values. */
int hero_math_eval(const float* x, float* out, int64_t n, void* stream);
/* Gemma 4's scalar functions on the device: out[2i] = gelu_pytorch_tanh(x[i])
 * (nm/src/components.hpp:73-81), out[2i+1] = cap * tanh(x[i] / cap)
 * (gemma_softcap, nm/src/gemma4.hpp:79); tanh returns exactly glibc's tanhf. */
int hero_gemma_math_eval(const float* x, float* out, int64_t n, float cap, void* stream);

/* Gated delta-net decode, one token for each of B sequences, all Hv heads:
 * conv step + SiLU, q/k L2 norm, beta/decay gates, the gated delta rule,
 * per-head RMSNorm, SiLU(z) gate, Q8_0 quantization of the output
 * projection's input. Replaces the per-token body of
 * QwenGatedDeltaNet mix_tokens (nm/src/qwen35.hpp:420-462) together with
 * gated_delta_step (nm/src/recurrent.hpp:146-177). Dk = Dv = 128. */
typedef struct hero_gdn_decode_args {
    const float* proj;       /* [B][proj_stride] input projections, fp32 */
    int64_t proj_stride;     /* floats per sequence */
    int64_t z_off, beta_off, alpha_off; /* offsets of z [Hv*Dv], beta [Hv], alpha [Hv]; qkv at 0 */
    const float* conv_taps;  /* [CC][W], CC = 2*Hk*Dk + Hv*Dv */
    float* conv_hist;        /* [B][W][CC] ring, zero-initialized for a new sequence */
    float* state;            /* [B][Hv][Dk][Dv] fp32, zero for a new sequence */
    const float* dt_bias;    /* [Hv] */
    const float* decay;      /* [Hv] = -exp(A_log) <= 0 */
    const float* norm_gamma; /* [Dv] */
    float eps;
    const int32_t* positions;/* [B] position of the token being decoded */
    void* act_out;           /* quantized act [B][Hv*Dv] */
    float* out_f32;          /* optional [B][Hv*Dv] */
    int32_t b, hk, hv, dk, dv, conv_width;
} hero_gdn_decode_args;
int hero_gdn_decode(const hero_gdn_decode_args* args, void* stream);

/* The same decode step split over value columns: 8 workgroups of one wave
 * per (sequence, head), 16 value columns each (the delta rule's columns are
 * independent, nm/src/recurrent.hpp:146-177). Writes the raw delta-rule
 * outputs o_raw [B][Hv*128] (before the head RMSNorm), the output gates
 * silu(z) into `gates` [B][Hv*128] if non-NULL, the new state and the conv
 * ring; args->act_out and args->out_f32 are not written (act_out may be
 * NULL). Followed by hero_gdn_norm_gate, or by hero_headgate_q8_0_gemv, the
 * results equal hero_gdn_decode's bit for bit. */
int hero_gdn_decode_cols(const hero_gdn_decode_args* args, float* o_raw, float* gates, void* stream);

/* The per-head RMSNorm, SiLU(z) gate and Q8_0 quantization of raw delta-net
 * outputs (the tail of nm/src/qwen35.hpp:457-460 and quantize_row_q8_0):
 * o_raw [args->b][Hv*128] -> args->act_out (and args->out_f32 if set); z is
 * read from args->proj at z_off. */
int hero_gdn_norm_gate(const float* o_raw, const hero_gdn_decode_args* args, void* stream);

/* y = W * quantize(head_rmsnorm(o_raw) * gates) (+ residual) in one launch:
 * the delta-net output projection (nm/src/qwen35.hpp:457-460) with the head
 * norm (32 heads of 128, weight gamma [128]), the gate (gates = silu(z), as
 * hero_gdn_decode_cols writes them) and the quantization formed in the GEMV's
 * prologue. k == 4096. Bit-exact. */
int hero_headgate_q8_0_gemv(const void* packed, const float* o_raw, const float* gates, const float* gamma, float eps, float* y, const float* residual, int64_t n, int64_t k, void* stream);

/* Delta-net prefill: the same work for T = args->b consecutive tokens of ONE
 * sequence at positions positions[0] .. positions[0]+T-1 (only positions[0]
 * is read). proj, act_out and out_f32 have T rows; conv_hist and state are
 * that sequence's ([W][CC] and [Hv][Dk][Dv]). The tokens run in order, as the
 * reference's token loop does (nm/src/qwen35.hpp:436-455), so the result equals
 * T calls of hero_gdn_decode bit for bit; the conv ring then holds the chunk's
 * last W positions. `work` is device scratch of at least
 * hero_gdn_prefill_work_bytes(T, hk, hv) bytes. */
int64_t hero_gdn_prefill_work_bytes(int64_t t, int32_t hk, int32_t hv);
int hero_gdn_prefill(const hero_gdn_decode_args* args, void* work, int64_t work_bytes, void* stream);

/* The same prefill in the chunked (WY) form of the delta rule over chunks of 64
 * tokens: the per-token recurrence unrolled into small matrix products per
 * chunk (the chunked-prefill form the reference's serial loop,
 * nm/src/qwen35.hpp:436-455, is pinned against). Equal to hero_gdn_prefill up
 * to fp32 rounding order (tolerance, not bit for bit); same workspace. */
int hero_gdn_prefill_chunked(const hero_gdn_decode_args* args, void* work, int64_t work_bytes, void* stream);

/* Gated GQA attention decode over an fp32 K/V cache, one token for each of
 * B sequences: head-pair split, q/k RMSNorm + RoPE (host table), cache
 * append, softmax(scale*q.k) over the visible rows, sum alpha*v,
 * sigmoid(gate), Q8_0 quantization for the output projection. Replaces the
 * attention body of nm/src/qwen35.hpp:343-395 (window == 0) and the
 * sliding-window visibility of nm/src/attention.hpp:159-176 (window > 0). */
typedef struct hero_attn_decode_args {
    const float* proj;       /* [B][proj_stride]: [q|gate] head pairs at 0, k, v */
    int64_t proj_stride, k_off, v_off;
    const float* q_gamma;    /* [Dh] */
    const float* k_gamma;    /* [Dh] */
    float eps;
    const float* rope_cs;    /* [max_pos][Dh/2][2] cos, sin */
    float* k_cache;          /* [B][Hkv][Dh][max_ctx], channel-major per K/V head */
    float* v_cache;          /* [B][max_ctx][Hkv*Dh] */
    int64_t max_ctx;
    const int32_t* positions;/* [B] */
    float* scores;           /* scratch [B][Hq][max_ctx] */
    float* q_rot;            /* scratch [B][Hq][Dh] */
    float score_scale;       /* 1/sqrt(Dh) for Qwen, 1 for Gemma-style */
    int32_t window;          /* 0 = full causal */
    void* act_out;           /* quantized act [B][Hq*Dh] */
    float* out_f32;          /* optional [B][Hq*Dh] */
    int32_t b, hq, hkv, dh;
} hero_attn_decode_args;
int hero_attn_decode(const hero_attn_decode_args* args, void* stream);

/* The same attention for B consecutive tokens of ONE sequence (a prefill
 * chunk): row b is the token at positions[b], all rows share cache 0 (k_cache
 * [1][Hkv][Dh][max_ctx], v_cache [1][max_ctx][Hkv*Dh]), every row's k and v
 * are appended before any row's scores, and row b attends to the rows at or
 * before positions[b] (within the window). Replaces the T-row reduction of
 * nm/src/qwen35.hpp:363-387: the whole batch is appended to the cache, then
 * each (row, head) is reduced over its visible rows. */
int hero_attn_prefill(const hero_attn_decode_args* args, void* stream);

/* The same attention over a paged fp16 K/V cache (north-star format; the
 * reference keeps fp32 rows, nm/src/attention.hpp:248-249). Keys and values
 * are stored rounded to nearest-even fp16; the visible keys of each (sequence,
 * KV head) are split across workgroups and the per-split softmax partials
 * merged, so results equal the reference over fp16-rounded K/V to a few ulp
 * (not bit for bit). Pages hold page_size positions: pool layout
 * [page][2 = K, V][hkv][page_size][dh] fp16; page_table [b][max_pages].
 * In `a`, k_cache, v_cache, scores and max_ctx are unused; the cache spans
 * max_pages * page_size positions.
 * q8 = 1: the pages hold Q8_0 rows instead (the K/V storage the reference
 * plans, nm/INFERENCE_PLAN.md:235-236): each page is [2][hkv][page_size][dh]
 * int8 followed by [2][hkv][page_size][dh/32] fp16 scales
 * (hero_attn_page_bytes); a row is appended through the reference's
 * activation quantizer (quant_i8.hpp:70-80) and read back as d * q
 * (quant.hpp:306-313), so results equal the reference over those values to a
 * few ulp. */
typedef struct hero_attn_paged_args {
    hero_attn_decode_args a;
    uint16_t* pages;
    const int32_t* page_table;
    int32_t page_size, max_pages;
    float* work;                /* split partials, hero_attn_paged_work_bytes */
    int64_t work_bytes;
    int32_t q8;
} hero_attn_paged_args;
/* Bytes of one page (head_dim 128 or 256; Q8_0 pages for 128 only) and of
 * the split workspace. Heads of 256 channels take fp16 pages of 64 positions. */
int64_t hero_attn_page_bytes(int32_t hkv, int32_t head_dim, int32_t page_size, int32_t q8);
int64_t hero_attn_paged_work_bytes(int64_t max_ctx, int32_t window, int32_t b, int32_t hq, int32_t hkv, int32_t head_dim);

/* Measurement (no counterpart in the reference): `workgroups` workgroups of
 * 256 lanes read `bytes` of p (a multiple of 16, 16-byte aligned) with 16-byte
 * loads, each its contiguous share, and store nothing (out is written only on
 * an impossible fold): the read bandwidth the memory-bound kernels are
 * compared with. */
int hero_read_probe(const void* p, int64_t bytes, int32_t workgroups, uint32_t* out, void* stream);
/* Measurement (no counterpart in the reference): read every byte of a packed
 * n x 4096 Q8_0 matrix as hero_q8_0_gemv will read it, workgroup g of this
 * launch what the GEMV's workgroup g reads (so on the same XCD), and store
 * nothing: the GEMV that follows finds its weights in its XCDs' L2. */
int hero_q8_0_gemv_prefetch(const void* packed, int64_t n, int64_t k, void* stream);
int hero_attn_decode_paged(const hero_attn_paged_args* args, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* HERO_KERNELS_H */
