// capi_kernels.cpp -- the extern "C" kernel entry points of include/hero_kernels.h:
// argument validation, then the launcher. No allocation happens here.
#include "hero_kernels.h"

#include <string>

#include "hero/errors.hpp"
#include "hero/kernels.hpp"

using namespace hero;

namespace {

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

void require(bool ok, const std::string& what) {
    if (!ok) throw Error(HERO_EINVAL, what);
}

void check_q8_shape(int64_t n, int64_t k) {
    require(n > 0 && k > 0, "shape must be positive");
    require(k % 32 == 0, "K must be a multiple of 32 (Q8_0 block)");
    require(n <= (int64_t(1) << 31) && k <= (int64_t(1) << 20), "shape too large");
}

}  // namespace

extern "C" {

const char* hero_last_error(void) { return last_error_message(); }
const char* hero_version(void) { return "hero_amd 0.1 (gfx950)"; }

int64_t hero_q8_0_packed_bytes(int64_t n, int64_t k) { return packed_q8_bytes(n, k); }
int64_t hero_q8_0_act_bytes(int64_t m, int64_t k) { return act_q8_bytes(m, k); }

int hero_q8_0_pack(const void* src, void* packed, int64_t n_total, int64_t k, int64_t row0, int64_t rows, void* stream) {
    return guard([&] {
        check_q8_shape(n_total, k);
        require(src && packed, "null pointer");
        require(aligned(packed, 16), "packed buffer must be 16-byte aligned");
        require(row0 >= 0 && rows > 0 && row0 + rows <= n_total, "row range outside the packed matrix");
        launch_pack_q8(src, packed, n_total, k, row0, rows, as_stream(stream));
        check_launch("hero_q8_0_pack");
    });
}

int hero_q8_0_quantize(const float* x, void* act, int64_t m, int64_t k, void* stream) {
    return guard([&] {
        check_q8_shape(m, k);
        require(x && act, "null pointer");
        require(aligned(x, 16) && aligned(act, 16), "x and act must be 16-byte aligned");
        launch_quantize_act(x, act, m, k, as_stream(stream));
        check_launch("hero_q8_0_quantize");
    });
}

int hero_sample_topk(const float* logits, int64_t v, int32_t top_k, float temp, float top_p, float u, int32_t* out, void* stream) {
    return guard([&] {
        require(logits && out, "null pointer");
        require(v > 0 && v <= (int64_t(1) << 30), "vocabulary size out of range");
        require(top_k >= 1 && top_k <= sample_max_top_k(), "top_k must be in 1 .. 1024 on the device");
        require(temp > 0.f, "temp must be positive (temp <= 0 is greedy: hero_argmax)");
        require(u >= 0.f && u < 1.f, "u must be in [0, 1)");
        launch_sample_topk(logits, v, top_k, temp, top_p, u, out, as_stream(stream));
        check_launch("hero_sample_topk");
    });
}

int64_t hero_sample_work_bytes(int64_t v) {
    if (v <= 0 || v > (int64_t(1) << 30)) return -1;
    try {
        return sample_full_work_bytes(v);
    } catch (...) {
        return -1;
    }
}

int hero_sample(const float* logits, int64_t v, int32_t top_k, float temp, float top_p, float u, void* work, int64_t work_bytes, int32_t* out, void* stream) {
    return guard([&] {
        require(logits && out, "null pointer");
        require(v > 0 && v <= (int64_t(1) << 30), "vocabulary size out of range");
        require(top_k >= 0, "top_k must be >= 0 (0: the whole vocabulary)");
        require(temp > 0.f, "temp must be positive (temp <= 0 is greedy: hero_argmax)");
        require(u >= 0.f && u < 1.f, "u must be in [0, 1)");
        if (top_k >= 1 && top_k <= sample_max_top_k()) {
            launch_sample_topk(logits, v, top_k, temp, top_p, u, out, as_stream(stream));
        } else {
            require(work != nullptr && aligned(work, 256), "work: 256-byte aligned device memory");
            require(work_bytes >= sample_full_work_bytes(v), "work_bytes below hero_sample_work_bytes(v)");
            launch_sample_full(logits, v, top_k, temp, top_p, u, work, out, as_stream(stream));
        }
        check_launch("hero_sample");
    });
}

int64_t hero_q8_K_act_bytes(int64_t m, int64_t k) { return act_q8_K_bytes(m, k); }

int hero_q8_K_quantize(const float* x, void* act, int64_t m, int64_t k, void* stream) {
    return guard([&] {
        require(m > 0 && k > 0 && k % 256 == 0, "K must be a positive multiple of 256 (Q8_K block)");
        require(m * (k / 256) <= (int64_t(1) << 31), "shape too large");
        require(x && act, "null pointer");
        require(aligned(x, 16) && aligned(act, 16), "x and act must be 16-byte aligned");
        launch_quantize_q8_K(x, act, m, k, as_stream(stream));
        check_launch("hero_q8_K_quantize");
    });
}

namespace {
void check_kquant_shape(int32_t type, int64_t n, int64_t k) {
    require(n > 0 && k > 0 && k % 256 == 0, "K must be a positive multiple of 256 (K-quant super-block)");
    require(k <= kquant_max_k(type) && n <= (int64_t(1) << 31) && n * (k / 256) <= (int64_t(1) << 31), "shape too large");
}
}  // namespace

int64_t hero_kquant_packed_bytes(int32_t type, int64_t n, int64_t k) {
    if (!(type == 12 || type == 13 || type == 14) || n <= 0 || k <= 0 || k % 256 != 0) return -1;
    return kquant_packed_bytes(type, n, k);
}

int hero_kquant_pack(int32_t type, const void* gguf, void* packed, int64_t n, int64_t k, void* stream) {
    return guard([&] {
        require(type == 12 || type == 13 || type == 14, "type must be 12 (Q4_K), 13 (Q5_K) or 14 (Q6_K)");
        check_kquant_shape(type, n, k);
        require(gguf && packed, "null pointer");
        require(aligned(packed, 16), "packed must be 16-byte aligned");
        require(gguf != packed, "the packed copy cannot overwrite its source");
        launch_kquant_pack(type, gguf, packed, n, k, as_stream(stream));
        check_launch("hero_kquant_pack");
    });
}

int hero_kquant_gemm(int32_t type, const void* w, const void* act, float* y, int64_t m, int64_t n, int64_t k, void* stream) {
    return guard([&] {
        require(type == 12 || type == 14, "type must be 12 (Q4_K) or 14 (Q6_K)");
        check_kquant_shape(type, n, k);
        require(m > 0 && m <= (int64_t(1) << 31) / (k / 256), "m out of range");
        require(w && act && y, "null pointer");
        require(aligned(w, 16) && aligned(act, 16) && aligned(y, 4), "w and act must be 16-byte aligned");
        launch_kquant_gemm(type, w, act, y, m, n, k, as_stream(stream));
        check_launch("hero_kquant_gemm");
    });
}

int hero_q5_K_gemm(const void* w, const float* x, float* y, int64_t m, int64_t n, int64_t k, void* stream) {
    return guard([&] {
        check_kquant_shape(13, n, k);
        require(m > 0 && m <= (int64_t(1) << 31) / (k / 256), "m out of range");
        require(w && x && y, "null pointer");
        require(aligned(w, 16) && aligned(x, 16) && aligned(y, 4), "w and x must be 16-byte aligned");
        launch_q5k_gemm(w, x, k, y, nullptr, m, n, k, n, as_stream(stream));
        check_launch("hero_q5_K_gemm");
    });
}

int hero_kquant_dequant_rows(int32_t type, const void* w, int64_t n, int64_t k, const int32_t* ids, int64_t n_ids, float* out, void* stream) {
    return guard([&] {
        require(type == 12 || type == 13 || type == 14, "type must be 12 (Q4_K), 13 (Q5_K) or 14 (Q6_K)");
        check_kquant_shape(type, n, k);
        require(n_ids > 0 && n_ids <= 65535, "n_ids out of range");
        require(w && ids && out, "null pointer");
        launch_kquant_dequant_rows(type, w, n, k, ids, n_ids, out, as_stream(stream));
        check_launch("hero_kquant_dequant_rows");
    });
}

int hero_q8_0_gemv(const void* packed, const void* act, float* y, const float* residual, int64_t n, int64_t k, void* stream) {
    return guard([&] {
        check_q8_shape(n, k);
        require(packed && act && y, "null pointer");
        require(aligned(packed, 16) && aligned(act, 16), "packed and act must be 16-byte aligned");
        launch_gemv_q8(packed, act, y, residual, n, k, residual ? kEpiResidual : kEpiStore, as_stream(stream));
        check_launch("hero_q8_0_gemv");
    });
}

int hero_rmsnorm_q8_0_gemv(const void* packed, const float* x, const float* gamma, float eps, float* y, const float* residual, int64_t n, int64_t k, void* act_scratch, void* stream) {
    return guard([&] {
        check_q8_shape(n, k);
        require(packed && x && gamma && y, "null pointer");
        require(k <= 16384, "row width above 16384 is not supported");
        require(aligned(packed, 16) && aligned(x, 16) && aligned(gamma, 16), "packed, x and gamma must be 16-byte aligned");
        if (k == 4096) {
            GemvInput in{};
            in.mode = kInRmsNorm;
            in.x = x;
            in.gamma = gamma;
            in.eps = eps;
            launch_gemv_q8_in(packed, in, y, residual, n, k, residual ? kEpiResidual : kEpiStore, as_stream(stream));
        } else {
            require(act_scratch && aligned(act_scratch, 16), "act_scratch (16-byte aligned) is required when K != 4096");
            launch_rmsnorm_quant(x, gamma, eps, nullptr, act_scratch, 1, k, as_stream(stream));
            launch_gemv_q8(packed, act_scratch, y, residual, n, k, residual ? kEpiResidual : kEpiStore, as_stream(stream));
        }
        check_launch("hero_rmsnorm_q8_0_gemv");
    });
}

int hero_swiglu_q8_0_gemv(const void* packed, const float* gate_up, float* y, const float* residual, int64_t n, int64_t k, void* act_scratch, void* stream) {
    return guard([&] {
        check_q8_shape(n, k);
        require(packed && gate_up && y, "null pointer");
        require(aligned(packed, 16) && aligned(gate_up, 16), "packed and gate_up must be 16-byte aligned");
        if (gemv_streams(k)) {
            GemvInput in{};
            in.mode = kInSwiglu;
            in.gate_up = gate_up;
            launch_gemv_q8_in(packed, in, y, residual, n, k, residual ? kEpiResidual : kEpiStore, as_stream(stream));
        } else {
            require(act_scratch && aligned(act_scratch, 16), "act_scratch (16-byte aligned) is required when K is not 4096, 8192 or 12288");
            launch_swiglu_quant(gate_up, act_scratch, 1, k, as_stream(stream));
            launch_gemv_q8(packed, act_scratch, y, residual, n, k, residual ? kEpiResidual : kEpiStore, as_stream(stream));
        }
        check_launch("hero_swiglu_q8_0_gemv");
    });
}

int hero_q8_0_pack_interleaved(const void* src, void* packed, int64_t n_total, int64_t k, int64_t row0, int64_t rows, int64_t interleave, void* stream) {
    return guard([&] {
        check_q8_shape(n_total, k);
        require(src && packed, "null pointer");
        require(aligned(packed, 16), "packed buffer must be 16-byte aligned");
        require(interleave > 0 && rows > 0 && rows % interleave == 0, "rows must be a positive multiple of interleave");
        require(row0 >= 0 && row0 + (rows / interleave - 1) * 2 * interleave + interleave <= n_total, "rows outside the packed matrix");
        launch_pack_q8(src, packed, n_total, k, row0, rows, as_stream(stream), interleave);
        check_launch("hero_q8_0_pack_interleaved");
    });
}

int hero_rmsnorm_q8_0_gemv_swiglu(const void* packed, const float* x, const float* gamma, float eps, void* act_out, int64_t ff, int64_t k, void* stream) {
    return guard([&] {
        require(k == 4096, "K must be 4096");
        require(ff > 0 && ff % 32 == 0 && 2 * ff <= (int64_t(1) << 31), "ff must be a positive multiple of 32");
        require(packed && x && gamma && act_out, "null pointer");
        require(aligned(packed, 16) && aligned(x, 16) && aligned(gamma, 16) && aligned(act_out, 16), "buffers must be 16-byte aligned");
        GemvInput in{};
        in.mode = kInRmsNorm;
        in.x = x;
        in.gamma = gamma;
        in.eps = eps;
        launch_gemv_q8_in(packed, in, static_cast<float*>(act_out), nullptr, 2 * ff, k, kEpiSwigluQuant, as_stream(stream));
        check_launch("hero_rmsnorm_q8_0_gemv_swiglu");
    });
}

int hero_q8_0_gemm(const void* packed, const void* act, float* y, const float* residual, int64_t m, int64_t n, int64_t k, void* stream) {
    return guard([&] {
        check_q8_shape(n, k);
        require(m > 0 && m <= (int64_t(1) << 20), "bad row count");
        require(packed && act && y, "null pointer");
        require(aligned(packed, 16) && aligned(act, 16), "packed and act must be 16-byte aligned");
        launch_gemm_q8(packed, act, y, residual, m, n, k, residual ? kEpiResidual : kEpiStore, as_stream(stream));
        check_launch("hero_q8_0_gemm");
    });
}

int hero_q8_0_gemm_plan(int64_t m, int64_t n, int64_t k, int32_t* kernel) {
    return guard([&] {
        check_q8_shape(n, k);
        require(m > 0 && m <= (int64_t(1) << 20), "bad row count");
        require(kernel, "null pointer");
        *kernel = gemm_q8_plan(m, n, k);
    });
}

int hero_q8_0_block_sums(const void* packed, const void* act, int32_t* out, int64_t n, int64_t k, void* stream) {
    return guard([&] {
        check_q8_shape(n, k);
        require(packed && act && out, "null pointer");
        require(aligned(packed, 16) && aligned(act, 16), "packed and act must be 16-byte aligned");
        launch_block_sums(packed, act, out, n, k, as_stream(stream));
        check_launch("hero_q8_0_block_sums");
    });
}

int hero_rmsnorm_quant(const float* x, const float* gamma, float eps, float* y, void* act, int64_t m, int64_t d, void* stream) {
    return guard([&] {
        check_q8_shape(m, d);
        require(x && gamma, "null pointer");
        require(d <= 16384, "row width above 16384 is not supported");
        require(aligned(x, 16) && aligned(gamma, 16) && aligned(y, 16) && aligned(act, 16), "buffers must be 16-byte aligned");
        launch_rmsnorm_quant(x, gamma, eps, y, act, m, d, as_stream(stream));
        check_launch("hero_rmsnorm_quant");
    });
}

int hero_swiglu_quant(const float* gate_up, void* act, int64_t m, int64_t ff, void* stream) {
    return guard([&] {
        check_q8_shape(m, ff);
        require(gate_up && act, "null pointer");
        require(aligned(gate_up, 16) && aligned(act, 16), "buffers must be 16-byte aligned");
        launch_swiglu_quant(gate_up, act, m, ff, as_stream(stream));
        check_launch("hero_swiglu_quant");
    });
}

int hero_q8_0_embed(const void* packed, int64_t v, int64_t d, const int32_t* ids, int64_t n, float* out, void* stream) {
    return guard([&] {
        check_q8_shape(v, d);
        require(n > 0 && packed && ids && out, "bad arguments");
        launch_embed_q8(packed, v, d, ids, n, out, as_stream(stream));
        check_launch("hero_q8_0_embed");
    });
}

int hero_argmax(const float* logits, int64_t m, int64_t n, int32_t* out, uint64_t* scratch, void* stream) {
    return guard([&] {
        require(m > 0 && n > 0 && n < (int64_t(1) << 31), "bad shape");
        require(logits && out && scratch, "null pointer");
        launch_argmax(logits, m, n, out, scratch, as_stream(stream));
        check_launch("hero_argmax");
    });
}

int hero_argmax_noalloc(const float* logits, int64_t m, int64_t n, int32_t* out, void* stream) {
    return guard([&] {
        require(m > 0 && n > 0 && n < (int64_t(1) << 31), "bad shape");
        require(logits && out, "null pointer");
        launch_argmax_noalloc(logits, m, n, out, as_stream(stream));
        check_launch("hero_argmax_noalloc");
    });
}

int hero_math_eval(const float* x, float* out, int64_t n, void* stream) {
    return guard([&] {
        require(x && out && n > 0 && n < (int64_t(1) << 40), "bad arguments");
        launch_math_eval(x, out, n, as_stream(stream));
        check_launch("hero_math_eval");
    });
}

int hero_gemma_math_eval(const float* x, float* out, int64_t n, float cap, void* stream) {
    return guard([&] {
        require(x && out && n > 0 && n < (int64_t(1) << 40) && cap > 0.f, "bad arguments");
        launch_gemma_math_eval(x, out, n, cap, as_stream(stream));
        check_launch("hero_gemma_math_eval");
    });
}

namespace {
GdnDecodeArgs gdn_args(const hero_gdn_decode_args* p, bool need_act = true) {
    require(p != nullptr, "null args");
    const hero_gdn_decode_args& a = *p;
    require(a.dk == 128 && a.dv == 128, "delta-net heads must be 128x128");
    require(a.b > 0 && a.hk > 0 && a.hv > 0 && a.hv % a.hk == 0, "bad head counts");
    require(a.conv_width >= 1 && a.conv_width <= 8, "conv width must be 1..8");
    require(a.proj && a.conv_taps && a.conv_hist && a.state && a.dt_bias && a.decay && a.norm_gamma && a.positions && (a.act_out || !need_act), "null pointer");
    const int64_t cc = 2 * int64_t(a.hk) * 128 + int64_t(a.hv) * 128;
    require(a.proj_stride >= cc && a.z_off >= cc && a.z_off + int64_t(a.hv) * 128 <= a.proj_stride, "z slice outside the projection row");
    require(a.beta_off >= 0 && a.beta_off + a.hv <= a.proj_stride && a.alpha_off >= 0 && a.alpha_off + a.hv <= a.proj_stride, "gate slices outside the projection row");
    GdnDecodeArgs g{};
    g.proj = a.proj;
    g.proj_stride = a.proj_stride;
    g.z_off = a.z_off;
    g.beta_off = a.beta_off;
    g.alpha_off = a.alpha_off;
    g.conv_taps = a.conv_taps;
    g.conv_hist = a.conv_hist;
    g.state = a.state;
    g.dt_bias = a.dt_bias;
    g.decay = a.decay;
    g.norm_gamma = a.norm_gamma;
    g.eps = a.eps;
    g.positions = a.positions;
    g.act_out = a.act_out;
    g.out_f32 = a.out_f32;
    g.B = a.b;
    g.Hk = a.hk;
    g.Hv = a.hv;
    g.Dk = a.dk;
    g.Dv = a.dv;
    g.W = a.conv_width;
    return g;
}
}  // namespace

int hero_gdn_decode(const hero_gdn_decode_args* p, void* stream) {
    return guard([&] {
        launch_gdn_decode(gdn_args(p), as_stream(stream));
        check_launch("hero_gdn_decode");
    });
}

int hero_gdn_decode_cols(const hero_gdn_decode_args* p, float* o_raw, float* gates, void* stream) {
    return guard([&] {
        const GdnDecodeArgs a = gdn_args(p, false);
        require(o_raw != nullptr, "null pointer");
        require(aligned(a.state, 16), "state must be 16-byte aligned");
        launch_gdn_decode_cols(a, o_raw, gates, as_stream(stream));
        check_launch("hero_gdn_decode_cols");
    });
}

int hero_gdn_norm_gate(const float* o_raw, const hero_gdn_decode_args* p, void* stream) {
    return guard([&] {
        const GdnDecodeArgs a = gdn_args(p);
        require(o_raw != nullptr, "null pointer");
        launch_gdn_norm_gate(o_raw, a, as_stream(stream));
        check_launch("hero_gdn_norm_gate");
    });
}

int hero_headgate_q8_0_gemv(const void* packed, const float* o_raw, const float* gates, const float* gamma, float eps, float* y, const float* residual, int64_t n, int64_t k, void* stream) {
    return guard([&] {
        check_q8_shape(n, k);
        require(k == 4096, "the head-gated input form needs K == 4096 (32 heads of 128)");
        require(packed && o_raw && gates && gamma && y, "null pointer");
        require(aligned(packed, 16) && aligned(o_raw, 16) && aligned(gates, 16) && aligned(gamma, 16), "packed, o_raw, gates and gamma must be 16-byte aligned");
        GemvInput in{};
        in.mode = kInHeadGate;
        in.x = o_raw;
        in.z = gates;
        in.gamma = gamma;
        in.eps = eps;
        launch_gemv_q8_in(packed, in, y, residual, n, k, residual ? kEpiResidual : kEpiStore, as_stream(stream));
        check_launch("hero_headgate_q8_0_gemv");
    });
}

int64_t hero_gdn_prefill_work_bytes(int64_t t, int32_t hk, int32_t hv) {
    if (t <= 0 || hk <= 0 || hv <= 0) return -1;
    return gdn_prefill_work_bytes(t, hk, hv);
}

int hero_gdn_prefill_chunked(const hero_gdn_decode_args* p, void* work, int64_t work_bytes, void* stream) {
    return guard([&] {
        const GdnDecodeArgs g = gdn_args(p);
        require(work != nullptr && work_bytes >= gdn_prefill_work_bytes(g.B, g.Hk, g.Hv), "prefill workspace too small");
        launch_gdn_prefill(g, work, as_stream(stream), true);
        check_launch("hero_gdn_prefill_chunked");
    });
}

int hero_gdn_prefill(const hero_gdn_decode_args* p, void* work, int64_t work_bytes, void* stream) {
    return guard([&] {
        const GdnDecodeArgs g = gdn_args(p);
        require(work != nullptr && work_bytes >= gdn_prefill_work_bytes(g.B, g.Hk, g.Hv), "prefill workspace too small");
        launch_gdn_prefill(g, work, as_stream(stream));
        check_launch("hero_gdn_prefill");
    });
}

namespace {
AttnDecodeArgs attn_args(const hero_attn_decode_args& a) {
    require(a.dh == 128 || a.dh == 256, "attention head dim must be 128 or 256");
    require(a.b > 0 && a.hkv > 0 && a.hq > 0 && a.hq % a.hkv == 0, "bad head counts");
    require(a.window >= 0, "bad window");
    require(a.proj && a.q_gamma && a.k_gamma && a.rope_cs && a.positions && a.q_rot && a.act_out, "null pointer");
    const int64_t kw = int64_t(a.hkv) * 128;
    require(a.proj_stride >= 2 * int64_t(a.hq) * 128 && a.k_off + kw <= a.proj_stride && a.v_off + kw <= a.proj_stride, "k/v slices outside the projection row");
    AttnDecodeArgs g{};
    g.proj = a.proj;
    g.proj_stride = a.proj_stride;
    g.k_off = a.k_off;
    g.v_off = a.v_off;
    g.q_gamma = a.q_gamma;
    g.k_gamma = a.k_gamma;
    g.eps = a.eps;
    g.rope_cs = a.rope_cs;
    g.k_cache = a.k_cache;
    g.v_cache = a.v_cache;
    g.max_ctx = a.max_ctx;
    g.positions = a.positions;
    g.shared_cache = 0;
    g.scores = a.scores;
    g.q_rot = a.q_rot;
    g.score_scale = a.score_scale;
    g.window = a.window;
    g.act_out = a.act_out;
    g.out_f32 = a.out_f32;
    g.B = a.b;
    g.Hq = a.hq;
    g.Hkv = a.hkv;
    g.Dh = a.dh;
    return g;
}
}  // namespace

int hero_attn_decode(const hero_attn_decode_args* p, void* stream) {
    return guard([&] {
        require(p != nullptr, "null args");
        const hero_attn_decode_args& a = *p;
        require(a.k_cache && a.v_cache && a.scores, "null pointer");
        require(a.max_ctx > 0 && a.max_ctx <= (int64_t(1) << 24), "max_ctx out of range");
        launch_attn_decode(attn_args(a), as_stream(stream));
        check_launch("hero_attn_decode");
    });
}

int hero_attn_prefill(const hero_attn_decode_args* p, void* stream) {
    return guard([&] {
        require(p != nullptr, "null args");
        const hero_attn_decode_args& a = *p;
        require(a.k_cache && a.v_cache && a.scores, "null pointer");
        require(a.max_ctx > 0 && a.max_ctx <= (int64_t(1) << 24), "max_ctx out of range");
        AttnDecodeArgs g = attn_args(a);
        g.shared_cache = 1;
        launch_attn_decode(g, as_stream(stream));
        check_launch("hero_attn_prefill");
    });
}

int64_t hero_attn_paged_work_bytes(int64_t max_ctx, int32_t window, int32_t b, int32_t hq, int32_t hkv, int32_t head_dim) {
    if (max_ctx <= 0 || b <= 0 || hkv <= 0 || hq <= 0 || window < 0 || (head_dim != 128 && head_dim != 256)) return -1;
    int split = 0, nsplit = 0;
    attn_paged_plan(max_ctx, window, b, hkv, &split, &nsplit);
    return attn_paged_work_floats(b, hq, nsplit, head_dim) * 4;
}

int hero_read_probe(const void* p, int64_t bytes, int32_t workgroups, uint32_t* out, void* stream) {
    return guard([&] {
        require(p && out, "null pointer");
        require(bytes > 0 && bytes % 16 == 0 && aligned(p, 16), "bytes: a positive multiple of 16, 16-byte aligned");
        require(workgroups > 0 && workgroups <= 65536, "workgroups out of range");
        launch_read_probe(p, bytes, workgroups, out, as_stream(stream));
        check_launch("hero_read_probe");
    });
}

int hero_q8_0_gemv_prefetch(const void* packed, int64_t n, int64_t k, void* stream) {
    return guard([&] {
        require(packed && aligned(packed, 16), "packed: a 16-byte aligned device pointer");
        require(n > 0 && n <= (int64_t(1) << 24) && k == 4096, "n in 1..2^24 and k == 4096 (the interleaved GEMV form)");
        launch_gemv_prefetch(gemv_prefetch_of(packed, n, k, kEpiStore), as_stream(stream));
        check_launch("hero_q8_0_gemv_prefetch");
    });
}

int64_t hero_attn_page_bytes(int32_t hkv, int32_t head_dim, int32_t page_size, int32_t q8) {
    if (hkv <= 0 || page_size <= 0 || (q8 != 0 && q8 != 1) || (head_dim != 128 && head_dim != 256) || (q8 && head_dim != 128)) return -1;
    return attn_page_bytes(hkv, head_dim, page_size, q8 != 0);
}

int hero_attn_decode_paged(const hero_attn_paged_args* p, void* stream) {
    return guard([&] {
        require(p != nullptr, "null args");
        AttnPagedArgs g{};
        g.a = attn_args(p->a);
        require(g.a.Dh == 128 || (g.a.Dh == 256 && p->q8 == 0 && p->page_size == 64),
                "the paged cache holds 128-wide heads, or 256-wide heads in fp16 pages of 64 positions");
        require(g.a.Hq / g.a.Hkv <= kAttnMaxGroup, "at most 8 query heads per KV head");
        require(p->pages && p->page_table && p->work, "null pointer");
        require(p->page_size > 0 && p->max_pages > 0 && int64_t(p->page_size) * p->max_pages <= (int64_t(1) << 24), "bad page geometry");
        require(p->q8 == 0 || p->q8 == 1, "q8 must be 0 or 1");
        require(p->q8 == 0 || aligned(p->pages, 16), "Q8_0 pages must be 16-byte aligned");
        g.pages = p->pages;
        g.q8 = p->q8;
        g.page_table = p->page_table;
        g.page_size = p->page_size;
        g.max_pages = p->max_pages;
        attn_paged_plan(int64_t(p->page_size) * p->max_pages, g.a.window, g.a.B, g.a.Hkv, &g.split, &g.nsplit);
        require(p->work_bytes >= attn_paged_work_floats(g.a.B, g.a.Hq, g.nsplit, g.a.Dh) * 4, "split workspace too small");
        g.work = p->work;
        launch_attn_paged(g, as_stream(stream));
        check_launch("hero_attn_decode_paged");
    });
}

}  // extern "C"
