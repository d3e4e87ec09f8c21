// gemma.hip -- the kernels of the Gemma 4 text model's decode step that the
// Qwen path does not have: the scaled embedding and per-layer inputs (PLE),
// the per-head norms with RoPE and the cache append, GQA attention with score
// scale 1 over a full or a sliding-window (ring) cache, the post-norm +
// residual + next norm step that closes every sub-block, the GELU-gated
// products and the logit soft-cap.
//
// Every fp32 expression follows the reference's operation order (see the
// comment of each kernel); sums the reference forms sequentially are summed
// exactly that way (hero/seqsum.hpp), tanh and exp are glibc's (hero/libm.hpp).
#include "hero/device.hpp"
#include "hero/kernels.hpp"
#include "hero/seqsum.hpp"

namespace hero {

// gelu_pytorch_tanh (nm/src/components.hpp:73-81):
// 0.5 v (1 + tanh(0.7978845608 (v + 0.044715 v^3))), left to right
__device__ __forceinline__ float gelu_tanh_f32(float v) {
    return 0.5f * v * (1.f + tanhf_glibc(0.7978845608f * (v + 0.044715f * v * v * v)));
}

// ---- embedding and per-layer inputs -----------------------------------------------
// x = dequant_row(id) * embed_scale (Gemma4E4BModel::embed, nm/src/gemma4.hpp:415-419),
// its Q8_0 quantization (the PLE projection's input), and the token part of
// the per-layer inputs tok = dequant_row(id) * token_scale of the packed table
// (GemmaPerLayerInputs, nm/src/gemma4.hpp:129-131). A lane per 8 values; the
// quads of x are whole Q8_0 blocks.
__global__ __launch_bounds__(256) void gemma_embed_kernel(const int8_t* __restrict__ eq, const uint16_t* __restrict__ ed, int64_t D, const int8_t* __restrict__ pq,
                                                          const uint16_t* __restrict__ pd, int64_t PL, const int32_t* __restrict__ id_ptr, float embed_scale,
                                                          float token_scale, float* __restrict__ x, int8_t* __restrict__ xq, float* __restrict__ xd,
                                                          float* __restrict__ tok) {
    const int64_t lane = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t id = *id_ptr;
    const int64_t gx = D / 8;
    if (lane < gx) {
        const int64_t c0 = lane * 8;
        const float d = half_bits_to_f32(ed[scale_index(id, c0 >> 5, D >> 5)]);
        const int2 q = reinterpret_cast<const int2*>(eq + id * D)[lane];
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int8_t b = int8_t(((k < 4 ? q.x : q.y) >> (8 * (k & 3))) & 0xFF);
            v[k] = d * float(b) * embed_scale;
        }
        reinterpret_cast<float4*>(x + c0)[0] = make_float4(v[0], v[1], v[2], v[3]);
        reinterpret_cast<float4*>(x + c0)[1] = make_float4(v[4], v[5], v[6], v[7]);
        uint16_t dh;
        reinterpret_cast<int2*>(xq)[lane] = quantize8_in_quad(v, &dh);
        if ((lane & 3) == 0) xd[lane >> 2] = half_bits_to_f32(dh);
        return;
    }
    const int64_t t = lane - gx;
    if (t >= PL / 8) return;
    const int64_t c0 = t * 8;
    const float d = half_bits_to_f32(pd[scale_index(id, c0 >> 5, PL >> 5)]);
    const int2 q = reinterpret_cast<const int2*>(pq + id * PL)[t];
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int8_t b = int8_t(((k < 4 ? q.x : q.y) >> (8 * (k & 3))) & 0xFF);
        v[k] = d * float(b) * token_scale;
    }
    reinterpret_cast<float4*>(tok + c0)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(tok + c0)[1] = make_float4(v[4], v[5], v[6], v[7]);
}

void launch_gemma_embed(const void* emb, int64_t V, int64_t D, const void* ple_table, int64_t PL, const int32_t* id, float embed_scale, float token_scale, float* x,
                        void* act, float* tok, hipStream_t s) {
    const int8_t* eq = static_cast<const int8_t*>(emb);
    const int8_t* pq = static_cast<const int8_t*>(ple_table);
    int8_t* xq = static_cast<int8_t*>(act);
    const int64_t lanes = D / 8 + PL / 8;
    hipLaunchKernelGGL(gemma_embed_kernel, dim3(unsigned((lanes + 255) / 256)), dim3(256), 0, s, eq, reinterpret_cast<const uint16_t*>(eq + V * D), D, pq,
                       reinterpret_cast<const uint16_t*>(pq + V * PL), PL, id, embed_scale, token_scale, x, xq, reinterpret_cast<float*>(xq + D), tok);
}

// The per-layer inputs of one row (GemmaPerLayerInputs, nm/src/gemma4.hpp:127-135):
// c = ctx * proj_scale; c = RMSNorm_P(c) with the shared weight, per layer
// slice; ple = (c + tok) * comb (scaled_sum, core.hpp:509-513). A workgroup of
// 256 lanes per layer slice of P values.
__global__ __launch_bounds__(256) void gemma_ple_kernel(const float* __restrict__ ctx, const float* __restrict__ tok, const float* __restrict__ gamma, float eps,
                                                        float proj_scale, float comb, float* __restrict__ ple, int P) {
    constexpr int NT = 256;
    __shared__ seqsum::Shared sm;
    __shared__ __align__(16) float sq[seqsum::kMaxN];
    const int64_t base = int64_t(blockIdx.x) * P;
    const int tid = threadIdx.x;
    for (int i = tid; i < seqsum::kMaxN; i += NT) {
        float v = 0.f;
        if (i < P) {
            const float c = ctx[base + i] * proj_scale;
            v = c * c;
        }
        sq[i] = v;
    }
    __syncthreads();
    const float s = seqsum::sum_nonneg<NT>(sq, P, sm);
    const float inv = 1.f / sqrtf(s / float(P) + eps);
    for (int i = tid; i < P; i += NT) {
        const float c = ctx[base + i] * proj_scale;
        const float n = gamma[i] * c * inv;
        ple[base + i] = (n + tok[base + i]) * comb;
    }
}

void launch_gemma_ple_inputs(const float* ctx, const float* tok, const float* gamma, float eps, float proj_scale, float comb, float* ple, int64_t L, int64_t P,
                             hipStream_t s) {
    hipLaunchKernelGGL(gemma_ple_kernel, dim3(unsigned(L)), dim3(256), 0, s, ctx, tok, gamma, eps, proj_scale, comb, ple, int(P));
}

// ---- attention -----------------------------------------------------------------------
__device__ __forceinline__ int64_t gemma_slot(const GemmaAttnArgs& a, int64_t pos) { return a.window > 0 ? pos % a.slots : pos; }

// One head of DH values, a lane per value: x (RMSNorm over the head: the
// learned weight gamma, or none for V), then RoPE on the planes (i, i + DH/2)
// with the position's (cos, sin) table row (RotaryEmbedding,
// nm/src/attention.hpp:82-91; unrotated planes carry (1, 0)).
// PerHeadNorm (components.hpp:248-258) with RMSNorm (:176-181) or RMSNormNoScale (:210-215).
template <int DH>
__device__ __forceinline__ float gemma_head_norm(float x, const float* gamma, float eps, float* sq, seqsum::Shared& sm) {
    const int j = threadIdx.x;
    for (int i = j; i < seqsum::kMaxN; i += DH) sq[i] = i == j ? x * x : 0.f;
    __syncthreads();
    const float s = seqsum::sum_nonneg<DH>(sq, DH, sm);
    const float inv = 1.f / sqrtf(s / float(DH) + eps);
    return gamma ? gamma[j] * x * inv : x * inv;
}

template <int DH>
__device__ __forceinline__ float gemma_rope(float n, const float* cs, float* buf) {
    const int j = threadIdx.x;
    __syncthreads();  // buf free
    buf[j] = n;
    __syncthreads();
    constexpr int half = DH / 2;
    const int i = j < half ? j : j - half;
    const float c = cs[2 * i], sn = cs[2 * i + 1];
    const float xx = buf[i], yy = buf[i + half];
    return j < half ? xx * c - yy * sn : yy * c + xx * sn;
}

// Workgroups [0, Hq): query head h -> q_rot; with append, [Hq, Hq + Hkv): key
// head g -> K cache; [Hq + Hkv, Hq + 2 Hkv): value head g -> V cache, at the
// position's slot. Q = rope(q_norm(WQ x)), K = rope(k_norm(WK x)),
// V = v_norm(WV x) (GemmaE4BLayer::attention, nm/src/gemma4.hpp:205-208).
template <int DH>
__global__ __launch_bounds__(DH) void gemma_attn_prep_kernel(GemmaAttnArgs a) {
    __shared__ seqsum::Shared sm;
    __shared__ __align__(16) float sq[seqsum::kMaxN];
    __shared__ float buf[DH];
    const int j = threadIdx.x, blk = blockIdx.x;
    const int64_t pos = *a.pos;
    const float* cs = a.rope_cs + pos * DH;  // [DH/2][2]
    if (blk < a.Hq) {
        const float n = gemma_head_norm<DH>(a.proj[int64_t(blk) * DH + j], a.q_gamma, a.eps, sq, sm);
        a.q_rot[int64_t(blk) * DH + j] = gemma_rope<DH>(n, cs, buf);
        return;
    }
    const int64_t slot = gemma_slot(a, pos);
    const int g = blk - a.Hq;
    if (g < a.Hkv) {
        const float n = gemma_head_norm<DH>(a.proj[a.k_off + int64_t(g) * DH + j], a.k_gamma, a.eps, sq, sm);
        a.k_cache[(int64_t(g) * DH + j) * a.slots + slot] = gemma_rope<DH>(n, cs, buf);  // [Hkv][DH][slots]
        return;
    }
    const int gv = g - a.Hkv;
    const float n = gemma_head_norm<DH>(a.proj[a.v_off + int64_t(gv) * DH + j], nullptr, a.eps, sq, sm);
    a.v_cache[(int64_t(gv) * a.slots + slot) * DH + j] = n;  // [Hkv][slots][DH]
}

// One query head per workgroup of DH lanes (Gemma's reduction,
// nm/src/gemma4.hpp:210-230: no score scale):
//   s_t = dot(q, k_t) over the visible positions, each the sequential DH-term sum;
//   alpha = softmax(s) (components.hpp:131-141: e_t = exp(s_t - max), their
//   sequential sum, e_t / total);
//   out[c] = sum_t alpha_t v_t[c], t in order (Vec::scaled_add, core.hpp:206-208);
// then the head's Q8_0 blocks of the W_o input.
template <int DH>
__global__ __launch_bounds__(DH) void gemma_attn_kernel(GemmaAttnArgs a) {
    __shared__ seqsum::Shared sm;
    __shared__ __align__(16) float chunk[seqsum::kMaxN];
    __shared__ __align__(16) float q[DH];
    __shared__ float red[DH / 64];
    const int j = threadIdx.x, h = blockIdx.x;
    const int g = h / (a.Hq / a.Hkv);  // adjacent query heads share a K/V head
    const int64_t pos = *a.pos;
    const int64_t first = (a.window > 0 && pos + 1 > a.window) ? pos + 1 - a.window : 0;
    const int64_t n = pos + 1 - first;
    q[j] = a.q_rot[int64_t(h) * DH + j];
    __syncthreads();
    const float* kh = a.k_cache + int64_t(g) * DH * a.slots;
    const float* vh = a.v_cache + int64_t(g) * a.slots * DH;
    float* sc = a.scores + int64_t(h) * a.max_ctx;
    float mx = -INFINITY;
    for (int64_t t = j; t < n; t += DH) {
        const int64_t slot = gemma_slot(a, first + t);
        float dot = 0.f;
#pragma unroll 8
        for (int c = 0; c < DH; ++c) dot += q[c] * kh[int64_t(c) * a.slots + slot];
        sc[t] = dot;
        mx = fmaxf(mx, dot);
    }
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if ((j & 63) == 0) red[j >> 6] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < DH / 64; ++w) mx = fmaxf(mx, red[w]);
    // exponentials and their sequential sum, chunk by chunk, each chunk
    // starting with the running total (fl(0 + e) == e: the first chunk is the
    // loop from 0). Chunks start at multiples of DH, so lane j handles the
    // positions t == j (mod DH) throughout: the scores it wrote itself.
    constexpr int CH = seqsum::kMaxN - DH;
    float total = 0.f;
    for (int64_t base = 0; base < n; base += CH) {
        const int len = int(min<int64_t>(n - base, CH));
        __syncthreads();  // chunk free
        for (int u = j; u < seqsum::kMaxN; u += DH) chunk[u] = 0.f;
        __syncthreads();
        for (int u = j; u < len; u += DH) {
            const float e = exp_f32(sc[base + u] - mx);
            sc[base + u] = e;
            chunk[1 + u] = e;
        }
        if (j == 0) chunk[0] = total;
        __syncthreads();
        total = seqsum::sum_nonneg<DH>(chunk, len + 1, sm);
    }
    // alpha_t = e_t / total, staged in shared memory chunk by chunk (again by
    // the lanes that own them), and the weighted sum of the value rows
    float acc = 0.f;
    for (int64_t base = 0; base < n; base += seqsum::kMaxN) {
        const int len = int(min<int64_t>(n - base, seqsum::kMaxN));
        __syncthreads();
        for (int u = j; u < len; u += DH) chunk[u] = sc[base + u] / total;
        __syncthreads();
        for (int u = 0; u < len; ++u) {
            const int64_t slot = gemma_slot(a, first + base + u);
            acc += chunk[u] * vh[slot * DH + j];
        }
    }
    // the W_o input: this head's DH / 32 Q8_0 blocks
    __syncthreads();
    chunk[j] = acc;
    __syncthreads();
    if (j < DH / 8) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = chunk[8 * j + k];
        uint16_t dh;
        int8_t* qs = static_cast<int8_t*>(a.act_out);
        float* qd = reinterpret_cast<float*>(qs + int64_t(a.Hq) * DH);
        reinterpret_cast<int2*>(qs + int64_t(h) * DH)[j] = quantize8_in_quad(v, &dh);
        if ((j & 3) == 0) qd[int64_t(h) * (DH / 32) + (j >> 2)] = half_bits_to_f32(dh);
    }
}

void launch_gemma_attention(const GemmaAttnArgs& a, hipStream_t s) {
    const unsigned prep = unsigned(a.Hq + (a.append ? 2 * a.Hkv : 0));
    if (a.Dh == 256) {
        hipLaunchKernelGGL(gemma_attn_prep_kernel<256>, dim3(prep), dim3(256), 0, s, a);
        hipLaunchKernelGGL(gemma_attn_kernel<256>, dim3(unsigned(a.Hq)), dim3(256), 0, s, a);
    } else {
        hipLaunchKernelGGL(gemma_attn_prep_kernel<512>, dim3(prep), dim3(512), 0, s, a);
        hipLaunchKernelGGL(gemma_attn_kernel<512>, dim3(unsigned(a.Hq)), dim3(512), 0, s, a);
    }
}

// ---- the end of a sub-block ------------------------------------------------------------
// out = (RMSNorm(a) * gamma + res) * scale, then the Q8_0 act of next_gamma ?
// RMSNorm(out) * next_gamma : out. The forms of GemmaE4BLayer::forward
// (nm/src/gemma4.hpp:258-272): H = X + post_attn_norm(attn) and
// H = H + post_ffn_norm(ffn) (scale 1: an exact identity), then the PLE
// residual branch + hidden (:102-104) times layer_output_scale; the next
// norm is the following block's pre-norm (or the final norm). 512 lanes, 8
// values each (D <= 4096, D % 32 == 0).
constexpr int kPostThreads = 512;

__global__ __launch_bounds__(kPostThreads) void gemma_post_norm_kernel(const float* __restrict__ a, const float* __restrict__ gamma, const float* __restrict__ res, float scale,
                                                                       float eps, float* __restrict__ out, const float* __restrict__ next_gamma, int8_t* __restrict__ qs,
                                                                       float* __restrict__ qd, int D) {
    constexpr int PT = seqsum::kMaxN / kPostThreads;  // 8
    __shared__ seqsum::Shared sm;
    __shared__ __align__(16) float sq[seqsum::kMaxN];
    const int tid = threadIdx.x, i0 = tid * PT;
    const bool on = i0 < D;
    float v[PT], s2[PT];
    if (on) {
        const float4 x0 = reinterpret_cast<const float4*>(a + i0)[0];
        const float4 x1 = reinterpret_cast<const float4*>(a + i0)[1];
        v[0] = x0.x, v[1] = x0.y, v[2] = x0.z, v[3] = x0.w, v[4] = x1.x, v[5] = x1.y, v[6] = x1.z, v[7] = x1.w;
    } else {
#pragma unroll
        for (int k = 0; k < PT; ++k) v[k] = 0.f;
    }
#pragma unroll
    for (int k = 0; k < PT; ++k) s2[k] = v[k] * v[k];
    const float s = seqsum::sum_nonneg_regs<kPostThreads>(s2, sq, D, sm);
    const float inv = 1.f / sqrtf(s / float(D) + eps);
    float o[PT];
    if (on) {
#pragma unroll
        for (int k = 0; k < PT; ++k) o[k] = (gamma[i0 + k] * v[k] * inv + res[i0 + k]) * scale;
        reinterpret_cast<float4*>(out + i0)[0] = make_float4(o[0], o[1], o[2], o[3]);
        reinterpret_cast<float4*>(out + i0)[1] = make_float4(o[4], o[5], o[6], o[7]);
    } else {
#pragma unroll
        for (int k = 0; k < PT; ++k) o[k] = 0.f;
    }
    if (next_gamma) {
#pragma unroll
        for (int k = 0; k < PT; ++k) s2[k] = o[k] * o[k];
        __syncthreads();  // the first sum's readers of sq and sm are done
        const float s_2 = seqsum::sum_nonneg_regs<kPostThreads>(s2, sq, D, sm);
        const float inv2 = 1.f / sqrtf(s_2 / float(D) + eps);
        if (on) {
#pragma unroll
            for (int k = 0; k < PT; ++k) o[k] = next_gamma[i0 + k] * o[k] * inv2;
        }
    }
    if (!on) return;
    uint16_t dh;
    reinterpret_cast<int2*>(qs)[tid] = quantize8_in_quad(o, &dh);
    if ((tid & 3) == 0) qd[tid >> 2] = half_bits_to_f32(dh);
}

void launch_gemma_post_norm(const float* a, const float* gamma, const float* res, float scale, float eps, float* out, const float* next_gamma, void* act, int64_t D,
                            hipStream_t s) {
    int8_t* qs = static_cast<int8_t*>(act);
    hipLaunchKernelGGL(gemma_post_norm_kernel, dim3(1), dim3(kPostThreads), 0, s, a, gamma, res, scale, eps, out, next_gamma, qs, reinterpret_cast<float*>(qs + D), int(D));
}

// ---- GELU-gated products --------------------------------------------------------------
// act = Q8_0 of gelu(gate[i]) * mul[i]: the GELU-gated MLP's down input
// (GatedMLP, components.hpp:294-299: g = gelu(gate(x)); g *= up(x)) and the
// PLE branch input (gemma4.hpp:100-101: hadamard(gelu(gate(h)), ple)).
// A lane per 8 values (N % 32 == 0).
__global__ __launch_bounds__(256) void gemma_gelu_mul_quant_kernel(const float* __restrict__ gate, const float* __restrict__ mul, int8_t* __restrict__ qs,
                                                                   float* __restrict__ qd, int64_t N) {
    const int64_t lane = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (lane >= N / 8) return;  // whole quads
    const float4 g0 = reinterpret_cast<const float4*>(gate)[2 * lane], g1 = reinterpret_cast<const float4*>(gate)[2 * lane + 1];
    const float4 m0 = reinterpret_cast<const float4*>(mul)[2 * lane], m1 = reinterpret_cast<const float4*>(mul)[2 * lane + 1];
    const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    const float m[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = gelu_tanh_f32(g[k]) * m[k];
    uint16_t dh;
    reinterpret_cast<int2*>(qs)[lane] = quantize8_in_quad(v, &dh);
    if ((lane & 3) == 0) qd[lane >> 2] = half_bits_to_f32(dh);
}

void launch_gemma_gelu_mul_quant(const float* gate, const float* mul, void* act, int64_t N, hipStream_t s) {
    int8_t* qs = static_cast<int8_t*>(act);
    hipLaunchKernelGGL(gemma_gelu_mul_quant_kernel, dim3(unsigned((N / 8 + 255) / 256)), dim3(256), 0, s, gate, mul, qs, reinterpret_cast<float*>(qs + N), N);
}

// ---- the logit soft-cap ---------------------------------------------------------------
// cap * tanh(v / cap) (gemma_softcap, nm/src/gemma4.hpp:79)
__global__ __launch_bounds__(256) void gemma_softcap_kernel(float* __restrict__ logits, int64_t n, float cap) {
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) logits[i] = cap * tanhf_glibc(logits[i] / cap);
}

void launch_gemma_softcap(float* logits, int64_t n, float cap, hipStream_t s) {
    hipLaunchKernelGGL(gemma_softcap_kernel, dim3(unsigned(std::min<int64_t>(1024, (n + 255) / 256))), dim3(256), 0, s, logits, n, cap);
}

// host-callable evaluation of the device GELU and soft-cap (tests)
__global__ void gemma_math_eval_kernel(const float* __restrict__ x, float* __restrict__ out, int64_t n, float cap) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    out[2 * i] = gelu_tanh_f32(x[i]);
    out[2 * i + 1] = cap * tanhf_glibc(x[i] / cap);
}

void launch_gemma_math_eval(const float* x, float* out, int64_t n, float cap, hipStream_t s) {
    hipLaunchKernelGGL(gemma_math_eval_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, s, x, out, n, cap);
}

}  // namespace hero
