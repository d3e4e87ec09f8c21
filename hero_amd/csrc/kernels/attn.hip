// attn.hip -- gated GQA attention decode over an fp32 K/V cache, one token
// per sequence (nm/src/qwen35.hpp:343-395; the sliding-window mask of
// nm/src/attention.hpp:159-176 when window > 0).
//
// One workgroup per (sequence, query head), one lane per head channel
// (Dh = 128). The workgroup fuses: the split of the packed [q | gate] head
// pair, q RMSNorm + RoPE, the K/V head's RMSNorm + RoPE and the cache append
// (done by the first query head of each group; the others use their own,
// identical copy of the new row), the softmax reduction over the visible rows,
// the sigmoid(gate) product, and Q8_0 quantization of the head's output.
//
// The reduction keeps the reference's order: each score is a sequential
// 128-term dot (core.hpp:496-500), the softmax total is a sequential sum over
// rows (components.hpp:132-141), and each output channel accumulates
// alpha_j * v_j in row order (core.hpp:206-208). RoPE uses a host-built
// cos/sin table computed with the same float expressions as
// attention.hpp:76-91, so it is bit-identical.
#include "hero/device.hpp"
#include "hero/kernels.hpp"

namespace hero {

constexpr int kAttnDim = 128;

// RMSNorm over one head held one value per lane, then RoPE (NEOX pairs).
__device__ __forceinline__ float norm_rope_head(float x, const float* gamma, float eps, const float* cs, float* buf, float* scal, int j) {
    buf[j] = x;
    __syncthreads();
    if (j == 0) {
        float ss = 0.f;
        for (int i = 0; i < kAttnDim; ++i) ss += buf[i] * buf[i];
        scal[0] = 1.f / sqrtf(ss / float(kAttnDim) + eps);
    }
    __syncthreads();
    const float n = gamma[j] * x * scal[0];
    __syncthreads();
    buf[j] = n;
    __syncthreads();
    const int half = kAttnDim / 2;
    const int i = j < half ? j : j - half;
    const float c = cs[2 * i], s = cs[2 * i + 1];
    const float xx = buf[i], yy = buf[i + half];
    const float r = j < half ? xx * c - yy * s : yy * c + xx * s;
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(kAttnDim) void attn_decode_kernel(AttnDecodeArgs a) {
    const int j = threadIdx.x;
    const int h = blockIdx.x, b = blockIdx.y;
    const int group = a.Hq / a.Hkv;
    const int g = h / group;  // grouped K/V heads (nm/src/qwen35.hpp:369)
    const int pos = a.positions[b];
    if (pos < 0 || pos >= a.max_ctx) return;  // the host keeps positions in range; never index past the cache
    const float* P = a.proj + int64_t(b) * a.proj_stride;
    const int64_t KW = int64_t(a.Hkv) * kAttnDim;
    const float* cs = a.rope_cs + int64_t(pos) * kAttnDim;  // [Dh/2][2]

    __shared__ float buf[kAttnDim], qs_[kAttnDim], ks_[kAttnDim], vs_[kAttnDim];
    __shared__ float scal[4];

    const float q_raw = P[int64_t(h) * 2 * kAttnDim + j];
    const float gate = P[int64_t(h) * 2 * kAttnDim + kAttnDim + j];
    const float q = norm_rope_head(q_raw, a.q_gamma, a.eps, cs, buf, scal, j);
    const float k = norm_rope_head(P[a.k_off + int64_t(g) * kAttnDim + j], a.k_gamma, a.eps, cs, buf, scal, j);
    const float v = P[a.v_off + int64_t(g) * kAttnDim + j];
    qs_[j] = q;
    ks_[j] = k;
    vs_[j] = v;
    float* kc = a.k_cache + int64_t(b) * a.max_ctx * KW;
    float* vc = a.v_cache + int64_t(b) * a.max_ctx * KW;
    if (h % group == 0) {
        kc[int64_t(pos) * KW + int64_t(g) * kAttnDim + j] = k;
        vc[int64_t(pos) * KW + int64_t(g) * kAttnDim + j] = v;
    }
    __syncthreads();

    // visible rows [first, pos]
    const int first = (a.window > 0 && pos + 1 > a.window) ? pos + 1 - a.window : 0;
    const int n = pos + 1 - first;
    float* sc = a.scores + (int64_t(b) * a.Hq + h) * a.max_ctx;

    // ---- scores: scale * dot(q, k_j), one key per lane, sequential over channels
    for (int t = j; t < n; t += kAttnDim) {
        const int row = first + t;
        float dotv = 0.f;
        if (row == pos) {
            for (int c = 0; c < kAttnDim; ++c) dotv += qs_[c] * ks_[c];
        } else {
            const float4* kr = reinterpret_cast<const float4*>(kc + int64_t(row) * KW + int64_t(g) * kAttnDim);
            for (int c4 = 0; c4 < kAttnDim / 4; ++c4) {
                const float4 kk = kr[c4];
                dotv += qs_[4 * c4] * kk.x;
                dotv += qs_[4 * c4 + 1] * kk.y;
                dotv += qs_[4 * c4 + 2] * kk.z;
                dotv += qs_[4 * c4 + 3] * kk.w;
            }
        }
        sc[t] = a.score_scale * dotv;
    }
    __syncthreads();

    // ---- softmax: max (order free), exp, sequential total, divide ----
    float mx = -INFINITY;
    for (int t = j; t < n; t += kAttnDim) mx = fmaxf(mx, sc[t]);
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if ((j & 63) == 0) buf[j >> 6] = mx;
    __syncthreads();
    mx = fmaxf(buf[0], buf[1]);
    for (int t = j; t < n; t += kAttnDim) sc[t] = exp_f32(sc[t] - mx);
    __syncthreads();
    if (j == 0) {
        float total = 0.f;
        for (int t = 0; t < n; ++t) total += sc[t];
        scal[1] = total;
    }
    __syncthreads();
    const float total = scal[1];
    for (int t = j; t < n; t += kAttnDim) sc[t] = sc[t] / total;
    __syncthreads();

    // ---- out[c] = sum_j alpha_j * v_j[c], rows in order ----
    float acc = 0.f;
    for (int t = 0; t < n; ++t) {
        const int row = first + t;
        const float vv = row == pos ? vs_[j] : vc[int64_t(row) * KW + int64_t(g) * kAttnDim + j];
        acc += sc[t] * vv;
    }
    const float out = acc * sigmoid_f32(gate);  // nm/src/qwen35.hpp:390-393

    const int64_t width = int64_t(a.Hq) * kAttnDim;
    const int64_t idx = int64_t(h) * kAttnDim + j;
    if (a.out_f32) a.out_f32[int64_t(b) * width + idx] = out;
    float amax = fabsf(out);
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    const float d = amax / 127.f;
    const float id = d != 0.f ? 1.f / d : 0.f;
    int8_t* qs = static_cast<int8_t*>(a.act_out);
    float* qd = reinterpret_cast<float*>(qs + int64_t(a.B) * width);
    qs[int64_t(b) * width + idx] = int8_t(int(roundf(out * id)));
    if ((j & 31) == 0) qd[(int64_t(b) * width + idx) >> 5] = half_bits_to_f32(fp32_to_fp16_ref(d));
}

void launch_attn_decode(const AttnDecodeArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(attn_decode_kernel, dim3(unsigned(a.Hq), unsigned(a.B)), dim3(kAttnDim), 0, s, a);
}

}  // namespace hero
