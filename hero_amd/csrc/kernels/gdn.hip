// gdn.hip -- gated delta-net decode: one token per sequence, all value heads.
//
// One workgroup per (sequence, value head), one lane per value column j
// (Dk = Dv = 128). The workgroup fuses, for its head, everything between the
// input projection and the output projection (nm/src/qwen35.hpp:420-462):
//   causal conv step + SiLU on its q, k, v channels (recurrent.hpp:75-106),
//   L2 normalisation of q and k and the 1/sqrt(Dk) query scale (:441-446),
//   beta = sigmoid, g = A*softplus(alpha + dt) (:400-415),
//   the gated delta rule (recurrent.hpp:146-177) with the head's 128x128
//   fp32 state column held in the lane's registers across both passes,
//   the per-head RMSNorm, the SiLU(z) gate, and Q8_0 quantization of the
//   head's 128 outputs (4 blocks) for the output projection.
// Every fp32 reduction runs in the reference's order (sequential chains).
//
// Conv history is a ring of W slots per channel: slot p % W holds the input
// at position p. A step at position p reads positions p-W+1 .. p-1 and writes
// slot p % W, which no reader of this step touches; unwritten slots are the
// causal zero padding.
#include "hero/device.hpp"
#include "hero/kernels.hpp"

namespace hero {

constexpr int kGdnDim = 128;

// sequential sum of squares of v[0..128) (nm/src/core.hpp:496-500 order),
// reading shared memory four values at a time
__device__ __forceinline__ float sum_squares_128(const float* v) {
    const float4* v4 = reinterpret_cast<const float4*>(v);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kGdnDim / 4; ++i) {
        const float4 x = v4[i];
        ss += x.x * x.x;
        ss += x.y * x.y;
        ss += x.z * x.z;
        ss += x.w * x.w;
    }
    return ss;
}

__device__ __forceinline__ float conv_channel(const GdnDecodeArgs& a, const float* hist, int64_t CC, int64_t c, int pos, float x) {
    const float* taps = a.conv_taps + c * a.W;
    float sum = taps[a.W - 1] * x;
    for (int i = 0; i < a.W - 1; ++i) {
        const int p = pos - (a.W - 1) + i;  // oldest first
        const int slot = ((p % a.W) + a.W) % a.W;
        sum += taps[i] * hist[int64_t(slot) * CC + c];
    }
    return sum;
}

__global__ __launch_bounds__(kGdnDim) void gdn_decode_kernel(GdnDecodeArgs a) {
    const int j = threadIdx.x;
    const int h = blockIdx.x, b = blockIdx.y;
    const int hk = h % a.Hk;  // tiled key heads (nm/src/qwen35.hpp:172)
    const int pos = a.positions[b];
    if (pos < 0) return;  // the host keeps positions in range
    const int64_t KW = int64_t(a.Hk) * kGdnDim;
    const int64_t CC = 2 * KW + int64_t(a.Hv) * kGdnDim;
    const float* P = a.proj + int64_t(b) * a.proj_stride;
    float* hist = a.conv_hist + int64_t(b) * a.W * CC;

    __shared__ __align__(16) float qv[kGdnDim], kv[kGdnDim], ov[kGdnDim];
    __shared__ float scal[4];

    // ---- conv + SiLU on this head's channels ----
    const int64_t cq = int64_t(hk) * kGdnDim + j, ck = KW + int64_t(hk) * kGdnDim + j, cv = 2 * KW + int64_t(h) * kGdnDim + j;
    const float xq = P[cq], xk = P[ck], xv = P[cv];
    const float sq = silu_f32(conv_channel(a, hist, CC, cq, pos, xq));
    const float sk = silu_f32(conv_channel(a, hist, CC, ck, pos, xk));
    const float v = silu_f32(conv_channel(a, hist, CC, cv, pos, xv));
    const int slot = pos % a.W;
    if (h < a.Hk) {  // the first value head of each key head owns its q/k history
        hist[int64_t(slot) * CC + cq] = xq;
        hist[int64_t(slot) * CC + ck] = xk;
    }
    hist[int64_t(slot) * CC + cv] = xv;
    qv[j] = sq;
    kv[j] = sk;
    __syncthreads();

    // ---- L2 norms (nm/src/recurrent.hpp:40-48), sequential sums ----
    if (j == 0 || j == 64) {
        const float ss = sum_squares_128(j == 0 ? qv : kv);
        scal[j == 0 ? 0 : 1] = 1.f / fmaxf(sqrtf(ss), 1e-6f);
    }
    __syncthreads();
    const float query_scale = 1.f / sqrtf(float(kGdnDim));
    const float qn = (sq * scal[0]) * query_scale;
    const float kn = sk * scal[1];
    __syncthreads();
    qv[j] = qn;
    kv[j] = kn;
    __syncthreads();

    // ---- beta and the decay gate ----
    const float beta = sigmoid_f32(P[a.beta_off + h]);
    const float g = a.decay[h] * softplus_f32(P[a.alpha_off + h] + a.dt_bias[h]);
    const float decay = exp_f32(g);

    // ---- the delta rule on column j ----
    float* S = a.state + (int64_t(b) * a.Hv + h) * kGdnDim * kGdnDim + j;
    float col[kGdnDim];
#pragma unroll
    for (int i = 0; i < kGdnDim; ++i) col[i] = S[int64_t(i) * kGdnDim];
    float pred = 0.f;
#pragma unroll
    for (int i = 0; i < kGdnDim; ++i) {
        col[i] = col[i] * decay;
        pred = pred + col[i] * kv[i];
    }
    const float delta = (v - pred) * beta;
    float o = 0.f;
#pragma unroll
    for (int i = 0; i < kGdnDim; ++i) {
        col[i] = col[i] + kv[i] * delta;
        o = o + col[i] * qv[i];
    }
#pragma unroll
    for (int i = 0; i < kGdnDim; ++i) S[int64_t(i) * kGdnDim] = col[i];

    // ---- per-head RMSNorm (components.hpp:176-181) and the SiLU(z) gate ----
    ov[j] = o;
    __syncthreads();
    if (j == 0) scal[2] = 1.f / sqrtf(sum_squares_128(ov) / float(kGdnDim) + a.eps);
    __syncthreads();
    const float normed = a.norm_gamma[j] * o * scal[2];
    const float z = P[a.z_off + int64_t(h) * kGdnDim + j];
    const float out = normed * silu_f32(z);
    const int64_t width = int64_t(a.Hv) * kGdnDim;
    const int64_t idx = int64_t(h) * kGdnDim + j;
    if (a.out_f32) a.out_f32[int64_t(b) * width + idx] = out;

    // ---- Q8_0 quantization, 32 lanes per block (quant_i8.hpp:70-80) ----
    float amax = fabsf(out);
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    const float d = amax / 127.f;
    const float id = d != 0.f ? 1.f / d : 0.f;
    int8_t* qs = static_cast<int8_t*>(a.act_out);
    float* qd = reinterpret_cast<float*>(qs + int64_t(a.B) * width);
    qs[int64_t(b) * width + idx] = int8_t(int(roundf(out * id)));
    if ((j & 31) == 0) qd[(int64_t(b) * width + idx) >> 5] = half_bits_to_f32(fp32_to_fp16_ref(d));
}

void launch_gdn_decode(const GdnDecodeArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(gdn_decode_kernel, dim3(unsigned(a.Hv), unsigned(a.B)), dim3(kGdnDim), 0, s, a);
}

}  // namespace hero
