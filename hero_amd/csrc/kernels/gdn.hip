// gdn.hip -- gated delta-net decode: one token per sequence, all value heads.
//
// One workgroup per (sequence, value head), one lane per value column j
// (Dk = Dv = 128). The workgroup fuses, for its head, everything between the
// input projection and the output projection (nm/src/qwen35.hpp:420-462):
//   causal conv step + SiLU on its q, k, v channels (recurrent.hpp:75-106),
//   L2 normalisation of q and k and the 1/sqrt(Dk) query scale (:441-446),
//   beta = sigmoid, g = A*softplus(alpha + dt) (:400-415),
//   the gated delta rule (recurrent.hpp:146-177) with the head's 128x128
//   fp32 state staged in shared memory (16-byte coalesced loads and stores,
//   all global reads issued before any compute),
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

// sequential sum of squares of v[0..128) (nm/src/core.hpp:496-500 order):
// all 128 values are read from shared memory first, then the chain of adds
__device__ __forceinline__ float sum_squares_128(const float* v) {
    const float4* v4 = reinterpret_cast<const float4*>(v);
    float4 x[kGdnDim / 4];
#pragma unroll
    for (int i = 0; i < kGdnDim / 4; ++i) x[i] = v4[i];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kGdnDim / 4; ++i) {
        ss += x[i].x * x[i].x;
        ss += x[i].y * x[i].y;
        ss += x[i].z * x[i].z;
        ss += x[i].w * x[i].w;
    }
    return ss;
}

// Causal conv of one channel (nm/src/recurrent.hpp:75-106): sum = taps[W-1]*x,
// then += taps[i] * (input at position p-(W-1)+i), oldest first. The history
// and taps were loaded by the caller.
template <int W>
__device__ __forceinline__ float conv_channel(const float (&taps)[W], const float (&past)[W > 1 ? W - 1 : 1], float x) {
    float sum = taps[W - 1] * x;
#pragma unroll
    for (int i = 0; i < W - 1; ++i) sum += taps[i] * past[i];
    return sum;
}

template <int W>
__device__ __forceinline__ void load_conv(const float* taps_row, const float* hist, int64_t CC, int64_t c, int pos, float (&taps)[W], float (&past)[W > 1 ? W - 1 : 1]) {
#pragma unroll
    for (int i = 0; i < W; ++i) taps[i] = taps_row[c * W + i];
#pragma unroll
    for (int i = 0; i < W - 1; ++i) {
        const int p = pos - (W - 1) + i;  // oldest first; slots of p < 0 were never written (zero)
        const int slot = ((p % W) + W) % W;
        past[i] = hist[int64_t(slot) * CC + c];
    }
}

// Layout of the dynamic shared memory: the head's state [Dk][Dv] (64 KB), then
// q, k, the head output (128 each) and a few scalars.
constexpr int kGdnState = kGdnDim * kGdnDim;

template <int W>
__global__ __launch_bounds__(kGdnDim) void gdn_decode_kernel(GdnDecodeArgs a) {
    extern __shared__ __align__(16) float sh[];
    float* Ssh = sh;                  // [i][j] = state row i (key), column j (value)
    float* qv = sh + kGdnState;       // [128]
    float* kv = qv + kGdnDim;         // [128]
    float* ov = kv + kGdnDim;         // [128]
    float* scal = ov + kGdnDim;       // [4]
    const int j = threadIdx.x;
    const int h = blockIdx.x, b = blockIdx.y;
    const int hk = h % a.Hk;  // tiled key heads (nm/src/qwen35.hpp:172)
    const int pos = a.positions[b];
    if (pos < 0) return;  // the host keeps positions in range
    const int64_t KW = int64_t(a.Hk) * kGdnDim;
    const int64_t CC = 2 * KW + int64_t(a.Hv) * kGdnDim;
    const float* P = a.proj + int64_t(b) * a.proj_stride;
    float* hist = a.conv_hist + int64_t(b) * W * CC;
    float* S = a.state + (int64_t(b) * a.Hv + h) * kGdnState;

    // ---- every global read first, so their latencies overlap ----
    constexpr int kVec = kGdnState / 4 / kGdnDim;  // 32 x 16 bytes per lane, coalesced
    float4 sv[kVec];
#pragma unroll
    for (int k = 0; k < kVec; ++k) sv[k] = reinterpret_cast<const float4*>(S)[j + kGdnDim * k];
    const int64_t cq = int64_t(hk) * kGdnDim + j, ck = KW + int64_t(hk) * kGdnDim + j, cv = 2 * KW + int64_t(h) * kGdnDim + j;
    const float xq = P[cq], xk = P[ck], xv = P[cv];
    float tq[W], tk[W], tv[W], pq[W > 1 ? W - 1 : 1], pk[W > 1 ? W - 1 : 1], pv[W > 1 ? W - 1 : 1];
    load_conv<W>(a.conv_taps, hist, CC, cq, pos, tq, pq);
    load_conv<W>(a.conv_taps, hist, CC, ck, pos, tk, pk);
    load_conv<W>(a.conv_taps, hist, CC, cv, pos, tv, pv);
    const float z = P[a.z_off + int64_t(h) * kGdnDim + j];
    const float gamma = a.norm_gamma[j];
    const float beta_in = P[a.beta_off + h], alpha_in = P[a.alpha_off + h];
    const float A = a.decay[h], dtb = a.dt_bias[h];
#pragma unroll
    for (int k = 0; k < kVec; ++k) reinterpret_cast<float4*>(Ssh)[j + kGdnDim * k] = sv[k];

    // ---- conv + SiLU on this head's channels ----
    const float sq = silu_f32(conv_channel<W>(tq, pq, xq));
    const float sk = silu_f32(conv_channel<W>(tk, pk, xk));
    const float v = silu_f32(conv_channel<W>(tv, pv, xv));
    const int slot = pos % W;
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
    const float beta = sigmoid_f32(beta_in);
    const float g = A * softplus_f32(alpha_in + dtb);
    const float decay = exp_f32(g);

    // ---- the delta rule on column j (recurrent.hpp:146-177) ----
    // The column is read from shared memory into registers once; the k and q
    // vectors are read 32 at a time ahead of the chains.
    float col[kGdnDim];
#pragma unroll
    for (int i = 0; i < kGdnDim; ++i) col[i] = Ssh[i * kGdnDim + j] * decay;  // pass 1: S[i][j] *= decay
    float pred = 0.f;
#pragma unroll
    for (int i0 = 0; i0 < kGdnDim; i0 += 32) {
        float4 k4[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) k4[u] = *reinterpret_cast<const float4*>(kv + i0 + 4 * u);
#pragma unroll
        for (int u = 0; u < 8; ++u) {  // pred += S[i][j] * k[i]
            pred = pred + col[i0 + 4 * u + 0] * k4[u].x;
            pred = pred + col[i0 + 4 * u + 1] * k4[u].y;
            pred = pred + col[i0 + 4 * u + 2] * k4[u].z;
            pred = pred + col[i0 + 4 * u + 3] * k4[u].w;
        }
    }
    const float delta = (v - pred) * beta;
    // pass 2: S[i][j] += k[i] * delta; o += S[i][j] * q[i]
    float o = 0.f;
#pragma unroll
    for (int i0 = 0; i0 < kGdnDim; i0 += 32) {
        float4 k4[8], q4[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            k4[u] = *reinterpret_cast<const float4*>(kv + i0 + 4 * u);
            q4[u] = *reinterpret_cast<const float4*>(qv + i0 + 4 * u);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            col[i0 + 4 * u + 0] = col[i0 + 4 * u + 0] + k4[u].x * delta;
            col[i0 + 4 * u + 1] = col[i0 + 4 * u + 1] + k4[u].y * delta;
            col[i0 + 4 * u + 2] = col[i0 + 4 * u + 2] + k4[u].z * delta;
            col[i0 + 4 * u + 3] = col[i0 + 4 * u + 3] + k4[u].w * delta;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            o = o + col[i0 + 4 * u + 0] * q4[u].x;
            o = o + col[i0 + 4 * u + 1] * q4[u].y;
            o = o + col[i0 + 4 * u + 2] * q4[u].z;
            o = o + col[i0 + 4 * u + 3] * q4[u].w;
        }
    }
#pragma unroll
    for (int i = 0; i < kGdnDim; ++i) Ssh[i * kGdnDim + j] = col[i];  // column j: this lane's own
    ov[j] = o;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kGdnState / 4 / kGdnDim; ++k) reinterpret_cast<float4*>(S)[j + kGdnDim * k] = reinterpret_cast<const float4*>(Ssh)[j + kGdnDim * k];

    // ---- per-head RMSNorm (components.hpp:176-181) and the SiLU(z) gate ----
    if (j == 0) scal[2] = 1.f / sqrtf(sum_squares_128(ov) / float(kGdnDim) + a.eps);
    __syncthreads();
    const float normed = gamma * o * scal[2];
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
    const size_t smem = size_t(kGdnState + 3 * kGdnDim + 4) * 4;
    const dim3 grid(unsigned(a.Hv), unsigned(a.B));
    switch (a.W) {
        case 1: hipLaunchKernelGGL(gdn_decode_kernel<1>, grid, dim3(kGdnDim), smem, s, a); break;
        case 2: hipLaunchKernelGGL(gdn_decode_kernel<2>, grid, dim3(kGdnDim), smem, s, a); break;
        case 3: hipLaunchKernelGGL(gdn_decode_kernel<3>, grid, dim3(kGdnDim), smem, s, a); break;
        case 4: hipLaunchKernelGGL(gdn_decode_kernel<4>, grid, dim3(kGdnDim), smem, s, a); break;
        case 5: hipLaunchKernelGGL(gdn_decode_kernel<5>, grid, dim3(kGdnDim), smem, s, a); break;
        case 6: hipLaunchKernelGGL(gdn_decode_kernel<6>, grid, dim3(kGdnDim), smem, s, a); break;
        case 7: hipLaunchKernelGGL(gdn_decode_kernel<7>, grid, dim3(kGdnDim), smem, s, a); break;
        default: hipLaunchKernelGGL(gdn_decode_kernel<8>, grid, dim3(kGdnDim), smem, s, a); break;
    }
}

}  // namespace hero
