// gdn.hip -- gated delta-net: decode (one token for each of B sequences) and
// prefill (T consecutive tokens of one sequence), all value heads.
//
// One workgroup per (sequence, value head), one lane per value column j
// (Dk = Dv = 128). For its head, the workgroup fuses everything between the
// input projection and the output projection (nm/src/qwen35.hpp:420-462):
//  * the causal conv step + SiLU on its q, k, v channels (recurrent.hpp:75-106);
//  * L2 normalisation of q and k and the 1/sqrt(Dk) query scale (:441-446);
//  * beta = sigmoid, g = A*softplus(alpha + dt) (:400-415);
//  * the gated delta rule (recurrent.hpp:146-177), with the head's 128x128
//    fp32 state staged in shared memory (16-byte coalesced loads and stores,
//    all global reads issued before any compute) and each lane's column read
//    into registers per token;
//  * the per-head RMSNorm, the SiLU(z) gate, and Q8_0 quantization of the
//    head's 128 outputs (4 blocks) for the output projection.
// Every fp32 reduction runs in the reference's order (sequential chains). The
// prefill kernel runs the same per-token steps for its tokens in order (the
// reference's token-serial loop, qwen35.hpp:436), the state staying in shared
// memory, so T prefill tokens equal T decode steps bit for bit.
//
// Conv history is a ring of W slots per channel: slot p % W holds the input
// at position p. A decode step at position p reads positions p-W+1 .. p-1 and
// writes slot p % W, which no reader of this step touches; unwritten slots are
// the causal zero padding. Prefill reads the inputs of earlier positions of
// its own chunk from the projection rows and the ring only for positions
// before the chunk; gdn_hist_kernel writes the chunk's last W positions into
// the ring afterwards.
#include "hero/device.hpp"
#include "hero/kernels.hpp"

namespace hero {

constexpr int kGdnDim = 128;
constexpr int kGdnState = kGdnDim * kGdnDim;
constexpr int kGdnVec = kGdnState / 4 / kGdnDim;  // 16-byte pieces of the state per lane
// dynamic shared memory: the state [Dk][Dv], q, k, the head output (128 each), scalars
constexpr size_t kGdnShared = size_t(kGdnState + 3 * kGdnDim + 4) * 4;

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
// then += taps[i] * (input at position p-(W-1)+i), oldest first.
template <int W>
struct ConvPast {
    float v[W > 1 ? W - 1 : 1];  // inputs at positions p-(W-1) .. p-1, oldest first
};

template <int W>
__device__ __forceinline__ float conv_channel(const float (&taps)[W], const ConvPast<W>& past, float x) {
    float sum = taps[W - 1] * x;
#pragma unroll
    for (int i = 0; i < W - 1; ++i) sum += taps[i] * past.v[i];
    return sum;
}

template <int W>
__device__ __forceinline__ void conv_shift(ConvPast<W>& past, float x) {  // the window moves on by one position
#pragma unroll
    for (int i = 0; i + 1 < W - 1; ++i) past.v[i] = past.v[i + 1];
    if constexpr (W > 1) past.v[W - 2] = x;
}

template <int W>
__device__ __forceinline__ void load_taps(const float* taps_all, int64_t c, float (&taps)[W]) {
#pragma unroll
    for (int i = 0; i < W; ++i) taps[i] = taps_all[c * W + i];
}

// the ring's inputs at positions pos-(W-1) .. pos-1 (zero before position 0)
template <int W>
__device__ __forceinline__ void load_past(const float* hist, int64_t CC, int64_t c, int pos, ConvPast<W>& past) {
#pragma unroll
    for (int i = 0; i < W - 1; ++i) {
        const int p = pos - (W - 1) + i;
        past.v[i] = p >= 0 ? hist[int64_t(p % W) * CC + c] : 0.f;
    }
}

// dynamic shared memory layout: the state [i][j] (row i = key, column j =
// value), then q, k, the head output (128 each) and 4 scalars
constexpr int kShQ = kGdnState, kShK = kShQ + kGdnDim, kShO = kShK + kGdnDim, kShScal = kShO + kGdnDim;

// One token of one head, lane j; q, k, v are the conv+SiLU outputs of the
// lane's channels. Returns the gated output of column j. The state lives in
// sh[0 .. kGdnState); the shared vectors are free again when this returns.
__device__ __forceinline__ float gdn_token(float* sh, int j, float sq, float sk, float v, float beta_in, float alpha_in, float A, float dtb, float gamma, float z, float eps) {
    float* qv = sh + kShQ;
    float* kv = sh + kShK;
    float* ov = sh + kShO;
    float* scal = sh + kShScal;
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
    for (int i = 0; i < kGdnDim; ++i) col[i] = sh[i * kGdnDim + j] * decay;  // pass 1: S[i][j] *= decay
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
    for (int i = 0; i < kGdnDim; ++i) sh[i * kGdnDim + j] = col[i];  // column j: this lane's own

    // ---- per-head RMSNorm (components.hpp:176-181) and the SiLU(z) gate ----
    ov[j] = o;
    __syncthreads();
    if (j == 0) scal[2] = 1.f / sqrtf(sum_squares_128(ov) / float(kGdnDim) + eps);
    __syncthreads();
    const float normed = gamma * o * scal[2];
    return normed * silu_f32(z);
}

// Q8_0 quantization of the head's outputs, 32 lanes per block (quant_i8.hpp:70-80)
__device__ __forceinline__ void gdn_quantize(float out, int64_t row, int64_t rows, int64_t width, int64_t idx, int j, void* act_out) {
    float amax = fabsf(out);
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    const float d = amax / 127.f;
    const float id = d != 0.f ? 1.f / d : 0.f;
    int8_t* qs = static_cast<int8_t*>(act_out);
    float* qd = reinterpret_cast<float*>(qs + rows * width);
    qs[row * width + idx] = int8_t(int(roundf(out * id)));
    if ((j & 31) == 0) qd[(row * width + idx) >> 5] = half_bits_to_f32(fp32_to_fp16_ref(d));
}

// ---- decode: one token for each of B sequences --------------------------------------
template <int W>
__global__ __launch_bounds__(kGdnDim) void gdn_decode_kernel(GdnDecodeArgs a) {
    extern __shared__ __align__(16) float sh[];
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
    float4 sv[kGdnVec];  // coalesced
#pragma unroll
    for (int k = 0; k < kGdnVec; ++k) sv[k] = reinterpret_cast<const float4*>(S)[j + kGdnDim * k];
    const int64_t cq = int64_t(hk) * kGdnDim + j, ck = KW + int64_t(hk) * kGdnDim + j, cv = 2 * KW + int64_t(h) * kGdnDim + j;
    const float xq = P[cq], xk = P[ck], xv = P[cv];
    float tq[W], tk[W], tv[W];
    ConvPast<W> pq, pk, pv;
    load_taps<W>(a.conv_taps, cq, tq);
    load_taps<W>(a.conv_taps, ck, tk);
    load_taps<W>(a.conv_taps, cv, tv);
    load_past<W>(hist, CC, cq, pos, pq);
    load_past<W>(hist, CC, ck, pos, pk);
    load_past<W>(hist, CC, cv, pos, pv);
    const float z = P[a.z_off + int64_t(h) * kGdnDim + j];
    const float gamma = a.norm_gamma[j];
    const float beta_in = P[a.beta_off + h], alpha_in = P[a.alpha_off + h];
    const float A = a.decay[h], dtb = a.dt_bias[h];
#pragma unroll
    for (int k = 0; k < kGdnVec; ++k) reinterpret_cast<float4*>(sh)[j + kGdnDim * k] = sv[k];

    // ---- conv + SiLU on this head's channels; the ring takes this position ----
    const float sq = silu_f32(conv_channel<W>(tq, pq, xq));
    const float sk = silu_f32(conv_channel<W>(tk, pk, xk));
    const float v = silu_f32(conv_channel<W>(tv, pv, xv));
    const int slot = pos % W;
    if (h < a.Hk) {  // the first value head of each key head owns its q/k history
        hist[int64_t(slot) * CC + cq] = xq;
        hist[int64_t(slot) * CC + ck] = xk;
    }
    hist[int64_t(slot) * CC + cv] = xv;

    const float out = gdn_token(sh, j, sq, sk, v, beta_in, alpha_in, A, dtb, gamma, z, a.eps);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kGdnVec; ++k) reinterpret_cast<float4*>(S)[j + kGdnDim * k] = reinterpret_cast<const float4*>(sh)[j + kGdnDim * k];
    const int64_t width = int64_t(a.Hv) * kGdnDim;
    const int64_t idx = int64_t(h) * kGdnDim + j;
    if (a.out_f32) a.out_f32[int64_t(b) * width + idx] = out;
    gdn_quantize(out, b, a.B, width, idx, j, a.act_out);
}

// ---- prefill: tokens t = 0..T-1 of one sequence at positions pos0 + t -------------
// a.B is T (rows of proj and of act_out); a.positions[0] is pos0; the state
// and the ring are sequence 0's.
template <int W>
__global__ __launch_bounds__(kGdnDim) void gdn_prefill_kernel(GdnDecodeArgs a) {
    extern __shared__ __align__(16) float sh[];
    const int j = threadIdx.x;
    const int h = blockIdx.x;
    const int hk = h % a.Hk;
    const int pos0 = a.positions[0];
    const int T = a.B;
    if (pos0 < 0) return;
    const int64_t KW = int64_t(a.Hk) * kGdnDim;
    const int64_t CC = 2 * KW + int64_t(a.Hv) * kGdnDim;
    const float* hist = a.conv_hist;
    float* S = a.state + int64_t(h) * kGdnState;
    const int64_t cq = int64_t(hk) * kGdnDim + j, ck = KW + int64_t(hk) * kGdnDim + j, cv = 2 * KW + int64_t(h) * kGdnDim + j;

    float4 sv[kGdnVec];
#pragma unroll
    for (int k = 0; k < kGdnVec; ++k) sv[k] = reinterpret_cast<const float4*>(S)[j + kGdnDim * k];
    float tq[W], tk[W], tv[W];
    ConvPast<W> pq, pk, pv;  // inputs before pos0 come from the ring
    load_taps<W>(a.conv_taps, cq, tq);
    load_taps<W>(a.conv_taps, ck, tk);
    load_taps<W>(a.conv_taps, cv, tv);
    load_past<W>(hist, CC, cq, pos0, pq);
    load_past<W>(hist, CC, ck, pos0, pk);
    load_past<W>(hist, CC, cv, pos0, pv);
    const float gamma = a.norm_gamma[j];
    const float A = a.decay[h], dtb = a.dt_bias[h];
    // the first token's inputs; each iteration reads the next token's ahead
    auto row_in = [&](int t, float& xq, float& xk, float& xv, float& z, float& bi, float& ai) {
        const float* P = a.proj + int64_t(t) * a.proj_stride;
        xq = P[cq];
        xk = P[ck];
        xv = P[cv];
        z = P[a.z_off + int64_t(h) * kGdnDim + j];
        bi = P[a.beta_off + h];
        ai = P[a.alpha_off + h];
    };
    float xq, xk, xv, z, bi, ai;
    row_in(0, xq, xk, xv, z, bi, ai);
#pragma unroll
    for (int k = 0; k < kGdnVec; ++k) reinterpret_cast<float4*>(sh)[j + kGdnDim * k] = sv[k];

    const int64_t width = int64_t(a.Hv) * kGdnDim;
    const int64_t idx = int64_t(h) * kGdnDim + j;
    for (int t = 0; t < T; ++t) {
        float nxq = 0.f, nxk = 0.f, nxv = 0.f, nz = 0.f, nbi = 0.f, nai = 0.f;
        if (t + 1 < T) row_in(t + 1, nxq, nxk, nxv, nz, nbi, nai);
        const float sq = silu_f32(conv_channel<W>(tq, pq, xq));
        const float sk = silu_f32(conv_channel<W>(tk, pk, xk));
        const float v = silu_f32(conv_channel<W>(tv, pv, xv));
        conv_shift<W>(pq, xq);
        conv_shift<W>(pk, xk);
        conv_shift<W>(pv, xv);
        const float out = gdn_token(sh, j, sq, sk, v, bi, ai, A, dtb, gamma, z, a.eps);
        if (a.out_f32) a.out_f32[int64_t(t) * width + idx] = out;
        gdn_quantize(out, t, T, width, idx, j, a.act_out);
        xq = nxq, xk = nxk, xv = nxv, z = nz, bi = nbi, ai = nai;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kGdnVec; ++k) reinterpret_cast<float4*>(S)[j + kGdnDim * k] = reinterpret_cast<const float4*>(sh)[j + kGdnDim * k];
}

// After a prefill of T tokens at pos0: the ring takes the inputs of the last
// min(T, W) positions (one lane per (position, channel)).
__global__ __launch_bounds__(256) void gdn_hist_kernel(const float* __restrict__ proj, int64_t proj_stride, float* __restrict__ hist, int64_t CC, int W, const int32_t* __restrict__ positions, int T) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int n = min(T, W);
    const int pos0 = positions[0];
    if (i >= int64_t(n) * CC || pos0 < 0) return;
    const int t = T - n + int(i / CC);
    const int64_t c = i % CC;
    hist[int64_t((pos0 + t) % W) * CC + c] = proj[int64_t(t) * proj_stride + c];
}

void launch_gdn_decode(const GdnDecodeArgs& a, hipStream_t s) {
    const dim3 grid(unsigned(a.Hv), unsigned(a.B));
    switch (a.W) {
        case 1: hipLaunchKernelGGL(gdn_decode_kernel<1>, grid, dim3(kGdnDim), kGdnShared, s, a); break;
        case 2: hipLaunchKernelGGL(gdn_decode_kernel<2>, grid, dim3(kGdnDim), kGdnShared, s, a); break;
        case 3: hipLaunchKernelGGL(gdn_decode_kernel<3>, grid, dim3(kGdnDim), kGdnShared, s, a); break;
        case 4: hipLaunchKernelGGL(gdn_decode_kernel<4>, grid, dim3(kGdnDim), kGdnShared, s, a); break;
        case 5: hipLaunchKernelGGL(gdn_decode_kernel<5>, grid, dim3(kGdnDim), kGdnShared, s, a); break;
        case 6: hipLaunchKernelGGL(gdn_decode_kernel<6>, grid, dim3(kGdnDim), kGdnShared, s, a); break;
        case 7: hipLaunchKernelGGL(gdn_decode_kernel<7>, grid, dim3(kGdnDim), kGdnShared, s, a); break;
        default: hipLaunchKernelGGL(gdn_decode_kernel<8>, grid, dim3(kGdnDim), kGdnShared, s, a); break;
    }
}

void launch_gdn_prefill(const GdnDecodeArgs& a, hipStream_t s) {
    const dim3 grid(unsigned(a.Hv));
    switch (a.W) {
        case 1: hipLaunchKernelGGL(gdn_prefill_kernel<1>, grid, dim3(kGdnDim), kGdnShared, s, a); break;
        case 2: hipLaunchKernelGGL(gdn_prefill_kernel<2>, grid, dim3(kGdnDim), kGdnShared, s, a); break;
        case 3: hipLaunchKernelGGL(gdn_prefill_kernel<3>, grid, dim3(kGdnDim), kGdnShared, s, a); break;
        case 4: hipLaunchKernelGGL(gdn_prefill_kernel<4>, grid, dim3(kGdnDim), kGdnShared, s, a); break;
        case 5: hipLaunchKernelGGL(gdn_prefill_kernel<5>, grid, dim3(kGdnDim), kGdnShared, s, a); break;
        case 6: hipLaunchKernelGGL(gdn_prefill_kernel<6>, grid, dim3(kGdnDim), kGdnShared, s, a); break;
        case 7: hipLaunchKernelGGL(gdn_prefill_kernel<7>, grid, dim3(kGdnDim), kGdnShared, s, a); break;
        default: hipLaunchKernelGGL(gdn_prefill_kernel<8>, grid, dim3(kGdnDim), kGdnShared, s, a); break;
    }
    const int64_t CC = 2 * int64_t(a.Hk) * kGdnDim + int64_t(a.Hv) * kGdnDim;
    const int64_t n = int64_t(std::min(a.B, a.W)) * CC;
    hipLaunchKernelGGL(gdn_hist_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, s, a.proj, a.proj_stride, a.conv_hist, CC, a.W, a.positions, a.B);
}

}  // namespace hero
