// norm.hip -- RMSNorm fused with Q8_0 activation quantization.
//
// nm/src/components.hpp:176-181: inv = 1/sqrt(dot(x,x)/N + eps), then
// x[c] = (gamma[c]*x[c])*inv. dot() is a sequential fp32 sum
// (nm/src/core.hpp:496-500): the squares are formed in parallel (one rounding
// each, like the reference's a[i]*b[i]) and summed in index order, bit for
// bit, by the workgroup's exact parallel form of that loop (hero/seqsum.hpp).
#include "hero/device.hpp"
#include "hero/kernels.hpp"
#include "hero/seqsum.hpp"

namespace hero {

__global__ __launch_bounds__(seqsum::kThreads) void rmsnorm_quant_kernel(const float* __restrict__ x, const float* __restrict__ gamma, float eps, float* __restrict__ y, int8_t* __restrict__ qs, float* __restrict__ qd, int D) {
    extern __shared__ __align__(16) float sq[];  // [D] squares
    __shared__ seqsum::Shared sm;
    const int64_t row = blockIdx.x;
    const float* xr = x + row * D;
    const int tid = threadIdx.x;
    for (int i = tid; i < D; i += seqsum::kThreads) {
        const float v = xr[i];
        sq[i] = v * v;
    }
    __syncthreads();
    float s;
    if (D <= seqsum::kMaxN) {
        s = seqsum::sum_nonneg(sq, D, sm);
    } else {
        if (tid == 0) sm.result = seqsum::serial_loop(sq, D);
        __syncthreads();
        s = sm.result;
    }
    const float inv = 1.f / sqrtf(s / float(D) + eps);
    const int groups = D >> 3;
    for (int g = tid; g < groups; g += seqsum::kThreads) {
        const float4 a = reinterpret_cast<const float4*>(xr)[2 * g];
        const float4 b = reinterpret_cast<const float4*>(xr)[2 * g + 1];
        const float4 ga = reinterpret_cast<const float4*>(gamma)[2 * g];
        const float4 gb = reinterpret_cast<const float4*>(gamma)[2 * g + 1];
        float v[8] = {ga.x * a.x * inv, ga.y * a.y * inv, ga.z * a.z * inv, ga.w * a.w * inv, gb.x * b.x * inv, gb.y * b.y * inv, gb.z * b.z * inv, gb.w * b.w * inv};
        if (y) {
            reinterpret_cast<float4*>(y + row * D)[2 * g] = make_float4(v[0], v[1], v[2], v[3]);
            reinterpret_cast<float4*>(y + row * D)[2 * g + 1] = make_float4(v[4], v[5], v[6], v[7]);
        }
        if (qs) {
            uint16_t dh;
            const int2 q = quantize8_in_quad(v, &dh);
            reinterpret_cast<int2*>(qs + row * D)[g] = q;
            if ((g & 3) == 0) qd[row * (D >> 5) + (g >> 2)] = half_bits_to_f32(dh);
        }
    }
}

// The same for D <= 4096, D % 32 == 0, with the row in registers: lane t
// holds elements 8t .. 8t+7 (one read of x), their squares go to the exact
// sum from registers, and the lane's 8 outputs are a quarter of a Q8_0 block
// (quantize8_in_quad). 512 lanes.
constexpr int kNormThreads = 512;

__global__ __launch_bounds__(kNormThreads) void rmsnorm_quant_regs_kernel(const float* __restrict__ x, const float* __restrict__ gamma, float eps, float* __restrict__ y, int8_t* __restrict__ qs, float* __restrict__ qd,
                                                                         int D) {
    constexpr int PT = seqsum::kMaxN / kNormThreads;  // 8
    __shared__ seqsum::Shared sm;
    __shared__ __align__(16) float sq[seqsum::kMaxN];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x, i0 = tid * PT;
    const bool on = i0 < D;  // whole quads (D % 32 == 0)
    float v[PT], s2[PT];
    // the weights are read at entry with the row (neither depends on the sum)
    float4 ga = make_float4(0.f, 0.f, 0.f, 0.f), gb = ga;
    if (on) {
        const float4 a = reinterpret_cast<const float4*>(x + row * D + i0)[0];
        const float4 b = reinterpret_cast<const float4*>(x + row * D + i0)[1];
        ga = reinterpret_cast<const float4*>(gamma + i0)[0];
        gb = reinterpret_cast<const float4*>(gamma + i0)[1];
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    } else {
#pragma unroll
        for (int k = 0; k < PT; ++k) v[k] = 0.f;
    }
#pragma unroll
    for (int k = 0; k < PT; ++k) s2[k] = v[k] * v[k];
    const float s = seqsum::sum_nonneg_regs<kNormThreads>(s2, sq, D, sm);
    const float inv = 1.f / sqrtf(s / float(D) + eps);
    if (!on) return;
    float o[8] = {ga.x * v[0] * inv, ga.y * v[1] * inv, ga.z * v[2] * inv, ga.w * v[3] * inv, gb.x * v[4] * inv, gb.y * v[5] * inv, gb.z * v[6] * inv, gb.w * v[7] * inv};
    if (y) {
        reinterpret_cast<float4*>(y + row * D + i0)[0] = make_float4(o[0], o[1], o[2], o[3]);
        reinterpret_cast<float4*>(y + row * D + i0)[1] = make_float4(o[4], o[5], o[6], o[7]);
    }
    if (qs) {
        uint16_t dh;
        const int2 q = quantize8_in_quad(o, &dh);
        reinterpret_cast<int2*>(qs + row * D)[tid] = q;
        if ((tid & 3) == 0) qd[row * (D >> 5) + (tid >> 2)] = half_bits_to_f32(dh);
    }
}

void launch_rmsnorm_quant(const float* x, const float* gamma, float eps, float* y, void* act, int64_t M, int64_t D, hipStream_t s) {
    int8_t* qs = static_cast<int8_t*>(act);
    float* qd = act ? reinterpret_cast<float*>(qs + M * D) : nullptr;
    if (D <= seqsum::kMaxN && D % 32 == 0)
        hipLaunchKernelGGL(rmsnorm_quant_regs_kernel, dim3(unsigned(M)), dim3(kNormThreads), 0, s, x, gamma, eps, y, qs, qd, int(D));
    else
        hipLaunchKernelGGL(rmsnorm_quant_kernel, dim3(unsigned(M)), dim3(seqsum::kThreads), size_t(D) * 4, s, x, gamma, eps, y, qs, qd, int(D));
}

}  // namespace hero
