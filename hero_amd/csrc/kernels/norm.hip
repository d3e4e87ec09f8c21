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

void launch_rmsnorm_quant(const float* x, const float* gamma, float eps, float* y, void* act, int64_t M, int64_t D, hipStream_t s) {
    int8_t* qs = static_cast<int8_t*>(act);
    float* qd = act ? reinterpret_cast<float*>(qs + M * D) : nullptr;
    hipLaunchKernelGGL(rmsnorm_quant_kernel, dim3(unsigned(M)), dim3(seqsum::kThreads), size_t(D) * 4, s, x, gamma, eps, y, qs, qd, int(D));
}

}  // namespace hero
