// ew.hip -- small elementwise kernels around the GEMVs: SwiGLU + quantize,
// the Q8_0 embedding gather, and the greedy argmax.
#include <mutex>

#include "hero/device.hpp"
#include "hero/errors.hpp"
#include "hero/kernels.hpp"

namespace hero {

// nm/src/components.hpp:300-304 (GatedMLP): g = silu(gate(x)) * up(x), then
// the down projection quantizes g. gate_up row = [gate FF | up FF].
// With y set the products are written as fp32 [M][FF] (the input of a
// K-quant down projection); with qs set, quantized to Q8_0.
__global__ __launch_bounds__(256) void swiglu_quant_kernel(const float* __restrict__ gu, int8_t* __restrict__ qs, float* __restrict__ qd, float* __restrict__ y, int64_t FF,
                                                           int64_t total8, int64_t il) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= total8) return;
    const int64_t per_row = FF >> 3;
    const int64_t row = i / per_row, c = (i - row * per_row) * 8;
    // 8 consecutive outputs never straddle an interleave chunk (il % 8 == 0)
    const float* gate = gu + row * 2 * FF + (il ? (c / il) * 2 * il + c % il : c);
    const float* up = gate + (il ? il : FF);
    // 16-byte reads (c % 8 == 0, rows of 2 FF floats)
    const float4 g0 = reinterpret_cast<const float4*>(gate)[0], g1 = reinterpret_cast<const float4*>(gate)[1];
    const float4 u0 = reinterpret_cast<const float4*>(up)[0], u1 = reinterpret_cast<const float4*>(up)[1];
    const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    const float u[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = silu_f32(g[j]) * u[j];
    if (y) {
        reinterpret_cast<float4*>(y)[2 * i] = make_float4(v[0], v[1], v[2], v[3]);
        reinterpret_cast<float4*>(y)[2 * i + 1] = make_float4(v[4], v[5], v[6], v[7]);
    }
    if (!qs) return;
    uint16_t dh;
    const int2 q = quantize8_in_quad(v, &dh);
    reinterpret_cast<int2*>(qs)[i] = q;
    if ((i & 3) == 0) qd[i >> 2] = half_bits_to_f32(dh);
}

void launch_swiglu_quant(const float* gate_up, void* act, int64_t M, int64_t FF, hipStream_t s, int64_t interleave) {
    int8_t* qs = static_cast<int8_t*>(act);
    float* qd = reinterpret_cast<float*>(qs + M * FF);
    const int64_t total8 = M * FF / 8;
    hipLaunchKernelGGL(swiglu_quant_kernel, dim3(unsigned((total8 + 255) / 256)), dim3(256), 0, s, gate_up, qs, qd, nullptr, FF, total8, interleave);
}

void launch_swiglu_f32(const float* gate_up, float* y, int64_t M, int64_t FF, hipStream_t s) {
    const int64_t total8 = M * FF / 8;
    hipLaunchKernelGGL(swiglu_quant_kernel, dim3(unsigned((total8 + 255) / 256)), dim3(256), 0, s, gate_up, nullptr, nullptr, y, FF, total8, int64_t(0));
}

// nm/src/quant.hpp:306-313: row = d * q
__global__ __launch_bounds__(256) void embed_kernel(const int8_t* __restrict__ qs, const uint16_t* __restrict__ d, int64_t D, int64_t Vpad, const int32_t* __restrict__ ids, float* __restrict__ out) {
    const int64_t t = blockIdx.y;
    const int64_t id = ids[t];
    for (int64_t c = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; c < D; c += int64_t(gridDim.x) * blockDim.x) {
        const float scale = half_bits_to_f32(d[scale_index(id, c >> 5, D >> 5)]);
        out[t * D + c] = scale * float(qs[id * D + c]);
    }
}

void launch_embed_q8(const void* packed, int64_t V, int64_t D, const int32_t* ids, int64_t n, float* out, hipStream_t s) {
    const int8_t* qs = static_cast<const int8_t*>(packed);
    const uint16_t* d = reinterpret_cast<const uint16_t*>(qs + V * D);
    hipLaunchKernelGGL(embed_kernel, dim3(unsigned((D + 255) / 256), unsigned(n)), dim3(256), 0, s, qs, d, D, packed_rows_pad(V), ids, out);
}

// Greedy argmax (nm/src/logits.hpp:61-66): largest value, ties to the lowest
// index. A key orders (value, -index): the value's bits mapped to an
// order-preserving unsigned, -0 folded onto +0 so they tie as in `>`.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t index) {
    uint32_t u = f32_bits(v == 0.f ? 0.f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (uint64_t(u) << 32) | uint64_t(0xFFFFFFFFu - index);
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
    for (int off = 32; off > 0; off >>= 1) {
        const uint64_t o = __shfl_xor(k, off);
        k = o > k ? o : k;
    }
    return k;
}


__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* __restrict__ logits, int64_t n, uint64_t* __restrict__ partial) {
    const int64_t row = blockIdx.y;
    const float* l = logits + row * n;
    uint64_t best = 0;
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256) {
        const uint64_t k = argmax_key(l[i], uint32_t(i));
        best = k > best ? k : best;
    }
    best = wave_max_u64(best);
    __shared__ uint64_t waves[4];
    if ((threadIdx.x & 63) == 0) waves[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = waves[0];
        for (int w = 1; w < 4; ++w) b = waves[w] > b ? waves[w] : b;
        partial[row * gridDim.x + blockIdx.x] = b;
    }
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const uint64_t* __restrict__ partial, int parts, int32_t* __restrict__ out) {
    const int64_t row = blockIdx.x;
    uint64_t best = 0;
    for (int i = threadIdx.x; i < parts; i += 64) best = partial[row * parts + i] > best ? partial[row * parts + i] : best;
    best = wave_max_u64(best);
    if (threadIdx.x == 0) out[row] = int32_t(0xFFFFFFFFu - uint32_t(best & 0xFFFFFFFFu));
}

void launch_argmax(const float* logits, int64_t M, int64_t n, int32_t* out_index, uint64_t* scratch, hipStream_t s) {
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(kArgmaxGroups, unsigned(M)), dim3(256), 0, s, logits, n, scratch);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(unsigned(M)), dim3(64), 0, s, scratch, kArgmaxGroups, out_index);
}

// ---- argmax without allocation ---------------------------------------------
// The partial keys of hero_argmax_noalloc live in this file-scope device array
// (kArgmaxNoallocRows rows of kArgmaxGroups keys, 64 KiB per GPU, held until
// the process ends). Host code never passes the array's name to a kernel: the
// name is a host-side stand-in, not a device address. Each device's address
// comes from hipGetSymbolAddress, called once per device with that device
// current. Every key is written before it is read, so no call clears it. Calls
// that overlap on one GPU (two streams at once) share the array and race.
static __device__ __align__(256) uint64_t scratch[kArgmaxNoallocRows * kArgmaxGroups];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint64_t* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

uint64_t* argmax_noalloc_scratch() {
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) throw Error(1, "device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        g_scratch_ptr[dev] = static_cast<uint64_t*>(ptr);
    }
    return g_scratch_ptr[dev];
}

void launch_argmax_noalloc(const float* logits, int64_t M, int64_t n, int32_t* out_index, hipStream_t s) {
    if (M > kArgmaxNoallocRows) throw Error(1, "hero_argmax_noalloc: at most 64 rows (the static key array's size)");
    launch_argmax(logits, M, n, out_index, argmax_noalloc_scratch(), s);
}

// Elementwise evaluation of the scalar functions the path uses, for parity
// checks: out = [exp | log1p | silu | sigmoid | softplus], each [n].
__global__ __launch_bounds__(256) void math_eval_kernel(const float* __restrict__ x, float* __restrict__ out, int64_t n) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    out[i] = exp_f32(v);
    out[n + i] = log1p_f32(v);
    out[2 * n + i] = silu_f32(v);
    out[3 * n + i] = sigmoid_f32(v);
    out[4 * n + i] = softplus_f32(v);
}

void launch_math_eval(const float* x, float* out, int64_t n, hipStream_t s) {
    hipLaunchKernelGGL(math_eval_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, s, x, out, n);
}

// ---- measurement: a plain HBM read ---------------------------------------------------
// Workgroup g reads its contiguous share of the buffer with 16-byte loads, 8
// in flight per lane, folded with XOR into one value that is stored only if
// it equals a constant nothing produces: the bandwidth a kernel that only
// reads reaches, the ceiling the memory-bound kernels are compared with.
__global__ __launch_bounds__(256) void read_probe_kernel(const uint4* __restrict__ p, int64_t n16, uint32_t* __restrict__ out) {
    const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const int64_t b0 = per * blockIdx.x, b1 = min(n16, b0 + per);
    uint32_t acc = 0;
    int64_t i = b0 + threadIdx.x;
    for (; i + 7 * 256 < b1; i += 8 * 256) {
        uint4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = p[i + u * 256];
#pragma unroll
        for (int u = 0; u < 8; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < b1; i += 256) {
        const uint4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u) out[0] = acc;
}

void launch_read_probe(const void* p, int64_t bytes, int workgroups, uint32_t* out, hipStream_t s) {
    hipLaunchKernelGGL(read_probe_kernel, dim3(unsigned(workgroups)), dim3(256), 0, s, static_cast<const uint4*>(p), bytes / 16, out);
}

}  // namespace hero
