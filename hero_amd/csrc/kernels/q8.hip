// q8.hip -- Q8_0 kernels for gfx950: activation quantization, weight packing,
// and the int8-activation matvec (GEMV) with the reference's accumulation
// order.
//
// Device layouts (all row-major by output row, like the GGUF tensor):
//   packed weight  [ qs: N*K int8 ][ d: N*(K/32) fp16 ]      34 bytes / 32 weights
//   quantized act  [ qs: M*K int8 ][ d: M*(K/32) fp32 ]      d = fp16-decoded scale
// The planar split lets a lane fetch 16 weight bytes with one aligned
// global_load_dwordx4, which the 34-byte GGUF block stride does not allow.
//
// GEMV numerics (nm/src/quant_i8.hpp:85-100): for output row o,
//   y[o] = sum over blocks b, IN BLOCK ORDER, of float(sumi_b) * (d_w * d_x)
// where sumi_b is the exact int32 dot of the two 32-byte blocks. The int32
// sums and the per-block terms are computed in parallel; the final fp32 sum
// is a sequential chain per row, so y is bit-identical to the reference.
#include "hero/device.hpp"
#include "hero/kernels.hpp"

namespace hero {

// ---------------------------------------------------------------------------
// activation quantization: x [M][K] fp32 -> act (nm/src/quant_i8.hpp:70-80)
// one lane per 8 values, four lanes per block
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void quantize_act_kernel(const float* __restrict__ x, int8_t* __restrict__ qs, float* __restrict__ d, int64_t total8) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    // total8 is a multiple of 4 and every quad is either fully in or fully out
    if (i >= total8) return;
    const float4 a = reinterpret_cast<const float4*>(x)[2 * i];
    const float4 b = reinterpret_cast<const float4*>(x)[2 * i + 1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint16_t dh;
    const int2 q = quantize8_in_quad(v, &dh);
    reinterpret_cast<int2*>(qs)[i] = q;
    if ((i & 3) == 0) d[i >> 2] = half_bits_to_f32(dh);
}

void launch_quantize_act(const float* x, void* act, int64_t M, int64_t K, hipStream_t s) {
    int8_t* qs = static_cast<int8_t*>(act);
    float* d = reinterpret_cast<float*>(qs + M * K);
    const int64_t total8 = M * K / 8;
    hipLaunchKernelGGL(quantize_act_kernel, dim3(unsigned((total8 + 255) / 256)), dim3(256), 0, s, x, qs, d, total8);
}

// ---------------------------------------------------------------------------
// weight packing: GGUF Q8_0 blocks [N][K/32] x 34 B -> planar, at row offset
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_q8_kernel(const uint8_t* __restrict__ src, int8_t* __restrict__ qs, uint16_t* __restrict__ d, int64_t blocks, int64_t row_blocks, int64_t row0) {
    const int64_t blk = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (blk >= blocks) return;
    const uint8_t* b = src + blk * 34;
    const int64_t dst_blk = row0 * row_blocks + blk;
    d[dst_blk] = uint16_t(b[0] | (b[1] << 8));
    int w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) w[j] = int(b[2 + 4 * j]) | (int(b[3 + 4 * j]) << 8) | (int(b[4 + 4 * j]) << 16) | (int(b[5 + 4 * j]) << 24);
    int4* dst = reinterpret_cast<int4*>(qs + dst_blk * 32);
    dst[0] = make_int4(w[0], w[1], w[2], w[3]);
    dst[1] = make_int4(w[4], w[5], w[6], w[7]);
}

void launch_pack_q8(const void* gguf_blocks, void* packed, int64_t N_total, int64_t K, int64_t row0, int64_t rows, hipStream_t s) {
    int8_t* qs = static_cast<int8_t*>(packed);
    uint16_t* d = reinterpret_cast<uint16_t*>(qs + N_total * K);
    const int64_t blocks = rows * (K / 32);
    hipLaunchKernelGGL(pack_q8_kernel, dim3(unsigned((blocks + 255) / 256)), dim3(256), 0, s, static_cast<const uint8_t*>(gguf_blocks), qs, d, blocks, K / 32, row0);
}

// ---------------------------------------------------------------------------
// GEMV, M = 1 (one activation row). Workgroup = 256 lanes, R output rows.
// Items are (row, 16-byte chunk) pairs; item i is handled by lane i % 256 in
// round i / 256, so the two chunks of a block sit in adjacent lanes and their
// partial int32 sums combine with one lane swap. All weight loads of a lane
// are issued before any is consumed (IPT in flight per lane).
// ---------------------------------------------------------------------------
template <int IPT, int EPI>
__global__ __launch_bounds__(256) void gemv_q8_kernel(const int8_t* __restrict__ wq, const uint16_t* __restrict__ wd, const int8_t* __restrict__ xq, const float* __restrict__ xd, float* __restrict__ y, const float* __restrict__ resid, int N, int K, int R) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x;
    const int nb = K >> 5, cpr = K >> 4;
    int4* xs = reinterpret_cast<int4*>(smem);                     // [cpr]
    float* xds = reinterpret_cast<float*>(smem + size_t(cpr) * 16);  // [nb]
    float* terms = xds + nb;                                       // [nb][R]
    const int row0 = blockIdx.x * R;
    const int rows_here = min(R, N - row0);
    const int items = rows_here * cpr;

    int4 w[IPT];
    float dw[IPT];
#pragma unroll
    for (int k = 0; k < IPT; ++k) {
        const int it = tid + k * 256;
        if (it < items) {
            const int r = it / cpr, c = it - r * cpr;
            const int64_t row = row0 + r;
            w[k] = reinterpret_cast<const int4*>(wq + row * K)[c];
            dw[k] = (c & 1) == 0 ? half_bits_to_f32(wd[row * nb + (c >> 1)]) : 0.f;
        }
    }
    for (int i = tid; i < cpr; i += 256) xs[i] = reinterpret_cast<const int4*>(xq)[i];
    for (int i = tid; i < nb; i += 256) xds[i] = xd[i];
    __syncthreads();

#pragma unroll
    for (int k = 0; k < IPT; ++k) {
        const int it = tid + k * 256;
        if (it < items) {
            const int r = it / cpr, c = it - r * cpr;
            int s = dot16_i8(w[k], xs[c], 0);
            s += __shfl_xor(s, 1);  // the other half of this block (exact)
            if ((c & 1) == 0) {
                const int b = c >> 1;
                terms[b * R + r] = float(s) * (dw[k] * xds[b]);
            }
        }
    }
    __syncthreads();

    if (tid < rows_here) {
        float acc = 0.f;
        for (int b = 0; b < nb; ++b) acc += terms[b * R + tid];
        const int64_t o = row0 + tid;
        if constexpr (EPI == kEpiResidual)
            y[o] = resid[o] + acc;  // h = x + m (nm/src/qwen35.hpp:321)
        else
            y[o] = acc;
    }
}

namespace {
template <int IPT>
void gemv_dispatch_epi(int epi, const int8_t* wq, const uint16_t* wd, const int8_t* xq, const float* xd, float* y, const float* resid, int N, int K, int R, size_t smem, hipStream_t s) {
    const dim3 grid(unsigned((N + R - 1) / R));
    if (epi == kEpiResidual)
        hipLaunchKernelGGL((gemv_q8_kernel<IPT, kEpiResidual>), grid, dim3(256), smem, s, wq, wd, xq, xd, y, resid, N, K, R);
    else
        hipLaunchKernelGGL((gemv_q8_kernel<IPT, kEpiStore>), grid, dim3(256), smem, s, wq, wd, xq, xd, y, resid, N, K, R);
}
}  // namespace

int gemv_rows_per_group(int64_t N, int64_t K) {
    const int64_t cpr = K / 16;
    // aim for 8 chunk loads in flight per lane, at least one row
    int64_t R = std::max<int64_t>(1, (8 * 256) / cpr);
    R = std::min<int64_t>(R, 64);
    (void)N;
    return int(R);
}

void launch_gemv_q8(const void* packed, const void* act, float* y, const float* resid, int64_t N, int64_t K, int epi, hipStream_t s) {
    const int8_t* wq = static_cast<const int8_t*>(packed);
    const uint16_t* wd = reinterpret_cast<const uint16_t*>(wq + N * K);
    const int8_t* xq = static_cast<const int8_t*>(act);
    const float* xd = reinterpret_cast<const float*>(xq + K);
    const int R = gemv_rows_per_group(N, K);
    const int cpr = int(K / 16), nb = int(K / 32);
    const int ipt = (R * cpr + 255) / 256;
    const size_t smem = size_t(cpr) * 16 + size_t(nb) * 4 + size_t(nb) * R * 4;
    if (ipt <= 4)
        gemv_dispatch_epi<4>(epi, wq, wd, xq, xd, y, resid, int(N), int(K), R, smem, s);
    else if (ipt <= 8)
        gemv_dispatch_epi<8>(epi, wq, wd, xq, xd, y, resid, int(N), int(K), R, smem, s);
    else if (ipt <= 12)
        gemv_dispatch_epi<12>(epi, wq, wd, xq, xd, y, resid, int(N), int(K), R, smem, s);
    else
        gemv_dispatch_epi<16>(epi, wq, wd, xq, xd, y, resid, int(N), int(K), R, smem, s);
}

// ---------------------------------------------------------------------------
// Debug export of the exact int32 block sums: out[o][b] for one act row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void block_sums_kernel(const int8_t* __restrict__ wq, const int8_t* __restrict__ xq, int32_t* __restrict__ out, int64_t N, int K) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;  // (row, block)
    const int nb = K >> 5;
    if (i >= N * nb) return;
    const int64_t row = i / nb;
    const int b = int(i - row * nb);
    const int4* w = reinterpret_cast<const int4*>(wq + row * K + b * 32);
    const int4* x = reinterpret_cast<const int4*>(xq + b * 32);
    out[i] = dot16_i8(w[1], x[1], dot16_i8(w[0], x[0], 0));
}

void launch_block_sums(const void* packed, const void* act, int32_t* out, int64_t N, int64_t K, hipStream_t s) {
    const int64_t total = N * (K / 32);
    hipLaunchKernelGGL(block_sums_kernel, dim3(unsigned((total + 255) / 256)), dim3(256), 0, s, static_cast<const int8_t*>(packed), static_cast<const int8_t*>(act), out, N, int(K));
}

}  // namespace hero
