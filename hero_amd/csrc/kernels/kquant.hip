// kquant.hip -- GGUF K-quant weights (Q4_K, Q6_K) against Q8_K activations:
// the activation quantizer and the matrix-vector / matrix products, bit-exact
// to the reference's x86 integer-activation dots.
//
//   quantize_row_q8_K      nm/src/quant_i8.hpp:31-64
//   vec_dot_q4_K_q8_K      nm/src/quant_i8.hpp:129-191 (scalar form)
//   vec_dot_q6_K_q8_K      nm/src/quant_i8.hpp:239-278 (scalar form)
//   Weight::matvec/matmul  nm/src/quant_i8.hpp:352-383, 430-474
//
// Layouts are GGUF's own (no repacking): a weight row is K/256 super-blocks
// of 144 (Q4_K) or 210 (Q6_K) bytes; a Q8_K activation row is K/256 blocks of
// 292 bytes {fp32 d, int8 qs[256], int16 bsums[16]}.
//
// Exactness: per super-block, the reference forms eight int32 sums aux[l]
// over the positions p with p % 8 == l (each product weighted by its
// sub-block's integer scale) and, for Q4_K, the integer mins term; all of
// that is exact, so any order gives the same integers. The fp32 part runs per
// row in block order exactly as written: d = fp16(w.d) * x.d;
// sums[l] += d * float(aux[l]); (Q4_K) sumf -= (fp16(w.dmin) * x.d) * float(summin);
// then sumf += sums[0..7].
//
// Work split: a workgroup takes R consecutive output rows of one activation
// row; its weight bytes (R rows, contiguous) and the activation row are staged
// in shared memory with coalesced 16-byte loads; lane (r, b) forms block b of
// row r's integers; lane r then chains row r's fp32 terms.
#include "hero/device.hpp"
#include "hero/kernels.hpp"

namespace hero {

namespace {

constexpr int kQ8KBytes = 292;
constexpr int kKqThreads = 256;
constexpr int kKqLdsMax = 65536;

__device__ __forceinline__ int nearest_int_magic(float v) {
    const float t = v + 12582912.f;  // 1.5 * 2^23: rounds to nearest, ties to even
    return (__float_as_int(t) & 0x007fffff) - 0x00400000;
}

// One wave per 256-element block; lane i holds elements 4i .. 4i+3.
// Besides the GGUF block, each block's 256 int8 are written regrouped (xt):
// per 32-element sub-block j, dword 8j + l = bytes (q[32j+l], q[32j+8+l],
// q[32j+16+l], q[32j+24+l]) -- the four positions that share a Q4_K integer
// sum and scale, so a Q4_K block's terms are 4-way int8 dots.
__global__ __launch_bounds__(64) void quantize_q8_K_kernel(const float* __restrict__ x, uint8_t* __restrict__ act, uint32_t* __restrict__ xt,
                                                           int64_t nblocks) {
    __shared__ uint32_t qsh[64];
    const int64_t blk = blockIdx.x;
    if (blk >= nblocks) return;
    const int lane = threadIdx.x;
    const float4 v = reinterpret_cast<const float4*>(x + blk * 256)[lane];
    const float e[4] = {v.x, v.y, v.z, v.w};
    // first element of largest magnitude (strict >, in index order)
    float amax = 0.f;
    int idx = 1 << 30;
    for (int u = 0; u < 4; ++u) {
        const float a = fabsf(e[u]);
        if (a > amax) amax = a, idx = 4 * lane + u;
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float oa = __shfl_xor(amax, off);
        const int oi = __shfl_xor(idx, off);
        if (oa > amax || (oa == amax && oi < idx)) amax = oa, idx = oi;
    }
    uint8_t* out = act + blk * kQ8KBytes;
    if (amax == 0.f) {  // the zero block: d = 0, quants and sums 0
        reinterpret_cast<uint32_t*>(out)[lane] = 0u;
        if (lane < 9) reinterpret_cast<uint32_t*>(out + 256)[lane] = 0u;
        xt[blk * 64 + lane] = 0u;
        return;
    }
    const float mx = __shfl(e[idx & 3], idx >> 2);
    const float iscale = -127.f / mx;
    int q[4];
    for (int u = 0; u < 4; ++u) q[u] = min(127, nearest_int_magic(iscale * e[u]));
    const uint32_t packed = (uint32_t(q[0]) & 0xFF) | ((uint32_t(q[1]) & 0xFF) << 8) | ((uint32_t(q[2]) & 0xFF) << 16) | (uint32_t(q[3]) << 24);
    reinterpret_cast<uint32_t*>(out + 4)[lane] = packed;
    qsh[lane] = packed;
    __syncthreads();
    {
        const uint8_t* qb = reinterpret_cast<const uint8_t*>(qsh) + 32 * (lane >> 3) + (lane & 7);
        xt[blk * 64 + lane] = uint32_t(qb[0]) | (uint32_t(qb[8]) << 8) | (uint32_t(qb[16]) << 16) | (uint32_t(qb[24]) << 24);
    }
    int s = q[0] + q[1] + q[2] + q[3];  // sums of 16 = four lanes
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    if ((lane & 3) == 0) reinterpret_cast<int16_t*>(out + 260)[lane >> 2] = int16_t(s);
    if (lane == 0) reinterpret_cast<float*>(out)[0] = 1.f / iscale;
}

template <int TYPE>
struct KqFormat;
template <>
struct KqFormat<12> {  // Q4_K
    static constexpr int kBytes = 144;
};
template <>
struct KqFormat<14> {  // Q6_K
    static constexpr int kBytes = 210;
};

// Per-block integer part of Q4_K. w = the 144 weight bytes; xt = the block's
// 256 activation int8 regrouped per 32-element sub-block j as eight dwords
// xt[8j + l] = bytes (x[32j+l], x[32j+8+l], x[32j+16+l], x[32j+24+l]): the
// four positions that share both aux[l] and the sub-block's scale, so each
// (j, l) term is one 4-way int8 dot of the same four weight nibbles, gathered
// with byte permutes. xs = the 16 activation sums. Exact integers.
__device__ __forceinline__ void q4k_block(const uint8_t* w, const uint32_t* xt, const int16_t* xs, int (&aux)[8], int& summin) {
    const uint8_t* sc = w + 4;
    const uint32_t* qs = reinterpret_cast<const uint32_t*>(w + 16);
#pragma unroll
    for (int l = 0; l < 8; ++l) aux[l] = 0;
    summin = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {  // sub-blocks 2c (low nibbles) and 2c+1 (high)
        uint32_t D[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) D[t] = qs[8 * c + t];
        int s[2], m[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int j = 2 * c + h;
            s[h] = j < 4 ? (sc[j] & 63) : ((sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4));
            m[h] = j < 4 ? (sc[j + 4] & 63) : ((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4));
            summin += m[h] * (int(xs[2 * j]) + int(xs[2 * j + 1]));
        }
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            // bytes l, 8+l, 16+l, 24+l of the 32 = byte l%4 of dwords l/4, l/4+2, l/4+4, l/4+6
            const int u = l & 3, o = l >> 2;
            const uint32_t sel = uint32_t(u) | (uint32_t(4 + u) << 8) | 0x0C0C0000u;
            const uint32_t lo2 = __builtin_amdgcn_perm(D[o + 2], D[o], sel);
            const uint32_t hi2 = __builtin_amdgcn_perm(D[o + 6], D[o + 4], sel);
            const uint32_t g = __builtin_amdgcn_perm(hi2, lo2, 0x05040100u);
            const int dl = dot4_i8(int(g & 0x0F0F0F0Fu), int(xt[8 * (2 * c) + l]), 0);
            const int dh = dot4_i8(int((g >> 4) & 0x0F0F0F0Fu), int(xt[8 * (2 * c + 1) + l]), 0);
            aux[l] += s[0] * dl;
            aux[l] += s[1] * dh;
        }
    }
}

__device__ __forceinline__ void q6k_block(const uint8_t* w, const int8_t* xq, int (&aux)[8]) {
    const uint8_t* ql = w;
    const uint8_t* qh = w + 128;
    const int8_t* sc = reinterpret_cast<const int8_t*>(w + 192);
#pragma unroll
    for (int l = 0; l < 8; ++l) aux[l] = 0;
#pragma unroll 2
    for (int p = 0; p < 256; p += 4) {
        const int h = p >> 7, e = p & 127;
        const uint8_t* lo = ql + 64 * h + (e & 63);
        const uint8_t* hi = qh + 32 * h + (e & 31);
        const int shl = (e >> 6) * 4, shh = 2 * (e >> 5);
        const int s = sc[p >> 4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int q = (((lo[u] >> shl) & 0xF) | (((hi[u] >> shh) & 3) << 4)) - 32;
            aux[(p + u) & 7] += s * (q * int(xq[p + u]));
        }
    }
}

// Q4_K: lane (r, b) loads its 144-byte block and the activation's regrouped
// block straight from memory (no staging), forms the block's integers, and
// leaves them with the block's scales in shared memory; lane r chains row r.
// grid (ceil(N / R), M), R * nb <= 256.
constexpr int kQ4Terms = 11;  // aux[8], summin, weight d | dmin << 16, activation d
constexpr int kQ4Threads = 256;

__global__ __launch_bounds__(kQ4Threads) void q4k_gemm_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ act, const uint32_t* __restrict__ xt,
                                                              float* __restrict__ y, int64_t N, int64_t K, int R) {
    __shared__ int terms[kQ4Threads * kQ4Terms];
    const int nb = int(K / 256), tid = threadIdx.x;
    const int64_t n0 = int64_t(blockIdx.x) * R, m = blockIdx.y;
    const int rows = int(min<int64_t>(R, N - n0));
    if (tid < rows * nb) {
        const int r = tid / nb, b = tid % nb;
        uint4 wv[9];
        const uint4* wsrc = reinterpret_cast<const uint4*>(w + ((n0 + r) * nb + b) * 144);
#pragma unroll
        for (int i = 0; i < 9; ++i) wv[i] = wsrc[i];
        uint4 xv[16];
        const uint4* xsrc = reinterpret_cast<const uint4*>(xt + (m * nb + b) * 64);
#pragma unroll
        for (int i = 0; i < 16; ++i) xv[i] = xsrc[i];
        const uint8_t* xb = act + (m * nb + b) * kQ8KBytes;
        int16_t bs[16];
        const uint32_t* bsrc = reinterpret_cast<const uint32_t*>(xb + 260);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t v = bsrc[i];
            bs[2 * i] = int16_t(v & 0xFFFF), bs[2 * i + 1] = int16_t(v >> 16);
        }
        const uint32_t xd_bits = *reinterpret_cast<const uint32_t*>(xb);
        int aux[8], summin;
        q4k_block(reinterpret_cast<const uint8_t*>(wv), reinterpret_cast<const uint32_t*>(xv), bs, aux, summin);
        int* t = terms + tid * kQ4Terms;
#pragma unroll
        for (int l = 0; l < 8; ++l) t[l] = aux[l];
        t[8] = summin;
        t[9] = int(wv[0].x);  // fp16 d | fp16 dmin << 16
        t[10] = int(xd_bits);
    }
    __syncthreads();
    for (int r = tid; r < rows; r += kQ4Threads) {
        float sums[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        float sumf = 0.f;
        for (int b = 0; b < nb; ++b) {
            const int* t = terms + (r * nb + b) * kQ4Terms;
            const float xd = __int_as_float(t[10]);
            const uint32_t dd = uint32_t(t[9]);
            const float d = half_bits_to_f32(uint16_t(dd & 0xFFFF)) * xd;
#pragma unroll
            for (int l = 0; l < 8; ++l) sums[l] += d * float(t[l]);
            const float dmin = half_bits_to_f32(uint16_t(dd >> 16)) * xd;
            sumf -= dmin * float(t[8]);
        }
#pragma unroll
        for (int l = 0; l < 8; ++l) sumf += sums[l];
        y[m * N + n0 + r] = sumf;
    }
}

// Q6_K: grid (ceil(N / R), M); dynamic shared: weights R * nb * 210 (+16),
// activation nb * 292, per-block terms R * nb * 10 ints
template <int TYPE>
__global__ __launch_bounds__(kKqThreads) void kquant_gemm_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ act, float* __restrict__ y,
                                                                int64_t N, int64_t K, int R) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int B = KqFormat<TYPE>::kBytes;
    const int nb = int(K / 256), tid = threadIdx.x;
    const int64_t n0 = int64_t(blockIdx.x) * R, m = blockIdx.y;
    const int rows = int(min<int64_t>(R, N - n0));
    const int64_t rb = int64_t(nb) * B;
    // the rows' bytes start at an even offset of the (16-byte aligned) tensor;
    // in shared memory they start at the same offset modulo 16, so the
    // 16-byte copies below are aligned on both sides
    const int64_t start = n0 * rb, len = int64_t(rows) * rb;
    const int head = int(start & 15);
    uint8_t* ws = smem + head;
    uint8_t* xs = smem + ((16 + int64_t(R) * rb + 15) & ~int64_t(15));
    int* terms = reinterpret_cast<int*>(xs + ((int64_t(nb) * kQ8KBytes + 15) & ~int64_t(15)));

    // stage: the rows' bytes (16-byte copies between 2-byte copies of the
    // unaligned head and tail) and the activation row (a multiple of 4 bytes)
    {
        const int64_t a0 = (start + 15) & ~int64_t(15), a1 = (start + len) & ~int64_t(15);
        if (a1 > a0) {
            const uint4* src = reinterpret_cast<const uint4*>(w + a0);
            uint4* dst = reinterpret_cast<uint4*>(smem + 16 * ((a0 - start + head) / 16));
            for (int64_t i = tid; i < (a1 - a0) / 16; i += kKqThreads) dst[i] = src[i];
            for (int64_t i = start + 2 * tid; i < a0; i += 2 * kKqThreads)
                *reinterpret_cast<uint16_t*>(ws + (i - start)) = *reinterpret_cast<const uint16_t*>(w + i);
            for (int64_t i = a1 + 2 * tid; i < start + len; i += 2 * kKqThreads)
                *reinterpret_cast<uint16_t*>(ws + (i - start)) = *reinterpret_cast<const uint16_t*>(w + i);
        } else {
            for (int64_t i = start + 2 * tid; i < start + len; i += 2 * kKqThreads)
                *reinterpret_cast<uint16_t*>(ws + (i - start)) = *reinterpret_cast<const uint16_t*>(w + i);
        }
        const uint32_t* xa = reinterpret_cast<const uint32_t*>(act + m * int64_t(nb) * kQ8KBytes);
        const int n4 = nb * kQ8KBytes / 4;
        for (int i = tid; i < n4; i += kKqThreads) reinterpret_cast<uint32_t*>(xs)[i] = xa[i];
    }
    __syncthreads();

    for (int item = tid; item < rows * nb; item += kKqThreads) {
        const int r = item / nb, b = item % nb;
        const uint8_t* wb = ws + int64_t(r) * rb + int64_t(b) * B;
        const uint8_t* xb = xs + b * kQ8KBytes;
        int aux[8], summin = 0;
        q6k_block(wb, reinterpret_cast<const int8_t*>(xb + 4), aux);
        int* t = terms + item * 10;
#pragma unroll
        for (int l = 0; l < 8; ++l) t[l] = aux[l];
        t[8] = summin;
    }
    __syncthreads();

    // fp32, in block order per row (one lane per row)
    for (int r = tid; r < rows; r += kKqThreads) {
        float sums[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        float sumf = 0.f;
        for (int b = 0; b < nb; ++b) {
            const uint8_t* wb = ws + int64_t(r) * rb + int64_t(b) * B;
            const float xd = *reinterpret_cast<const float*>(xs + b * kQ8KBytes);
            const int* t = terms + (r * nb + b) * 10;
            const float d = half_bits_to_f32(uint16_t(wb[208] | (wb[209] << 8))) * xd;
#pragma unroll
            for (int l = 0; l < 8; ++l) sums[l] += d * float(t[l]);
        }
#pragma unroll
        for (int l = 0; l < 8; ++l) sumf += sums[l];
        y[m * N + n0 + r] = sumf;
    }
}

}  // namespace

// GGUF Q8_K blocks, then (16-byte aligned) the regrouped int8 copy: 256 bytes per block
int64_t act_q8_K_bytes(int64_t m, int64_t k) { return ((m * (k / 256) * kQ8KBytes + 15) & ~int64_t(15)) + m * (k / 256) * 256; }

static const uint32_t* regrouped_of(const void* act, int64_t nblocks) {
    return reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(act) + ((nblocks * kQ8KBytes + 15) & ~int64_t(15)));
}

void launch_quantize_q8_K(const float* x, void* act, int64_t M, int64_t K, hipStream_t s) {
    const int64_t nblocks = M * (K / 256);
    auto* xt = const_cast<uint32_t*>(regrouped_of(act, nblocks));
    hipLaunchKernelGGL(quantize_q8_K_kernel, dim3(unsigned(nblocks)), dim3(64), 0, s, x, static_cast<uint8_t*>(act), xt, nblocks);
}

int kquant_rows_per_group(int type, int64_t K) {
    const int64_t nb = K / 256;
    const int64_t rb = nb * (type == 12 ? 144 : 210);
    const int64_t fixed = ((nb * kQ8KBytes + 15) & ~int64_t(15));
    int64_t r = std::min<int64_t>(kKqThreads / std::max<int64_t>(1, nb), 64);
    if (type == 12) return nb <= kQ4Threads ? int(std::max<int64_t>(1, kQ4Threads / nb)) : 0;  // no staging
    while (r > 0 && ((16 + r * rb + 15) & ~int64_t(15)) + fixed + r * nb * 10 * 4 > kKqLdsMax) --r;
    return int(std::max<int64_t>(r, 0));
}

void launch_kquant_gemm(int type, const void* w, const void* act, float* y, int64_t M, int64_t N, int64_t K, hipStream_t s) {
    if (type == 12) {
        const int nb = int(K / 256), R = std::max(1, kQ4Threads / nb);
        const dim3 grid(unsigned((N + R - 1) / R), unsigned(M));
        hipLaunchKernelGGL(q4k_gemm_kernel, grid, dim3(kQ4Threads), 0, s, static_cast<const uint8_t*>(w), static_cast<const uint8_t*>(act),
                           regrouped_of(act, M * nb), y, N, K, R);
        return;
    }
    const int R = kquant_rows_per_group(type, K);
    const int64_t nb = K / 256;
    const int64_t rb = nb * (type == 12 ? 144 : 210);
    const size_t lds = size_t(((16 + R * rb + 15) & ~int64_t(15)) + ((nb * kQ8KBytes + 15) & ~int64_t(15)) + int64_t(R) * nb * 10 * 4);
    const dim3 grid(unsigned((N + R - 1) / R), unsigned(M));
    const auto* wb = static_cast<const uint8_t*>(w);
    const auto* ab = static_cast<const uint8_t*>(act);
    hipLaunchKernelGGL(kquant_gemm_kernel<14>, grid, dim3(kKqThreads), lds, s, wb, ab, y, N, K, R);
}

}  // namespace hero
