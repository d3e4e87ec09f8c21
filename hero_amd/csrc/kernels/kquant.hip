// kquant.hip -- GGUF K-quant weights: Q4_K and Q6_K against Q8_K
// activations (the reference's integer-activation dots), Q5_K against fp32
// activations (its dequant-in-dot form), the activation quantizer, and the
// row gather of the embedding. Bit-exact to the reference.
//
//   quantize_row_q8_K      nm/src/quant_i8.hpp:31-64
//   vec_dot_q4_K_q8_K      nm/src/quant_i8.hpp:146-191 (scalar form)
//   vec_dot_q6_K_q8_K      nm/src/quant_i8.hpp:239-278 (scalar form)
//   dot_block_q5_K         nm/src/quant.hpp:207-229
//   Weight::matvec/matmul  nm/src/quant_i8.hpp:352-383, 415-495
//   dequant_to_f32         nm/src/quant.hpp:322-395
//
// Weights are repacked once at load (kq_pack_kernel): within a super-block the
// bytes of the four positions 32j + 8i + l (i = 0..3) that share sub-block j
// and residue l = p % 8 -- the positions whose products the reference adds
// into one of its eight sums -- become one dword, so each such group is one
// 4-way int8 dot; the blocks are laid out so that each wave's weight loads
// are contiguous (the tiled layout below). A Q8_K
// activation row is K/256 GGUF blocks of 292 bytes {fp32 d, int8 qs[256],
// int16 bsums[16]} followed by the same residue regrouping of its int8.
//
// Exactness: per super-block the reference forms eight int32 sums aux[l]
// (each product weighted by its sub-block's integer scale) and, for Q4_K, the
// integer mins term; all of that is exact, so any order gives the same
// integers. The fp32 part runs per output in block order exactly as written:
// d = fp16(w.d) * x.d; sums[l] += d * float(aux[l]); (Q4_K)
// sumf -= (fp16(w.dmin) * x.d) * float(summin); then sumf += sums[0..7].
#include <algorithm>

#include "hero/device.hpp"
#include "hero/errors.hpp"
#include "hero/kernels.hpp"

namespace hero {

namespace {

constexpr int kQ8KBytes = 292;
constexpr int kKqThreads = 256;

// ---- the packed weight layout -------------------------------------------------------
// A workgroup owns R = 256 / nb consecutive output rows (a tile) and its lane
// `item` = b * R + r the super-block b of row r. Packed, each tile's blocks are
// stored wave by wave (64 items) as structure-of-arrays: 16-byte chunk u of the
// 64 blocks of a wave is 1 KiB of contiguous memory, so each weight load of a
// wave is one coalesced access. Chunks per block: Q4_K 9 (16-byte header, 8 of
// residue-regrouped quants), Q5_K 11 (the GGUF bytes), Q6_K 13 (8 of ql, 4 of
// qh, both regrouped, 1 of scales) plus a plane of fp16 d, one per slot.
__host__ __device__ inline int kq_rows_per_tile(int64_t K) { return int(K / 256) >= kKqThreads ? 1 : kKqThreads / int(K / 256); }
__host__ __device__ inline int kq_waves_per_tile(int64_t K) { return (kq_rows_per_tile(K) * int(K / 256) + 63) / 64; }
__host__ __device__ inline int kq_chunks(int type) { return type == 12 ? 9 : type == 13 ? 11 : 13; }
// slot of block (n, b): (tile * waves_per_tile + wave) * 64 + lane
__host__ __device__ inline int64_t kq_slot(int64_t n, int b, int64_t K) {
    const int R = kq_rows_per_tile(K);
    const int64_t t = n / R;
    const int item = b * R + int(n % R);
    return (t * kq_waves_per_tile(K) + item / 64) * 64 + item % 64;
}
// uint4 index of chunk u of the block in `slot`
__host__ __device__ inline int64_t kq_chunk_index(int64_t slot, int u, int U) { return ((slot / 64) * U + u) * 64 + slot % 64; }
__host__ __device__ inline int64_t kq_slots(int64_t N, int64_t K) {
    const int R = kq_rows_per_tile(K);
    return (N + R - 1) / R * kq_waves_per_tile(K) * 64;
}

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

// Sign-extend four packed 6-bit values (bytes 0..63) minus 32 to int8:
// t = q ^ 32 has its sign in bit 5; the top two bits copy it (0x20 * 6 = 0xC0).
__device__ __forceinline__ uint32_t sext6_minus32(uint32_t q) {
    const uint32_t t = q ^ 0x20202020u;
    return t | ((t & 0x20202020u) * 6u);
}

// get_scale_min_k4 (nm/src/quant.hpp:153-162): 6-bit scale and min of sub-block j
__device__ __forceinline__ void scale_min_k4(const uint8_t* q, int j, int& sc, int& m) {
    if (j < 4) {
        sc = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// the same from the 12 packed bytes held as three dwords (j compile-time)
__device__ __forceinline__ void scale_min_k4_w(const uint32_t (&h)[3], int j, int& sc, int& m) {
    auto byte = [&](int i) { return int((h[i >> 2] >> (8 * (i & 3))) & 0xFFu); };
    if (j < 4) {
        sc = byte(j) & 63;
        m = byte(j + 4) & 63;
    } else {
        sc = (byte(j + 4) & 0xF) | ((byte(j - 4) >> 6) << 4);
        m = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
}
// int8 scale g of 16 held as four dwords (g compile-time), sign-extended
__device__ __forceinline__ int scale_i8_w(const uint32_t (&w)[4], int g) { return int(w[g >> 2] << (24 - 8 * (g & 3))) >> 24; }

constexpr int kKqTile = 4;  // activation rows per pass of the K-quant GEMM

// Q4_K / Q6_K GEMM over packed weights (kq_pack_kernel) and Q8_K activations.
//
// A workgroup owns R consecutive output rows; lane (b, r) = (tid / R, tid % R)
// holds super-block b of row n0 + r in registers for the whole kernel (each
// weight byte is read once per workgroup) and walks the workgroup's
// activation rows kKqTile at a time: per row it forms the block's eight
// residue sums aux[l] (exact integers, dot4 over the residue-grouped bytes)
// and the reference's per-block fp32 products d * aux[l] (and, for Q4_K,
// dmin * sum_of_mins), leaving them in shared memory; then lane (row, r)
// chains row r's blocks in order: sums[l] += P[b][l]; sumf -= Q[b]; and
// finally sumf += sums[0..7] (nm/src/quant_i8.hpp:146-191, 239-278).
// grid (ceil(N / R), ceil(M / rows_per_group)); R * nb <= 256.
// PER_ROW (the one-row form, M = 1): the weights are decoded in the row loop
// rather than once before it, which keeps the kernel at 104 / 112 VGPRs
// instead of 132 / 189 (Q4_K / Q6_K) and so four workgroups per CU, and each
// output's nine chains run on lanes of their own. Q4_K K = 12288 x 4096 rows:
// 17.5 -> 12.0 us; Q6_K 12288 x 4096: 17.8 -> 14.9 us. With several rows per
// workgroup the decode-once form and one lane per output are faster.
template <int TYPE, bool PER_ROW>
__global__ __launch_bounds__(kKqThreads) void kq_gemm_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ act, const uint32_t* __restrict__ xt,
                                                             float* __restrict__ y, const float* __restrict__ resid, int64_t M, int64_t N, int K, int64_t ldy,
                                                             int R, int rows_per_group) {
    extern __shared__ float terms[];  // [kKqTile][R * nb][T]
    constexpr int T = TYPE == 12 ? 9 : 8;
    const int nb = K >> 8, tid = threadIdx.x, items = R * nb;
    const int64_t n0 = int64_t(blockIdx.x) * R;
    const int64_t m_begin = int64_t(blockIdx.y) * rows_per_group;
    const int64_t m_end = min(M, m_begin + rows_per_group);
    const int b = tid / R, r = tid % R;
    const bool active = tid < items && n0 + r < N;
    // this lane's slot: tile blockIdx.x, item tid
    const int64_t slot = (int64_t(blockIdx.x) * ((items + 63) / 64) + tid / 64) * 64 + tid % 64;

    // the block: Q4_K 16-byte header (d, dmin, packed scales) + 32 residue
    // dwords; Q6_K 32 low-nibble dwords, 16 high-bit dwords, 16 int8 scales, d
    // scales stay packed (Q4_K: 12 bytes, Q6_K: 16 int8) and are unpacked where used
    uint32_t q[TYPE == 12 ? 32 : 48];
    uint32_t hs[3] = {0u, 0u, 0u}, s6[4] = {0u, 0u, 0u, 0u};
    int scv[TYPE == 12 ? 8 : 16], mnv[8];  // !PER_ROW: the scales unpacked once
    float wd = 0.f, wdmin = 0.f;
    if (active) {
        const uint4* w4 = reinterpret_cast<const uint4*>(w);
        if constexpr (TYPE == 12) {
            const uint4* src = w4 + kq_chunk_index(slot, 0, 9);  // chunk u at src[64 u]
            const uint4 hdr = src[0];
            hs[0] = hdr.y, hs[1] = hdr.z, hs[2] = hdr.w;
            if constexpr (!PER_ROW) {
#pragma unroll
                for (int j = 0; j < 8; ++j) scale_min_k4_w(hs, j, scv[j], mnv[j]);
            }
            wd = half_bits_to_f32(uint16_t(hdr.x & 0xFFFF));
            wdmin = half_bits_to_f32(uint16_t(hdr.x >> 16));
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint4 v = src[64 * (1 + i)];
                q[4 * i] = v.x, q[4 * i + 1] = v.y, q[4 * i + 2] = v.z, q[4 * i + 3] = v.w;
            }
        } else {
            const uint4* src = w4 + kq_chunk_index(slot, 0, 13);
#pragma unroll
            for (int i = 0; i < 12; ++i) {
                const uint4 v = src[64 * i];
                q[4 * i] = v.x, q[4 * i + 1] = v.y, q[4 * i + 2] = v.z, q[4 * i + 3] = v.w;
            }
            const uint4 sv = src[64 * 12];
            s6[0] = sv.x, s6[1] = sv.y, s6[2] = sv.z, s6[3] = sv.w;
            if constexpr (!PER_ROW) {
#pragma unroll
                for (int g = 0; g < 16; ++g) scv[g] = scale_i8_w(s6, g);
            }
            const uint16_t* dplane = reinterpret_cast<const uint16_t*>(w4 + kq_slots(N, K) * 13);
            wd = half_bits_to_f32(dplane[slot]);
        }
    }

    for (int64_t mt = m_begin; mt < m_end; mt += kKqTile) {
        const int mrows = int(min<int64_t>(kKqTile, m_end - mt));
        if (active) {
#pragma unroll 1
            for (int mi = 0; mi < mrows; ++mi) {
                const int64_t ab = (mt + mi) * nb + b;
                const float xd = *reinterpret_cast<const float*>(act + ab * kQ8KBytes);
                const uint4* xv = reinterpret_cast<const uint4*>(xt + ab * 64);
                int aux[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                float* t = terms + (int64_t(mi) * items + tid) * T;
                if constexpr (PER_ROW) {
                    // opaque to the compiler: the decode below stays in the row loop
                    if constexpr (TYPE == 12) {
                        asm volatile("" : "+v"(hs[0]), "+v"(hs[1]), "+v"(hs[2]));
                    } else {
                        asm volatile("" : "+v"(s6[0]), "+v"(s6[1]), "+v"(s6[2]), "+v"(s6[3]));
                    }
#pragma unroll
                    for (int i = 0; i < (TYPE == 12 ? 32 : 48); ++i) asm volatile("" : "+v"(q[i]));
                }
                if constexpr (TYPE == 12) {
                    if constexpr (PER_ROW) {
                        // the activation's 64 bytes for step c are read one step ahead of their use
                        uint4 xa[4], xb[4];
#pragma unroll
                        for (int k = 0; k < 4; ++k) xa[k] = xv[k];
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            if (c < 3) {
#pragma unroll
                                for (int k = 0; k < 4; ++k) xb[k] = xv[4 * (c + 1) + k];
                            }
                            __builtin_amdgcn_sched_barrier(0);
                            const uint32_t xlo[8] = {xa[0].x, xa[0].y, xa[0].z, xa[0].w, xa[1].x, xa[1].y, xa[1].z, xa[1].w};
                            const uint32_t xhi[8] = {xa[2].x, xa[2].y, xa[2].z, xa[2].w, xa[3].x, xa[3].y, xa[3].z, xa[3].w};
                            int s0, s1, m_unused;
                            scale_min_k4_w(hs, 2 * c, s0, m_unused);
                            scale_min_k4_w(hs, 2 * c + 1, s1, m_unused);
#pragma unroll
                            for (int l = 0; l < 8; ++l) {
                                const uint32_t g = q[8 * c + l];
                                aux[l] += s0 * dot4_i8(int(g & 0x0F0F0F0Fu), int(xlo[l]), 0);
                                aux[l] += s1 * dot4_i8(int((g >> 4) & 0x0F0F0F0Fu), int(xhi[l]), 0);
                            }
                            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                            for (int k = 0; k < 4; ++k) xa[k] = xb[k];
                        }
                    } else {
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            const uint4 xl0 = xv[4 * c], xl1 = xv[4 * c + 1], xh0 = xv[4 * c + 2], xh1 = xv[4 * c + 3];
                            const uint32_t xlo[8] = {xl0.x, xl0.y, xl0.z, xl0.w, xl1.x, xl1.y, xl1.z, xl1.w};
                            const uint32_t xhi[8] = {xh0.x, xh0.y, xh0.z, xh0.w, xh1.x, xh1.y, xh1.z, xh1.w};
#pragma unroll
                            for (int l = 0; l < 8; ++l) {
                                const uint32_t g = q[8 * c + l];
                                aux[l] += scv[2 * c] * dot4_i8(int(g & 0x0F0F0F0Fu), int(xlo[l]), 0);
                                aux[l] += scv[2 * c + 1] * dot4_i8(int((g >> 4) & 0x0F0F0F0Fu), int(xhi[l]), 0);
                            }
                        }
                    }
                    const uint32_t* bw = reinterpret_cast<const uint32_t*>(act + ab * kQ8KBytes + 260);  // 16 int16 sums
                    int sumi = 0;
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const uint32_t v = bw[i];
                        int mi;
                        if constexpr (PER_ROW) {
                            int sc_unused;
                            scale_min_k4_w(hs, i, sc_unused, mi);
                        } else {
                            mi = mnv[i];
                        }
                        sumi += int(int16_t(v & 0xFFFF)) * mi;  // sums 2i and 2i+1 share min i
                        sumi += int(int16_t(v >> 16)) * mi;
                    }
                    const float d = wd * xd;
#pragma unroll
                    for (int l = 0; l < 8; ++l) t[l] = d * float(aux[l]);
                    const float dmin = wdmin * xd;
                    t[8] = dmin * float(sumi);
                } else {
                    if constexpr (PER_ROW) {
                        // the activation's 32 bytes for step j are read one step ahead of their use
                        uint4 xa[2] = {xv[0], xv[1]}, xb[2];
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            if (j < 7) xb[0] = xv[2 * j + 2], xb[1] = xv[2 * j + 3];
                            __builtin_amdgcn_sched_barrier(0);
                            const int cp = 2 * (j / 4) + (j % 2), nib = 4 * ((j % 4) / 2), hh = j / 4, sh = 2 * (j % 4);
                            const uint32_t xs[8] = {xa[0].x, xa[0].y, xa[0].z, xa[0].w, xa[1].x, xa[1].y, xa[1].z, xa[1].w};
                            const int s0 = scale_i8_w(s6, 2 * j), s1 = scale_i8_w(s6, 2 * j + 1);
#pragma unroll
                            for (int l = 0; l < 8; ++l) {
                                const uint32_t lo = (q[8 * cp + l] >> nib) & 0x0F0F0F0Fu;
                                const uint32_t hi = ((q[32 + 8 * hh + l] >> sh) & 0x03030303u) << 4;
                                const uint32_t a = sext6_minus32(lo | hi);
                                // bytes 0, 1: positions of group 2j; bytes 2, 3: group 2j + 1
                                aux[l] += s0 * dot4_i8(int(a & 0x0000FFFFu), int(xs[l]), 0);
                                aux[l] += s1 * dot4_i8(int(a & 0xFFFF0000u), int(xs[l]), 0);
                            }
                            __builtin_amdgcn_sched_barrier(0);
                            xa[0] = xb[0], xa[1] = xb[1];
                        }
                    } else {
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const int cp = 2 * (j / 4) + (j % 2), nib = 4 * ((j % 4) / 2), hh = j / 4, sh = 2 * (j % 4);
                            const uint4 x0 = xv[2 * j], x1 = xv[2 * j + 1];
                            const uint32_t xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                            for (int l = 0; l < 8; ++l) {
                                const uint32_t lo = (q[8 * cp + l] >> nib) & 0x0F0F0F0Fu;
                                const uint32_t hi = ((q[32 + 8 * hh + l] >> sh) & 0x03030303u) << 4;
                                const uint32_t a = sext6_minus32(lo | hi);
                                // bytes 0, 1: positions of group 2j; bytes 2, 3: group 2j + 1
                                aux[l] += scv[2 * j] * dot4_i8(int(a & 0x0000FFFFu), int(xs[l]), 0);
                                aux[l] += scv[2 * j + 1] * dot4_i8(int(a & 0xFFFF0000u), int(xs[l]), 0);
                            }
                        }
                    }
                    const float d = wd * xd;
#pragma unroll
                    for (int l = 0; l < 8; ++l) t[l] = d * float(aux[l]);
                }
            }
        }
        __syncthreads();
        if constexpr (PER_ROW) {
            // 16 lanes per output: lane l < 8 of the group runs sums[l] over the
            // blocks, lane 8 (Q4_K) the mins chain 0 - Q[0] - Q[1] ..., and the
            // group's first lane then forms sumf += sums[0..7] in order: the
            // same operations one lane per output does below
            constexpr int NC = TYPE == 12 ? 9 : 8;  // chains per output
            const int lane = tid & 63;
            for (int idx0 = 0; idx0 < mrows * R * 16; idx0 += kKqThreads) {
                const int idx = idx0 + tid, oi = idx >> 4, part = idx & 15;
                const int mi = oi / R, rr = oi % R;
                const bool out_live = oi < mrows * R && n0 + rr < N;
                float v = 0.f;
                if (out_live && part < NC) {
                    const float* t = terms + (int64_t(mi) * items + rr) * T + part;
                    const bool mins = part == 8;
                    const int step = R * T;
#pragma unroll 4
                    for (int bb = 0; bb < nb; ++bb) {
                        const float x = t[bb * step];
                        v = mins ? v - x : v + x;
                    }
                }
                float c[NC];
#pragma unroll
                for (int l = 0; l < NC; ++l) c[l] = __shfl(v, (lane & ~15) + l);
                if (out_live && part == 0) {
                    float sumf = TYPE == 12 ? c[NC - 1] : 0.f;
#pragma unroll
                    for (int l = 0; l < 8; ++l) sumf += c[l];
                    const int64_t o = (mt + mi) * ldy + n0 + rr;
                    y[o] = resid ? resid[o] + sumf : sumf;
                }
            }
        } else {
            for (int idx = tid; idx < mrows * R; idx += kKqThreads) {
                const int mi = idx / R, rr = idx % R;
                const int64_t n = n0 + rr;
                if (n >= N) continue;
                float sums[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                float sumf = 0.f;
                for (int bb = 0; bb < nb; ++bb) {
                    const float* t = terms + (int64_t(mi) * items + bb * R + rr) * T;
#pragma unroll
                    for (int l = 0; l < 8; ++l) sums[l] += t[l];
                    if constexpr (TYPE == 12) sumf -= t[8];
                }
#pragma unroll
                for (int l = 0; l < 8; ++l) sumf += sums[l];
                const int64_t o = (mt + mi) * ldy + n;
                y[o] = resid ? resid[o] + sumf : sumf;
            }
        }
        __syncthreads();
    }
}

// Q5_K against fp32 activations (no integer-activation kernel in the
// reference): per block the dequant-in-dot chain of nm/src/quant.hpp:207-229
// -- acc += (d1 * q - m1) * x, 256 products in order from acc = 0 -- and per
// output the sum of its blocks' results in order (quant_i8.hpp:403-407).
// Lane (b, r) keeps its 176-byte block in registers; TILE activation rows at a
// time are staged in shared memory and each weight is decoded once for all of
// them. grid (ceil(N / R), ceil(M / rows_per_group)).
template <int TILE>
__global__ __launch_bounds__(kKqThreads) void q5k_gemm_kernel(const uint8_t* __restrict__ w, const float* __restrict__ x, int64_t ldx, float* __restrict__ y,
                                                              const float* __restrict__ resid, int64_t M, int64_t N, int K, int64_t ldy, int R,
                                                              int rows_per_group) {
    // x position-major [K][TILE] (the TILE rows' values of one position are
    // adjacent: one read, constant offsets from the lane's block); once every
    // lane has its results the same memory holds the block results
    // [TILE][R * nb] (R * nb <= 256 <= K)
    extern __shared__ __align__(16) float smem[];
    float* xs = smem;
    float* res = smem;
    const int nb = K >> 8, tid = threadIdx.x, items = R * nb;
    const int64_t n0 = int64_t(blockIdx.x) * R;
    const int64_t m_begin = int64_t(blockIdx.y) * rows_per_group;
    const int64_t m_end = min(M, m_begin + rows_per_group);
    const int b = tid / R, r = tid % R;
    const bool active = tid < items && n0 + r < N;

    uint32_t qh[8], qs[32];
    float d1[8], m1[8];
    if (active) {
        const int64_t slot = (int64_t(blockIdx.x) * ((items + 63) / 64) + tid / 64) * 64 + tid % 64;
        const uint4* src = reinterpret_cast<const uint4*>(w) + kq_chunk_index(slot, 0, 11);  // chunk u at src[64 u]
        const uint4 hdr = src[0];
        const uint8_t* hb = reinterpret_cast<const uint8_t*>(&hdr);
        const float d = half_bits_to_f32(uint16_t(hdr.x & 0xFFFF)), dmin = half_bits_to_f32(uint16_t(hdr.x >> 16));
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            int sc, m;
            scale_min_k4(hb + 4, j, sc, m);
            d1[j] = d * float(sc);
            m1[j] = dmin * float(m);
        }
        const uint4 h0 = src[64], h1 = src[128];
        qh[0] = h0.x, qh[1] = h0.y, qh[2] = h0.z, qh[3] = h0.w, qh[4] = h1.x, qh[5] = h1.y, qh[6] = h1.z, qh[7] = h1.w;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint4 v = src[64 * (3 + i)];
            qs[4 * i] = v.x, qs[4 * i + 1] = v.y, qs[4 * i + 2] = v.z, qs[4 * i + 3] = v.w;
        }
    }

    for (int64_t mt = m_begin; mt < m_end; mt += TILE) {
        const int mrows = int(min<int64_t>(TILE, m_end - mt));
        for (int i = tid; i < TILE * (K >> 2); i += kKqThreads) {
            const int mi = i / (K >> 2), c4 = i % (K >> 2);
            const float4 v = mi < mrows ? reinterpret_cast<const float4*>(x + (mt + mi) * ldx)[c4] : make_float4(0.f, 0.f, 0.f, 0.f);
            xs[(4 * c4) * TILE + mi] = v.x;
            xs[(4 * c4 + 1) * TILE + mi] = v.y;
            xs[(4 * c4 + 2) * TILE + mi] = v.z;
            xs[(4 * c4 + 3) * TILE + mi] = v.w;
        }
        __syncthreads();
        float acc[TILE];
#pragma unroll
        for (int mi = 0; mi < TILE; ++mi) acc[mi] = 0.f;
        if (active) {
            const float* xb = xs + 256 * TILE * b;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int j = 2 * c + h;
#pragma unroll
                    for (int i4 = 0; i4 < 8; ++i4) {  // 4 weights: bytes 4 i4 .. 4 i4 + 3 of the 32
                        // opaque copies: decoded per pass instead of 256 decoded
                        // weights hoisted out of the row loop into registers
                        uint32_t qw = qs[8 * c + i4], fifth = qh[i4];
                        asm volatile("" : "+v"(qw), "+v"(fifth) : : "memory");
                        // byte u = the 4-bit value + 16 * its fifth bit (bit j of
                        // byte u of qh): four 5-bit weights in one dword, each
                        // converted by a byte-to-float conversion
                        const uint32_t q5 = ((qw >> (4 * h)) & 0x0F0F0F0Fu) | (((fifth >> j) & 0x01010101u) << 4);
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            const float wv = d1[j] * float((q5 >> (8 * u)) & 0xFFu) - m1[j];
                            const float* xp = xb + (64 * c + 32 * h + 4 * i4 + u) * TILE;
#pragma unroll
                            for (int mi = 0; mi < TILE; ++mi) acc[mi] += wv * xp[mi];
                        }
                        // the chains advance group by group (not deferred behind
                        // every group's decoded weights and reads)
#pragma unroll
                        for (int mi = 0; mi < TILE; ++mi) asm volatile("" : "+v"(acc[mi]));
                    }
                }
            }
        }
        __syncthreads();  // every lane's reads of xs are done
        if (active) {
#pragma unroll
            for (int mi = 0; mi < TILE; ++mi)
                if (mi < mrows) res[mi * items + tid] = acc[mi];
        }
        __syncthreads();
        for (int idx = tid; idx < mrows * R; idx += kKqThreads) {
            const int mi = idx / R, rr = idx % R;
            const int64_t n = n0 + rr;
            if (n >= N) continue;
            float s = 0.f;
            for (int bb = 0; bb < nb; ++bb) s += res[mi * items + bb * R + rr];
            const int64_t o = (mt + mi) * ldy + n;
            y[o] = resid ? resid[o] + s : s;
        }
        __syncthreads();
    }
}

// GGUF -> packed K-quant layout. Within a block: Q4_K keeps its 16-byte
// header; its 128 quant bytes become 32 residue dwords: dword 8c + l, byte i =
// qs[32c + 8i + l] (low nibbles: sub-block 2c, high: 2c + 1). Q6_K's 128 ql
// bytes take the same permutation (pair c = sub-blocks {j, j + 2} of half
// c / 2), its 64 qh bytes too (dword 8h + l, byte i = qh[32h + 8i + l]: 2-bit
// fields of sub-blocks 4h .. 4h + 3), then the 16 scales; its d goes to the d
// plane. Q5_K keeps its bytes. The blocks then take the slots of the tiled
// structure-of-arrays layout above. One lane per output dword of a block.
__global__ __launch_bounds__(256) void kq_pack_kernel(int type, const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int64_t N, int64_t K) {
    const int nb = int(K / 256), U = kq_chunks(type), words = 4 * U + 1;  // + the Q6_K d
    const int64_t gid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid >= N * nb * words) return;
    const int64_t f = gid / words;  // GGUF block: row f / nb, block f % nb
    const int wi = int(gid % words);
    const int64_t slot = kq_slot(f / nb, int(f % nb), K);
    const int bytes = type == 12 ? 144 : type == 13 ? 176 : 210;
    const uint8_t* s = src + f * bytes;
    if (wi == 4 * U) {  // Q6_K d
        if (type == 14) reinterpret_cast<uint16_t*>(dst + kq_slots(N, K) * 13 * 16)[slot] = uint16_t(s[208] | (s[209] << 8));
        return;
    }
    const uint8_t* g;   // the dword's four source bytes: g[0], g[step], g[2 step], g[3 step]
    int step = 1;
    if (type == 13) {
        g = s + 4 * wi;
    } else if (type == 12) {
        if (wi < 4) {
            g = s + 4 * wi;
        } else {
            const int dw = wi - 4;
            g = s + 16 + 32 * (dw / 8) + dw % 8;
            step = 8;
        }
    } else if (wi < 32) {
        g = s + 32 * (wi / 8) + wi % 8;
        step = 8;
    } else if (wi < 48) {
        const int dw = wi - 32;
        g = s + 128 + 32 * (dw / 8) + dw % 8;
        step = 8;
    } else {
        g = s + 192 + 4 * (wi - 48);
    }
    const uint32_t v = uint32_t(g[0]) | (uint32_t(g[step]) << 8) | (uint32_t(g[2 * step]) << 16) | (uint32_t(g[3 * step]) << 24);
    reinterpret_cast<uint32_t*>(dst)[kq_chunk_index(slot, wi / 4, U) * 4 + wi % 4] = v;
}

// Weight::dequant_row (nm/src/quant.hpp:322-395) of the rows `ids` of a
// packed Q4_K / Q6_K or GGUF Q5_K tensor: Q4_K / Q5_K d1 * q - m1 with
// d1 = d * sc, m1 = dmin * m; Q6_K (d * sc) * (q - 32). grid (nb, n_ids), 256 lanes.
__global__ __launch_bounds__(256) void kq_dequant_rows_kernel(int type, const uint8_t* __restrict__ w, int64_t N, int K, const int32_t* __restrict__ ids,
                                                              float* __restrict__ out) {
    const int b = blockIdx.x, p = threadIdx.x;
    const int64_t t = blockIdx.y;
    const int32_t id = ids[t];
    float* o = out + t * K + 256 * b + p;
    if (id < 0 || id >= N) {  // the host validates ids; a bad one gives zeros, never a stray read
        *o = 0.f;
        return;
    }
    const int64_t slot = kq_slot(id, b, K);
    const int U = kq_chunks(type);
    // byte o of the block in `slot`
    auto at = [&](int o) { return w[kq_chunk_index(slot, o >> 4, U) * 16 + (o & 15)]; };
    const int j = p >> 5, i = (p & 31) >> 3, l = p & 7;
    if (type == 12 || type == 13) {
        uint8_t hdr[16];
#pragma unroll
        for (int o = 0; o < 16; ++o) hdr[o] = at(o);
        const uint8_t* s = hdr;
        const float d = half_bits_to_f32(uint16_t(s[0] | (s[1] << 8))), dmin = half_bits_to_f32(uint16_t(s[2] | (s[3] << 8)));
        int sc, m;
        scale_min_k4(s + 4, j, sc, m);
        const float dd = d * float(sc), mm = dmin * float(m);
        int q;
        if (type == 12) {
            q = (at(16 + 4 * (8 * (j >> 1) + l) + i) >> (4 * (j & 1))) & 0xF;
        } else {
            const int e = p & 31;
            q = ((at(48 + 32 * (j >> 1) + e) >> (4 * (j & 1))) & 0xF) + (((at(16 + e) >> j) & 1) << 4);
        }
        *o = dd * float(q) - mm;
        return;
    }
    const int cp = 2 * (j >> 2) + (j & 1);
    const int lo = (at(4 * (8 * cp + l) + i) >> (4 * ((j & 3) >> 1))) & 0xF;
    const int hi = (at(128 + 4 * (8 * (j >> 2) + l) + i) >> (2 * (j & 3))) & 3;
    const float d = half_bits_to_f32(reinterpret_cast<const uint16_t*>(w + kq_slots(N, K) * 13 * 16)[slot]);
    const int sc = int(int8_t(at(192 + (p >> 4))));
    *o = d * float(sc) * float((lo | (hi << 4)) - 32);
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

int64_t kquant_packed_bytes(int type, int64_t N, int64_t K) {
    const int64_t slots = kq_slots(N, K);
    return slots * kq_chunks(type) * 16 + (type == 14 ? slots * 2 : 0);
}

void launch_kquant_pack(int type, const void* gguf, void* packed, int64_t N, int64_t K, hipStream_t s) {
    // the padding slots stay zero (never read)
    hip_check(hipMemsetAsync(packed, 0, size_t(kquant_packed_bytes(type, N, K)), s), "pack clear");
    const int64_t work = N * (K / 256) * (4 * kq_chunks(type) + 1);
    hipLaunchKernelGGL(kq_pack_kernel, dim3(unsigned((work + 255) / 256)), dim3(256), 0, s, type, static_cast<const uint8_t*>(gguf),
                       static_cast<uint8_t*>(packed), N, K);
}

// rows per workgroup (R) and activation rows per workgroup for an (M, N, K)
// product: R * nb <= 256 lanes; rows split over grid.y while that leaves at
// least ~2048 workgroups
static void kq_plan(int64_t M, int64_t N, int64_t K, int tile, int* R, int* rows_per_group) {
    *R = kq_rows_per_tile(K);  // the packed layout's tile
    const int64_t gx = (N + *R - 1) / *R;
    const int64_t want_y = std::max<int64_t>(1, (2048 + gx - 1) / gx);
    const int64_t gy = std::min<int64_t>(want_y, (M + tile - 1) / tile);
    int64_t per = (M + gy - 1) / gy;
    per = (per + tile - 1) / tile * tile;
    *rows_per_group = int(per);
}

int kquant_max_k(int type) { return type == 13 ? 16384 : 65536; }

void launch_kquant_gemm_ld(int type, const void* w, const void* act, float* y, const float* resid, int64_t M, int64_t N, int64_t K, int64_t ldy,
                           hipStream_t s) {
    int R, per;
    kq_plan(M, N, K, kKqTile, &R, &per);
    const dim3 grid(unsigned((N + R - 1) / R), unsigned((M + per - 1) / per));
    const int nb = int(K / 256);
    const auto* wb = static_cast<const uint8_t*>(w);
    const auto* ab = static_cast<const uint8_t*>(act);
    const uint32_t* xt = regrouped_of(act, M * nb);
    if (type == 12) {
        const size_t lds = size_t(kKqTile) * R * nb * 9 * 4;
        auto kernel = M == 1 ? kq_gemm_kernel<12, true> : kq_gemm_kernel<12, false>;
        hipLaunchKernelGGL(kernel, grid, dim3(kKqThreads), lds, s, wb, ab, xt, y, resid, M, N, int(K), ldy, R, per);
    } else {
        const size_t lds = size_t(kKqTile) * R * nb * 8 * 4;
        auto kernel = M == 1 ? kq_gemm_kernel<14, true> : kq_gemm_kernel<14, false>;
        hipLaunchKernelGGL(kernel, grid, dim3(kKqThreads), lds, s, wb, ab, xt, y, resid, M, N, int(K), ldy, R, per);
    }
}

void launch_kquant_gemm(int type, const void* w, const void* act, float* y, int64_t M, int64_t N, int64_t K, hipStream_t s) {
    launch_kquant_gemm_ld(type, w, act, y, nullptr, M, N, K, N, s);
}

void launch_q5k_gemm(const void* w, const float* x, int64_t ldx, float* y, const float* resid, int64_t M, int64_t N, int64_t K, int64_t ldy, hipStream_t s) {
    // activation rows per pass: shared memory holds TILE rows of K floats (<= 64 KiB)
    const int tile = M == 1 ? 1 : K <= 4096 ? 4 : K <= 8192 ? 2 : 1;
    int R, per;
    kq_plan(M, N, K, tile, &R, &per);
    const dim3 grid(unsigned((N + R - 1) / R), unsigned((M + per - 1) / per));
    const size_t lds = size_t(tile) * K * 4;  // <= 64 KiB
    const auto* wb = static_cast<const uint8_t*>(w);
    if (tile == 4)
        hipLaunchKernelGGL(q5k_gemm_kernel<4>, grid, dim3(kKqThreads), lds, s, wb, x, ldx, y, resid, M, N, int(K), ldy, R, per);
    else if (tile == 2)
        hipLaunchKernelGGL(q5k_gemm_kernel<2>, grid, dim3(kKqThreads), lds, s, wb, x, ldx, y, resid, M, N, int(K), ldy, R, per);
    else
        hipLaunchKernelGGL(q5k_gemm_kernel<1>, grid, dim3(kKqThreads), lds, s, wb, x, ldx, y, resid, M, N, int(K), ldy, R, per);
}

void launch_kquant_dequant_rows(int type, const void* w, int64_t N, int64_t K, const int32_t* ids, int64_t n, float* out, hipStream_t s) {
    hipLaunchKernelGGL(kq_dequant_rows_kernel, dim3(unsigned(K / 256), unsigned(n)), dim3(256), 0, s, type, static_cast<const uint8_t*>(w), N, int(K), ids, out);
}

}  // namespace hero
