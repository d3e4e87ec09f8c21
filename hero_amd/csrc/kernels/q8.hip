// q8.hip -- Q8_0 kernels for gfx950: activation quantization, weight packing,
// and the int8-activation matvec (GEMV) with the reference's accumulation
// order.
//
// Device layouts:
//   packed weight  [ qs: N*K int8, row-major ][ d: (Npad/8) x (K/32) x 8 fp16 ]
//                  Npad = N rounded up to 8 (zero rows): the scales of 8
//                  consecutive rows of one block are one 16-byte load.
//   quantized act  [ qs: M*K int8 ][ d: M*(K/32) fp32 ]      d = fp16-decoded scale
// Splitting quants from scales lets a lane fetch 16 weight bytes with one
// aligned global_load_dwordx4, which the 34-byte GGUF block stride does not
// allow.
//
// GEMV numerics (nm/src/quant_i8.hpp:85-100): for output row o,
//   y[o] = sum over blocks b, IN BLOCK ORDER, of float(sumi_b) * (d_w * d_x)
// where sumi_b is the exact int32 dot of the two 32-byte blocks. The int32
// sums and the per-block terms are computed in parallel; the final fp32 sum
// is a sequential chain per row, so y is bit-identical to the reference.
#include "hero/device.hpp"
#include "hero/errors.hpp"
#include "hero/kernels.hpp"
#include "hero/seqsum.hpp"
#include "hero_kernels.h"

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
// weight packing: GGUF Q8_0 blocks [rows][K/32] x 34 B -> planar. Source row r
// lands on row row0 + r, or, with interleave il > 0, on row
// row0 + (r / il) * 2 il + r % il (two tensors sharing a matrix in alternating
// il-row chunks).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_q8_kernel(const uint8_t* __restrict__ src, int8_t* __restrict__ qs, uint16_t* __restrict__ d, int64_t blocks, int64_t row_blocks, int64_t row0, int64_t Npad, int64_t il) {
    const int64_t blk = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (blk >= blocks) return;
    const uint8_t* b = src + blk * 34;
    const int64_t r = blk / row_blocks, col = blk - r * row_blocks;
    const int64_t row = row0 + (il > 0 ? (r / il) * 2 * il + r % il : r);
    d[scale_index(row, col, row_blocks)] = uint16_t(b[0] | (b[1] << 8));
    int w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) w[j] = int(b[2 + 4 * j]) | (int(b[3 + 4 * j]) << 8) | (int(b[4 + 4 * j]) << 16) | (int(b[5 + 4 * j]) << 24);
    int4* dst = reinterpret_cast<int4*>(qs + (row * row_blocks + col) * 32);
    dst[0] = make_int4(w[0], w[1], w[2], w[3]);
    dst[1] = make_int4(w[4], w[5], w[6], w[7]);
}

void launch_pack_q8(const void* gguf_blocks, void* packed, int64_t N_total, int64_t K, int64_t row0, int64_t rows, hipStream_t s, int64_t interleave) {
    int8_t* qs = static_cast<int8_t*>(packed);
    uint16_t* d = reinterpret_cast<uint16_t*>(qs + N_total * K);
    const int64_t blocks = rows * (K / 32);
    hipLaunchKernelGGL(pack_q8_kernel, dim3(unsigned((blocks + 255) / 256)), dim3(256), 0, s, static_cast<const uint8_t*>(gguf_blocks), qs, d, blocks, K / 32, row0,
                       packed_rows_pad(N_total), interleave);
}

// ---------------------------------------------------------------------------
// GEMV, M = 1 (one activation row), K a multiple of 4096: the streaming kernel.
//
// A fixed grid of workgroups (one or two per CU) each owns a contiguous range
// of whole 8-row groups, so every workgroup moves the same bytes and there is
// no tail of late workgroups. A workgroup has K/16 lanes (LG = K/4096 groups
// of 256) and lane t always handles the 16-byte K-chunk t of every row, so its
// x chunk and act scale stay in registers. Rows
// are processed 8 at a time (a sub-batch) through a ring of D sub-batches of
// weight and scale registers, refilled as soon as a sub-batch is consumed, so
// loads stay in flight while the lanes compute. Each pair of lanes forms a
// block's exact int32 sum (DPP swap), the even lane multiplies it by
// (d_w * d_x) and stores the term in shared memory. Every TR rows (and at the
// end) one barrier, then lane r of wave 0 adds row r's terms in block order
// (the reference's chain) and stores y.
//
// The workgroup reads its rows, their scale groups and (residual epilogue)
// its slice of the residual through raw buffers sized to exactly that range.
// Rows past the range, the ring's padding sub-batches and the odd lanes'
// scale loads use out-of-range offsets that read zeros, so every ring refill
// is the same unconditional loads and each sub-batch waits only for its own
// loads, with the later sub-batches still in flight. The residual of the
// next chain pass is fetched right after the previous pass, long before its
// store needs it.
// ---------------------------------------------------------------------------
constexpr int kStreamRB = 8;  // rows per sub-batch

// KC = K / 16 lanes carry a row's 16-byte chunks; the workgroup is KC rounded
// up to whole waves, the lanes past KC issuing the same loads at out-of-range
// offsets (zeros) and storing nothing.
template <int KC>
constexpr int stream_threads() { return (KC + 63) / 64 * 64; }
// the post-norm input runs its exact sums over 256 lanes (16 values each)
template <int KC, int XM>
constexpr int stream_block() { return XM == kInPostNorm ? 256 : stream_threads<KC>(); }

template <int KC, int D, int EPI, int XM, int IL>
__global__ __launch_bounds__((stream_block<KC, XM>())) void gemv_q8_stream_kernel(const int8_t* __restrict__ wq, const uint16_t* __restrict__ wd, GemvInput in, float* __restrict__ y, const float* __restrict__ resid, int N, int Npad, int TR) {
    constexpr int K = 16 * KC, nb = K / 32, ts = nb + 4;  // ts: padded term row (conflict-free 16-byte reads)
    constexpr int CPL = 1;  // K-chunks per lane
    static_assert(KC % 2 == 0, "whole Q8_0 blocks");
    static_assert(XM == kInAct || XM == kInMul || (XM == kInPostNorm && KC <= 256) || KC % 256 == 0, "the fused inputs take whole 256-lane groups");
    // row ranges in whole units: 8-row groups, or for the SwiGLU epilogue
    // 64-row groups of [32 gate rows | 32 up rows]
    constexpr int UR = EPI == kEpiSwigluQuant ? 64 : 8;
    static_assert(!IL || UR == 8, "interleaved groups are 8-row groups");
    extern __shared__ __align__(16) float terms[];          // [TR][ts]; the prologue's squares before that
    const int tid = threadIdx.x;
    const int G = gridDim.x, U = Npad / UR;
    // IL: the 8-row groups g, g + G, g + 2G, ... of workgroup g (at any moment
    // the grid reads one contiguous stretch of the matrix); otherwise a
    // contiguous range of units
    const int r_begin = IL ? 0 : UR * int((int64_t(U) * blockIdx.x) / G);
    const int r_end = IL ? N : min(N, UR * int((int64_t(U) * (blockIdx.x + 1)) / G));
    const int rows = max(r_end - r_begin, 0);
    const int nsub = IL ? (U - int(blockIdx.x) + G - 1) / G : (rows + kStreamRB - 1) / kStreamRB;
    auto grp = [&](int j) { return IL ? int(blockIdx.x) + j * G : r_begin / kStreamRB + j; };  // 8-row group of sub-batch j
    const bool even = (tid & 1) == 0;
    const bool on = tid < KC;  // the lane carries a chunk
    // the workgroup's rows (rows * K bytes) and their scale groups (nsub groups
    // of nb blocks x 8 fp16; r_begin is a multiple of 8); IL: the whole matrix
    const __amdgpu_buffer_rsrc_t bw = buffer_of(wq + int64_t(r_begin) * K, uint32_t(rows) * uint32_t(K));
    const __amdgpu_buffer_rsrc_t bd = IL ? buffer_of(wd, uint32_t(Npad / 8) * uint32_t(nb) * 16u)
                                         : buffer_of(wd + scale_index(r_begin, 0, nb), uint32_t(nsub) * uint32_t(nb) * 16u);

    int4 ring[D][kStreamRB][CPL];
    int4 sring[D][CPL];  // even lanes: scales of the sub-batch's 8 rows for each of the lane's blocks
    // one sub-batch: its scales first, then its rows in order (the order the
    // compute consumes them); the scheduling fences keep that issue order, on
    // which the compiler's counted waits depend
    auto load = [&](int j, int4 (&dst)[kStreamRB][CPL], int4 (&sdst)[CPL]) {
        // past the workgroup's last sub-batch: out-of-range offsets (zeros)
        const bool live = !IL || j < nsub;
        const uint32_t gj = IL ? uint32_t(grp(j)) : uint32_t(j);
        const uint32_t row0 = gj * kStreamRB;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int m = 0; m < CPL; ++m)  // the group's 8 scales of block tid / 2
            sdst[m] = load_b128(bd, even && live && on ? (gj * uint32_t(nb) + uint32_t(tid >> 1)) * 16u : kOOB);
#pragma unroll
        for (int r = 0; r < kStreamRB; ++r)
#pragma unroll
            for (int m = 0; m < CPL; ++m) dst[r][m] = load_b128(bw, live && on ? (row0 + uint32_t(r)) * uint32_t(K) + uint32_t(tid) * 16u : kOOB);
        __builtin_amdgcn_sched_barrier(0);
    };
    // The lane's x chunk tid as Q8_0, and the residual of the first
    // chain pass. Their global reads are issued before the weight ring's:
    // loads retire in order, so a read issued after the ring would wait for
    // every weight in flight.
    int4 xv[CPL];
    float dx[CPL];
    float xr[16], gr[16], zr[16];               // kInRmsNorm / kInHeadGate: the lane's 16 inputs, weights (and gates); kInPostNorm: zr the residual
    float ng[16];                               // kInPostNorm: the next norm's weights
    float4 gv[CPL][4], uv[CPL][4];              // kInSwiglu / kInMul: the lane's two factors
    if constexpr (XM == kInAct) {
#pragma unroll
        for (int m = 0; m < CPL; ++m) {
            const int c = on ? tid : 0;
            xv[m] = reinterpret_cast<const int4*>(in.xq)[c];
            dx[m] = in.xd[c >> 1];
        }
    } else if constexpr (XM == kInRmsNorm) {
        static_assert(KC == 256, "RMSNorm input needs K == 4096");
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 a = reinterpret_cast<const float4*>(in.x)[4 * tid + k];
            const float4 g = reinterpret_cast<const float4*>(in.gamma)[4 * tid + k];
            xr[4 * k] = a.x, xr[4 * k + 1] = a.y, xr[4 * k + 2] = a.z, xr[4 * k + 3] = a.w;
            gr[4 * k] = g.x, gr[4 * k + 1] = g.y, gr[4 * k + 2] = g.z, gr[4 * k + 3] = g.w;
        }
    } else if constexpr (XM == kInHeadGate) {
        static_assert(KC == 256, "head-gate input needs K == 4096");
        // elements 16 tid .. +15: head tid / 8, columns 16 (tid % 8) .. +15
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 a = reinterpret_cast<const float4*>(in.x)[4 * tid + k];
            const float4 zz = reinterpret_cast<const float4*>(in.z)[4 * tid + k];
            const float4 g = reinterpret_cast<const float4*>(in.gamma)[4 * (tid % 8) + k];
            xr[4 * k] = a.x, xr[4 * k + 1] = a.y, xr[4 * k + 2] = a.z, xr[4 * k + 3] = a.w;
            zr[4 * k] = zz.x, zr[4 * k + 1] = zz.y, zr[4 * k + 2] = zz.z, zr[4 * k + 3] = zz.w;
            gr[4 * k] = g.x, gr[4 * k + 1] = g.y, gr[4 * k + 2] = g.z, gr[4 * k + 3] = g.w;
        }
    } else if constexpr (XM == kInPostNorm) {
        // lane t: elements 16t .. 16t+15 (zeros on the lanes past KC)
        auto load16 = [&](const float* p, float (&dst)[16]) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 a = on ? reinterpret_cast<const float4*>(p)[4 * tid + k] : make_float4(0.f, 0.f, 0.f, 0.f);
                dst[4 * k] = a.x, dst[4 * k + 1] = a.y, dst[4 * k + 2] = a.z, dst[4 * k + 3] = a.w;
            }
        };
        load16(in.x, xr);
        load16(in.gamma, gr);
        load16(in.res, zr);
        if (in.next_gamma) load16(in.next_gamma, ng);
    } else {
        const float* up = XM == kInSwiglu ? in.gate_up + K : in.up;
#pragma unroll
        for (int m = 0; m < CPL; ++m) {
            const int c = on ? tid : 0;  // lanes past KC: chunk 0 (their products are never stored)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                gv[m][k] = reinterpret_cast<const float4*>(in.gate_up)[4 * c + k];
                uv[m][k] = reinterpret_cast<const float4*>(up)[4 * c + k];
            }
        }
    }
    // residual epilogue: the workgroup's slice of the residual (empty otherwise)
    const __amdgpu_buffer_rsrc_t br = buffer_of(EPI == kEpiResidual ? resid + r_begin : y, EPI == kEpiResidual ? uint32_t(rows) * 4u : 0u);
    // chain lane t's row in a pass that starts at sub-batch j0 (IL) or row r0
    auto chain_row = [&](int j0, int r0) { return IL ? grp(j0 + tid / kStreamRB) * kStreamRB + (tid % kStreamRB) : r0 + tid; };
    float rnext = 0.f;  // residual of the lane's row in the next chain pass
    if constexpr (EPI == kEpiResidual) rnext = load_f32(br, uint32_t(chain_row(0, 0)) * 4u);
#pragma unroll
    for (int s = 0; s < D; ++s) load(s, ring[s], sring[s]);
    // the input loads are complete once at most the ring's loads are
    // outstanding; said explicitly, so the loop below does not inherit them as
    // pending (which makes the compiler wait for every load at its head)
    wait_vmcnt<D * (kStreamRB + 1) * CPL>();

    if constexpr (XM == kInRmsNorm) {
        // RMSNorm (nm/src/components.hpp:176-181) of the whole row, then the
        // reference's quantize_row_q8_0: the sum of squares is the exact
        // sequential sum (hero/seqsum.hpp), lane t holding elements 16t..16t+15
        __shared__ seqsum::Shared sm;
        float sq[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) sq[k] = xr[k] * xr[k];
        // terms holds the squares for the sum's plain-loop fallback, which ends
        // with a barrier; otherwise nothing reads them after the sum's last
        // barrier, so the main loop may overwrite them at once
        const float ss = seqsum::sum_nonneg_regs<256>(sq, terms, K, sm);
        const float inv = 1.f / sqrtf(ss / float(K) + in.eps);
        float v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = gr[k] * xr[k] * inv;
        uint16_t dh;
        xv[0] = quantize16_in_pair(v, &dh);
        dx[0] = half_bits_to_f32(dh);
    } else if constexpr (XM == kInHeadGate) {
        // the delta-net's per-head RMSNorm (nm/src/components.hpp:176-181) over
        // 32 heads of 128 and the gate silu(z) (nm/src/qwen35.hpp:457-460, the
        // gates computed by the delta-net kernel), then quantize_row_q8_0:
        // lane h < 32 chains head h's squares in order
        __shared__ float head_inv[32];
        float4* sq4 = reinterpret_cast<float4*>(terms);
#pragma unroll
        for (int k = 0; k < 4; ++k) sq4[4 * tid + k] = make_float4(xr[4 * k] * xr[4 * k], xr[4 * k + 1] * xr[4 * k + 1], xr[4 * k + 2] * xr[4 * k + 2], xr[4 * k + 3] * xr[4 * k + 3]);
        __syncthreads();
        if (tid < 32) {
            const float4* h4 = sq4 + tid * 32;
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                const float4 v = h4[i];
                ss += v.x;
                ss += v.y;
                ss += v.z;
                ss += v.w;
            }
            head_inv[tid] = 1.f / sqrtf(ss / 128.f + in.eps);
        }
        __syncthreads();  // after it the main loop may overwrite the squares
        const float inv = head_inv[tid / 8];
        float v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = (gr[k] * xr[k] * inv) * zr[k];  // zr: the gates silu(z)
        uint16_t dh;
        xv[0] = quantize16_in_pair(v, &dh);
        dx[0] = half_bits_to_f32(dh);
    } else if constexpr (XM == kInPostNorm) {
        // launch_gemma_post_norm's arithmetic in every workgroup (the sub-block
        // ends of GemmaE4BLayer::forward, nm/src/gemma4.hpp:258-272, and the
        // per-layer input residual, :102-104): o = (RMSNorm(x) * gamma + res)
        // * scale, then the next block's RMSNorm (components.hpp:176-181) and
        // quantize_row_q8_0; both sums of squares are the exact sequential
        // sums (hero/seqsum.hpp)
        __shared__ seqsum::Shared sm;
        float sq[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) sq[k] = xr[k] * xr[k];
        const float s1 = seqsum::sum_nonneg_regs<256>(sq, terms, K, sm);
        const float inv = 1.f / sqrtf(s1 / float(K) + in.eps);
        float o[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) o[k] = (gr[k] * xr[k] * inv + zr[k]) * in.scale;
        if (blockIdx.x == 0 && on) {
#pragma unroll
            for (int k = 0; k < 4; ++k) reinterpret_cast<float4*>(in.out)[4 * tid + k] = make_float4(o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3]);
        }
        if (in.next_gamma) {
#pragma unroll
            for (int k = 0; k < 16; ++k) sq[k] = o[k] * o[k];
            __syncthreads();  // the first sum's readers of terms and sm are done
            const float s2 = seqsum::sum_nonneg_regs<256>(sq, terms, K, sm);
            const float inv2 = 1.f / sqrtf(s2 / float(K) + in.eps);
#pragma unroll
            for (int k = 0; k < 16; ++k) o[k] = ng[k] * o[k] * inv2;
        }
        uint16_t dh;
        xv[0] = quantize16_in_pair(o, &dh);
        dx[0] = half_bits_to_f32(dh);
    } else if constexpr (XM == kInSwiglu || XM == kInMul) {
        // SwiGLU (nm/src/components.hpp:300-304): silu(gate) * up over the row
        // [gate K | up K]; or a * b, Gemma's gelu(gate) * up with the GELU
        // already applied by the GEMV that produced the gate (the GELU-gated
        // FFN, nm/src/components.hpp:294-304, and the per-layer input gate,
        // nm/src/gemma4.hpp:100-105); then quantize_row_q8_0
        auto act = [](float g) { if constexpr (XM == kInSwiglu) return silu_f32(g); else return g; };
#pragma unroll
        for (int m = 0; m < CPL; ++m) {
            float v[16];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 g = gv[m][k], u = uv[m][k];
                v[4 * k] = act(g.x) * u.x, v[4 * k + 1] = act(g.y) * u.y;
                v[4 * k + 2] = act(g.z) * u.z, v[4 * k + 3] = act(g.w) * u.w;
            }
            uint16_t dh;
            xv[m] = quantize16_in_pair(v, &dh);
            dx[m] = half_bits_to_f32(dh);
        }
    }

    int chain_row0 = r_begin;  // first row (IL: first term slot) of the pending chain pass
    int chain_j0 = 0;          // its first sub-batch
    const int nsub_pad = (nsub + D - 1) / D * D;
    for (int base = 0; base < nsub_pad; base += D) {
#pragma unroll
        for (int s = 0; s < D; ++s) {
            const int j = base + s;
            // rb - chain_row0: the sub-batch's first term slot; rvalid: its rows inside the matrix / range
            const int rb = IL ? chain_row0 + (j - chain_j0) * kStreamRB : r_begin + j * kStreamRB;
            const int rvalid = IL ? (j < nsub ? min(kStreamRB, N - grp(j) * kStreamRB) : 0) : r_end - rb;
#pragma unroll
            for (int r = 0; r < kStreamRB; ++r) {
                const uint32_t pair = uint32_t(r < 4 ? (r < 2 ? 0 : 1) : (r < 6 ? 2 : 3));
#pragma unroll
                for (int m = 0; m < CPL; ++m) {
                    int v = dot16_i8(ring[s][r][m], xv[m], 0);
                    v += pair_swap_i32(v);  // the block's other 16 bytes (exact)
                    if (even && on && r < rvalid) {
                        const int4 sc = sring[s][m];
                        const uint32_t two = uint32_t(pair == 0 ? sc.x : pair == 1 ? sc.y : pair == 2 ? sc.z : sc.w);
                        const uint16_t h = uint16_t((r & 1) ? (two >> 16) : (two & 0xFFFFu));
                        terms[(rb + r - chain_row0) * ts + (tid >> 1)] = float(v) * (half_bits_to_f32(h) * dx[m]);
                    }
                }
            }
            load(j + D, ring[s], sring[s]);  // zeros past the last sub-batch
            const int done = rb + kStreamRB - chain_row0;  // rows whose terms are all stored
            if (j < nsub && (done >= TR || j + 1 == nsub)) {
                const int prow = IL ? done : min(done, r_end - chain_row0);
                __syncthreads();
                if (tid < prow) {
                    const float4* t = reinterpret_cast<const float4*>(terms + tid * ts);
                    float acc = 0.f;
                    // four float4s of terms per step; past the row's nb / 4 the
                    // terms are zeros (acc + 0 == acc: acc is never -0)
                    static_assert(nb % 4 == 0, "K a multiple of 128");
                    float4 q[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) q[u] = u < nb / 4 ? t[u] : make_float4(0.f, 0.f, 0.f, 0.f);
                    for (int b4 = 0; b4 < nb / 4; b4 += 4) {
                        float4 nq[4];
#pragma unroll
                        for (int u = 0; u < 4; ++u) nq[u] = b4 + 4 + u < nb / 4 ? t[b4 + 4 + u] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            acc += q[u].x;
                            acc += q[u].y;
                            acc += q[u].z;
                            acc += q[u].w;
                        }
#pragma unroll
                        for (int u = 0; u < 4; ++u) q[u] = nq[u];
                    }
                    const int64_t o = chain_row(chain_j0, chain_row0);
                    if (IL && o >= N) {
                        // a padding row of the last 8-row group
                    } else if constexpr (EPI == kEpiResidual)
                        y[o] = rnext + acc;  // h = x + m (nm/src/qwen35.hpp:321)
                    else if constexpr (EPI == kEpiStore)
                        y[o] = acc;
                    else if constexpr (EPI == kEpiGelu)
                        y[o] = o < in.act_rows ? gelu_tanh_f32(acc) : acc;  // Gemma's GELU gates (nm/src/components.hpp:294-304)
                    else {
                        // rows chain_row0 .. +63 are 32 gate rows then the 32 up rows of
                        // the same FF indices: g = silu(gate) * up
                        // (nm/src/components.hpp:300-304), then quantize_row_q8_0 of the
                        // block, written as the down projection's input
                        const float up = __shfl_down(acc, 32, 64);
                        if (tid < 32) {
                            const float v = silu_f32(acc) * up;
                            float amax = fabsf(v);
                            for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
                            const float d = amax / 127.f;
                            const float id = d != 0.f ? 1.f / d : 0.f;
                            const int64_t blk = chain_row0 / 64;
                            int8_t* qs = reinterpret_cast<int8_t*>(y);
                            qs[blk * 32 + tid] = int8_t(int(roundf(v * id)));
                            if (tid == 0) reinterpret_cast<float*>(qs + N / 2)[blk] = half_bits_to_f32(fp32_to_fp16_ref(d));
                        }
                    }
                }
                __syncthreads();
                chain_row0 += prow;
                chain_j0 = j + 1;
                if constexpr (EPI == kEpiResidual) rnext = load_f32(br, uint32_t(chain_row(chain_j0, chain_row0) - r_begin) * 4u);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// GEMV for any K % 32 == 0 (used where K is not a multiple of 4096). One-shot
// workgroups of 256 lanes over R rows; items are (row, 16-byte chunk) pairs,
// item i handled by lane i % 256, so a block's two chunks sit in adjacent
// lanes. Terms go to shared memory, then lane r adds row r's terms in order.
// ---------------------------------------------------------------------------
template <int IPT, int EPI>
__global__ __launch_bounds__(256) void gemv_q8_kernel(const int8_t* __restrict__ wq, const uint16_t* __restrict__ wd, const int8_t* __restrict__ xq, const float* __restrict__ xd, float* __restrict__ y, const float* __restrict__ resid, int N, int Npad, int K, int R) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x;
    const int nb = K >> 5, cpr = K >> 4;
    int4* xs = reinterpret_cast<int4*>(smem);                        // [cpr]
    float* xds = reinterpret_cast<float*>(smem + size_t(cpr) * 16);  // [nb]
    float* terms = xds + nb;                                          // [R][nb + 4]
    const int ts = nb + 4;
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
            dw[k] = (c & 1) == 0 ? half_bits_to_f32(wd[scale_index(row, c >> 1, K >> 5)]) : 0.f;
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
                terms[r * ts + b] = float(s) * (dw[k] * xds[b]);
            }
        }
    }
    __syncthreads();

    if (tid < rows_here) {
        const float* t = terms + tid * ts;
        float acc = 0.f;
        int b = 0;
        for (; b + 16 <= nb; b += 16) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; u += 4) {
                const float4 q = *reinterpret_cast<const float4*>(t + b + u);
                v[u] = q.x, v[u + 1] = q.y, v[u + 2] = q.z, v[u + 3] = q.w;
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) acc += v[u];
        }
        for (; b < nb; ++b) acc += t[b];
        const int64_t o = row0 + tid;
        if constexpr (EPI == kEpiResidual)
            y[o] = resid[o] + acc;
        else
            y[o] = acc;
    }
}

int device_cus() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

namespace {

// Interleaved 8-row groups (the grid reads one contiguous stretch of the
// matrix at a time: 0.3-2.7 us less per launch at K = 4096) except for the
// SwiGLU epilogue and K = 8192, 12288, which keep contiguous ranges
template <int KC, int D, int XM>
void stream_dispatch(int epi, const int8_t* wq, const uint16_t* wd, const GemvInput& in, float* y, const float* resid, int N, int Npad, int G, int TR, size_t smem, hipStream_t s) {
    const dim3 block(stream_threads<KC>());
    constexpr int IL = KC == 256 || KC % 256 != 0;
    if constexpr (XM == kInAct) {
        if (epi == kEpiGelu) {
            hipLaunchKernelGGL((gemv_q8_stream_kernel<KC, D, kEpiGelu, XM, IL>), dim3(unsigned(G)), block, smem, s, wq, wd, in, y, resid, N, Npad, TR);
            return;
        }
    }
    if (epi == kEpiGelu) throw Error(HERO_EINVAL, "streaming GEMV: the GELU epilogue takes the quantized input");
    if (epi == kEpiResidual)
        hipLaunchKernelGGL((gemv_q8_stream_kernel<KC, D, kEpiResidual, XM, IL>), dim3(unsigned(G)), block, smem, s, wq, wd, in, y, resid, N, Npad, TR);
    else if constexpr (KC == 256)
        if (epi == kEpiSwigluQuant)
            hipLaunchKernelGGL((gemv_q8_stream_kernel<KC, D, kEpiSwigluQuant, XM, 0>), dim3(unsigned(G)), block, smem, s, wq, wd, in, y, resid, N, Npad, TR);
        else
            hipLaunchKernelGGL((gemv_q8_stream_kernel<KC, D, kEpiStore, XM, IL>), dim3(unsigned(G)), block, smem, s, wq, wd, in, y, resid, N, Npad, TR);
    else
        hipLaunchKernelGGL((gemv_q8_stream_kernel<KC, D, kEpiStore, XM, IL>), dim3(unsigned(G)), block, smem, s, wq, wd, in, y, resid, N, Npad, TR);
}

template <int KC, int D>
void stream_dispatch_in(int epi, const int8_t* wq, const uint16_t* wd, const GemvInput& in, float* y, const float* resid, int N, int Npad, int G, int TR, size_t smem, hipStream_t s) {
    if (in.mode == kInPostNorm) {  // Gemma's sub-block ends: stored rows or GELU gates
        if constexpr (KC == 160) {
            constexpr int IL = 1;
            const dim3 block(stream_block<KC, kInPostNorm>());
            if (epi == kEpiGelu)
                hipLaunchKernelGGL((gemv_q8_stream_kernel<KC, D, kEpiGelu, kInPostNorm, IL>), dim3(unsigned(G)), block, smem, s, wq, wd, in, y, resid, N, Npad, TR);
            else if (epi == kEpiStore)
                hipLaunchKernelGGL((gemv_q8_stream_kernel<KC, D, kEpiStore, kInPostNorm, IL>), dim3(unsigned(G)), block, smem, s, wq, wd, in, y, resid, N, Npad, TR);
            else
                throw Error(HERO_EINVAL, "streaming GEMV: the post-norm input takes the store or GELU epilogue");
            return;
        }
        throw Error(HERO_EINVAL, "streaming GEMV: no post-norm input at K = " + std::to_string(16 * KC));
    }
    if (in.mode == kInMul) {  // Gemma's FFN and per-layer input projections: stored rows only
        if (epi != kEpiStore) throw Error(HERO_EINVAL, "streaming GEMV: the product input takes the plain store epilogue");
        constexpr int IL = KC == 256 || KC % 256 != 0;
        hipLaunchKernelGGL((gemv_q8_stream_kernel<KC, D, kEpiStore, kInMul, IL>), dim3(unsigned(G)), dim3(stream_threads<KC>()), smem, s, wq, wd, in, y, resid, N, Npad, TR);
        return;
    }
    if constexpr (KC % 256 == 0) {
        if (in.mode == kInSwiglu) {
            stream_dispatch<KC, D, kInSwiglu>(epi, wq, wd, in, y, resid, N, Npad, G, TR, smem, s);
            return;
        }
    }
    if constexpr (KC == 256) {
        if (in.mode == kInRmsNorm)
            stream_dispatch<KC, D, kInRmsNorm>(epi, wq, wd, in, y, resid, N, Npad, G, TR, smem, s);
        else if (in.mode == kInHeadGate)
            stream_dispatch<KC, D, kInHeadGate>(epi, wq, wd, in, y, resid, N, Npad, G, TR, smem, s);
        else
            stream_dispatch<KC, D, kInAct>(epi, wq, wd, in, y, resid, N, Npad, G, TR, smem, s);
    } else {
        stream_dispatch<KC, D, kInAct>(epi, wq, wd, in, y, resid, N, Npad, G, TR, smem, s);
    }
}

template <int IPT>
void gemv_dispatch_epi(int epi, const int8_t* wq, const uint16_t* wd, const int8_t* xq, const float* xd, float* y, const float* resid, int N, int Npad, int K, int R, size_t smem, hipStream_t s) {
    const dim3 grid(unsigned((N + R - 1) / R));
    if (epi == kEpiResidual)
        hipLaunchKernelGGL((gemv_q8_kernel<IPT, kEpiResidual>), grid, dim3(256), smem, s, wq, wd, xq, xd, y, resid, N, Npad, K, R);
    else
        hipLaunchKernelGGL((gemv_q8_kernel<IPT, kEpiStore>), grid, dim3(256), smem, s, wq, wd, xq, xd, y, resid, N, Npad, K, R);
}

}  // namespace

// the row lengths with a streaming instantiation: K = 4096, 8192, 12288 (every
// input form) and the other decode widths of the Qwen and Gemma models (the
// plain quantized input)
bool gemv_streams(int64_t K) { return K % 4096 == 0 && K / 4096 <= 3; }
bool gemv_streams_act(int64_t K) {
    switch (K) {
        case 256: case 1024: case 2048: case 2560: case 2816: case 4096: case 8192: case 10240: case 12288: return true;
        default: return false;
    }
}
bool gemv_post_norm_fusable(int64_t K) { return K == 2560; }

int gemv_stream_grid(int64_t N, int epi) {
    const int64_t unit = epi == kEpiSwigluQuant ? 64 : 8;
    return int(std::min<int64_t>(N >= 16384 ? 2 * device_cus() : device_cus(), packed_rows_pad(N) / unit));
}

GemvPrefetch gemv_prefetch_of(const void* packed, int64_t N, int64_t K, int epi, int part) {
    if (!packed || !gemv_streams(K) || part < 1 || part > 8) return GemvPrefetch{};
    // the workgroup -> rows map of launch_gemv_q8_in: interleaved 8-row groups
    // at K = 4096 outside the SwiGLU epilogue, contiguous ranges of 8-row (or
    // 64-row, SwiGLU) units otherwise
    const bool il = K == 4096 && epi != kEpiSwigluQuant;
    return GemvPrefetch{packed, int32_t(N), int32_t(K), int32_t(gemv_stream_grid(N, epi)), epi == kEpiSwigluQuant ? 64 : 8, il ? 1 : 0, part};
}

__global__ __launch_bounds__(64) void gemv_prefetch_kernel(PrefetchList list) {
    __shared__ __align__(16) int4 sink[kPrefetchSinkBytes / 16];
    prefetch_gemvs(list, int(blockIdx.x), int(gridDim.x), lds_offset(sink));
}

void launch_gemv_prefetch(const GemvPrefetch& p, hipStream_t s) {
    if (!p.packed) return;
    PrefetchList list{};
    list.m[0] = p;
    hipLaunchKernelGGL(gemv_prefetch_kernel, dim3(unsigned(p.G)), dim3(64), 0, s, list);
}

void launch_gemv_q8_in(const void* packed, const GemvInput& in, float* y, const float* resid, int64_t N, int64_t K, int epi, hipStream_t s) {
    const int8_t* wq = static_cast<const int8_t*>(packed);
    const uint16_t* wd = reinterpret_cast<const uint16_t*>(wq + N * K);
    const int Npad = int(packed_rows_pad(N));
    // one workgroup per CU, two for the tall matrices; row ranges in whole
    // 8-row groups (64-row groups for the SwiGLU epilogue: one chain pass each)
    const int64_t unit = epi == kEpiSwigluQuant ? 64 : 8;
    const int G = gemv_stream_grid(N, epi);
    const int64_t rows_per = (Npad / unit + G - 1) / G * unit;
    const int nb = int(K / 32);
    // rows per chain pass: at most 64 (one wave) and 64 KB of terms
    const int64_t TR = epi == kEpiSwigluQuant ? 64 : std::min<int64_t>({64, rows_per, (65536 / ((nb + 4) * 4)) / 8 * 8});
    size_t smem = size_t(TR) * (nb + 4) * 4;
    if (in.mode == kInRmsNorm || in.mode == kInHeadGate) smem = std::max(smem, size_t(K) * 4);  // the squares
    if (in.mode == kInPostNorm) smem = std::max(smem, size_t(seqsum::kMaxN) * 4);  // the squares of the 256-lane sums
    // a ring of two 8-row sub-batches: deeper rings only add padding
    // sub-batches where a workgroup has few rows
    switch (K) {
        case 256: stream_dispatch_in<16, 2>(epi, wq, wd, in, y, resid, int(N), Npad, G, int(TR), smem, s); break;
        case 1024: stream_dispatch_in<64, 2>(epi, wq, wd, in, y, resid, int(N), Npad, G, int(TR), smem, s); break;
        case 2048: stream_dispatch_in<128, 2>(epi, wq, wd, in, y, resid, int(N), Npad, G, int(TR), smem, s); break;
        case 2560: stream_dispatch_in<160, 2>(epi, wq, wd, in, y, resid, int(N), Npad, G, int(TR), smem, s); break;
        case 2816: stream_dispatch_in<176, 2>(epi, wq, wd, in, y, resid, int(N), Npad, G, int(TR), smem, s); break;
        case 4096: stream_dispatch_in<256, 2>(epi, wq, wd, in, y, resid, int(N), Npad, G, int(TR), smem, s); break;
        case 8192: stream_dispatch_in<512, 2>(epi, wq, wd, in, y, resid, int(N), Npad, G, int(TR), smem, s); break;
        case 10240: stream_dispatch_in<640, 2>(epi, wq, wd, in, y, resid, int(N), Npad, G, int(TR), smem, s); break;
        case 12288: stream_dispatch_in<768, 2>(epi, wq, wd, in, y, resid, int(N), Npad, G, int(TR), smem, s); break;
        default: throw Error(HERO_EINVAL, "streaming GEMV: no instantiation for K = " + std::to_string(K));
    }
}

void launch_gemv_q8(const void* packed, const void* act, float* y, const float* resid, int64_t N, int64_t K, int epi, hipStream_t s) {
    if (epi == kEpiGelu) throw Error(HERO_EINVAL, "GEMV: the GELU epilogue takes its row count through launch_gemv_q8_in");
    const int8_t* xq = static_cast<const int8_t*>(act);
    const float* xd = reinterpret_cast<const float*>(xq + K);
    if (gemv_streams_act(K)) {
        GemvInput in{};
        in.mode = kInAct;
        in.xq = xq;
        in.xd = xd;
        launch_gemv_q8_in(packed, in, y, resid, N, K, epi, s);
        return;
    }
    const int8_t* wq = static_cast<const int8_t*>(packed);
    const uint16_t* wd = reinterpret_cast<const uint16_t*>(wq + N * K);
    const int Npad = int(packed_rows_pad(N));
    const int64_t cpr = K / 16;
    const int R = int(std::min<int64_t>(64, std::max<int64_t>(1, (8 * 256) / cpr)));  // ~8 chunk loads in flight per lane
    const int nb = int(K / 32);
    const int ipt = int((R * cpr + 255) / 256);
    const size_t smem = size_t(cpr) * 16 + size_t(nb) * 4 + size_t(nb + 4) * R * 4;
    if (ipt <= 4)
        gemv_dispatch_epi<4>(epi, wq, wd, xq, xd, y, resid, int(N), Npad, int(K), R, smem, s);
    else if (ipt <= 8)
        gemv_dispatch_epi<8>(epi, wq, wd, xq, xd, y, resid, int(N), Npad, int(K), R, smem, s);
    else if (ipt <= 12)
        gemv_dispatch_epi<12>(epi, wq, wd, xq, xd, y, resid, int(N), Npad, int(K), R, smem, s);
    else
        gemv_dispatch_epi<16>(epi, wq, wd, xq, xd, y, resid, int(N), Npad, int(K), R, smem, s);
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

namespace hero {

// ---------------------------------------------------------------------------
// GEMM, M > 1 rows (prefill, batched decode): Y[M][N] = X W^T in the
// reference's per-element order (Weight::matmul, nm/src/quant_i8.hpp:430-474:
// each y[m][n] is vec_dot_q8_0_q8_0 of weight row n and activation row m).
//
// int8 MFMA v_mfma_i32_16x16x32_i8 with K = 32 gives exactly one Q8_0 block's
// int32 sums for a 16x16 (m, n) tile (C zero per block); each lane then adds
// float(sumi) * (d_w * d_x) to its fp32 accumulators, blocks in order. That
// fp32 work (4 VALU operations per output and block) is the kernel's bound.
// Lane layout (checked on the device): A lane l = row l%16, k bytes
// 8*(l/16)..+7; B lane l = column l%16, the same k bytes; C lane l, register r
// = row 4*(l/16)+r, column l%16.
//
// Workgroup: 256 lanes, a BM x 64 tile of Y; the four waves form a grid over
// it (4 x 1 for BM >= 64: 32 or 16 rows x 64 columns each; 2 x 2 at BM = 32;
// 1 x 4 at BM = 16), so at the tall tiles a wave's operand and scale reads
// serve two or four MFMAs each (unrolling a whole chunk of 8 blocks measured
// slower: more registers, a worse schedule). K streams through shared memory
// in chunks of KC blocks (gemm_kc: 4 at BM = 128, 8 below), tile rows padded
// by 16 bytes (16 rows' 8-byte operand reads hit distinct banks); at BM = 128
// the 4-block chunk halves the staging registers (117 instead of 204 VGPRs:
// four waves per SIMD instead of two). The next chunk's bytes and scales are loaded into registers
// while the current chunk is computed (raw buffer loads sized to the tile, so
// rows, blocks and scales past the edges read zeros without a branch), then
// stored to shared memory between two barriers.
// ---------------------------------------------------------------------------
typedef int v4i_t __attribute__((ext_vector_type(4)));
constexpr int kGemmBN = 64;
// K blocks per shared-memory chunk: 4 at the 128-row tile (half the staging
// registers: four waves per SIMD), 8 below (fewer barriers; at BM = 64 the
// 4-block chunk measured 20% slower)
template <int BM>
constexpr int gemm_kc() { return BM >= 128 ? 4 : 8; }

template <int BM, int EPI>
__global__ __launch_bounds__(256) void gemm_q8_kernel(const int8_t* __restrict__ wq, const uint16_t* __restrict__ wd, const int8_t* __restrict__ xq, const float* __restrict__ xd, float* __restrict__ y, const float* __restrict__ resid, int M, int N, int Npad, int K) {
    constexpr int kGemmKC = gemm_kc<BM>(), kGemmRow = kGemmKC * 32 + 16;
    __shared__ __align__(16) int8_t Xs[BM * kGemmRow];
    __shared__ __align__(16) int8_t Ws[kGemmBN * kGemmRow];
    __shared__ __align__(16) float dxs[kGemmKC][BM];  // [block][row]: a lane's 4 rows are one 16-byte read
    __shared__ float dws[kGemmKC][kGemmBN];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int n0 = blockIdx.x * kGemmBN, m0 = blockIdx.y * BM;
    const int nb = K >> 5;
    const int mrows = min(BM, M - m0), nrows = min(kGemmBN, N - n0);
    // waves as a WR x WC grid over the tile: wave (wr, wc) owns MTW 16-row
    // and NTW 16-column sub-tiles (fewer operand and scale reads per MFMA
    // than one column strip per wave when the tile is tall)
    constexpr int WR = BM >= 64 ? 4 : BM / 16, WC = 4 / WR;
    constexpr int MTW = BM / 16 / WR, NTW = 4 / WC;
    const int wrow = w / WC, wc = w % WC;
    constexpr int PPR = 2 * kGemmKC;               // 16-byte pieces of a row per chunk
    constexpr int XP = (BM * PPR + 255) / 256;     // 16-byte X pieces per lane per chunk
    constexpr int WP = kGemmBN * PPR / 256;        // 16-byte W pieces per lane per chunk
    constexpr int DXP = (BM * kGemmKC + 255) / 256;
    constexpr int DWP = kGemmKC * kGemmBN / 256;
    // the tile's rows of X and W, their scales (n0 is a multiple of 8, so the
    // scale groups of W rows n0.. are contiguous)
    const __amdgpu_buffer_rsrc_t bx = buffer_of(xq + int64_t(m0) * K, uint32_t(mrows) * uint32_t(K));
    const __amdgpu_buffer_rsrc_t bw = buffer_of(wq + int64_t(n0) * K, uint32_t(nrows) * uint32_t(K));
    const __amdgpu_buffer_rsrc_t bdx = buffer_of(xd + int64_t(m0) * nb, uint32_t(mrows) * uint32_t(nb) * 4u);
    const __amdgpu_buffer_rsrc_t bdw = buffer_of(wd + scale_index(n0, 0, nb), uint32_t((min(kGemmBN, Npad - n0) + 7) / 8) * uint32_t(nb) * 16u);
    float acc[MTW][NTW][4];
#pragma unroll
    for (int i = 0; i < MTW; ++i)
#pragma unroll
        for (int j = 0; j < NTW; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.f;

    int4 xr[XP], wr[WP];
    float dxr[DXP], dwr[DWP];
    // chunk b0's bytes (16-byte piece c < 2*kc of each row) and scales into registers
    auto fetch = [&](int b0) {
        const int kc = min(kGemmKC, nb - b0);
#pragma unroll
        for (int q = 0; q < XP; ++q) {
            const int e = tid + 256 * q, r = e / PPR, c = e % PPR;
            xr[q] = load_b128(bx, e < BM * PPR && c < 2 * kc ? uint32_t(r) * uint32_t(K) + uint32_t(b0) * 32u + uint32_t(c) * 16u : kOOB);
        }
#pragma unroll
        for (int q = 0; q < WP; ++q) {
            const int e = tid + 256 * q, r = e / PPR, c = e % PPR;
            wr[q] = load_b128(bw, c < 2 * kc ? uint32_t(r) * uint32_t(K) + uint32_t(b0) * 32u + uint32_t(c) * 16u : kOOB);
        }
#pragma unroll
        for (int q = 0; q < DXP; ++q) {
            const int e = tid + 256 * q, r = e / kGemmKC, bb = e % kGemmKC;
            dxr[q] = load_f32(bdx, e < BM * kGemmKC && bb < kc ? (uint32_t(r) * uint32_t(nb) + uint32_t(b0 + bb)) * 4u : kOOB);
        }
#pragma unroll
        for (int q = 0; q < DWP; ++q) {
            const int e = tid + 256 * q, bb = e / kGemmBN, c = e % kGemmBN;
            const uint32_t off = (uint32_t(c >> 3) * uint32_t(nb) + uint32_t(b0 + bb)) * 16u + uint32_t(c & 7) * 2u;
            dwr[q] = half_bits_to_f32(uint16_t(__builtin_amdgcn_raw_buffer_load_b16(bdw, bb < kc ? off : kOOB, 0, 0)));
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int q = 0; q < XP; ++q) {
            const int e = tid + 256 * q;
            if (e < BM * PPR) *reinterpret_cast<int4*>(Xs + (e / PPR) * kGemmRow + (e % PPR) * 16) = xr[q];
        }
#pragma unroll
        for (int q = 0; q < WP; ++q) {
            const int e = tid + 256 * q;
            *reinterpret_cast<int4*>(Ws + (e / PPR) * kGemmRow + (e % PPR) * 16) = wr[q];
        }
#pragma unroll
        for (int q = 0; q < DXP; ++q) {
            const int e = tid + 256 * q;
            if (e < BM * kGemmKC) dxs[e % kGemmKC][e / kGemmKC] = dxr[q];
        }
#pragma unroll
        for (int q = 0; q < DWP; ++q) {
            const int e = tid + 256 * q;
            dws[e / kGemmBN][e % kGemmBN] = dwr[q];
        }
    };

    fetch(0);
    for (int b0 = 0; b0 < nb; b0 += kGemmKC) {
        const int kc = min(kGemmKC, nb - b0);  // blocks in this chunk
        stage();
        __syncthreads();
        if (b0 + kGemmKC < nb) fetch(b0 + kGemmKC);  // in flight during this chunk's compute
        for (int bb = 0; bb < kc; ++bb) {
            const int koff = bb * 32 + (lane >> 4) * 8;
            long bop[NTW];
            float dw[NTW];
#pragma unroll
            for (int j = 0; j < NTW; ++j) {
                const int n_l = 16 * (wc * NTW + j) + (lane & 15);
                bop[j] = *reinterpret_cast<const long*>(Ws + n_l * kGemmRow + koff);
                dw[j] = dws[bb][n_l];
            }
#pragma unroll
            for (int i = 0; i < MTW; ++i) {
                const int mi = wrow * MTW + i;
                const long aop = *reinterpret_cast<const long*>(Xs + (16 * mi + (lane & 15)) * kGemmRow + koff);
                const float4 dx4 = *reinterpret_cast<const float4*>(&dxs[bb][16 * mi + (lane >> 4) * 4]);
#pragma unroll
                for (int j = 0; j < NTW; ++j) {
                    const v4i_t zero = {0, 0, 0, 0};
                    const v4i_t c = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, bop[j], zero, 0, 0, 0);
                    acc[i][j][0] = acc[i][j][0] + float(c[0]) * (dw[j] * dx4.x);
                    acc[i][j][1] = acc[i][j][1] + float(c[1]) * (dw[j] * dx4.y);
                    acc[i][j][2] = acc[i][j][2] + float(c[2]) * (dw[j] * dx4.z);
                    acc[i][j][3] = acc[i][j][3] + float(c[3]) * (dw[j] * dx4.w);
                }
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < MTW; ++i)
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            const int n = n0 + 16 * (wc * NTW + j) + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + 16 * (wrow * MTW + i) + (lane >> 4) * 4 + r;
                if (m < M && n < N) {
                    const int64_t o = int64_t(m) * N + n;
                    if constexpr (EPI == kEpiResidual)
                        y[o] = resid[o] + acc[i][j][r];
                    else
                        y[o] = acc[i][j][r];
                }
            }
        }
}

// ---------------------------------------------------------------------------
// Skinny GEMM, 1 < M <= 16 activation rows (batched decode): the weights are
// streamed once, as in the GEMV, and each block's int32 sums come from the
// int8 MFMA 16x16x32 (16 activation rows x 16 weight rows x 32 k).
//
// A workgroup of NW waves owns a contiguous range of 16-row weight groups
// and walks each in rounds of kSkRound blocks; each wave takes kSkRound / NW
// blocks of a round (more waves for fewer groups: the rounds are what take
// the time). A lane reads 16 bytes of a block pair (b, b+1): lane group q = 0
// holds bytes 0-15 of b, q = 1 bytes 16-31 of b, q = 2 and 3 the same of
// b+1, for weight row n = lane % 16 and activation row m = lane % 16. The
// MFMA sums over all four lane groups, so each block takes two MFMAs (the
// low, then the high 8 bytes of each lane) with the activation operand
// zeroed in the lane groups that hold the other block: the int32 result is
// exactly that block's dot product. A lane turns its 4 results (rows
// m = 4q + r of column n) into terms float(sumi) * (d_w * d_x) in shared
// memory; after a barrier lane p = 16 m + n adds the round's terms to its
// chain in block order (the reference's order), and after the last round
// stores y. The terms alternate between two halves of shared memory, so the
// next round's MFMAs run while the chains read this one (one barrier a
// round), and each lane issues the next round's loads as soon as it has
// consumed this round's: deeper rings (2, 3, 4 rounds in flight) measured
// slower at batch 16.
// ---------------------------------------------------------------------------
constexpr int kSkRound = 32;                   // blocks per round
constexpr int kSkMaxK = 16384;
constexpr int kSkRing = 1;                     // steps (group, round) in flight per lane
// Every global access of the skinny kernel is a raw buffer access (kOOB),
// so invalid rows, blocks and padded steps need no branch.

template <int P>  // block pairs per wave per round
struct SkLoads {
    v4b_t w[P];
    v4b_t x[P];
    uint32_t d;  // two weight scales of the wave's blocks x 16 rows (see load)
};

__device__ __forceinline__ long lo64(v4b_t v) { return long((uint64_t(uint32_t(v.y)) << 32) | uint32_t(v.x)); }
__device__ __forceinline__ long hi64(v4b_t v) { return long((uint64_t(uint32_t(v.w)) << 32) | uint32_t(v.z)); }

template <int EPI, int NW>
__global__ __launch_bounds__(64 * NW) void gemm_q8_skinny_kernel(const int8_t* __restrict__ wq, const uint16_t* __restrict__ wd, const int8_t* __restrict__ xq, const float* __restrict__ xd, float* __restrict__ y, const float* __restrict__ resid, int M, int N, int Npad, int K) {
    // [step parity][block of the round][16 m + n]: step s writes half s % 2 while the
    // chains may still read the other half, so a step needs one barrier
    __shared__ __align__(16) float terms2[2][kSkRound][256];
    extern __shared__ __align__(16) float dxs_raw[];        // [block][m] activation scales, 0 for m >= M
    float (*dxs)[16] = reinterpret_cast<float (*)[16]>(dxs_raw);
    constexpr int kSkWaveBlocks = kSkRound / NW;  // blocks per wave per round
    constexpr int kSkPairs = kSkWaveBlocks / 2;   // 16-byte loads per lane per round
    static_assert(NW >= 4 && kSkPairs >= 1, "4 to 16 waves");
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int q = lane >> 4, c = lane & 15;
    const int nb = K >> 5, rounds = (nb + kSkRound - 1) / kSkRound;
    const int groups = (N + 15) >> 4, G = gridDim.x;
    const int g_begin = int(int64_t(groups) * blockIdx.x / G), g_end = int(int64_t(groups) * (blockIdx.x + 1) / G);
    const int steps = (g_end - g_begin) * rounds;
    const int steps_pad = (steps + kSkRing - 1) / kSkRing * kSkRing;
    const __amdgpu_buffer_rsrc_t bw = buffer_of(wq, uint32_t(N) * uint32_t(K));
    const __amdgpu_buffer_rsrc_t bx = buffer_of(xq, uint32_t(M) * uint32_t(K));
    const __amdgpu_buffer_rsrc_t bd = buffer_of(wd, uint32_t(nb) * uint32_t(Npad) * 2u);
    for (int e = tid; e < nb * 16; e += 64 * NW) {
        const int b = e >> 4, m = e & 15;
        dxs[b][m] = m < M ? xd[int64_t(m) * nb + b] : 0.f;
    }

    // the loads of one step (group, round) for this lane; past the last step
    // (padding) every offset is out of range
    auto load = [&](int step, SkLoads<kSkPairs>& L) {
        const int g = g_begin + step / rounds, r = step % rounds;
        const int n = g * 16 + c;
        const int b0 = r * kSkRound + wv * kSkWaveBlocks;
        const bool on = step < steps && b0 < nb;  // nb % 8 == 0: a wave's blocks are all in or all out
        const bool wrow = on && n < N, xrow = on && c < M;
#pragma unroll
        for (int i = 0; i < kSkPairs; ++i) {
            const uint32_t off = uint32_t(b0 + 2 * i) * 32u + 16u * uint32_t(q);
            L.w[i] = __builtin_amdgcn_raw_buffer_load_b128(bw, wrow ? uint32_t(n) * uint32_t(K) + off : kOOB, 0, 0);
            L.x[i] = __builtin_amdgcn_raw_buffer_load_b128(bx, xrow ? uint32_t(c) * uint32_t(K) + off : kOOB, 0, 0);
        }
        // the wave's 8 x 16 scales in one dword per lane: lane 8j + c' holds
        // rows 2c', 2c'+1 of block b0 + j (adjacent in their 8-row group);
        // compute() fetches its own with ds_bpermute
        const int j = lane >> 3, c2 = 2 * (lane & 7);
        const bool drow = on && g * 16 + c2 < N;
        L.d = uint32_t(__builtin_amdgcn_raw_buffer_load_b32(bd, drow ? uint32_t(scale_index(g * 16 + c2, b0 + j, nb)) * 2u : kOOB, 0, 0));
    };

    // a ring of kSkRing steps in flight; slot k is refilled with step s + kSkRing
    // as soon as step s has been consumed
    SkLoads<kSkPairs> ring[kSkRing];
#pragma unroll
    for (int k = 0; k < kSkRing; ++k) load(k, ring[k]);
    __syncthreads();  // dxs
    float acc = 0.f;
    for (int s0 = 0; s0 < steps_pad; s0 += kSkRing) {
#pragma unroll
        for (int k = 0; k < kSkRing; ++k) {
            const int s = s0 + k;
            const int g = g_begin + s / rounds, r = s % rounds;
            const int b0 = r * kSkRound + wv * kSkWaveBlocks;
            float (*terms)[256] = terms2[s & 1];
            if (b0 < nb) {
                const bool first = q < 2;  // lane groups 0, 1 hold block b; 2, 3 hold block b+1
#pragma unroll
                for (int i = 0; i < kSkPairs; ++i) {
                    const long wl = lo64(ring[k].w[i]), wh = hi64(ring[k].w[i]);
                    const long xl = lo64(ring[k].x[i]), xh = hi64(ring[k].x[i]);
                    const v4i_t zero = {0, 0, 0, 0};
                    v4i_t c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(first ? xl : 0L, wl, zero, 0, 0, 0);
                    c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(first ? xh : 0L, wh, c0, 0, 0, 0);
                    v4i_t c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(first ? 0L : xl, wl, zero, 0, 0, 0);
                    c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(first ? 0L : xh, wh, c1, 0, 0, 0);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const int jb = wv * kSkWaveBlocks + 2 * i + h;  // block within the round
                        const v4i_t& cc = h ? c1 : c0;
                        const int jj = 2 * i + h;
                        const uint32_t two = uint32_t(__builtin_amdgcn_ds_bpermute(4 * (8 * jj + (c >> 1)), int(ring[k].d)));
                        const float dw = half_bits_to_f32(uint16_t((c & 1) ? (two >> 16) : (two & 0xFFFFu)));
                        const float4 dx = *reinterpret_cast<const float4*>(&dxs[b0 + 2 * i + h][4 * q]);
                        // [m][n] with n = lane % 16 fastest: consecutive lanes,
                        // consecutive banks
                        terms[jb][(4 * q + 0) * 16 + c] = float(cc[0]) * (dw * dx.x);
                        terms[jb][(4 * q + 1) * 16 + c] = float(cc[1]) * (dw * dx.y);
                        terms[jb][(4 * q + 2) * 16 + c] = float(cc[2]) * (dw * dx.z);
                        terms[jb][(4 * q + 3) * 16 + c] = float(cc[3]) * (dw * dx.w);
                    }
                }
            }
            load(s + kSkRing, ring[k]);
            __syncthreads();
            const int kc = min(kSkRound, nb - r * kSkRound);
            if (tid < 256) {  // the chains: lane tid = 16 m + n, every read first
                float tv[kSkRound];
#pragma unroll
                for (int j = 0; j < kSkRound; ++j) tv[j] = terms[j][tid];
#pragma unroll
                for (int j = 0; j < kSkRound; ++j)
                    if (j < kc) acc = acc + tv[j];
            }
            const bool last = r == rounds - 1;
            const int n = g * 16 + (tid & 15), m = tid >> 4;
            if (tid < 256 && last && s < steps && m < M && n < N) {
                const int64_t o = int64_t(m) * N + n;
                if constexpr (EPI == kEpiResidual)
                    y[o] = resid[o] + acc;  // h = x + m (nm/src/qwen35.hpp:321)
                else
                    y[o] = acc;
            }
            acc = last ? 0.f : acc;
        }
    }
}

// The same for tall matrices (many 16-row groups): every workgroup is one wave and owns a contiguous range of 16-row weight
// groups, walked in rounds of kSkwRound blocks with kSkwRing rounds of loads in
// flight. A lane reads 16 bytes of a block pair (b, b+1) of weight row
// n = lane % 16 and the same bytes of activation row m = lane % 16: lane group
// q = 0 holds bytes 0-15 of b, q = 1 bytes 16-31 of b, q = 2 and 3 the same of
// b+1. The MFMA sums over all four lane groups, so each block takes two MFMAs
// (the low, then the high 8 bytes of each lane) with the activation operand
// zeroed in the lane groups that hold the other block: the int32 result is
// exactly that block's dot product, and lane (q, c) receives it for weight
// rows n = 4q + r (r = 0..3) and activation row m = c. The lane turns them
// into terms float(sumi) * (d_w * d_x) and adds each to the chain of its
// (n, m) output in block order (the reference's order): four independent
// chains per lane, all in registers, and no barrier in the loop.
// MG > 1 (M up to 16 MG): a workgroup of MG waves walks the same range, wave
// w taking activation rows 16w .. 16w+15; the waves read the same weights at
// about the same time, so HBM delivers each weight byte once and the other
// waves' reads hit the caches.
// ---------------------------------------------------------------------------
constexpr int kSkwRound = 8;                    // blocks per round
constexpr int kSkwPairs = kSkwRound / 2;         // 16-byte weight (and activation) loads per lane per round
constexpr int kSkwMaxK = 16384;
constexpr int kSkwRing = 4;                     // rounds in flight per wave
// Every global access of the skinny kernel is a raw buffer access (kOOB),
// so invalid rows, blocks and padded steps need no branch.

struct SkwLoads {
    v4b_t w[kSkwPairs];
    v4b_t x[kSkwPairs];
    v4b_t d;                   // weight scales: 8 rows (group q / 2 of the 16) of block c < kSkwRound of the round
    v4b_t dx[kSkwRound / 4];    // activation scales of row c for the round's blocks
};


template <int EPI, int MG>
__global__ __launch_bounds__(64 * MG) void gemm_q8_skinny_wave_kernel(const int8_t* __restrict__ wq, const uint16_t* __restrict__ wd, const int8_t* __restrict__ xq, const float* __restrict__ xd, float* __restrict__ y, const float* __restrict__ resid, int M, int N, int Npad, int K) {
    __shared__ __align__(16) uint16_t dws_all[MG][kSkwRing][2][kSkwRound][8];  // per wave, a round's weight scales: [8-row group][block][row]
    const int lane = threadIdx.x & 63, q = lane >> 4, c = lane & 15;
    const int m = 16 * int(threadIdx.x >> 6) + c;  // the lane's activation row
    auto& dws = dws_all[threadIdx.x >> 6];
    const int nb = K >> 5, rounds = nb / kSkwRound;
    const int groups = (N + 15) >> 4, G = gridDim.x;
    const int g_begin = int(int64_t(groups) * blockIdx.x / G), g_end = int(int64_t(groups) * (blockIdx.x + 1) / G);
    const int steps = (g_end - g_begin) * rounds;
    const int steps_pad = (steps + kSkwRing - 1) / kSkwRing * kSkwRing;
    const __amdgpu_buffer_rsrc_t bw = buffer_of(wq, uint32_t(N) * uint32_t(K));
    const __amdgpu_buffer_rsrc_t bx = buffer_of(xq, uint32_t(M) * uint32_t(K));
    const __amdgpu_buffer_rsrc_t bd = buffer_of(wd, uint32_t(nb) * uint32_t(Npad) * 2u);
    const __amdgpu_buffer_rsrc_t bxd = buffer_of(xd, uint32_t(M) * uint32_t(nb) * 4u);

    // the loads of one step (group, round) for this lane; past the last step
    // (padding) every offset is out of range
    auto load = [&](int step, SkwLoads& L) {
        const int g = g_begin + step / rounds, r = step % rounds;
        const bool on = step < steps;
        const int n = g * 16 + c, b0 = r * kSkwRound;
        const bool wrow = on && n < N, xrow = on && m < M;
#pragma unroll
        for (int i = 0; i < kSkwPairs; ++i) {
            const uint32_t off = uint32_t(b0 + 2 * i) * 32u + 16u * uint32_t(q);
            L.w[i] = __builtin_amdgcn_raw_buffer_load_b128(bw, wrow ? uint32_t(n) * uint32_t(K) + off : kOOB, 0, 0);
            L.x[i] = __builtin_amdgcn_raw_buffer_load_b128(bx, xrow ? uint32_t(m) * uint32_t(K) + off : kOOB, 0, 0);
        }
        // 8 rows x block b0 + c of 8-row group 2g + q / 2 (16 bytes; lanes q
        // and q ^ 1 read the same)
        const bool drow = on && c < kSkwRound && g * 16 + 8 * (q >> 1) < N;
        L.d = __builtin_amdgcn_raw_buffer_load_b128(bd, drow ? uint32_t(scale_index(g * 16 + 8 * (q >> 1), b0 + c, nb)) * 2u : kOOB, 0, 0);
#pragma unroll
        for (int i = 0; i < kSkwRound / 4; ++i)
            L.dx[i] = __builtin_amdgcn_raw_buffer_load_b128(bxd, xrow ? (uint32_t(m) * uint32_t(nb) + uint32_t(b0 + 4 * i)) * 4u : kOOB, 0, 0);
    };

    SkwLoads ring[kSkwRing];
#pragma unroll
    for (int k = 0; k < kSkwRing; ++k) load(k, ring[k]);

    float acc[4] = {0.f, 0.f, 0.f, 0.f};  // outputs (n = g*16 + 4q + r, m)
    for (int s0 = 0; s0 < steps_pad; s0 += kSkwRing) {
#pragma unroll
        for (int k = 0; k < kSkwRing; ++k) {
            const int s = s0 + k;
            const int g = g_begin + s / rounds, r = s % rounds;
            // the round's weight scales through shared memory: lane (q, c < kSkwRound)
            // stores block c's 8 rows of its group; block j's rows 4q .. 4q+3
            // are then 8 bytes at [q / 2][j][4 (q % 2)]
            // (one wave: its shared-memory accesses take effect in order)
            if ((q & 1) == 0 && c < kSkwRound) *reinterpret_cast<v4b_t*>(&dws[k][q >> 1][c][0]) = ring[k].d;
            const bool first = q < 2;  // lane groups 0, 1 hold block b; 2, 3 hold block b+1
#pragma unroll
            for (int i = 0; i < kSkwPairs; ++i) {
                const long wl = lo64(ring[k].w[i]), wh = hi64(ring[k].w[i]);
                const long xl = lo64(ring[k].x[i]), xh = hi64(ring[k].x[i]);
                const v4i_t zero = {0, 0, 0, 0};
                v4i_t c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(wl, first ? xl : 0L, zero, 0, 0, 0);
                c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(wh, first ? xh : 0L, c0, 0, 0, 0);
                v4i_t c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(wl, first ? 0L : xl, zero, 0, 0, 0);
                c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(wh, first ? 0L : xh, c1, 0, 0, 0);
                const v4b_t dx4 = ring[k].dx[i / 2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int j = 2 * i + h;  // block within the round
                    const v4i_t& cc = h ? c1 : c0;
                    const uint2 d2 = *reinterpret_cast<const uint2*>(&dws[k][q >> 1][j][4 * (q & 1)]);
                    const float dx = __builtin_bit_cast(float, (j & 3) == 0 ? dx4.x : (j & 3) == 1 ? dx4.y : (j & 3) == 2 ? dx4.z : dx4.w);
                    acc[0] = acc[0] + float(cc[0]) * (half_bits_to_f32(uint16_t(d2.x & 0xFFFFu)) * dx);
                    acc[1] = acc[1] + float(cc[1]) * (half_bits_to_f32(uint16_t(d2.x >> 16)) * dx);
                    acc[2] = acc[2] + float(cc[2]) * (half_bits_to_f32(uint16_t(d2.y & 0xFFFFu)) * dx);
                    acc[3] = acc[3] + float(cc[3]) * (half_bits_to_f32(uint16_t(d2.y >> 16)) * dx);
                }
                __builtin_amdgcn_sched_barrier(0);  // pair by pair: few MFMA results live at once
            }
            // the slot's next loads after its last use (keeps one set of ring registers)
            __builtin_amdgcn_sched_barrier(0);
            load(s + kSkwRing, ring[k]);
            __builtin_amdgcn_sched_barrier(0);
            if (r == rounds - 1 && s < steps) {  // the group's outputs
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const int n = g * 16 + 4 * q + rr;
                    if (n < N && m < M) {
                        const int64_t o = int64_t(m) * N + n;
                        if constexpr (EPI == kEpiResidual)
                            y[o] = resid[o] + acc[rr];  // h = x + m (nm/src/qwen35.hpp:321)
                        else
                            y[o] = acc[rr];
                    }
                    acc[rr] = 0.f;
                }
            }
        }
    }
}

// The tall form with the activation rows in shared memory: a workgroup of NW
// waves copies the 16 activation rows (K <= 4096 bytes each) and their
// scales into shared memory once, then each wave walks its own range of
// 16-row weight groups exactly as gemm_q8_skinny_wave_kernel does, but reads
// only the weights and their scales from memory: 5 load instructions per
// 4 KB of weights instead of 11. The copy's loads are issued first and the
// weight ring right after them, so both are in flight at once.
constexpr int kSklMaxK = 4096;
constexpr int kSklRowPad = 16;  // activation row stride K + 16: 16 lanes' 16-byte reads hit distinct banks
constexpr int kSklDxPad = 4;    // activation scale row stride nb + 4 (likewise)
constexpr int kSklRing = 2;     // rounds in flight per wave (deeper rings measured slower)

__host__ __device__ inline size_t skl_shared_bytes(int nw, int K) {
    const int nb = K / 32;
    return size_t(16) * size_t(K + kSklRowPad) + size_t(16) * size_t(nb + kSklDxPad) * 4 + size_t(nw) * kSklRing * 2 * kSkwRound * 8 * 2;
}

// EPI == kEpiSwigluQuant (NW = 8; rows interleaved as 64-row units [32 gate
// | 32 up], N % 64 == 0): workgroup x owns units 2x and 2x + 1, wave w the
// 16-row group w % 4 of unit 2x + w / 4; after the last round the four waves
// of a unit exchange their chains through shared memory and the unit's first
// wave forms silu(gate) * up (nm/src/components.hpp:300-304) and the Q8_0
// blocks of the down projection's input (quantize_row_q8_0) into y, read as
// int8 [M][N/2] then fp32 scales [M][N/64] -- the values swiglu_quant_kernel
// forms from the stored gate and up rows.
template <int EPI, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(4))) void gemm_q8_skinny_lds_kernel(const int8_t* __restrict__ wq, const uint16_t* __restrict__ wd, const int8_t* __restrict__ xq, const float* __restrict__ xd, float* __restrict__ y, const float* __restrict__ resid, int M, int N, int Npad, int K) {
    constexpr bool SW = EPI == kEpiSwigluQuant;
    static_assert(!SW || NW % 4 == 0, "whole 4-wave units per workgroup");
    extern __shared__ __align__(16) uint8_t skl_smem[];
    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63, q = lane >> 4, c = lane & 15;
    const int nb = K >> 5, rounds = nb / kSkwRound;
    const int rowb = K + kSklRowPad, dxrow = nb + kSklDxPad;
    int8_t* xs = reinterpret_cast<int8_t*>(skl_smem);                       // [16][K + 16]
    float* dxs = reinterpret_cast<float*>(skl_smem + 16 * rowb);             // [16][nb + 4]
    uint16_t (*dws)[2][kSkwRound][8] = reinterpret_cast<uint16_t (*)[2][kSkwRound][8]>(dxs + 16 * dxrow) + wv * kSklRing;  // this wave's [ring][8-row group][block][row]
    const int groups = (N + 15) >> 4, G = gridDim.x;
    const int wg_begin = int(int64_t(groups) * blockIdx.x / G), wg_end = int(int64_t(groups) * (blockIdx.x + 1) / G);
    const int sw_unit = (NW / 4) * int(blockIdx.x) + wv / 4;  // SW: this wave's unit
    const bool sw_live = sw_unit < groups / 4;
    const int g_begin = SW ? 4 * sw_unit + (wv & 3) : wg_begin + (wg_end - wg_begin) * wv / NW;
    const int g_end = SW ? (sw_live ? g_begin + 1 : g_begin) : wg_begin + (wg_end - wg_begin) * (wv + 1) / NW;
    const int steps = (g_end - g_begin) * rounds;
    const int steps_pad = (steps + kSklRing - 1) / kSklRing * kSklRing;
    const __amdgpu_buffer_rsrc_t bw = buffer_of(wq, uint32_t(N) * uint32_t(K));
    const __amdgpu_buffer_rsrc_t bx = buffer_of(xq, uint32_t(M) * uint32_t(K));
    const __amdgpu_buffer_rsrc_t bd = buffer_of(wd, uint32_t(nb) * uint32_t(Npad) * 2u);
    const __amdgpu_buffer_rsrc_t bxd = buffer_of(xd, uint32_t(M) * uint32_t(nb) * 4u);

    struct Ring {
        v4b_t w[kSkwPairs];
        v4b_t d;
    };
    auto load = [&](int step, Ring& L) {
        const int g = g_begin + step / rounds, r = step % rounds;
        const bool on = step < steps;
        const int n = g * 16 + c, b0 = r * kSkwRound;
        const bool wrow = on && n < N;
#pragma unroll
        for (int i = 0; i < kSkwPairs; ++i) {
            const uint32_t off = uint32_t(b0 + 2 * i) * 32u + 16u * uint32_t(q);
            L.w[i] = __builtin_amdgcn_raw_buffer_load_b128(bw, wrow ? uint32_t(n) * uint32_t(K) + off : kOOB, 0, 0);
        }
        const bool drow = on && c < kSkwRound && g * 16 + 8 * (q >> 1) < N;
        L.d = __builtin_amdgcn_raw_buffer_load_b128(bd, drow ? uint32_t(scale_index(g * 16 + 8 * (q >> 1), b0 + c, nb)) * 2u : kOOB, 0, 0);
    };
    // The activation rows and scales (rows >= M read as zeros) are loaded into
    // registers first and the weight ring after them: loads retire in order,
    // so the copy, on which the first MFMA waits, does not wait for the ring
    // (M = 16: 24576 x 4096 29.9 -> 28.3 us, 10240 x 4096 24.3 -> 21.5 us).
    constexpr int XP = (16 * kSklMaxK / 16 + 64 * NW - 1) / (64 * NW);  // 16-byte pieces per lane
    constexpr int DP = (16 * kSklMaxK / 32 + 64 * NW - 1) / (64 * NW);  // scales per lane
    const int cpr = K / 16;  // 16-byte pieces per row
    v4b_t xv[XP];
    float dv[DP];
#pragma unroll
    for (int u = 0; u < XP; ++u) {
        const int p = tid + u * 64 * NW, row = p / cpr, col = 16 * (p % cpr);
        xv[u] = __builtin_amdgcn_raw_buffer_load_b128(bx, p < 16 * cpr && row < M ? uint32_t(row) * uint32_t(K) + uint32_t(col) : kOOB, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < DP; ++u) {
        const int e = tid + u * 64 * NW, row = e / nb, b = e % nb;
        dv[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(bxd, e < 16 * nb && row < M ? uint32_t(row * nb + b) * 4u : kOOB, 0, 0));
    }
    __builtin_amdgcn_sched_barrier(0);
    Ring ring[kSklRing];
#pragma unroll
    for (int k = 0; k < kSklRing; ++k) load(k, ring[k]);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<kSklRing * (kSkwPairs + 1)>();  // the copy's loads have landed
#pragma unroll
    for (int u = 0; u < XP; ++u) {
        const int p = tid + u * 64 * NW, row = p / cpr, col = 16 * (p % cpr);
        if (p < 16 * cpr) *reinterpret_cast<v4b_t*>(xs + row * rowb + col) = xv[u];
    }
#pragma unroll
    for (int u = 0; u < DP; ++u) {
        const int e = tid + u * 64 * NW, row = e / nb, b = e % nb;
        if (e < 16 * nb) dxs[row * dxrow + b] = dv[u];
    }
    __syncthreads();

    const int8_t* xrow = xs + c * rowb + 16 * q;
    const float* dxr = dxs + c * dxrow;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};  // outputs (n = g*16 + 4q + r, m = c)
    float fin[4] = {0.f, 0.f, 0.f, 0.f};  // SW: the group's outputs
    for (int s0 = 0; s0 < steps_pad; s0 += kSklRing) {
#pragma unroll
        for (int k = 0; k < kSklRing; ++k) {
            const int s = s0 + k;
            const int g = g_begin + s / rounds, r = s % rounds;
            const int b0 = r * kSkwRound;
            if ((q & 1) == 0 && c < kSkwRound) *reinterpret_cast<v4b_t*>(&dws[k][q >> 1][c][0]) = ring[k].d;
            const bool first = q < 2;
            const float4 dxa = *reinterpret_cast<const float4*>(dxr + b0);
            const float4 dxb = *reinterpret_cast<const float4*>(dxr + b0 + 4);
#pragma unroll
            for (int i = 0; i < kSkwPairs; ++i) {
                const v4b_t xv = *reinterpret_cast<const v4b_t*>(xrow + (b0 + 2 * i) * 32);
                const long wl = lo64(ring[k].w[i]), wh = hi64(ring[k].w[i]);
                const long xl = lo64(xv), xh = hi64(xv);
                const v4i_t zero = {0, 0, 0, 0};
                v4i_t c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(wl, first ? xl : 0L, zero, 0, 0, 0);
                c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(wh, first ? xh : 0L, c0, 0, 0, 0);
                v4i_t c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(wl, first ? 0L : xl, zero, 0, 0, 0);
                c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(wh, first ? 0L : xh, c1, 0, 0, 0);
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int j = 2 * i + h;  // block within the round
                    const v4i_t& cc = h ? c1 : c0;
                    const uint2 d2 = *reinterpret_cast<const uint2*>(&dws[k][q >> 1][j][4 * (q & 1)]);
                    const float4& d4 = j < 4 ? dxa : dxb;
                    const float dx = (j & 3) == 0 ? d4.x : (j & 3) == 1 ? d4.y : (j & 3) == 2 ? d4.z : d4.w;
                    acc[0] = acc[0] + float(cc[0]) * (half_bits_to_f32(uint16_t(d2.x & 0xFFFFu)) * dx);
                    acc[1] = acc[1] + float(cc[1]) * (half_bits_to_f32(uint16_t(d2.x >> 16)) * dx);
                    acc[2] = acc[2] + float(cc[2]) * (half_bits_to_f32(uint16_t(d2.y & 0xFFFFu)) * dx);
                    acc[3] = acc[3] + float(cc[3]) * (half_bits_to_f32(uint16_t(d2.y >> 16)) * dx);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            __builtin_amdgcn_sched_barrier(0);
            load(s + kSklRing, ring[k]);
            __builtin_amdgcn_sched_barrier(0);
            if (r == rounds - 1 && s < steps) {
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const int n = g * 16 + 4 * q + rr;
                    if constexpr (SW) {
                        fin[rr] = acc[rr];
                    } else if (n < N && c < M) {
                        const int64_t o = int64_t(c) * N + n;
                        if constexpr (EPI == kEpiResidual)
                            y[o] = resid[o] + acc[rr];
                        else
                            y[o] = acc[rr];
                    }
                    acc[rr] = 0.f;
                }
            }
        }
    }
    if constexpr (SW) {
        // lane (q, c) of group j holds unit rows 16 j + 4 q + rr for activation
        // row c: j = 0, 1 the gates of FF offsets 4q + rr and 16 + 4q + rr, j = 2,
        // 3 the up values of the same offsets
        float4* xg = reinterpret_cast<float4*>(skl_smem + skl_shared_bytes(NW, K));  // [NW][64]
        xg[wv * 64 + lane] = make_float4(fin[0], fin[1], fin[2], fin[3]);
        __syncthreads();
        if ((wv & 3) == 0 && sw_live) {
            const float4 g1 = xg[(wv + 1) * 64 + lane], u0 = xg[(wv + 2) * 64 + lane], u1 = xg[(wv + 3) * 64 + lane];
            const float v[8] = {silu_f32(fin[0]) * u0.x, silu_f32(fin[1]) * u0.y, silu_f32(fin[2]) * u0.z, silu_f32(fin[3]) * u0.w,
                                silu_f32(g1.x) * u1.x, silu_f32(g1.y) * u1.y, silu_f32(g1.z) * u1.z, silu_f32(g1.w) * u1.w};
            // the 32-value block of (row c, unit) sits in lanes c, c + 16, c + 32, c + 48
            float amax = 0.f;
#pragma unroll
            for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(v[k]));
            amax = fmaxf(amax, __shfl_xor(amax, 16));
            amax = fmaxf(amax, __shfl_xor(amax, 32));
            const float d = amax / 127.f;
            const float id = d != 0.f ? 1.f / d : 0.f;
            int packed[2] = {0, 0};
#pragma unroll
            for (int k = 0; k < 8; ++k) packed[k / 4] |= (int(roundf(v[k] * id)) & 0xFF) << (8 * (k % 4));
            if (c < M) {
                const int FF = N / 2;
                int8_t* qs = reinterpret_cast<int8_t*>(y);
                int* row = reinterpret_cast<int*>(qs + int64_t(c) * FF + 32 * sw_unit);
                row[q] = packed[0];      // offsets 4q .. 4q + 3
                row[4 + q] = packed[1];  // offsets 16 + 4q .. 16 + 4q + 3
                if (q == 0) reinterpret_cast<float*>(qs + int64_t(M) * FF)[int64_t(c) * (FF / 32) + sw_unit] = half_bits_to_f32(fp32_to_fp16_ref(d));
            }
        }
    }
}

namespace {
template <int BM>
void gemm_dispatch(int epi, const int8_t* wq, const uint16_t* wd, const int8_t* xq, const float* xd, float* y, const float* resid, int M, int N, int Npad, int K, hipStream_t s) {
    const dim3 grid(unsigned((N + kGemmBN - 1) / kGemmBN), unsigned((M + BM - 1) / BM));
    if (epi == kEpiResidual)
        hipLaunchKernelGGL((gemm_q8_kernel<BM, kEpiResidual>), grid, dim3(256), 0, s, wq, wd, xq, xd, y, resid, M, N, Npad, K);
    else
        hipLaunchKernelGGL((gemm_q8_kernel<BM, kEpiStore>), grid, dim3(256), 0, s, wq, wd, xq, xd, y, resid, M, N, Npad, K);
}
}  // namespace

int gemm_q8_plan(int64_t M, int64_t N, int64_t K) {
    const int64_t groups = (N + 15) / 16;
    if (M <= 16 && groups >= 2 * device_cus() && K % (32 * kSkwRound) == 0 && K <= kSkwMaxK && N * K < (int64_t(1) << 31))
        return K <= kSklMaxK && groups >= 4 * device_cus() ? kGemmPlanSkinnyLds : kGemmPlanSkinnyWave;
    if (M <= 16 && K % 256 == 0 && K <= kSkMaxK && N * K < (int64_t(1) << 31)) return kGemmPlanSkinnyShared;
    // 16 < M <= 64 with at most a group per CU, where the row tiles leave
    // most CUs with one workgroup: the weights streamed once, every wave a
    // 16-row activation group (M = 64: 4096 x 4096 27.6 -> 23.2 us, 12288 x
    // 4096 77.6 -> 59.0 us). With more groups the waves' activation reads
    // load the caches more than the tiles do (151936 rows: 706 us against
    // 223; 12288 rows: 79 against 32).
    if (M > 16 && M <= 64 && groups <= device_cus() && K % (32 * kSkwRound) == 0 && K <= kSkwMaxK && N * K < (int64_t(1) << 31)) return kGemmPlanSkinnyWave4;
    // the tallest tile that still gives every CU two workgroups (the fp32
    // term work per CU is the same; more workgroups hide more latency)
    const int64_t tiles_n = (N + kGemmBN - 1) / kGemmBN, want = 2 * device_cus();
    auto grid_of = [&](int64_t bm) { return tiles_n * ((M + bm - 1) / bm); };
    if (M > 64 && grid_of(128) >= want) return 128;
    if (M > 32 && grid_of(64) >= want) return 64;
    if (M > 16 && grid_of(32) >= want) return 32;
    return 16;
}

constexpr int kSwNW = 8;  // waves per workgroup of the SwiGLU form: two 64-row units (one unit per four-wave workgroup: 3.59k -> 3.35k tok/s at B = 16)

bool launch_gemm_q8_swiglu(const void* packed, const void* act, void* out, int64_t M, int64_t N, int64_t K, hipStream_t s) {
    if (gemm_q8_plan(M, N, K) != kGemmPlanSkinnyLds || N % 64 != 0) return false;
    constexpr int NW = kSwNW;
    const unsigned grid = unsigned((N / 64 + NW / 4 - 1) / (NW / 4));
    const size_t smem = skl_shared_bytes(NW, int(K)) + NW * 64 * 16;
    auto kernel = gemm_q8_skinny_lds_kernel<kEpiSwigluQuant, NW>;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 64 * NW, smem) != hipSuccess || int64_t(per_cu) * device_cus() < grid) return false;
    const int8_t* wq = static_cast<const int8_t*>(packed);
    const uint16_t* wd = reinterpret_cast<const uint16_t*>(wq + N * K);
    const int8_t* xq = static_cast<const int8_t*>(act);
    const float* xd = reinterpret_cast<const float*>(xq + M * K);
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(64 * NW), smem, s, wq, wd, xq, xd, static_cast<float*>(out), nullptr, int(M), int(N), int(packed_rows_pad(N)), int(K));
    return true;
}

void launch_gemm_q8(const void* packed, const void* act, float* y, const float* resid, int64_t M, int64_t N, int64_t K, int epi, hipStream_t s) {
    const int8_t* wq = static_cast<const int8_t*>(packed);
    const uint16_t* wd = reinterpret_cast<const uint16_t*>(wq + N * K);
    const int8_t* xq = static_cast<const int8_t*>(act);
    const float* xd = reinterpret_cast<const float*>(xq + M * K);
    const int Npad = int(packed_rows_pad(N));
    const int64_t groups = (N + 15) / 16;
    // as many workgroups as are resident at once: a second wave of
    // workgroups would run after the first
    auto grid_for = [&](auto kernel, int threads, size_t smem) {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, smem) != hipSuccess || per_cu <= 0) per_cu = 1;
        return unsigned(std::min<int64_t>(int64_t(per_cu) * device_cus(), groups));
    };
    switch (gemm_q8_plan(M, N, K)) {
    case kGemmPlanSkinnyLds: {
        // tall at K <= 4096 with 4 or more groups per CU: the activations in
        // shared memory, read from L2 once per workgroup instead of once per
        // wave (at the same rows every round those reads keep the L2 busy on
        // a few channels), each wave a range of at least one group, 6 waves per
        // workgroup below 8 groups per CU and 8 above (M = 16: 24576 x 4096
        // 35 -> 27 us, 16448 x 4096 30-34 -> 21 us, the LM head 205 -> 152 us).
        // With fewer groups per CU the copy costs more than it saves (12288 x
        // 4096: 22 us against 17-19; 10240 x 4096: 19.8 against 19.0).
        const int64_t cus = device_cus();
        auto run = [&](auto kernel, int nw) {
            const size_t smem = skl_shared_bytes(nw, int(K));
            const unsigned grid = unsigned(std::max<int64_t>(1, std::min<int64_t>(grid_for(kernel, 64 * nw, smem), (groups + nw - 1) / nw)));
            hipLaunchKernelGGL(kernel, dim3(grid), dim3(64 * nw), smem, s, wq, wd, xq, xd, y, resid, int(M), int(N), Npad, int(K));
        };
        const bool r = epi == kEpiResidual;
        if (groups >= 8 * cus)
            r ? run(gemm_q8_skinny_lds_kernel<kEpiResidual, 8>, 8) : run(gemm_q8_skinny_lds_kernel<kEpiStore, 8>, 8);
        else
            r ? run(gemm_q8_skinny_lds_kernel<kEpiResidual, 6>, 6) : run(gemm_q8_skinny_lds_kernel<kEpiStore, 6>, 6);
        break;
    }
    case kGemmPlanSkinnyWave:
        // tall, below 4 groups per CU or at K > 4096: a wave per group range,
        // every chain in registers
        if (epi == kEpiResidual)
            hipLaunchKernelGGL((gemm_q8_skinny_wave_kernel<kEpiResidual, 1>), dim3(grid_for(gemm_q8_skinny_wave_kernel<kEpiResidual, 1>, 64, 0)), dim3(64), 0, s, wq, wd, xq, xd, y, resid, int(M), int(N), Npad, int(K));
        else
            hipLaunchKernelGGL((gemm_q8_skinny_wave_kernel<kEpiStore, 1>), dim3(grid_for(gemm_q8_skinny_wave_kernel<kEpiStore, 1>, 64, 0)), dim3(64), 0, s, wq, wd, xq, xd, y, resid, int(M), int(N), Npad, int(K));
        break;
    case kGemmPlanSkinnyWave4: {
        // 16 < M <= 64 at one group per CU or fewer: two or four waves per
        // group range, one per 16 activation rows
        auto run = [&](auto kernel, int mg) {
            hipLaunchKernelGGL(kernel, dim3(grid_for(kernel, 64 * mg, 0)), dim3(64 * mg), 0, s, wq, wd, xq, xd, y, resid, int(M), int(N), Npad, int(K));
        };
        const bool r = epi == kEpiResidual;
        if (M <= 32)
            r ? run(gemm_q8_skinny_wave_kernel<kEpiResidual, 2>, 2) : run(gemm_q8_skinny_wave_kernel<kEpiStore, 2>, 2);
        else
            r ? run(gemm_q8_skinny_wave_kernel<kEpiResidual, 4>, 4) : run(gemm_q8_skinny_wave_kernel<kEpiStore, 4>, 4);
        break;
    }
    case kGemmPlanSkinnyShared: {
        // few groups: sixteen waves share each group's blocks
        constexpr int NW = 16;
        const size_t smem = size_t(K / 32) * 16 * 4;  // the activation scales
        if (epi == kEpiResidual)
            hipLaunchKernelGGL((gemm_q8_skinny_kernel<kEpiResidual, NW>), dim3(grid_for(gemm_q8_skinny_kernel<kEpiResidual, NW>, 64 * NW, smem)), dim3(64 * NW), smem, s, wq, wd, xq, xd, y, resid, int(M), int(N), Npad, int(K));
        else
            hipLaunchKernelGGL((gemm_q8_skinny_kernel<kEpiStore, NW>), dim3(grid_for(gemm_q8_skinny_kernel<kEpiStore, NW>, 64 * NW, smem)), dim3(64 * NW), smem, s, wq, wd, xq, xd, y, resid, int(M), int(N), Npad, int(K));
        break;
    }
    case 128: gemm_dispatch<128>(epi, wq, wd, xq, xd, y, resid, int(M), int(N), Npad, int(K), s); break;
    case 64: gemm_dispatch<64>(epi, wq, wd, xq, xd, y, resid, int(M), int(N), Npad, int(K), s); break;
    case 32: gemm_dispatch<32>(epi, wq, wd, xq, xd, y, resid, int(M), int(N), Npad, int(K), s); break;
    default: gemm_dispatch<16>(epi, wq, wd, xq, xd, y, resid, int(M), int(N), Npad, int(K), s); break;
    }
}

}  // namespace hero
