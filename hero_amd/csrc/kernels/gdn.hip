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

// s = 0; s += p[i] for i = 0 .. 127, in order (128 floats in shared memory,
// 16-byte aligned), read 32 at a time one chunk ahead of their adds
__device__ __forceinline__ float seq_sum_128(const float* p) {
    const float4* p4 = reinterpret_cast<const float4*>(p);
    float4 a[8], b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = p4[i];
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        if (c < 3) {
#pragma unroll
            for (int i = 0; i < 8; ++i) b[i] = p4[8 * (c + 1) + i];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            s += a[i].x;
            s += a[i].y;
            s += a[i].z;
            s += a[i].w;
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 8; ++i) a[i] = b[i];
    }
    return s;
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
// A workgroup of 512 lanes per (sequence, value head). Lanes j < 128 own value
// column j and every sequential chain of it; all 512 lanes (column t % 128,
// key rows 32 (t / 128) .. +31) do the elementwise work on the state in
// registers and hand their products to the chains through shared memory,
// transposed [column][row], so a chain lane only adds, four terms per 16-byte
// read:
//  1. conv + SiLU of the head's q, k, v channels; the L2 norms of q and k
//     (one 128-term chain each, on two waves) while the state loads land;
//  2. S[i][j] *= decay and the products S[i][j] * k[i]; chain: pred_j;
//  3. S[i][j] += k[i] * delta_j (stored back), products S[i][j] * q[i];
//     chain: o_j;
//  4. the head RMSNorm chain over o_j^2 (lane 0), the SiLU(z) gate, quantize.
constexpr int kGdnThreads = 512;
constexpr int kGdnRows = kGdnDim * kGdnDim / kGdnThreads;  // state rows per lane: 32
constexpr int kGdnPStride = kGdnDim + 4;                    // product row stride (conflict-free 16-byte access)
struct GdnDecodeShared {
    float prod[kGdnDim][kGdnPStride];  // [column j][row i]
    float q[kGdnDim], k[kGdnDim];      // conv + SiLU outputs, then normalised
    float sq[2][kGdnDim];              // squares of q and k, then of the outputs
    float delta[kGdnDim];
    float scal[4];                     // 1/||q||, 1/||k||, 1/rms(o)
    uint64_t etab[32];                 // expf's table
};

// the ring's W slots of channel c (slot s holds the input of the latest
// position p with p % W == s), read without knowing the position
template <int W>
__device__ __forceinline__ void load_ring(const float* hist, int64_t CC, int64_t c, float (&ring)[W]) {
#pragma unroll
    for (int s = 0; s < W; ++s) ring[s] = hist[int64_t(s) * CC + c];
}
// the inputs at positions pos-(W-1) .. pos-1 out of the ring (zero before position 0)
template <int W>
__device__ __forceinline__ void past_from_ring(const float (&ring)[W], int pos, ConvPast<W>& past) {
#pragma unroll
    for (int i = 0; i < W - 1; ++i) {
        const int p = pos - (W - 1) + i;
        const int slot = p >= 0 ? p % W : -1;
        float v = 0.f;
#pragma unroll
        for (int s = 0; s < W; ++s) v = s == slot ? ring[s] : v;
        past.v[i] = v;
    }
}

template <int W, int NT>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(NT == 256 ? 2 : 1))) void gdn_decode_kernel(GdnDecodeArgs a) {
    constexpr int kGdnRows = kGdnDim * kGdnDim / NT;  // state rows per lane
    extern __shared__ __align__(16) float gdn_raw[];
    GdnDecodeShared& sh = *reinterpret_cast<GdnDecodeShared*>(gdn_raw);
    const int t = threadIdx.x, j = t % kGdnDim, i0 = (t / kGdnDim) * kGdnRows;
    const int h = blockIdx.x, b = blockIdx.y;
    const int hk = h % a.Hk;  // tiled key heads (nm/src/qwen35.hpp:172)
    const int64_t KW = int64_t(a.Hk) * kGdnDim;
    const int64_t CC = 2 * KW + int64_t(a.Hv) * kGdnDim;
    const float* P = a.proj + int64_t(b) * a.proj_stride;
    float* hist = a.conv_hist + int64_t(b) * W * CC;
    float* S = a.state + (int64_t(b) * a.Hv + h) * kGdnState;
    const bool owner = t < kGdnDim;  // column j's chains
    const ExpTab et{sh.etab};

    // ---- every load is issued before anything waits, none depends on the
    // position: expf's table, the gate inputs and the owners' conv inputs
    // first (loads retire in order: the conv and the q/k norms then run while
    // the state is still arriving), then the state rows i0 .. i0+31 of
    // column j ----
    const uint64_t etv = exp2_table(t & 31);  // lanes < 32 store it in shared memory below
    const int pos = a.positions[b];
    // the gate inputs as vector loads (the same in every lane), issued here
    // rather than where they are first used
    const uint32_t z0 = lane_zero();
    const float g_beta = load_f32(buffer_of(P, uint32_t(a.proj_stride) * 4u), uint32_t(a.beta_off + h) * 4u + z0);
    const float g_alpha = load_f32(buffer_of(P, uint32_t(a.proj_stride) * 4u), uint32_t(a.alpha_off + h) * 4u + z0);
    const float g_dt = load_f32(buffer_of(a.dt_bias, uint32_t(a.Hv) * 4u), uint32_t(h) * 4u + z0);
    const float g_a = load_f32(buffer_of(a.decay, uint32_t(a.Hv) * 4u), uint32_t(h) * 4u + z0);
    const int64_t cq = int64_t(hk) * kGdnDim + j, ck = KW + int64_t(hk) * kGdnDim + j, cv = 2 * KW + int64_t(h) * kGdnDim + j;
    float xq = 0.f, xk = 0.f, xv = 0.f, z = 0.f, gamma = 0.f;
    float tq[W], tk[W], tv[W], rq[W], rk[W], rv[W];
    if (owner) {
        xq = P[cq], xk = P[ck], xv = P[cv];
        load_taps<W>(a.conv_taps, cq, tq);
        load_taps<W>(a.conv_taps, ck, tk);
        load_taps<W>(a.conv_taps, cv, tv);
        load_ring<W>(hist, CC, cq, rq);
        load_ring<W>(hist, CC, ck, rk);
        load_ring<W>(hist, CC, cv, rv);
        z = P[a.z_off + int64_t(h) * kGdnDim + j];
        gamma = a.norm_gamma[j];
    }
    __builtin_amdgcn_sched_barrier(0);
    // raw buffer accesses with the row in the scalar offset: one address
    // register for all rows (64-bit addresses per row would hold 2 registers
    // each until the store-back)
    const __amdgpu_buffer_rsrc_t bS = buffer_of(S, uint32_t(kGdnState) * 4u);
    const uint32_t soff = uint32_t(i0 * kGdnDim + j) * 4u;
    float col[kGdnRows];
#pragma unroll
    for (int r = 0; r < kGdnRows; ++r) col[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(bS, soff, uint32_t(r * kGdnDim * 4), 0));
    __builtin_amdgcn_sched_barrier(0);
    if (t < 32) sh.etab[t] = etv;
    __syncthreads();  // the table
    if (pos < 0) {  // the host keeps positions in range; idle batch rows store nothing
        wait_vmcnt<0>();
        return;
    }
    const float beta = et.sigmoid(g_beta);
    const float decay = et.exp(g_a * et.softplus(g_alpha + g_dt));

    // ---- 1. conv + SiLU on the head's channels; the ring takes this position ----
    float v = 0.f;
    if (owner) {
        ConvPast<W> pq, pk, pv;
        past_from_ring<W>(rq, pos, pq);
        past_from_ring<W>(rk, pos, pk);
        past_from_ring<W>(rv, pos, pv);
        const float q = et.silu(conv_channel<W>(tq, pq, xq));
        const float k = et.silu(conv_channel<W>(tk, pk, xk));
        v = et.silu(conv_channel<W>(tv, pv, xv));
        const int slot = pos % W;
        if (h < a.Hk) {  // the first value head of each key head owns its q/k history
            hist[int64_t(slot) * CC + cq] = xq;
            hist[int64_t(slot) * CC + ck] = xk;
        }
        hist[int64_t(slot) * CC + cv] = xv;
        sh.q[j] = q;
        sh.k[j] = k;
        sh.sq[0][j] = q * q;
        sh.sq[1][j] = k * k;
    }
    __syncthreads();
    // ---- L2 norms (nm/src/recurrent.hpp:40-48), sequential sums ----
    if (t == 0 || t == 64) {
        const float ss = seq_sum_128(sh.sq[t == 0 ? 0 : 1]);
        sh.scal[t == 0 ? 0 : 1] = 1.f / fmaxf(sqrtf(ss), 1e-6f);
    }
    __syncthreads();
    if (owner) {
        const float query_scale = 1.f / sqrtf(float(kGdnDim));
        sh.q[j] = (sh.q[j] * sh.scal[0]) * query_scale;
        sh.k[j] = sh.k[j] * sh.scal[1];
    }
    __syncthreads();

    // ---- 2. decay and the prediction products (recurrent.hpp:146-177) ----
    float* prow = &sh.prod[j][i0];
#pragma unroll
    for (int r = 0; r < kGdnRows; r += 4) {
        const float4 k4 = *reinterpret_cast<const float4*>(sh.k + i0 + r);
        col[r] = col[r] * decay, col[r + 1] = col[r + 1] * decay, col[r + 2] = col[r + 2] * decay, col[r + 3] = col[r + 3] * decay;
        *reinterpret_cast<float4*>(prow + r) = make_float4(col[r] * k4.x, col[r + 1] * k4.y, col[r + 2] * k4.z, col[r + 3] * k4.w);
    }
    __syncthreads();
    if (owner) {  // pred_j = sum_i S[i][j] * k[i], in i order
        const float pred = seq_sum_128(&sh.prod[j][0]);
        sh.delta[j] = (v - pred) * beta;
    }
    __syncthreads();

    // ---- 3. the update, stored back, and the output products ----
    const float delta = sh.delta[j];
    // k read again from shared memory (not kept in registers across the
    // chain: the 64-row form would spill)
#pragma unroll
    for (int r = 0; r < kGdnRows; r += 4) {
        const float4 k4 = *reinterpret_cast<const float4*>(sh.k + i0 + r);
        col[r] = col[r] + k4.x * delta;
        col[r + 1] = col[r + 1] + k4.y * delta;
        col[r + 2] = col[r + 2] + k4.z * delta;
        col[r + 3] = col[r + 3] + k4.w * delta;
    }
#pragma unroll
    for (int r = 0; r < kGdnRows; ++r) __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, col[r]), bS, soff, uint32_t(r * kGdnDim * 4), 0);
#pragma unroll
    for (int r = 0; r < kGdnRows; r += 4) {
        const float4 q4 = *reinterpret_cast<const float4*>(sh.q + i0 + r);
        *reinterpret_cast<float4*>(prow + r) = make_float4(col[r] * q4.x, col[r + 1] * q4.y, col[r + 2] * q4.z, col[r + 3] * q4.w);
    }
    __syncthreads();
    float o = 0.f;
    if (owner) {  // o_j = sum_i S[i][j] * q[i], in i order
        o = seq_sum_128(&sh.prod[j][0]);
        sh.sq[0][j] = o * o;
    }
    __syncthreads();

    // ---- 4. per-head RMSNorm (components.hpp:176-181), SiLU(z) gate, quantize ----
    if (t == 0) {
        const float ss = seq_sum_128(sh.sq[0]);
        sh.scal[2] = 1.f / sqrtf(ss / float(kGdnDim) + a.eps);
    }
    __syncthreads();
    if (owner) {
        const float out = (gamma * o * sh.scal[2]) * et.silu(z);
        const int64_t width = int64_t(a.Hv) * kGdnDim;
        const int64_t idx = int64_t(h) * kGdnDim + j;
        if (a.out_f32) a.out_f32[int64_t(b) * width + idx] = out;
        gdn_quantize(out, b, a.B, width, idx, j, a.act_out);
    }
}

// ---- decode, split over value columns --------------------------------------------------
// One workgroup (one wave) per (sequence, value head, 16 value columns): the
// columns of the delta rule are independent (nm/src/recurrent.hpp:146-177:
// predicted[j], delta[j] and output[j] read only column j of the state), so
// 8 workgroups share a head and each recomputes the head's conv, SiLU and
// L2 norms of q and k. The four lanes 4j .. 4j+3 (one quad) own column
// c0 + j; lane 4j + r holds its rows 32r .. 32r+31 in registers with the
// matching k and q values. A column's 128-term chains (the decayed
// prediction, then the output) run in row order as four 32-term segments:
// the quad's lane r continues the running sum from lane r-1, handed over by
// a DPP quad permutation, so every term is added from registers.
// The kernel writes the raw outputs o (before the head RMSNorm) and, if asked,
// the gates SiLU(z); the output projection's prologue (or
// gdn_norm_gate_kernel) normalises, gates and quantizes.
constexpr int kGdnCols = 16;                      // value columns per workgroup
constexpr int kGdnSlices = kGdnDim / kGdnCols;    // workgroups per head
constexpr int kGdnSeg = kGdnDim / 4;              // rows per lane: 32
struct GdnColsShared {
    float q[kGdnDim], k[kGdnDim];                 // conv + SiLU outputs, then normalised
    float sq[2][kGdnDim];                         // their squares
    uint64_t etab[32];                            // expf's table
};

// the running sum of lane r-1 of each quad, in lane r (quad_perm 0,0,1,2)
__device__ __forceinline__ float quad_prev(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x90, 0xF, 0xF, false));
}
// lane 3's value of each quad, in all four lanes (quad_perm 3,3,3,3)
__device__ __forceinline__ float quad_last(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xFF, 0xF, 0xF, false));
}

template <int W>
__global__ __launch_bounds__(64) void gdn_decode_cols_kernel(GdnDecodeArgs a, float* __restrict__ o_raw, float* __restrict__ g_raw) {
    __shared__ __align__(16) GdnColsShared sh;
    const int t = threadIdx.x, j = t / 4, r = t % 4;
    const int h = blockIdx.x / kGdnSlices, slice = blockIdx.x % kGdnSlices, c0 = slice * kGdnCols, b = blockIdx.y;
    const int hk = h % a.Hk;  // tiled key heads (nm/src/qwen35.hpp:172)
    const int64_t KW = int64_t(a.Hk) * kGdnDim;
    const int64_t CC = 2 * KW + int64_t(a.Hv) * kGdnDim;
    const float* P = a.proj + int64_t(b) * a.proj_stride;
    float* hist = a.conv_hist + int64_t(b) * W * CC;
    float* S = a.state + (int64_t(b) * a.Hv + h) * kGdnState + c0 + j;  // column c0 + j
    // expf's table first: its read then waits for no other load
    const uint64_t etv = exp2_table(t & 31);
    const int pos = a.positions[b];

    // ---- every load first: gates, the q/k channels t and t + 64 and the v
    // channel c0 + j with their taps and ring slots, then the lane's 32 state
    // rows of its column ----
    const float g_beta = P[a.beta_off + h], g_alpha = P[a.alpha_off + h];
    const float g_dt = a.dt_bias[h], g_a = a.decay[h];
    const float zv = P[a.z_off + int64_t(h) * kGdnDim + c0 + j];
    float xq[2], xk[2], tq[2][W], tk[2][W], rq[2][W], rk[2][W];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int64_t cq = int64_t(hk) * kGdnDim + t + 64 * u, ck = KW + cq;
        xq[u] = P[cq];
        xk[u] = P[ck];
        load_taps<W>(a.conv_taps, cq, tq[u]);
        load_taps<W>(a.conv_taps, ck, tk[u]);
        load_ring<W>(hist, CC, cq, rq[u]);
        load_ring<W>(hist, CC, ck, rk[u]);
    }
    const int64_t cv = 2 * KW + int64_t(h) * kGdnDim + c0 + j;
    float tv[W], rv[W];
    const float xv = P[cv];
    load_taps<W>(a.conv_taps, cv, tv);
    load_ring<W>(hist, CC, cv, rv);
    float col[kGdnSeg];
#pragma unroll
    for (int m = 0; m < kGdnSeg; ++m) col[m] = S[(kGdnSeg * r + m) * kGdnDim];
    if (t < 32) sh.etab[t] = etv;
    __syncthreads();
    if (pos < 0) return;  // the host keeps positions in range; idle batch rows store nothing
    const ExpTab et{sh.etab};
    // the gates first, while the conv inputs and the state are still arriving
    const float beta = et.sigmoid(g_beta);
    const float decay = et.exp(g_a * et.softplus(g_alpha + g_dt));
    const float gate = et.silu(zv);  // the output gate SiLU(z) of column c0 + j (nm/src/qwen35.hpp:458)

    // ---- conv + SiLU; the ring takes this position (the state loads are
    // still in flight: they were issued last) ----
    const int slot = pos % W;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int c = t + 64 * u;
        ConvPast<W> pq, pk;
        past_from_ring<W>(rq[u], pos, pq);
        past_from_ring<W>(rk[u], pos, pk);
        const float q = et.silu(conv_channel<W>(tq[u], pq, xq[u]));
        const float k = et.silu(conv_channel<W>(tk[u], pk, xk[u]));
        if (h < a.Hk && slice == 0) {  // one workgroup per key head owns its q/k history
            const int64_t cq = int64_t(hk) * kGdnDim + c;
            hist[int64_t(slot) * CC + cq] = xq[u];
            hist[int64_t(slot) * CC + KW + cq] = xk[u];
        }
        sh.q[c] = q;
        sh.k[c] = k;
        sh.sq[0][c] = q * q;
        sh.sq[1][c] = k * k;
    }
    float v;
    {
        ConvPast<W> pv;
        past_from_ring<W>(rv, pos, pv);
        v = et.silu(conv_channel<W>(tv, pv, xv));
        if (r == 0) hist[int64_t(slot) * CC + cv] = xv;
    }
    __syncthreads();
    // ---- L2 norms of q and k (nm/src/recurrent.hpp:40-48): even lanes run
    // the sequential sum of q's squares, odd lanes k's (broadcast reads), and
    // lanes 0 and 1 hand the two sums to the wave ----
    float ssq, ssk;
    {
        const float4* s4 = reinterpret_cast<const float4*>(sh.sq[t & 1]);
        float4 cur[8], nxt[8];
        float ss = 0.f;
#pragma unroll
        for (int u = 0; u < 8; ++u) cur[u] = s4[u];
#pragma unroll
        for (int c = 0; c < kGdnDim / 32; ++c) {
            if (c + 1 < kGdnDim / 32) {
#pragma unroll
                for (int u = 0; u < 8; ++u) nxt[u] = s4[8 * (c + 1) + u];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                ss += cur[u].x;
                ss += cur[u].y;
                ss += cur[u].z;
                ss += cur[u].w;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) cur[u] = nxt[u];
        }
        ssq = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 0));
        ssk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ss), 1));
    }
    const float inv_q = 1.f / fmaxf(sqrtf(ssq), 1e-6f), inv_k = 1.f / fmaxf(sqrtf(ssk), 1e-6f);
    {
        const float query_scale = 1.f / sqrtf(float(kGdnDim));
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int c = t + 64 * u;
            sh.q[c] = (sh.q[c] * inv_q) * query_scale;
            sh.k[c] = sh.k[c] * inv_k;
        }
    }
    __syncthreads();
    // ---- the delta rule on column c0 + j, rows 32r .. 32r+31 in this lane ----
    float ks[kGdnSeg], qs[kGdnSeg];
    {
        const float4* k4 = reinterpret_cast<const float4*>(sh.k + kGdnSeg * r);
        const float4* q4 = reinterpret_cast<const float4*>(sh.q + kGdnSeg * r);
#pragma unroll
        for (int i = 0; i < kGdnSeg / 4; ++i) {
            const float4 kk = k4[i], qq = q4[i];
            ks[4 * i] = kk.x, ks[4 * i + 1] = kk.y, ks[4 * i + 2] = kk.z, ks[4 * i + 3] = kk.w;
            qs[4 * i] = qq.x, qs[4 * i + 1] = qq.y, qs[4 * i + 2] = qq.z, qs[4 * i + 3] = qq.w;
        }
    }
#pragma unroll
    for (int m = 0; m < kGdnSeg; ++m) col[m] = col[m] * decay;
    // pred = sum_i S[i][j] * k[i] in i order: segment r in lane r, handed on
    float acc = 0.f;
#pragma unroll
    for (int seg = 0; seg < 4; ++seg) {
        if (r == seg) {
#pragma unroll
            for (int m = 0; m < kGdnSeg; ++m) acc = acc + col[m] * ks[m];
        }
        if (seg < 3) acc = quad_prev(acc);
    }
    const float pred = quad_last(acc);
    const float delta = (v - pred) * beta;
#pragma unroll
    for (int m = 0; m < kGdnSeg; ++m) col[m] = col[m] + ks[m] * delta;
    // o = sum_i S'[i][j] * q[i] in i order, the same way
    acc = 0.f;
#pragma unroll
    for (int seg = 0; seg < 4; ++seg) {
        if (r == seg) {
#pragma unroll
            for (int m = 0; m < kGdnSeg; ++m) acc = acc + col[m] * qs[m];
        }
        if (seg < 3) acc = quad_prev(acc);
    }
    if (r == 3) {
        o_raw[(int64_t(b) * a.Hv + h) * kGdnDim + c0 + j] = acc;
        if (g_raw) g_raw[(int64_t(b) * a.Hv + h) * kGdnDim + c0 + j] = gate;
    }
#pragma unroll
    for (int m = 0; m < kGdnSeg; ++m) S[(kGdnSeg * r + m) * kGdnDim] = col[m];
}

// The per-head RMSNorm (nm/src/components.hpp:176-181), the SiLU(z) gate and
// Q8_0 quantization of raw delta-net outputs, one workgroup of 128 lanes per
// (row, head): o [rows][Hv*128], z at proj + row * proj_stride + z_off.
__global__ __launch_bounds__(kGdnDim) void gdn_norm_gate_kernel(const float* __restrict__ o_raw, const float* __restrict__ proj, int64_t proj_stride, int64_t z_off,
                                                                const float* __restrict__ gamma, float eps, void* act_out, float* out_f32, int rows, int Hv) {
    const int j = threadIdx.x, h = blockIdx.x, row = blockIdx.y;
    __shared__ __align__(16) float ov[kGdnDim];
    __shared__ float scal;
    const int64_t width = int64_t(Hv) * kGdnDim, idx = int64_t(h) * kGdnDim + j;
    const float o = o_raw[int64_t(row) * width + idx];
    const float z = proj[int64_t(row) * proj_stride + z_off + idx];
    ov[j] = o * o;
    __syncthreads();
    if (j == 0) {
        const float4* s4 = reinterpret_cast<const float4*>(ov);
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < kGdnDim / 4; ++i) {
            const float4 x = s4[i];
            ss += x.x;
            ss += x.y;
            ss += x.z;
            ss += x.w;
        }
        scal = 1.f / sqrtf(ss / float(kGdnDim) + eps);
    }
    __syncthreads();
    const float out = (gamma[j] * o * scal) * silu_f32(z);
    if (out_f32) out_f32[int64_t(row) * width + idx] = out;
    gdn_quantize(out, row, rows, width, idx, j, act_out);
}

// ---- prefill: tokens t = 0..T-1 of one sequence at positions pos0 + t -------------
// a.B is T (rows of proj and of act_out); a.positions[0] is pos0; the state
// and the ring are sequence 0's. Three kernels:
//  prep  (token, head) in parallel: conv + SiLU, L2 norms and the query scale,
//        beta and the decay -- nothing here depends on the state;
//  scan  the delta rule over the tokens in order, 8 workgroups per value
//        head, the state in registers for the whole chunk (below);
//  out   (token, head) in parallel: head RMSNorm, SiLU(z) gate, quantize.
// The scan's critical path per token is one 128-term chain: token t's output
// chain and token t+1's decay and prediction chain read the same updated
// column, so they run side by side. Every value is computed by the same
// operations in the same order as in gdn_decode_kernel.

__device__ __forceinline__ GdnPrefillWork gdn_work(void* ws, int64_t T, int Hk, int Hv) {
    GdnPrefillWork w;
    float* f = static_cast<float*>(ws);
    w.q = f;
    w.k = w.q + T * Hk * kGdnDim;
    w.v = w.k + T * Hk * kGdnDim;
    w.o = w.v + T * Hv * kGdnDim;
    w.bd = w.o + T * Hv * kGdnDim;
    w.g = w.bd + T * Hv * 2;
    w.u = w.g + T * Hv;
    w.wm = w.u + T * Hv * kGdnDim;
    w.p = w.wm + T * Hv * kGdnDim;
    w.G = w.p + (T + 63) / 64 * Hv * 64 * 64;
    return w;
}

template <int W>
__global__ __launch_bounds__(kGdnDim) void gdn_prep_kernel(GdnDecodeArgs a, void* ws) {
    const int j = threadIdx.x, slot = blockIdx.x, t = blockIdx.y;
    const int pos0 = a.positions[0];
    const int T = a.B;
    if (pos0 < 0) return;
    const GdnPrefillWork w = gdn_work(ws, T, a.Hk, a.Hv);
    const int64_t KW = int64_t(a.Hk) * kGdnDim;
    const int64_t CC = 2 * KW + int64_t(a.Hv) * kGdnDim;
    const float* P = a.proj + int64_t(t) * a.proj_stride;
    // the conv input of channel c at token index u (< 0: before the chunk, from the ring)
    auto input = [&](int64_t c, int u) -> float {
        if (u >= 0) return a.proj[int64_t(u) * a.proj_stride + c];
        const int p = pos0 + u;
        return p >= 0 ? a.conv_hist[int64_t(p % W) * CC + c] : 0.f;
    };
    auto conv_silu = [&](int64_t c) -> float {
        float taps[W];
        load_taps<W>(a.conv_taps, c, taps);
        ConvPast<W> past;
#pragma unroll
        for (int i = 0; i < W - 1; ++i) past.v[i] = input(c, t - (W - 1) + i);
        return silu_f32(conv_channel<W>(taps, past, P[c]));
    };
    __shared__ __align__(16) float buf[2][kGdnDim];
    __shared__ float inv[2];
    if (slot < a.Hk) {  // q and k of key head `slot`
        const float sq = conv_silu(int64_t(slot) * kGdnDim + j);
        const float sk = conv_silu(KW + int64_t(slot) * kGdnDim + j);
        buf[0][j] = sq;
        buf[1][j] = sk;
        __syncthreads();
        if (j == 0 || j == 64) {  // L2 norms (nm/src/recurrent.hpp:40-48)
            const float ss = sum_squares_128(buf[j == 0 ? 0 : 1]);
            inv[j == 0 ? 0 : 1] = 1.f / fmaxf(sqrtf(ss), 1e-6f);
        }
        __syncthreads();
        const float query_scale = 1.f / sqrtf(float(kGdnDim));
        const int64_t o = (int64_t(t) * a.Hk + slot) * kGdnDim + j;
        w.q[o] = (sq * inv[0]) * query_scale;
        w.k[o] = sk * inv[1];
    } else {  // v of value head h, and its beta and decay
        const int h = slot - a.Hk;
        w.v[(int64_t(t) * a.Hv + h) * kGdnDim + j] = conv_silu(2 * KW + int64_t(h) * kGdnDim + j);
        if (j == 0) {
            const float beta = sigmoid_f32(P[a.beta_off + h]);
            const float g = a.decay[h] * softplus_f32(P[a.alpha_off + h] + a.dt_bias[h]);
            w.bd[(int64_t(t) * a.Hv + h) * 2] = beta;
            w.bd[(int64_t(t) * a.Hv + h) * 2 + 1] = exp_f32(g);
            w.g[int64_t(t) * a.Hv + h] = g;
        }
    }
}

// ---- the token-serial scan, split over value columns and state rows ----------------------
// The delta rule over the chunk's tokens in order, each value column spread
// over 16 lanes (one DPP row): the columns of the delta rule are independent
// (nm/src/recurrent.hpp:146-177), so a workgroup of 256 lanes owns 16 columns
// and a head takes 8 workgroups. Lane 2s + c of a row holds rows 16s .. 16s+15
// of its column (segment s); lanes c = 0 run token t+1's decay-and-prediction
// chain and lanes c = 1 token t's output chain, both over the same updated
// rows, so one instruction stream advances both chains. A chain visits the
// segments in row order: segment s adds its 16 terms to the running sum that
// segment s-1 handed on (a DPP shift by two lanes), so every sum is the
// reference's left-to-right chain. Both lanes of a segment keep the same
// copy of the segment's rows. Per token and wave that is 16 rows of updates
// and products plus the chains' 128 steps, against 128 rows of each for a
// lane owning a whole column.
constexpr int kScCols = 16;                  // value columns per workgroup
constexpr int kScSeg = 8;                    // row segments per column
constexpr int kScRows = kGdnDim / kScSeg;    // rows per lane (16)
constexpr int kScTile = 16;                  // tokens per shared-memory tile
struct ScanColsTile {
    float k[kScTile][kGdnDim];
    float q[kScTile][kGdnDim];
    float v[kScTile][kScCols];
    float bd[kScTile][2];
};

// the running sum of lane i-2 of each row of 16 lanes, in lane i
__device__ __forceinline__ float row_shr2(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x112, 0xF, 0xF, false));
}
// segment s (lanes 2s, 2s+1 of each row) adds its terms, in row order, to the
// sum handed on by segment s-1; the final sums end in lanes 14 and 15
__device__ __forceinline__ float seg_chain(const float (&prod)[kScRows], int seg) {
    float acc = 0.f;
#pragma unroll
    for (int s = 0; s < kScSeg; ++s) {
        if (seg == s) {
#pragma unroll
            for (int m = 0; m < kScRows; ++m) acc = acc + prod[m];
        }
        if (s + 1 < kScSeg) acc = row_shr2(acc);
    }
    return acc;
}
// lane 14 of each row of the wave, in every lane of that row
__device__ __forceinline__ float row_lane14(float v, int row) {
    const int b = __float_as_int(v);
    const int r0 = __builtin_amdgcn_readlane(b, 14), r1 = __builtin_amdgcn_readlane(b, 30);
    const int r2 = __builtin_amdgcn_readlane(b, 46), r3 = __builtin_amdgcn_readlane(b, 62);
    return __int_as_float(row == 0 ? r0 : row == 1 ? r1 : row == 2 ? r2 : r3);
}

__global__ __launch_bounds__(256) void gdn_scan_cols_kernel(GdnDecodeArgs a, void* ws) {
    const int lane = threadIdx.x;
    const int h = blockIdx.x / (kGdnDim / kScCols), c0 = (blockIdx.x % (kGdnDim / kScCols)) * kScCols, hk = h % a.Hk;
    const int jl = lane / 16, seg = (lane % 16) / 2, ch = lane % 2, row = (lane % 64) / 16;
    const int j = c0 + jl, r0 = seg * kScRows;
    const int T = a.B;
    if (a.positions[0] < 0) return;
    const GdnPrefillWork w = gdn_work(ws, T, a.Hk, a.Hv);
    float* S = a.state + int64_t(h) * kGdnState + j;
    __shared__ __align__(16) ScanColsTile tiles[2];
    const int ntiles = (T + kScTile - 1) / kScTile;

    // a tile: k and q (2 float4 each per lane), v of the 16 columns (lanes
    // 0..63) and (beta, decay) (lanes 64..79); zeros past the last token
    float4 pk[2], pq[2], pv = make_float4(0.f, 0.f, 0.f, 0.f);
    float2 pbd = make_float2(0.f, 0.f);
    auto load = [&](int tile) {
        const int t0 = tile * kScTile;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int f = lane + 256 * u, tt = t0 + f / (kGdnDim / 4), c4 = f % (kGdnDim / 4);
            const int64_t o = (int64_t(tt) * a.Hk + hk) * kGdnDim;
            pk[u] = tt < T ? reinterpret_cast<const float4*>(w.k + o)[c4] : make_float4(0.f, 0.f, 0.f, 0.f);
            pq[u] = tt < T ? reinterpret_cast<const float4*>(w.q + o)[c4] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (lane < 64) {
            const int tt = t0 + lane / 4;
            pv = tt < T ? reinterpret_cast<const float4*>(w.v + (int64_t(tt) * a.Hv + h) * kGdnDim + c0)[lane % 4] : make_float4(0.f, 0.f, 0.f, 0.f);
        } else if (lane < 64 + kScTile) {
            const int tt = t0 + lane - 64;
            pbd = tt < T ? reinterpret_cast<const float2*>(w.bd)[int64_t(tt) * a.Hv + h] : make_float2(0.f, 0.f);
        }
    };
    auto store = [&](ScanColsTile& dst) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            reinterpret_cast<float4*>(&dst.k[0][0])[lane + 256 * u] = pk[u];
            reinterpret_cast<float4*>(&dst.q[0][0])[lane + 256 * u] = pq[u];
        }
        if (lane < 64)
            reinterpret_cast<float4*>(&dst.v[0][0])[lane] = pv;
        else if (lane < 64 + kScTile)
            reinterpret_cast<float2*>(&dst.bd[0][0])[lane - 64] = pbd;
    };
    auto rows16 = [&](const float* src, float (&dst)[kScRows]) {
        const float4* s4 = reinterpret_cast<const float4*>(src + r0);
#pragma unroll
        for (int u = 0; u < kScRows / 4; ++u) {
            const float4 x = s4[u];
            dst[4 * u] = x.x, dst[4 * u + 1] = x.y, dst[4 * u + 2] = x.z, dst[4 * u + 3] = x.w;
        }
    };

    float col[kScRows];  // S[r0 + m][j]
#pragma unroll
    for (int m = 0; m < kScRows; ++m) col[m] = S[int64_t(r0 + m) * kGdnDim];
    load(0);
    store(tiles[0]);
    if (ntiles > 1) {
        load(1);
        store(tiles[1]);
    }
    if (ntiles > 2) load(2);
    __syncthreads();

    // token 0: decay and prediction chain (nm/src/recurrent.hpp:152-160)
    float delta;
    {
        float kk[kScRows], prod[kScRows];
        rows16(tiles[0].k[0], kk);
        const float dec = tiles[0].bd[0][1];
#pragma unroll
        for (int m = 0; m < kScRows; ++m) {
            col[m] = col[m] * dec;
            prod[m] = col[m] * kk[m];
        }
        const float pred = row_lane14(seg_chain(prod, seg), row);
        delta = (tiles[0].v[0][jl] - pred) * tiles[0].bd[0][0];
    }
    for (int t = 0; t < T; ++t) {
        const int tile = t / kScTile, r = t % kScTile;
        if (r == 0 && tile > 0) {
            // tile-1's buffer is free: it takes tile+1 (loaded a tile ago)
            __syncthreads();
            if (tile + 1 < ntiles) store(tiles[(tile + 1) & 1]);
            if (tile + 2 < ntiles) load(tile + 2);
            __syncthreads();
        }
        const ScanColsTile& cur = tiles[tile & 1];
        const ScanColsTile& nxt = tiles[((t + 1) / kScTile) & 1];
        const int rn = (t + 1) % kScTile;
        float kc[kScRows], f[kScRows], prod[kScRows];
        rows16(cur.k[r], kc);
        // lanes c = 0: token t+1's key (zeros past the last token); c = 1: token t's query
        rows16(ch == 0 ? nxt.k[rn] : cur.q[r], f);
        float o;
        if (t + 1 < T) {
            const float dec = nxt.bd[rn][1];
#pragma unroll
            for (int m = 0; m < kScRows; ++m) {
                const float v = col[m] + kc[m] * delta;  // S[i][j] += k[i] * delta
                const float vd = v * dec;                // next token: S[i][j] *= decay
                col[m] = vd;
                prod[m] = (ch == 0 ? vd : v) * f[m];     // pred += S[i][j] * k'[i]  |  o += S[i][j] * q[i]
            }
            const float acc = seg_chain(prod, seg);
            o = acc;
            const float pred = row_lane14(acc, row);
            delta = (nxt.v[rn][jl] - pred) * nxt.bd[rn][0];
        } else {
#pragma unroll
            for (int m = 0; m < kScRows; ++m) {
                const float v = col[m] + kc[m] * delta;
                col[m] = v;
                prod[m] = v * f[m];
            }
            o = seg_chain(prod, seg);
        }
        if (lane % 16 == 15) w.o[(int64_t(t) * a.Hv + h) * kGdnDim + j] = o;
    }
    if (ch == 1) {
#pragma unroll
        for (int m = 0; m < kScRows; ++m) S[int64_t(r0 + m) * kGdnDim] = col[m];
    }
}

// ---- the chunked form (WY representation) ------------------------------------------------
// Within a chunk of C tokens starting from state S0, with G_t = sum_{s<=t} g_s
// (cumulative log-decay) and gamma_t = exp(G_t), the recurrence
//   S_t = decay_t S_{t-1} + k_t delta_t^T,  delta_t = beta_t (v_t - (decay_t S_{t-1})^T k_t),
//   o_t = S_t^T q_t
// unrolls to (I + L) delta = beta V - beta gamma K S0, L[t][s] = beta_t exp(G_t - G_s) k_t.k_s (s < t):
//   delta = U - W S0,  U = (I + L)^-1 beta V,  W = (I + L)^-1 beta gamma K,
//   o_t   = gamma_t (Q S0)_t + sum_{s<=t} P[t][s] delta_s,  P[t][s] = exp(G_t - G_s) q_t.k_s,
//   S_C   = gamma_C S0 + sum_s exp(G_C - G_s) k_s delta_s^T.
// U, W and P do not depend on the state: gdn_chunk_prep_kernel forms them for
// every (chunk, head) at once; gdn_chunk_scan_kernel then carries the state
// through the chunks in order with three small matrix products per chunk.
// This form is pinned to the serial one by tolerance (its sums run in another
// order), so it uses fused multiply-adds.
constexpr int kChunk = 64;             // tokens per chunk
constexpr int kChunkCols = 32;         // state columns per scan workgroup
constexpr int kChunkKp = kGdnDim + 4;  // padded rows

struct ChunkPrepShared {
    float K[kChunk][kChunkKp];
    float Q[kChunk][kChunkKp];
    float L[kChunk][kChunk + 4];
    float X[kChunk][2 * kGdnDim];  // the U and W columns being solved, one per thread
    float G[kChunk], beta[kChunk];
};
constexpr size_t kChunkPrepShared = sizeof(ChunkPrepShared);

// one workgroup per (chunk, value head)
__global__ __launch_bounds__(256) void gdn_chunk_prep_kernel(GdnDecodeArgs a, void* ws_) {
    extern __shared__ __align__(16) float cp_raw[];
    ChunkPrepShared& sh = *reinterpret_cast<ChunkPrepShared*>(cp_raw);
    const int tid = threadIdx.x, lane = tid & 63;
    const int c = blockIdx.x, h = blockIdx.y, hk = h % a.Hk;
    const int T = a.B;
    if (a.positions[0] < 0) return;
    const GdnPrefillWork w = gdn_work(ws_, T, a.Hk, a.Hv);
    const int t0 = c * kChunk, n = min(kChunk, T - t0);
    for (int e = tid; e < kChunk * (kGdnDim / 4); e += 256) {
        const int t = e / (kGdnDim / 4), c4 = e % (kGdnDim / 4);
        float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), qv = kv;
        if (t < n) {
            const int64_t row = (int64_t(t0 + t) * a.Hk + hk) * kGdnDim;
            kv = reinterpret_cast<const float4*>(w.k + row)[c4];
            qv = reinterpret_cast<const float4*>(w.q + row)[c4];
        }
        *reinterpret_cast<float4*>(&sh.K[t][4 * c4]) = kv;
        *reinterpret_cast<float4*>(&sh.Q[t][4 * c4]) = qv;
    }
    if (tid < kChunk) {  // wave 0: beta and the cumulative log-decay (an inclusive scan)
        const bool on = tid < n;
        sh.beta[tid] = on ? w.bd[(int64_t(t0 + tid) * a.Hv + h) * 2] : 0.f;
        float G = on ? w.g[int64_t(t0 + tid) * a.Hv + h] : 0.f;
        for (int off = 1; off < 64; off <<= 1) {
            const float o = __shfl_up(G, off);
            if (lane >= off) G += o;
        }
        sh.G[tid] = G;
        if (on) w.G[int64_t(t0 + tid) * a.Hv + h] = G;
    }
    __syncthreads();
    // L (s < t) and P (s <= t): a 4x4 block of (row t, column s) per thread
    {
        const int br = tid >> 4, bc = tid & 15;
        float kk[4][4] = {}, qk[4][4] = {};
        for (int i = 0; i < kGdnDim; i += 4) {
            float4 kr[4], qr[4], kc[4];
#pragma unroll
            for (int uu = 0; uu < 4; ++uu) {
                kr[uu] = *reinterpret_cast<const float4*>(&sh.K[4 * br + uu][i]);
                qr[uu] = *reinterpret_cast<const float4*>(&sh.Q[4 * br + uu][i]);
                kc[uu] = *reinterpret_cast<const float4*>(&sh.K[4 * bc + uu][i]);
            }
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) {
                    kk[rr][cc] = fmaf(kr[rr].x, kc[cc].x, fmaf(kr[rr].y, kc[cc].y, fmaf(kr[rr].z, kc[cc].z, fmaf(kr[rr].w, kc[cc].w, kk[rr][cc]))));
                    qk[rr][cc] = fmaf(qr[rr].x, kc[cc].x, fmaf(qr[rr].y, kc[cc].y, fmaf(qr[rr].z, kc[cc].z, fmaf(qr[rr].w, kc[cc].w, qk[rr][cc]))));
                }
        }
        float* P = w.p + (int64_t(c) * a.Hv + h) * kChunk * kChunk;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                const int t = 4 * br + rr, s = 4 * bc + cc;
                const float f = s <= t ? exp_f32(sh.G[t] - sh.G[s]) : 0.f;
                sh.L[t][s] = s < t ? sh.beta[t] * f * kk[rr][cc] : 0.f;
                P[t * kChunk + s] = f * qk[rr][cc];
            }
    }
    __syncthreads();
    // U and W by forward substitution, one column per thread:
    // x_t = b_t - sum_{s<t} L[t][s] x_s; columns 0..127 of beta v, 128..255 of beta gamma k
    {
        const bool is_u = tid < kGdnDim;
        const int col = tid & (kGdnDim - 1);
        for (int t = 0; t < kChunk; ++t) {
            float b = 0.f;
            if (t < n) b = is_u ? sh.beta[t] * w.v[(int64_t(t0 + t) * a.Hv + h) * kGdnDim + col] : sh.beta[t] * exp_f32(sh.G[t]) * sh.K[t][col];
            sh.X[t][tid] = b;
        }
        for (int t = 1; t < n; ++t) {
            float acc = sh.X[t][tid];
            for (int s2 = 0; s2 < t; ++s2) acc = fmaf(-sh.L[t][s2], sh.X[s2][tid], acc);
            sh.X[t][tid] = acc;
        }
        float* dst = is_u ? w.u : w.wm;
        for (int t = 0; t < n; ++t) dst[(int64_t(t0 + t) * a.Hv + h) * kGdnDim + col] = sh.X[t][tid];
    }
}

struct ChunkScanShared {
    float Wm[kChunk][kChunkKp];
    float Q[kChunk][kChunkKp];
    float K[kChunk][kChunkKp];
    float P[kChunk][kChunk + 4];
    float S[kGdnDim][kChunkCols + 4];  // rows of 16-byte multiples
    float D[kChunk][kChunkCols + 4];   // U, then delta
    float G[kChunk], wsf[kChunk];
};
constexpr size_t kChunkScanShared = sizeof(ChunkScanShared);

// one workgroup per (value head, 32 state columns); the chunks in order, the
// next chunk's inputs loading while this one computes
// v or zeros, component by component (a select of the whole float4 is lowered
// through scratch memory)
__device__ __forceinline__ float4 sel4(bool keep, float4 v) {
    return make_float4(keep ? v.x : 0.f, keep ? v.y : 0.f, keep ? v.z : 0.f, keep ? v.w : 0.f);
}

// one workgroup per CU (its shared memory): the whole register file is this wave's
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void gdn_chunk_scan_kernel(GdnDecodeArgs a, void* ws_) {
    extern __shared__ __align__(16) float cs_raw[];
    ChunkScanShared& sh = *reinterpret_cast<ChunkScanShared*>(cs_raw);
    const int tid = threadIdx.x;
    const int h = blockIdx.x, hk = h % a.Hk, j0 = blockIdx.y * kChunkCols;
    const int T = a.B;
    if (a.positions[0] < 0) return;
    const GdnPrefillWork w = gdn_work(ws_, T, a.Hk, a.Hv);
    float* S = a.state + int64_t(h) * kGdnState;
    const int nchunks = (T + kChunk - 1) / kChunk;

    // the chunk's inputs in flight in registers: thread -> rows t = tid/32 + 8m,
    // 16-byte piece tid % 32 of W, Q, K; 16 values of P; 8 of U. Rows past the
    // chunk's end load row 0 (in range) and are zeroed.
    float4 rw[8], rq[8], rk[8];
    float rp[16], ru[8], rg;
    auto load = [&](int c) __attribute__((always_inline)) {
        const int t0 = c * kChunk, n = min(kChunk, T - t0);
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const int t = (tid >> 5) + 8 * m, c4 = tid & 31;
            const int tc = t < n ? t : 0;
            const int64_t krow = (int64_t(t0 + tc) * a.Hk + hk) * kGdnDim;
            const float4 wv = reinterpret_cast<const float4*>(w.wm + (int64_t(t0 + tc) * a.Hv + h) * kGdnDim)[c4];
            const float4 qv = reinterpret_cast<const float4*>(w.q + krow)[c4];
            const float4 kv = reinterpret_cast<const float4*>(w.k + krow)[c4];
            rw[m] = sel4(t < n, wv);
            rq[m] = sel4(t < n, qv);
            rk[m] = sel4(t < n, kv);
        }
        const float* P = w.p + (int64_t(c) * a.Hv + h) * kChunk * kChunk;
#pragma unroll
        for (int m = 0; m < 16; ++m) rp[m] = P[tid + 256 * m];
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const int e = tid + 256 * m, t = e / kChunkCols, jj = e % kChunkCols;
            const float uv = w.u[(int64_t(t0 + (t < n ? t : 0)) * a.Hv + h) * kGdnDim + j0 + jj];
            ru[m] = t < n ? uv : 0.f;
        }
        const float gv = w.G[int64_t(t0 + (tid < n ? tid : 0)) * a.Hv + h];
        rg = tid < n ? gv : 0.f;
    };
    auto store = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const int t = (tid >> 5) + 8 * m, c4 = tid & 31;
            *reinterpret_cast<float4*>(&sh.Wm[t][4 * c4]) = rw[m];
            *reinterpret_cast<float4*>(&sh.Q[t][4 * c4]) = rq[m];
            *reinterpret_cast<float4*>(&sh.K[t][4 * c4]) = rk[m];
        }
#pragma unroll
        for (int m = 0; m < 16; ++m) {
            const int e = tid + 256 * m;
            sh.P[e / kChunk][e % kChunk] = rp[m];
        }
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const int e = tid + 256 * m;
            sh.D[e / kChunkCols][e % kChunkCols] = ru[m];
        }
        if (tid < kChunk) sh.G[tid] = rg;
    };

    for (int e = tid; e < kGdnDim * kChunkCols; e += 256) {
        const int i = e / kChunkCols, jj = e % kChunkCols;
        sh.S[i][jj] = S[i * kGdnDim + j0 + jj];
    }
    load(0);
    store();
    if (nchunks > 1) load(1);
    for (int c = 0; c < nchunks; ++c) {
        const int t0 = c * kChunk, n = min(kChunk, T - t0);
        __syncthreads();  // the chunk's tiles are in shared memory
        if (tid < kChunk) sh.wsf[tid] = exp_f32(sh.G[n - 1] - sh.G[tid]);
        // delta = U - W S0 and gamma (Q S0): thread -> row t, 8 columns
        const int t = tid >> 2, jq = (tid & 3) * 8;
        float qs0[8], ws0[8];
#pragma unroll
        for (int uu = 0; uu < 8; ++uu) qs0[uu] = ws0[uu] = 0.f;
        for (int i = 0; i < kGdnDim; i += 4) {
            const float4 w4 = *reinterpret_cast<const float4*>(&sh.Wm[t][i]);
            const float4 q4 = *reinterpret_cast<const float4*>(&sh.Q[t][i]);
            const float wv[4] = {w4.x, w4.y, w4.z, w4.w}, qv[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                const float4 s0 = *reinterpret_cast<const float4*>(&sh.S[i + ii][jq]);
                const float4 s1 = *reinterpret_cast<const float4*>(&sh.S[i + ii][jq + 4]);
                const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
                for (int uu = 0; uu < 8; ++uu) {
                    ws0[uu] = fmaf(wv[ii], sv[uu], ws0[uu]);
                    qs0[uu] = fmaf(qv[ii], sv[uu], qs0[uu]);
                }
            }
        }
        const float gt = exp_f32(sh.G[t]);
#pragma unroll
        for (int uu = 0; uu < 8; ++uu) {
            sh.D[t][jq + uu] -= ws0[uu];
            qs0[uu] *= gt;
        }
        __syncthreads();
        // outputs: o_t = gamma_t (Q S0)_t + sum_{s<=t} P[t][s] delta_s
        if (t < n) {
            for (int s2 = 0; s2 <= t; ++s2) {
                const float pv = sh.P[t][s2];
                const float4 d0 = *reinterpret_cast<const float4*>(&sh.D[s2][jq]);
                const float4 d1 = *reinterpret_cast<const float4*>(&sh.D[s2][jq + 4]);
                const float dv[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
#pragma unroll
                for (int uu = 0; uu < 8; ++uu) qs0[uu] = fmaf(pv, dv[uu], qs0[uu]);
            }
            float* dst = w.o + (int64_t(t0 + t) * a.Hv + h) * kGdnDim + j0 + jq;
            reinterpret_cast<float4*>(dst)[0] = make_float4(qs0[0], qs0[1], qs0[2], qs0[3]);
            reinterpret_cast<float4*>(dst)[1] = make_float4(qs0[4], qs0[5], qs0[6], qs0[7]);
        }
        // state: S = gamma_n S0 + sum_s exp(G_n - G_s) k_s delta_s^T: thread -> row i, 16 columns
        {
            const int i = tid >> 1, jh = (tid & 1) * 16;
            const float gl = exp_f32(sh.G[n - 1]);
            float acc[16];
#pragma unroll
            for (int uu = 0; uu < 16; ++uu) acc[uu] = gl * sh.S[i][jh + uu];
            for (int s2 = 0; s2 < n; ++s2) {
                const float f = sh.wsf[s2] * sh.K[s2][i];
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const float4 d = *reinterpret_cast<const float4*>(&sh.D[s2][jh + 4 * q4]);
                    acc[4 * q4 + 0] = fmaf(f, d.x, acc[4 * q4 + 0]);
                    acc[4 * q4 + 1] = fmaf(f, d.y, acc[4 * q4 + 1]);
                    acc[4 * q4 + 2] = fmaf(f, d.z, acc[4 * q4 + 2]);
                    acc[4 * q4 + 3] = fmaf(f, d.w, acc[4 * q4 + 3]);
                }
            }
#pragma unroll
            for (int uu = 0; uu < 16; ++uu) sh.S[i][jh + uu] = acc[uu];  // row i, this thread's columns only
        }
        __syncthreads();  // every tile of this chunk is consumed
        if (c + 1 < nchunks) {
            store();
            if (c + 2 < nchunks) load(c + 2);
        }
    }
    __syncthreads();
    for (int e = tid; e < kGdnDim * kChunkCols; e += 256) {
        const int i = e / kChunkCols, jj = e % kChunkCols;
        S[i * kGdnDim + j0 + jj] = sh.S[i][jj];
    }
}

__global__ __launch_bounds__(kGdnDim) void gdn_out_kernel(GdnDecodeArgs a, void* ws) {
    const int j = threadIdx.x, h = blockIdx.x, t = blockIdx.y;
    const int T = a.B;
    if (a.positions[0] < 0) return;
    const GdnPrefillWork w = gdn_work(ws, T, a.Hk, a.Hv);
    __shared__ __align__(16) float ov[kGdnDim];
    __shared__ float scal;
    const float o = w.o[(int64_t(t) * a.Hv + h) * kGdnDim + j];
    const float z = a.proj[int64_t(t) * a.proj_stride + a.z_off + int64_t(h) * kGdnDim + j];
    ov[j] = o;
    __syncthreads();
    // per-head RMSNorm (components.hpp:176-181) and the SiLU(z) gate
    if (j == 0) scal = 1.f / sqrtf(sum_squares_128(ov) / float(kGdnDim) + a.eps);
    __syncthreads();
    const float out = (a.norm_gamma[j] * o * scal) * silu_f32(z);
    const int64_t width = int64_t(a.Hv) * kGdnDim;
    const int64_t idx = int64_t(h) * kGdnDim + j;
    if (a.out_f32) a.out_f32[int64_t(t) * width + idx] = out;
    gdn_quantize(out, t, T, width, idx, j, a.act_out);
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

namespace {
template <int NT>
void gdn_decode_dispatch(const GdnDecodeArgs& a, hipStream_t s) {
    const dim3 grid(unsigned(a.Hv), unsigned(a.B));
    const size_t sm = sizeof(GdnDecodeShared);
    switch (a.W) {
        case 1: hipLaunchKernelGGL((gdn_decode_kernel<1, NT>), grid, dim3(NT), sm, s, a); break;
        case 2: hipLaunchKernelGGL((gdn_decode_kernel<2, NT>), grid, dim3(NT), sm, s, a); break;
        case 3: hipLaunchKernelGGL((gdn_decode_kernel<3, NT>), grid, dim3(NT), sm, s, a); break;
        case 4: hipLaunchKernelGGL((gdn_decode_kernel<4, NT>), grid, dim3(NT), sm, s, a); break;
        case 5: hipLaunchKernelGGL((gdn_decode_kernel<5, NT>), grid, dim3(NT), sm, s, a); break;
        case 6: hipLaunchKernelGGL((gdn_decode_kernel<6, NT>), grid, dim3(NT), sm, s, a); break;
        case 7: hipLaunchKernelGGL((gdn_decode_kernel<7, NT>), grid, dim3(NT), sm, s, a); break;
        default: hipLaunchKernelGGL((gdn_decode_kernel<8, NT>), grid, dim3(NT), sm, s, a); break;
    }
}
}  // namespace

void launch_gdn_decode(const GdnDecodeArgs& a, hipStream_t s) {
    // 512 lanes (32 state rows each) while every (sequence, head) gets a CU of
    // its own; with more workgroups than CUs, 256 lanes (64 rows each), so
    // that two fit per CU and every workgroup runs at once
    if (int64_t(a.Hv) * a.B > device_cus())
        gdn_decode_dispatch<256>(a, s);
    else
        gdn_decode_dispatch<kGdnThreads>(a, s);
}

void launch_gdn_decode_cols(const GdnDecodeArgs& a, float* o_raw, float* g_raw, hipStream_t s) {
    const dim3 grid(unsigned(a.Hv * kGdnSlices), unsigned(a.B));
    switch (a.W) {
        case 1: hipLaunchKernelGGL(gdn_decode_cols_kernel<1>, grid, dim3(64), 0, s, a, o_raw, g_raw); break;
        case 2: hipLaunchKernelGGL(gdn_decode_cols_kernel<2>, grid, dim3(64), 0, s, a, o_raw, g_raw); break;
        case 3: hipLaunchKernelGGL(gdn_decode_cols_kernel<3>, grid, dim3(64), 0, s, a, o_raw, g_raw); break;
        case 4: hipLaunchKernelGGL(gdn_decode_cols_kernel<4>, grid, dim3(64), 0, s, a, o_raw, g_raw); break;
        case 5: hipLaunchKernelGGL(gdn_decode_cols_kernel<5>, grid, dim3(64), 0, s, a, o_raw, g_raw); break;
        case 6: hipLaunchKernelGGL(gdn_decode_cols_kernel<6>, grid, dim3(64), 0, s, a, o_raw, g_raw); break;
        case 7: hipLaunchKernelGGL(gdn_decode_cols_kernel<7>, grid, dim3(64), 0, s, a, o_raw, g_raw); break;
        default: hipLaunchKernelGGL(gdn_decode_cols_kernel<8>, grid, dim3(64), 0, s, a, o_raw, g_raw); break;
    }
}

void launch_gdn_norm_gate(const float* o_raw, const GdnDecodeArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(gdn_norm_gate_kernel, dim3(unsigned(a.Hv), unsigned(a.B)), dim3(kGdnDim), 0, s, o_raw, a.proj, a.proj_stride, a.z_off, a.norm_gamma, a.eps,
                       a.act_out, a.out_f32, a.B, a.Hv);
}

int64_t gdn_prefill_work_bytes(int64_t T, int64_t Hk, int64_t Hv) {
    // q, k; v, o; beta, decay, g; u, wm; G; p
    return (T * (2 * Hk * kGdnDim + 2 * Hv * kGdnDim + 3 * Hv + 2 * Hv * kGdnDim + Hv) + (T + 63) / 64 * Hv * 64 * 64) * 4;
}

void launch_gdn_prefill(const GdnDecodeArgs& a, void* work, hipStream_t s, bool chunked) {
    const dim3 prep(unsigned(a.Hk + a.Hv), unsigned(a.B));
    switch (a.W) {
        case 1: hipLaunchKernelGGL(gdn_prep_kernel<1>, prep, dim3(kGdnDim), 0, s, a, work); break;
        case 2: hipLaunchKernelGGL(gdn_prep_kernel<2>, prep, dim3(kGdnDim), 0, s, a, work); break;
        case 3: hipLaunchKernelGGL(gdn_prep_kernel<3>, prep, dim3(kGdnDim), 0, s, a, work); break;
        case 4: hipLaunchKernelGGL(gdn_prep_kernel<4>, prep, dim3(kGdnDim), 0, s, a, work); break;
        case 5: hipLaunchKernelGGL(gdn_prep_kernel<5>, prep, dim3(kGdnDim), 0, s, a, work); break;
        case 6: hipLaunchKernelGGL(gdn_prep_kernel<6>, prep, dim3(kGdnDim), 0, s, a, work); break;
        case 7: hipLaunchKernelGGL(gdn_prep_kernel<7>, prep, dim3(kGdnDim), 0, s, a, work); break;
        default: hipLaunchKernelGGL(gdn_prep_kernel<8>, prep, dim3(kGdnDim), 0, s, a, work); break;
    }
    if (chunked)
    {
        hipLaunchKernelGGL(gdn_chunk_prep_kernel, dim3(unsigned((a.B + kChunk - 1) / kChunk), unsigned(a.Hv)), dim3(256), kChunkPrepShared, s, a, work);
        hipLaunchKernelGGL(gdn_chunk_scan_kernel, dim3(unsigned(a.Hv), unsigned(kGdnDim / kChunkCols)), dim3(256), kChunkScanShared, s, a, work);
    }
    else
        hipLaunchKernelGGL(gdn_scan_cols_kernel, dim3(unsigned(a.Hv * (kGdnDim / kScCols))), dim3(256), 0, s, a, work);
    hipLaunchKernelGGL(gdn_out_kernel, dim3(unsigned(a.Hv), unsigned(a.B)), dim3(kGdnDim), 0, s, a, work);
    const int64_t CC = 2 * int64_t(a.Hk) * kGdnDim + int64_t(a.Hv) * kGdnDim;
    const int64_t n = int64_t(std::min(a.B, a.W)) * CC;
    hipLaunchKernelGGL(gdn_hist_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, s, a.proj, a.proj_stride, a.conv_hist, CC, a.W, a.positions, a.B);
}

}  // namespace hero
