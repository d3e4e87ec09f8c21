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
// and the ring are sequence 0's. Three kernels:
//  prep  (token, head) in parallel: conv + SiLU, L2 norms and the query scale,
//        beta and the decay -- nothing here depends on the state;
//  scan  one workgroup per value head runs the delta rule over the tokens in
//        order, the state column of lane j in registers for the whole chunk;
//  out   (token, head) in parallel: head RMSNorm, SiLU(z) gate, quantize.
// The scan's critical path per token is one 128-term chain: token t's output
// chain and token t+1's decay and prediction chain read the same updated
// column, so they run in one pass over i. Every value is computed by the same
// operations in the same order as in gdn_decode_kernel.
constexpr int kScanTile = 16;   // tokens staged in shared memory per tile
constexpr int kScanChunk = 16;  // state rows per fenced step of the token loop
__device__ __forceinline__ void scan_fence() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);  // and no instruction scheduled across it
}

__device__ __forceinline__ GdnPrefillWork gdn_work(void* ws, int64_t T, int Hk, int Hv) {
    GdnPrefillWork w;
    float* f = static_cast<float*>(ws);
    w.q = f;
    w.k = w.q + T * Hk * kGdnDim;
    w.v = w.k + T * Hk * kGdnDim;
    w.o = w.v + T * Hv * kGdnDim;
    w.bd = w.o + T * Hv * kGdnDim;
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
        }
    }
}

// one tile of kScanTile tokens of a head: q, k (its key head), v, (beta, decay)
struct ScanTile {
    float q[kScanTile][kGdnDim];
    float k[kScanTile][kGdnDim];
    float v[kScanTile][kGdnDim];
    float bd[kScanTile][2];
};
constexpr int kScanVec = 3 * kScanTile * kGdnDim / 4 / kGdnDim;  // float4 per lane per tile (12)

__global__ __launch_bounds__(kGdnDim) void gdn_scan_kernel(GdnDecodeArgs a, void* ws) {
    const int j = threadIdx.x, h = blockIdx.x, hk = h % a.Hk;
    const int T = a.B;
    if (a.positions[0] < 0) return;
    const GdnPrefillWork w = gdn_work(ws, T, a.Hk, a.Hv);
    float* S = a.state + int64_t(h) * kGdnState;
    __shared__ __align__(16) ScanTile tiles[2];
    const int ntiles = (T + kScanTile - 1) / kScanTile;

    // tile loads: float4 f = j + 128u; u < 4: q, u < 8: k, else v; token (f % 512) / 32
    float4 pre[kScanVec];
    float2 pre_bd = make_float2(0.f, 0.f);
    auto load = [&](int tile) {
        const int t0 = tile * kScanTile;
#pragma unroll
        for (int u = 0; u < kScanVec; ++u) {
            const int f = (j + kGdnDim * u) % (kScanTile * kGdnDim / 4);
            const int tt = t0 + f / (kGdnDim / 4), c4 = f % (kGdnDim / 4);
            const float* src = u < 4 ? w.q + (int64_t(tt) * a.Hk + hk) * kGdnDim : u < 8 ? w.k + (int64_t(tt) * a.Hk + hk) * kGdnDim : w.v + (int64_t(tt) * a.Hv + h) * kGdnDim;
            pre[u] = tt < T ? reinterpret_cast<const float4*>(src)[c4] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (j < kScanTile && t0 + j < T) pre_bd = reinterpret_cast<const float2*>(w.bd)[int64_t(t0 + j) * a.Hv + h];
    };
    auto store = [&](ScanTile& dst) {
#pragma unroll
        for (int u = 0; u < kScanVec; ++u) {
            const int f = (j + kGdnDim * u) % (kScanTile * kGdnDim / 4);
            float* base = u < 4 ? &dst.q[0][0] : u < 8 ? &dst.k[0][0] : &dst.v[0][0];
            reinterpret_cast<float4*>(base)[f] = pre[u];
        }
        if (j < kScanTile) {
            dst.bd[j][0] = pre_bd.x;
            dst.bd[j][1] = pre_bd.y;
        }
    };

    float col[kGdnDim];  // S[i][j], i = 0..127: this lane's state column
#pragma unroll
    for (int i = 0; i < kGdnDim; ++i) col[i] = S[i * kGdnDim + j];
    load(0);
    store(tiles[0]);
    if (ntiles > 1) {
        load(1);
        store(tiles[1]);
    }
    if (ntiles > 2) load(2);
    __syncthreads();

    // token 0: decay and prediction chain
    float pred = 0.f;
    {
        const float dec = tiles[0].bd[0][1];
        const float* kn = tiles[0].k[0];
#pragma unroll
        for (int i0 = 0; i0 < kGdnDim; i0 += 4) {
            const float4 k4 = *reinterpret_cast<const float4*>(kn + i0);
            col[i0 + 0] = col[i0 + 0] * dec;
            pred = pred + col[i0 + 0] * k4.x;
            col[i0 + 1] = col[i0 + 1] * dec;
            pred = pred + col[i0 + 1] * k4.y;
            col[i0 + 2] = col[i0 + 2] * dec;
            pred = pred + col[i0 + 2] * k4.z;
            col[i0 + 3] = col[i0 + 3] * dec;
            pred = pred + col[i0 + 3] * k4.w;
        }
    }
    for (int t = 0; t < T; ++t) {
        const int tile = t / kScanTile, r = t % kScanTile;
        if (r == 0 && tile > 0) {
            // tile-1's buffer is free: it takes tile+1 (loaded a tile ago)
            __syncthreads();
            if (tile + 1 < ntiles) store(tiles[(tile + 1) & 1]);
            if (tile + 2 < ntiles) load(tile + 2);
            __syncthreads();
        }
        const ScanTile& cur = tiles[tile & 1];
        const float* qt = cur.q[r];
        const float* kt = cur.k[r];
        const float delta = (cur.v[r][j] - pred) * cur.bd[r][0];
        float o = 0.f;
        if (t + 1 < T) {
            const ScanTile& nxt = tiles[((t + 1) / kScanTile) & 1];
            const int rn = (t + 1) % kScanTile;
            const float* kn = nxt.k[rn];
            const float dec = nxt.bd[rn][1];
            float pn = 0.f;
            // k, q and the next k in chunks of kScanChunk rows, the next
            // chunk's shared-memory reads in flight while this one computes
            float4 bk[2][kScanChunk / 4], bq[2][kScanChunk / 4], bn[2][kScanChunk / 4];
            auto fetch = [&](int c, int buf) {
#pragma unroll
                for (int u = 0; u < kScanChunk / 4; ++u) {
                    bk[buf][u] = *reinterpret_cast<const float4*>(kt + c * kScanChunk + 4 * u);
                    bq[buf][u] = *reinterpret_cast<const float4*>(qt + c * kScanChunk + 4 * u);
                    bn[buf][u] = *reinterpret_cast<const float4*>(kn + c * kScanChunk + 4 * u);
                }
            };
            fetch(0, 0);
#pragma unroll
            for (int c = 0; c < kGdnDim / kScanChunk; ++c) {
                if (c + 1 < kGdnDim / kScanChunk) fetch(c + 1, (c + 1) & 1);
                scan_fence();
#pragma unroll
                for (int u = 0; u < kScanChunk / 4; ++u) {
                    const float4 k4 = bk[c & 1][u], q4 = bq[c & 1][u], n4 = bn[c & 1][u];
                    const float kk[4] = {k4.x, k4.y, k4.z, k4.w}, qq[4] = {q4.x, q4.y, q4.z, q4.w}, nn[4] = {n4.x, n4.y, n4.z, n4.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int i = c * kScanChunk + 4 * u + e;
                        float v = col[i] + kk[e] * delta;  // S[i][j] += k[i] * delta
                        o = o + v * qq[e];                 // o += S[i][j] * q[i]
                        v = v * dec;                       // next token: S[i][j] *= decay
                        pn = pn + v * nn[e];               //             pred += S[i][j] * k[i]
                        col[i] = v;
                    }
                }
            }
            pred = pn;
        } else {
#pragma unroll
            for (int i1 = 0; i1 < kGdnDim; i1 += kScanChunk) {
                scan_fence();
#pragma unroll
                for (int i0 = i1; i0 < i1 + kScanChunk; i0 += 4) {
                    const float4 k4 = *reinterpret_cast<const float4*>(kt + i0);
                    const float4 q4 = *reinterpret_cast<const float4*>(qt + i0);
                    const float kk[4] = {k4.x, k4.y, k4.z, k4.w}, qq[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float v = col[i0 + e] + kk[e] * delta;
                        o = o + v * qq[e];
                        col[i0 + e] = v;
                    }
                }
            }
        }
        w.o[(int64_t(t) * a.Hv + h) * kGdnDim + j] = o;
    }
    // a fresh base pointer: otherwise the 128 row addresses of the first
    // loads are kept alive across the token loop for these stores
    float* Sw = S;
    __asm__ volatile("" : "+s"(Sw));
#pragma unroll
    for (int i = 0; i < kGdnDim; ++i) Sw[i * kGdnDim + j] = col[i];
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

int64_t gdn_prefill_work_bytes(int64_t T, int64_t Hk, int64_t Hv) { return T * (2 * Hk * kGdnDim + 2 * Hv * kGdnDim + 2 * Hv) * 4; }

void launch_gdn_prefill(const GdnDecodeArgs& a, void* work, hipStream_t s) {
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
    hipLaunchKernelGGL(gdn_scan_kernel, dim3(unsigned(a.Hv)), dim3(kGdnDim), 0, s, a, work);
    hipLaunchKernelGGL(gdn_out_kernel, dim3(unsigned(a.Hv), unsigned(a.B)), dim3(kGdnDim), 0, s, a, work);
    const int64_t CC = 2 * int64_t(a.Hk) * kGdnDim + int64_t(a.Hv) * kGdnDim;
    const int64_t n = int64_t(std::min(a.B, a.W)) * CC;
    hipLaunchKernelGGL(gdn_hist_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, s, a.proj, a.proj_stride, a.conv_hist, CC, a.W, a.positions, a.B);
}

}  // namespace hero
