// gemma.hip -- the kernels of the Gemma 4 text model's decode step that the
// Qwen path does not have: the scaled embedding and per-layer inputs (PLE),
// the per-head norms with RoPE and the cache append, GQA attention with score
// scale 1 over a full or a sliding-window (ring) cache, the post-norm +
// residual + next norm step that closes every sub-block, the GELU-gated
// products and the logit soft-cap.
//
// Every fp32 expression follows the reference's operation order (see the
// comment of each kernel); sums the reference forms sequentially are summed
// exactly that way (hero/seqsum.hpp), tanh and exp are glibc's (hero/libm.hpp).
#include "hero/device.hpp"
#include "hero/kernels.hpp"
#include "hero/seqsum.hpp"

namespace hero {

// ---- embedding and per-layer inputs -----------------------------------------------
// x = dequant_row(id) * embed_scale (Gemma4E4BModel::embed, nm/src/gemma4.hpp:415-419),
// its Q8_0 quantization (the PLE projection's input), and the token part of
// the per-layer inputs tok = dequant_row(id) * token_scale of the packed table
// (GemmaPerLayerInputs, nm/src/gemma4.hpp:129-131). A lane per 8 values; the
// quads of x are whole Q8_0 blocks.
__global__ __launch_bounds__(256) void gemma_embed_kernel(const int8_t* __restrict__ eq, const uint16_t* __restrict__ ed, int64_t D, const int8_t* __restrict__ pq,
                                                          const uint16_t* __restrict__ pd, int64_t PL, const int32_t* __restrict__ id_ptr, float embed_scale,
                                                          float token_scale, float* __restrict__ x, int8_t* __restrict__ xq, float* __restrict__ xd,
                                                          float* __restrict__ tok) {
    const int64_t lane = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t id = *id_ptr;
    const int64_t gx = D / 8;
    if (lane < gx) {
        const int64_t c0 = lane * 8;
        const float d = half_bits_to_f32(ed[scale_index(id, c0 >> 5, D >> 5)]);
        const int2 q = reinterpret_cast<const int2*>(eq + id * D)[lane];
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int8_t b = int8_t(((k < 4 ? q.x : q.y) >> (8 * (k & 3))) & 0xFF);
            v[k] = d * float(b) * embed_scale;
        }
        reinterpret_cast<float4*>(x + c0)[0] = make_float4(v[0], v[1], v[2], v[3]);
        reinterpret_cast<float4*>(x + c0)[1] = make_float4(v[4], v[5], v[6], v[7]);
        uint16_t dh;
        reinterpret_cast<int2*>(xq)[lane] = quantize8_in_quad(v, &dh);
        if ((lane & 3) == 0) xd[lane >> 2] = half_bits_to_f32(dh);
        return;
    }
    const int64_t t = lane - gx;
    if (t >= PL / 8) return;
    const int64_t c0 = t * 8;
    const float d = half_bits_to_f32(pd[scale_index(id, c0 >> 5, PL >> 5)]);
    const int2 q = reinterpret_cast<const int2*>(pq + id * PL)[t];
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int8_t b = int8_t(((k < 4 ? q.x : q.y) >> (8 * (k & 3))) & 0xFF);
        v[k] = d * float(b) * token_scale;
    }
    reinterpret_cast<float4*>(tok + c0)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(tok + c0)[1] = make_float4(v[4], v[5], v[6], v[7]);
}

void launch_gemma_embed(const void* emb, int64_t V, int64_t D, const void* ple_table, int64_t PL, const int32_t* id, float embed_scale, float token_scale, float* x,
                        void* act, float* tok, hipStream_t s) {
    const int8_t* eq = static_cast<const int8_t*>(emb);
    const int8_t* pq = static_cast<const int8_t*>(ple_table);
    int8_t* xq = static_cast<int8_t*>(act);
    const int64_t lanes = D / 8 + PL / 8;
    hipLaunchKernelGGL(gemma_embed_kernel, dim3(unsigned((lanes + 255) / 256)), dim3(256), 0, s, eq, reinterpret_cast<const uint16_t*>(eq + V * D), D, pq,
                       reinterpret_cast<const uint16_t*>(pq + V * PL), PL, id, embed_scale, token_scale, x, xq, reinterpret_cast<float*>(xq + D), tok);
}

// The per-layer inputs of one row (GemmaPerLayerInputs, nm/src/gemma4.hpp:127-135):
// c = ctx * proj_scale; c = RMSNorm_P(c) with the shared weight, per layer
// slice; ple = (c + tok) * comb (scaled_sum, core.hpp:509-513). A workgroup of
// 256 lanes per layer slice of P values.
__global__ __launch_bounds__(256) void gemma_ple_kernel(const float* __restrict__ ctx, const float* __restrict__ tok, const float* __restrict__ gamma, float eps,
                                                        float proj_scale, float comb, float* __restrict__ ple, int P) {
    constexpr int NT = 256;
    __shared__ seqsum::Shared sm;
    __shared__ __align__(16) float sq[seqsum::kMaxN];
    const int64_t base = int64_t(blockIdx.x) * P;
    const int tid = threadIdx.x;
    for (int i = tid; i < seqsum::kMaxN; i += NT) {
        float v = 0.f;
        if (i < P) {
            const float c = ctx[base + i] * proj_scale;
            v = c * c;
        }
        sq[i] = v;
    }
    __syncthreads();
    const float s = seqsum::sum_nonneg<NT>(sq, P, sm);
    const float inv = 1.f / sqrtf(s / float(P) + eps);
    for (int i = tid; i < P; i += NT) {
        const float c = ctx[base + i] * proj_scale;
        const float n = gamma[i] * c * inv;
        ple[base + i] = (n + tok[base + i]) * comb;
    }
}

void launch_gemma_ple_inputs(const float* ctx, const float* tok, const float* gamma, float eps, float proj_scale, float comb, float* ple, int64_t L, int64_t P,
                             hipStream_t s) {
    hipLaunchKernelGGL(gemma_ple_kernel, dim3(unsigned(L)), dim3(256), 0, s, ctx, tok, gamma, eps, proj_scale, comb, ple, int(P));
}

// ---- attention -----------------------------------------------------------------------
// Position p lives in slot p % slots of a ring (window > 0) or slot p; the
// visible positions of a row at `pos` are [first, pos], first =
// max(0, pos + 1 - window) (CausalWindow::visible_rows, nm/src/attention.hpp:170-176).
// Slots are walked from first's slot with one wrap (n <= slots).
struct GemmaSpan {
    int first, n, slot0, slots;
    __device__ __forceinline__ int slot(int t) const {
        const int s = slot0 + t;
        return s >= slots ? s - slots : s;
    }
};
__device__ __forceinline__ GemmaSpan gemma_span(const GemmaAttnArgs& a) {
    const int pos = *a.pos;
    GemmaSpan v;
    v.first = (a.window > 0 && pos + 1 > a.window) ? pos + 1 - a.window : 0;
    v.n = pos + 1 - v.first;
    v.slots = int(a.slots);
    v.slot0 = a.window > 0 ? v.first % v.slots : v.first;
    return v;
}

// The sequential sum of n <= 4096 floats in shared memory by lane 0 (float4
// reads): the reference's loop, for sums short enough that one dependent
// chain beats the parallel exact form.
__device__ __forceinline__ float serial_sum_lds(const float* p, int n) {
    float s = 0.f;
    const float4* p4 = reinterpret_cast<const float4*>(p);
    int i = 0;
    for (; i + 32 <= n; i += 32) {  // 32 values read before their adds (one latency per 32)
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = p4[i / 4 + u];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            s += v[u].x;
            s += v[u].y;
            s += v[u].z;
            s += v[u].w;
        }
    }
    for (; i + 4 <= n; i += 4) {
        const float4 v = p4[i / 4];
        s += v.x;
        s += v.y;
        s += v.z;
        s += v.w;
    }
    for (; i < n; ++i) s += p[i];
    return s;
}

// One head of DH values, a lane per value: RMSNorm over the head (the learned
// weight gamma, or none for V; PerHeadNorm, components.hpp:248-258, with
// RMSNorm :176-181 or RMSNormNoScale :210-215), then with cs RoPE on the
// planes (i, i + DH/2) from the position's (cos, sin) row (RotaryEmbedding,
// nm/src/attention.hpp:82-91; unrotated planes carry (1, 0)).
template <int DH>
__device__ __forceinline__ float gemma_head(float x, const float* gamma, float eps, const float* cs, float* buf, float* scal) {
    const int j = threadIdx.x;
    buf[j] = x * x;
    __syncthreads();
    if (j == 0) scal[0] = 1.f / sqrtf(serial_sum_lds(buf, DH) / float(DH) + eps);
    __syncthreads();
    const float n = gamma ? gamma[j] * x * scal[0] : x * scal[0];
    if (!cs) return n;
    buf[j] = n;
    __syncthreads();
    constexpr int half = DH / 2;
    const int i = j < half ? j : j - half;
    const float c = cs[2 * i], sn = cs[2 * i + 1];
    const float xx = buf[i], yy = buf[i + half];
    return j < half ? xx * c - yy * sn : yy * c + xx * sn;
}

// Workgroups [0, Hq): query head h -> q_rot; with append, [Hq, Hq + Hkv): key
// head g -> K cache; [Hq + Hkv, Hq + 2 Hkv): value head g -> V cache, at the
// position's slot. Q = rope(q_norm(WQ x)), K = rope(k_norm(WK x)),
// V = v_norm(WV x) (GemmaE4BLayer::attention, nm/src/gemma4.hpp:205-208).
template <int DH>
__global__ __launch_bounds__(DH) void gemma_attn_prep_kernel(GemmaAttnArgs a) {
    __shared__ __align__(16) float buf[DH];
    __shared__ float scal[1];
    const int j = threadIdx.x, blk = blockIdx.x;
    const int pos = *a.pos;
    const float* cs = a.rope_cs + int64_t(pos) * DH;  // [DH/2][2]
    if (blk < a.Hq) {
        a.q_rot[int64_t(blk) * DH + j] = gemma_head<DH>(a.proj[int64_t(blk) * DH + j], a.q_gamma, a.eps, cs, buf, scal);
        return;
    }
    const int64_t slot = a.window > 0 ? pos % a.slots : pos;
    const int g = blk - a.Hq;
    if (g < a.Hkv) {
        a.k_cache[(int64_t(g) * a.slots + slot) * DH + j] = gemma_head<DH>(a.proj[a.k_off + int64_t(g) * DH + j], a.k_gamma, a.eps, cs, buf, scal);  // [Hkv][slots][DH]
        return;
    }
    const int gv = g - a.Hkv;
    a.v_cache[(int64_t(gv) * a.slots + slot) * DH + j] = gemma_head<DH>(a.proj[a.v_off + int64_t(gv) * DH + j], nullptr, a.eps, nullptr, buf, scal);  // [Hkv][slots][DH]
}

// Scores s_t = dot(q_h, k_t), each the sequential DH-term sum (core.hpp:496-500;
// no score scale: Gemma folds it into the Q norm, gemma4.hpp:197-200).
// Workgroup (KV head g, tile y): 64 positions per tile, tiles y, y + gridDim.y,
// ...; the tile's key rows are staged in shared memory (all its 16-byte loads
// in flight together; rows padded by one float: conflict-free column reads),
// then wave w forms heads w, w + 4, ... of the group, a lane per position.
constexpr int kGsTile = 64;

template <int DH>
__global__ __launch_bounds__(256) void gemma_scores_kernel(GemmaAttnArgs a) {
    constexpr int KS = DH + 1;  // padded key row
    extern __shared__ __align__(16) float kt[];  // [kGsTile][KS], then q [group][DH]
    float* q = kt + kGsTile * KS;
    const int g = blockIdx.x, group = a.Hq / a.Hkv;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const GemmaSpan sp = gemma_span(a);
    for (int i = tid; i < group * DH; i += 256) q[i] = a.q_rot[int64_t(g) * group * DH + i];
    const float* kh = a.k_cache + int64_t(g) * a.slots * DH;
    const int tiles = (sp.n + kGsTile - 1) / kGsTile;
    constexpr int Q4 = DH / 4;                    // float4s per key row
    constexpr int LOADS = kGsTile * Q4 / 256;     // per lane: 16 (DH 256) or 32 (DH 512)
    for (int tile = blockIdx.y; tile < tiles; tile += gridDim.y) {
        const int t0 = tile * kGsTile;
        float4 v[LOADS];
#pragma unroll
        for (int k = 0; k < LOADS; ++k) {
            const int e = tid + 256 * k, key = e / Q4, c4 = e % Q4;
            v[k] = t0 + key < sp.n ? reinterpret_cast<const float4*>(kh + int64_t(sp.slot(t0 + key)) * DH)[c4] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        __syncthreads();  // the previous tile's readers are done
#pragma unroll
        for (int k = 0; k < LOADS; ++k) {
            const int e = tid + 256 * k, key = e / Q4, c4 = e % Q4;
            float* dst = kt + key * KS + 4 * c4;
            dst[0] = v[k].x, dst[1] = v[k].y, dst[2] = v[k].z, dst[3] = v[k].w;
        }
        __syncthreads();
        const int t = t0 + lane;
        if (t < sp.n) {
            const float* kr = kt + lane * KS;
            for (int hh = wave; hh < group; hh += 4) {
                const float* qh = q + hh * DH;
                float dot = 0.f;
#pragma unroll 16
                for (int c = 0; c < DH; ++c) dot += qh[c] * kr[c];
                a.scores[int64_t(g * group + hh) * a.max_ctx + t] = dot;
            }
        }
    }
}

// gemma_head's operations for one head by one wave: lane l holds the values
// l + 64 m; buf is the wave's DH floats of shared memory (the squares, then
// the normed values for the RoPE pairs). A wave's shared-memory accesses take
// effect in order, so it needs no barrier.
template <int DH>
__device__ __forceinline__ void gemma_head_wave(const float* x, const float* gamma, float eps, const float* cs, float* buf, float* out) {
    constexpr int PL = DH / 64;
    const int lane = threadIdx.x & 63;
    float v[PL];
#pragma unroll
    for (int m = 0; m < PL; ++m) v[m] = x[lane + 64 * m];
#pragma unroll
    for (int m = 0; m < PL; ++m) buf[lane + 64 * m] = v[m] * v[m];
    float sc = 0.f;
    if (lane == 0) sc = 1.f / sqrtf(serial_sum_lds(buf, DH) / float(DH) + eps);
    sc = __shfl(sc, 0);
    float n[PL];
#pragma unroll
    for (int m = 0; m < PL; ++m) n[m] = gamma ? gamma[lane + 64 * m] * v[m] * sc : v[m] * sc;
    if (!cs) {
#pragma unroll
        for (int m = 0; m < PL; ++m) out[lane + 64 * m] = n[m];
        return;
    }
#pragma unroll
    for (int m = 0; m < PL; ++m) buf[lane + 64 * m] = n[m];
    constexpr int half = DH / 2;
#pragma unroll
    for (int m = 0; m < PL; ++m) {
        const int j = lane + 64 * m, i = j < half ? j : j - half;
        const float c = cs[2 * i], sn = cs[2 * i + 1];
        const float xx = buf[i], yy = buf[i + half];
        out[j] = j < half ? xx * c - yy * sn : yy * c + xx * sn;
    }
}

// The prep step folded into the scores: workgroup (KV head g, tile y) forms
// its group's query heads itself (one wave per head, gemma_head's
// operations) while its first tile's key rows land, and the workgroup whose
// tiles include the new position also forms that position's key and value
// (appending them to the caches) and puts the key into its tile in place of
// the cached row. Then the scores exactly as gemma_scores_kernel.
// Eight waves: every head's prep (the group's queries, and the new key and
// value) runs at once, one wave each.
constexpr int kPsThreads = 512, kPsWaves = kPsThreads / 64;
template <int DH>
constexpr size_t prep_scores_shared(int group) { return size_t(kGsTile * (DH + 1) + group * DH + DH + kPsWaves * DH) * 4; }

template <int DH>
__global__ __launch_bounds__(kPsThreads) void gemma_prep_scores_kernel(GemmaAttnArgs a) {
    constexpr int KS = DH + 1;  // padded key row
    extern __shared__ __align__(16) float kt[];  // [kGsTile][KS], q [group][DH], knew [DH], per-wave [kPsWaves][DH]
    const int g = blockIdx.x, group = a.Hq / a.Hkv;
    float* q = kt + kGsTile * KS;
    float* knew = q + group * DH;
    float* hb = knew + DH;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const GemmaSpan sp = gemma_span(a);
    const int tiles = (sp.n + kGsTile - 1) / kGsTile;
    if (int(blockIdx.y) >= tiles) return;  // no tile for this workgroup
    const int pos = sp.first + sp.n - 1;
    const int ptile = (sp.n - 1) / kGsTile, prow = (sp.n - 1) % kGsTile;  // the new position's tile and row
    const bool has_pos = a.append && ptile % int(gridDim.y) == int(blockIdx.y);
    const float* kh = a.k_cache + int64_t(g) * a.slots * DH;
    constexpr int Q4 = DH / 4;                    // float4s per key row
    constexpr int LOADS = kGsTile * Q4 / kPsThreads;  // per lane: 8 (DH 256) or 16 (DH 512)
    float4 v[LOADS];
    auto load_tile = [&](int tile) {
        const int t0 = tile * kGsTile;
#pragma unroll
        for (int k = 0; k < LOADS; ++k) {
            const int e = tid + kPsThreads * k, key = e / Q4, c4 = e % Q4;
            v[k] = t0 + key < sp.n ? reinterpret_cast<const float4*>(kh + int64_t(sp.slot(t0 + key)) * DH)[c4] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    int tile = blockIdx.y;
    load_tile(tile);
    // Q = rope(q_norm(WQ x)); with append, K = rope(k_norm(WK x)) and
    // V = v_norm(WV x) of the position (GemmaE4BLayer::attention,
    // nm/src/gemma4.hpp:205-208)
    const float* cs = a.rope_cs + int64_t(pos) * DH;  // [DH/2][2]
    const int64_t slot = a.window > 0 ? pos % a.slots : pos;
    const int items = group + (has_pos ? 2 : 0);
    for (int it = wave; it < items; it += kPsWaves) {
        float* buf = hb + wave * DH;
        if (it < group) {
            gemma_head_wave<DH>(a.proj + int64_t(g * group + it) * DH, a.q_gamma, a.eps, cs, buf, q + it * DH);
        } else if (it == group) {
            gemma_head_wave<DH>(a.proj + a.k_off + int64_t(g) * DH, a.k_gamma, a.eps, cs, buf, knew);
            float* kc = a.k_cache + (int64_t(g) * a.slots + slot) * DH;  // [Hkv][slots][DH]
            for (int c = lane; c < DH; c += 64) kc[c] = knew[c];
        } else {
            gemma_head_wave<DH>(a.proj + a.v_off + int64_t(g) * DH, nullptr, a.eps, nullptr, buf, a.v_cache + (int64_t(g) * a.slots + slot) * DH);
        }
    }
    while (true) {
        const int t0 = tile * kGsTile;
        __syncthreads();  // the previous tile's readers are done; the first time, the prep's results
        const bool patch = has_pos && tile == ptile;
#pragma unroll
        for (int k = 0; k < LOADS; ++k) {
            const int e = tid + kPsThreads * k, key = e / Q4, c4 = e % Q4;
            const float4 x = patch && key == prow ? reinterpret_cast<const float4*>(knew)[c4] : v[k];
            float* dst = kt + key * KS + 4 * c4;
            dst[0] = x.x, dst[1] = x.y, dst[2] = x.z, dst[3] = x.w;
        }
        __syncthreads();
        const int t = t0 + lane;
        if (t < sp.n) {
            const float* kr = kt + lane * KS;
            for (int hh = wave; hh < group; hh += kPsWaves) {
                const float* qh = q + hh * DH;
                float dot = 0.f;
#pragma unroll 16
                for (int c = 0; c < DH; ++c) dot += qh[c] * kr[c];
                a.scores[int64_t(g * group + hh) * a.max_ctx + t] = dot;
            }
        }
        tile += gridDim.y;
        if (tile >= tiles) break;
        load_tile(tile);
    }
}

// The softmax of head h's n scores (components.hpp:131-141: e_t = exp(s_t - max),
// their sequential sum in chunks, each starting with the running total,
// alpha_t = e_t / total) and the weighted sum of its value rows for 64
// channels, out[c] = sum_t alpha_t v_t[c] in order (Vec::scaled_add,
// core.hpp:206-208: out += alpha * v), then the two Q8_0 blocks of the W_o input
// those channels make (quantize_row_q8_0, quant_i8.hpp:70-80).
// Workgroup (head, 64 channels) of 256 lanes: chunks of kPvChunk positions,
// each chunk's value rows loaded by all lanes (the next chunk's loads in
// flight while wave 0, a lane per channel, runs the current chunk's chain
// out of shared memory).
constexpr int kPvChunk = 128;

template <int DH>
__global__ __launch_bounds__(256) void gemma_softmax_pv_kernel(GemmaAttnArgs a) {
    __shared__ seqsum::Shared sm;
    __shared__ __align__(16) float chunk[seqsum::kMaxN];
    __shared__ __align__(16) float vb[2][kPvChunk][64];
    __shared__ __align__(16) float al[2][kPvChunk];
    __shared__ float red[4];
    const int tid = threadIdx.x;
    int h, part;
    head_part_of(int(blockIdx.x), a.Hq, a.Hkv, DH / 64, h, part);
    const int c0 = part * 64;
    const int g = h / (a.Hq / a.Hkv);
    const GemmaSpan sp = gemma_span(a);
    const int n = sp.n;
    const float* sc = a.scores + int64_t(h) * a.max_ctx;
    // value rows [slot][DH] of KV head g, channels c0 .. c0+63: the first
    // chunk's loads are issued before the softmax (they do not depend on it)
    const float* vh = a.v_cache + int64_t(g) * a.slots * DH + c0;
    constexpr int LOADS = kPvChunk * 16 / 256;  // float4s per lane: 8
    float4 v[LOADS];
    auto fetch = [&](int base) {
#pragma unroll
        for (int k = 0; k < LOADS; ++k) {
            const int e = tid + 256 * k, key = e >> 4, c4 = e & 15;
            v[k] = base + key < n ? reinterpret_cast<const float4*>(vh + int64_t(sp.slot(base + key)) * DH)[c4] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    fetch(0);
    constexpr int CH = seqsum::kMaxN - 256;
    // short spans (n <= CH): the scores are read once into the chunk buffer,
    // which then holds the exponentials, and the weights are formed from those
    const bool short_span = n <= CH;
    // max, then the exponentials' sequential sum (components.hpp:131-141)
    float mx = -INFINITY;
    for (int t = tid; t < n; t += 256) {
        const float st = sc[t];
        if (short_span) chunk[1 + t] = st;
        mx = fmaxf(mx, st);
    }
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float total = 0.f;
    for (int base = 0; base < n; base += CH) {
        const int len = min(n - base, CH);
        if (short_span) {
            for (int u = tid; u < len; u += 256) chunk[1 + u] = exp_f32(chunk[1 + u] - mx);  // each lane its own entries
        } else {
            __syncthreads();  // chunk free
            for (int u = tid; u < len; u += 256) chunk[1 + u] = exp_f32(sc[base + u] - mx);
        }
        if (tid == 0) chunk[0] = total;
        __syncthreads();
        if (len < 1024) {  // a short chain: one lane
            if (tid == 0) sm.result = serial_sum_lds(chunk, len + 1);
            __syncthreads();
            total = sm.result;
        } else {
            for (int u = len + 1 + tid; u < seqsum::kMaxN; u += 256) chunk[u] = 0.f;
            __syncthreads();
            total = seqsum::sum_nonneg<256>(chunk, len + 1, sm);
        }
    }
    // the weighted sum (Vec::scaled_add, core.hpp:206-208): out += alpha * v
    float acc = 0.f;
    int buf = 0;
    for (int base = 0; base < n; base += kPvChunk) {
#pragma unroll
        for (int k = 0; k < LOADS; ++k) {
            const int e = tid + 256 * k;
            reinterpret_cast<float4*>(&vb[buf][0][0])[e] = v[k];
        }
        if (tid < kPvChunk && base + tid < n) al[buf][tid] = (short_span ? chunk[1 + base + tid] : exp_f32(sc[base + tid] - mx)) / total;
        __syncthreads();
        if (base + kPvChunk < n) fetch(base + kPvChunk);
        if (tid < 64) {
            // reads 16 keys ahead of the chain (the weights as float4s), so the
            // adds do not wait on shared-memory latency key by key; the same
            // products, added in key order
            const int len = min(kPvChunk, n - base);
            int k0 = 0;
            for (; k0 + 16 <= len; k0 += 16) {
                float4 aw[4];
                float vv[16];
#pragma unroll
                for (int u = 0; u < 4; ++u) aw[u] = reinterpret_cast<const float4*>(&al[buf][k0])[u];
#pragma unroll
                for (int u = 0; u < 16; ++u) vv[u] = vb[buf][k0 + u][tid];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    acc += aw[u].x * vv[4 * u];
                    acc += aw[u].y * vv[4 * u + 1];
                    acc += aw[u].z * vv[4 * u + 2];
                    acc += aw[u].w * vv[4 * u + 3];
                }
            }
            for (int k = k0; k < len; ++k) acc += al[buf][k] * vb[buf][k][tid];
        }
        buf ^= 1;
    }
    if (tid >= 64) return;
    // Q8_0 of the 32-channel block this lane is in
    float amax = fabsf(acc);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    const float d = amax / 127.f;
    const float id = d != 0.f ? 1.f / d : 0.f;
    int8_t* qs = static_cast<int8_t*>(a.act_out);
    float* qd = reinterpret_cast<float*>(qs + int64_t(a.Hq) * DH);
    const int64_t idx = int64_t(h) * DH + c0 + tid;
    qs[idx] = int8_t(int(roundf(acc * id)));
    if ((tid & 31) == 0) qd[idx >> 5] = half_bits_to_f32(fp32_to_fp16_ref(d));
}

// The same for a sliding-window layer (at most kShortMax visible keys): the
// head's scores and the workgroup's whole value span (kShortMax rows x 64
// channels, 128 KB) go straight into shared memory at entry (untracked
// global_load_lds, each wave waiting for its own), so the value rows stream in
// while the softmax runs; the weights are formed once, then the chain runs out
// of shared memory. Same operations and order as gemma_softmax_pv_kernel.
constexpr int kShortMax = 512;

template <int DH>
__global__ __launch_bounds__(256) void gemma_softmax_pv_short_kernel(GemmaAttnArgs a) {
    __shared__ __align__(16) float vrows[kShortMax][64];
    __shared__ __align__(16) float ex[kShortMax];        // the scores, as loaded
    __shared__ __align__(16) float chunk[kShortMax + 4];  // [0] = 0, then the exponentials
    __shared__ __align__(16) float al[kShortMax];         // the weights
    __shared__ float red[4];
    __shared__ float tot;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    int h, part;
    head_part_of(int(blockIdx.x), a.Hq, a.Hkv, DH / 64, h, part);
    const int c0 = part * 64;
    const int g = h / (a.Hq / a.Hkv);
    const GemmaSpan sp = gemma_span(a);
    const int n = sp.n;  // 1 .. kShortMax (the host's condition)
    const float* sc = a.scores + int64_t(h) * a.max_ctx;
    const float* vh = a.v_cache + int64_t(g) * a.slots * DH + c0;
    // wave w: scores [128 w, 128 w + 128) (two 64-lane pieces), then value
    // rows 128 w .. 128 w + 127 (32 pieces of 4 rows); positions past n read
    // position n - 1 (never used)
#pragma unroll
    for (int k = 0; k < 2; ++k) lds_dma_b32(sc + min(wave * 128 + k * 64 + lane, n - 1), lds_offset(ex + wave * 128 + k * 64));
    for (int j = 0; j < 32; ++j) {
        const int kb = 4 * (32 * wave + j), row = min(kb + (lane >> 4), n - 1);
        lds_dma_b128(vh + int64_t(sp.slot(row)) * DH + 4 * (lane & 15), lds_offset(&vrows[kb][0]));
    }
    wait_vmcnt<32>();  // this wave's scores have landed
    __syncthreads();
    // max, then the exponentials' sequential sum (components.hpp:131-141)
    float mx = -INFINITY;
    for (int t = tid; t < n; t += 256) mx = fmaxf(mx, ex[t]);
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int u = tid; u < n; u += 256) chunk[1 + u] = exp_f32(ex[u] - mx);
    if (tid == 0) chunk[0] = 0.f;
    __syncthreads();
    if (tid == 0) tot = serial_sum_lds(chunk, n + 1);
    __syncthreads();
    const float total = tot;
    // the weights (zeros up to the next 16) for the chain's float4 reads
    for (int u = tid; u < (n + 15) / 16 * 16; u += 256) al[u] = u < n ? chunk[1 + u] / total : 0.f;
    wait_vmcnt<0>();  // this wave's value rows have landed
    __syncthreads();
    if (tid >= 64) return;
    // the weighted sum (Vec::scaled_add, core.hpp:206-208), 16 keys read ahead
    float acc = 0.f;
    int k0 = 0;
    for (; k0 + 16 <= n; k0 += 16) {
        float4 aw[4];
        float vv[16];
#pragma unroll
        for (int u = 0; u < 4; ++u) aw[u] = reinterpret_cast<const float4*>(&al[k0])[u];
#pragma unroll
        for (int u = 0; u < 16; ++u) vv[u] = vrows[k0 + u][tid];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            acc += aw[u].x * vv[4 * u];
            acc += aw[u].y * vv[4 * u + 1];
            acc += aw[u].z * vv[4 * u + 2];
            acc += aw[u].w * vv[4 * u + 3];
        }
    }
    for (int k = k0; k < n; ++k) acc += al[k] * vrows[k][tid];
    // Q8_0 of the 32-channel block this lane is in
    float amax = fabsf(acc);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    const float d = amax / 127.f;
    const float id = d != 0.f ? 1.f / d : 0.f;
    int8_t* qs = static_cast<int8_t*>(a.act_out);
    float* qd = reinterpret_cast<float*>(qs + int64_t(a.Hq) * DH);
    const int64_t idx = int64_t(h) * DH + c0 + tid;
    qs[idx] = int8_t(int(roundf(acc * id)));
    if ((tid & 31) == 0) qd[idx >> 5] = half_bits_to_f32(fp32_to_fp16_ref(d));
}

constexpr size_t kPrepScoresMaxShared = 160 * 1024;  // shared memory per CU

void launch_gemma_attention(const GemmaAttnArgs& a, hipStream_t s) {
    const unsigned prep = unsigned(a.Hq + (a.append ? 2 * a.Hkv : 0));
    const int64_t vis = a.window > 0 ? std::min<int64_t>(a.window, a.slots) : a.max_ctx;
    const unsigned tiles = unsigned(std::min<int64_t>(128, (vis + kGsTile - 1) / kGsTile));
    const int group = a.Hq / a.Hkv;
    if (a.Dh == 256) {
        if (prep_scores_shared<256>(group) <= kPrepScoresMaxShared) {
            hipLaunchKernelGGL(gemma_prep_scores_kernel<256>, dim3(unsigned(a.Hkv), tiles), dim3(kPsThreads), prep_scores_shared<256>(group), s, a);
        } else {
            hipLaunchKernelGGL(gemma_attn_prep_kernel<256>, dim3(prep), dim3(256), 0, s, a);
            hipLaunchKernelGGL(gemma_scores_kernel<256>, dim3(unsigned(a.Hkv), tiles), dim3(256), size_t(kGsTile * 257 + group * 256) * 4, s, a);
        }
        if (a.window > 0 && a.window <= kShortMax)
            hipLaunchKernelGGL(gemma_softmax_pv_short_kernel<256>, dim3(unsigned(a.Hq * (256 / 64))), dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL(gemma_softmax_pv_kernel<256>, dim3(unsigned(a.Hq * (256 / 64))), dim3(256), 0, s, a);
    } else {
        if (prep_scores_shared<512>(group) <= kPrepScoresMaxShared) {
            hipLaunchKernelGGL(gemma_prep_scores_kernel<512>, dim3(unsigned(a.Hkv), tiles), dim3(kPsThreads), prep_scores_shared<512>(group), s, a);
        } else {
            hipLaunchKernelGGL(gemma_attn_prep_kernel<512>, dim3(prep), dim3(512), 0, s, a);
            hipLaunchKernelGGL(gemma_scores_kernel<512>, dim3(unsigned(a.Hkv), tiles), dim3(256), size_t(kGsTile * 513 + group * 512) * 4, s, a);
        }
        hipLaunchKernelGGL(gemma_softmax_pv_kernel<512>, dim3(unsigned(a.Hq * (512 / 64))), dim3(256), 0, s, a);
    }
}

// ---- the end of a sub-block ------------------------------------------------------------
// out = (RMSNorm(a) * gamma + res) * scale, then the Q8_0 act of next_gamma ?
// RMSNorm(out) * next_gamma : out. The forms of GemmaE4BLayer::forward
// (nm/src/gemma4.hpp:258-272): H = X + post_attn_norm(attn) and
// H = H + post_ffn_norm(ffn) (scale 1: an exact identity), then the PLE
// residual branch + hidden (:102-104) times layer_output_scale; the next
// norm is the following block's pre-norm (or the final norm). 512 lanes, 8
// values each (D <= 4096, D % 32 == 0).
constexpr int kPostThreads = 512;

__global__ __launch_bounds__(kPostThreads) void gemma_post_norm_kernel(const float* __restrict__ a, const float* __restrict__ gamma, const float* __restrict__ res, float scale,
                                                                       float eps, float* __restrict__ out, const float* __restrict__ next_gamma, int8_t* __restrict__ qs,
                                                                       float* __restrict__ qd, int D) {
    constexpr int PT = seqsum::kMaxN / kPostThreads;  // 8
    __shared__ seqsum::Shared sm;
    __shared__ __align__(16) float sq[seqsum::kMaxN];
    const int tid = threadIdx.x, i0 = tid * PT;
    const bool on = i0 < D;
    // every input read at entry (none depends on the sums): the weights and the
    // residual arrive while the first sum runs
    float v[PT], s2[PT], gm[PT], rs[PT], ng[PT];
    auto load8 = [&](const float* p, float (&dst)[PT]) {
        const float4 x0 = reinterpret_cast<const float4*>(p + i0)[0];
        const float4 x1 = reinterpret_cast<const float4*>(p + i0)[1];
        dst[0] = x0.x, dst[1] = x0.y, dst[2] = x0.z, dst[3] = x0.w, dst[4] = x1.x, dst[5] = x1.y, dst[6] = x1.z, dst[7] = x1.w;
    };
    if (on) {
        load8(a, v);
        load8(gamma, gm);
        load8(res, rs);
        if (next_gamma) load8(next_gamma, ng);
    } else {
#pragma unroll
        for (int k = 0; k < PT; ++k) v[k] = 0.f;
    }
#pragma unroll
    for (int k = 0; k < PT; ++k) s2[k] = v[k] * v[k];
    const float s = seqsum::sum_nonneg_regs<kPostThreads>(s2, sq, D, sm);
    const float inv = 1.f / sqrtf(s / float(D) + eps);
    float o[PT];
    if (on) {
#pragma unroll
        for (int k = 0; k < PT; ++k) o[k] = (gm[k] * v[k] * inv + rs[k]) * scale;
        reinterpret_cast<float4*>(out + i0)[0] = make_float4(o[0], o[1], o[2], o[3]);
        reinterpret_cast<float4*>(out + i0)[1] = make_float4(o[4], o[5], o[6], o[7]);
    } else {
#pragma unroll
        for (int k = 0; k < PT; ++k) o[k] = 0.f;
    }
    if (next_gamma) {
#pragma unroll
        for (int k = 0; k < PT; ++k) s2[k] = o[k] * o[k];
        __syncthreads();  // the first sum's readers of sq and sm are done
        const float s_2 = seqsum::sum_nonneg_regs<kPostThreads>(s2, sq, D, sm);
        const float inv2 = 1.f / sqrtf(s_2 / float(D) + eps);
        if (on) {
#pragma unroll
            for (int k = 0; k < PT; ++k) o[k] = ng[k] * o[k] * inv2;
        }
    }
    if (!on) return;
    uint16_t dh;
    reinterpret_cast<int2*>(qs)[tid] = quantize8_in_quad(o, &dh);
    if ((tid & 3) == 0) qd[tid >> 2] = half_bits_to_f32(dh);
}

void launch_gemma_post_norm(const float* a, const float* gamma, const float* res, float scale, float eps, float* out, const float* next_gamma, void* act, int64_t D,
                            hipStream_t s) {
    int8_t* qs = static_cast<int8_t*>(act);
    hipLaunchKernelGGL(gemma_post_norm_kernel, dim3(1), dim3(kPostThreads), 0, s, a, gamma, res, scale, eps, out, next_gamma, qs, reinterpret_cast<float*>(qs + D), int(D));
}

// ---- GELU-gated products --------------------------------------------------------------
// act = Q8_0 of gelu(gate[i]) * mul[i]: the GELU-gated MLP's down input
// (GatedMLP, components.hpp:294-299: g = gelu(gate(x)); g *= up(x)) and the
// PLE branch input (gemma4.hpp:100-101: hadamard(gelu(gate(h)), ple)).
// A lane per value (tanh's chain is long: every lane runs one); the 32 lanes
// of a Q8_0 block share its amax (N % 32 == 0).
__global__ __launch_bounds__(256) void gemma_gelu_mul_quant_kernel(const float* __restrict__ gate, const float* __restrict__ mul, int8_t* __restrict__ qs,
                                                                   float* __restrict__ qd, int64_t N) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= N) return;  // whole 32-lane blocks
    const float v = gelu_tanh_f32(gate[i]) * mul[i];
    float amax = fabsf(v);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    const float d = amax / 127.f;
    const float id = d != 0.f ? 1.f / d : 0.f;
    qs[i] = int8_t(int(roundf(v * id)));
    if ((i & 31) == 0) qd[i >> 5] = half_bits_to_f32(fp32_to_fp16_ref(d));
}

void launch_gemma_gelu_mul_quant(const float* gate, const float* mul, void* act, int64_t N, hipStream_t s) {
    int8_t* qs = static_cast<int8_t*>(act);
    hipLaunchKernelGGL(gemma_gelu_mul_quant_kernel, dim3(unsigned((N + 255) / 256)), dim3(256), 0, s, gate, mul, qs, reinterpret_cast<float*>(qs + N), N);
}

// ---- the logit soft-cap ---------------------------------------------------------------
// cap * tanh(v / cap) (gemma_softcap, nm/src/gemma4.hpp:79)
__global__ __launch_bounds__(256) void gemma_softcap_kernel(float* __restrict__ logits, int64_t n, float cap) {
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) logits[i] = cap * tanhf_glibc(logits[i] / cap);
}

void launch_gemma_softcap(float* logits, int64_t n, float cap, hipStream_t s) {
    hipLaunchKernelGGL(gemma_softcap_kernel, dim3(unsigned(std::min<int64_t>(1024, (n + 255) / 256))), dim3(256), 0, s, logits, n, cap);
}

// host-callable evaluation of the device GELU and soft-cap (tests)
__global__ void gemma_math_eval_kernel(const float* __restrict__ x, float* __restrict__ out, int64_t n, float cap) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    out[2 * i] = gelu_tanh_f32(x[i]);
    out[2 * i + 1] = cap * tanhf_glibc(x[i] / cap);
}

void launch_gemma_math_eval(const float* x, float* out, int64_t n, float cap, hipStream_t s) {
    hipLaunchKernelGGL(gemma_math_eval_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, s, x, out, n, cap);
}

}  // namespace hero
