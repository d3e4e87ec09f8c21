// attn.hip -- gated GQA attention over an fp32 K/V cache: decode, one token
// per sequence, and prefill chunks, many tokens of one sequence
// (nm/src/qwen35.hpp:343-395; with window > 0 the sliding-window visibility of
// nm/src/attention.hpp:159-176); and over a paged fp16 / Q8_0 cache (split-K,
// at the end of the file). Heads of 128 channels, and of 256 (the reference's
// Qwen 3.5 4B / 9B) through the kernels templated on the head width.
//
// Four stages, each keeping the reference's fp32 operation order (the fused
// and tiled forms further down -- score tiles with the prep folded in, the
// softmax and weighted sum in one kernel, the register softmax, the row-block
// weighted sum of prefill -- compute the same values):
//  1. prep    one workgroup per (sequence, query head), a lane per channel:
//             split of the packed [q | gate] pair, q RMSNorm + RoPE; the first
//             query head of each K/V group also normalises and rotates k and
//             appends k and v to the cache.
//  2. scores  a lane per visible key and KV head: s_j = scale * dot(q, k_j)
//             for each query head of the group, every dot a sequential
//             Dh-term sum (nm/src/core.hpp:496-500). K is cached channel-major
//             per head, [Dh][max_ctx], so lanes reading consecutive keys read
//             consecutive addresses.
//  3. softmax one workgroup per (sequence, query head): max, e_j = exp(s_j -
//             max), the softmax total as the sequential sum over j
//             (components.hpp:132-141) computed exactly in parallel
//             (hero/seqsum.hpp), alpha_j = e_j / total.
//  4. pv      a workgroup per (sequence, query head, 32 channels): the
//             products alpha_j * v_j[c] are formed in parallel, then a lane per
//             channel adds them in row order (core.hpp:206-208), multiplies by
//             sigmoid(gate) (qwen35.hpp:390-393) and quantizes the output (one
//             Q8_0 block).
// RoPE reads a host-built cos/sin table made with the reference's float
// expressions (attention.hpp:76-91).
// With shared_cache set, the B rows are consecutive tokens of one sequence
// (prefill): prep appends all their keys and values to the one cache before
// the scores kernel runs, and row b attends to positions <= positions[b] only,
// as the reference appends the whole batch and then reduces each row over its
// visible rows (qwen35.hpp:363, 386-387).
#include "hero/device.hpp"
#include "hero/kernels.hpp"
#include "hero/seqsum.hpp"

namespace hero {

constexpr int kAttnDim = 128;
constexpr int kScoreTiles = 128;  // most score tiles of 256 keys per head

// the cache row b reads and appends to
__device__ __forceinline__ int64_t cache_of(const AttnDecodeArgs& a, int b) { return a.shared_cache ? 0 : b; }

// ---- 1. prep ----------------------------------------------------------------------
// RMSNorm over one head of DH channels held one value per lane (sequential
// DH-term sum of squares by lane 0), then RoPE on the NEOX planes (i, i + DH/2).
template <int DH>
__device__ __forceinline__ float norm_rope_head(float x, const float* gamma, float eps, const float* cs, float* buf, float* scal, int j) {
    buf[j] = x * x;
    __syncthreads();
    if (j == 0) {
        float ss = 0.f;
        const float4* b4 = reinterpret_cast<const float4*>(buf);
#pragma unroll
        for (int i = 0; i < DH / 4; ++i) {
            const float4 v = b4[i];
            ss += v.x;
            ss += v.y;
            ss += v.z;
            ss += v.w;
        }
        scal[0] = 1.f / sqrtf(ss / float(DH) + eps);
    }
    __syncthreads();
    const float n = gamma[j] * x * scal[0];
    buf[j] = n;
    __syncthreads();
    const int half = DH / 2;
    const int i = j < half ? j : j - half;
    const float c = cs[2 * i], s = cs[2 * i + 1];
    const float xx = buf[i], yy = buf[i + half];
    const float r = j < half ? xx * c - yy * s : yy * c + xx * s;
    __syncthreads();
    return r;
}

template <int DH>
__global__ __launch_bounds__(DH) void attn_prep_kernel(AttnDecodeArgs a) {
    const int j = threadIdx.x, h = blockIdx.x, b = blockIdx.y;
    const int group = a.Hq / a.Hkv;
    const int g = h / group;  // grouped K/V heads (nm/src/qwen35.hpp:369)
    const int pos = a.positions[b];
    if (pos < 0 || pos >= a.max_ctx) return;  // the host keeps positions in range
    const float* P = a.proj + int64_t(b) * a.proj_stride;
    const float* cs = a.rope_cs + int64_t(pos) * DH;  // [Dh/2][2]
    __shared__ __align__(16) float buf[DH];
    __shared__ float scal[2];
    const float q = norm_rope_head<DH>(P[int64_t(h) * 2 * DH + j], a.q_gamma, a.eps, cs, buf, scal, j);
    a.q_rot[(int64_t(b) * a.Hq + h) * DH + j] = q;
    if (h % group == 0) {
        const float k = norm_rope_head<DH>(P[a.k_off + int64_t(g) * DH + j], a.k_gamma, a.eps, cs, buf, scal, j);
        const float v = P[a.v_off + int64_t(g) * DH + j];
        const int64_t cb = cache_of(a, b);
        const int64_t kv = cb * a.Hkv + g;
        a.k_cache[(kv * DH + j) * a.max_ctx + pos] = k;  // [B][Hkv][Dh][max_ctx]
        a.v_cache[(cb * a.max_ctx + pos) * (int64_t(a.Hkv) * DH) + int64_t(g) * DH + j] = v;  // [B][max_ctx][Hkv*Dh]
    }
}

__device__ __forceinline__ int visible_first(int pos, int window) { return (window > 0 && pos + 1 > window) ? pos + 1 - window : 0; }

// ---- 2. scores -------------------------------------------------------------------------
// A lane per visible key and KV head: it reads the key's DH cached channels
// once and forms the dot products of every query head of the group (up to
// kScoreHeads at a time), each the sequential DH-term sum, side by side. The
// grid covers max_ctx in tiles of 256 keys (at most kScoreTiles tiles; lanes
// loop when the context is longer).
constexpr int kScoreHeads = 4;

template <int DH>
__global__ __launch_bounds__(256) void attn_scores_kernel(AttnDecodeArgs a) {
    const int tile0 = blockIdx.y, b = blockIdx.z;
    const int group = a.Hq / a.Hkv, nchunk = (group + kScoreHeads - 1) / kScoreHeads;
    const int g = int(blockIdx.x) / nchunk, hq0 = g * group + (int(blockIdx.x) % nchunk) * kScoreHeads;
    const int nh = min(kScoreHeads, g * group + group - hq0);
    const int pos = a.positions[b];
    if (pos < 0 || pos >= a.max_ctx) return;
    const int first = visible_first(pos, a.window);
    const int n = pos + 1 - first;
    if (tile0 * 256 >= n) return;
    __shared__ float q[kScoreHeads][DH];
    for (int i = threadIdx.x; i < kScoreHeads * DH; i += 256) {
        const int hh = min(i / DH, nh - 1);
        q[i / DH][i % DH] = a.q_rot[(int64_t(b) * a.Hq + hq0 + hh) * DH + i % DH];
    }
    __syncthreads();
    const float* kh = a.k_cache + (cache_of(a, b) * a.Hkv + g) * DH * a.max_ctx;
    float* sc = a.scores + (int64_t(b) * a.Hq + hq0) * a.max_ctx;
    const int step = int(gridDim.y) * 256;
    for (int t = tile0 * 256 + int(threadIdx.x); t < n; t += step) {
        const float* kj = kh + first + t;
        float dot[kScoreHeads] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 16
        for (int c = 0; c < DH; ++c) {
            const float k = kj[int64_t(c) * a.max_ctx];
#pragma unroll
            for (int hh = 0; hh < kScoreHeads; ++hh) dot[hh] += q[hh][c] * k;
        }
#pragma unroll
        for (int hh = 0; hh < kScoreHeads; ++hh)
            if (hh < nh) sc[int64_t(hh) * a.max_ctx + t] = a.score_scale * dot[hh];
    }
}

// The decode form for one or two sequences, with the prep step folded in:
// 64-key tiles staged in shared memory, a workgroup per (KV group chunk of up
// to four query heads, tile, sequence). It copies the tile's keys (128
// channels x 64 keys, channel-major as cached) with global_load_lds; while
// they land, wave w forms query head w of the chunk (RMSNorm + RoPE, a lane per
// plane (i, i + 64)) and the workgroup whose tile holds the new position forms
// its key the same way, patches it into the tile and appends k and v to the
// cache (the prep kernel's work). Then wave w forms the dots of head w, a lane
// per key, the query held in registers. Tiles start at a multiple of 4 keys
// (the 16-byte copies need aligned keys; the host runs this form for
// max_ctx % 4 == 0); keys before the window's first are formed but not stored.
constexpr int kScTileKeys = 64;
constexpr int kScTiles = 1024;  // most tiles per head; workgroups loop beyond

// RMSNorm (sequential 128-term sum of squares by lane 0) and RoPE of one head
// held by a wave as x0 = channel lane, x1 = channel lane + 64 -- the
// operations of norm_rope_head; buf: 128 floats of the wave's own
__device__ __forceinline__ void norm_rope_pair(float& x0, float& x1, const float* gamma, float eps, const float* cs, float* buf, int lane) {
    buf[lane] = x0 * x0;
    buf[lane + 64] = x1 * x1;
    float scal = 0.f;
    if (lane == 0) {
        float ss = 0.f;
        const float4* b4 = reinterpret_cast<const float4*>(buf);
#pragma unroll
        for (int i = 0; i < kAttnDim / 4; ++i) {
            const float4 v = b4[i];
            ss += v.x;
            ss += v.y;
            ss += v.z;
            ss += v.w;
        }
        scal = 1.f / sqrtf(ss / float(kAttnDim) + eps);
    }
    scal = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(scal)));  // lane 0's value (it is active here)
    const float n0 = gamma[lane] * x0 * scal, n1 = gamma[lane + 64] * x1 * scal;
    const float c = cs[2 * lane], s = cs[2 * lane + 1];
    x0 = n0 * c - n1 * s;
    x1 = n1 * c + n0 * s;
}

__global__ __launch_bounds__(256) void attn_scores_tile_kernel(AttnDecodeArgs a) {
    __shared__ __align__(16) float kt[kAttnDim * kScTileKeys];  // [channel][key]
    __shared__ __align__(16) float qb[kScoreHeads][kAttnDim];    // per wave: squares, then its rotated query
    const int b = blockIdx.z;
    const int group = a.Hq / a.Hkv, nchunk = (group + kScoreHeads - 1) / kScoreHeads;
    const int g = int(blockIdx.x) / nchunk, hq0 = g * group + (int(blockIdx.x) % nchunk) * kScoreHeads;
    const int nh = min(kScoreHeads, g * group + group - hq0);
    const int pos = a.positions[b];
    if (pos < 0 || pos >= a.max_ctx) return;
    const int first = visible_first(pos, a.window);
    const int n = pos + 1 - first;
    const int base0 = first & ~3;  // keys from base0 on, in tiles of 64
    const int span = pos + 1 - base0;
    if (int(blockIdx.y) * kScTileKeys >= span) return;
    const int tid = int(threadIdx.x), wave = tid / 64, lane = tid % 64;
    const int hh = __builtin_amdgcn_readfirstlane(min(wave, nh - 1));  // waves past nh repeat the last head (not stored)
    const int64_t kv = cache_of(a, b) * a.Hkv + g;
    const float* kh = a.k_cache + kv * kAttnDim * a.max_ctx;
    float* sc = a.scores + (int64_t(b) * a.Hq + hq0 + hh) * a.max_ctx;
    const float* P = a.proj + int64_t(b) * a.proj_stride;
    const float* cs = a.rope_cs + int64_t(pos) * kAttnDim;  // [Dh/2][2]
    const int pos_tile = (pos - base0) / kScTileKeys;
    const bool has_pos = pos_tile % int(gridDim.y) == int(blockIdx.y);

    // 2048 16-byte chunks: chunk p = channel p / 16, keys key0 + 4 (p % 16) ..;
    // chunks past the cache's end read its last chunk (never stored)
    auto issue_tile = [&](int key0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int p = 256 * j + tid, c = p / 16;
            const int k4 = min(key0 + 4 * (p % 16), int(a.max_ctx) - 4);
            lds_dma_b128(kh + int64_t(c) * a.max_ctx + k4, lds_offset(kt + 4 * 256 * j + 4 * 64 * wave));
        }
    };
    int t0 = int(blockIdx.y) * kScTileKeys;
    issue_tile(base0 + t0);

    // ---- the prep step (nm/src/qwen35.hpp:343-362): the wave's query ----
    float q0 = P[int64_t(hq0 + hh) * 2 * kAttnDim + lane], q1 = P[int64_t(hq0 + hh) * 2 * kAttnDim + 64 + lane];
    norm_rope_pair(q0, q1, a.q_gamma, a.eps, cs, qb[wave], lane);
    qb[wave][lane] = q0;
    qb[wave][lane + 64] = q1;
    // the new key's inputs (the workgroups whose tiles hold it; wave 0 forms it)
    float k0 = 0.f, k1 = 0.f;
    if (has_pos && wave == 0) {
        k0 = P[a.k_off + int64_t(g) * kAttnDim + lane];
        k1 = P[a.k_off + int64_t(g) * kAttnDim + 64 + lane];
    }
    // the query in vector registers, the same in every lane, for all of the
    // wave's tiles (a lane-varying zero keeps it out of scalar registers)
    float qv[kAttnDim];
    {
        const uint32_t z0 = lane_zero();
#pragma unroll
        for (int c = 0; c < kAttnDim; c += 4) {
            const float4 v = reinterpret_cast<const float4*>(qb[wave])[c / 4 + z0];
            qv[c] = v.x, qv[c + 1] = v.y, qv[c + 2] = v.z, qv[c + 3] = v.w;
        }
    }
    if (has_pos && wave == 0) {  // qb[0] is free again: wave 0's query is in its registers
        norm_rope_pair(k0, k1, a.k_gamma, a.eps, cs, qb[0], lane);
        if (int(blockIdx.x) % nchunk == 0) {  // the cache, once per K/V head
            a.k_cache[(kv * kAttnDim + lane) * a.max_ctx + pos] = k0;  // [B][Hkv][Dh][max_ctx]
            a.k_cache[(kv * kAttnDim + 64 + lane) * a.max_ctx + pos] = k1;
            float* vrow = a.v_cache + (cache_of(a, b) * a.max_ctx + pos) * (int64_t(a.Hkv) * kAttnDim) + int64_t(g) * kAttnDim;
            vrow[lane] = P[a.v_off + int64_t(g) * kAttnDim + lane];  // [B][max_ctx][Hkv*Dh]
            vrow[64 + lane] = P[a.v_off + int64_t(g) * kAttnDim + 64 + lane];
        }
    }

    for (; t0 < span; t0 += int(gridDim.y) * kScTileKeys) {
        const int key0 = base0 + t0;
        if (t0 != int(blockIdx.y) * kScTileKeys) issue_tile(key0);
        wait_vmcnt<0>();
        __syncthreads();
        if (has_pos && (pos - base0) / kScTileKeys * kScTileKeys == t0) {  // the new key into its column
            if (wave == 0) {
                kt[lane * kScTileKeys + (pos - key0)] = k0;
                kt[(lane + 64) * kScTileKeys + (pos - key0)] = k1;
            }
            __syncthreads();
        }
        // s_j = scale * dot(q, k_j), the dot a sequential 128-term sum (core.hpp:496-500)
        float dot = 0.f;
#pragma unroll
        for (int c = 0; c < kAttnDim; ++c) dot += qv[c] * kt[c * kScTileKeys + lane];
        const int t = key0 + lane - first;  // index among the visible keys
        if (wave < nh && t >= 0 && t < n) sc[t] = a.score_scale * dot;
        __syncthreads();  // the tile is read before the next one lands
    }
}

// The same for heads of 256 channels (the reference's Qwen 3.5 4B / 9B
// attention): the [channel][key] tile is 64 KB, a wave's query (four values a
// lane: channels lane + 64 m, so both of a lane's RoPE planes (i, i + 128) are
// its own) stays in shared memory and is read four channels at a time, the
// same for every lane.
constexpr int kWideDim = 256;

__global__ __launch_bounds__(256) void attn_scores_tile_wide_kernel(AttnDecodeArgs a) {
    __shared__ __align__(16) float kt[kWideDim * kScTileKeys];  // [channel][key]
    __shared__ __align__(16) float qb[kScoreHeads][kWideDim];    // per wave: squares, then its rotated query
    __shared__ __align__(16) float kb[kWideDim];                 // the new key (workgroups holding its position)
    const int b = blockIdx.z;
    const int group = a.Hq / a.Hkv, nchunk = (group + kScoreHeads - 1) / kScoreHeads;
    const int g = int(blockIdx.x) / nchunk, hq0 = g * group + (int(blockIdx.x) % nchunk) * kScoreHeads;
    const int nh = min(kScoreHeads, g * group + group - hq0);
    const int pos = a.positions[b];
    if (pos < 0 || pos >= a.max_ctx) return;
    const int first = visible_first(pos, a.window);
    const int n = pos + 1 - first;
    const int base0 = first & ~3;  // keys from base0 on, in tiles of 64
    const int span = pos + 1 - base0;
    if (int(blockIdx.y) * kScTileKeys >= span) return;
    const int tid = int(threadIdx.x), wave = tid / 64, lane = tid % 64;
    const int hh = __builtin_amdgcn_readfirstlane(min(wave, nh - 1));  // waves past nh repeat the last head (not stored)
    const int64_t kv = cache_of(a, b) * a.Hkv + g;
    const float* kh = a.k_cache + kv * kWideDim * a.max_ctx;
    float* sc = a.scores + (int64_t(b) * a.Hq + hq0 + hh) * a.max_ctx;
    const float* P = a.proj + int64_t(b) * a.proj_stride;
    const float* cs = a.rope_cs + int64_t(pos) * kWideDim;  // [Dh/2][2]
    const int pos_tile = (pos - base0) / kScTileKeys;
    const bool has_pos = pos_tile % int(gridDim.y) == int(blockIdx.y);

    // 4096 16-byte chunks: chunk p = channel p / 16, keys key0 + 4 (p % 16) ..;
    // chunks past the cache's end read its last chunk (never stored)
    auto issue_tile = [&](int key0) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int p = 256 * j + tid, c = p / 16;
            const int k4 = min(key0 + 4 * (p % 16), int(a.max_ctx) - 4);
            lds_dma_b128(kh + int64_t(c) * a.max_ctx + k4, lds_offset(kt + 4 * 256 * j + 4 * 64 * wave));
        }
    };
    int t0 = int(blockIdx.y) * kScTileKeys;
    issue_tile(base0 + t0);

    // RMSNorm (the sequential 256-term sum of squares by lane 0) and RoPE of
    // one head held as x[m] = channel lane + 64 m: norm_rope_head's operations
    auto norm_rope4 = [&](float (&x)[4], const float* gamma, float* buf) {
#pragma unroll
        for (int m = 0; m < 4; ++m) buf[lane + 64 * m] = x[m] * x[m];
        float scal = 0.f;
        if (lane == 0) {
            float ss = 0.f;
            const float4* b4 = reinterpret_cast<const float4*>(buf);
#pragma unroll
            for (int i = 0; i < kWideDim / 4; ++i) {
                const float4 v = b4[i];
                ss += v.x;
                ss += v.y;
                ss += v.z;
                ss += v.w;
            }
            scal = 1.f / sqrtf(ss / float(kWideDim) + a.eps);
        }
        scal = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(scal)));  // lane 0's value
        float nn[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) nn[m] = gamma[lane + 64 * m] * x[m] * scal;
#pragma unroll
        for (int m = 0; m < 2; ++m) {  // planes (i, i + 128), i = lane + 64 m
            const int i = lane + 64 * m;
            const float c = cs[2 * i], sn = cs[2 * i + 1];
            x[m] = nn[m] * c - nn[m + 2] * sn;
            x[m + 2] = nn[m + 2] * c + nn[m] * sn;
        }
    };

    // ---- the prep step (nm/src/qwen35.hpp:343-362): the wave's query ----
    {
        float qx[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) qx[m] = P[int64_t(hq0 + hh) * 2 * kWideDim + lane + 64 * m];
        norm_rope4(qx, a.q_gamma, qb[wave]);
#pragma unroll
        for (int m = 0; m < 4; ++m) qb[wave][lane + 64 * m] = qx[m];
    }
    if (has_pos && wave == 0) {  // the new key (after the query: qb[0] then holds the query, kb the squares)
        float kx[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) kx[m] = P[a.k_off + int64_t(g) * kWideDim + lane + 64 * m];
        norm_rope4(kx, a.k_gamma, kb);
#pragma unroll
        for (int m = 0; m < 4; ++m) kb[lane + 64 * m] = kx[m];
        if (int(blockIdx.x) % nchunk == 0) {  // the cache, once per K/V head
            float* vrow = a.v_cache + (cache_of(a, b) * a.max_ctx + pos) * (int64_t(a.Hkv) * kWideDim) + int64_t(g) * kWideDim;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                a.k_cache[(kv * kWideDim + lane + 64 * m) * a.max_ctx + pos] = kx[m];  // [B][Hkv][Dh][max_ctx]
                vrow[lane + 64 * m] = P[a.v_off + int64_t(g) * kWideDim + lane + 64 * m];  // [B][max_ctx][Hkv*Dh]
            }
        }
    }

    const float4* q4 = reinterpret_cast<const float4*>(qb[wave]);
    for (; t0 < span; t0 += int(gridDim.y) * kScTileKeys) {
        const int key0 = base0 + t0;
        if (t0 != int(blockIdx.y) * kScTileKeys) issue_tile(key0);
        wait_vmcnt<0>();
        __syncthreads();
        if (has_pos && (pos - base0) / kScTileKeys * kScTileKeys == t0) {  // the new key into its column
            kt[tid * kScTileKeys + (pos - key0)] = kb[tid];
            __syncthreads();
        }
        // s_j = scale * dot(q, k_j), the dot a sequential 256-term sum (core.hpp:496-500)
        float dot = 0.f;
#pragma unroll 16
        for (int c4 = 0; c4 < kWideDim / 4; ++c4) {
            const float4 qv = q4[c4];
            dot += qv.x * kt[(4 * c4) * kScTileKeys + lane];
            dot += qv.y * kt[(4 * c4 + 1) * kScTileKeys + lane];
            dot += qv.z * kt[(4 * c4 + 2) * kScTileKeys + lane];
            dot += qv.w * kt[(4 * c4 + 3) * kScTileKeys + lane];
        }
        const int t = key0 + lane - first;  // index among the visible keys
        if (wave < nh && t >= 0 && t < n) sc[t] = a.score_scale * dot;
        __syncthreads();  // the tile is read before the next one lands
    }
}

// ---- 3. softmax ------------------------------------------------------------------------------
// max over the visible scores (order free), e_j = exp(s_j - max), the total as
// the sequential sum over j computed exactly in parallel, alpha_j = e_j / total
// written back over the scores.
// e_j = exp(s_j - max) written over the scores and the total of n terms,
// chunk by chunk, each chunk starting with the running total as its first
// term (fl(0 + e) == e, so the first chunk matches the loop from s = 0); then
// alpha_j = e_j / total. NT lanes; chunk: kMaxN floats of shared memory.
template <int NT>
__device__ inline void softmax_chunked(float* sc, int n, float mx, seqsum::Shared& sm, float* chunk) {
    const int tid = int(threadIdx.x);
    float total = 0.f;
    for (int base = 0; base < n; base += seqsum::kMaxN - 1) {
        const int len = min(n - base, seqsum::kMaxN - 1);
        for (int t = tid; t < len; t += NT) {
            const float e = exp_f32(sc[base + t] - mx);
            sc[base + t] = e;
            chunk[t + 1] = e;
        }
        if (tid == 0) chunk[0] = total;
        __syncthreads();
        total = seqsum::sum_nonneg<NT>(chunk, len + 1, sm);  // every wave gets the total
    }
    for (int t = tid; t < n; t += NT) sc[t] = sc[t] / total;
}

__global__ __launch_bounds__(seqsum::kThreads) void attn_softmax_kernel(AttnDecodeArgs a) {
    const int tid = threadIdx.x, h = blockIdx.x, b = blockIdx.y;
    const int pos = a.positions[b];
    if (pos < 0 || pos >= a.max_ctx) return;
    const int first = visible_first(pos, a.window);
    const int n = pos + 1 - first;
    float* sc = a.scores + (int64_t(b) * a.Hq + h) * a.max_ctx;
    __shared__ seqsum::Shared sm;
    __shared__ __align__(16) float chunk[seqsum::kMaxN];
    __shared__ float red[seqsum::kWaves];

    float mx = -INFINITY;
    for (int t = tid; t < n; t += seqsum::kThreads) mx = fmaxf(mx, sc[t]);
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = red[0];
    for (int w = 1; w < seqsum::kWaves; ++w) mx = fmaxf(mx, red[w]);
    softmax_chunked<seqsum::kThreads>(sc, n, mx, sm, chunk);
}

// ---- 4. weighted sum of values, gate, quantize -----------------------------------------------
// out[c] = sum_j alpha_j * v_j[c] with the rows in order (core.hpp:206-208).
// A workgroup per (sequence, query head, 32 channels = one Q8_0 block of the
// output), in tiles of kPvRows rows, with three roles:
//  * waves 3..4 stream the V rows (32 each) and the alpha values (wave 4) of
//    the tiles straight into a ring of R shared-memory slots (global_load_lds:
//    the same loads per lane every tile, so each wave waits for exactly its
//    oldest tile); R - 2 tiles stay in flight;
//  * waves 1..2 form the products alpha_j * v_j[c] (the reference's product,
//    one rounding) and store them transposed, [channel][row], into one of two
//    product buffers;
//  * lanes 0..31 of wave 0 each hold one channel's sum and only add, four
//    products per 16-byte read, which is the dependent chain the reference's
//    loop is.
// One barrier per tile: after it the loaders refill a freed slot, the
// producers fill the next tile's products and the chain adds the current
// tile's.
constexpr int kPvCh = 32;                                   // channels per workgroup
constexpr int kPvRows = 64;                                 // rows per tile
constexpr int kPvStride = kPvRows + 4;                      // product row stride (conflict-free 16-byte reads)
constexpr int kPvThreads = 320;                             // chain wave, two producer waves, two loader waves
constexpr int kPvVTile = kPvRows * kPvCh;                   // floats of V per tile
constexpr int kPvVLoads = kPvVTile / 4 / 128;               // 16-byte V loads per loader lane per tile: 4
static_assert(kPvVLoads == 4 && kPvRows == 64 && kPvCh * kPvRows / 4 / 4 == 128, "tile geometry");
constexpr size_t pv_shared_bytes(int R) { return (size_t(R) * (kPvVTile + kPvRows) + size_t(2) * kPvCh * kPvStride) * 4; }

template <int R>
__global__ __launch_bounds__(kPvThreads) void attn_pv_kernel(AttnDecodeArgs a) {
    static_assert(R >= 4 && (R - 2) * (kPvVLoads + 1) <= 63, "the oldest tile's wait count fits vmcnt");
    extern __shared__ __align__(16) float pv_smem[];  // [R][V tile] [R][alpha tile] [2][kPvCh][kPvStride]
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64, b = blockIdx.y;
    constexpr int parts = kAttnDim / kPvCh;
    int h, part;
    head_part_of(int(blockIdx.x), a.Hq, a.Hkv, parts, h, part);
    const int g = h / (a.Hq / a.Hkv);
    const int pos = a.positions[b];
    if (pos < 0 || pos >= a.max_ctx) return;
    const int first = visible_first(pos, a.window);
    const int n = pos + 1 - first;
    const float* alpha = a.scores + (int64_t(b) * a.Hq + h) * a.max_ctx;
    const int64_t kw = int64_t(a.Hkv) * kAttnDim;
    const float* vb = a.v_cache + (cache_of(a, b) * a.max_ctx + first) * kw + int64_t(g) * kAttnDim + part * kPvCh;
    const int ntiles = (n + kPvRows - 1) / kPvRows;
    float* vring = pv_smem;
    float* aring = vring + R * kPvVTile;
    float* prod = aring + R * kPvRows;
    constexpr int pstride = kPvCh * kPvStride;
    const bool loader = wave >= 3;
    const int half = wave - 3;  // loader: V rows 32 half .. 32 half + 31

    // loaders: V rows (rows past n read row n - 1, whose products the chain
    // never adds) and, on wave 4, the alpha values of a tile
    auto issue = [&](int tile) {
        const int slot = tile % R;
#pragma unroll
        for (int j = 0; j < kPvVLoads; ++j) {
            const int q = half * 256 + lane + 64 * j;  // 16-byte slot: row q / 8, channels 4 (q % 8) ..
            const int row = min(tile * kPvRows + q / 8, n - 1);
            lds_dma_b128(vb + int64_t(row) * kw + 4 * (q % 8), lds_offset(vring + slot * kPvVTile + 4 * (half * 256 + 64 * j)));
        }
        if (half == 1) lds_dma_b32(alpha + min(tile * kPvRows + lane, n - 1), lds_offset(aring + slot * kPvRows));
    };
    // this loader wave's loads of tile t have landed, given how many tiles it issued after t
    auto wait_tile = [&](bool full) {
        if (full) {
            if (half == 0)
                wait_vmcnt<(R - 3) * kPvVLoads>();
            else
                wait_vmcnt<(R - 3) * (kPvVLoads + 1)>();
        } else {
            wait_vmcnt<0>();
        }
    };
    // producers: channels c4 .. c4 + 3 and rows r4 .. r4 + 3 of a tile
    auto produce = [&](int tile) {
        const int slot = tile % R;
        const int c4 = (lane % 8) * 4, r4 = ((wave - 1) * 8 + lane / 8) * 4;
        const float* vt = vring + slot * kPvVTile;
        float4 v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = reinterpret_cast<const float4*>(vt + (r4 + k) * kPvCh + c4)[0];
        const float4 al = reinterpret_cast<const float4*>(aring + slot * kPvRows + r4)[0];
        float* d = prod + (tile & 1) * pstride + c4 * kPvStride + r4;
        reinterpret_cast<float4*>(d)[0] = make_float4(al.x * v[0].x, al.y * v[1].x, al.z * v[2].x, al.w * v[3].x);
        reinterpret_cast<float4*>(d + kPvStride)[0] = make_float4(al.x * v[0].y, al.y * v[1].y, al.z * v[2].y, al.w * v[3].y);
        reinterpret_cast<float4*>(d + 2 * kPvStride)[0] = make_float4(al.x * v[0].z, al.y * v[1].z, al.z * v[2].z, al.w * v[3].z);
        reinterpret_cast<float4*>(d + 3 * kPvStride)[0] = make_float4(al.x * v[0].w, al.y * v[1].w, al.z * v[2].w, al.w * v[3].w);
    };

    // tiles 0 .. R-2 in flight before the loop; iteration t issues tile
    // t + R - 1 into the slot of tile t - 1, whose products were formed two
    // barriers earlier
    if (loader) {
        for (int t = 0; t + 1 < R; ++t)
            if (t < ntiles) issue(t);
        if (ntiles >= R - 1) {
            if (half == 0)
                wait_vmcnt<(R - 2) * kPvVLoads>();
            else
                wait_vmcnt<(R - 2) * (kPvVLoads + 1)>();
        } else {
            wait_vmcnt<0>();
        }
    }
    __syncthreads();
    if (wave == 1 || wave == 2) produce(0);
    float acc = 0.f;
    for (int tile = 0; tile < ntiles; ++tile) {
        if (loader) wait_tile(tile + R - 1 <= ntiles);  // tile + 1 has landed
        __syncthreads();
        if (loader) {
            if (tile + R - 1 < ntiles) issue(tile + R - 1);
        } else if (wave > 0) {
            if (tile + 1 < ntiles) produce(tile + 1);  // the other buffer: its last reader was the chain before the barrier
        } else if (lane < kPvCh) {
            const float* row = prod + (tile & 1) * pstride + lane * kPvStride;
            const int rows = min(kPvRows, n - tile * kPvRows);
            if (rows == kPvRows) {
                float4 p[kPvRows / 4];
#pragma unroll
                for (int i = 0; i < kPvRows / 4; ++i) p[i] = reinterpret_cast<const float4*>(row)[i];
#pragma unroll
                for (int i = 0; i < kPvRows / 4; ++i) {
                    acc += p[i].x;
                    acc += p[i].y;
                    acc += p[i].z;
                    acc += p[i].w;
                }
            } else {
                for (int r = 0; r < rows; ++r) acc += row[r];
            }
        }
    }

    if (wave == 0 && lane < kPvCh) {
        const int ch = part * kPvCh + lane;
        const float gate = a.proj[int64_t(b) * a.proj_stride + int64_t(h) * 2 * kAttnDim + kAttnDim + ch];
        const float out = acc * sigmoid_f32(gate);
        const int64_t width = int64_t(a.Hq) * kAttnDim;
        const int64_t idx = int64_t(h) * kAttnDim + ch;
        if (a.out_f32) a.out_f32[int64_t(b) * width + idx] = out;
        float amax = fabsf(out);
        for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
        const float d = amax / 127.f;
        const float id = d != 0.f ? 1.f / d : 0.f;
        int8_t* qs = static_cast<int8_t*>(a.act_out);
        float* qd = reinterpret_cast<float*>(qs + int64_t(a.B) * width);
        qs[int64_t(b) * width + idx] = int8_t(int(roundf(out * id)));
        if (lane == 0) qd[(int64_t(b) * width + idx) >> 5] = half_bits_to_f32(fp32_to_fp16_ref(d));
    }
}

// ---- 3+4 fused: softmax and weighted sum ------------------------------------------------------
// For up to 4096 visible keys, one workgroup per (sequence, query head, 32
// channels) runs the softmax of its head itself and then the weighted sum, so
// the V stream starts at once and the weights never leave shared memory.
// Eight waves:
//  * all copy the head's scores into shared memory (global_load_lds), then
//    put the first R tiles of V in flight (one load per tile each);
//  * max; e_j = exp(s_j - max), lane t taking j = t, t + 512, ...; the total
//    as the exact sequential sum (hero/seqsum.hpp, 512 lanes); alpha_j =
//    e_j / total -- the operations of attn_softmax_kernel;
//  * the weighted sum as a pipeline of 64-row tiles with one barrier per tile:
//    the loaders stream V tiles into a ring of R slots (global_load_lds, two
//    16-byte loads per lane per tile, each tile's chunks placed so the
//    producers' reads are conflict-free), waves 1-2 form the products
//    alpha_j * v_j[c] of tile t + 2 from registers read during the previous
//    tile, and wave 0 adds tile t from registers while it reads tile t + 1's
//    products (a 3-slot product ring). Lanes 0-31 of wave 0 run the chains
//    (one per channel, rows in order); wave 3 only keeps the barriers.
constexpr int kSpvThreads = 512;
constexpr int kSpvMaxN = seqsum::kMaxN;        // visible keys at most
constexpr int kSpvR = 13;                      // V ring slots
constexpr int kSpvLoaders = 4;                 // waves 4 .. 7
constexpr int kSpvVLoads = kPvVTile / 4 / 64 / kSpvLoaders;  // 16-byte V loads per loader lane per tile: 2
constexpr int kSpvAhead = 4;                   // the tile the loaders wait for: t + 4 at the end of iteration t
static_assert(kSpvVLoads == 2 && 2 + kSpvR <= 63 && (kSpvR - kSpvAhead) * kSpvVLoads <= 63, "vmcnt range");
constexpr size_t spv_shared_bytes() {
    return (size_t(kSpvR) * kPvVTile + size_t(3) * kPvCh * kPvStride + kSpvMaxN) * 4 + sizeof(seqsum::Shared) + 32 + 32 * 8;
}
// 16-byte chunk cc (4 channels) of V row r sits at chunk r * 8 + (cc ^ spv_swz(r)) of its slot
__device__ __forceinline__ int spv_swz(int r) { return (r >> 2) & 7; }

template <int DH>
__global__ __launch_bounds__(kSpvThreads) void attn_softmax_pv_kernel(AttnDecodeArgs a) {
    extern __shared__ __align__(16) float spv_smem[];  // [R][V tile] [3][kPvCh][kPvStride] [kSpvMaxN] seqsum red etab
    float* vring = spv_smem;
    float* prod = vring + kSpvR * kPvVTile;
    float* al = prod + 3 * kPvCh * kPvStride;
    seqsum::Shared& sm = *reinterpret_cast<seqsum::Shared*>(al + kSpvMaxN);
    float* red = reinterpret_cast<float*>(&sm + 1);         // [8]
    uint64_t* etab = reinterpret_cast<uint64_t*>(red + 8);  // expf's table, read from shared memory
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64, b = blockIdx.y;
    constexpr int parts = DH / kPvCh;
    int h, part;
    head_part_of(int(blockIdx.x), a.Hq, a.Hkv, parts, h, part);
    const int g = h / (a.Hq / a.Hkv);
    const int pos = a.positions[b];
    if (pos < 0 || pos >= a.max_ctx) return;
    const int first = visible_first(pos, a.window);
    const int n = pos + 1 - first;  // <= kSpvMaxN (the host's condition for this kernel)
    const float* sc = a.scores + (int64_t(b) * a.Hq + h) * a.max_ctx;
    const int64_t kw = int64_t(a.Hkv) * DH;
    const float* vb = a.v_cache + (cache_of(a, b) * a.max_ctx + first) * kw + int64_t(g) * DH + part * kPvCh;
    const int ntiles = (n + kPvRows - 1) / kPvRows;
    constexpr int pstride = kPvCh * kPvStride;
    const bool loader = wave >= 8 - kSpvLoaders;
    const int li = wave - (8 - kSpvLoaders);

    // V tile `tile` into its slot: loader li's load j fills chunk
    // p = 64 (kSpvVLoads li + j) + lane, i.e. row p / 8 and channel chunk
    // (p % 8) ^ spv_swz(row); rows past n read row n - 1, whose products the
    // chain never adds
    auto issue_chunk = [&](int tile, int q) {  // load q (of 8) of a tile: chunks 64 q .. 64 q + 63
        const int p = 64 * q + lane, r = p / 8;
        const int row = min(tile * kPvRows + r, n - 1);
        lds_dma_b128(vb + int64_t(row) * kw + 4 * ((p % 8) ^ spv_swz(r)), lds_offset(vring + (tile % kSpvR) * kPvVTile + 4 * 64 * q));
    };
    auto issue = [&](int tile) {
#pragma unroll
        for (int j = 0; j < kSpvVLoads; ++j) issue_chunk(tile, kSpvVLoads * li + j);
    };

    // ---- the scores into shared memory: chunk q = 4 consecutive scores;
    // chunks past the visible ones read the last visible chunk (never used).
    // Then the whole V ring: every wave issues one of each tile's eight loads
    // (a load takes the issuing wave ~100 cycles, so the loaders alone would
    // hold up the softmax); all of them have landed by the end of the softmax ----
    if (tid < 32) etab[tid] = exp2_table(tid);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int q = min(wave * 128 + k * 64 + lane, (n - 1) / 4);
        lds_dma_b128(sc + 4 * q, lds_offset(al + 4 * (wave * 128 + k * 64)));
    }
    for (int t = 0; t < kSpvR; ++t)
        if (t < ntiles) issue_chunk(t, wave);
    if (ntiles >= kSpvR)
        wait_vmcnt<kSpvR>();  // the scores have landed
    else
        wait_vmcnt<0>();
    __syncthreads();

    // ---- softmax (nm/src/components.hpp:132-141) ----
    float s[8];
    float mx = -INFINITY;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const int j = tid + kSpvThreads * m;
        s[m] = al[j];
        if (j < n) mx = fmaxf(mx, s[m]);
    }
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < 8; ++w) mx = fmaxf(mx, red[w]);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const int j = tid + kSpvThreads * m;
        if (j < n) al[j] = expf_glibc_with(s[m] - mx, [etab](int i) { return etab[i]; });
    }
    __syncthreads();
    const float total = seqsum::sum_nonneg<kSpvThreads>(al, n, sm);  // every wave gets the total
    // alpha over the terms, zero past n up to the last tile's end (the same
    // lanes as the exps): no wave reads the terms after the sum unless it fell
    // back to the plain loop, which ends with a barrier
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const int j = tid + kSpvThreads * m;
        if (j < ntiles * kPvRows) al[j] = j < n ? al[j] / total : 0.f;
    }

    // ---- the weighted sum (core.hpp:206-208) ----
    wait_vmcnt<0>();  // the ring's first R tiles have landed
    __syncthreads();
    // producers: channels c4 .. c4 + 3 of rows r4 .. r4 + 3
    const int c4 = ((wave - 1) * 4 + lane / 16) * 4, r4 = (lane % 16) * 4;
    float4 pv[4], pa;  // the V chunks and weights of the next tile to form
    auto read_tile = [&](int tile) {
        const float* vt = vring + (tile % kSpvR) * kPvVTile;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int r = r4 + k;
            pv[k] = reinterpret_cast<const float4*>(vt)[r * 8 + ((c4 / 4) ^ spv_swz(r))];
        }
        pa = reinterpret_cast<const float4*>(al + tile * kPvRows + r4)[0];
    };
    auto form = [&](int tile) {  // the products alpha_j * v_j[c] (the reference's product, one rounding)
        float* d = prod + (tile % 3) * pstride + c4 * kPvStride + r4;
        reinterpret_cast<float4*>(d)[0] = make_float4(pa.x * pv[0].x, pa.y * pv[1].x, pa.z * pv[2].x, pa.w * pv[3].x);
        reinterpret_cast<float4*>(d + kPvStride)[0] = make_float4(pa.x * pv[0].y, pa.y * pv[1].y, pa.z * pv[2].y, pa.w * pv[3].y);
        reinterpret_cast<float4*>(d + 2 * kPvStride)[0] = make_float4(pa.x * pv[0].z, pa.y * pv[1].z, pa.z * pv[2].z, pa.w * pv[3].z);
        reinterpret_cast<float4*>(d + 3 * kPvStride)[0] = make_float4(pa.x * pv[0].w, pa.y * pv[1].w, pa.z * pv[2].w, pa.w * pv[3].w);
    };
    const bool producer = wave == 1 || wave == 2;
    if (producer) {
        read_tile(0);
        form(0);
        if (ntiles > 1) {
            read_tile(1);
            form(1);
        }
        if (ntiles > 2) read_tile(2);
    }
    __syncthreads();
    // chain: lane c < 32 adds channel c; cur / nxt hold a tile's products
    const bool chain = wave == 0 && lane < kPvCh;
    float4 cur[kPvRows / 4], nxt[kPvRows / 4];
    // tile t + 1's products, read while tile t is added: the reads land
    // before the iteration's closing barrier, which waits for them
    auto read_prod = [&](int tile, float4 (&dst)[kPvRows / 4]) {
        const uint32_t row = lds_offset(prod + (tile % 3) * pstride + lane * kPvStride);
        lds_read_b128x16_untracked(row, dst);
    };
    float acc = 0.f;
    auto add_tile = [&](const float4 (&p)[kPvRows / 4], int rows) {
        if (rows == kPvRows) {
#pragma unroll
            for (int i = 0; i < kPvRows / 4; ++i) {
                acc += p[i].x;
                acc += p[i].y;
                acc += p[i].z;
                acc += p[i].w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < kPvRows / 4; ++i) {
                acc = 4 * i < rows ? acc + p[i].x : acc;
                acc = 4 * i + 1 < rows ? acc + p[i].y : acc;
                acc = 4 * i + 2 < rows ? acc + p[i].z : acc;
                acc = 4 * i + 3 < rows ? acc + p[i].w : acc;
            }
        }
    };
    // one tile of the pipeline: the chain adds `have` (tile t) and reads tile
    // t + 1 into `next`; the loop runs tiles in pairs so the two buffers keep
    // their registers
    auto iteration = [&](int tile, const float4 (&have)[kPvRows / 4], float4 (&next)[kPvRows / 4]) {
        if (loader) {
            if (tile + kSpvR < ntiles) issue(tile + kSpvR);  // into the slot of tile `tile`, read three tiles ago
            // tile + kSpvAhead has landed: it is one of the ring's first R tiles,
            // or at most the loads of the tiles after it up to tile + kSpvR
            // were issued after its own
            if (tile + kSpvR < ntiles)
                wait_vmcnt<(kSpvR - kSpvAhead) * kSpvVLoads>();
            else
                wait_vmcnt<0>();
        } else if (producer) {
            if (tile + 2 < ntiles) form(tile + 2);  // from the registers read last iteration
            if (tile + 3 < ntiles) read_tile(tile + 3);
        } else if (chain) {
            if (tile + 1 < ntiles) read_prod(tile + 1, next);
            add_tile(have, min(kPvRows, n - tile * kPvRows));
        }
        __syncthreads();
    };
    if (chain) read_prod(0, cur);
    __syncthreads();  // tile 0's products in registers
    for (int tile = 0; tile < ntiles; tile += 2) {
        iteration(tile, cur, nxt);
        if (tile + 1 < ntiles) iteration(tile + 1, nxt, cur);
    }

    if (chain) {
        const int ch = part * kPvCh + lane;
        const float gate = a.proj[int64_t(b) * a.proj_stride + int64_t(h) * 2 * DH + DH + ch];
        const float out = acc * sigmoid_f32(gate);
        const int64_t width = int64_t(a.Hq) * DH;
        const int64_t idx = int64_t(h) * DH + ch;
        if (a.out_f32) a.out_f32[int64_t(b) * width + idx] = out;
        float amax = fabsf(out);
        for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
        const float d = amax / 127.f;
        const float id = d != 0.f ? 1.f / d : 0.f;
        int8_t* qs = static_cast<int8_t*>(a.act_out);
        float* qd = reinterpret_cast<float*>(qs + int64_t(a.B) * width);
        qs[int64_t(b) * width + idx] = int8_t(int(roundf(out * id)));
        if (lane == 0) qd[(int64_t(b) * width + idx) >> 5] = half_bits_to_f32(fp32_to_fp16_ref(d));
    }
}

// The same sum for many sequences at once (where the per-head workgroups above
// would outnumber the CUs several times): a workgroup per (sequence, K/V head,
// up to four query heads of its group, 32 channels) whose 256 lanes stream
// the V rows through a ring of register tiles into two channel-major
// shared-memory tiles that all of its query heads read (one V read for the
// group's heads), lane 32 hh + c multiplying and adding channel c of head hh
// from shared memory, four rows per read; small shared memory, so many fit
// per CU.
constexpr int kPvbCh = 32;                                    // channels per workgroup (64 measured slower: 8k, B = 16 275 -> 309 us)
constexpr int kPvbThreads = 256;
constexpr int kPvbHeads = 4;                                  // query heads per workgroup
constexpr int kPvbTile = 128;                                // rows per tile
constexpr int kPvbVec = kPvbTile * kPvbCh / 4 / kPvbThreads;    // float4 per lane per tile
constexpr int kPvbAlpha = kPvbHeads * kPvbTile / kPvbThreads;   // weights per lane per tile
constexpr int kPvbRing = 2;                                  // tiles in flight (4 and 6 measured no faster)
constexpr int kPvbLd = kPvbTile + 4;                         // channel stride in a tile (16-byte rows, 2-way stores)

template <int DH>
__global__ __launch_bounds__(kPvbThreads) void attn_pv_batch_kernel(AttnDecodeArgs a) {
    constexpr int kPvbSplit = DH / kPvbCh;  // channel slices per head
    const int tid = threadIdx.x, b = blockIdx.y;
    const int group = a.Hq / a.Hkv, nchunk = (group + kPvbHeads - 1) / kPvbHeads;
    const int part = int(blockIdx.x) % kPvbSplit, gc = int(blockIdx.x) / kPvbSplit;
    const int g = gc / nchunk, h0 = g * group + (gc % nchunk) * kPvbHeads;
    const int nh = min(kPvbHeads, g * group + group - h0);
    const int pos = a.positions[b];
    if (pos < 0 || pos >= a.max_ctx) return;
    const int first = visible_first(pos, a.window);
    const int n = pos + 1 - first;
    const float* alpha = a.scores + (int64_t(b) * a.Hq + h0) * a.max_ctx;  // head h0 + hh at hh * max_ctx
    const int64_t kw = int64_t(a.Hkv) * DH;
    const float* vb = a.v_cache + (cache_of(a, b) * a.max_ctx + first) * kw + int64_t(g) * DH + part * kPvbCh;
    __shared__ __align__(16) float vt[2][kPvbCh * kPvbLd];  // [channel][row]
    __shared__ __align__(16) float at[2][kPvbHeads][kPvbTile];
    const int ntiles = (n + kPvbTile - 1) / kPvbTile;

    float4 ring[kPvbRing][kPvbVec];
    float aring[kPvbRing][kPvbAlpha];
    // lane slot k of a tile: float4 q = tid + k*256 -> row q/8, channels
    // 4*(q%8)..+3; weight slot k: e = tid + k*256 -> head e / 128, row e % 128;
    // rows clamped to n - 1 and heads to nh - 1 (never used past the end)
    auto load = [&](int tile, float4* dst, float* adst) {
        const int r0 = tile * kPvbTile;
#pragma unroll
        for (int k = 0; k < kPvbVec; ++k) {
            const int q = tid + k * kPvbThreads;
            const int row = min(r0 + q / (kPvbCh / 4), n - 1);
            dst[k] = *reinterpret_cast<const float4*>(vb + int64_t(row) * kw + 4 * (q % (kPvbCh / 4)));
        }
#pragma unroll
        for (int k = 0; k < kPvbAlpha; ++k) {
            const int e = tid + k * kPvbThreads, hh = min(e / kPvbTile, nh - 1), r = min(r0 + e % kPvbTile, n - 1);
            adst[k] = alpha[int64_t(hh) * a.max_ctx + r];
        }
    };
#pragma unroll
    for (int s = 0; s < kPvbRing; ++s)
        if (s < ntiles) load(s, ring[s], aring[s]);

    const int hh = tid / kPvbCh, c = tid % kPvbCh;  // chain lanes: tid < kPvbCh * nh
    const bool chain = hh < nh;
    float acc = 0.f;
    for (int base = 0; base < ntiles; base += kPvbRing) {
#pragma unroll
        for (int s = 0; s < kPvbRing; ++s) {
            const int tile = base + s;
            if (tile >= ntiles) break;
            float* buf = vt[tile & 1];
#pragma unroll
            for (int k = 0; k < kPvbVec; ++k) {
                const int q = tid + k * kPvbThreads, row = q / (kPvbCh / 4), c0 = 4 * (q % (kPvbCh / 4));
                buf[(c0 + 0) * kPvbLd + row] = ring[s][k].x;
                buf[(c0 + 1) * kPvbLd + row] = ring[s][k].y;
                buf[(c0 + 2) * kPvbLd + row] = ring[s][k].z;
                buf[(c0 + 3) * kPvbLd + row] = ring[s][k].w;
            }
#pragma unroll
            for (int k = 0; k < kPvbAlpha; ++k) {
                const int e = tid + k * kPvbThreads;
                at[tile & 1][e / kPvbTile][e % kPvbTile] = aring[s][k];
            }
            // one barrier per tile: the other buffer's readers finished before it
            __syncthreads();
            if (tile + kPvbRing < ntiles) load(tile + kPvbRing, ring[s], aring[s]);
            if (chain) {
                // 16 rows at a time from two register sets (4 weight reads,
                // 4 V reads each), the next 16 rows' reads issued before the
                // current ones chain (scheduling barriers keep them there) so
                // that each chain waits for its own set only. Fetches are
                // unconditional (rows clamped into the tile; one past the last
                // group goes unused).
                const float* abuf = at[tile & 1][hh];
                const float* vcol = buf + c * kPvbLd;
                const int rows = min(kPvbTile, n - tile * kPvbTile), full = rows & ~15;
                float4 s0[8], s1[8];
                auto fetch = [&](int r0, float4 (&d)[8]) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        d[i] = *reinterpret_cast<const float4*>(abuf + r0 + 4 * i);
                        d[4 + i] = *reinterpret_cast<const float4*>(vcol + r0 + 4 * i);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                };
                auto chain16 = [&](const float4 (&d)[8]) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        acc += d[i].x * d[4 + i].x;
                        acc += d[i].y * d[4 + i].y;
                        acc += d[i].z * d[4 + i].z;
                        acc += d[i].w * d[4 + i].w;
                    }
                    __builtin_amdgcn_sched_barrier(0);
                };
                fetch(0, s0);
                for (int r0 = 0; r0 < full; r0 += 32) {
                    fetch(min(r0 + 16, kPvbTile - 16), s1);
                    chain16(s0);
                    if (r0 + 16 >= full) break;
                    fetch(min(r0 + 32, kPvbTile - 16), s0);
                    chain16(s1);
                }
                for (int r = full; r < rows; ++r) acc += abuf[r] * vcol[r];
            }
        }
    }

    if (chain) {
        const int h = h0 + hh, ch = part * kPvbCh + c;
        const float gate = a.proj[int64_t(b) * a.proj_stride + int64_t(h) * 2 * DH + DH + ch];
        const float out = acc * sigmoid_f32(gate);
        const int64_t width = int64_t(a.Hq) * DH;
        const int64_t idx = int64_t(h) * DH + ch;
        if (a.out_f32) a.out_f32[int64_t(b) * width + idx] = out;
        float amax = fabsf(out);
        for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
        const float d = amax / 127.f;
        const float id = d != 0.f ? 1.f / d : 0.f;
        int8_t* qs = static_cast<int8_t*>(a.act_out);
        float* qd = reinterpret_cast<float*>(qs + int64_t(a.B) * width);
        qs[int64_t(b) * width + idx] = int8_t(int(roundf(out * id)));
        if ((c & 31) == 0) qd[(int64_t(b) * width + idx) >> 5] = half_bits_to_f32(fp32_to_fp16_ref(d));
    }
}

// ---- prefill over the shared cache: softmax and weighted sum by row blocks ------------------
// The softmax of one (row, query head) for n <= 4096 visible keys with the
// scores held in registers: lane t holds elements PT t .. PT t + PT - 1, the
// max is order-free, e_j = exp(s_j - max) stays in registers, the total is the
// sequential sum over j computed exactly (hero/seqsum.hpp; the e_j also go to
// shared memory for its fallback) and alpha_j = e_j / total is written back:
// one read and one write of the scores where attn_softmax_kernel makes three
// reads and two writes. 256-lane workgroups (16 terms a lane) let eight run
// per CU when there are thousands of rows, as in a prefill chunk. The host
// runs it for max_ctx % 4 == 0 (16-byte aligned rows); rows of more than 4096
// keys take the chunked form.
template <int NT>
__global__ __launch_bounds__(NT) void attn_softmax_regs_kernel(AttnDecodeArgs a) {
    constexpr int PT = seqsum::kMaxN / NT;
    constexpr int W = NT / 64;
    const int tid = threadIdx.x, h = blockIdx.x, b = blockIdx.y;
    const int pos = a.positions[b];
    if (pos < 0 || pos >= a.max_ctx) return;
    const int first = visible_first(pos, a.window);
    const int n = pos + 1 - first;
    float* sc = a.scores + (int64_t(b) * a.Hq + h) * a.max_ctx;
    __shared__ seqsum::Shared sm;
    __shared__ __align__(16) float terms[seqsum::kMaxN];
    __shared__ float red[W];
    if (n > seqsum::kMaxN) {  // longer rows: the chunked form
        float mx = -INFINITY;
        for (int t = tid; t < n; t += NT) mx = fmaxf(mx, sc[t]);
        for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
        if ((tid & 63) == 0) red[tid >> 6] = mx;
        __syncthreads();
        mx = red[0];
#pragma unroll
        for (int w = 1; w < W; ++w) mx = fmaxf(mx, red[w]);
        softmax_chunked<NT>(sc, n, mx, sm, terms);
        return;
    }

    const int i0 = tid * PT;
    float v[PT];
#pragma unroll
    for (int k = 0; k < PT; k += 4) {
        float4 q = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        if (i0 + k + 4 <= n) {
            q = *reinterpret_cast<const float4*>(sc + i0 + k);
        } else if (i0 + k < n) {
            q.x = sc[i0 + k];
            if (i0 + k + 1 < n) q.y = sc[i0 + k + 1];
            if (i0 + k + 2 < n) q.z = sc[i0 + k + 2];
        }
        v[k] = q.x, v[k + 1] = q.y, v[k + 2] = q.z, v[k + 3] = q.w;
    }
    float mx = v[0];
#pragma unroll
    for (int k = 1; k < PT; ++k) mx = fmaxf(mx, v[k]);
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < W; ++w) mx = fmaxf(mx, red[w]);
    if (i0 < n) {  // whole waves past the row skip the exponentials
#pragma unroll
        for (int k = 0; k < PT; ++k) v[k] = i0 + k < n ? exp_f32(v[k] - mx) : 0.f;
    } else {
#pragma unroll
        for (int k = 0; k < PT; ++k) v[k] = 0.f;
    }
    const float total = seqsum::sum_nonneg_regs<NT>(v, terms, n, sm);
#pragma unroll
    for (int k = 0; k < PT; k += 4) {
        if (i0 + k + 4 <= n) {
            *reinterpret_cast<float4*>(sc + i0 + k) = make_float4(v[k] / total, v[k + 1] / total, v[k + 2] / total, v[k + 3] / total);
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (i0 + k + u < n) sc[i0 + k + u] = v[k + u] / total;
        }
    }
}

// out[c] = sum_j alpha_j * v_j[c] (rows in order, core.hpp:206-208) for a
// block of R consecutive rows of one sequence (a prefill chunk, full causal
// visibility), all query heads of one K/V group chunk (up to 4) and all 128
// channels: each V row and each weight is read from memory once per block
// instead of once per row and head. Wave w owns channels 32 w .. 32 w + 31;
// lane l owns row r = l % R and channels 32 w + CPL (l / R) .. + CPL - 1 of
// every head of the chunk (4 x CPL chains in registers). 32-key tiles of V
// ([key][128 channels]) and of the weights ([key quad][head, row][4 keys])
// land in shared memory through global_load_lds, two buffers deep; per key a
// lane reads its CPL channels (all lanes with the same channel group share
// the address) and, per 4 keys, one 16-byte weight read per head (lanes
// of consecutive rows read consecutive addresses), then does 8 CPL fp32
// operations. A row only adds keys at or before its position (the tiles past
// the block's first position test it per lane). Then the gate and the Q8_0
// block of 32 channels (spread over 32 / CPL lanes) as attn_pv_kernel.
// The host runs it for window 0 and max_ctx % 4 == 0 (16-byte aligned
// weight quads and V rows).
constexpr int kPrRows = 8;                         // rows per workgroup (16 measured 2% slower over a 2048-token prefill)
constexpr int kPrKeys = 32;                        // keys per tile
constexpr int kPrThreads = 256;                    // four waves: 32 channels each
constexpr int kPrHeads = 4;                        // query heads per workgroup
constexpr int kPrVQuads = kPrKeys * kAttnDim / 4;  // 16-byte pieces of a V tile: 1024

template <int R, int DH>
__global__ __launch_bounds__(kPrThreads) void attn_pv_rows_kernel(AttnDecodeArgs a) {
    constexpr int kParts = DH / kAttnDim;  // 128-channel parts of a head (one workgroup each)
    constexpr int CG = 64 / R;          // channel groups per wave
    constexpr int CPL = 32 / CG;        // channels per lane
    constexpr int NP = kPrHeads * R;    // (head, row) pairs
    constexpr int AQuads = kPrKeys / 4 * NP;  // 16-byte pieces of a weight tile
    static_assert(CPL % 4 == 0 && AQuads % kPrThreads == 0 && kPrVQuads % kPrThreads == 0, "tile geometry");
    __shared__ __align__(16) float vt[2][kPrKeys * kAttnDim];  // [key][channel]
    __shared__ __align__(16) float at[2][AQuads * 4];          // [key quad][head * R + row][4 keys]

    const int tid = int(threadIdx.x), wave = tid / 64, lane = tid % 64;
    const int r = lane % R, cg = lane / R;
    const int group = a.Hq / a.Hkv, nchunk = (group + kPrHeads - 1) / kPrHeads;
    const int part = int(blockIdx.x) % kParts, gcx = int(blockIdx.x) / kParts;
    const int g = gcx / nchunk, h0 = g * group + (gcx % nchunk) * kPrHeads;
    const int nh = min(kPrHeads, g * group + group - h0);
    const int row0 = int(blockIdx.y) * R;
    const int nrows = min(R, a.B - row0);
    // the block's positions: the first row's (every row sees keys up to it)
    // and the largest (the last tile)
    const int my_row = row0 + min(r, nrows - 1);
    const int my_pos = r < nrows ? a.positions[my_row] : -1;
    int pos_lo = INT32_MAX, pos_hi = -1;
    for (int i = 0; i < nrows; ++i) {
        const int p = a.positions[row0 + i];
        pos_lo = min(pos_lo, p);
        pos_hi = max(pos_hi, p);
    }
    if (pos_hi < 0 || pos_hi >= a.max_ctx || pos_lo < 0) return;  // the host keeps positions in range
    const int ntiles = (pos_hi + kPrKeys) / kPrKeys;
    const int full_tiles = (pos_lo + 1) / kPrKeys;  // tiles every row of the block sees whole
    const int64_t kw = int64_t(a.Hkv) * DH;
    const float* vb = a.v_cache + int64_t(g) * DH + part * kAttnDim;  // shared cache: sequence 0; this part's channels

    // staging: V piece q = key q / 32, channels 4 (q % 32) ..; weight piece
    // q = key quad q / NP, pair q % NP = head * R + row; rows past the block and
    // heads past nh read the last valid ones, keys past the cache its last
    // rows (never used)
    auto issue = [&](int tile) {
        const int j0 = tile * kPrKeys;
        float* vdst = vt[tile & 1];
        float* adst = at[tile & 1];
#pragma unroll
        for (int k = 0; k < kPrVQuads / kPrThreads; ++k) {
            const int q = k * kPrThreads + tid;
            const int key = min(j0 + q / 32, int(a.max_ctx) - 1);
            lds_dma_b128(vb + int64_t(key) * kw + 4 * (q % 32), lds_offset(vdst + 4 * (k * kPrThreads + wave * 64)));
        }
#pragma unroll
        for (int k = 0; k < AQuads / kPrThreads; ++k) {
            const int q = k * kPrThreads + tid;
            const int pair = q % NP, kq = q / NP;
            const int hh = min(pair / R, nh - 1), rr = min(pair % R, nrows - 1);
            const int key = min(j0 + 4 * kq, int(a.max_ctx) - 4);
            const float* src = a.scores + (int64_t(row0 + rr) * a.Hq + h0 + hh) * a.max_ctx + key;
            lds_dma_b128(src, lds_offset(adst + 4 * (k * kPrThreads + wave * 64)));
        }
    };

    float acc[kPrHeads][CPL];
#pragma unroll
    for (int hh = 0; hh < kPrHeads; ++hh)
#pragma unroll
        for (int i = 0; i < CPL; ++i) acc[hh][i] = 0.f;

    // one tile: keys j0 .. j0 + 31, four at a time; MASK: test each key
    // against the lane's position
    auto tile_sum = [&](const float* vbuf, const float* abuf, int j0, auto mask) {
        constexpr bool M = decltype(mask)::value;
#pragma unroll
        for (int kq = 0; kq < kPrKeys / 4; ++kq) {
            float4 al[kPrHeads];
#pragma unroll
            for (int hh = 0; hh < kPrHeads; ++hh) al[hh] = *reinterpret_cast<const float4*>(abuf + 4 * (kq * NP + hh * R + r));
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const float* vrow = vbuf + (4 * kq + kk) * kAttnDim + 32 * wave + CPL * cg;
                float vv[CPL];
#pragma unroll
                for (int i = 0; i < CPL; i += 4) {
                    const float4 q = *reinterpret_cast<const float4*>(vrow + i);
                    vv[i] = q.x, vv[i + 1] = q.y, vv[i + 2] = q.z, vv[i + 3] = q.w;
                }
                const bool use = !M || j0 + 4 * kq + kk <= my_pos;
#pragma unroll
                for (int hh = 0; hh < kPrHeads; ++hh) {
                    const float w = kk == 0 ? al[hh].x : kk == 1 ? al[hh].y : kk == 2 ? al[hh].z : al[hh].w;
#pragma unroll
                    for (int i = 0; i < CPL; ++i) {
                        const float sum = acc[hh][i] + w * vv[i];
                        acc[hh][i] = M ? (use ? sum : acc[hh][i]) : sum;
                    }
                }
            }
        }
    };

    issue(0);
    for (int tile = 0; tile < ntiles; ++tile) {
        wait_vmcnt<0>();
        __syncthreads();  // the tile has landed everywhere; the other buffer's readers are done
        if (tile + 1 < ntiles) issue(tile + 1);
        const float* vbuf = vt[tile & 1];
        const float* abuf = at[tile & 1];
        if (tile < full_tiles)
            tile_sum(vbuf, abuf, tile * kPrKeys, std::false_type{});
        else
            tile_sum(vbuf, abuf, tile * kPrKeys, std::true_type{});
    }

    // gate, Q8_0 block of each (row, head): 32 channels over the CG lanes of the row
    const int64_t width = int64_t(a.Hq) * DH;
    int8_t* qs = static_cast<int8_t*>(a.act_out);
    float* qd = reinterpret_cast<float*>(qs + int64_t(a.B) * width);
    const int ch0 = part * kAttnDim + 32 * wave + CPL * cg;
#pragma unroll
    for (int hh = 0; hh < kPrHeads; ++hh) {
        const int h = h0 + min(hh, nh - 1);
        const float* gate = a.proj + int64_t(my_row) * a.proj_stride + int64_t(h) * 2 * DH + DH + ch0;
        float out[CPL];
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            out[i] = acc[hh][i] * sigmoid_f32(gate[i]);
            amax = fmaxf(amax, fabsf(out[i]));
        }
#pragma unroll
        for (int off = R; off < 64; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
        const float d = amax / 127.f;
        const float id = d != 0.f ? 1.f / d : 0.f;
        if (r < nrows && hh < nh) {
            const int64_t idx = int64_t(my_row) * width + int64_t(h) * DH + ch0;
            if (a.out_f32)
#pragma unroll
                for (int i = 0; i < CPL; i += 4) *reinterpret_cast<float4*>(a.out_f32 + idx + i) = make_float4(out[i], out[i + 1], out[i + 2], out[i + 3]);
            uint32_t pk[CPL / 4];
#pragma unroll
            for (int i = 0; i < CPL; i += 4) {
                uint32_t w = 0;
#pragma unroll
                for (int u = 0; u < 4; ++u) w |= uint32_t(uint8_t(int8_t(int(roundf(out[i + u] * id))))) << (8 * u);
                pk[i / 4] = w;
            }
#pragma unroll
            for (int i = 0; i < CPL / 4; ++i) reinterpret_cast<uint32_t*>(qs + idx)[i] = pk[i];
            if (cg == 0) qd[idx >> 5] = half_bits_to_f32(fp32_to_fp16_ref(d));
        }
    }
}

// ---- paged fp16 cache, split-K ------------------------------------------------------------
// The keys and values are stored as fp16 (round to nearest even) in pages of
// page_size positions; a page table maps each sequence's pages into the pool.
// Scores are the reference's fp32 dot products over the fp16-rounded keys, in
// channel order; the softmax and the weighted sum are split over the keys
// (exp(s - m_split) per split, merged with exp(m_split - m)), so they agree
// with the sequential reference to a few ulp, not bit for bit.
constexpr int kPgTile = 64;  // keys per shared-memory tile

__device__ __forceinline__ uint16_t f32_to_f16_rne(float x) {
    const _Float16 h = _Float16(x);
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}

__device__ __forceinline__ const int32_t* page_row(const AttnPagedArgs& p, int b) { return p.page_table + int64_t(p.a.shared_cache ? 0 : b) * p.max_pages; }

// the fp16 row of position t, KV head g, K (kv = 0) or V (kv = 1), in heads of DH
template <int DH = kAttnDim>
__device__ __forceinline__ int64_t page_offset(const AttnPagedArgs& p, const int32_t* pt, int t, int g, int kv) {
    const int64_t page = pt[t / p.page_size];
    return ((page * 2 + kv) * p.a.Hkv + g) * int64_t(p.page_size) * DH + int64_t(t % p.page_size) * DH;
}

// Q8_0 pages: byte offsets of the int8 row and of its four fp16 scales
__device__ __forceinline__ int64_t q8_page_base(const AttnPagedArgs& p, const int32_t* pt, int t) {
    return int64_t(pt[t / p.page_size]) * (2 * int64_t(p.a.Hkv) * p.page_size * (kAttnDim + 8));
}
__device__ __forceinline__ int64_t q8_row(const AttnPagedArgs& p, int t, int g, int kv) {
    return ((int64_t(kv) * p.a.Hkv + g) * p.page_size + t % p.page_size);
}

// quantize_row_q8_0 (nm/src/quant_i8.hpp:70-80) of one 32-lane block held one
// value per lane (lanes j .. j of a 32-aligned group): d = amax / 127 stored
// through the reference's fp16 encoder, q = roundf(x / d)
__device__ __forceinline__ int8_t q8_of_block(float x, uint16_t* dh) {
    float amax = fabsf(x);
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
    const float d = amax / 127.f;
    const float id = d != 0.f ? 1.f / d : 0.f;
    *dh = fp32_to_fp16_ref(d);
    return int8_t(int(roundf(x * id)));
}

template <int DH>
__global__ __launch_bounds__(DH) void attn_paged_prep_kernel(AttnPagedArgs p) {
    const AttnDecodeArgs& a = p.a;
    const int j = threadIdx.x, h = blockIdx.x, b = blockIdx.y;
    const int group = a.Hq / a.Hkv;
    const int g = h / group;
    const int pos = a.positions[b];
    if (pos < 0 || pos >= p.max_pages * p.page_size) return;  // the host keeps positions in range
    const float* P = a.proj + int64_t(b) * a.proj_stride;
    const float* cs = a.rope_cs + int64_t(pos) * DH;
    __shared__ __align__(16) float buf[DH];
    __shared__ float scal[2];
    const float q = norm_rope_head<DH>(P[int64_t(h) * 2 * DH + j], a.q_gamma, a.eps, cs, buf, scal, j);
    a.q_rot[(int64_t(b) * a.Hq + h) * DH + j] = q;
    if (h % group == 0) {
        const float k = norm_rope_head<DH>(P[a.k_off + int64_t(g) * DH + j], a.k_gamma, a.eps, cs, buf, scal, j);
        const float v = P[a.v_off + int64_t(g) * DH + j];
        const int32_t* pt = page_row(p, b);
        if constexpr (DH == kAttnDim) {
            if (p.q8) {
                uint8_t* pool = reinterpret_cast<uint8_t*>(p.pages);
                const int64_t base = q8_page_base(p, pt, pos);
                const int64_t scales = base + 2 * int64_t(a.Hkv) * p.page_size * kAttnDim;
                uint16_t dk, dv;
                const int8_t qk = q8_of_block(k, &dk), qv = q8_of_block(v, &dv);
                pool[base + q8_row(p, pos, g, 0) * kAttnDim + j] = uint8_t(qk);
                pool[base + q8_row(p, pos, g, 1) * kAttnDim + j] = uint8_t(qv);
                if ((j & 31) == 0) {
                    reinterpret_cast<uint16_t*>(pool + scales)[q8_row(p, pos, g, 0) * 4 + j / 32] = dk;
                    reinterpret_cast<uint16_t*>(pool + scales)[q8_row(p, pos, g, 1) * 4 + j / 32] = dv;
                }
                return;
            }
        }
        p.pages[page_offset<DH>(p, pt, pos, g, 0) + j] = f32_to_f16_rne(k);
        p.pages[page_offset<DH>(p, pt, pos, g, 1) + j] = f32_to_f16_rne(v);
    }
}

// One workgroup per (KV head, split, row): the split's keys in tiles of 64.
// Lane (key r = tid / 4 of the tile, channel quarter cq = 32 (tid % 4)) loads
// its 32 channels of the key, and of the next tile's key before it uses the
// current one (a register double buffer: a tile's global reads are in flight
// while the previous tile computes).
// Scores: the lane's partial dots for every query head of the group (fused
// multiply-adds: this path is not the reference's operation order anyway),
// summed over the four quarter lanes. Softmax: a wave per head, local max and
// exp-sum. Weighted sum: the V tile stays in shared memory as stored (fp16
// pairs, or Q8_0 quads and scales); lane (channel c = tid % 128, half kh =
// tid / 128 of the tile's keys) adds p_h(j) v_j[c] for all heads of the group,
// the weights read four keys at a time.
// Q8: the rows are Q8_0, each value read back as d * q (dequant_row_q8_0,
// nm/src/quant.hpp:306-313), the fp32 value the oracle's Q8_0 cache holds.
template <bool Q8>
struct PgRaw {  // one lane's 32 channels of a row as stored
    uint4 w[Q8 ? 2 : 4];
    uint16_t d;  // Q8: the block scale
};

// G > 0: the query heads per KV head, known at compile time (the loops over
// the group's heads then carry no per-head conditions); G = 0: read from the
// arguments
template <bool Q8, int G>
__global__ __launch_bounds__(256) void attn_split_kernel(AttnPagedArgs p) {
    const AttnDecodeArgs& a = p.a;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int g = blockIdx.x, sp = blockIdx.y, b = blockIdx.z;
    const int Gs = G > 0 ? G : a.Hq / a.Hkv;
    const int pos = a.positions[b];
    if (pos < 0 || pos >= p.max_pages * p.page_size) return;
    const int first = visible_first(pos, a.window);
    const int t0 = first + sp * p.split, t1 = min(pos + 1, t0 + p.split);
    const int64_t rec = 2 + kAttnDim;
    float* out = p.work + ((int64_t(b) * a.Hq + int64_t(g) * Gs) * p.nsplit + sp) * rec;  // head h of the group: + h * nsplit * rec
    const int64_t hstride = int64_t(p.nsplit) * rec;
    if (t0 >= t1) {  // nothing visible in this split
        for (int e = tid; e < Gs * rec; e += 256) out[(e / rec) * hstride + e % rec] = (e % rec) == 0 ? -INFINITY : 0.f;
        return;
    }
    const int n = t1 - t0;
    const int32_t* pt = page_row(p, b);
    const uint8_t* pool = reinterpret_cast<const uint8_t*>(p.pages);
    // shared memory sized to the group and the split (more workgroups per CU):
    // queries [Gs][128], scores [Gs][split], the second half's sums [Gs][128]
    extern __shared__ __align__(16) float pg_smem[];
    float (*qs)[kAttnDim] = reinterpret_cast<float (*)[kAttnDim]>(pg_smem);
    float* const sc0 = pg_smem + Gs * kAttnDim;
    const int sstride = p.split;  // a multiple of 64
    float (*part)[kAttnDim] = reinterpret_cast<float (*)[kAttnDim]>(sc0 + Gs * sstride);
    auto sc = [&](int h) { return sc0 + h * sstride; };
    constexpr int kVw = Q8 ? kAttnDim / 4 : kAttnDim / 2;  // dwords per stored V row
    __shared__ uint32_t vt[kPgTile][kVw + 1];
    __shared__ float vsc[Q8 ? kPgTile : 1][4];
    for (int e = tid; e < Gs * kAttnDim; e += 256) qs[e / kAttnDim][e % kAttnDim] = a.q_rot[(int64_t(b) * a.Hq + int64_t(g) * Gs) * kAttnDim + e];

    const int r = tid >> 2, cq = (tid & 3) * 32;
    auto load_raw = [&](int t, int kv, PgRaw<Q8>& x) {
        if (t >= t1) {
#pragma unroll
            for (int u = 0; u < (Q8 ? 2 : 4); ++u) x.w[u] = make_uint4(0u, 0u, 0u, 0u);
            x.d = 0;
            return;
        }
        if constexpr (Q8) {
            const int64_t base = q8_page_base(p, pt, t), row = q8_row(p, t, g, kv);
            const uint4* src = reinterpret_cast<const uint4*>(pool + base + row * kAttnDim + cq);
            x.w[0] = src[0], x.w[1] = src[1];
            x.d = reinterpret_cast<const uint16_t*>(pool + base + 2 * int64_t(a.Hkv) * p.page_size * kAttnDim)[row * 4 + cq / 32];
        } else {
            const uint4* src = reinterpret_cast<const uint4*>(p.pages + page_offset(p, pt, t, g, kv) + cq);
#pragma unroll
            for (int u = 0; u < 4; ++u) x.w[u] = src[u];
            x.d = 0;
        }
    };
    auto to_f32 = [&](const PgRaw<Q8>& x, float (&v)[32]) {
        if constexpr (Q8) {
            const float d = half_bits_to_f32(x.d);
#pragma unroll
            for (int e = 0; e < 32; ++e) {
                const uint4 w = x.w[e / 16];
                const uint32_t dw = (e % 16) < 4 ? w.x : (e % 16) < 8 ? w.y : (e % 16) < 12 ? w.z : w.w;
                v[e] = d * float(int8_t((dw >> (8 * (e % 4))) & 0xFFu));
            }
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t w[4] = {x.w[u].x, x.w[u].y, x.w[u].z, x.w[u].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[8 * u + 2 * e] = half_bits_to_f32(uint16_t(w[e] & 0xFFFFu));
                    v[8 * u + 2 * e + 1] = half_bits_to_f32(uint16_t(w[e] >> 16));
                }
            }
        }
    };
    __syncthreads();  // qs

    // scores (core.hpp:496-500's dot, reordered): partial dots over the lane's
    // quarter, then the four quarters of the key
    const int ntiles = (n + kPgTile - 1) / kPgTile;
    PgRaw<Q8> cur, nxt;
    load_raw(t0 + r, 0, cur);
    for (int tile = 0; tile < ntiles; ++tile) {
        load_raw(t0 + (tile + 1) * kPgTile + r, 0, nxt);  // zeros past the split
        float kx[32];
        to_f32(cur, kx);
        const int jj = tile * kPgTile + r;
#pragma unroll
        for (int h = 0; h < kAttnMaxGroup; ++h) {
            if (h < Gs) {
                float dot = 0.f;
                const float4* q4 = reinterpret_cast<const float4*>(&qs[h][cq]);
#pragma unroll
                for (int e4 = 0; e4 < 8; ++e4) {
                    const float4 q = q4[e4];
                    dot = fmaf(q.x, kx[4 * e4], dot);
                    dot = fmaf(q.y, kx[4 * e4 + 1], dot);
                    dot = fmaf(q.z, kx[4 * e4 + 2], dot);
                    dot = fmaf(q.w, kx[4 * e4 + 3], dot);
                }
                dot += __shfl_xor(dot, 1);
                dot += __shfl_xor(dot, 2);
                if ((tid & 3) == 0 && jj < n) sc(h)[jj] = a.score_scale * dot;
            }
        }
        cur = nxt;
    }
    load_raw(t0 + r, 1, cur);  // the first V tile, in flight during the softmax
    __syncthreads();
    // per head (a wave each): local max, p = exp(s - m), local sum; the
    // weights past n are zero so the weighted sum reads whole quads
    for (int h = wv; h < Gs; h += 4) {
        float m = -INFINITY;
        for (int jj = lane; jj < n; jj += 64) m = fmaxf(m, sc(h)[jj]);
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        float l = 0.f;
        for (int jj = lane; jj < ntiles * kPgTile; jj += 64) {
            const float e = jj < n ? exp_f32(sc(h)[jj] - m) : 0.f;
            sc(h)[jj] = e;
            l += e;
        }
        for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
        if (lane == 0) {
            out[h * hstride] = m;
            out[h * hstride + 1] = l;
        }
    }
    // weighted sum of values: lane -> channel c, keys kh * 32 .. +31 of each tile
    const int c = tid & (kAttnDim - 1), kh = tid >> 7;
    float o[kAttnMaxGroup];
#pragma unroll
    for (int h = 0; h < kAttnMaxGroup; ++h) o[h] = 0.f;
    for (int tile = 0; tile < ntiles; ++tile) {
        load_raw(t0 + (tile + 1) * kPgTile + r, 1, nxt);
        __syncthreads();  // sc complete (first tile) / the previous tile's readers done
        if constexpr (Q8) {
            vt[r][cq / 4 + 0] = cur.w[0].x, vt[r][cq / 4 + 1] = cur.w[0].y, vt[r][cq / 4 + 2] = cur.w[0].z, vt[r][cq / 4 + 3] = cur.w[0].w;
            vt[r][cq / 4 + 4] = cur.w[1].x, vt[r][cq / 4 + 5] = cur.w[1].y, vt[r][cq / 4 + 6] = cur.w[1].z, vt[r][cq / 4 + 7] = cur.w[1].w;
            vsc[r][cq / 32] = half_bits_to_f32(cur.d);
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                vt[r][cq / 2 + 4 * u + 0] = cur.w[u].x;
                vt[r][cq / 2 + 4 * u + 1] = cur.w[u].y;
                vt[r][cq / 2 + 4 * u + 2] = cur.w[u].z;
                vt[r][cq / 2 + 4 * u + 3] = cur.w[u].w;
            }
        }
        __syncthreads();
        const int j0 = tile * kPgTile + 32 * kh;
#pragma unroll 2
        for (int q4i = 0; q4i < 8; ++q4i) {
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int jr = 32 * kh + 4 * q4i + u;
                if constexpr (Q8) {
                    const uint32_t dw = vt[jr][c >> 2];
                    v[u] = vsc[jr][c >> 5] * float(int8_t((dw >> (8 * (c & 3))) & 0xFFu));
                } else {
                    const uint32_t dw = vt[jr][c >> 1];
                    v[u] = half_bits_to_f32(uint16_t((c & 1) ? (dw >> 16) : (dw & 0xFFFFu)));
                }
            }
#pragma unroll
            for (int h = 0; h < kAttnMaxGroup; ++h) {
                if (h < Gs) {
                    const float4 w = *reinterpret_cast<const float4*>(sc(h) + j0 + 4 * q4i);
                    o[h] = fmaf(w.x, v[0], o[h]);
                    o[h] = fmaf(w.y, v[1], o[h]);
                    o[h] = fmaf(w.z, v[2], o[h]);
                    o[h] = fmaf(w.w, v[3], o[h]);
                }
            }
        }
        cur = nxt;
    }
    if (kh == 1) {
#pragma unroll
        for (int h = 0; h < kAttnMaxGroup; ++h)
            if (h < Gs) part[h][c] = o[h];
    }
    __syncthreads();
    if (kh == 0) {
#pragma unroll
        for (int h = 0; h < kAttnMaxGroup; ++h)
            if (h < Gs) out[h * hstride + 2 + c] = o[h] + part[h][c];
    }
}

// Pages of 64 positions, fp16 (the model's paged cache): one workgroup per
// (KV head, split, row) streams the pages its split touches, the K block of
// each page (64 keys x 128 channels, 16 KB, contiguous in the pool) and then
// the V blocks, through a ring of kRgSlots shared-memory slots filled by
// global_load_lds: up to three pages in flight while one is computed, instead
// of one register tile. The arithmetic is attn_split_kernel's: a lane's
// partial dot over a channel quarter with fused multiply-adds, the quarters
// summed, the split's max, exp and sum, and the weighted sum by fused
// multiply-adds (four key quarters summed at the end). Keys of a page outside
// the split [t0, t1) get no weight, and the rows past the newest position read
// as zero (the pool may hold anything there).
template <int DH>
constexpr int rg_slots() { return DH == 128 ? 4 : 3; }             // pages in flight per workgroup
template <int DH>
constexpr int rg_slot() { return kPgTile * DH * 2; }               // bytes of one page's K (or V) block of one KV head

template <int DH>
size_t attn_split_ring_smem(int Gs, int split) {
    return size_t(rg_slots<DH>()) * rg_slot<DH>() + size_t(Gs) * DH * 4 + size_t(Gs) * (split / kPgTile + 1) * kPgTile * 4;
}

template <int DH, int G>  // G as in attn_split_kernel
__global__ __launch_bounds__(256) void attn_split_ring_kernel(AttnPagedArgs p) {
    constexpr int kSlots = rg_slots<DH>(), kSlot = rg_slot<DH>();
    constexpr int kLoads = kSlot / (256 * 16);  // 16-byte loads per lane per block
    constexpr int CQ = DH / 32;                 // 16-byte chunks of a key's channel quarter
    constexpr int HP = DH == 128 ? 4 : 2;       // query heads per pass (their quarters in registers)
    constexpr int CPL = DH / 64;                // channels per lane in the weighted sum
    const AttnDecodeArgs& a = p.a;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int g = blockIdx.x, sp = blockIdx.y, b = blockIdx.z;
    const int Gs = G > 0 ? G : a.Hq / a.Hkv;
    const int pos = a.positions[b];
    if (pos < 0 || pos >= p.max_pages * p.page_size) return;
    const int first = visible_first(pos, a.window);
    const int t0 = first + sp * p.split, t1 = min(pos + 1, t0 + p.split);
    const int64_t rec = 2 + DH;
    float* out = p.work + ((int64_t(b) * a.Hq + int64_t(g) * Gs) * p.nsplit + sp) * rec;  // head h of the group: + h * nsplit * rec
    const int64_t hstride = int64_t(p.nsplit) * rec;
    if (t0 >= t1) {  // nothing visible in this split
        for (int e = tid; e < Gs * rec; e += 256) out[(e / rec) * hstride + e % rec] = (e % rec) == 0 ? -INFINITY : 0.f;
        return;
    }
    const int pg0 = t0 / kPgTile, np = (t1 - 1) / kPgTile - pg0 + 1;  // pages the split touches
    const int nblk = 2 * np;                                          // their K blocks, then their V blocks
    const int32_t* pt = page_row(p, b);
    extern __shared__ __align__(16) float rg_smem[];
    uint8_t* ring = reinterpret_cast<uint8_t*>(rg_smem);                  // [kSlots][kSlot]
    float* qs = reinterpret_cast<float*>(ring + kSlots * kSlot);          // [Gs][DH]
    float* sc0 = qs + Gs * DH;                                             // [Gs][np * 64]
    const int sstride = np * kPgTile;
    auto sc = [&](int h) { return sc0 + h * sstride; };
    // The pool page of each page the split touches (np <= 9) and expf's table
    // go to shared memory before any ring load: a global read issued after the
    // ring loads (the compiler cannot see them) would wait for all of them.
    __shared__ int pages_sh[kAttnMaxSplit / kPgTile + 1];
    __shared__ uint64_t etab[32];
    if (tid < np) pages_sh[tid] = pt[pg0 + tid];
    fill_exp_table(etab, tid);
    __syncthreads();
    const ExpTab et{etab};
    // block i of the split into slot i % kSlots: wave w's loads move the 1 KB
    // pieces kLoads w .. kLoads w + kLoads - 1 of the block, lane by lane
    auto issue = [&](int i) {
        const int kv = i < np ? 0 : 1;
        const int64_t page = pages_sh[i < np ? i : i - np];
        const uint8_t* src = reinterpret_cast<const uint8_t*>(p.pages) + ((page * 2 + kv) * a.Hkv + g) * int64_t(kSlot);
        const uint32_t dst = lds_offset(ring + (i % kSlots) * kSlot);
#pragma unroll
        for (int u = 0; u < kLoads; ++u) lds_dma_b128(src + ((wv * kLoads + u) * 64 + lane) * 16, dst + (wv * kLoads + u) * 1024);
    };
    // the group's rotated queries, through the same path, issued first
    for (int e = tid; e < Gs * DH / 4; e += 256)
        lds_dma_b128(a.q_rot + (int64_t(b) * a.Hq + int64_t(g) * Gs) * DH + 4 * e, lds_offset(qs + 4 * (e & ~63)));
    int issued = 0;  // blocks issued so far (uniform)
    for (; issued < kSlots && issued < nblk; ++issued) issue(issued);
    // block i has landed everywhere: this wave's loads of the blocks issued
    // after it may still be in flight (kLoads per block), then the barrier
    auto wait_block = [&](int i) {
        switch (issued - i - 1) {
            case 3: wait_vmcnt<3 * kLoads>(); break;
            case 2: wait_vmcnt<2 * kLoads>(); break;
            case 1: wait_vmcnt<kLoads>(); break;
            default: wait_vmcnt<0>(); break;
        }
        __syncthreads();
    };

    // ---- scores: lane (key kr of the page, channel quarter qq), HP query
    // heads at a time with their quarter in registers. The lane visits its CQ
    // 16-byte chunks from a key-dependent one (few bank conflicts), and its
    // query registers hold chunk (u + kr) % CQ in slot u ----
    const int qq = lane & 3, kr = wv * 16 + (lane >> 2);
    float qv[HP][DH / 4];
    auto load_q = [&](int hp) {
#pragma unroll
        for (int hh = 0; hh < HP; ++hh) {
            if (hp + hh < Gs) {
#pragma unroll
                for (int u = 0; u < CQ; ++u) {
                    const float4* q4 = reinterpret_cast<const float4*>(qs + (hp + hh) * DH + (DH / 4) * qq + 8 * ((u + kr) % CQ));
                    const float4 qa = q4[0], qb = q4[1];
                    qv[hh][8 * u] = qa.x, qv[hh][8 * u + 1] = qa.y, qv[hh][8 * u + 2] = qa.z, qv[hh][8 * u + 3] = qa.w;
                    qv[hh][8 * u + 4] = qb.x, qv[hh][8 * u + 5] = qb.y, qv[hh][8 * u + 6] = qb.z, qv[hh][8 * u + 7] = qb.w;
                }
            }
        }
    };
    for (int i = 0; i < np; ++i) {
        wait_block(i);
        if (issued < nblk && i > 0) issue(issued++);  // into the slot the previous block left
        const uint8_t* blk = ring + (i % kSlots) * kSlot + kr * (DH * 2);
        const int t = (pg0 + i) * kPgTile + kr;
        const bool live = t >= t0 && t < t1;
        for (int hp = 0; hp < Gs; hp += HP) {
            if (i == 0 || Gs > HP) load_q(hp);
            float dot[HP];
#pragma unroll
            for (int hh = 0; hh < HP; ++hh) dot[hh] = 0.f;
#pragma unroll
            for (int u = 0; u < CQ; ++u) {
                const uint4 w = *reinterpret_cast<const uint4*>(blk + (CQ * qq + ((u + kr) % CQ)) * 16);
                const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
                float kx[8];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    kx[2 * e] = half_bits_to_f32(uint16_t(wd[e] & 0xFFFFu));
                    kx[2 * e + 1] = half_bits_to_f32(uint16_t(wd[e] >> 16));
                }
#pragma unroll
                for (int hh = 0; hh < HP; ++hh)
#pragma unroll
                    for (int e = 0; e < 8; ++e) dot[hh] = fmaf(qv[hh][8 * u + e], kx[e], dot[hh]);
            }
#pragma unroll
            for (int hh = 0; hh < HP; ++hh) {
                if (hp + hh < Gs) {
                    float d = dot[hh];
                    d += __shfl_xor(d, 1);
                    d += __shfl_xor(d, 2);
                    if (qq == 0) sc(hp + hh)[i * kPgTile + kr] = live ? a.score_scale * d : -INFINITY;
                }
            }
        }
    }
    __syncthreads();
    // ---- per head (a wave each): the split's max, p = exp(s - m), the sum ----
    for (int h = wv; h < Gs; h += 4) {
        float m = -INFINITY;
        for (int jj = lane; jj < sstride; jj += 64) m = fmaxf(m, sc(h)[jj]);
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        float l = 0.f;
        for (int jj = lane; jj < sstride; jj += 64) {
            const float sv = sc(h)[jj];
            const float e = sv == -INFINITY ? 0.f : et.exp(sv - m);
            sc(h)[jj] = e;
            l += e;
        }
        for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
        if (lane == 0) {
            out[h * hstride] = m;
            out[h * hstride + 1] = l;
        }
    }
    // ---- weighted sum: lane (channels CPL lane .. CPL lane + CPL - 1), keys
    // 16 wv .. +15 of each page ----
    float o[kAttnMaxGroup][CPL];
#pragma unroll
    for (int h = 0; h < kAttnMaxGroup; ++h)
#pragma unroll
        for (int e = 0; e < CPL; ++e) o[h][e] = 0.f;
    for (int i = np; i < nblk; ++i) {
        wait_block(i);  // its barrier also publishes the weights (first V block)
        if (issued < nblk) issue(issued++);  // into the slot block i - 1 left
        const uint8_t* blk = ring + (i % kSlots) * kSlot;
        const int jb = (i - np) * kPgTile + wv * 16;  // the wave's first key of the page (weight index)
        const int tb = (pg0 + i - np) * kPgTile + wv * 16;
#pragma unroll
        for (int j4 = 0; j4 < 16; j4 += 4) {
            float4 w[kAttnMaxGroup];
#pragma unroll
            for (int h = 0; h < kAttnMaxGroup; ++h)
                if (h < Gs) w[h] = *reinterpret_cast<const float4*>(sc(h) + jb + j4);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint8_t* row = blk + (wv * 16 + j4 + u) * (DH * 2) + lane * (2 * CPL);
                uint32_t dw[CPL / 2];
                if constexpr (CPL == 2) {
                    dw[0] = *reinterpret_cast<const uint32_t*>(row);
                } else {
                    const uint2 d2 = *reinterpret_cast<const uint2*>(row);
                    dw[0] = d2.x, dw[1] = d2.y;
                }
                const bool live = tb + j4 + u < t1;
                float v[CPL];
#pragma unroll
                for (int e = 0; e < CPL / 2; ++e) {
                    v[2 * e] = live ? half_bits_to_f32(uint16_t(dw[e] & 0xFFFFu)) : 0.f;
                    v[2 * e + 1] = live ? half_bits_to_f32(uint16_t(dw[e] >> 16)) : 0.f;
                }
#pragma unroll
                for (int h = 0; h < kAttnMaxGroup; ++h) {
                    if (h < Gs) {
                        const float wu = u == 0 ? w[h].x : u == 1 ? w[h].y : u == 2 ? w[h].z : w[h].w;
#pragma unroll
                        for (int e = 0; e < CPL; ++e) o[h][e] = fmaf(wu, v[e], o[h][e]);
                    }
                }
            }
        }
    }
    __syncthreads();  // every wave is done with the ring: it holds the key quarters' sums now
    float* red = reinterpret_cast<float*>(ring);  // [4][Gs][DH]
#pragma unroll
    for (int h = 0; h < kAttnMaxGroup; ++h) {
        if (h < Gs) {
#pragma unroll
            for (int e = 0; e < CPL; ++e) red[(wv * Gs + h) * DH + CPL * lane + e] = o[h][e];
        }
    }
    __syncthreads();
    for (int e = tid; e < Gs * DH; e += 256) {
        const int h = e / DH, c = e % DH;
        float v = red[(0 * Gs + h) * DH + c];
        v += red[(1 * Gs + h) * DH + c];
        v += red[(2 * Gs + h) * DH + c];
        v += red[(3 * Gs + h) * DH + c];
        out[h * hstride + 2 + c] = v;
    }
}

// One workgroup per (query head, row): merge the splits, then the gate
// (qwen35.hpp:390-393) and the Q8_0 quantization for W_o. Lane (channel c,
// split group sg of 4) adds its channel over splits sg, sg + 4, ... with all
// of its record reads issued at once (kCombinePass per pass); the four
// groups' partial sums are then added in group order.
constexpr int kCombineGroups = 4;
constexpr int kCombinePass = 16;  // splits per lane per pass
template <int DH>
__global__ __launch_bounds__(DH * kCombineGroups) void attn_combine_kernel(AttnPagedArgs p) {
    const AttnDecodeArgs& a = p.a;
    const int tid = threadIdx.x, c = tid % DH, sg = tid / DH, h = blockIdx.x, b = blockIdx.y;
    const int pos = a.positions[b];
    if (pos < 0 || pos >= p.max_pages * p.page_size) return;
    const int64_t rec = 2 + DH;
    const float* w = p.work + (int64_t(b) * a.Hq + h) * p.nsplit * rec;
    __shared__ float red[DH * kCombineGroups / 64];
    __shared__ float part[kCombineGroups][2][DH];
    float l = 0.f, o = 0.f;
    if (p.nsplit <= kCombineGroups * kCombinePass) {
        // one pass: the lane's records all loaded at once, the maximum over
        // every split taken from them (a wave's lanes share a split group; the
        // waves together hold every group)
        float mv[kCombinePass], lv[kCombinePass], ov[kCombinePass];
#pragma unroll
        for (int u = 0; u < kCombinePass; ++u) {
            const int s = min(sg + u * kCombineGroups, p.nsplit - 1);
            mv[u] = w[s * rec];
            lv[u] = w[s * rec + 1];
            ov[u] = w[s * rec + 2 + c];
        }
        float mloc = -INFINITY;
#pragma unroll
        for (int u = 0; u < kCombinePass; ++u)
            if (sg + u * kCombineGroups < p.nsplit) mloc = fmaxf(mloc, mv[u]);
        for (int off = 32; off > 0; off >>= 1) mloc = fmaxf(mloc, __shfl_xor(mloc, off));
        if ((tid & 63) == 0) red[tid >> 6] = mloc;
        __syncthreads();
        float m = red[0];
        for (int i = 1; i < DH * kCombineGroups / 64; ++i) m = fmaxf(m, red[i]);
#pragma unroll
        for (int u = 0; u < kCombinePass; ++u) {
            if (sg + u * kCombineGroups < p.nsplit && mv[u] != -INFINITY) {
                const float f = exp_f32(mv[u] - m);
                l += lv[u] * f;
                o += ov[u] * f;
            }
        }
    } else {  // more splits: the maximum first, then passes of kCombinePass
        float mloc = -INFINITY;
        for (int s = tid; s < p.nsplit; s += DH * kCombineGroups) mloc = fmaxf(mloc, w[s * rec]);
        for (int off = 32; off > 0; off >>= 1) mloc = fmaxf(mloc, __shfl_xor(mloc, off));
        if ((tid & 63) == 0) red[tid >> 6] = mloc;
        __syncthreads();
        float m = red[0];
        for (int i = 1; i < DH * kCombineGroups / 64; ++i) m = fmaxf(m, red[i]);
        for (int base = sg; base < p.nsplit; base += kCombineGroups * kCombinePass) {
            float mv[kCombinePass], lv[kCombinePass], ov[kCombinePass];
#pragma unroll
            for (int u = 0; u < kCombinePass; ++u) {
                const int s = min(base + u * kCombineGroups, p.nsplit - 1);
                mv[u] = w[s * rec];
                lv[u] = w[s * rec + 1];
                ov[u] = w[s * rec + 2 + c];
            }
#pragma unroll
            for (int u = 0; u < kCombinePass; ++u) {
                if (base + u * kCombineGroups < p.nsplit && mv[u] != -INFINITY) {
                    const float f = exp_f32(mv[u] - m);
                    l += lv[u] * f;
                    o += ov[u] * f;
                }
            }
        }
    }
    part[sg][0][c] = l;
    part[sg][1][c] = o;
    __syncthreads();
    if (sg != 0) return;
    l = part[0][0][c], o = part[0][1][c];
#pragma unroll
    for (int g2 = 1; g2 < kCombineGroups; ++g2) {
        l += part[g2][0][c];
        o += part[g2][1][c];
    }
    const float gate = a.proj[int64_t(b) * a.proj_stride + int64_t(h) * 2 * DH + DH + c];
    const float out = (o / l) * sigmoid_f32(gate);
    const int64_t width = int64_t(a.Hq) * DH;
    const int64_t idx = int64_t(h) * DH + c;
    if (a.out_f32) a.out_f32[int64_t(b) * width + idx] = out;
    float amax = fabsf(out);
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    const float d = amax / 127.f;
    const float id = d != 0.f ? 1.f / d : 0.f;
    int8_t* qs = static_cast<int8_t*>(a.act_out);
    float* qd = reinterpret_cast<float*>(qs + int64_t(a.B) * width);
    qs[int64_t(b) * width + idx] = int8_t(int(roundf(out * id)));
    if ((c & 31) == 0) qd[(int64_t(b) * width + idx) >> 5] = half_bits_to_f32(fp32_to_fp16_ref(d));
}

namespace {
// the split kernels for the group size: compiled for 1, 2, 4 and 8 query
// heads per KV head (4: Qwen 3.5 and its tests), read at run time otherwise
template <int DH>
void split_ring_group(const AttnPagedArgs& p, int Gs, hipStream_t s) {
    const dim3 grid(unsigned(p.a.Hkv), unsigned(p.nsplit), unsigned(p.a.B));
    const size_t smem = attn_split_ring_smem<DH>(Gs, p.split);
    switch (Gs) {
        case 1: hipLaunchKernelGGL((attn_split_ring_kernel<DH, 1>), grid, dim3(256), smem, s, p); break;
        case 2: hipLaunchKernelGGL((attn_split_ring_kernel<DH, 2>), grid, dim3(256), smem, s, p); break;
        case 4: hipLaunchKernelGGL((attn_split_ring_kernel<DH, 4>), grid, dim3(256), smem, s, p); break;
        case 8: hipLaunchKernelGGL((attn_split_ring_kernel<DH, 8>), grid, dim3(256), smem, s, p); break;
        default: hipLaunchKernelGGL((attn_split_ring_kernel<DH, 0>), grid, dim3(256), smem, s, p); break;
    }
}
template <bool Q8>
void split_group(const AttnPagedArgs& p, int Gs, size_t smem, hipStream_t s) {
    const dim3 grid(unsigned(p.a.Hkv), unsigned(p.nsplit), unsigned(p.a.B));
    switch (Gs) {
        case 1: hipLaunchKernelGGL((attn_split_kernel<Q8, 1>), grid, dim3(256), smem, s, p); break;
        case 2: hipLaunchKernelGGL((attn_split_kernel<Q8, 2>), grid, dim3(256), smem, s, p); break;
        case 4: hipLaunchKernelGGL((attn_split_kernel<Q8, 4>), grid, dim3(256), smem, s, p); break;
        case 8: hipLaunchKernelGGL((attn_split_kernel<Q8, 8>), grid, dim3(256), smem, s, p); break;
        default: hipLaunchKernelGGL((attn_split_kernel<Q8, 0>), grid, dim3(256), smem, s, p); break;
    }
}
}  // namespace

void attn_paged_plan(int64_t max_ctx, int window, int B, int Hkv, int* split, int* nsplit) {
    const int64_t vis = window > 0 ? std::min<int64_t>(max_ctx, window) : max_ctx;
    // about two workgroups per CU over all rows and KV heads
    const int64_t want = std::max<int64_t>(1, 512 / std::max<int64_t>(1, int64_t(B) * Hkv));
    int64_t sp = (vis + want - 1) / want;
    sp = std::min<int64_t>(kAttnMaxSplit, std::max<int64_t>(kPgTile, (sp + kPgTile - 1) / kPgTile * kPgTile));
    *split = int(sp);
    *nsplit = int((vis + sp - 1) / sp);
}

int64_t attn_paged_work_floats(int B, int Hq, int nsplit, int Dh) { return int64_t(B) * Hq * nsplit * (2 + Dh); }

void launch_attn_paged(const AttnPagedArgs& p, hipStream_t s) {
    const AttnDecodeArgs& a = p.a;
    const int Gs = a.Hq / a.Hkv;
    if (a.Dh == 256) {  // fp16 pages of 64 positions (the host checks): the page-streaming form for any B
        hipLaunchKernelGGL(attn_paged_prep_kernel<256>, dim3(unsigned(a.Hq), unsigned(a.B)), dim3(256), 0, s, p);
        split_ring_group<256>(p, Gs, s);
        hipLaunchKernelGGL(attn_combine_kernel<256>, dim3(unsigned(a.Hq), unsigned(a.B)), dim3(256 * kCombineGroups), 0, s, p);
        return;
    }
    hipLaunchKernelGGL(attn_paged_prep_kernel<kAttnDim>, dim3(unsigned(a.Hq), unsigned(a.B)), dim3(kAttnDim), 0, s, p);
    const size_t smem = size_t(Gs) * (2 * kAttnDim + size_t(p.split)) * 4;
    // the page-streaming form for one or two sequences (the pages of a split
    // in flight at once); with more sequences the grid alone keeps enough
    // loads in flight, and the per-key form, with more workgroups per CU,
    // streams faster (32k context, 16 sequences: 536 vs 727 us)
    if (!p.q8 && p.page_size == kPgTile && a.B <= 2)
        split_ring_group<kAttnDim>(p, Gs, s);
    else if (p.q8)
        split_group<true>(p, Gs, smem, s);
    else
        split_group<false>(p, Gs, smem, s);
    hipLaunchKernelGGL(attn_combine_kernel<kAttnDim>, dim3(unsigned(a.Hq), unsigned(a.B)), dim3(kAttnDim * kCombineGroups), 0, s, p);
}

namespace {
// heads of 256 channels (the reference's Qwen 3.5 4B / 9B attention): the
// per-row kernels, each templated on the head width -- prep, 256-key score
// tiles, the softmax and the many-sequence weighted sum (32 channels per
// workgroup), for any B and for prefill rows
void attn_decode_wide(const AttnDecodeArgs& a, unsigned chunks, unsigned tiles, hipStream_t s) {
    constexpr int DH = 256;
    const int group = a.Hq / a.Hkv;
    const int64_t vis = a.window > 0 ? std::min<int64_t>(a.max_ctx, a.window) : a.max_ctx;
    if (a.max_ctx % 4 == 0 && a.B <= 2 && !a.shared_cache) {  // few sequences: 64-key tiles, the prep folded in
        hipLaunchKernelGGL(attn_scores_tile_wide_kernel, dim3(chunks, unsigned(std::min<int64_t>(kScTiles, (vis + 3 + kScTileKeys - 1) / kScTileKeys)), unsigned(a.B)),
                           dim3(256), 0, s, a);
    } else {
        hipLaunchKernelGGL(attn_prep_kernel<DH>, dim3(unsigned(a.Hq), unsigned(a.B)), dim3(DH), 0, s, a);
        hipLaunchKernelGGL(attn_scores_kernel<DH>, dim3(chunks, tiles, unsigned(a.B)), dim3(256), 0, s, a);
    }
    // few sequences: the per-head pipeline (softmax and weighted sum in one
    // kernel, a workgroup per head and 32 channels) while it fits the CUs
    if (!a.shared_cache && int64_t(a.B) * a.Hq * (DH / kPvCh) <= device_cus() && vis <= kSpvMaxN && a.max_ctx % 4 == 0) {
        hipLaunchKernelGGL(attn_softmax_pv_kernel<DH>, dim3(unsigned(a.Hq * (DH / kPvCh)), unsigned(a.B)), dim3(kSpvThreads), spv_shared_bytes(), s, a);
        return;
    }
    if (a.max_ctx % 4 == 0)
        hipLaunchKernelGGL(attn_softmax_regs_kernel<256>, dim3(unsigned(a.Hq), unsigned(a.B)), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(attn_softmax_kernel, dim3(unsigned(a.Hq), unsigned(a.B)), dim3(seqsum::kThreads), 0, s, a);
    if (a.shared_cache && a.window == 0 && a.max_ctx % 4 == 0) {  // a prefill chunk: the row-block weighted sum, per 128-channel part
        hipLaunchKernelGGL((attn_pv_rows_kernel<kPrRows, DH>), dim3(chunks * (DH / kAttnDim), unsigned((a.B + kPrRows - 1) / kPrRows)), dim3(kPrThreads), 0, s, a);
        return;
    }
    hipLaunchKernelGGL(attn_pv_batch_kernel<DH>, dim3(unsigned(a.Hkv * ((group + kPvbHeads - 1) / kPvbHeads) * (DH / kPvbCh)), unsigned(a.B)), dim3(kPvbThreads), 0, s,
                       a);
}
}  // namespace

void launch_attn_decode(const AttnDecodeArgs& a, hipStream_t s) {
    const int64_t vis = a.window > 0 ? std::min<int64_t>(a.max_ctx, a.window) : a.max_ctx;
    const unsigned tiles = unsigned(std::min<int64_t>(kScoreTiles, (vis + 255) / 256));
    const int group = a.Hq / a.Hkv;
    const unsigned chunks = unsigned(a.Hkv * ((group + kScoreHeads - 1) / kScoreHeads));
    if (a.Dh == 256) {
        attn_decode_wide(a, chunks, tiles, s);
        return;
    }
    // few sequences: 64-key tiles spread the keys over the CUs; many
    // sequences (and prefill rows) fill them with the 256-key form
    if (a.max_ctx % 4 == 0 && a.B <= 2 && !a.shared_cache) {  // prep folded in
        hipLaunchKernelGGL(attn_scores_tile_kernel, dim3(chunks, unsigned(std::min<int64_t>(kScTiles, (vis + 3 + kScTileKeys - 1) / kScTileKeys)), unsigned(a.B)), dim3(256), 0, s, a);
    } else {
        hipLaunchKernelGGL(attn_prep_kernel<kAttnDim>, dim3(unsigned(a.Hq), unsigned(a.B)), dim3(kAttnDim), 0, s, a);
        hipLaunchKernelGGL(attn_scores_kernel<kAttnDim>, dim3(chunks, tiles, unsigned(a.B)), dim3(256), 0, s, a);
    }
    // a prefill chunk (rows of one sequence, full causal visibility): the
    // register softmax and the row-block weighted sum
    if (a.shared_cache && a.window == 0 && a.max_ctx % 4 == 0) {
        hipLaunchKernelGGL(attn_softmax_regs_kernel<256>, dim3(unsigned(a.Hq), unsigned(a.B)), dim3(256), 0, s, a);
        hipLaunchKernelGGL((attn_pv_rows_kernel<kPrRows, kAttnDim>), dim3(unsigned(chunks), unsigned((a.B + kPrRows - 1) / kPrRows)), dim3(kPrThreads), 0, s, a);
        return;
    }
    // the per-head pipeline while its workgroups fit the CUs (a deep ring, one
    // workgroup per CU) or fit them twice over (a shallower ring); for up to
    // 4096 visible keys it runs the softmax itself
    const int64_t pv_blocks = int64_t(a.B) * a.Hq * (kAttnDim / kPvCh);
    const dim3 pv_grid(unsigned(a.Hq * (kAttnDim / kPvCh)), unsigned(a.B));
    if (pv_blocks <= device_cus() && vis <= kSpvMaxN && a.max_ctx % 4 == 0) {
        hipLaunchKernelGGL(attn_softmax_pv_kernel<kAttnDim>, pv_grid, dim3(kSpvThreads), spv_shared_bytes(), s, a);
        return;
    }
    if (a.max_ctx % 4 == 0)
        hipLaunchKernelGGL(attn_softmax_regs_kernel<256>, dim3(unsigned(a.Hq), unsigned(a.B)), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(attn_softmax_kernel, dim3(unsigned(a.Hq), unsigned(a.B)), dim3(seqsum::kThreads), 0, s, a);
    if (pv_blocks <= device_cus())
        hipLaunchKernelGGL(attn_pv_kernel<14>, pv_grid, dim3(kPvThreads), pv_shared_bytes(14), s, a);
    else if (pv_blocks <= 2 * device_cus())
        hipLaunchKernelGGL(attn_pv_kernel<7>, pv_grid, dim3(kPvThreads), pv_shared_bytes(7), s, a);
    else
        hipLaunchKernelGGL(attn_pv_batch_kernel<kAttnDim>, dim3(unsigned(a.Hkv * ((group + kPvbHeads - 1) / kPvbHeads) * (kAttnDim / kPvbCh)), unsigned(a.B)), dim3(kPvbThreads),
                           0, s, a);
}

}  // namespace hero
