// sample.hip -- top-k / top-p sampling on the device (nm/src/logits.hpp:71-105,
// Logits::sample with temp > 0), so a sampled decode needs no logits copy-back.
//
// The caller's RNG stays on the host (the reference's Sampler owns it): the
// caller passes u, the draw std::uniform_real_distribution<float>(0, s2)
// makes from it (libstdc++ returns generate_canonical<float, 24>(rng) * (s2 -
// 0) + 0, so u does not depend on s2).
//
// One workgroup of 1024 lanes:
//   1. the k-th largest logit by a 4-pass, 8-bit radix select on order keys;
//   2. the candidates (every logit above it, then the equal ones in id
//      order) gathered, and sorted by logit descending, equal logits by
//      ascending id (a bitonic sort of 1024);
//   3. p[i] = exp((v[i] - max) / temp) per candidate (glibc's expf);
//   4. one lane runs the reference's sequential loops: the sum of p, the first
//      prefix whose running sum of p / sum reaches top_p, that prefix's sum
//      s2, r = u * s2, and the first candidate whose running sum reaches r.
#include <rocprim/device/device_radix_sort.hpp>

#include "hero/device.hpp"
#include "hero/kernels.hpp"
#include "hero/libm.hpp"
#include "hero/seqsum.hpp"

namespace hero {

namespace {

constexpr int kSampleThreads = 1024;

// order key: larger logit -> larger key (fp32 total order on non-NaN values)
__device__ __forceinline__ uint32_t order_key(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// exclusive prefix sum over the workgroup (1024 lanes = 16 waves)
__device__ __forceinline__ int block_exclusive_scan(int v, int* wsum, int& total) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int x = v;
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off);
        if (lane >= off) x += y;
    }
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    int base = 0, all = 0;
    for (int w = 0; w < kSampleThreads / 64; ++w) {
        const int s = wsum[w];
        if (w < wave) base += s;
        all += s;
    }
    __syncthreads();
    total = all;
    return base + x - v;
}

// The reference's sequential loops over the k sorted candidates' p: their
// sum, the first prefix whose running sum of p / sum reaches top_p, that
// prefix's sum s2, r = u * s2, and the first candidate whose running sum
// reaches r (else the last kept).
__device__ int32_t sequential_pick(const float* pr, const int32_t* idx, int k, float top_p, float u) {
    float sum = 0.f;
    for (int i = 0; i < k; ++i) sum += pr[i];
    float cum = 0.f;
    int keep = k;
    for (int i = 0; i < k; ++i) {
        cum += pr[i] / sum;
        if (cum >= top_p) {
            keep = i + 1;
            break;
        }
    }
    float s2 = 0.f;
    for (int i = 0; i < keep; ++i) s2 += pr[i];
    const float r = u * (s2 - 0.f) + 0.f;
    float acc = 0.f;
    for (int i = 0; i < keep; ++i) {
        acc += pr[i];
        if (r <= acc) return idx[i];
    }
    return idx[keep - 1];
}

// The usual path. Each lane's largest logit over a strided pass; the k-th
// largest of those 1024 maxima, L, is at most the k-th largest logit (k of
// the maxima are logits >= L), so the top k lie among the logits >= L: a few
// hundred for small k. Those are gathered (up to kSampleCand) and sorted in
// shared memory; the first k are the candidates. More than kSampleCand of
// them (large k, heavy ties) sets *fallback for the radix form below.
constexpr int kSampleCand = 4096;

__global__ __launch_bounds__(kSampleThreads) void sample_topk_fast_kernel(const float* __restrict__ logits, int V, int k, float temp, float top_p, float u,
                                                                          int32_t* __restrict__ out, int32_t* __restrict__ fallback) {
    __shared__ uint32_t ckey[kSampleCand];
    __shared__ int32_t cidx[kSampleCand];
    __shared__ float pr[kSampleThreads];
    __shared__ int s_count;
    const int tid = threadIdx.x;

    uint32_t best = 0u;
    for (int i = tid; i < V; i += kSampleThreads) best = max(best, order_key(logits[i]));
    // L = the k-th largest of the lane maxima (k distinct logits are >= it);
    // lanes with no element (V < 1024) hold key 0 and sort last
    ckey[tid] = best;
    __syncthreads();
    for (int size = 2; size <= kSampleThreads; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const int j = tid ^ stride;
            if (j > tid) {
                const uint32_t ka = ckey[tid], kb = ckey[j];
                if ((ka >= kb) != ((tid & size) == 0)) ckey[tid] = kb, ckey[j] = ka;
            }
            __syncthreads();
        }
    }
    const uint32_t L = ckey[k - 1];
    __syncthreads();
    if (tid == 0) s_count = 0;
    for (int i = tid; i < kSampleCand; i += kSampleThreads) ckey[i] = 0u, cidx[i] = 0x7fffffff;
    __syncthreads();

    for (int i = tid; i < V; i += kSampleThreads) {
        const uint32_t key = order_key(logits[i]);
        if (key >= L) {
            const int slot = atomicAdd(&s_count, 1);
            if (slot < kSampleCand) ckey[slot] = key, cidx[slot] = i;
        }
    }
    __syncthreads();
    if (s_count > kSampleCand) {  // uniform: every lane reads the same count
        if (tid == 0) fallback[0] = 1;
        return;
    }
    // bitonic sort of the first n slots (n = the power of two >= the count,
    // at least k): key descending, id ascending
    int n = 2;
    while (n < max(s_count, k)) n <<= 1;
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int t = tid; t < n; t += kSampleThreads) {
                const int j = t ^ stride;
                if (j > t) {
                    const uint32_t ka = ckey[t], kb = ckey[j];
                    const int32_t ia = cidx[t], ib = cidx[j];
                    const bool a_first = ka > kb || (ka == kb && ia < ib);
                    const bool forward = (t & size) == 0;
                    if (a_first != forward) {
                        ckey[t] = kb, cidx[t] = ib;
                        ckey[j] = ka, cidx[j] = ia;
                    }
                }
            }
            __syncthreads();
        }
    }
    if (tid == 0) fallback[0] = 0;
    const float mx = logits[cidx[0]];
    if (tid < k) pr[tid] = expf_glibc((logits[cidx[tid]] - mx) / temp);
    __syncthreads();
    if (tid == 0) out[0] = sequential_pick(pr, cidx, k, top_p, u);
}

__global__ __launch_bounds__(kSampleThreads) void sample_topk_kernel(const float* __restrict__ logits, int V, int k, float temp, float top_p, float u,
                                                                     int32_t* __restrict__ out, const int32_t* __restrict__ fallback) {
    if (fallback[0] == 0) return;  // the usual path answered
    constexpr int kWaves = kSampleThreads / 64;
    __shared__ uint32_t hist[kWaves][256];  // one histogram per wave (less atomic contention)
    __shared__ int wsum[kWaves];
    __shared__ uint32_t skey[kSampleThreads];
    __shared__ int32_t sidx[kSampleThreads];
    __shared__ float pr[kSampleThreads];
    __shared__ uint32_t s_prefix;
    __shared__ int s_above, s_slot;
    const int tid = threadIdx.x, wave = tid >> 6;

    // 1. radix select: the key of the k-th largest and how many lie above it
    uint32_t prefix = 0, mask = 0;
    int above = 0;  // elements known to be larger than the selected prefix
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int i = tid; i < kWaves * 256; i += kSampleThreads) (&hist[0][0])[i] = 0;
        __syncthreads();
        for (int i = tid; i < V; i += kSampleThreads) {
            const uint32_t key = order_key(logits[i]);
            if ((key & mask) == prefix) atomicAdd(&hist[wave][(key >> shift) & 255], 1u);
        }
        __syncthreads();
        if (tid < 256) {
            uint32_t c = 0;
            for (int w = 0; w < kWaves; ++w) c += hist[w][tid];
            hist[0][tid] = c;
        }
        __syncthreads();
        if (tid == 0) {
            int acc = above, d = 255;
            for (; d > 0; --d) {
                if (acc + int(hist[0][d]) >= k) break;
                acc += int(hist[0][d]);
            }
            s_prefix = prefix | (uint32_t(d) << shift);
            s_above = acc;
        }
        __syncthreads();
        prefix = s_prefix;
        above = s_above;
        mask |= 255u << shift;
        __syncthreads();
    }
    const uint32_t T = prefix;  // key of the k-th largest; `above` keys exceed it

    // 2. gather. Counts over a strided (coalesced) pass; when every key equal
    // to T fits beside the `above` larger ones, all of them are collected in
    // any order (the sort below orders equal keys by id, so the first k slots
    // are the right ones); otherwise the equal keys are taken in id order
    // from contiguous per-lane ranges through prefix sums.
    skey[tid] = 0u;
    sidx[tid] = 0x7fffffff;
    int n_eq = 0;
    for (int i = tid; i < V; i += kSampleThreads) n_eq += order_key(logits[i]) == T;
    int tot_eq;
    block_exclusive_scan(n_eq, wsum, tot_eq);
    if (tid == 0) s_slot = 0;
    __syncthreads();
    if (above + tot_eq <= kSampleThreads) {
        for (int i = tid; i < V; i += kSampleThreads) {
            const uint32_t key = order_key(logits[i]);
            if (key >= T) {
                const int slot = atomicAdd(&s_slot, 1);
                skey[slot] = key, sidx[slot] = i;
            }
        }
    } else {
        const int chunk = (V + kSampleThreads - 1) / kSampleThreads;
        const int i0 = min(V, tid * chunk), i1 = min(V, i0 + chunk);
        int c_gt = 0, c_eq = 0;
        for (int i = i0; i < i1; ++i) {
            const uint32_t key = order_key(logits[i]);
            c_gt += key > T;
            c_eq += key == T;
        }
        int tot_gt, tot_eq2;
        int p_gt = block_exclusive_scan(c_gt, wsum, tot_gt);
        int p_eq = block_exclusive_scan(c_eq, wsum, tot_eq2);
        for (int i = i0; i < i1; ++i) {
            const uint32_t key = order_key(logits[i]);
            if (key > T) {
                skey[p_gt] = key, sidx[p_gt] = i;
                ++p_gt;
            } else if (key == T) {
                const int slot = tot_gt + p_eq;
                if (slot < k) skey[slot] = key, sidx[slot] = i;
                ++p_eq;
            }
        }
    }
    __syncthreads();

    // bitonic sort of the 1024 slots: key descending, id ascending (unused
    // slots carry key 0 and the largest id, so they sort last)
    for (int size = 2; size <= kSampleThreads; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const int j = tid ^ stride;
            if (j > tid) {
                const uint32_t ka = skey[tid], kb = skey[j];
                const int32_t ia = sidx[tid], ib = sidx[j];
                const bool a_first = ka > kb || (ka == kb && ia < ib);
                const bool forward = (tid & size) == 0;  // this pair keeps the sort order
                if (a_first != forward) {
                    skey[tid] = kb, sidx[tid] = ib;
                    skey[j] = ka, sidx[j] = ia;
                }
            }
            __syncthreads();
        }
    }

    // 3. probabilities of the k candidates
    const float mx = logits[sidx[0]];
    if (tid < k) pr[tid] = expf_glibc((logits[sidx[tid]] - mx) / temp);
    __syncthreads();

    // 4. the reference's sequential loops
    if (tid == 0) out[0] = sequential_pick(pr, sidx, k, top_p, u);
}

// ---- any k, the whole vocabulary included (top_k = 0) -------------------------------------
// The logits are sorted once, by a stable descending radix sort of (logit, id)
// pairs (rocPRIM; ids ascending within equal logits, -0 taken as +0 as the
// reference's comparison does), then one workgroup runs the reference's
// loops over the first k: the sum of p_i = exp((l_i - max) / temp), the first
// prefix whose running sum of p_i / sum reaches top_p, that prefix's sum s2,
// r = u * s2, and the first i whose running sum of p_i reaches r. Each loop is
// a sequential fp32 sum of non-negative terms, run in chunks of 4095 terms
// that start from the running total (the exact parallel sum of
// hero/seqsum.hpp equals the loop); where a loop stops early, the chunk whose
// end total meets the condition (running sums of non-negative terms never
// decrease) is walked term by term by one lane from its starting total.
__global__ void sample_full_prep_kernel(const float* __restrict__ logits, int V, float* __restrict__ keys, int32_t* __restrict__ ids) {
    const int i = int(blockIdx.x) * 256 + int(threadIdx.x);
    if (i < V) {
        keys[i] = logits[i] + 0.f;  // -0 -> +0; every other value unchanged
        ids[i] = i;
    }
}

struct FullPick {
    seqsum::Shared sm;
    __align__(16) float chunk[seqsum::kMaxN];
    int found;
};

// the running sum over i < n of term(i), chunk by chunk; with `find`, stops
// at the first i whose running sum s_i satisfies pred(s_i) and returns it in
// `at` (-1: none); returns the running sum there (or the total)
template <class Term, class Pred>
__device__ float running_sum(int n, Term term, bool find, Pred pred, int& at, FullPick& sh) {
    const int tid = int(threadIdx.x);
    float total = 0.f;
    at = -1;
    for (int base = 0; base < n; base += seqsum::kMaxN - 1) {
        const int len = min(n - base, seqsum::kMaxN - 1);
        for (int t = tid; t < len; t += kSampleThreads) sh.chunk[t + 1] = term(base + t);
        if (tid == 0) sh.chunk[0] = total;
        __syncthreads();
        const float after = seqsum::sum_nonneg<kSampleThreads>(sh.chunk, len + 1, sh.sm);
        if (find && pred(after)) {
            if (tid == 0) {
                float s = sh.chunk[0];
                int j = 1;
                for (; j <= len; ++j) {
                    s = s + sh.chunk[j];
                    if (pred(s)) break;
                }
                sh.found = base + min(j, len) - 1;  // j <= len: the walk repeats the exact sum
                sh.chunk[0] = s;
            }
            __syncthreads();
            at = sh.found;
            return sh.chunk[0];
        }
        total = after;
        __syncthreads();  // the chunk is rewritten next
    }
    return total;
}

__global__ __launch_bounds__(kSampleThreads) void sample_full_pick_kernel(const float* __restrict__ keys, const int32_t* __restrict__ ids, int k, float temp, float top_p, float u,
                                                                           int32_t* __restrict__ out) {
    __shared__ FullPick sh;
    const float mx = keys[0];
    auto p = [&](int i) { return exp_f32((keys[i] - mx) / temp); };
    auto never = [](float) { return false; };
    int at = -1;
    const float sum = running_sum(k, p, false, never, at, sh);
    running_sum(k, [&](int i) { return p(i) / sum; }, true, [&](float c) { return c >= top_p; }, at, sh);
    const int keep = at >= 0 ? at + 1 : k;
    const float s2 = keep == k ? sum : running_sum(keep, p, false, never, at, sh);
    const float r = u * (s2 - 0.f) + 0.f;
    running_sum(keep, p, true, [&](float a) { return r <= a; }, at, sh);
    if (threadIdx.x == 0) out[0] = ids[at >= 0 ? at : keep - 1];
}

// workspace: sorted and unsorted keys and ids, then rocPRIM's storage
constexpr size_t kFullAlign = 256;
size_t full_part(int64_t V) { return (size_t(V) * 4 + kFullAlign - 1) / kFullAlign * kFullAlign; }
size_t full_sort_bytes(int64_t V) {
    size_t bytes = 0;
    const hipError_t e = rocprim::radix_sort_pairs_desc(nullptr, bytes, static_cast<float*>(nullptr), static_cast<float*>(nullptr), static_cast<int32_t*>(nullptr),
                                                        static_cast<int32_t*>(nullptr), size_t(V));
    if (e != hipSuccess) throw std::runtime_error("rocprim::radix_sort_pairs_desc size query failed");
    return bytes;
}

}  // namespace

int sample_max_top_k() { return kSampleThreads; }

int64_t sample_full_work_bytes(int64_t V) { return int64_t(4 * full_part(V) + full_sort_bytes(V)); }

void launch_sample_full(const float* logits, int64_t V, int top_k, float temp, float top_p, float u, void* work, int32_t* out, hipStream_t s) {
    const int k = int(top_k <= 0 ? V : std::min<int64_t>(top_k, V));
    char* w = static_cast<char*>(work);
    float* keys_in = reinterpret_cast<float*>(w);
    float* keys = reinterpret_cast<float*>(w + full_part(V));
    int32_t* ids_in = reinterpret_cast<int32_t*>(w + 2 * full_part(V));
    int32_t* ids = reinterpret_cast<int32_t*>(w + 3 * full_part(V));
    size_t bytes = full_sort_bytes(V);
    hipLaunchKernelGGL(sample_full_prep_kernel, dim3(unsigned((V + 255) / 256)), dim3(256), 0, s, logits, int(V), keys_in, ids_in);
    if (rocprim::radix_sort_pairs_desc(w + 4 * full_part(V), bytes, keys_in, keys, ids_in, ids, size_t(V), 0, 32, s) != hipSuccess)
        throw std::runtime_error("rocprim::radix_sort_pairs_desc failed");
    hipLaunchKernelGGL(sample_full_pick_kernel, dim3(1), dim3(kSampleThreads), 0, s, keys, ids, k, temp, top_p, u, out);
}

void launch_sample_topk(const float* logits, int64_t V, int top_k, float temp, float top_p, float u, int32_t* out, hipStream_t s) {
    const int k = int(std::min<int64_t>(top_k, V));
    // out[1] is the fallback flag the usual path leaves for the radix form
    hipLaunchKernelGGL(sample_topk_fast_kernel, dim3(1), dim3(kSampleThreads), 0, s, logits, int(V), k, temp, top_p, u, out, out + 1);
    hipLaunchKernelGGL(sample_topk_kernel, dim3(1), dim3(kSampleThreads), 0, s, logits, int(V), k, temp, top_p, u, out, out + 1);
}

}  // namespace hero
