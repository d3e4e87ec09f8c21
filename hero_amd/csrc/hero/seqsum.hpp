// seqsum.hpp -- the sequential fp32 sum of n >= 0 terms,
//     s = 0; for i in 0..n-1: s = fl(s + p[i])
// computed by a workgroup of 1024 or 256 lanes, bit-identical to the loop.
//
// The reference's RMSNorm and L2 norms sum squares in index order
// (nm/src/core.hpp:496-500) and its softmax sums exponentials in index order
// (nm/src/components.hpp:132-141). One lane doing that loop costs n dependent
// adds (about 30 microseconds for n = 4096). This computes the same value in
// parallel, using what makes a sum of non-negative terms tractable:
//
//  * While the running sum s stays in one binade [2^e, 2^(e+1)) (e = -126
//    stands for every s below 2^-125), every addition rounds to the same grid
//    u = 2^(e-23). Unless p/u lies exactly halfway between two integers, the
//    step s -> fl(s + p) adds c = round(p/u) grid units whatever s is.
//  * The binade changes only when s crosses a power of two, a few dozen times
//    at most for non-negative terms. The partial sums are speculated (an fp32
//    prefix scan); element i is "serial" when the speculated interval
//    [S_(i-1) (1 - m), S_i (1 + m)], m = 2^-14, touches a power of two, when
//    p/u is a tie, or when p is negative, NaN or huge. Every lane decides
//    from values its neighbours see bit for bit (a lane's last "after" sum is
//    the next lane's "before" sum), so all elements of a run between two
//    serial elements share one speculated binade e.
//  * A run of non-serial elements therefore adds C = sum of its c's units,
//    i.e. s -> s + C*2^(e-23), which is one exact fp32 addition as long as
//    the result stays in binade e. The C's come from a plain prefix sum.
//  * One wave walks the serial elements in order: s += (the run before the
//    element), then s = fl(s + p) for the element itself. For every non-empty
//    run it checks that s is in binade e before and after it. A failed check
//    or more serial elements than the table holds makes the walk run the
//    plain loop instead, so the result is exact in every case; the fp32
//    partial sums stay far closer than m to the speculated ones except in
//    contrived inputs, so that fallback is rare.
//
// Lane t holds elements PT*t .. PT*t+PT-1 (PT = 4096 / lanes). The cross-lane
// steps are wave shuffles plus exchanges of per-wave totals through shared
// memory; the host emulation at the end runs the same per-lane functions in
// the same order.
#pragma once
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "hero/fp16.hpp"

namespace hero {
namespace seqsum {

// Workgroups of 1024 lanes (4 elements each) or 256 lanes (16 each); both sum
// up to 4096 terms. The 1024-lane form is the faster; the 256-lane form runs
// inside other kernels' workgroups.
constexpr int kThreads = 1024;  // the default workgroup
constexpr int kWaveSize = 64;
constexpr int kMaxWaves = 16;
constexpr int kMaxN = 4096;
constexpr int kMaxSerial = 512;
constexpr int kWaves = kThreads / kWaveSize;  // of the default workgroup
constexpr float kMarginLo = 1.0f - 1.0f / 16384.0f;
constexpr float kMarginHi = 1.0f + 1.0f / 16384.0f;

// binade exponent of a value >= 0 as the fp32 grid sees it: ulp(s) = 2^(e-23);
// every s below 2^-125 shares the finest grid 2^-149, i.e. e = -126.
__host__ __device__ inline int binade_f32(float s) {
    const int be = int((f32_bits(s) >> 23) & 0xFF);
    return be <= 1 ? -126 : be - 127;
}

struct Shared {
    float wsum[kMaxWaves];                 // wave totals of the speculation scan
    uint32_t wc[kMaxWaves], wn[kMaxWaves]; // wave totals of the increment and serial-count scans
    int32_t ser_idx[kMaxSerial];     // index of serial element r
    float ser_val[kMaxSerial];       // its term
    uint32_t ser_cx[kMaxSerial];     // increments of all non-serial elements before it (mod 2^32)
    int32_t ser_e[kMaxSerial];       // binade of the run that follows it
    uint32_t c_total;
    int32_t nser;
    int32_t fell_back;  // 1 if the walk ran the plain loop
    float result;
};

template <int PT>  // elements per lane
struct Lane {     // what a lane keeps in registers between steps
    static constexpr int kPerThread = PT;
    float v[PT];
    uint32_t c[PT];       // increment of each non-serial element, in its run's units
    int32_t e_after[PT];  // binade of the speculated sum after each element
    uint32_t serial;      // bit k: element k is serial
    uint32_t csum, cnt;   // the lane's increment total and serial count
};

template <int PT>
__host__ __device__ inline void lane_load(const float* p, int n, int i0, Lane<PT>& L) {
    if (i0 + PT <= n) {
#pragma unroll
        for (int k = 0; k < PT; k += 4) {
            const float4 q = *reinterpret_cast<const float4*>(p + i0 + k);
            L.v[k] = q.x, L.v[k + 1] = q.y, L.v[k + 2] = q.z, L.v[k + 3] = q.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < PT; ++k) L.v[k] = i0 + k < n ? p[i0 + k] : 0.f;
    }
}

template <int PT>
__host__ __device__ inline float lane_sum(const Lane<PT>& L) {
    float d = L.v[0];
#pragma unroll
    for (int k = 1; k < PT; ++k) d += L.v[k];
    return d;
}

// pre: speculated sum of everything before the lane's first element; next:
// the same value as the following lane sees it (its `pre`)
template <int PT>
__host__ __device__ inline void lane_classify(Lane<PT>& L, int i0, int n, float pre, float next) {
    constexpr int kPerThread = PT;
    float S[kPerThread + 1];
    S[0] = pre;
#pragma unroll
    for (int k = 0; k + 1 < kPerThread; ++k) S[k + 1] = S[k] + L.v[k];
    S[kPerThread] = next;
    uint32_t serial = 0, csum = 0, cnt = 0;
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) {  // straight-line: no early exits
        L.e_after[k] = binade_f32(S[k + 1]);
        const bool in = i0 + k < n;
        const float v = L.v[k];
        const float hi = S[k + 1] * kMarginHi;
        const int e = binade_f32(S[k]);
        // v * 2^(23-e): exact for every term that can stay in the binade
        const float P = ldexpf(v, 23 - e);
        const float m = floorf(P);
        const float f = P - m;
        const bool ser = binade_f32(S[k] * kMarginLo) != binade_f32(hi) || !(v >= 0.f) || !(v <= 3.0e38f) || !(hi <= 3.0e38f) ||
                         !(P < 67108864.f) || f == 0.5f;
        const uint32_t ck = in && !ser ? uint32_t(m) + (f > 0.5f ? 1u : 0u) : 0u;
        L.c[k] = ck;
        csum += ck;
        serial |= (in && ser ? 1u : 0u) << k;
        cnt += in && ser ? 1u : 0u;
    }
    L.serial = serial;
    L.csum = csum;
    L.cnt = cnt;
}

// cx, r: increments and serial elements before the lane's first element.
// Writes the table entries of the lane's serial elements, and the totals if
// the lane holds element n-1.
template <int PT>
__host__ __device__ inline void lane_emit(const Lane<PT>& L, int i0, int n, uint32_t cx, uint32_t r, Shared& sm) {
    constexpr int kPerThread = PT;
    // straight-line: c[k] is 0 for serial and out-of-range elements, and
    // serial bits are only set in range
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) {
        const bool ser = (L.serial >> k) & 1u;
        if (ser && r < uint32_t(kMaxSerial)) {
            sm.ser_idx[r] = i0 + k;
            sm.ser_val[r] = L.v[k];
            sm.ser_cx[r] = cx;
            sm.ser_e[r] = L.e_after[k];
        }
        r += ser ? 1u : 0u;
        cx += L.c[k];
    }
    if (i0 < n && n <= i0 + kPerThread) {
        sm.nser = int32_t(r);
        sm.c_total = cx;
    }
}

__host__ __device__ inline float serial_loop(const float* p, int n) {
    float s = 0.f;
    for (int i = 0; i < n; ++i) s += p[i];
    return s;
}

// step r of the walk: the run before serial element r (for r == nser, the
// final run), then element r itself
struct Step {
    float a;        // the run's exact contribution C * 2^(e-23)
    float val;      // the serial term (0 for r == nser)
    int32_t e;      // the run's binade
    int32_t flags;  // bit 0: the run is non-empty, bit 1: its C is too large
};

__host__ __device__ inline Step walk_entry(const Shared& sm, int r, int n) {
    const int nser = sm.nser;
    const int idx = r < nser ? sm.ser_idx[r] : n;
    const int idx_prev = r > 0 ? sm.ser_idx[r - 1] : -1;
    const uint32_t cx = r < nser ? sm.ser_cx[r] : sm.c_total;
    const uint32_t cx_prev = r > 0 ? sm.ser_cx[r - 1] : 0u;
    Step st;
    st.e = r > 0 ? sm.ser_e[r - 1] : -126;
    const uint32_t C = cx - cx_prev;
    const bool nonempty = idx > idx_prev + 1;
    const bool big = C >= (1u << 24);
    st.a = nonempty && !big ? ldexpf(float(C), st.e - 23) : 0.f;
    st.val = r < nser ? sm.ser_val[r] : 0.f;
    st.flags = (nonempty ? 1 : 0) | (big ? 2 : 0);
    return st;
}

// the dependent chain is s -> s + a -> s + val (a = 0 for an empty run, val =
// 0 after the final run: adding +0 to s >= 0 leaves it unchanged); the checks
// only read it
__host__ __device__ inline void walk_apply(float& s, bool& ok, float a, float val, int32_t e, int32_t flags) {
    const float s0 = s;
    const float s1 = s0 + a;
    const bool good = !(flags & 2) && s0 >= 0.f && binade_f32(s0) == e && binade_f32(s1) == e;
    ok = ok && (!(flags & 1) || good);
    s = s1 + val;
}

// ---- the whole sum on the device: NT lanes (the whole workgroup), p in shared
// memory (16-byte aligned), 0 <= n <= 4096 ---------------------------------------------
template <int NT = kThreads>
__device__ inline float sum_nonneg(const float* p, int n, Shared& sm) {
    static_assert(NT == 256 || NT == 1024, "256 or 1024 lanes");
    constexpr int kPerThread = kMaxN / NT, kWaves = NT / kWaveSize;
    if (n <= 0) return 0.f;
    const int tid = int(threadIdx.x), lane = tid & (kWaveSize - 1), w = tid / kWaveSize;
    const int i0 = tid * kPerThread;
    Lane<kPerThread> L;
    lane_load(p, n, i0, L);

    // speculation: inclusive scan of lane sums inside the wave, then of the
    // wave totals (every wave scans all of them in its lanes 0..15)
    float d = lane_sum(L);
#pragma unroll
    for (int off = 1; off < kWaveSize; off <<= 1) {
        const float y = __shfl_up(d, off, kWaveSize);
        if (lane >= off) d += y;
    }
    if (lane == kWaveSize - 1) sm.wsum[w] = d;
    __syncthreads();
    float ws = lane < kWaves ? sm.wsum[lane] : 0.f;
#pragma unroll
    for (int off = 1; off < kWaves; off <<= 1) {
        const float y = __shfl_up(ws, off, kWaveSize);
        if (lane >= off) ws += y;
    }
    float P = __shfl(ws, w > 0 ? w - 1 : 0, kWaveSize);
    if (w == 0) P = 0.f;
    const float P_next = __shfl(ws, w, kWaveSize);  // the next wave's P
    float excl = __shfl_up(d, 1, kWaveSize);
    if (lane == 0) excl = 0.f;
    const float pre = P + excl;
    float next = __shfl_down(pre, 1, kWaveSize);
    if (lane == kWaveSize - 1) next = P_next + 0.f;  // what the next wave's lane 0 computes

    lane_classify(L, i0, n, pre, next);

    // prefix sums of the increments (mod 2^32) and of the serial counts
    uint32_t c = L.csum, m = L.cnt;
#pragma unroll
    for (int off = 1; off < kWaveSize; off <<= 1) {
        const uint32_t yc = __shfl_up(c, off, kWaveSize), ym = __shfl_up(m, off, kWaveSize);
        if (lane >= off) c += yc, m += ym;
    }
    if (lane == kWaveSize - 1) {
        sm.wc[w] = c;
        sm.wn[w] = m;
    }
    __syncthreads();
    uint32_t bc = 0, bm = 0;
    for (int u = 0; u < w; ++u) bc += sm.wc[u], bm += sm.wn[u];
    lane_emit(L, i0, n, bc + c - L.csum, bm + m - L.cnt, sm);
    __syncthreads();

    // the walk: wave 0; lane l prepares step base+l, then the steps run in
    // order, reading each lane's values with readlane
    if (w == 0) {
        const int nser = sm.nser;
        bool ok = nser <= kMaxSerial;
        float s = 0.f;
        for (int base = 0; ok && base <= nser; base += kWaveSize) {
            const int r = base + lane;
            Step st{0.f, 0.f, 0, 0};
            if (r <= nser) st = walk_entry(sm, r, n);
            const int cnt = min(kWaveSize, nser + 1 - base);
            const int ia = int(f32_bits(st.a)), iv = int(f32_bits(st.val));
            int l = 0;
            for (; l + 8 <= cnt; l += 8) {  // the step data of 8 steps first, then the chain
                float a[8], v[8];
                int32_t e[8], f[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    a[u] = bits_f32(uint32_t(__builtin_amdgcn_readlane(ia, l + u)));
                    v[u] = bits_f32(uint32_t(__builtin_amdgcn_readlane(iv, l + u)));
                    e[u] = __builtin_amdgcn_readlane(st.e, l + u);
                    f[u] = __builtin_amdgcn_readlane(st.flags, l + u);
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) walk_apply(s, ok, a[u], v[u], e[u], f[u]);
            }
            for (; l < cnt; ++l)
                walk_apply(s, ok, bits_f32(uint32_t(__builtin_amdgcn_readlane(ia, l))), bits_f32(uint32_t(__builtin_amdgcn_readlane(iv, l))),
                           __builtin_amdgcn_readlane(st.e, l), __builtin_amdgcn_readlane(st.flags, l));
        }
        if (!ok) s = serial_loop(p, n);
        if (lane == 0) {
            sm.result = s;
            sm.fell_back = ok ? 0 : 1;
        }
    }
    __syncthreads();
    return sm.result;
}

// ---- the same steps on the host, lane after lane, in the device's order -------------
template <int NT = kThreads>
inline float sum_nonneg_host(const float* p, int n, Shared& sm) {
    constexpr int kThreads = NT, kPerThread = kMaxN / NT, kWaves = NT / kWaveSize;
    if (n <= 0) return 0.f;
    static Lane<kPerThread> L[kThreads];
    static float d[kThreads], pre[kThreads], next[kThreads];
    static uint32_t c[kThreads], m[kThreads];
    for (int t = 0; t < kThreads; ++t) {
        lane_load(p, n, t * kPerThread, L[t]);
        d[t] = lane_sum(L[t]);
    }
    for (int w = 0; w < kWaves; ++w) {
        float* x = d + w * kWaveSize;
        for (int off = 1; off < kWaveSize; off <<= 1) {
            float y[kWaveSize];
            for (int l = 0; l < kWaveSize; ++l) y[l] = x[l];
            for (int l = off; l < kWaveSize; ++l) x[l] += y[l - off];
        }
        sm.wsum[w] = x[kWaveSize - 1];
    }
    float ws[kWaves];
    for (int u = 0; u < kWaves; ++u) ws[u] = sm.wsum[u];
    for (int off = 1; off < kWaves; off <<= 1) {
        float y[kWaves];
        for (int l = 0; l < kWaves; ++l) y[l] = ws[l];
        for (int l = off; l < kWaves; ++l) ws[l] += y[l - off];
    }
    for (int w = 0; w < kWaves; ++w) {
        const float P = w > 0 ? ws[w - 1] : 0.f;
        for (int l = 0; l < kWaveSize; ++l) pre[w * kWaveSize + l] = P + (l > 0 ? d[w * kWaveSize + l - 1] : 0.f);
        for (int l = 0; l + 1 < kWaveSize; ++l) next[w * kWaveSize + l] = pre[w * kWaveSize + l + 1];
        next[w * kWaveSize + kWaveSize - 1] = ws[w] + 0.f;
    }
    for (int t = 0; t < kThreads; ++t) {
        lane_classify(L[t], t * kPerThread, n, pre[t], next[t]);
        c[t] = L[t].csum;
        m[t] = L[t].cnt;
    }
    for (int w = 0; w < kWaves; ++w) {
        uint32_t* xc = c + w * kWaveSize;
        uint32_t* xm = m + w * kWaveSize;
        for (int l = 1; l < kWaveSize; ++l) xc[l] += xc[l - 1], xm[l] += xm[l - 1];
        sm.wc[w] = xc[kWaveSize - 1];
        sm.wn[w] = xm[kWaveSize - 1];
    }
    for (int t = 0; t < kThreads; ++t) {
        const int w = t / kWaveSize;
        uint32_t bc = 0, bm = 0;
        for (int u = 0; u < w; ++u) bc += sm.wc[u], bm += sm.wn[u];
        lane_emit(L[t], t * kPerThread, n, bc + c[t] - L[t].csum, bm + m[t] - L[t].cnt, sm);
    }
    const int nser = sm.nser;
    bool ok = nser <= kMaxSerial;
    float s = 0.f;
    for (int r = 0; ok && r <= nser; ++r) {
        const Step st = walk_entry(sm, r, n);
        walk_apply(s, ok, st.a, st.val, st.e, st.flags);
    }
    if (!ok) s = serial_loop(p, n);
    sm.result = s;
    sm.fell_back = ok ? 0 : 1;
    return s;
}

}  // namespace seqsum
}  // namespace hero
