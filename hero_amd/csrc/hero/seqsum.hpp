// seqsum.hpp -- the sequential fp32 sum of n >= 0 terms,
//     s = 0; for i in 0..n-1: s = fl(s + p[i])
// computed by a workgroup of 1024, 512 or 256 lanes, bit-identical to the loop.
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
// Lane t holds elements PT*t .. PT*t+PT-1 (PT = 4096 / lanes). Every
// cross-lane step inside a wave is a DPP scan (no shared memory); the
// workgroup needs three barriers: one for the wave totals of the speculation,
// one for the wave totals of the serial counts and increments, after which
// every lane writes its serial elements' entries at their places in one table,
// and one for that table. Every wave then runs the walk itself (so the result
// needs no broadcast): its lanes prepare one step each, the dependent chain
// s -> s + a -> s + val runs over the steps with the step data read lane by
// lane, each lane keeps the chain values of its own step, and the binade
// checks of all steps run in parallel afterwards. The host emulation at the
// end runs the same per-lane functions and the same operations in the same
// order.
#pragma once
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <type_traits>

#include "hero/fp16.hpp"

namespace hero {
namespace seqsum {

// Workgroups of 1024, 512 or 256 lanes (4, 8 or 16 elements each); all sum up
// to 4096 terms. The 1024-lane form is the fastest; the smaller forms run
// inside other kernels' workgroups.
constexpr int kThreads = 1024;  // the default workgroup
constexpr int kWaveSize = 64;
constexpr int kMaxWaves = 16;
constexpr int kMaxN = 4096;
constexpr int kMaxSerial = 512;  // table entries
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
    float wsum[kMaxWaves];                  // wave totals of the speculation scan
    uint32_t wc[kMaxWaves], wn[kMaxWaves];  // wave totals of the increments and of the serial counts
    // the serial elements in index order, one 16-byte entry each: x = its
    // index, y = its term (bits), z = increments of the non-serial elements
    // before it (mod 2^32), w = binade of the run that follows it
    uint4 ser[kMaxSerial];
    int32_t fell_back;            // 1 if the last sum ran the plain loop (written by wave 0)
    float result;                 // for callers that broadcast a value of their own
};

template <int PT>  // elements per lane
struct Lane {     // what a lane keeps in registers between steps
    static constexpr int kPerThread = PT;
    float v[PT];
    uint32_t c[PT];       // increment of each non-serial element, in its run's units
    uint32_t be_after[PT];// exponent field of the speculated sum after each element
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
// the same value as the following lane sees it (its `pre`). Terms past the
// end of the data are +0 (the loaders fill them): adding +0 to a sum >= +0
// changes nothing, so they need no special case. An element is serial when
//  * the speculated interval [S (1 - m), S' (1 + m)] has two exponent fields
//    (a binade change; comparing raw fields also splits the two fields that
//    share the finest grid, which only adds serial elements),
//  * the term is not a finite value in [+0, 2^127) or S' (1 + m) is not finite
//    and <= 3e38,
//  * or p / u is a tie.
// A non-serial term is below 2^(e+1) (S' >= p and S' (1 + m) < 2^(e+1)), so
// p / u < 2^24 and its rounding to an integer is exact.
template <int PT>
__host__ __device__ inline void lane_classify(Lane<PT>& L, float pre, float next) {
    float S = pre;
    uint32_t be = f32_bits(S) >> 23;
    uint32_t serial = 0, csum = 0;
#pragma unroll
    for (int k = 0; k < PT; ++k) {  // straight-line: no early exits
        const float v = L.v[k];
        const float S1 = k + 1 < PT ? S + v : next;
        const uint32_t be1 = f32_bits(S1) >> 23;
        const float hi = S1 * kMarginHi;
        const bool cross = (f32_bits(S * kMarginLo) ^ f32_bits(hi)) > 0x007FFFFFu;
        const bool weird = f32_bits(v) >= 0x7F000000u || !(hi <= 3.0e38f);
        // v / u, u = 2^(e-23), e = max(be, 1) - 127: exact while it can stay in the binade
        const float P = ldexpf(v, 150 - int(be > 1u ? be : 1u));
        const float r = rintf(P);
        const bool tie = fabsf(r - P) == 0.5f;
        const bool ser = cross || weird || tie;
        const uint32_t ck = ser ? 0u : uint32_t(r);
        L.c[k] = ck;
        L.be_after[k] = be1;
        csum += ck;
        serial |= (ser ? 1u : 0u) << k;
        S = S1;
        be = be1;
    }
    L.serial = serial;
    L.csum = csum;
    L.cnt = uint32_t(__builtin_popcount(serial));
}

// Writes the table entries of the lane's serial elements at their places in
// the whole table: r = serial elements before the lane (all waves), cx =
// increments of the non-serial elements before the lane (mod 2^32); entries
// past the table's capacity are dropped (the walk then runs the plain loop).
template <int PT>
__host__ __device__ inline void lane_emit(const Lane<PT>& L, int i0, uint32_t cx, uint32_t r, Shared& sm) {
    if (L.serial == 0) return;  // most lanes
    // c[k] is 0 for serial elements
#pragma unroll
    for (int k = 0; k < PT; ++k) {
        const bool ser = (L.serial >> k) & 1u;
        if (ser && r < uint32_t(kMaxSerial)) {
            const uint32_t be = L.be_after[k];
            sm.ser[r] = make_uint4(uint32_t(i0 + k), f32_bits(L.v[k]), cx, uint32_t(int(be > 1u ? be : 1u) - 127));
        }
        r += ser ? 1u : 0u;
        cx += L.c[k];
    }
}

__host__ __device__ inline float serial_loop(const float* p, int n) {
    float s = 0.f;
    for (int i = 0; i < n; ++i) s += p[i];
    return s;
}

// the wave totals of serial counts and increments: the exclusive prefixes of
// wave w and the grand totals
template <int W>
__host__ __device__ inline void wave_prefix(const Shared& sm, int w, uint32_t& nbase, uint32_t& cbase, uint32_t& nser, uint32_t& c_total) {
    nbase = cbase = nser = c_total = 0;
#pragma unroll
    for (int u = 0; u < W; ++u) {
        const uint32_t n = sm.wn[u], c = sm.wc[u];
        nbase += u < w ? n : 0u;
        cbase += u < w ? c : 0u;
        nser += n;
        c_total += c;
    }
}

// step r of the walk: the run before serial element r (for r == nser, the
// final run), then element r itself
struct Step {
    float a;        // the run's exact contribution C * 2^(e-23)
    float val;      // the serial term (0 for r == nser)
    int32_t e;      // the run's binade
    int32_t flags;  // bit 0: the run is non-empty, bit 1: its C is too large
};

// r <= nser <= kMaxSerial
__host__ __device__ inline Step walk_entry(const Shared& sm, uint32_t nser, uint32_t c_total, uint32_t r, int n) {
    const uint4 cur = r < nser ? sm.ser[r] : make_uint4(uint32_t(n), 0u, c_total, 0u);
    const uint4 prev = r > 0 ? sm.ser[r - 1] : make_uint4(0xFFFFFFFFu, 0u, 0u, uint32_t(-126));
    Step st;
    st.e = int32_t(prev.w);
    const uint32_t C = cur.z - prev.z;
    const bool nonempty = int(cur.x) > int(prev.x) + 1;
    const bool big = C >= (1u << 24);
    st.a = nonempty && !big ? ldexpf(float(C), st.e - 23) : 0.f;
    st.val = bits_f32(cur.y);
    st.flags = (nonempty ? 1 : 0) | (big ? 2 : 0);
    return st;
}

// the checks of one step, given the chain value before it (s0) and after its
// run (s1 = s0 + a): a non-empty run must keep s in the binade it was
// classified in
__host__ __device__ inline bool step_ok(const Step& st, float s0, float s1) {
    const bool good = !(st.flags & 2) && s0 >= 0.f && binade_f32(s0) == st.e && binade_f32(s1) == st.e;
    return !(st.flags & 1) || good;
}

// ---- wave-level scans (DPP) --------------------------------------------------------------
// Inclusive scan over the 64 lanes, in this order: inside each row of 16
// lanes, Hillis-Steele steps of 1, 2, 4 and 8 lanes (a lane without a source
// adds +0); then rows 1 and 3 add the last lane of the row before
// (row_bcast:15), then rows 2 and 3 add lane 31 (row_bcast:31); rows without
// a source add +0 in both steps.
template <int CTRL, int ROW_MASK = 0xF>
__device__ inline int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xF, true);
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ inline float dpp_f(float v) {
    return bits_f32(uint32_t(dpp_i<CTRL, ROW_MASK>(int(f32_bits(v)))));
}
__device__ inline float scan_f32(float v) {
    v += dpp_f<0x111>(v);  // row_shr:1
    v += dpp_f<0x112>(v);  // row_shr:2
    v += dpp_f<0x114>(v);  // row_shr:4
    v += dpp_f<0x118>(v);  // row_shr:8
    v += dpp_f<0x142, 0xA>(v);  // row_bcast:15
    v += dpp_f<0x143, 0xC>(v);  // row_bcast:31
    return v;
}
__device__ inline uint32_t scan_u32(uint32_t v) {
    v += uint32_t(dpp_i<0x111>(int(v)));
    v += uint32_t(dpp_i<0x112>(int(v)));
    v += uint32_t(dpp_i<0x114>(int(v)));
    v += uint32_t(dpp_i<0x118>(int(v)));
    v += uint32_t(dpp_i<0x142, 0xA>(int(v)));
    v += uint32_t(dpp_i<0x143, 0xC>(int(v)));
    return v;
}

// ---- the whole sum on the device: NT lanes (the whole workgroup) -----------------------
// L holds the lane's PT terms (elements PT*tid ..); p holds all n terms in
// shared memory, read only by the plain-loop fallback (it runs after three
// barriers, so p may be written right before the call). Every wave returns
// the result; there is no barrier at the end unless the fallback ran.
template <int NT>
__device__ inline float sum_lanes(Lane<kMaxN / NT>& L, const float* p, int n, Shared& sm) {
    static_assert(NT == 256 || NT == 512 || NT == 1024, "256, 512 or 1024 lanes");
    constexpr int W = NT / kWaveSize;
    if (n <= 0) return 0.f;
    const int tid = int(threadIdx.x), lane = tid & (kWaveSize - 1), w = tid / kWaveSize;
    const int i0 = tid * (kMaxN / NT);

    // speculation: the lane sums, scanned in the wave, then the totals of the
    // waves before (left to right)
    const float incl = scan_f32(lane_sum(L));
    if (lane == kWaveSize - 1) sm.wsum[w] = incl;
    const float excl = dpp_f<0x138>(incl);  // wave_shr:1, lane 0 reads +0
    __syncthreads();
    float P = 0.f;
    for (int u = 0; u < w; ++u) P = P + sm.wsum[u];
    const float pre = P + excl;
    const float P_next = P + sm.wsum[w];
    float next = dpp_f<0x130>(pre);  // wave_shl:1: the next lane's pre
    if (lane == kWaveSize - 1) next = P_next + 0.f;                           // what the next wave's lane 0 computes

    lane_classify(L, pre, next);

    // wave-local prefixes of the increments (mod 2^32) and serial counts,
    // then the wave totals' prefixes: every entry goes to its global place
    const uint32_t c = scan_u32(L.csum), m = scan_u32(L.cnt);
    if (lane == kWaveSize - 1) {
        sm.wc[w] = c;
        sm.wn[w] = m;
    }
    __syncthreads();
    uint32_t nbase, cbase, nser, c_total;
    wave_prefix<W>(sm, w, nbase, cbase, nser, c_total);
    lane_emit(L, i0, cbase + c - L.csum, nbase + m - L.cnt, sm);
    __syncthreads();

    // the walk, in every wave: lane l prepares step base + l (steps past the
    // last add +0 twice), then the chain runs 8 steps at a time, the step data
    // of the 8 read from their lanes first, each lane keeping the chain values
    // of its own step for the checks
    bool ok = nser <= uint32_t(kMaxSerial);
    float s = 0.f;
    for (uint32_t base = 0; ok && base <= nser; base += kWaveSize) {
        const uint32_t r = base + uint32_t(lane);
        Step st{0.f, 0.f, 0, 0};
        if (r <= nser) st = walk_entry(sm, nser, c_total, r, n);
        const int cnt = int(min(uint32_t(kWaveSize), nser + 1 - base));
        const int ia = int(f32_bits(st.a)), iv = int(f32_bits(st.val));
        float my0 = 0.f, my1 = 0.f;  // the chain before this lane's step and after its run
        for (int l0 = 0; l0 < cnt; l0 += 8) {
            float av[8], vv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                av[u] = bits_f32(uint32_t(__builtin_amdgcn_readlane(ia, l0 + u)));
                vv[u] = bits_f32(uint32_t(__builtin_amdgcn_readlane(iv, l0 + u)));
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int l = l0 + u;
                const float s1 = s + av[u];
                my0 = lane == l ? s : my0;
                my1 = lane == l ? s1 : my1;
                s = s1 + vv[u];
            }
        }
        const bool bad = lane < cnt && !step_ok(st, my0, my1);
        ok = ok && !__any(bad);
    }
    if (!ok) {  // the same decision in every wave
        s = serial_loop(p, n);
        __syncthreads();
    }
    if (tid == 0) sm.fell_back = ok ? 0 : 1;
    return s;
}

// p: n terms in shared memory (16-byte aligned), 0 <= n <= 4096; written
// before a barrier
template <int NT = kThreads>
__device__ inline float sum_nonneg(const float* p, int n, Shared& sm) {
    Lane<kMaxN / NT> L;
    lane_load(p, n, int(threadIdx.x) * (kMaxN / NT), L);
    return sum_lanes<NT>(L, p, n, sm);
}

// v: the lane's terms (elements PT*tid ..), n = 4096 or fewer with the terms
// past n zero; they are also stored into p (shared memory, 4096 floats) for
// the fallback
template <int NT>
__device__ inline float sum_nonneg_regs(const float (&v)[kMaxN / NT], float* p, int n, Shared& sm) {
    constexpr int PT = kMaxN / NT;
    Lane<PT> L;
#pragma unroll
    for (int k = 0; k < PT; ++k) L.v[k] = v[k];
#pragma unroll
    for (int k = 0; k < PT; k += 4) reinterpret_cast<float4*>(p)[(int(threadIdx.x) * PT + k) / 4] = make_float4(v[k], v[k + 1], v[k + 2], v[k + 3]);
    return sum_lanes<NT>(L, p, n, sm);
}

// ---- the same steps on the host, lane after lane, in the device's order -------------
template <int NT = kThreads>
inline float sum_nonneg_host(const float* p, int n, Shared& sm) {
    constexpr int PT = kMaxN / NT, W = NT / kWaveSize;
    if (n <= 0) return 0.f;
    static Lane<PT> L[NT];
    static float incl[NT], pre[NT], next[NT];
    static uint32_t c[NT], m[NT];
    for (int t = 0; t < NT; ++t) {
        lane_load(p, n, t * PT, L[t]);
        incl[t] = lane_sum(L[t]);
    }
    // the device's wave scan, step by step
    auto scan = [](auto* x) {
        using T = std::remove_reference_t<decltype(x[0])>;
        for (int k = 1; k <= 8; k <<= 1) {
            T y[kWaveSize];
            for (int l = 0; l < kWaveSize; ++l) y[l] = x[l];
            for (int l = 0; l < kWaveSize; ++l) x[l] = x[l] + ((l & 15) >= k ? y[l - k] : T(0));
        }
        {
            T y[kWaveSize];
            for (int l = 0; l < kWaveSize; ++l) y[l] = x[l];
            for (int l = 0; l < kWaveSize; ++l) x[l] = x[l] + ((l >> 4) == 1 ? y[15] : (l >> 4) == 3 ? y[47] : T(0));
        }
        {
            T y[kWaveSize];
            for (int l = 0; l < kWaveSize; ++l) y[l] = x[l];
            for (int l = 0; l < kWaveSize; ++l) x[l] = x[l] + ((l >> 4) >= 2 ? y[31] : T(0));
        }
    };
    for (int w = 0; w < W; ++w) {
        scan(incl + w * kWaveSize);
        sm.wsum[w] = incl[w * kWaveSize + kWaveSize - 1];
    }
    for (int w = 0; w < W; ++w) {
        float P = 0.f;
        for (int u = 0; u < w; ++u) P = P + sm.wsum[u];
        const float P_next = P + sm.wsum[w];
        for (int l = 0; l < kWaveSize; ++l) pre[w * kWaveSize + l] = P + (l > 0 ? incl[w * kWaveSize + l - 1] : 0.f);
        for (int l = 0; l + 1 < kWaveSize; ++l) next[w * kWaveSize + l] = pre[w * kWaveSize + l + 1];
        next[w * kWaveSize + kWaveSize - 1] = P_next + 0.f;
    }
    for (int t = 0; t < NT; ++t) {
        lane_classify(L[t], pre[t], next[t]);
        c[t] = L[t].csum;
        m[t] = L[t].cnt;
    }
    for (int w = 0; w < W; ++w) {
        scan(c + w * kWaveSize);
        scan(m + w * kWaveSize);
        sm.wc[w] = c[w * kWaveSize + kWaveSize - 1];
        sm.wn[w] = m[w * kWaveSize + kWaveSize - 1];
    }
    uint32_t nser = 0, c_total = 0;
    for (int t = 0; t < NT; ++t) {
        uint32_t nbase, cbase;
        wave_prefix<W>(sm, t / kWaveSize, nbase, cbase, nser, c_total);
        lane_emit(L[t], t * PT, cbase + c[t] - L[t].csum, nbase + m[t] - L[t].cnt, sm);
    }
    bool ok = nser <= uint32_t(kMaxSerial);
    float s = 0.f;
    for (uint32_t r = 0; ok && r <= nser; ++r) {
        const Step st = walk_entry(sm, nser, c_total, r, n);
        const float s1 = s + st.a;
        ok = ok && step_ok(st, s, s1);
        s = s1 + st.val;
    }
    if (!ok) s = serial_loop(p, n);
    sm.fell_back = ok ? 0 : 1;
    return s;
}

}  // namespace seqsum
}  // namespace hero
