// seqsum.hpp -- the sequential fp32 sum of n >= 0 terms,
//     s = 0; for i in 0..n-1: s = fl(s + p[i])
// computed by a 1024-lane workgroup, bit-identical to the loop.
//
// The reference's RMSNorm and L2 norms sum squares in index order
// (nm/src/core.hpp:496-500) and its softmax sums exponentials in index order
// (nm/src/components.hpp:132-141). One lane doing that loop costs n dependent
// adds (about 30 microseconds for n = 4096). This computes the same value in
// parallel, using what makes a sum of non-negative terms tractable:
//
//  * While the running sum s stays in one binade [2^e, 2^(e+1)), every
//    addition rounds to the same grid u = 2^(e-23). In units of u, with
//    P = p/u = m + f (m integer, 0 <= f < 1), the step is
//        S -> S + m + [f > 1/2] + [f == 1/2] * ((S + m) & 1)
//    (round half to even). Every such step, and every composition of them,
//    has the form  S -> S + c + t*((S + d) & 1)  with t, d in {0,1}: after a
//    tie the parity no longer depends on S, so the family is closed under
//    composition and a scan can compose a whole run of steps.
//  * The binade changes only when s crosses a power of two, a few dozen times
//    at most for non-negative terms. The partial sums are speculated in fp64
//    (a prefix scan); element i is "serial" when the speculated interval
//    [S_(i-1) (1 - m), S_i (1 + m)], m = 2^-14, touches a power of two. The
//    fp32 partial sums stay far closer than m to the fp64 ones except in
//    contrived cases, which the walk below detects. Every lane decides from
//    values its neighbours see bit for bit (a lane's last "after" sum is the
//    next lane's "before" sum), so all elements of a run between two serial
//    elements share one speculated binade.
//  * Non-serial elements are composed per run (a segmented scan); serial
//    elements get real fp32 additions in a walk by one wave, which checks
//    before each run that s is in the binade the run was composed for and
//    after it that the result stayed below that binade's top. A failed check,
//    a non-finite term or more serial elements than the table holds makes the
//    walk run the plain loop instead, so the result is exact in every case.
//
// Lane t holds elements 4t .. 4t+3. The cross-lane steps are wave shuffles
// plus one exchange of per-wave aggregates through shared memory; the host
// emulation at the end runs the same per-lane functions with the same
// combination order.
#pragma once
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "hero/fp16.hpp"

namespace hero {
namespace seqsum {

constexpr int kThreads = 1024;
constexpr int kWaveSize = 64;
constexpr int kWaves = kThreads / kWaveSize;
constexpr int kPerThread = 4;
constexpr int kMaxN = kThreads * kPerThread;  // 4096
constexpr int kMaxSerial = 512;
constexpr double kMargin = 1.0 / 16384.0;

// ---- transfer functions S -> S + c + t*((S + d) & 1), packed in 32 bits ----------
// bit 0: t, bit 1: d, bits 2..31: c, saturated at kCap (any c >= 2^24 already
// fails the walk's range check, so saturation never changes a result)
constexpr uint32_t kIdentity = 0;
constexpr uint32_t kCap = 1u << 28;

__host__ __device__ inline uint32_t fn_pack(uint32_t c, uint32_t t, uint32_t d) { return ((c < kCap ? c : kCap) << 2) | (d << 1) | t; }
// x first, then y
__host__ __device__ inline uint32_t fn_then(uint32_t x, uint32_t y) {
    const uint32_t xc = x >> 2, yc = y >> 2, xt = x & 1u, yt = y & 1u, xd = (x >> 1) & 1u, yd = (y >> 1) & 1u;
    const uint32_t c = xc + yc;  // <= 2^29
    if (!yt) return fn_pack(c, xt, xd);
    if (!xt) return fn_pack(c, 1u, (xc + yd) & 1u);
    return fn_pack(c + ((xc - xd + yd) & 1u), 1u, xd);
}
__host__ __device__ inline uint32_t fn_apply(uint32_t f, uint32_t S) { return S + (f >> 2) + ((f & (S + ((f >> 1) & 1u))) & 1u); }

// ---- segment descriptors of the scan -------------------------------------------------
// bit 0: the segment holds a serial element; bits 1..9: binade code (e + 256,
// 0 = no open run) of the run open at its end; bits 10..: serial element count
__host__ __device__ inline uint32_t seg_pack(uint32_t sep, uint32_t ecode, uint32_t cnt) { return sep | (ecode << 1) | (cnt << 10); }
__host__ __device__ inline uint32_t seg_ecode(uint32_t g) { return (g >> 1) & 0x1FFu; }
// (bf, bg) := (af, ag) followed by (bf, bg)
__host__ __device__ inline void combine(uint32_t af, uint32_t ag, uint32_t& bf, uint32_t& bg) {
    const uint32_t bsep = bg & 1u, bec = seg_ecode(bg);
    const uint32_t f = bsep ? bf : fn_then(af, bf);
    const uint32_t ec = (bsep || bec) ? bec : seg_ecode(ag);
    bg = ((ag | bg) & 1u) | (ec << 1) | (((ag >> 10) + (bg >> 10)) << 10);
    bf = f;
}

// binade exponent of a value >= 0 as the fp32 grid sees it: ulp(s) = 2^(e-23);
// every s below 2^-125 shares the finest grid 2^-149, i.e. e = -126.
__host__ __device__ inline int binade_f32(float s) {
    const int be = int((f32_bits(s) >> 23) & 0xFF);
    return be <= 1 ? -126 : be - 127;
}
__host__ __device__ inline float pow2f(int k) { return bits_f32(uint32_t(127 + k) << 23); }  // -126 <= k <= 127

// x * 2^k for -252 <= k <= 254 as two scalings by normal powers of two. The
// product is exact whenever the result is representable (subnormal included)
// and the first factor moves x toward the result's exponent range.
__host__ __device__ inline float mul_pow2(float x, int k) {
    if (k > 127) return x * pow2f(127) * pow2f(k - 127);
    if (k < -126) return x * pow2f(-126) * pow2f(k + 126);
    return x * pow2f(k);
}

// one in-binade step for term p when the running sum is in binade e
__host__ __device__ inline uint32_t step_fn(float p, int e) {
    // an exact power-of-two scale for every term that can stay in the binade;
    // larger ones saturate (their run fails the walk's check)
    const float P = mul_pow2(p, 23 - e);
    if (!(P < 67108864.f)) return fn_pack(kCap, 0u, 0u);
    const float m = floorf(P);
    const float f = P - m;
    const uint32_t mi = uint32_t(m);
    if (f == 0.5f) return fn_pack(mi, 1u, mi & 1u);
    return fn_pack(mi + (f > 0.5f ? 1u : 0u), 0u, 0u);
}

struct Shared {
    double wsum[kWaves];                // wave totals of the fp64 scan
    uint32_t wfn[kWaves], wseg[kWaves]; // wave aggregates of the segmented scan
    uint32_t run_fn[kMaxSerial + 1];    // run ending just before serial element r; [nser] is the final run
    uint16_t run_e[kMaxSerial + 1];     // its binade code
    uint16_t ser_idx[kMaxSerial];
    float ser_val[kMaxSerial];
    int32_t nser;
    int32_t fell_back;  // 1 if the walk ran the plain loop
    float result;
};

struct Lane {  // what a lane keeps in registers between steps
    float v[kPerThread];
    uint32_t sf[kPerThread];     // step function of each non-serial element
    uint32_t ecode[kPerThread];  // its binade code
    uint32_t serial;             // bit k: element k is serial
    uint32_t agg_f, agg_g;       // the lane's aggregate for the segmented scan
};

__host__ __device__ inline void lane_load(const float* p, int n, int i0, Lane& L) {
    if (i0 + kPerThread <= n) {
        const float4 q = *reinterpret_cast<const float4*>(p + i0);
        L.v[0] = q.x, L.v[1] = q.y, L.v[2] = q.z, L.v[3] = q.w;
    } else {
#pragma unroll
        for (int k = 0; k < kPerThread; ++k) L.v[k] = i0 + k < n ? p[i0 + k] : 0.f;
    }
}

__host__ __device__ inline double lane_dsum(const Lane& L) {
    double d = double(L.v[0]);
#pragma unroll
    for (int k = 1; k < kPerThread; ++k) d += double(L.v[k]);
    return d;
}

// pre: fp64 sum of everything before the lane's first element; next: the
// same value as the following lane sees it (its `pre`)
__host__ __device__ inline void lane_classify(Lane& L, int i0, int n, double pre, double next) {
    double S[kPerThread + 1];
    S[0] = pre;
#pragma unroll
    for (int k = 0; k + 1 < kPerThread; ++k) S[k + 1] = S[k] + double(L.v[k]);
    S[kPerThread] = next;
    uint32_t serial = 0, tail = kIdentity, tail_e = 0, cnt = 0;
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) {
        L.sf[k] = kIdentity;
        L.ecode[k] = 0;
        if (i0 + k >= n) continue;
        const float lo = float(S[k] * (1.0 - kMargin)), hi = float(S[k + 1] * (1.0 + kMargin));
        // negative, NaN or huge terms and non-finite sums are serial too: the
        // walk then falls back. A zero sum is on the finest grid (e = -126).
        if (binade_f32(lo) != binade_f32(hi) || !(L.v[k] >= 0.f) || !(L.v[k] <= 3.0e38f) || !(hi <= 3.0e38f)) {
            serial |= 1u << k;
            ++cnt;
            tail = kIdentity;
            tail_e = 0;
        } else {
            const int e = binade_f32(float(S[k]));
            L.ecode[k] = uint32_t(e + 256);
            L.sf[k] = step_fn(L.v[k], e);
            tail = fn_then(tail, L.sf[k]);
            tail_e = L.ecode[k];
        }
    }
    L.serial = serial;
    L.agg_f = tail;
    L.agg_g = seg_pack(cnt > 0 ? 1u : 0u, tail_e, cnt);
}

// (xf, xg): everything before the lane, combined; writes the runs that end at
// the lane's serial elements, and the final run if the lane holds element n-1
__host__ __device__ inline void lane_emit(const Lane& L, int i0, int n, uint32_t xf, uint32_t xg, Shared& sm) {
    uint32_t r = xg >> 10, run = xf, ec = seg_ecode(xg);
#pragma unroll
    for (int k = 0; k < kPerThread; ++k) {
        const int i = i0 + k;
        if (i >= n) break;
        if ((L.serial >> k) & 1u) {
            if (r < uint32_t(kMaxSerial)) {
                sm.run_fn[r] = run;
                sm.run_e[r] = uint16_t(ec);
                sm.ser_idx[r] = uint16_t(i);
                sm.ser_val[r] = L.v[k];
            }
            ++r;
            run = kIdentity;
            ec = 0;
        } else {
            run = fn_then(run, L.sf[k]);
            ec = L.ecode[k];
        }
    }
    if (i0 < n && n <= i0 + kPerThread) {
        sm.nser = int32_t(r);
        if (r <= uint32_t(kMaxSerial)) {
            sm.run_fn[r] = run;
            sm.run_e[r] = uint16_t(ec);
        }
    }
}

__host__ __device__ inline float serial_loop(const float* p, int n) {
    float s = 0.f;
    for (int i = 0; i < n; ++i) s += p[i];
    return s;
}

// the walk over serial elements and runs, in order; the table entries of
// step r+1 are read while step r computes. Written without `break`: with an
// early exit from this loop, hipcc (ROCm 7.2) kept the binade code of the
// next run in a scalar register that it reused as a temporary on the
// non-empty-run path, so every later run saw a stale binade.
__host__ __device__ inline void walk(const float* p, int n, Shared& sm, bool writer) {
    const int nser = sm.nser;
    bool ok = nser <= kMaxSerial;
    float s = 0.f;
    int prev = -1;
    int j = ok && nser > 0 ? int(sm.ser_idx[0]) : n;
    uint32_t fn = ok ? sm.run_fn[0] : kIdentity, ec = ok ? sm.run_e[0] : 0u;
    float val = ok && nser > 0 ? sm.ser_val[0] : 0.f;
    for (int r = 0; ok && r <= nser; ++r) {
        int jn = n;
        uint32_t fnn = kIdentity, ecn = 0;
        float valn = 0.f;
        if (r < nser) {
            fnn = sm.run_fn[r + 1];
            ecn = sm.run_e[r + 1];
            if (r + 1 < nser) {
                jn = int(sm.ser_idx[r + 1]);
                valn = sm.ser_val[r + 1];
            }
        }
        if (j > prev + 1) {  // a non-empty run: elements prev+1 .. j-1
            const int e = int(ec) - 256;
            ok = ec != 0 && s >= 0.f && s <= 3.0e38f && binade_f32(s) == e;
            // S is an exact integer below 2^24 when ok
            const uint32_t S = ok ? uint32_t(mul_pow2(s, 23 - e)) : 0u;
            const uint32_t S2 = fn_apply(fn, S);
            ok = ok && S2 < (1u << 24);
            if (ok) s = mul_pow2(float(S2), e - 23);
        }
        if (ok && r < nser) s = s + val;
        prev = j;
        j = jn;
        fn = fnn;
        ec = ecn;
        val = valn;
    }
    if (!ok) s = serial_loop(p, n);
    if (writer) {
        sm.result = s;
        sm.fell_back = ok ? 0 : 1;
    }
}

// ---- the whole sum on the device: 1024 lanes, p in shared memory (16-byte
// aligned), 0 <= n <= 4096 ---------------------------------------------------------
__device__ inline float sum_nonneg(const float* p, int n, Shared& sm) {
    if (n <= 0) return 0.f;
    const int tid = int(threadIdx.x), lane = tid & (kWaveSize - 1), w = tid / kWaveSize;
    const int i0 = tid * kPerThread;
    Lane L;
    lane_load(p, n, i0, L);

    // fp64 inclusive scan: Hillis-Steele inside the wave, then wave totals
    double d = lane_dsum(L);
#pragma unroll
    for (int off = 1; off < kWaveSize; off <<= 1) {
        const double y = __shfl_up(d, off, kWaveSize);
        if (lane >= off) d += y;
    }
    if (lane == kWaveSize - 1) sm.wsum[w] = d;
    __syncthreads();
    double P = 0.0;
    for (int u = 0; u < w; ++u) P += sm.wsum[u];
    double excl = __shfl_up(d, 1, kWaveSize);
    if (lane == 0) excl = 0.0;
    const double pre = P + excl;
    double next = __shfl_down(pre, 1, kWaveSize);
    if (lane == kWaveSize - 1) next = P + sm.wsum[w];  // the next wave's P, summed in the same order

    lane_classify(L, i0, n, pre, next);

    // segmented inclusive scan inside the wave
    uint32_t f = L.agg_f, g = L.agg_g;
#pragma unroll
    for (int off = 1; off < kWaveSize; off <<= 1) {
        const uint32_t pf = __shfl_up(f, off, kWaveSize), pg = __shfl_up(g, off, kWaveSize);
        if (lane >= off) combine(pf, pg, f, g);
    }
    if (lane == kWaveSize - 1) {
        sm.wfn[w] = f;
        sm.wseg[w] = g;
    }
    __syncthreads();
    // every wave scans the wave aggregates in its lanes 0..kWaves-1
    uint32_t wf = kIdentity, wg = 0;
    if (lane < kWaves) {
        wf = sm.wfn[lane];
        wg = sm.wseg[lane];
    }
#pragma unroll
    for (int off = 1; off < kWaves; off <<= 1) {
        const uint32_t pf = __shfl_up(wf, off, kWaveSize), pg = __shfl_up(wg, off, kWaveSize);
        if (lane >= off) combine(pf, pg, wf, wg);
    }
    uint32_t cf = __shfl(wf, w > 0 ? w - 1 : 0, kWaveSize), cg = __shfl(wg, w > 0 ? w - 1 : 0, kWaveSize);
    if (w == 0) cf = kIdentity, cg = 0;
    uint32_t ef = __shfl_up(f, 1, kWaveSize), eg = __shfl_up(g, 1, kWaveSize);
    if (lane == 0) ef = kIdentity, eg = 0;
    combine(cf, cg, ef, eg);
    lane_emit(L, i0, n, ef, eg, sm);
    __syncthreads();
    if (w == 0) walk(p, n, sm, lane == 0);
    __syncthreads();
    return sm.result;
}

// ---- the same steps on the host, lane after lane, in the device's order -------------
inline float sum_nonneg_host(const float* p, int n, Shared& sm) {
    if (n <= 0) return 0.f;
    static Lane L[kThreads];
    static double d[kThreads], pre[kThreads], next[kThreads];
    static uint32_t f[kThreads], g[kThreads];
    for (int t = 0; t < kThreads; ++t) {
        lane_load(p, n, t * kPerThread, L[t]);
        d[t] = lane_dsum(L[t]);
    }
    for (int w = 0; w < kWaves; ++w) {
        double* x = d + w * kWaveSize;
        for (int off = 1; off < kWaveSize; off <<= 1) {
            double y[kWaveSize];
            for (int l = 0; l < kWaveSize; ++l) y[l] = x[l];
            for (int l = off; l < kWaveSize; ++l) x[l] += y[l - off];
        }
        sm.wsum[w] = x[kWaveSize - 1];
    }
    for (int w = 0; w < kWaves; ++w) {
        double P = 0.0;
        for (int u = 0; u < w; ++u) P += sm.wsum[u];
        for (int l = 0; l < kWaveSize; ++l) pre[w * kWaveSize + l] = P + (l > 0 ? d[w * kWaveSize + l - 1] : 0.0);
        for (int l = 0; l + 1 < kWaveSize; ++l) next[w * kWaveSize + l] = pre[w * kWaveSize + l + 1];
        next[w * kWaveSize + kWaveSize - 1] = P + sm.wsum[w];
    }
    for (int t = 0; t < kThreads; ++t) {
        lane_classify(L[t], t * kPerThread, n, pre[t], next[t]);
        f[t] = L[t].agg_f;
        g[t] = L[t].agg_g;
    }
    for (int w = 0; w < kWaves; ++w) {
        uint32_t* xf = f + w * kWaveSize;
        uint32_t* xg = g + w * kWaveSize;
        for (int off = 1; off < kWaveSize; off <<= 1) {
            uint32_t yf[kWaveSize], yg[kWaveSize];
            for (int l = 0; l < kWaveSize; ++l) yf[l] = xf[l], yg[l] = xg[l];
            for (int l = off; l < kWaveSize; ++l) combine(yf[l - off], yg[l - off], xf[l], xg[l]);
        }
        sm.wfn[w] = xf[kWaveSize - 1];
        sm.wseg[w] = xg[kWaveSize - 1];
    }
    uint32_t wf[kWaves], wg[kWaves];
    for (int u = 0; u < kWaves; ++u) wf[u] = sm.wfn[u], wg[u] = sm.wseg[u];
    for (int off = 1; off < kWaves; off <<= 1) {
        uint32_t yf[kWaves], yg[kWaves];
        for (int l = 0; l < kWaves; ++l) yf[l] = wf[l], yg[l] = wg[l];
        for (int l = off; l < kWaves; ++l) combine(yf[l - off], yg[l - off], wf[l], wg[l]);
    }
    for (int t = 0; t < kThreads; ++t) {
        const int w = t / kWaveSize, l = t % kWaveSize;
        uint32_t cf = w > 0 ? wf[w - 1] : kIdentity, cg = w > 0 ? wg[w - 1] : 0;
        uint32_t ef = l > 0 ? f[t - 1] : kIdentity, eg = l > 0 ? g[t - 1] : 0;
        combine(cf, cg, ef, eg);
        lane_emit(L[t], t * kPerThread, n, ef, eg, sm);
    }
    walk(p, n, sm, true);
    return sm.result;
}

}  // namespace seqsum
}  // namespace hero
