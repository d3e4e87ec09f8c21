// seqsum.hpp -- the sequential fp32 sum of n >= 0 terms,
//     s = 0; for i in 0..n-1: s = fl(s + p[i])
// computed by a 256-lane workgroup, bit-identical to the loop.
//
// The reference's RMSNorm and L2 norms sum squares in index order
// (nm/src/core.hpp:496-500). One lane doing that loop costs n dependent adds
// (tens of microseconds for n = 4096). This computes the same value in
// parallel, using what makes a sum of non-negative terms tractable:
//
//  * While the running sum s stays in one binade [2^e, 2^(e+1)), every
//    addition rounds to the same grid u = 2^(e-23). In units of u, with
//    P = p/u = m + f (m integer, 0 <= f < 1), the step is
//        S -> S + m + [f > 1/2] + [f == 1/2] * ((S + m) & 1)
//    (round half to even). Every such step, and every composition of them,
//    has the form  S -> S + c + t*((S + d) & 1)  with t in {0,1}: after a tie
//    the parity no longer depends on S, so the family is closed under
//    composition and a scan can compose a whole run of steps.
//  * The binade changes only when s crosses a power of two, a few dozen times
//    at most for non-negative terms. The binade of each partial sum is
//    speculated from an fp64 prefix sum; elements within one position of a
//    speculated crossing are "serial" and get real fp32 additions, the rest
//    are composed per run between serial elements (a segmented scan).
//  * One lane walks serial elements and runs in order. Before a run it checks
//    that s is in the binade the run was composed for, after it that the
//    result stayed below that binade's top. A failed check, a non-finite
//    term, or more serial elements than the table holds makes the lane run
//    the plain loop instead, so the result is exact in every case.
//
// The phases are separated by workgroup barriers; the same code runs on the
// device and in a host emulation (the tests).
#pragma once
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "hero/fp16.hpp"

namespace hero {
namespace seqsum {

constexpr int kThreads = 256;
constexpr int kPerThread = 16;
constexpr int kMaxN = kThreads * kPerThread;  // 4096
constexpr int kMaxSerial = 384;
constexpr int16_t kNoBinade = -1000;

struct Fn {  // S -> S + c + t*((S + d) & 1)
    int64_t c;
    int32_t t, d;
};

__host__ __device__ inline Fn fn_identity() { return Fn{0, 0, 0}; }
// x first, then y
__host__ __device__ inline Fn fn_then(const Fn& x, const Fn& y) {
    if (!y.t) return Fn{x.c + y.c, x.t, x.d};
    if (!x.t) return Fn{x.c + y.c, 1, int32_t((x.c + y.d) & 1)};
    return Fn{x.c + y.c + ((x.c - x.d + y.d) & 1), 1, x.d};
}
__host__ __device__ inline int64_t fn_apply(const Fn& f, int64_t s) { return s + f.c + (f.t ? ((s + f.d) & 1) : 0); }

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
__host__ __device__ inline Fn step_fn(float p, int e) {
    // p * 2^(23-e) is exact: a power-of-two scale below 2^24 for every term
    // that does not leave the binade (those are serial)
    const float P = mul_pow2(p, 23 - e);
    const float m = floorf(P);
    const float f = P - m;
    const int64_t mi = int64_t(m);
    if (f == 0.5f) return Fn{mi, 1, int32_t(mi & 1)};
    return Fn{mi + (f > 0.5f ? 1 : 0), 0, 0};
}

struct Shared {
    double dsum[2][kThreads];  // lane sums, then their inclusive scan (double buffered)
    uint16_t cross[kThreads];  // speculated crossing elements, 16 bits per lane
    uint16_t serial[kThreads];
    // segmented scan: any serial element, function of the open run, its binade, serial count
    int32_t sep[2][kThreads];
    int32_t cnt[2][kThreads];
    int32_t e[2][kThreads];
    Fn fn[2][kThreads];
    Fn run[kMaxSerial + 1];  // run ending just before serial element r; [nser] is the final run
    int16_t run_e[kMaxSerial + 1];
    int16_t ser_idx[kMaxSerial];
    int32_t nser;
    int32_t fell_back;  // 1 if the walk ran the plain loop
    float result;
};

struct Lane {  // values a lane keeps across phases
    double pre;  // fp64 sum of all elements before this lane's first
};

// ---- phase: lane sums in fp64 -------------------------------------------------
__host__ __device__ inline void phase_sums(const float* p, int n, int tid, Shared& sm) {
    double acc = 0;
    for (int k = 0; k < kPerThread; ++k) {
        const int i = tid * kPerThread + k;
        if (i < n) acc += double(p[i]);
    }
    sm.dsum[0][tid] = acc;
}

// ---- Hillis-Steele inclusive scan of dsum, rounds 0..7 (result in dsum[0]) ---
__host__ __device__ inline void phase_dscan(int round, int tid, Shared& sm) {
    const int src = round & 1, off = 1 << round;
    sm.dsum[src ^ 1][tid] = sm.dsum[src][tid] + (tid >= off ? sm.dsum[src][tid - off] : 0.0);
}

// ---- phase: speculated crossings ----------------------------------------------
// element i crosses if the partial sum before it is 0 or its binade differs
// from the one after it
__host__ __device__ inline void phase_cross(const float* p, int n, int tid, Shared& sm, Lane& ln) {
    ln.pre = tid > 0 ? sm.dsum[0][tid - 1] : 0.0;
    double s = ln.pre;
    uint32_t bits = 0;
    for (int k = 0; k < kPerThread; ++k) {
        const int i = tid * kPerThread + k;
        if (i >= n) break;
        const double after = s + double(p[i]);
        const float fb = float(s), fa = float(after);
        // non-finite terms or sums are crossings too: they end up serial and
        // the walk's checks send the sum to the plain loop
        if (fb == 0.f || binade_f32(fb) != binade_f32(fa) || !(fabsf(p[i]) <= 3.0e38f) || !(fa <= 3.0e38f)) bits |= 1u << k;
        s = after;
    }
    sm.cross[tid] = uint16_t(bits);
}

// ---- phase: serial mask and the lane's aggregate for the segmented scan -------
__host__ __device__ inline void phase_local(const float* p, int n, int tid, Shared& sm, Lane& ln) {
    const uint32_t prev = tid > 0 ? sm.cross[tid - 1] : 0u;
    const uint32_t cur = sm.cross[tid];
    const uint32_t next = tid + 1 < kThreads ? sm.cross[tid + 1] : 0u;
    // bit j of `window` is the crossing flag of element k = j - 1 of this lane
    const uint64_t window = uint64_t(prev >> 15) | (uint64_t(cur) << 1) | (uint64_t(next & 1u) << 17);
    uint32_t serial = 0;
    for (int k = 0; k < kPerThread; ++k)
        if ((window >> k) & 7u) serial |= 1u << k;
    sm.serial[tid] = uint16_t(serial);

    double s = ln.pre;
    Fn tail = fn_identity();
    int32_t tail_e = kNoBinade, nser = 0;
    for (int k = 0; k < kPerThread; ++k) {
        const int i = tid * kPerThread + k;
        if (i >= n) break;
        if ((serial >> k) & 1u) {
            ++nser;
            tail = fn_identity();
            tail_e = kNoBinade;
        } else {
            const int e = binade_f32(float(s));
            tail = fn_then(tail, step_fn(p[i], e));
            tail_e = e;
        }
        s += double(p[i]);
    }
    sm.sep[0][tid] = nser > 0;
    sm.cnt[0][tid] = nser;
    sm.fn[0][tid] = tail;
    sm.e[0][tid] = tail_e;
}

// ---- segmented inclusive scan over lanes, rounds 0..7 (result in [0]) ----------
// (a earlier, b later): sep = a|b; fn = b.sep ? b.fn : a.fn then b.fn;
// e = b.sep || b has elements in its open run ? b.e : a.e; cnt = a + b
__host__ __device__ inline void phase_segscan(int round, int tid, Shared& sm) {
    const int src = round & 1, off = 1 << round;
    int32_t sep = sm.sep[src][tid], cnt = sm.cnt[src][tid], e = sm.e[src][tid];
    Fn f = sm.fn[src][tid];
    if (tid >= off) {
        const int j = tid - off;
        if (!sep) {
            f = fn_then(sm.fn[src][j], f);
            if (e == kNoBinade) e = sm.e[src][j];
        }
        sep |= sm.sep[src][j];
        cnt += sm.cnt[src][j];
    }
    sm.sep[src ^ 1][tid] = sep;
    sm.fn[src ^ 1][tid] = f;
    sm.e[src ^ 1][tid] = e;
    sm.cnt[src ^ 1][tid] = cnt;
}

// ---- phase: emit every run (in the order of the serial elements that end them)
__host__ __device__ inline void phase_runs(const float* p, int n, int tid, Shared& sm, const Lane& ln) {
    const int first = tid * kPerThread;
    if (first >= n) return;
    Fn run = tid > 0 ? sm.fn[0][tid - 1] : fn_identity();  // the run carried into this lane
    int32_t run_e = tid > 0 ? sm.e[0][tid - 1] : kNoBinade;
    int32_t r = tid > 0 ? sm.cnt[0][tid - 1] : 0;
    const uint32_t serial = sm.serial[tid];
    double s = ln.pre;
    for (int k = 0; k < kPerThread; ++k) {
        const int i = first + k;
        if (i >= n) break;
        if ((serial >> k) & 1u) {
            if (r < kMaxSerial) {
                sm.run[r] = run;
                sm.run_e[r] = int16_t(run_e);
                sm.ser_idx[r] = int16_t(i);
            }
            ++r;
            run = fn_identity();
            run_e = kNoBinade;
        } else {
            const int e = binade_f32(float(s));
            run = fn_then(run, step_fn(p[i], e));
            run_e = e;
        }
        s += double(p[i]);
    }
    if (first + kPerThread >= n) {  // the lane holding element n-1 closes the final run
        sm.nser = r;
        if (r <= kMaxSerial) {
            sm.run[r] = run;
            sm.run_e[r] = int16_t(run_e);
        }
    }
}

__host__ __device__ inline float serial_loop(const float* p, int n) {
    float s = 0.f;
    for (int i = 0; i < n; ++i) s += p[i];
    return s;
}

// ---- phase: the walk (one lane) ----------------------------------------------------
__host__ __device__ inline void phase_walk(const float* p, int n, Shared& sm) {
    const int nser = sm.nser;
    bool ok = nser <= kMaxSerial;
    float s = 0.f;
    int prev = -1;
    for (int r = 0; ok && r <= nser; ++r) {
        const int j = r < nser ? int(sm.ser_idx[r]) : n;
        if (j > prev + 1) {  // a non-empty run: elements prev+1 .. j-1
            const int e = sm.run_e[r];
            if (!(s > 0.f) || !(s <= 3.0e38f) || e == kNoBinade || binade_f32(s) != e) {
                ok = false;
                break;
            }
            const int64_t S = int64_t(mul_pow2(s, 23 - e));  // exact integer below 2^24
            const int64_t S2 = fn_apply(sm.run[r], S);
            if (S2 >= (int64_t(1) << 24)) {
                ok = false;
                break;
            }
            s = mul_pow2(float(S2), e - 23);
        }
        if (r < nser) s = s + p[j];
        prev = j;
    }
    sm.fell_back = ok ? 0 : 1;
    sm.result = ok ? s : serial_loop(p, n);
}

// ---- the whole sum on the device: 256 lanes, p in shared memory, n <= 4096 ----
__device__ inline float sum_nonneg(const float* p, int n, Shared& sm) {
    const int tid = threadIdx.x;
    Lane ln;
    phase_sums(p, n, tid, sm);
    __syncthreads();
    for (int r = 0; r < 8; ++r) {
        phase_dscan(r, tid, sm);
        __syncthreads();
    }
    phase_cross(p, n, tid, sm, ln);
    __syncthreads();
    phase_local(p, n, tid, sm, ln);
    __syncthreads();
    for (int r = 0; r < 8; ++r) {
        phase_segscan(r, tid, sm);
        __syncthreads();
    }
    phase_runs(p, n, tid, sm, ln);
    __syncthreads();
    if (tid == 0) phase_walk(p, n, sm);
    __syncthreads();
    return sm.result;
}

// ---- the same phases, one lane after another, on the host -----------------------
inline float sum_nonneg_host(const float* p, int n, Shared& sm) {
    static Lane ln[kThreads];
    for (int t = 0; t < kThreads; ++t) phase_sums(p, n, t, sm);
    for (int r = 0; r < 8; ++r)
        for (int t = 0; t < kThreads; ++t) phase_dscan(r, t, sm);
    for (int t = 0; t < kThreads; ++t) phase_cross(p, n, t, sm, ln[t]);
    for (int t = 0; t < kThreads; ++t) phase_local(p, n, t, sm, ln[t]);
    for (int r = 0; r < 8; ++r)
        for (int t = 0; t < kThreads; ++t) phase_segscan(r, t, sm);
    for (int t = 0; t < kThreads; ++t) phase_runs(p, n, t, sm, ln[t]);
    phase_walk(p, n, sm);
    return sm.result;
}

}  // namespace seqsum
}  // namespace hero
