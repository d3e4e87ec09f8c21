// oracle.cpp -- CPU restatement of the reference's Q8_0 Qwen 3.5 hybrid path.
// TEST INFRASTRUCTURE ONLY (the checker and the timed CPU baseline); see
// oracle.hpp for the rules and the per-function parity status.
//
// Build flags matter: -O3 -ffp-contract=off (oracle/Makefile). Without the last
// flag the compiler fuses `s += a*b` into an FMA and the fp32 results depend
// on the host and compiler (the reference's own Release build does that).
#include "oracle.hpp"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <immintrin.h>
#include <mutex>
#include <stdexcept>
#include <thread>

namespace oracle {

// ---------------------------------------------------------------------------
// fp16 codec. nm/src/core.hpp:34-60 (decode) and :61-79 (encode). The encode
// rounds half-up in magnitude on ties (one bit test, no sticky bits) and maps
// NaN to Inf; both quirks are part of the format this path must reproduce.
// ---------------------------------------------------------------------------
float fp16_to_fp32(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    const uint32_t exponent = (h >> 10) & 0x1Fu;
    const uint32_t mantissa = h & 0x3FFu;
    uint32_t bits;
    if (exponent == 0) {
        if (mantissa == 0) {
            bits = sign;
        } else {
            // subnormal half: shift the leading one up to the implicit bit
            int shift = 0;
            uint32_t m = mantissa;
            while ((m & 0x400u) == 0) {
                m <<= 1;
                ++shift;
            }
            // value = m * 2^-24 * 2^-shift ; biased fp32 exponent = 127 - 14 - shift
            bits = sign | (uint32_t(113 - shift) << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (exponent == 0x1Fu) {
        bits = sign | 0x7F800000u | (mantissa << 13);
    } else {
        bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

uint16_t fp32_to_fp16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int32_t exponent = int32_t((x >> 23) & 0xFFu) - 112;  // rebias 127 -> 15
    uint32_t mantissa = x & 0x7FFFFFu;
    if (exponent <= 0) {
        if (exponent < -10) return uint16_t(sign);
        mantissa |= 0x800000u;
        const uint32_t shift = uint32_t(14 - exponent);
        uint32_t r = mantissa >> shift;
        r += (mantissa >> (shift - 1)) & 1u;  // half-up on the first dropped bit
        return uint16_t(sign | r);
    }
    if (exponent >= 0x1F) return uint16_t(sign | 0x7C00u);  // overflow, Inf and NaN -> Inf
    uint16_t h = uint16_t(sign | (uint32_t(exponent) << 10) | (mantissa >> 13));
    h = uint16_t(h + ((mantissa >> 12) & 1u));  // half-up, may carry into the exponent
    return h;
}

// ---------------------------------------------------------------------------
// Q8_0
// ---------------------------------------------------------------------------
// nm/src/quant_i8.hpp:70-80 (activations): d = amax/127, id = 1/d, roundf.
void quantize_row_q8_0(const float* x, BlockQ8* y, size_t k) {
    const size_t blocks = k / 32;
    for (size_t b = 0; b < blocks; ++b) {
        const float* xb = x + b * 32;
        float amax = 0.f;
        for (size_t j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(xb[j]));
        const float d = amax / 127.f;
        const float id = d != 0.f ? 1.f / d : 0.f;
        y[b].d = fp32_to_fp16(d);
        for (size_t j = 0; j < 32; ++j) y[b].qs[j] = int8_t(std::roundf(xb[j] * id));
    }
}

// nm/src/quant.hpp:404-413 (weights): the same scale, lround.
void quantize_q8_0(const float* x, BlockQ8* y, size_t n) {
    const size_t blocks = n / 32;
    for (size_t b = 0; b < blocks; ++b) {
        const float* xb = x + b * 32;
        float amax = 0.f;
        for (size_t j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(xb[j]));
        const float d = amax / 127.f;
        const float id = d != 0.f ? 1.f / d : 0.f;
        y[b].d = fp32_to_fp16(d);
        for (size_t j = 0; j < 32; ++j) y[b].qs[j] = int8_t(std::lround(xb[j] * id));
    }
}

// nm/src/quant_i8.hpp:85-100: exact int32 block sum, then the block's term
// sumi * (d_w * d_x) added to an fp32 accumulator in block order.
float vec_dot_q8_0_q8_0(size_t n, const BlockQ8* w, const BlockQ8* x) {
    const size_t blocks = n / 32;
    float sum = 0.f;
    for (size_t b = 0; b < blocks; ++b) {
        int sumi = 0;
        for (size_t j = 0; j < 32; ++j) sumi += int(w[b].qs[j]) * int(x[b].qs[j]);
        const float scale = fp16_to_fp32(w[b].d) * fp16_to_fp32(x[b].d);
        sum += float(sumi) * scale;
    }
    return sum;
}

// nm/src/quant.hpp:306-313
void dequant_row_q8_0(const BlockQ8* row, float* out, size_t k) {
    for (size_t b = 0; b < k / 32; ++b) {
        const float d = fp16_to_fp32(row[b].d);
        for (size_t j = 0; j < 32; ++j) out[b * 32 + j] = d * float(row[b].qs[j]);
    }
}

// ---------------------------------------------------------------------------
// Row-parallel pool: the reference's par_for policy (nm/src/core.cpp:22-117)
// restated: persistent workers plus the caller, an atomic chunk counter with
// chunk = max(1, n/(threads*16)), one job at a time, nested calls serial.
// ---------------------------------------------------------------------------
namespace {
thread_local bool tl_inside_job = false;

class Pool {
public:
    static Pool& instance() {
        static Pool pool;
        return pool;
    }
    size_t threads() const { return threads_; }

    void resize(size_t n) {
        std::lock_guard<std::mutex> job(job_mutex_);
        stop_workers();
        threads_ = n == 0 ? 1 : n;
        start_workers();
    }

    void run(size_t n, void (*fn)(size_t, void*), void* ctx) {
        if (n == 0) return;
        if (threads_ <= 1 || n == 1 || tl_inside_job) {
            for (size_t i = 0; i < n; ++i) fn(i, ctx);
            return;
        }
        std::lock_guard<std::mutex> job(job_mutex_);
        fn_ = fn;
        ctx_ = ctx;
        n_ = n;
        chunk_ = std::max<size_t>(1, n / (threads_ * 16));
        next_.store(0, std::memory_order_relaxed);
        pending_.store(threads_, std::memory_order_relaxed);
        {
            std::lock_guard<std::mutex> lk(mutex_);
            ++generation_;
        }
        wake_.notify_all();
        drain();
        std::unique_lock<std::mutex> lk(done_mutex_);
        done_.wait(lk, [&] { return pending_.load(std::memory_order_acquire) == 0; });
    }

    ~Pool() { stop_workers(); }

private:
    Pool() {
        const unsigned hc = std::thread::hardware_concurrency();
        threads_ = hc ? hc : 1;
        if (const char* env = std::getenv("NM_THREADS")) {
            const long v = std::atol(env);
            if (v > 0) threads_ = size_t(v);
        }
        start_workers();
    }

    void start_workers() {
        uint64_t g0;
        {
            std::lock_guard<std::mutex> lk(mutex_);
            stop_ = false;
            g0 = generation_;
        }
        // a worker starts from the generation before it existed, so it joins
        // any job begun while it was still starting up
        for (size_t i = 1; i < threads_; ++i) workers_.emplace_back([this, g0] { worker_main(g0); });
    }
    void stop_workers() {
        {
            std::lock_guard<std::mutex> lk(mutex_);
            stop_ = true;
            ++generation_;
        }
        wake_.notify_all();
        for (auto& t : workers_) t.join();
        workers_.clear();
    }

    void drain() {
        tl_inside_job = true;
        for (;;) {
            const size_t begin = next_.fetch_add(chunk_, std::memory_order_relaxed);
            if (begin >= n_) break;
            const size_t end = std::min(begin + chunk_, n_);
            for (size_t i = begin; i < end; ++i) fn_(i, ctx_);
        }
        tl_inside_job = false;
        if (pending_.fetch_sub(1, std::memory_order_acq_rel) == 1) {
            std::lock_guard<std::mutex> lk(done_mutex_);
            done_.notify_all();
        }
    }

    void worker_main(uint64_t seen) {
        for (;;) {
            std::unique_lock<std::mutex> lk(mutex_);
            wake_.wait(lk, [&] { return stop_ || generation_ != seen; });
            if (stop_) return;
            seen = generation_;
            lk.unlock();
            drain();
        }
    }

    size_t threads_ = 1;
    std::vector<std::thread> workers_;
    std::mutex mutex_, done_mutex_, job_mutex_;
    std::condition_variable wake_, done_;
    void (*fn_)(size_t, void*) = nullptr;
    void* ctx_ = nullptr;
    size_t n_ = 0, chunk_ = 1;
    std::atomic<size_t> next_{0}, pending_{0};
    uint64_t generation_ = 0;
    bool stop_ = false;
};

template <class F>
void par_for_lambda(size_t n, F&& f) {
    par_for(
        n, [](size_t i, void* ctx) { (*static_cast<F*>(ctx))(i); }, &f);
}
}  // namespace

void par_for(size_t n, void (*fn)(size_t, void*), void* ctx) { Pool::instance().run(n, fn, ctx); }
size_t num_threads() { return Pool::instance().threads(); }
void set_threads(size_t n) { Pool::instance().resize(n); }

// nm/src/quant_i8.hpp:352-383: quantize once on the caller, rows in parallel.
void matvec_q8_0(const BlockQ8* W, size_t N, size_t K, const float* x, float* y) {
    std::vector<BlockQ8> act(K / 32);
    quantize_row_q8_0(x, act.data(), K);
    const size_t row_blocks = K / 32;
    par_for_lambda(N, [&](size_t o) { y[o] = vec_dot_q8_0_q8_0(K, W + o * row_blocks, act.data()); });
}

// nm/src/quant_i8.hpp:430-474: rows quantized in parallel, then each output
// row held stationary while it sweeps the T activation rows.
void matmul_q8_0(const BlockQ8* W, size_t N, size_t K, const float* X, size_t T, float* Y) {
    if (T == 0) return;
    const size_t row_blocks = K / 32;
    std::vector<BlockQ8> act(T * row_blocks);
    par_for_lambda(T, [&](size_t t) { quantize_row_q8_0(X + t * K, act.data() + t * row_blocks, K); });
    par_for_lambda(N, [&](size_t o) {
        const BlockQ8* w = W + o * row_blocks;
        for (size_t t = 0; t < T; ++t) Y[t * N + o] = vec_dot_q8_0_q8_0(K, w, act.data() + t * row_blocks);
    });
}

// ---------------------------------------------------------------------------
// K-quants
// ---------------------------------------------------------------------------
// nm/src/quant_i8.hpp:31-36: round to nearest, ties to even, through the
// 1.5 * 2^23 offset (valid for |v| < 2^22).
static int nearest_int_magic(float v) {
    const float t = v + 12582912.f;
    int32_t i;
    std::memcpy(&i, &t, 4);
    return (i & 0x007fffff) - 0x00400000;
}

// nm/src/quant_i8.hpp:39-64. The scale is -127 over the signed value of the
// first element of largest magnitude, so that element maps to -127 exactly.
void quantize_row_q8_K(const float* x, BlockQ8K* y, size_t k) {
    for (size_t b = 0; b < k / 256; ++b, x += 256) {
        float mx = 0.f, amax = 0.f;
        for (size_t j = 0; j < 256; ++j) {
            const float a = std::fabs(x[j]);
            if (a > amax) {
                amax = a;
                mx = x[j];
            }
        }
        BlockQ8K& o = y[b];
        if (amax == 0.f) {
            std::memset(&o, 0, sizeof o);
            continue;
        }
        const float iscale = -127.f / mx;
        for (size_t j = 0; j < 256; ++j) o.qs[j] = int8_t(std::min(127, nearest_int_magic(iscale * x[j])));
        for (size_t g = 0; g < 16; ++g) {
            int s = 0;
            for (size_t l = 0; l < 16; ++l) s += o.qs[g * 16 + l];
            o.bsums[g] = int16_t(s);
        }
        o.d = 1.f / iscale;
    }
}

// 6-bit scales and mins of a Q4_K block: entries 0..3 in the low 6 bits of
// bytes 0..3 (scales) and 4..7 (mins); entries 4..7 from the nibbles of bytes
// 8..11 plus the top two bits of bytes 0..7 (nm/src/quant_i8.hpp:129-142
// computes the same values with word masks).
static void q4k_scale_min(const uint8_t* p, int j, int& sc, int& mn) {
    if (j < 4) {
        sc = p[j] & 63;
        mn = p[j + 4] & 63;
    } else {
        sc = (p[j + 4] & 0xF) | ((p[j - 4] >> 6) << 4);
        mn = (p[j + 4] >> 4) | ((p[j] >> 6) << 4);
    }
}

// nm/src/quant_i8.hpp:146-191. Per block: eight integer sums aux[l] over the
// positions l mod 8 (each product scaled by its 32-weight sub-block's scale),
// the mins term from the activation's 16-element sums; then in fp32 and block
// order: sums[l] += d * aux[l], sumf -= dmin * summin; finally sumf += sums[l]
// for l = 0..7.
float vec_dot_q4_K_q8_K(size_t n, const BlockQ4K* w, const BlockQ8K* x) {
    float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float sumf = 0.f;
    for (size_t b = 0; b < n / 256; ++b) {
        const BlockQ4K& wb = w[b];
        const BlockQ8K& xb = x[b];
        int32_t aux[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int summin = 0;
        for (int j = 0; j < 8; ++j) {  // sub-block j: weights 32j .. 32j+31
            int sc, mn;
            q4k_scale_min(wb.scales, j, sc, mn);
            for (int i = 0; i < 32; ++i) {
                const uint8_t byte = wb.qs[(j / 2) * 32 + i];
                const int q = (j & 1) ? (byte >> 4) : (byte & 0xF);
                aux[i % 8] += sc * (q * xb.qs[32 * j + i]);
            }
            summin += mn * (xb.bsums[2 * j] + xb.bsums[2 * j + 1]);
        }
        const float d = fp16_to_fp32(wb.d) * xb.d;
        for (int l = 0; l < 8; ++l) sums[l] += d * float(aux[l]);
        const float dmin = fp16_to_fp32(wb.dmin) * xb.d;
        sumf -= dmin * float(summin);
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

// nm/src/quant_i8.hpp:239-278. Weight e of a 128-weight half h: low nibble
// from ql (byte e % 64 of the half's 64, high nibble for e >= 64), two high
// bits from qh byte e % 32 at shift 2 * (e / 32), minus 32; the int8 scale of
// each 16 weights; then sums[l] += d * aux[l] per block and sumf = sum of
// sums[l].
float vec_dot_q6_K_q8_K(size_t n, const BlockQ6K* w, const BlockQ8K* x) {
    float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (size_t b = 0; b < n / 256; ++b) {
        const BlockQ6K& wb = w[b];
        const BlockQ8K& xb = x[b];
        int32_t aux[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int p = 0; p < 256; ++p) {
            const int h = p / 128, e = p % 128;
            const uint8_t lo = wb.ql[64 * h + e % 64];
            const int low = e < 64 ? (lo & 0xF) : (lo >> 4);
            const int high = (wb.qh[32 * h + e % 32] >> (2 * (e / 32))) & 3;
            const int q = (low | (high << 4)) - 32;
            aux[p % 8] += int(wb.scales[p / 16]) * (q * xb.qs[p]);
        }
        const float d = fp16_to_fp32(wb.d) * xb.d;
        for (int l = 0; l < 8; ++l) sums[l] += d * float(aux[l]);
    }
    float sumf = 0.f;
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

void matmul_kquant(int type, const void* W, size_t N, size_t K, const float* X, size_t T, float* Y) {
    if (T == 0) return;
    const size_t nb = K / 256;
    std::vector<BlockQ8K> act(T * nb);
    par_for_lambda(T, [&](size_t t) { quantize_row_q8_K(X + t * K, act.data() + t * nb, K); });
    par_for_lambda(N, [&](size_t o) {
        for (size_t t = 0; t < T; ++t)
            Y[t * N + o] = type == 12 ? vec_dot_q4_K_q8_K(K, static_cast<const BlockQ4K*>(W) + o * nb, act.data() + t * nb)
                                      : vec_dot_q6_K_q8_K(K, static_cast<const BlockQ6K*>(W) + o * nb, act.data() + t * nb);
    });
}

// nm/src/quant.hpp:207-229. Sub-block pair p (64 weights) uses scale/min
// entries 2p and 2p+1 and the nibbles of qs[32p .. 32p+31] (low for the first
// 32 weights, high for the next); its fifth bits are bits 2p and 2p+1 of qh[l].
// One fp32 accumulator over the 256 products in order, each product
// (d1*q - m1)*x rounded step by step.
float dot_block_q5_K(const BlockQ5K& b, const float* x) {
    const float d = fp16_to_fp32(b.d), mn = fp16_to_fp32(b.dmin);
    float acc = 0.f;
    for (int p = 0; p < 4; ++p) {
        int sc, m;
        q4k_scale_min(b.scales, 2 * p, sc, m);
        const float d1 = d * float(sc), m1 = mn * float(m);
        q4k_scale_min(b.scales, 2 * p + 1, sc, m);
        const float d2 = d * float(sc), m2 = mn * float(m);
        const uint8_t* ql = b.qs + 32 * p;
        for (int l = 0; l < 32; ++l) {
            const int q = (ql[l] & 0xF) + ((b.qh[l] >> (2 * p)) & 1) * 16;
            acc += (d1 * float(q) - m1) * x[64 * p + l];
        }
        for (int l = 0; l < 32; ++l) {
            const int q = (ql[l] >> 4) + ((b.qh[l] >> (2 * p + 1)) & 1) * 16;
            acc += (d2 * float(q) - m2) * x[64 * p + 32 + l];
        }
    }
    return acc;
}

// nm/src/quant_i8.hpp:487-495 (the fp32-activation branch of Weight::matmul):
// each output the sequential sum of its blocks' dots
void matmul_q5_K(const BlockQ5K* W, size_t N, size_t K, const float* X, size_t T, float* Y) {
    const size_t nb = K / 256;
    par_for_lambda(N, [&](size_t o) {
        for (size_t t = 0; t < T; ++t) {
            float acc = 0.f;
            for (size_t i = 0; i < nb; ++i) acc += dot_block_q5_K(W[o * nb + i], X + t * K + i * 256);
            Y[t * N + o] = acc;
        }
    });
}

size_t row_bytes(int type, size_t k) {
    switch (type) {
        case 8: return k / 32 * 34;
        case 12: return k / 256 * 144;
        case 13: return k / 256 * 176;
        case 14: return k / 256 * 210;
        default: throw std::invalid_argument("row_bytes: unsupported ggml type " + std::to_string(type));
    }
}

// nm/src/quant.hpp:322-395
void dequant_row(int type, const void* row, float* out, size_t k) {
    if (type == 8) return dequant_row_q8_0(static_cast<const BlockQ8*>(row), out, k);
    for (size_t i = 0; i < k / 256; ++i) {
        float* y = out + 256 * i;
        if (type == 12 || type == 13) {  // Q4_K, Q5_K: d1*q - m1
            const uint8_t* blk = static_cast<const uint8_t*>(row) + i * (type == 12 ? 144 : 176);
            uint16_t dh, mh;
            std::memcpy(&dh, blk, 2);
            std::memcpy(&mh, blk + 2, 2);
            const uint8_t* scales = blk + 4;
            const uint8_t* qh = type == 13 ? blk + 16 : nullptr;
            const uint8_t* qs = blk + (type == 13 ? 48 : 16);
            const float d = fp16_to_fp32(dh), mn = fp16_to_fp32(mh);
            for (int p = 0; p < 4; ++p) {
                for (int h = 0; h < 2; ++h) {
                    int sc, m;
                    q4k_scale_min(scales, 2 * p + h, sc, m);
                    const float d1 = d * float(sc), m1 = mn * float(m);
                    for (int l = 0; l < 32; ++l) {
                        int q = h ? (qs[32 * p + l] >> 4) : (qs[32 * p + l] & 0xF);
                        if (qh) q += ((qh[l] >> (2 * p + h)) & 1) * 16;
                        y[64 * p + 32 * h + l] = d1 * float(q) - m1;
                    }
                }
            }
        } else if (type == 14) {  // Q6_K: (d * scale) * q per group of 16
            const BlockQ6K& b = static_cast<const BlockQ6K*>(row)[i];
            const float d = fp16_to_fp32(b.d);
            for (int p = 0; p < 256; ++p) {
                const int h = p / 128, e = p % 128;
                const uint8_t lo = b.ql[64 * h + e % 64];
                const int low = e < 64 ? (lo & 0xF) : (lo >> 4);
                const int high = (b.qh[32 * h + e % 32] >> (2 * (e / 32))) & 3;
                y[p] = d * float(b.scales[p / 16]) * float((low | (high << 4)) - 32);
            }
        } else {
            throw std::invalid_argument("dequant_row: unsupported ggml type " + std::to_string(type));
        }
    }
}

void linear_rows(const Linear& lin, const float* X, size_t T, float* Y) {
    switch (lin.type) {
        case 8: return matmul_q8_0(static_cast<const BlockQ8*>(lin.w), lin.N, lin.K, X, T, Y);
        case 12:
        case 14: return matmul_kquant(lin.type, lin.w, lin.N, lin.K, X, T, Y);
        case 13: return matmul_q5_K(static_cast<const BlockQ5K*>(lin.w), lin.N, lin.K, X, T, Y);
        default: throw std::invalid_argument("linear: unsupported ggml type " + std::to_string(lin.type));
    }
}

// ---------------------------------------------------------------------------
// small ops
// ---------------------------------------------------------------------------
float dot(const float* a, const float* b, size_t n) {  // core.hpp:496-500
    float s = 0.f;
    for (size_t i = 0; i < n; ++i) s += a[i] * b[i];
    return s;
}
float sigmoid(float x) { return 1.f / (1.f + std::exp(-x)); }                 // core.hpp:579
float silu(float x) { return x / (1.f + std::exp(-x)); }                        // components.hpp:105
float softplus(float x) { return x > 20.f ? x : std::log1p(std::exp(x)); }      // recurrent.hpp:35

// components.hpp:176-181: inv = 1/sqrt(dot(x,x)/N + eps); x = (gamma*x)*inv
void rmsnorm(float* x, const float* gamma, size_t n, float eps) {
    const float inv = 1.f / std::sqrt(dot(x, x, n) / float(n) + eps);
    for (size_t c = 0; c < n; ++c) x[c] = gamma[c] * x[c] * inv;
}

// recurrent.hpp:40-48
void l2_normalize(const float* x, float* out, size_t n, float eps) {
    float ss = 0.f;
    for (size_t i = 0; i < n; ++i) ss += x[i] * x[i];
    const float scale = 1.f / std::max(std::sqrt(ss), eps);
    for (size_t i = 0; i < n; ++i) out[i] = x[i] * scale;
}

// components.hpp:132-141
void softmax(float* v, size_t n) {
    const float largest = *std::max_element(v, v + n);
    float total = 0.f;
    for (size_t i = 0; i < n; ++i) {
        v[i] = std::exp(v[i] - largest);
        total += v[i];
    }
    for (size_t i = 0; i < n; ++i) v[i] /= total;
}

// recurrent.hpp:75-106: sum = taps[W-1]*x, then += taps[i]*past(i), oldest first.
void conv_step(const float* input, const float* taps, float* history, float* out, size_t channels, size_t width) {
    const size_t hist = width - 1;
    for (size_t c = 0; c < channels; ++c) {
        const float* t = taps + c * width;
        float sum = t[hist] * input[c];
        for (size_t i = 0; i < hist; ++i) sum += t[i] * history[i * channels + c];
        out[c] = sum;
    }
    // shift: drop the oldest row, append the input as the newest
    if (hist > 0) {
        for (size_t i = 0; i + 1 < hist; ++i) std::memcpy(history + i * channels, history + (i + 1) * channels, channels * sizeof(float));
        std::memcpy(history + (hist - 1) * channels, input, channels * sizeof(float));
    }
}

// recurrent.hpp:146-177
void gated_delta_step(float* state, const float* q, const float* k, const float* v, float gate, float beta, float* out, size_t dk, size_t dv) {
    const float decay = std::exp(gate);
    std::vector<float> predicted(dv, 0.f), delta(dv);
    for (size_t i = 0; i < dk; ++i) {
        float* row = state + i * dv;
        const float ki = k[i];
        for (size_t j = 0; j < dv; ++j) {
            row[j] *= decay;
            predicted[j] += row[j] * ki;
        }
    }
    for (size_t j = 0; j < dv; ++j) delta[j] = (v[j] - predicted[j]) * beta;
    for (size_t j = 0; j < dv; ++j) out[j] = 0.f;
    for (size_t i = 0; i < dk; ++i) {
        float* row = state + i * dv;
        const float ki = k[i], qi = q[i];
        for (size_t j = 0; j < dv; ++j) {
            row[j] += ki * delta[j];
            out[j] += row[j] * qi;
        }
    }
}

// attention.hpp:76-80: inv_freq[i] = float(pow(double base, -2i/Dh)) for the
// rotary planes, 0 for the rest.
std::vector<float> rope_inv_freq(size_t head_dim, double base, size_t rotary_dims) {
    const size_t planes = head_dim / 2, rotary_planes = rotary_dims / 2;
    std::vector<float> inv(planes, 0.f);
    for (size_t i = 0; i < planes; ++i) inv[i] = i < rotary_planes ? float(std::pow(base, -double(2 * i) / double(head_dim))) : 0.f;
    return inv;
}

// attention.hpp:82-91: angle = float(pos)*inv_freq; planes (i, i+Dh/2).
void rope_apply(float* head, const float* inv_freq, size_t head_dim, size_t position) {
    const size_t planes = head_dim / 2;
    for (size_t i = 0; i < planes; ++i) {
        const float angle = float(position) * inv_freq[i];
        const float c = std::cos(angle), s = std::sin(angle);
        const float x = head[i], y = head[i + planes];
        head[i] = x * c - y * s;
        head[i + planes] = y * c + x * s;
    }
}

// qwen35.hpp:366-380: scores scale*dot(q,k_j), Softmax, then
// out += alpha_j * v_j in row order (Vec::scaled_add, core.hpp:206-208).
void attend_one(const float* q, const float* keys, const float* values, size_t kv_width, size_t kv_head, size_t head_dim, size_t first, size_t end, float scale, float* out) {
    if (end <= first) throw std::runtime_error("attention: query has no visible keys");
    std::vector<float> alpha(end - first);
    for (size_t j = first; j < end; ++j) alpha[j - first] = scale * dot(q, keys + j * kv_width + kv_head * head_dim, head_dim);
    softmax(alpha.data(), alpha.size());
    for (size_t c = 0; c < head_dim; ++c) out[c] = 0.f;
    for (size_t n = 0; n < alpha.size(); ++n) {
        const float* v = values + (first + n) * kv_width + kv_head * head_dim;
        for (size_t c = 0; c < head_dim; ++c) out[c] += alpha[n] * v[c];
    }
}

// F16C's conversion with imm 0 rounds to nearest even (IEEE 754 default).
float round_fp16_rne(float x) { return _cvtsh_ss(_cvtss_sh(x, 0)); }

// ---------------------------------------------------------------------------
// Qwen 3.5 hybrid (qwen35.hpp:288-462)
// ---------------------------------------------------------------------------
void State::reset(const Config& c) {
    tokens = 0;
    keys.assign(c.L, {});
    values.assign(c.L, {});
    conv_hist.assign(c.L, {});
    delta.assign(c.L, {});
    for (size_t l = 0; l < c.L; ++l) {
        if (c.is_recurrent(l)) {
            conv_hist[l].assign((c.conv_width - 1) * c.conv_channels(), 0.f);
            delta[l].assign(c.Hv * c.Dk * c.Dv, 0.f);
        }
    }
}

void embed(const Model& m, const int32_t* ids, size_t n, float* out) {
    const size_t D = m.c.D;
    for (size_t i = 0; i < n; ++i) {
        if (ids[i] < 0 || size_t(ids[i]) >= m.c.V) throw std::out_of_range("embed: token id out of range");
        dequant_row(m.embedding.type, static_cast<const uint8_t*>(m.embedding.w) + size_t(ids[i]) * row_bytes(m.embedding.type, D), out + i * D, D);
    }
}

namespace {

std::vector<float> linear(const Linear& lin, const float* X, size_t T) {
    std::vector<float> Y(T * lin.N);
    linear_rows(lin, X, T, Y.data());
    return Y;
}

std::vector<float> norm_rows(const float* X, size_t T, size_t n, const std::vector<float>& gamma, float eps) {
    std::vector<float> Y(X, X + T * n);
    for (size_t t = 0; t < T; ++t) rmsnorm(Y.data() + t * n, gamma.data(), n, eps);
    return Y;
}

// qwen35.hpp:343-395
std::vector<float> attention_mixer(const Model& m, const Layer& L, size_t layer, State& s, const float* X, size_t T) {
    const Config& c = m.c;
    const size_t Dh = c.head_dim, QW = c.Hq * Dh, KW = c.Hkv * Dh;
    const std::vector<float> QG = linear(L.wqg, X, T);
    std::vector<float> Q(T * QW), G(T * QW);
    for (size_t t = 0; t < T; ++t)  // split_head_pairs (attention.hpp:38-56)
        for (size_t h = 0; h < c.Hq; ++h)
            for (size_t i = 0; i < Dh; ++i) {
                Q[t * QW + h * Dh + i] = QG[t * 2 * QW + h * 2 * Dh + i];
                G[t * QW + h * Dh + i] = QG[t * 2 * QW + h * 2 * Dh + Dh + i];
            }
    std::vector<float> K = linear(L.wk, X, T);
    const std::vector<float> V = linear(L.wv, X, T);
    for (size_t t = 0; t < T; ++t) {
        for (size_t h = 0; h < c.Hq; ++h) {
            rmsnorm(Q.data() + t * QW + h * Dh, L.q_norm.data(), Dh, c.eps);
            rope_apply(Q.data() + t * QW + h * Dh, m.inv_freq.data(), Dh, s.tokens + t);
        }
        for (size_t h = 0; h < c.Hkv; ++h) {
            rmsnorm(K.data() + t * KW + h * Dh, L.k_norm.data(), Dh, c.eps);
            rope_apply(K.data() + t * KW + h * Dh, m.inv_freq.data(), Dh, s.tokens + t);
        }
    }
    // append all T rows, then reduce (qwen35.hpp:386-387)
    s.keys[layer].insert(s.keys[layer].end(), K.begin(), K.end());
    s.values[layer].insert(s.values[layer].end(), V.begin(), V.end());
    if (s.kv_fp16)
        for (size_t i = s.keys[layer].size() - K.size(); i < s.keys[layer].size(); ++i) {
            s.keys[layer][i] = round_fp16_rne(s.keys[layer][i]);
            s.values[layer][i] = round_fp16_rne(s.values[layer][i]);
        }
    if (s.kv_q8) {  // rows of KW values, blocks of 32 within a row
        const size_t first = s.keys[layer].size() - K.size();
        std::vector<BlockQ8> blocks(KW / 32);
        for (std::vector<float>* cache : {&s.keys[layer], &s.values[layer]})
            for (size_t r = first; r < cache->size(); r += KW) {
                quantize_row_q8_0(cache->data() + r, blocks.data(), KW);
                dequant_row_q8_0(blocks.data(), cache->data() + r, KW);
            }
    }
    const float score_scale = 1.f / std::sqrt(float(Dh));
    std::vector<float> A(T * QW);
    const size_t group = c.Hq / c.Hkv;
    par_for_lambda(T * c.Hq, [&](size_t task) {
        const size_t t = task / c.Hq, h = task % c.Hq;
        const size_t end = s.tokens + t + 1;  // causal: rows [0, pos+1)
        attend_one(Q.data() + t * QW + h * Dh, s.keys[layer].data(), s.values[layer].data(), KW, h / group, Dh, 0, end, score_scale, A.data() + t * QW + h * Dh);
    });
    for (size_t i = 0; i < T * QW; ++i) A[i] *= sigmoid(G[i]);
    return linear(L.wo, A.data(), T);
}

// qwen35.hpp:400-462
std::vector<float> recurrent_mixer(const Model& m, const Layer& L, size_t layer, State& s, const float* X, size_t T) {
    const Config& c = m.c;
    const size_t Dk = c.Dk, Dv = c.Dv, Hk = c.Hk, Hv = c.Hv, CC = c.conv_channels();
    const size_t KEY_WIDTH = Hk * Dk, VALUE_WIDTH = Hv * Dv;
    const float query_scale = 1.f / std::sqrt(float(Dk));

    const std::vector<float> qkv = linear(L.wqkv, X, T);
    std::vector<float> beta = linear(L.wbeta, X, T);
    for (float& b : beta) b = sigmoid(b);
    std::vector<float> gate = linear(L.walpha, X, T);
    for (size_t t = 0; t < T; ++t)
        for (size_t h = 0; h < Hv; ++h) gate[t * Hv + h] = L.decay_scale[h] * softplus(gate[t * Hv + h] + L.dt_bias[h]);

    std::vector<float> mixed(T * VALUE_WIDTH);
    std::vector<float> stream(CC), query(KEY_WIDTH), key(KEY_WIDTH);
    for (size_t t = 0; t < T; ++t) {
        conv_step(qkv.data() + t * CC, L.conv.data(), s.conv_hist[layer].data(), stream.data(), CC, c.conv_width);
        for (float& v : stream) v = silu(v);
        for (size_t hk = 0; hk < Hk; ++hk) {
            l2_normalize(stream.data() + hk * Dk, query.data() + hk * Dk, Dk, 1e-6f);
            l2_normalize(stream.data() + KEY_WIDTH + hk * Dk, key.data() + hk * Dk, Dk, 1e-6f);
            for (size_t i = 0; i < Dk; ++i) query[hk * Dk + i] *= query_scale;
        }
        for (size_t h = 0; h < Hv; ++h) {
            const size_t hk = h % Hk;  // tiled key heads (qwen35.hpp:172)
            gated_delta_step(s.delta[layer].data() + h * Dk * Dv, query.data() + hk * Dk, key.data() + hk * Dk, stream.data() + 2 * KEY_WIDTH + h * Dv, gate[t * Hv + h], beta[t * Hv + h], mixed.data() + t * VALUE_WIDTH + h * Dv, Dk, Dv);
        }
    }
    for (size_t t = 0; t < T; ++t)
        for (size_t h = 0; h < Hv; ++h) rmsnorm(mixed.data() + t * VALUE_WIDTH + h * Dv, L.ssm_norm.data(), Dv, c.eps);
    std::vector<float> z = linear(L.wz, X, T);
    for (size_t i = 0; i < z.size(); ++i) mixed[i] = mixed[i] * silu(z[i]);  // hadamard(mixed, Silu(z))
    return linear(L.wout, mixed.data(), T);
}

}  // namespace

void forward(const Model& m, State& s, const float* rows, size_t T, float* logits) {
    const Config& c = m.c;
    if (T == 0) throw std::invalid_argument("forward: empty input");
    if (T > c.CTX - s.tokens) throw std::length_error("forward: context exhausted");
    const size_t D = c.D;
    std::vector<float> X(rows, rows + T * D);
    for (size_t l = 0; l < c.L; ++l) {
        const Layer& L = m.layers[l];
        const std::vector<float> U = norm_rows(X.data(), T, D, L.mixer_norm, c.eps);
        const std::vector<float> M = c.is_recurrent(l) ? recurrent_mixer(m, L, l, s, U.data(), T) : attention_mixer(m, L, l, s, U.data(), T);
        std::vector<float> H(T * D);
        for (size_t i = 0; i < T * D; ++i) H[i] = X[i] + M[i];
        const std::vector<float> Z = norm_rows(H.data(), T, D, L.channel_norm, c.eps);
        std::vector<float> g = linear(L.gate, Z.data(), T);
        const std::vector<float> u = linear(L.up, Z.data(), T);
        for (size_t i = 0; i < g.size(); ++i) g[i] = silu(g[i]) * u[i];
        const std::vector<float> F = linear(L.down, g.data(), T);
        for (size_t i = 0; i < T * D; ++i) X[i] = H[i] + F[i];
    }
    s.tokens += T;
    std::vector<float> last(X.begin() + (T - 1) * D, X.begin() + T * D);
    rmsnorm(last.data(), m.final_norm.data(), D, c.eps);
    linear_rows(m.output, last.data(), 1, logits);  // matvec = the one-row matmul, output by output
}

// nm/src/logits.hpp:71-105: sort down to k candidates, exp((v - max) / temp)
// and their sequential sum, the first prefix whose sequential sum of p / sum
// reaches top_p, the kept prefix's sequential sum s2, r = u * s2, and the
// first candidate whose running sum reaches r.
int32_t sample_topk(const float* logits, size_t V, size_t top_k, float temp, float top_p, float u) {
    std::vector<int32_t> idx(V);
    for (size_t i = 0; i < V; ++i) idx[i] = int32_t(i);
    const size_t k = top_k > 0 ? std::min(top_k, V) : V;
    std::partial_sort(idx.begin(), idx.begin() + k, idx.end(), [&](int32_t a, int32_t b) {
        return logits[a] > logits[b] || (logits[a] == logits[b] && a < b);
    });
    const float mx = logits[idx[0]];
    std::vector<float> pr(k);
    float sum = 0.f;
    for (size_t i = 0; i < k; ++i) {
        pr[i] = std::exp((logits[idx[i]] - mx) / temp);
        sum += pr[i];
    }
    float cum = 0.f;
    size_t keep = k;
    for (size_t i = 0; i < k; ++i) {
        cum += pr[i] / sum;
        if (cum >= top_p) {
            keep = i + 1;
            break;
        }
    }
    float s2 = 0.f;
    for (size_t i = 0; i < keep; ++i) s2 += pr[i];
    const float r = u * (s2 - 0.f) + 0.f;
    float acc = 0.f;
    for (size_t i = 0; i < keep; ++i) {
        acc += pr[i];
        if (r <= acc) return idx[i];
    }
    return idx[keep - 1];
}

int32_t argmax(const float* logits, size_t n) {
    size_t best = 0;
    for (size_t v = 1; v < n; ++v)
        if (logits[v] > logits[best]) best = v;
    return int32_t(best);
}

}  // namespace oracle
