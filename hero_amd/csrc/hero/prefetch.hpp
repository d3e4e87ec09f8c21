// prefetch.hpp -- reading a streaming GEMV's weights ahead of the GEMV, into
// the L2 of the XCD that will read them (and the last-level cache on the way).
//
// gemv_q8_stream_kernel assigns rows to its G workgroups in whole work items:
// in the interleaved form (K = 4096) item i is the 8-row group i and belongs
// to workgroup i % G; in the contiguous form workgroup g owns the items
// [U g / G, U (g + 1) / G) of U items of `unit` rows (8, or 64 for the SwiGLU
// epilogue). Workgroups of a launch are dispatched to the eight XCDs round
// robin, workgroup i on XCD i % 8, and each XCD has its own L2. A workgroup
// of an earlier kernel whose index is congruent to g modulo 8 therefore runs
// on the XCD of the GEMV's workgroup g, and the bytes it reads stay in that
// XCD's L2 for the GEMV. Prefetch workgroup p of P (P a multiple of 8, the
// first one at a multiple of 8 in its grid) reads for GEMV workgroups
// g = p, p + P, ... The loads land in a shared-memory sink (global_load_lds:
// no registers, up to 63 in flight per wave) that nothing reads.
#pragma once

#include "hero/device.hpp"

namespace hero {

// the matrix a GEMV will read: packed Q8_0 (N rows of K int8, then the fp16
// scales in 8-row groups); packed == nullptr: nothing to read
struct GemvPrefetch {
    const void* packed;
    int32_t N, K, G;  // rows, row length, the GEMV's workgroups
    int32_t unit;     // rows per work item (8 or 64)
    int32_t il;       // 1: interleaved items, 0: contiguous ranges
    int32_t part;     // of each GEMV workgroup's rows, the first part / 8 are read (1..8)
};
// up to three matrices, read in list order
struct PrefetchList {
    GemvPrefetch m[3];
};

constexpr int kPrefetchSinkBytes = 64 * 16;  // one wave's 16-byte loads

// 16-byte pieces of [p, p + bytes) over the workgroup's lanes: one
// instruction covers blockDim.x consecutive pieces in lane order (so the
// loads coalesce), the instructions run from the range's end to its start
__device__ __forceinline__ void prefetch_range(const int8_t* p, int64_t bytes, uint32_t sink) {
    const int64_t n = (bytes + 15) / 16, lanes = blockDim.x;  // pieces
    for (int64_t c = (n + lanes - 1) / lanes - 1; c >= 0; --c) {
        const int64_t k = c * lanes + threadIdx.x;
        if (k < n) lds_dma_b128(p + k * 16, sink);
    }
}

// what GEMV workgroup g reads of matrix m (its rows, then their scale
// groups; items in reverse order, so the first rows it needs are the last
// ones read), or share `sub` of `nsub` of it
__device__ __forceinline__ void prefetch_owner(const GemvPrefetch& m, int g, int sub, int nsub, uint32_t sink) {
    const int8_t* wq = static_cast<const int8_t*>(m.packed);
    const int64_t K = m.K, nb = K / 32, Npad = (int64_t(m.N) + 7) / 8 * 8;
    const int8_t* wd = wq + int64_t(m.N) * K;  // scales: [Npad / 8][nb][8] fp16
    const int64_t U = Npad / m.unit;
    auto rows = [&](int64_t r0, int64_t r1) {  // rows [r0, r1), r0 a multiple of 8
        r1 = r1 < m.N ? r1 : m.N;
        if (r1 <= r0) return;
        prefetch_range(wd + (r0 / 8) * nb * 16, ((r1 + 7) / 8 - r0 / 8) * nb * 16, sink);
        prefetch_range(wq + r0 * K, (r1 - r0) * K, sink);
    };
    if (m.il) {
        const int64_t items = g < U ? (U - g + m.G - 1) / m.G : 0;
        for (int64_t k = (items * m.part + 7) / 8 - 1; k >= 0; --k) {
            if (k % nsub != sub) continue;
            const int64_t i = g + k * m.G;
            rows(i * m.unit, (i + 1) * m.unit);
        }
    } else {
        const int64_t r0 = (U * g / m.G) * m.unit, r1 = (U * (g + 1) / m.G) * m.unit;
        const int64_t groups = ((r1 - r0) * m.part / 8 + 7) / 8;  // 8-row groups read ahead
        rows(r0 + 8 * (groups * sub / nsub), r0 + 8 * (groups * (sub + 1) / nsub));
    }
}

// Prefetch workgroup p of P: every matrix of the list, for GEMV workgroups
// p, p + P, ... (P < G) or share p / G of workgroup p % G (P >= G); then wait
// for the loads (the sink must not be reused while they land).
__device__ __forceinline__ void prefetch_gemvs(const PrefetchList& list, int p, int P, uint32_t sink) {
#pragma unroll
    for (int l = 0; l < 3; ++l) {
        const GemvPrefetch& m = list.m[l];
        if (!m.packed) continue;
        if (P >= m.G) {
            if (p < P / m.G * m.G) prefetch_owner(m, p % m.G, p / m.G, P / m.G, sink);
        } else {
            for (int g = p; g < m.G; g += P) prefetch_owner(m, g, 0, 1, sink);
        }
    }
    wait_vmcnt<0>();
}

}  // namespace hero
