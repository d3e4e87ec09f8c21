// device.hpp -- small device-side building blocks shared by the kernels.
//
// Numerics contract (all kernels are built with -ffp-contract=off and the
// default correctly rounded fp32 division and square root):
//   * every fp32 expression below is evaluated in the same operation order as
//     the reference CPU code it replaces, one rounding per operation;
//   * exp and log1p return exactly what the reference's glibc expf / log1pf
//     return (hero/libm.hpp), so results that depend on them are bit-identical
//     too.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "hero/fp16.hpp"
#include "hero/libm.hpp"

namespace hero {

constexpr int kWave = 64;

__device__ __forceinline__ float exp_f32(float x) { return expf_glibc(x); }
__device__ __forceinline__ float log1p_f32(float x) { return log1pf_glibc(x); }

// nm/src/core.hpp:579
__device__ __forceinline__ float sigmoid_f32(float x) { return 1.f / (1.f + exp_f32(-x)); }
// nm/src/components.hpp:105 -- x/(1+e^-x), not x*sigmoid(x)
__device__ __forceinline__ float silu_f32(float x) { return x / (1.f + exp_f32(-x)); }
// nm/src/recurrent.hpp:35
__device__ __forceinline__ float softplus_f32(float x) { return x > 20.f ? x : log1p_f32(exp_f32(x)); }
// gelu_pytorch_tanh (nm/src/components.hpp:73-81):
// 0.5 v (1 + tanh(0.7978845608 (v + 0.044715 v^3))), left to right
__device__ __forceinline__ float gelu_tanh_f32(float v) { return 0.5f * v * (1.f + tanhf_glibc(0.7978845608f * (v + 0.044715f * v * v * v))); }

// 0, in a vector register the compiler cannot see through: added to an
// address, it keeps a load of a wave-uniform value a per-lane vector load
// (no scalar copy, no early wait for it)
__device__ __forceinline__ uint32_t lane_zero() {
    uint32_t z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    return z;
}

// The same functions with expf's 32-entry table read from shared memory
// (filled by fill_exp_table before a barrier). The plain forms read it from
// global memory: behind other loads still in flight (vector memory operations
// retire in order) each call would wait for all of them.
struct ExpTab {
    const uint64_t* t;
    __device__ __forceinline__ float exp(float x) const { return expf_glibc_with(x, [p = t](int i) { return p[i]; }); }
    __device__ __forceinline__ float sigmoid(float x) const { return 1.f / (1.f + exp(-x)); }
    __device__ __forceinline__ float silu(float x) const { return x / (1.f + exp(-x)); }
    __device__ __forceinline__ float softplus(float x) const { return x > 20.f ? x : log1p_f32(exp(x)); }
};
__device__ __forceinline__ void fill_exp_table(uint64_t* lds, int tid) {
    if (tid < 32) lds[tid] = exp2_table(tid);
}

__device__ __forceinline__ float half_bits_to_f32(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return float(v);
}

// Raw buffer accesses: a load at an offset at or past the buffer's size reads
// 0 and a store there is dropped, so a kernel can give invalid rows or padded
// steps an out-of-range offset instead of a branch. Every loop iteration then
// issues the same memory instructions, which lets the compiler wait for
// exactly the oldest loads instead of all of them.
constexpr uint32_t kOOB = 0x80000000u;       // beyond every buffer (sizes < 2 GiB)
constexpr uint32_t kBufWord3 = 0x00020000u;  // raw dword buffer, gfx9 family

typedef int v4b_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, int(bytes), int(kBufWord3));
}
__device__ __forceinline__ int4 load_b128(__amdgpu_buffer_rsrc_t b, uint32_t off) {
    const v4b_t v = __builtin_amdgcn_raw_buffer_load_b128(b, off, 0, 0);
    return make_int4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float load_f32(__amdgpu_buffer_rsrc_t b, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(b, off, 0, 0));
}

// Loads straight into shared memory (global_load_lds): every lane's 16 or 4
// bytes land at lds_base + lane * size, lds_base uniform over the wave. They
// are issued from inline assembly so the compiler does not track them: it
// would otherwise wait for every such load in flight before any shared-memory
// read. The caller waits for them itself (wait_vmcnt) and publishes them with
// a barrier. M0 carries the base and is restored afterwards.
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
    return uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)(p)));
}
__device__ __forceinline__ void lds_dma_b128(const void* g, uint32_t lds_base) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved) : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_base)) : "memory");
}
__device__ __forceinline__ void lds_dma_b32(const void* g, uint32_t lds_base) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved) : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_base)) : "memory");
}

// Sixteen 16-byte shared-memory reads (256 consecutive bytes from lds_addr)
// the compiler does not track (inline assembly): the results may only be used
// after a barrier or an explicit lgkmcnt wait. For reads issued one pipeline
// step ahead of their use, where the compiler's own counted waits would hold
// the current step's work until they land.
__device__ __forceinline__ void lds_read_b128x16_untracked(uint32_t lds_addr, float4 (&dst)[16]) {
    typedef float v4f_t __attribute__((ext_vector_type(4)));
    v4f_t v[16];
#define HERO_LDS_RD(i) asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v[i]) : "v"(lds_addr), "i"(16 * (i)) : "memory")
    HERO_LDS_RD(0); HERO_LDS_RD(1); HERO_LDS_RD(2); HERO_LDS_RD(3); HERO_LDS_RD(4); HERO_LDS_RD(5); HERO_LDS_RD(6); HERO_LDS_RD(7);
    HERO_LDS_RD(8); HERO_LDS_RD(9); HERO_LDS_RD(10); HERO_LDS_RD(11); HERO_LDS_RD(12); HERO_LDS_RD(13); HERO_LDS_RD(14); HERO_LDS_RD(15);
#undef HERO_LDS_RD
#pragma unroll
    for (int i = 0; i < 16; ++i) dst[i] = make_float4(v[i].x, v[i].y, v[i].z, v[i].w);
}

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt in bits 3:0 and 15:14; expcnt and
// lgkmcnt left at their maxima, i.e. not waited for): at most N vector memory
// operations of this wave still outstanding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// 4-way int8 dot product into an int32 accumulator (v_dot4_i32_i8), exact.
__device__ __forceinline__ int dot4_i8(int a, int b, int acc) { return __builtin_amdgcn_sdot4(a, b, acc, false); }

__device__ __forceinline__ int dot16_i8(const int4& w, const int4& x, int acc) {
    acc = dot4_i8(w.x, x.x, acc);
    acc = dot4_i8(w.y, x.y, acc);
    acc = dot4_i8(w.z, x.z, acc);
    acc = dot4_i8(w.w, x.w, acc);
    return acc;
}

// Quantize one 32-value block held 8 per lane by 4 consecutive lanes
// (nm/src/quant_i8.hpp:70-80): amax over the block, d = amax/127,
// id = 1/d (0 if d == 0), q = roundf(x*id), d stored through the reference
// fp16 encoder. Returns the 8 int8 values packed in two ints; *dh receives
// the fp16 bits of d (identical on all four lanes).
__device__ __forceinline__ int2 quantize8_in_quad(const float (&x)[8], uint16_t* dh) {
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(x[j]));
    // max over the 4 lanes of the quad (exact: max is order independent)
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    const float d = amax / 127.f;
    const float id = d != 0.f ? 1.f / d : 0.f;
    *dh = fp32_to_fp16_ref(d);
    int packed[2] = {0, 0};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int q = int(roundf(x[j] * id));
        packed[j / 4] |= (q & 0xFF) << (8 * (j % 4));
    }
    return make_int2(packed[0], packed[1]);
}

// The value of lane ^ 1 (DPP quad_perm [1,0,3,2]; all lanes active).
__device__ __forceinline__ int pair_swap_i32(int v) { return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false); }
__device__ __forceinline__ float pair_swap_f32(float v) { return __int_as_float(pair_swap_i32(__float_as_int(v))); }

// quantize_row_q8_0 (nm/src/quant_i8.hpp:70-80) for one 32-value block held
// 16 per lane by an even/odd lane pair: the same rules as quantize8_in_quad.
// Returns the lane's 16 int8 values packed in an int4; *dh receives the fp16
// bits of d (identical on both lanes). All lanes of the wave must be active.
__device__ __forceinline__ int4 quantize16_in_pair(const float (&x)[16], uint16_t* dh) {
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) amax = fmaxf(amax, fabsf(x[j]));
    amax = fmaxf(amax, pair_swap_f32(amax));
    const float d = amax / 127.f;
    const float id = d != 0.f ? 1.f / d : 0.f;
    *dh = fp32_to_fp16_ref(d);
    int packed[4] = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int q = int(roundf(x[j] * id));
        packed[j / 4] |= (q & 0xFF) << (8 * (j % 4));
    }
    return make_int4(packed[0], packed[1], packed[2], packed[3]);
}

// (query head, channel part) of workgroup x of a Hq x parts grid. Workgroups
// go to the eight XCDs round robin by index; when the (K/V head, part) pairs
// come in whole eights, the group's query heads of one part get indices equal
// mod 8, so they run on one XCD and read their shared value rows through one
// L2 (in index order they split over two, and the values were fetched from
// HBM about twice).
__device__ __forceinline__ void head_part_of(int x, int Hq, int Hkv, int parts, int& h, int& part) {
    const int group = Hq / Hkv, pairs = Hkv * parts;
    if (pairs % 8 == 0) {
        const int r = x / 8, pp = 8 * (r / group) + x % 8;  // pair pp = K/V head * parts + part
        part = pp % parts;
        h = (pp / parts) * group + r % group;
    } else {
        h = x / parts;
        part = x % parts;
    }
}

}  // namespace hero
