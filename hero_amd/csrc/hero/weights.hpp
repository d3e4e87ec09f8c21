// weights.hpp -- host-side helpers of the model loaders: F32/F16 vectors out
// of a GGUF file, uploads, and the packer that copies Q8_0 (and K-quant)
// tensors into the device layouts of hero/kernels.hpp.
#pragma once
#include <cstring>
#include <string>
#include <vector>

#include "hero/errors.hpp"
#include "hero/fp16.hpp"
#include "hero/gguf.hpp"
#include "hero/kernels.hpp"
#include "hero/model.hpp"
#include "hero_kernels.h"

namespace hero {

// a malformed or unsupported checkpoint
inline void loader_expect(bool ok, const std::string& what) {
    if (!ok) throw Error(HERO_EIO, "loader: " + what);
}

inline std::vector<float> host_vector(const GgufFile& g, const std::string& name, int64_t n) {
    const GgufFile::Tensor& t = g.require(name);
    loader_expect(int64_t(t.nelem) == n, name + " has length " + std::to_string(t.nelem) + ", expected " + std::to_string(n));
    std::vector<float> v(static_cast<size_t>(n));
    if (t.type == 0) {
        std::memcpy(v.data(), t.data, size_t(n) * 4);
    } else if (t.type == 1) {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(t.data);
        for (int64_t i = 0; i < n; ++i) v[size_t(i)] = fp16_to_fp32_ref(h[i]);
    } else {
        loader_expect(false, name + " must be F32 or F16");
    }
    return v;
}

inline DeviceBuffer upload(const std::vector<float>& v) {
    DeviceBuffer b(v.size() * sizeof(float));
    hip_check(hipMemcpy(b.get(), v.data(), v.size() * sizeof(float), hipMemcpyHostToDevice), "upload");
    return b;
}

struct WeightPacker {
    DeviceBuffer staging;
    hipStream_t stream;
    int64_t* counter;
    // copy one Q8_0 GGUF tensor [K, rows] into rows [row0, row0+rows) of a packed matrix
    void put(const GgufFile& g, const std::string& name, DeviceBuffer& dst, int64_t n_total, int64_t K, int64_t row0, int64_t rows, int64_t interleave = 0) {
        const GgufFile::Tensor& t = g.require(name);
        loader_expect(t.dims.size() == 2 && int64_t(t.dims[0]) == K && int64_t(t.dims[1]) == rows, name + " has the wrong shape");
        loader_expect(t.type == 8, name + " must be Q8_0");
        if (staging.bytes() < t.nbytes) {
            hip_check(hipStreamSynchronize(stream), "pack sync");
            staging = DeviceBuffer(t.nbytes);
        }
        hip_check(hipStreamSynchronize(stream), "pack sync");
        hip_check(hipMemcpy(staging.get(), t.data, t.nbytes, hipMemcpyHostToDevice), "weight upload");
        launch_pack_q8(staging.get(), dst.get(), n_total, K, row0, rows, stream, interleave);
        check_launch("pack");
    }
    DeviceBuffer alloc(int64_t n, int64_t K) {
        *counter += packed_q8_bytes(n, K);
        return DeviceBuffer(size_t(packed_q8_bytes(n, K)));
    }
    // one linear weight in its own type: Q8_0 packed as above, Q4_K / Q6_K
    // regrouped (launch_kquant_pack), Q5_K as stored
    TypedLinear typed(const GgufFile& g, const std::string& name, int64_t K, int64_t N) {
        const GgufFile::Tensor& t = g.require(name);
        loader_expect(t.dims.size() == 2 && int64_t(t.dims[0]) == K && int64_t(t.dims[1]) == N, name + " has the wrong shape");
        TypedLinear L;
        L.type = int(t.type);
        L.N = N;
        L.K = K;
        if (t.type == 8) {
            loader_expect(K % 32 == 0, name + ": In not divisible by the Q8_0 block length");
            L.w = alloc(N, K);
            put(g, name, L.w, N, K, 0, N);
            return L;
        }
        loader_expect(t.type == 12 || t.type == 13 || t.type == 14, name + " has ggml type " + std::to_string(t.type) + "; this build runs Q8_0, Q4_K, Q5_K and Q6_K weights");
        loader_expect(K % 256 == 0, name + ": In not divisible by the K-quant block length");
        loader_expect(K <= kquant_max_k(L.type), name + ": In too large for this type");
        if (staging.bytes() < t.nbytes) {
            hip_check(hipStreamSynchronize(stream), "pack sync");
            staging = DeviceBuffer(t.nbytes);
        }
        hip_check(hipStreamSynchronize(stream), "pack sync");
        hip_check(hipMemcpy(staging.get(), t.data, t.nbytes, hipMemcpyHostToDevice), "weight upload");
        const int64_t bytes = kquant_packed_bytes(L.type, N, K);
        L.w = DeviceBuffer(size_t(bytes));
        *counter += bytes;
        launch_kquant_pack(L.type, staging.get(), L.w.get(), N, K, stream);
        check_launch("pack");
        return L;
    }
};

}  // namespace hero
