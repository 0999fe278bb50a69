// Device-side helpers shared by the node kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../runtime/context.hpp"
#include "spkv2_mi355x.h"

namespace spk::kern {

typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef int intx4 __attribute__((ext_vector_type(4)));
typedef unsigned uintx4 __attribute__((ext_vector_type(4)));
typedef int intx16 __attribute__((ext_vector_type(16)));

// Fused activation codes of the SPK attr record (0 none, 1 Relu, 2 SiLU),
// as the reference applies them (kernel_common.c:100-108).  SiLU
// v / (1 + exp(-v)) is evaluated with the hardware exponential (v_exp_f32
// on v * log2(e)) and reciprocal (v_rcp_f32), within a few ulp of the
// reference's expf and division for |v| up to ~20 (relative error below
// ~|v| * 2^-24 from the exponent's rounding) and with its special values:
// +inf -> +inf, -inf -> NaN, NaN -> NaN, v below ~-88.7 -> -0.
__device__ __forceinline__ float apply_act(float v, int act) {
    if (act == 1) return v > 0.0f ? v : 0.0f;
    if (act == 2) return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v));
    return v;
}

inline size_t elem_count(const Spkv2TensorRecord *r) {
    size_t n = 1;
    for (uint16_t i = 0; i < r->rank; i++) n *= r->shape[i];
    return n;
}

inline const Spkv2TensorRecord *rec(const Spkv2Context *ctx, uint32_t id) { return &ctx->tensor_records[id]; }

template <typename T>
inline T *dptr(const Spkv2Context *ctx, uint32_t id) {
    return reinterpret_cast<T *>(ctx->tensors[id].data);
}

inline int launch_status(const char *what) {
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) return 0;
    set_last_error(what, e);
    return SPKV2_E_HIP;
}

inline unsigned blocks_for(size_t n, unsigned threads) {
    size_t b = (n + threads - 1) / threads;
    return static_cast<unsigned>(b == 0 ? 1 : b);
}

// A grid-stride loop bound: enough blocks to fill the GPU several times over,
// the kernel loops for the rest.
inline unsigned grid_for(size_t n, unsigned threads) {
    size_t b = (n + threads - 1) / threads;
    if (b > 65536) b = 65536;
    return static_cast<unsigned>(b == 0 ? 1 : b);
}

inline void set_kernel_name(Spkv2Context *ctx, const Spkv2NodeRecord *node, const std::string &name) {
    if (node->id < ctx->node_kernel_names.size()) ctx->node_kernel_names[node->id] = name;
}

}  // namespace spk::kern
