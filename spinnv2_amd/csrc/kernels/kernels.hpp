// Built-in device node kernels of the MI355X backend.
//
// Each `*_run` has the plug-in signature of Spkv2NodeKernelFn and enqueues HIP
// work on the context stream; each `*_prepare` runs once per node inside
// spkv2_prepare (weight upload/repack, launch planning) and reports the
// runtime workspace it needs.
#pragma once

#include <cstddef>

#include "../runtime/context.hpp"

namespace spk::kern {

using RunFn = int (*)(Spkv2Context *, const Spkv2NodeRecord *, void *);
using PrepFn = int (*)(Spkv2Context *, const Spkv2NodeRecord *, size_t *workspace_bytes);

// convolution: fp32 MFMA implicit GEMM (group 1), direct kernels (grouped,
// fallback), int8 MFMA implicit GEMM when the weight tensor is int8
int conv_run(Spkv2Context *, const Spkv2NodeRecord *, void *);
int conv_prepare(Spkv2Context *, const Spkv2NodeRecord *, size_t *);
int conv_direct_run(Spkv2Context *, const Spkv2NodeRecord *, void *);
// int8 accumulator test hook
int conv_int8_accumulators(Spkv2Context *, const Spkv2NodeRecord *, int32_t *dev_out);

int gemm_run(Spkv2Context *, const Spkv2NodeRecord *, void *);
int gemm_prepare(Spkv2Context *, const Spkv2NodeRecord *, size_t *);
int matmul_run(Spkv2Context *, const Spkv2NodeRecord *, void *);

int binary_run(Spkv2Context *, const Spkv2NodeRecord *, void *);  // Add Mul Sub Div Mod
int unary_run(Spkv2Context *, const Spkv2NodeRecord *, void *);   // Relu Sigmoid Clip LeakyRelu
int copy_run(Spkv2Context *, const Spkv2NodeRecord *, void *);    // Flatten Reshape Cast Unsqueeze
int concat_run(Spkv2Context *, const Spkv2NodeRecord *, void *);
int maxpool_run(Spkv2Context *, const Spkv2NodeRecord *, void *);
int maxpool_prepare(Spkv2Context *, const Spkv2NodeRecord *, size_t *);
int avgpool_run(Spkv2Context *, const Spkv2NodeRecord *, void *);
int global_avgpool_run(Spkv2Context *, const Spkv2NodeRecord *, void *);
int softmax_run(Spkv2Context *, const Spkv2NodeRecord *, void *);
int reduce_run(Spkv2Context *, const Spkv2NodeRecord *, void *);  // ReduceMean ReduceMax
int resize_run(Spkv2Context *, const Spkv2NodeRecord *, void *);
// indexing / layout (tensor_ops.hip)
int transpose_run(Spkv2Context *, const Spkv2NodeRecord *, void *);
int tile_run(Spkv2Context *, const Spkv2NodeRecord *, void *);
int split_run(Spkv2Context *, const Spkv2NodeRecord *, void *);
int slice_run(Spkv2Context *, const Spkv2NodeRecord *, void *);
int gather_run(Spkv2Context *, const Spkv2NodeRecord *, void *);
int gather_elements_run(Spkv2Context *, const Spkv2NodeRecord *, void *);
int topk_run(Spkv2Context *, const Spkv2NodeRecord *, void *);

// y[o * y_stride + j] = x[x_base + o * x_stride + j], o < outer, j < block
// (float elements; Concat, Split, Slice)
int strided_block_copy(hipStream_t s, const float *x, float *y, size_t outer, size_t block, size_t x_stride,
                       size_t x_base, size_t y_stride);
// The copies of several blocks with the same `outer` (a Split's outputs, a
// Concat's inputs) in one launch: segment k copies
// y_k[o * y_stride_k + j] = x_k[x_base_k + o * x_stride_k + j], j < block_k.
struct CopySeg {
    const float *x;
    float *y;
    size_t block, x_stride, x_base, y_stride;
};
int multi_block_copy(hipStream_t s, const CopySeg *segs, int count, size_t outer);

// channel-slice views of Concats at batch > 1 (views.cpp), after every
// node's prepare
int setup_concat_views(Spkv2Context *ctx);
// int8 conv -> MaxPool -> int8 convs: the conv hands the pool int8 (eltwise.hip)
int setup_pool_int8_inputs(Spkv2Context *ctx);

// INT8 configuration with int8 tensors between nodes (q8.hip): the int8
// activation tensors' buffers (before the node prepares), the check that
// built-in kernels run every node touching one (after them), and the
// MaxPool / spatial-mean kernels over them
int setup_q8_tensors(Spkv2Context *ctx);
int check_q8_winners(const Spkv2Context *ctx);
int q8_params(const Spkv2Context *ctx, uint32_t tensor_id, float *scale, int *zp);
int maxpool_q8_run(Spkv2Context *ctx, const Spkv2NodeRecord *node);
int mean_q8_run(Spkv2Context *ctx, const Spkv2NodeRecord *node);

// reliability helpers used by the executor
int flip_bit(hipStream_t s, void *data, uint64_t element, uint32_t bit);
int minmax(hipStream_t s, const float *x, size_t n, float *dev_out4);
int compare_bytes(hipStream_t s, const void *a, const void *b, size_t n, uint32_t *dev_flag);
int fill_u32(hipStream_t s, uint32_t *p, size_t n, uint32_t v);

}  // namespace spk::kern
