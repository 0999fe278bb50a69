/*
 * MI355X backend extensions to the SPINNV2 runtime API.
 *
 * None of these has a counterpart in the reference runtime; they exist because
 * tensors now live in device memory and work is enqueued on a HIP stream:
 *
 *  - accessors for node kernels: the reference lets kernels read the private
 *    Spkv2Context directly (runtime/core/context.h:15-59); here the context is
 *    opaque and a third-party kernel registered with spkv2_register_kernel
 *    reads records, device data pointers, attrs, quant params and the stream
 *    through these functions;
 *  - device memory helpers, so a host tool or ctypes driver can bind device
 *    buffers without linking HIP itself;
 *  - execution controls: HIP-graph replay of the node loop and per-node GPU
 *    timing with HIP events;
 *  - test hooks that expose intermediate results the parity tests pin
 *    (the int32 accumulators of the INT8 convolution).
 */
#ifndef SPKV2_MI355X_H
#define SPKV2_MI355X_H

#include <stddef.h>
#include <stdint.h>
#include "spkv2_format.h"
#include "spkv2_runtime.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Return codes added by this backend. */
#define SPKV2_E_NOT_DEVICE_MEMORY (-8) /* caller memory the GPU cannot address */
#define SPKV2_E_NO_DEVICE (-30)        /* no HIP device / not prepared on a device */
#define SPKV2_E_HIP (-31)              /* a HIP API call failed; see spkv2_mi355x_last_error */
#define SPKV2_E_UNSUPPORTED (-32)      /* shape/attribute combination no device kernel covers */
#define SPKV2_E_QUANT (-33)            /* INT8 node without its quantization records */

/* ---- accessors for node kernels ---------------------------------------- */
const Spkv2TensorRecord *spkv2_ctx_tensor_record(const Spkv2Context *ctx, uint32_t tensor_id);
/* device pointer bound to the tensor (arena, weights, or a bound buffer) */
void *spkv2_ctx_tensor_data(const Spkv2Context *ctx, uint32_t tensor_id);
/* copy of the node's attribute record; -10 if out of bounds (reference kernel_common.c:90) */
int spkv2_ctx_get_attr(const Spkv2Context *ctx, const Spkv2NodeRecord *node, Spkv2AttrRecord *attr);
/* the context's hipStream_t; every kernel enqueues its work here */
void *spkv2_ctx_stream(const Spkv2Context *ctx);
/* quantization record of a tensor and its host-resident scale array (NULL if none) */
const Spkv2QuantParamRecord *spkv2_ctx_find_quant_param(const Spkv2Context *ctx, uint32_t tensor_id);
const float *spkv2_ctx_quant_scales(const Spkv2Context *ctx, const Spkv2QuantParamRecord *qp);
/* the record's int32 zero points, which follow its scales in the
 * quantization section (reference compiler/packager/spk_writer.py writes
 * them there; its runtime reads only the scales), NULL if out of range */
const int32_t *spkv2_ctx_quant_zero_points(const Spkv2Context *ctx, const Spkv2QuantParamRecord *qp);
/* per-node cache slot (device allocations made at prepare time) and its destructor */
int spkv2_ctx_node_cache(Spkv2Context *ctx, uint32_t node_id, void ***slot, void (***dtor)(void *));

/* ---- device memory helpers ---------------------------------------------- */
int spkv2_device_malloc(void **ptr, size_t size);
int spkv2_device_free(void *ptr);
int spkv2_device_memcpy_h2d(void *dst, const void *src, size_t size);
int spkv2_device_memcpy_d2h(void *dst, const void *src, size_t size);
int spkv2_device_memcpy_d2d(void *dst, const void *src, size_t size);
int spkv2_device_synchronize(void);
/* number of compute units and the gcnArchName of the current device */
int spkv2_device_info(int *compute_units, char *arch_name, size_t arch_name_size);
/* text of the last HIP error seen by the runtime on this thread ("" if none) */
const char *spkv2_mi355x_last_error(void);

/* FNV-1a-32 of a byte range: the package checksum the loader verifies
 * (reference runtime/core/loader.c:25-32), exported for package writers. */
uint32_t spkv2_fnv1a32(const void *data, size_t size);

/* IEEE half -> float widening of `count` values (unaligned buffers allowed):
 * what the loader applies to FP16 weight tensors, replacing the reference's
 * per-node promotion in runtime/kernels/optimized/conv/conv.c:961-978 and
 * mm/gemm.c:150-162 with one pass at load. */
void spkv2_mi355x_fp16_to_fp32(const void *src, void *dst, size_t count);

/* ---- execution controls --------------------------------------------------- */
/* 1: after one eager run, capture the node loop into a HIP graph and replay it
 * (re-captured after any bind_*; never used while profiling, fault injection
 * or a protection plan is active).  Default 0; env SPKV2_HIP_GRAPH=1 sets it. */
int spkv2_mi355x_set_graph_mode(Spkv2Context *ctx, int enable);
/* 1: bracket every node with HIP events on the context stream; the per-node
 * device times of each run accumulate until reset.  Env SPKV2_PROFILE=1 sets
 * it for every context (the reference profiling switch, executor.c:96-105). */
int spkv2_mi355x_set_profiling(Spkv2Context *ctx, int enable);
/* accumulated device milliseconds and run count of one node */
int spkv2_mi355x_node_time(Spkv2Context *ctx, uint32_t node_id, double *total_ms, uint32_t *count);
void spkv2_mi355x_reset_node_times(Spkv2Context *ctx);
/* name of the device kernel configuration the runtime chose for a node
 * ("conv_igemm_f32<128x128x16,splitk=1>", ...), for reports and tests */
int spkv2_mi355x_node_kernel_name(Spkv2Context *ctx, uint32_t node_id, char *buf, size_t buf_size);

/* ---- test hooks ------------------------------------------------------------ */
/* Re-run the integer part of an INT8 convolution node (quantize-on-load +
 * int8 MFMA GEMM) on the node's current input and copy the raw int32
 * accumulators, laid out [N][Cout][OH][OW], to host memory `out`.
 * Call after spkv2_run.  size must be N*Cout*OH*OW*4. */
int spkv2_mi355x_conv_int8_accumulators(Spkv2Context *ctx, uint32_t node_id, int32_t *out, size_t size);
/* 1: from the next spkv2_run on, every INT8 convolution node also stores its
 * raw int32 accumulators (from the very input the run quantized, handed-off
 * or not) into a device buffer of its own, which
 * spkv2_mi355x_conv_int8_accumulators then returns instead of re-running the
 * node; 0 frees the buffers.  Allocates one N*Cout*OH*OW*4-byte buffer per
 * INT8 conv node when enabled. */
int spkv2_mi355x_set_int8_capture(Spkv2Context *ctx, int enable);
/* No counterpart in the reference.  The same as
 * spkv2_mi355x_conv_int8_accumulators, for callers that cannot allocate
 * device memory (HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc): the accumulators are staged through a fixed 16 MiB device
 * array the library holds on each GPU for the life of the process, and the
 * call makes no hipMalloc / hipFree.  size above 16 MiB is refused with
 * SPKV2_E_UNSUPPORTED (spkv2_mi355x_last_error says why).  Every call on one
 * GPU shares that GPU's array: calls that overlap on one GPU race. */
int spkv2_mi355x_conv_int8_accumulators_noalloc(Spkv2Context *ctx, uint32_t node_id, int32_t *out, size_t size);
/* No counterpart in the reference (its INT8 mode keeps fp32 tensors between
 * nodes).  In the INT8 configuration with int8 tensors between nodes, copy
 * one int8 activation tensor (package dtype int8, role activation), laid out
 * NCHW, to host memory `out` (the runtime keeps it as zero-point-padded NHWC
 * on the device).  Call after spkv2_run.  size must be N*C*H*W; -1 for a
 * tensor that is not such a tensor. */
int spkv2_mi355x_read_int8_tensor(Spkv2Context *ctx, uint32_t tensor_id, int8_t *out, size_t size);

#ifdef __cplusplus
}
#endif

#endif /* SPKV2_MI355X_H */
