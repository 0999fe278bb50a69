/*
 * SPINNV2 runtime C API, implemented by libspkv2_mi355x.so on one MI355X GPU.
 *
 * Every entry point below replaces the reference function of the same name
 * (runtime/include/spkv2_runtime.h:42-70); names, argument meaning and return
 * codes are unchanged, so tools and ctypes drivers written against the
 * reference (runtime/tools/spkv2_run.c, spkv2_bench.c,
 * research/reliability/runtime_driver.py:44-128) bind to this library as is.
 *
 * What differs is where memory lives:
 *   - the activation arena and the scratch arena are device memory;
 *   - weights are uploaded, and repacked per kernel, once in spkv2_prepare;
 *   - spkv2_set_input / spkv2_get_output copy host<->device;
 *   - spkv2_bind_input / spkv2_bind_output take DEVICE pointers (hipMalloc,
 *     or pinned host memory from hipHostMalloc, which the GPU can address);
 *   - a caller-supplied arena / scratch passed to spkv2_prepare* must be
 *     device memory as well (-8 otherwise);
 *   - spkv2_run enqueues every node on the context's HIP stream and returns
 *     after that stream has drained, so it is synchronous like the reference.
 *
 * Return codes (reference semantics): 0 ok; -1 bad argument / allocation;
 * load: -2 magic/version, -3 section bounds, -4 missing section, -5/-6
 * checksum; prepare: -2 arena too small, -3 weight out of bounds, -4 tensor
 * out of bounds; run: -5 unbound tensor, -99 no kernel for a node, other
 * negative codes from the kernel.  Codes added by this backend are listed in
 * spkv2_mi355x.h.
 */
#ifndef SPKV2_RUNTIME_H
#define SPKV2_RUNTIME_H

#include <stddef.h>
#include <stdint.h>
#include "spkv2_format.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct Spkv2Context Spkv2Context;

typedef struct {
    uint32_t node_id;
    uint32_t tensor_id;
    uint64_t element_index;
    uint8_t bit_index;
    uint32_t invocation_index;
    uint64_t seed;
    int enabled;
} Spkv2FaultEvent;

typedef struct {
    uint64_t injected_faults;
    uint64_t detected_faults;
    uint64_t recovered_faults;
    uint64_t unrecovered_faults;
    uint64_t rerun_count;
} Spkv2ReliabilityStats;

typedef struct {
    uint32_t node_id;
    uint32_t tensor_id;
    float observed_min;
    float observed_max;
    uint64_t observations;
} Spkv2RangeObservation;

/* Node kernel plug-in ABI (reference: runtime/include/spkv2_runtime.h:40).
 * On this runtime a kernel reads tensors through the accessors in
 * spkv2_mi355x.h; tensor data pointers are device pointers and work must be
 * enqueued on spkv2_ctx_stream(ctx).  `scratch` is device memory. */
typedef int (*Spkv2NodeKernelFn)(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *scratch);

/* reference: runtime/core/version.c:3 */
const char *spkv2_runtime_version(void);

/* reference: runtime/core/loader.c:105 */
int spkv2_load_file(const char *path, Spkv2Context **out_ctx);
/* reference: runtime/core/loader.c:140 (the blob must outlive the context) */
int spkv2_load_memory(const void *data, size_t size, Spkv2Context **out_ctx);
/* reference: runtime/core/executor.c:189 */
int spkv2_prepare(Spkv2Context *ctx, void *arena, size_t arena_size);
/* reference: runtime/core/executor.c:193.  The scratch arena (device memory,
 * at least header.scratch_arena_bytes, else -2) also holds the conv / Gemm
 * workspaces of mi355x packages (padded input copies, split-K partials): a
 * plan that fits its kernel spec's scratch_bytes runs there, so the runtime
 * allocates workspace only for plans that outgrow their spec. */
int spkv2_prepare_with_scratch(Spkv2Context *ctx, void *arena, size_t arena_size, void *scratch,
                               size_t scratch_size);
/* reference: runtime/core/executor.c:249 (host -> device copy) */
int spkv2_set_input(Spkv2Context *ctx, int index, const void *data, size_t size);
/* reference: runtime/core/executor.c:265 (data: device pointer) */
int spkv2_bind_input(Spkv2Context *ctx, int index, void *data, size_t size);
/* reference: runtime/core/executor.c:304 (data: device pointer) */
int spkv2_bind_output(Spkv2Context *ctx, int index, void *data, size_t size);
/* reference: runtime/core/executor.c:326 */
int spkv2_get_output_size(Spkv2Context *ctx, int index, size_t *out_size);
/* reference: runtime/core/executor.c:315 (device -> host copy) */
int spkv2_get_output(Spkv2Context *ctx, int index, void *data, size_t size);
/* reference: runtime/core/executor.c:500 */
int spkv2_run(Spkv2Context *ctx);
/* reference: runtime/core/executor.c:335 */
int spkv2_set_fault_event(Spkv2Context *ctx, const Spkv2FaultEvent *event);
/* reference: runtime/core/executor.c:342 */
void spkv2_clear_fault_event(Spkv2Context *ctx);
/* reference: runtime/core/executor.c:347 */
int spkv2_get_reliability_stats(Spkv2Context *ctx, Spkv2ReliabilityStats *stats);
/* reference: runtime/core/executor.c:353 */
void spkv2_reset_reliability_stats(Spkv2Context *ctx);
/* reference: runtime/core/executor.c:358 */
int spkv2_get_range_observation(Spkv2Context *ctx, uint32_t node_id, Spkv2RangeObservation *observation);
/* reference: runtime/core/executor.c:364 */
void spkv2_reset_range_observations(Spkv2Context *ctx);
/* reference: runtime/core/executor.c:539 (per-node GPU time from HIP events) */
void spkv2_profile_dump(void);
/* reference: runtime/core/loader.c:284 */
void spkv2_free(Spkv2Context *ctx);

/* reference: runtime/kernels/reference/kernels.c:18 (64 user slots; -1 NULL fn, -2 full;
 * a user entry wins ties against the built-in device kernels, all priority 0) */
int spkv2_register_kernel(uint16_t op_type, uint16_t backend, uint16_t kernel_kind, Spkv2NodeKernelFn fn,
                          int priority);
/* reference: runtime/kernels/reference/kernels.c:57 */
void spkv2_clear_user_kernels(void);

#ifdef __cplusplus
}
#endif

#endif /* SPKV2_RUNTIME_H */
