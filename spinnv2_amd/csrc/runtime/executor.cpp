// Prepare, IO, the node loop, reliability hooks and profiling.
//
// Semantics follow the reference executor (runtime/core/executor.c:189-541);
// the device boundary sits in prepare:
//   - the activation arena and the scratch arena are device allocations
//     (zero-filled like the reference's calloc) or caller device buffers;
//   - the weight section is uploaded once; node prepare hooks then repack
//     what their kernels need (conv weight panels, im2col offset tables);
//   - every tensor is bound exactly as planned by the compiler: weights at
//     weights + data_offset, external tensors unbound, everything else at
//     arena + data_offset, so in-place and Concat aliases carry over.
// spkv2_run enqueues each node on the context stream and waits for the stream
// at the end; with graph mode on, the whole loop is captured once into a HIP
// graph and replayed.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "../kernels/kernels.hpp"
#include "context.hpp"
#include "spkv2_mi355x.h"
#include "spkv2_platform.h"

namespace spk {

static thread_local std::string g_last_error;

void set_last_error(const char *what, hipError_t err) {
    g_last_error = std::string(what) + ": " + hipGetErrorString(err);
}
void set_last_error_text(const std::string &text) { g_last_error = text; }

int hip_check(hipError_t err, const char *what) {
    if (err == hipSuccess) return 0;
    set_last_error(what, err);
    return SPKV2_E_HIP;
}

}  // namespace spk

namespace {

using spk::hip_check;

bool env_flag(const char *name) {
    const char *v = getenv(name);
    return v && v[0] && v[0] != '0';
}

// Device-addressable: hipMalloc'd memory or pinned host memory.
bool is_device_accessible(const void *p) {
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged ||
           (attr.type == hipMemoryTypeHost && attr.devicePointer != nullptr);
}

int alloc_zeroed(uint8_t **out, size_t bytes, hipStream_t s) {
    *out = nullptr;
    if (bytes == 0) return 0;
    if (int rc = hip_check(hipMalloc(reinterpret_cast<void **>(out), bytes), "hipMalloc")) return rc;
    return hip_check(hipMemsetAsync(*out, 0, bytes, s), "hipMemsetAsync");
}

void drop_graph(Spkv2Context *ctx) {
    if (ctx->graph_exec) {
        (void)hipGraphExecDestroy(ctx->graph_exec);
        ctx->graph_exec = nullptr;
    }
    ctx->graph_epoch = 0;
}

const Spkv2TensorRecord *input_record(Spkv2Context *ctx, int index, uint32_t *tid) {
    int current = 0;
    for (uint32_t i = 0; i < ctx->header.num_tensors; i++) {
        if (ctx->tensor_records[i].role != SPKV2_ROLE_INPUT) continue;
        if (current == index) {
            *tid = i;
            return &ctx->tensor_records[i];
        }
        current++;
    }
    return nullptr;
}

// reference executor.c:281-302
int output_tensor_id(const Spkv2Context *ctx, int index, uint32_t *tid) {
    if (!ctx || !tid || index < 0) return -1;
    if (ctx->output_ids && static_cast<size_t>(index) < ctx->output_count) {
        uint32_t id = ctx->output_ids[index];
        if (id >= ctx->header.num_tensors || ctx->tensor_records[id].role != SPKV2_ROLE_OUTPUT) return -3;
        *tid = id;
        return 0;
    }
    int current = 0;
    for (uint32_t i = 0; i < ctx->header.num_tensors; i++) {
        if (ctx->tensor_records[i].role != SPKV2_ROLE_OUTPUT) continue;
        if (current == index) {
            *tid = i;
            return 0;
        }
        current++;
    }
    return -3;
}

// ---------------------------------------------------------------- reliability

const Spkv2ProtectionRecord *protection_for(const Spkv2Context *ctx, uint32_t node_id) {
    for (size_t i = 0; i < ctx->protection_count; i++)
        if (ctx->protection_records[i].node_id == node_id) return &ctx->protection_records[i];
    return nullptr;
}

// Bit flip in one fp32 output element after the node's n-th invocation
// (reference executor.c:377-398), done by a one-thread device kernel.
int maybe_inject_fault(Spkv2Context *ctx, const Spkv2NodeRecord *node) {
    const Spkv2FaultEvent &ev = ctx->fault_event;
    if (!ev.enabled || node->id != ev.node_id) return 0;
    if (node->id >= ctx->node_count || !ctx->invocations) return -20;
    ctx->invocations[node->id]++;
    if (ctx->invocations[node->id] != ev.invocation_index) return 0;
    if (ev.tensor_id >= ctx->header.num_tensors) return -21;
    const Spkv2TensorRecord *t = &ctx->tensor_records[ev.tensor_id];
    bool is_output = false;
    for (uint16_t i = 0; i < node->output_count; i++)
        if (node->outputs[i] == ev.tensor_id) is_output = true;
    if (!is_output || t->dtype != SPKV2_DTYPE_FP32) return -22;
    if (ev.element_index >= t->size_bytes / 4) return -23;
    if (int rc = spk::kern::flip_bit(ctx->stream, ctx->tensors[ev.tensor_id].data, ev.element_index, ev.bit_index))
        return rc;
    ctx->stats.injected_faults++;
    return 0;
}

int execute_once(Spkv2Context *ctx, const Spkv2NodeRecord *node) {
    int rc = spk::execute_node(ctx, node);
    if (rc != 0) return rc;
    return maybe_inject_fault(ctx, node);
}

// Device min / max / non-finite count of a tensor, read back to the host.
int tensor_range(Spkv2Context *ctx, uint32_t tid, float out[3]) {
    const Spkv2TensorRecord *t = &ctx->tensor_records[tid];
    size_t n = static_cast<size_t>(t->size_bytes / 4);
    if (int rc = spk::kern::minmax(ctx->stream, reinterpret_cast<const float *>(ctx->tensors[tid].data), n,
                                   ctx->dev_minmax))
        return rc;
    float host[4];
    if (int rc = hip_check(hipMemcpyAsync(host, ctx->dev_minmax, sizeof(host), hipMemcpyDeviceToHost, ctx->stream),
                           "hipMemcpyAsync"))
        return rc;
    if (int rc = hip_check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize")) return rc;
    out[0] = host[0];
    out[1] = host[1];
    out[2] = host[2];
    return 0;
}

int bytes_equal(Spkv2Context *ctx, const void *a, const void *b, size_t n, bool *equal) {
    if (int rc = spk::kern::compare_bytes(ctx->stream, a, b, n, ctx->dev_flag)) return rc;
    uint32_t flag = 1;
    if (int rc = hip_check(hipMemcpyAsync(&flag, ctx->dev_flag, 4, hipMemcpyDeviceToHost, ctx->stream),
                           "hipMemcpyAsync"))
        return rc;
    if (int rc = hip_check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize")) return rc;
    *equal = flag == 0;
    return 0;
}

int d2d(Spkv2Context *ctx, void *dst, const void *src, size_t n) {
    return hip_check(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, ctx->stream), "hipMemcpyAsync");
}

// reference executor.c:445-498
int execute_protected(Spkv2Context *ctx, const Spkv2NodeRecord *node) {
    const Spkv2ProtectionRecord *rec = protection_for(ctx, node->id);
    if (!rec || rec->mode == SPKV2_PROTECT_NONE) return execute_once(ctx, node);
    if (rec->tensor_id >= ctx->header.num_tensors || node->output_count != 1 || node->outputs[0] != rec->tensor_id)
        return -24;

    if (rec->mode == SPKV2_PROTECT_RANGE_GUARD_RERUN) {
        auto in_range = [&](const float r[3]) {
            return r[2] == 0.0f && r[0] >= rec->lower_bound && r[1] <= rec->upper_bound;
        };
        int rc = execute_once(ctx, node);
        if (rc != 0) return rc;
        float r[3];
        if ((rc = tensor_range(ctx, rec->tensor_id, r))) return rc;
        if (rec->node_id < ctx->node_count && ctx->tensor_records[rec->tensor_id].size_bytes >= 4) {
            Spkv2RangeObservation &o = ctx->ranges[rec->node_id];
            o.node_id = rec->node_id;
            o.tensor_id = rec->tensor_id;
            if (o.observations == 0) {
                o.observed_min = r[0];
                o.observed_max = r[1];
            } else {
                if (r[0] < o.observed_min) o.observed_min = r[0];
                if (r[1] > o.observed_max) o.observed_max = r[1];
            }
            o.observations++;
        }
        if (in_range(r)) return 0;
        ctx->stats.detected_faults++;
        ctx->stats.rerun_count++;
        if ((rc = execute_once(ctx, node))) return rc;
        if ((rc = tensor_range(ctx, rec->tensor_id, r))) return rc;
        if (in_range(r)) ctx->stats.recovered_faults++;
        else ctx->stats.unrecovered_faults++;
        return 0;
    }

    if (rec->mode == SPKV2_PROTECT_DMR_COMPARE_RERUN) {
        size_t bytes = static_cast<size_t>(ctx->tensor_records[rec->tensor_id].size_bytes);
        if (!ctx->scratch || rec->scratch_offset > ctx->scratch_size ||
            bytes * 2u > ctx->scratch_size - static_cast<size_t>(rec->scratch_offset))
            return -25;
        uint8_t *first = ctx->scratch + rec->scratch_offset;
        uint8_t *second = first + bytes;
        uint8_t *out = ctx->tensors[rec->tensor_id].data;
        int rc;
        if ((rc = execute_once(ctx, node)) || (rc = d2d(ctx, first, out, bytes))) return rc;
        if ((rc = execute_once(ctx, node)) || (rc = d2d(ctx, second, out, bytes))) return rc;
        bool eq = false;
        if ((rc = bytes_equal(ctx, first, second, bytes, &eq))) return rc;
        if (eq) return 0;
        ctx->stats.detected_faults++;
        ctx->stats.rerun_count++;
        if ((rc = execute_once(ctx, node))) return rc;
        if ((rc = bytes_equal(ctx, first, out, bytes, &eq))) return rc;
        if (eq) {
            if ((rc = d2d(ctx, out, first, bytes))) return rc;
            ctx->stats.recovered_faults++;
            return 0;
        }
        if ((rc = bytes_equal(ctx, second, out, bytes, &eq))) return rc;
        if (eq) {
            if ((rc = d2d(ctx, out, second, bytes))) return rc;
            ctx->stats.recovered_faults++;
        } else {
            ctx->stats.unrecovered_faults++;
        }
        return 0;
    }
    return -26;
}

// ------------------------------------------------------------------ profiling

const Spkv2Context *g_prof_last_ctx = nullptr;
int g_prof_env = -1;

const char *op_name(uint16_t op) {
    static const char *names[] = {"Unknown", "Add", "Conv", "Flatten", "Gemm", "MaxPool", "Relu", "Softmax", "Mul",
                                  "Sub", "Div", "Mod", "Sigmoid", "Reshape", "Transpose", "Concat", "Split",
                                  "ReduceMean", "ReduceMax", "MatMul", "Resize", "Tile", "Unsqueeze",
                                  "GatherElements", "TopK", "Cast", "Slice", "Gather", "AveragePool",
                                  "GlobalAveragePool", "Clip", "LeakyRelu"};
    return op < sizeof(names) / sizeof(names[0]) ? names[op] : "Unknown";
}

int ensure_events(Spkv2Context *ctx) {
    if (ctx->ev_begin.size() == ctx->node_count) return 0;
    ctx->ev_begin.resize(ctx->node_count, nullptr);
    ctx->ev_end.resize(ctx->node_count, nullptr);
    for (size_t i = 0; i < ctx->node_count; i++) {
        if (int rc = hip_check(hipEventCreate(&ctx->ev_begin[i]), "hipEventCreate")) return rc;
        if (int rc = hip_check(hipEventCreate(&ctx->ev_end[i]), "hipEventCreate")) return rc;
    }
    return 0;
}

int run_eager(Spkv2Context *ctx) {
    const bool prof = ctx->profiling;
    if (prof)
        if (int rc = ensure_events(ctx)) return rc;
    for (uint32_t i = 0; i < ctx->header.num_nodes; i++) {
        const Spkv2NodeRecord *node = &ctx->node_records[i];
        if (prof) (void)hipEventRecord(ctx->ev_begin[i], ctx->stream);
        int rc = execute_protected(ctx, node);
        if (prof) (void)hipEventRecord(ctx->ev_end[i], ctx->stream);
        if (rc != 0) {
            (void)hipStreamSynchronize(ctx->stream);
            return rc;
        }
    }
    if (int rc = hip_check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize")) return rc;
    if (int rc = hip_check(hipGetLastError(), "kernel launch")) return rc;
    if (prof) {
        for (uint32_t i = 0; i < ctx->header.num_nodes; i++) {
            float ms = 0.0f;
            if (hipEventElapsedTime(&ms, ctx->ev_begin[i], ctx->ev_end[i]) == hipSuccess) {
                ctx->node_ms[i] += ms;
                ctx->node_runs[i]++;
            }
        }
    }
    return 0;
}

int run_graph(Spkv2Context *ctx) {
    if (!ctx->graph_exec || ctx->graph_epoch != ctx->binding_epoch) {
        drop_graph(ctx);
        hipGraph_t graph = nullptr;
        if (int rc = hip_check(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal),
                               "hipStreamBeginCapture"))
            return rc;
        int node_rc = 0;
        for (uint32_t i = 0; i < ctx->header.num_nodes && node_rc == 0; i++)
            node_rc = spk::execute_node(ctx, &ctx->node_records[i]);
        hipError_t end_err = hipStreamEndCapture(ctx->stream, &graph);
        if (node_rc != 0) {
            if (graph) (void)hipGraphDestroy(graph);
            return node_rc;
        }
        if (int rc = hip_check(end_err, "hipStreamEndCapture")) return rc;
        hipError_t inst = hipGraphInstantiate(&ctx->graph_exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        if (int rc = hip_check(inst, "hipGraphInstantiate")) return rc;
        ctx->graph_epoch = ctx->binding_epoch;
    }
    if (int rc = hip_check(hipGraphLaunch(ctx->graph_exec, ctx->stream), "hipGraphLaunch")) return rc;
    return hip_check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

}  // namespace

// ===================================================================== prepare

extern "C" int spkv2_prepare(Spkv2Context *ctx, void *arena, size_t arena_size) {
    return spkv2_prepare_with_scratch(ctx, arena, arena_size, nullptr, 0);
}

extern "C" int spkv2_prepare_with_scratch(Spkv2Context *ctx, void *arena, size_t arena_size, void *scratch,
                                          size_t scratch_size) {
    if (!ctx) return -1;
    const uint64_t required = ctx->header.activation_arena_bytes;
    const uint64_t scratch_required = ctx->header.scratch_arena_bytes;
    if (arena && arena_size < required) return -2;
    if (scratch_required > 0 && scratch && scratch_size < scratch_required) return -2;

    const bool first = !ctx->prepared;
    if (first) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) {
            (void)hipGetLastError();
            spk::set_last_error_text("no HIP device");
            return SPKV2_E_NO_DEVICE;
        }
        ctx->device = dev;
        // a blocking stream: it orders with null-stream copies made by callers
        if (int rc = hip_check(hipStreamCreateWithFlags(&ctx->stream, hipStreamDefault), "hipStreamCreate"))
            return rc;
    } else {
        (void)hipSetDevice(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
        drop_graph(ctx);
        if (ctx->owns_arena && ctx->arena) (void)hipFree(ctx->arena);
        if (ctx->owns_scratch && ctx->scratch) (void)hipFree(ctx->scratch);
        ctx->arena = ctx->scratch = nullptr;
        ctx->owns_arena = ctx->owns_scratch = false;
    }

    if (arena) {
        if (required > 0 && !is_device_accessible(arena)) return SPKV2_E_NOT_DEVICE_MEMORY;
        ctx->arena = static_cast<uint8_t *>(arena);
        ctx->arena_size = arena_size;
    } else {
        if (int rc = alloc_zeroed(&ctx->arena, required, ctx->stream)) return rc;
        ctx->owns_arena = true;
        ctx->arena_size = required;
    }
    ctx->scratch_size = 0;
    if (scratch_required > 0) {
        if (scratch) {
            if (!is_device_accessible(scratch)) return SPKV2_E_NOT_DEVICE_MEMORY;
            ctx->scratch = static_cast<uint8_t *>(scratch);
            ctx->scratch_size = scratch_size;
        } else {
            if (int rc = alloc_zeroed(&ctx->scratch, scratch_required, ctx->stream)) return rc;
            ctx->owns_scratch = true;
            ctx->scratch_size = scratch_required;
        }
    }

    if (first && ctx->weights_size > 0) {
        if (int rc = hip_check(hipMalloc(reinterpret_cast<void **>(&ctx->weights_dev), ctx->weights_size), "hipMalloc"))
            return rc;
        if (int rc = hip_check(hipMemcpyAsync(ctx->weights_dev, ctx->weights_host, ctx->weights_size,
                                              hipMemcpyHostToDevice, ctx->stream),
                               "hipMemcpyAsync weights"))
            return rc;
        if (int rc = hip_check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize")) return rc;
    }

    for (uint32_t i = 0; i < ctx->header.num_tensors; i++) {
        const Spkv2TensorRecord *r = &ctx->tensor_records[i];
        if (r->role == SPKV2_ROLE_WEIGHT) {
            if (r->data_offset > ctx->weights_size || r->size_bytes > ctx->weights_size - r->data_offset) return -3;
            ctx->tensors[i].data = ctx->weights_dev + r->data_offset;
        } else if (r->memory_class == SPKV2_MEMORY_EXTERNAL) {
            ctx->tensors[i].data = nullptr;
        } else {
            if (r->data_offset + r->size_bytes > required) return -4;
            ctx->tensors[i].data = ctx->arena + r->data_offset;
        }
    }
    ctx->binding_epoch++;

    if (first) {
        if (int rc = alloc_zeroed(reinterpret_cast<uint8_t **>(&ctx->dev_minmax), 4 * sizeof(float), ctx->stream))
            return rc;
        if (int rc = alloc_zeroed(reinterpret_cast<uint8_t **>(&ctx->dev_flag), 4 * sizeof(uint32_t), ctx->stream))
            return rc;
        // int8 activation tensors (the INT8 configuration with int8 tensors
        // between nodes) get their buffers before the nodes plan against them
        if (int rc = spk::kern::setup_q8_tensors(ctx)) return rc;
        size_t workspace = 0;
        for (uint32_t i = 0; i < ctx->header.num_nodes; i++) {
            size_t ws = 0;
            int rc = spk::prepare_node(ctx, &ctx->node_records[i], &ws);
            if (rc != 0) return rc;
            if (ws > workspace) workspace = ws;
        }
        if (int rc = spk::kern::check_q8_winners(ctx)) return rc;
        if (int rc = spk::kern::setup_concat_views(ctx)) return rc;
        if (int rc = spk::kern::setup_pool_int8_inputs(ctx)) return rc;
        if (workspace > 0) {
            if (int rc = hip_check(hipMalloc(reinterpret_cast<void **>(&ctx->workspace), workspace), "hipMalloc workspace"))
                return rc;
            ctx->workspace_size = workspace;
        }
        if (g_prof_env < 0) g_prof_env = env_flag("SPKV2_PROFILE") ? 1 : 0;
        ctx->profiling = g_prof_env == 1;
        ctx->graph_mode = env_flag("SPKV2_HIP_GRAPH");
    }
    // node prepare hooks upload with synchronous copies; drain everything
    if (int rc = hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize")) return rc;
    ctx->prepared = true;
    return 0;
}

// ========================================================================== IO

extern "C" int spkv2_set_input(Spkv2Context *ctx, int index, const void *data, size_t size) {
    if (!ctx || !data || index < 0) return -1;
    uint32_t tid = 0;
    const Spkv2TensorRecord *r = input_record(ctx, index, &tid);
    if (!r) return -3;
    if (size != r->size_bytes) return -2;
    if (!ctx->tensors[tid].data) return -5;
    if (int rc = hip_check(hipMemcpyAsync(ctx->tensors[tid].data, data, size, hipMemcpyHostToDevice, ctx->stream),
                           "hipMemcpyAsync input"))
        return rc;
    return hip_check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

extern "C" int spkv2_bind_input(Spkv2Context *ctx, int index, void *data, size_t size) {
    if (!ctx || !data || index < 0) return -1;
    uint32_t tid = 0;
    const Spkv2TensorRecord *r = input_record(ctx, index, &tid);
    if (!r) return -3;
    if (size != r->size_bytes) return -2;
    if (!is_device_accessible(data)) return SPKV2_E_NOT_DEVICE_MEMORY;
    ctx->tensors[tid].data = static_cast<uint8_t *>(data);
    ctx->binding_epoch++;
    return 0;
}

extern "C" int spkv2_bind_output(Spkv2Context *ctx, int index, void *data, size_t size) {
    if (!ctx || !data || index < 0) return -1;
    uint32_t tid = 0;
    if (int rc = output_tensor_id(ctx, index, &tid)) return rc;
    if (size != ctx->tensor_records[tid].size_bytes) return -2;
    if (!is_device_accessible(data)) return SPKV2_E_NOT_DEVICE_MEMORY;
    ctx->tensors[tid].data = static_cast<uint8_t *>(data);
    ctx->binding_epoch++;
    return 0;
}

extern "C" int spkv2_get_output(Spkv2Context *ctx, int index, void *data, size_t size) {
    if (!ctx || !data || index < 0) return -1;
    uint32_t tid = 0;
    if (int rc = output_tensor_id(ctx, index, &tid)) return rc;
    if (size != ctx->tensor_records[tid].size_bytes) return -2;
    if (!ctx->tensors[tid].data) return -5;
    if (!ctx->stream) return SPKV2_E_NO_DEVICE;
    if (int rc = hip_check(hipMemcpyAsync(data, ctx->tensors[tid].data, size, hipMemcpyDeviceToHost, ctx->stream),
                           "hipMemcpyAsync output"))
        return rc;
    return hip_check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

extern "C" int spkv2_get_output_size(Spkv2Context *ctx, int index, size_t *out_size) {
    if (!ctx || !out_size || index < 0) return -1;
    uint32_t tid = 0;
    if (int rc = output_tensor_id(ctx, index, &tid)) return rc;
    *out_size = static_cast<size_t>(ctx->tensor_records[tid].size_bytes);
    return 0;
}

// ========================================================================= run

extern "C" int spkv2_run(Spkv2Context *ctx) {
    if (!ctx) return -1;
    if (!ctx->prepared) return SPKV2_E_NO_DEVICE;
    (void)hipSetDevice(ctx->device);
    g_prof_last_ctx = ctx;
    if (ctx->invocations) memset(ctx->invocations, 0, ctx->node_count * sizeof(uint32_t));
    for (uint32_t i = 0; i < ctx->header.num_tensors; i++)
        if (ctx->tensor_records[i].role != SPKV2_ROLE_WEIGHT && !ctx->tensors[i].data) return -5;
    spk::refresh_winners(ctx);
    if (ctx->has_q8 && !ctx->winners_match) {
        // a user kernel registered since prepare would now run a node whose
        // int8 tensors live in the built-in kernels' own buffers
        spk::set_last_error_text("the kernel registry changed since prepare: int8 tensors between nodes need the "
                                 "built-in kernels that prepared them");
        return SPKV2_E_UNSUPPORTED;
    }
    const bool can_graph =
        ctx->graph_mode && !ctx->profiling && spk::handoffs_live(ctx) && ctx->protection_count == 0;
    if (can_graph) return run_graph(ctx);
    return run_eager(ctx);
}

// ================================================================= reliability

extern "C" int spkv2_set_fault_event(Spkv2Context *ctx, const Spkv2FaultEvent *event) {
    if (!ctx || !event || event->bit_index >= 32u) return -1;
    if (event->node_id >= ctx->header.num_nodes || event->tensor_id >= ctx->header.num_tensors) return -2;
    ctx->fault_event = *event;
    return 0;
}

extern "C" void spkv2_clear_fault_event(Spkv2Context *ctx) {
    if (ctx) memset(&ctx->fault_event, 0, sizeof(ctx->fault_event));
}

extern "C" int spkv2_get_reliability_stats(Spkv2Context *ctx, Spkv2ReliabilityStats *stats) {
    if (!ctx || !stats) return -1;
    *stats = ctx->stats;
    return 0;
}

extern "C" void spkv2_reset_reliability_stats(Spkv2Context *ctx) {
    if (ctx) memset(&ctx->stats, 0, sizeof(ctx->stats));
}

extern "C" int spkv2_get_range_observation(Spkv2Context *ctx, uint32_t node_id, Spkv2RangeObservation *observation) {
    if (!ctx || !observation || node_id >= ctx->node_count || !ctx->ranges) return -1;
    *observation = ctx->ranges[node_id];
    return 0;
}

extern "C" void spkv2_reset_range_observations(Spkv2Context *ctx) {
    if (ctx && ctx->ranges) memset(ctx->ranges, 0, ctx->node_count * sizeof(Spkv2RangeObservation));
}

// =================================================================== profiling

// Same three tables as the reference dump (executor.c:107-183), from the HIP
// event times of the last profiled context.
extern "C" void spkv2_profile_dump(void) {
    const Spkv2Context *ctx = g_prof_last_ctx;
    if (!ctx || !ctx->profiling) return;
    uint32_t runs = 0;
    for (size_t i = 0; i < ctx->node_count; i++)
        if (ctx->node_runs[i] > runs) runs = ctx->node_runs[i];
    if (runs == 0) return;
    double op_total[64] = {0};
    int op_count[64] = {0};
    for (size_t i = 0; i < ctx->node_count; i++) {
        uint16_t op = ctx->node_records[i].op_type;
        if (op < 64) {
            op_total[op] += ctx->node_ms[i];
            op_count[op] += static_cast<int>(ctx->node_runs[i]);
        }
    }
    int idx[64], n = 0;
    for (int i = 0; i < 64; i++)
        if (op_count[i] > 0) idx[n++] = i;
    for (int i = 0; i < n; i++)
        for (int j = i + 1; j < n; j++)
            if (op_total[idx[j]] > op_total[idx[i]]) std::swap(idx[i], idx[j]);
    double grand = 0.0;
    for (int i = 0; i < n; i++) grand += op_total[idx[i]];
    fprintf(stderr, "\n[SPKV2_PROFILE] per-op totals over %u runs (device time):\n", runs);
    fprintf(stderr, "  %-20s %8s %12s %12s\n", "op", "count", "total_ms", "avg_ms");
    for (int i = 0; i < n; i++) {
        int op = idx[i];
        fprintf(stderr, "  %-20s %8u %12.3f %12.4f (%5.1f%%)\n", op_name(static_cast<uint16_t>(op)),
                op_count[op] / runs, op_total[op], op_total[op] / op_count[op],
                grand > 0 ? 100.0 * op_total[op] / grand : 0.0);
    }
    fprintf(stderr, "  %-20s %8s %12.3f\n", "TOTAL", "", grand);
    fprintf(stderr, "\n[SPKV2_PROFILE] conv nodes over %u runs:\n", runs);
    fprintf(stderr, "  %-5s %-34s %8s %10s %26s %12s\n", "node", "kernel", "count", "avg_ms", "N,C,H,W->OC,k,s,p,g",
            "total_ms");
    for (size_t i = 0; i < ctx->node_count; i++) {
        const Spkv2NodeRecord *node = &ctx->node_records[i];
        if (node->op_type != SPKV2_OP_CONV || ctx->node_runs[i] == 0 || node->input_count < 2) continue;
        const Spkv2TensorRecord *x = &ctx->tensor_records[node->inputs[0]];
        const Spkv2TensorRecord *w = &ctx->tensor_records[node->inputs[1]];
        Spkv2AttrRecord a;
        if (spkv2_ctx_get_attr(ctx, node, &a) != 0) continue;
        char shape[128];
        snprintf(shape, sizeof(shape), "%u,%u,%u,%u->%u,%ux%u,%dx%d,%d/%d/%d/%d,%d", x->shape[0], x->shape[1],
                 x->shape[2], x->shape[3], w->shape[0], w->shape[2], w->shape[3], a.strides[0], a.strides[1], a.pads[0],
                 a.pads[1], a.pads[2], a.pads[3], a.group);
        fprintf(stderr, "  %-5u %-34s %8u %10.4f %26s %12.3f\n", node->id, ctx->node_kernel_names[i].c_str(),
                ctx->node_runs[i] / runs, ctx->node_ms[i] / ctx->node_runs[i], shape, ctx->node_ms[i]);
    }
    fprintf(stderr, "\nnode_id,op_type,avg_ms,total_ms,count\n");
    for (size_t i = 0; i < ctx->node_count; i++) {
        if (ctx->node_runs[i] == 0) continue;
        fprintf(stderr, "%u,%s,%.9f,%.9f,%u\n", ctx->node_records[i].id, op_name(ctx->node_records[i].op_type),
                ctx->node_ms[i] / ctx->node_runs[i], ctx->node_ms[i], ctx->node_runs[i] / runs);
    }
    fprintf(stderr, "\n");
}

// ============================================================ mi355x extensions

extern "C" const Spkv2TensorRecord *spkv2_ctx_tensor_record(const Spkv2Context *ctx, uint32_t tensor_id) {
    if (!ctx || tensor_id >= ctx->header.num_tensors) return nullptr;
    return &ctx->tensor_records[tensor_id];
}

extern "C" void *spkv2_ctx_tensor_data(const Spkv2Context *ctx, uint32_t tensor_id) {
    if (!ctx || tensor_id >= ctx->header.num_tensors) return nullptr;
    return ctx->tensors[tensor_id].data;
}

extern "C" int spkv2_ctx_get_attr(const Spkv2Context *ctx, const Spkv2NodeRecord *node, Spkv2AttrRecord *attr) {
    if (!ctx || !node || !attr) return -1;
    if (node->attr_offset > ctx->attrs_size || node->attr_size > ctx->attrs_size - node->attr_offset ||
        node->attr_size < sizeof(Spkv2AttrRecord))
        return -10;
    memcpy(attr, ctx->attrs + node->attr_offset, sizeof(Spkv2AttrRecord));
    return 0;
}

extern "C" void *spkv2_ctx_stream(const Spkv2Context *ctx) { return ctx ? ctx->stream : nullptr; }

extern "C" const Spkv2QuantParamRecord *spkv2_ctx_find_quant_param(const Spkv2Context *ctx, uint32_t tensor_id) {
    if (!ctx) return nullptr;
    for (size_t i = 0; i < ctx->quant_count; i++)
        if (ctx->quant_records[i].tensor_id == tensor_id) return &ctx->quant_records[i];
    return nullptr;
}

extern "C" const float *spkv2_ctx_quant_scales(const Spkv2Context *ctx, const Spkv2QuantParamRecord *qp) {
    if (!ctx || !qp || !ctx->quant_data) return nullptr;
    if (qp->data_offset + static_cast<uint64_t>(qp->num_channels) * 4 > ctx->quant_data_size) return nullptr;
    return reinterpret_cast<const float *>(ctx->quant_data + qp->data_offset);
}

extern "C" const int32_t *spkv2_ctx_quant_zero_points(const Spkv2Context *ctx, const Spkv2QuantParamRecord *qp) {
    if (!ctx || !qp || !ctx->quant_data) return nullptr;
    if (qp->data_offset + static_cast<uint64_t>(qp->num_channels) * 8 > ctx->quant_data_size) return nullptr;
    return reinterpret_cast<const int32_t *>(ctx->quant_data + qp->data_offset + static_cast<uint64_t>(qp->num_channels) * 4);
}

extern "C" int spkv2_ctx_node_cache(Spkv2Context *ctx, uint32_t node_id, void ***slot, void (***dtor)(void *)) {
    if (!ctx || node_id >= ctx->node_count) return -1;
    if (slot) *slot = &ctx->node_cache[node_id];
    if (dtor) *dtor = &ctx->node_cache_dtors[node_id];
    return 0;
}

extern "C" int spkv2_device_malloc(void **ptr, size_t size) {
    if (!ptr) return -1;
    return hip_check(hipMalloc(ptr, size), "hipMalloc");
}
extern "C" int spkv2_device_free(void *ptr) { return hip_check(hipFree(ptr), "hipFree"); }
extern "C" int spkv2_device_memcpy_h2d(void *dst, const void *src, size_t size) {
    if (int rc = hip_check(hipMemcpy(dst, src, size, hipMemcpyHostToDevice), "hipMemcpy h2d")) return rc;
    return hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
}
extern "C" int spkv2_device_memcpy_d2h(void *dst, const void *src, size_t size) {
    if (int rc = hip_check(hipMemcpy(dst, src, size, hipMemcpyDeviceToHost), "hipMemcpy d2h")) return rc;
    return hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
}
extern "C" int spkv2_device_memcpy_d2d(void *dst, const void *src, size_t size) {
    if (int rc = hip_check(hipMemcpy(dst, src, size, hipMemcpyDeviceToDevice), "hipMemcpy d2d")) return rc;
    return hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
}
extern "C" int spkv2_device_synchronize(void) { return hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize"); }

extern "C" int spkv2_device_info(int *compute_units, char *arch_name, size_t arch_name_size) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return SPKV2_E_NO_DEVICE;
    }
    hipDeviceProp_t prop;
    if (int rc = hip_check(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties")) return rc;
    if (compute_units) *compute_units = prop.multiProcessorCount;
    if (arch_name && arch_name_size) snprintf(arch_name, arch_name_size, "%s", prop.gcnArchName);
    return 0;
}

extern "C" const char *spkv2_mi355x_last_error(void) { return spk::g_last_error.c_str(); }

extern "C" int spkv2_mi355x_set_graph_mode(Spkv2Context *ctx, int enable) {
    if (!ctx) return -1;
    ctx->graph_mode = enable != 0;
    if (!ctx->graph_mode) drop_graph(ctx);
    return 0;
}

extern "C" int spkv2_mi355x_set_profiling(Spkv2Context *ctx, int enable) {
    if (!ctx) return -1;
    ctx->profiling = enable != 0;
    return 0;
}

extern "C" int spkv2_mi355x_node_time(Spkv2Context *ctx, uint32_t node_id, double *total_ms, uint32_t *count) {
    if (!ctx || node_id >= ctx->node_count) return -1;
    if (total_ms) *total_ms = ctx->node_ms[node_id];
    if (count) *count = ctx->node_runs[node_id];
    return 0;
}

extern "C" void spkv2_mi355x_reset_node_times(Spkv2Context *ctx) {
    if (!ctx) return;
    std::fill(ctx->node_ms.begin(), ctx->node_ms.end(), 0.0);
    std::fill(ctx->node_runs.begin(), ctx->node_runs.end(), 0u);
}

extern "C" int spkv2_mi355x_node_kernel_name(Spkv2Context *ctx, uint32_t node_id, char *buf, size_t buf_size) {
    if (!ctx || !buf || buf_size == 0 || node_id >= ctx->node_count) return -1;
    snprintf(buf, buf_size, "%s", ctx->node_kernel_names[node_id].c_str());
    return 0;
}

// Bytes of a conv node's int32 accumulators: four per output element.
static size_t acc_bytes(const Spkv2TensorRecord *y) {
    size_t n = 1;
    for (uint16_t i = 0; i < y->rank; i++) n *= y->shape[i];
    return n * sizeof(int32_t);
}

extern "C" int spkv2_mi355x_set_int8_capture(Spkv2Context *ctx, int enable) {
    if (!ctx) return -1;
    if (!ctx->prepared) return SPKV2_E_NO_DEVICE;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    for (int32_t *&p : ctx->acc_capture) {
        if (p) (void)hipFree(p);
        p = nullptr;
    }
    ctx->acc_capture.assign(ctx->node_count, nullptr);
    ctx->binding_epoch++;  // a captured HIP graph holds the launches of the old setting
    if (!enable) return 0;
    for (uint32_t i = 0; i < ctx->header.num_nodes; i++) {
        const Spkv2NodeRecord *node = &ctx->node_records[i];
        if (node->op_type != SPKV2_OP_CONV || node->input_count < 2) continue;
        if (ctx->tensor_records[node->inputs[1]].dtype != SPKV2_DTYPE_INT8) continue;
        // int32 per output element, whatever the output's own dtype (an int8
        // tensor in the INT8 configuration with int8 tensors between nodes)
        const size_t bytes = acc_bytes(&ctx->tensor_records[node->outputs[0]]);
        if (int rc = hip_check(hipMalloc(reinterpret_cast<void **>(&ctx->acc_capture[node->id]), bytes),
                               "hipMalloc accumulator capture"))
            return rc;
        if (int rc = hip_check(hipMemset(ctx->acc_capture[node->id], 0, bytes), "hipMemset")) return rc;
    }
    return 0;
}

extern "C" int spkv2_mi355x_conv_int8_accumulators(Spkv2Context *ctx, uint32_t node_id, int32_t *out, size_t size) {
    if (!ctx || !out || node_id >= ctx->node_count) return -1;
    if (!ctx->prepared) return SPKV2_E_NO_DEVICE;
    const Spkv2NodeRecord *node = &ctx->node_records[node_id];
    if (node->op_type != SPKV2_OP_CONV) return -1;
    const Spkv2TensorRecord *y = &ctx->tensor_records[node->outputs[0]];
    if (size != acc_bytes(y)) return -2;
    if (node_id < ctx->acc_capture.size() && ctx->acc_capture[node_id]) {
        // captured during the last spkv2_run
        if (int rc = hip_check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize")) return rc;
        return hip_check(hipMemcpy(out, ctx->acc_capture[node_id], size, hipMemcpyDeviceToHost), "hipMemcpy");
    }
    int32_t *dev = nullptr;
    if (int rc = hip_check(hipMalloc(reinterpret_cast<void **>(&dev), size), "hipMalloc")) return rc;
    int rc = spk::kern::conv_int8_accumulators(ctx, node, dev);
    if (rc == 0) rc = hip_check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (rc == 0) rc = hip_check(hipMemcpy(out, dev, size, hipMemcpyDeviceToHost), "hipMemcpy");
    (void)hipFree(dev);
    return rc;
}

// ---------------------------------------------- allocation-free accumulators
//
// The raw accumulators staged through a fixed device array instead of a
// per-call hipMalloc.  Each GPU holds its own copy of `scratch` for the life
// of the process; host code uses only the per-device address from
// hipGetSymbolAddress (the array's name is a host-side stand-in, not a
// device address).  Every call on one GPU shares that GPU's array: calls
// that overlap on one GPU (other threads, other contexts' streams) race.
// Nothing in it must start at zero: the accumulator kernels write every
// element of the first `size` bytes, and only those are copied out.

constexpr size_t kAccScratchBytes = size_t(16) << 20;  // 16 MiB per GPU
static __device__ __align__(256) int32_t scratch[kAccScratchBytes / sizeof(int32_t)];

namespace {

std::mutex g_scratch_mu;
int32_t *g_scratch_ptr[64] = {};  // per device ordinal, resolved once with the device current

int32_t *scratch_for_device(int dev) {
    if (dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
            spk::set_last_error_text("hipGetSymbolAddress(scratch) failed");
            (void)hipGetLastError();
            return nullptr;
        }
        g_scratch_ptr[dev] = static_cast<int32_t *>(p);
    }
    return g_scratch_ptr[dev];
}

}  // namespace

extern "C" int spkv2_mi355x_conv_int8_accumulators_noalloc(Spkv2Context *ctx, uint32_t node_id, int32_t *out,
                                                           size_t size) {
    if (!ctx || !out || node_id >= ctx->node_count) return -1;
    if (!ctx->prepared) return SPKV2_E_NO_DEVICE;
    const Spkv2NodeRecord *node = &ctx->node_records[node_id];
    if (node->op_type != SPKV2_OP_CONV) return -1;
    const Spkv2TensorRecord *y = &ctx->tensor_records[node->outputs[0]];
    if (size != acc_bytes(y)) return -2;
    if (size > kAccScratchBytes) {
        spk::set_last_error_text("int8 accumulators of " + std::to_string(size) +
                                 " bytes exceed the 16 MiB allocation-free staging array");
        return SPKV2_E_UNSUPPORTED;
    }
    if (int rc = hip_check(hipSetDevice(ctx->device), "hipSetDevice")) return rc;
    int32_t *dev = scratch_for_device(ctx->device);
    if (!dev) return SPKV2_E_HIP;
    int rc = spk::kern::conv_int8_accumulators(ctx, node, dev);
    if (rc == 0) rc = hip_check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    if (rc == 0) rc = hip_check(hipMemcpy(out, dev, size, hipMemcpyDeviceToHost), "hipMemcpy");
    return rc;
}
