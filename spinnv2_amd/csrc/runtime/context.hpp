// Private state of one loaded SPK model on one GPU.
//
// The reference keeps an equivalent struct (runtime/core/context.h:15-59) and
// lets kernels dereference it; here it is opaque to everything outside
// libspkv2_mi355x.so and kernels use the accessors of spkv2_mi355x.h.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "spkv2_format.h"
#include "spkv2_runtime.h"

struct Spkv2TensorSlot {
    const Spkv2TensorRecord *record = nullptr;
    uint8_t *data = nullptr;  // device address (or a caller-bound device buffer)
};

// A channel-slice view: an fp32 NCHW activation that lives as a channel
// range of a Concat's device buffer instead of at its own arena offset, so
// the Concat need not copy it.  img_elems: elements between images; extent:
// bytes from base to the end of the tensor's last image.
struct Spkv2TensorView {
    uint8_t *base = nullptr;
    int64_t img_elems = 0;  // elements between images
    size_t extent = 0;      // bytes from base to the end of the buffer
    int64_t ch_elems = 0;   // elements between channels (0: the tensor's own plane size)
};

// An int8 activation tensor of the INT8 configuration with int8 tensors
// between nodes (package dtype int8, role activation): it lives in its own
// device buffer as zero-point-padded NHWC, [N][Hp][Wp][Cp] bytes, the image
// at rows pt.. and columns pl.., channels 0..C-1 of a Cp = 16k pitch.  The
// halo (the widest padding of the convs that read it) and the pitch's extra
// channels hold the zero point, written once at prepare: a padded tap then
// reads the real value 0.  Not in the arena: nothing but the built-in int8
// kernels reads it.
struct Spkv2Q8Tensor {
    int8_t *buf = nullptr;
    size_t bytes = 0;
    int N = 0, C = 0, H = 0, W = 0;
    int Hp = 0, Wp = 0, Cp = 0, pt = 0, pl = 0;
    float scale = 1.0f;
    int zp = 0;
};

struct Spkv2Context {
    // ---- the package (host memory, zero-copy views into the blob) ----
    uint8_t *owned_model = nullptr;
    // FP16-weight packages: tensor table copy whose half weights describe the
    // fp32 copies appended to `promoted_weights` (null when none)
    Spkv2TensorRecord *promoted_records = nullptr;
    uint8_t *promoted_weights = nullptr;
    const uint8_t *model = nullptr;
    size_t model_size = 0;
    Spkv2Header header{};
    const Spkv2SectionEntry *sections = nullptr;
    const Spkv2TensorRecord *tensor_records = nullptr;
    const Spkv2NodeRecord *node_records = nullptr;
    const Spkv2MemoryPlanRecord *plan_records = nullptr;
    size_t plan_count = 0;
    const Spkv2KernelSpecRecord *spec_records = nullptr;
    size_t spec_count = 0;
    const Spkv2ProtectionRecord *protection_records = nullptr;
    size_t protection_count = 0;
    const uint8_t *attrs = nullptr;
    size_t attrs_size = 0;
    const uint8_t *weights_host = nullptr;
    size_t weights_size = 0;
    const Spkv2QuantParamRecord *quant_records = nullptr;
    size_t quant_count = 0;
    const uint8_t *quant_data = nullptr;
    size_t quant_data_size = 0;
    uint32_t *output_ids = nullptr;  // graph output order from the metadata JSON
    size_t output_count = 0;
    Spkv2TensorSlot *tensors = nullptr;

    // ---- device state (valid after prepare) ----
    bool prepared = false;
    int device = -1;
    hipStream_t stream = nullptr;
    uint8_t *weights_dev = nullptr;
    uint8_t *arena = nullptr;
    bool owns_arena = false;
    size_t arena_size = 0;
    uint8_t *scratch = nullptr;
    bool owns_scratch = false;
    size_t scratch_size = 0;
    uint8_t *workspace = nullptr;  // runtime-owned device workspace (split-K partials)
    size_t workspace_size = 0;

    // per-node state
    size_t node_count = 0;
    // the per-node cache slots of the kernel ABI (reference context.h:46-48),
    // owned by whatever kernel runs the node: third-party kernels reach them
    // through spkv2_ctx_node_cache
    void **node_cache = nullptr;
    void (**node_cache_dtors)(void *) = nullptr;
    // the built-in device kernels' per-node plans (packed weights, tile and
    // split choice, handoff buffers), kept apart from node_cache so that a
    // user kernel winning a node at run time, or answering -99, never meets a
    // foreign object, and a built-in fallback always finds its plan
    std::vector<void *> plans;
    std::vector<void (*)(void *)> plan_dtors;
    std::vector<std::string> node_kernel_names;

    // ---- reliability (reference executor.c:335-498) ----
    Spkv2FaultEvent fault_event{};
    Spkv2ReliabilityStats stats{};
    Spkv2RangeObservation *ranges = nullptr;
    uint32_t *invocations = nullptr;
    float *dev_minmax = nullptr;  // 4 floats: min, max, nonfinite count, pad
    uint32_t *dev_flag = nullptr;

    // ---- execution controls ----
    bool graph_mode = false;
    hipGraphExec_t graph_exec = nullptr;
    uint64_t binding_epoch = 1;  // bumped by every bind_*
    uint64_t graph_epoch = 0;    // binding_epoch the graph was captured at
    // the kernel that runs each node (the first spec of its chain with a
    // registered kernel), as resolved at prepare; builtin_winner marks the
    // nodes a built-in device kernel runs.  Handoffs are set up only between
    // such nodes, and stay in force only while every node still resolves to
    // the kernel it had at prepare (re-checked when the registry changes).
    std::vector<Spkv2NodeKernelFn> winners;
    std::vector<uint8_t> builtin_winner;
    uint32_t checked_generation = 0;  // registry_generation() winners_match was computed at
    bool winners_match = true;
    bool profiling = false;
    std::vector<hipEvent_t> ev_begin, ev_end;
    std::vector<double> node_ms;
    std::vector<uint32_t> node_runs;
    // INT8 accumulator capture (test hook): per node, a device buffer that
    // each run of an int8 conv fills with its raw int32 accumulators
    std::vector<int32_t *> acc_capture;
    // Channel-slice views set up at prepare (Concat along channels at batch
    // > 1, detection-head chains), in force only while the handoffs are: per
    // tensor (base null: none), per node whether it is a Split whose outputs
    // are all views of its input (nothing to copy) or a node whose output
    // the views already hold (nothing to run), and the buffers (owned).
    std::vector<Spkv2TensorView> views;
    std::vector<uint8_t> view_split;
    std::vector<uint8_t> view_elide;  // nodes whose output the views already hold: nothing to run
    std::vector<void *> view_buffers;
    // int8 activation tensors (per tensor id; buf null for every other
    // tensor) and the nodes that read or write one
    std::vector<Spkv2Q8Tensor> q8;
    std::vector<uint8_t> q8_node;
    bool has_q8 = false;
};

// ---- internal helpers shared by the runtime translation units ----
namespace spk {

int execute_node(Spkv2Context *ctx, const Spkv2NodeRecord *node);
int prepare_node(Spkv2Context *ctx, const Spkv2NodeRecord *node, size_t *workspace_bytes);
const Spkv2KernelSpecRecord *spec_by_id(const Spkv2Context *ctx, uint32_t id);
// Bumped by every spkv2_register_kernel / spkv2_clear_user_kernels.
uint32_t registry_generation();
// Re-resolves every node's kernel when the registry changed since the last
// check, and sets ctx->winners_match to whether each node still resolves to
// the kernel it had at prepare.
void refresh_winners(Spkv2Context *ctx);

// Whether a built-in device kernel was resolved to run this node at prepare.
inline bool builtin_runs(const Spkv2Context *ctx, uint32_t node_id) {
    return node_id < ctx->builtin_winner.size() && ctx->builtin_winner[node_id] != 0;
}

// Whether the prepare-time handoffs (a producer writing its consumer's padded
// or int8 input) are in force for this run: not while a fault event is armed
// (a fault may change a tensor after its producer ran), nor while any node
// resolves to another kernel than at prepare (a user kernel registered or
// cleared since may now run a producer or consumer in place of the built-in
// the handoff relies on).  When they are not, every producer writes its
// output and every consumer reads it, as the reference does.
inline bool handoffs_live(const Spkv2Context *ctx) { return !ctx->fault_event.enabled && ctx->winners_match; }

// The channel-slice view a built-in kernel reads or writes a tensor through
// in this run, or null (the tensor is at its own slot).
inline const Spkv2TensorView *live_view(const Spkv2Context *ctx, uint32_t tensor_id) {
    if (tensor_id >= ctx->views.size() || !ctx->views[tensor_id].base || !handoffs_live(ctx)) return nullptr;
    return &ctx->views[tensor_id];
}
inline bool view_elided(const Spkv2Context *ctx, uint32_t node_id) {
    return node_id < ctx->view_elide.size() && ctx->view_elide[node_id] && handoffs_live(ctx);
}
void set_last_error(const char *what, hipError_t err);
void set_last_error_text(const std::string &text);
int hip_check(hipError_t err, const char *what);

// The int8 activation tensor record of a tensor id, or null.
inline const Spkv2Q8Tensor *q8_tensor(const Spkv2Context *ctx, uint32_t tensor_id) {
    return tensor_id < ctx->q8.size() && ctx->q8[tensor_id].buf ? &ctx->q8[tensor_id] : nullptr;
}

inline const uint8_t *host_weight_data(const Spkv2Context *ctx, uint32_t tensor_id) {
    const Spkv2TensorRecord *r = &ctx->tensor_records[tensor_id];
    if (r->role != SPKV2_ROLE_WEIGHT) return nullptr;
    return ctx->weights_host + r->data_offset;
}

}  // namespace spk
