// Kernel registry and KernelSpec dispatch.
//
// Lookup semantics are those of the reference dispatcher
// (runtime/kernels/reference/kernels.c:144-245): a node's KernelSpec record
// gives (backend, kind); the user table (64 slots) is scanned first, then the
// built-in table, and an entry replaces the current best only with a strictly
// higher priority, so user kernels win ties with the built-ins (priority 0).
// A missing kernel or a kernel returning -99 moves on to the spec's
// fallback_kernel_spec_id, then to the built-in (ref, reference) spec.
//
// The difference is the built-in table: every entry is a device kernel.
// Kernels are registered under the mi355x kinds AND under every existing
// (backend, kind) triple, so packages compiled for cpu_ref / cpu_generic /
// cpu_arm_neon run on the GPU unchanged, and the final (ref, reference)
// fallback is a device kernel too.  No node ever runs on the CPU.
#include <atomic>
#include <cstring>

#include "../kernels/kernels.hpp"
#include "context.hpp"
#include "spkv2_mi355x.h"

namespace {

using spk::kern::PrepFn;
using spk::kern::RunFn;

struct Entry {
    uint16_t op, backend, kind;
    int priority;
    RunFn run;
    PrepFn prepare;
};

constexpr int kUserMax = 64;
struct UserEntry {
    uint16_t op, backend, kind;
    int priority;
    Spkv2NodeKernelFn fn;
};
UserEntry g_user[kUserMax];
int g_user_count = 0;
std::atomic<uint32_t> g_generation{0};

#define E(op, be, kind, run, prep) {op, be, kind, 0, run, prep}
using namespace spk::kern;

// clang-format off
const Entry kBuiltins[] = {
    // ---- convolution ----
    E(SPKV2_OP_CONV, SPKV2_BACKEND_MI355X, SPKV2_KERNEL_IMPLICIT_GEMM_F32, conv_run, conv_prepare),
    E(SPKV2_OP_CONV, SPKV2_BACKEND_MI355X, SPKV2_KERNEL_IMPLICIT_GEMM_I8, conv_run, conv_prepare),
    E(SPKV2_OP_CONV, SPKV2_BACKEND_MI355X, SPKV2_KERNEL_REFERENCE, conv_direct_run, nullptr),
    E(SPKV2_OP_CONV, SPKV2_BACKEND_SIMD, SPKV2_KERNEL_IM2COL_GEMM, conv_run, conv_prepare),
    E(SPKV2_OP_CONV, SPKV2_BACKEND_SIMD, SPKV2_KERNEL_POINTWISE_1X1, conv_run, conv_prepare),
    E(SPKV2_OP_CONV, SPKV2_BACKEND_SIMD, SPKV2_KERNEL_DEPTHWISE_DIRECT, conv_run, conv_prepare),
    E(SPKV2_OP_CONV, SPKV2_BACKEND_SIMD, SPKV2_KERNEL_WINOGRAD_3X3S1, conv_run, conv_prepare),
    E(SPKV2_OP_CONV, SPKV2_BACKEND_SIMD, SPKV2_KERNEL_WINOGRAD_F43, conv_run, conv_prepare),
    E(SPKV2_OP_CONV, SPKV2_BACKEND_SIMD, SPKV2_KERNEL_CONV3X3S2_DIRECT, conv_run, conv_prepare),
    E(SPKV2_OP_CONV, SPKV2_BACKEND_SIMD, SPKV2_KERNEL_INT8_IM2COL_GEMM, conv_run, conv_prepare),
    E(SPKV2_OP_CONV, SPKV2_BACKEND_SIMD, SPKV2_KERNEL_BNNS_FP32, conv_run, conv_prepare),
    E(SPKV2_OP_CONV, SPKV2_BACKEND_CPU, SPKV2_KERNEL_IM2COL_GEMM, conv_run, conv_prepare),
    E(SPKV2_OP_CONV, SPKV2_BACKEND_REF, SPKV2_KERNEL_REFERENCE, conv_run, conv_prepare),
    // ---- Gemm / MatMul ----
    E(SPKV2_OP_GEMM, SPKV2_BACKEND_MI355X, SPKV2_KERNEL_GEMM_F32, gemm_run, gemm_prepare),
    E(SPKV2_OP_GEMM, SPKV2_BACKEND_SIMD, SPKV2_KERNEL_DIRECT, gemm_run, gemm_prepare),
    E(SPKV2_OP_GEMM, SPKV2_BACKEND_CPU, SPKV2_KERNEL_DIRECT, gemm_run, gemm_prepare),
    E(SPKV2_OP_GEMM, SPKV2_BACKEND_REF, SPKV2_KERNEL_REFERENCE, gemm_run, gemm_prepare),
    E(SPKV2_OP_MATMUL, SPKV2_BACKEND_MI355X, SPKV2_KERNEL_GEMM_F32, matmul_run, nullptr),
    E(SPKV2_OP_MATMUL, SPKV2_BACKEND_SIMD, SPKV2_KERNEL_DIRECT, matmul_run, nullptr),
    E(SPKV2_OP_MATMUL, SPKV2_BACKEND_REF, SPKV2_KERNEL_REFERENCE, matmul_run, nullptr),
// ---- memory-bound ops: mi355x kind, the SIMD "reference" kind, and ref ----
#define EW(op, run) \
    E(op, SPKV2_BACKEND_MI355X, SPKV2_KERNEL_DEVICE_ELEMENTWISE, run, nullptr), \
    E(op, SPKV2_BACKEND_SIMD, SPKV2_KERNEL_REFERENCE, run, nullptr), \
    E(op, SPKV2_BACKEND_REF, SPKV2_KERNEL_REFERENCE, run, nullptr)
    EW(SPKV2_OP_ADD, binary_run),
    EW(SPKV2_OP_MUL, binary_run),
    EW(SPKV2_OP_SUB, binary_run),
    EW(SPKV2_OP_DIV, binary_run),
    EW(SPKV2_OP_MOD, binary_run),
    EW(SPKV2_OP_RELU, unary_run),
    EW(SPKV2_OP_SIGMOID, unary_run),
    EW(SPKV2_OP_CLIP, unary_run),
    EW(SPKV2_OP_LEAKYRELU, unary_run),
    E(SPKV2_OP_MAXPOOL, SPKV2_BACKEND_MI355X, SPKV2_KERNEL_DEVICE_ELEMENTWISE, maxpool_run, maxpool_prepare),
    E(SPKV2_OP_MAXPOOL, SPKV2_BACKEND_SIMD, SPKV2_KERNEL_REFERENCE, maxpool_run, maxpool_prepare),
    E(SPKV2_OP_MAXPOOL, SPKV2_BACKEND_REF, SPKV2_KERNEL_REFERENCE, maxpool_run, maxpool_prepare),
    EW(SPKV2_OP_AVERAGEPOOL, avgpool_run),
    EW(SPKV2_OP_GLOBALAVGPOOL, global_avgpool_run),
    EW(SPKV2_OP_SOFTMAX, softmax_run),
    EW(SPKV2_OP_REDUCEMEAN, reduce_run),
    EW(SPKV2_OP_REDUCEMAX, reduce_run),
    EW(SPKV2_OP_RESIZE, resize_run),
    EW(SPKV2_OP_FLATTEN, copy_run),
    EW(SPKV2_OP_RESHAPE, copy_run),
    EW(SPKV2_OP_CAST, copy_run),
    EW(SPKV2_OP_UNSQUEEZE, copy_run),
    EW(SPKV2_OP_CONCAT, concat_run),
    EW(SPKV2_OP_TRANSPOSE, transpose_run),
    EW(SPKV2_OP_TILE, tile_run),
    EW(SPKV2_OP_SPLIT, split_run),
    EW(SPKV2_OP_SLICE, slice_run),
    EW(SPKV2_OP_GATHER, gather_run),
    EW(SPKV2_OP_GATHERELEMENTS, gather_elements_run),
    EW(SPKV2_OP_TOPK, topk_run),
#undef EW
};
// clang-format on
#undef E

// The reference's built-in fallback spec: (ref, reference), fp32, no scratch
// (kernels.c:169-182).  node_id is filled in per node.
Spkv2KernelSpecRecord ref_spec_for(uint32_t node_id) {
    Spkv2KernelSpecRecord s{};
    s.id = 0xFFFFFFFFu;
    s.node_id = node_id;
    s.kernel_kind = SPKV2_KERNEL_REFERENCE;
    s.backend = SPKV2_BACKEND_REF;
    s.dtype = SPKV2_DTYPE_FP32;
    s.layout = 1;
    s.weight_layout = 1;
    s.fallback_kernel_spec_id = 0xFFFFFFFFu;
    s.required_feature_mask = 1;
    return s;
}

struct Found {
    Spkv2NodeKernelFn fn = nullptr;
    const Entry *builtin = nullptr;  // set when the winner is a built-in
};

Found find_kernel(uint16_t op, const Spkv2KernelSpecRecord *spec) {
    Found best;
    int best_priority = -1;
    for (int i = 0; i < g_user_count; i++) {
        const UserEntry &u = g_user[i];
        if (u.op == op && u.backend == spec->backend && u.kind == spec->kernel_kind && u.priority > best_priority) {
            best.fn = u.fn;
            best.builtin = nullptr;
            best_priority = u.priority;
        }
    }
    for (const Entry &e : kBuiltins) {
        if (e.op == op && e.backend == spec->backend && e.kind == spec->kernel_kind && e.priority > best_priority) {
            best.fn = e.run;
            best.builtin = &e;
            best_priority = e.priority;
        }
    }
    return best;
}

const Spkv2KernelSpecRecord *selected_spec(const Spkv2Context *ctx, const Spkv2NodeRecord *node,
                                           Spkv2KernelSpecRecord *ref_storage) {
    const Spkv2KernelSpecRecord *s = spk::spec_by_id(ctx, node->kernel_spec_id);
    if (!s || s->node_id != node->id) {
        *ref_storage = ref_spec_for(node->id);
        return ref_storage;
    }
    return s;
}

int execute_with_spec(Spkv2Context *ctx, const Spkv2NodeRecord *node, const Spkv2KernelSpecRecord *spec) {
    Found f = find_kernel(node->op_type, spec);
    if (!f.fn) return -99;
    if (spec->scratch_bytes > ctx->scratch_size) return -14;
    if (spec->scratch_bytes > 0 && spec->scratch_offset > ctx->scratch_size - spec->scratch_bytes) return -14;
    void *scratch = spec->scratch_bytes > 0 ? ctx->scratch + spec->scratch_offset : nullptr;
    return f.fn(ctx, node, scratch);
}

const Entry *find_builtin(uint16_t op, const Spkv2KernelSpecRecord *spec) {
    for (const Entry &e : kBuiltins)
        if (e.op == op && e.backend == spec->backend && e.kind == spec->kernel_kind) return &e;
    return nullptr;
}

// Prepare walks the chain over the built-in table only: the first spec with a
// built-in kernel whose prepare step accepts the node is prepared, whether or
// not a user kernel wins that spec.  A user kernel that answers -99, or is
// cleared after prepare, then hands the node to a built-in that has its plan
// and its workspace.
int prepare_with_spec(Spkv2Context *ctx, const Spkv2NodeRecord *node, const Spkv2KernelSpecRecord *spec,
                      size_t *ws) {
    const Entry *b = find_builtin(node->op_type, spec);
    if (!b) return -99;
    return b->prepare ? b->prepare(ctx, node, ws) : 0;
}

// The kernel execute_node would call first for this node: the winner of the
// first spec in the chain that has one.
Found resolve(const Spkv2Context *ctx, const Spkv2NodeRecord *node) {
    Spkv2KernelSpecRecord ref_storage;
    const Spkv2KernelSpecRecord *spec = selected_spec(ctx, node, &ref_storage);
    Found f = find_kernel(node->op_type, spec);
    if (f.fn) return f;
    if (const Spkv2KernelSpecRecord *fb = spk::spec_by_id(ctx, spec->fallback_kernel_spec_id)) {
        f = find_kernel(node->op_type, fb);
        if (f.fn) return f;
    }
    Spkv2KernelSpecRecord ref = ref_spec_for(node->id);
    return find_kernel(node->op_type, &ref);
}

}  // namespace

namespace spk {

uint32_t registry_generation() { return g_generation.load(std::memory_order_relaxed); }

const Spkv2KernelSpecRecord *spec_by_id(const Spkv2Context *ctx, uint32_t id) {
    if (id == 0xFFFFFFFFu || id >= ctx->spec_count) return nullptr;
    return &ctx->spec_records[id];
}

// Ops the reference retries on the built-in (ref, reference) spec
// (kernels.c:211-237): every op code except Reshape.
static bool op_has_ref_fallback(uint16_t op) {
    return op >= SPKV2_OP_ADD && op <= SPKV2_OP_LEAKYRELU && op != SPKV2_OP_RESHAPE;
}

int execute_node(Spkv2Context *ctx, const Spkv2NodeRecord *node) {
    Spkv2KernelSpecRecord ref_storage;
    const Spkv2KernelSpecRecord *spec = selected_spec(ctx, node, &ref_storage);
    int rc = execute_with_spec(ctx, node, spec);
    if (rc != -99) return rc;
    if (const Spkv2KernelSpecRecord *fb = spec_by_id(ctx, spec->fallback_kernel_spec_id))
        return execute_with_spec(ctx, node, fb);
    if (!op_has_ref_fallback(node->op_type)) return -99;
    Spkv2KernelSpecRecord ref = ref_spec_for(node->id);
    return execute_with_spec(ctx, node, &ref);
}

void refresh_winners(Spkv2Context *ctx) {
    const uint32_t gen = registry_generation();
    if (gen == ctx->checked_generation) return;
    bool match = true;
    for (uint32_t i = 0; i < ctx->header.num_nodes && match; i++)
        match = i < ctx->winners.size() && resolve(ctx, &ctx->node_records[i]).fn == ctx->winners[i];
    ctx->winners_match = match;
    ctx->checked_generation = gen;
}

int prepare_node(Spkv2Context *ctx, const Spkv2NodeRecord *node, size_t *ws) {
    if (ctx->winners.size() != ctx->node_count) {
        ctx->winners.assign(ctx->node_count, nullptr);
        ctx->builtin_winner.assign(ctx->node_count, 0);
        ctx->checked_generation = registry_generation();
        ctx->winners_match = true;
    }
    // recorded before the node's prepare step, which may set up a handoff
    // with an earlier node when the built-ins run both
    const Found w = resolve(ctx, node);
    ctx->winners[node->id] = w.fn;
    ctx->builtin_winner[node->id] = w.builtin != nullptr;
    Spkv2KernelSpecRecord ref_storage;
    const Spkv2KernelSpecRecord *spec = selected_spec(ctx, node, &ref_storage);
    int rc = prepare_with_spec(ctx, node, spec, ws);
    if (rc != -99) return rc;
    if (const Spkv2KernelSpecRecord *fb = spec_by_id(ctx, spec->fallback_kernel_spec_id)) {
        rc = prepare_with_spec(ctx, node, fb, ws);
        if (rc != -99) return rc;
    }
    if (!op_has_ref_fallback(node->op_type)) return 0;  // reported by run as -99
    Spkv2KernelSpecRecord ref = ref_spec_for(node->id);
    rc = prepare_with_spec(ctx, node, &ref, ws);
    return rc == -99 ? 0 : rc;
}

}  // namespace spk

extern "C" int spkv2_register_kernel(uint16_t op_type, uint16_t backend, uint16_t kernel_kind, Spkv2NodeKernelFn fn,
                                     int priority) {
    if (!fn) return -1;
    if (g_user_count >= kUserMax) return -2;
    g_user[g_user_count++] = UserEntry{op_type, backend, kernel_kind, priority, fn};
    g_generation.fetch_add(1, std::memory_order_relaxed);
    return 0;
}

extern "C" void spkv2_clear_user_kernels(void) {
    g_user_count = 0;
    g_generation.fetch_add(1, std::memory_order_relaxed);
}
