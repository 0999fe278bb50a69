// Channel-slice views: Concat (and Split) along channels without copies.
//
// At batch 1 the compiler's memory plan may place a Concat's inputs inside
// its output (reference compiler/planner/memory_plan.py, Concat aliases),
// but not a Split's outputs inside its input; at batch > 1 an input's
// channels are one strided block per image, and the reference copies them
// (runtime/kernels/reference/tensor/concat.c, split.c).  Here such a Concat
// gets a device buffer of its own (at batch 1 only when every input can be
// placed, so that no aliased input turns into a copy), and the
// producers of its inputs write each input straight into its channel range
// of that buffer, the other readers read it there (a "view": base pointer,
// elements between images), and the Concat copies only what is left:
//   * an input written by an fp32 implicit-GEMM conv (without a residual: its
//     residual keeps y's natural layout), by a same-shape Add or by a 2x
//     nearest Resize is placed;
//   * an input that is one output of a channel Split whose outputs are
//     consecutive inputs of the Concat (YOLO's C2f blocks) is placed with all
//     of them, the Split's input covering their ranges: the Split itself then
//     has nothing to copy;
//   * every other reader of a placed tensor must be such a conv (as its x),
//     an Add or a stride-1 MaxPool (SPPF's, which also writes its output
//     into the buffer), so it can read through the view; the Concat's
//     output is the buffer itself, so its readers must be too.
// Every channel of a buffer has exactly one writer per run (its placed
// tensor's producer, or the Concat's copy), so no other tensor's data is
// ever overwritten there.  Like the other handoffs the views are in force
// only while handoffs_live(): otherwise every node reads and writes its own
// tensors, as the reference does.  SPKV2_CONCAT_VIEWS=0 turns them off.
#include <cstdlib>
#include <map>
#include <utility>
#include <vector>

#include "common.hpp"
#include "conv.hpp"
#include "kernels.hpp"

namespace spk::kern {
namespace {

struct Uses {
    std::vector<int> producer;                                   // node id per tensor, -1: none
    std::vector<std::vector<std::pair<uint32_t, int>>> readers;  // (node id, input slot) per tensor
    std::vector<uint8_t> graph_io;                               // graph outputs
};

// An fp32 NCHW activation the runtime places itself (not a graph input or
// output, not caller-bound).
bool movable(const Spkv2Context *ctx, const Uses &u, uint32_t t) {
    const Spkv2TensorRecord *r = rec(ctx, t);
    return r->rank == 4 && r->dtype == SPKV2_DTYPE_FP32 && r->role == SPKV2_ROLE_ACTIVATION &&
           r->memory_class == SPKV2_MEMORY_ACTIVATION_ARENA && !u.graph_io[t] && r->size_bytes > 0 &&
           !ctx->views[t].base;
}

// movable, of rank r (movable itself asks for an NCHW activation)
bool movable_rank(const Spkv2Context *ctx, const Uses &u, uint32_t t, int r) {
    const Spkv2TensorRecord *x = rec(ctx, t);
    return x->rank == r && x->dtype == SPKV2_DTYPE_FP32 && x->role == SPKV2_ROLE_ACTIVATION &&
           x->memory_class == SPKV2_MEMORY_ACTIVATION_ARENA && !u.graph_io[t] && x->size_bytes > 0 &&
           !ctx->views[t].base;
}

int axis_of(const Spkv2Context *ctx, const Spkv2NodeRecord *n, int rank) {
    Spkv2AttrRecord attr;
    if (spkv2_ctx_get_attr(ctx, n, &attr) != 0) return -1;
    return attr.axis < 0 ? attr.axis + rank : attr.axis;
}

// The node's fp32 implicit-GEMM conv plan, when a built-in runs it that way.
const ConvPlan *f32_conv(const Spkv2Context *ctx, uint32_t id) {
    const Spkv2NodeRecord *n = &ctx->node_records[id];
    if (n->op_type != SPKV2_OP_CONV || !builtin_runs(ctx, id) || ctx->plan_dtors[id] != conv_plan_free) return nullptr;
    const ConvPlan *p = static_cast<const ConvPlan *>(ctx->plans[id]);
    return p && p->path == CONV_IGEMM_F32 ? p : nullptr;
}

// An Add of two same-shape fp32 NCHW tensors (binary_run's image-strided
// kernels: float4s when every view base and image stride is 16-byte
// aligned, scalar elements otherwise).
bool same_shape_add(const Spkv2Context *ctx, uint32_t id) {
    const Spkv2NodeRecord *n = &ctx->node_records[id];
    if (n->op_type != SPKV2_OP_ADD || !builtin_runs(ctx, id) || n->input_count != 2 || n->output_count != 1)
        return false;
    const Spkv2TensorRecord *y = rec(ctx, n->outputs[0]);
    if (y->rank != 4 || y->dtype != SPKV2_DTYPE_FP32) return false;
    for (int k = 0; k < 2; k++) {
        const Spkv2TensorRecord *r = rec(ctx, n->inputs[k]);
        if (r->rank != 4 || r->dtype != SPKV2_DTYPE_FP32) return false;
        for (int d = 0; d < 4; d++)
            if (r->shape[d] != y->shape[d]) return false;
    }
    return true;
}

// A 2x nearest Resize of an fp32 NCHW tensor that resize_run's 2x kernel
// runs (even width, same N and C), which takes y's image stride.
bool resize2x(const Spkv2Context *ctx, uint32_t id) {
    const Spkv2NodeRecord *n = &ctx->node_records[id];
    if (n->op_type != SPKV2_OP_RESIZE || !builtin_runs(ctx, id) || n->input_count < 1 || n->output_count != 1)
        return false;
    const Spkv2TensorRecord *x = rec(ctx, n->inputs[0]), *y = rec(ctx, n->outputs[0]);
    return x->rank == 4 && y->rank == 4 && x->dtype == SPKV2_DTYPE_FP32 && y->dtype == SPKV2_DTYPE_FP32 &&
           y->shape[0] == x->shape[0] && y->shape[1] == x->shape[1] && y->shape[2] == 2 * x->shape[2] &&
           y->shape[3] == 2 * x->shape[3] && x->shape[3] % 2 == 0;
}

// A stride-1 MaxPool of an fp32 NCHW tensor (SPPF's): maxpool_run takes it
// on its generic kernel, which reads and writes through image strides.
bool stride1_maxpool(const Spkv2Context *ctx, uint32_t id) {
    const Spkv2NodeRecord *n = &ctx->node_records[id];
    if (n->op_type != SPKV2_OP_MAXPOOL || !builtin_runs(ctx, id) || n->input_count < 1 || n->output_count != 1)
        return false;
    Spkv2AttrRecord attr;
    if (spkv2_ctx_get_attr(ctx, n, &attr) != 0 || attr.strides[0] != 1 || attr.strides[1] != 1) return false;
    const Spkv2TensorRecord *x = rec(ctx, n->inputs[0]), *y = rec(ctx, n->outputs[0]);
    return x->rank == 4 && y->rank == 4 && x->dtype == SPKV2_DTYPE_FP32 && y->dtype == SPKV2_DTYPE_FP32;
}

// The producer of t can write it through a view.
bool strided_writer(const Spkv2Context *ctx, const Uses &u, uint32_t t) {
    const int p = u.producer[t];
    if (p < 0) return false;
    const Spkv2NodeRecord *n = &ctx->node_records[p];
    if (const ConvPlan *cp = f32_conv(ctx, static_cast<uint32_t>(p)))
        return !cp->g.has_res && n->output_count == 1 && n->outputs[0] == t;
    return same_shape_add(ctx, static_cast<uint32_t>(p)) || resize2x(ctx, static_cast<uint32_t>(p)) ||
           stride1_maxpool(ctx, static_cast<uint32_t>(p));
}

// Every reader of t but `owner` reads it through a view (a conv as its
// input x, an Add), and `owner` reads it at most once.
bool readers_ok(const Spkv2Context *ctx, const Uses &u, uint32_t t, uint32_t owner) {
    int owner_reads = 0;
    for (const auto &[id, slot] : u.readers[t]) {
        if (id == owner) {
            if (++owner_reads > 1) return false;
            continue;
        }
        if (f32_conv(ctx, id) && slot == 0) continue;
        if (same_shape_add(ctx, id)) continue;
        if (stride1_maxpool(ctx, id) && slot == 0) continue;
        return false;
    }
    return true;
}

struct Placement {
    std::map<uint32_t, int64_t> channel;  // tensor -> first channel in the Concat buffer
    std::vector<uint32_t> splits;         // Splits whose outputs all became views
};

// Places input i of Concat k (first channel c[i]) and, through a Split, its
// siblings: false when it stays a copy.
bool place_input(const Spkv2Context *ctx, const Uses &u, const Spkv2NodeRecord *k, int i, const std::vector<int64_t> &c,
                 Placement *pl) {
    const uint32_t t = k->inputs[i];
    if (!movable(ctx, u, t)) return false;
    const int p = u.producer[t];
    if (p >= 0 && ctx->node_records[p].op_type == SPKV2_OP_SPLIT) {
        const Spkv2NodeRecord *sp = &ctx->node_records[p];
        if (!builtin_runs(ctx, static_cast<uint32_t>(p)) || sp->input_count < 1) return false;
        const uint32_t s = sp->inputs[0];
        if (!movable(ctx, u, s) || axis_of(ctx, sp, 4) != 1) return false;
        int j = -1;
        for (int q = 0; q < sp->output_count; q++)
            if (sp->outputs[q] == t) j = q;
        // the Split's outputs, in order, are inputs i - j .. of the Concat
        const int first = i - j;
        if (j < 0 || first < 0 || first + sp->output_count > k->input_count) return false;
        for (int q = 0; q < sp->output_count; q++) {
            const uint32_t o = sp->outputs[q];
            if (k->inputs[first + q] != o || !movable(ctx, u, o) || !readers_ok(ctx, u, o, k->id)) return false;
        }
        if (!strided_writer(ctx, u, s) || !readers_ok(ctx, u, s, sp->id)) return false;
        pl->channel[s] = c[first];
        for (int q = 0; q < sp->output_count; q++) pl->channel[sp->outputs[q]] = c[first + q];
        pl->splits.push_back(sp->id);
        return true;
    }
    if (!strided_writer(ctx, u, t) || !readers_ok(ctx, u, t, k->id)) return false;
    pl->channel[t] = c[i];
    return true;
}

// Detection-head chains (YOLO's head): per level, a channel Concat of convs
// (box and class branches), flattened by a Reshape [N, C, H, W] ->
// [N, C, H*W]; the levels joined by a Concat along axis 2 into [N, C, L];
// that read by one channel Split (box and class again).  The convs write
// their outputs straight into one buffer laid out as the [N, C, L] tensor
// (channel stride L, each level at its offset along L), the per-level
// Concats, the Reshapes and the level Concat have nothing left to do, and the
// Split reads the buffer.  Every intermediate must have exactly one reader
// (the next node of the chain).
void setup_head_views(Spkv2Context *ctx, const Uses &u) {
    const uint32_t nn = ctx->header.num_nodes;
    auto sole_reader = [&](uint32_t t, uint32_t node) {
        return u.readers[t].size() == 1 && u.readers[t][0].first == node;
    };
    for (uint32_t id = 0; id < nn; id++) {
        const Spkv2NodeRecord *k2 = &ctx->node_records[id];
        if (k2->op_type != SPKV2_OP_CONCAT || !builtin_runs(ctx, id) || k2->output_count != 1) continue;
        const uint32_t o = k2->outputs[0];
        const Spkv2TensorRecord *orr = rec(ctx, o);
        if (!movable_rank(ctx, u, o, 3) || axis_of(ctx, k2, 3) != 2 || u.readers[o].size() != 1) continue;
        const uint32_t sp = u.readers[o][0].first;
        const Spkv2NodeRecord *split = &ctx->node_records[sp];
        if (split->op_type != SPKV2_OP_SPLIT || !builtin_runs(ctx, sp) || u.readers[o][0].second != 0 ||
            axis_of(ctx, split, 3) != 1)
            continue;
        const int64_t N = orr->shape[0], C = orr->shape[1], L = orr->shape[2];
        const int64_t zbytes = N * C * L * 4;
        if (zbytes >= (int64_t(1) << 31)) continue;
        struct Place {
            uint32_t t;
            int64_t off;  // elements from the buffer's start
        };
        std::vector<Place> places;
        std::vector<uint32_t> elide;
        int64_t l0 = 0;
        bool ok = true;
        for (uint16_t i = 0; i < k2->input_count && ok; i++) {
            const uint32_t r = k2->inputs[i];
            const int pr = u.producer[r];
            ok = movable_rank(ctx, u, r, 3) && sole_reader(r, id) && pr >= 0 &&
                 ctx->node_records[pr].op_type == SPKV2_OP_RESHAPE && builtin_runs(ctx, static_cast<uint32_t>(pr));
            if (!ok) break;
            const Spkv2TensorRecord *rr = rec(ctx, r);
            const uint32_t c = ctx->node_records[pr].inputs[0];
            const int pk = u.producer[c];
            ok = rr->shape[0] == N && rr->shape[1] == C && movable_rank(ctx, u, c, 4) &&
                 sole_reader(c, static_cast<uint32_t>(pr)) && pk >= 0 &&
                 ctx->node_records[pk].op_type == SPKV2_OP_CONCAT && builtin_runs(ctx, static_cast<uint32_t>(pk));
            if (!ok) break;
            const Spkv2TensorRecord *cr = rec(ctx, c);
            const Spkv2NodeRecord *k1 = &ctx->node_records[pk];
            const int64_t HW = static_cast<int64_t>(cr->shape[2]) * cr->shape[3];
            ok = cr->shape[0] == N && cr->shape[1] == C && HW == rr->shape[2] && k1->output_count == 1 &&
                 axis_of(ctx, k1, 4) == 1;
            int64_t c0 = 0;
            for (uint16_t j = 0; j < k1->input_count && ok; j++) {
                const uint32_t t = k1->inputs[j];
                const Spkv2TensorRecord *tr = rec(ctx, t);
                // a conv writer (its epilogues take a channel stride; the
                // Add kernel's image-strided form does not)
                ok = movable_rank(ctx, u, t, 4) && sole_reader(t, static_cast<uint32_t>(pk)) &&
                     strided_writer(ctx, u, t) && u.producer[t] >= 0 &&
                     f32_conv(ctx, static_cast<uint32_t>(u.producer[t])) && tr->shape[0] == N &&
                     tr->shape[2] == cr->shape[2] && tr->shape[3] == cr->shape[3];
                if (ok) places.push_back({t, c0 * L + l0});
                c0 += tr->shape[1];
            }
            ok = ok && c0 == C;
            elide.push_back(static_cast<uint32_t>(pk));
            elide.push_back(static_cast<uint32_t>(pr));
            l0 += HW;
        }
        if (!ok || l0 != L || places.empty()) continue;
        void *z = nullptr;
        if (hipMalloc(&z, static_cast<size_t>(zbytes)) != hipSuccess) {
            (void)hipGetLastError();
            continue;  // the chain keeps its copies
        }
        ctx->view_buffers.push_back(z);
        uint8_t *zb = static_cast<uint8_t *>(z);
        for (const Place &pl : places)
            ctx->views[pl.t] = Spkv2TensorView{zb + pl.off * 4, C * L, static_cast<size_t>(zbytes - pl.off * 4), L};
        ctx->views[o] = Spkv2TensorView{zb, C * L, static_cast<size_t>(zbytes), L};
        for (uint32_t e : elide) ctx->view_elide[e] = 1;
        ctx->view_elide[id] = 1;
    }
}

}  // namespace

int setup_concat_views(Spkv2Context *ctx) {
    const uint32_t nt = ctx->header.num_tensors, nn = ctx->header.num_nodes;
    ctx->views.assign(nt, Spkv2TensorView{});
    ctx->view_split.assign(nn, 0);
    ctx->view_elide.assign(nn, 0);
    if (ctx->protection_count > 0) return 0;  // protected packages keep every tensor where the reference has it
    if (const char *e = getenv("SPKV2_CONCAT_VIEWS"))
        if (e[0] == '0') return 0;
    Uses u;
    u.producer.assign(nt, -1);
    u.readers.assign(nt, {});
    u.graph_io.assign(nt, 0);
    for (size_t i = 0; i < ctx->output_count; i++)
        if (ctx->output_ids[i] < nt) u.graph_io[ctx->output_ids[i]] = 1;
    for (uint32_t i = 0; i < nn; i++) {
        const Spkv2NodeRecord *n = &ctx->node_records[i];
        for (uint16_t q = 0; q < n->output_count; q++)
            if (n->outputs[q] < nt) u.producer[n->outputs[q]] = static_cast<int>(i);
        for (uint16_t q = 0; q < n->input_count; q++)
            if (n->inputs[q] < nt) u.readers[n->inputs[q]].push_back({i, q});
    }
    for (uint32_t id = 0; id < nn; id++) {
        const Spkv2NodeRecord *k = &ctx->node_records[id];
        if (k->op_type != SPKV2_OP_CONCAT || !builtin_runs(ctx, id) || k->output_count != 1) continue;
        const uint32_t o = k->outputs[0];
        if (!movable(ctx, u, o) || axis_of(ctx, k, 4) != 1) continue;
        const Spkv2TensorRecord *yr = rec(ctx, o);
        const int64_t N = yr->shape[0], CZ = yr->shape[1], HW = static_cast<int64_t>(yr->shape[2]) * yr->shape[3];
        const int64_t zbytes = N * CZ * HW * 4;
        if (zbytes >= (int64_t(1) << 31)) continue;  // 32-bit byte offsets in the kernels
        bool shapes = true;
        std::vector<int64_t> c(k->input_count + 1, 0);
        for (uint16_t i = 0; i < k->input_count; i++) {
            const Spkv2TensorRecord *r = rec(ctx, k->inputs[i]);
            shapes = shapes && r->rank == 4 && r->dtype == SPKV2_DTYPE_FP32 && r->shape[0] == yr->shape[0] &&
                     r->shape[2] == yr->shape[2] && r->shape[3] == yr->shape[3];
            c[i + 1] = c[i] + r->shape[1];
        }
        // the output is read through its view: by convs and Adds only
        if (!shapes || c[k->input_count] != CZ || !readers_ok(ctx, u, o, id)) continue;
        Placement pl;
        for (int i = 0; i < k->input_count; i++) {
            const auto it = pl.channel.find(k->inputs[i]);
            if (it != pl.channel.end()) continue;  // placed with its Split siblings
            (void)place_input(ctx, u, k, i, c, &pl);
        }
        if (pl.channel.empty()) continue;
        // at batch 1 the memory plan may have placed inputs inside the output
        // already (no copy): views there only when no input is left to copy
        if (N == 1) {
            int placed = 0;
            for (uint16_t i = 0; i < k->input_count; i++) placed += pl.channel.count(k->inputs[i]) ? 1 : 0;
            if (placed < k->input_count) continue;
        }
        void *z = nullptr;
        if (hipMalloc(&z, static_cast<size_t>(zbytes)) != hipSuccess) {
            (void)hipGetLastError();
            continue;  // an optimization only: this Concat keeps its copies
        }
        ctx->view_buffers.push_back(z);
        uint8_t *zb = static_cast<uint8_t *>(z);
        for (const auto &[t, ch] : pl.channel) {
            const int64_t ct = rec(ctx, t)->shape[1];
            ctx->views[t] = Spkv2TensorView{zb + ch * HW * 4, CZ * HW, static_cast<size_t>(((N - 1) * CZ + ct) * HW * 4)};
        }
        ctx->views[o] = Spkv2TensorView{zb, CZ * HW, static_cast<size_t>(zbytes)};
        for (uint32_t s : pl.splits) ctx->view_split[s] = 1;
    }
    setup_head_views(ctx, u);
    return 0;
}

}  // namespace spk::kern
