// SPK loading and context teardown.
//
// Behaviour follows the reference loader (runtime/core/loader.c:105-305):
// magic / major version (-2), directory and section bounds (-3), required
// tensor/node/attr/weight sections (-4), FNV-1a checksum (-5 missing, -6
// mismatch), optional memory-plan / kernel-spec / quantization / protection
// tables, output order from the metadata JSON "outputs" array.
#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "context.hpp"
#include "spkv2_mi355x.h"
#include "spkv2_platform.h"

namespace {

const Spkv2SectionEntry *find_section(const Spkv2Context *ctx, uint32_t kind) {
    for (uint32_t i = 0; i < ctx->header.section_count; i++)
        if (ctx->sections[i].kind == kind) return &ctx->sections[i];
    return nullptr;
}

uint32_t fnv1a32(const uint8_t *p, size_t n) {
    uint32_t h = 2166136261u;
    for (size_t i = 0; i < n; i++) {
        h ^= p[i];
        h *= 16777619u;
    }
    return h;
}

// Finds `"outputs": [id, id, ...]` in the metadata JSON (reference
// loader.c:46-103).  A malformed or short list leaves output_ids unset, in
// which case outputs are taken in tensor-table order.
// IEEE binary16 -> binary32, exact for every input (subnormals normalised,
// infinities kept, NaN payloads shifted into the high mantissa bits).
uint32_t half_bits_to_float_bits(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0x1fu) return sign | 0x7f800000u | (man << 13);
    if (exp != 0) return sign | ((exp + 112u) << 23) | (man << 13);
    if (man == 0) return sign;
    uint32_t e = 113;  // value = man * 2^-24; normalise so bit 10 leads
    while (!(man & 0x400u)) {
        man <<= 1;
        e--;
    }
    return sign | (e << 23) | ((man & 0x3ffu) << 13);
}

// FP16 weights (the reference's --fp16-weights packages,
// compiler/passes/convert_fp16.py:11-25) are widened to fp32 once at load, as
// the reference's optimized conv and gemm do per node
// (runtime/kernels/optimized/conv/conv.c:961-978, mm/gemm.c:150-162).  The
// context's tensor table becomes a copy whose half weight records describe
// fp32 copies appended after the package's weight bytes, so every kernel
// (and every user kernel reading spkv2_ctx_tensor_record) sees fp32 weights.
int promote_fp16_weights(Spkv2Context *ctx) {
    const uint32_t nt = ctx->header.num_tensors;
    size_t extra = 0;
    const size_t base = (ctx->weights_size + 255) & ~static_cast<size_t>(255);
    for (uint32_t i = 0; i < nt; i++) {
        const Spkv2TensorRecord &r = ctx->tensor_records[i];
        if (r.role != SPKV2_ROLE_WEIGHT || r.dtype != SPKV2_DTYPE_FP16) continue;
        if (r.data_offset > ctx->weights_size || r.size_bytes > ctx->weights_size - r.data_offset ||
            r.size_bytes % 2)
            return -3;
        extra += ((r.size_bytes * 2) + 255) & ~static_cast<uint64_t>(255);
    }
    if (extra == 0) return 0;
    ctx->promoted_records = static_cast<Spkv2TensorRecord *>(spkv2_platform_malloc(nt * sizeof(Spkv2TensorRecord)));
    ctx->promoted_weights = static_cast<uint8_t *>(spkv2_platform_calloc(base + extra, 1));
    if (!ctx->promoted_records || !ctx->promoted_weights) return -1;
    memcpy(ctx->promoted_records, ctx->tensor_records, nt * sizeof(Spkv2TensorRecord));
    memcpy(ctx->promoted_weights, ctx->weights_host, ctx->weights_size);
    size_t off = base;
    for (uint32_t i = 0; i < nt; i++) {
        Spkv2TensorRecord &r = ctx->promoted_records[i];
        if (r.role != SPKV2_ROLE_WEIGHT || r.dtype != SPKV2_DTYPE_FP16) continue;
        const size_t n = static_cast<size_t>(r.size_bytes / 2);
        spkv2_mi355x_fp16_to_fp32(ctx->weights_host + r.data_offset, ctx->promoted_weights + off, n);
        r.dtype = SPKV2_DTYPE_FP32;
        r.size_bytes = n * 4;
        r.data_offset = off;
        off += (n * 4 + 255) & ~static_cast<size_t>(255);
    }
    ctx->tensor_records = ctx->promoted_records;
    ctx->weights_host = ctx->promoted_weights;
    ctx->weights_size = off;
    return 0;
}

int parse_output_order(Spkv2Context *ctx, const Spkv2SectionEntry *meta) {
    if (!meta || meta->size == 0 || ctx->header.num_outputs == 0) return 0;
    const char *p = reinterpret_cast<const char *>(ctx->model + meta->offset);
    const char *end = p + meta->size;
    static const char key[] = "\"outputs\"";
    const size_t klen = sizeof(key) - 1;
    auto skip_ws = [&](const char *q) {
        while (q < end && isspace(static_cast<unsigned char>(*q))) q++;
        return q;
    };
    for (const char *q = p; q + klen <= end; q++) {
        if (memcmp(q, key, klen) != 0) continue;
        const char *r = skip_ws(q + klen);
        if (r >= end || *r != ':') continue;
        r = skip_ws(r + 1);
        if (r >= end || *r != '[') continue;
        r++;
        uint32_t *ids = static_cast<uint32_t *>(spkv2_platform_calloc(ctx->header.num_outputs, sizeof(uint32_t)));
        if (!ids) return -1;
        size_t count = 0;
        bool ok = true;
        for (;;) {
            r = skip_ws(r);
            if (r >= end) break;
            if (*r == ']') break;
            // strtoul needs a terminated buffer: copy the digits out
            char digits[24];
            size_t nd = 0;
            while (r < end && nd + 1 < sizeof(digits) && isdigit(static_cast<unsigned char>(*r))) digits[nd++] = *r++;
            digits[nd] = 0;
            if (nd == 0) { ok = false; break; }
            unsigned long v = strtoul(digits, nullptr, 10);
            if (v >= ctx->header.num_tensors || count >= ctx->header.num_outputs) { ok = false; break; }
            ids[count++] = static_cast<uint32_t>(v);
            r = skip_ws(r);
            if (r < end && *r == ',') { r++; continue; }
            if (r < end && *r == ']') break;
            ok = false;
            break;
        }
        if (ok && count == ctx->header.num_outputs) {
            ctx->output_ids = ids;
            ctx->output_count = count;
        } else {
            spkv2_platform_free(ids);
        }
        return 0;
    }
    return 0;
}

void destroy(Spkv2Context *ctx) {
    if (!ctx) return;
    if (ctx->node_cache) {
        for (size_t i = 0; i < ctx->node_count; i++) {
            if (!ctx->node_cache[i]) continue;
            if (ctx->node_cache_dtors && ctx->node_cache_dtors[i]) ctx->node_cache_dtors[i](ctx->node_cache[i]);
            else spkv2_platform_free(ctx->node_cache[i]);
        }
    }
    for (size_t i = 0; i < ctx->plans.size(); i++)
        if (ctx->plans[i] && ctx->plan_dtors[i]) ctx->plan_dtors[i](ctx->plans[i]);
    if (ctx->prepared || ctx->stream) {
        (void)hipSetDevice(ctx->device);
        if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
        if (ctx->graph_exec) (void)hipGraphExecDestroy(ctx->graph_exec);
        for (hipEvent_t e : ctx->ev_begin) (void)hipEventDestroy(e);
        for (hipEvent_t e : ctx->ev_end) (void)hipEventDestroy(e);
        if (ctx->owns_arena && ctx->arena) (void)hipFree(ctx->arena);
        if (ctx->owns_scratch && ctx->scratch) (void)hipFree(ctx->scratch);
        if (ctx->workspace) (void)hipFree(ctx->workspace);
        if (ctx->weights_dev) (void)hipFree(ctx->weights_dev);
        if (ctx->dev_minmax) (void)hipFree(ctx->dev_minmax);
        if (ctx->dev_flag) (void)hipFree(ctx->dev_flag);
        for (int32_t *p : ctx->acc_capture)
            if (p) (void)hipFree(p);
        for (void *p : ctx->view_buffers) (void)hipFree(p);
        for (Spkv2Q8Tensor &t : ctx->q8)
            if (t.buf) (void)hipFree(t.buf);
        if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    }
    spkv2_platform_free(ctx->node_cache);
    spkv2_platform_free(ctx->node_cache_dtors);
    spkv2_platform_free(ctx->ranges);
    spkv2_platform_free(ctx->invocations);
    spkv2_platform_free(ctx->output_ids);
    spkv2_platform_free(ctx->tensors);
    spkv2_platform_free(ctx->owned_model);
    spkv2_platform_free(ctx->promoted_records);
    spkv2_platform_free(ctx->promoted_weights);
    ctx->~Spkv2Context();
    spkv2_platform_free(ctx);
}

}  // namespace

extern "C" int spkv2_load_memory(const void *data, size_t size, Spkv2Context **out_ctx) {
    if (!data || !out_ctx || size < sizeof(Spkv2Header)) return -1;
    void *mem = spkv2_platform_calloc(1, sizeof(Spkv2Context));
    if (!mem) return -1;
    Spkv2Context *ctx = new (mem) Spkv2Context();
    auto fail = [&](int rc) {
        destroy(ctx);
        return rc;
    };

    memcpy(&ctx->header, data, sizeof(Spkv2Header));
    if (ctx->header.magic != SPKV2_MAGIC || ctx->header.version_major != SPKV2_VERSION_MAJOR) return fail(-2);
    const size_t dir_off = ctx->header.header_size;
    const size_t dir_size = static_cast<size_t>(ctx->header.section_count) * sizeof(Spkv2SectionEntry);
    if (dir_off > size || dir_size > size - dir_off) return fail(-3);

    ctx->model = static_cast<const uint8_t *>(data);
    ctx->model_size = size;
    ctx->sections = reinterpret_cast<const Spkv2SectionEntry *>(ctx->model + dir_off);
    for (uint32_t i = 0; i < ctx->header.section_count; i++) {
        const Spkv2SectionEntry &s = ctx->sections[i];
        if (s.offset > size || s.size > size - s.offset) return fail(-3);
    }

    const Spkv2SectionEntry *tensor_sec = find_section(ctx, SPKV2_SECTION_TENSOR_TABLE);
    const Spkv2SectionEntry *node_sec = find_section(ctx, SPKV2_SECTION_NODE_TABLE);
    const Spkv2SectionEntry *attr_sec = find_section(ctx, SPKV2_SECTION_ATTRIBUTES);
    const Spkv2SectionEntry *weight_sec = find_section(ctx, SPKV2_SECTION_WEIGHTS);
    if (!tensor_sec || !node_sec || !attr_sec || !weight_sec) return fail(-4);
    if (tensor_sec->size < static_cast<uint64_t>(ctx->header.num_tensors) * sizeof(Spkv2TensorRecord)) return fail(-4);
    if (node_sec->size < static_cast<uint64_t>(ctx->header.num_nodes) * sizeof(Spkv2NodeRecord)) return fail(-4);

    if (ctx->header.checksum_type == 1) {
        const Spkv2SectionEntry *cs = find_section(ctx, SPKV2_SECTION_CHECKSUM);
        if (!cs || cs->size < sizeof(uint32_t)) return fail(-5);
        uint32_t expected;
        memcpy(&expected, ctx->model + cs->offset, sizeof(expected));
        if (fnv1a32(ctx->model, static_cast<size_t>(cs->offset)) != expected) return fail(-6);
    }

    ctx->tensor_records = reinterpret_cast<const Spkv2TensorRecord *>(ctx->model + tensor_sec->offset);
    ctx->node_records = reinterpret_cast<const Spkv2NodeRecord *>(ctx->model + node_sec->offset);
    if (const Spkv2SectionEntry *s = find_section(ctx, SPKV2_SECTION_MEMORY_PLAN)) {
        if (s->size >= static_cast<uint64_t>(ctx->header.num_tensors) * sizeof(Spkv2MemoryPlanRecord)) {
            ctx->plan_records = reinterpret_cast<const Spkv2MemoryPlanRecord *>(ctx->model + s->offset);
            ctx->plan_count = s->size / sizeof(Spkv2MemoryPlanRecord);
        }
    }
    if (const Spkv2SectionEntry *s = find_section(ctx, SPKV2_SECTION_KERNEL_SPEC)) {
        if (s->size >= static_cast<uint64_t>(ctx->header.num_nodes) * sizeof(Spkv2KernelSpecRecord)) {
            ctx->spec_records = reinterpret_cast<const Spkv2KernelSpecRecord *>(ctx->model + s->offset);
            ctx->spec_count = s->size / sizeof(Spkv2KernelSpecRecord);
        }
    }
    // Quantization: the first record's data_offset marks the end of the record
    // array, which gives the record count (reference loader.c:220-234).
    if (const Spkv2SectionEntry *s = find_section(ctx, SPKV2_SECTION_QUANTIZATION)) {
        if (s->size >= sizeof(Spkv2QuantParamRecord)) {
            const uint8_t *base = ctx->model + s->offset;
            Spkv2QuantParamRecord first;
            memcpy(&first, base, sizeof(first));
            if (first.data_offset > 0) {
                size_t count = first.data_offset / sizeof(Spkv2QuantParamRecord);
                if (count > 0 && count * sizeof(Spkv2QuantParamRecord) <= s->size) {
                    ctx->quant_records = reinterpret_cast<const Spkv2QuantParamRecord *>(base);
                    ctx->quant_count = count;
                    ctx->quant_data = base;
                    ctx->quant_data_size = s->size;
                }
            }
        }
    }
    if (const Spkv2SectionEntry *s = find_section(ctx, SPKV2_SECTION_PROTECTION_PLAN)) {
        if (s->size >= sizeof(Spkv2ProtectionRecord)) {
            ctx->protection_records = reinterpret_cast<const Spkv2ProtectionRecord *>(ctx->model + s->offset);
            ctx->protection_count = s->size / sizeof(Spkv2ProtectionRecord);
        }
    }
    ctx->attrs = ctx->model + attr_sec->offset;
    ctx->attrs_size = attr_sec->size;
    ctx->weights_host = ctx->model + weight_sec->offset;
    ctx->weights_size = weight_sec->size;
    if (int rc = promote_fp16_weights(ctx)) return fail(rc);

    ctx->tensors = static_cast<Spkv2TensorSlot *>(spkv2_platform_calloc(ctx->header.num_tensors ? ctx->header.num_tensors : 1,
                                                                        sizeof(Spkv2TensorSlot)));
    if (!ctx->tensors) return fail(-1);
    for (uint32_t i = 0; i < ctx->header.num_tensors; i++) ctx->tensors[i].record = &ctx->tensor_records[i];

    if (parse_output_order(ctx, find_section(ctx, SPKV2_SECTION_METADATA)) != 0) return fail(-1);

    ctx->node_count = ctx->header.num_nodes;
    if (ctx->node_count > 0) {
        ctx->node_cache = static_cast<void **>(spkv2_platform_calloc(ctx->node_count, sizeof(void *)));
        ctx->node_cache_dtors =
            static_cast<void (**)(void *)>(spkv2_platform_calloc(ctx->node_count, sizeof(void (*)(void *))));
        ctx->invocations = static_cast<uint32_t *>(spkv2_platform_calloc(ctx->node_count, sizeof(uint32_t)));
        ctx->ranges =
            static_cast<Spkv2RangeObservation *>(spkv2_platform_calloc(ctx->node_count, sizeof(Spkv2RangeObservation)));
        if (!ctx->node_cache || !ctx->node_cache_dtors || !ctx->invocations || !ctx->ranges) return fail(-1);
        ctx->node_kernel_names.resize(ctx->node_count);
        ctx->plans.assign(ctx->node_count, nullptr);
        ctx->plan_dtors.assign(ctx->node_count, nullptr);
        ctx->node_ms.assign(ctx->node_count, 0.0);
        ctx->node_runs.assign(ctx->node_count, 0);
    }
    *out_ctx = ctx;
    return 0;
}

extern "C" int spkv2_load_file(const char *path, Spkv2Context **out_ctx) {
    if (!path || !out_ctx) return -1;
    FILE *fp = fopen(path, "rb");
    if (!fp) return -1;
    if (fseek(fp, 0, SEEK_END) != 0) { fclose(fp); return -1; }
    long size = ftell(fp);
    if (size <= 0) { fclose(fp); return -1; }
    rewind(fp);
    uint8_t *blob = static_cast<uint8_t *>(spkv2_platform_malloc(static_cast<size_t>(size)));
    if (!blob) { fclose(fp); return -1; }
    size_t got = fread(blob, 1, static_cast<size_t>(size), fp);
    fclose(fp);
    if (got != static_cast<size_t>(size)) { spkv2_platform_free(blob); return -1; }
    int rc = spkv2_load_memory(blob, static_cast<size_t>(size), out_ctx);
    if (rc != 0) { spkv2_platform_free(blob); return rc; }
    (*out_ctx)->owned_model = blob;
    return 0;
}

extern "C" void spkv2_free(Spkv2Context *ctx) { destroy(ctx); }

extern "C" const char *spkv2_runtime_version(void) { return "0.3.0-mi355x"; }

extern "C" void spkv2_mi355x_fp16_to_fp32(const void *src, void *dst, size_t count) {
    const uint8_t *in = static_cast<const uint8_t *>(src);
    uint8_t *out = static_cast<uint8_t *>(dst);
    for (size_t i = 0; i < count; i++) {
        uint16_t h;
        memcpy(&h, in + 2 * i, 2);
        const uint32_t f = half_bits_to_float_bits(h);
        memcpy(out + 4 * i, &f, 4);
    }
}

extern "C" uint32_t spkv2_fnv1a32(const void *data, size_t size) {
    return data ? fnv1a32(static_cast<const uint8_t *>(data), size) : 2166136261u;
}
