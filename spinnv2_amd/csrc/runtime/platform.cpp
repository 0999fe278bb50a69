// Host platform hooks (reference: runtime/platform/platform.c).  Allocation
// goes to libc; the CPU tuning knobs are stored and reported but steer
// nothing, since all node work runs on the GPU.
#include <cstdlib>

#include "spkv2_platform.h"

namespace {
int g_threads = 0;
int g_kc = 256, g_nc = 256;
int g_cost_threshold_ns = 50000;
Spkv2CoreTopology g_topology{};
}  // namespace

extern "C" {
void *spkv2_platform_malloc(size_t size) { return malloc(size); }
void *spkv2_platform_calloc(size_t count, size_t size) { return calloc(count, size); }
void spkv2_platform_free(void *ptr) { free(ptr); }

void spkv2_set_num_threads(int n) { g_threads = n < 0 ? 0 : n; }
int spkv2_get_num_threads(void) { return g_threads; }
void spkv2_set_gemm_tiling(int kc, int nc) {
    if (kc > 0) g_kc = kc;
    if (nc > 0) g_nc = nc;
}
int spkv2_get_gemm_kc(void) { return g_kc; }
int spkv2_get_gemm_nc(void) { return g_nc; }
void spkv2_auto_tune_gemm(int l1_bytes, int l2_bytes) {
    (void)l1_bytes;
    (void)l2_bytes;
}
void spkv2_set_parallel_cost_threshold(int threshold_ns) { g_cost_threshold_ns = threshold_ns; }
int spkv2_get_parallel_cost_threshold(void) { return g_cost_threshold_ns; }
int spkv2_should_parallelize(int count, int cost_per_unit_ns) {
    return static_cast<long long>(count) * cost_per_unit_ns > g_cost_threshold_ns;
}
void spkv2_detect_topology(void) { g_topology.detected = 1; }
const Spkv2CoreTopology *spkv2_get_topology(void) { return &g_topology; }
void spkv2_set_affinity(int core_type) { (void)core_type; }
}
