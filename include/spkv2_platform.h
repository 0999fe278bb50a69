/*
 * Host platform hooks (reference: runtime/include/spkv2_platform.h).
 *
 * The allocation hooks back every host-side allocation the runtime makes
 * (context, tensor tables, output-id list).  The CPU threading and GEMM-tiling
 * knobs of the reference have no meaning for a GPU backend; they are exported
 * so that code linking against them keeps building, store their value, and
 * change nothing on the device.
 */
#ifndef SPKV2_PLATFORM_H
#define SPKV2_PLATFORM_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference: runtime/platform/platform.c:254-256 */
void *spkv2_platform_malloc(size_t size);
void *spkv2_platform_calloc(size_t count, size_t size);
void spkv2_platform_free(void *ptr);

/* reference: runtime/include/spkv2_platform.h:18-53 (stored, no device effect) */
void spkv2_set_num_threads(int n);
int spkv2_get_num_threads(void);
void spkv2_set_gemm_tiling(int kc, int nc);
int spkv2_get_gemm_kc(void);
int spkv2_get_gemm_nc(void);
void spkv2_auto_tune_gemm(int l1_bytes, int l2_bytes);
void spkv2_set_parallel_cost_threshold(int threshold_ns);
int spkv2_get_parallel_cost_threshold(void);
int spkv2_should_parallelize(int count, int cost_per_unit_ns);

#define SPKV2_CORES_ALL 0
#define SPKV2_CORES_BIG 1
#define SPKV2_CORES_LITTLE 2

typedef struct {
    int num_big;
    int num_little;
    int big_core_ids[16];
    int little_core_ids[16];
    int detected;
} Spkv2CoreTopology;

void spkv2_detect_topology(void);
const Spkv2CoreTopology *spkv2_get_topology(void);
void spkv2_set_affinity(int core_type);

#ifdef __cplusplus
}
#endif

#endif /* SPKV2_PLATFORM_H */
