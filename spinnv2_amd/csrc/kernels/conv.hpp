// Convolution geometry and the per-node plan kept in node_cache.
#pragma once

#include <cstdint>
#include <string>

#include "common.hpp"

namespace spk::kern {

// Shapes and attributes of one Conv node, read the way the reference kernel
// reads them (runtime/kernels/reference/conv/conv.c:5-30): x = inputs[0]
// NCHW, w = inputs[1] OIHW, bias = inputs[2] if present, residual =
// inputs[3] if present (FuseConvAdd), y = outputs[0] NCHW whose H/W come
// from the tensor record.
struct ConvGeom {
    int N, C, H, W;
    int M, KH, KW, OH, OW;
    int sh, sw, ph, pw, dh, dw;
    int group, act;
    bool has_bias, has_res;
    int x_dtype, w_dtype;
    int64_t x_elems, y_elems;
};

int read_conv_geom(const Spkv2Context *ctx, const Spkv2NodeRecord *node, ConvGeom *g);

// CONV_Q8: the int8 implicit GEMM of CONV_IGEMM_I8 in the INT8 configuration
// with int8 tensors between nodes (fixed-point requantizing epilogue)
enum ConvPath {
    CONV_IGEMM_F32 = 0,
    CONV_DIRECT_F32 = 1,
    CONV_IGEMM_I8 = 2,
    CONV_DW_F32 = 3,
    CONV_SMALLK_F32 = 4,
    CONV_Q8 = 5
};

// How an fp32 implicit-GEMM B source is laid out beyond its k-offset table.
// Per tap, for the skinny kernel: k = c * taps + tap sits at c * cstride +
// (tap / KW) * tap_h + (tap % KW) * tap_w elements from the column's base (C
// = 0 when the layer has no such form).  kvec: k is contiguous in aligned
// groups of four (16-byte loads along k).
struct GatherGeom {
    int C = 0, cstride = 0, KW = 1, tap_h = 0, tap_w = 0;
    bool kvec = false;
    // implicit padding: the B source is the unpadded input (H x W, padded by
    // ph / pw at the top / left), every tap bounds-checked through the tap
    // table ktap (device, owned by the plan)
    bool chk = false;
    int chk_H = 0, chk_W = 0, chk_ph = 0, chk_pw = 0;
    const int *ktap = nullptr;
    // row-window kernel (a conv over the padded input; win_len 0 when the
    // layer has no such form): per output row segment of 16 pixels the
    // input window is KH rows of win_len columns of C channels, kept in LDS
    // channel-minor; win_shift = log2 of the lanes one window row takes when
    // loading it; win_rows = N * OH output rows of win_owb 16-pixel
    // segments; kh steps win_dh input rows, kw win_dw columns.
    int win_KH = 0, win_len = 0, win_shift = 0, win_rows = 0, win_owb = 0, win_OH = 0, win_dh = 1, win_dw = 1;
};

struct ConvPlan {
    ConvPath path;
    ConvGeom g;
    int cfg;             // index of the tile configuration
    int BM, BN, BK;      // tile shape
    int m_tiles, n_tiles, k_tiles;
    int splitk, kt_per_split;  // split-K factor and k-tiles per slice
    int dp_tiles, ws_n0;       // hybrid schedule: whole tiles first, partials only from column ws_n0 on
    GatherGeom gather;  // fp32 path: the B source's layout (skinny configurations, KVEC loads)
    int K, Kpad;
    void *wpack;         // device: packed weight panels (fp32 or int8)
    void *ktab;          // device: per-k gather table (byte offsets into the B source)
    int Hp, Wp, pt, pl;  // fp32 path: zero-padded input geometry (Hp == H, Wp == W, no copy, when unpadded)
    bool padded;         // fp32 path: the input is copied into a padded workspace buffer first
    size_t pad_bytes;    // fp32 path: workspace bytes of that padded copy
    float *scales;       // device, int8 path: w_scale[m] * x_scale
    // device, CONV_Q8: per output channel, seven int32 rows of M:
    // -z_x * sum(w[m]), that plus bias_q[m], the multipliers m1[m], m2[m],
    // the shift S, and 2^(S-33), S - 32 (requantization constants computed
    // at prepare)
    int *qrow;
    int x_zp;            // CONV_Q8: the input's zero point
    bool q8_hi;          // CONV_Q8: every row's shift is at least 33 (the 32-bit rounding tail)
    float x_scale;       // int8 path: activation scale
    int quant_split;     // int8 path: first element index of the per-image tail (round half away)
    size_t workspace;    // bytes of device workspace needed per run
    // the workspace lives in the package's scratch arena at the node's
    // kernel spec (its scratch_bytes covers it), else in the runtime's own
    // allocation
    bool ws_in_scratch;
    uint32_t spec_id;
    // int8 requantize handoff.  Producer side: this conv's output is also
    // quantized in its epilogue, with the consuming int8 conv's scale and
    // rounding rule, into that conv's zero-padded NHWC buffer (not owned);
    // q_readers counts the consumers that read q_out; y_needed says whether
    // the fp32 output still has other readers.
    int8_t *q_out;
    int q_Hp, q_Wp, q_Cp, q_pt, q_pl, q_split;
    float q_inv_scale;
    int q_readers;
    bool y_needed;
    // Consumer side: the padded NHWC int8 input its producer writes (owned),
    // or, for a later consumer of the same tensor with the same scale and
    // layout, the first consumer's buffer (q_shared, not owned).
    int8_t *q_in;
    int8_t *q_shared;
    // fp32 handoff, the same for the zero-padded NCHW input of a padded
    // conv: producer side (not owned) and consumer side (owned, unless
    // pad_in_shared: a later consumer of the same tensor with the same
    // padded geometry reads the first consumer's buffer).
    float *pad_out;
    int pad_Hp, pad_Wp, pad_pt, pad_pl;
    int pad_m0, pad_C;  // producer side: only channels pad_m0 .. + pad_C - 1 go over (pad_C 0: all)
    float *pad_in;
    bool pad_in_shared;
};

void conv_plan_free(void *p);

// Node cache of a MaxPool (3x3 / stride 2 / pad 1 over fp32 NCHW, channels a
// multiple of 64) whose output int8 convs may take as an int8 handoff: the
// pooling kernel then also quantizes its output, with the consumers' scale
// and rounding rule, into their zero-padded NHWC buffer.  The q_* fields and
// y_needed mean what ConvPlan's producer-side fields mean; q_out stays null
// when no consumer takes the handoff.
struct PoolPlan {
    int8_t *q_out;
    int q_Hp, q_Wp, q_Cp, q_pt, q_pl, q_split;
    float q_inv_scale;
    int q_readers;
    bool y_needed;
    // When the pooled input comes from an int8 conv with Relu that nothing
    // else reads: that conv's epilogue quantizes it (consumers' scale, round
    // half to even) into this unpadded NHWC buffer [N][H][W][C] (owned), and
    // the pool takes the maximum of the int8 values (quantization is
    // monotone, so that is the quantized maximum).
    int8_t *q_src;
};

void pool_plan_free(void *p);

// Places the plan's workspace in the node's kernel-spec scratch when that
// spec reserves enough; returns the bytes the runtime must allocate for it
// instead (0 when the scratch arena holds it).
size_t claim_spec_scratch(const Spkv2Context *ctx, const Spkv2NodeRecord *node, ConvPlan *plan);
// Device workspace of a plan for this run, or nullptr when it is missing.
uint8_t *plan_workspace(const Spkv2Context *ctx, const ConvPlan *plan);

// Per-process table of measured tile choices, keyed by layer shape; with
// SPKV2_TUNE_DB set it is read from and appended to that file.
bool tuned_lookup(const std::string &key, int *cfg, int *split);
void tuned_store(const std::string &key, int cfg, int split);

// int8 path entry points (conv_i8.hip)
int conv_i8_prepare(Spkv2Context *ctx, const Spkv2NodeRecord *node, ConvPlan *plan);
int conv_i8_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, const ConvPlan *plan, int32_t *raw_acc_out);

}  // namespace spk::kern
