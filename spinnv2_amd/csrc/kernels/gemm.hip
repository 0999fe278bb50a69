// Gemm and MatMul.
//
// Gemm (reference runtime/kernels/reference/mm/gemm.c:3-33):
//   Y[r][n] = alpha * sum_k A'[r][k] * B'[k][n] + C[n]
// where A' / B' are A / B transposed when trans_a / trans_b are set, and beta
// is not applied (the x86 reference ignores it too).  On the device this is
// the fp32 MFMA implicit GEMM of a 1x1 convolution over an [rows, K, 1, 1]
// input: the GEMM's M is the output feature dimension, its N the rows.  B is
// constant weight data, transposed into [n][k] panels at prepare time;
// trans_a only changes the k-offset table and the per-row stride.
//
// MatMul (reference mm/matmul.c:3-49): batched, numpy-broadcast leading
// dimensions; one thread per output element, k inner, lanes along n.
#include <cstring>
#include <vector>

#include "conv.hpp"
#include "kernels.hpp"

namespace spk::kern {

int plan_igemm_gemm(hipStream_t st, const ConvGeom &g, const float *w_host, int k_stride, ConvPlan *plan);
int run_igemm_f32(Spkv2Context *ctx, const ConvPlan *p, const float *x, const float *bias, const float *res, float *y,
                  float alpha);
std::string igemm_name(const ConvPlan *p);

namespace {

struct GemmPlan {
    ConvPlan conv;
    int rows, K, Nout;
    int trans_a;
    float alpha;
    int x_stride;
};

void gemm_plan_free(void *p) {
    GemmPlan *g = static_cast<GemmPlan *>(p);
    if (!g) return;
    if (g->conv.wpack) (void)hipFree(g->conv.wpack);
    if (g->conv.ktab) (void)hipFree(g->conv.ktab);
    delete g;
}

struct MatmulArgs {
    const float *__restrict__ a;
    const float *__restrict__ b;
    float *__restrict__ y;
    int64_t M, N, K, batch;
    int yrank, arank, brank;
    int64_t yshape[8], ashape[8], bshape[8];
};

__global__ void __launch_bounds__(256) matmul_kernel(MatmulArgs p) {
    const size_t total = static_cast<size_t>(p.batch) * p.M * p.N;
    for (size_t idx = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; idx < total;
         idx += static_cast<size_t>(gridDim.x) * 256) {
        const int64_t n = idx % p.N;
        const int64_t m = (idx / p.N) % p.M;
        int64_t bi = idx / (p.N * p.M);
        // batch coordinates of y, then broadcast into a and b
        int64_t coords[8] = {0};
        for (int d = p.yrank - 3; d >= 0; d--) {
            coords[d] = bi % p.yshape[d];
            bi /= p.yshape[d];
        }
        int64_t ab = 0, bb = 0;
        for (int d = 0; d + 2 < p.arank; d++) {
            const int yd = p.yrank - p.arank + d;
            const int64_t c = yd >= 0 ? coords[yd] : 0;
            ab = ab * p.ashape[d] + (p.ashape[d] == 1 ? 0 : c);
        }
        for (int d = 0; d + 2 < p.brank; d++) {
            const int yd = p.yrank - p.brank + d;
            const int64_t c = yd >= 0 ? coords[yd] : 0;
            bb = bb * p.bshape[d] + (p.bshape[d] == 1 ? 0 : c);
        }
        const float *ar = p.a + (ab * p.M + m) * p.K;
        const float *bc = p.b + bb * p.K * p.N + n;
        float sum = 0.0f;
        for (int64_t k = 0; k < p.K; k++) sum += ar[k] * bc[k * p.N];
        p.y[idx] = sum;
    }
}

}  // namespace

int gemm_prepare(Spkv2Context *ctx, const Spkv2NodeRecord *node, size_t *ws) {
    void **slot = &ctx->node_cache[node->id];
    if (*slot) {
        const ConvPlan &p = static_cast<GemmPlan *>(*slot)->conv;
        *ws = p.ws_in_scratch ? 0 : p.workspace;
        return 0;
    }
    Spkv2AttrRecord attr;
    if (int rc = spkv2_ctx_get_attr(ctx, node, &attr)) return rc;
    if (node->input_count < 2 || node->output_count < 1) return -11;
    const Spkv2TensorRecord *ar = rec(ctx, node->inputs[0]), *br = rec(ctx, node->inputs[1]);
    if (ar->rank != 2 || br->rank != 2) return -11;
    if (ar->dtype != SPKV2_DTYPE_FP32 || br->dtype != SPKV2_DTYPE_FP32) return SPKV2_E_UNSUPPORTED;
    const float *bh = reinterpret_cast<const float *>(host_weight_data(ctx, node->inputs[1]));
    if (!bh) return SPKV2_E_UNSUPPORTED;  // B produced at run time
    GemmPlan *gp = new GemmPlan();
    memset(gp, 0, sizeof(*gp));
    *slot = gp;
    ctx->node_cache_dtors[node->id] = gemm_plan_free;
    gp->rows = attr.trans_a ? ar->shape[1] : ar->shape[0];
    gp->K = attr.trans_a ? ar->shape[0] : ar->shape[1];
    gp->Nout = attr.trans_b ? br->shape[0] : br->shape[1];
    gp->trans_a = attr.trans_a;
    gp->alpha = attr.alpha;
    // weight matrix of the 1x1 conv: W[n][k] = B'[k][n]
    std::vector<float> w(static_cast<size_t>(gp->Nout) * gp->K);
    for (int n = 0; n < gp->Nout; n++)
        for (int k = 0; k < gp->K; k++)
            w[static_cast<size_t>(n) * gp->K + k] =
                attr.trans_b ? bh[static_cast<size_t>(n) * gp->K + k] : bh[static_cast<size_t>(k) * gp->Nout + n];
    ConvGeom g{};
    g.N = gp->rows;
    g.C = gp->K;
    g.H = g.W = 1;
    g.M = gp->Nout;
    g.KH = g.KW = g.OH = g.OW = 1;
    g.sh = g.sw = g.dh = g.dw = 1;
    g.group = 1;
    g.has_bias = node->input_count > 2;
    g.x_elems = static_cast<int64_t>(gp->rows) * gp->K;
    g.y_elems = static_cast<int64_t>(gp->rows) * gp->Nout;
    gp->conv.g = g;
    if (int rc = plan_igemm_gemm(ctx->stream, g, w.data(), attr.trans_a ? gp->rows : 1, &gp->conv)) return rc;
    set_kernel_name(ctx, node, "gemm:" + igemm_name(&gp->conv));
    *ws = claim_spec_scratch(ctx, node, &gp->conv);
    return 0;
}

int run_igemm_f32_strided(Spkv2Context *ctx, const ConvPlan *p, const float *x, const float *bias, float *y,
                          float alpha, int x_img_stride);

int gemm_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    GemmPlan *gp = static_cast<GemmPlan *>(ctx->node_cache[node->id]);
    if (!gp) return SPKV2_E_UNSUPPORTED;
    const float *a = dptr<const float>(ctx, node->inputs[0]);
    const float *c = node->input_count > 2 ? dptr<const float>(ctx, node->inputs[2]) : nullptr;
    float *y = dptr<float>(ctx, node->outputs[0]);
    // A is [rows][K] (one "image" of K channels per row), or [K][rows] with trans_a
    return run_igemm_f32_strided(ctx, &gp->conv, a, c, y, gp->alpha, gp->trans_a ? 1 : gp->K);
}

int matmul_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    const Spkv2TensorRecord *ar = rec(ctx, node->inputs[0]), *br = rec(ctx, node->inputs[1]),
                            *yr = rec(ctx, node->outputs[0]);
    if (ar->rank < 2 || br->rank < 2 || yr->rank < 2) return -11;
    MatmulArgs p{};
    p.a = dptr<const float>(ctx, node->inputs[0]);
    p.b = dptr<const float>(ctx, node->inputs[1]);
    p.y = dptr<float>(ctx, node->outputs[0]);
    p.M = yr->shape[yr->rank - 2];
    p.N = yr->shape[yr->rank - 1];
    p.K = ar->shape[ar->rank - 1];
    p.batch = static_cast<int64_t>(elem_count(yr)) / (p.M * p.N == 0 ? 1 : p.M * p.N);
    p.yrank = yr->rank;
    p.arank = ar->rank;
    p.brank = br->rank;
    for (int i = 0; i < 8; i++) {
        p.yshape[i] = yr->shape[i];
        p.ashape[i] = ar->shape[i];
        p.bshape[i] = br->shape[i];
    }
    const size_t total = static_cast<size_t>(elem_count(yr));
    if (total == 0) return 0;
    set_kernel_name(ctx, node, "matmul_f32");
    hipLaunchKernelGGL(matmul_kernel, dim3(grid_for(total, 256)), dim3(256), 0, ctx->stream, p);
    return launch_status("matmul");
}

}  // namespace spk::kern
