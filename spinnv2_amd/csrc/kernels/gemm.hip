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
#include <cstdlib>
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
    // at most four rows of A (a classifier at batch 1-4), A not transposed,
    // K a multiple of 4: the matrix-vector kernel over these weights, W[n][k]
    // row-major (device); null otherwise
    float *wrow;
};

void gemm_plan_free(void *p) {
    GemmPlan *g = static_cast<GemmPlan *>(p);
    if (!g) return;
    if (g->conv.wpack) (void)hipFree(g->conv.wpack);
    if (g->conv.ktab) (void)hipFree(g->conv.ktab);
    if (g->wrow) (void)hipFree(g->wrow);
    delete g;
}

// Matrix-vector form of a Gemm with R <= 4 rows of A: y[r][n] = alpha *
// sum_k A[r][k] W[n][k] + c[n].  One wave per output n reads row n of W in
// 16-byte pieces (lane l takes k = 4 (l + 64 j) .. + 3, j = 0, 1, ...), all
// of a lane's pieces in flight together with the matching pieces of the R
// rows of A; each lane sums its products in k order, then the 64 lane sums
// are added in a fixed butterfly.  Bound by the HBM reads of W (4 K bytes per
// output), where the 16 x 16 MFMA tiles leave most CUs idle and each tile's
// k chain serial.
template <int R>
__global__ void __launch_bounds__(256) gemv_f32(const float *__restrict__ W, const float *__restrict__ A,
                                                const float *__restrict__ c, float *__restrict__ Y, int K, int Nout,
                                                float alpha) {
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= Nout) return;  // the whole wave (n is per wave)
    const floatx4 *w4 = reinterpret_cast<const floatx4 *>(W + static_cast<size_t>(n) * K);
    const floatx4 *a4 = reinterpret_cast<const floatx4 *>(A);
    const int K4 = K / 4;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    constexpr int U = 8;  // pieces per lane in flight
    for (int j0 = lane; j0 < K4; j0 += 64 * U) {
        floatx4 wv[U], av[U][R];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int j = j0 + 64 * u;
            const bool ok = j < K4;
            wv[u] = ok ? w4[j] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int r = 0; r < R; r++) av[u][r] = ok ? a4[r * K4 + j] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int e = 0; e < 4; e++) acc[r] = fmaf(wv[u][e], av[u][r][e], acc[r]);
    }
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) acc[r] += __shfl_xor(acc[r], off, 64);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; r++) Y[static_cast<size_t>(r) * Nout + n] = alpha * acc[r] + (c ? c[n] : 0.0f);
    }
}

// Batched MatMul y[b] = A[a(b)] x B[b(b)] (reference kernels/reference/mm/
// matmul.c:3-49: numpy broadcasting of the leading dims, K from A's last
// dim, no transposes).  One workgroup computes a 64x64 tile of one batch:
// 4 waves in a 2x2 grid, each a 32x32 block on v_mfma_f32_32x32x2f32.  k
// tiles of 16 are staged through LDS k-contiguous for both operands (B is
// transposed on the way in), double-buffered with the next tile's global
// loads in flight during the MFMAs.
struct MatmulArgs {
    const float *__restrict__ a;
    const float *__restrict__ b;
    float *__restrict__ y;
    int M, N, K;
    int yrank, arank, brank;
    int yshape[8], ashape[8], bshape[8];
};

constexpr int kMmTile = 64, kMmBK = 16, kMmLd = kMmBK + 1;

// Matrix indices into a and b of batch z of y (numpy broadcasting: a
// leading dim of 1 repeats).
__device__ __forceinline__ void matmul_batch(const MatmulArgs &p, int z, size_t *ab, size_t *bb) {
    int coords[8] = {0};
    int t = z;
    for (int d = p.yrank - 3; d >= 0; d--) {
        coords[d] = t % p.yshape[d];
        t /= p.yshape[d];
    }
    *ab = 0;
    *bb = 0;
    for (int d = 0; d + 2 < p.arank; d++) {
        const int yd = p.yrank - p.arank + d;
        *ab = *ab * p.ashape[d] + (p.ashape[d] == 1 || yd < 0 ? 0 : coords[yd]);
    }
    for (int d = 0; d + 2 < p.brank; d++) {
        const int yd = p.yrank - p.brank + d;
        *bb = *bb * p.bshape[d] + (p.bshape[d] == 1 || yd < 0 ? 0 : coords[yd]);
    }
}

__global__ void __launch_bounds__(256) matmul_mfma(MatmulArgs p) {
    __shared__ float As[2][kMmTile * kMmLd];
    __shared__ float Bs[2][kMmTile * kMmLd];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * kMmTile, n0 = blockIdx.x * kMmTile;
    size_t ab = 0, bb = 0;
    matmul_batch(p, blockIdx.z, &ab, &bb);
    const size_t M = p.M, N = p.N, K = p.K;
    const float *A = p.a + ab * M * K;
    const float *B = p.b + bb * K * N;
    float *Y = p.y + static_cast<size_t>(blockIdx.z) * M * N;

    const int ar = tid >> 2, ak = (tid & 3) * 4;   // A tile: row, 4 k's
    const int bk = tid >> 4, bn = (tid & 15) * 4;  // B tile: k, 4 columns
    float ra[4], rb[4];
    auto load = [&](int k0) {
        const int gm = m0 + ar;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int gk = k0 + ak + i;
            ra[i] = gm < p.M && gk < p.K ? A[static_cast<size_t>(gm) * K + gk] : 0.0f;
        }
        const int gk = k0 + bk;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int gn = n0 + bn + i;
            rb[i] = gk < p.K && gn < p.N ? B[static_cast<size_t>(gk) * N + gn] : 0.0f;
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            As[buf][ar * kMmLd + ak + i] = ra[i];
            Bs[buf][(bn + i) * kMmLd + bk] = rb[i];
        }
    };

    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;
    const int ktiles = (p.K + kMmBK - 1) / kMmBK;
    const int row = lane & 31, kh = lane >> 5;
    load(0);
    store(0);
    __syncthreads();
    for (int kt = 0; kt < ktiles; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < ktiles) load((kt + 1) * kMmBK);
#pragma unroll
        for (int s = 0; s < kMmBK / 2; s++) {
            // lanes 0-31 supply k = 2s, lanes 32-63 k = 2s+1, for A and B alike
            const float av = As[buf][(wm * 32 + row) * kMmLd + 2 * s + kh];
            const float bv = Bs[buf][(wn * 32 + row) * kMmLd + 2 * s + kh];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc, 0, 0, 0);
        }
        if (kt + 1 < ktiles) store(buf ^ 1);  // that buffer was last read before the previous barrier
        __syncthreads();
    }
    // accumulator layout: column lane & 31, rows 8*(r/4) + 4*(lane/32) + r%4
    const int col = n0 + wn * 32 + row;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int m = m0 + wm * 32 + 8 * (r >> 2) + 4 * kh + (r & 3);
        if (m < p.M && col < p.N) Y[static_cast<size_t>(m) * N + col] = acc[r];
    }
}

// Batched MatMul for grids too small to fill the GPU with 64x64 tiles (the
// PSA attention products at batch 1): one 32x32 tile per workgroup, its k
// range cut into four contiguous quarters (whole groups of 8 k), one per
// wave.  Each wave accumulates the whole tile over its quarter on
// v_mfma_f32_32x32x2f32 with its operands loaded straight into registers,
// four groups of loads in flight (lanes 0-31 take k = 8g + t and lanes 32-63
// k = 8g + 4 + t for MFMA step t of group g, for A and B alike, so every k
// is summed once); the four partial tiles are then summed through LDS in
// wave order, so the result does not depend on timing.
__global__ void __launch_bounds__(256) matmul_ksplit(MatmulArgs p) {
    __shared__ float red[4][1024];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row = lane & 31, half = lane >> 5;
    const int m0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
    size_t ab = 0, bb = 0;
    matmul_batch(p, blockIdx.z, &ab, &bb);
    const size_t M = p.M, N = p.N, K = p.K;
    const float *A = p.a + ab * M * K;
    const float *B = p.b + bb * K * N;
    float *Y = p.y + static_cast<size_t>(blockIdx.z) * M * N;
    const int groups = (p.K + 7) / 8;
    const int per = (groups + 3) / 4;
    const int g0 = wave * per, g1 = min(g0 + per, groups);
    const int am = m0 + row, bn = n0 + row;
    const bool arow = am < p.M, bcol = bn < p.N;
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;
    for (int gi = g0; gi < g1; gi += 4) {
        float av[4][4], bv[4][4];
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int k = (gi + u) * 8 + 4 * half + t;
                const bool ok = gi + u < g1 && k < p.K;
                av[u][t] = ok && arow ? A[static_cast<size_t>(am) * K + k] : 0.0f;
                bv[u][t] = ok && bcol ? B[static_cast<size_t>(k) * N + bn] : 0.0f;
            }
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int t = 0; t < 4; t++) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u][t], bv[u][t], acc, 0, 0, 0);
    }
    // accumulator layout: column lane & 31, rows 8*(r/4) + 4*(lane/32) + r%4
#pragma unroll
    for (int r = 0; r < 16; r++) red[wave][(8 * (r >> 2) + 4 * half + (r & 3)) * 32 + row] = acc[r];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int e = tid * 4 + i;
        const int m = m0 + (e >> 5), n = n0 + (e & 31);
        const float v = ((red[0][e] + red[1][e]) + red[2][e]) + red[3][e];
        if (m < p.M && n < p.N) Y[static_cast<size_t>(m) * N + n] = v;
    }
}

}  // namespace

int gemm_prepare(Spkv2Context *ctx, const Spkv2NodeRecord *node, size_t *ws) {
    void **slot = &ctx->plans[node->id];
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
    ctx->plan_dtors[node->id] = gemm_plan_free;
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
    // byte offsets inside the kernels are 32-bit signed
    if (g.x_elems * 4 >= (int64_t(1) << 31) || g.y_elems * 4 >= (int64_t(1) << 31)) return SPKV2_E_UNSUPPORTED;
    gp->conv.g = g;
    // (also the fallback of the matrix-vector kernel: an A not 16-byte aligned)
    if (int rc = plan_igemm_gemm(ctx->stream, g, w.data(), attr.trans_a ? gp->rows : 1, &gp->conv)) return rc;
    // a forced tile configuration (SPKV2_CONV_CFG) keeps the tiles
    if (gp->rows >= 1 && gp->rows <= 4 && !attr.trans_a && gp->K % 4 == 0 && !getenv("SPKV2_CONV_CFG")) {
        const size_t wb = w.size() * sizeof(float);
        if (hipMalloc(reinterpret_cast<void **>(&gp->wrow), wb) != hipSuccess) {
            (void)hipGetLastError();
            gp->wrow = nullptr;
        } else if (hipMemcpy(gp->wrow, w.data(), wb, hipMemcpyHostToDevice) != hipSuccess) {
            (void)hipGetLastError();
            (void)hipFree(gp->wrow);
            gp->wrow = nullptr;
        }
    }
    set_kernel_name(ctx, node, gp->wrow ? "gemm:gemv_f32<" + std::to_string(gp->rows) + ">"
                                        : "gemm:" + igemm_name(&gp->conv));
    *ws = claim_spec_scratch(ctx, node, &gp->conv);
    return 0;
}

int run_igemm_f32_strided(Spkv2Context *ctx, const ConvPlan *p, const float *x, const float *bias, float *y,
                          float alpha, int x_img_stride);

int gemm_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    if (ctx->plan_dtors[node->id] != gemm_plan_free) return SPKV2_E_UNSUPPORTED;  // not prepared as a Gemm
    GemmPlan *gp = static_cast<GemmPlan *>(ctx->plans[node->id]);
    if (!gp) return SPKV2_E_UNSUPPORTED;
    const float *a = dptr<const float>(ctx, node->inputs[0]);
    const float *c = node->input_count > 2 ? dptr<const float>(ctx, node->inputs[2]) : nullptr;
    float *y = dptr<float>(ctx, node->outputs[0]);
    if (gp->wrow && (reinterpret_cast<uintptr_t>(a) & 15) == 0) {
        const dim3 grid(static_cast<unsigned>((gp->Nout + 3) / 4));
        switch (gp->rows) {
            case 1: gemv_f32<1><<<grid, 256, 0, ctx->stream>>>(gp->wrow, a, c, y, gp->K, gp->Nout, gp->alpha); break;
            case 2: gemv_f32<2><<<grid, 256, 0, ctx->stream>>>(gp->wrow, a, c, y, gp->K, gp->Nout, gp->alpha); break;
            case 3: gemv_f32<3><<<grid, 256, 0, ctx->stream>>>(gp->wrow, a, c, y, gp->K, gp->Nout, gp->alpha); break;
            default: gemv_f32<4><<<grid, 256, 0, ctx->stream>>>(gp->wrow, a, c, y, gp->K, gp->Nout, gp->alpha); break;
        }
        return launch_status("gemv_f32");
    }
    // A is [rows][K] (one "image" of K channels per row), or [K][rows] with trans_a
    return run_igemm_f32_strided(ctx, &gp->conv, a, c, y, gp->alpha, gp->trans_a ? 1 : gp->K);
}

int matmul_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    const Spkv2TensorRecord *ar = rec(ctx, node->inputs[0]), *br = rec(ctx, node->inputs[1]),
                            *yr = rec(ctx, node->outputs[0]);
    if (ar->rank < 2 || br->rank < 2 || yr->rank < 2 || ar->rank > 8 || br->rank > 8 || yr->rank > 8) return -11;
    if (ar->dtype != SPKV2_DTYPE_FP32 || br->dtype != SPKV2_DTYPE_FP32) return SPKV2_E_UNSUPPORTED;
    const uint64_t M = yr->shape[yr->rank - 2], N = yr->shape[yr->rank - 1], K = ar->shape[ar->rank - 1];
    // operands must hold what the loops read (the reference trusts the records)
    if (ar->shape[ar->rank - 2] != M || br->shape[br->rank - 2] != K || br->shape[br->rank - 1] != N) return -11;
    const uint64_t total = elem_count(yr);
    if (total == 0) return 0;
    const uint64_t batch = total / (M * N);
    for (int d = 0; d + 2 < yr->rank; d++) {
        const int da = d - (yr->rank - ar->rank), db = d - (yr->rank - br->rank);
        if (da >= 0 && ar->shape[da] != 1 && ar->shape[da] != yr->shape[d]) return -11;
        if (db >= 0 && br->shape[db] != 1 && br->shape[db] != yr->shape[d]) return -11;
    }
    if (M > 0x7fffffffULL || N > 0x7fffffffULL || K > 0x7fffffffULL) return SPKV2_E_UNSUPPORTED;
    const uint64_t mt = (M + kMmTile - 1) / kMmTile, nt = (N + kMmTile - 1) / kMmTile;
    if (mt > 65535 || batch > 65535 || nt > 0x7fffffffULL) return SPKV2_E_UNSUPPORTED;
    // 64x64 tiles for fewer than half the CUs: 32x32 tiles with k split over
    // the waves instead (measured on the PSA attention products: 14 tiles at
    // batch 1 27 -> 15 us of node time; 224 tiles at batch 16 the 64x64
    // kernel is faster);
    // SPKV2_MATMUL_KSPLIT=0 / 1 forces either
    const uint64_t mt32 = (M + 31) / 32, nt32 = (N + 31) / 32;
    bool ksplit = mt * nt * batch < 128 && mt32 <= 65535;
    if (const char *e = getenv("SPKV2_MATMUL_KSPLIT")) ksplit = e[0] == '1' ? mt32 <= 65535 : false;
    MatmulArgs p{};
    p.a = dptr<const float>(ctx, node->inputs[0]);
    p.b = dptr<const float>(ctx, node->inputs[1]);
    p.y = dptr<float>(ctx, node->outputs[0]);
    p.M = static_cast<int>(M);
    p.N = static_cast<int>(N);
    p.K = static_cast<int>(K);
    p.yrank = yr->rank;
    p.arank = ar->rank;
    p.brank = br->rank;
    for (int i = 0; i < 8; i++) {
        p.yshape[i] = static_cast<int>(yr->shape[i]);
        p.ashape[i] = static_cast<int>(ar->shape[i]);
        p.bshape[i] = static_cast<int>(br->shape[i]);
    }
    if (ksplit) {
        set_kernel_name(ctx, node, "matmul_ksplit_f32<32x32>");
        hipLaunchKernelGGL(matmul_ksplit, dim3(static_cast<unsigned>(nt32), static_cast<unsigned>(mt32),
                                               static_cast<unsigned>(batch)),
                           dim3(256), 0, ctx->stream, p);
        return launch_status("matmul");
    }
    set_kernel_name(ctx, node, "matmul_mfma_f32<64x64x16>");
    hipLaunchKernelGGL(matmul_mfma, dim3(static_cast<unsigned>(nt), static_cast<unsigned>(mt),
                                         static_cast<unsigned>(batch)),
                       dim3(256), 0, ctx->stream, p);
    return launch_status("matmul");
}

}  // namespace spk::kern
