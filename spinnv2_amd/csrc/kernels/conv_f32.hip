// fp32 convolution on MI355X: MFMA implicit GEMM, plus a direct kernel for
// grouped convolutions and as the device fallback kind.
//
// Semantics (reference runtime/kernels/reference/conv/conv.c:3-62):
//   y[n,m,oh,ow] = act( bias[m]
//                       + sum_{c in group(m), kh, kw} x[n,c,oh*s-p+kh*d, ow*s-p+kw*d] * w[m,c',kh,kw]
//                       + residual[n,m,oh,ow] )
// with out-of-bounds taps skipped (i.e. zero), and the residual added before
// the activation.
//
// GEMM view (group == 1): M = Cout, N = batch*OH*OW, K = Cin*KH*KW.
//   A[m][k] = w (OIHW flattened), repacked once at prepare into contiguous
//             BM x BK panels per (m-tile, k-tile), zero padded;
//   B[k][n] = x gathered on the fly (no im2col buffer): each k has an entry
//             {c*H*W + kh*d*W + kw*d, kh*d, kw*d} in a per-layer table, each
//             n a base offset (img, oh*s-p, ow*s-p);
//   C[m][n] = y in NCHW, written from the MFMA accumulators with bias,
//             residual and activation applied in registers.
// Tiles: 256 threads = 4 waves in a WAVES_M x WAVES_N grid; each wave owns
// TM x TN blocks of 32x32 and issues v_mfma_f32_32x32x2f32.  LDS holds the A
// and B tiles k-contiguous (row stride BK+4 floats) double-buffered; one
// ds_read_b128 per operand row feeds four MFMA k-steps: lanes 0-31 supply
// k = 8j+s and lanes 32-63 k = 8j+4+s for step s, the same mapping for A and
// B, so every k is summed exactly once.
#include <algorithm>
#include <cstring>
#include <vector>

#include "conv.hpp"
#include "kernels.hpp"

namespace spk::kern {

// --------------------------------------------------------------- geometry

int read_conv_geom(const Spkv2Context *ctx, const Spkv2NodeRecord *node, ConvGeom *g) {
    Spkv2AttrRecord a;
    if (int rc = spkv2_ctx_get_attr(ctx, node, &a)) return rc;
    if (node->input_count < 2 || node->output_count < 1) return -11;
    const Spkv2TensorRecord *x = rec(ctx, node->inputs[0]);
    const Spkv2TensorRecord *w = rec(ctx, node->inputs[1]);
    const Spkv2TensorRecord *y = rec(ctx, node->outputs[0]);
    if (x->rank != 4 || w->rank != 4 || y->rank != 4) return -11;
    memset(g, 0, sizeof(*g));
    g->N = static_cast<int>(x->shape[0]);
    g->C = static_cast<int>(x->shape[1]);
    g->H = static_cast<int>(x->shape[2]);
    g->W = static_cast<int>(x->shape[3]);
    g->M = static_cast<int>(w->shape[0]);
    g->KH = static_cast<int>(w->shape[2]);
    g->KW = static_cast<int>(w->shape[3]);
    g->OH = static_cast<int>(y->shape[2]);
    g->OW = static_cast<int>(y->shape[3]);
    g->sh = a.strides[0];
    g->sw = a.strides[1];
    g->ph = a.pads[0];
    g->pw = a.pads[1];
    g->dh = a.dilations[0];
    g->dw = a.dilations[1];
    g->group = a.group > 0 ? a.group : 1;
    g->act = a.fused_activation;
    g->has_bias = node->input_count > 2;
    g->has_res = node->input_count > 3;
    g->x_dtype = x->dtype;
    g->w_dtype = w->dtype;
    g->x_elems = static_cast<int64_t>(elem_count(x));
    g->y_elems = static_cast<int64_t>(elem_count(y));
    if (g->C % g->group != 0 || g->M % g->group != 0) return -12;
    if (static_cast<int>(w->shape[1]) * g->group != g->C) return -12;
    if (static_cast<int>(y->shape[0]) != g->N || static_cast<int>(y->shape[1]) != g->M) return -11;
    // index arithmetic inside the kernels is 32-bit
    if (g->x_elems >= (int64_t(1) << 31) || g->y_elems >= (int64_t(1) << 31)) return SPKV2_E_UNSUPPORTED;
    if (g->H >= 16384 || g->W >= 16384) return SPKV2_E_UNSUPPORTED;
    return 0;
}

void conv_plan_free(void *p) {
    ConvPlan *plan = static_cast<ConvPlan *>(p);
    if (!plan) return;
    if (plan->wpack) (void)hipFree(plan->wpack);
    if (plan->ktab) (void)hipFree(plan->ktab);
    if (plan->scales) (void)hipFree(plan->scales);
    delete plan;
}

// ------------------------------------------------------- implicit GEMM kernel

struct IgemmArgs {
    const float *__restrict__ x;
    const float *__restrict__ wp;    // [m_tiles][k_tiles][BM][BK]
    const int2 *__restrict__ ktab;   // [Kpad] {offset, (kh*d << 16) | kw*d}
    const float *__restrict__ bias;  // [M] or null
    const float *__restrict__ res;   // like y, or null
    float *__restrict__ y;
    float *__restrict__ ws;          // split-K partials [splitk][M][Ntot]
    int H, W, M, OW, OHW, Ntot;
    int sh, sw, ph, pw;
    int x_img_stride;
    int m_tiles, k_tiles, kt_per_split;
    int act;
    float alpha;
};

template <int BM, int BN, int BK, int WAVES_M, int WAVES_N>
__global__ void __launch_bounds__(256) conv_igemm_f32(IgemmArgs a) {
    constexpr int TM = BM / (32 * WAVES_M);
    constexpr int TN = BN / (32 * WAVES_N);
    constexpr int LDK = BK + 4;
    constexpr int KPT = BK * BN / 256;  // B elements per thread per k-tile
    constexpr int APT = BM * BK / 1024; // A float4 per thread per k-tile
    static_assert(WAVES_M * WAVES_N == 4, "four waves");
    static_assert(TM >= 1 && TN >= 1 && KPT % 4 == 0 && APT >= 1 && BN >= 64, "tile shape");
    static_assert(BK % 8 == 0, "BK multiple of 8");

    __shared__ __attribute__((aligned(16))) float As[2][BM * LDK];
    __shared__ __attribute__((aligned(16))) float Bs[2][BN * LDK];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WAVES_N;
    const int wn = wave % WAVES_N;

    // Consecutive workgroups land on different XCDs (round robin over 8);
    // remap so each XCD walks a contiguous range of tiles, m fastest, and the
    // tiles sharing one activation panel share that XCD's L2.
    int bid = blockIdx.x;
    const int nb = gridDim.x;
    if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
    const int mt = bid % a.m_tiles;
    const int nt = bid / a.m_tiles;

    const int kt_begin = blockIdx.y * a.kt_per_split;
    const int kt_end = min(kt_begin + a.kt_per_split, a.k_tiles);

    // B gather: thread owns column bcol and KPT consecutive k rows of the tile
    const int bcol = tid % BN;
    const int bgrp = __builtin_amdgcn_readfirstlane(tid / BN);  // wave-uniform: BN >= 64
    int ih0 = -0x40000000, iw0 = 0, col_off = 0;
    {
        const int n = nt * BN + bcol;
        if (n < a.Ntot) {
            const int img = n / a.OHW;
            const int sp = n - img * a.OHW;
            const int oh = sp / a.OW;
            const int ow = sp - oh * a.OW;
            ih0 = oh * a.sh - a.ph;
            iw0 = ow * a.sw - a.pw;
            col_off = img * a.x_img_stride + ih0 * a.W + iw0;
        }
    }

    float4 areg[APT];
    float breg[KPT];

    auto load_tile = [&](int kt) {
        const float4 *src = reinterpret_cast<const float4 *>(a.wp + (static_cast<size_t>(mt) * a.k_tiles + kt) * (BM * BK));
#pragma unroll
        for (int i = 0; i < APT; i++) areg[i] = src[tid + i * 256];
        const int kbase = kt * BK + bgrp * KPT;
#pragma unroll
        for (int j = 0; j < KPT; j++) {
            const int2 e = a.ktab[kbase + j];
            const int ih = ih0 + (e.y >> 16);
            const int iw = iw0 + (e.y & 0xffff);
            const bool ok = static_cast<unsigned>(ih) < static_cast<unsigned>(a.H) &&
                            static_cast<unsigned>(iw) < static_cast<unsigned>(a.W);
            const float v = a.x[ok ? col_off + e.x : 0];
            breg[j] = ok ? v : 0.0f;
        }
    };

    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < APT; i++) {
            const int f = (tid + i * 256) * 4;
            *reinterpret_cast<float4 *>(&As[buf][(f / BK) * LDK + (f % BK)]) = areg[i];
        }
#pragma unroll
        for (int j = 0; j < KPT; j += 4)
            *reinterpret_cast<float4 *>(&Bs[buf][bcol * LDK + bgrp * KPT + j]) =
                make_float4(breg[j], breg[j + 1], breg[j + 2], breg[j + 3]);
    };

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const int row = lane & 31;
    const int khalf = 4 * (lane >> 5);
    if (kt_begin < kt_end) {
        load_tile(kt_begin);
        store_tile(0);
        __syncthreads();
        for (int kt = kt_begin; kt < kt_end; kt++) {
            const int cur = (kt - kt_begin) & 1;
            if (kt + 1 < kt_end) load_tile(kt + 1);
#pragma unroll
            for (int k8 = 0; k8 < BK / 8; k8++) {
                floatx4 af[TM], bf[TN];
#pragma unroll
                for (int i = 0; i < TM; i++)
                    af[i] = *reinterpret_cast<const floatx4 *>(
                        &As[cur][((wm * TM + i) * 32 + row) * LDK + k8 * 8 + khalf]);
#pragma unroll
                for (int j = 0; j < TN; j++)
                    bf[j] = *reinterpret_cast<const floatx4 *>(
                        &Bs[cur][((wn * TN + j) * 32 + row) * LDK + k8 * 8 + khalf]);
#pragma unroll
                for (int s = 0; s < 4; s++)
#pragma unroll
                    for (int i = 0; i < TM; i++)
#pragma unroll
                        for (int j = 0; j < TN; j++)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][s], bf[j][s], acc[i][j], 0, 0, 0);
            }
            if (kt + 1 < kt_end) store_tile(cur ^ 1);
            __syncthreads();
        }
    }

    // Epilogue.  32x32 accumulator layout: lane holds column (lane & 31) and
    // rows 8*(r/4) + 4*(lane/32) + (r%4) for r = 0..15.
    const int rsub = 4 * (lane >> 5);
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = nt * BN + (wn * TN + j) * 32 + row;
        if (n >= a.Ntot) continue;
        const int img = n / a.OHW;
        const int sp = n - img * a.OHW;
        const size_t ybase = static_cast<size_t>(img) * a.M * a.OHW + sp;
#pragma unroll
        for (int i = 0; i < TM; i++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = mt * BM + (wm * TM + i) * 32 + 8 * (r >> 2) + rsub + (r & 3);
                if (m >= a.M) continue;
                float v = acc[i][j][r];
                if (a.ws) {
                    a.ws[(static_cast<size_t>(blockIdx.y) * a.M + m) * a.Ntot + n] = v;
                } else {
                    v = a.alpha * v;
                    if (a.bias) v += a.bias[m];
                    const size_t yi = ybase + static_cast<size_t>(m) * a.OHW;
                    if (a.res) v += a.res[yi];
                    a.y[yi] = apply_act(v, a.act);
                }
            }
        }
    }
}

// Sums split-K partials in slice order, then applies the epilogue.
__global__ void __launch_bounds__(256) splitk_epilogue(const float *__restrict__ ws, int splitk, int M, int Ntot,
                                                       int OHW, const float *__restrict__ bias,
                                                       const float *__restrict__ res, float *__restrict__ y, int act,
                                                       float alpha) {
    const size_t total = static_cast<size_t>(M) * Ntot;
    const size_t plane = total;
    for (size_t idx = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; idx < total;
         idx += static_cast<size_t>(gridDim.x) * 256) {
        const int m = static_cast<int>(idx / Ntot);
        const int n = static_cast<int>(idx - static_cast<size_t>(m) * Ntot);
        float v = 0.0f;
        for (int s = 0; s < splitk; s++) v += ws[s * plane + idx];
        v = alpha * v;
        if (bias) v += bias[m];
        const int img = n / OHW;
        const int sp = n - img * OHW;
        const size_t yi = (static_cast<size_t>(img) * M + m) * OHW + sp;
        if (res) v += res[yi];
        y[yi] = apply_act(v, act);
    }
}

// ------------------------------------------------------------ direct kernel

struct DirectArgs {
    const float *__restrict__ x;
    const float *__restrict__ w;
    const float *__restrict__ bias;
    const float *__restrict__ res;
    float *__restrict__ y;
    int N, C, H, W, M, KH, KW, OH, OW;
    int sh, sw, ph, pw, dh, dw;
    int Cg, Mg, act;
};

// One thread per output element, taps visited in the reference order
// (c, kh, kw), accumulating from the bias.
__global__ void __launch_bounds__(256) conv_direct_f32(DirectArgs a) {
    const size_t total = static_cast<size_t>(a.N) * a.M * a.OH * a.OW;
    for (size_t idx = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; idx < total;
         idx += static_cast<size_t>(gridDim.x) * 256) {
        size_t t = idx;
        const int ow = static_cast<int>(t % a.OW);
        t /= a.OW;
        const int oh = static_cast<int>(t % a.OH);
        t /= a.OH;
        const int m = static_cast<int>(t % a.M);
        const int n = static_cast<int>(t / a.M);
        const int c0 = (m / a.Mg) * a.Cg;
        float sum = a.bias ? a.bias[m] : 0.0f;
        for (int c = 0; c < a.Cg; c++) {
            const float *xc = a.x + (static_cast<size_t>(n) * a.C + c0 + c) * a.H * a.W;
            const float *wc = a.w + (static_cast<size_t>(m) * a.Cg + c) * a.KH * a.KW;
            for (int kh = 0; kh < a.KH; kh++) {
                const int ih = oh * a.sh + kh * a.dh - a.ph;
                if (ih < 0 || ih >= a.H) continue;
                for (int kw = 0; kw < a.KW; kw++) {
                    const int iw = ow * a.sw + kw * a.dw - a.pw;
                    if (iw < 0 || iw >= a.W) continue;
                    sum += xc[ih * a.W + iw] * wc[kh * a.KW + kw];
                }
            }
        }
        if (a.res) sum += a.res[idx];
        a.y[idx] = apply_act(sum, a.act);
    }
}

// ------------------------------------------------------------- host side

namespace {

struct TileCfg {
    int BM, BN, BK;
    const char *name;
};

// Index order must match the dispatch switch in launch_igemm.
const TileCfg kCfgs[] = {
    {128, 128, 16, "128x128x16"},
    {64, 128, 16, "64x128x16"},
    {128, 64, 16, "128x64x16"},
    {64, 64, 16, "64x64x16"},
};
constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

int device_cu_count() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        hipDeviceProp_t p;
        if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&p, dev) == hipSuccess)
            cus = p.multiProcessorCount;
        else
            cus = 256;
    }
    return cus;
}

// Picks the tile shape and split-K factor for an (M, N, K) problem.  The cost
// model counts the MFMA work of the padded tiles, divided over the waves of
// workgroups the GPU can hold at once, with a per-shape efficiency factor
// (smaller tiles re-read more from L2 per flop).
void choose_tiles(int M, int Ntot, int K, int *cfg_out, int *splitk_out) {
    const int cus = device_cu_count();
    const double eff[kNumCfgs] = {1.0, 0.92, 0.92, 0.8};
    const int resident[kNumCfgs] = {2, 2, 2, 4};
    double best = 1e300;
    int best_cfg = 0, best_split = 1;
    for (int c = 0; c < kNumCfgs; c++) {
        const TileCfg &t = kCfgs[c];
        const int mt = (M + t.BM - 1) / t.BM;
        const int nt = (Ntot + t.BN - 1) / t.BN;
        const int kt = (K + t.BK - 1) / t.BK;
        const int tiles = mt * nt;
        for (int split = 1; split <= 16; split *= 2) {
            if (split > 1 && kt / split < 4) break;
            const int kps = (kt + split - 1) / split;
            const long wgs = static_cast<long>(tiles) * split;
            const long slots = static_cast<long>(cus) * resident[c];
            const long rounds = (wgs + slots - 1) / slots;
            // time ~ rounds * work per WG / efficiency; WGs in one round share a CU
            double work = static_cast<double>(t.BM) * t.BN * kps * t.BK;
            double per_round = work * std::min<long>(resident[c], (wgs + cus - 1) / cus);
            double cost = rounds * per_round / eff[c];
            if (split > 1) cost += static_cast<double>(M) * Ntot * split * 8.0 / 64.0;  // partial write + re-read
            if (cost < best * 0.999) {
                best = cost;
                best_cfg = c;
                best_split = split;
            }
        }
    }
    *cfg_out = best_cfg;
    *splitk_out = best_split;
}

template <int BM, int BN, int BK, int WM, int WN>
void launch_cfg(const IgemmArgs &a, int m_tiles, int n_tiles, int splitk, hipStream_t s) {
    dim3 grid(static_cast<unsigned>(m_tiles * n_tiles), static_cast<unsigned>(splitk));
    hipLaunchKernelGGL((conv_igemm_f32<BM, BN, BK, WM, WN>), grid, dim3(256), 0, s, a);
}

void launch_igemm(int cfg, const IgemmArgs &a, int m_tiles, int n_tiles, int splitk, hipStream_t s) {
    switch (cfg) {
    case 0: launch_cfg<128, 128, 16, 2, 2>(a, m_tiles, n_tiles, splitk, s); break;
    case 1: launch_cfg<64, 128, 16, 2, 2>(a, m_tiles, n_tiles, splitk, s); break;
    case 2: launch_cfg<128, 64, 16, 2, 2>(a, m_tiles, n_tiles, splitk, s); break;
    default: launch_cfg<64, 64, 16, 2, 2>(a, m_tiles, n_tiles, splitk, s); break;
    }
}

// Packs A[m][k] (row-major, lda = K) into [m_tiles][k_tiles][BM][BK] panels,
// zero-filling the ragged edges, and uploads it.
int upload_packed_f32(const float *w, int M, int K, int BM, int BK, int m_tiles, int k_tiles, void **out) {
    std::vector<float> packed(static_cast<size_t>(m_tiles) * k_tiles * BM * BK, 0.0f);
    for (int mt = 0; mt < m_tiles; mt++)
        for (int kt = 0; kt < k_tiles; kt++) {
            float *dst = packed.data() + (static_cast<size_t>(mt) * k_tiles + kt) * BM * BK;
            for (int i = 0; i < BM; i++) {
                const int m = mt * BM + i;
                if (m >= M) break;
                for (int kk = 0; kk < BK; kk++) {
                    const int k = kt * BK + kk;
                    if (k >= K) break;
                    dst[i * BK + kk] = w[static_cast<size_t>(m) * K + k];
                }
            }
        }
    const size_t bytes = packed.size() * sizeof(float);
    if (int rc = hip_check(hipMalloc(out, bytes), "hipMalloc packed weights")) return rc;
    return hip_check(hipMemcpy(*out, packed.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy packed weights");
}

}  // namespace

// Gather table for the implicit-GEMM B operand: entry k = (c, kh, kw) holds
// the input offset relative to the output pixel's window origin and the tap
// displacement used for the bounds test.  Entries past K point at a tap that
// is always out of bounds, so padded k contribute zeros.
int upload_ktab(const ConvGeom &g, int Kpad, void **out) {
    const int K = g.C / g.group * g.KH * g.KW;
    std::vector<int2> tab(static_cast<size_t>(Kpad));
    for (int k = 0; k < Kpad; k++) {
        if (k < K) {
            const int c = k / (g.KH * g.KW);
            const int r = k % (g.KH * g.KW);
            const int kh = r / g.KW;
            const int kw = r % g.KW;
            tab[k].x = c * g.H * g.W + kh * g.dh * g.W + kw * g.dw;
            tab[k].y = ((kh * g.dh) << 16) | (kw * g.dw);
        } else {
            tab[k].x = 0;
            tab[k].y = 0x7fff << 16;
        }
    }
    const size_t bytes = tab.size() * sizeof(int2);
    if (int rc = hip_check(hipMalloc(out, bytes), "hipMalloc ktab")) return rc;
    return hip_check(hipMemcpy(*out, tab.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy ktab");
}

// Shared with Gemm: plans an fp32 implicit GEMM for geometry g whose
// weight matrix is w[M][K] on the host.
int plan_igemm_f32(const ConvGeom &g, const float *w_host, ConvPlan *plan) {
    const int K = g.C * g.KH * g.KW;
    const int Ntot = g.N * g.OH * g.OW;
    int cfg = 0, split = 1;
    choose_tiles(g.M, Ntot, K, &cfg, &split);
    const TileCfg &t = kCfgs[cfg];
    plan->path = CONV_IGEMM_F32;
    plan->cfg = cfg;
    plan->BM = t.BM;
    plan->BN = t.BN;
    plan->BK = t.BK;
    plan->K = K;
    plan->m_tiles = (g.M + t.BM - 1) / t.BM;
    plan->n_tiles = (Ntot + t.BN - 1) / t.BN;
    plan->k_tiles = (K + t.BK - 1) / t.BK;
    plan->Kpad = plan->k_tiles * t.BK;
    plan->kt_per_split = (plan->k_tiles + split - 1) / split;
    plan->splitk = (plan->k_tiles + plan->kt_per_split - 1) / plan->kt_per_split;
    plan->workspace = plan->splitk > 1 ? static_cast<size_t>(plan->splitk) * g.M * Ntot * sizeof(float) : 0;
    if (int rc = upload_packed_f32(w_host, g.M, K, t.BM, t.BK, plan->m_tiles, plan->k_tiles, &plan->wpack)) return rc;
    return upload_ktab(g, plan->Kpad, &plan->ktab);
}

std::string igemm_name(const ConvPlan *p) {
    return std::string("conv_igemm_f32<") + kCfgs[p->cfg].name + ",splitk=" + std::to_string(p->splitk) + ">";
}

static int run_igemm_impl(Spkv2Context *ctx, const ConvPlan *p, const float *x, const float *bias, const float *res,
                          float *y, float alpha, int x_img_stride) {
    const ConvGeom &g = p->g;
    IgemmArgs a{};
    a.x = x;
    a.wp = static_cast<const float *>(p->wpack);
    a.ktab = static_cast<const int2 *>(p->ktab);
    a.bias = bias;
    a.res = res;
    a.y = y;
    a.H = g.H;
    a.W = g.W;
    a.M = g.M;
    a.OW = g.OW;
    a.OHW = g.OH * g.OW;
    a.Ntot = g.N * a.OHW;
    a.sh = g.sh;
    a.sw = g.sw;
    a.ph = g.ph;
    a.pw = g.pw;
    a.x_img_stride = x_img_stride;
    a.m_tiles = p->m_tiles;
    a.k_tiles = p->k_tiles;
    a.kt_per_split = p->kt_per_split;
    a.act = g.act;
    a.alpha = alpha;
    a.ws = nullptr;
    if (p->splitk > 1) {
        if (ctx->workspace_size < p->workspace) return SPKV2_E_UNSUPPORTED;
        a.ws = reinterpret_cast<float *>(ctx->workspace);
    }
    launch_igemm(p->cfg, a, p->m_tiles, p->n_tiles, p->splitk, ctx->stream);
    if (int rc = launch_status("conv_igemm_f32")) return rc;
    if (p->splitk > 1) {
        const size_t total = static_cast<size_t>(g.M) * a.Ntot;
        hipLaunchKernelGGL(splitk_epilogue, dim3(grid_for(total, 256)), dim3(256), 0, ctx->stream, a.ws, p->splitk,
                           g.M, a.Ntot, a.OHW, bias, res, y, g.act, alpha);
        if (int rc = launch_status("splitk_epilogue")) return rc;
    }
    return 0;
}

int run_igemm_f32(Spkv2Context *ctx, const ConvPlan *p, const float *x, const float *bias, const float *res, float *y,
                  float alpha) {
    return run_igemm_impl(ctx, p, x, bias, res, y, alpha, p->g.C * p->g.H * p->g.W);
}

// Gemm entry: no residual, caller-chosen row stride of the B operand source.
int run_igemm_f32_strided(Spkv2Context *ctx, const ConvPlan *p, const float *x, const float *bias, float *y,
                          float alpha, int x_img_stride) {
    return run_igemm_impl(ctx, p, x, bias, nullptr, y, alpha, x_img_stride);
}

static int run_direct(Spkv2Context *ctx, const Spkv2NodeRecord *node, const ConvGeom &g) {
    DirectArgs a{};
    a.x = dptr<const float>(ctx, node->inputs[0]);
    a.w = dptr<const float>(ctx, node->inputs[1]);
    a.bias = g.has_bias ? dptr<const float>(ctx, node->inputs[2]) : nullptr;
    a.res = g.has_res ? dptr<const float>(ctx, node->inputs[3]) : nullptr;
    a.y = dptr<float>(ctx, node->outputs[0]);
    a.N = g.N;
    a.C = g.C;
    a.H = g.H;
    a.W = g.W;
    a.M = g.M;
    a.KH = g.KH;
    a.KW = g.KW;
    a.OH = g.OH;
    a.OW = g.OW;
    a.sh = g.sh;
    a.sw = g.sw;
    a.ph = g.ph;
    a.pw = g.pw;
    a.dh = g.dh;
    a.dw = g.dw;
    a.Cg = g.C / g.group;
    a.Mg = g.M / g.group;
    a.act = g.act;
    hipLaunchKernelGGL(conv_direct_f32, dim3(grid_for(static_cast<size_t>(g.y_elems), 256)), dim3(256), 0,
                       ctx->stream, a);
    return launch_status("conv_direct_f32");
}

int conv_prepare(Spkv2Context *ctx, const Spkv2NodeRecord *node, size_t *ws) {
    ConvGeom g;
    if (int rc = read_conv_geom(ctx, node, &g)) return rc;
    void **slot = &ctx->node_cache[node->id];
    if (*slot) {
        *ws = static_cast<ConvPlan *>(*slot)->workspace;
        return 0;
    }
    ConvPlan *plan = new ConvPlan();
    memset(plan, 0, sizeof(*plan));
    plan->g = g;
    *slot = plan;
    ctx->node_cache_dtors[node->id] = conv_plan_free;
    int rc = 0;
    if (g.w_dtype == SPKV2_DTYPE_INT8) {
        rc = conv_i8_prepare(ctx, node, plan);
    } else if (g.w_dtype != SPKV2_DTYPE_FP32 || g.x_dtype != SPKV2_DTYPE_FP32) {
        rc = SPKV2_E_UNSUPPORTED;
    } else if (g.group == 1) {
        const float *w = reinterpret_cast<const float *>(host_weight_data(ctx, node->inputs[1]));
        if (!w) {
            rc = SPKV2_E_UNSUPPORTED;  // weights produced at run time
        } else {
            rc = plan_igemm_f32(g, w, plan);
            if (rc == 0) set_kernel_name(ctx, node, igemm_name(plan));
        }
    } else {
        plan->path = CONV_DIRECT_F32;
        set_kernel_name(ctx, node, "conv_direct_f32<grouped>");
    }
    if (rc == 0) *ws = plan->workspace;
    return rc;
}

int conv_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *scratch) {
    (void)scratch;
    ConvPlan *plan = static_cast<ConvPlan *>(ctx->node_cache[node->id]);
    if (!plan) return SPKV2_E_UNSUPPORTED;  // prepare did not run for this node
    switch (plan->path) {
    case CONV_IGEMM_F32:
        return run_igemm_f32(ctx, plan, dptr<const float>(ctx, node->inputs[0]),
                             plan->g.has_bias ? dptr<const float>(ctx, node->inputs[2]) : nullptr,
                             plan->g.has_res ? dptr<const float>(ctx, node->inputs[3]) : nullptr,
                             dptr<float>(ctx, node->outputs[0]), 1.0f);
    case CONV_DIRECT_F32: return run_direct(ctx, node, plan->g);
    case CONV_IGEMM_I8: return conv_i8_run(ctx, node, plan, nullptr);
    }
    return SPKV2_E_UNSUPPORTED;
}

int conv_direct_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *scratch) {
    ConvGeom g;
    if (int rc = read_conv_geom(ctx, node, &g)) return rc;
    if (g.w_dtype == SPKV2_DTYPE_INT8) return conv_run(ctx, node, scratch);
    if (g.w_dtype != SPKV2_DTYPE_FP32 || g.x_dtype != SPKV2_DTYPE_FP32) return SPKV2_E_UNSUPPORTED;
    set_kernel_name(ctx, node, "conv_direct_f32");
    return run_direct(ctx, node, g);
}

int conv_int8_accumulators(Spkv2Context *ctx, const Spkv2NodeRecord *node, int32_t *dev_out) {
    ConvPlan *plan = static_cast<ConvPlan *>(ctx->node_cache[node->id]);
    if (!plan || plan->path != CONV_IGEMM_I8) return SPKV2_E_UNSUPPORTED;
    return conv_i8_run(ctx, node, plan, dev_out);
}

}  // namespace spk::kern
