// INT8 convolution on MI355X with the reference runtime's semantics
// (runtime/kernels/optimized/conv/conv_int8.c:22-210):
//   per image, xq = sat8(round(x * (1/s_x))), rounding half to even for the
//   first floor(C*H*W/16)*16 elements and half away from zero for the tail;
//   padded taps are int8 zero;
//   acc[m][n] = sum_k wq[m][k] * xq[k][n]   (int32, exact);
//   y = act( fma((float)acc, s_w[m]*s_x, bias[m]) + residual ).
// Inputs and outputs stay fp32 NCHW; weights are int8 OIHW with per-output-
// channel scales, the activation scale is per tensor (quantization section).
//
// Device plan:
//   1. quantize_nhwc: one HBM pass reads x (NCHW fp32) and writes xq as
//      NHWC int8 into the runtime workspace, so the 16 channels of one tap
//      are one 16-byte load;
//   2. conv_igemm_i8: implicit GEMM with K ordered (kh, kw, c), weights
//      repacked at prepare to match, v_mfma_i32_32x32x32_i8 on LDS tiles
//      stored k-contiguous, dequantize/bias/residual/activation in registers.
//      Split-K writes int32 partials that a second kernel sums (exactly) and
//      dequantizes.
// Integer sums are order independent, so the accumulators equal the closed
// form bit for bit whatever the tiling.
#include <cmath>
#include <cstring>
#include <vector>

#include "conv.hpp"
#include "kernels.hpp"

namespace spk::kern {

namespace {

constexpr int I8_BM = 128, I8_BN = 128, I8_BK = 64;
constexpr int I8_LDK = I8_BK + 16;  // bytes per LDS row (80: conflict-free b128 reads)

// xq[img][h][w][c] = q(x[img][c][h][w]); 64 pixels x 32 channels per block,
// transposed through LDS so both sides are coalesced.
__global__ void __launch_bounds__(256) quantize_nhwc(const float *__restrict__ x, int8_t *__restrict__ xq, int C,
                                                     int HW, float inv_scale, int split) {
    __shared__ int8_t tile[32][64 + 4];
    const int img = blockIdx.z;
    const int p0 = blockIdx.x * 64;
    const int c0 = blockIdx.y * 32;
    const float *xi = x + static_cast<size_t>(img) * C * HW;
    const int tp = threadIdx.x & 63;
    const int tc = threadIdx.x >> 6;  // 0..3
    for (int cc = tc; cc < 32; cc += 4) {
        const int c = c0 + cc;
        const int p = p0 + tp;
        int8_t q = 0;
        if (c < C && p < HW) {
            const int idx = c * HW + p;
            const float v = xi[idx] * inv_scale;
            float r;
            if (v != v) r = 0.0f;
            else r = idx < split ? rintf(v) : roundf(v);
            r = fminf(fmaxf(r, -128.0f), 127.0f);
            q = static_cast<int8_t>(static_cast<int>(r));
        }
        tile[cc][tp] = q;
    }
    __syncthreads();
    // write: each thread one pixel row segment of 8 channels
    const int wp = threadIdx.x >> 2;   // pixel 0..63
    const int wc = (threadIdx.x & 3) * 8;  // channel chunk
    const int p = p0 + wp;
    if (p < HW) {
        int8_t *dst = xq + (static_cast<size_t>(img) * HW + p) * C + c0 + wc;
        for (int k = 0; k < 8; k++)
            if (c0 + wc + k < C) dst[k] = tile[wc + k][wp];
    }
}

struct I8Args {
    const int8_t *__restrict__ xq;      // NHWC int8
    const int8_t *__restrict__ wp;      // [m_tiles][k_tiles][BM][BK]
    const int2 *__restrict__ ktab;      // per 16-k group (vec) or per k (bytes)
    const float *__restrict__ scales;   // [M] s_w[m]*s_x
    const float *__restrict__ bias;
    const float *__restrict__ res;
    float *__restrict__ y;
    int32_t *__restrict__ ws;           // split-K partials or raw accumulator output
    int H, W, C, M, OW, OHW, Ntot;
    int sh, sw, ph, pw;
    int m_tiles, k_tiles, kt_per_split;
    int act;
    int mode;  // 0: dequant epilogue, 1: int32 partials to ws[split][M][Ntot], 2: raw acc to ws as NCHW
};

template <bool VEC>
__global__ void __launch_bounds__(256) conv_igemm_i8(I8Args a) {
    constexpr int BM = I8_BM, BN = I8_BN, BK = I8_BK, LDK = I8_LDK;
    constexpr int TM = 2, TN = 2;  // 2x2 waves, 64x64 each
    __shared__ __attribute__((aligned(16))) int8_t As[2][BM * LDK];
    __shared__ __attribute__((aligned(16))) int8_t Bs[2][BN * LDK];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    int bid = blockIdx.x;
    const int nb = gridDim.x;
    if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
    const int mt = bid % a.m_tiles;
    const int nt = bid / a.m_tiles;
    const int kt_begin = blockIdx.y * a.kt_per_split;
    const int kt_end = min(kt_begin + a.kt_per_split, a.k_tiles);

    // B: column bcol, 32 consecutive k of the tile (two 16-byte groups)
    const int bcol = tid & (BN - 1);
    const int bhalf = __builtin_amdgcn_readfirstlane(tid >> 7);  // waves 0,1 -> 0; 2,3 -> 1
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
            col_off = ((img * a.H + ih0) * a.W + iw0) * a.C;
        }
    }

    // native vector types: arrays of HIP's int4 class stay in scratch memory
    intx4 areg[2];
    intx4 breg[2];

    auto load_tile = [&](int kt) {
        const intx4 *src = reinterpret_cast<const intx4 *>(a.wp + (static_cast<size_t>(mt) * a.k_tiles + kt) * (BM * BK));
        areg[0] = src[tid];
        areg[1] = src[tid + 256];
        const int kbase = kt * BK + bhalf * 32;
        if constexpr (VEC) {
#pragma unroll
            for (int g = 0; g < 2; g++) {
                const int2 e = a.ktab[(kbase >> 4) + g];
                const int ih = ih0 + (e.y >> 16);
                const int iw = iw0 + (e.y & 0xffff);
                const bool ok = static_cast<unsigned>(ih) < static_cast<unsigned>(a.H) &&
                                static_cast<unsigned>(iw) < static_cast<unsigned>(a.W);
                const intx4 v = *reinterpret_cast<const intx4 *>(a.xq + (ok ? col_off + e.x : 0));
                breg[g] = ok ? v : intx4{0, 0, 0, 0};
            }
        } else {
            uint32_t words[8];
#pragma unroll
            for (int w = 0; w < 8; w++) {
                uint32_t packed = 0;
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const int2 e = a.ktab[kbase + w * 4 + b];
                    const int ih = ih0 + (e.y >> 16);
                    const int iw = iw0 + (e.y & 0xffff);
                    const bool ok = static_cast<unsigned>(ih) < static_cast<unsigned>(a.H) &&
                                    static_cast<unsigned>(iw) < static_cast<unsigned>(a.W);
                    const int8_t v = a.xq[ok ? col_off + e.x : 0];
                    packed |= static_cast<uint32_t>(static_cast<uint8_t>(ok ? v : 0)) << (8 * b);
                }
                words[w] = packed;
            }
            breg[0] = intx4{static_cast<int>(words[0]), static_cast<int>(words[1]), static_cast<int>(words[2]),
                            static_cast<int>(words[3])};
            breg[1] = intx4{static_cast<int>(words[4]), static_cast<int>(words[5]), static_cast<int>(words[6]),
                            static_cast<int>(words[7])};
        }
    };

    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int f = (tid + i * 256) * 16;  // byte index within the BM x BK tile
            *reinterpret_cast<intx4 *>(&As[buf][(f / BK) * LDK + (f % BK)]) = areg[i];
        }
        *reinterpret_cast<intx4 *>(&Bs[buf][bcol * LDK + bhalf * 32]) = breg[0];
        *reinterpret_cast<intx4 *>(&Bs[buf][bcol * LDK + bhalf * 32 + 16]) = breg[1];
    };

    intx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

    const int row = lane & 31;
    const int khalf = 16 * (lane >> 5);
    if (kt_begin < kt_end) {
        load_tile(kt_begin);
        store_tile(0);
        __syncthreads();
        for (int kt = kt_begin; kt < kt_end; kt++) {
            const int cur = (kt - kt_begin) & 1;
            if (kt + 1 < kt_end) load_tile(kt + 1);
#pragma unroll
            for (int k32 = 0; k32 < BK / 32; k32++) {
                intx4 af[TM], bf[TN];
#pragma unroll
                for (int i = 0; i < TM; i++)
                    af[i] = *reinterpret_cast<const intx4 *>(&As[cur][((wm * TM + i) * 32 + row) * LDK + k32 * 32 + khalf]);
#pragma unroll
                for (int j = 0; j < TN; j++)
                    bf[j] = *reinterpret_cast<const intx4 *>(&Bs[cur][((wn * TN + j) * 32 + row) * LDK + k32 * 32 + khalf]);
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
            if (kt + 1 < kt_end) store_tile(cur ^ 1);
            __syncthreads();
        }
    }

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
                const int32_t v = acc[i][j][r];
                const size_t yi = ybase + static_cast<size_t>(m) * a.OHW;
                if (a.mode == 1) {
                    a.ws[(static_cast<size_t>(blockIdx.y) * a.M + m) * a.Ntot + n] = v;
                } else if (a.mode == 2) {
                    a.ws[yi] = v;
                } else {
                    float f = fmaf(static_cast<float>(v), a.scales[m], a.bias ? a.bias[m] : 0.0f);
                    if (a.res) f += a.res[yi];
                    a.y[yi] = apply_act(f, a.act);
                }
            }
        }
    }
}

__global__ void __launch_bounds__(256) splitk_i8_epilogue(const int32_t *__restrict__ ws, int splitk, int M, int Ntot,
                                                          int OHW, const float *__restrict__ scales,
                                                          const float *__restrict__ bias, const float *__restrict__ res,
                                                          float *__restrict__ y, int32_t *__restrict__ raw, int act) {
    const size_t total = static_cast<size_t>(M) * Ntot;
    for (size_t idx = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; idx < total;
         idx += static_cast<size_t>(gridDim.x) * 256) {
        const int m = static_cast<int>(idx / Ntot);
        const int n = static_cast<int>(idx - static_cast<size_t>(m) * Ntot);
        int32_t v = 0;
        for (int s = 0; s < splitk; s++) v += ws[s * total + idx];
        const int img = n / OHW;
        const int sp = n - img * OHW;
        const size_t yi = (static_cast<size_t>(img) * M + m) * OHW + sp;
        if (raw) {
            raw[yi] = v;
            continue;
        }
        float f = fmaf(static_cast<float>(v), scales[m], bias ? bias[m] : 0.0f);
        if (res) f += res[yi];
        y[yi] = apply_act(f, act);
    }
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace

int conv_i8_prepare(Spkv2Context *ctx, const Spkv2NodeRecord *node, ConvPlan *plan) {
    const ConvGeom &g = plan->g;
    if (g.group != 1 || g.x_dtype != SPKV2_DTYPE_FP32) return SPKV2_E_UNSUPPORTED;
    const Spkv2QuantParamRecord *wq = spkv2_ctx_find_quant_param(ctx, node->inputs[1]);
    const Spkv2QuantParamRecord *xq = spkv2_ctx_find_quant_param(ctx, node->inputs[0]);
    if (!wq || !xq) return SPKV2_E_QUANT;
    const float *ws = spkv2_ctx_quant_scales(ctx, wq);
    const float *xs = spkv2_ctx_quant_scales(ctx, xq);
    if (!ws || !xs || static_cast<int>(wq->num_channels) < g.M || xq->num_channels < 1) return SPKV2_E_QUANT;
    const int8_t *w = reinterpret_cast<const int8_t *>(host_weight_data(ctx, node->inputs[1]));
    if (!w) return SPKV2_E_UNSUPPORTED;

    plan->path = CONV_IGEMM_I8;
    plan->x_scale = xs[0];
    const int K = g.C * g.KH * g.KW;
    const int Ntot = g.N * g.OH * g.OW;
    plan->K = K;
    plan->BM = I8_BM;
    plan->BN = I8_BN;
    plan->BK = I8_BK;
    plan->m_tiles = (g.M + I8_BM - 1) / I8_BM;
    plan->n_tiles = (Ntot + I8_BN - 1) / I8_BN;
    plan->k_tiles = (K + I8_BK - 1) / I8_BK;
    plan->Kpad = plan->k_tiles * I8_BK;
    plan->cfg = (g.C % 16 == 0) ? 1 : 0;  // 1: 16-byte channel groups, 0: byte gather

    // split-K only when the tile grid cannot fill the GPU
    int split = 1;
    {
        int dev = 0, cus = 256;
        hipDeviceProp_t p;
        if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&p, dev) == hipSuccess) cus = p.multiProcessorCount;
        const int tiles = plan->m_tiles * plan->n_tiles;
        while (split < 16 && tiles * split * 2 <= cus * 2 && plan->k_tiles / (split * 2) >= 2) split *= 2;
    }
    plan->kt_per_split = (plan->k_tiles + split - 1) / split;
    plan->splitk = (plan->k_tiles + plan->kt_per_split - 1) / plan->kt_per_split;
    const size_t xq_bytes = align_up(static_cast<size_t>(g.x_elems) + 64, 256);
    // partials also serve the raw-accumulator hook, which always takes the split path
    const size_t part_bytes = static_cast<size_t>(plan->splitk) * g.M * Ntot * sizeof(int32_t);
    plan->workspace = xq_bytes + part_bytes;

    // activation quantization constants (reference conv_int8.c:22-23)
    plan->quant_split = static_cast<int>((static_cast<int64_t>(g.C) * g.H * g.W / 16) * 16);

    // weights: K reordered to (kh, kw, c), packed [m_tiles][k_tiles][BM][BK]
    std::vector<int8_t> packed(static_cast<size_t>(plan->m_tiles) * plan->k_tiles * I8_BM * I8_BK, 0);
    for (int m = 0; m < g.M; m++) {
        const int mt = m / I8_BM, mi = m % I8_BM;
        for (int c = 0; c < g.C; c++)
            for (int kh = 0; kh < g.KH; kh++)
                for (int kw = 0; kw < g.KW; kw++) {
                    const int k = (kh * g.KW + kw) * g.C + c;
                    const int kt = k / I8_BK, kk = k % I8_BK;
                    packed[((static_cast<size_t>(mt) * plan->k_tiles + kt) * I8_BM + mi) * I8_BK + kk] =
                        w[((static_cast<size_t>(m) * g.C + c) * g.KH + kh) * g.KW + kw];
                }
    }
    if (int rc = hip_check(hipMalloc(&plan->wpack, packed.size()), "hipMalloc i8 weights")) return rc;
    if (int rc = hip_check(hipMemcpy(plan->wpack, packed.data(), packed.size(), hipMemcpyHostToDevice), "hipMemcpy"))
        return rc;

    // gather table over NHWC: offset of (kh, kw, c) relative to the window origin
    const bool vec = plan->cfg == 1;
    const int entries = vec ? plan->Kpad / 16 : plan->Kpad;
    std::vector<int2> tab(static_cast<size_t>(entries));
    for (int e = 0; e < entries; e++) {
        const int k = vec ? e * 16 : e;
        if (k < K) {
            const int tap = k / g.C, c = k % g.C;
            const int kh = tap / g.KW, kw = tap % g.KW;
            tab[e].x = (kh * g.dh * g.W + kw * g.dw) * g.C + c;
            tab[e].y = ((kh * g.dh) << 16) | (kw * g.dw);
        } else {
            tab[e].x = 0;
            tab[e].y = 0x7fff << 16;
        }
    }
    if (int rc = hip_check(hipMalloc(&plan->ktab, tab.size() * sizeof(int2)), "hipMalloc ktab")) return rc;
    if (int rc = hip_check(hipMemcpy(plan->ktab, tab.data(), tab.size() * sizeof(int2), hipMemcpyHostToDevice), "hipMemcpy"))
        return rc;

    std::vector<float> comb(static_cast<size_t>(g.M));
    for (int m = 0; m < g.M; m++) comb[m] = ws[m] * plan->x_scale;  // reference conv_int8.c:93
    if (int rc = hip_check(hipMalloc(reinterpret_cast<void **>(&plan->scales), comb.size() * 4), "hipMalloc")) return rc;
    if (int rc = hip_check(hipMemcpy(plan->scales, comb.data(), comb.size() * 4, hipMemcpyHostToDevice), "hipMemcpy"))
        return rc;
    set_kernel_name(ctx, node, std::string("conv_igemm_i8<128x128x64,") + (vec ? "vec16" : "bytes") +
                                   ",splitk=" + std::to_string(plan->splitk) + ">");
    return 0;
}

int conv_i8_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, const ConvPlan *plan, int32_t *raw_acc_out) {
    const ConvGeom &g = plan->g;
    if (ctx->workspace_size < plan->workspace) return SPKV2_E_UNSUPPORTED;
    const int HW = g.H * g.W;
    int8_t *xq = reinterpret_cast<int8_t *>(ctx->workspace);
    const size_t xq_bytes = align_up(static_cast<size_t>(g.x_elems) + 64, 256);
    int32_t *part = reinterpret_cast<int32_t *>(ctx->workspace + xq_bytes);
    const float inv_scale = 1.0f / plan->x_scale;  // reference conv_int8.c:23

    dim3 qgrid((HW + 63) / 64, (g.C + 31) / 32, g.N);
    hipLaunchKernelGGL(quantize_nhwc, qgrid, dim3(256), 0, ctx->stream, dptr<const float>(ctx, node->inputs[0]), xq,
                       g.C, HW, inv_scale, plan->quant_split);
    if (int rc = launch_status("quantize_nhwc")) return rc;

    I8Args a{};
    a.xq = xq;
    a.wp = static_cast<const int8_t *>(plan->wpack);
    a.ktab = static_cast<const int2 *>(plan->ktab);
    a.scales = plan->scales;
    a.bias = g.has_bias ? dptr<const float>(ctx, node->inputs[2]) : nullptr;
    a.res = g.has_res ? dptr<const float>(ctx, node->inputs[3]) : nullptr;
    a.y = dptr<float>(ctx, node->outputs[0]);
    a.H = g.H;
    a.W = g.W;
    a.C = g.C;
    a.M = g.M;
    a.OW = g.OW;
    a.OHW = g.OH * g.OW;
    a.Ntot = g.N * a.OHW;
    a.sh = g.sh;
    a.sw = g.sw;
    a.ph = g.ph;
    a.pw = g.pw;
    a.m_tiles = plan->m_tiles;
    a.k_tiles = plan->k_tiles;
    a.kt_per_split = plan->kt_per_split;
    a.act = g.act;
    const bool split = plan->splitk > 1;
    if (raw_acc_out && !split) {
        a.mode = 2;
        a.ws = raw_acc_out;
    } else if (split) {
        a.mode = 1;
        a.ws = part;
    } else {
        a.mode = 0;
    }
    dim3 grid(static_cast<unsigned>(plan->m_tiles * plan->n_tiles), static_cast<unsigned>(plan->splitk));
    if (plan->cfg == 1) hipLaunchKernelGGL(conv_igemm_i8<true>, grid, dim3(256), 0, ctx->stream, a);
    else hipLaunchKernelGGL(conv_igemm_i8<false>, grid, dim3(256), 0, ctx->stream, a);
    if (int rc = launch_status("conv_igemm_i8")) return rc;
    if (split) {
        const size_t total = static_cast<size_t>(g.M) * a.Ntot;
        hipLaunchKernelGGL(splitk_i8_epilogue, dim3(grid_for(total, 256)), dim3(256), 0, ctx->stream, part,
                           plan->splitk, g.M, a.Ntot, a.OHW, plan->scales, a.bias, a.res, a.y, raw_acc_out, g.act);
        if (int rc = launch_status("splitk_i8_epilogue")) return rc;
    }
    return 0;
}

}  // namespace spk::kern
