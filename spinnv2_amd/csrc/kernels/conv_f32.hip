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
//   B[k][n] = x gathered on the fly (no im2col buffer) from the input, or
//             from a zero-padded copy of it when the conv pads, so that every
//             tap is in bounds: element (k, n) is at col(n) + koff(k), a
//             per-lane base plus a per-layer table entry;
//   C[m][n] = y in NCHW, written from the MFMA accumulators with bias,
//             residual and activation applied in registers.
// Tiles: 256 threads = 4 waves in a WAVES_M x WAVES_N grid; each wave owns
// TM x TN blocks of 32x32 and issues v_mfma_f32_32x32x2f32.  LDS holds the A
// and B tiles k-contiguous (row stride BK+4 floats) double-buffered; one
// ds_read_b128 per operand row feeds four MFMA k-steps: lanes 0-31 supply
// k = 8j+s and lanes 32-63 k = 8j+4+s for step s, the same mapping for A and
// B, so every k is summed exactly once.
#include <dlfcn.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <map>
#include <mutex>
#include <string>
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
    // byte offsets and buffer extents inside the kernels are 32-bit signed:
    // every fp32 tensor of the node must stay below 2 GiB
    if (g->x_elems * 4 >= (int64_t(1) << 31) || g->y_elems * 4 >= (int64_t(1) << 31)) return SPKV2_E_UNSUPPORTED;
    if (g->H >= 16384 || g->W >= 16384) return SPKV2_E_UNSUPPORTED;
    return 0;
}

void conv_plan_free(void *p) {
    ConvPlan *plan = static_cast<ConvPlan *>(p);
    if (!plan) return;
    if (plan->wpack) (void)hipFree(plan->wpack);
    if (plan->ktab) (void)hipFree(plan->ktab);
    if (plan->scales) (void)hipFree(plan->scales);
    if (plan->qrow) (void)hipFree(plan->qrow);
    if (plan->q_in) (void)hipFree(plan->q_in);
    if (plan->pad_in && !plan->pad_in_shared) (void)hipFree(plan->pad_in);
    if (plan->gather.ktap) (void)hipFree(const_cast<int *>(plan->gather.ktap));
    delete plan;
}

// ------------------------------------------------------- implicit GEMM kernel

// gfx9 buffer resource word 3 (raw, untyped loads); loads whose offset is at
// or beyond num_records return 0.
constexpr int kBufferWord3 = 0x00020000;
// byte offset that is out of range for every tensor (they are < 2 GiB), and
// still does not wrap when a valid offset is added to it
constexpr int kOobOffset = 0x7fff0000;

struct IgemmArgs {
    const float *__restrict__ x;     // B-operand source: NCHW input, zero-padded when the conv pads
    const float *__restrict__ wp;    // [m_tiles][k_tiles] BM x BK tiles in MFMA fragment order
    const int *__restrict__ koff;    // [Kpad + 2*BK] byte offset of k = (c, kh, kw) in x, kOobOffset past K
    const float *__restrict__ bias;  // [M] or null
    const float *__restrict__ res;   // like y, or null
    float *__restrict__ y;
    float *__restrict__ ws;          // split-K partials [splitk][M][ws_ld], column n at n - ws_n0
    int ws_n0, ws_ld;                // first column with partials, columns per partial row
    int dp_tiles, rem_split;         // hybrid: whole tiles first; rem_split slices per split tile
    int x_bytes;                     // extent of x for the bounds-checked loads
    int y_bytes;                     // extent of y (and of the residual)
    int ws_bytes;                    // extent of the split-K partials
    int Wp;                          // row pitch of x (padded width)
    int M, OW, OHW, Ntot;
    int sh, sw;
    int x_img_stride;                // elements between images in x
    int y_img_stride;                // elements between images in y and the residual
    int y_cstride;                   // elements between channels in y (OHW unless y is a view)
    int m_tiles, k_tiles, kt_per_split;
    int act;
    float alpha;
    // handoff: also store the output into the consuming conv's zero-padded
    // input (NCHW, Hp x Wp planes); y may then be null (no other reader)
    float *__restrict__ yp;
    int yp_bytes, yp_Wp, yp_pt, yp_pl, yp_plane;
    int yp_m0, yp_C;  // the handed-off channels: m0 .. m0 + C - 1 of y, the target's channels 0 .. C - 1
    // skinny kernel: k = tap * sk_C + c (a tap's channels consecutive);
    // channel c of a tap is c * sk_cstride elements past channel 0, tap
    // (kh, kw) = (tap / sk_KW, tap % sk_KW) kh * sk_tap_h + kw * sk_tap_w
    // elements past tap 0
    int sk_C, sk_cstride, sk_KW, sk_tap_h, sk_tap_w;
    // implicit padding (kModeChk): per-k tap table ((kh*dh) << 16 | kw*dw,
    // 0x7fff7fff past K), the unpadded input's extent and the padding
    const int *__restrict__ ktap;
    int chk_H, chk_W, chk_ph, chk_pw;
    int th_steps;  // thin kernel: K / 4 MFMA steps (k' = tap * sk_C + c)
    // row-window kernel: the input window's geometry (GatherGeom's win_*)
    int win_KH, win_len, win_shift, win_owb, win_OH, win_dw;
};


// Implicit GEMM: one BM x BN output tile per 256-thread workgroup
// (blockIdx.x), the k range optionally split over blockIdx.y (split-K
// partials are summed by splitk_epilogue).
//
// B gather: every tap of the (padded) input is in bounds, so element (k, n)
// sits at byte offset col(n) + koff[k]: col(n) is a per-lane VGPR, koff[k] a
// wave-uniform SGPR from the per-layer table, and each element is a single
// buffer_load with (voffset, soffset) = (col(n), koff[k]).  Columns past N
// and k past K use out-of-range offsets and load 0.
// MODE kModeKvec: the B source holds k contiguously in aligned groups of four
// (a Gemm whose A is [rows][K] with K a multiple of 4), so each lane's four
// k of a column are one 16-byte load instead of four scalar ones.
// MODE kModeChk (implicit padding): the B source is the unpadded input, and
// each element is bounds-checked: tap table entry (kh*dh, kw*dw) of k against
// the lane's column base (oh*sh - ph, ow*sw - pw); taps outside the input
// load 0, so a padded conv needs no zero-padded copy of its input.
constexpr int kModePlain = 0, kModeKvec = 1, kModeChk = 2;

template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, int MODE = kModePlain>
__global__ void __launch_bounds__(256) conv_igemm_f32(IgemmArgs a) {
    constexpr bool KVEC = MODE == kModeKvec;
    constexpr bool CHK = MODE == kModeChk;
    constexpr int TM = BM / (32 * WAVES_M);
    constexpr int TN = BN / (32 * WAVES_N);
    constexpr int K8 = BK / 8;
    // Row pitch in floats: an odd multiple of 4 (BK + 4), so the 16-byte
    // accesses of 8 consecutive rows fall on 8 different 4-bank groups of
    // the LDS's 32 banks and the b128 traffic is conflict-free.
    constexpr int LDK = BK + 4;
    static_assert((LDK / 4) % 2 == 1, "row pitch an odd multiple of 16 bytes");
    constexpr int KPT = BK * BN / 256;  // B elements per thread per k-tile
    static_assert(WAVES_M * WAVES_N == 4, "four waves");
    static_assert(TM >= 1 && TN >= 1 && KPT % 4 == 0 && BN >= 64, "tile shape");
    static_assert(BK % 8 == 0, "BK multiple of 8");

    __shared__ __attribute__((aligned(16))) float Bs[2][BN * LDK];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WAVES_N;
    const int wn = wave % WAVES_N;

    // Consecutive workgroups land on different XCDs (round robin over 8);
    // remap so each XCD walks a contiguous range of tiles, m fastest, and the
    // tiles sharing one activation panel share that XCD's L2.
    //
    // Split-K: blockIdx.y is the k slice and every tile writes partials.
    // Hybrid (dp_tiles > 0, one grid row): the first dp_tiles workgroups
    // each compute a whole tile (the largest multiple of the CU count that is
    // whole n-tile columns, rounded down to such columns, so the CUs get
    // equal shares), the remaining tiles are cut into kt_per_split k-tile
    // slices, one workgroup each, whose partials splitk_epilogue sums.
    int bid = blockIdx.x;
    int slice = blockIdx.y;
    bool part = a.ws != nullptr;
    if (a.dp_tiles > 0) {
        if (bid < a.dp_tiles) {
            if ((a.dp_tiles & 7) == 0) bid = (bid & 7) * (a.dp_tiles >> 3) + (bid >> 3);
            part = false;
        } else {
            const int r = bid - a.dp_tiles;
            bid = a.dp_tiles + r / a.rem_split;
            slice = r - (r / a.rem_split) * a.rem_split;
        }
    } else {
        const int nb = gridDim.x;
        if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
    }
    const int mt = bid % a.m_tiles;
    const int nt = bid / a.m_tiles;
    const int kt0 = part ? slice * a.kt_per_split : 0;
    const int kt1 = part ? min(kt0 + a.kt_per_split, a.k_tiles) : a.k_tiles;

    const int bcol = tid % BN;
    const int bgrp = __builtin_amdgcn_readfirstlane(tid / BN);  // wave-uniform: BN >= 64
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(a.x), static_cast<short>(0), a.x_bytes, kBufferWord3);
    const int row = lane & 31;
    const int khalf = 4 * (lane >> 5);
    const int rsub = 4 * (lane >> 5);

    {
        int col = kOobOffset;
        int ihb = 0x40000000, iwb = 0;  // CHK: the column's input row / column at tap (0, 0)
        {
            const int n = nt * BN + bcol;
            if (n < a.Ntot) {
                const int img = n / a.OHW;
                const int sp = n - img * a.OHW;
                const int oh = sp / a.OW;
                const int ow = sp - oh * a.OW;
                if constexpr (CHK) {
                    ihb = oh * a.sh - a.chk_ph;
                    iwb = ow * a.sw - a.chk_pw;
                    col = (img * a.x_img_stride + ihb * a.Wp + iwb) * 4;  // may be negative: used only in bounds
                } else {
                    col = (img * a.x_img_stride + oh * a.sh * a.Wp + ow * a.sw) * 4;
                }
            }
        }

        // The weight operand goes straight from memory (L2: a layer's weights
        // are shared by all its workgroups) into MFMA fragment registers, one
        // k-tile ahead, in two register sets; the gathered activation operand
        // is staged through LDS (shared by the waves of a column), with two
        // register sets keeping the loads of tile t+2 in flight while tile t
        // is multiplied.  Native vector types: arrays of HIP's float4 class
        // are not promoted to registers.
        floatx4 a0[TM][K8], a1[TM][K8];
        float br0[KPT], br1[KPT];

#define IGEMM_LOAD_A(KT, AX)                                                                                         \
    {                                                                                                                \
        const int kt_ = min((KT), a.k_tiles - 1);                                                                    \
        const floatx4 *src =                                                                                         \
            reinterpret_cast<const floatx4 *>(a.wp + (static_cast<size_t>(mt) * a.k_tiles + kt_) * (BM * BK));       \
        _Pragma("unroll") for (int i = 0; i < TM; i++) _Pragma("unroll") for (int q = 0; q < K8; q++) AX[i][q] =      \
            src[((wm * TM + i) * K8 + q) * 64 + lane];                                                               \
    }
#define IGEMM_LOAD_B(KT, BR)                                                                                         \
    {                                                                                                                \
        /* the table has two tiles of out-of-range entries past Kpad */                                           \
        const int *ko = a.koff + (KT) * BK + bgrp * KPT;                                                              \
        if constexpr (KVEC) {                                                                                        \
            /* the four k of a quad are all below K or all past it (K % 4 == 0) */                                  \
            _Pragma("unroll") for (int j = 0; j < KPT; j += 4) {                                                     \
                const floatx4 v_ =                                                                                   \
                    __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(xrs, col, ko[j], 0));          \
                BR[j] = v_[0];                                                                                       \
                BR[j + 1] = v_[1];                                                                                   \
                BR[j + 2] = v_[2];                                                                                   \
                BR[j + 3] = v_[3];                                                                                   \
            }                                                                                                        \
        } else if constexpr (CHK) {                                                                                  \
            /* past K the tap entry is out of every input, so those k load 0 too */                                 \
            const int *kt_ = a.ktap + (KT) * BK + bgrp * KPT;                                                         \
            _Pragma("unroll") for (int j = 0; j < KPT; j++) {                                                        \
                const int tp_ = kt_[j];                                                                              \
                const bool in_ = static_cast<unsigned>(ihb + (tp_ >> 16)) < static_cast<unsigned>(a.chk_H) &&         \
                                 static_cast<unsigned>(iwb + (tp_ & 0xffff)) < static_cast<unsigned>(a.chk_W);        \
                BR[j] = __builtin_bit_cast(                                                                          \
                    float, __builtin_amdgcn_raw_buffer_load_b32(xrs, in_ ? col + ko[j] : kOobOffset, 0, 0));         \
            }                                                                                                        \
        } else {                                                                                                     \
            _Pragma("unroll") for (int j = 0; j < KPT; j++) BR[j] = __builtin_bit_cast(                              \
                float, __builtin_amdgcn_raw_buffer_load_b32(xrs, col, ko[j], 0));                                    \
        }                                                                                                            \
    }
#define IGEMM_STORE_B(BUF, BR)                                                                                       \
    {                                                                                                                \
        _Pragma("unroll") for (int j = 0; j < KPT; j += 4) *reinterpret_cast<floatx4 *>(                             \
            &Bs[BUF][bcol * LDK + bgrp * KPT + j]) = floatx4{BR[j], BR[j + 1], BR[j + 2], BR[j + 3]};                \
    }

    // B fragments of one 8-k step: one ds_read_b128 per 32-column block
    // (lane: column row, k = 8*q + khalf + 0..3, the same k order as the
    // packed weights).
#define IGEMM_FRAG_B(BUF, Q, BF)                                                                                     \
    {                                                                                                                \
        _Pragma("unroll") for (int j = 0; j < TN; j++) BF[j] =                                                       \
            *reinterpret_cast<const floatx4 *>(&Bs[BUF][((wn * TN + j) * 32 + row) * LDK + (Q) * 8 + khalf]);        \
    }
#define IGEMM_MMA(AX, Q, BF)                                                                                         \
    _Pragma("unroll") for (int s = 0; s < 4; s++) _Pragma("unroll") for (int i = 0; i < TM; i++)                     \
        _Pragma("unroll") for (int j = 0; j < TN; j++) acc[i][j] =                                                   \
            __builtin_amdgcn_mfma_f32_32x32x2f32(AX[i][Q][s], BF[j][s], acc[i][j], 0, 0, 0);
    // The B fragments of step q+1 are read while the MFMAs of step q run
    // (two register sets), so LDS latency stays off the MFMA chain.
#define IGEMM_COMPUTE(BUF, AX)                                                                                       \
    {                                                                                                                \
        floatx4 fb0[TN], fb1[TN];                                                                                    \
        IGEMM_FRAG_B(BUF, 0, fb0);                                                                                   \
        _Pragma("unroll") for (int q = 0; q < K8; q += 2) {                                                          \
            if (q + 1 < K8) IGEMM_FRAG_B(BUF, q + 1, fb1);                                                           \
            IGEMM_MMA(AX, q, fb0);                                                                                   \
            if (q + 2 < K8) IGEMM_FRAG_B(BUF, q + 2, fb0);                                                           \
            if (q + 1 < K8) { IGEMM_MMA(AX, q + 1, fb1); }                                                           \
        }                                                                                                            \
    }

    // One pipeline step: B of tile KT is in LDS buffer BUF and its A in AC;
    // B of tile KT+1 is in flight in BNX; B of tile KT+2 is loaded into the
    // free set BF and A of tile KT+1 into AN.
#define IGEMM_STEP(KT, BUF, AC, AN, BNX, BF)                                                                         \
    {                                                                                                                \
        IGEMM_LOAD_B((KT) + 2, BF);                                                                                  \
        IGEMM_LOAD_A((KT) + 1, AN);                                                                                  \
        __builtin_amdgcn_sched_barrier(0);                                                                           \
        IGEMM_COMPUTE(BUF, AC);                                                                                      \
        __builtin_amdgcn_sched_barrier(0);                                                                           \
        IGEMM_STORE_B((BUF) ^ 1, BNX);                                                                               \
        __syncthreads();                                                                                             \
    }

        floatx16 acc[TM][TN];
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

        if (kt0 >= kt1) return;  // empty split-K slice
        IGEMM_LOAD_B(kt0, br0);
        IGEMM_LOAD_B(kt0 + 1, br1);
        IGEMM_LOAD_A(kt0, a0);
        IGEMM_STORE_B(0, br0);
        __syncthreads();
        int kt = kt0;
        // Tiles past kt1 are loaded and ignored, which keeps the loop free of
        // data-dependent branches.
        for (; kt + 1 < kt1; kt += 2) {
            IGEMM_STEP(kt, 0, a0, a1, br1, br0);
            IGEMM_STEP(kt + 1, 1, a1, a0, br0, br1);
        }
        if (kt < kt1) {
            IGEMM_COMPUTE(0, a0);
        }
#undef IGEMM_STEP
#undef IGEMM_COMPUTE
#undef IGEMM_MMA
#undef IGEMM_FRAG_B
#undef IGEMM_LOAD_A
#undef IGEMM_LOAD_B
#undef IGEMM_STORE_B

        // 32x32 accumulator layout: lane holds column (lane & 31) and rows
        // 8*(r/4) + 4*(lane/32) + (r%4) for r = 0..15.  Output offsets are
        // 32-bit (tensors < 2 GiB); rows past M and columns past N get an
        // out-of-range offset, so the buffer stores drop them.
        int obase[TN];  // byte offset of (row 0, this lane's column) in y / res / ws
        int mrow[TM];   // first row of this lane in block i
#pragma unroll
        for (int i = 0; i < TM; i++) mrow[i] = mt * BM + (wm * TM + i) * 32 + rsub;
        if (part) {
            // split-K partials: ws[slice][m][n - ws_n0], rows of ws_ld columns
            const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
                a.ws, static_cast<short>(0), a.ws_bytes, kBufferWord3);
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int n = nt * BN + (wn * TN + j) * 32 + row;
                obase[j] = n < a.Ntot ? (slice * a.M * a.ws_ld + n - a.ws_n0) * 4 : kOobOffset;
            }
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int m = mrow[i] + 8 * (r >> 2) + (r & 3);
                        const int off = m < a.M ? obase[j] + m * a.ws_ld * 4 : kOobOffset;
                        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[i][j][r]), wrs, off, 0, 0);
                    }
            return;  // splitk_epilogue sums the partials
        }
        {
            const int ohw4 = a.OHW * 4;      // the residual's channel stride (natural layout)
            const int ycs4 = a.y_cstride * 4;  // y's
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int n = nt * BN + (wn * TN + j) * 32 + row;
                const int img = n / a.OHW;
                const int sp = n - img * a.OHW;
                obase[j] = n < a.Ntot ? (img * a.y_img_stride + sp) * 4 : kOobOffset;
            }
            float *const any = a.y ? a.y : a.yp;
            const __amdgpu_buffer_rsrc_t yrs =
                __builtin_amdgcn_make_buffer_rsrc(any, static_cast<short>(0), a.y ? a.y_bytes : 0, kBufferWord3);
            const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
                a.yp ? a.yp : any, static_cast<short>(0), a.yp ? a.yp_bytes : 0, kBufferWord3);
            const __amdgpu_buffer_rsrc_t rrs = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float *>(a.res ? a.res : any), static_cast<short>(0), a.res ? a.y_bytes : 0, kBufferWord3);
            const __amdgpu_buffer_rsrc_t brs = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float *>(a.bias ? a.bias : any), static_cast<short>(0), a.bias ? a.M * 4 : 0, kBufferWord3);
            // handoff target: this lane's pixel in the padded planes
            int pbase[TN];
            const int plane4 = a.yp_plane * 4;
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int n = nt * BN + (wn * TN + j) * 32 + row;
                const int img = n / a.OHW;
                const int sp = n - img * a.OHW;
                const int oh = sp / a.OW;
                const int ow = sp - oh * a.OW;
                pbase[j] = n < a.Ntot ? (img * a.yp_C * a.yp_plane + (oh + a.yp_pt) * a.yp_Wp + ow + a.yp_pl) * 4
                                      : kOobOffset;
            }
            // one 32x32 block at a time: its 16 bias and 16 residual loads are
            // all in flight before the first use
#pragma unroll
            for (int i = 0; i < TM; i++) {
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    floatx16 v = acc[i][j];
                    if (a.alpha != 1.0f) v *= a.alpha;
                    if (a.bias) {
                        floatx16 bv;
#pragma unroll
                        for (int r = 0; r < 16; r++)
                            bv[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                                  brs, (mrow[i] + 8 * (r >> 2) + (r & 3)) * 4, 0, 0));
                        v += bv;
                    }
                    if (a.res) {
                        floatx16 rv;
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const int m = mrow[i] + 8 * (r >> 2) + (r & 3);
                            rv[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                                  rrs, m < a.M ? obase[j] + m * ohw4 : kOobOffset, 0, 0));
                        }
                        v += rv;
                    }
                    if (a.act == 1) {
#pragma unroll
                        for (int r = 0; r < 16; r++) v[r] = v[r] > 0.0f ? v[r] : 0.0f;
                    } else if (a.act == 2) {
#pragma unroll
                        for (int r = 0; r < 16; r++) v[r] = apply_act(v[r], 2);
                    }
                    if (a.yp) {
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const unsigned mc = static_cast<unsigned>(mrow[i] + 8 * (r >> 2) + (r & 3) - a.yp_m0);
                            __builtin_amdgcn_raw_buffer_store_b32(
                                __float_as_uint(v[r]), prs,
                                mc < static_cast<unsigned>(a.yp_C) ? pbase[j] + static_cast<int>(mc) * plane4 : kOobOffset,
                                0, 0);
                        }
                    }
                    if (a.y) {
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const int m = mrow[i] + 8 * (r >> 2) + (r & 3);
                            // __float_as_uint takes the element by value (a bit
                            // cast applied to a vector element reads element 0)
                            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[r]), yrs,
                                                                  m < a.M ? obase[j] + m * ycs4 : kOobOffset, 0, 0);
                        }
                    }
                }
            }
        }
    }
}

// Skinny implicit GEMM, for layers whose output is too small to fill the GPU
// with 64-wide tiles (batch 1): one 16 x 16 output tile per workgroup, its
// k range cut into chunks of 64 dealt round robin to the W waves (chunk c to
// wave c % W), each wave accumulating the whole tile over its chunks on
// v_mfma_f32_16x16x4f32; the W partial tiles are summed through LDS in wave
// order, then the epilogue runs.  Many workgroups without split-K partials
// in memory and without a second kernel.
//
// k order: k = tap * C + c with C a multiple of 64, so a chunk is 64
// consecutive channels of one tap.  MFMA t (0..15) of a chunk takes its k
// slot g (lanes 16g..16g+15) from k = 64 * chunk + 16g + t: a lane's 16 A
// values (its row m) are one 64-byte run of the packed weights, and its 16 B
// values are channels 16g..16g+15 of the chunk at its column n, loaded with
// voffset = col(n) + chunk base and soffset = t * channel stride.  Columns
// past N use an out-of-range voffset and load 0.
//
// P chunks are in flight per wave (4 x 20 loads at most, within the 63
// vmcnt allows); the launch takes P = 1 or 2 when no wave has more chunks
// than that, so the unused load buffers do not cost registers (and
// workgroups per CU), and P = 2 for sixteen waves, whatever their chunks
// (128 registers a wave).  P does not change the summation order.
template <int W, int P>
__global__ void __launch_bounds__(64 * W) conv_skinny_f32(IgemmArgs a) {
    __shared__ float red[W][256];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // wave-uniform in a scalar register: a chunk's tap arithmetic is scalar
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4;
    const int l16 = lane & 15;
    int bid = blockIdx.x;
    const int nb = gridDim.x;
    if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
    // n-tiles of one m-tile consecutive: each XCD fetches only its m-tiles'
    // weights into its L2
    const int ntiles = nb / a.m_tiles;
    const int mt = bid / ntiles;
    const int nt = bid - mt * ntiles;
    const int KC = a.k_tiles;  // chunks of 64 k

    int col = kOobOffset;
    {
        const int n = nt * 16 + l16;
        if (n < a.Ntot) {
            const int img = n / a.OHW;
            const int sp = n - img * a.OHW;
            const int oh = sp / a.OW;
            const int ow = sp - oh * a.OW;
            col = (img * a.x_img_stride + oh * a.sh * a.Wp + ow * a.sw) * 4;
        }
    }
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(a.x), static_cast<short>(0), a.x_bytes, kBufferWord3);
    const int cs4 = a.sk_cstride * 4;
    // the lane's column and its k slot's channel offset within a chunk
    const int colg = col == kOobOffset ? kOobOffset : col + 16 * g * cs4;
    // packed weights [m_tiles][KC][4 slots][16 rows][16 k] (fewer than 2^31
    // bytes, checked at launch); a lane's 16 values of a chunk are one 64-byte
    // run at wbase + chunk * 4096
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(a.wp), static_cast<short>(0), a.m_tiles * KC * 4096, kBufferWord3);
    const int wbase = (mt * KC * 1024 + (g * 16 + l16) * 16) * 4;
    const int nch = wave < KC ? (KC - wave + W - 1) / W : 0;

    // the epilogue's element of this thread (tid < 256): its bias and
    // residual are loaded now, so their latency hides under the k loop
    const int em = mt * 16 + (tid >> 4);
    const int en = nt * 16 + (tid & 15);
    const bool eown = tid < 256 && em < a.M && en < a.Ntot;
    const int eimg = eown ? en / a.OHW : 0;
    const int esp = en - eimg * a.OHW;
    // (y's channel stride: a residual comes only with y's natural layout)
    const size_t eyi = static_cast<size_t>(eimg) * a.y_img_stride + static_cast<size_t>(em) * a.y_cstride + esp;
    const float ebias = eown && a.bias ? a.bias[em] : 0.0f;
    const float eres = eown && a.res ? a.res[eyi] : 0.0f;

    floatx4 av[P][4];
    float bv[P][16];
    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};

    // loads chunk I of this wave into register set S.  Past the wave's last
    // chunk (the pipeline's tail) every offset is out of range: the loads
    // return zeros without a memory access, and stay unconditional so the
    // compiler keeps exact counts of the loads in flight (a branch around
    // them makes it wait for all of them before each chunk's MFMAs).
#define SK_LOAD(I, S)                                                                                             \
    {                                                                                                             \
        const int kr_ = wave + W * (I);                                                                           \
        const bool own_ = kr_ < KC;                                                                               \
        const int kc_ = own_ ? kr_ : 0;                                                                           \
        const int ao_ = own_ ? wbase + kc_ * 4096 : kOobOffset;                                                   \
        _Pragma("unroll") for (int q = 0; q < 4; q++) av[S][q] =                                                  \
            __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(wrs, ao_, q * 16, 0));              \
        const int k0_ = kc_ * 64;                                                                                 \
        const int tap_ = k0_ / a.sk_C;                                                                            \
        const int c0_ = k0_ - tap_ * a.sk_C;                                                                      \
        const int kh_ = tap_ / a.sk_KW;                                                                           \
        const int kw_ = tap_ - kh_ * a.sk_KW;                                                                     \
        const int uo_ = (kh_ * a.sk_tap_h + kw_ * a.sk_tap_w + c0_ * a.sk_cstride) * 4;                           \
        const int vo_ = colg == kOobOffset || !own_ ? kOobOffset : colg + uo_;                                    \
        _Pragma("unroll") for (int t = 0; t < 16; t++) bv[S][t] =                                                 \
            __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xrs, vo_, t * cs4, 0));                \
    }
#define SK_MMA(S)                                                                                                 \
    _Pragma("unroll") for (int t = 0; t < 16; t++) acc =                                                          \
        __builtin_amdgcn_mfma_f32_16x16x4f32(av[S][t >> 2][t & 3], bv[S][t], acc, 0, 0, 0);

    if constexpr (P < 4) {
        // groups of P chunks, all loads of a group before its MFMAs (one
        // group when no wave has more than P chunks, as the launch arranges).
        // The MFMAs are unconditional (a branch around them lets the compiler
        // sink each load next to its MFMA, one round trip per load): past the
        // wave's last chunk both operands are zeros, which leave acc
        // bit-identical, as acc starts at +0 and a sum that starts at +0 is
        // never -0.
        for (int i0 = 0; i0 < nch; i0 += P) {
#pragma unroll
            for (int p = 0; p < P; p++) SK_LOAD(i0 + p, p);
#pragma unroll
            for (int p = 0; p < P; p++) { SK_MMA(p); }
        }
    } else if (nch > 0) {
        // a ring of P register sets: chunk i + P - 1 loads while chunk i
        // multiplies
#pragma unroll
        for (int p = 0; p < P - 1; p++) SK_LOAD(p, p);
        for (int i0 = 0; i0 < nch; i0 += P) {
#pragma unroll
            for (int p = 0; p < P; p++) {
                SK_LOAD(i0 + p + P - 1, (p + P - 1) % P);
                if (i0 + p < nch) { SK_MMA(p); }
            }
        }
    }
#undef SK_LOAD
#undef SK_MMA

    // 16x16 accumulator layout: lane (g, l16) holds rows 4g..4g+3 of column l16
#pragma unroll
    for (int i = 0; i < 4; i++) red[wave][(4 * g + i) * 16 + l16] = acc[i];
    __syncthreads();
    if (eown) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < W; w++) v += red[w][tid];
        if (a.alpha != 1.0f) v *= a.alpha;
        if (a.bias) v += ebias;
        if (a.res) v += eres;
        v = apply_act(v, a.act);
        if (a.yp && static_cast<unsigned>(em - a.yp_m0) < static_cast<unsigned>(a.yp_C)) {
            const int oh = esp / a.OW;
            const int ow = esp - oh * a.OW;
            a.yp[(static_cast<size_t>(eimg) * a.yp_C + em - a.yp_m0) * a.yp_plane + (oh + a.yp_pt) * a.yp_Wp + ow +
                 a.yp_pl] = v;
        }
        if (a.y) a.y[eyi] = v;
    }
}

// Row-window implicit GEMM: the skinny kernel's arithmetic (16 x 16 output
// tile, 64-k chunks dealt round robin to W waves, 16 MFMAs per chunk, the
// wave partials summed in wave order: the same k order and sums, so the same
// bits as conv_skinny_f32<W>) with the B operand staged once per workgroup.
// A workgroup takes 16 output channels by 16 consecutive pixels of one output
// row; the input those pixels read -- C channels of KH rows of win_len
// columns, each element once, against once per tap in the skinny kernel --
// is loaded into LDS first, every load of a thread in flight together, so
// only the weights stream through the k loop: four 16-byte loads per chunk,
// R chunks in flight.  The window is channel-minor, [kh][column][C + 4]
// floats (dynamic LDS): a lane's 16 channels of a chunk are four 16-byte
// LDS reads, the rows of 16 lanes 16 bytes apart mod 256 (no bank
// conflicts), issued before the previous chunk's MFMAs.  Pixels past the
// row's end read column 0 of the window and are not stored.
constexpr int kWinFloats = 24576;  // most LDS a window may take: 96 KB

template <int W, int R, int KH>
__global__ void __launch_bounds__(64 * W) conv_window_f32(IgemmArgs a) {
    extern __shared__ float win[];
    __shared__ float red[W][256];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4;
    const int l16 = lane & 15;
    int bid = blockIdx.x;
    const int nb = gridDim.x;
    if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
    // the n-tiles of one m-tile are consecutive, so each XCD (a contiguous
    // range after the remap) fetches only its m-tiles' weights, the larger
    // operand at batch 1, into its L2 (stage-4 3x3 conv: 23.8 -> 20.4 us)
    const int ntiles = nb / a.m_tiles;
    const int mt = bid / ntiles;
    const int nt = bid - mt * ntiles;  // (output row, 16-pixel segment)
    const int row = nt / a.win_owb;
    const int ow0 = (nt - row * a.win_owb) * 16;
    const int img = row / a.win_OH;
    const int oh = row - img * a.win_OH;
    const int KC = a.k_tiles;
    const int C = a.sk_C;
    const int CP = C + 4;  // LDS floats per window column

    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(a.wp), static_cast<short>(0), a.m_tiles * KC * 4096, kBufferWord3);
    const int wbase = (mt * KC * 1024 + (g * 16 + l16) * 16) * 4;
    const int nch = wave < KC ? (KC - wave + W - 1) / W : 0;
    floatx4 av[R][4];
    // weights of chunk I of this wave into register set S (out-of-range
    // offsets past the wave's last chunk: zeros, no memory access)
#define WN_LOAD(I, S)                                                                                             \
    {                                                                                                             \
        const int kr_ = wave + W * (I);                                                                           \
        const int ao_ = kr_ < KC ? wbase + kr_ * 4096 : kOobOffset;                                               \
        _Pragma("unroll") for (int q = 0; q < 4; q++) av[S][q] =                                                  \
            __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(wrs, ao_, q * 16, 0));              \
    }
    // the epilogue's element of this thread (tid < 256): bias and residual
    // loaded now
    const int em = mt * 16 + (tid >> 4);
    const int eow = ow0 + (tid & 15);
    const bool eown = tid < 256 && em < a.M && eow < a.OW;
    const int esp = oh * a.OW + eow;
    const size_t eyi = static_cast<size_t>(img) * a.y_img_stride + static_cast<size_t>(em) * a.y_cstride + esp;
    const float ebias = eown && a.bias ? a.bias[em] : 0.0f;
    const float eres = eown && a.res ? a.res[eyi] : 0.0f;

    // the window: element (kh, j, c) is input row oh * sh + kh * dh, column
    // ow0 * sw + j of channel c.  A wave instruction loads rpi = 64 >>
    // win_shift channels of one kh, one lane per column; a thread's channels
    // are c_first + u * cstep, their KH rows each, up to 48 loads in flight.
    // The ring's first R - 1 weight chunks go out after the window's loads
    // (which the barrier waits for) and before its LDS writes.
    {
        const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float *>(a.x), static_cast<short>(0), a.x_bytes, kBufferWord3);
        const int rpi = 64 >> a.win_shift;
        const int q = lane >> a.win_shift;
        const int j = lane & ((1 << a.win_shift) - 1);
        const int cstep = W * rpi;
        const int c_first = wave * rpi + q;
        const bool jload = j < a.win_len;
        const int xb = (img * a.x_img_stride + oh * a.sh * a.Wp + ow0 * a.sw + j + c_first * a.sk_cstride) * 4;
        const int xstep = cstep * a.sk_cstride * 4;
        const int tap4 = a.sk_tap_h * 4;
        constexpr int UC = (W >= 16 ? 24 : 48) / KH;  // channels per thread in flight
        float v[UC][KH];
#define WN_FILL_LOADS(U0)                                                                                         \
    _Pragma("unroll") for (int u = 0; u < UC; u++) {                                                              \
        const bool ok_ = c_first + ((U0) + u) * cstep < C && jload;                                               \
        _Pragma("unroll") for (int kh = 0; kh < KH; kh++) v[u][kh] = __builtin_bit_cast(                          \
            float, __builtin_amdgcn_raw_buffer_load_b32(xrs, ok_ ? xb + ((U0) + u) * xstep + kh * tap4 : kOobOffset,  \
                                                         0, 0));                                                  \
    }
#define WN_FILL_STORES(U0)                                                                                        \
    _Pragma("unroll") for (int u = 0; u < UC; u++) {                                                              \
        const int c_ = c_first + ((U0) + u) * cstep;                                                              \
        if (c_ < C && jload) {                                                                                    \
            _Pragma("unroll") for (int kh = 0; kh < KH; kh++) win[(kh * a.win_len + j) * CP + c_] = v[u][kh];     \
        }                                                                                                         \
    }
        // the first batch runs in every thread (lanes with no channel load
        // out-of-range offsets): the weight prologue after it must run in
        // every wave, also in waves with no window channels
        WN_FILL_LOADS(0);
        if (nch > 0) {
#pragma unroll
            for (int p = 0; p < R - 1; p++) WN_LOAD(p, p);
        }
        WN_FILL_STORES(0);
        for (int u0 = UC; c_first + u0 * cstep < C; u0 += UC) {
            WN_FILL_LOADS(u0);
            WN_FILL_STORES(u0);
        }
#undef WN_FILL_LOADS
#undef WN_FILL_STORES
    }
    __syncthreads();

    // a lane's column in the window (pixels past the row's end: column 0)
    const int jcol = ow0 + l16 < a.OW ? l16 * a.sw : 0;
    const int gbase = jcol * CP + 16 * g;
    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    float bv[2][16];
    // the 16 LDS values of chunk I of this wave into B set S
#define WN_BREAD(I, S)                                                                                            \
    {                                                                                                             \
        const int k0_ = min(wave + W * (I), KC - 1) * 64;                                                         \
        const int tap_ = k0_ / C;                                                                                 \
        const int c0_ = k0_ - tap_ * C;                                                                           \
        const int kh_ = tap_ / a.sk_KW;                                                                           \
        const int kw_ = tap_ - kh_ * a.sk_KW;                                                                     \
        const float *b_ = win + gbase + (kh_ * a.win_len + kw_ * a.win_dw) * CP + c0_;                            \
        _Pragma("unroll") for (int t4 = 0; t4 < 4; t4++) {                                                        \
            const floatx4 v4_ = *reinterpret_cast<const floatx4 *>(b_ + 4 * t4);                                  \
            _Pragma("unroll") for (int e = 0; e < 4; e++) bv[S][4 * t4 + e] = v4_[e];                             \
        }                                                                                                         \
    }
#define WN_MMA(A, S)                                                                                              \
    _Pragma("unroll") for (int t = 0; t < 16; t++) acc =                                                          \
        __builtin_amdgcn_mfma_f32_16x16x4f32(av[A][t >> 2][t & 3], bv[S][t], acc, 0, 0, 0);
    if (nch > 0) {
        WN_BREAD(0, 0);
        for (int i0 = 0; i0 < nch; i0 += R) {
#pragma unroll
            for (int p = 0; p < R; p++) {
                WN_LOAD(i0 + p + R - 1, (p + R - 1) % R);
                if (i0 + p < nch) {
                    if (i0 + p + 1 < nch) { WN_BREAD(i0 + p + 1, (p + 1) & 1); }
                    WN_MMA(p, p & 1);
                }
            }
        }
    }
#undef WN_LOAD
#undef WN_BREAD
#undef WN_MMA

    // 16x16 accumulator layout: lane (g, l16) holds rows 4g..4g+3 of column l16
#pragma unroll
    for (int i = 0; i < 4; i++) red[wave][(4 * g + i) * 16 + l16] = acc[i];
    __syncthreads();
    if (eown) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < W; w++) v += red[w][tid];
        if (a.alpha != 1.0f) v *= a.alpha;
        if (a.bias) v += ebias;
        if (a.res) v += eres;
        v = apply_act(v, a.act);
        if (a.yp && static_cast<unsigned>(em - a.yp_m0) < static_cast<unsigned>(a.yp_C))
            a.yp[(static_cast<size_t>(img) * a.yp_C + em - a.yp_m0) * a.yp_plane + (oh + a.yp_pt) * a.yp_Wp + eow +
                 a.yp_pl] = v;
        if (a.y) a.y[eyi] = v;
    }
}

// Thin implicit GEMM, for layers with few output channels and many output
// pixels (YOLO's 16- and 32-channel layers at 80x80 to 320x320): MB blocks
// of 16 rows by 256 columns per workgroup, each wave 64 of the columns as
// four 16x16 blocks on v_mfma_f32_16x16x4f32.  The waves share nothing, so
// there is no LDS and no barrier: each lane loads its B elements straight
// into registers and its A elements from the packed weights (the same for
// the four waves: L1 hits), with two 16-k chunks of loads in flight.
//
// k order k' = tap * C + c (C a multiple of 4): MFMA step s takes its k
// slot g (lanes 16g..16g+15) from channel 4 * (s % (C/4)) + g of tap
// s / (C/4), so the B element of a lane's column n sits at col(n) (per
// lane, with g's channel) plus a tap and channel-quad offset that is the
// same for the wave.  Steps past K / 4 load nothing (0) and meet zero
// weights.  Packed weights [m_tiles][k_tiles][MB][64 lanes][4 steps]: lane
// (g, r) of block b holds row 16b + r at k' = 16 kt + 4 step + g.  Columns
// past N and rows past M use out-of-range offsets (loads give 0, stores are
// dropped), as in conv_igemm_f32.
template <int MB>
__global__ void __launch_bounds__(256) conv_thin_f32(IgemmArgs a) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = lane >> 4;
    const int l16 = lane & 15;
    int bid = blockIdx.x;
    const int nb = gridDim.x;
    if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
    const int mt = bid % a.m_tiles;
    const int nt = bid / a.m_tiles;
    const int cs4 = a.sk_cstride * 4;
    const int n0 = nt * 256 + wave * 64;
    int col[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int n = n0 + 16 * j + l16;
        col[j] = kOobOffset;
        if (n < a.Ntot) {
            const int img = n / a.OHW;
            const int sp = n - img * a.OHW;
            const int oh = sp / a.OW;
            const int ow = sp - oh * a.OW;
            col[j] = (img * a.x_img_stride + oh * a.sh * a.Wp + ow * a.sw) * 4 + g * cs4;
        }
    }
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(a.x), static_cast<short>(0), a.x_bytes, kBufferWord3);
    const int CQ = a.sk_C >> 2;
    const floatx4 *wsrc = reinterpret_cast<const floatx4 *>(a.wp) + static_cast<size_t>(mt) * a.k_tiles * MB * 64 + lane;

    floatx4 acc[MB][4];
#pragma unroll
    for (int b = 0; b < MB; b++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[b][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    constexpr int P = 3;  // chunks in flight: 3 x (16 + MB) loads, within the 63 vmcnt counts
    floatx4 av[P][MB];
    float bv[P][4][4];  // [set][step][column block]

    // Chunks are loaded in order, so the next step's tap (kh, kw) and channel
    // quad are counters advanced once per step (wave-uniform; no division
    // in the loop, whose scalar unit the CU's waves share).
    int s_next = 0, st_cq = 0, st_kh = 0, st_kw = 0;
    // chunk KT (4 steps) into (AV, BV); past the last chunk a valid chunk of
    // weights and no B elements (steps past K / 4) are loaded, never used
#define TH_LOAD(KT, AV, BV)                                                                                       \
    {                                                                                                             \
        const int kt_ = min((KT), a.k_tiles - 1);                                                                 \
        _Pragma("unroll") for (int b = 0; b < MB; b++) AV[b] = wsrc[(static_cast<size_t>(kt_) * MB + b) * 64];   \
        _Pragma("unroll") for (int st = 0; st < 4; st++) {                                                        \
            if (s_next < a.th_steps) {                                                                            \
                const int so_ = (st_kh * a.sk_tap_h + st_kw * a.sk_tap_w) * 4 + st_cq * 4 * cs4;                 \
                _Pragma("unroll") for (int j = 0; j < 4; j++) BV[st][j] =                                         \
                    __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xrs, col[j], so_, 0));         \
            } else {                                                                                              \
                _Pragma("unroll") for (int j = 0; j < 4; j++) BV[st][j] = 0.0f;                                   \
            }                                                                                                     \
            s_next++;                                                                                             \
            if (++st_cq == CQ) {                                                                                  \
                st_cq = 0;                                                                                        \
                if (++st_kw == a.sk_KW) {                                                                         \
                    st_kw = 0;                                                                                    \
                    st_kh++;                                                                                      \
                }                                                                                                 \
            }                                                                                                     \
        }                                                                                                         \
    }
#define TH_MMA(AV, BV)                                                                                            \
    _Pragma("unroll") for (int st = 0; st < 4; st++) _Pragma("unroll") for (int b = 0; b < MB; b++)               \
        _Pragma("unroll") for (int j = 0; j < 4; j++) acc[b][j] =                                                 \
            __builtin_amdgcn_mfma_f32_16x16x4f32(AV[b][st], BV[st][j], acc[b][j], 0, 0, 0);

    // a ring of P register sets: chunk i in set i % P, loaded P - 1 chunks
    // ahead of its multiply (the loop is unrolled by P so set indices are
    // constants)
#pragma unroll
    for (int p = 0; p < P - 1; p++) TH_LOAD(p, av[p], bv[p]);
    for (int k0 = 0; k0 < a.k_tiles; k0 += P) {
#pragma unroll
        for (int p = 0; p < P; p++) {
            TH_LOAD(k0 + p + P - 1, av[(p + P - 1) % P], bv[(p + P - 1) % P]);
            if (k0 + p < a.k_tiles) { TH_MMA(av[p], bv[p]); }
        }
    }
#undef TH_LOAD
#undef TH_MMA

    // 16x16 accumulator layout: lane (g, l16) holds rows 4g..4g+3 of column l16
    const int ohw4 = a.OHW * 4;
    int obase[4], pbase[4];
    const int plane4 = a.yp_plane * 4;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int n = n0 + 16 * j + l16;
        obase[j] = kOobOffset;
        pbase[j] = kOobOffset;
        if (n < a.Ntot) {
            const int img = n / a.OHW;
            const int sp = n - img * a.OHW;
            const int oh = sp / a.OW;
            const int ow = sp - oh * a.OW;
            obase[j] = (img * a.y_img_stride + sp) * 4;
            pbase[j] = (img * a.yp_C * a.yp_plane + (oh + a.yp_pt) * a.yp_Wp + ow + a.yp_pl) * 4;
        }
    }
    float *const any = a.y ? a.y : a.yp;
    const __amdgpu_buffer_rsrc_t yrs =
        __builtin_amdgcn_make_buffer_rsrc(any, static_cast<short>(0), a.y ? a.y_bytes : 0, kBufferWord3);
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
        a.yp ? a.yp : any, static_cast<short>(0), a.yp ? a.yp_bytes : 0, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(a.res ? a.res : any), static_cast<short>(0), a.res ? a.y_bytes : 0, kBufferWord3);
    const __amdgpu_buffer_rsrc_t brs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(a.bias ? a.bias : any), static_cast<short>(0), a.bias ? a.M * 4 : 0, kBufferWord3);
#pragma unroll
    for (int b = 0; b < MB; b++) {
        const int m0 = mt * 16 * MB + 16 * b + 4 * g;  // this lane's first row in block b
        floatx4 bias4 = {0.0f, 0.0f, 0.0f, 0.0f};
        if (a.bias) {
#pragma unroll
            for (int r = 0; r < 4; r++)
                bias4[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(brs, (m0 + r) * 4, 0, 0));
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            floatx4 v = acc[b][j];
            if (a.alpha != 1.0f) v *= a.alpha;
            if (a.bias) v += bias4;
            if (a.res) {
                floatx4 rv;
#pragma unroll
                for (int r = 0; r < 4; r++)
                    rv[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                          rrs, m0 + r < a.M ? obase[j] + (m0 + r) * ohw4 : kOobOffset, 0, 0));
                v += rv;
            }
#pragma unroll
            for (int r = 0; r < 4; r++) v[r] = apply_act(v[r], a.act);
            if (a.yp) {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const unsigned mc = static_cast<unsigned>(m0 + r - a.yp_m0);
                    __builtin_amdgcn_raw_buffer_store_b32(
                        __float_as_uint(v[r]), prs,
                        mc < static_cast<unsigned>(a.yp_C) ? pbase[j] + static_cast<int>(mc) * plane4 : kOobOffset, 0, 0);
                }
            }
            if (a.y) {
#pragma unroll
                for (int r = 0; r < 4; r++)
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[r]), yrs,
                                                          m0 + r < a.M ? obase[j] + (m0 + r) * a.y_cstride * 4 : kOobOffset,
                                                          0, 0);
            }
        }
    }
}

// Sums split-K partials in slice order, then applies the epilogue.  Each
// thread owns VEC consecutive columns of one row (VEC = 4 when the partial
// columns start and end on multiples of 4: 16-byte loads).
template <int VEC>
__global__ void __launch_bounds__(256) splitk_epilogue(const float *__restrict__ ws, int splitk, int M, int ld,
                                                       int OHW, const float *__restrict__ bias,
                                                       const float *__restrict__ res, float *__restrict__ y, int act,
                                                       float alpha, IgemmArgs h) {
    typedef float vec_t __attribute__((ext_vector_type(VEC)));
    // partial rows hold ld columns starting at column h.ws_n0
    const size_t total = static_cast<size_t>(M) * ld;
    const size_t groups = total / VEC;
    for (size_t gi = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; gi < groups;
         gi += static_cast<size_t>(gridDim.x) * 256) {
        const size_t idx = gi * VEC;
        const int m = static_cast<int>(idx / ld);
        const int n = h.ws_n0 + static_cast<int>(idx - static_cast<size_t>(m) * ld);
        // bias and residual loads issued first: their latency overlaps the
        // partials'
        const float bm = bias ? bias[m] : 0.0f;
        float rv[VEC];
#pragma unroll
        for (int e = 0; e < VEC; e++) {
            const int img = (n + e) / OHW;
            rv[e] = res ? res[static_cast<size_t>(img) * h.y_img_stride + static_cast<size_t>(m) * OHW +
                              (n + e - img * OHW)]
                        : 0.0f;
        }
        // up to 16 slices' loads in flight before the first add (one round
        // trip for splitk <= 16); the adds stay in slice order
        vec_t v = 0.0f;
        for (int s = 0; s < splitk; s += 16) {
            vec_t p[16];
#pragma unroll
            for (int t = 0; t < 16; t++)
                if (s + t < splitk) p[t] = *reinterpret_cast<const vec_t *>(ws + (s + t) * total + idx);
#pragma unroll
            for (int t = 0; t < 16; t++)
                if (s + t < splitk) v += p[t];
        }
#pragma unroll
        for (int e = 0; e < VEC; e++) {
            float o = alpha * v[e];
            if (bias) o += bm;
            const int img = (n + e) / OHW;
            const int sp = n + e - img * OHW;
            const size_t yi = static_cast<size_t>(img) * h.y_img_stride + static_cast<size_t>(m) * h.y_cstride + sp;
            if (res) o += rv[e];
            o = apply_act(o, act);
            if (h.yp && static_cast<unsigned>(m - h.yp_m0) < static_cast<unsigned>(h.yp_C)) {
                const int oh = sp / h.OW, ow = sp - (sp / h.OW) * h.OW;
                h.yp[(static_cast<size_t>(img) * h.yp_C + m - h.yp_m0) * h.yp_plane + (oh + h.yp_pt) * h.yp_Wp + ow +
                     h.yp_pl] = o;
            }
            if (y) y[yi] = o;
        }
    }
}

// Zero-padded copy of an NCHW tensor: planes of H x W placed at (pt, pl) in
// planes of Hp x Wp, halo written as zeros.  grid.y strides over planes,
// grid.x over the elements of a plane (32-bit index math), so small
// batches still spread over the GPU.
__global__ void __launch_bounds__(256) pad_nchw(const float *__restrict__ x, float *__restrict__ xp, unsigned planes,
                                                unsigned C, size_t x_img, int H, int W, int Hp, int Wp, int pt,
                                                int pl) {
    const unsigned plane_sz = static_cast<unsigned>(Hp * Wp);
    for (unsigned plane = blockIdx.y; plane < planes; plane += gridDim.y) {
        // images x_img elements apart (more than C planes: a channel slice)
        const float *src = x + (plane / C) * x_img + static_cast<size_t>(plane % C) * H * W;
        float *dst = xp + static_cast<size_t>(plane) * plane_sz;
        for (unsigned r = blockIdx.x * 256 + threadIdx.x; r < plane_sz; r += gridDim.x * 256) {
            const int hq = static_cast<int>(r / static_cast<unsigned>(Wp));
            const int h = hq - pt, w = static_cast<int>(r) - hq * Wp - pl;
            dst[r] = (static_cast<unsigned>(h) < static_cast<unsigned>(H) && static_cast<unsigned>(w) < static_cast<unsigned>(W))
                         ? src[h * W + w]
                         : 0.0f;
        }
    }
}

// grid of a per-plane kernel: x covers `per_plane` elements with 256-thread
// blocks, y the planes (capped; the kernels stride over the rest)
inline dim3 plane_grid(size_t per_plane, size_t planes) {
    const size_t gx = std::min<size_t>((per_plane + 255) / 256, 1024);
    const size_t gy = std::min<size_t>(planes, 65535);
    return dim3(static_cast<unsigned>(gx == 0 ? 1 : gx), static_cast<unsigned>(gy == 0 ? 1 : gy));
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

// ------------------------------------------------ small-gather stem kernel

// Convs with a few input channels (C <= 4: RGB stems) and a short gather per
// output pixel (C*KH*KW <= 64) whose output channels fit one thread
// (M <= 64).  As an implicit GEMM such a layer is one or two k-tiles per
// output tile with most MFMA rows empty, bound by its prologue and epilogue;
// here each wave takes 64 consecutive output pixels of one output row, one
// per lane, and each lane keeps all MT (>= M) output channels in registers:
// per tap one input load (the row test is wave-uniform, the column test per
// lane) and MT weights read from LDS as broadcast 16-byte reads.  Each output
// is summed from the bias in the reference's order (c, kh, kw), out-of-bounds
// taps skipped (runtime/kernels/reference/conv/conv.c:3-62), one fused
// multiply-add per tap; then residual, activation, and the stores: y and/or
// the consuming conv's zero-padded input (the fp32 pad handoff).
constexpr int kSmallkMaxC = 4;
constexpr int kSmallkMaxK = 64;

struct SmallkArgs {
    const float *__restrict__ x;
    const float *__restrict__ w;  // OIHW: [M][K]
    const float *__restrict__ bias;
    const float *__restrict__ res;
    float *__restrict__ y;   // null: only the handoff is stored
    float *__restrict__ yp;  // the consuming conv's zero-padded input, or null
    int N, C, H, W, M, KH, KW, OH, OW;
    int sh, sw, ph, pw, dh, dw, act;
    int segs;     // 64-pixel segments per output row
    int x_bytes;  // extent of x for the bounds-checked loads
    int yp_Hp, yp_Wp, yp_pt, yp_pl, yp_m0, yp_C;
};

template <int MT>
__global__ void __launch_bounds__(256) conv_smallk_f32(SmallkArgs a) {
    __shared__ __attribute__((aligned(16))) float wl[kSmallkMaxK * MT];  // [k][m], zero past M
    __shared__ int toff[kSmallkMaxK];                                    // element offset of tap k from tap 0
    __shared__ int tdd[kSmallkMaxK];                                     // (kh*dh) << 16 | kw*dw
    const int K = a.C * a.KH * a.KW;
    for (int i = threadIdx.x; i < K * MT; i += 256) {
        const int k = i / MT, m = i - k * MT;
        wl[i] = m < a.M ? a.w[m * K + k] : 0.0f;
    }
    for (int k = threadIdx.x; k < K; k += 256) {
        const int taps = a.KH * a.KW;
        const int c = k / taps, r = k - c * taps;
        const int dy = (r / a.KW) * a.dh, dx = (r % a.KW) * a.dw;
        toff[k] = (c * a.H + dy) * a.W + dx;
        tdd[k] = (dy << 16) | dx;
    }
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const long long item = static_cast<long long>(blockIdx.x) * 4 + (threadIdx.x >> 6);  // (n, oh, segment)
    if (item >= static_cast<long long>(a.N) * a.OH * a.segs) return;
    const int seg = static_cast<int>(item % a.segs);
    const int rest = static_cast<int>(item / a.segs);
    const int oh = rest % a.OH, n = rest / a.OH;
    const int ow = seg * 64 + lane;
    const bool live = ow < a.OW;
    const int ihb = oh * a.sh - a.ph, iwb = ow * a.sw - a.pw;
    const int base = (n * a.C * a.H + ihb) * a.W + iwb;  // tap (0, 0, 0); used only for taps in bounds
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(a.x), static_cast<short>(0), a.x_bytes, kBufferWord3);
    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; m++) acc[m] = a.bias && m < a.M ? a.bias[m] : 0.0f;
    // KC taps at a time: all their loads in flight together (taps outside
    // the input, and past K, load from an out-of-range offset and are skipped)
    constexpr int KC = 16;
    for (int k0 = 0; k0 < K; k0 += KC) {
        float xv[KC];
        unsigned okm = 0;
#pragma unroll
        for (int j = 0; j < KC; j++) {
            const int k = min(k0 + j, K - 1);
            const int dd = tdd[k];
            const bool ok = k0 + j < K && live &&
                            static_cast<unsigned>(ihb + (dd >> 16)) < static_cast<unsigned>(a.H) &&
                            static_cast<unsigned>(iwb + (dd & 0xffff)) < static_cast<unsigned>(a.W);
            xv[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                  xrs, ok ? (base + toff[k]) * 4 : kOobOffset, 0, 0));
            okm |= static_cast<unsigned>(ok) << j;
        }
#pragma unroll
        for (int j = 0; j < KC; j++) {
            if (k0 + j >= K) break;
            if ((okm >> j) & 1u) {  // lanes whose tap is outside the input skip it (exec mask)
                const floatx4 *wr = reinterpret_cast<const floatx4 *>(&wl[(k0 + j) * MT]);
#pragma unroll
                for (int q = 0; q < MT / 4; q++) {
                    const floatx4 wv = wr[q];
#pragma unroll
                    for (int u = 0; u < 4; u++) acc[4 * q + u] = fmaf(xv[j], wv[u], acc[4 * q + u]);
                }
            }
        }
    }
    if (!live) return;
    const size_t plane = static_cast<size_t>(a.OH) * a.OW;
    const size_t ybase = static_cast<size_t>(n) * a.M * plane + static_cast<size_t>(oh) * a.OW + ow;
    const size_t pplane = static_cast<size_t>(a.yp_Hp) * a.yp_Wp;
    const size_t pbase = static_cast<size_t>(n) * a.yp_C * pplane + static_cast<size_t>(oh + a.yp_pt) * a.yp_Wp + ow + a.yp_pl;
#pragma unroll
    for (int m = 0; m < MT; m++) {
        if (m < a.M) {  // (a constant trip count: acc stays in registers)
            float v = acc[m];
            if (a.res) v += a.res[ybase + m * plane];
            v = apply_act(v, a.act);
            if (a.y) a.y[ybase + m * plane] = v;
            const unsigned mc = static_cast<unsigned>(m - a.yp_m0);
            if (a.yp && mc < static_cast<unsigned>(a.yp_C)) a.yp[pbase + mc * pplane] = v;
        }
    }
}

// ---------------------------------------------------------- depthwise kernel

// Depthwise conv (one input channel per group, any channel multiplier), K x K
// taps known at compile time: each thread computes kDwVO outputs of one
// column, in consecutive rows, and lanes take consecutive columns, so each
// load instruction of a wave reads a contiguous run of an input row.  All of
// a thread's tap loads, its bias and its residuals are issued before the
// first multiply-add (one memory round trip); each output is then summed in
// the reference's order (from the bias, kh then kw, out-of-bounds taps
// skipped, one fused multiply-add per tap), the residual added and the
// activation applied.  The host keeps the thread count below 2^31, so the
// index math is 32-bit.
constexpr int kDwVO = 4;

template <int K>
__global__ void __launch_bounds__(256) conv_dw_f32(DirectArgs a, int row_groups, unsigned total) {
    const unsigned t = blockIdx.x * 256u + threadIdx.x;
    if (t >= total) return;
    const int ow = static_cast<int>(t % static_cast<unsigned>(a.OW));
    unsigned r = t / static_cast<unsigned>(a.OW);
    const int oh0 = static_cast<int>(r % static_cast<unsigned>(row_groups)) * kDwVO;
    r /= static_cast<unsigned>(row_groups);
    const int m = static_cast<int>(r % static_cast<unsigned>(a.M));
    const int n = static_cast<int>(r / static_cast<unsigned>(a.M));
    const int c = m / a.Mg;
    const float *xc = a.x + (static_cast<size_t>(n) * a.C + c) * a.H * a.W;
    const float *wm = a.w + static_cast<size_t>(m) * K * K;
    const size_t ybase = (static_cast<size_t>(n) * a.M + m) * a.OH * a.OW + ow;
    float wv[K * K];
#pragma unroll
    for (int i = 0; i < K * K; i++) wv[i] = wm[i];
    float xv[kDwVO][K][K];
    bool ok[kDwVO][K][K];
#pragma unroll
    for (int v = 0; v < kDwVO; v++)
#pragma unroll
        for (int kh = 0; kh < K; kh++) {
            const int ih = (oh0 + v) * a.sh + kh * a.dh - a.ph;
            const bool hin = oh0 + v < a.OH && static_cast<unsigned>(ih) < static_cast<unsigned>(a.H);
#pragma unroll
            for (int kw = 0; kw < K; kw++) {
                const int iw = ow * a.sw + kw * a.dw - a.pw;
                ok[v][kh][kw] = hin && static_cast<unsigned>(iw) < static_cast<unsigned>(a.W);
                xv[v][kh][kw] = ok[v][kh][kw] ? xc[ih * a.W + iw] : 0.0f;
            }
        }
    const float b0 = a.bias ? a.bias[m] : 0.0f;
    float rv[kDwVO];
#pragma unroll
    for (int v = 0; v < kDwVO; v++)
        rv[v] = a.res && oh0 + v < a.OH ? a.res[ybase + static_cast<size_t>(oh0 + v) * a.OW] : 0.0f;
#pragma unroll
    for (int v = 0; v < kDwVO; v++) {
        if (oh0 + v >= a.OH) break;
        float sum = b0;
#pragma unroll
        for (int kh = 0; kh < K; kh++)
#pragma unroll
            for (int kw = 0; kw < K; kw++)
                if (ok[v][kh][kw]) sum = fmaf(xv[v][kh][kw], wv[kh * K + kw], sum);
        if (a.res) sum += rv[v];
        a.y[ybase + static_cast<size_t>(oh0 + v) * a.OW] = apply_act(sum, a.act);
    }
}

// ------------------------------------------------------------- host side

namespace {

using IgemmKernel = void (*)(IgemmArgs);

struct TileCfg {
    int BM, BN, BK;  // skinny kernel: 16, 16 and the 64-k chunk
    const char *name;
    IgemmKernel kernel;
    IgemmKernel kernel_kvec;  // the same tile with 16-byte B loads along k (kModeKvec)
    IgemmKernel kernel_chk;   // the same tile with implicit padding (kModeChk)
    double eff;  // relative per-CU MFMA efficiency of the shape (measured on ResNet layers)
    int skinny_waves = 0;  // > 0: conv_skinny_f32 with this many waves (no split-K)
    int thin_mb = 0;       // > 0: conv_thin_f32 with this many 16-row blocks (no split-K)
    // with skinny_waves: conv_window_f32 instead (the skinny kernel's sums,
    // the input window in LDS; convolutions only)
    bool window = false;
};

#define CFGW(BM, BN, BK, WM, WN, EFF)                                                                        \
    {BM, BN, BK, #BM "x" #BN "x" #BK, conv_igemm_f32<BM, BN, BK, WM, WN, kModePlain>,                          \
     conv_igemm_f32<BM, BN, BK, WM, WN, kModeKvec>, conv_igemm_f32<BM, BN, BK, WM, WN, kModeChk>, EFF}
#define CFG(BM, BN, BK, EFF) CFGW(BM, BN, BK, 2, 2, EFF)
// the same with the wave layout in the name (tiles that another entry has
// with 2 x 2 waves)
#define CFGWL(BM, BN, BK, WM, WN, EFF)                                                                        \
    {BM, BN, BK, #BM "x" #BN "x" #BK ",w" #WM "x" #WN, conv_igemm_f32<BM, BN, BK, WM, WN, kModePlain>,       \
     conv_igemm_f32<BM, BN, BK, WM, WN, kModeKvec>, conv_igemm_f32<BM, BN, BK, WM, WN, kModeChk>, EFF}
const TileCfg kCfgs[] = {
    CFG(128, 128, 16, 0.85), CFG(128, 128, 32, 0.85), CFG(64, 128, 16, 0.90), CFG(64, 128, 32, 0.88),
    CFG(128, 64, 16, 1.00),  CFG(128, 64, 32, 0.95),  CFG(64, 64, 16, 0.96),  CFG(64, 64, 32, 0.98),
    // deep k-tiles: a short split-K slice (batch 1) is one or two of them,
    // so its operand loads are in flight together instead of one k-tile of
    // latency per 16 k
    CFG(64, 64, 64, 0.95),   CFG(64, 64, 128, 0.95), CFG(128, 64, 64, 0.95),  CFG(64, 128, 64, 0.90),
    // 16 x 16 tiles, k over 4 or 8 waves: small outputs without split-K
    // (kernel: the four-chunk pipeline; the launch picks a shallower one
    // by the chunks per wave, skinny_kernel)
    {16, 16, 64, "skinny16x16w4", conv_skinny_f32<4, 4>, conv_skinny_f32<4, 4>, conv_skinny_f32<4, 4>, 1.0, 4},
    {16, 16, 64, "skinny16x16w8", conv_skinny_f32<8, 4>, conv_skinny_f32<8, 4>, conv_skinny_f32<8, 4>, 1.0, 8},
    // 32-row tiles, the four waves side by side along n: layers with 16-48
    // output channels (YOLO) fill half or more of the MFMA rows instead of
    // a quarter to three quarters of a 64-row tile
    CFGW(32, 128, 16, 1, 4, 0.90), CFGW(32, 128, 32, 1, 4, 0.90), CFGW(32, 256, 16, 1, 4, 0.90),
    // thin tiles: 16 or 32 rows by 256 columns, one wave per 64 columns, no
    // LDS (layers with 16-32 output channels and many pixels)
    {16, 256, 16, "thin16x256", conv_thin_f32<1>, conv_thin_f32<1>, conv_thin_f32<1>, 1.0, 0, 1},
    {32, 256, 16, "thin32x256", conv_thin_f32<2>, conv_thin_f32<2>, conv_thin_f32<2>, 1.0, 0, 2},
    // 96-row tiles, the four waves side by side along n, each three 32x32
    // blocks: 65-96 output channels (YOLO's 80-class head) in one m-tile
    CFGW(96, 128, 16, 1, 4, 0.90), CFGW(96, 128, 32, 1, 4, 0.90),
    // row-window tiles: the skinny tiles' arithmetic (the same bits as
    // entries 12 and 13), one output row segment per workgroup, the input
    // window in LDS (kernel: the eight-chunk ring; the launch picks a
    // shallower one by the chunks per wave, window_kernel)
    {16, 16, 64, "win16x16w4", conv_window_f32<4, 8, 3>, conv_window_f32<4, 8, 3>, conv_window_f32<4, 8, 3>, 1.0, 4, 0,
     true},
    {16, 16, 64, "win16x16w8", conv_window_f32<8, 4, 3>, conv_window_f32<8, 4, 3>, conv_window_f32<8, 4, 3>, 1.0, 8, 0,
     true},
    // sixteen waves (four per SIMD, 128 registers each): the skinny tile and
    // its row-window form, the same bits as each other
    {16, 16, 64, "skinny16x16w16", conv_skinny_f32<16, 2>, conv_skinny_f32<16, 2>, conv_skinny_f32<16, 2>, 1.0, 16},
    {16, 16, 64, "win16x16w16", conv_window_f32<16, 2, 3>, conv_window_f32<16, 2, 3>, conv_window_f32<16, 2, 3>, 1.0,
     16, 0, true},
    // the four waves stacked along M (each 32 rows by the whole tile
    // width): every weight fragment is loaded by one wave only
    CFGWL(128, 64, 16, 4, 1, 0.95), CFGWL(128, 64, 32, 4, 1, 0.95),
};
#undef CFG
#undef CFGW
#undef CFGWL
constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

// threads per workgroup of configuration c
int cfg_threads(int c) { return kCfgs[c].skinny_waves > 0 ? 64 * kCfgs[c].skinny_waves : 256; }

// The row-window kernel of W waves for k_tiles 64-k chunks and KH (1 or 3)
// window rows per channel: a ring of weight chunks no deeper than the
// busiest wave's chunks
template <int KH>
IgemmKernel window_kernel_kh(int W, int per_wave) {
    if (W == 4)
        return per_wave <= 2 ? conv_window_f32<4, 2, KH> : per_wave <= 4 ? conv_window_f32<4, 4, KH>
                                                                        : conv_window_f32<4, 8, KH>;
    // eight waves: two per SIMD, 256 registers each, room for a ring of four;
    // sixteen: 128 registers, a ring of two
    if (W == 8) return per_wave <= 2 ? conv_window_f32<8, 2, KH> : conv_window_f32<8, 4, KH>;
    return conv_window_f32<16, 2, KH>;
}
IgemmKernel window_kernel(int W, int k_tiles, int KH) {
    const int per_wave = (k_tiles + W - 1) / W;
    return KH == 1 ? window_kernel_kh<1>(W, per_wave) : window_kernel_kh<3>(W, per_wave);
}

// The skinny kernel of W waves for k_tiles 64-k chunks: chunks in flight
// per wave no more than the busiest wave has
IgemmKernel skinny_kernel(int W, int k_tiles) {
    const int per_wave = (k_tiles + W - 1) / W;
    if (W == 4) return per_wave <= 1 ? conv_skinny_f32<4, 1> : per_wave <= 2 ? conv_skinny_f32<4, 2> : conv_skinny_f32<4, 4>;
    if (W == 8) return per_wave <= 1 ? conv_skinny_f32<8, 1> : per_wave <= 2 ? conv_skinny_f32<8, 2> : conv_skinny_f32<8, 4>;
    // sixteen waves (128 registers): groups of at most two chunks
    return per_wave <= 1 ? conv_skinny_f32<16, 1> : conv_skinny_f32<16, 2>;
}

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

// Workgroups of configuration c one CU holds at once; 0 when its kernels
// cannot launch on this device (e.g. more LDS than a workgroup may have),
// which takes the configuration out of every choice.
int resident_wgs(int c) {
    static int cache[kNumCfgs] = {0};
    static bool known[kNumCfgs] = {false};
    if (!known[c]) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void *>(kCfgs[c].kernel),
                                                         cfg_threads(c), 0) != hipSuccess ||
            n < 1) {
            (void)hipGetLastError();
            n = 0;
        }
        cache[c] = n;
        known[c] = true;
    }
    return cache[c];
}

// Tile counts of configuration c for an (M, Ntot, K) problem with split-K
// request `split`, as a plan stores them.
struct TileCounts {
    int m_tiles, n_tiles, k_tiles, kt_per_split, splitk;
    // hybrid: dp_tiles whole tiles (n-tile columns below ws_n0), the rest cut
    // into splitk slices of kt_per_split k-tiles; 0 otherwise
    int dp_tiles = 0, ws_n0 = 0;
};

// Split requests at or above kHybrid ask for the hybrid schedule with
// (split - kHybrid) k slices per remaining tile.
constexpr int kHybrid = 1000;

TileCounts tile_counts(int c, int M, int Ntot, int K, int split) {
    const TileCfg &t = kCfgs[c];
    TileCounts tc;
    tc.m_tiles = (M + t.BM - 1) / t.BM;
    tc.n_tiles = (Ntot + t.BN - 1) / t.BN;
    tc.k_tiles = (K + t.BK - 1) / t.BK;
    const bool whole = t.skinny_waves > 0 || t.thin_mb > 0;  // skinny, thin: no split-K
    const int req = whole ? 1 : split >= kHybrid ? split - kHybrid : split;
    tc.kt_per_split = (tc.k_tiles + req - 1) / req;
    tc.splitk = (tc.k_tiles + tc.kt_per_split - 1) / tc.kt_per_split;
    if (split >= kHybrid && !whole) {
        // whole tiles: the largest multiple of the CU count that is whole
        // n-tile columns (so the remaining tiles are the last columns)
        const int tiles = tc.m_tiles * tc.n_tiles;
        const int cus = device_cu_count();
        const int dp_n = (tiles / cus) * cus / tc.m_tiles;
        if (dp_n <= 0 || dp_n >= tc.n_tiles || tc.splitk <= 1) {
            tc.kt_per_split = tc.k_tiles;  // no hybrid for this shape: one whole-tile launch
            tc.splitk = 1;
        } else {
            tc.dp_tiles = dp_n * tc.m_tiles;
            tc.ws_n0 = dp_n * t.BN;
        }
    }
    return tc;
}

size_t partial_bytes_of(const TileCounts &tc, int M, int Ntot) {
    return tc.splitk > 1 ? static_cast<size_t>(tc.splitk) * M * (Ntot - tc.ws_n0) * sizeof(float) : 0;
}

// Modelled time (us) of a candidate: the MFMA work of the busiest CU over
// the rounds of resident workgroups, floored by the serial latency of one
// workgroup's k loop (a k-tile step costs ~35 ns per k when a workgroup
// runs alone on its CU), plus split-K partial traffic and the extra
// epilogue launch.  Used to prune the candidates the tuner times, and alone
// when tuning is off.
double model_us(int c, const TileCounts &tc, int M, int Ntot) {
    const TileCfg &t = kCfgs[c];
    const int cus = device_cu_count();
    if (t.skinny_waves > 0) {
        // a wave's chunks are 16 MFMAs of 32 cycles each; rounds of resident
        // workgroups; ~1 us of load latency per round
        const long wgs = static_cast<long>(tc.m_tiles) * tc.n_tiles;
        const long slots = static_cast<long>(cus) * resident_wgs(c);
        const long rounds = (wgs + slots - 1) / slots;
        const int chunks = (tc.k_tiles + t.skinny_waves - 1) / t.skinny_waves;
        return static_cast<double>(rounds) * (chunks * 16 * 32 / 2400.0 + 1.0) + 2.0;
    }
    if (t.thin_mb > 0) {
        // a wave's 16-k chunk is 16 * MB MFMAs of 32 cycles; the busiest
        // CU's waves per SIMD share its MFMA pipe; ~1 us of latency per round
        const long wgs = static_cast<long>(tc.m_tiles) * tc.n_tiles;
        const long slots = static_cast<long>(cus) * resident_wgs(c);
        const long rounds = (wgs + slots - 1) / slots;
        const long per_cu = std::min<long>(resident_wgs(c), (wgs + cus - 1) / cus);
        return static_cast<double>(rounds) * (per_cu * tc.k_tiles * 16.0 * t.thin_mb * 32 / 2400.0 + 1.0) + 2.0;
    }
    const long wgs = static_cast<long>(tc.m_tiles) * tc.n_tiles * tc.splitk;
    const long slots = static_cast<long>(cus) * resident_wgs(c);
    const long rounds = (wgs + slots - 1) / slots;
    const long per_cu = std::min<long>(resident_wgs(c), (wgs + cus - 1) / cus);
    const double tile_us = 2.0 * t.BM * t.BN * t.BK / (256.0 * 2400.0 * t.eff);  // one k-tile on a whole CU
    const double mfma = static_cast<double>(rounds) * per_cu * tc.kt_per_split * tile_us;
    const double latency = static_cast<double>(rounds) * tc.kt_per_split * t.BK * 0.035;
    double us = std::max(mfma, latency) + 2.0;
    if (tc.dp_tiles > 0) {
        // whole tiles spread evenly, then one slice's share of each remaining tile
        const long rem = static_cast<long>(tc.m_tiles) * tc.n_tiles - tc.dp_tiles;
        const double units = std::ceil(static_cast<double>(tc.dp_tiles) / cus) +
                             std::ceil(static_cast<double>(rem) * tc.splitk / cus) * tc.kt_per_split / tc.k_tiles;
        us = std::max(units * tc.k_tiles * tile_us, static_cast<double>(tc.k_tiles) * t.BK * 0.035) + 2.0;
    }
    if (tc.splitk > 1)
        us += 4.0 * M * static_cast<double>(Ntot - tc.ws_n0) * (tc.splitk + 1) / 4.0e6 + 3.0;
    return us;
}

// The order in which a candidate sums each output's products, as a key:
// candidates with equal keys give bit-identical fp32 results (up to the sign
// of an exact zero, which the zero-padded k tail may turn positive).  Every
// implicit-GEMM tile, whatever its BM, BN, BK and wave layout, feeds its MFMAs
// the k pairs (8q + s, 8q + 4 + s), s = 0..3, of each 8-k group in the same
// order, one group after the other, so its order depends only on where
// split-K cuts k (slices of kt_per_split * BK k, summed in slice order by the
// epilogue) and, for the hybrid schedule, on which columns are cut (ws_n0).
// The skinny and thin kernels sum in orders of their own (tap-major k, wave
// partials through LDS).
std::string numerics_class(int c, const TileCounts &tc) {
    const TileCfg &t = kCfgs[c];
    if (t.skinny_waves > 0) return "skinny" + std::to_string(t.skinny_waves);
    if (t.thin_mb > 0) return "thin" + std::to_string(c);
    if (tc.splitk <= 1) return "igemm";
    const std::string cut = "/" + std::to_string(tc.kt_per_split * t.BK);
    return tc.dp_tiles > 0 ? "hybrid" + std::to_string(tc.ws_n0) + cut : "splitk" + cut;
}

const int kSplits[] = {1, 2, 3, 4, 6, 8, 12, 16, 24, 32};

// Fewest k-tiles a split-K slice may hold: two for the shallow tiles (a
// slice of one 16- or 32-k tile is all pipeline fill), one for the deep ones.
int min_slice_tiles(int c) { return kCfgs[c].BK >= 64 ? 1 : 2; }
const int kHybridSplits[] = {2, 4, 8, 16};

// What the tuner needs to launch a candidate: the B source geometry and
// the k -> byte offset rule of the layer.
struct GatherSpec {
    int K;
    int Wp;            // row pitch of the B source
    int x_bytes;       // extent of the B source
    int x_img_stride;  // elements between images of the B source
    std::function<int(int)> koff;  // byte offset of k < K
    std::string key;   // everything the timing depends on
    GatherGeom gather;  // the same rule per tap (skinny kernel), 16-byte k loads (KVEC)
};

// The skinny kernel takes a layer whose channels per tap are a multiple of
// its 64-k chunk (so a chunk never straddles two taps).
bool skinny_fits(const GatherSpec &gs) { return gs.gather.C > 0 && gs.gather.C % 64 == 0; }

// The thin kernel takes a layer whose channels per tap are a multiple of
// its 4-k MFMA step.
bool thin_fits(const GatherSpec &gs) { return gs.gather.C > 0 && gs.gather.C % 4 == 0 && gs.K % 4 == 0; }

// The row-window kernel takes a skinny layer that is a convolution whose
// input window fits its LDS (win_len set at planning).
bool window_fits(const GatherSpec &gs) { return skinny_fits(gs) && gs.gather.win_len > 0; }

// Configuration c can run the layer.
bool cfg_fits(int c, const GatherSpec &gs) {
    return resident_wgs(c) > 0 && (kCfgs[c].skinny_waves == 0 || skinny_fits(gs)) &&
           (!kCfgs[c].window || window_fits(gs)) && (kCfgs[c].thin_mb == 0 || thin_fits(gs));
}

std::vector<int> build_koff(const GatherSpec &gs, int BK) {
    const int kpad = (gs.K + BK - 1) / BK * BK;
    // two extra tiles of out-of-range entries: the pipeline prefetches up to
    // two tiles past the last one
    std::vector<int> koff(static_cast<size_t>(kpad + 2 * BK), kOobOffset);
    for (int k = 0; k < gs.K; k++) koff[k] = gs.koff(k);
    return koff;
}

}  // namespace

// Launches the implicit GEMM of configuration cfg with tile counts tc over
// an already prepared (padded) B source, then the split-K epilogue.
// y's layout when it is a channel slice of a larger buffer (a Concat's):
// elements between images and the byte extent from y; 0 for the natural
// M x OH x OW images (the residual, when there is one, always has those).
struct YLayout {
    int img = 0;
    int bytes = 0;
    int cstride = 0;  // elements between channels; 0: OH x OW
};

static int launch_igemm(hipStream_t st, int cfg, const TileCounts &tc, const ConvGeom &g, int Wp, const float *xs,
                        int x_bytes, int x_img_stride, const float *wpack, const int *koff, const float *bias,
                        const float *res, float *y, float alpha, float *ws, const GatherGeom &gg,
                        const ConvPlan *handoff = nullptr, YLayout yl = YLayout{}) {
    const TileCfg &t = kCfgs[cfg];
    IgemmArgs a{};
    a.x = xs;
    a.x_bytes = x_bytes;
    a.x_img_stride = x_img_stride;
    a.wp = wpack;
    a.koff = koff;
    a.bias = bias;
    a.res = res;
    a.y = y;
    a.Wp = Wp;
    a.M = g.M;
    a.OW = g.OW;
    a.OHW = g.OH * g.OW;
    a.Ntot = g.N * a.OHW;
    a.sh = g.sh;
    a.sw = g.sw;
    a.m_tiles = tc.m_tiles;
    a.k_tiles = tc.k_tiles;
    a.kt_per_split = tc.kt_per_split;
    a.act = g.act;
    a.alpha = alpha;
    a.ws = tc.splitk > 1 ? ws : nullptr;
    a.ws_n0 = tc.ws_n0;
    a.ws_ld = a.Ntot - tc.ws_n0;
    a.dp_tiles = tc.dp_tiles;
    a.rem_split = tc.splitk;
    if (handoff) {
        a.yp = handoff->pad_out;
        a.yp_plane = handoff->pad_Hp * handoff->pad_Wp;
        a.yp_m0 = handoff->pad_C > 0 ? handoff->pad_m0 : 0;
        a.yp_C = handoff->pad_C > 0 ? handoff->pad_C : g.M;
        a.yp_bytes = static_cast<int>(static_cast<size_t>(g.N) * a.yp_C * a.yp_plane * 4);
        a.yp_Wp = handoff->pad_Wp;
        a.yp_pt = handoff->pad_pt;
        a.yp_pl = handoff->pad_pl;
    }
    a.y_bytes = yl.bytes > 0 ? yl.bytes : static_cast<int>(g.y_elems * 4);
    a.y_img_stride = yl.img > 0 ? yl.img : g.M * a.OHW;
    a.y_cstride = yl.cstride > 0 ? yl.cstride : a.OHW;
    a.ws_bytes = static_cast<int>(partial_bytes_of(tc, g.M, a.Ntot));
    const int tiles = tc.m_tiles * tc.n_tiles;
    if (t.skinny_waves > 0) {
        // the kernel's chunks never straddle taps: checked here as well as
        // at planning, since a chunk past its tap would read other channels
        if (gg.C <= 0 || gg.C % 64 != 0 || tc.k_tiles * 64 != gg.C * (g.KH * g.KW)) {
            set_last_error_text("conv_skinny_f32: layer without whole 64-channel chunks per tap");
            return SPKV2_E_UNSUPPORTED;
        }
        // the packed weights are addressed with 32-bit buffer offsets
        if (static_cast<long long>(tc.m_tiles) * tc.k_tiles * 4096 >= kOobOffset) {
            set_last_error_text("conv_skinny_f32: packed weights of 2 GiB or more");
            return SPKV2_E_UNSUPPORTED;
        }
        a.sk_C = gg.C;
        a.sk_cstride = gg.cstride;
        a.sk_KW = gg.KW;
        a.sk_tap_h = gg.tap_h;
        a.sk_tap_w = gg.tap_w;
        a.ws = nullptr;
        if (t.window) {
            // the window's rows and columns: checked here as well as at
            // planning, since the kernel's LDS holds kWinFloats floats
            if (gg.win_len <= 0 || gg.win_len > 64 || (1 << gg.win_shift) < gg.win_len || gg.win_shift > 6 ||
                (gg.win_KH != 1 && gg.win_KH != 3) ||
                static_cast<long long>(gg.C + 4) * gg.win_KH * gg.win_len > kWinFloats ||
                gg.win_KH != g.KH || gg.win_rows != g.N * g.OH || gg.win_owb != (g.OW + 15) / 16) {
                set_last_error_text("conv_window_f32: layer without a row window that fits the kernel's LDS");
                return SPKV2_E_UNSUPPORTED;
            }
            a.win_KH = gg.win_KH;
            a.win_len = gg.win_len;
            a.win_shift = gg.win_shift;
            a.win_owb = gg.win_owb;
            a.win_OH = g.OH;
            a.win_dw = gg.win_dw;
            const long long wgs = static_cast<long long>(tc.m_tiles) * gg.win_rows * gg.win_owb;
            if (wgs >= (1LL << 31)) return SPKV2_E_UNSUPPORTED;
            const size_t lds = static_cast<size_t>(gg.C + 4) * gg.win_KH * gg.win_len * 4;
            window_kernel(t.skinny_waves, tc.k_tiles, gg.win_KH)<<<dim3(static_cast<unsigned>(wgs)),
                                                                    dim3(64 * t.skinny_waves), lds, st>>>(a);
            return launch_status("conv_window_f32");
        }
        skinny_kernel(t.skinny_waves, tc.k_tiles)<<<dim3(static_cast<unsigned>(tiles)), dim3(64 * t.skinny_waves), 0,
                                                    st>>>(a);
        return launch_status("conv_skinny_f32");
    }
    if (t.thin_mb > 0) {
        // k' = tap * C + c in whole 4-channel steps: checked here as well as
        // at planning, since a step past its tap would read other channels
        const int K = gg.C * g.KH * g.KW;
        if (gg.C <= 0 || gg.C % 4 != 0 || gg.chk || tc.k_tiles * 16 < K || tc.k_tiles * 16 >= K + 16) {
            set_last_error_text("conv_thin_f32: layer without whole 4-channel steps per tap");
            return SPKV2_E_UNSUPPORTED;
        }
        a.sk_C = gg.C;
        a.sk_cstride = gg.cstride;
        a.sk_KW = gg.KW;
        a.sk_tap_h = gg.tap_h;
        a.sk_tap_w = gg.tap_w;
        a.th_steps = K / 4;
        a.ws = nullptr;
        t.kernel<<<dim3(static_cast<unsigned>(tiles)), dim3(256), 0, st>>>(a);
        return launch_status("conv_thin_f32");
    }
    const dim3 grid = tc.dp_tiles > 0
                          ? dim3(static_cast<unsigned>(tc.dp_tiles + (tiles - tc.dp_tiles) * tc.splitk), 1)
                          : dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(tc.splitk));
    a.ktap = gg.ktap;
    a.chk_H = gg.chk_H;
    a.chk_W = gg.chk_W;
    a.chk_ph = gg.chk_ph;
    a.chk_pw = gg.chk_pw;
    // 16-byte B loads need a 16-byte aligned source (a caller-bound input may not be)
    const bool kvec = gg.kvec && (reinterpret_cast<uintptr_t>(xs) & 15) == 0;
    (kvec ? t.kernel_kvec : gg.chk ? t.kernel_chk : t.kernel)<<<grid, dim3(256), 0, st>>>(a);
    if (int rc = launch_status("conv_igemm_f32")) return rc;
    if (tc.splitk > 1) {
        const size_t total = static_cast<size_t>(g.M) * a.ws_ld;
        // four columns per thread where that still gives every CU a
        // workgroup; small (batch-1) outputs take one column per thread, so
        // the partial loads spread over more CUs
        if (a.ws_ld % 4 == 0 && a.ws_n0 % 4 == 0 && total / 4 >= 256u * 256u)
            hipLaunchKernelGGL(splitk_epilogue<4>, dim3(grid_for(total / 4, 256)), dim3(256), 0, st, ws, tc.splitk,
                               g.M, a.ws_ld, a.OHW, bias, res, y, g.act, alpha, a);
        else
            hipLaunchKernelGGL(splitk_epilogue<1>, dim3(grid_for(total, 256)), dim3(256), 0, st, ws, tc.splitk, g.M,
                               a.ws_ld, a.OHW, bias, res, y, g.act, alpha, a);
        if (int rc = launch_status("splitk_epilogue")) return rc;
    }
    return 0;
}

namespace {

std::mutex g_tune_mu;
std::map<std::string, std::pair<int, int>> g_tuned;  // key -> (cfg, split request), fp32 and int8 layers
bool g_tune_db_loaded = false;

// Tune tables are text files of "key cfg split" lines.  mi355x.tune beside
// the library holds the choices for the benchmark networks' layer shapes
// (read-only), so every process picks the same tiles and split-K for them
// and their fp32 results are bit-reproducible across processes.
// SPKV2_TUNE_DB names a file of the caller's: read after it (its entries
// win), and every newly tuned shape is appended, so later processes reuse
// those choices without timing again.
const char *tune_db_path() {
    const char *p = getenv("SPKV2_TUNE_DB");
    return p && p[0] ? p : nullptr;
}

void load_tune_file_locked(const char *path) {
    FILE *f = fopen(path, "r");
    if (!f) return;
    char key[512];
    int cfg = 0, split = 0;
    // split: 1..64, or a hybrid request (1000 + slices per remaining tile)
    while (fscanf(f, "%511s %d %d", key, &cfg, &split) == 3)
        if (cfg >= 0 && cfg < 64 && ((split >= 1 && split <= 64) || (split >= 1002 && split <= 1064)))
            g_tuned[key] = {cfg, split};
    fclose(f);
}

void load_tune_db_locked() {
    if (g_tune_db_loaded) return;
    g_tune_db_loaded = true;
    const char *use_table = getenv("SPKV2_TUNE_TABLE");  // "0": ignore the built-in table (to regenerate it)
    Dl_info info;
    if (!(use_table && use_table[0] == '0') && dladdr(reinterpret_cast<void *>(&load_tune_file_locked), &info) &&
        info.dli_fname) {
        std::string dir(info.dli_fname);
        const size_t slash = dir.rfind('/');
        dir = slash == std::string::npos ? std::string(".") : dir.substr(0, slash);
        load_tune_file_locked((dir + "/mi355x.tune").c_str());
    }
    if (const char *path = tune_db_path()) load_tune_file_locked(path);
}

void store_tune_db_locked(const std::string &key, int cfg, int split) {
    const char *path = tune_db_path();
    if (!path) return;
    if (FILE *f = fopen(path, "a")) {
        fprintf(f, "%s %d %d\n", key.c_str(), cfg, split);
        fclose(f);
    }
}

}  // namespace

bool tuned_lookup(const std::string &key, int *cfg, int *split) {
    std::lock_guard<std::mutex> lk(g_tune_mu);
    load_tune_db_locked();
    auto it = g_tuned.find(key);
    if (it == g_tuned.end()) return false;
    *cfg = it->second.first;
    *split = it->second.second;
    return true;
}

void tuned_store(const std::string &key, int cfg, int split) {
    std::lock_guard<std::mutex> lk(g_tune_mu);
    g_tuned[key] = {cfg, split};
    store_tune_db_locked(key, cfg, split);
}

namespace {

// Device buffers of one tuning session, freed on scope exit.
struct TuneBuffers {
    std::vector<void *> ptrs;
    void *alloc(size_t bytes) {
        void *p = nullptr;
        if (hipMalloc(&p, bytes ? bytes : 16) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        ptrs.push_back(p);
        return p;
    }
    ~TuneBuffers() {
        for (void *p : ptrs) (void)hipFree(p);
    }
};

// Times every candidate (configuration x split-K) the model does not rule
// out on scratch buffers of the layer's real shape, and returns the fastest
// (cfg, split request).  Results are cached per shape for the process, so
// every context sees the same choice for the same layer.  Returns false
// when the device could not be used (the caller then trusts the model).
bool tune_tiles(hipStream_t st, const ConvGeom &g, const GatherSpec &gs, int *cfg_out, int *split_out) {
    if (tuned_lookup(gs.key, cfg_out, split_out) && *cfg_out >= 0 && *cfg_out < kNumCfgs && cfg_fits(*cfg_out, gs))
        return true;
    const int Ntot = g.N * g.OH * g.OW;
    struct Cand {
        int cfg, split;
        TileCounts tc;
        double model, t;
    };
    std::vector<Cand> cands;
    double best_model = 1e300;
    for (int c = 0; c < kNumCfgs; c++) {
        if (!cfg_fits(c, gs)) continue;
        int last_splitk = -1;
        for (int split : kSplits) {
            const TileCounts tc = tile_counts(c, g.M, Ntot, gs.K, split);
            if (tc.splitk == last_splitk) continue;
            if (split > 1 && tc.kt_per_split < min_slice_tiles(c)) break;
            last_splitk = tc.splitk;
            if (partial_bytes_of(tc, g.M, Ntot) > (size_t(1) << 29)) continue;
            const double m = model_us(c, tc, g.M, Ntot);
            best_model = std::min(best_model, m);
            cands.push_back({c, split, tc, m, 0.0});
        }
        for (int rs : kHybridSplits) {
            const TileCounts tc = tile_counts(c, g.M, Ntot, gs.K, kHybrid + rs);
            if (tc.dp_tiles == 0 || tc.kt_per_split < min_slice_tiles(c)) continue;
            if (partial_bytes_of(tc, g.M, Ntot) > (size_t(1) << 29)) continue;
            const double m = model_us(c, tc, g.M, Ntot);
            best_model = std::min(best_model, m);
            cands.push_back({c, kHybrid + rs, tc, m, 0.0});
        }
    }
    if (cands.empty()) return false;
    // SPKV2_TUNE_DETERMINISTIC=1: the model picks the summation order -- the
    // class of its best candidate -- and timing only picks among the
    // candidates of that class, which all give the same fp32 bits, so no
    // measurement noise can change a result (at some speed: the model's
    // order is not always the fastest one).  By default every candidate
    // within 3x of the model's best is timed.
    const char *det_env = getenv("SPKV2_TUNE_DETERMINISTIC");
    const bool deterministic = det_env && det_env[0] == '1';
    // the model's best implicit-GEMM candidate (its estimates of the skinny
    // and thin kernels are too rough to choose between orders)
    auto igemm_family = [](int c) { return kCfgs[c].skinny_waves == 0 && kCfgs[c].thin_mb == 0; };
    size_t mb = cands.size();
    for (size_t i = 0; i < cands.size(); i++)
        if (igemm_family(cands[i].cfg) && (mb == cands.size() || cands[i].model < cands[mb].model)) mb = i;
    if (mb == cands.size()) mb = 0;
    // when timing fails: the model's own choice in the deterministic mode
    // (the caller's split-only model otherwise)
    auto untimed = [&]() {
        *cfg_out = cands[mb].cfg;
        *split_out = cands[mb].split;
        return deterministic;
    };
    std::vector<Cand> keep;
    if (deterministic) {
        const std::string cls = numerics_class(cands[mb].cfg, cands[mb].tc);
        for (const Cand &cd : cands)
            if (numerics_class(cd.cfg, cd.tc) == cls) keep.push_back(cd);
    } else {
        for (const Cand &cd : cands)
            if (cd.model <= 3.0 * best_model) keep.push_back(cd);
    }
    if (keep.empty()) return false;

    TuneBuffers tb;
    size_t wpack_bytes = 0, ws_bytes = 16;
    for (const Cand &cd : keep) {
        const TileCfg &t = kCfgs[cd.cfg];
        wpack_bytes = std::max(wpack_bytes, static_cast<size_t>(cd.tc.m_tiles) * cd.tc.k_tiles * t.BM * t.BK * 4);
        ws_bytes = std::max(ws_bytes, partial_bytes_of(cd.tc, g.M, Ntot));
    }
    const size_t y_bytes = static_cast<size_t>(g.y_elems) * 4;
    float *xs = static_cast<float *>(tb.alloc(gs.x_bytes));
    float *wp = static_cast<float *>(tb.alloc(wpack_bytes));
    float *y = static_cast<float *>(tb.alloc(y_bytes));
    float *ws = static_cast<float *>(tb.alloc(ws_bytes));
    float *bias = g.has_bias ? static_cast<float *>(tb.alloc(static_cast<size_t>(g.M) * 4)) : nullptr;
    float *res = g.has_res ? static_cast<float *>(tb.alloc(y_bytes)) : nullptr;
    int *koff[4] = {nullptr, nullptr, nullptr, nullptr};  // BK 16, 32, 64, 128
    for (int i = 0; i < 4; i++) {
        const std::vector<int> kv = build_koff(gs, 16 << i);
        koff[i] = static_cast<int *>(tb.alloc(kv.size() * sizeof(int)));
        if (koff[i] && hipMemcpy(koff[i], kv.data(), kv.size() * sizeof(int), hipMemcpyHostToDevice) != hipSuccess)
            koff[i] = nullptr;
    }
    if (!xs || !wp || !y || !ws || (g.has_bias && !bias) || (g.has_res && !res) || !koff[0] || !koff[1] || !koff[2] || !koff[3])
        return untimed();
    // operands of zeros: the timing does not depend on the values
    (void)hipMemsetAsync(xs, 0, gs.x_bytes, st);
    (void)hipMemsetAsync(wp, 0, wpack_bytes, st);
    if (bias) (void)hipMemsetAsync(bias, 0, static_cast<size_t>(g.M) * 4, st);
    if (res) (void)hipMemsetAsync(res, 0, y_bytes, st);

    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
        (void)hipGetLastError();
        return untimed();
    }
    auto time_it = [&](const Cand &cd, int reps) -> double {
        const int bk = kCfgs[cd.cfg].BK;
        const int *ko = koff[bk == 16 ? 0 : bk == 32 ? 1 : bk == 64 ? 2 : 3];
        if (hipEventRecord(e0, st) != hipSuccess) return 1e300;
        for (int r = 0; r < reps; r++)
            if (launch_igemm(st, cd.cfg, cd.tc, g, gs.Wp, xs, gs.x_bytes, gs.x_img_stride, wp, ko, bias, res, y, 1.0f,
                             ws, gs.gather) != 0)
                return 1e300;
        if (hipEventRecord(e1, st) != hipSuccess || hipEventSynchronize(e1) != hipSuccess) return 1e300;
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, e0, e1) != hipSuccess) return 1e300;
        return 1e3 * ms / reps;
    };
    // Each timing covers about 100 us of back-to-back launches (1 to 20 of
    // them): a batch-1 candidate runs for a few microseconds, where one
    // launch's time is mostly event and launch noise.
    auto reps_for = [](double t) { return std::max(1, std::min(20, static_cast<int>(100.0 / std::max(t, 1.0)))); };
    bool ok = true;
    for (Cand &cd : keep) {
        const double t1 = time_it(cd, 1);  // also the warm-up (first launch of a kernel variant)
        cd.t = t1 >= 1e300 ? t1 : time_it(cd, reps_for(t1));
        if (cd.t >= 1e300) ok = false;
    }
    std::sort(keep.begin(), keep.end(), [](const Cand &a, const Cand &b) { return a.t < b.t; });
    const size_t finalists = std::min<size_t>(keep.size(), 4);
    for (size_t i = 0; i < finalists && ok; i++) {
        const double t = time_it(keep[i], 3 * reps_for(keep[i].t));
        keep[i].t = std::min(keep[i].t, t);
    }
    std::sort(keep.begin(), keep.begin() + finalists, [](const Cand &a, const Cand &b) { return a.t < b.t; });
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (!ok || hipStreamSynchronize(st) != hipSuccess) {
        (void)hipGetLastError();
        return untimed();
    }
    // timings within the tie band of the fastest (5%, SPKV2_TUNE_TIE in
    // percent) are a tie, broken by the model (then the candidate order), not
    // by the noise of this process's measurement: two processes then pick
    // the same configuration, and so give the same fp32 bits (its k order),
    // unless two candidates' times straddle the band's edge
    double tie = 1.05;
    if (const char *e = getenv("SPKV2_TUNE_TIE")) tie = 1.0 + std::max(0.0, std::min(50.0, atof(e))) / 100.0;
    size_t pick = 0;
    for (size_t i = 1; i < finalists; i++)
        if (keep[i].t <= keep[0].t * tie &&
            (keep[i].model < keep[pick].model ||
             (keep[i].model == keep[pick].model &&
              std::make_pair(keep[i].cfg, keep[i].split) < std::make_pair(keep[pick].cfg, keep[pick].split))))
            pick = i;
    *cfg_out = keep[pick].cfg;
    *split_out = keep[pick].split;
    tuned_store(gs.key, keep[pick].cfg, keep[pick].split);
    if (const char *e = getenv("SPKV2_TUNE_LOG"))
        if (e[0] == '1') {
            // every timed candidate, fastest first: config, split request,
            // model estimate and measured time (us)
            fprintf(stderr, "[tune] %s -> cfg %d split %d\n", gs.key.c_str(), keep[pick].cfg, keep[pick].split);
            for (const Cand &cd : keep)
                fprintf(stderr, "[tune]   %-10s split %4d splitk %2d  model %7.2f  time %7.2f\n", kCfgs[cd.cfg].name,
                        cd.split, cd.tc.splitk, cd.model, cd.t);
        }
    return true;
}

// Picks (cfg, split) for a layer: SPKV2_CONV_CFG / SPKV2_CONV_SPLITK /
// SPKV2_CONV_HYBRID (slices per remaining tile) force a choice; otherwise
// the tuner measures unless SPKV2_CONV_TUNE=0, and the model decides when it
// does not.
void choose_tiles(hipStream_t st, const ConvGeom &g, const GatherSpec &gs, int *cfg_out, int *split_out) {
    const int Ntot = g.N * g.OH * g.OW;
    int best_cfg = 0, best_split = 1;
    const char *tune_env = getenv("SPKV2_CONV_TUNE");
    const bool tune = !(tune_env && tune_env[0] == '0');
    if (!(tune && tune_tiles(st, g, gs, &best_cfg, &best_split))) {
        double best = 1e300;
        for (int c = 0; c < kNumCfgs; c++) {
            if (!cfg_fits(c, gs)) continue;
            for (int split : kSplits) {
                const TileCounts tc = tile_counts(c, g.M, Ntot, gs.K, split);
                if (split > 1 && tc.kt_per_split < min_slice_tiles(c)) break;
                if (partial_bytes_of(tc, g.M, Ntot) > (size_t(1) << 29)) continue;
                const double m = model_us(c, tc, g.M, Ntot);
                if (m < best * 0.999) {
                    best = m;
                    best_cfg = c;
                    best_split = split;
                }
            }
        }
    }
    if (const char *e = getenv("SPKV2_CONV_CFG")) {
        const int c = atoi(e);
        if (c >= 0 && c < kNumCfgs && cfg_fits(c, gs)) best_cfg = c;
    }
    if (const char *e = getenv("SPKV2_CONV_SPLITK")) {
        const int sk = atoi(e);
        if (sk >= 1 && sk <= 64) best_split = sk;
    }
    if (const char *e = getenv("SPKV2_CONV_HYBRID")) {
        const int rs = atoi(e);
        if (rs >= 2 && rs <= 64) best_split = kHybrid + rs;
    }
    *cfg_out = best_cfg;
    *split_out = best_split;
}

// Packs A[m][k] (row-major, lda = K) into BM x BK tiles [m_tiles][k_tiles],
// each laid out in MFMA fragment order [BM/32][BK/8][64 lanes][4]: lane l of
// fragment (b, q) holds row b*32 + (l & 31), k = q*8 + 4*(l >> 5) + 0..3 --
// the A operand of the four 32x32x2 steps of that 8-k slice, one 16-byte
// load per lane.  Ragged edges are zero-filled.
int upload_packed_f32(const float *w, int M, int K, int BM, int BK, int m_tiles, int k_tiles, void **out) {
    std::vector<float> packed(static_cast<size_t>(m_tiles) * k_tiles * BM * BK, 0.0f);
    const int K8 = BK / 8;
    for (int mt = 0; mt < m_tiles; mt++)
        for (int kt = 0; kt < k_tiles; kt++) {
            float *dst = packed.data() + (static_cast<size_t>(mt) * k_tiles + kt) * BM * BK;
            for (int i = 0; i < BM; i++) {
                const int m = mt * BM + i;
                if (m >= M) break;
                for (int kk = 0; kk < BK; kk++) {
                    const int k = kt * BK + kk;
                    if (k >= K) break;
                    const int lane = ((kk % 8) / 4) * 32 + i % 32;
                    dst[((static_cast<size_t>(i / 32) * K8 + kk / 8) * 64 + lane) * 4 + kk % 4] =
                        w[static_cast<size_t>(m) * K + k];
                }
            }
        }
    const size_t bytes = packed.size() * sizeof(float);
    if (int rc = hip_check(hipMalloc(out, bytes), "hipMalloc packed weights")) return rc;
    return hip_check(hipMemcpy(*out, packed.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy packed weights");
}

// Packs w[m][c][tap] (k = c * taps + tap, the reference's order) for the
// skinny kernel: k' = tap * C + c in chunks of 64, tile [m_tiles][KC][4 slots
// g][16 rows][16 t] holding row m, k' = 64 * chunk + 16g + t -- lane (g, row)
// of MFMA t reads element t of its 64-byte run.  Rows past M are zero.
int upload_packed_skinny(const float *w, int M, int C, int taps, int m_tiles, int KC, void **out) {
    std::vector<float> packed(static_cast<size_t>(m_tiles) * KC * 1024, 0.0f);
    for (int m = 0; m < M; m++) {
        const int mt = m / 16, ml = m % 16;
        for (int kp = 0; kp < KC * 64; kp++) {
            const int tap = kp / C, c = kp % C;
            const int kc = kp / 64, g = (kp % 64) / 16, t = kp % 16;
            packed[(static_cast<size_t>(mt) * KC + kc) * 1024 + (g * 16 + ml) * 16 + t] =
                w[(static_cast<size_t>(m) * C + c) * taps + tap];
        }
    }
    const size_t bytes = packed.size() * sizeof(float);
    if (int rc = hip_check(hipMalloc(out, bytes), "hipMalloc packed weights")) return rc;
    return hip_check(hipMemcpy(*out, packed.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy packed weights");
}

// Packs w[m][c][tap] (k = c * taps + tap, the reference's order) for the
// thin kernel: k' = tap * C + c, tile [m_tiles][k_tiles][MB][64 lanes][4
// steps] holding, for lane (g, r) of 16-row block b, row 16b + r at
// k' = 16 kt + 4 step + g.  Rows past M and k' past K are zero.
int upload_packed_thin(const float *w, int M, int C, int taps, int MB, int m_tiles, int k_tiles, void **out) {
    std::vector<float> packed(static_cast<size_t>(m_tiles) * k_tiles * MB * 256, 0.0f);
    const int K = C * taps;
    for (int m = 0; m < M; m++) {
        const int mt = m / (16 * MB), b = (m % (16 * MB)) / 16, r = m % 16;
        for (int kp = 0; kp < K; kp++) {
            const int tap = kp / C, c = kp % C;
            const int kt = kp / 16, st = (kp % 16) / 4, g = kp % 4;
            packed[(((static_cast<size_t>(mt) * k_tiles + kt) * MB + b) * 64 + g * 16 + r) * 4 + st] =
                w[(static_cast<size_t>(m) * C + c) * taps + tap];
        }
    }
    const size_t bytes = packed.size() * sizeof(float);
    if (int rc = hip_check(hipMalloc(out, bytes), "hipMalloc packed weights")) return rc;
    return hip_check(hipMemcpy(*out, packed.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy packed weights");
}

int upload_koff(const std::vector<int> &koff, void **out) {
    const size_t bytes = koff.size() * sizeof(int);
    if (int rc = hip_check(hipMalloc(out, bytes), "hipMalloc koff")) return rc;
    return hip_check(hipMemcpy(*out, koff.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy koff");
}

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

}  // namespace

static TileCounts plan_counts(const ConvPlan *p) {
    return TileCounts{p->m_tiles, p->n_tiles, p->k_tiles, p->kt_per_split, p->splitk, p->dp_tiles, p->ws_n0};
}

static size_t partial_bytes(const ConvPlan *p) {
    return partial_bytes_of(plan_counts(p), p->g.M, p->g.N * p->g.OH * p->g.OW);
}

// Chooses tiles and split-K for the layer, packs and uploads its weights and
// k-offset table.
static int plan_tiles_and_weights(hipStream_t st, const ConvGeom &g, const GatherSpec &gs, const float *w_host,
                                  ConvPlan *plan) {
    const int Ntot = g.N * g.OH * g.OW;
    int cfg = 0, split = 1;
    choose_tiles(st, g, gs, &cfg, &split);
    const TileCfg &t = kCfgs[cfg];
    const TileCounts tc = tile_counts(cfg, g.M, Ntot, gs.K, split);
    plan->path = CONV_IGEMM_F32;
    plan->cfg = cfg;
    plan->BM = t.BM;
    plan->BN = t.BN;
    plan->BK = t.BK;
    plan->K = gs.K;
    plan->m_tiles = tc.m_tiles;
    plan->n_tiles = tc.n_tiles;
    plan->k_tiles = tc.k_tiles;
    plan->Kpad = tc.k_tiles * t.BK;
    plan->kt_per_split = tc.kt_per_split;
    plan->splitk = tc.splitk;
    plan->dp_tiles = tc.dp_tiles;
    plan->ws_n0 = tc.ws_n0;
    if (partial_bytes(plan) >= 0x7fff0000ULL) return SPKV2_E_UNSUPPORTED;
    plan->gather = gs.gather;
    if (t.skinny_waves > 0) {
        if (int rc = upload_packed_skinny(w_host, g.M, gs.gather.C, gs.K / gs.gather.C, plan->m_tiles, plan->k_tiles,
                                          &plan->wpack))
            return rc;
    } else if (t.thin_mb > 0) {
        if (int rc = upload_packed_thin(w_host, g.M, gs.gather.C, gs.K / gs.gather.C, t.thin_mb, plan->m_tiles,
                                        plan->k_tiles, &plan->wpack))
            return rc;
    } else if (int rc = upload_packed_f32(w_host, g.M, gs.K, t.BM, t.BK, plan->m_tiles, plan->k_tiles, &plan->wpack)) {
        return rc;
    }
    return upload_koff(build_koff(gs, t.BK), &plan->ktab);
}

static std::string shape_key(const char *kind, const ConvGeom &g, const ConvPlan *p, int x_img_stride) {
    char buf[256];
    snprintf(buf, sizeof(buf), "%s|%d,%d,%d,%d|%d,%d,%d,%d,%d,%d,%d,%d|%d,%d,%d|%d,%d,%d,%d", kind, g.N, g.C, g.H, g.W,
             g.M, g.KH, g.KW, g.OH, g.OW, g.sh, g.sw, g.dh, g.dw, p->Hp, p->Wp, x_img_stride, g.has_bias ? 1 : 0,
             g.has_res ? 1 : 0, g.act);
    return buf;
}

// Rows and columns of the zero-padded input conv g reads, from the top /
// left padding on (its taps' span, at least the input's), when it needs one.
static bool padded_extent(const ConvGeom &g, int *Hp, int *Wp) {
    const int hspan = (g.OH - 1) * g.sh + (g.KH - 1) * g.dh + 1;  // rows the taps touch, from -ph
    const int wspan = (g.OW - 1) * g.sw + (g.KW - 1) * g.dw + 1;
    *Hp = std::max(g.H + g.ph, hspan);
    *Wp = std::max(g.W + g.pw, wspan);
    return g.ph > 0 || g.pw > 0 || hspan - g.ph > g.H || wspan - g.pw > g.W;
}

// Plans an fp32 implicit GEMM for convolution g (group 1) with weights
// w_host[M][C*KH*KW].  When some tap falls outside the input, the input is
// first copied into a zero-padded buffer so the kernel needs no bounds tests;
// min_Hp / min_Wp enlarge that buffer's planes (a geometry shared with the
// other padded readers of the same input).
int plan_igemm_f32(hipStream_t st, const ConvGeom &g, const float *w_host, ConvPlan *plan, int min_Hp = 0,
                   int min_Wp = 0) {
    const int K = g.C * g.KH * g.KW;
    int ext_h = 0, ext_w = 0;
    plan->padded = padded_extent(g, &ext_h, &ext_w);
    plan->pt = plan->padded ? g.ph : 0;
    plan->pl = plan->padded ? g.pw : 0;
    plan->Hp = plan->padded ? std::max(ext_h, min_Hp) : g.H;
    plan->Wp = plan->padded ? std::max(ext_w, min_Wp) : g.W;
    const int64_t xp_elems = static_cast<int64_t>(g.N) * g.C * plan->Hp * plan->Wp;
    if (xp_elems * 4 >= 0x7fff0000LL) return SPKV2_E_UNSUPPORTED;  // byte offsets are 31-bit
    plan->pad_bytes = plan->padded ? align256(static_cast<size_t>(xp_elems) * 4) : 0;
    GatherSpec gs;
    gs.K = K;
    gs.Wp = plan->Wp;
    gs.x_bytes = static_cast<int>(xp_elems * 4);
    gs.x_img_stride = g.C * plan->Hp * plan->Wp;
    const int Hp = plan->Hp, Wp = plan->Wp;
    gs.koff = [g, Hp, Wp](int k) {
        const int c = k / (g.KH * g.KW), r = k % (g.KH * g.KW);
        const int kh = r / g.KW, kw = r % g.KW;
        return ((c * Hp + kh * g.dh) * Wp + kw * g.dw) * 4;
    };
    gs.key = shape_key("conv", g, plan, gs.x_img_stride);
    gs.gather.C = g.C;
    gs.gather.cstride = Hp * Wp;
    gs.gather.KW = g.KW;
    gs.gather.tap_h = g.dh * Wp;
    gs.gather.tap_w = g.dw;
    {
        // the row window of a 16-pixel output segment (conv_window_f32):
        // KH rows of wlen columns of C + 4 floats
        const int wlen = (std::min(16, g.OW) - 1) * g.sw + (g.KW - 1) * g.dw + 1;
        if ((g.KH == 1 || g.KH == 3) && wlen <= 64 && static_cast<long long>(g.C + 4) * g.KH * wlen <= kWinFloats) {
            gs.gather.win_KH = g.KH;
            gs.gather.win_len = wlen;
            while ((1 << gs.gather.win_shift) < wlen) gs.gather.win_shift++;
            gs.gather.win_rows = g.N * g.OH;
            gs.gather.win_owb = (g.OW + 15) / 16;
            gs.gather.win_OH = g.OH;
            gs.gather.win_dh = g.dh;
            gs.gather.win_dw = g.dw;
        }
    }
    if (int rc = plan_tiles_and_weights(st, g, gs, w_host, plan)) return rc;
    plan->workspace = plan->pad_bytes + partial_bytes(plan);
    return 0;
}

// Plans the implicit GEMM of a Gemm node: the B source is A [rows][K]
// (k_stride 1, rows K apart) or, with trans_a, [K][rows] (k_stride rows,
// rows 1 apart).
int plan_igemm_gemm(hipStream_t st, const ConvGeom &g, const float *w_host, int k_stride, ConvPlan *plan) {
    plan->padded = false;
    plan->Hp = plan->Wp = 1;
    GatherSpec gs;
    gs.K = g.C;
    gs.Wp = 1;
    gs.x_bytes = static_cast<int>(g.x_elems * 4);
    gs.x_img_stride = k_stride == 1 ? g.C : 1;
    gs.koff = [k_stride](int k) { return k * k_stride * 4; };
    gs.key = shape_key(k_stride == 1 ? "gemm" : "gemm_ta", g, plan, gs.x_img_stride);
    gs.gather.C = g.C;  // one tap
    gs.gather.cstride = k_stride;
    gs.gather.kvec = k_stride == 1 && g.C % 4 == 0;  // A is [rows][K]: four k of a row are 16 contiguous bytes
    if (int rc = plan_tiles_and_weights(st, g, gs, w_host, plan)) return rc;
    plan->workspace = partial_bytes(plan);
    return 0;
}

std::string igemm_name(const ConvPlan *p) {
    if (kCfgs[p->cfg].thin_mb > 0)
        return std::string("conv_thin_f32<") + kCfgs[p->cfg].name + (p->padded ? ",pad" : "") + ">";
    if (kCfgs[p->cfg].window)
        return std::string("conv_window_f32<16x16,w") + std::to_string(kCfgs[p->cfg].skinny_waves) +
               (p->padded ? ",pad" : "") + ">";
    if (kCfgs[p->cfg].skinny_waves > 0)
        return std::string("conv_skinny_f32<16x16,w") + std::to_string(kCfgs[p->cfg].skinny_waves) +
               (p->padded ? ",pad" : "") + ">";
    return std::string("conv_igemm_f32<") + kCfgs[p->cfg].name +
           (p->gather.chk ? ",ipad" : p->padded ? ",pad" : "") +
           ",splitk=" + std::to_string(p->splitk) + (p->dp_tiles ? ",dp=" + std::to_string(p->dp_tiles) : "") + ">";
}

size_t claim_spec_scratch(const Spkv2Context *ctx, const Spkv2NodeRecord *node, ConvPlan *plan) {
    plan->ws_in_scratch = false;
    if (plan->workspace == 0) return 0;
    const Spkv2KernelSpecRecord *s = spec_by_id(ctx, node->kernel_spec_id);
    if (s && s->node_id == node->id && s->scratch_bytes >= plan->workspace) {
        plan->ws_in_scratch = true;
        plan->spec_id = node->kernel_spec_id;
        return 0;
    }
    return plan->workspace;
}

uint8_t *plan_workspace(const Spkv2Context *ctx, const ConvPlan *p) {
    if (p->workspace == 0) return ctx->workspace;  // not dereferenced
    if (p->ws_in_scratch) {
        // the same bounds the dispatcher checks before handing a kernel its scratch
        const Spkv2KernelSpecRecord *s = spec_by_id(ctx, p->spec_id);
        if (!s || !ctx->scratch || s->scratch_bytes < p->workspace || s->scratch_bytes > ctx->scratch_size ||
            s->scratch_offset > ctx->scratch_size - s->scratch_bytes)
            return nullptr;
        return ctx->scratch + s->scratch_offset;
    }
    return ctx->workspace_size >= p->workspace ? ctx->workspace : nullptr;
}

// x_img_stride: elements between consecutive "images" of the B source (a
// Gemm with trans_a reads A as [K][rows]: stride 1).
static int run_igemm_impl(Spkv2Context *ctx, const ConvPlan *p, const float *x, const float *bias, const float *res,
                          float *y, float alpha, int x_img_stride, int x_bytes, YLayout yl) {
    const ConvGeom &g = p->g;
    uint8_t *wsb = plan_workspace(ctx, p);
    if (p->workspace > 0 && !wsb) return SPKV2_E_UNSUPPORTED;
    const float *xs = x;
    // with the handoffs not live (a fault event armed, or the kernel registry
    // changed since prepare) every tensor is materialized and padded here
    const bool handoff = handoffs_live(ctx);
    int Wp = p->Wp;
    if (p->gather.chk) {
        Wp = g.W;  // implicit padding: the kernel reads the unpadded input, taps checked
    } else if (p->padded && p->pad_in && handoff) {
        xs = p->pad_in;  // written, zero halo included, by the producer's epilogue
        x_bytes = static_cast<int>(static_cast<size_t>(g.N) * g.C * p->Hp * p->Wp * 4);
        x_img_stride = g.C * p->Hp * p->Wp;
    } else if (p->padded) {
        float *xp = reinterpret_cast<float *>(wsb);
        const unsigned planes = static_cast<unsigned>(g.N * g.C);
        hipLaunchKernelGGL(pad_nchw, plane_grid(static_cast<size_t>(p->Hp) * p->Wp, planes), dim3(256), 0,
                           ctx->stream, x, xp, planes, static_cast<unsigned>(g.C), static_cast<size_t>(x_img_stride),
                           g.H, g.W, p->Hp, p->Wp, p->pt, p->pl);
        if (int rc = launch_status("pad_nchw")) return rc;
        xs = xp;
        x_bytes = static_cast<int>(static_cast<size_t>(planes) * p->Hp * p->Wp * 4);
        x_img_stride = g.C * p->Hp * p->Wp;
    }
    float *ws = p->workspace > 0 ? reinterpret_cast<float *>(wsb + p->pad_bytes) : nullptr;
    const bool give = p->pad_out && handoff;
    return launch_igemm(ctx->stream, p->cfg, plan_counts(p), g, Wp, xs, x_bytes, x_img_stride,
                        static_cast<const float *>(p->wpack), static_cast<const int *>(p->ktab), bias, res,
                        give && !p->y_needed ? nullptr : y, alpha, ws, p->gather, give ? p : nullptr, yl);
}

// Implicit padding.  A padded conv whose input no producer hands over in
// padded form, and whose gather per output pixel is short (C*KH*KW <= 160:
// RGB stems, 3x3 convs of up to 16 channels), reads the unpadded input with
// every tap bounds-checked (kModeChk) instead of copying it into a
// zero-padded buffer first: the k -> offset table is rebuilt for the
// unpadded input, a tap table gives (kh*dh, kw*dw) per k, and the padded
// copy's workspace is dropped.  For longer gathers the checks on every
// element cost more than the copy saves (a 64-channel 3x3 conv at 80x80,
// batch 16: 170 against 124 us with its copy), so they keep the copy; so
// do the skinny kernel (it reads a padded input) and inputs 16384 or more
// rows or columns tall (the tap table packs a tap into 16 bits).
// SPKV2_IMPLICIT_PAD=0 keeps the copy everywhere, =1 takes the checks
// wherever they apply.
static int use_implicit_padding(ConvPlan *plan) {
    const ConvGeom &g = plan->g;
    if (!plan->padded || plan->pad_in || kCfgs[plan->cfg].skinny_waves > 0 || kCfgs[plan->cfg].thin_mb > 0) return 0;
    if (g.H >= 16384 || g.W >= 16384 || (g.KH - 1) * g.dh >= 32768 || (g.KW - 1) * g.dw >= 32768) return 0;
    const char *e = getenv("SPKV2_IMPLICIT_PAD");
    if (e && e[0] == '0') return 0;
    if (!(e && e[0] == '1') && g.C * g.KH * g.KW > 160) return 0;
    const int BK = plan->BK;
    const int K = g.C * g.KH * g.KW;
    const size_t entries = static_cast<size_t>(plan->Kpad) + 2 * BK;  // as build_koff: two tiles past Kpad
    std::vector<int> koff(entries, kOobOffset), ktap(entries, 0x7fff7fff);
    for (int k = 0; k < K; k++) {
        const int c = k / (g.KH * g.KW), r = k % (g.KH * g.KW);
        const int th = (r / g.KW) * g.dh, tw = (r % g.KW) * g.dw;
        koff[k] = ((c * g.H + th) * g.W + tw) * 4;
        ktap[k] = (th << 16) | tw;
    }
    void *kt = nullptr, *tt = nullptr;
    if (int rc = upload_koff(koff, &kt)) return rc;
    if (int rc = upload_koff(ktap, &tt)) {
        (void)hipFree(kt);
        return rc;
    }
    if (plan->ktab) (void)hipFree(plan->ktab);
    plan->ktab = kt;
    plan->gather.ktap = static_cast<const int *>(tt);
    plan->gather.chk = true;
    plan->gather.chk_H = g.H;
    plan->gather.chk_W = g.W;
    plan->gather.chk_ph = g.ph;
    plan->gather.chk_pw = g.pw;
    plan->workspace -= plan->pad_bytes;
    plan->pad_bytes = 0;
    return 0;
}

static bool smallk_fits(const ConvGeom &g);

// The padded planes every padded fp32 implicit-GEMM conv reading this
// node's input plans with, when that input comes straight from a conv: the
// largest any of them needs (with the same top / left padding), so that they
// can all read one zero-padded copy, the pad handoff's buffer.  0 x 0 when
// the input has another producer.
static void shared_pad_extent(const Spkv2Context *ctx, const Spkv2NodeRecord *node, const ConvGeom &g, int *Hp,
                              int *Wp) {
    *Hp = *Wp = 0;
    const uint32_t t = node->inputs[0];
    bool from_conv = false;
    for (uint32_t i = 0; i < node->id && i < ctx->header.num_nodes; i++) {
        const Spkv2NodeRecord *n = &ctx->node_records[i];
        for (uint16_t k = 0; k < n->output_count; k++)
            if (n->outputs[k] == t) from_conv = n->op_type == SPKV2_OP_CONV;
    }
    if (!from_conv) return;
    for (uint32_t i = 0; i < ctx->header.num_nodes; i++) {
        const Spkv2NodeRecord *n = &ctx->node_records[i];
        if (n->op_type != SPKV2_OP_CONV || n->input_count < 2 || n->inputs[0] != t) continue;
        ConvGeom r;
        if (read_conv_geom(ctx, n, &r) != 0 || r.group != 1 || r.w_dtype != SPKV2_DTYPE_FP32 ||
            r.x_dtype != SPKV2_DTYPE_FP32 || smallk_fits(r) || r.ph != g.ph || r.pw != g.pw)
            continue;
        int h = 0, w = 0;
        if (!padded_extent(r, &h, &w)) continue;
        *Hp = std::max(*Hp, h);
        *Wp = std::max(*Wp, w);
    }
}

// fp32 handoff.  When this padded conv's input is the only output of an
// earlier fp32 implicit-GEMM conv, or one output of a channel Split of such
// a conv's output (then that conv stores only the Split output's channel
// range), that conv stores its result straight into
// a zero-padded buffer owned by this plan (halo zeroed once here, never
// written), and this conv skips its padding pass.  The producer still writes
// the unpadded tensor when anything else reads it.  Packages with a
// protection plan keep every tensor as written by the reference.
static int setup_pad_handoff(Spkv2Context *ctx, const Spkv2NodeRecord *node, ConvPlan *plan) {
    if (!plan->padded || ctx->protection_count > 0) return 0;
    if (const char *e = getenv("SPKV2_PAD_HANDOFF"))
        if (e[0] == '0') return 0;
    const uint32_t t = node->inputs[0];
    const Spkv2NodeRecord *prod = nullptr;
    int readers = 0;
    for (uint32_t i = 0; i < ctx->header.num_nodes; i++) {
        const Spkv2NodeRecord *n = &ctx->node_records[i];
        for (uint16_t k = 0; k < n->input_count; k++)
            if (n->inputs[k] == t) readers++;
        if (n->id < node->id)
            for (uint16_t k = 0; k < n->output_count; k++)
                if (n->outputs[k] == t) prod = n;
    }
    // through a channel Split (a C2f block's halves): the conv whose output
    // the Split cuts hands over the channel range of this conv's input
    int m0 = 0;
    bool via_split = false;
    if (prod && prod->op_type == SPKV2_OP_SPLIT && prod->input_count >= 1 && builtin_runs(ctx, prod->id)) {
        Spkv2AttrRecord attr;
        const Spkv2TensorRecord *sr = rec(ctx, prod->inputs[0]);
        if (spkv2_ctx_get_attr(ctx, prod, &attr) != 0 || sr->rank != 4 || (attr.axis < 0 ? attr.axis + 4 : attr.axis) != 1)
            return 0;
        for (uint16_t k = 0; k < prod->output_count && prod->outputs[k] != t; k++) m0 += rec(ctx, prod->outputs[k])->shape[1];
        const uint32_t s_in = prod->inputs[0];
        const Spkv2NodeRecord *sp = prod;
        prod = nullptr;
        for (uint32_t i = 0; i < sp->id; i++) {
            const Spkv2NodeRecord *n = &ctx->node_records[i];
            for (uint16_t k = 0; k < n->output_count; k++)
                if (n->outputs[k] == s_in) prod = n;
        }
        via_split = true;
    }
    if (!prod || prod->op_type != SPKV2_OP_CONV || prod->output_count != 1) return 0;
    if (!builtin_runs(ctx, prod->id) || !builtin_runs(ctx, node->id)) return 0;  // a user kernel runs one end
    if (ctx->plan_dtors[prod->id] != conv_plan_free) return 0;
    ConvPlan *pp = static_cast<ConvPlan *>(ctx->plans[prod->id]);
    if (!pp || (pp->path != CONV_IGEMM_F32 && pp->path != CONV_SMALLK_F32)) return 0;
    const ConvGeom &g = plan->g;
    if (pp->g.N != g.N || pp->g.OH != g.H || pp->g.OW != g.W) return 0;
    if (via_split ? m0 + g.C > pp->g.M : pp->g.M != g.C) return 0;
    if (pp->pad_out) {
        // the producer already hands this tensor to an earlier consumer: a
        // consumer with the same padded geometry and channel range reads
        // that consumer's buffer (the producer writes y as well, since the
        // tensor has more than one reader)
        if (pp->pad_Hp == plan->Hp && pp->pad_Wp == plan->Wp && pp->pad_pt == plan->pt && pp->pad_pl == plan->pl &&
            pp->pad_m0 == m0 && pp->pad_C == (via_split ? g.C : 0)) {
            plan->pad_in = pp->pad_out;
            plan->pad_in_shared = true;
        }
        return 0;
    }
    bool is_output = false;
    for (size_t i = 0; i < ctx->output_count; i++)
        if (ctx->output_ids[i] == t) is_output = true;
    const size_t bytes = static_cast<size_t>(g.N) * g.C * plan->Hp * plan->Wp * 4;
    if (int rc = hip_check(hipMalloc(reinterpret_cast<void **>(&plan->pad_in), bytes), "hipMalloc pad handoff"))
        return rc;
    if (int rc = hip_check(hipMemset(plan->pad_in, 0, bytes), "hipMemset pad handoff")) return rc;
    pp->pad_out = plan->pad_in;
    pp->pad_Hp = plan->Hp;
    pp->pad_Wp = plan->Wp;
    pp->pad_pt = plan->pt;
    pp->pad_pl = plan->pl;
    pp->pad_m0 = m0;
    pp->pad_C = via_split ? g.C : 0;
    pp->y_needed = via_split || readers > 1 || is_output;  // through a Split: the Split reads all of it
    return 0;
}

int run_igemm_f32(Spkv2Context *ctx, const ConvPlan *p, const float *x, const float *bias, const float *res, float *y,
                  float alpha) {
    return run_igemm_impl(ctx, p, x, bias, res, y, alpha, p->g.C * p->g.H * p->g.W, static_cast<int>(p->g.x_elems * 4),
                          YLayout{});
}

// Gemm entry: no residual, caller-chosen row stride of the B source.
int run_igemm_f32_strided(Spkv2Context *ctx, const ConvPlan *p, const float *x, const float *bias, float *y,
                          float alpha, int x_img_stride) {
    return run_igemm_impl(ctx, p, x, bias, nullptr, y, alpha, x_img_stride, static_cast<int>(p->g.x_elems * 4),
                          YLayout{});
}

// A conv node's run: its input and output through their channel-slice
// views when they have them (a Concat's buffer; never with a residual, so
// the residual keeps y's natural layout).
static int run_igemm_node(Spkv2Context *ctx, const ConvPlan *p, const Spkv2NodeRecord *node) {
    const ConvGeom &g = p->g;
    const float *x = dptr<const float>(ctx, node->inputs[0]);
    int x_img = g.C * g.H * g.W, x_bytes = static_cast<int>(g.x_elems * 4);
    if (const Spkv2TensorView *v = live_view(ctx, node->inputs[0])) {
        x = reinterpret_cast<const float *>(v->base);
        x_img = static_cast<int>(v->img_elems);
        x_bytes = static_cast<int>(v->extent);
    }
    float *y = dptr<float>(ctx, node->outputs[0]);
    YLayout yl;
    if (const Spkv2TensorView *v = live_view(ctx, node->outputs[0])) {
        if (g.has_res) return SPKV2_E_UNSUPPORTED;  // not set up that way
        y = reinterpret_cast<float *>(v->base);
        yl.img = static_cast<int>(v->img_elems);
        yl.bytes = static_cast<int>(v->extent);
        yl.cstride = static_cast<int>(v->ch_elems);
    }
    return run_igemm_impl(ctx, p, x, g.has_bias ? dptr<const float>(ctx, node->inputs[2]) : nullptr,
                          g.has_res ? dptr<const float>(ctx, node->inputs[3]) : nullptr, y, 1.0f, x_img, x_bytes, yl);
}

// The depthwise kernel takes group convs with one input channel per group and
// square 3x3, 5x5 or 7x7 taps.
static bool dw_fits(const ConvGeom &g) {
    return g.group > 1 && g.C == g.group && g.M % g.group == 0 && g.KH == g.KW &&
           (g.KH == 3 || g.KH == 5 || g.KH == 7);
}

static int run_direct(Spkv2Context *ctx, const Spkv2NodeRecord *node, const ConvGeom &g);

static int run_dw(Spkv2Context *ctx, const Spkv2NodeRecord *node, const ConvGeom &g) {
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
    a.Cg = 1;
    a.Mg = g.M / g.group;
    a.act = g.act;
    const int row_groups = (g.OH + kDwVO - 1) / kDwVO;
    const size_t threads = static_cast<size_t>(g.N) * g.M * row_groups * g.OW;
    if (threads >= (size_t(1) << 31)) return run_direct(ctx, node, g);
    const unsigned total = static_cast<unsigned>(threads);
    const dim3 grid((total + 255) / 256);
    if (g.KH == 3)
        hipLaunchKernelGGL(conv_dw_f32<3>, grid, dim3(256), 0, ctx->stream, a, row_groups, total);
    else if (g.KH == 5)
        hipLaunchKernelGGL(conv_dw_f32<5>, grid, dim3(256), 0, ctx->stream, a, row_groups, total);
    else
        hipLaunchKernelGGL(conv_dw_f32<7>, grid, dim3(256), 0, ctx->stream, a, row_groups, total);
    return launch_status("conv_dw_f32");
}

// The small-gather stem kernel takes ungrouped convs with at most
// kSmallkMaxC input channels, a gather of at most kSmallkMaxK taps and at
// most 64 output channels (SPKV2_CONV_SMALLK=0 keeps them on the implicit
// GEMM).
static bool smallk_fits(const ConvGeom &g) {
    if (const char *e = getenv("SPKV2_CONV_SMALLK"))
        if (e[0] == '0') return false;
    return g.group == 1 && g.C <= kSmallkMaxC && g.C * g.KH * g.KW <= kSmallkMaxK && g.M <= 64 &&
           g.H < 32768 && g.W < 32768 && (g.KH - 1) * g.dh < 32768 && (g.KW - 1) * g.dw < 32768;
}

static int run_smallk(Spkv2Context *ctx, const Spkv2NodeRecord *node, const ConvPlan *p) {
    const ConvGeom &g = p->g;
    SmallkArgs a{};
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
    a.act = g.act;
    a.segs = (g.OW + 63) / 64;
    a.x_bytes = static_cast<int>(g.x_elems * 4);
    // with the handoffs not live every tensor is materialized as written
    if (p->pad_out && handoffs_live(ctx)) {
        a.yp = p->pad_out;
        a.yp_Hp = p->pad_Hp;
        a.yp_Wp = p->pad_Wp;
        a.yp_pt = p->pad_pt;
        a.yp_pl = p->pad_pl;
        a.yp_m0 = p->pad_C > 0 ? p->pad_m0 : 0;
        a.yp_C = p->pad_C > 0 ? p->pad_C : g.M;
        if (!p->y_needed) a.y = nullptr;
    }
    const long long waves = static_cast<long long>(g.N) * g.OH * a.segs;
    if (waves <= 0) return 0;
    const long long blocks = (waves + 3) / 4;
    if (blocks > 0x7fffffffLL) return SPKV2_E_UNSUPPORTED;
    const dim3 grid(static_cast<unsigned>(blocks));
    if (g.M <= 16)
        hipLaunchKernelGGL(conv_smallk_f32<16>, grid, dim3(256), 0, ctx->stream, a);
    else if (g.M <= 32)
        hipLaunchKernelGGL(conv_smallk_f32<32>, grid, dim3(256), 0, ctx->stream, a);
    else
        hipLaunchKernelGGL(conv_smallk_f32<64>, grid, dim3(256), 0, ctx->stream, a);
    return launch_status("conv_smallk_f32");
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
    void **slot = &ctx->plans[node->id];
    if (*slot) {
        const ConvPlan *p = static_cast<ConvPlan *>(*slot);
        *ws = p->ws_in_scratch ? 0 : p->workspace;
        return 0;
    }
    ConvPlan *plan = new ConvPlan();
    memset(plan, 0, sizeof(*plan));
    plan->g = g;
    *slot = plan;
    ctx->plan_dtors[node->id] = conv_plan_free;
    int rc = 0;
    if (g.w_dtype == SPKV2_DTYPE_INT8) {
        rc = conv_i8_prepare(ctx, node, plan);
    } else if (g.w_dtype != SPKV2_DTYPE_FP32 || g.x_dtype != SPKV2_DTYPE_FP32) {
        rc = SPKV2_E_UNSUPPORTED;
    } else if (smallk_fits(g)) {
        plan->path = CONV_SMALLK_F32;
        set_kernel_name(ctx, node, "conv_smallk_f32");
    } else if (g.group == 1) {
        const float *w = reinterpret_cast<const float *>(host_weight_data(ctx, node->inputs[1]));
        if (!w) {
            rc = SPKV2_E_UNSUPPORTED;  // weights produced at run time
        } else {
            int hp = 0, wp = 0;
            shared_pad_extent(ctx, node, g, &hp, &wp);
            rc = plan_igemm_f32(ctx->stream, g, w, plan, hp, wp);
            if (rc == 0) rc = setup_pad_handoff(ctx, node, plan);
            if (rc == 0) rc = use_implicit_padding(plan);
            if (rc == 0) set_kernel_name(ctx, node, igemm_name(plan) + (plan->pad_in ? "+handoff" : ""));
        }
    } else if (dw_fits(g)) {
        plan->path = CONV_DW_F32;
        set_kernel_name(ctx, node, "conv_dw_f32");
    } else {
        plan->path = CONV_DIRECT_F32;
        set_kernel_name(ctx, node, "conv_direct_f32<grouped>");
    }
    if (rc == 0) *ws = claim_spec_scratch(ctx, node, plan);
    return rc;
}

int conv_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *scratch) {
    (void)scratch;
    if (ctx->plan_dtors[node->id] != conv_plan_free) return SPKV2_E_UNSUPPORTED;  // not prepared as a conv
    ConvPlan *plan = static_cast<ConvPlan *>(ctx->plans[node->id]);
    if (!plan) return SPKV2_E_UNSUPPORTED;  // prepare did not run for this node
    switch (plan->path) {
    case CONV_IGEMM_F32: return run_igemm_node(ctx, plan, node);
    case CONV_DIRECT_F32: return run_direct(ctx, node, plan->g);
    case CONV_DW_F32: return run_dw(ctx, node, plan->g);
    case CONV_IGEMM_I8:
    case CONV_Q8: return conv_i8_run(ctx, node, plan, nullptr);
    case CONV_SMALLK_F32: return run_smallk(ctx, node, plan);
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
    if (ctx->plan_dtors[node->id] != conv_plan_free) return SPKV2_E_UNSUPPORTED;
    ConvPlan *plan = static_cast<ConvPlan *>(ctx->plans[node->id]);
    if (!plan || (plan->path != CONV_IGEMM_I8 && plan->path != CONV_Q8)) return SPKV2_E_UNSUPPORTED;
    return conv_i8_run(ctx, node, plan, dev_out);
}

}  // namespace spk::kern
