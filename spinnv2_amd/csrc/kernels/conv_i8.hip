// INT8 convolution on MI355X with the reference runtime's semantics
// (runtime/kernels/optimized/conv/conv_int8.c:22-210):
//   per image, xq = sat8(round(x * (1/s_x))), rounding half to even for the
//   first floor(C*H*W/16)*16 elements (NCHW order) and half away from zero
//   for the tail; padded taps are int8 zero;
//   acc[m][n] = sum_k wq[m][k] * xq[k][n]   (int32, exact);
//   y = act( fma((float)acc, s_w[m]*s_x, bias[m]) + residual ).
// Inputs and outputs stay fp32 NCHW; weights are int8 OIHW with per-output-
// channel scales, the activation scale is per tensor (quantization section).
//
// Device plan:
//   1. quantize_pad_nhwc: one HBM pass reads x (NCHW fp32) and writes xq as
//      zero-padded NHWC int8 ([N][Hp][Wp][Cp], halo and padded channels 0)
//      into the runtime workspace, so every tap of the convolution is in
//      bounds and 16 consecutive k are 16 contiguous bytes;
//   2. conv_igemm_i8<BM,BN,BK>: implicit GEMM.  K is a sequence of 16-byte
//      groups: with dilation 1 the KW*Cp bytes of one kernel row form one
//      contiguous run (pixels iw..iw+KW-1), padded to a multiple of 16 with
//      zero weights; otherwise each (kh, kw) tap is Cp/16 groups.  Group g of
//      output column n sits at byte col(n) + koff[g] of xq: one
//      buffer_load_dwordx4 with (voffset, soffset) = (col(n), koff[g]).
//      Weights are repacked at prepare into [m_tile][k_tile][BM][BK] panels
//      in the same k order.  v_mfma_i32_32x32x32_i8 on LDS tiles stored
//      k-contiguous, two-tile register prefetch, dequantize / bias /
//      residual / activation in registers with buffer stores.
//   3. split-K (small grids): int32 partials summed by a second kernel.
// Integer sums are order independent, so the accumulators equal the closed
// form bit for bit whatever the tiling or split.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "conv.hpp"
#include "kernels.hpp"
#include "q8_math.hpp"

namespace spk::kern {

namespace {

// gfx9 buffer resource word 3 (raw, untyped); loads at or beyond num_records
// return 0, stores there are dropped
constexpr int kBufWord3 = 0x00020000;
// byte offset out of range for every buffer (all < 2 GiB)
constexpr int kOob = 0x7fff0000;

// xq[img][hp][wp][c] = q(x[img][c][hp-pt][wp-pl]) inside the image and for
// c < C, 0 elsewhere.  A block covers 64 padded pixels x 64 channels,
// transposed through LDS so reads (along w) and writes (along c) are both
// contiguous.
// In the INT8 configuration with int8 tensors between nodes (q8) every
// value is sat8(roundf(v) + zp) and the halo and padded channels hold zp.
__device__ __forceinline__ int quantize_q8(float v, float inv_scale, int zp) {
    const float t = v * inv_scale;
    if (t != t) return zp;
    const float r = fminf(fmaxf(roundf(t), -512.0f), 512.0f);
    return min(max(static_cast<int>(r) + zp, -128), 127);
}

__global__ void __launch_bounds__(256) quantize_pad_nhwc(const float *__restrict__ x, int8_t *__restrict__ xq, int C,
                                                         int H, int W, int Hp, int Wp, int Cp, int pt, int pl,
                                                         float inv_scale, int split, int zp, int q8) {
    __shared__ int8_t tile[64][64 + 4];
    const int img = blockIdx.z;
    const int p0 = blockIdx.x * 64;
    const int c0 = blockIdx.y * 64;
    const int HW = H * W;
    const int HWp = Hp * Wp;
    const float *xi = x + static_cast<size_t>(img) * C * HW;
    const int tp = threadIdx.x & 63;
    const int pp = p0 + tp;
    const int hp = pp / Wp;
    const int h = hp - pt, w = pp - hp * Wp - pl;
    const bool inside = pp < HWp && static_cast<unsigned>(h) < static_cast<unsigned>(H) &&
                        static_cast<unsigned>(w) < static_cast<unsigned>(W);
    for (int cc = threadIdx.x >> 6; cc < 64; cc += 4) {
        const int c = c0 + cc;
        int8_t q = static_cast<int8_t>(zp);
        if (inside && c < C) {
            const int idx = c * HW + h * W + w;  // NCHW index inside the image
            if (q8) {
                q = static_cast<int8_t>(quantize_q8(xi[idx], inv_scale, zp));
            } else {
                const float v = xi[idx] * inv_scale;
                float r;
                if (v != v) r = 0.0f;  // NaN quantizes to 0 (the ARM conversions)
                else r = idx < split ? rintf(v) : roundf(v);
                r = fminf(fmaxf(r, -128.0f), 127.0f);
                q = static_cast<int8_t>(static_cast<int>(r));
            }
        }
        tile[cc][tp] = q;
    }
    __syncthreads();
    // each thread writes 16 channels (four dwords) of one pixel
    const int wpix = threadIdx.x >> 2;
    const int wc = (threadIdx.x & 3) * 16;
    const int p = p0 + wpix;
    if (p >= HWp || c0 + wc >= Cp) return;
    uint32_t *dst = reinterpret_cast<uint32_t *>(xq + (static_cast<size_t>(img) * HWp + p) * Cp + c0 + wc);
    const int ndw = min(4, (Cp - c0 - wc) / 4);
    for (int d = 0; d < ndw; d++) {
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) word |= static_cast<uint32_t>(static_cast<uint8_t>(tile[wc + 4 * d + b][wpix])) << (8 * b);
        dst[d] = word;
    }
}

// The same quantization for inputs with few channels (Cp <= 16, e.g. an RGB
// stem): one thread per padded pixel reads its C values and writes its Cp
// bytes as dwords, instead of 64-channel tiles that would sit mostly idle.
__global__ void __launch_bounds__(256) quantize_pad_nhwc_narrow(const float *__restrict__ x, int8_t *__restrict__ xq,
                                                                int C, int H, int W, int Hp, int Wp, int Cp, int pt,
                                                                int pl, float inv_scale, int split, int images, int zp,
                                                                int q8) {
    const int HW = H * W;
    const int HWp = Hp * Wp;
    const size_t total = static_cast<size_t>(images) * HWp;
    for (size_t t = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; t < total;
         t += static_cast<size_t>(gridDim.x) * 256) {
        const int img = static_cast<int>(t / HWp);
        const int pp = static_cast<int>(t - static_cast<size_t>(img) * HWp);
        const int hp = pp / Wp;
        const int h = hp - pt, w = pp - hp * Wp - pl;
        const bool inside = static_cast<unsigned>(h) < static_cast<unsigned>(H) &&
                            static_cast<unsigned>(w) < static_cast<unsigned>(W);
        const float *xi = x + static_cast<size_t>(img) * C * HW;
        uint32_t *dst = reinterpret_cast<uint32_t *>(xq + t * Cp);
        for (int c0 = 0; c0 < Cp; c0 += 4) {
            uint32_t word = 0;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const int c = c0 + b;
                int8_t q = static_cast<int8_t>(zp);
                if (inside && c < C) {
                    const int idx = c * HW + h * W + w;  // NCHW index inside the image
                    if (q8) {
                        q = static_cast<int8_t>(quantize_q8(xi[idx], inv_scale, zp));
                    } else {
                        const float v = xi[idx] * inv_scale;
                        float r;
                        if (v != v) r = 0.0f;  // NaN quantizes to 0 (the ARM conversions)
                        else r = idx < split ? rintf(v) : roundf(v);
                        r = fminf(fmaxf(r, -128.0f), 127.0f);
                        q = static_cast<int8_t>(static_cast<int>(r));
                    }
                }
                word |= static_cast<uint32_t>(static_cast<uint8_t>(q)) << (8 * b);
            }
            dst[c0 / 4] = word;
        }
    }
}

struct I8Args {
    const int8_t *__restrict__ xq;      // padded NHWC int8
    const int8_t *__restrict__ wp;      // [m_tiles][k_tiles][BM][BK]
    const int *__restrict__ koff;       // byte offset of each 16-byte k group; kOob past K
    const float *__restrict__ scales;   // [M] s_w[m]*s_x
    const float *__restrict__ bias;
    const float *__restrict__ res;
    float *__restrict__ y;
    int32_t *__restrict__ ws;           // split-K partials [split][M][Ntot], or raw accumulators (NCHW)
    int x_bytes, y_bytes, ws_bytes;
    int img_stride;                     // bytes per padded image
    int Wp, Cp, M, OW, OHW, Ntot;
    // n / OHW and n / OW as a multiply and shift (div_fast), for column
    // indices below 2^31: most of the per-pixel address arithmetic
    unsigned ohw_m, ow_m;
    int ohw_s, ow_s;
    int sh, sw;
    int m_tiles, k_tiles, kt_per_split;
    int act;
    int mode;  // 0: dequant epilogue, 1: int32 partials to ws[split][M][Ntot], 2: raw acc to ws as NCHW
    // requantize handoff (mode 0): also write q(y) into the consuming conv's
    // padded NHWC int8 input; y may then be null (no other reader)
    int8_t *__restrict__ q_out;
    int q_bytes, q_Hp, q_Wp, q_Cp, q_pt, q_pl, q_split;
    float q_inv;
    // INT8 configuration with int8 tensors between nodes (q8 = 1): mode 0
    // requantizes in fixed point into q_out (an int8 tensor's padded NHWC
    // buffer, zero point y_zp) instead of dequantizing; qrow holds five rows
    // of M int32 (-z_x * sum(w), that plus bias_q, m1, m2, shift); the
    // residual is the int8 tensor r8 (zero point r_zp); mode 2 adds the
    // first row, giving sum(w (x - z_x)).
    int q8;
    int q8_hi;  // every row's shift is at least 33: q8_requant_hi
    const int *__restrict__ qrow;
    const int8_t *__restrict__ r8;
    int r_bytes, r_Hp, r_Wp, r_Cp, r_pt, r_pl, r_zp;
    int y_zp;
};



// The reference's activation quantization of one value (conv_int8.c:26-55):
// round half to even below `split` (the 16-wide vector body), half away
// from zero in the tail, saturate to int8, NaN -> 0.
__device__ __forceinline__ int quantize_one(float v, float inv_scale, bool even) {
    const float t = v * inv_scale;
    float r;
    if (t != t) r = 0.0f;
    else r = even ? rintf(t) : roundf(t);
    r = fminf(fmaxf(r, -128.0f), 127.0f);
    return static_cast<int>(r);
}

// n / d for 0 <= n < 2^31 with (m, s) from div_magic(d): m = ceil(2^s / d),
// s = 31 + ceil(log2 d), so n m / 2^s is within 2^-ceil(log2 d) <= 1/d of
// n / d and its floor is exact.  One 32 x 32 -> 64 multiply and a shift
// instead of a division sequence.
__device__ __forceinline__ int div_fast(int n, unsigned m, int s) {
    return static_cast<int>((static_cast<uint64_t>(static_cast<unsigned>(n)) * m) >> s);
}

constexpr int i8_stage_bytes(int BM, int BN);
template <int BM, int Q8>
__device__ __forceinline__ void i8_load_row_params(const I8Args &a, int mt0, float *s_par);
template <int BM, int BN, int TM, int TN>
__device__ __forceinline__ void i8_epilogue(intx16 (&acc)[TM][TN], const I8Args &a, int mt0, int nt0, int wmo, int wno,
                                            int lane, const float *s_par, int8_t *s_q);
// 16-byte pieces of a BM x BN tile's int8 channels (BM/16 per pixel) each
// thread of a 256-thread workgroup stages
template <int BM, int BN>
constexpr int q8_pieces() { return (BN * (BM / 16) + 255) / 256; }
template <int BM, int BN>
__device__ __forceinline__ void q8_residual_load(const I8Args &a, int mt0, int nt0, uintx4 (&rr)[q8_pieces<BM, BN>()]);
template <int BM, int BN, int TM, int TN>
__device__ __forceinline__ void q8_epilogue(intx16 (&acc)[TM][TN], const I8Args &a, int mt0, int nt0, int wmo, int wno,
                                            int lane, const float *s_par, int8_t *s_q,
                                            const uintx4 (&rr)[q8_pieces<BM, BN>()]);

// Q8: the INT8 configuration's epilogue (q8_epilogue) instead of i8_epilogue,
// a separate instantiation so that neither epilogue's registers weigh on the
// other's kernels.
template <int BM, int BN, int BK, int BMAP, int Q8>
__global__ void __launch_bounds__(256) conv_igemm_i8(I8Args a) {
    constexpr int TM = BM / 64, TN = BN / 64;  // 2x2 waves, each (32*TM) x (32*TN)
    constexpr int LDK = BK + 16;               // bytes per LDS row
    constexpr int GPT = BK * BN / 4096;        // 16-byte B groups per thread per k-tile
    constexpr int APT = BM * BK / 4096;        // 16-byte A chunks per thread per k-tile
    static_assert(TM >= 1 && TN >= 1 && GPT >= 1 && APT >= 1 && BK % 32 == 0, "tile shape");
    static_assert(BMAP == 0 || BN % (4096 / BK) == 0, "BMAP 1: whole pixel passes");
    // the operand buffers, reused by the epilogue's staging area
    constexpr int OPS = 2 * (BM + BN) * LDK;
    constexpr int SMEM = OPS > i8_stage_bytes(BM, BN) ? OPS : i8_stage_bytes(BM, BN);
    __shared__ __attribute__((aligned(16))) int8_t smem[SMEM];
    __shared__ float s_par[5 * BM];  // per-row epilogue constants
    int8_t(*As)[BM * LDK] = reinterpret_cast<int8_t(*)[BM * LDK]>(smem);
    int8_t(*Bs)[BN * LDK] = reinterpret_cast<int8_t(*)[BN * LDK]>(smem + 2 * BM * LDK);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // consecutive workgroups land on different XCDs: give each XCD a
    // contiguous range of tiles, m fastest, so tiles sharing an activation
    // panel share that XCD's L2
    int bid = blockIdx.x;
    const int nb = gridDim.x;
    if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
    const int mt = bid % a.m_tiles;
    const int nt = bid / a.m_tiles;
    const int kt0 = blockIdx.y * a.kt_per_split;
    const int kt1 = min(kt0 + a.kt_per_split, a.k_tiles);

    const __amdgpu_buffer_rsrc_t xrs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(a.xq), static_cast<short>(0), a.x_bytes, kBufWord3);
    // byte offset of output column n's receptive-field origin in xq
    auto col_of = [&](int n) -> int {
        if (n >= a.Ntot) return kOob;
        const int img = div_fast(n, a.ohw_m, a.ohw_s);
        const int sp = n - img * a.OHW;
        const int oh = div_fast(sp, a.ow_m, a.ow_s);
        const int ow = sp - oh * a.OW;
        return img * a.img_stride + (oh * a.sh * a.Wp + ow * a.sw) * a.Cp;
    };
    // B gather, two lane maps:
    //  BMAP 0: lane = column n, one wave-uniform k group per load (koff[g] in
    //          the scalar offset) -- any K layout, but the 64 lanes of a load
    //          touch 64 pixels Cp bytes apart;
    //  BMAP 1: lane = (pixel, k group), groups fastest, so 8 lanes read 128
    //          contiguous bytes of one pixel -- for layers whose BK/16 groups
    //          of a k-tile are contiguous in xq (the tile's base offset in the
    //          scalar offset, the group's 16-byte step in the lane offset).
    constexpr int G = BK / 16;       // 16-byte k groups per tile
    constexpr int PPP = 256 / G;     // pixels per pass of the whole workgroup (BMAP 1)
    const int bcol = BMAP ? (tid / G) : (tid % BN);
    const int bgrp = BMAP ? (tid % G) : __builtin_amdgcn_readfirstlane(tid / BN);  // wave-uniform for BMAP 0
    int colp[BMAP ? GPT : 1];
    if constexpr (BMAP) {
#pragma unroll
        for (int p = 0; p < GPT; p++) colp[p] = col_of(nt * BN + p * PPP + bcol) + bgrp * 16;
    } else {
        colp[0] = col_of(nt * BN + bcol);
    }

    intx4 ar0[APT], ar1[APT], br0[GPT], br1[GPT];

#define I8_LOAD_TILE(KT, AR, BR)                                                                                     \
    {                                                                                                                \
        const int kt_ = min((KT), a.k_tiles - 1);                                                                    \
        const intx4 *src =                                                                                           \
            reinterpret_cast<const intx4 *>(a.wp + (static_cast<size_t>(mt) * a.k_tiles + kt_) * (BM * BK));        \
        _Pragma("unroll") for (int i = 0; i < APT; i++) AR[i] = src[tid + i * 256];                                  \
        /* the table has two tiles of out-of-range entries past the last */                                       \
        if constexpr (BMAP) {                                                                                        \
            const int kbase = a.koff[(KT) * G];                                                                      \
            _Pragma("unroll") for (int p = 0; p < GPT; p++) BR[p] =                                                  \
                __builtin_bit_cast(intx4, __builtin_amdgcn_raw_buffer_load_b128(xrs, colp[p], kbase, 0));            \
        } else {                                                                                                     \
            const int *ko = a.koff + (KT) * G + bgrp * GPT;                                                          \
            _Pragma("unroll") for (int g = 0; g < GPT; g++) BR[g] =                                                  \
                __builtin_bit_cast(intx4, __builtin_amdgcn_raw_buffer_load_b128(xrs, colp[0], ko[g], 0));            \
        }                                                                                                            \
    }

#define I8_STORE_TILE(BUF, AR, BR)                                                                                   \
    {                                                                                                                \
        _Pragma("unroll") for (int i = 0; i < APT; i++) {                                                            \
            const int f = (tid + i * 256) * 16;                                                                      \
            *reinterpret_cast<intx4 *>(&As[BUF][(f / BK) * LDK + (f % BK)]) = AR[i];                                 \
        }                                                                                                             \
        if constexpr (BMAP) {                                                                                        \
            _Pragma("unroll") for (int p = 0; p < GPT; p++) * reinterpret_cast<intx4 *>(                             \
                &Bs[BUF][(p * PPP + bcol) * LDK + bgrp * 16]) = BR[p];                                               \
        } else {                                                                                                     \
            _Pragma("unroll") for (int g = 0; g < GPT; g++) * reinterpret_cast<intx4 *>(                             \
                &Bs[BUF][bcol * LDK + (bgrp * GPT + g) * 16]) = BR[g];                                               \
        }                                                                                                            \
    }

#define I8_COMPUTE(BUF)                                                                                              \
    _Pragma("unroll") for (int k32 = 0; k32 < BK / 32; k32++) {                                                      \
        intx4 af[TM], bf[TN];                                                                                        \
        _Pragma("unroll") for (int i = 0; i < TM; i++) af[i] =                                                       \
            *reinterpret_cast<const intx4 *>(&As[BUF][((wm * TM + i) * 32 + row) * LDK + k32 * 32 + khalf]);         \
        _Pragma("unroll") for (int j = 0; j < TN; j++) bf[j] =                                                       \
            *reinterpret_cast<const intx4 *>(&Bs[BUF][((wn * TN + j) * 32 + row) * LDK + k32 * 32 + khalf]);         \
        _Pragma("unroll") for (int i = 0; i < TM; i++) _Pragma("unroll") for (int j = 0; j < TN; j++) acc[i][j] =    \
            __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);                                 \
    }

    // one pipeline step: tile KT in LDS buffer BUF, tile KT+1 in flight in
    // (AN, BNX), the free register set (AF, BF) receives tile KT+2
#define I8_STEP(KT, BUF, AN, BNX, AF, BF)                                                                            \
    {                                                                                                                \
        I8_LOAD_TILE((KT) + 2, AF, BF);                                                                              \
        __builtin_amdgcn_sched_barrier(0);                                                                           \
        I8_COMPUTE(BUF);                                                                                             \
        __builtin_amdgcn_sched_barrier(0);                                                                           \
        I8_STORE_TILE((BUF) ^ 1, AN, BNX);                                                                           \
        __syncthreads();                                                                                             \
    }

    const int row = lane & 31;
    const int khalf = 16 * (lane >> 5);  // lanes 32-63 supply bytes 16..31 of each 32-k step
    intx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

    if (kt0 >= kt1) return;  // empty split-K slice
    i8_load_row_params<BM, Q8>(a, mt * BM, s_par);  // read after the loop's barriers
    I8_LOAD_TILE(kt0, ar0, br0);
    I8_LOAD_TILE(kt0 + 1, ar1, br1);
    I8_STORE_TILE(0, ar0, br0);
    __syncthreads();
    int kt = kt0;
    // tiles past kt1 are loaded and ignored: no data-dependent branches
    for (; kt + 1 < kt1; kt += 2) {
        I8_STEP(kt, 0, ar1, br1, ar0, br0);
        I8_STEP(kt + 1, 1, ar0, br0, ar1, br1);
    }
    if (kt < kt1) {
        I8_COMPUTE(0);
    }
#undef I8_STEP
#undef I8_COMPUTE
#undef I8_LOAD_TILE
#undef I8_STORE_TILE
    if constexpr (Q8) {
        uintx4 rr[q8_pieces<BM, BN>()];
        if (a.mode == 0 && a.r8) q8_residual_load<BM, BN>(a, mt * BM, nt * BN, rr);
        q8_epilogue<BM, BN, TM, TN>(acc, a, mt * BM, nt * BN, wm * TM * 32, wn * TN * 32, lane, s_par, smem, rr);
    } else {
        i8_epilogue<BM, BN, TM, TN>(acc, a, mt * BM, nt * BN, wm * TM * 32, wn * TN * 32, lane, s_par, smem);
    }
}

// Workgroup-shared memory of the int8 GEMM kernels' epilogue: the tile's
// per-row combined scales and biases (BM each, loaded in the prologue), and
// a [BN pixels][BM + 16 bytes] staging area for the handoff's int8 values
// that aliases the k-loop's operand buffers (free once the loop is done).
constexpr int i8_stage_bytes(int BM, int BN) { return BN * (BM + 16); }

// s_par: [BM] combined scales and [BM] biases, or with q8 [BM][4] int32
// (c, m1, m2, shift of each row: rows 1-4 of the plan's qrow table), one
// 16-byte LDS read per row in the epilogue.
template <int BM, int Q8>
__device__ __forceinline__ void i8_load_row_params(const I8Args &a, int mt0, float *s_par) {
    if constexpr (Q8) {
        // [BM][4] (c, m1, m2, S or with q8_hi 2^(S-33)), then [BM] S - 32
        int *s_i = reinterpret_cast<int *>(s_par);
        for (int i = threadIdx.x; i < BM; i += 256) {
            const int m = mt0 + i;
            const bool in = m < a.M;
            s_i[4 * i] = in ? a.qrow[a.M + m] : 0;
            s_i[4 * i + 1] = in ? a.qrow[2 * a.M + m] : 0;
            s_i[4 * i + 2] = in ? a.qrow[3 * a.M + m] : 0;
            s_i[4 * i + 3] = in ? a.qrow[(a.q8_hi ? 5 : 4) * a.M + m] : (a.q8_hi ? 1 : 33);
            s_i[4 * BM + i] = in ? a.qrow[6 * a.M + m] : 1;
        }
        return;
    }
    for (int i = threadIdx.x; i < BM; i += 256) {
        const int m = mt0 + i;
        s_par[i] = m < a.M ? a.scales[m] : 0.0f;
        s_par[BM + i] = a.bias && m < a.M ? a.bias[m] : 0.0f;
    }
}

// The epilogue of the int8 GEMM kernels: one wave's TM x TN blocks of 32x32
// accumulators, at rows wmo.. and columns wno.. of the workgroup's BM x BN
// tile at (mt0, nt0) (blockIdx.y is the split-K slice).  mode 1 stores int32
// partials, mode 2 the raw accumulators as NCHW, mode 0 dequantizes (+ bias,
// residual, activation) into y and/or requantizes into the consumer's padded
// NHWC int8 buffer: through the LDS staging area when its channel pitch is a
// multiple of 16, so each pixel's channels of the tile leave as contiguous
// 16-byte pieces (the other waves' channels of the same pixel beside them).
template <int BM, int BN, int TM, int TN>
__device__ __forceinline__ void i8_epilogue(intx16 (&acc)[TM][TN], const I8Args &a, int mt0, int nt0, int wmo, int wno,
                                            int lane, const float *s_par, int8_t *s_q) {
    const float *s_sc = s_par, *s_bi = s_par + BM;
    const int m0 = mt0 + wmo, n0 = nt0 + wno;
    const int row = lane & 31;
    // 32x32 accumulator layout: lane holds column (lane & 31) and rows
    // 8*(r/4) + 4*(lane/32) + (r%4).  Offsets are unsigned bytes; rows past
    // M and columns past N get out-of-range offsets (stores dropped).
    const unsigned M = a.M;
    const unsigned rsub = 4 * (lane >> 5);
    unsigned mrow[TM];
#pragma unroll
    for (int i = 0; i < TM; i++) mrow[i] = m0 + i * 32 + rsub;
    if (a.mode == 1) {
        const __amdgpu_buffer_rsrc_t wrs =
            __builtin_amdgcn_make_buffer_rsrc(a.ws, static_cast<short>(0), a.ws_bytes, kBufWord3);
        const unsigned nt4 = static_cast<unsigned>(a.Ntot) * 4u;
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = n0 + j * 32 + row;
            const unsigned wcol = n < a.Ntot ? static_cast<unsigned>(n) * 4u : static_cast<unsigned>(kOob);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const unsigned m = mrow[i] + 8 * (r >> 2) + (r & 3);
                    __builtin_amdgcn_raw_buffer_store_b32(acc[i][j][r], wrs, m < M ? wcol + m * nt4 : kOob,
                                                          blockIdx.y * M * nt4, 0);
                }
        }
        return;
    }
    const unsigned ohw4 = static_cast<unsigned>(a.OHW) * 4u;
    unsigned obase[TN];
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = n0 + j * 32 + row;
        const int img = div_fast(n, a.ohw_m, a.ohw_s);
        const int sp = n - img * a.OHW;
        obase[j] = n < a.Ntot
                       ? (static_cast<unsigned>(img) * M * static_cast<unsigned>(a.OHW) + static_cast<unsigned>(sp)) * 4u
                       : static_cast<unsigned>(kOob);
    }
    if (a.mode == 2) {
        const __amdgpu_buffer_rsrc_t wrs =
            __builtin_amdgcn_make_buffer_rsrc(a.ws, static_cast<short>(0), a.ws_bytes, kBufWord3);
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const unsigned m = mrow[i] + 8 * (r >> 2) + (r & 3);
                    __builtin_amdgcn_raw_buffer_store_b32(acc[i][j][r], wrs, m < M ? obase[j] + m * ohw4 : kOob, 0, 0);
                }
        return;
    }
    const __amdgpu_buffer_rsrc_t yrs = __builtin_amdgcn_make_buffer_rsrc(a.y ? a.y : const_cast<float *>(a.scales), static_cast<short>(0),
                                                                         a.y ? a.y_bytes : 0, kBufWord3);
    const __amdgpu_buffer_rsrc_t rrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(a.res ? a.res : a.scales), static_cast<short>(0), a.res ? a.y_bytes : 0, kBufWord3);
    const __amdgpu_buffer_rsrc_t qrs = __builtin_amdgcn_make_buffer_rsrc(
        a.q_out ? a.q_out : const_cast<int8_t *>(a.xq), static_cast<short>(0), a.q_out ? a.q_bytes : 0, kBufWord3);
    // handoff: byte offset of this lane's pixel in the consumer's padded NHWC
    // buffer, and its spatial index (for the NCHW rounding split)
    unsigned qbase[TN];
    int qsp[TN];
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = n0 + j * 32 + row;
        const int img = div_fast(n, a.ohw_m, a.ohw_s);
        const int sp = n - img * a.OHW;
        const int oh = div_fast(sp, a.ow_m, a.ow_s);
        const int ow = sp - oh * a.OW;
        qsp[j] = sp;
        qbase[j] = n < a.Ntot ? static_cast<unsigned>(((img * a.q_Hp + oh + a.q_pt) * a.q_Wp + ow + a.q_pl) * a.q_Cp)
                              : static_cast<unsigned>(kOob);
    }
    // staged handoff (workgroup-uniform): the staging area aliases the
    // k-loop's LDS operands, so every wave must be past its last read
    const bool stage = a.q_out && a.q_Cp % 16 == 0;
    constexpr int SQ = BM + 16;  // staging row pitch: an odd multiple of 16 bytes
    if (stage) __syncthreads();
#pragma unroll
    for (int i = 0; i < TM; i++) {
        // per-row constants of this block (LDS), for all TN blocks
        floatx16 sc, bi;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int ml = wmo + i * 32 + static_cast<int>(rsub) + 8 * (r >> 2) + (r & 3);
            sc[r] = s_sc[ml];
            bi[r] = s_bi[ml];
        }
#pragma unroll
        for (int j = 0; j < TN; j++) {
            floatx16 v;
#pragma unroll
            for (int r = 0; r < 16; r++) v[r] = fmaf(static_cast<float>(acc[i][j][r]), sc[r], bi[r]);
            if (a.res) {
                floatx16 rv;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const unsigned m = mrow[i] + 8 * (r >> 2) + (r & 3);
                    rv[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                          rrs, m < M ? obase[j] + m * ohw4 : kOob, 0, 0));
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
            if (a.q_out) {
                // four consecutive channels of the lane -> one dword; channels
                // past M are written 0 (the padded channels stay zero)
                unsigned words[4];
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++) {
                    const unsigned m0 = mrow[i] + 8 * q4;
                    unsigned word = 0;
#pragma unroll
                    for (int b = 0; b < 4; b++) {
                        const unsigned m = m0 + b;
                        const int idx = static_cast<int>(m) * a.OHW + qsp[j];
                        const int qv = m < M ? quantize_one(v[4 * q4 + b], a.q_inv, idx < a.q_split) : 0;
                        word |= (static_cast<unsigned>(qv) & 0xffu) << (8 * b);
                    }
                    words[q4] = word;
                }
                if (stage) {
                    // the tile's pixel row in LDS: 4 channels per dword
                    const int pl = wno + j * 32 + row;
#pragma unroll
                    for (int q4 = 0; q4 < 4; q4++) {
                        const int cl = wmo + i * 32 + static_cast<int>(rsub) + 8 * q4;
                        *reinterpret_cast<unsigned *>(&s_q[pl * SQ + cl]) = words[q4];
                    }
                } else {
#pragma unroll
                    for (int q4 = 0; q4 < 4; q4++) {
                        const unsigned m0 = mrow[i] + 8 * q4;
                        __builtin_amdgcn_raw_buffer_store_b32(words[q4], qrs, m0 < M ? qbase[j] + m0 : kOob, 0, 0);
                    }
                }
            }
            if (a.y) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const unsigned m = mrow[i] + 8 * (r >> 2) + (r & 3);
                    // __float_as_uint takes the element by value
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[r]), yrs,
                                                          m < M ? obase[j] + m * ohw4 : kOob, 0, 0);
                }
            }
        }
    }
    if (!stage) return;
    __syncthreads();
    // 16-byte pieces of the staged tile, the BM/16 pieces of one pixel on
    // consecutive threads; a piece is stored when its first channel is below
    // M (channels from M to the padded pitch hold 0)
    constexpr int PPX = BM / 16;
    for (int t = threadIdx.x; t < BN * PPX; t += 256) {
        const int pl = t / PPX;
        const int c16 = (t - pl * PPX) * 16;
        const int n = nt0 + pl;
        if (n >= a.Ntot || mt0 + c16 >= a.M) continue;
        const int img = div_fast(n, a.ohw_m, a.ohw_s);
        const int sp = n - img * a.OHW;
        const int oh = div_fast(sp, a.ow_m, a.ow_s);
        const int ow = sp - oh * a.OW;
        const unsigned off =
            static_cast<unsigned>(((img * a.q_Hp + oh + a.q_pt) * a.q_Wp + ow + a.q_pl) * a.q_Cp + mt0 + c16);
        const uintx4 val = *reinterpret_cast<const uintx4 *>(&s_q[pl * SQ + c16]);
        __builtin_amdgcn_raw_buffer_store_b128(val, qrs, off, 0, 0);
    }
}

// The epilogue of the INT8 configuration with int8 tensors between nodes
// (conv_igemm_i8* with Q8): mode 1 and mode 2 as in i8_epilogue (mode 2
// adds -z_x sum(w) per row, giving sum(w (x - z_x))); mode 0 requantizes in
// fixed point into the output int8 tensor.  The tile goes through the LDS
// staging area ([BN pixels][BM + 16 bytes]): the residual tile, when there
// is one, is first loaded into it as 16-byte pieces of each pixel's
// channels; each lane then replaces its residual dwords (four channels of a
// pixel) with its four requantized outputs; the tile leaves as 16-byte
// pieces.  Per-row constants (c, m1, m2, shift) come from LDS four rows at a
// time, so only the accumulators stay live.
// The residual tile's 16-byte pieces for this thread (the BM/16 pieces of
// one pixel on consecutive threads), loaded into registers; pieces past the
// output's pixels or channels read 0 (out-of-range offsets).
template <int BM, int BN>
__device__ __forceinline__ void q8_residual_load(const I8Args &a, int mt0, int nt0, uintx4 (&rr)[q8_pieces<BM, BN>()]) {
    constexpr int PPX = BM / 16;
    const __amdgpu_buffer_rsrc_t r8s = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t *>(a.r8 ? a.r8 : reinterpret_cast<const int8_t *>(a.wp)), static_cast<short>(0),
        a.r8 ? a.r_bytes : 0, kBufWord3);
#pragma unroll
    for (int k = 0; k < q8_pieces<BM, BN>(); k++) {
        const int t = threadIdx.x + 256 * k;
        const int pl = t / PPX;
        const int c16 = (t - pl * PPX) * 16;
        const int n = nt0 + pl;
        unsigned off = static_cast<unsigned>(kOob);
        if (t < BN * PPX && n < a.Ntot && mt0 + c16 < a.M) {
            const int img = div_fast(n, a.ohw_m, a.ohw_s);
            const int sp = n - img * a.OHW;
            const int oh = div_fast(sp, a.ow_m, a.ow_s);
            const int ow = sp - oh * a.OW;
            off = static_cast<unsigned>(((img * a.r_Hp + oh + a.r_pt) * a.r_Wp + ow + a.r_pl) * a.r_Cp + mt0 + c16);
        }
        rr[k] = __builtin_amdgcn_raw_buffer_load_b128(r8s, off, 0, 0);
    }
}

// clamp(v, lo) to [lo, 127] (lo <= 127) in one instruction: the median of
// v, lo and 127
__device__ __forceinline__ int med3_127(int v, int lo) {
    int r;
    asm("v_med3_i32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "v"(lo), "v"(127));
    return r;
}

// The requantization of one wave's TM x TN accumulator blocks in the LDS
// staging area ([pixel][BM + 16 bytes]): each lane's four consecutive
// channels of a pixel are one dword there, holding the residual's bytes on
// entry (RES) and the int8 outputs on exit.  HI: every row's shift is at
// least 33 (q8_requant_hi).  Rows past M get z_y.
template <int BM, int TM, int TN, bool HI, bool RES>
__device__ __forceinline__ void q8_requant_tile(intx16 (&acc)[TM][TN], const I8Args &a, int mt0, int wmo, int wno,
                                                int lane, const float *s_par, int8_t *s_q) {
    constexpr int SQ = BM + 16;
    const int row = lane & 31;
    const int rsub = 4 * (lane >> 5);
    const intx4 *s_row = reinterpret_cast<const intx4 *>(s_par);
    const int *s_k = reinterpret_cast<const int *>(s_par) + 4 * BM;
    const int lo = a.act == 1 ? a.y_zp : -128;  // Relu clamps at the zero point
    const int zy = a.y_zp, zr = a.r_zp;
    (void)mt0;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            // rows ml .. ml + 3 of the tile: four consecutive channels (rows
            // past M compute from zero constants; the channels they land in
            // are never read)
            const int ml = wmo + i * 32 + rsub + 8 * q4;
            intx4 p[4];
            int k[4];
#pragma unroll
            for (int b = 0; b < 4; b++) {
                p[b] = s_row[ml + b];
                if (HI) k[b] = s_k[ml + b];
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                unsigned *cell = reinterpret_cast<unsigned *>(&s_q[(wno + j * 32 + row) * SQ + ml]);
                const unsigned rw = RES ? *cell : 0u;
                unsigned word = 0;
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const int rd = RES ? static_cast<int>(static_cast<int8_t>(rw >> (8 * b))) - zr : 0;
                    const int x = acc[i][j][4 * q4 + b];
                    const int qv = HI ? q8_requant_hi(x, p[b][0], p[b][1], p[b][2], p[b][3], k[b], rd, lo, med3_127)
                                      : q8_requant(x, p[b][0], p[b][1], p[b][2], p[b][3], rd, zy, lo);
                    word |= (static_cast<unsigned>(qv) & 0xffu) << (8 * b);
                }
                *cell = word;
            }
        }
}

template <int BM, int BN, int TM, int TN>
__device__ __forceinline__ void q8_epilogue(intx16 (&acc)[TM][TN], const I8Args &a, int mt0, int nt0, int wmo, int wno,
                                            int lane, const float *s_par, int8_t *s_q,
                                            const uintx4 (&rr)[q8_pieces<BM, BN>()]) {
    const int m0 = mt0 + wmo, n0 = nt0 + wno;
    const int row = lane & 31;
    const unsigned M = a.M;
    const unsigned rsub = 4 * (lane >> 5);
    if (a.mode == 1 || a.mode == 2) {
        const __amdgpu_buffer_rsrc_t wrs =
            __builtin_amdgcn_make_buffer_rsrc(a.ws, static_cast<short>(0), a.ws_bytes, kBufWord3);
        const unsigned nt4 = static_cast<unsigned>(a.Ntot) * 4u;
        const unsigned ohw4 = static_cast<unsigned>(a.OHW) * 4u;
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = n0 + j * 32 + row;
            const int img = div_fast(n, a.ohw_m, a.ohw_s);
            const int sp = n - img * a.OHW;
            // mode 1: partials [split][M][Ntot]; mode 2: NCHW accumulators
            const unsigned col = n >= a.Ntot ? static_cast<unsigned>(kOob)
                                 : a.mode == 1
                                     ? static_cast<unsigned>(n) * 4u
                                     : (static_cast<unsigned>(img) * M * static_cast<unsigned>(a.OHW) + sp) * 4u;
            const unsigned mstride = a.mode == 1 ? nt4 : ohw4;
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const unsigned m = m0 + i * 32 + rsub + 8 * (r >> 2) + (r & 3);
                    const int v = acc[i][j][r] + (a.mode == 2 && m < M ? a.qrow[m] : 0);
                    __builtin_amdgcn_raw_buffer_store_b32(v, wrs, m < M ? col + m * mstride : kOob,
                                                          a.mode == 1 ? blockIdx.y * M * nt4 : 0u, 0);
                }
        }
        return;
    }
    const __amdgpu_buffer_rsrc_t qrs =
        __builtin_amdgcn_make_buffer_rsrc(a.q_out, static_cast<short>(0), a.q_bytes, kBufWord3);
    constexpr int SQ = BM + 16;  // staging row pitch: an odd multiple of 16 bytes
    constexpr int PPX = BM / 16;
    // the staging area aliases the k-loop's LDS operands: every wave must be
    // past its last read
    __syncthreads();
    if (a.r8) {
        // the residual tile (loaded by the caller) into the staging area
#pragma unroll
        for (int k = 0; k < q8_pieces<BM, BN>(); k++) {
            const int t = threadIdx.x + 256 * k;
            const int pl = t / PPX;
            const int c16 = (t - pl * PPX) * 16;
            if (t < BN * PPX) *reinterpret_cast<uintx4 *>(&s_q[pl * SQ + c16]) = rr[k];
        }
        __syncthreads();
    }
    // one copy of the loop per (shift form, residual) pair, chosen once per
    // tile, so no per-element branch remains
    if (a.q8_hi) {
        if (a.r8) q8_requant_tile<BM, TM, TN, true, true>(acc, a, m0 - wmo, wmo, wno, lane, s_par, s_q);
        else q8_requant_tile<BM, TM, TN, true, false>(acc, a, m0 - wmo, wmo, wno, lane, s_par, s_q);
    } else {
        if (a.r8) q8_requant_tile<BM, TM, TN, false, true>(acc, a, m0 - wmo, wmo, wno, lane, s_par, s_q);
        else q8_requant_tile<BM, TM, TN, false, false>(acc, a, m0 - wmo, wmo, wno, lane, s_par, s_q);
    }
    __syncthreads();
    // 16-byte pieces of the staged tile, the BM/16 pieces of one pixel on
    // consecutive threads; a piece is stored when its first channel is below
    // M (channels from M to the padded pitch hold z_y)
    for (int t = threadIdx.x; t < BN * PPX; t += 256) {
        const int pl = t / PPX;
        const int c16 = (t - pl * PPX) * 16;
        const int n = nt0 + pl;
        if (n >= a.Ntot || mt0 + c16 >= a.M) continue;
        const int img = div_fast(n, a.ohw_m, a.ohw_s);
        const int sp = n - img * a.OHW;
        const int oh = div_fast(sp, a.ow_m, a.ow_s);
        const int ow = sp - oh * a.OW;
        const unsigned off =
            static_cast<unsigned>(((img * a.q_Hp + oh + a.q_pt) * a.q_Wp + ow + a.q_pl) * a.q_Cp + mt0 + c16);
        const uintx4 val = *reinterpret_cast<const uintx4 *>(&s_q[pl * SQ + c16]);
        __builtin_amdgcn_raw_buffer_store_b128(val, qrs, off, 0, 0);
    }
}

// Implicit GEMM with the weight operand straight from memory: the packed
// weights of a k-tile are stored in MFMA fragment order ([BM/32 row blocks]
// [BK/32 k steps][64 lanes][16 bytes]: lane l holds row l%32 and bytes
// 16*(l/32)..+15 of the 32-byte k step), so each wave loads its A fragments
// with one 16-byte load per fragment from L2 (a layer's weights are shared
// by all its workgroups) into registers, two k-tiles ahead, and only the
// gathered activations go through LDS (pixel-major gather, as BMAP 1 of
// conv_igemm_i8).  WAVES_M x WAVES_N waves, each (32*TM) x (32*TN).
template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, int Q8>
__global__ void __launch_bounds__(256) conv_igemm_i8x(I8Args a) {
    constexpr int TM = BM / (32 * WAVES_M), TN = BN / (32 * WAVES_N);
    constexpr int K32 = BK / 32;       // 32-byte k steps per tile
    constexpr int LDK = BK + 16;       // bytes per LDS row: an odd multiple of 16
    constexpr int G = BK / 16;         // 16-byte k groups per tile
    constexpr int PPP = 256 / G;       // pixels per pass of the workgroup
    constexpr int GPT = BN / PPP;      // 16-byte B loads per thread per tile
    static_assert(WAVES_M * WAVES_N == 4 && TM >= 1 && TN >= 1 && BK % 32 == 0, "tile shape");
    static_assert(GPT >= 1 && BN % PPP == 0 && (LDK / 16) % 2 == 1, "B gather shape");
    // the operand buffers, reused by the epilogue's staging area
    constexpr int SMEM = 2 * BN * LDK > i8_stage_bytes(BM, BN) ? 2 * BN * LDK : i8_stage_bytes(BM, BN);
    __shared__ __attribute__((aligned(16))) int8_t smem[SMEM];
    __shared__ float s_par[5 * BM];  // per-row epilogue constants
    int8_t(*Bs)[BN * LDK] = reinterpret_cast<int8_t(*)[BN * LDK]>(smem);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;

    // each XCD walks a contiguous range of tiles, m fastest (see conv_igemm_i8)
    int bid = blockIdx.x;
    const int nb = gridDim.x;
    if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
    const int mt = bid % a.m_tiles;
    const int nt = bid / a.m_tiles;
    const int kt0 = blockIdx.y * a.kt_per_split;
    const int kt1 = min(kt0 + a.kt_per_split, a.k_tiles);

    const __amdgpu_buffer_rsrc_t xrs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(a.xq), static_cast<short>(0), a.x_bytes, kBufWord3);
    const int bpix = tid / G, bgrp = tid % G;
    int colp[GPT];
#pragma unroll
    for (int p = 0; p < GPT; p++) {
        const int n = nt * BN + p * PPP + bpix;
        int c = kOob;
        if (n < a.Ntot) {
            const int img = div_fast(n, a.ohw_m, a.ohw_s);
            const int sp = n - img * a.OHW;
            const int oh = div_fast(sp, a.ow_m, a.ow_s);
            const int ow = sp - oh * a.OW;
            c = img * a.img_stride + (oh * a.sh * a.Wp + ow * a.sw) * a.Cp;
        }
        colp[p] = c + bgrp * 16;
    }
    const int row = lane & 31;
    const int khalf = 16 * (lane >> 5);

    intx4 a0[TM][K32], a1[TM][K32], br0[GPT], br1[GPT];

#define I8X_LOAD_A(KT, AX)                                                                                           \
    {                                                                                                                \
        const int kt_ = min((KT), a.k_tiles - 1);                                                                    \
        const intx4 *src =                                                                                           \
            reinterpret_cast<const intx4 *>(a.wp + (static_cast<size_t>(mt) * a.k_tiles + kt_) * (BM * BK));        \
        _Pragma("unroll") for (int i = 0; i < TM; i++) _Pragma("unroll") for (int q = 0; q < K32; q++) AX[i][q] =     \
            src[((wm * TM + i) * K32 + q) * 64 + lane];                                                              \
    }
    // the table has two tiles of out-of-range entries past the last
#define I8X_LOAD_B(KT, BR)                                                                                           \
    {                                                                                                                \
        const int kbase = a.koff[(KT) * G];                                                                          \
        _Pragma("unroll") for (int p = 0; p < GPT; p++) BR[p] =                                                      \
            __builtin_bit_cast(intx4, __builtin_amdgcn_raw_buffer_load_b128(xrs, colp[p], kbase, 0));                \
    }
#define I8X_STORE_B(BUF, BR)                                                                                         \
    {                                                                                                                \
        _Pragma("unroll") for (int p = 0; p < GPT; p++) * reinterpret_cast<intx4 *>(                                 \
            &Bs[BUF][(p * PPP + bpix) * LDK + bgrp * 16]) = BR[p];                                                   \
    }
#define I8X_FRAG_B(BUF, Q, BF)                                                                                       \
    {                                                                                                                \
        _Pragma("unroll") for (int j = 0; j < TN; j++) BF[j] =                                                       \
            *reinterpret_cast<const intx4 *>(&Bs[BUF][((wn * TN + j) * 32 + row) * LDK + (Q) * 32 + khalf]);        \
    }
#define I8X_MMA(AX, Q, BF)                                                                                           \
    _Pragma("unroll") for (int i = 0; i < TM; i++) _Pragma("unroll") for (int j = 0; j < TN; j++) acc[i][j] =        \
        __builtin_amdgcn_mfma_i32_32x32x32_i8(AX[i][Q], BF[j], acc[i][j], 0, 0, 0);
    // the B fragments of step q+1 are read while the MFMAs of step q run
#define I8X_COMPUTE(BUF, AX)                                                                                         \
    {                                                                                                                \
        intx4 fb0[TN], fb1[TN];                                                                                      \
        I8X_FRAG_B(BUF, 0, fb0);                                                                                     \
        _Pragma("unroll") for (int q = 0; q < K32; q += 2) {                                                         \
            if (q + 1 < K32) I8X_FRAG_B(BUF, q + 1, fb1);                                                            \
            I8X_MMA(AX, q, fb0);                                                                                     \
            if (q + 2 < K32) I8X_FRAG_B(BUF, q + 2, fb0);                                                            \
            if (q + 1 < K32) { I8X_MMA(AX, q + 1, fb1); }                                                            \
        }                                                                                                            \
    }
    // one pipeline step: B of tile KT in LDS buffer BUF, its A in AC; B of
    // tile KT+1 in flight in BNX; B of tile KT+2 into the free set BF and A
    // of tile KT+1 into AN
#define I8X_STEP(KT, BUF, AC, AN, BNX, BF)                                                                           \
    {                                                                                                                \
        I8X_LOAD_B((KT) + 2, BF);                                                                                    \
        I8X_LOAD_A((KT) + 1, AN);                                                                                    \
        __builtin_amdgcn_sched_barrier(0);                                                                           \
        I8X_COMPUTE(BUF, AC);                                                                                        \
        __builtin_amdgcn_sched_barrier(0);                                                                           \
        I8X_STORE_B((BUF) ^ 1, BNX);                                                                                 \
        __syncthreads();                                                                                             \
    }

    intx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

    if (kt0 >= kt1) return;  // empty split-K slice
    i8_load_row_params<BM, Q8>(a, mt * BM, s_par);  // read after the loop's barriers
    I8X_LOAD_B(kt0, br0);
    I8X_LOAD_B(kt0 + 1, br1);
    I8X_LOAD_A(kt0, a0);
    I8X_STORE_B(0, br0);
    __syncthreads();
    int kt = kt0;
    // tiles past kt1 are loaded and ignored: no data-dependent branches
    for (; kt + 1 < kt1; kt += 2) {
        I8X_STEP(kt, 0, a0, a1, br1, br0);
        I8X_STEP(kt + 1, 1, a1, a0, br0, br1);
    }
    if (kt < kt1) {
        I8X_COMPUTE(0, a0);
    }
#undef I8X_STEP
#undef I8X_COMPUTE
#undef I8X_MMA
#undef I8X_FRAG_B
#undef I8X_STORE_B
#undef I8X_LOAD_B
#undef I8X_LOAD_A
    if constexpr (Q8) {
        uintx4 rr[q8_pieces<BM, BN>()];
        if (a.mode == 0 && a.r8) q8_residual_load<BM, BN>(a, mt * BM, nt * BN, rr);
        q8_epilogue<BM, BN, TM, TN>(acc, a, mt * BM, nt * BN, wm * TM * 32, wn * TN * 32, lane, s_par, smem, rr);
    } else {
        i8_epilogue<BM, BN, TM, TN>(acc, a, mt * BM, nt * BN, wm * TM * 32, wn * TN * 32, lane, s_par, smem);
    }
}

// Persistent form of conv_igemm_i8x (no split-K): a grid of at most the
// workgroups the GPU holds at once (a multiple of 8), workgroup b walking the
// tiles of XCD b % 8's contiguous share (m fastest) with a stride of the
// workgroups on that XCD.  Before a tile's epilogue the next tile's first two
// B k-tiles, its first A k-tile and (Q8) its residual tile are loaded into
// registers, so their memory latency overlaps the epilogue's arithmetic and
// stores; short-K layers (1x1 convs: one or two k-tiles) are otherwise a
// chain of dependent round trips per tile.
template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, int Q8>
__global__ void __launch_bounds__(256) conv_igemm_i8p(I8Args a) {
    constexpr int TM = BM / (32 * WAVES_M), TN = BN / (32 * WAVES_N);
    constexpr int K32 = BK / 32;
    constexpr int LDK = BK + 16;
    constexpr int G = BK / 16;
    constexpr int PPP = 256 / G;
    constexpr int GPT = BN / PPP;
    constexpr int RP = q8_pieces<BM, BN>();
    static_assert(WAVES_M * WAVES_N == 4 && TM >= 1 && TN >= 1 && BK % 32 == 0, "tile shape");
    static_assert(GPT >= 1 && BN % PPP == 0 && (LDK / 16) % 2 == 1, "B gather shape");
    constexpr int SMEM = 2 * BN * LDK > i8_stage_bytes(BM, BN) ? 2 * BN * LDK : i8_stage_bytes(BM, BN);
    __shared__ __attribute__((aligned(16))) int8_t smem[SMEM];
    __shared__ float s_par[5 * BM];
    int8_t(*Bs)[BN * LDK] = reinterpret_cast<int8_t(*)[BN * LDK]>(smem);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int row = lane & 31;
    const int khalf = 16 * (lane >> 5);
    const int bpix = tid / G, bgrp = tid % G;

    const int n_tiles = (a.Ntot + BN - 1) / BN;
    const int T = a.m_tiles * n_tiles;
    const int xcd = blockIdx.x & 7, per = gridDim.x >> 3;
    const int t_end = static_cast<int>((static_cast<int64_t>(xcd) + 1) * T / 8);
    int t = static_cast<int>(static_cast<int64_t>(xcd) * T / 8) + (blockIdx.x >> 3);
    if (t >= t_end) return;  // workgroup-uniform

    const __amdgpu_buffer_rsrc_t xrs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(a.xq), static_cast<short>(0), a.x_bytes, kBufWord3);
    // byte offsets of this thread's B pixels of tile column nt (+ its group)
    auto columns = [&](int nt, int (&cp)[GPT]) {
#pragma unroll
        for (int p = 0; p < GPT; p++) {
            const int n = nt * BN + p * PPP + bpix;
            int c = kOob;
            if (n < a.Ntot) {
                const int img = div_fast(n, a.ohw_m, a.ohw_s);
                const int sp = n - img * a.OHW;
                const int oh = div_fast(sp, a.ow_m, a.ow_s);
                const int ow = sp - oh * a.OW;
                c = img * a.img_stride + (oh * a.sh * a.Wp + ow * a.sw) * a.Cp;
            }
            cp[p] = c + bgrp * 16;
        }
    };

    intx4 a0[TM][K32], a1[TM][K32], br0[GPT], br1[GPT];
    int colp[GPT];
    uintx4 rr[RP];

#define I8P_LOAD_A(MT, KT, AX)                                                                                       \
    {                                                                                                                \
        const int kt_ = min((KT), a.k_tiles - 1);                                                                    \
        const intx4 *src =                                                                                           \
            reinterpret_cast<const intx4 *>(a.wp + (static_cast<size_t>(MT) * a.k_tiles + kt_) * (BM * BK));        \
        _Pragma("unroll") for (int i = 0; i < TM; i++) _Pragma("unroll") for (int q = 0; q < K32; q++) AX[i][q] =     \
            src[((wm * TM + i) * K32 + q) * 64 + lane];                                                              \
    }
#define I8P_LOAD_B(CP, KT, BR)                                                                                       \
    {                                                                                                                \
        const int kbase = a.koff[(KT) * G];                                                                          \
        _Pragma("unroll") for (int p = 0; p < GPT; p++) BR[p] =                                                      \
            __builtin_bit_cast(intx4, __builtin_amdgcn_raw_buffer_load_b128(xrs, CP[p], kbase, 0));                  \
    }
#define I8P_STORE_B(BUF, BR)                                                                                         \
    {                                                                                                                \
        _Pragma("unroll") for (int p = 0; p < GPT; p++) * reinterpret_cast<intx4 *>(                                 \
            &Bs[BUF][(p * PPP + bpix) * LDK + bgrp * 16]) = BR[p];                                                   \
    }
#define I8P_FRAG_B(BUF, Q, BF)                                                                                       \
    {                                                                                                                \
        _Pragma("unroll") for (int j = 0; j < TN; j++) BF[j] =                                                       \
            *reinterpret_cast<const intx4 *>(&Bs[BUF][((wn * TN + j) * 32 + row) * LDK + (Q) * 32 + khalf]);        \
    }
#define I8P_MMA(AX, Q, BF)                                                                                           \
    _Pragma("unroll") for (int i = 0; i < TM; i++) _Pragma("unroll") for (int j = 0; j < TN; j++) acc[i][j] =        \
        __builtin_amdgcn_mfma_i32_32x32x32_i8(AX[i][Q], BF[j], acc[i][j], 0, 0, 0);
#define I8P_COMPUTE(BUF, AX)                                                                                         \
    {                                                                                                                \
        intx4 fb0[TN], fb1[TN];                                                                                      \
        I8P_FRAG_B(BUF, 0, fb0);                                                                                     \
        _Pragma("unroll") for (int q = 0; q < K32; q += 2) {                                                         \
            if (q + 1 < K32) I8P_FRAG_B(BUF, q + 1, fb1);                                                            \
            I8P_MMA(AX, q, fb0);                                                                                     \
            if (q + 2 < K32) I8P_FRAG_B(BUF, q + 2, fb0);                                                            \
            if (q + 1 < K32) { I8P_MMA(AX, q + 1, fb1); }                                                            \
        }                                                                                                            \
    }
#define I8P_STEP(KT, BUF, AC, AN, BNX, BF)                                                                           \
    {                                                                                                                \
        I8P_LOAD_B(colp, (KT) + 2, BF);                                                                              \
        I8P_LOAD_A(mt, (KT) + 1, AN);                                                                                \
        __builtin_amdgcn_sched_barrier(0);                                                                           \
        I8P_COMPUTE(BUF, AC);                                                                                        \
        __builtin_amdgcn_sched_barrier(0);                                                                           \
        I8P_STORE_B((BUF) ^ 1, BNX);                                                                                 \
        __syncthreads();                                                                                             \
    }

    // the first tile's prologue loads
    int mt = t % a.m_tiles, nt = t / a.m_tiles;
    columns(nt, colp);
    I8P_LOAD_B(colp, 0, br0);
    I8P_LOAD_B(colp, 1, br1);
    I8P_LOAD_A(mt, 0, a0);
    if constexpr (Q8)
        if (a.r8) q8_residual_load<BM, BN>(a, mt * BM, nt * BN, rr);
    for (;;) {
        i8_load_row_params<BM, Q8>(a, mt * BM, s_par);  // read after the loop's barriers
        I8P_STORE_B(0, br0);
        __syncthreads();
        intx16 acc[TM][TN];
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][j][r] = 0;
        int kt = 0;
        for (; kt + 1 < a.k_tiles; kt += 2) {
            I8P_STEP(kt, 0, a0, a1, br1, br0);
            I8P_STEP(kt + 1, 1, a1, a0, br0, br1);
        }
        if (kt < a.k_tiles) {
            I8P_COMPUTE(0, a0);
        }
        // the next tile's prologue loads, in flight during this epilogue
        const int tn = t + per;
        const bool more = tn < t_end;
        const int mt_n = more ? tn % a.m_tiles : mt, nt_n = more ? tn / a.m_tiles : nt;
        uintx4 rr_n[RP];
        if (more) {
            int cp[GPT];
            columns(nt_n, cp);
#pragma unroll
            for (int p = 0; p < GPT; p++) colp[p] = cp[p];
            I8P_LOAD_B(cp, 0, br0);
            I8P_LOAD_B(cp, 1, br1);
            I8P_LOAD_A(mt_n, 0, a0);
            if constexpr (Q8)
                if (a.r8) q8_residual_load<BM, BN>(a, mt_n * BM, nt_n * BN, rr_n);
        }
        if constexpr (Q8)
            q8_epilogue<BM, BN, TM, TN>(acc, a, mt * BM, nt * BN, wm * TM * 32, wn * TN * 32, lane, s_par, smem, rr);
        else
            i8_epilogue<BM, BN, TM, TN>(acc, a, mt * BM, nt * BN, wm * TM * 32, wn * TN * 32, lane, s_par, smem);
        if (!more) break;
        t = tn;
        mt = mt_n;
        nt = nt_n;
#pragma unroll
        for (int k = 0; k < RP; k++) rr[k] = rr_n[k];
        // every wave is past this tile's epilogue (its LDS staging and row
        // constants) before the next tile writes them
        __syncthreads();
    }
#undef I8P_STEP
#undef I8P_COMPUTE
#undef I8P_MMA
#undef I8P_FRAG_B
#undef I8P_STORE_B
#undef I8P_LOAD_B
#undef I8P_LOAD_A
}

// Sums the int32 split-K partials (exact in any order), then dequantizes or
// writes the raw accumulators.  Four consecutive columns per thread when N
// is a multiple of 4.
template <int VEC>
__global__ void __launch_bounds__(256) splitk_i8_epilogue(const int32_t *__restrict__ ws, int splitk, int M, int Ntot,
                                                          int OHW, const float *__restrict__ scales,
                                                          const float *__restrict__ bias, const float *__restrict__ res,
                                                          float *__restrict__ y, int32_t *__restrict__ raw, int act,
                                                          I8Args q) {
    typedef int vec_t __attribute__((ext_vector_type(VEC)));
    const size_t total = static_cast<size_t>(M) * Ntot;
    const size_t groups = total / VEC;
    for (size_t gi = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; gi < groups;
         gi += static_cast<size_t>(gridDim.x) * 256) {
        const size_t idx = gi * VEC;
        const int m = static_cast<int>(idx / Ntot);
        const int n = static_cast<int>(idx - static_cast<size_t>(m) * Ntot);
        // up to 16 slices' loads in flight before the first add
        vec_t v = 0;
        for (int s = 0; s < splitk; s += 16) {
            vec_t p[16];
#pragma unroll
            for (int t = 0; t < 16; t++)
                if (s + t < splitk) p[t] = *reinterpret_cast<const vec_t *>(ws + (s + t) * total + idx);
#pragma unroll
            for (int t = 0; t < 16; t++)
                if (s + t < splitk) v += p[t];
        }
        if (q.q8) {
            // the INT8 configuration: raw accumulators corrected for the
            // input zero point, or the fixed-point requantization into the
            // output int8 tensor (one byte per output)
#pragma unroll
            for (int e = 0; e < VEC; e++) {
                const int img = div_fast(n + e, q.ohw_m, q.ohw_s);
                const int sp = n + e - img * OHW;
                if (raw) {
                    raw[(static_cast<size_t>(img) * M + m) * OHW + sp] = v[e] + q.qrow[m];
                    continue;
                }
                const int oh = div_fast(sp, q.ow_m, q.ow_s), ow = sp - oh * q.OW;
                const int rd = q.r8 ? static_cast<int>(q.r8[(static_cast<size_t>(img * q.r_Hp + oh + q.r_pt) * q.r_Wp +
                                                             ow + q.r_pl) * q.r_Cp + m]) - q.r_zp
                                    : 0;
                q.q_out[(static_cast<size_t>(img * q.q_Hp + oh + q.q_pt) * q.q_Wp + ow + q.q_pl) * q.q_Cp + m] =
                    static_cast<int8_t>(q8_requant(v[e], q.qrow[M + m], q.qrow[2 * M + m], q.qrow[3 * M + m],
                                                   q.qrow[4 * M + m], rd, q.y_zp, act == 1 ? q.y_zp : -128));
            }
            continue;
        }
        const float sm = scales[m];
        const float bm = bias ? bias[m] : 0.0f;
#pragma unroll
        for (int e = 0; e < VEC; e++) {
            const int img = div_fast(n + e, q.ohw_m, q.ohw_s);
            const int sp = n + e - img * OHW;
            const size_t yi = (static_cast<size_t>(img) * M + m) * OHW + sp;
            if (raw) {
                raw[yi] = v[e];
                continue;
            }
            float f = fmaf(static_cast<float>(v[e]), sm, bm);
            if (res) f += res[yi];
            f = apply_act(f, act);
            if (q.q_out) {
                const int oh = div_fast(sp, q.ow_m, q.ow_s), ow = sp - oh * q.OW;
                q.q_out[(static_cast<size_t>(img * q.q_Hp + oh + q.q_pt) * q.q_Wp + ow + q.q_pl) * q.q_Cp + m] =
                    static_cast<int8_t>(quantize_one(f, q.q_inv, m * OHW + sp < q.q_split));
            }
            if (y) y[yi] = f;
        }
    }
}

using I8Kernel = void (*)(I8Args);

struct I8Cfg {
    int BM, BN, BK;
    int bmap;     // B gather lane map (see conv_igemm_i8)
    int adirect;  // 1: conv_igemm_i8x / i8p, weights packed in MFMA fragment order and loaded straight to registers
    int persist;  // 1: conv_igemm_i8p, a resident grid walking the tiles (no split-K)
    const char *name;
    I8Kernel kernel;     // reference semantics (i8_epilogue)
    I8Kernel kernel_q8;  // the INT8 configuration (q8_epilogue)
};

// New configurations go at the end: the tune tables store indices.
#define I8CFG(BM, BN, BK) \
    {BM, BN, BK, 0, 0, 0, #BM "x" #BN "x" #BK, conv_igemm_i8<BM, BN, BK, 0, 0>, conv_igemm_i8<BM, BN, BK, 0, 1>}
#define I8CFGP(BM, BN, BK)                                                                                          \
    {BM, BN, BK, 1, 0, 0, #BM "x" #BN "x" #BK ",px", conv_igemm_i8<BM, BN, BK, 1, 0>,                             \
     conv_igemm_i8<BM, BN, BK, 1, 1>}
#define I8CFGX(BM, BN, BK, WM, WN)                                                                                  \
    {BM, BN, BK, 1, 1, 0, #BM "x" #BN "x" #BK ",ax" #WM "x" #WN, conv_igemm_i8x<BM, BN, BK, WM, WN, 0>,          \
     conv_igemm_i8x<BM, BN, BK, WM, WN, 1>}
#define I8CFGR(BM, BN, BK, WM, WN)                                                                                  \
    {BM, BN, BK, 1, 1, 1, #BM "x" #BN "x" #BK ",ax" #WM "x" #WN ",persist", conv_igemm_i8p<BM, BN, BK, WM, WN, 0>, \
     conv_igemm_i8p<BM, BN, BK, WM, WN, 1>}
const I8Cfg kI8Cfgs[] = {
    I8CFG(128, 128, 64),  I8CFG(128, 128, 128),  I8CFG(128, 64, 64),  I8CFG(128, 64, 128),
    I8CFG(64, 128, 64),   I8CFG(64, 64, 64),     I8CFG(64, 64, 128),
    I8CFGP(128, 128, 64), I8CFGP(128, 128, 128), I8CFGP(128, 64, 64), I8CFGP(128, 64, 128),
    I8CFGP(64, 128, 64),  I8CFGP(64, 64, 64),    I8CFGP(64, 64, 128),
    I8CFGX(128, 128, 128, 2, 2), I8CFGX(128, 64, 128, 2, 2), I8CFGX(64, 128, 128, 2, 2),
    I8CFGX(64, 64, 128, 2, 2),   I8CFGX(128, 128, 64, 2, 2),  I8CFGX(128, 64, 64, 2, 2),
    I8CFGX(64, 64, 64, 2, 2),    I8CFGX(256, 64, 64, 4, 1),   I8CFGX(256, 64, 128, 4, 1),
    I8CFGR(64, 64, 64, 2, 2),    I8CFGR(128, 64, 64, 2, 2),   I8CFGR(64, 128, 64, 2, 2),
    I8CFGR(128, 128, 64, 2, 2),  I8CFGR(64, 64, 128, 2, 2),   I8CFGR(128, 64, 128, 2, 2),
    I8CFGR(256, 64, 64, 4, 1),   I8CFGR(256, 64, 128, 4, 1),
    I8CFGX(128, 64, 64, 4, 1),   I8CFGX(128, 64, 128, 4, 1),  I8CFGX(128, 128, 64, 4, 1),
    I8CFGX(128, 128, 128, 4, 1), I8CFGR(128, 64, 64, 4, 1),   I8CFGR(128, 64, 128, 4, 1),
};
#undef I8CFG
#undef I8CFGP
#undef I8CFGX
#undef I8CFGR
constexpr int kNumI8Cfgs = sizeof(kI8Cfgs) / sizeof(kI8Cfgs[0]);

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// K layout of a layer: 16-byte groups and where each sits in padded NHWC.
struct I8Layout {
    int Cp;        // channel stride of xq (bytes per pixel)
    bool runs;     // dilation-1 kernel rows as contiguous (kw, c) runs
    int run_groups;  // groups per kernel row (runs) or per tap
    int groups;    // total 16-byte groups of K
    int Hp, Wp, pt, pl;
    // bytes from a column's window origin to where xq's padding puts it:
    // 0 for a buffer padded for this conv; an int8 tensor padded for a wider
    // reader (pt > ph or pl > pw) shifts every window by the difference
    int origin = 0;
};

// The layout of a conv reading an int8 activation tensor in place: the
// tensor's padded NHWC buffer (its halo at least this conv's padding and
// wide enough for its windows, as setup_q8_tensors sizes it).
I8Layout i8_layout_q8(const ConvGeom &g, const Spkv2Q8Tensor &t) {
    I8Layout L{};
    L.runs = g.dw == 1;
    L.Cp = t.Cp;
    L.run_groups = L.runs ? static_cast<int>((static_cast<size_t>(g.KW) * L.Cp + 15) / 16) : L.Cp / 16;
    L.groups = L.runs ? g.KH * L.run_groups : g.KH * g.KW * L.run_groups;
    L.Hp = t.Hp;
    L.Wp = t.Wp;
    L.pt = t.pt;
    L.pl = t.pl;
    L.origin = ((t.pt - g.ph) * t.Wp + (t.pl - g.pw)) * t.Cp;
    return L;
}

I8Layout i8_layout(const ConvGeom &g) {
    I8Layout L{};
    L.runs = g.dw == 1;
    L.Cp = L.runs ? static_cast<int>(align_up(g.C, 4)) : static_cast<int>(align_up(g.C, 16));
    L.run_groups = L.runs ? static_cast<int>(align_up(static_cast<size_t>(g.KW) * L.Cp, 16) / 16) : L.Cp / 16;
    L.groups = L.runs ? g.KH * L.run_groups : g.KH * g.KW * L.run_groups;
    const int hspan = (g.OH - 1) * g.sh + (g.KH - 1) * g.dh + 1;
    const int wspan = (g.OW - 1) * g.sw + (g.KW - 1) * g.dw + 1;
    L.pt = g.ph;
    L.pl = g.pw;
    L.Hp = std::max(g.H + g.ph, hspan);
    L.Wp = std::max(g.W + g.pw, wspan);
    return L;
}

// Whether configuration c can run a layer: the BMAP 1 gather needs the
// BK/16 groups of every k-tile contiguous in xq, i.e. no tile crosses from
// one kernel row (or tap) to the next.  A tile past the last group reads
// memory beyond the layer's K, which meets zero weights.
bool i8_cfg_fits(const I8Layout &L, int c) {
    const I8Cfg &t = kI8Cfgs[c];
    if (!t.bmap) return true;
    const int G = t.BK / 16;
    return L.run_groups % G == 0 || L.groups == L.run_groups;
}

// byte offset of group q relative to the window origin in padded NHWC
int i8_group_offset(const ConvGeom &g, const I8Layout &L, int q) {
    if (L.runs) {
        const int kh = q / L.run_groups, r = q % L.run_groups;
        return kh * g.dh * L.Wp * L.Cp + r * 16;
    }
    const int tap = q / L.run_groups, c16 = q % L.run_groups;
    const int kh = tap / g.KW, kw = tap % g.KW;
    return (kh * g.dh * L.Wp + kw * g.dw) * L.Cp + c16 * 16;
}

// weight of packed k byte kb (group kb/16, byte kb%16) for output channel m
int8_t i8_weight_at(const ConvGeom &g, const I8Layout &L, const int8_t *w, int m, int kb) {
    const int q = kb / 16, b = kb % 16;
    int kh, kw, c;
    if (L.runs) {
        kh = q / L.run_groups;
        const int byte = (q % L.run_groups) * 16 + b;
        kw = byte / L.Cp;
        c = byte % L.Cp;
        if (kw >= g.KW) return 0;
    } else {
        const int tap = q / L.run_groups;
        kh = tap / g.KW;
        kw = tap % g.KW;
        c = (q % L.run_groups) * 16 + b;
    }
    if (kh >= g.KH || c >= g.C) return 0;
    return w[((static_cast<size_t>(m) * g.C + c) * g.KH + kh) * g.KW + kw];
}

struct I8Counts {
    int m_tiles, n_tiles, k_tiles, kt_per_split, splitk;
};

I8Counts i8_counts(int c, int M, int Ntot, int Kbytes, int split) {
    const I8Cfg &t = kI8Cfgs[c];
    I8Counts tc;
    tc.m_tiles = (M + t.BM - 1) / t.BM;
    tc.n_tiles = (Ntot + t.BN - 1) / t.BN;
    tc.k_tiles = (Kbytes + t.BK - 1) / t.BK;
    tc.kt_per_split = (tc.k_tiles + split - 1) / split;
    tc.splitk = (tc.k_tiles + tc.kt_per_split - 1) / tc.kt_per_split;
    return tc;
}

int cu_count() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        hipDeviceProp_t p;
        cus = (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&p, dev) == hipSuccess)
                  ? p.multiProcessorCount
                  : 256;
    }
    return cus;
}

// Modelled time (us): int8 MFMA work of the busiest CU (two workgroups per
// CU share it), floored by one workgroup's serial k loop, plus split-K
// partial traffic.  Prunes what the tuner times.
double i8_model_us(int c, const I8Counts &tc, int M, int Ntot) {
    const I8Cfg &t = kI8Cfgs[c];
    const int cus = cu_count();
    const long wgs = static_cast<long>(tc.m_tiles) * tc.n_tiles * tc.splitk;
    const long rounds = (wgs + 2L * cus - 1) / (2L * cus);
    const long per_cu = std::min<long>(2, (wgs + cus - 1) / cus);
    const double tile_us = 2.0 * t.BM * t.BN * t.BK / (8192.0 * 2400.0 * 0.85);
    const double mfma = static_cast<double>(rounds) * per_cu * tc.kt_per_split * tile_us;
    const double latency = static_cast<double>(rounds) * tc.kt_per_split * 0.5;
    double us = std::max(mfma, latency) + 2.0;
    if (tc.splitk > 1) us += 4.0 * M * static_cast<double>(Ntot) * (tc.splitk + 1) / 4.0e6 + 3.0;
    return us;
}

const int kI8Splits[] = {1, 2, 3, 4, 6, 8, 12, 16};

size_t i8_partial_bytes(const I8Counts &tc, int M, int Ntot) {
    return tc.splitk > 1 ? static_cast<size_t>(tc.splitk) * M * Ntot * sizeof(int32_t) : 0;
}

// (m, s) of div_fast for divisor d >= 1 (dividends below 2^31)
void div_magic(unsigned d, unsigned *m, int *s) {
    int l = 0;
    while ((uint64_t(1) << l) < d) l++;
    *s = 31 + l;
    *m = static_cast<unsigned>(((uint64_t(1) << *s) + d - 1) / d);
}

void fill_i8_args(I8Args &a, const ConvGeom &g, const I8Layout &L, const I8Counts &tc) {
    a.x_bytes = static_cast<int>(static_cast<size_t>(g.N) * L.Hp * L.Wp * L.Cp);
    a.y_bytes = static_cast<int>(g.y_elems * 4);
    a.img_stride = L.Hp * L.Wp * L.Cp;
    a.Wp = L.Wp;
    a.Cp = L.Cp;
    a.M = g.M;
    a.OW = g.OW;
    a.OHW = g.OH * g.OW;
    a.Ntot = g.N * a.OHW;
    div_magic(static_cast<unsigned>(a.OHW), &a.ohw_m, &a.ohw_s);
    div_magic(static_cast<unsigned>(a.OW), &a.ow_m, &a.ow_s);
    a.sh = g.sh;
    a.sw = g.sw;
    a.m_tiles = tc.m_tiles;
    a.k_tiles = tc.k_tiles;
    a.kt_per_split = tc.kt_per_split;
    a.act = g.act;
}

// Launches the GEMM (and the split-K epilogue) of configuration c.
// Workgroups of a persistent kernel: as many as the GPU holds at once (the
// occupancy calculator's figure per CU times the CUs), a multiple of 8 (one
// share per XCD), and no more than the tiles need.
unsigned persistent_grid(I8Kernel kern, int tiles) {
    static std::mutex mu;
    static std::map<I8Kernel, int> per_cu;
    int occ = 0;
    {
        std::lock_guard<std::mutex> lk(mu);
        auto it = per_cu.find(kern);
        if (it == per_cu.end()) {
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, 256, 0) != hipSuccess || occ < 1) {
                (void)hipGetLastError();
                occ = 1;
            }
            per_cu[kern] = occ;
        } else {
            occ = it->second;
        }
    }
    const long resident = static_cast<long>(cu_count()) * occ;
    const long need = (static_cast<long>(tiles) + 7) / 8 * 8;
    return static_cast<unsigned>(std::max(8L, std::min(resident / 8 * 8, need)));
}

int launch_i8(hipStream_t st, int c, const I8Counts &tc, I8Args a, int32_t *part, int32_t *raw) {
    const bool split = tc.splitk > 1;
    if (split) {
        a.mode = 1;
        a.ws = part;
        a.ws_bytes = static_cast<int>(i8_partial_bytes(tc, a.M, a.Ntot));
    } else if (raw) {
        a.mode = 2;
        a.ws = raw;
        a.ws_bytes = a.y_bytes;
    } else {
        a.mode = 0;
    }
    const I8Kernel kern = a.q8 ? kI8Cfgs[c].kernel_q8 : kI8Cfgs[c].kernel;
    dim3 grid(static_cast<unsigned>(tc.m_tiles * tc.n_tiles), static_cast<unsigned>(tc.splitk));
    if (kI8Cfgs[c].persist) {
        if (split) return SPKV2_E_UNSUPPORTED;  // the persistent kernels take whole tiles
        grid = dim3(persistent_grid(kern, tc.m_tiles * tc.n_tiles), 1);
    }
    kern<<<grid, dim3(256), 0, st>>>(a);
    if (int rc = launch_status("conv_igemm_i8")) return rc;
    if (split) {
        const size_t total = static_cast<size_t>(a.M) * a.Ntot;
        if (a.Ntot % 4 == 0)
            hipLaunchKernelGGL(splitk_i8_epilogue<4>, dim3(grid_for(total / 4, 256)), dim3(256), 0, st, part, tc.splitk,
                               a.M, a.Ntot, a.OHW, a.scales, a.bias, a.res, a.y, raw, a.act, a);
        else
            hipLaunchKernelGGL(splitk_i8_epilogue<1>, dim3(grid_for(total, 256)), dim3(256), 0, st, part, tc.splitk,
                               a.M, a.Ntot, a.OHW, a.scales, a.bias, a.res, a.y, raw, a.act, a);
        if (int rc = launch_status("splitk_i8_epilogue")) return rc;
    }
    return 0;
}

std::vector<int> build_i8_koff(const ConvGeom &g, const I8Layout &L, int k_tiles, int BK) {
    const int per_tile = BK / 16;
    // two extra tiles of out-of-range entries: the pipeline prefetches up to
    // two tiles past the last one
    std::vector<int> koff(static_cast<size_t>((k_tiles + 2) * per_tile), kOob);
    for (int q = 0; q < L.groups; q++) koff[q] = L.origin + i8_group_offset(g, L, q);
    return koff;
}


struct DevBufs {
    std::vector<void *> p;
    void *get(size_t n) {
        void *q = nullptr;
        if (hipMalloc(&q, n ? n : 16) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        p.push_back(q);
        return q;
    }
    ~DevBufs() {
        for (void *q : p) (void)hipFree(q);
    }
};

// Times the candidates the model keeps on zero-filled scratch buffers of the
// layer's shape and returns the fastest (cfg, split); cached per shape.
// q8: the INT8 configuration's epilogue (int8 output and residual) is timed,
// and the choice is kept under its own key.
bool tune_i8(hipStream_t st, const ConvGeom &g, const I8Layout &L, int *cfg_out, int *split_out, bool q8 = false) {
    char key[256];
    snprintf(key, sizeof(key), "i8|%d,%d,%d,%d|%d,%d,%d,%d,%d,%d,%d,%d,%d|%d,%d,%d%s", g.N, g.C, g.H, g.W, g.M, g.KH,
             g.KW, g.OH, g.OW, g.sh, g.sw, g.dh, g.dw, g.has_bias ? 1 : 0, g.has_res ? 1 : 0, g.act, q8 ? "|q8" : "");
    // a stored choice is taken only if this layer's K layout allows it (a
    // tune DB written by another build may name another configuration)
    if (tuned_lookup(key, cfg_out, split_out) && *cfg_out >= 0 && *cfg_out < kNumI8Cfgs && i8_cfg_fits(L, *cfg_out))
        return true;
    const int Ntot = g.N * g.OH * g.OW;
    const int Kbytes = L.groups * 16;
    struct Cand {
        int cfg, split;
        I8Counts tc;
        double model, t;
    };
    std::vector<Cand> cands;
    double best = 1e300;
    for (int c = 0; c < kNumI8Cfgs; c++) {
        if (!i8_cfg_fits(L, c)) continue;
        int last = -1;
        for (int s : kI8Splits) {
            if (s > 1 && kI8Cfgs[c].persist) break;  // whole tiles only
            const I8Counts tc = i8_counts(c, g.M, Ntot, Kbytes, s);
            if (tc.splitk == last) continue;
            if (s > 1 && tc.kt_per_split < 2) break;
            last = tc.splitk;
            if (i8_partial_bytes(tc, g.M, Ntot) > (size_t(1) << 29)) continue;
            const double m = i8_model_us(c, tc, g.M, Ntot);
            best = std::min(best, m);
            cands.push_back({c, s, tc, m, 0.0});
        }
    }
    std::vector<Cand> keep;
    for (const Cand &cd : cands)
        if (cd.model <= 3.0 * best) keep.push_back(cd);
    if (keep.empty()) return false;
    DevBufs db;
    size_t wbytes = 16, pbytes = 16, kentries = 16;
    for (const Cand &cd : keep) {
        const I8Cfg &t = kI8Cfgs[cd.cfg];
        wbytes = std::max(wbytes, static_cast<size_t>(cd.tc.m_tiles) * cd.tc.k_tiles * t.BM * t.BK);
        pbytes = std::max(pbytes, i8_partial_bytes(cd.tc, g.M, Ntot));
        kentries = std::max(kentries, static_cast<size_t>((cd.tc.k_tiles + 2) * t.BK / 16));
    }
    const size_t xbytes = static_cast<size_t>(g.N) * L.Hp * L.Wp * L.Cp;
    const size_t ybytes = static_cast<size_t>(g.y_elems) * 4;
    int8_t *xq = static_cast<int8_t *>(db.get(xbytes));
    int8_t *wp = static_cast<int8_t *>(db.get(wbytes));
    int *ko = static_cast<int *>(db.get(kentries * sizeof(int)));
    float *sc = static_cast<float *>(db.get(static_cast<size_t>(g.M) * 4));
    float *y = static_cast<float *>(db.get(ybytes));
    float *res = g.has_res ? static_cast<float *>(db.get(ybytes)) : nullptr;
    int32_t *part = static_cast<int32_t *>(db.get(pbytes));
    if (!xq || !wp || !ko || !sc || !y || (g.has_res && !res) || !part) return false;
    // q8: an int8 output (and residual) of the layer's shape, unpadded, and
    // constant rows whose values do not matter for the timing
    const int q_Cp = static_cast<int>(align_up(static_cast<size_t>(g.M), 16));
    const size_t q_bytes = static_cast<size_t>(g.N) * g.OH * g.OW * q_Cp;
    int8_t *q_out = q8 ? static_cast<int8_t *>(db.get(q_bytes)) : nullptr;
    int8_t *q_res = q8 && g.has_res ? static_cast<int8_t *>(db.get(q_bytes)) : nullptr;
    int *qrow = q8 ? static_cast<int *>(db.get(static_cast<size_t>(7) * g.M * sizeof(int))) : nullptr;
    if (q8 && (!q_out || (g.has_res && !q_res) || !qrow)) return false;
    if (qrow) {
        std::vector<int> rows(static_cast<size_t>(7) * g.M, 0);
        for (int m = 0; m < g.M; m++) {
            rows[2 * g.M + m] = 1 << 30;  // m1: multiplier 2^-10 at shift 40 (the high-word path)
            rows[4 * g.M + m] = 40;
            rows[5 * g.M + m] = 1 << 7;
            rows[6 * g.M + m] = 8;
        }
        if (hipMemcpy(qrow, rows.data(), rows.size() * sizeof(int), hipMemcpyHostToDevice) != hipSuccess) {
            (void)hipGetLastError();
            return false;
        }
    }
    if (q_res) (void)hipMemsetAsync(q_res, 0, q_bytes, st);
    (void)hipMemsetAsync(xq, 0, xbytes, st);
    (void)hipMemsetAsync(wp, 0, wbytes, st);
    (void)hipMemsetAsync(sc, 0, static_cast<size_t>(g.M) * 4, st);
    if (res) (void)hipMemsetAsync(res, 0, ybytes, st);
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    std::vector<int> last_kv;
    int last_bk = -1;
    bool ok = true;
    auto time_it = [&](const Cand &cd, int reps) -> double {
        const I8Cfg &t = kI8Cfgs[cd.cfg];
        const std::vector<int> kv = build_i8_koff(g, L, cd.tc.k_tiles, t.BK);
        if (t.BK != last_bk || kv.size() != last_kv.size()) {
            if (hipMemcpy(ko, kv.data(), kv.size() * sizeof(int), hipMemcpyHostToDevice) != hipSuccess) return 1e300;
            last_kv = kv;
            last_bk = t.BK;
        }
        I8Args a{};
        fill_i8_args(a, g, L, cd.tc);
        a.xq = xq;
        a.wp = wp;
        a.koff = ko;
        a.scales = sc;
        a.bias = g.has_bias ? sc : nullptr;
        a.res = res;
        a.y = y;
        if (q8) {
            a.q8 = 1;
            a.q8_hi = 1;
            a.qrow = qrow;
            a.scales = nullptr;
            a.bias = nullptr;
            a.res = nullptr;
            a.y = nullptr;
            a.q_out = q_out;
            a.q_bytes = static_cast<int>(q_bytes);
            a.q_Hp = g.OH;
            a.q_Wp = g.OW;
            a.q_Cp = q_Cp;
            a.r8 = q_res;
            a.r_bytes = q_res ? static_cast<int>(q_bytes) : 0;
            a.r_Hp = g.OH;
            a.r_Wp = g.OW;
            a.r_Cp = q_Cp;
        }
        if (hipEventRecord(e0, st) != hipSuccess) return 1e300;
        for (int r = 0; r < reps; r++)
            if (launch_i8(st, cd.cfg, cd.tc, a, part, nullptr) != 0) return 1e300;
        if (hipEventRecord(e1, st) != hipSuccess || hipEventSynchronize(e1) != hipSuccess) return 1e300;
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, e0, e1) != hipSuccess) return 1e300;
        return 1e3 * ms / reps;
    };
    for (Cand &cd : keep) {
        (void)time_it(cd, 1);
        cd.t = time_it(cd, 1);
        if (cd.t >= 1e300) ok = false;
    }
    std::sort(keep.begin(), keep.end(), [](const Cand &x, const Cand &y2) { return x.t < y2.t; });
    const size_t fin = std::min<size_t>(keep.size(), 3);
    for (size_t i = 0; i < fin && ok; i++) keep[i].t = std::min(keep[i].t, time_it(keep[i], 3));
    std::sort(keep.begin(), keep.begin() + fin, [](const Cand &x, const Cand &y2) { return x.t < y2.t; });
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (!ok || hipStreamSynchronize(st) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    *cfg_out = keep[0].cfg;
    *split_out = keep[0].split;
    tuned_store(key, keep[0].cfg, keep[0].split);
    return true;
}

}  // namespace

// Requantize handoff.  When this int8 conv's input is the only output of an
// earlier int8 conv, that conv quantizes its result in registers (with this
// conv's scale and rounding split) straight into a zero-padded NHWC buffer
// owned by this plan, and this conv skips its quantize pass.  A later int8
// consumer of the same tensor whose quantization is identical (same scale,
// rounding split and padded layout: e.g. the 1x1 stride-2 projection beside
// the next block's 1x1 conv) reads that same buffer.  The producer still
// writes the fp32 tensor when anything else reads it (a consumer served by
// neither, a graph output).  Packages with a protection plan keep every
// tensor materialized and do not hand off.
// Joins this conv to its producer's int8 handoff: the producer (an int8 conv
// or a MaxPool, plan type P, both with the q_* fields) writes the quantized
// input straight into this conv's padded NHWC buffer.  The first consumer
// owns the buffer; a later one with identical quantization shares it.
template <class P>
static int join_handoff(P *pp, ConvPlan *plan, const I8Layout &L, int readers, bool is_output) {
    const ConvGeom &g = plan->g;
    const float inv = 1.0f / plan->x_scale;  // reference conv_int8.c:23
    if (pp->q_out) {
        // the tensor is already handed off to an earlier consumer: share its
        // buffer when this conv would quantize to exactly the same bytes
        if (pp->q_Hp != L.Hp || pp->q_Wp != L.Wp || pp->q_Cp != L.Cp || pp->q_pt != L.pt || pp->q_pl != L.pl ||
            pp->q_split != plan->quant_split || __builtin_bit_cast(uint32_t, pp->q_inv_scale) != __builtin_bit_cast(uint32_t, inv))
            return 0;
        plan->q_shared = pp->q_out;
        pp->q_readers++;
        pp->y_needed = readers > pp->q_readers || is_output;
        return 0;
    }
    const size_t bytes = static_cast<size_t>(g.N) * L.Hp * L.Wp * L.Cp;
    if (int rc = hip_check(hipMalloc(reinterpret_cast<void **>(&plan->q_in), bytes), "hipMalloc int8 handoff"))
        return rc;
    // zero once: the producer writes only the interior, so the halo and the
    // padded channels stay 0
    if (int rc = hip_check(hipMemset(plan->q_in, 0, bytes), "hipMemset int8 handoff")) return rc;
    pp->q_out = plan->q_in;
    pp->q_Hp = L.Hp;
    pp->q_Wp = L.Wp;
    pp->q_Cp = L.Cp;
    pp->q_pt = L.pt;
    pp->q_pl = L.pl;
    pp->q_split = plan->quant_split;
    pp->q_inv_scale = inv;
    pp->q_readers = 1;
    pp->y_needed = readers > pp->q_readers || is_output;
    return 0;
}

static int setup_handoff(Spkv2Context *ctx, const Spkv2NodeRecord *node, ConvPlan *plan, const I8Layout &L) {
    if (ctx->protection_count > 0) return 0;
    if (const char *e = getenv("SPKV2_I8_HANDOFF"))
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
    if (!prod || prod->output_count != 1) return 0;
    if (!builtin_runs(ctx, prod->id) || !builtin_runs(ctx, node->id)) return 0;  // a user kernel runs one end
    bool is_output = false;
    for (size_t i = 0; i < ctx->output_count; i++)
        if (ctx->output_ids[i] == t) is_output = true;
    const ConvGeom &g = plan->g;
    if (prod->op_type == SPKV2_OP_MAXPOOL) {
        // prepared by the built-in MaxPool as a fused pooling + quantization
        // candidate: 64-channel blocks, 16-byte pixel stores
        if (ctx->plan_dtors[prod->id] != pool_plan_free) return 0;
        PoolPlan *pp = static_cast<PoolPlan *>(ctx->plans[prod->id]);
        if (!pp || L.Cp != g.C || g.C % 64 != 0) return 0;
        return join_handoff(pp, plan, L, readers, is_output);
    }
    if (prod->op_type != SPKV2_OP_CONV) return 0;
    if (ctx->plan_dtors[prod->id] != conv_plan_free) return 0;
    ConvPlan *pp = static_cast<ConvPlan *>(ctx->plans[prod->id]);
    if (!pp || pp->path != CONV_IGEMM_I8) return 0;
    if (pp->g.N != g.N || pp->g.M != g.C || pp->g.OH != g.H || pp->g.OW != g.W) return 0;
    return join_handoff(pp, plan, L, readers, is_output);
}

// The INT8 configuration's per-channel requantization constants (the same
// definition as the oracle's restatement): bias_q = round_half_away(b /
// (s_x s_w)) clamped to +-2^30; m1 ~ (s_x s_w / s_y) 2^S and m2 ~ (s_r /
// s_y) 2^S with S = 31 - e for max(ratio) = f 2^e, f in [0.5, 1), one less
// if a multiplier rounds to 2^31.  Rows of qrow: -z_x sum(w), that plus
// bias_q, m1, m2, S, and for q8_requant_hi 2^(S-33) and S - 32.  False when
// a shift leaves [1, 62].
bool q8_requant_rows(const ConvGeom &g, const int8_t *w, const float *ws, float sx, int zx, float sy, int zy,
                     float sr, const float *bias, std::vector<int> &rows) {
    const int M = g.M;
    const size_t K = static_cast<size_t>(g.C) * g.KH * g.KW;
    rows.assign(static_cast<size_t>(7) * M, 0);
    for (int m = 0; m < M; m++) {
        int64_t wsum = 0;
        for (size_t k = 0; k < K; k++) wsum += w[m * K + k];
        const double r1 = (static_cast<double>(sx) * static_cast<double>(ws[m])) / static_cast<double>(sy);
        const double r2 = sr > 0.0f ? static_cast<double>(sr) / static_cast<double>(sy) : 0.0;
        int e = 0;
        (void)std::frexp(std::max(r1, r2), &e);
        int sh = 31 - e;
        double a1 = std::floor(std::ldexp(r1, sh) + 0.5), a2 = std::floor(std::ldexp(r2, sh) + 0.5);
        if (a1 >= 2147483648.0 || a2 >= 2147483648.0) {
            sh -= 1;
            a1 = std::floor(std::ldexp(r1, sh) + 0.5);
            a2 = std::floor(std::ldexp(r2, sh) + 0.5);
        }
        if (sh < 1 || sh > 62) return false;
        double bq = 0.0;
        if (bias) {
            const double v = static_cast<double>(bias[m]) / (static_cast<double>(sx) * static_cast<double>(ws[m]));
            bq = v >= 0.0 ? std::floor(v + 0.5) : -std::floor(-v + 0.5);
            bq = std::min(std::max(bq, -1073741824.0), 1073741824.0);
        }
        const int zw = static_cast<int>(-static_cast<int64_t>(zx) * wsum);
        rows[m] = zw;
        rows[M + m] = zw + static_cast<int>(bq);
        rows[2 * M + m] = static_cast<int>(a1);
        rows[3 * M + m] = static_cast<int>(a2);
        rows[4 * M + m] = sh;
        // the high-word form's rounding constant with z_y folded in, and shift
        rows[5 * M + m] = sh >= 33 && sh <= 55 ? (1 << (sh - 33)) + zy * (1 << (sh - 32)) : 0;
        rows[6 * M + m] = sh - 32;
    }
    return true;
}

int conv_i8_prepare(Spkv2Context *ctx, const Spkv2NodeRecord *node, ConvPlan *plan) {
    const ConvGeom &g = plan->g;
    // the INT8 configuration with int8 tensors between nodes: the input is
    // an int8 tensor (or fp32, quantized asymmetrically on load), the output
    // an int8 tensor, the residual (if any) an int8 tensor
    const Spkv2Q8Tensor *tx = q8_tensor(ctx, node->inputs[0]);
    const Spkv2Q8Tensor *ty = q8_tensor(ctx, node->outputs[0]);
    const Spkv2Q8Tensor *tr = g.has_res ? q8_tensor(ctx, node->inputs[3]) : nullptr;
    const bool q8 = tx || ty;
    if (g.group != 1 || (!tx && g.x_dtype != SPKV2_DTYPE_FP32)) return SPKV2_E_UNSUPPORTED;
    if (q8 && (!ty || (g.has_res && !tr) || (g.act != 0 && g.act != 1))) {
        set_last_error_text("conv node " + std::to_string(node->id) +
                            ": int8 tensors between nodes need an int8 output, an int8 residual and no SiLU");
        return SPKV2_E_UNSUPPORTED;
    }
    if (tr && (tr->N != g.N || tr->C != g.M || tr->H != g.OH || tr->W != g.OW)) return -11;
    const Spkv2QuantParamRecord *wq = spkv2_ctx_find_quant_param(ctx, node->inputs[1]);
    const Spkv2QuantParamRecord *xq = spkv2_ctx_find_quant_param(ctx, node->inputs[0]);
    if (!wq || !xq) return SPKV2_E_QUANT;
    const float *ws = spkv2_ctx_quant_scales(ctx, wq);
    const float *xs = spkv2_ctx_quant_scales(ctx, xq);
    if (!ws || !xs || static_cast<int>(wq->num_channels) < g.M || xq->num_channels < 1) return SPKV2_E_QUANT;
    const int8_t *w = reinterpret_cast<const int8_t *>(host_weight_data(ctx, node->inputs[1]));
    if (!w) return SPKV2_E_UNSUPPORTED;
    int zx = 0;
    if (q8) {
        float sx = 0.0f;
        if (int rc = q8_params(ctx, node->inputs[0], &sx, &zx)) return rc;
    }

    const I8Layout L = tx ? i8_layout_q8(g, *tx) : i8_layout(g);
    // an int8 input is read in place: only the fp32 input needs the workspace copy
    const size_t xq_bytes = static_cast<size_t>(g.N) * L.Hp * L.Wp * L.Cp;
    if (xq_bytes >= 0x7fff0000ULL) return SPKV2_E_UNSUPPORTED;  // byte offsets are 31-bit
    plan->path = q8 ? CONV_Q8 : CONV_IGEMM_I8;
    plan->x_zp = zx;
    plan->x_scale = xs[0];
    plan->Hp = L.Hp;
    plan->Wp = L.Wp;
    plan->pt = L.pt;
    plan->pl = L.pl;
    const int Ntot = g.N * g.OH * g.OW;
    const int Kbytes = L.groups * 16;

    int cfg = 0, split = 1;
    const char *tune_env = getenv("SPKV2_CONV_TUNE");
    if ((tune_env && tune_env[0] == '0') || !tune_i8(ctx->stream, g, L, &cfg, &split, q8)) {
        double best = 1e300;
        for (int c = 0; c < kNumI8Cfgs; c++)
            for (int s : kI8Splits) {
                if (!i8_cfg_fits(L, c) || (s > 1 && kI8Cfgs[c].persist)) break;
                const I8Counts tc = i8_counts(c, g.M, Ntot, Kbytes, s);
                if (s > 1 && tc.kt_per_split < 2) break;
                const double m = i8_model_us(c, tc, g.M, Ntot);
                if (m < best * 0.999) {
                    best = m;
                    cfg = c;
                    split = s;
                }
            }
    }
    if (const char *e = getenv("SPKV2_I8_CFG")) {
        const int c = atoi(e);
        if (c >= 0 && c < kNumI8Cfgs) {
            if (!i8_cfg_fits(L, c)) {
                set_last_error_text("SPKV2_I8_CFG names a configuration whose gather this layer's K layout does not allow");
                return SPKV2_E_UNSUPPORTED;
            }
            cfg = c;
        }
    }
    if (const char *e = getenv("SPKV2_I8_SPLITK")) {
        const int s = atoi(e);
        if (s >= 1 && s <= 64) split = s;
    }
    if (kI8Cfgs[cfg].persist) split = 1;  // the persistent kernels take whole tiles
    const I8Cfg &t = kI8Cfgs[cfg];
    const I8Counts tc = i8_counts(cfg, g.M, Ntot, Kbytes, split);
    plan->cfg = cfg;
    plan->K = Kbytes;
    plan->BM = t.BM;
    plan->BN = t.BN;
    plan->BK = t.BK;
    plan->m_tiles = tc.m_tiles;
    plan->n_tiles = tc.n_tiles;
    plan->k_tiles = tc.k_tiles;
    plan->Kpad = tc.k_tiles * t.BK;
    plan->kt_per_split = tc.kt_per_split;
    plan->splitk = tc.splitk;
    // partials also serve the raw-accumulator hook when the layer splits K
    const size_t part_bytes = i8_partial_bytes(tc, g.M, Ntot);
    // partial offsets (slice, row, out-of-range column) must stay below 2^32
    if (part_bytes >= 0x40000000ULL) return SPKV2_E_UNSUPPORTED;
    plan->pad_bytes = tx ? 0 : align_up(xq_bytes + 64, 256);
    plan->workspace = plan->pad_bytes + part_bytes;

    // activation quantization constants (reference conv_int8.c:22-23)
    plan->quant_split = static_cast<int>((static_cast<int64_t>(g.C) * g.H * g.W / 16) * 16);

    // weights packed per (m_tile, k_tile) in the layer's k order: [BM][BK]
    // rows, or for conv_igemm_i8x in MFMA fragment order [BM/32][BK/32][64
    // lanes][16 bytes], lane = 32 * (16-byte half of the k step) + row % 32
    std::vector<int8_t> packed(static_cast<size_t>(tc.m_tiles) * tc.k_tiles * t.BM * t.BK, 0);
    for (int m = 0; m < g.M; m++) {
        const int mt = m / t.BM, mi = m % t.BM;
        for (int kb = 0; kb < Kbytes; kb++) {
            const int kt = kb / t.BK, kk = kb % t.BK;
            const size_t tile = (static_cast<size_t>(mt) * tc.k_tiles + kt) * t.BM * t.BK;
            size_t at = static_cast<size_t>(mi) * t.BK + kk;
            if (t.adirect) {
                const int q = kk / 32, h = (kk % 32) / 16, b = kk % 16;
                at = ((static_cast<size_t>(mi / 32) * (t.BK / 32) + q) * 64 + h * 32 + mi % 32) * 16 + b;
            }
            packed[tile + at] = i8_weight_at(g, L, w, m, kb);
        }
    }
    if (int rc = hip_check(hipMalloc(&plan->wpack, packed.size()), "hipMalloc i8 weights")) return rc;
    if (int rc = hip_check(hipMemcpy(plan->wpack, packed.data(), packed.size(), hipMemcpyHostToDevice), "hipMemcpy"))
        return rc;
    const std::vector<int> koff = build_i8_koff(g, L, tc.k_tiles, t.BK);
    if (int rc = hip_check(hipMalloc(&plan->ktab, koff.size() * sizeof(int)), "hipMalloc i8 koff")) return rc;
    if (int rc = hip_check(hipMemcpy(plan->ktab, koff.data(), koff.size() * sizeof(int), hipMemcpyHostToDevice),
                           "hipMemcpy"))
        return rc;

    if (q8) {
        float sy = 0.0f, sr = 0.0f;
        int zy = 0, zr = 0;
        if (int rc = q8_params(ctx, node->outputs[0], &sy, &zy)) return rc;
        if (tr)
            if (int rc = q8_params(ctx, node->inputs[3], &sr, &zr)) return rc;
        const float *bias = g.has_bias ? reinterpret_cast<const float *>(host_weight_data(ctx, node->inputs[2])) : nullptr;
        if (g.has_bias && (!bias || rec(ctx, node->inputs[2])->dtype != SPKV2_DTYPE_FP32)) return SPKV2_E_UNSUPPORTED;
        // |acc + c| < 2^31 (the kernels add them in 32 bits): |sum w x| and
        // |z_x sum w| are each below 2^14 K, |bias_q| <= 2^30
        if (static_cast<int64_t>(g.C) * g.KH * g.KW > 32768) {
            set_last_error_text("conv node " + std::to_string(node->id) + ": K above 32768 in the INT8 configuration");
            return SPKV2_E_UNSUPPORTED;
        }
        std::vector<int> rows;
        if (!q8_requant_rows(g, w, ws, plan->x_scale, zx, sy, zy, sr, bias, rows)) {
            set_last_error_text("conv node " + std::to_string(node->id) + ": requantization shift out of range");
            return SPKV2_E_QUANT;
        }
        plan->q8_hi = true;
        for (int m = 0; m < g.M; m++) plan->q8_hi = plan->q8_hi && rows[4 * g.M + m] >= 33 && rows[4 * g.M + m] <= 55;
        if (int rc = hip_check(hipMalloc(reinterpret_cast<void **>(&plan->qrow), rows.size() * sizeof(int)), "hipMalloc"))
            return rc;
        if (int rc = hip_check(hipMemcpy(plan->qrow, rows.data(), rows.size() * sizeof(int), hipMemcpyHostToDevice),
                               "hipMemcpy"))
            return rc;
        set_kernel_name(ctx, node, std::string("conv_igemm_q8<") + t.name + (L.runs ? ",runs" : ",taps") +
                                       ",splitk=" + std::to_string(plan->splitk) + ">");
        return 0;
    }
    std::vector<float> comb(static_cast<size_t>(g.M));
    for (int m = 0; m < g.M; m++) comb[m] = ws[m] * plan->x_scale;  // reference conv_int8.c:93
    if (int rc = hip_check(hipMalloc(reinterpret_cast<void **>(&plan->scales), comb.size() * 4), "hipMalloc")) return rc;
    if (int rc = hip_check(hipMemcpy(plan->scales, comb.data(), comb.size() * 4, hipMemcpyHostToDevice), "hipMemcpy"))
        return rc;
    if (int rc = setup_handoff(ctx, node, plan, L)) return rc;
    set_kernel_name(ctx, node, std::string("conv_igemm_i8<") + t.name + (L.runs ? ",runs" : ",taps") +
                                   ",splitk=" + std::to_string(plan->splitk) + (plan->q_in ? ",handoff" : plan->q_shared ? ",shared" : "") + ">");
    return 0;
}

int conv_i8_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, const ConvPlan *plan, int32_t *raw_acc_out) {
    const ConvGeom &g = plan->g;
    const bool q8 = plan->path == CONV_Q8;
    const Spkv2Q8Tensor *tx = q8 ? q8_tensor(ctx, node->inputs[0]) : nullptr;
    const Spkv2Q8Tensor *ty = q8 ? q8_tensor(ctx, node->outputs[0]) : nullptr;
    const Spkv2Q8Tensor *tr = q8 && g.has_res ? q8_tensor(ctx, node->inputs[3]) : nullptr;
    if (q8 && (!ty || (g.has_res && !tr))) return SPKV2_E_UNSUPPORTED;
    uint8_t *wsb = plan_workspace(ctx, plan);
    if (!wsb && plan->workspace > 0) return SPKV2_E_UNSUPPORTED;
    const I8Layout L = tx ? i8_layout_q8(g, *tx) : i8_layout(g);
    int8_t *xq = reinterpret_cast<int8_t *>(wsb);
    int32_t *part = reinterpret_cast<int32_t *>(wsb + plan->pad_bytes);
    const float inv_scale = 1.0f / plan->x_scale;  // reference conv_int8.c:23

    // with the handoffs not live (a fault event armed, or the kernel registry
    // changed since prepare) every tensor is materialized and quantized here
    const bool handoff = handoffs_live(ctx);
    if (tx) {
        xq = tx->buf;  // an int8 tensor, read in place
    } else if ((plan->q_in || plan->q_shared) && handoff) {
        xq = plan->q_in ? plan->q_in : plan->q_shared;  // written by the producer's epilogue
    } else if (L.Cp <= 16) {
        const size_t pixels = static_cast<size_t>(g.N) * L.Hp * L.Wp;
        hipLaunchKernelGGL(quantize_pad_nhwc_narrow, dim3(grid_for(pixels, 256)), dim3(256), 0, ctx->stream,
                           dptr<const float>(ctx, node->inputs[0]), xq, g.C, g.H, g.W, L.Hp, L.Wp, L.Cp, L.pt, L.pl,
                           inv_scale, plan->quant_split, g.N, q8 ? plan->x_zp : 0, q8 ? 1 : 0);
        if (int rc = launch_status("quantize_pad_nhwc_narrow")) return rc;
    } else {
        dim3 qgrid(static_cast<unsigned>((L.Hp * L.Wp + 63) / 64), static_cast<unsigned>((L.Cp + 63) / 64),
                   static_cast<unsigned>(g.N));
        hipLaunchKernelGGL(quantize_pad_nhwc, qgrid, dim3(256), 0, ctx->stream, dptr<const float>(ctx, node->inputs[0]),
                           xq, g.C, g.H, g.W, L.Hp, L.Wp, L.Cp, L.pt, L.pl, inv_scale, plan->quant_split,
                           q8 ? plan->x_zp : 0, q8 ? 1 : 0);
        if (int rc = launch_status("quantize_pad_nhwc")) return rc;
    }

    const I8Counts tc{plan->m_tiles, plan->n_tiles, plan->k_tiles, plan->kt_per_split, plan->splitk};
    I8Args a{};
    fill_i8_args(a, g, L, tc);
    a.xq = xq;
    a.wp = static_cast<const int8_t *>(plan->wpack);
    a.koff = static_cast<const int *>(plan->ktab);
    if (q8) {
        a.q8 = 1;
        a.qrow = plan->qrow;
        a.q8_hi = plan->q8_hi ? 1 : 0;
        a.q_out = ty->buf;
        a.q_bytes = static_cast<int>(ty->bytes);
        a.q_Hp = ty->Hp;
        a.q_Wp = ty->Wp;
        a.q_Cp = ty->Cp;
        a.q_pt = ty->pt;
        a.q_pl = ty->pl;
        a.y_zp = ty->zp;
        if (tr) {
            a.r8 = tr->buf;
            a.r_bytes = static_cast<int>(tr->bytes);
            a.r_Hp = tr->Hp;
            a.r_Wp = tr->Wp;
            a.r_Cp = tr->Cp;
            a.r_pt = tr->pt;
            a.r_pl = tr->pl;
            a.r_zp = tr->zp;
        }
    } else {
        a.scales = plan->scales;
        a.bias = g.has_bias ? dptr<const float>(ctx, node->inputs[2]) : nullptr;
        a.res = g.has_res ? dptr<const float>(ctx, node->inputs[3]) : nullptr;
        a.y = dptr<float>(ctx, node->outputs[0]);
        if (plan->q_out && handoff) {
            a.q_out = plan->q_out;
            a.q_bytes = static_cast<int>(static_cast<size_t>(g.N) * plan->q_Hp * plan->q_Wp * plan->q_Cp);
            a.q_Hp = plan->q_Hp;
            a.q_Wp = plan->q_Wp;
            a.q_Cp = plan->q_Cp;
            a.q_pt = plan->q_pt;
            a.q_pl = plan->q_pl;
            a.q_split = plan->q_split;
            a.q_inv = plan->q_inv_scale;
            if (!plan->y_needed) a.y = nullptr;
        }
    }
    if (int rc = launch_i8(ctx->stream, plan->cfg, tc, a, part, raw_acc_out)) return rc;
    // accumulator capture: the same GEMM again on the same quantized input,
    // storing the raw int32 sums (the outputs above are already written)
    if (!raw_acc_out && node->id < ctx->acc_capture.size() && ctx->acc_capture[node->id])
        return launch_i8(ctx->stream, plan->cfg, tc, a, part, ctx->acc_capture[node->id]);
    return 0;
}

}  // namespace spk::kern
