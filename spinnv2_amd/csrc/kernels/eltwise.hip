// Memory-bound node kernels: binary/unary elementwise, copies, Concat, pools,
// Softmax, Reduce, Resize, plus the reliability helpers.  All are coalesced
// wavefront kernels: consecutive lanes touch consecutive addresses of the
// NCHW output, wide (float4) accesses where shapes allow, one wave per row for
// row reductions.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "common.hpp"
#include "conv.hpp"
#include "kernels.hpp"

namespace spk::kern {

namespace {

constexpr int kMaxRank = 8;

struct BcastDesc {
    int rank;
    int64_t ydim[kMaxRank];
    int64_t astride[kMaxRank];
    int64_t bstride[kMaxRank];
};

// Right-aligned numpy broadcasting of a and b onto y: size-1 dims get
// stride 0 (reference kernel_common.c:37-48).
void make_bcast(const Spkv2TensorRecord *a, const Spkv2TensorRecord *b, const Spkv2TensorRecord *y, BcastDesc *d) {
    d->rank = y->rank;
    for (int i = 0; i < kMaxRank; i++) d->ydim[i] = 1, d->astride[i] = 0, d->bstride[i] = 0;
    for (int i = 0; i < y->rank; i++) d->ydim[i] = y->shape[i];
    auto fill = [&](const Spkv2TensorRecord *t, int64_t *stride) {
        int64_t s = 1;
        const int delta = y->rank - t->rank;
        for (int i = t->rank - 1; i >= 0; i--) {
            stride[i + delta] = t->shape[i] == 1 ? 0 : s;
            s *= t->shape[i];
        }
    };
    fill(a, d->astride);
    fill(b, d->bstride);
}

enum BinOp { BIN_ADD = 0, BIN_MUL, BIN_SUB, BIN_DIV, BIN_MOD };

template <int OP>
__device__ __forceinline__ float bin(float a, float b) {
    if constexpr (OP == BIN_ADD) return a + b;
    if constexpr (OP == BIN_MUL) return a * b;
    if constexpr (OP == BIN_SUB) return a - b;
    if constexpr (OP == BIN_DIV) return a / b;
    // Mod as the reference computes it: C integer remainder of truncated
    // operands (reference math/binary.c:27); a zero divisor yields 0 here
    const int ib = static_cast<int>(b);
    return ib == 0 ? 0.0f : static_cast<float>(static_cast<int>(a) % ib);
}

template <int OP>
__global__ void __launch_bounds__(256) binary_same4(const float4 *__restrict__ a, const float4 *__restrict__ b,
                                                    float4 *__restrict__ y, size_t n4, int act) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n4; i += static_cast<size_t>(gridDim.x) * 256) {
        const float4 u = a[i], v = b[i];
        float4 r;
        r.x = apply_act(bin<OP>(u.x, v.x), act);
        r.y = apply_act(bin<OP>(u.y, v.y), act);
        r.z = apply_act(bin<OP>(u.z, v.z), act);
        r.w = apply_act(bin<OP>(u.w, v.w), act);
        y[i] = r;
    }
}

// The same-shape op over image-strided operands (channel slices of a
// Concat buffer): grid.y walks the images, grid.x the float4s of one image.
template <int OP>
__global__ void __launch_bounds__(256) binary_img4(const float4 *__restrict__ a, const float4 *__restrict__ b,
                                                   float4 *__restrict__ y, unsigned images, size_t per4, size_t as4,
                                                   size_t bs4, size_t ys4, int act) {
    for (unsigned img = blockIdx.y; img < images; img += gridDim.y)
        for (size_t j = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; j < per4;
             j += static_cast<size_t>(gridDim.x) * 256) {
            const float4 u = a[img * as4 + j], v = b[img * bs4 + j];
            float4 r;
            r.x = apply_act(bin<OP>(u.x, v.x), act);
            r.y = apply_act(bin<OP>(u.y, v.y), act);
            r.z = apply_act(bin<OP>(u.z, v.z), act);
            r.w = apply_act(bin<OP>(u.w, v.w), act);
            y[img * ys4 + j] = r;
        }
}

// The same over scalar elements, for views whose bases or image strides are
// not whole float4s (e.g. a channel offset times an odd plane size).
template <int OP>
__global__ void __launch_bounds__(256) binary_img1(const float *__restrict__ a, const float *__restrict__ b,
                                                   float *__restrict__ y, unsigned images, size_t per, size_t as,
                                                   size_t bs, size_t ys, int act) {
    for (unsigned img = blockIdx.y; img < images; img += gridDim.y)
        for (size_t j = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; j < per;
             j += static_cast<size_t>(gridDim.x) * 256)
            y[img * ys + j] = apply_act(bin<OP>(a[img * as + j], b[img * bs + j]), act);
}

template <int OP>
__global__ void __launch_bounds__(256) binary_bcast(const float *__restrict__ a, const float *__restrict__ b,
                                                    float *__restrict__ y, size_t n, BcastDesc d, int act) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256) {
        size_t t = i;
        int64_t ao = 0, bo = 0;
        for (int k = d.rank - 1; k >= 0; k--) {
            const int64_t c = static_cast<int64_t>(t % d.ydim[k]);
            t /= d.ydim[k];
            ao += c * d.astride[k];
            bo += c * d.bstride[k];
        }
        y[i] = apply_act(bin<OP>(a[ao], b[bo]), act);
    }
}

// One operand a single element (a tensor times a constant: YOLO's attention
// scale): 16-byte accesses, the reference's operand order kept
// (scalar_first: the scalar is the left operand).
template <int OP>
__global__ void __launch_bounds__(256) binary_scalar4(const float4 *__restrict__ t, const float *__restrict__ sc,
                                                      float4 *__restrict__ y, size_t n4, int act, int scalar_first) {
    const float c = *sc;
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n4; i += static_cast<size_t>(gridDim.x) * 256) {
        const float4 u = t[i];
        float4 r;
        r.x = apply_act(scalar_first ? bin<OP>(c, u.x) : bin<OP>(u.x, c), act);
        r.y = apply_act(scalar_first ? bin<OP>(c, u.y) : bin<OP>(u.y, c), act);
        r.z = apply_act(scalar_first ? bin<OP>(c, u.z) : bin<OP>(u.z, c), act);
        r.w = apply_act(scalar_first ? bin<OP>(c, u.w) : bin<OP>(u.w, c), act);
        y[i] = r;
    }
}

template <int OP>
int launch_binary(hipStream_t s, const Spkv2TensorRecord *ar, const Spkv2TensorRecord *br, const Spkv2TensorRecord *yr,
                  const float *a, const float *b, float *y, int act) {
    const size_t n = elem_count(yr);
    if (n == 0) return 0;
    const bool same = elem_count(ar) == n && elem_count(br) == n && ar->rank == yr->rank && br->rank == yr->rank;
    const bool aligned = ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                           reinterpret_cast<uintptr_t>(y)) & 15) == 0;
    const bool a_scalar = elem_count(ar) == 1 && elem_count(br) == n;
    const bool b_scalar = elem_count(br) == 1 && elem_count(ar) == n;
    const float *t = a_scalar ? b : a;
    const bool t_aligned = ((reinterpret_cast<uintptr_t>(t) | reinterpret_cast<uintptr_t>(y)) & 15) == 0;
    if (same && aligned && n % 4 == 0) {
        hipLaunchKernelGGL((binary_same4<OP>), dim3(grid_for(n / 4, 256)), dim3(256), 0, s,
                           reinterpret_cast<const float4 *>(a), reinterpret_cast<const float4 *>(b),
                           reinterpret_cast<float4 *>(y), n / 4, act);
    } else if ((a_scalar || b_scalar) && t_aligned && n % 4 == 0) {
        hipLaunchKernelGGL((binary_scalar4<OP>), dim3(grid_for(n / 4, 256)), dim3(256), 0, s,
                           reinterpret_cast<const float4 *>(t), a_scalar ? a : b, reinterpret_cast<float4 *>(y), n / 4,
                           act, a_scalar ? 1 : 0);
    } else {
        BcastDesc d;
        make_bcast(ar, br, yr, &d);
        hipLaunchKernelGGL((binary_bcast<OP>), dim3(grid_for(n, 256)), dim3(256), 0, s, a, b, y, n, d, act);
    }
    return launch_status("binary");
}

enum UnOp { UN_RELU = 0, UN_SIGMOID, UN_CLIP, UN_LEAKY };

// 1 / (1 + exp(-v)) on the hardware exponential and reciprocal, as the
// conv epilogues' SiLU: within a few ulp of the reference's expf and
// division, with its special values (+inf -> 1, -inf and v below about
// -88.7 -> 0, NaN -> NaN).
__device__ __forceinline__ float sigmoid_hw(float v) { return __builtin_amdgcn_rcpf(1.0f + __expf(-v)); }

// Sigmoid over 16-byte groups (n a multiple of 4, aligned operands).
__global__ void __launch_bounds__(256) sigmoid4(const float4 *__restrict__ x, float4 *__restrict__ y, size_t n4) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n4; i += static_cast<size_t>(gridDim.x) * 256) {
        const float4 u = x[i];
        y[i] = float4{sigmoid_hw(u.x), sigmoid_hw(u.y), sigmoid_hw(u.z), sigmoid_hw(u.w)};
    }
}

template <int OP>
__global__ void __launch_bounds__(256) unary_kernel(const float *__restrict__ x, float *__restrict__ y, size_t n,
                                                    const float *__restrict__ lo, const float *__restrict__ hi,
                                                    float alpha) {
    const float minv = (OP == UN_CLIP && lo) ? *lo : -INFINITY;
    const float maxv = (OP == UN_CLIP && hi) ? *hi : INFINITY;
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256) {
        float v = x[i];
        if constexpr (OP == UN_RELU) v = v > 0.0f ? v : 0.0f;                  // relu.c:11
        if constexpr (OP == UN_SIGMOID) v = sigmoid_hw(v);                      // sigmoid.c:11
        if constexpr (OP == UN_CLIP) {                                         // clip_leakyrelu.c:23-27
            if (v < minv) v = minv;
            if (v > maxv) v = maxv;
        }
        if constexpr (OP == UN_LEAKY) v = v >= 0.0f ? v : v * alpha;           // clip_leakyrelu.c:47
        y[i] = v;
    }
}

__global__ void __launch_bounds__(256) copy_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                                                   size_t n) {
    const size_t n16 = n / 16;
    const int4 *s4 = reinterpret_cast<const int4 *>(src);
    int4 *d4 = reinterpret_cast<int4 *>(dst);
    const size_t stride = static_cast<size_t>(gridDim.x) * 256;
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n16; i += stride) d4[i] = s4[i];
    for (size_t i = n16 * 16 + static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

__global__ void __launch_bounds__(256) copy_kernel_bytes(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                                                         size_t n) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256)
        dst[i] = src[i];
}

int launch_copy(hipStream_t s, const void *src, void *dst, size_t bytes) {
    if (bytes == 0 || src == dst) return 0;
    const bool aligned = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0;
    if (aligned)
        hipLaunchKernelGGL(copy_kernel, dim3(grid_for(bytes / 16 + 1, 256)), dim3(256), 0, s,
                           static_cast<const uint8_t *>(src), static_cast<uint8_t *>(dst), bytes);
    else
        hipLaunchKernelGGL(copy_kernel_bytes, dim3(grid_for(bytes, 256)), dim3(256), 0, s,
                           static_cast<const uint8_t *>(src), static_cast<uint8_t *>(dst), bytes);
    return launch_status("copy");
}

struct PoolArgs {
    const float *__restrict__ x;
    float *__restrict__ y;
    int N, C, H, W, OH, OW, kh, kw, sh, sw, ph, pw;
    size_t x_img, y_img;  // elements between images (maxpool_kernel; C*H*W and C*OH*OW unless views)
};

// reference pool/maxpool.c:20-40: -inf start, out-of-bounds taps skipped.
// grid.y strides over the N*C planes, grid.x over the outputs of a plane
// (32-bit index math).
__global__ void __launch_bounds__(256) maxpool_kernel(PoolArgs a) {
    const unsigned planes = static_cast<unsigned>(a.N * a.C);
    const unsigned per_plane = static_cast<unsigned>(a.OH * a.OW);
    for (unsigned plane = blockIdx.y; plane < planes; plane += gridDim.y) {
        const unsigned img = plane / static_cast<unsigned>(a.C), c = plane - img * static_cast<unsigned>(a.C);
        const float *xp = a.x + img * a.x_img + static_cast<size_t>(c) * a.H * a.W;
        float *yp = a.y + img * a.y_img + static_cast<size_t>(c) * per_plane;
        for (unsigned r = blockIdx.x * 256 + threadIdx.x; r < per_plane; r += gridDim.x * 256) {
            const int oh = static_cast<int>(r / static_cast<unsigned>(a.OW));
            const int ow = static_cast<int>(r) - oh * a.OW;
            float m = -INFINITY;
            for (int i = 0; i < a.kh; i++) {
                const int ih = oh * a.sh + i - a.ph;
                if (ih < 0 || ih >= a.H) continue;
                for (int j = 0; j < a.kw; j++) {
                    const int iw = ow * a.sw + j - a.pw;
                    if (iw < 0 || iw >= a.W) continue;
                    const float v = xp[ih * a.W + iw];
                    if (v > m) m = v;
                }
            }
            yp[r] = m;
        }
    }
}

// The same for a K x K window (any stride and padding), unrolled: every
// tap's load is issued before the first comparison (the generic loop's
// bounds tests keep its loads one after another: YOLO's SPPF 5x5 pools took
// 16.7 us for 6.6 MB at batch 16).  A tap outside the input reads -inf,
// which the strict > never takes, so it counts as skipped; the taps are
// compared in the reference's order (rows, then columns), which decides the
// sign of a zero maximum.
template <int K>
__global__ void __launch_bounds__(256) maxpool_unrolled(PoolArgs a) {
    const unsigned planes = static_cast<unsigned>(a.N * a.C);
    const unsigned per_plane = static_cast<unsigned>(a.OH * a.OW);
    for (unsigned plane = blockIdx.y; plane < planes; plane += gridDim.y) {
        const unsigned img = plane / static_cast<unsigned>(a.C), c = plane - img * static_cast<unsigned>(a.C);
        const float *xp = a.x + img * a.x_img + static_cast<size_t>(c) * a.H * a.W;
        float *yp = a.y + img * a.y_img + static_cast<size_t>(c) * per_plane;
        for (unsigned r = blockIdx.x * 256 + threadIdx.x; r < per_plane; r += gridDim.x * 256) {
            const int oh = static_cast<int>(r / static_cast<unsigned>(a.OW));
            const int ow = static_cast<int>(r) - oh * a.OW;
            float v[K][K];
#pragma unroll
            for (int i = 0; i < K; i++)
#pragma unroll
                for (int j = 0; j < K; j++) {
                    const int ih = oh * a.sh + i - a.ph, iw = ow * a.sw + j - a.pw;
                    const bool in = static_cast<unsigned>(ih) < static_cast<unsigned>(a.H) &&
                                    static_cast<unsigned>(iw) < static_cast<unsigned>(a.W);
                    v[i][j] = in ? xp[ih * a.W + iw] : -INFINITY;
                }
            float m = -INFINITY;
#pragma unroll
            for (int i = 0; i < K; i++)
#pragma unroll
                for (int j = 0; j < K; j++)
                    if (v[i][j] > m) m = v[i][j];
            yp[r] = m;
        }
    }
}

// The ResNet stem's 3x3 / stride 2 / pad 1 MaxPool when W is a multiple of 8
// and W == 2*OW: 4 consecutive outputs (oh, ow0..ow0+3) of one plane from a
// scalar and two 16-byte loads per input row (the 9 columns its windows
// touch), visiting each window in the reference's order (rows, then
// columns, strict >).
__device__ __forceinline__ void pool3s2_x4(const float *__restrict__ xp, int H, int W, int oh, int ow0, float m[4]) {
#pragma unroll
    for (int t = 0; t < 4; t++) m[t] = -INFINITY;
#pragma unroll
    for (int i = 0; i < 3; i++) {
        const int ih = 2 * oh - 1 + i;
        if (ih < 0 || ih >= H) continue;
        const float *row = xp + ih * W + 2 * ow0;
        float c[9];  // input columns 2*ow0-1 .. 2*ow0+7
        c[0] = ow0 > 0 ? row[-1] : 0.0f;
        const floatx4 lo = *reinterpret_cast<const floatx4 *>(row);
        const floatx4 hi = *reinterpret_cast<const floatx4 *>(row + 4);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            c[1 + e] = lo[e];
            c[5 + e] = hi[e];
        }
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int j = 0; j < 3; j++) {
                if (t == 0 && j == 0 && ow0 == 0) continue;  // column -1: outside the input
                const float v = c[2 * t + j];
                if (v > m[t]) m[t] = v;
            }
    }
}

// Each thread makes 4 outputs of one row and stores them as one 16-byte write.
__global__ void __launch_bounds__(256) maxpool3s2_x4(const float *__restrict__ x, float *__restrict__ y, unsigned planes,
                                                     int H, int W, int OH, int OW) {
    const unsigned groups = static_cast<unsigned>(OH * (OW / 4));
    for (unsigned plane = blockIdx.y; plane < planes; plane += gridDim.y) {
        const float *xp = x + static_cast<size_t>(plane) * H * W;
        float *yp = y + static_cast<size_t>(plane) * OH * OW;
        for (unsigned g = blockIdx.x * 256 + threadIdx.x; g < groups; g += gridDim.x * 256) {
            const int oh = static_cast<int>(g / static_cast<unsigned>(OW / 4));
            const int ow0 = 4 * (static_cast<int>(g) - oh * (OW / 4));
            float m[4];
            pool3s2_x4(xp, H, W, oh, ow0, m);
            *reinterpret_cast<floatx4 *>(yp + oh * OW + ow0) = floatx4{m[0], m[1], m[2], m[3]};
        }
    }
}

// The same pooling with the output handed to int8 convs: each pooled value
// is quantized as those convs quantize their input (v * inv_scale; NaN to 0;
// element index < split: round half to even, else half away from zero;
// clamp to [-128, 127]; the index is the NCHW index inside one image of the
// pooled tensor) and written into their zero-padded NHWC int8 buffer
// [N][Hp][Wp][Cp] at pixel (oh + pt, ow + pl); the fp32 output is written
// too when y is non-null.  Block (x, y, z) = (64 consecutive outputs of a
// plane, 64 channels, image): each thread pools four (channel, 4-output
// group) items, 16 groups of one channel per 16 lanes so a wave reads 512
// contiguous bytes per input row, the bytes are transposed through LDS, and
// each thread stores 16 channels of one pixel (one 16-byte store).  Needs
// C % 64 == 0 and Cp a multiple of 16; the halo and channels C..Cp-1 of xq
// are never written (they stay zero).
__global__ void __launch_bounds__(256) maxpool3s2_q8(const float *__restrict__ x, float *__restrict__ y,
                                                     int8_t *__restrict__ xq, int C, int H, int W, int OH, int OW,
                                                     int Hp, int Wp, int Cp, int pt, int pl, float inv_scale,
                                                     int split) {
    __shared__ uint32_t tile[64][16 + 1];  // [channel][4-output group]: 4 bytes, one per output
    const int img = blockIdx.z;
    const int OHW = OH * OW;
    const int gl = threadIdx.x & 15;
    const int g = blockIdx.x * 16 + gl;  // 4-output group of the plane
    if (4 * g < OHW) {
        const int oh = g / (OW / 4);
        const int ow0 = 4 * (g - oh * (OW / 4));
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int cl = (threadIdx.x >> 4) + 16 * i;
            const int c = blockIdx.y * 64 + cl;
            const size_t plane = static_cast<size_t>(img) * C + c;
            float m[4];
            pool3s2_x4(x + plane * H * W, H, W, oh, ow0, m);
            if (y) *reinterpret_cast<floatx4 *>(y + plane * OHW + oh * OW + ow0) = floatx4{m[0], m[1], m[2], m[3]};
            uint32_t word = 0;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int idx = c * OHW + oh * OW + ow0 + t;  // NCHW index inside the image
                const float v = m[t] * inv_scale;
                float r;
                if (v != v) r = 0.0f;
                else r = idx < split ? rintf(v) : roundf(v);
                r = fminf(fmaxf(r, -128.0f), 127.0f);
                word |= static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int8_t>(static_cast<int>(r)))) << (8 * t);
            }
            tile[cl][gl] = word;
        }
    }
    __syncthreads();
    const int px = threadIdx.x >> 2;        // output 0..63 of the block
    const int ch = (threadIdx.x & 3) * 16;  // first of the 16 channels this thread stores
    const int p = blockIdx.x * 64 + px;
    if (p >= OHW) return;
    const int oh = p / OW;
    const int ow = p - oh * OW;
    uint32_t w[4];
#pragma unroll
    for (int d = 0; d < 4; d++) {
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; b++)
            word |= ((tile[ch + 4 * d + b][px >> 2] >> (8 * (px & 3))) & 0xffu) << (8 * b);
        w[d] = word;
    }
    int8_t *dst = xq + ((static_cast<size_t>(img) * Hp + oh + pt) * Wp + ow + pl) * Cp + blockIdx.y * 64 + ch;
    *reinterpret_cast<uintx4 *>(dst) = uintx4{w[0], w[1], w[2], w[3]};
}

// The pooling of maxpool3s2_q8 over an input its producer already quantized
// with the consumers' scale and round-half-even rounding (the pooled tensor
// has no half-away tail when its channels are a multiple of 64): int8 NHWC
// [N][H][W][C] in, the consumers' zero-padded NHWC int8 buffer out.  The
// quantization is monotone, so the maximum of the quantized in-bounds taps
// is the quantized maximum of the fp32 taps, byte for byte.  One thread per
// (output pixel, 16 channels): 9 taps of 16 bytes, one 16-byte store.
__global__ void __launch_bounds__(256) maxpool3s2_i8(const int8_t *__restrict__ xq_in, int8_t *__restrict__ xq,
                                                     unsigned pixels, int C16, int H, int W, int OH, int OW, int Hp,
                                                     int Wp, int Cp, int pt, int pl) {
    typedef signed char char16 __attribute__((ext_vector_type(16)));
    const size_t total = static_cast<size_t>(pixels) * C16;
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
         i += static_cast<size_t>(gridDim.x) * 256) {
        const int c16 = static_cast<int>(i % C16);
        const size_t pix = i / C16;
        const int ow = static_cast<int>(pix % OW);
        const size_t t = pix / OW;
        const int oh = static_cast<int>(t % OH);
        const size_t img = t / OH;
        char16 m = static_cast<char16>(static_cast<signed char>(-128));
#pragma unroll
        for (int kh = 0; kh < 3; kh++) {
            const int ih = 2 * oh - 1 + kh;
            if (ih < 0 || ih >= H) continue;
#pragma unroll
            for (int kw = 0; kw < 3; kw++) {
                const int iw = 2 * ow - 1 + kw;
                if (iw < 0 || iw >= W) continue;
                const char16 v = *reinterpret_cast<const char16 *>(
                    xq_in + ((img * H + ih) * W + iw) * (static_cast<size_t>(C16) * 16) + c16 * 16);
                m = __builtin_elementwise_max(m, v);
            }
        }
        *reinterpret_cast<char16 *>(xq + ((img * Hp + oh + pt) * Wp + ow + pl) * Cp + c16 * 16) = m;
    }
}

// reference pool/avgpool.c:21-45: mean over the in-bounds taps
__global__ void __launch_bounds__(256) avgpool_kernel(PoolArgs a) {
    const size_t total = static_cast<size_t>(a.N) * a.C * a.OH * a.OW;
    for (size_t idx = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; idx < total;
         idx += static_cast<size_t>(gridDim.x) * 256) {
        const int ow = static_cast<int>(idx % a.OW);
        const size_t t = idx / a.OW;
        const int oh = static_cast<int>(t % a.OH);
        const size_t plane = t / a.OH;
        const float *xp = a.x + plane * a.H * a.W;
        float sum = 0.0f;
        int count = 0;
        for (int i = 0; i < a.kh; i++) {
            const int ih = oh * a.sh + i - a.ph;
            if (ih < 0 || ih >= a.H) continue;
            for (int j = 0; j < a.kw; j++) {
                const int iw = ow * a.sw + j - a.pw;
                if (iw < 0 || iw >= a.W) continue;
                sum += xp[ih * a.W + iw];
                count++;
            }
        }
        a.y[idx] = count > 0 ? sum / static_cast<float>(count) : 0.0f;
    }
}

// Wave-wide sum / max through DPP lane moves (no LDS round trips): an
// inclusive scan within each 16-lane row (row_shr 1, 2, 4, 8), then row 0's
// total into row 1 and row 2's into row 3 (row_bcast 15), then rows 0-1's
// into rows 2-3 (row_bcast 31); lane 63 ends with the whole wave's, read
// back as a scalar.  Lanes a move has no source for, or whose row it
// leaves out, take the identity.
template <bool MAX>
__device__ __forceinline__ float wave_reduce(float v) {
    const int id = __float_as_int(MAX ? -INFINITY : 0.0f);
    auto step = [&](float o) { v = MAX ? (o > v ? o : v) : v + o; };
    step(__int_as_float(__builtin_amdgcn_update_dpp(id, __float_as_int(v), 0x111, 0xf, 0xf, false)));
    step(__int_as_float(__builtin_amdgcn_update_dpp(id, __float_as_int(v), 0x112, 0xf, 0xf, false)));
    step(__int_as_float(__builtin_amdgcn_update_dpp(id, __float_as_int(v), 0x114, 0xf, 0xf, false)));
    step(__int_as_float(__builtin_amdgcn_update_dpp(id, __float_as_int(v), 0x118, 0xf, 0xf, false)));
    step(__int_as_float(__builtin_amdgcn_update_dpp(id, __float_as_int(v), 0x142, 0xa, 0xf, false)));
    step(__int_as_float(__builtin_amdgcn_update_dpp(id, __float_as_int(v), 0x143, 0xc, 0xf, false)));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float wave_sum(float v) { return wave_reduce<false>(v); }
__device__ __forceinline__ float wave_max(float v) { return wave_reduce<true>(v); }

// Max over short contiguous rows (len <= 128: YOLO's 80 class scores per
// anchor): 16 lanes per row, four rows per wave; each lane keeps the max of
// its elements (v > acc, so NaN never wins, as row_reduce), then four DPP
// shifts within the 16-lane row leave the row's max in its lane 15.
__global__ void __launch_bounds__(256) row_max16(const float *__restrict__ x, float *__restrict__ y, size_t rows,
                                                 int len) {
    const int l16 = threadIdx.x & 15;
    const size_t row = (static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x) >> 4;
    const bool live = row < rows;
    float acc = -INFINITY;
    if (live) {
        const float *xr = x + row * len;
        for (int i = l16; i < len; i += 16) {
            const float v = xr[i];
            acc = v > acc ? v : acc;
        }
    }
    const int id = __float_as_int(-INFINITY);
    auto step = [&](float o) { acc = o > acc ? o : acc; };
    step(__int_as_float(__builtin_amdgcn_update_dpp(id, __float_as_int(acc), 0x111, 0xf, 0xf, false)));
    step(__int_as_float(__builtin_amdgcn_update_dpp(id, __float_as_int(acc), 0x112, 0xf, 0xf, false)));
    step(__int_as_float(__builtin_amdgcn_update_dpp(id, __float_as_int(acc), 0x114, 0xf, 0xf, false)));
    step(__int_as_float(__builtin_amdgcn_update_dpp(id, __float_as_int(acc), 0x118, 0xf, 0xf, false)));
    if (live && l16 == 15) y[row] = acc;
}

// One wave per contiguous row of `len` elements.  MODE 0: mean of x/denom
// terms (ReduceMean, reference reduce.c:37-40); 1: max (ReduceMax);
// 2: sum * inv (GlobalAveragePool, avgpool.c:62-67).
template <int MODE>
__global__ void __launch_bounds__(256) row_reduce(const float *__restrict__ x, float *__restrict__ y, size_t rows,
                                                  int len, float denom) {
    const int lane = threadIdx.x & 63;
    const size_t row = static_cast<size_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + row * len;
    float acc = MODE == 1 ? -INFINITY : 0.0f;
    for (int i = lane; i < len; i += 64) {
        const float v = xr[i];
        if (MODE == 0) acc += v / denom;
        else if (MODE == 1) acc = v > acc ? v : acc;
        else acc += v;
    }
    acc = MODE == 1 ? wave_max(acc) : wave_sum(acc);
    if (lane == 0) y[row] = MODE == 2 ? acc * (1.0f / denom) : acc;
}

// Generic reduction: thread per output element, walking the reduced
// sub-space.  rdim/rstride describe the reduced axes, odim/ostride the kept
// axes (in x strides), in row-major order of the output.
struct ReduceDesc {
    int nr, no;
    int64_t rdim[kMaxRank], rstride[kMaxRank];
    int64_t odim[kMaxRank], ostride[kMaxRank];
    int64_t rcount;
};

template <int MODE>
__global__ void __launch_bounds__(256) generic_reduce(const float *__restrict__ x, float *__restrict__ y, size_t nout,
                                                      ReduceDesc d, float denom) {
    for (size_t o = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; o < nout; o += static_cast<size_t>(gridDim.x) * 256) {
        size_t t = o;
        int64_t base = 0;
        for (int k = d.no - 1; k >= 0; k--) {
            base += static_cast<int64_t>(t % d.odim[k]) * d.ostride[k];
            t /= d.odim[k];
        }
        float acc = MODE == 1 ? -INFINITY : 0.0f;
        for (int64_t r = 0; r < d.rcount; r++) {
            int64_t rr = r, off = 0;
            for (int k = d.nr - 1; k >= 0; k--) {
                off += (rr % d.rdim[k]) * d.rstride[k];
                rr /= d.rdim[k];
            }
            const float v = x[base + off];
            if (MODE == 0) acc += v / denom;
            else acc = v > acc ? v : acc;
        }
        y[o] = acc;
    }
}

// Softmax over contiguous rows (inner == 1): one wave per row.
__global__ void __launch_bounds__(256) softmax_rows(const float *__restrict__ x, float *__restrict__ y, size_t rows,
                                                    int dim) {
    const int lane = threadIdx.x & 63;
    const size_t row = static_cast<size_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + row * dim;
    float *yr = y + row * dim;
    float m = -INFINITY;
    for (int i = lane; i < dim; i += 64) m = fmaxf(m, xr[i]);
    m = wave_max(m);
    float s = 0.0f;
    for (int i = lane; i < dim; i += 64) {
        const float e = __expf(xr[i] - m);
        yr[i] = e;
        s += e;
    }
    const float r = 1.0f / wave_sum(s);
    for (int i = lane; i < dim; i += 64) yr[i] = yr[i] * r;
}

// Rows of at most 256 * Q values that are a multiple of 4 long: one
// 64-thread workgroup per row holds the row in registers (Q float4 per
// lane), so the row is read once and written once.  NT: the output leaves
// through non-temporal stores, measured faster for outputs several times an
// XCD's 4 MB L2 (4096 rows of 1000: 6.8 -> 5.5 us; non-temporal loads as
// well were slower).
template <int Q, bool NT>
__global__ void __launch_bounds__(64) softmax_rows_reg(const float *__restrict__ x, float *__restrict__ y, int dim) {
    const int lane = threadIdx.x;
    const size_t row = blockIdx.x;
    const floatx4 *xr = reinterpret_cast<const floatx4 *>(x + row * dim);
    floatx4 *yr = reinterpret_cast<floatx4 *>(y + row * dim);
    const int quads = dim / 4;
    floatx4 v[Q];
    float m = -INFINITY;
#pragma unroll
    for (int t = 0; t < Q; t++) {
        const int q = t * 64 + lane;
        v[t] = q < quads ? xr[q] : floatx4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        m = fmaxf(m, fmaxf(fmaxf(v[t][0], v[t][1]), fmaxf(v[t][2], v[t][3])));
    }
    m = wave_max(m);
    float s = 0.0f;
#pragma unroll
    for (int t = 0; t < Q; t++) {
        if (t * 64 + lane < quads) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                v[t][e] = __expf(v[t][e] - m);
                s += v[t][e];
            }
        }
    }
    const float r = 1.0f / wave_sum(s);
#pragma unroll
    for (int t = 0; t < Q; t++) {
        const int q = t * 64 + lane;
        if (q < quads) {
            const floatx4 o = floatx4{v[t][0] * r, v[t][1] * r, v[t][2] * r, v[t][3] * r};
            if (NT) __builtin_nontemporal_store(o, yr + q);
            else yr[q] = o;
        }
    }
}

// Softmax along a strided axis: thread per (outer, inner) column, lanes
// adjacent in `inner` so every pass over d is coalesced.
__global__ void __launch_bounds__(256) softmax_strided(const float *__restrict__ x, float *__restrict__ y, size_t outer,
                                                       int dim, size_t inner) {
    const size_t cols = outer * inner;
    for (size_t c = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; c < cols; c += static_cast<size_t>(gridDim.x) * 256) {
        const size_t o = c / inner, in = c - o * inner;
        const float *xc = x + o * dim * inner + in;
        float *yc = y + o * dim * inner + in;
        float m = -INFINITY;
        for (int d = 0; d < dim; d++) m = fmaxf(m, xc[static_cast<size_t>(d) * inner]);
        float s = 0.0f;
        for (int d = 0; d < dim; d++) {
            const float e = __expf(xc[static_cast<size_t>(d) * inner] - m);
            yc[static_cast<size_t>(d) * inner] = e;
            s += e;
        }
        const float r = 1.0f / s;
        for (int d = 0; d < dim; d++) yc[static_cast<size_t>(d) * inner] = yc[static_cast<size_t>(d) * inner] * r;
    }
}

// The same for a short axis (dim <= D: YOLO's 16-bin DFL softmax): the
// column stays in registers, so it is read once with every load in flight and
// written once; the arithmetic and its order are softmax_strided's.
template <int D>
__global__ void __launch_bounds__(256) softmax_strided_reg(const float *__restrict__ x, float *__restrict__ y,
                                                           size_t outer, int dim, size_t inner) {
    const size_t cols = outer * inner;
    for (size_t c = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; c < cols; c += static_cast<size_t>(gridDim.x) * 256) {
        const size_t o = c / inner, in = c - o * inner;
        const float *xc = x + o * dim * inner + in;
        float *yc = y + o * dim * inner + in;
        float v[D];
#pragma unroll
        for (int d = 0; d < D; d++) v[d] = d < dim ? xc[static_cast<size_t>(d) * inner] : -INFINITY;
        float m = -INFINITY;
#pragma unroll
        for (int d = 0; d < D; d++)
            if (d < dim) m = fmaxf(m, v[d]);
        float s = 0.0f;
#pragma unroll
        for (int d = 0; d < D; d++)
            if (d < dim) {
                v[d] = __expf(v[d] - m);
                s += v[d];
            }
        const float r = 1.0f / s;
#pragma unroll
        for (int d = 0; d < D; d++)
            if (d < dim) yc[static_cast<size_t>(d) * inner] = v[d] * r;
    }
}

// Nearest resize with the reference index rule (reference shape/resize.c:15-26).
__global__ void __launch_bounds__(256) resize_nearest(const float *__restrict__ x, float *__restrict__ y, int N, int C,
                                                      int H, int W, int OH, int OW, float scale_h, float scale_w) {
    const size_t total = static_cast<size_t>(N) * C * OH * OW;
    for (size_t idx = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; idx < total;
         idx += static_cast<size_t>(gridDim.x) * 256) {
        const int ow = static_cast<int>(idx % OW);
        const size_t t = idx / OW;
        const int oh = static_cast<int>(t % OH);
        const size_t plane = t / OH;
        int ih = static_cast<int>(floorf(static_cast<float>(oh) / scale_h));
        if (ih >= H) ih = H - 1;
        int iw = static_cast<int>(floorf(static_cast<float>(ow) / scale_w));
        if (iw >= W) iw = W - 1;
        y[idx] = x[(plane * H + ih) * W + iw];
    }
}

// ------------------------------------------------ reliability helpers

__global__ void flip_bit_kernel(uint32_t *p, uint32_t bit) { *p ^= (1u << bit); }

// Range of an fp32 tensor with the reference's fold semantics
// (runtime/core/executor.c:400-443): min / max start from element 0 and are
// replaced only on a strict < / >, so NaNs after element 0 never enter, a NaN
// at element 0 sticks, infinities count, and among equal extrema (+0 / -0)
// the first by index is kept.  out[2] flags any non-finite element (the
// in-range test rejects those).  One block: this runs only on protected
// nodes.
__device__ inline void minmax_take(float &v, unsigned long long &i, float ov, unsigned long long oi, bool less) {
    const bool better = less ? (ov < v) : (ov > v);
    if (better || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

__global__ void __launch_bounds__(256) minmax_kernel(const float *__restrict__ x, size_t n, float *__restrict__ out) {
    __shared__ float s_lo[4], s_hi[4], s_bad[4];
    __shared__ unsigned long long s_li[4], s_hi_i[4];
    float lo = INFINITY, hi = -INFINITY, bad = 0.0f;
    unsigned long long li = ~0ull, hi_i = ~0ull;
    for (size_t i = threadIdx.x; i < n; i += 256) {
        const float v = x[i];
        if (!isfinite(v)) bad = 1.0f;
        if (v == v) {
            minmax_take(lo, li, v, i, true);
            minmax_take(hi, hi_i, v, i, false);
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        minmax_take(lo, li, __shfl_xor(lo, off, 64), __shfl_xor(li, off, 64), true);
        minmax_take(hi, hi_i, __shfl_xor(hi, off, 64), __shfl_xor(hi_i, off, 64), false);
        bad = fmaxf(bad, __shfl_xor(bad, off, 64));
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        s_lo[w] = lo;
        s_li[w] = li;
        s_hi[w] = hi;
        s_hi_i[w] = hi_i;
        s_bad[w] = bad;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < 4; k++) {
            minmax_take(lo, li, s_lo[k], s_li[k], true);
            minmax_take(hi, hi_i, s_hi[k], s_hi_i[k], false);
            bad = fmaxf(bad, s_bad[k]);
        }
        if (n > 0 && x[0] != x[0]) {
            lo = x[0];
            hi = x[0];
        }
        out[0] = lo;
        out[1] = hi;
        out[2] = bad;
        out[3] = 0.0f;
    }
}

__global__ void __launch_bounds__(256) compare_kernel(const uint8_t *__restrict__ a, const uint8_t *__restrict__ b,
                                                      size_t n, uint32_t *flag) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256)
        if (a[i] != b[i]) *flag = 1u;
}

__global__ void fill_u32_kernel(uint32_t *p, size_t n, uint32_t v) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256)
        p[i] = v;
}

int axis_norm(int axis, int rank) { return axis < 0 ? axis + rank : axis; }

}  // namespace

// ================================================================ node kernels

int binary_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    if (node->input_count < 2 || node->output_count < 1) return -11;
    int act = 0;
    if (node->op_type == SPKV2_OP_ADD) {
        Spkv2AttrRecord attr;
        if (int rc = spkv2_ctx_get_attr(ctx, node, &attr)) return rc;
        act = attr.fused_activation;
    }
    const Spkv2TensorRecord *ar = rec(ctx, node->inputs[0]), *br = rec(ctx, node->inputs[1]), *yr = rec(ctx, node->outputs[0]);
    const float *a = dptr<const float>(ctx, node->inputs[0]), *b = dptr<const float>(ctx, node->inputs[1]);
    float *y = dptr<float>(ctx, node->outputs[0]);
    hipStream_t s = ctx->stream;
    const Spkv2TensorView *av = live_view(ctx, node->inputs[0]), *bv = live_view(ctx, node->inputs[1]),
                          *yv = live_view(ctx, node->outputs[0]);
    if (av || bv || yv) {
        // an Add over channel slices of Concat buffers (same-shape NCHW, as
        // set up at prepare): float4s when every base and image stride
        // allows, scalar elements otherwise
        if (node->op_type != SPKV2_OP_ADD || yr->rank != 4) return SPKV2_E_UNSUPPORTED;
        const unsigned images = yr->shape[0];
        const size_t per = elem_count(yr) / std::max(images, 1u);
        const size_t as = av ? av->img_elems : per, bs = bv ? bv->img_elems : per, ys = yv ? yv->img_elems : per;
        if (av) a = reinterpret_cast<const float *>(av->base);
        if (bv) b = reinterpret_cast<const float *>(bv->base);
        if (yv) y = reinterpret_cast<float *>(yv->base);
        if (((per | as | bs | ys) & 3) != 0 ||
            ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) | reinterpret_cast<uintptr_t>(y)) & 15)) {
            set_kernel_name(ctx, node, "binary_img1");
            if (per == 0 || images == 0) return 0;
            const dim3 grid(static_cast<unsigned>(std::min<size_t>((per + 255) / 256, 1024)), std::min(images, 65535u));
            hipLaunchKernelGGL((binary_img1<BIN_ADD>), grid, dim3(256), 0, s, a, b, y, images, per, as, bs, ys, act);
            return launch_status("binary_img1");
        }
        set_kernel_name(ctx, node, "binary_img4");
        if (per == 0 || images == 0) return 0;
        const dim3 grid(static_cast<unsigned>(std::min<size_t>((per / 4 + 255) / 256, 1024)), std::min(images, 65535u));
        hipLaunchKernelGGL((binary_img4<BIN_ADD>), grid, dim3(256), 0, s, reinterpret_cast<const float4 *>(a),
                           reinterpret_cast<const float4 *>(b), reinterpret_cast<float4 *>(y), images, per / 4, as / 4,
                           bs / 4, ys / 4, act);
        return launch_status("binary_img4");
    }
    set_kernel_name(ctx, node, "binary");
    switch (node->op_type) {
    case SPKV2_OP_ADD: return launch_binary<BIN_ADD>(s, ar, br, yr, a, b, y, act);
    case SPKV2_OP_MUL: return launch_binary<BIN_MUL>(s, ar, br, yr, a, b, y, 0);
    case SPKV2_OP_SUB: return launch_binary<BIN_SUB>(s, ar, br, yr, a, b, y, 0);
    case SPKV2_OP_DIV: return launch_binary<BIN_DIV>(s, ar, br, yr, a, b, y, 0);
    case SPKV2_OP_MOD: return launch_binary<BIN_MOD>(s, ar, br, yr, a, b, y, 0);
    }
    return -99;
}

int unary_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    const Spkv2TensorRecord *xr = rec(ctx, node->inputs[0]);
    const float *x = dptr<const float>(ctx, node->inputs[0]);
    float *y = dptr<float>(ctx, node->outputs[0]);
    const size_t n = elem_count(xr);
    if (n == 0) return 0;
    const dim3 grid(grid_for(n, 256));
    hipStream_t s = ctx->stream;
    set_kernel_name(ctx, node, "unary");
    switch (node->op_type) {
    case SPKV2_OP_RELU: hipLaunchKernelGGL(unary_kernel<UN_RELU>, grid, dim3(256), 0, s, x, y, n, nullptr, nullptr, 0.0f); break;
    case SPKV2_OP_SIGMOID:
        if (n % 4 == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15) == 0)
            hipLaunchKernelGGL(sigmoid4, dim3(grid_for(n / 4, 256)), dim3(256), 0, s, reinterpret_cast<const float4 *>(x),
                               reinterpret_cast<float4 *>(y), n / 4);
        else
            hipLaunchKernelGGL(unary_kernel<UN_SIGMOID>, grid, dim3(256), 0, s, x, y, n, nullptr, nullptr, 0.0f);
        break;
    case SPKV2_OP_CLIP: {
        const float *lo = node->input_count >= 2 ? dptr<const float>(ctx, node->inputs[1]) : nullptr;
        const float *hi = node->input_count >= 3 ? dptr<const float>(ctx, node->inputs[2]) : nullptr;
        hipLaunchKernelGGL(unary_kernel<UN_CLIP>, grid, dim3(256), 0, s, x, y, n, lo, hi, 0.0f);
        break;
    }
    case SPKV2_OP_LEAKYRELU: {
        Spkv2AttrRecord attr;
        if (int rc = spkv2_ctx_get_attr(ctx, node, &attr)) return rc;
        hipLaunchKernelGGL(unary_kernel<UN_LEAKY>, grid, dim3(256), 0, s, x, y, n, nullptr, nullptr, attr.alpha);
        break;
    }
    default: return -99;
    }
    return launch_status("unary");
}

// Flatten / Reshape / Cast / Unsqueeze: a byte copy unless the planner
// aliased output and input (reference shape/copy.c, shape/flatten.c).
int copy_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    if (view_elided(ctx, node->id)) {  // a detection-head chain's Reshape: its data already sit in place
        set_kernel_name(ctx, node, "copy_elided");
        return 0;
    }
    const size_t bytes = node->op_type == SPKV2_OP_FLATTEN ? rec(ctx, node->inputs[0])->size_bytes
                                                           : rec(ctx, node->outputs[0])->size_bytes;
    set_kernel_name(ctx, node, "copy");
    return launch_copy(ctx->stream, ctx->tensors[node->inputs[0]].data, ctx->tensors[node->outputs[0]].data, bytes);
}

// reference tensor/concat.c; inputs the planner placed inside the output
// (memory_plan.py Concat aliases) are already in place and are skipped.
int concat_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    if (view_elided(ctx, node->id)) {  // a detection-head chain's Concat: its inputs were written in place
        set_kernel_name(ctx, node, "concat_elided");
        return 0;
    }
    Spkv2AttrRecord attr;
    if (int rc = spkv2_ctx_get_attr(ctx, node, &attr)) return rc;
    const Spkv2TensorRecord *yr = rec(ctx, node->outputs[0]);
    const int axis = axis_norm(attr.axis, yr->rank);
    if (axis < 0 || axis >= yr->rank) return -11;
    size_t outer = 1, inner = 1;
    for (int i = 0; i < axis; i++) outer *= yr->shape[i];
    for (int i = axis + 1; i < yr->rank; i++) inner *= yr->shape[i];
    const size_t y_axis = yr->shape[axis];
    float *y = dptr<float>(ctx, node->outputs[0]);
    size_t y_stride = y_axis * inner;
    // channel-slice views (set up at prepare for axis 1): the output is the
    // Concat buffer, and the inputs that are views into it are in place
    const Spkv2TensorView *ov = live_view(ctx, node->outputs[0]);
    if (ov) {
        if (axis != 1) return SPKV2_E_UNSUPPORTED;
        y = reinterpret_cast<float *>(ov->base);
        y_stride = static_cast<size_t>(ov->img_elems);
    }
    size_t axis_off = 0;
    set_kernel_name(ctx, node, ov ? "concat_views" : "concat");
    CopySeg segs[8];  // a node record has at most eight inputs
    int count = 0;
    for (uint16_t i = 0; i < node->input_count && i < 8; i++) {
        const Spkv2TensorRecord *xr = rec(ctx, node->inputs[i]);
        const float *x = dptr<const float>(ctx, node->inputs[i]);
        const size_t block = static_cast<size_t>(xr->shape[axis]) * inner;
        size_t x_stride = block;
        if (const Spkv2TensorView *xv = live_view(ctx, node->inputs[i])) {
            x = reinterpret_cast<const float *>(xv->base);
            x_stride = static_cast<size_t>(xv->img_elems);
        }
        float *dst = y + axis_off * inner;
        if (!((outer == 1 || x_stride == y_stride) && dst == x) && outer * block > 0)
            segs[count++] = CopySeg{x, dst, block, x_stride, 0, y_stride};
        axis_off += xr->shape[axis];
    }
    return multi_block_copy(ctx->stream, segs, count, outer);  // one launch for the aligned inputs
}

static int pool_args(Spkv2Context *ctx, const Spkv2NodeRecord *node, PoolArgs *p) {
    Spkv2AttrRecord attr;
    if (int rc = spkv2_ctx_get_attr(ctx, node, &attr)) return rc;
    const Spkv2TensorRecord *xr = rec(ctx, node->inputs[0]), *yr = rec(ctx, node->outputs[0]);
    if (xr->rank != 4 || yr->rank != 4) return -11;
    p->x = dptr<const float>(ctx, node->inputs[0]);
    p->y = dptr<float>(ctx, node->outputs[0]);
    p->N = xr->shape[0];
    p->C = xr->shape[1];
    p->H = xr->shape[2];
    p->W = xr->shape[3];
    p->OH = yr->shape[2];
    p->OW = yr->shape[3];
    p->kh = attr.kernel_shape[0];
    p->kw = attr.kernel_shape[1];
    p->sh = attr.strides[0];
    p->sw = attr.strides[1];
    p->ph = attr.pads[0];
    p->pw = attr.pads[1];
    p->x_img = static_cast<size_t>(p->C) * p->H * p->W;
    p->y_img = static_cast<size_t>(p->C) * p->OH * p->OW;
    return 0;
}

static bool is_pool3s2_x4(const PoolArgs &p) {
    return p.kh == 3 && p.kw == 3 && p.sh == 2 && p.sw == 2 && p.ph == 1 && p.pw == 1 && p.W % 8 == 0 &&
           p.W == 2 * p.OW && p.H == 2 * p.OH && p.OW % 4 == 0;
}

void pool_plan_free(void *p) {
    // q_out belongs to the first consuming conv, q_src to this plan
    PoolPlan *plan = static_cast<PoolPlan *>(p);
    if (plan->q_src) (void)hipFree(plan->q_src);
    delete plan;
}

// A MaxPool that the fused pooling + int8 quantization kernel can run gets a
// PoolPlan, which an int8 conv reading its output fills in at its own
// prepare (the conv nodes come later in the node table).
int maxpool_prepare(Spkv2Context *ctx, const Spkv2NodeRecord *node, size_t *ws) {
    *ws = 0;
    void **slot = &ctx->plans[node->id];
    if (*slot) return 0;
    PoolArgs p;
    if (pool_args(ctx, node, &p) != 0) return 0;  // the run reports it
    if (rec(ctx, node->inputs[0])->dtype != SPKV2_DTYPE_FP32 || !is_pool3s2_x4(p) || p.C % 64 != 0 || p.N < 1 || p.N > 65535 ||
        static_cast<int64_t>(p.N) * p.C * p.H * p.W * 4 >= (int64_t(1) << 31))
        return 0;
    PoolPlan *plan = new PoolPlan();
    memset(plan, 0, sizeof(*plan));
    *slot = plan;
    ctx->plan_dtors[node->id] = pool_plan_free;
    return 0;
}

// After every node's prepare: a MaxPool whose output every reader takes in
// int8 (no fp32 output needed) and whose input is the only output of an
// int8 conv with Relu, read by nothing else, gets that input in int8: the
// conv's epilogue quantizes it with the pool consumers' scale (their
// rounding is half to even throughout: 64-channel planes leave no tail)
// into the plan's NHWC buffer, and the conv skips its fp32 output.  Relu
// keeps NaN out (the fp32 pool would skip a NaN tap; its int8 value is 0).
// Off for protected packages and under SPKV2_I8_HANDOFF=0, bypassed like
// every handoff while handoffs_live() is false.
int setup_pool_int8_inputs(Spkv2Context *ctx) {
    if (ctx->protection_count > 0) return 0;
    if (const char *e = getenv("SPKV2_I8_HANDOFF"))
        if (e[0] == '0') return 0;
    for (uint32_t id = 0; id < ctx->header.num_nodes; id++) {
        const Spkv2NodeRecord *node = &ctx->node_records[id];
        if (node->op_type != SPKV2_OP_MAXPOOL || !builtin_runs(ctx, id) || ctx->plan_dtors[id] != pool_plan_free) continue;
        PoolPlan *q = static_cast<PoolPlan *>(ctx->plans[id]);
        PoolArgs p;
        if (!q || !q->q_out || q->y_needed || q->q_src || pool_args(ctx, node, &p) != 0) continue;
        if (!is_pool3s2_x4(p) || p.C % 64 != 0 || q->q_split < p.C * p.OH * p.OW) continue;
        const uint32_t t = node->inputs[0];
        const Spkv2NodeRecord *prod = nullptr;
        int readers = 0;
        for (uint32_t i = 0; i < ctx->header.num_nodes; i++) {
            const Spkv2NodeRecord *n = &ctx->node_records[i];
            for (uint16_t k = 0; k < n->input_count; k++)
                if (n->inputs[k] == t) readers++;
            for (uint16_t k = 0; k < n->output_count; k++)
                if (n->outputs[k] == t) prod = n;
        }
        bool is_output = false;
        for (size_t i = 0; i < ctx->output_count; i++)
            if (ctx->output_ids[i] == t) is_output = true;
        if (!prod || prod->id >= id || prod->op_type != SPKV2_OP_CONV || prod->output_count != 1 || readers != 1 ||
            is_output || !builtin_runs(ctx, prod->id) || ctx->plan_dtors[prod->id] != conv_plan_free)
            continue;
        ConvPlan *cp = static_cast<ConvPlan *>(ctx->plans[prod->id]);
        if (!cp || cp->path != CONV_IGEMM_I8 || cp->q_out || cp->g.act != 1 || cp->g.M != p.C || cp->g.N != p.N ||
            cp->g.OH != p.H || cp->g.OW != p.W)
            continue;
        const size_t bytes = static_cast<size_t>(p.N) * p.H * p.W * p.C;
        if (bytes >= 0x7fff0000ULL) continue;  // the epilogue's byte offsets are 31-bit
        if (int rc = hip_check(hipMalloc(reinterpret_cast<void **>(&q->q_src), bytes), "hipMalloc int8 pool input"))
            return rc;
        cp->q_out = q->q_src;
        cp->q_Hp = p.H;
        cp->q_Wp = p.W;
        cp->q_Cp = p.C;
        cp->q_pt = cp->q_pl = 0;
        cp->q_split = 0x7fffffff;  // round half to even everywhere
        cp->q_inv_scale = q->q_inv_scale;
        cp->q_readers = 1;
        cp->y_needed = false;
    }
    return 0;
}

int maxpool_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    if (q8_tensor(ctx, node->inputs[0])) return maxpool_q8_run(ctx, node);
    PoolArgs p;
    if (int rc = pool_args(ctx, node, &p)) return rc;
    const size_t total = static_cast<size_t>(p.N) * p.C * p.OH * p.OW;
    if (total == 0) return 0;
    // int8 handoff while the handoffs are live (no fault event armed, the
    // kernel registry as at prepare); otherwise the consumers quantize the
    // fp32 output themselves
    const PoolPlan *q = ctx->plan_dtors[node->id] == pool_plan_free
                            ? static_cast<const PoolPlan *>(ctx->plans[node->id])
                            : nullptr;
    // views are set up for stride-1 pools only, which take the generic kernel
    if ((live_view(ctx, node->inputs[0]) || live_view(ctx, node->outputs[0])) && is_pool3s2_x4(p))
        return SPKV2_E_UNSUPPORTED;
    if (q && q->q_out && q->q_src && handoffs_live(ctx) && is_pool3s2_x4(p) && p.C % 64 == 0) {
        // the producer quantized the input for this pool's consumers
        set_kernel_name(ctx, node, "maxpool3s2_i8");
        const size_t pixels = static_cast<size_t>(p.N) * p.OH * p.OW;
        const size_t work = pixels * (p.C / 16);
        if (pixels > 0xffffffffULL) return SPKV2_E_UNSUPPORTED;
        hipLaunchKernelGGL(maxpool3s2_i8, dim3(grid_for(work, 256)), dim3(256), 0, ctx->stream, q->q_src, q->q_out,
                           static_cast<unsigned>(pixels), p.C / 16, p.H, p.W, p.OH, p.OW, q->q_Hp, q->q_Wp, q->q_Cp,
                           q->q_pt, q->q_pl);
        return launch_status("maxpool");
    }
    if (q && q->q_out && handoffs_live(ctx) && is_pool3s2_x4(p) && p.C % 64 == 0) {
        set_kernel_name(ctx, node, q->y_needed ? "maxpool3s2_q8+y" : "maxpool3s2_q8");
        const dim3 grid(static_cast<unsigned>((p.OH * p.OW + 63) / 64), static_cast<unsigned>(p.C / 64),
                        static_cast<unsigned>(p.N));
        hipLaunchKernelGGL(maxpool3s2_q8, grid, dim3(256), 0, ctx->stream, p.x, q->y_needed ? p.y : nullptr, q->q_out,
                           p.C, p.H, p.W, p.OH, p.OW, q->q_Hp, q->q_Wp, q->q_Cp, q->q_pt, q->q_pl, q->q_inv_scale,
                           q->q_split);
        return launch_status("maxpool");
    }
    if (is_pool3s2_x4(p)) {
        set_kernel_name(ctx, node, "maxpool3s2_x4");
        const size_t groups = static_cast<size_t>(p.OH) * (p.OW / 4), planes = static_cast<size_t>(p.N) * p.C;
        if (groups > 0x7fffffffULL || planes > 0x7fffffffULL) return SPKV2_E_UNSUPPORTED;
        const dim3 grid(static_cast<unsigned>(std::min<size_t>((groups + 255) / 256, 1024)),
                        static_cast<unsigned>(std::min<size_t>(planes, 65535)));
        hipLaunchKernelGGL(maxpool3s2_x4, grid, dim3(256), 0, ctx->stream, p.x, p.y, static_cast<unsigned>(planes), p.H,
                           p.W, p.OH, p.OW);
        return launch_status("maxpool");
    }
    set_kernel_name(ctx, node, "maxpool");
    const size_t per_plane = static_cast<size_t>(p.OH) * p.OW, planes = static_cast<size_t>(p.N) * p.C;
    if (per_plane > 0x7fffffffULL || planes > 0x7fffffffULL) return SPKV2_E_UNSUPPORTED;
    const dim3 grid(static_cast<unsigned>(std::min<size_t>((per_plane + 255) / 256, 1024)),
                    static_cast<unsigned>(std::min<size_t>(planes, 65535)));
    // input and output through their channel-slice views when they have them
    // (SPPF's stride-1 pools: a Concat's buffer)
    if (const Spkv2TensorView *v = live_view(ctx, node->inputs[0])) {
        p.x = reinterpret_cast<const float *>(v->base);
        p.x_img = static_cast<size_t>(v->img_elems);
    }
    if (const Spkv2TensorView *v = live_view(ctx, node->outputs[0])) {
        p.y = reinterpret_cast<float *>(v->base);
        p.y_img = static_cast<size_t>(v->img_elems);
    }
    if (p.kh == p.kw && (p.kh == 2 || p.kh == 3 || p.kh == 5)) {
        set_kernel_name(ctx, node, "maxpool_unrolled");
        hipLaunchKernelGGL(p.kh == 2 ? maxpool_unrolled<2> : p.kh == 3 ? maxpool_unrolled<3> : maxpool_unrolled<5>,
                           grid, dim3(256), 0, ctx->stream, p);
    } else {
        hipLaunchKernelGGL(maxpool_kernel, grid, dim3(256), 0, ctx->stream, p);
    }
    return launch_status("maxpool");
}

int avgpool_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    PoolArgs p;
    if (int rc = pool_args(ctx, node, &p)) return rc;
    const size_t total = static_cast<size_t>(p.N) * p.C * p.OH * p.OW;
    if (total == 0) return 0;
    set_kernel_name(ctx, node, "avgpool");
    hipLaunchKernelGGL(avgpool_kernel, dim3(grid_for(total, 256)), dim3(256), 0, ctx->stream, p);
    return launch_status("avgpool");
}

int global_avgpool_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    if (q8_tensor(ctx, node->inputs[0])) return mean_q8_run(ctx, node);
    const Spkv2TensorRecord *xr = rec(ctx, node->inputs[0]);
    if (xr->rank != 4) return -11;
    const size_t rows = static_cast<size_t>(xr->shape[0]) * xr->shape[1];
    const int len = static_cast<int>(xr->shape[2] * xr->shape[3]);
    if (rows == 0) return 0;
    set_kernel_name(ctx, node, "global_avgpool");
    hipLaunchKernelGGL(row_reduce<2>, dim3(blocks_for(rows, 4)), dim3(256), 0, ctx->stream,
                       dptr<const float>(ctx, node->inputs[0]), dptr<float>(ctx, node->outputs[0]), rows, len,
                       static_cast<float>(len));
    return launch_status("global_avgpool");
}

int softmax_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    Spkv2AttrRecord attr;
    if (int rc = spkv2_ctx_get_attr(ctx, node, &attr)) return rc;
    const Spkv2TensorRecord *xr = rec(ctx, node->inputs[0]);
    const int axis = axis_norm(attr.axis, xr->rank);
    if (axis < 0 || axis >= xr->rank) return -11;
    size_t outer = 1, inner = 1;
    const int dim = static_cast<int>(xr->shape[axis]);
    for (int i = 0; i < axis; i++) outer *= xr->shape[i];
    for (int i = axis + 1; i < xr->rank; i++) inner *= xr->shape[i];
    const float *x = dptr<const float>(ctx, node->inputs[0]);
    float *y = dptr<float>(ctx, node->outputs[0]);
    if (outer * inner == 0 || dim == 0) return 0;
    set_kernel_name(ctx, node, "softmax");
    if (inner == 1 && dim % 4 == 0 && dim <= 2048 && outer < (size_t(1) << 26)) {  // 64 * rows work-items < 2^32
        const bool nt = outer * dim * sizeof(float) >= (size_t(8) << 20);
        using RowKernel = void (*)(const float *, float *, int);
        const RowKernel k = dim <= 1024 ? (nt ? softmax_rows_reg<4, true> : softmax_rows_reg<4, false>)
                                        : (nt ? softmax_rows_reg<8, true> : softmax_rows_reg<8, false>);
        hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(outer)), dim3(64), 0, ctx->stream, x, y, dim);
    } else if (inner == 1)
        hipLaunchKernelGGL(softmax_rows, dim3(blocks_for(outer, 4)), dim3(256), 0, ctx->stream, x, y, outer, dim);
    else
        hipLaunchKernelGGL(dim <= 16 ? softmax_strided_reg<16> : dim <= 32 ? softmax_strided_reg<32> : softmax_strided,
                           dim3(grid_for(outer * inner, 256)), dim3(256), 0, ctx->stream, x, y, outer,
                           dim, inner);
    return launch_status("softmax");
}

// ReduceMean / ReduceMax (reference reduce/reduce.c).  Axes come from a
// second (weight) input holding float axis values, else from the attr extra
// list, else all axes (kernel_common.c:50-81).
int reduce_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    Spkv2AttrRecord attr;
    if (int rc = spkv2_ctx_get_attr(ctx, node, &attr)) return rc;
    const Spkv2TensorRecord *xr = rec(ctx, node->inputs[0]);
    const int rank = xr->rank;
    bool reduced[kMaxRank] = {false};
    int naxes = 0;
    if (node->input_count > 1) {
        const Spkv2TensorRecord *ar = rec(ctx, node->inputs[1]);
        const float *av = reinterpret_cast<const float *>(host_weight_data(ctx, node->inputs[1]));
        if (!av) return SPKV2_E_UNSUPPORTED;  // axes computed at run time
        const size_t cnt = elem_count(ar);
        if (cnt > 8) return -11;
        for (size_t i = 0; i < cnt; i++) {
            const int ax = axis_norm(static_cast<int>(av[i]), rank);
            if (ax < 0 || ax >= rank) return -11;
            if (!reduced[ax]) naxes++;
            reduced[ax] = true;
        }
    } else if (attr.extra_count > 0) {
        if (attr.extra_count > 8) return -11;
        for (int i = 0; i < attr.extra_count; i++) {
            const int ax = axis_norm(attr.extra[i], rank);
            if (ax < 0 || ax >= rank) return -11;
            if (!reduced[ax]) naxes++;
            reduced[ax] = true;
        }
    } else {
        for (int i = 0; i < rank; i++) reduced[i] = true;
        naxes = rank;
    }
    if (q8_tensor(ctx, node->inputs[0])) {
        // an int8 activation: ReduceMean over H, W only
        if (node->op_type != SPKV2_OP_REDUCEMEAN || rank != 4 || naxes != 2 || !reduced[2] || !reduced[3])
            return SPKV2_E_UNSUPPORTED;
        return mean_q8_run(ctx, node);
    }
    float denom = 1.0f;
    for (int i = 0; i < rank; i++)
        if (reduced[i]) denom *= static_cast<float>(xr->shape[i]);
    const bool is_max = node->op_type == SPKV2_OP_REDUCEMAX;
    const float *x = dptr<const float>(ctx, node->inputs[0]);
    float *y = dptr<float>(ctx, node->outputs[0]);
    set_kernel_name(ctx, node, is_max ? "reduce_max" : "reduce_mean");

    // trailing contiguous axes -> one wave per output row
    int first = rank;
    for (int i = rank - 1; i >= 0 && reduced[i]; i--) first = i;
    int n_trailing = rank - first;
    if (n_trailing == naxes && naxes > 0) {
        size_t rows = 1, len = 1;
        for (int i = 0; i < first; i++) rows *= xr->shape[i];
        for (int i = first; i < rank; i++) len *= xr->shape[i];
        if (rows * len == 0) return 0;
        if (is_max && len <= 128)
            hipLaunchKernelGGL(row_max16, dim3(blocks_for(rows, 16)), dim3(256), 0, ctx->stream, x, y, rows,
                               static_cast<int>(len));
        else if (is_max)
            hipLaunchKernelGGL(row_reduce<1>, dim3(blocks_for(rows, 4)), dim3(256), 0, ctx->stream, x, y, rows,
                               static_cast<int>(len), denom);
        else
            hipLaunchKernelGGL(row_reduce<0>, dim3(blocks_for(rows, 4)), dim3(256), 0, ctx->stream, x, y, rows,
                               static_cast<int>(len), denom);
        return launch_status("reduce");
    }
    ReduceDesc d{};
    int64_t stride[kMaxRank];
    int64_t s = 1;
    for (int i = rank - 1; i >= 0; i--) {
        stride[i] = s;
        s *= xr->shape[i];
    }
    d.rcount = 1;
    size_t nout = 1;
    for (int i = 0; i < rank; i++) {
        if (reduced[i]) {
            d.rdim[d.nr] = xr->shape[i];
            d.rstride[d.nr++] = stride[i];
            d.rcount *= xr->shape[i];
        } else {
            d.odim[d.no] = xr->shape[i];
            d.ostride[d.no++] = stride[i];
            nout *= xr->shape[i];
        }
    }
    if (nout == 0) return 0;
    if (is_max)
        hipLaunchKernelGGL(generic_reduce<1>, dim3(grid_for(nout, 256)), dim3(256), 0, ctx->stream, x, y, nout, d, denom);
    else
        hipLaunchKernelGGL(generic_reduce<0>, dim3(grid_for(nout, 256)), dim3(256), 0, ctx->stream, x, y, nout, d, denom);
    return launch_status("reduce");
}

// Exact 2x nearest upsampling (OH == 2H, OW == 2W, W even; the reference's
// floor(o / 2) index): each thread reads 2 input columns (8 bytes) and
// writes them doubled to both output rows (two 16-byte stores).
__global__ void __launch_bounds__(256) resize2x_x2(const float *__restrict__ x, float *__restrict__ y, unsigned planes,
                                                   int H, int W, unsigned C, size_t y_img) {
    const unsigned pairs = static_cast<unsigned>(H * (W / 2));
    const int OW = 2 * W;
    for (unsigned plane = blockIdx.y; plane < planes; plane += gridDim.y) {
        const float *xp = x + static_cast<size_t>(plane) * H * W;
        // y's images y_img elements apart (a Concat buffer's channel slice, or C * 4HW)
        const unsigned img = plane / C;
        float *yp = y + img * y_img + static_cast<size_t>(plane - img * C) * 4 * H * W;
        for (unsigned q = blockIdx.x * 256 + threadIdx.x; q < pairs; q += gridDim.x * 256) {
            const int ih = static_cast<int>(q / static_cast<unsigned>(W / 2));
            const int iw = 2 * (static_cast<int>(q) - ih * (W / 2));
            const floatx2 v = *reinterpret_cast<const floatx2 *>(xp + ih * W + iw);
            const floatx4 o = floatx4{v[0], v[0], v[1], v[1]};
            *reinterpret_cast<floatx4 *>(yp + (2 * ih) * OW + 2 * iw) = o;
            *reinterpret_cast<floatx4 *>(yp + (2 * ih + 1) * OW + 2 * iw) = o;
        }
    }
}

int resize_run(Spkv2Context *ctx, const Spkv2NodeRecord *node, void *) {
    const Spkv2TensorRecord *xr = rec(ctx, node->inputs[0]), *yr = rec(ctx, node->outputs[0]);
    if (xr->rank != 4 || yr->rank != 4) return -11;
    const int N = yr->shape[0], C = yr->shape[1], OH = yr->shape[2], OW = yr->shape[3];
    const int H = xr->shape[2], W = xr->shape[3];
    const size_t total = static_cast<size_t>(N) * C * OH * OW;
    if (total == 0) return 0;
    if (OH == 2 * H && OW == 2 * W && W % 2 == 0 && static_cast<int>(xr->shape[0]) == N &&
        static_cast<int>(xr->shape[1]) == C) {
        set_kernel_name(ctx, node, "resize2x_x2");
        const size_t pairs = static_cast<size_t>(H) * (W / 2), planes = static_cast<size_t>(N) * C;
        if (pairs > 0x7fffffffULL || planes > 0x7fffffffULL) return SPKV2_E_UNSUPPORTED;
        const dim3 grid(static_cast<unsigned>(std::min<size_t>((pairs + 255) / 256, 1024)),
                        static_cast<unsigned>(std::min<size_t>(planes, 65535)));
        float *y = dptr<float>(ctx, node->outputs[0]);
        size_t y_img = static_cast<size_t>(C) * OH * OW;
        if (const Spkv2TensorView *v = live_view(ctx, node->outputs[0])) {  // written into a Concat's buffer
            y = reinterpret_cast<float *>(v->base);
            y_img = static_cast<size_t>(v->img_elems);
        }
        hipLaunchKernelGGL(resize2x_x2, grid, dim3(256), 0, ctx->stream, dptr<const float>(ctx, node->inputs[0]), y,
                           static_cast<unsigned>(planes), H, W, static_cast<unsigned>(C), y_img);
        return launch_status("resize");
    }
    if (live_view(ctx, node->outputs[0])) return SPKV2_E_UNSUPPORTED;  // views only for the 2x path
    const float scale_h = static_cast<float>(OH) / static_cast<float>(H);
    const float scale_w = static_cast<float>(OW) / static_cast<float>(W);
    set_kernel_name(ctx, node, "resize_nearest");
    hipLaunchKernelGGL(resize_nearest, dim3(grid_for(total, 256)), dim3(256), 0, ctx->stream,
                       dptr<const float>(ctx, node->inputs[0]), dptr<float>(ctx, node->outputs[0]), N, C, H, W, OH, OW,
                       scale_h, scale_w);
    return launch_status("resize");
}

int flip_bit(hipStream_t s, void *data, uint64_t element, uint32_t bit) {
    hipLaunchKernelGGL(flip_bit_kernel, dim3(1), dim3(1), 0, s, static_cast<uint32_t *>(data) + element, bit);
    return launch_status("flip_bit");
}

int minmax(hipStream_t s, const float *x, size_t n, float *dev_out4) {
    hipLaunchKernelGGL(minmax_kernel, dim3(1), dim3(256), 0, s, x, n, dev_out4);
    return launch_status("minmax");
}

int fill_u32(hipStream_t s, uint32_t *p, size_t n, uint32_t v) {
    hipLaunchKernelGGL(fill_u32_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, p, n, v);
    return launch_status("fill_u32");
}

int compare_bytes(hipStream_t s, const void *a, const void *b, size_t n, uint32_t *dev_flag) {
    if (int rc = fill_u32(s, dev_flag, 1, 0u)) return rc;
    if (n == 0) return 0;
    hipLaunchKernelGGL(compare_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, static_cast<const uint8_t *>(a),
                       static_cast<const uint8_t *>(b), n, dev_flag);
    return launch_status("compare");
}

}  // namespace spk::kern
