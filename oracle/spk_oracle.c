/*
 * CPU oracle for the MI355X hot path: plain C restatement of the reference
 * kernels.  TEST INFRASTRUCTURE ONLY (see spk_oracle.h).
 *
 * Built with -ffp-contract=off, so the compiler fuses nothing on its own;
 * the multiply-adds the reference's release build fuses are written as
 * explicit fmaf.  The reference's CMake build (runtime/CMakeLists.txt:8-14)
 * adds -mfma on x86, and gcc then contracts `sum += a * b` in the conv,
 * Gemm and MatMul loops and `alpha * sum + bias` in Gemm into one fused
 * multiply-add each; the INT8 dequantize is an fmaf because the
 * reference's vector path fuses it (vfmaq_f32).  With this, the oracle's
 * conv / Gemm / MatMul outputs equal the reference runtime's bit for bit.
 * OpenMP splits work across output planes only, so each output element is
 * computed by exactly the sequential arithmetic shown.
 */
#include "spk_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static float act_scalar(float v, int act) {
    if (act == 1) return v > 0.0f ? v : 0.0f;
    if (act == 2) return v / (1.0f + expf(-v));
    return v;
}

/* reference kernels/reference/conv/conv.c:31-59: accumulate from the bias in
 * the order c -> kh -> kw, skip out-of-bounds taps, add the residual, then
 * apply the activation */
int oracle_conv2d_f32(const float *x, const float *w, const float *bias, const float *res, float *y, int N, int C,
                      int H, int W, int M, int KH, int KW, int OH, int OW, int sh, int sw, int ph, int pw, int dh,
                      int dw, int group, int act) {
    if (group <= 0) group = 1;
    if (C % group != 0 || M % group != 0) return -12;
    const int Cg = C / group, Mg = M / group;
#pragma omp parallel for collapse(2) schedule(static)
    for (int n = 0; n < N; n++) {
        for (int m = 0; m < M; m++) {
            const int c0 = (m / Mg) * Cg;
            for (int oh = 0; oh < OH; oh++) {
                for (int ow = 0; ow < OW; ow++) {
                    float sum = bias ? bias[m] : 0.0f;
                    for (int c = 0; c < Cg; c++) {
                        for (int kh = 0; kh < KH; kh++) {
                            const int ih = oh * sh + kh * dh - ph;
                            if (ih < 0 || ih >= H) continue;
                            for (int kw = 0; kw < KW; kw++) {
                                const int iw = ow * sw + kw * dw - pw;
                                if (iw < 0 || iw >= W) continue;
                                sum = fmaf(x[(((size_t)n * C + c0 + c) * H + ih) * W + iw],
                                           w[(((size_t)m * Cg + c) * KH + kh) * KW + kw], sum);
                            }
                        }
                    }
                    const size_t yi = (((size_t)n * M + m) * OH + oh) * OW + ow;
                    if (res) sum += res[yi];
                    y[yi] = act_scalar(sum, act);
                }
            }
        }
    }
    return 0;
}

/* reference kernels/reference/mm/gemm.c:17-31.  Rounding of the k loop as
 * the reference's release build executes it: when both operands run
 * contiguously along k (trans_a == 0, trans_b == 1) gcc vectorizes the
 * products (8- then 4-wide multiplies, each rounded) and adds them to the
 * sum one by one in k order, and only the last K % 4 terms are fused
 * multiply-adds; otherwise every term is a fused multiply-add. */
void oracle_gemm_f32(const float *a, const float *b, const float *c, float *y, int rows, int K, int nout,
                     int trans_a, int trans_b, float alpha) {
    const int k_split = (!trans_a && trans_b) ? (K & ~3) : 0;
#pragma omp parallel for schedule(static)
    for (int m = 0; m < rows; m++) {
        for (int n = 0; n < nout; n++) {
            float sum = 0.0f;
            for (int k = 0; k < K; k++) {
                const float av = trans_a ? a[(size_t)k * rows + m] : a[(size_t)m * K + k];
                const float bv = trans_b ? b[(size_t)n * K + k] : b[(size_t)k * nout + n];
                if (k < k_split) {
                    const float prod = av * bv;
                    sum = sum + prod;
                } else {
                    sum = fmaf(av, bv, sum);
                }
            }
            y[(size_t)m * nout + n] = fmaf(alpha, sum, c ? c[n] : 0.0f);
        }
    }
}

/* reference kernels/reference/mm/matmul.c:40-46 */
void oracle_matmul_f32(const float *a, const float *b, float *y, int batch, const int64_t *a_off,
                       const int64_t *b_off, int M, int K, int N) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int bi = 0; bi < batch; bi++) {
        for (int m = 0; m < M; m++) {
            const float *ab = a + a_off[bi];
            const float *bb = b + b_off[bi];
            for (int n = 0; n < N; n++) {
                float sum = 0.0f;
                for (int k = 0; k < K; k++) sum = fmaf(ab[(size_t)m * K + k], bb[(size_t)k * N + n], sum);
                y[((size_t)bi * M + m) * N + n] = sum;
            }
        }
    }
}

/* reference kernels/reference/pool/maxpool.c:20-40 */
void oracle_maxpool_f32(const float *x, float *y, int N, int C, int H, int W, int OH, int OW, int kh, int kw, int sh,
                        int sw, int ph, int pw) {
    for (size_t plane = 0; plane < (size_t)N * C; plane++) {
        const float *xp = x + plane * H * W;
        for (int oh = 0; oh < OH; oh++) {
            for (int ow = 0; ow < OW; ow++) {
                float m = -INFINITY;
                for (int i = 0; i < kh; i++) {
                    const int ih = oh * sh + i - ph;
                    if (ih < 0 || ih >= H) continue;
                    for (int j = 0; j < kw; j++) {
                        const int iw = ow * sw + j - pw;
                        if (iw < 0 || iw >= W) continue;
                        const float v = xp[ih * W + iw];
                        if (v > m) m = v;
                    }
                }
                y[(plane * OH + oh) * OW + ow] = m;
            }
        }
    }
}

/* reference kernels/reference/pool/avgpool.c:21-45 */
void oracle_avgpool_f32(const float *x, float *y, int N, int C, int H, int W, int OH, int OW, int kh, int kw, int sh,
                        int sw, int ph, int pw) {
    for (size_t plane = 0; plane < (size_t)N * C; plane++) {
        const float *xp = x + plane * H * W;
        for (int oh = 0; oh < OH; oh++) {
            for (int ow = 0; ow < OW; ow++) {
                float sum = 0.0f;
                int count = 0;
                for (int i = 0; i < kh; i++) {
                    const int ih = oh * sh + i - ph;
                    if (ih < 0 || ih >= H) continue;
                    for (int j = 0; j < kw; j++) {
                        const int iw = ow * sw + j - pw;
                        if (iw < 0 || iw >= W) continue;
                        sum += xp[ih * W + iw];
                        count++;
                    }
                }
                y[(plane * OH + oh) * OW + ow] = count > 0 ? sum / (float)count : 0.0f;
            }
        }
    }
}

/* reference kernels/reference/pool/avgpool.c:60-68 */
void oracle_global_avgpool_f32(const float *x, float *y, int N, int C, int HW) {
    const float inv = 1.0f / (float)HW;
    for (size_t plane = 0; plane < (size_t)N * C; plane++) {
        float sum = 0.0f;
        for (int i = 0; i < HW; i++) sum += x[plane * HW + i];
        y[plane] = sum * inv;
    }
}

/* broadcast index of reference kernel_common.c:37-48 */
static size_t bcast_index(size_t out, const uint32_t *in_shape, int in_rank, const uint32_t *y_shape, int y_rank) {
    uint32_t coords[8] = {0};
    size_t t = out;
    for (int i = y_rank - 1; i >= 0; i--) {
        coords[i] = y_shape[i] ? (uint32_t)(t % y_shape[i]) : 0;
        t = y_shape[i] ? t / y_shape[i] : 0;
    }
    const int delta = y_rank - in_rank;
    size_t idx = 0;
    for (int i = 0; i < in_rank; i++) idx = idx * in_shape[i] + (in_shape[i] == 1 ? 0 : coords[i + delta]);
    return idx;
}

int oracle_binary_f32(int op, const float *a, const uint32_t *a_shape, int a_rank, const float *b,
                      const uint32_t *b_shape, int b_rank, float *y, const uint32_t *y_shape, int y_rank, int act) {
    size_t n = 1;
    for (int i = 0; i < y_rank; i++) n *= y_shape[i];
    for (size_t i = 0; i < n; i++) {
        const float av = a[bcast_index(i, a_shape, a_rank, y_shape, y_rank)];
        const float bv = b[bcast_index(i, b_shape, b_rank, y_shape, y_rank)];
        float v;
        switch (op) {
        case 1: v = act_scalar(av + bv, act); break;  /* add.c:16-17 */
        case 8: v = av * bv; break;                    /* binary.c:17-27 */
        case 9: v = av - bv; break;
        case 10: v = av / bv; break;
        case 11: v = (int)bv == 0 ? 0.0f : (float)((int)av % (int)bv); break;
        default: return -99;
        }
        y[i] = v;
    }
    return 0;
}

void oracle_relu_f32(const float *x, float *y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = x[i] > 0.0f ? x[i] : 0.0f;
}

void oracle_sigmoid_f32(const float *x, float *y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = 1.0f / (1.0f + expf(-x[i]));
}

/* reference kernels/reference/activation/softmax.c:22-38 */
void oracle_softmax_f32(const float *x, float *y, size_t outer, size_t dim, size_t inner) {
    for (size_t o = 0; o < outer; o++) {
        for (size_t in = 0; in < inner; in++) {
            float m = -INFINITY;
            for (size_t d = 0; d < dim; d++) {
                const float v = x[(o * dim + d) * inner + in];
                if (v > m) m = v;
            }
            float sum = 0.0f;
            for (size_t d = 0; d < dim; d++) {
                const float e = expf(x[(o * dim + d) * inner + in] - m);
                y[(o * dim + d) * inner + in] = e;
                sum += e;
            }
            for (size_t d = 0; d < dim; d++) y[(o * dim + d) * inner + in] /= sum;
        }
    }
}

/* reference kernels/reference/reduce/reduce.c:19-44: y starts at 0 (or
 * -inf), then every x element in order adds x/denom (or takes the max) */
void oracle_reduce_f32(const float *x, const uint32_t *x_shape, int rank, uint32_t axis_mask, int is_max, float *y) {
    size_t nx = 1, ny = 1;
    float denom = 1.0f;
    uint32_t y_shape[8];
    int yr = 0;
    for (int i = 0; i < rank; i++) {
        nx *= x_shape[i];
        if (axis_mask & (1u << i)) denom *= (float)x_shape[i];
        else {
            ny *= x_shape[i];
            y_shape[yr++] = x_shape[i];
        }
    }
    for (size_t i = 0; i < ny; i++) y[i] = is_max ? -INFINITY : 0.0f;
    for (size_t xi = 0; xi < nx; xi++) {
        size_t t = xi, yi = 0, mul = 1;
        for (int i = rank - 1; i >= 0; i--) {
            const size_t c = t % x_shape[i];
            t /= x_shape[i];
            if (!(axis_mask & (1u << i))) {
                yi += c * mul;
                mul *= x_shape[i];
            }
        }
        if (is_max) {
            if (x[xi] > y[yi]) y[yi] = x[xi];
        } else {
            y[yi] += x[xi] / denom;
        }
    }
    (void)y_shape;
}

/* reference kernels/reference/shape/resize.c:14-28 */
void oracle_resize_nearest_f32(const float *x, float *y, int N, int C, int H, int W, int OH, int OW) {
    const float scale_h = (float)OH / (float)H;
    const float scale_w = (float)OW / (float)W;
    for (size_t plane = 0; plane < (size_t)N * C; plane++) {
        for (int oh = 0; oh < OH; oh++) {
            int ih = (int)floorf((float)oh / scale_h);
            if (ih >= H) ih = H - 1;
            for (int ow = 0; ow < OW; ow++) {
                int iw = (int)floorf((float)ow / scale_w);
                if (iw >= W) iw = W - 1;
                y[(plane * OH + oh) * OW + ow] = x[(plane * H + ih) * W + iw];
            }
        }
    }
}

/* ------------------------------------------------------------------ INT8 */

static int8_t sat8(float r) {
    if (r != r) return 0; /* the ARM conversions map NaN to 0 */
    if (r < -128.0f) return -128;
    if (r > 127.0f) return 127;
    return (int8_t)(int)r;
}

/* reference conv_int8.c:22-56: the 16-wide vector loop converts with
 * vcvtnq (round half to even) and narrows with saturation; the scalar tail
 * uses roundf (half away from zero) and a clamp */
void oracle_quantize_act(const float *x, int8_t *q, size_t count, float scale) {
    const float inv = 1.0f / scale;
    const size_t split = count / 16 * 16;
    for (size_t i = 0; i < count; i++) {
        const float v = x[i] * inv;
        q[i] = sat8(i < split ? nearbyintf(v) : roundf(v));
    }
}

/* reference conv_int8.c:58-84 (zero-padded im2col) and the exact integer
 * GEMM of int8_gemm.c, written as the closed-form sum */
void oracle_conv_int8_acc(const int8_t *xq, const int8_t *wq, int32_t *acc, int N, int C, int H, int W, int M,
                          int KH, int KW, int OH, int OW, int sh, int sw, int ph, int pw, int dh, int dw) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int n = 0; n < N; n++) {
        for (int m = 0; m < M; m++) {
            for (int oh = 0; oh < OH; oh++) {
                for (int ow = 0; ow < OW; ow++) {
                    int64_t s = 0;
                    for (int c = 0; c < C; c++)
                        for (int kh = 0; kh < KH; kh++) {
                            const int ih = oh * sh - ph + kh * dh;
                            if (ih < 0 || ih >= H) continue;
                            for (int kw = 0; kw < KW; kw++) {
                                const int iw = ow * sw - pw + kw * dw;
                                if (iw < 0 || iw >= W) continue;
                                s += (int64_t)wq[(((size_t)m * C + c) * KH + kh) * KW + kw] *
                                     (int64_t)xq[(((size_t)n * C + c) * H + ih) * W + iw];
                            }
                        }
                    acc[(((size_t)n * M + m) * OH + oh) * OW + ow] = (int32_t)s;
                }
            }
        }
    }
}

/* reference conv_int8.c:92-118 */
void oracle_dequant(const int32_t *acc, const float *w_scales, float x_scale, const float *bias, const float *res,
                    float *y, int N, int M, int spatial, int act) {
    for (int n = 0; n < N; n++)
        for (int m = 0; m < M; m++) {
            const float scale = w_scales[m] * x_scale;
            const float b = bias ? bias[m] : 0.0f;
            for (int j = 0; j < spatial; j++) {
                const size_t i = ((size_t)n * M + m) * spatial + j;
                float v = fmaf((float)acc[i], scale, b);
                if (res) v += res[i];
                y[i] = act_scalar(v, act);
            }
        }
}

int oracle_conv2d_int8(const float *x, const int8_t *wq, const float *w_scales, float x_scale, const float *bias,
                       const float *res, float *y, int32_t *acc_out, int N, int C, int H, int W, int M, int KH,
                       int KW, int OH, int OW, int sh, int sw, int ph, int pw, int dh, int dw, int act) {
    const size_t chw = (size_t)C * H * W;
    int8_t *xq = (int8_t *)calloc(chw * N + 1, 1);
    int32_t *acc = acc_out ? acc_out : (int32_t *)malloc((size_t)N * M * OH * OW * sizeof(int32_t) + 4);
    if (!xq || !acc) {
        free(xq);
        if (!acc_out) free(acc);
        return -1;
    }
    for (int n = 0; n < N; n++) oracle_quantize_act(x + n * chw, xq + n * chw, chw, x_scale);
    oracle_conv_int8_acc(xq, wq, acc, N, C, H, W, M, KH, KW, OH, OW, sh, sw, ph, pw, dh, dw);
    oracle_dequant(acc, w_scales, x_scale, bias, res, y, N, M, OH * OW, act);
    free(xq);
    if (!acc_out) free(acc);
    return 0;
}

/* ------------------------------------------- INT8 with int8 tensors (Q8)
 *
 * The INT8 configuration the benchmark names (per-channel symmetric int8
 * weights, per-tensor asymmetric int8 activations between nodes, int32
 * accumulation, fixed-point requantization with round-half-away, fused Relu
 * clamp).  The reference runtime has no such mode: its INT8 conv keeps fp32
 * tensors between nodes with zero point 0 (conv_int8.c:121-210,
 * compiler/quantization/calibrate.py:16).  This is the mode's definition,
 * restated independently of the device code; tests/test_oracle_q8.py pins it
 * with int64 brute force, the zero-point identity, and exact rationals. */

/* t / 2^s rounded to nearest, ties away from zero (s >= 1) */
int64_t oracle_q8_round_shift(int64_t t, int s) {
    const int64_t half = (int64_t)1 << (s - 1);
    if (t >= 0) return (t + half) >> s;
    return -((-t + half) >> s);
}

static double rha_double(double v) { return v >= 0.0 ? floor(v + 0.5) : -floor(-v + 0.5); }

/* Per output channel m: bias_q[m] = round_half_away(bias[m] / (s_x s_w[m]))
 * clamped to +-2^30, and the fixed-point multipliers of
 *   R1 = (s_x s_w[m]) / s_y  (accumulator -> output units)
 *   R2 = s_r / s_y           (residual -> output units; 0 without one)
 * with one shift S[m] for both: S = 31 - e where max(R1, R2) = f 2^e,
 * f in [0.5, 1), and Mi = floor(Ri 2^S + 0.5), one less S if that reaches
 * 2^31.  Returns -1 when S leaves [1, 62]. */
int oracle_q8_requant_params(float s_x, const float *s_w, float s_y, float s_r, const float *bias, int M,
                             int32_t *bias_q, int32_t *m1, int32_t *m2, int32_t *shift) {
    for (int m = 0; m < M; m++) {
        const double r1 = ((double)s_x * (double)s_w[m]) / (double)s_y;
        const double r2 = s_r > 0.0f ? (double)s_r / (double)s_y : 0.0;
        const double rmax = r1 > r2 ? r1 : r2;
        int e = 0;
        (void)frexp(rmax, &e);
        int sh = 31 - e;
        double a = floor(ldexp(r1, sh) + 0.5), b = floor(ldexp(r2, sh) + 0.5);
        if (a >= 2147483648.0 || b >= 2147483648.0) {
            sh -= 1;
            a = floor(ldexp(r1, sh) + 0.5);
            b = floor(ldexp(r2, sh) + 0.5);
        }
        if (sh < 1 || sh > 62) return -1;
        m1[m] = (int32_t)a;
        m2[m] = (int32_t)b;
        shift[m] = sh;
        double bq = bias ? rha_double((double)bias[m] / ((double)s_x * (double)s_w[m])) : 0.0;
        if (bq > 1073741824.0) bq = 1073741824.0;
        if (bq < -1073741824.0) bq = -1073741824.0;
        bias_q[m] = (int32_t)bq;
    }
    return 0;
}

/* fp32 -> int8 with (s, z): sat8(roundf(x * (1/s)) + z), NaN -> z */
void oracle_q8_quantize(const float *x, int8_t *q, size_t count, float scale, int zp) {
    const float inv = 1.0f / scale;
    for (size_t i = 0; i < count; i++) {
        const float t = x[i] * inv;
        int v = zp;
        if (t == t) {
            float r = roundf(t);
            if (r < -512.0f) r = -512.0f;
            if (r > 512.0f) r = 512.0f;
            v = (int)r + zp;
        }
        q[i] = (int8_t)(v < -128 ? -128 : v > 127 ? 127 : v);
    }
}

/* one requantized output: q = rha((acc + bq) m1 + (r - z_r) m2, S) + z_y,
 * Relu as max(q, z_y), saturated */
int oracle_q8_requant_one(int32_t acc, int32_t bq, int32_t m1, int32_t m2, int32_t sh, int r, int zy, int relu) {
    const int64_t t = ((int64_t)acc + bq) * (int64_t)m1 + (int64_t)r * (int64_t)m2;
    int64_t q = oracle_q8_round_shift(t, sh) + zy;
    if (relu && q < zy) q = zy;
    return (int)(q < -128 ? -128 : q > 127 ? 127 : q);
}

/* Conv over NCHW int8 x with zero point zx: acc = sum over in-bounds taps of
 * w (x - zx) (out-of-bounds taps are real zeros), then requantized into y
 * (NCHW int8, zero point zy) with the residual res (NCHW int8, zero point
 * zr) when given.  acc_out (optional) receives the int32 accumulators. */
void oracle_q8_conv(const int8_t *x, int zx, const int8_t *wq, const int32_t *bias_q, const int32_t *m1,
                    const int32_t *m2, const int32_t *shift, const int8_t *res, int zr, int zy, int relu, int8_t *y,
                    int32_t *acc_out, int N, int C, int H, int W, int M, int KH, int KW, int OH, int OW, int sh,
                    int sw, int ph, int pw, int dh, int dw) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int n = 0; n < N; n++) {
        for (int m = 0; m < M; m++) {
            for (int oh = 0; oh < OH; oh++) {
                for (int ow = 0; ow < OW; ow++) {
                    int64_t s = 0;
                    for (int c = 0; c < C; c++)
                        for (int kh = 0; kh < KH; kh++) {
                            const int ih = oh * sh - ph + kh * dh;
                            if (ih < 0 || ih >= H) continue;
                            for (int kw = 0; kw < KW; kw++) {
                                const int iw = ow * sw - pw + kw * dw;
                                if (iw < 0 || iw >= W) continue;
                                s += (int64_t)wq[(((size_t)m * C + c) * KH + kh) * KW + kw] *
                                     ((int64_t)x[(((size_t)n * C + c) * H + ih) * W + iw] - zx);
                            }
                        }
                    const size_t yi = (((size_t)n * M + m) * OH + oh) * OW + ow;
                    if (acc_out) acc_out[yi] = (int32_t)s;
                    const int r = res ? (int)res[yi] - zr : 0;
                    y[yi] = (int8_t)oracle_q8_requant_one((int32_t)s, bias_q[m], m1[m], m2[m], shift[m], r, zy, relu);
                }
            }
        }
    }
}

/* MaxPool over NCHW int8 (one (s, z) for input and output): the maximum of
 * the in-bounds taps */
void oracle_q8_maxpool(const int8_t *x, int8_t *y, int N, int C, int H, int W, int OH, int OW, int kh, int kw, int sh,
                       int sw, int ph, int pw) {
    for (size_t plane = 0; plane < (size_t)N * C; plane++)
        for (int oh = 0; oh < OH; oh++)
            for (int ow = 0; ow < OW; ow++) {
                int best = -129;
                for (int i = 0; i < kh; i++) {
                    const int ih = oh * sh - ph + i;
                    if (ih < 0 || ih >= H) continue;
                    for (int j = 0; j < kw; j++) {
                        const int iw = ow * sw - pw + j;
                        if (iw < 0 || iw >= W) continue;
                        const int v = x[(plane * H + ih) * W + iw];
                        if (v > best) best = v;
                    }
                }
                y[(plane * OH + oh) * OW + ow] = (int8_t)(best < -128 ? -128 : best);
            }
}

/* mean over each of `planes` planes of `hw` int8 values with (s, z), to
 * fp32: (float)(((double)sum(q - z) * s) / hw) */
void oracle_q8_plane_mean(const int8_t *x, float *y, size_t planes, int hw, float scale, int zp) {
    for (size_t p = 0; p < planes; p++) {
        int64_t sum = 0;
        for (int i = 0; i < hw; i++) sum += (int64_t)x[p * hw + i] - zp;
        y[p] = (float)(((double)sum * (double)scale) / (double)hw);
    }
}

/* ------------------------------------------------------------------ TopK */

typedef struct {
    float v;
    uint32_t idx;
} OracleTopkPair;

/* reference tensor/topk.c:7-17 (min-heap) and 19-29 (max-heap) */
static void topk_sift(OracleTopkPair *h, size_t n, size_t i, int min_heap) {
    for (;;) {
        size_t l = 2 * i + 1, r = 2 * i + 2, m = i;
        if (min_heap) {
            if (l < n && h[l].v < h[m].v) m = l;
            if (r < n && h[r].v < h[m].v) m = r;
        } else {
            if (l < n && h[l].v > h[m].v) m = l;
            if (r < n && h[r].v > h[m].v) m = r;
        }
        if (m == i) break;
        OracleTopkPair t = h[i];
        h[i] = h[m];
        h[m] = t;
        i = m;
    }
}

/* reference tensor/topk.c:31-48: best first, ties by smaller index */
static int topk_cmp_desc(const void *a, const void *b) {
    float av = ((const OracleTopkPair *)a)->v, bv = ((const OracleTopkPair *)b)->v;
    if (av < bv) return 1;
    if (av > bv) return -1;
    return ((const OracleTopkPair *)a)->idx < ((const OracleTopkPair *)b)->idx ? -1 : 1;
}

static int topk_cmp_asc(const void *a, const void *b) {
    float av = ((const OracleTopkPair *)a)->v, bv = ((const OracleTopkPair *)b)->v;
    if (av < bv) return -1;
    if (av > bv) return 1;
    return ((const OracleTopkPair *)a)->idx < ((const OracleTopkPair *)b)->idx ? -1 : 1;
}

void oracle_topk_row(const float *x, size_t inner, int dim, int k, int largest, float *values, float *indices) {
    if (k <= 0 || dim <= 0) return;
    if (k > dim) k = dim;
    OracleTopkPair *h = (OracleTopkPair *)malloc((size_t)k * sizeof(OracleTopkPair));
    if (!h) return;
    for (int d = 0; d < k; d++) {
        h[d].v = x[(size_t)d * inner];
        h[d].idx = (uint32_t)d;
    }
    for (long i = (long)(k / 2) - 1; i >= 0; i--) topk_sift(h, (size_t)k, (size_t)i, largest);
    for (int d = k; d < dim; d++) {
        const float v = x[(size_t)d * inner];
        if (largest ? (v > h[0].v) : (v < h[0].v)) {
            h[0].v = v;
            h[0].idx = (uint32_t)d;
            topk_sift(h, (size_t)k, 0, largest);
        }
    }
    qsort(h, (size_t)k, sizeof(OracleTopkPair), largest ? topk_cmp_desc : topk_cmp_asc);
    for (int j = 0; j < k; j++) {
        values[(size_t)j * inner] = h[j].v;
        indices[(size_t)j * inner] = (float)h[j].idx;
    }
    free(h);
}
