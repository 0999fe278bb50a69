/*
 * CPU oracle: a plain-C restatement of the reference SPINNV2 kernels on the
 * MI355X hot path, with plain pointer + shape signatures.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py call it, always as the checker, never as the
 * thing measured or shipped.  The product library never links it.
 *
 * Layouts: activations NCHW fp32, conv weights OIHW, Gemm operands row-major.
 * act: 0 none, 1 Relu, 2 SiLU (reference kernel_common.c:100-108).
 */
#ifndef SPK_ORACLE_H
#define SPK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference kernels/reference/conv/conv.c:3-62 */
int oracle_conv2d_f32(const float *x, const float *w, const float *bias, const float *res, float *y, int N, int C,
                      int H, int W, int M, int KH, int KW, int OH, int OW, int sh, int sw, int ph, int pw, int dh,
                      int dw, int group, int act);

/* reference kernels/reference/mm/gemm.c:3-33 (beta not applied) */
void oracle_gemm_f32(const float *a, const float *b, const float *c, float *y, int rows, int K, int nout,
                     int trans_a, int trans_b, float alpha);

/* reference kernels/reference/mm/matmul.c:3-49 for one broadcast batch list:
 * a_off[i], b_off[i] are the element offsets of batch i's A and B panels */
void oracle_matmul_f32(const float *a, const float *b, float *y, int batch, const int64_t *a_off,
                       const int64_t *b_off, int M, int K, int N);

/* reference kernels/reference/pool/maxpool.c:5-43 */
void oracle_maxpool_f32(const float *x, float *y, int N, int C, int H, int W, int OH, int OW, int kh, int kw, int sh,
                        int sw, int ph, int pw);
/* reference kernels/reference/pool/avgpool.c:3-48 */
void oracle_avgpool_f32(const float *x, float *y, int N, int C, int H, int W, int OH, int OW, int kh, int kw, int sh,
                        int sw, int ph, int pw);
/* reference kernels/reference/pool/avgpool.c:50-70 */
void oracle_global_avgpool_f32(const float *x, float *y, int N, int C, int HW);

/* reference kernels/reference/math/add.c:3-20 and math/binary.c:3-33:
 * op 1 Add, 8 Mul, 9 Sub, 10 Div, 11 Mod (SPK op codes); numpy broadcast of
 * a and b onto y via the reference's broadcast index (kernel_common.c:37-48) */
int oracle_binary_f32(int op, const float *a, const uint32_t *a_shape, int a_rank, const float *b,
                      const uint32_t *b_shape, int b_rank, float *y, const uint32_t *y_shape, int y_rank, int act);

/* reference activation/relu.c, activation/sigmoid.c */
void oracle_relu_f32(const float *x, float *y, size_t n);
void oracle_sigmoid_f32(const float *x, float *y, size_t n);

/* reference kernels/reference/activation/softmax.c:5-41 */
void oracle_softmax_f32(const float *x, float *y, size_t outer, size_t dim, size_t inner);

/* reference kernels/reference/reduce/reduce.c:5-45; axis_mask bit i = reduce
 * axis i; is_max selects ReduceMax; y has the kept dims in order */
void oracle_reduce_f32(const float *x, const uint32_t *x_shape, int rank, uint32_t axis_mask, int is_max, float *y);

/* reference kernels/reference/shape/resize.c:5-31 (nearest, floor) */
void oracle_resize_nearest_f32(const float *x, float *y, int N, int C, int H, int W, int OH, int OW);

/* reference kernels/reference/tensor/topk.c:56-121 for one row of `dim`
 * elements at x[d*inner]: heap selection of the k largest (largest=1) or
 * smallest, then sorted best first, ties by smaller index; values and
 * indices written at out[j*inner] */
void oracle_topk_row(const float *x, size_t inner, int dim, int k, int largest, float *values, float *indices);

/* ---- INT8 path (reference kernels/optimized/conv/conv_int8.c) ---- */

/* conv_int8.c:22-56: q = sat8(round(x * (1/scale))), half-to-even for the
 * first floor(count/16)*16 elements, half-away-from-zero for the tail */
void oracle_quantize_act(const float *x, int8_t *q, size_t count, float scale);

/* conv_int8.c:58-84 + int8_gemm.c closed form: acc[n][m][oh][ow] =
 * sum_{c,kh,kw} wq[m][c][kh][kw] * xq[n][c][ih][iw] over in-bounds taps,
 * summed in int64 and narrowed to int32; xq is per-image quantized NCHW */
void oracle_conv_int8_acc(const int8_t *xq, const int8_t *wq, int32_t *acc, int N, int C, int H, int W, int M,
                          int KH, int KW, int OH, int OW, int sh, int sw, int ph, int pw, int dh, int dw);

/* conv_int8.c:86-119: y = act(fmaf((float)acc, w_scale[m]*x_scale, bias[m]) + res) */
void oracle_dequant(const int32_t *acc, const float *w_scales, float x_scale, const float *bias, const float *res,
                    float *y, int N, int M, int spatial, int act);

/* conv_int8.c:121-210 end to end: quantize each image, accumulate,
 * dequantize.  acc_out (optional) receives the int32 accumulators. */
int oracle_conv2d_int8(const float *x, const int8_t *wq, const float *w_scales, float x_scale, const float *bias,
                       const float *res, float *y, int32_t *acc_out, int N, int C, int H, int W, int M, int KH,
                       int KW, int OH, int OW, int sh, int sw, int ph, int pw, int dh, int dw, int act);

/* INT8 with int8 tensors between nodes (the benchmark's INT8 configuration;
 * no reference counterpart): asymmetric per-tensor activations, fixed-point
 * requantization with round-half-away (spk_oracle.c) */
int64_t oracle_q8_round_shift(int64_t t, int s);
int oracle_q8_requant_params(float s_x, const float *s_w, float s_y, float s_r, const float *bias, int M,
                             int32_t *bias_q, int32_t *m1, int32_t *m2, int32_t *shift);
void oracle_q8_quantize(const float *x, int8_t *q, size_t count, float scale, int zp);
int oracle_q8_requant_one(int32_t acc, int32_t bq, int32_t m1, int32_t m2, int32_t sh, int r, int zy, int relu);
void oracle_q8_conv(const int8_t *x, int zx, const int8_t *wq, const int32_t *bias_q, const int32_t *m1,
                    const int32_t *m2, const int32_t *shift, const int8_t *res, int zr, int zy, int relu, int8_t *y,
                    int32_t *acc_out, int N, int C, int H, int W, int M, int KH, int KW, int OH, int OW, int sh,
                    int sw, int ph, int pw, int dh, int dw);
void oracle_q8_maxpool(const int8_t *x, int8_t *y, int N, int C, int H, int W, int OH, int OW, int kh, int kw, int sh,
                       int sw, int ph, int pw);
void oracle_q8_plane_mean(const int8_t *x, float *y, size_t planes, int hw, float scale, int zp);

#ifdef __cplusplus
}
#endif

#endif /* SPK_ORACLE_H */
