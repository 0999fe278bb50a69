// The INT8 configuration with int8 tensors between nodes: the int8
// activation tensors' device buffers, MaxPool over them, and the spatial
// mean that returns to fp32.  (The convolutions of this mode are the int8
// implicit-GEMM kernels of conv_i8.hip with their fixed-point requantizing
// epilogue.)
//
// The reference runtime has no such mode; the package marks the tensors
// (dtype int8, role activation) and carries each one's per-tensor scale and
// zero point in its quantization section (the record's zero-point array,
// reference runtime/include/spkv2_format.h:211-226).  Semantics:
//   MaxPool: the maximum of the in-bounds taps, input and output sharing one
//            scale and zero point;
//   ReduceMean over H, W / GlobalAveragePool: y = (float)((double)sum(q - z)
//            * (double)s / (double)(H*W)), an exact integer sum and two
//            IEEE double operations, so any summation order gives the same
//            bits.
#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "conv.hpp"
#include "kernels.hpp"

namespace spk::kern {

namespace {

// One thread per (output pixel, 16 channels): the in-bounds taps' 16-byte
// pieces, byte-wise maxima, one 16-byte store into the output's padded NHWC
// buffer.  Both buffers have a channel pitch that is a multiple of 16.
// Workgroup b (after the XCD remap below) covers chunk b % chunks of output
// row b / chunks (one wave-uniform division per workgroup; threads along the
// row's OW x C16 pieces).  K > 0: a K x K window, unrolled, every tap's load in
// flight before the first maximum; K = 0: any window.
template <int K>
__global__ void __launch_bounds__(256) maxpool_q8(const int8_t *__restrict__ x, int8_t *__restrict__ y, int chunks,
                                                  int C16, int H, int W, int xHp, int xWp, int xCp, int xpt, int xpl,
                                                  int OH, int OW, int yHp, int yWp, int yCp, int ypt, int ypl, int kh,
                                                  int kw, int sh, int sw, int ph, int pw) {
    typedef signed char char16 __attribute__((ext_vector_type(16)));
    // consecutive workgroups land on different XCDs: give each XCD a
    // contiguous range of rows, so the input row two neighbouring output
    // rows share is fetched into one L2
    int bid = static_cast<int>(blockIdx.x);
    const int nb = static_cast<int>(gridDim.x);
    if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
    const int row = bid / chunks;  // image * OH + oh
    const int t = (bid - row * chunks) * 256 + static_cast<int>(threadIdx.x);
    if (t >= OW * C16) return;
    const int img = row / OH;
    const int oh = row - img * OH;
    const int ow = t / C16;
    const int c16 = t - ow * C16;
    const int8_t *xi = x + static_cast<size_t>(img) * xHp * xWp * xCp + c16 * 16;
    char16 m = static_cast<char16>(static_cast<signed char>(-128));
    if constexpr (K > 0) {
        char16 v[K][K];
#pragma unroll
        for (int a = 0; a < K; a++)
#pragma unroll
            for (int b = 0; b < K; b++) {
                const int ih = oh * sh - ph + a, iw = ow * sw - pw + b;
                const bool in = static_cast<unsigned>(ih) < static_cast<unsigned>(H) &&
                                static_cast<unsigned>(iw) < static_cast<unsigned>(W);
                v[a][b] = in ? *reinterpret_cast<const char16 *>(
                                   xi + (static_cast<size_t>(ih + xpt) * xWp + iw + xpl) * xCp)
                             : m;
            }
#pragma unroll
        for (int a = 0; a < K; a++)
#pragma unroll
            for (int b = 0; b < K; b++) m = __builtin_elementwise_max(m, v[a][b]);
    } else {
        for (int a = 0; a < kh; a++) {
            const int ih = oh * sh - ph + a;
            if (ih < 0 || ih >= H) continue;
            for (int b = 0; b < kw; b++) {
                const int iw = ow * sw - pw + b;
                if (iw < 0 || iw >= W) continue;
                m = __builtin_elementwise_max(
                    m, *reinterpret_cast<const char16 *>(xi + (static_cast<size_t>(ih + xpt) * xWp + iw + xpl) * xCp));
            }
        }
    }
    *reinterpret_cast<char16 *>(y + ((static_cast<size_t>(img) * yHp + oh + ypt) * yWp + ow + ypl) * yCp + c16 * 16) = m;
}

// One wave per (image, 16 channels): lane l sums pixels l, l + 64, ... of
// the image, 16 channels at a time from one 16-byte load (the channel pitch
// is a multiple of 16), and the 64 lanes' sums are added through LDS.  The
// sums are integers, so any order gives the same total; lane c < 16 then
// subtracts the zero point's share and writes channel c.
__global__ void __launch_bounds__(64) plane_mean_q8(const int8_t *__restrict__ x, float *__restrict__ y, int C, int H,
                                                    int W, int Hp, int Wp, int Cp, int pt, int pl, float scale,
                                                    int zp) {
    typedef signed char char16 __attribute__((ext_vector_type(16)));
    __shared__ int part[64][17];
    const int groups = (C + 15) / 16;
    const int img = static_cast<int>(blockIdx.x) / groups;
    const int g = static_cast<int>(blockIdx.x) - img * groups;
    const int lane = threadIdx.x;
    const int HW = H * W;
    int sum[16];
#pragma unroll
    for (int b = 0; b < 16; b++) sum[b] = 0;
    // |sum| <= 128 * H * W: exact for H * W < 2^23
    for (int p = lane; p < HW; p += 64) {
        const int h = p / W, w = p - h * W;
        const char16 v = *reinterpret_cast<const char16 *>(
            x + ((static_cast<size_t>(img) * Hp + h + pt) * Wp + w + pl) * static_cast<size_t>(Cp) + g * 16);
#pragma unroll
        for (int b = 0; b < 16; b++) sum[b] += static_cast<int>(v[b]);
    }
#pragma unroll
    for (int b = 0; b < 16; b++) part[lane][b] = sum[b];
    __syncthreads();
    const int c = g * 16 + lane;
    if (lane < 16 && c < C) {
        int total = 0;
        for (int l = 0; l < 64; l++) total += part[l][lane];
        const int centered = total - zp * HW;  // sum(q - z)
        y[static_cast<size_t>(img) * C + c] =
            static_cast<float>((static_cast<double>(centered) * static_cast<double>(scale)) / static_cast<double>(HW));
    }
}

size_t align_to(size_t v, size_t a) { return (v + a - 1) / a * a; }

bool readable_by_builtin_q8(const Spkv2Context *ctx, const Spkv2NodeRecord *n, uint16_t slot) {
    switch (n->op_type) {
    case SPKV2_OP_CONV:
        return (slot == 0 || slot == 3) && n->input_count >= 2 &&
               ctx->tensor_records[n->inputs[1]].dtype == SPKV2_DTYPE_INT8;
    case SPKV2_OP_MAXPOOL:
    case SPKV2_OP_REDUCEMEAN:
    case SPKV2_OP_GLOBALAVGPOOL:
        return slot == 0;
    default:
        return false;
    }
}

}  // namespace

int q8_params(const Spkv2Context *ctx, uint32_t tid, float *scale, int *zp) {
    const Spkv2QuantParamRecord *q = spkv2_ctx_find_quant_param(ctx, tid);
    const float *s = q ? spkv2_ctx_quant_scales(ctx, q) : nullptr;
    const int32_t *z = q ? spkv2_ctx_quant_zero_points(ctx, q) : nullptr;
    if (!s || !z || q->num_channels < 1 || !(s[0] > 0.0f) || z[0] < -128 || z[0] > 127) return SPKV2_E_QUANT;
    *scale = s[0];
    *zp = z[0];
    return 0;
}

int setup_q8_tensors(Spkv2Context *ctx) {
    const uint32_t nt = ctx->header.num_tensors, nn = ctx->header.num_nodes;
    ctx->q8.assign(nt, Spkv2Q8Tensor{});
    ctx->q8_node.assign(nn, 0);
    ctx->has_q8 = false;
    for (uint32_t t = 0; t < nt; t++) {
        const Spkv2TensorRecord *r = &ctx->tensor_records[t];
        if (r->dtype != SPKV2_DTYPE_INT8 || r->role == SPKV2_ROLE_WEIGHT || r->role == SPKV2_ROLE_CONSTANT) continue;
        if (r->role != SPKV2_ROLE_ACTIVATION || r->rank != 4) {
            set_last_error_text("int8 tensor " + std::to_string(t) +
                                " is not a rank-4 activation (graph inputs and outputs stay fp32)");
            return SPKV2_E_UNSUPPORTED;
        }
        Spkv2Q8Tensor q;
        if (int rc = q8_params(ctx, t, &q.scale, &q.zp)) {
            set_last_error_text("int8 tensor " + std::to_string(t) + " has no per-tensor scale and zero point");
            return rc;
        }
        q.N = static_cast<int>(r->shape[0]);
        q.C = static_cast<int>(r->shape[1]);
        q.H = static_cast<int>(r->shape[2]);
        q.W = static_cast<int>(r->shape[3]);
        q.Cp = static_cast<int>(align_to(static_cast<size_t>(q.C), 16));
        // the halo: the widest padding of the convs reading it as their
        // input, and room for every such conv's receptive field
        for (uint32_t i = 0; i < nn; i++) {
            const Spkv2NodeRecord *n = &ctx->node_records[i];
            for (uint16_t k = 0; k < n->input_count; k++) {
                if (n->inputs[k] != t) continue;
                if (!readable_by_builtin_q8(ctx, n, k)) {
                    set_last_error_text("int8 tensor " + std::to_string(t) + " is read by node " + std::to_string(i) +
                                        ", which has no int8 kernel");
                    return SPKV2_E_UNSUPPORTED;
                }
                ctx->q8_node[i] = 1;
                if (n->op_type == SPKV2_OP_CONV && k == 0) {
                    ConvGeom g;
                    if (int rc = read_conv_geom(ctx, n, &g)) return rc;
                    q.pt = std::max(q.pt, g.ph);
                    q.pl = std::max(q.pl, g.pw);
                }
            }
            for (uint16_t k = 0; k < n->output_count; k++)
                if (n->outputs[k] == t) {
                    if (n->op_type != SPKV2_OP_CONV && n->op_type != SPKV2_OP_MAXPOOL) {
                        set_last_error_text("int8 tensor " + std::to_string(t) + " is written by node " +
                                            std::to_string(i) + ", which has no int8 kernel");
                        return SPKV2_E_UNSUPPORTED;
                    }
                    ctx->q8_node[i] = 1;
                }
        }
        q.Hp = q.pt + q.H;
        q.Wp = q.pl + q.W;
        for (uint32_t i = 0; i < nn; i++) {
            const Spkv2NodeRecord *n = &ctx->node_records[i];
            if (n->op_type != SPKV2_OP_CONV || n->input_count < 1 || n->inputs[0] != t) continue;
            ConvGeom g;
            if (int rc = read_conv_geom(ctx, n, &g)) return rc;
            q.Hp = std::max(q.Hp, q.pt - g.ph + (g.OH - 1) * g.sh + (g.KH - 1) * g.dh + 1);
            q.Wp = std::max(q.Wp, q.pl - g.pw + (g.OW - 1) * g.sw + (g.KW - 1) * g.dw + 1);
        }
        q.bytes = static_cast<size_t>(q.N) * q.Hp * q.Wp * q.Cp;
        if (q.bytes >= 0x7fff0000ULL) {
            set_last_error_text("int8 tensor " + std::to_string(t) + " exceeds the kernels' 31-bit byte offsets");
            return SPKV2_E_UNSUPPORTED;
        }
        if (int rc = hip_check(hipMalloc(reinterpret_cast<void **>(&q.buf), q.bytes), "hipMalloc int8 tensor")) return rc;
        // the zero point everywhere; producers write the interior each run
        if (int rc = hip_check(hipMemset(q.buf, q.zp & 0xff, q.bytes), "hipMemset int8 tensor")) {
            (void)hipFree(q.buf);
            return rc;
        }
        ctx->q8[t] = q;
        ctx->has_q8 = true;
    }
    if (ctx->has_q8)
        for (size_t i = 0; i < ctx->protection_count; i++)
            if (ctx->protection_records[i].tensor_id < nt && ctx->q8[ctx->protection_records[i].tensor_id].buf) {
                set_last_error_text("a protection plan entry names an int8 tensor (the guards read fp32 tensors)");
                return SPKV2_E_UNSUPPORTED;
            }
    return 0;
}

int check_q8_winners(const Spkv2Context *ctx) {
    if (!ctx->has_q8) return 0;
    for (uint32_t i = 0; i < ctx->header.num_nodes; i++)
        if (ctx->q8_node[i] && !builtin_runs(ctx, i)) {
            set_last_error_text("node " + std::to_string(i) +
                                " reads or writes an int8 tensor between nodes and must run on a built-in kernel");
            return SPKV2_E_UNSUPPORTED;
        }
    return 0;
}

int maxpool_q8_run(Spkv2Context *ctx, const Spkv2NodeRecord *node) {
    const Spkv2Q8Tensor *x = q8_tensor(ctx, node->inputs[0]);
    const Spkv2Q8Tensor *y = node->output_count ? q8_tensor(ctx, node->outputs[0]) : nullptr;
    if (!x || !y || x->N != y->N || x->C != y->C || x->zp != y->zp ||
        __builtin_bit_cast(uint32_t, x->scale) != __builtin_bit_cast(uint32_t, y->scale)) {
        set_last_error_text("int8 MaxPool needs int8 input and output with one scale and zero point");
        return SPKV2_E_UNSUPPORTED;
    }
    Spkv2AttrRecord attr;
    if (int rc = spkv2_ctx_get_attr(ctx, node, &attr)) return rc;
    set_kernel_name(ctx, node, "maxpool_q8");
    const int C16 = x->Cp / 16;
    const size_t rows = static_cast<size_t>(y->N) * y->H;
    const size_t per_row = static_cast<size_t>(y->W) * C16;  // 16-byte pieces of one output row
    if (rows == 0 || per_row == 0) return 0;
    const size_t chunks = (per_row + 255) / 256;
    if (per_row > 0x7fffffffULL || rows * chunks >= 0x80000000ULL) return SPKV2_E_UNSUPPORTED;
    const bool k3 = attr.kernel_shape[0] == 3 && attr.kernel_shape[1] == 3;
    hipLaunchKernelGGL(k3 ? maxpool_q8<3> : maxpool_q8<0>, dim3(static_cast<unsigned>(rows * chunks)), dim3(256), 0,
                       ctx->stream, x->buf, y->buf, static_cast<int>(chunks), C16, x->H, x->W, x->Hp, x->Wp, x->Cp,
                       x->pt, x->pl, y->H, y->W, y->Hp, y->Wp, y->Cp, y->pt, y->pl, attr.kernel_shape[0],
                       attr.kernel_shape[1], attr.strides[0], attr.strides[1], attr.pads[0], attr.pads[1]);
    return launch_status("maxpool_q8");
}

int mean_q8_run(Spkv2Context *ctx, const Spkv2NodeRecord *node) {
    const Spkv2Q8Tensor *x = q8_tensor(ctx, node->inputs[0]);
    const Spkv2TensorRecord *yr = rec(ctx, node->outputs[0]);
    if (!x || yr->dtype != SPKV2_DTYPE_FP32 || elem_count(yr) != static_cast<size_t>(x->N) * x->C) {
        set_last_error_text("int8 spatial mean needs an int8 input and an fp32 [N, C] output");
        return SPKV2_E_UNSUPPORTED;
    }
    if (static_cast<int64_t>(x->H) * x->W >= (int64_t(1) << 23)) return SPKV2_E_UNSUPPORTED;
    set_kernel_name(ctx, node, "plane_mean_q8");
    const size_t waves = static_cast<size_t>(x->N) * ((x->C + 15) / 16);  // one per (image, 16 channels)
    if (waves == 0) return 0;
    if (waves >= 0x80000000ULL) return SPKV2_E_UNSUPPORTED;
    hipLaunchKernelGGL(plane_mean_q8, dim3(static_cast<unsigned>(waves)), dim3(64), 0, ctx->stream, x->buf,
                       dptr<float>(ctx, node->outputs[0]), x->C, x->H, x->W, x->Hp, x->Wp, x->Cp, x->pt, x->pl,
                       x->scale, x->zp);
    return launch_status("plane_mean_q8");
}

}  // namespace spk::kern

// Test hook: an int8 activation tensor's interior, NCHW, to host memory.
extern "C" int spkv2_mi355x_read_int8_tensor(Spkv2Context *ctx, uint32_t tensor_id, int8_t *out, size_t size) {
    if (!ctx || !out || tensor_id >= ctx->header.num_tensors) return -1;
    if (!ctx->prepared) return SPKV2_E_NO_DEVICE;
    const Spkv2Q8Tensor *q = spk::q8_tensor(ctx, tensor_id);
    if (!q) return -1;
    if (size != static_cast<size_t>(q->N) * q->C * q->H * q->W) return -2;
    if (int rc = spk::hip_check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize")) return rc;
    std::vector<int8_t> host(q->bytes);
    if (int rc = spk::hip_check(hipMemcpy(host.data(), q->buf, q->bytes, hipMemcpyDeviceToHost), "hipMemcpy")) return rc;
    for (int n = 0; n < q->N; n++)
        for (int c = 0; c < q->C; c++)
            for (int h = 0; h < q->H; h++)
                for (int w = 0; w < q->W; w++)
                    out[((static_cast<size_t>(n) * q->C + c) * q->H + h) * q->W + w] =
                        host[((static_cast<size_t>(n) * q->Hp + h + q->pt) * q->Wp + w + q->pl) * q->Cp + c];
    return 0;
}
