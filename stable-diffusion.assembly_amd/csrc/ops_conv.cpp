// CONV_2D on the device: the predicates of conv2d_supported
// (conv2d.cc:320-331) and winograd_supported (winograd.cc:2107-2123), the
// choice between F(4x4, 3x3), F(2x2, 3x3) and the direct convolution that
// hooks.cc:36-41 and winograd.cc:1204-1206, 194-196 make, and the launch.

#include <hip/hip_runtime.h>

#include "host.h"
#include "kernels.h"
#include "quant.h"
#include "winograd.h"

namespace sdhip {

namespace {

struct Geometry {
    int64_t iw, ih, ic, n, kw, kh, oc, ow, oh;
    int32_t s0, s1, p0, p1, d0, d1;
};

Geometry geometry(const sdhip_tensor *kernel, const sdhip_tensor *input, const sdhip_tensor *y,
                  const int32_t *op) {
    Geometry g{};
    g.iw = input->ne[0];
    g.ih = input->ne[1];
    g.ic = input->ne[2];
    g.n = input->ne[3];
    g.kw = kernel->ne[0];
    g.kh = kernel->ne[1];
    g.oc = kernel->ne[3];
    g.ow = y->ne[0];
    g.oh = y->ne[1];
    g.s0 = op[0];
    g.s1 = op[1];
    g.p0 = op[2];
    g.p1 = op[3];
    g.d0 = op[4];
    g.d1 = op[5];
    return g;
}

// The output extent of a convolution along one dimension (ggml_calc_conv_output_size).
int64_t out_size(int64_t in, int64_t k, int32_t s, int32_t p, int32_t d) {
    return (in + 2 * p - d * (k - 1) - 1) / s + 1;
}

// Whether bits asks for the convolutions' products quantized (quantized(
// Quantized_op::convolution), quant.cc:53-56): then the convolutions Winograd
// takes are F(2x2) with quantized products (winograd.cc:2230-2244) and the
// others direct ones with quantized products (conv2d.cc:338-483).
bool conv_quantized() {
    const Tuning &t = tuning();
    return t.bits >= 2 && t.bits <= 8 && (t.quantize & 2) != 0;
}

bool direct_supported(const sdhip_tensor *kernel, const sdhip_tensor *input, const sdhip_tensor *y, const int32_t *op) {
    if (kernel == nullptr || input == nullptr || y == nullptr || op == nullptr) return false;
    // FP16 or single-precision kernels (conv2d.cc:320-331).
    const bool weights = (holds_f16(kernel) || holds_f32(kernel)) && contiguous(kernel);
    if (!(weights && holds_f32(input) && holds_f32(y) && contiguous(y) && kernel->ne[2] == input->ne[2] &&
          op[0] > 0 && op[1] > 0 && op[4] > 0 && op[5] > 0 && op[2] >= 0 && op[3] >= 0)) {
        return false;
    }
    return y->ne[0] == out_size(input->ne[0], kernel->ne[0], op[0], op[2], op[4]) &&
           y->ne[1] == out_size(input->ne[1], kernel->ne[1], op[1], op[3], op[5]) && y->ne[2] == kernel->ne[3] &&
           y->ne[3] == input->ne[3] && input->nb[1] % 4 == 0 && input->nb[2] % 4 == 0 && input->nb[3] % 4 == 0;
}

// Small images: every tile of every image in one block (winograd.cc:194-196).
bool small(const Geometry &g) {
    return g.n * ((g.ow + 1) / 2) * ((g.oh + 1) / 2) <= tuning().winograd_small_tiles;
}

bool winograd_taken(const sdhip_tensor *kernel, const sdhip_tensor *input, const sdhip_tensor *y, const int32_t *op) {
    if (tuning().winograd == 0 || !direct_supported(kernel, input, y, op)) return false;
    const Geometry g = geometry(kernel, input, y, op);
    if (!(g.kw == 3 && g.kh == 3 && g.s0 == 1 && g.s1 == 1 && g.d0 == 1 && g.d1 == 1 && g.p0 <= 2 && g.p1 <= 2)) {
        return false;
    }
    return g.ow * g.oh >= tuning().winograd_positions || small(g);
}

// F(4x4, 3x3) for FP16 kernels and images of winograd4_positions outputs and
// more (winograd.cc:1204-1206); single-precision kernels take F(2x2).
bool four(const Geometry &g, const sdhip_tensor *kernel) {
    return tuning().winograd == 2 && kernel->type == SDHIP_TYPE_F16 && g.ow * g.oh >= tuning().winograd4_positions;
}

int path_of(const sdhip_tensor *kernel, const sdhip_tensor *input, const sdhip_tensor *y, const int32_t *op) {
    if (!direct_supported(kernel, input, y, op)) return -1;
    if (winograd_taken(kernel, input, y, op)) {
        // The bits mode's Winograd is F(2x2) (winograd.cc:2236-2244 before four()).
        return !conv_quantized() && four(geometry(kernel, input, y, op), kernel) ? 4 : 2;
    }
    return 0;
}

ConvArgs conv_args(const sdhip_tensor *kernel, const sdhip_tensor *input, const sdhip_tensor *y,
                   const int32_t *op) {
    ConvArgs c{};
    c.x = static_cast<const float *>(input->data);
    c.xnb1 = input->nb[1] / 4;
    c.xnb2 = input->nb[2] / 4;
    c.xnb3 = input->nb[3] / 4;
    c.iw = input->ne[0];
    c.ih = input->ne[1];
    c.ic = input->ne[2];
    c.n = input->ne[3];
    c.w = kernel->type == SDHIP_TYPE_F16 ? static_cast<const _Float16 *>(kernel->data) : nullptr;
    c.w32 = kernel->type == SDHIP_TYPE_F32 ? static_cast<const float *>(kernel->data) : nullptr;
    c.kw = kernel->ne[0];
    c.kh = kernel->ne[1];
    c.oc = kernel->ne[3];
    c.y = static_cast<float *>(y->data);
    c.ynb1 = y->nb[1] / 4;
    c.ynb2 = y->nb[2] / 4;
    c.ynb3 = y->nb[3] / 4;
    c.ow = y->ne[0];
    c.oh = y->ne[1];
    c.s0 = op[0];
    c.s1 = op[1];
    c.p0 = op[2];
    c.p1 = op[3];
    c.d0 = op[4];
    c.d1 = op[5];
    c.K = c.ic * c.kh * c.kw;
    c.ldw = c.K;
    // The products of 16 bits: FP16 kernels by the columns rounded to FP16
    // (cpu.cc:336-366; Winograd's products stay single precision there), or
    // with half_format=1 both rounded to bfloat16 (cpu.cc:319-321).
    c.half16 = tuning().bits == 16 && kernel->type == SDHIP_TYPE_F16 ? (tuning().half_format == 1 ? 2 : 1) : 0;
    c.taps = c.kh * c.kw;
    c.plane = c.oh * c.ow;
    c.P = c.n * c.plane;
    return c;
}

// A convolution of single-precision kernels, which the call splits into two
// FP16 planes of rows 32-aligned (split_weights) before the products.
void mark_split(ConvArgs &c) {
    c.w_split = 1;
    c.ldw = split_weights_ld(c.K);
}

WinogradArgs winograd_args(const sdhip_tensor *kernel, const sdhip_tensor *input, const sdhip_tensor *y,
                           const int32_t *op, int m) {
    WinogradArgs a{};
    a.m = m;
    a.x = static_cast<const float *>(input->data);
    a.xnb1 = input->nb[1] / 4;
    a.xnb2 = input->nb[2] / 4;
    a.xnb3 = input->nb[3] / 4;
    a.iw = input->ne[0];
    a.ih = input->ne[1];
    a.ic = input->ne[2];
    a.n = input->ne[3];
    a.w = kernel->type == SDHIP_TYPE_F16 ? static_cast<const _Float16 *>(kernel->data) : nullptr;
    a.w32 = kernel->type == SDHIP_TYPE_F32 ? static_cast<const float *>(kernel->data) : nullptr;
    a.oc = kernel->ne[3];
    a.ow = y->ne[0];
    a.oh = y->ne[1];
    a.ynb1 = y->nb[1] / 4;
    a.ynb2 = y->nb[2] / 4;
    a.ynb3 = y->nb[3] / 4;
    a.p0 = op[2];
    a.p1 = op[3];
    a.tw = ceil_div(a.ow, m);
    a.th = ceil_div(a.oh, m);
    a.tiles = a.n * a.tw * a.th;
    return a;
}

}  // namespace

}  // namespace sdhip

using namespace sdhip;

extern "C" {

int sdhip_conv2d_supported(const sdhip_tensor *kernel, const sdhip_tensor *input, const sdhip_tensor *y,
                           const int32_t op_params[6]) {
    return direct_supported(kernel, input, y, op_params) ? 1 : 0;
}

int sdhip_conv2d_path(const sdhip_tensor *kernel, const sdhip_tensor *input, const sdhip_tensor *y,
                      const int32_t op_params[6]) {
    return path_of(kernel, input, y, op_params);
}

size_t sdhip_conv2d_work_size(const sdhip_tensor *kernel, const sdhip_tensor *input, const sdhip_tensor *y,
                              const int32_t op_params[6]) {
    const int path = path_of(kernel, input, y, op_params);
    if (path >= 0 && conv_quantized()) {
        return quantized_conv_work_size(conv_args(kernel, input, y, op_params), path == 2);
    }
    if (path == 2 || path == 4) {
        return winograd_work_size(winograd_args(kernel, input, y, op_params, path));
    }
    if (path == 0) {
        ConvArgs c = conv_args(kernel, input, y, op_params);
        // Single-precision kernels: split into two FP16 planes at every call,
        // after the columns' work (the split's rows are 32-aligned).
        const size_t split = kernel->type == SDHIP_TYPE_F32 ? split_weights_bytes(c.oc, c.K) : 0;
        if (split > 0) mark_split(c);
        return (conv_columns_taken(c) ? round_up(conv_columns_work_size(c), 256) : 0) + split;
    }
    return 0;
}

sdhip_status sdhip_conv2d(const sdhip_tensor *kernel, const sdhip_tensor *input, const sdhip_tensor *y,
                          const int32_t op_params[6], const sdhip_epilogue *chain, void *work, size_t work_size,
                          void *stream) {
    const int path = path_of(kernel, input, y, op_params);
    if (path < 0) {
        return fail(SDHIP_UNSUPPORTED, "conv2d: operands not taken");
    }
    ChainRun run;
    sdhip_status s = chain_plan(y, chain, run);
    if (s != SDHIP_OK) return s;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (conv_quantized()) {
        ConvArgs c = conv_args(kernel, input, y, op_params);
        c.y = run.out;
        c.from_redirect = run.from_redirect;
        c.chain = run.fused;
        const size_t need = quantized_conv_work_size(c, path == 2);
        if (const sdhip_status ws = check_work("conv2d", work, work_size, need); ws != SDHIP_OK) return ws;
        s = quantized_conv(c, path == 2, work, st);
        return s == SDHIP_OK ? chain_after(run, st) : s;
    }
    if (path == 2 || path == 4) {
        WinogradArgs a = winograd_args(kernel, input, y, op_params, path);
        a.y = run.out;
        a.from_redirect = run.from_redirect;
        a.chain = run.fused;
        const size_t need = winograd_work_size(a);
        if (const sdhip_status ws = check_work("conv2d", work, work_size, need); ws != SDHIP_OK) return ws;
        s = winograd(a, work, st);
        return s == SDHIP_OK ? chain_after(run, st) : s;
    }
    ConvArgs c = conv_args(kernel, input, y, op_params);
    c.y = run.out;
    c.from_redirect = run.from_redirect;
    c.chain = run.fused;
    if (kernel->type == SDHIP_TYPE_F32) {
        mark_split(c);
        const size_t cols = conv_columns_taken(c) ? round_up(conv_columns_work_size(c), 256) : 0;
        const size_t need = cols + split_weights_bytes(c.oc, c.K);
        if (const sdhip_status ws = check_work("conv2d", work, work_size, need); ws != SDHIP_OK) return ws;
        void *split = static_cast<char *>(work) + cols;
        s = launched(launch_split_weights(static_cast<const float *>(kernel->data), c.K, c.oc, c.K, split, st),
                     "conv2d split kernels");
        if (s != SDHIP_OK) return s;
        c.w = split_weights_hi(split);
        c.w_scale = split_weights_scale(split, c.oc, c.K);
        c.w_plane = c.oc * c.ldw;
    }
    if (conv_columns_taken(c)) {
        const size_t need = conv_columns_work_size(c);
        if (const sdhip_status ws = check_work("conv2d", work, work_size, need); ws != SDHIP_OK) return ws;
        s = launched(launch_conv_columns(c, work, gemm_shape(), st), "conv2d by columns");
    } else if (conv_panels_taken(c, tuning().conv_panels != 0)) {
        s = launched(launch_conv_panels(c, st), "conv2d by panels");
    } else {
        s = launched(launch_conv_direct(c, gemm_shape(), st), "conv2d direct");
    }
    return s == SDHIP_OK ? chain_after(run, st) : s;
}

}  // extern "C"
