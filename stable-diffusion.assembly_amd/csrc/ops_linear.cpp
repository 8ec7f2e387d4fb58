// MUL_MAT and MUL_MAT with the gated GELU after it (mul_mat.cc), on the
// device: the predicates of mul_mat_supported (mul_mat.cc:181-194) and
// mul_mat_gated_supported (mul_mat.cc:1128-1151), then the split-FP16 MFMA
// product (gemm.hip) or, with bits, the quantized one (quant.hip).

#include <hip/hip_runtime.h>

#include "host.h"
#include "kernels.h"
#include "quant.h"

namespace sdhip {

namespace {

bool overlaps(const void *a, size_t an, const void *b, size_t bn) { return spans_overlap(a, an, b, bn); }

size_t nbytes(const sdhip_tensor *t) { return tensor_span(t); }

MulMatArgs args_of(const sdhip_tensor *w, const sdhip_tensor *x, const sdhip_tensor *y) {
    MulMatArgs a{};
    a.x = static_cast<const float *>(x->data);
    a.ldx = x->nb[1] / 4;
    if (w->type == SDHIP_TYPE_F32) {
        a.w32 = static_cast<const float *>(w->data);
        a.ldw32 = w->nb[1] / 4;
    } else {
        a.w = static_cast<const _Float16 *>(w->data);
        a.ldw = w->nb[1] / 2;
    }
    a.K = w->ne[0];
    a.N = w->ne[1];
    a.M = x->ne[1] * x->ne[2] * x->ne[3];
    a.ne1 = y->ne[1];
    a.ne2 = y->ne[2];
    a.ldy = y->nb[1] / 4;
    // The products of 16 bits: FP16 weights by x rounded to FP16
    // (split_form's first parts alone, cpu.cc:336-366), or with
    // half_format=1 both rounded to bfloat16 (cpu.cc:319-321, the first parts
    // of sdasm_amx_pack_rows and _f16); 0 and 2 take FP16, the form that
    // fits here.
    a.half16 = tuning().bits == 16 && w->type == SDHIP_TYPE_F16 ? (tuning().half_format == 1 ? 2 : 1) : 0;
    return a;
}

}  // namespace

// Whether the product is quantized (mul_mat.cc:95-105): bits asks for the
// linear layers, and the product is of 256 rows or more.
bool mul_mat_quantized(const sdhip_tensor *x) {
    const Tuning &t = tuning();
    const int64_t m = x->ne[1] * x->ne[2] * x->ne[3];
    return t.bits >= 2 && t.bits <= 8 && (t.quantize & 1) != 0 && m >= 256;
}

}  // namespace sdhip

using namespace sdhip;

extern "C" {

int sdhip_mul_mat_supported(const sdhip_tensor *w, const sdhip_tensor *x, const sdhip_tensor *y) {
    if (w == nullptr || x == nullptr || y == nullptr) return 0;
    // The weights are one matrix of FP16 or single precision, the other
    // operand and the result contiguous single precision, the products large
    // enough to pay for the launch (mul_mat.cc:181-194).
    const bool weights = (holds_f16(w) || holds_f32(w)) && w->ne[2] == 1 && w->ne[3] == 1 &&
                         w->nb[1] % w->nb[0] == 0 && w->nb[1] >= w->nb[0] * w->ne[0];
    const bool shapes = x->ne[0] == w->ne[0] && y->ne[0] == w->ne[1] && y->ne[1] == x->ne[1] &&
                        y->ne[2] == x->ne[2] && y->ne[3] == x->ne[3];
    return weights && shapes && holds_f32(x) && contiguous(x) && holds_f32(y) && contiguous(y) &&
           x->ne[1] * x->ne[2] * x->ne[3] >= 16 && w->ne[0] >= 16;
}

size_t sdhip_mul_mat_work_size(const sdhip_tensor *w, const sdhip_tensor *x, const sdhip_tensor *y) {
    if (!sdhip_mul_mat_supported(w, x, y)) return 0;
    if (mul_mat_quantized(x)) {
        return quantized_linear_work_size(w->ne[0], w->ne[1], x->ne[1] * x->ne[2] * x->ne[3]);
    }
    const MulMatArgs a = args_of(w, x, y);
    // Single-precision weights: split into two FP16 planes at every call.
    if (a.w32 != nullptr) return split_weights_bytes(a.N, a.K);
    return mul_mat_split_taken(a) ? mul_mat_split_work_size(a) : 0;
}

namespace sdhip {

// Single-precision weights split into the work buffer (split_weights), and
// the product's description pointed at the planes.
sdhip_status split_into(MulMatArgs &a, void *work, size_t work_size, hipStream_t st, const char *what) {
    const size_t need = split_weights_bytes(a.N, a.K);
    if (const sdhip_status ws = check_work(what, work, work_size, need); ws != SDHIP_OK) return ws;
    const sdhip_status s = launched(launch_split_weights(a.w32, a.ldw32, a.N, a.K, work, st), "split weights");
    if (s != SDHIP_OK) return s;
    a.w = split_weights_hi(work);
    a.ldw = split_weights_ld(a.K);
    a.w_plane = a.N * a.ldw;
    a.w_scale = split_weights_scale(work, a.N, a.K);
    return SDHIP_OK;
}

}  // namespace sdhip

sdhip_status sdhip_mul_mat(const sdhip_tensor *w, const sdhip_tensor *x, const sdhip_tensor *y,
                           const sdhip_epilogue *chain, void *work, size_t work_size, void *stream) {
    if (!sdhip_mul_mat_supported(w, x, y)) {
        return fail(SDHIP_UNSUPPORTED, "mul_mat: operands not taken");
    }
    MulMatArgs a = args_of(w, x, y);
    ChainRun run;
    sdhip_status s = chain_plan(y, chain, run);
    if (s != SDHIP_OK) return s;
    a.chain = run.fused;
    a.y = run.out;
    a.from_redirect = run.from_redirect;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (mul_mat_quantized(x)) {
        const size_t need = quantized_linear_work_size(a.K, a.N, a.M);
        if (const sdhip_status ws = check_work("mul_mat", work, work_size, need); ws != SDHIP_OK) return ws;
        s = quantized_linear(a, false, work, st);
    } else if (a.w32 != nullptr) {
        s = split_into(a, work, work_size, st, "mul_mat");
        if (s == SDHIP_OK) s = launched(launch_mul_mat(a, gemm_shape(), st), "mul_mat");
    } else if (mul_mat_panels_taken(a, tuning().mul_mat_panels)) {
        s = launched(launch_mul_mat_panels(a, tuning().mul_mat_panels, st), "mul_mat");
    } else if (mul_mat_split_taken(a)) {
        const size_t need = mul_mat_split_work_size(a);
        if (const sdhip_status ws = check_work("mul_mat", work, work_size, need); ws != SDHIP_OK) return ws;
        s = launched(launch_mul_mat_split(a, work, gemm_shape(), tuning().mul_mat_panels != 0, st), "mul_mat split along K");
    } else {
        s = launched(launch_mul_mat(a, gemm_shape(), st), "mul_mat");
    }
    return s == SDHIP_OK ? chain_after(run, st) : s;
}

int sdhip_mul_mat_gated_supported(const sdhip_tensor *w, const sdhip_tensor *x, const sdhip_tensor *y,
                                  const sdhip_tensor *out) {
    if (!sdhip_mul_mat_supported(w, x, y) || out == nullptr || y->ne[0] % 2 != 0) return 0;
    const int64_t half = y->ne[0] / 2;
    // Quantized, each half's columns begin a panel (mul_mat.cc:1129-1132).
    if (mul_mat_quantized(x) && half % 16 != 0) return 0;
    // What the result is written to is not what the product reads
    // (mul_mat.cc:1133-1149).
    const size_t on = nbytes(out);
    if (overlaps(out->data, on, w->data, nbytes(w)) || overlaps(out->data, on, x->data, nbytes(x)) ||
        overlaps(out->data, on, y->data, nbytes(y))) {
        return 0;
    }
    return holds_f32(out) && contiguous(out) && out->ne[0] == half && out->ne[1] == y->ne[1] &&
           out->ne[2] == y->ne[2] && out->ne[3] == y->ne[3];
}

sdhip_status sdhip_mul_mat_gated(const sdhip_tensor *w, const sdhip_tensor *x, const sdhip_tensor *y,
                                 const sdhip_epilogue *chain, const sdhip_tensor *out, void *work, size_t work_size,
                                 void *stream) {
    if (!sdhip_mul_mat_gated_supported(w, x, y, out)) {
        return fail(SDHIP_UNSUPPORTED, "mul_mat_gated: operands not taken");
    }
    if (chain != nullptr && chain->redirect != nullptr) {
        return fail(SDHIP_UNSUPPORTED, "mul_mat_gated: a chain with a residual redirect is not gated");
    }
    if (tuning().fuse == 0) {
        // The gated GELU apart, as ggml's nodes compute it when nothing is
        // fused: the product and its chain into y, then out from y's halves.
        sdhip_status s = sdhip_mul_mat(w, x, y, chain, work, work_size, stream);
        if (s != SDHIP_OK) return s;
        return gated_after(static_cast<const float *>(y->data), static_cast<float *>(out->data),
                           x->ne[1] * x->ne[2] * x->ne[3], y->ne[0] / 2, y->nb[1] / 4, out->nb[1] / 4,
                           static_cast<hipStream_t>(stream));
    }
    MulMatArgs a = args_of(w, x, y);
    sdhip_status s = device_chain(chain, y->ne, a.chain);
    if (s != SDHIP_OK) return s;
    const size_t on = nbytes(out);
    for (int i = 0; chain != nullptr && i < chain->count; ++i) {
        const sdhip_tensor &op = chain->steps[i].operand;
        if (chain->steps[i].kind != SDHIP_STEP_SILU && overlaps(out->data, on, op.data, nbytes(&op))) {
            return fail(SDHIP_UNSUPPORTED, "mul_mat_gated: the output overlaps a chain operand");
        }
    }
    a.y = static_cast<float *>(out->data);
    a.ldy = out->nb[1] / 4;
    a.half = y->ne[0] / 2;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (mul_mat_quantized(x)) {
        const size_t need = quantized_linear_work_size(a.K, a.N, a.M);
        if (const sdhip_status ws = check_work("mul_mat_gated", work, work_size, need); ws != SDHIP_OK) return ws;
        return quantized_linear(a, true, work, st);
    }
    if (a.w32 != nullptr) {
        const sdhip_status s = split_into(a, work, work_size, st, "mul_mat_gated");
        if (s != SDHIP_OK) return s;
    }
    return launched(launch_mul_mat_gated(a, gemm_shape(), st), "mul_mat_gated");
}

}  // extern "C"
