// GROUP_NORM and NORM on the device: the predicates of group_norm_supported
// (norm.cc:93-98) and norm_supported (norm.cc:142-146), and the launch.

#include <hip/hip_runtime.h>

#include "host.h"
#include "norm.h"

using namespace sdhip;

extern "C" {

int sdhip_group_norm_supported(const sdhip_tensor *x, const sdhip_tensor *y, int groups) {
    if (x == nullptr || y == nullptr) return 0;
    if (!(holds_f32(x) && holds_f32(y) && contiguous(x) && contiguous(y) && same_shape(x, y) && groups > 0)) return 0;
    // Empty tensors are the caller's (nothing to compute; the split of the
    // groups into slices takes at least one image and number).
    if (nelements(x) <= 0) return 0;
    // A group's numbers are indexed in 32 bits.
    return ceil_div(x->ne[2], groups) * x->ne[0] * x->ne[1] < (int64_t(1) << 31);
}

size_t sdhip_group_norm_work_size(const sdhip_tensor *x, const sdhip_tensor *y, int groups) {
    if (!sdhip_group_norm_supported(x, y, groups)) return 0;
    return group_norm_shape(x->ne[0], x->ne[1], x->ne[2], x->ne[3], groups).work;
}

sdhip_status sdhip_group_norm(const sdhip_tensor *x, const sdhip_tensor *y, int groups, float eps,
                              const sdhip_epilogue *chain, void *work, size_t work_size, void *stream) {
    if (!sdhip_group_norm_supported(x, y, groups)) {
        return fail(SDHIP_UNSUPPORTED, "group_norm: operands not taken");
    }
    if (chain != nullptr && chain->redirect != nullptr) {
        return fail(SDHIP_UNSUPPORTED, "group_norm: no residual redirect after a normalisation");
    }
    GroupNormArgs a{};
    ChainRun run;
    sdhip_status s = chain_plan(y, chain, run);
    if (s != SDHIP_OK) return s;
    a.chain = run.fused;
    a.x = static_cast<const float *>(x->data);
    a.y = static_cast<float *>(y->data);
    a.ne0 = x->ne[0];
    a.ne1 = x->ne[1];
    a.ne2 = x->ne[2];
    a.ne3 = x->ne[3];
    a.xnb2 = x->nb[2] / 4;
    a.xnb3 = x->nb[3] / 4;
    a.ynb2 = y->nb[2] / 4;
    a.ynb3 = y->nb[3] / 4;
    a.groups = groups;
    a.per_group = ceil_div(a.ne2, groups);
    a.eps = eps;
    const GroupNormShape shape = group_norm_shape(a.ne0, a.ne1, a.ne2, a.ne3, groups);
    if (const sdhip_status ws = check_work("group_norm", work, work_size, shape.work); ws != SDHIP_OK) return ws;
    a.chunk = shape.chunk;
    a.slices = shape.slices;
    a.partials = static_cast<double *>(work);
    s = launched(launch_group_norm(a, static_cast<hipStream_t>(stream)), "group_norm");
    return s == SDHIP_OK ? chain_after(run, static_cast<hipStream_t>(stream)) : s;
}

sdhip_status sdhip_group_norm_static(const sdhip_tensor *x, const sdhip_tensor *y, int groups, float eps,
                                     const sdhip_epilogue *chain, void *stream) {
    if (!sdhip_group_norm_supported(x, y, groups)) {
        return fail(SDHIP_UNSUPPORTED, "group_norm_static: operands not taken");
    }
    const GroupNormShape shape = group_norm_shape(x->ne[0], x->ne[1], x->ne[2], x->ne[3], groups);
    if (shape.work > kStaticScratchBytes) {
        return fail(SDHIP_ERROR, "group_norm_static: %zu bytes of partial sums, the static scratch holds %zu",
                    shape.work, kStaticScratchBytes);
    }
    int device = -1;
    if (hipGetDevice(&device) != hipSuccess) return fail(SDHIP_ERROR, "group_norm_static: no current device");
    double *ptr = nullptr;
    const sdhip_status s = static_scratch(device, ptr);
    if (s != SDHIP_OK) return s;
    return sdhip_group_norm(x, y, groups, eps, chain, ptr, kStaticScratchBytes, stream);
}

int sdhip_norm_supported(const sdhip_tensor *x, const sdhip_tensor *y) {
    if (x == nullptr || y == nullptr) return 0;
    return holds_f32(x) && holds_f32(y) && same_shape(x, y) && x->nb[1] % 4 == 0 && x->nb[2] % 4 == 0 &&
           x->nb[3] % 4 == 0 && y->nb[1] % 4 == 0 && y->nb[2] % 4 == 0 && y->nb[3] % 4 == 0;
}

sdhip_status sdhip_norm(const sdhip_tensor *x, const sdhip_tensor *y, float eps, const sdhip_epilogue *chain,
                        void *stream) {
    if (!sdhip_norm_supported(x, y)) {
        return fail(SDHIP_UNSUPPORTED, "norm: operands not taken");
    }
    if (chain != nullptr && chain->redirect != nullptr) {
        return fail(SDHIP_UNSUPPORTED, "norm: no residual redirect after a normalisation");
    }
    NormArgs a{};
    ChainRun run;
    sdhip_status s = chain_plan(y, chain, run);
    if (s != SDHIP_OK) return s;
    a.chain = run.fused;
    a.x = static_cast<const float *>(x->data);
    a.y = static_cast<float *>(y->data);
    a.ne0 = x->ne[0];
    a.ne1 = x->ne[1];
    a.ne2 = x->ne[2];
    a.rows = x->ne[1] * x->ne[2] * x->ne[3];
    a.xnb1 = x->nb[1] / 4;
    a.xnb2 = x->nb[2] / 4;
    a.xnb3 = x->nb[3] / 4;
    a.ynb1 = y->nb[1] / 4;
    a.ynb2 = y->nb[2] / 4;
    a.ynb3 = y->nb[3] / 4;
    a.eps = eps;
    s = launched(launch_norm(a, static_cast<hipStream_t>(stream)), "norm");
    return s == SDHIP_OK ? chain_after(run, static_cast<hipStream_t>(stream)) : s;
}

}  // extern "C"
