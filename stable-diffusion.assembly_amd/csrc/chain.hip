// The chain computed apart from its operation (Tuning::fuse = 0, or
// fuse_residual = 0 for the residual connection that ends it): the operation
// writes its own output, and one pass over it applies the steps in the order
// of the graph and writes where the chain's last node writes -- what ggml's
// own ADD, MUL and UNARY nodes compute one after another when the reference
// does not fuse them (hooks.cc:113-131).  Also the gated GELU apart, out =
// x GELU(gate) of the halves of a product already written.

#include "device.h"
#include "host.h"
#include "profile.h"

namespace sdhip {

namespace {

// Element i of a contiguous output of extents ne, its steps' operands at
// sum(ik nb[k]); the values into out (the output itself, or the redirect).
__global__ __launch_bounds__(256) void chain_apart_kernel(const float *in, float *out, int64_t n,
                                                          uint32_t ne0, uint32_t ne1, uint32_t ne2, DevChain c) {
    for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256) {
        const uint32_t row = static_cast<uint32_t>(i / ne0);
        const uint32_t i0 = static_cast<uint32_t>(i - static_cast<int64_t>(row) * ne0);
        uint32_t i1, i2, i3;
        split_index(row, ne1, ne2, i1, i2, i3);
        float v[1] = {in[i]};
        apply_chain_block(c, v, [&](int s, int) {
            const DevStep &st = c.steps[s];
            return i0 * st.nb[0] + i1 * st.nb[1] + i2 * st.nb[2] + i3 * st.nb[3];
        });
        out[i] = v[0];
    }
}

// out[m][j] = p[m][j] GELU(p[m][half + j]) (fusion.cc:290-310), p rows of 2 half.
__global__ __launch_bounds__(256) void gated_apart_kernel(const float *__restrict__ p, float *__restrict__ out,
                                                          int64_t rows, int64_t half, int64_t ldp, int64_t ldo) {
    const int64_t n = rows * half;
    for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t m = i / half;
        const int64_t j = i - m * half;
        out[m * ldo + j] = p[m * ldp + j] * gelu(p[m * ldp + half + j]);
    }
}

int grid_of(int64_t n) {
    const int64_t blocks = (n + 255) / 256;
    return static_cast<int>(blocks < 8192 ? (blocks > 0 ? blocks : 1) : 8192);
}

}  // namespace

sdhip_status chain_plan(const sdhip_tensor *y, const sdhip_epilogue *e, ChainRun &r) {
    r = ChainRun{};
    for (int k = 0; k < 4; ++k) r.ne[k] = y->ne[k];
    const Tuning &t = tuning();
    const bool has_redirect = e != nullptr && e->redirect != nullptr;
    const bool apart_all = e != nullptr && (e->count > 0 || has_redirect) && t.fuse == 0;
    const bool apart_residual = has_redirect && !apart_all && t.fuse_residual == 0;
    if (!apart_all && !apart_residual) {
        sdhip_status s = device_chain(e, y->ne, r.fused);
        if (s != SDHIP_OK) return s;
        return output_of(y, e, r.out, r.from_redirect);
    }
    // Checked as the fused form would be: the same chains are taken.
    DevChain all;
    sdhip_status s = device_chain(e, y->ne, all);
    if (s != SDHIP_OK) return s;
    float *target = nullptr;
    int32_t from = 0;
    s = output_of(y, e, target, from);
    if (s != SDHIP_OK) return s;
    if (!contiguous(y)) {
        return fail(SDHIP_ERROR, "a chain apart needs a contiguous output");
    }
    r.out = static_cast<float *>(y->data);
    r.from_redirect = 0;
    r.apart = true;
    r.apart_in = r.out;
    r.apart_out = target;
    // The steps the operation applies itself, and those of the pass after.
    int fused = 0;
    if (apart_residual && !from) {
        fused = all.count - 1;  // all but the residual's addition, the last step
        if (fused < 0 || all.steps[all.count - 1].kind != kAdd) {
            return fail(SDHIP_ERROR, "a redirect whose chain does not end in the residual's addition");
        }
    } else if (apart_residual) {
        fused = all.count;
    }
    r.fused = DevChain{};
    for (int i = 0; i < fused; ++i) r.fused.steps[i] = all.steps[i];
    r.fused.count = fused;
    r.after = DevChain{};
    int n = 0;
    for (int i = fused; i < all.count; ++i) r.after.steps[n++] = all.steps[i];
    if (from) {
        // The sum in the residual's memory: the residual added last, as the
        // graph's ADD node adds it.
        if (n >= kMaxSteps) return fail(SDHIP_ERROR, "chain too long to add the residual apart");
        DevStep &add = r.after.steps[n++];
        add = DevStep{};
        add.kind = kAdd;
        add.operand = target;
        add.nb[0] = 1;
        add.nb[1] = y->ne[0];
        add.nb[2] = y->ne[0] * y->ne[1];
        add.nb[3] = y->ne[0] * y->ne[1] * y->ne[2];
    }
    r.after.count = n;
    return SDHIP_OK;
}

sdhip_status chain_after(const ChainRun &r, hipStream_t stream) {
    if (!r.apart) return SDHIP_OK;
    const int64_t n = r.ne[0] * r.ne[1] * r.ne[2] * r.ne[3];
    if (n == 0) return SDHIP_OK;
    KernelScope prof("chain.apart", stream);
    SDHIP_LAUNCH(chain_apart_kernel, dim3(grid_of(n)), dim3(256), 0, stream, r.apart_in, r.apart_out, n,
                 static_cast<uint32_t>(r.ne[0]), static_cast<uint32_t>(r.ne[1]), static_cast<uint32_t>(r.ne[2]),
                 r.after);
    return launched(hipGetLastError(), "chain apart");
}

sdhip_status gated_after(const float *p, float *out, int64_t rows, int64_t half, int64_t ldp, int64_t ldo,
                         hipStream_t stream) {
    if (rows * half == 0) return SDHIP_OK;
    KernelScope prof("gated.apart", stream);
    SDHIP_LAUNCH(gated_apart_kernel, dim3(grid_of(rows * half)), dim3(256), 0, stream, p, out, rows, half, ldp,
                 ldo);
    return launched(hipGetLastError(), "gated GELU apart");
}

}  // namespace sdhip
