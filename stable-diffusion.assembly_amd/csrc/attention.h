// FLASH_ATTN_EXT (attention.cc) on the device.  Strides in elements.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace sdhip {

struct AttentionArgs {
    const float *q;
    int64_t qnb1, qnb2, qnb3;
    const void *k;  // F32 or F16 (khalf)
    int64_t knb1, knb2, knb3;
    const void *v;
    int64_t vnb1, vnb2, vnb3;
    float *y;  // [b][lq][h][dv]
    int64_t ynb1, ynb2, ynb3;
    int64_t d, dv, lq, lk, h, hk, b;
    float scale;
    int32_t khalf, vhalf;
    // The products of 16 bits in bfloat16 (bits=16, half_format=1): the
    // queries, keys, values and exponentials rounded to bfloat16 before their
    // products, which are summed in single precision.
    int32_t bf16;
    // Set by the launcher.
    int32_t dp, ldq, ldk, ldv;
    int64_t qblocks;
};

// The most dimensions of a head the quantized form takes (queries, keys and
// values).  The single-precision forms take any: up to 256 in one pass, wider
// heads (the VAE's 512) by chunks of 128, values past 512 in slices of 512.
constexpr int64_t kAttentionMaxDims = 512;

// The bits mode of self-attention (qattention.hip): the operands, the
// quantization (levels, wmax, group), the stretch of keys of the
// exponentials, and the work buffer's parts, set by qattention_layout.
struct QAttentionArgs {
    const float *q;
    int64_t qnb1, qnb2, qnb3;
    const void *k;
    int64_t knb1, knb2, knb3;
    const void *v;
    int64_t vnb1, vnb2, vnb3;
    float *y;
    int64_t ynb1, ynb2, ynb3;
    int64_t d, dv, lq, lk, h, hk, b;
    float scale;
    int32_t khalf, vhalf;
    int32_t levels, wmax;
    int64_t group, key_block;
    // Set by qattention_layout.
    int64_t gd, sd, lkp, lqp, groups, slot, dvp, dvc, tail_from, qblocks;
    int8_t *kq, *vq, *qq;
    float *ks, *ko, *vs, *vo, *qs, *qo;
    int32_t *ksum, *vsum;
};

struct QAttentionLayout {
    size_t kq, ks, ko, ksum, vq, vs, vo, vsum, qq, qs, qo, total;
};

QAttentionLayout qattention_layout(QAttentionArgs &a);
hipError_t launch_quantized_attention(QAttentionArgs a, void *work, hipStream_t stream);

size_t attention_lds_bytes(int64_t d, int64_t dv);
// The work buffer the attention takes (the split form's tiles of the keys and
// values; nothing for the other forms), and the launch, `work` at least that.
size_t attention_work_bytes(const AttentionArgs &a);
hipError_t launch_attention(AttentionArgs a, void *work, hipStream_t stream);

}  // namespace sdhip
