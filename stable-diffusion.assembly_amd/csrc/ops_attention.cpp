// FLASH_ATTN_EXT on the device: the predicate of attention_supported
// (attention.cc:828-845) and the launch.

#include <hip/hip_runtime.h>

#include <cstring>

#include "attention.h"
#include "host.h"

using namespace sdhip;

namespace {

bool kv_type(const sdhip_tensor *t) { return holds_f32(t) || holds_f16(t); }

// Whether the attention is computed with quantized products
// (quantized_attention, attention.cc:622-624): bits asks for attention, and
// there are kQuantizedKeys keys and more.
bool quantized_attention(const sdhip_tensor *k) {
    const Tuning &t = tuning();
    return t.bits >= 2 && t.bits <= 8 && (t.quantize & 4) != 0 && k->ne[1] >= 256;
}

QAttentionArgs qargs_of(const sdhip_tensor *q, const sdhip_tensor *k, const sdhip_tensor *v, const sdhip_tensor *y,
                        float scale) {
    const Tuning &t = tuning();
    QAttentionArgs a{};
    a.q = static_cast<const float *>(q->data);
    a.qnb1 = q->nb[1] / 4;
    a.qnb2 = q->nb[2] / 4;
    a.qnb3 = q->nb[3] / 4;
    a.k = k->data;
    a.khalf = k->type == SDHIP_TYPE_F16;
    a.knb1 = k->nb[1] / k->nb[0];
    a.knb2 = k->nb[2] / k->nb[0];
    a.knb3 = k->nb[3] / k->nb[0];
    a.v = v->data;
    a.vhalf = v->type == SDHIP_TYPE_F16;
    a.vnb1 = v->nb[1] / v->nb[0];
    a.vnb2 = v->nb[2] / v->nb[0];
    a.vnb3 = v->nb[3] / v->nb[0];
    a.y = static_cast<float *>(y->data);
    a.ynb1 = y->nb[1] / 4;
    a.ynb2 = y->nb[2] / 4;
    a.ynb3 = y->nb[3] / 4;
    a.d = q->ne[0];
    a.dv = v->ne[0];
    a.lq = q->ne[1];
    a.lk = k->ne[1];
    a.h = q->ne[2];
    a.hk = k->ne[2];
    a.b = q->ne[3];
    a.scale = scale;
    // quant() and over_keys() (quant.cc:59-67; attention.cc:639-643).
    int quads = t.group / 4;
    quads = quads < 1 ? 1 : (quads > 256 ? 256 : quads);
    a.group = 4 * quads;
    const int ib = t.input_bits < 2 ? 2 : (t.input_bits > 8 ? 8 : t.input_bits);
    const int wb = t.bits < 2 ? 2 : (t.bits > 8 ? 8 : t.bits);
    a.levels = (1 << ib) - 1;
    a.wmax = (1 << (wb - 1)) - 1;
    // The stretch of the exponentials (attention.cc:154, 663-664).
    const int64_t keys = t.attention_keys / 8 * 8 > 8 ? t.attention_keys / 8 * 8 : 8;
    a.key_block = keys / a.group * a.group > a.group ? keys / a.group * a.group : a.group;
    return a;
}


// The launch's description of the operands (ggml's ne and nb, in elements).
AttentionArgs args_of(const sdhip_tensor *q, const sdhip_tensor *k, const sdhip_tensor *v, const sdhip_tensor *y,
                      float scale) {
    AttentionArgs a{};
    a.q = static_cast<const float *>(q->data);
    a.qnb1 = q->nb[1] / 4;
    a.qnb2 = q->nb[2] / 4;
    a.qnb3 = q->nb[3] / 4;
    a.k = k->data;
    a.khalf = k->type == SDHIP_TYPE_F16;
    a.knb1 = k->nb[1] / k->nb[0];
    a.knb2 = k->nb[2] / k->nb[0];
    a.knb3 = k->nb[3] / k->nb[0];
    a.v = v->data;
    a.vhalf = v->type == SDHIP_TYPE_F16;
    a.vnb1 = v->nb[1] / v->nb[0];
    a.vnb2 = v->nb[2] / v->nb[0];
    a.vnb3 = v->nb[3] / v->nb[0];
    a.y = static_cast<float *>(y->data);
    a.ynb1 = y->nb[1] / 4;
    a.ynb2 = y->nb[2] / 4;
    a.ynb3 = y->nb[3] / 4;
    a.d = q->ne[0];
    a.dv = v->ne[0];
    a.lq = q->ne[1];
    a.lk = k->ne[1];
    a.h = q->ne[2];
    a.hk = k->ne[2];
    a.b = q->ne[3];
    a.scale = scale;
    // bits=16 with half_format=1: the products of the first parts in
    // bfloat16, as on the reference's vector units of AVX512-BF16
    // (attention.cc:309-323, 466-467).  With the FP16 format attention stays
    // single precision there, and here.
    a.bf16 = tuning().bits == 16 && tuning().half_format == 1 ? 1 : 0;
    return a;
}

}  // namespace

extern "C" {

int sdhip_attention_supported(const sdhip_tensor *q, const sdhip_tensor *k, const sdhip_tensor *v,
                              const sdhip_tensor *y, float max_bias, float softcap) {
    if (q == nullptr || k == nullptr || v == nullptr || y == nullptr) return 0;
    // No mask, ALiBi or soft cap; q single precision, k and v single
    // precision or FP16, each of elements one after another along ne[0]; the
    // heads of q a multiple of those of k (attention.cc:828-845), heads of
    // any size.  The quantized form (the bits mode, from 256 keys) takes heads
    // of up to kAttentionMaxDims dimensions; wider ones in that mode are left
    // to the caller.
    const bool shapes = q->ne[0] == k->ne[0] && k->ne[1] == v->ne[1] && k->ne[2] == v->ne[2] && k->ne[2] > 0 &&
                        q->ne[2] % k->ne[2] == 0 && q->ne[3] == k->ne[3] && q->ne[3] == v->ne[3] && k->ne[1] >= 1 &&
                        y->ne[0] == v->ne[0] && y->ne[1] == q->ne[2] && y->ne[2] == q->ne[1] && y->ne[3] == q->ne[3];
    const bool taken = max_bias == 0.0f && softcap == 0.0f && holds_f32(q) && kv_type(k) && kv_type(v) &&
                       holds_f32(y) && contiguous(y) && shapes &&
                       (!quantized_attention(k) || (q->ne[0] <= kAttentionMaxDims && v->ne[0] <= kAttentionMaxDims)) &&
                       q->nb[1] % 4 == 0 && q->nb[2] % 4 == 0 &&
                       q->nb[3] % 4 == 0 && k->nb[1] % k->nb[0] == 0 && k->nb[2] % k->nb[0] == 0 &&
                       k->nb[3] % k->nb[0] == 0 && v->nb[1] % v->nb[0] == 0 && v->nb[2] % v->nb[0] == 0 &&
                       v->nb[3] % v->nb[0] == 0;
    // In the bits mode the quantized form takes the same heads (up to
    // kAttentionMaxDims dimensions) and every group quant() gives (a multiple
    // of 4 from 4 to 1024 keys).
    return taken ? 1 : 0;
}

size_t sdhip_attention_work_size(const sdhip_tensor *q, const sdhip_tensor *k, const sdhip_tensor *v,
                                 const sdhip_tensor *y) {
    if (!sdhip_attention_supported(q, k, v, y, 0.0f, 0.0f)) return 0;
    if (!quantized_attention(k)) return attention_work_bytes(args_of(q, k, v, y, 1.0f));
    QAttentionArgs a = qargs_of(q, k, v, y, 1.0f);
    return qattention_layout(a).total;
}

sdhip_status sdhip_attention(const sdhip_tensor *q, const sdhip_tensor *k, const sdhip_tensor *v,
                             const sdhip_tensor *y, float scale, float max_bias, float softcap, void *work,
                             size_t work_size, void *stream) {
    if (!sdhip_attention_supported(q, k, v, y, max_bias, softcap)) {
        return fail(SDHIP_UNSUPPORTED, "attention: operands not taken");
    }
    if (quantized_attention(k)) {
        QAttentionArgs qa = qargs_of(q, k, v, y, scale);
        const size_t need = qattention_layout(qa).total;
        if (const sdhip_status ws = check_work("attention", work, work_size, need); ws != SDHIP_OK) return ws;
        if (qa.lq == 0 || qa.h == 0 || qa.b == 0) return SDHIP_OK;
        return launched(launch_quantized_attention(qa, work, static_cast<hipStream_t>(stream)),
                        "quantized attention");
    }
    const AttentionArgs a = args_of(q, k, v, y, scale);
    const size_t need = attention_work_bytes(a);
    if (const sdhip_status ws = check_work("attention", work, work_size, need); ws != SDHIP_OK) return ws;
    return launched(launch_attention(a, work, static_cast<hipStream_t>(stream)), "attention");
}

}  // extern "C"
