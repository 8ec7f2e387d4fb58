// The C ABI of sdhip.h: the descriptors checked as the reference's
// *_supported predicates check ggml's nodes, the path chosen as hooks.cc and
// the ops choose it, and the kernels launched on the caller's stream.

#include "../../include/sdhip.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <climits>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

#include "host.h"
#include "kernels.h"
#include "norm.h"

namespace sdhip {

namespace {

thread_local std::string g_error;

}  // namespace

sdhip_status fail(sdhip_status s, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return s;
}

sdhip_status check_work(const char *what, const void *work, size_t work_size, size_t need) {
    if (need == 0) return SDHIP_OK;
    if (work == nullptr || work_size < need) {
        return fail(SDHIP_ERROR, "%s: work buffer of %zu bytes, %zu needed", what, work_size, need);
    }
    if ((reinterpret_cast<uintptr_t>(work) & 15) != 0) {
        return fail(SDHIP_ERROR, "%s: work buffer not 16-byte aligned", what);
    }
    return SDHIP_OK;
}

sdhip_status launched(hipError_t e, const char *what) {
    if (e != hipSuccess) {
        return fail(SDHIP_ERROR, "%s: %s", what, hipGetErrorString(e));
    }
    return SDHIP_OK;
}

// ------------------------------------------------------------------ tuning

Tuning &tuning() {
    static Tuning t;
    return t;
}

namespace {

// A tuning name, its field, and the values it takes.  The reference's own
// names take any integer, as its parser does (cpu.cc:180-212), and clamp or
// read them as it does (quant.cc:53-67, winograd.cc:1204-1206): kAny.  This
// library's own names take only the values they are documented with.
enum Range { kAny, kFlag, kStages, kTiles, kNonNegative, kBits, kCore, kFlag2, kPanels };

struct Field {
    const char *name;
    int Tuning::*member;
    Range range;
};

const Field kFields[] = {
    {"bits", &Tuning::bits, kBits},
    {"input_bits", &Tuning::input_bits, kAny},
    {"group", &Tuning::group, kAny},
    {"weight_group", &Tuning::weight_group, kAny},
    {"quantize", &Tuning::quantize, kAny},
    {"winograd", &Tuning::winograd, kAny},
    {"winograd_positions", &Tuning::winograd_positions, kAny},
    {"winograd4_positions", &Tuning::winograd4_positions, kAny},
    {"winograd_small_tiles", &Tuning::winograd_small_tiles, kAny},
    {"fuse", &Tuning::fuse, kAny},
    {"fuse_residual", &Tuning::fuse_residual, kAny},
    {"todo", &Tuning::todo, kAny},
    {"todo_tokens", &Tuning::todo_tokens, kAny},
    {"attention_keys", &Tuning::attention_keys, kAny},
    {"store_forget", &Tuning::store_forget, kAny},
    // The reference's CPU blocking and form names: taken, no effect here.
    {"conv_kc", &Tuning::conv_kc, kAny},
    {"conv_mc", &Tuning::conv_mc, kAny},
    {"conv_nc", &Tuning::conv_nc, kAny},
    {"conv_rows_outer", &Tuning::conv_rows_outer, kAny},
    {"conv_shared_columns", &Tuning::conv_shared_columns, kAny},
    {"conv_columns_bytes", &Tuning::conv_columns_bytes, kAny},
    {"mul_mat_kc", &Tuning::mul_mat_kc, kAny},
    {"mul_mat_mc", &Tuning::mul_mat_mc, kAny},
    {"mul_mat_shared_rows", &Tuning::mul_mat_shared_rows, kAny},
    {"amx_kc", &Tuning::amx_kc, kAny},
    {"amx_mc", &Tuning::amx_mc, kAny},
    {"amx_attention", &Tuning::amx_attention, kAny},
    {"amx_queries", &Tuning::amx_queries, kAny},
    {"amx_fp16", &Tuning::amx_fp16, kAny},
    {"attention_queries", &Tuning::attention_queries, kAny},
    {"attention_sum_keys", &Tuning::attention_sum_keys, kAny},
    {"attention_sum_dims", &Tuning::attention_sum_dims, kAny},
    {"winograd_kc", &Tuning::winograd_kc, kAny},
    {"winograd_mc", &Tuning::winograd_mc, kAny},
    {"winograd_tiles", &Tuning::winograd_tiles, kAny},
    {"winograd_small_mc", &Tuning::winograd_small_mc, kAny},
    {"winograd_small_kc", &Tuning::winograd_small_kc, kAny},
    {"prefetch", &Tuning::prefetch, kAny},
    {"wide", &Tuning::wide, kAny},
    {"bf16", &Tuning::bf16, kAny},
    {"guided", &Tuning::guided, kAny},
    {"half_format", &Tuning::half_format, kAny},
    // This library's own.
    {"winograd_splits", &Tuning::winograd_splits, kNonNegative},
    {"winograd_fp32", &Tuning::winograd_fp32, kFlag},
    {"gemm_stages", &Tuning::gemm_stages, kStages},
    {"gemm_tiles", &Tuning::gemm_tiles, kTiles},
    {"gemm_core", &Tuning::gemm_core, kCore},
    {"mul_mat_panels", &Tuning::mul_mat_panels, kPanels},
    {"conv_panels", &Tuning::conv_panels, kFlag},
    {"qgemm_core", &Tuning::qgemm_core, kFlag2},
    {"attention_generic", &Tuning::attention_generic, kFlag},
    {"attention_fp32", &Tuning::attention_fp32, kFlag},
};

// Whether `v` is a value `r` takes; else the values it does, for the error.
bool in_range(Range r, long v, const char *&takes) {
    switch (r) {
    case kAny:
        takes = "an int";
        return v >= INT32_MIN && v <= INT32_MAX;
    case kFlag:
        takes = "0 or 1";
        return v == 0 || v == 1;
    case kStages:
        takes = "2 or 4";
        return v == 2 || v == 4;
    case kTiles:
        takes = "0, 11, 12, 21, 22 or 41 (gemm_core=3)";
        return v == 0 || v == 11 || v == 12 || v == 21 || v == 22 || v == 41;
    case kCore:
        takes = "0, 1 or 3";
        return v == 0 || v == 1 || v == 3;
    case kFlag2:
        takes = "1 or 2";
        return v == 1 || v == 2;
    case kPanels:
        takes = "0, 1 or 2";
        return v >= 0 && v <= 2;
    case kNonNegative:
        takes = "0 or more";
        return v >= 0 && v <= INT32_MAX;
    case kBits:
        takes = "an int";
        return v >= INT32_MIN && v <= INT32_MAX;
    }
    return false;
}

}  // namespace

// ------------------------------------------------------------------ descriptors

bool holds_f32(const sdhip_tensor *t) { return t != nullptr && t->type == SDHIP_TYPE_F32 && t->nb[0] == 4; }
bool holds_f16(const sdhip_tensor *t) { return t != nullptr && t->type == SDHIP_TYPE_F16 && t->nb[0] == 2; }

bool contiguous(const sdhip_tensor *t) {
    const int64_t size = t->type == SDHIP_TYPE_F16 ? 2 : 4;
    return t->nb[0] == size && t->nb[1] == t->nb[0] * t->ne[0] && t->nb[2] == t->nb[1] * t->ne[1] &&
           t->nb[3] == t->nb[2] * t->ne[2];
}

bool same_shape(const sdhip_tensor *a, const sdhip_tensor *b) {
    for (int k = 0; k < 4; ++k) {
        if (a->ne[k] != b->ne[k]) return false;
    }
    return true;
}

bool same_layout(const sdhip_tensor *a, const sdhip_tensor *b) {
    if (!same_shape(a, b)) return false;
    for (int k = 0; k < 4; ++k) {
        if (a->nb[k] != b->nb[k]) return false;
    }
    return a->type == b->type;
}

int64_t nelements(const sdhip_tensor *t) { return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]; }

size_t tensor_span(const sdhip_tensor *t) {
    size_t n = t->type == SDHIP_TYPE_F16 ? 2 : 4;
    for (int k = 0; k < 4; ++k) {
        if (t->ne[k] <= 0) return 0;
        if (t->nb[k] < 0) return SIZE_MAX;
        const uint64_t reach = static_cast<uint64_t>(t->ne[k] - 1) * static_cast<uint64_t>(t->nb[k]);
        if (reach > SIZE_MAX - n) return SIZE_MAX;
        n += static_cast<size_t>(reach);
    }
    return n;
}

bool spans_overlap(const void *a, size_t an, const void *b, size_t bn) {
    const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
    const uintptr_t ea = an > UINTPTR_MAX - pa ? UINTPTR_MAX : pa + an;
    const uintptr_t eb = bn > UINTPTR_MAX - pb ? UINTPTR_MAX : pb + bn;
    return pa < eb && pb < ea;
}

int compute_units() {
    constexpr int kDevices = 64;
    static std::atomic<int> known[kDevices] = {};
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kDevices) return 256;
    int n = known[device].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || n <= 0) n = 256;
    known[device].store(n, std::memory_order_relaxed);
    return n;
}

// The chain for an output of extents `ne`: each operand F32, nb[0] = 4, and
// of the output's extent or 1 along each dimension (the broadcast ggml's ADD
// and MUL take, fusion.cc:174-186).
sdhip_status device_chain(const sdhip_epilogue *e, const int64_t ne[4], DevChain &c) {
    c = DevChain{};
    if (e == nullptr) return SDHIP_OK;
    if (e->count < 0 || e->count > kMaxSteps) {
        return fail(SDHIP_ERROR, "chain of %d steps (at most %d)", e->count, kMaxSteps);
    }
    for (int s = 0; s < e->count; ++s) {
        const sdhip_step &st = e->steps[s];
        DevStep &d = c.steps[s];
        d.kind = st.kind;
        if (st.kind == SDHIP_STEP_SILU) {
            continue;
        }
        if (st.kind != SDHIP_STEP_ADD && st.kind != SDHIP_STEP_MUL) {
            return fail(SDHIP_ERROR, "chain step %d of unknown kind %d", s, st.kind);
        }
        if (!holds_f32(&st.operand) || st.operand.data == nullptr) {
            return fail(SDHIP_ERROR, "chain step %d: operand is not single precision with nb[0] = 4", s);
        }
        d.operand = static_cast<const float *>(st.operand.data);
        for (int k = 0; k < 4; ++k) {
            if (st.operand.ne[k] != ne[k] && st.operand.ne[k] != 1) {
                return fail(SDHIP_ERROR, "chain step %d: operand extent %lld along %d is neither %lld nor 1", s,
                            static_cast<long long>(st.operand.ne[k]), k, static_cast<long long>(ne[k]));
            }
            if (st.operand.nb[k] % 4 != 0) {
                return fail(SDHIP_ERROR, "chain step %d: stride not a multiple of 4 bytes", s);
            }
            d.nb[k] = st.operand.ne[k] == 1 ? 0 : st.operand.nb[k] / 4;
        }
        d.flat01 = d.nb[1] == ne[0] * d.nb[0] ? 1 : 0;
        d.flat123 = d.nb[2] == ne[1] * d.nb[1] && d.nb[3] == ne[2] * d.nb[2] ? 1 : 0;
    }
    c.count = e->count;
    return SDHIP_OK;
}

// The tensor the operation writes: its own, or the chain's redirect, which
// must have the output's extents and strides (fusion.cc:227-240).
sdhip_status output_of(const sdhip_tensor *y, const sdhip_epilogue *e, float *&out, int32_t &from_redirect) {
    out = static_cast<float *>(y->data);
    from_redirect = 0;
    if (e == nullptr || e->redirect == nullptr) {
        if (e != nullptr && e->from_redirect) {
            return fail(SDHIP_ERROR, "from_redirect without a redirect");
        }
        return SDHIP_OK;
    }
    const sdhip_tensor *r = e->redirect;
    for (int k = 0; k < 4; ++k) {
        if (r->ne[k] != y->ne[k] || r->nb[k] != y->nb[k]) {
            return fail(SDHIP_ERROR, "redirect of another layout than the output");
        }
    }
    if (r->type != SDHIP_TYPE_F32 || r->data == nullptr) {
        return fail(SDHIP_ERROR, "redirect is not single precision");
    }
    out = static_cast<float *>(r->data);
    from_redirect = e->from_redirect ? 1 : 0;
    return SDHIP_OK;
}

}  // namespace sdhip

using namespace sdhip;

extern "C" {

sdhip_status sdhip_init(int device) {
    if (hipSetDevice(device) != hipSuccess) {
        return fail(SDHIP_ERROR, "hipSetDevice(%d) failed", device);
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
        return fail(SDHIP_ERROR, "hipGetDeviceProperties(%d) failed", device);
    }
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        return fail(SDHIP_ERROR, "device %d is %s; this library is built for gfx950", device, prop.gcnArchName);
    }
    // The address of the static scratch on this device (sdhip_group_norm_static).
    double *scratch_ptr = nullptr;
    return static_scratch(device, scratch_ptr);
}

const char *sdhip_last_error(void) { return g_error.c_str(); }

sdhip_status sdhip_set_tuning(const char *text) {
    Tuning t;  // the defaults; the text changes them
    if (text != nullptr) {
        std::string s(text);
        size_t at = 0;
        while (at < s.size()) {
            size_t end = s.find(',', at);
            if (end == std::string::npos) end = s.size();
            const std::string item = s.substr(at, end - at);
            at = end + 1;
            if (item.empty()) continue;
            const size_t eq = item.find('=');
            if (eq == std::string::npos) {
                return fail(SDHIP_ERROR, "tuning item '%s' is not name=value", item.c_str());
            }
            const std::string name = item.substr(0, eq);
            const std::string value = item.substr(eq + 1);
            char *stop = nullptr;
            const long v = std::strtol(value.c_str(), &stop, 10);
            if (value.empty() || stop == nullptr || *stop != '\0') {
                return fail(SDHIP_ERROR, "tuning value '%s' of %s is not a number", value.c_str(), name.c_str());
            }
            bool known = false;
            for (const Field &f : kFields) {
                if (name == f.name) {
                    const char *takes = "";
                    if (!in_range(f.range, v, takes)) {
                        return fail(SDHIP_ERROR, "tuning %s=%ld: %s takes %s", name.c_str(), v, name.c_str(), takes);
                    }
                    t.*(f.member) = static_cast<int>(v);
                    known = true;
                }
            }
            if (!known) {
                return fail(SDHIP_ERROR, "unknown tuning name '%s'", name.c_str());
            }
        }
    }
    tuning() = t;
    return SDHIP_OK;
}

int sdhip_get_tuning(const char *name) {
    if (name == nullptr) return -1;
    for (const Field &f : kFields) {
        if (std::strcmp(name, f.name) == 0) return tuning().*(f.member);
    }
    return -1;
}

void sdhip_forget(const void *begin, size_t size) {
    // store_forget=0 keeps every entry: the store's canary test (store.cc:241-266).
    if (tuning().store_forget != 0) store_forget(begin, size);
}

int sdhip_token_downsampling(int64_t width, int64_t height) {
    // hooks.cc:166-172: every todo-th row and column of a grid of todo_tokens
    // tokens or more; 1 (none) otherwise.
    const Tuning &t = tuning();
    if (t.todo < 2 || width <= 0 || height <= 0 || width * height < t.todo_tokens) return 1;
    return t.todo;
}

void sdhip_store_arena(void *arena, size_t bytes) { store_arena(arena, bytes); }

size_t sdhip_store_used(size_t *entries) { return store_used(entries); }

}  // extern "C"
