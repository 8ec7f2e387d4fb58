// Host-side helpers shared by the operations of the C ABI.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "../../include/sdhip.h"
#include "device.h"
#include "kernels.h"

namespace sdhip {

// The fields of the reference's Tuning that change what is computed
// (sources/kernels.h:91-135), with its defaults.
struct Tuning {
    // 0 single precision; 2..8 quantized products (quant.h); 16 products of
    // 16 bits: MUL_MAT and direct convolutions of FP16 weights by their other
    // operand rounded to FP16, one product each, summed in single precision
    // (the reference's FP16 format of gemm.h:226-237); Winograd and attention
    // stay single precision, as on the reference's vector units.  With
    // half_format=1 (below), the bfloat16 format: both operands of those
    // products rounded to bfloat16, and attention's too (cpu.cc:319-321,
    // attention.cc:309-323).
    int bits = 0;
    int input_bits = 8;              // the inputs' bits, unsigned with a zero point
    int group = 64;                  // numbers of k sharing a scale, a multiple of 4
    int weight_group = 1;            // the weights' scale per group: 1; per whole row of k: 0
    int quantize = 7;                // with bits: 1 linear, 2 convolution, 4 attention
    int winograd = 2;                // 2: F(2x2) and F(4x4); 1: F(2x2) alone; 0: direct
    int winograd_positions = 1024;   // the least outputs of an image Winograd is used for
    int winograd4_positions = 256;   // the least outputs of an image F(4x4) is used for
    int winograd_small_tiles = 256;  // the most tiles of all images taken as small images
    // This library's own: the splits of the input channels of the small
    // images' Winograd products, or 0 to choose by the size.
    int winograd_splits = 0;
    // The chains after operations: 1 fused into them; 0 apart -- the planner
    // (graph.cpp) matches none, and an entry point handed one applies it in a
    // pass of its own after the operation, as ggml's nodes would one by one.
    int fuse = 1;
    // The residual connections that end chains (fusion.h:64-80): 1 fused as a
    // redirect; 0 apart -- the planner matches none, and an entry point handed
    // one writes its own output and adds the residual in a pass of its own.
    int fuse_residual = 1;
    // ToDo (token downsampling, sdasm.h:61-67): attention of an image's tokens
    // with keys and values from every todo-th row and column of the grid, for
    // grids of todo_tokens tokens or more; 0 or 1 none.
    int todo = 0;
    int todo_tokens = 2048;
    // This library's own: Winograd's products on the single-precision MFMA
    // (1) instead of split FP16 parts (0), for comparison; results agree
    // within the same bound.
    int winograd_fp32 = 0;
    // This library's own: the K steps a product's loads run ahead of its
    // MFMAs, 2 or 4.
    int gemm_stages = 2;
    // This library's own: a product's block of 64 TM x 64 TN as TM TN (11,
    // 12, 21, 22), or 0 to choose by the size.
    int gemm_tiles = 0;
    // This library's own: Winograd's products by the core staged through
    // registers (1) or by the one whose copies into LDS global_load_lds
    // makes (2), for comparison: the same bits, measured no faster.
    int gemm_core = 0;
    int qgemm_core = 2;
    // This library's own: MUL_MAT of many output panels by the panel core (1)
    // or by the 64 x 64 core everywhere (0), for comparison; results agree
    // within the same bound.
    int mul_mat_panels = 1;
    int conv_panels = 1;
    // This library's own: attention by its generic form (1) even where the
    // fast one takes the operands (0), for comparison; results agree within
    // the same bound.
    int attention_generic = 0;
    // This library's own: attention's products on the single-precision MFMA
    // (1) instead of split FP16 parts (0), for comparison; results agree
    // within the same bound.
    int attention_fp32 = 0;
    // The keys of a stretch of attention's second product (kernels.h:107):
    // with bits, it sets where the exponentials switch to std::exp.
    int attention_keys = 256;
    // The reference's names that size its CPU blocks and choose among its CPU
    // forms (kernels.h:92-120, 124-125, 129): taken so that SDASM_TUNE
    // strings carry over, held for sdhip_get_tuning, and without effect on
    // what this library computes or how.
    int conv_kc = 256, conv_mc = 480, conv_nc = 128, conv_rows_outer = 0, conv_shared_columns = 1024,
        conv_columns_bytes = 4 << 20, mul_mat_kc = 256, mul_mat_mc = 96, mul_mat_shared_rows = 1024, amx_kc = 256,
        amx_mc = 128, amx_attention = 0, amx_queries = 64, amx_fp16 = 1, attention_queries = 32,
        attention_sum_keys = 32, attention_sum_dims = 40, winograd_kc = 256, winograd_mc = 512, winograd_tiles = 64,
        winograd_small_mc = 48, winograd_small_kc = 128, prefetch = 1, wide = 1, bf16 = 0, guided = 1,
        half_format = 0;
    // The store forgets what sdhip_forget names: 1; 0 keeps every entry, only
    // for the store's canary test (kernels.h:126).
    int store_forget = 1;
};

Tuning &tuning();

inline GemmShape gemm_shape() { return GemmShape{tuning().gemm_stages, tuning().gemm_tiles}; }

sdhip_status fail(sdhip_status s, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// The caller's work buffer of a call that needs `need` bytes of it (none: any
// buffer, or none): present, at least that large, and 16-byte aligned, as the
// kernels move 16-byte vectors through it.  SDHIP_ERROR naming `what` else.
sdhip_status check_work(const char *what, const void *work, size_t work_size, size_t need);
sdhip_status launched(hipError_t e, const char *what);

bool holds_f32(const sdhip_tensor *t);
bool holds_f16(const sdhip_tensor *t);
bool contiguous(const sdhip_tensor *t);
bool same_shape(const sdhip_tensor *a, const sdhip_tensor *b);
bool same_layout(const sdhip_tensor *a, const sdhip_tensor *b);
int64_t nelements(const sdhip_tensor *t);
// The bytes from a tensor's first element to one past its last (ggml_nbytes
// of one-element blocks); 0 for an empty tensor, SIZE_MAX where a stride is
// negative (its reach is not bounded here, so it is taken to reach anything).
size_t tensor_span(const sdhip_tensor *t);
// Whether the bytes [a, a + an) and [b, b + bn) share any: the addresses
// compared as integers, the ends saturating, nothing read.
bool spans_overlap(const void *a, size_t an, const void *b, size_t bn);
// The compute units of the current device (looked up once a device; 256,
// MI355X's, where the runtime cannot say).
int compute_units();
// The address `bytes` past p as an integer (no pointer arithmetic on what
// may be a null or foreign pointer).
inline uintptr_t address_past(const void *p, int64_t bytes) {
    return reinterpret_cast<uintptr_t>(p) + static_cast<uintptr_t>(bytes);
}

sdhip_status device_chain(const sdhip_epilogue *e, const int64_t ne[4], DevChain &c);
sdhip_status output_of(const sdhip_tensor *y, const sdhip_epilogue *e, float *&out, int32_t &from_redirect);

// How an operation computes the chain it is handed (chain.hip): `fused`, the
// steps it applies to its tile, into `out` (begun from what out holds if
// from_redirect); and, with Tuning::fuse = 0 or (for a redirect)
// fuse_residual = 0, a pass `after` the operation over its own output
// (apart_in) into apart_out -- the steps it did not apply and, from a
// redirect, the residual's addition.  With a redirect and no from_redirect,
// the chain's last step is the residual's addition (fusion.cc:262-271).
struct ChainRun {
    DevChain fused;
    float *out = nullptr;
    int32_t from_redirect = 0;
    bool apart = false;
    DevChain after;
    const float *apart_in = nullptr;
    float *apart_out = nullptr;
    int64_t ne[4] = {0, 0, 0, 0};
};
sdhip_status chain_plan(const sdhip_tensor *y, const sdhip_epilogue *e, ChainRun &r);
sdhip_status chain_after(const ChainRun &r, hipStream_t stream);
// out[m][j] = p[m][j] GELU(p[m][half + j]), rows of p ldp apart, of out ldo.
sdhip_status gated_after(const float *p, float *out, int64_t rows, int64_t half, int64_t ldp, int64_t ldo,
                         hipStream_t stream);

// The device store of derived weights (store.cpp).  store_entry: the entry of
// `bytes` for the form `layout`/`variant` of the tensor at `begin` (of
// `source` bytes), made if the arena has room and the stream is not being
// captured, or null; `ready` whether an earlier call filled it.  The call that
// gets an entry not ready fills it on its stream, then store_publish()es it.
enum StoreLayout : int32_t { kStoreQuantizedLinear = 1, kStoreWinograd = 2, kStoreWinogradSmall = 3 };
void *store_entry(const void *begin, int32_t type, const int64_t ne[4], const int64_t nb[4], int32_t layout,
                  uint64_t variant, size_t source, size_t bytes, hipStream_t stream, bool &ready);
void store_publish(const void *entry);
void store_forget(const void *begin, size_t size);
void store_arena(void *arena, size_t bytes);
size_t store_used(size_t *entries);

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

}  // namespace sdhip
