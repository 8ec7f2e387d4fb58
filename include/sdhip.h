/*
 * sdhip.h -- the C ABI of the MI355X (gfx950) form of the operations that
 * stable-diffusion.assembly takes over from ggml's CPU backend.
 *
 * The reference offers its operations to ggml through sources/sdasm.h
 * (sdasm_compute_nodes, sdasm_work_size, sdasm_forget) and, inside, through
 * one supported / work_size / compute triple per operation (sources/ops.h:26-62).
 * This header is the same surface with ggml's types taken out: a tensor is a
 * plain descriptor (ggml's type number, extents ne[4], strides nb[4] in bytes,
 * a DEVICE pointer), the chain of element-wise nodes after an operation is a
 * plain array of steps, and every compute call takes the caller's device work
 * buffer (as ggml hands its wdata, sized by sdasm_work_size) and a HIP stream.
 *
 * Nothing here allocates device memory: the caller owns every tensor and the
 * work buffer, as ggml owns them for the reference (sdasm.h:51-54).  A work
 * buffer must be 16-byte aligned (the kernels move 16-byte vectors through
 * it; hipMalloc's are 256-byte aligned): a call that needs one and is handed
 * a misaligned, missing or short one returns SDHIP_ERROR.
 *
 * Errors.  SDHIP_UNSUPPORTED is the reference's "not taken" (false / 0 from
 * sdasm_compute_nodes, hooks.cc:29-55): the caller computes the node itself.
 * SDHIP_ERROR is a programming error or a failed launch; sdhip_last_error()
 * says which.  The reference aborts on those (SDASM_REQUIRE, memory.h:68-77);
 * a library returns instead.
 */
#ifndef SDHIP_H
#define SDHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types, numbered as ggml numbers them (GGML_TYPE_F32 = 0,
 * GGML_TYPE_F16 = 1); the only two the reference's operations take
 * (mul_mat.cc:181-194, conv2d.cc:320-331, attention.cc:828-845). */
enum { SDHIP_TYPE_F32 = 0, SDHIP_TYPE_F16 = 1 };

typedef enum { SDHIP_OK = 0, SDHIP_UNSUPPORTED = 1, SDHIP_ERROR = 2 } sdhip_status;

/* A tensor as ggml_tensor describes its memory: ne[] extents, nb[] strides in
 * bytes (nb[0] the element size for the layouts taken), data on the device. */
typedef struct sdhip_tensor {
    int32_t type;
    int64_t ne[4];
    int64_t nb[4];
    void *data;
} sdhip_tensor;

/* One node of the chain after an operation (sources/fusion.h:51-61): an
 * addition or a multiplication by `operand`, broadcast along each dimension
 * whose extent is 1, in place on the operation's output; or SiLU of it. */
enum { SDHIP_STEP_ADD = 0, SDHIP_STEP_MUL = 1, SDHIP_STEP_SILU = 2 };

typedef struct sdhip_step {
    int32_t kind;
    sdhip_tensor operand; /* f32, nb[0] = 4; unused for SILU */
} sdhip_step;

#define SDHIP_MAX_STEPS 6

/* The chain (sources/fusion.h:63-108, Epilogue): `count` steps applied in
 * order to each output element while it is still on chip.  With `redirect`
 * the operation writes into that tensor (same extents and strides as its own
 * output) instead of its own -- a residual connection that ends the chain;
 * with `from_redirect` its sum begins from what `redirect` holds (the
 * residual already there), as Epilogue::from_redirect does. */
typedef struct sdhip_epilogue {
    int32_t count;
    sdhip_step steps[SDHIP_MAX_STEPS];
    const sdhip_tensor *redirect;
    int32_t from_redirect;
} sdhip_epilogue;

/* ---------------------------------------------------------------- library */

/* Makes `device` current for the calls of this thread and checks that it is
 * a gfx950; returns SDHIP_ERROR on any other. */
sdhip_status sdhip_init(int device);

/* The text of the last SDHIP_ERROR or SDHIP_UNSUPPORTED of this thread. */
const char *sdhip_last_error(void);

/* The tuning that changes what is computed, in the reference's SDASM_TUNE
 * syntax "name=value,..." (sources/kernels.h:91-135, parsed by cpu.cc:121-212):
 * every name of the reference's Tuning is taken, with its default.  Those
 * that change what is computed: bits (2..8, the quantized products; 16, the
 * reference's products of 16-bit numbers: MUL_MAT, the gated GELU and direct
 * convolutions of FP16 weights take the other operand rounded to FP16; with
 * half_format=1 both operands rounded to bfloat16 instead, and attention's
 * queries, keys, values and exponentials too, cpu.cc:319-321,
 * attention.cc:309-323),
 * input_bits, group, weight_group, quantize (with bits 2..8: 1 linear layers,
 * 2 convolutions -- direct, or F(2x2,3x3) for those Winograd takes -- 4
 * attention), winograd, winograd_positions, winograd4_positions,
 * winograd_small_tiles, attention_keys, fuse and fuse_residual (0: the
 * planner fuses no chain, or no residual connection, and an entry point
 * handed one computes it in a pass of its own after the operation, as ggml's
 * nodes would), todo and todo_tokens (sdhip_token_downsampling) and
 * store_forget (0 keeps every store entry, for the store's canary test).  Two
 * names of the reference's CPU blocking also change results, and act here as
 * there: winograd_kc and winograd_small_kc set the stretch of input channels
 * over which the bits mode quantizes Winograd's transformed weights at a time
 * (winograd.cc:238-255, 1859-1866).  The other names that size the
 * reference's CPU blocks or choose among its CPU forms (conv_kc, mul_mat_mc,
 * amx_*, wide, prefetch, guided, ...) are taken and have no effect here;
 * half_format (1: bits=16's bfloat16 products; any other value its FP16 form)
 * is described with bits.  The reference's names take any int, as its
 * parser does, and are clamped where it clamps them (quant.cc:59-67).  This
 * library's own: winograd_fp32, winograd_splits, gemm_stages, gemm_tiles,
 * gemm_core, qgemm_core, mul_mat_panels (0: MUL_MAT by the 64 x 64 core
 * instead of the panel kernels; 2: panels of 64 x 160 only, not 64 x 64),
 * conv_panels (0:
 * 1x1 convolutions by the 64 x 64 core),
 * attention_generic, attention_fp32 (forms to compare, same results within
 * the bounds -- qgemm_core's bit for bit), each taking only its documented
 * values.  Returns SDHIP_ERROR
 * naming the first unknown name or refused value.  "" resets the defaults. */
sdhip_status sdhip_set_tuning(const char *text);
/* The value of one tuning field, or -1 if it has no such name. */
int sdhip_get_tuning(const char *name);

/* Forgets what the library keeps derived from device memory in
 * [begin, begin + size) -- the reference's sdasm_forget (sdasm.h:56-60,
 * store.cc:241-266), called when that memory is about to change. */
void sdhip_forget(const void *begin, size_t size);

/* The device store of the forms the library derives from weights and keeps
 * from one call to the next -- the reference's store (sources/store.h,
 * store.cc), whose quantized layouts are kept by default within a budget
 * (store.cc:64-99).  Here the budget is memory the caller gives: `arena`,
 * `bytes` of device memory, 256-byte aligned, that the library places its
 * entries in (the quantized weights of the bits mode's MUL_MATs: bytes,
 * scales, offsets and sums; Winograd's transformed weights in single
 * precision with their exponents, which the reference keeps when its budget
 * allows, winograd.cc:2147-2149; for the small images' Winograd, each split's
 * exponents of the weights).  A NULL arena or 0 bytes keeps nothing (the
 * default); a new arena forgets every entry of the last.  An entry is filled
 * by the first call that needs it, on that call's stream, and read by later
 * calls: they must be ordered after it on the device (one stream, or an
 * event), and no entry is made while a stream is captured into a graph.
 * sdhip_forget drops the entries derived from the memory it names. */
void sdhip_store_arena(void *arena, size_t bytes);
/* The bytes of the arena in use, and (if not NULL) how many entries. */
size_t sdhip_store_used(size_t *entries);

/* The profile of the kernels (the reference's sdasm_profile_*, sdasm.h:63-76,
 * profile.cc): with profiling on, each kernel launch is bracketed by HIP
 * events on its own stream; sdhip_profile_collect() waits for them and adds
 * the times up per kernel name, returning how many names there are, and
 * sdhip_profile_entry() reads entry i (total milliseconds, launches). */
void sdhip_profile_enable(int on);
void sdhip_profile_reset(void);
int sdhip_profile_collect(void);
int sdhip_profile_entry(int i, const char **name, double *total_ms, int64_t *launches);

/* ---------------------------------------------------------------- MUL_MAT */

/* GGML_OP_MUL_MAT of one weight matrix w (F16/F32, ne = [K, N, 1, 1]) by
 * x (F32 contiguous, ne = [K, M1, M2, M3]) into y (F32 contiguous,
 * ne = [N, M1, M2, M3]): y[n, m] = sum_k w[k, n] x[k, m].  Single-precision
 * weights are taken as the reference takes them (mul_mat.cc:187-194): split
 * into two FP16 planes with a power-of-two scale per row, products of both
 * parts.  The work buffer: in the bits mode the quantized operands; for
 * single-precision weights their planes; otherwise, for a product of few
 * output blocks and long K (split along K), the splits' partial sums; 0
 * else.  A buffer short of sdhip_mul_mat_work_size is SDHIP_ERROR.
 * Replaces mul_mat_supported / mul_mat_work_size / mul_mat_compute
 * (sources/ops.h:40-44; mul_mat.cc:181-194, 205-215, 1175-1196). */
int sdhip_mul_mat_supported(const sdhip_tensor *w, const sdhip_tensor *x, const sdhip_tensor *y);
size_t sdhip_mul_mat_work_size(const sdhip_tensor *w, const sdhip_tensor *x, const sdhip_tensor *y);
sdhip_status sdhip_mul_mat(const sdhip_tensor *w, const sdhip_tensor *x, const sdhip_tensor *y,
                           const sdhip_epilogue *chain, void *work, size_t work_size, void *stream);

/* The same product with the GEGLU after it (fusion.h:110-127, fusion.cc:347-394):
 * P = the product with its chain, split into halves along dimension 0;
 * out[j, m] = P[j, m] * GELU(P[half + j, m]); the product itself (y) is never
 * written.  Replaces mul_mat_gated_supported / mul_mat_compute_gated
 * (ops.h:45-49; mul_mat.cc:1128-1173). */
int sdhip_mul_mat_gated_supported(const sdhip_tensor *w, const sdhip_tensor *x, const sdhip_tensor *y,
                                  const sdhip_tensor *out);
sdhip_status sdhip_mul_mat_gated(const sdhip_tensor *w, const sdhip_tensor *x, const sdhip_tensor *y,
                                 const sdhip_epilogue *chain, const sdhip_tensor *out, void *work, size_t work_size,
                                 void *stream);

/* ---------------------------------------------------------------- CONV_2D */

/* GGML_OP_CONV_2D (ggml_conv_2d_direct): kernel ne = [KW, KH, IC, OC]
 * (F16/F32 contiguous), input ne = [IW, IH, IC, N] (F32, nb[0] = 4), y
 * ne = [OW, OH, OC, N] (F32 contiguous), op_params = {s0, s1, p0, p1, d0, d1}.
 * The library takes it by Winograd F(4x4,3x3) / F(2x2,3x3) where the
 * reference would (winograd_supported, four, small; winograd.cc:194-196,
 * 1204-1206, 2107-2123) and directly otherwise (conv2d_supported,
 * conv2d.cc:320-331); in the bits mode with quantize & 2, the direct
 * convolution's products quantized (conv2d.cc:338-483) or F(2x2,3x3) with
 * quantized products (winograd.cc:1826-2103).  The work buffer: Winograd's
 * exponents, transformed operands and products; for a direct convolution of
 * a kernel other than 1x1 with IC KH KW a multiple of 32 (and of a 1x1 one
 * whose output has few blocks and whose K is long), its columns and the
 * partial sums of its splits of K; single-precision kernels' FP16
 * planes; the quantized columns and products; 0 else.  A buffer short of sdhip_conv2d_work_size is
 * SDHIP_ERROR.  Replaces conv2d_* and winograd_* of ops.h:26-38. */
int sdhip_conv2d_supported(const sdhip_tensor *kernel, const sdhip_tensor *input, const sdhip_tensor *y,
                           const int32_t op_params[6]);
/* Which path a supported convolution takes: 0 direct, 2 Winograd F(2x2,3x3),
 * 4 Winograd F(4x4,3x3); -1 if not supported. */
int sdhip_conv2d_path(const sdhip_tensor *kernel, const sdhip_tensor *input, const sdhip_tensor *y,
                      const int32_t op_params[6]);
size_t sdhip_conv2d_work_size(const sdhip_tensor *kernel, const sdhip_tensor *input, const sdhip_tensor *y,
                              const int32_t op_params[6]);
sdhip_status sdhip_conv2d(const sdhip_tensor *kernel, const sdhip_tensor *input, const sdhip_tensor *y,
                          const int32_t op_params[6], const sdhip_epilogue *chain, void *work, size_t work_size,
                          void *stream);

/* ---------------------------------------------------------------- FLASH_ATTN_EXT */

/* GGML_OP_FLASH_ATTN_EXT without a mask (attention.cc:828-845): q ne =
 * [d, lq, h, b] F32 (any strides, nb[0] = 4), k ne = [d, lk, hk, b] and v ne =
 * [dv, lk, hk, b] F32 or F16, y ne = [dv, h, lq, b] F32 contiguous; head h
 * reads key head h / (h / hk).  scale, max_bias and softcap are op_params[0..2];
 * only max_bias = softcap = 0 is taken, heads of any size (values of more
 * than 512 dimensions in slices of 512, each computing the same scores); in
 * the bits mode, where its quantized form applies (256 keys or more), heads
 * of up to 512 dimensions, with every group of keys its tuning gives (a
 * multiple of 4 from 4 to 1024, quant.cc:59-67).  The work
 * buffer: in the bits mode the quantized operands; otherwise, for
 * single-precision keys and values of the head sizes 32, 40, 64, 80, 96, 128
 * and 160, the keys and values split into FP16 parts, tile by tile, and,
 * where the queries alone leave the device's CUs idle and the keys are split
 * across blocks, each split's maximum, sum and output; the same for heads of
 * more than 256 dimensions whose keys are split across blocks; 0 for the
 * other forms.  A buffer short of
 * sdhip_attention_work_size is SDHIP_ERROR.  Replaces attention_supported /
 * attention_work_size / attention_compute (ops.h:51-56). */
int sdhip_attention_supported(const sdhip_tensor *q, const sdhip_tensor *k, const sdhip_tensor *v,
                              const sdhip_tensor *y, float max_bias, float softcap);
size_t sdhip_attention_work_size(const sdhip_tensor *q, const sdhip_tensor *k, const sdhip_tensor *v,
                                 const sdhip_tensor *y);
sdhip_status sdhip_attention(const sdhip_tensor *q, const sdhip_tensor *k, const sdhip_tensor *v,
                             const sdhip_tensor *y, float scale, float max_bias, float softcap, void *work,
                             size_t work_size, void *stream);

/* ---------------------------------------------------------------- GROUP_NORM, NORM */

/* GGML_OP_GROUP_NORM (norm.cc:100-140): x, y F32 contiguous of one shape,
 * `groups` groups of ceil(ne2 / groups) channels over ne[2], per image ne[3];
 * then the chain (scale, shift, SiLU).  Replaces group_norm_supported /
 * group_norm_compute (ops.h:58-61).  The work buffer holds
 * the partial sums of the group's slices: the bytes sdasm_work_size would
 * report for the node (sdasm.h:51-54), where the reference's own form needs
 * none. */
int sdhip_group_norm_supported(const sdhip_tensor *x, const sdhip_tensor *y, int groups);
size_t sdhip_group_norm_work_size(const sdhip_tensor *x, const sdhip_tensor *y, int groups);
sdhip_status sdhip_group_norm(const sdhip_tensor *x, const sdhip_tensor *y, int groups, float eps,
                              const sdhip_epilogue *chain, void *work, size_t work_size, void *stream);

/* sdhip_group_norm without a work buffer, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc): no counterpart in the reference, whose GROUP_NORM
 * takes no work buffer (sdasm_work_size reports none for it, hooks.cc:188-191).
 * The partial sums go to a static scratch of 1 MiB in the library's device
 * code, one copy per GPU, held until the process ends: shapes whose sums need
 * more (sdhip_group_norm_work_size > 1 MiB) are SDHIP_ERROR.  Allocates
 * nothing, on the current device; the scratch keeps the last call's sums and
 * every call on one GPU shares it, so calls that overlap on one GPU (two
 * streams, or two threads) race.  Results are those of sdhip_group_norm. */
sdhip_status sdhip_group_norm_static(const sdhip_tensor *x, const sdhip_tensor *y, int groups, float eps,
                                     const sdhip_epilogue *chain, void *stream);

/* GGML_OP_NORM over ne[0] (norm.cc:148-175), then the chain.  Replaces
 * norm_supported / norm_compute (ops.h:62-63). */
int sdhip_norm_supported(const sdhip_tensor *x, const sdhip_tensor *y);
sdhip_status sdhip_norm(const sdhip_tensor *x, const sdhip_tensor *y, float eps, const sdhip_epilogue *chain,
                        void *stream);

/* ---------------------------------------------------------------- the graph */

/* A node of a ggml graph, as the planner reads it: what ggml_tensor holds of
 * it, without ggml's types.  `op` is ggml's operation by this enumeration
 * (GGML_OP_NONE, VIEW, RESHAPE, PERMUTE, TRANSPOSE -- the empty ones,
 * ggml_op_is_empty -- and the rest the planner looks at; any other operation
 * is SDHIP_OP_OTHER), `unary` ggml_get_unary_op of a UNARY node, `flags`
 * GGML_TENSOR_FLAG_COMPUTE and GGML_TENSOR_FLAG_OUTPUT as these bits,
 * `op_params` ggml's op_params words, `tensor` the node's own type, ne, nb
 * and data, `src` and `view_src` the nodes ggml points at (NULL where none). */
enum {
    SDHIP_OP_NONE = 0,
    SDHIP_OP_VIEW,
    SDHIP_OP_RESHAPE,
    SDHIP_OP_PERMUTE,
    SDHIP_OP_TRANSPOSE,
    SDHIP_OP_ADD,
    SDHIP_OP_MUL,
    SDHIP_OP_CONT,
    SDHIP_OP_UNARY,
    SDHIP_OP_MUL_MAT,
    SDHIP_OP_CONV_2D,
    SDHIP_OP_FLASH_ATTN_EXT,
    SDHIP_OP_GROUP_NORM,
    SDHIP_OP_NORM,
    SDHIP_OP_OTHER
};
enum { SDHIP_UNARY_OTHER = 0, SDHIP_UNARY_SILU = 1, SDHIP_UNARY_GELU = 2 };
enum { SDHIP_FLAG_COMPUTE = 1, SDHIP_FLAG_OUTPUT = 2 };
#define SDHIP_MAX_SRC 10
#define SDHIP_MAX_OP_PARAMS 16

typedef struct sdhip_node {
    int32_t op;
    int32_t unary;
    int32_t flags;
    int32_t op_params[SDHIP_MAX_OP_PARAMS];
    sdhip_tensor tensor;
    const struct sdhip_node *src[SDHIP_MAX_SRC];
    const struct sdhip_node *view_src;
} sdhip_node;

/* What the library does with node `index` of a graph: `taken`, the operation
 * it computes it as (SDHIP_OP_MUL_MAT, CONV_2D, FLASH_ATTN_EXT, GROUP_NORM,
 * NORM), or SDHIP_OP_NONE; `count`, the nodes that computation stands for
 * (1 + the chain's and the gated GELU's nodes, the views between included);
 * `chain`, the nodes after it computed along with it (its redirect pointing
 * at a node's tensor); `gated_out`, GEGLU's output node when the gated GELU
 * is fused, else NULL.  The decisions of hooks.cc:100-147 -- match_chain,
 * redirect_apart and match_gated_gelu (fusion.cc:136-394), under the tuning's
 * fuse and fuse_residual -- made over sdhip_node.  SDHIP_UNSUPPORTED where the
 * node is not taken. */
typedef struct sdhip_node_plan {
    int32_t taken;
    int32_t count;
    sdhip_epilogue chain;
    const sdhip_node *gated_out;
} sdhip_node_plan;

sdhip_status sdhip_plan_nodes(const sdhip_node *const *nodes, int n_nodes, int index, sdhip_node_plan *plan);

/* Computes node `index` of the graph with the nodes its plan fuses, on the
 * device, and returns how many nodes that was; 0 when the node is not taken
 * (the caller computes it), -1 on an error (sdhip_last_error).  Replaces
 * sdasm_compute_nodes (sdasm.h:41-51, hooks.cc:100-164): as there, the memory
 * the node (and a redirect or gated output) writes is forgotten by the store
 * first, taken or not.  `work` is the caller's buffer, of at least
 * sdhip_node_work_size bytes. */
int sdhip_compute_nodes(const sdhip_node *const *nodes, int n_nodes, int index, void *work, size_t work_size,
                        void *stream);

/* Sets *size to the work buffer node needs and returns 1, or returns 0 when
 * the node is not taken.  Replaces sdasm_work_size (sdasm.h:53-56,
 * hooks.cc:174-196). */
int sdhip_node_work_size(const sdhip_node *node, size_t *size);

/* ToDo's step for a grid of width x height tokens: the tuning's todo where it
 * is 2 or more and the grid has todo_tokens tokens or more, else 1.  Replaces
 * sdasm_token_downsampling (sdasm.h:61-67, hooks.cc:166-172), which
 * stable-diffusion.cpp calls to thin its self-attention's keys and values. */
int sdhip_token_downsampling(int64_t width, int64_t height);

#ifdef __cplusplus
}
#endif

#endif
