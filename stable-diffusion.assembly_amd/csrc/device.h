// Device-side pieces shared by every kernel of the library: vector types of
// the MFMA operands, the split of a single-precision number into two FP16
// parts, the element-wise chain an operation applies to its output while it
// is still in registers, and the single-precision functions the chain and the
// gated GELU compute with.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sdhip {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef int int4v __attribute__((ext_vector_type(4)));
typedef int int16v __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// ------------------------------------------------------------------ split

// The single-precision operand is scaled by 2^-4 before it is split, so that
// numbers up to 65504 * 16 ~ 1.05e6 stay finite in FP16, and the product is
// scaled back by 2^4 (both exact).  x * 2^-4 = hi + lo + r with hi =
// fp16(x * 2^-4), lo = fp16(x * 2^-4 - hi) (the difference is exact in single
// precision) and |r| <= 2^-22 |x * 2^-4| while lo is normal, 2^-25 once it is
// subnormal: 22 bits of x, against 11 in ggml's own rounding of x to FP16.
// FP16 weights are exact in FP16, so w * x = w hi + w lo + w r, and the two
// products are exact in the MFMA's single-precision sums.
constexpr float kSplitDown = 0.0625f;
constexpr float kSplitUp = 16.0f;

// The two parts of s, a number already scaled by 2^-4 (with whatever other
// power of two a caller folds into the same factor).
__device__ __forceinline__ void split_scaled(float s, _Float16 &hi, _Float16 &lo) {
    hi = static_cast<_Float16>(s);
    lo = static_cast<_Float16>(s - static_cast<float>(hi));
}

__device__ __forceinline__ void split2(float x, _Float16 &hi, _Float16 &lo) { split_scaled(x * kSplitDown, hi, lo); }

// x rounded to bfloat16, to nearest with ties to even, and widened back: the
// product of two such numbers is exact in single precision.
__device__ __forceinline__ float bf16_round(float x) { return static_cast<float>(static_cast<__bf16>(x)); }

// x as a product of 16 bits takes it: rounded to bfloat16 where bf says so.
__device__ __forceinline__ float bf16_operand(float x, int32_t bf) { return bf ? bf16_round(x) : x; }

// ------------------------------------------------------------------ scalar math

// exp(x) by Cephes' expf method, as the reference's exponential()
// (sources/scalar_math.h:34-51) computes it, so that the chain's SiLU and the
// gated GELU round as the reference's do: x clamped to [-87.3, 88.73], n =
// round(x / ln 2) by the sum with 1.5 * 2^23, r = x - n ln 2 in two steps,
// exp(r) by Cephes' minimax polynomial, 2^n built in the exponent field.
__device__ __forceinline__ float cephes_exp(float x) {
    x = fminf(fmaxf(x, -87.3f), 88.73f);
    const float magic = 12582912.0f;  // 1.5 * 2^23
    const float z = __builtin_fmaf(x, 1.44269504088896341f, magic);
    const float n = z - magic;
    float r = __builtin_fmaf(n, -0.693359375f, x);
    r = __builtin_fmaf(n, 2.12194440e-4f, r);
    float p = 1.9875691500e-4f;
    p = __builtin_fmaf(p, r, 1.3981999507e-3f);
    p = __builtin_fmaf(p, r, 8.3334519073e-3f);
    p = __builtin_fmaf(p, r, 4.1665795894e-2f);
    p = __builtin_fmaf(p, r, 1.6666665459e-1f);
    p = __builtin_fmaf(p, r, 5.0000001201e-1f);
    p = __builtin_fmaf(p * r, r, r) + 1.0f;
    const uint32_t e = static_cast<uint32_t>(__float_as_int(z) - 0x4b400000 + 127) << 23;
    return p * __uint_as_float(e);
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + cephes_exp(-x)); }

// GELU by its tanh form, 0.5 x (1 + tanh(y)) = x / (1 + exp(-2y)),
// y = sqrt(2/pi) (x + 0.044715 x^3) (scalar_math.h:58-63).
__device__ __forceinline__ float gelu(float x) {
    const float y = x * __builtin_fmaf(0.044715f * x, x, 1.0f);
    return x / (1.0f + cephes_exp(-1.5957691216057308f * y));
}

// ------------------------------------------------------------------ chain

enum StepKind : int32_t { kAdd = 0, kMul = 1, kSilu = 2 };

struct DevStep {
    int32_t kind;
    // flat01: nb[1] = ne[0] nb[0], so i0 nb[0] + i1 nb[1] = (i1 ne0 + i0) nb[0];
    // flat123: nb[2] = ne[1] nb[1] and nb[3] = ne[2] nb[2], so that
    // i1 nb[1] + i2 nb[2] + i3 nb[3] = (row of the output) nb[1].  Either lets
    // an epilogue index the operand without dividing.
    int32_t flat01, flat123;
    const float *operand;
    int64_t nb[4];  // elements; 0 along a broadcast dimension
};

constexpr int kMaxSteps = 6;

struct DevChain {
    int32_t count;
    DevStep steps[kMaxSteps];
};

// The chain (fusion.cc:77-99) applied to E values at once, in the order of
// the graph and in single precision (no contraction of an addition into a
// multiplication before it), step after step: the operands of a step are all
// loaded before any is used and nothing is stored meanwhile, so that the
// loads go out together rather than one round trip per element.  off(s, e)
// gives the offset of element e in the operand of step s.
template <int E, class Off>
__device__ __forceinline__ void apply_chain_block(const DevChain &c, float (&v)[E], Off off) {
#pragma unroll 1
    for (int s = 0; s < c.count; ++s) {
        const DevStep &st = c.steps[s];
        if (st.kind == 2) {
#pragma unroll
            for (int e = 0; e < E; ++e) v[e] = silu(v[e]);
            continue;
        }
        float o[E];
#pragma unroll
        for (int e = 0; e < E; ++e) o[e] = st.operand[off(s, e)];
        if (st.kind == 0) {
#pragma unroll
            for (int e = 0; e < E; ++e) v[e] = __fadd_rn(v[e], o[e]);
        } else {
#pragma unroll
            for (int e = 0; e < E; ++e) v[e] = __fmul_rn(v[e], o[e]);
        }
    }
}

// x, which the compiler may not see through: what is computed from it is
// computed where it is used, not hoisted out of loops into registers held for
// their whole length.
template <class T>
__device__ __forceinline__ T opaque(T x) {
    asm volatile("" : "+v"(x));
    return x;
}

// The row, within a 32 x 32 MFMA result tile, of register e (of 16) of a lane
// of the first half of the wave; the second half's are 4 further down.
__device__ __forceinline__ constexpr int tile_row(int e) { return 8 * (e >> 2) + (e & 3); }

// The chain over the 16 values a lane holds of a 32 x 32 MFMA result tile,
// one column of it.  Where the tile lies wholly inside the output (`full`) and
// a step's operand is strided along the tile's rows (stride(s) >= 0), its
// values are at base(s) + tile_row(e) * stride(s) -- one broadcast load when
// the stride is 0; elsewhere (the edges, operands broadcast over only some of
// the row's dimensions) general(s, e) gives each offset.  The operands of a
// step are all loaded before any is used.
template <class Base, class Stride, class General>
__device__ __forceinline__ void apply_chain_tile(const DevChain &c, float (&v)[16], bool full, Base base,
                                                 Stride stride, General general) {
#pragma unroll 1
    for (int s = 0; s < c.count; ++s) {
        const DevStep &st = c.steps[s];
        if (st.kind == 2) {
#pragma unroll
            for (int e = 0; e < 16; ++e) v[e] = silu(v[e]);
            continue;
        }
        float o[16];
        const int64_t rs = stride(s);
        if (full && rs == 0) {
            const float b = st.operand[base(s)];
#pragma unroll
            for (int e = 0; e < 16; ++e) o[e] = b;
        } else if (full && rs > 0) {
            const float *p = st.operand + base(s);
#pragma unroll
            for (int e = 0; e < 16; ++e) o[e] = p[tile_row(e) * rs];
        } else {
            // Four at a time, so that the offsets of all sixteen are not held
            // at once: this path's registers count for the whole kernel.
#pragma unroll
            for (int g = 0; g < 16; g += 4) {
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int e = g; e < g + 4; ++e) o[e] = st.operand[general(s, e)];
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (st.kind == 0) {
#pragma unroll
            for (int e = 0; e < 16; ++e) v[e] = __fadd_rn(v[e], o[e]);
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) v[e] = __fmul_rn(v[e], o[e]);
        }
    }
}

// Row r of an output of ne1 rows and ne2 matrices as (i1, i2, i3), in 32-bit
// unsigned division (the host keeps every extent below 2^31): 64-bit division
// is a long software sequence on the GPU.
__device__ __forceinline__ void split_index(uint32_t r, uint32_t ne1, uint32_t ne2, uint32_t &i1, uint32_t &i2,
                                            uint32_t &i3) {
    const uint32_t q = r / ne1;
    i1 = r - q * ne1;
    i3 = q / ne2;
    i2 = q - i3 * ne2;
}

// ------------------------------------------------------------------ copies into LDS

// Waits until at most N of the wave's vector memory loads are in flight
// (s_waitcnt vmcnt(N), the other counters left alone).
template <int N>
__device__ __forceinline__ void wait_loads() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// The workgroup's barrier alone, with no wait for the loads in flight (which
// __syncthreads drains): what a wave must have in LDS before it, it waits for
// itself (wait_loads).  The memory clobber keeps the compiler from moving
// loads or stores across it.
__device__ __forceinline__ void barrier_only() { asm volatile("s_barrier" ::: "memory"); }

// The wave's own LDS accesses done (lgkmcnt(0), nothing else waited for),
// then the workgroup's barrier: what __syncthreads gives the LDS without its
// wait for every global load in flight.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xC07F);
    barrier_only();
}

// One 16-byte piece a lane of a 1 KB copy from global memory into LDS; the
// LDS address is the wave's (lane l's piece lands 16 l bytes past it).
__device__ __forceinline__ void copy_lds(const void *src, char *lds) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds, 16, 0, 0);
}

// The same with 4 bytes a lane: a copy of 256 bytes.
__device__ __forceinline__ void copy_lds4(const void *src, char *lds) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds, 4, 0, 0);
}

// copy_lds through a buffer resource: the piece at rsrc's base + voffset +
// soffset, the lane's constant offset in a vector register and the rest in a
// scalar one, so that a copy takes no vector instruction for its address.
__device__ __forceinline__ void copy_lds_buffer(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset, uint32_t soffset,
                                                char *lds) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)lds, 16, voffset,
                                             soffset, 0, 0);
}

// ------------------------------------------------------------------ grid

// The 8 XCDs of an MI355X each take every 8th workgroup of a launch, and each
// has its own L2.  A launch whose neighbouring blocks share an operand panel
// maps hardware block b to logical block so that the blocks of one XCD are
// consecutive logical blocks.  Blocks past the last multiple of 8 keep their
// number.
__device__ __forceinline__ uint32_t xcd_swizzle(uint32_t b, uint32_t nblocks) {
    const uint32_t whole = nblocks / 8u * 8u;
    if (b >= whole) {
        return b;
    }
    return (b % 8u) * (whole / 8u) + b / 8u;
}

}  // namespace sdhip
