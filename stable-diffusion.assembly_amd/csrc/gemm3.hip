// Winograd's batched products, each wave's tiles on v_mfma_f32_32x32x16_f16:
// C[b][m][n] = sum_k A[b][m][k] B[b][n][k], both operands two FP16 planes,
// hi and lo, A held in blocks of 32 of K ([k / 32][row][k % 32]: a row's 32
// halves are 64 contiguous bytes) and B in runs of 8 ([k / 8][row][k % 8]:
// the 16 bytes of one run of consecutive rows are next to each other), three
// MFMAs a product (a_hi b_hi + a_lo b_hi + a_hi b_lo).
//
// Shape.  A workgroup's 4 waves stand along N: wave w computes the block's
// 32 TM rows of A (transformed weights, output channels) by its own 32 TN
// rows of B (transformed inputs, tiles).  The rows of A are every wave's, so
// each wave loads a quarter of a step's A into registers and writes it to
// LDS, where all four read it; a wave's rows of B are its own, so they go
// from memory straight into its registers in the MFMA's operand order (lane
// l takes row l % 32 and the run 2 h + l / 32 of the step's four, h the half
// of the step: each 32 lanes read 512 contiguous bytes).  Of the 16 x 16 x
// 32 MFMA, a wave sustains about half the rate with one wave a SIMD; of the
// 32 x 32 x 16, nearly all of it.
//
// Pipeline.  Every load goes into registers S steps ahead of its MFMAs (S
// register stages), and A's from its stage into one of two LDS buffers one
// step ahead.  Step s: the MFMAs of s (A from buffer s % 2), A of s + 1 into
// the other buffer, the loads of s + S into the stage s freed, then the
// workgroup's barrier -- a bare s_barrier after the wave's LDS writes are
// done, not __syncthreads, which would also wait for every load in flight.
// Every load is unconditional: rows past M or N read the last row (their
// products are never stored), steps past the last repeat it, so that the
// compiler's counts of the loads in flight are the same on every path.
//
// A32: A in single precision instead (the transformed weights kept in the
// store, [batch][row][K]), each column k times a_scale[k]: a wave loads its
// groups of 16 rows, a lane 8 consecutive columns of one row, scales and
// splits them on their way into LDS, as the register-staged core does
// (bit-identical parts).
//
// LDS layout of a buffer: per plane, the block's 32 TM rows of 64 bytes, the
// 16-byte piece p of row r at piece p ^ s(r), s(r) = ((r >> 1) ^ (r >> 2)) & 3,
// so that the 32 rows a fragment read takes spread over every bank whether
// the LDS serves 8 or 16 lanes of a 16-byte read at a time.

#include "device.h"
#include "kernels.h"
#include "profile.h"

namespace sdhip {

namespace {

constexpr int kRowBytes = 64;  // a row's 32 halves of one plane and K-step

__device__ __forceinline__ int swizzle(int row) { return ((row >> 1) ^ (row >> 2)) & 3; }

template <int TM, int TN, int S, bool A32>
__global__ __launch_bounds__(256) void split_batched3_kernel(SplitBatchedArgs p) {
    constexpr int kPlaneA = 32 * TM * kRowBytes;  // bytes of one plane of a step of A
    constexpr int kBuf = 2 * kPlaneA;
    // A wave's 1 KB pieces of A a step (A32: its groups of 16 rows, each both
    // planes' pieces).
    constexpr int CA = A32 ? TM / 2 : TM;
    static_assert(!A32 || TM % 2 == 0, "A32 takes blocks of 64 rows or more");
    __shared__ __attribute__((aligned(1024))) char lds[2 * kBuf];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r32 = lane & 31, half = lane >> 5;

    const int64_t per_batch = p.m_blocks * p.n_blocks;
    const uint32_t bid = xcd_swizzle(blockIdx.x, gridDim.x);
    const int64_t batch = bid / per_batch;
    const int64_t rem = bid - batch * per_batch;
    const int64_t mb = rem / p.n_blocks;
    const int64_t nb = rem - mb * p.n_blocks;
    const int64_t m0 = mb * 32 * TM;
    const int64_t n0 = (4 * nb + wave) * 32 * TN;

    const _Float16 *A = p.a + batch * p.a_batch;
    const float *A32p = p.a32 + batch * p.a_batch;
    const _Float16 *B = p.b + batch * p.b_batch;
    const int64_t a_step = A32 ? 32 : p.M * 32, b_step = p.N * 32;

    // A: piece g = wave + 4 q of the 4 TM pieces of a step (plane g / (2 TM),
    // rows 16 (g % (2 TM)) ..), the lane's row lane / 4 and 16 bytes lane % 4
    // of it, written to LDS at its swizzled place.
    int64_t aoff[CA];
    int adst[CA];
#pragma unroll
    for (int q = 0; q < CA; ++q) {
        const int g = wave + 4 * q;
        const int plane = A32 ? 0 : g / (2 * TM), u = A32 ? g : g % (2 * TM);
        const int row = 16 * u + (lane >> 2), pc = lane & 3;
        const int64_t grow = m0 + row < p.M ? m0 + row : p.M - 1;
        aoff[q] = A32 ? grow * p.K + 8 * pc : plane * p.a_plane + grow * 32 + 8 * pc;
        adst[q] = plane * kPlaneA + row * kRowBytes + ((pc ^ swizzle(row)) << 4);
    }
    const float *fcol = p.a_scale + 8 * (lane & 3);  // A32: the lane's columns' scales
    // B: the lane's row of each tile j (clamped) in its run of each half of
    // the step (runs half and 2 + half of the step's four, N rows of 8 apart).
    int64_t boff[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int64_t row = n0 + 32 * j + r32;
        boff[j] = (row < p.N ? row : p.N - 1) * 8 + half * p.N * 8;
    }
    const int64_t b_half = 2 * p.N * 8;

    const int64_t steps = p.K / 32;
    const int64_t last = steps - 1;
    half8 av[S][A32 ? 1 : CA];
    float4v aw[S][A32 ? CA : 1][2];  // A32: a lane's 8 numbers of each group
    float4v fw[S][2];                // A32: their columns' scales
    half8 bv[S][TN][2][2];  // [stage][tile][plane][half of k]
    const auto load = [&](int stage, int64_t s) {
        const int64_t k = s < last ? s : last;
        if constexpr (A32) {
            const float *a = A32p + k * a_step;
#pragma unroll
            for (int q = 0; q < CA; ++q) {
                aw[stage][q][0] = *reinterpret_cast<const float4v *>(a + aoff[q]);
                aw[stage][q][1] = *reinterpret_cast<const float4v *>(a + aoff[q] + 4);
            }
            fw[stage][0] = *reinterpret_cast<const float4v *>(fcol + k * 32);
            fw[stage][1] = *reinterpret_cast<const float4v *>(fcol + k * 32 + 4);
        } else {
            const _Float16 *a = A + k * a_step;
#pragma unroll
            for (int q = 0; q < CA; ++q) av[stage][q] = *reinterpret_cast<const half8 *>(a + aoff[q]);
        }
        const _Float16 *b = B + k * b_step;
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int pl = 0; pl < 2; ++pl)
#pragma unroll
                for (int hk = 0; hk < 2; ++hk)
                    bv[stage][j][pl][hk] = *reinterpret_cast<const half8 *>(b + pl * p.b_plane + boff[j] + hk * b_half);
    };
    const auto store_a = [&](int stage, int buf) {
        if constexpr (A32) {
#pragma unroll
            for (int q = 0; q < CA; ++q) {
                half8 h, l;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    _Float16 x, y;
                    split2(aw[stage][q][e >> 2][e & 3] * fw[stage][e >> 2][e & 3], x, y);
                    h[e] = x;
                    l[e] = y;
                }
                *reinterpret_cast<half8 *>(lds + buf * kBuf + adst[q]) = h;
                *reinterpret_cast<half8 *>(lds + buf * kBuf + kPlaneA + adst[q]) = l;
            }
        } else {
#pragma unroll
            for (int q = 0; q < CA; ++q) *reinterpret_cast<half8 *>(lds + buf * kBuf + adst[q]) = av[stage][q];
        }
    };

    float16v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = float16v{};

    // A's fragment of tile i and half hk of k: row 32 i + r32, piece 2 hk +
    // half, at its swizzled place.
    int aread[2];
#pragma unroll
    for (int hk = 0; hk < 2; ++hk) aread[hk] = r32 * kRowBytes + (((2 * hk + half) ^ swizzle(r32)) << 4);
    // Each step's MFMAs at raised wave priority (s_setprio), ahead of the
    // other workgroups' split and stores of A on the SIMD.
    const auto compute = [&](int stage, int buf) {
        __builtin_amdgcn_s_setprio(1);
        const char *base = lds + buf * kBuf;
#pragma unroll
        for (int hk = 0; hk < 2; ++hk) {
            half8 ah[TM], al[TM];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                ah[i] = *reinterpret_cast<const half8 *>(base + 32 * i * kRowBytes + aread[hk]);
                al[i] = *reinterpret_cast<const half8 *>(base + kPlaneA + 32 * i * kRowBytes + aread[hk]);
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const half8 bh = bv[stage][j][0][hk], bl = bv[stage][j][1][hk];
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bh, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], bh, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bl, acc[i][j], 0, 0, 0);
                }
        }
        __builtin_amdgcn_s_setprio(0);
    };

#pragma unroll
    for (int q = 0; q < S; ++q) load(q, q);
    store_a(0, 0);
    lds_barrier();
    // At the top of step t: buffer t % 2 holds A of t, stage (t + q) % S the
    // loads of t + q (q = 0 .. S - 1).  Passes of U steps, U a multiple of
    // both S and 2, so that stages and buffers are the same at every pass;
    // one exit, at the top.
    constexpr int U = S % 2 == 0 ? S : 2 * S;
    for (int64_t s = 0; s < steps; s += U) {
#pragma unroll
        for (int q = 0; q < U; ++q) {
            if (s + q < steps) compute(q % S, q & 1);
            store_a((q + 1) % S, (q + 1) & 1);
            load(q % S, s + q + S);
            lds_barrier();
        }
    }

    // Both operands were scaled by 2^-4 in the split: the product by 2^-8.
    float *Cp = p.c + batch * p.c_batch;
    const int64_t lane_row = 4 * half;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int64_t n = n0 + 32 * j + r32;
        if (n >= p.N) continue;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int64_t tile0 = m0 + 32 * i;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int64_t m = tile0 + lane_row + tile_row(e);
                if (m < p.M) Cp[m * p.N + n] = acc[i][j][e] * (kSplitUp * kSplitUp);
            }
        }
    }
}

template <int TM, int TN, int S>
hipError_t launch3(SplitBatchedArgs p, hipStream_t stream) {
    p.m_blocks = (p.M + 32 * TM - 1) / (32 * TM);
    p.n_blocks = (p.N + 128 * TN - 1) / (128 * TN);
    const dim3 grid(static_cast<uint32_t>(p.batches * p.m_blocks * p.n_blocks));
    if constexpr (TM % 2 == 0) {
        if (p.a32 != nullptr) {
            SDHIP_LAUNCH((split_batched3_kernel<TM, TN, S, true>), grid, dim3(256), 0, stream, p);
            return hipGetLastError();
        }
    }
    SDHIP_LAUNCH((split_batched3_kernel<TM, TN, S, false>), grid, dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace

bool split_batched3_takes(const SplitBatchedArgs &p) {
    const auto al16 = [](const void *q) { return (reinterpret_cast<uintptr_t>(q) % 16) == 0; };
    const bool b_ok = al16(p.b) && p.b_plane % 8 == 0 && p.b_batch % 8 == 0;
    const bool a_ok = p.a32 != nullptr ? al16(p.a32) && al16(p.a_scale) && p.a_batch % 4 == 0
                                       : al16(p.a) && p.a_plane % 8 == 0 && p.a_batch % 8 == 0;
    return a_ok && b_ok && p.K % 32 == 0 && p.K > 0 && p.M > 0 && p.N > 0;
}

hipError_t launch_split_batched3(const SplitBatchedArgs &p, int tiles, int stages, hipStream_t stream) {
    if (!split_batched3_takes(p)) return hipErrorInvalidValue;
    const bool deep = stages == 4;
    // A32 takes blocks of 64 rows or more: tiles=12 (32 rows) takes the default.
    if (p.a32 != nullptr && tiles == 12) tiles = 0;
    switch (tiles) {
    case 22:
        return deep ? launch3<2, 2, 4>(p, stream) : launch3<2, 2, 3>(p, stream);
    case 41:
        return deep ? launch3<4, 1, 4>(p, stream) : launch3<4, 1, 3>(p, stream);
    case 12:
        return deep ? launch3<1, 2, 4>(p, stream) : launch3<1, 2, 3>(p, stream);
    default:
        // 64 rows of A by 128 of B: the workgroups fill the chip at cfg2's
        // 320 x 512 and at the VAE's 512 x 1024, with no part of a block idle
        // where M is a multiple of 64.
        return deep ? launch3<2, 1, 4>(p, stream) : launch3<2, 1, 3>(p, stream);
    }
}

}  // namespace sdhip
