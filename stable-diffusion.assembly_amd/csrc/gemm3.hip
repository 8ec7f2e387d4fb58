// Winograd's batched products with wide wave tiles: C[b][m][n] = sum_k
// A[b][m][k] B[b][n][k], both operands two FP16 planes, hi and lo, held in
// blocks of 32 of K ([k / 32][row][k % 32]: a row's 32 halves are 64
// contiguous bytes), three MFMAs a product (a_hi b_hi + a_lo b_hi +
// a_hi b_lo) of v_mfma_f32_16x16x32_f16.
//
// Shape.  A workgroup's 4 waves stand along M: wave w computes rows
// 16 WM (4 m + w) .. + 16 WM of C by the workgroup's 16 WN columns, WM x WN
// tiles of 16 x 16, each K-step of 32 one MFMA deep.  A wave's rows of A are
// its own, so they go from memory straight into its registers (lane l takes
// row l % 16 and the 16 bytes (l / 16) of the row's 64: one load of a tile's
// 1 KB, in the MFMA's operand order); the columns of B are every wave's, so
// each wave loads a quarter of a step's B and writes it to LDS, where all
// four read it.  Per K-step a wave reads (WM + WN) 2 KB for 3 WM WN MFMAs:
// at WM = WN = 5, 20 KB for 75 MFMAs, against 8 KB for 24 in a 2 x 2
// workgroup of 32 x 32 wave tiles, so that neither the LDS nor the caches
// bound the MFMAs.
//
// Pipeline.  Every load goes into registers S steps ahead of its MFMAs (S
// register stages), and B's from its stage into one of two LDS buffers one
// step ahead.  Step s: the MFMAs of s (B from buffer s % 2), B of s + 1 into
// the other buffer, the loads of s + S into the stage s freed, then the
// workgroup's barrier -- a bare s_barrier after the wave's LDS writes are
// done, not __syncthreads, which would also wait for every load in flight
// and so empty the pipeline at every step.  Every load is unconditional:
// rows past M or N read the last row (their products are never stored),
// steps past the last repeat it, so that the compiler's counts of the loads
// in flight are the same on every path.
//
// LDS layout of a buffer: per plane, the block's 16 WN rows of 64 bytes, the
// 16-byte piece p of row r at piece p ^ s(r), s(r) = ((r >> 1) ^ (r >> 2)) & 3,
// so that the rows a read of 16 rows takes spread over every bank whether
// the LDS serves 8 or 16 lanes of a 16-byte read at a time.  s(16 j + r) =
// s(r), so a lane reads every tile of a buffer at one address plus 1 KB steps.

#include "device.h"
#include "kernels.h"
#include "profile.h"

namespace sdhip {

namespace {

constexpr int kRowBytes = 64;  // a row's 32 halves of one plane and K-step

__device__ __forceinline__ int swizzle(int row) { return ((row >> 1) ^ (row >> 2)) & 3; }

// Copies of a stage: 2 planes x WN tiles of 16 rows, 1 KB each, shared out
// over the 4 waves; waves with fewer repeat their last, so that each issues
// kCopies.
template <int WN>
constexpr int kCopies = (2 * WN + 3) / 4;

template <int WM, int WN, int S>
__global__ __launch_bounds__(256) void split_batched3_kernel(SplitBatchedArgs p) {
    constexpr int BN = 16 * WN;
    constexpr int kPlane = BN * kRowBytes;
    constexpr int kBuf = 2 * kPlane;
    constexpr int C = kCopies<WN>;
    __shared__ __attribute__((aligned(1024))) char lds[2 * kBuf];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15;
    const int piece = lane >> 4;

    const int64_t per_batch = p.m_blocks * p.n_blocks;
    const uint32_t bid = xcd_swizzle(blockIdx.x, gridDim.x);
    const int64_t batch = bid / per_batch;
    const int64_t rem = bid - batch * per_batch;
    const int64_t mb = rem / p.n_blocks;
    const int64_t nb = rem - mb * p.n_blocks;
    const int64_t m0 = (4 * mb + wave) * 16 * WM;
    const int64_t n0 = nb * BN;

    const _Float16 *A = p.a + batch * p.a_batch;
    const _Float16 *B = p.b + batch * p.b_batch;
    const int64_t a_step = p.M * 32, b_step = p.N * 32;

    // The lane's element offset in a step of A, per tile (row clamped).
    int64_t aoff[WM];
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        const int64_t row = m0 + 16 * i + r16;
        aoff[i] = (row < p.M ? row : p.M - 1) * 32 + 8 * piece;
    }
    // The lane's share of B: load q of this wave is the workgroup's piece
    // g = wave + 4 q (plane g / WN, tile g % WN) of 1 KB; the lane's 16 bytes
    // land at row lane / 4, piece lane % 4 of it in LDS, from the global
    // piece the swizzle puts there.
    int64_t boff[C];
    int bdst[C];
#pragma unroll
    for (int q = 0; q < C; ++q) {
        int g = wave + 4 * q;
        g = g < 2 * WN ? g : 2 * WN - 1;
        const int plane = g / WN, tile = g % WN;
        const int row = 16 * tile + (lane >> 2);
        const int gp = (lane & 3) ^ swizzle(row);
        int64_t grow = n0 + row;
        grow = grow < p.N ? grow : p.N - 1;
        boff[q] = plane * p.b_plane + grow * 32 + 8 * gp;
        bdst[q] = plane * kPlane + 16 * tile * kRowBytes + 16 * lane;
    }

    const int64_t steps = p.K / 32;
    const int64_t last = steps - 1;
    half8 ah[S][WM], al[S][WM], bv[S][C];
    const auto load = [&](int stage, int64_t s) {
        const int64_t k = s < last ? s : last;
        const _Float16 *b = B + k * b_step;
#pragma unroll
        for (int q = 0; q < C; ++q) bv[stage][q] = *reinterpret_cast<const half8 *>(b + boff[q]);
        const _Float16 *a = A + k * a_step;
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            ah[stage][i] = *reinterpret_cast<const half8 *>(a + aoff[i]);
            al[stage][i] = *reinterpret_cast<const half8 *>(a + p.a_plane + aoff[i]);
        }
    };
    const auto store_b = [&](int stage, int buf) {
#pragma unroll
        for (int q = 0; q < C; ++q) *reinterpret_cast<half8 *>(lds + buf * kBuf + bdst[q]) = bv[stage][q];
    };

    float4v acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[i][j] = float4v{};

    // Where this lane reads B's tile 0 of a buffer's plane: row r16, piece
    // `piece` of the global row, at its swizzled place (tile j 1 KB on).
    const int bread = r16 * kRowBytes + ((piece ^ swizzle(r16)) << 4);
    const auto compute = [&](int stage, int buf) {
        const char *base = lds + buf * kBuf + bread;
        half8 bh[WN], bl[WN];
#pragma unroll
        for (int j = 0; j < WN; ++j) {
            bh[j] = *reinterpret_cast<const half8 *>(base + 1024 * j);
            bl[j] = *reinterpret_cast<const half8 *>(base + kPlane + 1024 * j);
        }
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[stage][i], bh[j], acc[i][j], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[stage][i], bh[j], acc[i][j], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[stage][i], bl[j], acc[i][j], 0, 0, 0);
    };
    // The wave's LDS writes done, then the workgroup's barrier; the memory
    // clobbers keep the compiler's LDS accesses on their side of it.
    const auto sync = [&]() {
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        barrier_only();
    };

#pragma unroll
    for (int q = 0; q < S; ++q) load(q, q);
    store_b(0, 0);
    sync();
    // At the top of step t: buffer t % 2 holds B of t, stage (t + q) % S the
    // loads of t + q (q = 0 .. S - 1).  Passes of U steps, U a multiple of
    // both S and 2, so that stages and buffers are the same at every pass;
    // one exit, at the top.
    constexpr int U = S % 2 == 0 ? S : 2 * S;
    for (int64_t s = 0; s < steps; s += U) {
#pragma unroll
        for (int q = 0; q < U; ++q) {
            if (s + q < steps) compute(q % S, q & 1);
            store_b((q + 1) % S, (q + 1) & 1);
            load(q % S, s + q + S);
            sync();
        }
    }

    // Both operands were scaled by 2^-4 in the split: the product by 2^-8.
    // Lane l holds rows 4 (l / 16) + e of column l % 16 of each tile.
    float *Cp = p.c + batch * p.c_batch;
#pragma unroll
    for (int j = 0; j < WN; ++j) {
        const int64_t n = n0 + 16 * j + r16;
        if (n >= p.N) continue;
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            const int64_t row0 = m0 + 16 * i + 4 * piece;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (row0 + e < p.M) Cp[(row0 + e) * p.N + n] = acc[i][j][e] * (kSplitUp * kSplitUp);
            }
        }
    }
}

template <int WM, int WN, int S>
hipError_t launch3(SplitBatchedArgs p, hipStream_t stream) {
    p.m_blocks = (p.M + 64 * WM - 1) / (64 * WM);
    p.n_blocks = (p.N + 16 * WN - 1) / (16 * WN);
    const dim3 grid(static_cast<uint32_t>(p.batches * p.m_blocks * p.n_blocks));
    SDHIP_LAUNCH((split_batched3_kernel<WM, WN, S>), grid, dim3(256), 0, stream, p);
    return hipGetLastError();
}

// The time of a launch in units of one tile-step, for a choice of wave tile:
// the rounds of workgroups the chip's 256 CUs take (one a CU), each a
// workgroup's tiles plus a fixed cost of a step.
double cost3(const SplitBatchedArgs &p, int wm, int wn) {
    const int64_t blocks = p.batches * ((p.M + 64 * wm - 1) / (64 * wm)) * ((p.N + 16 * wn - 1) / (16 * wn));
    const int64_t rounds = (blocks + 255) / 256;
    return static_cast<double>(rounds) * (wm * wn + 6);
}

}  // namespace

hipError_t launch_split_batched3(const SplitBatchedArgs &p, int tiles, int stages, hipStream_t stream) {
    if (!split_batched2_takes(p)) return hipErrorInvalidValue;
    const bool deep = stages == 4;
    int pick = tiles;
    if (pick == 0) {
        const int shapes[][2] = {{5, 5}, {4, 4}, {5, 2}, {4, 2}, {2, 2}, {2, 1}};
        double best = 0.0;
        for (const auto &sh : shapes) {
            const double c = cost3(p, sh[0], sh[1]);
            if (pick == 0 || c < best) {
                best = c;
                pick = 10 * sh[0] + sh[1];
            }
        }
    }
    switch (pick) {
    case 55:
        return deep ? launch3<5, 5, 4>(p, stream) : launch3<5, 5, 3>(p, stream);
    case 44:
        return deep ? launch3<4, 4, 4>(p, stream) : launch3<4, 4, 3>(p, stream);
    case 52:
        return deep ? launch3<5, 2, 4>(p, stream) : launch3<5, 2, 3>(p, stream);
    case 42:
        return deep ? launch3<4, 2, 4>(p, stream) : launch3<4, 2, 3>(p, stream);
    case 22:
        return deep ? launch3<2, 2, 4>(p, stream) : launch3<2, 2, 3>(p, stream);
    default:
        return deep ? launch3<2, 1, 4>(p, stream) : launch3<2, 1, 3>(p, stream);
    }
}

}  // namespace sdhip
