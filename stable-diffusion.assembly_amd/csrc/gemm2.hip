// Products of operands already split into FP16 planes, with the copies into
// LDS made by the memory system itself (global_load_lds): Winograd's batched
// products C[b][m][n] = sum_k A[b][m][k] B[b][n][k], both operands held in
// blocks of 32 of K as two planes, hi and lo ([k / 32][row][k % 32]), three
// MFMAs a product (a_hi b_hi + a_hi b_lo + a_lo b_hi).
//
// Shape.  A block of 4 waves (2 x 2) computes 64 WM x 64 WN of C, each wave
// 32 WM x 32 WN as WM x WN tiles of v_mfma_f32_32x32x16_f16.  K goes in steps
// of 32 through a ring of NS stages of LDS: each wave copies its share of a
// step's rows (1 KB an instruction, 16 rows of 64 bytes) NS - 1 steps ahead of
// the MFMAs, with no register staging -- the loads are in flight for NS - 1
// steps of MFMAs.  The 16-byte pieces of a row are stored XOR-swizzled by the
// row's quad (piece ^ ((row >> 2) & 3)) so that the 32 rows a fragment read
// takes fall in distinct banks: the copy picks which global piece each lane
// brings so that the swizzled layout lands where the reads expect it.
//
// Every copy is unconditional: rows past the operand's last read its last row
// (their products are never stored), and past the last step the copies repeat
// it into a stage no wave reads again, so that each wave has the same count of
// loads in flight at every wait.

#include "device.h"
#include "kernels.h"
#include "profile.h"

namespace sdhip {

namespace {

constexpr int kStep = 32;         // K a stage
constexpr int kRowBytes = 64;     // one plane's 32 halves of a row
constexpr int kCopyRows = 16;     // rows of one 1 KB copy instruction

// The LDS byte offset of piece `piece` (0..3, 8 halves each) of row `row` in
// a plane of a stage.
__device__ __forceinline__ int swz(int row, int piece) { return row * kRowBytes + ((piece ^ ((row >> 2) & 3)) << 4); }

// Copies one plane's rows [r0, r0 + ROWS) of a K-step into LDS: the wave's
// share, ROWS / 16 / 4 instructions, each of 16 rows.  `src` is the plane's
// first row at this step, rows kStep halves apart; rows at or past `rows`
// read the last row.
template <int ROWS>
__device__ __forceinline__ void copy_plane(const _Float16 *src, int64_t rows, int64_t r0, char *lds, int wave,
                                           int lane) {
    static_assert(ROWS % (4 * kCopyRows) == 0, "rows a multiple of 64");
    const int rq = lane >> 2;                // row within the copy
    const int piece = lane & 3;              // the LDS piece the lane fills
#pragma unroll
    for (int i = 0; i < ROWS / (4 * kCopyRows); ++i) {
        const int group = wave + 4 * i;      // which 16 rows
        const int row = group * kCopyRows + rq;
        const int gp = piece ^ ((row >> 2) & 3);  // the global piece that lands in `piece`
        int64_t r = r0 + row;
        r = r < rows ? r : rows - 1;
        copy_lds(src + r * kStep + gp * 8, lds + group * (kCopyRows * kRowBytes));
    }
}

template <int WM, int WN, int NS>
__global__ __launch_bounds__(256) void split_batched2_kernel(SplitBatchedArgs p) {
    constexpr int BM = 64 * WM;
    constexpr int BN = 64 * WN;
    constexpr int kPlaneA = BM * kRowBytes, kPlaneB = BN * kRowBytes;
    constexpr int kStage = 2 * kPlaneA + 2 * kPlaneB;
    constexpr int kCopies = 2 * (BM + BN) / (4 * kCopyRows);  // copy instructions of a wave a step
    __shared__ __attribute__((aligned(1024))) char lds[NS * kStage];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = wave >> 1, wc = wave & 1;

    const int64_t per_batch = p.m_blocks * p.n_blocks;
    const uint32_t bid = xcd_swizzle(blockIdx.x, gridDim.x);
    const int64_t batch = bid / per_batch;
    const int64_t rem = bid - batch * per_batch;
    const int64_t mb = rem / p.n_blocks;
    const int64_t nb = rem - mb * p.n_blocks;
    const int64_t m0 = mb * BM, n0 = nb * BN;
    const _Float16 *A = p.a + batch * p.a_batch;
    const _Float16 *B = p.b + batch * p.b_batch;
    float *C = p.c + batch * p.c_batch;
    const int64_t steps = p.K / kStep;

    // A step's four planes into stage `st`.
    const auto copy_step = [&](int64_t s, int st) {
        char *base = lds + st * kStage;
        const _Float16 *a = A + s * p.M * kStep;
        const _Float16 *b = B + s * p.N * kStep;
        copy_plane<BM>(a + m0 * kStep, p.M - m0, 0, base, wave, lane);
        copy_plane<BM>(a + p.a_plane + m0 * kStep, p.M - m0, 0, base + kPlaneA, wave, lane);
        copy_plane<BN>(b + n0 * kStep, p.N - n0, 0, base + 2 * kPlaneA, wave, lane);
        copy_plane<BN>(b + p.b_plane + n0 * kStep, p.N - n0, 0, base + 2 * kPlaneA + kPlaneB, wave, lane);
    };

    float16v acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[i][j] = float16v{};

    const int r = lane & 31;
    const int half = lane >> 5;
    const int64_t last = steps - 1;
#pragma unroll
    for (int s = 0; s < NS - 1; ++s) copy_step(s < last ? s : last, s);

    for (int64_t s = 0; s < steps; ++s) {
        // This wave's copies of step s are in (those of the NS - 2 steps
        // after it may still be in flight), and every wave's, past the
        // barrier -- which also means every wave is done with the stage the
        // next copies overwrite, read at step s - 1.
        wait_loads<(NS - 2) * kCopies>();
        barrier_only();
        const int64_t ahead = s + NS - 1;
        copy_step(ahead < last ? ahead : last, static_cast<int>(ahead % NS));
        const char *base = lds + static_cast<int>(s % NS) * kStage;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int piece = 2 * ks + half;
            half8 ah[WM], al[WM], bh[WN], bl[WN];
#pragma unroll
            for (int i = 0; i < WM; ++i) {
                const int row = wr * 32 * WM + 32 * i + r;
                ah[i] = *reinterpret_cast<const half8 *>(base + swz(row, piece));
                al[i] = *reinterpret_cast<const half8 *>(base + kPlaneA + swz(row, piece));
            }
#pragma unroll
            for (int j = 0; j < WN; ++j) {
                const int row = wc * 32 * WN + 32 * j + r;
                bh[j] = *reinterpret_cast<const half8 *>(base + 2 * kPlaneA + swz(row, piece));
                bl[j] = *reinterpret_cast<const half8 *>(base + 2 * kPlaneA + kPlaneB + swz(row, piece));
            }
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j) {
                    // In the register-staged core's order (a_hi b_hi, a_lo b_hi,
                    // a_hi b_lo), so that both give the same bits.
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bh[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], bh[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bl[j], acc[i][j], 0, 0, 0);
                }
        }
    }
    // No copy may still be landing in LDS when the block ends.
    wait_loads<0>();

    // Both operands were scaled by 2^-4 in the split: the product by 2^-8.
    const int64_t lane_row = 4 * half;
#pragma unroll
    for (int j = 0; j < WN; ++j) {
        const int64_t n = n0 + wc * 32 * WN + 32 * j + r;
        if (n >= p.N) continue;
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            const int64_t tile0 = m0 + wr * 32 * WM + 32 * i;
            const bool full = tile0 + 32 <= p.M;
            float *out = C + (tile0 + lane_row) * p.N + n;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                if (full || tile0 + lane_row + tile_row(e) < p.M) {
                    out[tile_row(e) * p.N] = acc[i][j][e] * (kSplitUp * kSplitUp);
                }
            }
        }
    }
}

template <int WM, int WN, int NS>
hipError_t launch2(SplitBatchedArgs p, hipStream_t stream) {
    p.m_blocks = (p.M + 64 * WM - 1) / (64 * WM);
    p.n_blocks = (p.N + 64 * WN - 1) / (64 * WN);
    const dim3 grid(static_cast<uint32_t>(p.batches * p.m_blocks * p.n_blocks));
    SDHIP_LAUNCH((split_batched2_kernel<WM, WN, NS>), grid, dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace

bool split_batched2_takes(const SplitBatchedArgs &p) {
    const bool aligned = (reinterpret_cast<uintptr_t>(p.a) % 16) == 0 && (reinterpret_cast<uintptr_t>(p.b) % 16) == 0 &&
                         p.a_plane % 8 == 0 && p.a_batch % 8 == 0 && p.b_plane % 8 == 0 && p.b_batch % 8 == 0;
    return p.a32 == nullptr && aligned && p.K % kStep == 0 && p.K > 0 && p.M > 0 && p.N > 0;
}

hipError_t launch_split_batched2(const SplitBatchedArgs &p, int tiles, int stages, hipStream_t stream) {
    if (!split_batched2_takes(p)) return hipErrorInvalidValue;
    const bool deep = stages == 4;
    switch (tiles) {
    case 11:
        return deep ? launch2<1, 1, 8>(p, stream) : launch2<1, 1, 4>(p, stream);
    case 12:
        return deep ? launch2<1, 2, 6>(p, stream) : launch2<1, 2, 4>(p, stream);
    case 21:
        return deep ? launch2<2, 1, 6>(p, stream) : launch2<2, 1, 4>(p, stream);
    case 22:
        return deep ? launch2<2, 2, 4>(p, stream) : launch2<2, 2, 3>(p, stream);
    default: {
        // The largest blocks that leave no part of the last block along M
        // idle and still give the chip two blocks a CU.
        const auto blocks = [&](int wm, int wn) {
            return p.batches * ((p.M + 64 * wm - 1) / (64 * wm)) * ((p.N + 64 * wn - 1) / (64 * wn));
        };
        const bool rows128 = p.M % 128 == 0 || p.M % 128 > 64;
        if (rows128 && blocks(2, 2) >= 512) return launch2<2, 2, 3>(p, stream);
        if (blocks(1, 2) >= 512) return launch2<1, 2, 4>(p, stream);
        return launch2<1, 1, 4>(p, stream);
    }
    }
}

}  // namespace sdhip
