// Winograd's minimal filtering F(m x m, 3x3) (Lavin and Gray, 2016), as the
// reference computes 3x3 convolutions at stride 1 (winograd.cc):
//
//     Y = A^T [ sum over ic of (G g G^T) (.) (B^T d B) ] A
//
// F(2x2, 3x3) with the matrices of winograd.cc:19-22 and F(4x4, 3x3) with the
// points 0, 1, -1, 2, -1/2, infinity of winograd.cc:1146-1183, 1259-1264.
//
// On the device, in four launches:
//   1. the weights, U[xi][oc][ic] = (G g G^T)[xi], single precision;
//   2. the inputs,  V[xi][ic][tile] = (B^T d B)[xi], one thread per (tile, ic);
//   3. the alpha^2 products M[xi] = U[xi] V[xi] on the single-precision MFMA
//      (v_mfma_f32_16x16x4_f32), so that the sums are as exact as the
//      reference's single-precision ones and the transforms' rounding is all
//      that Winograd adds -- FP16 parts would not hold the transformed
//      numbers (1/3, 1/15 of F(4x4)'s G) exactly;
//   4. the outputs, A^T M A, with the sum begun from the residual when the
//      chain says so and the chain after, one thread per (oc, tile).

#include "host.h"
#include "profile.h"
#include "winograd.h"

namespace sdhip {

namespace {

// ------------------------------------------------------------------ matrices

__constant__ float kBT2[4][4] = {{1, 0, -1, 0}, {0, 1, 1, 0}, {0, -1, 1, 0}, {0, 1, 0, -1}};
__constant__ float kG2[4][3] = {{1, 0, 0}, {0.5f, 0.5f, 0.5f}, {0.5f, -0.5f, 0.5f}, {0, 0, 1}};
__constant__ float kAT2[2][4] = {{1, 1, 1, 0}, {0, 1, -1, -1}};

__constant__ float kBT4[6][6] = {{1.0f, 1.5f, -2.0f, -1.5f, 1.0f, 0.0f},  {0.0f, -1.0f, -2.5f, -0.5f, 1.0f, 0.0f},
                                 {0.0f, 1.0f, 0.5f, -2.5f, 1.0f, 0.0f},   {0.0f, -0.5f, -1.0f, 0.5f, 1.0f, 0.0f},
                                 {0.0f, 2.0f, -1.0f, -2.0f, 1.0f, 0.0f},  {0.0f, 1.0f, 1.5f, -2.0f, -1.5f, 1.0f}};
__constant__ float kG4[6][3] = {{1.0f, 0.0f, 0.0f},
                                {-1.0f / 3, -1.0f / 3, -1.0f / 3},
                                {1.0f / 3, -1.0f / 3, 1.0f / 3},
                                {1.0f / 15, 2.0f / 15, 4.0f / 15},
                                {-16.0f / 15, 8.0f / 15, -4.0f / 15},
                                {0.0f, 0.0f, 1.0f}};
__constant__ float kAT4[4][6] = {{1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 0.0f},
                                 {0.0f, 1.0f, -1.0f, 2.0f, -0.5f, 0.0f},
                                 {0.0f, 1.0f, 1.0f, 4.0f, 0.25f, 0.0f},
                                 {0.0f, 1.0f, -1.0f, 8.0f, -0.125f, 1.0f}};

template <int M>
struct Mat;
template <>
struct Mat<2> {
    static constexpr int A = 4;
    __device__ static float bt(int i, int j) { return kBT2[i][j]; }
    __device__ static float g(int i, int j) { return kG2[i][j]; }
    __device__ static float at(int i, int j) { return kAT2[i][j]; }
};
template <>
struct Mat<4> {
    static constexpr int A = 6;
    __device__ static float bt(int i, int j) { return kBT4[i][j]; }
    __device__ static float g(int i, int j) { return kG4[i][j]; }
    __device__ static float at(int i, int j) { return kAT4[i][j]; }
};

// ------------------------------------------------------------------ 1. weights

// U[xi][oc][ic] = (G g G^T)[xi]: G g a column at a time, then (G g) G^T a row
// at a time (winograd.cc:1281-1300), one thread per (oc, ic).
template <int M>
__global__ __launch_bounds__(256) void weights_kernel(const _Float16 *__restrict__ w, float *__restrict__ u, int64_t oc,
                                                      int64_t ic) {
    constexpr int A = Mat<M>::A;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (t >= oc * ic) return;
    float g[3][3];
#pragma unroll
    for (int i = 0; i < 9; ++i) g[i / 3][i % 3] = static_cast<float>(w[t * 9 + i]);
    float gg[A][3];
#pragma unroll
    for (int i = 0; i < A; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j)
            gg[i][j] = Mat<M>::g(i, 0) * g[0][j] + Mat<M>::g(i, 1) * g[1][j] + Mat<M>::g(i, 2) * g[2][j];
    const int64_t plane = oc * ic;
#pragma unroll
    for (int i = 0; i < A; ++i)
#pragma unroll
        for (int j = 0; j < A; ++j)
            u[(i * A + j) * plane + t] =
                gg[i][0] * Mat<M>::g(j, 0) + gg[i][1] * Mat<M>::g(j, 1) + gg[i][2] * Mat<M>::g(j, 2);
}

// ------------------------------------------------------------------ 2. inputs

// V[xi][ic][tile] = (B^T d B)[xi] of the alpha x alpha inputs of the tile,
// zeros outside the image: B^T d (a row r of B^T takes its combination of the
// rows of d), then each of those times B.  One thread per (tile, ic),
// consecutive threads consecutive tiles.
template <int M>
__global__ __launch_bounds__(256) void inputs_kernel(WinogradArgs a, float *__restrict__ v) {
    constexpr int A = Mat<M>::A;
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;
    if (t >= static_cast<uint32_t>(a.tiles * a.ic)) return;
    const uint32_t c = t / static_cast<uint32_t>(a.tiles);
    const uint32_t tile = t - c * static_cast<uint32_t>(a.tiles);
    uint32_t tx, ty, n;
    split_index(tile, static_cast<uint32_t>(a.tw), static_cast<uint32_t>(a.th), tx, ty, n);
    const int64_t y0 = static_cast<int64_t>(ty) * M - a.p1;
    const int64_t x0 = static_cast<int64_t>(tx) * M - a.p0;
    const float *plane = a.x + static_cast<int64_t>(n) * a.xnb3 + static_cast<int64_t>(c) * a.xnb2;
    float d[A][A];
#pragma unroll
    for (int i = 0; i < A; ++i) {
        const int64_t yy = y0 + i;
        const bool row_in = yy >= 0 && yy < a.ih;
#pragma unroll
        for (int j = 0; j < A; ++j) {
            const int64_t xx = x0 + j;
            d[i][j] = (row_in && xx >= 0 && xx < a.iw) ? plane[yy * a.xnb1 + xx] : 0.0f;
        }
    }
    float bd[A][A];
#pragma unroll
    for (int r = 0; r < A; ++r)
#pragma unroll
        for (int j = 0; j < A; ++j) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < A; ++i) s += Mat<M>::bt(r, i) * d[i][j];
            bd[r][j] = s;
        }
    const int64_t plane_v = a.ic * a.tiles;
#pragma unroll
    for (int r = 0; r < A; ++r)
#pragma unroll
        for (int s = 0; s < A; ++s) {
            float x = 0.0f;
#pragma unroll
            for (int j = 0; j < A; ++j) x += bd[r][j] * Mat<M>::bt(s, j);
            v[(r * A + s) * plane_v + static_cast<int64_t>(c) * a.tiles + tile] = x;
        }
}

// ------------------------------------------------------------------ 3. products

// C[b][m][n] = sum_k A[b][m][k] B[b][k][n] for the alpha^2 batches b, A rows
// K-contiguous (U: [oc][ic]), B rows N-contiguous (V: [ic][tile]), on
// v_mfma_f32_16x16x4_f32.  A block of 64 x 128 by 4 waves of 32 x 64 (2 x 4
// tiles of 16 x 16), K in steps of 16 through LDS, double-buffered; LDS holds
// both operands k-major, [k][row] and [k][col], padded so that the four k-rows
// a wave reads at once fall in four distinct sets of banks.
constexpr int kGBM = 64, kGBN = 128, kGBK = 16;
constexpr int kPadA = kGBM + 16, kPadB = kGBN + 16;

__global__ __launch_bounds__(256) void batched_gemm_f32(const float *__restrict__ A, const float *__restrict__ B,
                                                        float *__restrict__ C, int64_t M, int64_t N, int64_t K,
                                                        int64_t m_blocks, int64_t n_blocks) {
    __shared__ float la[2][kGBK * kPadA];
    __shared__ float lb[2][kGBK * kPadB];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wr = wave >> 1, wc = wave & 1;

    const int64_t per_batch = m_blocks * n_blocks;
    const int64_t bid = blockIdx.x;
    const int64_t batch = bid / per_batch;
    const int64_t rem = bid - batch * per_batch;
    const int64_t mb = rem / n_blocks;
    const int64_t nb = rem - mb * n_blocks;
    const int64_t m0 = mb * kGBM, n0 = nb * kGBN;
    const float *Ab = A + batch * M * K;
    const float *Bb = B + batch * K * N;
    float *Cb = C + batch * M * N;
    const bool vec_a = (K % 4) == 0;
    const bool vec_b = (N % 4) == 0;

    // Global loads: A 64 x 16 = 256 float4 (one a thread), B 16 x 128 = 512 (two).
    float4 ra, rb[2];
    const auto load = [&](int64_t k0) {
        {
            const int r = tid / 4, kq = (tid % 4) * 4;
            const int64_t row = m0 + r, k = k0 + kq;
            float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
            if (row < M) {
                const float *p = Ab + row * K + k;
                if (vec_a && k + 4 <= K) {
                    x = *reinterpret_cast<const float4 *>(p);
                } else {
                    if (k + 0 < K) x.x = p[0];
                    if (k + 1 < K) x.y = p[1];
                    if (k + 2 < K) x.z = p[2];
                    if (k + 3 < K) x.w = p[3];
                }
            }
            ra = x;
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 256 * i;
            const int kr = idx / 32, nq = (idx % 32) * 4;
            const int64_t k = k0 + kr, col = n0 + nq;
            float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
            if (k < K) {
                const float *p = Bb + k * N + col;
                if (vec_b && col + 4 <= N) {
                    x = *reinterpret_cast<const float4 *>(p);
                } else {
                    if (col + 0 < N) x.x = p[0];
                    if (col + 1 < N) x.y = p[1];
                    if (col + 2 < N) x.z = p[2];
                    if (col + 3 < N) x.w = p[3];
                }
            }
            rb[i] = x;
        }
    };
    const auto store = [&](int buf) {
        const int r = tid / 4, kq = (tid % 4) * 4;
        la[buf][(kq + 0) * kPadA + r] = ra.x;
        la[buf][(kq + 1) * kPadA + r] = ra.y;
        la[buf][(kq + 2) * kPadA + r] = ra.z;
        la[buf][(kq + 3) * kPadA + r] = ra.w;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 256 * i;
            const int kr = idx / 32, nq = (idx % 32) * 4;
            *reinterpret_cast<float4 *>(&lb[buf][kr * kPadB + nq]) = rb[i];
        }
    };

    float4v acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = float4v{};

    const int64_t steps = (K + kGBK - 1) / kGBK;
    load(0);
    store(0);
    __syncthreads();
    const int lr = lane & 15, lk = lane >> 4;
    for (int64_t s = 0; s < steps; ++s) {
        const int cur = s & 1;
        if (s + 1 < steps) load((s + 1) * kGBK);
#pragma unroll
        for (int kk = 0; kk < kGBK; kk += 4) {
            float av[2], bv[4];
#pragma unroll
            for (int i = 0; i < 2; ++i) av[i] = la[cur][(kk + lk) * kPadA + wr * 32 + 16 * i + lr];
#pragma unroll
            for (int j = 0; j < 4; ++j) bv[j] = lb[cur][(kk + lk) * kPadB + wc * 64 + 16 * j + lr];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[j], acc[i][j], 0, 0, 0);
        }
        if (s + 1 < steps) store(cur ^ 1);
        __syncthreads();
    }
    // Row 4 (lane / 16) + e, column lane % 16 of each 16 x 16 tile.
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int64_t row = m0 + wr * 32 + 16 * i + 4 * lk + e;
                const int64_t col = n0 + wc * 64 + 16 * j + lr;
                if (row < M && col < N) Cb[row * N + col] = acc[i][j][e];
            }
}

// ------------------------------------------------------------------ 4. outputs

// Y = A^T M A of the tile's alpha^2 products, then the sum begun from the
// residual (from_redirect) and the chain, one thread per (oc, tile),
// consecutive threads consecutive tiles.
template <int M>
__global__ __launch_bounds__(256) void outputs_kernel(WinogradArgs a, const float *__restrict__ prod) {
    constexpr int A = Mat<M>::A;
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;
    if (t >= static_cast<uint32_t>(a.tiles * a.oc)) return;
    const uint32_t oc = t / static_cast<uint32_t>(a.tiles);
    const uint32_t tile = t - oc * static_cast<uint32_t>(a.tiles);
    uint32_t tx, ty, n;
    split_index(tile, static_cast<uint32_t>(a.tw), static_cast<uint32_t>(a.th), tx, ty, n);
    const int64_t plane = a.oc * a.tiles;
    float m[A][A];
#pragma unroll
    for (int i = 0; i < A; ++i)
#pragma unroll
        for (int j = 0; j < A; ++j) m[i][j] = prod[(i * A + j) * plane + static_cast<int64_t>(oc) * a.tiles + tile];
    float am[M][A];
#pragma unroll
    for (int i = 0; i < M; ++i)
#pragma unroll
        for (int j = 0; j < A; ++j) {
            float s = 0.0f;
#pragma unroll
            for (int x = 0; x < A; ++x) s += Mat<M>::at(i, x) * m[x][j];
            am[i][j] = s;
        }
    // The tile's M x M outputs, their loads (the residual, the chain's
    // operands) all before their stores; outputs past the image's edge read
    // its last row or column and are not stored.
    float v[M * M];
#pragma unroll
    for (int i = 0; i < M; ++i)
#pragma unroll
        for (int jj = 0; jj < M; ++jj) {
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < A; ++j) s += am[i][j] * Mat<M>::at(jj, j);
            v[i * M + jj] = s;
        }
    const auto yy = [&](int e) -> int64_t {
        const int64_t y = static_cast<int64_t>(ty) * M + e / M;
        return y < a.oh ? y : a.oh - 1;
    };
    const auto xx = [&](int e) -> int64_t {
        const int64_t x = static_cast<int64_t>(tx) * M + e % M;
        return x < a.ow ? x : a.ow - 1;
    };
    float *out = a.y + static_cast<int64_t>(n) * a.ynb3 + static_cast<int64_t>(oc) * a.ynb2;
    if (a.from_redirect) {
        float r[M * M];
#pragma unroll
        for (int e = 0; e < M * M; ++e) r[e] = out[yy(e) * a.ynb1 + xx(e)];
#pragma unroll
        for (int e = 0; e < M * M; ++e) v[e] = __fadd_rn(r[e], v[e]);
    }
    apply_chain_block(a.chain, v, [&](int s, int e) {
        const DevStep &st = a.chain.steps[s];
        const int64_t xy = st.flat01 ? (yy(e) * a.ow + xx(e)) * st.nb[0] : xx(e) * st.nb[0] + yy(e) * st.nb[1];
        return xy + static_cast<int64_t>(oc) * st.nb[2] + static_cast<int64_t>(n) * st.nb[3];
    });
#pragma unroll
    for (int e = 0; e < M * M; ++e) {
        const int64_t y = static_cast<int64_t>(ty) * M + e / M;
        const int64_t x = static_cast<int64_t>(tx) * M + e % M;
        if (y < a.oh && x < a.ow) out[y * a.ynb1 + x] = v[e];
    }
}

struct WorkLayout {
    size_t u, v, m, total;  // byte offsets of U, V, M and the whole
};

WorkLayout work_layout(const WinogradArgs &a) {
    const int64_t alpha2 = (a.m + 2) * (a.m + 2);
    WorkLayout l{};
    const size_t u = static_cast<size_t>(alpha2 * a.oc * a.ic) * 4;
    const size_t v = static_cast<size_t>(alpha2 * a.ic * a.tiles) * 4;
    const size_t m = static_cast<size_t>(alpha2 * a.oc * a.tiles) * 4;
    l.u = 0;
    l.v = round_up(static_cast<int64_t>(u), 256);
    l.m = l.v + round_up(static_cast<int64_t>(v), 256);
    l.total = l.m + round_up(static_cast<int64_t>(m), 256);
    return l;
}

template <int M>
sdhip_status run(const WinogradArgs &a, void *work, hipStream_t stream) {
    constexpr int A = Mat<M>::A;
    const WorkLayout l = work_layout(a);
    char *base = static_cast<char *>(work);
    float *u = reinterpret_cast<float *>(base + l.u);
    float *v = reinterpret_cast<float *>(base + l.v);
    float *m = reinterpret_cast<float *>(base + l.m);
    const int64_t nw = a.oc * a.ic;
    {
        KernelScope scope(M == 4 ? "winograd4.weights" : "winograd2.weights", stream);
        hipLaunchKernelGGL((weights_kernel<M>), dim3(ceil_div(nw, 256)), dim3(256), 0, stream, a.w, u, a.oc, a.ic);
    }
    {
        KernelScope scope(M == 4 ? "winograd4.inputs" : "winograd2.inputs", stream);
        const int64_t ni = a.tiles * a.ic;
        hipLaunchKernelGGL((inputs_kernel<M>), dim3(ceil_div(ni, 256)), dim3(256), 0, stream, a, v);
    }
    {
        KernelScope scope(M == 4 ? "winograd4.products" : "winograd2.products", stream);
        const int64_t mb = ceil_div(a.oc, kGBM), nb = ceil_div(a.tiles, kGBN);
        hipLaunchKernelGGL(batched_gemm_f32, dim3(A * A * mb * nb), dim3(256), 0, stream, u, v, m, a.oc, a.tiles,
                           a.ic, mb, nb);
    }
    {
        KernelScope scope(M == 4 ? "winograd4.outputs" : "winograd2.outputs", stream);
        const int64_t no = a.tiles * a.oc;
        hipLaunchKernelGGL((outputs_kernel<M>), dim3(ceil_div(no, 256)), dim3(256), 0, stream, a, m);
    }
    return launched(hipGetLastError(), "winograd");
}

}  // namespace

size_t winograd_work_size(const WinogradArgs &a) { return work_layout(a).total; }

sdhip_status winograd(const WinogradArgs &a, void *work, hipStream_t stream) {
    return a.m == 4 ? run<4>(a, work, stream) : run<2>(a, work, stream);
}

}  // namespace sdhip
