// Dense layers of every block: Y = epi(X W^T + b), W [out][in] as PyTorch stores it.
//
// The main kernel is an fp32 MFMA GEMM for CDNA4 (v_mfma_f32_16x16x4_f32): a 256-thread workgroup computes a
// 64 x 64 tile of Y as 2 x 2 wavefronts of 32 x 32 (2 x 2 MFMA tiles of 16 x 16 each), staging 64 x 16 slices of X
// and W through LDS. Both operands are K-contiguous, so each lane reads four consecutive K values with one
// 128-bit LDS load and feeds them to four MFMA steps: step t gives lane l the K index 4*(l/16) + t, the same
// permutation on both operands, which leaves the sum unchanged. The epilogue fuses bias, GELU and the block's
// residual add (src/nn.rs:156-164, src/predict.rs:542-568). Shapes whose K is not a multiple of 4 (the input
// layer's 3 features) use a plain one-thread-per-output kernel.
#include "common.hpp"
#include "device_math.hpp"

namespace tah {

// Epilogues: bias, then GELU, or the block's residual add, or the scalable softmax's query modulation
// (EPI_QMOD: the output is R * scale * (1 + tanh(acc + b)), src/nn.rs:145-149, with R the query projection viewed
// as [rows * heads][hd] and scale[(m % heads) * hd + n]).
struct EpiArgs {
    const float *R;
    int ldr;
    const float *scale;
    int heads;
};

template <int EPI>
__device__ __forceinline__ float epilogue(float acc, const float *b, int n, const EpiArgs &e, int m, int N) {
    float y = acc + (b ? b[n] : 0.0f);
    if (EPI == EPI_GELU) y = gelu(y);
    if (EPI == EPI_RESID) y += e.R[(size_t)m * e.ldr + n];
    if (EPI == EPI_QMOD) y = e.R[(size_t)m * e.ldr + n] * (e.scale[(m % e.heads) * N + n] * (1.0f + tanh1(y)));
    if (EPI == EPI_SCALE) y *= e.scale[n];
    return y;
}

constexpr int GB = 64;   // tile rows and columns
constexpr int GK = 16;   // K slice
constexpr int GKP = 20;  // padded LDS row

template <int EPI>
__global__ __launch_bounds__(256) void k_gemm_mfma(int M, int N, int K, const float *__restrict__ X, int ldx,
                                                    const float *__restrict__ W, const float *__restrict__ b,
                                                    float *Y, int ldy, EpiArgs ea) {
    __shared__ float As[2][GB][GKP];
    __shared__ float Bs[2][GB][GKP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * GB, n0 = blockIdx.x * GB;
    const int lr = tid >> 2, lc = (tid & 3) * 4;
    const int gm = m0 + lr, gn = n0 + lr;
    floatx4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    auto load = [&](int k0, float4 &av, float4 &bv) {
        const int gk = k0 + lc;
        av = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        bv = av;
        if (gk < K) {
            if (gm < M) av = *reinterpret_cast<const float4 *>(X + (size_t)gm * ldx + gk);
            if (gn < N) bv = *reinterpret_cast<const float4 *>(W + (size_t)gn * K + gk);
        }
    };
    float4 av, bv;
    load(0, av, bv);
    int buf = 0;
    *reinterpret_cast<float4 *>(&As[0][lr][lc]) = av;
    *reinterpret_cast<float4 *>(&Bs[0][lr][lc]) = bv;
    __syncthreads();
    const int kq = (lane >> 4) * 4, r16 = lane & 15;
    for (int k0 = 0; k0 < K; k0 += GK) {
        const bool more = k0 + GK < K;
        if (more) load(k0 + GK, av, bv);  // next slice in flight while this one is multiplied
        const float4 a0 = *reinterpret_cast<const float4 *>(&As[buf][wm * 32 + r16][kq]);
        const float4 a1 = *reinterpret_cast<const float4 *>(&As[buf][wm * 32 + 16 + r16][kq]);
        const float4 b0 = *reinterpret_cast<const float4 *>(&Bs[buf][wn * 32 + r16][kq]);
        const float4 b1 = *reinterpret_cast<const float4 *>(&Bs[buf][wn * 32 + 16 + r16][kq]);
        acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0.x, b0.x, acc[0][0], 0, 0, 0);
        acc[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0.x, b1.x, acc[0][1], 0, 0, 0);
        acc[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1.x, b0.x, acc[1][0], 0, 0, 0);
        acc[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1.x, b1.x, acc[1][1], 0, 0, 0);
        acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0.y, b0.y, acc[0][0], 0, 0, 0);
        acc[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0.y, b1.y, acc[0][1], 0, 0, 0);
        acc[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1.y, b0.y, acc[1][0], 0, 0, 0);
        acc[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1.y, b1.y, acc[1][1], 0, 0, 0);
        acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0.z, b0.z, acc[0][0], 0, 0, 0);
        acc[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0.z, b1.z, acc[0][1], 0, 0, 0);
        acc[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1.z, b0.z, acc[1][0], 0, 0, 0);
        acc[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1.z, b1.z, acc[1][1], 0, 0, 0);
        acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0.w, b0.w, acc[0][0], 0, 0, 0);
        acc[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0.w, b1.w, acc[0][1], 0, 0, 0);
        acc[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1.w, b0.w, acc[1][0], 0, 0, 0);
        acc[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1.w, b1.w, acc[1][1], 0, 0, 0);
        if (more) {
            *reinterpret_cast<float4 *>(&As[buf ^ 1][lr][lc]) = av;
            *reinterpret_cast<float4 *>(&Bs[buf ^ 1][lr][lc]) = bv;
        }
        __syncthreads();
        buf ^= 1;
    }
    // lane l holds D[4*(l/16) + v][l % 16] of each 16 x 16 tile
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + wn * 32 + j * 16 + r16;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int m = m0 + wm * 32 + i * 16 + kq + v;
                if (m < M && n < N) Y[(size_t)m * ldy + n] = epilogue<EPI>(acc[i][j][v], b, n, ea, m, N);
            }
        }
}

// Few rows (single-row and small-batch prediction): a workgroup computes one 16 x 16 tile of Y and its four
// wavefronts split K between them, loading MFMA operands straight from global memory (each weight row is read
// once per tile, coalesced in 64-byte runs); the four partial tiles are summed through LDS before the epilogue.
// Many more workgroups than the 64 x 64 kernel has at small M, so the weights stream at a useful rate.
// With LN, the workgroup first normalises its 16 rows into LDS (two passes, biased variance, eps 1e-5, as
// k_layer_norm; 16 threads a row), and the products read them from there: the separate layer-norm launch, which at
// these sizes costs as much as the product, goes away.
constexpr int SKINNY_LN_K = 1024;  // widest rows the fused layer norm takes
// most rows the 16 x 16 tile kernel takes (the column and row stages' width-128 layers of up to 16 table rows: 3 rows
// 0.817 -> 0.707 ms a prediction, 8 rows 0.826 -> 0.753, 16 rows 0.845 -> 0.832, against the 64 x 64 tiles; from
// 32 table rows, 3,300 rows, the stages' tile kernels are faster)
constexpr int SKINNY_ROWS = 2048;
template <int EPI, bool LN>
__global__ __launch_bounds__(256) void k_gemm_skinny(int M, int N, int K, const float *__restrict__ X, int ldx,
                                                      const float *__restrict__ W, const float *__restrict__ b,
                                                      float *Y, int ldy, EpiArgs ea, const float *__restrict__ lnw,
                                                      const float *__restrict__ lnb) {
    __shared__ float red[4][16][17];
    __shared__ __align__(16) float xs[LN ? 16 * (SKINNY_LN_K + 4) : 4];  // rows padded by 4: no bank conflicts
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m0 = blockIdx.y * 16, n0 = blockIdx.x * 16;
    const int r16 = lane & 15, g4 = lane >> 4;
    const int gm = m0 + r16, gn = n0 + r16;
    const int xstride = K + 4;
    if (LN) {
        const int rr = tid >> 4, cc = tid & 15, gmr = m0 + rr;
        float *xw = xs + rr * xstride;
        float sum = 0.0f;
        for (int k = 4 * cc; k < K; k += 64) {
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (gmr < M) v = *reinterpret_cast<const float4 *>(X + (size_t)gmr * ldx + k);
            *reinterpret_cast<float4 *>(xw + k) = v;
            sum += (v.x + v.y) + (v.z + v.w);
        }
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) sum += __shfl_xor(sum, o, 64);
        const float mean = sum / (float)K;
        float sq = 0.0f;
        for (int k = 4 * cc; k < K; k += 64) {
            const float4 v = *reinterpret_cast<const float4 *>(xw + k);
            const float d0 = v.x - mean, d1 = v.y - mean, d2 = v.z - mean, d3 = v.w - mean;
            sq += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
        }
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) sq += __shfl_xor(sq, o, 64);
        const float inv = 1.0f / sqrtf(sq / (float)K + 1e-5f);
        for (int k = 4 * cc; k < K; k += 64) {
            const float4 v = *reinterpret_cast<const float4 *>(xw + k);
            const float4 w4 = *reinterpret_cast<const float4 *>(lnw + k), b4 = *reinterpret_cast<const float4 *>(lnb + k);
            *reinterpret_cast<float4 *>(xw + k) =
                make_float4((v.x - mean) * inv * w4.x + b4.x, (v.y - mean) * inv * w4.y + b4.y,
                            (v.z - mean) * inv * w4.z + b4.z, (v.w - mean) * inv * w4.w + b4.w);
        }
        __syncthreads();
    }
    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const float *xr = X + (size_t)gm * ldx, *wr = W + (size_t)gn * K;
    const float *xl = xs + r16 * xstride;
#pragma unroll 4
    for (int k0 = 16 * wave; k0 < K; k0 += 64) {
        const int gk = k0 + 4 * g4;
        float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), bb = a;
        if (gk < K) {
            if (LN) a = *reinterpret_cast<const float4 *>(xl + gk);
            else if (gm < M) a = *reinterpret_cast<const float4 *>(xr + gk);
            if (gn < N) bb = *reinterpret_cast<const float4 *>(wr + gk);
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, bb.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, bb.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, bb.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, bb.w, acc, 0, 0, 0);
    }
#pragma unroll
    for (int v = 0; v < 4; v++) red[wave][4 * g4 + v][r16] = acc[v];
    __syncthreads();
    const int i = tid >> 4, j = tid & 15;
    const int m = m0 + i, n = n0 + j;
    if (m < M && n < N) {
        const float a = (red[0][i][j] + red[1][i][j]) + (red[2][i][j] + red[3][i][j]);
        Y[(size_t)m * ldy + n] = epilogue<EPI>(a, b, n, ea, m, N);
    }
}

// At most 8 rows (single-row prediction): one wavefront per output column, its lanes over K (four consecutive
// columns a lane per 256), the rows held in LDS, the rows' dot products summed across the wavefront. Every global
// read is issued first -- the column's weights, with LN the norm's weights at the same K positions, the rows, and
// the bias and residual of the epilogue (lane r holds row r's) -- so that one memory latency precedes the sums
// rather than a chain of them; with LN each row's mean and inverse deviation go through LDS and the normalisation
// is applied inside the dot products. Every compute unit gets a few columns' weight streams, where the 16 x 16 tile
// kernel would occupy N / 16 of them.
constexpr int GEMV_ROWS = 8;
template <int EPI, bool LN>
__global__ __launch_bounds__(256) void k_gemv(int M, int N, int K, const float *__restrict__ X, int ldx,
                                               const float *__restrict__ W, const float *__restrict__ b, float *Y,
                                               int ldy, EpiArgs ea, const float *__restrict__ lnw,
                                               const float *__restrict__ lnb) {
    constexpr int KJ = SKINNY_LN_K / 256;
    __shared__ __align__(16) float xs[GEMV_ROWS][SKINNY_LN_K];
    __shared__ float stat[GEMV_ROWS][2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = blockIdx.x * 4 + wave;
    const bool col = n < N;
    // (slots past the row's end, or of a column past N, read clamped in-range addresses and are never used)
    float4 w4[KJ], g4[KJ], c4[KJ];
    const float *wr = W + (size_t)min(n, N - 1) * K;
#pragma unroll
    for (int j = 0; j < KJ; j++) {
        const int k = min(4 * lane + 256 * j, K - 4);
        w4[j] = *reinterpret_cast<const float4 *>(wr + k);
        if (LN) {
            g4[j] = *reinterpret_cast<const float4 *>(lnw + k);
            c4[j] = *reinterpret_cast<const float4 *>(lnb + k);
        }
    }
    float bias = 0.0f, res = 0.0f;
    if (col && lane < M) {
        if (b) bias = b[n];
        if (EPI == EPI_RESID) res = ea.R[(size_t)lane * ea.ldr + n];
    }
    for (int i = 4 * tid; i < M * K; i += 1024) {
        const int r = i / K, k = i - r * K;
        *reinterpret_cast<float4 *>(&xs[r][k]) = *reinterpret_cast<const float4 *>(X + (size_t)r * ldx + k);
    }
    __syncthreads();
    if (LN) {
        // wavefront w takes rows w and w + 4 (two passes: mean, then biased variance; eps 1e-5)
        for (int r = wave; r < M; r += 4) {
            float sum = 0.0f;
            for (int k = lane; k < K; k += 64) sum += xs[r][k];
            const float mean = wave_sum(sum) / (float)K;
            float sq = 0.0f;
            for (int k = lane; k < K; k += 64) {
                const float dv = xs[r][k] - mean;
                sq += dv * dv;
            }
            const float inv = 1.0f / sqrtf(wave_sum(sq) / (float)K + 1e-5f);
            if (lane == 0) {
                stat[r][0] = mean;
                stat[r][1] = inv;
            }
        }
        __syncthreads();
    }
    if (!col) return;
    float acc[GEMV_ROWS];
#pragma unroll
    for (int r = 0; r < GEMV_ROWS; r++) acc[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < KJ; j++) {
        const int k = 4 * lane + 256 * j;
        if (k >= K) break;
#pragma unroll
        for (int r = 0; r < GEMV_ROWS; r++) {
            if (r >= M) break;
            float4 x4 = *reinterpret_cast<const float4 *>(&xs[r][k]);
            if (LN) {
                const float mean = stat[r][0], inv = stat[r][1];
                x4.x = (x4.x - mean) * inv * g4[j].x + c4[j].x;
                x4.y = (x4.y - mean) * inv * g4[j].y + c4[j].y;
                x4.z = (x4.z - mean) * inv * g4[j].z + c4[j].z;
                x4.w = (x4.w - mean) * inv * g4[j].w + c4[j].w;
            }
            acc[r] += (w4[j].x * x4.x + w4[j].y * x4.y) + (w4[j].z * x4.z + w4[j].w * x4.w);
        }
    }
    float mine = 0.0f;  // lane r: row r's sum
#pragma unroll
    for (int r = 0; r < GEMV_ROWS; r++) {
        if (r >= M) break;
        const float a = wave_sum(acc[r]);
        if (lane == r) mine = a;
    }
    if (lane >= M) return;
    float y;
    if (EPI == EPI_QMOD || EPI == EPI_SCALE) {
        y = epilogue<EPI>(mine, b, n, ea, lane, N);
    } else {
        y = mine + bias;
        if (EPI == EPI_GELU) y = gelu(y);
        if (EPI == EPI_RESID) y += res;
    }
    Y[(size_t)lane * ldy + n] = y;
}

template <int EPI>
__global__ __launch_bounds__(256) void k_gemm_plain(int M, int N, int K, const float *__restrict__ X, int ldx,
                                                     const float *__restrict__ W, const float *__restrict__ b,
                                                     float *Y, int ldy, EpiArgs ea) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)M * N) return;
    const int m = (int)(i / N), n = (int)(i % N);
    const float *xr = X + (size_t)m * ldx, *wr = W + (size_t)n * K;
    float a = 0.0f;
    for (int k = 0; k < K; k++) a += xr[k] * wr[k];
    Y[(size_t)m * ldy + n] = epilogue<EPI>(a, b, n, ea, m, N);
}

template <int EPI>
static void launch(hipStream_t s, int M, int N, int K, const float *X, int ldx, const float *W, const float *b, float *Y,
                   int ldy, EpiArgs ea, const float *lnw = nullptr, const float *lnb = nullptr) {
    const bool aligned = K % 4 == 0 && ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(X) & 15) == 0 &&
                         (reinterpret_cast<uintptr_t>(W) & 15) == 0;
    const bool wq = (reinterpret_cast<uintptr_t>(W) & 15) == 0 && K % 4 == 0;
    if (aligned && wq && M <= GEMV_ROWS && K <= SKINNY_LN_K) {
        if (lnw)
            hipLaunchKernelGGL((k_gemv<EPI, true>), dim3((N + 3) / 4), dim3(256), 0, s, M, N, K, X, ldx, W, b, Y, ldy,
                               ea, lnw, lnb);
        else
            hipLaunchKernelGGL((k_gemv<EPI, false>), dim3((N + 3) / 4), dim3(256), 0, s, M, N, K, X, ldx, W, b, Y, ldy,
                               ea, nullptr, nullptr);
    } else if (lnw) {
        if (!(aligned && M <= SKINNY_ROWS && K <= SKINNY_LN_K)) throw ArgError{"gemm: fused layer norm needs the few-rows kernel"};
        dim3 grid((N + 15) / 16, (M + 15) / 16);
        hipLaunchKernelGGL((k_gemm_skinny<EPI, true>), grid, dim3(256), 0, s, M, N, K, X, ldx, W, b, Y, ldy, ea, lnw,
                           lnb);
    } else if (aligned && (M <= SKINNY_ROWS || N <= 32)) {  // few rows, or few columns (the decoder's last layer)
        dim3 grid((N + 15) / 16, (M + 15) / 16);
        hipLaunchKernelGGL((k_gemm_skinny<EPI, false>), grid, dim3(256), 0, s, M, N, K, X, ldx, W, b, Y, ldy, ea,
                           nullptr, nullptr);
    } else if (aligned) {
        dim3 grid((N + GB - 1) / GB, (M + GB - 1) / GB);
        hipLaunchKernelGGL(k_gemm_mfma<EPI>, grid, dim3(256), 0, s, M, N, K, X, ldx, W, b, Y, ldy, ea);
    } else {
        const size_t n = (size_t)M * N;
        hipLaunchKernelGGL(k_gemm_plain<EPI>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, M, N, K, X, ldx, W, b,
                           Y, ldy, ea);
    }
    TAH_LAUNCHED();
}

// Rows per launch: the tile kernel's grid covers 64 rows a workgroup in its second dimension (at most 65,535), so
// taller matrices (a fit's column stage: feature groups x training rows) go in slabs of rows, which are independent.
constexpr size_t SLAB_ROWS = (size_t)65535 * GB;

void gemm(hipStream_t s, int M, int N, int K, const float *X, int ldx, const float *W, const float *b, float *Y, int ldy,
          Epi epi, const float *R, int ldr, const float *lnw, const float *lnb, const float *scale) {
    if (M <= 0 || N <= 0) return;
    if (epi == EPI_SCALE && !scale) throw ArgError{"gemm: the scale epilogue needs its scales"};
    for (size_t r0 = 0; r0 < (size_t)M; r0 += SLAB_ROWS) {
        const int m = (int)std::min(SLAB_ROWS, (size_t)M - r0);
        const float *Xs = X + r0 * ldx;
        float *Ys = Y + r0 * ldy;
        const EpiArgs ea{R ? R + r0 * ldr : nullptr, ldr, scale, 1};
        switch (epi) {
            case EPI_NONE: launch<EPI_NONE>(s, m, N, K, Xs, ldx, W, b, Ys, ldy, ea, lnw, lnb); break;
            case EPI_GELU: launch<EPI_GELU>(s, m, N, K, Xs, ldx, W, b, Ys, ldy, ea, lnw, lnb); break;
            case EPI_RESID: launch<EPI_RESID>(s, m, N, K, Xs, ldx, W, b, Ys, ldy, ea, lnw, lnb); break;
            case EPI_SCALE: launch<EPI_SCALE>(s, m, N, K, Xs, ldx, W, b, Ys, ldy, ea, lnw, lnb); break;
            default: throw ArgError{"gemm: unknown epilogue"};
        }
    }
}

bool gemm_ln_fits(int M, int K, const float *X, int ldx, const float *W) {
    return M <= SKINNY_ROWS && K <= SKINNY_LN_K && K % 4 == 0 && ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(X) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(W) & 15) == 0;
}

void gemm_qmod(hipStream_t s, int M, int N, int K, const float *X, int ldx, const float *W, const float *b, float *q,
               const float *scale, int heads) {
    if (M <= 0 || N <= 0) return;
    if (heads <= 0) throw ArgError{"gemm: the query modulation needs its head count"};
    // slabs of whole rows of heads, so that row m of a slab is still head m % heads
    const size_t slab = SLAB_ROWS / heads * heads;
    for (size_t r0 = 0; r0 < (size_t)M; r0 += slab) {
        const int m = (int)std::min(slab, (size_t)M - r0);
        launch<EPI_QMOD>(s, m, N, K, X + r0 * ldx, ldx, W, b, q + r0 * N, N, EpiArgs{q + r0 * N, N, scale, heads});
    }
}

}  // namespace tah
