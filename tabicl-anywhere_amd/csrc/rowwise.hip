// Row-wise kernels of the in-context stage: layer normalisation and the query's scalable-softmax modulation.
//
// layer_norm follows src/kern.rs:326-347 (two passes: mean, then biased variance; eps 1e-5), one wavefront per row
// with the sums reduced across the 64 lanes. query_modulate follows src/nn.rs:130-152 after the query projection:
// per head, hid = gelu(q0 q_h + q0b), mm = q2 hid + q2b, q_h *= scale_h * (1 + tanh(mm)), as two GEMMs over the
// queries viewed as [rows * heads][hd] with the modulation in the second one's epilogue.
#include "common.hpp"
#include "device_math.hpp"

namespace tah {

__global__ __launch_bounds__(256) void k_layer_norm(int rows, int n, const float *__restrict__ x, int ldx,
                                                     const float *__restrict__ w, const float *__restrict__ b,
                                                     float *__restrict__ y, int ldy) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;  // whole wavefronts leave together
    const float *xr = x + (size_t)row * ldx;
    float s = 0.0f;
    for (int i = lane; i < n; i += 64) s += xr[i];
    const float mean = wave_sum(s) / (float)n;
    float q = 0.0f;
    for (int i = lane; i < n; i += 64) {
        const float d = xr[i] - mean;
        q += d * d;
    }
    const float var = wave_sum(q) / (float)n;
    const float inv = 1.0f / sqrtf(var + 1e-5f);
    float *yr = y + (size_t)row * ldy;
    for (int i = lane; i < n; i += 64) yr[i] = (xr[i] - mean) * inv * w[i] + b[i];
}

void layer_norm(hipStream_t s, int rows, int n, const float *x, int ldx, const float *w, const float *b, float *y,
                int ldy) {
    if (rows <= 0) return;
    hipLaunchKernelGGL(k_layer_norm, dim3((rows + 3) / 4), dim3(256), 0, s, rows, n, x, ldx, w, b, y, ldy);
    TAH_LAUNCHED();
}

__global__ void k_scale_cols(int rows, int d, const float *__restrict__ scale, float *__restrict__ q) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < (size_t)rows * d) q[i] *= scale[i % d];
}

size_t query_scratch_floats(int rows, const DevBlock &b) { return (size_t)rows * b.heads * b.ss_hidden; }

// The query MLP as two GEMMs over q viewed as [rows * heads][hd]: hid = gelu(q0 q_h + q0b), then the modulation
// fused into the second GEMM's epilogue.
void query_modulate(hipStream_t s, int rows, const DevBlock &b, const float *scale, float *q, float *scratch) {
    if (rows <= 0) return;
    if (b.ss_hidden == 0) {
        const size_t n = (size_t)rows * b.d;
        hipLaunchKernelGGL(k_scale_cols, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, rows, b.d, scale, q);
        TAH_LAUNCHED();
        return;
    }
    const int hd = b.d / b.heads, M = rows * b.heads;
    if (M >= 32 && qmlp_fused(b)) {
        qmlp(s, rows, b, scale, q);
        return;
    }
    dense(s, M, b.ss_hidden, hd, q, hd, b.q0w, b.q0_s, b.q0b, scratch, b.ss_hidden, EPI_GELU, nullptr, 0);
    if (M >= 32 && b.q2_s.img && gemm_split_fits(hd, b.ss_hidden) && b.ss_hidden % 4 == 0)
        gemm_split(s, M, hd, b.ss_hidden, scratch, b.ss_hidden, b.q2_s, b.q2b, q, hd, EPI_QMOD, q, hd, scale, b.heads);
    else
        gemm_qmod(s, M, hd, b.ss_hidden, scratch, b.ss_hidden, b.q2w, b.q2b, q, scale, b.heads);
}

// ---- the whole query path for a few rows ------------------------------------------------------------------------
// q = modulate(Wq norm1(h) + bq) (src/nn.rs:130-152 with the projection before it) for at most QF_ROWS rows, head
// width 64 and query-MLP width 64: grid (heads), 512 threads, one launch where the general path takes a layer norm, a
// projection and two MLP products. Every global read is issued at the start (weights, rows, the norm's weights, the
// biases and scales), so that one memory latency precedes the arithmetic. Workgroup h forms head h's 64 query columns
// for every row: wavefront w takes columns 8 w .. 8 w + 7 of Wq (their rows read with the lanes over K in float4
// steps of 256), each lane sums its share of the 64 (column, row) dot products, and a butterfly across the wavefront
// (six exchanges, each halving what a lane holds) leaves lane l with column l / 8 of row l % 8. The query MLP then
// runs in f32 on the 64 values of each row, one thread per (row, unit), its weights staged in LDS (rows padded to 65
// floats, so the 64 lanes reading 64 different rows at one column hit 64 different banks). (Spreading a head over
// several workgroups, the last to finish running the MLP, measured slower: the hand-over between workgroups on
// different XCDs costs about what a second launch does.)
constexpr int QF_ROWS = 8;
constexpr int QF_MAXD = 512;

__global__ __launch_bounds__(512) void k_query_few(int M, int d, const float *__restrict__ h, int ldh,
                                                   const float *__restrict__ lnw, const float *__restrict__ lnb,
                                                   const float *__restrict__ wq, const float *__restrict__ bq,
                                                   const float *__restrict__ w0, const float *__restrict__ b0,
                                                   const float *__restrict__ w2, const float *__restrict__ b2,
                                                   const float *__restrict__ scale, float *__restrict__ q) {
    __shared__ __align__(16) float xs[QF_ROWS][QF_MAXD];
    __shared__ float ws[2][64][65];
    __shared__ float qs[QF_ROWS][64], hs[QF_ROWS][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int head = blockIdx.x, kj = d / 256;
    float4 wv[8][QF_MAXD / 256];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float *wr = wq + (size_t)(head * 64 + 8 * wave + i) * d + 4 * lane;
#pragma unroll
        for (int j = 0; j < QF_MAXD / 256; j++) wv[i][j] = *reinterpret_cast<const float4 *>(wr + 256 * min(j, kj - 1));
    }
    for (int i = 4 * tid; i < M * d; i += 2048) {
        const int r = i / d, k = i - r * d;
        *reinterpret_cast<float4 *>(&xs[r][k]) = *reinterpret_cast<const float4 *>(h + (size_t)r * ldh + k);
    }
    for (int i = tid; i < 2 * 4096; i += 512) {
        const int m = i >> 12, j = (i >> 6) & 63, k = i & 63;
        ws[m][j][k] = (m ? w2 : w0)[j * 64 + k];
    }
    float lw[QF_MAXD / 64], lb[QF_MAXD / 64];  // the norm's weights at this lane's columns lane + 64 i
#pragma unroll
    for (int i = 0; i < QF_MAXD / 64; i++) {
        const int k = min(lane + 64 * i, d - 1);
        lw[i] = lnw[k];
        lb[i] = lnb[k];
    }
    const int col = 8 * wave + (lane >> 3), row = lane & 7;
    const float bqc = bq[head * 64 + col];
    const float b0j = b0[lane], b2j = b2[lane], scj = scale[head * 64 + lane];
    __syncthreads();
    // layer normalisation (two passes, biased variance, eps 1e-5): wavefront r takes row r
    if (wave < M) {
        float xv[QF_MAXD / 64];
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < QF_MAXD / 64; i++) {
            xv[i] = lane + 64 * i < d ? xs[wave][lane + 64 * i] : 0.0f;
            s += xv[i];
        }
        const float mean = wave_sum(s) / (float)d;
        float sq = 0.0f;
#pragma unroll
        for (int i = 0; i < QF_MAXD / 64; i++) {
            const float dv = lane + 64 * i < d ? xv[i] - mean : 0.0f;
            sq += dv * dv;
        }
        const float inv = 1.0f / sqrtf(wave_sum(sq) / (float)d + 1e-5f);
#pragma unroll
        for (int i = 0; i < QF_MAXD / 64; i++)
            if (lane + 64 * i < d) xs[wave][lane + 64 * i] = (xv[i] - mean) * inv * lw[i] + lb[i];
    }
    __syncthreads();
    float v[64];  // (column i, row r) at 8 i + r
#pragma unroll
    for (int e = 0; e < 64; e++) v[e] = 0.0f;
#pragma unroll
    for (int j = 0; j < QF_MAXD / 256; j++) {
        if (j >= kj) break;
#pragma unroll
        for (int r = 0; r < QF_ROWS; r++) {
            if (r >= M) break;
            const float4 x4 = *reinterpret_cast<const float4 *>(&xs[r][4 * lane + 256 * j]);
#pragma unroll
            for (int i = 0; i < 8; i++)
                v[8 * i + r] += (wv[i][j].x * x4.x + wv[i][j].y * x4.y) + (wv[i][j].z * x4.z + wv[i][j].w * x4.w);
        }
    }
    // exchange o: lanes with bit o keep the upper half of what they hold and add their partner's copy of it
#pragma unroll
    for (int st = 0; st < 6; st++) {
        const int o = 32 >> st, half = 32 >> st;
        const bool up = (lane & o) != 0;
#pragma unroll
        for (int e = 0; e < half; e++) {
            const float keep = up ? v[e + half] : v[e];
            const float give = up ? v[e] : v[e + half];
            v[e] = keep + __shfl_xor(give, o, 64);
        }
    }
    if (row < M) qs[row][col] = v[0] + bqc;
    __syncthreads();
    const int r = wave, j = lane;  // one thread per (row, unit)
    if (r >= M) return;
    float a = b0j;
#pragma unroll 16
    for (int k = 0; k < 64; k++) a += ws[0][j][k] * qs[r][k];
    hs[r][j] = gelu(a);  // wavefront r reads back only row r, which it wrote itself (no barrier)
    float y = b2j;
#pragma unroll 16
    for (int k = 0; k < 64; k++) y += ws[1][j][k] * hs[r][k];
    q[(size_t)r * d + head * 64 + j] = qs[r][j] * (scj * (1.0f + tanh1(y)));
}

bool query_few_fits(const DevBlock &b, int rows, const float *h, int ldh) {
    return rows >= 1 && rows <= QF_ROWS && b.heads > 0 && b.d == 64 * b.heads && b.d % 256 == 0 && b.d <= QF_MAXD &&
           b.ss_hidden == 64 && b.q0w && b.q2w && b.in_w && b.n1w && ldh % 4 == 0 &&
           (reinterpret_cast<uintptr_t>(h) & 15) == 0 && (reinterpret_cast<uintptr_t>(b.in_w) & 15) == 0;
}

void query_few(hipStream_t s, int rows, const float *h, int ldh, const DevBlock &b, const float *scale, float *q) {
    if (!query_few_fits(b, rows, h, ldh)) throw ArgError{"query_few: shape not supported"};
    hipLaunchKernelGGL(k_query_few, dim3(b.heads), dim3(512), 0, s, rows, b.d, h, ldh, b.n1w, b.n1b, b.in_w, b.in_b,
                       b.q0w, b.q0b, b.q2w, b.q2b, scale, q);
    TAH_LAUNCHED();
}

}  // namespace tah
