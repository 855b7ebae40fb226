// Row-wise kernels of the in-context stage: layer normalisation and the query's scalable-softmax modulation.
//
// layer_norm follows src/kern.rs:326-347 (two passes: mean, then biased variance; eps 1e-5), one wavefront per row
// with the sums reduced across the 64 lanes. query_modulate follows src/nn.rs:130-152 after the query projection:
// per head, hid = gelu(q0 q_h + q0b), mm = q2 hid + q2b, q_h *= scale_h * (1 + tanh(mm)); one wavefront per
// (row, head), the hidden layer staged in LDS.
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

// q [rows][d]: one wavefront per (row, head). hid <= 256, hd <= 256.
__global__ __launch_bounds__(256) void k_query_ss(int rows, int d, int heads, int hid, const float *__restrict__ scale,
                                                   const float *__restrict__ q0w, const float *__restrict__ q0b,
                                                   const float *__restrict__ q2w, const float *__restrict__ q2b,
                                                   float *__restrict__ q) {
    __shared__ float hs[4][256];
    __shared__ float qs[4][256];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int item = blockIdx.x * 4 + wv;
    const int hd = d / heads;
    const bool live = item < rows * heads;
    const int row = live ? item / heads : 0, h = live ? item % heads : 0;
    float *qh = q + (size_t)row * d + h * hd;
    if (live)
        for (int c = lane; c < hd; c += 64) qs[wv][c] = qh[c];
    __syncthreads();
    if (live)
        for (int j = lane; j < hid; j += 64) {
            const float *wr = q0w + (size_t)j * hd;
            float a = q0b[j];
            for (int c = 0; c < hd; c++) a += wr[c] * qs[wv][c];
            hs[wv][j] = gelu(a);
        }
    __syncthreads();
    if (live)
        for (int i = lane; i < hd; i += 64) {
            const float *wr = q2w + (size_t)i * hid;
            float a = q2b[i];
            for (int j = 0; j < hid; j++) a += wr[j] * hs[wv][j];
            qh[i] = qs[wv][i] * (scale[h * hd + i] * (1.0f + tanhf(a)));
        }
}

__global__ void k_scale_cols(int rows, int d, const float *__restrict__ scale, float *__restrict__ q) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < (size_t)rows * d) q[i] *= scale[i % d];
}

void query_modulate(hipStream_t s, int rows, const DevBlock &b, const float *scale, float *q) {
    if (rows <= 0) return;
    if (b.ss_hidden == 0) {
        const size_t n = (size_t)rows * b.d;
        hipLaunchKernelGGL(k_scale_cols, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, rows, b.d, scale, q);
    } else {
        if (b.ss_hidden > 256 || b.d / b.heads > 256) throw ArgError{"query MLP wider than 256 is not supported"};
        const int items = rows * b.heads;
        hipLaunchKernelGGL(k_query_ss, dim3((items + 3) / 4), dim3(256), 0, s, rows, b.d, b.heads, b.ss_hidden, scale,
                           b.q0w, b.q0b, b.q2w, b.q2b, q);
    }
    TAH_LAUNCHED();
}

}  // namespace tah
