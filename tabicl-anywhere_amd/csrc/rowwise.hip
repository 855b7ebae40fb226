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
    if (qmlp_fused(b)) {  // (one row's eight query-heads included: 1 workgroup against two few-row GEMMs)
        qmlp(s, rows, b, scale, q);
        return;
    }
    dense(s, M, b.ss_hidden, hd, q, hd, b.q0w, b.q0_s, b.q0b, scratch, b.ss_hidden, EPI_GELU, nullptr, 0);
    if (M >= 32 && b.q2_s.img && gemm_split_fits(hd, b.ss_hidden) && b.ss_hidden % 4 == 0)
        gemm_split(s, M, hd, b.ss_hidden, scratch, b.ss_hidden, b.q2_s, b.q2b, q, hd, EPI_QMOD, q, hd, scale, b.heads);
    else
        gemm_qmod(s, M, hd, b.ss_hidden, scratch, b.ss_hidden, b.q2w, b.q2b, q, scale, b.heads);
}

}  // namespace tah
