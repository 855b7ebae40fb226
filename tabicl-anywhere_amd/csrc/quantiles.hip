// The regression head's reading of a row of predicted quantiles as a distribution (QuantileDist, src/table.rs:
// 292-346), on the card for every row of a member's output at once (src/table.rs:479-486 applies it per row):
// sorted by the total order of f32 (f32::total_cmp), levels i / (n + 1), straight lines between neighbours,
// exponential tails fitted by least squares to the first and last k = clamp(n / 4, 1, 20) points. Per row it
// writes the mean, the sample variance (divisor n - 1), the median (icdf at 0.5) and the icdf at each requested
// level, in f32.
//
// One workgroup per row: the row's values, mapped to unsigned keys that order as total_cmp orders the floats
// (positives with the sign bit set, negatives complemented; NaNs after +inf or before -inf by their sign), are
// sorted by a bitonic network over 1,024 keys in LDS (past n: all-ones keys, which sort last). The sums run in the
// reference's order -- left to right over the sorted values, one lane, with no contraction of a product into an
// addition -- so that the moments, the median and every quantile between the first and last level come out as
// the reference computes them; the tails take the device logf (within 1 ulp of the host's).
#include "common.hpp"
#include "device_math.hpp"

namespace tah {

constexpr int QS_MAX = 1024;     // values a row at most
constexpr int QS_ALPHAS = 64;    // requested levels at most

__device__ __forceinline__ uint32_t total_order_key(float v) {
    const uint32_t u = __float_as_uint(v);
    return u ^ ((u >> 31) ? 0xFFFFFFFFu : 0x80000000u);
}
__device__ __forceinline__ float from_total_order_key(uint32_t k) {
    return __uint_as_float((k >> 31) ? (k ^ 0x80000000u) : ~k);
}

// f32::clamp: NaN stays NaN (fminf/fmaxf alone would return a bound)
__device__ __forceinline__ float clamp_keep_nan(float x, float lo, float hi) {
    return x != x ? x : fminf(fmaxf(x, lo), hi);
}

// (a, b) least-squares slope of ys on xs over k points, |.| clamped to [0.01, 100] (src/table.rs:305-310)
__device__ float tail_slope(const float *xs, const float *ys, int k) {
#pragma clang fp contract(off)
    float sx = 0.0f, sy = 0.0f;
    for (int i = 0; i < k; i++) sx += xs[i];
    for (int i = 0; i < k; i++) sy += ys[i];
    const float mx = sx / (float)k, my = sy / (float)k;
    float c = 0.0f, v = 0.0f;
    for (int i = 0; i < k; i++) c += (xs[i] - mx) * (ys[i] - my);
    for (int i = 0; i < k; i++) v += (xs[i] - mx) * (xs[i] - mx);
    const float cov = c / (float)k, var = v / (float)k;
    return clamp_keep_nan(fabsf(cov / fmaxf(var, 1e-6f)), 0.01f, 100.0f);
}

__device__ __forceinline__ float level(int i, int n) { return (float)(i + 1) / (float)(n + 1); }

// grid (rows); 256 threads. q [rows][n] (n in [2, QS_MAX]); alphas [na]; stats [rows][3 + na].
__global__ __launch_bounds__(256) void k_quantile_stats(int n, const float *__restrict__ q, int na,
                                                        const float *__restrict__ alphas, float *__restrict__ stats) {
#pragma clang fp contract(off)
    __shared__ uint32_t key[QS_MAX];
    __shared__ float qs[QS_MAX];
    __shared__ float lnx[2][20];
    __shared__ float tails[4], mom[2];
    const int row = blockIdx.x, tid = threadIdx.x;
    const float *src = q + (size_t)row * n;
    for (int i = tid; i < QS_MAX; i += 256) key[i] = i < n ? total_order_key(src[i]) : 0xFFFFFFFFu;
    __syncthreads();
    for (int size = 2; size <= QS_MAX; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < QS_MAX / 2; i += 256) {
                const int lo = 2 * i - (i & (stride - 1)), hi = lo + stride;
                const bool up = (lo & size) == 0;
                const uint32_t a = key[lo], b = key[hi];
                if ((a > b) == up) {
                    key[lo] = b;
                    key[hi] = a;
                }
            }
            __syncthreads();
        }
    for (int i = tid; i < n; i += 256) qs[i] = from_total_order_key(key[i]);
    __syncthreads();
    const int k = max(min(20, n / 4), 1);
    if (tid == 0) {
        // mean and sample variance, left to right (src/table.rs:322-330)
        float s = 0.0f;
        for (int i = 0; i < n; i++) s += qs[i];
        const float m = s / (float)n;
        float v = 0.0f;
        for (int i = 0; i < n; i++) v += (qs[i] - m) * (qs[i] - m);
        mom[0] = m;
        mom[1] = v / (float)(n - 1);
    } else if (tid == 64) {
        // the tails (src/table.rs:311-315)
        for (int i = 0; i < k; i++) lnx[0][i] = logf(fmaxf(level(i, n), 1e-6f));
        for (int i = 0; i < k; i++) lnx[1][i] = logf(fmaxf(1.0f - level(n - k + i, n), 1e-6f));
        const float bl = tail_slope(lnx[0], qs, k), br = tail_slope(lnx[1], qs + n - k, k);
        tails[0] = bl;
        tails[1] = qs[0] - bl * logf(fmaxf(level(0, n), 1e-6f));
        tails[2] = -br;
        tails[3] = qs[n - 1] + br * logf(1.0f - fminf(level(n - 1, n), 1.0f - 1e-6f));
    }
    __syncthreads();
    float *out = stats + (size_t)row * (3 + na);
    if (tid < 2) out[tid] = mom[tid];
    if (tid > na) return;
    // icdf at 0.5 (thread 0) and at alphas[t - 1] (src/table.rs:333-345)
    const float alpha = tid == 0 ? 0.5f : alphas[tid - 1];
    float y;
    if (alpha < level(0, n)) {
        y = tails[0] * logf(fmaxf(alpha, 1e-6f)) + tails[1];
    } else if (alpha > level(n - 1, n)) {
        y = tails[2] * logf(fmaxf(1.0f - alpha, 1e-6f)) + tails[3];
    } else if (alpha >= level(n - 1, n)) {
        y = qs[n - 1];
    } else {
        // the number of levels[0 .. n - 2] at most alpha, less one (the segment's left end), within [0, n - 2]
        int lo = 0, hi = n - 1;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (level(mid, n) <= alpha) lo = mid + 1;
            else hi = mid;
        }
        const int i = min(max(lo - 1, 0), n - 2);
        const float t = clamp_keep_nan((alpha - level(i, n)) / fmaxf(level(i + 1, n) - level(i, n), 1e-6f), 0.0f, 1.0f);
        y = qs[i] + t * (qs[i + 1] - qs[i]);
    }
    out[2 + tid] = y;
}

void quantile_stats(hipStream_t s, int rows, int n, const float *q, int na, const float *alphas, float *stats) {
    if (rows <= 0) return;
    if (n < 2 || n > QS_MAX || na < 0 || na > QS_ALPHAS || (na > 0 && !alphas))
        throw ArgError{"quantile_stats: 2 to 1024 quantiles a row and at most 64 levels"};
    if (rows > 0x7FFFFFFF) throw ArgError{"quantile_stats: too many rows"};
    hipLaunchKernelGGL(k_quantile_stats, dim3(rows), dim3(256), 0, s, n, q, na, alphas, stats);
    TAH_LAUNCHED();
}

}  // namespace tah
