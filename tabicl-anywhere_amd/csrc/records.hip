// The fit-time side of the stored cache: keys and values of every training row, laid out in the reference's chunk
// records and quantised on the card.
//
// * k_to_records: a layer's keys and values as the projection wrote them, row-major [rows][2d], to f32 chunk
//   records [K: d][rc][V: d][rc] per chunk (src/fit.rs:633-647). 64 x 64 tiles are transposed through LDS so both
//   the reads (along coordinates) and the writes (along rows of a chunk) are coalesced.
// * k_pack: f32 records to i16/i8 records, bit for bit as the reference's quantiser (src/fit.rs:549-576): per chunk
//   and coordinate row, big = max |v| (NaN ignored, as f32::max does), s = big > 0 ? big / top : 1 with top 32767
//   or 127, inv = 1 / s, code = round-half-away(v * inv) saturated to the integer range; the 2d scales first.
//   One wavefront per coordinate row. Division is the correctly rounded one (__fdiv_rn), so the same f32 input
//   gives the same scales and codes as the CPU.
#include "common.hpp"
#include "device_math.hpp"

namespace tah {

__global__ __launch_bounds__(256) void k_to_records(int rows, int d2, int chunk, const float *__restrict__ kv,
                                                     float *__restrict__ rec) {
    __shared__ float tile[64][65];
    const int m0 = blockIdx.x * 64, n0 = blockIdx.y * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int i = ty; i < 64; i += 4) {
        const int m = m0 + i, n = n0 + tx;
        tile[i][tx] = (m < rows && n < d2) ? kv[(size_t)m * d2 + n] : 0.0f;
    }
    __syncthreads();
    const int n_chunks = (rows + chunk - 1) / chunk;
    const int last_rc = rows - (n_chunks - 1) * chunk;
    for (int j = ty; j < 64; j += 4) {
        const int n = n0 + j, m = m0 + tx;
        if (m >= rows || n >= d2) continue;
        const int ci = m / chunk, r = m - ci * chunk;
        const int rc = ci == n_chunks - 1 ? last_rc : chunk;
        rec[(size_t)ci * d2 * chunk + (size_t)n * rc + r] = tile[tx][j];
    }
}

template <int FMT>
__global__ __launch_bounds__(256) void k_pack(int rows, int d, int chunk, const float *__restrict__ rec32,
                                               uint8_t *__restrict__ recq) {
    const int ci = blockIdx.x, j = blockIdx.y * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (j >= 2 * d) return;
    const int n_chunks = (rows + chunk - 1) / chunk;
    const int rc = ci == n_chunks - 1 ? rows - (n_chunks - 1) * chunk : chunk;
    const float *src = rec32 + (size_t)ci * 2 * d * chunk + (size_t)j * rc;
    constexpr size_t W = FMT == TAH_KV_I16 ? 2 : 1;
    uint8_t *rec = recq + (size_t)ci * (2 * (size_t)d * chunk * W + 8 * (size_t)d);
    float big = 0.0f;
    for (int r = lane; r < rc; r += 64) big = fmaxf(big, fabsf(src[r]));
    big = wave_max(big);
    const float top = FMT == TAH_KV_I16 ? 32767.0f : 127.0f;
    const float s = big > 0.0f ? __fdiv_rn(big, top) : 1.0f;
    const float inv = __fdiv_rn(1.0f, s);
    if (lane == 0) reinterpret_cast<float *>(rec)[j] = s;
    uint8_t *body = rec + 8 * (size_t)d;
    for (int r = lane; r < rc; r += 64) {
        const float v = roundf(__fmul_rn(src[r], inv));
        if (FMT == TAH_KV_I16) {
            const int16_t code = v != v ? 0 : (v >= 32767.0f ? 32767 : (v <= -32768.0f ? -32768 : (int16_t)v));
            reinterpret_cast<int16_t *>(body)[(size_t)j * rc + r] = code;
        } else {
            const int8_t code = v != v ? 0 : (v >= 127.0f ? 127 : (v <= -128.0f ? -128 : (int8_t)v));
            reinterpret_cast<int8_t *>(body)[(size_t)j * rc + r] = code;
        }
    }
}

void to_records(hipStream_t s, int rows, int d, int chunk, const float *kv, float *rec32) {
    if (rows <= 0) return;
    dim3 grid((rows + 63) / 64, (2 * d + 63) / 64);
    hipLaunchKernelGGL(k_to_records, grid, dim3(256), 0, s, rows, 2 * d, chunk, kv, rec32);
    TAH_LAUNCHED();
}

void pack(hipStream_t s, int rows, int d, int chunk, int fmt, const float *rec32, uint8_t *recq) {
    if (rows <= 0 || fmt == TAH_KV_F32) return;
    const int n_chunks = (rows + chunk - 1) / chunk;
    dim3 grid(n_chunks, (2 * d + 3) / 4);
    if (fmt == TAH_KV_I16)
        hipLaunchKernelGGL(k_pack<TAH_KV_I16>, grid, dim3(256), 0, s, rows, d, chunk, rec32, recq);
    else if (fmt == TAH_KV_I8)
        hipLaunchKernelGGL(k_pack<TAH_KV_I8>, grid, dim3(256), 0, s, rows, d, chunk, rec32, recq);
    else
        throw ArgError{"pack: unknown key/value format"};
    TAH_LAUNCHED();
}

}  // namespace tah
